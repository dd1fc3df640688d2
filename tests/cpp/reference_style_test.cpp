// reference_style_test.cpp — the drop-in C++ API end to end on the GPU.
//
// Written the way the reference's own tests (tests/*.cpp of
// Ligo04/lc_parallel_primitive) drive its classes: DeviceReduce, DeviceScan,
// DeviceRadixSort and DeviceSegmentReduce from <lcpp/parallel_primitive.h>,
// temp storage sized by the Get*TempStorageBytes queries, inputs built with
// std::mt19937(114521) + std::shuffle, expectations from std:: algorithms.
// Only the resource types differ (hipMalloc'd pointers wrapped in
// BufferView, a CommandList holding a hipStream_t).  Prints one line per case
// and exits non-zero on the first mismatch.  Built by __graft_entry__.build()
// (g++, links liblcpp_amd.so); run by tests/test_gpu_cpp_api.py.
//
// Built as a release build (NDEBUG): check() records a failed call's status
// instead of aborting, so the debug-stream case below can read last_status().
#define NDEBUG
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <functional>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <random>
#include <vector>

#include "lcpp/parallel_primitive.h"

using namespace luisa::parallel_primitive;

namespace {

hipStream_t g_stream = nullptr;
int g_failures = 0;

void hip_ok(hipError_t e, const char *what)
{
    if (e != hipSuccess) {
        std::fprintf(stderr, "HIP error in %s: %s\n", what, hipGetErrorString(e));
        std::exit(2);
    }
}

// Device buffer of T holding `n` elements (at least one byte allocated).
template <class T>
struct DevBuf {
    T *ptr = nullptr;
    size_t n = 0;
    explicit DevBuf(size_t count) : n(count) { hip_ok(hipMalloc(&ptr, std::max<size_t>(count * sizeof(T), 256)), "hipMalloc"); }
    DevBuf(const std::vector<T> &host) : DevBuf(host.size()) { upload(host); }
    ~DevBuf() { (void)hipFree(ptr); }
    DevBuf(const DevBuf &) = delete;
    DevBuf &operator=(const DevBuf &) = delete;
    void upload(const std::vector<T> &host)
    {
        hip_ok(hipMemcpy(ptr, host.data(), host.size() * sizeof(T), hipMemcpyHostToDevice), "upload");
    }
    std::vector<T> download(size_t count) const
    {
        hip_ok(hipStreamSynchronize(g_stream), "sync");
        std::vector<T> h(count);
        hip_ok(hipMemcpy(h.data(), ptr, count * sizeof(T), hipMemcpyDeviceToHost), "download");
        return h;
    }
    BufferView<T> view() const { return BufferView<T>{ptr, n}; }
};

// Temp storage as the reference tests make it: a uint buffer of
// bytes_to_uint_count(bytes) elements.
struct Temp {
    DevBuf<uint> buf;
    explicit Temp(size_t bytes) : buf(std::max<size_t>(1, bytes_to_uint_count(bytes))) {}
    BufferView<uint> view() const { return buf.view(); }
};

void expect(bool ok, const char *name)
{
    std::printf("%s %s\n", ok ? "ok" : "FAIL", name);
    if (!ok) ++g_failures;
}

std::vector<int> shuffled(int n)
{
    std::vector<int> a(n);
    std::iota(a.begin(), a.end(), 0);
    std::mt19937 rng(114521);
    std::shuffle(a.begin(), a.end(), rng);
    return a;
}

void test_reduce()
{
    CommandList cmdlist{g_stream};
    Device device{0};
    DeviceReduce<> reducer;
    reducer.create(device);

    bool ok = true;
    for (int k = 0; k < 24 && ok; ++k) {  // N ones, N = 2^k + 1
        const size_t n = (size_t(1) << k) + 1;
        DevBuf<uint> in(std::vector<uint>(n, 1u));
        DevBuf<uint> out(1);
        Temp temp(DeviceReduce<>::GetTempStorageBytes<uint>(n));
        reducer.Sum(cmdlist, temp.view(), in.view(), out.view(), n);
        ok = out.download(1)[0] == n;
    }
    expect(ok, "DeviceReduce::Sum ones 2^k+1");

    const std::vector<int> a = shuffled(1 << 12);
    DevBuf<int> in(a);
    DevBuf<int> out(1);
    DevBuf<uint> idx(1);
    Temp temp(std::max(DeviceReduce<>::GetTempStorageBytes<int>(a.size()),
                       DeviceReduce<>::GetArgTempStorageBytes<int>(a.size())));
    reducer.Min(cmdlist, temp.view(), in.view(), out.view(), a.size());
    expect(out.download(1)[0] == *std::min_element(a.begin(), a.end()), "DeviceReduce::Min shuffled");
    reducer.Max(cmdlist, temp.view(), in.view(), out.view(), a.size());
    expect(out.download(1)[0] == *std::max_element(a.begin(), a.end()), "DeviceReduce::Max shuffled");
    reducer.Sum(cmdlist, temp.view(), in.view(), out.view(), a.size());
    expect(out.download(1)[0] == std::accumulate(a.begin(), a.end(), 0), "DeviceReduce::Sum shuffled");
    reducer.Reduce(cmdlist, temp.view(), in.view(), out.view(), a.size(), SumOp{}, 1000);
    expect(out.download(1)[0] == std::accumulate(a.begin(), a.end(), 1000), "DeviceReduce::Reduce SumOp init 1000");
    reducer.Reduce(cmdlist, temp.view(), in.view(), out.view(), a.size(), MinOp{}, -7);
    expect(out.download(1)[0] == -7, "DeviceReduce::Reduce MinOp init below every element");
    reducer.Reduce(cmdlist, temp.view(), in.view(), out.view(), a.size(), MaxOp{}, 100);
    expect(out.download(1)[0] == *std::max_element(a.begin(), a.end()), "DeviceReduce::Reduce MaxOp");
    reducer.ArgMax(cmdlist, temp.view(), in.view(), out.view(), idx.view(), a.size());
    expect(idx.download(1)[0] == uint(std::max_element(a.begin(), a.end()) - a.begin()), "DeviceReduce::ArgMax shuffled");
    reducer.ArgMin(cmdlist, temp.view(), in.view(), out.view(), idx.view(), a.size());
    expect(idx.download(1)[0] == uint(std::min_element(a.begin(), a.end()) - a.begin()), "DeviceReduce::ArgMin shuffled");
    reducer.TransformReduce(cmdlist, temp.view(), in.view(), out.view(), a.size(), MaxOp{}, SquareOp{}, 0);
    expect(out.download(1)[0] == 4095 * 4095, "DeviceReduce::TransformReduce max of squares");

    // ReduceByKey: keys i / 100 over the shuffled values
    std::vector<int> keys(a.size());
    for (size_t i = 0; i < keys.size(); ++i) keys[i] = int(i / 100);
    const int segments = int((a.size() + 99) / 100);
    DevBuf<int> dk(keys), uk(segments), agg(segments);
    DevBuf<uint> runs(1);
    Temp t2(DeviceReduce<>::GetReduceByKeyTempStorageBytes<int, int>(a.size()));
    reducer.ReduceByKey(cmdlist, t2.view(), dk.view(), in.view(), uk.view(), agg.view(), runs.view(), SumOp{},
                        a.size());
    const std::vector<int> h_agg = agg.download(segments), h_uk = uk.download(segments);
    ok = runs.download(1)[0] == uint(segments);
    for (int s = 0; s < segments && ok; ++s) {
        const size_t b = size_t(s) * 100, e = std::min(b + 100, a.size());
        ok = h_uk[s] == s && h_agg[s] == std::accumulate(a.begin() + b, a.begin() + e, 0);
    }
    expect(ok, "DeviceReduce::ReduceByKey keys i/100");
}

void test_scan()
{
    CommandList cmdlist{g_stream};
    DeviceScan<> scanner;
    bool ok = true;
    for (int k = 0; k < 24 && ok; ++k) {  // ones, N = 2^k
        const size_t n = size_t(1) << k;
        DevBuf<uint> in(std::vector<uint>(n, 1u));
        DevBuf<uint> ex(n), inc(n);
        Temp temp(DeviceScan<>::GetTempStorageBytes<uint>(n));
        scanner.ExclusiveSum(cmdlist, temp.view(), in.view(), ex.view(), n);
        scanner.InclusiveSum(cmdlist, temp.view(), in.view(), inc.view(), n);
        const std::vector<uint> he = ex.download(n), hi = inc.download(n);
        for (size_t i = 0; i < n && ok; ++i) ok = he[i] == i && hi[i] == i + 1;
    }
    expect(ok, "DeviceScan::Exclusive/InclusiveSum ones 2^k");

    ok = true;
    for (int k = 0; k < 22 && ok; k += 3) {  // ExclusiveScan / InclusiveScan with an initial value
        const size_t n = (size_t(1) << k) + 7;
        std::vector<int> h(n);
        for (size_t i = 0; i < n; ++i) h[i] = int((i * 2654435761u) % 1001) - 500;
        DevBuf<int> in(h), ex(n), inc(n), mx(n);
        Temp temp(DeviceScan<>::GetTempStorageBytes<int>(n));
        scanner.ExclusiveScan(cmdlist, temp.view(), in.view(), ex.view(), n, SumOp{}, 1000);
        const std::vector<int> he = ex.download(n);
        scanner.InclusiveScan(cmdlist, temp.view(), in.view(), inc.view(), n, SumOp{}, -3);
        const std::vector<int> hi = inc.download(n);
        scanner.InclusiveScan(cmdlist, temp.view(), in.view(), mx.view(), n, MaxOp{}, 450);
        const std::vector<int> hm = mx.download(n);
        int run_ex = 1000, run_in = -3, run_mx = 450;
        for (size_t i = 0; i < n && ok; ++i) {
            ok = he[i] == run_ex;
            run_ex += h[i];
            run_in += h[i];
            run_mx = std::max(run_mx, h[i]);
            ok = ok && hi[i] == run_in && hm[i] == run_mx;
        }
    }
    expect(ok, "DeviceScan::ExclusiveScan / InclusiveScan (SumOp, MaxOp) with initial_value");

    ok = true;
    for (int k = 5; k < 21 && ok; ++k) {  // ExclusiveSumByKey: keys i / 100, ones -> i % 100
        const size_t n = size_t(1) << k;
        std::vector<int> keys(n);
        for (size_t i = 0; i < n; ++i) keys[i] = int(i / 100);
        DevBuf<int> dk(keys), dv(std::vector<int>(n, 1)), out(n);
        Temp temp(DeviceScan<>::GetScanByKeyTempStorageBytes<int, int>(n));
        scanner.ExclusiveSumByKey(cmdlist, temp.view(), dk.view(), dv.view(), out.view(), n);
        const std::vector<int> h = out.download(n);
        for (size_t i = 0; i < n && ok; ++i) ok = h[i] == int(i % 100);
    }
    expect(ok, "DeviceScan::ExclusiveSumByKey keys i/100");
}

void test_sort()
{
    CommandList cmdlist{g_stream};
    DeviceRadixSort<> sorter;
    bool ok = true;
    for (int k = 0; k < 21 && ok; ++k) {  // reversed keys, N = 2^k
        const uint n = 1u << k;
        std::vector<uint> keys(n);
        for (uint i = 0; i < n; ++i) keys[i] = n - 1 - i;
        DevBuf<uint> in(keys), out(n);
        Temp temp(DeviceRadixSort<>::GetSortKeysTempStorageBytes<uint>(n));
        sorter.SortKeys(cmdlist, temp.view(), in.view(), out.view(), n);
        const std::vector<uint> h = out.download(n);
        for (uint i = 0; i < n && ok; ++i) ok = h[i] == i;
    }
    expect(ok, "DeviceRadixSort::SortKeys reversed 2^k");

    const uint n = 1u << 16;
    std::vector<int> keys = shuffled(int(n));
    std::vector<float> vals(n);
    for (uint i = 0; i < n; ++i) vals[i] = float(keys[i]) * 0.5f;
    DevBuf<int> kin(keys), kout(n);
    DevBuf<float> vin(vals), vout(n);
    Temp temp(DeviceRadixSort<>::GetSortPairsTempStorageBytes<int, float>(n));
    sorter.SortPairs(cmdlist, temp.view(), kin.view(), kout.view(), vin.view(), vout.view(), n);
    std::vector<int> hk = kout.download(n);
    std::vector<float> hv = vout.download(n);
    ok = true;
    for (uint i = 0; i < n && ok; ++i) ok = hk[i] == int(i) && hv[i] == float(i) * 0.5f;
    expect(ok, "DeviceRadixSort::SortPairs shuffled");
    sorter.SortPairsDescending(cmdlist, temp.view(), kin.view(), kout.view(), vin.view(), vout.view(), n);
    hk = kout.download(n);
    hv = vout.download(n);
    ok = true;
    for (uint i = 0; i < n && ok; ++i) ok = hk[i] == int(n - 1 - i) && hv[i] == float(n - 1 - i) * 0.5f;
    expect(ok, "DeviceRadixSort::SortPairsDescending shuffled");

    std::vector<float> f(n);
    std::mt19937 rng(114521);
    std::uniform_real_distribution<float> dist(-100.f, 100.f);
    for (auto &x : f) x = dist(rng);
    DevBuf<float> fin(f), fout(n);
    Temp t2(DeviceRadixSort<>::GetSortKeysTempStorageBytes<float>(n));
    sorter.SortKeysDescending(cmdlist, t2.view(), fin.view(), fout.view(), n);
    std::vector<float> expect_f = f;
    std::sort(expect_f.begin(), expect_f.end(), std::greater<float>());
    expect(fout.download(n) == expect_f, "DeviceRadixSort::SortKeysDescending float");
}

void test_segment_reduce()
{
    CommandList cmdlist{g_stream};
    DeviceSegmentReduce<> reducer;
    const int n = 1024, per = 100;
    const std::vector<int> a = shuffled(n);
    const int segs = n / per + 1;
    std::vector<uint> b(segs), e(segs);
    for (int s = 0; s < segs; ++s) {
        b[s] = uint(s * per);
        e[s] = uint(std::min(s * per + per, n));
    }
    DevBuf<int> in(a), out(segs);
    DevBuf<uint> db(b), de(e), idx(segs);
    Temp temp(std::max<size_t>(DeviceSegmentReduce<>::GetTempStorageBytes<int>(n),
                               DeviceSegmentReduce<>::GetArgTempStorageBytes<int>(n, segs)));
    reducer.Sum(cmdlist, temp.view(), in.view(), out.view(), segs, db.view(), de.view());
    std::vector<int> h = out.download(segs);
    bool ok = true;
    for (int s = 0; s < segs && ok; ++s) ok = h[s] == std::accumulate(a.begin() + b[s], a.begin() + e[s], 0);
    expect(ok, "DeviceSegmentReduce::Sum segments of 100");

    reducer.ArgMax(cmdlist, temp.view(), in.view(), out.view(), idx.view(), segs, db.view(), de.view());
    h = out.download(segs);
    std::vector<uint> hi = idx.download(segs);
    ok = true;
    for (int s = 0; s < segs && ok; ++s) {
        const auto it = std::max_element(a.begin() + b[s], a.begin() + e[s]);
        ok = h[s] == *it && hi[s] == uint(it - (a.begin() + b[s]));
    }
    expect(ok, "DeviceSegmentReduce::ArgMax segments of 100");

    const int fixed_n = 1024, fixed_per = 32, fixed_segs = fixed_n / fixed_per;
    std::vector<int> ramp(fixed_n);
    std::iota(ramp.begin(), ramp.end(), 0);
    DevBuf<int> rin(ramp), rout(fixed_segs);
    reducer.Sum(cmdlist, temp.view(), rin.view(), rout.view(), fixed_segs, uint(fixed_per));
    h = rout.download(fixed_segs);
    ok = true;
    for (int s = 0; s < fixed_segs && ok; ++s)
        ok = h[s] == std::accumulate(ramp.begin() + s * fixed_per, ramp.begin() + (s + 1) * fixed_per, 0);
    expect(ok, "DeviceSegmentReduce::Sum fixed 32");

    const std::vector<int> sh = shuffled(fixed_n);
    DevBuf<int> sin(sh), sout(fixed_segs);
    DevBuf<uint> sidx(fixed_segs);
    reducer.ArgMin(cmdlist, temp.view(), sin.view(), sout.view(), sidx.view(), fixed_segs, uint(fixed_per));
    h = sout.download(fixed_segs);
    hi = sidx.download(fixed_segs);
    ok = true;
    for (int s = 0; s < fixed_segs && ok; ++s) {
        const auto it = std::min_element(sh.begin() + s * fixed_per, sh.begin() + (s + 1) * fixed_per);
        ok = h[s] == *it && hi[s] == uint(it - (sh.begin() + s * fixed_per));
    }
    expect(ok, "DeviceSegmentReduce::ArgMin fixed 32");
}

// create(device, &stream), as the reference's modules take a debug stream:
// every call is synchronized and its device status word read, so a
// look-back wait that gave up is reported by the call that caused it.  The
// give-up is forced with the test hook (a tile that never publishes; every
// kernel still drains).
void test_debug_stream()
{
    Device device{0};
    Stream debug{g_stream};
    CommandList cmdlist{g_stream};
    DeviceScan<> scanner;
    scanner.create(device, &debug);
    const size_t n = size_t(1) << 20;
    DevBuf<uint> in(std::vector<uint>(n, 1u)), out(n);
    Temp temp(DeviceScan<>::GetTempStorageBytes<uint>(n));
    scanner.ExclusiveSum(cmdlist, temp.view(), in.view(), out.view(), n);
    expect(scanner.last_status() == LCPP_OK, "debug stream: DeviceScan::ExclusiveSum status");
    lcpp_test_set_lookback_fault(3, 32);
    scanner.ExclusiveSum(cmdlist, temp.view(), in.view(), out.view(), n);
    lcpp_test_set_lookback_fault(0xFFFFFFFFu, 0);
    expect(scanner.last_status() == LCPP_ERR_LOOKBACK_TIMEOUT, "debug stream: withheld scan tile reported");
    scanner.ExclusiveSum(cmdlist, temp.view(), in.view(), out.view(), n);
    const std::vector<uint> h = out.download(n);
    bool ok = scanner.last_status() == LCPP_OK;
    for (size_t i = 0; i < n && ok; ++i) ok = h[i] == i;
    expect(ok, "debug stream: DeviceScan::ExclusiveSum after the fault");

    DeviceRadixSort<> sorter;
    sorter.create(device, &debug);
    const uint m = 1u << 20;
    std::vector<uint> keys(m);
    for (uint i = 0; i < m; ++i) keys[i] = (i * 2654435761u) ^ 0x5bd1e995u;
    DevBuf<uint> kin(keys), kout(m);
    Temp t2(DeviceRadixSort<>::GetSortKeysTempStorageBytes<uint>(m));
    lcpp_test_set_lookback_fault(9, 32);
    sorter.SortKeys(cmdlist, t2.view(), kin.view(), kout.view(), m);
    lcpp_test_set_lookback_fault(0xFFFFFFFFu, 0);
    expect(sorter.last_status() == LCPP_ERR_LOOKBACK_TIMEOUT, "debug stream: withheld sort tile reported");
    sorter.SortKeys(cmdlist, t2.view(), kin.view(), kout.view(), m);
    std::vector<uint> hk = kout.download(m);
    std::sort(keys.begin(), keys.end());
    expect(sorter.last_status() == LCPP_OK && hk == keys, "debug stream: DeviceRadixSort::SortKeys after the fault");
}

}  // namespace

int main()
{
    hip_ok(hipStreamCreate(&g_stream), "hipStreamCreate");
    test_reduce();
    test_scan();
    test_sort();
    test_segment_reduce();
    test_debug_stream();
    hip_ok(hipStreamDestroy(g_stream), "hipStreamDestroy");
    std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "PASSED", g_failures);
    return g_failures ? 1 : 0;
}
