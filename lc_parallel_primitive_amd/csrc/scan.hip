// scan.hip — DeviceScan::ExclusiveScan/InclusiveScan (Sum, Min, Max with an
// initial value) and ExclusiveSum/InclusiveSum for gfx950.
//
// Reference: device/device_scan.h:114-204, 349-411 (init kernel + one
// single-pass scan kernel), device/details/scan.h:59-147,
// device/details/single_pass_scan_operator.h:25-251 (decoupled look-back),
// block/detail/block_scan_warp.h, thread/thread_scan.h.
//
// MI355X design: single pass, 8N bytes (read N, write N elements).
//  * Tile = 256 threads x 16 vectors of 16 bytes = 64 KiB (16384 x 32-bit or
//    8192 x 64-bit elements).  Vector k of thread t holds elements
//    [k*256*V + t*V, +V) of the tile, so every load and store instruction
//    covers 4 KiB of contiguous memory.  The 16 chunks are scanned in place
//    without an LDS transpose: per chunk, a thread scan of its V elements, a
//    wave scan of the thread totals and the wave offset folded in; only the
//    4 x 16 wave totals go through LDS.  A look-back wait costs several
//    microseconds under full HBM load, during which the tile sits in
//    registers, so the tile is as large as the register file allows at ~4
//    workgroups per CU (~100 VGPRs).
//  * Loads and stores are raw-buffer instructions on a resource that ends at
//    the tile's last valid byte: a ragged last tile and unaligned pointers take
//    the element-wise path with no per-element bounds logic.  That path keeps
//    the whole offset in the VGPR operand, which the range check covers (the
//    scalar offset operand is used only by full tiles).
//  * Tile id = blockIdx.x, as the reference (scan.h:76).  Workgroups are
//    dispatched in id order, so every predecessor of a waiting tile is
//    already resident or finished.  (A dynamic ticket costs one same-address
//    atomic per tile, ~11 ns each, which serialises the whole grid.)
//  * Look-back (lookback.hpp): one self-validating packed word per tile
//    (two for 64-bit types) written with agent-scope relaxed stores
//    (release/acquire pairs cost an L2 write-back/invalidate per publish on
//    this part: 7.8 ms for 2^27 x 64-bit); wave 0 polls 16 predecessors at
//    once and stops at the nearest INCLUSIVE.
#include <cstring>

#include "lookback.hpp"

namespace lcpp {
namespace {

constexpr int kScanBlock = 256;
// 16-byte vectors per thread per tile. Measured at 2^28 elements (us per
// call, 16 / 20 / 24 vectors): exclusive u32 372 / 362 / 368, exclusive i64
// 744 / 722 / 735; inclusive u32 374 / 377 / 398, inclusive f32 371 / 374 /
// 364, inclusive i64 741 / 787 / 855. The inclusive integer kernels keep each
// chunk's wave prefix live until the second pass (integer adds reassociate),
// so they reach 152 VGPRs (3 workgroups per SIMD) at 20 vectors where the
// exclusive ones stay at 122 (4 workgroups).
template <class T, bool INCLUSIVE>
constexpr int scan_vecs()
{
    return !INCLUSIVE ? 20 : (std::is_same<T, float>::value ? 24 : 16);
}
template <class T, bool INCLUSIVE>
constexpr uint32_t scan_tile()
{
    return kScanBlock * scan_vecs<T, INCLUSIVE>() * (16 / sizeof(T));
}

// Temp layout: the status header, then packed look-back words, 8 bytes per
// tile (32-bit T) or 16 bytes per tile (64-bit T).  The query covers the
// smaller of the two tiles.
template <class T, bool INCLUSIVE>
uint64_t scan_tiles(uint64_t n)
{
    return n ? ceil_div(n, scan_tile<T, INCLUSIVE>()) : 0;
}
template <class T>
uint64_t scan_temp_bytes(uint64_t n)
{
    const uint64_t tiles = std::max(scan_tiles<T, false>(n), scan_tiles<T, true>(n));
    return tiles ? kStatusBytes + align_up(tiles * (sizeof(T) == 4 ? 8 : 16), 256) : 0;
}

// 4-byte integer kernels are held to 128 VGPRs (4 workgroups per SIMD):
// with the DPP wave scan the compiler otherwise takes 132 (exclusive u32, 20
// vectors; the scan slows from 357 to 367 us) or 134 (inclusive).  The
// inclusive float kernel (24 vectors) would spill, and the 64-bit kernels
// stay under 128 anyway but measured 3 % slower with the limit.
template <class T, bool INCLUSIVE>
constexpr int scan_min_waves()
{
    return sizeof(T) == 4 && !(INCLUSIVE && std::is_same<T, float>::value) ? 4 : 1;
}
// out[i] = op(init, in[0..i)) (exclusive) or op(init, in[0..i]) (inclusive);
// op is SumOp, MinOp or MaxOp (commutative: the look-back folds windows as
// trees).  The Sum scans are init = 0.
template <class T, bool INCLUSIVE, class Op>
__global__ __launch_bounds__(kScanBlock) __attribute__((amdgpu_waves_per_eu(scan_min_waves<T, INCLUSIVE>())))
void scan_kernel(const T *__restrict__ in, T *__restrict__ out, uint64_t n, uint64_t *words, int vec_ok, T init,
                 WaitCtl ctl)
{
    constexpr int V = 16 / sizeof(T);
    constexpr int K = scan_vecs<T, INCLUSIVE>();
    constexpr uint32_t TILE = scan_tile<T, INCLUSIVE>();
    constexpr uint32_t CHUNK = kScanBlock * 16;  // bytes per vector instruction
    constexpr int W = kScanBlock / kWave;
    __shared__ T s_wtot[K][W];
    __shared__ T s_prefix;

    Op op;
    const T id = Op::template identity<T>();
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint64_t base = (uint64_t)tile * TILE;
    const uint32_t valid = n - base < TILE ? (uint32_t)(n - base) : TILE;
    const bool fast = valid == TILE && vec_ok;
    const __amdgpu_buffer_rsrc_t rin = make_rsrc(in + base, valid * (uint32_t)sizeof(T));
    const __amdgpu_buffer_rsrc_t rout = make_rsrc(out + base, valid * (uint32_t)sizeof(T));

    T x[K][V];
    if (fast) {
#pragma unroll
        for (int k = 0; k < K; ++k) unpack16<T>(buf_ld16_nt(rin, tid * 16, k * CHUNK), x[k]);
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int j = 0; j < V; ++j) x[k][j] = buf_ld_elem<T>(rin, k * CHUNK + tid * 16 + j * sizeof(T), 0);
    }

    // Per chunk: thread scan in place, wave scan of the thread totals, wave
    // offset folded in; the wave totals go to LDS.
#pragma unroll
    for (int k = 0; k < K; ++k) {
        T r;
        if constexpr (INCLUSIVE) {
#pragma unroll
            for (int j = 1; j < V; ++j) x[k][j] = op(x[k][j - 1], x[k][j]);
            r = x[k][V - 1];
        } else {
            r = x[k][0];
            x[k][0] = id;
#pragma unroll
            for (int j = 1; j < V; ++j) {
                const T v = x[k][j];
                x[k][j] = r;
                r = op(r, v);
            }
        }
        const T inc = wave_inclusive_scan(r, op);
        const T wex = wave_shr1(inc, id);
        if (lane == kWave - 1) s_wtot[k][wave] = inc;
#pragma unroll
        for (int j = 0; j < V; ++j) x[k][j] = op(wex, x[k][j]);
    }
    __syncthreads();
    if (wave == 0) {
        T agg = id;
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int w = 0; w < W; ++w) agg = op(agg, s_wtot[k][w]);
        const T ex = lb_scan_tile_init(words, tile, agg, op, id, init, ctl);
        if (lane == 0) s_prefix = ex;
    }
    __syncthreads();

    // out = tile prefix + (chunks before k) + (waves before this one in k) + x
    T run = s_prefix;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        T pre = id, tot = id;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const T v = s_wtot[k][w];
            if ((uint32_t)w < wave) pre = op(pre, v);
            tot = op(tot, v);
        }
        const T b = op(run, pre);
#pragma unroll
        for (int j = 0; j < V; ++j) x[k][j] = op(b, x[k][j]);
        run = op(run, tot);
    }
    if (fast) {
#pragma unroll
        for (int k = 0; k < K; ++k) buf_st16_nt(rout, tid * 16, k * CHUNK, pack16<T>(x[k]));
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int j = 0; j < V; ++j) buf_st_elem<T>(rout, k * CHUNK + tid * 16 + j * sizeof(T), 0, x[k][j]);
    }
}

// Enqueue one scan whose status header + look-back words start at `head`
// (zeroed here by a fill kernel, so the call can be graph-captured).
// `instrument`: bracket the launches with the profiling events when enabled.
template <class T, class Op>
int scan_run(bool inclusive, uint64_t *head, const T *in, T *out, uint64_t n, uint64_t tiles, T init, hipStream_t s,
             bool instrument)
{
    uint64_t *words = head + kStatusBytes / 8;
    const uint64_t nwords = kStatusBytes / 8 + tiles * (sizeof(T) == 4 ? 1 : 2);
    const WaitCtl ctl = wait_ctl(reinterpret_cast<uint32_t *>(head));
    const int vec_ok = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (instrument) {
        if (lb_init(head, nwords, s, "scan_init") != LCPP_OK) return LCPP_ERR_HIP;
        if (inclusive)
            LCPP_LAUNCH("scan_inclusive", s,
                        (scan_kernel<T, true, Op><<<(uint32_t)tiles, kScanBlock, 0, s>>>(in, out, n, words, vec_ok,
                                                                                          init, ctl)));
        else
            LCPP_LAUNCH("scan_exclusive", s,
                        (scan_kernel<T, false, Op><<<(uint32_t)tiles, kScanBlock, 0, s>>>(in, out, n, words, vec_ok,
                                                                                           init, ctl)));
    } else {
        const uint64_t g = ceil_div(nwords, 256);
        lb_init_kernel<<<(uint32_t)(g < 1024 ? g : 1024), 256, 0, s>>>(head, nwords);
        if (hipGetLastError() != hipSuccess) return LCPP_ERR_HIP;
        if (inclusive)
            scan_kernel<T, true, Op><<<(uint32_t)tiles, kScanBlock, 0, s>>>(in, out, n, words, vec_ok, init, ctl);
        else
            scan_kernel<T, false, Op><<<(uint32_t)tiles, kScanBlock, 0, s>>>(in, out, n, words, vec_ok, init, ctl);
    }
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

// `init_`: a host value of type T, or NULL for the operator's identity.
template <class T, class Op>
int scan_launch(bool inclusive, void *temp, size_t temp_bytes, const void *in_, void *out_, uint64_t n,
                const void *init_, hipStream_t s)
{
    if (n == 0) return LCPP_OK;
    const T *in = static_cast<const T *>(in_);
    T *out = static_cast<T *>(out_);
    if (!in || !out) return LCPP_ERR_INVALID_ARG;
    const uint64_t tiles = inclusive ? scan_tiles<T, true>(n) : scan_tiles<T, false>(n);
    if (tiles > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;
    if (temp_bytes < scan_temp_bytes<T>(n)) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    T init = Op::template identity<T>();
    if (init_) memcpy(&init, init_, sizeof(T));
    return scan_run<T, Op>(inclusive, static_cast<uint64_t *>(temp), in, out, n, tiles, init, s, true);
}

template <class T>
int scan_op_dispatch(bool inclusive, lcpp_reduce_op op, void *temp, size_t tb, const void *in, void *out, uint64_t n,
                     const void *init, hipStream_t s)
{
    switch (op) {
    case LCPP_OP_SUM: return scan_launch<T, SumOp>(inclusive, temp, tb, in, out, n, init, s);
    case LCPP_OP_MIN: return scan_launch<T, MinOp>(inclusive, temp, tb, in, out, n, init, s);
    case LCPP_OP_MAX: return scan_launch<T, MaxOp>(inclusive, temp, tb, in, out, n, init, s);
    default: return LCPP_ERR_INVALID_ARG;
    }
}

int scan_dispatch(bool inclusive, lcpp_dtype t, lcpp_reduce_op op, void *temp, size_t tb, const void *in, void *out,
                  uint64_t n, const void *init, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (t) {
    case LCPP_INT32: return scan_op_dispatch<int32_t>(inclusive, op, temp, tb, in, out, n, init, s);
    case LCPP_UINT32: return scan_op_dispatch<uint32_t>(inclusive, op, temp, tb, in, out, n, init, s);
    case LCPP_FLOAT32: return scan_op_dispatch<float>(inclusive, op, temp, tb, in, out, n, init, s);
    case LCPP_INT64: return scan_op_dispatch<int64_t>(inclusive, op, temp, tb, in, out, n, init, s);
    case LCPP_UINT64: return scan_op_dispatch<uint64_t>(inclusive, op, temp, tb, in, out, n, init, s);
    case LCPP_FLOAT64: return scan_op_dispatch<double>(inclusive, op, temp, tb, in, out, n, init, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

}  // namespace
}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_scan_temp_bytes(lcpp_dtype t, uint64_t n, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    // sizes the scans reject (more than 2^32-1 tiles) are rejected here too
    switch (t) {
    case LCPP_INT32: case LCPP_UINT32: case LCPP_FLOAT32:
        if (scan_tiles<uint32_t, false>(n) > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;
        *bytes = scan_temp_bytes<uint32_t>(n);
        return LCPP_OK;
    case LCPP_INT64: case LCPP_UINT64: case LCPP_FLOAT64:
        if (scan_tiles<uint64_t, false>(n) > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;
        *bytes = scan_temp_bytes<uint64_t>(n);
        return LCPP_OK;
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

extern "C" int lcpp_scan_exclusive_sum(lcpp_dtype t, void *temp, size_t tb, const void *in,
                                       void *out, uint64_t n, void *stream)
{
    return scan_dispatch(false, t, LCPP_OP_SUM, temp, tb, in, out, n, nullptr, stream);
}

extern "C" int lcpp_scan_inclusive_sum(lcpp_dtype t, void *temp, size_t tb, const void *in,
                                       void *out, uint64_t n, void *stream)
{
    return scan_dispatch(true, t, LCPP_OP_SUM, temp, tb, in, out, n, nullptr, stream);
}

extern "C" int lcpp_scan_exclusive(lcpp_dtype t, lcpp_reduce_op op, void *temp, size_t tb, const void *in, void *out,
                                   uint64_t n, const void *init, void *stream)
{
    return scan_dispatch(false, t, op, temp, tb, in, out, n, init, stream);
}

extern "C" int lcpp_scan_inclusive(lcpp_dtype t, lcpp_reduce_op op, void *temp, size_t tb, const void *in, void *out,
                                   uint64_t n, const void *init, void *stream)
{
    return scan_dispatch(true, t, op, temp, tb, in, out, n, init, stream);
}

// ---------------------------------------------------------------- no-allocation variant
// lcpp_scan_exclusive_sum_noalloc: the status header and look-back words live
// in `scratch`, a file-scope device array (each GPU the library runs on holds
// its own copy until the process ends), so the call allocates nothing.  Host
// code never uses the array's name as an address: its device address is
// fetched once per device with hipGetSymbolAddress and kept per device.
// Calls that overlap on one GPU share the array and race.
namespace {
constexpr uint64_t kNoAllocWords = kStatusBytes / 8 + 65536;  // 512 KiB of look-back words
}  // namespace
static __device__ __align__(256) uint64_t scratch[kNoAllocWords];

namespace {
std::atomic<uint64_t *> g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch` (looked up on its first use).
int scratch_ptr(uint64_t **out)
{
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return LCPP_ERR_HIP;
    uint64_t *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        void *q = nullptr;
        if (hipGetSymbolAddress(&q, HIP_SYMBOL(scratch)) != hipSuccess || !q) return LCPP_ERR_HIP;
        p = static_cast<uint64_t *>(q);
        g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
    *out = p;
    return LCPP_OK;
}

template <class T>
int scan_noalloc(const void *in_, void *out_, uint64_t n, hipStream_t s)
{
    if (n == 0) return LCPP_OK;
    const T *in = static_cast<const T *>(in_);
    T *out = static_cast<T *>(out_);
    if (!in || !out) return LCPP_ERR_INVALID_ARG;
    const uint64_t tiles = scan_tiles<T, false>(n);
    if (kStatusBytes / 8 + tiles * (sizeof(T) == 4 ? 1 : 2) > kNoAllocWords) return LCPP_ERR_SIZE_LIMIT;
    uint64_t *head = nullptr;
    if (scratch_ptr(&head) != LCPP_OK) return LCPP_ERR_HIP;
    return scan_run<T, SumOp>(false, head, in, out, n, tiles, T(0), s, false);
}
}  // namespace

extern "C" int lcpp_scan_exclusive_sum_noalloc(lcpp_dtype t, const void *in, void *out, uint64_t n, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (t) {
    case LCPP_INT32: return scan_noalloc<int32_t>(in, out, n, s);
    case LCPP_UINT32: return scan_noalloc<uint32_t>(in, out, n, s);
    case LCPP_FLOAT32: return scan_noalloc<float>(in, out, n, s);
    case LCPP_INT64: return scan_noalloc<int64_t>(in, out, n, s);
    case LCPP_UINT64: return scan_noalloc<uint64_t>(in, out, n, s);
    case LCPP_FLOAT64: return scan_noalloc<double>(in, out, n, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}
