// scan.hip — DeviceScan::ExclusiveSum/InclusiveSum for gfx950.
//
// Reference: device/device_scan.h:114-204, 349-411 (init kernel + one
// single-pass scan kernel), device/details/scan.h:59-147,
// device/details/single_pass_scan_operator.h:25-251 (decoupled look-back),
// block/detail/block_scan_warp.h, thread/thread_scan.h.
//
// MI355X design: single pass, 8N bytes.
//  * Tile = 256 threads x 4 vectors of 16 bytes (4096 x 32-bit or 2048 x
//    64-bit elements).  Vector k of thread t holds elements
//    [k*256*V + t*V, +V) of the tile, so every load and store instruction
//    covers 4 KiB of contiguous memory; no LDS transpose is needed because
//    the four chunks are scanned together: each thread scans its vectors,
//    the wave scans the four vector totals at once, one barrier exchanges
//    wave totals, and each chunk gets the chunk prefix of the chunks before
//    it.
//  * Tile order comes from a dynamic ticket (the reference uses the static
//    block id, scan.h:76, which relies on in-order dispatch).
//  * Look-back state for 32-bit types is one packed 64-bit word per tile,
//    {value:32 | status:32}, published and polled with agent-scope atomics
//    (the reference keeps status and value in separate arrays with no
//    ordering between them, single_pass_scan_operator.h:81-93).  64-bit
//    types use a status word plus separate PARTIAL / INCLUSIVE value arrays
//    with release/acquire ordering.
//  * Wave 0 polls a window of 64 predecessors per step (64-lane ballots),
//    combines values up to the nearest INCLUSIVE one, slides by 64.
#include "common.hpp"

namespace lcpp {
namespace {

constexpr int kScanBlock = 256;
constexpr int kScanVecs = 4;
constexpr uint32_t kStInvalid = 0, kStPartial = 1, kStInclusive = 2;

template <class T>
constexpr uint32_t scan_tile()
{
    return kScanBlock * kScanVecs * (16 / sizeof(T));
}

// Temp layout (offsets 256-byte aligned):
//   [0]      uint32 ticket
//   [256]    32-bit T: uint64 words[tiles]
//            64-bit T: uint32 status[tiles] | T partial[tiles] | T inclusive[tiles]
struct ScanLayout {
    uint64_t tiles;
    uint64_t status_off, partial_off, incl_off, total;
};

template <class T>
ScanLayout scan_layout(uint64_t n)
{
    ScanLayout L;
    L.tiles = n ? ceil_div(n, scan_tile<T>()) : 0;
    L.status_off = 256;
    if constexpr (sizeof(T) == 4) {
        L.partial_off = L.incl_off = 0;
        L.total = L.status_off + align_up(L.tiles * 8, 256);
    } else {
        L.partial_off = L.status_off + align_up(L.tiles * 4, 256);
        L.incl_off = L.partial_off + align_up(L.tiles * 8, 256);
        L.total = L.incl_off + align_up(L.tiles * 8, 256);
    }
    return L;
}

template <class T>
struct LookbackState {
    uint32_t *ticket;
    uint32_t *status;     // 64-bit T
    uint64_t *words;      // 32-bit T: packed {value, status}
    uint64_t *partial;    // 64-bit T raw bits
    uint64_t *inclusive;  // 64-bit T raw bits
};

template <class T>
__device__ __forceinline__ uint64_t to_bits(T v)
{
    if constexpr (sizeof(T) == 4) return __builtin_bit_cast(uint32_t, v);
    else return __builtin_bit_cast(uint64_t, v);
}
template <class T>
__device__ __forceinline__ T from_bits(uint64_t b)
{
    if constexpr (sizeof(T) == 4) return __builtin_bit_cast(T, (uint32_t)b);
    else return __builtin_bit_cast(T, b);
}

template <class T>
__device__ __forceinline__ void publish(const LookbackState<T> &st, uint32_t tile, T v, uint32_t status)
{
    if constexpr (sizeof(T) == 4) {
        st_relaxed(&st.words[tile], (to_bits(v) << 32) | status);
    } else {
        uint64_t *arr = status == kStPartial ? st.partial : st.inclusive;
        st_relaxed(&arr[tile], to_bits(v));
        st_release(&st.status[tile], status);
    }
}

// Poll predecessor j (j < 0 reads as INCLUSIVE identity).  Returns status,
// writes the matching value.
template <class T>
__device__ __forceinline__ uint32_t poll(const LookbackState<T> &st, int64_t j, T &v)
{
    if (j < 0) {
        v = T(0);
        return kStInclusive;
    }
    if constexpr (sizeof(T) == 4) {
        uint64_t w = ld_relaxed(&st.words[j]);
        v = from_bits<T>(w >> 32);
        return (uint32_t)w;
    } else {
        uint32_t s = ld_acquire(&st.status[j]);
        if (s == kStPartial) v = from_bits<T>(ld_relaxed(&st.partial[j]));
        else if (s == kStInclusive) v = from_bits<T>(ld_relaxed(&st.inclusive[j]));
        else v = T(0);
        return s;
    }
}

// Decoupled look-back, executed by all 64 lanes of one wave.  Returns the
// exclusive prefix of `tile` in every lane and publishes INCLUSIVE.
template <class T>
__device__ T lookback(const LookbackState<T> &st, uint32_t tile, T agg)
{
    SumOp op;
    const uint32_t lane = lane_id();
    if (tile == 0) {
        if (lane == 0) publish(st, 0, agg, kStInclusive);
        return T(0);
    }
    if (lane == 0) publish(st, tile, agg, kStPartial);
    T excl = T(0);
    int64_t top = (int64_t)tile - 1;
    for (;;) {
        const int64_t j = top - (int64_t)lane;
        T v;
        uint32_t s = poll(st, j, v);
        for (uint32_t spins = 0; ballot(s == kStInvalid) != 0 && spins < kSpinLimit; ++spins) {
            __builtin_amdgcn_s_sleep(1);
            if (s == kStInvalid) s = poll(st, j, v);
        }
        const uint64_t incl = ballot(s == kStInclusive);
        const uint32_t stop = incl ? (uint32_t)__builtin_ctzll(incl) : 63u;
        T contrib = lane <= stop ? v : T(0);
        excl = op(excl, wave_allreduce(contrib, op));
        if (incl) break;
        top -= kWave;
    }
    if (lane == 0) publish(st, tile, op(excl, agg), kStInclusive);
    return excl;
}

template <class T>
__global__ __launch_bounds__(256) void scan_init_kernel(LookbackState<T> st, uint64_t tiles)
{
    const uint64_t i0 = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    if (i0 == 0) st.ticket[0] = 0;
    for (uint64_t i = i0; i < tiles; i += stride) {
        if constexpr (sizeof(T) == 4) st.words[i] = 0;
        else st.status[i] = 0;
    }
}

template <class T, bool INCLUSIVE>
__global__ __launch_bounds__(kScanBlock) void scan_kernel(const T *__restrict__ in,
                                                          T *__restrict__ out, uint64_t n,
                                                          LookbackState<T> st, int vec_ok)
{
    constexpr int V = 16 / sizeof(T);
    constexpr int K = kScanVecs;
    constexpr uint32_t TILE = scan_tile<T>();
    constexpr int W = kScanBlock / kWave;
    __shared__ uint32_t s_tile;
    __shared__ T s_wtot[K][W];
    __shared__ T s_prefix;

    SumOp op;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;

    if (tid == 0) s_tile = ticket(st.ticket);
    __syncthreads();
    const uint32_t tile = s_tile;
    const uint64_t base = (uint64_t)tile * TILE;
    const bool full = base + TILE <= n;

    T x[K][V];
    if (full && vec_ok) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            unpack16<T>(ld16_nt(in + base + (uint64_t)k * kScanBlock * V + (uint64_t)tid * V), x[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int j = 0; j < V; ++j) {
                const uint64_t e = base + (uint64_t)k * kScanBlock * V + (uint64_t)tid * V + j;
                x[k][j] = e < n ? in[e] : T(0);
            }
    }

    // thread-local inclusive scan of each vector
    T agg[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int j = 1; j < V; ++j) x[k][j] = op(x[k][j - 1], x[k][j]);
        agg[k] = x[k][V - 1];
    }
    // wave scans of the four vector totals
    T wexcl[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        T inc = wave_inclusive_scan(agg[k], op);
        T up = shfl_up(inc, 1);
        wexcl[k] = lane == 0 ? T(0) : up;
        if (lane == kWave - 1) s_wtot[k][wave] = inc;
    }
    __syncthreads();
    T base_k[K];
    T run = T(0);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        T tot = T(0), pre = T(0);
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const T v = s_wtot[k][w];
            if ((uint32_t)w < wave) pre = op(pre, v);
            tot = op(tot, v);
        }
        base_k[k] = op(op(run, pre), wexcl[k]);
        run = op(run, tot);
    }
    if (wave == 0) {
        const T ex = lookback(st, tile, run);
        if (lane == 0) s_prefix = ex;
    }
    __syncthreads();
    const T prefix = s_prefix;

    T y[K][V];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const T b = op(prefix, base_k[k]);
#pragma unroll
        for (int j = 0; j < V; ++j) {
            if constexpr (INCLUSIVE) y[k][j] = op(b, x[k][j]);
            else y[k][j] = j == 0 ? b : op(b, x[k][j - 1]);
        }
    }
    if (full && vec_ok) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const u32x4 v = pack16<T>(y[k]);
            st16_nt(out + base + (uint64_t)k * kScanBlock * V + (uint64_t)tid * V, v);
        }
    } else {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int j = 0; j < V; ++j) {
                const uint64_t e = base + (uint64_t)k * kScanBlock * V + (uint64_t)tid * V + j;
                if (e < n) out[e] = y[k][j];
            }
    }
}

template <class T>
int scan_launch(bool inclusive, void *temp, size_t temp_bytes, const void *in_, void *out_,
                uint64_t n, hipStream_t s)
{
    if (n == 0) return LCPP_OK;
    const T *in = static_cast<const T *>(in_);
    T *out = static_cast<T *>(out_);
    if (!in || !out) return LCPP_ERR_INVALID_ARG;
    const ScanLayout L = scan_layout<T>(n);
    if (L.tiles > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;
    if (temp_bytes < L.total) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    char *t = static_cast<char *>(temp);
    LookbackState<T> st{};
    st.ticket = reinterpret_cast<uint32_t *>(t);
    if constexpr (sizeof(T) == 4) {
        st.words = reinterpret_cast<uint64_t *>(t + L.status_off);
    } else {
        st.status = reinterpret_cast<uint32_t *>(t + L.status_off);
        st.partial = reinterpret_cast<uint64_t *>(t + L.partial_off);
        st.inclusive = reinterpret_cast<uint64_t *>(t + L.incl_off);
    }
    const uint32_t init_grid = (uint32_t)(ceil_div(L.tiles, 256) < 1024 ? ceil_div(L.tiles, 256) : 1024);
    LCPP_LAUNCH("scan_init", s, scan_init_kernel<T><<<init_grid ? init_grid : 1, 256, 0, s>>>(st, L.tiles));
    LCPP_CHECK_LAUNCH();
    const int vec_ok = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (inclusive)
        LCPP_LAUNCH("scan_inclusive", s,
                    scan_kernel<T, true><<<(uint32_t)L.tiles, kScanBlock, 0, s>>>(in, out, n, st, vec_ok));
    else
        LCPP_LAUNCH("scan_exclusive", s,
                    scan_kernel<T, false><<<(uint32_t)L.tiles, kScanBlock, 0, s>>>(in, out, n, st, vec_ok));
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

int scan_dispatch(bool inclusive, lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                  uint64_t n, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (t) {
    case LCPP_INT32: return scan_launch<int32_t>(inclusive, temp, tb, in, out, n, s);
    case LCPP_UINT32: return scan_launch<uint32_t>(inclusive, temp, tb, in, out, n, s);
    case LCPP_FLOAT32: return scan_launch<float>(inclusive, temp, tb, in, out, n, s);
    case LCPP_INT64: return scan_launch<int64_t>(inclusive, temp, tb, in, out, n, s);
    case LCPP_UINT64: return scan_launch<uint64_t>(inclusive, temp, tb, in, out, n, s);
    case LCPP_FLOAT64: return scan_launch<double>(inclusive, temp, tb, in, out, n, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

}  // namespace
}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_scan_temp_bytes(lcpp_dtype t, uint64_t n, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    switch (t) {
    case LCPP_INT32: case LCPP_UINT32: case LCPP_FLOAT32: *bytes = scan_layout<uint32_t>(n).total; return LCPP_OK;
    case LCPP_INT64: case LCPP_UINT64: case LCPP_FLOAT64: *bytes = scan_layout<uint64_t>(n).total; return LCPP_OK;
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

extern "C" int lcpp_scan_exclusive_sum(lcpp_dtype t, void *temp, size_t tb, const void *in,
                                       void *out, uint64_t n, void *stream)
{
    return scan_dispatch(false, t, temp, tb, in, out, n, stream);
}

extern "C" int lcpp_scan_inclusive_sum(lcpp_dtype t, void *temp, size_t tb, const void *in,
                                       void *out, uint64_t n, void *stream)
{
    return scan_dispatch(true, t, temp, tb, in, out, n, stream);
}
