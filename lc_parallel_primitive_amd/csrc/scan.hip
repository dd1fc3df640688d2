// scan.hip — DeviceScan::ExclusiveSum/InclusiveSum for gfx950.
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
//    the element-wise path with no per-element bounds logic.
//  * Tile id = blockIdx.x, as the reference (scan.h:76).  Workgroups are
//    dispatched in id order, so every predecessor of a waiting tile is
//    already resident or finished.  (A dynamic ticket costs one same-address
//    atomic per tile, ~11 ns each, which serialises the whole grid.)
//  * Look-back state per tile is self-validating packed words written with
//    agent-scope relaxed stores: 32-bit types use one 64-bit word
//    {value:32 | status:32}; 64-bit types use two words {value_lo | status}
//    and {value_hi | status}, read as valid only when both statuses agree
//    (each status is written once per word, so agreeing statuses come from
//    one publish).  The reference keeps status and value in separate arrays
//    with no ordering between them (single_pass_scan_operator.h:81-93);
//    release/acquire pairs instead cost an L2 write-back/invalidate per
//    publish on this part (7.8 ms for 2^27 x 64-bit).
//  * Wave 0 issues all 64 predecessor polls at once (branch-free, so they
//    are in flight together), stops at the nearest INCLUSIVE and only waits
//    for predecessors closer than it.
#include "common.hpp"

namespace lcpp {
namespace {

constexpr int kScanBlock = 256;
constexpr int kScanVecs = 16;
constexpr uint32_t kStInvalid = 0, kStPartial = 1, kStInclusive = 2;

template <class T>
constexpr uint32_t scan_tile()
{
    return kScanBlock * kScanVecs * (16 / sizeof(T));
}

// Temp layout: packed look-back words, 8 bytes per tile (32-bit T) or 16
// bytes per tile (64-bit T).
template <class T>
uint64_t scan_tiles(uint64_t n)
{
    return n ? ceil_div(n, scan_tile<T>()) : 0;
}
template <class T>
uint64_t scan_temp_bytes(uint64_t n)
{
    return align_up(scan_tiles<T>(n) * (sizeof(T) == 4 ? 8 : 16), 256);
}

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
__device__ __forceinline__ void publish(uint64_t *words, uint32_t tile, T v, uint32_t status)
{
    const uint64_t b = to_bits(v);
    if constexpr (sizeof(T) == 4) {
        st_relaxed(&words[tile], (b << 32) | status);
    } else {
        st_relaxed(&words[2 * (uint64_t)tile], (uint64_t)((b << 32) | status));
        st_relaxed(&words[2 * (uint64_t)tile + 1], (uint64_t)((b & 0xFFFFFFFF00000000ull) | status));
    }
}

// Decoupled look-back, executed by all 64 lanes of one wave.  Returns the
// exclusive prefix of `tile` in every lane and publishes INCLUSIVE.
template <class T>
__device__ T lookback(uint64_t *words, uint32_t tile, T agg)
{
    SumOp op;
    const uint32_t lane = lane_id();
    if (tile == 0) {
        if (lane == 0) publish(words, 0, agg, kStInclusive);
        return T(0);
    }
    if (lane == 0) publish(words, tile, agg, kStPartial);
    T excl = T(0);
    int64_t top = (int64_t)tile - 1;
    uint32_t spins = 0;
    for (;;) {
        // Lane l polls predecessor top - l.  The load is unconditional (an
        // index below 0 reads word 0 and is then treated as INCLUSIVE 0), so
        // the compiler issues it without a branch around it.
        const int64_t j = top - (int64_t)lane;
        const uint64_t jj = j < 0 ? 0 : (uint64_t)j;
        uint32_t s;
        T v;
        if constexpr (sizeof(T) == 4) {
            const uint64_t w = ld_relaxed(&words[jj]);
            s = (uint32_t)w;
            v = from_bits<T>(w >> 32);
        } else {
            const uint64_t lo = ld_relaxed(&words[2 * jj]);
            const uint64_t hi = ld_relaxed(&words[2 * jj + 1]);
            s = (uint32_t)lo == (uint32_t)hi ? (uint32_t)lo : kStInvalid;
            v = from_bits<T>((hi & 0xFFFFFFFF00000000ull) | (lo >> 32));
        }
        if (j < 0) {
            s = kStInclusive;
            v = T(0);
        }
        const uint64_t incl = ballot(s == kStInclusive);
        const uint32_t stop = incl ? (uint32_t)__builtin_ctzll(incl) : (uint32_t)(kWave - 1);
        const bool in_range = lane <= stop;
        if (ballot(in_range && s == kStInvalid) != 0 && ++spins < kSpinLimit) {
            __builtin_amdgcn_s_sleep(1);
            continue;  // re-poll the same window
        }
        excl = op(excl, wave_allreduce(in_range ? v : T(0), op));
        if (incl) break;
        top -= kWave;
    }
    if (lane == 0) publish(words, tile, op(excl, agg), kStInclusive);
    return excl;
}

__global__ __launch_bounds__(256) void scan_init_kernel(uint64_t *words, uint64_t count)
{
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += stride) words[i] = 0;
}

template <class T, bool INCLUSIVE>
__global__ __launch_bounds__(kScanBlock) void scan_kernel(const T *__restrict__ in,
                                                          T *__restrict__ out, uint64_t n,
                                                          uint64_t *words, int vec_ok)
{
    constexpr int V = 16 / sizeof(T);
    constexpr int K = kScanVecs;
    constexpr uint32_t TILE = scan_tile<T>();
    constexpr uint32_t CHUNK = kScanBlock * 16;  // bytes per vector instruction
    constexpr int W = kScanBlock / kWave;
    __shared__ T s_wtot[K][W];
    __shared__ T s_prefix;

    SumOp op;
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
            for (int j = 0; j < V; ++j) x[k][j] = buf_ld_elem<T>(rin, tid * 16 + j * sizeof(T), k * CHUNK);
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
            x[k][0] = T(0);
#pragma unroll
            for (int j = 1; j < V; ++j) {
                const T v = x[k][j];
                x[k][j] = r;
                r = op(r, v);
            }
        }
        const T inc = wave_inclusive_scan(r, op);
        const T up = shfl_up(inc, 1);
        const T wex = lane == 0 ? T(0) : up;
        if (lane == kWave - 1) s_wtot[k][wave] = inc;
#pragma unroll
        for (int j = 0; j < V; ++j) x[k][j] = op(wex, x[k][j]);
    }
    __syncthreads();
    if (wave == 0) {
        T agg = T(0);
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int w = 0; w < W; ++w) agg = op(agg, s_wtot[k][w]);
        const T ex = lookback(words, tile, agg);
        if (lane == 0) s_prefix = ex;
    }
    __syncthreads();

    // out = tile prefix + (chunks before k) + (waves before this one in k) + x
    T run = s_prefix;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        T pre = T(0), tot = T(0);
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
            for (int j = 0; j < V; ++j) buf_st_elem<T>(rout, tid * 16 + j * sizeof(T), k * CHUNK, x[k][j]);
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
    const uint64_t tiles = scan_tiles<T>(n);
    if (tiles > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;
    if (temp_bytes < scan_temp_bytes<T>(n)) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    uint64_t *words = static_cast<uint64_t *>(temp);
    const uint64_t nwords = tiles * (sizeof(T) == 4 ? 1 : 2);
    const uint32_t init_grid = (uint32_t)(ceil_div(nwords, 256) < 1024 ? ceil_div(nwords, 256) : 1024);
    LCPP_LAUNCH("scan_init", s, scan_init_kernel<<<init_grid, 256, 0, s>>>(words, nwords));
    LCPP_CHECK_LAUNCH();
    const int vec_ok = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (inclusive)
        LCPP_LAUNCH("scan_inclusive", s,
                    scan_kernel<T, true><<<(uint32_t)tiles, kScanBlock, 0, s>>>(in, out, n, words, vec_ok));
    else
        LCPP_LAUNCH("scan_exclusive", s,
                    scan_kernel<T, false><<<(uint32_t)tiles, kScanBlock, 0, s>>>(in, out, n, words, vec_ok));
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
    case LCPP_INT32: case LCPP_UINT32: case LCPP_FLOAT32: *bytes = scan_temp_bytes<uint32_t>(n); return LCPP_OK;
    case LCPP_INT64: case LCPP_UINT64: case LCPP_FLOAT64: *bytes = scan_temp_bytes<uint64_t>(n); return LCPP_OK;
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
