// reduce.hip — DeviceReduce::Sum/Min/Max for gfx950.
//
// Reference: device/device_reduce.h:131-185, 396-460 (multi-level tree of
// 1024-item tiles, one kernel per level), agent/agent_reduce.h:52-157,
// block/detail/block_reduce_warp.h:29-70, warp/details/warp_reduce_shlf.h.
//
// MI355X design: one streaming pass.  A grid of at most 2048 workgroups
// (256 CUs x 8) partitions the input into equal contiguous chunks whose
// length is a multiple of the 16 KiB tile, so every workgroup's range is
// exact (the reference dispatches more blocks than it partitions for
// N > 10,485,760 and reads past the end).  Each thread streams 16-byte
// vectors (8 in flight), folds them in registers, the workgroup folds its
// four wave totals, and one partial per workgroup lands in temp storage.  A
// one-workgroup kernel folds the partials in a fixed order, so the float
// result is deterministic for a given N.  N <= one tile needs no temp and
// one launch.
#include "common.hpp"

namespace lcpp {
namespace {

constexpr int kRedBlock = 256;
constexpr int kRedVecs = 8;            // 16-byte vectors per thread per tile
constexpr uint32_t kRedMaxGrid = 2048; // 256 CUs x 8 workgroups

template <class T>
constexpr uint64_t red_tile()
{
    return (uint64_t)kRedBlock * kRedVecs * (16 / sizeof(T));
}

struct RedGrid {
    uint32_t grid;
    uint64_t chunk;  // elements per workgroup, multiple of the tile
};

template <class T>
RedGrid red_grid(uint64_t n)
{
    const uint64_t tile = red_tile<T>();
    uint64_t tiles = ceil_div(n, tile);
    if (tiles == 0) tiles = 1;
    uint64_t grid = tiles < kRedMaxGrid ? tiles : kRedMaxGrid;
    uint64_t chunk = ceil_div(tiles, grid) * tile;
    grid = n ? ceil_div(n, chunk) : 1;
    return {(uint32_t)grid, chunk};
}

template <class T, class Op>
__device__ __forceinline__ T fold16(T acc, u32x4 v, Op op)
{
    T e[16 / sizeof(T)];
    unpack16<T>(v, e);
#pragma unroll
    for (int j = 0; j < (int)(16 / sizeof(T)); ++j) acc = op(acc, e[j]);
    return acc;
}

// Workgroup fold: wave butterflies, then thread 0 folds the wave totals in
// wave order.  Result valid in thread 0.
template <class T, class Op>
__device__ __forceinline__ T block_reduce(T x, Op op)
{
    __shared__ T s_wave[kRedBlock / kWave];
    x = wave_allreduce(x, op);
    if (lane_id() == 0) s_wave[threadIdx.x / kWave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kRedBlock / kWave; ++w) x = op(x, s_wave[w]);
    }
    return x;
}

template <class T, class Op>
__global__ __launch_bounds__(kRedBlock) void reduce_partials_kernel(const T *__restrict__ in,
                                                                    uint64_t n, uint64_t chunk,
                                                                    T *__restrict__ partials)
{
    Op op;
    T acc = Op::template identity<T>();
    const uint64_t b0 = (uint64_t)blockIdx.x * chunk;
    const uint64_t b1 = b0 + chunk < n ? b0 + chunk : n;
    const uint32_t tid = threadIdx.x;
    constexpr uint64_t V = 16 / sizeof(T);
    constexpr uint64_t tile = red_tile<T>();
    uint64_t tail = b0;
    if ((reinterpret_cast<uintptr_t>(in) & 15) == 0) {
        const uint64_t full_end = b0 + (b1 - b0) / tile * tile;
        for (uint64_t t = b0; t < full_end; t += tile) {
            u32x4 v[kRedVecs];
#pragma unroll
            for (int i = 0; i < kRedVecs; ++i)
                v[i] = ld16_nt((in + t + ((uint64_t)i * kRedBlock + tid) * V));
#pragma unroll
            for (int i = 0; i < kRedVecs; ++i) acc = fold16<T>(acc, v[i], op);
        }
        tail = full_end;
    }
    for (uint64_t i = tail + tid; i < b1; i += kRedBlock) acc = op(acc, in[i]);
    acc = block_reduce(acc, op);
    if (tid == 0) partials[blockIdx.x] = acc;
}

template <class T, class Op>
__global__ __launch_bounds__(kRedBlock) void reduce_final_kernel(const T *__restrict__ partials,
                                                                 uint32_t count,
                                                                 T *__restrict__ out)
{
    Op op;
    T acc = Op::template identity<T>();
    for (uint32_t i = threadIdx.x; i < count; i += kRedBlock) acc = op(acc, partials[i]);
    acc = block_reduce(acc, op);
    if (threadIdx.x == 0) out[0] = op(Op::template identity<T>(), acc);
}

template <class T>
uint64_t reduce_temp(uint64_t n)
{
    RedGrid g = red_grid<T>(n);
    return g.grid > 1 ? align_up((uint64_t)g.grid * sizeof(T), 256) : 0;
}

template <class T, class Op>
int reduce_launch(void *temp, size_t temp_bytes, const void *in_, void *out_, uint64_t n,
                  hipStream_t s)
{
    const T *in = static_cast<const T *>(in_);
    T *out = static_cast<T *>(out_);
    if (!out || (n && !in)) return LCPP_ERR_INVALID_ARG;
    RedGrid g = red_grid<T>(n);
    if (g.grid == 1) {
        // one workgroup: its partial is the result (init is the identity)
        if (n == 0) {
            LCPP_LAUNCH("reduce_final", s,
                        reduce_final_kernel<T, Op><<<1, kRedBlock, 0, s>>>(out, 0, out));
        } else {
            LCPP_LAUNCH("reduce_partials", s,
                        reduce_partials_kernel<T, Op><<<1, kRedBlock, 0, s>>>(in, n, g.chunk, out));
        }
        LCPP_CHECK_LAUNCH();
        return LCPP_OK;
    }
    if (temp_bytes < reduce_temp<T>(n)) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    T *partials = static_cast<T *>(temp);
    LCPP_LAUNCH("reduce_partials", s,
                reduce_partials_kernel<T, Op><<<g.grid, kRedBlock, 0, s>>>(in, n, g.chunk, partials));
    LCPP_CHECK_LAUNCH();
    LCPP_LAUNCH("reduce_final", s,
                reduce_final_kernel<T, Op><<<1, kRedBlock, 0, s>>>(partials, g.grid, out));
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

template <class Op>
int reduce_dispatch(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out, uint64_t n,
                    void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (t) {
    case LCPP_INT32: return reduce_launch<int32_t, Op>(temp, tb, in, out, n, s);
    case LCPP_UINT32: return reduce_launch<uint32_t, Op>(temp, tb, in, out, n, s);
    case LCPP_FLOAT32: return reduce_launch<float, Op>(temp, tb, in, out, n, s);
    case LCPP_INT64: return reduce_launch<int64_t, Op>(temp, tb, in, out, n, s);
    case LCPP_UINT64: return reduce_launch<uint64_t, Op>(temp, tb, in, out, n, s);
    case LCPP_FLOAT64: return reduce_launch<double, Op>(temp, tb, in, out, n, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

}  // namespace
}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_reduce_temp_bytes(lcpp_dtype t, uint64_t n, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    switch (t) {
    case LCPP_INT32: case LCPP_UINT32: case LCPP_FLOAT32: *bytes = reduce_temp<uint32_t>(n); return LCPP_OK;
    case LCPP_INT64: case LCPP_UINT64: case LCPP_FLOAT64: *bytes = reduce_temp<uint64_t>(n); return LCPP_OK;
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

extern "C" int lcpp_reduce_sum(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                               uint64_t n, void *stream)
{
    return reduce_dispatch<SumOp>(t, temp, tb, in, out, n, stream);
}

extern "C" int lcpp_reduce_min(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                               uint64_t n, void *stream)
{
    return reduce_dispatch<MinOp>(t, temp, tb, in, out, n, stream);
}

extern "C" int lcpp_reduce_max(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                               uint64_t n, void *stream)
{
    return reduce_dispatch<MaxOp>(t, temp, tb, in, out, n, stream);
}
