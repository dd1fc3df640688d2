// reduce.hip — DeviceReduce::Sum/Min/Max/ArgMin/ArgMax/TransformReduce for
// gfx950.
//
// Reference: device/device_reduce.h:131-274, 331-348, 396-460 (multi-level
// tree of 1024-item tiles, one kernel per level), agent/agent_reduce.h:52-157,
// block/detail/block_reduce_warp.h:29-70, warp/details/warp_reduce_shlf.h,
// common/thread_operators.h:19-47 (ArgMaxOp/ArgMinOp).
//
// MI355X design: one streaming pass.  A grid of at most 512 workgroups
// (1024 for ArgMin/ArgMax) partitions the input into equal contiguous chunks
// whose length is a multiple of the tile (128 KiB; 48 KiB for Arg*), so
// every workgroup's range is exact (the reference dispatches more blocks
// than it partitions for N > 10,485,760 and reads past the end).  Each thread
// streams 16-byte vectors (32 per tile; 12 for Arg*), folds them in
// registers, the workgroup folds its four wave totals, and one partial per
// workgroup lands in temp storage.  A
// one-workgroup kernel folds the partials in a fixed order, so the float
// result is deterministic for a given N.  N <= one tile needs no temp and
// one launch.
//
// ArgMin/ArgMax fold (value, index) pairs in the same kernels (the reference
// first materialises an N-element pair array in temp storage, then reduces
// it: 3 passes over N; here the index is the loop counter, one pass).
// TransformReduce applies one of a fixed set of element transforms while
// loading and folds the caller's init in last.
#include "common.hpp"

namespace lcpp {
namespace {

constexpr int kRedBlock = 256;
// Geometry (most workgroups x 16-byte vectors per thread per tile), measured
// at 2^28 int32 (us, Sum / ArgMin): 2048 x 8: 158 / 163; 1024 x 16: 154 /
// 159; 1024 x 12: - / 157; 4096 x 4: - / 162; 512 x 16: 152 / 181; 512 x
// 32: 150 / 177; 256 x 32: 186 / 289; 512 x 48: 154 / 191.  Plain folds take
// 512 workgroups of 32 vectors (two per CU, each streaming 2 MiB); the
// (value, index) folds 1024 of 12.
template <bool ARG>
constexpr int red_vecs()
{
    return ARG ? 12 : 32;
}
template <bool ARG>
constexpr uint32_t red_max_grid()
{
    return ARG ? 1024 : 512;
}

template <class T, bool ARG>
constexpr uint64_t red_tile()
{
    return (uint64_t)kRedBlock * red_vecs<ARG>() * (16 / sizeof(T));
}

struct RedGrid {
    uint32_t grid;
    uint64_t chunk;  // elements per workgroup, multiple of the tile
};

template <class T, bool ARG>
RedGrid red_grid(uint64_t n)
{
    const uint64_t tile = red_tile<T, ARG>();
    uint64_t tiles = ceil_div(n, tile);
    if (tiles == 0) tiles = 1;
    uint64_t grid = tiles < red_max_grid<ARG>() ? tiles : red_max_grid<ARG>();
    uint64_t chunk = ceil_div(tiles, grid) * tile;
    grid = n ? ceil_div(n, chunk) : 1;
    return {(uint32_t)grid, chunk};
}

// ---------------------------------------------------------------- transforms
struct XfIdentity {
    template <class T>
    __device__ __forceinline__ T operator()(T x) const { return x; }
};
struct XfNegate {
    template <class T>
    __device__ __forceinline__ T operator()(T x) const
    {
        if constexpr (std::is_integral_v<T>) return (T)(std::make_unsigned_t<T>(0) - (std::make_unsigned_t<T>)x);
        else return -x;
    }
};
struct XfAbs {
    template <class T>
    __device__ __forceinline__ T operator()(T x) const
    {
        if constexpr (std::is_unsigned_v<T>) return x;
        else if constexpr (std::is_integral_v<T>) return x < 0 ? XfNegate()(x) : x;
        else return __builtin_fabs(x);
    }
};
struct XfSquare {
    template <class T>
    __device__ __forceinline__ T operator()(T x) const
    {
        if constexpr (std::is_integral_v<T>) {
            using U = std::make_unsigned_t<T>;
            return (T)((U)x * (U)x);  // two's-complement wraparound
        } else {
            return x * x;
        }
    }
};

// ---------------------------------------------------------------- (value, index)
template <class T>
struct IdxVal {
    T value;
    uint32_t index;
};
// common/thread_operators.h:19-47: ArgMin keeps the smaller value, on ties
// the smaller index; ArgMax keeps the larger value, on ties the larger index.
// Both are total orders on distinct (value, index) pairs, so the result does
// not depend on the folding order.
template <bool IS_MAX>
struct ArgOp {
    template <class P>
    __device__ __forceinline__ P operator()(P a, P b) const
    {
        const bool take = IS_MAX ? (b.value > a.value || (b.value == a.value && b.index > a.index))
                                 : (b.value < a.value || (b.value == a.value && b.index < a.index));
        return take ? b : a;
    }
    // device_reduce.h:230-235 / 267-272 (Max starts from lowest(), see ArgMax below)
    template <class T>
    static constexpr IdxVal<T> identity()
    {
        return IS_MAX ? IdxVal<T>{std::numeric_limits<T>::lowest(), 0u}
                      : IdxVal<T>{std::numeric_limits<T>::max(), 0xFFFFFFFFu};
    }
};

template <class P>
__device__ __forceinline__ P shfl_xor_pair(P x, int m)
{
    static_assert(sizeof(P) == 8 || sizeof(P) == 16, "pair of 4- or 8-byte value and index");
    P r;
    r.value = shfl_xor(x.value, m);
    r.index = (uint32_t)__shfl_xor((int)x.index, m);
    return r;
}

template <class T, class Op, class Xf>
__device__ __forceinline__ T fold16(T acc, u32x4 v, Op op, Xf xf)
{
    T e[16 / sizeof(T)];
    unpack16<T>(v, e);
#pragma unroll
    for (int j = 0; j < (int)(16 / sizeof(T)); ++j) acc = op(acc, xf(e[j]));
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

// Partials: one per workgroup, or with `direct` (a single workgroup) the
// result op(init, fold) itself.
template <class T, class Op, class Xf>
__global__ __launch_bounds__(kRedBlock) void reduce_partials_kernel(const T *__restrict__ in,
                                                                    uint64_t n, uint64_t chunk,
                                                                    T *__restrict__ partials,
                                                                    T init, int direct, uint32_t *status)
{
    Op op;
    Xf xf;
    if (status && blockIdx.x == 0 && threadIdx.x == 0) *status = 0;  // nothing here waits
    T acc = Op::template identity<T>();
    const uint64_t b0 = (uint64_t)blockIdx.x * chunk;
    const uint64_t b1 = b0 + chunk < n ? b0 + chunk : n;
    const uint32_t tid = threadIdx.x;
    constexpr uint64_t V = 16 / sizeof(T);
    constexpr uint64_t tile = red_tile<T, false>();
    constexpr int VECS = red_vecs<false>();
    uint64_t tail = b0;
    if ((reinterpret_cast<uintptr_t>(in) & 15) == 0) {
        const uint64_t full_end = b0 + (b1 - b0) / tile * tile;
        for (uint64_t t = b0; t < full_end; t += tile) {
            u32x4 v[VECS];
#pragma unroll
            for (int i = 0; i < VECS; ++i)
                v[i] = ld16_nt((in + t + ((uint64_t)i * kRedBlock + tid) * V));
#pragma unroll
            for (int i = 0; i < VECS; ++i) acc = fold16<T>(acc, v[i], op, xf);
        }
        tail = full_end;
    }
    for (uint64_t i = tail + tid; i < b1; i += kRedBlock) acc = op(acc, xf(in[i]));
    acc = block_reduce(acc, op);
    if (tid == 0) partials[blockIdx.x] = direct ? op(init, acc) : acc;
}

template <class T, class Op>
__global__ __launch_bounds__(kRedBlock) void reduce_final_kernel(const T *__restrict__ partials,
                                                                 uint32_t count,
                                                                 T *__restrict__ out, T init, uint32_t *status)
{
    Op op;
    if (status && threadIdx.x == 0) *status = 0;
    T acc = Op::template identity<T>();
    for (uint32_t i = threadIdx.x; i < count; i += kRedBlock) acc = op(acc, partials[i]);
    acc = block_reduce(acc, op);
    if (threadIdx.x == 0) out[0] = op(init, acc);
}

template <class T>
uint64_t reduce_temp(uint64_t n)
{
    RedGrid g = red_grid<T, false>(n);
    return g.grid > 1 ? kStatusBytes + align_up((uint64_t)g.grid * sizeof(T), 256) : 0;
}

template <class T, class Op, class Xf>
int reduce_launch(void *temp, size_t temp_bytes, const void *in_, void *out_, uint64_t n,
                  T init, hipStream_t s)
{
    const T *in = static_cast<const T *>(in_);
    T *out = static_cast<T *>(out_);
    if (!out || (n && !in)) return LCPP_ERR_INVALID_ARG;
    RedGrid g = red_grid<T, false>(n);
    if (g.grid == 1) {
        // one workgroup writes op(init, fold) itself; a temp buffer, if one
        // is passed, only has its status word cleared
        uint32_t *st = temp && temp_bytes >= kStatusBytes && !(reinterpret_cast<uintptr_t>(temp) & 255)
                           ? static_cast<uint32_t *>(temp)
                           : nullptr;
        if (n == 0) {
            LCPP_LAUNCH("reduce_final", s,
                        (reduce_final_kernel<T, Op><<<1, kRedBlock, 0, s>>>(out, 0, out, init, st)));
        } else {
            LCPP_LAUNCH("reduce_partials", s,
                        (reduce_partials_kernel<T, Op, Xf><<<1, kRedBlock, 0, s>>>(in, n, g.chunk, out, init, 1, st)));
        }
        LCPP_CHECK_LAUNCH();
        return LCPP_OK;
    }
    if (temp_bytes < reduce_temp<T>(n)) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    T *partials = reinterpret_cast<T *>(static_cast<char *>(temp) + kStatusBytes);
    LCPP_LAUNCH("reduce_partials", s,
                (reduce_partials_kernel<T, Op, Xf><<<g.grid, kRedBlock, 0, s>>>(
                    in, n, g.chunk, partials, init, 0, static_cast<uint32_t *>(temp))));
    LCPP_CHECK_LAUNCH();
    LCPP_LAUNCH("reduce_final", s,
                (reduce_final_kernel<T, Op><<<1, kRedBlock, 0, s>>>(partials, g.grid, out, init, nullptr)));
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

// ---------------------------------------------------------------- ArgMin / ArgMax
template <class P, class Op>
__device__ __forceinline__ P block_reduce_pair(P x, Op op)
{
    __shared__ P s_wave[kRedBlock / kWave];
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) x = op(x, shfl_xor_pair(x, m));
    if (lane_id() == 0) s_wave[threadIdx.x / kWave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kRedBlock / kWave; ++w) x = op(x, s_wave[w]);
    }
    return x;
}

template <class T, bool IS_MAX>
__global__ __launch_bounds__(kRedBlock) void arg_partials_kernel(const T *__restrict__ in, uint64_t n,
                                                                 uint64_t chunk,
                                                                 IdxVal<T> *__restrict__ partials,
                                                                 T *__restrict__ out,
                                                                 uint32_t *__restrict__ out_index,
                                                                 uint32_t *status)
{
    using P = IdxVal<T>;
    ArgOp<IS_MAX> op;
    P acc = ArgOp<IS_MAX>::template identity<T>();
    if (status && blockIdx.x == 0 && threadIdx.x == 0) *status = 0;  // nothing here waits
    const uint64_t b0 = (uint64_t)blockIdx.x * chunk;
    const uint64_t b1 = b0 + chunk < n ? b0 + chunk : n;
    const uint32_t tid = threadIdx.x;
    constexpr uint64_t V = 16 / sizeof(T);
    constexpr uint64_t tile = red_tile<T, true>();
    constexpr int VECS = red_vecs<true>();
    uint64_t tail = b0;
    if ((reinterpret_cast<uintptr_t>(in) & 15) == 0) {
        const uint64_t full_end = b0 + (b1 - b0) / tile * tile;
        for (uint64_t t = b0; t < full_end; t += tile) {
            u32x4 v[VECS];
#pragma unroll
            for (int i = 0; i < VECS; ++i)
                v[i] = ld16_nt((in + t + ((uint64_t)i * kRedBlock + tid) * V));
#pragma unroll
            for (int i = 0; i < VECS; ++i) {
                T e[V];
                unpack16<T>(v[i], e);
                const uint32_t i0 = (uint32_t)(t + ((uint64_t)i * kRedBlock + tid) * V);
#pragma unroll
                for (int j = 0; j < (int)V; ++j) acc = op(acc, P{e[j], i0 + (uint32_t)j});
            }
        }
        tail = full_end;
    }
    for (uint64_t i = tail + tid; i < b1; i += kRedBlock) acc = op(acc, P{in[i], (uint32_t)i});
    acc = block_reduce_pair(acc, op);
    if (tid == 0) {
        if (out) {
            out[0] = acc.value;
            out_index[0] = acc.index;
        } else {
            partials[blockIdx.x] = acc;
        }
    }
}

template <class T, bool IS_MAX>
__global__ __launch_bounds__(kRedBlock) void arg_final_kernel(const IdxVal<T> *__restrict__ partials,
                                                              uint32_t count, T *__restrict__ out,
                                                              uint32_t *__restrict__ out_index, uint32_t *status)
{
    using P = IdxVal<T>;
    ArgOp<IS_MAX> op;
    if (status && threadIdx.x == 0) *status = 0;
    P acc = ArgOp<IS_MAX>::template identity<T>();
    for (uint32_t i = threadIdx.x; i < count; i += kRedBlock) acc = op(acc, partials[i]);
    acc = block_reduce_pair(acc, op);
    if (threadIdx.x == 0) {
        out[0] = acc.value;
        out_index[0] = acc.index;
    }
}

template <class T>
uint64_t arg_temp(uint64_t n)
{
    RedGrid g = red_grid<T, true>(n);
    return g.grid > 1 ? kStatusBytes + align_up((uint64_t)g.grid * sizeof(IdxVal<T>), 256) : 0;
}

template <class T, bool IS_MAX>
int arg_launch(void *temp, size_t temp_bytes, const void *in_, void *out_, uint32_t *out_index, uint64_t n,
               hipStream_t s)
{
    const T *in = static_cast<const T *>(in_);
    T *out = static_cast<T *>(out_);
    if (!out || !out_index || (n && !in)) return LCPP_ERR_INVALID_ARG;
    if (n > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;  // 32-bit indices, as the reference
    RedGrid g = red_grid<T, true>(n);
    if (g.grid == 1) {
        uint32_t *st = temp && temp_bytes >= kStatusBytes && !(reinterpret_cast<uintptr_t>(temp) & 255)
                           ? static_cast<uint32_t *>(temp)
                           : nullptr;
        if (n == 0) {
            LCPP_LAUNCH("arg_final", s,
                        (arg_final_kernel<T, IS_MAX><<<1, kRedBlock, 0, s>>>(nullptr, 0, out, out_index, st)));
        } else {
            LCPP_LAUNCH("arg_partials", s,
                        (arg_partials_kernel<T, IS_MAX><<<1, kRedBlock, 0, s>>>(in, n, g.chunk, nullptr, out, out_index,
                                                                                  st)));
        }
        LCPP_CHECK_LAUNCH();
        return LCPP_OK;
    }
    if (temp_bytes < arg_temp<T>(n)) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    IdxVal<T> *partials = reinterpret_cast<IdxVal<T> *>(static_cast<char *>(temp) + kStatusBytes);
    LCPP_LAUNCH("arg_partials", s,
                (arg_partials_kernel<T, IS_MAX><<<g.grid, kRedBlock, 0, s>>>(in, n, g.chunk, partials, nullptr, nullptr,
                                                                             static_cast<uint32_t *>(temp))));
    LCPP_CHECK_LAUNCH();
    LCPP_LAUNCH("arg_final", s,
                (arg_final_kernel<T, IS_MAX><<<1, kRedBlock, 0, s>>>(partials, g.grid, out, out_index, nullptr)));
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

template <bool IS_MAX>
int arg_dispatch(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out, uint32_t *idx, uint64_t n,
                 void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (t) {
    case LCPP_INT32: return arg_launch<int32_t, IS_MAX>(temp, tb, in, out, idx, n, s);
    case LCPP_UINT32: return arg_launch<uint32_t, IS_MAX>(temp, tb, in, out, idx, n, s);
    case LCPP_FLOAT32: return arg_launch<float, IS_MAX>(temp, tb, in, out, idx, n, s);
    case LCPP_INT64: return arg_launch<int64_t, IS_MAX>(temp, tb, in, out, idx, n, s);
    case LCPP_UINT64: return arg_launch<uint64_t, IS_MAX>(temp, tb, in, out, idx, n, s);
    case LCPP_FLOAT64: return arg_launch<double, IS_MAX>(temp, tb, in, out, idx, n, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

template <class Op, class Xf = XfIdentity>
int reduce_dispatch(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out, uint64_t n,
                    const void *init, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    // init: the caller's value of type t, or the operator's identity
    auto iv = [&](auto zero) {
        using T = decltype(zero);
        if (!init) return Op::template identity<T>();
        T v;
        __builtin_memcpy(&v, init, sizeof(T));
        return v;
    };
    switch (t) {
    case LCPP_INT32: return reduce_launch<int32_t, Op, Xf>(temp, tb, in, out, n, iv(int32_t()), s);
    case LCPP_UINT32: return reduce_launch<uint32_t, Op, Xf>(temp, tb, in, out, n, iv(uint32_t()), s);
    case LCPP_FLOAT32: return reduce_launch<float, Op, Xf>(temp, tb, in, out, n, iv(float()), s);
    case LCPP_INT64: return reduce_launch<int64_t, Op, Xf>(temp, tb, in, out, n, iv(int64_t()), s);
    case LCPP_UINT64: return reduce_launch<uint64_t, Op, Xf>(temp, tb, in, out, n, iv(uint64_t()), s);
    case LCPP_FLOAT64: return reduce_launch<double, Op, Xf>(temp, tb, in, out, n, iv(double()), s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

template <class Op>
int transform_dispatch(lcpp_transform xf, lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                       uint64_t n, const void *init, void *stream)
{
    switch (xf) {
    case LCPP_XFORM_IDENTITY: return reduce_dispatch<Op, XfIdentity>(t, temp, tb, in, out, n, init, stream);
    case LCPP_XFORM_NEGATE: return reduce_dispatch<Op, XfNegate>(t, temp, tb, in, out, n, init, stream);
    case LCPP_XFORM_ABS: return reduce_dispatch<Op, XfAbs>(t, temp, tb, in, out, n, init, stream);
    case LCPP_XFORM_SQUARE: return reduce_dispatch<Op, XfSquare>(t, temp, tb, in, out, n, init, stream);
    default: return LCPP_ERR_INVALID_ARG;
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
    return reduce_dispatch<SumOp>(t, temp, tb, in, out, n, nullptr, stream);
}

extern "C" int lcpp_reduce_min(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                               uint64_t n, void *stream)
{
    return reduce_dispatch<MinOp>(t, temp, tb, in, out, n, nullptr, stream);
}

extern "C" int lcpp_reduce_max(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                               uint64_t n, void *stream)
{
    return reduce_dispatch<MaxOp>(t, temp, tb, in, out, n, nullptr, stream);
}

extern "C" int lcpp_reduce_transform(lcpp_dtype t, lcpp_reduce_op op, lcpp_transform xf, void *temp,
                                     size_t tb, const void *in, void *out, uint64_t n, const void *init,
                                     void *stream)
{
    if (!init) return LCPP_ERR_INVALID_ARG;
    switch (op) {
    case LCPP_OP_SUM: return transform_dispatch<SumOp>(xf, t, temp, tb, in, out, n, init, stream);
    case LCPP_OP_MIN: return transform_dispatch<MinOp>(xf, t, temp, tb, in, out, n, init, stream);
    case LCPP_OP_MAX: return transform_dispatch<MaxOp>(xf, t, temp, tb, in, out, n, init, stream);
    default: return LCPP_ERR_INVALID_ARG;
    }
}

extern "C" int lcpp_reduce_arg_temp_bytes(lcpp_dtype t, uint64_t n, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    if (n > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;  // 32-bit indices, as the call
    switch (t) {
    case LCPP_INT32: case LCPP_UINT32: case LCPP_FLOAT32: *bytes = arg_temp<uint32_t>(n); return LCPP_OK;
    case LCPP_INT64: case LCPP_UINT64: case LCPP_FLOAT64: *bytes = arg_temp<uint64_t>(n); return LCPP_OK;
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

extern "C" int lcpp_reduce_argmin(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                                  uint32_t *index_out, uint64_t n, void *stream)
{
    return arg_dispatch<false>(t, temp, tb, in, out, index_out, n, stream);
}

extern "C" int lcpp_reduce_argmax(lcpp_dtype t, void *temp, size_t tb, const void *in, void *out,
                                  uint32_t *index_out, uint64_t n, void *stream)
{
    return arg_dispatch<true>(t, temp, tb, in, out, index_out, n, stream);
}
