// segment_reduce.hip — DeviceSegmentReduce::Sum with CSR begin/end offsets.
//
// Reference: device/device_segment_reduce.h:94-135, 353-381 and
// device/details/segment_reduce.h:43-86: one 256-thread workgroup per
// segment (2^20 workgroups at the benchmark size, most lanes idle for a mean
// segment length of 128); no temp storage.
//
// MI355X design, one launch, no temp storage, length-adaptive:
//  * A workgroup (4 waves) owns a batch of 256 consecutive segments; thread t
//    loads begin/end of segment t of the batch (coalesced).
//  * Short segments (<= kSegLong elements): wave-per-segment.  Wave w walks
//    its 64 segments 8 at a time: the bounds are read out of the lanes into
//    scalar registers and each lane accumulates element (lane + 64c) of each
//    of the 8 segments, two 64-element chunks per segment in flight (16
//    independent loads per wave).  Each total is a 64-lane butterfly; lane l
//    keeps the total of segment l and the wave stores its 64 results with
//    one coalesced store.
//  * Long segments: workgroup-per-segment.  Their indices are compacted into
//    LDS and the whole workgroup streams each one (4 loads in flight per
//    thread), then folds the four wave totals.
//  * An empty segment (end <= begin) gives exactly +0 (the reference writes
//    its init value, 0).
#include "common.hpp"

namespace lcpp {
namespace {

constexpr int kSegBlock = 256;
constexpr int kSegWaves = kSegBlock / kWave;
constexpr int kSegUnroll = 8;
constexpr uint32_t kSegLong = 8192;

template <class T>
__global__ __launch_bounds__(kSegBlock) void segment_sum_kernel(const T *__restrict__ in,
                                                                T *__restrict__ out,
                                                                uint64_t num_segments,
                                                                const uint32_t *__restrict__ begin,
                                                                const uint32_t *__restrict__ end)
{
    __shared__ uint32_t s_long[kSegBlock];
    __shared__ uint32_t s_nlong;
    __shared__ T s_wave[kSegWaves];
    SumOp op;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint64_t batch0 = (uint64_t)blockIdx.x * kSegBlock;
    const uint64_t my_seg = batch0 + tid;

    uint32_t b = 0, len = 0;
    if (my_seg < num_segments) {
        b = begin[my_seg];
        const uint32_t e = end[my_seg];
        len = e > b ? e - b : 0;
    }
    if (tid == 0) s_nlong = 0;
    __syncthreads();
    const bool is_long = len > kSegLong;
    if (is_long) s_long[atomicAdd(&s_nlong, 1u)] = tid;
    if (is_long) len = 0;  // summed by the whole workgroup below

    // ---- short segments: wave per segment
    T mine = T(0);
#pragma unroll 1
    for (int j0 = 0; j0 < kWave; j0 += kSegUnroll) {
        uint32_t bj[kSegUnroll], lj[kSegUnroll];
        uint32_t maxlen = 0;
#pragma unroll
        for (int u = 0; u < kSegUnroll; ++u) {
            bj[u] = __builtin_amdgcn_readlane(b, j0 + u);
            lj[u] = __builtin_amdgcn_readlane(len, j0 + u);
            maxlen = lj[u] > maxlen ? lj[u] : maxlen;
        }
        if (maxlen == 0) continue;
        T acc[kSegUnroll];
#pragma unroll
        for (int u = 0; u < kSegUnroll; ++u) acc[u] = T(0);
#pragma unroll 1
        for (uint32_t c = lane; c < maxlen; c += 2 * kWave) {
            T x0[kSegUnroll], x1[kSegUnroll];
#pragma unroll
            for (int u = 0; u < kSegUnroll; ++u) {
                x0[u] = c < lj[u] ? in[(uint64_t)bj[u] + c] : T(0);
                x1[u] = c + kWave < lj[u] ? in[(uint64_t)bj[u] + c + kWave] : T(0);
            }
#pragma unroll
            for (int u = 0; u < kSegUnroll; ++u) acc[u] = op(op(acc[u], x0[u]), x1[u]);
        }
#pragma unroll
        for (int u = 0; u < kSegUnroll; ++u) {
            if (lj[u] == 0) continue;
            const T r = wave_allreduce(acc[u], op);
            if (lane == (uint32_t)(j0 + u)) mine = r;
        }
    }
    if (my_seg < num_segments && !is_long) out[my_seg] = mine;

    // ---- long segments: workgroup per segment
    __syncthreads();
    const uint32_t nlong = s_nlong;
    for (uint32_t q = 0; q < nlong; ++q) {
        const uint64_t s = batch0 + s_long[q];
        const uint64_t lb = begin[s], le = end[s];
        T acc0 = T(0), acc1 = T(0), acc2 = T(0), acc3 = T(0);
        uint64_t i = lb + tid;
        for (; i + 3 * kSegBlock < le; i += 4 * kSegBlock) {
            acc0 = op(acc0, in[i]);
            acc1 = op(acc1, in[i + kSegBlock]);
            acc2 = op(acc2, in[i + 2 * kSegBlock]);
            acc3 = op(acc3, in[i + 3 * kSegBlock]);
        }
        for (; i < le; i += kSegBlock) acc0 = op(acc0, in[i]);
        T acc = op(op(acc0, acc1), op(acc2, acc3));
        acc = wave_allreduce(acc, op);
        if (lane == 0) s_wave[wave] = acc;
        __syncthreads();
        if (tid == 0) {
            T r = s_wave[0];
#pragma unroll
            for (int w = 1; w < kSegWaves; ++w) r = op(r, s_wave[w]);
            out[s] = r;
        }
        __syncthreads();
    }
}

template <class T>
int segment_launch(const void *in_, void *out_, uint64_t S, const uint32_t *begin,
                   const uint32_t *end, hipStream_t s)
{
    if (S == 0) return LCPP_OK;
    const T *in = static_cast<const T *>(in_);
    T *out = static_cast<T *>(out_);
    if (!out || !begin || !end) return LCPP_ERR_INVALID_ARG;
    const uint64_t blocks = ceil_div(S, kSegBlock);
    if (blocks > 0x7FFFFFFFull) return LCPP_ERR_INVALID_ARG;
    LCPP_LAUNCH("segment_sum", s,
                segment_sum_kernel<T><<<(uint32_t)blocks, kSegBlock, 0, s>>>(in, out, S, begin, end));
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

}  // namespace
}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_segment_reduce_temp_bytes(lcpp_dtype t, uint64_t, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    if ((int)t < LCPP_INT32 || (int)t > LCPP_FLOAT64) return LCPP_ERR_UNSUPPORTED_DTYPE;
    *bytes = 0;
    return LCPP_OK;
}

extern "C" int lcpp_segment_reduce_sum(lcpp_dtype t, void *, size_t, const void *in, void *out,
                                       uint64_t S, const uint32_t *begin, const uint32_t *end,
                                       void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (t) {
    case LCPP_INT32: return segment_launch<int32_t>(in, out, S, begin, end, s);
    case LCPP_UINT32: return segment_launch<uint32_t>(in, out, S, begin, end, s);
    case LCPP_FLOAT32: return segment_launch<float>(in, out, S, begin, end, s);
    case LCPP_INT64: return segment_launch<int64_t>(in, out, S, begin, end, s);
    case LCPP_UINT64: return segment_launch<uint64_t>(in, out, S, begin, end, s);
    case LCPP_FLOAT64: return segment_launch<double>(in, out, S, begin, end, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}
