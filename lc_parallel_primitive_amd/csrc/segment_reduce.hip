// segment_reduce.hip — DeviceSegmentReduce::Reduce/Sum/Min/Max/ArgMin/ArgMax
// over CSR begin/end offsets or fixed-size segments, for gfx950.
//
// Reference: device/device_segment_reduce.h:94-349 (entry points), 353-431
// (dispatch: one workgroup per segment, or for fixed-size segments of at
// most small_items_per_tile a warp per segment), device/details/
// segment_reduce.h:43-164 (kernels: out[s] = reduce_op(init, aggregate),
// an empty segment writes init), segment_reduce.h:166-240 (Arg*: (index,
// value) pairs over the whole input, then index - begin per segment).
//
// MI355X design, one launch, no temp storage, segment-length adaptive:
//  * A workgroup (4 waves) owns 256 consecutive segments, 64 per wave; lanes
//    0..63 of a wave load the bounds of its segments with one coalesced load
//    (or compute them, for fixed-size segments).
//  * Wave-per-segment for segments up to kSegLong elements: the wave walks its
//    64 segments 8 at a time; the 8 bounds are read out of the lanes into
//    scalar registers and lane l accumulates elements l, l + 64, ... of each,
//    two 64-element chunks per segment in flight (16 independent loads per
//    lane); a 64-lane butterfly per segment leaves its result in the lane of
//    that segment, and the wave stores its 64 results together.
//  * Workgroup-per-segment for longer ones: their indices are compacted into
//    LDS and the whole workgroup streams each one (4 loads in flight per
//    thread) after its waves are done.  Fixed-size segments longer than
//    kSegLong take a workgroup-per-segment launch directly.
//  * Flat path: a wave whose 64 segments tile one contiguous range (CSR
//    offsets with end[s] == begin[s + 1], or fixed-size segments), none of
//    them long, streams that range in 4 KiB chunks of coalesced 16-byte
//    loads, transposes each chunk through LDS so that every lane holds
//    consecutive elements, folds them in order and joins the lanes with a
//    segmented scan (flat_segments below).
//  * Sum/Min/Max write op(init, fold) (init defaults to the operator's
//    identity; Min starts from max(), Max from lowest()); an empty segment
//    (end <= begin, or segment_size 0) writes init.  Arg* keep
//    (value, element index) pairs with the reference's tie rules (ArgMin:
//    smaller value, then smaller index; ArgMax: larger value, then larger
//    index, common/thread_operators.h:19-47) and report the index relative
//    to the segment's first element; an empty segment gives index 1 and
//    value max() (ArgMin) / lowest() (ArgMax).  The fold starts from the
//    segment's own elements (no sentinel value takes part), so +-inf
//    elements are found like any other.
#include <cstring>

#include "common.hpp"

namespace lcpp {
namespace {

constexpr int kSegBlock = 256;
constexpr int kSegWaves = kSegBlock / kWave;
// Segments in flight per wave and segments per wave.  Measured at C5
// (2^27 f32, 2^20 segments of mean length 128, us): 4 / 8 / 16 in flight:
// 128 / 118 / 142; 16 / 32 / 64 per wave: 121 / 119 / 117.  A persistent
// grid of waves striding over groups of 8 measured 141-190 us, and 16-byte
// vector loads with index masking 127 us (fewer waves fit).  The per-segment
// wave reductions use DPP and readlane instead of __shfl_xor (ds_bpermute
// through LDS): 119-122 -> 113 us.  The flat path takes C5 to 97 us (a copy
// of it that only sums each wave's range, with no segment logic, runs in
// 87.5 us): per-element branches 105 us, branch-free fold 99 us, segment of
// each lane's first element by a 7-step binary search in LDS 99 us against
// a slot histogram and a DPP scan 97 us.
constexpr int kSegGroup = 8;
constexpr int kSegPerWave = 64;
constexpr uint32_t kSegLong = 8192;
constexpr uint32_t kNoIndex = 0xFFFFFFFFu;

enum SegOpKind { kSegSum = 0, kSegMin = 1, kSegMax = 2, kSegArgMin = 3, kSegArgMax = 4 };

template <class T>
struct SegPair {
    T value;
    uint32_t index;  // kNoIndex: no element folded yet
};

// Accumulator of one segment: T for Sum/Min/Max, SegPair<T> for Arg*.
template <class T, int OP>
struct SegAcc {
    static constexpr bool kArg = OP >= kSegArgMin;
    using A = std::conditional_t<kArg, SegPair<T>, T>;

    static __host__ __device__ __forceinline__ A identity()
    {
        if constexpr (OP == kSegSum) return SumOp::identity<T>();
        else if constexpr (OP == kSegMin) return MinOp::identity<T>();
        else if constexpr (OP == kSegMax) return MaxOp::identity<T>();
        else return A{T(0), kNoIndex};
    }
    static __device__ __forceinline__ A combine(A a, A b)
    {
        if constexpr (OP == kSegSum) return SumOp()(a, b);
        else if constexpr (OP == kSegMin) return MinOp()(a, b);
        else if constexpr (OP == kSegMax) return MaxOp()(a, b);
        else {
            if (b.index == kNoIndex) return a;
            if (a.index == kNoIndex) return b;
            const bool take = OP == kSegArgMax ? (b.value > a.value || (b.value == a.value && b.index > a.index))
                                               : (b.value < a.value || (b.value == a.value && b.index < a.index));
            return take ? b : a;
        }
    }
    // fold element x at global index i
    static __device__ __forceinline__ A fold(A a, T x, uint32_t i)
    {
        if constexpr (kArg) return combine(a, A{x, i});
        else return combine(a, x);
    }
    // DPP inside rows of 16, then the four row results (wave-uniform)
    template <int CTRL>
    static __device__ __forceinline__ A dpp_acc(A a)
    {
        if constexpr (kArg) return A{dpp_perm<CTRL>(a.value), dpp_perm<CTRL>(a.index)};
        else return dpp_perm<CTRL>(a);
    }
    template <int CTRL, int ROW_MASK>
    static __device__ __forceinline__ A dpp_mv(A a, A old)
    {
        if constexpr (kArg)
            return A{dpp_move<CTRL, ROW_MASK>(a.value, old.value), dpp_move<CTRL, ROW_MASK>(a.index, old.index)};
        else return dpp_move<CTRL, ROW_MASK>(a, old);
    }
    static __device__ __forceinline__ A readlane_acc(A a, int l)
    {
        if constexpr (kArg) return A{read_lane(a.value, l), read_lane(a.index, l)};
        else return read_lane(a, l);
    }
    static __device__ __forceinline__ A wave_reduce(A a)
    {
        a = combine(a, dpp_acc<kDppQuadXor1>(a));
        a = combine(a, dpp_acc<kDppQuadXor2>(a));
        a = combine(a, dpp_acc<kDppRowHalfMirror>(a));
        a = combine(a, dpp_acc<kDppRowMirror>(a));
        return combine(combine(readlane_acc(a, 0), readlane_acc(a, 16)), combine(readlane_acc(a, 32), readlane_acc(a, 48)));
    }
};

// Where the segments come from: CSR begin/end arrays or fixed-size runs.
struct SegBounds {
    const uint32_t *begin, *end;  // CSR (null for fixed-size)
    uint32_t size;                // fixed-size segment length
};

template <bool FIXED>
__device__ __forceinline__ void seg_bounds(const SegBounds &sb, uint64_t s, uint64_t S, uint32_t &b, uint32_t &len)
{
    b = 0;
    len = 0;
    if (s < S) {
        if constexpr (FIXED) {
            b = (uint32_t)s * sb.size;
            len = sb.size;
        } else {
            b = sb.begin[s];
            const uint32_t e = sb.end[s];
            len = e > b ? e - b : 0;
        }
    }
}

// Result of one segment: out[s] (+ index_out[s] for Arg*).
template <class T, int OP>
__device__ __forceinline__ void seg_store(typename SegAcc<T, OP>::A acc, uint32_t b, T init, T *out,
                                          uint32_t *index_out, uint64_t s)
{
    using Acc = SegAcc<T, OP>;
    if constexpr (Acc::kArg) {
        const bool empty = acc.index == kNoIndex;
        out[s] = empty ? (OP == kSegArgMax ? std::numeric_limits<T>::lowest() : std::numeric_limits<T>::max())
                       : acc.value;
        index_out[s] = empty ? 1u : acc.index - b;
    } else {
        out[s] = Acc::combine(init, acc);
    }
}

// The whole workgroup streams segment s (4 loads in flight per thread) and
// thread 0 stores its result.  Every thread must call it (barriers).
template <class T, int OP, bool FIXED>
__device__ __forceinline__ void wg_reduce_segment(const T *__restrict__ in, T *__restrict__ out,
                                                  uint32_t *__restrict__ index_out, uint64_t s, uint64_t S,
                                                  const SegBounds &sb, T init,
                                                  typename SegAcc<T, OP>::A (&s_wave)[kSegWaves])
{
    using Acc = SegAcc<T, OP>;
    using A = typename Acc::A;
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    uint32_t lb, llen;
    seg_bounds<FIXED>(sb, s, S, lb, llen);
    const uint64_t le = (uint64_t)lb + llen;
    A a0 = Acc::identity(), a1 = a0, a2 = a0, a3 = a0;
    uint64_t i = (uint64_t)lb + tid;
    for (; i + 3 * kSegBlock < le; i += 4 * kSegBlock) {
        const T x0 = in[i], x1 = in[i + kSegBlock], x2 = in[i + 2 * kSegBlock], x3 = in[i + 3 * kSegBlock];
        a0 = Acc::fold(a0, x0, (uint32_t)i);
        a1 = Acc::fold(a1, x1, (uint32_t)(i + kSegBlock));
        a2 = Acc::fold(a2, x2, (uint32_t)(i + 2 * kSegBlock));
        a3 = Acc::fold(a3, x3, (uint32_t)(i + 3 * kSegBlock));
    }
    for (; i < le; i += kSegBlock) a0 = Acc::fold(a0, in[i], (uint32_t)i);
    A a = Acc::combine(Acc::combine(a0, a1), Acc::combine(a2, a3));
    a = Acc::wave_reduce(a);
    if (lane == 0) s_wave[wave] = a;
    __syncthreads();
    if (tid == 0) {
        A r = s_wave[0];
#pragma unroll
        for (int w = 1; w < kSegWaves; ++w) r = Acc::combine(r, s_wave[w]);
        seg_store<T, OP>(r, lb, init, out, index_out, s);
    }
    __syncthreads();
}

// ---- flat path: a wave whose 64 segments tile one contiguous range
// [B, E) streams that range in chunks with coalesced 16-byte loads instead
// of walking its segments 8 at a time (24 dependent load round trips per
// wave for mean length 128).  Each chunk goes through LDS so that lane l
// then holds kFlatEpl consecutive elements; the lane folds them in order,
// writing every segment that starts and ends inside it.  The open segment
// at each lane's start comes from a segmented scan across the lanes (plus
// the open segment carried from the previous chunk): with it a lane writes
// the first segment that ends inside it.  The last segment of the range is
// written after the last chunk, empty segments at the start.  Per segment the
// fold order is the element order: first the lanes before, then the lane's
// own elements.
template <class T>
constexpr int flat_epl()
{
    return 64 / (int)sizeof(T);  // 4 KiB of elements per wave per chunk
}
template <class T>
struct FlatSmem {
    uint32_t bnd[kSegWaves][kSegPerWave + 1];
    uint32_t slots[kSegWaves][kWave];
    T stage[kSegWaves][kWave * (flat_epl<T>() + 1)];  // +1: conflict-free column reads
};

// Segmented inclusive scan of (flag, acc) pairs across the lanes (DPP steps
// of wave_inclusive_scan): a flagged lane restarts the fold.
template <class Acc>
__device__ __forceinline__ void flat_seg_scan(bool &f, typename Acc::A &v)
{
    using A = typename Acc::A;
    const A id = Acc::identity();
    auto step = [&](int fu, A vu) {
        v = f ? v : Acc::combine(vu, v);
        f = f || fu != 0;
    };
    step(dpp_move<kDppRowShr + 1>((int)f, 0), Acc::template dpp_mv<kDppRowShr + 1, 0xF>(v, id));
    step(dpp_move<kDppRowShr + 2>((int)f, 0), Acc::template dpp_mv<kDppRowShr + 2, 0xF>(v, id));
    step(dpp_move<kDppRowShr + 4>((int)f, 0), Acc::template dpp_mv<kDppRowShr + 4, 0xF>(v, id));
    step(dpp_move<kDppRowShr + 8>((int)f, 0), Acc::template dpp_mv<kDppRowShr + 8, 0xF>(v, id));
    step(dpp_move<kDppRowBcast15, 0xA>((int)f, 0), Acc::template dpp_mv<kDppRowBcast15, 0xA>(v, id));
    step(dpp_move<kDppRowBcast31, 0xC>((int)f, 0), Acc::template dpp_mv<kDppRowBcast31, 0xC>(v, id));
}

template <class T, int OP>
__device__ __forceinline__ void flat_segments(const T *__restrict__ in, T *__restrict__ out,
                                              uint32_t *__restrict__ index_out, T init, uint64_t wseg0,
                                              uint32_t nvalid, uint32_t b, uint32_t len, uint32_t *bnd,
                                              uint32_t *slots, T *stage)
{
    using Acc = SegAcc<T, OP>;
    using A = typename Acc::A;
    constexpr int EPL = flat_epl<T>();
    constexpr int VEC = 16 / (int)sizeof(T);
    constexpr int LOADS = EPL / VEC;
    constexpr uint32_t CH = kWave * EPL;
    const uint32_t lane = lane_id();
    const bool valid = lane < nvalid;
    const uint32_t B = (uint32_t)__builtin_amdgcn_readfirstlane((int)b);
    const uint32_t E = (uint32_t)__builtin_amdgcn_readlane((int)(b + len), (int)nvalid - 1);
    bnd[lane] = valid ? b : E;
    if (lane == 0) bnd[kSegPerWave] = E;
    __builtin_amdgcn_wave_barrier();
    if (valid && len == 0) seg_store<T, OP>(Acc::identity(), b, init, out, index_out, wseg0 + lane);
    const uint32_t A0 = B & ~(uint32_t)(VEC - 1);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(in + A0, (E - A0) * (uint32_t)sizeof(T));  // reads past E give 0
    const uint32_t nch = (E - A0 + CH - 1) / CH;
    auto emit = [&](uint32_t sid, A acc) { seg_store<T, OP>(acc, bnd[sid], init, out, index_out, wseg0 + sid); };
    A carry = Acc::identity();
    // coalesced loads of chunk c: lane l, load k -> elements k*64*VEC + l*VEC .. + VEC - 1
    u32x4 v[LOADS];
    auto load_chunk = [&](uint32_t c) {
#pragma unroll
        for (int k = 0; k < LOADS; ++k)
            v[k] = buf_ld16_nt(r, (c * CH + (uint32_t)k * kWave * VEC + lane * VEC) * (uint32_t)sizeof(T), 0);
    };
    if (nch) load_chunk(0);
#pragma unroll 1
    for (uint32_t c = 0; c < nch; ++c) {
        const uint32_t base = A0 + c * CH;  // element index of the chunk's first element
        // chunk element q = k*64*VEC + lane*VEC + j belongs to lane q / EPL, position q % EPL
#pragma unroll
        for (int k = 0; k < LOADS; ++k) {
            T e[VEC];
            unpack16<T>(v[k], e);
#pragma unroll
            for (int j = 0; j < VEC; ++j) {
                const uint32_t q = (uint32_t)k * kWave * VEC + lane * VEC + (uint32_t)j;
                stage[(q / EPL) * (EPL + 1) + q % EPL] = e[j];
            }
        }
        if (c + 1 < nch) load_chunk(c + 1);  // in flight while this chunk is folded
        __builtin_amdgcn_wave_barrier();
        T x[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) x[j] = stage[lane * (EPL + 1) + j];
        __builtin_amdgcn_wave_barrier();

        // the segment holding element p0 - 1 is the last boundary below p0.
        // Boundaries are counted per lane: boundary i (lane i's) is below
        // the first element of every lane after slot (b_i - base) / EPL, so
        // the count is a prefix sum of a 64-entry histogram of slots (those
        // below the chunk counted by one ballot).
        const uint32_t p0 = base + lane * EPL;
        const uint32_t bi = valid ? b : E;
        const uint32_t below = (uint32_t)__builtin_popcountll(ballot(bi < base));
        slots[lane] = 0;
        __builtin_amdgcn_wave_barrier();
        if (bi >= base && bi - base < CH - EPL) atomicAdd(&slots[(bi - base) / EPL + 1], 1u);
        __builtin_amdgcn_wave_barrier();
        const uint32_t cnt = below + wave_inclusive_scan(slots[lane], SumOp());
        uint32_t sid = cnt > 0 ? (cnt - 1 < kSegPerWave ? cnt - 1 : kSegPerWave - 1) : 0u;
        A acc = Acc::identity(), first_acc = Acc::identity();
        uint32_t first_sid = 0;
        bool seen = false;
        if constexpr (!Acc::kArg) {
            // branch-free: bit t of hmask = a segment starts at p0 + t; fold
            // with restarts, values back into this lane's LDS row
            const uint32_t lim = p0 + EPL < E ? p0 + EPL : E;
            uint32_t hmask = 0;
            {
                uint32_t i = sid + 1, q = bnd[i];
                while (q < lim) {
                    hmask |= 1u << (q - p0);
                    q = bnd[++i];
                }
            }
            const uint32_t vlo = B > p0 ? B - p0 : 0u;
            const uint32_t vhi = lim > p0 ? lim - p0 : 0u;
            A v = Acc::identity();
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const A xj = (uint32_t)j >= vlo && (uint32_t)j < vhi ? A(x[j]) : Acc::identity();
                v = ((hmask >> j) & 1u) ? xj : Acc::combine(v, xj);
                x[j] = v;
            }
            acc = v;
            seen = hmask != 0;
            if (__builtin_amdgcn_ballot_w64(seen)) {
#pragma unroll
                for (int j = 0; j < EPL; ++j) stage[lane * (EPL + 1) + j] = x[j];
                __builtin_amdgcn_wave_barrier();
                if (seen) {
                    // walk the boundaries again: the segment before each one
                    // ends at t - 1; the first of them may have started in
                    // earlier lanes (written after the scan below)
                    uint32_t prev = sid, i = sid + 1, q = bnd[i];
                    bool first = true;
                    while (q < lim) {
                        uint32_t q2 = bnd[i + 1];
                        while (q2 == q) q2 = bnd[++i + 1];  // empty segments starting at q
                        const uint32_t t = q - p0;
                        const A val = t ? A(stage[lane * (EPL + 1) + t - 1]) : Acc::identity();
                        if (first) {
                            first_sid = prev;
                            first_acc = val;
                            first = false;
                        } else {
                            emit(prev, val);
                        }
                        prev = i++;
                        q = q2;
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
        } else {
            uint32_t nb = bnd[sid + 1];
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const uint32_t p = p0 + (uint32_t)j;
                if (p >= B && p < E) {
                    if (p == nb) {  // segment sid ended at p - 1
                        if (!seen) {
                            first_sid = sid;
                            first_acc = acc;
                            seen = true;
                        } else {
                            emit(sid, acc);
                        }
                        do {  // skip the empty segments that start and end at p
                            ++sid;
                            nb = bnd[sid + 1];
                        } while (nb == p);
                        acc = Acc::identity();
                    }
                    acc = Acc::fold(acc, x[j], p);
                }
            }
        }
        // open segment at each lane's start: carry, then the lanes before
        bool f = seen;
        A inc = acc;
        flat_seg_scan<Acc>(f, inc);
        const int fprev = wave_shr1((int)f, 0);
        const A iprev = Acc::template dpp_mv<kDppWaveShr1, 0xF>(inc, Acc::identity());
        const A open = lane == 0 ? carry : (fprev ? iprev : Acc::combine(carry, iprev));
        if (seen) emit(first_sid, Acc::combine(open, first_acc));
        const bool f63 = __builtin_amdgcn_readlane((int)f, kWave - 1) != 0;
        const A i63 = Acc::readlane_acc(inc, kWave - 1);
        carry = f63 ? i63 : Acc::combine(carry, i63);
    }
    // the range's last non-empty segment ends at E
    const uint64_t ne = ballot(valid && len > 0);
    if (ne && lane == 0) emit(63u - (uint32_t)__builtin_clzll(ne), carry);
}

template <class T, int OP, bool FIXED>
__global__ __launch_bounds__(kSegBlock) void segment_reduce_kernel(const T *__restrict__ in, T *__restrict__ out,
                                                                   uint32_t *__restrict__ index_out, uint64_t S,
                                                                   SegBounds sb, T init, int vec_ok)
{
    using Acc = SegAcc<T, OP>;
    using A = typename Acc::A;
    constexpr int kBatch = kSegWaves * kSegPerWave;
    __shared__ uint32_t s_long[kBatch];
    __shared__ uint32_t s_nlong;
    __shared__ A s_wave[kSegWaves];
    __shared__ FlatSmem<T> s_flat;

    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const uint64_t wseg0 = (uint64_t)blockIdx.x * kBatch + (uint64_t)wave * kSegPerWave;
    // lanes 0..kSegPerWave-1 hold the bounds of the wave's segments (one coalesced load)
    uint32_t b = 0, len = 0;
    if (lane < (uint32_t)kSegPerWave) seg_bounds<FIXED>(sb, wseg0 + lane, S, b, len);
    if (tid == 0) s_nlong = 0;
    __syncthreads();
    const bool is_long = len > kSegLong;
    if (is_long) s_long[atomicAdd(&s_nlong, 1u)] = (uint32_t)(wave * kSegPerWave + lane);

    // flat path when the wave's segments tile one range and none is long
    const uint32_t nvalid = wseg0 < S ? (uint32_t)(S - wseg0 < kSegPerWave ? S - wseg0 : kSegPerWave) : 0u;
    const uint32_t b_next = (uint32_t)__shfl_down((int)b, 1);
    const bool breaks = lane < nvalid && (len > kSegLong || (lane + 1 < nvalid && b + len != b_next));
    if (vec_ok && nvalid > 0 && ballot(breaks) == 0) {
        flat_segments<T, OP>(in, out, index_out, init, wseg0, nvalid, b, len, s_flat.bnd[wave], s_flat.slots[wave],
                             s_flat.stage[wave]);
    } else {
    A mine = Acc::identity();
#pragma unroll 1
    for (int j0 = 0; j0 < kSegPerWave; j0 += kSegGroup) {
        uint32_t bj[kSegGroup], lj[kSegGroup];
        uint32_t maxlen = 0;
#pragma unroll
        for (int u = 0; u < kSegGroup; ++u) {
            bj[u] = __builtin_amdgcn_readlane(b, j0 + u);
            const uint32_t l = __builtin_amdgcn_readlane(len, j0 + u);
            lj[u] = l > kSegLong ? 0u : l;  // long segments: workgroup path below
            maxlen = lj[u] > maxlen ? lj[u] : maxlen;
        }
        if (maxlen == 0) continue;
        A acc[kSegGroup];
#pragma unroll
        for (int u = 0; u < kSegGroup; ++u) acc[u] = Acc::identity();
#pragma unroll 1
            for (uint32_t c = lane; c < maxlen; c += 2 * kWave) {
                T x0[kSegGroup], x1[kSegGroup];
#pragma unroll
                for (int u = 0; u < kSegGroup; ++u) {
                    x0[u] = c < lj[u] ? in[(uint64_t)bj[u] + c] : T(0);
                    x1[u] = c + kWave < lj[u] ? in[(uint64_t)bj[u] + c + kWave] : T(0);
                }
#pragma unroll
                for (int u = 0; u < kSegGroup; ++u) {
                    if constexpr (OP == kSegSum) {
                        acc[u] = Acc::fold(Acc::fold(acc[u], x0[u], 0), x1[u], 0);  // out-of-range loads are 0
                    } else {
                        if (c < lj[u]) acc[u] = Acc::fold(acc[u], x0[u], bj[u] + c);
                        if (c + kWave < lj[u]) acc[u] = Acc::fold(acc[u], x1[u], bj[u] + c + kWave);
                    }
                }
            }
#pragma unroll
        for (int u = 0; u < kSegGroup; ++u) {
            if (lj[u] == 0) continue;
            const A r = Acc::wave_reduce(acc[u]);
            if (lane == (uint32_t)(j0 + u)) mine = r;
        }
    }
    if (lane < (uint32_t)kSegPerWave && wseg0 + lane < S && !is_long)
        seg_store<T, OP>(mine, b, init, out, index_out, wseg0 + lane);
    }

    // ---- long segments: the whole workgroup streams each one
    __syncthreads();
    const uint32_t nlong = s_nlong;
    for (uint32_t q = 0; q < nlong; ++q)
        wg_reduce_segment<T, OP, FIXED>(in, out, index_out, (uint64_t)blockIdx.x * kBatch + s_long[q], S, sb, init,
                                        s_wave);
}

// Fixed-size segments longer than kSegLong: one workgroup per segment.
template <class T, int OP>
__global__ __launch_bounds__(kSegBlock) void segment_reduce_wg_kernel(const T *__restrict__ in, T *__restrict__ out,
                                                                      uint32_t *__restrict__ index_out, uint64_t S,
                                                                      SegBounds sb, T init)
{
    __shared__ typename SegAcc<T, OP>::A s_wave[kSegWaves];
    for (uint64_t s = blockIdx.x; s < S; s += gridDim.x) wg_reduce_segment<T, OP, true>(in, out, index_out, s, S, sb, init, s_wave);
}

// Workgroups of `kernel` the current device holds at once (cached per kernel
// and device).
template <class K>
int resident_blocks(K kernel, DeviceCache &cache)
{
    return device_cached(cache, [kernel] {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void *>(kernel), kSegBlock, 0) !=
                hipSuccess ||
            per_cu <= 0)
            per_cu = 4;
        return per_cu * device_cus();
    });
}

template <class T, int OP, bool FIXED>
int segment_launch(const void *in_, void *out_, uint32_t *index_out, uint64_t S, SegBounds sb, const void *init_,
                   hipStream_t s)
{
    if (S == 0) return LCPP_OK;
    const T *in = static_cast<const T *>(in_);
    T *out = static_cast<T *>(out_);
    if (!out || (OP >= kSegArgMin && !index_out)) return LCPP_ERR_INVALID_ARG;
    if (!FIXED && (!sb.begin || !sb.end || !in)) return LCPP_ERR_INVALID_ARG;
    if (FIXED && sb.size && !in) return LCPP_ERR_INVALID_ARG;
    if (S > 0xFFFFFFFFull || ceil_div(S, (uint64_t)kSegWaves * kSegPerWave) > 0x7FFFFFFFull) return LCPP_ERR_INVALID_ARG;
    if (FIXED && (uint64_t)sb.size * S > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;  // 32-bit element offsets
    T init = SegAcc<T, OP >= kSegArgMin ? kSegSum : OP>::identity();
    if constexpr (OP < kSegArgMin) {
        if (init_) memcpy(&init, init_, sizeof(T));
    }
    if (FIXED && sb.size > kSegLong) {
        static DeviceCache cap;
        const uint64_t c = (uint64_t)resident_blocks(&segment_reduce_wg_kernel<T, OP>, cap);
        const uint32_t grid = (uint32_t)(S < c ? S : c);
        LCPP_LAUNCH("segment_reduce_wg", s,
                    (segment_reduce_wg_kernel<T, OP><<<grid, kSegBlock, 0, s>>>(in, out, index_out, S, sb, init)));
        LCPP_CHECK_LAUNCH();
        return LCPP_OK;
    }
    const uint64_t blocks = ceil_div(S, (uint64_t)kSegWaves * kSegPerWave);
    const uint32_t grid = (uint32_t)blocks;
    const int vec_ok = (reinterpret_cast<uintptr_t>(in) & 15) == 0;
    LCPP_LAUNCH("segment_reduce", s,
                (segment_reduce_kernel<T, OP, FIXED><<<grid, kSegBlock, 0, s>>>(in, out, index_out, S, sb, init, vec_ok)));
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

template <int OP, bool FIXED>
int segment_dispatch(lcpp_dtype t, const void *in, void *out, uint32_t *index_out, uint64_t S, SegBounds sb,
                     const void *init, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (t) {
    case LCPP_INT32: return segment_launch<int32_t, OP, FIXED>(in, out, index_out, S, sb, init, s);
    case LCPP_UINT32: return segment_launch<uint32_t, OP, FIXED>(in, out, index_out, S, sb, init, s);
    case LCPP_FLOAT32: return segment_launch<float, OP, FIXED>(in, out, index_out, S, sb, init, s);
    case LCPP_INT64: return segment_launch<int64_t, OP, FIXED>(in, out, index_out, S, sb, init, s);
    case LCPP_UINT64: return segment_launch<uint64_t, OP, FIXED>(in, out, index_out, S, sb, init, s);
    case LCPP_FLOAT64: return segment_launch<double, OP, FIXED>(in, out, index_out, S, sb, init, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

template <bool FIXED>
int segment_op_dispatch(lcpp_dtype t, lcpp_reduce_op op, const void *in, void *out, uint64_t S, SegBounds sb,
                        const void *init, void *stream)
{
    switch (op) {
    case LCPP_OP_SUM: return segment_dispatch<kSegSum, FIXED>(t, in, out, nullptr, S, sb, init, stream);
    case LCPP_OP_MIN: return segment_dispatch<kSegMin, FIXED>(t, in, out, nullptr, S, sb, init, stream);
    case LCPP_OP_MAX: return segment_dispatch<kSegMax, FIXED>(t, in, out, nullptr, S, sb, init, stream);
    default: return LCPP_ERR_INVALID_ARG;
    }
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

extern "C" int lcpp_segment_reduce_arg_temp_bytes(lcpp_dtype t, uint64_t, uint64_t, size_t *bytes)
{
    return lcpp_segment_reduce_temp_bytes(t, 0, bytes);
}

extern "C" int lcpp_segment_reduce_sum(lcpp_dtype t, void *, size_t, const void *in, void *out, uint64_t S,
                                       const uint32_t *begin, const uint32_t *end, void *stream)
{
    return segment_op_dispatch<false>(t, LCPP_OP_SUM, in, out, S, SegBounds{begin, end, 0}, nullptr, stream);
}

extern "C" int lcpp_segment_reduce(lcpp_dtype t, lcpp_reduce_op op, void *, size_t, const void *in, void *out,
                                   uint64_t S, const uint32_t *begin, const uint32_t *end, const void *init,
                                   void *stream)
{
    return segment_op_dispatch<false>(t, op, in, out, S, SegBounds{begin, end, 0}, init, stream);
}

extern "C" int lcpp_segment_reduce_fixed(lcpp_dtype t, lcpp_reduce_op op, void *, size_t, const void *in, void *out,
                                         uint64_t S, uint32_t segment_size, const void *init, void *stream)
{
    return segment_op_dispatch<true>(t, op, in, out, S, SegBounds{nullptr, nullptr, segment_size}, init, stream);
}

extern "C" int lcpp_segment_reduce_argmin(lcpp_dtype t, void *, size_t, const void *in, void *out,
                                          uint32_t *index_out, uint64_t S, const uint32_t *begin,
                                          const uint32_t *end, void *stream)
{
    return segment_dispatch<kSegArgMin, false>(t, in, out, index_out, S, SegBounds{begin, end, 0}, nullptr, stream);
}

extern "C" int lcpp_segment_reduce_argmax(lcpp_dtype t, void *, size_t, const void *in, void *out,
                                          uint32_t *index_out, uint64_t S, const uint32_t *begin,
                                          const uint32_t *end, void *stream)
{
    return segment_dispatch<kSegArgMax, false>(t, in, out, index_out, S, SegBounds{begin, end, 0}, nullptr, stream);
}

extern "C" int lcpp_segment_reduce_argmin_fixed(lcpp_dtype t, void *, size_t, const void *in, void *out,
                                                uint32_t *index_out, uint64_t S, uint32_t segment_size,
                                                void *stream)
{
    return segment_dispatch<kSegArgMin, true>(t, in, out, index_out, S, SegBounds{nullptr, nullptr, segment_size},
                                              nullptr, stream);
}

extern "C" int lcpp_segment_reduce_argmax_fixed(lcpp_dtype t, void *, size_t, const void *in, void *out,
                                                uint32_t *index_out, uint64_t S, uint32_t segment_size,
                                                void *stream)
{
    return segment_dispatch<kSegArgMax, true>(t, in, out, index_out, S, SegBounds{nullptr, nullptr, segment_size},
                                              nullptr, stream);
}
