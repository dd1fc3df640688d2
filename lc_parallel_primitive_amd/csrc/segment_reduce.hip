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
//  * Contiguous flat path: a wave whose 64 segments are sorted and disjoint
//    (begin[s + 1] >= end[s]: CSR offsets that tile a range, or ranges with
//    gaps that hold fewer elements than the segments), none of them long,
//    streams the range from its first begin to its last end in 4 KiB chunks
//    of coalesced 16-byte loads, transposes each chunk through LDS so that
//    every lane holds consecutive elements, folds them in order restarting
//    at each segment begin, and completes the segment open at each lane's
//    start with a segmented scan (flat_segments below).
//  * Gather path, every other layout (unsorted, overlapping, wide gaps, an
//    input pointer that is not 16-byte aligned): the wave's segments are
//    concatenated into one virtual range and the same fold runs over it;
//    each chunk is gathered with one load per element, 64 consecutive
//    virtual elements per wave load, each element's segment found from a
//    bitmap of the segment ends in the chunk.  A wave whose segments span
//    2 GiB or more (one buffer resource covers less) folds one segment at a
//    time instead.
//  * Segments longer than kSegLong: their indices are compacted into LDS and
//    the whole workgroup streams each one (4 loads in flight per thread)
//    after its waves are done.  Fixed-size segments longer than kSegLong
//    take a workgroup-per-segment launch directly.
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
// Measured at C5 (2^27 f32, 2^20 segments of mean length 128, us): a wave
// walking its segments 8 at a time (one 64-lane load per segment and step)
// 113-124; the contiguous flat path 94 (a copy of it that only sums each
// wave's range, with no segment logic, runs in 87.5): per-element branches
// 105, branch-free fold 99, segment of each lane's first element by a
// binary search in LDS 99 against a slot histogram and a DPP scan 97, begin
// and end bitmaps of each chunk (no LDS walks) 95 -> 93 (the same 2-3 %
// for every op and layout).  Arg*
// on the flat path: per-element branches 166-173, branch-free fold with the
// arg positions packed in registers 111, combining in element order (one
// empty check, no index tie break) 104.  The same segments in a random
// order (gather path): walking 124 (Sum) / 155 (Min) / 312 (ArgMin); gather
// with each lane walking the segment ends in LDS 135 / 142 / 165, with a
// scalar walk over the chunk's ends 131 / 135 / 173, with the end bitmap
// and mbcnt 124 / 124 / 145, with the ordered combine 123 / 125 / 136
// (gathering the tiling layout: 104; with no segment lookup at all 96).
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
    // a then b in element order (every index of b above every index of a),
    // b not the identity: Arg* need neither b's empty check nor the index tie
    // break (the earlier pair wins a tie for ArgMin, the later for ArgMax)
    static __device__ __forceinline__ A combine_ordered(A a, A b)
    {
        if constexpr (!kArg) {
            return combine(a, b);
        } else {
            const bool take = a.index == kNoIndex || (OP == kSegArgMax ? b.value >= a.value : b.value < a.value);
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

// ---- flat path: a wave whose 64 segments are sorted and do not overlap
// (begin[s + 1] >= end[s]: CSR offsets that tile one range, or ranges with
// gaps between them that hold fewer elements than the segments do) streams
// the range [B, E) from its first begin to its last end in chunks with
// coalesced 16-byte loads, whatever the lengths of its segments (reading
// each segment on its own, with one 64-lane load per segment and step, took
// 24 dependent load round trips per wave for mean length 128).  Each chunk
// goes through LDS so that lane l then holds EPL consecutive elements p0 .. p0 +
// EPL - 1.  The lane folds them in order, restarting at every segment begin
// inside it, and the fold at a segment's last element is that segment's
// result when the segment began inside the lane.  The one segment that began
// before p0 and ends inside the lane (the open segment) is completed with
// the fold of the lanes before it, from a segmented scan restarted at the
// segment begins (plus the fold carried over from the previous chunk).
// Elements outside every segment (before B, in gaps, past E) are folded too
// but never reach a result: every result is read from a fold that restarted
// at its own segment's begin.  Empty segments are written at the start.  Per
// segment the fold order is the element order.
template <class T>
constexpr int flat_epl()
{
    return 64 / (int)sizeof(T);  // 4 KiB of elements per wave per chunk
}
// Largest range end the flat path takes: element indices of the last chunk
// stay below 2^32.
constexpr uint32_t kFlatMaxEnd = 0xFFFFFFFFu - 2u * kWave * 16u;
template <class T>
struct FlatSmem {
    uint32_t bnd[kSegWaves][kSegPerWave];     // begins
    uint32_t seg_of[kSegWaves][kSegPerWave];  // the r-th non-empty segment
    // bitmaps of a chunk (one bit per element): non-empty segment begins, and
    // their last elements
    uint32_t bbits[kSegWaves][kWave * flat_epl<T>() / 32];
    uint32_t ebits[kSegWaves][kWave * flat_epl<T>() / 32];
    T stage[kSegWaves][kWave * (flat_epl<T>() + 1)];  // +1: conflict-free column reads
    // gather: bitmap of the segment ends inside a chunk, one bit per virtual
    // element, and the element-index offset of each non-empty segment
    uint32_t gbits[kSegWaves][kWave * flat_epl<T>() / 32];
    uint32_t gdelta[kSegWaves][kSegPerWave];
};

// Segmented inclusive scan of (flag, acc) pairs across the lanes (DPP steps
// of wave_inclusive_scan): a flagged lane restarts the fold.  Every lane's
// acc holds at least one element (lanes without a DPP source get the
// identity, which the ordered combine passes over).
template <class Acc>
__device__ __forceinline__ void flat_seg_scan(bool &f, typename Acc::A &v)
{
    using A = typename Acc::A;
    const A id = Acc::identity();
    auto step = [&](int fu, A vu) {
        v = f ? v : Acc::combine_ordered(vu, v);
        f = f || fu != 0;
    };
    step(dpp_move<kDppRowShr + 1>((int)f, 0), Acc::template dpp_mv<kDppRowShr + 1, 0xF>(v, id));
    step(dpp_move<kDppRowShr + 2>((int)f, 0), Acc::template dpp_mv<kDppRowShr + 2, 0xF>(v, id));
    step(dpp_move<kDppRowShr + 4>((int)f, 0), Acc::template dpp_mv<kDppRowShr + 4, 0xF>(v, id));
    step(dpp_move<kDppRowShr + 8>((int)f, 0), Acc::template dpp_mv<kDppRowShr + 8, 0xF>(v, id));
    step(dpp_move<kDppRowBcast15, 0xA>((int)f, 0), Acc::template dpp_mv<kDppRowBcast15, 0xA>(v, id));
    step(dpp_move<kDppRowBcast31, 0xC>((int)f, 0), Acc::template dpp_mv<kDppRowBcast31, 0xC>(v, id));
}

// The element range [B, E) a wave's flat pass reads: the first begin and the
// last end of its NON-EMPTY segments (lanes < nvalid, in lane order; B = E = 0
// when every segment is empty).  An empty segment (end <= begin) need not lie
// inside the input at all, so it never widens the range: taking E from a
// last lane that is an empty segment with its begin past the input would let
// the wave's loads run past the input allocation.  Wave-uniform.
__device__ __forceinline__ void flat_range(uint32_t nvalid, uint32_t b, uint32_t len, uint32_t &B, uint32_t &E)
{
    const uint64_t ne = ballot(lane_id() < nvalid && len > 0);
    if (ne == 0) {
        B = E = 0;
        return;
    }
    const int first = __builtin_ctzll(ne), last = 63 - __builtin_clzll(ne);
    B = (uint32_t)__builtin_amdgcn_readlane((int)b, first);
    E = (uint32_t)__builtin_amdgcn_readlane((int)(b + len), last);
}

// Whether the wave's segments take the flat path: sorted, not overlapping,
// none long, gaps holding at most as many elements as the segments plus one
// chunk, and a range end below kFlatMaxEnd.  Wave-uniform.
template <class T>
__device__ __forceinline__ bool flat_eligible(uint32_t nvalid, uint32_t b, uint32_t len)
{
    constexpr uint32_t CH = kWave * flat_epl<T>();
    const uint32_t lane = lane_id();
    const uint32_t b_next = (uint32_t)__shfl_down((int)b, 1);
    const bool breaks = lane < nvalid && (len > kSegLong || (lane + 1 < nvalid && b + len > b_next));
    if (nvalid == 0 || ballot(breaks) != 0) return false;
    uint32_t B, E;
    flat_range(nvalid, b, len, B, E);
    const uint32_t total = wave_allreduce(lane < nvalid ? len : 0u, SumOp());  // <= 64 * kSegLong
    return E <= kFlatMaxEnd && (uint64_t)(E - B) <= 2ull * total + CH;
}

// GATHER: the wave's segments in any layout, concatenated into one virtual
// range (b, len: virtual begin and length; delta: element index minus
// g_lo minus virtual index, where [g_lo, g_lo + g_bytes / sizeof(T)) holds
// every element the wave reads).  Chunks are gathered with one load per
// element, 64 consecutive virtual elements per wave load (one or two runs of
// addresses); the fold runs on virtual indices, so Arg* positions relative
// to a segment's begin are the same.  write_empty: whether a zero-length
// lane is an empty segment to write (long segments, left to the workgroup
// path, are not).
template <class T, int OP, bool GATHER>
__device__ __forceinline__ void flat_segments(const T *__restrict__ in, T *__restrict__ out,
                                              uint32_t *__restrict__ index_out, T init, uint64_t wseg0,
                                              uint32_t nvalid, uint32_t b, uint32_t len, bool write_empty,
                                              uint32_t delta, uint32_t g_lo, uint32_t g_bytes, uint32_t *bnd,
                                              uint32_t *seg_of, uint32_t *bbits, uint32_t *ebits, T *stage,
                                              uint32_t *gbits, uint32_t *gdelta)
{
    using Acc = SegAcc<T, OP>;
    using A = typename Acc::A;
    constexpr int EPL = flat_epl<T>();
    constexpr int VEC = 16 / (int)sizeof(T);
    constexpr int LOADS = EPL / VEC;
    constexpr uint32_t CH = kWave * EPL;
    // Arg*: the position (0 .. EPL - 1) of each prefix's arg element, 4 bits
    // each, 8 per word
    constexpr int kPosWords = (EPL + 7) / 8;
    const uint32_t lane = lane_id();
    const bool valid = lane < nvalid;
    const uint32_t e = b + len;
    uint32_t B, E;
    flat_range(nvalid, b, len, B, E);
    // segments in order of their ends: the non-empty ones get ranks (their
    // ends are distinct and increasing), seg_of maps a rank to its segment
    const bool nonempty = valid && len > 0;
    const uint64_t ne_mask = ballot(nonempty);
    const uint32_t ne_rank = (uint32_t)__builtin_popcountll(ne_mask & ((1ull << lane) - 1));
    bnd[lane] = b;
    if (nonempty) {
        seg_of[ne_rank] = lane;
        if constexpr (GATHER) gdelta[ne_rank] = delta;
    }
    __builtin_amdgcn_wave_barrier();
    if (valid && len == 0 && write_empty) seg_store<T, OP>(Acc::identity(), b, init, out, index_out, wseg0 + lane);
    const uint32_t A0 = B & ~(uint32_t)(VEC - 1);
    // reads past E (contiguous) or outside [g_lo, ...) (gather) give 0
    const __amdgpu_buffer_rsrc_t r =
        GATHER ? make_rsrc(in + g_lo, g_bytes) : make_rsrc(in + A0, (E - A0) * (uint32_t)sizeof(T));
    const uint32_t nch = (E - A0 + CH - 1) / CH;
    auto emit = [&](uint32_t sid, A acc) { seg_store<T, OP>(acc, bnd[sid], init, out, index_out, wseg0 + sid); };
    A carry = Acc::identity();
    // contiguous: coalesced loads of chunk c, lane l, load k -> elements
    // k*64*VEC + l*VEC .. + VEC - 1.  Gather: load j -> virtual element
    // W + l (W = c*CH + j*64), read at W + l + the offset of the non-empty
    // segment holding it.  That segment's rank among the non-empty ones is
    // the count of non-empty segments whose last element lies before W + l:
    // those before the chunk, plus bits of a bitmap of the chunk's last
    // elements (the windows before this one, and this window's bits below
    // the lane: mbcnt).  Loads past E read some element of [g_lo, ...) or 0:
    // they only reach folds that never become results.
    u32x4 v[GATHER ? 1 : LOADS];
    T g[GATHER ? EPL : 1];
    const uint32_t gend = nonempty ? e : 0u;  // non-empty ends are distinct and >= 1
    auto load_chunk = [&](uint32_t c) {
        if constexpr (GATHER) {
            const uint32_t cb = c * CH;
            if (lane < CH / 32) gbits[lane] = 0;
            __builtin_amdgcn_wave_barrier();
            const uint32_t t = gend - 1u - cb;  // last element, chunk-relative
            if (nonempty && t < CH) atomicOr(&gbits[t / 32], 1u << (t % 32));
            __builtin_amdgcn_wave_barrier();
            const uint32_t word = lane < CH / 32 ? gbits[lane] : 0u;
            uint32_t rank = (uint32_t)__builtin_popcountll(ballot(nonempty && gend <= cb));
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const uint32_t wlo = (uint32_t)__builtin_amdgcn_readlane((int)word, 2 * j);
                const uint32_t whi = (uint32_t)__builtin_amdgcn_readlane((int)word, 2 * j + 1);
                const uint32_t rk = __builtin_amdgcn_mbcnt_hi(whi, __builtin_amdgcn_mbcnt_lo(wlo, rank));
                rank += (uint32_t)__builtin_popcount(wlo) + (uint32_t)__builtin_popcount(whi);
                const uint32_t dl = gdelta[rk < kSegPerWave ? rk : kSegPerWave - 1];
                // The byte offset of a segment's element is non-negative, but
                // its lane part (lane + dl) is not: left to itself the compiler
                // moves j * 64 (and cb) into the load's immediate / SGPR offset
                // and passes the lane part as the VGPR offset, wrapped below
                // zero.  Such loads are not reliably taken modulo 2^32: in a
                // random-order layout (wave's lowest-addressed segment in its
                // second 64-element window) a few of ~10^5 per launch read
                // wrong data, different ones from launch to launch.  The
                // opaque copy keeps the whole offset in the VGPR.
                uint32_t off = (cb + (uint32_t)j * kWave + lane + dl) * (uint32_t)sizeof(T);
                asm("" : "+v"(off));
                g[j] = buf_ld_elem_nt<T>(r, off);
            }
        } else {
#pragma unroll
            for (int k = 0; k < LOADS; ++k)
                v[k] = buf_ld16_nt(r, (c * CH + (uint32_t)k * kWave * VEC + lane * VEC) * (uint32_t)sizeof(T), 0);
        }
    };
    if (nch) load_chunk(0);
#pragma unroll 1
    for (uint32_t c = 0; c < nch; ++c) {
        const uint32_t base = A0 + c * CH;  // element index of the chunk's first element
        // chunk element q belongs to lane q / EPL, position q % EPL
        if constexpr (GATHER) {
            // q = j*64 + lane: row j*64/EPL + lane/EPL, column lane % EPL
            T *srow = stage + (lane / EPL) * (EPL + 1) + lane % EPL;
#pragma unroll
            for (int j = 0; j < EPL; ++j) srow[j * (kWave / EPL) * (EPL + 1)] = g[j];
        } else {
#pragma unroll
            for (int k = 0; k < LOADS; ++k) {
                T ev[VEC];
                unpack16<T>(v[k], ev);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    const uint32_t q = (uint32_t)k * kWave * VEC + lane * VEC + (uint32_t)j;
                    stage[(q / EPL) * (EPL + 1) + q % EPL] = ev[j];
                }
            }
        }
        if (c + 1 < nch) load_chunk(c + 1);  // in flight while this chunk is folded
        __builtin_amdgcn_wave_barrier();
        T x[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) x[j] = stage[lane * (EPL + 1) + j];
        __builtin_amdgcn_wave_barrier();

        // the chunk's begins and last elements as bitmaps: a lane's EPL bits are
        // its restarts (hmask) and the segments it completes (emask); the rank
        // of its first completed segment counts the ends before it
        const uint32_t p0 = base + lane * EPL;
        if (lane < CH / 32) {
            bbits[lane] = 0;
            ebits[lane] = 0;
        }
        __builtin_amdgcn_wave_barrier();
        {
            const uint32_t tb = b - base, te = e - 1u - base;  // past the chunk or below it: >= CH
            if (nonempty && tb < CH) atomicOr(&bbits[tb / 32], 1u << (tb % 32));
            if (nonempty && te < CH) atomicOr(&ebits[te / 32], 1u << (te % 32));
        }
        __builtin_amdgcn_wave_barrier();
        constexpr uint32_t kLaneBits = EPL >= 32 ? ~0u : (1u << EPL) - 1u;
        const uint32_t bw = lane * EPL / 32, bsh = lane * EPL % 32;
        const uint32_t hmask = (bbits[bw] >> bsh) & kLaneBits;
        const uint32_t emask = (ebits[bw] >> bsh) & kLaneBits;
        const uint32_t below = (uint32_t)__builtin_popcountll(ballot(nonempty && e <= base));
        const uint32_t ecount = (uint32_t)__builtin_popcount(emask);
        const uint32_t rank0 = below + wave_inclusive_scan(ecount, SumOp()) - ecount;
        // in-order fold with restarts; the lane's own prefix folds stay
        // readable at every position (Sum/Min/Max: in LDS; Arg*: the element
        // positions in pos, the values still in LDS)
        A lane_acc;
        uint32_t pos[kPosWords] = {};
        if constexpr (!Acc::kArg) {
            T run = x[0];
#pragma unroll
            for (int j = 1; j < EPL; ++j) {
                run = ((hmask >> j) & 1u) ? x[j] : Acc::combine(run, x[j]);
                x[j] = run;
            }
            lane_acc = run;
        } else {
            T av = x[0];
            uint32_t ap = 0;
#pragma unroll
            for (int j = 1; j < EPL; ++j) {
                // in-order fold: the later element wins ties only for ArgMax
                const bool better = OP == kSegArgMax ? x[j] >= av : x[j] < av;
                const bool take = ((hmask >> j) & 1u) || better;
                av = take ? x[j] : av;
                ap = take ? (uint32_t)j : ap;
                pos[j / 8] |= ap << (4 * (j % 8));
            }
            lane_acc = A{av, p0 + ap};
        }
        auto prefix_at = [&](uint32_t t) -> A {
            if constexpr (!Acc::kArg) {
                return stage[lane * (EPL + 1) + t];
            } else {
                const uint32_t pw = kPosWords > 1 && t >= 8 ? pos[kPosWords - 1] : pos[0];
                const uint32_t pt = (pw >> (4 * (t & 7))) & 15u;
                return A{stage[lane * (EPL + 1) + pt], p0 + pt};
            }
        };
        // segments ending inside the lane
        const bool has_end = emask != 0;
        if constexpr (!Acc::kArg) {
            if (ballot(has_end)) {
#pragma unroll
                for (int j = 0; j < EPL; ++j) stage[lane * (EPL + 1) + j] = x[j];
            }
            __builtin_amdgcn_wave_barrier();
        }
        bool has_first = false;
        uint32_t first_sid = 0;
        A first_acc = Acc::identity();
        if (has_end) {
            // the first completed segment began before p0 when no begin bit
            // precedes its last element (a later segment begins after it ends)
            uint32_t m = emask, rk = rank0;
            const uint32_t k0 = (uint32_t)__builtin_ctz(m);
            if ((hmask & ((2u << k0) - 1u)) == 0) {
                has_first = true;
                first_sid = seg_of[rk];
                first_acc = prefix_at(k0);
                m &= m - 1;
                ++rk;
            }
            while (m) {
                emit(seg_of[rk], prefix_at((uint32_t)__builtin_ctz(m)));
                m &= m - 1;
                ++rk;
            }
        }
        __builtin_amdgcn_wave_barrier();  // LDS reads done before the next chunk's stage writes
        // open segment at each lane's start: carry, then the lanes before
        bool f = hmask != 0;
        A inc = lane_acc;
        flat_seg_scan<Acc>(f, inc);
        const int fprev = wave_shr1((int)f, 0);
        const A iprev = Acc::template dpp_mv<kDppWaveShr1, 0xF>(inc, Acc::identity());
        const A open = lane == 0 ? carry : (fprev ? iprev : Acc::combine_ordered(carry, iprev));
        if (has_first) emit(first_sid, Acc::combine_ordered(open, first_acc));
        const bool f63 = __builtin_amdgcn_readlane((int)f, kWave - 1) != 0;
        const A i63 = Acc::readlane_acc(inc, kWave - 1);
        carry = f63 ? i63 : Acc::combine_ordered(carry, i63);
    }
}

// A wave whose segments span 2 GiB or more: one segment at a time,
// lane l folding elements l, l + 64, ... (long segments are left to the
// workgroup path).
template <class T, int OP>
__device__ __forceinline__ void wave_segments(const T *__restrict__ in, T *__restrict__ out,
                                              uint32_t *__restrict__ index_out, T init, uint64_t wseg0,
                                              uint32_t nvalid, uint32_t b, uint32_t len)
{
    using Acc = SegAcc<T, OP>;
    using A = typename Acc::A;
    const uint32_t lane = lane_id();
#pragma unroll 1
    for (uint32_t s = 0; s < nvalid; ++s) {
        const uint32_t bs = (uint32_t)__builtin_amdgcn_readlane((int)b, (int)s);
        const uint32_t ls = (uint32_t)__builtin_amdgcn_readlane((int)len, (int)s);
        if (ls > kSegLong) continue;
        A acc = Acc::identity();
#pragma unroll 1
        for (uint32_t i = lane; i < ls; i += kWave) acc = Acc::fold(acc, in[(uint64_t)bs + i], bs + i);
        const A res = Acc::wave_reduce(acc);
        if (lane == 0) seg_store<T, OP>(res, bs, init, out, index_out, wseg0 + s);
    }
}

// Six waves per SIMD: the register allocator is held to 80 VGPRs (the gather
// path's full-offset loads otherwise take Arg* of 4-byte types to 82, five
// waves); nothing spills.  Interleaved A/B at C5 against the split-offset
// loads, us: Sum 91.1 / 90.9, ArgMin 101.2 / 99.9; segments in a random
// order, Sum 120.8 / 121.4, ArgMin 133.5 / 134.3.
template <class T, int OP, bool FIXED>
__global__ __launch_bounds__(kSegBlock) __attribute__((amdgpu_waves_per_eu(6))) void segment_reduce_kernel(const T *__restrict__ in, T *__restrict__ out,
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

    // contiguous flat path when the wave's segments are sorted, disjoint and
    // none is long; else the gather form over the concatenated segments
    const uint32_t nvalid = wseg0 < S ? (uint32_t)(S - wseg0 < kSegPerWave ? S - wseg0 : kSegPerWave) : 0u;
    if (vec_ok && flat_eligible<T>(nvalid, b, len)) {
        flat_segments<T, OP, false>(in, out, index_out, init, wseg0, nvalid, b, len, true, 0u, 0u, 0u,
                                    s_flat.bnd[wave], s_flat.seg_of[wave], s_flat.bbits[wave], s_flat.ebits[wave],
                                    s_flat.stage[wave], s_flat.gbits[wave], s_flat.gdelta[wave]);
    } else if (nvalid > 0) {
        const uint32_t vlen = is_long ? 0u : len;
        // elements the gather reads: [lo, hi), under 2 GiB for one buffer
        // resource (offsets stay below 2^31)
        uint32_t lo = wave_allreduce(vlen ? b : ~0u, MinOp());
        const uint32_t hi = wave_allreduce(vlen ? b + vlen : 0u, MaxOp());
        if (hi <= lo) lo = 0;  // nothing to read
        const uint64_t bytes = hi > lo ? (uint64_t)(hi - lo) * sizeof(T) : 0;
        if (bytes <= 0x7FFFFFFFull) {
            const uint32_t vb = wave_inclusive_scan(vlen, SumOp()) - vlen;  // <= 64 * kSegLong
            flat_segments<T, OP, true>(in, out, index_out, init, wseg0, nvalid, vb, vlen, !is_long, b - lo - vb, lo,
                                       (uint32_t)bytes, s_flat.bnd[wave], s_flat.seg_of[wave], s_flat.bbits[wave],
                                       s_flat.ebits[wave], s_flat.stage[wave], s_flat.gbits[wave],
                                       s_flat.gdelta[wave]);
        } else {
            wave_segments<T, OP>(in, out, index_out, init, wseg0, nvalid, b, len);
        }
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
