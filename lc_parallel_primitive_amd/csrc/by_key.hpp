// by_key.hpp — tile machinery shared by ScanByKey and ReduceByKey (gfx950).
//
// Reference: device/details/scan_by_key.h:77-258 and
// device/details/reduce_by_key.h:61-258 (BlockLoad of keys and values,
// BlockDiscontinuity::FlagHeads, a BlockScan of (flag, value) pairs with
// ScanBySegmentOp / ReduceBySegmentOp, TilePrefixCallbackOp look-back).
//
// MI355X design: one 256-thread workgroup per tile of 8 x 16-byte value
// vectors per thread (8192 4-byte or 4096 8-byte values).  Thread t, vector
// k holds elements k*256*VP + t*VP + j (VP = 16 / sizeof(V), j < VP), so every
// load and store instruction covers contiguous memory; its keys sit at the
// same element indices.  Segment heads (key != previous key, compared in the
// key type) are one bit per element.  The tile is processed reduce-then-
// rescan: pass 1 folds each thread's elements into (has-head, value since
// the last head) pairs, a wave64 segmented scan of those pairs per vector,
// the wave totals through LDS; one wave runs the decoupled look-back
// (lookback.hpp), where a tile containing a head publishes INCLUSIVE at
// once; pass 2 rescans each thread's elements seeded with its exact prefix.
#pragma once

#include "lookback.hpp"

namespace lcpp {
namespace {

constexpr int kBkBlock = 256;
constexpr int kBkWaves = kBkBlock / kWave;
constexpr int kBkVecs = 8;

template <class V>
constexpr int bk_vp()
{
    return 16 / (int)sizeof(V);
}
template <class V>
constexpr uint32_t bk_tile()
{
    return (uint32_t)(kBkBlock * kBkVecs * bk_vp<V>());
}
template <class V>
uint64_t bk_tiles(uint64_t n)
{
    return n ? ceil_div(n, bk_tile<V>()) : 0;
}

// Binary operators with their identities (common/thread_operators.h:49-74).
template <class Op, class T>
__device__ __forceinline__ T op_identity()
{
    return Op::template identity<T>();
}

// Segment-pair fold (ScanBySegmentOp / ReduceBySegmentOp,
// common/thread_operators.h:85-127): (fa, a) then (fb, b).
template <class T, class Op>
__device__ __forceinline__ void seg_fold(bool &fa, T &a, bool fb, T b, Op op)
{
    a = fb ? b : op(a, b);
    fa = fa || fb;
}

// Inclusive wave64 segmented scan of (f, s) over lanes (lane order).
template <class T, class Op>
__device__ __forceinline__ void wave_seg_scan(bool &f, T &s, Op op)
{
    // the DPP steps of wave_inclusive_scan over (flag, value) pairs; lanes
    // with no source take (false, identity)
    const T id = op_identity<Op, T>();
    auto step = [&](int fu, T su) {
        s = f ? s : op(su, s);
        f = f || fu != 0;
    };
    step(dpp_move<kDppRowShr + 1>((int)f, 0), dpp_move<kDppRowShr + 1>(s, id));
    step(dpp_move<kDppRowShr + 2>((int)f, 0), dpp_move<kDppRowShr + 2>(s, id));
    step(dpp_move<kDppRowShr + 4>((int)f, 0), dpp_move<kDppRowShr + 4>(s, id));
    step(dpp_move<kDppRowShr + 8>((int)f, 0), dpp_move<kDppRowShr + 8>(s, id));
    step(dpp_move<kDppRowBcast15, 0xA>((int)f, 0), dpp_move<kDppRowBcast15, 0xA>(s, id));
    step(dpp_move<kDppRowBcast31, 0xC>((int)f, 0), dpp_move<kDppRowBcast31, 0xC>(s, id));
}

// Keys and values of one thread.
template <class K, class V>
struct BkRegs {
    static constexpr int VP = bk_vp<V>();
    K key[kBkVecs][VP];
    V val[kBkVecs][VP];
};

// Element offset (within the tile) of item (k, j) of thread t.
template <class V>
__device__ __forceinline__ uint32_t bk_elem(int k, uint32_t t, int j)
{
    return (uint32_t)k * kBkBlock * bk_vp<V>() + t * bk_vp<V>() + (uint32_t)j;
}

// Loads one tile.  `fast`: full tile and 16-byte aligned pointers; otherwise
// element-wise raw-buffer loads whose offsets (all in the VGPR operand) are
// range-checked against `valid` elements, returning 0 past it.  KEYS_FIRST
// issues every key load before the value loads, so that work on the keys
// alone can start while the values are still in flight (loads complete in
// issue order).
template <bool KEYS_FIRST = false, class K, class V>
__device__ __forceinline__ void bk_load(BkRegs<K, V> &r, const K *keys, const V *vals, uint64_t base,
                                        uint32_t valid, bool fast, uint32_t tid)
{
    constexpr int VP = bk_vp<V>();
    constexpr uint32_t KB = VP * sizeof(K);  // key bytes per thread and vector
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(keys + base, valid * (uint32_t)sizeof(K));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vals + base, valid * (uint32_t)sizeof(V));
    if (fast) {
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k) {
            if constexpr (!KEYS_FIRST) unpack16<V>(buf_ld16_nt(rv, tid * 16 + (uint32_t)k * kBkBlock * 16, 0), r.val[k]);
            const uint32_t ko = tid * KB + (uint32_t)k * kBkBlock * KB;
            if constexpr (KB == 16) {
                unpack16<K>(buf_ld16_nt(rk, ko, 0), r.key[k]);
            } else if constexpr (KB == 32) {
                K lo[2], hi[2];
                unpack16<K>(buf_ld16_nt(rk, ko, 0), lo);
                unpack16<K>(buf_ld16_nt(rk, ko + 16, 0), hi);
                r.key[k][0] = lo[0];
                r.key[k][1] = lo[1];
                r.key[k][2] = hi[0];
                r.key[k][3] = hi[1];
            } else {
                static_assert(KB == 8, "4-byte keys with 8-byte values");
                const auto w = __builtin_amdgcn_raw_buffer_load_b64(rk, (int)ko, 0, kPolicyNT);
                const uint32_t a = w[0], b = w[1];
                r.key[k][0] = __builtin_bit_cast(K, a);
                r.key[k][1] = __builtin_bit_cast(K, b);
            }
        }
        if constexpr (KEYS_FIRST) {
#pragma unroll
            for (int k = 0; k < kBkVecs; ++k)
                unpack16<V>(buf_ld16_nt(rv, tid * 16 + (uint32_t)k * kBkBlock * 16, 0), r.val[k]);
        }
    } else {
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
#pragma unroll
            for (int j = 0; j < VP; ++j) {
                const uint32_t e = bk_elem<V>(k, tid, j);
                r.val[k][j] = buf_ld_elem<V>(rv, e * (uint32_t)sizeof(V), 0);
                r.key[k][j] = buf_ld_elem<K>(rk, e * (uint32_t)sizeof(K), 0);
            }
    }
}

// Segment-head bits: bit k*VP + j is set when item (k, j) starts a segment
// (element 0 of the input, or key != previous key in the key type).  The
// previous key of a thread's first item comes from lane - 1 (a shuffle), the
// last lane of the previous wave or vector (LDS), or the key just before the
// tile.  prev0[k] receives the previous key of item (k, 0).  Contains a
// workgroup barrier.
template <class K, int VP>
__device__ __forceinline__ uint32_t bk_heads(const K (&key)[kBkVecs][VP], K (&prev0)[kBkVecs],
                                             K (&s_last)[kBkVecs][kBkWaves], K &s_pred, const K *keys,
                                             uint64_t base, uint32_t tile, uint32_t tid)
{
    const uint32_t lane = lane_id(), wave = tid / kWave;
    if (lane == kWave - 1) {
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k) s_last[k][wave] = key[k][VP - 1];
    }
    if (tid == 0) s_pred = tile > 0 ? keys[base - 1] : K(0);
    __syncthreads();
    uint32_t fl = 0;
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        const K up = shfl_up(key[k][VP - 1], 1);
        const K prev = lane > 0 ? up : wave > 0 ? s_last[k][wave - 1] : k > 0 ? s_last[k - 1][kBkWaves - 1] : s_pred;
        prev0[k] = prev;
        bool h = key[k][0] != prev;
        if (k == 0 && tid == 0 && tile == 0) h = true;
        fl |= (uint32_t)h << (k * VP);
#pragma unroll
        for (int j = 1; j < VP; ++j) fl |= (uint32_t)(key[k][j] != key[k][j - 1]) << (k * VP + j);
    }
    return fl;
}

// Pass 1 of one vector: (has-head, fold since the last head) of a thread's
// VP items.
template <class V, class Op, int VP>
__device__ __forceinline__ void bk_thread_pair(const V (&x)[VP], uint32_t bits, Op op, bool &f, V &s)
{
    f = false;
    s = op_identity<Op, V>();
#pragma unroll
    for (int j = 0; j < VP; ++j) seg_fold(f, s, ((bits >> j) & 1u) != 0, x[j], op);
}

}  // namespace
}  // namespace lcpp
