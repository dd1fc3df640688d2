// reduce_by_key.hip — DeviceReduce::ReduceByKey for gfx950.
//
// Reference: device/device_reduce.h:110-125 (temp bytes), 277-318 (entry
// point), 462-516 (dispatch), device/details/reduce_by_key.h:61-258.
//
// Semantics: run r = the r-th maximal run of equal consecutive keys (keys
// compared in their own type); unique_out[r] = its key, aggregates_out[r] =
// the op-fold of its values, *num_runs_out = the number of runs.
//
// Design (tile machinery in by_key.hpp): two launches, and no wait in the
// pass over the data.
//  * rbk_tile: one 256-thread workgroup per tile of 8192 4-byte values
//    (4096 8-byte).  It finds the tile's segment heads and folds its runs with
//    tile-local prefixes (reduce-then-rescan, by_key.hpp; the prefixes of the
//    32 (vector, wave) slices are scanned once per tile by wave 0).  Entry i
//    of the tile is the run closed by its i-th head: that run's key and its
//    fold over this tile's elements (entry 0 lacks the part of its run in
//    earlier tiles).  The first 128 entries are gathered in LDS and stored
//    contiguously into the tile's slot of a dense staging area (runs of mean
//    128 give 64 per tile); further ones go to the tile's entries of a sparse
//    overflow area.  It also writes the tile's summary: its head count,
//    whether it has a head, and the fold since its last head (or of the whole
//    tile).  Tile 0 zeroes the status word and the emit launch's look-back
//    words (this launch reads none of them).
//    The reference's single pass (reduce_by_key.h:90-258) waits on two
//    decoupled look-backs per tile instead: the run count before the tile (a
//    plain scan) and the fold of the run entering it (a segmented scan).  On
//    this part those waits cost ~130 of ~500 us at 2^28 (int32 keys, f32
//    values, runs of mean 128): a tile here carries only 64 KiB against the
//    scan's 160 KiB, so a wait of a few microseconds is a large share of its
//    life.
//  * rbk_emit: one workgroup per 64 tiles.  Wave 0 scans their head counts;
//    the group's prefix is the sum of the counts every earlier group
//    publishes at its start (read 512 groups per round trip, no chain of
//    inclusive prefixes).  Wave 1 scans their segmented folds and takes the
//    fold entering the group from a decoupled look-back over groups (it stops
//    at the nearest group with a head).  Then the staged runs move to their
//    final positions, entry 0 of each tile completed with the fold entering
//    the tile, and the last group writes the last run and the run count (the
//    reference writes them from its last tile, reduce_by_key.h:231-254).
// Bytes: keys + values read once, plus (sizeof K + sizeof V) per run
// written, staged and moved (16 MB each way at 2^28, runs of 128).  Temp:
// the dense slots (128 entries per tile) and the overflow area (one entry per
// element, since every element may start a run; only entries of tiles with
// more than 128 runs are touched).
#include "by_key.hpp"

namespace lcpp {
namespace {

constexpr uint32_t kRbkGroup = 64;     // tiles per rbk_emit workgroup (one wave's lanes)
// Runs per tile gathered in LDS and stored contiguously into the tile's slot
// of the dense staging area (runs of mean 128 give 64 per tile); a tile's
// further runs go to its entries of the sparse overflow area.
constexpr uint32_t kRbkSlot = 128;

template <class K, class V>
struct RbkLayout {
    uint64_t tiles, groups, count_off, fold_off, cwords_off, vwords_off, pkeys_off, pvals_off, skeys_off, svals_off,
        total;
};
template <class K, class V>
RbkLayout<K, V> rbk_layout(uint64_t n)
{
    RbkLayout<K, V> L{};
    L.tiles = bk_tiles<V>(n);
    L.groups = ceil_div(L.tiles, kRbkGroup);
    // [status header | group look-back words (zeroed by tile 0) | tile
    //  summaries | dense staging slots | overflow staging]
    L.cwords_off = kStatusBytes;
    L.vwords_off = L.cwords_off + align_up(L.groups * 8, 256);
    L.count_off = L.vwords_off + align_up(L.groups * 8 * lb_words<V>(), 256);
    L.fold_off = L.count_off + align_up(L.tiles * 4, 256);
    L.pkeys_off = L.fold_off + align_up(L.tiles * sizeof(V), 256);
    L.pvals_off = L.pkeys_off + align_up(L.tiles * kRbkSlot * sizeof(K), 256);
    L.skeys_off = L.pvals_off + align_up(L.tiles * kRbkSlot * sizeof(V), 256);
    L.svals_off = L.skeys_off + align_up(L.tiles * bk_tile<V>() * sizeof(K), 256);
    L.total = L.svals_off + align_up(L.tiles * bk_tile<V>() * sizeof(V), 256);
    return L;
}

__global__ void rbk_zero_runs(uint32_t *num_runs) { *num_runs = 0; }

constexpr uint32_t kRbkHeadBit = 0x80000000u;  // summary count word: has a head

template <class K, class V, class Op>
__global__ __launch_bounds__(kBkBlock) void rbk_tile_kernel(const K *__restrict__ keys, const V *__restrict__ vin,
                                                            uint32_t n, uint32_t *__restrict__ tile_count,
                                                            V *__restrict__ tile_fold, K *__restrict__ pkeys,
                                                            V *__restrict__ pvals, K *__restrict__ skeys,
                                                            V *__restrict__ svals, int vec_ok,
                                                            uint64_t *__restrict__ zero_words, uint32_t zero_count)
{
    constexpr int VP = bk_vp<V>();
    constexpr uint32_t TILE = bk_tile<V>();
    // keys of the tile in LDS when they fit in 32 KiB: the registers that
    // held them are free for pass 2 (150 -> ~100 VGPRs)
    constexpr bool kKeysInLds = TILE * sizeof(K) <= 32768;
    __shared__ K s_keys[kKeysInLds ? TILE : 1];
    __shared__ K s_last[kBkVecs][kBkWaves];
    __shared__ K s_pred;
    __shared__ V s_S[kBkVecs][kBkWaves];
    __shared__ uint32_t s_C[kBkVecs][kBkWaves];
    __shared__ uint32_t s_F[kBkVecs];
    __shared__ K s_stk[kRbkSlot];
    __shared__ V s_stv[kRbkSlot];
    __shared__ V s_pw[kBkVecs * kBkWaves];
    __shared__ uint32_t s_cw[kBkVecs * kBkWaves];
    __shared__ uint32_t s_tc;

    Op op;
    const V ident = op_identity<Op, V>();
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint32_t base = tile * TILE;
    const uint32_t valid = n - base < TILE ? n - base : TILE;
    const bool fast = valid == TILE && vec_ok;

    BkRegs<K, V> r;
    bk_load<true>(r, keys, vin, base, valid, fast, tid);
    // the call's status word and the emit launch's look-back words start at
    // zero (this launch reads none of them: no separate fill launch)
    if (tile == 0)
        for (uint32_t i = tid; i < zero_count; i += kBkBlock) zero_words[i] = 0;
    if (tid < kBkVecs) s_F[tid] = 0;
    K prev0[kBkVecs];
    uint32_t fl = bk_heads<K, VP>(r.key, prev0, s_last, s_pred, keys, base, tile, tid);
    if (valid != TILE) {
        // a ragged last tile: items past n are neither heads nor folded
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
#pragma unroll
            for (int j = 0; j < VP; ++j)
                if (bk_elem<V>(k, tid, j) >= valid) {
                    fl &= ~(1u << (k * VP + j));
                    r.val[k][j] = ident;
                }
    }
    if constexpr (kKeysInLds) {
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
#pragma unroll
            for (int j = 0; j < VP; ++j) s_keys[bk_elem<V>(k, tid, j)] = r.key[k][j];
    }

    // head counts: per vector a wave scan, wave totals to LDS
    uint32_t exC[kBkVecs];
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        const uint32_t c = (uint32_t)__builtin_popcount((fl >> (k * VP)) & ((1u << VP) - 1u));
        const uint32_t ci = wave_inclusive_scan(c, SumOp());
        exC[k] = ci - c;
        if (lane == kWave - 1) s_C[k][wave] = ci;
    }

    // pass 1: per vector, (has-head, open fold) pairs, their wave scan, wave
    // totals to LDS
    V exS[kBkVecs];
    uint32_t exF = 0;
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        const uint32_t bits = (fl >> (k * VP)) & ((1u << VP) - 1u);
        bool f;
        V s;
        bk_thread_pair<V>(r.val[k], bits, op, f, s);
        wave_seg_scan(f, s, op);
        // a ds_bpermute shift measured faster here than the DPP wave shift
        const int fu = __shfl_up((int)f, 1);
        const V su = shfl_up(s, 1);
        exS[k] = lane == 0 ? ident : su;
        exF |= (uint32_t)(lane != 0 && fu) << k;
        if (lane == kWave - 1) {
            s_S[k][wave] = s;
            if (f) atomicOr(&s_F[k], 1u << wave);
        }
    }
    __syncthreads();

    // wave 0: the exclusive prefixes of the (vector, wave) slices in tile
    // order (lane k * 4 + w: its fold since the tile's last earlier head and
    // its head count), once per tile instead of a serial loop in every
    // thread; their inclusive totals are the tile's summary
    static_assert(kBkVecs * kBkWaves <= kWave, "one lane per slice");
    constexpr uint32_t kSlices = kBkVecs * kBkWaves;
    if (wave == 0) {
        const bool in = lane < kSlices;
        const uint32_t sk_ = in ? lane / kBkWaves : 0, sw = in ? lane % kBkWaves : 0;
        bool f = in && ((s_F[sk_] >> sw) & 1u) != 0;
        V v = in ? s_S[sk_][sw] : ident;
        const uint32_t c = in ? s_C[sk_][sw] : 0u;
        wave_seg_scan(f, v, op);
        const uint32_t ci = wave_inclusive_scan(c, SumOp());
        const V vu = shfl_up(v, 1);
        if (in) {
            s_pw[lane] = lane == 0 ? ident : vu;
            s_cw[lane] = ci - c;
        }
        const bool tf = read_lane((int)f, kSlices - 1) != 0;
        const V ts = read_lane(v, kSlices - 1);
        const uint32_t tc = read_lane(ci, kSlices - 1);
        if (lane == 0) {
            tile_count[tile] = tc | (tf ? kRbkHeadBit : 0u);
            tile_fold[tile] = ts;
            s_tc = tc;
        }
    }
    __syncthreads();

    // pass 2: rescan from the tile-local prefixes; the i-th head of the tile
    // closes staged entry i (the run before it)
    K *const sk = skeys + (uint64_t)tile * TILE;
    V *const sv = svals + (uint64_t)tile * TILE;
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        const V pw = s_pw[k * kBkWaves + wave];
        V s = ((exF >> k) & 1u) ? exS[k] : op(pw, exS[k]);
        uint32_t c = s_cw[k * kBkWaves + wave] + exC[k];
#pragma unroll
        for (int j = 0; j < VP; ++j) {
            const uint32_t e = bk_elem<V>(k, tid, j);
            if ((fl >> (k * VP + j)) & 1u) {
                K key;
                if constexpr (kKeysInLds) key = e > 0 ? s_keys[e - 1] : s_pred;
                else key = j > 0 ? r.key[k][j - 1] : prev0[k];
                // the first kRbkSlot entries are gathered in LDS and stored
                // contiguously below; c < the tile's head count <= TILE
                // keeps the rest inside the tile's overflow entries
                if (c < kRbkSlot) {
                    s_stk[c] = key;
                    s_stv[c] = s;
                } else {
                    sk[c] = key;
                    sv[c] = s;
                }
                ++c;
                s = r.val[k][j];
            } else {
                s = op(s, r.val[k][j]);  // identity past n
            }
        }
    }
    __syncthreads();
    const uint32_t m = s_tc < kRbkSlot ? s_tc : kRbkSlot;
    for (uint32_t i = tid; i < m; i += kBkBlock) {
        pkeys[(uint64_t)tile * kRbkSlot + i] = s_stk[i];
        pvals[(uint64_t)tile * kRbkSlot + i] = s_stv[i];
    }
}

// Sum of the head counts that groups 0 .. g-1 publish (each as PARTIAL, at
// its start, without waiting for any other group): up to 8 windows of 64
// groups are loaded before the first wait, so a group finds its prefix in one
// round trip per 512 predecessors instead of walking a chain of inclusive
// prefixes.  A word still unpublished is re-polled up to the spin limit, then
// counted as 0 and reported in the status word.  Every lane returns the sum.
__device__ uint32_t rbk_sum_before(const uint64_t *words, uint32_t g, const WaitCtl &ctl)
{
    constexpr uint32_t kBatch = 8;
    const uint32_t lane = lane_id();
    uint32_t acc = 0;
    for (uint32_t top = 0; top < g; top += kBatch * kWave) {
        uint64_t w[kBatch];
#pragma unroll
        for (uint32_t b = 0; b < kBatch; ++b) {
            const uint32_t j = top + b * kWave + lane;
            w[b] = j < g ? ld_relaxed(&words[j]) : (uint64_t)kStPartial;
        }
        for (uint32_t spins = 0;; ++spins) {
            bool missing = false;
#pragma unroll
            for (uint32_t b = 0; b < kBatch; ++b) missing |= (uint32_t)w[b] == kStInvalid;
            if (ballot(missing) == 0) break;
            if (spins + 1 >= ctl.spin_limit) {
                if (lane == 0) report_timeout(ctl);  // count what has been published
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (uint32_t b = 0; b < kBatch; ++b) {
                const uint32_t j = top + b * kWave + lane;
                if ((uint32_t)w[b] == kStInvalid) w[b] = ld_relaxed(&words[j]);
            }
        }
        uint32_t s = 0;
#pragma unroll
        for (uint32_t b = 0; b < kBatch; ++b) s += (uint32_t)(w[b] >> 32);
        acc += wave_allreduce(s, SumOp());
    }
    return acc;
}

template <class K, class V, class Op>
__global__ __launch_bounds__(kBkBlock) void rbk_emit_kernel(const K *__restrict__ keys, uint32_t n, uint32_t tiles,
                                                            const uint32_t *__restrict__ tile_count,
                                                            const V *__restrict__ tile_fold,
                                                            const K *__restrict__ pkeys, const V *__restrict__ pvals,
                                                            const K *__restrict__ skeys, const V *__restrict__ svals,
                                                            K *__restrict__ unique_out, V *__restrict__ agg_out,
                                                            uint32_t *__restrict__ num_runs, uint64_t *cwords,
                                                            uint64_t *vwords, WaitCtl ctl)
{
    constexpr uint32_t TILE = bk_tile<V>();
    __shared__ uint32_t s_cnt[kRbkGroup], s_base[kRbkGroup];
    __shared__ V s_vpre[kRbkGroup];
    __shared__ uint32_t s_gcount;
    __shared__ V s_gfold;

    Op op;
    const V ident = op_identity<Op, V>();
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const uint32_t g = blockIdx.x;
    const uint32_t t0 = g * kRbkGroup;
    const uint32_t ng = tiles - t0 < kRbkGroup ? tiles - t0 : kRbkGroup;

    // waves 0 and 1: the group's summaries, one tile per lane; wave 0 scans
    // the head counts and runs their look-back over groups, wave 1 the
    // segmented folds
    if (wave < 2) {
        const bool in = lane < ng;
        const uint32_t cw = in ? tile_count[t0 + lane] : 0u;
        const uint32_t cnt = cw & ~kRbkHeadBit;
        if (wave == 0) {
            const uint32_t ci = wave_inclusive_scan(cnt, SumOp());
            const uint32_t total = read_lane(ci, kWave - 1);
            if (lane == 0) lb_publish(cwords, g, total, kStPartial, ctl);
            const uint32_t pre = rbk_sum_before(cwords, g, ctl);
            s_cnt[lane] = cnt;
            s_base[lane] = pre + ci - cnt;
            if (lane == 0) s_gcount = pre + total;
        } else {
            bool f = in && (cw & kRbkHeadBit) != 0;
            V v = in ? tile_fold[t0 + lane] : ident;
            wave_seg_scan(f, v, op);
            const bool gf = read_lane((int)f, kWave - 1) != 0;
            const V gv = read_lane(v, kWave - 1);
            const V pre = lb_segmented_tile<kWave>(vwords, g, gv, gf, true, op, ident, ctl);
            // exclusive segmented fold entering tile t0 + lane
            const int fu = __shfl_up((int)f, 1);
            const V vu = shfl_up(v, 1);
            const V ex = lane == 0 ? pre : (fu ? vu : op(pre, vu));
            s_vpre[lane] = ex;
            if (lane == kWave - 1) s_gfold = gf ? gv : op(pre, gv);
        }
    }
    __syncthreads();

    // move the staged runs: wave w takes tiles w, w + 4, ... (16 of them),
    // lanes the entries of their dense slots (2 per lane); all of them are
    // loaded before any is stored, so the wave waits for memory once, not
    // once per tile
    constexpr uint32_t kPerWave = kRbkGroup / kBkWaves;
    constexpr uint32_t kSlotLoads = kRbkSlot / kWave;
    K mk[kPerWave][kSlotLoads];
    V mv[kPerWave][kSlotLoads];
#pragma unroll
    for (uint32_t u = 0; u < kPerWave; ++u) {
        const uint32_t l = wave + u * kBkWaves;
#pragma unroll
        for (uint32_t h = 0; h < kSlotLoads; ++h) {
            const uint32_t i = lane + h * kWave;
            if (l < ng && i < s_cnt[l]) {
                const uint64_t src = (uint64_t)(t0 + l) * kRbkSlot + i;
                mk[u][h] = pkeys[src];
                mv[u][h] = pvals[src];
            }
        }
    }
    auto emit = [&](uint32_t l, uint32_t i, K key, V v) {
        const uint32_t idx = s_base[l] + i;  // the i-th head of tile t0 + l closes run idx - 1
        if (i == 0) v = op(s_vpre[l], v);
        // idx <= n by construction; the bound keeps a broken invariant (a
        // look-back wait past its spin limit) from writing outside
        if (idx > 0 && idx <= n) {
            unique_out[idx - 1] = key;
            agg_out[idx - 1] = v;
        }
    };
#pragma unroll
    for (uint32_t u = 0; u < kPerWave; ++u) {
        const uint32_t l = wave + u * kBkWaves;
#pragma unroll
        for (uint32_t h = 0; h < kSlotLoads; ++h) {
            const uint32_t i = lane + h * kWave;
            if (l < ng && i < s_cnt[l]) emit(l, i, mk[u][h], mv[u][h]);
        }
    }
    // tiles with more than kRbkSlot runs: the rest from their overflow entries
    for (uint32_t l = wave; l < ng; l += kBkWaves) {
        const uint32_t cnt = s_cnt[l];
        const uint64_t src = (uint64_t)(t0 + l) * TILE;
        for (uint32_t i = kRbkSlot + lane; i < cnt; i += kWave) emit(l, i, skeys[src + i], svals[src + i]);
    }
    // the last run (open at element n - 1) and the run count
    if (g == gridDim.x - 1 && tid == 0) {
        const uint32_t runs = s_gcount;
        if (runs >= 1 && runs <= n) {
            unique_out[runs - 1] = keys[n - 1];
            agg_out[runs - 1] = s_gfold;
        }
        *num_runs = runs;
    }
}

template <class K, class V, class Op>
int rbk_launch(void *temp, size_t tb, const void *keys_, const void *in_, void *uk_, void *agg_,
               uint32_t *num_runs, uint64_t n, hipStream_t s)
{
    if (!num_runs) return LCPP_ERR_INVALID_ARG;
    if (n == 0) {
        LCPP_LAUNCH("reduce_by_key_empty", s, rbk_zero_runs<<<1, 1, 0, s>>>(num_runs));
        LCPP_CHECK_LAUNCH();
        return LCPP_OK;
    }
    const K *keys = static_cast<const K *>(keys_);
    const V *in = static_cast<const V *>(in_);
    K *uk = static_cast<K *>(uk_);
    V *agg = static_cast<V *>(agg_);
    if (!keys || !in || !uk || !agg) return LCPP_ERR_INVALID_ARG;
    if (n > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;
    const RbkLayout<K, V> L = rbk_layout<K, V>(n);
    if (tb < L.total) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    char *t = static_cast<char *>(temp);
    uint32_t *tile_count = reinterpret_cast<uint32_t *>(t + L.count_off);
    V *tile_fold = reinterpret_cast<V *>(t + L.fold_off);
    uint64_t *cwords = reinterpret_cast<uint64_t *>(t + L.cwords_off);
    uint64_t *vwords = reinterpret_cast<uint64_t *>(t + L.vwords_off);
    K *pkeys = reinterpret_cast<K *>(t + L.pkeys_off);
    V *pvals = reinterpret_cast<V *>(t + L.pvals_off);
    K *skeys = reinterpret_cast<K *>(t + L.skeys_off);
    V *svals = reinterpret_cast<V *>(t + L.svals_off);
    const WaitCtl ctl = wait_ctl(reinterpret_cast<uint32_t *>(t));
    const int vec_ok = ((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(in)) & 15) == 0;
    LCPP_LAUNCH("reduce_by_key_tile", s,
                (rbk_tile_kernel<K, V, Op><<<(uint32_t)L.tiles, kBkBlock, 0, s>>>(
                    keys, in, (uint32_t)n, tile_count, tile_fold, pkeys, pvals, skeys, svals, vec_ok,
                    reinterpret_cast<uint64_t *>(t), (uint32_t)(L.count_off / 8))));
    LCPP_CHECK_LAUNCH();
    LCPP_LAUNCH("reduce_by_key_emit", s,
                (rbk_emit_kernel<K, V, Op><<<(uint32_t)L.groups, kBkBlock, 0, s>>>(
                    keys, (uint32_t)n, (uint32_t)L.tiles, tile_count, tile_fold, pkeys, pvals, skeys, svals, uk, agg,
                    num_runs,
                    cwords, vwords, ctl)));
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

template <class V, class Op>
int rbk_keys(lcpp_dtype kt, void *temp, size_t tb, const void *k, const void *in, void *uk, void *agg,
             uint32_t *runs, uint64_t n, hipStream_t s)
{
    switch (kt) {
    case LCPP_INT32: case LCPP_UINT32: return rbk_launch<uint32_t, V, Op>(temp, tb, k, in, uk, agg, runs, n, s);
    case LCPP_INT64: case LCPP_UINT64: return rbk_launch<uint64_t, V, Op>(temp, tb, k, in, uk, agg, runs, n, s);
    case LCPP_FLOAT32: return rbk_launch<float, V, Op>(temp, tb, k, in, uk, agg, runs, n, s);
    case LCPP_FLOAT64: return rbk_launch<double, V, Op>(temp, tb, k, in, uk, agg, runs, n, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

template <class V>
int rbk_op(lcpp_dtype kt, lcpp_reduce_op op, void *temp, size_t tb, const void *k, const void *in, void *uk,
           void *agg, uint32_t *runs, uint64_t n, hipStream_t s)
{
    switch (op) {
    case LCPP_OP_SUM: return rbk_keys<V, SumOp>(kt, temp, tb, k, in, uk, agg, runs, n, s);
    case LCPP_OP_MIN: return rbk_keys<V, MinOp>(kt, temp, tb, k, in, uk, agg, runs, n, s);
    case LCPP_OP_MAX: return rbk_keys<V, MaxOp>(kt, temp, tb, k, in, uk, agg, runs, n, s);
    default: return LCPP_ERR_INVALID_ARG;
    }
}

bool rbk_valid_dtype(lcpp_dtype t) { return t >= LCPP_INT32 && t <= LCPP_FLOAT64; }
bool rbk_wide(lcpp_dtype t) { return t == LCPP_INT64 || t == LCPP_UINT64 || t == LCPP_FLOAT64; }

}  // namespace
}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_reduce_by_key_temp_bytes(lcpp_dtype k, lcpp_dtype v, uint64_t n, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    if (!rbk_valid_dtype(k) || !rbk_valid_dtype(v)) return LCPP_ERR_UNSUPPORTED_DTYPE;
    if (n > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;  // 32-bit run counts, as the call
    const bool wk = rbk_wide(k), wv = rbk_wide(v);
    *bytes = wk ? (wv ? rbk_layout<uint64_t, uint64_t>(n).total : rbk_layout<uint64_t, uint32_t>(n).total)
                : (wv ? rbk_layout<uint32_t, uint64_t>(n).total : rbk_layout<uint32_t, uint32_t>(n).total);
    return LCPP_OK;
}

extern "C" int lcpp_reduce_by_key(lcpp_dtype k, lcpp_dtype v, lcpp_reduce_op op, void *temp, size_t temp_bytes,
                                  const void *keys_in, const void *vals_in, void *unique_out, void *aggregates_out,
                                  uint32_t *num_runs_out, uint64_t n, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (v) {
    case LCPP_INT32: return rbk_op<int32_t>(k, op, temp, temp_bytes, keys_in, vals_in, unique_out, aggregates_out, num_runs_out, n, s);
    case LCPP_UINT32: return rbk_op<uint32_t>(k, op, temp, temp_bytes, keys_in, vals_in, unique_out, aggregates_out, num_runs_out, n, s);
    case LCPP_FLOAT32: return rbk_op<float>(k, op, temp, temp_bytes, keys_in, vals_in, unique_out, aggregates_out, num_runs_out, n, s);
    case LCPP_INT64: return rbk_op<int64_t>(k, op, temp, temp_bytes, keys_in, vals_in, unique_out, aggregates_out, num_runs_out, n, s);
    case LCPP_UINT64: return rbk_op<uint64_t>(k, op, temp, temp_bytes, keys_in, vals_in, unique_out, aggregates_out, num_runs_out, n, s);
    case LCPP_FLOAT64: return rbk_op<double>(k, op, temp, temp_bytes, keys_in, vals_in, unique_out, aggregates_out, num_runs_out, n, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}
