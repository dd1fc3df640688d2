// reduce_by_key.hip — DeviceReduce::ReduceByKey for gfx950.
//
// Reference: device/device_reduce.h:110-125 (temp bytes), 277-318 (entry
// point), 462-516 (dispatch), device/details/reduce_by_key.h:61-258.
//
// Semantics: run r = the r-th maximal run of equal consecutive keys (keys
// compared in their own type); unique_out[r] = its key, aggregates_out[r] =
// the op-fold of its values, *num_runs_out = the number of runs.
//
// Design (tile machinery in by_key.hpp): the pass over the data waits only
// in tiles with many runs.
//  * rbk_tile: one 256-thread workgroup per tile of 8192 4-byte values
//    (4096 8-byte).  It finds the tile's segment heads and folds its runs with
//    tile-local prefixes (reduce-then-rescan, by_key.hpp; the prefixes of the
//    32 (vector, wave) slices are scanned once per tile by wave 0), writes the
//    tile's summary (its head count, whether it has a head, the fold since its
//    last head or of the whole tile) and publishes the same as decoupled
//    look-back words (the count as PARTIAL; the fold as INCLUSIVE when the
//    tile has a head, else PARTIAL).
//    - A tile with at most 128 heads does not wait: entry i = the run closed
//      by its i-th head (that run's key and its fold over this tile's
//      elements; entry 0 lacks the part of its run in earlier tiles) is
//      gathered in LDS and stored contiguously into the tile's slot of a
//      dense staging area.  Runs of mean 128 give 64 per tile.
//    - A tile with more heads waits for the run count before it and the
//      fold entering it (to the nearest tile with a head) and writes its runs
//      to the outputs directly.  The run count is two-level: every tile adds
//      its head count to its batch word (8 tiles) as it publishes, so a
//      waiting tile sums its batch-mates' counts and walks the batch words
//      back (whole batches add their totals) to batch 0 or to a batch whose
//      last tile, having waited itself, published the inclusive count.  No
//      tile waits for another tile's wait.
//    The reference's single pass (reduce_by_key.h:90-258) waits on both
//    look-backs in every tile.  On this part those waits cost ~130 of ~500
//    us at 2^28 (int32 keys, f32 values, runs of mean 128): a tile here
//    carries only 64 KiB against the scan's 160 KiB, so a wait of a few
//    microseconds is a large share of its life.
//  * rbk_emit: one workgroup per 64 tiles.  Wave 0 scans their head counts;
//    the group's prefix is the sum of the counts every earlier group
//    publishes at its start (read 512 groups per round trip, no chain of
//    inclusive prefixes).  Wave 1 scans their segmented folds and takes the
//    fold entering the group from a decoupled look-back over groups (it stops
//    at the nearest group with a head).  Staged runs move to their final
//    positions, entry 0 of each tile completed with the fold entering the
//    tile.  The last group writes the last run and the run count (the
//    reference writes them from its last tile, reduce_by_key.h:231-254).
// Bytes: keys + values read once, plus (sizeof K + sizeof V) per run written
// (runs of tiles with at most 128 heads twice, and read once).  Temp: O(n /
// 64) for the dense slots, plus per-tile summaries and look-back words.
#include "by_key.hpp"

namespace lcpp {
namespace {

constexpr uint32_t kRbkGroup = 64;  // tiles per rbk_emit workgroup (one wave's lanes)
constexpr uint32_t kRbkSlot = 128;  // runs a tile may stage (its dense slot)
constexpr uint32_t kRbkHeadBit = 0x80000000u;   // summary count word: the tile has a head
constexpr uint32_t kRbkDenseBit = 0x40000000u;  // summary count word: more than kRbkSlot heads
constexpr uint32_t kRbkCountMask = 0x3FFFFFFFu;
// Run-count batch words, 64-bit, one per kRbkBatch tiles: the low half is
// (tiles arrived << 20) + their head counts (at most 8 x 8192 = 2^16), plus
// kRbkGlobal once the batch's last tile has added the batch's inclusive run
// count to the high half.
constexpr uint32_t kRbkBatch = 8;
constexpr uint64_t kRbkArrive = 1ull << 20;
constexpr uint32_t kRbkGlobal = 0x80000000u;
// Each batch word has a 128-byte line to itself (stride in words): with 8
// words to a 64-byte line the atomic adds of 64 tiles queue on one line
// (2^28 int32 keys, runs of mean 8: 937 us per call against 558 us padded;
// runs of mean 128, where no tile waits: 367 against 353 us).
constexpr uint32_t kRbkBwStride = 16;

template <class K, class V>
struct RbkLayout {
    uint64_t tiles, groups, cwords_off, vwords_off, tcwords_off, tvwords_off, bwords_off, count_off, fold_off,
        pkeys_off, pvals_off, total;
};
template <class K, class V>
RbkLayout<K, V> rbk_layout(uint64_t n)
{
    RbkLayout<K, V> L{};
    L.tiles = bk_tiles<V>(n);
    L.groups = ceil_div(L.tiles, kRbkGroup);
    // [status header | group look-back words | tile look-back words | batch
    //  run-count words (all zeroed by one fill) | tile summaries | dense
    //  slots]
    L.cwords_off = kStatusBytes;
    L.vwords_off = L.cwords_off + align_up(L.groups * 8, 256);
    L.tcwords_off = L.vwords_off + align_up(L.groups * 8 * lb_words<V>(), 256);
    L.tvwords_off = L.tcwords_off + align_up(L.tiles * 8, 256);
    L.bwords_off = L.tvwords_off + align_up(L.tiles * 8 * lb_words<V>(), 256);
    L.count_off = L.bwords_off + align_up(ceil_div(L.tiles, (uint64_t)kRbkBatch) * kRbkBwStride * 8, 256);
    L.fold_off = L.count_off + align_up(L.tiles * 4, 256);
    L.pkeys_off = L.fold_off + align_up(L.tiles * sizeof(V), 256);
    L.pvals_off = L.pkeys_off + align_up(L.tiles * kRbkSlot * sizeof(K), 256);
    L.total = L.pvals_off + align_up(L.tiles * kRbkSlot * sizeof(V), 256);
    return L;
}

__global__ void rbk_zero_runs(uint32_t *num_runs) { *num_runs = 0; }

// The bits of `f` as a To of the same size (pass 2 stages values in the key
// array only when the sizes match; other instantiations never call it).
template <class To, class From>
__device__ __forceinline__ To same_size_bits(From f)
{
    if constexpr (sizeof(To) == sizeof(From)) return __builtin_bit_cast(To, f);
    else return To{};
}

// LDS of one tile.  Keys sit in LDS when they fit in 32 KiB: the registers
// that held them are free for pass 2 (150 -> ~100 VGPRs).
template <class K, class V>
struct RbkSmem {
    static constexpr bool kKeysInLds = bk_tile<V>() * sizeof(K) <= 32768;
    K keys[kKeysInLds ? bk_tile<V>() : 1];
    K last[kBkVecs][kBkWaves];
    K pred;
    V S[kBkVecs][kBkWaves];
    uint32_t C[kBkVecs][kBkWaves];
    uint32_t F[kBkVecs];
    K stk[kRbkSlot];
    V stv[kRbkSlot];
    V pw[kBkVecs * kBkWaves];
    uint32_t cw[kBkVecs * kBkWaves];
    uint32_t pf;  // bit l: a head before slice l
    uint32_t tc;
};

// Heads before `tile` (tile > 0, one wave): the counts of its batch-mates
// before it (tile words, published before any wait) plus the batch words
// before its batch, walked back in windows of 64 (the first round trip one
// window, later ones kRbkWalkWindows) until batch 0 or a word carrying
// kRbkGlobal (its inclusive count ends the walk); a batch word without it
// must be complete (all kRbkBatch tiles arrived).  A late word is re-polled
// (all late words of the round trip at once) up to the spin limit, then
// counted as it is and reported.  Every lane returns the count.
constexpr int kRbkWalkWindows = 8;
__device__ uint32_t rbk_count_before(const uint64_t *tcwords, const uint64_t *bwords, uint32_t tile,
                                     const WaitCtl &ctl)
{
    const uint32_t lane = lane_id();
    const uint32_t b = tile / kRbkBatch, mates = tile % kRbkBatch;
    const bool im = lane < mates;
    uint64_t wm = im ? ld_relaxed(&tcwords[b * kRbkBatch + lane]) : 0ull;
    uint32_t acc = 0;
    int64_t top = (int64_t)b - 1;  // nearest batch not yet summed
    uint32_t spins = 0;
    for (bool first = true;; first = false) {
        const int nw = first ? 1 : kRbkWalkWindows;
        uint64_t w[kRbkWalkWindows];
#pragma unroll
        for (int k = 0; k < kRbkWalkWindows; ++k) {
            const int64_t j = top - (int64_t)k * kWave - (int64_t)lane;
            w[k] = k < nw && j >= 0 ? ld_relaxed(&bwords[j * kRbkBwStride]) : 0ull;
        }
        int k0 = kRbkWalkWindows;  // the nearest GLOBAL word (or batch 0's end): window k0, lane l0
        uint32_t l0 = kWave;
        bool late = false;
        uint32_t v = 0;
        for (;; ++spins) {
            k0 = kRbkWalkWindows;
            l0 = kWave;
#pragma unroll
            for (int k = kRbkWalkWindows - 1; k >= 0; --k) {
                const int64_t j = top - (int64_t)k * kWave - (int64_t)lane;
                const bool stop = k < nw && (j < 0 || ((uint32_t)w[k] & kRbkGlobal) != 0);
                const uint64_t m = ballot(stop);
                if (m) {
                    k0 = k;
                    l0 = (uint32_t)__builtin_ctzll(m);
                }
            }
            late = first && im && (uint32_t)wm == kStInvalid;
            v = 0;
#pragma unroll
            for (int k = 0; k < kRbkWalkWindows; ++k) {
                const int64_t j = top - (int64_t)k * kWave - (int64_t)lane;
                const bool in_range = k < nw && j >= 0 && (k < k0 || (k == k0 && lane <= l0));
                if (!in_range) continue;
                const uint32_t lo = (uint32_t)w[k];
                if (lo & kRbkGlobal) v += (uint32_t)(w[k] >> 32);  // the stop word
                else if ((lo >> 20) == kRbkBatch) v += lo & (uint32_t)(kRbkArrive - 1);
                else late = true;
            }
            if (ballot(late) == 0) break;
            if (spins + 1 >= ctl.spin_limit) {
                if (lane == 0) report_timeout(ctl);  // count what has been published
                break;
            }
            __builtin_amdgcn_s_sleep(2);
            if (first && im && (uint32_t)wm == kStInvalid) wm = ld_relaxed(&tcwords[b * kRbkBatch + lane]);
#pragma unroll
            for (int k = 0; k < kRbkWalkWindows; ++k) {
                const int64_t j = top - (int64_t)k * kWave - (int64_t)lane;
                if (k < nw && j >= 0 && ((uint32_t)w[k] & kRbkGlobal) == 0 &&
                    ((uint32_t)w[k] >> 20) != kRbkBatch)
                    w[k] = ld_relaxed(&bwords[j * kRbkBwStride]);
            }
        }
        if (first) v += im ? (uint32_t)(wm >> 32) : 0u;
        acc += wave_allreduce(v, SumOp());
        if (k0 < kRbkWalkWindows || top - (int64_t)nw * kWave < 0) break;
        top -= (int64_t)nw * kWave;
    }
    return acc;
}

template <class K, class V, class Op>
__global__ __launch_bounds__(kBkBlock) void rbk_tile_kernel(const K *__restrict__ keys, const V *__restrict__ vin,
                                                            uint32_t n, uint32_t *__restrict__ tile_count,
                                                            V *__restrict__ tile_fold, K *__restrict__ pkeys,
                                                            V *__restrict__ pvals, K *__restrict__ unique_out,
                                                            V *__restrict__ agg_out, uint64_t *tcwords,
                                                            uint64_t *tvwords, uint64_t *bwords, int vec_ok,
                                                            WaitCtl ctl)
{
    constexpr int VP = bk_vp<V>();
    constexpr uint32_t TILE = bk_tile<V>();
    constexpr bool kKeysInLds = RbkSmem<K, V>::kKeysInLds;
    __shared__ RbkSmem<K, V> sm;
    __shared__ uint32_t s_cpre;
    __shared__ V s_vpre;
    Op op;
    const V ident = op_identity<Op, V>();
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint32_t base = tile * TILE;
    const uint32_t valid = n - base < TILE ? n - base : TILE;
    const bool fast = valid == TILE && vec_ok;

    BkRegs<K, V> r;
    bk_load<true>(r, keys, vin, base, valid, fast, tid);
    if (tid < kBkVecs) sm.F[tid] = 0;
    K prev0[kBkVecs];
    uint32_t fl = bk_heads<K, VP>(r.key, prev0, sm.last, sm.pred, keys, base, tile, tid);
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
            for (int j = 0; j < VP; ++j) sm.keys[bk_elem<V>(k, tid, j)] = r.key[k][j];
    }

    // head counts: per vector a wave scan, wave totals to LDS
    uint32_t exC[kBkVecs];
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        const uint32_t c = (uint32_t)__builtin_popcount((fl >> (k * VP)) & ((1u << VP) - 1u));
        const uint32_t ci = wave_inclusive_scan(c, SumOp());
        exC[k] = ci - c;
        if (lane == kWave - 1) sm.C[k][wave] = ci;
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
            sm.S[k][wave] = s;
            if (f) atomicOr(&sm.F[k], 1u << wave);
        }
    }
    __syncthreads();

    // wave 0: the exclusive prefixes of the (vector, wave) slices in tile
    // order (lane k * 4 + w: its fold since the tile's last earlier head, a
    // head before it, its head count), once per tile instead of a serial loop
    // in every thread; their inclusive totals are the tile's summary, also
    // published as look-back words
    static_assert(kBkVecs * kBkWaves <= 32, "one lane and one pf bit per slice");
    constexpr uint32_t kSlices = kBkVecs * kBkWaves;
    if (wave == 0) {
        const bool in = lane < kSlices;
        const uint32_t k_ = in ? lane / kBkWaves : 0, w_ = in ? lane % kBkWaves : 0;
        bool f = in && ((sm.F[k_] >> w_) & 1u) != 0;
        V v = in ? sm.S[k_][w_] : ident;
        const uint32_t c = in ? sm.C[k_][w_] : 0u;
        wave_seg_scan(f, v, op);
        const uint32_t ci = wave_inclusive_scan(c, SumOp());
        const V vu = shfl_up(v, 1);
        const uint64_t heads_incl = ballot(f);
        if (in) {
            sm.pw[lane] = lane == 0 ? ident : vu;
            sm.cw[lane] = ci - c;
        }
        const uint32_t tc = read_lane(ci, kSlices - 1);
        const V ts = read_lane(v, kSlices - 1);
        const bool tf = ((heads_incl >> (kSlices - 1)) & 1u) != 0;
        if (lane == 0) {
            sm.pf = (uint32_t)(heads_incl << 1);  // a head in slices < l
            sm.tc = tc;
            tile_count[tile] = tc | (tf ? kRbkHeadBit : 0u) | (tc > kRbkSlot ? kRbkDenseBit : 0u);
            tile_fold[tile] = ts;
            lb_publish(tcwords, tile, tc, kStPartial, ctl);
            lb_publish(tvwords, tile, ts, tile == 0 || tf ? kStInclusive : kStPartial, ctl);
            if (tile != ctl.withhold)  // a withheld tile publishes nothing (test hook)
                __hip_atomic_fetch_add(&bwords[(tile / kRbkBatch) * kRbkBwStride], kRbkArrive + tc,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __syncthreads();

    // more than kRbkSlot heads: wait for the run count before the tile (wave
    // 0) and the fold entering it (wave 1), then write the runs directly
    const bool direct = sm.tc > kRbkSlot;
    if (direct) {
        if (wave == 0) {
            const uint32_t p = tile > 0 ? rbk_count_before(tcwords, bwords, tile, ctl) : 0u;
            // the batch's last tile closes the batch's walk for later tiles
            if (lane == 0 && tile % kRbkBatch == kRbkBatch - 1 && tile != ctl.withhold)
                __hip_atomic_fetch_add(&bwords[(tile / kRbkBatch) * kRbkBwStride],
                                       ((uint64_t)(p + sm.tc) << 32) | kRbkGlobal, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            if (lane == 0) s_cpre = p;
        } else if (wave == 1) {
            const V p = tile > 0 ? lb_wait_prefix(tvwords, tile, op, ident, ctl) : ident;
            if (lane == 0) s_vpre = p;
        }
        __syncthreads();
    }
    const uint32_t cpre = direct ? s_cpre : 0u;
    const V vpre = direct ? s_vpre : ident;

    // pass 2: rescan from the slice prefixes; a head closes the run before it.
    // STAGE (a direct tile with more runs than a quarter of its elements,
    // keys in LDS, keys and values of one size): each (vector, wave) slice's
    // runs go out through that slice's own part of sm.keys once its keys are
    // read, so that consecutive lanes store consecutive runs.  A slice with
    // at most half as many runs as elements puts keys and values there side
    // by side and is stored after the last vector (one wait for all of
    // them); a denser one goes out at once, keys then values.  Other direct
    // tiles store each run where it closes (staging from an eighth on cost
    // 15 us at 2^28 with runs of mean 4).
    constexpr bool kStageDirect = kKeysInLds && sizeof(K) == sizeof(V);
    auto pass2 = [&](auto stage_tag) {
        constexpr bool STAGE = decltype(stage_tag)::value;
        constexpr uint32_t kSliceHalf = kWave * VP / 2;
        uint32_t deferred = 0;  // STAGE, bit k: slice (k, wave) waits in LDS for the final stores
        const uint32_t pf = sm.pf;
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k) {
            const uint32_t sl = k * kBkWaves + wave;
            const V pw0 = sm.pw[sl];
            const V pw = ((pf >> sl) & 1u) ? pw0 : op(vpre, pw0);
            V s = ((exF >> k) & 1u) ? exS[k] : op(pw, exS[k]);
            // staged: the tile's heads before this item (its entry index);
            // direct: all heads before it (it closes run c - 1)
            uint32_t c = cpre + sm.cw[sl] + exC[k];
            K ek[VP];  // STAGE: this thread's runs, in order
            V ev[VP];
#pragma unroll
            for (int j = 0; j < VP; ++j) {
                const uint32_t e = bk_elem<V>(k, tid, j);
                if ((fl >> (k * VP + j)) & 1u) {
                    K key;
                    if constexpr (STAGE) {
                        // a slice's key before it is the previous slice's
                        // last key (its part of sm.keys may be rewritten)
                        if (j == 0 && lane == 0)
                            key = wave > 0 ? sm.last[k][wave - 1] : k > 0 ? sm.last[k - 1][kBkWaves - 1] : sm.pred;
                        else
                            key = sm.keys[e - 1];
                        ek[j] = key;
                        ev[j] = s;
                    } else {
                        if constexpr (kKeysInLds) key = e > 0 ? sm.keys[e - 1] : sm.pred;
                        else key = j > 0 ? r.key[k][j - 1] : prev0[k];
                        if (direct) {
                            // c - 1 < n by construction; the bound keeps a
                            // broken invariant (a wait past its spin limit)
                            // from writing outside the outputs
                            if (c > 0 && c - 1 < n) {
                                unique_out[c - 1] = key;
                                agg_out[c - 1] = s;
                            }
                        } else {
                            sm.stk[c] = key;  // c < the tile's head count <= kRbkSlot
                            sm.stv[c] = s;
                        }
                        ++c;
                    }
                    s = r.val[k][j];
                } else {
                    s = op(s, r.val[k][j]);  // identity past n
                }
            }
            if constexpr (STAGE) {
                // the slice: elements [ss, ss + 64 VP), runs [cb, cb + nsl)
                // of the count (run i closes at output position cb + i - 1)
                const uint32_t ss = bk_elem<V>(k, wave * kWave, 0);
                const uint32_t cb = cpre + sm.cw[sl], nsl = sm.C[k][wave];
                wave_lds_sync();  // every lane has read its keys of the slice
                uint32_t li = exC[k];
                if (nsl <= kSliceHalf) {
#pragma unroll
                    for (int j = 0; j < VP; ++j)
                        if ((fl >> (k * VP + j)) & 1u) {
                            sm.keys[ss + li] = ek[j];
                            sm.keys[ss + kSliceHalf + li] = same_size_bits<K>(ev[j]);
                            ++li;
                        }
                    deferred |= 1u << k;
                    continue;
                }
#pragma unroll
                for (int j = 0; j < VP; ++j)
                    if ((fl >> (k * VP + j)) & 1u) sm.keys[ss + li++] = ek[j];
                wave_lds_sync();
#pragma unroll
                for (int q = 0; q < VP; ++q) {
                    const uint32_t i = q * kWave + lane;
                    // the bound keeps a broken invariant (a wait past its
                    // spin limit) from writing outside the outputs
                    if (i < nsl && cb + i > 0 && cb + i - 1 < n) unique_out[cb + i - 1] = sm.keys[ss + i];
                }
                wave_lds_sync();
                li = exC[k];
#pragma unroll
                for (int j = 0; j < VP; ++j)
                    if ((fl >> (k * VP + j)) & 1u) sm.keys[ss + li++] = same_size_bits<K>(ev[j]);
                wave_lds_sync();
#pragma unroll
                for (int q = 0; q < VP; ++q) {
                    const uint32_t i = q * kWave + lane;
                    if (i < nsl && cb + i > 0 && cb + i - 1 < n)
                        agg_out[cb + i - 1] = same_size_bits<V>(sm.keys[ss + i]);
                }
            }
        }
        if constexpr (STAGE) {
            if (deferred) {
                wave_lds_sync();
#pragma unroll
                for (int k = 0; k < kBkVecs; ++k) {
                    if (!((deferred >> k) & 1u)) continue;
                    const uint32_t ss = bk_elem<V>(k, wave * kWave, 0);
                    const uint32_t cb = cpre + sm.cw[k * kBkWaves + wave], nsl = sm.C[k][wave];
#pragma unroll
                    for (uint32_t q = 0; q < kSliceHalf / kWave; ++q) {
                        const uint32_t i = q * kWave + lane;
                        if (i < nsl && cb + i > 0 && cb + i - 1 < n) {
                            unique_out[cb + i - 1] = sm.keys[ss + i];
                            agg_out[cb + i - 1] = same_size_bits<V>(sm.keys[ss + kSliceHalf + i]);
                        }
                    }
                }
            }
        }
    };
    if constexpr (kStageDirect) {
        if (direct && sm.tc > TILE / 4) pass2(std::true_type{});
        else pass2(std::false_type{});
    } else {
        pass2(std::false_type{});
    }
    if (!direct) {
        __syncthreads();
        for (uint32_t i = tid; i < sm.tc; i += kBkBlock) {
            pkeys[(uint64_t)tile * kRbkSlot + i] = sm.stk[i];
            pvals[(uint64_t)tile * kRbkSlot + i] = sm.stv[i];
        }
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
                                                            K *__restrict__ unique_out, V *__restrict__ agg_out,
                                                            uint32_t *__restrict__ num_runs, uint64_t *cwords,
                                                            uint64_t *vwords, WaitCtl ctl)
{
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
    // the head counts, wave 1 the segmented folds
    if (wave < 2) {
        const bool in = lane < ng;
        const uint32_t cwd = in ? tile_count[t0 + lane] : 0u;
        const uint32_t cnt = cwd & kRbkCountMask;
        if (wave == 0) {
            const uint32_t ci = wave_inclusive_scan(cnt, SumOp());
            const uint32_t total = read_lane(ci, kWave - 1);
            if (lane == 0) lb_publish(cwords, g, total, kStPartial, ctl);
            const uint32_t pre = rbk_sum_before(cwords, g, ctl);
            // tiles with more than kRbkSlot heads wrote their runs themselves
            s_cnt[lane] = (cwd & kRbkDenseBit) ? 0u : cnt;  // staged entries to move
            s_base[lane] = pre + ci - cnt;
            if (lane == 0) s_gcount = pre + total;
        } else {
            bool f = in && (cwd & kRbkHeadBit) != 0;
            V v = in ? tile_fold[t0 + lane] : ident;
            wave_seg_scan(f, v, op);
            const bool gf = read_lane((int)f, kWave - 1) != 0;
            const V gv = read_lane(v, kWave - 1);
            // 64 groups polled per round trip: few workgroups compete here
            const V pre = lb_segmented_tile<kWave>(vwords, g, gv, gf, true, op, ident, ctl);
            // exclusive segmented fold entering tile t0 + lane
            const int fu = __shfl_up((int)f, 1);
            const V vu = shfl_up(v, 1);
            s_vpre[lane] = lane == 0 ? pre : (fu ? vu : op(pre, vu));
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
#pragma unroll
    for (uint32_t u = 0; u < kPerWave; ++u) {
        const uint32_t l = wave + u * kBkWaves;
#pragma unroll
        for (uint32_t h = 0; h < kSlotLoads; ++h) {
            const uint32_t i = lane + h * kWave;
            if (l < ng && i < s_cnt[l]) {
                const uint32_t idx = s_base[l] + i;  // the i-th head of tile t0 + l closes run idx - 1
                const V v = i == 0 ? op(s_vpre[l], mv[u][h]) : mv[u][h];
                // idx <= n by construction; the bound keeps a broken
                // invariant (a wait past its spin limit) from writing outside
                if (idx > 0 && idx <= n) {
                    unique_out[idx - 1] = mk[u][h];
                    agg_out[idx - 1] = v;
                }
            }
        }
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
    uint64_t *tcwords = reinterpret_cast<uint64_t *>(t + L.tcwords_off);
    uint64_t *tvwords = reinterpret_cast<uint64_t *>(t + L.tvwords_off);
    uint64_t *bwords = reinterpret_cast<uint64_t *>(t + L.bwords_off);
    K *pkeys = reinterpret_cast<K *>(t + L.pkeys_off);
    V *pvals = reinterpret_cast<V *>(t + L.pvals_off);
    // the status header, both sets of look-back words and the batch
    // run-count words are contiguous up to alignment padding: one fill
    if (lb_init(reinterpret_cast<uint64_t *>(t), L.count_off / 8, s, "reduce_by_key_init") != LCPP_OK)
        return LCPP_ERR_HIP;
    const WaitCtl ctl = wait_ctl(reinterpret_cast<uint32_t *>(t));
    const int vec_ok = ((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(in)) & 15) == 0;
    LCPP_LAUNCH("reduce_by_key_tile", s,
                (rbk_tile_kernel<K, V, Op><<<(uint32_t)L.tiles, kBkBlock, 0, s>>>(
                    keys, in, (uint32_t)n, tile_count, tile_fold, pkeys, pvals, uk, agg, tcwords, tvwords, bwords,
                    vec_ok, ctl)));
    LCPP_CHECK_LAUNCH();
    LCPP_LAUNCH("reduce_by_key_emit", s,
                (rbk_emit_kernel<K, V, Op><<<(uint32_t)L.groups, kBkBlock, 0, s>>>(
                    keys, (uint32_t)n, (uint32_t)L.tiles, tile_count, tile_fold, pkeys, pvals, uk, agg, num_runs,
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
