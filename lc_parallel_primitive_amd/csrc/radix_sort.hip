// radix_sort.hip — DeviceRadixSort::SortKeys/SortPairs(Descending) (onesweep)
// for gfx950.
//
// Reference: device/device_radix_sort.h:129-184, 187-378 (reset, histogram,
// bin exclusive sum, then per pass x portion: look-back memset + onesweep),
// agent/agent_radix_sort_histogram.h:45-198, agent/agent_radix_sort_onesweep.h
// :43-500, block/block_radix_rank.h:66-336, agent/radix_rank_sort_operations.h,
// common/util_type.h:98-175 (twiddles), common/utils.h:273-324 (MatchAny).
//
// MI355X design (HBM-bound integer/byte work, no MFMA).  Measured on the
// device: a cross-workgroup publish is observed ~0.5 us later (1.5-2 us under
// full HBM load), and 65536 same-address atomics take ~0.75 ms.  The
// reference's shape (1024-key tiles, a per-tile ticket, a per-digit walk over
// every earlier tile) therefore cannot keep up at 8 TB/s: at the tile rate
// the pass needs, each tile would walk ~100 predecessors per digit.  The pass
// here is built around that:
//
//  * launch 0 "rs_init": zero the status word, the P digit histograms and an
//    arrival counter.
//  * launch 1 "rs_histogram": one 1024-thread workgroup per CU streams a
//    contiguous chunk of keys and counts all P = sizeof(K) 8-bit digits at
//    once into an LDS table in which every lane of a wave counts into its
//    own column (16 lane copies of every counter for 8-byte keys), so that
//    equal digits in one wave (skewed or constant key bytes) never hit one
//    LDS address; flushed with one global atomic per non-zero bin.  It also
//    zeroes the look-back state of four passes.  The last workgroup to finish
//    (the arrival counter, release/acquire at agent scope) finds each pass's
//    hot digit and plans the passes from the finished histograms (below).
//  * launches 2..P+1 "rs_onesweep": one 16384-key tile (8192 for 8-byte keys
//    or values) per 512-thread workgroup.  No ticket: tiles are mapped from
//    the workgroup id so that every R consecutive tiles (R = 16 on a full
//    MI355X) run on one XCD (workgroups are dispatched round-robin over the 8
//    XCDs), which lets that XCD's L2 merge the adjacent digit runs those
//    tiles write (1, 8, 16, 32 tiles per run: 751, 606, 529, 544 us per pass
//    at 2^28).  A tile only ever waits on tiles dispatched at most 8R-1
//    workgroups after it, so R is chosen on the host such that 8R is at most
//    half of the workgroups the device holds at once (R = 1 is plain
//    dispatch order).
//  * Ranking: keys are loaded wave-striped (lane l of wave w, item u -> key
//    w*64*IPT + u*64 + l) so items in order u and lanes in order l are input
//    order; a key's rank in its (wave, digit) is one returning LDS atomic add
//    on the wave's counter for that digit.  gfx950 serves same-address LDS
//    atomics of one instruction in lane order, so the ranks are stable.  This
//    is a property of the hardware, not of the ISA documentation: the GPU
//    test suite checks it directly (a probe kernel over uniform, skewed and
//    constant digits) and checks stability on every sort it runs.  Ranks are
//    kept two per register (16 bits each).
//  * Two-level decoupled look-back.  Tiles form batches of 8.  Each tile
//    publishes its 256 digit counts once.  A tile's exclusive prefix = the
//    exclusive prefix of its batch + the counts of the earlier tiles of its
//    batch (at most 7 parallel reads per digit, by waves 4..7).  Tile counts
//    are 32-bit words {PARTIAL:1 | value}.  Batch words are 64-bit: every tile
//    of the batch adds its counts into the low half atomically, and the
//    batch's last tile, once it has walked the earlier batch words (waves
//    0..3, two of them per poll), adds GLOBAL (low half, bit 31) and the
//    batch's 32-bit inclusive prefix (high half) in one atomic, so n may use
//    all 32 bits.  Every wait is on an earlier tile, every re-poll reloads all
//    the words it still waits on, and a wait that exhausts its bounded spin
//    records the give-up in the call's status word.  Words are accessed with
//    agent-scope atomics (the 8 XCD L2s are not coherent).  Four look-back
//    regions, zeroed by the histogram launch, whose write bandwidth is
//    otherwise idle, serve four passes (no memset launch; only sorts with
//    more than four data-moving passes re-zero a region inside a pass); tile
//    counts are 16-bit words.
//  * The sorted tile leaves through LDS in two halves (32 KB of staging
//    instead of 64 KB), which lets keys-only passes run three workgroups per
//    CU: consecutive threads write consecutive positions of each digit run.
//    Values follow with the same ranks.
//  * The pass plan is made on the device: a pass whose digit is the same for
//    every key (from the histogram) is skipped, and the others ping-pong so
//    that the last one writes the output.
//  * Descending order sorts the bit-inverted sort keys (one XOR in, one out,
//    compiled only into the descending kernels), as RadixSortTwiddle<true>
//    does; equal keys keep their input order.
//  * Keys-only sorts reserve no value scratch (the reference reserves N
//    values it never uses, device_radix_sort.h:118-122).
#include <mutex>

#include "common.hpp"

namespace lcpp {
namespace {

constexpr int kRadixBits = 8;
constexpr int kRadix = 256;
constexpr int kOsBlock = 512;  // onesweep workgroup
constexpr int kOsWaves = kOsBlock / kWave;
constexpr int kBatch = 8;      // tiles per look-back batch
constexpr int kHistBlock = 1024;
constexpr uint32_t kLbGlobal = 0x80000000u;
// Tile count words are 16-bit: {published:1 | count:15} (a count is at most
// 16384); 0 = not published yet.
constexpr uint32_t kTcPublished = 0x8000u;
constexpr uint32_t kTcMask = 0x7FFFu;
constexpr uint64_t kMaxItems = 0xFFFFFFFFull;  // 32-bit positions and counts

enum KeyKind { kUnsigned = 0, kSigned = 1, kFloat = 2 };

// Twiddles of common/util_type.h:98-175 (BaseTraits::TwiddleIn/Out).
template <class UK, int KIND>
__device__ __forceinline__ UK tw_in(UK k)
{
    constexpr UK high = UK(1) << (sizeof(UK) * 8 - 1);
    if constexpr (KIND == kSigned) return k ^ high;
    else if constexpr (KIND == kFloat) return (k & high) ? UK(~k) : UK(k ^ high);
    else return k;
}
template <class UK, int KIND>
__device__ __forceinline__ UK tw_out(UK k)
{
    constexpr UK high = UK(1) << (sizeof(UK) * 8 - 1);
    if constexpr (KIND == kSigned) return k ^ high;
    else if constexpr (KIND == kFloat) return (k & high) ? UK(k ^ high) : UK(~k);
    else return k;
}
// Sort key of a raw key: twiddled, then bit-inverted for descending order
// (RadixSortTwiddle::In, agent/radix_rank_sort_operations.h:124-155).
template <class UK, int KIND, bool DESC>
__device__ __forceinline__ UK sort_key(UK raw)
{
    const UK t = tw_in<UK, KIND>(raw);
    return DESC ? UK(~t) : t;
}
template <class UK, int KIND, bool DESC>
__device__ __forceinline__ UK raw_key(UK sk)
{
    return tw_out<UK, KIND>(DESC ? UK(~sk) : sk);
}
// Digit of a sort key.  -0.0 and +0.0 are given the same digits
// (radix_rank_sort_operations.h:33-62, ProcessFloatMinusZero); their two sort
// keys are adjacent, so folding either onto the other yields the same stable
// order.
template <class UK, int KIND, bool DESC>
__device__ __forceinline__ uint32_t digit_of(UK tk, uint32_t shift)
{
    if constexpr (KIND == kFloat) {
        constexpr UK high = UK(1) << (sizeof(UK) * 8 - 1);
        constexpr UK flip = DESC ? UK(~UK(0)) : UK(0);
        constexpr UK minus_zero = UK(~high) ^ flip;  // sort key of -0.0
        if (tk == minus_zero) tk = high ^ flip;      // sort key of +0.0
    }
    return (uint32_t)(tk >> shift) & (kRadix - 1);
}

// Exclusive scan of the values x held by threads 0..255 (one digit each) of
// the workgroup; other threads pass 0 and get garbage.  Every thread of the
// workgroup must call it (it contains a barrier).
__device__ __forceinline__ uint32_t digit_excl_scan(uint32_t x, uint32_t *s_wsum)
{
    const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
    const uint32_t inc = wave_inclusive_scan(x, SumOp());
    if (lane == kWave - 1 && wave < kRadix / kWave) s_wsum[wave] = inc;
    __syncthreads();
    uint32_t pre = 0;
#pragma unroll
    for (int w = 0; w < kRadix / kWave; ++w)
        if ((uint32_t)w < wave) pre += s_wsum[w];
    return pre + inc - x;
}

// Look-back polls are bounded (WaitCtl::spin_limit re-polls; a wait that
// gives up records it in the status word and continues with what it has).
// Agent-scope polls compete with the data stream under full HBM load, so the
// re-poll interval is long: s_sleep 16 (~1000 cycles) between polls measured
// 2.17 ms per 2^28 u32 sort against 2.21 ms with s_sleep 1 (s_sleep 64:
// 2.26 ms); passes that move values prefer s_sleep 4.
//
// Agent-scope (sc1) loads through a buffer resource: one VGPR offset per
// load, constant strides folded into the immediate offset (the look-back
// runs while every key of the tile is held in registers).
__device__ __forceinline__ uint32_t ld_agent16(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, kPolicySc1);
}
__device__ __forceinline__ uint64_t ld_agent64(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kPolicySc1);
    return ((uint64_t)v[1] << 32) | v[0];
}

// Batch look-back words, 64-bit.  The low half is (tiles arrived << 24) +
// their summed digit counts: every tile of the batch adds its counts with a
// relaxed agent-scope atomic as it publishes them, so the batch aggregate is
// complete one publish latency after the batch's last count, with no
// read-and-republish round trip by one of its tiles.  The batch's last tile
// adds, in one atomic, GLOBAL into bit 31 of the low half and the batch's
// inclusive prefix into the high half (a full 32-bit count).  Measured at
// 2^28 u32 keys against 32-bit {GLOBAL | PARTIAL | value} words stored by
// the batch's last tile: 2.13 -> 2.05 ms per sort (AND-of-3 keys 2.15 ->
// 2.03 ms); SortPairs u64 -> u32 at 2^27: 5.42 -> 5.19 ms.
constexpr uint64_t kBwArrive = 1ull << 24;
constexpr uint32_t kBwSumMask = (1u << 24) - 1;
// 0 = not complete yet (v = 0: the word may hold the counts of some of its
// tiles), 1 = batch aggregate in v, 2 = inclusive prefix in v
__device__ __forceinline__ int batch_word_state(uint64_t w, uint32_t &v)
{
    const uint32_t hi = (uint32_t)(w >> 32), lo = (uint32_t)w;
    const int st = (lo & kLbGlobal) ? 2 : ((lo >> 24) & 0x7Fu) == (uint32_t)kBatch ? 1 : 0;
    v = st == 2 ? hi : st == 1 ? lo & kBwSumMask : 0u;
    return st;
}

// ------------------------------------------------------------------ init
__global__ __launch_bounds__(256) void rs_init_kernel(uint32_t *words, uint32_t count)
{
    for (uint32_t i = threadIdx.x; i < count; i += 256) words[i] = 0;
}

// ------------------------------------------------------------------ hot digits, pass plan
// hot[p] = the most frequent digit of pass p (the smallest on ties) when it
// holds at least 1/16 of the keys, else kRadix (none).
//
// plan[p]: a pass whose digit is the same for every key is the identity
// permutation (the sort is stable), so it is skipped: its launch returns at
// once.  The other passes ping-pong between the scratch and the output so
// that the last of them writes the output (the input is never written).
// The k-th of them uses look-back region k % 4; the histogram zeroed all four,
// and when more than four passes move data, pass k >= 1 zeroes region
// (k - 1) % 4 again for pass k + 3.  When every pass is skipped, the last
// launch copies the input to the output.  SortPairs of
// u64 keys with 16 random low bits (6 of 8 passes skipped): 5.21 -> ~1.5 ms.
// One workgroup; one wave per pass at a time.
constexpr uint32_t kPlanSkip = 1u, kPlanCopy = 2u;
constexpr int kPlanSrcShift = 2, kPlanDstShift = 4, kPlanRegionShift = 6;
constexpr uint32_t kPlanClearPrev = 1u << 8;  // zero region (k - 1) % 4 for pass k + 3
constexpr int kLbRegions = 4;
enum PlanBuf : uint32_t { kBufIn = 0, kBufTmp = 1, kBufOut = 2 };
// Runs in the histogram's last workgroup (NT threads), after the acquire that
// pairs with every workgroup's release of its bin adds.
template <int NT>
__device__ void rs_make_plan(const uint32_t *bins, uint32_t passes, uint64_t n, uint32_t *__restrict__ hot,
                             uint32_t *__restrict__ plan, uint32_t *s_trivial)
{
    const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
    for (uint32_t p = wave; p < passes; p += NT / kWave) {
        // lane l looks at digits l, l + 64, l + 128, l + 192
        uint64_t best = 0;  // (count << 8) | (255 - digit): max picks the larger count, then the smaller digit
#pragma unroll
        for (int q = 0; q < kRadix / kWave; ++q) {
            const uint32_t d = lane + (uint32_t)q * kWave;
            const uint64_t c = ((uint64_t)ld_relaxed(&bins[p * kRadix + d]) << 8) | (255u - d);
            best = c > best ? c : best;
        }
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            const uint64_t o = shfl_xor(best, m);
            best = o > best ? o : best;
        }
        if (lane == 0) {
            hot[p] = (best >> 8) * 16 >= n ? 255u - (uint32_t)(best & 255u) : (uint32_t)kRadix;
            s_trivial[p] = (best >> 8) == n;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t m = 0;
        for (uint32_t p = 0; p < passes; ++p) m += s_trivial[p] ? 0u : 1u;
        uint32_t k = 0, cur = kBufIn;
        for (uint32_t p = 0; p < passes; ++p) {
            if (s_trivial[p]) {
                plan[p] = kPlanSkip | (p + 1 == passes && m == 0 ? kPlanCopy : 0u);
            } else {
                const uint32_t dst = (m - 1 - k) % 2 == 0 ? kBufOut : kBufTmp;  // the last one writes the output
                plan[p] = (cur << kPlanSrcShift) | (dst << kPlanDstShift) | ((k % kLbRegions) << kPlanRegionShift) |
                          (k >= 1 && k + kLbRegions - 1 < m ? kPlanClearPrev : 0u);
                cur = dst;
                ++k;
            }
        }
    }
}

// ------------------------------------------------------------------ histogram
// Counter layout in LDS, lane columns (128 KiB for either key size): a
// [P][128][COLS] table of 32-bit words, each holding the 16-bit counters of
// digits d and d + 128 (d < 128) of one pass; lane l of every wave counts in
// column l % COLS.
//  * 4-byte keys, COLS = 64: a wave's counting atomic touches 64 distinct
//    words in 64 distinct banks whatever the digits are (no bank conflicts,
//    no same-address lanes).
//  * 8-byte keys (8 passes), COLS = 32: lanes l and l + 32 share a column,
//    so at most two lanes of an atomic meet on one word.  Against 16 copies
//    of a [P][256] table (lane l counting in copy l % 16; four lanes on one
//    word whenever they share a digit, as every lane does on a constant key
//    byte): SortPairs C4 (six constant key bytes) 1.694 -> 1.677 ms,
//    full-range keys 5.816 -> 5.825 ms.
// A column counts at most 1/COLS of the keys a workgroup has seen since its
// last flush, so the table is flushed every kHistRoundSteps loop steps
// (4-byte keys: 4,177,920 keys < 64 x 65536; 8-byte: 2,088,960 < 32 x 65536).
template <class UK>
constexpr uint32_t hist_cols()
{
    return sizeof(UK) == 4 ? 64u : 32u;
}
// Dynamic LDS: the counter table, then 17 words of planning state for the
// last workgroup (the kernel has no static LDS).
template <class UK>
constexpr size_t hist_table_words()
{
    return sizeof(UK) * (kRadix / 2) * hist_cols<UK>();
}
template <class UK>
constexpr size_t hist_lds_bytes()
{
    return (hist_table_words<UK>() + 17) * 4;
}
constexpr uint64_t kHistRoundSteps = 255;  // loop steps between flushes of the lane-column table

template <class UK, int KIND, bool DESC>
__global__ __launch_bounds__(kHistBlock) void rs_histogram_kernel(
    const UK *__restrict__ keys, uint64_t n, uint64_t chunk, uint32_t *bins, u32x4 *__restrict__ clear,
    uint64_t clear_vecs, uint32_t *arrivals, uint32_t *__restrict__ hot, uint32_t *__restrict__ plan)
{
    constexpr int P = sizeof(UK);
    constexpr uint32_t CO = hist_cols<UK>();
    constexpr uint32_t W = (uint32_t)hist_table_words<UK>();
    extern __shared__ uint32_t s_hist[];  // the counter table, then s_last, s_trivial[16]
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    uint32_t *s_last = s_hist + W, *s_trivial = s_last + 1;
    for (uint32_t i = tid; i < W; i += kHistBlock) s_hist[i] = 0;
    __syncthreads();
    // The look-back state of four passes is zeroed here, one 16-byte store per
    // thread per loop step (this workgroup's share of it, front to back), so
    // the stores go out beside the key stream instead of before it (2^28 u32
    // keys: 48 MiB of state).  The arrival's release below covers them.
    const uint64_t cshare = ceil_div(clear_vecs, (uint64_t)gridDim.x);
    const uint64_t c0 = (uint64_t)blockIdx.x * cshare;
    const uint64_t c1 = c0 + cshare < clear_vecs ? c0 + cshare : clear_vecs;
    uint64_t cnext = c0 + tid;
    auto clear_step = [&]() {
        if (cnext < c1) __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u}, clear + cnext);
        cnext += kHistBlock;
    };

    const uint64_t b0 = (uint64_t)blockIdx.x * chunk;
    const uint64_t b1 = b0 + chunk < n ? b0 + chunk : n;
    auto count = [&](UK raw) {
        const UK tk = sort_key<UK, KIND, DESC>(raw);
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint32_t dg = digit_of<UK, KIND, DESC>(tk, p * kRadixBits);
            atomicAdd(&s_hist[((uint32_t)p * (kRadix / 2) + (dg & 127u)) * CO + lane % CO], dg & 128u ? 0x10000u : 1u);
        }
    };
    // one global add per non-zero bin (the sum of its counters); the table is
    // zeroed again when more keys follow
    auto flush = [&](bool more) {
        __syncthreads();
        for (uint32_t i = tid; i < (uint32_t)(P * kRadix); i += kHistBlock) {
            uint32_t c = 0;
            const uint32_t d = i % kRadix;
            const uint32_t *col = s_hist + (i / kRadix * (kRadix / 2) + (d & 127u)) * CO;
            const uint32_t sh = (d >> 7) * 16u;
            // threads of a wave start at different columns
#pragma unroll 8
            for (uint32_t k = 0; k < CO; ++k) c += (col[(k + d) % CO] >> sh) & 0xFFFFu;
            if (c) __hip_atomic_fetch_add(&bins[i], c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (more) {
            __syncthreads();
            for (uint32_t i = tid; i < W; i += kHistBlock) s_hist[i] = 0;
        }
    };
    constexpr uint64_t V = 16 / sizeof(UK);
    constexpr int kVecs = 4;
    constexpr uint64_t step = (uint64_t)kHistBlock * V * kVecs;
    const bool vec = (reinterpret_cast<uintptr_t>(keys) & 15) == 0;
    // rounds of whole steps (every round but the last is a multiple of the step)
    const uint64_t round_len = kHistRoundSteps * step;
    for (uint64_t r0 = b0; r0 < b1;) {
        const uint64_t r1 = b1 - r0 > round_len ? r0 + round_len : b1;
        uint64_t tail = r0;
        if (vec) {
            const uint64_t full_end = r0 + (r1 - r0) / step * step;
            for (uint64_t t = r0; t < full_end; t += step) {
                u32x4 v[kVecs];
#pragma unroll
                for (int i = 0; i < kVecs; ++i) v[i] = ld16_nt(keys + t + ((uint64_t)i * kHistBlock + tid) * V);
                clear_step();
#pragma unroll
                for (int i = 0; i < kVecs; ++i) {
                    UK e[V];
                    unpack16<UK>(v[i], e);
#pragma unroll
                    for (int j = 0; j < (int)V; ++j) count(e[j]);
                }
            }
            tail = full_end;
        }
        for (uint64_t i = tail + tid; i < r1; i += kHistBlock) count(keys[i]);
        r0 = r1;
        if (r0 < b1) flush(true);
    }
    while (cnext < c1) clear_step();  // what the loop steps did not cover
    flush(false);

    // The last workgroup to arrive plans the passes (hot digits, skipped
    // passes, buffer routing) from the finished bins: every workgroup's adds
    // (and clears) are released before its arrival, and the last one
    // acquires them all before it reads the bins.
    // (The workgroup barrier orders every thread's adds before thread 0's
    // release; one agent-scope fence per workgroup: fences in all 16 waves
    // measured 16 us slower per sort, relaxed ordering no faster.)
    __syncthreads();
    if (tid == 0)
        *s_last = __hip_atomic_fetch_add(arrivals, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (*s_last) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        rs_make_plan<kHistBlock>(bins, (uint32_t)P, n, hot, plan, s_trivial);
    }
}

// ------------------------------------------------------------------ onesweep pass
// LDS of one onesweep workgroup.  The sorted tile goes through LDS in two
// halves (sorted positions [0, TILE/2) then [TILE/2, TILE)), so a 16384-key
// tile needs 32 KB of staging and three workgroups fit a CU.
template <int IPT, class UK, class UV>
struct OnesweepSmem {
    static constexpr int HALF = kOsBlock * IPT / 2;
    union {
        UK keys[HALF];
        UV vals[HALF];
    };
    uint32_t cnt[kOsWaves][kRadix];  // per-wave digit counters, then wave bases in the sorted tile
    uint32_t goff[kRadix];           // output position of sorted tile position 0 of digit d
    uint32_t total[kRadix];          // digit counts of this tile
    uint32_t within[kRadix];         // digit counts of the earlier tiles of this batch
    uint32_t wsum[2][kRadix / kWave];
};

// Waves per SIMD the register allocation targets: 6 (three 512-thread
// workgroups per CU) for keys-only passes and 4-byte pairs, 4 (two) when an
// 8-byte key or value rides along, and for the match ranking (at 6 its
// 16384-key kernel spills 26 VGPRs: 3.19 against 2.93 ms per 2^28 sort).
template <class UK, class UV, bool PAIRS, bool MATCH = false>
constexpr int os_waves_per_eu()
{
    return MATCH || (PAIRS && (sizeof(UK) == 8 || sizeof(UV) == 8)) ? 4 : 6;
}

// Look-back state: kLbRegions regions, each of tcount[tiles][256] (16-bit
// tile digit counts, written once) and bword[batches][256] (batch aggregate
// and batch inclusive prefix, see batch_word_state); the plan names a pass's
// region.  Regions are zeroed before their pass starts (by the histogram, or
// by a pass that ran before it), so no pass waits on stale words.
struct LbState {
    uint16_t *tcount;     // region 0; region r starts at tcount + r * tc_stride
    uint64_t *bword;      // region 0; region r starts at bword + r * bw_stride
    uint64_t tc_stride, bw_stride;
};
// The three key (and value) buffers a pass may read or write, picked by the
// pass plan.
template <class UK, class UV>
struct RsBuffers {
    const UK *kin;
    UK *ktmp, *kout;
    const UV *vin;
    UV *vtmp, *vout;
};

// Workgroup -> tile with R = 2^log_run tiles per XCD run: in every full group
// of 8R workgroups, b = 8Rq + 8j + x (x = the XCD that b is dispatched to)
// processes tile 8Rq + Rx + j, so tiles 8Rq + Rx .. +R-1 run on XCD x.  A
// partial last group maps identically.
__device__ __forceinline__ uint32_t xcd_tile(uint32_t b, uint32_t grid, uint32_t log_run)
{
    const uint32_t log_group = log_run + 3;
    const uint32_t g = b >> log_group;
    if ((g + 1) << log_group > grid) return b;
    const uint32_t r = b & ((1u << log_group) - 1);
    return (g << log_group) + ((r & 7) << log_run) + (r >> 3);
}

// 16-bit halves of the packed rank registers
__device__ __forceinline__ uint32_t half16(uint32_t w, int hi) { return hi ? w >> 16 : w & 0xFFFFu; }
__device__ __forceinline__ uint32_t set_half16(uint32_t w, int hi, uint32_t v)
{
    return hi ? (w & 0xFFFFu) | (v << 16) : (w & 0xFFFF0000u) | v;
}

// MATCH: rank by ballot match (stable by construction) instead of relying on
// the lane order of same-address LDS atomics (rs_rank_path picks one).
template <int IPT, class UK, class UV, int KIND, bool PAIRS, bool DESC, bool MATCH>
__global__ __launch_bounds__(kOsBlock)
__attribute__((amdgpu_waves_per_eu(os_waves_per_eu<UK, UV, PAIRS, MATCH>(), os_waves_per_eu<UK, UV, PAIRS, MATCH>())))
void rs_onesweep_kernel(RsBuffers<UK, UV> buf, uint32_t n, uint32_t shift, const uint32_t *__restrict__ bins,
                        LbState regions, uint32_t log_run, const uint32_t *__restrict__ hot_digits,
                        const uint32_t *__restrict__ pass_plan, WaitCtl ctl)
{
    constexpr int TILE = kOsBlock * IPT;
    constexpr int HALF = TILE / 2;
    constexpr int WAVE_ITEMS = kWave * IPT;
    constexpr int kSleep = PAIRS ? 4 : 16;
    // batch words per look-back poll: 2 keeps the 16384-key kernel within
    // 80 VGPRs (a window of 4 spills 20 VGPRs: 2.59 ms per sort; 3: same as 2).
    // Pairs kernels at four waves per SIMD have registers to spare and read
    // 8: their walk spans ~8 batch words, and a wave walks until its slowest
    // digit ends (SortPairs u64 -> u32 at 2^27, all 8 passes: 5851 -> 5805
    // us; 6 of 8 passes skipped: 1686 -> 1676 us; a window of 4 gains half).
    constexpr int kWindow = PAIRS && os_waves_per_eu<UK, UV, PAIRS, MATCH>() == 4 ? 8 : 2;
    static_assert(TILE <= 65536, "tile ranks are packed in 16 bits");
    __shared__ OnesweepSmem<IPT, UK, UV> sm;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t tile = xcd_tile(blockIdx.x, gridDim.x, log_run);
    const uint32_t hot_digit = __builtin_amdgcn_readfirstlane(*hot_digits);
    const uint32_t plan = __builtin_amdgcn_readfirstlane(*pass_plan);
    const uint32_t base = tile * (uint32_t)TILE;
    const uint32_t valid = n - base < (uint32_t)TILE ? n - base : (uint32_t)TILE;
    if (plan & kPlanSkip) {
        if (plan & kPlanCopy) {  // every pass skipped: the output is the input
            for (uint32_t i = tid; i < valid; i += kOsBlock) {
                buf.kout[base + i] = buf.kin[base + i];
                if constexpr (PAIRS) buf.vout[base + i] = buf.vin[base + i];
            }
        }
        return;
    }
    const uint32_t src_sel = (plan >> kPlanSrcShift) & 3u, dst_sel = (plan >> kPlanDstShift) & 3u;
    const UK *__restrict__ kin = src_sel == kBufIn ? buf.kin : src_sel == kBufTmp ? buf.ktmp : buf.kout;
    UK *__restrict__ kout = dst_sel == kBufTmp ? buf.ktmp : buf.kout;
    const UV *__restrict__ vin = src_sel == kBufIn ? buf.vin : src_sel == kBufTmp ? buf.vtmp : buf.vout;
    UV *__restrict__ vout = dst_sel == kBufTmp ? buf.vtmp : buf.vout;
    const uint32_t region = (plan >> kPlanRegionShift) & (kLbRegions - 1);
    const struct {
        uint16_t *tcount;
        uint64_t *bword;
    } lb{regions.tcount + region * regions.tc_stride, regions.bword + region * regions.bw_stride};
    const bool publish = tile != ctl.withhold;  // test hook: a withheld tile never publishes

    for (uint32_t i = tid; i < (uint32_t)(kOsWaves * kRadix); i += kOsBlock) (&sm.cnt[0][0])[i] = 0;

    // The tile's loads are issued at raised wave priority, so a tile that
    // starts while the CU's other tiles rank or write gets its whole 64 KiB in
    // flight first (2.067 -> 2.058 ms per 2^28 u32 sort; SortPairs u64 -> u32
    // at 2^27: 1.72 -> 1.68 ms).
    __builtin_amdgcn_s_setprio(3);
    // ---- load (wave-striped), sort keys; pads are all-ones -> digit 255, last
    UK tk[IPT];
    UV v[PAIRS ? IPT : 1];
    const uint32_t wbase = base + wave * WAVE_ITEMS + lane;
    if (valid == (uint32_t)TILE) {
#pragma unroll
        for (int u = 0; u < IPT; ++u) tk[u] = sort_key<UK, KIND, DESC>(__builtin_nontemporal_load(kin + wbase + u * kWave));
        if constexpr (PAIRS) {
#pragma unroll
            for (int u = 0; u < IPT; ++u) v[u] = __builtin_nontemporal_load(vin + wbase + u * kWave);
        }
    } else {
#pragma unroll
        for (int u = 0; u < IPT; ++u) {
            const uint32_t idx = wbase + u * kWave;
            tk[u] = idx < n ? sort_key<UK, KIND, DESC>(kin[idx]) : UK(~UK(0));
            if constexpr (PAIRS) v[u] = idx < n ? vin[idx] : UV(0);
        }
    }
    __builtin_amdgcn_s_setprio(0);
    __syncthreads();  // counters zeroed

    // ---- stable rank within (wave, digit); two 16-bit ranks per register.
    // Atomic path: lane-ordered LDS atomics.  MATCH path: the lanes holding
    // one digit (match_any8) are ranked by position among them on a base that
    // their lowest lane fetches with one atomic add of their number, so no
    // two lanes of an instruction touch one counter
    // (block/block_radix_rank.h:254-280, ComputeRanksItem<WARP_MATCH_ANY>).
    // The wave's LDS instructions complete in program order either way.
    uint32_t rank2[IPT / 2];
    uint32_t *cnt = sm.cnt[wave];
    // Lanes holding the pass's hot digit (skewed inputs: up to a third of the
    // keys) are represented in the instruction by their lowest lane, which
    // adds their number; the others rank by position among them.  Every key
    // still takes one lane of one atomic instruction, in lane order.  (A
    // separate loop for passes without a hot digit measured no faster.)
    const uint32_t hot = hot_digit;
    auto rank_of = [&](uint32_t dd) -> uint32_t {
        if constexpr (MATCH) {
            const uint64_t peers = match_any8(dd);
            const uint32_t below = mask_rank(peers);
            uint32_t b = 0;
            if (below == 0) b = atomicAdd(&cnt[dd], (uint32_t)__builtin_popcountll(peers));
            return (uint32_t)__shfl((int)b, (int)__builtin_ctzll(peers)) + below;
        }
        const bool in_hot = dd == hot;
        const uint64_t m = ballot(in_hot);
        const uint32_t leader = m ? (uint32_t)__builtin_ctzll(m) : (uint32_t)kWave;
        uint32_t res = 0;
        if (!in_hot || lane == leader)
            res = atomicAdd(&cnt[dd], lane == leader ? (uint32_t)__builtin_popcountll(m) : 1u);
        if (!m) return res;
        const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)res, (int)leader);
        return in_hot ? b + mask_rank(m) : res;
    };
#pragma unroll
    for (int u = 0; u < IPT; u += 2) {
        const uint32_t r0 = rank_of(digit_of<UK, KIND, DESC>(tk[u], shift));
        const uint32_t r1 = rank_of(digit_of<UK, KIND, DESC>(tk[u + 1], shift));
        rank2[u / 2] = r0 | (r1 << 16);
        // (match path: one pair at a time keeps its ballot masks from spilling)
        if (MATCH || (u & 7) == 6) __builtin_amdgcn_sched_barrier(0);
    }
    // Opaque copies: the counter addresses are recomputed after the barrier
    // (two VALU ops) instead of being kept live (one register per key).
#pragma unroll
    for (int u = 0; u < IPT; ++u) asm volatile("" : "+v"(tk[u]));
#pragma unroll
    for (int u = 0; u < IPT / 2; ++u) asm volatile("" : "+v"(rank2[u]));
    __syncthreads();

    // ---- threads 0..255 own digit d: tile counts, publish, clear next slots
    const bool owner = tid < (uint32_t)kRadix;
    const uint32_t d = owner ? tid : 0u;
    const uint32_t batch = tile / kBatch;
    const uint32_t bpos = tile % kBatch;
    const bool batch_last = bpos == kBatch - 1;
    uint32_t total = 0;
    if (owner) {
#pragma unroll
        for (int w = 0; w < kOsWaves; ++w) {
            const uint32_t c = sm.cnt[w][d];
            sm.cnt[w][d] = total;  // wave prefix within the tile
            total += c;
        }
        if (d == kRadix - 1) total -= (uint32_t)TILE - valid;  // drop the pads
        if (publish) {
            st_relaxed(&lb.tcount[(size_t)tile * kRadix + d], (uint16_t)(total | kTcPublished));
            // batch 0's word only ever carries its inclusive prefix
            if (batch > 0)
                __hip_atomic_fetch_add(&lb.bword[(size_t)batch * kRadix + d], kBwArrive + total, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
        sm.total[d] = total;
        if (plan & kPlanClearPrev) {
            const uint32_t prev = (region + kLbRegions - 1) % kLbRegions;
            regions.tcount[prev * regions.tc_stride + (size_t)tile * kRadix + d] = 0;
            if (bpos == 0) regions.bword[prev * regions.bw_stride + (size_t)batch * kRadix + d] = 0;
        }
    }
    const uint32_t dexcl = digit_excl_scan(owner ? total : 0u, sm.wsum[0]);
    if (owner) {
#pragma unroll
        for (int w = 0; w < kOsWaves; ++w) sm.cnt[w][d] += dexcl;  // wave base in the sorted tile
    }
    uint32_t gbase = 0;
    if (batch == 0) gbase = digit_excl_scan(owner ? bins[d] : 0u, sm.wsum[1]);
    __syncthreads();

    // ---- tile ranks (repacked in place); first half of the sorted tile into
    // LDS.  (Reading the wave bases of 8 keys in one burst before their stores
    // measured slower: 2.13 against 2.07 ms per sort.)
#pragma unroll
    for (int u = 0; u < IPT; ++u) {
        const uint32_t dd = digit_of<UK, KIND, DESC>(tk[u], shift);
        const uint32_t r = half16(rank2[u / 2], u & 1) + sm.cnt[wave][dd];
        rank2[u / 2] = set_half16(rank2[u / 2], u & 1, r);
        if (r < (uint32_t)HALF) sm.keys[r] = tk[u];
        if ((u & 7) == 7) __builtin_amdgcn_sched_barrier(0);
    }

    // ---- two-level look-back.  Waves 4..7 read the counts of the earlier
    // tiles of the batch; waves 0..3 walk the earlier batch words.
    // Every re-poll (after s_sleep) reloads all the words still unpublished,
    // so a wait costs one round trip however many words it waits on.
    if (!owner && tid < 2u * kRadix) {
        const uint32_t d2 = tid - kRadix;
        const __amdgpu_buffer_rsrc_t rt = make_rsrc(lb.tcount + (size_t)(tile - bpos) * kRadix, kBatch * kRadix * 2);
        const uint32_t o2 = d2 * 2u;
        uint32_t w7[kBatch - 1];
#pragma unroll
        for (int k = 0; k < kBatch - 1; ++k) w7[k] = (uint32_t)k < bpos ? ld_agent16(rt, o2 + k * kRadix * 2) : 1u;
        for (uint32_t spins = 0;; ++spins) {
            bool all = true;
#pragma unroll
            for (int k = 0; k < kBatch - 1; ++k) all &= w7[k] != 0;
            if (all) break;
            if (spins >= ctl.spin_limit) {
                report_timeout(ctl);
                break;
            }
            __builtin_amdgcn_s_sleep(kSleep);
            asm volatile("" ::: "memory");  // the reloads below are new reads
#pragma unroll
            for (int k = 0; k < kBatch - 1; ++k)
                if (w7[k] == 0) w7[k] = ld_agent16(rt, o2 + k * kRadix * 2);
        }
        uint32_t within = 0;
#pragma unroll
        for (int k = 0; k < kBatch - 1; ++k)
            if ((uint32_t)k < bpos) within += w7[k] & kTcMask;
        sm.within[d2] = within;
    }
    uint32_t bexcl = gbase;
    if (owner && batch > 0) {
        // Each poll reads a window of batch words ending at batch j: their
        // aggregates add up until an inclusive prefix ends the walk; an
        // unpublished word is where the next poll (after s_sleep) starts.
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(lb.bword, batch * kRadix * 8u);
        uint32_t acc = 0;
        int32_t j = (int32_t)batch - 1;
        for (uint32_t spins = 0;; ++spins) {
            uint64_t w[kWindow];
            asm volatile("" ::: "memory");  // every poll is a new read
            if (j >= kWindow - 1) {
                const uint32_t o = ((uint32_t)(j - (kWindow - 1)) * kRadix + d) * 8u;
#pragma unroll
                for (int k = 0; k < kWindow; ++k) w[k] = ld_agent64(rb, o + (kWindow - 1 - k) * kRadix * 8u);
            } else {
#pragma unroll
                for (int k = 0; k < kWindow; ++k)
                    w[k] = j - k >= 0 ? ld_agent64(rb, ((uint32_t)(j - k) * kRadix + d) * 8u) : 0ull;
            }
            bool done = false, stall = false;
            int adv = 0;
#pragma unroll
            for (int k = 0; k < kWindow; ++k) {
                if (!done && !stall) {
                    uint32_t vv = 0;
                    const int st = j - k >= 0 ? batch_word_state(w[k], vv) : 2;
                    stall = st == 0;
                    done = st == 2;
                    acc += vv;
                    adv = stall ? adv : k + 1;
                }
            }
            if (done) break;
            j -= adv;
            if (stall) {
                if (spins >= ctl.spin_limit) {
                    report_timeout(ctl);
                    break;
                }
                __builtin_amdgcn_s_sleep(kSleep);
            }
        }
        bexcl = acc;
    }
    __syncthreads();
    if (owner) {
        const uint32_t within = sm.within[d];
        const uint32_t incl = bexcl + within + total;
        if (batch_last && publish)
            __hip_atomic_fetch_add(&lb.bword[(size_t)batch * kRadix + d], ((uint64_t)incl << 32) | kLbGlobal,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sm.goff[d] = bexcl + within - dexcl;
    }
    __syncthreads();

    // ---- write out, one half at a time: consecutive threads -> consecutive
    // positions of a digit run; values follow with the same ranks.  Sorted
    // positions >= valid (the pads of the last tile) land at p >= n.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if (h == 1) {
            __syncthreads();  // first half written out
#pragma unroll
            for (int u = 0; u < IPT; ++u) {
                const uint32_t r = half16(rank2[u / 2], u & 1);
                if (r >= (uint32_t)HALF) sm.keys[r - HALF] = tk[u];
                if ((u & 7) == 7) __builtin_amdgcn_sched_barrier(0);
            }
            __syncthreads();
        }
        uint32_t pos[PAIRS ? IPT / 2 : 1];
#pragma unroll
        for (int j = 0; j < IPT / 2; ++j) {
            const uint32_t li = j * kOsBlock + tid;
            const uint32_t i = h * HALF + li;
            const UK k = sm.keys[li];
            const uint32_t p = i + sm.goff[digit_of<UK, KIND, DESC>(k, shift)];
            if constexpr (PAIRS) pos[j] = p;
            if (p < n) kout[p] = raw_key<UK, KIND, DESC>(k);
            if ((j & 7) == 7) __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (PAIRS) {
            __syncthreads();  // keys of this half read out
#pragma unroll
            for (int u = 0; u < IPT; ++u) {
                const uint32_t r = half16(rank2[u / 2], u & 1);
                if (r - h * HALF < (uint32_t)HALF) sm.vals[r - h * HALF] = v[u];
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < IPT / 2; ++j) {
                const uint32_t li = j * kOsBlock + tid;
                if (pos[j] < n) vout[pos[j]] = sm.vals[li];
            }
        }
    }
}

// ------------------------------------------------------------------ host side
// Items per thread: 32 (16384-key tiles) for 4-byte keys alone, 16 (8192-key
// tiles) for 8-byte keys or when values ride along (a tile's keys, values,
// ranks and output positions then stay in registers without spilling).
constexpr int os_ipt(int key_bytes, int val_bytes) { return key_bytes == 8 || val_bytes ? 16 : 32; }

// Temp layout: status header | bins[P][256] | hot[P] | plan[P] | arrivals
// (zeroed together by rs_init) | tile counts x 4 regions | batch words x 4
// regions (all zeroed by the histogram launch) | key scratch | value scratch
// (pairs only).
struct RsLayout {
    uint64_t passes, tiles, batches, bins_off, hot_off, tc_off, tc_region, bw_off, bw_region, ktmp_off, vtmp_off,
        total;
};

RsLayout rs_layout(uint64_t n, int key_bytes, int val_bytes)
{
    RsLayout L{};
    L.passes = (uint64_t)key_bytes;  // 8-bit digits
    const uint64_t tile = (uint64_t)kOsBlock * os_ipt(key_bytes, val_bytes);
    L.tiles = n ? ceil_div(n, tile) : 0;
    L.batches = ceil_div(L.tiles, kBatch);
    L.bins_off = kStatusBytes;
    L.hot_off = L.bins_off + L.passes * kRadix * 4;  // hot digits, then the pass plan: one word each per pass
    L.tc_off = align_up(L.hot_off + (2 * L.passes + 1) * 4, 256);  // + the histogram's arrival counter
    L.tc_region = align_up(L.tiles * kRadix * 2, 256);  // 16-bit tile counts
    L.bw_off = L.tc_off + kLbRegions * L.tc_region;
    L.bw_region = align_up(L.batches * kRadix * 8, 256);  // 64-bit batch words
    L.ktmp_off = L.bw_off + kLbRegions * L.bw_region;
    L.vtmp_off = L.ktmp_off + align_up(n * key_bytes, 256);
    L.total = n ? L.vtmp_off + align_up(n * val_bytes, 256) : 0;
    return L;
}

// ------------------------------------------------------------------ rank path
// The atomic ranking path gives stable ranks only if the LDS serves the lanes
// of one returning atomic that hit one address in lane order.  That is how
// gfx950 behaves, but no ISA document promises it, so the first sort on each
// device runs a probe (~70 us, in bounds): 1024 waves x 32 instructions of
// same-address LDS atomics over uniform, hot, constant and two-value digits
// with varying addends, every result checked against the lane-order value.
// Any violation selects the match path, which is stable by construction.
constexpr int kRankAtomic = 1, kRankMatch = 2;
constexpr uint32_t kProbeBlocks = 256, kProbeRounds = 32;

// splitmix64's output function (Vigna): the probe's digits
__device__ __forceinline__ uint64_t probe_mix(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Four waves per workgroup, each on its own 256 counters; pattern = block & 3.
// *violations += lanes whose atomic result differs from the counter's value
// before the instruction plus the addends of the lower lanes with its digit.
// Every LDS index is below 256 per wave.
__global__ __launch_bounds__(256) void rs_lane_order_probe_kernel(uint32_t rounds, unsigned long long *violations)
{
    __shared__ uint32_t cnt[4][kRadix];
    __shared__ uint32_t before[4][kRadix];
    const uint32_t lane = lane_id(), w = threadIdx.x / kWave, pattern = blockIdx.x & 3u;
    for (uint32_t i = lane; i < (uint32_t)kRadix; i += kWave) cnt[w][i] = 0;
    __builtin_amdgcn_wave_barrier();
    const uint64_t wid = (uint64_t)blockIdx.x * 4 + w;
    uint32_t bad = 0;
    for (uint32_t r = 0; r < rounds; ++r) {
        const uint64_t h = probe_mix((wid * rounds + r) * kWave + lane);
        uint32_t d;
        if (pattern == 0) d = (uint32_t)h & 255u;
        else if (pattern == 1) d = (h >> 40) % 3 == 0 ? 0u : (uint32_t)h & 255u;
        else if (pattern == 2) d = (uint32_t)probe_mix(wid * rounds + r) & 255u;
        else d = (h >> 12) & 1u ? 17u : 200u;
        const uint32_t add = 1u + (uint32_t)((h >> 20) & 3u);
        for (uint32_t i = lane; i < (uint32_t)kRadix; i += kWave) before[w][i] = cnt[w][i];
        __builtin_amdgcn_wave_barrier();
        const uint32_t got = atomicAdd(&cnt[w][d], add);
        uint32_t lower = 0;
        for (int j = 0; j < kWave; ++j) {
            const uint32_t dj = (uint32_t)__builtin_amdgcn_readlane((int)d, j);
            const uint32_t aj = (uint32_t)__builtin_amdgcn_readlane((int)add, j);
            lower += ((uint32_t)j < lane && dj == d) ? aj : 0u;
        }
        bad += got != before[w][d] + lower ? 1u : 0u;
        __builtin_amdgcn_wave_barrier();
    }
    if (bad) atomicAdd(violations, (unsigned long long)bad);
}

}  // namespace
}  // namespace lcpp

// The probe's violation counter (one per GPU the library runs on).  Host code
// uses the address hipGetSymbolAddress returns, never the name.
static __device__ __align__(8) unsigned long long rs_probe_violations;

namespace lcpp {
namespace {

std::atomic<int> g_rank_force{0};  // lcpp_test_set_sort_rank_path
std::mutex g_probe_mu;
DeviceCache g_rank_cache;

// Runs the probe on a private stream and waits for it: kRankAtomic when no
// violation was seen, kRankMatch otherwise, -1 when a HIP call failed.
int rs_run_probe()
{
    void *addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(rs_probe_violations)) != hipSuccess || !addr) return -1;
    hipStream_t ps = nullptr;
    if (hipStreamCreateWithFlags(&ps, hipStreamNonBlocking) != hipSuccess) return -1;
    unsigned long long v = ~0ull;
    rs_init_kernel<<<1, 256, 0, ps>>>(static_cast<uint32_t *>(addr), 2);
    rs_lane_order_probe_kernel<<<kProbeBlocks, 256, 0, ps>>>(kProbeRounds, static_cast<unsigned long long *>(addr));
    const bool ok = hipGetLastError() == hipSuccess &&
                    hipMemcpyAsync(&v, addr, sizeof(v), hipMemcpyDeviceToHost, ps) == hipSuccess &&
                    hipStreamSynchronize(ps) == hipSuccess;
    (void)hipStreamDestroy(ps);
    if (!ok) return -1;
    return v == 0 ? kRankAtomic : kRankMatch;
}

// The ranking path of the sorts on the current device.  The probe runs once
// per device, on its first sort.  A first sort made while its stream is being
// captured into a graph cannot wait for a probe: it takes the match path
// (correct everywhere) and the probe runs on a later call.
int rs_rank_path(hipStream_t s)
{
    const int forced = g_rank_force.load(std::memory_order_relaxed);
    if (forced) return forced;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return kRankMatch;
    int x = g_rank_cache.v[dev].load(std::memory_order_relaxed);
    if (x) return x;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return kRankMatch;
    }
    std::lock_guard<std::mutex> lk(g_probe_mu);
    x = g_rank_cache.v[dev].load(std::memory_order_relaxed);
    if (x) return x;
    x = rs_run_probe();
    if (x < 0) {
        (void)hipGetLastError();  // the probe's own failure; this call takes the match path
        return kRankMatch;
    }
    g_rank_cache.v[dev].store(x, std::memory_order_relaxed);
    return x;
}

// XCD run length of one onesweep instantiation: 8R <= half the workgroups
// resident at once.  log2(R) + 1, or -1 when the occupancy query fails.
template <int IPT, class UK, class UV, int KIND, bool PAIRS, bool DESC, bool MATCH>
int rs_log_run()
{
    static DeviceCache run_cache;
    return device_cached(run_cache, [] {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, reinterpret_cast<const void *>(&rs_onesweep_kernel<IPT, UK, UV, KIND, PAIRS, DESC, MATCH>),
                kOsBlock, 0) != hipSuccess)
            return -1;
        const uint64_t resident = (uint64_t)(per_cu > 0 ? per_cu : 1) * (uint64_t)device_cus();
        int lr = 0;
        while (lr < 4 && (8ull << (lr + 1)) * 2 <= resident) ++lr;
        return lr + 1;
    });
}

// The P onesweep launches of one sort.
template <int IPT, class UK, class UV, int KIND, bool PAIRS, bool DESC, bool MATCH>
int rs_passes(const RsBuffers<UK, UV> &buf, uint64_t n, const RsLayout &L, char *t, const uint32_t *bins,
              const uint32_t *hot, const uint32_t *plan, const WaitCtl &ctl, hipStream_t s)
{
    const int lr1 = rs_log_run<IPT, UK, UV, KIND, PAIRS, DESC, MATCH>();
    if (lr1 < 0) return LCPP_ERR_HIP;
    const uint32_t log_run = (uint32_t)(lr1 - 1);
    for (int p = 0; p < (int)L.passes; ++p) {
        const LbState lb{reinterpret_cast<uint16_t *>(t + L.tc_off), reinterpret_cast<uint64_t *>(t + L.bw_off),
                         L.tc_region / 2, L.bw_region / 8};
        LCPP_LAUNCH("rs_onesweep", s,
                    (rs_onesweep_kernel<IPT, UK, UV, KIND, PAIRS, DESC, MATCH><<<(uint32_t)L.tiles, kOsBlock, 0, s>>>(
                        buf, (uint32_t)n, (uint32_t)(p * kRadixBits), bins + p * kRadix, lb, log_run, hot + p,
                        plan + p, ctl)));
        LCPP_CHECK_LAUNCH();
    }
    return LCPP_OK;
}

template <class UK, class UV, int KIND, bool PAIRS, bool DESC>
int rs_run(void *temp, size_t temp_bytes, const void *kin_, void *kout_, const void *vin_, void *vout_, uint64_t n,
           hipStream_t s)
{
    constexpr int IPT = os_ipt(sizeof(UK), PAIRS ? sizeof(UV) : 0);
    if (n == 0) return LCPP_OK;
    if (n > kMaxItems) return LCPP_ERR_INVALID_ARG;
    const UK *kin = static_cast<const UK *>(kin_);
    UK *kout = static_cast<UK *>(kout_);
    const UV *vin = static_cast<const UV *>(vin_);
    UV *vout = static_cast<UV *>(vout_);
    if (!kin || !kout || (PAIRS && (!vin || !vout))) return LCPP_ERR_INVALID_ARG;
    const RsLayout L = rs_layout(n, sizeof(UK), PAIRS ? sizeof(UV) : 0);
    if (temp_bytes < L.total) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    char *t = static_cast<char *>(temp);
    uint32_t *status = reinterpret_cast<uint32_t *>(t);
    uint32_t *bins = reinterpret_cast<uint32_t *>(t + L.bins_off);
    uint32_t *hot = reinterpret_cast<uint32_t *>(t + L.hot_off);
    uint32_t *plan = hot + L.passes;
    UK *ktmp = reinterpret_cast<UK *>(t + L.ktmp_off);
    UV *vtmp = reinterpret_cast<UV *>(t + L.vtmp_off);
    const int P = (int)L.passes;

    // status header, bins, hot digits, plan and the arrival counter are contiguous
    const uint32_t init_words = (uint32_t)((L.hot_off + (2 * L.passes + 1) * 4) / 4);
    LCPP_LAUNCH("rs_init", s, rs_init_kernel<<<1, 256, 0, s>>>(status, init_words));
    LCPP_CHECK_LAUNCH();
    {
        // one 1024-thread workgroup per CU (128 KB of LDS each)
        constexpr size_t lds = hist_lds_bytes<UK>();
        static DeviceCache lds_set;
        if (device_cached(lds_set, [] {
                return hipFuncSetAttribute(reinterpret_cast<const void *>(&rs_histogram_kernel<UK, KIND, DESC>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess
                           ? 1
                           : -1;
            }) < 0)
            return LCPP_ERR_HIP;
        const uint64_t htile = (uint64_t)kHistBlock * 4 * (16 / sizeof(UK));
        const uint64_t htiles = ceil_div(n, htile);
        const uint64_t cus = (uint64_t)device_cus();
        uint64_t grid = htiles < cus ? htiles : cus;
        const uint64_t chunk = ceil_div(htiles, grid) * htile;
        grid = ceil_div(n, chunk);
        LCPP_LAUNCH("rs_histogram", s,
                    rs_histogram_kernel<UK, KIND, DESC><<<(uint32_t)grid, kHistBlock, lds, s>>>(
                        kin, n, chunk, bins, reinterpret_cast<u32x4 *>(t + L.tc_off),
                        (L.ktmp_off - L.tc_off) / 16, plan + P, hot, plan));
        LCPP_CHECK_LAUNCH();
    }
    const int path = rs_rank_path(s);
    const WaitCtl ctl = wait_ctl(status);
    // buffers per pass come from the device-side plan
    const RsBuffers<UK, UV> buf{kin, ktmp, kout, vin, vtmp, vout};
    return path == kRankMatch ? rs_passes<IPT, UK, UV, KIND, PAIRS, DESC, true>(buf, n, L, t, bins, hot, plan, ctl, s)
                              : rs_passes<IPT, UK, UV, KIND, PAIRS, DESC, false>(buf, n, L, t, bins, hot, plan, ctl, s);
}

int key_kind(lcpp_dtype k)
{
    switch (k) {
    case LCPP_UINT32: case LCPP_UINT64: return kUnsigned;
    case LCPP_INT32: case LCPP_INT64: return kSigned;
    case LCPP_FLOAT32: case LCPP_FLOAT64: return kFloat;
    default: return -1;
    }
}
int dtype_bytes(lcpp_dtype t)
{
    switch (t) {
    case LCPP_INT32: case LCPP_UINT32: case LCPP_FLOAT32: return 4;
    case LCPP_INT64: case LCPP_UINT64: case LCPP_FLOAT64: return 8;
    default: return 0;
    }
}

template <class UK, class UV, bool PAIRS, bool DESC>
int rs_kind_dispatch(int kind, void *temp, size_t tb, const void *ki, void *ko, const void *vi, void *vo, uint64_t n,
                     hipStream_t s)
{
    switch (kind) {
    case kUnsigned: return rs_run<UK, UV, kUnsigned, PAIRS, DESC>(temp, tb, ki, ko, vi, vo, n, s);
    case kSigned: return rs_run<UK, UV, kSigned, PAIRS, DESC>(temp, tb, ki, ko, vi, vo, n, s);
    case kFloat: return rs_run<UK, UV, kFloat, PAIRS, DESC>(temp, tb, ki, ko, vi, vo, n, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}
template <class UK, class UV, bool PAIRS>
int rs_order_dispatch(bool desc, int kind, void *temp, size_t tb, const void *ki, void *ko, const void *vi, void *vo,
                      uint64_t n, hipStream_t s)
{
    return desc ? rs_kind_dispatch<UK, UV, PAIRS, true>(kind, temp, tb, ki, ko, vi, vo, n, s)
                : rs_kind_dispatch<UK, UV, PAIRS, false>(kind, temp, tb, ki, ko, vi, vo, n, s);
}

}  // namespace
}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_radix_sort_keys_temp_bytes(lcpp_dtype k, uint64_t n, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    const int kb = dtype_bytes(k);
    if (!kb) return LCPP_ERR_UNSUPPORTED_DTYPE;
    if (n > kMaxItems) return LCPP_ERR_INVALID_ARG;  // as the sort itself
    *bytes = rs_layout(n, kb, 0).total;
    return LCPP_OK;
}

extern "C" int lcpp_radix_sort_pairs_temp_bytes(lcpp_dtype k, lcpp_dtype v, uint64_t n,
                                                size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    const int kb = dtype_bytes(k), vb = dtype_bytes(v);
    if (!kb || !vb) return LCPP_ERR_UNSUPPORTED_DTYPE;
    if (n > kMaxItems) return LCPP_ERR_INVALID_ARG;
    *bytes = rs_layout(n, kb, vb).total;
    return LCPP_OK;
}

namespace {
int sort_keys(lcpp_dtype k, void *temp, size_t tb, const void *keys_in, void *keys_out, uint64_t n,
              bool desc, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int kind = key_kind(k);
    if (kind < 0) return LCPP_ERR_UNSUPPORTED_DTYPE;
    if (dtype_bytes(k) == 4)
        return rs_order_dispatch<uint32_t, uint32_t, false>(desc, kind, temp, tb, keys_in, keys_out, nullptr, nullptr,
                                                            n, s);
    return rs_order_dispatch<uint64_t, uint32_t, false>(desc, kind, temp, tb, keys_in, keys_out, nullptr, nullptr, n,
                                                        s);
}

int sort_pairs(lcpp_dtype k, lcpp_dtype v, void *temp, size_t tb, const void *keys_in, void *keys_out,
               const void *vals_in, void *vals_out, uint64_t n, bool desc, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int kind = key_kind(k);
    const int kb = dtype_bytes(k), vb = dtype_bytes(v);
    if (kind < 0 || !vb) return LCPP_ERR_UNSUPPORTED_DTYPE;
    if (kb == 4 && vb == 4)
        return rs_order_dispatch<uint32_t, uint32_t, true>(desc, kind, temp, tb, keys_in, keys_out, vals_in, vals_out,
                                                           n, s);
    if (kb == 4 && vb == 8)
        return rs_order_dispatch<uint32_t, uint64_t, true>(desc, kind, temp, tb, keys_in, keys_out, vals_in, vals_out,
                                                           n, s);
    if (kb == 8 && vb == 4)
        return rs_order_dispatch<uint64_t, uint32_t, true>(desc, kind, temp, tb, keys_in, keys_out, vals_in, vals_out,
                                                           n, s);
    return rs_order_dispatch<uint64_t, uint64_t, true>(desc, kind, temp, tb, keys_in, keys_out, vals_in, vals_out, n,
                                                       s);
}
}  // namespace

extern "C" int lcpp_radix_sort_keys(lcpp_dtype k, void *temp, size_t tb, const void *keys_in,
                                    void *keys_out, uint64_t n, void *stream)
{
    return sort_keys(k, temp, tb, keys_in, keys_out, n, false, stream);
}

extern "C" int lcpp_radix_sort_pairs(lcpp_dtype k, lcpp_dtype v, void *temp, size_t tb,
                                     const void *keys_in, void *keys_out, const void *vals_in,
                                     void *vals_out, uint64_t n, void *stream)
{
    return sort_pairs(k, v, temp, tb, keys_in, keys_out, vals_in, vals_out, n, false, stream);
}

extern "C" int lcpp_radix_sort_keys_descending(lcpp_dtype k, void *temp, size_t tb, const void *keys_in,
                                               void *keys_out, uint64_t n, void *stream)
{
    return sort_keys(k, temp, tb, keys_in, keys_out, n, true, stream);
}

extern "C" int lcpp_radix_sort_pairs_descending(lcpp_dtype k, lcpp_dtype v, void *temp, size_t tb,
                                                const void *keys_in, void *keys_out, const void *vals_in,
                                                void *vals_out, uint64_t n, void *stream)
{
    return sort_pairs(k, v, temp, tb, keys_in, keys_out, vals_in, vals_out, n, true, stream);
}

extern "C" int lcpp_test_set_sort_rank_path(int mode)
{
    if (mode < 0 || mode > 2) return LCPP_ERR_INVALID_ARG;
    g_rank_force.store(mode, std::memory_order_relaxed);
    return LCPP_OK;
}

extern "C" int lcpp_radix_sort_rank_path(int *path)
{
    if (!path) return LCPP_ERR_INVALID_ARG;
    *path = rs_rank_path(nullptr);
    return LCPP_OK;
}
