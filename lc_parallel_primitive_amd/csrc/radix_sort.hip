// radix_sort.hip — DeviceRadixSort::SortKeys/SortPairs (onesweep) for gfx950.
//
// Reference: device/device_radix_sort.h:129-153, 187-378 (reset, histogram,
// bin exclusive sum, then per pass x portion: look-back memset + onesweep),
// agent/agent_radix_sort_histogram.h:45-198, agent/agent_radix_sort_onesweep.h
// :43-500, block/block_radix_rank.h:66-336, agent/radix_rank_sort_operations.h,
// common/util_type.h:98-175 (twiddles), common/utils.h:273-324 (MatchAny).
//
// MI355X design (all HBM-bound integer/byte work, no MFMA):
//  * launch 0 "rs_init": zero the P digit histograms and the P tile tickets.
//  * launch 1 "rs_histogram": one read of the keys builds all P = sizeof(K)
//    8-bit digit histograms in LDS (one copy per wave to split same-address
//    atomic traffic), flushed with one global atomic per non-zero bin; the
//    same kernel zeroes the look-back region of pass 0.
//  * launches 2..P+1 "rs_onesweep": one tile of 256 x IPT keys per
//    workgroup, tile index from a dynamic ticket.  Keys are loaded
//    wave-striped (lane l of wave w, item u -> key w*64*IPT + u*64 + l), so
//    processing items in order u and lanes in order l visits keys in input
//    order.  Ranking: the 64-lane peer mask of equal digits comes from 8
//    ballots (wave64 MatchAny); each lane's rank inside its wave and digit is
//    counter + popcount(peers below it), and the lowest peer advances the
//    wave's LDS counter.  No LDS atomics, ranks are stable.  Thread d then
//    owns digit d: it sums the wave counters, publishes the tile count
//    (PARTIAL) at once, takes the tile's exclusive digit prefix with a
//    workgroup scan and walks back over earlier tiles until a GLOBAL word
//    (the tile-0 word carries the pass's global digit base, so every GLOBAL
//    word is already an absolute output offset).  Keys are scattered into
//    LDS in sorted order and written out so that consecutive threads write
//    consecutive positions of each digit run.  Values follow with the same
//    ranks.
//  * Look-back words are 32-bit {GLOBAL:1 | PARTIAL:1 | count:30}, polled
//    with agent-scope atomic loads (the 8 XCD L2s are not coherent).  Two
//    regions alternate between passes and each tile clears its own slots of
//    the other region for the next pass, so there is no per-pass memset
//    launch (the reference resets 256 MiB per pass, device_radix_sort.h:341).
//  * Keys-only sorts reserve no value scratch (the reference reserves N
//    values it never uses, device_radix_sort.h:118-122).
#include "common.hpp"

namespace lcpp {
namespace {

constexpr int kRsBlock = 256;
constexpr int kRsWaves = kRsBlock / kWave;
constexpr int kRadixBits = 8;
constexpr int kRadix = 256;
constexpr uint32_t kLbGlobal = 0x80000000u;
constexpr uint32_t kLbPartial = 0x40000000u;
constexpr uint32_t kLbMask = 0x3FFFFFFFu;
constexpr uint64_t kMaxItems = (1ull << 30) - 1;

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
// Digit of a twiddled key; -0.0 is folded onto +0.0
// (agent/radix_rank_sort_operations.h:33-62, ProcessFloatMinusZero).
template <class UK, int KIND>
__device__ __forceinline__ uint32_t digit_of(UK tk, uint32_t shift)
{
    if constexpr (KIND == kFloat) {
        constexpr UK high = UK(1) << (sizeof(UK) * 8 - 1);
        constexpr UK minus_zero = UK(~high);  // tw_in(-0.0)
        if (tk == minus_zero) tk = high;      // tw_in(+0.0)
    }
    return (uint32_t)(tk >> shift) & (kRadix - 1);
}

// 64-lane mask of the lanes whose 8-bit digit equals this lane's.
__device__ __forceinline__ uint64_t match_digit(uint32_t d)
{
    uint64_t m = ~0ull;
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t bal = ballot(bit);
        m &= bit ? bal : ~bal;
    }
    return m;
}

// Exclusive scan of one value per thread over the 256-thread workgroup.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t x, uint32_t *s_wsum)
{
    const uint32_t lane = lane_id(), wave = threadIdx.x / kWave;
    const uint32_t inc = wave_inclusive_scan(x, SumOp());
    if (lane == kWave - 1) s_wsum[wave] = inc;
    __syncthreads();
    uint32_t pre = 0;
#pragma unroll
    for (int w = 0; w < kRsWaves; ++w)
        if ((uint32_t)w < wave) pre += s_wsum[w];
    return pre + inc - x;
}

// ------------------------------------------------------------------ init
__global__ __launch_bounds__(256) void rs_init_kernel(uint32_t *bins, uint32_t nbins,
                                                      uint32_t *tickets, uint32_t ntickets)
{
    for (uint32_t i = threadIdx.x; i < nbins; i += 256) bins[i] = 0;
    for (uint32_t i = threadIdx.x; i < ntickets; i += 256) tickets[i] = 0;
}

// ------------------------------------------------------------------ histogram
template <class UK, int KIND>
__global__ __launch_bounds__(kRsBlock) void rs_histogram_kernel(const UK *__restrict__ keys,
                                                                uint64_t n, uint64_t chunk,
                                                                uint32_t *__restrict__ bins,
                                                                uint32_t *__restrict__ lb0,
                                                                uint64_t lb0_words)
{
    constexpr int P = sizeof(UK);
    __shared__ uint32_t s_hist[kRsWaves][P][kRadix];
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid / kWave;
    for (uint32_t i = tid; i < kRsWaves * P * kRadix; i += kRsBlock) (&s_hist[0][0][0])[i] = 0;
    __syncthreads();

    const uint64_t b0 = (uint64_t)blockIdx.x * chunk;
    const uint64_t b1 = b0 + chunk < n ? b0 + chunk : n;
    auto count = [&](UK raw) {
        const UK tk = tw_in<UK, KIND>(raw);
#pragma unroll
        for (int p = 0; p < P; ++p) atomicAdd(&s_hist[wave][p][digit_of<UK, KIND>(tk, p * kRadixBits)], 1u);
    };
    constexpr uint64_t V = 16 / sizeof(UK);
    constexpr uint64_t step = (uint64_t)kRsBlock * V * 4;
    uint64_t tail = b0;
    if ((reinterpret_cast<uintptr_t>(keys) & 15) == 0) {
        const uint64_t full_end = b0 + (b1 - b0) / step * step;
        for (uint64_t t = b0; t < full_end; t += step) {
            u32x4 v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                v[i] = ld16_nt((keys + t + ((uint64_t)i * kRsBlock + tid) * V));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (sizeof(UK) == 4) {
                    count(v[i].x);
                    count(v[i].y);
                    count(v[i].z);
                    count(v[i].w);
                } else {
                    count(((uint64_t)v[i].y << 32) | v[i].x);
                    count(((uint64_t)v[i].w << 32) | v[i].z);
                }
            }
        }
        tail = full_end;
    }
    for (uint64_t i = tail + tid; i < b1; i += kRsBlock) count(keys[i]);
    __syncthreads();
    for (uint32_t i = tid; i < P * kRadix; i += kRsBlock) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < kRsWaves; ++w) c += (&s_hist[w][0][0])[i];
        if (c) atomicAdd(&bins[i], c);
    }
    // zero the pass-0 look-back region
    const uint64_t stride = (uint64_t)gridDim.x * kRsBlock;
    for (uint64_t i = (uint64_t)blockIdx.x * kRsBlock + tid; i < lb0_words; i += stride) lb0[i] = 0;
}

// ------------------------------------------------------------------ onesweep pass
template <int IPT, class UK, class UV>
struct OnesweepSmem {
    static constexpr int TILE = kRsBlock * IPT;
    union {
        UK keys[TILE];
        UV vals[TILE];
    };
    uint32_t cnt[kRsWaves][kRadix];  // per-wave digit counters, then wave prefixes
    uint32_t dexcl[kRadix];          // tile exclusive digit prefix
    uint32_t goff[kRadix];           // output offset of sorted tile position 0 of digit d
    uint32_t wsum[2][kRsWaves];
    uint32_t tile;
};

template <int IPT, class UK, class UV, int KIND, bool PAIRS>
__global__ __launch_bounds__(kRsBlock) void rs_onesweep_kernel(
    const UK *__restrict__ kin, UK *__restrict__ kout, const UV *__restrict__ vin,
    UV *__restrict__ vout, uint32_t n, uint32_t shift, uint32_t *__restrict__ tickets,
    const uint32_t *__restrict__ bins, uint32_t *__restrict__ lb, uint32_t *__restrict__ lb_next)
{
    constexpr int TILE = kRsBlock * IPT;
    constexpr int WAVE_ITEMS = kWave * IPT;
    __shared__ OnesweepSmem<IPT, UK, UV> sm;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;

    for (int w = 0; w < kRsWaves; ++w) sm.cnt[w][tid] = 0;
    if (tid == 0) sm.tile = ticket(tickets);
    __syncthreads();
    const uint32_t tile = sm.tile;
    const uint32_t base = tile * TILE;
    const uint32_t valid = n - base < (uint32_t)TILE ? n - base : (uint32_t)TILE;

    // ---- load (wave-striped), twiddle; pads are all-ones -> digit 255, last
    UK tk[IPT];
    UV v[PAIRS ? IPT : 1];
    const uint32_t wbase = base + wave * WAVE_ITEMS + lane;
    if (valid == (uint32_t)TILE) {
#pragma unroll
        for (int u = 0; u < IPT; ++u) tk[u] = tw_in<UK, KIND>(__builtin_nontemporal_load(kin + wbase + u * kWave));
        if constexpr (PAIRS) {
#pragma unroll
            for (int u = 0; u < IPT; ++u) v[u] = __builtin_nontemporal_load(vin + wbase + u * kWave);
        }
    } else {
#pragma unroll
        for (int u = 0; u < IPT; ++u) {
            const uint32_t idx = wbase + u * kWave;
            tk[u] = idx < n ? tw_in<UK, KIND>(kin[idx]) : UK(~UK(0));
            if constexpr (PAIRS) v[u] = idx < n ? vin[idx] : UV(0);
        }
    }

    // ---- stable rank within (wave, digit)
    uint32_t rank[IPT];
    uint32_t *cnt = sm.cnt[wave];
#pragma unroll
    for (int u = 0; u < IPT; ++u) {
        const uint32_t d = digit_of<UK, KIND>(tk[u], shift);
        const uint64_t peers = match_digit(d);
        const uint32_t below = mask_rank(peers);
        const uint32_t c = cnt[d];
        rank[u] = c + below;
        if (below == 0) cnt[d] = c + (uint32_t)__popcll(peers);
    }
    __syncthreads();

    // ---- thread d owns digit d
    const uint32_t d = tid;
    uint32_t total = 0;
#pragma unroll
    for (int w = 0; w < kRsWaves; ++w) {
        const uint32_t c = sm.cnt[w][d];
        sm.cnt[w][d] = total;  // wave prefix within the tile
        total += c;
    }
    if (d == kRadix - 1) total -= (uint32_t)TILE - valid;  // drop the pads
    if (tile > 0) st_relaxed(&lb[(size_t)tile * kRadix + d], total | kLbPartial);
    lb_next[(size_t)tile * kRadix + d] = 0;  // slot of the next pass
    const uint32_t dexcl = block_excl_scan(total, sm.wsum[0]);
    sm.dexcl[d] = dexcl;
    uint32_t gbase = 0;
    if (tile == 0) gbase = block_excl_scan(bins[d], sm.wsum[1]);
    __syncthreads();

    // ---- scatter keys into LDS in sorted-tile order
#pragma unroll
    for (int u = 0; u < IPT; ++u) {
        const uint32_t dd = digit_of<UK, KIND>(tk[u], shift);
        rank[u] += sm.dexcl[dd] + sm.cnt[wave][dd];
        sm.keys[rank[u]] = tk[u];
    }

    // ---- decoupled look-back for digit d
    uint32_t excl;
    if (tile == 0) {
        excl = gbase;
        st_relaxed(&lb[d], (gbase + total) | kLbGlobal);
    } else {
        uint32_t acc = 0;
        int64_t j = (int64_t)tile - 1;
        for (;;) {
            const uint32_t *p = &lb[(size_t)j * kRadix + d];
            uint32_t w = ld_relaxed(p);
            for (uint32_t spins = 0; w == 0 && spins < kSpinLimit; ++spins) {
                __builtin_amdgcn_s_sleep(1);
                w = ld_relaxed(p);
            }
            if (w == 0) w = kLbGlobal;  // gave up: terminate the walk
            acc += w & kLbMask;
            if (w & kLbGlobal) break;
            --j;
        }
        excl = acc;
        st_relaxed(&lb[(size_t)tile * kRadix + d], (acc + total) | kLbGlobal);
    }
    sm.goff[d] = excl - dexcl;
    __syncthreads();

    // ---- write out: consecutive threads -> consecutive positions of a digit run
    uint32_t dg[PAIRS ? IPT : 1];
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const uint32_t i = j * kRsBlock + tid;
        const UK k = sm.keys[i];
        const uint32_t dd = digit_of<UK, KIND>(k, shift);
        if constexpr (PAIRS) dg[j] = dd;
        const uint32_t pos = i + sm.goff[dd];
        if (i < valid && pos < n) kout[pos] = tw_out<UK, KIND>(k);
    }
    if constexpr (PAIRS) {
        __syncthreads();
#pragma unroll
        for (int u = 0; u < IPT; ++u) sm.vals[rank[u]] = v[u];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const uint32_t i = j * kRsBlock + tid;
            const uint32_t pos = i + sm.goff[dg[j]];
            if (i < valid && pos < n) vout[pos] = sm.vals[i];
        }
    }
}

// ------------------------------------------------------------------ host side
template <class UK>
constexpr int rs_ipt()
{
    return sizeof(UK) == 4 ? 16 : 16;
}

struct RsLayout {
    uint64_t passes, tiles, bins_off, tickets_off, lb_off, lb_words, ktmp_off, vtmp_off, total;
};

RsLayout rs_layout(uint64_t n, int key_bytes, int val_bytes, int ipt)
{
    RsLayout L{};
    L.passes = (uint64_t)key_bytes;  // 8-bit digits
    const uint64_t tile = (uint64_t)kRsBlock * ipt;
    L.tiles = n ? ceil_div(n, tile) : 0;
    L.bins_off = 0;
    L.tickets_off = align_up(L.passes * kRadix * 4, 256);
    L.lb_off = L.tickets_off + 256;
    L.lb_words = L.tiles * kRadix;
    L.ktmp_off = L.lb_off + align_up(2 * L.lb_words * 4, 256);
    L.vtmp_off = L.ktmp_off + align_up(n * key_bytes, 256);
    L.total = L.vtmp_off + align_up(n * val_bytes, 256);
    return L;
}

template <class UK, class UV, int KIND, bool PAIRS>
int rs_run(void *temp, size_t temp_bytes, const void *kin_, void *kout_, const void *vin_,
           void *vout_, uint64_t n, hipStream_t s)
{
    constexpr int IPT = rs_ipt<UK>();
    if (n == 0) return LCPP_OK;
    if (n > kMaxItems) return LCPP_ERR_INVALID_ARG;
    const UK *kin = static_cast<const UK *>(kin_);
    UK *kout = static_cast<UK *>(kout_);
    const UV *vin = static_cast<const UV *>(vin_);
    UV *vout = static_cast<UV *>(vout_);
    if (!kin || !kout || (PAIRS && (!vin || !vout))) return LCPP_ERR_INVALID_ARG;
    const RsLayout L = rs_layout(n, sizeof(UK), PAIRS ? sizeof(UV) : 0, IPT);
    if (temp_bytes < L.total) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    char *t = static_cast<char *>(temp);
    uint32_t *bins = reinterpret_cast<uint32_t *>(t + L.bins_off);
    uint32_t *tickets = reinterpret_cast<uint32_t *>(t + L.tickets_off);
    uint32_t *lb[2] = {reinterpret_cast<uint32_t *>(t + L.lb_off),
                       reinterpret_cast<uint32_t *>(t + L.lb_off) + L.lb_words};
    UK *ktmp = reinterpret_cast<UK *>(t + L.ktmp_off);
    UV *vtmp = reinterpret_cast<UV *>(t + L.vtmp_off);
    const int P = (int)L.passes;

    LCPP_LAUNCH("rs_init", s, rs_init_kernel<<<1, 256, 0, s>>>(bins, P * kRadix, tickets, P));
    LCPP_CHECK_LAUNCH();
    {
        const uint64_t htile = (uint64_t)kRsBlock * 4 * (16 / sizeof(UK));
        const uint64_t htiles = ceil_div(n, htile);
        uint64_t grid = htiles < 1024 ? htiles : 1024;
        const uint64_t chunk = ceil_div(htiles, grid) * htile;
        grid = ceil_div(n, chunk);
        LCPP_LAUNCH("rs_histogram", s,
                    rs_histogram_kernel<UK, KIND><<<(uint32_t)grid, kRsBlock, 0, s>>>(kin, n, chunk, bins,
                                                                                      lb[0], L.lb_words));
        LCPP_CHECK_LAUNCH();
    }
    // ping-pong so that the last pass lands in the output and the input is preserved
    const UK *src_k = kin;
    const UV *src_v = vin;
    for (int p = 0; p < P; ++p) {
        const bool to_out = ((P - 1 - p) % 2) == 0;
        UK *dst_k = to_out ? kout : ktmp;
        UV *dst_v = to_out ? vout : vtmp;
        LCPP_LAUNCH("rs_onesweep", s,
                    (rs_onesweep_kernel<IPT, UK, UV, KIND, PAIRS><<<(uint32_t)L.tiles, kRsBlock, 0, s>>>(
                        src_k, dst_k, src_v, dst_v, (uint32_t)n, (uint32_t)(p * kRadixBits),
                        tickets + p, bins + p * kRadix, lb[p & 1], lb[(p + 1) & 1])));
        LCPP_CHECK_LAUNCH();
        src_k = dst_k;
        src_v = dst_v;
    }
    return LCPP_OK;
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

template <class UK, class UV, bool PAIRS>
int rs_kind_dispatch(int kind, void *temp, size_t tb, const void *ki, void *ko, const void *vi,
                     void *vo, uint64_t n, hipStream_t s)
{
    switch (kind) {
    case kUnsigned: return rs_run<UK, UV, kUnsigned, PAIRS>(temp, tb, ki, ko, vi, vo, n, s);
    case kSigned: return rs_run<UK, UV, kSigned, PAIRS>(temp, tb, ki, ko, vi, vo, n, s);
    case kFloat: return rs_run<UK, UV, kFloat, PAIRS>(temp, tb, ki, ko, vi, vo, n, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

}  // namespace
}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_radix_sort_keys_temp_bytes(lcpp_dtype k, uint64_t n, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    const int kb = dtype_bytes(k);
    if (!kb) return LCPP_ERR_UNSUPPORTED_DTYPE;
    *bytes = rs_layout(n, kb, 0, kb == 4 ? rs_ipt<uint32_t>() : rs_ipt<uint64_t>()).total;
    return LCPP_OK;
}

extern "C" int lcpp_radix_sort_pairs_temp_bytes(lcpp_dtype k, lcpp_dtype v, uint64_t n,
                                                size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    const int kb = dtype_bytes(k), vb = dtype_bytes(v);
    if (!kb || !vb) return LCPP_ERR_UNSUPPORTED_DTYPE;
    *bytes = rs_layout(n, kb, vb, kb == 4 ? rs_ipt<uint32_t>() : rs_ipt<uint64_t>()).total;
    return LCPP_OK;
}

extern "C" int lcpp_radix_sort_keys(lcpp_dtype k, void *temp, size_t tb, const void *keys_in,
                                    void *keys_out, uint64_t n, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int kind = key_kind(k);
    if (kind < 0) return LCPP_ERR_UNSUPPORTED_DTYPE;
    if (dtype_bytes(k) == 4)
        return rs_kind_dispatch<uint32_t, uint32_t, false>(kind, temp, tb, keys_in, keys_out, nullptr, nullptr, n, s);
    return rs_kind_dispatch<uint64_t, uint32_t, false>(kind, temp, tb, keys_in, keys_out, nullptr, nullptr, n, s);
}

extern "C" int lcpp_radix_sort_pairs(lcpp_dtype k, lcpp_dtype v, void *temp, size_t tb,
                                     const void *keys_in, void *keys_out, const void *vals_in,
                                     void *vals_out, uint64_t n, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int kind = key_kind(k);
    const int kb = dtype_bytes(k), vb = dtype_bytes(v);
    if (kind < 0 || !vb) return LCPP_ERR_UNSUPPORTED_DTYPE;
    if (kb == 4 && vb == 4)
        return rs_kind_dispatch<uint32_t, uint32_t, true>(kind, temp, tb, keys_in, keys_out, vals_in, vals_out, n, s);
    if (kb == 4 && vb == 8)
        return rs_kind_dispatch<uint32_t, uint64_t, true>(kind, temp, tb, keys_in, keys_out, vals_in, vals_out, n, s);
    if (kb == 8 && vb == 4)
        return rs_kind_dispatch<uint64_t, uint32_t, true>(kind, temp, tb, keys_in, keys_out, vals_in, vals_out, n, s);
    return rs_kind_dispatch<uint64_t, uint64_t, true>(kind, temp, tb, keys_in, keys_out, vals_in, vals_out, n, s);
}
