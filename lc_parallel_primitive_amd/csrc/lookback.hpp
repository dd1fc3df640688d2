// lookback.hpp — single-pass decoupled look-back over packed 64-bit words.
//
// Reference: device/details/single_pass_scan_operator.h:25-251
// (ScanTileStatus, ScanTileStateViewer, TilePrefixCallbackOp).
//
// Each tile owns self-validating words written with agent-scope relaxed
// stores (the 8 XCD L2s of an MI355X are not coherent with each other):
//   4-byte payload: one word  {payload:32 | status:32}
//   8-byte payload: two words {lo:32 | status:32}, {hi:32 | status:32}
// A reader accepts a tile only when the statuses of its words agree.  Each
// status value is written at most once per word, so agreeing statuses come
// from one publish and no fence is needed.  The reference keeps status and
// values in separate arrays with no ordering between them
// (single_pass_scan_operator.h:81-93); release/acquire pairs instead cost
// an L2 write-back/invalidate per publish on this part.
//
// The prefix wait is executed by one wave: lane l < 16 polls predecessor
// top - l, all loads issued before any wait, and the wave stops at the
// nearest INCLUSIVE tile, waiting only for closer predecessors.  A wait
// that exhausts its bounded spin gives up and records the fact in the call's
// status word (WaitCtl), so a wrong result is reported, never a hung GPU.
#pragma once

#include "common.hpp"

namespace lcpp {

constexpr uint32_t kStInvalid = 0, kStPartial = 1, kStInclusive = 2;

template <class T>
constexpr int lb_words()
{
    return sizeof(T) == 4 ? 1 : 2;
}

template <class T>
__device__ __forceinline__ uint64_t lb_bits(T v)
{
    if constexpr (sizeof(T) == 4) return __builtin_bit_cast(uint32_t, v);
    else return __builtin_bit_cast(uint64_t, v);
}
template <class T>
__device__ __forceinline__ T lb_from_bits(uint64_t b)
{
    if constexpr (sizeof(T) == 4) return __builtin_bit_cast(T, (uint32_t)b);
    else return __builtin_bit_cast(T, b);
}

template <class T>
__device__ __forceinline__ void lb_publish(uint64_t *words, uint32_t tile, T v, uint32_t status, const WaitCtl &ctl)
{
    if (tile == ctl.withhold) return;  // test hook: this tile never publishes
    const uint64_t b = lb_bits(v);
    if constexpr (sizeof(T) == 4) {
        st_relaxed(&words[tile], (b << 32) | status);
    } else {
        st_relaxed(&words[2 * (uint64_t)tile], (uint64_t)((b << 32) | status));
        st_relaxed(&words[2 * (uint64_t)tile + 1], (uint64_t)((b & 0xFFFFFFFF00000000ull) | status));
    }
}

// Predecessors polled per round trip.  A poll is an agent-scope load that
// is served past the XCD's L2; under full HBM load the polls of ~1000
// resident tiles compete with the data stream.  Measured at 2^28 (us per
// scan, u32): 64 lanes 423, 32 lanes 386, 16 lanes 371, 8 lanes 383, 4
// lanes 387 (a 16-word window is one 128-byte line of 8-byte words).
// Polling 2 or 4 windows of 64 per round trip: 488 / 565 us.
constexpr int kLbPollWidth = 16;

// Exclusive prefix of `tile` (tile > 0): the op-fold of the aggregates of
// the tiles after the nearest INCLUSIVE predecessor, folded onto that
// predecessor's inclusive value.  Every lane returns it.  `op` must be
// commutative (sum, min, max): a window is reduced as a tree.
// W = predecessors polled per round trip (kLbPollWidth, or up to 64 where few
// tiles compete for the memory system, as in ReduceByKey's emit launch).
template <int W = kLbPollWidth, class T, class Op>
__device__ T lb_wait_prefix(const uint64_t *words, uint32_t tile, Op op, T identity, const WaitCtl &ctl)
{
    const uint32_t lane = lane_id();
    T excl = identity;
    int64_t top = (int64_t)tile - 1;
    uint32_t spins = 0;
    for (;;) {
        // Lane l < W polls predecessor top - l; the other lanes
        // re-read lane 0's word (same cache line) and are neutral.  The load
        // is unconditional (an index below 0 reads word 0 and is then treated
        // as INCLUSIVE identity), so no branch separates issue and wait.
        static_assert(W >= 1 && W <= kWave, "poll width");
        const bool poller = lane < (uint32_t)W;
        const int64_t j = top - (int64_t)(poller ? lane : 0u);
        const uint64_t jj = j < 0 ? 0 : (uint64_t)j;
        uint32_t s;
        T v;
        if constexpr (sizeof(T) == 4) {
            const uint64_t w = ld_relaxed(&words[jj]);
            s = (uint32_t)w;
            v = lb_from_bits<T>(w >> 32);
        } else {
            const uint64_t lo = ld_relaxed(&words[2 * jj]);
            const uint64_t hi = ld_relaxed(&words[2 * jj + 1]);
            s = (uint32_t)lo == (uint32_t)hi ? (uint32_t)lo : kStInvalid;
            v = lb_from_bits<T>((hi & 0xFFFFFFFF00000000ull) | (lo >> 32));
        }
        if (j < 0) {
            s = kStInclusive;
            v = identity;
        }
        if (!poller) {
            s = kStPartial;
            v = identity;
        }
        const uint64_t incl = ballot(s == kStInclusive);
        const uint32_t stop = incl ? (uint32_t)__builtin_ctzll(incl) : (uint32_t)(kWave - 1);
        const bool in_range = lane <= stop;
        if (ballot(in_range && s == kStInvalid) != 0) {
            if (++spins < ctl.spin_limit) {
                __builtin_amdgcn_s_sleep(1);
                continue;  // re-poll the same window
            }
            if (lane == 0) report_timeout(ctl);  // give up with what has been published
        }
        const T acc = in_range ? v : identity;
        const bool found = incl != 0;
        excl = op(excl, wave_allreduce(acc, op));
        if (found) break;
        top -= W;
    }
    return excl;
}

// Plain scan tile: publish PARTIAL(agg), wait for the prefix, publish
// INCLUSIVE(prefix op agg).  Returns the exclusive prefix (identity for
// tile 0) in every lane.
template <int W = kLbPollWidth, class T, class Op>
__device__ __forceinline__ T lb_scan_tile(uint64_t *words, uint32_t tile, T agg, Op op, T identity,
                                          const WaitCtl &ctl)
{
    const uint32_t lane = lane_id();
    if (tile == 0) {
        if (lane == 0) lb_publish(words, 0, agg, kStInclusive, ctl);
        return identity;
    }
    if (lane == 0) lb_publish(words, tile, agg, kStPartial, ctl);
    const T excl = lb_wait_prefix<W>(words, tile, op, identity, ctl);
    if (lane == 0) lb_publish(words, tile, op(excl, agg), kStInclusive, ctl);
    return excl;
}

// Plain scan tile of a scan that starts from `init` (the exclusive prefix of
// tile 0): tile 0 publishes INCLUSIVE(init op agg), so every later prefix
// holds init exactly once.
template <int W = kLbPollWidth, class T, class Op>
__device__ __forceinline__ T lb_scan_tile_init(uint64_t *words, uint32_t tile, T agg, Op op, T identity, T init,
                                               const WaitCtl &ctl)
{
    if (tile == 0) {
        if (lane_id() == 0) lb_publish(words, 0, op(init, agg), kStInclusive, ctl);
        return init;
    }
    return lb_scan_tile<W>(words, tile, agg, op, identity, ctl);
}

// Segmented (by-key) scan tile.  A tile that contains a segment head knows
// its inclusive value at once (the fold since its last head) and publishes
// INCLUSIVE(agg) before it waits; it waits only if its first element is not
// a head (`need_prefix`).  A tile without a head is a plain scan tile.
template <int W = kLbPollWidth, class T, class Op>
__device__ __forceinline__ T lb_segmented_tile(uint64_t *words, uint32_t tile, T agg, bool has_head,
                                              bool need_prefix, Op op, T identity, const WaitCtl &ctl)
{
    if (!has_head) return lb_scan_tile<W>(words, tile, agg, op, identity, ctl);
    if (lane_id() == 0) lb_publish(words, tile, agg, kStInclusive, ctl);
    if (tile == 0 || !need_prefix) return identity;
    return lb_wait_prefix<W>(words, tile, op, identity, ctl);
}

namespace {
__global__ __launch_bounds__(256) void lb_init_kernel(uint64_t *words, uint64_t count)
{
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += stride) words[i] = 0;
}

// Zero `count` words on stream s (grid-stride fill kernel; a kernel rather
// than hipMemsetAsync so the call can be graph-captured).  Callers pass the
// status header and the look-back words behind it as one range.
int lb_init(uint64_t *words, uint64_t count, hipStream_t s, const char *name)
{
    if (!count) return LCPP_OK;
    const uint64_t g = ceil_div(count, 256);
    const uint32_t grid = (uint32_t)(g < 1024 ? g : 1024);
    LCPP_LAUNCH(name, s, lb_init_kernel<<<grid, 256, 0, s>>>(words, count));
    return hipGetLastError() == hipSuccess ? LCPP_OK : LCPP_ERR_HIP;
}
}  // namespace

}  // namespace lcpp
