// reduce_by_key.hip — DeviceReduce::ReduceByKey for gfx950.
//
// Reference: device/device_reduce.h:110-125 (temp bytes), 277-318 (entry
// point), 462-516 (dispatch), device/details/reduce_by_key.h:61-258.
//
// Semantics: run r = the r-th maximal run of equal consecutive keys (keys
// compared in their own type); unique_out[r] = its key, aggregates_out[r] =
// the op-fold of its values, *num_runs_out = the number of runs.
//
// Design (tile machinery in by_key.hpp): single pass.  Two look-backs run
// side by side in two waves of each tile: the number of heads before the
// tile (a plain sum scan over tiles, it fixes the output index of every run)
// and the fold of the open run entering the tile (a segmented scan: a tile
// that contains a head publishes INCLUSIVE at once).  The key loads are
// issued before the value loads, and the tile's head count is published as
// soon as the keys are in, while the values are still arriving: the count
// chain is the longer wait (2^28 int32 keys, f32 values, runs of mean 128:
// 531-546 -> 495-500 us per call).  A head at element
// i > 0 closes the run that ends at i - 1 and writes its key and aggregate;
// element n - 1 writes the last run and the run count, as the reference
// does (reduce_by_key.h:231-254).  Consecutive runs land at consecutive
// output positions, so the writes of one wave coalesce in L2.
//
// Bytes: keys + values read, plus (sizeof K + sizeof V) per run written.
#include "by_key.hpp"

namespace lcpp {
namespace {

template <class V>
struct RbkLayout {
    uint64_t tiles, cwords_off, vwords_off, total;
};
template <class V>
RbkLayout<V> rbk_layout(uint64_t n)
{
    RbkLayout<V> L{};
    L.tiles = bk_tiles<V>(n);
    L.cwords_off = kStatusBytes;  // after the status header
    L.vwords_off = L.cwords_off + align_up(L.tiles * 8, 256);
    L.total = L.vwords_off + align_up(L.tiles * 8 * lb_words<V>(), 256);
    return L;
}

__global__ void rbk_zero_runs(uint32_t *num_runs) { *num_runs = 0; }

template <class K, class V, class Op>
__global__ __launch_bounds__(kBkBlock) void reduce_by_key_kernel(const K *__restrict__ keys,
                                                                 const V *__restrict__ vin,
                                                                 K *__restrict__ unique_out,
                                                                 V *__restrict__ agg_out,
                                                                 uint32_t *__restrict__ num_runs, uint32_t n,
                                                                 uint64_t *cwords, uint64_t *vwords, int vec_ok,
                                                                 WaitCtl ctl)
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
    __shared__ V s_vprefix;
    __shared__ uint32_t s_cprefix;

    Op op;
    const V ident = op_identity<Op, V>();
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint32_t base = tile * TILE;
    const uint32_t valid = n - base < TILE ? n - base : TILE;
    const bool fast = valid == TILE && vec_ok;

    BkRegs<K, V> r;
    bk_load<true>(r, keys, vin, base, valid, fast, tid);
    if (tid < kBkVecs) s_F[tid] = 0;
    K prev0[kBkVecs];
    const uint32_t fl = bk_heads<K, VP>(r.key, prev0, s_last, s_pred, keys, base, tile, tid);
    if constexpr (kKeysInLds) {
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
#pragma unroll
            for (int j = 0; j < VP; ++j) s_keys[bk_elem<V>(k, tid, j)] = r.key[k][j];
    }

    // head counts first (keys only; the values are still arriving): per
    // vector a wave scan, wave totals to LDS, and the tile's count is
    // published before the values are folded, so successors' count
    // look-backs find it as early as possible
    uint32_t exC[kBkVecs];
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        const uint32_t c = (uint32_t)__builtin_popcount((fl >> (k * VP)) & ((1u << VP) - 1u));
        const uint32_t ci = wave_inclusive_scan(c, SumOp());
        exC[k] = ci - c;
        if (lane == kWave - 1) s_C[k][wave] = ci;
    }
    __syncthreads();
    uint32_t tcount = 0;
    if (wave == 1) {
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
#pragma unroll
            for (int w = 0; w < kBkWaves; ++w) tcount += s_C[k][w];
        if (lane == 0) lb_publish(cwords, tile, tcount, tile == 0 ? kStInclusive : kStPartial, ctl);
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

    // look-backs: wave 0 the open-run fold, wave 1 the head count (its
    // PARTIAL is already published)
    if (wave == 0) {
        bool tf = false;
        V ts = ident;
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
#pragma unroll
            for (int w = 0; w < kBkWaves; ++w) seg_fold(tf, ts, ((s_F[k] >> w) & 1u) != 0, s_S[k][w], op);
        // always wait: a head at the tile's first element closes the run the
        // previous tile left open, whose aggregate is exactly this prefix
        const V p = lb_segmented_tile(vwords, tile, ts, tf, true, op, ident, ctl);
        if (lane == 0) s_vprefix = p;
    } else if (wave == 1) {
        uint32_t p = 0;
        if (tile > 0) {
            p = lb_wait_prefix(cwords, tile, SumOp(), 0u, ctl);
            if (lane == 0) lb_publish(cwords, tile, p + tcount, kStInclusive, ctl);
        }
        if (lane == 0) s_cprefix = p;
    }
    __syncthreads();

    // pass 2: rescan from the exact prefixes; heads close the previous run
    V vrun = s_vprefix;
    uint32_t crun = s_cprefix;
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        V pw = vrun;
        uint32_t cw = crun;
#pragma unroll
        for (int w = 0; w < kBkWaves; ++w) {
            const bool f = ((s_F[k] >> w) & 1u) != 0;
            const V sv = s_S[k][w];
            const uint32_t cv = s_C[k][w];
            if ((uint32_t)w < wave) {
                pw = f ? sv : op(pw, sv);
                cw += cv;
            }
            vrun = f ? sv : op(vrun, sv);
            crun += cv;
        }
        V s = ((exF >> k) & 1u) ? exS[k] : op(pw, exS[k]);
        uint32_t c = cw + exC[k];
#pragma unroll
        for (int j = 0; j < VP; ++j) {
            const uint32_t e = bk_elem<V>(k, tid, j);
            if (e < valid) {
                const uint32_t gi = base + e;
                const bool h = ((fl >> (k * VP + j)) & 1u) != 0;
                const V x = r.val[k][j];
                // run indices are < n by construction; the bound keeps a
                // broken invariant (a look-back wait past its spin limit)
                // from ever writing outside the outputs
                if (h) {
                    if (gi > 0 && c - 1 < n) {
                        if constexpr (kKeysInLds) unique_out[c - 1] = e > 0 ? s_keys[e - 1] : s_pred;
                        else unique_out[c - 1] = j > 0 ? r.key[k][j - 1] : prev0[k];
                        agg_out[c - 1] = s;
                    }
                    ++c;
                    s = x;
                } else {
                    s = op(s, x);
                }
                if (gi == n - 1 && c - 1 < n) {
                    if constexpr (kKeysInLds) unique_out[c - 1] = s_keys[e];
                    else unique_out[c - 1] = r.key[k][j];
                    agg_out[c - 1] = s;
                    *num_runs = c;
                }
            }
        }
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
    const RbkLayout<V> L = rbk_layout<V>(n);
    if (tb < L.total) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    char *t = static_cast<char *>(temp);
    uint64_t *cwords = reinterpret_cast<uint64_t *>(t + L.cwords_off);
    uint64_t *vwords = reinterpret_cast<uint64_t *>(t + L.vwords_off);
    // the status header and both regions are contiguous up to alignment
    // padding: one fill
    if (lb_init(reinterpret_cast<uint64_t *>(t), L.total / 8, s, "reduce_by_key_init") != LCPP_OK)
        return LCPP_ERR_HIP;
    const WaitCtl ctl = wait_ctl(reinterpret_cast<uint32_t *>(t));
    const int vec_ok = ((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(in)) & 15) == 0;
    LCPP_LAUNCH("reduce_by_key", s,
                (reduce_by_key_kernel<K, V, Op><<<(uint32_t)L.tiles, kBkBlock, 0, s>>>(
                    keys, in, uk, agg, num_runs, (uint32_t)n, cwords, vwords, vec_ok, ctl)));
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
    *bytes = rbk_wide(v) ? rbk_layout<uint64_t>(n).total : rbk_layout<uint32_t>(n).total;
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
