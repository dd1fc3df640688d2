// scan_by_key.hip — DeviceScan::Exclusive/InclusiveScanByKey and
// Exclusive/InclusiveSumByKey for gfx950.
//
// Reference: device/device_scan.h:91-107 (temp bytes), 206-339 (the four
// entry points), 413-482 (dispatch), device/details/scan_by_key.h:77-258.
//
// Semantics: segments are maximal runs of equal consecutive keys;
//   exclusive: out[i] = init at a head, else op(fold(in[head..i)), init)
//   inclusive: out[i] = op(fold(in[head..i]), init)
// The reference applies AddInitToScan to inclusive results too, which
// overwrites every head with init (scan_by_key.h:113-128); here heads of an
// inclusive scan get op(in[head], init), the inclusive scan's definition.
//
// Bytes: keys + values read, values written: sizeof K + 2 sizeof V per
// element, single pass (by_key.hpp for the tile design).
#include <cstring>

#include "by_key.hpp"

namespace lcpp {
namespace {

template <class V>
uint64_t sbk_temp_bytes(uint64_t n)
{
    const uint64_t tiles = bk_tiles<V>(n);
    return tiles ? kStatusBytes + align_up(tiles * 8 * lb_words<V>(), 256) : 0;  // status header, look-back words
}

template <class K, class V, class Op, bool INCLUSIVE>
__global__ __launch_bounds__(kBkBlock) void scan_by_key_kernel(const K *__restrict__ keys,
                                                               const V *__restrict__ vin,
                                                               V *__restrict__ vout, uint64_t n,
                                                               uint64_t *words, V init, int vec_ok,
                                                               WaitCtl ctl)
{
    constexpr int VP = bk_vp<V>();
    constexpr uint32_t TILE = bk_tile<V>();
    __shared__ K s_last[kBkVecs][kBkWaves];
    __shared__ K s_pred;
    __shared__ V s_S[kBkVecs][kBkWaves];
    __shared__ uint32_t s_F[kBkVecs];  // bit w: wave w of vector k has a head
    __shared__ V s_prefix;
    __shared__ uint32_t s_first_head;

    Op op;
    const V ident = op_identity<Op, V>();
    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint64_t base = (uint64_t)tile * TILE;
    const uint32_t valid = n - base < TILE ? (uint32_t)(n - base) : TILE;
    const bool fast = valid == TILE && vec_ok;

    BkRegs<K, V> r;
    bk_load(r, keys, vin, base, valid, fast, tid);
    if (tid < kBkVecs) s_F[tid] = 0;
    K prev0[kBkVecs];
    const uint32_t fl = bk_heads<K, VP>(r.key, prev0, s_last, s_pred, keys, base, tile, tid);
    if (tid == 0) s_first_head = fl & 1u;

    // pass 1: thread pairs, wave segmented scans, wave totals to LDS
    V exS[kBkVecs];
    uint32_t exF = 0;
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        bool f;
        V s;
        bk_thread_pair<V>(r.val[k], fl >> (k * VP), op, f, s);
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

    // tile aggregate and look-back (wave 0)
    if (wave == 0) {
        bool tf = false;
        V ts = ident;
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
#pragma unroll
            for (int w = 0; w < kBkWaves; ++w) seg_fold(tf, ts, ((s_F[k] >> w) & 1u) != 0, s_S[k][w], op);
        const V p = lb_segmented_tile(words, tile, ts, tf, s_first_head == 0, op, ident, ctl);
        if (lane == 0) s_prefix = p;
    }
    __syncthreads();

    // pass 2: rescan each thread's items from its exact prefix
    V run = s_prefix;  // fold since the last head before vector k
#pragma unroll
    for (int k = 0; k < kBkVecs; ++k) {
        V pw = run;
#pragma unroll
        for (int w = 0; w < kBkWaves; ++w) {
            const bool f = ((s_F[k] >> w) & 1u) != 0;
            const V sv = s_S[k][w];
            if ((uint32_t)w < wave) pw = f ? sv : op(pw, sv);
            run = f ? sv : op(run, sv);
        }
        V s = ((exF >> k) & 1u) ? exS[k] : op(pw, exS[k]);
#pragma unroll
        for (int j = 0; j < VP; ++j) {
            const bool h = ((fl >> (k * VP + j)) & 1u) != 0;
            const V x = r.val[k][j];
            if constexpr (INCLUSIVE) {
                s = h ? x : op(s, x);
                r.val[k][j] = op(s, init);
            } else {
                r.val[k][j] = h ? init : op(s, init);
                s = h ? x : op(s, x);
            }
        }
    }

    const __amdgpu_buffer_rsrc_t ro = make_rsrc(vout + base, valid * (uint32_t)sizeof(V));
    if (fast) {
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
            buf_st16_nt(ro, tid * 16 + (uint32_t)k * kBkBlock * 16, 0, pack16<V>(r.val[k]));
    } else {
#pragma unroll
        for (int k = 0; k < kBkVecs; ++k)
#pragma unroll
            for (int j = 0; j < VP; ++j)
                buf_st_elem<V>(ro, bk_elem<V>(k, tid, j) * (uint32_t)sizeof(V), 0, r.val[k][j]);
    }
}

template <class K, class V, class Op>
int sbk_launch(bool inclusive, void *temp, size_t tb, const void *keys_, const void *in_, void *out_,
               uint64_t n, const void *init_, hipStream_t s)
{
    if (n == 0) return LCPP_OK;
    const K *keys = static_cast<const K *>(keys_);
    const V *in = static_cast<const V *>(in_);
    V *out = static_cast<V *>(out_);
    if (!keys || !in || !out) return LCPP_ERR_INVALID_ARG;
    const uint64_t tiles = bk_tiles<V>(n);
    if (tiles > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;
    if (tb < sbk_temp_bytes<V>(n)) return LCPP_ERR_TEMP_TOO_SMALL;
    if (!temp || (reinterpret_cast<uintptr_t>(temp) & 255)) return LCPP_ERR_INVALID_ARG;
    V init;
    if (init_) memcpy(&init, init_, sizeof(V));
    else init = V(0);
    uint64_t *head = static_cast<uint64_t *>(temp);  // status header, then the look-back words
    uint64_t *words = head + kStatusBytes / 8;
    if (lb_init(head, kStatusBytes / 8 + tiles * lb_words<V>(), s, "scan_by_key_init") != LCPP_OK)
        return LCPP_ERR_HIP;
    const WaitCtl ctl = wait_ctl(static_cast<uint32_t *>(temp));
    const int vec_ok = ((reinterpret_cast<uintptr_t>(keys) | reinterpret_cast<uintptr_t>(in) |
                         reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (inclusive)
        LCPP_LAUNCH("scan_by_key_inclusive", s,
                    (scan_by_key_kernel<K, V, Op, true><<<(uint32_t)tiles, kBkBlock, 0, s>>>(keys, in, out, n, words,
                                                                                            init, vec_ok, ctl)));
    else
        LCPP_LAUNCH("scan_by_key_exclusive", s,
                    (scan_by_key_kernel<K, V, Op, false><<<(uint32_t)tiles, kBkBlock, 0, s>>>(keys, in, out, n, words,
                                                                                             init, vec_ok, ctl)));
    LCPP_CHECK_LAUNCH();
    return LCPP_OK;
}

// Keys only matter through equality: integer keys compare their bits,
// floating keys compare as floats (-0.0 == +0.0, NaN != NaN).
template <class V, class Op>
int sbk_keys(bool inc, lcpp_dtype kt, void *temp, size_t tb, const void *k, const void *in, void *out, uint64_t n,
             const void *init, hipStream_t s)
{
    switch (kt) {
    case LCPP_INT32: case LCPP_UINT32: return sbk_launch<uint32_t, V, Op>(inc, temp, tb, k, in, out, n, init, s);
    case LCPP_INT64: case LCPP_UINT64: return sbk_launch<uint64_t, V, Op>(inc, temp, tb, k, in, out, n, init, s);
    case LCPP_FLOAT32: return sbk_launch<float, V, Op>(inc, temp, tb, k, in, out, n, init, s);
    case LCPP_FLOAT64: return sbk_launch<double, V, Op>(inc, temp, tb, k, in, out, n, init, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

template <class V>
int sbk_op(bool inc, lcpp_dtype kt, lcpp_reduce_op op, void *temp, size_t tb, const void *k, const void *in,
           void *out, uint64_t n, const void *init, hipStream_t s)
{
    switch (op) {
    case LCPP_OP_SUM: return sbk_keys<V, SumOp>(inc, kt, temp, tb, k, in, out, n, init, s);
    case LCPP_OP_MIN: return sbk_keys<V, MinOp>(inc, kt, temp, tb, k, in, out, n, init, s);
    case LCPP_OP_MAX: return sbk_keys<V, MaxOp>(inc, kt, temp, tb, k, in, out, n, init, s);
    default: return LCPP_ERR_INVALID_ARG;
    }
}

int sbk_dispatch(bool inc, lcpp_dtype kt, lcpp_dtype vt, lcpp_reduce_op op, void *temp, size_t tb,
                 const void *k, const void *in, void *out, uint64_t n, const void *init, void *stream)
{
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (vt) {
    case LCPP_INT32: return sbk_op<int32_t>(inc, kt, op, temp, tb, k, in, out, n, init, s);
    case LCPP_UINT32: return sbk_op<uint32_t>(inc, kt, op, temp, tb, k, in, out, n, init, s);
    case LCPP_FLOAT32: return sbk_op<float>(inc, kt, op, temp, tb, k, in, out, n, init, s);
    case LCPP_INT64: return sbk_op<int64_t>(inc, kt, op, temp, tb, k, in, out, n, init, s);
    case LCPP_UINT64: return sbk_op<uint64_t>(inc, kt, op, temp, tb, k, in, out, n, init, s);
    case LCPP_FLOAT64: return sbk_op<double>(inc, kt, op, temp, tb, k, in, out, n, init, s);
    default: return LCPP_ERR_UNSUPPORTED_DTYPE;
    }
}

bool valid_dtype(lcpp_dtype t) { return t >= LCPP_INT32 && t <= LCPP_FLOAT64; }

}  // namespace
}  // namespace lcpp

using namespace lcpp;

extern "C" int lcpp_scan_by_key_temp_bytes(lcpp_dtype k, lcpp_dtype v, uint64_t n, size_t *bytes)
{
    if (!bytes) return LCPP_ERR_INVALID_ARG;
    if (!valid_dtype(k) || !valid_dtype(v)) return LCPP_ERR_UNSUPPORTED_DTYPE;
    const bool wide = v == LCPP_INT64 || v == LCPP_UINT64 || v == LCPP_FLOAT64;
    if ((wide ? bk_tiles<uint64_t>(n) : bk_tiles<uint32_t>(n)) > 0xFFFFFFFFull) return LCPP_ERR_INVALID_ARG;
    *bytes = wide ? sbk_temp_bytes<uint64_t>(n) : sbk_temp_bytes<uint32_t>(n);
    return LCPP_OK;
}

extern "C" int lcpp_scan_exclusive_by_key(lcpp_dtype k, lcpp_dtype v, lcpp_reduce_op op, void *temp,
                                          size_t temp_bytes, const void *keys_in, const void *vals_in,
                                          void *vals_out, uint64_t n, const void *init, void *stream)
{
    return sbk_dispatch(false, k, v, op, temp, temp_bytes, keys_in, vals_in, vals_out, n, init, stream);
}

extern "C" int lcpp_scan_inclusive_by_key(lcpp_dtype k, lcpp_dtype v, lcpp_reduce_op op, void *temp,
                                          size_t temp_bytes, const void *keys_in, const void *vals_in,
                                          void *vals_out, uint64_t n, const void *init, void *stream)
{
    return sbk_dispatch(true, k, v, op, temp, temp_bytes, keys_in, vals_in, vals_out, n, init, stream);
}

extern "C" int lcpp_scan_exclusive_sum_by_key(lcpp_dtype k, lcpp_dtype v, void *temp, size_t temp_bytes,
                                              const void *keys_in, const void *vals_in, void *vals_out,
                                              uint64_t n, void *stream)
{
    return sbk_dispatch(false, k, v, LCPP_OP_SUM, temp, temp_bytes, keys_in, vals_in, vals_out, n, nullptr, stream);
}

extern "C" int lcpp_scan_inclusive_sum_by_key(lcpp_dtype k, lcpp_dtype v, void *temp, size_t temp_bytes,
                                              const void *keys_in, const void *vals_in, void *vals_out,
                                              uint64_t n, void *stream)
{
    return sbk_dispatch(true, k, v, LCPP_OP_SUM, temp, temp_bytes, keys_in, vals_in, vals_out, n, nullptr, stream);
}
