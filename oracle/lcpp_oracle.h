/*
 * lcpp_oracle.h — CPU restatement of LCPP's device-level primitives.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library (the HIP
 * kernels, the C ABI, the C++ host API) may call, link or load this code.
 * It is used by tests/ as the parity checker, by __graft_entry__.smoke() as
 * the checker of the smoke run, and by bench.py's cpu_baseline leg as the
 * timed "reference CPU path" stand-in (the reference's LuisaCompute CPU
 * backend cannot be built: LuisaCompute is not vendored).
 *
 * Each function cites the reference file:line it restates (paths relative
 * to the reference root, src/lcpp/...).  Integer results are exact
 * (two's-complement wraparound, as the GPU computes them); floating-point
 * results are provided in double precision together with the sum of
 * absolute values so callers can apply the normwise tolerance
 * |err| <= rtol * sum|x|.
 *
 * Pinning (what each function is checked against, in tests/test_oracle.py):
 *   generators      splitmix64 published test vector (Vigna, seed 1234567)
 *   reduce          Python big-int closed form, numpy min/max, reference KATs
 *                   (N ones -> N; shuffled 0..4095 -> 0 / 4095)
 *   arg reduce      numpy argmin (first index) and reversed argmax (last
 *                   index), reference KAT (shuffled 0..4095 -> positions of
 *                   0 and 4095)
 *   transform       numpy transforms + reductions in the element type,
 *                   reference KAT (max of squares of shuffled 0..4095)
 *   scan            numpy cumsum in the element type (wraparound), KATs
 *                   (ones -> i / i+1), look-back KAT (102400 tiles)
 *   scan with op    numpy cumsum / minimum.accumulate / maximum.accumulate
 *                   with init prepended, init = identity == the Sum scan,
 *                   constant input closed forms, planted mistakes
 *   radix sort      numpy stable argsort/sort, reversed-keys KAT, float KAT
 *                   (libstdc++ mt19937 inputs, std::sort golden), stability
 *                   checker (planted-mistake tests)
 *   segment reduce  numpy per-segment sums / min / max (with init), numpy
 *                   argmin / reversed argmax per segment, reference KATs
 *                   (1024 shuffled ints in segments of 100: sums and ArgMax;
 *                   0..1023 in fixed segments of 32: sums; shuffled, fixed 32:
 *                   ArgMin)
 *   scan by key     numpy cumsum differences inside runs (wraparound), single
 *                   run == plain scan, all-distinct keys == init / op(x, init),
 *                   reference KAT (keys i/100, ones -> i % 100)
 *   reduce by key   numpy add/minimum/maximum.reduceat over run heads, run
 *                   count from np.diff, reference KAT (keys i/100 over the
 *                   shuffled 0..4095 golden -> chunk sums)
 */
#ifndef LCPP_ORACLE_H
#define LCPP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: identical to lcpp_dtype in include/lcpp_amd.h */
enum {
    LCOR_I32 = 0,
    LCOR_U32 = 1,
    LCOR_F32 = 2,
    LCOR_I64 = 3,
    LCOR_U64 = 4,
    LCOR_F64 = 5
};

enum { LCOR_OP_SUM = 0, LCOR_OP_MIN = 1, LCOR_OP_MAX = 2 };

/* ---------------- synthetic inputs (counter-based splitmix64) ---------- */
uint64_t lcor_splitmix64_next(uint64_t *state);
uint64_t lcor_word(uint64_t seed, uint64_t i);
void lcor_gen_words(uint64_t seed, uint64_t start, uint64_t n, uint64_t *out);
void lcor_gen_reduce_i32(uint64_t seed, uint64_t n, int32_t *out);
void lcor_gen_u8_u32(uint64_t seed, uint64_t n, uint32_t *out);
void lcor_gen_normal_f32(uint64_t seed, uint64_t n, float *out);
void lcor_gen_keys_u32(uint64_t seed, uint64_t n, uint32_t *out);
void lcor_gen_keys_u32_and3(uint64_t sa, uint64_t sb, uint64_t sc, uint64_t n, uint32_t *out);
void lcor_gen_keys_u64_low16(uint64_t seed, uint64_t n, uint64_t *out);
void lcor_gen_iota_u32(uint64_t n, uint32_t *out);
int lcor_gen_segments(uint64_t seed_empty, uint64_t seed_len, uint64_t n_items,
                      uint64_t n_segments, uint32_t *begin, uint32_t *end);

/* ---------------- reduce ----------------------------------------------- */
int lcor_reduce(int op, int dtype, const void *in, uint64_t n, void *out);
int lcor_reduce_f64(int dtype, const void *in, uint64_t n, double *sum, double *abs_sum);
int lcor_reduce_mt(int op, int dtype, const void *in, uint64_t n, void *out, int nthreads);
/* ArgMin (is_max = 0) / ArgMax (is_max = 1): value and 32-bit index */
int lcor_reduce_arg(int is_max, int dtype, const void *in, uint64_t n, void *out_value, uint32_t *out_index);
/* TransformReduce: out = op(init, op over i of xf(in[i])); xf 0 identity, 1 negate, 2 abs, 3 square */
int lcor_reduce_transform(int op, int xf, int dtype, const void *in, uint64_t n, const void *init, void *out);

/* ---------------- scan ------------------------------------------------- */
int lcor_scan(int inclusive, int dtype, const void *in, void *out, uint64_t n);
int lcor_scan_op(int inclusive, int op, int dtype, const void *in, void *out, uint64_t n, const void *init);
int lcor_scan_f64(int inclusive, int dtype, const void *in, double *out, double *abs_prefix,
                  uint64_t n);
int lcor_scan_mt(int inclusive, int dtype, const void *in, void *out, uint64_t n, int nthreads);
int lcor_lookback_kat(uint32_t num_tiles, int nthreads, int32_t *excl, int32_t *incl);
/* Look-back over per-tile aggregates with bounded waits (windows of `width`
 * predecessors, give-up after `spin_limit` re-polls, tile `withhold` never
 * publishes; UINT32_MAX withholds none).  *status gets bit 0 if a wait gave up. */
int lcor_lookback_bounded(const int32_t *agg, uint32_t num_tiles, int nthreads, uint32_t withhold,
                          uint32_t spin_limit, uint32_t width, int32_t *excl, int32_t *incl, uint32_t *status);

/* ---------------- radix sort (onesweep restatement) -------------------- */
int lcor_radix_sort(int key_dtype, int val_bytes, const void *keys_in, void *keys_out,
                    const void *vals_in, void *vals_out, uint64_t n, int descending,
                    int nthreads, uint32_t tile_items);
/* 1 if (keys_out, vals_out) is the stable ascending sort of keys_in with
 * vals_in[i] == i (u32 values), checked in O(n) without sorting. */
int lcor_check_stable_pairs_u64_u32(const uint64_t *keys_in, const uint64_t *keys_out,
                                    const uint32_t *vals_out, uint64_t n);
int lcor_check_sorted_permutation_u32(const uint32_t *keys_in, const uint32_t *keys_out,
                                      uint64_t n);

/* ---------------- scan by key / reduce by key -------------------------- */
/* heads: i == 0 or keys[i] != keys[i-1] (compared in the key type) */
int lcor_scan_by_key(int inclusive, int op, int key_dtype, int val_dtype, const void *keys,
                     const void *vals, void *out, uint64_t n, const void *init);
int lcor_scan_by_key_f64(int inclusive, int key_dtype, int val_dtype, const void *keys,
                         const void *vals, double *out, double *abs_prefix, uint64_t n);
int lcor_reduce_by_key(int op, int key_dtype, int val_dtype, const void *keys, const void *vals,
                       void *unique_out, void *aggregates_out, uint64_t n, uint64_t *num_runs);
int lcor_reduce_by_key_f64(int key_dtype, int val_dtype, const void *keys, const void *vals,
                           uint64_t n, double *sums, double *abs_sums, uint64_t *num_runs);

/* ---------------- segment reduce -------------------------------------- */
/* out[s] = op(init, fold(in[begin[s] .. end[s]))); init NULL means the op's identity */
int lcor_segment_reduce(int op, int dtype, const void *in, void *out, uint64_t num_segments,
                        const uint32_t *begin, const uint32_t *end, const void *init);
/* ArgMin (is_max 0) / ArgMax (is_max 1) per segment, index relative to begin[s];
 * an empty segment gives (1, max()) / (1, lowest()) */
int lcor_segment_reduce_arg(int is_max, int dtype, const void *in, void *out, uint32_t *index_out,
                            uint64_t num_segments, const uint32_t *begin, const uint32_t *end);
int lcor_segment_reduce_f64(int dtype, const void *in, uint64_t num_segments,
                            const uint32_t *begin, const uint32_t *end, double *sum,
                            double *abs_sum);
int lcor_segment_reduce_mt(int dtype, const void *in, void *out, uint64_t num_segments,
                           const uint32_t *begin, const uint32_t *end, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
