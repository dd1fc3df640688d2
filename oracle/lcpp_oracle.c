/*
 * lcpp_oracle.c — CPU restatement of LCPP's device-level primitives.
 *
 * TEST INFRASTRUCTURE ONLY (see lcpp_oracle.h).  Never linked into the
 * shipped library.  Reference paths are relative to src/lcpp/ of the
 * reference tree.
 */
#define _GNU_SOURCE
#include "lcpp_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 * Synthetic inputs.  Counter-based splitmix64 (Vigna, public domain):
 *   w_i = mix(seed + (i + 1) * 0x9E3779B97F4A7C15)
 * which equals the i-th output of the sequential splitmix64 generator
 * started from state `seed`.
 * ====================================================================== */
#define GOLDEN_GAMMA 0x9E3779B97F4A7C15ull

static inline uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t lcor_splitmix64_next(uint64_t *state)
{
    *state += GOLDEN_GAMMA;
    return mix64(*state);
}

uint64_t lcor_word(uint64_t seed, uint64_t i) { return mix64(seed + (i + 1) * GOLDEN_GAMMA); }

void lcor_gen_words(uint64_t seed, uint64_t start, uint64_t n, uint64_t *out)
{
    for (uint64_t i = 0; i < n; ++i) out[i] = lcor_word(seed, start + i);
}

/* a_i = -1000 + floor(hi32(w_i) * 2001 / 2^32): uniform in [-1000, 1000] */
void lcor_gen_reduce_i32(uint64_t seed, uint64_t n, int32_t *out)
{
    for (uint64_t i = 0; i < n; ++i) {
        uint64_t hi = lcor_word(seed, i) >> 32;
        out[i] = (int32_t)((hi * 2001ull) >> 32) - 1000;
    }
}

/* x_i = hi32(w_i) >> 24: uniform in [0, 255] */
void lcor_gen_u8_u32(uint64_t seed, uint64_t n, uint32_t *out)
{
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint32_t)(lcor_word(seed, i) >> 56);
}

/* Box-Muller (cos branch) in double from words 2i and 2i+1, cast to f32. */
void lcor_gen_normal_f32(uint64_t seed, uint64_t n, float *out)
{
    const double two_pi = 6.283185307179586476925286766559;
    const double inv53 = 1.0 / 9007199254740992.0; /* 2^-53 */
    for (uint64_t i = 0; i < n; ++i) {
        double u1 = (double)((lcor_word(seed, 2 * i) >> 11) + 1) * inv53; /* (0, 1] */
        double u2 = (double)(lcor_word(seed, 2 * i + 1) >> 11) * inv53;   /* [0, 1) */
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(two_pi * u2));
    }
}

void lcor_gen_keys_u32(uint64_t seed, uint64_t n, uint32_t *out)
{
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint32_t)lcor_word(seed, i);
}

void lcor_gen_keys_u32_and3(uint64_t sa, uint64_t sb, uint64_t sc, uint64_t n, uint32_t *out)
{
    for (uint64_t i = 0; i < n; ++i)
        out[i] = (uint32_t)lcor_word(sa, i) & (uint32_t)lcor_word(sb, i) &
                 (uint32_t)lcor_word(sc, i);
}

void lcor_gen_keys_u64_low16(uint64_t seed, uint64_t n, uint64_t *out)
{
    for (uint64_t i = 0; i < n; ++i) out[i] = lcor_word(seed, i) & 0xFFFFull;
}

void lcor_gen_iota_u32(uint64_t n, uint32_t *out)
{
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint32_t)i;
}

/* CSR segments: L_s = 0 with p = 0.05 (stream seed_empty), otherwise
 * geometric on {1,2,...} with mean 128/0.95 (stream seed_len).  Cumulative
 * offsets C are rescaled so the total is exactly n_items:
 * off[s] = floor(C[s] * n_items / C[S]); begin[s] = off[s], end[s] = off[s+1]. */
int lcor_gen_segments(uint64_t seed_empty, uint64_t seed_len, uint64_t n_items,
                      uint64_t n_segments, uint32_t *begin, uint32_t *end)
{
    if (n_segments == 0) return 0;
    if (n_items > 0xFFFFFFFFull) return -1;
    const double inv53 = 1.0 / 9007199254740992.0;
    const double p = 0.95 / 128.0;
    const double log1mp = log1p(-p);
    uint64_t *c = (uint64_t *)malloc((n_segments + 1) * sizeof(uint64_t));
    if (!c) return -1;
    c[0] = 0;
    for (uint64_t s = 0; s < n_segments; ++s) {
        double ue = (double)(lcor_word(seed_empty, s) >> 11) * inv53;
        uint64_t len = 0;
        if (ue >= 0.05) {
            double ul = (double)((lcor_word(seed_len, s) >> 11) + 1) * inv53; /* (0,1] */
            len = 1 + (uint64_t)floor(log(ul) / log1mp);
        }
        c[s + 1] = c[s] + len;
    }
    uint64_t total = c[n_segments];
    for (uint64_t s = 0; s <= n_segments; ++s) {
        uint64_t off =
            total ? (uint64_t)(((unsigned __int128)c[s] * n_items) / total) : (s ? n_items : 0);
        if (s < n_segments) begin[s] = (uint32_t)off;
        if (s > 0) end[s - 1] = (uint32_t)off;
    }
    free(c);
    return 0;
}

/* ======================================================================
 * Element-type helpers
 * ====================================================================== */
static size_t dtype_size(int dt)
{
    switch (dt) {
    case LCOR_I32: case LCOR_U32: case LCOR_F32: return 4;
    case LCOR_I64: case LCOR_U64: case LCOR_F64: return 8;
    default: return 0;
    }
}

/* Fold `n` elements of `in` into `acc` (same type) with op.  Integer sums
 * wrap (two's complement); Min/Max use the identities of
 * device/device_reduce.h:169-185 (Max uses lowest(), not min(): the
 * reference's numeric_limits<float>::min() init is a known divergence). */
#define DEFINE_FOLD(NAME, T, UT)                                                            \
    static T NAME(int op, const T *in, uint64_t n, T acc)                                 \
    {                                                                                      \
        if (op == LCOR_OP_SUM) {                                                           \
            for (uint64_t i = 0; i < n; ++i) acc = (T)((UT)acc + (UT)in[i]);               \
        } else if (op == LCOR_OP_MIN) {                                                    \
            for (uint64_t i = 0; i < n; ++i) acc = in[i] < acc ? in[i] : acc;              \
        } else {                                                                           \
            for (uint64_t i = 0; i < n; ++i) acc = in[i] > acc ? in[i] : acc;              \
        }                                                                                  \
        return acc;                                                                        \
    }
DEFINE_FOLD(fold_i32, int32_t, uint32_t)
DEFINE_FOLD(fold_u32, uint32_t, uint32_t)
DEFINE_FOLD(fold_f32, float, float)
DEFINE_FOLD(fold_i64, int64_t, uint64_t)
DEFINE_FOLD(fold_u64, uint64_t, uint64_t)
DEFINE_FOLD(fold_f64, double, double)

/* init values: Sum 0, Min max(), Max lowest() */
static void init_value(int op, int dt, void *out)
{
    switch (dt) {
    case LCOR_I32: *(int32_t *)out = op == LCOR_OP_SUM ? 0 : op == LCOR_OP_MIN ? INT32_MAX : INT32_MIN; break;
    case LCOR_U32: *(uint32_t *)out = op == LCOR_OP_SUM ? 0 : op == LCOR_OP_MIN ? UINT32_MAX : 0; break;
    case LCOR_F32: *(float *)out = op == LCOR_OP_SUM ? 0.0f : op == LCOR_OP_MIN ? 3.402823466e38f : -3.402823466e38f; break;
    case LCOR_I64: *(int64_t *)out = op == LCOR_OP_SUM ? 0 : op == LCOR_OP_MIN ? INT64_MAX : INT64_MIN; break;
    case LCOR_U64: *(uint64_t *)out = op == LCOR_OP_SUM ? 0 : op == LCOR_OP_MIN ? UINT64_MAX : 0; break;
    case LCOR_F64: *(double *)out = op == LCOR_OP_SUM ? 0.0 : op == LCOR_OP_MIN ? 1.7976931348623157e308 : -1.7976931348623157e308; break;
    }
}

static void fold_any(int op, int dt, const void *in, uint64_t n, void *acc)
{
    switch (dt) {
    case LCOR_I32: *(int32_t *)acc = fold_i32(op, (const int32_t *)in, n, *(int32_t *)acc); break;
    case LCOR_U32: *(uint32_t *)acc = fold_u32(op, (const uint32_t *)in, n, *(uint32_t *)acc); break;
    case LCOR_F32: *(float *)acc = fold_f32(op, (const float *)in, n, *(float *)acc); break;
    case LCOR_I64: *(int64_t *)acc = fold_i64(op, (const int64_t *)in, n, *(int64_t *)acc); break;
    case LCOR_U64: *(uint64_t *)acc = fold_u64(op, (const uint64_t *)in, n, *(uint64_t *)acc); break;
    case LCOR_F64: *(double *)acc = fold_f64(op, (const double *)in, n, *(double *)acc); break;
    }
}

/* ======================================================================
 * Reduce — device/device_reduce.h:131-185 (Sum/Min/Max = Reduce with
 * SumOp/MinOp/MaxOp and the init above).  The reference splits the input
 * into 1024-item tiles over a capped grid (device/device_reduce.h:396-460,
 * common/grid_even_shared.h:33-99), folds per thread then per block; for
 * integers every order gives the same bits, so the checker folds
 * sequentially.  Floating-point sums are checked in double precision.
 * ====================================================================== */
int lcor_reduce(int op, int dtype, const void *in, uint64_t n, void *out)
{
    if (!dtype_size(dtype) || op < 0 || op > 2) return -1;
    if (dtype == LCOR_F32 && op == LCOR_OP_SUM) {
        double s, a;
        lcor_reduce_f64(dtype, in, n, &s, &a);
        *(float *)out = (float)s;
        return 0;
    }
    init_value(op, dtype, out);
    fold_any(op, dtype, in, n, out);
    return 0;
}

int lcor_reduce_f64(int dtype, const void *in, uint64_t n, double *sum, double *abs_sum)
{
    double s = 0.0, a = 0.0, c = 0.0; /* Kahan-compensated double sum */
    for (uint64_t i = 0; i < n; ++i) {
        double x;
        switch (dtype) {
        case LCOR_F32: x = ((const float *)in)[i]; break;
        case LCOR_F64: x = ((const double *)in)[i]; break;
        case LCOR_I32: x = ((const int32_t *)in)[i]; break;
        case LCOR_U32: x = ((const uint32_t *)in)[i]; break;
        case LCOR_I64: x = (double)((const int64_t *)in)[i]; break;
        case LCOR_U64: x = (double)((const uint64_t *)in)[i]; break;
        default: return -1;
        }
        double y = x - c;
        double t = s + y;
        c = (t - s) - y;
        s = t;
        a += fabs(x);
    }
    *sum = s;
    *abs_sum = a;
    return 0;
}

/* ======================================================================
 * ArgMin / ArgMax — device/device_reduce.h:187-272 with ArgMinOp / ArgMaxOp
 * (common/thread_operators.h:19-47): the running pair (value, index) is
 * replaced by element i when its value is smaller (ArgMin) / larger (ArgMax),
 * or equal with a smaller (ArgMin) / larger (ArgMax) index.  Init is
 * (numeric max, 0xFFFFFFFF) for ArgMin (device_reduce.h:222-223) and
 * (numeric lowest, 0) for ArgMax; the reference's ArgMax init is
 * numeric_limits::min() (device_reduce.h:267), which differs from lowest()
 * for floating point only (the GPU build uses lowest(), as the checker).
 * ====================================================================== */
#define ARG_FOLD(T, MAXV, LOWV)                                                        \
    do {                                                                               \
        const T *a = (const T *)in;                                                    \
        T v = is_max ? (LOWV) : (MAXV);                                                \
        uint32_t ix = is_max ? 0u : 0xFFFFFFFFu;                                       \
        for (uint64_t i = 0; i < n; ++i) {                                             \
            const T x = a[i];                                                          \
            const uint32_t xi = (uint32_t)i;                                           \
            const int take = is_max ? (x > v || (x == v && xi > ix))                   \
                                    : (x < v || (x == v && xi < ix));                  \
            if (take) { v = x; ix = xi; }                                              \
        }                                                                              \
        *(T *)out_value = v;                                                           \
        *out_index = ix;                                                               \
    } while (0)

int lcor_reduce_arg(int is_max, int dtype, const void *in, uint64_t n, void *out_value, uint32_t *out_index)
{
    if (n > 0xFFFFFFFFull) return -1;
    switch (dtype) {
    case LCOR_I32: ARG_FOLD(int32_t, INT32_MAX, INT32_MIN); break;
    case LCOR_U32: ARG_FOLD(uint32_t, UINT32_MAX, 0u); break;
    case LCOR_F32: ARG_FOLD(float, 3.402823466e38f, -3.402823466e38f); break;
    case LCOR_I64: ARG_FOLD(int64_t, INT64_MAX, INT64_MIN); break;
    case LCOR_U64: ARG_FOLD(uint64_t, UINT64_MAX, 0u); break;
    case LCOR_F64: ARG_FOLD(double, 1.7976931348623157e308, -1.7976931348623157e308); break;
    default: return -1;
    }
    return 0;
}

/* ======================================================================
 * TransformReduce — device/device_reduce.h:331-348 (reduce_array_recursive
 * with a transform applied to every loaded item and `init` folded in):
 * out = op(init, op over i of xf(in[i])), folded sequentially.  Integer
 * transforms wrap (two's complement); |INT_MIN| = INT_MIN.
 * ====================================================================== */
#define XF_INT(T, U, SIGNED)                                                           \
    static T xf_##T(int xf, T x)                                                       \
    {                                                                                  \
        switch (xf) {                                                                  \
        case 1: return (T)((U)0 - (U)x);                                               \
        case 2: return (SIGNED && ((U)x >> (sizeof(U) * 8 - 1))) ? (T)((U)0 - (U)x) : x; \
        case 3: return (T)((U)x * (U)x);                                               \
        default: return x;                                                             \
        }                                                                              \
    }
XF_INT(int32_t, uint32_t, 1)
XF_INT(uint32_t, uint32_t, 0)
XF_INT(int64_t, uint64_t, 1)
XF_INT(uint64_t, uint64_t, 0)
static float xf_float(int xf, float x) { return xf == 1 ? -x : xf == 2 ? fabsf(x) : xf == 3 ? x * x : x; }
static double xf_double(int xf, double x) { return xf == 1 ? -x : xf == 2 ? fabs(x) : xf == 3 ? x * x : x; }

#define XFOLD(T, XFN, FOLD1)                                                           \
    do {                                                                               \
        const T *a = (const T *)in;                                                    \
        T acc;                                                                         \
        init_value(op, dtype, &acc);                                                   \
        for (uint64_t i = 0; i < n; ++i) {                                             \
            const T x = XFN(xf, a[i]);                                                 \
            acc = FOLD1(op, &x, 1, acc);                                               \
        }                                                                              \
        const T iv = *(const T *)init;                                                 \
        *(T *)out = FOLD1(op, &acc, 1, iv);                                            \
    } while (0)

int lcor_reduce_transform(int op, int xf, int dtype, const void *in, uint64_t n, const void *init, void *out)
{
    if (op < 0 || op > 2 || xf < 0 || xf > 3 || !init) return -1;
    switch (dtype) {
    case LCOR_I32: XFOLD(int32_t, xf_int32_t, fold_i32); break;
    case LCOR_U32: XFOLD(uint32_t, xf_uint32_t, fold_u32); break;
    case LCOR_F32: XFOLD(float, xf_float, fold_f32); break;
    case LCOR_I64: XFOLD(int64_t, xf_int64_t, fold_i64); break;
    case LCOR_U64: XFOLD(uint64_t, xf_uint64_t, fold_u64); break;
    case LCOR_F64: XFOLD(double, xf_double, fold_f64); break;
    default: return -1;
    }
    return 0;
}

/* ---------------- multithreaded reduce (CPU baseline) ----------------- */
typedef struct {
    int op, dtype;
    const char *in;
    uint64_t begin, end;
    uint64_t acc[1];
} reduce_job;

static void *reduce_worker(void *p)
{
    reduce_job *j = (reduce_job *)p;
    size_t es = dtype_size(j->dtype);
    init_value(j->op, j->dtype, j->acc);
    fold_any(j->op, j->dtype, j->in + j->begin * es, j->end - j->begin, j->acc);
    return NULL;
}

int lcor_reduce_mt(int op, int dtype, const void *in, uint64_t n, void *out, int nthreads)
{
    if (!dtype_size(dtype) || nthreads < 1) return -1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    reduce_job jobs[256];
    for (int t = 0; t < nthreads; ++t) {
        jobs[t].op = op;
        jobs[t].dtype = dtype;
        jobs[t].in = (const char *)in;
        jobs[t].begin = n * (uint64_t)t / (uint64_t)nthreads;
        jobs[t].end = n * (uint64_t)(t + 1) / (uint64_t)nthreads;
        pthread_create(&th[t], NULL, reduce_worker, &jobs[t]);
    }
    init_value(op, dtype, out);
    for (int t = 0; t < nthreads; ++t) {
        pthread_join(th[t], NULL);
        fold_any(op, dtype, jobs[t].acc, 1, out);
    }
    return 0;
}

/* ======================================================================
 * Scan — device/device_scan.h:180-204 (ExclusiveSum/InclusiveSum = scan
 * with a+b and init 0).  out_i = sum_{j<i} x_j (exclusive) or
 * sum_{j<=i} x_j (inclusive), integer arithmetic wrapping in the type.
 * ====================================================================== */
#define DEFINE_SCAN(NAME, T, UT)                                                             \
    static void NAME(int inclusive, const T *in, T *out, uint64_t n, T carry)                \
    {                                                                                       \
        for (uint64_t i = 0; i < n; ++i) {                                                  \
            T x = in[i];                                                                    \
            if (inclusive) { carry = (T)((UT)carry + (UT)x); out[i] = carry; }              \
            else { out[i] = carry; carry = (T)((UT)carry + (UT)x); }                        \
        }                                                                                   \
    }
DEFINE_SCAN(scan_i32, int32_t, uint32_t)
DEFINE_SCAN(scan_u32, uint32_t, uint32_t)
DEFINE_SCAN(scan_f32, float, float)
DEFINE_SCAN(scan_i64, int64_t, uint64_t)
DEFINE_SCAN(scan_u64, uint64_t, uint64_t)
DEFINE_SCAN(scan_f64, double, double)

static void scan_any(int inclusive, int dt, const void *in, void *out, uint64_t n, const void *carry)
{
    switch (dt) {
    case LCOR_I32: scan_i32(inclusive, in, out, n, *(const int32_t *)carry); break;
    case LCOR_U32: scan_u32(inclusive, in, out, n, *(const uint32_t *)carry); break;
    case LCOR_F32: scan_f32(inclusive, in, out, n, *(const float *)carry); break;
    case LCOR_I64: scan_i64(inclusive, in, out, n, *(const int64_t *)carry); break;
    case LCOR_U64: scan_u64(inclusive, in, out, n, *(const uint64_t *)carry); break;
    case LCOR_F64: scan_f64(inclusive, in, out, n, *(const double *)carry); break;
    }
}

int lcor_scan(int inclusive, int dtype, const void *in, void *out, uint64_t n)
{
    if (!dtype_size(dtype)) return -1;
    uint64_t zero = 0;
    scan_any(inclusive, dtype, in, out, n, &zero);
    return 0;
}

/* DeviceScan::ExclusiveScan / InclusiveScan (device/device_scan.h:114-178)
 * with scan_op Sum/Min/Max and initial_value, as CUB defines them: a left
 * fold that starts from init, out_i = op(init, x_0, ..., x_{i-1}) (exclusive)
 * or op(init, x_0, ..., x_i) (inclusive).  Integer sums wrap; Min/Max use the
 * comparisons of fold_any.  init NULL = the op's identity.  (The reference's
 * first tile folds initial_value in once per warp, block_scan_warp.h:223-236;
 * the two agree whenever init is the op's identity or the op is Min/Max.) */
int lcor_scan_op(int inclusive, int op, int dtype, const void *in, void *out, uint64_t n, const void *init)
{
    const size_t es = dtype_size(dtype);
    if (!es || op < 0 || op > 2) return -1;
    uint64_t carry = 0;
    if (init) memcpy(&carry, init, es);
    else init_value(op, dtype, &carry);
    for (uint64_t i = 0; i < n; ++i) {
        const char *x = (const char *)in + i * es;
        char *o = (char *)out + i * es;
        if (!inclusive) memcpy(o, &carry, es);
        fold_any(op, dtype, x, 1, &carry);
        if (inclusive) memcpy(o, &carry, es);
    }
    return 0;
}

int lcor_scan_f64(int inclusive, int dtype, const void *in, double *out, double *abs_prefix,
                  uint64_t n)
{
    if (dtype != LCOR_F32 && dtype != LCOR_F64) return -1;
    double s = 0.0, a = 0.0, c = 0.0;
    for (uint64_t i = 0; i < n; ++i) {
        double x;
        switch (dtype) {
        case LCOR_F32: x = ((const float *)in)[i]; break;
        case LCOR_F64: x = ((const double *)in)[i]; break;
        default: return -1;
        }
        if (!inclusive) { out[i] = s; abs_prefix[i] = a; }
        double y = x - c;
        double t = s + y;
        c = (t - s) - y;
        s = t;
        a += fabs(x);
        if (inclusive) { out[i] = s; abs_prefix[i] = a; }
    }
    return 0;
}

/* ---------------- decoupled look-back across threads ------------------
 * Restates device/details/single_pass_scan_operator.h:60-251: each tile
 * publishes PARTIAL(aggregate), walks back over its predecessors summing
 * PARTIAL values until it meets an INCLUSIVE one, then publishes
 * INCLUSIVE(prefix + aggregate).  Status and value live in one 64-bit word
 * (value << 32 | status) stored with release and loaded with acquire
 * semantics, which removes the value/status ordering gap of the reference's
 * separate arrays (single_pass_scan_operator.h:81-93). */
enum { LB_INVALID = 0, LB_PARTIAL = 1, LB_INCLUSIVE = 2 };

typedef struct {
    _Atomic uint64_t *words;
    _Atomic uint32_t ticket;
    uint32_t num_tiles;
    int32_t *excl, *incl;
} lbkat_ctx;

static int32_t lookback_i32(_Atomic uint64_t *words, uint32_t tile)
{
    int32_t prefix = 0;
    for (int64_t j = (int64_t)tile - 1; j >= 0; --j) {
        uint64_t w;
        do { w = atomic_load_explicit(&words[j], memory_order_acquire); } while ((w & 3u) == LB_INVALID);
        prefix = (int32_t)((uint32_t)prefix + (uint32_t)(w >> 32));
        if ((w & 3u) == LB_INCLUSIVE) break;
    }
    return prefix;
}

static void *lbkat_worker(void *p)
{
    lbkat_ctx *c = (lbkat_ctx *)p;
    for (;;) {
        uint32_t t = atomic_fetch_add_explicit(&c->ticket, 1, memory_order_relaxed);
        if (t >= c->num_tiles) break;
        const int32_t agg = 1;
        if (t == 0) {
            atomic_store_explicit(&c->words[0], ((uint64_t)(uint32_t)agg << 32) | LB_INCLUSIVE, memory_order_release);
            c->excl[0] = 0;
            c->incl[0] = agg;
            continue;
        }
        atomic_store_explicit(&c->words[t], ((uint64_t)(uint32_t)agg << 32) | LB_PARTIAL, memory_order_release);
        int32_t ex = lookback_i32(c->words, t);
        int32_t in = ex + agg;
        atomic_store_explicit(&c->words[t], ((uint64_t)(uint32_t)in << 32) | LB_INCLUSIVE, memory_order_release);
        c->excl[t] = ex;
        c->incl[t] = in;
    }
    return NULL;
}

int lcor_lookback_kat(uint32_t num_tiles, int nthreads, int32_t *excl, int32_t *incl)
{
    if (nthreads < 1) return -1;
    if (nthreads > 256) nthreads = 256;
    lbkat_ctx c;
    c.words = (_Atomic uint64_t *)calloc(num_tiles ? num_tiles : 1, sizeof(uint64_t));
    if (!c.words) return -1;
    atomic_init(&c.ticket, 0);
    c.num_tiles = num_tiles;
    c.excl = excl;
    c.incl = incl;
    pthread_t th[256];
    for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, lbkat_worker, &c);
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    free((void *)c.words);
    return 0;
}

/* ---------------- bounded look-back with a status word ----------------
 * The look-back above with this library's failure reporting instead of the
 * reference's unbounded wait (single_pass_scan_operator.h:96-104, 191-240:
 * WaitForValid spins while any polled predecessor is INVALID).  A wait polls
 * `width` predecessors at once (top, top-1, .., top-width+1; words below tile
 * 0 read as INCLUSIVE 0); the predecessors in range are those up to and
 * including the nearest INCLUSIVE one.  While one in range is INVALID the
 * wait re-polls the same window; after `spin_limit` re-polls it gives up:
 * it ORs LOOKBACK_TIMEOUT (bit 0) into *status and folds what has been
 * published (an unpublished word reads as 0).  Tile `withhold` never
 * publishes (the device library's test hook); every wait still ends.
 * Tiles take tickets in order, as workgroups are dispatched in id order.
 * Tile t's aggregate is agg[t]; excl/incl receive its prefixes (wrapping
 * int32 sums). */
#define LCOR_STATUS_LOOKBACK_TIMEOUT 1u
typedef struct {
    _Atomic uint64_t *words;
    _Atomic uint32_t ticket;
    _Atomic uint32_t *status;
    uint32_t num_tiles, withhold, spin_limit, width;
    const int32_t *agg;
    int32_t *excl, *incl;
} lbb_ctx;

static void lbb_publish(lbb_ctx *c, uint32_t t, int32_t v, uint32_t st)
{
    if (t == c->withhold) return;
    atomic_store_explicit(&c->words[t], ((uint64_t)(uint32_t)v << 32) | st, memory_order_release);
}

static int32_t lbb_wait(lbb_ctx *c, uint32_t tile)
{
    uint32_t excl = 0, spins = 0;
    int64_t top = (int64_t)tile - 1;
    for (;;) {
        uint32_t st[64], val[64], stop = c->width - 1;
        int found = 0, missing = 0;
        for (uint32_t l = 0; l < c->width; ++l) {
            const int64_t j = top - (int64_t)l;
            const uint64_t w = j < 0 ? LB_INCLUSIVE : atomic_load_explicit(&c->words[j], memory_order_acquire);
            st[l] = (uint32_t)(w & 3u);
            val[l] = (uint32_t)(w >> 32);
            if (st[l] == LB_INCLUSIVE && !found) { found = 1; stop = l; }
        }
        for (uint32_t l = 0; l <= stop; ++l) missing |= st[l] == LB_INVALID;
        if (missing) {
            if (++spins < c->spin_limit) { sched_yield(); continue; }
            atomic_fetch_or_explicit(c->status, LCOR_STATUS_LOOKBACK_TIMEOUT, memory_order_relaxed);
        }
        for (uint32_t l = 0; l <= stop; ++l) excl += val[l];
        if (found) return (int32_t)excl;
        top -= c->width;
    }
}

static void *lbb_worker(void *p)
{
    lbb_ctx *c = (lbb_ctx *)p;
    for (;;) {
        const uint32_t t = atomic_fetch_add_explicit(&c->ticket, 1, memory_order_relaxed);
        if (t >= c->num_tiles) break;
        const int32_t agg = c->agg[t];
        int32_t ex = 0;
        if (t == 0) {
            lbb_publish(c, 0, agg, LB_INCLUSIVE);
        } else {
            lbb_publish(c, t, agg, LB_PARTIAL);
            ex = lbb_wait(c, t);
            lbb_publish(c, t, (int32_t)((uint32_t)ex + (uint32_t)agg), LB_INCLUSIVE);
        }
        c->excl[t] = ex;
        c->incl[t] = (int32_t)((uint32_t)ex + (uint32_t)agg);
    }
    return NULL;
}

int lcor_lookback_bounded(const int32_t *agg, uint32_t num_tiles, int nthreads, uint32_t withhold,
                          uint32_t spin_limit, uint32_t width, int32_t *excl, int32_t *incl, uint32_t *status)
{
    if (nthreads < 1 || width < 1 || width > 64 || spin_limit < 1 || !status) return -1;
    if (nthreads > 256) nthreads = 256;
    lbb_ctx c;
    c.words = (_Atomic uint64_t *)calloc(num_tiles ? num_tiles : 1, sizeof(uint64_t));
    if (!c.words) return -1;
    _Atomic uint32_t st;
    atomic_init(&st, 0);
    atomic_init(&c.ticket, 0);
    c.status = &st;
    c.num_tiles = num_tiles;
    c.withhold = withhold;
    c.spin_limit = spin_limit;
    c.width = width;
    c.agg = agg;
    c.excl = excl;
    c.incl = incl;
    pthread_t th[256];
    int started = 0;
    for (; started < nthreads; ++started)
        if (pthread_create(&th[started], NULL, lbb_worker, &c) != 0) break;
    if (started == 0) lbb_worker(&c);
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
    free((void *)c.words);
    *status = atomic_load(&st);
    return 0;
}

/* ---------------- multithreaded single-pass scan (CPU baseline) -------
 * Same tile decomposition as the reference (device/details/scan.h:59-147):
 * tile = ticket, aggregate, look-back, then the tile's scan seeded with the
 * exclusive prefix.  Values are kept in the element type (wrapping for
 * integers). */
#define SCAN_MT_TILE 16384u
/* Sanitizer self-test: built with LCOR_PLANT_RELAXED_PUBLISH, the status
 * stores that publish a tile's values lose their release ordering, a planted
 * race that the TSan run must report (oracle/Makefile, tsan-planted). */
#ifdef LCOR_PLANT_RELAXED_PUBLISH
#define SCAN_MT_PUBLISH memory_order_relaxed
#else
#define SCAN_MT_PUBLISH memory_order_release
#endif
typedef struct {
    int inclusive, dtype;
    const char *in;
    char *out;
    uint64_t n;
    uint32_t num_tiles;
    _Atomic uint32_t ticket;
    _Atomic uint32_t *status;
    uint64_t *partial, *inclusive_v; /* raw bits of the element type */
} scan_mt_ctx;

static void *scan_mt_worker(void *p)
{
    scan_mt_ctx *c = (scan_mt_ctx *)p;
    size_t es = dtype_size(c->dtype);
    for (;;) {
        uint32_t t = atomic_fetch_add_explicit(&c->ticket, 1, memory_order_relaxed);
        if (t >= c->num_tiles) break;
        uint64_t b = (uint64_t)t * SCAN_MT_TILE;
        uint64_t e = b + SCAN_MT_TILE < c->n ? b + SCAN_MT_TILE : c->n;
        uint64_t agg = 0, prefix = 0;
        fold_any(LCOR_OP_SUM, c->dtype, c->in + b * es, e - b, &agg);
        if (t > 0) {
            c->partial[t] = agg;
            atomic_store_explicit(&c->status[t], LB_PARTIAL, SCAN_MT_PUBLISH);
            for (int64_t j = (int64_t)t - 1; j >= 0; --j) {
                uint32_t s;
                do { s = atomic_load_explicit(&c->status[j], memory_order_acquire); } while (s == LB_INVALID);
                uint64_t v = s == LB_INCLUSIVE ? c->inclusive_v[j] : c->partial[j];
                fold_any(LCOR_OP_SUM, c->dtype, &v, 1, &prefix);
                if (s == LB_INCLUSIVE) break;
            }
        }
        uint64_t inc = prefix;
        fold_any(LCOR_OP_SUM, c->dtype, &agg, 1, &inc);
        c->inclusive_v[t] = inc;
        atomic_store_explicit(&c->status[t], LB_INCLUSIVE, SCAN_MT_PUBLISH);
        scan_any(c->inclusive, c->dtype, c->in + b * es, c->out + b * es, e - b, &prefix);
    }
    return NULL;
}

int lcor_scan_mt(int inclusive, int dtype, const void *in, void *out, uint64_t n, int nthreads)
{
    if (!dtype_size(dtype) || nthreads < 1) return -1;
    if (nthreads > 256) nthreads = 256;
    scan_mt_ctx c;
    c.inclusive = inclusive;
    c.dtype = dtype;
    c.in = (const char *)in;
    c.out = (char *)out;
    c.n = n;
    c.num_tiles = (uint32_t)((n + SCAN_MT_TILE - 1) / SCAN_MT_TILE);
    atomic_init(&c.ticket, 0);
    size_t nt = c.num_tiles ? c.num_tiles : 1;
    c.status = (_Atomic uint32_t *)calloc(nt, sizeof(uint32_t));
    c.partial = (uint64_t *)calloc(nt, sizeof(uint64_t));
    c.inclusive_v = (uint64_t *)calloc(nt, sizeof(uint64_t));
    if (!c.status || !c.partial || !c.inclusive_v) return -1;
    pthread_t th[256];
    for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, scan_mt_worker, &c);
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    free((void *)c.status);
    free(c.partial);
    free(c.inclusive_v);
    return 0;
}

/* ======================================================================
 * Radix sort — onesweep restatement.
 *   device/device_radix_sort.h:187-378   host orchestration
 *   agent/agent_radix_sort_histogram.h:161-187   all-pass histogram
 *   device/details/radix_sort.h:86-122   exclusive sum of bins
 *   agent/agent_radix_sort_onesweep.h:205-335, 394-473   per-tile rank,
 *        look-back (PARTIAL bit 30 / GLOBAL bit 31), scatter
 *   agent/radix_rank_sort_operations.h:19-62, 124-155; common/util_type.h
 *        :98-175   twiddles, -0.0 folded onto +0.0 for digit extraction
 * Ascending LSD over 8-bit digits; every pass is a stable counting sort
 * (the per-tile ranking is stable), so the result is the stable sort of
 * the keys by their twiddled bits.
 * ====================================================================== */
#define RADIX_BITS 8
#define RADIX_DIGITS 256
#define LB_GLOBAL_BIT 0x80000000u
#define LB_PARTIAL_BIT 0x40000000u
#define LB_VALUE_MASK 0x3FFFFFFFu

typedef struct {
    int key_dtype, descending, key_bytes;
    uint64_t high_bit, minus_zero_tw, zero_tw;
} twiddle_t;

static uint64_t tw_in_raw(int dt, uint64_t bits, uint64_t high)
{
    switch (dt) {
    case LCOR_I32: case LCOR_I64: return bits ^ high;
    case LCOR_F32: case LCOR_F64: return (bits & high) ? ~bits : (bits ^ high);
    default: return bits;
    }
}

static void twiddle_init(twiddle_t *t, int dt, int descending)
{
    t->key_dtype = dt;
    t->descending = descending;
    t->key_bytes = (int)dtype_size(dt);
    t->high_bit = t->key_bytes == 4 ? 0x80000000ull : 0x8000000000000000ull;
    /* ProcessFloatMinusZero compares against TwiddleIn(-0) and substitutes
     * TwiddleIn(+0), without the descending inversion
     * (radix_rank_sort_operations.h:33-40). */
    const uint64_t mask = t->key_bytes == 4 ? 0xFFFFFFFFull : ~0ull;
    t->minus_zero_tw = tw_in_raw(dt, t->high_bit, t->high_bit) & mask;
    t->zero_tw = tw_in_raw(dt, 0, t->high_bit) & mask;
}

static inline uint64_t load_key(const void *keys, int kb, uint64_t i)
{
    return kb == 4 ? ((const uint32_t *)keys)[i] : ((const uint64_t *)keys)[i];
}

static inline uint32_t key_digit(const twiddle_t *t, uint64_t raw, uint32_t shift)
{
    uint64_t k = tw_in_raw(t->key_dtype, raw, t->high_bit);
    if (t->key_bytes == 4) k &= 0xFFFFFFFFull;
    if (t->descending) k = ~k & (t->key_bytes == 4 ? 0xFFFFFFFFull : ~0ull);
    if (t->key_dtype == LCOR_F32 || t->key_dtype == LCOR_F64)
        if (k == t->minus_zero_tw) k = t->zero_tw;
    return (uint32_t)(k >> shift) & (RADIX_DIGITS - 1);
}

typedef struct {
    const twiddle_t *tw;
    int kb, vb;
    uint32_t shift, tile_items, num_tiles;
    uint64_t n;
    const char *kin, *vin;
    char *kout, *vout;
    const uint32_t *bins_excl; /* this pass's global exclusive digit prefix */
    _Atomic uint32_t *lookback; /* [num_tiles][256] */
    _Atomic uint32_t ticket;
} pass_ctx;

/* One onesweep tile: local counts -> PARTIAL publish -> per-digit look-back
 * (LookbackGlobal, agent_radix_sort_onesweep.h:283-317) -> GLOBAL publish ->
 * stable scatter in tile order. */
static void sort_tile(pass_ctx *c, uint32_t t)
{
    uint64_t b = (uint64_t)t * c->tile_items;
    uint64_t e = b + c->tile_items < c->n ? b + c->tile_items : c->n;
    uint32_t cnt[RADIX_DIGITS] = {0};
    uint32_t off[RADIX_DIGITS];
    for (uint64_t i = b; i < e; ++i) cnt[key_digit(c->tw, load_key(c->kin, c->kb, i), c->shift)]++;
    _Atomic uint32_t *mine = c->lookback + (size_t)t * RADIX_DIGITS;
    for (int d = 0; d < RADIX_DIGITS; ++d)
        atomic_store_explicit(&mine[d], cnt[d] | LB_PARTIAL_BIT, memory_order_release);
    for (int d = 0; d < RADIX_DIGITS; ++d) {
        uint32_t excl = 0;
        for (int64_t j = (int64_t)t - 1; j >= 0; --j) {
            uint32_t w;
            do {
                w = atomic_load_explicit(&c->lookback[(size_t)j * RADIX_DIGITS + d], memory_order_acquire);
            } while (w == 0);
            excl += w & LB_VALUE_MASK;
            if (w & LB_GLOBAL_BIT) break;
        }
        atomic_store_explicit(&mine[d], (excl + cnt[d]) | LB_GLOBAL_BIT, memory_order_release);
        off[d] = c->bins_excl[d] + excl;
    }
    for (uint64_t i = b; i < e; ++i) {
        uint64_t raw = load_key(c->kin, c->kb, i);
        uint32_t pos = off[key_digit(c->tw, raw, c->shift)]++;
        if (c->kb == 4) ((uint32_t *)c->kout)[pos] = (uint32_t)raw;
        else ((uint64_t *)c->kout)[pos] = raw;
        if (c->vb) memcpy(c->vout + (size_t)pos * c->vb, c->vin + i * c->vb, c->vb);
    }
}

static void *sort_pass_worker(void *p)
{
    pass_ctx *c = (pass_ctx *)p;
    for (;;) {
        uint32_t t = atomic_fetch_add_explicit(&c->ticket, 1, memory_order_relaxed);
        if (t >= c->num_tiles) break;
        sort_tile(c, t);
    }
    return NULL;
}

int lcor_radix_sort(int key_dtype, int val_bytes, const void *keys_in, void *keys_out,
                    const void *vals_in, void *vals_out, uint64_t n, int descending,
                    int nthreads, uint32_t tile_items)
{
    int kb = (int)dtype_size(key_dtype);
    if (!kb || (val_bytes != 0 && val_bytes != 4 && val_bytes != 8)) return -1;
    if (n >= (1ull << 30)) return -1; /* 30-bit look-back counts */
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if (tile_items == 0) tile_items = 4096;
    if (n == 0) return 0;
    twiddle_t tw;
    twiddle_init(&tw, key_dtype, descending);
    const int passes = kb * 8 / RADIX_BITS;

    /* all-pass histogram + exclusive sums (agent_radix_sort_histogram.h:161-187,
     * device/details/radix_sort.h:86-122) */
    uint32_t *bins = (uint32_t *)calloc((size_t)passes * RADIX_DIGITS, sizeof(uint32_t));
    for (uint64_t i = 0; i < n; ++i) {
        uint64_t raw = load_key(keys_in, kb, i);
        for (int p = 0; p < passes; ++p) bins[p * RADIX_DIGITS + key_digit(&tw, raw, p * RADIX_BITS)]++;
    }
    for (int p = 0; p < passes; ++p) {
        uint32_t run = 0;
        for (int d = 0; d < RADIX_DIGITS; ++d) {
            uint32_t c = bins[p * RADIX_DIGITS + d];
            bins[p * RADIX_DIGITS + d] = run;
            run += c;
        }
    }

    /* ping-pong buffers: the input is preserved and the last pass lands in
     * keys_out (device_radix_sort.h:307-375). */
    char *ktmp = (char *)malloc((size_t)n * kb);
    char *vtmp = val_bytes ? (char *)malloc((size_t)n * val_bytes) : NULL;
    uint32_t num_tiles = (uint32_t)((n + tile_items - 1) / tile_items);
    _Atomic uint32_t *lookback =
        (_Atomic uint32_t *)malloc((size_t)num_tiles * RADIX_DIGITS * sizeof(uint32_t));
    if (!bins || !ktmp || (val_bytes && !vtmp) || !lookback) return -1;

    const char *src_k = (const char *)keys_in, *src_v = (const char *)vals_in;
    for (int p = 0; p < passes; ++p) {
        int last = p == passes - 1;
        /* even passes write the scratch buffer, odd ones the output */
        char *dst_k = ((passes - 1 - p) % 2 == 0) ? (char *)keys_out : ktmp;
        char *dst_v = ((passes - 1 - p) % 2 == 0) ? (char *)vals_out : vtmp;
        (void)last;
        pass_ctx c;
        c.tw = &tw;
        c.kb = kb;
        c.vb = val_bytes;
        c.shift = (uint32_t)(p * RADIX_BITS);
        c.tile_items = tile_items;
        c.num_tiles = num_tiles;
        c.n = n;
        c.kin = src_k;
        c.vin = src_v;
        c.kout = dst_k;
        c.vout = dst_v;
        c.bins_excl = bins + p * RADIX_DIGITS;
        c.lookback = lookback;
        memset((void *)lookback, 0, (size_t)num_tiles * RADIX_DIGITS * sizeof(uint32_t));
        atomic_init(&c.ticket, 0);
        if (nthreads == 1) {
            sort_pass_worker(&c);
        } else {
            pthread_t th[256];
            for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, sort_pass_worker, &c);
            for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
        }
        src_k = dst_k;
        src_v = dst_v;
    }
    free(bins);
    free(ktmp);
    free(vtmp);
    free((void *)lookback);
    return 0;
}

int lcor_check_stable_pairs_u64_u32(const uint64_t *keys_in, const uint64_t *keys_out,
                                    const uint32_t *vals_out, uint64_t n)
{
    uint8_t *seen = (uint8_t *)calloc(n ? n : 1, 1);
    if (!seen) return -1;
    int ok = 1;
    for (uint64_t i = 0; i < n && ok; ++i) {
        uint32_t v = vals_out[i];
        if (v >= n || seen[v]) { ok = 0; break; }
        seen[v] = 1;
        if (keys_out[i] != keys_in[v]) { ok = 0; break; }
        if (i > 0) {
            if (keys_out[i - 1] > keys_out[i]) ok = 0;
            else if (keys_out[i - 1] == keys_out[i] && vals_out[i - 1] >= v) ok = 0;
        }
    }
    free(seen);
    return ok;
}

int lcor_check_sorted_permutation_u32(const uint32_t *keys_in, const uint32_t *keys_out,
                                      uint64_t n)
{
    /* sortedness + exact multiset equality via a 2^16-bucket count on the
     * high half and a per-bucket count on the low half (keys_out is sorted,
     * so each bucket is a contiguous run). */
    for (uint64_t i = 1; i < n; ++i)
        if (keys_out[i - 1] > keys_out[i]) return 0;
    uint64_t *hist = (uint64_t *)calloc(65536 + 1, sizeof(uint64_t));
    if (!hist) return -1;
    for (uint64_t i = 0; i < n; ++i) hist[(keys_in[i] >> 16) + 1]++;
    for (int b = 0; b < 65536; ++b) hist[b + 1] += hist[b];
    uint64_t *cursor = (uint64_t *)malloc(65536 * sizeof(uint64_t));
    uint16_t *lo = (uint16_t *)malloc((n ? n : 1) * sizeof(uint16_t));
    if (!cursor || !lo) return -1;
    memcpy(cursor, hist, 65536 * sizeof(uint64_t));
    for (uint64_t i = 0; i < n; ++i) lo[cursor[keys_in[i] >> 16]++] = (uint16_t)keys_in[i];
    int ok = 1;
    uint32_t *cnt = (uint32_t *)calloc(65536, sizeof(uint32_t));
    for (int b = 0; b < 65536 && ok; ++b) {
        uint64_t s = hist[b], e = hist[b + 1];
        if (e == s) continue;
        for (uint64_t i = s; i < e; ++i) {
            if ((keys_out[i] >> 16) != (uint32_t)b) { ok = 0; break; }
            cnt[keys_out[i] & 0xFFFF]++;
        }
        for (uint64_t i = s; i < e && ok; ++i) {
            if (cnt[lo[i]] == 0) ok = 0;
            else cnt[lo[i]]--;
        }
        for (uint64_t i = s; i < e; ++i) cnt[keys_out[i] & 0xFFFF] = 0;
    }
    free(cnt);
    free(hist);
    free(cursor);
    free(lo);
    return ok;
}

/* ======================================================================
 * Segment reduce — device/device_segment_reduce.h:125-135 (Sum with
 * begin/end offsets) and device/details/segment_reduce.h:43-86:
 * out[s] = init op reduce(in[begin[s] .. end[s])), empty -> init (+0).
 * ====================================================================== */
int lcor_segment_reduce(int op, int dtype, const void *in, void *out, uint64_t num_segments,
                        const uint32_t *begin, const uint32_t *end, const void *init)
{
    size_t es = dtype_size(dtype);
    if (!es || op < 0 || op > 2) return -1;
    for (uint64_t s = 0; s < num_segments; ++s) {
        char *o = (char *)out + s * es;
        uint64_t acc = 0;
        init_value(op, dtype, &acc);
        if (end[s] > begin[s]) {
            if (dtype == LCOR_F32 && op == LCOR_OP_SUM) {
                double sum, a;
                lcor_reduce_f64(dtype, (const char *)in + (size_t)begin[s] * es, end[s] - begin[s], &sum, &a);
                float f = (float)sum;
                memcpy(&acc, &f, 4);
            } else {
                fold_any(op, dtype, (const char *)in + (size_t)begin[s] * es, end[s] - begin[s], &acc);
            }
        }
        if (init) {  /* out = op(init, aggregate) (segment_reduce.h:81) */
            uint64_t r = 0;
            memcpy(&r, init, es);
            fold_any(op, dtype, &acc, 1, &r);
            acc = r;
        }
        memcpy(o, &acc, es);
    }
    return 0;
}

/* Segment ArgMin / ArgMax — device/device_segment_reduce.h:197-349 and
 * details/segment_reduce.h:166-240: (index, value) pairs folded with
 * ArgMinOp / ArgMaxOp (common/thread_operators.h:19-47: ArgMin keeps the
 * smaller value, on ties the smaller index; ArgMax the larger value, on ties
 * the larger index), the index reported relative to begin[s].  An empty
 * segment gives index 1 and value max() (ArgMin) / lowest() (ArgMax); the
 * reference's arg_assign computes 1 - begin[s] there (segment_reduce.h
 * :214-216), which wraps for begin > 1. */
/* the first element of a non-empty segment starts the fold (no sentinel
 * value takes part, so +-inf elements are found like any other) */
#define SEG_ARG_FOLD(T)                                                                \
    do {                                                                               \
        const T *a = (const T *)in;                                                    \
        if (e > b) {                                                                   \
            T best = a[b];                                                             \
            uint32_t bi = b;                                                           \
            for (uint32_t i = b + 1; i < e; ++i) {                                     \
                const T x = a[i];                                                      \
                const int take = is_max ? (x > best || (x == best && i > bi))          \
                                        : (x < best || (x == best && i < bi));         \
                if (take) { best = x; bi = i; }                                        \
            }                                                                          \
            memcpy(&v, &best, sizeof(T));                                              \
            idx = bi - b;                                                              \
        }                                                                              \
    } while (0)

int lcor_segment_reduce_arg(int is_max, int dtype, const void *in, void *out, uint32_t *index_out,
                            uint64_t num_segments, const uint32_t *begin, const uint32_t *end)
{
    const size_t es = dtype_size(dtype);
    if (!es) return -1;
    for (uint64_t s = 0; s < num_segments; ++s) {
        uint64_t v = 0;
        init_value(is_max ? LCOR_OP_MAX : LCOR_OP_MIN, dtype, &v);
        uint32_t idx = 1;
        const uint32_t b = begin[s], e = end[s];
        switch (dtype) {
        case LCOR_I32: SEG_ARG_FOLD(int32_t); break;
        case LCOR_U32: SEG_ARG_FOLD(uint32_t); break;
        case LCOR_F32: SEG_ARG_FOLD(float); break;
        case LCOR_I64: SEG_ARG_FOLD(int64_t); break;
        case LCOR_U64: SEG_ARG_FOLD(uint64_t); break;
        case LCOR_F64: SEG_ARG_FOLD(double); break;
        }
        memcpy((char *)out + s * es, &v, es);
        index_out[s] = idx;
    }
    return 0;
}

int lcor_segment_reduce_f64(int dtype, const void *in, uint64_t num_segments,
                            const uint32_t *begin, const uint32_t *end, double *sum,
                            double *abs_sum)
{
    size_t es = dtype_size(dtype);
    if (!es) return -1;
    for (uint64_t s = 0; s < num_segments; ++s) {
        if (end[s] > begin[s]) {
            lcor_reduce_f64(dtype, (const char *)in + (size_t)begin[s] * es, end[s] - begin[s], &sum[s], &abs_sum[s]);
        } else {
            sum[s] = 0.0;
            abs_sum[s] = 0.0;
        }
    }
    return 0;
}

typedef struct {
    int dtype;
    const char *in;
    char *out;
    const uint32_t *begin, *end;
    uint64_t s0, s1;
} seg_job;

static void *seg_worker(void *p)
{
    seg_job *j = (seg_job *)p;
    size_t es = dtype_size(j->dtype);
    for (uint64_t s = j->s0; s < j->s1; ++s) {
        uint64_t acc = 0;
        if (j->end[s] > j->begin[s])
            fold_any(LCOR_OP_SUM, j->dtype, j->in + (size_t)j->begin[s] * es, j->end[s] - j->begin[s], &acc);
        memcpy(j->out + s * es, &acc, es);
    }
    return NULL;
}

int lcor_segment_reduce_mt(int dtype, const void *in, void *out, uint64_t num_segments,
                           const uint32_t *begin, const uint32_t *end, int nthreads)
{
    if (!dtype_size(dtype) || nthreads < 1) return -1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    seg_job jobs[256];
    for (int t = 0; t < nthreads; ++t) {
        jobs[t].dtype = dtype;
        jobs[t].in = (const char *)in;
        jobs[t].out = (char *)out;
        jobs[t].begin = begin;
        jobs[t].end = end;
        jobs[t].s0 = num_segments * (uint64_t)t / (uint64_t)nthreads;
        jobs[t].s1 = num_segments * (uint64_t)(t + 1) / (uint64_t)nthreads;
        pthread_create(&th[t], NULL, seg_worker, &jobs[t]);
    }
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    return 0;
}

/* ======================================================================
 * Scan by key / reduce by key.
 *
 * Segments are maximal runs of consecutive equal keys: element i starts a
 * segment (a "head") when i == 0 or keys[i] != keys[i-1], the comparison
 * made in the key's own type, so floating keys treat -0.0 == +0.0 and
 * NaN != NaN (BlockDiscontinuity::FlagHeads with `a != b`,
 * block/block_discontinuity.h:97-130; device/details/scan_by_key.h:196-202,
 * device/details/reduce_by_key.h:168-192).
 * ====================================================================== */
static int key_differs(int kd, const void *keys, uint64_t i)
{
    switch (kd) {
    case LCOR_I32: case LCOR_U32: return ((const uint32_t *)keys)[i] != ((const uint32_t *)keys)[i - 1];
    case LCOR_I64: case LCOR_U64: return ((const uint64_t *)keys)[i] != ((const uint64_t *)keys)[i - 1];
    case LCOR_F32: return ((const float *)keys)[i] != ((const float *)keys)[i - 1];
    case LCOR_F64: return ((const double *)keys)[i] != ((const double *)keys)[i - 1];
    default: return 1;
    }
}

/* op(a, b) on one element of dtype dt, into a (integer sums wrap) */
static void op1(int op, int dt, void *a, const void *b)
{
    fold_any(op, dt, b, 1, a);
}

/* ScanByKey — device/device_scan.h:206-303 (Exclusive/InclusiveScanByKey with
 * scan_op and init), device/details/scan_by_key.h:77-258 (ScanBySegmentOp
 * over (head flag, value) pairs, then AddInitToScan):
 *   exclusive: out[i] = init at a head, else op(fold(values[head..i)), init)
 *   inclusive: out[i] = op(fold(values[head..i]), init)
 * The reference's inclusive variant overwrites every head with init
 * (AddInitToScan, scan_by_key.h:113-128, applied to inclusive results too);
 * this restatement, like the GPU path, gives heads op(value, init).
 * Folds run in element order (floating-point results are order-dependent;
 * lcor_scan_by_key_f64 gives the checker's double-precision values). */
int lcor_scan_by_key(int inclusive, int op, int key_dtype, int val_dtype, const void *keys,
                     const void *vals, void *out, uint64_t n, const void *init)
{
    const size_t es = dtype_size(val_dtype);
    if (!dtype_size(key_dtype) || !es || op < 0 || op > 2) return -1;
    uint64_t run = 0, tmp = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const void *x = (const char *)vals + i * es;
        char *o = (char *)out + i * es;
        const int head = i == 0 || key_differs(key_dtype, keys, i);
        if (head) {
            if (inclusive) { memcpy(&run, x, es); memcpy(&tmp, &run, es); op1(op, val_dtype, &tmp, init); memcpy(o, &tmp, es); }
            else { memcpy(o, init, es); memcpy(&run, x, es); }
        } else {
            if (inclusive) { op1(op, val_dtype, &run, x); memcpy(&tmp, &run, es); op1(op, val_dtype, &tmp, init); memcpy(o, &tmp, es); }
            else { memcpy(&tmp, &run, es); op1(op, val_dtype, &tmp, init); memcpy(o, &tmp, es); op1(op, val_dtype, &run, x); }
        }
    }
    return 0;
}

/* Double-precision segmented sums of floating values (init 0) and the
 * matching segmented sums of |x|, for the normwise tolerance. */
int lcor_scan_by_key_f64(int inclusive, int key_dtype, int val_dtype, const void *keys,
                         const void *vals, double *out, double *abs_prefix, uint64_t n)
{
    if (!dtype_size(key_dtype) || (val_dtype != LCOR_F32 && val_dtype != LCOR_F64)) return -1;
    double s = 0.0, a = 0.0;
    for (uint64_t i = 0; i < n; ++i) {
        const double x = val_dtype == LCOR_F32 ? ((const float *)vals)[i] : ((const double *)vals)[i];
        if (i == 0 || key_differs(key_dtype, keys, i)) { s = 0.0; a = 0.0; }
        if (!inclusive) { out[i] = s; abs_prefix[i] = a; }
        s += x;
        a += fabs(x);
        if (inclusive) { out[i] = s; abs_prefix[i] = a; }
    }
    return 0;
}

/* ReduceByKey — device/device_reduce.h:277-318, device/details/
 * reduce_by_key.h:61-258 (ReduceBySegmentOp over (head count, value) pairs,
 * scatter at heads): run r = r-th maximal run of equal keys;
 * unique_out[r] = its key, aggregates_out[r] = op-fold of its values (no
 * init, element order), *num_runs = number of runs (0 when n = 0). */
int lcor_reduce_by_key(int op, int key_dtype, int val_dtype, const void *keys, const void *vals,
                       void *unique_out, void *aggregates_out, uint64_t n, uint64_t *num_runs)
{
    const size_t ks = dtype_size(key_dtype), es = dtype_size(val_dtype);
    if (!ks || !es || op < 0 || op > 2) return -1;
    uint64_t r = 0, acc = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const void *x = (const char *)vals + i * es;
        if (i > 0 && key_differs(key_dtype, keys, i)) {
            memcpy((char *)unique_out + r * ks, (const char *)keys + (i - 1) * ks, ks);
            memcpy((char *)aggregates_out + r * es, &acc, es);
            ++r;
        }
        if (i == 0 || key_differs(key_dtype, keys, i)) memcpy(&acc, x, es);
        else op1(op, val_dtype, &acc, x);
    }
    if (n) {
        memcpy((char *)unique_out + r * ks, (const char *)keys + (n - 1) * ks, ks);
        memcpy((char *)aggregates_out + r * es, &acc, es);
        ++r;
    }
    *num_runs = r;
    return 0;
}

/* Double-precision run sums of floating values and run sums of |x|. */
int lcor_reduce_by_key_f64(int key_dtype, int val_dtype, const void *keys, const void *vals,
                           uint64_t n, double *sums, double *abs_sums, uint64_t *num_runs)
{
    if (!dtype_size(key_dtype) || (val_dtype != LCOR_F32 && val_dtype != LCOR_F64)) return -1;
    uint64_t r = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const double x = val_dtype == LCOR_F32 ? ((const float *)vals)[i] : ((const double *)vals)[i];
        if (i > 0 && key_differs(key_dtype, keys, i)) ++r;
        if (i == 0 || key_differs(key_dtype, keys, i)) { sums[r] = 0.0; abs_sums[r] = 0.0; }
        sums[r] += x;
        abs_sums[r] += fabs(x);
    }
    *num_runs = n ? r + 1 : 0;
    return 0;
}
