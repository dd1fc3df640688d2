/*
 * oracle_check.c — sanitizer driver for the CPU oracle (test infrastructure).
 *
 * Runs every function of lcpp_oracle.c on seeded inputs at sizes that finish
 * in seconds under ASan/UBSan/TSan, and cross-checks the multithreaded
 * restatements (the decoupled look-back KAT, the bounded look-back with a
 * withheld predecessor, the single-pass scan, the onesweep sort passes, the
 * multithreaded reduce and segment reduce) against the single-threaded ones.
 * Exit status 0 and "oracle_check: OK" when every check holds; the
 * sanitizers abort on the first error they find.
 */
#include "../lcpp_oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int g_checks, g_failed;

#define CHECK(cond, ...)                                        \
    do {                                                        \
        ++g_checks;                                             \
        if (!(cond)) {                                          \
            ++g_failed;                                         \
            fprintf(stderr, "FAILED %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                       \
            fputc('\n', stderr);                                \
        }                                                       \
    } while (0)

static void *xmalloc(size_t bytes)
{
    void *p = malloc(bytes ? bytes : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

static const int kThreads[] = {1, 2, 3, 8};
static const uint64_t kSizes[] = {0, 1, 2, 1000, 16384, 16385, 100003};
#define COUNT(a) (sizeof(a) / sizeof((a)[0]))

static void check_generators(void)
{
    const uint64_t n = 4099;
    uint64_t *w = xmalloc(n * 8);
    lcor_gen_words(7, 0, n, w);
    CHECK(w[5] == lcor_word(7, 5), "gen_words");
    int32_t *r = xmalloc(n * 4);
    uint32_t *u = xmalloc(n * 4);
    float *f = xmalloc(n * 4);
    uint64_t *k = xmalloc(n * 8);
    lcor_gen_reduce_i32(1, n, r);
    lcor_gen_u8_u32(2, n, u);
    for (uint64_t i = 0; i < n; ++i) CHECK(u[i] < 256, "u8_u32 range");
    lcor_gen_normal_f32(3, n, f);
    lcor_gen_keys_u32(4, n, u);
    lcor_gen_keys_u32_and3(4, 5, 6, n, u);
    lcor_gen_keys_u64_low16(8, n, k);
    for (uint64_t i = 0; i < n; ++i) CHECK(k[i] < 65536, "keys_u64_low16 range");
    lcor_gen_iota_u32(n, u);
    CHECK(u[n - 1] == n - 1, "iota");
    uint32_t b[100], e[100];
    CHECK(lcor_gen_segments(9, 10, 5000, 100, b, e) == 0, "gen_segments");
    CHECK(b[0] == 0 && e[99] == 5000, "gen_segments covers the items");
    free(w), free(r), free(u), free(f), free(k);
}

static void check_reduce_and_scan(void)
{
    const int dtypes[] = {LCOR_I32, LCOR_U32, LCOR_F32, LCOR_I64, LCOR_U64, LCOR_F64};
    const uint64_t nmax = 100003;
    uint64_t *raw = xmalloc(nmax * 8);
    lcor_gen_words(11, 0, nmax, raw);
    double *dv = xmalloc(nmax * 8);
    float *fv = xmalloc(nmax * 4);
    for (uint64_t i = 0; i < nmax; ++i) {
        dv[i] = (double)(raw[i] >> 40) / 1024.0;
        fv[i] = (float)dv[i];
    }
    char *out1 = xmalloc(nmax * 8), *out2 = xmalloc(nmax * 8);
    for (size_t d = 0; d < COUNT(dtypes); ++d) {
        const int dt = dtypes[d];
        const void *in = dt == LCOR_F32 ? (const void *)fv : dt == LCOR_F64 ? (const void *)dv : (const void *)raw;
        for (size_t s = 0; s < COUNT(kSizes); ++s) {
            const uint64_t n = kSizes[s];
            for (int op = 0; op < 3; ++op) {
                uint64_t a = 0, b = 0;
                CHECK(lcor_reduce(op, dt, in, n, &a) == 0, "reduce");
                for (size_t t = 0; t < COUNT(kThreads); ++t) {
                    b = 0;
                    CHECK(lcor_reduce_mt(op, dt, in, n, &b, kThreads[t]) == 0, "reduce_mt");
                    if (dt != LCOR_F32 && dt != LCOR_F64 && op == LCOR_OP_SUM)
                        CHECK(memcmp(&a, &b, 8) == 0, "reduce_mt == reduce (dtype %d n %llu)", dt,
                              (unsigned long long)n);
                }
            }
            if (n) {
                uint64_t v = 0;
                uint32_t idx = 0;
                CHECK(lcor_reduce_arg(0, dt, in, n, &v, &idx) == 0 && idx < n, "argmin");
                CHECK(lcor_reduce_arg(1, dt, in, n, &v, &idx) == 0 && idx < n, "argmax");
            }
            uint64_t init = 0, o = 0;
            for (int xf = 0; xf < 4; ++xf) CHECK(lcor_reduce_transform(0, xf, dt, in, n, &init, &o) == 0, "transform");
            double sum, abs_sum;
            CHECK(lcor_reduce_f64(dt, in, n, &sum, &abs_sum) == 0, "reduce_f64");
            for (int inc = 0; inc < 2; ++inc) {
                CHECK(lcor_scan(inc, dt, in, out1, n) == 0, "scan");
                for (size_t t = 0; t < COUNT(kThreads); ++t) {
                    CHECK(lcor_scan_mt(inc, dt, in, out2, n, kThreads[t]) == 0, "scan_mt");
                    if (dt != LCOR_F32 && dt != LCOR_F64)
                        CHECK(memcmp(out1, out2, n * (dt >= LCOR_I64 ? 8 : 4)) == 0,
                              "scan_mt == scan (dtype %d inclusive %d n %llu threads %d)", dt, inc,
                              (unsigned long long)n, kThreads[t]);
                }
                double *ap = xmalloc((n ? n : 1) * 8);
                const int want = dt == LCOR_F32 || dt == LCOR_F64 ? 0 : -1;  /* float types only */
                CHECK(lcor_scan_f64(inc, dt, in, (double *)out2, ap, n) == want, "scan_f64");
                free(ap);
            }
        }
    }
    free(raw), free(dv), free(fv), free(out1), free(out2);
}

static void check_lookback(void)
{
    const uint32_t tiles = 10240;
    int32_t *ex = xmalloc(tiles * 4), *in = xmalloc(tiles * 4), *agg = xmalloc(tiles * 4);
    for (size_t t = 0; t < COUNT(kThreads); ++t) {
        CHECK(lcor_lookback_kat(tiles, kThreads[t], ex, in) == 0, "lookback_kat");
        int ok = 1;
        for (uint32_t i = 0; i < tiles; ++i) ok &= ex[i] == (int32_t)i && in[i] == (int32_t)i + 1;
        CHECK(ok, "lookback KAT (threads %d)", kThreads[t]);
    }
    uint64_t *w = xmalloc(tiles * 8);
    lcor_gen_words(21, 0, tiles, w);
    for (uint32_t i = 0; i < tiles; ++i) agg[i] = (int32_t)(uint32_t)w[i];
    const uint32_t widths[] = {1, 16, 64};
    for (size_t t = 0; t < COUNT(kThreads); ++t)
        for (size_t k = 0; k < COUNT(widths); ++k) {
            uint32_t status = 7;
            CHECK(lcor_lookback_bounded(agg, tiles, kThreads[t], 0xFFFFFFFFu, 1u << 20, widths[k], ex, in, &status) == 0,
                  "lookback_bounded");
            uint32_t run = 0;
            int ok = status == 0;
            for (uint32_t i = 0; i < tiles; ++i) {
                ok &= ex[i] == (int32_t)run;
                run += (uint32_t)agg[i];
                ok &= in[i] == (int32_t)run;
            }
            CHECK(ok, "bounded look-back exact (threads %d width %u status %u)", kThreads[t], widths[k], status);
        }
    /* a withheld predecessor: the wait gives up and says so; every thread ends */
    const uint32_t held[] = {0, 5, 3000};
    for (size_t h = 0; h < COUNT(held); ++h)
        for (size_t t = 0; t < COUNT(kThreads); ++t) {
            uint32_t status = 0;
            CHECK(lcor_lookback_bounded(agg, 4096, kThreads[t], held[h], 2000, 16, ex, in, &status) == 0,
                  "lookback_bounded withheld");
            CHECK(held[h] >= 4095 || (status & 1u), "withheld tile %u reported (threads %d)", held[h], kThreads[t]);
        }
    free(ex), free(in), free(agg), free(w);
}

static void check_sort(void)
{
    const uint64_t nmax = 100003;
    uint32_t *k = xmalloc(nmax * 4), *ko = xmalloc(nmax * 4), *ko2 = xmalloc(nmax * 4);
    uint64_t *k64 = xmalloc(nmax * 8), *k64o = xmalloc(nmax * 8);
    uint32_t *v = xmalloc(nmax * 4), *vo = xmalloc(nmax * 4);
    lcor_gen_keys_u32(31, nmax, k);
    lcor_gen_keys_u64_low16(32, nmax, k64);
    lcor_gen_iota_u32(nmax, v);
    for (size_t s = 0; s < COUNT(kSizes); ++s) {
        const uint64_t n = kSizes[s];
        CHECK(lcor_radix_sort(LCOR_U32, 0, k, ko, NULL, NULL, n, 0, 1, 0) == 0, "sort keys");
        CHECK(lcor_check_sorted_permutation_u32(k, ko, n) == 1, "sorted permutation (n %llu)", (unsigned long long)n);
        for (size_t t = 0; t < COUNT(kThreads); ++t) {
            CHECK(lcor_radix_sort(LCOR_U32, 0, k, ko2, NULL, NULL, n, 0, kThreads[t], 1024) == 0, "sort keys mt");
            CHECK(memcmp(ko, ko2, n * 4) == 0, "sort keys mt == single (n %llu threads %d)", (unsigned long long)n,
                  kThreads[t]);
            CHECK(lcor_radix_sort(LCOR_U64, 4, k64, k64o, v, vo, n, 0, kThreads[t], 1024) == 0, "sort pairs");
            CHECK(lcor_check_stable_pairs_u64_u32(k64, k64o, vo, n) == 1, "stable pairs (n %llu threads %d)",
                  (unsigned long long)n, kThreads[t]);
            CHECK(lcor_radix_sort(LCOR_I32, 4, k, ko2, v, vo, n, 1, kThreads[t], 2048) == 0, "sort descending");
        }
    }
    free(k), free(ko), free(ko2), free(k64), free(k64o), free(v), free(vo);
}

static void check_by_key_and_segments(void)
{
    const uint64_t nmax = 100003;
    int32_t *keys = xmalloc(nmax * 4), *vals = xmalloc(nmax * 4), *out = xmalloc(nmax * 4), *uk = xmalloc(nmax * 4);
    uint64_t *w = xmalloc(nmax * 8);
    lcor_gen_words(41, 0, nmax, w);
    int32_t key = 0;
    for (uint64_t i = 0; i < nmax; ++i) {
        key += (w[i] & 127) == 0;
        keys[i] = key;
        vals[i] = (int32_t)(w[i] >> 40);
    }
    double *dsum = xmalloc(nmax * 8), *dabs = xmalloc(nmax * 8);
    float *fin = xmalloc(nmax * 4);
    for (uint64_t i = 0; i < nmax; ++i) fin[i] = (float)(vals[i] & 1023);
    for (size_t s = 0; s < COUNT(kSizes); ++s) {
        const uint64_t n = kSizes[s];
        const int32_t init = 3;
        for (int inc = 0; inc < 2; ++inc)
            for (int op = 0; op < 3; ++op)
                CHECK(lcor_scan_by_key(inc, op, LCOR_I32, LCOR_I32, keys, vals, out, n, &init) == 0, "scan_by_key");
        CHECK(lcor_scan_by_key_f64(1, LCOR_I32, LCOR_F32, keys, fin, dsum, dabs, n) == 0, "scan_by_key_f64");
        uint64_t runs = 0, runs2 = 0;
        for (int op = 0; op < 3; ++op)
            CHECK(lcor_reduce_by_key(op, LCOR_I32, LCOR_I32, keys, vals, uk, out, n, &runs) == 0, "reduce_by_key");
        CHECK(lcor_reduce_by_key_f64(LCOR_I32, LCOR_F32, keys, fin, n, dsum, dabs, &runs2) == 0 && runs == runs2,
              "reduce_by_key_f64 runs");
    }
    const uint64_t segs = 5000;
    uint32_t *b = xmalloc(segs * 4), *e = xmalloc(segs * 4), *idx = xmalloc(segs * 4);
    float *fo1 = xmalloc(segs * 4), *fo2 = xmalloc(segs * 4);
    CHECK(lcor_gen_segments(42, 43, nmax, segs, b, e) == 0, "gen_segments");
    CHECK(lcor_segment_reduce(0, LCOR_F32, fin, fo1, segs, b, e, NULL) == 0, "segment_reduce");
    for (size_t t = 0; t < COUNT(kThreads); ++t) {
        CHECK(lcor_segment_reduce_mt(LCOR_F32, fin, fo2, segs, b, e, kThreads[t]) == 0, "segment_reduce_mt");
        CHECK(memcmp(fo1, fo2, segs * 4) == 0, "segment_reduce_mt == single (threads %d)", kThreads[t]);
    }
    for (int op = 1; op < 3; ++op) CHECK(lcor_segment_reduce(op, LCOR_I32, vals, out, segs, b, e, NULL) == 0, "seg op");
    CHECK(lcor_segment_reduce_arg(0, LCOR_F32, fin, fo1, idx, segs, b, e) == 0, "segment argmin");
    CHECK(lcor_segment_reduce_arg(1, LCOR_I32, vals, out, idx, segs, b, e) == 0, "segment argmax");
    CHECK(lcor_segment_reduce_f64(LCOR_F32, fin, segs, b, e, dsum, dabs) == 0, "segment f64");
    free(keys), free(vals), free(out), free(uk), free(w), free(dsum), free(dabs), free(b), free(e), free(idx);
    free(fin), free(fo1), free(fo2);
}

int main(int argc, char **argv)
{
    const char *only = argc > 1 ? argv[1] : "";
    if (!*only || !strcmp(only, "gen")) check_generators();
    if (!*only || !strcmp(only, "reduce")) check_reduce_and_scan();
    if (!*only || !strcmp(only, "lookback")) check_lookback();
    if (!*only || !strcmp(only, "sort")) check_sort();
    if (!*only || !strcmp(only, "bykey")) check_by_key_and_segments();
    if (g_failed) {
        fprintf(stderr, "oracle_check: %d of %d checks FAILED\n", g_failed, g_checks);
        return 1;
    }
    printf("oracle_check: OK (%d checks)\n", g_checks);
    return 0;
}
