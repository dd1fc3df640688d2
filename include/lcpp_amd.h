/*
 * lcpp_amd.h — C ABI of the MI355X-native (gfx950) device-level primitives.
 *
 * Every entry point here replaces a method of the reference's C++ class
 * templates (paths relative to src/lcpp/ of Ligo04/lc_parallel_primitive).
 * The reference has no C ABI of its own; the C++ wrapper in
 * include/lcpp/parallel_primitive.h restores its class/method names on top
 * of these functions.
 *
 * Conventions
 *   - Every function returns an lcpp_status (0 = success, negative = error);
 *     nothing is thrown across the ABI.
 *   - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *     All work is enqueued asynchronously on it; results are valid once the
 *     stream is synchronized.  No primitive synchronizes the stream (only the
 *     validation calls lcpp_temp_status and lcpp_stream_sync do).
 *   - The caller owns all memory, including temp storage sized by the
 *     matching *_temp_bytes query.  The library never allocates device
 *     memory on these paths.  Temp storage must be 256-byte aligned.
 *   - Inputs are read only.  The sort preserves keys_in / values_in
 *     (as the reference's DoubleBuffer ping-pong does).
 *   - Calls that share one temp buffer must not overlap in time (the
 *     look-back state lives in temp storage).  Calls with distinct temp
 *     buffers are thread-safe.
 *   - *_temp_bytes queries are pure host arithmetic and need no GPU.
 */
#ifndef LCPP_AMD_H
#define LCPP_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LCPP_AMD_VERSION 100 /* 1.0.0 */

/* The enums are int-sized in C.  C++ fixes int as their underlying type, so
 * that every int a C, Go or Python caller passes is a value of the enum type
 * in the library (which rejects unknown codes with a status instead of
 * reading an out-of-range enum). */
#ifdef __cplusplus
#define LCPP_ENUM_INT : int
#else
#define LCPP_ENUM_INT
#endif

typedef enum lcpp_dtype LCPP_ENUM_INT {
    LCPP_INT32 = 0,
    LCPP_UINT32 = 1,
    LCPP_FLOAT32 = 2,
    LCPP_INT64 = 3,
    LCPP_UINT64 = 4,
    LCPP_FLOAT64 = 5
} lcpp_dtype;

/* Reduction operators and element transforms of lcpp_reduce_transform (the
 * reference takes arbitrary device functors; a C ABI carries a fixed set). */
typedef enum lcpp_reduce_op LCPP_ENUM_INT {
    LCPP_OP_SUM = 0,
    LCPP_OP_MIN = 1,
    LCPP_OP_MAX = 2
} lcpp_reduce_op;

typedef enum lcpp_transform LCPP_ENUM_INT {
    LCPP_XFORM_IDENTITY = 0,
    LCPP_XFORM_NEGATE = 1, /* integers wrap (two's complement) */
    LCPP_XFORM_ABS = 2,    /* identity for unsigned types */
    LCPP_XFORM_SQUARE = 3  /* integers wrap */
} lcpp_transform;

typedef enum lcpp_status LCPP_ENUM_INT {
    LCPP_OK = 0,
    LCPP_ERR_INVALID_ARG = -1,      /* null pointer, misaligned temp, size out of range */
    LCPP_ERR_TEMP_TOO_SMALL = -2,   /* temp_bytes < the *_temp_bytes query result */
    LCPP_ERR_UNSUPPORTED_DTYPE = -3,
    LCPP_ERR_HIP = -4,              /* a HIP runtime call or kernel launch failed */
    LCPP_ERR_LOOKBACK_TIMEOUT = -5, /* reported by lcpp_temp_status: a look-back wait gave up,
                                       so that call's output is wrong */
    LCPP_ERR_SIZE_LIMIT = -6        /* n exceeds what lcpp_scan_exclusive_sum_noalloc's fixed
                                       scratch covers */
} lcpp_status;

/* Bits of the device status word kept in the first 4 bytes of temp storage. */
#define LCPP_DEVICE_STATUS_LOOKBACK_TIMEOUT 1u

/* Library version (LCPP_AMD_VERSION of the build). */
int lcpp_version(void);
/* Static, human-readable name of a status code. */
const char *lcpp_status_string(int status);

/* ---------------------------------------------------------------------
 * Device-side status (the counterpart of the reference's debug-stream check,
 * lcpp_check in runtime/core.h:56-64, which commits, synchronizes and asserts
 * after each step).  Every primitive that uses temp storage reserves its
 * first 256 bytes as a status header; the call's first kernel zeroes the
 * status word and a decoupled look-back wait that exhausts its bounded spin
 * sets LCPP_DEVICE_STATUS_LOOKBACK_TIMEOUT in it (its output is then wrong;
 * the kernels still finish).  A wait can only give up when the workgroups it
 * waits on cannot run, e.g. when other kernels hold the whole device.
 * ------------------------------------------------------------------- */
/* Synchronizes `stream`, then reads the status word of the last call that used
 * `temp` (temp_bytes as passed to that call; calls whose temp query is 0 do not
 * use temp storage).  Returns LCPP_OK, LCPP_ERR_LOOKBACK_TIMEOUT or LCPP_ERR_HIP.
 * temp == NULL or temp_bytes < 256: synchronizes and returns LCPP_OK.  This is
 * the one function here that synchronizes (a debug / validation path). */
int lcpp_temp_status(const void *temp, size_t temp_bytes, void *stream);
/* The same check without synchronizing: enqueues on `stream` a one-thread kernel that ORs the
 * status word of the last call that used `temp` into *dst (device memory, or pinned host memory
 * the device can write).  A caller can accumulate the words of many calls into one and decode it
 * with lcpp_device_status_decode at its own synchronization point.  Returns LCPP_OK without a
 * launch when temp == NULL or temp_bytes < 256 (calls whose temp query is 0 keep no status word).
 * No counterpart in the reference (whose debug check synchronizes). */
int lcpp_temp_status_record(const void *temp, size_t temp_bytes, uint32_t *dst, void *stream);
/* The lcpp_status a device status word stands for (pure host arithmetic). */
int lcpp_device_status_decode(uint32_t word);
/* hipStreamSynchronize(stream): LCPP_OK or LCPP_ERR_HIP. */
int lcpp_stream_sync(void *stream);
/* Test hook, process-wide: look-back waits give up after `spin_limit` re-polls
 * (0 = the default, about half a second of polling), and the tile or sort tile
 * numbered `withhold_tile` does not publish its look-back words
 * (0xFFFFFFFF = none), so the waits behind it give up and report through the
 * status word.  Outputs of calls made while a tile is withheld are wrong.  Not
 * for production use; calls running concurrently see the same setting. */
int lcpp_test_set_lookback_fault(uint32_t withhold_tile, uint32_t spin_limit);

/* ---------------------------------------------------------------------
 * DeviceReduce — device/device_reduce.h
 * ------------------------------------------------------------------- */
/* replaces DeviceReduce::GetTempStorageBytes<T>(num_item), device_reduce.h:85-91 */
int lcpp_reduce_temp_bytes(lcpp_dtype t, uint64_t n, size_t *bytes);
/* replaces DeviceReduce::Sum(cmdlist, temp, d_in, d_out, num_item), device_reduce.h:169-173
 * out[0] = 0 + sum(in[0..n)); integers wrap (two's complement). */
int lcpp_reduce_sum(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                    uint64_t n, void *stream);
/* replaces DeviceReduce::Min, device_reduce.h:175-179 (init = numeric max) */
int lcpp_reduce_min(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                    uint64_t n, void *stream);
/* replaces DeviceReduce::Max, device_reduce.h:181-185 (init = numeric lowest; the reference
 * uses numeric_limits<T>::min(), which differs for floating point only) */
int lcpp_reduce_max(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                    uint64_t n, void *stream);
/* replaces DeviceReduce::TransformReduce(cmdlist, temp, d_in, d_out, num_item, reduce_op,
 * transform_op, init), device_reduce.h:331-348:
 * out[0] = op(init, op over i of xf(in[i])); *init is a host value of type t.
 * Temp storage as for lcpp_reduce_temp_bytes. */
int lcpp_reduce_transform(lcpp_dtype t, lcpp_reduce_op op, lcpp_transform xf, void *temp,
                          size_t temp_bytes, const void *in, void *out, uint64_t n, const void *init,
                          void *stream);
/* replaces DeviceReduce::GetArgTempStorageBytes<T>(num_item), device_reduce.h:94-107 */
int lcpp_reduce_arg_temp_bytes(lcpp_dtype t, uint64_t n, size_t *bytes);
/* replaces DeviceReduce::ArgMin(cmdlist, temp, d_in, d_out, d_index_out, num_item),
 * device_reduce.h:187-227: the smallest value and its index; ties go to the smallest index
 * (ArgMinOp, common/thread_operators.h:34-47).  n = 0 gives (numeric max, 0xFFFFFFFF).
 * n < 2^32. */
int lcpp_reduce_argmin(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                       uint32_t *index_out, uint64_t n, void *stream);
/* replaces DeviceReduce::ArgMax, device_reduce.h:229-272: the largest value and its index;
 * ties go to the LARGEST index (ArgMaxOp, common/thread_operators.h:19-31).  Starts from
 * numeric lowest() (the reference: numeric_limits<T>::min()), so n = 0 gives (lowest, 0). */
int lcpp_reduce_argmax(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                       uint32_t *index_out, uint64_t n, void *stream);

/* ---------------------------------------------------------------------
 * DeviceScan — device/device_scan.h
 * ------------------------------------------------------------------- */
/* replaces DeviceScan::GetTempStorageBytes<T>(num_items), device_scan.h:76-89 */
int lcpp_scan_temp_bytes(lcpp_dtype t, uint64_t n, size_t *bytes);
/* replaces DeviceScan::ExclusiveSum, device_scan.h:180-191: out[i] = sum(in[0..i)) */
int lcpp_scan_exclusive_sum(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in,
                            void *out, uint64_t n, void *stream);
/* replaces DeviceScan::InclusiveSum, device_scan.h:193-204: out[i] = sum(in[0..i]) */
int lcpp_scan_inclusive_sum(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in,
                            void *out, uint64_t n, void *stream);
/* replaces DeviceScan::ExclusiveScan(cmdlist, temp, d_in, d_out, num_items, scan_op,
 * initial_value), device_scan.h:114-145: out[i] = op(init, in[0..i)), so out[0] = init.
 * *init is a host value of type t (NULL: the op's identity, 0 for the sum).  Temp storage as
 * for lcpp_scan_temp_bytes.  (The reference folds initial_value in once per warp in its first
 * tile, block/detail/block_scan_warp.h:223-236; with an init other than the op's identity
 * its sums differ from this definition, which follows CUB's.) */
int lcpp_scan_exclusive(lcpp_dtype t, lcpp_reduce_op op, void *temp, size_t temp_bytes, const void *in,
                        void *out, uint64_t n, const void *init, void *stream);
/* replaces DeviceScan::InclusiveScan(cmdlist, temp, d_in, d_out, num_items, scan_op,
 * initial_value), device_scan.h:147-178: out[i] = op(init, in[0..i]). */
int lcpp_scan_inclusive(lcpp_dtype t, lcpp_reduce_op op, void *temp, size_t temp_bytes, const void *in,
                        void *out, uint64_t n, const void *init, void *stream);
/* No counterpart in the reference.  For callers that cannot allocate (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * same result as lcpp_scan_exclusive_sum with no temp argument and no allocation.
 * Its look-back state lives in a fixed 512 KiB device array inside the library,
 * one per GPU, so n <= 1,342,177,280 for 4-byte types and n <= 335,544,320 for
 * 8-byte types (larger n: LCPP_ERR_SIZE_LIMIT).  Every call on a GPU shares that
 * GPU's array: calls that overlap in time on one GPU race (serialize them, e.g.
 * on one stream).  A look-back give-up is not reported (no temp to query). */
int lcpp_scan_exclusive_sum_noalloc(lcpp_dtype t, const void *in, void *out, uint64_t n, void *stream);

/* ---------------------------------------------------------------------
 * ScanByKey / ReduceByKey — device/device_scan.h, device/device_reduce.h
 * Segments are maximal runs of equal consecutive keys: element i is a
 * segment head when i == 0 or keys[i] != keys[i-1], compared in the key
 * type (floating keys: -0.0 == +0.0, NaN != NaN).  Keys and values: any
 * lcpp_dtype.  The reference takes arbitrary device functors; the C ABI
 * carries lcpp_reduce_op.  *init is a host value of the value type (NULL
 * means 0).
 * ------------------------------------------------------------------- */
/* replaces DeviceScan::GetScanByKeyTempStorageBytes<K,V>(num_items), device_scan.h:91-107 */
int lcpp_scan_by_key_temp_bytes(lcpp_dtype k, lcpp_dtype v, uint64_t n, size_t *bytes);
/* replaces DeviceScan::ExclusiveScanByKey(cmdlist, temp, d_keys_in, d_values_in, d_values_out,
 * scan_op, num_items, initial_value), device_scan.h:206-254:
 * out[i] = init at a head, else op(fold(vals_in[head..i)), init) */
int lcpp_scan_exclusive_by_key(lcpp_dtype k, lcpp_dtype v, lcpp_reduce_op op, void *temp,
                               size_t temp_bytes, const void *keys_in, const void *vals_in,
                               void *vals_out, uint64_t n, const void *init, void *stream);
/* replaces DeviceScan::InclusiveScanByKey, device_scan.h:256-303:
 * out[i] = op(fold(vals_in[head..i]), init).  (The reference overwrites every head with init,
 * scan_by_key.h:113-128; heads here get op(vals_in[head], init).) */
int lcpp_scan_inclusive_by_key(lcpp_dtype k, lcpp_dtype v, lcpp_reduce_op op, void *temp,
                               size_t temp_bytes, const void *keys_in, const void *vals_in,
                               void *vals_out, uint64_t n, const void *init, void *stream);
/* replaces DeviceScan::ExclusiveSumByKey, device_scan.h:306-322 (sum, init 0) */
int lcpp_scan_exclusive_sum_by_key(lcpp_dtype k, lcpp_dtype v, void *temp, size_t temp_bytes,
                                   const void *keys_in, const void *vals_in, void *vals_out,
                                   uint64_t n, void *stream);
/* replaces DeviceScan::InclusiveSumByKey, device_scan.h:324-339 (sum, init 0) */
int lcpp_scan_inclusive_sum_by_key(lcpp_dtype k, lcpp_dtype v, void *temp, size_t temp_bytes,
                                   const void *keys_in, const void *vals_in, void *vals_out,
                                   uint64_t n, void *stream);
/* replaces DeviceReduce::GetReduceByKeyTempStorageBytes<K,V>(num_elements), device_reduce.h:110-125.
 * Besides the reference's O(tiles) look-back state, the temp holds a run staging area of
 * about n * (sizeof K + sizeof V) / 64 bytes: tiles with at most 128 runs stage them instead
 * of waiting for the run count before the tile, and a second launch moves them.  n < 2^32. */
int lcpp_reduce_by_key_temp_bytes(lcpp_dtype k, lcpp_dtype v, uint64_t n, size_t *bytes);
/* replaces DeviceReduce::ReduceByKey(cmdlist, temp, d_keys_in, d_values_in, d_unique_out,
 * g_aggregates_out, g_num_runs_out, reduce_op, num_elements), device_reduce.h:277-318:
 * run r: unique_out[r] = its key, aggregates_out[r] = op-fold of its values;
 * *num_runs_out (device memory) = number of runs.  Outputs hold up to n entries.  n < 2^32. */
int lcpp_reduce_by_key(lcpp_dtype k, lcpp_dtype v, lcpp_reduce_op op, void *temp, size_t temp_bytes,
                       const void *keys_in, const void *vals_in, void *unique_out,
                       void *aggregates_out, uint32_t *num_runs_out, uint64_t n, void *stream);

/* ---------------------------------------------------------------------
 * DeviceRadixSort (onesweep, all key bits) — device/device_radix_sort.h
 * Keys: any lcpp_dtype (signed and floating keys are bit-twiddled as in
 * common/util_type.h:98-175; -0.0 and +0.0 compare equal).  Values: any
 * lcpp_dtype (moved as raw 4- or 8-byte words).  n < 2^32.
 * ------------------------------------------------------------------- */
/* replaces DeviceRadixSort::GetSortKeysTempStorageBytes<K>(num_items), device_radix_sort.h:118-122 */
int lcpp_radix_sort_keys_temp_bytes(lcpp_dtype k, uint64_t n, size_t *bytes);
/* replaces DeviceRadixSort::SortKeys(cmdlist, temp, keys_in, keys_out, num_items),
 * device_radix_sort.h:145-153 */
int lcpp_radix_sort_keys(lcpp_dtype k, void *temp, size_t temp_bytes, const void *keys_in,
                         void *keys_out, uint64_t n, void *stream);
/* replaces DeviceRadixSort::GetSortPairsTempStorageBytes<K,V>(num_items), device_radix_sort.h:83-115 */
int lcpp_radix_sort_pairs_temp_bytes(lcpp_dtype k, lcpp_dtype v, uint64_t n, size_t *bytes);
/* replaces DeviceRadixSort::SortPairs(cmdlist, temp, keys_in, keys_out, values_in,
 * values_out, num_items), device_radix_sort.h:129-143.  Stable. */
int lcpp_radix_sort_pairs(lcpp_dtype k, lcpp_dtype v, void *temp, size_t temp_bytes,
                          const void *keys_in, void *keys_out, const void *vals_in,
                          void *vals_out, uint64_t n, void *stream);
/* replaces DeviceRadixSort::SortKeysDescending(cmdlist, temp, keys_in, keys_out, num_items),
 * device_radix_sort.h:172-184: keys in non-increasing order (bit-inverted sort keys,
 * RadixSortTwiddle<true>, agent/radix_rank_sort_operations.h:124-155).  Temp storage as for
 * lcpp_radix_sort_keys_temp_bytes. */
int lcpp_radix_sort_keys_descending(lcpp_dtype k, void *temp, size_t temp_bytes, const void *keys_in,
                                    void *keys_out, uint64_t n, void *stream);
/* replaces DeviceRadixSort::SortPairsDescending, device_radix_sort.h:156-170.  Stable: equal
 * keys keep their input order.  Temp storage as for lcpp_radix_sort_pairs_temp_bytes. */
int lcpp_radix_sort_pairs_descending(lcpp_dtype k, lcpp_dtype v, void *temp, size_t temp_bytes,
                                     const void *keys_in, void *keys_out, const void *vals_in,
                                     void *vals_out, uint64_t n, void *stream);

/* No counterpart in the reference (whose MatchAny ranking, common/utils.h:273-324 and
 * block/block_radix_rank.h:254-280, has no alternative).  The onesweep ranks keys either with
 * returning LDS atomics, which are stable only if the LDS serves the lanes of one instruction
 * that hit one address in lane order (gfx950 does; no ISA document promises it), or with a
 * ballot match, stable by construction.  The first sort on each device runs an in-bounds
 * probe of that lane order (~70 us, synchronizes a private stream) and takes the atomic path
 * only if the probe sees no violation.  A first sort made while its stream is being captured
 * into a graph takes the match path.  Writes the path the sorts on the current device use:
 * 1 = LDS atomics, 2 = ballot match (running the probe if it has not run on this device). */
int lcpp_radix_sort_rank_path(int *path);
/* Test hook, process-wide: 0 = the probe's choice (default), 1 = force the LDS-atomic
 * ranking, 2 = force the ballot-match ranking.  Calls running concurrently see the same
 * setting. */
int lcpp_test_set_sort_rank_path(int mode);

/* ---------------------------------------------------------------------
 * DeviceSegmentReduce — device/device_segment_reduce.h
 * ------------------------------------------------------------------- */
/* replaces DeviceSegmentReduce::GetTempStorageBytes<T>(num_item), device_segment_reduce.h:71-75
 * (always 0) */
int lcpp_segment_reduce_temp_bytes(lcpp_dtype t, uint64_t num_segments, size_t *bytes);
/* replaces DeviceSegmentReduce::Sum(cmdlist, temp, d_in, d_out, num_segments, d_begin_offsets,
 * d_end_offsets), device_segment_reduce.h:125-135:
 * out[s] = 0 + sum(in[begin[s] .. end[s])); an empty segment (end <= begin) gives 0. */
int lcpp_segment_reduce_sum(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in,
                            void *out, uint64_t num_segments, const uint32_t *begin,
                            const uint32_t *end, void *stream);
/* replaces DeviceSegmentReduce::Reduce(cmdlist, temp, d_in, d_out, num_segments, d_begin_offsets,
 * d_end_offsets, reduce_op, initial_value), device_segment_reduce.h:94-107, and Min/Max
 * (:144-195, init max() / lowest()): out[s] = op(init, op-fold of in[begin[s] .. end[s]));
 * an empty segment gives init.  *init is a host value of type t (NULL: the op's identity). */
int lcpp_segment_reduce(lcpp_dtype t, lcpp_reduce_op op, void *temp, size_t temp_bytes, const void *in,
                        void *out, uint64_t num_segments, const uint32_t *begin, const uint32_t *end,
                        const void *init, void *stream);
/* replaces DeviceSegmentReduce::Reduce(cmdlist, temp, d_in, d_out, num_segments, segment_size,
 * reduce_op, initial_value), device_segment_reduce.h:109-123 (and the fixed-size Sum/Min/Max):
 * segment s = in[s * segment_size .. (s + 1) * segment_size).  num_segments * segment_size < 2^32. */
int lcpp_segment_reduce_fixed(lcpp_dtype t, lcpp_reduce_op op, void *temp, size_t temp_bytes,
                              const void *in, void *out, uint64_t num_segments, uint32_t segment_size,
                              const void *init, void *stream);
/* replaces DeviceSegmentReduce::GetArgTempStorageBytes<T>(num_item, num_segments),
 * device_segment_reduce.h:77-89 (always 0 here) */
int lcpp_segment_reduce_arg_temp_bytes(lcpp_dtype t, uint64_t n, uint64_t num_segments, size_t *bytes);
/* replaces DeviceSegmentReduce::Argmin (CSR offsets), device_segment_reduce.h:274-312:
 * out[s] = smallest value of the segment, index_out[s] = its index relative to begin[s] (ties:
 * the smallest index); an empty segment gives (max(), 1) (the reference writes 1 - begin[s]). */
int lcpp_segment_reduce_argmin(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                               uint32_t *index_out, uint64_t num_segments, const uint32_t *begin,
                               const uint32_t *end, void *stream);
/* replaces DeviceSegmentReduce::ArgMax (CSR offsets), device_segment_reduce.h:197-234: largest
 * value, ties to the largest index; an empty segment gives (lowest(), 1). */
int lcpp_segment_reduce_argmax(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                               uint32_t *index_out, uint64_t num_segments, const uint32_t *begin,
                               const uint32_t *end, void *stream);
/* replaces DeviceSegmentReduce::ArgMin(..., num_segments, segment_size), device_segment_reduce.h:314-349 */
int lcpp_segment_reduce_argmin_fixed(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                                     uint32_t *index_out, uint64_t num_segments, uint32_t segment_size,
                                     void *stream);
/* replaces DeviceSegmentReduce::ArgMax(..., num_segments, segment_size), device_segment_reduce.h:236-272 */
int lcpp_segment_reduce_argmax_fixed(lcpp_dtype t, void *temp, size_t temp_bytes, const void *in, void *out,
                                     uint32_t *index_out, uint64_t num_segments, uint32_t segment_size,
                                     void *stream);

/* ---------------------------------------------------------------------
 * Instrumentation (no counterpart in the reference).  When enabled, every
 * kernel launch made by the entry points above is bracketed by two HIP
 * events recorded on the launch stream, so per-kernel device time can be
 * read back.  Disabled by default; enabling it clears earlier records.
 * ------------------------------------------------------------------- */
int lcpp_profile_enable(int on);
/* Synchronizes the recorded events and returns the number of distinct kernel names. */
int lcpp_profile_count(void);
/* Kernel i: name (truncated to name_cap), number of launches, summed duration in ms. */
int lcpp_profile_get(int i, char *name, size_t name_cap, uint64_t *launches, double *total_ms);

#ifdef __cplusplus
}
#endif
#endif /* LCPP_AMD_H */
