/*
 * lcpp/parallel_primitive.h — the reference's C++ host API over the C ABI.
 *
 * Same class, method and argument names as src/lcpp/device/device_*.h of
 * Ligo04/lc_parallel_primitive (umbrella header src/lcpp/parallel_primitive.h),
 * so code written against the reference switches by changing its types:
 *
 *   reference (LuisaCompute)                 here (HIP)
 *   ---------------------------------------  ------------------------------------
 *   Device / Stream                          Device{ordinal} / Stream{hipStream_t}
 *   CommandList& cmdlist                     CommandList{hipStream_t}: work is
 *                                            enqueued on the stream at the call
 *   BufferView<T>                            BufferView<T>{T* device pointer, count}
 *   BufferView<uint> temp_storage            caller-owned, Get*TempStorageBytes
 *
 * Errors: the reference asserts in debug builds (lcpp_check, runtime/core.h
 * :56-67) and ignores failures in release.  Here every call returns through
 * check(): debug builds print the status and abort, release builds keep the
 * last status, readable with last_status().  With a debug stream
 * (create(device, &stream)), as the reference's lcpp_check commits and
 * synchronizes, every call is synchronized and the device status word in its
 * temp storage is read (lcpp_temp_status), so a look-back wait that gave up
 * (LCPP_ERR_LOOKBACK_TIMEOUT) or a failed kernel (LCPP_ERR_HIP) is reported
 * by the call that caused it; this also holds in release builds.
 *
 * Template parameters <BLOCK_SIZE, WARP_NUMS, ITEMS_PER_THREAD> are accepted
 * for source compatibility; the geometry is fixed per dtype inside the
 * library (64-lane waves, tuned for gfx950).
 */
#ifndef LCPP_PARALLEL_PRIMITIVE_H
#define LCPP_PARALLEL_PRIMITIVE_H

#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <limits>
#include <type_traits>

#include "../lcpp_amd.h"

namespace luisa::parallel_primitive {

using uint = unsigned int;

template <class T>
struct BufferView {
    T *ptr = nullptr;
    size_t count = 0;
    BufferView() = default;
    BufferView(T *p, size_t n) : ptr(p), count(n) {}
    [[nodiscard]] size_t size() const noexcept { return count; }
    [[nodiscard]] size_t size_bytes() const noexcept { return count * sizeof(T); }
    [[nodiscard]] T *data() const noexcept { return ptr; }
    [[nodiscard]] BufferView subview(size_t offset, size_t n) const noexcept { return {ptr + offset, n}; }
};

struct Device {
    int ordinal = 0;
};
struct Stream {
    void *handle = nullptr; /* hipStream_t */
};
struct CommandList {
    void *stream = nullptr; /* hipStream_t; work is enqueued here at the call */
};

template <class T>
constexpr lcpp_dtype dtype_of()
{
    using U = std::remove_cv_t<T>;
    if constexpr (std::is_same_v<U, float>) return LCPP_FLOAT32;
    else if constexpr (std::is_same_v<U, double>) return LCPP_FLOAT64;
    else if constexpr (std::is_integral_v<U> && sizeof(U) == 4 && std::is_signed_v<U>) return LCPP_INT32;
    else if constexpr (std::is_integral_v<U> && sizeof(U) == 4) return LCPP_UINT32;
    else if constexpr (std::is_integral_v<U> && sizeof(U) == 8 && std::is_signed_v<U>) return LCPP_INT64;
    else if constexpr (std::is_integral_v<U> && sizeof(U) == 8) return LCPP_UINT64;
    else static_assert(sizeof(U) == 0, "NumericT: 4- or 8-byte integer or floating type");
}

/* Reduction operators and element transforms TransformReduce can name.  The
 * reference's SumOp / MinOp / MaxOp / IdentityOp are in
 * common/thread_operators.h:49-80; its TransformReduce accepts any device
 * functor, which a prebuilt library behind a C ABI cannot compile, so the set
 * here is fixed (see lcpp_reduce_op / lcpp_transform). */
struct SumOp {};
struct MinOp {};
struct MaxOp {};
struct IdentityOp {};
struct NegateOp {};
struct AbsOp {};
struct SquareOp {};

template <class Op>
constexpr lcpp_reduce_op reduce_op_of()
{
    if constexpr (std::is_same_v<Op, SumOp>) return LCPP_OP_SUM;
    else if constexpr (std::is_same_v<Op, MinOp>) return LCPP_OP_MIN;
    else if constexpr (std::is_same_v<Op, MaxOp>) return LCPP_OP_MAX;
    else static_assert(sizeof(Op) == 0, "reduce_op / scan_op must be SumOp, MinOp or MaxOp");
}
template <class Xf>
constexpr lcpp_transform transform_of()
{
    if constexpr (std::is_same_v<Xf, IdentityOp>) return LCPP_XFORM_IDENTITY;
    else if constexpr (std::is_same_v<Xf, NegateOp>) return LCPP_XFORM_NEGATE;
    else if constexpr (std::is_same_v<Xf, AbsOp>) return LCPP_XFORM_ABS;
    else if constexpr (std::is_same_v<Xf, SquareOp>) return LCPP_XFORM_SQUARE;
    else static_assert(sizeof(Xf) == 0, "TransformReduce: transform_op must be IdentityOp, NegateOp, AbsOp or SquareOp");
}

/* bytes -> count of uint words, as the reference's bytes_to_uint_count (common/utils.h:166-169) */
inline size_t bytes_to_uint_count(size_t bytes) { return (bytes + sizeof(uint) - 1) / sizeof(uint); }

namespace details {
constexpr size_t BLOCK_SIZE = 256;
constexpr size_t WARP_SIZE = 64;
constexpr size_t ITEMS_PER_THREAD = 16;
}  // namespace details

class LuisaModule {
  public:
    void create(Device &device, Stream *debug_stream = nullptr)
    {
        m_device = device;
        m_debug_stream = debug_stream;
        m_created = true;
    }
    [[nodiscard]] int last_status() const noexcept { return m_last_status; }

  protected:
    // `stream` / `temp` are the call's stream and temp storage; without a
    // debug stream they are not touched.
    void check(int status, const char *what, void *stream, BufferView<uint> temp = {})
    {
        if (status == LCPP_OK && m_debug_stream) status = lcpp_temp_status(temp.data(), temp.size_bytes(), stream);
        m_last_status = status;
#ifndef NDEBUG
        if (status != LCPP_OK) {
            std::fprintf(stderr, "lcpp: %s failed: %s\n", what, lcpp_status_string(status));
            std::abort();
        }
#else
        (void)what;
#endif
    }
    Device m_device{};
    Stream *m_debug_stream = nullptr;
    bool m_created = false;
    int m_last_status = LCPP_OK;
};

/* device/device_reduce.h:37-348 */
template <size_t BLOCK_SIZE = details::BLOCK_SIZE, size_t WARP_NUMS = details::WARP_SIZE,
          size_t ITEMS_PER_THREAD = details::ITEMS_PER_THREAD>
class DeviceReduce : public LuisaModule {
  public:
    template <class T>
    static size_t GetTempStorageBytes(size_t num_item)
    {
        size_t b = 0;
        lcpp_reduce_temp_bytes(dtype_of<T>(), num_item, &b);
        return b;
    }
    template <class T>
    void Sum(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out, size_t num_item)
    {
        check(lcpp_reduce_sum(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(), d_out.data(),
                              num_item, cmdlist.stream),
              "DeviceReduce::Sum", cmdlist.stream, temp_storage);
    }
    template <class T>
    void Min(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out, size_t num_item)
    {
        check(lcpp_reduce_min(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(), d_out.data(),
                              num_item, cmdlist.stream),
              "DeviceReduce::Min", cmdlist.stream, temp_storage);
    }
    template <class T>
    void Max(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out, size_t num_item)
    {
        check(lcpp_reduce_max(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(), d_out.data(),
                              num_item, cmdlist.stream),
              "DeviceReduce::Max", cmdlist.stream, temp_storage);
    }
    /* device/device_reduce.h:94-107 */
    template <class T>
    static size_t GetArgTempStorageBytes(size_t num_item)
    {
        size_t b = 0;
        lcpp_reduce_arg_temp_bytes(dtype_of<T>(), num_item, &b);
        return b;
    }
    /* device/device_reduce.h:187-227 */
    template <class T>
    void ArgMin(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, size_t num_item)
    {
        check(lcpp_reduce_argmin(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(),
                                 d_out.data(), d_index_out.data(), num_item, cmdlist.stream),
              "DeviceReduce::ArgMin", cmdlist.stream, temp_storage);
    }
    /* device/device_reduce.h:229-272 */
    template <class T>
    void ArgMax(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, size_t num_item)
    {
        check(lcpp_reduce_argmax(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(),
                                 d_out.data(), d_index_out.data(), num_item, cmdlist.stream),
              "DeviceReduce::ArgMax", cmdlist.stream, temp_storage);
    }
    /* device/device_reduce.h:131-147 (reduce_op: SumOp, MinOp or MaxOp):
     * d_out[0] = reduce_op(initial_value, reduce_op over d_in[0..num_item)) */
    template <class T, class ReduceOp>
    void Reduce(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                size_t num_item, ReduceOp, T initial_value)
    {
        check(lcpp_reduce_transform(dtype_of<T>(), reduce_op_of<ReduceOp>(), LCPP_XFORM_IDENTITY,
                                    temp_storage.data(), temp_storage.size_bytes(), d_in.data(), d_out.data(),
                                    num_item, &initial_value, cmdlist.stream),
              "DeviceReduce::Reduce", cmdlist.stream, temp_storage);
    }
    /* device/device_reduce.h:331-348 */
    template <class T, class ReduceOp, class TransformOp>
    void TransformReduce(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                         size_t num_item, ReduceOp, TransformOp, T init)
    {
        check(lcpp_reduce_transform(dtype_of<T>(), reduce_op_of<ReduceOp>(), transform_of<TransformOp>(),
                                    temp_storage.data(), temp_storage.size_bytes(), d_in.data(), d_out.data(),
                                    num_item, &init, cmdlist.stream),
              "DeviceReduce::TransformReduce", cmdlist.stream, temp_storage);
    }
    /* device/device_reduce.h:110-125 */
    template <class KeyType, class ValueType>
    static size_t GetReduceByKeyTempStorageBytes(size_t num_elements)
    {
        size_t b = 0;
        lcpp_reduce_by_key_temp_bytes(dtype_of<KeyType>(), dtype_of<ValueType>(), num_elements, &b);
        return b;
    }
    /* device/device_reduce.h:277-318 (reduce_op: SumOp, MinOp or MaxOp) */
    template <class KeyType, class ValueType, class ReduceOp>
    void ReduceByKey(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                     BufferView<ValueType> d_values_in, BufferView<KeyType> d_unique_out,
                     BufferView<ValueType> g_aggregates_out, BufferView<uint> g_num_runs_out, ReduceOp,
                     size_t num_elements)
    {
        check(lcpp_reduce_by_key(dtype_of<KeyType>(), dtype_of<ValueType>(), reduce_op_of<ReduceOp>(),
                                 temp_storage.data(), temp_storage.size_bytes(), d_keys_in.data(), d_values_in.data(),
                                 d_unique_out.data(), g_aggregates_out.data(), g_num_runs_out.data(), num_elements,
                                 cmdlist.stream),
              "DeviceReduce::ReduceByKey", cmdlist.stream, temp_storage);
    }
};

/* device/device_scan.h:33-339 */
template <size_t BLOCK_SIZE = details::BLOCK_SIZE, size_t WARP_NUMS = details::WARP_SIZE,
          size_t ITEMS_PER_THREAD = details::ITEMS_PER_THREAD>
class DeviceScan : public LuisaModule {
  public:
    template <class T>
    static size_t GetTempStorageBytes(size_t num_items)
    {
        size_t b = 0;
        lcpp_scan_temp_bytes(dtype_of<T>(), num_items, &b);
        return b;
    }
    /* device/device_scan.h:114-145 (scan_op: SumOp, MinOp or MaxOp):
     * d_out[i] = scan_op(initial_value, d_in[0..i)) */
    template <class T, class ScanOp>
    void ExclusiveScan(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                       size_t num_items, ScanOp, T initial_value)
    {
        check(lcpp_scan_exclusive(dtype_of<T>(), reduce_op_of<ScanOp>(), temp_storage.data(),
                                  temp_storage.size_bytes(), d_in.data(), d_out.data(), num_items, &initial_value,
                                  cmdlist.stream),
              "DeviceScan::ExclusiveScan", cmdlist.stream, temp_storage);
    }
    /* device/device_scan.h:147-178: d_out[i] = scan_op(initial_value, d_in[0..i]) */
    template <class T, class ScanOp>
    void InclusiveScan(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                       size_t num_items, ScanOp, T initial_value)
    {
        check(lcpp_scan_inclusive(dtype_of<T>(), reduce_op_of<ScanOp>(), temp_storage.data(),
                                  temp_storage.size_bytes(), d_in.data(), d_out.data(), num_items, &initial_value,
                                  cmdlist.stream),
              "DeviceScan::InclusiveScan", cmdlist.stream, temp_storage);
    }
    template <class T>
    void ExclusiveSum(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                      size_t num_items)
    {
        check(lcpp_scan_exclusive_sum(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(),
                                      d_out.data(), num_items, cmdlist.stream),
              "DeviceScan::ExclusiveSum", cmdlist.stream, temp_storage);
    }
    template <class T>
    void InclusiveSum(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                      size_t num_items)
    {
        check(lcpp_scan_inclusive_sum(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(),
                                      d_out.data(), num_items, cmdlist.stream),
              "DeviceScan::InclusiveSum", cmdlist.stream, temp_storage);
    }
    /* device/device_scan.h:91-107 */
    template <class KeyType, class ValueType>
    static size_t GetScanByKeyTempStorageBytes(size_t num_items)
    {
        size_t b = 0;
        lcpp_scan_by_key_temp_bytes(dtype_of<KeyType>(), dtype_of<ValueType>(), num_items, &b);
        return b;
    }
    /* device/device_scan.h:206-254 (scan_op: SumOp, MinOp or MaxOp) */
    template <class KeyType, class ValueType, class ScanOp>
    void ExclusiveScanByKey(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                            BufferView<ValueType> d_values_in, BufferView<ValueType> d_values_out, ScanOp,
                            size_t num_items, ValueType initial_value)
    {
        check(lcpp_scan_exclusive_by_key(dtype_of<KeyType>(), dtype_of<ValueType>(), reduce_op_of<ScanOp>(),
                                         temp_storage.data(), temp_storage.size_bytes(), d_keys_in.data(),
                                         d_values_in.data(), d_values_out.data(), num_items, &initial_value,
                                         cmdlist.stream),
              "DeviceScan::ExclusiveScanByKey", cmdlist.stream, temp_storage);
    }
    /* device/device_scan.h:256-303 (heads get scan_op(value, init); the reference gives init) */
    template <class KeyType, class ValueType, class ScanOp>
    void InclusiveScanByKey(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                            BufferView<ValueType> d_values_in, BufferView<ValueType> d_values_out, ScanOp,
                            size_t num_items, ValueType initial_value)
    {
        check(lcpp_scan_inclusive_by_key(dtype_of<KeyType>(), dtype_of<ValueType>(), reduce_op_of<ScanOp>(),
                                         temp_storage.data(), temp_storage.size_bytes(), d_keys_in.data(),
                                         d_values_in.data(), d_values_out.data(), num_items, &initial_value,
                                         cmdlist.stream),
              "DeviceScan::InclusiveScanByKey", cmdlist.stream, temp_storage);
    }
    /* device/device_scan.h:306-322 */
    template <class T>
    void ExclusiveSumByKey(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_keys_in,
                           BufferView<T> d_values_in, BufferView<T> d_values_out, size_t num_items)
    {
        check(lcpp_scan_exclusive_sum_by_key(dtype_of<T>(), dtype_of<T>(), temp_storage.data(),
                                             temp_storage.size_bytes(), d_keys_in.data(), d_values_in.data(),
                                             d_values_out.data(), num_items, cmdlist.stream),
              "DeviceScan::ExclusiveSumByKey", cmdlist.stream, temp_storage);
    }
    /* device/device_scan.h:324-339 */
    template <class T>
    void InclusiveSumByKey(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_keys_in,
                           BufferView<T> d_values_in, BufferView<T> d_values_out, size_t num_items)
    {
        check(lcpp_scan_inclusive_sum_by_key(dtype_of<T>(), dtype_of<T>(), temp_storage.data(),
                                             temp_storage.size_bytes(), d_keys_in.data(), d_values_in.data(),
                                             d_values_out.data(), num_items, cmdlist.stream),
              "DeviceScan::InclusiveSumByKey", cmdlist.stream, temp_storage);
    }
};

/* device/device_radix_sort.h:37-184 */
template <size_t BLOCK_SIZE = details::BLOCK_SIZE, size_t WARP_NUMS = details::WARP_SIZE,
          size_t ITEMS_PER_THREAD = details::ITEMS_PER_THREAD>
class DeviceRadixSort : public LuisaModule {
  public:
    template <class KeyType, class ValueType>
    static size_t GetSortPairsTempStorageBytes(uint num_items)
    {
        size_t b = 0;
        lcpp_radix_sort_pairs_temp_bytes(dtype_of<KeyType>(), dtype_of<ValueType>(), num_items, &b);
        return b;
    }
    template <class KeyType>
    static size_t GetSortKeysTempStorageBytes(uint num_items)
    {
        size_t b = 0;
        lcpp_radix_sort_keys_temp_bytes(dtype_of<KeyType>(), num_items, &b);
        return b;
    }
    template <class KeyType, class ValueType>
    void SortPairs(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                   BufferView<KeyType> d_keys_out, BufferView<ValueType> d_values_in,
                   BufferView<ValueType> d_values_out, uint num_items)
    {
        check(lcpp_radix_sort_pairs(dtype_of<KeyType>(), dtype_of<ValueType>(), temp_storage.data(),
                                    temp_storage.size_bytes(), d_keys_in.data(), d_keys_out.data(),
                                    d_values_in.data(), d_values_out.data(), num_items, cmdlist.stream),
              "DeviceRadixSort::SortPairs", cmdlist.stream, temp_storage);
    }
    template <class KeyType>
    void SortKeys(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                  BufferView<KeyType> d_keys_out, uint num_items)
    {
        check(lcpp_radix_sort_keys(dtype_of<KeyType>(), temp_storage.data(), temp_storage.size_bytes(),
                                   d_keys_in.data(), d_keys_out.data(), num_items, cmdlist.stream),
              "DeviceRadixSort::SortKeys", cmdlist.stream, temp_storage);
    }
    /* device/device_radix_sort.h:156-170 */
    template <class KeyType, class ValueType>
    void SortPairsDescending(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                             BufferView<KeyType> d_keys_out, BufferView<ValueType> d_values_in,
                             BufferView<ValueType> d_values_out, uint num_items)
    {
        check(lcpp_radix_sort_pairs_descending(dtype_of<KeyType>(), dtype_of<ValueType>(), temp_storage.data(),
                                               temp_storage.size_bytes(), d_keys_in.data(), d_keys_out.data(),
                                               d_values_in.data(), d_values_out.data(), num_items, cmdlist.stream),
              "DeviceRadixSort::SortPairsDescending", cmdlist.stream, temp_storage);
    }
    /* device/device_radix_sort.h:172-184 */
    template <class KeyType>
    void SortKeysDescending(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                            BufferView<KeyType> d_keys_out, uint num_items)
    {
        check(lcpp_radix_sort_keys_descending(dtype_of<KeyType>(), temp_storage.data(), temp_storage.size_bytes(),
                                              d_keys_in.data(), d_keys_out.data(), num_items, cmdlist.stream),
              "DeviceRadixSort::SortKeysDescending", cmdlist.stream, temp_storage);
    }
};

/* device/device_segment_reduce.h:26-349.  Overloads take CSR begin/end offsets or a fixed
 * segment_size, as the reference's do. */
template <size_t BLOCK_SIZE = details::BLOCK_SIZE, size_t WARP_NUMS = details::WARP_SIZE,
          size_t ITEMS_PER_THREAD = details::ITEMS_PER_THREAD>
class DeviceSegmentReduce : public LuisaModule {
  public:
    template <class T>
    static size_t GetTempStorageBytes(size_t /*num_item*/)
    {
        size_t b = 0;
        lcpp_segment_reduce_temp_bytes(dtype_of<T>(), 0, &b);
        return b;
    }
    /* device/device_segment_reduce.h:77-89 */
    template <class T>
    static size_t GetArgTempStorageBytes(size_t num_item, size_t num_segments)
    {
        size_t b = 0;
        lcpp_segment_reduce_arg_temp_bytes(dtype_of<T>(), num_item, num_segments, &b);
        return b;
    }
    /* device/device_segment_reduce.h:94-107 (reduce_op: SumOp, MinOp or MaxOp) */
    template <class T, class ReduceOp>
    void Reduce(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                uint num_segments, BufferView<uint> d_begin_offsets, BufferView<uint> d_end_offsets, ReduceOp,
                T initial_value)
    {
        check(lcpp_segment_reduce(dtype_of<T>(), reduce_op_of<ReduceOp>(), temp_storage.data(),
                                  temp_storage.size_bytes(), d_in.data(), d_out.data(), num_segments,
                                  d_begin_offsets.data(), d_end_offsets.data(), &initial_value, cmdlist.stream),
              "DeviceSegmentReduce::Reduce", cmdlist.stream);
    }
    /* device/device_segment_reduce.h:109-123 */
    template <class T, class ReduceOp>
    void Reduce(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                uint num_segments, uint segment_size, ReduceOp, T initial_value)
    {
        check(lcpp_segment_reduce_fixed(dtype_of<T>(), reduce_op_of<ReduceOp>(), temp_storage.data(),
                                        temp_storage.size_bytes(), d_in.data(), d_out.data(), num_segments,
                                        segment_size, &initial_value, cmdlist.stream),
              "DeviceSegmentReduce::Reduce", cmdlist.stream);
    }
    template <class T>
    void Sum(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             uint num_segments, BufferView<uint> d_begin_offsets, BufferView<uint> d_end_offsets)
    {
        check(lcpp_segment_reduce_sum(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(),
                                      d_out.data(), num_segments, d_begin_offsets.data(), d_end_offsets.data(),
                                      cmdlist.stream),
              "DeviceSegmentReduce::Sum", cmdlist.stream);
    }
    template <class T>
    void Sum(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             uint num_segments, uint segment_size)
    {
        Reduce(cmdlist, temp_storage, d_in, d_out, num_segments, segment_size, SumOp{}, T(0));
    }
    template <class T>
    void Min(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             uint num_segments, BufferView<uint> d_begin_offsets, BufferView<uint> d_end_offsets)
    {
        Reduce(cmdlist, temp_storage, d_in, d_out, num_segments, d_begin_offsets, d_end_offsets, MinOp{},
               std::numeric_limits<T>::max());
    }
    template <class T>
    void Min(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             uint num_segments, uint segment_size)
    {
        Reduce(cmdlist, temp_storage, d_in, d_out, num_segments, segment_size, MinOp{}, std::numeric_limits<T>::max());
    }
    template <class T>
    void Max(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             uint num_segments, BufferView<uint> d_begin_offsets, BufferView<uint> d_end_offsets)
    {
        Reduce(cmdlist, temp_storage, d_in, d_out, num_segments, d_begin_offsets, d_end_offsets, MaxOp{},
               std::numeric_limits<T>::lowest());
    }
    template <class T>
    void Max(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             uint num_segments, uint segment_size)
    {
        Reduce(cmdlist, temp_storage, d_in, d_out, num_segments, segment_size, MaxOp{},
               std::numeric_limits<T>::lowest());
    }
    /* device/device_segment_reduce.h:197-234 */
    template <class T>
    void ArgMax(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, uint num_segments, BufferView<uint> d_begin_offsets,
                BufferView<uint> d_end_offsets)
    {
        check(lcpp_segment_reduce_argmax(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(),
                                         d_out.data(), d_index_out.data(), num_segments, d_begin_offsets.data(),
                                         d_end_offsets.data(), cmdlist.stream),
              "DeviceSegmentReduce::ArgMax", cmdlist.stream);
    }
    /* device/device_segment_reduce.h:236-272 */
    template <class T>
    void ArgMax(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, uint num_segments, uint segment_size)
    {
        check(lcpp_segment_reduce_argmax_fixed(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(),
                                               d_in.data(), d_out.data(), d_index_out.data(), num_segments,
                                               segment_size, cmdlist.stream),
              "DeviceSegmentReduce::ArgMax", cmdlist.stream);
    }
    /* device/device_segment_reduce.h:274-312 (the reference spells this overload Argmin) */
    template <class T>
    void ArgMin(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, uint num_segments, BufferView<uint> d_begin_offsets,
                BufferView<uint> d_end_offsets)
    {
        check(lcpp_segment_reduce_argmin(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(), d_in.data(),
                                         d_out.data(), d_index_out.data(), num_segments, d_begin_offsets.data(),
                                         d_end_offsets.data(), cmdlist.stream),
              "DeviceSegmentReduce::ArgMin", cmdlist.stream);
    }
    template <class T>
    void Argmin(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, uint num_segments, BufferView<uint> d_begin_offsets,
                BufferView<uint> d_end_offsets)
    {
        ArgMin(cmdlist, temp_storage, d_in, d_out, d_index_out, num_segments, d_begin_offsets, d_end_offsets);
    }
    /* device/device_segment_reduce.h:314-349 */
    template <class T>
    void ArgMin(CommandList &cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, uint num_segments, uint segment_size)
    {
        check(lcpp_segment_reduce_argmin_fixed(dtype_of<T>(), temp_storage.data(), temp_storage.size_bytes(),
                                               d_in.data(), d_out.data(), d_index_out.data(), num_segments,
                                               segment_size, cmdlist.stream),
              "DeviceSegmentReduce::ArgMin", cmdlist.stream);
    }
};

}  // namespace luisa::parallel_primitive

#endif /* LCPP_PARALLEL_PRIMITIVE_H */
