// DeviceSegmentedRadixSort over the MI355X C-ABI (lcpp_hip_segmented_sort_*), with the reference's
// module shape (src/lcpp/device/device_segmented_radix_sort.h:14-39: template, create, temp queries
// forwarded to DeviceSegmentedSort) and entry points SortKeys / SortKeysDescending / SortPairs /
// SortPairsDescending, copy and DoubleBuffer forms, with begin_bit / end_bit (:41-205).  Each segment
// is sorted stably by the twiddled key bits [begin_bit, end_bit) (:216-243: radix order, so -0.0 sorts
// before +0.0); a DoubleBuffer sort of zero bits checks its arguments and records nothing (:67-71).
#pragma once

#include "lcpp/device/device_segmented_sort.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE = 256>
class DeviceSegmentedRadixSort : public LuisaModule {
  private:
    DeviceSegmentedSort<BLOCK_SIZE> m_segmented_sort;

  public:
    void create(Device& device) {
        m_segmented_sort.create(device);
        create_module(device);
    }

    template <NumericT KeyT>
    [[nodiscard]] static size_t GetSortKeysTempStorageBytes(size_t num_items) {
        return DeviceSegmentedSort<BLOCK_SIZE>::template GetSortKeysTempStorageBytes<KeyT>(num_items);
    }

    template <NumericT KeyT, NumericT ValueT>
    [[nodiscard]] static size_t GetSortPairsTempStorageBytes(size_t num_items) {
        return DeviceSegmentedSort<BLOCK_SIZE>::template GetSortPairsTempStorageBytes<KeyT, ValueT>(num_items);
    }

#define LCPP_SEGRADIX_KEYS_METHOD(NAME, DESC)                                                                      \
    template <NumericT KeyT>                                                                                       \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyT> keys_input,                   \
              BufferView<KeyT> keys_output, size_t num_items, size_t num_segments, BufferView<uint> begin_offsets, \
              BufferView<uint> end_offsets, uint begin_bit = 0u, uint end_bit = sizeof(KeyT) * 8u) {               \
        validate_bit_range<KeyT>(begin_bit, end_bit);                                                              \
        m_segmented_sort.record_keys(cmdlist, temp_storage, keys_input, keys_output, num_items, num_segments,      \
                                     begin_offsets, end_offsets, begin_bit, end_bit, DESC, 0,                      \
                                     "DeviceSegmentedRadixSort::" #NAME);                                          \
    }                                                                                                              \
    template <NumericT KeyT>                                                                                       \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyT>& keys, size_t num_items,     \
              size_t num_segments, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,                   \
              uint begin_bit = 0u, uint end_bit = sizeof(KeyT) * 8u) {                                             \
        validate_bit_range<KeyT>(begin_bit, end_bit);                                                              \
        if (begin_bit == end_bit) {                                                                                \
            m_segmented_sort.validate_key_double_buffer(keys, num_items, num_segments, begin_offsets, end_offsets); \
            return;                                                                                                \
        }                                                                                                          \
        m_segmented_sort.record_keys_db(cmdlist, temp_storage, keys, num_items, num_segments, begin_offsets,       \
                                        end_offsets, begin_bit, end_bit, DESC, 0,                                  \
                                        "DeviceSegmentedRadixSort::" #NAME);                                       \
    }
    LCPP_SEGRADIX_KEYS_METHOD(SortKeys, 0)
    LCPP_SEGRADIX_KEYS_METHOD(SortKeysDescending, 1)
#undef LCPP_SEGRADIX_KEYS_METHOD

#define LCPP_SEGRADIX_PAIRS_METHOD(NAME, DESC)                                                                     \
    template <NumericT KeyT, NumericT ValueT>                                                                      \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyT> keys_input,                   \
              BufferView<KeyT> keys_output, BufferView<ValueT> values_input, BufferView<ValueT> values_output,    \
              size_t num_items, size_t num_segments, BufferView<uint> begin_offsets, BufferView<uint> end_offsets, \
              uint begin_bit = 0u, uint end_bit = sizeof(KeyT) * 8u) {                                             \
        validate_bit_range<KeyT>(begin_bit, end_bit);                                                              \
        m_segmented_sort.record_pairs(cmdlist, temp_storage, keys_input, keys_output, values_input, values_output, \
                                      num_items, num_segments, begin_offsets, end_offsets, begin_bit, end_bit,     \
                                      DESC, 0, "DeviceSegmentedRadixSort::" #NAME);                                \
    }                                                                                                              \
    template <NumericT KeyT, NumericT ValueT>                                                                      \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyT>& keys,                       \
              DoubleBuffer<ValueT>& values, size_t num_items, size_t num_segments, BufferView<uint> begin_offsets, \
              BufferView<uint> end_offsets, uint begin_bit = 0u, uint end_bit = sizeof(KeyT) * 8u) {               \
        validate_bit_range<KeyT>(begin_bit, end_bit);                                                              \
        if (begin_bit == end_bit) {                                                                                \
            m_segmented_sort.validate_pair_double_buffers(keys, values, num_items, num_segments, begin_offsets,    \
                                                          end_offsets);                                            \
            return;                                                                                                \
        }                                                                                                          \
        m_segmented_sort.record_pairs_db(cmdlist, temp_storage, keys, values, num_items, num_segments,             \
                                         begin_offsets, end_offsets, begin_bit, end_bit, DESC, 0,                  \
                                         "DeviceSegmentedRadixSort::" #NAME);                                      \
    }
    LCPP_SEGRADIX_PAIRS_METHOD(SortPairs, 0)
    LCPP_SEGRADIX_PAIRS_METHOD(SortPairsDescending, 1)
#undef LCPP_SEGRADIX_PAIRS_METHOD

  private:
    template <NumericT KeyT>
    static void validate_bit_range(uint begin_bit, uint end_bit) {
        constexpr uint bit_width = static_cast<uint>(sizeof(KeyT) * 8u);
        LCPP_ASSERT(begin_bit <= end_bit, "DeviceSegmentedRadixSort begin_bit must not exceed end_bit.");
        LCPP_ASSERT(end_bit <= bit_width, "DeviceSegmentedRadixSort end_bit exceeds the key width.");
    }
};

}  // namespace luisa::parallel_primitive
