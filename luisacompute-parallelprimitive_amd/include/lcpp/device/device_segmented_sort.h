// DeviceSegmentedSort over the MI355X C-ABI (lcpp_hip_segmented_sort_*), with the reference's module
// shape (src/lcpp/device/device_segmented_sort.h:24-75: template, create, GetSortKeysTempStorageBytes,
// GetSortPairsTempStorageBytes) and entry points SortKeys / SortKeysDescending / StableSortKeys /
// StableSortKeysDescending and the SortPairs family, copy and DoubleBuffer forms (:77-505), checked like
// validate_key_views / validate_pair_views / validate_key_double_buffer (:566-720).  Every sort is stable
// and orders by the key values (lhs < rhs, or lhs > rhs descending: -0.0 and +0.0 are equal).
//
// DoubleBuffer forms: the selector is flipped ceil(log2 num_items) times when the call is recorded, as
// the reference does (:234-250), so after commit `keys.current()` holds the sorted keys.  The forms that
// take a user comparator (`const Callable<bool(KeyT, KeyT)>&`, :107-162) take device lambdas and have no
// counterpart here.
#pragma once

#include <limits>
#include <string>

#include "lcpp/device/segsort_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE>
class DeviceSegmentedRadixSort;

template <size_t BLOCK_SIZE = 256>
class DeviceSegmentedSort : public LuisaModule {
    template <size_t>
    friend class DeviceSegmentedRadixSort;

  public:
    void create(Device& device) { create_module(device); }

    template <NumericT KeyT>
    [[nodiscard]] static size_t GetSortKeysTempStorageBytes(size_t num_items) {
        static_assert(detail::segsort_key_ok<KeyT>, "DeviceSegmentedSort keys: 4- or 8-byte numbers");
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DeviceSegmentedSort.");
        return lcpp_hip_segmented_sort_keys_temp_bytes(num_items, sizeof(KeyT));
    }

    template <NumericT KeyT, NumericT ValueT>
    [[nodiscard]] static size_t GetSortPairsTempStorageBytes(size_t num_items) {
        static_assert(detail::segsort_key_ok<KeyT>, "DeviceSegmentedSort keys: 4- or 8-byte numbers");
        static_assert(detail::segsort_value_ok<ValueT>, "DeviceSegmentedSort values: 4- or 8-byte types");
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DeviceSegmentedSort.");
        return lcpp_hip_segmented_sort_pairs_temp_bytes(num_items, sizeof(KeyT), sizeof(ValueT));
    }

#define LCPP_SEGSORT_KEYS_METHOD(NAME, DESC)                                                                       \
    template <NumericT KeyT>                                                                                       \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyT> keys_input,                   \
              BufferView<KeyT> keys_output, size_t num_items, size_t num_segments, BufferView<uint> begin_offsets, \
              BufferView<uint> end_offsets) {                                                                      \
        record_keys(cmdlist, temp_storage, keys_input, keys_output, num_items, num_segments, begin_offsets,        \
                    end_offsets, 0u, sizeof(KeyT) * 8u, DESC, 1, "DeviceSegmentedSort::" #NAME);                  \
    }                                                                                                              \
    template <NumericT KeyT>                                                                                       \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyT>& keys, size_t num_items,     \
              size_t num_segments, BufferView<uint> begin_offsets, BufferView<uint> end_offsets) {                 \
        record_keys_db(cmdlist, temp_storage, keys, num_items, num_segments, begin_offsets, end_offsets, 0u,       \
                       sizeof(KeyT) * 8u, DESC, 1, "DeviceSegmentedSort::" #NAME);                                 \
    }
    LCPP_SEGSORT_KEYS_METHOD(SortKeys, 0)
    LCPP_SEGSORT_KEYS_METHOD(SortKeysDescending, 1)
    LCPP_SEGSORT_KEYS_METHOD(StableSortKeys, 0)
    LCPP_SEGSORT_KEYS_METHOD(StableSortKeysDescending, 1)
#undef LCPP_SEGSORT_KEYS_METHOD

#define LCPP_SEGSORT_PAIRS_METHOD(NAME, DESC)                                                                      \
    template <NumericT KeyT, NumericT ValueT>                                                                      \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyT> keys_input,                   \
              BufferView<KeyT> keys_output, BufferView<ValueT> values_input, BufferView<ValueT> values_output,    \
              size_t num_items, size_t num_segments, BufferView<uint> begin_offsets,                               \
              BufferView<uint> end_offsets) {                                                                      \
        record_pairs(cmdlist, temp_storage, keys_input, keys_output, values_input, values_output, num_items,       \
                     num_segments, begin_offsets, end_offsets, 0u, sizeof(KeyT) * 8u, DESC, 1,                    \
                     "DeviceSegmentedSort::" #NAME);                                                               \
    }                                                                                                              \
    template <NumericT KeyT, NumericT ValueT>                                                                      \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyT>& keys,                       \
              DoubleBuffer<ValueT>& values, size_t num_items, size_t num_segments, BufferView<uint> begin_offsets, \
              BufferView<uint> end_offsets) {                                                                      \
        record_pairs_db(cmdlist, temp_storage, keys, values, num_items, num_segments, begin_offsets, end_offsets,  \
                        0u, sizeof(KeyT) * 8u, DESC, 1, "DeviceSegmentedSort::" #NAME);                            \
    }
    LCPP_SEGSORT_PAIRS_METHOD(SortPairs, 0)
    LCPP_SEGSORT_PAIRS_METHOD(SortPairsDescending, 1)
    LCPP_SEGSORT_PAIRS_METHOD(StableSortPairs, 0)
    LCPP_SEGSORT_PAIRS_METHOD(StableSortPairsDescending, 1)
#undef LCPP_SEGSORT_PAIRS_METHOD

  private:
    void validate_common(size_t num_items, size_t num_segments, BufferView<uint> begin_offsets,
                         BufferView<uint> end_offsets) const {
        LCPP_ASSERT(m_created, "DeviceSegmentedSort::create must be called before dispatch.");
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DeviceSegmentedSort.");
        LCPP_ASSERT(num_segments <= std::numeric_limits<uint>::max(), "Too many segments for DeviceSegmentedSort.");
        LCPP_ASSERT(begin_offsets.size() >= num_segments, "DeviceSegmentedSort begin-offset view is too small.");
        LCPP_ASSERT(end_offsets.size() >= num_segments, "DeviceSegmentedSort end-offset view is too small.");
    }

    template <typename T>
    static void validate_double_buffer(const DoubleBuffer<T>& buffer, size_t num_items, const char* name) {
        LCPP_ASSERT(buffer.selector == 0 || buffer.selector == 1,
                    std::string("DeviceSegmentedSort ") + name + " DoubleBuffer selector must be 0 or 1.");
        LCPP_ASSERT(buffer.d_buffer[0].size() >= num_items,
                    std::string("DeviceSegmentedSort ") + name + " DoubleBuffer slot 0 is too small.");
        LCPP_ASSERT(buffer.d_buffer[1].size() >= num_items,
                    std::string("DeviceSegmentedSort ") + name + " DoubleBuffer slot 1 is too small.");
    }

    template <typename KeyT>
    void validate_key_double_buffer(const DoubleBuffer<KeyT>& keys, size_t num_items, size_t num_segments,
                                    BufferView<uint> begin_offsets, BufferView<uint> end_offsets) const {
        validate_common(num_items, num_segments, begin_offsets, end_offsets);
        validate_double_buffer(keys, num_items, "key");
    }

    template <typename KeyT, typename ValueT>
    void validate_pair_double_buffers(const DoubleBuffer<KeyT>& keys, const DoubleBuffer<ValueT>& values,
                                      size_t num_items, size_t num_segments, BufferView<uint> begin_offsets,
                                      BufferView<uint> end_offsets) const {
        validate_key_double_buffer(keys, num_items, num_segments, begin_offsets, end_offsets);
        validate_double_buffer(values, num_items, "value");
        LCPP_ASSERT(keys.selector == values.selector,
                    "DeviceSegmentedSort key and value DoubleBuffer selectors must match.");
    }

    template <typename KeyT>
    void record_keys(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyT> keys_input,
                     BufferView<KeyT> keys_output, size_t num_items, size_t num_segments,
                     BufferView<uint> begin_offsets, BufferView<uint> end_offsets, uint begin_bit, uint end_bit,
                     int desc, int value_order, const char* what) {
        static_assert(detail::segsort_key_ok<KeyT>, "DeviceSegmentedSort keys: 4- or 8-byte numbers");
        validate_common(num_items, num_segments, begin_offsets, end_offsets);
        if (num_items == 0u || num_segments == 0u) return;
        LCPP_ASSERT(keys_input.size() >= num_items, "DeviceSegmentedSort key input view is too small.");
        LCPP_ASSERT(keys_output.size() >= num_items, "DeviceSegmentedSort key output view is too small.");
        if (num_items > 1u)
            LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetSortKeysTempStorageBytes<KeyT>(num_items)),
                        "DeviceSegmentedSort temporary storage is too small.");
        using A = detail::by_key_abi_t<KeyT>;
        void* temp = temp_storage.data();
        const size_t tb = temp_storage.size_bytes();
        const A* kin = reinterpret_cast<const A*>(keys_input.data());
        A* kout = reinterpret_cast<A*>(keys_output.data());
        const uint32_t* b = begin_offsets.data();
        const uint32_t* e = end_offsets.data();
        cmdlist << [=](hipStream_t s) {
            luisa::detail::abi_check(detail::segsort_keys(temp, tb, kin, kout, num_items, num_segments, b, e,
                                                          begin_bit, end_bit, desc, value_order,
                                                          detail::stream_ptr(s)),
                                     what);
        };
    }

    template <typename KeyT, typename ValueT>
    void record_pairs(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyT> keys_input,
                      BufferView<KeyT> keys_output, BufferView<ValueT> values_input, BufferView<ValueT> values_output,
                      size_t num_items, size_t num_segments, BufferView<uint> begin_offsets,
                      BufferView<uint> end_offsets, uint begin_bit, uint end_bit, int desc, int value_order,
                      const char* what) {
        static_assert(detail::segsort_key_ok<KeyT>, "DeviceSegmentedSort keys: 4- or 8-byte numbers");
        static_assert(detail::segsort_value_ok<ValueT>, "DeviceSegmentedSort values: 4- or 8-byte types");
        validate_common(num_items, num_segments, begin_offsets, end_offsets);
        if (num_items == 0u || num_segments == 0u) return;
        LCPP_ASSERT(keys_input.size() >= num_items, "DeviceSegmentedSort key input view is too small.");
        LCPP_ASSERT(keys_output.size() >= num_items, "DeviceSegmentedSort key output view is too small.");
        LCPP_ASSERT(values_input.size() >= num_items, "DeviceSegmentedSort value input view is too small.");
        LCPP_ASSERT(values_output.size() >= num_items, "DeviceSegmentedSort value output view is too small.");
        if (num_items > 1u)
            LCPP_ASSERT(temp_storage.size() >=
                            bytes_to_uint_count(GetSortPairsTempStorageBytes<KeyT, ValueT>(num_items)),
                        "DeviceSegmentedSort temporary storage is too small.");
        using A = detail::by_key_abi_t<KeyT>;
        using VB = detail::segsort_value_bits_t<ValueT>;
        void* temp = temp_storage.data();
        const size_t tb = temp_storage.size_bytes();
        const A* kin = reinterpret_cast<const A*>(keys_input.data());
        A* kout = reinterpret_cast<A*>(keys_output.data());
        const VB* vin = reinterpret_cast<const VB*>(values_input.data());
        VB* vout = reinterpret_cast<VB*>(values_output.data());
        const uint32_t* b = begin_offsets.data();
        const uint32_t* e = end_offsets.data();
        cmdlist << [=](hipStream_t s) {
            luisa::detail::abi_check(detail::segsort_pairs(temp, tb, kin, kout, vin, vout, num_items, num_segments,
                                                           b, e, begin_bit, end_bit, desc, value_order,
                                                           detail::stream_ptr(s)),
                                     what);
        };
    }

    template <typename KeyT>
    void record_keys_db(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyT>& keys,
                        size_t num_items, size_t num_segments, BufferView<uint> begin_offsets,
                        BufferView<uint> end_offsets, uint begin_bit, uint end_bit, int desc, int value_order,
                        const char* what) {
        static_assert(detail::segsort_key_ok<KeyT>, "DeviceSegmentedSort keys: 4- or 8-byte numbers");
        (void)temp_storage;
        validate_key_double_buffer(keys, num_items, num_segments, begin_offsets, end_offsets);
        if (num_items <= 1u || num_segments == 0u) return;
        using A = detail::by_key_abi_t<KeyT>;
        A* k0 = reinterpret_cast<A*>(keys.d_buffer[0].data());
        A* k1 = reinterpret_cast<A*>(keys.d_buffer[1].data());
        const uint32_t* b = begin_offsets.data();
        const uint32_t* e = end_offsets.data();
        const int sel = keys.selector;
        keys.selector ^= static_cast<int>(detail::segsort_pass_count(num_items) & 1u);
        cmdlist << [=](hipStream_t s) {
            int local = sel;
            luisa::detail::abi_check(detail::segsort_keys_db(k0, k1, &local, num_items, num_segments, b, e, begin_bit,
                                                             end_bit, desc, value_order, detail::stream_ptr(s)),
                                     what);
        };
    }

    template <typename KeyT, typename ValueT>
    void record_pairs_db(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyT>& keys,
                         DoubleBuffer<ValueT>& values, size_t num_items, size_t num_segments,
                         BufferView<uint> begin_offsets, BufferView<uint> end_offsets, uint begin_bit, uint end_bit,
                         int desc, int value_order, const char* what) {
        static_assert(detail::segsort_key_ok<KeyT>, "DeviceSegmentedSort keys: 4- or 8-byte numbers");
        static_assert(detail::segsort_value_ok<ValueT>, "DeviceSegmentedSort values: 4- or 8-byte types");
        (void)temp_storage;
        validate_pair_double_buffers(keys, values, num_items, num_segments, begin_offsets, end_offsets);
        if (num_items <= 1u || num_segments == 0u) return;
        using A = detail::by_key_abi_t<KeyT>;
        using VB = detail::segsort_value_bits_t<ValueT>;
        A* k0 = reinterpret_cast<A*>(keys.d_buffer[0].data());
        A* k1 = reinterpret_cast<A*>(keys.d_buffer[1].data());
        VB* v0 = reinterpret_cast<VB*>(values.d_buffer[0].data());
        VB* v1 = reinterpret_cast<VB*>(values.d_buffer[1].data());
        const uint32_t* b = begin_offsets.data();
        const uint32_t* e = end_offsets.data();
        const int sel = keys.selector;
        const int flip = static_cast<int>(detail::segsort_pass_count(num_items) & 1u);
        keys.selector ^= flip;
        values.selector ^= flip;
        cmdlist << [=](hipStream_t s) {
            int ks = sel;
            int vs = sel;
            luisa::detail::abi_check(detail::segsort_pairs_db(k0, k1, &ks, v0, v1, &vs, num_items, num_segments, b,
                                                              e, begin_bit, end_bit, desc, value_order,
                                                              detail::stream_ptr(s)),
                                     what);
        };
    }
};

}  // namespace luisa::parallel_primitive
