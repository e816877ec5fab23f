// DeviceRadixSort (onesweep, 8-bit digits, stable LSD) over the MI355X C-ABI
// (lcpp_hip_radix_sort_*), with the reference's module shape (src/lcpp/device/device_radix_sort.h:50-56
// template, :179-193 create, :337-362 temp queries) and entry points: copy form SortKeys / SortPairs /
// SortKeysDescending / SortPairsDescending (:369-466) and DoubleBuffer form (:468-554), checked like
// validate_key_views / validate_pair_views / validate_double_buffer (:941-1016).
//
// DoubleBuffer form: the selector is flipped once per 8-bit pass when the call is recorded, as the
// reference does (:1462-1471), so after commit `d_keys.current()` holds the sorted keys.
#pragma once

#include <type_traits>

#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

namespace detail {

template <typename K>
constexpr bool radix_key_supported = std::is_same_v<K, uint32_t> || std::is_same_v<K, int32_t> ||
                                     std::is_same_v<K, float> || (std::is_integral_v<K> && sizeof(K) == 8) ||
                                     std::is_same_v<K, double>;

// Copy-form sort through the C-ABI; values == nullptr sorts keys only.
template <typename K, size_t VB>
int radix_copy(void* temp, size_t temp_bytes, const K* kin, K* kout, const void* vin, void* vout, uint n, uint b,
               uint e, int desc, void* s) {
    if constexpr (VB == 0) {
        if constexpr (std::is_same_v<K, uint32_t>) return lcpp_hip_radix_sort_keys_u32(temp, temp_bytes, kin, kout, n, b, e, desc, s);
        else if constexpr (std::is_same_v<K, int32_t>) return lcpp_hip_radix_sort_keys_i32(temp, temp_bytes, kin, kout, n, b, e, desc, s);
        else if constexpr (std::is_same_v<K, float>) return lcpp_hip_radix_sort_keys_f32(temp, temp_bytes, kin, kout, n, b, e, desc, s);
        else if constexpr (std::is_same_v<K, double>) return lcpp_hip_radix_sort_keys_f64(temp, temp_bytes, kin, kout, n, b, e, desc, s);
        else if constexpr (std::is_signed_v<K>)
            return lcpp_hip_radix_sort_keys_i64(temp, temp_bytes, reinterpret_cast<const int64_t*>(kin),
                                                reinterpret_cast<int64_t*>(kout), n, b, e, desc, s);
        else
            return lcpp_hip_radix_sort_keys_u64(temp, temp_bytes, reinterpret_cast<const uint64_t*>(kin),
                                                reinterpret_cast<uint64_t*>(kout), n, b, e, desc, s);
    } else {
#define LCPP_FACADE_PAIRS(SUFFIX, KT)                                                                              \
    if constexpr (VB == 4)                                                                                         \
        return lcpp_hip_radix_sort_pairs_##SUFFIX##_v32(temp, temp_bytes, reinterpret_cast<const KT*>(kin),        \
                                                        reinterpret_cast<KT*>(kout), vin, vout, n, b, e, desc, s); \
    else                                                                                                           \
        return lcpp_hip_radix_sort_pairs_##SUFFIX##_v64(temp, temp_bytes, reinterpret_cast<const KT*>(kin),        \
                                                        reinterpret_cast<KT*>(kout), vin, vout, n, b, e, desc, s);
        if constexpr (std::is_same_v<K, uint32_t>) { LCPP_FACADE_PAIRS(u32, uint32_t) }
        else if constexpr (std::is_same_v<K, int32_t>) { LCPP_FACADE_PAIRS(i32, int32_t) }
        else if constexpr (std::is_same_v<K, float>) { LCPP_FACADE_PAIRS(f32, float) }
        else if constexpr (std::is_same_v<K, double>) { LCPP_FACADE_PAIRS(f64, double) }
        else if constexpr (std::is_signed_v<K>) { LCPP_FACADE_PAIRS(i64, int64_t) }
        else { LCPP_FACADE_PAIRS(u64, uint64_t) }
#undef LCPP_FACADE_PAIRS
    }
}

// DoubleBuffer-form sort through the C-ABI; `sel` is a private copy of the recorded selector.
template <typename K, size_t VB>
int radix_db(void* temp, size_t temp_bytes, K* k0, K* k1, void* v0, void* v1, int* sel, uint n, uint b, uint e,
             int desc, void* s) {
    if constexpr (VB == 0) {
        if constexpr (std::is_same_v<K, uint32_t>) return lcpp_hip_radix_sort_keys_db_u32(temp, temp_bytes, k0, k1, sel, n, b, e, desc, s);
        else if constexpr (std::is_same_v<K, int32_t>) return lcpp_hip_radix_sort_keys_db_i32(temp, temp_bytes, k0, k1, sel, n, b, e, desc, s);
        else if constexpr (std::is_same_v<K, float>) return lcpp_hip_radix_sort_keys_db_f32(temp, temp_bytes, k0, k1, sel, n, b, e, desc, s);
        else if constexpr (std::is_same_v<K, double>) return lcpp_hip_radix_sort_keys_db_f64(temp, temp_bytes, k0, k1, sel, n, b, e, desc, s);
        else if constexpr (std::is_signed_v<K>)
            return lcpp_hip_radix_sort_keys_db_i64(temp, temp_bytes, reinterpret_cast<int64_t*>(k0),
                                                   reinterpret_cast<int64_t*>(k1), sel, n, b, e, desc, s);
        else
            return lcpp_hip_radix_sort_keys_db_u64(temp, temp_bytes, reinterpret_cast<uint64_t*>(k0),
                                                   reinterpret_cast<uint64_t*>(k1), sel, n, b, e, desc, s);
    } else {
#define LCPP_FACADE_PAIRS_DB(SUFFIX, KT)                                                                            \
    if constexpr (VB == 4)                                                                                          \
        return lcpp_hip_radix_sort_pairs_db_##SUFFIX##_v32(temp, temp_bytes, reinterpret_cast<KT*>(k0),             \
                                                           reinterpret_cast<KT*>(k1), v0, v1, sel, n, b, e, desc, s); \
    else                                                                                                            \
        return lcpp_hip_radix_sort_pairs_db_##SUFFIX##_v64(temp, temp_bytes, reinterpret_cast<KT*>(k0),             \
                                                           reinterpret_cast<KT*>(k1), v0, v1, sel, n, b, e, desc, s);
        if constexpr (std::is_same_v<K, uint32_t>) { LCPP_FACADE_PAIRS_DB(u32, uint32_t) }
        else if constexpr (std::is_same_v<K, int32_t>) { LCPP_FACADE_PAIRS_DB(i32, int32_t) }
        else if constexpr (std::is_same_v<K, float>) { LCPP_FACADE_PAIRS_DB(f32, float) }
        else if constexpr (std::is_same_v<K, double>) { LCPP_FACADE_PAIRS_DB(f64, double) }
        else if constexpr (std::is_signed_v<K>) { LCPP_FACADE_PAIRS_DB(i64, int64_t) }
        else { LCPP_FACADE_PAIRS_DB(u64, uint64_t) }
#undef LCPP_FACADE_PAIRS_DB
    }
}

}  // namespace detail

template <size_t BLOCK_SIZE = 256, size_t WARP_NUMS = 32, size_t ITEMS_PER_THREAD = 16,
          bool CUB_SMALL_KEY_POLICY = true>
class DeviceRadixSort : public LuisaModule {
  public:
    void create(Device& device, Stream* debug_stream = nullptr, InteropContext* interop = nullptr) {
        (void)debug_stream;
        (void)interop;
        create_module(device);
    }

    template <NumericT KeyType>
    static size_t GetSortKeysTempStorageBytes(uint num_items) {
        return lcpp_hip_radix_sort_temp_bytes_policy(num_items, sizeof(KeyType), sizeof(KeyType), 1,
                                                     static_cast<uint32_t>(BLOCK_SIZE),
                                                     static_cast<uint32_t>(ITEMS_PER_THREAD),
                                                     CUB_SMALL_KEY_POLICY ? 1 : 0);
    }

    template <NumericT KeyType, NumericT ValueType>
    static size_t GetSortPairsTempStorageBytes(uint num_items) {
        return lcpp_hip_radix_sort_temp_bytes_policy(num_items, sizeof(KeyType), sizeof(ValueType), 0,
                                                     static_cast<uint32_t>(BLOCK_SIZE),
                                                     static_cast<uint32_t>(ITEMS_PER_THREAD),
                                                     CUB_SMALL_KEY_POLICY ? 1 : 0);
    }

    // ---- copy form -------------------------------------------------------------------------------
    template <NumericT KeyType, NumericT ValueType>
    void SortPairs(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                   BufferView<KeyType> d_keys_out, BufferView<ValueType> d_values_in,
                   BufferView<ValueType> d_values_out, uint num_items, uint begin_bit = 0u,
                   uint end_bit = sizeof(KeyType) * 8u) {
        record_pairs<KeyType, ValueType>(cmdlist, temp_storage, d_keys_in, d_keys_out, d_values_in, d_values_out,
                                         num_items, begin_bit, end_bit, 0);
    }

    template <NumericT KeyType>
    void SortKeys(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                  BufferView<KeyType> d_keys_out, uint num_items, uint begin_bit = 0u,
                  uint end_bit = sizeof(KeyType) * 8u) {
        record_keys<KeyType>(cmdlist, temp_storage, d_keys_in, d_keys_out, num_items, begin_bit, end_bit, 0);
    }

    template <NumericT KeyType, NumericT ValueType>
    void SortPairsDescending(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                             BufferView<KeyType> d_keys_out, BufferView<ValueType> d_values_in,
                             BufferView<ValueType> d_values_out, uint num_items, uint begin_bit = 0u,
                             uint end_bit = sizeof(KeyType) * 8u) {
        record_pairs<KeyType, ValueType>(cmdlist, temp_storage, d_keys_in, d_keys_out, d_values_in, d_values_out,
                                         num_items, begin_bit, end_bit, 1);
    }

    template <NumericT KeyType>
    void SortKeysDescending(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                            BufferView<KeyType> d_keys_out, uint num_items, uint begin_bit = 0u,
                            uint end_bit = sizeof(KeyType) * 8u) {
        record_keys<KeyType>(cmdlist, temp_storage, d_keys_in, d_keys_out, num_items, begin_bit, end_bit, 1);
    }

    // ---- DoubleBuffer form -----------------------------------------------------------------------
    template <NumericT KeyType, NumericT ValueType>
    void SortPairs(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyType>& d_keys,
                   DoubleBuffer<ValueType>& d_values, uint num_items, uint begin_bit = 0u,
                   uint end_bit = sizeof(KeyType) * 8u) {
        record_pairs_db<KeyType, ValueType>(cmdlist, temp_storage, d_keys, d_values, num_items, begin_bit, end_bit, 0);
    }

    template <NumericT KeyType>
    void SortKeys(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyType>& d_keys, uint num_items,
                  uint begin_bit = 0u, uint end_bit = sizeof(KeyType) * 8u) {
        record_keys_db<KeyType>(cmdlist, temp_storage, d_keys, num_items, begin_bit, end_bit, 0);
    }

    template <NumericT KeyType, NumericT ValueType>
    void SortPairsDescending(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyType>& d_keys,
                             DoubleBuffer<ValueType>& d_values, uint num_items, uint begin_bit = 0u,
                             uint end_bit = sizeof(KeyType) * 8u) {
        record_pairs_db<KeyType, ValueType>(cmdlist, temp_storage, d_keys, d_values, num_items, begin_bit, end_bit, 1);
    }

    template <NumericT KeyType>
    void SortKeysDescending(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyType>& d_keys,
                            uint num_items, uint begin_bit = 0u, uint end_bit = sizeof(KeyType) * 8u) {
        record_keys_db<KeyType>(cmdlist, temp_storage, d_keys, num_items, begin_bit, end_bit, 1);
    }

  private:
    static uint passes(uint begin_bit, uint end_bit) { return (end_bit - begin_bit + 7u) / 8u; }

    template <typename KeyType>
    void validate_key_views(BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                            BufferView<KeyType> d_keys_out, uint num_items, uint begin_bit, uint end_bit,
                            bool keys_only = true) const {
        static_assert(detail::radix_key_supported<KeyType>, "DeviceRadixSort: unsupported key type");
        LCPP_ASSERT(m_created, "DeviceRadixSort::create must be called before dispatch.");
        LCPP_ASSERT(begin_bit <= end_bit, "DeviceRadixSort begin_bit must not exceed end_bit.");
        LCPP_ASSERT(end_bit <= sizeof(KeyType) * 8u, "DeviceRadixSort end_bit exceeds the key width.");
        LCPP_ASSERT(d_keys_in.size() >= num_items, "DeviceRadixSort key input view is too small.");
        LCPP_ASSERT(d_keys_out.size() >= num_items, "DeviceRadixSort key output view is too small.");
        if (keys_only && num_items > 0u && begin_bit < end_bit) {
            LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetSortKeysTempStorageBytes<KeyType>(num_items)),
                        "DeviceRadixSort temporary storage is too small.");
        }
    }

    template <typename KeyType, typename ValueType>
    void validate_pair_views(BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                             BufferView<KeyType> d_keys_out, BufferView<ValueType> d_values_in,
                             BufferView<ValueType> d_values_out, uint num_items, uint begin_bit, uint end_bit) const {
        static_assert(sizeof(ValueType) == 4 || sizeof(ValueType) == 8, "DeviceRadixSort: values must be 4 or 8 bytes");
        // Only the pairs formula is checked.  The reference also applies the keys-only check here
        // (device_radix_sort.h:1007), which rejects GetSortPairsTempStorageBytes-sized storage
        // whenever the value type is narrower than the key (e.g. 8-byte keys with 4-byte values).
        validate_key_views(temp_storage, d_keys_in, d_keys_out, num_items, begin_bit, end_bit, false);
        LCPP_ASSERT(d_values_in.size() >= num_items, "DeviceRadixSort value input view is too small.");
        LCPP_ASSERT(d_values_out.size() >= num_items, "DeviceRadixSort value output view is too small.");
        if (num_items > 0u && begin_bit < end_bit) {
            LCPP_ASSERT(temp_storage.size() >=
                            bytes_to_uint_count(GetSortPairsTempStorageBytes<KeyType, ValueType>(num_items)),
                        "DeviceRadixSort temporary storage is too small.");
        }
    }

    template <typename T>
    static void validate_double_buffer(const DoubleBuffer<T>& buffer, uint num_items, const char* name) {
        LCPP_ASSERT(buffer.selector == 0 || buffer.selector == 1,
                    std::string("DeviceRadixSort ") + name + " DoubleBuffer selector must be 0 or 1.");
        LCPP_ASSERT(buffer.d_buffer[0].size() >= num_items,
                    std::string("DeviceRadixSort ") + name + " DoubleBuffer slot 0 is too small.");
        LCPP_ASSERT(buffer.d_buffer[1].size() >= num_items,
                    std::string("DeviceRadixSort ") + name + " DoubleBuffer slot 1 is too small.");
    }

    template <typename KeyType>
    void record_keys(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                     BufferView<KeyType> d_keys_out, uint num_items, uint begin_bit, uint end_bit, int desc) {
        validate_key_views(temp_storage, d_keys_in, d_keys_out, num_items, begin_bit, end_bit);
        if (num_items == 0u) return;
        uint* temp = temp_storage.data();
        const size_t tb = temp_storage.size_bytes();
        const KeyType* kin = d_keys_in.data();
        KeyType* kout = d_keys_out.data();
        cmdlist << [=](hipStream_t s) {
            const int rc = detail::radix_copy<KeyType, 0>(temp, tb, kin, kout, nullptr, nullptr, num_items, begin_bit,
                                                          end_bit, desc, detail::stream_ptr(s));
            luisa::detail::abi_check(rc, "DeviceRadixSort::SortKeys");
        };
    }

    template <typename KeyType, typename ValueType>
    void record_pairs(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                      BufferView<KeyType> d_keys_out, BufferView<ValueType> d_values_in,
                      BufferView<ValueType> d_values_out, uint num_items, uint begin_bit, uint end_bit, int desc) {
        validate_pair_views(temp_storage, d_keys_in, d_keys_out, d_values_in, d_values_out, num_items, begin_bit,
                            end_bit);
        if (num_items == 0u) return;
        uint* temp = temp_storage.data();
        const size_t tb = temp_storage.size_bytes();
        const KeyType* kin = d_keys_in.data();
        KeyType* kout = d_keys_out.data();
        const void* vin = d_values_in.data();
        void* vout = d_values_out.data();
        cmdlist << [=](hipStream_t s) {
            const int rc = detail::radix_copy<KeyType, sizeof(ValueType)>(temp, tb, kin, kout, vin, vout, num_items,
                                                                          begin_bit, end_bit, desc,
                                                                          detail::stream_ptr(s));
            luisa::detail::abi_check(rc, "DeviceRadixSort::SortPairs");
        };
    }

    template <typename KeyType>
    void record_keys_db(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyType>& d_keys,
                        uint num_items, uint begin_bit, uint end_bit, int desc) {
        validate_double_buffer(d_keys, num_items, "key");
        validate_key_views(temp_storage, d_keys.current(), d_keys.alternate(), num_items, begin_bit, end_bit);
        if (num_items == 0u || begin_bit == end_bit) return;
        uint* temp = temp_storage.data();
        const size_t tb = temp_storage.size_bytes();
        KeyType* k0 = d_keys.d_buffer[0].data();
        KeyType* k1 = d_keys.d_buffer[1].data();
        const int sel = d_keys.selector;
        d_keys.selector ^= static_cast<int>(passes(begin_bit, end_bit) & 1u);
        cmdlist << [=](hipStream_t s) {
            int local = sel;
            const int rc = detail::radix_db<KeyType, 0>(temp, tb, k0, k1, nullptr, nullptr, &local, num_items,
                                                        begin_bit, end_bit, desc, detail::stream_ptr(s));
            luisa::detail::abi_check(rc, "DeviceRadixSort::SortKeys(DoubleBuffer)");
        };
    }

    template <typename KeyType, typename ValueType>
    void record_pairs_db(CommandList& cmdlist, BufferView<uint> temp_storage, DoubleBuffer<KeyType>& d_keys,
                         DoubleBuffer<ValueType>& d_values, uint num_items, uint begin_bit, uint end_bit, int desc) {
        validate_double_buffer(d_keys, num_items, "key");
        validate_double_buffer(d_values, num_items, "value");
        LCPP_ASSERT(d_keys.selector == d_values.selector,
                    "DeviceRadixSort key and value DoubleBuffer selectors must match.");
        validate_pair_views(temp_storage, d_keys.current(), d_keys.alternate(), d_values.current(),
                            d_values.alternate(), num_items, begin_bit, end_bit);
        if (num_items == 0u || begin_bit == end_bit) return;
        uint* temp = temp_storage.data();
        const size_t tb = temp_storage.size_bytes();
        KeyType* k0 = d_keys.d_buffer[0].data();
        KeyType* k1 = d_keys.d_buffer[1].data();
        void* v0 = d_values.d_buffer[0].data();
        void* v1 = d_values.d_buffer[1].data();
        const int sel = d_keys.selector;
        const int flip = static_cast<int>(passes(begin_bit, end_bit) & 1u);
        d_keys.selector ^= flip;
        d_values.selector ^= flip;
        cmdlist << [=](hipStream_t s) {
            int local = sel;
            const int rc = detail::radix_db<KeyType, sizeof(ValueType)>(temp, tb, k0, k1, v0, v1, &local, num_items,
                                                                        begin_bit, end_bit, desc,
                                                                        detail::stream_ptr(s));
            luisa::detail::abi_check(rc, "DeviceRadixSort::SortPairs(DoubleBuffer)");
        };
    }
};

}  // namespace luisa::parallel_primitive
