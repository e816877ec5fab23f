// Overloads binding the segmented-sort facade (DeviceSegmentedSort, DeviceSegmentedRadixSort) to the
// C-ABI symbols lcpp_hip_segmented_sort_*.  Keys: 4- and 8-byte integers, float, double; values: any
// 4- or 8-byte type, moved as raw bits.
#pragma once

#include <cstdint>
#include <type_traits>

#include "lcpp/device/by_key_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive::detail {

template <typename K>
inline constexpr bool segsort_key_ok = (std::is_integral_v<K> && !std::is_same_v<K, bool> &&
                                        (sizeof(K) == 4 || sizeof(K) == 8)) ||
                                       std::is_same_v<K, float> || std::is_same_v<K, double>;
template <typename V>
inline constexpr bool segsort_value_ok = sizeof(V) == 4 || sizeof(V) == 8;
template <typename V>
using segsort_value_bits_t = std::conditional_t<sizeof(V) == 8, uint64_t, uint32_t>;

#define LCPP_FACADE_SEGSORT_PAIRS(KS, KT, VS, VT)                                                                  \
    inline int segsort_pairs(void* t, size_t tb, const KT* kin, KT* kout, const VT* vin, VT* vout, uint64_t n,     \
                             uint64_t m, const uint32_t* b, const uint32_t* e, uint32_t bb, uint32_t eb, int desc,  \
                             int vo, void* s) {                                                                     \
        return lcpp_hip_segmented_sort_pairs_##KS##_##VS(t, tb, kin, kout, vin, vout, n, m, b, e, bb, eb, desc, vo, \
                                                         s);                                                        \
    }                                                                                                               \
    inline int segsort_pairs_db(KT* k0, KT* k1, int* ks, VT* v0, VT* v1, int* vs, uint64_t n, uint64_t m,          \
                                const uint32_t* b, const uint32_t* e, uint32_t bb, uint32_t eb, int desc, int vo,   \
                                void* s) {                                                                          \
        return lcpp_hip_segmented_sort_pairs_db_##KS##_##VS(k0, k1, ks, v0, v1, vs, n, m, b, e, bb, eb, desc, vo,   \
                                                            s);                                                     \
    }
#define LCPP_FACADE_SEGSORT(KS, KT)                                                                                 \
    inline int segsort_keys(void* t, size_t tb, const KT* kin, KT* kout, uint64_t n, uint64_t m, const uint32_t* b, \
                            const uint32_t* e, uint32_t bb, uint32_t eb, int desc, int vo, void* s) {              \
        return lcpp_hip_segmented_sort_keys_##KS(t, tb, kin, kout, n, m, b, e, bb, eb, desc, vo, s);               \
    }                                                                                                               \
    inline int segsort_keys_db(KT* k0, KT* k1, int* ks, uint64_t n, uint64_t m, const uint32_t* b,                 \
                               const uint32_t* e, uint32_t bb, uint32_t eb, int desc, int vo, void* s) {            \
        return lcpp_hip_segmented_sort_keys_db_##KS(k0, k1, ks, n, m, b, e, bb, eb, desc, vo, s);                  \
    }                                                                                                               \
    LCPP_FACADE_SEGSORT_PAIRS(KS, KT, v32, uint32_t)                                                                \
    LCPP_FACADE_SEGSORT_PAIRS(KS, KT, v64, uint64_t)
LCPP_FACADE_SEGSORT(u32, uint32_t)
LCPP_FACADE_SEGSORT(i32, int32_t)
LCPP_FACADE_SEGSORT(f32, float)
LCPP_FACADE_SEGSORT(u64, uint64_t)
LCPP_FACADE_SEGSORT(i64, int64_t)
LCPP_FACADE_SEGSORT(f64, double)
#undef LCPP_FACADE_SEGSORT
#undef LCPP_FACADE_SEGSORT_PAIRS

// Host copy of the reference's merge_pass_count (device_segmented_sort.h:529-541): ceil(log2 n) for
// n > 1, the number of times a DoubleBuffer sort flips the selector.
inline uint32_t segsort_pass_count(size_t n) {
    uint32_t passes = 0;
    for (size_t width = 1; width < n; width *= 2) ++passes;
    return passes;
}

}  // namespace luisa::parallel_primitive::detail
