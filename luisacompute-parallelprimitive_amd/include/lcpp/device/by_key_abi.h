// Overloads binding the by-key facade entry points to the C-ABI symbols
// lcpp_hip_{scan,reduce}_by_key_{sum,min,max}_<key>_<value>, plus the key equality those kernels evaluate.
#pragma once

#include <cstdint>
#include <type_traits>

#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

// Key equality of the by-key entry points: two keys are equal when they agree on the bits of
// `mask`, i.e. ((a ^ b) & mask) == 0.  The default (all ones) is the reference's default
// `lhs == rhs` (device_scan.h:434-435); other masks express bit-class equalities such as the
// parity test of tests/device_scan_test.cpp:419-447.
struct KeyMaskEquality {
    uint64_t mask = ~uint64_t(0);
};

namespace detail {

// The fixed-width type whose C-ABI symbol serves T (long and long long both map to int64_t).
template <typename T>
using by_key_abi_t = std::conditional_t<
    std::is_floating_point_v<T>, T,
    std::conditional_t<sizeof(T) == 8, std::conditional_t<std::is_signed_v<T>, int64_t, uint64_t>,
                       std::conditional_t<std::is_signed_v<T>, int32_t, uint32_t>>>;

template <typename K>
inline constexpr bool by_key_key_ok = std::is_integral_v<K> && !std::is_same_v<K, bool> &&
                                      (sizeof(K) == 4 || sizeof(K) == 8);
template <typename V>
inline constexpr bool by_key_value_ok = (std::is_integral_v<V> && !std::is_same_v<V, bool> &&
                                         (sizeof(V) == 4 || sizeof(V) == 8)) ||
                                        std::is_same_v<V, float> || std::is_same_v<V, double>;

// One overload per operator tag (SumOp, MinOp, MaxOp) and key / value type.
#define LCPP_FACADE_BY_KEY_OP(TAG, NAME, KS, KT, VS, VT)                                                         \
    inline int scan_by_key(TAG, void* t, size_t tb, const KT* k, const VT* vi, VT* vo, uint64_t n, int inc,       \
                           int use_init, VT init, uint64_t mask, void* s) {                                    \
        return lcpp_hip_scan_by_key_##NAME##_##KS##_##VS(t, tb, k, vi, vo, n, inc, use_init, init, mask, s);    \
    }                                                                                                          \
    inline int reduce_by_key(TAG, void* t, size_t tb, const KT* k, const VT* v, KT* uo, VT* ao, uint32_t* ro,     \
                             uint64_t n, uint64_t mask, void* s) {                                              \
        return lcpp_hip_reduce_by_key_##NAME##_##KS##_##VS(t, tb, k, v, uo, ao, ro, n, mask, s);                 \
    }
#define LCPP_FACADE_BY_KEY(KS, KT, VS, VT)                 \
    LCPP_FACADE_BY_KEY_OP(SumOp, sum, KS, KT, VS, VT)      \
    LCPP_FACADE_BY_KEY_OP(MinOp, min, KS, KT, VS, VT)      \
    LCPP_FACADE_BY_KEY_OP(MaxOp, max, KS, KT, VS, VT)
#define LCPP_FACADE_BY_KEY_VALUES(KS, KT)       \
    LCPP_FACADE_BY_KEY(KS, KT, i32, int32_t)    \
    LCPP_FACADE_BY_KEY(KS, KT, u32, uint32_t)   \
    LCPP_FACADE_BY_KEY(KS, KT, f32, float)      \
    LCPP_FACADE_BY_KEY(KS, KT, i64, int64_t)    \
    LCPP_FACADE_BY_KEY(KS, KT, u64, uint64_t)   \
    LCPP_FACADE_BY_KEY(KS, KT, f64, double)
LCPP_FACADE_BY_KEY_VALUES(i32, int32_t)
LCPP_FACADE_BY_KEY_VALUES(u32, uint32_t)
LCPP_FACADE_BY_KEY_VALUES(i64, int64_t)
LCPP_FACADE_BY_KEY_VALUES(u64, uint64_t)
#undef LCPP_FACADE_BY_KEY_VALUES
#undef LCPP_FACADE_BY_KEY
#undef LCPP_FACADE_BY_KEY_OP

template <typename Op>
inline constexpr bool by_key_op_ok = std::is_same_v<Op, SumOp> || std::is_same_v<Op, MinOp> || std::is_same_v<Op, MaxOp>;

}  // namespace detail
}  // namespace luisa::parallel_primitive
