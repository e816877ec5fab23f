// Overloads binding the stream-compaction facade (DeviceSelect, DevicePartition,
// DeviceRunLengthEncode) to the C-ABI symbols lcpp_hip_{select,partition,run_length}_*, and the item
// predicates those kernels evaluate.
#pragma once

#include <cstdint>
#include <cstring>
#include <type_traits>

#include "lcpp/device/by_key_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

// A predicate the compaction kernels evaluate on the device: up to two clauses that must both hold,
// each comparing the item with operands of its own type.  It stands in for the reference's
// Callable<bool(T)> (device lambdas compiled by LuisaCompute's DSL, device_select.h:119-175).
template <typename T>
class ItemPredicate {
  public:
    ItemPredicate() { std::memset(&m_pred, 0, sizeof(m_pred)); }
    static ItemPredicate less(T a) { return clause(LCPP_HIP_PRED_LT, a, T{}); }
    static ItemPredicate less_equal(T a) { return clause(LCPP_HIP_PRED_LE, a, T{}); }
    static ItemPredicate greater(T a) { return clause(LCPP_HIP_PRED_GT, a, T{}); }
    static ItemPredicate greater_equal(T a) { return clause(LCPP_HIP_PRED_GE, a, T{}); }
    static ItemPredicate equal(T a) { return clause(LCPP_HIP_PRED_EQ, a, T{}); }
    static ItemPredicate not_equal(T a) { return clause(LCPP_HIP_PRED_NE, a, T{}); }
    static ItemPredicate in_range(T lo, T hi) { return clause(LCPP_HIP_PRED_RANGE, lo, hi); }  // lo <= x < hi
    static ItemPredicate remainder_equal(T m, T r) { return clause(LCPP_HIP_PRED_MOD_EQ, m, r); }  // x % m == r
    static ItemPredicate remainder_not_equal(T m, T r) { return clause(LCPP_HIP_PRED_MOD_NE, m, r); }
    static ItemPredicate bits_equal(T mask, T bits) { return clause(LCPP_HIP_PRED_MASK_EQ, mask, bits); }
    static ItemPredicate bits_not_equal(T mask, T bits) { return clause(LCPP_HIP_PRED_MASK_NE, mask, bits); }

    // Both predicates must hold (each side must be a single clause).
    friend ItemPredicate operator&&(const ItemPredicate& x, const ItemPredicate& y) {
        LCPP_ASSERT(x.m_pred.op[1] == LCPP_HIP_PRED_TRUE && y.m_pred.op[1] == LCPP_HIP_PRED_TRUE,
                    "ItemPredicate: at most two clauses");
        ItemPredicate r = x;
        r.m_pred.op[1] = y.m_pred.op[0];
        r.m_pred.a[1] = y.m_pred.a[0];
        r.m_pred.b[1] = y.m_pred.b[0];
        return r;
    }
    [[nodiscard]] const lcpp_hip_predicate& c_predicate() const noexcept { return m_pred; }

  private:
    static uint64_t bits(T v) {
        uint64_t b = 0;
        std::memcpy(&b, &v, sizeof(T));
        return b;
    }
    static ItemPredicate clause(int op, T a, T b) {
        ItemPredicate p;
        p.m_pred.op[0] = op;
        p.m_pred.a[0] = bits(a);
        p.m_pred.b[0] = bits(b);
        return p;
    }
    lcpp_hip_predicate m_pred;
};

namespace detail {

// Flag types of the flagged forms: bool travels as a byte.
template <typename F>
using flag_abi_t = std::conditional_t<std::is_same_v<F, bool>, uint8_t, by_key_abi_t<F>>;

template <typename F>
inline constexpr bool flag_ok = std::is_same_v<F, bool> ||
                                (std::is_integral_v<F> && (sizeof(F) == 4 || sizeof(F) == 8));

#define LCPP_FACADE_COMPACT_FLAGS(TS, TT, FS, FT)                                                                  \
    inline int select_flagged(void* t, size_t tb, const TT* in, const FT* f, TT* out, uint32_t* num, uint64_t n,   \
                              void* s) {                                                                           \
        return lcpp_hip_select_flagged_##TS##_##FS(t, tb, in, f, out, num, n, s);                                  \
    }                                                                                                              \
    inline int select_flagged_if(void* t, size_t tb, const TT* in, const FT* f, TT* out, uint32_t* num,            \
                                 uint64_t n, const lcpp_hip_predicate* p, void* s) {                              \
        return lcpp_hip_select_flagged_if_##TS##_##FS(t, tb, in, f, out, num, n, p, s);                            \
    }                                                                                                              \
    inline int partition_flagged(void* t, size_t tb, const TT* in, const FT* f, TT* out, uint32_t* num,            \
                                 uint64_t n, void* s) {                                                            \
        return lcpp_hip_partition_flagged_##TS##_##FS(t, tb, in, f, out, num, n, s);                               \
    }
#define LCPP_FACADE_COMPACT_UBK(KS, KT, VS, VT)                                                                    \
    inline int select_unique_by_key(void* t, size_t tb, const KT* k, const VT* v, KT* ko, VT* vo, uint32_t* num,   \
                                    uint64_t n, uint64_t mask, void* s) {                                          \
        return lcpp_hip_select_unique_by_key_##KS##_##VS(t, tb, k, v, ko, vo, num, n, mask, s);                    \
    }
#define LCPP_FACADE_COMPACT_ITEMS(TS, TT)                                                                          \
    inline int select_if(void* t, size_t tb, const TT* in, TT* out, uint32_t* num, uint64_t n,                     \
                         const lcpp_hip_predicate* p, void* s) {                                                   \
        return lcpp_hip_select_if_##TS(t, tb, in, out, num, n, p, s);                                              \
    }                                                                                                              \
    inline int partition_if(void* t, size_t tb, const TT* in, TT* out, uint32_t* num, uint64_t n,                  \
                            const lcpp_hip_predicate* p, void* s) {                                                \
        return lcpp_hip_partition_if_##TS(t, tb, in, out, num, n, p, s);                                           \
    }                                                                                                              \
    inline int partition_three_way(void* t, size_t tb, const TT* in, TT* o1, TT* o2, TT* o3, uint32_t* num,        \
                                   uint64_t n, const lcpp_hip_predicate* p1, const lcpp_hip_predicate* p2,         \
                                   void* s) {                                                                      \
        return lcpp_hip_partition_three_way_##TS(t, tb, in, o1, o2, o3, num, n, p1, p2, s);                        \
    }                                                                                                              \
    inline int select_unique(void* t, size_t tb, const TT* in, TT* out, uint32_t* num, uint64_t n, uint64_t mask,  \
                             void* s) {                                                                            \
        return lcpp_hip_select_unique_##TS(t, tb, in, out, num, n, mask, s);                                       \
    }                                                                                                              \
    inline int run_length_encode(void* t, size_t tb, const TT* in, TT* uo, uint32_t* co, uint32_t* num,           \
                                 uint64_t n, void* s) {                                                            \
        return lcpp_hip_run_length_encode_##TS(t, tb, in, uo, co, num, n, s);                                      \
    }                                                                                                              \
    inline int run_length_non_trivial(void* t, size_t tb, const TT* in, uint32_t* oo, uint32_t* lo, uint32_t* num, \
                                      uint64_t n, void* s) {                                                       \
        return lcpp_hip_run_length_non_trivial_##TS(t, tb, in, oo, lo, num, n, s);                                 \
    }                                                                                                              \
    LCPP_FACADE_COMPACT_FLAGS(TS, TT, b8, uint8_t)                                                                 \
    LCPP_FACADE_COMPACT_FLAGS(TS, TT, i32, int32_t)                                                                \
    LCPP_FACADE_COMPACT_FLAGS(TS, TT, u32, uint32_t)                                                               \
    LCPP_FACADE_COMPACT_FLAGS(TS, TT, i64, int64_t)                                                                \
    LCPP_FACADE_COMPACT_FLAGS(TS, TT, u64, uint64_t)                                                               \
    LCPP_FACADE_COMPACT_UBK(TS, TT, i32, int32_t)                                                                  \
    LCPP_FACADE_COMPACT_UBK(TS, TT, u32, uint32_t)                                                                 \
    LCPP_FACADE_COMPACT_UBK(TS, TT, f32, float)                                                                    \
    LCPP_FACADE_COMPACT_UBK(TS, TT, i64, int64_t)                                                                  \
    LCPP_FACADE_COMPACT_UBK(TS, TT, u64, uint64_t)                                                                 \
    LCPP_FACADE_COMPACT_UBK(TS, TT, f64, double)
LCPP_FACADE_COMPACT_ITEMS(i32, int32_t)
LCPP_FACADE_COMPACT_ITEMS(u32, uint32_t)
LCPP_FACADE_COMPACT_ITEMS(f32, float)
LCPP_FACADE_COMPACT_ITEMS(i64, int64_t)
LCPP_FACADE_COMPACT_ITEMS(u64, uint64_t)
LCPP_FACADE_COMPACT_ITEMS(f64, double)
#undef LCPP_FACADE_COMPACT_ITEMS
#undef LCPP_FACADE_COMPACT_UBK
#undef LCPP_FACADE_COMPACT_FLAGS

template <typename T>
inline constexpr bool compact_item_ok = by_key_value_ok<T>;

template <typename T>
auto abi(const T* p) {
    return reinterpret_cast<const by_key_abi_t<T>*>(p);
}
template <typename T>
auto abi(T* p) {
    return reinterpret_cast<by_key_abi_t<T>*>(p);
}
template <typename F>
auto flag_abi(const F* p) {
    return reinterpret_cast<const flag_abi_t<F>*>(p);
}

}  // namespace detail
}  // namespace luisa::parallel_primitive
