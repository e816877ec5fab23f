// Overloads binding the segmented facade (DeviceSegmentReduce, DeviceSegmentedScan) to the C-ABI
// symbols lcpp_hip_segment_* and lcpp_hip_segmented_scan_sum_*.
#pragma once

#include <cstdint>

#include "lcpp/device/by_key_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive::detail {

#define LCPP_FACADE_SEGMENT_OP(OPS, TS, TT)                                                                         \
    inline int segment_reduce_##OPS(const TT* in, TT* out, uint64_t m, const uint32_t* b, const uint32_t* e,       \
                                    void* s) {                                                                      \
        return lcpp_hip_segment_reduce_##OPS##_##TS(nullptr, 0, in, out, m, b, e, s);                               \
    }                                                                                                               \
    inline int segment_reduce_fixed_##OPS(const TT* in, TT* out, uint64_t m, uint32_t size, void* s) {              \
        return lcpp_hip_segment_reduce_fixed_##OPS##_##TS(nullptr, 0, in, out, m, size, s);                         \
    }
#define LCPP_FACADE_SEGMENT_ARG(OPS, TS, TT)                                                                        \
    inline int segment_##OPS(const TT* in, TT* out, uint32_t* idx, uint64_t m, const uint32_t* b, const uint32_t* e, \
                             void* s) {                                                                             \
        return lcpp_hip_segment_##OPS##_##TS(nullptr, 0, in, out, idx, m, b, e, s);                                 \
    }                                                                                                               \
    inline int segment_fixed_##OPS(const TT* in, TT* out, uint32_t* idx, uint64_t m, uint32_t size, void* s) {      \
        return lcpp_hip_segment_fixed_##OPS##_##TS(nullptr, 0, in, out, idx, m, size, s);                           \
    }
#define LCPP_FACADE_SEGMENTED(TS, TT)                                                                               \
    LCPP_FACADE_SEGMENT_OP(sum, TS, TT)                                                                             \
    LCPP_FACADE_SEGMENT_OP(min, TS, TT)                                                                             \
    LCPP_FACADE_SEGMENT_OP(max, TS, TT)                                                                             \
    inline int segmented_scan_sum(const TT* in, TT* out, const uint32_t* b, const uint32_t* e, const uint32_t* ob,  \
                                  uint64_t m, int inclusive, int use_init, TT init, void* s) {                      \
        return lcpp_hip_segmented_scan_sum_##TS(nullptr, 0, in, out, b, e, ob, m, inclusive, use_init, init, s);    \
    }
LCPP_FACADE_SEGMENTED(i32, int32_t)
LCPP_FACADE_SEGMENTED(u32, uint32_t)
LCPP_FACADE_SEGMENTED(f32, float)
LCPP_FACADE_SEGMENTED(i64, int64_t)
LCPP_FACADE_SEGMENTED(u64, uint64_t)
LCPP_FACADE_SEGMENTED(f64, double)
LCPP_FACADE_SEGMENT_ARG(argmin, i32, int32_t)
LCPP_FACADE_SEGMENT_ARG(argmin, u32, uint32_t)
LCPP_FACADE_SEGMENT_ARG(argmin, f32, float)
LCPP_FACADE_SEGMENT_ARG(argmax, i32, int32_t)
LCPP_FACADE_SEGMENT_ARG(argmax, u32, uint32_t)
LCPP_FACADE_SEGMENT_ARG(argmax, f32, float)
#undef LCPP_FACADE_SEGMENTED
#undef LCPP_FACADE_SEGMENT_ARG
#undef LCPP_FACADE_SEGMENT_OP

}  // namespace luisa::parallel_primitive::detail
