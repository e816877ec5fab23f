// DeviceSpmv::CsrMV (y = A * x, CSR) over the MI355X C-ABI (lcpp_hip_spmv_csr_*), with the reference's
// module shape (src/lcpp/device/device_spmv.h:19-46) and record-time checks (validate_views, :157-186).
// rows == 0 records nothing; nnz == 0 zero-fills y (:61-68).
#pragma once

#include <concepts>
#include <limits>
#include <type_traits>

#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE = 256>
class DeviceSpmv : public LuisaModule {
    static constexpr size_t WARP_SIZE = 32;  // the reference's rows-per-launch bound keeps its 32-lane rows

  public:
    void create(Device& device) { create_module(device); }

    [[nodiscard]] static constexpr size_t GetTempStorageBytes(size_t, size_t, size_t) noexcept { return 0u; }

    template <NumericT ValueT, std::integral IndexT>
    void CsrMV(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<ValueT> values,
               BufferView<IndexT> row_offsets, BufferView<IndexT> column_indices, BufferView<ValueT> vector_x,
               BufferView<ValueT> vector_y, size_t num_rows, size_t num_cols, size_t num_nonzeros) {
        static_assert(std::is_same_v<ValueT, float> || std::is_same_v<ValueT, double> ||
                          std::is_same_v<ValueT, int32_t> || std::is_same_v<ValueT, uint32_t>,
                      "DeviceSpmv values: float, double, int or uint");
        static_assert(sizeof(IndexT) == 4, "DeviceSpmv indices: int or uint");
        LCPP_ASSERT(m_created, "DeviceSpmv::create must be called before dispatch.");
        LCPP_ASSERT(num_rows <= std::numeric_limits<uint>::max() / WARP_SIZE, "Too many rows for DeviceSpmv.");
        LCPP_ASSERT(num_cols <= std::numeric_limits<uint>::max(), "Too many columns for DeviceSpmv.");
        LCPP_ASSERT(num_nonzeros <= std::numeric_limits<uint>::max(), "Too many nonzero values for DeviceSpmv.");
        if (num_rows == 0u) return;
        LCPP_ASSERT(row_offsets.size() >= num_rows + 1u, "DeviceSpmv row-offset view is too small.");
        LCPP_ASSERT(vector_y.size() >= num_rows, "DeviceSpmv output-vector view is too small.");
        if (num_nonzeros > 0u) {
            LCPP_ASSERT(values.size() >= num_nonzeros, "DeviceSpmv value view is too small.");
            LCPP_ASSERT(column_indices.size() >= num_nonzeros, "DeviceSpmv column-index view is too small.");
            LCPP_ASSERT(vector_x.size() >= num_cols, "DeviceSpmv input-vector view is too small.");
            LCPP_ASSERT(num_cols > 0u, "A DeviceSpmv matrix with zero columns cannot contain nonzero values.");
        }
        uint* temp = temp_storage.data();
        const size_t tb = temp_storage.size_bytes();
        const ValueT* a = values.data();
        const IndexT* ro = row_offsets.data();
        const IndexT* ci = column_indices.data();
        const ValueT* x = vector_x.data();
        ValueT* y = vector_y.data();
        cmdlist << [=](hipStream_t s) {
            void* st = detail::stream_ptr(s);
            int rc;
#define LCPP_FACADE_SPMV(V, VT)                                                                                  \
    if constexpr (std::is_signed_v<IndexT>)                                                                      \
        rc = lcpp_hip_spmv_csr_##V##_i32(temp, tb, reinterpret_cast<const VT*>(a),                              \
                                         reinterpret_cast<const int32_t*>(ro), reinterpret_cast<const int32_t*>(ci), \
                                         reinterpret_cast<const VT*>(x), reinterpret_cast<VT*>(y), num_rows,    \
                                         num_cols, num_nonzeros, st);                                            \
    else                                                                                                         \
        rc = lcpp_hip_spmv_csr_##V##_u32(temp, tb, reinterpret_cast<const VT*>(a),                              \
                                         reinterpret_cast<const uint32_t*>(ro),                                  \
                                         reinterpret_cast<const uint32_t*>(ci), reinterpret_cast<const VT*>(x), \
                                         reinterpret_cast<VT*>(y), num_rows, num_cols, num_nonzeros, st);
            if constexpr (std::is_same_v<ValueT, float>) { LCPP_FACADE_SPMV(f32, float) }
            else if constexpr (std::is_same_v<ValueT, double>) { LCPP_FACADE_SPMV(f64, double) }
            else if constexpr (std::is_same_v<ValueT, int32_t>) { LCPP_FACADE_SPMV(i32, int32_t) }
            else { LCPP_FACADE_SPMV(u32, uint32_t) }
#undef LCPP_FACADE_SPMV
            luisa::detail::abi_check(rc, "DeviceSpmv::CsrMV");
        };
    }
};

}  // namespace luisa::parallel_primitive
