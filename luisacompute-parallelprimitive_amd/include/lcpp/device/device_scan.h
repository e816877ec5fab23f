// DeviceScan sums over the MI355X C-ABI (lcpp_hip_scan_*), with the reference's module shape
// (src/lcpp/device/device_scan.h:40-49 template, :269-284 create, :295-308 temp query) and entry
// points ExclusiveSum (:370-385), InclusiveSum (:409-422), ExclusiveScan / InclusiveScan /
// InclusiveScanInit with a sum operator (:321-368), checked like validate_scan_views (:213-226).
// The single-pass kernel is a decoupled look-back over the caller's temp storage.
#pragma once

#include <limits>
#include <type_traits>

#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

enum class BlockLoadAlgorithm { BLOCK_LOAD_DIRECT, BLOCK_LOAD_WARP_TRANSPOSE, BLOCK_LOAD_VECTORIZE };
enum class BlockStoreAlgorithm { BLOCK_STORE_DIRECT, BLOCK_STORE_WARP_TRANSPOSE, BLOCK_STORE_VECTORIZE };

template <size_t BLOCK_SIZE = 256, size_t WARP_NUMS = 32, size_t ITEMS_PER_THREAD = 15,
          BlockLoadAlgorithm LOAD_ALGORITHM = BlockLoadAlgorithm::BLOCK_LOAD_DIRECT,
          BlockStoreAlgorithm STORE_ALGORITHM = BlockStoreAlgorithm::BLOCK_STORE_DIRECT, bool WARP_SYNC = false,
          bool PACKED_TILE_STATE = false>
class DeviceScan : public LuisaModule {
    static constexpr bool DEFAULT_POLICY = BLOCK_SIZE == 256 && WARP_NUMS == 32 && ITEMS_PER_THREAD == 15 &&
                                           LOAD_ALGORITHM == BlockLoadAlgorithm::BLOCK_LOAD_DIRECT &&
                                           STORE_ALGORITHM == BlockStoreAlgorithm::BLOCK_STORE_DIRECT &&
                                           !WARP_SYNC && !PACKED_TILE_STATE;

  public:
    void create(Device& device, Stream* debug_stream = nullptr, InteropContext* interop = nullptr) {
        (void)debug_stream;
        (void)interop;
        create_module(device);
    }

    template <typename T>
    static size_t GetTempStorageBytes(size_t num_items) {
        return lcpp_hip_scan_temp_bytes_policy(num_items, sizeof(T), static_cast<uint32_t>(BLOCK_SIZE),
                                               static_cast<uint32_t>(ITEMS_PER_THREAD), DEFAULT_POLICY ? 1 : 0,
                                               PACKED_TILE_STATE ? 1 : 0);
    }

    template <NumericT T>
    void ExclusiveSum(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                      size_t num_items) {
        record(cmdlist, temp_storage, d_in, d_out, num_items, false, T(0));
    }

    template <NumericT T>
    void InclusiveSum(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                      size_t num_items) {
        record(cmdlist, temp_storage, d_in, d_out, num_items, true, T(0));
    }

    template <NumericT T>
    void ExclusiveScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                       size_t num_items, SumOp, T initial_value) {
        record(cmdlist, temp_storage, d_in, d_out, num_items, false, initial_value);
    }

    template <NumericT T>
    void InclusiveScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                       size_t num_items, SumOp) {
        record(cmdlist, temp_storage, d_in, d_out, num_items, true, T(0));
    }

    template <NumericT T>
    void InclusiveScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                       size_t num_items, SumOp, T initial_value) {
        record(cmdlist, temp_storage, d_in, d_out, num_items, true, initial_value);
    }

    template <NumericT T>
    void InclusiveScanInit(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in,
                           BufferView<T> d_out, size_t num_items, SumOp, T initial_value) {
        record(cmdlist, temp_storage, d_in, d_out, num_items, true, initial_value);
    }

  private:
    template <NumericT T>
    void record(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                size_t num_items, bool inclusive, T init) {
        static_assert(std::is_same_v<T, int32_t> || std::is_same_v<T, uint32_t> || std::is_same_v<T, float>,
                      "DeviceScan sums support int, uint and float");
        LCPP_ASSERT(m_created, "DeviceScan::create must be called before dispatch.");
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DeviceScan.");
        if (num_items == 0u) return;
        LCPP_ASSERT(d_in.size() >= num_items, "DeviceScan input view is too small.");
        LCPP_ASSERT(d_out.size() >= num_items, "DeviceScan output view is too small.");
        LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetTempStorageBytes<T>(num_items)),
                    "DeviceScan temporary storage is too small.");
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        const T* in = d_in.data();
        T* out = d_out.data();
        const int inc = inclusive ? 1 : 0;
        cmdlist << [=](hipStream_t s) {
            void* st = detail::stream_ptr(s);
            int rc;
            if constexpr (std::is_same_v<T, int32_t>) rc = lcpp_hip_scan_sum_init_i32(temp, temp_bytes, in, out, num_items, inc, init, st);
            else if constexpr (std::is_same_v<T, uint32_t>) rc = lcpp_hip_scan_sum_init_u32(temp, temp_bytes, in, out, num_items, inc, init, st);
            else rc = lcpp_hip_scan_sum_init_f32(temp, temp_bytes, in, out, num_items, inc, init, st);
            luisa::detail::abi_check(rc, inc ? "DeviceScan::InclusiveSum" : "DeviceScan::ExclusiveSum");
        };
    }
};

}  // namespace luisa::parallel_primitive
