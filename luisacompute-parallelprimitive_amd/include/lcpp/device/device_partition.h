// DevicePartition over the MI355X C-ABI (lcpp_hip_partition_*), with the reference's module shape
// (src/lcpp/device/device_partition.h:19-71: template, create, GetTempStorageBytes,
// GetThreeWayTempStorageBytes) and entry points Flagged / If / three-way If (:73-209), checked like
// _validate_views / _validate_three_way_views (:228-268).  Selected items keep their order at the
// front, rejected items follow in reverse order; the three-way form writes both category sizes.
#pragma once

#include <limits>
#include <type_traits>

#include "lcpp/device/compact_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE = 256, size_t WARP_NUMS = 32, size_t ITEMS_PER_THREAD = 4>
class DevicePartition : public LuisaModule {
  public:
    void create(Device& device) { create_module(device); }

    [[nodiscard]] static size_t GetTempStorageBytes(size_t num_items) {
        return lcpp_hip_select_temp_bytes_policy(num_items, static_cast<uint32_t>(BLOCK_SIZE),
                                                 static_cast<uint32_t>(ITEMS_PER_THREAD));
    }

    [[nodiscard]] static size_t GetThreeWayTempStorageBytes(size_t num_items) {
        return lcpp_hip_partition_three_way_temp_bytes_policy(num_items, static_cast<uint32_t>(BLOCK_SIZE),
                                                              static_cast<uint32_t>(ITEMS_PER_THREAD));
    }

    template <NumericT T, NumericT FlagT>
    void Flagged(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                 BufferView<FlagT> selection_flags, BufferView<T> output, BufferView<uint> num_selected_out,
                 size_t num_items) {
        static_assert(detail::flag_ok<FlagT>, "DevicePartition flags: bool or 4- / 8-byte integers");
        validate(temp_storage, input, output, num_selected_out, num_items, GetTempStorageBytes(num_items));
        LCPP_ASSERT(selection_flags.size() >= num_items, "Partition flag view is too small.");
        const T* in = input.data();
        const FlagT* f = selection_flags.data();
        T* out = output.data();
        record(cmdlist, temp_storage, num_selected_out, num_items, "DevicePartition::Flagged",
               [=](void* t, size_t tb, uint32_t* num, uint64_t n, void* s) {
                   return detail::partition_flagged(t, tb, detail::abi(in), detail::flag_abi(f), detail::abi(out),
                                                    num, n, s);
               });
    }

    template <NumericT T>
    void If(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input, BufferView<T> output,
            BufferView<uint> num_selected_out, size_t num_items, const ItemPredicate<T>& predicate) {
        validate(temp_storage, input, output, num_selected_out, num_items, GetTempStorageBytes(num_items));
        const T* in = input.data();
        T* out = output.data();
        const lcpp_hip_predicate p = predicate.c_predicate();
        record(cmdlist, temp_storage, num_selected_out, num_items, "DevicePartition::If",
               [=](void* t, size_t tb, uint32_t* num, uint64_t n, void* s) {
                   return detail::partition_if(t, tb, detail::abi(in), detail::abi(out), num, n, &p, s);
               });
    }

    template <NumericT T>
    void If(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input, BufferView<T> first_output,
            BufferView<T> second_output, BufferView<T> unselected_output, BufferView<uint> num_selected_out,
            size_t num_items, const ItemPredicate<T>& select_first, const ItemPredicate<T>& select_second) {
        validate(temp_storage, input, first_output, num_selected_out, num_items,
                 GetThreeWayTempStorageBytes(num_items));
        LCPP_ASSERT(second_output.size() >= num_items, "Partition second output view is too small.");
        LCPP_ASSERT(unselected_output.size() >= num_items, "Partition unselected output view is too small.");
        LCPP_ASSERT(num_selected_out.size() >= 2u, "Three-way partition selected-count output requires two items.");
        const T* in = input.data();
        T* o1 = first_output.data();
        T* o2 = second_output.data();
        T* o3 = unselected_output.data();
        const lcpp_hip_predicate p1 = select_first.c_predicate(), p2 = select_second.c_predicate();
        record(cmdlist, temp_storage, num_selected_out, num_items, "DevicePartition::If (three-way)",
               [=](void* t, size_t tb, uint32_t* num, uint64_t n, void* s) {
                   return detail::partition_three_way(t, tb, detail::abi(in), detail::abi(o1), detail::abi(o2),
                                                      detail::abi(o3), num, n, &p1, &p2, s);
               });
    }

  private:
    template <NumericT T>
    void validate(BufferView<uint> temp_storage, BufferView<T> input, BufferView<T> output,
                  BufferView<uint> num_selected_out, size_t num_items, size_t temp_bytes) const {
        static_assert(detail::compact_item_ok<T>, "DevicePartition items: 4- or 8-byte numbers");
        LCPP_ASSERT(m_created, "DevicePartition::create must be called before dispatch.");
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DevicePartition.");
        LCPP_ASSERT(input.size() >= num_items, "Partition input view is too small.");
        LCPP_ASSERT(output.size() >= num_items, "Partition output view is too small.");
        LCPP_ASSERT(num_selected_out.size() >= 1u, "Partition selected-count output is empty.");
        LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(temp_bytes),
                    "DevicePartition temporary storage is too small.");
    }

    // Every call goes to the library, which writes zero counts for n == 0 with its fill kernel.
    template <typename F>
    static void record(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<uint> num_selected_out,
                       size_t num_items, const char* what, F call) {
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        uint32_t* num = num_selected_out.data();
        cmdlist << [=](hipStream_t s) {
            luisa::detail::abi_check(call(temp, temp_bytes, num, num_items, detail::stream_ptr(s)), what);
        };
    }
};

}  // namespace luisa::parallel_primitive
