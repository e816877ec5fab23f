// DeviceSelect over the MI355X C-ABI (lcpp_hip_select_*), with the reference's module shape
// (src/lcpp/device/device_select.h:19-63: template, create, GetTempStorageBytes) and entry points
// Flagged / If / FlaggedIf / Unique / UniqueByKey in copy and in-place forms (:65-344), checked like
// validate_views / validate_in_place_views (:346-374).  Predicates are ItemPredicate<T> (the
// reference's Callable<bool(T)> device lambdas have no run-time compiler here); key equalities are
// KeyMaskEquality (all ones = lhs == rhs; floats always compare by value).
#pragma once

#include <limits>
#include <type_traits>

#include "lcpp/device/compact_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE = 256, size_t WARP_NUMS = 32, size_t ITEMS_PER_THREAD = 4>
class DeviceSelect : public LuisaModule {
  public:
    void create(Device& device) { create_module(device); }

    [[nodiscard]] static size_t GetTempStorageBytes(size_t num_items) {
        return lcpp_hip_select_temp_bytes_policy(num_items, static_cast<uint32_t>(BLOCK_SIZE),
                                                 static_cast<uint32_t>(ITEMS_PER_THREAD));
    }

    template <NumericT T, NumericT FlagT>
    void Flagged(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                 BufferView<FlagT> selection_flags, BufferView<T> output, BufferView<uint> num_selected_out,
                 size_t num_items) {
        flagged(cmdlist, temp_storage, input, selection_flags, output, num_selected_out, num_items, static_cast<const ItemPredicate<FlagT>*>(nullptr),
                "DeviceSelect::Flagged");
    }

    template <NumericT T, NumericT FlagT>
    void Flagged(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> data,
                 BufferView<FlagT> selection_flags, BufferView<uint> num_selected_out, size_t num_items) {
        flagged(cmdlist, temp_storage, data, selection_flags, data, num_selected_out, num_items, static_cast<const ItemPredicate<FlagT>*>(nullptr),
                "DeviceSelect::Flagged");
    }

    template <NumericT T>
    void If(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input, BufferView<T> output,
            BufferView<uint> num_selected_out, size_t num_items, const ItemPredicate<T>& predicate) {
        validate(temp_storage, input, output, num_selected_out, num_items);
        if (num_items == 0u) return write_zero(cmdlist, num_selected_out);
        record(cmdlist, temp_storage, num_selected_out, num_items, "DeviceSelect::If",
               [in = input.data(), out = output.data(), p = predicate.c_predicate()](
                   void* t, size_t tb, uint32_t* num, uint64_t n, void* s) {
                   return detail::select_if(t, tb, detail::abi(in), detail::abi(out), num, n, &p, s);
               });
    }

    template <NumericT T>
    void If(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> data,
            BufferView<uint> num_selected_out, size_t num_items, const ItemPredicate<T>& predicate) {
        If(cmdlist, temp_storage, data, data, num_selected_out, num_items, predicate);
    }

    template <NumericT T, NumericT FlagT>
    void FlaggedIf(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                   BufferView<FlagT> selection_flags, BufferView<T> output, BufferView<uint> num_selected_out,
                   size_t num_items, const ItemPredicate<FlagT>& predicate) {
        flagged(cmdlist, temp_storage, input, selection_flags, output, num_selected_out, num_items, &predicate,
                "DeviceSelect::FlaggedIf");
    }

    template <NumericT T, NumericT FlagT>
    void FlaggedIf(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> data,
                   BufferView<FlagT> selection_flags, BufferView<uint> num_selected_out, size_t num_items,
                   const ItemPredicate<FlagT>& predicate) {
        flagged(cmdlist, temp_storage, data, selection_flags, data, num_selected_out, num_items, &predicate,
                "DeviceSelect::FlaggedIf");
    }

    template <NumericT T>
    void Unique(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input, BufferView<T> output,
                BufferView<uint> num_selected_out, size_t num_items, KeyMaskEquality equality = {}) {
        validate(temp_storage, input, output, num_selected_out, num_items);
        if (num_items == 0u) return write_zero(cmdlist, num_selected_out);
        record(cmdlist, temp_storage, num_selected_out, num_items, "DeviceSelect::Unique",
               [in = input.data(), out = output.data(), mask = equality.mask](void* t, size_t tb, uint32_t* num,
                                                                              uint64_t n, void* s) {
                   return detail::select_unique(t, tb, detail::abi(in), detail::abi(out), num, n, mask, s);
               });
    }

    template <NumericT T>
    void Unique(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> data,
                BufferView<uint> num_selected_out, size_t num_items, KeyMaskEquality equality = {}) {
        Unique(cmdlist, temp_storage, data, data, num_selected_out, num_items, equality);
    }

    template <NumericT KeyT, NumericT ValueT>
    void UniqueByKey(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyT> keys_input,
                     BufferView<ValueT> values_input, BufferView<KeyT> keys_output, BufferView<ValueT> values_output,
                     BufferView<uint> num_selected_out, size_t num_items, KeyMaskEquality equality = {}) {
        validate(temp_storage, keys_input, keys_output, num_selected_out, num_items);
        LCPP_ASSERT(values_input.size() >= num_items, "Input value view is too small.");
        LCPP_ASSERT(values_output.size() >= num_items, "Output value view is too small.");
        static_assert(detail::compact_item_ok<ValueT>, "DeviceSelect values: 4- or 8-byte numbers");
        if (num_items == 0u) return write_zero(cmdlist, num_selected_out);
        record(cmdlist, temp_storage, num_selected_out, num_items, "DeviceSelect::UniqueByKey",
               [k = keys_input.data(), v = values_input.data(), ko = keys_output.data(), vo = values_output.data(),
                mask = equality.mask](void* t, size_t tb, uint32_t* num, uint64_t n, void* s) {
                   return detail::select_unique_by_key(t, tb, detail::abi(k), detail::abi(v), detail::abi(ko),
                                                       detail::abi(vo), num, n, mask, s);
               });
    }

  private:
    template <NumericT T, NumericT FlagT>
    void flagged(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                 BufferView<FlagT> selection_flags, BufferView<T> output, BufferView<uint> num_selected_out,
                 size_t num_items, const ItemPredicate<FlagT>* predicate, const char* what) {
        static_assert(detail::flag_ok<FlagT>, "DeviceSelect flags: bool or 4- / 8-byte integers");
        validate(temp_storage, input, output, num_selected_out, num_items);
        LCPP_ASSERT(selection_flags.size() >= num_items, "Selection flag view is too small.");
        if (num_items == 0u) return write_zero(cmdlist, num_selected_out);
        const bool has_pred = predicate != nullptr;
        const lcpp_hip_predicate p = has_pred ? predicate->c_predicate() : lcpp_hip_predicate{};
        record(cmdlist, temp_storage, num_selected_out, num_items, what,
               [in = input.data(), f = selection_flags.data(), out = output.data(), has_pred, p](
                   void* t, size_t tb, uint32_t* num, uint64_t n, void* s) {
                   if (has_pred)
                       return detail::select_flagged_if(t, tb, detail::abi(in), detail::flag_abi(f), detail::abi(out),
                                                        num, n, &p, s);
                   return detail::select_flagged(t, tb, detail::abi(in), detail::flag_abi(f), detail::abi(out), num,
                                                 n, s);
               });
    }

    template <NumericT T>
    void validate(BufferView<uint> temp_storage, BufferView<T> input, BufferView<T> output,
                  BufferView<uint> num_selected_out, size_t num_items) const {
        static_assert(detail::compact_item_ok<T>, "DeviceSelect items: 4- or 8-byte numbers");
        LCPP_ASSERT(m_created, "DeviceSelect::create must be called before dispatch.");
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DeviceSelect.");
        LCPP_ASSERT(input.size() >= num_items, "Input view is too small.");
        LCPP_ASSERT(output.size() >= num_items, "Output view is too small.");
        LCPP_ASSERT(num_selected_out.size() >= 1u, "Selected-count output is empty.");
        LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetTempStorageBytes(num_items)),
                    "DeviceSelect temporary storage is too small.");
    }

    // n == 0 writes a zero count (device_select.h:384-396), with the library's fill kernel.
    static void write_zero(CommandList& cmdlist, BufferView<uint> num_selected_out) {
        uint32_t* num = num_selected_out.data();
        cmdlist << [num](hipStream_t s) {
            luisa::detail::abi_check(
                lcpp_hip_select_unique_u32(nullptr, 0, nullptr, nullptr, num, 0, ~uint64_t(0), detail::stream_ptr(s)),
                "DeviceSelect (empty input)");
        };
    }

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
