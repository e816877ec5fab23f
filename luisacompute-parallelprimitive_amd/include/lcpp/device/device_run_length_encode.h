// DeviceRunLengthEncode over the MI355X C-ABI (lcpp_hip_run_length_*), with the reference's module
// shape (src/lcpp/device/device_run_length_encode.h:19-69: template, create, GetTempStorageBytes) and
// entry points Encode / NonTrivialRuns (:71-153), checked like validate_common /
// validate_encode_views / validate_non_trivial_views (:286-324).  n == 0 writes a zero run count.
#pragma once

#include <limits>
#include <type_traits>

#include "lcpp/device/compact_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE = 256, size_t WARP_NUMS = 32, size_t ITEMS_PER_THREAD = 4>
class DeviceRunLengthEncode : public LuisaModule {
  public:
    void create(Device& device) { create_module(device); }

    [[nodiscard]] static size_t GetTempStorageBytes(size_t num_items) {
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DeviceRunLengthEncode.");
        return lcpp_hip_run_length_encode_temp_bytes_policy(num_items, static_cast<uint32_t>(BLOCK_SIZE),
                                                            static_cast<uint32_t>(ITEMS_PER_THREAD));
    }

    template <NumericT T>
    void Encode(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input, BufferView<T> unique_output,
                BufferView<uint> counts_output, BufferView<uint> num_runs_output, size_t num_items) {
        validate(temp_storage, num_runs_output, num_items);
        LCPP_ASSERT(input.size() >= num_items, "DeviceRunLengthEncode input view is too small.");
        LCPP_ASSERT(unique_output.size() >= num_items, "DeviceRunLengthEncode unique output view is too small.");
        LCPP_ASSERT(counts_output.size() >= num_items, "DeviceRunLengthEncode counts output view is too small.");
        static_assert(detail::compact_item_ok<T>, "DeviceRunLengthEncode items: 4- or 8-byte numbers");
        const T* in = input.data();
        T* uo = unique_output.data();
        uint32_t* co = counts_output.data();
        record(cmdlist, temp_storage, num_runs_output, num_items, "DeviceRunLengthEncode::Encode",
               [=](void* t, size_t tb, uint32_t* num, uint64_t n, void* s) {
                   return detail::run_length_encode(t, tb, detail::abi(in), detail::abi(uo), co, num, n, s);
               });
    }

    template <NumericT T>
    void NonTrivialRuns(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                        BufferView<uint> offsets_output, BufferView<uint> lengths_output,
                        BufferView<uint> num_runs_output, size_t num_items) {
        validate(temp_storage, num_runs_output, num_items);
        LCPP_ASSERT(input.size() >= num_items, "DeviceRunLengthEncode input view is too small.");
        LCPP_ASSERT(offsets_output.size() >= num_items, "DeviceRunLengthEncode offsets output view is too small.");
        LCPP_ASSERT(lengths_output.size() >= num_items, "DeviceRunLengthEncode lengths output view is too small.");
        static_assert(detail::compact_item_ok<T>, "DeviceRunLengthEncode items: 4- or 8-byte numbers");
        const T* in = input.data();
        uint32_t* oo = offsets_output.data();
        uint32_t* lo = lengths_output.data();
        record(cmdlist, temp_storage, num_runs_output, num_items, "DeviceRunLengthEncode::NonTrivialRuns",
               [=](void* t, size_t tb, uint32_t* num, uint64_t n, void* s) {
                   return detail::run_length_non_trivial(t, tb, detail::abi(in), oo, lo, num, n, s);
               });
    }

  private:
    void validate(BufferView<uint> temp_storage, BufferView<uint> num_runs_output, size_t num_items) const {
        LCPP_ASSERT(m_created, "DeviceRunLengthEncode::create must be called before dispatch.");
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DeviceRunLengthEncode.");
        LCPP_ASSERT(num_runs_output.size() >= 1u, "DeviceRunLengthEncode run-count output is empty.");
        if (num_items != 0u)
            LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetTempStorageBytes(num_items)),
                        "DeviceRunLengthEncode temporary storage is too small.");
    }

    template <typename F>
    static void record(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<uint> num_runs_output,
                       size_t num_items, const char* what, F call) {
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        uint32_t* num = num_runs_output.data();
        cmdlist << [=](hipStream_t s) {
            luisa::detail::abi_check(call(temp, temp_bytes, num, num_items, detail::stream_ptr(s)), what);
        };
    }
};

}  // namespace luisa::parallel_primitive
