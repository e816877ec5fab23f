// DeviceSegmentedScan over the MI355X C-ABI (lcpp_hip_segmented_scan_sum_*), with the reference's
// module shape (src/lcpp/device/device_segmented_scan.h:17-56: template, create, GetTempStorageBytes)
// and its sum entry points ExclusiveSegmentedSum / InclusiveSegmentedSum and the Scan / ScanInit forms
// with SumOp, each with or without separate output offsets (:58-224), checked like dispatch_scan
// (:564-590).  Other scan operators are device lambdas and have no counterpart here.
#pragma once

#include <limits>
#include <type_traits>

#include "lcpp/device/segmented_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE = 256>
class DeviceSegmentedScan : public LuisaModule {
  public:
    void create(Device& device) { create_module(device); }

    template <NumericT T>
    [[nodiscard]] static constexpr size_t GetTempStorageBytes(size_t, size_t) noexcept {
        return 0u;
    }

    template <NumericT T>
    void ExclusiveSegmentedSum(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                               BufferView<T> output, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,
                               size_t num_segments) {
        record(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, begin_offsets, num_segments, false,
               true, T{});
    }
    template <NumericT T>
    void ExclusiveSegmentedSum(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                               BufferView<T> output, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,
                               BufferView<uint> output_begin_offsets, size_t num_segments) {
        record(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, output_begin_offsets, num_segments,
               false, true, T{});
    }
    template <NumericT T>
    void ExclusiveSegmentedScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                                BufferView<T> output, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,
                                size_t num_segments, SumOp, T initial_value) {
        record(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, begin_offsets, num_segments, false,
               true, initial_value);
    }
    template <NumericT T>
    void ExclusiveSegmentedScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                                BufferView<T> output, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,
                                BufferView<uint> output_begin_offsets, size_t num_segments, SumOp, T initial_value) {
        record(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, output_begin_offsets, num_segments,
               false, true, initial_value);
    }
    template <NumericT T>
    void InclusiveSegmentedSum(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                               BufferView<T> output, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,
                               size_t num_segments) {
        record(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, begin_offsets, num_segments, true,
               false, T{});
    }
    template <NumericT T>
    void InclusiveSegmentedSum(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                               BufferView<T> output, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,
                               BufferView<uint> output_begin_offsets, size_t num_segments) {
        record(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, output_begin_offsets, num_segments,
               true, false, T{});
    }
    template <NumericT T>
    void InclusiveSegmentedScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                                BufferView<T> output, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,
                                size_t num_segments, SumOp) {
        InclusiveSegmentedSum(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, num_segments);
    }
    template <NumericT T>
    void InclusiveSegmentedScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                                BufferView<T> output, BufferView<uint> begin_offsets, BufferView<uint> end_offsets,
                                BufferView<uint> output_begin_offsets, size_t num_segments, SumOp) {
        InclusiveSegmentedSum(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, output_begin_offsets,
                              num_segments);
    }
    template <NumericT T>
    void InclusiveSegmentedScanInit(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                                    BufferView<T> output, BufferView<uint> begin_offsets,
                                    BufferView<uint> end_offsets, size_t num_segments, SumOp, T initial_value) {
        record(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, begin_offsets, num_segments, true,
               true, initial_value);
    }
    template <NumericT T>
    void InclusiveSegmentedScanInit(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> input,
                                    BufferView<T> output, BufferView<uint> begin_offsets,
                                    BufferView<uint> end_offsets, BufferView<uint> output_begin_offsets,
                                    size_t num_segments, SumOp, T initial_value) {
        record(cmdlist, temp_storage, input, output, begin_offsets, end_offsets, output_begin_offsets, num_segments,
               true, true, initial_value);
    }

  private:
    template <NumericT T>
    void record(CommandList& cmdlist, BufferView<uint>, BufferView<T> input, BufferView<T> output,
                BufferView<uint> begin_offsets, BufferView<uint> end_offsets, BufferView<uint> output_begin_offsets,
                size_t num_segments, bool inclusive, bool use_init, T init) {
        static_assert(detail::by_key_value_ok<T>, "DeviceSegmentedScan: 4- or 8-byte numbers");
        LCPP_ASSERT(m_created, "DeviceSegmentedScan::create must be called before dispatch.");
        LCPP_ASSERT(num_segments <= std::numeric_limits<uint>::max(), "Too many segments for DeviceSegmentedScan.");
        if (num_segments == 0u) return;
        LCPP_ASSERT(begin_offsets.size() >= num_segments, "DeviceSegmentedScan begin-offset view is too small.");
        LCPP_ASSERT(end_offsets.size() >= num_segments, "DeviceSegmentedScan end-offset view is too small.");
        LCPP_ASSERT(output_begin_offsets.size() >= num_segments,
                    "DeviceSegmentedScan output-begin-offset view is too small.");
        using A = detail::by_key_abi_t<T>;
        const A* in = reinterpret_cast<const A*>(input.data());
        A* out = reinterpret_cast<A*>(output.data());
        const uint32_t* b = begin_offsets.data();
        const uint32_t* e = end_offsets.data();
        const uint32_t* ob = output_begin_offsets.data();
        const int inc = inclusive ? 1 : 0, with_init = use_init ? 1 : 0;
        const A init_abi = static_cast<A>(init);
        cmdlist << [=](hipStream_t s) {
            luisa::detail::abi_check(detail::segmented_scan_sum(in, out, b, e, ob, num_segments, inc, with_init,
                                                                init_abi, detail::stream_ptr(s)),
                                     inc ? "DeviceSegmentedScan::InclusiveSegmentedSum"
                                         : "DeviceSegmentedScan::ExclusiveSegmentedSum");
        };
    }
};

}  // namespace luisa::parallel_primitive
