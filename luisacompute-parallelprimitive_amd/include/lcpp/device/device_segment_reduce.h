// DeviceSegmentReduce over the MI355X C-ABI (lcpp_hip_segment_*), with the reference's module shape
// (src/lcpp/device/device_segment_reduce.h:60-104: template, create, GetTempStorageBytes,
// GetArgTempStorageBytes) and entry points Sum / Min / Max / ArgMin / ArgMax / Argmin over begin/end
// offsets or a fixed segment size (:151-420).  num_segments == 0 records nothing.  The general
// Reduce(…, ReduceOp, initial) form takes device lambdas and has no counterpart here.
#pragma once

#include <limits>
#include <type_traits>

#include "lcpp/device/segmented_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE = 256, size_t WARP_NUMS = 32, size_t ITEMS_PER_THREAD = 4>
class DeviceSegmentReduce : public LuisaModule {
  public:
    void create(Device& device, Stream* debug_stream = nullptr, InteropContext* interop = nullptr) {
        (void)debug_stream;
        (void)interop;
        create_module(device);
    }

    template <typename T>
    static size_t GetTempStorageBytes(size_t) {
        return 0u;
    }

    template <typename T>
    static size_t GetArgTempStorageBytes(size_t num_item, size_t num_segments) {
        return lcpp_hip_segment_reduce_arg_temp_bytes(num_item, num_segments);
    }

#define LCPP_SEGMENT_REDUCE_METHOD(NAME, OPS)                                                                      \
    template <NumericT T>                                                                                          \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,       \
              uint num_segments, BufferView<uint> d_begin_offsets, BufferView<uint> d_end_offsets) {              \
        (void)temp_storage;                                                                                        \
        if (!check(d_out, num_segments)) return;                                                                   \
        LCPP_ASSERT(d_begin_offsets.size() >= num_segments && d_end_offsets.size() >= num_segments,               \
                    "DeviceSegmentReduce offset views are too small.");                                            \
        using A = detail::by_key_abi_t<T>;                                                                         \
        const A* in = reinterpret_cast<const A*>(d_in.data());                                                     \
        A* out = reinterpret_cast<A*>(d_out.data());                                                               \
        const uint32_t* b = d_begin_offsets.data();                                                                \
        const uint32_t* e = d_end_offsets.data();                                                                  \
        cmdlist << [=](hipStream_t s) {                                                                            \
            luisa::detail::abi_check(detail::segment_reduce_##OPS(in, out, num_segments, b, e, detail::stream_ptr(s)), \
                                     "DeviceSegmentReduce::" #NAME);                                              \
        };                                                                                                         \
    }                                                                                                              \
    template <NumericT T>                                                                                          \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,       \
              uint num_segments, uint segment_size) {                                                              \
        (void)temp_storage;                                                                                        \
        if (!check(d_out, num_segments)) return;                                                                   \
        LCPP_ASSERT(d_in.size() >= static_cast<size_t>(num_segments) * segment_size,                              \
                    "DeviceSegmentReduce input view is too small.");                                               \
        using A = detail::by_key_abi_t<T>;                                                                         \
        const A* in = reinterpret_cast<const A*>(d_in.data());                                                     \
        A* out = reinterpret_cast<A*>(d_out.data());                                                               \
        cmdlist << [=](hipStream_t s) {                                                                            \
            luisa::detail::abi_check(                                                                              \
                detail::segment_reduce_fixed_##OPS(in, out, num_segments, segment_size, detail::stream_ptr(s)),    \
                "DeviceSegmentReduce::" #NAME);                                                                    \
        };                                                                                                         \
    }
    LCPP_SEGMENT_REDUCE_METHOD(Sum, sum)
    LCPP_SEGMENT_REDUCE_METHOD(Min, min)
    LCPP_SEGMENT_REDUCE_METHOD(Max, max)
#undef LCPP_SEGMENT_REDUCE_METHOD

#define LCPP_SEGMENT_ARG_METHOD(NAME, OPS)                                                                         \
    template <NumericT T>                                                                                          \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,       \
              BufferView<uint> d_index_out, uint num_segments, BufferView<uint> d_begin_offsets,                  \
              BufferView<uint> d_end_offsets) {                                                                    \
        static_assert(sizeof(T) == 4, "ArgMin / ArgMax take 4-byte values");                                       \
        (void)temp_storage;                                                                                        \
        if (!check(d_out, num_segments)) return;                                                                   \
        LCPP_ASSERT(d_index_out.size() >= num_segments, "DeviceSegmentReduce index output view is too small.");    \
        LCPP_ASSERT(d_begin_offsets.size() >= num_segments && d_end_offsets.size() >= num_segments,               \
                    "DeviceSegmentReduce offset views are too small.");                                            \
        using A = detail::by_key_abi_t<T>;                                                                         \
        const A* in = reinterpret_cast<const A*>(d_in.data());                                                     \
        A* out = reinterpret_cast<A*>(d_out.data());                                                               \
        uint32_t* idx = d_index_out.data();                                                                        \
        const uint32_t* b = d_begin_offsets.data();                                                                \
        const uint32_t* e = d_end_offsets.data();                                                                  \
        cmdlist << [=](hipStream_t s) {                                                                            \
            luisa::detail::abi_check(detail::segment_##OPS(in, out, idx, num_segments, b, e, detail::stream_ptr(s)), \
                                     "DeviceSegmentReduce::" #NAME);                                              \
        };                                                                                                         \
    }                                                                                                              \
    template <NumericT T>                                                                                          \
    void NAME(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,       \
              BufferView<uint> d_index_out, uint num_segments, uint segment_size) {                                \
        static_assert(sizeof(T) == 4, "ArgMin / ArgMax take 4-byte values");                                       \
        (void)temp_storage;                                                                                        \
        if (!check(d_out, num_segments)) return;                                                                   \
        LCPP_ASSERT(d_index_out.size() >= num_segments, "DeviceSegmentReduce index output view is too small.");    \
        using A = detail::by_key_abi_t<T>;                                                                         \
        const A* in = reinterpret_cast<const A*>(d_in.data());                                                     \
        A* out = reinterpret_cast<A*>(d_out.data());                                                               \
        uint32_t* idx = d_index_out.data();                                                                        \
        cmdlist << [=](hipStream_t s) {                                                                            \
            luisa::detail::abi_check(                                                                              \
                detail::segment_fixed_##OPS(in, out, idx, num_segments, segment_size, detail::stream_ptr(s)),      \
                "DeviceSegmentReduce::" #NAME);                                                                    \
        };                                                                                                         \
    }
    LCPP_SEGMENT_ARG_METHOD(ArgMin, argmin)
    LCPP_SEGMENT_ARG_METHOD(ArgMax, argmax)
#undef LCPP_SEGMENT_ARG_METHOD

    // Alias of ArgMin (device_segment_reduce.h:408-420).
    template <NumericT T>
    void Argmin(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, uint num_segments, BufferView<uint> d_begin_offsets,
                BufferView<uint> d_end_offsets) {
        ArgMin(cmdlist, temp_storage, d_in, d_out, d_index_out, num_segments, d_begin_offsets, d_end_offsets);
    }

  private:
    template <typename T>
    bool check(BufferView<T> d_out, uint num_segments) const {
        static_assert(detail::by_key_value_ok<T>, "DeviceSegmentReduce: 4- or 8-byte numbers");
        LCPP_ASSERT(m_created, "DeviceSegmentReduce::create must be called before dispatch.");
        if (num_segments == 0u) return false;
        LCPP_ASSERT(d_out.size() >= num_segments, "DeviceSegmentReduce output view is too small.");
        return true;
    }
};

}  // namespace luisa::parallel_primitive
