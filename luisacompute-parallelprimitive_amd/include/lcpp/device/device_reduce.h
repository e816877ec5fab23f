// DeviceReduce::Sum / Min / Max / ArgMin / ArgMax / Reduce / TransformReduce over the MI355X C-ABI
// (lcpp_hip_reduce_{sum,min,max,argmin,argmax}_*, lcpp_hip_transform_reduce_*), with the reference's module
// shape (src/lcpp/device/device_reduce.h:102-113 template, :154-173 create, :184-210 temp queries,
// :229-252 Reduce, :280-436 Sum to ArgMax, :491-515 TransformReduce) and its record-time checks (:238-264).  Sum records one command; the kernels run on
// the stream the command list is committed to.  ReduceByKey with a sum operator (:437-487, temp
// query :207-223) with SumOp, MinOp or MaxOp runs lcpp_hip_reduce_by_key_{sum,min,max}_*, which writes 0
// runs for empty input (:449-458).
#pragma once

#include <limits>
#include <type_traits>

#include "lcpp/device/by_key_abi.h"
#include "lcpp/runtime/core.h"

namespace luisa::parallel_primitive {

template <size_t BLOCK_SIZE = 256, size_t WARP_NUMS = 32, size_t ITEMS_PER_THREAD = 8, bool CUDA_WARP_REDUX = false,
          bool AUTO_CUDA_TUNED_POLICY = true>
class DeviceReduce : public LuisaModule {
  public:
    void create(Device& device, Stream* debug_stream = nullptr, InteropContext* interop = nullptr) {
        (void)debug_stream;
        (void)interop;
        create_module(device);
    }

    // Same bytes as the reference formula for this tile (device_reduce.h:517-536).
    template <typename T>
    static size_t GetTempStorageBytes(size_t num_item) {
        return lcpp_hip_reduce_temp_bytes_policy(num_item, sizeof(T), static_cast<uint32_t>(BLOCK_SIZE),
                                                 static_cast<uint32_t>(ITEMS_PER_THREAD));
    }

    // Temp bytes of ReduceByKey: tiles of REDUCE_BY_KEY_ITEMS_PER_THREAD (4) x BLOCK_SIZE items.
    template <typename KeyType, typename ValueType>
    static size_t GetReduceByKeyTempStorageBytes(size_t num_elements) {
        return lcpp_hip_reduce_by_key_temp_bytes_policy(num_elements, sizeof(KeyType), sizeof(ValueType),
                                                        static_cast<uint32_t>(BLOCK_SIZE));
    }

    // Runs of equal keys (under `equality_op`) reduce to (first key, aggregate); g_num_runs_out[0] = runs.
    // d_unique_out and g_aggregates_out must hold one element per run.
    // The reduce operator: SumOp, MinOp or MaxOp.
    template <NumericT KeyType, NumericT ValueType, typename Op>
        requires(detail::by_key_op_ok<Op>)
    void ReduceByKey(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                     BufferView<ValueType> d_values_in, BufferView<KeyType> d_unique_out,
                     BufferView<ValueType> g_aggregates_out, BufferView<uint> g_num_runs_out, Op op,
                     size_t num_elements, KeyMaskEquality equality_op = {}) {
        static_assert(detail::by_key_key_ok<KeyType>, "ReduceByKey takes 4- or 8-byte integer keys");
        static_assert(detail::by_key_value_ok<ValueType>, "ReduceByKey takes 4- or 8-byte integers, float or double");
        LCPP_ASSERT(m_created, "DeviceReduce::create must be called before dispatch.");
        LCPP_ASSERT(num_elements <= std::numeric_limits<uint>::max(), "Too many items for DeviceReduce.");
        LCPP_ASSERT(g_num_runs_out.size() >= 1u, "DeviceReduce run-count output view is empty.");
        if (num_elements > 0) {
            LCPP_ASSERT(d_keys_in.size() >= num_elements, "DeviceReduce key view is too small.");
            LCPP_ASSERT(d_values_in.size() >= num_elements, "DeviceReduce value view is too small.");
            LCPP_ASSERT(temp_storage.size() >=
                            bytes_to_uint_count(GetReduceByKeyTempStorageBytes<KeyType, ValueType>(num_elements)),
                        "DeviceReduce temporary storage is too small.");
        }
        using KA = detail::by_key_abi_t<KeyType>;
        using VA = detail::by_key_abi_t<ValueType>;
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        const KA* keys = reinterpret_cast<const KA*>(d_keys_in.data());
        const VA* values = reinterpret_cast<const VA*>(d_values_in.data());
        KA* unique = reinterpret_cast<KA*>(d_unique_out.data());
        VA* aggregates = reinterpret_cast<VA*>(g_aggregates_out.data());
        uint32_t* runs = g_num_runs_out.data();
        const uint64_t mask = equality_op.mask;
        cmdlist << [=](hipStream_t s) {
            const int rc = detail::reduce_by_key(op, temp, temp_bytes, keys, values, unique, aggregates, runs,
                                                 num_elements, mask, detail::stream_ptr(s));
            luisa::detail::abi_check(rc, "DeviceReduce::ReduceByKey");
        };
    }

    // Temp bytes of ArgMin / ArgMax: the reference's layout of (index, value) pairs (:198-210).
    template <typename T>
    static size_t GetArgTempStorageBytes(size_t num_item) {
        return lcpp_hip_reduce_arg_temp_bytes(num_item, sizeof(T));
    }

    // The smallest / largest item, folded from the type's max / lowest (an empty input writes it).
    template <NumericT T>
    void Min(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             size_t num_item) {
        record_ext<false>(cmdlist, temp_storage, d_in, d_out, num_item);
    }
    template <NumericT T>
    void Max(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             size_t num_item) {
        record_ext<true>(cmdlist, temp_storage, d_in, d_out, num_item);
    }

    // The smallest / largest item and its index (the lowest among equal items); an empty input writes
    // the type's max / lowest and index 1.
    template <NumericT T>
    void ArgMin(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, size_t num_item) {
        record_arg<false>(cmdlist, temp_storage, d_in, d_out, d_index_out, num_item);
    }
    template <NumericT T>
    void ArgMax(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                BufferView<uint> d_index_out, size_t num_item) {
        record_arg<true>(cmdlist, temp_storage, d_in, d_out, d_index_out, num_item);
    }

    // Reduce with SumOp, MinOp or MaxOp and an initial value (device_reduce.h:229-252):
    // d_out[0] = op(initial_value, fold of the items); an empty input writes initial_value.
    template <NumericT T, typename ReduceOp>
        requires(detail::by_key_op_ok<ReduceOp>)
    void Reduce(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                size_t num_item, ReduceOp reduce_op, T initial_value) {
        record_transform(cmdlist, temp_storage, d_in, d_out, num_item, reduce_op, IdentityOp{}, initial_value,
                         "DeviceReduce::Reduce");
    }

    // TransformReduce (device_reduce.h:491-515): d_out[0] = op(init, fold of transform_op(item)); the
    // transform is IdentityOp, AffineOp<T>{scale, shift}, SquareOp or AbsOp.
    template <NumericT T, typename ReduceOp, typename TransformOp>
        requires(detail::by_key_op_ok<ReduceOp>)
    void TransformReduce(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                         size_t num_item, ReduceOp reduce_op, TransformOp transform_op, T init) {
        record_transform(cmdlist, temp_storage, d_in, d_out, num_item, reduce_op, transform_op, init,
                         "DeviceReduce::TransformReduce");
    }

    template <NumericT T>
    void Sum(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
             size_t num_item) {
        static_assert(sizeof(T) == 4 || sizeof(T) == 8, "DeviceReduce::Sum supports 4- and 8-byte numbers");
        LCPP_ASSERT(m_created, "DeviceReduce::create must be called before dispatch.");
        LCPP_ASSERT(num_item <= std::numeric_limits<uint>::max(), "Too many items for DeviceReduce.");
        LCPP_ASSERT(d_out.size() >= 1u, "DeviceReduce output view is empty.");
        if (num_item > 0) {
            LCPP_ASSERT(d_in.size() >= num_item, "DeviceReduce input view is too small.");
            LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetTempStorageBytes<T>(num_item)),
                        "DeviceReduce temporary storage is too small.");
        }
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        const T* in = d_in.data();
        T* out = d_out.data();
        cmdlist << [=](hipStream_t s) {
            void* st = detail::stream_ptr(s);
            int rc;
            if constexpr (std::is_same_v<T, int32_t>) rc = lcpp_hip_reduce_sum_i32(temp, temp_bytes, in, out, num_item, st);
            else if constexpr (std::is_same_v<T, uint32_t>) rc = lcpp_hip_reduce_sum_u32(temp, temp_bytes, in, out, num_item, st);
            else if constexpr (std::is_same_v<T, float>) rc = lcpp_hip_reduce_sum_f32(temp, temp_bytes, in, out, num_item, st);
            else if constexpr (std::is_integral_v<T> && std::is_signed_v<T> && sizeof(T) == 8)
                rc = lcpp_hip_reduce_sum_i64(temp, temp_bytes, reinterpret_cast<const int64_t*>(in),
                                             reinterpret_cast<int64_t*>(out), num_item, st);
            else if constexpr (std::is_integral_v<T> && std::is_unsigned_v<T> && sizeof(T) == 8)
                rc = lcpp_hip_reduce_sum_u64(temp, temp_bytes, reinterpret_cast<const uint64_t*>(in),
                                             reinterpret_cast<uint64_t*>(out), num_item, st);
            else if constexpr (std::is_same_v<T, double>) rc = lcpp_hip_reduce_sum_f64(temp, temp_bytes, in, out, num_item, st);
            else static_assert(sizeof(T) == 0, "DeviceReduce::Sum: unsupported element type");
            luisa::detail::abi_check(rc, "DeviceReduce::Sum");
        };
    }

  private:
    // The C-ABI suffix type of T: signed and unsigned integers compare differently, so each keeps its own.
    template <typename T>
    using ExtAbi = std::conditional_t<std::is_floating_point_v<T>, T,
                                      std::conditional_t<std::is_signed_v<T>,
                                                         std::conditional_t<sizeof(T) == 4, int32_t, int64_t>,
                                                         std::conditional_t<sizeof(T) == 4, uint32_t, uint64_t>>>;

    template <NumericT T, typename ReduceOp, typename TransformOp>
    void record_transform(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                          size_t num_item, ReduceOp, TransformOp transform_op, T init, const char* what) {
        static_assert(sizeof(T) == 4 || sizeof(T) == 8, "DeviceReduce::Reduce supports 4- and 8-byte numbers");
        LCPP_ASSERT(m_created, "DeviceReduce::create must be called before dispatch.");
        LCPP_ASSERT(num_item <= std::numeric_limits<uint>::max(), "Too many items for DeviceReduce.");
        LCPP_ASSERT(d_out.size() >= 1u, "DeviceReduce output view is empty.");
        if (num_item > 0) {
            LCPP_ASSERT(d_in.size() >= num_item, "DeviceReduce input view is too small.");
            LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetTempStorageBytes<T>(num_item)),
                        "DeviceReduce temporary storage is too small.");
        }
        constexpr int op = std::is_same_v<ReduceOp, SumOp>   ? LCPP_HIP_REDUCE_SUM
                           : std::is_same_v<ReduceOp, MinOp> ? LCPP_HIP_REDUCE_MIN
                                                             : LCPP_HIP_REDUCE_MAX;
        int transform = LCPP_HIP_TRANSFORM_IDENTITY;
        T scale = T(0), shift = T(0);
        if constexpr (std::is_same_v<TransformOp, AffineOp<T>>) {
            transform = LCPP_HIP_TRANSFORM_AFFINE;
            scale = transform_op.scale;
            shift = transform_op.shift;
        } else if constexpr (std::is_same_v<TransformOp, SquareOp>) {
            transform = LCPP_HIP_TRANSFORM_SQUARE;
        } else if constexpr (std::is_same_v<TransformOp, AbsOp>) {
            transform = LCPP_HIP_TRANSFORM_ABS;
        } else {
            static_assert(std::is_same_v<TransformOp, IdentityOp>,
                          "TransformReduce takes IdentityOp, AffineOp<T>, SquareOp or AbsOp");
        }
        using A = ExtAbi<T>;
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        const A* in = reinterpret_cast<const A*>(d_in.data());
        A* out = reinterpret_cast<A*>(d_out.data());
        const A a_scale = static_cast<A>(scale), a_shift = static_cast<A>(shift), a_init = static_cast<A>(init);
        cmdlist << [=](hipStream_t s) {
            void* st = detail::stream_ptr(s);
            int rc;
            if constexpr (std::is_same_v<A, int32_t>)
                rc = lcpp_hip_transform_reduce_i32(temp, temp_bytes, in, out, num_item, op, transform, a_scale, a_shift, a_init, st);
            else if constexpr (std::is_same_v<A, uint32_t>)
                rc = lcpp_hip_transform_reduce_u32(temp, temp_bytes, in, out, num_item, op, transform, a_scale, a_shift, a_init, st);
            else if constexpr (std::is_same_v<A, float>)
                rc = lcpp_hip_transform_reduce_f32(temp, temp_bytes, in, out, num_item, op, transform, a_scale, a_shift, a_init, st);
            else if constexpr (std::is_same_v<A, int64_t>)
                rc = lcpp_hip_transform_reduce_i64(temp, temp_bytes, in, out, num_item, op, transform, a_scale, a_shift, a_init, st);
            else if constexpr (std::is_same_v<A, uint64_t>)
                rc = lcpp_hip_transform_reduce_u64(temp, temp_bytes, in, out, num_item, op, transform, a_scale, a_shift, a_init, st);
            else
                rc = lcpp_hip_transform_reduce_f64(temp, temp_bytes, in, out, num_item, op, transform, a_scale, a_shift, a_init, st);
            luisa::detail::abi_check(rc, what);
        };
    }

    template <bool MAX, NumericT T>
    void record_ext(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                    size_t num_item) {
        static_assert(sizeof(T) == 4 || sizeof(T) == 8, "DeviceReduce::Min / Max support 4- and 8-byte numbers");
        LCPP_ASSERT(m_created, "DeviceReduce::create must be called before dispatch.");
        LCPP_ASSERT(num_item <= std::numeric_limits<uint>::max(), "Too many items for DeviceReduce.");
        LCPP_ASSERT(d_out.size() >= 1u, "DeviceReduce output view is empty.");
        if (num_item > 0) {
            LCPP_ASSERT(d_in.size() >= num_item, "DeviceReduce input view is too small.");
            LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetTempStorageBytes<T>(num_item)),
                        "DeviceReduce temporary storage is too small.");
        }
        using A = ExtAbi<T>;
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        const A* in = reinterpret_cast<const A*>(d_in.data());
        A* out = reinterpret_cast<A*>(d_out.data());
        cmdlist << [=](hipStream_t s) {
            void* st = detail::stream_ptr(s);
            int rc;
#define LCPP_REDUCE_EXT_CALL(SFX, U)                                                                          \
    rc = MAX ? lcpp_hip_reduce_max_##SFX(temp, temp_bytes, reinterpret_cast<const U*>(in), reinterpret_cast<U*>(out), \
                                         num_item, st)                                                          \
             : lcpp_hip_reduce_min_##SFX(temp, temp_bytes, reinterpret_cast<const U*>(in), reinterpret_cast<U*>(out), \
                                         num_item, st)
            if constexpr (std::is_same_v<A, int32_t>) LCPP_REDUCE_EXT_CALL(i32, int32_t);
            else if constexpr (std::is_same_v<A, uint32_t>) LCPP_REDUCE_EXT_CALL(u32, uint32_t);
            else if constexpr (std::is_same_v<A, float>) LCPP_REDUCE_EXT_CALL(f32, float);
            else if constexpr (std::is_same_v<A, int64_t>) LCPP_REDUCE_EXT_CALL(i64, int64_t);
            else if constexpr (std::is_same_v<A, uint64_t>) LCPP_REDUCE_EXT_CALL(u64, uint64_t);
            else LCPP_REDUCE_EXT_CALL(f64, double);
#undef LCPP_REDUCE_EXT_CALL
            luisa::detail::abi_check(rc, MAX ? "DeviceReduce::Max" : "DeviceReduce::Min");
        };
    }

    template <bool MAX, NumericT T>
    void record_arg(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                    BufferView<uint> d_index_out, size_t num_item) {
        static_assert(sizeof(T) == 4 || sizeof(T) == 8, "DeviceReduce::ArgMin / ArgMax support 4- and 8-byte numbers");
        LCPP_ASSERT(m_created, "DeviceReduce::create must be called before dispatch.");
        LCPP_ASSERT(num_item <= std::numeric_limits<uint>::max(), "Too many items for DeviceReduce.");
        LCPP_ASSERT(d_out.size() >= 1u && d_index_out.size() >= 1u, "DeviceReduce output view is empty.");
        if (num_item > 0) {
            LCPP_ASSERT(d_in.size() >= num_item, "DeviceReduce input view is too small.");
            LCPP_ASSERT(temp_storage.size() >= bytes_to_uint_count(GetArgTempStorageBytes<T>(num_item)),
                        "DeviceReduce temporary storage is too small.");
        }
        using A = ExtAbi<T>;
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        const A* in = reinterpret_cast<const A*>(d_in.data());
        A* out = reinterpret_cast<A*>(d_out.data());
        uint32_t* index = d_index_out.data();
        cmdlist << [=](hipStream_t s) {
            void* st = detail::stream_ptr(s);
            int rc;
#define LCPP_REDUCE_ARG_CALL(SFX, U)                                                                             \
    rc = MAX ? lcpp_hip_reduce_argmax_##SFX(temp, temp_bytes, reinterpret_cast<const U*>(in), reinterpret_cast<U*>(out), \
                                            index, num_item, st)                                                   \
             : lcpp_hip_reduce_argmin_##SFX(temp, temp_bytes, reinterpret_cast<const U*>(in), reinterpret_cast<U*>(out), \
                                            index, num_item, st)
            if constexpr (std::is_same_v<A, int32_t>) LCPP_REDUCE_ARG_CALL(i32, int32_t);
            else if constexpr (std::is_same_v<A, uint32_t>) LCPP_REDUCE_ARG_CALL(u32, uint32_t);
            else if constexpr (std::is_same_v<A, float>) LCPP_REDUCE_ARG_CALL(f32, float);
            else if constexpr (std::is_same_v<A, int64_t>) LCPP_REDUCE_ARG_CALL(i64, int64_t);
            else if constexpr (std::is_same_v<A, uint64_t>) LCPP_REDUCE_ARG_CALL(u64, uint64_t);
            else LCPP_REDUCE_ARG_CALL(f64, double);
#undef LCPP_REDUCE_ARG_CALL
            luisa::detail::abi_check(rc, MAX ? "DeviceReduce::ArgMax" : "DeviceReduce::ArgMin");
        };
    }
};

}  // namespace luisa::parallel_primitive
