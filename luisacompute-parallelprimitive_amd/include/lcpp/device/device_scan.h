// DeviceScan sums over the MI355X C-ABI (lcpp_hip_scan_*), with the reference's module shape
// (src/lcpp/device/device_scan.h:40-49 template, :269-284 create, :295-308 temp query) and entry
// points ExclusiveSum (:370-385), InclusiveSum (:409-422), ExclusiveScan / InclusiveScan /
// InclusiveScanInit with a sum, min or max operator (:321-368; operators common/thread_operators.h:49-74),
// checked like validate_scan_views (:213-226).
// The single-pass kernel is a decoupled look-back over the caller's temp storage.  The by-key
// entry points (:424-597, temp query :310-315; SumOp, MinOp or MaxOp) run lcpp_hip_scan_by_key_{sum,min,max}_*,
// checked like validate_scan_by_key_views (:228-246).
#pragma once

#include <limits>
#include <type_traits>

#include "lcpp/device/by_key_abi.h"
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

    // ---- min / max operators (lcpp_hip_scan_min_* / lcpp_hip_scan_max_*) ---------------------------
    // ExclusiveScan (:321-335) seeds the scan with initial_value; InclusiveScan without one (:337-350)
    // folds the items alone; InclusiveScanInit (:352-368) folds initial_value in front of them.
    template <NumericT T, typename Op>
        requires(std::is_same_v<Op, MinOp> || std::is_same_v<Op, MaxOp>)
    void ExclusiveScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                       size_t num_items, Op, T initial_value) {
        record_minmax<Op>(cmdlist, temp_storage, d_in, d_out, num_items, false, true, initial_value);
    }

    template <NumericT T, typename Op>
        requires(std::is_same_v<Op, MinOp> || std::is_same_v<Op, MaxOp>)
    void InclusiveScan(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                       size_t num_items, Op) {
        record_minmax<Op>(cmdlist, temp_storage, d_in, d_out, num_items, true, false, T(0));
    }

    template <NumericT T, typename Op>
        requires(std::is_same_v<Op, MinOp> || std::is_same_v<Op, MaxOp>)
    void InclusiveScanInit(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in,
                           BufferView<T> d_out, size_t num_items, Op, T initial_value) {
        record_minmax<Op>(cmdlist, temp_storage, d_in, d_out, num_items, true, true, initial_value);
    }

    // ---- by key ---------------------------------------------------------------------------------
    template <typename KeyType, typename ValueType>
    static size_t GetScanByKeyTempStorageBytes(size_t num_items) {
        return lcpp_hip_scan_by_key_temp_bytes_policy(num_items, sizeof(KeyType), sizeof(ValueType),
                                                      static_cast<uint32_t>(BLOCK_SIZE),
                                                      static_cast<uint32_t>(ITEMS_PER_THREAD));
    }

    // The scan operator: SumOp, MinOp or MaxOp.
    template <NumericT KeyType, NumericT ValueType, typename Op>
        requires(detail::by_key_op_ok<Op>)
    void ExclusiveScanByKey(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                            BufferView<ValueType> d_values_in, BufferView<ValueType> d_values_out, Op op,
                            size_t num_items, ValueType initial_value, KeyMaskEquality equality_op = {}) {
        record_by_key(op, cmdlist, temp_storage, d_keys_in, d_values_in, d_values_out, num_items, false, true,
                      initial_value, equality_op, "DeviceScan::ExclusiveScanByKey");
    }

    template <NumericT KeyType, NumericT ValueType, typename Op>
        requires(detail::by_key_op_ok<Op>)
    void InclusiveScanByKey(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                            BufferView<ValueType> d_values_in, BufferView<ValueType> d_values_out, Op op,
                            size_t num_items, KeyMaskEquality equality_op = {}) {
        record_by_key(op, cmdlist, temp_storage, d_keys_in, d_values_in, d_values_out, num_items, true, false,
                      ValueType(0), equality_op, "DeviceScan::InclusiveScanByKey");
    }

    // Inclusive scan with `initial_value` prepended to every segment (device_scan.h:488-519).
    template <NumericT KeyType, NumericT ValueType, typename Op>
        requires(detail::by_key_op_ok<Op>)
    void InclusiveScanByKey(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                            BufferView<ValueType> d_values_in, BufferView<ValueType> d_values_out, Op op,
                            size_t num_items, ValueType initial_value, KeyMaskEquality equality_op = {}) {
        record_by_key(op, cmdlist, temp_storage, d_keys_in, d_values_in, d_values_out, num_items, true, true,
                      initial_value, equality_op, "DeviceScan::InclusiveScanByKey");
    }

    template <NumericT KeyType, NumericT ValueType>
    void ExclusiveSumByKey(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                           BufferView<ValueType> d_values_in, BufferView<ValueType> d_values_out, size_t num_items,
                           KeyMaskEquality equality_op = {}) {
        record_by_key(SumOp{}, cmdlist, temp_storage, d_keys_in, d_values_in, d_values_out, num_items, false, true,
                      ValueType(0), equality_op, "DeviceScan::ExclusiveSumByKey");
    }

    template <NumericT KeyType, NumericT ValueType>
    void InclusiveSumByKey(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                           BufferView<ValueType> d_values_in, BufferView<ValueType> d_values_out, size_t num_items,
                           KeyMaskEquality equality_op = {}) {
        record_by_key(SumOp{}, cmdlist, temp_storage, d_keys_in, d_values_in, d_values_out, num_items, true, false,
                      ValueType(0), equality_op, "DeviceScan::InclusiveSumByKey");
    }

  private:
    template <typename Op, NumericT KeyType, NumericT ValueType>
    void record_by_key(Op op, CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<KeyType> d_keys_in,
                       BufferView<ValueType> d_values_in, BufferView<ValueType> d_values_out, size_t num_items,
                       bool inclusive, bool use_init, ValueType init, KeyMaskEquality equality_op, const char* what) {
        static_assert(detail::by_key_key_ok<KeyType>, "scan by key takes 4- or 8-byte integer keys");
        static_assert(detail::by_key_value_ok<ValueType>, "scan by key takes 4- or 8-byte integers, float or double");
        LCPP_ASSERT(m_created, "DeviceScan::create must be called before dispatch.");
        LCPP_ASSERT(num_items <= std::numeric_limits<uint>::max(), "Too many items for DeviceScan.");
        if (num_items == 0u) return;
        LCPP_ASSERT(d_keys_in.size() >= num_items, "DeviceScan key view is too small.");
        LCPP_ASSERT(d_values_in.size() >= num_items, "DeviceScan value view is too small.");
        LCPP_ASSERT(d_values_out.size() >= num_items, "DeviceScan output view is too small.");
        LCPP_ASSERT(temp_storage.size() >=
                        bytes_to_uint_count(GetScanByKeyTempStorageBytes<KeyType, ValueType>(num_items)),
                    "DeviceScan temporary storage is too small.");
        using KA = detail::by_key_abi_t<KeyType>;
        using VA = detail::by_key_abi_t<ValueType>;
        uint* temp = temp_storage.data();
        const size_t temp_bytes = temp_storage.size_bytes();
        const KA* keys = reinterpret_cast<const KA*>(d_keys_in.data());
        const VA* in = reinterpret_cast<const VA*>(d_values_in.data());
        VA* out = reinterpret_cast<VA*>(d_values_out.data());
        const VA init_abi = static_cast<VA>(init);
        const int inc = inclusive ? 1 : 0;
        const int with_init = use_init ? 1 : 0;
        const uint64_t mask = equality_op.mask;
        cmdlist << [=](hipStream_t s) {
            const int rc = detail::scan_by_key(op, temp, temp_bytes, keys, in, out, num_items, inc, with_init,
                                               init_abi, mask, detail::stream_ptr(s));
            luisa::detail::abi_check(rc, what);
        };
    }

    template <NumericT T>
    void record(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                size_t num_items, bool inclusive, T init) {
        static_assert((std::is_integral_v<T> && (sizeof(T) == 4 || sizeof(T) == 8) && !std::is_same_v<T, bool>) ||
                          std::is_same_v<T, float> || std::is_same_v<T, double>,
                      "DeviceScan sums support 4- and 8-byte integers, float and double");
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
            // Integer sums wrap, so signed and unsigned items of one width share the unsigned entry point.
            if constexpr (std::is_same_v<T, float>) {
                rc = lcpp_hip_scan_sum_init_f32(temp, temp_bytes, in, out, num_items, inc, init, st);
            } else if constexpr (std::is_same_v<T, double>) {
                rc = lcpp_hip_scan_sum_init_f64(temp, temp_bytes, in, out, num_items, inc, init, st);
            } else if constexpr (sizeof(T) == 4) {
                rc = lcpp_hip_scan_sum_init_u32(temp, temp_bytes, reinterpret_cast<const uint32_t*>(in),
                                                reinterpret_cast<uint32_t*>(out), num_items, inc,
                                                static_cast<uint32_t>(init), st);
            } else {
                rc = lcpp_hip_scan_sum_init_u64(temp, temp_bytes, reinterpret_cast<const uint64_t*>(in),
                                                reinterpret_cast<uint64_t*>(out), num_items, inc,
                                                static_cast<uint64_t>(init), st);
            }
            luisa::detail::abi_check(rc, inc ? "DeviceScan::InclusiveSum" : "DeviceScan::ExclusiveSum");
        };
    }

    template <typename Op, NumericT T>
    void record_minmax(CommandList& cmdlist, BufferView<uint> temp_storage, BufferView<T> d_in, BufferView<T> d_out,
                       size_t num_items, bool inclusive, bool use_init, T init) {
        static_assert((std::is_integral_v<T> && (sizeof(T) == 4 || sizeof(T) == 8) && !std::is_same_v<T, bool>) ||
                          std::is_same_v<T, float> || std::is_same_v<T, double>,
                      "DeviceScan min / max support 4- and 8-byte integers, float and double");
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
        const int inc = inclusive ? 1 : 0, ui = use_init ? 1 : 0;
        constexpr bool is_min = std::is_same_v<Op, MinOp>;
        cmdlist << [=](hipStream_t s) {
            void* st = detail::stream_ptr(s);
            int rc;
            // Signed and unsigned items compare differently, so each has its own entry point.
#define LCPP_SCAN_MINMAX_CALL(SFX, U)                                                                           \
    rc = is_min ? lcpp_hip_scan_min_##SFX(temp, temp_bytes, reinterpret_cast<const U*>(in), reinterpret_cast<U*>(out), \
                                          num_items, inc, ui, static_cast<U>(init), st)                          \
                : lcpp_hip_scan_max_##SFX(temp, temp_bytes, reinterpret_cast<const U*>(in), reinterpret_cast<U*>(out), \
                                          num_items, inc, ui, static_cast<U>(init), st)
            if constexpr (std::is_same_v<T, float>) LCPP_SCAN_MINMAX_CALL(f32, float);
            else if constexpr (std::is_same_v<T, double>) LCPP_SCAN_MINMAX_CALL(f64, double);
            else if constexpr (sizeof(T) == 4 && std::is_signed_v<T>) LCPP_SCAN_MINMAX_CALL(i32, int32_t);
            else if constexpr (sizeof(T) == 4) LCPP_SCAN_MINMAX_CALL(u32, uint32_t);
            else if constexpr (std::is_signed_v<T>) LCPP_SCAN_MINMAX_CALL(i64, int64_t);
            else LCPP_SCAN_MINMAX_CALL(u64, uint64_t);
#undef LCPP_SCAN_MINMAX_CALL
            luisa::detail::abi_check(rc, is_min ? "DeviceScan::Scan(MinOp)" : "DeviceScan::Scan(MaxOp)");
        };
    }
};

}  // namespace luisa::parallel_primitive
