/*
 * lcpp_hip.h — C-ABI of the MI355X (gfx950) implementation of the LuisaCompute-ParallelPrimitive
 * (LCPP) device hot path: DeviceReduce::Sum, DeviceScan::ExclusiveSum/InclusiveSum, onesweep
 * DeviceRadixSort::SortKeys/SortPairs and DeviceSpmv::CsrMV.
 *
 * Conventions
 *   - Every pointer argument except `stream` is a device pointer (hipMalloc'd or a sub-range of one).
 *   - `stream` is a hipStream_t passed as void*; NULL means the null stream.  Work is enqueued
 *     asynchronously, in order, on that stream; no entry point synchronises the host (the reference
 *     records into a CommandList that runs on commit, README.md:182-184).
 *   - `temp` / `temp_bytes` is caller-owned scratch of at least the size the matching
 *     *_temp_bytes function returns.  Those functions return exactly the byte counts of the
 *     reference's Get*TempStorageBytes, so a buffer sized for LCPP is always large enough.
 *   - Return value: LCPP_HIP_OK (0) or a negative status; lcpp_hip_last_error() describes it
 *     (thread-local).  The reference aborts through LUISA_ASSERT on the same preconditions.
 *   - One stream per call; calls that share a temp buffer must be ordered on one stream.
 *
 * Element-type suffixes: i32 int32_t, u32 uint32_t, f32 float, i64 int64_t, u64 uint64_t,
 * f64 double.  Value-size suffixes for SortPairs: v32 (any 4-byte value), v64 (any 8-byte value).
 */
#ifndef LCPP_HIP_H_
#define LCPP_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The library is built with hidden visibility; only the declarations below are exported. */
#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

#define LCPP_HIP_OK 0
#define LCPP_HIP_ERR_INVALID_ARGUMENT (-1)
#define LCPP_HIP_ERR_TEMP_TOO_SMALL (-2)
#define LCPP_HIP_ERR_HIP (-3)
#define LCPP_HIP_ERR_UNSUPPORTED (-4)

/* ---------------------------------------------------------------------------------------------
 * Library
 * ------------------------------------------------------------------------------------------- */
const char* lcpp_hip_version(void);
const char* lcpp_hip_last_error(void);

/* Per-kernel device-time accounting (hipEvents recorded around each launch on its stream).
 * No reference counterpart: LCPP relies on external profilers (tests/lcpp_cub_bench.cpp:124-260). */
int lcpp_hip_profile_enable(int enable);
int lcpp_hip_profile_reset(void);
int lcpp_hip_profile_query(const char* kernel, double* total_ms, uint64_t* launches);
int lcpp_hip_profile_names(char* buffer, size_t buffer_bytes);

/* Device-to-device copy of `bytes` bytes on `stream` by a library kernel (16-byte non-temporal lanes
 * in a grid-stride loop when both pointers and the size are 16-byte aligned, 8-byte lanes when they are
 * 8-byte aligned, bytes otherwise).  No reference counterpart: the sorts' zero-width
 * case (begin_bit == end_bit) copies with it, and bench.py times it as the achievable copy rate. */
int lcpp_hip_device_copy(void* dst, const void* src, uint64_t bytes, void* stream);

#ifdef LCPP_HIP_PHASE_TRACE
/* Diagnostic build (liblcpp_hip_trace.so) only: the onesweep and scan kernels write one record of
 * 16 64-bit words per tile to `buffer` (device memory holding `records` records; null stops it).  No
 * counterpart in the reference; its analogue is the per-phase timing of docs/epoch3_radix_sort.md:38-57. */
int lcpp_hip_trace_set_buffer(void* buffer, uint64_t records);
#endif

/* Polls of a look-back predecessor that has not published yet before the waiting workgroup computes
 * that predecessor's contribution from the input itself (scan and onesweep sort).  Any value is
 * correct; 0 takes the fallback at once (used by tests), the default is 64.  Process-wide.
 * No reference counterpart (the reference spins until the predecessor publishes,
 * device/details/single_pass_scan_operator.h:96-113, agent/agent_radix_sort_onesweep.h:309-357). */
int lcpp_hip_set_lookback_spin_limit(uint32_t polls);
uint32_t lcpp_hip_get_lookback_spin_limit(void);

/* ---------------------------------------------------------------------------------------------
 * DeviceReduce::Sum
 * replaces DeviceReduce<>::Sum (src/lcpp/device/device_reduce.h:280-288) and its temp query
 * DeviceReduce<>::GetTempStorageBytes<T> (device_reduce.h:184-189, formula :517-536).
 * n == 0 writes 0 to *out (device_reduce.h:238-243).  Integer sums wrap modulo 2^bits.
 * ------------------------------------------------------------------------------------------- */
size_t lcpp_hip_reduce_temp_bytes_policy(uint64_t n, size_t elem_bytes, uint32_t block_size, uint32_t items_per_thread);
size_t lcpp_hip_reduce_temp_bytes(uint64_t n, size_t elem_bytes); /* default policy 256 x 8 */
int lcpp_hip_reduce_sum_i32(void* temp, size_t temp_bytes, const int32_t* in, int32_t* out, uint64_t n, void* stream);
int lcpp_hip_reduce_sum_u32(void* temp, size_t temp_bytes, const uint32_t* in, uint32_t* out, uint64_t n, void* stream);
int lcpp_hip_reduce_sum_f32(void* temp, size_t temp_bytes, const float* in, float* out, uint64_t n, void* stream);
int lcpp_hip_reduce_sum_i64(void* temp, size_t temp_bytes, const int64_t* in, int64_t* out, uint64_t n, void* stream);
int lcpp_hip_reduce_sum_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint64_t n, void* stream);
int lcpp_hip_reduce_sum_f64(void* temp, size_t temp_bytes, const double* in, double* out, uint64_t n, void* stream);
/* DeviceReduce<>::Min / Max (device_reduce.h:291-309): the fold of the items with the reference's MinOp /
 * MaxOp (common/thread_operators.h:58-74) and its initial value, the type's max / lowest (so an empty
 * input writes that value).  Signed types compare as signed; floats like fmin / fmax (a NaN item is
 * skipped; of -0.0 and +0.0 either may result).  Temp: lcpp_hip_reduce_temp_bytes(n, sizeof(T)). */
#define LCPP_HIP_DECLARE_REDUCE_EXT(S, T)                                                                        \
    int lcpp_hip_reduce_min_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, void* stream);  \
    int lcpp_hip_reduce_max_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, void* stream);  \
    int lcpp_hip_reduce_argmin_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint32_t* out_index,      \
                                   uint64_t n, void* stream);                                                  \
    int lcpp_hip_reduce_argmax_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint32_t* out_index,      \
                                   uint64_t n, void* stream);
/* DeviceReduce<>::ArgMin / ArgMax (device_reduce.h:311-436, ArgMinOp / ArgMaxOp of
 * common/thread_operators.h:10-47): *out = the smallest (largest) item, *out_index = its index, the lowest
 * index among equal items (-0.0 == +0.0); NaN items never win (an all-NaN input gives the initial pair:
 * the type's max / lowest and index 0xFFFFFFFF); n == 0 writes the type's max / lowest and index 1.
 * Temp: lcpp_hip_reduce_arg_temp_bytes(n, sizeof(T)), the reference's GetArgTempStorageBytes (the
 * kernels use 8-12 bytes per workgroup of it). */
LCPP_HIP_DECLARE_REDUCE_EXT(i32, int32_t)
LCPP_HIP_DECLARE_REDUCE_EXT(u32, uint32_t)
LCPP_HIP_DECLARE_REDUCE_EXT(f32, float)
LCPP_HIP_DECLARE_REDUCE_EXT(i64, int64_t)
LCPP_HIP_DECLARE_REDUCE_EXT(u64, uint64_t)
LCPP_HIP_DECLARE_REDUCE_EXT(f64, double)
#undef LCPP_HIP_DECLARE_REDUCE_EXT
size_t lcpp_hip_reduce_arg_temp_bytes(uint64_t n, size_t elem_bytes);

/* DeviceReduce<>::Reduce(cmdlist, temp, in, out, n, reduce_op, initial_value) (device_reduce.h:229-252)
 * and TransformReduce(cmdlist, temp, in, out, n, reduce_op, transform_op, init) (:491-515):
 * *out = op(init, fold over i of op(transform(in[i]))); n == 0 writes init.  The transform is applied
 * to input items only, once each (tests/device_reduce_test.cpp:148-173), and init enters last, on the
 * left, as in the reference's single-tile kernel (device/details/reduce.h:227-237).  The reference
 * takes device callables; this vocabulary covers its tests:
 *   op:        LCPP_HIP_REDUCE_SUM (wrapping for integers), LCPP_HIP_REDUCE_MIN, LCPP_HIP_REDUCE_MAX
 *              (MinOp / MaxOp: signed types compare as signed, floats like fmin / fmax);
 *   transform: LCPP_HIP_TRANSFORM_IDENTITY, LCPP_HIP_TRANSFORM_AFFINE (scale * x + shift: x + c, 2x,
 *              2x + 1 ...), LCPP_HIP_TRANSFORM_SQUARE (x * x), LCPP_HIP_TRANSFORM_ABS (|x|).
 * Integer transforms wrap modulo 2^bits; float transforms round after every operation (no fused
 * multiply-add).  scale / shift are read by the affine transform only.  An unknown op or transform
 * returns LCPP_HIP_ERR_INVALID_ARGUMENT.  Temp: lcpp_hip_reduce_temp_bytes(n, sizeof(T)). */
#define LCPP_HIP_REDUCE_SUM 0
#define LCPP_HIP_REDUCE_MIN 1
#define LCPP_HIP_REDUCE_MAX 2
#define LCPP_HIP_TRANSFORM_IDENTITY 0
#define LCPP_HIP_TRANSFORM_AFFINE 1
#define LCPP_HIP_TRANSFORM_SQUARE 2
#define LCPP_HIP_TRANSFORM_ABS 3
#define LCPP_HIP_DECLARE_REDUCE_OP(S, T)                                                                         \
    int lcpp_hip_reduce_op_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int op, T init, \
                               void* stream);                                                                   \
    int lcpp_hip_transform_reduce_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int op,   \
                                      int transform, T scale, T shift, T init, void* stream);
LCPP_HIP_DECLARE_REDUCE_OP(i32, int32_t)
LCPP_HIP_DECLARE_REDUCE_OP(u32, uint32_t)
LCPP_HIP_DECLARE_REDUCE_OP(f32, float)
LCPP_HIP_DECLARE_REDUCE_OP(i64, int64_t)
LCPP_HIP_DECLARE_REDUCE_OP(u64, uint64_t)
LCPP_HIP_DECLARE_REDUCE_OP(f64, double)
#undef LCPP_HIP_DECLARE_REDUCE_OP

/* ---------------------------------------------------------------------------------------------
 * DeviceScan::ExclusiveSum / InclusiveSum (decoupled look-back, single pass)
 * replaces DeviceScan<>::ExclusiveSum (src/lcpp/device/device_scan.h:370-385),
 * DeviceScan<>::InclusiveSum (device_scan.h:409-422), InclusiveScanInit / ExclusiveScan with a
 * sum operator and an initial value (device_scan.h:321-368), and
 * DeviceScan<>::GetTempStorageBytes<T> (device_scan.h:295-308, layout :111-126).
 * n == 0 is a no-op.  Integer sums wrap modulo 2^bits.
 * ------------------------------------------------------------------------------------------- */
size_t lcpp_hip_scan_temp_bytes_policy(uint64_t n, size_t elem_bytes, uint32_t block_size, uint32_t items_per_thread,
                                       int default_policy, int packed_tile_state);
size_t lcpp_hip_scan_temp_bytes(uint64_t n, size_t elem_bytes); /* default policy 256 x 15 (+ 320 x 25 packed) */
int lcpp_hip_scan_exclusive_sum_i32(void* temp, size_t temp_bytes, const int32_t* in, int32_t* out, uint64_t n, void* stream);
int lcpp_hip_scan_exclusive_sum_u32(void* temp, size_t temp_bytes, const uint32_t* in, uint32_t* out, uint64_t n, void* stream);
int lcpp_hip_scan_exclusive_sum_f32(void* temp, size_t temp_bytes, const float* in, float* out, uint64_t n, void* stream);
int lcpp_hip_scan_exclusive_sum_i64(void* temp, size_t temp_bytes, const int64_t* in, int64_t* out, uint64_t n, void* stream);
int lcpp_hip_scan_exclusive_sum_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint64_t n, void* stream);
int lcpp_hip_scan_exclusive_sum_f64(void* temp, size_t temp_bytes, const double* in, double* out, uint64_t n, void* stream);
int lcpp_hip_scan_inclusive_sum_i32(void* temp, size_t temp_bytes, const int32_t* in, int32_t* out, uint64_t n, void* stream);
int lcpp_hip_scan_inclusive_sum_u32(void* temp, size_t temp_bytes, const uint32_t* in, uint32_t* out, uint64_t n, void* stream);
int lcpp_hip_scan_inclusive_sum_f32(void* temp, size_t temp_bytes, const float* in, float* out, uint64_t n, void* stream);
int lcpp_hip_scan_inclusive_sum_i64(void* temp, size_t temp_bytes, const int64_t* in, int64_t* out, uint64_t n, void* stream);
int lcpp_hip_scan_inclusive_sum_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint64_t n, void* stream);
int lcpp_hip_scan_inclusive_sum_f64(void* temp, size_t temp_bytes, const double* in, double* out, uint64_t n, void* stream);
/* Sum scan with an initial value: exclusive: out[i] = init + sum(in[0..i)); inclusive: init + sum(in[0..i]). */
int lcpp_hip_scan_sum_init_i32(void* temp, size_t temp_bytes, const int32_t* in, int32_t* out, uint64_t n, int inclusive, int32_t init, void* stream);
int lcpp_hip_scan_sum_init_u32(void* temp, size_t temp_bytes, const uint32_t* in, uint32_t* out, uint64_t n, int inclusive, uint32_t init, void* stream);
int lcpp_hip_scan_sum_init_f32(void* temp, size_t temp_bytes, const float* in, float* out, uint64_t n, int inclusive, float init, void* stream);
int lcpp_hip_scan_sum_init_i64(void* temp, size_t temp_bytes, const int64_t* in, int64_t* out, uint64_t n, int inclusive, int64_t init, void* stream);
int lcpp_hip_scan_sum_init_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint64_t n, int inclusive, uint64_t init, void* stream);
int lcpp_hip_scan_sum_init_f64(void* temp, size_t temp_bytes, const double* in, double* out, uint64_t n, int inclusive, double init, void* stream);
/* Min / max scans: DeviceScan<>::ExclusiveScan / InclusiveScan / InclusiveScanInit with MinOp or MaxOp
 * (device_scan.h:321-368, operators common/thread_operators.h:58-74).  exclusive: out[i] = op(init,
 * in[0], ..., in[i-1]) (out[0] = init); inclusive: op(init, in[0], ..., in[i]), init omitted when
 * use_init is 0 (the operator's identity: the type's max / lowest; a quiet NaN for floats, so an
 * exclusive scan's out[0] is NaN).  Signed types compare as signed; floats like fmin / fmax (a NaN
 * operand yields the other one; of -0.0 and +0.0 the earlier is kept). */
int lcpp_hip_scan_min_i32(void* temp, size_t temp_bytes, const int32_t* in, int32_t* out, uint64_t n, int inclusive, int use_init, int32_t init, void* stream);
int lcpp_hip_scan_min_u32(void* temp, size_t temp_bytes, const uint32_t* in, uint32_t* out, uint64_t n, int inclusive, int use_init, uint32_t init, void* stream);
int lcpp_hip_scan_min_f32(void* temp, size_t temp_bytes, const float* in, float* out, uint64_t n, int inclusive, int use_init, float init, void* stream);
int lcpp_hip_scan_min_i64(void* temp, size_t temp_bytes, const int64_t* in, int64_t* out, uint64_t n, int inclusive, int use_init, int64_t init, void* stream);
int lcpp_hip_scan_min_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint64_t n, int inclusive, int use_init, uint64_t init, void* stream);
int lcpp_hip_scan_min_f64(void* temp, size_t temp_bytes, const double* in, double* out, uint64_t n, int inclusive, int use_init, double init, void* stream);
int lcpp_hip_scan_max_i32(void* temp, size_t temp_bytes, const int32_t* in, int32_t* out, uint64_t n, int inclusive, int use_init, int32_t init, void* stream);
int lcpp_hip_scan_max_u32(void* temp, size_t temp_bytes, const uint32_t* in, uint32_t* out, uint64_t n, int inclusive, int use_init, uint32_t init, void* stream);
int lcpp_hip_scan_max_f32(void* temp, size_t temp_bytes, const float* in, float* out, uint64_t n, int inclusive, int use_init, float init, void* stream);
int lcpp_hip_scan_max_i64(void* temp, size_t temp_bytes, const int64_t* in, int64_t* out, uint64_t n, int inclusive, int use_init, int64_t init, void* stream);
int lcpp_hip_scan_max_u64(void* temp, size_t temp_bytes, const uint64_t* in, uint64_t* out, uint64_t n, int inclusive, int use_init, uint64_t init, void* stream);
int lcpp_hip_scan_max_f64(void* temp, size_t temp_bytes, const double* in, double* out, uint64_t n, int inclusive, int use_init, double init, void* stream);
/* DeviceScan<>::ExclusiveScan / InclusiveScan / InclusiveScanInit with the left projection
 * op(lhs, rhs) = lhs (the operator of tests/device_scan_test.cpp:129-155 and
 * tests/scan_optimization_regression_test.cpp:195-205): every output is the scan's first operand, init
 * when use_init, else in[0]; items compare by bits only.  It does not commute, so it runs the general scan
 * kernels with their operand order.  An exclusive scan without init returns LCPP_HIP_ERR_INVALID_ARGUMENT
 * (the operator has no identity).  Temp: lcpp_hip_scan_temp_bytes(n, sizeof(T)). */
#define LCPP_HIP_DECLARE_SCAN_LEFT(S, T)                                                                          \
    int lcpp_hip_scan_left_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int inclusive,     \
                               int use_init, T init, void* stream);
LCPP_HIP_DECLARE_SCAN_LEFT(i32, int32_t)
LCPP_HIP_DECLARE_SCAN_LEFT(u32, uint32_t)
LCPP_HIP_DECLARE_SCAN_LEFT(f32, float)
LCPP_HIP_DECLARE_SCAN_LEFT(i64, int64_t)
LCPP_HIP_DECLARE_SCAN_LEFT(u64, uint64_t)
LCPP_HIP_DECLARE_SCAN_LEFT(f64, double)
#undef LCPP_HIP_DECLARE_SCAN_LEFT
/* ExclusiveSum over uint32 with no temp argument: the same kernels, with their tile status words in a
 * static device array of the library (349,528 bytes per GPU, held until the process ends) instead of
 * caller-provided temp storage, and no allocation of any kind.  No counterpart in the reference: it is
 * for callers that cannot allocate (code under graph capture, allocation-free serving loops).  At most
 * 2^30 items (larger n returns LCPP_HIP_ERR_INVALID_ARGUMENT).  The array used is that of the stream's
 * device.  The first call on a device looks up the device's array and must run outside graph capture
 * (a first call with n > 0 under capture returns LCPP_HIP_ERR_UNSUPPORTED and records nothing); a call
 * with n == 0 does only that lookup, so callers that capture make one such call per device first.
 * Every call on one GPU shares the array: calls that overlap in time on one GPU race (calls in order on
 * one stream are safe, and so are replays of a graph holding such calls, in order on one stream). */
int lcpp_hip_scan_exclusive_sum_u32_noalloc(const uint32_t* in, uint32_t* out, uint64_t n, void* stream);

/* ---------------------------------------------------------------------------------------------
 * DeviceRadixSort (onesweep, 8-bit digits, stable LSD)
 * replaces DeviceRadixSort<>::SortKeys / SortKeysDescending / SortPairs / SortPairsDescending in
 * their copy form (src/lcpp/device/device_radix_sort.h:369-466) and DoubleBuffer form
 * (device_radix_sort.h:468-554), and GetSortKeysTempStorageBytes / GetSortPairsTempStorageBytes
 * (device_radix_sort.h:337-362, layout :212-335).
 * Copy form: keys_in/values_in are never written; results land in keys_out/values_out.
 * DoubleBuffer form: buffers[*selector] holds the input; both buffers may be overwritten; *selector
 * is flipped once per 8-bit pass before the function returns (host-side, like the reference).
 * begin_bit == end_bit copies (copy form) or leaves *selector unchanged (DoubleBuffer form).
 * Float keys order by IEEE total order with -0.0 == +0.0 (common/util_type.h:141-175,
 * agent/radix_rank_sort_operations.h:31-42); signed keys in two's-complement order.
 * ------------------------------------------------------------------------------------------- */
size_t lcpp_hip_radix_sort_temp_bytes_policy(uint32_t n, size_t key_bytes, size_t value_bytes, int keys_only,
                                             uint32_t block_size, uint32_t items_per_thread, int cub_small_key_policy);
size_t lcpp_hip_radix_sort_keys_temp_bytes(uint32_t n, size_t key_bytes);                      /* default policy */
size_t lcpp_hip_radix_sort_pairs_temp_bytes(uint32_t n, size_t key_bytes, size_t value_bytes);  /* default policy */

#define LCPP_HIP_DECLARE_SORT(K, KT)                                                                             \
    int lcpp_hip_radix_sort_keys_##K(void* temp, size_t temp_bytes, const KT* keys_in, KT* keys_out, uint32_t n,  \
                                     uint32_t begin_bit, uint32_t end_bit, int descending, void* stream);         \
    int lcpp_hip_radix_sort_keys_db_##K(void* temp, size_t temp_bytes, KT* keys0, KT* keys1, int* selector,       \
                                        uint32_t n, uint32_t begin_bit, uint32_t end_bit, int descending,         \
                                        void* stream);                                                            \
    int lcpp_hip_radix_sort_pairs_##K##_v32(void* temp, size_t temp_bytes, const KT* keys_in, KT* keys_out,       \
                                            const void* values_in, void* values_out, uint32_t n,                  \
                                            uint32_t begin_bit, uint32_t end_bit, int descending, void* stream);  \
    int lcpp_hip_radix_sort_pairs_##K##_v64(void* temp, size_t temp_bytes, const KT* keys_in, KT* keys_out,       \
                                            const void* values_in, void* values_out, uint32_t n,                  \
                                            uint32_t begin_bit, uint32_t end_bit, int descending, void* stream);  \
    int lcpp_hip_radix_sort_pairs_db_##K##_v32(void* temp, size_t temp_bytes, KT* keys0, KT* keys1,               \
                                               void* values0, void* values1, int* selector, uint32_t n,           \
                                               uint32_t begin_bit, uint32_t end_bit, int descending,              \
                                               void* stream);                                                     \
    int lcpp_hip_radix_sort_pairs_db_##K##_v64(void* temp, size_t temp_bytes, KT* keys0, KT* keys1,               \
                                               void* values0, void* values1, int* selector, uint32_t n,           \
                                               uint32_t begin_bit, uint32_t end_bit, int descending,              \
                                               void* stream);

LCPP_HIP_DECLARE_SORT(u32, uint32_t)
LCPP_HIP_DECLARE_SORT(i32, int32_t)
LCPP_HIP_DECLARE_SORT(f32, float)
LCPP_HIP_DECLARE_SORT(u64, uint64_t)
LCPP_HIP_DECLARE_SORT(i64, int64_t)
LCPP_HIP_DECLARE_SORT(f64, double)
#undef LCPP_HIP_DECLARE_SORT

/* Largest number of keys one onesweep launch ranks before the sort is split into portions.
 * Setting a smaller limit (a multiple of the tile, >= one tile) exercises the multi-portion
 * path on small inputs; 0 restores the default.  Process-wide; not thread-safe with running sorts.
 * Replaces the fixed PORTION_SIZE of device_radix_sort.h:1056. */
int lcpp_hip_radix_set_portion_limit(uint32_t max_items_per_portion);
/* Tile (keys per workgroup) of the onesweep kernel for the given key/value sizes. */
uint32_t lcpp_hip_radix_tile_items(size_t key_bytes, size_t value_bytes);

/* ---------------------------------------------------------------------------------------------
 * DeviceSpmv::CsrMV  y = A * x  (CSR)
 * replaces DeviceSpmv<>::CsrMV (src/lcpp/device/device_spmv.h:48-130) and
 * GetTempStorageBytes == 0 (device_spmv.h:43-46).  rows == 0: no-op; nnz == 0: y[0..rows) = 0;
 * a row whose offsets are decreasing or exceed nnz yields 0; columns >= cols are skipped.
 * Limits (status -1 beyond them): rows < 2^27, cols < 2^32, nnz <= 2^32 - 513.
 * ------------------------------------------------------------------------------------------- */
size_t lcpp_hip_spmv_temp_bytes(uint64_t rows, uint64_t cols, uint64_t nnz);

#define LCPP_HIP_DECLARE_SPMV(V, VT, I, IT)                                                                    \
    int lcpp_hip_spmv_csr_##V##_##I(void* temp, size_t temp_bytes, const VT* values, const IT* row_offsets,    \
                                    const IT* column_indices, const VT* x, VT* y, uint64_t rows, uint64_t cols, \
                                    uint64_t nnz, void* stream);
LCPP_HIP_DECLARE_SPMV(f32, float, i32, int32_t)
LCPP_HIP_DECLARE_SPMV(f32, float, u32, uint32_t)
LCPP_HIP_DECLARE_SPMV(f64, double, i32, int32_t)
LCPP_HIP_DECLARE_SPMV(f64, double, u32, uint32_t)
LCPP_HIP_DECLARE_SPMV(i32, int32_t, i32, int32_t)
LCPP_HIP_DECLARE_SPMV(i32, int32_t, u32, uint32_t)
LCPP_HIP_DECLARE_SPMV(u32, uint32_t, i32, int32_t)
LCPP_HIP_DECLARE_SPMV(u32, uint32_t, u32, uint32_t)
#undef LCPP_HIP_DECLARE_SPMV

/* ---------------------------------------------------------------------------------------------
 * Scan-by-key and reduce-by-key with the sum operator (decoupled look-back, single pass)
 * replaces DeviceScan<>::ExclusiveSumByKey / InclusiveSumByKey and ExclusiveScanByKey /
 * InclusiveScanByKey with a sum operator and an initial value (src/lcpp/device/device_scan.h:
 * 424-597), DeviceScan<>::GetScanByKeyTempStorageBytes<K, V> (:310-315, layout :129-142),
 * DeviceReduce<>::ReduceByKey with a sum operator (src/lcpp/device/device_reduce.h:437-487) and
 * DeviceReduce<>::GetReduceByKeyTempStorageBytes<K, V> (:207-223).
 * A run is a maximal range of consecutive items whose keys are equal; keys compare by bits under
 * `key_mask` (equal when ((a ^ b) & key_mask) == 0): all-ones is the reference's default
 * equality_op (lhs == rhs) for integer keys, other masks express bit-class equalities such as the
 * parity test of tests/device_scan_test.cpp:419-447.
 * Scan: exclusive (inclusive == 0): out[i] = init + (sum of the run's items before i), out[head] =
 * init (ExclusiveSumByKey passes init = 0); inclusive without init (use_init == 0): out[i] = sum of
 * the run's items up to i; with init: init + that sum (the reference's "prepend an initial value to
 * every segment" overloads, device_scan.h:488-519).  values_out may equal values_in.
 * Reduce: unique_out[r] = first key of run r, aggregates_out[r] = sum of run r, *num_runs_out = runs;
 * n == 0 writes 0 runs (device_reduce.h:449-458).  Integer sums wrap; n <= 2^32 - 1.  The outputs
 * need room for the run count only and must not overlap the inputs: an output whose first item lies
 * inside keys_in or values_in is rejected (-1); buffers that overlap further in are undefined.
 * Key suffixes: i32, u32, i64, u64; value suffixes i32, u32, f32, i64, u64, f64.
 * ------------------------------------------------------------------------------------------- */
size_t lcpp_hip_scan_by_key_temp_bytes(uint64_t n, size_t key_bytes, size_t value_bytes);
size_t lcpp_hip_reduce_by_key_temp_bytes(uint64_t n, size_t key_bytes, size_t value_bytes);
/* The same queries for other DeviceScan<BLOCK, 32, ITEMS> / DeviceReduce<BLOCK> policies
 * (device_scan.h:129-142,310-315; device_reduce.h:207-223).  Where a policy's tiles are so large
 * that the reference layout is smaller than the by-key kernel's tile states, the result is raised
 * to the kernel's need; for the default policies it is the reference's figure exactly. */
size_t lcpp_hip_scan_by_key_temp_bytes_policy(uint64_t n, size_t key_bytes, size_t value_bytes, uint32_t block_size,
                                              uint32_t items_per_thread);
size_t lcpp_hip_reduce_by_key_temp_bytes_policy(uint64_t n, size_t key_bytes, size_t value_bytes,
                                                uint32_t block_size);

#define LCPP_HIP_DECLARE_BY_KEY(KS, KT, VS, VT)                                                                      \
    int lcpp_hip_scan_by_key_sum_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys, const VT* values_in,     \
                                             VT* values_out, uint64_t n, int inclusive, int use_init, VT init,       \
                                             uint64_t key_mask, void* stream);                                       \
    int lcpp_hip_reduce_by_key_sum_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys_in, const VT* values_in, \
                                               KT* unique_out, VT* aggregates_out, uint32_t* num_runs_out, uint64_t n, \
                                               uint64_t key_mask, void* stream);
#define LCPP_HIP_DECLARE_BY_KEY_VALUES(KS, KT)          \
    LCPP_HIP_DECLARE_BY_KEY(KS, KT, i32, int32_t)       \
    LCPP_HIP_DECLARE_BY_KEY(KS, KT, u32, uint32_t)      \
    LCPP_HIP_DECLARE_BY_KEY(KS, KT, f32, float)         \
    LCPP_HIP_DECLARE_BY_KEY(KS, KT, i64, int64_t)       \
    LCPP_HIP_DECLARE_BY_KEY(KS, KT, u64, uint64_t)      \
    LCPP_HIP_DECLARE_BY_KEY(KS, KT, f64, double)
LCPP_HIP_DECLARE_BY_KEY_VALUES(i32, int32_t)
LCPP_HIP_DECLARE_BY_KEY_VALUES(u32, uint32_t)
LCPP_HIP_DECLARE_BY_KEY_VALUES(i64, int64_t)
LCPP_HIP_DECLARE_BY_KEY_VALUES(u64, uint64_t)
#undef LCPP_HIP_DECLARE_BY_KEY_VALUES
#undef LCPP_HIP_DECLARE_BY_KEY
/* The same entry points with MinOp / MaxOp in place of the sum (device_scan.h:424-597 and
 * device_reduce.h:437-487 take any ScanOp / ReduceOp; common/thread_operators.h:58-74): values compare
 * in their own type (signed as signed; floats like fmin / fmax, a NaN item skipped), an exclusive scan
 * without an initial value gives run heads the operator's identity (the type's max / lowest, a quiet
 * NaN for floats), and with one out[i] = op(init, the run's items before i).  Same temp queries. */
#define LCPP_HIP_DECLARE_BY_KEY_OP(NAME, KS, KT, VS, VT)                                                              \
    int lcpp_hip_scan_by_key_##NAME##_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys, const VT* values_in, \
                                                 VT* values_out, uint64_t n, int inclusive, int use_init, VT init,    \
                                                 uint64_t key_mask, void* stream);                                   \
    int lcpp_hip_reduce_by_key_##NAME##_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys_in,                \
                                                   const VT* values_in, KT* unique_out, VT* aggregates_out,          \
                                                   uint32_t* num_runs_out, uint64_t n, uint64_t key_mask,            \
                                                   void* stream);
#define LCPP_HIP_DECLARE_BY_KEY_OP_VALUES(KS, KT)                                                                      \
    LCPP_HIP_DECLARE_BY_KEY_OP(min, KS, KT, i32, int32_t) LCPP_HIP_DECLARE_BY_KEY_OP(min, KS, KT, u32, uint32_t)       \
    LCPP_HIP_DECLARE_BY_KEY_OP(min, KS, KT, f32, float) LCPP_HIP_DECLARE_BY_KEY_OP(min, KS, KT, i64, int64_t)         \
    LCPP_HIP_DECLARE_BY_KEY_OP(min, KS, KT, u64, uint64_t) LCPP_HIP_DECLARE_BY_KEY_OP(min, KS, KT, f64, double)       \
    LCPP_HIP_DECLARE_BY_KEY_OP(max, KS, KT, i32, int32_t) LCPP_HIP_DECLARE_BY_KEY_OP(max, KS, KT, u32, uint32_t)       \
    LCPP_HIP_DECLARE_BY_KEY_OP(max, KS, KT, f32, float) LCPP_HIP_DECLARE_BY_KEY_OP(max, KS, KT, i64, int64_t)         \
    LCPP_HIP_DECLARE_BY_KEY_OP(max, KS, KT, u64, uint64_t) LCPP_HIP_DECLARE_BY_KEY_OP(max, KS, KT, f64, double)
LCPP_HIP_DECLARE_BY_KEY_OP_VALUES(i32, int32_t)
LCPP_HIP_DECLARE_BY_KEY_OP_VALUES(u32, uint32_t)
LCPP_HIP_DECLARE_BY_KEY_OP_VALUES(i64, int64_t)
LCPP_HIP_DECLARE_BY_KEY_OP_VALUES(u64, uint64_t)
#undef LCPP_HIP_DECLARE_BY_KEY_OP_VALUES
#undef LCPP_HIP_DECLARE_BY_KEY_OP

/* ---------------------------------------------------------------------------------------------
 * Stream compaction: DeviceSelect, DevicePartition, DeviceRunLengthEncode.
 * Replaces DeviceSelect<>::Flagged / If / FlaggedIf / Unique / UniqueByKey (device_select.h:65-344,
 * temp query :56-63), DevicePartition<>::Flagged / If / three-way If (device_partition.h:73-209, temp
 * queries :55-71) and DeviceRunLengthEncode<>::Encode / NonTrivialRuns (device_run_length_encode.h:
 * 56-153).  Semantics as the reference: selected items keep their order and *num_selected_out
 * receives their count; partition writes the rejected items after them in reverse order
 * (out[n - 1 - j] for the j-th reject, device_partition.h:530-579); the three-way partition writes the
 * first and second categories in order and the unselected items reversed within their own output,
 * with num_selected_out[0..1] = the two category sizes (:581-663); Unique / UniqueByKey keep the
 * first item (key and value) of every run of equal items; Encode writes each run's value and length,
 * NonTrivialRuns the offset and length of every run longer than one item (CUB's conventions).
 * n == 0 writes zero counts.  Selects whose output overlaps their input or flags are the in-place
 * forms (device_select.h:106-117,160-175,201-212,226-265).
 *
 * The reference's predicates and equalities are device lambdas.  Here a predicate is two clauses
 * that must both hold (op[c] with operands a[c], b[c], given as the bits of values of the item or
 * flag type in the low bytes); flags select when != 0; adjacent keys are equal when
 * ((x ^ y) & key_mask) == 0 for integers, and by value (x == y) for floats, as lhs == rhs is.
 * Item suffixes T: i32 u32 f32 i64 u64 f64; flag suffixes F: b8 (bool / uint8) i32 u32 i64 u64.
 * ------------------------------------------------------------------------------------------- */
#define LCPP_HIP_PRED_TRUE 0     /* always                                   */
#define LCPP_HIP_PRED_LT 1       /* x <  a                                   */
#define LCPP_HIP_PRED_LE 2       /* x <= a                                   */
#define LCPP_HIP_PRED_GT 3       /* x >  a                                   */
#define LCPP_HIP_PRED_GE 4       /* x >= a                                   */
#define LCPP_HIP_PRED_EQ 5       /* x == a                                   */
#define LCPP_HIP_PRED_NE 6       /* x != a                                   */
#define LCPP_HIP_PRED_RANGE 7    /* a <= x && x < b                          */
#define LCPP_HIP_PRED_MASK_EQ 8  /* (bits(x) & bits(a)) == bits(b)           */
#define LCPP_HIP_PRED_MASK_NE 9  /* (bits(x) & bits(a)) != bits(b)           */
#define LCPP_HIP_PRED_MOD_EQ 10  /* x % a == b (integers, C remainder; a != 0) */
#define LCPP_HIP_PRED_MOD_NE 11  /* x % a != b                               */
typedef struct lcpp_hip_predicate {
    int32_t op[2];
    uint64_t a[2];
    uint64_t b[2];
} lcpp_hip_predicate;

/* DeviceSelect<BLOCK, 32, ITEMS>::GetTempStorageBytes (and DevicePartition's, the same formula):
 * 0 for n == 0, else 8 n + DeviceScan<BLOCK, 32, ITEMS>::GetTempStorageBytes<uint>(n); three-way
 * 12 n + that; DeviceRunLengthEncode: align256(4 (6 n + 1)) + that.  The *_policy forms take the
 * module's BLOCK_SIZE and ITEMS_PER_THREAD (defaults 256 and 4, runtime/core.h:17-23) and are raised
 * to the kernels' need where a policy's scan layout would be smaller. */
size_t lcpp_hip_select_temp_bytes(uint64_t n);
size_t lcpp_hip_select_temp_bytes_policy(uint64_t n, uint32_t block_size, uint32_t items_per_thread);
size_t lcpp_hip_partition_three_way_temp_bytes(uint64_t n);
size_t lcpp_hip_partition_three_way_temp_bytes_policy(uint64_t n, uint32_t block_size, uint32_t items_per_thread);
size_t lcpp_hip_run_length_encode_temp_bytes(uint64_t n);
size_t lcpp_hip_run_length_encode_temp_bytes_policy(uint64_t n, uint32_t block_size, uint32_t items_per_thread);

#define LCPP_HIP_DECLARE_SELECT_FLAGS(TS, TT, FS, FT)                                                               \
    int lcpp_hip_select_flagged_##TS##_##FS(void* temp, size_t temp_bytes, const TT* in, const FT* flags, TT* out, \
                                            uint32_t* num_selected_out, uint64_t n, void* stream);                \
    int lcpp_hip_select_flagged_if_##TS##_##FS(void* temp, size_t temp_bytes, const TT* in, const FT* flags,      \
                                               TT* out, uint32_t* num_selected_out, uint64_t n,                   \
                                               const lcpp_hip_predicate* pred, void* stream);                     \
    int lcpp_hip_partition_flagged_##TS##_##FS(void* temp, size_t temp_bytes, const TT* in, const FT* flags,      \
                                               TT* out, uint32_t* num_selected_out, uint64_t n, void* stream);
#define LCPP_HIP_DECLARE_SELECT_ITEMS(TS, TT)                                                                        \
    int lcpp_hip_select_if_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out, uint32_t* num_selected_out,  \
                                uint64_t n, const lcpp_hip_predicate* pred, void* stream);                         \
    int lcpp_hip_partition_if_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out,                           \
                                   uint32_t* num_selected_out, uint64_t n, const lcpp_hip_predicate* pred,          \
                                   void* stream);                                                                   \
    int lcpp_hip_partition_three_way_##TS(void* temp, size_t temp_bytes, const TT* in, TT* first_out,              \
                                          TT* second_out, TT* unselected_out, uint32_t* num_selected_out,           \
                                          uint64_t n, const lcpp_hip_predicate* select_first,                      \
                                          const lcpp_hip_predicate* select_second, void* stream);                  \
    int lcpp_hip_select_unique_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out,                          \
                                    uint32_t* num_selected_out, uint64_t n, uint64_t key_mask, void* stream);      \
    int lcpp_hip_run_length_encode_##TS(void* temp, size_t temp_bytes, const TT* in, TT* unique_out,               \
                                        uint32_t* counts_out, uint32_t* num_runs_out, uint64_t n, void* stream);   \
    int lcpp_hip_run_length_non_trivial_##TS(void* temp, size_t temp_bytes, const TT* in, uint32_t* offsets_out,   \
                                             uint32_t* lengths_out, uint32_t* num_runs_out, uint64_t n,             \
                                             void* stream);                                                         \
    LCPP_HIP_DECLARE_SELECT_FLAGS(TS, TT, b8, uint8_t)                                                               \
    LCPP_HIP_DECLARE_SELECT_FLAGS(TS, TT, i32, int32_t)                                                              \
    LCPP_HIP_DECLARE_SELECT_FLAGS(TS, TT, u32, uint32_t)                                                             \
    LCPP_HIP_DECLARE_SELECT_FLAGS(TS, TT, i64, int64_t)                                                              \
    LCPP_HIP_DECLARE_SELECT_FLAGS(TS, TT, u64, uint64_t)                                                             \
    LCPP_HIP_DECLARE_UNIQUE_BY_KEY(TS, TT, i32, int32_t)                                                             \
    LCPP_HIP_DECLARE_UNIQUE_BY_KEY(TS, TT, u32, uint32_t)                                                            \
    LCPP_HIP_DECLARE_UNIQUE_BY_KEY(TS, TT, f32, float)                                                               \
    LCPP_HIP_DECLARE_UNIQUE_BY_KEY(TS, TT, i64, int64_t)                                                             \
    LCPP_HIP_DECLARE_UNIQUE_BY_KEY(TS, TT, u64, uint64_t)                                                            \
    LCPP_HIP_DECLARE_UNIQUE_BY_KEY(TS, TT, f64, double)
#define LCPP_HIP_DECLARE_UNIQUE_BY_KEY(KS, KT, VS, VT)                                                               \
    int lcpp_hip_select_unique_by_key_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys_in,                \
                                                  const VT* values_in, KT* keys_out, VT* values_out,                \
                                                  uint32_t* num_selected_out, uint64_t n, uint64_t key_mask,        \
                                                  void* stream);
LCPP_HIP_DECLARE_SELECT_ITEMS(i32, int32_t)
LCPP_HIP_DECLARE_SELECT_ITEMS(u32, uint32_t)
LCPP_HIP_DECLARE_SELECT_ITEMS(f32, float)
LCPP_HIP_DECLARE_SELECT_ITEMS(i64, int64_t)
LCPP_HIP_DECLARE_SELECT_ITEMS(u64, uint64_t)
LCPP_HIP_DECLARE_SELECT_ITEMS(f64, double)
#undef LCPP_HIP_DECLARE_UNIQUE_BY_KEY
#undef LCPP_HIP_DECLARE_SELECT_ITEMS
#undef LCPP_HIP_DECLARE_SELECT_FLAGS

/* ---------------------------------------------------------------------------------------------
 * Segmented reductions and scans: DeviceSegmentReduce, DeviceSegmentedScan.
 * Replaces DeviceSegmentReduce<>::Sum / Min / Max (begin/end offsets or fixed segment_size) and
 * ArgMin / ArgMax (device_segment_reduce.h:87-420) and DeviceSegmentedScan<>::ExclusiveSegmentedSum /
 * InclusiveSegmentedSum / InclusiveSegmentedScanInit with the sum operator
 * (device_segmented_scan.h:52-224).  Segment s covers input[begin[s], end[s]); a segment with
 * begin >= end is empty and reduces to the initial value (0 for Sum, the type's max for Min, lowest for
 * Max; ArgMin / ArgMax write that value with index 1, details/segment_reduce.h:138-146).  Arg indices
 * are relative to the segment's begin, ties go to the lower index.  Scans write
 * output[out_begin[s] + k] (out_begin_offsets may be NULL: the input offsets), exclusive scans start
 * from init; in-place (output == input, same offsets) is allowed.  Integer sums wrap; float Min / Max
 * ignore NaN operands.  Temp storage: none (the Arg query returns the reference's figure).
 * Suffixes: Sum / Min / Max / scans i32 u32 f32 i64 u64 f64; ArgMin / ArgMax i32 u32 f32.
 * ------------------------------------------------------------------------------------------- */
size_t lcpp_hip_segment_reduce_temp_bytes(uint64_t n);
size_t lcpp_hip_segment_reduce_arg_temp_bytes(uint64_t n, uint64_t num_segments);
size_t lcpp_hip_segmented_scan_temp_bytes(uint64_t n, uint64_t num_segments);
#define LCPP_HIP_DECLARE_SEGMENT_REDUCE(OPS, TS, TT)                                                                 \
    int lcpp_hip_segment_reduce_##OPS##_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out,                 \
                                             uint64_t num_segments, const uint32_t* begin_offsets,                 \
                                             const uint32_t* end_offsets, void* stream);                           \
    int lcpp_hip_segment_reduce_fixed_##OPS##_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out,           \
                                                   uint64_t num_segments, uint32_t segment_size, void* stream);
#define LCPP_HIP_DECLARE_SEGMENT_ARG(OPS, TS, TT)                                                                    \
    int lcpp_hip_segment_##OPS##_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out, uint32_t* index_out,   \
                                      uint64_t num_segments, const uint32_t* begin_offsets,                        \
                                      const uint32_t* end_offsets, void* stream);                                  \
    int lcpp_hip_segment_fixed_##OPS##_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out,                  \
                                            uint32_t* index_out, uint64_t num_segments, uint32_t segment_size,     \
                                            void* stream);
#define LCPP_HIP_DECLARE_SEGMENTED(TS, TT)                                                                           \
    LCPP_HIP_DECLARE_SEGMENT_REDUCE(sum, TS, TT)                                                                     \
    LCPP_HIP_DECLARE_SEGMENT_REDUCE(min, TS, TT)                                                                     \
    LCPP_HIP_DECLARE_SEGMENT_REDUCE(max, TS, TT)                                                                     \
    int lcpp_hip_segmented_scan_sum_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out,                     \
                                         const uint32_t* begin_offsets, const uint32_t* end_offsets,               \
                                         const uint32_t* out_begin_offsets, uint64_t num_segments, int inclusive,  \
                                         int use_init, TT init, void* stream);
LCPP_HIP_DECLARE_SEGMENTED(i32, int32_t)
LCPP_HIP_DECLARE_SEGMENTED(u32, uint32_t)
LCPP_HIP_DECLARE_SEGMENTED(f32, float)
LCPP_HIP_DECLARE_SEGMENTED(i64, int64_t)
LCPP_HIP_DECLARE_SEGMENTED(u64, uint64_t)
LCPP_HIP_DECLARE_SEGMENTED(f64, double)
LCPP_HIP_DECLARE_SEGMENT_ARG(argmin, i32, int32_t)
LCPP_HIP_DECLARE_SEGMENT_ARG(argmin, u32, uint32_t)
LCPP_HIP_DECLARE_SEGMENT_ARG(argmin, f32, float)
LCPP_HIP_DECLARE_SEGMENT_ARG(argmax, i32, int32_t)
LCPP_HIP_DECLARE_SEGMENT_ARG(argmax, u32, uint32_t)
LCPP_HIP_DECLARE_SEGMENT_ARG(argmax, f32, float)
#undef LCPP_HIP_DECLARE_SEGMENTED
#undef LCPP_HIP_DECLARE_SEGMENT_ARG
#undef LCPP_HIP_DECLARE_SEGMENT_REDUCE

/* ---------------------------------------------------------------------------------------------
 * Segmented sorts: DeviceSegmentedRadixSort and DeviceSegmentedSort.
 * Replaces DeviceSegmentedRadixSort<>::SortKeys / SortPairs (+Descending; copy and DoubleBuffer
 * forms; begin_bit / end_bit, device_segmented_radix_sort.h:28-205) and DeviceSegmentedSort<>::SortKeys
 * / StableSortKeys / SortPairs / StableSortPairs (+Descending, device_segmented_sort.h:49-505) with the
 * default comparators.  Each segment [begin[s], end[s]) is sorted stably (begins ascending, segments
 * disjoint, end <= n; items outside every segment are not written).  value_order == 0: radix order of
 * the twiddled key bits [begin_bit, end_bit) (DeviceSegmentedRadixSort); value_order == 1: lhs < rhs on
 * the key values (DeviceSegmentedSort; differs only for floats: -0.0 equals +0.0).  descending flips
 * the order.  DoubleBuffer forms (*_db_*) sort from the buffer *selector picks into the one the
 * reference's selector points to after its ceil(log2 n) flips, flipping *selector the same way; a radix
 * sort of zero bits leaves them untouched.  Key suffixes u32 i32 f32 u64 i64 f64; values v32 / v64.
 * Temp (copy forms): 0 for n <= 1, else n keys (+ n values at their alignment), each rounded to 4 bytes.
 * ------------------------------------------------------------------------------------------- */
size_t lcpp_hip_segmented_sort_keys_temp_bytes(uint64_t n, size_t key_bytes);
size_t lcpp_hip_segmented_sort_pairs_temp_bytes(uint64_t n, size_t key_bytes, size_t value_bytes);
#define LCPP_HIP_DECLARE_SEGSORT_PAIRS(KS, KT, VS, VT)                                                               \
    int lcpp_hip_segmented_sort_pairs_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys_in, KT* keys_out,  \
                                                  const VT* values_in, VT* values_out, uint64_t n,                \
                                                  uint64_t num_segments, const uint32_t* begin_offsets,            \
                                                  const uint32_t* end_offsets, uint32_t begin_bit,                 \
                                                  uint32_t end_bit, int descending, int value_order, void* stream); \
    int lcpp_hip_segmented_sort_pairs_db_##KS##_##VS(KT* keys0, KT* keys1, int* key_selector, VT* values0,         \
                                                     VT* values1, int* value_selector, uint64_t n,                \
                                                     uint64_t num_segments, const uint32_t* begin_offsets,         \
                                                     const uint32_t* end_offsets, uint32_t begin_bit,              \
                                                     uint32_t end_bit, int descending, int value_order,            \
                                                     void* stream);
#define LCPP_HIP_DECLARE_SEGSORT(KS, KT)                                                                             \
    int lcpp_hip_segmented_sort_keys_##KS(void* temp, size_t temp_bytes, const KT* keys_in, KT* keys_out,          \
                                          uint64_t n, uint64_t num_segments, const uint32_t* begin_offsets,        \
                                          const uint32_t* end_offsets, uint32_t begin_bit, uint32_t end_bit,       \
                                          int descending, int value_order, void* stream);                          \
    int lcpp_hip_segmented_sort_keys_db_##KS(KT* keys0, KT* keys1, int* key_selector, uint64_t n,                  \
                                             uint64_t num_segments, const uint32_t* begin_offsets,                 \
                                             const uint32_t* end_offsets, uint32_t begin_bit, uint32_t end_bit,    \
                                             int descending, int value_order, void* stream);                       \
    LCPP_HIP_DECLARE_SEGSORT_PAIRS(KS, KT, v32, uint32_t)                                                            \
    LCPP_HIP_DECLARE_SEGSORT_PAIRS(KS, KT, v64, uint64_t)
LCPP_HIP_DECLARE_SEGSORT(u32, uint32_t)
LCPP_HIP_DECLARE_SEGSORT(i32, int32_t)
LCPP_HIP_DECLARE_SEGSORT(f32, float)
LCPP_HIP_DECLARE_SEGSORT(u64, uint64_t)
LCPP_HIP_DECLARE_SEGSORT(i64, int64_t)
LCPP_HIP_DECLARE_SEGSORT(f64, double)
#undef LCPP_HIP_DECLARE_SEGSORT
#undef LCPP_HIP_DECLARE_SEGSORT_PAIRS

/* ---------------------------------------------------------------------------------------------
 * Seeded synthetic workloads for tests and benchmarks (no reference counterpart; the reference
 * generates on the host, e.g. tests/lcpp_cub_bench.cpp:516-521,666-672,814).
 * Stream: splitmix64, r_i = mix(seed + (start + i + 1) * 0x9E3779B97F4A7C15).
 * ------------------------------------------------------------------------------------------- */
#define LCPP_HIP_GEN_U64 0            /* out[i] = r_i (uint64)                                   */
#define LCPP_HIP_GEN_U32_HI 1         /* out[i] = r_i >> 32 (uint32)                             */
#define LCPP_HIP_GEN_I32_PM1000 2     /* out[i] = (int32)(r_i % 2001) - 1000                     */
#define LCPP_HIP_GEN_U32_LT16 3       /* out[i] = r_i & 15 (uint32)                              */
#define LCPP_HIP_GEN_U64_AND3 4       /* out[i] = r_{3i} & r_{3i+1} & r_{3i+2} (uint64)          */
#define LCPP_HIP_GEN_U32_IOTA 5       /* out[i] = start + i (uint32)                             */
#define LCPP_HIP_GEN_F32_PM1 6        /* out[i] = uniform float in [-1, 1): ((r_i>>40) * 2^-23) - 1 */
int lcpp_hip_generate(int kind, void* out, uint64_t n, uint64_t seed, uint64_t start, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Introspection and test hooks (no reference counterpart): the bytes of temp storage the kernels
 * actually carve, the onesweep portion count for a given temp size, and the in-wave ranking variant
 * of the onesweep kernel (0 ballot match in every wave, 1 LDS lane-mask tables in every wave, 2 a
 * split of the waves between them, the default; all give the same ranks).
 * ------------------------------------------------------------------------------------------- */
size_t lcpp_hip_internal_scan_needed_bytes(uint64_t n, size_t elem_bytes);
size_t lcpp_hip_internal_radix_needed_bytes(uint32_t n, size_t key_bytes, size_t value_bytes, uint32_t begin_bit,
                                            uint32_t end_bit, int double_buffer);
uint32_t lcpp_hip_internal_radix_portions(uint32_t n, size_t key_bytes, size_t value_bytes, uint32_t begin_bit,
                                          uint32_t end_bit, int double_buffer, size_t temp_bytes);
int lcpp_hip_internal_radix_rank_mode(int mode);
/* 1: a single-portion sort of 4-byte keys without values, 16-byte aligned, with room in its temp storage
 * takes its first pass's tile offsets from the histogram instead of a look-back; 0 (the default): every
 * pass looks back.  Both give the same results.  Returns the previous setting. */
int lcpp_hip_internal_radix_precount(int enable);
size_t lcpp_hip_internal_by_key_needed_bytes(uint64_t n, size_t value_bytes);
size_t lcpp_hip_internal_compact_needed_bytes(uint64_t n, size_t item_bytes, int words, int staged);
/* Test hook: 1 (the default) lets selects and partitions that are not in place, whose input is 16-byte
 * aligned (and flags of at most 4 bytes aligned to a thread's row of them), run the register-resident rows
 * kernel; 0 sends every call to the staging kernel.  Both give the same results.  Returns the previous
 * setting. */
int lcpp_hip_internal_compact_rows(int enable);
/* The device words a segmented sort called now on `stream` would use, without taking them: 1 the stream's
 * slot (eager calls), 2 a slot of the call's own (calls recorded into a graph, which may replay on any
 * stream), 0 none (slots used up: the kernels then run without their early exits). */
int lcpp_hip_internal_segsort_slot_kind(void* stream);

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif

#endif /* LCPP_HIP_H_ */
