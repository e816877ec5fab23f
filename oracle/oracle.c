/*
 * CPU oracle for the LCPP device hot path — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library, and only
 * as the reference results the GPU results are compared with (or the timed CPU baseline).  The product
 * (liblcpp_hip.so) never calls it.
 *
 * The reference (LuisaCompute-ParallelPrimitive) cannot be built here: every header includes
 * LuisaCompute (src/lcpp/runtime/core.h:10-13), which is fetched from the network at configure time
 * (CMakeLists.txt:7-30) and whose CPU backend is disabled (CMakeLists.txt:24).  This file therefore
 * restates the reference's semantics from its sources and tests; each function cites what it follows.
 * How each function is pinned (golden vectors, closed forms, independent algorithms) is listed in
 * tests/test_oracle.py.
 *
 * Conventions: sizes are uint64_t; integer sums wrap modulo 2^bits (two's complement), as the
 * reference's int32/uint32 arithmetic does on the device.
 */
#include <float.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

static uint64_t load_bits_any(const void* p, uint64_t i, int bytes) {
    return bytes == 4 ? ((const uint32_t*)p)[i] : ((const uint64_t*)p)[i];
}
static void store_bits_any(void* p, uint64_t i, int bytes, uint64_t v) {
    if (bytes == 4) ((uint32_t*)p)[i] = (uint32_t)v;
    else ((uint64_t*)p)[i] = v;
}

/* ------------------------------------------------------------------------------------------------
 * Seeded streams.  splitmix64 (Steele, Lea, Flood 2014; the generator of java.util.SplittableRandom):
 * r_i = mix(seed + (i + 1) * 0x9E3779B97F4A7C15).  Known answer: seed 0 gives 0xE220A8397B1DCDAF,
 * 0x6E789E6AA1B965F4, 0x06C45D188009454F (tests/test_oracle.py).
 * ---------------------------------------------------------------------------------------------- */
uint64_t oracle_splitmix64_at(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Same kinds and mappings as lcpp_hip_generate (include/lcpp_hip.h). */
int oracle_generate(int kind, void* out, uint64_t n, uint64_t seed, uint64_t start) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t g = start + i;
        switch (kind) {
            case 0: ((uint64_t*)out)[i] = oracle_splitmix64_at(seed, g); break;
            case 1: ((uint32_t*)out)[i] = (uint32_t)(oracle_splitmix64_at(seed, g) >> 32); break;
            case 2: ((int32_t*)out)[i] = (int32_t)(oracle_splitmix64_at(seed, g) % 2001ull) - 1000; break;
            case 3: ((uint32_t*)out)[i] = (uint32_t)(oracle_splitmix64_at(seed, g) & 15ull); break;
            case 4:
                ((uint64_t*)out)[i] = oracle_splitmix64_at(seed, 3 * g) & oracle_splitmix64_at(seed, 3 * g + 1) &
                                      oracle_splitmix64_at(seed, 3 * g + 2);
                break;
            case 5: ((uint32_t*)out)[i] = (uint32_t)g; break;
            case 6:
                ((float*)out)[i] = (float)(uint32_t)(oracle_splitmix64_at(seed, g) >> 40) * (1.0f / 8388608.0f) - 1.0f;
                break;
            default: return -1;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------
 * DeviceReduce::Sum (src/lcpp/device/device_reduce.h:280-288; n == 0 -> init = 0, :238-243).
 * Integer sum is associative modulo 2^bits, so any order gives the device result:
 * (int32) sum_int64.  Also reports the exact int64 sum (for the "int64-safe" check).
 * ---------------------------------------------------------------------------------------------- */
int32_t oracle_reduce_sum_i32(const int32_t* in, uint64_t n, int64_t* exact) {
    int64_t s = 0;
    for (uint64_t i = 0; i < n; ++i) s += in[i];
    if (exact) *exact = s;
    return (int32_t)(uint32_t)(uint64_t)s;
}
uint32_t oracle_reduce_sum_u32(const uint32_t* in, uint64_t n) {
    uint32_t s = 0;
    for (uint64_t i = 0; i < n; ++i) s += in[i];
    return s;
}
uint64_t oracle_reduce_sum_u64(const uint64_t* in, uint64_t n) {
    uint64_t s = 0;
    for (uint64_t i = 0; i < n; ++i) s += in[i];
    return s;
}
/* Floating-point: sum in long double plus the sum of magnitudes (for a condition-aware tolerance). */
double oracle_reduce_sum_f32(const float* in, uint64_t n, double* abs_sum) {
    long double s = 0, a = 0;
    for (uint64_t i = 0; i < n; ++i) { s += in[i]; a += fabsl((long double)in[i]); }
    if (abs_sum) *abs_sum = (double)a;
    return (double)s;
}
double oracle_reduce_sum_f64(const double* in, uint64_t n, double* abs_sum) {
    long double s = 0, a = 0;
    for (uint64_t i = 0; i < n; ++i) { s += in[i]; a += fabsl((long double)in[i]); }
    if (abs_sum) *abs_sum = (double)a;
    return (double)s;
}

/* ------------------------------------------------------------------------------------------------
 * DeviceScan::ExclusiveSum / InclusiveSum / InclusiveScanInit with a sum operator
 * (src/lcpp/device/device_scan.h:321-422; tests compare with std::exclusive_scan,
 * tests/device_scan_test.cpp:117-118).  Exclusive: out[i] = init + sum(in[0..i)); inclusive:
 * out[i] = init + sum(in[0..i]).  32-bit words wrap (signed and unsigned share the bits).
 * ---------------------------------------------------------------------------------------------- */
void oracle_scan_sum_u32(const uint32_t* in, uint32_t* out, uint64_t n, int inclusive, uint32_t init) {
    uint32_t run = init;
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t x = in[i];
        if (inclusive) { run += x; out[i] = run; }
        else { out[i] = run; run += x; }
    }
}
/* The same over 64-bit words (int64 and uint64 share the bits; sums wrap modulo 2^64). */
void oracle_scan_sum_u64(const uint64_t* in, uint64_t* out, uint64_t n, int inclusive, uint64_t init) {
    uint64_t run = init;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t x = in[i];
        if (inclusive) { run += x; out[i] = run; }
        else { out[i] = run; run += x; }
    }
}
/* Double-precision scan accumulated in long double (reference value for a tolerance check), plus
 * running |x| sums. */
void oracle_scan_sum_f64(const double* in, long double* out, long double* abs_out, uint64_t n, int inclusive,
                         double init) {
    long double run = init, arun = fabsl((long double)init);
    for (uint64_t i = 0; i < n; ++i) {
        const long double x = in[i];
        if (inclusive) { run += x; arun += fabsl(x); out[i] = run; abs_out[i] = arun; }
        else { out[i] = run; abs_out[i] = arun; run += x; arun += fabsl(x); }
    }
}
/* Min / max scan and reduce by key (device_scan.h:424-597, device_reduce.h:437-487 with MinOp / MaxOp):
 * item i starts a run when i == 0 or ((key[i] ^ key[i-1]) & mask) != 0 (4- or 8-byte keys).  At each
 * run start run = start (init when use_init, else the identity: the type's max / lowest, NaN for
 * floats); exclusive: out[i] = run, run = op(run, x); inclusive: run = op(run, x), out[i] = run, with
 * op(run, x) = x when x is strictly smaller (larger) or run is a NaN.  Reduce: per run, the fold of its
 * items from the identity; returns the run count. */
static uint64_t by_key_load(const void* keys, int kb, uint64_t i) {
    return kb == 4 ? ((const uint32_t*)keys)[i] : ((const uint64_t*)keys)[i];
}
#define ORACLE_BY_KEY_MINMAX(NAME, T, IDMIN, IDMAX)                                                          \
    static T by_key_op_##NAME(T run, T x, int is_max) {                                                      \
        return ((is_max ? x > run : x < run) || run != run) ? x : run;                                       \
    }                                                                                                        \
    void oracle_scan_by_key_minmax_##NAME(const void* keys, int kb, const T* in, T* out, uint64_t n,         \
                                          int inclusive, int use_init, T init, uint64_t mask, int is_max) {  \
        const T start = use_init ? init : (is_max ? IDMAX : IDMIN);                                          \
        T run = start;                                                                                       \
        for (uint64_t i = 0; i < n; ++i) {                                                                   \
            if (i == 0 || ((by_key_load(keys, kb, i) ^ by_key_load(keys, kb, i - 1)) & mask) != 0) run = start; \
            if (!inclusive) out[i] = run;                                                                    \
            run = by_key_op_##NAME(run, in[i], is_max);                                                      \
            if (inclusive) out[i] = run;                                                                     \
        }                                                                                                    \
    }                                                                                                        \
    uint64_t oracle_reduce_by_key_minmax_##NAME(const void* keys, int kb, const T* in, void* unique, T* agg,  \
                                                uint64_t n, uint64_t mask, int is_max) {                     \
        uint64_t runs = 0;                                                                                   \
        for (uint64_t i = 0; i < n; ++i) {                                                                   \
            if (i == 0 || ((by_key_load(keys, kb, i) ^ by_key_load(keys, kb, i - 1)) & mask) != 0) {         \
                if (kb == 4) ((uint32_t*)unique)[runs] = ((const uint32_t*)keys)[i];                         \
                else ((uint64_t*)unique)[runs] = ((const uint64_t*)keys)[i];                                 \
                agg[runs++] = (is_max ? IDMAX : IDMIN);                                                      \
            }                                                                                                \
            agg[runs - 1] = by_key_op_##NAME(agg[runs - 1], in[i], is_max);                                  \
        }                                                                                                    \
        return runs;                                                                                         \
    }
ORACLE_BY_KEY_MINMAX(i32, int32_t, INT32_MAX, INT32_MIN)
ORACLE_BY_KEY_MINMAX(u32, uint32_t, UINT32_MAX, 0u)
ORACLE_BY_KEY_MINMAX(f32, float, NAN, NAN)
ORACLE_BY_KEY_MINMAX(i64, int64_t, INT64_MAX, INT64_MIN)
ORACLE_BY_KEY_MINMAX(u64, uint64_t, UINT64_MAX, 0ull)
ORACLE_BY_KEY_MINMAX(f64, double, NAN, NAN)
#undef ORACLE_BY_KEY_MINMAX

/* DeviceReduce<>::Min / Max (device_reduce.h:291-309): run = the type's max (min) / lowest (max), then
 * run = op(run, in[i]) left to right with the min / max scans' operator (a NaN item is skipped).
 * ArgMin / ArgMax (device_reduce.h:311-436 with ArgMinOp / ArgMaxOp, common/thread_operators.h:10-47):
 * best = (that value, index 0xFFFFFFFF); item i replaces it when it is strictly smaller (larger), or
 * equal at a lower index; NaN items never replace it.  n == 0: the initial value and index 1. */
#define ORACLE_REDUCE_EXT(NAME, T, TMAX, TLOW)                                                          \
    T oracle_reduce_min_##NAME(const T* in, uint64_t n) {                                               \
        T run = TMAX;                                                                                   \
        for (uint64_t i = 0; i < n; ++i) if (in[i] < run || run != run) run = in[i];                    \
        return run;                                                                                     \
    }                                                                                                   \
    T oracle_reduce_max_##NAME(const T* in, uint64_t n) {                                               \
        T run = TLOW;                                                                                   \
        for (uint64_t i = 0; i < n; ++i) if (in[i] > run || run != run) run = in[i];                    \
        return run;                                                                                     \
    }                                                                                                   \
    void oracle_reduce_arg_##NAME(const T* in, uint64_t n, int is_max, T* value, uint32_t* index) {     \
        T best = is_max ? TLOW : TMAX;                                                                  \
        uint32_t at = 0xFFFFFFFFu;                                                                      \
        for (uint64_t i = 0; i < n; ++i) {                                                              \
            const T x = in[i];                                                                          \
            if (x != x) continue;                                                                       \
            if ((is_max ? x > best : x < best) || (x == best && (uint32_t)i < at)) {                    \
                best = x;                                                                               \
                at = (uint32_t)i;                                                                       \
            }                                                                                           \
        }                                                                                               \
        *value = best;                                                                                  \
        *index = n == 0 ? 1u : at;                                                                      \
    }
ORACLE_REDUCE_EXT(i32, int32_t, INT32_MAX, INT32_MIN)
ORACLE_REDUCE_EXT(u32, uint32_t, UINT32_MAX, 0u)
ORACLE_REDUCE_EXT(f32, float, FLT_MAX, -FLT_MAX)
ORACLE_REDUCE_EXT(i64, int64_t, INT64_MAX, INT64_MIN)
ORACLE_REDUCE_EXT(u64, uint64_t, UINT64_MAX, 0ull)
ORACLE_REDUCE_EXT(f64, double, DBL_MAX, -DBL_MAX)
#undef ORACLE_REDUCE_EXT

/* Min / max scans (DeviceScan<>::ExclusiveScan / InclusiveScan with MinOp / MaxOp, device_scan.h:321-368,
 * common/thread_operators.h:58-74): run = init; exclusive: out[i] = run, run = op(run, in[i]);
 * inclusive: run = op(run, in[i]), out[i] = run.  op(run, x) keeps run unless x is strictly smaller
 * (larger) or run is a NaN; so a NaN operand yields the other one, as fmin / fmax do, and of -0.0 and
 * +0.0 the older is kept. */
#define ORACLE_SCAN_MINMAX(NAME, T)                                                                      \
    void oracle_scan_min_##NAME(const T* in, T* out, uint64_t n, int inclusive, T init) {              \
        T run = init;                                                                                  \
        for (uint64_t i = 0; i < n; ++i) {                                                             \
            const T x = in[i];                                                                         \
            if (!inclusive) out[i] = run;                                                              \
            if (x < run || run != run) run = x;                                                        \
            if (inclusive) out[i] = run;                                                               \
        }                                                                                              \
    }                                                                                                  \
    void oracle_scan_max_##NAME(const T* in, T* out, uint64_t n, int inclusive, T init) {              \
        T run = init;                                                                                  \
        for (uint64_t i = 0; i < n; ++i) {                                                             \
            const T x = in[i];                                                                         \
            if (!inclusive) out[i] = run;                                                              \
            if (x > run || run != run) run = x;                                                        \
            if (inclusive) out[i] = run;                                                               \
        }                                                                                              \
    }
ORACLE_SCAN_MINMAX(i32, int32_t)
ORACLE_SCAN_MINMAX(u32, uint32_t)
ORACLE_SCAN_MINMAX(f32, float)
ORACLE_SCAN_MINMAX(i64, int64_t)
ORACLE_SCAN_MINMAX(u64, uint64_t)
ORACLE_SCAN_MINMAX(f64, double)
#undef ORACLE_SCAN_MINMAX

/* DeviceReduce::Reduce(op, init) / TransformReduce(op, transform, init) (device_reduce.h:229-252,491-515;
 * the initial value enters last, on the left: reduce_op(init, aggregate), device/details/reduce.h:227-237).
 * y_i = transform(in[i]) in the item type: 0 identity, 1 scale * y + shift, 2 y * y, 3 |y| (integers
 * wrap modulo 2^bits; floats round after every operation, no fused multiply-add).  op 0 sum, 1 min,
 * 2 max (the min / max scans' operator: a NaN operand yields the other one, ties keep the left one).
 * Returns op(init, fold of the y_i from the op's identity) in the item type; for float sums the value is
 * the long-double sum rounded to T, *exact gets it in double and *abs_sum the sum of |init| and |y_i|.
 * n == 0 gives init. */
#define ORACLE_XFORM_INT(NAME, T, UT, SIGNED)                                                              \
    static T xform_##NAME(T x, int transform, T scale, T shift) {                                         \
        if (transform == 1) return (T)(UT)((UT)x * (UT)scale + (UT)shift);                                \
        if (transform == 2) return (T)(UT)((UT)x * (UT)x);                                                \
        if (transform == 3 && SIGNED && ((UT)x >> (8 * sizeof(T) - 1)) != 0) return (T)(UT)((UT)0 - (UT)x); \
        return x;                                                                                         \
    }
#define ORACLE_XFORM_FLOAT(NAME, T, FABS)                                                                  \
    static T xform_##NAME(T x, int transform, T scale, T shift) {                                         \
        if (transform == 1) { const T p = x * scale; return p + shift; }                                   \
        if (transform == 2) return x * x;                                                                 \
        if (transform == 3) return FABS(x);                                                               \
        return x;                                                                                         \
    }
ORACLE_XFORM_INT(i32, int32_t, uint32_t, 1)
ORACLE_XFORM_INT(u32, uint32_t, uint32_t, 0)
ORACLE_XFORM_FLOAT(f32, float, fabsf)
ORACLE_XFORM_INT(i64, int64_t, uint64_t, 1)
ORACLE_XFORM_INT(u64, uint64_t, uint64_t, 0)
ORACLE_XFORM_FLOAT(f64, double, fabs)
#undef ORACLE_XFORM_INT
#undef ORACLE_XFORM_FLOAT
#define ORACLE_TRANSFORM_REDUCE(NAME, T, UT, IS_FLOAT, TMAX, TLOW)                                         \
    static T fold_##NAME(T run, T x, int op) {                                                            \
        if (op == 1) return (x < run || run != run) ? x : run;                                            \
        if (op == 2) return (x > run || run != run) ? x : run;                                            \
        return IS_FLOAT ? run + x : (T)(UT)((UT)run + (UT)x);                                             \
    }                                                                                                     \
    T oracle_transform_reduce_##NAME(const T* in, uint64_t n, int op, int transform, T scale, T shift,     \
                                     T init, double* exact, double* abs_sum) {                            \
        if (op == 0 && IS_FLOAT) {                                                                        \
            long double s = init, a = fabsl((long double)init);                                           \
            for (uint64_t i = 0; i < n; ++i) {                                                            \
                const T y = xform_##NAME(in[i], transform, scale, shift);                                 \
                s += y;                                                                                   \
                a += fabsl((long double)y);                                                               \
            }                                                                                             \
            if (exact) *exact = (double)s;                                                                \
            if (abs_sum) *abs_sum = (double)a;                                                            \
            return (T)s;                                                                                  \
        }                                                                                                 \
        T run = op == 1 ? (IS_FLOAT ? (T)NAN : TMAX) : op == 2 ? (IS_FLOAT ? (T)NAN : TLOW) : (T)0;        \
        for (uint64_t i = 0; i < n; ++i) run = fold_##NAME(run, xform_##NAME(in[i], transform, scale, shift), op); \
        const T r = fold_##NAME(init, run, op); /* init is the left operand */                            \
        if (exact) *exact = (double)r;                                                                    \
        if (abs_sum) *abs_sum = 0;                                                                        \
        return r;                                                                                         \
    }
ORACLE_TRANSFORM_REDUCE(i32, int32_t, uint32_t, 0, INT32_MAX, INT32_MIN)
ORACLE_TRANSFORM_REDUCE(u32, uint32_t, uint32_t, 0, UINT32_MAX, 0u)
ORACLE_TRANSFORM_REDUCE(f32, float, uint32_t, 1, FLT_MAX, -FLT_MAX)
ORACLE_TRANSFORM_REDUCE(i64, int64_t, uint64_t, 0, INT64_MAX, INT64_MIN)
ORACLE_TRANSFORM_REDUCE(u64, uint64_t, uint64_t, 0, UINT64_MAX, 0ull)
ORACLE_TRANSFORM_REDUCE(f64, double, uint64_t, 1, DBL_MAX, -DBL_MAX)
#undef ORACLE_TRANSFORM_REDUCE

/* Scan with the left projection op(lhs, rhs) = lhs (tests/device_scan_test.cpp:129-155,
 * tests/scan_optimization_regression_test.cpp:195-205), folded literally left to right over the bits of
 * 4- or 8-byte items: with init, run = init and every output is op(run, ...) = init; without init an
 * inclusive scan starts from in[0].  Exclusive without init has no value (the operator has no identity)
 * and returns -1. */
int oracle_scan_left(const void* in, void* out, uint64_t n, int item_bytes, int inclusive, int use_init, uint64_t init) {
    if (!inclusive && !use_init) return -1;
    uint64_t run = init;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t x = load_bits_any(in, i, item_bytes);
        if (!inclusive) store_bits_any(out, i, item_bytes, run);
        run = (i == 0 && !use_init) ? x : run; /* op(run, x) = run */
        if (inclusive) store_bits_any(out, i, item_bytes, run);
    }
    return 0;
}

/* Floating-point scan in double (reference value for a tolerance check), plus running |x| sums. */
void oracle_scan_sum_f32(const float* in, double* out, double* abs_out, uint64_t n, int inclusive, float init) {
    double run = init, arun = fabs((double)init);
    for (uint64_t i = 0; i < n; ++i) {
        const double x = in[i];
        if (inclusive) { run += x; arun += fabs(x); out[i] = run; abs_out[i] = arun; }
        else { out[i] = run; abs_out[i] = arun; run += x; arun += fabs(x); }
    }
}

/* ------------------------------------------------------------------------------------------------
 * DeviceRadixSort: stable LSD radix sort with 8-bit digits, restated from
 * onesweep_radix_sort (src/lcpp/device/device_radix_sort.h:1380-1472: passes from begin_bit in steps
 * of 8, num_bit = min(end_bit - current_bit, 8)), the key twiddles (common/util_type.h:97-175;
 * descending inverts, agent/radix_rank_sort_operations.h:123-155) and ShiftDigitExtractor with the
 * float -0.0 -> +0.0 digit rule (radix_rank_sort_operations.h:18-62).  Keys keep their original bits.
 * key_kind: 0 unsigned, 1 signed, 2 floating point.  key_bytes / value_bytes: 4 or 8 (value_bytes 0:
 * keys only).  Each pass is a counting sort on one digit (stable by construction).
 * ---------------------------------------------------------------------------------------------- */
static uint64_t load_bits(const void* p, uint64_t i, int bytes) {
    return bytes == 4 ? ((const uint32_t*)p)[i] : ((const uint64_t*)p)[i];
}
static void store_bits(void* p, uint64_t i, int bytes, uint64_t v) {
    if (bytes == 4) ((uint32_t*)p)[i] = (uint32_t)v;
    else ((uint64_t*)p)[i] = v;
}

uint64_t oracle_twiddle_in(uint64_t key, int key_bytes, int key_kind, int descending) {
    const uint64_t all = key_bytes == 4 ? 0xFFFFFFFFull : ~0ull;
    const uint64_t high = 1ull << (key_bytes * 8 - 1);
    key &= all;
    if (key_kind == 1) key ^= high;
    if (key_kind == 2) key ^= (key & high) ? all : high;
    if (descending) key = ~key & all;
    return key;
}

uint32_t oracle_radix_digit(uint64_t key, int key_bytes, int key_kind, int descending, uint32_t shift, uint32_t bits) {
    uint64_t o = oracle_twiddle_in(key, key_bytes, key_kind, descending);
    if (key_kind == 2) {
        const uint64_t all = key_bytes == 4 ? 0xFFFFFFFFull : ~0ull;
        const uint64_t high = 1ull << (key_bytes * 8 - 1);
        if (o == (all & ~high)) o = high; /* ordered image of -0.0 -> that of +0.0 */
    }
    return (uint32_t)(o >> shift) & ((1u << bits) - 1u);
}

int oracle_radix_sort(const void* keys_in, void* keys_out, const void* values_in, void* values_out, uint64_t n,
                      int key_bytes, int key_kind, int value_bytes, uint32_t begin_bit, uint32_t end_bit,
                      int descending) {
    if ((key_bytes != 4 && key_bytes != 8) || (value_bytes != 0 && value_bytes != 4 && value_bytes != 8)) return -1;
    if (begin_bit > end_bit || end_bit > (uint32_t)key_bytes * 8) return -1;
    if (n == 0) return 0;
    void* ka = malloc(n * key_bytes);
    void* kb = malloc(n * key_bytes);
    void* va = value_bytes ? malloc(n * value_bytes) : NULL;
    void* vb = value_bytes ? malloc(n * value_bytes) : NULL;
    if (!ka || !kb || (value_bytes && (!va || !vb))) { free(ka); free(kb); free(va); free(vb); return -2; }
    memcpy(ka, keys_in, n * key_bytes);
    if (value_bytes) memcpy(va, values_in, n * value_bytes);
    for (uint32_t cur = begin_bit; cur < end_bit; cur += 8) {
        const uint32_t bits = end_bit - cur < 8 ? end_bit - cur : 8;
        uint64_t count[257];
        memset(count, 0, sizeof(count));
        for (uint64_t i = 0; i < n; ++i)
            count[oracle_radix_digit(load_bits(ka, i, key_bytes), key_bytes, key_kind, descending, cur, bits) + 1]++;
        for (int d = 0; d < 256; ++d) count[d + 1] += count[d];
        for (uint64_t i = 0; i < n; ++i) {
            const uint64_t k = load_bits(ka, i, key_bytes);
            const uint64_t pos = count[oracle_radix_digit(k, key_bytes, key_kind, descending, cur, bits)]++;
            store_bits(kb, pos, key_bytes, k);
            if (value_bytes) store_bits(vb, pos, value_bytes, load_bits(va, i, value_bytes));
        }
        void* t = ka; ka = kb; kb = t;
        t = va; va = vb; vb = t;
    }
    memcpy(keys_out, ka, n * key_bytes);
    if (value_bytes) memcpy(values_out, va, n * value_bytes);
    free(ka); free(kb); free(va); free(vb);
    return 0;
}

/* ------------------------------------------------------------------------------------------------
 * DeviceSpmv::CsrMV (src/lcpp/device/device_spmv.h:48-130): rows whose offsets decrease or pass nnz
 * give 0; columns >= cols are skipped; nnz == 0 gives zeros.
 *  - f64 reference (long double accumulation) plus sum |a*x| per row (condition-aware tolerance),
 *    for float/double values;
 *  - exact wrap-around sums for 32-bit integer values (signed and unsigned share the bits).
 * index_bytes 4 (int32 or uint32; negative int32 reads as a large unsigned column, as the reference's
 * cast<uint> does).
 * ---------------------------------------------------------------------------------------------- */
void oracle_spmv_csr_fp(const void* values, int value_bytes, const uint32_t* row_offsets, const uint32_t* cols_idx,
                        const void* x, double* y, double* abs_y, uint64_t rows, uint64_t cols, uint64_t nnz) {
    for (uint64_t r = 0; r < rows; ++r) {
        long double s = 0, a = 0;
        const uint32_t b = row_offsets[r], e = row_offsets[r + 1];
        if (nnz != 0 && b <= e && e <= nnz) {
            for (uint32_t i = b; i < e; ++i) {
                const uint32_t c = cols_idx[i];
                if (c >= cols) continue;
                const long double v = value_bytes == 4 ? ((const float*)values)[i] : ((const double*)values)[i];
                const long double xv = value_bytes == 4 ? ((const float*)x)[c] : ((const double*)x)[c];
                s += v * xv;
                a += fabsl(v * xv);
            }
        }
        y[r] = (double)s;
        if (abs_y) abs_y[r] = (double)a;
    }
}

void oracle_spmv_csr_u32(const uint32_t* values, const uint32_t* row_offsets, const uint32_t* cols_idx,
                         const uint32_t* x, uint32_t* y, uint64_t rows, uint64_t cols, uint64_t nnz) {
    for (uint64_t r = 0; r < rows; ++r) {
        uint32_t s = 0;
        const uint32_t b = row_offsets[r], e = row_offsets[r + 1];
        if (nnz != 0 && b <= e && e <= nnz) {
            for (uint32_t i = b; i < e; ++i) {
                const uint32_t c = cols_idx[i];
                if (c < cols) s += values[i] * x[c];
            }
        }
        y[r] = s;
    }
}

/* ------------------------------------------------------------------------------------------------
 * Scan-by-key and reduce-by-key with the sum operator.  Follows DeviceScan<>::ExclusiveScanByKey /
 * InclusiveScanByKey (src/lcpp/device/device_scan.h:424-519; ExclusiveSumByKey passes init 0,
 * :520-558) and DeviceReduce<>::ReduceByKey (src/lcpp/device/device_reduce.h:437-487): a run starts at
 * item 0 and wherever an item's key differs from the previous item's, compared bitwise under
 * key_mask (all-ones = the default lhs == rhs for integer keys).
 *   exclusive: out[i] = init + (sum of the run's items before i); a head gets init;
 *   inclusive: out[i] = sum of the run's items up to i, plus init when use_init;
 *   reduce: unique[r] = first key of run r, aggregates[r] = sum of run r; returns the run count.
 * Integer values (value_bytes 4 or 8) sum exactly modulo 2^bits; float values (4 = float,
 * 8 = double) sum in long double, with the matching sums of |items| for condition-aware tolerances.
 * ---------------------------------------------------------------------------------------------- */
static int by_key_head(const void* keys, int key_bytes, uint64_t i, uint64_t key_mask) {
    if (i == 0) return 1;
    return ((load_bits(keys, i, key_bytes) ^ load_bits(keys, i - 1, key_bytes)) & key_mask) != 0;
}

static long double fp_at(const void* values, int value_bytes, uint64_t i) {
    return value_bytes == 4 ? (long double)((const float*)values)[i] : (long double)((const double*)values)[i];
}

void oracle_scan_by_key_int(const void* keys, int key_bytes, const void* values, int value_bytes, void* out,
                            uint64_t n, int inclusive, int use_init, uint64_t init, uint64_t key_mask) {
    const uint64_t vmask = value_bytes == 4 ? 0xFFFFFFFFull : ~0ull;
    uint64_t run = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t v = load_bits(values, i, value_bytes);
        const int head = by_key_head(keys, key_bytes, i, key_mask);
        uint64_t o = 0;
        if (!inclusive) o = head ? init : init + run;
        run = head ? v : run + v;
        if (inclusive) o = use_init ? init + run : run;
        store_bits(out, i, value_bytes, o & vmask);
    }
}

void oracle_scan_by_key_fp(const void* keys, int key_bytes, const void* values, int value_bytes, double* out,
                           double* abs_out, uint64_t n, int inclusive, int use_init, double init, uint64_t key_mask) {
    long double run = 0, arun = 0;
    const long double ai = fabsl((long double)init);
    for (uint64_t i = 0; i < n; ++i) {
        const long double v = fp_at(values, value_bytes, i);
        const int head = by_key_head(keys, key_bytes, i, key_mask);
        if (!inclusive) {
            out[i] = head ? init : (double)((long double)init + run);
            abs_out[i] = head ? (double)ai : (double)(ai + arun);
        }
        run = head ? v : run + v;
        arun = head ? fabsl(v) : arun + fabsl(v);
        if (inclusive) {
            out[i] = use_init ? (double)((long double)init + run) : (double)run;
            abs_out[i] = use_init ? (double)(ai + arun) : (double)arun;
        }
    }
}

uint64_t oracle_reduce_by_key_int(const void* keys, int key_bytes, const void* values, int value_bytes,
                                  void* unique_out, void* aggregates_out, uint64_t n, uint64_t key_mask) {
    const uint64_t vmask = value_bytes == 4 ? 0xFFFFFFFFull : ~0ull;
    uint64_t runs = 0, s = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t v = load_bits(values, i, value_bytes);
        if (by_key_head(keys, key_bytes, i, key_mask)) {
            if (runs > 0) store_bits(aggregates_out, runs - 1, value_bytes, s & vmask);
            store_bits(unique_out, runs, key_bytes, load_bits(keys, i, key_bytes));
            ++runs;
            s = v;
        } else {
            s += v;
        }
    }
    if (runs > 0) store_bits(aggregates_out, runs - 1, value_bytes, s & vmask);
    return runs;
}

uint64_t oracle_reduce_by_key_fp(const void* keys, int key_bytes, const void* values, int value_bytes,
                                 void* unique_out, double* aggregates_out, double* abs_out, uint64_t n,
                                 uint64_t key_mask) {
    uint64_t runs = 0;
    long double s = 0, a = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const long double v = fp_at(values, value_bytes, i);
        if (by_key_head(keys, key_bytes, i, key_mask)) {
            if (runs > 0) {
                aggregates_out[runs - 1] = (double)s;
                abs_out[runs - 1] = (double)a;
            }
            store_bits(unique_out, runs, key_bytes, load_bits(keys, i, key_bytes));
            ++runs;
            s = v;
            a = fabsl(v);
        } else {
            s += v;
            a += fabsl(v);
        }
    }
    if (runs > 0) {
        aggregates_out[runs - 1] = (double)s;
        abs_out[runs - 1] = (double)a;
    }
    return runs;
}

/* ------------------------------------------------------------------------------------------------
 * Stream compaction.  Follows DeviceSelect<> (src/lcpp/device/device_select.h:65-344: an item is
 * kept when its flag != 0 or the predicate holds, kept items keep their order, the count is written
 * once), DevicePartition<> (src/lcpp/device/device_partition.h:530-579: kept items in order at the
 * front, the j-th rejected item at out[n - 1 - j]; three-way :581-663: first category, then second
 * (not first), in order; the j-th unselected item at unselected[u - 1 - j] for u unselected items)
 * and DeviceRunLengthEncode<> (src/lcpp/device/device_run_length_encode.h:71-153: the value and
 * length of every run; offset and length of every run longer than one item).  A run starts at item
 * 0 and wherever an item differs from the previous one: integers compare bitwise under key_mask,
 * floats by value (lhs == rhs: -0.0 equals +0.0, NaN equals nothing).
 * Predicates: two clauses that must both hold; see oracle_predicate below.
 * Item types: 0 int32, 1 uint32, 2 float, 3 int64, 4 uint64, 5 double, 6 uint8.
 * ---------------------------------------------------------------------------------------------- */
static int type_bytes(int type) { return type == 6 ? 1 : (type <= 2 ? 4 : 8); }

static int item_equal(int type, const void* p, uint64_t i, uint64_t j, uint64_t key_mask) {
    if (type == 2) return ((const float*)p)[i] == ((const float*)p)[j];
    if (type == 5) return ((const double*)p)[i] == ((const double*)p)[j];
    const int b = type_bytes(type);
    return ((load_bits(p, i, b) ^ load_bits(p, j, b)) & key_mask) == 0;
}

void oracle_run_heads(int type, const void* in, uint64_t n, uint64_t key_mask, uint8_t* heads) {
    for (uint64_t i = 0; i < n; ++i) heads[i] = (uint8_t)(i == 0 || !item_equal(type, in, i, i - 1, key_mask));
}

/* Clause ops (same numbering as the C-ABI): 0 true, 1 <, 2 <=, 3 >, 4 >=, 5 ==, 6 !=,
 * 7 a <= x < b, 8 (x & a) == b, 9 (x & a) != b, 10 x % a == b, 11 x % a != b (C remainder). */
static int clause_holds(int type, const void* p, uint64_t i, int op, uint64_t a_bits, uint64_t b_bits) {
    if (op == 0) return 1;
    const int bytes = type_bytes(type);
    const uint64_t mask = bytes == 8 ? ~0ull : ((1ull << (8 * bytes)) - 1);
    if (op == 8 || op == 9) {
        const int eq = (load_bits(p, i, bytes) & a_bits & mask) == (b_bits & mask);
        return op == 8 ? eq : !eq;
    }
    if (type == 2 || type == 5) {
        double x, a, b;
        if (type == 2) {
            float fa, fb;
            const uint32_t ua = (uint32_t)a_bits, ub = (uint32_t)b_bits;
            memcpy(&fa, &ua, 4);
            memcpy(&fb, &ub, 4);
            x = ((const float*)p)[i];
            a = fa;
            b = fb;
        } else {
            memcpy(&a, &a_bits, 8);
            memcpy(&b, &b_bits, 8);
            x = ((const double*)p)[i];
        }
        switch (op) {
            case 1: return x < a;
            case 2: return x <= a;
            case 3: return x > a;
            case 4: return x >= a;
            case 5: return x == a;
            case 6: return x != a;
            case 7: return a <= x && x < b;
            default: return 0;
        }
    }
    const int is_signed = type == 0 || type == 3;
    if (is_signed) {
        const int64_t x = bytes == 4 ? (int64_t)(int32_t)load_bits(p, i, 4) : (int64_t)load_bits(p, i, 8);
        const int64_t a = bytes == 4 ? (int64_t)(int32_t)(uint32_t)a_bits : (int64_t)a_bits;
        const int64_t b = bytes == 4 ? (int64_t)(int32_t)(uint32_t)b_bits : (int64_t)b_bits;
        switch (op) {
            case 1: return x < a;
            case 2: return x <= a;
            case 3: return x > a;
            case 4: return x >= a;
            case 5: return x == a;
            case 6: return x != a;
            case 7: return a <= x && x < b;
            case 10: return a != 0 && x % a == b;
            case 11: return a != 0 && x % a != b;
            default: return 0;
        }
    }
    const uint64_t x = load_bits(p, i, bytes);
    const uint64_t a = a_bits & mask, b = b_bits & mask;
    switch (op) {
        case 1: return x < a;
        case 2: return x <= a;
        case 3: return x > a;
        case 4: return x >= a;
        case 5: return x == a;
        case 6: return x != a;
        case 7: return a <= x && x < b;
        case 10: return a != 0 && x % a == b;
        case 11: return a != 0 && x % a != b;
        default: return 0;
    }
}

/* sel[i] = clause 0 and clause 1 hold for item i. */
void oracle_predicate(int type, const void* in, uint64_t n, const int32_t* ops, const uint64_t* a, const uint64_t* b,
                      uint8_t* sel) {
    for (uint64_t i = 0; i < n; ++i)
        sel[i] = (uint8_t)(clause_holds(type, in, i, ops[0], a[0], b[0]) && clause_holds(type, in, i, ops[1], a[1], b[1]));
}

/* Kept items in order; with `partition`, the j-th rejected item at out[n - 1 - j].  Returns the
 * number kept. */
uint64_t oracle_select(int item_bytes, const void* in, const uint8_t* sel, uint64_t n, void* out, int partition) {
    uint64_t kept = 0, rejected = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t v = load_bits(in, i, item_bytes);
        if (sel[i]) store_bits(out, kept++, item_bytes, v);
        else if (partition) store_bits(out, n - 1 - rejected++, item_bytes, v);
    }
    return kept;
}

void oracle_partition_three_way(int item_bytes, const void* in, const uint8_t* first, const uint8_t* second,
                                uint64_t n, void* first_out, void* second_out, void* unselected_out,
                                uint64_t* counts) {
    uint64_t c1 = 0, c2 = 0, u = 0;
    for (uint64_t i = 0; i < n; ++i) {
        if (first[i]) ++c1;
        else if (second[i]) ++c2;
        else ++u;
    }
    uint64_t k1 = 0, k2 = 0, ku = 0;
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t v = load_bits(in, i, item_bytes);
        if (first[i]) store_bits(first_out, k1++, item_bytes, v);
        else if (second[i]) store_bits(second_out, k2++, item_bytes, v);
        else store_bits(unselected_out, u - 1 - ku++, item_bytes, v);
    }
    counts[0] = c1;
    counts[1] = c2;
}

/* unique[r] = value of run r, counts[r] = its length; returns the number of runs. */
uint64_t oracle_run_length_encode(int type, const void* in, uint64_t n, void* unique_out, uint32_t* counts) {
    const int bytes = type_bytes(type);
    uint64_t runs = 0;
    for (uint64_t i = 0; i < n; ++i) {
        if (i == 0 || !item_equal(type, in, i, i - 1, ~0ull)) {
            store_bits(unique_out, runs, bytes, load_bits(in, i, bytes));
            counts[runs++] = 1;
        } else {
            counts[runs - 1] += 1;
        }
    }
    return runs;
}

/* offsets[r], lengths[r] of the r-th run longer than one item; returns how many there are. */
uint64_t oracle_non_trivial_runs(int type, const void* in, uint64_t n, uint32_t* offsets, uint32_t* lengths) {
    uint64_t found = 0, start = 0;
    for (uint64_t i = 1; i <= n; ++i) {
        if (i == n || !item_equal(type, in, i, i - 1, ~0ull)) {
            if (i - start > 1) {
                offsets[found] = (uint32_t)start;
                lengths[found] = (uint32_t)(i - start);
                ++found;
            }
            start = i;
        }
    }
    return n == 0 ? 0 : found;
}

/* ------------------------------------------------------------------------------------------------
 * Segmented reductions and scans.  Follows DeviceSegmentReduce<> (src/lcpp/device/
 * device_segment_reduce.h:110-420, details/segment_reduce.h:120-165,302-345) and DeviceSegmentedScan<>
 * (src/lcpp/device/device_segmented_scan.h:52-224).  Segment s covers [begin[s], end[s]); begin >= end
 * is empty.  op: 0 sum, 1 min, 2 max, 3 argmin, 4 argmax.  Empty segments: sum 0, min = the type's
 * max, max = lowest, arg: that value and index 1.  Arg indices are relative to begin, ties go to the
 * lower index.  Integer sums wrap; float min / max ignore NaN (fmin / fmax); float sums are long
 * double with the sum of |items| in abs_out (may be NULL).
 * ---------------------------------------------------------------------------------------------- */
static long double fp_type_at(int type, const void* p, uint64_t i) {
    return type == 2 ? (long double)((const float*)p)[i] : (long double)((const double*)p)[i];
}

static int int_less(int type, uint64_t a, uint64_t b) {
    if (type == 0) return (int32_t)(uint32_t)a < (int32_t)(uint32_t)b;
    if (type == 3) return (int64_t)a < (int64_t)b;
    return a < b;
}

void oracle_segment_reduce(int type, int op, const void* in, const uint32_t* begins, const uint32_t* ends,
                           uint64_t num_segments, void* out, uint32_t* index_out, double* abs_out) {
    const int bytes = type_bytes(type);
    const int is_fp = type == 2 || type == 5;
    const uint64_t mask = bytes == 8 ? ~0ull : 0xFFFFFFFFull;
    for (uint64_t s = 0; s < num_segments; ++s) {
        const uint64_t b = begins[s], e = ends[s];
        if (op == 0) {
            if (is_fp) {
                long double acc = 0, ab = 0;
                for (uint64_t i = b; i < e; ++i) {
                    acc += fp_type_at(type, in, i);
                    ab += fabsl(fp_type_at(type, in, i));
                }
                if (type == 2) ((float*)out)[s] = (float)acc;
                else ((double*)out)[s] = (double)acc;
                if (abs_out) abs_out[s] = (double)ab;
            } else {
                uint64_t acc = 0;
                for (uint64_t i = b; i < e; ++i) acc += load_bits(in, i, bytes);
                store_bits(out, s, bytes, acc & mask);
            }
            continue;
        }
        const int want_min = op == 1 || op == 3;
        int have = 0;
        uint64_t best_bits = 0, best_i = 0;
        double best_fp = 0;
        for (uint64_t i = b; i < e; ++i) {
            if (is_fp) {
                const double v = (double)fp_type_at(type, in, i);
                if (v != v) continue; /* NaN never wins */
                if (!have || (want_min ? v < best_fp : v > best_fp)) {
                    best_fp = v;
                    best_i = i;
                    have = 1;
                }
            } else {
                const uint64_t v = load_bits(in, i, bytes);
                if (!have || (want_min ? int_less(type, v, best_bits) : int_less(type, best_bits, v))) {
                    best_bits = v;
                    best_i = i;
                    have = 1;
                }
            }
        }
        if (!have) {
            /* initial value: the type's max for min forms, lowest for max forms */
            if (type == 2) ((float*)out)[s] = want_min ? 3.40282347e+38f : -3.40282347e+38f;
            else if (type == 5) ((double*)out)[s] = want_min ? 1.7976931348623157e308 : -1.7976931348623157e308;
            else if (type == 0) store_bits(out, s, 4, want_min ? 0x7FFFFFFFull : 0x80000000ull);
            else if (type == 3) store_bits(out, s, 8, want_min ? 0x7FFFFFFFFFFFFFFFull : 0x8000000000000000ull);
            else store_bits(out, s, bytes, want_min ? mask : 0);
            if (index_out) index_out[s] = 1;
        } else {
            if (type == 2) ((float*)out)[s] = (float)best_fp;
            else if (type == 5) ((double*)out)[s] = best_fp;
            else store_bits(out, s, bytes, best_bits);
            if (index_out) index_out[s] = (uint32_t)(best_i - b);
        }
    }
}

/* out[out_begin[s] + k] = init + sum of the segment's items before k (exclusive) or up to k
 * (inclusive; plus init when use_init). */
void oracle_segmented_scan(int type, const void* in, const uint32_t* begins, const uint32_t* ends,
                           const uint32_t* out_begins, uint64_t num_segments, int inclusive, int use_init,
                           uint64_t init_bits, double init_fp, void* out, double* abs_out) {
    const int bytes = type_bytes(type);
    const int is_fp = type == 2 || type == 5;
    const uint64_t mask = bytes == 8 ? ~0ull : 0xFFFFFFFFull;
    for (uint64_t s = 0; s < num_segments; ++s) {
        const uint64_t b = begins[s], e = ends[s], ob = out_begins[s];
        uint64_t acc = (use_init || !inclusive) ? init_bits : 0;
        long double facc = (use_init || !inclusive) ? init_fp : 0, ab = fabsl((long double)init_fp);
        for (uint64_t i = b; i < e; ++i) {
            const uint64_t o = ob + (i - b);
            if (is_fp) {
                const long double v = fp_type_at(type, in, i);
                if (inclusive) {
                    facc += v;
                    ab += fabsl(v);
                }
                if (type == 2) ((float*)out)[o] = (float)facc;
                else ((double*)out)[o] = (double)facc;
                if (abs_out) abs_out[o] = (double)ab;
                if (!inclusive) {
                    facc += v;
                    ab += fabsl(v);
                }
            } else {
                const uint64_t v = load_bits(in, i, bytes);
                if (inclusive) acc += v;
                store_bits(out, o, bytes, acc & mask);
                if (!inclusive) acc += v;
            }
        }
    }
}

/* ------------------------------------------------------------------------------------------------
 * Segmented sorts.  Follows DeviceSegmentedSort<> (src/lcpp/device/device_segmented_sort.h:43-505):
 * every segment [begin[s], end[s]) (begin < end <= n) is sorted stably by the comparator; items outside
 * every segment are not written.  DeviceSegmentedRadixSort<> (device_segmented_radix_sort.h:215-246)
 * compares ((TwiddleIn(bits) >> begin_bit) & mask) for bits [begin_bit, end_bit); value_order compares
 * the values (lhs < rhs; for floats -0.0 equals +0.0).  descending reverses the comparison.
 * ---------------------------------------------------------------------------------------------- */
static uint64_t sort_order_key(int type, uint64_t bits, uint32_t begin_bit, uint32_t end_bit) {
    const int width = type_bytes(type) * 8;
    const uint64_t sign = 1ull << (width - 1);
    const uint64_t full = width == 64 ? ~0ull : ((1ull << width) - 1);
    uint64_t t = bits & full;
    if (type == 0 || type == 3) t ^= sign;
    else if (type == 2 || type == 5) t = (t & sign) ? (~t & full) : (t | sign);
    const uint32_t nb = end_bit - begin_bit;
    if (nb == 0) return 0;
    const uint64_t mask = nb >= 64 ? ~0ull : ((1ull << nb) - 1);
    return (t >> begin_bit) & mask;
}

typedef struct {
    int type, descending, value_order;
    uint32_t begin_bit, end_bit;
    const void* keys;
} sort_ctx;

/* a strictly before b */
static int sort_before(const sort_ctx* c, uint64_t a, uint64_t b) {
    if (c->value_order && (c->type == 2 || c->type == 5)) {
        const double x = (double)fp_type_at(c->type, c->keys, a), y = (double)fp_type_at(c->type, c->keys, b);
        return c->descending ? y < x : x < y;
    }
    const int bytes = type_bytes(c->type);
    const uint64_t x = sort_order_key(c->type, load_bits(c->keys, a, bytes), c->begin_bit, c->end_bit);
    const uint64_t y = sort_order_key(c->type, load_bits(c->keys, b, bytes), c->begin_bit, c->end_bit);
    return c->descending ? y < x : x < y;
}

/* Stable bottom-up merge sort of idx[0, len) by sort_before. */
static void stable_sort_indices(const sort_ctx* c, uint64_t* idx, uint64_t* tmp, uint64_t len) {
    for (uint64_t w = 1; w < len; w *= 2) {
        for (uint64_t lo = 0; lo < len; lo += 2 * w) {
            const uint64_t mid = lo + w < len ? lo + w : len, hi = lo + 2 * w < len ? lo + 2 * w : len;
            uint64_t i = lo, j = mid, k = lo;
            while (i < mid && j < hi) tmp[k++] = sort_before(c, idx[j], idx[i]) ? idx[j++] : idx[i++];
            while (i < mid) tmp[k++] = idx[i++];
            while (j < hi) tmp[k++] = idx[j++];
        }
        memcpy(idx, tmp, len * sizeof(uint64_t));
    }
}

int oracle_segmented_sort(int type, const void* keys_in, void* keys_out, int value_bytes, const void* values_in,
                          void* values_out, uint64_t n, uint64_t num_segments, const uint32_t* begins,
                          const uint32_t* ends, uint32_t begin_bit, uint32_t end_bit, int descending,
                          int value_order) {
    const int kb = type_bytes(type);
    sort_ctx c = {type, descending, value_order, begin_bit, end_bit, keys_in};
    for (uint64_t s = 0; s < num_segments; ++s) {
        const uint64_t b = begins[s], e = ends[s];
        if (b >= e || e > n) continue;
        const uint64_t len = e - b;
        uint64_t* idx = (uint64_t*)malloc(len * sizeof(uint64_t));
        uint64_t* tmp = (uint64_t*)malloc(len * sizeof(uint64_t));
        if (!idx || !tmp) {
            free(idx);
            free(tmp);
            return -1;
        }
        for (uint64_t i = 0; i < len; ++i) idx[i] = b + i;
        stable_sort_indices(&c, idx, tmp, len);
        for (uint64_t i = 0; i < len; ++i) {
            store_bits(keys_out, b + i, kb, load_bits(keys_in, idx[i], kb));
            if (value_bytes) store_bits(values_out, b + i, value_bytes, load_bits(values_in, idx[i], value_bytes));
        }
        free(idx);
        free(tmp);
    }
    return 0;
}
