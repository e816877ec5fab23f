// Shared building blocks for the gfx950 (CDNA4, wave64) kernels of the LCPP device hot path:
// wave-level scans built from DPP lane moves, agent-scope atomics for cross-workgroup state,
// launch helpers with optional per-kernel event timing, and the C-ABI status plumbing.
//
// Reference counterparts (LuisaCompute-ParallelPrimitive):
//   warp/details/warp_scan_shlf.h:161-205   32-lane Kogge-Stone inclusive scan  -> wave_inclusive_scan
//   warp/details/warp_reduce_shlf.h:37-76   32-lane reduce-down tree             -> wave_reduce
//   common/cuda_tile_state.h:15-80          relaxed GPU-scope 32/64-bit ld/st    -> atomic_load_agent / atomic_store_agent
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <cstddef>
#include <limits>
#include <type_traits>

namespace lcpp_hip {

constexpr int kWave = 64;

// Returned by an alternative implementation that leaves a call to the general one (not an error).
constexpr int kRunsDeclined = 1;
// by_key.hip: DeviceRunLengthEncode::Encode (counts_out non-null) or DeviceSelect::Unique (null) over the
// by-key reduce kernels; K is uint32_t, uint64_t, float or double.
template <typename K>
int runs_by_key(void* temp, size_t temp_bytes, const K* in, K* unique_out, uint32_t* counts_out, uint32_t* num_out,
                uint64_t n, uint64_t key_mask, hipStream_t stream);

// ------------------------------------------------------------------------------------------------
// Arithmetic operators (the subset of common/thread_operators.h used on the hot path).
// ------------------------------------------------------------------------------------------------
struct SumOp {
    template <typename T>
    __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
    template <typename T>
    __device__ __forceinline__ static constexpr T identity() { return T(0); }
};

// Min / max operators: the reference's MinOp and MaxOp (common/thread_operators.h:58-74).  They compare
// in the item's own type, floats like fmin / fmax (a NaN operand yields the other one; -0.0 and +0.0
// compare equal, so the older is kept).  Identities: the type's max / lowest for integers; a quiet NaN
// for floats, the one value that every float operand, NaN included, absorbs (op(x, NaN) = op(NaN, x) =
// x), so padding and empty prefixes leave a scan or a reduction equal to the left-to-right fold of its
// items.
struct MinValueOp {
    template <typename T>
    __device__ __forceinline__ T operator()(T a, T b) const {
        if constexpr (std::is_floating_point_v<T>) return (b < a || a != a) ? b : a;  // a NaN operand yields the other
        else return b < a ? b : a;
    }
    template <typename T>
    __host__ __device__ __forceinline__ static constexpr T identity() {
        if constexpr (std::is_floating_point_v<T>) return std::numeric_limits<T>::quiet_NaN();
        else return std::numeric_limits<T>::max();
    }
};
struct MaxValueOp {
    template <typename T>
    __device__ __forceinline__ T operator()(T a, T b) const {
        if constexpr (std::is_floating_point_v<T>) return (b > a || a != a) ? b : a;
        else return b > a ? b : a;
    }
    template <typename T>
    __host__ __device__ __forceinline__ static constexpr T identity() {
        if constexpr (std::is_floating_point_v<T>) return std::numeric_limits<T>::quiet_NaN();
        else return std::numeric_limits<T>::lowest();
    }
};

// ------------------------------------------------------------------------------------------------
// DPP lane moves. `__builtin_amdgcn_update_dpp(old, src, ctrl, row_mask, bank_mask, bound_ctrl)`:
// lanes whose source lane is invalid, or whose row is masked off, receive `old`.
// Control codes (GFX9 DPP): row_shr:n = 0x110+n, wave_shl:1 = 0x130, wave_shr:1 = 0x138, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.
// ------------------------------------------------------------------------------------------------
namespace dpp {
constexpr int kRowShr1 = 0x111;
constexpr int kRowShr2 = 0x112;
constexpr int kRowShr4 = 0x114;
constexpr int kRowShr8 = 0x118;
constexpr int kWaveShl1 = 0x130;
constexpr int kWaveShr1 = 0x138;
constexpr int kRowBcast15 = 0x142;
constexpr int kRowBcast31 = 0x143;
}  // namespace dpp

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_move_u32(uint32_t old, uint32_t src) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(src), CTRL,
                                                             ROW_MASK, BANK_MASK, false));
}

// Moves a value of any 4- or 8-byte type through DPP (8-byte values move as two halves).
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf, typename T>
__device__ __forceinline__ T dpp_move(T old, T src) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "dpp_move supports 4- and 8-byte values");
    if constexpr (sizeof(T) == 4) {
        uint32_t o = __builtin_bit_cast(uint32_t, old);
        uint32_t s = __builtin_bit_cast(uint32_t, src);
        return __builtin_bit_cast(T, dpp_move_u32<CTRL, ROW_MASK, BANK_MASK>(o, s));
    } else {
        uint64_t o = __builtin_bit_cast(uint64_t, old);
        uint64_t s = __builtin_bit_cast(uint64_t, src);
        uint32_t lo = dpp_move_u32<CTRL, ROW_MASK, BANK_MASK>(static_cast<uint32_t>(o), static_cast<uint32_t>(s));
        uint32_t hi = dpp_move_u32<CTRL, ROW_MASK, BANK_MASK>(static_cast<uint32_t>(o >> 32),
                                                              static_cast<uint32_t>(s >> 32));
        return __builtin_bit_cast(T, (static_cast<uint64_t>(hi) << 32) | lo);
    }
}

// Inclusive scan over the 64 lanes of a wave (all lanes must be active).
// Rows of 16 lanes are scanned with row_shr 1/2/4/8, then row totals are carried with
// row_bcast:15 (row r-1's last lane into rows 1 and 3) and row_bcast:31 (lane 31 into rows 2, 3).
// The value from lower lanes is always the left operand, so an operator that is associative but not
// commutative (a min that keeps the earlier of two equal values) sees its operands in lane order.
template <typename T, typename Op>
__device__ __forceinline__ T wave_inclusive_scan(T x, Op op) {
    const T id = Op::template identity<T>();
    x = op(dpp_move<dpp::kRowShr1>(id, x), x);
    x = op(dpp_move<dpp::kRowShr2>(id, x), x);
    x = op(dpp_move<dpp::kRowShr4>(id, x), x);
    x = op(dpp_move<dpp::kRowShr8>(id, x), x);
    x = op(dpp_move<dpp::kRowBcast15, 0xa>(id, x), x);
    x = op(dpp_move<dpp::kRowBcast31, 0xc>(id, x), x);
    return x;
}

// Shifts an inclusive scan right by one lane; lane 0 receives the identity.
template <typename T, typename Op>
__device__ __forceinline__ T wave_shift_exclusive(T inclusive) {
    return dpp_move<dpp::kWaveShr1>(Op::template identity<T>(), inclusive);
}

template <typename T>
__device__ __forceinline__ T wave_read_lane(T x, int lane) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
    } else {
        uint64_t v = __builtin_bit_cast(uint64_t, x);
        uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), lane));
        uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), lane));
        return __builtin_bit_cast(T, (static_cast<uint64_t>(hi) << 32) | lo);
    }
}

// Reduction over the 64 lanes of a wave; every lane receives the total.
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T x, Op op) {
    return wave_read_lane(wave_inclusive_scan(x, op), kWave - 1);
}

__device__ __forceinline__ uint32_t lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// Number of set bits of `mask` in lanes strictly below the calling lane.
__device__ __forceinline__ uint32_t popc_lanes_below(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

__device__ __forceinline__ uint64_t wave_ballot(bool p) { return __ballot(p); }

// Lanes of the wave whose 8-bit digit equals this lane's.  Per digit bit: t = 0 or ~0 (the bit,
// sign-extended by one bit-field extract), one ballot of t != 0, and differ |= ballot ^ t on each 32-bit
// half as one three-input bit operation (truth table 0xF6: S0 | (S1 ^ S2)); peers = ~differ.  Four VALU
// operations per bit.  The empty asm keeps t opaque, so that the ballot compares t itself instead of a
// shifted copy of the digit (which costs a shift more per bit).
__device__ __forceinline__ uint64_t match_digit(uint32_t d) {
    uint32_t lo = 0u, hi = 0u;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        uint32_t t = static_cast<uint32_t>(__builtin_amdgcn_sbfe(static_cast<int32_t>(d), b, 1));
        asm volatile("" : "+v"(t));
        const uint64_t m = wave_ballot(t != 0);
        lo = __builtin_amdgcn_bitop3_b32(lo, static_cast<uint32_t>(m), t, 0xF6);
        hi = __builtin_amdgcn_bitop3_b32(hi, static_cast<uint32_t>(m >> 32), t, 0xF6);
    }
    return (static_cast<uint64_t>(~hi) << 32) | ~lo;
}


// ------------------------------------------------------------------------------------------------
// Agent-scope (whole-GPU, all XCDs) relaxed atomics for cross-workgroup status words.
// ------------------------------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ T atomic_load_agent(const T* p) {
    return __hip_atomic_load(const_cast<T*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ void atomic_store_agent(T* p, T v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T atomic_add_agent(T* p, T v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------------------------------------
// Per-tile phase stamps, compiled in only when LCPP_HIP_PHASE_TRACE is defined (the diagnostic
// library liblcpp_hip_trace.so; the product library carries none of this).  A kernel takes
// `s_memtime` (shader clock cycles) at its phase boundaries and thread 0 writes one record of
// kTraceWords 64-bit words per tile: [0] s_memrealtime at start (100 MHz), [1..N] s_memtime
// stamps, [13] kernel-specific counters, [14] HW_ID, [15] s_memrealtime at the end.
// ------------------------------------------------------------------------------------------------
#ifdef LCPP_HIP_PHASE_TRACE
constexpr bool kPhaseTrace = true;
#else
constexpr bool kPhaseTrace = false;
#endif
constexpr int kTraceWords = 16;
constexpr int kTraceStamps = 12;  // s_memtime slots 1..12

struct PhaseClock {
    uint64_t wall0 = 0;
    uint64_t t[kTraceStamps] = {};
    __device__ __forceinline__ void start() {
        if constexpr (kPhaseTrace) {
            wall0 = __builtin_amdgcn_s_memrealtime();
            t[0] = __builtin_amdgcn_s_memtime();
        }
    }
    // Stamp I (1 <= I < kTraceStamps).  `drain` first waits for the wave's outstanding memory
    // operations, so the stamp marks their completion rather than their issue.
    template <int I>
    __device__ __forceinline__ void mark(bool drain = false) {
        static_assert(I > 0 && I < kTraceStamps, "stamp index");
        if constexpr (kPhaseTrace) {
            if (drain) __builtin_amdgcn_s_waitcnt(0);
            t[I] = __builtin_amdgcn_s_memtime();
        }
    }
    // Called by one thread: writes the record of `slot` if the buffer has room for it.
    __device__ __forceinline__ void write(uint64_t* buffer, uint64_t records, uint64_t slot, uint64_t counters) {
        if constexpr (kPhaseTrace) {
            if (buffer == nullptr || slot >= records) return;
            uint64_t* r = buffer + slot * kTraceWords;
            r[0] = wall0;
#pragma unroll
            for (int i = 0; i < kTraceStamps; ++i) r[1 + i] = t[i];
            r[13] = counters;
            // HW_ID (wave, SIMD, CU, shader array and engine of this wave): s_getreg_b32 of hwreg 4, bits 0..31.
            r[14] = static_cast<uint32_t>(__builtin_amdgcn_s_getreg((31 << 11) | 4));
            r[15] = __builtin_amdgcn_s_memrealtime();
        }
    }
};

// ------------------------------------------------------------------------------------------------
// Small fill kernel (used instead of hipMemsetAsync so that callers may capture our launches
// into HIP graphs).
// ------------------------------------------------------------------------------------------------
__global__ void fill_u32_kernel(uint32_t* dst, uint64_t count, uint32_t value);

// ------------------------------------------------------------------------------------------------
// Host-side helpers (defined in capi.cpp).
// ------------------------------------------------------------------------------------------------
constexpr size_t kViewAlign = 256;  // every carved temp region starts on a 256-byte boundary
inline constexpr size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
inline constexpr uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// Status codes of the C-ABI (mirrored in include/lcpp_hip.h).
enum Status : int {
    kOk = 0,
    kInvalidArgument = -1,
    kTempTooSmall = -2,
    kHipError = -3,
    kUnsupported = -4,
};

int set_error(int status, const char* fmt, ...);
int check_hip(hipError_t e, const char* what);

// Launch bookkeeping: when profiling is enabled, events are recorded around each launch on the
// launch stream so that per-kernel device time can be reported.
struct LaunchScope {
    const char* name;
    hipStream_t stream;
    void* begin_event;
    LaunchScope(const char* name, hipStream_t stream);
    ~LaunchScope();
};

int launch_fill_u32(uint32_t* dst, uint64_t count, uint32_t value, hipStream_t stream);

// Device-to-device copy of `bytes` (a kernel, so graph capture records no memcpy node).  Ranges must not overlap.
int launch_copy(void* dst, const void* src, uint64_t bytes, hipStream_t stream);

#ifdef LCPP_HIP_PHASE_TRACE
// Points the phase-trace records of one translation unit's kernels at `buffer` (diagnostic build).
int radix_trace_set_buffer(void* buffer, uint64_t records);
int scan_trace_set_buffer(void* buffer, uint64_t records);
#endif

// Number of compute units of the current device (cached per device).
int device_cu_count();

// Polls of an INVALID look-back predecessor before the waiting workgroup computes that
// predecessor's contribution itself (0: at once).  Shared by every look-back kernel.  A test hook: any
// value gives the same results.  Entry points read it once per call, so a concurrent change on another
// thread takes effect at the next call.
extern std::atomic<uint32_t> g_lookback_spin_limit;
inline uint32_t lookback_spin_limit() { return g_lookback_spin_limit.load(std::memory_order_relaxed); }

}  // namespace lcpp_hip
