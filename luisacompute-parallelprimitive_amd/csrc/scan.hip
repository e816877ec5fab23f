// DeviceScan::ExclusiveSum / InclusiveSum for gfx950: single-pass decoupled look-back.
//
// Reference path: DeviceScan<>::ExclusiveSum -> dispatch_scan (src/lcpp/device/device_scan.h:370-385,
// 868-948) -> ScanModule/build_scan (device/details/scan.h:241-335) with TilePrefixCallbackOp
// (device/details/single_pass_scan_operator.h:219-332) over packed (status, value) words
// (single_pass_scan_operator.h:119-172) and tile statuses INVALID / PARTIAL / INCLUSIVE (:26-32).
//
// MI355X design
//   * Tile = 256 threads x 24 rows x one 128-bit vector per thread per row (96 x 4-byte items per
//     thread, 24,576 items; 48 x 8-byte items, 12,288), held in registers.  Row r of a tile is a
//     contiguous 4 KiB range and thread t holds the t-th 16 bytes of every row, so each row is one
//     fully coalesced 4 KiB load and store.
//   * Tile = workgroup index.  There is no tile ticket: a same-address agent-scope atomic costs
//     ~11 ns on MI355X and serialises, which would cap a 2^28 scan at ~0.75 ms.  Workgroups are
//     dispatched in index order in practice, so predecessors are normally running; forward progress
//     does not rely on it: a look-back that finds a predecessor still INVALID after a bounded spin
//     claims that tile (compare-and-swap INVALID -> CLAIMED), computes its aggregate from the input
//     itself (same summation order as its owner, so float results do not depend on timing) and
//     publishes it as PARTIAL ("decoupled fallback").  The owner publishes with a compare-and-swap
//     too; when it finds its tile CLAIMED it waits for the claimer's PARTIAL before writing any
//     output, so an in-place scan (in == out) never overwrites input that a claimer still reads.
//   * In-tile scan: per-thread 4-item scans, one wave64 DPP scan per row (independent, so they
//     interleave), and a rows x waves table of wave totals in LDS.
//   * Look-back: wave 0 publishes PARTIAL, then inspects 4 predecessors per step (one per lane of
//     its first 4) with agent-scope loads, sums back to the nearest INCLUSIVE predecessor with a DPP
//     reduction,
//     and publishes INCLUSIVE.  Status and value share one 64-bit word: flag in the low half,
//     value bits in the high half, so one relaxed atomic load observes both consistently.  An
//     8-byte value takes two such words (low and high 32 bits); a reader accepts a state only when
//     both words carry the same published flag, and every publication writes word 1 before word 0
//     (word 0 with release ordering where a helper and the owner could both write word 1), so the
//     flag pair identifies one publication.
// Algorithmic traffic: 2 * n * sizeof(T) bytes (read input, write output) + 8 * sizeof(T) / 4 bytes per tile.
#include "common.hpp"
#include "../../include/lcpp_hip.h"

#include <limits>
#include <mutex>
#include <type_traits>

namespace lcpp_hip {
namespace {

// 24 rows: 96 items per thread and 24,576 per tile (measured best on MI355X among 4K..48K-item tiles
// and 256..1024-thread workgroups).  Large tiles matter because a tile's look-back waits on its
// predecessors' publications; fewer, larger tiles shorten that chain relative to the data moved.
constexpr int kScanBlock = 256;
constexpr int kScanRows = 24;
constexpr int kScanWaves = kScanBlock / kWave;
template <typename T>
constexpr int kVec = 16 / static_cast<int>(sizeof(T));  // items per thread per row
template <typename T>
constexpr uint32_t kScanTile = kScanBlock * kScanRows * kVec<T>;  // 24,576 4-byte or 12,288 8-byte items
template <typename T>
constexpr int kStateWords = static_cast<int>(sizeof(T)) / 4;  // 64-bit status words per tile
// Three workgroups per CU (at most 168 VGPRs): one workgroup's look-back wait is covered by the others'
// loads and stores.  (Measured at 2^28 u32: 0.388 ms, against 0.395 ms at two per CU with row bases
// kept in registers, and 0.405 ms with 16-row tiles at four per CU.)
constexpr int kScanBlocksPerCu = 3;

constexpr uint32_t kFlagInvalid = 0;
constexpr uint32_t kFlagPartial = 1;
constexpr uint32_t kFlagInclusive = 2;
constexpr uint32_t kFlagClaimed = 3;  // a look-back is computing this tile's aggregate

// Scan operators: SumOp, MinValueOp and MaxValueOp (common.hpp), the reference's SumOp, MinOp and MaxOp
// (common/thread_operators.h:49-74).

#ifdef LCPP_HIP_PHASE_TRACE
// Phase-trace buffer of the diagnostic build: one record per tile.
__device__ uint64_t* g_trace_buffer = nullptr;
__device__ uint64_t g_trace_records = 0;
#endif

// Temp layout: sizeof(T) / 4 status words of 8 bytes per tile.
size_t scan_needed_bytes(uint64_t n, size_t elem_bytes) {
    const uint64_t tile = static_cast<uint64_t>(kScanBlock) * kScanRows * (16 / elem_bytes);
    return ceil_div(n, tile) * 8 * (elem_bytes / 4);
}

// Status word w of a tile: flag in the low half, bits 32w..32w+31 of the value in the high half.
template <typename T>
__device__ __forceinline__ uint64_t pack_word(uint32_t flag, T value, int w) {
    uint64_t bits;
    if constexpr (sizeof(T) == 4) bits = __builtin_bit_cast(uint32_t, value);
    else bits = __builtin_bit_cast(uint64_t, value) >> (32 * w);
    return (static_cast<uint64_t>(static_cast<uint32_t>(bits)) << 32) | flag;
}

template <typename T>
struct TileState {
    uint32_t flag;  // kFlagInvalid also stands for "words of two different publications"
    T value;
};

// PARTIAL or INCLUSIVE: the state carries a usable value.
__device__ __forceinline__ bool flag_published(uint32_t flag) { return flag - kFlagPartial < 2u; }

template <typename T>
__device__ __forceinline__ TileState<T> load_state(uint64_t* states, uint64_t tile) {
    if constexpr (sizeof(T) == 4) {
        const uint64_t w = atomic_load_agent(&states[tile]);
        return {static_cast<uint32_t>(w), __builtin_bit_cast(T, static_cast<uint32_t>(w >> 32))};
    } else {
        const uint64_t w0 = atomic_load_agent(&states[2 * tile]);
        const uint64_t w1 = atomic_load_agent(&states[2 * tile + 1]);
        const uint32_t f0 = static_cast<uint32_t>(w0), f1 = static_cast<uint32_t>(w1);
        // CLAIMED lives in word 0 only; any other mismatch is a publication in progress.
        const uint32_t flag = f0 == f1 ? f0 : (f0 == kFlagClaimed ? kFlagClaimed : kFlagInvalid);
        return {flag, __builtin_bit_cast(T, (w0 >> 32) | (w1 & 0xFFFFFFFF00000000ull))};
    }
}

// Publishes (flag, value) for `tile`: word 1 first, then word 0 (release when `release`, so that a
// reader of word 0 with acquire ordering also observes word 1).
template <typename T>
__device__ __forceinline__ void store_state(uint64_t* states, uint64_t tile, uint32_t flag, T value, bool release) {
    if constexpr (sizeof(T) == 4) {
        (void)release;
        atomic_store_agent(&states[tile], pack_word(flag, value, 0));
    } else {
        atomic_store_agent(&states[2 * tile + 1], pack_word(flag, value, 1));
        if (release)
            __hip_atomic_store(&states[2 * tile], pack_word(flag, value, 0), __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        else
            atomic_store_agent(&states[2 * tile], pack_word(flag, value, 0));
    }
}

// Left projection, op(a, b) = a: the reference's left-operand lambda (tests/device_scan_test.cpp:129-155,
// tests/scan_optimization_regression_test.cpp:195-205), an associative operator that does not commute,
// so its results show the order in which every level of the scan combines operands.  It has no identity;
// the kernels adjoin one, the all-ones bit pattern (the sentinel): op(a, b) = b when a holds the sentinel,
// else a.  That monoid gives exactly the left projection whenever the scan's first operand (init, or
// in[0] without init) is not the sentinel; when it is, every output is the sentinel, which the scan
// writes directly.
struct LeftOp {
    template <typename T>
    __host__ __device__ __forceinline__ static constexpr bool is_sentinel(T x) {
        using U = std::conditional_t<sizeof(T) == 4, uint32_t, uint64_t>;
        return __builtin_bit_cast(U, x) == ~U(0);
    }
    template <typename T>
    __device__ __forceinline__ T operator()(T a, T b) const { return is_sentinel(a) ? b : a; }
    template <typename T>
    __host__ __device__ __forceinline__ static constexpr T identity() {
        using U = std::conditional_t<sizeof(T) == 4, uint32_t, uint64_t>;
        return __builtin_bit_cast(T, ~U(0));
    }
};

// Item `idx` of the input, or the operator's identity past the end.
template <typename T, typename Op>
__device__ __forceinline__ T load_item(const T* in, uint64_t n, uint64_t idx) {
    return idx < n ? in[idx] : Op::template identity<T>();
}

// Aggregate of (full) tile `tile`, computed by one wave in exactly the order its owner uses: per
// thread ((x0+x1)+x2)+x3, a DPP wave scan per (row, wave), wave totals summed per row in wave order,
// rows summed in row order.
template <typename T, typename Op>
__device__ T tile_aggregate(const T* in, uint64_t n, uint32_t tile, int vector_io) {
    constexpr int V = kVec<T>;
    using Vec = T __attribute__((ext_vector_type(V)));
    const uint32_t lane = lane_id();
    const uint64_t tile_base = static_cast<uint64_t>(tile) * kScanTile<T>;
    const Op op{};
    T running = Op::template identity<T>();
    for (int r = 0; r < kScanRows; ++r) {
        T row_total = Op::template identity<T>();
        for (int w = 0; w < kScanWaves; ++w) {
            const uint64_t first = tile_base + (static_cast<uint64_t>(r) * kScanBlock + w * kWave + lane) * V;
            Vec v;
            if (vector_io && tile_base + kScanTile<T> <= n) {
                v = *reinterpret_cast<const Vec*>(in + first);
            } else {
#pragma unroll
                for (int j = 0; j < V; ++j) v[j] = load_item<T, Op>(in, n, first + j);
            }
#pragma unroll
            for (int j = 1; j < V; ++j) v[j] = op(v[j - 1], v[j]);
            row_total = op(row_total, wave_read_lane(wave_inclusive_scan(v[V - 1], op), kWave - 1));
        }
        running = op(running, row_total);
    }
    return running;
}

// Predecessors inspected per look-back step, one per lane.  Short windows win: a step waits until every
// entry of its window is published, and a wide window keeps waiting on entries that a walk of short
// steps would not have needed (ExclusiveSum 2^28 u32: 0.360 ms with 4, 0.361 with 2 or 8, 0.364 with 16,
// 0.373 with 32, 0.387 with 64 and 0.390 with 1; 2^27 u64: 0.364 ms with 4, 0.414 with 64).
constexpr int kScanWindow = 4;

// Exclusive prefix of tile `tile` (> 0) over all earlier tiles; called by all 64 lanes of one wave (lanes
// kScanWindow and up take no entry: they hold a PARTIAL identity).
template <typename T, typename Op>
__device__ T scan_lookback(uint64_t* states, uint32_t tile, const T* in, uint64_t n, int vector_io,
                           uint32_t spin_limit, uint64_t& trace_counters) {
    const uint32_t lane = lane_id();
    const Op op{};
    T prefix = Op::template identity<T>();
    int64_t end = tile;  // exclusive end of the window of predecessors
    while (true) {
        const int64_t idx = end - kScanWindow + static_cast<int64_t>(lane);
        const bool in_window = lane < static_cast<uint32_t>(kScanWindow);
        TileState<T> st = !in_window ? TileState<T>{kFlagPartial, Op::template identity<T>()}
                          : idx >= 0 ? load_state<T>(states, static_cast<uint64_t>(idx))
                                     : TileState<T>{kFlagInclusive, Op::template identity<T>()};
        uint32_t spins = 0;
        while (wave_ballot(!flag_published(st.flag)) != 0) {
            if (spins >= spin_limit) {
                // Fallback: claim every still-INVALID predecessor and compute its aggregate here.
                // Predecessors CLAIMED by another look-back are simply polled until published.
                uint64_t invalid = wave_ballot(st.flag == kFlagInvalid);
                while (invalid != 0) {
                    const uint32_t src = static_cast<uint32_t>(__builtin_ctzll(invalid));
                    invalid &= invalid - 1;
                    const uint32_t j = static_cast<uint32_t>(end - kScanWindow + src);
                    bool won = false;
                    if (lane == src) {
                        // Word 0 INVALID with value 0, as the clear leaves it.  (A tile whose words are
                        // mid-publication fails the exchange and is polled again.)
                        uint64_t expected = 0;
                        won = __hip_atomic_compare_exchange_strong(&states[static_cast<uint64_t>(j) * kStateWords<T>],
                                                                   &expected, uint64_t(kFlagClaimed), __ATOMIC_RELAXED,
                                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if (won) st.flag = kFlagClaimed;
                    }
                    if (wave_ballot(won) != 0) {
                        if constexpr (kPhaseTrace) trace_counters += 1ull << 32;
                        const T agg = tile_aggregate<T, Op>(in, n, j, vector_io);
                        if (lane == src) {
                            st = TileState<T>{kFlagPartial, agg};
                            store_state(states, j, kFlagPartial, agg, true);
                        }
                    }
                }
            }
            __builtin_amdgcn_s_sleep(1);
            ++spins;
            if constexpr (kPhaseTrace) trace_counters += 1ull << 16;
            if (!flag_published(st.flag) && in_window) st = load_state<T>(states, static_cast<uint64_t>(idx));
        }
        if constexpr (kPhaseTrace) trace_counters += 1;
        const T value = st.value;
        const uint64_t inclusive = wave_ballot(st.flag == kFlagInclusive);
        if (inclusive != 0) {
            const uint32_t last = 63 - __builtin_clzll(inclusive);
            return op(wave_reduce(lane >= last ? value : Op::template identity<T>(), op), prefix);
        }
        // The window precedes everything folded so far: it is the left operand.
        prefix = op(wave_reduce(value, op), prefix);
        end -= kScanWindow;
    }
}

template <typename T, bool INCLUSIVE, typename Op>
__global__ __launch_bounds__(kScanBlock, kScanBlocksPerCu) void scan_kernel(const T* in, T* out, uint64_t n,
                                                                             uint64_t* __restrict__ states, T init,
                                                                             int vector_io, uint32_t spin_limit) {
    constexpr int V = kVec<T>;
    constexpr uint32_t TILE = kScanTile<T>;
    using Vec = T __attribute__((ext_vector_type(V)));
    __shared__ T s_wave_totals[kScanRows][kScanWaves];
    __shared__ T s_tile_prefix;
    const Op op{};

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint64_t tile_base = static_cast<uint64_t>(tile) * TILE;
    const bool full = vector_io && tile_base + TILE <= n;
    PhaseClock clk;
    clk.start();
    uint64_t trace_counters = 0;  // look-back steps | spins << 16 | fallback tiles << 32

    if constexpr (std::is_same_v<Op, LeftOp>) {
        // Inclusive scan without an initial value (init holds the sentinel) of an input whose first item
        // is the sentinel: every output is the sentinel.  in[0] never changes (an in-place scan writes
        // in[0] back to out[0]), so every workgroup reads the same value and takes this path alike.
        if (LeftOp::is_sentinel(init) && LeftOp::is_sentinel(in[0])) {
            const uint64_t end = tile_base + TILE < n ? tile_base + TILE : n;
            for (uint64_t i = tile_base + tid; i < end; i += kScanBlock) out[i] = init;
            return;
        }
    }

    Vec v[kScanRows];
    if (full) {
        const Vec* src = reinterpret_cast<const Vec*>(in + tile_base);
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) v[r] = __builtin_nontemporal_load(&src[r * kScanBlock + tid]);
    } else {
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) {
#pragma unroll
            for (int j = 0; j < V; ++j) {
                const uint64_t idx = tile_base + (static_cast<uint64_t>(r) * kScanBlock + tid) * V + j;
                v[r][j] = idx < n ? in[idx] : Op::template identity<T>();
            }
        }
    }

    // Thread-local inclusive scans and per-row wave scans; the wave totals go to LDS.  Only
    // v[r][0..V-2] and the wave scan stay live: the thread's row total is the wave scan minus its
    // shifted copy, and row offsets are re-read from LDS when the outputs are formed, so the kernel
    // fits 128 VGPRs (four workgroups per CU).
    T wave_incl[kScanRows];
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
#pragma unroll
        for (int j = 1; j < V; ++j) v[r][j] = op(v[r][j - 1], v[r][j]);
        wave_incl[r] = wave_inclusive_scan(v[r][V - 1], op);
        if (lane == kWave - 1) s_wave_totals[r][wave] = wave_incl[r];
    }
    __syncthreads();

    // Tile aggregate: rows in order, each row's wave totals in wave order (the order tile_aggregate
    // repeats for a helper).
    T aggregate = Op::template identity<T>();
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
        T row_total = Op::template identity<T>();
#pragma unroll
        for (int w = 0; w < kScanWaves; ++w) row_total = op(row_total, s_wave_totals[r][w]);
        aggregate = op(aggregate, row_total);
    }
    clk.mark<1>(true);  // tile loaded and scanned in registers

    // Publish (tile 0: INCLUSIVE at once; others PARTIAL, then INCLUSIVE after the look-back).  The
    // publication ends with a compare-and-swap of word 0 from INVALID: if a look-back has CLAIMED
    // this tile, the owner waits for the claimer's PARTIAL (the claimer has finished reading this
    // tile's input) before the barrier that precedes every output store.
    if (wave == 0) {
        bool claimed_by_other = false;
        if (lane == 0) {
            const uint32_t flag = tile == 0 ? kFlagInclusive : kFlagPartial;
            if constexpr (kStateWords<T> == 2) atomic_store_agent(&states[2 * tile + 1], pack_word(flag, aggregate, 1));
            uint64_t expected = 0;
            claimed_by_other = !__hip_atomic_compare_exchange_strong(
                &states[static_cast<uint64_t>(tile) * kStateWords<T>], &expected, pack_word(flag, aggregate, 0),
                __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const T excl =
            tile == 0 ? Op::template identity<T>()
                      : scan_lookback<T, Op>(states, tile, in, n, vector_io, spin_limit, trace_counters);
        clk.mark<2>();  // look-back walked
        if (lane == 0) {
            if (claimed_by_other) {
                // The claimer's word 0 is stored with release ordering after its word 1.
                while (static_cast<uint32_t>(__hip_atomic_load(&states[static_cast<uint64_t>(tile) * kStateWords<T>],
                                                               __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT)) !=
                       kFlagPartial)
                    __builtin_amdgcn_s_sleep(1);
            }
            if (tile != 0 || claimed_by_other) store_state(states, tile, kFlagInclusive, op(excl, aggregate), false);
            s_tile_prefix = excl;
        }
    }
    __syncthreads();

    T running = op(init, s_tile_prefix);  // tile prefix + rows before r
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
        T before = Op::template identity<T>(), row_total = Op::template identity<T>();
#pragma unroll
        for (int w = 0; w < kScanWaves; ++w) {
            const T x = s_wave_totals[r][w];
            if (w < static_cast<int>(wave)) before = op(before, x);
            row_total = op(row_total, x);
        }
        const T thread_excl = wave_shift_exclusive<T, Op>(wave_incl[r]);
        const T p = op(op(running, before), thread_excl);
        Vec o;
        if constexpr (INCLUSIVE) {
#pragma unroll
            for (int j = 0; j < V - 1; ++j) o[j] = op(p, v[r][j]);
            o[V - 1] = op(op(running, before), wave_incl[r]);
        } else {
            o[0] = p;
#pragma unroll
            for (int j = 1; j < V; ++j) o[j] = op(p, v[r][j - 1]);
        }
        v[r] = o;
        running = op(running, row_total);
    }
    if (full) {
        Vec* dst = reinterpret_cast<Vec*>(out + tile_base);
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) __builtin_nontemporal_store(v[r], &dst[r * kScanBlock + tid]);
    } else {
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) {
#pragma unroll
            for (int j = 0; j < V; ++j) {
                const uint64_t idx = tile_base + (static_cast<uint64_t>(r) * kScanBlock + tid) * V + j;
                if (idx < n) out[idx] = v[r][j];
            }
        }
    }
#ifdef LCPP_HIP_PHASE_TRACE
    clk.mark<3>();  // outputs issued (this wave)
    if (tid == 0) clk.write(g_trace_buffer, g_trace_records, tile, trace_counters);
#endif
}

template <typename T, typename Op>
int scan_op(const char* what, void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, bool inclusive, T init,
            void* stream_ptr) {
    static_assert(sizeof(T) == 4 || sizeof(T) == 8, "4- and 8-byte items");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items (%llu > UINT_MAX)", what,
                                            static_cast<unsigned long long>(n));
    if (n == 0) return kOk;
    if (!in || !out) return set_error(kInvalidArgument, "%s: null input or output", what);
    if (reinterpret_cast<uintptr_t>(in) % sizeof(T) != 0 || reinterpret_cast<uintptr_t>(out) % sizeof(T) != 0)
        return set_error(kInvalidArgument, "%s: input/output not aligned to the element size", what);
    const size_t needed = scan_needed_bytes(n, sizeof(T));
    if (!temp || temp_bytes < needed)
        return set_error(kTempTooSmall, "%s: temp storage too small (%zu < %zu bytes)", what, temp_bytes, needed);
    if (reinterpret_cast<uintptr_t>(temp) % 8 != 0)
        return set_error(kInvalidArgument, "%s: temp storage must be 8-byte aligned", what);

    const uint64_t tiles = ceil_div(n, kScanTile<T>);
    uint64_t* states = static_cast<uint64_t*>(temp);
    int st = launch_fill_u32(static_cast<uint32_t*>(temp), needed / 4, 0u, stream);
    if (st != kOk) return st;

    const int vector_io = (reinterpret_cast<uintptr_t>(in) % 16 == 0) && (reinterpret_cast<uintptr_t>(out) % 16 == 0);
    const uint32_t spin_limit = lookback_spin_limit();
    LaunchScope scope(std::is_same_v<Op, SumOp> ? "scan_sum" : std::is_same_v<Op, LeftOp> ? "scan_left" : "scan_minmax",
                      stream);
    if (inclusive)
        scan_kernel<T, true, Op><<<static_cast<unsigned>(tiles), kScanBlock, 0, stream>>>(in, out, n, states, init,
                                                                                        vector_io, spin_limit);
    else
        scan_kernel<T, false, Op><<<static_cast<unsigned>(tiles), kScanBlock, 0, stream>>>(in, out, n, states, init,
                                                                                         vector_io, spin_limit);
    return check_hip(hipGetLastError(), "scan launch");
}

template <typename T>
int scan_sum(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, bool inclusive, T init, void* stream) {
    return scan_op<T, SumOp>("DeviceScan", temp, temp_bytes, in, out, n, inclusive, init, stream);
}

// Scan with the left projection.  Exclusive without an initial value is rejected (the operator has no
// identity; the reference's ExclusiveScan always takes one).  An initial value equal to the sentinel makes
// every output that value, which a fill writes; everything else runs the scan kernel.
template <typename T>
int scan_left(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, bool inclusive, bool use_init, T init,
              void* stream_ptr) {
    const char* what = "DeviceScan (left projection)";
    if (!inclusive && !use_init)
        return set_error(kInvalidArgument, "%s: the operator has no identity, so an exclusive scan needs an initial value",
                         what);
    if (!(use_init && LeftOp::is_sentinel(init)))
        return scan_op<T, LeftOp>(what, temp, temp_bytes, in, out, n, inclusive, use_init ? init : LeftOp::identity<T>(),
                                  stream_ptr);
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items (%llu > UINT_MAX)", what,
                                            static_cast<unsigned long long>(n));
    if (n == 0) return kOk;
    if (!in || !out) return set_error(kInvalidArgument, "%s: null input or output", what);
    if (reinterpret_cast<uintptr_t>(out) % sizeof(T) != 0)
        return set_error(kInvalidArgument, "%s: output not aligned to the element size", what);
    const size_t needed = scan_needed_bytes(n, sizeof(T));
    if (!temp || temp_bytes < needed)
        return set_error(kTempTooSmall, "%s: temp storage too small (%zu < %zu bytes)", what, temp_bytes, needed);
    return launch_fill_u32(reinterpret_cast<uint32_t*>(out), n * sizeof(T) / 4, 0xFFFFFFFFu,
                           static_cast<hipStream_t>(stream_ptr));
}

// ---- ExclusiveSum over uint32 with no temp argument and no allocation ------------------------------
// The tile status words live in `scratch`, a static device array (each GPU holds its own copy until the
// process ends).  Host code never uses the array's name as an address: the first call on a device looks
// up that device's copy with hipGetSymbolAddress (with the device of the call's stream current) and keeps
// it.  The lookup runs outside graph capture only, so a first call under capture is an error; any earlier
// call on the device, with n == 0 included, does the lookup.  Every call on one GPU shares that copy, so
// calls that overlap in time on one GPU (other streams, other threads) race; calls in order on one stream
// do not, since each clears the words it uses (fill kernel) before its scan.
constexpr uint64_t kNoAllocMaxItems = 1ull << 30;
constexpr uint64_t kNoAllocWords = (kNoAllocMaxItems + kScanTile<uint32_t> - 1) / kScanTile<uint32_t>;  // 43,691
static __device__ __align__(256) uint64_t scratch[kNoAllocWords];  // 349,528 bytes per GPU

// Sets *words to the device's copy of `scratch` for a call on `stream`.  Status kUnsupported when the
// copy is not looked up yet and the stream is recording a graph; other failures kHipError / kUnsupported.
int scratch_of_stream(hipStream_t stream, uint64_t** words) {
    static std::mutex mu;
    static uint64_t* ptrs[64] = {};
    *words = nullptr;
    int dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) {
        (void)hipGetLastError();
        return set_error(kHipError, "ExclusiveSum (no allocation): the stream's device is unknown");
    }
    if (dev < 0 || dev >= 64)
        return set_error(kUnsupported, "ExclusiveSum (no allocation): device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(mu);
    if ((*words = ptrs[dev]) != nullptr) return kOk;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
        (void)hipGetLastError();
        return set_error(kHipError, "ExclusiveSum (no allocation): the stream's capture state is unknown");
    }
    if (capture != hipStreamCaptureStatusNone)
        return set_error(kUnsupported,
                         "ExclusiveSum (no allocation): the first call on device %d is under graph capture; the "
                         "static scratch is looked up outside capture only, so make one call on the device (n may "
                         "be 0) first",
                         dev);
    int current = 0;
    if (hipGetDevice(&current) != hipSuccess || (current != dev && hipSetDevice(dev) != hipSuccess)) {
        (void)hipGetLastError();
        return set_error(kHipError, "ExclusiveSum (no allocation): cannot make device %d current", dev);
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (current != dev) (void)hipSetDevice(current);
    if (e != hipSuccess || p == nullptr) {
        (void)hipGetLastError();
        return set_error(kHipError,
                         "ExclusiveSum (no allocation): hipGetSymbolAddress of the static scratch failed: %s",
                         hipGetErrorString(e));
    }
    *words = ptrs[dev] = static_cast<uint64_t*>(p);
    return kOk;
}

}  // namespace

#ifdef LCPP_HIP_PHASE_TRACE
int scan_trace_set_buffer(void* buffer, uint64_t records) {
    uint64_t* p = static_cast<uint64_t*>(buffer);
    int st = check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_buffer), &p, sizeof(p)), "trace buffer");
    if (st != kOk) return st;
    return check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_records), &records, sizeof(records)), "trace records");
}
#endif
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

size_t lcpp_hip_internal_scan_needed_bytes(uint64_t n, size_t elem_bytes) {
    if (elem_bytes != 4 && elem_bytes != 8) return 0;
    return n == 0 ? 0 : scan_needed_bytes(n, elem_bytes);
}

// Signed sums run in the unsigned type of the same width (identical two's-complement bits).
#define LCPP_HIP_DEFINE_SCAN(S, T, A)                                                                           \
    int lcpp_hip_scan_exclusive_sum_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n,         \
                                        void* stream) {                                                         \
        return scan_sum<A>(temp, temp_bytes, reinterpret_cast<const A*>(in), reinterpret_cast<A*>(out), n, false, \
                           A(0), stream);                                                                       \
    }                                                                                                           \
    int lcpp_hip_scan_inclusive_sum_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n,         \
                                        void* stream) {                                                         \
        return scan_sum<A>(temp, temp_bytes, reinterpret_cast<const A*>(in), reinterpret_cast<A*>(out), n, true,  \
                           A(0), stream);                                                                       \
    }                                                                                                           \
    int lcpp_hip_scan_sum_init_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int inclusive, \
                                   T init, void* stream) {                                                      \
        return scan_sum<A>(temp, temp_bytes, reinterpret_cast<const A*>(in), reinterpret_cast<A*>(out), n,        \
                           inclusive != 0, __builtin_bit_cast(A, init), stream);                                \
    }
LCPP_HIP_DEFINE_SCAN(i32, int32_t, uint32_t)
LCPP_HIP_DEFINE_SCAN(u32, uint32_t, uint32_t)
LCPP_HIP_DEFINE_SCAN(f32, float, float)
LCPP_HIP_DEFINE_SCAN(i64, int64_t, uint64_t)
LCPP_HIP_DEFINE_SCAN(u64, uint64_t, uint64_t)
LCPP_HIP_DEFINE_SCAN(f64, double, double)
#undef LCPP_HIP_DEFINE_SCAN

// Min / max scans compare in the item's own type (signed integers as signed).
#define LCPP_HIP_DEFINE_SCAN_MINMAX(S, T)                                                                        \
    int lcpp_hip_scan_min_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int inclusive,    \
                              int use_init, T init, void* stream) {                                             \
        return scan_op<T, MinValueOp>("DeviceScan (MinOp)", temp, temp_bytes, in, out, n, inclusive != 0,         \
                                     use_init ? init : MinValueOp::identity<T>(), stream);                         \
    }                                                                                                           \
    int lcpp_hip_scan_max_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int inclusive,    \
                              int use_init, T init, void* stream) {                                             \
        return scan_op<T, MaxValueOp>("DeviceScan (MaxOp)", temp, temp_bytes, in, out, n, inclusive != 0,         \
                                     use_init ? init : MaxValueOp::identity<T>(), stream);                         \
    }
LCPP_HIP_DEFINE_SCAN_MINMAX(i32, int32_t)
LCPP_HIP_DEFINE_SCAN_MINMAX(u32, uint32_t)
LCPP_HIP_DEFINE_SCAN_MINMAX(f32, float)
LCPP_HIP_DEFINE_SCAN_MINMAX(i64, int64_t)
LCPP_HIP_DEFINE_SCAN_MINMAX(u64, uint64_t)
LCPP_HIP_DEFINE_SCAN_MINMAX(f64, double)
#undef LCPP_HIP_DEFINE_SCAN_MINMAX

// Left projection: items compare by bits only (floats included).
#define LCPP_HIP_DEFINE_SCAN_LEFT(S, T, A)                                                                      \
    int lcpp_hip_scan_left_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int inclusive,   \
                               int use_init, T init, void* stream) {                                            \
        return scan_left<A>(temp, temp_bytes, reinterpret_cast<const A*>(in), reinterpret_cast<A*>(out), n,      \
                            inclusive != 0, use_init != 0, __builtin_bit_cast(A, init), stream);                 \
    }
LCPP_HIP_DEFINE_SCAN_LEFT(i32, int32_t, uint32_t)
LCPP_HIP_DEFINE_SCAN_LEFT(u32, uint32_t, uint32_t)
LCPP_HIP_DEFINE_SCAN_LEFT(f32, float, uint32_t)
LCPP_HIP_DEFINE_SCAN_LEFT(i64, int64_t, uint64_t)
LCPP_HIP_DEFINE_SCAN_LEFT(u64, uint64_t, uint64_t)
LCPP_HIP_DEFINE_SCAN_LEFT(f64, double, uint64_t)
#undef LCPP_HIP_DEFINE_SCAN_LEFT

int lcpp_hip_scan_exclusive_sum_u32_noalloc(const uint32_t* in, uint32_t* out, uint64_t n, void* stream) {
    if (n > kNoAllocMaxItems)
        return set_error(kInvalidArgument,
                         "ExclusiveSum (no allocation): %llu items exceed the static scratch (at most %llu items)",
                         static_cast<unsigned long long>(n), static_cast<unsigned long long>(kNoAllocMaxItems));
    uint64_t* words = nullptr;
    const int st = scratch_of_stream(static_cast<hipStream_t>(stream), &words);
    if (n == 0) return st == kUnsupported ? kOk : st;  // nothing to scan; a lookup failure still reports
    if (st != kOk) return st;
    return scan_sum<uint32_t>(words, kNoAllocWords * sizeof(uint64_t), in, out, n, false, 0u, stream);
}

}  // extern "C"
