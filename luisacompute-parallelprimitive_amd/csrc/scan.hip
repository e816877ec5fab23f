// DeviceScan::ExclusiveSum / InclusiveSum for gfx950: single-pass decoupled look-back.
//
// Reference path: DeviceScan<>::ExclusiveSum -> dispatch_scan (src/lcpp/device/device_scan.h:370-385,
// 868-948) -> ScanModule/build_scan (device/details/scan.h:241-335) with TilePrefixCallbackOp
// (device/details/single_pass_scan_operator.h:219-332) over packed (status, value) words
// (single_pass_scan_operator.h:119-172) and tile statuses INVALID / PARTIAL / INCLUSIVE (:26-32).
//
// MI355X design
//   * Tile = 256 threads x 24 rows x one 128-bit vector per thread per row (96 x 4-byte items per
//     thread, 24,576 items, held in registers).  Row r of a tile is the contiguous range
//     [r*1024, (r+1)*1024) and thread t holds items 4t..4t+3 of every row, so each row is one fully
//     coalesced 4 KiB load and store.
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
//   * Look-back: wave 0 publishes PARTIAL, then inspects 64 predecessors per step (one per lane)
//     with agent-scope loads, sums back to the nearest INCLUSIVE predecessor with a DPP reduction,
//     and publishes INCLUSIVE.  Status and value share one 64-bit word: flag in the low half,
//     value bits in the high half, so one relaxed atomic load observes both consistently.
// Algorithmic traffic: 2 * n * sizeof(T) bytes (read input, write output) + 8 bytes per tile.
#include "common.hpp"
#include "../../include/lcpp_hip.h"

namespace lcpp_hip {
namespace {

// 24 rows: 96 items per thread and 24,576 per tile (measured best on MI355X among 4K..48K-item tiles
// and 256..1024-thread workgroups).  Large tiles matter because a tile's look-back waits on its
// predecessors' publications; fewer, larger tiles shorten that chain relative to the data moved.
constexpr int kScanBlock = 256;
constexpr int kScanRows = 24;
constexpr int kScanWaves = kScanBlock / kWave;
constexpr uint32_t kScanTile = kScanBlock * kScanRows * 4;  // 24,576 items of 4 bytes

constexpr uint32_t kFlagInvalid = 0;
constexpr uint32_t kFlagPartial = 1;
constexpr uint32_t kFlagInclusive = 2;
constexpr uint32_t kFlagClaimed = 3;  // a look-back is computing this tile's aggregate

// Temp layout: one 8-byte status word per tile.
size_t scan_needed_bytes(uint64_t n) { return ceil_div(n, kScanTile) * 8; }


template <typename T>
__device__ __forceinline__ uint64_t pack_status(uint32_t flag, T value) {
    return (static_cast<uint64_t>(__builtin_bit_cast(uint32_t, value)) << 32) | flag;
}

// PARTIAL or INCLUSIVE: the word carries a usable value.
__device__ __forceinline__ bool status_published(uint64_t st) {
    return static_cast<uint32_t>(st) - kFlagPartial < 2u;
}

// Item `idx` of the input, or 0 past the end.
template <typename T>
__device__ __forceinline__ T load_item(const T* in, uint64_t n, uint64_t idx) {
    return idx < n ? in[idx] : T(0);
}

// Aggregate of (full) tile `tile`, computed by one wave in exactly the order its owner uses: per
// thread ((x0+x1)+x2)+x3, a DPP wave scan per (row, wave), wave totals summed per row in wave order,
// rows summed in row order.
template <typename T>
__device__ T tile_aggregate(const T* in, uint64_t n, uint32_t tile, int vector_io) {
    using Vec = T __attribute__((ext_vector_type(4)));
    const uint32_t lane = lane_id();
    const uint64_t tile_base = static_cast<uint64_t>(tile) * kScanTile;
    T running = T(0);
    for (int r = 0; r < kScanRows; ++r) {
        T row_total = T(0);
        for (int w = 0; w < kScanWaves; ++w) {
            const uint64_t first = tile_base + (static_cast<uint64_t>(r) * kScanBlock + w * kWave + lane) * 4;
            Vec v;
            if (vector_io && tile_base + kScanTile <= n) {
                v = *reinterpret_cast<const Vec*>(in + first);
            } else {
                v[0] = load_item(in, n, first);
                v[1] = load_item(in, n, first + 1);
                v[2] = load_item(in, n, first + 2);
                v[3] = load_item(in, n, first + 3);
            }
            v[1] += v[0];
            v[2] += v[1];
            v[3] += v[2];
            row_total += wave_read_lane(wave_inclusive_scan(v[3], SumOp{}), kWave - 1);
        }
        running += row_total;
    }
    return running;
}

// Exclusive prefix of tile `tile` (> 0) over all earlier tiles; called by all 64 lanes of one wave.
template <typename T>
__device__ T scan_lookback(uint64_t* states, uint32_t tile, const T* in, uint64_t n, int vector_io,
                           uint32_t spin_limit) {
    const uint32_t lane = lane_id();
    T prefix = T(0);
    int64_t end = tile;  // exclusive end of the window of predecessors
    while (true) {
        const int64_t idx = end - kWave + static_cast<int64_t>(lane);
        uint64_t st = idx >= 0 ? atomic_load_agent(&states[idx]) : pack_status(kFlagInclusive, T(0));
        uint32_t spins = 0;
        while (wave_ballot(!status_published(st)) != 0) {
            if (spins >= spin_limit) {
                // Fallback: claim every still-INVALID predecessor and compute its aggregate here.
                // Predecessors CLAIMED by another look-back are simply polled until published.
                uint64_t invalid = wave_ballot(static_cast<uint32_t>(st) == kFlagInvalid);
                while (invalid != 0) {
                    const uint32_t src = static_cast<uint32_t>(__builtin_ctzll(invalid));
                    invalid &= invalid - 1;
                    const uint32_t j = static_cast<uint32_t>(end - kWave + src);
                    bool won = false;
                    if (lane == src) {
                        uint64_t expected = 0;  // INVALID with value 0, as the clear leaves it
                        won = __hip_atomic_compare_exchange_strong(&states[j], &expected, uint64_t(kFlagClaimed),
                                                                   __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                                   __HIP_MEMORY_SCOPE_AGENT);
                        st = won ? uint64_t(kFlagClaimed) : expected;
                    }
                    if (wave_ballot(won) != 0) {
                        const T agg = tile_aggregate(in, n, j, vector_io);
                        if (lane == src) {
                            st = pack_status(kFlagPartial, agg);
                            atomic_store_agent(&states[j], st);
                        }
                    }
                }
            }
            __builtin_amdgcn_s_sleep(1);
            ++spins;
            if (!status_published(st)) st = atomic_load_agent(&states[idx]);
        }
        const T value = __builtin_bit_cast(T, static_cast<uint32_t>(st >> 32));
        const uint64_t inclusive = wave_ballot(static_cast<uint32_t>(st) == kFlagInclusive);
        if (inclusive != 0) {
            const uint32_t last = 63 - __builtin_clzll(inclusive);
            prefix += wave_reduce(lane >= last ? value : T(0), SumOp{});
            return prefix;
        }
        prefix += wave_reduce(value, SumOp{});
        end -= kWave;
    }
}

template <typename T, bool INCLUSIVE>
__global__ __launch_bounds__(kScanBlock, 2) void scan_sum_kernel(const T* in, T* out,
                                                              uint64_t n, uint64_t* __restrict__ states, T init,
                                                              int vector_io, uint32_t spin_limit) {
    using Vec = T __attribute__((ext_vector_type(4)));
    __shared__ T s_wave_totals[kScanRows][kScanWaves];
    __shared__ T s_tile_prefix;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint64_t tile_base = static_cast<uint64_t>(tile) * kScanTile;
    const bool full = vector_io && tile_base + kScanTile <= n;

    Vec v[kScanRows];
    if (full) {
        const Vec* src = reinterpret_cast<const Vec*>(in + tile_base);
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) v[r] = __builtin_nontemporal_load(&src[r * kScanBlock + tid]);
    } else {
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint64_t idx = tile_base + (static_cast<uint64_t>(r) * kScanBlock + tid) * 4 + j;
                v[r][j] = idx < n ? in[idx] : T(0);
            }
        }
    }

    // Thread-local inclusive scans and per-row wave scans.
    T wave_incl[kScanRows];
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
        v[r][1] += v[r][0];
        v[r][2] += v[r][1];
        v[r][3] += v[r][2];
        wave_incl[r] = wave_inclusive_scan(v[r][3], SumOp{});
    }
    if (lane == kWave - 1) {
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) s_wave_totals[r][wave] = wave_incl[r];
    }
    __syncthreads();

    // Exclusive in-tile offset of (row r, this wave) and the tile aggregate.
    T row_base[kScanRows];
    T running = T(0);
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
        T before = T(0);
        T row_total = T(0);
#pragma unroll
        for (int w = 0; w < kScanWaves; ++w) {
            const T x = s_wave_totals[r][w];
            if (w < static_cast<int>(wave)) before += x;
            row_total += x;
        }
        row_base[r] = running + before;
        running += row_total;
    }
    const T aggregate = running;

    // Publish (tile 0: INCLUSIVE at once; others PARTIAL, then INCLUSIVE after the look-back).  The
    // publication is a compare-and-swap from INVALID: if a look-back has CLAIMED this tile, the owner
    // waits for the claimer's PARTIAL (the claimer has finished reading this tile's input) before the
    // barrier that precedes every output store.
    if (wave == 0) {
        bool claimed_by_other = false;
        if (lane == 0) {
            uint64_t expected = 0;
            claimed_by_other = !__hip_atomic_compare_exchange_strong(
                &states[tile], &expected, pack_status(tile == 0 ? kFlagInclusive : kFlagPartial, aggregate),
                __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const T excl = tile == 0 ? T(0) : scan_lookback<T>(states, tile, in, n, vector_io, spin_limit);
        if (lane == 0) {
            if (claimed_by_other) {
                while (static_cast<uint32_t>(atomic_load_agent(&states[tile])) != kFlagPartial)
                    __builtin_amdgcn_s_sleep(1);
            }
            if (tile != 0 || claimed_by_other)
                atomic_store_agent(&states[tile], pack_status(kFlagInclusive, excl + aggregate));
            s_tile_prefix = excl;
        }
    }
    __syncthreads();
    const T tile_prefix = s_tile_prefix;

    const T base_all = init + tile_prefix;
#pragma unroll
    for (int r = 0; r < kScanRows; ++r) {
        const T thread_excl = wave_shift_exclusive<T, SumOp>(wave_incl[r]);
        const T p = base_all + row_base[r] + thread_excl;
        Vec o;
        if constexpr (INCLUSIVE) {
            // The last item's inclusive value comes from the wave scan, so v[r][3] need not stay live
            // (keeps the kernel within 256 VGPRs, two workgroups per CU).
            o[0] = p + v[r][0];
            o[1] = p + v[r][1];
            o[2] = p + v[r][2];
            o[3] = base_all + row_base[r] + wave_incl[r];
        } else {
            o[0] = p;
            o[1] = p + v[r][0];
            o[2] = p + v[r][1];
            o[3] = p + v[r][2];
        }
        v[r] = o;
    }
    if (full) {
        Vec* dst = reinterpret_cast<Vec*>(out + tile_base);
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) __builtin_nontemporal_store(v[r], &dst[r * kScanBlock + tid]);
    } else {
#pragma unroll
        for (int r = 0; r < kScanRows; ++r) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint64_t idx = tile_base + (static_cast<uint64_t>(r) * kScanBlock + tid) * 4 + j;
                if (idx < n) out[idx] = v[r][j];
            }
        }
    }
}

template <typename T>
int scan_sum(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, bool inclusive, T init,
             void* stream_ptr) {
    static_assert(sizeof(T) == 4, "packed tile status holds 4-byte values");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "DeviceScan: too many items (%llu > UINT_MAX)",
                                            static_cast<unsigned long long>(n));
    if (n == 0) return kOk;
    if (!in || !out) return set_error(kInvalidArgument, "DeviceScan: null input or output");
    if (reinterpret_cast<uintptr_t>(in) % sizeof(T) != 0 || reinterpret_cast<uintptr_t>(out) % sizeof(T) != 0)
        return set_error(kInvalidArgument, "DeviceScan: input/output not aligned to the element size");
    const size_t needed = scan_needed_bytes(n);
    if (!temp || temp_bytes < needed)
        return set_error(kTempTooSmall, "DeviceScan: temp storage too small (%zu < %zu bytes)", temp_bytes, needed);
    if (reinterpret_cast<uintptr_t>(temp) % 8 != 0)
        return set_error(kInvalidArgument, "DeviceScan: temp storage must be 8-byte aligned");

    const uint64_t tiles = ceil_div(n, kScanTile);
    uint64_t* states = static_cast<uint64_t*>(temp);
    int st = launch_fill_u32(static_cast<uint32_t*>(temp), needed / 4, 0u, stream);
    if (st != kOk) return st;

    const int vector_io = (reinterpret_cast<uintptr_t>(in) % 16 == 0) && (reinterpret_cast<uintptr_t>(out) % 16 == 0);
    LaunchScope scope("scan_sum", stream);
    if (inclusive)
        scan_sum_kernel<T, true><<<static_cast<unsigned>(tiles), kScanBlock, 0, stream>>>(in, out, n, states, init,
                                                                                         vector_io, g_lookback_spin_limit);
    else
        scan_sum_kernel<T, false><<<static_cast<unsigned>(tiles), kScanBlock, 0, stream>>>(in, out, n, states, init,
                                                                                          vector_io, g_lookback_spin_limit);
    return check_hip(hipGetLastError(), "scan_sum launch");
}

}  // namespace
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

size_t lcpp_hip_internal_scan_needed_bytes(uint64_t n) { return n == 0 ? 0 : scan_needed_bytes(n); }

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
#undef LCPP_HIP_DEFINE_SCAN

}  // extern "C"
