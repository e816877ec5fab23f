// Onesweep DeviceRadixSort for gfx950 (stable LSD, 8-bit digits).
//
// Reference path: DeviceRadixSort<>::SortKeys/SortPairs (src/lcpp/device/device_radix_sort.h:369-554)
// -> onesweep_radix_sort (:1018-1475): reset, all-pass histogram (device/details/radix_sort.h:51-79,
// agent/agent_radix_sort_histogram.h:32-198), exclusive sum of the bins (radix_sort.h:81-123), then per
// pass and portion a fused onesweep kernel (radix_sort.h:125-167, agent/agent_radix_sort_onesweep.h:
// 45-540): atomic tile ticket, load + twiddle, block rank by match-any (block/block_radix_rank.h:
// 207-486), PARTIAL publish, per-digit look-back, LDS scatter, global scatter.
//
// MI355X design
//   * Histogram: one read of the keys counts every pass's digits in LDS copies private to each bank
//     (see histogram_kernel); the bins are scanned once per sort.
//   * Onesweep tiles: 1024 threads x 18 keys (4-byte keys without values), 1024 x 9 (8-byte keys)
//     or 512 x 28 / 512 x 18 (4-byte keys with 4- / 8-byte values); two workgroups per CU (see
//     geometry_for).  Keys are loaded wave-striped (item k of lane l of wave w is
//     tile[w*64*ITEMS + k*64 + l]), so every load instruction is one coalesced access and each wave
//     ranks its keys in index order (stability).
//   * Rank: per wave and round, the 64-bit mask of lanes holding the same digit comes from an LDS
//     table of lane masks (every lane ORs its bit into its digit's entry and reads it back) or, as an
//     alternative, from 8 ballots; the rank is the wave's running count of the digit plus the
//     popcount of the mask below the lane, and the highest lane of each digit group advances the
//     count.  OR is order-independent, so ranks never depend on how conflicting lanes are serialised.
//   * Tile order: workgroup b is tile tile_of_block(b): 16 consecutive tiles per XCD at a time, so
//     the boundary cache lines of neighbouring tiles' digit runs merge in one L2 (groups of 8, 32 and 64
//     measured slower: longer groups make longer look-back chains between XCDs).  There is no tile
//     ticket (a same-address agent-scope atomic serialises at ~11 ns on MI355X).
//   * Look-back: per-digit counts go to a row of 256 32-bit words per tile: bits 31:30 hold the
//     status (1 PARTIAL, 2 INCLUSIVE), bits 29:0 the count, read and written with agent-scope atomics
//     because the 8 XCDs do not share an L2.  The four waves that own one digit per lane walk back
//     independently over windows of 8 or 16 predecessor tiles per step (lookback_digit), or, for
//     8-byte keys with values, every 256-thread group of the workgroup takes its own 2-tile window of
//     each step; an entry unpublished after a bounded spin is counted by the waiting wave or workgroup
//     from that tile's keys and published by compare-and-swap, so progress never depends on dispatch
//     order.
//   * Keys are reordered by digit in LDS (before the look-back) and written out from LDS in order, so
//     consecutive lanes write consecutive addresses inside each digit's run.  Pairs move values the
//     same way after the keys.
//   * Portions: one launch ranks at most 2^30 - tile keys so look-back counts fit in 30 bits.  The
//     upfront histogram gives each pass's global digit offsets for portion 0.  Within a pass, the
//     last tile of portion q holds the inclusive count of every digit in that portion and writes
//     portion q+1's offsets (offset + count); the next launch reads them.  (The reference intends the
//     same carry, but selects the writing block by `(block+1) * RADIX_DIGITS >= n`,
//     agent/agent_radix_sort_onesweep.h:362, so it never fires for large inputs.)
// Algorithmic traffic per pass: n * 2 * (sizeof(K) + sizeof(V)) bytes; the histogram reads n*sizeof(K).
#include "common.hpp"
#include "../../include/lcpp_hip.h"

#include <algorithm>

namespace lcpp_hip {
namespace radix {

constexpr uint32_t kDigits = 256;
constexpr uint32_t kFlagPartial = 1u << 30;
constexpr uint32_t kFlagInclusive = 2u << 30;
constexpr uint32_t kCountMask = (1u << 30) - 1;
constexpr uint32_t kMaxPasses = 8;
// In-wave ranking: the last `ballot_sixteenths` / 16 of a workgroup's waves match digits with ballots
// (VALU), the others with LDS lane-mask tables (LDS pipe); the test hook selects all-ballot (mode 0),
// all-table (mode 1) or the geometry's default split (mode 2, Geometry::ballot_sixteenths).
constexpr int kRankBallot = 0;
constexpr int kRankLdsMatch = 1;
constexpr int kRankMixed = 2;
constexpr uint32_t ballot_sixteenths_for(int mode, uint32_t mixed) {
    return mode == kRankBallot ? 16u : mode == kRankLdsMatch ? 0u : mixed;
}

#ifdef LCPP_HIP_PHASE_TRACE
// Phase-trace buffer of the diagnostic build: one record per (pass, tile), slot (shift / 8) * tiles + tile.
__device__ uint64_t* g_trace_buffer = nullptr;
__device__ uint64_t g_trace_records = 0;
#endif

enum KeyKind { kUnsigned = 0, kSigned = 1, kFloat = 2 };

template <typename K> struct KeyTraits;
template <> struct KeyTraits<uint32_t> { using U = uint32_t; static constexpr int kind = kUnsigned; };
template <> struct KeyTraits<int32_t> { using U = uint32_t; static constexpr int kind = kSigned; };
template <> struct KeyTraits<float> { using U = uint32_t; static constexpr int kind = kFloat; };
template <> struct KeyTraits<uint64_t> { using U = uint64_t; static constexpr int kind = kUnsigned; };
template <> struct KeyTraits<int64_t> { using U = uint64_t; static constexpr int kind = kSigned; };
template <> struct KeyTraits<double> { using U = uint64_t; static constexpr int kind = kFloat; };

template <int VB> struct ValueWord { using type = uint32_t; };
template <> struct ValueWord<8> { using type = uint64_t; };

// Bit-ordered transform (common/util_type.h:97-175 TwiddleIn/TwiddleOut; descending inverts,
// agent/radix_rank_sort_operations.h:123-155).
template <typename U, int KIND, bool DESC>
__device__ __forceinline__ U twiddle_in(U k) {
    constexpr U kHigh = U(1) << (sizeof(U) * 8 - 1);
    if constexpr (KIND == kSigned) k ^= kHigh;
    if constexpr (KIND == kFloat) k ^= (k & kHigh) ? U(~U(0)) : kHigh;
    if constexpr (DESC) k = ~k;
    return k;
}

template <typename U, int KIND, bool DESC>
__device__ __forceinline__ U twiddle_out(U k) {
    constexpr U kHigh = U(1) << (sizeof(U) * 8 - 1);
    if constexpr (DESC) k = ~k;
    if constexpr (KIND == kSigned) k ^= kHigh;
    if constexpr (KIND == kFloat) k ^= (k & kHigh) ? kHigh : U(~U(0));
    return k;
}

// Digit of a bit-ordered key.  For floats the ordered image of -0.0 is mapped to that of +0.0
// before extraction (ShiftDigitExtractor / ProcessFloatMinusZero,
// agent/radix_rank_sort_operations.h:31-62), so both zeros rank as equal keys.
template <typename U, int KIND>
__device__ __forceinline__ uint32_t digit_of(U ordered, uint32_t shift, uint32_t mask) {
    if constexpr (KIND == kFloat) {
        constexpr U kHigh = U(1) << (sizeof(U) * 8 - 1);
        if (ordered == U(~kHigh)) ordered = kHigh;
    }
    return static_cast<uint32_t>(ordered >> shift) & mask;
}

// The same digit from the bit count of the pass: one bit-field extract for 4-byte keys.
template <typename U, int KIND>
__device__ __forceinline__ uint32_t digit_bits(U ordered, uint32_t shift, uint32_t num_bits) {
    if constexpr (KIND == kFloat) {
        constexpr U kHigh = U(1) << (sizeof(U) * 8 - 1);
        if (ordered == U(~kHigh)) ordered = kHigh;
    }
    if constexpr (sizeof(U) == 4) return __builtin_amdgcn_ubfe(ordered, shift, num_bits);
    else return static_cast<uint32_t>(ordered >> shift) & ((1u << num_bits) - 1u);
}

// --------------------------------------------------------------------------------------------
// Histogram: digit counts of every pass for one portion.
//
// Random digits make the lanes of one ds_add collide on LDS banks, so the counters have 32 copies: lane l
// counts into copy l & 31, the word of (pass, digit, copy) sitting at bank (digit & 1) * 32 + copy of the
// 64, and the lanes of an instruction meet at most two to a bank whatever the digits are (skewed digits
// included).  4-byte keys: one 32-bit counter per digit and copy, 4 passes x 32 KB of LDS, one
// 1024-thread workgroup per CU.  8-byte keys: a word packs the 16-bit counters of an even/odd digit pair
// (8 passes x 16 KB; each counter stays below kHistMaxItems / 32 + a few head/tail keys < 2^16), which
// costs a multiply-add per key and pass more.  (SortKeys 2^28 u32: histogram 179 -> 168 us unpacked; two
// workgroups per CU of packed counters, or unpacked ones with 16 copies, 174-180 us; 64 copies or the
// next loads issued before the counting changed nothing.)
// --------------------------------------------------------------------------------------------
constexpr int kHistCopies = 32;
// One 32-bit counter per digit and copy (else 16-bit pairs).
template <typename U>
constexpr bool kHistWide = sizeof(U) == 4;
constexpr int kHistBlock = 1024;
constexpr int kHistVecItems = 8;  // 16-byte loads per thread per step (2^28 u32: 169 us with 4 or 8, 178 with 16)
constexpr uint32_t kHistMaxItems = 1u << 20;  // keys per workgroup

// FULL: every 8-bit digit of the key (begin_bit 0, end_bit = key bits), so digit positions are
// compile-time constants and each pass costs two bit-field extracts, one address and one increment.
template <typename K, bool DESC, bool FULL>
__global__ __launch_bounds__(kHistBlock) void histogram_kernel(const K* __restrict__ keys, uint32_t n,
                                                                uint32_t per_block, uint32_t* __restrict__ bins,
                                                                uint32_t begin_bit, uint32_t end_bit, uint32_t passes) {
    using U = typename KeyTraits<K>::U;
    constexpr int KIND = KeyTraits<K>::kind;
    constexpr int PASSES_MAX = sizeof(U);
    constexpr int PER_VEC = 16 / sizeof(U);  // keys per 16-byte load
    constexpr bool WIDE = kHistWide<U>;
    constexpr uint32_t PASS_WORDS = (WIDE ? kDigits : kDigits / 2) * kHistCopies;
    __shared__ uint32_t s_hist[PASSES_MAX * PASS_WORDS];
    if constexpr (FULL) passes = PASSES_MAX;
    for (uint32_t i = threadIdx.x; i < passes * PASS_WORDS; i += kHistBlock) s_hist[i] = 0;
    __syncthreads();

    const uint32_t copy = threadIdx.x % kHistCopies;
    const uint64_t first = static_cast<uint64_t>(blockIdx.x) * per_block;
    const uint64_t last = min(static_cast<uint64_t>(n), first + per_block);
    auto count = [&](U key) {
        U ordered = twiddle_in<U, KIND, DESC>(key);
        if constexpr (KIND == kFloat) {
            // -0.0 counts as +0.0 (digit_of applies the same mapping).
            constexpr U kHigh = U(1) << (sizeof(U) * 8 - 1);
            if (ordered == U(~kHigh)) ordered = kHigh;
        }
#pragma unroll
        for (uint32_t p = 0; p < PASSES_MAX; ++p) {
            uint32_t pair, odd;  // digit / 2 and digit % 2
            if constexpr (FULL) {
                pair = static_cast<uint32_t>(ordered >> (8 * p + 1)) & 0x7Fu;
                odd = static_cast<uint32_t>(ordered >> (8 * p)) & 1u;
            } else {
                if (p >= passes) break;
                const uint32_t shift = begin_bit + 8 * p;
                const uint32_t nb = min(8u, end_bit - shift);
                const uint32_t d = static_cast<uint32_t>(ordered >> shift) & ((1u << nb) - 1u);
                pair = d >> 1;
                odd = d & 1u;
            }
            if constexpr (WIDE)
                atomicAdd(&s_hist[p * PASS_WORDS + (2 * pair + odd) * kHistCopies + copy], 1u);
            else
                atomicAdd(&s_hist[p * PASS_WORDS + pair * kHistCopies + copy], 1u + odd * 0xFFFFu);
        }
    };
    const U* ukeys = reinterpret_cast<const U*>(keys);
    // Scalar head up to 16-byte alignment, vector body, scalar tail.
    const uint64_t misalign = (reinterpret_cast<uintptr_t>(ukeys + first) % 16) / sizeof(U);
    const uint64_t head_end = misalign ? min(last, first + (PER_VEC - misalign)) : first;
    for (uint64_t i = first + threadIdx.x; i < head_end; i += kHistBlock) count(ukeys[i]);
    using Vec = U __attribute__((ext_vector_type(PER_VEC)));
    constexpr uint64_t STEP = static_cast<uint64_t>(PER_VEC) * kHistVecItems * kHistBlock;
    const uint64_t body_items = (last - head_end) / STEP * STEP;
    const Vec* vkeys = reinterpret_cast<const Vec*>(ukeys + head_end);
    for (uint64_t v = 0; v < body_items / PER_VEC; v += static_cast<uint64_t>(kHistVecItems) * kHistBlock) {
        Vec k[kHistVecItems];
#pragma unroll
        for (int u = 0; u < kHistVecItems; ++u) k[u] = __builtin_nontemporal_load(&vkeys[v + u * kHistBlock + threadIdx.x]);
#pragma unroll
        for (int u = 0; u < kHistVecItems; ++u)
#pragma unroll
            for (int e = 0; e < PER_VEC; ++e) count(k[u][e]);
    }
    for (uint64_t i = head_end + body_items + threadIdx.x; i < last; i += kHistBlock) count(ukeys[i]);
    __syncthreads();

    // Sum the 32 copies of each (pass, digit); lanes start at different copies so the reads spread
    // over the banks.
    for (uint32_t i = threadIdx.x; i < passes * kDigits; i += kHistBlock) {
        const uint32_t p = i / kDigits, d = i % kDigits;
        uint32_t total = 0;
        if constexpr (WIDE) {
            const uint32_t* row = &s_hist[p * PASS_WORDS + d * kHistCopies];
            for (uint32_t c = 0; c < kHistCopies; ++c) total += row[(c + i) % kHistCopies];
        } else {
            const uint32_t* row = &s_hist[p * PASS_WORDS + (d >> 1) * kHistCopies];
            for (uint32_t c = 0; c < kHistCopies; ++c) total += (row[(c + i) % kHistCopies] >> ((d & 1u) * 16u)) & 0xFFFFu;
        }
        if (total) atomic_add_agent(&bins[p * kDigits + d], total);
    }
}

// In place: counts[p][d] -> exclusive scan over d, the first output position of digit d in pass p
// (device/details/radix_sort.h:81-123).
__global__ __launch_bounds__(kDigits) void bins_scan_kernel(uint32_t* __restrict__ bins, uint32_t passes) {
    __shared__ uint32_t s_wave_totals[kDigits / kWave];
    const uint32_t d = threadIdx.x;
    const uint32_t wave = d / kWave;
    for (uint32_t p = 0; p < passes; ++p) {
        const uint32_t count = bins[p * kDigits + d];
        const uint32_t incl = wave_inclusive_scan(count, SumOp{});
        if (lane_id() == kWave - 1) s_wave_totals[wave] = incl;
        __syncthreads();
        uint32_t run = incl - count;
        for (uint32_t w = 0; w < wave; ++w) run += s_wave_totals[w];
        bins[p * kDigits + d] = run;
        __syncthreads();
    }
}

// --------------------------------------------------------------------------------------------
// First-pass tile offsets without a look-back.
//
// The histogram reads every key anyway, so it can also count the first pass's digits per onesweep
// tile.  An exclusive scan of those counts over the tiles (per digit, plus the digit's base) gives
// every tile of the first pass its output offsets before that pass starts, so the pass skips its
// publish and look-back.  Used for single-portion sorts of 4-byte keys without values whose keys are
// 16-byte aligned, when the caller's temp storage has room for the per-workgroup totals.
// --------------------------------------------------------------------------------------------

// histogram_kernel plus the first pass's digit counts per TILE keys: tile_counts[t][d] for every tile
// of the slice, and the slice's totals in chunk_sums[blockIdx.x][d].  The slice starts on a tile
// boundary and holds whole tiles (the last slice may end in a partial one).  The first pass's
// counters are two buffers of bank-private copies: one counts a tile while the other, the previous
// tile's, is summed and cleared by 128 threads, so a tile costs one barrier.
template <typename K, bool DESC, bool FULL, uint32_t TILE>
// Two workgroups per CU for 4-byte keys (80 KB of LDS each, at most 64 VGPRs), one for 8-byte keys.
__global__ __launch_bounds__(kHistBlock, (sizeof(K) == 4 ? 8 : 4)) void histogram_tiles_kernel(const K* __restrict__ keys, uint32_t n,
                                                                      uint32_t per_block, uint32_t* __restrict__ bins,
                                                                      uint32_t begin_bit, uint32_t end_bit,
                                                                      uint32_t passes,
                                                                      uint32_t* __restrict__ tile_counts,
                                                                      uint32_t* __restrict__ chunk_sums) {
    using U = typename KeyTraits<K>::U;
    constexpr int KIND = KeyTraits<K>::kind;
    constexpr int PASSES_MAX = sizeof(U);
    constexpr int PER_VEC = 16 / sizeof(U);
    constexpr uint32_t PASS_WORDS = kDigits / 2 * kHistCopies;
    // A tile is TILE / PER_VEC 16-byte vectors: VECS loads per thread, the last of them by the first
    // LAST_THREADS threads only (all of them when the tile is whole 16-byte steps of the workgroup).
    static_assert(TILE % PER_VEC == 0, "a tile is whole 16-byte vectors");
    constexpr uint32_t TILE_VECS = TILE / PER_VEC;
    constexpr int VECS = static_cast<int>((TILE_VECS + kHistBlock - 1) / kHistBlock);
    constexpr uint32_t LAST_THREADS = TILE_VECS - static_cast<uint32_t>(VECS - 1) * kHistBlock;
    // Slots 0 and 1: the first pass's tile buffers; slot p + 1: pass p >= 1.
    __shared__ uint32_t s_hist[(PASSES_MAX + 1) * PASS_WORDS];
    if constexpr (FULL) passes = PASSES_MAX;
    for (uint32_t i = threadIdx.x; i < (passes + 1) * PASS_WORDS; i += kHistBlock) s_hist[i] = 0;
    __syncthreads();

    const uint32_t tid = threadIdx.x;
    const uint32_t copy = tid % kHistCopies;
    const uint64_t first = static_cast<uint64_t>(blockIdx.x) * per_block;
    const uint64_t last = min(static_cast<uint64_t>(n), first + per_block);
    auto count = [&](U key, uint32_t buf) {
        U ordered = twiddle_in<U, KIND, DESC>(key);
        if constexpr (KIND == kFloat) {
            constexpr U kHigh = U(1) << (sizeof(U) * 8 - 1);
            if (ordered == U(~kHigh)) ordered = kHigh;
        }
#pragma unroll
        for (uint32_t p = 0; p < PASSES_MAX; ++p) {
            uint32_t pair, odd;
            if constexpr (FULL) {
                pair = static_cast<uint32_t>(ordered >> (8 * p + 1)) & 0x7Fu;
                odd = static_cast<uint32_t>(ordered >> (8 * p)) & 1u;
            } else {
                if (p >= passes) break;
                const uint32_t shift = begin_bit + 8 * p;
                const uint32_t nb = min(8u, end_bit - shift);
                const uint32_t d = static_cast<uint32_t>(ordered >> shift) & ((1u << nb) - 1u);
                pair = d >> 1;
                odd = d & 1u;
            }
            // Pass 0 counts into this tile's buffer; pass p >= 1 at a fixed offset from the same base.
            uint32_t* const base = p == 0 ? s_hist + buf * PASS_WORDS + copy : s_hist + (p + 1) * PASS_WORDS + copy;
            atomicAdd(base + pair * kHistCopies, 1u + odd * 0xFFFFu);
        }
    };
    const U* ukeys = reinterpret_cast<const U*>(keys);
    using Vec = U __attribute__((ext_vector_type(PER_VEC)));
    uint32_t chunk_lo = 0, chunk_hi = 0;  // threads < 128: the slice's first-pass counts of digits 2 tid, 2 tid + 1
    const uint32_t tiles = static_cast<uint32_t>(ceil_div(last - first, TILE));
    const uint32_t full_tiles = static_cast<uint32_t>((last - first) / TILE);
    // Sums and clears buffer `buf` (tile t0) once every thread has counted it: thread w < 128 takes the
    // word of digits 2w and 2w + 1, starting at a different copy per lane so the reads spread over the
    // banks.  (The copy index rotates in the loop; precomputed, its 32 values would stay in registers.)
    auto flush = [&](uint32_t buf, uint64_t t0) {
        if (tid < kDigits / 2) {
            uint32_t* row = &s_hist[buf * PASS_WORDS + tid * kHistCopies];
            uint32_t lo = 0, hi = 0;
            uint32_t c = tid % kHistCopies;
#pragma unroll 4
            for (uint32_t k = 0; k < kHistCopies; ++k) {
                asm volatile("" : "+v"(c));
                const uint32_t x = row[c];
                lo += x & 0xFFFFu;
                hi += x >> 16;
                row[c] = 0;
                c = (c + 1) % kHistCopies;
            }
            uint32_t* out = tile_counts + (t0 / TILE) * kDigits + 2 * tid;
            out[0] = lo;
            out[1] = hi;
            chunk_lo += lo;
            chunk_hi += hi;
        }
    };
    // Full tiles, software-pipelined: the next tile's loads are issued before this tile is counted, so
    // they are in flight across the barrier and the flush.
    Vec k[VECS], next[VECS];
    if constexpr (LAST_THREADS < kHistBlock) {
#pragma unroll
        for (int e = 0; e < PER_VEC; ++e) next[VECS - 1][e] = U(0);  // not loaded by the other threads
    }
    if (full_tiles > 0) {
        const Vec* vkeys = reinterpret_cast<const Vec*>(ukeys + first);
#pragma unroll
        for (int u = 0; u < VECS; ++u)
            if (u + 1 < VECS || tid < LAST_THREADS) next[u] = __builtin_nontemporal_load(&vkeys[u * kHistBlock + tid]);
    }
    for (uint32_t j = 0; j < full_tiles; ++j) {
        const uint32_t buf = j & 1u;
        const uint64_t t0 = first + static_cast<uint64_t>(j) * TILE;
#pragma unroll
        for (int u = 0; u < VECS; ++u) k[u] = next[u];
        if (j + 1 < full_tiles) {
            const Vec* vkeys = reinterpret_cast<const Vec*>(ukeys + t0 + TILE);
#pragma unroll
            for (int u = 0; u < VECS; ++u)
                if (u + 1 < VECS || tid < LAST_THREADS) next[u] = __builtin_nontemporal_load(&vkeys[u * kHistBlock + tid]);
        }
#pragma unroll
        for (int u = 0; u < VECS; ++u)
            if (u + 1 < VECS || tid < LAST_THREADS) {
#pragma unroll
                for (int e = 0; e < PER_VEC; ++e) count(k[u][e], buf);
            }
        // Tile j is counted; the flush of buffer buf ^ 1 (tile j - 1) is finished.
        __syncthreads();
        flush(buf, t0);
    }
    if (full_tiles < tiles) {  // the slice's last, partial tile
        const uint32_t buf = full_tiles & 1u;
        const uint64_t t0 = first + static_cast<uint64_t>(full_tiles) * TILE;
        for (uint64_t i = t0 + tid; i < last; i += kHistBlock) count(ukeys[i], buf);
        __syncthreads();
        flush(buf, t0);
    }
    if (tid < kDigits / 2) {
        chunk_sums[static_cast<uint64_t>(blockIdx.x) * kDigits + 2 * tid] = chunk_lo;
        chunk_sums[static_cast<uint64_t>(blockIdx.x) * kDigits + 2 * tid + 1] = chunk_hi;
        if (chunk_lo) atomic_add_agent(&bins[2 * tid], chunk_lo);
        if (chunk_hi) atomic_add_agent(&bins[2 * tid + 1], chunk_hi);
    }
    // The other passes as in histogram_kernel.  (Their counting ended before the loop's last barrier.)
    for (uint32_t i = tid; i < (passes - 1) * kDigits; i += kHistBlock) {
        const uint32_t p = 1 + i / kDigits, d = i % kDigits;
        const uint32_t* row = &s_hist[(p + 1) * PASS_WORDS + (d >> 1) * kHistCopies];
        uint32_t total = 0;
        for (uint32_t c = 0; c < kHistCopies; ++c) total += (row[(c + i) % kHistCopies] >> ((d & 1u) * 16u)) & 0xFFFFu;
        if (total) atomic_add_agent(&bins[p * kDigits + d], total);
    }
}

// chunk_sums[c][d] -> the first output position of digit d's keys in chunk c's slice: the digit's base
// (bins[d], already scanned over the digits) plus the counts of the slices before c.  One workgroup per
// digit; thread t takes the consecutive chunks [t k, t k + k).
__global__ __launch_bounds__(kDigits) void chunk_scan_kernel(uint32_t* __restrict__ chunk_sums,
                                                             const uint32_t* __restrict__ bins, uint32_t chunks) {
    __shared__ uint32_t s_wave_totals[kDigits / kWave];
    const uint32_t d = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t per = (chunks + kDigits - 1) / kDigits;
    constexpr uint32_t kMaxPer = 8;  // chunks <= 2,048
    uint32_t v[kMaxPer];
    uint32_t sum = 0;
#pragma unroll
    for (uint32_t k = 0; k < kMaxPer; ++k) {
        const uint32_t c = tid * per + k;
        v[k] = (k < per && c < chunks) ? chunk_sums[static_cast<uint64_t>(c) * kDigits + d] : 0u;
        sum += v[k];
    }
    const uint32_t incl = wave_inclusive_scan(sum, SumOp{});
    const uint32_t wave = tid / kWave;
    if (lane_id() == kWave - 1) s_wave_totals[wave] = incl;
    __syncthreads();
    uint32_t run = bins[d] + incl - sum;
    for (uint32_t w = 0; w < wave; ++w) run += s_wave_totals[w];
#pragma unroll
    for (uint32_t k = 0; k < kMaxPer; ++k) {
        const uint32_t c = tid * per + k;
        if (k < per && c < chunks) chunk_sums[static_cast<uint64_t>(c) * kDigits + d] = run;
        run += v[k];
    }
}

// tile_counts[t][d] -> tile t's first output position for digit d: its chunk's position plus the
// counts of the chunk's tiles before t.  One workgroup per chunk, one thread per digit.
__global__ __launch_bounds__(kDigits) void tile_offsets_kernel(uint32_t* __restrict__ tile_counts,
                                                               const uint32_t* __restrict__ chunk_sums,
                                                               uint32_t tiles_per_chunk, uint32_t tiles) {
    const uint32_t d = threadIdx.x;
    const uint32_t t0 = blockIdx.x * tiles_per_chunk;
    const uint32_t t1 = min(tiles, t0 + tiles_per_chunk);
    uint32_t run = chunk_sums[static_cast<uint64_t>(blockIdx.x) * kDigits + d];
    constexpr uint32_t kBatch = 16;
    for (uint32_t t = t0; t < t1; t += kBatch) {
        uint32_t c[kBatch];
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) c[k] = t + k < t1 ? tile_counts[static_cast<uint64_t>(t + k) * kDigits + d] : 0u;
#pragma unroll
        for (uint32_t k = 0; k < kBatch; ++k) {
            if (t + k < t1) tile_counts[static_cast<uint64_t>(t + k) * kDigits + d] = run;
            run += c[k];
        }
    }
}

// --------------------------------------------------------------------------------------------
// Onesweep pass.
// --------------------------------------------------------------------------------------------

// Tile of a workgroup.  The dispatcher sends workgroup b to XCD b % 8 (measured), and tile t's digit
// runs end in the same cache lines where tile t + 1's begin.  So XCD x's j-th workgroup takes tile
// ((j / G) * 8 + x) * G + j % G: each XCD handles G consecutive tiles at a time, their shared boundary
// lines merge in that XCD's L2, and the write traffic of a pass drops (the scatter pattern alone runs
// 0.69 -> 0.52 ms at 2^28 with G = 16).  A full super-block of 8 G tiles is permuted; the remainder
// keeps its order, so the map is a bijection on [0, tiles).  Look-back stays deadlock-free: a tile
// waits only on tiles of lower index, which are dispatched no more than G - 1 steps later on the
// lower-numbered XCDs (and the look-back fallback computes any predecessor that stays unpublished).
constexpr uint32_t kXcds = 8;
constexpr uint32_t kXcdGroup = 16;

__device__ __forceinline__ uint32_t tile_of_block(uint32_t b, uint32_t tiles) {
    constexpr uint32_t kSuper = kXcds * kXcdGroup;
    if (b >= tiles / kSuper * kSuper) return b;
    const uint32_t x = b % kXcds, j = b / kXcds;
    return ((j / kXcdGroup) * kXcds + x) * kXcdGroup + j % kXcdGroup;
}

struct MinOpU32 {
    template <typename T>
    __device__ __forceinline__ T operator()(T a, T b) const { return a < b ? a : b; }
    template <typename T>
    __device__ __forceinline__ static constexpr T identity() { return ~T(0); }
};

// One look-back window of one wave.  Lane l (digit d) loads the entries of the WIN predecessor tiles
// top, top - 1, ..., top - WIN + 1 (`top` is wave-uniform; entries before tile 0 read as an empty
// INCLUSIVE entry, so a window that holds tile 0 always stops: tile 0 publishes INCLUSIVE at once) and
// returns the sum of their counts, newest first, down to and including the lane's nearest INCLUSIVE entry;
// `stop` says whether the window held one.  A window of PARTIAL entries only is summed with min / max /
// add alone (the status bits 01 of WIN words add up to a multiple of 2^32, as WIN is a multiple of 4).
// Lanes with `done` set load and wait for nothing.
//
// An entry still unpublished before the lane's nearest INCLUSIVE one is polled; after `spin_limit`
// polls the wave counts the digits of the newest such tile itself (its 64 digits d - l .. d - l + 63
// only, in the wave's 64 words of `s_fb`) and publishes them as PARTIAL by compare-and-swap, so progress
// never depends on dispatch order.  A predecessor tile is always full (only the last tile is partial).
template <typename K, bool DESC, int BLOCK, int ITEMS, int WIN>
__device__ __forceinline__ uint32_t lookback_window(uint32_t* __restrict__ lookback, int32_t top, uint32_t d, bool done,
                                                    bool& stop, const K* __restrict__ keys_in, uint32_t shift,
                                                    uint32_t mask, uint32_t spin_limit, uint32_t* s_fb,
                                                    uint32_t& spins_total, uint32_t& fallbacks) {
    static_assert(WIN % 4 == 0, "WIN * 2^30 must vanish modulo 2^32");
    using U = typename KeyTraits<K>::U;
    constexpr int KIND = KeyTraits<K>::kind;
    constexpr uint32_t TILE = static_cast<uint32_t>(BLOCK) * ITEMS;
    const uint32_t lane = lane_id();
    top = __builtin_amdgcn_readfirstlane(top);
    // The row addresses are recomputed at each load site rather than kept in registers across the
    // polling loop (an empty asm statement hides `top` from loop-invariant code motion).
    asm volatile("" : "+s"(top));
    uint32_t v[WIN];
#pragma unroll
    for (int w = 0; w < WIN; ++w) {
        v[w] = kFlagInclusive;  // entries before tile 0 stop the walk
        if (top >= w && !done) v[w] = atomic_load_agent(lookback + static_cast<uint64_t>(top - w) * kDigits + d);
    }
    uint32_t spins = 0;
    uint32_t sum = 0;
    stop = false;
    while (true) {
        uint32_t lo = v[0], hi = v[0], all = 0;
#pragma unroll
        for (int w = 0; w < WIN; ++w) {
            lo = min(lo, v[w]);
            hi = max(hi, v[w]);
            all += v[w];
        }
        bool wait = false;
        uint32_t first_wait = ~0u;
        if (lo >= kFlagPartial && hi < kFlagInclusive) {
            sum = all;
            stop = false;
        } else {
            sum = 0;
            stop = false;
#pragma unroll
            for (int w = 0; w < WIN; ++w) {
                if (!stop && !wait) {
                    if ((v[w] & ~kCountMask) == 0) {
                        wait = true;
                        first_wait = static_cast<uint32_t>(w);
                    } else {
                        sum += v[w] & kCountMask;
                        stop = (v[w] & kFlagInclusive) != 0;
                    }
                }
            }
        }
        wait = wait && !done;
        if (wave_ballot(wait) == 0) break;
        if (spins >= spin_limit) {
            // Count the newest tile some lane waits for and publish this wave's 64 digits of it (a
            // compare-and-swap from 0 that loses to the owner's own publication changes nothing); the
            // reload below then reads it.
            if constexpr (kPhaseTrace) ++fallbacks;
            const uint32_t wf = wave_reduce(wait ? first_wait : ~0u, MinOpU32{});
            const uint64_t jf = static_cast<uint32_t>(top) - wf;
            const uint32_t d0 = d - lane;
            __hip_atomic_store(&s_fb[lane], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            const U* ukeys = reinterpret_cast<const U*>(keys_in) + jf * TILE;
            for (uint32_t i = lane; i < TILE; i += kWave) {
                const uint32_t dk = digit_of<U, KIND>(twiddle_in<U, KIND, DESC>(ukeys[i]), shift, mask) - d0;
                if (dk < kWave) __hip_atomic_fetch_add(&s_fb[dk], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            }
            __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
            const uint32_t cnt = __hip_atomic_load(&s_fb[lane], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            uint32_t expected = 0;
            __hip_atomic_compare_exchange_strong(lookback + jf * kDigits + d, &expected, kFlagPartial | cnt,
                                                 __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            __builtin_amdgcn_s_sleep(1);
            ++spins;
            if constexpr (kPhaseTrace) ++spins_total;
        }
        asm volatile("" : "+s"(top));
#pragma unroll
        for (int w = 0; w < WIN; ++w) {
            if (top >= w && wait && (v[w] & ~kCountMask) == 0)
                v[w] = atomic_load_agent(lookback + static_cast<uint64_t>(top - w) * kDigits + d);
        }
    }
    return done ? 0u : sum;
}

// Look-back of one wave.  Lane l owns digit d = 64 w + l (w = the wave, one of the four waves that hold
// the 256 digits) and returns the number of keys with digit d in the tiles before `tile` of this
// portion: the counts the predecessors published for d, newest first, down to and including the
// nearest INCLUSIVE entry.  Each step is one window of WIN consecutive predecessors (one cross-XCD
// round trip); waves walk independently, with no barrier.
template <typename K, bool DESC, int BLOCK, int ITEMS, int WIN>
__device__ __forceinline__ uint32_t lookback_digit(uint32_t* __restrict__ lookback, uint32_t tile, uint32_t d,
                                                   const K* __restrict__ keys_in, uint32_t shift, uint32_t mask,
                                                   uint32_t spin_limit, uint32_t* s_fb, uint32_t& steps,
                                                   uint32_t& spins_total, uint32_t& fallbacks) {
    uint32_t excl = 0;
    bool done = false;
    // Newest predecessor of the window.  It never goes below 0: the window holding tile 0 ends every walk.
    int32_t top = static_cast<int32_t>(tile) - 1;
    while (true) {
        bool stop;
        excl += lookback_window<K, DESC, BLOCK, ITEMS, WIN>(lookback, top, d, done, stop, keys_in, shift, mask,
                                                            spin_limit, s_fb, spins_total, fallbacks);
        done = done || stop;
        if constexpr (kPhaseTrace) ++steps;
        if (wave_ballot(!done) == 0) break;
        top -= WIN;  // some lane has not reached an INCLUSIVE entry, so the window held no tile 0
    }
    return excl;
}

// Digit counts of one predecessor tile (always a full tile), by the whole workgroup, into counts[256].
template <typename K, bool DESC, int BLOCK, int ITEMS>
__device__ void count_tile_digits(const K* __restrict__ keys, uint32_t tile, uint32_t shift, uint32_t mask,
                                  uint32_t* counts) {
    using U = typename KeyTraits<K>::U;
    constexpr int KIND = KeyTraits<K>::kind;
    constexpr uint32_t TILE = static_cast<uint32_t>(BLOCK) * ITEMS;
    for (uint32_t i = threadIdx.x; i < kDigits; i += BLOCK) counts[i] = 0;
    __syncthreads();
    const U* ukeys = reinterpret_cast<const U*>(keys) + static_cast<uint64_t>(tile) * TILE;
    for (uint32_t i = threadIdx.x; i < TILE; i += BLOCK)
        atomicAdd(&counts[digit_of<U, KIND>(twiddle_in<U, KIND, DESC>(ukeys[i]), shift, mask)], 1u);
    __syncthreads();
}

template <typename K, bool DESC, int VB, int BLOCK, int ITEMS, int WINDOW, bool GROUPED>
// Register budget for two workgroups per CU: BLOCK / 128 waves per SIMD (128 VGPRs at 512 threads,
// 64 at 1024).
__global__ __launch_bounds__(BLOCK, BLOCK / 128) void onesweep_kernel(const K* __restrict__ keys_in,
                                                                               K* __restrict__ keys_out,
                                                         const void* __restrict__ values_in,
                                                         void* __restrict__ values_out, uint32_t n,
                                                         const uint32_t* __restrict__ digit_offsets,
                                                         uint32_t* __restrict__ next_offsets,
                                                         uint32_t* __restrict__ lookback,
                                                         const uint32_t* __restrict__ tile_offsets,
                                                         uint32_t* __restrict__ clear_rows, uint32_t clear_words,
                                                         uint32_t shift, uint32_t num_bits, uint32_t out_items,
                                                         uint32_t spin_limit, uint32_t ballot_sixteenths) {
    using U = typename KeyTraits<K>::U;
    using VW = typename ValueWord<VB>::type;
    constexpr int KIND = KeyTraits<K>::kind;
    constexpr int W = BLOCK / kWave;
    constexpr uint32_t TILE = static_cast<uint32_t>(BLOCK) * ITEMS;
    constexpr size_t ELEM = (VB > static_cast<int>(sizeof(U))) ? VB : sizeof(U);
    static_assert(BLOCK >= static_cast<int>(kDigits) && BLOCK % static_cast<int>(kDigits) == 0,
                  "one thread per digit");

    // The tile buffer first holds, per wave, the lane-mask table of the LDS ranker (256 x 8 B) and the
    // digit-count row (256 x 4 B; running counts during the rank, then the wave's offsets inside the
    // tile).  Once every thread has read its offsets back (a barrier), the buffer holds the keys
    // reordered by digit, and after the key scatter the values.
    static_assert(W * kDigits * (sizeof(uint64_t) + sizeof(uint32_t)) <= TILE * ELEM,
                  "rank tables and count rows must fit the tile buffer");
    __shared__ __attribute__((aligned(16))) unsigned char s_tile[TILE * ELEM];
    // Each digit's global-minus-local output offset.  Before a look-back wave writes its 64 entries,
    // they are its scratch for the look-back fallback.
    __shared__ uint32_t s_global_minus_local[kDigits];
    __shared__ uint32_t s_scan[kDigits / kWave];
    // Grouped look-back only: window sums of groups 1 .. and the digits' done flags, the fallback's tile.
    constexpr int LB_GROUPS = BLOCK / static_cast<int>(kDigits);
    static_assert(!GROUPED || LB_GROUPS > 1, "the grouped look-back needs at least two groups");
    __shared__ uint32_t s_lb[GROUPED ? LB_GROUPS : 1][kDigits];
    __shared__ uint32_t s_lb_tile;
    uint64_t (*s_match)[kDigits] = reinterpret_cast<uint64_t (*)[kDigits]>(s_tile);
    uint32_t (*s_counts)[kDigits] =
        reinterpret_cast<uint32_t (*)[kDigits]>(s_tile + W * kDigits * sizeof(uint64_t));

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t mask = (1u << num_bits) - 1u;
    PhaseClock clk;
    clk.start();
    uint32_t trace_steps = 0, trace_spins = 0, trace_fallbacks = 0;

    // Wave-private tables: no barrier needed before the wave uses them.
#pragma unroll
    for (uint32_t i = lane; i < kDigits; i += kWave) {
        s_counts[wave][i] = 0;
        s_match[wave][i] = 0;
    }
    const uint32_t tile = tile_of_block(blockIdx.x, gridDim.x);
    const uint32_t tile_base = tile * TILE;
    const uint32_t valid = min(TILE, n - tile_base);
    // With precomputed first-pass offsets (tile_offsets[tile][d]: the tile's first output position of
    // digit d), the tile neither publishes nor looks back; the offset is read now, behind the rank.
    const bool precomputed = tile_offsets != nullptr;
    const uint32_t tile_offset = (precomputed && tid < kDigits) ? tile_offsets[tile * kDigits + tid] : 0u;

    // Load (wave-striped) and twiddle; missing items become all-ones keys, which rank last.
    const U* ukeys = reinterpret_cast<const U*>(keys_in) + tile_base;
    const uint32_t wave_off = wave * kWave * ITEMS + lane;
    U keys[ITEMS];
    if (valid == TILE) {
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) keys[k] = twiddle_in<U, KIND, DESC>(__builtin_nontemporal_load(&ukeys[wave_off + k * kWave]));
    } else {
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const uint32_t i = wave_off + k * kWave;
            keys[k] = i < valid ? twiddle_in<U, KIND, DESC>(ukeys[i]) : U(~U(0));
        }
    }
    VW vals[VB ? ITEMS : 1];
    if constexpr (VB != 0) {
        const VW* uvals = reinterpret_cast<const VW*>(values_in) + tile_base;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const uint32_t i = wave_off + k * kWave;
            vals[k] = i < valid ? __builtin_nontemporal_load(&uvals[i]) : VW(0);
        }
    }

    // Zero the next launch's look-back rows (the other of the two regions, which the previous launch
    // used and no launch reads until the next one): a grid-stride sweep of 16-byte stores, behind the
    // loads.  This replaces a fill kernel before every launch.
    if (clear_rows != nullptr) {
        uint4* rows = reinterpret_cast<uint4*>(clear_rows);
        const uint32_t vecs = clear_words / 4;
        for (uint32_t i = blockIdx.x * BLOCK + tid; i < vecs; i += gridDim.x * BLOCK) rows[i] = make_uint4(0, 0, 0, 0);
    }

    clk.mark<1>(true);  // keys loaded

    // Rank inside the wave: rank = keys of the same digit in earlier rounds (the wave's LDS counter)
    // + lanes of the same digit below this lane in this round.  The highest such lane advances the
    // counter.  The peer mask comes from 8 ballots (ballot waves) or from an LDS table of 64-bit lane
    // masks, one per digit (table waves): every lane ORs its bit into its half-wave's 32-bit word of its
    // digit's entry (one bank per lane rather than two: SortKeys 2^28 u32 2.203 -> 2.182 ms against a
    // 64-bit OR), reads the whole entry back (all ORs of the instruction have landed: a wave's LDS
    // operations complete in issue order), and the highest peer clears it.  OR is order-independent, so
    // the mask does not depend on how the hardware serialises conflicting lanes.
    uint32_t rank[ITEMS];
    // Mixed ranking splits the work between the LDS pipe (tables) and the VALU (ballots); the choice is
    // per wave, so the branch is uniform.
    // The ballot waves are the last ones: waves 0..3 publish and walk the look-back after the rank, so
    // they take the faster table ranking.
    const bool table_rank = (W - 1 - __builtin_amdgcn_readfirstlane(wave)) * 16 >= ballot_sixteenths * W;
    if (table_rank) {
        const uint32_t half_bit = 1u << (lane & 31u);
        const uint32_t half = lane >> 5;
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const uint32_t d = digit_bits<U, KIND>(keys[k], shift, num_bits);
            uint64_t* slot = &s_match[wave][d];
            __hip_atomic_fetch_or(reinterpret_cast<uint32_t*>(slot) + half, half_bit, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_WORKGROUP);
            __builtin_amdgcn_wave_barrier();
            const uint64_t peers = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            const uint32_t base = s_counts[wave][d];
            const uint32_t below = popc_lanes_below(peers);
            rank[k] = base + below;
            __builtin_amdgcn_wave_barrier();
            if ((peers >> lane) == 1ull) {
                s_counts[wave][d] = base + below + 1;
                __hip_atomic_store(slot, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            __builtin_amdgcn_wave_barrier();
        }
    } else {
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) {
            const uint32_t d = digit_bits<U, KIND>(keys[k], shift, num_bits);
            const uint64_t peers = match_digit(d);
            const uint32_t below = popc_lanes_below(peers);
            const uint32_t base = s_counts[wave][d];
            rank[k] = base + below;
            if ((peers >> lane) == 1ull) s_counts[wave][d] = base + below + 1;
        }
    }
    __syncthreads();
    clk.mark<2>();  // every wave ranked

    // Per digit: wave offsets, tile count, PARTIAL publish, tile-local start.
    uint32_t count = 0, local_start = 0;
    if (tid < kDigits) {
        const uint32_t d = tid;
        uint32_t run = 0;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const uint32_t c = s_counts[w][d];
            s_counts[w][d] = run;
            run += c;
        }
        count = run;
        const uint32_t real = (d == mask) ? count - (TILE - valid) : count;  // missing items excluded
        if (!precomputed)
            atomic_store_agent(&lookback[tile * kDigits + d], (tile == 0 ? kFlagInclusive : kFlagPartial) | real);
        const uint32_t incl = wave_inclusive_scan(count, SumOp{});
        if (lane == kWave - 1) s_scan[wave] = incl;
        local_start = incl - count;
    }
    __syncthreads();
    const uint32_t d = tid;  // digit owned by this thread (threads >= 256 own none)
    const uint32_t real = (tid < kDigits) ? ((d == mask) ? count - (TILE - valid) : count) : 0;
    if (tid < kDigits) {
        for (uint32_t w = 0; w < wave; ++w) local_start += s_scan[w];
#pragma unroll
        for (int w = 0; w < W; ++w) s_counts[w][d] += local_start;
    }
    __syncthreads();
    clk.mark<3>();  // PARTIAL published, tile offsets scanned

    // Reorder keys by digit in LDS now: local positions do not depend on the look-back, and the key
    // registers are free while the look-back runs.  The offsets are read first: their rows share
    // the buffer the keys go to.
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) rank[k] += s_counts[wave][digit_bits<U, KIND>(keys[k], shift, num_bits)];
    __syncthreads();
    U* s_keys = reinterpret_cast<U*>(s_tile);
#pragma unroll
    for (int k = 0; k < ITEMS; ++k) s_keys[rank[k]] = keys[k];
    clk.mark<4>();  // keys reordered in LDS (this wave)

    // Look-back: either the four waves that hold one digit per lane walk independently (lookback_digit;
    // the other waves go straight to the barrier below) or the whole workgroup walks, in LB_GROUPS groups
    // of four waves, workgroup-synchronous (written out here: as a separate inlined function the same
    // steps measured 2 % slower on SortPairs 2^27).
    //
    // Grouped look-back.  Thread t takes digit t % 256 in group g = t / 256.  Each step covers LB_GROUPS *
    // WINDOW predecessors: group g loads the WINDOW tiles just older than group g - 1's, so every thread
    // holds WINDOW entries and all of a step's loads are in flight together (one cross-XCD round trip per
    // step).  The workgroup polls until no thread waits for an unpublished entry before its window's
    // nearest INCLUSIVE one (entries past it may stay unpublished; older tiles publish without waiting on
    // this one); each group sums its window down to that entry, and group 0 chains the sums, newest
    // window first, up to a window that stopped.  An entry still unpublished after `spin_limit` polls is
    // counted by the workgroup from its tile's keys (the newest such tile of any thread) and published as
    // PARTIAL by compare-and-swap.  s_lb rows 0 .. LB_GROUPS - 2 carry the window sums of groups 1 ..
    // (bit 31: the window stopped), row LB_GROUPS - 1 the digits' done flags.
    uint32_t excl = 0;
    if constexpr (GROUPED) {
        if (!precomputed && tile > 0) {
            const uint32_t grp = tid / kDigits;
            const uint32_t ld = tid % kDigits;  // look-back digit of this thread
            bool done = false;                  // the same in every group: group 0 decides
            int64_t top = static_cast<int64_t>(tile) - 1;  // newest predecessor not yet consumed
            uint32_t* const column = lookback + ld;
            while (true) {
                const int64_t gtop = top - static_cast<int64_t>(grp) * WINDOW;  // this group's newest
                uint32_t v[WINDOW];
#pragma unroll
                for (int w = 0; w < WINDOW; ++w) {
                    const int64_t j = gtop - w;
                    v[w] = (!done && j >= 0) ? atomic_load_agent(&column[static_cast<uint64_t>(j) * kDigits]) : 0u;
                }
                uint32_t spins = 0;
                while (true) {
                    // Newest unpublished entry of the window before its nearest INCLUSIVE one (and not
                    // past tile 0).
                    int waiting = -1;
                    bool scanning = !done;
#pragma unroll
                    for (int w = 0; w < WINDOW; ++w) {
                        const bool live = scanning && gtop - w >= 0;
                        if (live && (v[w] & ~kCountMask) == 0) waiting = w;
                        scanning = live && (v[w] & ~kCountMask) != 0 && (v[w] & kFlagInclusive) == 0;
                    }
                    if (!__syncthreads_or(waiting >= 0)) break;
                    if (spins >= spin_limit) {
                        if constexpr (kPhaseTrace) ++trace_fallbacks;
                        if (tid == 0) s_lb_tile = 0;
                        __syncthreads();
                        if (waiting >= 0) atomicMax(&s_lb_tile, static_cast<uint32_t>(gtop - waiting) + 1u);
                        __syncthreads();
                        const uint32_t jf = s_lb_tile - 1u;
                        count_tile_digits<K, DESC, BLOCK, ITEMS>(keys_in, jf, shift, mask, s_global_minus_local);
                        const int wf = static_cast<int>(gtop - static_cast<int64_t>(jf));
                        if (!done) {
#pragma unroll
                            for (int w = 0; w < WINDOW; ++w) {
                                if (w == wf && (v[w] & ~kCountMask) == 0) {
                                    // A compare-and-swap from 0 that loses to the owner's publication reads it.
                                    uint32_t expected = 0;
                                    const uint32_t desired = kFlagPartial | s_global_minus_local[ld];
                                    v[w] = __hip_atomic_compare_exchange_strong(
                                               &column[static_cast<uint64_t>(jf) * kDigits], &expected, desired,
                                               __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                               ? desired
                                               : expected;
                                }
                            }
                        }
                        continue;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    ++spins;
                    if constexpr (kPhaseTrace) ++trace_spins;
                    if (!done) {
#pragma unroll
                        for (int w = 0; w < WINDOW; ++w) {
                            const int64_t j = gtop - w;
                            if (j >= 0 && (v[w] & ~kCountMask) == 0)
                                v[w] = atomic_load_agent(&column[static_cast<uint64_t>(j) * kDigits]);
                        }
                    }
                }
                // The window's sum down to and including its nearest INCLUSIVE entry (tile 0's is INCLUSIVE).
                uint32_t window_sum = 0;
                bool window_stops = false;
                if (!done) {
#pragma unroll
                    for (int w = 0; w < WINDOW; ++w) {
                        if (!window_stops && gtop - w >= 0) {
                            window_sum += v[w] & kCountMask;
                            if ((v[w] & kFlagInclusive) || gtop - w == 0) window_stops = true;
                        }
                    }
                }
                if (grp > 0) s_lb[grp - 1][ld] = window_sum | (window_stops ? 0x80000000u : 0u);
                __syncthreads();
                if (grp == 0 && !done) {
#pragma unroll
                    for (int g = 1; g < LB_GROUPS; ++g) {
                        if (window_stops) break;
                        const uint32_t x = s_lb[g - 1][ld];
                        window_sum += x & 0x7FFFFFFFu;
                        window_stops = (x >> 31) != 0;
                    }
                    excl += window_sum;
                    done = window_stops;
                    s_lb[LB_GROUPS - 1][ld] = done ? 1u : 0u;
                }
                if constexpr (kPhaseTrace) ++trace_steps;
                const bool more = __syncthreads_or(grp == 0 && !done);
                if (grp > 0) done = s_lb[LB_GROUPS - 1][ld] != 0;
                if (!more) break;
                top -= static_cast<int64_t>(LB_GROUPS) * WINDOW;
            }
            clk.mark<5>();  // look-back walked (wave 0)
            if (tid < kDigits) atomic_store_agent(&lookback[tile * kDigits + d], kFlagInclusive | (excl + real));
        }
    } else if (!precomputed && tile > 0 && tid < kDigits) {
        excl = lookback_digit<K, DESC, BLOCK, ITEMS, WINDOW>(lookback, tile, d, keys_in, shift, mask, spin_limit,
                                                             &s_global_minus_local[wave * kWave], trace_steps,
                                                             trace_spins, trace_fallbacks);
        clk.mark<5>();  // look-back walked (wave 0)
        atomic_store_agent(&lookback[tile * kDigits + d], kFlagInclusive | (excl + real));
    }
    if (tid < kDigits) {
        const uint32_t base = digit_offsets[d];
        // Carry to the next portion of this pass: first position of digit d after this portion.
        if (next_offsets != nullptr && tile == gridDim.x - 1) next_offsets[d] = base + excl + real;
        s_global_minus_local[d] = (precomputed ? tile_offset : base + excl) - local_start;
    }
    __syncthreads();
    clk.mark<6>();  // global offsets known

    // Scatter from LDS in digit order.  Full tiles (all but the last) take a branch-free path, so the
    // reads of all ITEMS keys and offsets are in flight together; the clamp to the output keeps every
    // store in bounds whatever the offsets (a correct sort never needs it).
    U* ukeys_out = reinterpret_cast<U*>(keys_out);
    uint32_t gpos[VB ? ITEMS : 1];
    if (valid == TILE) {
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const uint32_t i = tid + j * BLOCK;
            const U key = s_keys[i];
            const uint32_t g = min(s_global_minus_local[digit_bits<U, KIND>(key, shift, num_bits)] + i, out_items - 1u);
            ukeys_out[g] = twiddle_out<U, KIND, DESC>(key);
            if constexpr (VB != 0) gpos[j] = g;
        }
    } else {
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const uint32_t i = tid + j * BLOCK;
            if (i < valid) {
                const U key = s_keys[i];
                const uint32_t g = s_global_minus_local[digit_bits<U, KIND>(key, shift, num_bits)] + i;
                if (g < out_items) ukeys_out[g] = twiddle_out<U, KIND, DESC>(key);  // always true for a correct sort
                if constexpr (VB != 0) gpos[j] = g;
            }
        }
    }

    if constexpr (VB != 0) {
        __syncthreads();
        VW* s_vals = reinterpret_cast<VW*>(s_tile);
#pragma unroll
        for (int k = 0; k < ITEMS; ++k) s_vals[rank[k]] = vals[k];
        __syncthreads();
        VW* uvals_out = reinterpret_cast<VW*>(values_out);
        if (valid == TILE) {
#pragma unroll
            for (int j = 0; j < ITEMS; ++j) uvals_out[gpos[j]] = s_vals[tid + j * BLOCK];
        } else {
#pragma unroll
            for (int j = 0; j < ITEMS; ++j) {
                const uint32_t i = tid + j * BLOCK;
                if (i < valid && gpos[j] < out_items) uvals_out[gpos[j]] = s_vals[i];
            }
        }
    }
#ifdef LCPP_HIP_PHASE_TRACE
    clk.mark<7>();  // scatter stores issued (this wave)
    if (tid == 0)
        clk.write(g_trace_buffer, g_trace_records, static_cast<uint64_t>(shift / 8) * gridDim.x + tile,
                  trace_steps | (static_cast<uint64_t>(trace_spins) << 16) |
                      (static_cast<uint64_t>(trace_fallbacks) << 32));
#endif
}

// --------------------------------------------------------------------------------------------
// Host orchestration.
// --------------------------------------------------------------------------------------------
struct Geometry {
    int block;
    int items;
    int window;    // predecessor tiles per 256-thread group and look-back step
    bool grouped;  // look-back by the whole workgroup (lookback_groups) rather than the four digit waves
    uint32_t ballot_sixteenths;  // waves ranked by ballots, in sixteenths of the workgroup (default mode)
    constexpr uint32_t tile() const { return static_cast<uint32_t>(block) * items; }
};

// Tiles are as large as two workgroups per CU allow (the reordering buffer holds the tile's widest
// items: at most 77 KB of LDS each out of the CU's 160 KB, within the register budget of
// __launch_bounds__): the look-back (one cross-XCD round trip per step), the publish and the digit scan
// cost the same per tile whatever its length, so fewer, longer tiles spread them over more keys.
//   * 4-byte keys without values: 1024 x 18 (SortKeys 2^28 u32 with the first pass looking back: 2.317 ms
//     with 16 keys per thread, 2.215 with 18, 2.219 with 19, whose 64 VGPRs spill; 20 would leave one
//     workgroup per CU, and one workgroup per CU measured 2.49-2.50 ms per sort with 1024 x 32 or
//     1024 x 36 tiles against 2.01 ms at 1024 x 18: a second workgroup's scatter no longer overlaps
//     each rank; four 512 x 18 or 512 x 19 workgroups per CU: 2.49-2.57 ms).  1024-thread workgroups (32 waves per CU, 64 VGPRs) beat 512 threads with twice
//     the items per thread: every wave's rank is a chain of dependent LDS round trips, and shorter chains
//     on more waves hide them better (SortKeys 2^28 u32 3.04 -> 2.81 ms when measured).
//   * 8-byte keys: 1024 x 9 (SortKeys 2^27 u64 4.52 -> 4.31 ms, SortPairs 2^27 u64 + u32 5.98 -> 5.92 ms
//     against 1024 x 8).
//   * 4-byte keys with 4-byte values: 512 x 28, 128 VGPRs (SortPairs 2^27 u32 + u32: 2.42 ms at
//     512 x 16, 2.21 at 512 x 24, 2.14 at 512 x 28; 768 x 16 spills); with 8-byte values 512 x 18, whose
//     72 KB of values fit beside the other workgroup's (SortPairs 2^27 u32 + u64: 3.36 -> 3.28 ms).
// Look-back: the four digit waves walk windows of WINDOW tiles independently, except for 8-byte keys
// with values, whose tiles are the shortest and whose registers are tighter: there the whole workgroup
// walks, four groups of WINDOW-tile windows per step, and every wave ranks by ballots.  Short windows
// win: a step waits for every unpublished entry of its window up to the nearest INCLUSIVE one, so a
// long window waits on predecessors that a shorter first step would not have needed, and it loads more
// rows per step.  SortKeys 2^28 u32 (digit waves): 2.06 ms with 4-tile windows, 2.05 with 8, 2.08 with
// 12, 2.09 with 16, 2.17-2.20 with 32 (20 and 24 spill).  SortKeys 2^27 u64: 4.17 ms with 8, 4.15 with
// 16, 4.33 with 32.  SortPairs 2^27 u32 + u32: 2.03 ms with 8, 2.07 with 16, 2.13 with 32; u32 + u64:
// 3.12 with 8, 3.28 with 32.  SortPairs 2^27 u64 + u32 uniform / AND-of-3 keys (grouped): 6.17 / 6.02
// ms with 1-tile windows per group, 5.83 / 5.48 with 2, 5.93 / 5.58 with 3 or 4, 6.15 / 5.82 with 6
// (at 8 pairs per thread: digit waves with 12-tile windows and a quarter of the waves on ballots 6.19 /
// 5.82 ms, grouped 4-tile windows with ballots only 6.01 / 5.64).  The grouped walk measured slower for
// 8-byte keys without values (SortKeys 2^27 u64 4.61 against 4.51 ms), for 4-byte keys with values
// (SortPairs 2^27 u32 + u32 2.48 against 2.41 ms) and for SortKeys of 4-byte keys (2.38-2.51 against
// 2.20 ms), each against 32-tile digit-wave windows.  Ballot ranking costs more VALU per key than the
// LDS tables but has no bank conflicts, which skewed digits (few distinct values per wave) make heavy in
// the tables.  SortKeys of 4-byte keys ranks half of the waves by ballots (2^28 u32 with 8-tile windows:
// 2.083 ms with 2/16, 2.063-2.072 with 4/16, 2.056 with 6/16, 2.041-2.050 with 8/16, 2.064 with 10/16;
// at 16-key tiles and 32-tile windows a quarter was best: 2.430 ms, against 2.455 ms with tables only and
// 2.563 ms with ballots only).  SortPairs of 8-byte keys keeps ballots only (5.82 / 5.48 ms uniform /
// AND-of-3, against 5.85 / 5.51 with half and 5.84 / 5.62 with a quarter).
constexpr Geometry geometry_for(size_t key_bytes, size_t value_bytes) {
    if (key_bytes <= 4 && value_bytes == 0) return Geometry{1024, 18, 8, false, 8};
    if (key_bytes == 8) return value_bytes ? Geometry{1024, 9, 2, true, 16} : Geometry{1024, 9, 16, false, 4};
    return value_bytes > 4 ? Geometry{512, 18, 8, false, 4} : Geometry{512, 28, 8, false, 4};
}

template <typename K, int VB>
constexpr Geometry geometry() {
    return geometry_for(sizeof(K), VB);
}

// Test hooks (any setting gives the same results): the largest portion a launch ranks (0: the
// default) and the in-wave ranking variant.  Each sort reads them once, so a concurrent change on
// another thread applies from the next call.
std::atomic<uint32_t> g_portion_limit{0};
std::atomic<int> g_rank_mode{kRankMixed};
std::atomic<bool> g_precount{false};  // precomputed first-pass offsets when the call allows them

// Keys ranked per launch.  The large portion keeps every look-back count below 2^30; the compact
// portion matches the reference's PORTION_SIZE (device_radix_sort.h:1056), so its look-back region is
// never larger than the reference's and the layout always fits a reference-sized temp buffer.
uint32_t portion_size(uint32_t tile, bool compact, uint32_t limit) {
    const uint32_t def = compact ? ((1u << 28) - 1u) / tile * tile : ((1u << 30) - 1u) / tile * tile;
    if (limit == 0) return def;
    uint32_t p = limit / tile * tile;
    if (p < tile) p = tile;
    return std::min(p, def);
}

struct Layout {
    uint32_t passes, portions, portion, tiles_max;
    size_t bins_off, lookback_off, keys_tmp_off, values_tmp_off, total;
    // First-pass tile offsets precomputed by the histogram (0: the first pass looks back like the
    // others): the per-workgroup totals start here, past `total`, when the caller's temp has room.
    size_t chunk_off = 0;
    size_t clear_bytes;  // bins, zeroed per call
    // Two look-back regions of tiles_max rows: launch k of a call (passes in order, portions in order
    // within a pass) uses region k % 2 and zeroes the other one's rows for launch k + 1.
    size_t region_words;
    int rank_mode = kRankMixed;  // test hooks as read at the start of the call
    uint32_t spin_limit = 64;
};

Layout make_layout(uint32_t n, size_t key_bytes, size_t value_bytes, uint32_t begin_bit, uint32_t end_bit,
                   uint32_t tile, bool need_tmp, bool compact, uint32_t portion_limit) {
    Layout L{};
    L.passes = (end_bit - begin_bit + 7) / 8;
    L.portion = portion_size(tile, compact, portion_limit);
    L.portions = static_cast<uint32_t>(ceil_div(n, L.portion));
    L.tiles_max = static_cast<uint32_t>(ceil_div(std::min(n, L.portion), tile));
    size_t off = 0;
    L.bins_off = off;
    off += static_cast<size_t>(L.portions) * L.passes * kDigits * 4;
    L.clear_bytes = off;
    off = align_up(off, kViewAlign);
    L.lookback_off = off;
    L.region_words = static_cast<size_t>(L.tiles_max) * kDigits;
    off += 2 * L.region_words * 4;
    L.keys_tmp_off = L.values_tmp_off = 0;
    if (need_tmp && L.passes > 1) {
        off = align_up(off, kViewAlign);
        L.keys_tmp_off = off;
        off += static_cast<size_t>(n) * key_bytes;
        if (value_bytes) {
            off = align_up(off, kViewAlign);
            L.values_tmp_off = off;
            off += static_cast<size_t>(n) * value_bytes;
        }
    }
    L.total = off;
    return L;
}

// Histogram workgroups over `len` keys: one per CU for histogram_kernel (128 KB of counters), and for
// histogram_tiles_kernel two per CU for 4-byte keys (80 KB each), one for 8-byte keys; contiguous slices
// of at most kHistMaxItems keys, each a whole number of `granule` keys: 16-byte steps of the workgroup for
// histogram_kernel, onesweep tiles for histogram_tiles_kernel.
struct HistPlan {
    uint64_t per;
    unsigned grid;
};
template <typename K>
constexpr uint32_t hist_step() {
    return static_cast<uint32_t>(kHistBlock) * kHistVecItems * (16 / sizeof(K));
}
template <typename K>
HistPlan hist_plan(uint32_t len, uint32_t granule = hist_step<K>(), bool tiles = false) {
    const uint64_t hist_target = static_cast<uint64_t>(device_cu_count()) * (tiles && sizeof(K) == 4 ? 2 : 1);
    uint64_t per = ceil_div(ceil_div(len, hist_target), granule) * granule;
    per = std::min<uint64_t>(per, kHistMaxItems / granule * granule);
    return HistPlan{per, static_cast<unsigned>(ceil_div(len, per))};
}

template <typename K, bool DESC, int VB>
int launch_sort(char* temp, const Layout& L, const K* keys_in, K* keys_out, const void* values_in, void* values_out,
                K* keys_tmp, void* values_tmp, K* const* db_keys, void* const* db_values, int sel, uint32_t n,
                uint32_t begin_bit, uint32_t end_bit, hipStream_t stream) {
    constexpr Geometry G = geometry<K, VB>();
    uint32_t* bins = reinterpret_cast<uint32_t*>(temp + L.bins_off);
    uint32_t* regions = reinterpret_cast<uint32_t*>(temp + L.lookback_off);

    // Precomputed first-pass offsets (a single portion): the histogram also writes the first pass's
    // per-tile digit counts into look-back region 0 and per-workgroup totals into the chunk region.
    const bool precount = L.chunk_off != 0;
    // One fill per call: the bins and, unless the histogram writes it, region 0 for the first launch
    // (the bins come first in the layout; the alignment gap between them is zeroed with them).
    int st = launch_fill_u32(bins, precount ? L.clear_bytes / 4 : (L.lookback_off - L.bins_off) / 4 + L.region_words,
                             0u, stream);
    if (st != kOk) return st;

    const K* hist_src = db_keys ? db_keys[sel] : keys_in;
    const bool full = begin_bit == 0 && end_bit == sizeof(K) * 8;
    uint32_t* chunk_sums = precount ? reinterpret_cast<uint32_t*>(temp + L.chunk_off) : nullptr;
    HistPlan hp0{};
    for (uint32_t q = 0; q < L.portions; ++q) {
        const uint32_t len = std::min(L.portion, n - q * L.portion);
        const HistPlan hp = precount ? hist_plan<K>(len, G.tile(), true) : hist_plan<K>(len);
        const uint64_t per = hp.per;
        const unsigned grid = hp.grid;
        if (q == 0) hp0 = hp;
        LaunchScope scope("radix_histogram", stream);
        // Every portion adds into the totals of portion 0's slots.
        if (precount) {
            static_assert(G.tile() <= kHistMaxItems, "a histogram slice holds whole onesweep tiles");
            if (full)
                histogram_tiles_kernel<K, DESC, true, G.tile()><<<grid, kHistBlock, 0, stream>>>(
                    hist_src, len, static_cast<uint32_t>(per), bins, begin_bit, end_bit, L.passes, regions, chunk_sums);
            else
                histogram_tiles_kernel<K, DESC, false, G.tile()><<<grid, kHistBlock, 0, stream>>>(
                    hist_src, len, static_cast<uint32_t>(per), bins, begin_bit, end_bit, L.passes, regions, chunk_sums);
        } else if (full)
            histogram_kernel<K, DESC, true><<<grid, kHistBlock, 0, stream>>>(
                hist_src + static_cast<size_t>(q) * L.portion, len, static_cast<uint32_t>(per), bins, begin_bit,
                end_bit, L.passes);
        else
            histogram_kernel<K, DESC, false><<<grid, kHistBlock, 0, stream>>>(
                hist_src + static_cast<size_t>(q) * L.portion, len, static_cast<uint32_t>(per), bins, begin_bit,
                end_bit, L.passes);
        st = check_hip(hipGetLastError(), "radix_histogram launch");
        if (st != kOk) return st;
    }
    {
        LaunchScope scope("radix_bins_scan", stream);
        bins_scan_kernel<<<1, kDigits, 0, stream>>>(bins, L.passes);
        st = check_hip(hipGetLastError(), "radix_bins_scan launch");
        if (st != kOk) return st;
    }
    if (precount) {
        LaunchScope scope("radix_tile_offsets", stream);
        chunk_scan_kernel<<<kDigits, kDigits, 0, stream>>>(chunk_sums, bins, hp0.grid);
        st = check_hip(hipGetLastError(), "radix_chunk_scan launch");
        if (st != kOk) return st;
        tile_offsets_kernel<<<hp0.grid, kDigits, 0, stream>>>(regions, chunk_sums,
                                                               static_cast<uint32_t>(hp0.per / G.tile()),
                                                               static_cast<uint32_t>(ceil_div(n, G.tile())));
        st = check_hip(hipGetLastError(), "radix_tile_offsets launch");
        if (st != kOk) return st;
    }

    using VW = typename ValueWord<VB>::type;
    for (uint32_t p = 0; p < L.passes; ++p) {
        const K* src;
        K* dst;
        const void* vsrc;
        void* vdst;
        if (db_keys) {
            src = db_keys[sel];
            dst = db_keys[sel ^ 1];
            vsrc = VB ? db_values[sel] : nullptr;
            vdst = VB ? db_values[sel ^ 1] : nullptr;
            sel ^= 1;
        } else {
            // The last pass writes keys_out; earlier passes alternate so that pass 0 reads keys_in.
            const bool to_out = ((L.passes - 1 - p) % 2) == 0;
            dst = to_out ? keys_out : keys_tmp;
            vdst = to_out ? values_out : values_tmp;
            if (p == 0) {
                src = keys_in;
                vsrc = values_in;
            } else {
                src = to_out ? keys_tmp : keys_out;
                vsrc = to_out ? values_tmp : values_out;
            }
        }
        const uint32_t shift = begin_bit + 8 * p;
        const uint32_t nb = std::min(8u, end_bit - shift);
        for (uint32_t q = 0; q < L.portions; ++q) {
            const uint32_t len = std::min(L.portion, n - q * L.portion);
            const uint32_t tiles = static_cast<uint32_t>(ceil_div(len, G.tile()));
            const bool pre = precount && p == 0;  // region 0 holds the first pass's offsets
            const uint32_t k = p * L.portions + q;
            uint32_t* lookback = regions + (k & 1u) * L.region_words;
            // Rows the next launch walks: the next portion of this pass, else the first of the next pass.
            uint32_t next_tiles = 0;
            if (q + 1 < L.portions)
                next_tiles = static_cast<uint32_t>(ceil_div(std::min(L.portion, n - (q + 1) * L.portion), G.tile()));
            else if (p + 1 < L.passes)
                next_tiles = static_cast<uint32_t>(ceil_div(std::min(L.portion, n), G.tile()));
            uint32_t* clear_rows = next_tiles ? regions + ((k + 1) & 1u) * L.region_words : nullptr;
            const size_t qoff = static_cast<size_t>(q) * L.portion;
            LaunchScope scope("radix_onesweep", stream);
            const VW* vs = VB ? static_cast<const VW*>(vsrc) + qoff : nullptr;
            uint32_t* offsets = bins + (static_cast<size_t>(q) * L.passes + p) * kDigits;
            uint32_t* next = q + 1 < L.portions ? bins + (static_cast<size_t>(q + 1) * L.passes + p) * kDigits : nullptr;
            onesweep_kernel<K, DESC, VB, G.block, G.items, G.window, G.grouped><<<tiles, G.block, 0, stream>>>(
                src + qoff, dst, vs, vdst, len, offsets, next, lookback, pre ? lookback : nullptr, clear_rows,
                next_tiles * kDigits, shift, nb, n, L.spin_limit, ballot_sixteenths_for(L.rank_mode, G.ballot_sixteenths));
            st = check_hip(hipGetLastError(), "radix_onesweep launch");
            if (st != kOk) return st;
        }
    }
    return kOk;
}

template <typename K, int VB>
int sort_entry(void* temp, size_t temp_bytes, const K* keys_in, K* keys_out, const void* values_in, void* values_out,
               K* db0, K* db1, void* vdb0, void* vdb1, int* selector, uint32_t n, uint32_t begin_bit, uint32_t end_bit,
               int descending, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const bool db = selector != nullptr;
    const char* what = VB ? "DeviceRadixSort::SortPairs" : "DeviceRadixSort::SortKeys";
    if (begin_bit > end_bit) return set_error(kInvalidArgument, "%s: begin_bit must not exceed end_bit", what);
    if (end_bit > sizeof(K) * 8) return set_error(kInvalidArgument, "%s: end_bit exceeds the key width", what);
    if (db && *selector != 0 && *selector != 1)
        return set_error(kInvalidArgument, "%s: DoubleBuffer selector must be 0 or 1", what);
    if (n == 0) return kOk;
    if (db) {
        if (!db0 || !db1 || (VB && (!vdb0 || !vdb1))) return set_error(kInvalidArgument, "%s: null buffer", what);
    } else {
        if (!keys_in || !keys_out || (VB && (!values_in || !values_out)))
            return set_error(kInvalidArgument, "%s: null buffer", what);
    }
    if (begin_bit == end_bit) {
        if (db) return kOk;
        int st = launch_copy(keys_out, keys_in, static_cast<uint64_t>(n) * sizeof(K), stream);
        if (st != kOk || !VB) return st;
        return launch_copy(values_out, values_in, static_cast<uint64_t>(n) * VB, stream);
    }
    constexpr Geometry G = geometry<K, VB>();
    const uint32_t portion_limit = g_portion_limit.load(std::memory_order_relaxed);
    Layout L = make_layout(n, sizeof(K), VB, begin_bit, end_bit, G.tile(), !db, false, portion_limit);
    if (temp_bytes < L.total) L = make_layout(n, sizeof(K), VB, begin_bit, end_bit, G.tile(), !db, true, portion_limit);
    L.rank_mode = g_rank_mode.load(std::memory_order_relaxed);
    L.spin_limit = lookback_spin_limit();
    if (!temp || temp_bytes < L.total)
        return set_error(kTempTooSmall, "%s: temp storage too small (%zu < %zu bytes)", what, temp_bytes, L.total);
    {
        // First-pass offsets from the histogram (off by default; the test hook switches them on): 4-byte
        // keys without values, one portion, 16-byte aligned keys (the histogram's slices of whole tiles
        // then load 16-byte vectors) and room for the per-workgroup totals.  With 32-tile look-back
        // windows they paid (SortKeys 2^28 u32, kernel trace: first pass 586 -> 504 us for 14 us more
        // histogram and 12 us of offset kernels); with 8-tile windows every pass that looks back runs
        // as fast as the first pass, and the tile counts cost more than they save (2.028 ms per sort
        // without them, 2.042 ms with them: the tiles histogram 196 us against 178 us for the plain one,
        // plus 11 us of offset kernels).  For 8-byte keys with values both the histogram and the first
        // pass got slower (737 -> 801 us).
        const void* first_src = db ? (*selector ? db1 : db0) : keys_in;
        const size_t off = align_up(L.total, kViewAlign);
        if (sizeof(K) == 4 && VB == 0 && L.portions == 1 && reinterpret_cast<uintptr_t>(first_src) % 16 == 0 &&
            g_precount.load(std::memory_order_relaxed) &&
            temp_bytes >= off + static_cast<size_t>(hist_plan<K>(n, G.tile(), true).grid) * kDigits * 4)
            L.chunk_off = off;
    }
    if (reinterpret_cast<uintptr_t>(temp) % 4 != 0) return set_error(kInvalidArgument, "%s: temp not 4-byte aligned", what);
    char* t = static_cast<char*>(temp);
    K* keys_tmp = L.keys_tmp_off ? reinterpret_cast<K*>(t + L.keys_tmp_off) : nullptr;
    void* values_tmp = L.values_tmp_off ? static_cast<void*>(t + L.values_tmp_off) : nullptr;
    K* db_keys[2] = {db0, db1};
    void* db_values[2] = {vdb0, vdb1};
    const int sel = db ? *selector : 0;
    int st;
    if (descending)
        st = launch_sort<K, true, VB>(t, L, keys_in, keys_out, values_in, values_out, keys_tmp, values_tmp,
                                      db ? db_keys : nullptr, db ? db_values : nullptr, sel, n, begin_bit, end_bit, stream);
    else
        st = launch_sort<K, false, VB>(t, L, keys_in, keys_out, values_in, values_out, keys_tmp, values_tmp,
                                       db ? db_keys : nullptr, db ? db_values : nullptr, sel, n, begin_bit, end_bit, stream);
    if (st == kOk && db) *selector = (*selector) ^ static_cast<int>(L.passes & 1u);
    return st;
}

}  // namespace radix
}  // namespace lcpp_hip

using namespace lcpp_hip;
using namespace lcpp_hip::radix;

#ifdef LCPP_HIP_PHASE_TRACE
namespace lcpp_hip {
int radix_trace_set_buffer(void* buffer, uint64_t records) {
    uint64_t* p = static_cast<uint64_t*>(buffer);
    int st = check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_buffer), &p, sizeof(p)), "trace buffer");
    if (st != kOk) return st;
    return check_hip(hipMemcpyToSymbol(HIP_SYMBOL(g_trace_records), &records, sizeof(records)), "trace records");
}
}  // namespace lcpp_hip
#endif

extern "C" {

int lcpp_hip_radix_set_portion_limit(uint32_t max_items_per_portion) {
    g_portion_limit.store(max_items_per_portion, std::memory_order_relaxed);
    return kOk;
}

// Selects the in-wave ranking of the onesweep kernel: 0 ballot match in every wave, 1 LDS lane-mask
// tables in every wave, 2 both (default).  All give the same stable ranks; the switch exists for tests
// and measurements.
int lcpp_hip_internal_radix_rank_mode(int mode) {
    if (mode != kRankBallot && mode != kRankLdsMatch && mode != kRankMixed)
        return set_error(kInvalidArgument, "rank mode must be 0, 1 or 2");
    g_rank_mode.store(mode, std::memory_order_relaxed);
    return kOk;
}

int lcpp_hip_internal_radix_precount(int enable) {
    return g_precount.exchange(enable != 0, std::memory_order_relaxed) ? 1 : 0;
}

uint32_t lcpp_hip_radix_tile_items(size_t key_bytes, size_t value_bytes) {
    (void)key_bytes;
    (void)value_bytes;
    return geometry_for(key_bytes, value_bytes).tile();
}

// Smallest temp storage this implementation accepts for the call (the compact-portion layout); it is
// never more than the reference's Get*TempStorageBytes for the same sizes.
size_t lcpp_hip_internal_radix_needed_bytes(uint32_t n, size_t key_bytes, size_t value_bytes, uint32_t begin_bit,
                                            uint32_t end_bit, int double_buffer) {
    if (n == 0 || begin_bit >= end_bit) return 0;
    return make_layout(n, key_bytes, value_bytes, begin_bit, end_bit, geometry_for(key_bytes, value_bytes).tile(), !double_buffer,
                       true, g_portion_limit.load(std::memory_order_relaxed))
        .total;
}

// Portions the sort would use with `temp_bytes` of temp storage (0 if it does not fit).
uint32_t lcpp_hip_internal_radix_portions(uint32_t n, size_t key_bytes, size_t value_bytes, uint32_t begin_bit,
                                          uint32_t end_bit, int double_buffer, size_t temp_bytes) {
    if (n == 0 || begin_bit >= end_bit) return 0;
    const uint32_t tile = geometry_for(key_bytes, value_bytes).tile();
    const uint32_t portion_limit = g_portion_limit.load(std::memory_order_relaxed);
    Layout L = make_layout(n, key_bytes, value_bytes, begin_bit, end_bit, tile, !double_buffer, false, portion_limit);
    if (temp_bytes < L.total)
        L = make_layout(n, key_bytes, value_bytes, begin_bit, end_bit, tile, !double_buffer, true, portion_limit);
    return temp_bytes < L.total ? 0 : L.portions;
}

#define LCPP_HIP_DEFINE_SORT(S, K)                                                                                  \
    int lcpp_hip_radix_sort_keys_##S(void* temp, size_t temp_bytes, const K* keys_in, K* keys_out, uint32_t n,       \
                                     uint32_t begin_bit, uint32_t end_bit, int descending, void* stream) {           \
        return sort_entry<K, 0>(temp, temp_bytes, keys_in, keys_out, nullptr, nullptr, nullptr, nullptr, nullptr,   \
                                nullptr, nullptr, n, begin_bit, end_bit, descending, stream);                       \
    }                                                                                                               \
    int lcpp_hip_radix_sort_keys_db_##S(void* temp, size_t temp_bytes, K* keys0, K* keys1, int* selector, uint32_t n, \
                                        uint32_t begin_bit, uint32_t end_bit, int descending, void* stream) {        \
        if (!selector) return set_error(kInvalidArgument, "DeviceRadixSort::SortKeys: null selector");              \
        return sort_entry<K, 0>(temp, temp_bytes, nullptr, nullptr, nullptr, nullptr, keys0, keys1, nullptr,        \
                                nullptr, selector, n, begin_bit, end_bit, descending, stream);                      \
    }                                                                                                               \
    int lcpp_hip_radix_sort_pairs_##S##_v32(void* temp, size_t temp_bytes, const K* keys_in, K* keys_out,           \
                                            const void* values_in, void* values_out, uint32_t n, uint32_t begin_bit, \
                                            uint32_t end_bit, int descending, void* stream) {                       \
        return sort_entry<K, 4>(temp, temp_bytes, keys_in, keys_out, values_in, values_out, nullptr, nullptr,       \
                                nullptr, nullptr, nullptr, n, begin_bit, end_bit, descending, stream);              \
    }                                                                                                               \
    int lcpp_hip_radix_sort_pairs_##S##_v64(void* temp, size_t temp_bytes, const K* keys_in, K* keys_out,           \
                                            const void* values_in, void* values_out, uint32_t n, uint32_t begin_bit, \
                                            uint32_t end_bit, int descending, void* stream) {                       \
        return sort_entry<K, 8>(temp, temp_bytes, keys_in, keys_out, values_in, values_out, nullptr, nullptr,       \
                                nullptr, nullptr, nullptr, n, begin_bit, end_bit, descending, stream);              \
    }                                                                                                               \
    int lcpp_hip_radix_sort_pairs_db_##S##_v32(void* temp, size_t temp_bytes, K* keys0, K* keys1, void* values0,     \
                                               void* values1, int* selector, uint32_t n, uint32_t begin_bit,        \
                                               uint32_t end_bit, int descending, void* stream) {                    \
        if (!selector) return set_error(kInvalidArgument, "DeviceRadixSort::SortPairs: null selector");             \
        return sort_entry<K, 4>(temp, temp_bytes, nullptr, nullptr, nullptr, nullptr, keys0, keys1, values0,        \
                                values1, selector, n, begin_bit, end_bit, descending, stream);                      \
    }                                                                                                               \
    int lcpp_hip_radix_sort_pairs_db_##S##_v64(void* temp, size_t temp_bytes, K* keys0, K* keys1, void* values0,     \
                                               void* values1, int* selector, uint32_t n, uint32_t begin_bit,        \
                                               uint32_t end_bit, int descending, void* stream) {                    \
        if (!selector) return set_error(kInvalidArgument, "DeviceRadixSort::SortPairs: null selector");             \
        return sort_entry<K, 8>(temp, temp_bytes, nullptr, nullptr, nullptr, nullptr, keys0, keys1, values0,        \
                                values1, selector, n, begin_bit, end_bit, descending, stream);                      \
    }

LCPP_HIP_DEFINE_SORT(u32, uint32_t)
LCPP_HIP_DEFINE_SORT(i32, int32_t)
LCPP_HIP_DEFINE_SORT(f32, float)
LCPP_HIP_DEFINE_SORT(u64, uint64_t)
LCPP_HIP_DEFINE_SORT(i64, int64_t)
LCPP_HIP_DEFINE_SORT(f64, double)
#undef LCPP_HIP_DEFINE_SORT

}  // extern "C"
