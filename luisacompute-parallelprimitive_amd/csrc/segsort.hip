// DeviceSegmentedRadixSort and DeviceSegmentedSort (keys and key-value pairs, ascending and
// descending, bit ranges, DoubleBuffer) for gfx950: a stable sort per segment.
//
// Reference paths (src/lcpp/device/): DeviceSegmentedSort<> (device_segmented_sort.h:43-505): a
// stable merge sort by a comparator (lhs < rhs, or lhs > rhs for the descending forms) in passes of
// doubling width over all items; the segment of item i is found by binary search over the begin
// offsets (ascending, disjoint segments), only items inside a segment are written
// (dispatch_key_merge, :300-420); DoubleBuffer forms flip the selector once per pass, ceil(log2 n)
// times.  DeviceSegmentedRadixSort<> (device_segmented_radix_sort.h:26-246) is that sort with the
// comparator "twiddled key bits [begin_bit, end_bit) compare less (greater)"; begin_bit == end_bit
// leaves a DoubleBuffer untouched.  Any stable sort by the same order gives the same output, so the
// sort here is free to differ from the reference's merge passes.
//
// MI355X design:
//   * Block phase: chunks sorted in LDS by one 256-thread workgroup each, C = 4,096 items in radix
//     order and 2,048 in value order.  Tiny segments (<= 16 items) are sorted by one thread each, in
//     registers; small ones (<= 512 items) together per 2,048-item tile of the item range (a joint sort
//     with position labels when a tile holds more than two), medium ones (<= C) by one workgroup each, and long ones chunk by chunk by a grid-stride
//     kernel over C-item tiles, so neither many tiny segments nor a few long ones leave the GPU idle.
//   * Radix order, medium segments and chunks: a stable LSD radix sort in LDS, 8-bit digits, 4, 8 or
//     16 items per thread by length; per pass a ballot match ranks each wave's items against per-wave
//     digit counters, one workgroup scan orders (digit, wave), items are scattered to LDS and read back.
//   * Value order, and small segments in either order: a stable odd-even transposition sort of each
//     thread's 8 items in registers, then merge-path passes in LDS (widths 8 .. 1,024), each thread
//     producing 8 outputs after one binary search.
//   * Global phase, only for segments longer than C: merge-path passes of width C, 2 C, ... between the
//     output and a scratch buffer, over 2,048-item output tiles (merge-path splits by wave-level
//     searches, inputs staged in LDS); a segment takes part while the width is below its length.  The
//     block phase writes a segment with an odd number of global passes to the scratch buffer, so that
//     every segment's last pass lands in the output.  The block phase also records the longest segment
//     (and whether a small one exists) in per-stream device words (a slot of a static device array);
//     launches with nothing to do exit after reading them.
//   * Orders: radix order compares (twiddled bits >> begin_bit) & mask (descending: the complement);
//     value order (floats of DeviceSegmentedSort) compares the values, so -0.0 equals +0.0.
// Algorithmic traffic: 2 * (sizeof(K) + sizeof(V)) per item in segments up to C items, plus the
// same per global pass for longer segments.
#include "common.hpp"
#include "../../include/lcpp_hip.h"

#include <map>
#include <mutex>
#include <utility>

namespace lcpp_hip {
namespace {

constexpr int kSsBlock = 256;
constexpr int kSsItems = 8;
constexpr uint32_t kSsChunk = kSsBlock * kSsItems;  // 2048
// Segments of at most this many items are sorted jointly per 2,048-item tile (tile kernel); longer ones
// up to a chunk by one workgroup each (block kernel), longer still chunk by chunk (chunk kernel).  The
// crossover was measured: 2^24 keys in 256-item segments 0.31 ms jointly vs 0.42 ms per segment, in
// 1,024-item segments 0.27 vs 0.22 ms.
constexpr uint32_t kSsSmall = 512;
// Pair sorts' LDS arrays hold one pad word per 8 items: a thread's 8 consecutive outputs then start 9
// words after its neighbour's, so the 64 lanes of a store hit distinct banks (measured: SortPairs block
// phase 1.13 -> 1.03 ms; keys-only sorts ran slower padded, 0.75 -> 0.87 ms, and stay unpadded).
template <bool PAD>
inline constexpr uint32_t kSsPadded = PAD ? kSsChunk + kSsChunk / 8 : kSsChunk;
template <bool PAD>
__device__ __forceinline__ uint32_t pad(uint32_t p) {
    return PAD ? p + (p >> 3) : p;
}

enum : int { kKindUnsigned = 0, kKindSigned = 1, kKindFloat = 2 };

struct SortOrder {
    uint64_t mask;       // bit_count ones (all ones for the full width)
    uint32_t begin_bit;
    uint32_t descending;
    uint32_t value_order;  // compare float values instead of twiddled bits
};

template <typename K, int KIND>
__device__ __forceinline__ K twiddle(K bits) {
    constexpr K sign = static_cast<K>(K(1) << (sizeof(K) * 8 - 1));
    if constexpr (KIND == kKindSigned) {
        return bits ^ sign;
    } else if constexpr (KIND == kKindFloat) {
        return (bits & sign) ? static_cast<K>(~bits) : static_cast<K>(bits | sign);
    } else {
        return bits;
    }
}

// a strictly before b in the sort order.
template <typename K, int KIND>
__device__ __forceinline__ bool before(K a, K b, const SortOrder& o) {
    if constexpr (KIND == kKindFloat) {
        if (o.value_order) {
            using F = std::conditional_t<sizeof(K) == 8, double, float>;
            const F fa = __builtin_bit_cast(F, a), fb = __builtin_bit_cast(F, b);
            return o.descending ? fb < fa : fa < fb;
        }
    }
    const K ka = static_cast<K>((twiddle<K, KIND>(a) >> o.begin_bit) & static_cast<K>(o.mask));
    const K kb = static_cast<K>((twiddle<K, KIND>(b) >> o.begin_bit) & static_cast<K>(o.mask));
    return o.descending ? kb < ka : ka < kb;
}

// Number of items taken from `left` among the first `diag` outputs of the stable merge of left[0, lw)
// and right[0, rw) (ties take left first).
template <typename RightFirst>
__device__ __forceinline__ uint32_t merge_split(uint32_t diag, uint32_t lw, uint32_t rw, RightFirst right_first) {
    uint32_t lo = diag > rw ? diag - rw : 0u;
    uint32_t hi = diag < lw ? diag : lw;
    while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (right_first(mid)) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

// merge_split with right_first(mid) = "right[diag - 1 - mid] goes before left[mid]".
template <typename K, int KIND, typename GetLeft, typename GetRight>
__device__ __forceinline__ uint32_t merge_path(uint32_t diag, uint32_t lw, uint32_t rw, GetLeft left, GetRight right,
                                               const SortOrder& o) {
    return merge_split(diag, lw, rw, [&](uint32_t mid) { return before<K, KIND>(right(diag - 1 - mid), left(mid), o); });
}

// Number of global passes a segment of `len` items takes after its chunks of `chunk` items are sorted
// (widths chunk, 2 chunk, ... below len).
__device__ __forceinline__ uint32_t global_passes(uint64_t len, uint32_t chunk) {
    uint32_t p = 0;
    for (uint64_t w = chunk; w < len; w *= 2) ++p;
    return p;
}

// Sorts the chunk [c, c + len) (len <= 2,048) of keys_in / values_in into kdst / vdst with the whole
// workgroup (it may be in place: every item is read before any is written).  Collective: every thread of
// the workgroup calls it with the same arguments.
//
// LABELS: the chunk holds several groups (contiguous position ranges; s_label[p], bits 0-14, numbers the
// group of position p in ascending order) that are sorted independently, and only positions with bit 15
// set are written.  Because groups are contiguous and their labels ascend, every sorted run keeps each
// group on the group's own positions, so a label is read by position and never moves: a right-run item
// goes before a left-run item only when both positions have the same label and its key is before.
template <typename K, typename V, bool PAIRS, int KIND, bool LABELS>
__device__ __forceinline__ void sort_chunk(const K* keys_in, K* kdst, const V* values_in, V* vdst, uint64_t c,
                                           uint32_t len, const SortOrder& o, K (*s_keys)[kSsPadded<PAIRS>],
                                           V (*s_vals)[PAIRS ? kSsPadded<PAIRS> : 1], const uint16_t* s_label) {
    const uint32_t tid = threadIdx.x;
    auto same_group = [&](uint32_t pa, uint32_t pb) { return !LABELS || s_label[pa] == s_label[pb]; };
    // Thread-local stable sort of items [8 tid, 8 tid + 8) of the chunk (padding never moves
    // before real items: it is only compared with other padding).
    K k[kSsItems];
    V v[kSsItems];
    const uint32_t base = tid * kSsItems;
#pragma unroll
    for (int j = 0; j < kSsItems; ++j) {
        const bool ok = base + j < len;
        k[j] = ok ? keys_in[c + base + j] : K(0);
        if constexpr (PAIRS) v[j] = ok ? values_in[c + base + j] : V(0);
    }
    const uint32_t mine = base < len ? (len - base < kSsItems ? len - base : kSsItems) : 0u;
#pragma unroll
    for (int round = 0; round < kSsItems; ++round) {
#pragma unroll
        for (int j = round & 1; j + 1 < kSsItems; j += 2) {
            if (static_cast<uint32_t>(j + 1) < mine && before<K, KIND>(k[j + 1], k[j], o) &&
                same_group(base + j, base + j + 1)) {
                const K tk = k[j];
                k[j] = k[j + 1];
                k[j + 1] = tk;
                if constexpr (PAIRS) {
                    const V tv = v[j];
                    v[j] = v[j + 1];
                    v[j + 1] = tv;
                }
            }
        }
    }
    __syncthreads();  // the previous chunk's readers of s_keys are done
#pragma unroll
    for (int j = 0; j < kSsItems; ++j) {
        s_keys[0][pad<PAIRS>(base + j)] = k[j];
        if constexpr (PAIRS) s_vals[0][pad<PAIRS>(base + j)] = v[j];
    }
    __syncthreads();
    int cur = 0;
    for (uint32_t w = kSsItems; w < len; w *= 2) {
        // Output positions [base, base + 8) of the merged pair of runs that holds them.
        if (base < len) {
            const uint32_t l0 = base / (2 * w) * (2 * w);
            const uint32_t lw = len - l0 < w ? len - l0 : w;
            const uint32_t r0 = l0 + lw;
            const uint32_t rw = r0 < len ? (len - r0 < w ? len - r0 : w) : 0u;
            const uint32_t diag = base - l0;
            const K* sk = s_keys[cur];
            uint32_t li = merge_split(diag, lw, rw, [&](uint32_t mid) {
                const uint32_t pr = r0 + diag - 1 - mid, pl = l0 + mid;
                return before<K, KIND>(sk[pad<PAIRS>(pr)], sk[pad<PAIRS>(pl)], o) && same_group(pr, pl);
            });
            uint32_t ri = diag - li;
            const uint32_t count = len - base < kSsItems ? len - base : kSsItems;
            for (uint32_t j = 0; j < count; ++j) {
                const K rk = sk[pad<PAIRS>(r0 + ri)], lk = sk[pad<PAIRS>(l0 + li)];
                const bool take_left =
                    li < lw && (ri >= rw || !(before<K, KIND>(rk, lk, o) && same_group(r0 + ri, l0 + li)));
                const uint32_t src = pad<PAIRS>(take_left ? l0 + li : r0 + ri);
                s_keys[cur ^ 1][pad<PAIRS>(base + j)] = sk[src];
                if constexpr (PAIRS) s_vals[cur ^ 1][pad<PAIRS>(base + j)] = s_vals[cur][src];
                if (take_left) ++li;
                else ++ri;
            }
        }
        cur ^= 1;
        __syncthreads();
    }
    for (uint32_t q = tid; q < len; q += kSsBlock) {
        if (LABELS && !(s_label[q] >> 15)) continue;
        kdst[c + q] = s_keys[cur][pad<PAIRS>(q)];
        if constexpr (PAIRS) vdst[c + q] = s_vals[cur][pad<PAIRS>(q)];
    }
}

// Radix order (o.value_order == 0): sorts the chunk [c, c + len) (len <= 256 ITEMS) like sort_chunk, by a
// stable LSD radix sort in LDS over 8-bit digits of (twiddled bits >> begin_bit) & mask (complemented
// for descending orders).  Wave w holds items [64 ITEMS w, 64 ITEMS (w + 1)): item 64 k + lane of its
// range in register k.  Per pass: digits; each wave ranks its items with ballot matches and per-wave
// digit counters; one workgroup scan turns the (digit, wave) counts into output offsets (digit-major,
// wave order within a digit: stable); every item goes to LDS at its offset and is read back in the same
// layout.  Items past len take digit 255 in every pass, so they stay behind the real ones; a wave with no
// real item (its range starts at or past len) takes no part in ranking or scatter.  s_k / s_v hold
// 256 ITEMS entries, s_cnt 4 x 256 counters, s_tot 4 words.  Collective, and may be in place like
// sort_chunk (every item is read before the first barrier, written after the last).
//
// LABELS (the groups of sort_chunk: contiguous position ranges numbered in ascending order by bits 0-14
// of s_label, written where bit 15 is set): every item carries its position's label, and after the key
// passes `label_passes` more passes sort by the label's bytes.  Labels are the most significant part of
// the order and ascend with position, so every group returns to its own positions, sorted by key.  The
// carried labels move through s_l (256 ITEMS entries).
template <typename K, typename V, bool PAIRS, int KIND, int ITEMS, bool LABELS = false>
__device__ __forceinline__ void radix_sort_chunk(const K* keys_in, K* kdst, const V* values_in, V* vdst, uint64_t c,
                                                 uint32_t len, const SortOrder& o, K* s_k, V* s_v, uint32_t* s_cnt,
                                                 uint32_t* s_tot, const uint16_t* s_label = nullptr,
                                                 uint16_t* s_l = nullptr, uint32_t label_passes = 0) {
    static_assert(kSsBlock == 256, "thread t scans digit t");
    static_assert(kSsBlock * ITEMS <= 0x10000, "ranks are packed in 16 bits");
    constexpr int kWaves = kSsBlock / kWave;
    constexpr uint32_t kPerWave = kWave * ITEMS;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t first = wave * kPerWave + lane;  // item of register 0
    // Register j is real when 64 j < left; items are addressed from per-lane bases, so that only these
    // stay live and every register's offset is an instruction immediate.
    const int32_t left = static_cast<int32_t>(len) - static_cast<int32_t>(first);
    const K* kin = keys_in + c + first;
    const V* vin = PAIRS ? values_in + c + first : nullptr;
    K k[ITEMS];
    V v[PAIRS ? ITEMS : 1];
    uint32_t lab[LABELS ? ITEMS : 1];
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        k[j] = j * kWave < left ? kin[j * kWave] : K(0);
        if constexpr (PAIRS) v[j] = j * kWave < left ? vin[j * kWave] : V(0);
        if constexpr (LABELS) lab[j] = j * kWave < left ? s_label[first + j * kWave] : 0u;
    }
    const uint32_t bits = o.mask == 0 ? 0u : 64u - static_cast<uint32_t>(__builtin_clzll(o.mask));
    const uint32_t key_passes = (bits + 7) / 8;
    const uint32_t passes = key_passes + (LABELS ? label_passes : 0u);
    for (uint32_t i = tid; i < kWaves * 256; i += kSsBlock) s_cnt[i] = 0;
    __syncthreads();  // the previous chunk's readers of s_k / s_v and s_cnt are done
    uint32_t* cnt = s_cnt + wave * 256;
    const bool idle = wave * kPerWave >= len;  // wave-uniform
    for (uint32_t p = 0; p < passes; ++p) {
        const uint32_t shift = o.begin_bit + 8 * p;
        const uint32_t nb = bits - 8 * p < 8 ? bits - 8 * p : 8u;
        uint32_t rd[ITEMS];  // digit << 16 | rank within the wave's digit
        if (!idle) {
#pragma unroll
            for (int j = 0; j < ITEMS; ++j) {
                uint32_t d;
                if (!LABELS || p < key_passes) {
                    d = static_cast<uint32_t>((twiddle<K, KIND>(k[j]) >> shift)) & ((1u << nb) - 1u);
                    if (o.descending) d ^= (1u << nb) - 1u;
                } else {
                    d = ((lab[j] & 0x7FFFu) >> (8 * (p - key_passes))) & 0xFFu;
                }
                d = j * kWave < left ? d : 255u;
                const uint64_t peers = match_digit(d);
                const uint32_t below = popc_lanes_below(peers);
                const uint32_t base = cnt[d];
                rd[j] = (d << 16) | (base + below);
                if ((peers >> lane) == 1ull) cnt[d] = base + below + 1;
            }
        }
        __syncthreads();
        // Thread t owns digit t: the digit's total over the waves, scanned over the digits.
        uint32_t wc[kWaves];
        uint32_t total = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            wc[w] = s_cnt[w * 256 + tid];
            total += wc[w];
        }
        const uint32_t incl = wave_inclusive_scan(total, SumOp{});
        if (lane == kWave - 1) s_tot[wave] = incl;
        __syncthreads();
        uint32_t off = incl - total;
        for (uint32_t w = 0; w < wave; ++w) off += s_tot[w];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            s_cnt[w * 256 + tid] = off;
            off += wc[w];
        }
        __syncthreads();
        if (!idle) {
#pragma unroll
            for (int j = 0; j < ITEMS; ++j) {
                const uint32_t pos = cnt[rd[j] >> 16] + (rd[j] & 0xFFFFu);
                s_k[pos] = k[j];
                if constexpr (PAIRS) s_v[pos] = v[j];
                if constexpr (LABELS) s_l[pos] = static_cast<uint16_t>(lab[j]);
            }
        }
        __syncthreads();
        if (!idle) {
            const K* sk = s_k + first;
            const V* sv = s_v + first;
#pragma unroll
            for (int j = 0; j < ITEMS; ++j) {
                k[j] = sk[j * kWave];
                if constexpr (PAIRS) v[j] = sv[j * kWave];
                if constexpr (LABELS) lab[j] = s_l[first + j * kWave];
            }
        }
        // Each wave clears its own counters (only it writes them before the next barrier).
        for (uint32_t i = lane; i < 256; i += kWave) cnt[i] = 0;
    }
    K* kout = kdst + c + first;
    V* vout = PAIRS ? vdst + c + first : nullptr;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        if (j * kWave < left && (!LABELS || (lab[j] >> 15))) {
            kout[j * kWave] = k[j];
            if constexpr (PAIRS) vout[j * kWave] = v[j];
        }
    }
}

// Radix order sorts chunks of up to kSsRadixChunk items in LDS; value order merges 2,048-item chunks.
constexpr uint32_t kSsRadixChunk = 2 * kSsChunk;  // 4096

// Items sorted in LDS per chunk, the width the global passes start from, and the longest medium segment.
__device__ __forceinline__ uint32_t chunk_items(const SortOrder& o) {
    return o.value_order ? kSsChunk : kSsRadixChunk;
}

// LDS of the block and chunk kernels, one byte array used either way: the merge sort's two padded key
// (and value) buffers, or the radix sort's flat key (and value) arrays of kSsRadixChunk entries followed
// by its 4 x 256 digit counters.  Integer keys are always sorted in radix order and need only the latter.
template <typename K, typename V, bool PAIRS, int KIND>
struct ChunkLds {
    using KeyBuf = K[kSsPadded<PAIRS>];
    using ValBuf = V[PAIRS ? kSsPadded<PAIRS> : 1];
    static constexpr size_t kMergeKeys = sizeof(K) * 2 * kSsPadded<PAIRS>;
    static constexpr size_t kMergeBytes = kMergeKeys + (PAIRS ? sizeof(V) * 2 * kSsPadded<PAIRS> : 0);
    static constexpr size_t kRadixKeys = sizeof(K) * kSsRadixChunk;
    static constexpr size_t kRadixVals = PAIRS ? sizeof(V) * kSsRadixChunk : 0;
    static constexpr size_t kRadixBytes = kRadixKeys + kRadixVals + 4 * 256 * sizeof(uint32_t);
    static constexpr size_t kBytes = (KIND == kKindFloat && kMergeBytes > kRadixBytes) ? kMergeBytes : kRadixBytes;
    static_assert(kRadixKeys % 16 == 0 && kMergeKeys % 16 == 0, "value arrays stay aligned");
};

// Sorts one chunk of len <= chunk_items(o) items: radix order with 4, 8 or 16 items per thread
// (whichever fits len), value order by sort_chunk.  `lds` is the kernel's ChunkLds array.
template <typename K, typename V, bool PAIRS, int KIND>
__device__ __forceinline__ void sort_any_chunk(const K* keys_in, K* kdst, const V* values_in, V* vdst, uint64_t c,
                                               uint32_t len, const SortOrder& o, unsigned char* lds,
                                               uint32_t* s_tot) {
    using L = ChunkLds<K, V, PAIRS, KIND>;
    if constexpr (KIND == kKindFloat) {
        if (o.value_order) {
            sort_chunk<K, V, PAIRS, KIND, false>(keys_in, kdst, values_in, vdst, c, len, o,
                                                 reinterpret_cast<typename L::KeyBuf*>(lds),
                                                 reinterpret_cast<typename L::ValBuf*>(lds + L::kMergeKeys), nullptr);
            return;
        }
    }
    K* s_k = reinterpret_cast<K*>(lds);
    V* s_v = reinterpret_cast<V*>(lds + L::kRadixKeys);
    uint32_t* s_cnt = reinterpret_cast<uint32_t*>(lds + L::kRadixKeys + L::kRadixVals);
    if (len <= kSsBlock * 4)
        radix_sort_chunk<K, V, PAIRS, KIND, 4>(keys_in, kdst, values_in, vdst, c, len, o, s_k, s_v, s_cnt, s_tot);
    else if (len <= kSsBlock * 8)
        radix_sort_chunk<K, V, PAIRS, KIND, 8>(keys_in, kdst, values_in, vdst, c, len, o, s_k, s_v, s_cnt, s_tot);
    else
        radix_sort_chunk<K, V, PAIRS, KIND, 16>(keys_in, kdst, values_in, vdst, c, len, o, s_k, s_v, s_cnt, s_tot);
}

// Segments of at most this many items are sorted by one thread each, in registers, when the block
// kernel reads their offsets (the tile kernel leaves them alone).
constexpr uint32_t kSsTiny = 16;

// Stable odd-even transposition sort of [b, b + len) (len <= kSsTiny) by one thread, into the outputs.
template <typename K, typename V, bool PAIRS, int KIND>
__device__ __forceinline__ void sort_tiny(const K* keys_in, K* keys_out, const V* values_in, V* values_out, uint64_t b,
                                          uint32_t len, const SortOrder& o) {
    K k[kSsTiny];
    V v[PAIRS ? kSsTiny : 1];
#pragma unroll
    for (int j = 0; j < static_cast<int>(kSsTiny); ++j) {
        const bool ok = static_cast<uint32_t>(j) < len;
        k[j] = ok ? keys_in[b + j] : K(0);
        if constexpr (PAIRS) v[j] = ok ? values_in[b + j] : V(0);
    }
#pragma unroll
    for (int round = 0; round < static_cast<int>(kSsTiny); ++round) {
#pragma unroll
        for (int j = round & 1; j + 1 < static_cast<int>(kSsTiny); j += 2) {
            if (static_cast<uint32_t>(j + 1) < len && before<K, KIND>(k[j + 1], k[j], o)) {
                const K tk = k[j];
                k[j] = k[j + 1];
                k[j + 1] = tk;
                if constexpr (PAIRS) {
                    const V tv = v[j];
                    v[j] = v[j + 1];
                    v[j + 1] = tv;
                }
            }
        }
    }
#pragma unroll
    for (int j = 0; j < static_cast<int>(kSsTiny); ++j) {
        if (static_cast<uint32_t>(j) < len) {
            keys_out[b + j] = k[j];
            if constexpr (PAIRS) values_out[b + j] = v[j];
        }
    }
}

// Segment of item i (begins ascending): the last segment whose begin <= i, or -1.
__device__ __forceinline__ int64_t find_segment(const uint32_t* begins, uint32_t num_segments, uint64_t i) {
    uint32_t lo = 0, hi = num_segments;
    while (lo < hi) {
        const uint32_t mid = lo + (hi - lo) / 2;
        if (begins[mid] <= i) lo = mid + 1;
        else hi = mid;
    }
    return static_cast<int64_t>(lo) - 1;
}

// First x in [lo, hi) with pred(x) true, or hi (pred false ... false true ... true), found by one wave
// in 64-ary steps: each lane tests the end of one of 64 buckets, the first true bucket is kept.  All 64
// lanes take part and get the same result.
template <typename Pred>
__device__ __forceinline__ uint64_t wave_search(uint64_t lo, uint64_t hi, Pred pred) {
    const uint32_t lane = threadIdx.x & 63u;
    while (lo < hi) {
        const uint64_t step = (hi - lo + 63) / 64;
        const uint64_t valid = (hi - lo) / step < 64 ? (hi - lo) / step : 64;
        const uint64_t m = lo + (lane + 1) * step - 1;
        const uint64_t mask = __ballot(lane < valid && pred(m));
        if (mask) {
            const uint32_t f = static_cast<uint32_t>(__builtin_ctzll(mask));
            hi = lo + (f + 1) * step - 1;
            lo = lo + f * step;
        } else {
            lo = lo + valid * step;
        }
    }
    return lo;
}

// Medium segments (kSsSmall < items <= chunk_items(o)): one workgroup sorts each.  Workgroup g takes segment
// indices [g * per_group, (g + 1) * per_group), one per thread at a time, so that many small segments
// cost a read of their offsets rather than a workgroup each; per_group is 1 whenever segments average
// more than kSsSmall items.  The thread that reads a tiny segment's offsets (at most kSsTiny items) sorts
// it at once (sort_tiny).  The kernel also sets words[1] when a small segment (more than kSsTiny, at most
// kSsSmall items) exists and posts the
// longest segment above a chunk to words[0] (a relaxed load first: same-address atomics serialise at
// ~11 ns each).
template <typename K, typename V, bool PAIRS, int KIND>
__global__ __launch_bounds__(kSsBlock) void segsort_block_kernel(const K* keys_in, K* keys_out, const V* values_in,
                                                                 V* values_out, const uint32_t* __restrict__ begins,
                                                                 const uint32_t* __restrict__ ends,
                                                                 uint32_t num_segments, uint32_t per_group,
                                                                 uint64_t n, SortOrder o, uint32_t* words) {
    __shared__ __align__(16) unsigned char s_lds[ChunkLds<K, V, PAIRS, KIND>::kBytes];
    __shared__ uint32_t s_medium[kSsBlock];
    __shared__ uint32_t s_tot[kSsBlock / kWave];
    __shared__ uint32_t s_count, s_small, s_long;
    const uint32_t tid = threadIdx.x;
    const uint32_t chunk = chunk_items(o);
    const uint64_t g0 = static_cast<uint64_t>(blockIdx.x) * per_group;
    const uint64_t g1 = g0 + per_group < num_segments ? g0 + per_group : num_segments;
    if (tid == 0) s_small = 0, s_long = 0;
    for (uint64_t x0 = g0; x0 < g1; x0 += kSsBlock) {
        if (tid == 0) s_count = 0;
        __syncthreads();
        const uint64_t x = x0 + tid;
        if (x < g1) {
            const uint64_t b = begins[x], e = ends[x];
            if (b < e && e <= n) {
                const uint64_t len = e - b;
                if (len <= kSsTiny)
                    sort_tiny<K, V, PAIRS, KIND>(keys_in, keys_out, values_in, values_out, b,
                                                 static_cast<uint32_t>(len), o);
                else if (len <= kSsSmall) s_small = 1;  // benign race: every writer stores 1
                else if (len <= chunk) s_medium[atomicAdd(&s_count, 1u)] = static_cast<uint32_t>(x);
                else atomicMax(&s_long, static_cast<uint32_t>(len));
            }
        }
        __syncthreads();
        const uint32_t count = s_count;
        for (uint32_t k = 0; k < count; ++k) {
            const uint32_t x2 = s_medium[k];
            const uint64_t b = begins[x2], e = ends[x2];
            sort_any_chunk<K, V, PAIRS, KIND>(keys_in, keys_out, values_in, values_out, b,
                                              static_cast<uint32_t>(e - b), o, s_lds, s_tot);
        }
        __syncthreads();  // s_medium and s_count are rewritten next
    }
    if (words && tid == 0) {
        if (s_small && __hip_atomic_load(&words[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0)
            __hip_atomic_store(&words[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (s_long && __hip_atomic_load(&words[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < s_long)
            atomicMax(&words[0], s_long);
    }
}

// Long segments (more than C = chunk_items(o) items): grid-stride over C-item tiles of the item range; a
// tile sorts the segment-aligned chunks [b + C k, ...) that start inside it.  A long segment is longer
// than a tile, so it meets a tile only as the segment holding the tile's first or last item, and its
// chunk starts are a tile apart: a tile sorts at most two chunks.  A segment that takes an odd number of
// global passes is sorted into the scratch buffer, so that its last pass writes the output (in place
// when the scratch buffer is the input of a DoubleBuffer sort).
template <typename K, typename V, bool PAIRS, int KIND>
__global__ __launch_bounds__(kSsBlock) void segsort_chunk_kernel(const K* keys_in, K* keys_out, K* keys_scratch,
                                                                 const V* values_in, V* values_out, V* values_scratch,
                                                                 const uint32_t* __restrict__ begins,
                                                                 const uint32_t* __restrict__ ends,
                                                                 uint32_t num_segments, uint64_t n, SortOrder o,
                                                                 const uint32_t* longest) {
    const uint32_t chunk = chunk_items(o);
    if (longest && *longest <= chunk) return;  // no segment is longer than a chunk
    __shared__ __align__(16) unsigned char s_lds[ChunkLds<K, V, PAIRS, KIND>::kBytes];
    __shared__ uint64_t s_seg[2];
    __shared__ uint32_t s_tot[kSsBlock / kWave];
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint64_t tiles = ceil_div(n, chunk);
    for (uint64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
        const uint64_t t0 = t * chunk;
        const uint64_t t1 = t0 + chunk < n ? t0 + chunk : n;
        if (wave < 2) {
            const uint64_t at = wave == 0 ? t0 : t1 - 1;
            const uint64_t c = wave_search(0, num_segments, [&](uint64_t x) { return begins[x] > at; });
            if ((tid & 63u) == 0) s_seg[wave] = c;  // segment index + 1 (0: before every segment)
        }
        __syncthreads();
        const uint64_t c0 = s_seg[0], c1 = s_seg[1];
        __syncthreads();
        for (uint64_t c = c0; c <= c1; c = (c == c0 && c1 != c0) ? c1 : c1 + 1) {
            if (c == 0) continue;
            const uint64_t b = begins[c - 1], e = ends[c - 1];
            if (b >= e || e > n || e - b <= chunk || e <= t0 || b >= t1) continue;
            const uint64_t from = b > t0 ? b : t0;
            const uint64_t cs = b + ceil_div(from - b, chunk) * chunk;  // first chunk start >= from
            if (cs >= t1 || cs >= e) continue;
            const bool to_scratch = global_passes(e - b, chunk) & 1u;
            sort_any_chunk<K, V, PAIRS, KIND>(keys_in, to_scratch ? keys_scratch : keys_out, values_in,
                                              to_scratch ? values_scratch : values_out, cs,
                                              static_cast<uint32_t>(e - cs < chunk ? e - cs : chunk), o, s_lds,
                                              s_tot);
        }
    }
}

// Small segments (at most kSsSmall items): grid-stride over 2,048-item tiles [t0, t1) of the item range,
// one workgroup per tile.  The segments wholly inside the tile are sorted together: one or two on their
// own, more in one joint sort of the tile (sort_chunk with labels: a position's label counts the begins
// and ends of those segments at or before it, so each segment and each gap between them is one group;
// only segment positions are written).  A small segment that starts in the tile and ends after it is
// sorted on its own.  The block kernel sets words[1] when any small segment exists; otherwise this
// kernel exits at once.
template <typename K, typename V, bool PAIRS, int KIND>
__global__ __launch_bounds__(kSsBlock) void segsort_tile_kernel(const K* keys_in, K* keys_out, K* keys_scratch,
                                                                const V* values_in, V* values_out, V* values_scratch,
                                                                const uint32_t* __restrict__ begins,
                                                                const uint32_t* __restrict__ ends,
                                                                uint32_t num_segments, uint64_t n, SortOrder o,
                                                                const uint32_t* words) {
    if (words && words[1] == 0) return;  // no small segment
    using L = ChunkLds<K, V, PAIRS, KIND>;
    __shared__ __align__(16) unsigned char s_lds[L::kBytes];
    __shared__ uint16_t s_label[kSsChunk];
    __shared__ uint64_t s_seg[2];
    __shared__ uint32_t s_tot[kSsBlock / kWave];
    __shared__ uint32_t s_inside;       // segments of at most 2,048 items wholly inside the tile
    __shared__ uint32_t s_pick[2][2];   // the first two of them (begin, end relative to t0)
    // Thread totals of the label scan share s_label's space (they are read before labels are written).
    uint32_t* s_total = reinterpret_cast<uint32_t*>(s_label);
    // Boundary counts per position, packed (begins in the low half, ends in the high half), live in the
    // sort's LDS before the joint sort uses it (2,048 words: the array holds at least 2 x 2,048 keys).
    static_assert(L::kBytes >= kSsChunk * sizeof(uint32_t), "boundary counts fit the sort's LDS");
    uint32_t* s_count = reinterpret_cast<uint32_t*>(s_lds);
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint64_t tiles = ceil_div(n, kSsChunk);
    for (uint64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
        const uint64_t t0 = t * kSsChunk;
        const uint64_t t1 = t0 + kSsChunk < n ? t0 + kSsChunk : n;
        const uint32_t tlen = static_cast<uint32_t>(t1 - t0);
        if (wave < 2) {
            const uint64_t at = wave == 0 ? t0 : t1 - 1;
            const uint64_t c = wave_search(0, num_segments, [&](uint64_t x) { return begins[x] > at; });
            if ((tid & 63u) == 0) s_seg[wave] = c;  // segment index + 1 (0: before every segment)
        }
        if (tid == 0) s_inside = 0;
        __syncthreads();
        const uint64_t c0 = s_seg[0], c1 = s_seg[1];
        // Segments c0 - 1 .. c1 - 1 meet the tile; count the small ones wholly inside it.  One or two are
        // sorted on their own; more take one joint sort with labels.
        const uint64_t first = c0 > 0 ? c0 - 1 : 0;
        for (uint64_t x = first + tid; x < c1; x += kSsBlock) {
            const uint64_t b = begins[x], e = ends[x];
            if (b >= e || e > n || b < t0 || e > t1 || e - b > kSsSmall || e - b <= kSsTiny) continue;
            const uint32_t slot = atomicAdd(&s_inside, 1u);
            if (slot < 2) {
                s_pick[slot][0] = static_cast<uint32_t>(b - t0);
                s_pick[slot][1] = static_cast<uint32_t>(e - t0);
            }
        }
        __syncthreads();
        const uint32_t inside = s_inside;
        if (inside > 0 && inside <= 2) {
            for (uint32_t k = 0; k < inside; ++k) {
                const uint32_t pb = s_pick[k][0], pe = s_pick[k][1];
                sort_any_chunk<K, V, PAIRS, KIND>(keys_in, keys_out, values_in, values_out, t0 + pb, pe - pb, o,
                                                  s_lds, s_tot);
            }
        } else if (inside > 2) {
            for (uint32_t q = tid; q < kSsChunk; q += kSsBlock) s_count[q] = 0;
            __syncthreads();
            for (uint64_t x = first + tid; x < c1; x += kSsBlock) {
                const uint64_t b = begins[x], e = ends[x];
                if (b >= e || e > n || b < t0 || e > t1 || e - b > kSsSmall || e - b <= kSsTiny) continue;
                atomicAdd(&s_count[b - t0], 1u);
                if (e < t1) atomicAdd(&s_count[e - t0], 1u << 16);
            }
            __syncthreads();
            // Inclusive prefix of the packed counts: thread totals, a DPP wave scan, the four wave totals
            // through LDS, then labels.
            const uint32_t base = tid * kSsItems;
            uint32_t run = 0;
#pragma unroll
            for (int j = 0; j < kSsItems; ++j) run += s_count[base + j];
            uint32_t inc = run;
            inc += dpp_move<dpp::kRowShr1>(0u, inc);
            inc += dpp_move<dpp::kRowShr2>(0u, inc);
            inc += dpp_move<dpp::kRowShr4>(0u, inc);
            inc += dpp_move<dpp::kRowShr8>(0u, inc);
            inc += dpp_move<dpp::kRowBcast15, 0xa>(0u, inc);
            inc += dpp_move<dpp::kRowBcast31, 0xc>(0u, inc);
            if ((tid & 63u) == 63u) s_total[wave] = inc;
            __syncthreads();
            uint32_t acc = inc - run;  // this thread's exclusive prefix within its wave
            for (uint32_t w = 0; w < wave; ++w) acc += s_total[w];
            __syncthreads();  // every total is read before labels overwrite them
#pragma unroll
            for (int j = 0; j < kSsItems; ++j) {
                acc += s_count[base + j];
                const uint32_t opened = acc & 0xFFFFu, closed = acc >> 16;
                s_label[base + j] = static_cast<uint16_t>((opened + closed) | (opened > closed ? 0x8000u : 0u));
            }
            __syncthreads();  // labels complete; s_count (in the sort's LDS) is free again
            bool merged = false;
            if constexpr (KIND == kKindFloat) {
                if (o.value_order) {
                    sort_chunk<K, V, PAIRS, KIND, true>(keys_in, keys_out, values_in, values_out, t0, tlen, o,
                                                        reinterpret_cast<typename L::KeyBuf*>(s_lds),
                                                        reinterpret_cast<typename L::ValBuf*>(s_lds + L::kMergeKeys),
                                                        s_label);
                    merged = true;
                }
            }
            if (!merged) {
                // Labels ascend with position: the last one is the largest.
                const uint32_t label_passes = (s_label[tlen - 1] & 0x7FFFu) < 256u ? 1u : 2u;
                static_assert(L::kRadixKeys >= kSsChunk * (sizeof(K) + sizeof(uint16_t)), "labels fit");
                radix_sort_chunk<K, V, PAIRS, KIND, kSsItems, true>(
                    keys_in, keys_out, values_in, values_out, t0, tlen, o, reinterpret_cast<K*>(s_lds),
                    reinterpret_cast<V*>(s_lds + L::kRadixKeys),
                    reinterpret_cast<uint32_t*>(s_lds + L::kRadixKeys + L::kRadixVals), s_tot, s_label,
                    reinterpret_cast<uint16_t*>(s_lds + kSsChunk * sizeof(K)), label_passes);
            }
        }
        __syncthreads();
        // A small segment that starts in the tile and ends after it holds the tile's last item.
        if (c1 > 0) {
            const uint64_t b = begins[c1 - 1], e = ends[c1 - 1];
            if (b < e && e <= n && e - b <= kSsSmall && e - b > kSsTiny && b >= t0 && e > t1)
                sort_any_chunk<K, V, PAIRS, KIND>(keys_in, keys_out, values_in, values_out, b,
                                                  static_cast<uint32_t>(e - b), o, s_lds, s_tot);
        }
        __syncthreads();  // s_seg, s_count and s_label are rewritten by the next tile
    }
}

// One piece of a global pass: outputs [p0, p1) (at most 2,048) of the merge of the runs
// [l0, l0 + lw) and [r0, r0 + rw) of src into dst.
struct MergePiece {
    uint64_t p0, p1, l0, lw, r0, rw;
    uint32_t to_out;
};

// Global pass `pass` (width w = chunk_items(o) << pass) over 2,048-item output tiles, grid-stride.  A segment of
// P > pass global passes writes the output when P - 1 - pass is even and the scratch buffer otherwise,
// reading the other one.  A segment longer than w is longer than a tile, so a tile meets at most two
// such segments: the one holding its first item and the one holding its last; any other segment in the
// tile is shorter than a tile and already sorted.  Per piece (the tile's part of one merge of two
// runs): waves 0 and 1 find the merge-path split at the piece's two ends, the inputs are staged in LDS,
// every thread merges 8 outputs and the piece is stored whole.
template <typename K, typename V, bool PAIRS, int KIND>
__global__ __launch_bounds__(256) void segsort_merge_kernel(K* __restrict__ out_k, K* __restrict__ scr_k,
                                                            V* __restrict__ out_v, V* __restrict__ scr_v,
                                                            const uint32_t* __restrict__ begins,
                                                            const uint32_t* __restrict__ ends, uint32_t num_segments,
                                                            uint64_t n, uint32_t pass, SortOrder o,
                                                            const uint32_t* longest) {
    const uint32_t chunk = chunk_items(o);
    const uint64_t w = static_cast<uint64_t>(chunk) << pass;
    if (longest && w >= *longest) return;  // no segment is longer than this width
    __shared__ K s_keys[2][kSsPadded<PAIRS>];
    __shared__ V s_vals[PAIRS ? 2 : 1][PAIRS ? kSsPadded<PAIRS> : 1];
    __shared__ uint64_t s_seg[2];
    __shared__ uint64_t s_split[2];
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid >> 6;
    const uint64_t tiles = ceil_div(n, kSsChunk);
    for (uint64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
        const uint64_t t0 = t * kSsChunk;
        const uint64_t t1 = t0 + kSsChunk < n ? t0 + kSsChunk : n;
        if (wave < 2) {
            const uint64_t at = wave == 0 ? t0 : t1 - 1;
            const uint64_t c = wave_search(0, num_segments, [&](uint64_t x) { return begins[x] > at; });
            if ((tid & 63u) == 0) s_seg[wave] = c;  // segment index + 1 (0: before every segment)
        }
        __syncthreads();
        const uint64_t c0 = s_seg[0], c1 = s_seg[1];
        __syncthreads();
        for (uint64_t c = c0; c <= c1; c = (c == c0 && c1 != c0) ? c1 : c1 + 1) {
            if (c == 0) continue;
            const uint64_t b = begins[c - 1], e = ends[c - 1];
            if (b >= e || e > n || e - b <= w || e <= t0 || b >= t1) continue;
            const bool to_out = ((global_passes(e - b, chunk) - 1u - pass) & 1u) == 0;
            K* src_k = to_out ? scr_k : out_k;
            K* dst_k = to_out ? out_k : scr_k;
            V* src_v = to_out ? scr_v : out_v;
            V* dst_v = to_out ? out_v : scr_v;
            uint64_t p0 = b > t0 ? b : t0;
            const uint64_t pend = e < t1 ? e : t1;
            while (p0 < pend) {
                MergePiece pc;
                pc.l0 = b + (p0 - b) / (2 * w) * (2 * w);
                pc.lw = e - pc.l0 < w ? e - pc.l0 : w;
                pc.r0 = pc.l0 + pc.lw;
                pc.rw = pc.r0 < e ? (e - pc.r0 < w ? e - pc.r0 : w) : 0;
                pc.p0 = p0;
                pc.p1 = pc.r0 + pc.rw < pend ? pc.r0 + pc.rw : pend;
                // Merge-path splits at the piece's ends: left items among the first d outputs.
                if (wave < 2) {
                    const uint64_t d = (wave == 0 ? pc.p0 : pc.p1) - pc.l0;
                    const uint64_t lo = d > pc.rw ? d - pc.rw : 0;
                    const uint64_t hi = d < pc.lw ? d : pc.lw;
                    const uint64_t li = wave_search(lo, hi, [&](uint64_t x) {
                        return before<K, KIND>(src_k[pc.r0 + (d - 1 - x)], src_k[pc.l0 + x], o);
                    });
                    if ((tid & 63u) == 0) s_split[wave] = li;
                }
                __syncthreads();
                const uint64_t li0 = s_split[0], li1 = s_split[1];
                const uint32_t nl = static_cast<uint32_t>(li1 - li0);
                const uint32_t len = static_cast<uint32_t>(pc.p1 - pc.p0);
                const uint32_t nr = len - nl;
                const uint64_t lbase = pc.l0 + li0;
                const uint64_t rbase = pc.r0 + (pc.p0 - pc.l0 - li0);
                for (uint32_t q = tid; q < len; q += kSsBlock) {
                    const uint64_t from = q < nl ? lbase + q : rbase + (q - nl);
                    s_keys[0][pad<PAIRS>(q)] = src_k[from];
                    if constexpr (PAIRS) s_vals[0][pad<PAIRS>(q)] = src_v[from];
                }
                __syncthreads();
                const uint32_t base = tid * kSsItems;
                if (base < len) {
                    const K* sk = s_keys[0];
                    auto left = [&](uint32_t x) { return sk[pad<PAIRS>(x)]; };
                    auto right = [&](uint32_t x) { return sk[pad<PAIRS>(nl + x)]; };
                    uint32_t li = merge_path<K, KIND>(base, nl, nr, left, right, o);
                    uint32_t ri = base - li;
                    const uint32_t count = len - base < kSsItems ? len - base : kSsItems;
                    for (uint32_t j = 0; j < count; ++j) {
                        const K rk = sk[pad<PAIRS>(nl + ri)], lk = sk[pad<PAIRS>(li)];
                        const bool take_left = li < nl && (ri >= nr || !before<K, KIND>(rk, lk, o));
                        const uint32_t from = pad<PAIRS>(take_left ? li : nl + ri);
                        s_keys[1][pad<PAIRS>(base + j)] = sk[from];
                        if constexpr (PAIRS) s_vals[1][pad<PAIRS>(base + j)] = s_vals[0][from];
                        if (take_left) ++li;
                        else ++ri;
                    }
                }
                __syncthreads();
                for (uint32_t q = tid; q < len; q += kSsBlock) {
                    dst_k[pc.p0 + q] = s_keys[1][pad<PAIRS>(q)];
                    if constexpr (PAIRS) dst_v[pc.p0 + q] = s_vals[1][pad<PAIRS>(q)];
                }
                __syncthreads();  // LDS is reused by the next piece
                p0 = pc.p1;
            }
        }
    }
}

// Merge passes of a DoubleBuffer sort in the reference: ceil(log2 n) for n >= 2.
uint32_t reference_pass_count(uint64_t n) {
    uint32_t p = 0;
    for (uint64_t w = 1; w < n; w *= 2) ++p;
    return p;
}

// Two device words per call receive the longest segment and the small-segment flag: slots of a static
// device array (each GPU holds its own copy, found by hipGetSymbolAddress); no entry point allocates.
// An eager call uses its stream's slot, handed out on the stream's first call: eager calls on one stream
// run in order, so they never share it while running.  A call recorded into a graph gets a slot of its
// own, never handed out again, so the graph's replays share their words with no eager call and no other
// graph (only with concurrent replays of the same graph, which share every buffer of the call anyway).
// Past kLongestSlots slots, for a call recorded before any eager call on its device (the array's address
// is not looked up during a capture), for a stream of a device other than the current one (the lookup
// needs the stream's device current), and for hipStreamPerThread (one handle naming another stream in
// each host thread, so calls through it are not ordered with each other), a call gets nullptr and its
// kernels run without the early exits (same results).
constexpr uint32_t kLongestSlots = 16384;
__device__ uint32_t g_longest_slots[2 * kLongestSlots];

enum : int { kSlotNone = 0, kSlotStream = 1, kSlotOwn = 2 };

struct SlotPool {
    std::mutex mu;
    std::map<std::pair<int, hipStream_t>, uint32_t*> stream_words;
    std::map<int, std::pair<uint32_t*, uint32_t>> devices;  // device -> (array address, next slot)
};
SlotPool& slot_pool() {
    static SlotPool pool;
    return pool;
}

// 0: eager, 1: recording into a graph, -1: the query failed.
int capture_state(hipStream_t stream) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    return capture != hipStreamCaptureStatusNone ? 1 : 0;
}

// The slot a call on `stream` would use now (kSlot*); with `take`, the slot itself (nullptr for
// kSlotNone), handed out if it is new.
int longest_slot(hipStream_t stream, bool take, uint32_t** word) {
    if (word) *word = nullptr;
    if (stream == hipStreamPerThread) return kSlotNone;
    const int capturing = capture_state(stream);
    if (capturing < 0) return kSlotNone;
    int dev = 0, current = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess || hipGetDevice(&current) != hipSuccess) {
        (void)hipGetLastError();
        return kSlotNone;
    }
    if (dev != current) return kSlotNone;
    SlotPool& pool = slot_pool();
    std::lock_guard<std::mutex> lock(pool.mu);
    const auto key = std::make_pair(dev, stream);
    if (!capturing) {
        const auto it = pool.stream_words.find(key);
        if (it != pool.stream_words.end()) {
            if (word) *word = it->second;
            return kSlotStream;
        }
    }
    auto& d = pool.devices[dev];
    if (d.second >= kLongestSlots) return kSlotNone;
    // The array's address is looked up by an eager call only: no runtime query runs inside a capture.
    if (capturing && !d.first) return kSlotNone;
    if (!take) return capturing ? kSlotOwn : kSlotStream;
    if (!d.first) {
        void* base = nullptr;
        if (hipGetSymbolAddress(&base, HIP_SYMBOL(g_longest_slots)) != hipSuccess || !base) {
            (void)hipGetLastError();
            return kSlotNone;
        }
        d.first = static_cast<uint32_t*>(base);
    }
    uint32_t* w = d.first + 2 * d.second++;
    if (!capturing) pool.stream_words.emplace(key, w);
    if (word) *word = w;
    return capturing ? kSlotOwn : kSlotStream;
}

uint32_t* longest_word(hipStream_t stream) {
    uint32_t* w = nullptr;
    longest_slot(stream, true, &w);
    return w;
}

template <typename K, typename V, bool PAIRS, int KIND>
int segsort(K* keys_in, K* keys_out, K* keys_scratch, V* values_in, V* values_out, V* values_scratch, uint64_t n,
            uint64_t num_segments, const uint32_t* begins, const uint32_t* ends, uint32_t begin_bit, uint32_t end_bit,
            int descending, int value_order, hipStream_t stream) {
    const uint32_t width = sizeof(K) * 8;
    SortOrder o;
    o.begin_bit = begin_bit;
    o.descending = descending ? 1u : 0u;
    o.value_order = (KIND == kKindFloat && value_order) ? 1u : 0u;
    const uint32_t bits = end_bit - begin_bit;
    o.mask = bits >= 64 ? ~0ull : ((1ull << bits) - 1);
    if (bits == 0 && !o.value_order) {
        o.mask = 0;  // every key compares equal: a stable copy
        o.begin_bit = 0;
    }
    (void)width;
    int st;
    // words[0]: the longest segment above a chunk; words[1]: set when a small segment exists.
    uint32_t* words = longest_word(stream);
    if (words) {
        st = launch_fill_u32(words, 2, 0u, stream);
        if (st != kOk) return st;
    }
    const uint64_t tiles = ceil_div(n, kSsChunk);
    const uint64_t cap = static_cast<uint64_t>(device_cu_count()) * 8;
    {
        // About one workgroup per 4,096 items (groups of segment offsets: with tiny and small segments each
        // workgroup reads many), but at least 8 per CU where the input allows, and never more than n / kSsSmall
        // (the most segments that can be medium).  Measured on 2^26 u32 keys against one per 512 items:
        // 16-item segments 0.80 -> 0.43 ms, 8-item pairs 0.95 -> 0.56, 1,024-item keys 0.474 -> 0.440.
        const uint64_t most = n / kSsSmall > 0 ? n / kSsSmall : 1;
        const uint64_t fill = cap < most ? cap : most;
        const uint64_t target = n / (8 * kSsSmall) > fill ? n / (8 * kSsSmall) : fill;
        const uint64_t per_group = ceil_div(num_segments, target);
        const unsigned groups = static_cast<unsigned>(ceil_div(num_segments, per_group));
        LaunchScope scope("segsort_block", stream);
        segsort_block_kernel<K, V, PAIRS, KIND><<<groups, kSsBlock, 0, stream>>>(
            keys_in, keys_out, values_in, values_out, begins, ends, static_cast<uint32_t>(num_segments),
            static_cast<uint32_t>(per_group), n, o, words);
        st = check_hip(hipGetLastError(), "segsort block launch");
        if (st != kOk) return st;
    }
    {
        // Tile and chunk kernels: grid-stride over 2,048-item tiles with enough workgroups to hide each
        // tile's segment searches; with no small (long) segment they exit after one word read.
        const uint64_t tile_cap = cap * 4;
        const unsigned tile_grid = static_cast<unsigned>(tiles < tile_cap ? tiles : tile_cap);
        LaunchScope scope("segsort_tile", stream);
        segsort_tile_kernel<K, V, PAIRS, KIND><<<tile_grid, kSsBlock, 0, stream>>>(
            keys_in, keys_out, keys_scratch, values_in, values_out, values_scratch, begins, ends,
            static_cast<uint32_t>(num_segments), n, o, words);
        st = check_hip(hipGetLastError(), "segsort tile launch");
        if (st != kOk) return st;
        const uint32_t chunk = o.value_order ? kSsChunk : kSsRadixChunk;
        if (n <= chunk) return kOk;
        LaunchScope scope2("segsort_chunk", stream);
        segsort_chunk_kernel<K, V, PAIRS, KIND><<<tile_grid, kSsBlock, 0, stream>>>(
            keys_in, keys_out, keys_scratch, values_in, values_out, values_scratch, begins, ends,
            static_cast<uint32_t>(num_segments), n, o, words);
        st = check_hip(hipGetLastError(), "segsort chunk launch");
        if (st != kOk) return st;
    }
    // Global passes: grid-stride over 2,048-item tiles on a bounded grid; a pass with no work (no segment
    // longer than its width) costs one word read per workgroup.
    const uint32_t* longest = words;
    const unsigned grid = static_cast<unsigned>(tiles < cap ? tiles : cap);
    uint32_t pass = 0;
    for (uint64_t w = o.value_order ? kSsChunk : kSsRadixChunk; w < n; w *= 2, ++pass) {
        LaunchScope scope("segsort_merge", stream);
        segsort_merge_kernel<K, V, PAIRS, KIND><<<grid, 256, 0, stream>>>(
            keys_out, keys_scratch, values_out, values_scratch, begins, ends, static_cast<uint32_t>(num_segments), n,
            pass, o, longest);
        st = check_hip(hipGetLastError(), "segsort merge launch");
        if (st != kOk) return st;
    }
    return kOk;
}

size_t round4(size_t bytes) { return (bytes + 3) / 4 * 4; }

// Temp layout of the copy forms (the reference's GetSort*TempStorageBytes): n scratch keys, then (pairs)
// n scratch values at the value type's alignment.
size_t segsort_temp_bytes(uint64_t n, size_t key_bytes, size_t value_bytes) {
    if (n <= 1) return 0;
    const size_t kb = round4(n * key_bytes);
    if (!value_bytes) return kb;
    return align_up(kb, value_bytes) + round4(n * value_bytes);
}

template <typename K, typename V, bool PAIRS, int KIND>
int segsort_entry(const char* what, void* temp, size_t temp_bytes, const K* keys_in, K* keys_out, const V* values_in,
                  V* values_out, uint64_t n, uint64_t num_segments, const uint32_t* begins, const uint32_t* ends,
                  uint32_t begin_bit, uint32_t end_bit, int descending, int value_order, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items", what);
    if (num_segments > 0x7FFFFFFFull) return set_error(kInvalidArgument, "%s: too many segments", what);
    if (begin_bit > end_bit || end_bit > sizeof(K) * 8)
        return set_error(kInvalidArgument, "%s: bad bit range [%u, %u)", what, begin_bit, end_bit);
    if (n == 0 || num_segments == 0) return kOk;
    if (!keys_in || !keys_out || !begins || !ends || (PAIRS && (!values_in || !values_out)))
        return set_error(kInvalidArgument, "%s: null input or output", what);
    const size_t need = segsort_temp_bytes(n, sizeof(K), PAIRS ? sizeof(V) : 0);
    if (n > kSsChunk && (!temp || temp_bytes < need))
        return set_error(kTempTooSmall, "%s: temp storage too small (%zu < %zu bytes)", what, temp_bytes, need);
    K* ks = static_cast<K*>(temp);
    V* vs = PAIRS ? reinterpret_cast<V*>(static_cast<unsigned char*>(temp) + align_up(round4(n * sizeof(K)), sizeof(V)))
                  : nullptr;
    return segsort<K, V, PAIRS, KIND>(const_cast<K*>(keys_in), keys_out, ks, const_cast<V*>(values_in), values_out,
                                      vs, n, num_segments, begins, ends, begin_bit, end_bit, descending, value_order,
                                      stream);
}

// DoubleBuffer forms: the result lands where the reference's selector points after its
// ceil(log2 n) flips; the other buffer is the scratch.
template <typename K, typename V, bool PAIRS, int KIND>
int segsort_db(const char* what, K* keys0, K* keys1, int* key_selector, V* values0, V* values1, int* value_selector,
               uint64_t n, uint64_t num_segments, const uint32_t* begins, const uint32_t* ends, uint32_t begin_bit,
               uint32_t end_bit, int descending, int value_order, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (!key_selector || (PAIRS && !value_selector)) return set_error(kInvalidArgument, "%s: null selector", what);
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items", what);
    if (num_segments > 0x7FFFFFFFull) return set_error(kInvalidArgument, "%s: too many segments", what);
    if (begin_bit > end_bit || end_bit > sizeof(K) * 8)
        return set_error(kInvalidArgument, "%s: bad bit range [%u, %u)", what, begin_bit, end_bit);
    if (n <= 1 || num_segments == 0) return kOk;
    if (!value_order && begin_bit == end_bit) return kOk;  // radix sort of no bits: buffers untouched
    if (!keys0 || !keys1 || !begins || !ends || (PAIRS && (!values0 || !values1)))
        return set_error(kInvalidArgument, "%s: null buffer", what);
    const uint32_t passes = reference_pass_count(n);
    const int ks = *key_selector & 1;
    K* kcur = ks ? keys1 : keys0;
    K* kalt = ks ? keys0 : keys1;
    V* vcur = nullptr;
    V* valt = nullptr;
    if constexpr (PAIRS) {
        const int vsel = *value_selector & 1;
        vcur = vsel ? values1 : values0;
        valt = vsel ? values0 : values1;
    }
    const bool odd = passes & 1u;
    K* kout = odd ? kalt : kcur;
    K* kscr = odd ? kcur : kalt;
    V* vout = odd ? valt : vcur;
    V* vscr = odd ? vcur : valt;
    // When the result goes to the alternate buffer the input stays in current, which the global phase
    // then uses as scratch (the block phase has read it by then).
    const int st = segsort<K, V, PAIRS, KIND>(kcur, kout, kscr, vcur, vout, vscr, n, num_segments, begins, ends,
                                              begin_bit, end_bit, descending, value_order, stream);
    if (st != kOk) return st;
    if (odd) {
        *key_selector ^= 1;
        if constexpr (PAIRS) *value_selector ^= 1;
    }
    return kOk;
}

template <typename T>
using Storage = std::conditional_t<sizeof(T) == 8, uint64_t, uint32_t>;
template <typename T>
constexpr int kKindOf = std::is_floating_point_v<T> ? kKindFloat : (std::is_signed_v<T> ? kKindSigned : kKindUnsigned);

}  // namespace
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

// The words a segmented sort called now on `stream` would use, without taking them: 1 the stream's slot
// (an eager call), 2 a slot of its own (a call recorded into a graph), 0 none (past the slot count).
int lcpp_hip_internal_segsort_slot_kind(void* stream) {
    return longest_slot(static_cast<hipStream_t>(stream), false, nullptr);
}

size_t lcpp_hip_segmented_sort_keys_temp_bytes(uint64_t n, size_t key_bytes) {
    return segsort_temp_bytes(n, key_bytes, 0);
}
size_t lcpp_hip_segmented_sort_pairs_temp_bytes(uint64_t n, size_t key_bytes, size_t value_bytes) {
    return segsort_temp_bytes(n, key_bytes, value_bytes);
}

#define LCPP_HIP_DEFINE_SEGSORT_PAIRS(KS, KT, VS, VT)                                                                 \
    int lcpp_hip_segmented_sort_pairs_##KS##_##VS(                                                                    \
        void* temp, size_t temp_bytes, const KT* keys_in, KT* keys_out, const VT* values_in, VT* values_out,         \
        uint64_t n, uint64_t num_segments, const uint32_t* begin_offsets, const uint32_t* end_offsets,              \
        uint32_t begin_bit, uint32_t end_bit, int descending, int value_order, void* stream) {                      \
        using K = Storage<KT>;                                                                                        \
        return segsort_entry<K, VT, true, kKindOf<KT>>(                                                               \
            "DeviceSegmentedSort::SortPairs", temp, temp_bytes, reinterpret_cast<const K*>(keys_in),                  \
            reinterpret_cast<K*>(keys_out), values_in, values_out, n, num_segments, begin_offsets, end_offsets,     \
            begin_bit, end_bit, descending, value_order, stream);                                                     \
    }                                                                                                                 \
    int lcpp_hip_segmented_sort_pairs_db_##KS##_##VS(                                                                 \
        KT* keys0, KT* keys1, int* key_selector, VT* values0, VT* values1, int* value_selector, uint64_t n,         \
        uint64_t num_segments, const uint32_t* begin_offsets, const uint32_t* end_offsets, uint32_t begin_bit,      \
        uint32_t end_bit, int descending, int value_order, void* stream) {                                          \
        using K = Storage<KT>;                                                                                        \
        return segsort_db<K, VT, true, kKindOf<KT>>(                                                                  \
            "DeviceSegmentedSort::SortPairs", reinterpret_cast<K*>(keys0), reinterpret_cast<K*>(keys1),             \
            key_selector, values0, values1, value_selector, n, num_segments, begin_offsets, end_offsets, begin_bit,  \
            end_bit, descending, value_order, stream);                                                                \
    }
#define LCPP_HIP_DEFINE_SEGSORT(KS, KT)                                                                               \
    int lcpp_hip_segmented_sort_keys_##KS(void* temp, size_t temp_bytes, const KT* keys_in, KT* keys_out,           \
                                          uint64_t n, uint64_t num_segments, const uint32_t* begin_offsets,         \
                                          const uint32_t* end_offsets, uint32_t begin_bit, uint32_t end_bit,        \
                                          int descending, int value_order, void* stream) {                          \
        using K = Storage<KT>;                                                                                        \
        return segsort_entry<K, uint32_t, false, kKindOf<KT>>(                                                        \
            "DeviceSegmentedSort::SortKeys", temp, temp_bytes, reinterpret_cast<const K*>(keys_in),                   \
            reinterpret_cast<K*>(keys_out), nullptr, nullptr, n, num_segments, begin_offsets, end_offsets,           \
            begin_bit, end_bit, descending, value_order, stream);                                                     \
    }                                                                                                                 \
    int lcpp_hip_segmented_sort_keys_db_##KS(KT* keys0, KT* keys1, int* key_selector, uint64_t n,                   \
                                             uint64_t num_segments, const uint32_t* begin_offsets,                  \
                                             const uint32_t* end_offsets, uint32_t begin_bit, uint32_t end_bit,     \
                                             int descending, int value_order, void* stream) {                       \
        using K = Storage<KT>;                                                                                        \
        return segsort_db<K, uint32_t, false, kKindOf<KT>>(                                                           \
            "DeviceSegmentedSort::SortKeys", reinterpret_cast<K*>(keys0), reinterpret_cast<K*>(keys1),              \
            key_selector, nullptr, nullptr, nullptr, n, num_segments, begin_offsets, end_offsets, begin_bit,        \
            end_bit, descending, value_order, stream);                                                                \
    }                                                                                                                 \
    LCPP_HIP_DEFINE_SEGSORT_PAIRS(KS, KT, v32, uint32_t)                                                              \
    LCPP_HIP_DEFINE_SEGSORT_PAIRS(KS, KT, v64, uint64_t)
LCPP_HIP_DEFINE_SEGSORT(u32, uint32_t)
LCPP_HIP_DEFINE_SEGSORT(i32, int32_t)
LCPP_HIP_DEFINE_SEGSORT(f32, float)
LCPP_HIP_DEFINE_SEGSORT(u64, uint64_t)
LCPP_HIP_DEFINE_SEGSORT(i64, int64_t)
LCPP_HIP_DEFINE_SEGSORT(f64, double)
#undef LCPP_HIP_DEFINE_SEGSORT
#undef LCPP_HIP_DEFINE_SEGSORT_PAIRS

}  // extern "C"
