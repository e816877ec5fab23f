// DeviceScan::ExclusiveScanByKey / InclusiveScanByKey (sum operator) and DeviceReduce::ReduceByKey
// (sum operator) for gfx950: single-pass decoupled look-back over run-segmented sums.
//
// Reference path: DeviceScan<>::ExclusiveSumByKey / InclusiveSumByKey / Exclusive- and
// InclusiveScanByKey (src/lcpp/device/device_scan.h:424-597) -> dispatch_scan_by_key (:993-1012) ->
// ScanByKeyModule (device/details/scan_by_key.h); DeviceReduce<>::ReduceByKey (device_reduce.h:
// 437-487) -> reduce_by_key_array (:1024-1153) -> ReduceByKeyModule (device/details/reduce_by_key.h).
// Both pair a run-head flag with each value (KeyValuePair<int, V>, common/util_type.h:17-21) and scan
// with the segmented operator over decoupled look-back tile states
// (device/details/single_pass_scan_operator.h).
//
// Semantics: item i starts a run when i == 0 or its key differs from key i-1; keys compare by bits
// under a caller mask ((a ^ b) & mask == 0 means equal; all-ones is plain equality, 1 is the
// reference test's parity equality).  Scan: exclusive out[i] = init + (sum of the run's items before
// i), out[head] = init; inclusive out[i] = (sum of the run's items up to i), plus init when one is
// given.  Reduce: unique_out[r] = first key of run r, aggregates_out[r] = sum of run r,
// num_runs_out[0] = runs (0 for n == 0).  Integer sums wrap.
//
// MI355X design
//   * Tile = 256 threads x R rows x 4 consecutive items per thread and row (R = 12 for 4-byte keys and
//     values in the scan, 15 in the reduce, 22 in the count mode: 12,288 / 15,360 / 22,528 items; fewer
//     for 8-byte types), every row a contiguous 1,024 items read (and, for the scan, written) with
//     16-byte vectors, all rows' loads in flight together; four workgroups per CU (three for the
//     reduce).  The key before a thread-row is the previous
//     lane's last key (DPP wave shift) or, for lane 0, the last key of the previous wave or row (a
//     small LDS table).
//   * State of a span of items: (heads, sum since the last head).  States combine as
//     (c1, s1) + (c2, s2) = (c1 + c2, c2 ? s2 : s1 + s2), which is associative.  Each thread folds a
//     row's 4 items serially, a DPP wave scan (the shared row_shr / row_bcast pattern) per row gives
//     the lanes' carries, and one more wave scan over the (row, wave) totals gives every (row, wave)
//     its carry inside the tile and the tile its aggregate.
//   * Tile states are 64-bit words with the status in the low half and 32 payload bits in the high
//     half.  Reduce-by-key: word 0 holds the head count, words 1.. the sum.  Scan-by-key needs only
//     a has-head flag, kept beside the status, so its state is just the sum words (one word for
//     4-byte values: half the look-back loads).  A reader accepts a state only when every
//     word shows the same published status, so each word is one relaxed agent-scope atomic (the 8
//     XCDs do not share an L2) and no fence is needed.  The owner publishes PARTIAL (tile 0:
//     INCLUSIVE) with plain stores from lane 0 of its last wave: a wave's vector memory operations
//     complete in issue order, so stores issued by wave 0 would delay its own look-back loads.
//   * Look-back: wave 0 reads 32 predecessors per step (one per lane).  Ballots find the newest
//     INCLUSIVE state (or tile 0) and, for the scan, the newest state with a head: the scan stops
//     there because older sums cannot reach this tile; ReduceByKey continues to an INCLUSIVE state
//     since run indices need the full head count.  Counts and sums reduce with DPP.  Meanwhile the
//     other waves store the scan outputs that need no prefix (a head lies before them in the tile).
//   * Forward progress never depends on dispatch order.  Each tile has a claim word (in an array
//     after the state slots).  A predecessor still unpublished after `spin_limit` polls is claimed
//     by compare-and-swap (OPEN -> HELPER), its state computed by the whole waiting workgroup row by
//     row with the owner's own arithmetic (the same float summation order) and published PARTIAL, then the claim is marked DONE with
//     release ordering.  The owner closes its claim word (OPEN -> OWNED) right after publishing and
//     looks at the result only after its look-back; if a helper got there first it waits for DONE
//     before publishing INCLUSIVE or storing outputs, so no PARTIAL store can land after its
//     INCLUSIVE ones and an in-place scan never overwrites input a helper still reads.
// Algorithmic traffic: scan n*(sizeof(K) + 2*sizeof(V)); reduce n*(sizeof(K) + sizeof(V)) plus
// runs*(sizeof(K) + sizeof(V)) written.
#include "common.hpp"

#include <algorithm>
#include "../../include/lcpp_hip.h"

namespace lcpp_hip {
namespace {

constexpr int kBkBlock = 256;
constexpr int kBkWaves = kBkBlock / kWave;
constexpr int kBkVec = 4;  // consecutive items per thread and row (one 16-byte vector of 4-byte items)
// Predecessor states wave 0 inspects per look-back step, one per lane.  Every poll of a step ends in a
// workgroup barrier, and a step waits for its window's unpublished entries up to the nearest stop, so
// windows shorter than the wave win (2^28 i32 keys / u32 values, runs of mean 64: ExclusiveSumByKey
// 0.604 ms with 64, 0.57-0.60 with 32, 0.58-0.59 with 16, 0.57-0.60 with 8, 0.60-0.62 with 4; ReduceByKey
// 0.437 / 0.405-0.424 / 0.413-0.416 / 0.431 / 0.476 ms; encode 0.252 / 0.251 / 0.254 / 0.266 / 0.299 ms).
constexpr int kBkWindow = 32;
// Workgroups per CU: the others' loads and stores cover one workgroup's look-back wait.  Four (at most 128
// VGPRs) for the scan and the count mode, three (at most 168) for the reduce, whose 15 rows outrun 11 rows
// at four (ReduceByKey 2^28: 0.418 against 0.426 ms; ExclusiveSumByKey 0.592 ms at 16 rows and three,
// 0.574 at 12 rows and four, 0.581 at 10 rows and four; with non-temporal output stores 0.533 at 12 rows,
// 0.531 at 10 and 0.549 at 14, which spills).
template <int MODE>
constexpr int kBkBlocksPerCu = MODE == 1 ? 3 : 4;
// Rows per tile: a thread's keys and values of every row are in flight together (4 * R * (sizeof(K) +
// sizeof(V)) / 4 VGPRs, 96 for 4-byte keys and values at 12 rows).  The scan keeps its values through
// the look-back; the reduce stages its run heads in LDS before it, so nothing of the rows stays live and
// 120 VGPRs of keys and values fit (15 rows of 4-byte keys and values; ReduceByKey 2^28 0.61 -> 0.49 ms
// against 10 rows kept in registers through the look-back; later 0.414 ms at 15 rows, 0.419 at 14 and 0.512
// at 16, which spills).
#ifndef LCPP_BK_SCAN_VGPRS
#define LCPP_BK_SCAN_VGPRS 96
#endif
#ifndef LCPP_BK_REDUCE_VGPRS
#define LCPP_BK_REDUCE_VGPRS 120
#endif
// Run lengths and unique items load keys only and keep no per-row scans, so four workgroups per CU fit:
// 22 rows of 4-byte keys, 11 of 8-byte keys (Encode / Unique 2^28 u32 in runs of 64: 0.242 / 0.237 ms at 22
// rows and four workgroups per CU, 0.247 / 0.242 at 20, 0.263 / 0.262 at 24, which spills, 0.262 / 0.259 at
// 16 rows and four, 0.255 / 0.253 at 28 rows and three;
// earlier, before the PARTIAL state was published ahead of the staging, 0.316 ms at 16 rows, 0.314 at 24,
// 0.303 at 28, three per CU).
#ifndef LCPP_BK_COUNT_VGPRS
#define LCPP_BK_COUNT_VGPRS 88
#endif
template <typename K, typename V, int MODE>
constexpr int kBkRows =
    MODE == 2 ? (LCPP_BK_COUNT_VGPRS / static_cast<int>(sizeof(K)) < 32 ? LCPP_BK_COUNT_VGPRS / static_cast<int>(sizeof(K)) : 32)
              : (MODE == 0 ? LCPP_BK_SCAN_VGPRS - (sizeof(V) == 8 ? 16 : 0) : LCPP_BK_REDUCE_VGPRS) /
                    static_cast<int>(sizeof(K) + sizeof(V));
// Runs a reduce tile stages in LDS (32 KiB of keys and sums).
template <typename K, typename V>
constexpr uint32_t kBkStageItems = 32768u / static_cast<uint32_t>(sizeof(K) + sizeof(V));
template <typename K, typename V, int MODE>
constexpr uint32_t kBkTileItems = static_cast<uint32_t>(kBkBlock * kBkVec * kBkRows<K, V, MODE>);

constexpr uint32_t kStInvalid = 0;
constexpr uint32_t kStPartial = 1;
constexpr uint32_t kStInclusive = 2;

// Claim word of a tile (a separate array after all state slots, so the slots the look-back reads
// stay densely packed).
constexpr uint64_t kClaimOpen = 0;    // nobody has closed or claimed the tile yet
constexpr uint64_t kClaimOwned = 1;   // the owner closed it: no helper will ever read its input
constexpr uint64_t kClaimHelper = 2;  // a helper is computing the tile's state from its input
constexpr uint64_t kClaimDone = 3;    // the helper's PARTIAL stores have all been performed

constexpr int kModeScan = 0;
constexpr int kModeReduce = 1;
// Reduce of implicit ones (V = uint32_t, no value input): run lengths, the unique items and their run
// count (DeviceRunLengthEncode::Encode; DeviceSelect::Unique when no lengths are asked for).
constexpr int kModeCount = 2;

// Look-back decisions broadcast from wave 0.
constexpr uint32_t kActDone = 0;
constexpr uint32_t kActAdvance = 1;
constexpr uint32_t kActWait = 2;
constexpr uint32_t kActHelp = 3;

template <typename V>
struct Seg {
    uint32_t count;  // run heads in the span
    V sum;           // the items from the span's last head on (all items if it has none) folded by Op
};

// The value operator Op is SumOp (the reference's SumOp), MinValueOp or MaxValueOp (MinOp / MaxOp):
// Op{}(a, b) and Op::identity<V>().
template <typename Op, typename V>
__device__ __forceinline__ V op_apply(V a, V b) {
    return static_cast<V>(Op{}(a, b));
}
template <typename Op, typename V>
__device__ __forceinline__ V op_identity() {
    return Op::template identity<V>();
}

// Op with its operands swapped: a wave reduction over lanes ordered newest first (the look-back's
// predecessor windows) then still folds older before newer, which decides ties of a min / max.
template <typename Op>
struct SwappedOp {
    template <typename T>
    __device__ __forceinline__ T operator()(T a, T b) const { return static_cast<T>(Op{}(b, a)); }
    template <typename T>
    __device__ __forceinline__ static constexpr T identity() { return Op::template identity<T>(); }
};

template <typename Op, typename V>
__device__ __forceinline__ Seg<V> seg_combine(Seg<V> older, Seg<V> newer) {
    Seg<V> r;
    r.count = older.count + newer.count;
    r.sum = newer.count != 0 ? newer.sum : op_apply<Op>(older.sum, newer.sum);
    return r;
}

template <typename V>
constexpr int kValueWords = static_cast<int>(sizeof(V) / 4);
// Words of a tile state.  Reduce-by-key keeps the head count in a word of its own (word 0) ahead
// of the sum words; scan-by-key only needs to know whether a span holds a head, which rides in bit 2
// of the status half of the first sum word, so a 4-byte sum makes a one-word state.
template <typename V, bool COUNTED>
constexpr int kStateWords = (COUNTED ? 1 : 0) + kValueWords<V>;

// Temp layout: tiles x state words, then one claim word per tile.
size_t state_bytes(uint64_t n, uint32_t tile_items, size_t value_bytes, bool counted) {
    return ceil_div(n, tile_items) * ((counted ? 2 : 1) + value_bytes / 4) * sizeof(uint64_t);
}

constexpr uint32_t kStatusMask = 3;
constexpr uint32_t kHeadFlag = 4;

__device__ __forceinline__ uint64_t state_word(uint32_t status, uint32_t payload) {
    return (static_cast<uint64_t>(payload) << 32) | status;
}

template <typename V>
__device__ __forceinline__ uint32_t value_part(V v, int w) {
    if constexpr (sizeof(V) == 4) {
        return __builtin_bit_cast(uint32_t, v);
    } else {
        return static_cast<uint32_t>(__builtin_bit_cast(uint64_t, v) >> (32 * w));
    }
}

// Publishes state `s` with `status` (by the owner, or by the helper that claimed the tile).
template <typename V, bool COUNTED>
__device__ __forceinline__ void publish_state(uint64_t* slot, uint32_t status, Seg<V> s) {
    if constexpr (COUNTED) {
#pragma unroll
        for (int w = 0; w < kValueWords<V>; ++w) atomic_store_agent(&slot[1 + w], state_word(status, value_part(s.sum, w)));
        atomic_store_agent(&slot[0], state_word(status, s.count));
    } else {
#pragma unroll
        for (int w = 1; w < kValueWords<V>; ++w) atomic_store_agent(&slot[w], state_word(status, value_part(s.sum, w)));
        atomic_store_agent(&slot[0], state_word(status | (s.count != 0 ? kHeadFlag : 0u), value_part(s.sum, 0)));
    }
}

// Reads a tile state; returns its status if every word carries the same published status
// (PARTIAL or INCLUSIVE), kStInvalid otherwise.  Without COUNTED, s.count is 1 when the span holds
// a head, else 0.
template <typename V, bool COUNTED>
__device__ __forceinline__ uint32_t read_state(const uint64_t* slot, Seg<V>& s) {
    constexpr int N = kStateWords<V, COUNTED>;
    constexpr int B = COUNTED ? 1 : 0;  // first sum word
    uint64_t w[N];
#pragma unroll
    for (int i = 0; i < N; ++i) w[i] = atomic_load_agent(&slot[i]);
    const uint32_t st = static_cast<uint32_t>(w[0]) & kStatusMask;
    bool ok = st == kStPartial || st == kStInclusive;
#pragma unroll
    for (int i = 1; i < N; ++i) ok = ok && (static_cast<uint32_t>(w[i]) & kStatusMask) == st;
    if constexpr (COUNTED) {
        s.count = static_cast<uint32_t>(w[0] >> 32);
    } else {
        s.count = (static_cast<uint32_t>(w[0]) & kHeadFlag) != 0 ? 1u : 0u;
    }
    if constexpr (sizeof(V) == 4) {
        s.sum = __builtin_bit_cast(V, static_cast<uint32_t>(w[B] >> 32));
    } else {
        s.sum = __builtin_bit_cast(V, (w[B + 1] & 0xFFFFFFFF00000000ull) | (w[B] >> 32));
    }
    return ok ? st : kStInvalid;
}

// One step of the wave scan: combine with the state DPP brings from an older lane (identity where
// the pattern has no source).
template <typename Op, int CTRL, int ROW_MASK, typename V>
__device__ __forceinline__ Seg<V> seg_dpp_step(Seg<V> x) {
    Seg<V> o;
    o.count = dpp_move_u32<CTRL, ROW_MASK>(0u, x.count);
    o.sum = dpp_move<CTRL, ROW_MASK>(op_identity<Op, V>(), x.sum);
    return seg_combine<Op>(o, x);
}

// Inclusive scan of a segmented state over the 64 lanes of a wave (row_shr / row_bcast pattern).
template <typename Op, typename V>
__device__ __forceinline__ Seg<V> wave_seg_scan(Seg<V> x) {
    x = seg_dpp_step<Op, dpp::kRowShr1, 0xf>(x);
    x = seg_dpp_step<Op, dpp::kRowShr2, 0xf>(x);
    x = seg_dpp_step<Op, dpp::kRowShr4, 0xf>(x);
    x = seg_dpp_step<Op, dpp::kRowShr8, 0xf>(x);
    x = seg_dpp_step<Op, dpp::kRowBcast15, 0xa>(x);
    x = seg_dpp_step<Op, dpp::kRowBcast31, 0xc>(x);
    return x;
}

// The previous lane's inclusive state (identity in lane 0).
template <typename Op, typename V>
__device__ __forceinline__ Seg<V> wave_seg_exclusive(Seg<V> inclusive) {
    Seg<V> e;
    e.count = dpp_move_u32<dpp::kWaveShr1>(0u, inclusive.count);
    e.sum = dpp_move<dpp::kWaveShr1>(op_identity<Op, V>(), inclusive.sum);
    return e;
}

// Items [first, first + 4) of `p`, in range, 16-byte aligned: one (or, for 8-byte items, two) vector loads.
template <typename T>
__device__ __forceinline__ void load_quad_vec(const T* p, uint64_t first, T (&out)[kBkVec]) {
    typedef T Vec __attribute__((ext_vector_type(kBkVec), aligned(16)));
    const Vec q = __builtin_nontemporal_load(reinterpret_cast<const Vec*>(p + first));
#pragma unroll
    for (int k = 0; k < kBkVec; ++k) out[k] = q[k];
}

// Items [first, first + 4) of `p`, 0 past n, any alignment.
template <typename T>
__device__ __forceinline__ void load_quad_any(const T* p, uint64_t first, uint64_t n, T (&out)[kBkVec]) {
#pragma unroll
    for (int k = 0; k < kBkVec; ++k) out[k] = first + k < n ? p[first + k] : T(0);
}

template <typename T>
__device__ __forceinline__ void load_quad(const T* p, uint64_t first, uint64_t n, bool vec, T (&out)[kBkVec]) {
    if (vec && first + kBkVec <= n) load_quad_vec(p, first, out);
    else load_quad_any(p, first, n, out);
}

// Stores the items of `valid` (bit k: item first + k exists) of a thread-row: one non-temporal vector
// store when all four exist and the array is 16-byte aligned.  The lanes of a row store consecutive 16-byte
// vectors, so every instruction covers whole lines (ExclusiveSumByKey 2^28 i32 / u32: 0.581 -> 0.533 ms
// per call against plain stores; non-temporal stores of single items measured slower in compaction).
template <typename T>
__device__ __forceinline__ void store_quad(T* p, uint64_t first, uint32_t valid, bool vec, const T (&in)[kBkVec]) {
    if (vec && valid == 0xFu) {
        typedef T Vec __attribute__((ext_vector_type(kBkVec), aligned(16)));
        Vec q;
#pragma unroll
        for (int k = 0; k < kBkVec; ++k) q[k] = in[k];
        __builtin_nontemporal_store(q, reinterpret_cast<Vec*>(p + first));
    } else {
#pragma unroll
        for (int k = 0; k < kBkVec; ++k) {
            if ((valid >> k) & 1u) p[first + k] = in[k];
        }
    }
}

// Bit k set when item first + k < n.
__device__ __forceinline__ uint32_t quad_valid(uint64_t first, uint64_t n) {
    return first >= n ? 0u : (n - first >= kBkVec ? 0xFu : (1u << static_cast<uint32_t>(n - first)) - 1u);
}

// Adjacent keys differ: integers on the masked bits, floats by value (-0.0 == +0.0, a NaN differs from
// everything), as the reference's lhs == rhs does.
template <typename K>
__device__ __forceinline__ bool keys_differ(K a, K b, K mask) {
    if constexpr (std::is_floating_point_v<K>) {
        (void)mask;
        return !(a == b);
    } else {
        return ((a ^ b) & mask) != 0;
    }
}

// Values of a thread-row: loaded, or implicit ones (kModeCount).
template <int MODE, typename V>
__device__ __forceinline__ void load_values(const V* p, uint64_t first, uint64_t n, bool vec, V (&out)[kBkVec]) {
    if constexpr (MODE == kModeCount) {
#pragma unroll
        for (int k = 0; k < kBkVec; ++k) out[k] = V(1);
    } else {
        load_quad(p, first, n, vec, out);
    }
}

// Head bits (bit k: item first + k starts a run) of a thread-row, given the key before it; `at_start`:
// the row's first item is item 0.
template <typename K>
__device__ __forceinline__ uint32_t quad_heads(const K (&key)[kBkVec], K prev, uint32_t valid, bool at_start, K mask) {
    uint32_t heads = 0;
#pragma unroll
    for (int k = 0; k < kBkVec; ++k) {
        const bool head = (k == 0 && at_start) || keys_differ(key[k], prev, mask);
        heads |= (head ? 1u : 0u) << k;
        prev = key[k];
    }
    return heads & valid;
}

// State of a thread-row: its items folded in order.
template <typename Op, typename V>
__device__ __forceinline__ Seg<V> fold_quad(const V (&val)[kBkVec], uint32_t heads, uint32_t valid) {
    Seg<V> s{0u, op_identity<Op, V>()};
#pragma unroll
    for (int k = 0; k < kBkVec; ++k) {
        const bool head = (heads >> k) & 1u;
        const V x = ((valid >> k) & 1u) ? val[k] : op_identity<Op, V>();
        s.count += head ? 1u : 0u;
        s.sum = head ? x : op_apply<Op>(s.sum, x);
    }
    return s;
}

// Item index of thread `tid`'s first item in row r of a tile.
template <int R>
__device__ __forceinline__ uint64_t row_first(uint32_t tile, int r, uint32_t tid) {
    return static_cast<uint64_t>(tile) * (kBkBlock * kBkVec * R) + static_cast<uint64_t>(r) * (kBkBlock * kBkVec) +
           static_cast<uint64_t>(tid) * kBkVec;
}

// Carries and aggregate from the (row, wave) totals, by wave 0: lane l takes total l (row l / 4, wave
// l % 4) when R * 4 <= 64, else P = ceil(R * 4 / 64) consecutive totals folded in order; one wave scan gives
// every (row, wave) its in-tile carry (the totals before it, in row-major order), written back over
// the table, and lane 63 the tile aggregate, which wave 0 returns.
template <typename Op, typename V, int R>
__device__ __forceinline__ Seg<V> scan_totals(Seg<V> (*s_wave)[kBkWaves]) {
    constexpr int E = R * kBkWaves;
    constexpr int P = (E + kWave - 1) / kWave;
    const uint32_t lane = lane_id();
    Seg<V>* flat = &s_wave[0][0];
    Seg<V> incl;
    if constexpr (P == 1) {
        const Seg<V> t = lane < static_cast<uint32_t>(E) ? flat[lane] : Seg<V>{0u, op_identity<Op, V>()};
        incl = wave_seg_scan<Op>(t);
        if (lane < static_cast<uint32_t>(E)) flat[lane] = wave_seg_exclusive<Op>(incl);
    } else {
        const uint32_t first = lane * P;
        Seg<V> t = first < static_cast<uint32_t>(E) ? flat[first] : Seg<V>{0u, op_identity<Op, V>()};
#pragma unroll
        for (int p = 1; p < P; ++p)
            if (first + p < static_cast<uint32_t>(E)) t = seg_combine<Op>(t, flat[first + p]);
        incl = wave_seg_scan<Op>(t);
        Seg<V> run = wave_seg_exclusive<Op>(incl);
#pragma unroll
        for (int p = 0; p < P; ++p) {
            if (first + p < static_cast<uint32_t>(E)) {
                const Seg<V> x = flat[first + p];
                flat[first + p] = run;
                run = seg_combine<Op>(run, x);
            }
        }
    }
    Seg<V> agg;
    agg.count = wave_read_lane(incl.count, kWave - 1);
    agg.sum = wave_read_lane(incl.sum, kWave - 1);
    return agg;
}

// Aggregate of tile `tile`, computed by the whole workgroup with the owner's own arithmetic (same
// heads, folds, wave scans and combination order, so float sums match bit for bit).  Row by row, with
// the key before each thread-row read from memory, to keep the helper's registers small.
template <typename Op, typename K, typename V, int MODE, int R>
__device__ Seg<V> tile_aggregate(const K* keys, const V* values, uint64_t n, uint32_t tile, K mask, bool vec_k,
                                 bool vec_v, Seg<V> (*s_help)[kBkWaves]) {
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid / kWave;
#pragma unroll 1
    for (int r = 0; r < R; ++r) {
        const uint64_t first = row_first<R>(tile, r, tid);
        K key[kBkVec];
        V val[kBkVec];
        load_quad(keys, first, n, vec_k, key);
        load_values<MODE>(values, first, n, vec_v, val);
        const K prev = (first > 0 && first - 1 < n) ? keys[first - 1] : K(0);
        const uint32_t valid = quad_valid(first, n);
        const Seg<V> incl = wave_seg_scan<Op>(fold_quad<Op>(val, quad_heads(key, prev, valid, first == 0, mask), valid));
        if (lane_id() == kWave - 1) s_help[r][wave] = incl;
    }
    __syncthreads();
    // Only thread 0 publishes the helped state, so wave 0's result is all that is needed.
    Seg<V> agg{0u, op_identity<Op, V>()};
    if (wave == 0) agg = scan_totals<Op, V, R>(s_help);
    __syncthreads();  // s_help is free again
    return agg;
}

// Outputs of one thread-row of a scan from the state carried into its first item.
template <typename Op, typename V>
__device__ __forceinline__ void scan_quad_outputs(const V (&val)[kBkVec], uint32_t heads, Seg<V> run, int inclusive,
                                                  int use_init, V init, V* values_out, uint64_t first, uint32_t valid,
                                                  bool vec_o) {
    V out[kBkVec];
#pragma unroll
    for (int k = 0; k < kBkVec; ++k) {
        const bool head = (heads >> k) & 1u;
        if (!inclusive) out[k] = head ? init : op_apply<Op>(init, run.sum);
        if (head) {
            run.count += 1;
            run.sum = val[k];
        } else {
            run.sum = op_apply<Op>(run.sum, val[k]);
        }
        if (inclusive) out[k] = use_init ? op_apply<Op>(init, run.sum) : run.sum;
    }
    store_quad(values_out, first, valid, vec_o, out);
}

// Reduce outputs of a tile with more runs than the LDS stage holds, after its look-back: each row is
// read again and folded exactly as before (heads from the edge table, the same wave scans), and every
// run head writes its key and the sum of the run before it.
template <typename Op, typename K, typename V, int MODE, int R>
__device__ void reduce_rows_direct(const K* keys, const V* values, K* unique_out, V* aggregates_out,
                                   uint32_t* num_runs_out, uint64_t n, K mask, uint32_t tile, Seg<V> prefix,
                                   Seg<V> (*s_wave)[kBkWaves], K (*s_edge)[kBkWaves], bool vec_k, bool vec_v) {
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint64_t tile_base = static_cast<uint64_t>(tile) * (kBkBlock * kBkVec * R);
    const K before_tile = (tid == 0 && tile_base > 0) ? keys[tile_base - 1] : K(0);
#pragma unroll 1
    for (int r = 0; r < R; ++r) {
        const uint64_t first = row_first<R>(tile, r, tid);
        K key[kBkVec];
        V val[kBkVec];
        load_quad(keys, first, n, vec_k, key);
        load_values<MODE>(values, first, n, vec_v, val);
        K prev = dpp_move<dpp::kWaveShr1>(K(0), key[kBkVec - 1]);
        if (lane == 0) prev = wave > 0 ? s_edge[r][wave - 1] : (r > 0 ? s_edge[r - 1][kBkWaves - 1] : before_tile);
        const uint32_t valid = quad_valid(first, n);
        const uint32_t h = quad_heads(key, prev, valid, tile == 0 && r == 0 && tid == 0, mask);
        const Seg<V> incl = wave_seg_scan<Op>(fold_quad<Op>(val, h, valid));
        Seg<V> run = seg_combine<Op>(prefix, seg_combine<Op>(s_wave[r][wave], wave_seg_exclusive<Op>(incl)));
#pragma unroll
        for (int k = 0; k < kBkVec; ++k) {
            if ((valid >> k) & 1u) {
                if ((h >> k) & 1u) {
                    if (run.count > 0 && aggregates_out) aggregates_out[run.count - 1] = run.sum;
                    unique_out[run.count] = key[k];
                    run.count += 1;
                    run.sum = val[k];
                } else {
                    run.sum = op_apply<Op>(run.sum, val[k]);
                }
            }
        }
        if (valid != 0 && n - first <= kBkVec) {  // this thread-row holds the last item
            if (aggregates_out) aggregates_out[run.count - 1] = run.sum;
            num_runs_out[0] = run.count;
        }
    }
}

template <typename K, typename V, int MODE, int R, typename Op>
__global__ __launch_bounds__(kBkBlock, kBkBlocksPerCu<MODE>) void by_key_kernel(
    const K* __restrict__ keys, const V* values_in, V* values_out, K* __restrict__ unique_out,
    V* __restrict__ aggregates_out, uint32_t* __restrict__ num_runs_out, uint64_t n, K mask,
    uint64_t* __restrict__ states, int inclusive, int use_init, V init, bool vec_k, bool vec_v, bool vec_o,
    bool in_place, uint32_t spin_limit) {
    constexpr bool COUNTED = MODE != kModeScan;
    constexpr int W = kStateWords<V, COUNTED>;
    uint64_t* const claims = states + static_cast<uint64_t>(gridDim.x) * W;
    // The thread that publishes this tile's states and closes its claim word: lane 0 of the last
    // wave.  A wave's vector memory operations complete in issue order, so publishing from wave 0
    // would make its look-back loads wait for the publishing stores and the compare-and-swap.
    constexpr uint32_t kPublisher = kBkBlock - kWave;
    __shared__ Seg<V> s_wave[R][kBkWaves];  // (row, wave) totals of this tile, then their in-tile carries
    __shared__ Seg<V> s_help[R][kBkWaves];  // the same for a tile this workgroup computes as a helper
    __shared__ K s_edge[R][kBkWaves];       // last key of each (row, wave)
    __shared__ uint32_t s_ctl[2][2];        // look-back decision and helped tile, two alternating rows
    __shared__ Seg<V> s_prefix;
    __shared__ Seg<V> s_agg;
    // Reduce: the tile's run heads in order (key, and the sum of the items before the head back to the
    // previous head in the tile, or to the tile's start for the first), staged before the look-back.
    constexpr uint32_t kStage = MODE != kModeScan ? kBkStageItems<K, V> : 1u;
    __shared__ K s_run_key[kStage];
    __shared__ V s_run_sum[kStage];

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint64_t tile_base = static_cast<uint64_t>(tile) * (kBkBlock * kBkVec * R);

    // Load every row (row r: 4 KiB of keys and of values per 1,024 items, thread t the t-th quad).  A
    // full, aligned tile takes only unconditional vector loads, so all of them are in flight together.
    constexpr uint32_t TILE = kBkBlock * kBkVec * R;
    const bool full = vec_k && vec_v && tile_base + TILE <= n;
    K key[R][kBkVec];
    V val[R][kBkVec];
    if (full) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            load_quad_vec(keys, row_first<R>(tile, r, tid), key[r]);
            if constexpr (MODE == kModeCount) load_values<MODE>(values_in, 0, 0, true, val[r]);
            else load_quad_vec(values_in, row_first<R>(tile, r, tid), val[r]);
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            load_quad_any(keys, row_first<R>(tile, r, tid), n, key[r]);
            load_values<MODE>(values_in, row_first<R>(tile, r, tid), n, false, val[r]);
        }
    }
    const K before_tile = (tid == 0 && tile_base > 0) ? keys[tile_base - 1] : K(0);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (lane == kWave - 1) s_edge[r][wave] = key[r][kBkVec - 1];
    }
    __syncthreads();

    // Heads (the key before a thread-row: the previous lane's last key, across waves and rows through
    // the edge table), folds and per-row wave scans.
    uint32_t heads[(R + 7) / 8];  // four bits per row
#pragma unroll
    for (int i = 0; i < (R + 7) / 8; ++i) heads[i] = 0;
    // Run lengths (kModeCount) need no per-row scan: a wave-row's state is its head count and the
    // items after its last head, both read off four ballots of the head bits.
    constexpr bool kBallotRuns = MODE == kModeCount;
    Seg<V> incl[kBallotRuns ? 1 : R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        K prev = dpp_move<dpp::kWaveShr1>(K(0), key[r][kBkVec - 1]);
        if (lane == 0) prev = wave > 0 ? s_edge[r][wave - 1] : (r > 0 ? s_edge[r - 1][kBkWaves - 1] : before_tile);
        const uint32_t valid = full ? 0xFu : quad_valid(row_first<R>(tile, r, tid), n);
        const uint32_t h = quad_heads(key[r], prev, valid, tile == 0 && r == 0 && tid == 0, mask);
        heads[r / 8] |= h << (4 * (r % 8));
        if constexpr (kBallotRuns) {
            // Heads of the wave-row, and the item index of its last head (the state's sum counts the
            // items from that head on; all items when there is none).
            uint32_t count = 0, last = 0;
#pragma unroll
            for (int k = 0; k < kBkVec; ++k) {
                const uint64_t b = wave_ballot((h >> k) & 1u);
                count += static_cast<uint32_t>(__builtin_popcountll(b));
                if (b != 0) last = max(last, 4u * (63u - static_cast<uint32_t>(__builtin_clzll(b))) + k);
            }
            if (lane == 0) {
                const uint64_t row_base = row_first<R>(tile, r, wave * kWave);
                const uint32_t items = row_base >= n ? 0u : static_cast<uint32_t>(min<uint64_t>(n - row_base, kWave * kBkVec));
                s_wave[r][wave] = Seg<V>{count, static_cast<V>(count != 0 ? items - last : items)};
            }
        } else {
            incl[r] = wave_seg_scan<Op>(fold_quad<Op>(val[r], h, valid));
            if (lane == kWave - 1) s_wave[r][wave] = incl[r];
        }
    }
    __syncthreads();
    // Wave 0 turns the totals into in-tile carries and the aggregate (to LDS for the publisher).
    if (wave == 0) {
        const Seg<V> a = scan_totals<Op, V, R>(s_wave);
        if (lane == 0) s_agg = a;
    }
    __syncthreads();
    const Seg<V> agg = s_agg;

    // Publish PARTIAL (INCLUSIVE for tile 0) with plain stores, then close the claim word; the
    // compare-and-swap's result is only needed after the look-back.  A helper that claimed the tile
    // first stores the same PARTIAL values.  Before the reduce's staging, so successors see it sooner.
    uint64_t* const my_slot = states + static_cast<uint64_t>(tile) * W;
    bool owned = true;
    if (tid == kPublisher) {
        const uint32_t st = tile == 0 ? kStInclusive : kStPartial;
        publish_state<V, COUNTED>(my_slot, st, agg);
        uint64_t expected = kClaimOpen;
        owned = __hip_atomic_compare_exchange_strong(&claims[tile], &expected, kClaimOwned, __ATOMIC_RELAXED,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Reduce: a tile of at most kStage runs stages its outputs in LDS now, so its keys and values are
    // dead during the look-back and the outputs leave as contiguous stores; a tile of more runs reads
    // its rows again after the look-back (reduce_rows_direct).
    const bool staged = MODE != kModeScan && agg.count <= kStage;
    if constexpr (kBallotRuns) {
        // Run heads in order: the wave-row's carry, the heads of lower lanes (ballot ranks) and of the
        // quad's lower items.  Staged: key and tile-local position (lengths are position differences).
        if (staged) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t h = (heads[r / 8] >> (4 * (r % 8))) & 0xFu;
                uint32_t idx = s_wave[r][wave].count;
#pragma unroll
                for (int k = 0; k < kBkVec; ++k) idx += popc_lanes_below(wave_ballot((h >> k) & 1u));
                const uint32_t pos = static_cast<uint32_t>(r) * (kBkBlock * kBkVec) + tid * kBkVec;
#pragma unroll
                for (int k = 0; k < kBkVec; ++k) {
                    if ((h >> k) & 1u) {
                        s_run_key[idx] = key[r][k];
                        s_run_sum[idx] = static_cast<V>(pos + k);
                        ++idx;
                    }
                }
            }
        }
    } else if constexpr (MODE != kModeScan) {
        if (staged) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                Seg<V> run = seg_combine<Op>(s_wave[r][wave], wave_seg_exclusive<Op>(incl[r]));
                const uint32_t h = (heads[r / 8] >> (4 * (r % 8))) & 0xFu;
                const uint32_t valid = full ? 0xFu : quad_valid(row_first<R>(tile, r, tid), n);
#pragma unroll
                for (int k = 0; k < kBkVec; ++k) {
                    if ((valid >> k) & 1u) {
                        if ((h >> k) & 1u) {
                            s_run_key[run.count] = key[r][k];
                            s_run_sum[run.count] = run.sum;
                            run.count += 1;
                            run.sum = val[r][k];
                        } else {
                            run.sum = op_apply<Op>(run.sum, val[r][k]);
                        }
                    }
                }
            }
        }
    }

    // In-tile carry into each thread-row: rows before it, waves before it in its row, lanes before it.
    // Scan outputs whose carry already holds a head (or whose first item is one) do not depend on the
    // tile's prefix; waves other than wave 0 store them now, while wave 0 walks the look-back (a
    // wave's vector memory operations complete in issue order).  Not for in-place scans: their input
    // may still be read by a helper until the claim is settled.
    uint32_t stored = 0;  // rows already stored
    if constexpr (MODE == kModeScan) {
        if (!in_place && wave != 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const Seg<V> carry = seg_combine<Op>(s_wave[r][wave], wave_seg_exclusive<Op>(incl[r]));
                const uint32_t h = (heads[r / 8] >> (4 * (r % 8))) & 0xFu;
                if (carry.count != 0 || (h & 1u) != 0) {
                    const uint64_t first = row_first<R>(tile, r, tid);
                    scan_quad_outputs<Op>(val[r], h, carry, inclusive, use_init, init, values_out, first,
                                      full ? 0xFu : quad_valid(first, n), vec_o);
                    stored |= 1u << r;
                }
            }
        }
    }

    Seg<V> prefix{0u, op_identity<Op, V>()};
    if (tile > 0) {
        int64_t top = static_cast<int64_t>(tile) - 1;  // newest predecessor not yet consumed
        Seg<V> acc{0u, op_identity<Op, V>()};           // states consumed so far (wave 0)
        uint32_t spins = 0;
        uint32_t row = 0;
        while (true) {
            if (wave == 0) {
                const int64_t j = top - static_cast<int64_t>(lane);
                Seg<V> s{0u, op_identity<Op, V>()};
                const bool exists = j >= 0 && lane < static_cast<uint32_t>(kBkWindow);
                const uint32_t st = exists ? read_state<V, COUNTED>(states + static_cast<uint64_t>(j) * W, s) : kStInvalid;
                const bool published = st != kStInvalid;
                // A complete prefix: an INCLUSIVE state, or tile 0 (nothing precedes it).
                const uint64_t stop_mask = wave_ballot(published && (st == kStInclusive || j == 0));
                uint32_t cut = stop_mask ? static_cast<uint32_t>(__builtin_ctzll(stop_mask)) : kWave - 1;
                const uint64_t head_mask = wave_ballot(published && s.count != 0);
                if constexpr (MODE == kModeScan) {
                    if (head_mask) cut = min(cut, static_cast<uint32_t>(__builtin_ctzll(head_mask)));
                }
                const uint64_t upto = cut >= kWave - 1 ? ~0ull : ((2ull << cut) - 1);
                const uint64_t missing = upto & wave_ballot(exists) & ~wave_ballot(published);
                uint32_t action;
                uint32_t help_tile = 0;
                if (missing) {
                    if (spins >= spin_limit) {
                        action = kActHelp;
                        help_tile = static_cast<uint32_t>(top - __builtin_ctzll(missing));
                    } else {
                        action = kActWait;
                    }
                } else {
                    const bool take = exists && lane <= cut;
                    // Sum of the lanes from the newest up to the newest head (or the cut).
                    const uint64_t heads_in = head_mask & upto;
                    const uint32_t sum_cut = heads_in ? min(cut, static_cast<uint32_t>(__builtin_ctzll(heads_in))) : cut;
                    Seg<V> window;
                    window.count = wave_reduce(take ? s.count : 0u, SumOp{});
                    window.sum = wave_reduce((exists && lane <= sum_cut) ? s.sum : op_identity<Op, V>(), SwappedOp<Op>{});
                    acc = seg_combine<Op>(window, acc);
                    const bool complete = stop_mask != 0 && cut == static_cast<uint32_t>(__builtin_ctzll(stop_mask));
                    const bool found_head = MODE == kModeScan && heads_in != 0;
                    action = (complete || found_head || top < kBkWindow) ? kActDone : kActAdvance;
                }
                if (lane == 0) {
                    s_ctl[row][0] = action;
                    s_ctl[row][1] = help_tile;
                    if (action == kActDone) s_prefix = acc;
                }
            }
            __syncthreads();
            const uint32_t action = s_ctl[row][0];
            const uint32_t help_tile = s_ctl[row][1];
            row ^= 1u;
            if (action == kActDone) break;
            if (action == kActAdvance) {
                top -= kBkWindow;
                spins = 0;
                continue;
            }
            if (action == kActWait) {
                __builtin_amdgcn_s_sleep(1);
                ++spins;
                continue;
            }
            // kActHelp: claim the unpublished predecessor, compute its state, publish it PARTIAL, and
            // mark the claim DONE with release ordering (after every PARTIAL store is performed).
            uint64_t* const slot = states + static_cast<uint64_t>(help_tile) * W;
            if (tid == 0) {
                uint64_t expected = kClaimOpen;
                s_ctl[row][0] = __hip_atomic_compare_exchange_strong(&claims[help_tile], &expected, kClaimHelper,
                                                                     __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                                     __HIP_MEMORY_SCOPE_AGENT)
                                    ? 1u
                                    : 0u;
            }
            __syncthreads();
            const bool claimed = s_ctl[row][0] != 0;
            row ^= 1u;
            if (claimed) {
                const Seg<V> h = tile_aggregate<Op, K, V, MODE, R>(keys, values_in, n, help_tile, mask, vec_k, vec_v, s_help);
                if (tid == 0) {
                    publish_state<V, COUNTED>(slot, kStPartial, h);
                    __hip_atomic_store(&claims[help_tile], kClaimDone, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            spins = 0;
        }
        prefix = s_prefix;
    }

    // A tile a helper claimed first: wait until the helper is DONE, so none of its PARTIAL stores can
    // land after the INCLUSIVE ones and no input it reads is overwritten (in-place scans).  Then
    // publish this tile's INCLUSIVE state (tile 0's initial state already was, unless helped).
    if (tid == kPublisher) {
        if (!owned) {
            while (__hip_atomic_load(&claims[tile], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) != kClaimDone)
                __builtin_amdgcn_s_sleep(1);
        }
        if (tile > 0 || !owned) {
            const Seg<V> incl_state = seg_combine<Op>(prefix, agg);
            publish_state<V, COUNTED>(my_slot, kStInclusive, incl_state);
        }
    }
    __syncthreads();  // outputs only after the claim is settled

    if constexpr (MODE == kModeScan) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const Seg<V> run = seg_combine<Op>(prefix, seg_combine<Op>(s_wave[r][wave], wave_seg_exclusive<Op>(incl[r])));
            const uint32_t h = (heads[r / 8] >> (4 * (r % 8))) & 0xFu;
            const uint64_t first = row_first<R>(tile, r, tid);
            if (((stored >> r) & 1u) == 0)
                scan_quad_outputs<Op>(val[r], h, run, inclusive, use_init, init, values_out, first,
                                  full ? 0xFu : quad_valid(first, n), vec_o);
        }
    } else if (staged) {
        // Run i of the tile is run prefix.count + i overall; the run before the tile's first head
        // began in an earlier tile (none before item 0) and takes the prefix's sum.
        const uint32_t base = prefix.count;
        for (uint32_t i = tid; i < agg.count; i += kBkBlock) {
            unique_out[base + i] = s_run_key[i];
            if (aggregates_out) {
                // Run lengths: staged positions (differences of consecutive heads) for kModeCount.
                const V before = i > 0 ? (kBallotRuns ? static_cast<V>(s_run_sum[i] - s_run_sum[i - 1]) : s_run_sum[i])
                                       : op_apply<Op>(prefix.sum, s_run_sum[0]);
                if (i > 0 || base > 0) aggregates_out[base + i - 1] = before;
            }
        }
        if (tid == 0 && tile_base + TILE >= n) {  // the tile holding the last item closes the last run
            const Seg<V> total = seg_combine<Op>(prefix, agg);
            if (aggregates_out) aggregates_out[total.count - 1] = total.sum;
            num_runs_out[0] = total.count;
        }
    } else {
        reduce_rows_direct<Op, K, V, MODE, R>(keys, values_in, unique_out, aggregates_out, num_runs_out, n, mask, tile, prefix,
                                    s_wave, s_edge, vec_k, vec_v);
    }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

bool ranges_overlap(const void* a, uint64_t a_bytes, const void* b, uint64_t b_bytes) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return a_bytes != 0 && b_bytes != 0 && x < y + b_bytes && y < x + a_bytes;
}

template <typename K, typename V, int MODE, typename Op = SumOp>
int by_key(void* temp, size_t temp_bytes, const K* keys, const V* values_in, V* values_out, K* unique_out,
           V* aggregates_out, uint32_t* num_runs_out, uint64_t n, uint64_t key_mask, int inclusive, int use_init,
           V init, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const char* what = MODE == kModeScan     ? "DeviceScan::ScanByKey"
                       : MODE == kModeReduce ? "DeviceReduce::ReduceByKey"
                                             : "DeviceRunLengthEncode::Encode";
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items", what);
    if constexpr (MODE != kModeScan) {
        if (!num_runs_out) return set_error(kInvalidArgument, "%s: null run-count output", what);
        if (n == 0) return launch_fill_u32(num_runs_out, 1, 0u, stream);
        if (!unique_out || (MODE == kModeReduce && !aggregates_out)) return set_error(kInvalidArgument, "%s: null output", what);
    } else {
        if (n == 0) return kOk;
        if (!values_out) return set_error(kInvalidArgument, "%s: null output", what);
    }
    if (!keys || (MODE != kModeCount && !values_in)) return set_error(kInvalidArgument, "%s: null input", what);
    if constexpr (MODE != kModeScan) {
        // A tile with more runs than its LDS stage reads its input again after its look-back, when later
        // tiles may already be writing runs, so outputs must not overlap the inputs.  An output holds as
        // many items as there are runs, which only the kernel learns; the host rejects what must overlap
        // whatever that count is: an output whose first item (always written, n > 0) lies inside an input.
        // An output that starts below an input and is as long as the run count never reaches it.
        const uint64_t out_bytes[2] = {sizeof(K), aggregates_out ? sizeof(V) : 0};
        const uint64_t in_bytes[2] = {n * sizeof(K), MODE == kModeReduce ? n * sizeof(V) : 0};
        const void* outs[2] = {unique_out, aggregates_out};
        const void* ins[2] = {keys, values_in};
        for (int o = 0; o < 2; ++o)
            for (int i = 0; i < 2; ++i)
                if (ranges_overlap(outs[o], out_bytes[o], ins[i], in_bytes[i]))
                    return set_error(kInvalidArgument, "%s: outputs must not overlap the inputs", what);
    }
    constexpr uint32_t kTile = kBkTileItems<K, V, MODE>;
    const size_t need = state_bytes(n, kTile, sizeof(V), MODE != kModeScan);
    if (!temp || temp_bytes < need)
        return set_error(kTempTooSmall, "%s: temp storage too small (%zu < %zu bytes)", what, temp_bytes, need);
    if (reinterpret_cast<uintptr_t>(temp) % 8 != 0) return set_error(kInvalidArgument, "%s: temp not 8-byte aligned", what);
    uint64_t* states = static_cast<uint64_t*>(temp);
    int st = launch_fill_u32(reinterpret_cast<uint32_t*>(states), need / 4, 0u, stream);
    if (st != kOk) return st;
    const uint32_t tiles = static_cast<uint32_t>(ceil_div(n, kTile));
    LaunchScope scope(MODE == kModeScan ? "scan_by_key" : MODE == kModeReduce ? "reduce_by_key" : "runs_by_key", stream);
    by_key_kernel<K, V, MODE, kBkRows<K, V, MODE>, Op><<<tiles, kBkBlock, 0, stream>>>(
        keys, values_in, values_out, unique_out, aggregates_out, num_runs_out, n, static_cast<K>(key_mask), states,
        inclusive, use_init, init, aligned16(keys), aligned16(values_in), values_out != nullptr && aligned16(values_out),
        values_out != nullptr && values_out == values_in, lookback_spin_limit());
    return check_hip(hipGetLastError(), MODE == kModeScan ? "scan_by_key launch" : "reduce_by_key launch");
}

}  // namespace

// Run-length encode (counts_out non-null) or unique (counts_out null) over the by-key reduce kernels
// with implicit ones: keys compare on the masked bits (integers) or by value (floats).  Returns
// kRunsDeclined without doing anything when the outputs overlap the input (in-place forms) or the
// temp storage is smaller than the tile states, so the caller can take its general path.
template <typename K>
int runs_by_key(void* temp, size_t temp_bytes, const K* in, K* unique_out, uint32_t* counts_out, uint32_t* num_out,
                uint64_t n, uint64_t key_mask, hipStream_t stream) {
    if (n > 0 && n <= 0xFFFFFFFFull) {
        const size_t need = state_bytes(n, kBkTileItems<K, uint32_t, kModeCount>, sizeof(uint32_t), true);
        if (!temp || temp_bytes < need || ranges_overlap(unique_out, n * sizeof(K), in, n * sizeof(K)) ||
            ranges_overlap(counts_out, counts_out ? n * 4 : 0, in, n * sizeof(K)))
            return kRunsDeclined;
    }
    return by_key<K, uint32_t, kModeCount>(temp, temp_bytes, in, nullptr, nullptr, unique_out, counts_out, num_out, n,
                                           key_mask, 0, 0, 0u, stream);
}
template int runs_by_key<uint32_t>(void*, size_t, const uint32_t*, uint32_t*, uint32_t*, uint32_t*, uint64_t, uint64_t,
                                   hipStream_t);
template int runs_by_key<uint64_t>(void*, size_t, const uint64_t*, uint64_t*, uint32_t*, uint32_t*, uint64_t, uint64_t,
                                   hipStream_t);
template int runs_by_key<float>(void*, size_t, const float*, float*, uint32_t*, uint32_t*, uint64_t, uint64_t,
                                hipStream_t);
template int runs_by_key<double>(void*, size_t, const double*, double*, uint32_t*, uint32_t*, uint64_t, uint64_t,
                                 hipStream_t);

}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

// Temp storage the by-key kernels carve for values of `value_bytes`, whatever the key width and mode:
// the reduce layout (per tile a count word, sizeof(V)/4 sum words and a claim word) at the smallest
// tile of those instantiations; never more than the reference's GetScanByKeyTempStorageBytes /
// GetReduceByKeyTempStorageBytes.
size_t lcpp_hip_internal_by_key_needed_bytes(uint64_t n, size_t value_bytes) {
    const uint32_t tile = value_bytes == 8
                              ? std::min({kBkTileItems<uint32_t, uint64_t, kModeScan>, kBkTileItems<uint64_t, uint64_t, kModeScan>,
                                          kBkTileItems<uint32_t, uint64_t, kModeReduce>, kBkTileItems<uint64_t, uint64_t, kModeReduce>})
                              : std::min({kBkTileItems<uint32_t, uint32_t, kModeScan>, kBkTileItems<uint64_t, uint32_t, kModeScan>,
                                          kBkTileItems<uint32_t, uint32_t, kModeReduce>, kBkTileItems<uint64_t, uint32_t, kModeReduce>});
    return state_bytes(n, tile, value_bytes, true);
}

#define LCPP_HIP_DEFINE_BY_KEY(KS, KT, KU, VS, VT, VU)                                                                 \
    int lcpp_hip_scan_by_key_sum_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys, const VT* values_in,      \
                                             VT* values_out, uint64_t n, int inclusive, int use_init, VT init,        \
                                             uint64_t key_mask, void* stream) {                                      \
        return by_key<KU, VU, kModeScan>(temp, temp_bytes, reinterpret_cast<const KU*>(keys),                         \
                                         reinterpret_cast<const VU*>(values_in), reinterpret_cast<VU*>(values_out),   \
                                         nullptr, nullptr, nullptr, n, key_mask, inclusive, use_init,                 \
                                         __builtin_bit_cast(VU, init), stream);                                      \
    }                                                                                                                 \
    int lcpp_hip_reduce_by_key_sum_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys_in, const VT* values_in, \
                                               KT* unique_out, VT* aggregates_out, uint32_t* num_runs_out, uint64_t n, \
                                               uint64_t key_mask, void* stream) {                                    \
        return by_key<KU, VU, kModeReduce>(temp, temp_bytes, reinterpret_cast<const KU*>(keys_in),                    \
                                           reinterpret_cast<const VU*>(values_in), nullptr,                           \
                                           reinterpret_cast<KU*>(unique_out), reinterpret_cast<VU*>(aggregates_out),  \
                                           num_runs_out, n, key_mask, 0, 0, VU(0), stream);                          \
    }

#define LCPP_HIP_DEFINE_BY_KEY_VALUES(KS, KT, KU)                  \
    LCPP_HIP_DEFINE_BY_KEY(KS, KT, KU, i32, int32_t, uint32_t)     \
    LCPP_HIP_DEFINE_BY_KEY(KS, KT, KU, u32, uint32_t, uint32_t)    \
    LCPP_HIP_DEFINE_BY_KEY(KS, KT, KU, f32, float, float)          \
    LCPP_HIP_DEFINE_BY_KEY(KS, KT, KU, i64, int64_t, uint64_t)     \
    LCPP_HIP_DEFINE_BY_KEY(KS, KT, KU, u64, uint64_t, uint64_t)    \
    LCPP_HIP_DEFINE_BY_KEY(KS, KT, KU, f64, double, double)

LCPP_HIP_DEFINE_BY_KEY_VALUES(i32, int32_t, uint32_t)
LCPP_HIP_DEFINE_BY_KEY_VALUES(u32, uint32_t, uint32_t)
LCPP_HIP_DEFINE_BY_KEY_VALUES(i64, int64_t, uint64_t)
LCPP_HIP_DEFINE_BY_KEY_VALUES(u64, uint64_t, uint64_t)
#undef LCPP_HIP_DEFINE_BY_KEY_VALUES
#undef LCPP_HIP_DEFINE_BY_KEY

// Min / max by key: values compare in their own type (signed as signed; floats like fmin / fmax); without
// an initial value an exclusive scan's run heads get the operator's identity (the type's max / lowest,
// a quiet NaN for floats).
#define LCPP_HIP_DEFINE_BY_KEY_OP(NAME, OPT, KS, KT, KU, VS, VT)                                                       \
    int lcpp_hip_scan_by_key_##NAME##_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys, const VT* values_in, \
                                                 VT* values_out, uint64_t n, int inclusive, int use_init, VT init,    \
                                                 uint64_t key_mask, void* stream) {                                  \
        return by_key<KU, VT, kModeScan, OPT>(temp, temp_bytes, reinterpret_cast<const KU*>(keys), values_in,         \
                                              values_out, nullptr, nullptr, nullptr, n, key_mask, inclusive, use_init, \
                                              use_init ? init : OPT::identity<VT>(), stream);                        \
    }                                                                                                                 \
    int lcpp_hip_reduce_by_key_##NAME##_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys_in,                \
                                                   const VT* values_in, KT* unique_out, VT* aggregates_out,          \
                                                   uint32_t* num_runs_out, uint64_t n, uint64_t key_mask,            \
                                                   void* stream) {                                                   \
        return by_key<KU, VT, kModeReduce, OPT>(temp, temp_bytes, reinterpret_cast<const KU*>(keys_in), values_in,    \
                                                nullptr, reinterpret_cast<KU*>(unique_out), aggregates_out,           \
                                                num_runs_out, n, key_mask, 0, 0, OPT::identity<VT>(), stream);       \
    }
#define LCPP_HIP_DEFINE_BY_KEY_OP_VALUES(KS, KT, KU)                          \
    LCPP_HIP_DEFINE_BY_KEY_OP(min, MinValueOp, KS, KT, KU, i32, int32_t)      \
    LCPP_HIP_DEFINE_BY_KEY_OP(min, MinValueOp, KS, KT, KU, u32, uint32_t)     \
    LCPP_HIP_DEFINE_BY_KEY_OP(min, MinValueOp, KS, KT, KU, f32, float)        \
    LCPP_HIP_DEFINE_BY_KEY_OP(min, MinValueOp, KS, KT, KU, i64, int64_t)      \
    LCPP_HIP_DEFINE_BY_KEY_OP(min, MinValueOp, KS, KT, KU, u64, uint64_t)     \
    LCPP_HIP_DEFINE_BY_KEY_OP(min, MinValueOp, KS, KT, KU, f64, double)       \
    LCPP_HIP_DEFINE_BY_KEY_OP(max, MaxValueOp, KS, KT, KU, i32, int32_t)      \
    LCPP_HIP_DEFINE_BY_KEY_OP(max, MaxValueOp, KS, KT, KU, u32, uint32_t)     \
    LCPP_HIP_DEFINE_BY_KEY_OP(max, MaxValueOp, KS, KT, KU, f32, float)        \
    LCPP_HIP_DEFINE_BY_KEY_OP(max, MaxValueOp, KS, KT, KU, i64, int64_t)      \
    LCPP_HIP_DEFINE_BY_KEY_OP(max, MaxValueOp, KS, KT, KU, u64, uint64_t)     \
    LCPP_HIP_DEFINE_BY_KEY_OP(max, MaxValueOp, KS, KT, KU, f64, double)
LCPP_HIP_DEFINE_BY_KEY_OP_VALUES(i32, int32_t, uint32_t)
LCPP_HIP_DEFINE_BY_KEY_OP_VALUES(u32, uint32_t, uint32_t)
LCPP_HIP_DEFINE_BY_KEY_OP_VALUES(i64, int64_t, uint64_t)
LCPP_HIP_DEFINE_BY_KEY_OP_VALUES(u64, uint64_t, uint64_t)
#undef LCPP_HIP_DEFINE_BY_KEY_OP_VALUES
#undef LCPP_HIP_DEFINE_BY_KEY_OP

}  // extern "C"
