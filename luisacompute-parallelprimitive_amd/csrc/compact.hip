// DeviceSelect (Flagged, If, FlaggedIf, Unique, UniqueByKey; copy and in-place forms),
// DevicePartition (Flagged, If, three-way If) and DeviceRunLengthEncode (Encode, NonTrivialRuns) for
// gfx950: single-pass stream compaction over a decoupled look-back of per-tile selection counts.
//
// Reference paths (src/lcpp/device/): DeviceSelect<> (device_select.h:65-344: flags or predicate ->
// DeviceScan<>::ExclusiveSum of the selection flags -> scatter, count written by the last item),
// DevicePartition<> (device_partition.h:73-209: selected items in order at the front, rejected items
// in reverse order from the back, :530-579; three-way: first and second categories in order, the
// unselected items reversed within their own output, :581-663), DeviceRunLengthEncode<>
// (device_run_length_encode.h:71-153: unique values with run lengths; offsets and lengths of the runs
// longer than one item).  The reference runs each as flag, scan and scatter kernels over n-sized
// temp arrays; its predicates and equalities are device lambdas compiled at run time.
//
// Selection vocabulary here: a predicate is two clauses that must both hold, each comparing the
// item with operands (<, <=, >, >=, ==, !=, a half-open range, a C remainder test, a bit-mask test);
// flags select when != 0; adjacent keys are equal under a bit mask (integers) or by value (floats,
// where -0.0 == +0.0 and NaN differs from everything, like the reference's lhs == rhs).
//
// MI355X design
//   * One workgroup of 256 threads (4 waves) per tile.  A wave owns 64 x ITEMS consecutive items
//     (ITEMS = 128 / item bytes: 32 four-byte or 16 eight-byte items per lane), lane l holding items
//     seg + 64 j + l, so every load instruction of a wave reads consecutive addresses and a tile is
//     8,192 or 4,096 items.  Select and partition read a whole wave of an aligned input as 16-byte
//     vectors and move them to that layout through the wave's part of the staging buffer.
//   * Selection masks are per-lane bit sets (bit j = item j of the lane).  Ranks come from wave ballots:
//     row j's selected items take consecutive tile ranks (k + selected lanes below), so they are
//     staged in LDS at consecutive addresses (no bank conflicts) and the workgroup copies each
//     category out with full-width coalesced stores.  Run heads compare each item with the item
//     before it, moved across lanes with DPP wave shifts.
//   * Wave counts (W = 1 or 2 words) are combined across the tile's 4 waves in LDS; the tile
//     publishes its aggregate, wave 0 walks back 32 predecessor tiles per step to the newest
//     INCLUSIVE state, and the tile publishes INCLUSIVE.  Tile states are 64-bit words (status in the
//     low half, count in the high half) read with agent-scope relaxed atomics; a multi-word state is
//     accepted only when all its words show the same status.  A predecessor still unpublished after
//     `spin_limit` polls is claimed (a claim word per tile) and counted by the waiting workgroup with
//     the owner's own code; the owner waits for such a helper to finish before publishing INCLUSIVE.
//   * Partition rejects are written backwards from the end the same way.  Run lengths come from a
//     second state word combined by max: the position of the last run head before each item, so a
//     run crossing any number of tiles needs no second pass.
//   * In-place selects (output overlapping the input or the flags) compact into temp storage and
//     copy the selected prefix back; the three-way partition stages its unselected items in temp
//     storage and reverses them into their output in a second small kernel.
// Algorithmic traffic: select / partition n*(sizeof(T) [+ sizeof(F)]) read + selected (or n) items
// written; run-length encode n*sizeof(T) read + runs*(sizeof(T) + 4) written.
#include "common.hpp"
#include "../../include/lcpp_hip.h"

#include <atomic>
#include <cstring>

namespace lcpp_hip {
namespace {

constexpr int kCpBlock = 256;
constexpr int kCpWaves = kCpBlock / kWave;
// Predecessor states wave 0 inspects per look-back step, one per lane.  Every poll of a step ends in a
// workgroup barrier, and a step waits for its window's unpublished entries up to the nearest INCLUSIVE
// one, so windows shorter than the wave win (2^28 u32, half kept: select-if 0.435 ms with 64, 0.409-0.411
// with 32, 0.415-0.419 with 16, 0.458-0.461 with 8, 0.546-0.548 with 4; partition-if 0.536 / 0.497-0.499 /
// 0.494-0.495 / 0.539-0.541 / 0.627-0.629 ms).
constexpr int kCompactWindow = 32;

constexpr uint32_t kStInvalid = 0;
constexpr uint32_t kStPartial = 1;
constexpr uint32_t kStInclusive = 2;
constexpr uint32_t kStatusMask = 3;

constexpr uint64_t kClaimOpen = 0;    // nobody has closed or claimed the tile yet
constexpr uint64_t kClaimOwned = 1;   // the owner closed it
constexpr uint64_t kClaimHelper = 2;  // a helper is counting the tile
constexpr uint64_t kClaimDone = 3;    // the helper's PARTIAL stores have all been performed

constexpr uint32_t kActDone = 0;
constexpr uint32_t kActAdvance = 1;
constexpr uint32_t kActWait = 2;
constexpr uint32_t kActHelp = 3;

enum : int {
    kSelect = 0,       // items (or flags) tested by a predicate; optional partition of the rejects
    kThreeWay = 1,     // first / second / unselected categories
    kUnique = 2,       // first item of every run of equal items
    kUniqueByKey = 3,  // first (key, value) of every run of equal keys
    kEncode = 4,       // unique values and run lengths
    kNonTrivial = 5,   // offsets and lengths of runs longer than one item
};

template <int MODE>
constexpr int kWords = (MODE == kThreeWay || MODE == kEncode || MODE == kNonTrivial) ? 2 : 1;
// Word 1 of the run-length modes is the position of the last run head, combined by max.
template <int MODE>
constexpr bool kWord1Max = MODE == kEncode || MODE == kNonTrivial;

template <typename U, typename V>
constexpr int kCpItems = static_cast<int>(128 / (sizeof(U) > sizeof(V) ? sizeof(U) : sizeof(V)));

template <typename P>
struct Clause {
    int32_t op;
    P a;
    P b;
};

template <typename P>
struct Predicate {
    Clause<P> c[2];
};

template <typename T>
using Bits = std::conditional_t<sizeof(T) == 8, uint64_t, std::conditional_t<sizeof(T) == 4, uint32_t, uint8_t>>;

// Bit k set when clause `c` holds for x[k].  The switch is uniform (a kernel argument), so each
// thread runs one branch over all of its items.
template <typename P, int N, typename M>
__device__ __forceinline__ M clause_bits(const Clause<P>& c, const P (&x)[N]) {
    M bits = 0;
#define LCPP_CLAUSE(OP, EXPR)                                               \
    case OP: {                                                              \
        _Pragma("unroll") for (int k = 0; k < N; ++k) {                     \
            const P v = x[k];                                               \
            bits |= static_cast<M>((EXPR) ? 1 : 0) << k;                     \
        }                                                                   \
        return bits;                                                        \
    }
    switch (c.op) {
        LCPP_CLAUSE(LCPP_HIP_PRED_LT, v < c.a)
        LCPP_CLAUSE(LCPP_HIP_PRED_LE, v <= c.a)
        LCPP_CLAUSE(LCPP_HIP_PRED_GT, v > c.a)
        LCPP_CLAUSE(LCPP_HIP_PRED_GE, v >= c.a)
        LCPP_CLAUSE(LCPP_HIP_PRED_EQ, v == c.a)
        LCPP_CLAUSE(LCPP_HIP_PRED_NE, v != c.a)
        LCPP_CLAUSE(LCPP_HIP_PRED_RANGE, c.a <= v && v < c.b)
        LCPP_CLAUSE(LCPP_HIP_PRED_MASK_EQ, (__builtin_bit_cast(Bits<P>, v) & __builtin_bit_cast(Bits<P>, c.a)) ==
                                               __builtin_bit_cast(Bits<P>, c.b))
        LCPP_CLAUSE(LCPP_HIP_PRED_MASK_NE, (__builtin_bit_cast(Bits<P>, v) & __builtin_bit_cast(Bits<P>, c.a)) !=
                                               __builtin_bit_cast(Bits<P>, c.b))
        default:
            break;
    }
    if constexpr (std::is_integral_v<P>) {
        switch (c.op) {
            LCPP_CLAUSE(LCPP_HIP_PRED_MOD_EQ, v % c.a == c.b)
            LCPP_CLAUSE(LCPP_HIP_PRED_MOD_NE, v % c.a != c.b)
            default:
                break;
        }
    }
#undef LCPP_CLAUSE
    return c.op == LCPP_HIP_PRED_TRUE ? static_cast<M>(~static_cast<M>(0)) : static_cast<M>(0);
}

// Bit k of words[k / 32] set when clause `c` holds for x[k]: one uniform switch for all N items (a switch
// per small group of items would multiply the kernel's code, the clause pairs being expanded together).
template <typename P, int N>
__device__ __forceinline__ void clause_words(const Clause<P>& c, const P (&x)[N], uint32_t (&words)[(N + 31) / 32]) {
#pragma unroll
    for (int w = 0; w < (N + 31) / 32; ++w) words[w] = 0;
#define LCPP_CLAUSE_WORDS(OP, EXPR)                                         \
    case OP: {                                                              \
        _Pragma("unroll") for (int k = 0; k < N; ++k) {                     \
            const P v = x[k];                                               \
            words[k / 32] |= static_cast<uint32_t>((EXPR) ? 1 : 0) << (k % 32); \
        }                                                                   \
        return;                                                             \
    }
    switch (c.op) {
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_LT, v < c.a)
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_LE, v <= c.a)
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_GT, v > c.a)
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_GE, v >= c.a)
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_EQ, v == c.a)
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_NE, v != c.a)
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_RANGE, c.a <= v && v < c.b)
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_MASK_EQ, (__builtin_bit_cast(Bits<P>, v) & __builtin_bit_cast(Bits<P>, c.a)) ==
                                                     __builtin_bit_cast(Bits<P>, c.b))
        LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_MASK_NE, (__builtin_bit_cast(Bits<P>, v) & __builtin_bit_cast(Bits<P>, c.a)) !=
                                                     __builtin_bit_cast(Bits<P>, c.b))
        default:
            break;
    }
    if constexpr (std::is_integral_v<P>) {
        switch (c.op) {
            LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_MOD_EQ, v % c.a == c.b)
            LCPP_CLAUSE_WORDS(LCPP_HIP_PRED_MOD_NE, v % c.a != c.b)
            default:
                break;
        }
    }
#undef LCPP_CLAUSE_WORDS
    if (c.op == LCPP_HIP_PRED_TRUE) {
#pragma unroll
        for (int w = 0; w < (N + 31) / 32; ++w) words[w] = ~0u;
    }
}

template <typename K>
__device__ __forceinline__ bool keys_equal(K a, K b, uint64_t mask) {
    if constexpr (std::is_floating_point_v<K>) {
        return a == b;
    } else {
        return ((a ^ b) & static_cast<K>(mask)) == 0;
    }
}

// Per-lane item masks: bit j stands for item j of the lane.
template <int ITEMS>
using LaneMask = std::conditional_t<(ITEMS > 32), uint64_t, uint32_t>;

template <typename U, typename P, typename V>
struct CompactArgs {
    const U* in;          // items (keys for unique-by-key)
    const P* flags;       // selection flags (flagged forms)
    const V* values_in;   // unique-by-key values
    U* out;               // selected / first category / unique items or keys
    U* out2;              // three-way: second category
    U* out3;              // three-way: unselected items in order (temp staging)
    V* values_out;        // unique-by-key values
    uint32_t* aux0;       // run-length encode: counts; non-trivial runs: offsets
    uint32_t* aux1;       // non-trivial runs: lengths
    uint32_t* num_out;    // selected count(s)
    uint64_t* states;     // tiles x W state words, then one claim word per tile
    uint64_t n;
    uint64_t key_mask;
    Predicate<P> pred;    // select / flagged-if / three-way first
    Predicate<P> pred2;   // three-way second
    uint32_t spin_limit;
    bool partition;       // select: write the rejected items backwards after the selected ones
};

// A wave owns 64 * ITEMS consecutive items starting at `seg`; item j of lane l is seg + 64 j + l, so
// every load and every output store of the wave covers consecutive addresses.
template <typename U, typename V, int ITEMS>
struct LaneItems {
    U x[ITEMS];
    V v[ITEMS];
    LaneMask<ITEMS> valid;
    LaneMask<ITEMS> sel;    // selected / first category / run heads (encode) / non-trivial run starts
    LaneMask<ITEMS> sel2;   // three-way second category / run ends (encode) / non-trivial run ends
    LaneMask<ITEMS> heads;  // run heads (run-length modes)
};

// LOADED: t.x already holds the items (vector_load_items); only the masks are computed.
template <typename U, typename P, typename V, int MODE, bool FLAGS, int ITEMS, bool LOADED = false>
__device__ __forceinline__ void load_lane(const CompactArgs<U, P, V>& a, uint64_t seg, LaneItems<U, V, ITEMS>& t) {
    using M = LaneMask<ITEMS>;
    const uint32_t lane = lane_id();
    M valid = 0;
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        const uint64_t i = seg + static_cast<uint64_t>(kWave) * j + lane;
        const bool ok = i < a.n;
        valid |= static_cast<M>(ok ? 1 : 0) << j;
        if constexpr (!LOADED) t.x[j] = ok ? a.in[i] : U(0);
        if constexpr (MODE == kUniqueByKey) t.v[j] = ok ? a.values_in[i] : V(0);
    }
    t.valid = valid;
    t.sel2 = 0;
    t.heads = 0;
    if constexpr (MODE == kSelect || MODE == kThreeWay) {
        M s1, s2 = 0;
        if constexpr (FLAGS) {
            P f[ITEMS];
#pragma unroll
            for (int j = 0; j < ITEMS; ++j) {
                const uint64_t i = seg + static_cast<uint64_t>(kWave) * j + lane;
                f[j] = i < a.n ? a.flags[i] : P(0);
            }
            s1 = clause_bits<P, ITEMS, M>(a.pred.c[0], f) & clause_bits<P, ITEMS, M>(a.pred.c[1], f);
        } else {
            s1 = clause_bits<P, ITEMS, M>(a.pred.c[0], t.x) & clause_bits<P, ITEMS, M>(a.pred.c[1], t.x);
            if constexpr (MODE == kThreeWay)
                s2 = clause_bits<P, ITEMS, M>(a.pred2.c[0], t.x) & clause_bits<P, ITEMS, M>(a.pred2.c[1], t.x);
        }
        t.sel = s1 & valid;
        t.sel2 = s2 & ~s1 & valid;
    } else {
        // Item i starts a run when i == 0 or it differs from item i - 1: lane l - 1's item j, lane 63's
        // item j - 1, or the item before the segment.
        U carry = seg > 0 && seg - 1 < a.n ? a.in[seg - 1] : U(0);
        M heads = 0;
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const U prev = dpp_move<dpp::kWaveShr1>(carry, t.x[j]);
            const uint64_t i = seg + static_cast<uint64_t>(kWave) * j + lane;
            const bool head = i == 0 || !keys_equal(t.x[j], prev, a.key_mask);
            heads |= static_cast<M>(head ? 1 : 0) << j;
            carry = wave_read_lane(t.x[j], kWave - 1);
        }
        heads &= valid;
        t.heads = heads;
        if constexpr (MODE == kUnique || MODE == kUniqueByKey) {
            t.sel = heads;
        } else {
            // Item i ends a run when it is the last item or item i + 1 is a head: lane l + 1's item j,
            // lane 0's item j + 1, or the item after the segment.
            const uint64_t after = seg + static_cast<uint64_t>(kWave) * ITEMS;
            const bool after_head = after < a.n && !keys_equal(a.in[after], wave_read_lane(t.x[ITEMS - 1], kWave - 1),
                                                               a.key_mask);
            const M top = (wave_read_lane(heads, 0) >> 1) | (static_cast<M>(after_head ? 1 : 0) << (ITEMS - 1));
            const M next_heads = dpp_move<dpp::kWaveShl1>(top, heads);
            M last = 0;
            if (a.n > seg && a.n - 1 - seg < static_cast<uint64_t>(kWave) * ITEMS &&
                (a.n - 1 - seg) % kWave == lane)
                last = static_cast<M>(1) << ((a.n - 1 - seg) / kWave);
            const M ends = valid & (next_heads | last);
            if constexpr (MODE == kEncode) {
                t.sel = heads;
                t.sel2 = ends;
            } else {
                t.sel = heads & ~ends;   // a head whose run continues: a run longer than one item
                t.sel2 = ends & ~heads;  // the end of such a run
            }
        }
    }
}

// The wave's 64 x ITEMS items (all inside the input, which is 16-byte aligned) read as 16-byte vectors,
// lane l taking vector r of every 64: items seg + 64 VEC r + VEC l + c.  They reach the lane-strided
// layout (item seg + 64 j + l in register j) through the wave's own region of LDS `wst`: vectors are
// written at their item offsets and read back strided.  Measured on select-if / partition-if over
// 2^28 u32: 0.463 -> 0.439 ms and 0.581 -> 0.549 ms against one 4-byte load per item and register.
template <typename U, int ITEMS>
__device__ __forceinline__ void vector_load_items(const U* in, uint64_t seg, U* wst, U (&x)[ITEMS]) {
    constexpr int VEC = 16 / sizeof(U);
    struct alignas(16) Vec {
        U c[VEC];
    };
    static_assert(sizeof(Vec) == 16 && ITEMS % VEC == 0, "whole 16-byte vectors per lane");
    const uint32_t lane = lane_id();
    const Vec* src = reinterpret_cast<const Vec*>(in + seg);
    Vec q[ITEMS / VEC];
#pragma unroll
    for (int r = 0; r < ITEMS / VEC; ++r) q[r] = src[kWave * r + lane];
#pragma unroll
    for (int r = 0; r < ITEMS / VEC; ++r) {
#pragma unroll
        for (int c = 0; c < VEC; ++c) wst[kWave * VEC * r + VEC * lane + c] = q[r].c[c];
    }
    // Same wave, same element type: the reads follow the writes in LDS order.
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) x[j] = wst[kWave * j + lane];
}

struct MaxU32Op {
    __device__ __forceinline__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
    template <typename T>
    __device__ __forceinline__ static constexpr T identity() { return T(0); }
};

template <int MODE>
__device__ __forceinline__ uint32_t combine_word(int w, uint32_t older, uint32_t newer) {
    if (kWord1Max<MODE> && w == 1) return older > newer ? older : newer;
    return older + newer;
}

template <typename M>
__device__ __forceinline__ uint32_t popcount(M m) {
    if constexpr (sizeof(M) == 8) {
        return static_cast<uint32_t>(__builtin_popcountll(m));
    } else {
        return static_cast<uint32_t>(__builtin_popcount(m));
    }
}

// The wave's count words: selected items (and the second category), or run heads / non-trivial
// starts and the position of the wave's last run head (0 when it has none).  Uniform results.
template <int MODE, typename U, typename V, int ITEMS>
__device__ __forceinline__ void wave_words(const LaneItems<U, V, ITEMS>& t, uint64_t seg, uint32_t (&w)[kWords<MODE>]) {
    w[0] = wave_reduce(popcount(t.sel), SumOp{});
    if constexpr (MODE == kThreeWay) {
        w[1] = wave_reduce(popcount(t.sel2), SumOp{});
    } else if constexpr (kWord1Max<MODE>) {
        uint32_t last = 0;
        if (t.heads) {
            const int j = static_cast<int>(sizeof(t.heads) == 8 ? 63 - __builtin_clzll(static_cast<uint64_t>(t.heads))
                                                                : 31 - __builtin_clz(static_cast<uint32_t>(t.heads)));
            last = static_cast<uint32_t>(seg + static_cast<uint64_t>(kWave) * j + lane_id());
        }
        w[1] = wave_reduce(last, MaxU32Op{});
    }
}

// Combines the waves' words: each wave's prefix within the tile and the tile aggregate.  Called by
// every thread; barriers on both sides of the use of s_wave.
template <int MODE>
__device__ __forceinline__ void block_words(const uint32_t (&x)[kWords<MODE>], uint32_t (*s_wave)[kCpWaves],
                                            uint32_t (&wave_prefix)[kWords<MODE>], uint32_t (&agg)[kWords<MODE>]) {
    constexpr int W = kWords<MODE>;
    const uint32_t wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane_id() == 0) {
#pragma unroll
        for (int w = 0; w < W; ++w) s_wave[w][wave] = x[w];
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < W; ++w) {
        uint32_t prefix = 0, total = 0;
#pragma unroll
        for (int j = 0; j < kCpWaves; ++j) {
            if (static_cast<uint32_t>(j) == wave) prefix = total;
            total = combine_word<MODE>(w, total, s_wave[w][j]);
        }
        wave_prefix[w] = prefix;
        agg[w] = total;
    }
}

template <int W>
__device__ __forceinline__ void publish_words(uint64_t* slot, uint32_t status, const uint32_t (&v)[W]) {
#pragma unroll
    for (int w = 0; w < W; ++w) atomic_store_agent(&slot[w], (static_cast<uint64_t>(v[w]) << 32) | status);
}

// Status of a tile state if all its words carry the same published status, else kStInvalid.
template <int W>
__device__ __forceinline__ uint32_t read_words(const uint64_t* slot, uint32_t (&v)[W]) {
    uint64_t s[W];
#pragma unroll
    for (int w = 0; w < W; ++w) s[w] = atomic_load_agent(&slot[w]);
    const uint32_t st = static_cast<uint32_t>(s[0]) & kStatusMask;
    bool ok = st == kStPartial || st == kStInclusive;
#pragma unroll
    for (int w = 0; w < W; ++w) {
        ok = ok && (static_cast<uint32_t>(s[w]) & kStatusMask) == st;
        v[w] = static_cast<uint32_t>(s[w] >> 32);
    }
    return ok ? st : kStInvalid;
}

// Aggregate words of tile `tile`, computed by the whole workgroup exactly as its owner computes them.
template <typename U, typename P, typename V, int MODE, bool FLAGS, int ITEMS>
__device__ void tile_aggregate(const CompactArgs<U, P, V>& a, uint32_t tile, uint32_t (*s_wave)[kCpWaves],
                               uint32_t (&agg)[kWords<MODE>]) {
    constexpr uint64_t kTile = static_cast<uint64_t>(kCpBlock) * ITEMS;
    const uint64_t seg = static_cast<uint64_t>(tile) * kTile + static_cast<uint64_t>(threadIdx.x / kWave) * kWave * ITEMS;
    LaneItems<U, V, ITEMS> t;
    load_lane<U, P, V, MODE, FLAGS, ITEMS>(a, seg, t);
    uint32_t w[kWords<MODE>], wp[kWords<MODE>];
    wave_words<MODE>(t, seg, w);
    block_words<MODE>(w, s_wave, wp, agg);
}

// Exclusive prefix words of tile `tile` (> 0) over its predecessors, called by the whole workgroup.  Wave 0
// reads WINDOW predecessor states per step (one per lane), newest first, and sums them down to the
// nearest INCLUSIVE one; its decision (done, next window, wait, help) reaches the workgroup through
// s_ctl (two rows used alternately, so one barrier per poll suffices).  A predecessor still unpublished
// after `spin_limit` polls is claimed (claims[t]: OPEN -> HELPER) and counted by the workgroup with
// help(t, words), which must compute exactly what its owner publishes; the helper publishes it PARTIAL and
// marks the claim DONE with release ordering.
template <int MODE, int WINDOW, typename Help>
__device__ void compact_lookback(uint64_t* states, uint64_t* claims, uint32_t tile, uint32_t spin_limit,
                                 uint32_t (*s_ctl)[2], uint32_t* s_prefix, uint32_t (&prefix)[kWords<MODE>],
                                 Help help) {
    constexpr int W = kWords<MODE>;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    int64_t top = static_cast<int64_t>(tile) - 1;
    uint32_t acc[W];
#pragma unroll
    for (int w = 0; w < W; ++w) acc[w] = 0;
    uint32_t spins = 0;
    uint32_t row = 0;
    while (true) {
        if (wave == 0) {
            const int64_t j = top - static_cast<int64_t>(lane);
            uint32_t v[W];
            const bool exists = j >= 0 && lane < static_cast<uint32_t>(WINDOW);
            const uint32_t st = exists ? read_words<W>(states + static_cast<uint64_t>(j) * W, v) : kStInvalid;
            const bool published = st != kStInvalid;
            const uint64_t stop_mask = wave_ballot(published && (st == kStInclusive || j == 0));
            const uint32_t cut = stop_mask ? static_cast<uint32_t>(__builtin_ctzll(stop_mask)) : kWave - 1;
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
#pragma unroll
                for (int w = 0; w < W; ++w) {
                    const uint32_t mine = take ? v[w] : 0u;
                    const uint32_t window = (kWord1Max<MODE> && w == 1) ? wave_reduce(mine, MaxU32Op{})
                                                                       : wave_reduce(mine, SumOp{});
                    acc[w] = combine_word<MODE>(w, window, acc[w]);
                }
                action = (stop_mask != 0 || top < WINDOW) ? kActDone : kActAdvance;
            }
            if (lane == 0) {
                s_ctl[row][0] = action;
                s_ctl[row][1] = help_tile;
                if (action == kActDone) {
#pragma unroll
                    for (int w = 0; w < W; ++w) s_prefix[w] = acc[w];
                }
            }
        }
        __syncthreads();
        const uint32_t action = s_ctl[row][0];
        const uint32_t help_tile = s_ctl[row][1];
        row ^= 1u;
        if (action == kActDone) break;
        if (action == kActAdvance) {
            top -= WINDOW;
            spins = 0;
            continue;
        }
        if (action == kActWait) {
            __builtin_amdgcn_s_sleep(1);
            ++spins;
            continue;
        }
        // kActHelp: claim the unpublished predecessor, count it, publish it PARTIAL and mark the claim
        // DONE with release ordering.
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
            uint32_t h[W];
            help(help_tile, h);
            if (tid == 0) {
                publish_words<W>(states + static_cast<uint64_t>(help_tile) * W, kStPartial, h);
                __hip_atomic_store(&claims[help_tile], kClaimDone, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        spins = 0;
    }
#pragma unroll
    for (int w = 0; w < W; ++w) prefix[w] = s_prefix[w];
}

template <typename U, typename P, typename V, int MODE, bool FLAGS>
__global__ __launch_bounds__(kCpBlock) void compact_kernel(const CompactArgs<U, P, V> a) {
    constexpr int ITEMS = kCpItems<U, V>;
    constexpr int W = kWords<MODE>;
    constexpr uint64_t kTile = static_cast<uint64_t>(kCpBlock) * ITEMS;
    constexpr uint32_t kPublisher = kCpBlock - kWave;
    constexpr size_t kStageBytes = kTile * (sizeof(U) > sizeof(V) ? sizeof(U) : sizeof(V));
    __shared__ __align__(16) unsigned char s_stage[kStageBytes];
    __shared__ uint32_t s_wave[W][kCpWaves];
    __shared__ uint32_t s_ctl[2][2];
    __shared__ uint32_t s_prefix[W];

    uint64_t* const states = a.states;
    uint64_t* const claims = states + static_cast<uint64_t>(gridDim.x) * W;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint64_t seg = static_cast<uint64_t>(tile) * kTile + static_cast<uint64_t>(wave) * kWave * ITEMS;

    LaneItems<U, V, ITEMS> t;
    bool vector_loaded = false;
    if constexpr ((MODE == kSelect || MODE == kThreeWay) && sizeof(U) >= 4) {
        // s_stage is free until the staging below (after block_words' barriers); each wave uses its own
        // 64 x ITEMS items of it.
        if (seg + static_cast<uint64_t>(kWave) * ITEMS <= a.n && (reinterpret_cast<uintptr_t>(a.in) & 15u) == 0) {
            U* wst = reinterpret_cast<U*>(s_stage) + static_cast<uint64_t>(wave) * kWave * ITEMS;
            vector_load_items<U, ITEMS>(a.in, seg, wst, t.x);
            load_lane<U, P, V, MODE, FLAGS, ITEMS, true>(a, seg, t);
            vector_loaded = true;
        }
    }
    if (!vector_loaded) load_lane<U, P, V, MODE, FLAGS, ITEMS>(a, seg, t);
    uint32_t words[W], wp[W], agg[W];
    wave_words<MODE>(t, seg, words);
    block_words<MODE>(words, s_wave, wp, agg);

    uint64_t* const my_slot = states + static_cast<uint64_t>(tile) * W;
    bool owned = true;
    if (tid == kPublisher) {
        publish_words<W>(my_slot, tile == 0 ? kStInclusive : kStPartial, agg);
        uint64_t expected = kClaimOpen;
        owned = __hip_atomic_compare_exchange_strong(&claims[tile], &expected, kClaimOwned, __ATOMIC_RELAXED,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // ---- staging --------------------------------------------------------------------------------
    // Tile ranks are known before the look-back: row j of a wave puts its selected items at
    // consecutive ranks (ballot ranks), staged in LDS without bank conflicts, while predecessors
    // publish.  After the look-back the workgroup copies each category out with full-width stores.
    U* const stage = reinterpret_cast<U*>(s_stage);
    if constexpr (MODE == kEncode) {
        uint32_t l1 = wp[0];
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const bool is_sel = (t.sel >> j) & 1;
            const uint64_t sb = wave_ballot(is_sel);
            if (is_sel) stage[l1 + popc_lanes_below(sb)] = t.x[j];
            l1 += static_cast<uint32_t>(__builtin_popcountll(sb));
        }
    } else if constexpr (MODE != kNonTrivial) {
        const bool rejects = (MODE == kSelect && a.partition) || MODE == kThreeWay;
        uint32_t l1 = wp[0];
        uint32_t l2 = 0;
        if constexpr (MODE == kThreeWay) l2 = agg[0] + wp[1];
        uint32_t base = agg[0];
        if constexpr (MODE == kThreeWay) base += agg[1];
        // Rejects before the wave's items within the tile (every earlier item of the tile is valid).
        uint32_t lr = base + wave * kWave * ITEMS - wp[0];
        if constexpr (MODE == kThreeWay) lr -= wp[1];
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const bool s1 = (t.sel >> j) & 1;
            const uint64_t b1 = wave_ballot(s1);
            if (s1) stage[l1 + popc_lanes_below(b1)] = t.x[j];
            l1 += static_cast<uint32_t>(__builtin_popcountll(b1));
            if constexpr (MODE == kThreeWay) {
                const bool s2 = (t.sel2 >> j) & 1;
                const uint64_t b2 = wave_ballot(s2);
                if (s2) stage[l2 + popc_lanes_below(b2)] = t.x[j];
                l2 += static_cast<uint32_t>(__builtin_popcountll(b2));
            }
            if (rejects) {
                const bool r = ((t.valid & ~t.sel & ~t.sel2) >> j) & 1;
                const uint64_t rb = wave_ballot(r);
                if (r) stage[lr + popc_lanes_below(rb)] = t.x[j];
                lr += static_cast<uint32_t>(__builtin_popcountll(rb));
            }
        }
    }

    uint32_t prefix[W];
#pragma unroll
    for (int w = 0; w < W; ++w) prefix[w] = 0;
    if (tile > 0)
        compact_lookback<MODE, kCompactWindow>(states, claims, tile, a.spin_limit, s_ctl, s_prefix, prefix,
                                               [&](uint32_t help_tile, uint32_t (&h)[W]) {
                                                   tile_aggregate<U, P, V, MODE, FLAGS, ITEMS>(a, help_tile, s_wave, h);
                                               });

    if (tid == kPublisher) {
        if (!owned) {
            while (__hip_atomic_load(&claims[tile], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) != kClaimDone)
                __builtin_amdgcn_s_sleep(1);
        }
        if (tile > 0 || !owned) {
            uint32_t incl[W];
#pragma unroll
            for (int w = 0; w < W; ++w) incl[w] = combine_word<MODE>(w, prefix[w], agg[w]);
            publish_words<W>(my_slot, kStInclusive, incl);
        }
    }
    if (tile + 1 == gridDim.x && tid == 0) {
        a.num_out[0] = prefix[0] + agg[0];
        if constexpr (MODE == kThreeWay) a.num_out[1] = prefix[1] + agg[1];
    }

    // ---- outputs -------------------------------------------------------------------------------
    // Run lengths and non-trivial run offsets (one store per run) are written directly.
    if constexpr (MODE == kEncode || MODE == kNonTrivial) {
        const uint64_t lanes_le = lane == kWave - 1 ? ~0ull : ((2ull << lane) - 1);
        uint32_t k1 = prefix[0] + wp[0];  // heads / starts before the wave's items
        uint32_t last = prefix[1] > wp[1] ? prefix[1] : wp[1];  // last head position before them
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const bool is_sel = (t.sel >> j) & 1;
            const bool is_end = (t.sel2 >> j) & 1;
            const uint64_t hb = wave_ballot((t.heads >> j) & 1);
            const uint64_t sb = wave_ballot(is_sel);
            const uint32_t row_first = static_cast<uint32_t>(seg + static_cast<uint64_t>(kWave) * j);
            const uint32_t i = row_first + lane;
            if constexpr (MODE == kNonTrivial) {
                if (is_sel) a.aux0[k1 + popc_lanes_below(sb)] = i;
            }
            if (is_end) {
                const uint64_t le = hb & lanes_le;
                const uint32_t start = le ? row_first + static_cast<uint32_t>(63 - __builtin_clzll(le)) : last;
                const uint32_t run = k1 + static_cast<uint32_t>(__builtin_popcountll(sb & lanes_le)) - 1;
                if constexpr (MODE == kEncode) {
                    a.aux0[run] = i + 1 - start;
                } else {
                    a.aux1[run] = i + 1 - start;
                }
            }
            k1 += static_cast<uint32_t>(__builtin_popcountll(sb));
            if (hb) last = row_first + static_cast<uint32_t>(63 - __builtin_clzll(hb));
        }
        if constexpr (MODE == kNonTrivial) return;
    }
    __syncthreads();  // staged items visible to every thread (tile 0 has no look-back barrier)
    const uint64_t tile_first = static_cast<uint64_t>(tile) * kTile;
    const uint32_t tile_valid = static_cast<uint32_t>(a.n - tile_first < kTile ? a.n - tile_first : kTile);
    for (uint32_t q = tid; q < agg[0]; q += kCpBlock) a.out[prefix[0] + q] = stage[q];
    if constexpr (MODE == kThreeWay) {
        for (uint32_t q = tid; q < agg[1]; q += kCpBlock) a.out2[prefix[1] + q] = stage[agg[0] + q];
        const uint32_t rejected = tile_valid - agg[0] - agg[1];
        const uint64_t before = tile_first - prefix[0] - prefix[1];
        for (uint32_t q = tid; q < rejected; q += kCpBlock) a.out3[before + q] = stage[agg[0] + agg[1] + q];
    } else if constexpr (MODE == kSelect) {
        if (a.partition) {
            const uint32_t rejected = tile_valid - agg[0];
            const uint64_t before = tile_first - prefix[0];
            for (uint32_t q = tid; q < rejected; q += kCpBlock) a.out[a.n - 1 - (before + q)] = stage[agg[0] + q];
        }
    } else if constexpr (MODE == kUniqueByKey) {
        __syncthreads();
        V* const vstage = reinterpret_cast<V*>(s_stage);
        uint32_t r1 = wp[0];
#pragma unroll
        for (int j = 0; j < ITEMS; ++j) {
            const bool s1 = (t.sel >> j) & 1;
            const uint64_t b1 = wave_ballot(s1);
            if (s1) vstage[r1 + popc_lanes_below(b1)] = t.v[j];
            r1 += static_cast<uint32_t>(__builtin_popcountll(b1));
        }
        __syncthreads();
        for (uint32_t q = tid; q < agg[0]; q += kCpBlock) a.values_out[prefix[0] + q] = vstage[q];
    }
}

// ---- Select / partition over register-resident rows ---------------------------------------------------
// DeviceSelect::If / Flagged / FlaggedIf and DevicePartition::If / Flagged of 4- or 8-byte items, not in
// place, with a 16-byte aligned input (and flags of at most 4 bytes aligned to a thread's row of them).
// Like the scan's tiles, a tile is 256 threads x ROWS rows x one 16-byte vector of items per thread and
// row, held in registers (four workgroups per CU), rather than staged whole in LDS as by the kernel above
// (whose 32 KB stage per tile bounds the input in flight).  Per thread and row a mask of the selected items
// (each clause one uniform switch over all of the thread's items).  The tile's count comes first (one wave
// reduce per wave and one barrier: select-if / partition-if 0.387 / 0.444 -> 0.385 / 0.437 ms against
// publishing after the per-row totals), and wave 0 publishes it and walks back alone, without a workgroup
// barrier per poll, while the other waves put their per-row counts into a rows x waves table in LDS.  Then
// each wave stages its part of every row in 1 KB of LDS (selected items from the front,
// partition rejects from the back) and reads it back one slot per lane, so every store covers consecutive
// addresses.  (Stored straight from registers, four scattered stores per row, select-if took 0.53 ms.)
constexpr int kRowsBlock = 256;
constexpr int kRowsWaves = kRowsBlock / kWave;
// Predecessor states per look-back step (one per lane of wave 0): 0.393 / 0.450 ms with 8, 0.417 / 0.464 with
// 4, 0.390 / 0.452 with 12, 0.389 / 0.453 with 16 (select-if / partition-if as above).
constexpr int kRowsWindow = 8;
template <typename U>
constexpr int kRowItems = static_cast<int>(16 / sizeof(U));
// Rows per tile: four workgroups per CU (at most 128 VGPRs) with 16 rows, 12 with flags (whose vectors take
// registers too) or 8-byte items (whose remainder clauses do).  Select-if / partition-if of 2^28 u32, half
// kept: 0.393 / 0.450 ms with 16 rows at four workgroups per CU, 0.445 / 0.493 with 20 rows at three,
// 0.392 / 0.449 with 12 rows at five, 0.400 / 0.462 with 10 rows at six.
template <typename U, bool FLAGS>
constexpr int kSelRows = (FLAGS || sizeof(U) == 8) ? 12 : 16;
template <typename U, bool FLAGS>
constexpr uint32_t kRowsTile = static_cast<uint32_t>(kRowsBlock) * kSelRows<U, FLAGS> * kRowItems<U>;

// One thread's items (and flags) of one row: items base + (256 r + tid) V + j, j < V, as one vector each.
template <typename U, typename P>
struct RowVecs {
    static constexpr int V = kRowItems<U>;
    using Items = U __attribute__((ext_vector_type(V)));
    using Flags = P __attribute__((ext_vector_type(V)));
};

// Selection mask of one row (bit j: item j of the thread's vector), valid items only.
template <typename U, typename P, bool FLAGS>
__device__ __forceinline__ uint32_t row_selection(const Predicate<P>& pred, const typename RowVecs<U, P>::Items& it,
                                                  const typename RowVecs<U, P>::Flags& fl, uint32_t valid) {
    constexpr int V = kRowItems<U>;
    P x[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        if constexpr (FLAGS) {
            x[j] = fl[j];
        } else {
            x[j] = it[j];
        }
    }
    return clause_bits<P, V, uint32_t>(pred.c[0], x) & clause_bits<P, V, uint32_t>(pred.c[1], x) & valid;
}

// Loads row r of the tile at `base` for this thread; items past n read as 0 and are not valid.  A vector
// wholly before n is one vector load (of a full tile, without the test); only the vector holding item
// n - 1 is read item by item.
template <typename U, typename P, bool FLAGS>
__device__ __forceinline__ void load_row(const CompactArgs<U, P, U>& a, uint64_t base, int r, bool full,
                                         typename RowVecs<U, P>::Items& it, typename RowVecs<U, P>::Flags& fl,
                                         uint32_t& valid) {
    using RV = RowVecs<U, P>;
    constexpr int V = RV::V;
    const uint64_t vec = static_cast<uint64_t>(r) * kRowsBlock + threadIdx.x;
    const uint64_t first = base + vec * V;
    if (full || first + V <= a.n) {
        it = __builtin_nontemporal_load(reinterpret_cast<const typename RV::Items*>(a.in + base) + vec);
        if constexpr (FLAGS) fl = __builtin_nontemporal_load(reinterpret_cast<const typename RV::Flags*>(a.flags + base) + vec);
        valid = (1u << V) - 1u;
    } else {
        valid = 0;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const bool ok = first + j < a.n;
            it[j] = ok ? a.in[first + j] : U(0);
            if constexpr (FLAGS) fl[j] = ok ? a.flags[first + j] : P(0);
            valid |= (ok ? 1u : 0u) << j;
        }
    }
}

// Selected items of tile `tile`, counted by one wave (a predecessor's count for the look-back fallback;
// integer counts, so any order gives its owner's result).
template <typename U, typename P, bool FLAGS>
__device__ uint32_t rows_tile_count(const CompactArgs<U, P, U>& a, uint32_t tile) {
    using RV = RowVecs<U, P>;
    constexpr int V = RV::V;
    constexpr uint32_t TILE = kRowsTile<U, FLAGS>;
    const uint64_t base = static_cast<uint64_t>(tile) * TILE;
    const uint32_t lane = lane_id();
    uint32_t c = 0;
#pragma unroll 1
    for (uint32_t vec = lane; vec < TILE / V; vec += kWave) {
        const uint64_t first = base + static_cast<uint64_t>(vec) * V;
        typename RV::Items it;
        typename RV::Flags fl;
        uint32_t valid = 0;
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const bool ok = first + j < a.n;
            it[j] = ok ? a.in[first + j] : U(0);
            if constexpr (FLAGS) fl[j] = ok ? a.flags[first + j] : P(0);
            valid |= (ok ? 1u : 0u) << j;
        }
        c += static_cast<uint32_t>(__builtin_popcount(row_selection<U, P, FLAGS>(a.pred, it, fl, valid)));
    }
    return wave_reduce(c, SumOp{});
}

// Selected items before tile `tile` (> 0), by wave 0 alone (no workgroup barrier per poll): each step reads
// kRowsWindow predecessor states, newest first, and sums them down to the nearest INCLUSIVE one.  A
// predecessor still unpublished after `spin_limit` polls is claimed (claims[t]: OPEN -> HELPER), counted by
// this wave and published PARTIAL, and its claim marked DONE with release ordering; a claim lost to the
// owner or to another helper is simply polled again.
template <typename U, typename P, bool FLAGS>
__device__ uint32_t rows_lookback(const CompactArgs<U, P, U>& a, uint64_t* states, uint64_t* claims, uint32_t tile) {
    const uint32_t lane = lane_id();
    uint32_t acc = 0;
    int64_t top = static_cast<int64_t>(tile) - 1;
    uint32_t spins = 0;
    while (true) {
        const int64_t j = top - static_cast<int64_t>(lane);
        const bool exists = j >= 0 && lane < static_cast<uint32_t>(kRowsWindow);
        uint32_t v[1] = {0};
        const uint32_t st = exists ? read_words<1>(states + j, v) : kStInvalid;
        const bool published = st != kStInvalid;
        const uint64_t stop_mask = wave_ballot(published && (st == kStInclusive || j == 0));
        const uint32_t cut = stop_mask ? static_cast<uint32_t>(__builtin_ctzll(stop_mask)) : kWave - 1;
        const uint64_t upto = cut >= kWave - 1 ? ~0ull : ((2ull << cut) - 1);
        const uint64_t missing = upto & wave_ballot(exists) & ~wave_ballot(published);
        if (missing) {
            if (spins < a.spin_limit) {
                __builtin_amdgcn_s_sleep(1);
                ++spins;
                continue;
            }
            const uint32_t help_tile = static_cast<uint32_t>(top - __builtin_ctzll(missing));
            uint32_t won = 0;
            if (lane == 0) {
                uint64_t expected = kClaimOpen;
                won = __hip_atomic_compare_exchange_strong(&claims[help_tile], &expected, kClaimHelper, __ATOMIC_RELAXED,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          ? 1u
                          : 0u;
            }
            if (wave_read_lane(won, 0) != 0) {
                const uint32_t h[1] = {rows_tile_count<U, P, FLAGS>(a, help_tile)};
                if (lane == 0) {
                    publish_words<1>(states + help_tile, kStPartial, h);
                    __hip_atomic_store(&claims[help_tile], kClaimDone, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            spins = 0;
            continue;
        }
        acc += wave_reduce(exists && lane <= cut ? v[0] : 0u, SumOp{});
        if (stop_mask != 0 || top < kRowsWindow) break;
        top -= kRowsWindow;
        spins = 0;
    }
    return acc;
}

template <typename U, typename P, bool FLAGS>
__global__ __launch_bounds__(kRowsBlock, 4) void select_rows_kernel(const CompactArgs<U, P, U> a) {
    using RV = RowVecs<U, P>;
    constexpr int V = RV::V;
    constexpr int R = kSelRows<U, FLAGS>;
    constexpr uint32_t TILE = kRowsTile<U, FLAGS>;
    constexpr int ROWS_PER_WORD = 32 / V;  // row masks packed into 32-bit words
    constexpr int MW = (R + ROWS_PER_WORD - 1) / ROWS_PER_WORD;
    constexpr uint32_t kRowSlots = static_cast<uint32_t>(kWave) * V;  // items of one wave's part of a row
    __shared__ uint32_t s_tot[R][kRowsWaves];
    __shared__ U s_stage[kRowsWaves][kRowSlots];
    __shared__ uint32_t s_prefix[1];
    __shared__ uint32_t s_wtot[kRowsWaves];

    uint64_t* const states = a.states;
    uint64_t* const claims = states + gridDim.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint64_t base = static_cast<uint64_t>(tile) * TILE;
    const bool full = base + TILE <= a.n;

    typename RV::Items it[R];
    uint32_t masks[MW];
    {
        typename RV::Flags fl[FLAGS ? R : 1];
        uint32_t valid[MW];
#pragma unroll
        for (int w = 0; w < MW; ++w) valid[w] = 0;
        if (full) {
            // Every row's loads in flight before any is used.
            const typename RV::Items* src = reinterpret_cast<const typename RV::Items*>(a.in + base);
#pragma unroll
            for (int r = 0; r < R; ++r) it[r] = __builtin_nontemporal_load(&src[r * kRowsBlock + tid]);
            if constexpr (FLAGS) {
                const typename RV::Flags* fsrc = reinterpret_cast<const typename RV::Flags*>(a.flags + base);
#pragma unroll
                for (int r = 0; r < R; ++r) fl[r] = __builtin_nontemporal_load(&fsrc[r * kRowsBlock + tid]);
            }
#pragma unroll
            for (int w = 0; w < MW; ++w) valid[w] = ~0u;
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                uint32_t v;
                load_row<U, P, FLAGS>(a, base, r, false, it[r], fl[FLAGS ? r : 0], v);
                valid[r / ROWS_PER_WORD] |= v << (V * (r % ROWS_PER_WORD));
            }
        }
        // Both clauses over all R x V items (item k = V r + j is bit k % 32 of word k / 32).
        P x[R * V];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int j = 0; j < V; ++j) {
                if constexpr (FLAGS) {
                    x[r * V + j] = fl[r][j];
                } else {
                    x[r * V + j] = it[r][j];
                }
            }
        }
        uint32_t second[MW];
        clause_words<P, R * V>(a.pred.c[0], x, masks);
        clause_words<P, R * V>(a.pred.c[1], x, second);
#pragma unroll
        for (int w = 0; w < MW; ++w) masks[w] &= second[w] & valid[w];
    }
    auto row_mask = [&](int r) { return (masks[r / ROWS_PER_WORD] >> (V * (r % ROWS_PER_WORD))) & ((1u << V) - 1u); };

    // The tile's count first (one wave reduce and one barrier), so the PARTIAL state goes out as early as
    // possible; the per-row totals follow behind the publish.
    {
        uint32_t c_all = 0;
#pragma unroll
        for (int w = 0; w < MW; ++w) c_all += static_cast<uint32_t>(__builtin_popcount(masks[w]));
        const uint32_t wt = wave_reduce(c_all, SumOp{});
        if (lane == 0) s_wtot[wave] = wt;
    }
    __syncthreads();
    uint32_t agg[1] = {0};
#pragma unroll
    for (int w = 0; w < kRowsWaves; ++w) agg[0] += s_wtot[w];

    // Wave 0 publishes the tile's count, walks back over its predecessors and publishes the inclusive count
    // at once (a helper that claimed this tile first publishes its PARTIAL state; the owner then waits for
    // the helper to finish before it publishes INCLUSIVE).
    uint32_t prefix[1] = {0};
    if (wave == 0) {
        uint32_t owned = 1;
        if (lane == 0) {
            publish_words<1>(&states[tile], tile == 0 ? kStInclusive : kStPartial, agg);
            uint64_t expected = kClaimOpen;
            owned = __hip_atomic_compare_exchange_strong(&claims[tile], &expected, kClaimOwned, __ATOMIC_RELAXED,
                                                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                        ? 1u
                        : 0u;
        }
        if (tile > 0) prefix[0] = rows_lookback<U, P, FLAGS>(a, states, claims, tile);
        if (lane == 0) {
            if (!owned) {
                while (__hip_atomic_load(&claims[tile], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) != kClaimDone)
                    __builtin_amdgcn_s_sleep(1);
            }
            if (tile > 0 || !owned) {
                const uint32_t incl[1] = {prefix[0] + agg[0]};
                publish_words<1>(&states[tile], kStInclusive, incl);
            }
            s_prefix[0] = prefix[0];
        }
    }

    // Each wave compacts its part of every row in registers through its own LDS slots: selected items from
    // slot 0 up in order, partition rejects from the last slot down, then lane l reads back slots 64 j + l.
    // The order inside a row does not depend on the tile's prefix, so waves 1-3 do this while wave 0 walks
    // back (wave 0 after its walk).
    // Row totals per wave (read after the next barrier); each thread's offset within its row is scanned
    // again at output time, so no per-row scan stays live across the look-back.
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t total = wave_reduce(static_cast<uint32_t>(__builtin_popcount(row_mask(r))), SumOp{});
        if (lane == 0) s_tot[r][wave] = total;
    }
    U* const stage = s_stage[wave];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t m = row_mask(r);
        const uint32_t c = static_cast<uint32_t>(__builtin_popcount(m));
        const uint32_t before = wave_inclusive_scan(c, SumOp{}) - c;  // selected items before the lane's
        const uint64_t row_first = base + (static_cast<uint64_t>(r) * kRowsBlock + wave * kWave) * V;
        const uint32_t in_row = row_first < a.n ? static_cast<uint32_t>(min<uint64_t>(a.n - row_first, kRowSlots)) : 0u;
        uint32_t k = before;                  // slot of the lane's next selected item
        uint32_t q = lane * V - before;       // rejects before the lane's next item
#pragma unroll
        for (int j = 0; j < V; ++j) {
            if ((m >> j) & 1u) {
                stage[k++] = it[r][j];
            } else {
                if (a.partition && lane * V + j < in_row) stage[kRowSlots - 1 - q] = it[r][j];
                ++q;
            }
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < V; ++j) it[r][j] = stage[static_cast<uint32_t>(j) * kWave + lane];
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    prefix[0] = s_prefix[0];
    if (tile + 1 == gridDim.x && tid == 0) a.num_out[0] = prefix[0] + agg[0];
    // Lane r (< R) of every wave takes row r: its total over the waves, the part in waves before this
    // one, and (scanned over the lanes) the selected items of the tile's earlier rows.
    uint32_t row_total = 0, row_before = 0;
    if (lane < static_cast<uint32_t>(R)) {
#pragma unroll
        for (int w = 0; w < kRowsWaves; ++w) {
            const uint32_t x = s_tot[lane][w];
            if (w < static_cast<int>(wave)) row_before += x;
            row_total += x;
        }
    }
    const uint32_t rows_incl = wave_inclusive_scan(row_total, SumOp{});

    // Stores.  Lane r's row_base: the selected items before this wave's part of row r (the tile prefix, the
    // earlier rows, the earlier waves of row r).  Every store of the wave covers consecutive addresses: a
    // selected run, then a run of rejects, whose output runs backwards from the end.
    const uint32_t row_base = prefix[0] + (rows_incl - row_total) + row_before;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t sel_base = wave_read_lane(row_base, r);
        const uint32_t kept = s_tot[r][wave];  // selected items of the wave's part of the row
        const uint64_t row_first = base + (static_cast<uint64_t>(r) * kRowsBlock + wave * kWave) * V;
        const uint32_t in_row = row_first < a.n ? static_cast<uint32_t>(min<uint64_t>(a.n - row_first, kRowSlots)) : 0u;
        // Rejects before the wave's row: its first item's index minus the selected items before it.
        const uint64_t rej_end = a.n - 1 - (row_first - sel_base);  // output position of the row's first reject
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const uint32_t slot = static_cast<uint32_t>(j) * kWave + lane;
            if (slot < kept) {
                a.out[sel_base + slot] = it[r][j];
            } else if (a.partition && slot >= kRowSlots - (in_row - kept)) {
                // Slot kRowSlots - 1 - q holds reject q, which goes to rej_end - q.
                a.out[rej_end - (kRowSlots - 1 - slot)] = it[r][j];
            }
        }
    }
}

// dst[q] = src[q] for q < *count (the in-place select's copy back).
template <typename U>
__global__ __launch_bounds__(256) void copy_prefix_kernel(U* __restrict__ dst, const U* __restrict__ src,
                                                          const uint32_t* __restrict__ count) {
    const uint64_t c = *count;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t q = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; q < c; q += stride) dst[q] = src[q];
}

// dst[u - 1 - j] = src[j] for j < u = n - counts[0] - counts[1] (three-way unselected, reversed).
template <typename U>
__global__ __launch_bounds__(256) void reverse_rejects_kernel(U* __restrict__ dst, const U* __restrict__ src,
                                                              const uint32_t* __restrict__ counts, uint64_t n) {
    const uint64_t u = n - counts[0] - counts[1];
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t j = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < u; j += stride)
        dst[u - 1 - j] = src[j];
}

// Test hook: the rows kernel for selects and partitions that allow it (default) or the staging kernel for
// every call.  Both give the same results.
std::atomic<bool> g_select_rows{true};

bool overlaps(const void* a, size_t a_bytes, const void* b, size_t b_bytes) {
    if (!a || !b || a_bytes == 0 || b_bytes == 0) return false;
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + b_bytes && y < x + a_bytes;
}

unsigned grid_for(uint64_t n) {
    const uint64_t blocks = ceil_div(n, 256 * 8);
    return static_cast<unsigned>(blocks < 1 ? 1 : (blocks > 8192 ? 8192 : blocks));
}

// Temp layout: [states: tiles x W words | claims: tiles words] (256-byte aligned), then the staging
// array of n items when the call needs one.
struct TempPlan {
    uint64_t tiles;
    size_t state_bytes;
    size_t stage_offset;
    size_t total;
};

TempPlan plan_temp(uint64_t n, uint64_t tile, int words, size_t stage_item_bytes) {
    TempPlan p;
    p.tiles = ceil_div(n, tile);
    p.state_bytes = p.tiles * (static_cast<size_t>(words) + 1) * sizeof(uint64_t);
    p.stage_offset = align_up(p.state_bytes, kViewAlign);
    p.total = stage_item_bytes ? p.stage_offset + n * stage_item_bytes : p.state_bytes;
    return p;
}

template <typename P>
int convert_predicate(const lcpp_hip_predicate* in, Predicate<P>& out, const char* what) {
    if (!in) return set_error(kInvalidArgument, "%s: null predicate", what);
    for (int c = 0; c < 2; ++c) {
        const int op = in->op[c];
        if (op < LCPP_HIP_PRED_TRUE || op > LCPP_HIP_PRED_MOD_NE)
            return set_error(kInvalidArgument, "%s: unknown predicate clause %d", what, op);
        out.c[c].op = op;
        std::memcpy(&out.c[c].a, &in->a[c], sizeof(P));
        std::memcpy(&out.c[c].b, &in->b[c], sizeof(P));
        if (op == LCPP_HIP_PRED_MOD_EQ || op == LCPP_HIP_PRED_MOD_NE) {
            if constexpr (!std::is_integral_v<P>) {
                return set_error(kInvalidArgument, "%s: remainder clauses need integer operands", what);
            } else {
                if (out.c[c].a == P(0)) return set_error(kInvalidArgument, "%s: remainder by zero", what);
            }
        }
    }
    return kOk;
}

template <typename P>
Predicate<P> nonzero_predicate() {
    Predicate<P> p{};
    p.c[0].op = LCPP_HIP_PRED_NE;
    p.c[0].a = P(0);
    p.c[1].op = LCPP_HIP_PRED_TRUE;
    return p;
}

struct Outputs {
    void* out = nullptr;
    void* out2 = nullptr;
    void* out3 = nullptr;  // caller's three-way unselected output
    void* values_out = nullptr;
    uint32_t* aux0 = nullptr;
    uint32_t* aux1 = nullptr;
    uint32_t* num_out = nullptr;
};

// Shared host path: checks, temp carving, state reset, launch, and the second kernel of the in-place
// select and of the three-way partition.
template <typename U, typename P, typename V, int MODE, bool FLAGS>
int run_compact(const char* what, void* temp, size_t temp_bytes, const U* in, const P* flags, const V* values_in,
                const Outputs& o, uint64_t n, uint64_t key_mask, const Predicate<P>& pred,
                const Predicate<P>& pred2, bool partition, hipStream_t stream) {
    constexpr int ITEMS = kCpItems<U, V>;
    constexpr uint64_t kTile = static_cast<uint64_t>(kCpBlock) * ITEMS;
    constexpr int W = kWords<MODE>;
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items", what);
    if (!o.num_out) return set_error(kInvalidArgument, "%s: null count output", what);
    if (n == 0) return launch_fill_u32(o.num_out, MODE == kThreeWay ? 2 : 1, 0u, stream);
    if (!in || (FLAGS && !flags) || (MODE == kUniqueByKey && !values_in))
        return set_error(kInvalidArgument, "%s: null input", what);
    if (!o.out && MODE != kNonTrivial) return set_error(kInvalidArgument, "%s: null output", what);
    if ((MODE == kThreeWay && (!o.out2 || !o.out3)) || (MODE == kUniqueByKey && !o.values_out) ||
        ((MODE == kEncode || MODE == kNonTrivial) && !o.aux0) || (MODE == kNonTrivial && !o.aux1))
        return set_error(kInvalidArgument, "%s: null output", what);
    // Selects whose output overlaps their input or flags run into temp storage and copy back.
    const bool in_place = MODE != kNonTrivial && MODE != kThreeWay &&
                          (overlaps(o.out, n * sizeof(U), in, n * sizeof(U)) ||
                           (FLAGS && overlaps(o.out, n * sizeof(U), flags, n * sizeof(P))));
    if (in_place && (partition || MODE == kUniqueByKey))
        return set_error(kInvalidArgument, "%s: output overlaps the input", what);
    const TempPlan plan = plan_temp(n, kTile, W, (in_place || MODE == kThreeWay) ? sizeof(U) : 0);
    if (!temp || temp_bytes < plan.total)
        return set_error(kTempTooSmall, "%s: temp storage too small (%zu < %zu bytes)", what, temp_bytes, plan.total);
    if (reinterpret_cast<uintptr_t>(temp) % 8 != 0) return set_error(kInvalidArgument, "%s: temp not 8-byte aligned", what);
    if (plan.tiles > 0x7FFFFFFFull) return set_error(kInvalidArgument, "%s: too many tiles", what);
    U* const stage = reinterpret_cast<U*>(static_cast<unsigned char*>(temp) + plan.stage_offset);

    CompactArgs<U, P, V> a{};
    a.in = in;
    a.flags = flags;
    a.values_in = values_in;
    a.out = in_place ? stage : static_cast<U*>(o.out);
    a.out2 = static_cast<U*>(o.out2);
    a.out3 = MODE == kThreeWay ? stage : nullptr;
    a.values_out = static_cast<V*>(o.values_out);
    a.aux0 = o.aux0;
    a.aux1 = o.aux1;
    a.num_out = o.num_out;
    a.states = static_cast<uint64_t*>(temp);
    a.n = n;
    a.key_mask = key_mask;
    a.pred = pred;
    a.pred2 = pred2;
    a.spin_limit = lookback_spin_limit();
    a.partition = partition;

    if constexpr (MODE == kSelect && std::is_same_v<U, V> && (sizeof(U) == 4 || sizeof(U) == 8) &&
                  (!FLAGS || sizeof(P) <= 4)) {
        // Selects and partitions that are not in place take the register-resident rows kernel when the
        // input (and the flags) allow whole-vector row loads.  Its tiles are larger, so its states take
        // less temp storage than the plan checked above.
        if (!in_place && g_select_rows.load(std::memory_order_relaxed) && reinterpret_cast<uintptr_t>(in) % 16 == 0 &&
            (!FLAGS || reinterpret_cast<uintptr_t>(flags) % (kRowItems<U> * sizeof(P)) == 0)) {
            const TempPlan rp = plan_temp(n, kRowsTile<U, FLAGS>, 1, 0);
            int st = launch_fill_u32(reinterpret_cast<uint32_t*>(temp), rp.state_bytes / 4, 0u, stream);
            if (st != kOk) return st;
            LaunchScope scope("compact", stream);
            select_rows_kernel<U, P, FLAGS><<<static_cast<unsigned>(rp.tiles), kRowsBlock, 0, stream>>>(a);
            return check_hip(hipGetLastError(), "compact rows launch");
        }
    }
    int st = launch_fill_u32(reinterpret_cast<uint32_t*>(temp), plan.state_bytes / 4, 0u, stream);
    if (st != kOk) return st;
    {
        LaunchScope scope("compact", stream);
        compact_kernel<U, P, V, MODE, FLAGS><<<static_cast<unsigned>(plan.tiles), kCpBlock, 0, stream>>>(a);
        st = check_hip(hipGetLastError(), "compact launch");
        if (st != kOk) return st;
    }
    if (in_place) {
        LaunchScope scope("compact_copy_back", stream);
        copy_prefix_kernel<U><<<grid_for(n), 256, 0, stream>>>(static_cast<U*>(o.out), stage, o.num_out);
        return check_hip(hipGetLastError(), "compact copy-back launch");
    }
    if constexpr (MODE == kThreeWay) {
        LaunchScope scope("compact_reverse_rejects", stream);
        reverse_rejects_kernel<U><<<grid_for(n), 256, 0, stream>>>(static_cast<U*>(o.out3), stage, o.num_out, n);
        return check_hip(hipGetLastError(), "compact reverse launch");
    }
    return kOk;
}

template <typename T>
using Storage = std::conditional_t<sizeof(T) == 8, uint64_t, uint32_t>;

// Key type for adjacency tests: floats compare by value, integers by bits under the mask.
template <typename T>
using KeyOf = std::conditional_t<std::is_floating_point_v<T>, T, Storage<T>>;

}  // namespace
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

// Temp storage the compaction kernels carve: per tile of 8192 (4-byte items) or 4096 (8-byte items)
// one or two state words and a claim word, plus n items of staging for in-place selects and the
// three-way partition; never more than the reference's Get*TempStorageBytes.
size_t lcpp_hip_internal_compact_needed_bytes(uint64_t n, size_t item_bytes, int words, int staged) {
    if (n == 0) return 0;
    const uint64_t tile = static_cast<uint64_t>(kCpBlock) * (128 / item_bytes);
    return plan_temp(n, tile, words, staged ? item_bytes : 0).total;
}

int lcpp_hip_internal_compact_rows(int enable) {
    return g_select_rows.exchange(enable != 0, std::memory_order_relaxed) ? 1 : 0;
}

#define LCPP_HIP_DEFINE_SELECT_FLAGS(TS, TT, FS, FT)                                                                 \
    int lcpp_hip_select_flagged_##TS##_##FS(void* temp, size_t temp_bytes, const TT* in, const FT* flags, TT* out,   \
                                            uint32_t* num_selected_out, uint64_t n, void* stream) {                 \
        using U = Storage<TT>;                                                                                       \
        Outputs o;                                                                                                   \
        o.out = out;                                                                                                 \
        o.num_out = num_selected_out;                                                                                \
        const auto p = nonzero_predicate<FT>();                                                                      \
        return run_compact<U, FT, U, kSelect, true>("DeviceSelect::Flagged", temp, temp_bytes,                       \
                                                    reinterpret_cast<const U*>(in), flags, nullptr, o, n, 0, p, p,   \
                                                    false, static_cast<hipStream_t>(stream));                        \
    }                                                                                                                \
    int lcpp_hip_select_flagged_if_##TS##_##FS(void* temp, size_t temp_bytes, const TT* in, const FT* flags,        \
                                               TT* out, uint32_t* num_selected_out, uint64_t n,                     \
                                               const lcpp_hip_predicate* pred, void* stream) {                      \
        using U = Storage<TT>;                                                                                       \
        Predicate<FT> p;                                                                                             \
        const int st = convert_predicate(pred, p, "DeviceSelect::FlaggedIf");                                        \
        if (st != kOk) return st;                                                                                    \
        Outputs o;                                                                                                   \
        o.out = out;                                                                                                 \
        o.num_out = num_selected_out;                                                                                \
        return run_compact<U, FT, U, kSelect, true>("DeviceSelect::FlaggedIf", temp, temp_bytes,                     \
                                                    reinterpret_cast<const U*>(in), flags, nullptr, o, n, 0, p, p,   \
                                                    false, static_cast<hipStream_t>(stream));                        \
    }                                                                                                                \
    int lcpp_hip_partition_flagged_##TS##_##FS(void* temp, size_t temp_bytes, const TT* in, const FT* flags,        \
                                               TT* out, uint32_t* num_selected_out, uint64_t n, void* stream) {     \
        using U = Storage<TT>;                                                                                       \
        Outputs o;                                                                                                   \
        o.out = out;                                                                                                 \
        o.num_out = num_selected_out;                                                                                \
        const auto p = nonzero_predicate<FT>();                                                                      \
        return run_compact<U, FT, U, kSelect, true>("DevicePartition::Flagged", temp, temp_bytes,                    \
                                                    reinterpret_cast<const U*>(in), flags, nullptr, o, n, 0, p, p,   \
                                                    true, static_cast<hipStream_t>(stream));                         \
    }

#define LCPP_HIP_DEFINE_SELECT_FLAG_TYPES(TS, TT)           \
    LCPP_HIP_DEFINE_SELECT_FLAGS(TS, TT, b8, uint8_t)       \
    LCPP_HIP_DEFINE_SELECT_FLAGS(TS, TT, i32, int32_t)      \
    LCPP_HIP_DEFINE_SELECT_FLAGS(TS, TT, u32, uint32_t)     \
    LCPP_HIP_DEFINE_SELECT_FLAGS(TS, TT, i64, int64_t)      \
    LCPP_HIP_DEFINE_SELECT_FLAGS(TS, TT, u64, uint64_t)

#define LCPP_HIP_DEFINE_SELECT_ITEMS(TS, TT)                                                                         \
    int lcpp_hip_select_if_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out, uint32_t* num_selected_out,   \
                                uint64_t n, const lcpp_hip_predicate* pred, void* stream) {                          \
        Predicate<TT> p;                                                                                             \
        const int st = convert_predicate(pred, p, "DeviceSelect::If");                                               \
        if (st != kOk) return st;                                                                                    \
        Outputs o;                                                                                                   \
        o.out = out;                                                                                                 \
        o.num_out = num_selected_out;                                                                                \
        return run_compact<TT, TT, TT, kSelect, false>("DeviceSelect::If", temp, temp_bytes, in, nullptr, nullptr,  \
                                                       o, n, 0, p, p, false, static_cast<hipStream_t>(stream));      \
    }                                                                                                                \
    int lcpp_hip_partition_if_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out,                            \
                                   uint32_t* num_selected_out, uint64_t n, const lcpp_hip_predicate* pred,           \
                                   void* stream) {                                                                   \
        Predicate<TT> p;                                                                                             \
        const int st = convert_predicate(pred, p, "DevicePartition::If");                                            \
        if (st != kOk) return st;                                                                                    \
        Outputs o;                                                                                                   \
        o.out = out;                                                                                                 \
        o.num_out = num_selected_out;                                                                                \
        return run_compact<TT, TT, TT, kSelect, false>("DevicePartition::If", temp, temp_bytes, in, nullptr,        \
                                                       nullptr, o, n, 0, p, p, true, static_cast<hipStream_t>(stream)); \
    }                                                                                                                \
    int lcpp_hip_partition_three_way_##TS(void* temp, size_t temp_bytes, const TT* in, TT* first_out,               \
                                          TT* second_out, TT* unselected_out, uint32_t* num_selected_out,            \
                                          uint64_t n, const lcpp_hip_predicate* select_first,                       \
                                          const lcpp_hip_predicate* select_second, void* stream) {                  \
        Predicate<TT> p1, p2;                                                                                        \
        int st = convert_predicate(select_first, p1, "DevicePartition::If (three-way)");                            \
        if (st != kOk) return st;                                                                                    \
        st = convert_predicate(select_second, p2, "DevicePartition::If (three-way)");                               \
        if (st != kOk) return st;                                                                                    \
        Outputs o;                                                                                                   \
        o.out = first_out;                                                                                           \
        o.out2 = second_out;                                                                                         \
        o.out3 = unselected_out;                                                                                     \
        o.num_out = num_selected_out;                                                                                \
        return run_compact<TT, TT, TT, kThreeWay, false>("DevicePartition::If (three-way)", temp, temp_bytes, in,  \
                                                         nullptr, nullptr, o, n, 0, p1, p2, false,                  \
                                                         static_cast<hipStream_t>(stream));                          \
    }                                                                                                                \
    int lcpp_hip_select_unique_##TS(void* temp, size_t temp_bytes, const TT* in, TT* out,                           \
                                    uint32_t* num_selected_out, uint64_t n, uint64_t key_mask, void* stream) {      \
        using K = KeyOf<TT>;                                                                                         \
        const int fast = runs_by_key<K>(temp, temp_bytes, reinterpret_cast<const K*>(in), reinterpret_cast<K*>(out), \
                                        nullptr, num_selected_out, n, key_mask, static_cast<hipStream_t>(stream));  \
        if (fast != kRunsDeclined) return fast;                                                                      \
        Outputs o;                                                                                                   \
        o.out = out;                                                                                                 \
        o.num_out = num_selected_out;                                                                                \
        const Predicate<K> none{};                                                                                   \
        return run_compact<K, K, K, kUnique, false>("DeviceSelect::Unique", temp, temp_bytes,                        \
                                                    reinterpret_cast<const K*>(in), nullptr, nullptr, o, n, key_mask, \
                                                    none, none, false, static_cast<hipStream_t>(stream));            \
    }                                                                                                                \
    int lcpp_hip_run_length_encode_##TS(void* temp, size_t temp_bytes, const TT* in, TT* unique_out,                \
                                        uint32_t* counts_out, uint32_t* num_runs_out, uint64_t n, void* stream) {   \
        using K = KeyOf<TT>;                                                                                         \
        const int fast = runs_by_key<K>(temp, temp_bytes, reinterpret_cast<const K*>(in),                           \
                                        reinterpret_cast<K*>(unique_out), counts_out, num_runs_out, n, ~0ull,       \
                                        static_cast<hipStream_t>(stream));                                           \
        if (fast != kRunsDeclined) return fast;                                                                      \
        Outputs o;                                                                                                   \
        o.out = unique_out;                                                                                          \
        o.aux0 = counts_out;                                                                                         \
        o.num_out = num_runs_out;                                                                                    \
        const Predicate<K> none{};                                                                                   \
        return run_compact<K, K, K, kEncode, false>("DeviceRunLengthEncode::Encode", temp, temp_bytes,               \
                                                    reinterpret_cast<const K*>(in), nullptr, nullptr, o, n, ~0ull,  \
                                                    none, none, false, static_cast<hipStream_t>(stream));            \
    }                                                                                                                \
    int lcpp_hip_run_length_non_trivial_##TS(void* temp, size_t temp_bytes, const TT* in, uint32_t* offsets_out,    \
                                             uint32_t* lengths_out, uint32_t* num_runs_out, uint64_t n,              \
                                             void* stream) {                                                         \
        using K = KeyOf<TT>;                                                                                         \
        Outputs o;                                                                                                   \
        o.aux0 = offsets_out;                                                                                        \
        o.aux1 = lengths_out;                                                                                        \
        o.num_out = num_runs_out;                                                                                    \
        const Predicate<K> none{};                                                                                   \
        return run_compact<K, K, K, kNonTrivial, false>("DeviceRunLengthEncode::NonTrivialRuns", temp, temp_bytes,  \
                                                        reinterpret_cast<const K*>(in), nullptr, nullptr, o, n,     \
                                                        ~0ull, none, none, false, static_cast<hipStream_t>(stream)); \
    }                                                                                                                \
    LCPP_HIP_DEFINE_SELECT_FLAG_TYPES(TS, TT)

LCPP_HIP_DEFINE_SELECT_ITEMS(i32, int32_t)
LCPP_HIP_DEFINE_SELECT_ITEMS(u32, uint32_t)
LCPP_HIP_DEFINE_SELECT_ITEMS(f32, float)
LCPP_HIP_DEFINE_SELECT_ITEMS(i64, int64_t)
LCPP_HIP_DEFINE_SELECT_ITEMS(u64, uint64_t)
LCPP_HIP_DEFINE_SELECT_ITEMS(f64, double)

#define LCPP_HIP_DEFINE_UNIQUE_BY_KEY(KS, KT, VS, VT)                                                                \
    int lcpp_hip_select_unique_by_key_##KS##_##VS(void* temp, size_t temp_bytes, const KT* keys_in,                 \
                                                  const VT* values_in, KT* keys_out, VT* values_out,                 \
                                                  uint32_t* num_selected_out, uint64_t n, uint64_t key_mask,         \
                                                  void* stream) {                                                    \
        using K = KeyOf<KT>;                                                                                         \
        using V = Storage<VT>;                                                                                       \
        Outputs o;                                                                                                   \
        o.out = keys_out;                                                                                            \
        o.values_out = values_out;                                                                                   \
        o.num_out = num_selected_out;                                                                                \
        const Predicate<K> none{};                                                                                   \
        return run_compact<K, K, V, kUniqueByKey, false>("DeviceSelect::UniqueByKey", temp, temp_bytes,              \
                                                         reinterpret_cast<const K*>(keys_in), nullptr,               \
                                                         reinterpret_cast<const V*>(values_in), o, n, key_mask,      \
                                                         none, none, false, static_cast<hipStream_t>(stream));       \
    }
#define LCPP_HIP_DEFINE_UNIQUE_BY_KEY_VALUES(KS, KT)          \
    LCPP_HIP_DEFINE_UNIQUE_BY_KEY(KS, KT, i32, int32_t)       \
    LCPP_HIP_DEFINE_UNIQUE_BY_KEY(KS, KT, u32, uint32_t)      \
    LCPP_HIP_DEFINE_UNIQUE_BY_KEY(KS, KT, f32, float)         \
    LCPP_HIP_DEFINE_UNIQUE_BY_KEY(KS, KT, i64, int64_t)       \
    LCPP_HIP_DEFINE_UNIQUE_BY_KEY(KS, KT, u64, uint64_t)      \
    LCPP_HIP_DEFINE_UNIQUE_BY_KEY(KS, KT, f64, double)
LCPP_HIP_DEFINE_UNIQUE_BY_KEY_VALUES(i32, int32_t)
LCPP_HIP_DEFINE_UNIQUE_BY_KEY_VALUES(u32, uint32_t)
LCPP_HIP_DEFINE_UNIQUE_BY_KEY_VALUES(f32, float)
LCPP_HIP_DEFINE_UNIQUE_BY_KEY_VALUES(i64, int64_t)
LCPP_HIP_DEFINE_UNIQUE_BY_KEY_VALUES(u64, uint64_t)
LCPP_HIP_DEFINE_UNIQUE_BY_KEY_VALUES(f64, double)

#undef LCPP_HIP_DEFINE_UNIQUE_BY_KEY_VALUES
#undef LCPP_HIP_DEFINE_UNIQUE_BY_KEY
#undef LCPP_HIP_DEFINE_SELECT_ITEMS
#undef LCPP_HIP_DEFINE_SELECT_FLAG_TYPES
#undef LCPP_HIP_DEFINE_SELECT_FLAGS

}  // extern "C"
