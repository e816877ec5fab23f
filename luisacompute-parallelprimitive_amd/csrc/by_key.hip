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
//   * Tile = 512 threads x 16 consecutive items per thread (8192 items), read and written as
//     16-byte vectors when the arrays are 16-byte aligned.  The previous item of a thread's first
//     item is read from global memory (it sits in the neighbour's cache line).
//   * State of a span of items: (heads, sum since the last head).  States combine as
//     (c1, s1) + (c2, s2) = (c1 + c2, c2 ? s2 : s1 + s2), which is associative.  Each thread folds its
//     items serially; a DPP wave scan (the shared row_shr / row_bcast pattern) and one pass over the
//     8 wave totals in LDS give each thread its carry-in and the tile its aggregate.
//   * Tile states are 64-bit words with the status in the low half and 32 payload bits in the high
//     half.  Reduce-by-key: word 0 holds the head count, words 1.. the sum.  Scan-by-key needs only
//     a has-head flag, kept beside the status, so its state is just the sum words (one word for
//     4-byte values: half the look-back loads).  A reader accepts a state only when every
//     word shows the same published status, so each word is one relaxed agent-scope atomic (the 8
//     XCDs do not share an L2) and no fence is needed.  The owner publishes PARTIAL (tile 0:
//     INCLUSIVE) with plain stores from lane 0 of its last wave: a wave's vector memory operations
//     complete in issue order, so stores issued by wave 0 would delay its own look-back loads.
//   * Look-back: wave 0 reads 64 predecessors per step (one per lane).  Ballots find the newest
//     INCLUSIVE state (or tile 0) and, for the scan, the newest state with a head: the scan stops
//     there because older sums cannot reach this tile; ReduceByKey continues to an INCLUSIVE state
//     since run indices need the full head count.  Counts and sums reduce with DPP.
//   * Forward progress never depends on dispatch order.  Each tile has a claim word (in an array
//     after the state slots).  A predecessor still unpublished after `spin_limit` polls is claimed
//     by compare-and-swap
//     (OPEN -> HELPER), its state computed by the whole waiting workgroup with the owner's own code
//     (the same float summation order) and published PARTIAL, then the claim is marked DONE with
//     release ordering.  The owner closes its claim word (OPEN -> OWNED) right after publishing and
//     looks at the result only after its look-back; if a helper got there first it waits for DONE
//     before publishing INCLUSIVE or storing outputs, so no PARTIAL store can land after its
//     INCLUSIVE ones and an in-place scan never overwrites input a helper still reads.
// Algorithmic traffic: scan n*(sizeof(K) + 2*sizeof(V)); reduce n*(sizeof(K) + sizeof(V)) plus
// runs*(sizeof(K) + sizeof(V)) written.
#include "common.hpp"
#include "../../include/lcpp_hip.h"

namespace lcpp_hip {
namespace {

constexpr int kBkItems = 16;
// 512 threads: 8192-item tiles halve the tiles (and look-backs) of 256-thread ones at the same items
// per CU in flight (two workgroups per CU at the register use of the reduce instantiations);
// ExclusiveSumByKey 2^28 0.906 -> 0.819 ms, ReduceByKey 0.802 -> 0.760 ms, 1024 threads no better.
constexpr int kBkBlock = 512;
constexpr uint32_t kBkTile = static_cast<uint32_t>(kBkBlock) * kBkItems;  // 8192 items

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

// Look-back decisions broadcast from wave 0.
constexpr uint32_t kActDone = 0;
constexpr uint32_t kActAdvance = 1;
constexpr uint32_t kActWait = 2;
constexpr uint32_t kActHelp = 3;

template <typename V>
struct Seg {
    uint32_t count;  // run heads in the span
    V sum;           // sum of the items after the span's last head (all items if it has none)
};

template <typename V>
__device__ __forceinline__ Seg<V> seg_combine(Seg<V> older, Seg<V> newer) {
    Seg<V> r;
    r.count = older.count + newer.count;
    r.sum = newer.count != 0 ? newer.sum : static_cast<V>(older.sum + newer.sum);
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
size_t state_bytes(uint64_t n, size_t value_bytes, bool counted) {
    return ceil_div(n, kBkTile) * ((counted ? 2 : 1) + value_bytes / 4) * sizeof(uint64_t);
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

template <typename T>
struct alignas(16) Run16 {
    T v[kBkItems];
};

// The 16 items [first, first + 16) of `p` (0 past n): one 64/128-byte vector load when aligned.
template <typename T>
__device__ __forceinline__ void load_items(const T* p, uint64_t first, uint64_t n, bool vec, T (&out)[kBkItems]) {
    if (vec && first + kBkItems <= n) {
        const Run16<T> r = *reinterpret_cast<const Run16<T>*>(p + first);
#pragma unroll
        for (int k = 0; k < kBkItems; ++k) out[k] = r.v[k];
    } else {
#pragma unroll
        for (int k = 0; k < kBkItems; ++k) out[k] = first + k < n ? p[first + k] : T(0);
    }
}

template <typename T>
__device__ __forceinline__ void store_items(T* p, uint64_t first, uint64_t n, bool vec, const T (&in)[kBkItems]) {
    if (vec && first + kBkItems <= n) {
        Run16<T> r;
#pragma unroll
        for (int k = 0; k < kBkItems; ++k) r.v[k] = in[k];
        *reinterpret_cast<Run16<T>*>(p + first) = r;
    } else {
#pragma unroll
        for (int k = 0; k < kBkItems; ++k) {
            if (first + k < n) p[first + k] = in[k];
        }
    }
}

template <typename K, typename V>
struct ThreadItems {
    K key[kBkItems];
    V val[kBkItems];
    uint32_t heads;  // bit k: item k starts a run
};

template <typename K, typename V>
__device__ __forceinline__ void load_thread(const K* keys, const V* values, uint64_t n, uint64_t first, K mask,
                                            bool vec_k, bool vec_v, ThreadItems<K, V>& t) {
    load_items(keys, first, n, vec_k, t.key);
    load_items(values, first, n, vec_v, t.val);
    K prev = (first > 0 && first - 1 < n) ? keys[first - 1] : K(0);
    uint32_t heads = 0;
#pragma unroll
    for (int k = 0; k < kBkItems; ++k) {
        const uint64_t i = first + k;
        const bool head = i < n && (i == 0 || ((t.key[k] ^ prev) & mask) != 0);
        heads |= (head ? 1u : 0u) << k;
        prev = t.key[k];
    }
    t.heads = heads;
}

template <typename K, typename V>
__device__ __forceinline__ Seg<V> fold_thread(const ThreadItems<K, V>& t, uint64_t first, uint64_t n) {
    Seg<V> s{0u, V(0)};
#pragma unroll
    for (int k = 0; k < kBkItems; ++k) {
        if (first + k < n) {
            if ((t.heads >> k) & 1u) {
                s.count += 1;
                s.sum = t.val[k];
            } else {
                s.sum = static_cast<V>(s.sum + t.val[k]);
            }
        }
    }
    return s;
}

// One step of the wave scan: combine with the state DPP brings from an older lane (identity where
// the pattern has no source).
template <int CTRL, int ROW_MASK = 0xf, typename V>
__device__ __forceinline__ Seg<V> seg_dpp_step(Seg<V> x) {
    Seg<V> o;
    o.count = dpp_move_u32<CTRL, ROW_MASK>(0u, x.count);
    o.sum = dpp_move<CTRL, ROW_MASK>(V(0), x.sum);
    return seg_combine(o, x);
}

// Exclusive prefix of each thread's state within the tile, and the tile aggregate.  Called by every
// thread; leaves `s_wave` free for reuse (barriers on both sides of its use).
template <int BLOCK, typename V>
__device__ __forceinline__ void block_seg_scan(Seg<V> x, Seg<V>* s_wave, Seg<V>& exclusive, Seg<V>& aggregate) {
    Seg<V> inc = x;
    inc = seg_dpp_step<dpp::kRowShr1>(inc);
    inc = seg_dpp_step<dpp::kRowShr2>(inc);
    inc = seg_dpp_step<dpp::kRowShr4>(inc);
    inc = seg_dpp_step<dpp::kRowShr8>(inc);
    inc = seg_dpp_step<dpp::kRowBcast15, 0xa>(inc);
    inc = seg_dpp_step<dpp::kRowBcast31, 0xc>(inc);
    Seg<V> ex;
    ex.count = dpp_move_u32<dpp::kWaveShr1>(0u, inc.count);
    ex.sum = dpp_move<dpp::kWaveShr1>(V(0), inc.sum);
    const uint32_t wave = threadIdx.x / kWave;
    __syncthreads();  // earlier readers of s_wave are done
    if (lane_id() == kWave - 1) s_wave[wave] = inc;
    __syncthreads();
    Seg<V> prefix{0u, V(0)};
    Seg<V> total{0u, V(0)};
#pragma unroll
    for (int w = 0; w < BLOCK / kWave; ++w) {
        if (static_cast<uint32_t>(w) == wave) prefix = total;
        total = seg_combine(total, s_wave[w]);
    }
    exclusive = seg_combine(prefix, ex);
    aggregate = total;
}

// Aggregate of tile `tile`, computed by the whole workgroup exactly as the tile's owner computes it.
template <int BLOCK, typename K, typename V>
__device__ Seg<V> tile_aggregate(const K* keys, const V* values, uint64_t n, uint32_t tile, K mask, bool vec_k,
                                 bool vec_v, Seg<V>* s_wave) {
    const uint64_t first = static_cast<uint64_t>(tile) * (BLOCK * kBkItems) + static_cast<uint64_t>(threadIdx.x) * kBkItems;
    ThreadItems<K, V> t;
    load_thread(keys, values, n, first, mask, vec_k, vec_v, t);
    Seg<V> ex, agg;
    block_seg_scan<BLOCK>(fold_thread(t, first, n), s_wave, ex, agg);
    return agg;
}

// Scan outputs of a thread's items from the state carried into its first item.
template <typename K, typename V>
__device__ __forceinline__ void scan_outputs(const ThreadItems<K, V>& t, Seg<V> run, int inclusive, int use_init, V init,
                                             V* values_out, uint64_t first, uint64_t n, bool vec_o) {
    V out[kBkItems];
#pragma unroll
    for (int k = 0; k < kBkItems; ++k) {
        const bool head = (t.heads >> k) & 1u;
        if (!inclusive) out[k] = head ? init : static_cast<V>(init + run.sum);
        if (head) {
            run.count += 1;
            run.sum = t.val[k];
        } else {
            run.sum = static_cast<V>(run.sum + t.val[k]);
        }
        if (inclusive) out[k] = use_init ? static_cast<V>(init + run.sum) : run.sum;
    }
    store_items(values_out, first, n, vec_o, out);
}

template <int BLOCK, typename K, typename V, int MODE>
__global__ __launch_bounds__(BLOCK) void by_key_kernel(const K* __restrict__ keys, const V* values_in,
                                                          V* values_out, K* __restrict__ unique_out,
                                                          V* __restrict__ aggregates_out,
                                                          uint32_t* __restrict__ num_runs_out, uint64_t n, K mask,
                                                          uint64_t* __restrict__ states, int inclusive, int use_init,
                                                          V init, bool vec_k, bool vec_v, bool vec_o,
                                                          bool in_place, uint32_t spin_limit) {
    constexpr bool COUNTED = MODE == kModeReduce;
    constexpr int W = kStateWords<V, COUNTED>;
    uint64_t* const claims = states + static_cast<uint64_t>(gridDim.x) * W;
    // The thread that publishes this tile's states and closes its claim word: lane 0 of the last
    // wave.  A wave's vector memory operations complete in issue order, so publishing from wave 0
    // would make its look-back loads wait for the publishing stores and the compare-and-swap.
    constexpr uint32_t kPublisher = BLOCK - kWave;
    __shared__ Seg<V> s_wave[BLOCK / kWave];
    __shared__ uint32_t s_ctl[2][2];  // look-back decision and helped tile, two alternating rows
    __shared__ Seg<V> s_prefix;

    const uint32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t wave = tid / kWave;
    const uint32_t tile = blockIdx.x;
    const uint64_t first = static_cast<uint64_t>(tile) * (BLOCK * kBkItems) + static_cast<uint64_t>(tid) * kBkItems;

    ThreadItems<K, V> t;
    load_thread(keys, values_in, n, first, mask, vec_k, vec_v, t);
    Seg<V> in_tile, agg;
    block_seg_scan<BLOCK>(fold_thread(t, first, n), s_wave, in_tile, agg);

    // Publish PARTIAL (INCLUSIVE for tile 0) with plain stores, then close the claim word; the
    // compare-and-swap's result is only needed after the look-back.  A helper that claimed the tile
    // first stores the same PARTIAL values.
    uint64_t* const my_slot = states + static_cast<uint64_t>(tile) * W;
    bool owned = true;
    if (tid == kPublisher) {
        const uint32_t st = tile == 0 ? kStInclusive : kStPartial;
        publish_state<V, COUNTED>(my_slot, st, agg);
        uint64_t expected = kClaimOpen;
        owned = __hip_atomic_compare_exchange_strong(&claims[tile], &expected, kClaimOwned, __ATOMIC_RELAXED,
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Scan outputs that do not depend on the tile's prefix (a run starts in this tile before or at the
    // thread's first item) are stored now, after the publish and by waves other than wave 0, so they
    // overlap the look-back without delaying the publish or wave 0's look-back loads (a wave's
    // vector memory operations complete in issue order).  Not for in-place scans: their input may
    // still be read by a helper until the claim is settled.
    bool early = false;
    if constexpr (MODE == kModeScan) {
        early = !in_place && wave != 0 && (in_tile.count != 0 || (t.heads & 1u) != 0);
        if (early) scan_outputs(t, in_tile, inclusive, use_init, init, values_out, first, n, vec_o);
    }

    Seg<V> prefix{0u, V(0)};
    if (tile > 0) {
        int64_t top = static_cast<int64_t>(tile) - 1;  // newest predecessor not yet consumed
        Seg<V> acc{0u, V(0)};                           // states consumed so far (wave 0)
        uint32_t spins = 0;
        uint32_t row = 0;
        while (true) {
            if (wave == 0) {
                const int64_t j = top - static_cast<int64_t>(lane);
                Seg<V> s{0u, V(0)};
                const uint32_t st = j >= 0 ? read_state<V, COUNTED>(states + static_cast<uint64_t>(j) * W, s) : kStInvalid;
                const bool exists = j >= 0;
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
                    window.sum = wave_reduce((exists && lane <= sum_cut) ? s.sum : V(0), SumOp{});
                    acc = seg_combine(window, acc);
                    const bool complete = stop_mask != 0 && cut == static_cast<uint32_t>(__builtin_ctzll(stop_mask));
                    const bool found_head = MODE == kModeScan && heads_in != 0;
                    action = (complete || found_head || top < kWave) ? kActDone : kActAdvance;
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
                top -= kWave;
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
                const Seg<V> h = tile_aggregate<BLOCK, K, V>(keys, values_in, n, help_tile, mask, vec_k, vec_v, s_wave);
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
            const Seg<V> incl = seg_combine(prefix, agg);
            publish_state<V, COUNTED>(my_slot, kStInclusive, incl);
        }
    }
    __syncthreads();  // outputs only after the claim is settled

    Seg<V> run = seg_combine(prefix, in_tile);
    if constexpr (MODE == kModeScan) {
        if (!early) scan_outputs(t, run, inclusive, use_init, init, values_out, first, n, vec_o);
    } else {
#pragma unroll
        for (int k = 0; k < kBkItems; ++k) {
            if (first + k < n) {
                if ((t.heads >> k) & 1u) {
                    if (run.count > 0) aggregates_out[run.count - 1] = run.sum;
                    unique_out[run.count] = t.key[k];
                    run.count += 1;
                    run.sum = t.val[k];
                } else {
                    run.sum = static_cast<V>(run.sum + t.val[k]);
                }
            }
        }
        if (first < n && n - first <= kBkItems) {  // this thread holds the last item
            aggregates_out[run.count - 1] = run.sum;
            num_runs_out[0] = run.count;
        }
    }
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

template <typename K, typename V, int MODE>
int by_key(void* temp, size_t temp_bytes, const K* keys, const V* values_in, V* values_out, K* unique_out,
           V* aggregates_out, uint32_t* num_runs_out, uint64_t n, uint64_t key_mask, int inclusive, int use_init,
           V init, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const char* what = MODE == kModeScan ? "DeviceScan::ScanByKey" : "DeviceReduce::ReduceByKey";
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items", what);
    if constexpr (MODE == kModeReduce) {
        if (!num_runs_out) return set_error(kInvalidArgument, "%s: null run-count output", what);
        if (n == 0) return launch_fill_u32(num_runs_out, 1, 0u, stream);
        if (!unique_out || !aggregates_out) return set_error(kInvalidArgument, "%s: null output", what);
    } else {
        if (n == 0) return kOk;
        if (!values_out) return set_error(kInvalidArgument, "%s: null output", what);
    }
    if (!keys || !values_in) return set_error(kInvalidArgument, "%s: null input", what);
    const size_t need = state_bytes(n, sizeof(V), MODE == kModeReduce);
    if (!temp || temp_bytes < need)
        return set_error(kTempTooSmall, "%s: temp storage too small (%zu < %zu bytes)", what, temp_bytes, need);
    if (reinterpret_cast<uintptr_t>(temp) % 8 != 0) return set_error(kInvalidArgument, "%s: temp not 8-byte aligned", what);
    uint64_t* states = static_cast<uint64_t*>(temp);
    int st = launch_fill_u32(reinterpret_cast<uint32_t*>(states), need / 4, 0u, stream);
    if (st != kOk) return st;
    const uint32_t tiles = static_cast<uint32_t>(ceil_div(n, kBkTile));
    LaunchScope scope(MODE == kModeScan ? "scan_by_key" : "reduce_by_key", stream);
    by_key_kernel<kBkBlock, K, V, MODE><<<tiles, kBkBlock, 0, stream>>>(
        keys, values_in, values_out, unique_out, aggregates_out, num_runs_out, n, static_cast<K>(key_mask), states,
        inclusive, use_init, init, aligned16(keys), aligned16(values_in), values_out != nullptr && aligned16(values_out),
        values_out != nullptr && values_out == values_in, lookback_spin_limit());
    return check_hip(hipGetLastError(), MODE == kModeScan ? "scan_by_key launch" : "reduce_by_key launch");
}

}  // namespace
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

// Temp storage the reduce-by-key kernel carves (the larger of the two layouts: per 8192-item tile a
// count word, sizeof(V)/4 sum words and a claim word); never more than the reference's
// GetScanByKeyTempStorageBytes / GetReduceByKeyTempStorageBytes.
size_t lcpp_hip_internal_by_key_needed_bytes(uint64_t n, size_t value_bytes) { return state_bytes(n, value_bytes, true); }

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

}  // extern "C"
