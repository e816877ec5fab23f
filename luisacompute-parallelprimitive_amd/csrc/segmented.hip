// DeviceSegmentReduce (Sum, Min, Max, ArgMin, ArgMax over begin/end offsets or fixed-size segments)
// and DeviceSegmentedScan (exclusive / inclusive sums, optional initial value, separate output
// offsets) for gfx950.
//
// Reference paths (src/lcpp/device/): DeviceSegmentReduce<> (device_segment_reduce.h:110-420): one
// block per segment; an empty segment (begin == end) writes the initial value (0, the type's max for
// Min, lowest for Max); otherwise reduce_op(initial, aggregate) (details/segment_reduce.h:120-165).
// ArgMin / ArgMax reduce (global index, value) pairs with the lower index winning ties
// (common/thread_operators.h:19-47) and report the index relative to the segment's begin; an empty
// segment reports index 1 and the initial value (details/segment_reduce.h:141-146, 302-345).
// DeviceSegmentedScan<> (device_segmented_scan.h:52-224): segment s scans input[begin[s], end[s]) into
// output[out_begin[s] + k]; exclusive scans start from the initial value (0 for the Sum forms).
//
// MI355X design: one 256-thread workgroup per segment, up to 65,536 segments.  Reductions stream the
// segment with eight loads in flight per thread (consecutive lanes read consecutive items; four 16-byte
// vectors per lane for ranges of at least 512 items), fold in registers, then a DPP wave reduction and a
// 4-wave combine in LDS.  With more segments each wave
// takes batches of consecutive segments (about num_segments / 65,536 of them, 1 to 64): a batch whose
// segments all hold at most 16 items is reduced or scanned one segment per lane, with coalesced offset
// loads; any other batch one segment at a time, a wave taking a segment of at most 1,024 items alone and
// the workgroup longer ones together (workgroup dispatch bounds one-workgroup-per-segment grids).
// Workgroup scans walk the segment in chunks of 2048 items (the next chunk's loads issued before the
// current one is scanned): each thread folds 8 consecutive items (16-byte accesses when the segment
// start is aligned),
// a DPP wave scan and the LDS wave totals give every thread its chunk prefix, and a running carry
// crosses chunks.  Segments with begin >= end are empty.  Integer sums wrap; float sums are ordered
// (per-thread folds, then a fixed tree).
// Algorithmic traffic: reduce sizeof(T) per item + 8 bytes of offsets and sizeof(T) (+4) per segment;
// scan 2 * sizeof(T) per item.
#include "common.hpp"
#include "../../include/lcpp_hip.h"

#include <limits>

namespace lcpp_hip {
namespace {

constexpr int kSgBlock = 256;
constexpr int kSgWaves = kSgBlock / kWave;
constexpr int kSgUnroll = 8;
constexpr int kScanItems = 8;  // consecutive items per thread and scan chunk

enum : int { kOpSum = 0, kOpMin = 1, kOpMax = 2, kOpArgMin = 3, kOpArgMax = 4 };

template <typename T>
struct Arith {
    using type = T;
};
template <>
struct Arith<int32_t> {
    using type = uint32_t;  // wrapping sums
};
template <>
struct Arith<int64_t> {
    using type = uint64_t;
};

template <typename T>
__device__ __forceinline__ T add_wrap(T a, T b) {
    using A = typename Arith<T>::type;
    return static_cast<T>(static_cast<A>(a) + static_cast<A>(b));
}

template <typename T>
struct Arg {
    T value;
    uint32_t index;
};

template <typename T, int OP>
struct Reducer {
    using Acc = std::conditional_t<(OP == kOpArgMin || OP == kOpArgMax), Arg<T>, T>;
    __device__ __forceinline__ static Acc identity() {
        if constexpr (OP == kOpSum) return T(0);
        else if constexpr (OP == kOpMin) return std::numeric_limits<T>::max();
        else if constexpr (OP == kOpMax) return std::numeric_limits<T>::lowest();
        else if constexpr (OP == kOpArgMin) return Arg<T>{std::numeric_limits<T>::max(), 0xFFFFFFFFu};
        else return Arg<T>{std::numeric_limits<T>::lowest(), 0xFFFFFFFFu};
    }
    __device__ __forceinline__ static Acc lift(T v, uint32_t i) {
        if constexpr (OP == kOpArgMin || OP == kOpArgMax) return Arg<T>{v, i};
        else return v;
    }
    __device__ __forceinline__ static Acc combine(Acc a, Acc b) {
        if constexpr (OP == kOpSum) {
            return add_wrap(a, b);
        } else if constexpr (OP == kOpMin) {
            if constexpr (std::is_floating_point_v<T>) return fmin(a, b);
            else return b < a ? b : a;
        } else if constexpr (OP == kOpMax) {
            if constexpr (std::is_floating_point_v<T>) return fmax(a, b);
            else return b > a ? b : a;
        } else if constexpr (OP == kOpArgMin) {
            return (b.value < a.value || (b.value == a.value && b.index < a.index)) ? b : a;
        } else {
            return (b.value > a.value || (b.value == a.value && b.index < a.index)) ? b : a;
        }
    }
};

// Lane `src`'s value of v (src the same in every lane), for 32- and 64-bit types, as a scalar read.
template <typename T>
__device__ __forceinline__ T read_lane_any(T v, int src) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, v), src));
    } else {
        const uint64_t u = __builtin_bit_cast(uint64_t, v);
        const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(u), src);
        const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(u >> 32), src);
        return __builtin_bit_cast(T, (static_cast<uint64_t>(hi) << 32) | lo);
    }
}

// One DPP step of the wave reduction: combine with the accumulator of the lane the pattern names
// (the identity where it names none).
template <int CTRL, int ROW_MASK, typename T, int OP>
__device__ __forceinline__ typename Reducer<T, OP>::Acc dpp_combine(typename Reducer<T, OP>::Acc x) {
    using R = Reducer<T, OP>;
    const typename R::Acc id = R::identity();
    typename R::Acc o;
    if constexpr (OP == kOpArgMin || OP == kOpArgMax) {
        o.value = dpp_move<CTRL, ROW_MASK>(id.value, x.value);
        o.index = dpp_move_u32<CTRL, ROW_MASK>(id.index, x.index);
    } else {
        o = dpp_move<CTRL, ROW_MASK>(id, x);
    }
    return R::combine(x, o);
}

// Reduction over the 64 lanes, the result in every lane: the row_shr / row_bcast scan pattern on the
// DPP datapath (no LDS traffic) leaves the total in lane 63, which is then read into a scalar.
template <typename T, int OP>
__device__ __forceinline__ typename Reducer<T, OP>::Acc wave_combine(typename Reducer<T, OP>::Acc x) {
    x = dpp_combine<dpp::kRowShr1, 0xf, T, OP>(x);
    x = dpp_combine<dpp::kRowShr2, 0xf, T, OP>(x);
    x = dpp_combine<dpp::kRowShr4, 0xf, T, OP>(x);
    x = dpp_combine<dpp::kRowShr8, 0xf, T, OP>(x);
    x = dpp_combine<dpp::kRowBcast15, 0xa, T, OP>(x);
    x = dpp_combine<dpp::kRowBcast31, 0xc, T, OP>(x);
    if constexpr (OP == kOpArgMin || OP == kOpArgMax) {
        x.value = read_lane_any(x.value, kWave - 1);
        x.index = __builtin_amdgcn_readlane(x.index, kWave - 1);
        return x;
    } else {
        return read_lane_any(x, kWave - 1);
    }
}

// Writes segment seg's result (relative index for the Arg forms; empty segments take the identity and
// index 1).
template <typename T, int OP>
__device__ __forceinline__ void write_result(T* out, uint32_t* index_out, uint64_t seg, uint64_t b, bool empty,
                                             typename Reducer<T, OP>::Acc total) {
    if constexpr (OP == kOpArgMin || OP == kOpArgMax) {
        out[seg] = total.value;
        index_out[seg] = empty ? 1u : total.index - static_cast<uint32_t>(b);
    } else {
        out[seg] = total;
    }
}

// Lane-strided fold of [b, e) with kSgUnroll loads in flight per lane; `stride` lanes take part.  From
// the first 16-byte boundary on, the lanes read 16-byte vectors, four in flight each, non-temporally (2^28
// i32 Sum in 4,096-item segments 0.162 -> 0.150 ms; the items before the boundary and after the last whole
// vector one per lane).  The vector path changes the order of the
// fold, so it is left out for float Min / Max, where fmin / fmax may pick either zero of -0.0 and +0.0
// by operand order; sums of floats are held to a tolerance, and the other operators select.  VECTOR
// false: the item loads only (short ranges: the vector path's set-up measured 6-20 % slower on 37-item
// segments).
template <typename T, int OP, bool VECTOR = true>
__device__ __forceinline__ typename Reducer<T, OP>::Acc fold_range(const T* __restrict__ in, uint64_t b, uint64_t e,
                                                                   uint32_t lane, uint32_t stride) {
    using R = Reducer<T, OP>;
    typename R::Acc acc = R::identity();
    constexpr bool kVector =
        VECTOR && sizeof(T) >= 4 && !(std::is_floating_point_v<T> && (OP == kOpMin || OP == kOpMax));
    if constexpr (kVector) {
        constexpr int VEC = 16 / static_cast<int>(sizeof(T));
        const uint64_t a0 = b + ((16u - (reinterpret_cast<uintptr_t>(in + b) & 15u)) & 15u) / sizeof(T);
        if (a0 + static_cast<uint64_t>(VEC) * stride <= e && (reinterpret_cast<uintptr_t>(in) % sizeof(T)) == 0) {
            using Vec = T __attribute__((ext_vector_type(VEC)));
            // a0 - b < VEC <= stride.  Combined with the identity, not assigned: an Arg accumulator holding a
            // NaN would never be replaced, while the identity drops NaN items.
            if (b + lane < a0) acc = R::combine(acc, R::lift(in[b + lane], static_cast<uint32_t>(b + lane)));
            const Vec* vin = reinterpret_cast<const Vec*>(in + a0);
            const uint64_t nvec = (e - a0) / VEC;
            uint64_t v = lane;
            for (; v + 3ull * stride < nvec; v += 4ull * stride) {
                Vec q[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) q[u] = __builtin_nontemporal_load(&vin[v + static_cast<uint64_t>(u) * stride]);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint64_t i0 = a0 + (v + static_cast<uint64_t>(u) * stride) * VEC;
#pragma unroll
                    for (int c = 0; c < VEC; ++c) acc = R::combine(acc, R::lift(q[u][c], static_cast<uint32_t>(i0 + c)));
                }
            }
            for (; v < nvec; v += stride) {
                const Vec q = __builtin_nontemporal_load(&vin[v]);
#pragma unroll
                for (int c = 0; c < VEC; ++c) acc = R::combine(acc, R::lift(q[c], static_cast<uint32_t>(a0 + v * VEC + c)));
            }
            const uint64_t t = a0 + nvec * VEC + lane;
            if (t < e) acc = R::combine(acc, R::lift(in[t], static_cast<uint32_t>(t)));  // e - (a0 + nvec VEC) < VEC
            return acc;
        }
    }
    uint64_t i = b + lane;
    for (; i + static_cast<uint64_t>(kSgUnroll - 1) * stride < e; i += static_cast<uint64_t>(kSgUnroll) * stride) {
        T v[kSgUnroll];
#pragma unroll
        for (int k = 0; k < kSgUnroll; ++k) v[k] = in[i + static_cast<uint64_t>(k) * stride];
#pragma unroll
        for (int k = 0; k < kSgUnroll; ++k)
            acc = R::combine(acc, R::lift(v[k], static_cast<uint32_t>(i + static_cast<uint64_t>(k) * stride)));
    }
    for (; i < e; i += stride) acc = R::combine(acc, R::lift(in[i], static_cast<uint32_t>(i)));
    return acc;
}

// When workgroups take several segments, segments of at most this many items are reduced by one wave and
// longer ones by the whole workgroup.
constexpr uint64_t kSgWaveMax = 1024;
// A wave reads segments of at least this many items as 16-byte vectors.
constexpr uint64_t kSgWaveVector = 512;
// Workgroups of the reduce grid: one per segment up to this many segments; beyond, each wave takes
// batches of `batch` consecutive segments (workgroup g's waves take batches 4 g .. 4 g + 3 of every round
// of 4 G), so that many short segments do not each cost a workgroup dispatch while the grid still fills
// the GPU.  The host sizes the batch to about num_segments / 65,536 (1 to 64): calls with somewhat more
// than 65,536 segments keep about one segment per wave, calls with millions fill every lane.
constexpr uint64_t kSgMaxGroups = 65536;
constexpr uint64_t kSgBatchWaves = 65536;
// A batch whose segments all hold at most this many items is reduced one segment per lane (coalesced
// offset loads and result stores); otherwise the wave takes its segments one at a time.  Measured on 2^28
// i32 Sum, ms per call against one wave per segment: 4-item segments 10.2 -> 0.40, 16: 2.51 -> 0.49,
// 37: 1.17 -> 0.76, 60: 0.75 -> 0.50, 300: 0.44 -> 0.37; with lanes up to 64 items, 60-item segments
// took 1.06 ms.
constexpr uint64_t kSgLaneMax = 16;

template <typename T, int OP>
__global__ __launch_bounds__(kSgBlock) void segment_reduce_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                                  uint32_t* __restrict__ index_out,
                                                                  const uint32_t* __restrict__ begins,
                                                                  const uint32_t* __restrict__ ends,
                                                                  uint64_t fixed_size, uint64_t num_segments,
                                                                  uint32_t batch) {
    using R = Reducer<T, OP>;
    using Acc = typename R::Acc;
    __shared__ Acc s_wave[kSgWaves];
    __shared__ uint64_t s_big[kSgBlock];
    __shared__ uint32_t s_nbig;
    const uint32_t wave = threadIdx.x / kWave;
    const uint64_t groups = gridDim.x;
    auto bounds = [&](uint64_t seg, uint64_t& b, uint64_t& e) {
        if (begins) {
            b = begins[seg];
            e = ends[seg];
        } else {
            b = seg * fixed_size;
            e = b + fixed_size;
        }
    };
    auto block_reduce = [&](uint64_t seg, uint64_t b, uint64_t e) {
        const Acc acc = wave_combine<T, OP>(fold_range<T, OP>(in, b, e, threadIdx.x, kSgBlock));
        if (lane_id() == 0) s_wave[wave] = acc;
        __syncthreads();
        if (threadIdx.x == 0) {
            Acc total = s_wave[0];
#pragma unroll
            for (int w = 1; w < kSgWaves; ++w) total = R::combine(total, s_wave[w]);
            write_result<T, OP>(out, index_out, seg, b, false, total);
        }
    };
    if (num_segments <= groups) {  // one segment per workgroup, which takes it whole
        uint64_t b, e;
        bounds(blockIdx.x, b, e);
        if (b >= e) {
            if (threadIdx.x == 0) write_result<T, OP>(out, index_out, blockIdx.x, b, true, R::identity());
            return;
        }
        block_reduce(blockIdx.x, b, e);
        return;
    }
    for (uint64_t r = 0;; ++r) {
        // Batches of this round: 4 (blockIdx.x + r groups) + w for waves w = 0..3, `batch` segments each.
        const uint64_t batch0 = (blockIdx.x + r * groups) * kSgWaves;
        if (batch0 * batch >= num_segments) break;
        if (threadIdx.x == 0) s_nbig = 0;
        __syncthreads();
        const uint64_t first = (batch0 + wave) * batch;
        if (first < num_segments) {
            const uint32_t count = num_segments - first < batch ? static_cast<uint32_t>(num_segments - first) : batch;
            const uint64_t seg = first + lane_id();
            uint64_t b = 0, e = 0;
            if (lane_id() < count) bounds(seg, b, e);
            const uint64_t len = e > b ? e - b : 0;
            if (wave_ballot(len > kSgLaneMax) == 0) {
                // One segment per lane, 8 loads in flight per step.
                Acc acc = R::identity();
                for (uint64_t i = b; i < e; i += 8) {
                    T v[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) v[k] = i + k < e ? in[i + k] : T(0);
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        if (i + k < e) acc = R::combine(acc, R::lift(v[k], static_cast<uint32_t>(i + k)));
                    }
                }
                if (lane_id() < count) write_result<T, OP>(out, index_out, seg, b, b >= e, acc);
            } else {
                for (uint32_t k = 0; k < count; ++k) {
                    // The wave's segment bounds are uniform: scalar registers, so its branches are scalar.
                    const uint64_t bk = read_lane_any(b, static_cast<int>(k));
                    const uint64_t ek = read_lane_any(e, static_cast<int>(k));
                    if (bk >= ek) {
                        if (lane_id() == 0) write_result<T, OP>(out, index_out, first + k, bk, true, R::identity());
                    } else if (ek - bk <= kSgWaveMax) {
                        const Acc total = wave_combine<T, OP>(ek - bk >= kSgWaveVector
                                                                  ? fold_range<T, OP>(in, bk, ek, lane_id(), kWave)
                                                                  : fold_range<T, OP, false>(in, bk, ek, lane_id(), kWave));
                        if (lane_id() == 0) write_result<T, OP>(out, index_out, first + k, bk, false, total);
                    } else if (lane_id() == 0) {
                        s_big[atomicAdd(&s_nbig, 1u)] = first + k;
                    }
                }
            }
        }
        __syncthreads();
        const uint32_t nbig = s_nbig;
        for (uint32_t k = 0; k < nbig; ++k) {
            const uint64_t big = s_big[k];
            uint64_t b, e;
            bounds(big, b, e);
            block_reduce(big, b, e);
            __syncthreads();
        }
    }
}

template <typename T>
struct alignas(16) ScanRun {
    T v[kScanItems];
};

// Inclusive scan of one 32-/64-bit value per lane with wrapping or float addition.
template <typename T>
__device__ __forceinline__ T wave_scan_sum(T x) {
    x = add_wrap(x, dpp_move<dpp::kRowShr1>(T(0), x));
    x = add_wrap(x, dpp_move<dpp::kRowShr2>(T(0), x));
    x = add_wrap(x, dpp_move<dpp::kRowShr4>(T(0), x));
    x = add_wrap(x, dpp_move<dpp::kRowShr8>(T(0), x));
    x = add_wrap(x, dpp_move<dpp::kRowBcast15, 0xa>(T(0), x));
    x = add_wrap(x, dpp_move<dpp::kRowBcast31, 0xc>(T(0), x));
    return x;
}

// Scan of the non-empty segment [b, e) into out + ob by the whole workgroup (collective).
template <typename T>
__device__ __forceinline__ void block_scan_segment(const T* __restrict__ in, T* __restrict__ out, uint64_t b,
                                                   uint64_t e, uint64_t ob, int inclusive, int use_init, T init,
                                                   T* s_wave) {
    constexpr uint64_t kChunk = static_cast<uint64_t>(kSgBlock) * kScanItems;
    const uint32_t wave = threadIdx.x / kWave;
    // Every thread's run of items starts at a multiple of kScanItems from the segment's begin, so
    // 16-byte vector accesses apply when the segment starts on a 16-byte boundary.
    const bool vec_in = (reinterpret_cast<uintptr_t>(in + b) & 15) == 0;
    const bool vec_out = (reinterpret_cast<uintptr_t>(out + ob) & 15) == 0;
    T carry = use_init ? init : T(0);
    // This thread's run of the chunk at c; the next chunk's run is loaded before the current one is
    // scanned and stored, so its loads are in flight across the barriers.
    auto load_run = [&](uint64_t c, T (&v)[kScanItems]) {
        const uint64_t first = c + static_cast<uint64_t>(threadIdx.x) * kScanItems;
        if (vec_in && first + kScanItems <= e) {
            const ScanRun<T> r = *reinterpret_cast<const ScanRun<T>*>(in + first);
#pragma unroll
            for (int k = 0; k < kScanItems; ++k) v[k] = r.v[k];
        } else {
#pragma unroll
            for (int k = 0; k < kScanItems; ++k) v[k] = first + k < e ? in[first + k] : T(0);
        }
    };
    T nv[kScanItems];
    load_run(b, nv);
    for (uint64_t c = b; c < e; c += kChunk) {
        const uint64_t first = c + static_cast<uint64_t>(threadIdx.x) * kScanItems;
        T v[kScanItems];
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) v[k] = nv[k];
        if (c + kChunk < e) load_run(c + kChunk, nv);
        T own = v[0];
#pragma unroll
        for (int k = 1; k < kScanItems; ++k) own = add_wrap(own, v[k]);
        const T inc = wave_scan_sum(own);
        __syncthreads();  // earlier readers of s_wave are done
        if (lane_id() == kWave - 1) s_wave[wave] = inc;
        __syncthreads();
        T before = T(0), total = T(0);
#pragma unroll
        for (int w = 0; w < kSgWaves; ++w) {
            if (static_cast<uint32_t>(w) == wave) before = total;
            total = add_wrap(total, s_wave[w]);
        }
        // Prefix of this thread's first item: carry + earlier waves + earlier lanes of this wave.
        const T lanes_before = dpp_move<dpp::kWaveShr1>(T(0), inc);
        T run = add_wrap(carry, add_wrap(before, lanes_before));
        T o[kScanItems];
#pragma unroll
        for (int k = 0; k < kScanItems; ++k) {
            const T next = add_wrap(run, v[k]);
            o[k] = inclusive ? next : run;
            run = next;
        }
        // Plain stores: a lane's run is 32 or 64 bytes, so one 16-byte store instruction of the wave covers
        // every other vector of its lines, and non-temporal stores of that pattern measured much slower
        // (2^28 i32 InclusiveSegmentedSum in 4,096-item segments 0.375 -> 0.443 ms; non-temporal loads of
        // the runs 0.382 ms).
        T* const dst = out + ob + (first - b);
        if (vec_out && first + kScanItems <= e) {
            ScanRun<T> r;
#pragma unroll
            for (int k = 0; k < kScanItems; ++k) r.v[k] = o[k];
            *reinterpret_cast<ScanRun<T>*>(dst) = r;
        } else {
#pragma unroll
            for (int k = 0; k < kScanItems; ++k) {
                if (first + k < e) dst[k] = o[k];
            }
        }
        carry = add_wrap(carry, total);
    }
}

// Scan of the non-empty segment [b, e) into out + ob by one wave: 64 items per step, a DPP wave scan and
// a running carry.
template <typename T>
__device__ __forceinline__ void wave_scan_segment(const T* __restrict__ in, T* __restrict__ out, uint64_t b,
                                                  uint64_t e, uint64_t ob, int inclusive, int use_init, T init) {
    const uint32_t lane = lane_id();
    T carry = use_init ? init : T(0);
    for (uint64_t c = b; c < e; c += kWave) {
        const uint64_t i = c + lane;
        const T v = i < e ? in[i] : T(0);
        const T inc = wave_scan_sum(v);
        const T run = add_wrap(carry, dpp_move<dpp::kWaveShr1>(T(0), inc));
        if (i < e) out[ob + (i - b)] = inclusive ? add_wrap(run, v) : run;
        carry = add_wrap(carry, read_lane_any(inc, kWave - 1));
    }
}

// Up to 65,536 segments: one workgroup per segment.  Above that, each wave takes batches of `batch`
// consecutive segments like the reduce: a batch whose segments all hold at most kSgLaneMax items is
// scanned one segment per lane; any other batch one segment at a time, a wave scanning a segment of at
// most 1,024 items alone and the workgroup longer ones together (one workgroup per segment is bound by
// dispatch).
template <typename T>
__global__ __launch_bounds__(kSgBlock) void segmented_scan_kernel(const T* __restrict__ in, T* __restrict__ out,
                                                                  const uint32_t* __restrict__ begins,
                                                                  const uint32_t* __restrict__ ends,
                                                                  const uint32_t* __restrict__ out_begins,
                                                                  int inclusive, int use_init, T init,
                                                                  uint64_t num_segments, uint32_t batch) {
    __shared__ T s_wave[kSgWaves];
    __shared__ uint64_t s_big[kSgBlock];
    __shared__ uint32_t s_nbig;
    const uint64_t groups = gridDim.x;
    if (num_segments <= groups) {
        const uint32_t seg = blockIdx.x;
        const uint64_t b = begins[seg], e = ends[seg];
        if (b < e) block_scan_segment(in, out, b, e, static_cast<uint64_t>(out_begins[seg]), inclusive, use_init, init,
                                      s_wave);
        return;
    }
    const uint32_t wave = threadIdx.x / kWave;
    for (uint64_t r = 0;; ++r) {
        const uint64_t batch0 = (blockIdx.x + r * groups) * kSgWaves;
        if (batch0 * batch >= num_segments) break;
        if (threadIdx.x == 0) s_nbig = 0;
        __syncthreads();
        const uint64_t first = (batch0 + wave) * batch;
        if (first < num_segments) {
            const uint32_t count = num_segments - first < batch ? static_cast<uint32_t>(num_segments - first) : batch;
            const uint64_t seg = first + lane_id();
            uint64_t b = 0, e = 0, ob = 0;
            if (lane_id() < count) {
                b = begins[seg];
                e = ends[seg];
                ob = out_begins[seg];
            }
            const uint64_t len = e > b ? e - b : 0;
            if (wave_ballot(len > kSgLaneMax) == 0) {
                // One segment per lane, 8 loads in flight per step.
                T run = use_init ? init : T(0);
                for (uint64_t i = b; i < e; i += 8) {
                    T v[8];
#pragma unroll
                    for (int k = 0; k < 8; ++k) v[k] = i + k < e ? in[i + k] : T(0);
#pragma unroll
                    for (int k = 0; k < 8; ++k) {
                        if (i + k < e) {
                            const T next = add_wrap(run, v[k]);
                            out[ob + (i + k - b)] = inclusive ? next : run;
                            run = next;
                        }
                    }
                }
            } else {
                for (uint32_t k = 0; k < count; ++k) {
                    const uint64_t bk = read_lane_any(b, static_cast<int>(k));
                    const uint64_t ek = read_lane_any(e, static_cast<int>(k));
                    if (bk < ek) {
                        if (ek - bk <= kSgWaveMax)
                            wave_scan_segment(in, out, bk, ek, read_lane_any(ob, static_cast<int>(k)), inclusive,
                                              use_init, init);
                        else if (lane_id() == 0)
                            s_big[atomicAdd(&s_nbig, 1u)] = first + k;
                    }
                }
            }
        }
        __syncthreads();
        const uint32_t nbig = s_nbig;
        for (uint32_t k = 0; k < nbig; ++k) {
            const uint64_t big = s_big[k];
            block_scan_segment(in, out, begins[big], ends[big], static_cast<uint64_t>(out_begins[big]), inclusive,
                               use_init, init, s_wave);
            __syncthreads();
        }
    }
}

unsigned checked_grid(uint64_t segments) { return static_cast<unsigned>(segments); }

template <typename T, int OP>
int segment_reduce(const T* in, T* out, uint32_t* index_out, uint64_t num_segments, const uint32_t* begins,
                   const uint32_t* ends, uint64_t fixed_size, void* stream_ptr, const char* what) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (num_segments == 0) return kOk;
    if (num_segments > 0x7FFFFFFFull) return set_error(kInvalidArgument, "%s: too many segments", what);
    if (!out || ((OP == kOpArgMin || OP == kOpArgMax) && !index_out))
        return set_error(kInvalidArgument, "%s: null output", what);
    if (!begins && fixed_size == 0) {
        // Every fixed-size-0 segment is empty: the kernel writes the initial values without reading.
    } else if (!in) {
        return set_error(kInvalidArgument, "%s: null input", what);
    }
    if (!begins && num_segments * fixed_size > 0xFFFFFFFFull + 1)
        return set_error(kInvalidArgument, "%s: segments exceed 2^32 items", what);
    if (begins == nullptr && ends != nullptr) return set_error(kInvalidArgument, "%s: bad offsets", what);
    LaunchScope scope("segment_reduce", stream);
    // Up to kSgMaxGroups segments one workgroup each; beyond, batches of about num_segments / kSgBatchWaves
    // segments (1 to 64) per wave and enough workgroups for one round of them, at most kSgMaxGroups.
    uint64_t batch = num_segments / kSgBatchWaves;
    batch = batch < 1 ? 1 : (batch > static_cast<uint64_t>(kWave) ? kWave : batch);
    const uint64_t wave_batches = ceil_div(num_segments, batch);
    const uint64_t wg_batches = ceil_div(wave_batches, static_cast<uint64_t>(kSgWaves));
    const uint64_t groups = num_segments <= kSgMaxGroups ? num_segments
                                                         : (wg_batches < kSgMaxGroups ? wg_batches : kSgMaxGroups);
    segment_reduce_kernel<T, OP><<<checked_grid(groups), kSgBlock, 0, stream>>>(
        in, out, index_out, begins, ends, fixed_size, num_segments, static_cast<uint32_t>(batch));
    return check_hip(hipGetLastError(), "segment_reduce launch");
}

template <typename T>
int segmented_scan(const T* in, T* out, const uint32_t* begins, const uint32_t* ends, const uint32_t* out_begins,
                   uint64_t num_segments, int inclusive, int use_init, T init, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const char* what = "DeviceSegmentedScan";
    if (num_segments == 0) return kOk;
    if (num_segments > 0x7FFFFFFFull) return set_error(kInvalidArgument, "%s: too many segments", what);
    if (!in || !out || !begins || !ends) return set_error(kInvalidArgument, "%s: null input or output", what);
    LaunchScope scope("segmented_scan", stream);
    // Batches as for the reduce (segment_reduce above).
    uint64_t batch = num_segments / kSgBatchWaves;
    batch = batch < 1 ? 1 : (batch > static_cast<uint64_t>(kWave) ? kWave : batch);
    const uint64_t wg_batches = ceil_div(ceil_div(num_segments, batch), static_cast<uint64_t>(kSgWaves));
    const uint64_t groups = num_segments <= kSgMaxGroups ? num_segments
                                                         : (wg_batches < kSgMaxGroups ? wg_batches : kSgMaxGroups);
    segmented_scan_kernel<T><<<checked_grid(groups), kSgBlock, 0, stream>>>(
        in, out, begins, ends, out_begins ? out_begins : begins, inclusive, use_init, init, num_segments,
        static_cast<uint32_t>(batch));
    return check_hip(hipGetLastError(), "segmented_scan launch");
}

}  // namespace
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

#define LCPP_HIP_DEFINE_SEGMENT_REDUCE(OPS, OP, TS, TT)                                                               \
    int lcpp_hip_segment_reduce_##OPS##_##TS(void*, size_t, const TT* in, TT* out, uint64_t num_segments,             \
                                             const uint32_t* begin_offsets, const uint32_t* end_offsets,             \
                                             void* stream) {                                                         \
        if (num_segments && (!begin_offsets || !end_offsets))                                                        \
            return set_error(kInvalidArgument, "DeviceSegmentReduce: null offsets");                                 \
        return segment_reduce<TT, OP>(in, out, nullptr, num_segments, begin_offsets, end_offsets, 0, stream,          \
                                      "DeviceSegmentReduce");                                                         \
    }                                                                                                                 \
    int lcpp_hip_segment_reduce_fixed_##OPS##_##TS(void*, size_t, const TT* in, TT* out, uint64_t num_segments,       \
                                                   uint32_t segment_size, void* stream) {                            \
        return segment_reduce<TT, OP>(in, out, nullptr, num_segments, nullptr, nullptr, segment_size, stream,         \
                                      "DeviceSegmentReduce");                                                         \
    }
#define LCPP_HIP_DEFINE_SEGMENT_ARG(OPS, OP, TS, TT)                                                                  \
    int lcpp_hip_segment_##OPS##_##TS(void*, size_t, const TT* in, TT* out, uint32_t* index_out,                     \
                                      uint64_t num_segments, const uint32_t* begin_offsets,                          \
                                      const uint32_t* end_offsets, void* stream) {                                   \
        if (num_segments && (!begin_offsets || !end_offsets))                                                        \
            return set_error(kInvalidArgument, "DeviceSegmentReduce: null offsets");                                 \
        return segment_reduce<TT, OP>(in, out, index_out, num_segments, begin_offsets, end_offsets, 0, stream,        \
                                      "DeviceSegmentReduce::Arg");                                                    \
    }                                                                                                                 \
    int lcpp_hip_segment_fixed_##OPS##_##TS(void*, size_t, const TT* in, TT* out, uint32_t* index_out,               \
                                            uint64_t num_segments, uint32_t segment_size, void* stream) {            \
        return segment_reduce<TT, OP>(in, out, index_out, num_segments, nullptr, nullptr, segment_size, stream,       \
                                      "DeviceSegmentReduce::Arg");                                                    \
    }
#define LCPP_HIP_DEFINE_SEGMENTED(TS, TT)                                                                             \
    LCPP_HIP_DEFINE_SEGMENT_REDUCE(sum, kOpSum, TS, TT)                                                               \
    LCPP_HIP_DEFINE_SEGMENT_REDUCE(min, kOpMin, TS, TT)                                                               \
    LCPP_HIP_DEFINE_SEGMENT_REDUCE(max, kOpMax, TS, TT)                                                               \
    int lcpp_hip_segmented_scan_sum_##TS(void*, size_t, const TT* in, TT* out, const uint32_t* begin_offsets,         \
                                         const uint32_t* end_offsets, const uint32_t* out_begin_offsets,             \
                                         uint64_t num_segments, int inclusive, int use_init, TT init,                 \
                                         void* stream) {                                                             \
        return segmented_scan<TT>(in, out, begin_offsets, end_offsets, out_begin_offsets, num_segments, inclusive,    \
                                  use_init, init, stream);                                                            \
    }
LCPP_HIP_DEFINE_SEGMENTED(i32, int32_t)
LCPP_HIP_DEFINE_SEGMENTED(u32, uint32_t)
LCPP_HIP_DEFINE_SEGMENTED(f32, float)
LCPP_HIP_DEFINE_SEGMENTED(i64, int64_t)
LCPP_HIP_DEFINE_SEGMENTED(u64, uint64_t)
LCPP_HIP_DEFINE_SEGMENTED(f64, double)
LCPP_HIP_DEFINE_SEGMENT_ARG(argmin, kOpArgMin, i32, int32_t)
LCPP_HIP_DEFINE_SEGMENT_ARG(argmin, kOpArgMin, u32, uint32_t)
LCPP_HIP_DEFINE_SEGMENT_ARG(argmin, kOpArgMin, f32, float)
LCPP_HIP_DEFINE_SEGMENT_ARG(argmax, kOpArgMax, i32, int32_t)
LCPP_HIP_DEFINE_SEGMENT_ARG(argmax, kOpArgMax, u32, uint32_t)
LCPP_HIP_DEFINE_SEGMENT_ARG(argmax, kOpArgMax, f32, float)
#undef LCPP_HIP_DEFINE_SEGMENTED
#undef LCPP_HIP_DEFINE_SEGMENT_ARG
#undef LCPP_HIP_DEFINE_SEGMENT_REDUCE

}  // extern "C"
