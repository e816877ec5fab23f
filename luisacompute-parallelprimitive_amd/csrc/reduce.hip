// DeviceReduce::Sum, Min, Max, ArgMin and ArgMax for gfx950.
//
// Reference path: DeviceReduce<>::Sum / Min / Max -> Reduce -> reduce_array_recursive
// (src/lcpp/device/device_reduce.h:280-288,229-252,728-958) with AgentReduce tiles of 256x8 striped
// loads (agent/agent_reduce.h:58-173) and a 32-lane warp tree (warp/details/warp_reduce_shlf.h:37-76).
//
// MI355X design: one persistent pass over HBM.  A grid of (CUs x 8) workgroups of 256 threads (2^28 i32
// Sum: 0.156 ms per call with 8 or 16 per CU, 0.158 with 32, 0.159 with 64, 0.172 with one workgroup per
// 4,096 items) streams the input with 128-bit loads, UNROLL loads in flight per thread, folds them in registers,
// reduces each wave with DPP row shifts / row broadcasts, and writes one partial per workgroup into
// the caller's temp storage.  A single 1024-thread workgroup folds the partials and writes *out.
// Inputs of at most one persistent round fall back to one workgroup that writes *out directly.
// Min and max run the same pass with the NaN-ignoring operators (reference MinOp / MaxOp, folded from
// the type's max / lowest as the reference's initial value, device_reduce.h:291-309).  ArgMin / ArgMax
// (device_reduce.h:311-436) fold (value, index) pairs: the smaller (larger) value wins, equal values the
// lower index, NaNs never win; the reference builds an n-sized pair array first, here each thread
// carries the index of its best item, so the pass reads the items once.
// Reduce(op, init) and TransformReduce(op, transform, init) (device_reduce.h:229-252,491-515) run the
// same pass with the operator and the transform as template parameters: the transform is applied once
// to every item (never to partials), and the final kernel folds the initial value in on the left,
// op(init, aggregate), as the reference's single-tile kernel does (device/details/reduce.h:227-237).
// Algorithmic traffic: n * sizeof(T) bytes read (+ grid partials).
#include "common.hpp"
#include "../../include/lcpp_hip.h"

namespace lcpp_hip {
namespace {

constexpr int kReduceBlock = 256;
constexpr int kReduceUnroll = 4;
constexpr int kFinalBlock = 1024;

template <typename T>
using Vec16 = T __attribute__((ext_vector_type(16 / sizeof(T))));

template <typename T>
__device__ __forceinline__ T block_sum(T x, T* s_waves) {
    constexpr int W = kReduceBlock / kWave;
    x = wave_reduce(x, SumOp{});
    const int wave = threadIdx.x / kWave;
    if (lane_id() == 0) s_waves[wave] = x;
    __syncthreads();
    T total = s_waves[0];
#pragma unroll
    for (int w = 1; w < W; ++w) total += s_waves[w];
    return total;
}

// Folds in[0..n) into partials[blockIdx.x].  `head` leading elements precede the first 16-byte
// aligned address; `nvec` aligned vectors follow; the remaining tail elements end the range.
template <typename T>
__global__ __launch_bounds__(kReduceBlock) void reduce_sum_partials_kernel(const T* __restrict__ in, uint64_t n,
                                                                           uint32_t head, uint64_t nvec,
                                                                           T* __restrict__ partials) {
    constexpr int V = 16 / sizeof(T);
    using Vec = Vec16<T>;
    __shared__ T s_waves[kReduceBlock / kWave];
    const Vec* __restrict__ vin = reinterpret_cast<const Vec*>(in + head);
    const uint32_t tid = threadIdx.x;

    T acc[kReduceUnroll];
#pragma unroll
    for (int u = 0; u < kReduceUnroll; ++u) acc[u] = T(0);

    const uint64_t chunk = static_cast<uint64_t>(kReduceBlock) * kReduceUnroll;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * chunk;
    uint64_t base = static_cast<uint64_t>(blockIdx.x) * chunk;
    for (; base + chunk <= nvec; base += stride) {
        Vec v[kReduceUnroll];
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) v[u] = __builtin_nontemporal_load(&vin[base + u * kReduceBlock + tid]);
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) {
            T s = v[u][0];
#pragma unroll
            for (int j = 1; j < V; ++j) s += v[u][j];
            acc[u] += s;
        }
    }
    if (base < nvec) {  // last, partial chunk of this workgroup
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) {
            const uint64_t idx = base + u * kReduceBlock + tid;
            if (idx < nvec) {
                Vec v = vin[idx];
                T s = v[0];
#pragma unroll
                for (int j = 1; j < V; ++j) s += v[j];
                acc[u] += s;
            }
        }
    }
    if (blockIdx.x == 0) {
        if (tid < head) acc[0] += in[tid];
        const uint64_t t = head + nvec * V + tid;
        if (t < n) acc[1] += in[t];
    }
    T x = acc[0];
#pragma unroll
    for (int u = 1; u < kReduceUnroll; ++u) x += acc[u];
    x = block_sum(x, s_waves);
    if (tid == 0) partials[blockIdx.x] = x;
}

template <typename T>
__global__ __launch_bounds__(kFinalBlock) void reduce_sum_final_kernel(const T* __restrict__ partials, uint32_t count,
                                                                       T* __restrict__ out) {
    __shared__ T s_waves[kFinalBlock / kWave];
    T x = T(0);
    for (uint32_t i = threadIdx.x; i < count; i += kFinalBlock) x += partials[i];
    x = wave_reduce(x, SumOp{});
    if (lane_id() == 0) s_waves[threadIdx.x / kWave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        T total = s_waves[0];
        for (int w = 1; w < kFinalBlock / kWave; ++w) total += s_waves[w];
        *out = total;
    }
}

template <typename T>
__global__ void write_scalar_kernel(T* out, T value) {
    *out = value;
}
// ---- transforms and operators of Reduce / TransformReduce ---------------------------------------
// The reference takes any device callable; with no JIT here, a fixed vocabulary covers its tests:
// identity, scale * x + shift (x + c, 2x, 2x + 1 ...), x * x and |x|.  Integer arithmetic wraps (it runs
// in the unsigned type of the same width); float arithmetic rounds after every operation, with no
// fused multiply-add, so a host loop evaluating the same expression gets the same transformed items.
enum : int { kXformIdentity = 0, kXformAffine = 1, kXformSquare = 2, kXformAbs = 3 };

template <typename T, int XF>
__device__ __forceinline__ T apply_transform(T x, T scale, T shift) {
#pragma clang fp contract(off)
    if constexpr (XF == kXformIdentity) {
        return x;
    } else if constexpr (std::is_floating_point_v<T>) {
        if constexpr (XF == kXformAffine) {
            const T p = x * scale;
            return p + shift;
        } else if constexpr (XF == kXformSquare) {
            return x * x;
        } else {
            return std::fabs(x);
        }
    } else {
        using UT = std::make_unsigned_t<T>;
        const UT u = static_cast<UT>(x);
        if constexpr (XF == kXformAffine) return static_cast<T>(static_cast<UT>(u * static_cast<UT>(scale) + static_cast<UT>(shift)));
        else if constexpr (XF == kXformSquare) return static_cast<T>(static_cast<UT>(u * u));
        else if constexpr (std::is_signed_v<T>) return x < 0 ? static_cast<T>(static_cast<UT>(UT(0) - u)) : x;
        else return x;
    }
}

// The sum operator in the item's own type, wrapping for signed integers too.
struct WrapSumOp {
    template <typename T>
    __device__ __forceinline__ T operator()(T a, T b) const {
        if constexpr (std::is_integral_v<T>) {
            using UT = std::make_unsigned_t<T>;
            return static_cast<T>(static_cast<UT>(static_cast<UT>(a) + static_cast<UT>(b)));
        } else {
            return a + b;
        }
    }
    template <typename T>
    __host__ __device__ __forceinline__ static constexpr T identity() { return T(0); }
};

// ---- min / max ---------------------------------------------------------------------------------
template <typename T, typename Op>
__device__ __forceinline__ T block_fold(T x, T* s_waves, Op op) {
    constexpr int W = kReduceBlock / kWave;
    x = wave_reduce(x, op);
    const int wave = threadIdx.x / kWave;
    if (lane_id() == 0) s_waves[wave] = x;
    __syncthreads();
    T total = s_waves[0];
#pragma unroll
    for (int w = 1; w < W; ++w) total = op(total, s_waves[w]);
    return total;
}

// reduce_sum_partials_kernel with another operator (min / max, or the sum in the item's own type) and a
// transform of every item; partials[blockIdx.x] = the workgroup's fold.
template <typename T, typename Op, int XF = kXformIdentity>
__global__ __launch_bounds__(kReduceBlock) void reduce_ext_partials_kernel(const T* __restrict__ in, uint64_t n,
                                                                           uint32_t head, uint64_t nvec,
                                                                           T* __restrict__ partials, T scale,
                                                                           T shift) {
    constexpr int V = 16 / sizeof(T);
    using Vec = Vec16<T>;
    const Op op{};
    __shared__ T s_waves[kReduceBlock / kWave];
    const Vec* __restrict__ vin = reinterpret_cast<const Vec*>(in + head);
    const uint32_t tid = threadIdx.x;
    T acc[kReduceUnroll];
#pragma unroll
    for (int u = 0; u < kReduceUnroll; ++u) acc[u] = Op::template identity<T>();
    const uint64_t chunk = static_cast<uint64_t>(kReduceBlock) * kReduceUnroll;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * chunk;
    uint64_t base = static_cast<uint64_t>(blockIdx.x) * chunk;
    for (; base + chunk <= nvec; base += stride) {
        Vec v[kReduceUnroll];
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) v[u] = __builtin_nontemporal_load(&vin[base + u * kReduceBlock + tid]);
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) {
#pragma unroll
            for (int j = 0; j < V; ++j) acc[u] = op(acc[u], apply_transform<T, XF>(v[u][j], scale, shift));
        }
    }
    if (base < nvec) {
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) {
            const uint64_t idx = base + u * kReduceBlock + tid;
            if (idx < nvec) {
                const Vec v = vin[idx];
#pragma unroll
                for (int j = 0; j < V; ++j) acc[u] = op(acc[u], apply_transform<T, XF>(v[j], scale, shift));
            }
        }
    }
    if (blockIdx.x == 0) {
        if (tid < head) acc[0] = op(acc[0], apply_transform<T, XF>(in[tid], scale, shift));
        const uint64_t t = head + nvec * V + tid;
        if (t < n) acc[1] = op(acc[1], apply_transform<T, XF>(in[t], scale, shift));
    }
    T x = acc[0];
#pragma unroll
    for (int u = 1; u < kReduceUnroll; ++u) x = op(x, acc[u]);
    x = block_fold(x, s_waves, op);
    if (tid == 0) partials[blockIdx.x] = x;
}

// Folds `count` partials, then folds the result into the initial value: op(init, aggregate) (the type's
// max for Min, lowest for Max, the caller's value for Reduce / TransformReduce).
template <typename T, typename Op>
__global__ __launch_bounds__(kFinalBlock) void reduce_ext_final_kernel(const T* __restrict__ partials, uint32_t count,
                                                                       T init, T* __restrict__ out) {
    const Op op{};
    __shared__ T s_waves[kFinalBlock / kWave];
    T x = Op::template identity<T>();
    for (uint32_t i = threadIdx.x; i < count; i += kFinalBlock) x = op(x, partials[i]);
    x = wave_reduce(x, op);
    if (lane_id() == 0) s_waves[threadIdx.x / kWave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        T total = init;
        for (int w = 0; w < kFinalBlock / kWave; ++w) total = op(total, s_waves[w]);
        *out = total;
    }
}

// ---- arg min / arg max ---------------------------------------------------------------------------
// A (value, index) pair; `index` UINT32_MAX with a NaN (float) or the type's max / lowest (integer)
// value is the identity.
template <typename T>
struct ArgPair {
    T value;
    uint32_t index;
};

// b beats a: a strictly better value, or an equal one at a lower index; a NaN never beats anything and
// anything that is not a NaN beats a NaN.
template <bool MAX, typename T>
__device__ __forceinline__ bool arg_beats(T bv, uint32_t bi, T av, uint32_t ai) {
    if constexpr (std::is_floating_point_v<T>) {
        if (bv != bv) return false;
        if (av != av) return true;
    }
    return (MAX ? bv > av : bv < av) || (bv == av && bi < ai);
}

template <bool MAX, typename T>
__device__ __forceinline__ ArgPair<T> arg_identity() {
    if constexpr (MAX) return ArgPair<T>{MaxValueOp::identity<T>(), 0xFFFFFFFFu};
    else return ArgPair<T>{MinValueOp::identity<T>(), 0xFFFFFFFFu};
}

template <bool MAX, typename T>
__device__ __forceinline__ void arg_fold(ArgPair<T>& a, T v, uint32_t i) {
    if (arg_beats<MAX>(v, i, a.value, a.index)) a = ArgPair<T>{v, i};
}

// Wave reduction of pairs: the DPP pattern of wave_inclusive_scan on both fields, lane 63's result.
template <bool MAX, typename T>
__device__ __forceinline__ ArgPair<T> arg_wave_reduce(ArgPair<T> p) {
    const ArgPair<T> id = arg_identity<MAX, T>();
    auto step = [&](T v, uint32_t i) { arg_fold<MAX>(p, v, i); };
    step(dpp_move<dpp::kRowShr1>(id.value, p.value), dpp_move<dpp::kRowShr1>(id.index, p.index));
    step(dpp_move<dpp::kRowShr2>(id.value, p.value), dpp_move<dpp::kRowShr2>(id.index, p.index));
    step(dpp_move<dpp::kRowShr4>(id.value, p.value), dpp_move<dpp::kRowShr4>(id.index, p.index));
    step(dpp_move<dpp::kRowShr8>(id.value, p.value), dpp_move<dpp::kRowShr8>(id.index, p.index));
    step(dpp_move<dpp::kRowBcast15, 0xa>(id.value, p.value), dpp_move<dpp::kRowBcast15, 0xa>(id.index, p.index));
    step(dpp_move<dpp::kRowBcast31, 0xc>(id.value, p.value), dpp_move<dpp::kRowBcast31, 0xc>(id.index, p.index));
    return ArgPair<T>{wave_read_lane(p.value, kWave - 1), wave_read_lane(p.index, kWave - 1)};
}

template <bool MAX, typename T, int BLOCK>
__device__ __forceinline__ ArgPair<T> arg_block_reduce(ArgPair<T> p, T* s_v, uint32_t* s_i) {
    p = arg_wave_reduce<MAX>(p);
    const int wave = threadIdx.x / kWave;
    if (lane_id() == 0) {
        s_v[wave] = p.value;
        s_i[wave] = p.index;
    }
    __syncthreads();
    ArgPair<T> total = arg_identity<MAX, T>();
#pragma unroll
    for (int w = 0; w < BLOCK / kWave; ++w) arg_fold<MAX>(total, s_v[w], s_i[w]);
    return total;
}

// Each thread keeps its best (value, index); partial values and indices go to two arrays.
template <typename T, bool MAX>
__global__ __launch_bounds__(kReduceBlock) void reduce_arg_partials_kernel(const T* __restrict__ in, uint64_t n,
                                                                           uint32_t head, uint64_t nvec,
                                                                           T* __restrict__ part_v,
                                                                           uint32_t* __restrict__ part_i) {
    constexpr int V = 16 / sizeof(T);
    using Vec = Vec16<T>;
    __shared__ T s_v[kReduceBlock / kWave];
    __shared__ uint32_t s_i[kReduceBlock / kWave];
    const Vec* __restrict__ vin = reinterpret_cast<const Vec*>(in + head);
    const uint32_t tid = threadIdx.x;
    ArgPair<T> acc[kReduceUnroll];
#pragma unroll
    for (int u = 0; u < kReduceUnroll; ++u) acc[u] = arg_identity<MAX, T>();
    const uint64_t chunk = static_cast<uint64_t>(kReduceBlock) * kReduceUnroll;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * chunk;
    uint64_t base = static_cast<uint64_t>(blockIdx.x) * chunk;
    for (; base + chunk <= nvec; base += stride) {
        Vec v[kReduceUnroll];
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) v[u] = __builtin_nontemporal_load(&vin[base + u * kReduceBlock + tid]);
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) {
            const uint32_t first = static_cast<uint32_t>(head + (base + u * kReduceBlock + tid) * V);
#pragma unroll
            for (int j = 0; j < V; ++j) arg_fold<MAX>(acc[u], v[u][j], first + j);
        }
    }
    if (base < nvec) {
#pragma unroll
        for (int u = 0; u < kReduceUnroll; ++u) {
            const uint64_t idx = base + u * kReduceBlock + tid;
            if (idx < nvec) {
                const Vec v = vin[idx];
                const uint32_t first = static_cast<uint32_t>(head + idx * V);
#pragma unroll
                for (int j = 0; j < V; ++j) arg_fold<MAX>(acc[u], v[j], first + j);
            }
        }
    }
    if (blockIdx.x == 0) {
        if (tid < head) arg_fold<MAX>(acc[0], in[tid], tid);
        const uint64_t t = head + nvec * V + tid;
        if (t < n) arg_fold<MAX>(acc[1], in[t], static_cast<uint32_t>(t));
    }
    ArgPair<T> x = acc[0];
#pragma unroll
    for (int u = 1; u < kReduceUnroll; ++u) arg_fold<MAX>(x, acc[u].value, acc[u].index);
    x = arg_block_reduce<MAX, T, kReduceBlock>(x, s_v, s_i);
    if (tid == 0) {
        part_v[blockIdx.x] = x.value;
        part_i[blockIdx.x] = x.index;
    }
}

// Folds the partials, then the reference's initial pair (index UINT32_MAX with the type's max for
// ArgMin, lowest for ArgMax), and writes value and index.
template <typename T, bool MAX>
__global__ __launch_bounds__(kFinalBlock) void reduce_arg_final_kernel(const T* __restrict__ part_v,
                                                                       const uint32_t* __restrict__ part_i,
                                                                       uint32_t count, T init, T* __restrict__ out,
                                                                       uint32_t* __restrict__ out_index) {
    __shared__ T s_v[kFinalBlock / kWave];
    __shared__ uint32_t s_i[kFinalBlock / kWave];
    ArgPair<T> x = arg_identity<MAX, T>();
    for (uint32_t i = threadIdx.x; i < count; i += kFinalBlock) arg_fold<MAX>(x, part_v[i], part_i[i]);
    x = arg_block_reduce<MAX, T, kFinalBlock>(x, s_v, s_i);
    if (threadIdx.x == 0) {
        ArgPair<T> total{init, 0xFFFFFFFFu};
        arg_fold<MAX>(total, x.value, x.index);
        *out = total.value;
        *out_index = total.index;
    }
}

template <typename T>
__global__ void write_pair_kernel(T* out, T value, uint32_t* out_index, uint32_t index) {
    *out = value;
    *out_index = index;
}


template <typename T>
int reduce_sum(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "DeviceReduce: too many items (%llu > UINT_MAX)",
                                            static_cast<unsigned long long>(n));
    if (!out) return set_error(kInvalidArgument, "DeviceReduce: null output");
    if (n == 0) {
        LaunchScope scope("reduce_write_init", stream);
        write_scalar_kernel<T><<<1, 1, 0, stream>>>(out, T(0));
        return check_hip(hipGetLastError(), "reduce_write_init launch");
    }
    if (!in) return set_error(kInvalidArgument, "DeviceReduce: null input");
    if (reinterpret_cast<uintptr_t>(in) % sizeof(T) != 0)
        return set_error(kInvalidArgument, "DeviceReduce: input not aligned to its element size");

    constexpr int V = 16 / sizeof(T);
    const uintptr_t addr = reinterpret_cast<uintptr_t>(in);
    uint64_t head = ((16 - (addr & 15)) & 15) / sizeof(T);
    if (head > n) head = n;
    const uint64_t nvec = (n - head) / V;

    const uint64_t chunk = static_cast<uint64_t>(kReduceBlock) * kReduceUnroll;
    uint64_t grid = ceil_div(nvec, chunk);
    const uint64_t max_grid = static_cast<uint64_t>(device_cu_count()) * 8;
    if (grid > max_grid) grid = max_grid;
    if (grid < 1) grid = 1;
    const uint64_t temp_slots = temp ? temp_bytes / sizeof(T) : 0;
    if (grid > 1 && temp_slots < 2) grid = 1;
    if (grid > temp_slots && grid > 1) grid = temp_slots;

    if (grid == 1) {
        LaunchScope scope("reduce_sum_partials", stream);
        reduce_sum_partials_kernel<T><<<1, kReduceBlock, 0, stream>>>(in, n, static_cast<uint32_t>(head), nvec, out);
        return check_hip(hipGetLastError(), "reduce_sum_partials launch");
    }
    T* partials = static_cast<T*>(temp);
    {
        LaunchScope scope("reduce_sum_partials", stream);
        reduce_sum_partials_kernel<T><<<static_cast<unsigned>(grid), kReduceBlock, 0, stream>>>(
            in, n, static_cast<uint32_t>(head), nvec, partials);
        int st = check_hip(hipGetLastError(), "reduce_sum_partials launch");
        if (st != kOk) return st;
    }
    LaunchScope scope("reduce_sum_final", stream);
    reduce_sum_final_kernel<T><<<1, kFinalBlock, 0, stream>>>(partials, static_cast<uint32_t>(grid), out);
    return check_hip(hipGetLastError(), "reduce_sum_final launch");
}

// Grid of the persistent pass over n items at `in` (shared by every operator): the number of
// unaligned leading items, the 16-byte vectors after them, and the workgroups (at most 8 per CU, at
// most the partial slots the temp storage holds, one when it holds fewer than two).
struct ReducePlan {
    uint64_t head, nvec, grid;
};
template <typename T>
ReducePlan reduce_plan(const T* in, uint64_t n, uint64_t partial_slots) {
    constexpr int V = 16 / sizeof(T);
    const uintptr_t addr = reinterpret_cast<uintptr_t>(in);
    uint64_t head = ((16 - (addr & 15)) & 15) / sizeof(T);
    if (head > n) head = n;
    const uint64_t nvec = (n - head) / V;
    const uint64_t chunk = static_cast<uint64_t>(kReduceBlock) * kReduceUnroll;
    uint64_t grid = ceil_div(nvec, chunk);
    const uint64_t max_grid = static_cast<uint64_t>(device_cu_count()) * 8;
    if (grid > max_grid) grid = max_grid;
    if (grid < 1) grid = 1;
    if (grid > 1 && partial_slots < 2) grid = 1;
    if (grid > partial_slots && grid > 1) grid = partial_slots;
    return ReducePlan{head, nvec, grid};
}

// op(init, fold of the transformed items) over the persistent pass and a final kernel; n == 0 writes
// init.  DeviceReduce::Min / Max are the identity transform with the type's max / lowest as init.
template <typename T, typename Op, int XF>
int reduce_generic(const char* what, const char* scope_name, void* temp, size_t temp_bytes, const T* in, T* out,
                   uint64_t n, T scale, T shift, T init, hipStream_t stream) {
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items (%llu > UINT_MAX)", what,
                                            static_cast<unsigned long long>(n));
    if (!out) return set_error(kInvalidArgument, "%s: null output", what);
    if (n == 0) {
        LaunchScope scope("reduce_write_init", stream);
        write_scalar_kernel<T><<<1, 1, 0, stream>>>(out, init);
        return check_hip(hipGetLastError(), "reduce_write_init launch");
    }
    if (!in) return set_error(kInvalidArgument, "%s: null input", what);
    if (reinterpret_cast<uintptr_t>(in) % sizeof(T) != 0)
        return set_error(kInvalidArgument, "%s: input not aligned to its element size", what);
    const ReducePlan pl = reduce_plan(in, n, temp ? temp_bytes / sizeof(T) : 0);
    T* partials = static_cast<T*>(temp);
    LaunchScope scope(scope_name, stream);
    if (pl.grid == 1) {
        // One workgroup folds everything into the first temp slot (into *out when there is no temp);
        // the final kernel then folds that value into the initial value.
        T* slot = temp && temp_bytes >= sizeof(T) ? partials : out;
        reduce_ext_partials_kernel<T, Op, XF><<<1, kReduceBlock, 0, stream>>>(in, n, static_cast<uint32_t>(pl.head),
                                                                              pl.nvec, slot, scale, shift);
        int st = check_hip(hipGetLastError(), "reduce launch");
        if (st != kOk) return st;
        reduce_ext_final_kernel<T, Op><<<1, kFinalBlock, 0, stream>>>(slot, 1u, init, out);
        return check_hip(hipGetLastError(), "reduce final launch");
    }
    reduce_ext_partials_kernel<T, Op, XF><<<static_cast<unsigned>(pl.grid), kReduceBlock, 0, stream>>>(
        in, n, static_cast<uint32_t>(pl.head), pl.nvec, partials, scale, shift);
    int st = check_hip(hipGetLastError(), "reduce launch");
    if (st != kOk) return st;
    reduce_ext_final_kernel<T, Op><<<1, kFinalBlock, 0, stream>>>(partials, static_cast<uint32_t>(pl.grid), init, out);
    return check_hip(hipGetLastError(), "reduce final launch");
}

// DeviceReduce::Min (MAX false) / Max (true): the fold of the items and the type's max / lowest.
template <typename T, bool MAX>
int reduce_ext(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, void* stream_ptr) {
    using Op = std::conditional_t<MAX, MaxValueOp, MinValueOp>;
    const T init = MAX ? std::numeric_limits<T>::lowest() : std::numeric_limits<T>::max();
    return reduce_generic<T, Op, kXformIdentity>(MAX ? "DeviceReduce::Max" : "DeviceReduce::Min", "reduce_extremum",
                                                 temp, temp_bytes, in, out, n, T(0), T(0), init,
                                                 static_cast<hipStream_t>(stream_ptr));
}

// DeviceReduce::Reduce(op, init) (transform identity) and TransformReduce(op, transform, init): op 0 sum
// (wrapping for integers), 1 min, 2 max (the NaN-ignoring MinOp / MaxOp); transform as kXform*.
template <typename T, typename Op>
int transform_reduce_op(const char* what, int transform, void* temp, size_t temp_bytes, const T* in, T* out,
                        uint64_t n, T scale, T shift, T init, hipStream_t stream) {
    switch (transform) {
        case kXformIdentity:
            return reduce_generic<T, Op, kXformIdentity>(what, "reduce_op", temp, temp_bytes, in, out, n, scale, shift,
                                                         init, stream);
        case kXformAffine:
            return reduce_generic<T, Op, kXformAffine>(what, "reduce_op", temp, temp_bytes, in, out, n, scale, shift,
                                                       init, stream);
        case kXformSquare:
            return reduce_generic<T, Op, kXformSquare>(what, "reduce_op", temp, temp_bytes, in, out, n, scale, shift,
                                                       init, stream);
        case kXformAbs:
            return reduce_generic<T, Op, kXformAbs>(what, "reduce_op", temp, temp_bytes, in, out, n, scale, shift, init,
                                                    stream);
        default:
            return set_error(kInvalidArgument, "%s: unknown transform %d", what, transform);
    }
}

template <typename T>
int transform_reduce(const char* what, void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int op,
                     int transform, T scale, T shift, T init, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    switch (op) {
        case 0:
            return transform_reduce_op<T, WrapSumOp>(what, transform, temp, temp_bytes, in, out, n, scale, shift, init,
                                                     stream);
        case 1:
            return transform_reduce_op<T, MinValueOp>(what, transform, temp, temp_bytes, in, out, n, scale, shift, init,
                                                      stream);
        case 2:
            return transform_reduce_op<T, MaxValueOp>(what, transform, temp, temp_bytes, in, out, n, scale, shift, init,
                                                      stream);
        default:
            return set_error(kInvalidArgument, "%s: unknown reduce operator %d", what, op);
    }
}

// DeviceReduce::ArgMin (MAX false) / ArgMax (true).  n == 0 writes the type's max / lowest and index 1
// (device_reduce.h:320-325,383-388).  Temp holds the partial values, then (4-byte aligned) their indices.
template <typename T, bool MAX>
int reduce_arg(void* temp, size_t temp_bytes, const T* in, T* out, uint32_t* out_index, uint64_t n,
               void* stream_ptr) {
    const char* what = MAX ? "DeviceReduce::ArgMax" : "DeviceReduce::ArgMin";
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const T init = MAX ? std::numeric_limits<T>::lowest() : std::numeric_limits<T>::max();
    if (n > 0xFFFFFFFFull) return set_error(kInvalidArgument, "%s: too many items (%llu > UINT_MAX)", what,
                                            static_cast<unsigned long long>(n));
    if (!out || !out_index) return set_error(kInvalidArgument, "%s: null output", what);
    if (n == 0) {
        LaunchScope scope("reduce_write_init", stream);
        write_pair_kernel<T><<<1, 1, 0, stream>>>(out, init, out_index, 1u);
        return check_hip(hipGetLastError(), "reduce_write_init launch");
    }
    if (!in) return set_error(kInvalidArgument, "%s: null input", what);
    if (reinterpret_cast<uintptr_t>(in) % sizeof(T) != 0)
        return set_error(kInvalidArgument, "%s: input not aligned to its element size", what);
    if (!temp || reinterpret_cast<uintptr_t>(temp) % sizeof(T) != 0 || temp_bytes < sizeof(T) + 4)
        return set_error(kTempTooSmall, "%s: temp storage too small (%zu < %zu bytes)", what, temp_bytes,
                         sizeof(T) + 4);
    const ReducePlan pl = reduce_plan(in, n, temp_bytes / (sizeof(T) + 4));
    T* part_v = static_cast<T*>(temp);
    uint32_t* part_i = reinterpret_cast<uint32_t*>(part_v + pl.grid);
    LaunchScope scope("reduce_arg", stream);
    reduce_arg_partials_kernel<T, MAX><<<static_cast<unsigned>(pl.grid), kReduceBlock, 0, stream>>>(
        in, n, static_cast<uint32_t>(pl.head), pl.nvec, part_v, part_i);
    int st = check_hip(hipGetLastError(), "reduce_arg launch");
    if (st != kOk) return st;
    reduce_arg_final_kernel<T, MAX><<<1, kFinalBlock, 0, stream>>>(part_v, part_i, static_cast<uint32_t>(pl.grid), init,
                                                                  out, out_index);
    return check_hip(hipGetLastError(), "reduce_arg final launch");
}

}  // namespace
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

// Signed sums are computed in the unsigned type of the same width: two's-complement addition
// wraps identically and unsigned overflow is well defined.
#define LCPP_HIP_DEFINE_REDUCE(S, T, A)                                                                       \
    int lcpp_hip_reduce_sum_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, void* stream) { \
        return reduce_sum<A>(temp, temp_bytes, reinterpret_cast<const A*>(in), reinterpret_cast<A*>(out), n,  \
                             stream);                                                                        \
    }
LCPP_HIP_DEFINE_REDUCE(i32, int32_t, uint32_t)
LCPP_HIP_DEFINE_REDUCE(u32, uint32_t, uint32_t)
LCPP_HIP_DEFINE_REDUCE(f32, float, float)
LCPP_HIP_DEFINE_REDUCE(i64, int64_t, uint64_t)
LCPP_HIP_DEFINE_REDUCE(u64, uint64_t, uint64_t)
LCPP_HIP_DEFINE_REDUCE(f64, double, double)
#undef LCPP_HIP_DEFINE_REDUCE

// Min / max compare in the item's own type (signed as signed).
#define LCPP_HIP_DEFINE_REDUCE_EXT(S, T)                                                                        \
    int lcpp_hip_reduce_min_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, void* stream) {  \
        return reduce_ext<T, false>(temp, temp_bytes, in, out, n, stream);                                      \
    }                                                                                                           \
    int lcpp_hip_reduce_max_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, void* stream) {  \
        return reduce_ext<T, true>(temp, temp_bytes, in, out, n, stream);                                       \
    }                                                                                                           \
    int lcpp_hip_reduce_argmin_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint32_t* out_index,      \
                                   uint64_t n, void* stream) {                                                  \
        return reduce_arg<T, false>(temp, temp_bytes, in, out, out_index, n, stream);                           \
    }                                                                                                           \
    int lcpp_hip_reduce_argmax_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint32_t* out_index,      \
                                   uint64_t n, void* stream) {                                                  \
        return reduce_arg<T, true>(temp, temp_bytes, in, out, out_index, n, stream);                            \
    }
LCPP_HIP_DEFINE_REDUCE_EXT(i32, int32_t)
LCPP_HIP_DEFINE_REDUCE_EXT(u32, uint32_t)
LCPP_HIP_DEFINE_REDUCE_EXT(f32, float)
LCPP_HIP_DEFINE_REDUCE_EXT(i64, int64_t)
LCPP_HIP_DEFINE_REDUCE_EXT(u64, uint64_t)
LCPP_HIP_DEFINE_REDUCE_EXT(f64, double)
#undef LCPP_HIP_DEFINE_REDUCE_EXT

// Reduce(op, init) and TransformReduce(op, transform, init): signed integers keep their own type (min /
// max compare as signed; sums wrap through the unsigned type).
#define LCPP_HIP_DEFINE_REDUCE_OP(S, T)                                                                          \
    int lcpp_hip_reduce_op_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int op, T init,  \
                               void* stream) {                                                                   \
        return transform_reduce<T>("DeviceReduce::Reduce", temp, temp_bytes, in, out, n, op, kXformIdentity, T(0), \
                                   T(0), init, stream);                                                          \
    }                                                                                                            \
    int lcpp_hip_transform_reduce_##S(void* temp, size_t temp_bytes, const T* in, T* out, uint64_t n, int op,    \
                                      int transform, T scale, T shift, T init, void* stream) {                   \
        return transform_reduce<T>("DeviceReduce::TransformReduce", temp, temp_bytes, in, out, n, op, transform,  \
                                   scale, shift, init, stream);                                                  \
    }
LCPP_HIP_DEFINE_REDUCE_OP(i32, int32_t)
LCPP_HIP_DEFINE_REDUCE_OP(u32, uint32_t)
LCPP_HIP_DEFINE_REDUCE_OP(f32, float)
LCPP_HIP_DEFINE_REDUCE_OP(i64, int64_t)
LCPP_HIP_DEFINE_REDUCE_OP(u64, uint64_t)
LCPP_HIP_DEFINE_REDUCE_OP(f64, double)
#undef LCPP_HIP_DEFINE_REDUCE_OP

}  // extern "C"
