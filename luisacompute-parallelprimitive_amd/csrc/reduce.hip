// DeviceReduce::Sum for gfx950.
//
// Reference path: DeviceReduce<>::Sum -> Reduce -> reduce_array_recursive
// (src/lcpp/device/device_reduce.h:280-288,229-252,728-958) with AgentReduce tiles of 256x8 striped
// loads (agent/agent_reduce.h:58-173) and a 32-lane warp tree (warp/details/warp_reduce_shlf.h:37-76).
//
// MI355X design: one persistent pass over HBM.  A grid of (CUs x 8) workgroups of 256 threads
// streams the input with 128-bit loads, UNROLL loads in flight per thread, folds them in registers,
// reduces each wave with DPP row shifts / row broadcasts, and writes one partial per workgroup into
// the caller's temp storage.  A single 1024-thread workgroup folds the partials and writes *out.
// Inputs of at most one persistent round fall back to one workgroup that writes *out directly.
// Algorithmic traffic: n * sizeof(T) bytes read (+ grid * sizeof(T) partials).
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

}  // extern "C"
