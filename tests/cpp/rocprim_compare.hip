// Comparator: ROCm's own rocPRIM (header-only, built here from /opt/rocm/include) timed on the inputs
// of the benchmark: radix_sort_keys of 2^28 uniform uint32, radix_sort_pairs of 2^27 uniform uint64 keys
// with uint32 index values, exclusive_scan and reduce of 2^28 uint32.  Same splitmix64 streams as the
// library's generator; hipEvent timing over repeated calls after warm-up.  Prints one JSON line per op.
#include <hip/hip_runtime.h>
#include <cstring>
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>
#include <rocprim/device/device_reduce.hpp>
#include <cstdio>
#include <cstdint>
#include <vector>
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s line %d\n", hipGetErrorString(e), __LINE__); return 1; } } while (0)
__global__ void gen_u32(uint32_t* o, size_t n, uint64_t seed) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < n) { uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull; z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull; z = (z ^ (z >> 27)) * 0x94D049BB133111EBull; o[i] = (uint32_t)((z ^ (z >> 31)) >> 32); }
}
__global__ void gen_u64(uint64_t* o, uint32_t* v, size_t n, uint64_t seed) {
    size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (i < n) { uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull; z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull; z = (z ^ (z >> 27)) * 0x94D049BB133111EBull; o[i] = z ^ (z >> 31); v[i] = (uint32_t)i; }
}
int main() {
    const size_t n = size_t(1) << 28;
    uint32_t *k, *ko; CK(hipMalloc(&k, n * 4)); CK(hipMalloc(&ko, n * 4));
    gen_u32<<<(n + 255) / 256, 256>>>(k, n, 114521);
    size_t tb = 0; CK(rocprim::radix_sort_keys(nullptr, tb, k, ko, n));
    void* temp; CK(hipMalloc(&temp, tb));
    hipEvent_t a, b; CK(hipEventCreate(&a)); CK(hipEventCreate(&b));
    for (int i = 0; i < 3; ++i) CK(rocprim::radix_sort_keys(temp, tb, k, ko, n));
    CK(hipDeviceSynchronize());
    const int reps = 10;
    CK(hipEventRecord(a));
    for (int i = 0; i < reps; ++i) CK(rocprim::radix_sort_keys(temp, tb, k, ko, n));
    CK(hipEventRecord(b)); CK(hipEventSynchronize(b));
    float ms = 0; CK(hipEventElapsedTime(&ms, a, b)); ms /= reps;
    std::vector<uint32_t> h(n); CK(hipMemcpy(h.data(), ko, n * 4, hipMemcpyDeviceToHost));
    bool sorted = true; for (size_t i = 1; i < n; ++i) if (h[i - 1] > h[i]) { sorted = false; break; }
    printf("{\"lib\": \"rocprim\", \"op\": \"radix_sort_keys u32 2^28\", \"ms\": %.4f, \"gkeys_per_s\": %.2f, \"temp_bytes\": %zu, \"sorted\": %d}\n", ms, n / (ms * 1e-3) / 1e9, tb, (int)sorted);
    CK(hipFree(temp)); CK(hipFree(k)); CK(hipFree(ko));
    // pairs: 2^27 u64 keys + u32 values
    const size_t m = size_t(1) << 27;
    uint64_t *pk, *pko; uint32_t *pv, *pvo;
    CK(hipMalloc(&pk, m * 8)); CK(hipMalloc(&pko, m * 8)); CK(hipMalloc(&pv, m * 4)); CK(hipMalloc(&pvo, m * 4));
    gen_u64<<<(m + 255) / 256, 256>>>(pk, pv, m, 114521);
    tb = 0; CK(rocprim::radix_sort_pairs(nullptr, tb, pk, pko, pv, pvo, m));
    CK(hipMalloc(&temp, tb));
    for (int i = 0; i < 2; ++i) CK(rocprim::radix_sort_pairs(temp, tb, pk, pko, pv, pvo, m));
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(a));
    for (int i = 0; i < 5; ++i) CK(rocprim::radix_sort_pairs(temp, tb, pk, pko, pv, pvo, m));
    CK(hipEventRecord(b)); CK(hipEventSynchronize(b));
    CK(hipEventElapsedTime(&ms, a, b)); ms /= 5;
    printf("{\"lib\": \"rocprim\", \"op\": \"radix_sort_pairs u64+u32 2^27 uniform\", \"ms\": %.4f, \"gpairs_per_s\": %.2f}\n", ms, m / (ms * 1e-3) / 1e9);
    // scan and reduce 2^28
    uint32_t *s, *so; CK(hipMalloc(&s, n * 4)); CK(hipMalloc(&so, n * 4));
    gen_u32<<<(n + 255) / 256, 256>>>(s, n, 7);
    tb = 0; CK(rocprim::exclusive_scan(nullptr, tb, s, so, 0u, n, rocprim::plus<uint32_t>()));
    void* t2; CK(hipMalloc(&t2, tb));
    for (int i = 0; i < 3; ++i) CK(rocprim::exclusive_scan(t2, tb, s, so, 0u, n, rocprim::plus<uint32_t>()));
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(a));
    for (int i = 0; i < 10; ++i) CK(rocprim::exclusive_scan(t2, tb, s, so, 0u, n, rocprim::plus<uint32_t>()));
    CK(hipEventRecord(b)); CK(hipEventSynchronize(b));
    CK(hipEventElapsedTime(&ms, a, b)); ms /= 10;
    printf("{\"lib\": \"rocprim\", \"op\": \"exclusive_scan u32 2^28\", \"ms\": %.4f, \"GBps\": %.1f}\n", ms, 8.0 * n / (ms * 1e-3) / 1e9);
    tb = 0; CK(rocprim::reduce(nullptr, tb, s, so, 0u, n, rocprim::plus<uint32_t>()));
    void* t3; CK(hipMalloc(&t3, tb));
    for (int i = 0; i < 3; ++i) CK(rocprim::reduce(t3, tb, s, so, 0u, n, rocprim::plus<uint32_t>()));
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(a));
    for (int i = 0; i < 10; ++i) CK(rocprim::reduce(t3, tb, s, so, 0u, n, rocprim::plus<uint32_t>()));
    CK(hipEventRecord(b)); CK(hipEventSynchronize(b));
    CK(hipEventElapsedTime(&ms, a, b)); ms /= 10;
    printf("{\"lib\": \"rocprim\", \"op\": \"reduce u32 2^28\", \"ms\": %.4f, \"GBps\": %.1f}\n", ms, 4.0 * n / (ms * 1e-3) / 1e9);
    return 0;
}
