// Achievable read+write bandwidth on this device: copies of 1 GiB -> 1 GiB with hipMemcpy and with
// hand-written kernels of two shapes - a persistent grid-stride loop (2..16 workgroups per CU, 4 or 8
// 16-byte vectors per thread in flight, plain or non-temporal) and one tile per workgroup of
// ROWS x BLOCK 16-byte vectors (the shape of the scan kernel).  Mean of 20 calls after a warm-up;
// one JSON line per variant.  It bounds what a streaming read+write kernel (scan) can reach.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#define CK(x) do { hipError_t e = (x); if (e != hipSuccess) { printf("HIP error %s line %d\n", hipGetErrorString(e), __LINE__); return 1; } } while (0)
using V4 = uint32_t __attribute__((ext_vector_type(4)));
template <int UNROLL, bool NT>
__global__ __launch_bounds__(256) void grid_stride(const V4* __restrict__ a, V4* __restrict__ b, size_t nvec) {
    const size_t stride = (size_t)gridDim.x * 256 * UNROLL;
    for (size_t base = (size_t)blockIdx.x * 256 * UNROLL + threadIdx.x; base < nvec; base += stride) {
        V4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) { size_t i = base + u * 256; if (i < nvec) v[u] = NT ? __builtin_nontemporal_load(&a[i]) : a[i]; }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) { size_t i = base + u * 256; if (i < nvec) { if (NT) __builtin_nontemporal_store(v[u], &b[i]); else b[i] = v[u]; } }
    }
}
// one tile of ROWS x BLOCK vectors per workgroup (scan-like)
template <int BLOCK, int ROWS, bool NTL, bool NTS>
__global__ __launch_bounds__(BLOCK) void tiled(const V4* __restrict__ a, V4* __restrict__ b) {
    const size_t base = (size_t)blockIdx.x * BLOCK * ROWS;
    V4 v[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) v[r] = NTL ? __builtin_nontemporal_load(&a[base + r * BLOCK + threadIdx.x]) : a[base + r * BLOCK + threadIdx.x];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) { if (NTS) __builtin_nontemporal_store(v[r], &b[base + r * BLOCK + threadIdx.x]); else b[base + r * BLOCK + threadIdx.x] = v[r]; }
}
template <typename F>
float timeit(F f) {
    hipEvent_t s, e; hipEventCreate(&s); hipEventCreate(&e);
    f(); hipDeviceSynchronize();
    hipEventRecord(s);
    for (int i = 0; i < 20; ++i) f();
    hipEventRecord(e); hipEventSynchronize(e);
    float ms; hipEventElapsedTime(&ms, s, e); return ms / 20;
}
int main() {
    const size_t bytes = size_t(1) << 30, nvec = bytes / 16;
    V4 *a, *b; CK(hipMalloc(&a, bytes)); CK(hipMalloc(&b, bytes)); CK(hipMemset(a, 1, bytes)); CK(hipMemset(b, 0, bytes));
    int cus = 0; hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
    auto rep = [&](const char* name, float ms) { printf("{\"kernel\": \"%s\", \"ms\": %.4f, \"GBps\": %.1f}\n", name, ms, 2.0 * bytes / ms / 1e6); };
    rep("hipMemcpyDtoD", timeit([&] { hipMemcpyAsync(b, a, bytes, hipMemcpyDeviceToDevice, 0); }));
    for (int mult : {2, 4, 8, 16}) {
        char nm[64];
        snprintf(nm, 64, "grid_stride_u4_x%d", mult); rep(nm, timeit([&] { grid_stride<4, false><<<cus * mult, 256>>>(a, b, nvec); }));
        snprintf(nm, 64, "grid_stride_u4_nt_x%d", mult); rep(nm, timeit([&] { grid_stride<4, true><<<cus * mult, 256>>>(a, b, nvec); }));
        snprintf(nm, 64, "grid_stride_u8_x%d", mult); rep(nm, timeit([&] { grid_stride<8, false><<<cus * mult, 256>>>(a, b, nvec); }));
    }
    rep("tiled_256x24_plain", timeit([&] { tiled<256, 24, false, false><<<nvec / (256 * 24) , 256>>>(a, b); }));
    rep("tiled_256x24_ntload", timeit([&] { tiled<256, 24, true, false><<<nvec / (256 * 24), 256>>>(a, b); }));
    rep("tiled_256x24_nt_both", timeit([&] { tiled<256, 24, true, true><<<nvec / (256 * 24), 256>>>(a, b); }));
    rep("tiled_256x16_plain", timeit([&] { tiled<256, 16, false, false><<<nvec / (256 * 16), 256>>>(a, b); }));
    rep("tiled_256x16_ntload", timeit([&] { tiled<256, 16, true, false><<<nvec / (256 * 16), 256>>>(a, b); }));
    rep("tiled_512x8_ntload", timeit([&] { tiled<512, 8, true, false><<<nvec / (512 * 8), 512>>>(a, b); }));
    rep("tiled_256x4_ntload", timeit([&] { tiled<256, 4, true, false><<<nvec / (256 * 4), 256>>>(a, b); }));
    return 0;
}
