// Seeded synthetic inputs generated on the device (counter-based splitmix64, so any element can be
// produced independently and the host can reproduce the same stream).
#include "common.hpp"
#include "../../include/lcpp_hip.h"

namespace lcpp_hip {
namespace {

__device__ __forceinline__ uint64_t splitmix64_at(uint64_t seed, uint64_t index) {
    uint64_t z = seed + (index + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void generate_kernel(int kind, void* out, uint64_t n, uint64_t seed, uint64_t start) {
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (; i < n; i += stride) {
        const uint64_t g = start + i;
        switch (kind) {
            case LCPP_HIP_GEN_U64: static_cast<uint64_t*>(out)[i] = splitmix64_at(seed, g); break;
            case LCPP_HIP_GEN_U32_HI: static_cast<uint32_t*>(out)[i] = static_cast<uint32_t>(splitmix64_at(seed, g) >> 32); break;
            case LCPP_HIP_GEN_I32_PM1000:
                static_cast<int32_t*>(out)[i] = static_cast<int32_t>(splitmix64_at(seed, g) % 2001ull) - 1000;
                break;
            case LCPP_HIP_GEN_U32_LT16: static_cast<uint32_t*>(out)[i] = static_cast<uint32_t>(splitmix64_at(seed, g) & 15ull); break;
            case LCPP_HIP_GEN_U64_AND3:
                static_cast<uint64_t*>(out)[i] =
                    splitmix64_at(seed, 3 * g) & splitmix64_at(seed, 3 * g + 1) & splitmix64_at(seed, 3 * g + 2);
                break;
            case LCPP_HIP_GEN_U32_IOTA: static_cast<uint32_t*>(out)[i] = static_cast<uint32_t>(g); break;
            case LCPP_HIP_GEN_F32_PM1:
                static_cast<float*>(out)[i] =
                    static_cast<float>(static_cast<uint32_t>(splitmix64_at(seed, g) >> 40)) * (1.0f / 8388608.0f) - 1.0f;
                break;
            default: break;
        }
    }
}

}  // namespace
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" int lcpp_hip_generate(int kind, void* out, uint64_t n, uint64_t seed, uint64_t start, void* stream_ptr) {
    if (kind < LCPP_HIP_GEN_U64 || kind > LCPP_HIP_GEN_F32_PM1) return set_error(kInvalidArgument, "generate: bad kind %d", kind);
    if (n == 0) return kOk;
    if (!out) return set_error(kInvalidArgument, "generate: null output");
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const uint64_t blocks = ceil_div(n, 256);
    const unsigned grid = static_cast<unsigned>(blocks < 8192 ? blocks : 8192);
    LaunchScope scope("generate", stream);
    generate_kernel<<<grid, 256, 0, stream>>>(kind, out, n, seed, start);
    return check_hip(hipGetLastError(), "generate launch");
}
