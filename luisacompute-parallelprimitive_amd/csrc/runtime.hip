// Runtime plumbing of the C-ABI: error strings, HIP error mapping, the fill kernel, per-kernel
// event timing and device queries.  The reference's equivalent is `lcpp_check`
// (runtime/core.h:56-67), which asserts in debug builds; here every entry point returns a status
// code and keeps a thread-local message.
#include "common.hpp"
#include "../../include/lcpp_hip.h"

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace lcpp_hip {

namespace {
thread_local char g_last_error[512] = "";

struct ProfileRecord {
    std::string name;
    hipEvent_t begin;
    hipEvent_t end;
};

struct ProfileState {
    std::mutex mu;
    bool enabled = false;
    std::vector<ProfileRecord> pending;
    std::map<std::string, std::pair<double, uint64_t>> totals;  // name -> (ms, launches)
    std::vector<hipEvent_t> pool;

    hipEvent_t take_event() {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        return e;
    }
};

ProfileState& profile() {
    static ProfileState s;
    return s;
}
}  // namespace

int set_error(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

int check_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return kOk;
    return set_error(kHipError, "%s: %s", what, hipGetErrorString(e));
}

__global__ void fill_u32_kernel(uint32_t* dst, uint64_t count, uint32_t value) {
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (; i < count; i += stride) dst[i] = value;
}

int launch_fill_u32(uint32_t* dst, uint64_t count, uint32_t value, hipStream_t stream) {
    if (count == 0) return kOk;
    const uint64_t blocks = ceil_div(count, 256);
    const unsigned grid = static_cast<unsigned>(blocks < 4096 ? blocks : 4096);
    LaunchScope scope("fill_u32", stream);
    fill_u32_kernel<<<grid, 256, 0, stream>>>(dst, count, value);
    return check_hip(hipGetLastError(), "fill_u32 launch");
}

// Device-to-device copy.  16-byte-aligned ranges: a grid-stride loop of 256-thread workgroups, 32 per CU,
// each thread moving four 16-byte vectors per step with non-temporal loads and stores (1 GiB on MI355X:
// 0.3505 ms = 6.13 TB/s, against 0.372 ms for one 64 KiB tile of 8-byte words per workgroup, 0.355 ms at
// 16 workgroups per CU and 0.384-0.402 ms with plain stores).  8-byte-aligned ranges: one workgroup per
// 64 KiB tile of 8-byte words.  Other ranges copy bytewise.
using CopyVec = uint32_t __attribute__((ext_vector_type(4)));
constexpr int kCopyVecBlock = 256;
constexpr int kCopyVecUnroll = 4;
constexpr int kCopyWorkgroupsPerCu = 32;

__global__ __launch_bounds__(kCopyVecBlock) void copy_vec_kernel(CopyVec* __restrict__ dst,
                                                                 const CopyVec* __restrict__ src, uint64_t vecs) {
    constexpr uint64_t kChunk = static_cast<uint64_t>(kCopyVecBlock) * kCopyVecUnroll;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kChunk;
    uint64_t base = static_cast<uint64_t>(blockIdx.x) * kChunk + threadIdx.x;
    for (; base + (kCopyVecUnroll - 1) * kCopyVecBlock < vecs; base += stride) {
        CopyVec v[kCopyVecUnroll];
#pragma unroll
        for (int k = 0; k < kCopyVecUnroll; ++k) v[k] = __builtin_nontemporal_load(&src[base + k * kCopyVecBlock]);
#pragma unroll
        for (int k = 0; k < kCopyVecUnroll; ++k) __builtin_nontemporal_store(v[k], &dst[base + k * kCopyVecBlock]);
    }
    // This workgroup's last, partial chunk (the next one starts past the end: stride > kChunk).
#pragma unroll
    for (int k = 0; k < kCopyVecUnroll; ++k)
        if (base + k * kCopyVecBlock < vecs) dst[base + k * kCopyVecBlock] = src[base + k * kCopyVecBlock];
}

constexpr int kCopyBlock = 1024;
constexpr int kCopyWords = 8;  // 8-byte words per thread
constexpr uint64_t kCopyTileBytes = static_cast<uint64_t>(kCopyBlock) * kCopyWords * 8;

__global__ __launch_bounds__(kCopyBlock) void copy_words_kernel(uint64_t* __restrict__ dst, const uint64_t* __restrict__ src,
                                                                 uint64_t words) {
    const uint64_t base = static_cast<uint64_t>(blockIdx.x) * kCopyBlock * kCopyWords + threadIdx.x;
    if (base + (kCopyWords - 1) * kCopyBlock < words) {
        uint64_t v[kCopyWords];
#pragma unroll
        for (int k = 0; k < kCopyWords; ++k) v[k] = __builtin_nontemporal_load(&src[base + k * kCopyBlock]);
#pragma unroll
        for (int k = 0; k < kCopyWords; ++k) dst[base + k * kCopyBlock] = v[k];
    } else {
        for (int k = 0; k < kCopyWords; ++k)
            if (base + k * kCopyBlock < words) dst[base + k * kCopyBlock] = src[base + k * kCopyBlock];
    }
}

__global__ void copy_bytes_kernel(unsigned char* __restrict__ dst, const unsigned char* __restrict__ src, uint64_t bytes) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride) dst[i] = src[i];
}

int launch_copy(void* dst, const void* src, uint64_t bytes, hipStream_t stream) {
    if (bytes == 0 || dst == src) return kOk;
    LaunchScope scope("device_copy", stream);
    if (reinterpret_cast<uintptr_t>(dst) % 16 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 && bytes % 16 == 0) {
        const uint64_t vecs = bytes / 16;
        uint64_t grid = ceil_div(vecs, static_cast<uint64_t>(kCopyVecBlock) * kCopyVecUnroll);
        const uint64_t cap = static_cast<uint64_t>(device_cu_count()) * kCopyWorkgroupsPerCu;
        if (grid > cap) grid = cap;
        copy_vec_kernel<<<static_cast<unsigned>(grid), kCopyVecBlock, 0, stream>>>(
            static_cast<CopyVec*>(dst), static_cast<const CopyVec*>(src), vecs);
        return check_hip(hipGetLastError(), "device copy launch");
    }
    if (reinterpret_cast<uintptr_t>(dst) % 8 == 0 && reinterpret_cast<uintptr_t>(src) % 8 == 0 && bytes % 8 == 0) {
        const uint64_t tiles = ceil_div(bytes, kCopyTileBytes);
        if (tiles > 0x7FFFFFFFull) return set_error(kInvalidArgument, "device copy: too many bytes");
        copy_words_kernel<<<static_cast<unsigned>(tiles), kCopyBlock, 0, stream>>>(
            static_cast<uint64_t*>(dst), static_cast<const uint64_t*>(src), bytes / 8);
    } else {
        const uint64_t blocks = ceil_div(bytes, 256);
        copy_bytes_kernel<<<static_cast<unsigned>(blocks < 8192 ? blocks : 8192), 256, 0, stream>>>(
            static_cast<unsigned char*>(dst), static_cast<const unsigned char*>(src), bytes);
    }
    return check_hip(hipGetLastError(), "device copy launch");
}

LaunchScope::LaunchScope(const char* n, hipStream_t s) : name(n), stream(s), begin_event(nullptr) {
    ProfileState& p = profile();
    std::lock_guard<std::mutex> lock(p.mu);
    if (!p.enabled) return;
    hipEvent_t e = p.take_event();
    if (e && hipEventRecord(e, s) == hipSuccess) begin_event = e;
}

LaunchScope::~LaunchScope() {
    if (!begin_event) return;
    ProfileState& p = profile();
    std::lock_guard<std::mutex> lock(p.mu);
    hipEvent_t e = p.take_event();
    if (e && hipEventRecord(e, stream) == hipSuccess) {
        p.pending.push_back({name, static_cast<hipEvent_t>(begin_event), e});
    }
}

std::atomic<uint32_t> g_lookback_spin_limit{64};

int device_cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}

}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

const char* lcpp_hip_last_error(void) { return g_last_error; }

const char* lcpp_hip_version(void) { return "lcpp-hip 0.1.0 (gfx950)"; }

int lcpp_hip_set_lookback_spin_limit(uint32_t polls) {
    g_lookback_spin_limit.store(polls, std::memory_order_relaxed);
    return kOk;
}

uint32_t lcpp_hip_get_lookback_spin_limit(void) { return lookback_spin_limit(); }

int lcpp_hip_device_copy(void* dst, const void* src, uint64_t bytes, void* stream) {
    if (bytes == 0) return kOk;
    if (!dst || !src) return set_error(kInvalidArgument, "device copy: null buffer");
    return launch_copy(dst, src, bytes, static_cast<hipStream_t>(stream));
}

#ifdef LCPP_HIP_PHASE_TRACE
// Diagnostic build only: per-tile phase records of the onesweep and scan kernels go to `buffer`
// (device memory, `records` records of kTraceWords 64-bit words; null to stop).
int lcpp_hip_trace_set_buffer(void* buffer, uint64_t records) {
    int st = radix_trace_set_buffer(buffer, records);
    if (st != kOk) return st;
    return scan_trace_set_buffer(buffer, records);
}
#endif

int lcpp_hip_profile_enable(int enable) {
    ProfileState& p = profile();
    std::lock_guard<std::mutex> lock(p.mu);
    p.enabled = enable != 0;
    return kOk;
}

int lcpp_hip_profile_reset(void) {
    ProfileState& p = profile();
    std::lock_guard<std::mutex> lock(p.mu);
    for (auto& r : p.pending) {
        p.pool.push_back(r.begin);
        p.pool.push_back(r.end);
    }
    p.pending.clear();
    p.totals.clear();
    return kOk;
}

// Waits for every recorded launch and folds its duration into the per-kernel totals.
static int profile_collect_locked(ProfileState& p) {
    for (auto& r : p.pending) {
        if (hipEventSynchronize(r.end) != hipSuccess) return set_error(kHipError, "profile: event sync failed");
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, r.begin, r.end) != hipSuccess) return set_error(kHipError, "profile: elapsed failed");
        auto& t = p.totals[r.name];
        t.first += ms;
        t.second += 1;
        p.pool.push_back(r.begin);
        p.pool.push_back(r.end);
    }
    p.pending.clear();
    return kOk;
}

int lcpp_hip_profile_query(const char* kernel, double* total_ms, uint64_t* launches) {
    if (!kernel || !total_ms || !launches) return set_error(kInvalidArgument, "profile_query: null argument");
    ProfileState& p = profile();
    std::lock_guard<std::mutex> lock(p.mu);
    int st = profile_collect_locked(p);
    if (st != kOk) return st;
    auto it = p.totals.find(kernel);
    *total_ms = it == p.totals.end() ? 0.0 : it->second.first;
    *launches = it == p.totals.end() ? 0 : it->second.second;
    return kOk;
}

int lcpp_hip_profile_names(char* buffer, size_t buffer_bytes) {
    ProfileState& p = profile();
    std::lock_guard<std::mutex> lock(p.mu);
    int st = profile_collect_locked(p);
    if (st != kOk) return st;
    std::string all;
    for (auto& kv : p.totals) {
        all += kv.first;
        all += '\n';
    }
    if (!buffer || buffer_bytes < all.size() + 1) return set_error(kInvalidArgument, "profile_names: buffer too small");
    std::memcpy(buffer, all.c_str(), all.size() + 1);
    return kOk;
}

}  // extern "C"
