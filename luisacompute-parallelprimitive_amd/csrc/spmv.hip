// DeviceSpmv::CsrMV for gfx950: y = A * x with A in CSR.
//
// Reference: DeviceSpmv<>::CsrMV (src/lcpp/device/device_spmv.h:48-130): one 32-lane warp per row,
// lane-strided products, warp tree reduction, lane 0 writes y; rows with decreasing offsets or
// offsets past nnz produce 0; columns >= num_cols are skipped; nnz == 0 writes zeros (:133-155).
//
// MI355X design (no temp storage, like the reference): each wave owns 64 consecutive rows.
//   * Every lane reads its row's bounds (one coalesced load of 65 offsets per wave).
//   * Rows with at most kShortRow nonzeros are summed by their own lane, in order.
//   * Longer rows are taken one at a time by the whole wave: 64 lanes stride the row with coalesced
//     value/column loads, then a DPP wave reduction; the row's lane writes y.  Rows longer than
//     kVecRow read both streams in groups of kGroup consecutive elements per lane (16-byte-aligned
//     vector loads) when the arrays are 16-byte aligned, cutting the vector memory instructions per
//     nonzero, two groups per lane in flight.  The gathers of x bound the kernel: one L1 -> L2
//     request per nonzero (random columns never share an L1 line), so the texture addresser and the
//     L2 request rate, not HBM bytes, set its time; with x wholly L2-resident it would still need
//     one request per nonzero.
//   Power-law row lengths therefore cost each wave about (longest short row) + sum(long/64) steps,
//   instead of one 64-lane pass per row.
// Floating-point order: short rows are summed left to right; other rows as 64 per-lane partial sums
// (lane-strided elements, or for the grouped path the lane's groups of kGroup consecutive elements)
// combined by the DPP scan tree.  Integer values wrap modulo 2^32.
// Algorithmic traffic: nnz * (sizeof(V) + sizeof(I)) + (rows + 1) * sizeof(I) + rows * sizeof(V)
// + gathered x (at least cols * sizeof(V)).
#include "common.hpp"
#include "../../include/lcpp_hip.h"

namespace lcpp_hip {
namespace {

constexpr int kSpmvBlock = 256;
constexpr uint32_t kShortRow = 8;
constexpr int kLongUnroll = 4;  // wave-strided elements of a long row loaded together per lane
constexpr uint32_t kVecRow = 64;   // rows longer than this stream columns and values in element groups
constexpr uint32_t kGroup = 8;     // consecutive elements per lane and group (a multiple of 4)

// kGroup consecutive elements starting at a 16-byte-aligned address, as 16-byte vectors of the element
// type, widened to the accumulator type.  The main loop of long rows loads non-temporally: each matrix
// element is read once, and marking its lines for early eviction leaves the L2 to the gathered x
// (2^20 x 2^20 Zipf(1.5) matrix: L2 misses 12.46 M -> 11.52 M, 0.395 -> 0.373 ms per call); the same
// hint on the row tails and the shorter rows' element loads measured slower (0.397 / 0.422 ms).
template <bool NONTEMPORAL, typename T, typename R>
__device__ __forceinline__ void load_group(const T* p, R (&out)[kGroup]) {
    constexpr uint32_t E = 16 / sizeof(T);
    using Vec = T __attribute__((ext_vector_type(E)));
    const Vec* vp = reinterpret_cast<const Vec*>(p);
#pragma unroll
    for (uint32_t j = 0; j < kGroup / E; ++j) {
        const Vec q = NONTEMPORAL ? __builtin_nontemporal_load(vp + j) : vp[j];
#pragma unroll
        for (uint32_t e = 0; e < E; ++e) out[j * E + e] = static_cast<R>(q[e]);
    }
}

template <typename V> struct AccumType { using type = V; };
template <> struct AccumType<int32_t> { using type = uint32_t; };

template <typename V, typename I>
__global__ __launch_bounds__(kSpmvBlock) void spmv_csr_kernel(const V* __restrict__ values,
                                                              const I* __restrict__ row_offsets,
                                                              const I* __restrict__ column_indices,
                                                              const V* __restrict__ x, V* __restrict__ y,
                                                              uint32_t rows, uint32_t cols, uint32_t nnz,
                                                              bool vec_ok) {
    using A = typename AccumType<V>::type;
    const uint32_t lane = lane_id();
    const uint64_t wave_global = (static_cast<uint64_t>(blockIdx.x) * kSpmvBlock + threadIdx.x) / kWave;
    const uint64_t row64 = wave_global * kWave + lane;
    const bool in_range = row64 < rows;
    const uint32_t row = static_cast<uint32_t>(row64);

    uint32_t begin = 0, end = 0;
    if (in_range) {
        begin = static_cast<uint32_t>(row_offsets[row]);
        end = static_cast<uint32_t>(row_offsets[row + 1]);
    }
    const bool valid = in_range && begin <= end && end <= nnz;
    const uint32_t len = valid ? end - begin : 0;

    // Every load of a row (or of an unrolled group of a long row's elements) is issued before any
    // of them is used, so a lane waits for two memory round trips per group rather than two per
    // nonzero; products are still added in element order.
    A acc = A(0);
    const bool is_short = len <= kShortRow;
    if (is_short) {
        uint32_t c[kShortRow];
        A v[kShortRow];
#pragma unroll
        for (uint32_t k = 0; k < kShortRow; ++k) {
            if (k < len) {
                c[k] = static_cast<uint32_t>(column_indices[begin + k]);
                v[k] = static_cast<A>(values[begin + k]);
            }
        }
        A xv[kShortRow];
#pragma unroll
        for (uint32_t k = 0; k < kShortRow; ++k) xv[k] = (k < len && c[k] < cols) ? static_cast<A>(x[c[k]]) : A(0);
#pragma unroll
        for (uint32_t k = 0; k < kShortRow; ++k) {
            if (k < len && c[k] < cols) acc += v[k] * xv[k];
        }
    }

    uint64_t long_rows = wave_ballot(!is_short);
    while (long_rows) {
        const uint32_t src = static_cast<uint32_t>(__builtin_ctzll(long_rows));
        long_rows &= long_rows - 1;
        const uint32_t rb = __builtin_amdgcn_readlane(begin, src);
        const uint32_t re = __builtin_amdgcn_readlane(end, src);
        A part = A(0);
        if (vec_ok && re - rb > kVecRow) {
            // Lane l takes the kGroup-element groups starting at (rb & ~3) + kGroup l, then every
            // kGroup * kWave elements: 16-byte column and value loads instead of one load per element,
            // two groups in flight per iteration while both lie before nnz (the partial sum still adds
            // the groups in order).  Group elements outside [rb, re) belong to neighbouring rows and
            // are masked; a group reaching past the arrays' end is loaded element-wise.
            constexpr uint32_t kStride = kGroup * kWave;
            uint32_t g = (rb & ~3u) + kGroup * lane;
            // Two groups per lane in flight while both lie wholly before nnz.
            for (; g + kStride < re && g + kStride + (kGroup - 1) < nnz; g += 2 * kStride) {
                uint32_t c[2][kGroup];
                A v[2][kGroup];
                load_group<true>(column_indices + g, c[0]);
                load_group<true>(column_indices + g + kStride, c[1]);
                load_group<true>(values + g, v[0]);
                load_group<true>(values + g + kStride, v[1]);
                bool use[2][kGroup];
                A xv[2][kGroup];
#pragma unroll
                for (uint32_t h = 0; h < 2; ++h)
#pragma unroll
                for (uint32_t k = 0; k < kGroup; ++k) {
                    const uint32_t e = g + h * kStride + k;
                    use[h][k] = e >= rb && e < re && c[h][k] < cols;
                    xv[h][k] = use[h][k] ? static_cast<A>(x[c[h][k]]) : A(0);
                }
#pragma unroll
                for (uint32_t h = 0; h < 2; ++h)
#pragma unroll
                for (uint32_t k = 0; k < kGroup; ++k) {
                    if (use[h][k]) part += v[h][k] * xv[h][k];
                }
            }
            for (; g < re; g += kStride) {
                uint32_t c[kGroup];
                A v[kGroup];
                if (g + (kGroup - 1) < nnz) {
                    load_group<false>(column_indices + g, c);
                    load_group<false>(values + g, v);
                } else {
#pragma unroll
                    for (uint32_t k = 0; k < kGroup; ++k) {
                        c[k] = g + k < nnz ? static_cast<uint32_t>(column_indices[g + k]) : cols;
                        v[k] = g + k < nnz ? static_cast<A>(values[g + k]) : A(0);
                    }
                }
                bool use[kGroup];
                A xv[kGroup];
#pragma unroll
                for (uint32_t k = 0; k < kGroup; ++k) {
                    use[k] = g + k >= rb && g + k < re && c[k] < cols;
                    xv[k] = use[k] ? static_cast<A>(x[c[k]]) : A(0);
                }
#pragma unroll
                for (uint32_t k = 0; k < kGroup; ++k) {
                    if (use[k]) part += v[k] * xv[k];
                }
            }
            part = wave_reduce(part, SumOp{});
            if (lane == src) acc = part;
            continue;
        }
        uint32_t e = rb + lane;
        for (; e + (kLongUnroll - 1) * kWave < re; e += kLongUnroll * kWave) {
            uint32_t c[kLongUnroll];
            A v[kLongUnroll];
#pragma unroll
            for (int j = 0; j < kLongUnroll; ++j) {
                c[j] = static_cast<uint32_t>(column_indices[e + j * kWave]);
                v[j] = static_cast<A>(values[e + j * kWave]);
            }
            A xv[kLongUnroll];
#pragma unroll
            for (int j = 0; j < kLongUnroll; ++j) xv[j] = c[j] < cols ? static_cast<A>(x[c[j]]) : A(0);
#pragma unroll
            for (int j = 0; j < kLongUnroll; ++j) {
                if (c[j] < cols) part += v[j] * xv[j];
            }
        }
        for (; e < re; e += kWave) {
            const uint32_t c = static_cast<uint32_t>(column_indices[e]);
            if (c < cols) part += static_cast<A>(values[e]) * static_cast<A>(x[c]);
        }
        part = wave_reduce(part, SumOp{});
        if (lane == src) acc = part;
    }
    if (in_range) y[row] = static_cast<V>(acc);
}

template <typename V, typename I>
int spmv_csr(void* /*temp*/, size_t /*temp_bytes*/, const V* values, const I* row_offsets, const I* column_indices,
             const V* x, V* y, uint64_t rows, uint64_t cols, uint64_t nnz, void* stream_ptr) {
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    if (rows > 0xFFFFFFFFull / 32) return set_error(kInvalidArgument, "DeviceSpmv: too many rows");
    if (cols > 0xFFFFFFFFull) return set_error(kInvalidArgument, "DeviceSpmv: too many columns");
    // 32-bit element indices run up to 2 * max(kLongUnroll, kGroup) * kWave past a row's end (the
    // grouped loop tests the group after next) without wrapping.
    if (nnz > 0xFFFFFFFFull - 4 * (kLongUnroll > kGroup ? kLongUnroll : kGroup) * kWave)
        return set_error(kInvalidArgument, "DeviceSpmv: too many nonzero values");
    if (rows == 0) return kOk;
    if (!y) return set_error(kInvalidArgument, "DeviceSpmv: null output vector");
    if (nnz == 0) return launch_fill_u32(reinterpret_cast<uint32_t*>(y), rows * sizeof(V) / 4, 0u, stream);
    if (!values || !row_offsets || !column_indices || !x)
        return set_error(kInvalidArgument, "DeviceSpmv: null matrix or vector");
    if (cols == 0) return set_error(kInvalidArgument, "DeviceSpmv: a matrix with zero columns cannot hold nonzeros");
    const uint64_t waves = ceil_div(rows, kWave);
    const uint64_t blocks = ceil_div(waves * kWave, kSpmvBlock);
    // 16-byte group loads need both streams 16-byte aligned (element 4k then is, for 4- and 8-byte values).
    const bool vec_ok = reinterpret_cast<uintptr_t>(values) % 16 == 0 && reinterpret_cast<uintptr_t>(column_indices) % 16 == 0;
    LaunchScope scope("spmv_csr", stream);
    spmv_csr_kernel<V, I><<<static_cast<unsigned>(blocks), kSpmvBlock, 0, stream>>>(
        values, row_offsets, column_indices, x, y, static_cast<uint32_t>(rows), static_cast<uint32_t>(cols),
        static_cast<uint32_t>(nnz), vec_ok);
    return check_hip(hipGetLastError(), "spmv_csr launch");
}

}  // namespace
}  // namespace lcpp_hip

using namespace lcpp_hip;

extern "C" {

#define LCPP_HIP_DEFINE_SPMV(VS, VT, IS, IT)                                                                      \
    int lcpp_hip_spmv_csr_##VS##_##IS(void* temp, size_t temp_bytes, const VT* values, const IT* row_offsets,     \
                                      const IT* column_indices, const VT* x, VT* y, uint64_t rows, uint64_t cols, \
                                      uint64_t nnz, void* stream) {                                               \
        return spmv_csr<VT, IT>(temp, temp_bytes, values, row_offsets, column_indices, x, y, rows, cols, nnz,     \
                                stream);                                                                          \
    }
LCPP_HIP_DEFINE_SPMV(f32, float, i32, int32_t)
LCPP_HIP_DEFINE_SPMV(f32, float, u32, uint32_t)
LCPP_HIP_DEFINE_SPMV(f64, double, i32, int32_t)
LCPP_HIP_DEFINE_SPMV(f64, double, u32, uint32_t)
LCPP_HIP_DEFINE_SPMV(i32, int32_t, i32, int32_t)
LCPP_HIP_DEFINE_SPMV(i32, int32_t, u32, uint32_t)
LCPP_HIP_DEFINE_SPMV(u32, uint32_t, i32, int32_t)
LCPP_HIP_DEFINE_SPMV(u32, uint32_t, u32, uint32_t)
#undef LCPP_HIP_DEFINE_SPMV

}  // extern "C"
