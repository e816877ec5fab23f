// Host baselines of the five benchmark configurations, single-threaded or split over std::threads.
//
// Test and measurement infrastructure, like oracle.c: bench.py's cpu_baseline leg times these on the
// host cores of the GPU machine, and tests/test_oracle.py checks every function against the serial
// oracle.  Nothing of the library links or calls this file.
//
// They restate the reference's own host checks, the "host reference" of its tests and benchmark:
//   reduce  - integer accumulation (tests/lcpp_cub_bench.cpp:516-521), here in int64 per thread chunk;
//   scan    - running sum (tests/lcpp_cub_bench.cpp:666-672, std::exclusive_scan in
//             tests/device_scan_test.cpp:117), as chunk sums, a scan of the chunk sums, and a second pass;
//   sort    - stable LSD radix sort with 8-bit digits (the semantics the reference asserts with std::sort
//             and std::stable_sort, tests/lcpp_cub_bench.cpp:892-893,
//             tests/device_radix_sort_interface_test.cpp:86-93): per pass every thread counts its
//             contiguous chunk, the (digit, thread) counts are scanned digit-major, and every thread
//             scatters its chunk in order, so equal digits keep their input order;
//   spmv    - CSR row loop (tests/device_spmv_test.cpp:69-76) in float, rows split by nonzeros.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace {

template <typename F>
void parallel_for(int threads, F&& f) {
    if (threads <= 1) {
        f(0);
        return;
    }
    std::vector<std::thread> pool;
    pool.reserve(static_cast<size_t>(threads - 1));
    for (int t = 1; t < threads; ++t) pool.emplace_back(f, t);
    f(0);
    for (auto& th : pool) th.join();
}

inline uint64_t chunk_begin(uint64_t n, int threads, int t) { return n * static_cast<uint64_t>(t) / static_cast<uint64_t>(threads); }

// One stable counting pass of 8-bit digits at `shift` from (ks, vs) into (kd, vd).
template <typename K, typename V>
void radix_pass(const K* ks, const V* vs, K* kd, V* vd, uint64_t n, unsigned shift, int threads,
                std::vector<uint64_t>& counts) {
    counts.assign(static_cast<size_t>(threads) * 256, 0);
    parallel_for(threads, [&](int t) {
        uint64_t* c = &counts[static_cast<size_t>(t) * 256];
        const uint64_t b = chunk_begin(n, threads, t), e = chunk_begin(n, threads, t + 1);
        for (uint64_t i = b; i < e; ++i) ++c[(ks[i] >> shift) & 0xFF];
    });
    uint64_t run = 0;
    for (int d = 0; d < 256; ++d)
        for (int t = 0; t < threads; ++t) {
            uint64_t& c = counts[static_cast<size_t>(t) * 256 + d];
            const uint64_t x = c;
            c = run;
            run += x;
        }
    parallel_for(threads, [&](int t) {
        uint64_t* c = &counts[static_cast<size_t>(t) * 256];
        const uint64_t b = chunk_begin(n, threads, t), e = chunk_begin(n, threads, t + 1);
        for (uint64_t i = b; i < e; ++i) {
            const uint64_t pos = c[(ks[i] >> shift) & 0xFF]++;
            kd[pos] = ks[i];
            if (vs) vd[pos] = vs[i];
        }
    });
}

}  // namespace

extern "C" {

int64_t oracle_par_reduce_sum_i32(const int32_t* a, uint64_t n, int threads) {
    std::vector<int64_t> part(static_cast<size_t>(std::max(threads, 1)), 0);
    parallel_for(threads, [&](int t) {
        int64_t s = 0;
        const uint64_t b = chunk_begin(n, threads, t), e = chunk_begin(n, threads, t + 1);
        for (uint64_t i = b; i < e; ++i) s += a[i];
        part[static_cast<size_t>(t)] = s;
    });
    int64_t s = 0;
    for (int64_t x : part) s += x;
    return s;
}

// Exclusive sum scan with 32-bit wrap-around.
void oracle_par_scan_sum_u32(const uint32_t* in, uint32_t* out, uint64_t n, int threads) {
    std::vector<uint32_t> sums(static_cast<size_t>(std::max(threads, 1)), 0);
    parallel_for(threads, [&](int t) {
        uint32_t s = 0;
        const uint64_t b = chunk_begin(n, threads, t), e = chunk_begin(n, threads, t + 1);
        for (uint64_t i = b; i < e; ++i) s += in[i];
        sums[static_cast<size_t>(t)] = s;
    });
    uint32_t run = 0;
    for (auto& s : sums) {
        const uint32_t x = s;
        s = run;
        run += x;
    }
    parallel_for(threads, [&](int t) {
        uint32_t s = sums[static_cast<size_t>(t)];
        const uint64_t b = chunk_begin(n, threads, t), e = chunk_begin(n, threads, t + 1);
        for (uint64_t i = b; i < e; ++i) {
            out[i] = s;
            s += in[i];
        }
    });
}

// Stable ascending sort of unsigned 32-bit keys in place (tmp: n scratch keys).
void oracle_par_radix_sort_u32(uint32_t* keys, uint32_t* tmp, uint64_t n, int threads) {
    std::vector<uint64_t> counts;
    for (unsigned p = 0; p < 4; p += 2) {
        radix_pass<uint32_t, uint32_t>(keys, nullptr, tmp, nullptr, n, 8 * p, threads, counts);
        radix_pass<uint32_t, uint32_t>(tmp, nullptr, keys, nullptr, n, 8 * (p + 1), threads, counts);
    }
}

// std::sort of the same keys on one thread (the reference benchmark's own host check).
void oracle_std_sort_u32(uint32_t* keys, uint64_t n) { std::sort(keys, keys + n); }

// Stable ascending sort of unsigned 64-bit keys with 32-bit values, in place (tk, tv: scratch).
void oracle_par_radix_sort_u64_u32(uint64_t* keys, uint32_t* vals, uint64_t* tk, uint32_t* tv, uint64_t n, int threads) {
    std::vector<uint64_t> counts;
    for (unsigned p = 0; p < 8; p += 2) {
        radix_pass<uint64_t, uint32_t>(keys, vals, tk, tv, n, 8 * p, threads, counts);
        radix_pass<uint64_t, uint32_t>(tk, tv, keys, vals, n, 8 * (p + 1), threads, counts);
    }
}

// y = A x for a CSR matrix with float values and int32 column indices; each row sums its products in
// order in float.  Rows are split so that every thread gets about the same number of nonzeros.
void oracle_par_spmv_csr_f32(const float* values, const int32_t* row_offsets, const int32_t* cols, const float* x,
                             float* y, uint64_t rows, int threads) {
    const uint64_t nnz = static_cast<uint64_t>(row_offsets[rows]);
    std::vector<uint64_t> first(static_cast<size_t>(threads) + 1, rows);
    for (int t = 0; t < threads; ++t) {
        const uint64_t target = nnz * static_cast<uint64_t>(t) / static_cast<uint64_t>(threads);
        first[static_cast<size_t>(t)] = static_cast<uint64_t>(
            std::lower_bound(row_offsets, row_offsets + rows, static_cast<int64_t>(target),
                             [](int32_t a, int64_t b) { return static_cast<int64_t>(a) < b; }) -
            row_offsets);
    }
    first[0] = 0;
    parallel_for(threads, [&](int t) {
        for (uint64_t r = first[static_cast<size_t>(t)]; r < first[static_cast<size_t>(t) + 1]; ++r) {
            float s = 0.0f;
            for (int32_t j = row_offsets[r]; j < row_offsets[r + 1]; ++j) s += values[j] * x[cols[j]];
            y[r] = s;
        }
    });
}

}  // extern "C"
