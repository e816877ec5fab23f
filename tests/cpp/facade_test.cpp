// C++20 facade tests: the reference's module-level test cases, written against
// luisa::parallel_primitive::{DeviceReduce, DeviceScan, DeviceRadixSort, DeviceSpmv} as a reference
// user would call them (CommandList recording, commit on a Stream, host checks with std:: algorithms).
//
// Case sources: tests/device_reduce_test.cpp:95-173,425-514, tests/device_scan_test.cpp:80-447,
// tests/device_select_test.cpp:248-500, tests/device_partition_test.cpp:103-377,
// tests/device_run_length_encode_test.cpp:172-340, tests/device_segment_reduce.cpp:438-548,
// tests/device_segmented_scan_test.cpp:11-257, tests/device_segmented_sort_test.cpp:19-790,
// tests/device_radix_sort_interface_test.cpp:68-283, tests/device_radix_sort_one_sweep.cpp:79-333,
// tests/device_spmv_test.cpp:41-203 and the bench generators of tests/lcpp_cub_bench.cpp:516-521,
// 666-672, 814.
//
// Usage: facade_test [--list] [case-substring]
#include <lcpp/parallel_primitive.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <numeric>
#include <random>
#include <string>
#include <vector>

using namespace luisa;
using namespace luisa::compute;
using namespace luisa::parallel_primitive;

namespace {

struct Case {
    const char* name;
    std::function<void()> body;
};

int g_failures = 0;
std::string g_current;

#define EXPECT(cond)                                                                               \
    do {                                                                                           \
        if (!(cond)) {                                                                             \
            ++g_failures;                                                                          \
            std::printf("  FAILED %s:%d in %s: %s\n", __FILE__, __LINE__, g_current.c_str(), #cond); \
        }                                                                                          \
    } while (0)

template <typename F>
bool throws_error(F&& f) {
    try {
        f();
    } catch (const luisa::Error&) {
        return true;
    }
    return false;
}

// splitmix64 stream, the generator the repository's tests and benchmarks use.
uint64_t mix64(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Env {
    Context context;
    Device device;
    Stream stream;
    DeviceReduce<> reduce;
    DeviceScan<> scan;
    DeviceRadixSort<> radix_sort;
    DeviceSpmv<> spmv;
    DeviceSelect<> select;
    DevicePartition<> partition;
    DeviceRunLengthEncode<> rle;
    DeviceSegmentReduce<> segment_reduce;
    DeviceSegmentedScan<> segmented_scan;
    DeviceSegmentedSort<> segmented_sort;
    DeviceSegmentedRadixSort<> segmented_radix_sort;
    Env() : device(context.create_device("hip")), stream(device.create_stream()) {
        segment_reduce.create(device);
        segmented_scan.create(device);
        segmented_sort.create(device);
        segmented_radix_sort.create(device);
        select.create(device);
        partition.create(device);
        rle.create(device);
        reduce.create(device, &stream);
        scan.create(device, &stream);
        radix_sort.create(device, &stream);
        spmv.create(device);
    }
};

Env* g_env = nullptr;

// ---- DeviceReduce ------------------------------------------------------------------------------

void reduce_sum_of_ones() {
    auto& e = *g_env;
    for (uint k : {0u, 5u, 11u, 12u, 17u, 20u, 24u}) {
        const uint n = (1u << k) + 1u;
        std::vector<int> ones(n, 1);
        auto in = e.device.create_buffer<int>(n);
        auto out = e.device.create_buffer<int>(1);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetTempStorageBytes<int>(n)));
        CommandList cmd;
        e.reduce.Sum(cmd, temp.view(), in.view(), out.view(), n);
        int result = -1;
        e.stream << in.copy_from(luisa::span{ones}) << cmd.commit() << out.copy_to(&result) << synchronize();
        EXPECT(result == static_cast<int>(n));
    }
}

void reduce_empty_writes_init() {
    auto& e = *g_env;
    auto out = e.device.create_buffer<int>(1);
    int sentinel = 77;
    CommandList cmd;
    e.reduce.Sum(cmd, BufferView<uint>{}, BufferView<int>{}, out.view(), 0u);
    int result = -1;
    e.stream << out.copy_from(&sentinel) << cmd.commit() << out.copy_to(&result) << synchronize();
    EXPECT(result == 0);
}

// tests/device_reduce_test.cpp:175-345: Min / Max against std::min_element / max_element, Max of floats
// from the lowest identity, ArgMax's first equal extremum, ArgMax of negative floats, and the empty-input
// sentinels (value max / lowest, index 1).
void reduce_min_max_and_arg() {
    auto& e = *g_env;
    {
        const uint n = 100003u;
        std::vector<int> a(n);
        uint32_t x = 12345u;
        for (uint i = 0; i < n; ++i) {
            x = x * 1664525u + 1013904223u;
            a[i] = static_cast<int>(x);
        }
        auto in = e.device.create_buffer<int>(n);
        auto lo = e.device.create_buffer<int>(1);
        auto hi = e.device.create_buffer<int>(1);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetTempStorageBytes<int>(n)));
        CommandList cmd;
        e.reduce.Min(cmd, temp.view(), in.view(), lo.view(), n);
        e.reduce.Max(cmd, temp.view(), in.view(), hi.view(), n);
        int rlo = 0, rhi = 0;
        e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << lo.copy_to(&rlo) << hi.copy_to(&rhi)
                 << synchronize();
        EXPECT(rlo == *std::min_element(a.begin(), a.end()));
        EXPECT(rhi == *std::max_element(a.begin(), a.end()));
    }
    {
        std::vector<float> a{-8.0f, -2.5f, -9.0f, -4.0f};
        auto in = e.device.create_buffer<float>(a.size());
        auto out = e.device.create_buffer<float>(1);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetTempStorageBytes<float>(a.size())));
        CommandList cmd;
        e.reduce.Max(cmd, temp.view(), in.view(), out.view(), a.size());
        float r = 0.0f;
        e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << out.copy_to(&r) << synchronize();
        EXPECT(r == -2.5f);
    }
    {
        std::vector<int> a{1, 9, 4, 9, 3};
        auto in = e.device.create_buffer<int>(a.size());
        auto value = e.device.create_buffer<int>(1);
        auto index = e.device.create_buffer<uint>(1);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetArgTempStorageBytes<int>(a.size())));
        CommandList cmd;
        e.reduce.ArgMax(cmd, temp.view(), in.view(), value.view(), index.view(), a.size());
        int v = 0;
        uint i = 0;
        e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << value.copy_to(&v) << index.copy_to(&i)
                 << synchronize();
        EXPECT(v == 9 && i == 1u);
    }
    {
        std::vector<float> a{-7.0f, -3.0f, -5.0f};
        auto in = e.device.create_buffer<float>(a.size());
        auto value = e.device.create_buffer<float>(1);
        auto index = e.device.create_buffer<uint>(1);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetArgTempStorageBytes<float>(a.size())));
        CommandList cmd;
        e.reduce.ArgMax(cmd, temp.view(), in.view(), value.view(), index.view(), a.size());
        float v = 0.0f;
        uint i = 0;
        e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << value.copy_to(&v) << index.copy_to(&i)
                 << synchronize();
        EXPECT(v == -3.0f && i == 1u);
    }
    {
        auto min_value = e.device.create_buffer<int>(1);
        auto min_index = e.device.create_buffer<uint>(1);
        auto max_value = e.device.create_buffer<int>(1);
        auto max_index = e.device.create_buffer<uint>(1);
        CommandList cmd;
        e.reduce.ArgMin(cmd, BufferView<uint>{}, BufferView<int>{}, min_value.view(), min_index.view(), 0u);
        e.reduce.ArgMax(cmd, BufferView<uint>{}, BufferView<int>{}, max_value.view(), max_index.view(), 0u);
        int vmin = 0, vmax = 0;
        uint imin = 0, imax = 0;
        e.stream << cmd.commit() << min_value.copy_to(&vmin) << min_index.copy_to(&imin) << max_value.copy_to(&vmax)
                 << max_index.copy_to(&imax) << synchronize();
        EXPECT(vmin == std::numeric_limits<int>::max() && imin == 1u);
        EXPECT(vmax == std::numeric_limits<int>::lowest() && imax == 1u);
    }
}

void reduce_bench_pattern_int_and_float() {
    auto& e = *g_env;
    const uint n = (1u << 22) + 13u;
    std::vector<int> a(n);
    std::vector<float> f(n);
    int64_t exact = 0;
    double fexact = 0.0, fabs_sum = 0.0;
    for (uint i = 0; i < n; ++i) {
        a[i] = static_cast<int>(i % 13u) - 6;
        exact += a[i];
        f[i] = static_cast<float>(static_cast<int64_t>(mix64(5, i) >> 40) - (1 << 23)) / float(1 << 23);
        fexact += f[i];
        fabs_sum += std::fabs(f[i]);
    }
    auto in = e.device.create_buffer<int>(n);
    auto fin = e.device.create_buffer<float>(n);
    auto out = e.device.create_buffer<int>(1);
    auto fout = e.device.create_buffer<float>(1);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetTempStorageBytes<float>(n)));
    CommandList cmd;
    e.reduce.Sum(cmd, temp.view(), in.view(), out.view(), n);
    e.reduce.Sum(cmd, temp.view(), fin.view(), fout.view(), n);
    int result = 0;
    float fresult = 0.0f;
    e.stream << in.copy_from(luisa::span{a}) << fin.copy_from(luisa::span{f}) << cmd.commit()
             << out.copy_to(&result) << fout.copy_to(&fresult) << synchronize();
    EXPECT(result == static_cast<int>(static_cast<uint32_t>(exact)));
    // Any summation order is within n * eps * sum|x| of the exact sum.
    EXPECT(std::fabs(double(fresult) - fexact) <= double(n) * 1.2e-7 * fabs_sum);
}

// tests/device_reduce_test.cpp:120-173: TransformReduce of the squares with max and init 0 over a shuffled
// 0..4095, and of 2x + 1 with the sum and init 17 at eight sizes (the transform applied once per item);
// tests/pr6_review_regression_test.cpp:144-240: Reduce with sum and max, TransformReduce with x + 1,
// x + 7, 2x, x * x and the identity over i % 7 + 1.
void reduce_with_operator_and_transform() {
    auto& e = *g_env;
    {
        std::vector<int> a(4096);
        std::iota(a.begin(), a.end(), 0);
        std::mt19937 rng(114521);
        std::shuffle(a.begin(), a.end(), rng);
        auto in = e.device.create_buffer<int>(a.size());
        auto out = e.device.create_buffer<int>(1);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetTempStorageBytes<int>(a.size())));
        CommandList cmd;
        e.reduce.TransformReduce(cmd, temp.view(), in.view(), out.view(), a.size(), MaxOp{}, SquareOp{}, 0);
        int result = 0;
        e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << out.copy_to(&result) << synchronize();
        EXPECT(result == 4095 * 4095);
    }
    for (size_t size : {1u, 31u, 256u, 1023u, 1024u, 1025u, 1048577u, 4194304u}) {
        std::vector<int> a(size);
        int expected = 17;
        for (size_t i = 0; i < size; ++i) {
            a[i] = static_cast<int>(i % 13u) - 6;
            expected += 2 * a[i] + 1;
        }
        auto in = e.device.create_buffer<int>(size);
        auto out = e.device.create_buffer<int>(1);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetTempStorageBytes<int>(size)));
        CommandList cmd;
        e.reduce.TransformReduce(cmd, temp.view(), in.view(), out.view(), size, SumOp{}, AffineOp<int>{2, 1}, 17);
        int result = -12345;
        e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << out.copy_to(&result) << synchronize();
        EXPECT(result == expected);
    }
    const size_t n = 4097;
    std::vector<int> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = static_cast<int>(i % 7u) + 1;
    const int sum = std::accumulate(h.begin(), h.end(), 0);
    int sum_square = 0;
    for (int x : h) sum_square += x * x;
    auto in = e.device.create_buffer<int>(n);
    auto out = e.device.create_buffer<int>(8);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceReduce<>::GetTempStorageBytes<int>(n)));
    CommandList cmd;
    e.reduce.Reduce(cmd, temp.view(), in.view(), out.view(0, 1), n, SumOp{}, 0);
    e.reduce.Reduce(cmd, temp.view(), in.view(), out.view(1, 1), n, MaxOp{}, 0);
    e.reduce.TransformReduce(cmd, temp.view(), in.view(), out.view(2, 1), n, SumOp{}, AffineOp<int>{1, 1}, 0);
    e.reduce.TransformReduce(cmd, temp.view(), in.view(), out.view(3, 1), n, SumOp{}, AffineOp<int>{1, 7}, 0);
    e.reduce.TransformReduce(cmd, temp.view(), in.view(), out.view(4, 1), n, SumOp{}, AffineOp<int>{2, 0}, 0);
    e.reduce.TransformReduce(cmd, temp.view(), in.view(), out.view(5, 1), n, SumOp{}, SquareOp{}, 0);
    e.reduce.TransformReduce(cmd, temp.view(), in.view(), out.view(6, 1), n, SumOp{}, IdentityOp{}, 0);
    e.reduce.Reduce(cmd, BufferView<uint>{}, BufferView<int>{}, out.view(7, 1), 0u, MinOp{}, -9);  // empty: init
    std::vector<int> r(8, 0);
    e.stream << in.copy_from(luisa::span{h}) << cmd.commit() << out.copy_to(luisa::span{r}) << synchronize();
    EXPECT(r[0] == sum && r[1] == 7 && r[2] == sum + static_cast<int>(n) && r[3] == sum + 7 * static_cast<int>(n));
    EXPECT(r[4] == 2 * sum && r[5] == sum_square && r[6] == sum && r[7] == -9);
}

// ---- DeviceScan --------------------------------------------------------------------------------

void scan_sums_of_ones() {
    auto& e = *g_env;
    for (uint k : {0u, 1u, 7u, 12u, 15u, 20u}) {
        const uint n = 1u << k;
        std::vector<uint> ones(n, 1u), ex(n), inc(n);
        auto in = e.device.create_buffer<uint>(n);
        auto out_ex = e.device.create_buffer<uint>(n);
        auto out_in = e.device.create_buffer<uint>(n);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceScan<>::GetTempStorageBytes<uint>(n)));
        CommandList cmd;
        e.scan.ExclusiveSum(cmd, temp.view(), in.view(), out_ex.view(), n);
        e.scan.InclusiveSum(cmd, temp.view(), in.view(), out_in.view(), n);
        e.stream << in.copy_from(luisa::span{ones}) << cmd.commit() << out_ex.copy_to(luisa::span{ex})
                 << out_in.copy_to(luisa::span{inc}) << synchronize();
        bool ok = true;
        for (uint i = 0; i < n; ++i) ok = ok && ex[i] == i && inc[i] == i + 1;
        EXPECT(ok);
    }
}

// tests/device_scan_test.cpp:267-286: InclusiveSum<double> over 17 ones with reference-sized temp storage.
void scan_double_inclusive_sum() {
    auto& e = *g_env;
    constexpr size_t n = 17u;
    std::vector<double> input(n, 1.0), result(n, -1.0);
    auto in = e.device.create_buffer<double>(n);
    auto out = e.device.create_buffer<double>(n);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceScan<>::GetTempStorageBytes<double>(n)));
    CommandList cmd;
    e.scan.InclusiveSum(cmd, temp.view(), in.view(), out.view(), n);
    e.stream << in.copy_from(luisa::span{input}) << cmd.commit() << out.copy_to(luisa::span{result}) << synchronize();
    bool ok = true;
    for (size_t i = 0; i < n; ++i) ok = ok && result[i] == static_cast<double>(i + 1u);
    EXPECT(ok);
}

// 64-bit integers wrap modulo 2^64 like std::exclusive_scan over int64_t bits.
void scan_int64_exclusive_vs_std() {
    auto& e = *g_env;
    const uint n = 100003u;
    std::vector<int64_t> a(n), got(n), want(n);
    uint64_t x = 0x9E3779B97F4A7C15ull;
    for (uint i = 0; i < n; ++i) {
        x ^= x << 13; x ^= x >> 7; x ^= x << 17;
        a[i] = static_cast<int64_t>(x);
    }
    uint64_t run = 0;
    for (uint i = 0; i < n; ++i) { want[i] = static_cast<int64_t>(run); run += static_cast<uint64_t>(a[i]); }
    auto in = e.device.create_buffer<int64_t>(n);
    auto out = e.device.create_buffer<int64_t>(n);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceScan<>::GetTempStorageBytes<int64_t>(n)));
    CommandList cmd;
    e.scan.ExclusiveSum(cmd, temp.view(), in.view(), out.view(), n);
    e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << out.copy_to(luisa::span{got}) << synchronize();
    EXPECT(got == want);
}

void scan_inclusive_init_in_place() {
    auto& e = *g_env;
    std::array<int, 4> input{1, 2, 3, 4};
    const std::array<int, 4> expected{11, 13, 16, 20};
    auto data = e.device.create_buffer<int>(input.size());
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceScan<>::GetTempStorageBytes<int>(input.size())));
    CommandList cmd;
    e.scan.InclusiveScanInit(cmd, temp.view(), data.view(), data.view(), input.size(), SumOp{}, 10);
    e.scan.InclusiveScanInit(cmd, BufferView<uint>{}, BufferView<int>{}, BufferView<int>{}, 0u, SumOp{}, 10);
    std::array<int, 4> result{};
    e.stream << data.copy_from(luisa::span{input}) << cmd.commit() << data.copy_to(luisa::span{result})
             << synchronize();
    EXPECT(result == expected);
}

// tests/pr6_review_regression_test.cpp:146-151,247-265: ExclusiveScan with a max operator and init 0
// over i % 7 + 1 gives min(i, 7); InclusiveScan / InclusiveScanInit with MinOp against std::inclusive_scan
// over signed 64-bit items (signed comparison: negative items are the smaller).
void scan_min_max_operators() {
    auto& e = *g_env;
    {
        constexpr uint n = 4097u;
        std::vector<int> a(n), got(n);
        for (uint i = 0; i < n; ++i) a[i] = static_cast<int>(i % 7u) + 1;
        auto in = e.device.create_buffer<int>(n);
        auto out = e.device.create_buffer<int>(n);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceScan<>::GetTempStorageBytes<int>(n)));
        CommandList cmd;
        e.scan.ExclusiveScan(cmd, temp.view(), in.view(), out.view(), n, MaxOp{}, 0);
        e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << out.copy_to(luisa::span{got}) << synchronize();
        bool ok = true;
        for (uint i = 0; i < n; ++i) ok = ok && got[i] == static_cast<int>(std::min(i, 7u));
        EXPECT(ok);
    }
    {
        const uint n = 3u * 12288u + 11u;
        std::vector<int64_t> a(n), got(n), got_init(n), want(n), want_init(n);
        uint64_t x = 0x2545F4914F6CDD1Dull;
        for (uint i = 0; i < n; ++i) {
            x ^= x << 13; x ^= x >> 7; x ^= x << 17;
            a[i] = static_cast<int64_t>(x);
        }
        const auto lesser = [](int64_t p, int64_t q) { return std::min(p, q); };
        std::inclusive_scan(a.begin(), a.end(), want.begin(), lesser);
        std::inclusive_scan(a.begin(), a.end(), want_init.begin(), lesser, int64_t(-5));
        auto in = e.device.create_buffer<int64_t>(n);
        auto out = e.device.create_buffer<int64_t>(n);
        auto out_init = e.device.create_buffer<int64_t>(n);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceScan<>::GetTempStorageBytes<int64_t>(n)));
        CommandList cmd;
        e.scan.InclusiveScan(cmd, temp.view(), in.view(), out.view(), n, MinOp{});
        e.scan.InclusiveScanInit(cmd, temp.view(), in.view(), out_init.view(), n, MinOp{}, int64_t(-5));
        e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << out.copy_to(luisa::span{got})
                 << out_init.copy_to(luisa::span{got_init}) << synchronize();
        EXPECT(got == want);
        EXPECT(got_init == want_init);
    }
}

void scan_bench_pattern_vs_std() {
    auto& e = *g_env;
    const uint n = (1u << 22) + 5u;
    std::vector<int> a(n), got(n), want(n), got_init(n), want_init(n);
    for (uint i = 0; i < n; ++i) a[i] = static_cast<int>(i % 7u) - 3;
    std::exclusive_scan(a.begin(), a.end(), want.begin(), 0);
    std::exclusive_scan(a.begin(), a.end(), want_init.begin(), 1000);
    auto in = e.device.create_buffer<int>(n);
    auto out = e.device.create_buffer<int>(n);
    auto out2 = e.device.create_buffer<int>(n);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceScan<>::GetTempStorageBytes<int>(n)));
    CommandList cmd;
    e.scan.ExclusiveSum(cmd, temp.view(), in.view(), out.view(), n);
    e.scan.ExclusiveScan(cmd, temp.view(), in.view(), out2.view(), n, SumOp{}, 1000);
    e.stream << in.copy_from(luisa::span{a}) << cmd.commit() << out.copy_to(luisa::span{got})
             << out2.copy_to(luisa::span{got_init}) << synchronize();
    EXPECT(got == want);
    EXPECT(got_init == want_init);
}

// ---- DeviceRadixSort ---------------------------------------------------------------------------

template <typename T, typename Sel>
std::vector<uint> stable_order(const std::vector<T>& keys, Sel sel, bool descending) {
    std::vector<uint> order(keys.size());
    std::iota(order.begin(), order.end(), 0u);
    std::stable_sort(order.begin(), order.end(), [&](uint l, uint r) {
        return descending ? sel(keys[l]) > sel(keys[r]) : sel(keys[l]) < sel(keys[r]);
    });
    return order;
}

template <typename T>
bool follows(const std::vector<T>& result, const std::vector<T>& source, const std::vector<uint>& order) {
    for (size_t i = 0; i < order.size(); ++i)
        if (std::memcmp(&result[i], &source[order[i]], sizeof(T)) != 0) return false;
    return true;
}

void radix_stable_partial_bit_ranges() {
    auto& e = *g_env;
    constexpr uint n = 257u, b = 1u, en = 6u;
    std::vector<uint> keys(n), values(n);
    for (uint i = 0; i < n; ++i) {
        keys[i] = ((i * 53u) % 64u) | (((i * 17u) % 11u) << 8u);
        values[i] = i;
    }
    auto bits = [](uint k) { return (k >> b) & ((1u << (en - b)) - 1u); };
    const auto asc = stable_order(keys, bits, false);
    const auto desc = stable_order(keys, bits, true);
    auto kin = e.device.create_buffer<uint>(n), vin = e.device.create_buffer<uint>(n);
    auto ka = e.device.create_buffer<uint>(n), kd = e.device.create_buffer<uint>(n);
    auto pka = e.device.create_buffer<uint>(n), pva = e.device.create_buffer<uint>(n);
    auto pkd = e.device.create_buffer<uint>(n), pvd = e.device.create_buffer<uint>(n);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceRadixSort<>::GetSortPairsTempStorageBytes<uint, uint>(n)));
    CommandList cmd;
    e.radix_sort.SortKeys(cmd, temp.view(), kin.view(), ka.view(), n, b, en);
    e.radix_sort.SortKeysDescending(cmd, temp.view(), kin.view(), kd.view(), n, b, en);
    e.radix_sort.SortPairs(cmd, temp.view(), kin.view(), pka.view(), vin.view(), pva.view(), n, b, en);
    e.radix_sort.SortPairsDescending(cmd, temp.view(), kin.view(), pkd.view(), vin.view(), pvd.view(), n, b, en);
    e.stream << kin.copy_from(luisa::span{keys}) << vin.copy_from(luisa::span{values}) << cmd.commit();
    std::vector<uint> r_ka(n), r_kd(n), r_pka(n), r_pva(n), r_pkd(n), r_pvd(n);
    e.stream << ka.copy_to(luisa::span{r_ka}) << kd.copy_to(luisa::span{r_kd}) << pka.copy_to(luisa::span{r_pka})
             << pva.copy_to(luisa::span{r_pva}) << pkd.copy_to(luisa::span{r_pkd})
             << pvd.copy_to(luisa::span{r_pvd}) << synchronize();
    EXPECT(follows(r_ka, keys, asc));
    EXPECT(follows(r_kd, keys, desc));
    EXPECT(follows(r_pka, keys, asc));
    EXPECT(follows(r_pva, values, asc));
    EXPECT(follows(r_pkd, keys, desc));
    EXPECT(follows(r_pvd, values, desc));
}

void radix_zero_width_copies() {
    auto& e = *g_env;
    constexpr uint n = 17u;
    std::vector<int> keys(n);
    std::vector<uint> values(n);
    for (uint i = 0; i < n; ++i) {
        keys[i] = static_cast<int>(i * 7u) - 31;
        values[i] = n - i;
    }
    auto kin = e.device.create_buffer<int>(n), kout = e.device.create_buffer<int>(n);
    auto vin = e.device.create_buffer<uint>(n), vout = e.device.create_buffer<uint>(n);
    CommandList cmd;
    e.radix_sort.SortPairs(cmd, BufferView<uint>{}, kin.view(), kout.view(), vin.view(), vout.view(), n, 9u, 9u);
    e.stream << kin.copy_from(luisa::span{keys}) << vin.copy_from(luisa::span{values}) << cmd.commit();
    std::vector<int> rk(n);
    std::vector<uint> rv(n);
    e.stream << kout.copy_to(luisa::span{rk}) << vout.copy_to(luisa::span{rv}) << synchronize();
    EXPECT(rk == keys);
    EXPECT(rv == values);
}

void radix_empty_input() {
    auto& e = *g_env;
    CommandList cmd;
    e.radix_sort.SortKeys(cmd, BufferView<uint>{}, BufferView<int>{}, BufferView<int>{}, 0u);
    e.stream << cmd.commit() << synchronize();
    EXPECT(DeviceRadixSort<>::GetSortKeysTempStorageBytes<int>(0u) == 0u);
}

void radix_double_buffer_selectors() {
    auto& e = *g_env;
    constexpr uint n = 65u, b = 0u, en = 5u;
    std::vector<uint> keys(n), values(n);
    for (uint i = 0; i < n; ++i) {
        keys[i] = ((i * 19u) % 32u) | ((i % 7u) << 8u);
        values[i] = i;
    }
    auto bits = [](uint k) { return k & 31u; };
    const auto asc = stable_order(keys, bits, false);
    const auto desc = stable_order(keys, bits, true);
    auto k0 = e.device.create_buffer<uint>(n), k1 = e.device.create_buffer<uint>(n);
    auto pk0 = e.device.create_buffer<uint>(n), pk1 = e.device.create_buffer<uint>(n);
    auto pv0 = e.device.create_buffer<uint>(n), pv1 = e.device.create_buffer<uint>(n);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceRadixSort<>::GetSortPairsTempStorageBytes<uint, uint>(n)));
    DoubleBuffer<uint> kb(k0.view(), k1.view());
    kb.selector = 1;
    DoubleBuffer<uint> pk(pk0.view(), pk1.view());
    DoubleBuffer<uint> pv(pv0.view(), pv1.view());
    CommandList cmd;
    e.radix_sort.SortKeys(cmd, temp.view(), kb, n, b, en);
    e.radix_sort.SortPairsDescending(cmd, temp.view(), pk, pv, n, b, en);
    EXPECT(kb.selector == 0);  // one pass flips the selector once, at record time
    EXPECT(pk.selector == 1);
    EXPECT(pv.selector == pk.selector);
    e.stream << k1.copy_from(luisa::span{keys}) << pk0.copy_from(luisa::span{keys})
             << pv0.copy_from(luisa::span{values}) << cmd.commit();
    std::vector<uint> ra(n), rdk(n), rdv(n);
    e.stream << kb.current().copy_to(luisa::span{ra}) << pk.current().copy_to(luisa::span{rdk})
             << pv.current().copy_to(luisa::span{rdv}) << synchronize();
    EXPECT(follows(ra, keys, asc));
    EXPECT(follows(rdk, keys, desc));
    EXPECT(follows(rdv, values, desc));
}

void radix_double_buffer_zero_width_keeps_current() {
    auto& e = *g_env;
    std::array<int, 3> input{7, 2, 5};
    auto b0 = e.device.create_buffer<int>(3), b1 = e.device.create_buffer<int>(3);
    DoubleBuffer<int> buffers(b0.view(), b1.view());
    buffers.selector = 1;
    CommandList cmd;
    e.radix_sort.SortKeys(cmd, BufferView<uint>{}, buffers, 3u, 4u, 4u);
    EXPECT(buffers.selector == 1);
    e.stream << b1.copy_from(luisa::span{input}) << cmd.commit();
    std::array<int, 3> result{};
    e.stream << buffers.current().copy_to(luisa::span{result}) << synchronize();
    EXPECT(result == input);
}

void radix_large_keys_and_pairs() {
    auto& e = *g_env;
    const uint n = (1u << 22) + 1234u;
    std::vector<uint> keys(n);
    for (uint i = 0; i < n; ++i) keys[i] = (i * 2654435761u) ^ (i >> 7);  // lcpp_cub_bench.cpp:814
    std::vector<uint> want = keys;
    std::sort(want.begin(), want.end());
    std::vector<uint64_t> k64(n);
    std::vector<uint> idx(n);
    for (uint i = 0; i < n; ++i) {
        k64[i] = mix64(9, i) & mix64(10, i) & mix64(11, i);  // low-entropy keys: long runs of equal digits
        idx[i] = i;
    }
    const auto order = stable_order(k64, [](uint64_t k) { return k; }, false);
    auto kin = e.device.create_buffer<uint>(n), kout = e.device.create_buffer<uint>(n);
    auto pin = e.device.create_buffer<uint64_t>(n), pout = e.device.create_buffer<uint64_t>(n);
    auto vin = e.device.create_buffer<uint>(n), vout = e.device.create_buffer<uint>(n);
    const size_t tb = std::max(DeviceRadixSort<>::GetSortKeysTempStorageBytes<uint>(n),
                               DeviceRadixSort<>::GetSortPairsTempStorageBytes<uint64_t, uint>(n));
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(tb));
    CommandList cmd;
    e.radix_sort.SortKeys(cmd, temp.view(), kin.view(), kout.view(), n);
    e.radix_sort.SortPairs(cmd, temp.view(), pin.view(), pout.view(), vin.view(), vout.view(), n);
    std::vector<uint> got(n), gv(n);
    std::vector<uint64_t> gk(n);
    e.stream << kin.copy_from(luisa::span{keys}) << pin.copy_from(luisa::span{k64}) << vin.copy_from(luisa::span{idx})
             << cmd.commit() << kout.copy_to(luisa::span{got}) << pout.copy_to(luisa::span{gk})
             << vout.copy_to(luisa::span{gv}) << synchronize();
    EXPECT(got == want);
    EXPECT(follows(gk, k64, order));
    EXPECT(gv == order);
}

void radix_float_and_signed_keys() {
    auto& e = *g_env;
    const uint n = 100003u;
    std::vector<float> f(n);
    std::vector<int64_t> s(n);
    for (uint i = 0; i < n; ++i) {
        const uint64_t r = mix64(3, i);
        f[i] = (i % 97u == 0u) ? ((i & 1u) ? -0.0f : 0.0f)
                               : static_cast<float>(static_cast<int64_t>(r >> 40) - (1 << 23)) * 1e-3f;
        s[i] = static_cast<int64_t>(mix64(4, i));
    }
    // -0.0 and +0.0 share a digit pattern (common/util_type.h:141-175), so they stay in input order.
    auto fkey = [](float x) { return x == 0.0f ? 0.0f : x; };
    const auto forder = stable_order(f, fkey, true);
    const auto sorder = stable_order(s, [](int64_t x) { return x; }, false);
    auto fin = e.device.create_buffer<float>(n), fout = e.device.create_buffer<float>(n);
    auto sin = e.device.create_buffer<int64_t>(n), sout = e.device.create_buffer<int64_t>(n);
    const size_t tb = DeviceRadixSort<>::GetSortKeysTempStorageBytes<int64_t>(n);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(tb));
    CommandList cmd;
    e.radix_sort.SortKeysDescending(cmd, temp.view(), fin.view(), fout.view(), n);
    e.radix_sort.SortKeys(cmd, temp.view(), sin.view(), sout.view(), n);
    std::vector<float> gf(n);
    std::vector<int64_t> gs(n);
    e.stream << fin.copy_from(luisa::span{f}) << sin.copy_from(luisa::span{s}) << cmd.commit()
             << fout.copy_to(luisa::span{gf}) << sout.copy_to(luisa::span{gs}) << synchronize();
    EXPECT(follows(gf, f, forder));
    EXPECT(follows(gs, s, sorder));
}

// ---- DeviceSpmv --------------------------------------------------------------------------------

void spmv_float_unsigned_indices() {
    auto& e = *g_env;
    constexpr uint rows = 4u, cols = 5u;
    const std::vector<uint> ro{0u, 3u, 3u, 6u, 8u};
    const std::vector<uint> ci{0u, 2u, 4u, 1u, 2u, 3u, 0u, 4u};
    const std::vector<float> a{1.5f, -2.0f, 0.25f, 3.0f, 1.25f, -0.5f, 2.0f, 4.0f};
    const std::vector<float> x{2.0f, -1.0f, 0.5f, 3.0f, -2.0f};
    std::vector<float> want(rows, 0.0f);
    for (uint r = 0; r < rows; ++r)
        for (uint k = ro[r]; k < ro[r + 1]; ++k) want[r] += a[k] * x[ci[k]];
    auto da = e.device.create_buffer<float>(a.size());
    auto dro = e.device.create_buffer<uint>(ro.size());
    auto dci = e.device.create_buffer<uint>(ci.size());
    auto dx = e.device.create_buffer<float>(x.size());
    auto dy = e.device.create_buffer<float>(rows);
    CommandList cmd;
    e.spmv.CsrMV(cmd, BufferView<uint>{}, da.view(), dro.view(), dci.view(), dx.view(), dy.view(), rows, cols,
                 a.size());
    e.stream << da.copy_from(luisa::span{a}) << dro.copy_from(luisa::span{ro}) << dci.copy_from(luisa::span{ci})
             << dx.copy_from(luisa::span{x}) << cmd.commit();
    std::vector<float> got(rows);
    e.stream << dy.copy_to(luisa::span{got}) << synchronize();
    for (uint r = 0; r < rows; ++r) EXPECT(std::fabs(got[r] - want[r]) < 1.0e-5f);
}

void spmv_int_values_and_empty_work() {
    auto& e = *g_env;
    constexpr uint rows = 3u, cols = 4u;
    const std::vector<int> ro{0, 2, 2, 5};
    const std::vector<int> ci{1, 3, 0, 2, 3};
    const std::vector<int> a{2, -3, 4, 5, -1};
    const std::vector<int> x{7, -2, 3, 6};
    const std::vector<int> want{2 * -2 + -3 * 6, 0, 4 * 7 + 5 * 3 + -1 * 6};
    auto da = e.device.create_buffer<int>(a.size());
    auto dro = e.device.create_buffer<int>(ro.size());
    auto dci = e.device.create_buffer<int>(ci.size());
    auto dx = e.device.create_buffer<int>(x.size());
    auto dy = e.device.create_buffer<int>(rows);
    auto dz = e.device.create_buffer<int>(rows);
    const std::vector<int> junk(rows, 99);
    CommandList cmd;
    e.spmv.CsrMV(cmd, BufferView<uint>{}, da.view(), dro.view(), dci.view(), dx.view(), dy.view(), rows, cols,
                 a.size());
    // nnz == 0 zero-fills y; rows == 0 records nothing (tests/device_spmv_test.cpp:157-203).
    e.spmv.CsrMV(cmd, BufferView<uint>{}, BufferView<int>{}, dro.view(), BufferView<int>{}, BufferView<int>{},
                 dz.view(), rows, 0u, 0u);
    e.spmv.CsrMV(cmd, BufferView<uint>{}, BufferView<int>{}, BufferView<int>{}, BufferView<int>{},
                 BufferView<int>{}, BufferView<int>{}, 0u, 0u, 0u);
    e.stream << da.copy_from(luisa::span{a}) << dro.copy_from(luisa::span{ro}) << dci.copy_from(luisa::span{ci})
             << dx.copy_from(luisa::span{x}) << dz.copy_from(luisa::span{junk}) << cmd.commit();
    std::vector<int> got(rows), zeros(rows, -1);
    e.stream << dy.copy_to(luisa::span{got}) << dz.copy_to(luisa::span{zeros}) << synchronize();
    EXPECT(got == want);
    EXPECT(zeros == std::vector<int>(rows, 0));
}

// ---- by key -------------------------------------------------------------------------------------

// tests/device_scan_test.cpp:323-377: keys i / 100, ones, for sizes 2^5 .. 2^20 (plus a ragged size).
void scan_exclusive_sum_by_key_segments_of_100() {
    auto& e = *g_env;
    for (uint n : {32u, 100u, 4096u, 65536u, (1u << 20), (1u << 20) + 37u}) {
        std::vector<int> keys(n), ones(n, 1), want(n);
        for (uint i = 0; i < n; ++i) {
            keys[i] = static_cast<int>(i / 100u);
            want[i] = static_cast<int>(i % 100u);
        }
        auto kb = e.device.create_buffer<int>(n), vb = e.device.create_buffer<int>(n), ob = e.device.create_buffer<int>(n);
        auto temp = e.device.create_buffer<uint>(
            bytes_to_uint_count(DeviceScan<>::GetScanByKeyTempStorageBytes<int, int>(n)));
        CommandList cmd;
        e.scan.ExclusiveSumByKey(cmd, temp.view(), kb.view(), vb.view(), ob.view(), n);
        std::vector<int> got(n, -1);
        e.stream << kb.copy_from(luisa::span{keys}) << vb.copy_from(luisa::span{ones}) << cmd.commit()
                 << ob.copy_to(luisa::span{got}) << synchronize();
        EXPECT(got == want);
    }
}

// tests/device_scan_test.cpp:380-416: int keys, 64-bit values, runs crossing two 256 x 15 tiles.
void scan_inclusive_sum_by_key_three_tiles_int64() {
    auto& e = *g_env;
    constexpr size_t tile = 256u * 15u;
    constexpr size_t n = tile * 2u + 2u;
    std::vector<int> keys(n);
    std::vector<int64_t> ones(n, 1), want(n);
    int64_t run = 0;
    for (size_t i = 0; i < n; ++i) {
        keys[i] = i < tile + 1u ? 1 : i < tile * 2u + 1u ? 2 : 3;
        if (i == 0 || keys[i] != keys[i - 1]) run = 0;
        want[i] = ++run;
    }
    auto kb = e.device.create_buffer<int>(n);
    auto vb = e.device.create_buffer<int64_t>(n), ob = e.device.create_buffer<int64_t>(n);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceScan<>::GetScanByKeyTempStorageBytes<int, int64_t>(n)));
    CommandList cmd;
    e.scan.InclusiveSumByKey(cmd, temp.view(), kb.view(), vb.view(), ob.view(), n);
    std::vector<int64_t> got(n, -1);
    e.stream << kb.copy_from(luisa::span{keys}) << vb.copy_from(luisa::span{ones}) << cmd.commit()
             << ob.copy_to(luisa::span{got}) << synchronize();
    EXPECT(got == want);
}

// tests/device_scan_test.cpp:419-447: keys equal when their parities match.
void scan_by_key_custom_equality() {
    auto& e = *g_env;
    const std::vector<int> keys{1, 3, 5, 2, 4};
    const std::vector<int> ones(keys.size(), 1);
    auto kb = e.device.create_buffer<int>(keys.size()), vb = e.device.create_buffer<int>(keys.size());
    auto ob = e.device.create_buffer<int>(keys.size());
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceScan<>::GetScanByKeyTempStorageBytes<int, int>(keys.size())));
    CommandList cmd;
    e.scan.InclusiveSumByKey(cmd, temp.view(), kb.view(), vb.view(), ob.view(), keys.size(), KeyMaskEquality{1u});
    std::vector<int> got(keys.size(), -1);
    e.stream << kb.copy_from(luisa::span{keys}) << vb.copy_from(luisa::span{ones}) << cmd.commit()
             << ob.copy_to(luisa::span{got}) << synchronize();
    EXPECT((got == std::vector<int>{1, 2, 3, 1, 2}));
}

// ExclusiveScanByKey / InclusiveScanByKey with an initial value (device_scan.h:424-519), float
// values holding small integers (exact sums) and 64-bit unsigned keys; the inclusive scan runs in place.
void scan_by_key_initial_values_float_in_place() {
    auto& e = *g_env;
    const size_t n = 50000u;
    std::vector<uint64_t> keys(n);
    std::vector<float> vals(n), want_ex(n), want_in(n);
    uint64_t key = 0;
    float run = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        if (mix64(9, i) % 37u == 0u) ++key;
        keys[i] = key * 0x100000001ull;
        vals[i] = static_cast<float>(static_cast<int>(mix64(10, i) % 9u) - 4);
        if (i == 0 || keys[i] != keys[i - 1]) run = 0.0f;
        want_ex[i] = 2.5f + run;
        run += vals[i];
        want_in[i] = -1.0f + run;
    }
    auto kb = e.device.create_buffer<uint64_t>(n);
    auto vb = e.device.create_buffer<float>(n), ob = e.device.create_buffer<float>(n);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceScan<>::GetScanByKeyTempStorageBytes<uint64_t, float>(n)));
    CommandList cmd;
    e.scan.ExclusiveScanByKey(cmd, temp.view(), kb.view(), vb.view(), ob.view(), SumOp{}, n, 2.5f);
    std::vector<float> got_ex(n), got_in(n);
    e.stream << kb.copy_from(luisa::span{keys}) << vb.copy_from(luisa::span{vals}) << cmd.commit()
             << ob.copy_to(luisa::span{got_ex}) << synchronize();
    CommandList cmd2;
    e.scan.InclusiveScanByKey(cmd2, temp.view(), kb.view(), vb.view(), vb.view(), SumOp{}, n, -1.0f);
    e.stream << cmd2.commit() << vb.copy_to(luisa::span{got_in}) << synchronize();
    EXPECT(got_ex == want_ex);
    EXPECT(got_in == want_in);
}

// tests/device_reduce_test.cpp:425-480: keys i / 100 over 4096 items of value i.
void reduce_by_key_segments_of_100() {
    auto& e = *g_env;
    for (uint n : {4096u, 1000003u}) {
        const uint segments = (n + 99u) / 100u;
        std::vector<int> keys(n), vals(n);
        for (uint i = 0; i < n; ++i) {
            keys[i] = static_cast<int>(i / 100u);
            vals[i] = static_cast<int>(i % 1000u);
        }
        auto kb = e.device.create_buffer<int>(n), vb = e.device.create_buffer<int>(n);
        auto ub = e.device.create_buffer<int>(segments), ab = e.device.create_buffer<int>(segments);
        auto rb = e.device.create_buffer<uint>(1);
        auto temp = e.device.create_buffer<uint>(
            bytes_to_uint_count(DeviceReduce<>::GetReduceByKeyTempStorageBytes<int, int>(n)));
        CommandList cmd;
        e.reduce.ReduceByKey(cmd, temp.view(), kb.view(), vb.view(), ub.view(), ab.view(), rb.view(), SumOp{}, n);
        std::vector<int> uniq(segments, -1), agg(segments, -1);
        uint runs = 0;
        e.stream << kb.copy_from(luisa::span{keys}) << vb.copy_from(luisa::span{vals}) << cmd.commit()
                 << ub.copy_to(luisa::span{uniq}) << ab.copy_to(luisa::span{agg}) << rb.copy_to(&runs)
                 << synchronize();
        EXPECT(runs == segments);
        bool ok = true;
        for (uint r = 0; r < segments; ++r) {
            int sum = 0;
            for (uint i = r * 100u; i < std::min(n, r * 100u + 100u); ++i) sum += vals[i];
            ok = ok && uniq[r] == static_cast<int>(r) && agg[r] == sum;
        }
        EXPECT(ok);
    }
}

// tests/device_reduce_test.cpp:483-513: empty input writes zero runs.
// Scan and reduce by key with MinOp / MaxOp: keys {1,1,1,2,2,3}, values {5,3,7,1,9,4}.
void by_key_min_max() {
    auto& e = *g_env;
    std::vector<int> keys{1, 1, 1, 2, 2, 3}, vals{5, 3, 7, 1, 9, 4}, scan_max(6), scan_min_init(6), uniq(6), mins(6);
    uint runs = 0;
    const size_t n = keys.size();
    auto k = e.device.create_buffer<int>(n);
    auto v = e.device.create_buffer<int>(n);
    auto o1 = e.device.create_buffer<int>(n);
    auto o2 = e.device.create_buffer<int>(n);
    auto u = e.device.create_buffer<int>(n);
    auto a = e.device.create_buffer<int>(n);
    auto r = e.device.create_buffer<uint>(1);
    auto st = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceScan<>::GetScanByKeyTempStorageBytes<int, int>(n)));
    auto rt = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceReduce<>::GetReduceByKeyTempStorageBytes<int, int>(n)));
    CommandList cmd;
    e.scan.InclusiveScanByKey(cmd, st.view(), k.view(), v.view(), o1.view(), MaxOp{}, n);
    e.scan.ExclusiveScanByKey(cmd, st.view(), k.view(), v.view(), o2.view(), MinOp{}, n, 4);
    e.reduce.ReduceByKey(cmd, rt.view(), k.view(), v.view(), u.view(), a.view(), r.view(), MinOp{}, n);
    e.stream << k.copy_from(luisa::span{keys}) << v.copy_from(luisa::span{vals}) << cmd.commit()
             << o1.copy_to(luisa::span{scan_max}) << o2.copy_to(luisa::span{scan_min_init}) << u.copy_to(luisa::span{uniq})
             << a.copy_to(luisa::span{mins}) << r.copy_to(&runs) << synchronize();
    EXPECT((scan_max == std::vector<int>{5, 5, 7, 1, 9, 4}));
    EXPECT((scan_min_init == std::vector<int>{4, 4, 3, 4, 1, 4}));
    EXPECT(runs == 3u);
    EXPECT(uniq[0] == 1 && uniq[1] == 2 && uniq[2] == 3 && mins[0] == 3 && mins[1] == 1 && mins[2] == 4);
}

void reduce_by_key_empty_input() {
    auto& e = *g_env;
    auto kb = e.device.create_buffer<int>(1), vb = e.device.create_buffer<int>(1);
    auto ub = e.device.create_buffer<int>(1), ab = e.device.create_buffer<int>(1);
    auto rb = e.device.create_buffer<uint>(1);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceReduce<>::GetReduceByKeyTempStorageBytes<int, int>(0u)));
    uint runs = 17u;
    CommandList cmd;
    e.reduce.ReduceByKey(cmd, temp.view(), kb.view(), vb.view(), ub.view(), ab.view(), rb.view(), SumOp{}, 0u);
    e.stream << rb.copy_from(&runs) << cmd.commit() << rb.copy_to(&runs) << synchronize();
    EXPECT(runs == 0u);
}

// ---- stream compaction ----------------------------------------------------------------------------

template <typename T>
std::vector<T> download(Env& e, Buffer<T>& b, size_t n) {
    std::vector<T> h(n);
    if (n) e.stream << b.view(0, n).copy_to(luisa::span{h}) << synchronize();
    return h;
}

uint read_count(Env& e, Buffer<uint>& b, size_t i = 0) {
    uint v = 0;
    e.stream << b.view(i, 1).copy_to(&v) << synchronize();
    return v;
}

// tests/device_select_test.cpp:248-299.
void select_flagged_and_if_are_stable() {
    auto& e = *g_env;
    constexpr uint n = 17u;
    std::vector<int> in(n);
    std::vector<uint> flags(n);
    for (uint i = 0; i < n; ++i) {
        in[i] = static_cast<int>(100u + i);
        flags[i] = i % 3u == 1u ? 7u : 0u;
    }
    auto ib = e.device.create_buffer<int>(n), fo = e.device.create_buffer<int>(n), io = e.device.create_buffer<int>(n);
    auto fb = e.device.create_buffer<uint>(n);
    auto fc = e.device.create_buffer<uint>(1), ic = e.device.create_buffer<uint>(1);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceSelect<>::GetTempStorageBytes(n)));
    CommandList cmd;
    e.select.Flagged(cmd, temp.view(), ib.view(), fb.view(), fo.view(), fc.view(), n);
    e.select.If(cmd, temp.view(), ib.view(), io.view(), ic.view(), n, ItemPredicate<int>::remainder_equal(2, 0));
    e.stream << ib.copy_from(luisa::span{in}) << fb.copy_from(luisa::span{flags}) << cmd.commit() << synchronize();
    std::vector<int> want_f, want_i;
    for (uint i = 0; i < n; ++i) {
        if (flags[i]) want_f.push_back(in[i]);
        if (in[i] % 2 == 0) want_i.push_back(in[i]);
    }
    const uint kf = read_count(e, fc), ki = read_count(e, ic);
    EXPECT(kf == want_f.size() && ki == want_i.size());
    EXPECT(download(e, fo, kf) == want_f);
    EXPECT(download(e, io, ki) == want_i);
}

// tests/device_select_test.cpp:301-357 and :359-425.
void select_unique_by_key_and_flagged_if() {
    auto& e = *g_env;
    const std::vector<int> keys{1, 1, 2, 2, 2, 4, 7, 7, 9}, vals{10, 11, 20, 21, 22, 40, 70, 71, 90};
    const uint n = static_cast<uint>(keys.size());
    auto kb = e.device.create_buffer<int>(n), vb = e.device.create_buffer<int>(n), uo = e.device.create_buffer<int>(n);
    auto ko = e.device.create_buffer<int>(n), vo = e.device.create_buffer<int>(n);
    auto c1 = e.device.create_buffer<uint>(1), c2 = e.device.create_buffer<uint>(1);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceSelect<>::GetTempStorageBytes(n)));
    CommandList cmd;
    e.select.Unique(cmd, temp.view(), kb.view(), uo.view(), c1.view(), n);
    e.select.UniqueByKey(cmd, temp.view(), kb.view(), vb.view(), ko.view(), vo.view(), c2.view(), n);
    e.stream << kb.copy_from(luisa::span{keys}) << vb.copy_from(luisa::span{vals}) << cmd.commit() << synchronize();
    EXPECT(read_count(e, c1) == 5u && read_count(e, c2) == 5u);
    EXPECT((download(e, uo, 5) == std::vector<int>{1, 2, 4, 7, 9}));
    EXPECT((download(e, ko, 5) == std::vector<int>{1, 2, 4, 7, 9}));
    EXPECT((download(e, vo, 5) == std::vector<int>{10, 20, 40, 70, 90}));

    const std::vector<int> data{100, 101, 102, 103, 104, 105, 106, 107, 108}, flags{-3, -2, -1, 0, 1, 2, 3, 4, 5};
    auto db = e.device.create_buffer<int>(9), ip = e.device.create_buffer<int>(9), fl = e.device.create_buffer<int>(9);
    auto co = e.device.create_buffer<int>(9);
    auto cc = e.device.create_buffer<uint>(1), pc = e.device.create_buffer<uint>(1);
    const auto positive_odd = ItemPredicate<int>::greater(0) && ItemPredicate<int>::remainder_not_equal(2, 0);
    CommandList cmd2;
    e.select.FlaggedIf(cmd2, temp.view(), db.view(), fl.view(), co.view(), cc.view(), 9u, positive_odd);
    e.select.FlaggedIf(cmd2, temp.view(), ip.view(), fl.view(), pc.view(), 9u, positive_odd);
    e.stream << db.copy_from(luisa::span{data}) << ip.copy_from(luisa::span{data}) << fl.copy_from(luisa::span{flags})
             << cmd2.commit() << synchronize();
    EXPECT(read_count(e, cc) == 3u && read_count(e, pc) == 3u);
    EXPECT((download(e, co, 3) == std::vector<int>{104, 106, 108}));
    EXPECT((download(e, ip, 3) == std::vector<int>{104, 106, 108}));
    EXPECT(download(e, db, 9) == data);
}

// tests/device_select_test.cpp:427-500: in-place forms, flags aliased with the data, empty input.
void select_in_place_forms() {
    auto& e = *g_env;
    const std::vector<int> aliased{0, 2, 0, 3, 4, 0, 5, 0}, pred{-3, 4, -1, 6, 0, 2, 7, -8};
    const std::vector<int> uniq{1, 3, 2, 4, 5, 7, 8, 10}, dflt{1, 1, 2, 2, 2, 4, 4, 9};
    auto ab = e.device.create_buffer<int>(8), pb = e.device.create_buffer<int>(8);
    auto ub = e.device.create_buffer<int>(8), db = e.device.create_buffer<int>(8);
    auto counts = e.device.create_buffer<uint>(5);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceSelect<>::GetTempStorageBytes(8)));
    const uint ones[5] = {9, 9, 9, 9, 9};
    CommandList cmd;
    e.select.Flagged(cmd, temp.view(), ab.view(), ab.view(), counts.view(0, 1), 8u);
    e.select.If(cmd, temp.view(), pb.view(), counts.view(1, 1), 8u, ItemPredicate<int>::greater(0));
    e.select.Unique(cmd, temp.view(), ub.view(), counts.view(2, 1), 8u, KeyMaskEquality{1u});
    e.select.Unique(cmd, temp.view(), db.view(), counts.view(3, 1), 8u);
    e.select.If(cmd, BufferView<uint>{}, BufferView<int>{}, counts.view(4, 1), 0u, ItemPredicate<int>::greater(0));
    e.stream << ab.copy_from(luisa::span{aliased}) << pb.copy_from(luisa::span{pred}) << ub.copy_from(luisa::span{uniq})
             << db.copy_from(luisa::span{dflt}) << counts.copy_from(static_cast<const void*>(ones)) << cmd.commit()
             << synchronize();
    EXPECT((download(e, ab, read_count(e, counts, 0)) == std::vector<int>{2, 3, 4, 5}));
    EXPECT((download(e, pb, read_count(e, counts, 1)) == std::vector<int>{4, 6, 2, 7}));
    EXPECT((download(e, ub, read_count(e, counts, 2)) == std::vector<int>{1, 2, 5, 8}));
    EXPECT((download(e, db, read_count(e, counts, 3)) == std::vector<int>{1, 2, 4, 9}));
    EXPECT(read_count(e, counts, 4) == 0u);
}

// tests/device_partition_test.cpp:103-177 and :292-377.
void partition_ordering_and_three_way() {
    auto& e = *g_env;
    constexpr uint n = 12u;
    std::vector<int> in(n);
    std::vector<uint> flags(n);
    for (uint i = 0; i < n; ++i) {
        in[i] = static_cast<int>(i);
        flags[i] = i % 3u == 0u ? 1u : 0u;
    }
    auto ib = e.device.create_buffer<int>(n), fo = e.device.create_buffer<int>(n), po = e.device.create_buffer<int>(n);
    auto fb = e.device.create_buffer<uint>(n);
    auto o1 = e.device.create_buffer<int>(n), o2 = e.device.create_buffer<int>(n), o3 = e.device.create_buffer<int>(n);
    auto counts = e.device.create_buffer<uint>(6);
    auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DevicePartition<>::GetThreeWayTempStorageBytes(n)));
    const uint nines[6] = {9, 9, 9, 9, 9, 9};
    CommandList cmd;
    e.partition.Flagged(cmd, temp.view(), ib.view(), fb.view(), fo.view(), counts.view(0, 1), n);
    e.partition.If(cmd, temp.view(), ib.view(), po.view(), counts.view(1, 1), n, ItemPredicate<int>::less(7));
    e.partition.If(cmd, temp.view(), ib.view(), o1.view(), o2.view(), o3.view(), counts.view(2, 2), n,
                   ItemPredicate<int>::remainder_equal(3, 0), ItemPredicate<int>::less(8));
    e.partition.If(cmd, BufferView<uint>{}, BufferView<int>{}, BufferView<int>{}, BufferView<int>{}, BufferView<int>{},
                   counts.view(4, 2), 0u, ItemPredicate<int>::less(0), ItemPredicate<int>::greater(0));
    e.stream << ib.copy_from(luisa::span{in}) << fb.copy_from(luisa::span{flags})
             << counts.copy_from(static_cast<const void*>(nines)) << cmd.commit() << synchronize();
    EXPECT(read_count(e, counts, 0) == 4u && read_count(e, counts, 1) == 7u);
    EXPECT((download(e, fo, n) == std::vector<int>{0, 3, 6, 9, 11, 10, 8, 7, 5, 4, 2, 1}));
    EXPECT((download(e, po, n) == std::vector<int>{0, 1, 2, 3, 4, 5, 6, 11, 10, 9, 8, 7}));
    EXPECT(read_count(e, counts, 2) == 4u && read_count(e, counts, 3) == 5u);
    EXPECT((download(e, o1, 4) == std::vector<int>{0, 3, 6, 9}));
    EXPECT((download(e, o2, 5) == std::vector<int>{1, 2, 4, 5, 7}));
    EXPECT((download(e, o3, 3) == std::vector<int>{11, 10, 8}));
    EXPECT(read_count(e, counts, 4) == 0u && read_count(e, counts, 5) == 0u);
}

// tests/device_run_length_encode_test.cpp:172-340: CUB's example, 180 runs of length run % 7 + 1,
// and zero counts for empty input.
void run_length_encode_examples() {
    auto& e = *g_env;
    std::vector<int> in{0, 2, 2, 9, 5, 5, 5, 8};
    std::vector<int> want_u{0, 2, 9, 5, 8};
    std::vector<uint> want_c{1, 2, 1, 3, 1}, want_o{1, 4}, want_l{2, 3};
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) {
            in.clear();
            want_u.clear();
            want_c.clear();
            want_o.clear();
            want_l.clear();
            for (uint run = 0; run < 180u; ++run) {
                const uint len = run % 7u + 1u;
                want_u.push_back(static_cast<int>(run));
                want_c.push_back(len);
                if (len > 1u) {
                    want_o.push_back(static_cast<uint>(in.size()));
                    want_l.push_back(len);
                }
                for (uint k = 0; k < len; ++k) in.push_back(static_cast<int>(run));
            }
        }
        const uint n = static_cast<uint>(in.size());
        auto ib = e.device.create_buffer<int>(n), uo = e.device.create_buffer<int>(n);
        auto co = e.device.create_buffer<uint>(n), oo = e.device.create_buffer<uint>(n), lo = e.device.create_buffer<uint>(n);
        auto counts = e.device.create_buffer<uint>(2);
        auto temp = e.device.create_buffer<uint>(bytes_to_uint_count(DeviceRunLengthEncode<>::GetTempStorageBytes(n)));
        CommandList cmd;
        e.rle.Encode(cmd, temp.view(), ib.view(), uo.view(), co.view(), counts.view(0, 1), n);
        e.rle.NonTrivialRuns(cmd, temp.view(), ib.view(), oo.view(), lo.view(), counts.view(1, 1), n);
        e.stream << ib.copy_from(luisa::span{in}) << cmd.commit() << synchronize();
        const uint runs = read_count(e, counts, 0), nt = read_count(e, counts, 1);
        EXPECT(runs == want_u.size() && nt == want_o.size());
        EXPECT(download(e, uo, runs) == want_u);
        EXPECT(download(e, co, runs) == want_c);
        EXPECT(download(e, oo, nt) == want_o);
        EXPECT(download(e, lo, nt) == want_l);
    }
    auto counts = e.device.create_buffer<uint>(2);
    const uint nines[2] = {99, 99};
    CommandList cmd;
    e.rle.Encode(cmd, BufferView<uint>{}, BufferView<int>{}, BufferView<int>{}, BufferView<uint>{}, counts.view(0, 1), 0u);
    e.rle.NonTrivialRuns(cmd, BufferView<uint>{}, BufferView<int>{}, BufferView<uint>{}, BufferView<uint>{},
                         counts.view(1, 1), 0u);
    e.stream << counts.copy_from(static_cast<const void*>(nines)) << cmd.commit() << synchronize();
    EXPECT(read_count(e, counts, 0) == 0u && read_count(e, counts, 1) == 0u);
}

// ---- segmented ------------------------------------------------------------------------------------

// tests/device_segment_reduce.cpp:438-548.
void segment_reduce_known_answers() {
    auto& e = *g_env;
    const std::vector<int> a{4, 6, 8, 10};
    const std::vector<uint> ab{0u, 2u, 2u}, ae{2u, 2u, 4u};
    const std::vector<float> f{-9.0f, -2.0f, -2.0f, -8.0f, -5.0f};
    const std::vector<uint> fb{0u, 1u, 4u}, fe{0u, 4u, 4u};
    const std::vector<int> g{7, 1, 1, 9, 4, 2};
    const std::vector<uint> gb{0u, 3u}, ge{3u, 6u};
    auto ai = e.device.create_buffer<int>(4), ao = e.device.create_buffer<int>(3);
    auto abb = e.device.create_buffer<uint>(3), aeb = e.device.create_buffer<uint>(3);
    auto fi = e.device.create_buffer<float>(5), fo = e.device.create_buffer<float>(3);
    auto fbb = e.device.create_buffer<uint>(3), feb = e.device.create_buffer<uint>(3), fx = e.device.create_buffer<uint>(3);
    auto gi = e.device.create_buffer<int>(6), go = e.device.create_buffer<int>(2);
    auto gbb = e.device.create_buffer<uint>(2), geb = e.device.create_buffer<uint>(2), gx = e.device.create_buffer<uint>(2);
    auto fsum = e.device.create_buffer<int>(2);
    CommandList cmd;
    e.segment_reduce.Sum(cmd, BufferView<uint>{}, ai.view(), ao.view(), 3u, abb.view(), aeb.view());
    e.segment_reduce.ArgMax(cmd, BufferView<uint>{}, fi.view(), fo.view(), fx.view(), 3u, fbb.view(), feb.view());
    e.segment_reduce.ArgMin(cmd, BufferView<uint>{}, gi.view(), go.view(), gx.view(), 2u, gbb.view(), geb.view());
    e.segment_reduce.Max(cmd, BufferView<uint>{}, gi.view(), fsum.view(), 2u, 3u);  // fixed size 3
    e.stream << ai.copy_from(luisa::span{a}) << abb.copy_from(luisa::span{ab}) << aeb.copy_from(luisa::span{ae})
             << fi.copy_from(luisa::span{f}) << fbb.copy_from(luisa::span{fb}) << feb.copy_from(luisa::span{fe})
             << gi.copy_from(luisa::span{g}) << gbb.copy_from(luisa::span{gb}) << geb.copy_from(luisa::span{ge})
             << cmd.commit() << synchronize();
    EXPECT((download(e, ao, 3) == std::vector<int>{10, 0, 18}));
    const float lo = std::numeric_limits<float>::lowest();
    EXPECT((download(e, fo, 3) == std::vector<float>{lo, -2.0f, lo}));
    EXPECT((download(e, fx, 3) == std::vector<uint>{1u, 0u, 1u}));
    EXPECT((download(e, go, 2) == std::vector<int>{1, 2}));
    EXPECT((download(e, gx, 2) == std::vector<uint>{1u, 2u}));
    EXPECT((download(e, fsum, 2) == std::vector<int>{7, 9}));
}

// tests/device_segmented_scan_test.cpp:104-257 (sum forms): same and packed output offsets, and the
// exact in-place inclusive sum.
void segmented_scan_known_answers() {
    auto& e = *g_env;
    const std::vector<int> x{100, 1, 2, 3, 5, 6, 7, 200, 9, 10, 11, 12, 300, 400};
    const std::vector<uint> b{1u, 4u, 4u, 8u}, en{4u, 4u, 7u, 12u}, packed{0u, 4u, 6u, 10u};
    constexpr int S = -777;
    auto xi = e.device.create_buffer<int>(14);
    auto bb = e.device.create_buffer<uint>(4), eb = e.device.create_buffer<uint>(4), pb = e.device.create_buffer<uint>(4);
    auto ex = e.device.create_buffer<int>(14), in = e.device.create_buffer<int>(14), ini = e.device.create_buffer<int>(14);
    auto pex = e.device.create_buffer<int>(14), inplace = e.device.create_buffer<int>(14);
    const std::vector<int> sentinel(14, S);
    CommandList cmd;
    e.segmented_scan.ExclusiveSegmentedSum(cmd, BufferView<uint>{}, xi.view(), ex.view(), bb.view(), eb.view(), 4u);
    e.segmented_scan.InclusiveSegmentedSum(cmd, BufferView<uint>{}, xi.view(), in.view(), bb.view(), eb.view(), 4u);
    e.segmented_scan.InclusiveSegmentedScanInit(cmd, BufferView<uint>{}, xi.view(), ini.view(), bb.view(), eb.view(), 4u,
                                                SumOp{}, 10);
    e.segmented_scan.ExclusiveSegmentedSum(cmd, BufferView<uint>{}, xi.view(), pex.view(), bb.view(), eb.view(), pb.view(),
                                           4u);
    e.segmented_scan.InclusiveSegmentedSum(cmd, BufferView<uint>{}, inplace.view(), inplace.view(), bb.view(), eb.view(),
                                           4u);
    e.segmented_scan.InclusiveSegmentedSum(cmd, BufferView<uint>{}, inplace.view(), inplace.view(), BufferView<uint>{},
                                           BufferView<uint>{}, 0u);
    e.stream << xi.copy_from(luisa::span{x}) << bb.copy_from(luisa::span{b}) << eb.copy_from(luisa::span{en})
             << pb.copy_from(luisa::span{packed}) << ex.copy_from(luisa::span{sentinel})
             << in.copy_from(luisa::span{sentinel}) << ini.copy_from(luisa::span{sentinel})
             << pex.copy_from(luisa::span{sentinel}) << inplace.copy_from(luisa::span{x}) << cmd.commit() << synchronize();
    EXPECT((download(e, ex, 14) == std::vector<int>{S, 0, 1, 3, 0, 5, 11, S, 0, 9, 19, 30, S, S}));
    EXPECT((download(e, in, 14) == std::vector<int>{S, 1, 3, 6, 5, 11, 18, S, 9, 19, 30, 42, S, S}));
    EXPECT((download(e, ini, 14) == std::vector<int>{S, 11, 13, 16, 15, 21, 28, S, 19, 29, 40, 52, S, S}));
    EXPECT((download(e, pex, 14) == std::vector<int>{0, 1, 3, S, S, S, 0, 5, 11, S, 0, 9, 19, 30}));
    EXPECT((download(e, inplace, 14) == std::vector<int>{100, 1, 3, 6, 5, 11, 18, 200, 9, 19, 30, 42, 300, 400}));
}

// ---- segmented sorts ----------------------------------------------------------------------------

// Stable per-segment order of `keys` under `less`; items outside every segment map to UINT_MAX.
template <typename K, typename Less>
std::vector<uint> segment_order(const std::vector<K>& keys, const std::vector<uint>& b, const std::vector<uint>& en,
                                Less less) {
    std::vector<uint> order(keys.size(), std::numeric_limits<uint>::max());
    for (size_t s = 0; s < b.size(); ++s) {
        if (en[s] <= b[s]) continue;
        std::vector<uint> idx(en[s] - b[s]);
        std::iota(idx.begin(), idx.end(), b[s]);
        std::stable_sort(idx.begin(), idx.end(), [&](uint x, uint y) { return less(keys[x], keys[y]); });
        std::copy(idx.begin(), idx.end(), order.begin() + b[s]);
    }
    return order;
}

template <typename T>
bool matches_order(const std::vector<T>& got, const std::vector<T>& src, const std::vector<uint>& order, T sentinel) {
    for (size_t i = 0; i < got.size(); ++i) {
        const T want = order[i] == std::numeric_limits<uint>::max() ? sentinel : src[order[i]];
        if (std::memcmp(&got[i], &want, sizeof(T)) != 0) return false;
    }
    return true;
}

const std::vector<int> kSegKeys{91, 3, -2, 3, 92, 8, 1, 8, 4, 93, 5, -1, 5, 2, -1, 7, 2, 5, 0};
const std::vector<uint> kSegBegin{1u, 5u, 5u, 10u}, kSegEnd{4u, 5u, 9u, 19u};

// tests/device_segmented_sort_test.cpp:84-264: every copy-form entry point of DeviceSegmentedSort on
// the 19-item, 4-segment case (one empty segment, items outside every segment keep the sentinel).
void segmented_sort_all_entry_points() {
    auto& e = *g_env;
    constexpr uint n = 19u, m = 4u;
    constexpr int KS = -777;
    constexpr uint VS = std::numeric_limits<uint>::max();
    std::vector<uint> vals(n);
    std::iota(vals.begin(), vals.end(), 0u);
    const auto asc = segment_order(kSegKeys, kSegBegin, kSegEnd, std::less<>{});
    const auto desc = segment_order(kSegKeys, kSegBegin, kSegEnd, std::greater<>{});
    auto ki = e.device.create_buffer<int>(n);
    auto vi = e.device.create_buffer<uint>(n);
    auto bb = e.device.create_buffer<uint>(m), eb = e.device.create_buffer<uint>(m);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceSegmentedSort<>::GetSortPairsTempStorageBytes<int, uint>(n)));
    std::vector<Buffer<int>> ko;
    std::vector<Buffer<uint>> vo;
    for (int i = 0; i < 8; ++i) ko.push_back(e.device.create_buffer<int>(n));
    for (int i = 0; i < 4; ++i) vo.push_back(e.device.create_buffer<uint>(n));
    CommandList cmd;
    auto t = temp.view();
    e.segmented_sort.SortKeys(cmd, t, ki.view(), ko[0].view(), n, m, bb.view(), eb.view());
    e.segmented_sort.SortKeysDescending(cmd, t, ki.view(), ko[1].view(), n, m, bb.view(), eb.view());
    e.segmented_sort.StableSortKeys(cmd, t, ki.view(), ko[2].view(), n, m, bb.view(), eb.view());
    e.segmented_sort.StableSortKeysDescending(cmd, t, ki.view(), ko[3].view(), n, m, bb.view(), eb.view());
    e.segmented_sort.SortPairs(cmd, t, ki.view(), ko[4].view(), vi.view(), vo[0].view(), n, m, bb.view(), eb.view());
    e.segmented_sort.SortPairsDescending(cmd, t, ki.view(), ko[5].view(), vi.view(), vo[1].view(), n, m, bb.view(),
                                         eb.view());
    e.segmented_sort.StableSortPairs(cmd, t, ki.view(), ko[6].view(), vi.view(), vo[2].view(), n, m, bb.view(),
                                     eb.view());
    e.segmented_sort.StableSortPairsDescending(cmd, t, ki.view(), ko[7].view(), vi.view(), vo[3].view(), n, m,
                                               bb.view(), eb.view());
    const std::vector<int> kfill(n, KS);
    const std::vector<uint> vfill(n, VS);
    e.stream << ki.copy_from(luisa::span{kSegKeys}) << vi.copy_from(luisa::span{vals})
             << bb.copy_from(luisa::span{kSegBegin}) << eb.copy_from(luisa::span{kSegEnd});
    for (auto& b : ko) e.stream << b.copy_from(luisa::span{kfill});
    for (auto& b : vo) e.stream << b.copy_from(luisa::span{vfill});
    e.stream << cmd.commit() << synchronize();
    for (int i = 0; i < 8; ++i) EXPECT(matches_order(download(e, ko[i], n), kSegKeys, (i & 1) ? desc : asc, KS));
    for (int i = 0; i < 4; ++i) EXPECT(matches_order(download(e, vo[i], n), vals, (i & 1) ? desc : asc, VS));
    // Stability: the two 3s of segment 0 and the 8s of segment 2 keep their input order.
    EXPECT((download(e, vo[0], n)[2] == 1u && download(e, vo[0], n)[3] == 3u));
}

// tests/device_segmented_sort_test.cpp:266-435: DoubleBuffer forms; 19 items take ceil(log2 19) = 5
// merge passes, so the selector flips once (1 -> 0 for keys, 0 -> 1 for pairs) when the call is recorded.
void segmented_sort_double_buffers() {
    auto& e = *g_env;
    constexpr uint n = 19u, m = 4u;
    constexpr int KS = -777;
    constexpr uint VS = std::numeric_limits<uint>::max();
    std::vector<int> keys = kSegKeys;
    std::vector<uint> vals(n);
    std::iota(vals.begin(), vals.end(), 0u);
    for (uint i : {0u, 4u, 9u}) keys[i] = KS, vals[i] = VS;
    auto bb = e.device.create_buffer<uint>(m), eb = e.device.create_buffer<uint>(m);
    e.stream << bb.copy_from(luisa::span{kSegBegin}) << eb.copy_from(luisa::span{kSegEnd});
    const std::vector<int> kfill(n, KS);
    const std::vector<uint> vfill(n, VS);
    for (int desc = 0; desc < 2; ++desc) {
        const auto order = desc ? segment_order(keys, kSegBegin, kSegEnd, std::greater<>{})
                                : segment_order(keys, kSegBegin, kSegEnd, std::less<>{});
        auto k0 = e.device.create_buffer<int>(n), k1 = e.device.create_buffer<int>(n);
        DoubleBuffer<int> kb(k0.view(), k1.view());
        kb.selector = 1;
        CommandList cmd;
        if (desc) e.segmented_sort.StableSortKeysDescending(cmd, BufferView<uint>{}, kb, n, m, bb.view(), eb.view());
        else e.segmented_sort.SortKeys(cmd, BufferView<uint>{}, kb, n, m, bb.view(), eb.view());
        EXPECT(kb.selector == 0);
        e.stream << k0.copy_from(luisa::span{kfill}) << k1.copy_from(luisa::span{keys}) << cmd.commit()
                 << synchronize();
        EXPECT(matches_order(download(e, k0, n), keys, order, KS));

        auto pk0 = e.device.create_buffer<int>(n), pk1 = e.device.create_buffer<int>(n);
        auto pv0 = e.device.create_buffer<uint>(n), pv1 = e.device.create_buffer<uint>(n);
        DoubleBuffer<int> pk(pk0.view(), pk1.view());
        DoubleBuffer<uint> pv(pv0.view(), pv1.view());
        CommandList cmd2;
        if (desc) e.segmented_sort.SortPairsDescending(cmd2, BufferView<uint>{}, pk, pv, n, m, bb.view(), eb.view());
        else e.segmented_sort.StableSortPairs(cmd2, BufferView<uint>{}, pk, pv, n, m, bb.view(), eb.view());
        EXPECT(pk.selector == 1 && pv.selector == 1);
        e.stream << pk0.copy_from(luisa::span{keys}) << pk1.copy_from(luisa::span{kfill})
                 << pv0.copy_from(luisa::span{vals}) << pv1.copy_from(luisa::span{vfill}) << cmd2.commit()
                 << synchronize();
        EXPECT(matches_order(download(e, pk1, n), keys, order, KS));
        EXPECT(matches_order(download(e, pv1, n), vals, order, VS));
    }
}

// tests/device_segmented_sort_test.cpp:438-640: DeviceSegmentedRadixSort over bits [2, 6), copy and
// DoubleBuffer forms, keys and pairs, ascending and descending.
void segmented_radix_sort_partial_bits() {
    auto& e = *g_env;
    constexpr uint n = 19u, m = 4u, lo = 2u, hi = 6u;
    constexpr uint VS = std::numeric_limits<uint>::max();
    const std::vector<uint> keys{999u, 44u, 12u, 76u, 998u, 63u, 31u, 95u, 27u, 997u,
                                 84u, 20u, 52u, 16u, 80u, 48u, 24u, 56u, 4u};
    std::vector<uint> vals(n);
    std::iota(vals.begin(), vals.end(), 0u);
    auto field = [](uint k) { return (k >> lo) & ((1u << (hi - lo)) - 1u); };
    const auto asc = segment_order(keys, kSegBegin, kSegEnd, [&](uint x, uint y) { return field(x) < field(y); });
    const auto desc = segment_order(keys, kSegBegin, kSegEnd, [&](uint x, uint y) { return field(x) > field(y); });
    auto ki = e.device.create_buffer<uint>(n), vi = e.device.create_buffer<uint>(n);
    auto bb = e.device.create_buffer<uint>(m), eb = e.device.create_buffer<uint>(m);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceSegmentedRadixSort<>::GetSortPairsTempStorageBytes<uint, uint>(n)));
    std::vector<Buffer<uint>> out;
    for (int i = 0; i < 6; ++i) out.push_back(e.device.create_buffer<uint>(n));
    CommandList cmd;
    auto t = temp.view();
    e.segmented_radix_sort.SortKeys(cmd, t, ki.view(), out[0].view(), n, m, bb.view(), eb.view(), lo, hi);
    e.segmented_radix_sort.SortKeysDescending(cmd, t, ki.view(), out[1].view(), n, m, bb.view(), eb.view(), lo, hi);
    e.segmented_radix_sort.SortPairs(cmd, t, ki.view(), out[2].view(), vi.view(), out[3].view(), n, m, bb.view(),
                                     eb.view(), lo, hi);
    e.segmented_radix_sort.SortPairsDescending(cmd, t, ki.view(), out[4].view(), vi.view(), out[5].view(), n, m,
                                               bb.view(), eb.view(), lo, hi);
    const std::vector<uint> fill(n, VS);
    e.stream << ki.copy_from(luisa::span{keys}) << vi.copy_from(luisa::span{vals})
             << bb.copy_from(luisa::span{kSegBegin}) << eb.copy_from(luisa::span{kSegEnd});
    for (auto& b : out) e.stream << b.copy_from(luisa::span{fill});
    e.stream << cmd.commit() << synchronize();
    EXPECT(matches_order(download(e, out[0], n), keys, asc, VS));
    EXPECT(matches_order(download(e, out[1], n), keys, desc, VS));
    EXPECT(matches_order(download(e, out[2], n), keys, asc, VS));
    EXPECT(matches_order(download(e, out[3], n), vals, asc, VS));
    EXPECT(matches_order(download(e, out[4], n), keys, desc, VS));
    EXPECT(matches_order(download(e, out[5], n), vals, desc, VS));

    // DoubleBuffer forms start from selector 0 and 1 (the reference's :556-640).
    std::vector<uint> dkeys = keys, dvals = vals;
    for (uint i : {0u, 4u, 9u}) dkeys[i] = VS, dvals[i] = VS;
    const auto dasc = segment_order(dkeys, kSegBegin, kSegEnd, [&](uint x, uint y) { return field(x) < field(y); });
    for (int sel = 0; sel < 2; ++sel) {
        auto a0 = e.device.create_buffer<uint>(n), a1 = e.device.create_buffer<uint>(n);
        auto b0 = e.device.create_buffer<uint>(n), b1 = e.device.create_buffer<uint>(n);
        DoubleBuffer<uint> kb(a0.view(), a1.view()), vb(b0.view(), b1.view());
        kb.selector = vb.selector = sel;
        CommandList c2;
        e.segmented_radix_sort.SortPairs(c2, BufferView<uint>{}, kb, vb, n, m, bb.view(), eb.view(), lo, hi);
        EXPECT(kb.selector == (sel ^ 1) && vb.selector == kb.selector);
        e.stream << (sel ? a1 : a0).copy_from(luisa::span{dkeys}) << (sel ? a0 : a1).copy_from(luisa::span{fill})
                 << (sel ? b1 : b0).copy_from(luisa::span{dvals}) << (sel ? b0 : b1).copy_from(luisa::span{fill})
                 << c2.commit() << synchronize();
        EXPECT(matches_order(download(e, sel ? a0 : a1, n), dkeys, dasc, VS));
        EXPECT(matches_order(download(e, sel ? b0 : b1, n), dvals, dasc, VS));
    }
}

// tests/device_segmented_sort_test.cpp:700-790: empty work, temp sizes of one item, signed keys over
// the full width, and zero-width sorts (copy form copies, DoubleBuffer form keeps its selector).
void segmented_sort_empty_signed_zero_width() {
    auto& e = *g_env;
    CommandList empty;
    e.segmented_sort.SortKeys(empty, BufferView<uint>{}, BufferView<int>{}, BufferView<int>{}, 0u, 0u,
                              BufferView<uint>{}, BufferView<uint>{});
    e.segmented_radix_sort.SortKeys(empty, BufferView<uint>{}, BufferView<uint>{}, BufferView<uint>{}, 0u, 0u,
                                    BufferView<uint>{}, BufferView<uint>{});
    EXPECT(empty.empty());
    EXPECT(DeviceSegmentedSort<>::GetSortKeysTempStorageBytes<int>(1u) == 0u);
    EXPECT(DeviceSegmentedRadixSort<>::GetSortKeysTempStorageBytes<uint>(1u) == 0u);
    // Temp layout of the reference (device_segmented_sort.h:49-75): keys, then values at their alignment.
    EXPECT((DeviceSegmentedSort<>::GetSortKeysTempStorageBytes<int>(1000u) == 4000u));
    EXPECT((DeviceSegmentedSort<>::GetSortPairsTempStorageBytes<int, double>(1001u) == 4008u + 8008u));

    constexpr uint n = 8u;
    const std::vector<int> keys{41, -7, 3, -7, 0, 22, -1, 3};
    std::vector<uint> vals(n);
    std::iota(vals.begin(), vals.end(), 0u);
    std::vector<int> sorted = keys;
    std::stable_sort(sorted.begin(), sorted.end());
    auto ki = e.device.create_buffer<int>(n), sk = e.device.create_buffer<int>(n), zk = e.device.create_buffer<int>(n);
    auto vi = e.device.create_buffer<uint>(n), zv = e.device.create_buffer<uint>(n);
    auto d0 = e.device.create_buffer<int>(n), d1 = e.device.create_buffer<int>(n);
    auto bb = e.device.create_buffer<uint>(1), eb = e.device.create_buffer<uint>(1);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceSegmentedRadixSort<>::GetSortPairsTempStorageBytes<int, uint>(n)));
    DoubleBuffer<int> db(d0.view(), d1.view());
    db.selector = 1;
    CommandList cmd;
    e.segmented_radix_sort.SortKeys(cmd, temp.view(), ki.view(), sk.view(), n, 1u, bb.view(), eb.view());
    e.segmented_radix_sort.SortPairs(cmd, temp.view(), ki.view(), zk.view(), vi.view(), zv.view(), n, 1u, bb.view(),
                                     eb.view(), 13u, 13u);
    e.segmented_radix_sort.SortKeys(cmd, temp.view(), db, n, 1u, bb.view(), eb.view(), 13u, 13u);
    EXPECT(db.selector == 1);
    const uint b0 = 0u, e0 = n;
    const std::vector<int> fill(n, -777);
    e.stream << ki.copy_from(luisa::span{keys}) << vi.copy_from(luisa::span{vals}) << d0.copy_from(luisa::span{fill})
             << d1.copy_from(luisa::span{keys}) << bb.copy_from(luisa::span{&b0, 1u})
             << eb.copy_from(luisa::span{&e0, 1u}) << cmd.commit() << synchronize();
    EXPECT(download(e, sk, n) == sorted);
    EXPECT(download(e, zk, n) == keys);
    EXPECT(download(e, zv, n) == vals);
    EXPECT(download(e, d1, n) == keys);
}

// Larger inputs: 300,000 float keys (many ties, both zero signs) in 500 random segments, one of them
// 70,000 items long (global merge passes); value order (DeviceSegmentedSort, -0.0 == +0.0) and radix
// order (DeviceSegmentedRadixSort, -0.0 before +0.0) against std::stable_sort per segment.
void segmented_sort_large_float_keys() {
    auto& e = *g_env;
    constexpr uint n = 300000u, m = 500u;
    std::vector<float> keys(n);
    for (uint i = 0; i < n; ++i) {
        keys[i] = static_cast<float>(static_cast<int>(mix64(77, i) % 601u) - 300) / 8.0f;
        if (keys[i] == 0.0f && (mix64(79, i) & 1u)) keys[i] = -0.0f;
    }
    std::vector<uint> cuts;
    for (uint s = 1; s < m; ++s) cuts.push_back(static_cast<uint>(mix64(78, s) % n));
    cuts.push_back(70000u);
    std::sort(cuts.begin(), cuts.end());
    cuts.erase(std::unique(cuts.begin(), cuts.end()), cuts.end());
    // Segments: [0, 70000), then the random cuts above 70000 (contiguous up to n).
    std::vector<uint> b2{0u}, e2{70000u};
    for (uint c : cuts)
        if (c > 70000u) e2.push_back(c), b2.push_back(c);
    b2.insert(b2.begin() + 1, 70000u);
    e2.push_back(n);
    const uint segs = static_cast<uint>(b2.size());
    std::vector<uint> vals(n);
    std::iota(vals.begin(), vals.end(), 0u);
    auto bits = [](float f) {
        uint u;
        std::memcpy(&u, &f, 4);
        return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    };
    const auto vorder = segment_order(keys, b2, e2, std::less<>{});
    const auto rorder = segment_order(keys, b2, e2, [&](float x, float y) { return bits(x) > bits(y); });
    auto ki = e.device.create_buffer<float>(n), k1 = e.device.create_buffer<float>(n);
    auto k2 = e.device.create_buffer<float>(n);
    auto vi = e.device.create_buffer<uint>(n), v1 = e.device.create_buffer<uint>(n);
    auto bb = e.device.create_buffer<uint>(segs), eb = e.device.create_buffer<uint>(segs);
    auto temp = e.device.create_buffer<uint>(
        bytes_to_uint_count(DeviceSegmentedSort<>::GetSortPairsTempStorageBytes<float, uint>(n)));
    CommandList cmd;
    e.segmented_sort.SortPairs(cmd, temp.view(), ki.view(), k1.view(), vi.view(), v1.view(), n, segs, bb.view(),
                               eb.view());
    e.segmented_radix_sort.SortKeysDescending(cmd, temp.view(), ki.view(), k2.view(), n, segs, bb.view(), eb.view());
    e.stream << ki.copy_from(luisa::span{keys}) << vi.copy_from(luisa::span{vals}) << bb.copy_from(luisa::span{b2})
             << eb.copy_from(luisa::span{e2}) << cmd.commit() << synchronize();
    EXPECT(matches_order(download(e, k1, n), keys, vorder, 0.0f));
    EXPECT(matches_order(download(e, v1, n), vals, vorder, 0u));
    EXPECT(matches_order(download(e, k2, n), keys, rorder, 0.0f));
}

// ---- record-time checks ------------------------------------------------------------------------

void precondition_errors() {
    auto& e = *g_env;
    const uint n = 100000u;
    auto a = e.device.create_buffer<uint>(n);
    auto small = e.device.create_buffer<uint>(2);
    CommandList cmd;
    EXPECT(throws_error([&] { e.scan.ExclusiveSum(cmd, small.view(), a.view(), a.view(), n); }));
    EXPECT(throws_error([&] { e.reduce.Sum(cmd, small.view(), a.view(), a.view(), n); }));
    EXPECT(throws_error([&] { e.scan.ExclusiveSumByKey(cmd, small.view(), a.view(), a.view(), a.view(), n); }));
    EXPECT(throws_error([&] { e.select.Flagged(cmd, small.view(), a.view(), a.view(), a.view(), small.view(), n); }));
    EXPECT(throws_error([&] {
        e.partition.If(cmd, small.view(), a.view(), a.view(), small.view(), n, ItemPredicate<uint>::less(3u));
    }));
    EXPECT(throws_error([&] { e.rle.Encode(cmd, small.view(), a.view(), a.view(), a.view(), small.view(), n); }));
    DeviceSelect<> no_select;
    EXPECT(throws_error([&] { no_select.Unique(cmd, small.view(), a.view(), small.view(), 1u); }));
    EXPECT(throws_error(
        [&] { e.reduce.ReduceByKey(cmd, small.view(), a.view(), a.view(), a.view(), a.view(), small.view(), SumOp{}, n); }));
    EXPECT(throws_error([&] {
        e.reduce.ReduceByKey(cmd, small.view(), a.view(), a.view(), a.view(), a.view(), BufferView<uint>{}, SumOp{}, 0u);
    }));
    EXPECT(throws_error([&] { e.radix_sort.SortKeys(cmd, small.view(), a.view(), a.view(), n); }));
    EXPECT(throws_error([&] { e.radix_sort.SortKeys(cmd, small.view(), a.view(), a.view(), 4u, 5u, 3u); }));
    EXPECT(throws_error([&] { e.radix_sort.SortKeys(cmd, small.view(), a.view(), a.view(), 4u, 0u, 33u); }));
    EXPECT(throws_error([&] { e.scan.ExclusiveSum(cmd, small.view(), a.view(), a.view(), n + 1u); }));
    DeviceScan<> not_created;
    EXPECT(throws_error([&] { not_created.ExclusiveSum(cmd, small.view(), a.view(), a.view(), 1u); }));
    DoubleBuffer<uint> bad(a.view(), a.view());
    bad.selector = 2;
    EXPECT(throws_error([&] { e.radix_sort.SortKeys(cmd, small.view(), bad, 4u); }));
    EXPECT(throws_error([&] {
        e.segmented_radix_sort.SortKeys(cmd, small.view(), a.view(), a.view(), 4u, 1u, small.view(), small.view(), 5u, 4u);
    }));
    EXPECT(throws_error([&] {
        e.segmented_sort.SortKeys(cmd, small.view(), a.view(), a.view(), n, 1u, small.view(), small.view());
    }));
    EXPECT(throws_error([&] {
        e.segmented_sort.SortKeys(cmd, small.view(), a.view(), a.view(), 4u, 3u, small.view(), small.view());
    }));
    DeviceSegmentedSort<> no_segsort;
    EXPECT(throws_error([&] {
        no_segsort.SortKeys(cmd, small.view(), a.view(), a.view(), 1u, 1u, small.view(), small.view());
    }));
    EXPECT(cmd.empty());  // nothing was recorded by a rejected call
}

const std::vector<Case>& cases() {
    static const std::vector<Case> all{
        {"reduce_sum_of_ones", reduce_sum_of_ones},
        {"reduce_empty_writes_init", reduce_empty_writes_init},
        {"reduce_bench_pattern_int_and_float", reduce_bench_pattern_int_and_float},
        {"reduce_min_max_and_arg", reduce_min_max_and_arg},
        {"reduce_with_operator_and_transform", reduce_with_operator_and_transform},
        {"scan_sums_of_ones", scan_sums_of_ones},
        {"scan_inclusive_init_in_place", scan_inclusive_init_in_place},
        {"scan_double_inclusive_sum", scan_double_inclusive_sum},
        {"scan_int64_exclusive_vs_std", scan_int64_exclusive_vs_std},
        {"scan_min_max_operators", scan_min_max_operators},
        {"scan_bench_pattern_vs_std", scan_bench_pattern_vs_std},
        {"radix_stable_partial_bit_ranges", radix_stable_partial_bit_ranges},
        {"radix_zero_width_copies", radix_zero_width_copies},
        {"radix_empty_input", radix_empty_input},
        {"radix_double_buffer_selectors", radix_double_buffer_selectors},
        {"radix_double_buffer_zero_width_keeps_current", radix_double_buffer_zero_width_keeps_current},
        {"radix_large_keys_and_pairs", radix_large_keys_and_pairs},
        {"radix_float_and_signed_keys", radix_float_and_signed_keys},
        {"scan_exclusive_sum_by_key_segments_of_100", scan_exclusive_sum_by_key_segments_of_100},
        {"scan_inclusive_sum_by_key_three_tiles_int64", scan_inclusive_sum_by_key_three_tiles_int64},
        {"scan_by_key_custom_equality", scan_by_key_custom_equality},
        {"scan_by_key_initial_values_float_in_place", scan_by_key_initial_values_float_in_place},
        {"reduce_by_key_segments_of_100", reduce_by_key_segments_of_100},
        {"reduce_by_key_empty_input", reduce_by_key_empty_input},
        {"by_key_min_max", by_key_min_max},
        {"select_flagged_and_if_are_stable", select_flagged_and_if_are_stable},
        {"select_unique_by_key_and_flagged_if", select_unique_by_key_and_flagged_if},
        {"select_in_place_forms", select_in_place_forms},
        {"partition_ordering_and_three_way", partition_ordering_and_three_way},
        {"run_length_encode_examples", run_length_encode_examples},
        {"segment_reduce_known_answers", segment_reduce_known_answers},
        {"segmented_scan_known_answers", segmented_scan_known_answers},
        {"segmented_sort_all_entry_points", segmented_sort_all_entry_points},
        {"segmented_sort_double_buffers", segmented_sort_double_buffers},
        {"segmented_radix_sort_partial_bits", segmented_radix_sort_partial_bits},
        {"segmented_sort_empty_signed_zero_width", segmented_sort_empty_signed_zero_width},
        {"segmented_sort_large_float_keys", segmented_sort_large_float_keys},
        {"spmv_float_unsigned_indices", spmv_float_unsigned_indices},
        {"spmv_int_values_and_empty_work", spmv_int_values_and_empty_work},
        {"precondition_errors", precondition_errors},
    };
    return all;
}

}  // namespace

int main(int argc, char** argv) {
    const char* filter = nullptr;
    for (int i = 1; i < argc; ++i) {
        if (std::strcmp(argv[i], "--list") == 0) {
            for (const auto& c : cases()) std::printf("%s\n", c.name);
            return 0;
        }
        filter = argv[i];
    }
    Env env;
    g_env = &env;
    int run = 0;
    for (const auto& c : cases()) {
        if (filter && !std::strstr(c.name, filter)) continue;
        g_current = c.name;
        std::printf("case %s\n", c.name);
        std::fflush(stdout);
        const int before = g_failures;
        try {
            c.body();
        } catch (const std::exception& ex) {
            ++g_failures;
            std::printf("  FAILED %s: exception %s\n", c.name, ex.what());
        }
        std::printf("  %s\n", g_failures == before ? "ok" : "FAILED");
        std::fflush(stdout);
        ++run;
    }
    std::printf("%d cases, %d failures\n", run, g_failures);
    return g_failures == 0 && run > 0 ? 0 : 1;
}
