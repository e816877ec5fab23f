"""Temp-storage contract: the C-ABI returns the reference's Get*TempStorageBytes values, and the HIP
kernels never carve more than that.  Known answers are the byte counts of the reference formulas
evaluated by hand at the benchmark sizes (device_reduce.h:517-536, device_scan.h:295-308,
device_radix_sort.h:267-362, device_spmv.h:43-46)."""
import pytest


def test_reduce_temp_known_answers(hip):
    # 2^24 int32, tile 256x8 = 2048: levels of 8192, 4 and 1 partials:
    # 8192*4 = 32768; +4*4 = 32784; align to 256 -> 33024; +1*4 = 33028.
    assert hip.reduce_temp_bytes(1 << 24, 4) == 33028
    # 2^28: 131072*4 = 524288; +64*4 = 524544; align -> 524544; +4 = 524548.
    assert hip.reduce_temp_bytes(1 << 28, 4) == 524548
    for n in (0, 1, 2047, 2048):
        assert hip.reduce_temp_bytes(n, 4) == 4  # a single block writes one partial
    assert hip.reduce_temp_bytes(2049, 4) == 256 + 4  # 2 partials (8 B), align to 256, + 1 partial
    assert hip.reduce_temp_bytes(2049, 8) == 256 + 8


def test_scan_temp_known_answers(hip):
    # 2^28 u32, 256x15 tiles: 69906 tiles + 32 pad = 69938 entries x (4 + 4 + 4) with 256-byte alignment.
    assert hip.scan_temp_bytes(1 << 28, 4) == 839368
    # 1 item: 33 entries -> 132 | 256 + 132 | 512 + 132 = 644 vs packed 33*8 = 264 -> 644.
    assert hip.scan_temp_bytes(1, 4) == 644
    # packed 320x25 layout alone (CUDA policy) at 2^28: 33555 + 32 tiles x 8 -> 268696 -> 268800.
    assert hip.lib().lcpp_hip_scan_temp_bytes_policy(1 << 28, 4, 320, 25, 0, 1) == 268800


def test_radix_temp_known_answers(hip):
    # SortKeys 2^28 u32: the conservative 256x16 tile dominates: 2,214,601,728 B.
    assert hip.sort_keys_temp_bytes(1 << 28, 4) == 2214601728
    # SortPairs 2^27 u64 keys + u32 values: tile 256x8: 1,677,731,840 B.
    assert hip.sort_pairs_temp_bytes(1 << 27, 8, 4) == 1677731840
    # tests/device_radix_sort_interface_test.cpp:197-203: GetSortKeysTempStorageBytes(0) == 0.
    assert hip.sort_keys_temp_bytes(0, 4) == 0
    assert hip.sort_pairs_temp_bytes(0, 4, 4) == 0


def test_spmv_temp_is_zero(hip):
    # tests/device_spmv_test.cpp:157-172.
    assert hip.lib().lcpp_hip_spmv_temp_bytes(0, 0, 0) == 0
    assert hip.lib().lcpp_hip_spmv_temp_bytes(1 << 20, 1 << 20, 1 << 25) == 0


SIZES = [1, 2, 63, 64, 255, 256, 257, 1000, 2047, 2048, 2049, 3839, 3840, 3841, 4095, 4096, 4097, 7679, 7680,
         7681, 8191, 8192, 8193, 65535, 65536, 65537, 1000003, 1 << 20, (1 << 24) + 1, 1 << 27, (1 << 28) - 1,
         1 << 28, (1 << 28) + 4096, 3 << 28, 1 << 30, (1 << 31) + 12345, (1 << 32) - 1]


@pytest.mark.parametrize("n", SIZES)
def test_scan_needs_fit_reference_temp(hip, n):
    for eb in (4, 8):
        assert hip.lib().lcpp_hip_internal_scan_needed_bytes(n, eb) <= hip.scan_temp_bytes(n, eb)


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("kb,vb", [(4, 0), (8, 0), (4, 4), (8, 4), (4, 8), (8, 8)])
@pytest.mark.parametrize("double_buffer", [0, 1])
def test_radix_needs_fit_reference_temp(hip, n, kb, vb, double_buffer):
    lib = hip.lib()
    ref = hip.sort_keys_temp_bytes(n, kb) if vb == 0 else hip.sort_pairs_temp_bytes(n, kb, vb)
    for begin, end in ((0, kb * 8), (0, 8), (3, 17), (kb * 8 - 1, kb * 8)):
        assert lib.lcpp_hip_internal_radix_needed_bytes(n, kb, vb, begin, end, double_buffer) <= ref


def test_radix_forced_small_portions_report_their_needs(hip):
    """The portion-limit knob (a test hook for the multi-portion carry) may need more bins than the
    reference formula reserves; the needed-bytes query reports the actual requirement."""
    lib = hip.lib()
    tile = lib.lcpp_hip_radix_tile_items(4, 0)
    try:
        lib.lcpp_hip_radix_set_portion_limit(tile * 3)
        n = tile * 10 + 17
        need = lib.lcpp_hip_internal_radix_needed_bytes(n, 4, 0, 0, 32, 0)
        assert lib.lcpp_hip_internal_radix_portions(n, 4, 0, 0, 32, 0, need) == 4
        assert lib.lcpp_hip_internal_radix_portions(n, 4, 0, 0, 32, 0, need - 1) == 0
    finally:
        lib.lcpp_hip_radix_set_portion_limit(0)


def test_radix_single_portion_at_benchmark_sizes(hip):
    """With reference-sized temp storage, the 2^28-key SortKeys and the 2^27-pair SortPairs each run as
    one onesweep portion per pass (the reference needs two portions for 2^28 keys)."""
    lib = hip.lib()
    n = 1 << 28
    assert lib.lcpp_hip_internal_radix_portions(n, 4, 0, 0, 32, 0, hip.sort_keys_temp_bytes(n, 4)) == 1
    n = 1 << 27
    assert lib.lcpp_hip_internal_radix_portions(n, 8, 4, 0, 64, 0, hip.sort_pairs_temp_bytes(n, 8, 4)) == 1
    # Above 2^30 keys the sort always splits into portions, and reference-sized temp always suffices.
    for n, kb, vb in ((3 << 28, 4, 4), ((1 << 32) - 1, 4, 0), ((1 << 31) + 5, 8, 4)):
        ref = hip.sort_keys_temp_bytes(n, kb) if vb == 0 else hip.sort_pairs_temp_bytes(n, kb, vb)
        portions = lib.lcpp_hip_internal_radix_portions(n, kb, vb, 0, kb * 8, 0, ref)
        assert portions >= (2 if n >= (1 << 30) else 1)


def test_by_key_temp_bytes_known_values(hip):
    """GetScanByKeyTempStorageBytes (device_scan.h:129-142, 310-315) and GetReduceByKeyTempStorageBytes
    (device_reduce.h:207-223) worked by hand.
    scan, n = 10000, int32 keys and values: tiles = ceil(10000 / 3840) = 3, tile_count = 35:
      35*4 = 140 -> 256; + 35*8 = 280 -> 536 -> 768; + 280 -> 1048 -> 1280; + 3*4 = 12 -> 1292.
    scan, n = 10000, int32 keys, int64 values: pairs of 16 B: 256 + 560 = 816 -> 1024 + 560 = 1584 -> 1792 + 12 = 1804.
    reduce, n = 10000, int32 / int32: tiles = ceil(10000 / 1024) = 10, tile_count = 42:
      168 -> 256; + 336 = 592 -> 768; + 336 = 1104.
    n = 0 still reserves one tile (max(1, ...))."""
    lib = hip.lib()
    assert lib.lcpp_hip_scan_by_key_temp_bytes(10000, 4, 4) == 1292
    assert lib.lcpp_hip_scan_by_key_temp_bytes(10000, 4, 8) == 1804
    assert lib.lcpp_hip_reduce_by_key_temp_bytes(10000, 4, 4) == 1104
    assert lib.lcpp_hip_scan_by_key_temp_bytes(0, 4, 4) == lib.lcpp_hip_scan_by_key_temp_bytes(1, 4, 4)
    assert lib.lcpp_hip_reduce_by_key_temp_bytes(0, 4, 4) == lib.lcpp_hip_reduce_by_key_temp_bytes(1024, 4, 4)


@pytest.mark.parametrize("kb,vb", [(4, 4), (4, 8), (8, 4), (8, 8)])
def test_by_key_kernels_fit_reference_temp(hip, kb, vb):
    """The by-key kernels carve at most what the reference formulas return, for every size."""
    lib = hip.lib()
    sizes = list(range(0, 50000, 61)) + [1 << 20, (1 << 24) + 1, 1 << 28, (1 << 32) - 1]
    for n in sizes:
        need = lib.lcpp_hip_internal_by_key_needed_bytes(n, vb)
        assert need <= lib.lcpp_hip_scan_by_key_temp_bytes(n, kb, vb)
        assert need <= lib.lcpp_hip_reduce_by_key_temp_bytes(n, kb, vb)


def test_by_key_temp_bytes_policies(hip):
    """Policy queries: the default tiles reproduce the default queries; a smaller tile gives the
    reference formula (DeviceScan<128, 32, 8>, n = 10000: tiles = ceil(10000 / 1024) = 10,
    tile_count = 42: 168 -> 256; + 336 = 592 -> 768; + 336 = 1104 -> 1280; + 40 = 1320;
    DeviceReduce<128>: tiles = ceil(10000 / 512) = 20, tile_count = 52: 208 -> 256; + 416 = 672 -> 768;
    + 416 = 1184); tiles so large that the reference layout is smaller than the kernel's tile states
    are raised to the kernel's need."""
    lib = hip.lib()
    for n in (0, 1, 3840, 10000, 1 << 20, (1 << 32) - 1):
        for kb, vb in ((4, 4), (8, 8), (4, 8)):
            assert lib.lcpp_hip_scan_by_key_temp_bytes_policy(n, kb, vb, 256, 15) == \
                lib.lcpp_hip_scan_by_key_temp_bytes(n, kb, vb)
            assert lib.lcpp_hip_reduce_by_key_temp_bytes_policy(n, kb, vb, 256) == \
                lib.lcpp_hip_reduce_by_key_temp_bytes(n, kb, vb)
    assert lib.lcpp_hip_scan_by_key_temp_bytes_policy(10000, 4, 4, 128, 8) == 1320
    assert lib.lcpp_hip_reduce_by_key_temp_bytes_policy(10000, 4, 4, 128) == 1184
    for n in (1 << 20, (1 << 28) + 5):
        need = lib.lcpp_hip_internal_by_key_needed_bytes(n, 8)
        assert lib.lcpp_hip_scan_by_key_temp_bytes_policy(n, 4, 8, 1024, 64) == need
        assert lib.lcpp_hip_reduce_by_key_temp_bytes_policy(n, 4, 8, 8192) == need
    assert lib.lcpp_hip_scan_by_key_temp_bytes_policy(100, 4, 4, 0, 15) == 0


def test_compaction_temp_bytes_known_values(hip):
    """DeviceSelect / DevicePartition / DeviceRunLengthEncode temp queries worked by hand
    (device_select.h:56-63, device_partition.h:55-71, device_run_length_encode.h:56-69) at n = 1000 with
    the default DeviceScan<256, 32, 4> scan: tiles = ceil(1000 / 1024) = 1, tile_count = 33:
      scan = 132 -> 256; + 132 = 388 -> 512; + 132 = 644 bytes;
      select = 8 * 1000 + 644 = 8644; three-way = 12 * 1000 + 644 = 12644;
      run-length encode = align256(4 * 6001 = 24004) = 24064 + 644 = 24708.  n = 0 needs nothing."""
    lib = hip.lib()
    assert lib.lcpp_hip_select_temp_bytes(1000) == 8644
    assert lib.lcpp_hip_partition_three_way_temp_bytes(1000) == 12644
    assert lib.lcpp_hip_run_length_encode_temp_bytes(1000) == 24708
    for f in ("select", "partition_three_way", "run_length_encode"):
        assert getattr(lib, f"lcpp_hip_{f}_temp_bytes")(0) == 0
    # DeviceSelect<256, 32, 15> uses the default scan policy, which reserves the packed 320 x 25 layout too.
    assert lib.lcpp_hip_select_temp_bytes_policy(1000, 256, 15) == 8000 + lib.lcpp_hip_scan_temp_bytes(1000, 4)


def test_compaction_kernels_fit_reference_temp(hip):
    """The compaction kernels carve at most what the reference formulas return, for every size: one
    state word (select, unique) or two (three-way, run-length) per tile, plus n items of staging
    (in-place selects, the three-way partition, in-place encode)."""
    lib = hip.lib()
    sizes = list(range(1, 60000, 97)) + [1 << 20, (1 << 24) + 3, 1 << 28, (1 << 32) - 1]
    for n in sizes:
        sel = lib.lcpp_hip_select_temp_bytes(n)
        three = lib.lcpp_hip_partition_three_way_temp_bytes(n)
        rle = lib.lcpp_hip_run_length_encode_temp_bytes(n)
        for item in (4, 8):
            assert lib.lcpp_hip_internal_compact_needed_bytes(n, item, 1, 1) <= sel
            assert lib.lcpp_hip_internal_compact_needed_bytes(n, item, 2, 1) <= three
            assert lib.lcpp_hip_internal_compact_needed_bytes(n, item, 2, 1) <= rle
    # Large-tile policies are raised to the kernels' need.
    n = 1 << 24
    assert lib.lcpp_hip_select_temp_bytes_policy(n, 1024, 64) >= lib.lcpp_hip_internal_compact_needed_bytes(n, 8, 1, 1)
