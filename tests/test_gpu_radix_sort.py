"""Onesweep DeviceRadixSort on the GPU vs the oracle (bit-exact keys and values, stable).

Cases follow the reference tests: float keys 2^5..2^24 asc/desc (tests/device_radix_sort_one_sweep.cpp:
79-136), reversed uint keys (:138-173), 65,536 u64 keys (n-i-1)*2654435761 (:175-205), shuffled-iota
pairs asc/desc (:207-333), the stable partial bit range [1,6) on 257 items, zero-width copy, empty
input and DoubleBuffer selector flips (tests/device_radix_sort_interface_test.cpp:68-283), plus the
benchmark inputs: 2^28 uniform u32 keys and 2^27 u64/u32 pairs with uniform and AND-of-3 keys.
"""
import numpy as np
import pytest
import torch

from gpu_util import empty_dev, fill_dev, log, to_dev, to_host

pytestmark = pytest.mark.gpu

SUFFIX = {np.dtype(np.uint32): "u32", np.dtype(np.int32): "i32", np.dtype(np.float32): "f32",
          np.dtype(np.uint64): "u64", np.dtype(np.int64): "i64", np.dtype(np.float64): "f64"}


def gpu_sort(hip, keys, values=None, begin_bit=0, end_bit=None, descending=False):
    n = keys.size
    sfx = SUFFIX[keys.dtype]
    kin = to_dev(keys)
    kout = fill_dev(n, keys.dtype.itemsize, -1)
    if values is None:
        hip.sort_keys(sfx, kin, kout, n, begin_bit, end_bit, descending)
        check_bits(to_host(kin, keys.dtype, n), keys)  # the copy form never writes its input
        return to_host(kout, keys.dtype, n)
    vin = to_dev(values)
    vout = fill_dev(n, values.dtype.itemsize, -1)
    hip.sort_pairs(sfx, values.dtype.itemsize, kin, kout, vin, vout, n, begin_bit, end_bit, descending)
    check_bits(to_host(kin, keys.dtype, n), keys)
    check_bits(to_host(vin, values.dtype, n), values)
    return to_host(kout, keys.dtype, n), to_host(vout, values.dtype, n)


def check_bits(got, exp):
    assert got.dtype == exp.dtype
    assert np.array_equal(got.view(f"u{got.dtype.itemsize}"), exp.view(f"u{exp.dtype.itemsize}"))


@pytest.mark.parametrize("k", [0, 1, 5, 8, 11, 12, 13, 16, 20, 23])
def test_reversed_uint_keys(hip, orc, dev, k):
    n = 1 << k
    log(f"sort reversed n={n}")
    keys = np.arange(n, dtype=np.uint32)[::-1].copy()
    check_bits(gpu_sort(hip, keys), np.arange(n, dtype=np.uint32))


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 255, 256, 257, 4095, 4096, 4097, 8191, 8193, 65537, 1000003])
def test_random_u32_sizes(hip, orc, dev, n):
    keys = orc.generate(1, n, 1000 + n)
    log(f"sort u32 n={n}")
    check_bits(gpu_sort(hip, keys), orc.radix_sort(keys))


@pytest.mark.parametrize("k", [5, 10, 16, 20])
@pytest.mark.parametrize("descending", [False, True])
def test_float_keys(hip, orc, dev, k, descending):
    n = 1 << k
    keys = (orc.generate(6, n, k) * 1000.0).astype(np.float32)
    keys[::9] = 0.0
    keys[1::13] = -0.0
    check_bits(gpu_sort(hip, keys, descending=descending), orc.radix_sort(keys, descending=descending))


def test_float_special_values_pairs(hip, orc, dev):
    import struct
    neg_nan = struct.unpack("<f", struct.pack("<I", 0xFFC00000))[0]
    pos_nan = struct.unpack("<f", struct.pack("<I", 0x7FC00000))[0]
    keys = np.array([1.5, -0.0, 0.0, -2.0, np.inf, pos_nan, -0.0, -np.inf, neg_nan, 0.0, -1e-30], np.float32)
    vals = np.arange(keys.size, dtype=np.uint32)
    for desc in (False, True):
        ko, vo = gpu_sort(hip, keys, vals, descending=desc)
        eko, evo = orc.radix_sort(keys, vals, descending=desc)
        check_bits(ko, eko)
        assert np.array_equal(vo, evo)


def test_u64_reversed_known_answer(hip, orc, dev):
    n = 65536
    keys = ((n - np.arange(n, dtype=np.uint64) - 1) * np.uint64(2654435761)).astype(np.uint64)
    check_bits(gpu_sort(hip, keys), np.sort(keys))


@pytest.mark.parametrize("dtype", [np.int32, np.int64, np.float64, np.uint64])
@pytest.mark.parametrize("descending", [False, True])
def test_other_key_types(hip, orc, dev, dtype, descending):
    n = 300007
    raw = orc.generate(0, n, 77)
    if np.dtype(dtype).itemsize == 4:
        keys = (raw >> np.uint64(32)).astype(np.uint32).view(dtype)
    elif dtype == np.float64:
        keys = orc.generate(6, n, 78).astype(np.float64) * 1e3
    else:
        keys = raw.view(dtype)
    keys = keys.copy()
    keys[::17] = keys[5]
    vals = np.arange(n, dtype=np.uint32)
    ko, vo = gpu_sort(hip, keys, vals, descending=descending)
    eko, evo = orc.radix_sort(keys, vals, descending=descending)
    check_bits(ko, eko)
    assert np.array_equal(vo, evo)


@pytest.mark.parametrize("descending", [False, True])
def test_shuffled_iota_pairs(hip, orc, dev, descending):
    n = 524288
    keys = np.random.default_rng(114521).permutation(n).astype(np.uint32)
    vals = keys.copy()
    ko, vo = gpu_sort(hip, keys, vals, descending=descending)
    exp = np.arange(n, dtype=np.uint32)
    if descending:
        exp = exp[::-1]
    assert np.array_equal(ko, exp) and np.array_equal(vo, exp)


def test_partial_bits_known_answer(hip, orc, dev):
    n, b, e = 257, 1, 6
    keys = np.array([((i * 53) % 64) | (((i * 17) % 11) << 8) for i in range(n)], np.uint32)
    vals = np.arange(n, dtype=np.uint32)
    sel = lambda k: (int(k) >> b) & ((1 << (e - b)) - 1)
    asc = sorted(range(n), key=lambda i: sel(keys[i]))
    desc = sorted(range(n), key=lambda i: -sel(keys[i]))
    assert np.array_equal(gpu_sort(hip, keys, begin_bit=b, end_bit=e), keys[asc])
    assert np.array_equal(gpu_sort(hip, keys, begin_bit=b, end_bit=e, descending=True), keys[desc])
    ko, vo = gpu_sort(hip, keys, vals, begin_bit=b, end_bit=e)
    assert np.array_equal(ko, keys[asc]) and np.array_equal(vo, vals[asc])
    ko, vo = gpu_sort(hip, keys, vals, begin_bit=b, end_bit=e, descending=True)
    assert np.array_equal(ko, keys[desc]) and np.array_equal(vo, vals[desc])


@pytest.mark.parametrize("begin,end", [(0, 5), (3, 17), (8, 24), (31, 32), (0, 12)])
def test_partial_bit_ranges_random(hip, orc, dev, begin, end):
    n = 200003
    keys = orc.generate(1, n, begin * 100 + end)
    vals = np.arange(n, dtype=np.uint32)
    ko, vo = gpu_sort(hip, keys, vals, begin, end)
    eko, evo = orc.radix_sort(keys, vals, begin, end)
    assert np.array_equal(ko, eko) and np.array_equal(vo, evo)


def test_double_buffer_selectors_known_answer(hip, orc, dev):
    n, b, e = 65, 0, 5
    keys = np.array([((i * 19) % 32) | ((i % 7) << 8) for i in range(n)], np.uint32)
    vals = np.arange(n, dtype=np.uint32)
    asc = sorted(range(n), key=lambda i: int(keys[i]) & 31)
    desc = sorted(range(n), key=lambda i: -(int(keys[i]) & 31))
    k0, k1 = empty_dev(n, 4), to_dev(keys)
    sel = hip.sort_keys_db("u32", k0, k1, 1, n, b, e)
    assert sel == 0
    assert np.array_equal(to_host([k0, k1][sel], np.uint32, n), keys[asc])
    pk0, pk1, pv0, pv1 = to_dev(keys), empty_dev(n, 4), to_dev(vals), empty_dev(n, 4)
    sel = hip.sort_pairs_db("u32", 4, pk0, pk1, pv0, pv1, 0, n, b, e, descending=True)
    assert sel == 1
    assert np.array_equal(to_host([pk0, pk1][sel], np.uint32, n), keys[desc])
    assert np.array_equal(to_host([pv0, pv1][sel], np.uint32, n), vals[desc])


@pytest.mark.parametrize("dtype", [np.uint32, np.uint64])
def test_double_buffer_full_width(hip, orc, dev, dtype):
    n = 100003
    keys = orc.generate(0, n, 31).astype(dtype) if dtype == np.uint64 else orc.generate(1, n, 31)
    vals = np.arange(n, dtype=np.uint32)
    sfx = SUFFIX[np.dtype(dtype)]
    k0, k1, v0, v1 = to_dev(keys), empty_dev(n, keys.itemsize), to_dev(vals), empty_dev(n, 4)
    sel = hip.sort_pairs_db(sfx, 4, k0, k1, v0, v1, 0, n)
    passes = keys.itemsize  # 8-bit digits
    assert sel == passes % 2
    eko, evo = orc.radix_sort(keys, vals)
    assert np.array_equal(to_host([k0, k1][sel], dtype, n), eko)
    assert np.array_equal(to_host([v0, v1][sel], np.uint32, n), evo)


def test_double_buffer_zero_width_keeps_current(hip, dev):
    k0, k1 = empty_dev(3, 4), to_dev(np.array([7, 2, 5], np.int32))
    sel = hip.sort_keys_db("i32", k0, k1, 1, 3, 4, 4)
    assert sel == 1
    assert to_host(k1, np.int32, 3).tolist() == [7, 2, 5]


def test_zero_width_copies_and_empty(hip, dev):
    keys = np.array([9, 3, 7, 1], np.uint32)
    vals = np.array([0, 1, 2, 3], np.uint32)
    ko, vo = gpu_sort(hip, keys, vals, 4, 4)
    assert ko.tolist() == [9, 3, 7, 1] and vo.tolist() == [0, 1, 2, 3]
    assert hip.lib().lcpp_hip_radix_sort_keys_u32(None, 0, None, None, 0, 0, 32, 0, None) == hip.OK


def test_temp_too_small_is_an_error(hip, dev):
    a = torch.zeros(10000, dtype=torch.int32, device=dev)
    temp = torch.empty(4, dtype=torch.int32, device=dev)
    with pytest.raises(hip.LcppHipError) as e:
        hip.sort_keys("u32", a, a.clone(), 10000, temp=temp)
    assert e.value.status == hip.ERR_TEMP_TOO_SMALL


@pytest.mark.parametrize("kdtype,vbytes", [(np.uint32, 0), (np.uint32, 4), (np.uint64, 4), (np.float32, 8)])
@pytest.mark.parametrize("descending", [False, True])
def test_multi_portion_carry(hip, orc, dev, kdtype, vbytes, descending):
    """Forces portions of 3 tiles so the per-portion digit offsets (the carry the reference drops at
    device_radix_sort.h:1056 / agent_radix_sort_onesweep.h:362) are exercised on a small input."""
    lib = hip.lib()
    tile = lib.lcpp_hip_radix_tile_items(4, 0)
    n = tile * 10 + 123
    log(f"multi-portion {kdtype.__name__} vbytes={vbytes} desc={descending}")
    raw = orc.generate(0, n, 555)
    keys = (raw & np.uint64(0xF0F0F0F0F0F0F0F0)).astype(np.uint64)
    keys = keys.astype(kdtype) if kdtype == np.uint64 else (keys >> np.uint64(32)).astype(np.uint32).view(kdtype)
    keys = keys.copy()
    vals = None if vbytes == 0 else np.arange(n, dtype=np.uint32 if vbytes == 4 else np.uint64)
    try:
        lib.lcpp_hip_radix_set_portion_limit(tile * 3)
        need = lib.lcpp_hip_internal_radix_needed_bytes(n, keys.itemsize, vbytes, 0, keys.itemsize * 8, 0)
        # The limit rounds down to whole tiles of this key / value type (4 or 5 portions here).
        kv_tile = lib.lcpp_hip_radix_tile_items(keys.itemsize, vbytes)
        portion = max(tile * 3 // kv_tile, 1) * kv_tile
        portions = lib.lcpp_hip_internal_radix_portions(n, keys.itemsize, vbytes, 0, keys.itemsize * 8, 0, need)
        assert portions == -(-n // portion) and portions >= 4
        temp = torch.empty((need + 3) // 4, dtype=torch.int32, device=dev)
        sfx = SUFFIX[keys.dtype]
        kin, kout = to_dev(keys), empty_dev(n, keys.itemsize)
        if vals is None:
            hip.sort_keys(sfx, kin, kout, n, descending=descending, temp=temp)
            check_bits(to_host(kout, keys.dtype, n), orc.radix_sort(keys, descending=descending))
        else:
            vin, vout = to_dev(vals), empty_dev(n, vbytes)
            hip.sort_pairs(sfx, vbytes, kin, kout, vin, vout, n, descending=descending, temp=temp)
            eko, evo = orc.radix_sort(keys, vals, descending=descending)
            check_bits(to_host(kout, keys.dtype, n), eko)
            assert np.array_equal(to_host(vout, vals.dtype, n), evo)
    finally:
        lib.lcpp_hip_radix_set_portion_limit(0)


def complete_stable_check(in_keys: np.ndarray, out_keys: np.ndarray, out_vals: np.ndarray) -> None:
    """O(n) characterisation of the stable ascending sort when values are the original indices:
    keys non-decreasing, values a permutation, out_key[i] == in_key[out_val[i]], and values strictly
    increasing within runs of equal keys."""
    n = in_keys.size
    assert np.all(out_keys[1:] >= out_keys[:-1])
    assert np.array_equal(out_keys, in_keys[out_vals])
    seen = np.zeros(n, dtype=bool)
    seen[out_vals] = True
    assert seen.all()
    same = out_keys[1:] == out_keys[:-1]
    assert np.all(out_vals[1:][same] > out_vals[:-1][same])


def test_benchmark_sort_keys_2p28(hip, orc, dev):
    """2^28 uniform u32 keys (4 passes): full output compared bit-exact with the oracle."""
    n = 1 << 28
    log("sort keys 2^28")
    d = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_HI, d, n, 114521)
    out = torch.empty_like(d)
    hip.sort_keys("u32", d, out, n)
    got = to_host(out, np.uint32)
    keys = to_host(d, np.uint32)
    assert np.array_equal(got, orc.radix_sort(keys))


@pytest.mark.parametrize("kind", ["uniform", "and3"])
def test_benchmark_sort_pairs_2p27(hip, orc, dev, kind):
    """2^27 u64 keys + u32 index values (8 passes), complete stability check."""
    n = 1 << 27
    log(f"sort pairs 2^27 {kind}")
    k = torch.empty(n, dtype=torch.int64, device=dev)
    hip.generate(hip.GEN_U64 if kind == "uniform" else hip.GEN_U64_AND3, k, n, 114521)
    v = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_IOTA, v, n, 0)
    ko, vo = torch.empty_like(k), torch.empty_like(v)
    hip.sort_pairs("u64", 4, k, ko, v, vo, n)
    complete_stable_check(to_host(k, np.uint64), to_host(ko, np.uint64), to_host(vo, np.uint32))


@pytest.mark.parametrize("kdtype,vbytes,descending,n", [(np.uint32, 0, False, (1 << 20) + 4321),
                                                        (np.uint32, 4, True, (1 << 20) + 4321),
                                                        (np.uint64, 4, False, (1 << 20) + 4321),
                                                        (np.float32, 0, True, (1 << 20) + 4321),
                                                        (np.uint32, 0, False, (1 << 23) + 17)])
def test_forced_lookback_fallback(hip, orc, dev, kdtype, vbytes, descending, n):
    """Spin limit 0: every unpublished predecessor's digit counts are computed by the waiting
    workgroup from that tile's keys and published by compare-and-swap (the largest case walks back
    over hundreds of tiles, several look-back steps per tile)."""
    lib = hip.lib()
    log(f"sort forced fallback {kdtype.__name__} vbytes={vbytes} desc={descending}")
    raw = orc.generate(0, n, 808)
    keys = raw.copy() if kdtype == np.uint64 else (raw >> np.uint64(32)).astype(np.uint32).view(kdtype).copy()
    vals = None if vbytes == 0 else np.arange(n, dtype=np.uint32)
    old = lib.lcpp_hip_get_lookback_spin_limit()
    try:
        lib.lcpp_hip_set_lookback_spin_limit(0)
        if vals is None:
            check_bits(gpu_sort(hip, keys, descending=descending), orc.radix_sort(keys, descending=descending))
        else:
            ko, vo = gpu_sort(hip, keys, vals, descending=descending)
            eko, evo = orc.radix_sort(keys, vals, descending=descending)
            check_bits(ko, eko)
            assert np.array_equal(vo, evo)
    finally:
        lib.lcpp_hip_set_lookback_spin_limit(old)


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("case", ["u32_random", "u64_and3_pairs", "u32_low_entropy_desc", "f32_pairs"])
def test_rank_modes_agree_with_oracle(hip, orc, dev, mode, case):
    """Every in-wave ranker (ballot match in all waves, LDS lane-mask tables in all waves, and the default
    split between them) gives the stable ranks; low-entropy keys put many lanes of a wave on the same
    digit entry."""
    lib = hip.lib()
    n = 500009
    raw = orc.generate(0, n, 4040)
    vals = np.arange(n, dtype=np.uint32)
    desc = case.endswith("desc")
    if case == "u32_random":
        keys, vals = (raw >> np.uint64(32)).astype(np.uint32), None
    elif case == "u64_and3_pairs":
        keys = orc.generate(4, n, 4041)
    elif case == "u32_low_entropy_desc":
        keys, vals = ((raw >> np.uint64(32)) & np.uint64(0x01010101)).astype(np.uint32), None
    else:
        keys = orc.generate(6, n, 4042)
        keys[::3] = keys[7]
    try:
        assert lib.lcpp_hip_internal_radix_rank_mode(mode) == 0
        if vals is None:
            check_bits(gpu_sort(hip, keys, descending=desc), orc.radix_sort(keys, descending=desc))
        else:
            ko, vo = gpu_sort(hip, keys, vals, descending=desc)
            eko, evo = orc.radix_sort(keys, vals, descending=desc)
            check_bits(ko, eko)
            assert np.array_equal(vo, evo)
    finally:
        lib.lcpp_hip_internal_radix_rank_mode(2)


@pytest.mark.parametrize("precount", [0, 1])
@pytest.mark.parametrize("case", ["u32_random", "u64_pairs_desc", "f32_bits_3_29", "i32_partial_tile", "u32_db"])
def test_first_pass_offsets_from_histogram(hip, orc, dev, precount, case):
    """The first pass takes its tile offsets from the histogram's per-tile counts (precount 1, for a single
    portion with aligned keys) or walks the look-back like the other passes (0, the default): the same
    stable order either way, for full and partial bit ranges, a partial last tile, pairs, descending
    order and the DoubleBuffer form."""
    lib = hip.lib()
    raw = orc.generate(0, 1 << 20, 5150)
    try:
        old = lib.lcpp_hip_internal_radix_precount(precount)
        if case == "u32_random":
            keys = (raw >> np.uint64(32)).astype(np.uint32)
            check_bits(gpu_sort(hip, keys), orc.radix_sort(keys))
        elif case == "u64_pairs_desc":
            keys = raw[:300007] & np.uint64(0x0F0F0F0F0F0F0F0F)
            vals = np.arange(keys.size, dtype=np.uint32)
            ko, vo = gpu_sort(hip, keys, vals, descending=True)
            eko, evo = orc.radix_sort(keys, vals, descending=True)
            check_bits(ko, eko)
            assert np.array_equal(vo, evo)
        elif case == "f32_bits_3_29":
            keys = orc.generate(6, 250001, 5151)
            check_bits(gpu_sort(hip, keys, begin_bit=3, end_bit=29), orc.radix_sort(keys, begin_bit=3, end_bit=29))
        elif case == "i32_partial_tile":
            keys = (raw[:16384 * 7 + 1234] >> np.uint64(40)).astype(np.int32) - (1 << 23)
            check_bits(gpu_sort(hip, keys), orc.radix_sort(keys))
        else:
            n = 1 << 19
            keys = (raw[:n] >> np.uint64(16)).astype(np.uint32)
            d0, d1 = to_dev(keys), fill_dev(n, 4, -1)
            sel = hip.sort_keys_db("u32", d0, d1, 0, n)
            got = to_host(d1 if sel == 1 else d0, np.uint32, n)
            check_bits(got, orc.radix_sort(keys))
    finally:
        lib.lcpp_hip_internal_radix_precount(old)


def test_constant_keys_large(hip, dev):
    """2^25 identical keys: every histogram count lands in one digit of every pass (the packed 16-bit
    per-bank counters of one workgroup must not overflow), and the sort is the identity."""
    n = 1 << 25
    log("sort constant keys 2^25")
    d = torch.full((n,), 0x12345678, dtype=torch.int32, device=dev)
    out = torch.empty_like(d)
    hip.sort_keys("u32", d, out, n)
    assert torch.equal(out, d)


def test_two_valued_u64_pairs_large(hip, dev):
    """2^24 u64 keys taking two values (1/3 vs 2/3 of the items) with index values: keys grouped,
    values increasing inside each group (stability), counts exact."""
    n = 1 << 24
    log("sort pairs two-valued u64 2^24")
    idx = torch.arange(n, dtype=torch.int64, device=dev)
    k = torch.where(idx % 3 == 0, torch.tensor(7 << 40, device=dev), torch.tensor(5 << 40, device=dev))
    v = idx.to(torch.int32)
    ko, vo = torch.empty_like(k), torch.empty_like(v)
    hip.sort_pairs("u64", 4, k, ko, v, vo, n)
    n7 = (n + 2) // 3
    expect_v = torch.cat([idx[idx % 3 != 0], idx[idx % 3 == 0]]).to(torch.int32)
    assert torch.equal(vo, expect_v)
    assert torch.equal(ko[: n - n7], torch.full((n - n7,), 5 << 40, dtype=torch.int64, device=dev))
    assert torch.equal(ko[n - n7:], torch.full((n7,), 7 << 40, dtype=torch.int64, device=dev))
