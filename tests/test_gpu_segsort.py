"""DeviceSegmentedRadixSort / DeviceSegmentedSort on the GPU through the C-ABI: stable per-segment sorts
of keys and pairs, ascending and descending, partial bit ranges, value order for floats, DoubleBuffer
forms, bit-exact against the oracle (items outside every segment must stay untouched).

Known answer of the reference's test (device_segmented_sort_test.cpp:19-264) exactly; segments from
1 item to 2^20 items (the block phase sorts 2,048-item chunks in LDS, longer segments take global
merge passes), many small segments, and a 2^24-item input."""
import numpy as np
import pytest
import torch

from gpu_util import fill_dev, log, to_dev, to_host

pytestmark = pytest.mark.gpu

NP = {"u32": np.uint32, "i32": np.int32, "f32": np.float32, "u64": np.uint64, "i64": np.int64, "f64": np.float64}
SEG_KEYS = [91, 3, -2, 3, 92, 8, 1, 8, 4, 93, 5, -1, 5, 2, -1, 7, 2, 5, 0]
SEG_B, SEG_E = [1, 5, 5, 10], [4, 5, 9, 19]


def keys_for(rng, n, ks):
    dt = NP[ks]
    if ks in ("f32", "f64"):
        return (rng.integers(-300, 300, n) / 8.0).astype(dt)      # many ties, both zero signs
    info = np.iinfo(dt)
    return rng.integers(max(info.min, -5000), min(info.max, 5000), n, endpoint=True).astype(dt)


def contiguous_segments(rng, n, m, empty_every=7):
    cuts = np.sort(rng.choice(np.arange(1, n), m - 1, replace=False)) if m > 1 else np.array([], np.int64)
    b = np.concatenate([[0], cuts]).astype(np.uint32)
    e = np.concatenate([cuts, [n]]).astype(np.uint32)
    b[::empty_every] = e[::empty_every]      # some empty segments (begin == end)
    return b, e


def g_sort(hip, keys, b, e, values=None, **kw):
    ks = {v: k for k, v in NP.items()}[keys.dtype.type]
    n = keys.size
    d_k = to_dev(keys)
    ko = fill_dev(n, keys.itemsize, 0x3C)
    vi = to_dev(values) if values is not None else None
    vo = fill_dev(n, values.itemsize, 0x3C) if values is not None else None
    hip.segmented_sort(ks, d_k, ko, n, len(b), to_dev(np.asarray(b, np.uint32)), to_dev(np.asarray(e, np.uint32)),
                       values_in=vi, values_out=vo, **kw)
    return to_host(ko, keys.dtype, n), (to_host(vo, values.dtype, n) if values is not None else None)


def check(orc, keys, b, e, got_k, got_v=None, values=None, **kw):
    n = keys.size
    # fill_dev stores the integer 0x3C in every element (untouched items must still hold it).
    fill_k = np.full(n, 0x3C, np.uint64 if keys.itemsize == 8 else np.uint32).view(keys.dtype)
    fill_v = None
    if values is not None:
        fill_v = np.full(n, 0x3C, np.uint64 if values.itemsize == 8 else np.uint32).view(values.dtype)
    wk, wv = orc.segmented_sort(keys, b, e, values=values, keys_out=fill_k, values_out=fill_v, **kw)
    np.testing.assert_array_equal(got_k.view(np.uint8), wk.view(np.uint8))
    if values is not None:
        np.testing.assert_array_equal(got_v.view(np.uint8), wv.view(np.uint8))


def test_segmented_sort_known_answer(hip, orc, dev):
    """device_segmented_sort_test.cpp:19-264: ascending / descending keys and pairs (values = index)."""
    keys = np.array(SEG_KEYS, np.int32)
    vals = np.arange(19, dtype=np.uint32)
    for desc in (False, True):
        for value_order in (False, True):
            gk, gv = g_sort(hip, keys, SEG_B, SEG_E, values=vals, descending=desc, value_order=value_order)
            check(orc, keys, SEG_B, SEG_E, gk, gv, values=vals, descending=desc, value_order=value_order)
            gk2, _ = g_sort(hip, keys, SEG_B, SEG_E, descending=desc, value_order=value_order)
            assert np.array_equal(gk2, gk)
    asc, _ = g_sort(hip, keys, SEG_B, SEG_E)
    assert asc[1:4].tolist() == [-2, 3, 3] and asc[5:9].tolist() == [1, 4, 8, 8] and asc[0] != 91


@pytest.mark.parametrize("ks", ["u32", "i32", "f32", "u64", "i64", "f64"])
def test_types_small_segments(hip, orc, dev, ks):
    rng = np.random.default_rng(sum(map(ord, ks)))
    n = 100_000
    keys = keys_for(rng, n, ks)
    b, e = contiguous_segments(rng, n, 400)
    vals = np.arange(n, dtype=np.uint32)
    for desc in (False, True):
        gk, gv = g_sort(hip, keys, b, e, values=vals, descending=desc)
        check(orc, keys, b, e, gk, gv, values=vals, descending=desc)
    if ks in ("f32", "f64"):
        gk, gv = g_sort(hip, keys, b, e, values=vals, value_order=True)
        check(orc, keys, b, e, gk, gv, values=vals, value_order=True)


@pytest.mark.parametrize("lo,hi", [(2, 6), (0, 1), (5, 31), (7, 7)])
def test_partial_bit_ranges(hip, orc, dev, lo, hi):
    """device_segmented_sort_test.cpp:438-556 (bits [2, 6)), plus 1 bit, 26 bits and no bits (a copy)."""
    rng = np.random.default_rng(lo * 100 + hi)
    n = 20_000
    keys = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    b, e = contiguous_segments(rng, n, 50)
    vals = rng.integers(0, 1 << 63, n, dtype=np.uint64)
    gk, gv = g_sort(hip, keys, b, e, values=vals, begin_bit=lo, end_bit=hi)
    check(orc, keys, b, e, gk, gv, values=vals, begin_bit=lo, end_bit=hi)


@pytest.mark.parametrize("length", [1024, 1025, 2047, 2048, 2049, 4095, 4096, 4097, 5000, 8193, 65_537, 1 << 20])
def test_long_segments_global_passes(hip, orc, dev, length):
    """Segment lengths at the in-LDS sort's size classes (radix order: 4, 8 or 16 items per thread up to
    4,096 items; value order: 2,048-item chunks) and longer ones that take the global merge passes (odd
    and even counts)."""
    rng = np.random.default_rng(length)
    n = length * 2 + 123
    keys = keys_for(rng, n, "i32")
    vals = np.arange(n, dtype=np.uint32)
    b = np.array([3, 3 + length, n - 100], np.uint32)
    e = np.array([3 + length, 3 + 2 * length if 3 + 2 * length <= n - 100 else n - 100, n - 3], np.uint32)
    for desc in (False, True):
        gk, gv = g_sort(hip, keys, b, e, values=vals, descending=desc)
        check(orc, keys, b, e, gk, gv, values=vals, descending=desc)
    fk = keys_for(rng, n, "f32")
    for value_order in (False, True):
        gk, gv = g_sort(hip, fk, b, e, values=vals, value_order=value_order)
        check(orc, fk, b, e, gk, gv, values=vals, value_order=value_order)


@pytest.mark.parametrize("ks", ["u64", "i64", "f64"])
def test_eight_byte_keys_and_values(hip, orc, dev, ks):
    """8-byte keys with 8-byte values (the largest LDS footprint: 72 KiB per workgroup), short segments and
    segments that take global passes, ascending and descending; value order for f64."""
    rng = np.random.default_rng(64 + len(ks))
    n = 60_000
    keys = keys_for(rng, n, ks)
    vals = rng.integers(0, 1 << 63, n, dtype=np.uint64)
    b = np.array([0, 5, 2000, 2049, 6145, 9000, 31_000], np.uint32)
    e = np.array([5, 2000, 2049, 6145, 9000, 31_000, n - 7], np.uint32)
    for desc in (False, True):
        gk, gv = g_sort(hip, keys, b, e, values=vals, descending=desc)
        check(orc, keys, b, e, gk, gv, values=vals, descending=desc)
    if ks == "f64":
        gk, gv = g_sort(hip, keys, b, e, values=vals, value_order=True)
        check(orc, keys, b, e, gk, gv, values=vals, value_order=True)


def test_double_buffer_forms(hip, orc, dev):
    """DoubleBuffer sorts: the result lands where the selector points after ceil(log2 n) flips; a radix
    sort of zero bits leaves buffers and selector alone."""
    rng = np.random.default_rng(8)
    for n in (19, 4000, 70_001):
        keys = keys_for(rng, n, "u64")
        vals = np.arange(n, dtype=np.uint32)
        b, e = contiguous_segments(rng, n, 9)
        flips = int(np.ceil(np.log2(n)))
        for sel0 in (0, 1):
            k0 = to_dev(keys) if sel0 == 0 else fill_dev(n, 8, 1)
            k1 = to_dev(keys) if sel0 == 1 else fill_dev(n, 8, 1)
            v0 = to_dev(vals) if sel0 == 0 else fill_dev(n, 4, 2)
            v1 = to_dev(vals) if sel0 == 1 else fill_dev(n, 4, 2)
            ks, vs = hip.segmented_sort_db("u64", k0, k1, sel0, n, len(b), to_dev(b), to_dev(e), values0=v0,
                                           values1=v1, value_selector=sel0)
            assert ks == vs == sel0 ^ (flips & 1)
            gk = to_host(k1 if ks else k0, np.uint64, n)
            gv = to_host(v1 if vs else v0, np.uint32, n)
            inside = np.zeros(n, bool)
            for s in range(len(b)):
                inside[b[s]:e[s]] = True
            wk, wv = orc.segmented_sort(keys, b, e, values=vals)
            assert np.array_equal(gk[inside], wk[inside]) and np.array_equal(gv[inside], wv[inside])
        k0, k1 = to_dev(keys), fill_dev(n, 8, 1)
        ks, _ = hip.segmented_sort_db("u64", k0, k1, 0, n, len(b), to_dev(b), to_dev(e), begin_bit=5, end_bit=5)
        assert ks == 0 and np.array_equal(to_host(k0, np.uint64, n), keys)


def test_many_tiny_segments_and_large_input(hip, orc, dev):
    """2^24 keys in segments of 1 to 64 items, and 2^22 keys in 16 segments of 2^18."""
    rng = np.random.default_rng(24)
    n = 1 << 24
    keys = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    lengths = rng.integers(1, 65, n // 16)
    cuts = np.cumsum(lengths)
    cuts = cuts[cuts < n]
    b = np.concatenate([[0], cuts]).astype(np.uint32)
    e = np.concatenate([cuts, [n]]).astype(np.uint32)
    log("segsort tiny segments 2^24")
    gk, _ = g_sort(hip, keys, b, e)
    check(orc, keys, b, e, gk)
    m = 1 << 22
    keys2 = keys[:m].copy()
    b2 = (np.arange(16) * (m // 16)).astype(np.uint32)
    e2 = (b2 + m // 16).astype(np.uint32)
    log("segsort 16 x 2^18")
    gk, _ = g_sort(hip, keys2, b2, e2, descending=True)
    check(orc, keys2, b2, e2, gk, descending=True)


@pytest.mark.parametrize("ks", ["u32", "f32", "i64"])
def test_tiles_of_hundreds_of_segments(hip, orc, dev, ks):
    """Segments of 1 to 8 items with gaps: a 2,048-item tile holds hundreds of them, so its position
    labels exceed one byte (the radix order's joint sort then takes two label passes); pairs, ascending
    and descending, a partial bit range, and value order for floats."""
    rng = np.random.default_rng(31 + len(ks))
    n = 1 << 18
    keys = keys_for(rng, n, ks)
    vals = np.arange(n, dtype=np.uint32)
    lengths = rng.integers(1, 9, n // 4)
    gaps = rng.integers(0, 2, n // 4)
    b = np.cumsum(lengths + gaps) - lengths
    keep = b + lengths <= n
    b = b[keep].astype(np.uint32)
    e = (b + lengths[keep]).astype(np.uint32)
    for desc in (False, True):
        gk, gv = g_sort(hip, keys, b, e, values=vals, descending=desc)
        check(orc, keys, b, e, gk, gv, values=vals, descending=desc)
    gk, gv = g_sort(hip, keys, b, e, values=vals, begin_bit=3, end_bit=13)
    check(orc, keys, b, e, gk, gv, values=vals, begin_bit=3, end_bit=13)
    if ks == "f32":
        gk, gv = g_sort(hip, keys, b, e, values=vals, value_order=True)
        check(orc, keys, b, e, gk, gv, values=vals, value_order=True)


def test_errors(hip, dev):
    n = 10_000
    a = torch.zeros(n, dtype=torch.int32, device=dev)
    b = to_dev(np.array([0], np.uint32))
    e = to_dev(np.array([n], np.uint32))
    with pytest.raises(hip.LcppHipError) as err:
        hip.segmented_sort("u32", a, a.clone(), n, 1, b, e, begin_bit=5, end_bit=4)
    assert err.value.status == hip.ERR_INVALID_ARGUMENT
    with pytest.raises(hip.LcppHipError) as err:
        hip.segmented_sort("u32", a, a.clone(), n, 1, b, e, temp=torch.empty(4, dtype=torch.int32, device=dev))
    assert err.value.status == hip.ERR_TEMP_TOO_SMALL


def test_concurrent_streams_keep_their_own_longest_segment(hip, orc, dev):
    """Two streams sort at the same time, one with a 300,000-item segment (nine global passes) and one whose
    longest segment is 3,000 items: each stream's passes stop at its own longest segment, and both results
    are exact."""
    rng = np.random.default_rng(77)
    n = 400_000
    keys = keys_for(rng, n, "u32")
    cases = [(np.array([0, 300_000], np.uint32), np.array([300_000, n], np.uint32)),
             (np.arange(0, n, 3000, dtype=np.uint32), np.minimum(np.arange(0, n, 3000) + 3000, n).astype(np.uint32))]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    d_keys = to_dev(keys)
    outs = [fill_dev(n, 4, 0x3C), fill_dev(n, 4, 0x3C)]
    temps = [torch.empty(hip.bytes_to_uint_count(hip.segmented_sort_keys_temp_bytes(n, 4)), dtype=torch.int32,
                         device=dev) for _ in range(2)]
    offs = [(to_dev(b), to_dev(e)) for b, e in cases]
    torch.cuda.synchronize()
    for rep in range(3):
        for i in (0, 1):
            with torch.cuda.stream(streams[i]):
                hip.segmented_sort("u32", d_keys, outs[i], n, len(cases[i][0]), offs[i][0], offs[i][1], temp=temps[i],
                                   stream=streams[i])
        torch.cuda.synchronize()
        for i in (0, 1):
            check(orc, keys, cases[i][0], cases[i][1], to_host(outs[i], np.uint32, n))


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_mixed_lengths_with_gaps(hip, orc, dev, seed):
    """Small (joint per-tile sorts with labels, including ones that cross a tile edge), medium (one
    workgroup each) and long (chunked, global passes) segments in one call, with gaps of unsorted items
    between segments that must stay untouched; pairs, ascending and descending."""
    rng = np.random.default_rng(500 + seed)
    n = 300_000
    keys = keys_for(rng, n, "i32")
    vals = np.arange(n, dtype=np.uint32)
    b, e, pos = [], [], 0
    while pos < n:
        kind = rng.random()
        length = int(rng.integers(1, 40) if kind < 0.6 else rng.integers(513, 2049) if kind < 0.85
                     else rng.integers(2049, 20_000))
        gap = int(rng.integers(0, 5)) if rng.random() < 0.5 else 0
        start = pos + gap
        end = min(start + length, n)
        if start >= n:
            break
        b.append(start)
        e.append(end)
        pos = end
    b = np.array(b, np.uint32)
    e = np.array(e, np.uint32)
    for desc in (False, True):
        gk, gv = g_sort(hip, keys, b, e, values=vals, descending=desc)
        check(orc, keys, b, e, gk, gv, values=vals, descending=desc)
