"""Stream compaction on the GPU through the C-ABI: DeviceSelect (Flagged, If, FlaggedIf, Unique,
UniqueByKey; copy and in-place), DevicePartition (Flagged, If, three-way If) and DeviceRunLengthEncode
(Encode, NonTrivialRuns).

Every result is compared bit-exactly with the oracle (counts and the written prefix of every output;
partition outputs in full).  Known answers of the reference's tests (device_select_test.cpp,
device_partition_test.cpp, device_run_length_encode_test.cpp) exactly.  Also: all item and flag
types, tile-boundary sizes (8192-item tiles for 4-byte items, 4096 for 8-byte), runs crossing many
tiles, the forced look-back fallback (spin limit 0), misaligned views and 2^26-item inputs."""
import numpy as np
import pytest
import torch

from gpu_util import fill_dev, log, to_dev, to_host

pytestmark = pytest.mark.gpu

NP = {"i32": np.int32, "u32": np.uint32, "f32": np.float32, "i64": np.int64, "u64": np.uint64, "f64": np.float64,
      "b8": np.uint8}
SUFFIX = {np.dtype(v): k for k, v in NP.items()}
T4, T8 = 8192, 4096


def items_for(rng, n, ts):
    dt = NP[ts]
    if ts in ("f32", "f64"):
        return np.round(rng.uniform(-100.0, 100.0, n), 1).astype(dt)
    info = np.iinfo(dt)
    return rng.integers(max(info.min, -1000), min(info.max, 1000), n, endpoint=True).astype(dt)


def runs_of(rng, n, mean_len, dtype, distinct=50):
    lengths = rng.geometric(1.0 / mean_len, size=n // max(1, int(mean_len)) + 16)
    while lengths.sum() < n:
        lengths = np.concatenate([lengths, rng.geometric(1.0 / mean_len, size=len(lengths))])
    vals = rng.integers(0, distinct, lengths.size)
    return np.repeat(vals, lengths)[:n].astype(dtype)


def clauses_for(ts):
    if ts in ("f32", "f64"):
        return [(1, 25.5, 0), (3, -60.0, 0)]          # -60 < x < 25.5
    if ts in ("u32", "u64"):
        return [(10, 3, 1), (6, 0, 0)]                # x % 3 == 1 and x != 0
    return [(10, 3, 0), (3, -500, 0)]                 # x % 3 == 0 and x > -500


# ---- GPU calls (outputs pre-filled with a poison pattern) -------------------------------------------
def dev_at(x, offset_items):
    """x on the device, starting `offset_items` items into its allocation (a view off the 16-byte
    alignment of a fresh tensor when offset_items * itemsize is not a multiple of 16)."""
    return to_dev(np.concatenate([np.zeros(offset_items, x.dtype), x]))[offset_items:] if offset_items else to_dev(x)


def g_select_if(hip, x, clauses, partition=False, in_place=False, offset_items=0):
    ts, n = SUFFIX[x.dtype], x.size
    d_in = dev_at(x, offset_items)
    d_out = d_in if in_place else fill_dev(n, x.itemsize, 0x5A)
    num = fill_dev(1, 4, 99)
    pred = hip.predicate(ts, *clauses)
    (hip.partition_if if partition else hip.select_if)(ts, d_in, d_out, num, n, pred)
    k = int(to_host(num, np.uint32, 1)[0])
    return to_host(d_out, x.dtype, n), k


def g_select_flagged(hip, x, flags, partition=False, in_place=False, clauses=None):
    ts, fs, n = SUFFIX[x.dtype], SUFFIX[flags.dtype], x.size
    d_in, d_f = to_dev(x), to_dev(flags)
    d_out = d_in if in_place else fill_dev(n, x.itemsize, 0x5A)
    num = fill_dev(1, 4, 99)
    if clauses is not None:
        hip.select_flagged_if(ts, fs, d_in, d_f, d_out, num, n, hip.predicate(fs, *clauses))
    elif partition:
        hip.partition_flagged(ts, fs, d_in, d_f, d_out, num, n)
    else:
        hip.select_flagged(ts, fs, d_in, d_f, d_out, num, n)
    return to_host(d_out, x.dtype, n), int(to_host(num, np.uint32, 1)[0])


def g_three_way(hip, x, c1, c2, offset_items=0):
    ts, n = SUFFIX[x.dtype], x.size
    d_in = dev_at(x, offset_items)
    o1, o2, o3 = (fill_dev(n, x.itemsize, 0x5A) for _ in range(3))
    num = fill_dev(2, 4, 99)
    hip.partition_three_way(ts, d_in, o1, o2, o3, num, n, hip.predicate(ts, *c1), hip.predicate(ts, *c2))
    c = to_host(num, np.uint32, 2)
    return to_host(o1, x.dtype, n), to_host(o2, x.dtype, n), to_host(o3, x.dtype, n), (int(c[0]), int(c[1]))


def g_unique(hip, x, key_mask=-1, in_place=False):
    ts, n = SUFFIX[x.dtype], x.size
    d_in = to_dev(x)
    d_out = d_in if in_place else fill_dev(n, x.itemsize, 0x5A)
    num = fill_dev(1, 4, 99)
    hip.select_unique(ts, d_in, d_out, num, n, key_mask=key_mask)
    k = int(to_host(num, np.uint32, 1)[0])
    return to_host(d_out, x.dtype, n)[:k], k


def g_unique_by_key(hip, keys, vals, key_mask=-1):
    n = keys.size
    d_k, d_v = to_dev(keys), to_dev(vals)
    ko, vo = fill_dev(n, keys.itemsize, 0x5A), fill_dev(n, vals.itemsize, 0x5A)
    num = fill_dev(1, 4, 99)
    hip.select_unique_by_key(SUFFIX[keys.dtype], SUFFIX[vals.dtype], d_k, d_v, ko, vo, num, n, key_mask=key_mask)
    k = int(to_host(num, np.uint32, 1)[0])
    return to_host(ko, keys.dtype, n)[:k], to_host(vo, vals.dtype, n)[:k], k


def g_encode(hip, x):
    ts, n = SUFFIX[x.dtype], x.size
    d_in = to_dev(x)
    uo, co = fill_dev(n, x.itemsize, 0x5A), fill_dev(n, 4, 0x5A)
    num = fill_dev(1, 4, 99)
    hip.run_length_encode(ts, d_in, uo, co, num, n)
    r = int(to_host(num, np.uint32, 1)[0])
    return to_host(uo, x.dtype, n)[:r], to_host(co, np.uint32, n)[:r]


def g_non_trivial(hip, x):
    ts, n = SUFFIX[x.dtype], x.size
    d_in = to_dev(x)
    oo, lo = fill_dev(n, 4, 0x5A), fill_dev(n, 4, 0x5A)
    num = fill_dev(1, 4, 99)
    hip.run_length_non_trivial(ts, d_in, oo, lo, num, n)
    r = int(to_host(num, np.uint32, 1)[0])
    return to_host(oo, np.uint32, n)[:r], to_host(lo, np.uint32, n)[:r]


# ---- checks against the oracle ----------------------------------------------------------------------
def check_select(orc, x, sel, got, k, partition=False):
    want, wk = orc.select(x, sel, partition=partition)
    assert k == wk
    if partition:
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8))
    else:
        np.testing.assert_array_equal(got[:k].view(np.uint8), want[:k].view(np.uint8))


def check_all_runs(hip, orc, x):
    u, c = g_encode(hip, x)
    wu, wc = orc.run_length_encode(x)
    np.testing.assert_array_equal(u.view(np.uint8), wu.view(np.uint8))
    np.testing.assert_array_equal(c, wc)
    o, ln = g_non_trivial(hip, x)
    wo, wl = orc.non_trivial_runs(x)
    np.testing.assert_array_equal(o, wo)
    np.testing.assert_array_equal(ln, wl)
    g, k = g_unique(hip, x)
    want, wk = orc.select(x, orc.run_heads(x))
    assert k == wk
    np.testing.assert_array_equal(g.view(np.uint8), want[:k].view(np.uint8))


# ---- known answers of the reference's tests -----------------------------------------------------------
def test_select_flagged_and_if_are_stable_known_answer(hip, dev):
    """device_select_test.cpp:248-299: 100..116, flags 7 where i % 3 == 1, is_even."""
    x = np.arange(100, 117, dtype=np.int32)
    flags = np.where(np.arange(17) % 3 == 1, 7, 0).astype(np.uint32)
    got, k = g_select_flagged(hip, x, flags)
    assert got[:k].tolist() == [101, 104, 107, 110, 113, 116]
    got, k = g_select_if(hip, x, [(hip.PRED_MOD_EQ, 2, 0)])
    assert got[:k].tolist() == list(range(100, 117, 2))


def test_select_wide_values_and_boolean_flags_known_answer(hip, dev):
    """device_select_test.cpp:113-170: 2^40 | i/3 over 17 items; bool flags i % 3 == 1; even; Unique."""
    x = np.array([(1 << 40) | (i // 3) for i in range(17)], np.uint64)
    flags = (np.arange(17) % 3 == 1).astype(np.uint8)
    got, k = g_select_flagged(hip, x, flags)
    assert got[:k].tolist() == [x[i] for i in range(17) if i % 3 == 1]
    got, k = g_select_if(hip, x, [(hip.PRED_MOD_EQ, 2, 0)])
    assert got[:k].tolist() == [v for v in x.tolist() if v % 2 == 0]
    got, k = g_unique(hip, x)
    assert got.tolist() == [x[i] for i in range(17) if i % 3 == 0]


def test_select_unique_and_unique_by_key_known_answer(hip, dev):
    """device_select_test.cpp:301-357."""
    keys = np.array([1, 1, 2, 2, 2, 4, 7, 7, 9], np.int32)
    vals = np.array([10, 11, 20, 21, 22, 40, 70, 71, 90], np.int32)
    got, k = g_unique(hip, keys)
    assert got.tolist() == [1, 2, 4, 7, 9]
    ku, vu, k = g_unique_by_key(hip, keys, vals)
    assert ku.tolist() == [1, 2, 4, 7, 9] and vu.tolist() == [10, 20, 40, 70, 90]


def test_select_flagged_if_copy_and_in_place_known_answer(hip, dev):
    """device_select_test.cpp:359-425: flags -3..5, flag > 0 and flag % 2 != 0; input unchanged."""
    data = np.arange(100, 109, dtype=np.int32)
    flags = np.arange(-3, 6, dtype=np.int32)
    pos_odd = [(hip.PRED_GT, 0), (hip.PRED_MOD_NE, 2, 0)]
    got, k = g_select_flagged(hip, data, flags, clauses=pos_odd)
    assert k == 3 and got[:3].tolist() == [104, 106, 108]
    got, k = g_select_flagged(hip, data, flags, clauses=pos_odd, in_place=True)
    assert k == 3 and got[:3].tolist() == [104, 106, 108]


def test_select_in_place_cases_known_answer(hip, dev):
    """device_select_test.cpp:427-500: flags aliased with the data, x > 0, same-parity Unique (mask 1),
    default Unique, and an empty If that still writes a zero count."""
    aliased = np.array([0, 2, 0, 3, 4, 0, 5, 0], np.int32)
    d = to_dev(aliased)
    num = fill_dev(1, 4, 99)
    hip.select_flagged("i32", "i32", d, d, d, num, 8)
    k = int(to_host(num, np.uint32, 1)[0])
    assert to_host(d, np.int32, k).tolist() == [2, 3, 4, 5]
    got, k = g_select_if(hip, np.array([-3, 4, -1, 6, 0, 2, 7, -8], np.int32), [(hip.PRED_GT, 0)], in_place=True)
    assert got[:k].tolist() == [4, 6, 2, 7]
    got, k = g_unique(hip, np.array([1, 3, 2, 4, 5, 7, 8, 10], np.int32), key_mask=1, in_place=True)
    assert got.tolist() == [1, 2, 5, 8]
    got, k = g_unique(hip, np.array([1, 1, 2, 2, 2, 4, 4, 9], np.int32), in_place=True)
    assert got.tolist() == [1, 2, 4, 9]
    num = fill_dev(1, 4, 1)
    hip.select_if("i32", None, None, num, 0, hip.predicate("i32", (hip.PRED_GT, 0)))
    assert int(to_host(num, np.uint32, 1)[0]) == 0


def test_partition_flagged_and_if_ordering_known_answer(hip, dev):
    """device_partition_test.cpp:103-177."""
    x = np.arange(12, dtype=np.int32)
    got, k = g_select_flagged(hip, x, (np.arange(12) % 3 == 0).astype(np.uint32), partition=True)
    assert k == 4 and got.tolist() == [0, 3, 6, 9, 11, 10, 8, 7, 5, 4, 2, 1]
    got, k = g_select_if(hip, x, [(hip.PRED_LT, 7)], partition=True)
    assert k == 7 and got.tolist() == [0, 1, 2, 3, 4, 5, 6, 11, 10, 9, 8, 7]


def test_partition_three_way_known_answer(hip, dev):
    """device_partition_test.cpp:292-349, and zero input writes both counts (:351-377)."""
    x = np.arange(12, dtype=np.int32)
    o1, o2, o3, c = g_three_way(hip, x, [(hip.PRED_MOD_EQ, 3, 0)], [(hip.PRED_LT, 8)])
    assert c == (4, 5)
    assert o1[:4].tolist() == [0, 3, 6, 9] and o2[:5].tolist() == [1, 2, 4, 5, 7] and o3[:3].tolist() == [11, 10, 8]
    num = fill_dev(2, 4, 7)
    p = hip.predicate("i32", (hip.PRED_LT, 0))
    hip.partition_three_way("i32", None, None, None, None, num, 0, p, p)
    assert to_host(num, np.uint32, 2).tolist() == [0, 0]


def test_run_length_encode_known_answers(hip, dev):
    """device_run_length_encode_test.cpp:41-72 (wide values) and :172-245 (CUB example); empty input
    writes zero counts (:247-280)."""
    x = np.array([1 << 40, 1 << 40, 1 << 41, 1 << 42, 1 << 42, 1 << 42, 1 << 43], np.uint64)
    u, c = g_encode(hip, x)
    assert u.tolist() == [1 << 40, 1 << 41, 1 << 42, 1 << 43] and c.tolist() == [2, 1, 3, 1]
    x = np.array([0, 2, 2, 9, 5, 5, 5, 8], np.int32)
    u, c = g_encode(hip, x)
    assert u.tolist() == [0, 2, 9, 5, 8] and c.tolist() == [1, 2, 1, 3, 1]
    o, ln = g_non_trivial(hip, x)
    assert o.tolist() == [1, 4] and ln.tolist() == [2, 3]
    for f in (hip.run_length_encode, hip.run_length_non_trivial):
        num = fill_dev(1, 4, 99)
        f("i32", None, None, None, num, 0)
        assert int(to_host(num, np.uint32, 1)[0]) == 0


# Tile edges: 4,096 and 8,192 (the compaction kernel's eight- and four-byte tiles), 11,264 and 22,528 (the
# run kernels' tiles of eight- and four-byte items) and their multiples, and other sizes.
@pytest.mark.parametrize("count", [1, 2, 3, 31, 32, 33, 3839, 3840, 3841, 4095, 4096, 4097, 5761, 8191, 8192, 8193,
                                   10240, 11263, 11264, 11265, 14336, 16383, 16384, 16385, 20480, 22527, 22528,
                                   22529, 28672, 33793, 45057, 230413])
def test_run_length_encode_long_runs_across_tiles(hip, orc, dev, count):
    """device_run_length_encode_test.cpp:74-136: x[i] = i / run_length for run lengths 1, 2, 17, 18001, n."""
    for run_length in (1, 2, 17, 18001, count):
        x = (np.arange(count) // run_length).astype(np.int32)
        check_all_runs(hip, orc, x)


def test_run_length_encode_mixed_tiles_and_views(hip, orc, dev):
    """device_run_length_encode_test.cpp:138-170: dense, sparse and headless 3840-item phases, read
    through a view offset by 64 items, for uint and float values."""
    count, pad = 23054, 64
    i = np.arange(count)
    phase = (i // 3840) % 6
    key = np.where((phase == 0) | (phase == 4), i, np.where((phase == 1) | (phase == 2), -7,
                   np.where(phase == 3, (i // 17) % 23 - 11, -4)))
    for dt in (np.uint32, np.float32, np.int32):
        x = key.astype(dt)
        buf = np.concatenate([np.full(pad, 99, dt), x, np.full(pad, 99, dt)])
        d = to_dev(buf)[pad:pad + count]
        uo, co = fill_dev(count, 4, 0x5A), fill_dev(count, 4, 0x5A)
        num = fill_dev(1, 4, 99)
        hip.run_length_encode(SUFFIX[np.dtype(dt)], d, uo, co, num, count)
        r = int(to_host(num, np.uint32, 1)[0])
        wu, wc = orc.run_length_encode(x)
        assert r == wu.size
        np.testing.assert_array_equal(to_host(uo, dt, r), wu)
        np.testing.assert_array_equal(to_host(co, np.uint32, r), wc)


# ---- types, sizes and patterns against the oracle ------------------------------------------------------
@pytest.mark.parametrize("ts", ["i32", "u32", "f32", "i64", "u64", "f64"])
def test_select_and_partition_if_types(hip, orc, dev, ts):
    rng = np.random.default_rng(sum(map(ord, ts)))
    for n in (1, 33, 4099, 3 * T4 + 17):
        x = items_for(rng, n, ts)
        cl = clauses_for(ts)
        sel = orc.predicate(x, cl)
        for partition in (False, True):
            got, k = g_select_if(hip, x, cl, partition=partition)
            check_select(orc, x, sel, got, k, partition)


@pytest.mark.parametrize("ts", ["i32", "f32", "u64", "f64"])
@pytest.mark.parametrize("fs", ["b8", "i32", "u32", "i64", "u64"])
def test_select_flagged_types(hip, orc, dev, ts, fs):
    rng = np.random.default_rng(sum(map(ord, ts + fs)))
    n = 2 * T4 + 1234
    x = items_for(rng, n, ts)
    raw = rng.integers(-2, 3, n)
    flags = (raw != 0).astype(np.uint8) if fs == "b8" else raw.astype(NP[fs])
    sel = (flags != 0).astype(np.uint8)
    for partition in (False, True):
        got, k = g_select_flagged(hip, x, flags, partition=partition)
        check_select(orc, x, sel, got, k, partition)
    if fs in ("i32", "i64"):
        cl = [(hip.PRED_GT, 0), (hip.PRED_MOD_NE, 2, 0)]
        got, k = g_select_flagged(hip, x, flags, clauses=cl)
        check_select(orc, x, orc.predicate(flags, cl), got, k)


@pytest.mark.parametrize("n", [1, 5759, 5760, 5761, T8 - 1, T8, T8 + 1, T4 - 1, T4, T4 + 1, 230413])
def test_flagged_patterns_multitile(hip, orc, dev, n):
    """device_select_test.cpp:172-246 and device_partition_test.cpp:241-290: none, all, i % 3, first 11
    and beyond 200000 flagged."""
    x = np.arange(n, dtype=np.int32)
    i = np.arange(n)
    for pattern in range(4):
        flags = [np.zeros(n), np.ones(n), i % 3, (i < 11) | (i > 200000)][pattern].astype(np.uint32)
        sel = (flags != 0).astype(np.uint8)
        for partition in (False, True):
            got, k = g_select_flagged(hip, x, flags, partition=partition)
            check_select(orc, x, sel, got, k, partition)


@pytest.mark.parametrize("ts", ["i32", "u32", "f32", "i64", "u64", "f64"])
def test_three_way_types(hip, orc, dev, ts):
    rng = np.random.default_rng(sum(map(ord, ts)) + 7)
    for n in (1, 100, 3 * T4 + 5):
        x = items_for(rng, n, ts)
        if ts in ("f32", "f64"):
            c1, c2 = [(hip.PRED_LT, -30.0)], [(hip.PRED_RANGE, -10.0, 40.0)]
        else:
            c1, c2 = [(hip.PRED_MOD_EQ, 5, 0)], [(hip.PRED_LT, 300)]
        o1, o2, o3, c = g_three_way(hip, x, c1, c2)
        w1, w2, w3, wc = orc.partition_three_way(x, orc.predicate(x, c1), orc.predicate(x, c2))
        assert c == wc
        u = n - wc[0] - wc[1]
        np.testing.assert_array_equal(o1[:wc[0]], w1[:wc[0]])
        np.testing.assert_array_equal(o2[:wc[1]], w2[:wc[1]])
        np.testing.assert_array_equal(o3[:u], w3[:u])


@pytest.mark.parametrize("ts", ["i32", "u32", "f32", "i64", "u64", "f64"])
def test_run_length_and_unique_types(hip, orc, dev, ts):
    rng = np.random.default_rng(sum(map(ord, ts)) + 3)
    for mean in (1.2, 9.0, 700.0):
        x = runs_of(rng, 5 * T4 + 77, mean, NP[ts])
        check_all_runs(hip, orc, x)


@pytest.mark.parametrize("ts", ["u32", "f32", "i64", "f64"])
def test_runs_staged_and_direct_tiles(hip, orc, dev, ts):
    """Run lengths 1..6 in 4,096-item stretches: tiles with more runs than the run kernel stages in LDS
    (4,096 for four-byte items, 2,730 for eight-byte ones) write them row by row, the others from LDS."""
    n = 20 * 28672 + 5
    length = 1 + (np.arange(n) // 4096) % 6
    starts = np.zeros(n, bool)
    pos = 0
    while pos < n:
        starts[pos] = True
        pos += int(length[pos])
    x = (np.cumsum(starts) % 1000).astype(NP[ts])
    log(f"runs staged/direct {ts}")
    check_all_runs(hip, orc, x)


def test_unique_and_encode_overlapping_outputs(hip, orc, dev):
    """Unique in place (a select's in-place form) and an encode whose unique output is its input take the
    general compaction path; results match the oracle."""
    rng = np.random.default_rng(8)
    x = runs_of(rng, 40 * T4 + 3, 5.0, np.int32, distinct=7)
    g, k = g_unique(hip, x, in_place=True)
    want, wk = orc.select(x, orc.run_heads(x))
    assert k == wk and np.array_equal(g, want[:k])
    d = to_dev(x)
    co = fill_dev(x.size, 4, 0x5A)
    num = fill_dev(1, 4, 99)
    hip.run_length_encode("i32", d, d, co, num, x.size)
    r = int(to_host(num, np.uint32, 1)[0])
    wu, wc = orc.run_length_encode(x)
    assert r == wu.size
    np.testing.assert_array_equal(to_host(d, np.int32, r), wu)
    np.testing.assert_array_equal(to_host(co, np.uint32, r), wc)


def test_float_run_equality_is_by_value(hip, orc, dev):
    """-0.0 and +0.0 form one run; NaNs never extend a run (lhs == rhs)."""
    x = np.array([1.0, -0.0, 0.0, 0.0, np.nan, np.nan, 2.0, 2.0], np.float32)
    u, c = g_encode(hip, x)
    assert c.tolist() == [1, 3, 1, 1, 2]
    check_all_runs(hip, orc, x)


@pytest.mark.parametrize("ks", ["i32", "f32", "u64", "f64"])
@pytest.mark.parametrize("vs", ["u32", "f64"])
def test_unique_by_key_types(hip, orc, dev, ks, vs):
    rng = np.random.default_rng(sum(map(ord, ks + vs)))
    n = 4 * T4 + 999
    keys = runs_of(rng, n, 6.0, NP[ks])
    vals = items_for(rng, n, vs)
    ku, vu, k = g_unique_by_key(hip, keys, vals)
    heads = orc.run_heads(keys)
    wk, kk = orc.select(keys, heads)
    wv, _ = orc.select(vals, heads)
    assert k == kk
    np.testing.assert_array_equal(ku.view(np.uint8), wk[:k].view(np.uint8))
    np.testing.assert_array_equal(vu.view(np.uint8), wv[:k].view(np.uint8))


def test_unique_key_mask(hip, orc, dev):
    rng = np.random.default_rng(12)
    x = rng.integers(0, 1 << 12, 3 * T4 + 1).astype(np.uint32)
    got, k = g_unique(hip, x, key_mask=0xF00)
    want, wk = orc.select(x, orc.run_heads(x, key_mask=0xF00))
    assert k == wk and got.tolist() == want[:k].tolist()


def test_forced_fallback_and_in_place(hip, orc, dev):
    """Every look-back takes the fallback (spin limit 0), for in-place selects, partitions and runs."""
    rng = np.random.default_rng(77)
    n = 200 * T4 + 9
    x = items_for(rng, n, "i32")
    lib = hip.lib()
    old = lib.lcpp_hip_get_lookback_spin_limit()
    try:
        lib.lcpp_hip_set_lookback_spin_limit(0)
        cl = clauses_for("i32")
        sel = orc.predicate(x, cl)
        log("compact fallback: select in place")
        got, k = g_select_if(hip, x, cl, in_place=True)
        check_select(orc, x, sel, got, k)
        log("compact fallback: partition")
        got, k = g_select_if(hip, x, cl, partition=True)
        check_select(orc, x, sel, got, k, True)
        log("compact fallback: three-way")
        o1, o2, o3, c = g_three_way(hip, x, [(hip.PRED_MOD_EQ, 5, 0)], [(hip.PRED_LT, 300)])
        w1, w2, w3, wc = orc.partition_three_way(x, orc.predicate(x, [(10, 5, 0)]), orc.predicate(x, [(1, 300, 0)]))
        assert c == wc and np.array_equal(o3[:n - sum(wc)], w3[:n - sum(wc)])
        log("compact fallback: runs")
        check_all_runs(hip, orc, runs_of(rng, n, 40.0, np.int32))
    finally:
        lib.lcpp_hip_set_lookback_spin_limit(old)


@pytest.mark.parametrize("which", ["in", "flags", "out"])
def test_misaligned_views(hip, orc, dev, which):
    rng = np.random.default_rng(31)
    n = 3 * T4 + 11
    x = items_for(rng, n, "u32")
    flags = rng.integers(0, 2, n).astype(np.uint8)
    d_in = to_dev(np.concatenate([[5], x]).astype(np.uint32))[1:] if which == "in" else to_dev(x)
    d_f = to_dev(np.concatenate([[1], flags]).astype(np.uint8))[1:] if which == "flags" else to_dev(flags)
    d_out = (torch.empty(n + 1, dtype=torch.int32, device=dev)[1:] if which == "out"
             else torch.empty(n, dtype=torch.int32, device=dev))
    num = fill_dev(1, 4, 99)
    hip.partition_flagged("u32", "b8", d_in, d_f, d_out, num, n)
    check_select(orc, x, flags, to_host(d_out, np.uint32, n), int(to_host(num, np.uint32, 1)[0]), True)


@pytest.mark.parametrize("ts", ["u32", "i64", "f32"])
@pytest.mark.parametrize("offset_items", [0, 1])
def test_vector_loads_and_unaligned_inputs(hip, orc, dev, ts, offset_items):
    """Select-if, partition-if and the three-way partition read a wave's items as 16-byte vectors when the
    input is 16-byte aligned and the wave's items all exist; an input one item off that alignment, and the
    last, partial waves, take one load per item.  Both bit-exact."""
    rng = np.random.default_rng(311 + offset_items + len(ts))
    n = 5 * T4 + 37
    x = items_for(rng, n, ts)
    cl = clauses_for(ts)
    sel = orc.predicate(x, cl)
    for partition in (False, True):
        got, k = g_select_if(hip, x, cl, partition=partition, offset_items=offset_items)
        check_select(orc, x, sel, got, k, partition)
    c2 = [(1, 100, 0)] if ts != "f32" else [(1, 0.0, 0)]  # x < 100 (x < 0.0) as the second category
    o1, o2, o3, c = g_three_way(hip, x, cl, c2, offset_items=offset_items)
    w1, w2, w3, wc = orc.partition_three_way(x, sel, orc.predicate(x, c2))
    assert c == wc
    assert np.array_equal(o1[:wc[0]], w1[:wc[0]]) and np.array_equal(o2[:wc[1]], w2[:wc[1]])
    assert np.array_equal(o3[:n - sum(wc)], w3[:n - sum(wc)])


def test_large_inputs(hip, orc, dev):
    """2^26 items: select-if, partition, three-way and run-length encode bit-exact against the oracle."""
    rng = np.random.default_rng(2026)
    n = 1 << 26
    x = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    cl = [(hip.PRED_LT, 1 << 31)]
    sel = orc.predicate(x, cl)
    log("compact large: select")
    got, k = g_select_if(hip, x, cl)
    check_select(orc, x, sel, got, k)
    log("compact large: partition")
    got, k = g_select_if(hip, x, cl, partition=True)
    check_select(orc, x, sel, got, k, True)
    log("compact large: runs")
    check_all_runs(hip, orc, runs_of(rng, n, 64.0, np.uint32, distinct=1000))


def test_errors(hip, dev):
    n = 10 * T4
    a = torch.zeros(n, dtype=torch.int32, device=dev)
    num = fill_dev(1, 4, 0)
    temp = torch.empty(4, dtype=torch.int32, device=dev)
    with pytest.raises(hip.LcppHipError) as e:
        hip.select_if("i32", a, a.clone(), num, n, hip.predicate("i32", (hip.PRED_GT, 0)), temp=temp)
    assert e.value.status == hip.ERR_TEMP_TOO_SMALL
    f = torch.zeros(n, dtype=torch.float32, device=dev)
    with pytest.raises(hip.LcppHipError) as e:
        hip.select_if("f32", f, f.clone(), num, n, hip.predicate("f32", (hip.PRED_MOD_EQ, 2.0, 0.0)))
    assert e.value.status == hip.ERR_INVALID_ARGUMENT
    with pytest.raises(hip.LcppHipError) as e:
        hip.select_if("i32", a, a.clone(), num, n, hip.predicate("i32", (hip.PRED_MOD_EQ, 0, 0)))
    assert e.value.status == hip.ERR_INVALID_ARGUMENT
    with pytest.raises(hip.LcppHipError) as e:
        hip.partition_if("i32", a, a, num, n, hip.predicate("i32", (hip.PRED_GT, 0)))
    assert e.value.status == hip.ERR_INVALID_ARGUMENT


# ---- the register-resident rows kernel (selects and partitions not in place) and the staging kernel ----
R4, R8, R4F, R8F = 16384, 6144, 12288, 6144  # rows-kernel tiles: 4- / 8-byte items, without / with flags


@pytest.fixture(params=[True, False], ids=["rows", "staging"])
def rows_kernel(hip, request):
    """Runs the test with the rows kernel allowed (the default) and with every call on the staging kernel."""
    lib = hip.lib()
    old = lib.lcpp_hip_internal_compact_rows(1 if request.param else 0)
    yield request.param
    lib.lcpp_hip_internal_compact_rows(old)


@pytest.mark.parametrize("ts", ["i32", "u32", "f32", "i64", "u64", "f64"])
def test_select_partition_if_at_rows_tile_boundaries(hip, orc, dev, rows_kernel, ts):
    rng = np.random.default_rng(900 + sum(map(ord, ts)))
    tile = R8 if ts in ("i64", "u64", "f64") else R4
    cl = clauses_for(ts)
    for n in (1, 255, 1024, tile - 1, tile, tile + 1, 2 * tile + 7, 5 * tile - 3):
        log(f"rows={rows_kernel} {ts} select/partition-if n={n}")
        x = items_for(rng, n, ts)
        sel = orc.predicate(x, cl)
        for partition in (False, True):
            got, k = g_select_if(hip, x, cl, partition=partition)
            check_select(orc, x, sel, got, k, partition)


@pytest.mark.parametrize("ts", ["i32", "u64"])
@pytest.mark.parametrize("fs", ["b8", "i32", "u32", "u64"])
def test_select_partition_flagged_at_rows_tile_boundaries(hip, orc, dev, rows_kernel, ts, fs):
    """Flags of 1 and 4 bytes take the rows kernel (8-byte flags the staging kernel); every pattern of the
    reference's flagged tests, at the rows tiles' boundaries."""
    tile = R8F if ts == "u64" else R4F
    rng = np.random.default_rng(77 + len(ts + fs))
    for n in (tile - 1, tile, tile + 1, 3 * tile + 5):
        x = items_for(rng, n, ts)
        i = np.arange(n)
        for pattern in range(4):
            raw = [np.zeros(n), np.ones(n), i % 3, rng.integers(-2, 3, n)][pattern]
            flags = (raw != 0).astype(np.uint8) if fs == "b8" else raw.astype(NP[fs])
            sel = (flags != 0).astype(np.uint8)
            for partition in (False, True):
                got, k = g_select_flagged(hip, x, flags, partition=partition)
                check_select(orc, x, sel, got, k, partition)
        if fs in ("i32", "u32"):
            cl = [(hip.PRED_GT, 0), (hip.PRED_MOD_NE, 2, 0)]
            flags = rng.integers(-3, 4, n).astype(NP[fs])
            got, k = g_select_flagged(hip, x, flags, clauses=cl)
            check_select(orc, x, orc.predicate(flags, cl), got, k)


def test_rows_kernel_forced_fallback(hip, orc, dev, rows_kernel):
    """Every look-back of the rows kernel takes the fallback (spin limit 0): predecessors counted by their
    successors, select and partition, with and without flags."""
    rng = np.random.default_rng(4242)
    n = 60 * R4 + 13
    x = items_for(rng, n, "u32")
    flags = rng.integers(0, 2, n).astype(np.uint8)
    cl = clauses_for("u32")
    lib = hip.lib()
    old = lib.lcpp_hip_get_lookback_spin_limit()
    try:
        lib.lcpp_hip_set_lookback_spin_limit(0)
        for partition in (False, True):
            log(f"rows={rows_kernel} fallback partition={partition}")
            got, k = g_select_if(hip, x, cl, partition=partition)
            check_select(orc, x, orc.predicate(x, cl), got, k, partition)
            got, k = g_select_flagged(hip, x, flags, partition=partition)
            check_select(orc, x, flags, got, k, partition)
    finally:
        lib.lcpp_hip_set_lookback_spin_limit(old)


def test_rows_kernel_predicates_and_flag_alignment(hip, orc, dev):
    """Every clause kind through the rows kernel (single clauses and pairs); flags one item off their row
    alignment (the staging kernel) against aligned flags (the rows kernel)."""
    rng = np.random.default_rng(99)
    n = 3 * R4 + 77
    x = rng.integers(-5000, 5000, n).astype(np.int32)
    P = hip
    cases = [[(P.PRED_LT, 7)], [(P.PRED_LE, -3)], [(P.PRED_GT, 100)], [(P.PRED_GE, 0)], [(P.PRED_EQ, 5)],
             [(P.PRED_NE, 0)], [(P.PRED_RANGE, -100, 250)], [(P.PRED_MOD_EQ, 7, 3)], [(P.PRED_MOD_NE, 4, 0)],
             [(P.PRED_MASK_EQ, 0xF0, 0x30)], [(P.PRED_MASK_NE, 0x3, 0x1)], [(P.PRED_TRUE,)],
             [(P.PRED_GT, -1000), (P.PRED_MOD_EQ, 3, 1)]]
    for cl in cases:
        sel = orc.predicate(x, cl)
        for partition in (False, True):
            got, k = g_select_if(hip, x, cl, partition=partition)
            check_select(orc, x, sel, got, k, partition)
    flags = rng.integers(0, 3, n + 1).astype(np.int32)
    d_f = to_dev(flags)[1:]  # 4 bytes off the 16-byte row alignment
    d_in = to_dev(x)
    d_out = fill_dev(n, 4, 0x5A)
    num = fill_dev(1, 4, 99)
    hip.partition_flagged("i32", "i32", d_in, d_f, d_out, num, n)
    check_select(orc, x, (flags[1:] != 0).astype(np.uint8), to_host(d_out, np.int32, n),
                 int(to_host(num, np.uint32, 1)[0]), True)
