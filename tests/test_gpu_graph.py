"""The library's calls under HIP graph capture (torch.cuda.CUDAGraph on a capture stream): no entry point
allocates or records a memset, so a captured sequence of SortKeys, ExclusiveSum, Reduce::Sum, select-if,
ReduceByKey, segment reduce and segmented sort (with segments that take global merge passes) replays
correctly.  Each of four replays runs on freshly generated inputs, with eager work and synchronisations
between replays, and is checked bit for bit against the same sequence run eagerly on the same inputs."""
import numpy as np
import pytest
import torch

from gpu_util import log

pytestmark = pytest.mark.gpu

N = 1 << 20


def _buffers(hip, dev):
    i32 = lambda m: torch.empty(m, dtype=torch.int32, device=dev)
    b = {"keys": i32(N), "small": i32(N), "sorted": i32(N), "scanned": i32(N), "sum": i32(1), "selected": i32(N),
         "num": torch.zeros(2, dtype=torch.int32, device=dev), "runs_keys": i32(N), "uniq": i32(N), "agg": i32(N),
         "runs": torch.zeros(1, dtype=torch.int32, device=dev), "seg_sum": i32(6), "seg_sorted": i32(N)}
    tb = lambda nbytes: torch.empty(hip.bytes_to_uint_count(nbytes), dtype=torch.int32, device=dev)
    b["t_sort"] = tb(hip.sort_keys_temp_bytes(N, 4))
    b["t_scan"] = tb(hip.scan_temp_bytes(N, 4))
    b["t_reduce"] = tb(hip.reduce_temp_bytes(N, 4))
    b["t_select"] = tb(hip.select_temp_bytes(N))
    b["t_rbk"] = tb(hip.reduce_by_key_temp_bytes(N, 4, 4))
    b["t_segsort"] = tb(hip.segmented_sort_keys_temp_bytes(N, 4))
    # Segments: a tiny one, an empty one, one of 2,049 items (one global pass), one of 300,000 (eight
    # passes), a gap, and one reaching the end.
    begins = np.array([0, 10, 10, 3000, 303_000, 400_000], np.int32)
    ends = np.array([7, 10, 2059, 303_000, 399_000, N], np.int32)
    b["begins"] = torch.from_numpy(begins).to(dev)
    b["ends"] = torch.from_numpy(ends).to(dev)
    return b


def _sequence(hip, b):
    half = hip.predicate("u32", (hip.PRED_LT, 1 << 31))
    hip.sort_keys("u32", b["keys"], b["sorted"], N, temp=b["t_sort"])
    hip.scan_sum("u32", b["small"], b["scanned"], N, temp=b["t_scan"])
    hip.reduce_sum("i32", b["small"], b["sum"], N, temp=b["t_reduce"])
    hip.select_if("u32", b["keys"], b["selected"], b["num"], N, half, temp=b["t_select"])
    hip.reduce_by_key("i32", "u32", b["runs_keys"], b["small"], b["uniq"], b["agg"], b["runs"], N, temp=b["t_rbk"])
    hip.segment_reduce("sum", "i32", b["small"], b["seg_sum"], 6, begins=b["begins"], ends=b["ends"])
    hip.segmented_sort("u32", b["keys"], b["seg_sorted"], N, 6, b["begins"], b["ends"], temp=b["t_segsort"])


OUTPUTS = ("sorted", "scanned", "sum", "selected", "num", "uniq", "agg", "runs", "seg_sum", "seg_sorted")


def _fresh_inputs(hip, b, seed):
    hip.generate(hip.GEN_U32_HI, b["keys"], N, seed)
    hip.generate(hip.GEN_U32_LT16, b["small"], N, seed + 1)
    b["runs_keys"].copy_(torch.cumsum((b["keys"] & 15) == 0, 0, dtype=torch.int32))
    for name in OUTPUTS:
        b[name].fill_(-1)  # stale results must not pass for new ones


def test_captured_sequence_replays_match_eager(hip, dev):
    b = _buffers(hip, dev)
    _fresh_inputs(hip, b, 1000)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _sequence(hip, b)  # warm-up on the capture stream (first call from a stream takes its slot)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _sequence(hip, b)
    torch.cuda.synchronize()
    for rep in range(4):
        log(f"graph replay {rep}")
        _fresh_inputs(hip, b, 2000 + 17 * rep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = {name: b[name].clone() for name in OUTPUTS}
        for name in OUTPUTS:
            b[name].fill_(-1)
        _sequence(hip, b)
        torch.cuda.synchronize()
        for name in OUTPUTS:
            if name == "selected":
                k = int(b["num"][0].item())
                assert torch.equal(replayed[name][:k], b[name][:k]), (rep, name)
            elif name in ("uniq", "agg"):
                k = int(b["runs"][0].item())
                assert torch.equal(replayed[name][:k], b[name][:k]), (rep, name)
            else:
                assert torch.equal(replayed[name], b[name]), (rep, name)
        # The eager results themselves: sorted keys ascend, the segmented sort ascends inside segments.
        s = b["sorted"].cpu().numpy().view(np.uint32)
        assert np.all(s[1:] >= s[:-1])
        g = b["seg_sorted"].cpu().numpy().view(np.uint32)
        for lo, hi in ((3000, 303_000), (400_000, N)):
            assert np.all(g[lo + 1:hi] >= g[lo:hi - 1])


def test_segmented_sort_slot_kinds_under_capture(hip, dev):
    """An eager segmented sort uses its stream's device words for the early exits; a call recorded into a
    graph gets words of its own (the graph may replay on any stream beside eager calls and other
    replays).  Checked through the library's own query, which takes no slot, inside and outside a capture
    on the same stream."""
    import ctypes
    lib = hip.lib()
    handle = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    side = torch.cuda.Stream()
    n = 5000
    keys = torch.arange(n, 0, -1, dtype=torch.int32, device=dev)
    out = torch.empty_like(keys)
    b = torch.tensor([0, 2000], dtype=torch.int32, device=dev)
    e = torch.tensor([2000, n], dtype=torch.int32, device=dev)
    temp = torch.empty(hip.bytes_to_uint_count(hip.segmented_sort_keys_temp_bytes(n, 4)), dtype=torch.int32,
                       device=dev)
    with torch.cuda.stream(side):
        hip.segmented_sort("u32", keys, out, n, 2, b, e, temp=temp)  # eager: the stream's slot
        assert lib.lcpp_hip_internal_segsort_slot_kind(handle()) == 1
    torch.cuda.synchronize()
    seen = []
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        seen.append(lib.lcpp_hip_internal_segsort_slot_kind(handle()))
        hip.segmented_sort("u32", keys, out, n, 2, b, e, temp=temp)
    out.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert seen == [2]
    with torch.cuda.stream(side):
        assert lib.lcpp_hip_internal_segsort_slot_kind(handle()) == 1
    want = torch.cat([torch.arange(n - 1999, n + 1, dtype=torch.int32, device=dev),
                      torch.arange(1, n - 1999, dtype=torch.int32, device=dev)])
    assert torch.equal(out, want)


def test_segmented_sort_graphs_replayed_beside_each_other(hip, orc, dev):
    """Two segmented sorts recorded on one stream into two graphs (one with small and medium segments, one
    with segments that take global passes) replay at the same time on two other streams while an eager
    segmented sort runs on the capture stream: each call has its own device words, so every result is
    exact on every repetition."""
    rng = np.random.default_rng(91)
    n = 300_000
    keys = rng.integers(0, 1 << 32, n, dtype=np.uint64).astype(np.uint32)
    cases = [(np.arange(0, n, 700, dtype=np.uint32), np.minimum(np.arange(0, n, 700) + 700, n).astype(np.uint32)),
             (np.array([0, 100_000], np.uint32), np.array([100_000, n], np.uint32)),
             (np.arange(0, n, 37, dtype=np.uint32), np.minimum(np.arange(0, n, 37) + 37, n).astype(np.uint32))]
    d_keys = torch.from_numpy(keys.view(np.int32)).to(dev)
    outs = [torch.empty_like(d_keys) for _ in cases]
    temps = [torch.empty(hip.bytes_to_uint_count(hip.segmented_sort_keys_temp_bytes(n, 4)), dtype=torch.int32,
                         device=dev) for _ in cases]
    offs = [(torch.from_numpy(b.view(np.int32)).to(dev), torch.from_numpy(e.view(np.int32)).to(dev))
            for b, e in cases]
    call = lambda i: hip.segmented_sort("u32", d_keys, outs[i], n, len(cases[i][0]), offs[i][0], offs[i][1],
                                        temp=temps[i])
    capture = torch.cuda.Stream()
    with torch.cuda.stream(capture):
        call(2)  # an eager call first: the capture stream's slot
    torch.cuda.synchronize()
    graphs = [torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()]
    for i in (0, 1):
        with torch.cuda.graph(graphs[i], stream=capture):
            call(i)
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    want = [orc.segmented_sort(keys, b, e, keys_out=np.zeros(n, np.uint32))[0] for b, e in cases]
    for rep in range(4):
        for o in outs:
            o.zero_()
        torch.cuda.synchronize()
        for i in (0, 1):
            with torch.cuda.stream(streams[i]):
                graphs[i].replay()
        with torch.cuda.stream(capture):
            call(2)
        torch.cuda.synchronize()
        for i in range(3):
            got = outs[i].cpu().numpy().view(np.uint32)
            np.testing.assert_array_equal(got, want[i], err_msg=f"rep {rep} call {i}")
