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


def test_segmented_sort_takes_no_stream_slot_under_capture(hip, dev):
    """An eager segmented sort uses a per-stream device word for its early exits; a call recorded into a
    graph must not (the graph may replay on any stream beside eager calls and other replays), so its
    kernels run without the early exits.  Checked through the library's own query, inside and outside
    a capture on the same stream."""
    import ctypes
    lib = hip.lib()
    handle = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert lib.lcpp_hip_internal_segsort_uses_stream_slot(handle()) == 1
    x = torch.ones(5000, dtype=torch.int32, device=dev)
    y = torch.empty_like(x)
    temp = torch.empty(hip.bytes_to_uint_count(hip.scan_temp_bytes(5000, 4)), dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    seen = []
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        seen.append(lib.lcpp_hip_internal_segsort_uses_stream_slot(handle()))
        hip.scan_sum("u32", x, y, 5000, temp=temp)
    graph.replay()
    torch.cuda.synchronize()
    assert seen == [0]
    with torch.cuda.stream(side):
        assert lib.lcpp_hip_internal_segsort_uses_stream_slot(handle()) == 1
    assert torch.equal(y, torch.arange(5000, dtype=torch.int32, device=dev))
