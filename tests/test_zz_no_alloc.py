"""lcpp_hip_scan_exclusive_sum_u32_noalloc (no temp argument, no allocation) through the C-ABI against the
existing ExclusiveSum entry point with caller temp storage: bit-exact on two calls in a row, the second on
a smaller input (the static words keep the first call's contents, which the second must clear); recorded
into a graph (with and without an eager call on the device first) and replayed on fresh inputs; a clear
error above the static scratch's maximum."""
import ctypes

import pytest
import torch

from gpu_util import log

pytestmark = pytest.mark.gpu


def _noalloc(lib, a, out, n, stream):
    return lib.lcpp_hip_scan_exclusive_sum_u32_noalloc(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                                                       n, ctypes.c_void_p(stream))


def test_no_alloc_exclusive_sum_under_graph_capture(hip, dev):
    """Recorded into a torch CUDAGraph and replayed three times on fresh inputs, with eager work and
    synchronisations between replays, each replay checked against the entry point with temp storage.  In a
    process that has made no call on the device yet, the first capture gets a clear error (the scratch is
    looked up outside capture only) and records nothing; an eager call with n == 0 then does the lookup."""
    lib = hip.lib()
    n = 3_000_017
    a = torch.empty(n, dtype=torch.int32, device=dev)
    got = torch.empty_like(a)
    want = torch.empty_like(a)
    hip.generate(hip.GEN_U32_HI, a, n, 80)
    torch.cuda.synchronize()
    statuses = []
    for attempt in range(2):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            statuses.append(_noalloc(lib, a, got, n, torch.cuda.current_stream().cuda_stream))
        if statuses[-1] == hip.OK:
            break
        log(f"no-alloc capture before any eager call: status {statuses[-1]}")
        assert statuses[-1] == hip.ERR_UNSUPPORTED
        assert b"outside capture" in lib.lcpp_hip_last_error()
        assert lib.lcpp_hip_scan_exclusive_sum_u32_noalloc(None, None, 0,
                                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == hip.OK
    assert statuses[-1] == hip.OK, lib.lcpp_hip_last_error()
    for rep, seed in enumerate((81, 82, 83)):
        log(f"no-alloc graph replay {rep}")
        hip.generate(hip.GEN_U32_HI, a, n, seed)  # full 32-bit words: the sum wraps
        hip.scan_sum("u32", a, want, n)
        got.fill_(0x7E7E7E7E)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), rep


def test_no_alloc_exclusive_sum_matches_entry_point_with_temp(hip, dev):
    lib = hip.lib()
    stream = torch.cuda.current_stream().cuda_stream
    for n, seed in ((5_000_011, 71), (70_001, 72)):  # the second call is smaller
        log(f"no-alloc ExclusiveSum n={n}")
        a = torch.empty(n, dtype=torch.int32, device=dev)
        hip.generate(hip.GEN_U32_HI, a, n, seed)  # full 32-bit words: the sum wraps
        want = torch.empty_like(a)
        hip.scan_sum("u32", a, want, n)  # lcpp_hip_scan_exclusive_sum_u32 with caller temp storage
        got = torch.full_like(a, 0x7E7E7E7E)
        st = _noalloc(lib, a, got, n, stream)
        assert st == hip.OK, lib.lcpp_hip_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_no_alloc_exclusive_sum_on_a_side_stream(hip, dev):
    """The array is the stream's device's; a call on a non-default stream matches the temp-storage form."""
    lib = hip.lib()
    n = 1_000_003
    a = torch.empty(n, dtype=torch.int32, device=dev)
    hip.generate(hip.GEN_U32_HI, a, n, 90)
    want = torch.empty_like(a)
    hip.scan_sum("u32", a, want, n)
    got = torch.full_like(a, 0x7E7E7E7E)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=dev)
    assert _noalloc(lib, a, got, n, side.cuda_stream) == hip.OK, lib.lcpp_hip_last_error()
    side.synchronize()
    assert torch.equal(got, want)


def test_no_alloc_exclusive_sum_rejects_sizes_above_its_maximum(hip, dev):
    lib = hip.lib()
    assert lib.lcpp_hip_scan_exclusive_sum_u32_noalloc(None, None, (1 << 30) + 1, None) == hip.ERR_INVALID_ARGUMENT
    assert b"static scratch" in lib.lcpp_hip_last_error()
    assert lib.lcpp_hip_scan_exclusive_sum_u32_noalloc(None, None, 0, None) == hip.OK
