"""lcpp_hip_scan_exclusive_sum_u32_noalloc (no temp argument, no allocation) through the C-ABI against the
existing ExclusiveSum entry point with caller temp storage: bit-exact on two calls in a row, the second on
a smaller input (the static words keep the first call's contents, which the second must clear), and a
clear error above the static scratch's maximum."""
import ctypes

import pytest
import torch

from gpu_util import log

pytestmark = pytest.mark.gpu


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
        st = lib.lcpp_hip_scan_exclusive_sum_u32_noalloc(ctypes.c_void_p(a.data_ptr()),
                                                         ctypes.c_void_p(got.data_ptr()), n,
                                                         ctypes.c_void_p(stream))
        assert st == hip.OK, lib.lcpp_hip_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_no_alloc_exclusive_sum_rejects_sizes_above_its_maximum(hip, dev):
    lib = hip.lib()
    assert lib.lcpp_hip_scan_exclusive_sum_u32_noalloc(None, None, (1 << 30) + 1, None) == hip.ERR_INVALID_ARGUMENT
    assert b"static scratch" in lib.lcpp_hip_last_error()
    assert lib.lcpp_hip_scan_exclusive_sum_u32_noalloc(None, None, 0, None) == hip.OK
