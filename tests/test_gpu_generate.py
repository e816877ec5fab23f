"""The device workload generator reproduces the oracle's splitmix64 streams bit for bit."""
import numpy as np
import pytest
import torch

from gpu_util import to_host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", range(7))
def test_generate_matches_oracle(hip, orc, dev, kind):
    n, seed, start = 100003, 114521, 12345
    itemsize = np.dtype(orc.GEN_DTYPES[kind]).itemsize
    t = torch.empty(n, dtype=torch.int32 if itemsize == 4 else torch.int64, device=dev)
    hip.generate(kind, t, n, seed, start)
    got = to_host(t, orc.GEN_DTYPES[kind])
    assert np.array_equal(got.view(f"u{itemsize}"), orc.generate(kind, n, seed, start).view(f"u{itemsize}"))
