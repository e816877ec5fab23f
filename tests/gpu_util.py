"""Host <-> device helpers for the GPU parity tests (torch tensors carry device memory only)."""
import numpy as np
import torch

_STORAGE = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}


def to_dev(a: np.ndarray, device="cuda:0") -> torch.Tensor:
    """Copies a numpy array to the device, bit for bit (unsigned types travel as same-width signed)."""
    a = np.ascontiguousarray(a)
    if a.dtype in (np.float32, np.float64):
        return torch.from_numpy(a.copy()).to(device)
    return torch.from_numpy(a.view(np.dtype(f"i{a.dtype.itemsize}")).copy()).to(device)


def empty_dev(n: int, itemsize: int, device="cuda:0") -> torch.Tensor:
    return torch.empty(max(n, 1), dtype=_STORAGE[itemsize], device=device)


def fill_dev(n: int, itemsize: int, value: int, device="cuda:0") -> torch.Tensor:
    return torch.full((max(n, 1),), value, dtype=_STORAGE[itemsize], device=device)


def to_host(t: torch.Tensor, dtype, n: int | None = None) -> np.ndarray:
    torch.cuda.synchronize()
    a = t.detach().cpu().numpy()
    if n is not None:
        a = a[:n]
    return a.view(dtype)


def log(msg: str) -> None:
    print(msg, flush=True)
