"""Synthetic benchmark inputs that are built on the host (the device generator, lcpp_hip.generate, covers
the flat key/value streams).

zipf_csr: the CSR matrix of the SpMV benchmark.  Row lengths follow a Zipf law with exponent s,
truncated to [1, max_len] and drawn by inverse CDF; each row's column indices are distinct, uniform
over [0, cols) and sorted; A values and x are uniform in [-1, 1).  With s = 1.5 and max_len = 4096 the
mean row length is about 49, so 2^20 rows hold about 51.4 M nonzeros (the truncated law is kept as is;
the nonzero count is reported with every measurement).
"""
from __future__ import annotations

import numpy as np


def zipf_lengths(rng: np.random.Generator, rows: int, s: float = 1.5, max_len: int = 4096) -> np.ndarray:
    k = np.arange(1, max_len + 1, dtype=np.float64)
    cdf = np.cumsum(k ** -s)
    cdf /= cdf[-1]
    u = rng.random(rows)
    return (np.searchsorted(cdf, u, side="right") + 1).clip(1, max_len).astype(np.int64)


def zipf_csr(rows: int, cols: int, seed: int, s: float = 1.5, max_len: int = 4096, value_dtype=np.float32):
    """Returns (values, row_offsets int32, column_indices int32, x, nnz)."""
    rng = np.random.default_rng(seed)
    lengths = np.minimum(zipf_lengths(rng, rows, s, max_len), cols)
    offsets = np.zeros(rows + 1, dtype=np.int64)
    np.cumsum(lengths, out=offsets[1:])
    nnz = int(offsets[-1])
    if nnz >= 2 ** 31:
        raise ValueError("too many nonzeros for 32-bit offsets")
    # Draw with replacement, sort within rows, then redraw every row that came out with a duplicate
    # column using exact sampling without replacement.
    keys = np.repeat(np.arange(rows, dtype=np.int64) * cols, lengths)
    keys += rng.integers(0, cols, nnz, dtype=np.int64)
    keys.sort()
    dup_rows = np.unique(keys[1:][keys[1:] == keys[:-1]] // cols)
    columns = (keys % cols).astype(np.int32)
    del keys
    for r in dup_rows:
        b, e = int(offsets[r]), int(offsets[r + 1])
        columns[b:e] = np.sort(rng.choice(cols, e - b, replace=False)).astype(np.int32)
    values = rng.uniform(-1.0, 1.0, nnz).astype(value_dtype)
    x = rng.uniform(-1.0, 1.0, cols).astype(value_dtype)
    return values, offsets.astype(np.int32), columns, x, nnz
