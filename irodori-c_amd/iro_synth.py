"""Seeded synthetic inputs for the int8 W8A8 workloads.

Every value is a deterministic function of integers and IEEE-754
+, -, *, / and sqrt (no libm, no SIMD-order-dependent reductions), so the
same seed gives the same bits on any host: the inputs a test builds here and
on a GPU host are identical, and committed digests of outputs stay valid.

`gauss` is an Irwin-Hall sum of twelve 16-bit uniforms from numpy's PCG64
stream (mean 0, variance 1, support +-6): a Gaussian stand-in whose bits do
not depend on libm.
"""
from __future__ import annotations

import numpy as np

_CHUNK = 1 << 20


def gauss(seed: int, shape, std: float = 1.0) -> np.ndarray:
    shape = tuple(int(s) for s in np.atleast_1d(shape))
    n = int(np.prod(shape)) if shape else 1
    bg = np.random.PCG64(seed)
    out = np.empty(n, np.float32)
    for off in range(0, n, _CHUNK):
        m = min(_CHUNK, n - off)
        raw = bg.random_raw(3 * m).astype("<u8")
        # integer sum: exact, so independent of numpy's reduction order
        s = raw.view("<u2").reshape(m, 12).sum(axis=1, dtype=np.int64)
        # sum of 12 U(0,1) draws (l + 1/2) / 65536, minus the mean 6
        z = (s.astype(np.float64) + 6.0) / 65536.0 - 6.0
        out[off:off + m] = (z * float(std)).astype(np.float32)
    return out.reshape(shape)


def rms_rows(x: np.ndarray) -> np.ndarray:
    """Scale each row to unit RMS (RMSNorm without weight, eps 0), with a
    fixed left-to-right float64 accumulation per row."""
    x = np.asarray(x, np.float32)
    acc = np.zeros(x.shape[0], np.float64)
    xd = x.astype(np.float64)
    for k in range(x.shape[1]):
        acc += xd[:, k] * xd[:, k]
    rms = np.sqrt(acc / x.shape[1])
    rms[rms == 0] = 1.0
    return (xd / rms[:, None]).astype(np.float32)


def heavy_tail(x: np.ndarray, seed: int, frac: float = 0.01, factor: float = 20.0) -> np.ndarray:
    """Multiply a seeded `frac` of the entries by `factor`."""
    x = np.array(x, np.float32, copy=True)
    bg = np.random.PCG64(seed)
    u = bg.random_raw(x.size) >> np.uint64(40)  # 24-bit uniforms
    mask = u < np.uint64(int(frac * (1 << 24)))
    flat = x.reshape(-1)
    flat[mask] = flat[mask] * np.float32(factor)
    return x
