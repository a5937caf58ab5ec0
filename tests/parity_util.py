"""Shared helpers for the parity tests (HIP path vs the oracle)."""
from __future__ import annotations

import numpy as np


def bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.int32) if a.dtype == np.float32 else a


def assert_bits_equal(got, want, what):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.dtype == np.float32:
        bad = bits(got) != bits(want)
    else:
        bad = got != want
    n = int(bad.sum())
    if n:
        idx = np.argwhere(bad)[:5]
        samples = [(tuple(i), got[tuple(i)], want[tuple(i)]) for i in idx]
        raise AssertionError(f"{what}: {n} of {got.size} differ, e.g. {samples}")


def rel_err(got, want, floor_frac=1e-3):
    """|got - want| / max(|want|, floor_frac * rms(want)), elementwise."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = float(np.sqrt(np.mean(want * want))) if want.size else 0.0
    den = np.maximum(np.abs(want), floor_frac * rms + 1e-30)
    return np.abs(got - want) / den
