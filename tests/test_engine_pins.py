"""Pins of the oracle's timestep conditioner (CPU, no GPU).

iro_dit_condition (dit.c:488-530): the sinusoidal embedding computed with
glibc's expf, cosf and sinf in the reference's op order, then three scalar
linears with SiLU between them.  The oracle's composition is compared bit
for bit with the reference's strict build (oracle/_ref) at the model's
shapes; the embedding's constant logf(10000) with libm.
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import HERE, Reference

TDIM, D, COND = 512, 1280, 3840  # TIMESTEP_DIM, MODEL_DIM, COND_DIM of dit.c:12-14


def _ref():
    if not os.path.exists(os.path.join(HERE, "_ref", "libref_strict.so")):
        pytest.skip("reference build absent (oracle/_ref needs the reference sources)")
    return Reference("strict")


def conditioner_weights(seed):
    rng = np.random.default_rng(seed)
    return ((rng.standard_normal((D, TDIM), dtype=np.float32) * 0.05),
            (rng.standard_normal((D, D), dtype=np.float32) * 0.03),
            (rng.standard_normal((COND, D), dtype=np.float32) * 0.03))


def test_log_theta_constant_is_libm_logf():
    libm = ctypes.CDLL("libm.so.6")
    libm.logf.argtypes = [ctypes.c_float]
    libm.logf.restype = ctypes.c_float
    assert np.float32(libm.logf(10000.0)) == np.float32(float.fromhex("0x1.26bb1cp+3"))


def test_condition_equals_reference_strict_build(oracle):
    ref = _ref()
    w0, w1, w2 = conditioner_weights(11)
    t = np.array([1.0, 0.5, 1e-3, 0.999, 0.0, 1.0 / 3.0], np.float32)
    want = ref.dit_condition(w0, w1, w2, t)
    got = oracle.dit_condition(w0, w1, w2, t)
    assert np.array_equal(got.view(np.int32), want.view(np.int32))
    # A plausible slip, sin before cos in the embedding, is caught.
    w0_swapped = np.ascontiguousarray(np.concatenate([w0[:, TDIM // 2:], w0[:, :TDIM // 2]], 1))
    assert not np.array_equal(oracle.dit_condition(w0_swapped, w1, w2, t), want)
