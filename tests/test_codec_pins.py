"""Pins of the oracle's decoder pieces around Conv7 (CPU, no GPU).

glibc's sinf and cosf are restated and checked on every float input against
libm itself; the snake forms (dacvae.c:803-931), the residual unit
(run_residual_int8, dacvae.c:934-1018) and the int8 core of
iro_dacvae_decode (dacvae.c:1213-1277, read through its own trace observer)
are checked bit for bit against the reference's strict build (oracle/_ref).
Each pin is shown to discriminate: the neighbouring form of the same
formula (quotient for reciprocal, one plane for two) fails it.

The fast build's snake calls libmvec's vectorised sinf, which is not
restated: that convention is parity unpinned here and is checked only
within a stated tolerance.
"""
import ctypes
import os

import numpy as np
import pytest

import codec_params as cp
from oracle import GCC_FASTMATH, HERE, STRICT, Reference

REF_DIR = os.path.join(HERE, "_ref")


def _ref(flavour):
    if not os.path.exists(os.path.join(REF_DIR, f"libref_{flavour}.so")):
        pytest.skip("reference build absent (oracle/_ref needs the reference sources)")
    return Reference(flavour)


def _ndiff(a, b):
    return int((np.ascontiguousarray(a, np.float32).view(np.int32) !=
                np.ascontiguousarray(b, np.float32).view(np.int32)).sum())


def _snake_inputs(T, C, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, C), dtype=np.float32) * 3).astype(np.float32)
    x[0, :4] = [0.0, 1e-30, -0.0, 200.0]  # the tiny, signed-zero and |a x| > 120 branches
    if T > 1:
        x[1, :2] = [1e4, -3e3]
    alpha = (rng.random(C, dtype=np.float32) * 2 + 0.05).astype(np.float32)
    bias = (rng.standard_normal(C, dtype=np.float32) * 0.1).astype(np.float32)
    return x, alpha, bias


def test_sinf_cosf_restatement_equals_libm_on_every_float(oracle):
    assert oracle.sincosf_mismatches(0) == 0
    assert oracle.sincosf_mismatches(1) == 0


def test_sinf_restatement_special_values(oracle):
    f = oracle.lib.orc_sinf
    g = oracle.lib.orc_cosf
    assert f(0.0) == 0.0 and np.signbit(np.float32(f(-0.0)))
    assert g(0.0) == 1.0
    assert np.isnan(f(float("inf"))) and np.isnan(g(float("-inf")))
    libm = ctypes.CDLL("libm.so.6")
    libm.sinf.argtypes = libm.cosf.argtypes = [ctypes.c_float]
    libm.sinf.restype = libm.cosf.restype = ctypes.c_float
    for v in (0.5, 1.0, 3.0, 100.0, 1e6, 3e38):
        assert f(v) == libm.sinf(v) and g(v) == libm.cosf(v)


@pytest.mark.parametrize("C", [96, 768, 1536, 1540])
def test_snake_forms_equal_reference_strict_build(oracle, C):
    ref = _ref("strict")
    x, alpha, bias = _snake_inputs(37, C, C)
    # iro_snake_forward out of place and in place: reciprocal up to 1536.
    want = ref.snake(x, alpha)
    assert _ndiff(oracle.snake(STRICT, x, alpha), want) == 0
    assert _ndiff(ref.snake(x, alpha, inplace=True), want) == 0
    # snake_bias_forward: reciprocal only in place and up to 1536.
    assert _ndiff(oracle.snake(STRICT, x, alpha, bias=bias, inv_form=C <= 1536),
                  ref.snake_bias(x, bias, alpha, inplace=True)) == 0
    assert _ndiff(oracle.snake(STRICT, x, alpha, bias=bias, inv_form=False),
                  ref.snake_bias(x, bias, alpha, inplace=False)) == 0
    # The pin discriminates: the other division form differs somewhere.
    if C <= 1536:
        assert _ndiff(oracle.snake(STRICT, x, alpha, inv_form=False), want) > 0


@pytest.mark.parametrize("C", [96, 1536])
def test_snake_fast_within_tolerance_of_fast_build(oracle, C):
    """Parity unpinned (libmvec sinf): the fast form stays within 4 ulp of the
    terms it adds."""
    ref = _ref("fast")
    x, alpha, bias = _snake_inputs(200, C, C + 1)
    got = oracle.snake(GCC_FASTMATH, x, alpha).astype(np.float64)
    want = ref.snake(x, alpha).astype(np.float64)
    scale = np.abs(x.astype(np.float64)) + 1.0 / alpha.astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * np.finfo(np.float32).eps * scale)


UNITS = [(96, 300, 9, 3), (96, 300, 1, 2), (192, 120, 3, 3), (384, 50, 1, 0), (96, 5, 9, 3),
         (768, 24, 3, 1)]


@pytest.mark.parametrize("C,T,dil,stage", UNITS)
def test_residual_unit_equals_reference_strict_build(oracle, C, T, dil, stage):
    ref = _ref("strict")
    rng = np.random.default_rng(C + T + dil)
    u = cp.residual_unit(rng, C, dil)
    x = rng.standard_normal((T, C), dtype=np.float32)
    want = ref.residual_unit(x, u, stage)
    two = stage == 3  # the default policy's stage mask (dacvae.c:64-72)
    assert _ndiff(oracle.residual_unit(STRICT, x, u, two, two), want) == 0
    if T > 20:
        assert _ndiff(oracle.residual_unit(STRICT, x, u, not two, not two), want) > 0


@pytest.mark.parametrize("frames", [1, 2])
def test_decode_core_equals_reference_decode_strict_build(oracle, frames):
    ref = _ref("strict")
    p = cp.decoder(5 + frames)
    latent = np.random.default_rng(9).standard_normal((frames, cp.CODEBOOK), dtype=np.float32)
    state, core, _ = ref.decode_trace(cp.reference_order(p), latent)
    got = oracle.decode_core(STRICT, state, p)
    assert got.shape == core.shape == (frames * 1920, cp.FINAL)
    assert _ndiff(got, core) == 0
    # All residual groups in every stage change the result.
    assert _ndiff(oracle.decode_core(STRICT, state, p, residual_stages=15), core) > 0
