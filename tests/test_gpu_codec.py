"""Parity of the decoder's int8 path around Conv7 on the GPU against the
oracle: glibc sinf / cosf on every float input, the snake forms
(dacvae.c:803-931), the residual unit (run_residual_int8,
dacvae.c:934-1018), the decoder's int8 weight set (dacvae.c:228-262) and the
int8 core of iro_dacvae_decode (dacvae.c:1221-1277) at the reference's
channel counts.  The oracle's pieces are pinned bit for bit to the
reference's strict build on the CPU; the fast convention's snake is parity
unpinned (libmvec sinf) and is compared with the oracle's own fast form.
"""
import numpy as np
import pytest

import codec_params as cp
from parity_util import assert_bits_equal

pytestmark = pytest.mark.gpu


def test_sincosf_digests_equal_glibc(ctx_strict, oracle):
    s, c = ctx_strict.selfcheck_sincosf()
    assert s == oracle.sincosf_digest(0), "device sinf differs from glibc on some float"
    assert c == oracle.sincosf_digest(1), "device cosf differs from glibc on some float"


def _snake_inputs(T, C, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((T, C), dtype=np.float32) * 3).astype(np.float32)
    x[0, :4] = [0.0, 1e-30, -0.0, 200.0]
    if T > 1:
        x[1, :2] = [1e4, -3e3]
    alpha = (rng.random(C, dtype=np.float32) * 2 + 0.05).astype(np.float32)
    bias = (rng.standard_normal(C, dtype=np.float32) * 0.1).astype(np.float32)
    return x, alpha, bias


@pytest.mark.parametrize("T,C", [(37, 96), (64, 768), (9, 1536), (5, 1540), (1, 4),
                                 (4000, 192)])
def test_snake_forms(ctx, oracle, T, C):
    conv = ctx.convention
    x, alpha, bias = _snake_inputs(T, C, T + C)
    xd, ad, bd = ctx.to_device(x), ctx.to_device(alpha), ctx.to_device(bias)
    y = ctx.empty((T, C), np.float32)
    ctx.snake(xd, T, C, ad, y)
    want = oracle.snake(conv, x, alpha)
    assert_bits_equal(y.numpy(), want, "snake out of place")
    xi = ctx.to_device(x)
    ctx.snake(xi, T, C, ad, xi)
    assert_bits_equal(xi.numpy(), want, "snake in place")
    # snake_bias: the reciprocal only in place up to 1536 channels.
    ctx.snake_bias(xd, T, C, bd, ad, y)
    assert_bits_equal(y.numpy(), oracle.snake(conv, x, alpha, bias=bias, inv_form=False),
                      "snake_bias out of place")
    xi = ctx.to_device(x)
    ctx.snake_bias(xi, T, C, bd, ad, xi)
    assert_bits_equal(xi.numpy(), oracle.snake(conv, x, alpha, bias=bias, inv_form=C <= 1536),
                      "snake_bias in place")


def test_snake_refuses_unaligned_channels(ctx_strict):
    import iro_hip
    x = ctx_strict.to_device(np.ones((3, 6), np.float32))
    a = ctx_strict.to_device(np.ones(6, np.float32))
    with pytest.raises(iro_hip.HipError):
        ctx_strict.snake(x, 3, 6, a, x)


# The 1x1 with its in-place snake_bias and row quantization is one kernel
# for C % 32 == 0 up to 192 channels (two planes up to 160; half a wavefront
# per row up to 128); above, the snake runs inside the 1x1's quantizer up to
# 1536 channels (one row per half wave up to 128, 1..6 column chunks above)
# and as its own quotient-form pass beyond.
UNITS = [(96, 300, 9, True), (96, 300, 1, False), (192, 120, 3, True), (384, 50, 1, False),
         (96, 5, 9, True), (768, 24, 3, False), (96, 20000, 9, True), (4, 33, 1, True),
         (136, 40, 3, False), (1280, 7, 1, True), (1536, 6, 1, True), (1540, 4, 3, False),
         (192, 70, 9, False), (128, 66, 1, True), (64, 65, 3, False), (160, 40, 1, True),
         (160, 129, 3, False)]


@pytest.mark.parametrize("C,T,dil,two", UNITS)
def test_residual_unit(ctx, oracle, C, T, dil, two):
    conv = ctx.convention
    rng = np.random.default_rng(C + T + dil)
    u = cp.residual_unit(rng, C, dil)
    x = rng.standard_normal((T, C), dtype=np.float32)
    w0 = ctx.weight(ctx.to_device(u["w0"]), C, 7 * C)
    w1 = ctx.weight(ctx.to_device(u["w1"]), C, C)
    out = ctx.empty((T, C), np.float32)
    ctx.dacvae_residual(ctx.to_device(x), T, C, w0, ctx.to_device(u["alpha0"]),
                        ctx.to_device(u["b0"]), ctx.to_device(u["alpha1"]), dil, w1,
                        ctx.to_device(u["b1"]), two, two, out)
    assert_bits_equal(out.numpy(), oracle.residual_unit(conv, x, u, two, two), "residual unit")


@pytest.mark.parametrize("two", [True, False], ids=["two-plane", "one-plane"])
@pytest.mark.parametrize("C,T", [(96, 50), (192, 30), (768, 9)])
def test_residual_unit_large_hidden(ctx, oracle, C, T, two):
    """Inputs scaled so some sines of the fused snake take sinf's |y| >= 120
    path next to ordinary ones in the same four columns."""
    conv = ctx.convention
    rng = np.random.default_rng(7 * C + T)
    u = cp.residual_unit(rng, C, 3)
    x = (rng.standard_normal((T, C), dtype=np.float32) * 400).astype(np.float32)
    w0 = ctx.weight(ctx.to_device(u["w0"]), C, 7 * C)
    w1 = ctx.weight(ctx.to_device(u["w1"]), C, C)
    out = ctx.empty((T, C), np.float32)
    ctx.dacvae_residual(ctx.to_device(x), T, C, w0, ctx.to_device(u["alpha0"]),
                        ctx.to_device(u["b0"]), ctx.to_device(u["alpha1"]), 3, w1,
                        ctx.to_device(u["b1"]), two, two, out)
    want = oracle.residual_unit(conv, x, u, two, two)
    assert_bits_equal(out.numpy(), want, "residual unit, large hidden values")


@pytest.mark.parametrize("two", [True, False], ids=["two-plane", "one-plane"])
@pytest.mark.parametrize("C,T", [(32, 90), (64, 70), (96, 70), (192, 45), (256, 33), (160, 40)])
def test_residual_unit_snake_quantizer_path(ctx, oracle, C, T, two):
    """Conv mode 1 routes the unit's 1x1 through the row quantizer that
    applies the snake_bias itself (eight lanes per row where the channels
    are a multiple of 32 up to 256, one wavefront or half of one per row
    otherwise)."""
    conv = ctx.convention
    rng = np.random.default_rng(11 * C + T)
    u = cp.residual_unit(rng, C, 3)
    x = rng.standard_normal((T, C), dtype=np.float32)
    w0 = ctx.weight(ctx.to_device(u["w0"]), C, 7 * C)
    w1 = ctx.weight(ctx.to_device(u["w1"]), C, C)
    out = ctx.empty((T, C), np.float32)
    ctx.set_gemm_tile(-6, 1)
    try:
        ctx.dacvae_residual(ctx.to_device(x), T, C, w0, ctx.to_device(u["alpha0"]),
                            ctx.to_device(u["b0"]), ctx.to_device(u["alpha1"]), 3, w1,
                            ctx.to_device(u["b1"]), two, two, out)
    finally:
        ctx.set_gemm_tile(-6, 2)
    want = oracle.residual_unit(conv, x, u, two, two)
    assert_bits_equal(out.numpy(), want, "residual unit, snake in the row quantizer")


def test_residual_unit_long_384_modes_agree(ctx):
    """At 384 channels on 16384 steps or more the unit's Conv7 takes the
    snake pass with row ranges and the GEMM that codes its own rows; its
    output equals the im2col form's (conv mode 1), which the oracle tests
    above pin at shorter lengths."""
    C, T, dil = 384, 16500, 3
    rng = np.random.default_rng(C + T)
    u = cp.residual_unit(rng, C, dil)
    x = rng.standard_normal((T, C), dtype=np.float32)
    w0 = ctx.weight(ctx.to_device(u["w0"]), C, 7 * C)
    w1 = ctx.weight(ctx.to_device(u["w1"]), C, C)
    xd = ctx.to_device(x)
    outs = []
    for mode in (2, 1):
        ctx.set_gemm_tile(-6, mode)
        try:
            out = ctx.empty((T, C), np.float32)
            ctx.dacvae_residual(xd, T, C, w0, ctx.to_device(u["alpha0"]), ctx.to_device(u["b0"]),
                                ctx.to_device(u["alpha1"]), dil, w1, ctx.to_device(u["b1"]),
                                False, False, out)
            outs.append(out.numpy())
        finally:
            ctx.set_gemm_tile(-6, 2)
    assert_bits_equal(outs[0], outs[1], "residual unit, GEMM codes vs im2col")


def _decoder(ctx, seed):
    import iro_hip
    p = cp.decoder(seed)
    d = iro_hip.DACVAE(ctx, cp.to_device(ctx, p))
    return p, d


@pytest.mark.parametrize("frames", [1, 2, 5])
def test_decode_core(ctx, oracle, frames):
    conv = ctx.convention
    p, d = _decoder(ctx, 30 + frames)
    try:
        # The quantizer_out state: any [frames, 1024] fp32 rows.
        state = np.random.default_rng(frames).standard_normal((frames, cp.LATENT),
                                                              dtype=np.float32)
        T = d.output_frames(frames)
        assert T == frames * 1920
        out = ctx.empty((T, cp.FINAL), np.float32)
        d.decode_int8(ctx.to_device(state), frames, out)
        assert_bits_equal(out.numpy(), oracle.decode_core(conv, state, p), "decoder core")
    finally:
        d.destroy()


def test_decoder_int8_bytes(ctx_strict):
    """IroDACVAEInt8.bytes: iro_int8_weight_bytes (N K + 8 N) over the 26 weights."""
    p, d = _decoder(ctx_strict, 3)
    try:
        want = cp.CHANNELS * 7 * cp.LATENT + 8 * cp.CHANNELS
        for st in p["stages"]:
            n = st["kernel"] * st["c_out"]
            want += n * st["c_in"] + 8 * n
            C = st["c_out"]
            want += 3 * (C * 7 * C + 8 * C + C * C + 8 * C)
        assert d.nbytes() == want
    finally:
        d.destroy()
