"""Parity of the int8 Conv1d (dacvae.c:543-688) on the GPU against the oracle.

Edge cases follow the reference's window logic: output rows whose taps
fall before 0 or after T-1 (padding holds the zero point and does not widen
the row range), dilation, stride > 1, all-zero windows (scale 1), channel
counts that are not a multiple of 4, and the fixed-scale second plane of the
last decoder stage (dacvae.c:637-663).  The BASELINE shapes run at full size.
"""
import numpy as np
import pytest

from iro_synth import gauss
from parity_util import assert_bits_equal

pytestmark = pytest.mark.gpu

CASES = [  # T, C, N, kernel, stride, dilation, padding
    (50, 16, 24, 7, 1, 1, 3),
    (50, 16, 24, 7, 1, 3, 9),
    (40, 8, 8, 7, 2, 1, 3),
    (64, 32, 16, 3, 1, 9, 9),
    (33, 6, 10, 7, 1, 1, 3),
    (300, 96, 96, 7, 1, 9, 27),
    (5, 4, 4, 7, 1, 1, 3),
    # kernel 7 with C % 32 == 0, 64 <= C <= 256: the GEMM that codes its own rows
    (50, 64, 64, 7, 1, 1, 3),
    (70, 80, 40, 7, 2, 2, 6),
    (130, 64, 300, 7, 1, 5, 15),
    (100, 128, 256, 7, 1, 1, 3),
    (90, 96, 96, 7, 1, 2, 0),
    (3, 192, 192, 7, 1, 9, 27),
]


def _conv(ctx, oracle, T, C, N, k, st, dil, pad, residual, seed, zero_band=True):
    conv = ctx.convention
    x = gauss(seed, (T, C))
    if zero_band and T > 30:
        x[10:30] = 0.0  # all-zero windows
    w = gauss(seed + 1, (N, k * C), 0.02)
    b = gauss(seed + 2, (N,), 0.01)
    W = ctx.weight(ctx.to_device(w), N, k * C)
    To = oracle.conv_out_len(T, k, st, dil, pad)
    yd = ctx.empty((To, N), np.float32)
    got_len = ctx.conv1d(ctx.to_device(x), T, C, W, k, st, dil, pad, ctx.to_device(b), residual,
                         yd)
    assert got_len == To
    yo, _, _, _ = oracle.conv1d(conv, x, *oracle.weight_quantize(conv, w), k, st, dil, pad,
                                bias=b, residual=residual)
    return yd.numpy(), yo


@pytest.mark.parametrize("T,C,N,k,st,dil,pad", CASES)
@pytest.mark.parametrize("residual", [0, 1], ids=["one-plane", "two-plane"])
def test_conv_small(ctx, oracle, T, C, N, k, st, dil, pad, residual):
    got, want = _conv(ctx, oracle, T, C, N, k, st, dil, pad, residual, 70 + T + C)
    assert_bits_equal(got, want, "conv output")


@pytest.mark.parametrize("mode,cols", [(0, 0), (1, 0), (2, 0), (2, 128), (2, 256)],
                         ids=["two-pass", "one-pass", "gemm-codes", "gemm-codes-128",
                              "gemm-codes-256"])
@pytest.mark.parametrize("residual", [0, 1], ids=["one-plane", "two-plane"])
def test_conv7_modes_agree(ctx, oracle, mode, cols, residual):
    """Each kernel-7 form (two-pass im2col, one-pass im2col, the GEMM that
    codes its own rows with either column tile) gives the reference's
    output."""
    ctx.set_gemm_tile(-6, mode)
    ctx.set_gemm_tile(-8, cols)
    try:
        got, want = _conv(ctx, oracle, 2000, 96, 256, 7, 1, 3, 9, residual, 55)
    finally:
        ctx.set_gemm_tile(-6, 2)
        ctx.set_gemm_tile(-8, 0)
    assert_bits_equal(got, want, "conv output")


@pytest.mark.parametrize("T,C,N", [(65600, 320, 256), (16500, 384, 384)],
                         ids=["C320-T65600-256cols", "C384-T16500"])
def test_conv7_gemm_codes_wide_long(ctx, T, C, N):
    """Above 256 channels the GEMM that codes its own rows runs on long
    inputs only (384 channels from 16384 steps, wider from 65536); its
    output equals the one-pass im2col form's, which the oracle tests above
    pin."""
    x = gauss(31, (T, C))
    x[100:140] = 0.0
    w = gauss(32, (N, 7 * C), 0.02)
    b = gauss(33, (N,), 0.01)
    W = ctx.weight(ctx.to_device(w), N, 7 * C)
    xd, bd = ctx.to_device(x), ctx.to_device(b)
    outs = []
    for mode in (2, 1):
        ctx.set_gemm_tile(-6, mode)
        try:
            yd = ctx.empty((T, N), np.float32)
            ctx.conv1d(xd, T, C, W, 7, 1, 3, 9, bd, 0, yd)
            outs.append(yd.numpy())
        finally:
            ctx.set_gemm_tile(-6, 2)
    assert_bits_equal(outs[0], outs[1], "conv output, GEMM codes vs im2col")


@pytest.mark.parametrize("T,C,N,dil,pad", [(24000, 512, 512, 1, 3), (6000, 1024, 256, 3, 9)],
                         ids=["cfg4-T24000-C512", "cfg4-T6000-C1024-dil3"])
def test_conv_baseline_shapes(ctx, oracle, T, C, N, dil, pad):
    got, want = _conv(ctx, oracle, T, C, N, 7, 1, dil, pad, 0, 90, zero_band=False)
    assert_bits_equal(got, want, "conv output")


# (T_in, C_in, C_out, kernel, stride, padding, output_padding); the first
# four are the decoder's upsampling geometry at its rates 12/10/8/2
# (dacvae.c:150-160, 177-179) on short inputs, the last is stage 0 at full
# width on 200 latent frames.
CONVT_CASES = [(37, 48, 16, 24, 12, 6, 0), (20, 40, 24, 20, 10, 5, 0), (31, 32, 8, 16, 8, 4, 0),
               (50, 24, 12, 4, 2, 1, 0), (9, 16, 8, 6, 3, 2, 1), (1, 8, 4, 4, 2, 1, 0),
               (13, 12, 20, 3, 1, 0, 0), (11, 8, 8, 2, 3, 0, 2), (200, 1536, 768, 24, 12, 6, 0)]


@pytest.mark.parametrize("T,Ci,Co,k,st,pad,opad", CONVT_CASES)
@pytest.mark.parametrize("residual", [0, 1], ids=["one-plane", "two-plane"])
def test_convtranspose(ctx, oracle, T, Ci, Co, k, st, pad, opad, residual):
    conv = ctx.convention
    x = gauss(80 + T, (T, Ci))
    if T > 8:
        x[3:6] = 0.0
    w_export = gauss(81 + T, (Ci, k * Co), 0.02)  # [C_in, kernel, C_out]
    b = gauss(82 + T, (Co,), 0.01)
    W = ctx.weight(ctx.to_device(w_export), k * Co, Ci, transposed=True)
    To = oracle.convt_out_len(T, k, st, pad, opad)
    yd = ctx.empty((To, Co), np.float32)
    got_len = ctx.convtranspose1d(ctx.to_device(x), T, Ci, W, Co, k, st, pad, opad,
                                  ctx.to_device(b), residual, yd)
    assert got_len == To
    wq = oracle.weight_quantize_transposed(conv, w_export, k * Co, Ci)
    want = oracle.convtranspose1d(conv, x, *wq, Co, k, st, pad, opad, bias=b, residual=residual)
    assert_bits_equal(yd.numpy(), want, "convtranspose output")


@pytest.mark.parametrize("T,C", [(40, 96), (7, 24), (3000, 192), (1200, 768)])
@pytest.mark.parametrize("residual", [0, 1], ids=["one-plane", "two-plane"])
@pytest.mark.parametrize("in_place", [False, True], ids=["out", "in-place"])
def test_conv1x1_skip(ctx, oracle, T, C, residual, in_place):
    conv = ctx.convention
    hidden = gauss(60 + T, (T, C))
    hidden[2:4] = 0.0
    skip = gauss(61 + T, (T, C))
    w = gauss(62, (C, C), 0.02)
    b = gauss(63, (C,), 0.01)
    W = ctx.weight(ctx.to_device(w), C, C)
    sd = ctx.to_device(skip)
    out = sd if in_place else ctx.empty((T, C), np.float32)
    ctx.conv1x1_skip(ctx.to_device(hidden), sd, T, W, ctx.to_device(b), residual, out)
    want = oracle.conv1x1_skip(conv, hidden, skip, *oracle.weight_quantize(conv, w), bias=b,
                               residual=residual)
    assert_bits_equal(out.numpy(), want, "conv1x1 onto skip")
    if not in_place:
        assert_bits_equal(sd.numpy(), skip, "skip rows left unchanged")


def test_convtranspose_long_short_k_tiles(ctx):
    """A long ConvTranspose with a short reduction (the decoder's last
    upsample: k = 192) takes 128 x 128 tiles of the chunked GEMM kernel;
    its output equals the 64 x 256 tile path's, which the oracle tests
    above pin."""
    T, Ci, Co, k, st, pad, opad = 140000, 192, 96, 4, 2, 1, 0
    x = gauss(41, (T, Ci))
    w_export = gauss(42, (Ci, k * Co), 0.02)
    b = gauss(43, (Co,), 0.01)
    W = ctx.weight(ctx.to_device(w_export), k * Co, Ci, transposed=True)
    xd, bd = ctx.to_device(x), ctx.to_device(b)
    outs = []
    for tile in ((0, 0), (2, 2)):
        ctx.set_gemm_tile(*tile)
        try:
            To = (T - 1) * st - 2 * pad + k + opad
            yd = ctx.empty((To, Co), np.float32)
            ctx.convtranspose1d(xd, T, Ci, W, Co, k, st, pad, opad, bd, 0, yd)
            outs.append(yd.numpy())
        finally:
            ctx.set_gemm_tile(0, 0)
    assert_bits_equal(outs[0], outs[1], "convtranspose output, 128x128 vs 64x256 tiles")


def test_conv1x1_skip_long_short_k_tiles(ctx):
    """A long 1x1 with a 384-row weight (the decoder's stage-1 1x1) takes
    128 x 128 tiles of the chunked GEMM kernel; its output equals the
    64-row whole-tile path's, which the oracle tests above pin."""
    T, C = 30000, 384
    hidden = gauss(71, (T, C))
    skip = gauss(72, (T, C))
    w = gauss(73, (C, C), 0.02)
    b = gauss(74, (C,), 0.01)
    W = ctx.weight(ctx.to_device(w), C, C)
    hd, sd, bd = ctx.to_device(hidden), ctx.to_device(skip), ctx.to_device(b)
    outs = []
    for tile in ((0, 0), (2, 1)):
        ctx.set_gemm_tile(*tile)
        try:
            out = ctx.empty((T, C), np.float32)
            ctx.conv1x1_skip(hd, sd, T, W, bd, 0, out)
            outs.append(out.numpy())
        finally:
            ctx.set_gemm_tile(0, 0)
    assert_bits_equal(outs[0], outs[1], "conv1x1 onto skip, 128x128 vs whole 64-row tiles")


def test_convtranspose_wide_lds_kernel(ctx):
    """The decoder's stage-1 upsample (3000 rows, k = 768, 20 taps of 384
    channels) takes the LDS-pipelined GEMM; its output equals the output
    with that kernel switched off, which the oracle tests above pin."""
    T, Ci, Co, k, st, pad, opad = 3000, 768, 384, 20, 10, 5, 0
    x = gauss(51, (T, Ci))
    w_export = gauss(52, (Ci, k * Co), 0.02)
    b = gauss(53, (Co,), 0.01)
    W = ctx.weight(ctx.to_device(w_export), k * Co, Ci, transposed=True)
    xd, bd = ctx.to_device(x), ctx.to_device(b)
    outs = []
    for lds in (0, -1):
        ctx.set_gemm_tile(-4, lds)
        try:
            To = (T - 1) * st - 2 * pad + k + opad
            yd = ctx.empty((To, Co), np.float32)
            ctx.convtranspose1d(xd, T, Ci, W, Co, k, st, pad, opad, bd, 0, yd)
            outs.append(yd.numpy())
        finally:
            ctx.set_gemm_tile(-4, 0)
    assert_bits_equal(outs[0], outs[1], "convtranspose output, LDS-pipelined vs whole-tile GEMM")
