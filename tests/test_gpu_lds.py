"""The LDS-pipelined GEMM kernel (iro_gemm_lds.hip) in every shape it
offers, forced through iro_hip_set_gemm_tile(ctx, -4, shape), against the
register-streamed kernels (shape -1): the whole stack step (QKVG split
store, Wo and W2 gated residuals with one and two planes, W1/W3 + SiLU) must
give identical bits.  Shapes a GEMM cannot take fall back; the default (0)
runs QKVG through it."""
import numpy as np
import pytest

from iro_synth import gauss

import iro_hip

pytestmark = pytest.mark.gpu


def _step(ctx, shape, ws, x0, cond, B, S, D, H, rm):
    ctx.lib.iro_hip_set_gemm_tile(ctx.h, -4, shape)
    stack = iro_hip.DiTStack(ctx, len(ws), D, H, rm)
    try:
        stack.use_graph(False)
        for b, w in enumerate(ws):
            stack.set_block(b, *[ctx.to_device(a) for a in w])
        x = ctx.to_device(x0)
        stack.step(x, ctx.to_device(cond), B, S)
        ctx.sync()
        bufs = stack.buffers(B, S)
        return x.numpy(), bufs["q"].numpy(), bufs["hidden"].numpy()
    finally:
        stack.destroy()
        ctx.lib.iro_hip_set_gemm_tile(ctx.h, -4, 0)


@pytest.mark.parametrize("B,S,D,H,rm", [(3, 100, 512, 768, 8), (1, 233, 256, 512, 0),
                                        (2, 17, 256, 256, 8)])
def test_lds_shapes_match_register_kernels(ctx, B, S, D, H, rm):
    shapes = [(6 * D, D), (D, D), (D, D), (D, D), (D, D), (D, D), (H, D), (H, D), (D, H)]
    ws = [[gauss(1400 + 20 * b + i, s, 0.02) for i, s in enumerate(shapes)] for b in range(2)]
    x0 = gauss(1450, (B * S, D))
    cond = gauss(1451, (B, D), 0.1)
    want = _step(ctx, -1, ws, x0, cond, B, S, D, H, rm)
    for shape in (0, 1, 2, 3, 4, 5):
        got = _step(ctx, shape, ws, x0, cond, B, S, D, H, rm)
        for name, g, w in zip(("x", "q", "hidden"), got, want):
            assert np.array_equal(g.view(np.int32), w.view(np.int32)), f"shape {shape}: {name}"
