"""iro_hip_dit_linear_gated_noalloc (the allocation-free variant of the Wo
site, dit.c:876-884 + 1013-1020) against iro_hip_dit_linear_gated, through
the C ABI: two calls in a row, the second with fewer rows, in both the plain
output and the gated-residual form, one and two planes; and the size limit
refused with an error."""
import ctypes as C

import numpy as np
import pytest

from iro_synth import gauss

pytestmark = pytest.mark.gpu


def _call(ctx, fn, mix, M, w, residual, out, x_res, gate, S):
    rc = getattr(ctx.lib, fn)(ctx.h, mix.vp, M, w.h, int(residual),
                              None if out is None else out.vp,
                              None if x_res is None else x_res.vp,
                              None if gate is None else gate.vp, S)
    if rc != 0:
        msg = ctx.lib.iro_hip_error(ctx.h).decode()
        ctx.lib.iro_hip_clear_error(ctx.h)
        raise RuntimeError(f"{fn}: {msg}")


# The contexts are taken by name (not through the session-parametrized `ctx`
# fixture, which would regroup these tests among the others): this file runs
# last.
CONVS = pytest.mark.parametrize("ctx_name", ["ctx_strict", "ctx_fast"], ids=["strict", "fastmath"])


@CONVS
@pytest.mark.parametrize("residual", [0, 1], ids=["one-plane", "two-term"])
def test_noalloc_matches_allocating_entry(request, ctx_name, residual):
    ctx = request.getfixturevalue(ctx_name)
    D, B = 1024, 3
    w = ctx.weight(ctx.to_device(gauss(501, (D, D), 0.02)), D, D)
    gate = ctx.to_device(gauss(502, (B, D), 0.3))
    for M, S in ((2250, 750), (771, 257)):   # second call smaller
        mix = ctx.to_device(gauss(503 + M, (M, D)))
        x0 = gauss(504 + M, (M, D))
        outs = {}
        for fn in ("iro_hip_dit_linear_gated", "iro_hip_dit_linear_gated_noalloc"):
            out = ctx.empty((M, D), np.float32)
            _call(ctx, fn, mix, M, w, residual, out, None, None, S)
            xr = ctx.to_device(x0)
            _call(ctx, fn, mix, M, w, residual, None, xr, gate, S)
            ctx.sync()
            outs[fn] = (out.numpy(), xr.numpy())
        (ya, xa), (yb, xb) = outs.values()
        assert np.array_equal(ya.view(np.int32), yb.view(np.int32)), f"out differs at M={M}"
        assert np.array_equal(xa.view(np.int32), xb.view(np.int32)), f"x_res differs at M={M}"
        assert not np.array_equal(xa, x0)


@CONVS
def test_noalloc_refuses_beyond_scratch(request, ctx_name):
    ctx = request.getfixturevalue(ctx_name)
    D = 1024
    w = ctx.weight(ctx.to_device(gauss(511, (D, D), 0.02)), D, D)
    M = 9000   # 9000 x 1024 two-plane codes exceed the 16 MiB scratch
    mix = ctx.to_device(np.zeros((M, D), np.float32))
    out = ctx.empty((M, D), np.float32)
    with pytest.raises(RuntimeError, match="scratch"):
        _call(ctx, "iro_hip_dit_linear_gated_noalloc", mix, M, w, 1, out, None, None, M)
