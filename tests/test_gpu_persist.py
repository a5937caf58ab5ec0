"""The persistent stack kernel (iro_persist.hip: one kernel per step whose
workgroups take quantization and GEMM items of their own XCD's row bands
from a queue) against the per-kernel path and the host's block sequence.

Shapes cover a single 96-row band (most XCDs own no rows), ragged last
bands, one- and two-plane W2 (residual mask 0 and 8), several blocks, the
model's D = 1024 / H = 2816 at 3 x 750 rows, and graph replays."""
import numpy as np
import pytest

from iro_synth import gauss

import iro_hip

pytestmark = pytest.mark.gpu


def _weights(D, H, blocks, seed):
    shapes = [(6 * D, D), (D, D), (D, D), (D, D), (D, D), (D, D), (H, D), (H, D), (D, H)]
    return [[gauss(seed + 100 * b + i, s, 0.02) for i, s in enumerate(shapes)]
            for b in range(blocks)]


def _run(ctx, ws, x0, cond, B, S, D, H, rm, persistent, graph=False, steps=1):
    blocks = len(ws)
    stack = iro_hip.DiTStack(ctx, blocks, D, H, rm)
    try:
        stack.use_persistent(persistent)
        stack.use_graph(graph)
        for b in range(blocks):
            dev = [ctx.to_device(w) for w in ws[b]]
            stack.set_block(b, *dev)
            for a in dev:
                a.free()
        x_init = ctx.to_device(x0)
        x = ctx.to_device(x0)
        c = ctx.to_device(cond)
        outs = []
        for _ in range(steps):
            ctx.copy(x, x_init)
            stack.step(x, c, B, S)
            outs.append(x.numpy())
        ctx.sync()
        q = stack.buffers(B, S)["q"].numpy()
        return outs, q
    finally:
        stack.destroy()


CASES = [(2, 2, 37, 256, 256, 8), (2, 3, 333, 512, 768, 8), (3, 1, 100, 1024, 2816, 0),
         (1, 3, 750, 1024, 2816, 8), (2, 1, 1, 256, 512, 8)]


@pytest.mark.parametrize("blocks,B,S,D,H,rm", CASES,
                         ids=["one-band", "ragged-bands", "one-plane-w2", "model-3x750", "one-row"])
def test_persistent_matches_per_kernel_path(ctx, blocks, B, S, D, H, rm):
    ws = _weights(D, H, blocks, 1300)
    x0 = gauss(1301, (B * S, D))
    cond = gauss(1302, (B, D), 0.1)
    (want,), qw = _run(ctx, ws, x0, cond, B, S, D, H, rm, persistent=False)
    (got,), qg = _run(ctx, ws, x0, cond, B, S, D, H, rm, persistent=True)
    bad = int((got.view(np.int32) != want.view(np.int32)).sum())
    assert bad == 0, f"{bad} of {got.size} elements of x differ"
    assert np.array_equal(qg.view(np.int32), qw.view(np.int32)), "last block's q differs"


def test_persistent_matches_reference_sequence(ctx, oracle):
    from oracle import CpuBaseline
    conv = ctx.convention
    blocks, B, S, D, H, rm = 2, 3, 333, 512, 768, 8
    ws = _weights(D, H, blocks, 1310)
    x0 = gauss(1311, (B * S, D))
    cond = gauss(1312, (B, D), 0.1)
    (got,), _ = _run(ctx, ws, x0, cond, B, S, D, H, rm, persistent=True)
    cpu = CpuBaseline(8)
    want = np.array(x0, copy=True)
    for b in range(blocks):
        cpu.dit_block(conv, [oracle.weight_quantize(conv, w) for w in ws[b]], want, cond, B, S,
                      D, H, rm)
    bad = int((got.view(np.int32) != want.view(np.int32)).sum())
    assert bad == 0, f"{bad} of {got.size} elements of x differ"


def test_persistent_graph_replays_match(ctx):
    blocks, B, S, D, H, rm = 2, 3, 200, 512, 512, 8
    ws = _weights(D, H, blocks, 1320)
    x0 = gauss(1321, (B * S, D))
    cond = gauss(1322, (B, D), 0.1)
    (want,), _ = _run(ctx, ws, x0, cond, B, S, D, H, rm, persistent=True)
    outs, _ = _run(ctx, ws, x0, cond, B, S, D, H, rm, persistent=True, graph=True, steps=5)
    for i, got in enumerate(outs):
        assert np.array_equal(got.view(np.int32), want.view(np.int32)), f"step {i} differs"
