"""The int8 DiT linear stack on the GPU (iro_hip_dit_stack_step) against the
host-side block of oracle/cpu_baseline.c, which runs the reference's call
sequence per block (dit.c:780-798, 876-884, 939-972, 1013-1039) with the
oracle's quantizers and epilogues.  x after the step must match bit for bit.
"""
import numpy as np
import pytest

from iro_synth import gauss

import iro_hip

pytestmark = pytest.mark.gpu


def _weights(D, H, blocks, seed):
    shapes = [(6 * D, D), (D, D), (D, D), (D, D), (D, D), (D, D), (H, D), (H, D), (D, H)]
    return [[gauss(seed + 100 * b + i, s, 0.02) for i, s in enumerate(shapes)]
            for b in range(blocks)]


@pytest.mark.parametrize("blocks,B,S,D,H,rm", [(2, 2, 40, 256, 320, 8), (2, 1, 33, 128, 96, 15),
                                               (1, 3, 750, 1024, 2816, 8)],
                         ids=["small-w2two", "small-alltwo", "baseline-1block"])
def test_stack_step_matches_reference_sequence(ctx, oracle, blocks, B, S, D, H, rm):
    from oracle import CpuBaseline
    conv = ctx.convention
    ws = _weights(D, H, blocks, 900)
    x0 = gauss(901, (B * S, D))
    cond = gauss(902, (B, D), 0.1)
    stack = iro_hip.DiTStack(ctx, blocks, D, H, rm)
    try:
        for b in range(blocks):
            stack.set_block(b, *[ctx.to_device(w) for w in ws[b]])
        x = ctx.to_device(x0)
        stack.step(x, ctx.to_device(cond), B, S)
        got = x.numpy()
        assert stack.nbytes() == blocks * sum(w.shape[0] * (w.shape[1] + 8) for w in ws[0])
    finally:
        stack.destroy()
    cpu = CpuBaseline(8)
    want = np.array(x0, copy=True)
    for b in range(blocks):
        cpu.dit_block(conv, [oracle.weight_quantize(conv, w) for w in ws[b]], want, cond, B, S,
                      D, H, rm)
    bad = int((got.view(np.int32) != want.view(np.int32)).sum())
    assert bad == 0, f"{bad} of {got.size} elements of x differ"


def test_stack_graph_replays_match_direct_steps(ctx):
    """The step replayed from its HIP graph equals the directly launched step
    on every replay, with other eager work and synchronizations between the
    replays."""
    D, H, B, S, blocks = 256, 320, 2, 40, 2
    ws = _weights(D, H, blocks, 910)
    x0 = gauss(911, (B * S, D))
    cond = ctx.to_device(gauss(912, (B, D), 0.1))
    stack = iro_hip.DiTStack(ctx, blocks, D, H, 8)
    try:
        for b in range(blocks):
            stack.set_block(b, *[ctx.to_device(w) for w in ws[b]])
        x_init = ctx.to_device(x0)
        x = ctx.to_device(x0)
        stack.use_graph(False)
        stack.step(x, cond, B, S)
        want = x.numpy()
        stack.use_graph(True)
        other = ctx.to_device(gauss(913, (64, D)))
        q = ctx.empty((64, D), np.uint8)
        s_, z_ = ctx.empty(64, np.float32), ctx.empty(64, np.int32)
        for i in range(5):  # direct, capture, then three replays
            ctx.copy(x, x_init)
            stack.step(x, cond, B, S)
            got = x.numpy()
            assert np.array_equal(got.view(np.int32), want.view(np.int32)), f"step {i} differs"
            ctx.quantize_rows(other, q, s_, z_)
            ctx.sync()
    finally:
        stack.destroy()


def _rolled(base, b):
    """Block b's weights: the base draws with rows rotated by a block-dependent
    offset (distinct matrices per block at the cost of one draw)."""
    return [np.ascontiguousarray(np.roll(w, 97 * b + 13 * i, axis=0)) for i, w in enumerate(base)]


def test_stack_full_configuration_matches_reference_sequence(ctx, oracle):
    """The bench's configuration end to end: 12 blocks of hidden 1024, MLP
    2816, 3 x 750 rows, the two-term W2 (mask 8): one step, every block with
    its own weights, against the host's block sequence."""
    from oracle import CpuBaseline
    conv = ctx.convention
    blocks, B, S, D, H, rm = 12, 3, 750, 1024, 2816, 8
    shapes = [(6 * D, D), (D, D), (D, D), (D, D), (D, D), (D, D), (H, D), (H, D), (D, H)]
    base = [gauss(1000 + i, s, 0.02) for i, s in enumerate(shapes)]
    x0 = gauss(7, (B * S, D))
    cond = gauss(8, (B, D), 0.1)
    stack = iro_hip.DiTStack(ctx, blocks, D, H, rm)
    try:
        for b in range(blocks):
            dev = [ctx.to_device(w) for w in _rolled(base, b)]
            stack.set_block(b, *dev)
            for a in dev:
                a.free()
        x = ctx.to_device(x0)
        stack.step(x, ctx.to_device(cond), B, S)
        got = x.numpy()
    finally:
        stack.destroy()
    cpu = CpuBaseline(16)
    want = np.array(x0, copy=True)
    for b in range(blocks):
        cpu.dit_block(conv, [oracle.weight_quantize(conv, w) for w in _rolled(base, b)], want,
                      cond, B, S, D, H, rm)
    bad = int((got.view(np.int32) != want.view(np.int32)).sum())
    assert bad == 0, f"{bad} of {got.size} elements of x differ"


def test_stacked_modulation_gemm_twelve_blocks(ctx, oracle):
    """The 12 blocks' modulation linears (1024 -> 6 x 1024 each) run as one
    stacked [12 x 6144, 1024] GEMM on the 3 conditioning rows (the skinny
    kernel); block b's rows must equal the per-block int8 linear
    (dit.c:469-486 quantize + iro_int8_linear_ex, no bias)."""
    conv = ctx.convention
    blocks, B, S, D, H = 12, 3, 8, 1024, 64
    shapes = [(6 * D, D), (D, D), (D, D), (D, D), (D, D), (D, D), (H, D), (H, D), (D, H)]
    base = [gauss(1100 + i, s, 0.02) for i, s in enumerate(shapes)]
    cond = gauss(1120, (B, D), 0.1)
    stack = iro_hip.DiTStack(ctx, blocks, D, H, 8)
    try:
        for b in range(blocks):
            dev = [ctx.to_device(w) for w in _rolled(base, b)]
            stack.set_block(b, *dev)
            for a in dev:
                a.free()
        x = ctx.to_device(gauss(1121, (B * S, D)))
        stack.step(x, ctx.to_device(cond), B, S)
        mod = stack.buffers(B, S)["mod"]
        ctx.sync()
        q, s, z = oracle.quantize_rows(conv, cond)
        P = mod.shape[1] // blocks
        got_all = mod.numpy()
        for b in range(blocks):
            ada = _rolled(base, b)[0]
            want = oracle.linear(conv, q, s, z, *oracle.weight_quantize(conv, ada))[0]
            got = np.ascontiguousarray(got_all[:, b * P:b * P + 6 * D])
            assert np.array_equal(got.view(np.int32), want.view(np.int32)), f"block {b} differs"
    finally:
        stack.destroy()


@pytest.mark.parametrize("B,S,runs", [(3, 200, 3), (1, 300, 3), (2, 90, 4)])
def test_concurrent_row_runs_equal_one_stream(ctx, B, S, runs):
    """iro_hip_dit_stack_set_runs: the rows split over streams (one per CFG
    branch, or slices of 32-row blocks) give x bit-identical to one stream,
    eagerly and from the captured graph."""
    D, H, blocks = 256, 320, 2
    ws = _weights(D, H, blocks, 930)
    x0 = gauss(931, (B * S, D))
    cond = ctx.to_device(gauss(932, (B, D), 0.1))
    stack = iro_hip.DiTStack(ctx, blocks, D, H, 8)
    try:
        for b in range(blocks):
            stack.set_block(b, *[ctx.to_device(w) for w in ws[b]])
        x = ctx.to_device(x0)
        stack.step(x, cond, B, S)
        want = x.numpy()
        stack.set_runs(runs)
        x = ctx.to_device(x0)
        for i in range(4):  # eager, capture, replay, replay
            ctx.copy(x, ctx.to_device(x0))
            stack.step(x, cond, B, S)
            ctx.sync()
            got = x.numpy()
            bad = int((got.view(np.int32) != want.view(np.int32)).sum())
            assert bad == 0, f"step {i}: {bad} of {got.size} elements differ"
    finally:
        stack.destroy()
