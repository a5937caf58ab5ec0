"""The DiT evaluation of one sampler step on the device against the
reference's own (sampler.c:259-278).

tests/golden/dit_step_ref.npz holds the velocity of the reference's scalar
build (made by tests/golden/make_step_golden.py from oracle/_ref) over two
layers with distinct weights: the input projection of one latent row set
(iro_dit_input), broadcast to the three CFG rows, two
iro_dit_block_shared_context calls with a masked shared context, and the
output head (iro_dit_output: RMSNorm and the 1280 -> 32 projection).  The
device runs iro_hip_linear_f32, two adaLN parameter / block forward pairs,
iro_hip_rmsnorm_f32 and iro_hip_linear_f32, and must give the same bits.
"""
import os
import sys

import numpy as np
import pytest

import iro_hip
from parity_util import assert_bits_equal

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_step_golden as golden  # noqa: E402

pytestmark = pytest.mark.gpu


def test_dit_step_matches_reference(ctx_strict):
    ctx = ctx_strict
    g = np.load(os.path.join(HERE, "golden", "dit_step_ref.npz"))
    x, cond, head, ada, blk, ck, cv, mask = golden.step_inputs()
    assert golden.input_digest(x, cond, head, ada, blk, ck, cv) == str(g["inputs_sha256"]), \
        "seeded inputs changed; regenerate the fixture"
    B, S, D, H, R, LAT, L = golden.B, golden.S, golden.D, golden.H, golden.R, golden.LAT, \
        golden.LAYERS
    stack = iro_hip.DiTStack(ctx, L, D, H, 8)
    actx = ctx.attn_context(mask, 1)
    try:
        zeros = ctx.to_device(np.zeros((6 * D, D), np.float32))
        blkd = [ctx.to_device(a) for a in blk]
        for l in range(L):
            w = blkd[10 * l:10 * l + 10]
            stack.set_block(l, zeros, w[0], w[1], w[2], w[3], w[4], w[7], w[8], w[9])
        adad = [ctx.to_device(a) for a in ada]
        headd = [ctx.to_device(a) for a in head]
        condd, ckd, cvd = ctx.to_device(cond), ctx.to_device(ck), ctx.to_device(cv)
        xd = ctx.to_device(x)
        proj = ctx.empty((B * S, D), np.float32)
        first = proj.view(0, (S, D))
        ctx.linear_f32(xd, S, LAT, headd[0], D, headd[1], first)
        for b in range(1, B):
            ctx.copy(proj.view(b * S * D, (S, D)), first)
        params = ctx.empty((2, 3, B, D), np.float32)
        for l in range(L):
            ctx.dit_adaln_params(condd, B, D, R, adad[18 * l:18 * l + 18], params)
            w = blkd[10 * l:10 * l + 10]
            stack.block_forward(l, proj, B, S, params.view(0, (3, B, D)),
                                params.view(3 * B * D, (3, B, D)), w[5], w[6], golden.EPS, actx,
                                ckd, cvd)
        norm = ctx.empty((B * S, D), np.float32)
        ctx.rmsnorm_f32(proj, B * S, D, headd[2], golden.EPS, norm)
        vel = ctx.empty((B * S, LAT), np.float32)
        ctx.linear_f32(norm, B * S, D, headd[3], LAT, headd[4], vel)
        assert_bits_equal(vel.numpy(), g["velocity"], "velocity")
    finally:
        actx.destroy()
        stack.destroy()


def _sampler_stack(ctx, with_modulation):
    x, cond, head, ada, blk, ck, cv, mask = golden.step_inputs()
    B, S, D, H, R, LAT, L = golden.B, golden.S, golden.D, golden.H, golden.R, golden.LAT, \
        golden.LAYERS
    stack = iro_hip.DiTStack(ctx, L, D, H, 8)
    zeros = ctx.to_device(np.zeros((6 * D, D), np.float32)) if with_modulation else None
    blkd = [ctx.to_device(a) for a in blk]
    adad = [ctx.to_device(a) for a in ada]
    headd = [ctx.to_device(a) for a in head]
    ckd, cvd = ctx.to_device(ck), ctx.to_device(cv)
    for l in range(L):
        w = blkd[10 * l:10 * l + 10]
        stack.set_block(l, zeros, w[0], w[1], w[2], w[3], w[4], w[7], w[8], w[9])
        stack.set_layer_f32(l, adad[18 * l:18 * l + 18], w[5], w[6], ckd, cvd)
    stack.set_head(*headd, LAT, R, golden.EPS)
    return stack


def test_sampler_step_entry_point_matches_reference(ctx_strict, oracle):
    # iro_hip_dit_sampler_step owns the whole step: the same velocity bits as
    # the reference's DiT evaluation above, then the CFG / Euler update of the
    # state (sampler.c:281-297) as the oracle restates it; then a plain step
    # (batch 1, CFG off, sampler.c:247-249) on the same attention context,
    # whose velocity must equal the reference's batch-1 evaluation of the
    # same state (its row 0 of the CFG batch).
    from oracle import STRICT
    ctx = ctx_strict
    g = np.load(os.path.join(HERE, "golden", "dit_step_ref.npz"))
    x, cond, head, ada, blk, ck, cv, mask = golden.step_inputs()
    B, S, LAT = golden.B, golden.S, golden.LAT
    stack = _sampler_stack(ctx, with_modulation=False)
    actx = ctx.attn_context(mask, 1)
    try:
        rows, scales, dt = (1, 2, -1), (1.5, 0.75, 0.0), np.float32(-0.125)
        state = ctx.to_device(x)
        condd = ctx.to_device(cond)
        vel = ctx.empty((B * S, LAT), np.float32)
        stack.sampler_step(state, condd, B, S, actx, True, rows, scales, dt, vel)
        assert_bits_equal(vel.numpy(), g["velocity"], "sampler step velocity")
        want = oracle.euler_update(STRICT, x, g["velocity"].reshape(B, S * LAT), True, rows,
                                   scales, dt)
        got1 = state.numpy().reshape(-1)
        assert_bits_equal(got1, want, "sampler step state")
        # A plain step from the fixture's state: batch 1 on the CFG context.
        state1 = ctx.to_device(x)
        vel1 = ctx.empty((S, LAT), np.float32)
        stack.sampler_step(state1, condd, 1, S, actx, False, rows, scales, dt, vel1)
        assert_bits_equal(vel1.numpy(), g["velocity_b1"], "plain step velocity (batch 1)")
        want1 = oracle.euler_update(STRICT, x, g["velocity_b1"].reshape(1, S * LAT), False,
                                    rows, scales, dt)
        assert_bits_equal(state1.numpy().reshape(-1), want1, "plain step state")
        # Then a plain step from the CFG step's state: the composition.
        vel2 = ctx.empty((S, LAT), np.float32)
        stack.sampler_step(state, condd, 1, S, actx, False, rows, scales, dt, vel2)
        want2 = oracle.euler_update(STRICT, got1, vel2.numpy().reshape(1, S * LAT), False, rows,
                                    scales, dt)
        assert_bits_equal(state.numpy().reshape(-1), want2, "second step state")
    finally:
        actx.destroy()
        stack.destroy()


def test_sampler_step_rejects_bad_rows_before_any_launch(ctx_strict):
    # A CFG row outside the step's batch, or a batch above the attention
    # context's, is refused at entry: the state and velocity stay untouched.
    ctx = ctx_strict
    x, cond, head, ada, blk, ck, cv, mask = golden.step_inputs()
    B, S, LAT = golden.B, golden.S, golden.LAT
    stack = _sampler_stack(ctx, with_modulation=False)
    actx = ctx.attn_context(mask[:2], 1)
    try:
        state = ctx.to_device(x)
        condd = ctx.to_device(np.repeat(cond[:1], 4, axis=0))
        vel = ctx.to_device(np.full((4 * S, LAT), 7.0, np.float32))
        for batch, rows in ((2, (1, 2, -1)), (3, (1, 2, -1)), (2, (0, -1, -1))):
            with pytest.raises(iro_hip.HipError):
                stack.sampler_step(state, condd, batch, S, actx, True, rows, (1.0, 1.0, 0.0),
                                   -0.125, vel)
        ctx.sync()
        assert_bits_equal(state.numpy(), x, "state after refused steps")
        assert np.all(vel.numpy() == 7.0)
    finally:
        actx.destroy()
        stack.destroy()
