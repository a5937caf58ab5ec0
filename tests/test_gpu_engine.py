"""The engine-level pieces around the int8 linears on the device.

- The lifecycle of tests/test_int8_engine.c:42-139 through the C ABI: an
  invalid configuration is refused, the int8 payload is reported with the
  reference's accounting, two warm requests (two sampler steps each, the
  second replaying HIP graphs) are byte-identical, an all-fp32 stack on the
  same inputs differs (the int8 path is really taken), a known-answer
  failure forced from the host makes context creation refuse (the
  counterpart of generate.c:527-536), and everything frees cleanly.
- IRO_INT8_MASK (dit.c:273-291): one DiT block with groups in fp32 against
  the reference's own block under the same mask
  (tests/golden/dit_block_mask_ref.npz, made by make_block_golden.py).
- The sampler step's graph: every replay equals the eager step.
- The timestep conditioner (dit.c:488-530), SiLU and the gated residual
  against the oracle (pinned to the reference's strict build on the CPU).
"""
import os
import sys

import numpy as np
import pytest

import iro_hip
from parity_util import assert_bits_equal

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_block_golden as block_golden  # noqa: E402
import make_step_golden as step_golden  # noqa: E402

pytestmark = pytest.mark.gpu


def _stack(ctx, mask=15):
    """The two-layer stack of the step fixture with every layer set."""
    x, cond, head, ada, blk, ck, cv, _ = step_golden.step_inputs()
    D, H, R, LAT, L = step_golden.D, step_golden.H, step_golden.R, step_golden.LAT, \
        step_golden.LAYERS
    stack = iro_hip.DiTStack(ctx, L, D, H, 8)
    if mask != 15:
        stack.set_int8_mask(mask)
    blkd = [ctx.to_device(a) for a in blk]
    adad = [ctx.to_device(a) for a in ada]
    headd = [ctx.to_device(a) for a in head]
    ckd, cvd = ctx.to_device(ck), ctx.to_device(cv)
    for l in range(L):
        w = blkd[10 * l:10 * l + 10]
        stack.set_block(l, None, w[0], w[1], w[2], w[3], w[4], w[7], w[8], w[9])
        stack.set_layer_f32(l, adad[18 * l:18 * l + 18], w[5], w[6], ckd, cvd)
    stack.set_head(*headd, LAT, R, step_golden.EPS)
    return stack


def _request(ctx, stack, actx):
    """Two sampler steps from the fixture's state (a CFG step, then a plain
    one): the final state and both velocities, as host arrays."""
    x, cond, *_ = step_golden.step_inputs()
    B, S, LAT = step_golden.B, step_golden.S, step_golden.LAT
    state = ctx.to_device(x)
    condd = ctx.to_device(cond)
    v1 = ctx.empty((B * S, LAT), np.float32)
    v2 = ctx.empty((S, LAT), np.float32)
    stack.sampler_step(state, condd, B, S, actx, True, (1, 2, -1), (1.5, 0.75, 0.0),
                       np.float32(-0.125), v1)
    stack.sampler_step(state, condd, 1, S, actx, False, (1, 2, -1), (1.5, 0.75, 0.0),
                       np.float32(-0.25), v2)
    return state.numpy(), v1.numpy(), v2.numpy()


def test_engine_lifecycle_through_the_c_abi(ctx_strict):
    ctx = ctx_strict
    lib = iro_hip.load()
    # An invalid configuration is refused (test_int8_engine.c:43-50).
    h = iro_hip.C.c_void_p()
    assert lib.iro_hip_create(0, 7, iro_hip.C.byref(h)) != 0 and not h.value
    with pytest.raises(iro_hip.HipError):
        iro_hip.DiTStack(ctx, 1, 1024, 2000, 8)  # H not a multiple of 32
    D, H, L = step_golden.D, step_golden.H, step_golden.LAYERS
    stack = _stack(ctx)
    actx = ctx.attn_context(step_golden.step_inputs()[7], 1)
    fp32 = None
    try:
        # The payload, iro_int8_weight_bytes over wq, wk, wv, gate, wo, w1,
        # w3, w2 of every layer (dit.c:235-271, generate.h:43-46).
        per_layer = 5 * (D * D + 8 * D) + 2 * (H * D + 8 * H) + (D * H + 8 * D)
        assert stack.nbytes() == L * per_layer
        with pytest.raises(iro_hip.HipError):
            stack.set_int8_mask(3)  # the mask is fixed once weights are set
        # Two warm requests are byte-identical (test_int8_engine.c:69-78):
        # the first runs eagerly and captures, the second replays.
        a = _request(ctx, stack, actx)
        b = _request(ctx, stack, actx)
        for got, want, what in zip(b, a, ("state", "CFG velocity", "plain velocity")):
            assert_bits_equal(got, want, f"warm request {what}")
        # An all-fp32 stack on the same inputs differs (test_int8_engine.c:82-94).
        fp32 = _stack(ctx, mask=0)
        assert fp32.nbytes() == stack.nbytes()
        c = _request(ctx, fp32, actx)
        assert np.all(np.isfinite(c[0]))
        assert not np.array_equal(c[0].view(np.int32), a[0].view(np.int32))
    finally:
        actx.destroy()
        stack.destroy()
        if fp32 is not None:
            fp32.destroy()
    # A known-answer failure makes the backend refuse (generate.c:527-536).
    lib.iro_hip_selfcheck_inject_fault(1)
    try:
        h = iro_hip.C.c_void_p()
        assert lib.iro_hip_create(0, 0, iro_hip.C.byref(h)) != 0 and not h.value
        assert lib.iro_hip_selfcheck(ctx.h) != 0
        assert b"known answer" in lib.iro_hip_error(ctx.h)
    finally:
        lib.iro_hip_selfcheck_inject_fault(0)
        lib.iro_hip_clear_error(ctx.h)
    assert lib.iro_hip_selfcheck(ctx.h) == 0


@pytest.mark.parametrize("mask", block_golden.MASKS)
def test_block_under_int8_mask_matches_reference(ctx_strict, mask):
    ctx = ctx_strict
    g = np.load(os.path.join(HERE, "golden", "dit_block_mask_ref.npz"))
    x, cond, ada, w, ck, cv, cmask = block_golden.block_inputs()
    assert block_golden.input_digest(x, cond, ada, w, ck, cv) == str(g["inputs_sha256"]), \
        "seeded inputs changed; regenerate the fixture"
    B, S, D, H, R = block_golden.B, block_golden.S, block_golden.D, block_golden.H, \
        block_golden.R
    stack = iro_hip.DiTStack(ctx, 1, D, H, 8)
    stack.set_int8_mask(mask)
    actx = ctx.attn_context(cmask, B)
    try:
        wq, wk, wv, wgate, wo, qn, kn, w1, w3, w2 = [ctx.to_device(a) for a in w]
        stack.set_block(0, None, wq, wk, wv, wgate, wo, w1, w3, w2)
        adad = [ctx.to_device(a) for a in ada]
        condd = ctx.to_device(cond)
        both = ctx.empty((2, 3, B, D), np.float32)
        ctx.dit_adaln_params(condd, B, D, R, adad, both)
        xd = ctx.to_device(x)
        stack.block_forward(0, xd, B, S, both.view(0, (3, B, D)), both.view(3 * B * D, (3, B, D)),
                            qn, kn, block_golden.EPS, actx, ctx.to_device(ck), ctx.to_device(cv))
        assert_bits_equal(xd.numpy(), g[f"x_out_mask{mask}"], f"x under IRO_INT8_MASK={mask}")
    finally:
        actx.destroy()
        stack.destroy()


def test_sampler_step_graph_replays_equal_eager(ctx_strict):
    ctx = ctx_strict
    x, cond, *_ = step_golden.step_inputs()
    B, S, LAT = step_golden.B, step_golden.S, step_golden.LAT
    stack = _stack(ctx)
    actx = ctx.attn_context(step_golden.step_inputs()[7], 1)
    try:
        condd = ctx.to_device(cond)
        rows, scales = (1, 2, -1), (1.5, 0.75, 0.0)

        def run(n):
            state = ctx.to_device(x)
            vel = ctx.empty((B * S, LAT), np.float32)
            out = []
            for i in range(n):
                stack.sampler_step(state, condd, B, S, actx, True, rows, scales,
                                   np.float32(-0.0625 * (i + 1)), vel)
                ctx.sync()
                out.append((state.numpy(), vel.numpy()))
                # eager work between the replays
                scratch = ctx.to_device(np.full((1024,), i, np.float32))
                ctx.fill(scratch, 0)
                ctx.sync()
            return out

        stack.use_graph(False)
        eager = run(4)
        stack.use_graph(True)
        replayed = run(4)  # step 1 eager, step 2 captures, steps 3-4 replay
        for i, ((s1, v1), (s2, v2)) in enumerate(zip(replayed, eager)):
            assert_bits_equal(v1, v2, f"velocity of step {i}")
            assert_bits_equal(s1, s2, f"state after step {i}")
    finally:
        actx.destroy()
        stack.destroy()


def test_condition_matches_oracle(ctx_strict, oracle):
    import test_engine_pins as pins
    ctx = ctx_strict
    w0, w1, w2 = pins.conditioner_weights(11)
    t = np.array([1.0, 0.5, 1e-3, 0.999, 0.0, 1.0 / 3.0], np.float32)
    cond = ctx.empty((t.size, pins.COND), np.float32)
    ctx.dit_condition(ctx.to_device(t), t.size, ctx.to_device(w0), ctx.to_device(w1),
                      ctx.to_device(w2), pins.TDIM, pins.D, pins.COND, cond)
    assert_bits_equal(cond.numpy(), oracle.dit_condition(w0, w1, w2, t), "cond")


def test_silu_and_gated_residual_match_oracle(ctx, oracle):
    rng = np.random.default_rng(5)
    a = (rng.standard_normal(10007, dtype=np.float32) * 6).astype(np.float32)
    a[:6] = [0.0, -0.0, -90.0, 90.0, 1e-30, -1e-42]
    g = rng.standard_normal(10007, dtype=np.float32)
    d = ctx.to_device(a)
    ctx.silu(d, a.size)
    assert_bits_equal(d.numpy(), oracle.silu_mul(a, np.ones_like(a)), "silu")
    d = ctx.to_device(a)
    ctx.silu(d, a.size, ctx.to_device(g))
    assert_bits_equal(d.numpy(), oracle.silu_mul(a, g), "silu * gate")
    B, S, D = 3, 7, 96
    x = rng.standard_normal((B * S, D), dtype=np.float32)
    gate = rng.standard_normal((B, D), dtype=np.float32)
    br = rng.standard_normal((B * S, D), dtype=np.float32)
    xd = ctx.to_device(x)
    ctx.gated_residual(xd, ctx.to_device(gate), D, ctx.to_device(br), B * S, D, S)
    assert_bits_equal(xd.numpy(), oracle.gated_residual(ctx.convention, x, gate, br, B, S),
                      "gated residual")


def test_code_packing_equals_reference_rounding_on_every_float(ctx_strict):
    # Every activation quantizer packs its unrounded values with
    # v_cvt_pk_u8_f32; that must equal the reference's clamp(nearbyintf(v),
    # 0, 255) conversion (ops.c:341-345) for every float v.
    assert ctx_strict.selfcheck_codes() == 0
