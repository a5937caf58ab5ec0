"""The CFG combine + Euler update of sampler.c:281-297.

CPU: the oracle restatement reproduces every state transition of the
reference's own sampler, traced step by step in both of its builds
(tests/golden/sampler_update_ref.npz, tests/golden/make_sampler_golden.py):
seven CFG combinations (text, speaker, caption rows on or off), CFG and
plain steps.  The fixture also pins the host-side arithmetic the device
entry point leaves to its caller (the traced timesteps and the CFG batch
follow sampler.c:243-249), and planted mistakes in the oracle's arguments
(a swapped row, a dropped term, the other build's rounding) fail it.

GPU: iro_hip_euler_update reproduces the same transitions bit for bit, and
agrees with the oracle at the production size (3 x 750 latent frames of 32
values, four CFG rows).
"""
import os

import numpy as np
import pytest

from iro_synth import gauss
from oracle import GCC_FASTMATH, STRICT
from parity_util import assert_bits_equal
from sampler_cases import COMBOS, euler_times, transitions

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "sampler_update_ref.npz")
FLAVOUR = {STRICT: "strict", GCC_FASTMATH: "fast"}


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


@pytest.mark.parametrize("conv", [STRICT, GCC_FASTMATH], ids=["strict", "fast"])
@pytest.mark.parametrize("name", COMBOS)
def test_oracle_reproduces_reference_sampler_steps(oracle, golden, conv, name):
    cfg_steps = 0
    for st, v, use, rows, sc, dt, nxt, traced, t in transitions(golden, FLAVOUR[conv], name):
        assert traced == t, "timestep differs from sampler.c:243-245"
        got = oracle.euler_update(conv, st, v, use, rows, sc, dt)
        assert_bits_equal(got, nxt, f"{name} state")
        cfg_steps += bool(use)
    assert cfg_steps == 3  # steps 0-2 with CFG, step 3 without


def _mismatches(oracle, golden, conv, name, mutate):
    bad = 0
    for st, v, use, rows, sc, dt, nxt, _, _ in transitions(golden, FLAVOUR[conv], name):
        conv2, rows2, sc2 = mutate(conv, list(rows), list(sc))
        got = oracle.euler_update(conv2, st, v, use, rows2, sc2, dt)
        bad += int((got.view(np.int32) != nxt.view(np.int32)).sum())
    return bad


def test_planted_mistakes_fail_the_reference_traces(oracle, golden):
    def swap_rows(c, r, s):
        r[0], r[1] = r[1], r[0]
        return c, r, s

    def drop_caption(c, r, s):
        r[2] = -1
        return c, r, s

    def other_build(c, r, s):
        return (GCC_FASTMATH if c == STRICT else STRICT), r, s

    for conv in (STRICT, GCC_FASTMATH):
        assert _mismatches(oracle, golden, conv, "tsc", swap_rows) > 0
        assert _mismatches(oracle, golden, conv, "tsc", drop_caption) > 0
        assert _mismatches(oracle, golden, conv, "tsc", lambda c, r, s: (c, r, s)) == 0
    assert _mismatches(oracle, golden, STRICT, "tsc", other_build) > 0
    assert _mismatches(oracle, golden, GCC_FASTMATH, "tsc", other_build) > 0
    assert _mismatches(oracle, golden, GCC_FASTMATH, "ts", other_build) > 0


def test_euler_times_closed_forms():
    # timestep runs from init_scale down by init_scale / steps; the last step
    # lands on zero: sum of the dts is -init_scale within rounding
    for steps, scale in ((4, 1.0), (8, 1.0), (40, 0.999)):
        ts = [euler_times(s, steps, scale) for s in range(steps)]
        assert ts[0][0] == np.float32(scale)
        total = sum(float(dt) for _, dt in ts)
        assert abs(total + scale) < 1e-5
        for s, (t, dt) in enumerate(ts):
            t_next = euler_times(s + 1, steps, scale)[0] if s + 1 < steps else np.float32(0)
            assert np.float32(t + dt) == t_next or abs(float(t + dt - t_next)) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("name", COMBOS)
def test_device_reproduces_reference_sampler_steps(ctx, golden, name):
    flavour = FLAVOUR[ctx.convention]
    for st, v, use, rows, sc, dt, nxt, _, _ in transitions(golden, flavour, name):
        sd = ctx.to_device(np.ascontiguousarray(st))
        vd = ctx.to_device(np.ascontiguousarray(v))
        ctx.euler_update(sd, vd, st.size, v.shape[0], use, rows, sc, dt)
        assert_bits_equal(sd.numpy(), nxt, f"{name} device state")


@pytest.mark.gpu
@pytest.mark.parametrize("scales", [(3.0, 1.5, 0.0), (1.5, 0.75, 2.25), (0.0, 0.0, 4.0)])
def test_device_euler_update_at_production_size(ctx, oracle, scales):
    from sampler_cases import cfg_rows
    n = 750 * 32
    rows = cfg_rows(scales)
    batch = 1 + sum(r >= 0 for r in rows)
    state = gauss(61, (n,))
    vel = gauss(62, (batch, n), 0.7)
    vel[:, ::97] = 0.0
    vel[0, 5::131] = -0.0
    for step, use in ((0, True), (5, False)):
        _, dt = euler_times(step, 8, 1.0)
        want = oracle.euler_update(ctx.convention, state, vel, use, rows, scales, dt)
        sd = ctx.to_device(state)
        ctx.euler_update(sd, ctx.to_device(vel), n, batch, use, rows, scales, dt)
        assert_bits_equal(sd.numpy(), want, f"euler update step {step}")


@pytest.mark.gpu
def test_device_euler_update_rejects_bad_rows(ctx):
    import iro_hip
    sd, vd = ctx.empty(64, np.float32), ctx.empty((2, 64), np.float32)
    for rows in ((2, -1, -1), (0, -1, -1), (-2, -1, -1)):
        with pytest.raises(iro_hip.HipError):
            ctx.euler_update(sd, vd, 64, 2, True, rows, (1.0, 0.0, 0.0), -0.125)
    with pytest.raises(iro_hip.HipError):
        ctx.euler_update(sd, vd, 64, 1, False, (4, -1, -1), (1.0, 0.0, 0.0), -0.125)
    ctx.euler_update(sd, vd, 64, 1, False, (1, 2, 3), (1.0, 0.5, 0.25), -0.125)  # plain step
