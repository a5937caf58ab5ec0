"""One whole DiT block on the device against the reference's own block.

tests/golden/dit_block_ref.npz holds the output of iro_dit_block
(dit.c:1042-1047) of the reference's scalar build on seeded inputs (made by
tests/golden/make_block_golden.py from oracle/_ref): the adaLN parameters
from cond (SiLU, rank-192 linears, tanhf gate), adaLN modulate, int8
QKVG (one quantization), QK-norm + half-RoPE, the attention core with a
masked context, Wo with the gated residual, adaLN modulate, int8 W1/W3 with
the SiLU gate, the two-term W2 (the reference's default residual mask) with
the gated residual.  The device computes the adaLN parameters (iro_hip_dit_adaln_params) and
composes its own kernels for every step (iro_hip_dit_stack_block_forward) and
must reproduce the parameters and x bit for bit.
"""
import os
import sys

import numpy as np
import pytest

import iro_hip
from parity_util import assert_bits_equal

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_block_golden as golden  # noqa: E402

pytestmark = pytest.mark.gpu


def test_dit_block_matches_reference_block(ctx_strict):
    ctx = ctx_strict
    g = np.load(os.path.join(HERE, "golden", "dit_block_ref.npz"))
    x, cond, ada, w, ck, cv, mask = golden.block_inputs()
    assert golden.input_digest(x, cond, ada, w, ck, cv) == str(g["inputs_sha256"]), \
        "seeded inputs changed; regenerate the fixture"
    assert np.array_equal(mask, g["mask"])
    B, S, D, H, R = golden.B, golden.S, golden.D, golden.H, golden.R
    stack = iro_hip.DiTStack(ctx, 1, D, H, 8)
    actx = ctx.attn_context(mask, B)
    try:
        wd = [ctx.to_device(a) for a in w]
        wq, wk, wv, wgate, wo, qn, kn, w1, w3, w2 = wd
        stack.set_block(0, ctx.to_device(np.zeros((6 * D, D), np.float32)), wq, wk, wv, wgate,
                        wo, w1, w3, w2)
        adad = [ctx.to_device(a) for a in ada]
        condd = ctx.to_device(cond)
        ada_attn = ctx.empty((3, B, D), np.float32)
        ada_mlp = ctx.empty((3, B, D), np.float32)
        ctx.dit_adaln_params(condd, B, D, R, adad[:9], ada_attn)
        ctx.dit_adaln_params(condd, B, D, R, adad[9:], ada_mlp)
        assert_bits_equal(ada_attn.numpy(), g["ada"][0], "attention adaLN parameters")
        assert_bits_equal(ada_mlp.numpy(), g["ada"][1], "MLP adaLN parameters")
        both = ctx.empty((2, 3, B, D), np.float32)
        ctx.dit_adaln_params(condd, B, D, R, adad, both)
        assert_bits_equal(both.numpy(), g["ada"], "both adaLNs in one call")
        ckd, cvd = ctx.to_device(ck), ctx.to_device(cv)
        for call in range(2):  # the second call reuses the workspace and buffers
            xd = ctx.to_device(x)
            stack.block_forward(0, xd, B, S, ada_attn, ada_mlp, qn, kn, golden.EPS, actx, ckd,
                                cvd)
            assert_bits_equal(xd.numpy(), g["x_out"], f"x after the block, call {call}")
    finally:
        actx.destroy()
        stack.destroy()
