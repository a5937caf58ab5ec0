"""One whole DiT block on the device against the reference's own block.

tests/golden/dit_block_ref.npz holds the output of iro_dit_block
(dit.c:1042-1047) of the reference's scalar build on seeded inputs (made by
tests/golden/make_block_golden.py from oracle/_ref): adaLN modulate, int8
QKVG (one quantization), QK-norm + half-RoPE, the attention core with a
masked context, Wo with the gated residual, adaLN modulate, int8 W1/W3 with
the SiLU gate, the two-term W2 (the reference's default residual mask) with
the gated residual.  The device composes its own kernels for every step
(iro_hip_dit_stack_block_forward) and must reproduce x bit for bit.
"""
import hashlib
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
    got_digest = hashlib.sha256(np.concatenate(
        [a.ravel() for a in [x, cond, ada, *w, ck, cv]]).tobytes()).hexdigest()
    assert got_digest == str(g["inputs_sha256"]), "seeded inputs changed; regenerate the fixture"
    assert np.array_equal(mask, g["mask"])
    B, S, D, H = golden.B, golden.S, golden.D, golden.H
    stack = iro_hip.DiTStack(ctx, 1, D, H, 8)
    actx = ctx.attn_context(mask, B)
    try:
        wd = [ctx.to_device(a) for a in w]
        wq, wk, wv, wgate, wo, qn, kn, w1, w3, w2 = wd
        stack.set_block(0, ctx.to_device(np.zeros((6 * D, D), np.float32)), wq, wk, wv, wgate,
                        wo, w1, w3, w2)
        xd = ctx.to_device(x)
        ada_attn = ctx.to_device(np.ascontiguousarray(g["ada"][0]))
        ada_mlp = ctx.to_device(np.ascontiguousarray(g["ada"][1]))
        stack.block_forward(0, xd, B, S, ada_attn, ada_mlp, qn, kn, golden.EPS, actx,
                            ctx.to_device(ck), ctx.to_device(cv))
        assert_bits_equal(xd.numpy(), g["x_out"], "x after the block")
        # The same call again from the same input gives the same bits (the
        # attention workspace and stack buffers are reused).
        xd2 = ctx.to_device(x)
        stack.block_forward(0, xd2, B, S, ada_attn, ada_mlp, qn, kn, golden.EPS, actx,
                            ctx.to_device(ck), ctx.to_device(cv))
        assert_bits_equal(xd2.numpy(), g["x_out"], "x after the block, second call")
    finally:
        actx.destroy()
        stack.destroy()
