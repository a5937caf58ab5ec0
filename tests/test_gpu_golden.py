"""The HIP path against the committed fixtures of the reference's own int8
path (tests/golden/make_golden.py), including SHA-256 digests at the BASELINE
single-linear shape (256 x 1024 -> 1024) and the QKVG input rows
(2250 x 1024, RMS-normalized, heavy-tailed)."""
import hashlib
import os
import sys

import numpy as np
import pytest

from parity_util import assert_bits_equal

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(__file__)
G = np.load(os.path.join(HERE, "golden", "int8_ref_vectors.npz"))


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _p(ctx):
    return "strict_" if ctx.convention == 0 else "fast_"


def test_hip_reproduces_reference_vectors(ctx):
    p = _p(ctx)
    x, w, b, y0 = G["in_x"], G["in_w"], G["in_b"], G["in_y0"]
    M, K = x.shape
    N = w.shape[0]
    W = ctx.weight(ctx.to_device(w), N, K)
    for got, key in zip(W.export(), ("wq", "ws", "wcs")):
        assert_bits_equal(got, G[p + key], key)
    xd = ctx.to_device(x)
    q, s, z = ctx.empty((M, K), np.uint8), ctx.empty(M, np.float32), ctx.empty(M, np.int32)
    ctx.quantize_rows(xd, q, s, z)
    for got, key in zip((q, s, z), ("q", "s", "z")):
        assert_bits_equal(got.numpy(), G[p + key], key)
    for bias in (0, 1):
        for acc in (0, 1):
            yd, work = ctx.to_device(y0), ctx.empty((M, N), np.int32)
            ctx.linear_ex(q, s, z, W, ctx.to_device(b) if bias else None, yd, M, work, acc)
            assert_bits_equal(yd.numpy(), G[f"{p}y_b{bias}_a{acc}"], f"y bias={bias} acc={acc}")
            assert_bits_equal(work.numpy(), G[p + "work"], "work")
    cx, cw, cb = G["in_cx"], G["in_cw"], G["in_cb"]
    CW = ctx.weight(ctx.to_device(cw), cw.shape[0], cw.shape[1])
    for res in (0, 1):
        yd = ctx.empty((50, cw.shape[0]), np.float32)
        ctx.conv1d(ctx.to_device(cx), 50, 16, CW, 7, 1, 3, 9, ctx.to_device(cb), res, yd)
        assert_bits_equal(yd.numpy(), G[f"{p}conv_r{res}"], f"conv residual={res}")


def test_hip_matches_reference_digests_at_baseline_shapes(ctx):
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_golden import baseline_inputs
    x0, w0, b0, x1 = baseline_inputs()
    W = ctx.weight(ctx.to_device(w0), 1024, 1024)
    wq, ws, _ = W.export()
    xd = ctx.to_device(x0)
    q, s, z = ctx.empty((256, 1024), np.uint8), ctx.empty(256, np.float32), ctx.empty(256, np.int32)
    ctx.quantize_rows(xd, q, s, z)
    yd, work = ctx.empty((256, 1024), np.float32), ctx.empty((256, 1024), np.int32)
    ctx.linear_ex(q, s, z, W, ctx.to_device(b0), yd, 256, work)
    x1d = ctx.to_device(x1)
    q1, s1, z1 = ctx.empty((2250, 1024), np.uint8), ctx.empty(2250, np.float32), ctx.empty(2250, np.int32)
    ctx.quantize_rows(x1d, q1, s1, z1)
    got = [digest(wq), digest(ws), digest(q.numpy()), digest(s.numpy()), digest(work.numpy()),
           digest(yd.numpy()), digest(q1.numpy()), digest(s1.numpy()), digest(z1.numpy())]
    assert got == list(G[_p(ctx) + "digests"])
