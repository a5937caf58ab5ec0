"""The oracle against the committed fixtures written by the reference's own
int8 path (tests/golden/make_golden.py): runs without the reference and
without a GPU."""
import hashlib
import os

import numpy as np
import pytest

from oracle import GCC_FASTMATH, STRICT

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "int8_ref_vectors.npz"))
FLAVOURS = [(STRICT, "strict"), (GCC_FASTMATH, "fast")]


def eq(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.int32), b.view(np.int32))
    return np.array_equal(a, b)


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.mark.parametrize("conv,p", FLAVOURS, ids=["strict", "fastmath"])
def test_oracle_reproduces_reference_vectors(oracle, conv, p):
    p += "_"
    wq = oracle.weight_quantize(conv, G["in_w"])
    assert eq(wq[0], G[p + "wq"]) and eq(wq[1], G[p + "ws"]) and eq(wq[2], G[p + "wcs"])
    q = oracle.quantize_rows(conv, G["in_x"])
    assert eq(q[0], G[p + "q"]) and eq(q[1], G[p + "s"]) and eq(q[2], G[p + "z"])
    (q1, s1, z1), r, (q2, s2, z2) = oracle.quantize_rows_residual(conv, G["in_x"])
    for name, v in dict(q1=q1, s1=s1, z1=z1, res=r, q2=q2, s2=s2, z2=z2).items():
        assert eq(v, G[p + "r_" + name]), name
    for bias in (0, 1):
        for acc in (0, 1):
            y, work = oracle.linear(conv, *q, *wq, bias=G["in_b"] if bias else None,
                                    y=G["in_y0"], accumulate=acc)
            assert eq(y, G[f"{p}y_b{bias}_a{acc}"]) and eq(work, G[p + "work"])
    cwq = oracle.weight_quantize(conv, G["in_cw"])
    for res in (0, 1):
        y, _, _, _ = oracle.conv1d(conv, G["in_cx"], *cwq, 7, 1, 3, 9, bias=G["in_cb"],
                                   residual=res)
        assert eq(y, G[f"{p}conv_r{res}"]), f"conv residual={res}"


def test_oracle_silu_reproduces_strict_reference(oracle):
    # the fast-math build's gate depends on the host CPU (rcpps): strict only
    assert eq(oracle.silu_mul(G["in_sa"], G["in_sg"]), G["strict_silu"])


@pytest.mark.parametrize("conv,p", FLAVOURS, ids=["strict", "fastmath"])
def test_oracle_matches_reference_digests_at_baseline_shapes(oracle, conv, p):
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(__file__), "golden"))
    from make_golden import baseline_inputs
    x0, w0, b0, x1 = baseline_inputs()
    wq0 = oracle.weight_quantize(conv, w0)
    q0 = oracle.quantize_rows(conv, x0)
    y0, work0 = oracle.linear(conv, *q0, *wq0, bias=b0)
    q1 = oracle.quantize_rows(conv, x1)
    got = [digest(wq0[0]), digest(wq0[1]), digest(q0[0]), digest(q0[1]), digest(work0),
           digest(y0), digest(q1[0]), digest(q1[1]), digest(q1[2])]
    assert got == list(G[p + "_digests"])
