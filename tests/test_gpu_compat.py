"""The ops.h drop-in (include/iro_int8_ops.h): the reference's host-pointer
int8 API served by the GPU, exercised the way tests/test_int8_ops.c does
(weight quantize, row quantize, linear with `work`, cross-M sub-call,
selfcheck, free resets the struct), bit-exact against the oracle.  The
process-wide default context runs the strict convention (IRO_HIP_CONVENTION
unset)."""
import numpy as np
import pytest

from iro_synth import gauss, heavy_tail
from parity_util import assert_bits_equal

import iro_hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    return iro_hip.Ops()


def test_backend_queries(ops):
    assert ops.lib.iro_int8_fast_available() == 1
    name = ops.lib.iro_int8_prepare_backend()
    assert name and b"gfx950" in name
    assert ops.selfcheck() == 0


@pytest.mark.parametrize("M,N,K,outlier", [(7, 32, 64, 0), (23, 96, 128, 1), (112, 160, 1280, 0),
                                           (37, 184, 1280, 1), (9, 40, 100, 0)])
def test_int8_ops_flow(ops, oracle, M, N, K, outlier):
    conv = 0
    w = gauss(11 + N, (N, K), 0.02)
    x = gauss(12 + M, (M, K), 1.5)
    if outlier:
        x = heavy_tail(x, 13)
        x[:, 17 % K] = 20.0
    bias = gauss(14, (N,), 0.3)
    st = ops.weight_quantize(w)
    q_w, s_w, cs_w = ops.weight_arrays(st)
    want_w = oracle.weight_quantize(conv, w)
    for got, want, what in zip((q_w, s_w, cs_w), want_w, ("codes", "scales", "colsum")):
        assert_bits_equal(got, want, "weight " + what)
    assert ops.weight_bytes(st) == N * K + N * 8
    q, s, z = ops.quantize_rows(x)
    qo = oracle.quantize_rows(conv, x)
    for got, want, what in zip((q, s, z), qo, ("q", "s", "z")):
        assert_bits_equal(got, want, what)
    y, work = ops.linear_ex(q, s, z, st, bias)
    yo, wo = oracle.linear(conv, q, s, z, *want_w, bias=bias)
    assert_bits_equal(work, wo, "work")
    assert_bits_equal(y, yo, "y")
    y2, work2 = ops.linear_ex(q, s, z, st, bias, y=yo, accumulate=True)
    yo2, _ = oracle.linear(conv, q, s, z, *want_w, bias=bias, y=yo, accumulate=True)
    assert_bits_equal(y2, yo2, "y accumulate")
    sub = min(5, M)
    _, work_sub = ops.linear_ex(q[-sub:], s[-sub:], z[-sub:], st, bias)
    assert_bits_equal(work_sub, wo[-sub:], "cross-M work")
    (r1, rr, r2) = ops.quantize_rows_residual(x)
    (o1, orr, o2) = oracle.quantize_rows_residual(conv, x)
    for got, want in zip(r1 + (rr,) + r2, o1 + (orr,) + o2):
        assert_bits_equal(got, want, "residual quantization")
    ops.weight_free(st)
    assert not st.data and ops.weight_bytes(st) == 0
    assert ops.last_error() == 0


def test_hand_built_weight_struct(ops, oracle):
    # ops.c:388-391 builds an IroInt8Weight by hand (unit scales, zero colsum)
    a, b, want = oracle.selfcheck_kat()
    st = iro_hip._Int8Weight()
    bq = np.ascontiguousarray(b, np.int8)
    sc = np.ones(5, np.float32)
    cs = np.zeros(5, np.int32)
    import ctypes as C
    st.data = bq.ctypes.data_as(C.POINTER(C.c_int8))
    st.scale = sc.ctypes.data_as(C.POINTER(C.c_float))
    st.colsum = cs.ctypes.data_as(C.POINTER(C.c_int32))
    st.N, st.K = 5, 64
    _, work = ops.linear_ex(a, np.ones(3, np.float32), np.zeros(3, np.int32), st)
    assert np.array_equal(work, want)
