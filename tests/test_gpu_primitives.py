"""Parity of the ops.h-level primitives on the GPU against the oracle.

Every comparison is bit-exact: int8/u8 codes, scales, zero points, int32
sums and fp32 epilogue outputs, in both rounding conventions.  Cases follow
tests/test_int8_ops.c:118-134 (shapes, outlier column, degenerate rows) and
the BASELINE shapes (K = 1024 / 2816, N up to 4096).
"""
import numpy as np
import pytest

from iro_synth import gauss, heavy_tail
from parity_util import assert_bits_equal

pytestmark = pytest.mark.gpu


def test_selfcheck_known_answer(ctx):
    # ops.c:375-398 through the MFMA GEMM (also run at context creation)
    assert ctx.selfcheck() == 0


@pytest.mark.parametrize("N,K", [(32, 64), (96, 128), (160, 1280), (184, 1280), (1024, 1024),
                                 (300, 100), (7, 3584)])
def test_weight_quantize(ctx, oracle, N, K):
    w = gauss(43 + N + K, (N, K), 0.02)
    w[min(3, N - 1)] = 0.0  # all-zero row: scale 1, codes 0
    if N > 5:
        w[5, K // 2] = 0.3  # one large weight
    W = ctx.weight(ctx.to_device(w), N, K)
    q, s, cs = W.export()
    qo, so, cso = oracle.weight_quantize(ctx.convention, w)
    assert_bits_equal(q, qo, "weight codes")
    assert_bits_equal(s, so, "weight scales")
    assert_bits_equal(cs, cso, "weight colsum")
    assert W.nbytes() == N * K + N * 8  # ops.c:316-319


def test_weight_quantize_transposed(ctx, oracle):
    N, K = 96, 80
    w_kn = gauss(7, (K, N), 0.02)
    W = ctx.weight(ctx.to_device(w_kn), N, K, transposed=True)
    got = W.export()
    want = oracle.weight_quantize_transposed(ctx.convention, w_kn, N, K)
    for g, o, what in zip(got, want, ("codes", "scales", "colsum")):
        assert_bits_equal(g, o, "transposed weight " + what)


def _rows(M, K, seed, heavy):
    x = gauss(seed, (M, K))
    if heavy:
        x = heavy_tail(x, seed + 1)
    if M > 2:
        x[1] = 0.0          # zero row (tests/test_int8_ops.c:127-134)
        x[2] = 2.5          # constant positive row
    if M > 4:
        x[3] = -np.abs(x[3])  # all non-positive row
        x[4, 17 % K] = 20.0   # outlier (tests/test_int8_ops.c:49-53)
    if M > 6:
        x[5] = -0.0           # signed zeros only: range [0, 0] whatever its signs
        x[6] = -np.abs(x[6])  # non-positive with negative zeros: hi = +0
        x[6, ::3] = -0.0
    return x


QROWS = [(1, 64, 0), (7, 64, 0), (23, 128, 1), (256, 1024, 0), (2250, 1024, 1),
         (300, 2816, 1), (2249, 2816, 1), (37, 3000, 1), (5, 100, 0), (33, 4100, 0),
         (9, 5000, 1), (4, 16, 0)]


@pytest.mark.parametrize("M,K,heavy", QROWS)
def test_quantize_rows(ctx, oracle, M, K, heavy):
    x = _rows(M, K, 100 + M + K, heavy)
    xd = ctx.to_device(x)
    q, s, z = ctx.empty((M, K), np.uint8), ctx.empty(M, np.float32), ctx.empty(M, np.int32)
    ctx.quantize_rows(xd, q, s, z)
    qo, so, zo = oracle.quantize_rows(ctx.convention, x)
    assert_bits_equal(q.numpy(), qo, "codes")
    assert_bits_equal(s.numpy(), so, "row scales")
    assert_bits_equal(z.numpy(), zo, "zero points")
    if M > 2:
        # closed forms: zero row -> s=1, zp=0, q=0; constant c>0 -> zp=0, q=255
        assert so[1] == 1.0 and zo[1] == 0 and not qo[1].any()
        assert zo[2] == 0 and (qo[2] == 255).all()


@pytest.mark.parametrize("M,K,heavy", QROWS)
def test_quantize_rows_residual(ctx, oracle, M, K, heavy):
    x = _rows(M, K, 200 + M + K, heavy)
    xd = ctx.to_device(x)
    q1, q2 = ctx.empty((M, K), np.uint8), ctx.empty((M, K), np.uint8)
    s1, s2 = ctx.empty(M, np.float32), ctx.empty(M, np.float32)
    z1, z2 = ctx.empty(M, np.int32), ctx.empty(M, np.int32)
    r = ctx.empty((M, K), np.float32)
    ctx.quantize_rows_residual(xd, q1, s1, z1, r, q2, s2, z2)
    (q1o, s1o, z1o), ro, (q2o, s2o, z2o) = oracle.quantize_rows_residual(ctx.convention, x)
    for got, want, what in ((q1, q1o, "q1"), (s1, s1o, "s1"), (z1, z1o, "z1"), (r, ro, "residual"),
                            (q2, q2o, "q2"), (s2, s2o, "s2"), (z2, z2o, "z2")):
        assert_bits_equal(got.numpy(), want, what)


LIN = [(7, 32, 64), (23, 96, 128), (112, 160, 1280), (37, 184, 1280), (256, 1024, 1024),
       (300, 4096, 1024), (129, 300, 2816), (1, 1, 16), (5, 40, 100), (200, 512, 3584)]


def _linear_inputs(oracle, conv, M, N, K, seed):
    x = _rows(M, K, seed, heavy=True)
    w = gauss(seed + 1, (N, K), 0.02)
    b = gauss(seed + 2, (N,), 0.01)
    y0 = gauss(seed + 3, (M, N))
    wq = oracle.weight_quantize(conv, w)
    q = oracle.quantize_rows(conv, x)
    return x, w, b, y0, wq, q


@pytest.mark.parametrize("M,N,K", LIN)
@pytest.mark.parametrize("bias,accumulate", [(0, 0), (1, 0), (0, 1), (1, 1)],
                         ids=["plain", "bias", "acc", "acc+bias"])
def test_int8_linear_ex(ctx, oracle, M, N, K, bias, accumulate):
    conv = ctx.convention
    x, w, b, y0, wq, (q, s, z) = _linear_inputs(oracle, conv, M, N, K, 300 + M + N + K)
    W = ctx.weight(ctx.to_device(w), N, K)  # quantized and packed on the GPU
    qd, sd, zd = ctx.to_device(q), ctx.to_device(s), ctx.to_device(z)
    bd = ctx.to_device(b) if bias else None
    yd = ctx.to_device(y0)
    work = ctx.empty((M, N), np.int32)
    ctx.linear_ex(qd, sd, zd, W, bd, yd, M, work, accumulate)
    yo, wo = oracle.linear(conv, q, s, z, *wq, bias=b if bias else None, y=y0,
                           accumulate=accumulate)
    assert_bits_equal(work.numpy(), wo, "int32 work")
    assert_bits_equal(yd.numpy(), yo, "fp32 y")


@pytest.mark.parametrize("M,N,K", [(37, 184, 1280), (300, 1024, 2816), (8, 64, 48)])
def test_int8_linear_two_term(ctx, oracle, M, N, K):
    conv = ctx.convention
    x = _rows(M, K, 400 + M, heavy=True)
    w = gauss(401, (N, K), 0.02)
    b = gauss(402, (N,), 0.01)
    wq = oracle.weight_quantize(conv, w)
    (q1, s1, z1), _, (q2, s2, z2) = oracle.quantize_rows_residual(conv, x)
    W = ctx.weight_from_host(*wq)
    dev = [ctx.to_device(a) for a in (q1, s1, z1, q2, s2, z2)]
    yd = ctx.empty((M, N), np.float32)
    ctx.linear_two_term(*dev, W, ctx.to_device(b), yd, M)
    # dacvae.c:677-681 order: plane 1 with bias, plane 2 accumulated
    y1, _ = oracle.linear(conv, q1, s1, z1, *wq, bias=b)
    yo, _ = oracle.linear(conv, q2, s2, z2, *wq, y=y1, accumulate=True)
    assert_bits_equal(yd.numpy(), yo, "two-term y")


def test_cross_m_determinism(ctx, oracle):
    # tests/test_int8_ops.c:87-97: the last rows alone give identical sums
    conv = ctx.convention
    M, N, K = 37, 184, 1280
    x, w, b, y0, wq, (q, s, z) = _linear_inputs(oracle, conv, M, N, K, 500)
    W = ctx.weight_from_host(*wq)
    full = ctx.empty((M, N), np.int32)
    ctx.linear_ex(ctx.to_device(q), ctx.to_device(s), ctx.to_device(z), W, None,
                  ctx.empty((M, N), np.float32), M, full)
    sub = ctx.empty((5, N), np.int32)
    ctx.linear_ex(ctx.to_device(q[-5:]), ctx.to_device(s[-5:]), ctx.to_device(z[-5:]), W, None,
                  ctx.empty((5, N), np.float32), 5, sub)
    assert_bits_equal(sub.numpy(), full.numpy()[-5:], "cross-M int32")


def test_inconsistent_colsum_keeps_raw_sums(ctx, oracle):
    # ops.c:388-391 builds a weight whose colsum is zero: `work` must still be
    # the raw u8 x s8 sum (cblas_gemm_s8u8s32 semantics), and the epilogue
    # uses the colsum as given.
    conv = ctx.convention
    M, N, K = 9, 70, 192
    x, w, b, y0, (wq, sw, cs), (q, s, z) = _linear_inputs(oracle, conv, M, N, K, 600)
    fake = np.arange(N, dtype=np.int32) * 3 - 50
    W = ctx.weight_from_host(wq, sw, fake)
    yd, work = ctx.empty((M, N), np.float32), ctx.empty((M, N), np.int32)
    ctx.linear_ex(ctx.to_device(q), ctx.to_device(s), ctx.to_device(z), W, None, yd, M, work)
    yo, wo = oracle.linear(conv, q, s, z, wq, sw, fake)
    assert_bits_equal(work.numpy(), wo, "raw sums")
    assert_bits_equal(yd.numpy(), yo, "y with the given colsum")


def test_silu_gate_pieces_on_every_float(ctx, oracle):
    """The SiLU gate (ops.c:781-784) on the device: its glibc-exact expf gives,
    over all 2^32 inputs, the digest of the oracle's restatement (itself equal
    to libm's expf on every input, tests/test_oracle_pins.py), and its fast
    correctly rounded quotient a / (1 + expf(-a)) equals the IEEE division for
    every a."""
    digest, mismatches = ctx.selfcheck_silu()
    assert mismatches == 0
    assert digest == oracle.expf_digest()


def test_sqrt_and_reciprocal_on_every_float(ctx, oracle):
    """The device's sqrtf and 1 / x, which the adaLN apply uses, equal the
    host's IEEE results on all 2^32 inputs (digests of every result)."""
    assert ctx.selfcheck_fp32() == oracle.fp32_digests()


def test_tanhf_on_every_float(ctx_strict, oracle):
    """The device's fdlibm tanhf (the adaLN gate, dit.c:588) hashed over all
    2^32 inputs equals the hash of the oracle's restatement, which equals
    libm's tanhf on every input (tests/test_oracle_pins.py)."""
    assert ctx_strict.selfcheck_tanhf() == oracle.tanhf_digest()


@pytest.mark.parametrize("M,K,N,bias", [(750, 32, 1280, True), (48, 1280, 32, True),
                                        (200, 512, 1280, False), (3, 100, 130, True),
                                        (1, 1, 1, False), (2250, 1280, 32, True),
                                        (37, 300, 50, False), (9, 1000, 64, True)])
def test_linear_f32(ctx, oracle, M, K, N, bias):
    """ops.c:221-234 on the device: K-order chains, bit for bit against the
    oracle (pinned against the scalar reference build); zero rows and -0
    weights included."""
    x, w = gauss(750, (M, K)), gauss(751, (N, K), 0.05)
    x[0, :] = 0.0
    if N > 1:
        w[1, :] = -w[1, :] * 0.0
    b = gauss(752, (N,), 0.1) if bias else None
    y = ctx.empty((M, N), np.float32)
    ctx.linear_f32(ctx.to_device(x), M, K, ctx.to_device(w), N,
                   None if b is None else ctx.to_device(b), y)
    assert_bits_equal(y.numpy(), oracle.linear_f32(x, w, b), "y")


@pytest.mark.parametrize("M,D", [(60, 1280), (2250, 1024), (1, 64)])
def test_rmsnorm_f32(ctx, oracle, M, D):
    """ops.c:738-747 on the device, bit for bit against the oracle."""
    x, w = gauss(753, (M, D)), gauss(754, (D,), 0.2) + 1.0
    x[0] = 0.0
    y = ctx.empty((M, D), np.float32)
    ctx.rmsnorm_f32(ctx.to_device(x), M, D, ctx.to_device(w), 1e-6, y)
    assert_bits_equal(y.numpy(), oracle.rmsnorm(x, w, 1e-6), "y")
