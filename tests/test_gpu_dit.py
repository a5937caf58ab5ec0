"""Parity of the fused DiT projections on the GPU against the oracle.

The oracle runs the reference's call sequence: one shared quantization and
separate GEMMs (dit.c:786-792 QKVG, dit.c:944-947 W1/W3), the SwiGLU gate
(ops.c:781-784), the two-term W2 input (dit.c:963-966, ops.c:427-442) and
the gated residual (dit.c:1013-1020, 1032-1039).  The fused kernels must
give the same bits.

The SwiGLU gate calls expf.  The strict build calls glibc's scalar expf,
which the kernel restates exactly (the restatement equals glibc's expf on
all 2^32 inputs, see tests/test_oracle_pins.py), so the hidden state is
bit-exact.  The fast-math build evaluates the gate with libmvec expf and an
rcpps Newton step whose results depend on the host CPU, so that convention
has no portable reference for the gate: the kernel keeps the strict gate
there too ("parity unpinned" for the fast-math hidden state), and W2 is
still pinned bit-exactly at its own boundary from the GPU's hidden state.
"""
import numpy as np
import pytest

import iro_hip
from iro_synth import gauss, heavy_tail, rms_rows
from parity_util import assert_bits_equal, rel_err

pytestmark = pytest.mark.gpu

# D = 1024, H = 2816, M = 3 CFG branches x 750 frames.
SHAPES = [  # (B, S, D, H)
    (1, 37, 128, 96),
    (3, 750, 1024, 2816),
]


def _qkvg_weights(D, seed):
    return [gauss(seed + i, (D, D), 0.02) for i in range(4)]


@pytest.mark.parametrize("B,S,D,H", SHAPES)
@pytest.mark.parametrize("residual", [0, 1], ids=["one-term", "two-term"])
def test_qkvg(ctx, oracle, B, S, D, H, residual):
    conv = ctx.convention
    M = B * S
    x = rms_rows(gauss(11, (M, D)))
    ws = _qkvg_weights(D, 20)
    W = ctx.weight_fused([ctx.to_device(w) for w in ws], [D] * 4, D, layout=0)
    outs = [ctx.empty((M, D), np.float32) for _ in range(4)]
    ctx.dit_qkvg(ctx.to_device(x), M, W, *outs, residual=residual)
    if residual:
        (q1, s1, z1), _, (q2, s2, z2) = oracle.quantize_rows_residual(conv, x)
    else:
        q1, s1, z1 = oracle.quantize_rows(conv, x)
    for name, w, got in zip("qkvg", ws, outs):
        wq = oracle.weight_quantize(conv, w)
        y, _ = oracle.linear(conv, q1, s1, z1, *wq)
        if residual:
            y, _ = oracle.linear(conv, q2, s2, z2, *wq, y=y, accumulate=True)
        assert_bits_equal(got.numpy(), y, f"{name} projection")


@pytest.mark.parametrize("B,S,D,H", SHAPES)
@pytest.mark.parametrize("residual", [0, 1], ids=["one-term", "two-term"])
def test_wo_gated_residual(ctx, oracle, B, S, D, H, residual):
    conv = ctx.convention
    M = B * S
    mix = gauss(31, (M, D))
    w = gauss(32, (D, D), 0.02)
    gate = gauss(33, (B, D), 0.5)
    x0 = gauss(34, (M, D))
    W = ctx.weight(ctx.to_device(w), D, D)
    xres = ctx.to_device(x0)
    ctx.dit_linear_gated(ctx.to_device(mix), M, W, residual, x_res=xres, gate=ctx.to_device(gate),
                         S=S)
    out = ctx.empty((M, D), np.float32)
    ctx.dit_linear_gated(ctx.to_device(mix), M, W, residual, out=out)
    wq = oracle.weight_quantize(conv, w)
    if residual:
        (q1, s1, z1), _, (q2, s2, z2) = oracle.quantize_rows_residual(conv, mix)
        y, _ = oracle.linear(conv, q1, s1, z1, *wq)
        y, _ = oracle.linear(conv, q2, s2, z2, *wq, y=y, accumulate=True)
    else:
        y, _ = oracle.linear(conv, *oracle.quantize_rows(conv, mix), *wq)
    assert_bits_equal(out.numpy(), y, "Wo branch")
    want = oracle.gated_residual(conv, x0, gate, y, B, S)
    assert_bits_equal(xres.numpy(), want, "x += gate * Wo")


def _swiglu_case(ctx, oracle, B, S, D, H, heavy, residual_w2):
    conv = ctx.convention
    M = B * S
    h = gauss(41, (M, D))
    if heavy:
        h = heavy_tail(h, 42)  # 1% of activations x20 (BASELINE cfg2 variant)
    w1, w3 = gauss(43, (H, D), 0.02), gauss(44, (H, D), 0.02)
    w2 = gauss(45, (D, H), 0.02)
    gate = gauss(46, (B, D), 0.5)
    x0 = gauss(47, (M, D))
    W13 = ctx.weight_fused([ctx.to_device(w1), ctx.to_device(w3)], [H, H], D, layout=1)
    W2 = ctx.weight(ctx.to_device(w2), D, H)
    hidden = ctx.empty((M, H), np.float32)
    xres = ctx.to_device(x0)
    ctx.dit_swiglu(ctx.to_device(h), M, W13, W2, residual_w13=False, residual_w2=residual_w2,
                   hidden=hidden, x_res=xres, gate=ctx.to_device(gate), S=S)
    hid = hidden.numpy()
    # W1, W3 on one shared quantization, then the gate (glibc expf)
    q, s, z = oracle.quantize_rows(conv, h)
    a, _ = oracle.linear(conv, q, s, z, *oracle.weight_quantize(conv, w1))
    b, _ = oracle.linear(conv, q, s, z, *oracle.weight_quantize(conv, w3))
    hid_o = oracle.silu_mul(a, b)
    err = rel_err(hid, hid_o)
    mism = int((hid.view(np.int32) != hid_o.view(np.int32)).sum())
    # W2 at its own boundary, from the GPU's hidden state
    w2q = oracle.weight_quantize(conv, w2)
    if residual_w2:
        (q1, s1, z1), _, (q2, s2, z2) = oracle.quantize_rows_residual(conv, hid)
        y, _ = oracle.linear(conv, q1, s1, z1, *w2q)
        y, _ = oracle.linear(conv, q2, s2, z2, *w2q, y=y, accumulate=True)
    else:
        y, _ = oracle.linear(conv, *oracle.quantize_rows(conv, hid), *w2q)
    want = oracle.gated_residual(conv, x0, gate, y, B, S)
    return err, mism, hid.size, xres.numpy(), want


@pytest.mark.parametrize("B,S,D,H", SHAPES)
@pytest.mark.parametrize("heavy", [0, 1], ids=["gauss", "heavy-tail"])
def test_swiglu_mlp(ctx, oracle, B, S, D, H, heavy):
    err, mism, n, got, want = _swiglu_case(ctx, oracle, B, S, D, H, heavy, residual_w2=True)
    assert mism == 0, f"hidden state: {mism}/{n} differ from silu(w1)*w3, max rel {err.max():.3g}"
    assert_bits_equal(got, want, "x += gate * W2(two-term)")


def test_swiglu_mlp_single_term_w2(ctx, oracle):
    err, mism, n, got, want = _swiglu_case(ctx, oracle, 2, 40, 256, 320, 0, residual_w2=False)
    assert mism == 0, f"hidden state: {mism}/{n} differ"
    assert_bits_equal(got, want, "x += gate * W2(one-term)")


# The bench's rows, one CFG branch, a last band of 2 rows (M = 130), and a
# hidden width (320) that leaves padded 32-column blocks in the last slab.
BAND_SHAPES = [  # (B, S, D, H)
    (3, 750, 1024, 2816),
    (1, 750, 1024, 2816),
    (2, 65, 256, 320),
]


@pytest.mark.parametrize("B,S,D,H", BAND_SHAPES)
@pytest.mark.parametrize("residual_w2", [True, False], ids=["two-term", "one-term"])
def test_swiglu_band_quant_equals_row_quant(ctx, B, S, D, H, residual_w2):
    """With the band quantization switched on and no hidden buffer, the
    W1/W3 kernel quantizes the hidden state itself (the blocks of each
    64-row band merge their row ranges through device memory); x must equal
    the path that stores the hidden state in fp32 and quantizes its rows, on
    two launches in a row and then on fewer rows (the band state is back to
    zero after every launch)."""
    M = B * S
    h = heavy_tail(gauss(51, (M, D)), 52)  # ranges set by a few columns
    w1, w3 = gauss(53, (H, D), 0.02), gauss(54, (H, D), 0.02)
    w2 = gauss(55, (D, H), 0.02)
    gate = ctx.to_device(gauss(56, (B, D), 0.5))
    x0 = gauss(57, (M, D))
    W13 = ctx.weight_fused([ctx.to_device(w1), ctx.to_device(w3)], [H, H], D, layout=1)
    W2 = ctx.weight(ctx.to_device(w2), D, H)
    hd = ctx.to_device(h)
    hidden = ctx.empty((M, H), np.float32)

    def run(rows, b, s, hid):
        xres = ctx.to_device(x0[:rows])
        ctx.dit_swiglu(hd, rows, W13, W2, residual_w2=residual_w2, hidden=hid, x_res=xres,
                       gate=gate, S=s)
        ctx.sync()  # a band wait that gave up is reported here
        return xres.numpy()

    want = run(M, B, S, hidden)
    ctx.set_gemm_tile(-7, 1)
    ctx.profile(True)
    ctx.profile_reset()
    try:
        first = run(M, B, S, None)
        second = run(M, B, S, None)
        M2 = M // 3 if M >= 99 else M - 33
        want2 = run(M2, 1, M2, hidden)
        third = run(M2, 1, M2, None)
        kinds = ctx.profile_read()
    finally:
        ctx.profile(False)
        ctx.set_gemm_tile(-7, 0)
    assert kinds.get("gemm_swiglu_quant", (0,))[0] == 3, f"fused W1/W3 not taken: {kinds}"
    assert_bits_equal(first, want, "band-quantized hidden state, first launch")
    assert_bits_equal(second, want, "band-quantized hidden state, second launch")
    assert_bits_equal(third, want2, f"band-quantized hidden state at {M2} rows")


@pytest.mark.parametrize("B,S,D", [
    (3, 750, 1024), (3, 40, 1280), (1, 1, 1024),    # registers, 2 rows per wave
    (2, 5, 600), (1, 3, 1500),                      # partial chunks; 1 row per wave
    (2, 33, 98), (2, 17, 2052),                     # rows kept in LDS
    (1, 9, 20000), (1, 7, 16390),                   # rows too long for LDS: chunked
])
def test_adaln_apply(ctx, oracle, B, S, D):
    """dit.c:593-606 on the device: bit-identical to the strict build's
    evaluation (the oracle's restatement, pinned against the reference build
    in tests/test_oracle_pins.py); the device evaluates the strict order in
    both conventions.  The shapes reach each of the three kernels."""
    x = gauss(620, (B * S, D))
    x[0] = 0.0
    if B * S > 2:
        x[1] = 1e-20
        x[2, ::5] *= 1e4
    shift = gauss(621, (B, D), 0.3)
    scale = gauss(622, (B, D), 0.3)
    h = ctx.empty((B * S, D), np.float32)
    ctx.dit_adaln_apply(ctx.to_device(x), B, S, D, ctx.to_device(shift), ctx.to_device(scale),
                        1e-6, h)
    assert_bits_equal(h.numpy(), oracle.adaln_apply(x, shift, scale, B, S, 1e-6), "adaLN h")


@pytest.mark.parametrize("B,S,D", [(3, 750, 1024), (2, 40, 1280), (1, 1, 64), (3, 7, 192)])
def test_qk_norm_rope(ctx, oracle, B, S, D):
    """dit.c:638-706 on the device, in place on q and k: bit-identical to the
    oracle's restatement (pinned bit for bit against the strict reference
    build in tests/test_oracle_pins.py), rotated and plain heads, positions
    across the rotation table, zero, tiny and large head rows."""
    q = gauss(640, (B * S, D))
    k = gauss(641, (B * S, D))
    q[0, :64] = 0.0
    if B * S > 2:
        k[1, :64] = 1e-20
        q[2, -64:] *= 1e4
    qw, kw = gauss(642, (D,), 0.2) + 1.0, gauss(643, (D,), 0.2) + 1.0
    qd, kd = ctx.to_device(q), ctx.to_device(k)
    ctx.dit_qk_norm_rope(qd, ctx.to_device(qw), kd, ctx.to_device(kw), B, S, D, 1e-6)
    want_q, want_k = oracle.head_norm_rope(q, qw, k, kw, B, S, 1e-6)
    assert_bits_equal(qd.numpy(), want_q, "q")
    assert_bits_equal(kd.numpy(), want_k, "k")


def test_qk_norm_rope_table_grows(ctx, oracle):
    """A call with more positions than any before rebuilds the context's
    rotation table; shorter calls after it use the prefix."""
    D = 1280
    qw, kw = gauss(652, (D,), 0.2) + 1.0, gauss(653, (D,), 0.2) + 1.0
    qwd, kwd = ctx.to_device(qw), ctx.to_device(kw)
    for (B, S) in [(1, 300), (1, 2500), (2, 100)]:
        q, k = gauss(650 + S, (B * S, D)), gauss(651 + S, (B * S, D))
        qd, kd = ctx.to_device(q), ctx.to_device(k)
        ctx.dit_qk_norm_rope(qd, qwd, kd, kwd, B, S, D, 1e-6)
        want_q, want_k = oracle.head_norm_rope(q, qw, k, kw, B, S, 1e-6)
        assert_bits_equal(qd.numpy(), want_q, f"q S={S}")
        assert_bits_equal(kd.numpy(), want_k, f"k S={S}")


@pytest.mark.parametrize("B,T,D", [(3, 64, 1280), (1, 5, 1024)])
def test_head_rmsnorm(ctx, oracle, B, T, D):
    """dit.c:619-636 (text and speaker keys): no rotation, one tensor."""
    x = gauss(660, (B * T, D))
    x[0, 64:128] = 0.0
    w = gauss(661, (D,), 0.2) + 1.0
    xd = ctx.to_device(x)
    ctx.dit_head_rmsnorm(xd, ctx.to_device(w), B, T, D, 1e-6)
    want, _ = oracle.head_norm_rope(x, w, None, None, B, T, 1e-6, rope=False)
    assert_bits_equal(xd.numpy(), want, "x")


def test_qk_norm_rope_rejects_bad_shapes(ctx):
    q = ctx.empty((4, 100), np.float32)
    with pytest.raises(iro_hip.HipError):
        ctx.dit_qk_norm_rope(q, q, q, q, 1, 4, 100, 1e-6)


def _attn_case(seed, B, S, C, D, shared, keep):
    """q, k, v, gate [B*S, D], context rows and a mask keeping `keep` rows of
    batch 0 (other batches keep every other row, the last keeps none)."""
    q, k, v, gate = (gauss(seed + i, (B * S, D)) for i in range(4))
    rows = 1 if shared else B
    ck, cv = gauss(seed + 4, (rows * C, D)), gauss(seed + 5, (rows * C, D))
    mask = np.zeros((B, C), np.uint8)
    mask[0, :keep] = 1
    for b in range(1, B - 1):
        mask[b, ::2] = 1
    return q, k, v, gate, ck, cv, mask


@pytest.mark.parametrize("B,D,R", [(1, 1280, 192), (4, 96, 40), (2, 200, 70), (3, 102, 30)])
def test_adaln_params_shapes(ctx, oracle, B, D, R):
    """dit.c:543-588 on the device against the oracle for both adaLNs of a
    block: one batch row (a plain step), four rows, widths and ranks that
    leave partial 64-wide tiles, and a width that is not a multiple of 4
    (the per-row-chain kernel instead of the LDS ring)."""
    cond = gauss(770, (B, 3 * D), 0.8)
    w = []
    for i in range(6):
        w += [gauss(771 + 3 * i, (R, D), 0.05), gauss(772 + 3 * i, (D, R), 0.05),
              gauss(773 + 3 * i, (D,), 0.1)]
    out = ctx.empty((2, 3, B, D), np.float32)
    ctx.dit_adaln_params(ctx.to_device(cond), B, D, R, [ctx.to_device(a) for a in w], out)
    got = out.numpy()
    for a in range(2):
        ws = w[9 * a:9 * a + 9]
        want = oracle.adaln_params(cond, ws[0::3], ws[1::3], ws[2::3])
        assert_bits_equal(got[a], want, f"adaLN {a}")


@pytest.mark.parametrize("B,S,C,D,shared,keep", [
    (2, 24, 9, 1280, 0, 4),       # reference-sized heads, per-batch context
    (3, 150, 40, 1024, 1, 40),    # shared context, ragged key tiles
    (3, 200, 130, 1024, 0, 130),  # more than one 128-key tile of context
    (1, 1, 1, 64, 0, 1),          # one query, one head, one context row
    (2, 70, 3, 128, 1, 0),        # no kept context rows in any batch
])
def test_attention_core(ctx, oracle, B, S, C, D, shared, keep):
    """dit.c:808-870 on the device: bit-identical to the oracle's attention
    core (pinned bit for bit against the scalar reference build's
    iro_dit_attention in tests/test_oracle_pins.py); large and tiny scores so
    that softmax terms and gates underflow."""
    q, k, v, gate, ck, cv, mask = _attn_case(680, B, S, C, D, shared, keep)
    q[0] *= 20.0
    gate[1 % (B * S)] *= 60.0
    actx = ctx.attn_context(mask, 1 if shared else B)
    try:
        mix = ctx.empty((B * S, D), np.float32)
        dev = [ctx.to_device(a) for a in (q, k, v, gate, ck, cv)]
        ctx.dit_attention(actx, dev[0], dev[1], dev[2], dev[3], B, S, D, dev[4], dev[5], mix)
        want = oracle.attention_core(q, k, v, gate, B, S, ck, cv, mask, 1 if shared else B)
        assert_bits_equal(mix.numpy(), want, "mix")
    finally:
        actx.destroy()


def test_attention_core_full_shape(ctx, oracle):
    """The stack's shape (3 x 750 tokens, 16 heads) with up to 250 kept
    context rows: the whole output bit for bit against the oracle."""
    B, S, C, D = 3, 750, 300, 1024
    q, k, v, gate, ck, cv, mask = _attn_case(690, B, S, C, D, False, 250)
    actx = ctx.attn_context(mask, B)
    try:
        mix = ctx.empty((B * S, D), np.float32)
        dev = [ctx.to_device(a) for a in (q, k, v, gate, ck, cv)]
        ctx.dit_attention(actx, dev[0], dev[1], dev[2], dev[3], B, S, D, dev[4], dev[5], mix)
        want = oracle.attention_core(q, k, v, gate, B, S, ck, cv, mask, B)
        assert_bits_equal(mix.numpy(), want, "mix")
    finally:
        actx.destroy()


def test_attention_rejects_mismatched_context(ctx):
    mask = np.ones((2, 3), np.uint8)
    actx = ctx.attn_context(mask, 2)
    try:
        x = ctx.empty((3 * 4, 64), np.float32)
        with pytest.raises(iro_hip.HipError):
            ctx.dit_attention(actx, x, x, x, x, 3, 4, 64, x, x, x)
    finally:
        actx.destroy()


@pytest.mark.parametrize("K,T", [(512, 120), (768, 16)])
def test_context_kv(ctx, oracle, K, T):
    """dit.c:708-726 on the device: iro_hip_linear_f32 for K and V (no bias),
    iro_hip_dit_head_rmsnorm on K; bit for bit against the oracle's
    composition (pinned against iro_dit_text_kv / iro_dit_speaker_kv of the
    scalar reference build in tests/test_oracle_pins.py)."""
    D, eps = 1280, 1e-6
    x = gauss(770, (T, K))
    wk, wv = gauss(771, (D, K), 0.05), gauss(772, (D, K), 0.05)
    kn = gauss(773, (D,), 0.2) + 1.0
    xd = ctx.to_device(x)
    k, v = ctx.empty((T, D), np.float32), ctx.empty((T, D), np.float32)
    ctx.linear_f32(xd, T, K, ctx.to_device(wk), D, None, k)
    ctx.linear_f32(xd, T, K, ctx.to_device(wv), D, None, v)
    ctx.dit_head_rmsnorm(k, ctx.to_device(kn), 1, T, D, eps)
    want_k, _ = oracle.head_norm_rope(oracle.linear_f32(x, wk), kn, None, None, 1, T, eps,
                                      rope=False)
    assert_bits_equal(k.numpy(), want_k, "k")
    assert_bits_equal(v.numpy(), oracle.linear_f32(x, wv), "v")
