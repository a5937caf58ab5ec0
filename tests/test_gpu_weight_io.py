"""Weights from a checkpoint and the packed weight as a file, on the GPU.

A weight built from a safetensors tensor must equal the weight built from
the same fp32 values on the device (codes, scales, sums: the quantization of
ops.c:259-293, checked against the oracle too); F16 / BF16 tensors are widened
exactly first.  A packed weight written to a file and read back must give the
same bits and the same GEMM outputs, keep its layout and parts, and refuse a
corrupted file or a context of the other rounding convention.
"""
import json
import os
import struct

import numpy as np
import pytest

import iro_hip
from iro_synth import gauss
from parity_util import assert_bits_equal

pytestmark = pytest.mark.gpu


def _bf16_file(path, name, a32):
    bits = (a32.view(np.uint32) >> 16).astype(np.uint16)  # truncation: exact bf16 values
    h = json.dumps({name: {"dtype": "BF16", "shape": list(a32.shape),
                           "data_offsets": [0, bits.nbytes]}}).encode()
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + bits.tobytes())
    return (bits.astype(np.uint32) << 16).view(np.float32).reshape(a32.shape)


def test_weight_from_checkpoint_equals_device_path(ctx, oracle, tmp_path):
    from safetensors.numpy import save_file
    w32 = gauss(501, (300, 200), 0.02)
    w16 = gauss(502, (64, 96), 0.02).astype(np.float16)
    wt = gauss(503, (80, 48), 0.02)  # [K, N] source
    p = str(tmp_path / "m.safetensors")
    save_file({"a.weight": w32, "b.weight": w16, "t.weight": wt}, p)
    pb = str(tmp_path / "bf.safetensors")
    wb = _bf16_file(pb, "c.weight", gauss(504, (40, 128), 0.02))
    st, sb = iro_hip.Safetensors(p), iro_hip.Safetensors(pb)
    try:
        cases = [(ctx.weight_from_st(st, "a.weight"), w32, False),
                 (ctx.weight_from_st(st, "b.weight"), w16.astype(np.float32), False),
                 (ctx.weight_from_st(sb, "c.weight"), wb, False),
                 (ctx.weight_from_st(st, "t.weight", transposed=True), wt, True)]
        for W, src, tr in cases:
            N, K = (src.shape[1], src.shape[0]) if tr else src.shape
            ref = ctx.weight(ctx.to_device(np.ascontiguousarray(src)), N, K, transposed=tr)
            for got, want, what in zip(W.export(), ref.export(), ("codes", "scales", "colsum")):
                assert_bits_equal(got, want, what)
            want = (oracle.weight_quantize_transposed(ctx.convention, src, N, K) if tr
                    else oracle.weight_quantize(ctx.convention, src))
            for got, o, what in zip(W.export(), want, ("codes", "scales", "colsum")):
                assert_bits_equal(got, o, "oracle " + what)
        with pytest.raises(iro_hip.HipError, match="no tensor"):
            ctx.weight_from_st(st, "missing")
    finally:
        st.close()
        sb.close()


def test_packed_weight_file_round_trip(ctx, oracle, tmp_path):
    D, M = 256, 70
    parts = [gauss(510 + i, (D, D), 0.02) for i in range(4)]
    Wq = ctx.weight_fused([ctx.to_device(w) for w in parts], [D] * 4, D, layout=0)
    w1, w3 = gauss(520, (320, D), 0.02), gauss(521, (320, D), 0.02)
    W13 = ctx.weight_fused([ctx.to_device(w1), ctx.to_device(w3)], [320, 320], D, layout=1)
    x = ctx.to_device(gauss(530, (M, D)))
    for W in (Wq, W13):
        path = str(tmp_path / "w.iro8")
        ctx.weight_save(W, path)
        L = ctx.weight_load(path)
        assert (L.N, L.K, L.nbytes()) == (W.N, W.K, W.nbytes())
        for got, want, what in zip(L.export(), W.export(), ("codes", "scales", "colsum")):
            assert_bits_equal(got, want, what)
    # the loaded fused weights run the fused projections with the same bits
    path = str(tmp_path / "q.iro8")
    ctx.weight_save(Wq, path)
    Lq = ctx.weight_load(path)
    outs = [[ctx.empty((M, D), np.float32) for _ in range(4)] for _ in range(2)]
    ctx.dit_qkvg(x, M, Wq, *outs[0])
    ctx.dit_qkvg(x, M, Lq, *outs[1])
    for a, b in zip(*outs):
        assert_bits_equal(b.numpy(), a.numpy(), "QKVG from the loaded weight")


def test_packed_weight_file_keeps_given_sums(ctx, tmp_path):
    # a caller-supplied colsum that disagrees with the codes (ops.c:388-391)
    N, K = 40, 64
    q = np.random.default_rng(1).integers(-127, 128, (N, K), dtype=np.int8)
    s = np.full(N, 0.01, np.float32)
    cs = np.zeros(N, np.int32)
    W = ctx.weight_from_host(q, s, cs)
    path = str(tmp_path / "h.iro8")
    ctx.weight_save(W, path)
    L = ctx.weight_load(path)
    for got, want, what in zip(L.export(), W.export(), ("codes", "scales", "colsum")):
        assert_bits_equal(got, want, what)


def test_packed_weight_file_refusals(ctx, tmp_path):
    W = ctx.weight(ctx.to_device(gauss(540, (64, 128), 0.02)), 64, 128)
    path = str(tmp_path / "w.iro8")
    ctx.weight_save(W, path)
    raw = bytearray(open(path, "rb").read())
    bad = str(tmp_path / "bad.iro8")
    raw2 = bytearray(raw)
    raw2[-5] ^= 0x40  # a payload byte
    open(bad, "wb").write(raw2)
    with pytest.raises(iro_hip.HipError, match="checksum"):
        ctx.weight_load(bad)
    open(bad, "wb").write(raw[:-10])  # truncated
    with pytest.raises(iro_hip.HipError, match="not a packed int8 weight"):
        ctx.weight_load(bad)
    open(bad, "wb").write(b"IROW8PK0" + raw[8:])  # wrong magic
    with pytest.raises(iro_hip.HipError, match="not a packed int8 weight"):
        ctx.weight_load(bad)
    from conftest import _ctx
    other = _ctx(1 - ctx.convention)  # the session's context of the other convention
    with pytest.raises(iro_hip.HipError, match="convention"):
        other.weight_load(path)
