"""ctypes bindings for the CPU checker (TEST INFRASTRUCTURE ONLY).

`Oracle` wraps liboracle.so, the C restatement of irodori-c's int8 W8A8
path (iro_oracle.c).  `Reference` wraps oracle/_ref/libref_{strict,fast}.so,
the reference's own ops.c/dacvae.c compiled from its sources by
`make -C oracle ref`; it only exists where the reference sources were
present when the checker was built.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  The HIP product path never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
STRICT, GCC_FASTMATH = 0, 1

_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)


def _p(a, ct):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ct)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    """The C restatement (iro_oracle.c), both rounding conventions."""

    def __init__(self, path: str | None = None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        self.lib = L = C.CDLL(path)
        L.orc_weight_quantize.argtypes = [C.c_int, _f32p, C.c_int, C.c_int, _i8p, _f32p, _i32p]
        L.orc_weight_quantize_transposed.argtypes = L.orc_weight_quantize.argtypes
        L.orc_quantize_rows.argtypes = [C.c_int, _f32p, C.c_int, C.c_int, _u8p, _f32p, _i32p]
        L.orc_quantize_rows_residual.argtypes = [C.c_int, _f32p, C.c_int, C.c_int, _u8p, _f32p,
                                                 _i32p, _f32p, _u8p, _f32p, _i32p]
        L.orc_gemm_u8s8.argtypes = [_u8p, _i8p, _i32p, C.c_int, C.c_int, C.c_int, C.c_int]
        L.orc_epilogue.argtypes = [C.c_int, _i32p, _f32p, _i32p, _f32p, _i32p, _f32p, _f32p,
                                   C.c_int, C.c_int, C.c_int]
        L.orc_selfcheck_kat.argtypes = [_u8p, _i8p, _i32p]
        L.orc_silu_mul.argtypes = [_f32p, _f32p, C.c_size_t]
        L.orc_expf_restated.argtypes = [C.c_float]
        L.orc_expf_restated.restype = C.c_float
        L.orc_expf_mismatches.argtypes = [C.c_int]
        L.orc_expf_mismatches.restype = C.c_longlong
        L.orc_expf_digest.argtypes = [C.c_int]
        L.orc_expf_digest.restype = C.c_ulonglong
        L.orc_fp32_digests.argtypes = [C.c_int, C.POINTER(C.c_ulonglong),
                                       C.POINTER(C.c_ulonglong)]
        L.orc_adaln_apply.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_float,
                                      _f32p]
        L.orc_gated_residual.argtypes = [C.c_int, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        L.orc_rope_table.argtypes = [C.c_int, _f32p, _f32p]
        L.orc_linear_f32.argtypes = [_f32p, C.c_int, C.c_int, _f32p, C.c_int, _f32p, _f32p]
        L.orc_euler_update.argtypes = [C.c_int, _f32p, _f32p, C.c_size_t, C.c_int, C.c_int,
                                       C.c_int, C.c_int, C.c_float, C.c_float, C.c_float,
                                       C.c_float]
        L.orc_rmsnorm.argtypes = [_f32p, C.c_int, C.c_int, _f32p, C.c_float, _f32p]
        L.orc_tanhf.argtypes = [C.c_float]
        L.orc_tanhf.restype = C.c_float
        L.orc_tanhf_mismatches.argtypes = [C.c_int]
        L.orc_tanhf_mismatches.restype = C.c_longlong
        L.orc_tanhf_digest.argtypes = [C.c_int]
        L.orc_tanhf_digest.restype = C.c_ulonglong
        L.orc_adaln_params.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.POINTER(_f32p),
                                       C.POINTER(_f32p), C.POINTER(_f32p), _f32p]
        L.orc_head_norm_rope.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int,
                                         C.c_float, C.c_int]
        L.orc_head_norm_rope.restype = C.c_int
        L.orc_attention_core.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int,
                                         _f32p, _f32p, _u8p, C.c_int, C.c_int, _f32p, C.c_int]
        L.orc_attention_core.restype = C.c_int
        L.orc_conv1d_int8.argtypes = [C.c_int, _f32p, C.c_int, C.c_int, _i8p, _f32p, _i32p,
                                      C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _f32p, C.c_int,
                                      _f32p, _u8p, _f32p, _i32p, C.c_int]
        L.orc_conv1d_int8.restype = C.c_int
        L.orc_conv1d_output_length.argtypes = [C.c_int] * 5
        L.orc_conv1d_output_length.restype = C.c_int
        L.orc_convtranspose1d_int8.argtypes = [C.c_int, _f32p, C.c_int, C.c_int, _i8p, _f32p,
                                               _i32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                               _f32p, C.c_int, _f32p, C.c_int]
        L.orc_convtranspose1d_int8.restype = C.c_int
        L.orc_convtranspose1d_output_length.argtypes = [C.c_int] * 5
        L.orc_convtranspose1d_output_length.restype = C.c_int
        L.orc_conv1x1_skip_int8.argtypes = [C.c_int, _f32p, _f32p, C.c_int, _i8p, _f32p, _i32p,
                                            C.c_int, C.c_int, _f32p, C.c_int, _f32p, C.c_int]
        L.orc_conv1x1_skip_int8.restype = C.c_int
        L.orc_sinf.argtypes = [C.c_float]
        L.orc_sinf.restype = C.c_float
        L.orc_cosf.argtypes = [C.c_float]
        L.orc_cosf.restype = C.c_float
        L.orc_sincosf_mismatches.argtypes = [C.c_int, C.c_int]
        L.orc_sincosf_mismatches.restype = C.c_longlong
        L.orc_sincosf_digest.argtypes = [C.c_int, C.c_int]
        L.orc_sincosf_digest.restype = C.c_ulonglong
        L.orc_snake.argtypes = [C.c_int, _f32p, C.c_int, C.c_int, _f32p, _f32p, C.c_int, _f32p]
        self.threads = min(8, os.cpu_count() or 1)

    def weight_quantize(self, conv, w):
        w = _f32(w)
        N, K = w.shape
        q = np.empty((N, K), np.int8)
        s = np.empty(N, np.float32)
        cs = np.empty(N, np.int32)
        rc = self.lib.orc_weight_quantize(conv, _p(w, _f32p), N, K, _p(q, _i8p), _p(s, _f32p),
                                          _p(cs, _i32p))
        assert rc == 0
        return q, s, cs

    def weight_quantize_transposed(self, conv, w_kn, N, K):
        w_kn = _f32(w_kn)
        q = np.empty((N, K), np.int8)
        s = np.empty(N, np.float32)
        cs = np.empty(N, np.int32)
        rc = self.lib.orc_weight_quantize_transposed(conv, _p(w_kn, _f32p), N, K, _p(q, _i8p),
                                                     _p(s, _f32p), _p(cs, _i32p))
        assert rc == 0
        return q, s, cs

    def quantize_rows(self, conv, x):
        x = _f32(x)
        M, K = x.shape
        q = np.empty((M, K), np.uint8)
        s = np.empty(M, np.float32)
        z = np.empty(M, np.int32)
        self.lib.orc_quantize_rows(conv, _p(x, _f32p), M, K, _p(q, _u8p), _p(s, _f32p),
                                   _p(z, _i32p))
        return q, s, z

    def quantize_rows_residual(self, conv, x):
        x = _f32(x)
        M, K = x.shape
        q1 = np.empty((M, K), np.uint8)
        q2 = np.empty((M, K), np.uint8)
        r = np.empty((M, K), np.float32)
        s1, s2 = np.empty(M, np.float32), np.empty(M, np.float32)
        z1, z2 = np.empty(M, np.int32), np.empty(M, np.int32)
        self.lib.orc_quantize_rows_residual(conv, _p(x, _f32p), M, K, _p(q1, _u8p), _p(s1, _f32p),
                                            _p(z1, _i32p), _p(r, _f32p), _p(q2, _u8p),
                                            _p(s2, _f32p), _p(z2, _i32p))
        return (q1, s1, z1), r, (q2, s2, z2)

    def gemm(self, a, b):
        a = np.ascontiguousarray(a, np.uint8)
        b = np.ascontiguousarray(b, np.int8)
        M, K = a.shape
        N = b.shape[0]
        c = np.empty((M, N), np.int32)
        self.lib.orc_gemm_u8s8(_p(a, _u8p), _p(b, _i8p), _p(c, _i32p), M, N, K, self.threads)
        return c

    def epilogue(self, conv, acc, sx, zx, sw, colsum, bias=None, y=None, accumulate=False):
        acc = np.ascontiguousarray(acc, np.int32)
        M, N = acc.shape
        if y is None:
            y = np.zeros((M, N), np.float32)
        else:
            y = np.array(y, np.float32, copy=True)
        self.lib.orc_epilogue(conv, _p(acc, _i32p), _p(_f32(sx), _f32p),
                              _p(np.ascontiguousarray(zx, np.int32), _i32p), _p(_f32(sw), _f32p),
                              _p(np.ascontiguousarray(colsum, np.int32), _i32p),
                              _p(None if bias is None else _f32(bias), _f32p), _p(y, _f32p), M, N,
                              int(bool(accumulate)))
        return y

    def linear(self, conv, q, sx, zx, wq, sw, colsum, bias=None, y=None, accumulate=False):
        """ops.c:450-491: returns (y, work)."""
        work = self.gemm(q, wq)
        return self.epilogue(conv, work, sx, zx, sw, colsum, bias, y, accumulate), work

    def selfcheck_kat(self):
        a = np.empty(3 * 64, np.uint8)
        b = np.empty(5 * 64, np.int8)
        want = np.empty(15, np.int32)
        self.lib.orc_selfcheck_kat(_p(a, _u8p), _p(b, _i8p), _p(want, _i32p))
        return a.reshape(3, 64), b.reshape(5, 64), want.reshape(3, 5)

    def silu_mul(self, a, g):
        a = np.array(a, np.float32, copy=True)
        g = _f32(g)
        self.lib.orc_silu_mul(_p(a, _f32p), _p(g, _f32p), a.size)
        return a

    def euler_update(self, conv, state, velocity, use_cfg, rows, scales, dt):
        """sampler.c:281-297: returns the next state; velocity [batch, n],
        rows = (text_row, speaker_row, caption_row) with -1 for absent."""
        st = np.array(state, np.float32, copy=True).reshape(-1)
        vel = _f32(velocity)
        self.lib.orc_euler_update(conv, _p(st, _f32p), _p(vel, _f32p), st.size, int(use_cfg),
                                  *[int(r) for r in rows], *[float(x) for x in scales], float(dt))
        return st

    def expf_mismatches(self):
        return self.lib.orc_expf_mismatches(self.threads)

    def expf_digest(self):
        return int(self.lib.orc_expf_digest(self.threads))

    def fp32_digests(self):
        d, r = C.c_ulonglong(0), C.c_ulonglong(0)
        self.lib.orc_fp32_digests(self.threads, C.byref(d), C.byref(r))
        return int(d.value), int(r.value)

    def adaln_apply(self, x, shift, scale, B, S, eps):
        x, shift, scale = _f32(x), _f32(shift), _f32(scale)
        D = x.shape[-1]
        h = np.empty_like(x)
        self.lib.orc_adaln_apply(_p(x, _f32p), _p(shift, _f32p), _p(scale, _f32p), B, S, D,
                                 eps, _p(h, _f32p))
        return h

    def linear_f32(self, x, w, bias=None):
        """ops.c:221-234: x [M, K] @ w [N, K]^T in K order, + bias (or + 0)."""
        x, w = _f32(x), _f32(w)
        M, K = x.shape
        N = w.shape[0]
        y = np.empty((M, N), np.float32)
        self.lib.orc_linear_f32(_p(x, _f32p), M, K, _p(w, _f32p), N,
                                None if bias is None else _p(_f32(bias), _f32p), _p(y, _f32p))
        return y

    def rmsnorm(self, x, w, eps):
        """ops.c:738-747."""
        x = _f32(x)
        y = np.empty_like(x)
        self.lib.orc_rmsnorm(_p(x, _f32p), x.shape[0], x.shape[1], _p(_f32(w), _f32p), eps,
                             _p(y, _f32p))
        return y

    def tanhf_mismatches(self):
        """Inputs (of all 2^32) where the fdlibm tanhf restatement differs from libm."""
        return self.lib.orc_tanhf_mismatches(self.threads)

    def tanhf_digest(self):
        """The device self-check's hash of tanhf over all 2^32 inputs."""
        return int(self.lib.orc_tanhf_digest(self.threads))

    def adaln_params(self, cond, down, up, bias):
        """dit.c:543-588 for one adaLN: [3, B, D] (shift, scale, tanhf gate) from
        cond [B, 3D] and three (down [R, D], up [D, R], bias [D]) branches."""
        cond = _f32(cond)
        B, D = cond.shape[0], cond.shape[1] // 3
        R = down[0].shape[0]
        ds, us, bs = [_f32(a) for a in down], [_f32(a) for a in up], [_f32(a) for a in bias]
        out = np.empty((3, B, D), np.float32)
        arr = lambda xs: (_f32p * 3)(*[_p(a, _f32p) for a in xs])
        self.lib.orc_adaln_params(_p(cond, _f32p), B, D, R, arr(ds), arr(us), arr(bs),
                                  _p(out, _f32p))
        return out

    def rope_table(self, S):
        """(cos, sin) [S, 32] of head_rmsnorm_rope_pair (dit.c:641-657, 697-703)."""
        c = np.empty((S, 32), np.float32)
        s = np.empty((S, 32), np.float32)
        self.lib.orc_rope_table(S, _p(c, _f32p), _p(s, _f32p))
        return c, s

    def head_norm_rope(self, q, qw, k, kw, B, S, eps, rope=True):
        """dit.c:638-706 (rope) or dit.c:619-636 (no rope, k may be None) on
        copies of q, k [B*S, heads*64]; returns (q, k)."""
        q = np.array(q, np.float32, copy=True)
        heads = q.shape[-1] // 64
        kk = None if k is None else np.array(k, np.float32, copy=True)
        rc = self.lib.orc_head_norm_rope(_p(q, _f32p), _p(_f32(qw), _f32p),
                                         None if kk is None else _p(kk, _f32p),
                                         None if kw is None else _p(_f32(kw), _f32p),
                                         B, S, heads, eps, 1 if rope else 0)
        assert rc == 0
        return q, kk

    def attention_core(self, q, k, v, gate, B, S, ck, cv, mask, context_batch):
        """dit.c:808-870 (scalar ops): mix [B*S, D] from q, k, v, gate [B*S, D],
        context rows ck, cv [(1 or B) * C, D] and mask [B, C]."""
        q, k, v, gate, ck, cv = (_f32(a) for a in (q, k, v, gate, ck, cv))
        mask = np.ascontiguousarray(mask, np.uint8)
        D = q.shape[-1]
        C = mask.shape[-1]
        mix = np.empty_like(q)
        rc = self.lib.orc_attention_core(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p),
                                         _p(gate, _f32p), B, S, D, _p(ck, _f32p), _p(cv, _f32p),
                                         _p(mask, _u8p), C, context_batch, _p(mix, _f32p),
                                         self.threads)
        assert rc == 0
        return mix

    def gated_residual(self, conv, x, gate, branch, B, S):
        x = np.array(x, np.float32, copy=True)
        D = x.shape[-1]
        self.lib.orc_gated_residual(conv, _p(x, _f32p), _p(_f32(gate), _f32p),
                                    _p(_f32(branch), _f32p), B, S, D)
        return x

    def conv_out_len(self, T, kernel, stride, dilation, padding):
        return self.lib.orc_conv1d_output_length(T, kernel, stride, dilation, padding)

    def conv1d(self, conv, x, wq, sw, colsum, kernel, stride, dilation, padding, bias=None,
               residual=False, want_cols=False):
        x = _f32(x)
        T, Cin = x.shape
        N = wq.shape[0]
        To = self.conv_out_len(T, kernel, stride, dilation, padding)
        assert To > 0
        y = np.empty((To, N), np.float32)
        cols = np.empty((To, kernel * Cin), np.uint8) if want_cols else None
        s = np.empty(To, np.float32)
        z = np.empty(To, np.int32)
        rc = self.lib.orc_conv1d_int8(conv, _p(x, _f32p), T, Cin,
                                      _p(np.ascontiguousarray(wq, np.int8), _i8p),
                                      _p(_f32(sw), _f32p),
                                      _p(np.ascontiguousarray(colsum, np.int32), _i32p), N, kernel,
                                      stride, dilation, padding,
                                      _p(None if bias is None else _f32(bias), _f32p),
                                      int(bool(residual)), _p(y, _f32p), _p(cols, _u8p),
                                      _p(s, _f32p), _p(z, _i32p), self.threads)
        assert rc == To
        return y, cols, s, z

    def conv1x1_skip(self, conv, hidden, skip, wq, sw, colsum, bias=None, residual=False):
        """dacvae.c:974-1012: skip + lin(q1) + bias (+ lin(q2)); wq [C_out, C_in]."""
        hidden = _f32(hidden)
        T, Cin = hidden.shape
        Cout = wq.shape[0]
        out = np.empty((T, Cout), np.float32)
        rc = self.lib.orc_conv1x1_skip_int8(
            conv, _p(hidden, _f32p), _p(_f32(skip), _f32p), T,
            _p(np.ascontiguousarray(wq, np.int8), _i8p), _p(_f32(sw), _f32p),
            _p(np.ascontiguousarray(colsum, np.int32), _i32p), Cout, Cin,
            _p(None if bias is None else _f32(bias), _f32p), int(bool(residual)), _p(out, _f32p),
            self.threads)
        assert rc == 0
        return out

    def convt_out_len(self, T_in, kernel, stride, padding, output_padding):
        return self.lib.orc_convtranspose1d_output_length(T_in, kernel, stride, padding,
                                                          output_padding)

    def convtranspose1d(self, conv, x, wq, sw, colsum, C_out, kernel, stride, padding,
                        output_padding, bias=None, residual=False):
        """dacvae.c:696-795 without snake; wq [kernel*C_out, C_in]."""
        x = _f32(x)
        T_in, Cin = x.shape
        To = self.convt_out_len(T_in, kernel, stride, padding, output_padding)
        assert To > 0
        y = np.empty((To, C_out), np.float32)
        rc = self.lib.orc_convtranspose1d_int8(
            conv, _p(x, _f32p), T_in, Cin, _p(np.ascontiguousarray(wq, np.int8), _i8p),
            _p(_f32(sw), _f32p), _p(np.ascontiguousarray(colsum, np.int32), _i32p), C_out, kernel,
            stride, padding, output_padding, _p(None if bias is None else _f32(bias), _f32p),
            int(bool(residual)), _p(y, _f32p), self.threads)
        assert rc == To
        return y


    def dit_condition(self, w0, w1, w2, t):
        """iro_dit_condition (dit.c:488-530) composed from the restated pieces:
        the timestep embedding with the restated expf, cosf and sinf in the
        reference's op order, then linear / SiLU / linear / SiLU / linear
        (the scalar linear, no biases)."""
        L = self.lib
        w0, w1, w2 = _f32(w0), _f32(w1), _f32(w2)
        t = _f32(t).reshape(-1)
        B, tdim = t.shape[0], w0.shape[1]
        half = tdim // 2
        log_theta = np.float32(float.fromhex("0x1.26bb1cp+3"))  # logf(10000.0f)
        emb = np.empty((B, tdim), np.float32)
        for i in range(half):
            e = (np.float32(-log_theta) * np.float32(i)) / np.float32(half)
            freq = np.float32(1000.0) * np.float32(L.orc_expf_restated(float(e)))
            for b in range(B):
                arg = np.float32(t[b] * freq)
                emb[b, i] = L.orc_cosf(float(arg))
                emb[b, half + i] = L.orc_sinf(float(arg))
        ones = np.ones(1, np.float32)
        h0 = self.linear_f32(emb, w0)
        h0 = self.silu_mul(h0, np.broadcast_to(ones, h0.shape))
        h1 = self.linear_f32(h0, w1)
        h1 = self.silu_mul(h1, np.broadcast_to(ones, h1.shape))
        return self.linear_f32(h1, w2)

    def sincosf_mismatches(self, which):
        """Inputs (of all 2^32) where the restated sinf (0) / cosf (1) differs from libm."""
        return self.lib.orc_sincosf_mismatches(which, self.threads)

    def sincosf_digest(self, which):
        """The device self-check's hash of sinf (0) / cosf (1) over all 2^32 inputs."""
        return int(self.lib.orc_sincosf_digest(which, self.threads))

    def snake(self, conv, x, alpha, bias=None, inv_form=None):
        """dacvae.c:830-931 on [T, C]; inv_form defaults to iro_snake_forward's
        choice (C <= 1536).  With bias it is snake_bias_forward, whose
        reciprocal form needs in-place (pass inv_form=True for that case)."""
        x = _f32(x)
        T, Cc = x.shape
        if inv_form is None:
            inv_form = Cc <= 1536 and bias is None
        y = np.empty_like(x)
        self.lib.orc_snake(conv, _p(x, _f32p), T, Cc, _p(None if bias is None else _f32(bias),
                                                          _f32p),
                           _p(_f32(alpha), _f32p), int(bool(inv_form)), _p(y, _f32p))
        return y

    def residual_unit(self, conv, x, u, two7, two1):
        """run_residual_int8 (dacvae.c:934-1018) composed from the restated
        pieces: u = dict(alpha0, w0 [C,7,C], b0, alpha1, w1 [C,1,C], b1, dil)."""
        x = _f32(x)
        T, Cc = x.shape
        q0, s0, c0 = self.weight_quantize(conv, np.asarray(u["w0"]).reshape(Cc, 7 * Cc))
        q1, s1, c1 = self.weight_quantize(conv, np.asarray(u["w1"]).reshape(Cc, Cc))
        act = self.snake(conv, x, u["alpha0"])
        d = u["dil"]
        hidden, _, _, _ = self.conv1d(conv, act, q0, s0, c0, 7, 1, d, 3 * d, None, two7)
        hidden = self.snake(conv, hidden, u["alpha1"], bias=u["b0"], inv_form=Cc <= 1536)
        return self.conv1x1_skip(conv, hidden, x, q1, s1, c1, u["b1"], two1)

    def decode_core(self, conv, state, p, residual_mask=12, residual_stages=8):
        """The int8 core of iro_dacvae_decode (dacvae.c:1221-1277) composed
        from the restated pieces; p = dict(initial_w [1536,7,1024], initial_b,
        stages=[dict(alpha, up_w [c_in,k,c_out], up_b, c_out, kernel, stride,
        padding, output_padding, residual=[u, u, u])])."""
        state = _f32(state)
        lat = state.shape[1]
        iw = np.asarray(p["initial_w"])
        q, s_, c_ = self.weight_quantize(conv, iw.reshape(iw.shape[0], 7 * lat))
        x, _, _, _ = self.conv1d(conv, state, q, s_, c_, 7, 1, 1, 3, p["initial_b"],
                                 bool(residual_mask & 1))
        for si, st in enumerate(p["stages"]):
            c_in = x.shape[1]
            k, c_out = st["kernel"], st["c_out"]
            uq, us, uc = self.weight_quantize_transposed(conv, np.asarray(st["up_w"]).reshape(
                c_in, k * c_out), k * c_out, c_in)
            act = self.snake(conv, x, st["alpha"])
            x = self.convtranspose1d(conv, act, uq, us, uc, c_out, k, st["stride"], st["padding"],
                                     st["output_padding"], st["up_b"], bool(residual_mask & 2))
            on = bool(residual_stages >> si & 1)
            for u in st["residual"]:
                x = self.residual_unit(conv, x, u, bool(residual_mask & 4) and on,
                                       bool(residual_mask & 8) and on)
        return x


class _Weight(C.Structure):
    # ops.h:23-28 IroInt8Weight
    _fields_ = [("data", _i8p), ("scale", _f32p), ("colsum", _i32p), ("N", C.c_int),
                ("K", C.c_int)]


class Reference:
    """The reference's own ops.c/dacvae.c built from source (oracle/_ref)."""

    def __init__(self, flavour: str):
        path = os.path.join(HERE, "_ref", f"libref_{flavour}.so")
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = L = C.CDLL(path)
        L.iro_int8_weight_quantize.argtypes = [C.POINTER(_Weight), _f32p, C.c_int, C.c_int]
        L.iro_int8_weight_quantize.restype = C.c_int
        L.iro_int8_weight_quantize_transposed.argtypes = L.iro_int8_weight_quantize.argtypes
        L.iro_int8_weight_quantize_transposed.restype = C.c_int
        L.iro_int8_weight_free.argtypes = [C.POINTER(_Weight)]
        L.iro_int8_quantize_rows.argtypes = [_f32p, C.c_int, C.c_int, _u8p, _f32p, _i32p]
        L.iro_int8_quantize_rows_residual.argtypes = [_f32p, C.c_int, C.c_int, _u8p, _f32p, _i32p,
                                                      _f32p, _u8p, _f32p, _i32p]
        L.iro_int8_linear_ex.argtypes = [_u8p, _f32p, _i32p, C.POINTER(_Weight), _f32p, _f32p,
                                         C.c_int, _i32p, C.c_int]
        L.iro_int8_selfcheck.restype = C.c_int
        L.iro_silu_mul_inplace.argtypes = [_f32p, _f32p, C.c_size_t]
        L.ref_conv1d_int8.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_int, _i8p, _f32p, _i32p, _f32p, C.c_int, _f32p]
        L.ref_conv1d_int8.restype = C.c_int
        L.ref_convtranspose1d_int8.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                               C.c_int, C.c_int, _i8p, _f32p, _i32p, _f32p, _f32p]
        L.ref_convtranspose1d_int8.restype = C.c_int
        L.ref_dit_adaln_zero_rank.argtypes = [C.c_float, _f32p, _f32p, _f32p, _f32p, _f32p,
                                               C.c_int, C.c_int, _f32p, _f32p,
                                               C.POINTER(C.c_int)]
        L.ref_dit_adaln_zero_rank.restype = C.c_int
        L.ref_head_rmsnorm_rope_pair.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int,
                                                 C.c_float, C.POINTER(C.c_int),
                                                 C.POINTER(C.c_int)]
        L.ref_head_rmsnorm.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_float]
        L.ref_dit_attention_identity.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _u8p,
                                                 C.c_int, C.c_int, C.c_int, C.c_int, C.c_float,
                                                 _f32p]
        L.ref_dit_attention_identity.restype = C.c_int
        L.ref_snake.argtypes = [_f32p, _f32p, C.c_int, C.c_int, _f32p]
        L.ref_snake_bias.argtypes = [_f32p, _f32p, C.c_int, C.c_int, _f32p, _f32p]
        L.ref_dacvae_residual_int8.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _f32p, _f32p,
                                               _f32p, _f32p, _f32p, C.c_int, C.c_int, _f32p]
        L.ref_dacvae_residual_int8.restype = C.c_int
        L.ref_dacvae_decode_trace.argtypes = [C.POINTER(_f32p), _f32p, C.c_int, _f32p, _f32p,
                                              _f32p]
        L.ref_dacvae_decode_trace.restype = C.c_int

    def dit_block(self, x, cond, ada, w, ck, cv, mask, B, S, eps, use_int8=True):
        """iro_dit_block (dit.c:1042-1047) of one layer: ada = 18 adaLN arrays
        (attention then MLP, dit.h order), w = (wq, wk, wv, wgate, wo, q_norm,
        k_norm, w1, w3, w2); returns the updated x."""
        x = np.array(x, np.float32, copy=True)
        mask = np.ascontiguousarray(mask, np.uint8)
        dims = (C.c_int * 3)()
        ws = [_f32(a) for a in w]
        adas = [_f32(a) for a in ada]
        self.lib.ref_dit_block.argtypes = ([_f32p, _f32p, C.POINTER(_f32p)] + [_f32p] * 12 +
                                           [_u8p] + [C.c_int] * 3 +
                                           [C.c_float, C.c_int, C.POINTER(C.c_int)])
        self.lib.ref_dit_block.restype = C.c_int
        rc = self.lib.ref_dit_block(
            _p(x, _f32p), _p(_f32(cond), _f32p), (_f32p * 18)(*[_p(a, _f32p) for a in adas]),
            *[_p(a, _f32p) for a in ws], _p(_f32(ck), _f32p), _p(_f32(cv), _f32p),
            _p(mask, _u8p), B, S, mask.shape[-1], eps, int(bool(use_int8)), dims)
        assert rc == 0 and dims[0] == x.shape[-1], (rc, dims[0])
        return x

    def dit_attn_parts(self, x, cond, ada, w, ck, cv, mask, B, S, eps, use_int8=True):
        """The operands of the attention half's gated residual inside
        iro_dit_block (dit.c:1004-1020), computed by the functions dit_block
        calls on the same layer: returns (gate [B, D], branch [B*S, D])."""
        mask = np.ascontiguousarray(mask, np.uint8)
        x = _f32(x)
        D = x.shape[-1]
        gate = np.empty((B, D), np.float32)
        branch = np.empty((B * S, D), np.float32)
        ws = [_f32(a) for a in w]
        adas = [_f32(a) for a in ada]
        self.lib.ref_dit_attn_parts.argtypes = ([_f32p, _f32p, C.POINTER(_f32p)] + [_f32p] * 12 +
                                                [_u8p] + [C.c_int] * 3 +
                                                [C.c_float, C.c_int, _f32p, _f32p])
        self.lib.ref_dit_attn_parts.restype = C.c_int
        rc = self.lib.ref_dit_attn_parts(
            _p(x, _f32p), _p(_f32(cond), _f32p), (_f32p * 18)(*[_p(a, _f32p) for a in adas]),
            *[_p(a, _f32p) for a in ws], _p(_f32(ck), _f32p), _p(_f32(cv), _f32p),
            _p(mask, _u8p), B, S, mask.shape[-1], eps, int(bool(use_int8)), _p(gate, _f32p),
            _p(branch, _f32p))
        assert rc == 0, rc
        return gate, branch

    def linear_f32(self, x, w, bias=None):
        """The scalar build's iro_linear (ops.c:236-254)."""
        x, w = _f32(x), _f32(w)
        M, K = x.shape
        N = w.shape[0]
        y = np.empty((M, N), np.float32)
        self.lib.iro_linear.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int]
        self.lib.iro_linear(_p(x, _f32p), _p(w, _f32p),
                            None if bias is None else _p(_f32(bias), _f32p), _p(y, _f32p), M, K, N)
        return y

    def rmsnorm(self, x, w, eps):
        """The scalar build's iro_rmsnorm (ops.c:738-747)."""
        x = _f32(x)
        y = np.empty_like(x)
        self.lib.iro_rmsnorm.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_float]
        self.lib.iro_rmsnorm(_p(x, _f32p), _p(_f32(w), _f32p), _p(y, _f32p), x.shape[0],
                             x.shape[1], eps)
        return y

    def dit_step(self, x, cond, head, ada, blk, ck, cv, mask, B, S, eps):
        """The sampler's DiT evaluation (sampler.c:259-278): input projection
        of x [S, 32], broadcast to B rows, len(ada) // 18 shared-context
        blocks, output head; returns velocity [B*S, 32]."""
        mask = np.ascontiguousarray(mask, np.uint8)
        heads_ = [_f32(a) for a in head]
        adas = [_f32(a) for a in ada]
        blks = [_f32(a) for a in blk]
        layers = len(adas) // 18
        vel = np.empty((B * S, 32), np.float32)
        self.lib.ref_dit_step.argtypes = [_f32p, _f32p, C.POINTER(_f32p), C.POINTER(_f32p),
                                          C.POINTER(_f32p), C.c_int, _f32p, _f32p, _u8p,
                                          C.c_int, C.c_int, C.c_int, C.c_float, _f32p]
        self.lib.ref_dit_step.restype = C.c_int
        rc = self.lib.ref_dit_step(
            _p(_f32(x), _f32p), _p(_f32(cond), _f32p), (_f32p * 5)(*[_p(a, _f32p) for a in heads_]),
            (_f32p * len(adas))(*[_p(a, _f32p) for a in adas]),
            (_f32p * len(blks))(*[_p(a, _f32p) for a in blks]), layers, _p(_f32(ck), _f32p),
            _p(_f32(cv), _f32p), _p(mask, _u8p), B, S, mask.shape[-1], eps, _p(vel, _f32p))
        assert rc == 0
        return vel

    def sample_euler(self, pool, eps, text, text_mask, speaker, caption, noise, cfg):
        """The reference's whole Euler sampler (sampler.c:101-324) on a DiT
        whose every weight aliases `pool` (at least 3*1280*1280 floats),
        with a trace of every step.  cfg = (steps, init_scale, cfg_scale_text,
        cfg_scale_speaker, cfg_scale_caption, cfg_min_t, cfg_max_t).  Returns
        (output [S*32], x_t [steps, 4, S*32], velocity [steps, 4, S*32],
        batch [steps], timestep [steps]); row 0 of x_t[s] is the state that
        enters step s."""
        noise = _f32(noise)
        S = noise.shape[0]
        steps = int(cfg[0])
        n = S * 32
        cfgv = np.asarray(cfg, np.float32)
        out = np.zeros(n, np.float32)
        xt = np.zeros((steps, 4, n), np.float32)
        vel = np.zeros((steps, 4, n), np.float32)
        bt = np.zeros(steps, np.int32)
        ts = np.zeros(steps, np.float32)
        L = self.lib
        L.ref_sample_euler.argtypes = [_f32p, C.c_float, _f32p, _u8p, C.c_int, _f32p, C.c_int,
                                       _f32p, C.c_int, _f32p, C.c_int, _f32p, _f32p, _f32p,
                                       _f32p, _i32p, _f32p]
        L.ref_sample_euler.restype = C.c_int
        pool = _f32(pool)
        assert pool.size >= 3 * 1280 * 1280
        text, caption_ = _f32(text), None if caption is None else _f32(caption)
        speaker_ = None if speaker is None else _f32(speaker)
        rc = L.ref_sample_euler(
            _p(pool, _f32p), eps, _p(text, _f32p), _p(np.ascontiguousarray(text_mask, np.uint8), _u8p),
            text.shape[0], _p(speaker_, _f32p), 0 if speaker_ is None else speaker_.shape[0],
            _p(caption_, _f32p), 0 if caption_ is None else caption_.shape[0], _p(noise, _f32p),
            S, _p(cfgv, _f32p), _p(out, _f32p), _p(xt, _f32p), _p(vel, _f32p), _p(bt, _i32p),
            _p(ts, _f32p))
        assert rc == 0, "ref_sample_euler failed"
        return out, xt, vel, bt, ts

    def dit_context_kv(self, kind, x, wk, wv, k_norm, B, T, eps):
        """iro_dit_text_kv (kind 0) / iro_dit_speaker_kv (kind 1), dit.c:708-726:
        (k, v) [B*T, MODEL_DIM]."""
        x = _f32(x)
        D = wk.shape[0]
        k = np.empty((B * T, D), np.float32)
        v = np.empty((B * T, D), np.float32)
        dim = C.c_int(0)
        self.lib.ref_dit_context_kv.argtypes = [C.c_int, _f32p, _f32p, _f32p, _f32p, C.c_int,
                                                C.c_int, C.c_float, _f32p, _f32p,
                                                C.POINTER(C.c_int)]
        self.lib.ref_dit_context_kv.restype = C.c_int
        rc = self.lib.ref_dit_context_kv(kind, _p(x, _f32p), _p(_f32(wk), _f32p),
                                         _p(_f32(wv), _f32p), _p(_f32(k_norm), _f32p), B, T, eps,
                                         _p(k, _f32p), _p(v, _f32p), C.byref(dim))
        assert rc == 0 and dim.value == x.shape[-1], (rc, dim.value)
        return k, v

    def dit_adaln_full(self, eps, x, cond, w, B, S):
        """iro_dit_adaln (dit.c:614) with low-rank weights w (9 arrays, dit.h
        order): (h [B*S, D], gate [B, D])."""
        x, cond = _f32(x), _f32(cond)
        ws = [_f32(a) for a in w]
        h = np.empty_like(x)
        gate = np.empty((B, x.shape[-1]), np.float32)
        self.lib.ref_dit_adaln_full.argtypes = [C.c_float, _f32p, _f32p, C.POINTER(_f32p),
                                                C.c_int, C.c_int, _f32p, _f32p]
        self.lib.ref_dit_adaln_full.restype = C.c_int
        rc = self.lib.ref_dit_adaln_full(eps, _p(x, _f32p), _p(cond, _f32p),
                                         (_f32p * 9)(*[_p(a, _f32p) for a in ws]), B, S,
                                         _p(h, _f32p), _p(gate, _f32p))
        assert rc == 0
        return h, gate

    def dit_attention_identity(self, x, q_norm, k_norm, ck, cv, mask, B, S, shared, eps):
        """iro_dit_attention(_shared_context) (dit.c:895-911) with identity
        projections: the attention core on (normed x, normed x, x, gate x)."""
        x = _f32(x)
        mask = np.ascontiguousarray(mask, np.uint8)
        out = np.empty_like(x)
        rc = self.lib.ref_dit_attention_identity(_p(x, _f32p), _p(_f32(q_norm), _f32p),
                                                 _p(_f32(k_norm), _f32p), _p(_f32(ck), _f32p),
                                                 _p(_f32(cv), _f32p), _p(mask, _u8p), B, S,
                                                 mask.shape[-1], int(bool(shared)), eps,
                                                 _p(out, _f32p))
        assert rc == 0
        return out

    def head_rmsnorm_rope_pair(self, q, qw, k, kw, B, S, eps):
        """dit.c:638-706 on copies of q, k [B*S, MODEL_DIM]: (q, k, heads)."""
        q, k = np.array(q, np.float32, copy=True), np.array(k, np.float32, copy=True)
        dim, heads = C.c_int(0), C.c_int(0)
        self.lib.ref_head_rmsnorm_rope_pair(_p(q, _f32p), _p(_f32(qw), _f32p), _p(k, _f32p),
                                            _p(_f32(kw), _f32p), B, S, eps, C.byref(dim),
                                            C.byref(heads))
        assert dim.value == q.shape[-1], (dim.value, q.shape)
        return q, k, heads.value

    def head_rmsnorm(self, x, w, B, S, eps):
        """dit.c:619-636 on a copy of x [B*S, MODEL_DIM]."""
        x = np.array(x, np.float32, copy=True)
        self.lib.ref_head_rmsnorm(_p(x, _f32p), _p(_f32(w), _f32p), B, S, eps)
        return x

    def dit_adaln_zero_rank(self, eps, x, cond, shift_bias, scale_bias, gate_bias, B, S):
        """iro_dit_adaln (dit.c:614) with zero low-rank linears: (h, gate, D)."""
        x, cond = _f32(x), _f32(cond)
        D = x.shape[-1]
        h = np.empty_like(x)
        gate = np.empty((B, D), np.float32)
        dim = C.c_int(0)
        rc = self.lib.ref_dit_adaln_zero_rank(eps, _p(x, _f32p), _p(cond, _f32p),
                                              _p(_f32(shift_bias), _f32p),
                                              _p(_f32(scale_bias), _f32p),
                                              _p(_f32(gate_bias), _f32p), B, S, _p(h, _f32p),
                                              _p(gate, _f32p), C.byref(dim))
        assert rc == 0 and dim.value == D, (rc, dim.value, D)
        return h, gate

    def weight_quantize(self, w, transposed_shape=None):
        w = _f32(w)
        wt = _Weight()
        if transposed_shape is None:
            N, K = w.shape
            rc = self.lib.iro_int8_weight_quantize(C.byref(wt), _p(w, _f32p), N, K)
        else:
            N, K = transposed_shape
            rc = self.lib.iro_int8_weight_quantize_transposed(C.byref(wt), _p(w, _f32p), N, K)
        assert rc == 0
        q = np.ctypeslib.as_array(wt.data, (N * K,)).reshape(N, K).copy()
        s = np.ctypeslib.as_array(wt.scale, (N,)).copy()
        cs = np.ctypeslib.as_array(wt.colsum, (N,)).copy()
        self.lib.iro_int8_weight_free(C.byref(wt))
        return q, s, cs

    def quantize_rows(self, x):
        x = _f32(x)
        M, K = x.shape
        q = np.empty((M, K), np.uint8)
        s = np.empty(M, np.float32)
        z = np.empty(M, np.int32)
        self.lib.iro_int8_quantize_rows(_p(x, _f32p), M, K, _p(q, _u8p), _p(s, _f32p),
                                        _p(z, _i32p))
        return q, s, z

    def quantize_rows_residual(self, x):
        x = _f32(x)
        M, K = x.shape
        q1 = np.empty((M, K), np.uint8)
        q2 = np.empty((M, K), np.uint8)
        r = np.empty((M, K), np.float32)
        s1, s2 = np.empty(M, np.float32), np.empty(M, np.float32)
        z1, z2 = np.empty(M, np.int32), np.empty(M, np.int32)
        self.lib.iro_int8_quantize_rows_residual(_p(x, _f32p), M, K, _p(q1, _u8p), _p(s1, _f32p),
                                                 _p(z1, _i32p), _p(r, _f32p), _p(q2, _u8p),
                                                 _p(s2, _f32p), _p(z2, _i32p))
        return (q1, s1, z1), r, (q2, s2, z2)

    def linear(self, q, sx, zx, wq, sw, colsum, bias=None, y=None, accumulate=False):
        q = np.ascontiguousarray(q, np.uint8)
        M, K = q.shape
        N = wq.shape[0]
        wq = np.ascontiguousarray(wq, np.int8)
        sw = _f32(sw)
        colsum = np.ascontiguousarray(colsum, np.int32)
        wt = _Weight(_p(wq, _i8p), _p(sw, _f32p), _p(colsum, _i32p), N, K)
        y = np.zeros((M, N), np.float32) if y is None else np.array(y, np.float32, copy=True)
        work = np.empty((M, N), np.int32)
        self.lib.iro_int8_linear_ex(_p(q, _u8p), _p(_f32(sx), _f32p),
                                    _p(np.ascontiguousarray(zx, np.int32), _i32p), C.byref(wt),
                                    _p(None if bias is None else _f32(bias), _f32p), _p(y, _f32p),
                                    M, _p(work, _i32p), int(bool(accumulate)))
        return y, work

    def selfcheck(self):
        return self.lib.iro_int8_selfcheck()

    def silu_mul(self, a, g):
        a = np.array(a, np.float32, copy=True)
        self.lib.iro_silu_mul_inplace(_p(a, _f32p), _p(_f32(g), _f32p), a.size)
        return a

    def conv1d(self, x, wq, sw, colsum, kernel, stride, dilation, padding, bias=None,
               residual=False, out_len=None):
        x = _f32(x)
        T, Cin = x.shape
        N = wq.shape[0]
        y = np.empty((out_len, N), np.float32)
        rc = self.lib.ref_conv1d_int8(_p(x, _f32p), T, Cin, N, kernel, stride, dilation, padding,
                                      _p(np.ascontiguousarray(wq, np.int8), _i8p),
                                      _p(_f32(sw), _f32p),
                                      _p(np.ascontiguousarray(colsum, np.int32), _i32p),
                                      _p(None if bias is None else _f32(bias), _f32p),
                                      int(bool(residual)), _p(y, _f32p))
        assert rc == 0
        return y

    def convtranspose1d(self, x, wq, sw, colsum, C_out, kernel, stride, padding, output_padding,
                        bias, out_len):
        """The reference's convtranspose1d_forward_impl (int8, no snake); its
        two-term choice follows IRO_CODEC_INT8_RESIDUAL, read once per process."""
        x = _f32(x)
        T_in, Cin = x.shape
        y = np.empty((out_len, C_out), np.float32)
        rc = self.lib.ref_convtranspose1d_int8(
            _p(x, _f32p), T_in, Cin, C_out, kernel, stride, padding, output_padding,
            _p(np.ascontiguousarray(wq, np.int8), _i8p), _p(_f32(sw), _f32p),
            _p(np.ascontiguousarray(colsum, np.int32), _i32p), _p(_f32(bias), _f32p), _p(y, _f32p))
        assert rc == 0
        return y


    def dit_condition(self, w0, w1, w2, t):
        """iro_dit_condition (dit.c:501-530) of this build."""
        t = _f32(t).reshape(-1)
        dims = (C.c_int * 3)()
        self.lib.ref_dit_condition.argtypes = [_f32p, _f32p, _f32p, _f32p, C.c_int, _f32p,
                                               C.POINTER(C.c_int)]
        self.lib.ref_dit_condition.restype = C.c_int
        cond = np.empty((t.shape[0], np.asarray(w2).shape[0]), np.float32)
        rc = self.lib.ref_dit_condition(_p(_f32(w0), _f32p), _p(_f32(w1), _f32p),
                                        _p(_f32(w2), _f32p), _p(t, _f32p), t.shape[0],
                                        _p(cond, _f32p), dims)
        assert rc == 0 and dims[2] == cond.shape[1], (rc, list(dims))
        return cond

    def snake(self, x, alpha, inplace=False):
        """iro_snake_forward (dacvae.c:830-857), out of place or in place."""
        x = np.array(x, np.float32, copy=True, order="C")
        y = x if inplace else np.empty_like(x)
        self.lib.ref_snake(_p(x, _f32p), _p(y, _f32p), x.shape[0], x.shape[1],
                           _p(_f32(alpha), _f32p))
        return y

    def snake_bias(self, x, bias, alpha, inplace=True):
        """snake_bias_forward (dacvae.c:910-931)."""
        x = np.array(x, np.float32, copy=True, order="C")
        y = x if inplace else np.empty_like(x)
        self.lib.ref_snake_bias(_p(x, _f32p), _p(y, _f32p), x.shape[0], x.shape[1],
                                _p(_f32(bias), _f32p), _p(_f32(alpha), _f32p))
        return y

    def residual_unit(self, x, u, stage):
        """run_residual_int8 (dacvae.c:934-1018) of a unit in decoder `stage`
        under the default policy (second plane in stage 3 only)."""
        x = _f32(x)
        T, Cc = x.shape
        y = np.empty_like(x)
        rc = self.lib.ref_dacvae_residual_int8(
            _p(x, _f32p), T, Cc, _p(_f32(u["alpha0"]), _f32p), _p(_f32(u["w0"]), _f32p),
            _p(_f32(u["b0"]), _f32p), _p(_f32(u["alpha1"]), _f32p), _p(_f32(u["w1"]), _f32p),
            _p(_f32(u["b1"]), _f32p), u["dil"], stage, _p(y, _f32p))
        assert rc == 0
        return y

    def decode_trace(self, params, latent):
        """iro_dacvae_decode (dacvae.c:1213-1300) with int8 weights: returns the
        quantizer_out state, the state after stage 3 and the waveform.
        params: the 91 fp32 arrays in ref_dacvae_decode_trace's order."""
        keep = [_f32(a) for a in params]
        assert len(keep) == 91
        arr = (_f32p * 91)(*[_p(a, _f32p) for a in keep])
        latent = _f32(latent)
        frames = latent.shape[0]
        state = np.empty((frames, 1024), np.float32)
        core = np.empty((frames * 1920, 96), np.float32)
        wave = np.empty(frames * 1920, np.float32)
        rc = self.lib.ref_dacvae_decode_trace(arr, _p(latent, _f32p), frames, _p(state, _f32p),
                                              _p(core, _f32p), _p(wave, _f32p))
        assert rc == frames * 1920, rc
        return state, core, wave


class _CpubWeight(C.Structure):
    _fields_ = [("q", _i8p), ("s", _f32p), ("cs", _i32p), ("N", C.c_int), ("K", C.c_int)]


class CpuBaseline:
    """libcpubase.so: the reference's oneMKL int8 path as a CPU timing harness
    (bench.py's cpu_baseline leg; also a host-side DiT block for tests)."""

    def __init__(self, threads: int, mkl_path: str | None = None):
        path = os.path.join(HERE, "libcpubase.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        self.lib = L = C.CDLL(path)
        L.cpub_init.argtypes = [C.c_char_p, C.c_int, C.c_char_p, C.c_size_t]
        L.cpub_init.restype = C.c_int
        L.cpub_dit_block.argtypes = [C.c_int, C.POINTER(_CpubWeight), _f32p, _f32p, C.c_int,
                                     C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double)]
        L.cpub_dit_block.restype = C.c_int
        L.cpub_gemm.argtypes = [_u8p, _i8p, _i32p, C.c_int, C.c_int, C.c_int]
        L.cpub_conv1d.argtypes = [C.c_int, _f32p, C.c_int, C.c_int, _i8p, _f32p, _i32p, C.c_int,
                                  C.c_int, C.c_int, C.c_int, C.c_int, _f32p, C.c_int, _f32p,
                                  C.POINTER(C.c_double)]
        L.cpub_conv1d.restype = C.c_int
        buf = C.create_string_buffer(256)
        self.mkl = bool(L.cpub_init((mkl_path or "").encode(), threads, buf, 256))
        self.backend = buf.value.decode()
        self.threads = threads

    def dit_block(self, conv, weights, x, cond, B, S, D, H, residual_mask=8):
        """weights: 9 (q, s, cs) tuples {ada, wq, wk, wv, wgate, wo, w1, w3, w2}.
        Updates x in place; returns seconds (quantize, gemm, epilogue)."""
        arr = (_CpubWeight * 9)()
        keep = []
        for i, (q, s, cs) in enumerate(weights):
            q = np.ascontiguousarray(q, np.int8)
            s = _f32(s)
            cs = np.ascontiguousarray(cs, np.int32)
            keep += [q, s, cs]
            arr[i] = _CpubWeight(_p(q, _i8p), _p(s, _f32p), _p(cs, _i32p), q.shape[0], q.shape[1])
        assert x.dtype == np.float32 and x.flags["C_CONTIGUOUS"]
        t = (C.c_double * 3)()
        rc = self.lib.cpub_dit_block(conv, arr, _p(x, _f32p), _p(_f32(cond), _f32p), B, S, D, H,
                                     residual_mask, t)
        assert rc == 0
        return tuple(t)

    def conv1d(self, conv, x, wq, sw, colsum, kernel, stride, dilation, padding, bias=None,
               residual=False):
        """The reference's int8 Conv1d on the host (oneMKL GEMM); returns
        (y, seconds (quantize, gemm, epilogue))."""
        x = _f32(x)
        T, Cin = x.shape
        N = wq.shape[0]
        To = (T + 2 * padding - dilation * (kernel - 1) - 1) // stride + 1
        y = np.zeros((To, N), np.float32)
        t = (C.c_double * 3)()
        rc = self.lib.cpub_conv1d(conv, _p(x, _f32p), T, Cin,
                                  _p(np.ascontiguousarray(wq, np.int8), _i8p), _p(_f32(sw), _f32p),
                                  _p(np.ascontiguousarray(colsum, np.int32), _i32p), N, kernel,
                                  stride, dilation, padding,
                                  _p(None if bias is None else _f32(bias), _f32p),
                                  int(bool(residual)), _p(y, _f32p), t)
        assert rc == To
        return y, tuple(t)
