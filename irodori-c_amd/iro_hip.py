"""ctypes binding of libiro_hip.so (include/iro_hip.h, include/iro_int8_ops.h).

The host-side mirror of the reference's int8 operator interface for tests,
the smoke check and the benchmark.  Everything runs through the C ABI of the
HIP library; there is no other implementation behind these calls, and
loading fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libiro_hip.so")
INCLUDE_DIR = os.path.join(os.path.dirname(HERE), "include")

STRICT, GCC_FASTMATH = 0, 1

_vp = C.c_void_p
_i = C.c_int


class DiTLayerF32(C.Structure):
    """IroHipDiTLayerF32: per-layer fp32 parameters of a sampler step."""
    _fields_ = [("adaln", _vp * 18), ("q_norm", _vp), ("k_norm", _vp), ("context_k", _vp),
                ("context_v", _vp)]


class DiTHead(C.Structure):
    """IroHipDiTHead: input / output heads, adaLN rank, norm epsilon."""
    _fields_ = [("in_w", _vp), ("in_b", _vp), ("out_norm", _vp), ("out_w", _vp), ("out_b", _vp),
                ("latent", C.c_int), ("rank", C.c_int), ("eps", C.c_float)]
_lib = None


class DACVAEResidualF32(C.Structure):
    # iro_hip.h IroHipDACVAEResidualF32 (dacvae.h:36-41)
    _fields_ = [("alpha0", C.c_void_p), ("conv0_weight", C.c_void_p), ("conv0_bias", C.c_void_p),
                ("alpha1", C.c_void_p), ("conv1_weight", C.c_void_p), ("conv1_bias", C.c_void_p),
                ("dilation", C.c_int)]


class DACVAEStageF32(C.Structure):
    # iro_hip.h IroHipDACVAEStageF32 (dacvae.h:43-47)
    _fields_ = [("alpha", C.c_void_p), ("up_weight", C.c_void_p), ("up_bias", C.c_void_p),
                ("c_in", C.c_int), ("c_out", C.c_int), ("kernel", C.c_int), ("stride", C.c_int),
                ("padding", C.c_int), ("output_padding", C.c_int),
                ("residual", DACVAEResidualF32 * 3)]


class DACVAEDecoderF32(C.Structure):
    # iro_hip.h IroHipDACVAEDecoderF32 (dacvae.h:69-76, the int8-path part)
    _fields_ = [("initial_weight", C.c_void_p), ("initial_bias", C.c_void_p),
                ("latent_channels", C.c_int), ("channels", C.c_int),
                ("stage", DACVAEStageF32 * 4)]


def declared_symbols() -> list[str]:
    """Every function name the C headers in include/ declare."""
    names = []
    for hdr in sorted(os.listdir(INCLUDE_DIR)):
        if not hdr.endswith(".h"):
            continue
        text = open(os.path.join(INCLUDE_DIR, hdr)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(iro_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build() "
                           f"or make -C irodori-c_amd")
    L = C.CDLL(LIB_PATH)
    sig = {
        "iro_hip_create": ([_i, _i, C.POINTER(_vp)], _i),
        "iro_hip_st_open": ([C.c_char_p, C.POINTER(_vp)], _i),
        "iro_hip_st_close": ([_vp], None),
        "iro_hip_st_last_error": ([], C.c_char_p),
        "iro_hip_st_count": ([_vp], _i),
        "iro_hip_st_name": ([_vp, _i], C.c_char_p),
        "iro_hip_st_tensor": ([_vp, C.c_char_p, C.POINTER(_i), C.POINTER(_i),
                               C.POINTER(C.c_uint64), C.POINTER(_vp), C.POINTER(C.c_uint64)], _i),
        "iro_hip_st_meta": ([_vp, C.c_char_p], C.c_char_p),
        "iro_hip_weight_from_st": ([_vp, _vp, C.c_char_p, _i, C.POINTER(_vp)], _i),
        "iro_hip_weight_save": ([_vp, _vp, C.c_char_p], _i),
        "iro_hip_weight_load": ([_vp, C.c_char_p, C.POINTER(_vp)], _i),
        "iro_hip_destroy": ([_vp], None),
        "iro_hip_get_convention": ([_vp], _i),
        "iro_hip_error": ([_vp], C.c_char_p),
        "iro_hip_clear_error": ([_vp], None),
        "iro_hip_sync": ([_vp], _i),
        "iro_hip_stream": ([_vp], _vp),
        "iro_hip_set_gemm_tile": ([_vp, _i, _i], _i),
        "iro_hip_alloc": ([_vp, C.c_size_t, C.POINTER(_vp)], _i),
        "iro_hip_free": ([_vp, _vp], _i),
        "iro_hip_upload": ([_vp, _vp, _vp, C.c_size_t], _i),
        "iro_hip_download": ([_vp, _vp, _vp, C.c_size_t], _i),
        "iro_hip_fill": ([_vp, _vp, _i, C.c_size_t], _i),
        "iro_hip_copy": ([_vp, _vp, _vp, C.c_size_t], _i),
        "iro_hip_event_create": ([C.POINTER(_vp)], _i),
        "iro_hip_event_destroy": ([_vp], None),
        "iro_hip_event_record": ([_vp, _vp], _i),
        "iro_hip_event_elapsed_ms": ([_vp, _vp, C.POINTER(C.c_float)], _i),
        "iro_hip_weight_create": ([_vp, _vp, _i, _i, C.POINTER(_vp)], _i),
        "iro_hip_weight_create_transposed": ([_vp, _vp, _i, _i, C.POINTER(_vp)], _i),
        "iro_hip_weight_create_fused": ([_vp, C.POINTER(_vp), C.POINTER(_i), _i, _i, _i,
                                         C.POINTER(_vp)], _i),
        "iro_hip_weight_from_host": ([_vp, _vp, _vp, _vp, _i, _i, C.POINTER(_vp)], _i),
        "iro_hip_weight_export": ([_vp, _vp, _vp, _vp, _vp], _i),
        "iro_hip_weight_destroy": ([_vp], None),
        "iro_hip_weight_dims": ([_vp, C.POINTER(_i), C.POINTER(_i)], _i),
        "iro_hip_weight_bytes": ([_vp], C.c_size_t),
        "iro_hip_quantize_rows": ([_vp, _vp, _i, _i, _vp, _vp, _vp], _i),
        "iro_hip_quantize_rows_residual": ([_vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                                            _vp], _i),
        "iro_hip_int8_linear_ex": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i], _i),
        "iro_hip_int8_linear_two_term": ([_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                          _i, _i], _i),
        "iro_hip_dit_qkvg": ([_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _i], _i),
        "iro_hip_dit_linear_gated": ([_vp, _vp, _i, _vp, _i, _vp, _vp, _vp, _i], _i),
        "iro_hip_dit_linear_gated_noalloc": ([_vp, _vp, _i, _vp, _i, _vp, _vp, _vp, _i], _i),
        "iro_hip_dit_swiglu": ([_vp, _vp, _i, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _i], _i),
        "iro_hip_conv1d_int8": ([_vp, _vp, _i, _i, _vp, _i, _i, _i, _i, _vp, _i, _vp,
                                 C.POINTER(_i)], _i),
        "iro_hip_convtranspose1d_int8": ([_vp, _vp, _i, _i, _vp, _i, _i, _i, _i, _i, _vp, _i,
                                          _vp, C.POINTER(_i)], _i),
        "iro_hip_conv1x1_skip_int8": ([_vp, _vp, _vp, _i, _vp, _vp, _i, _vp], _i),
        "iro_hip_dit_stack_create": ([_vp, _i, _i, _i, _i, C.POINTER(_vp)], _i),
        "iro_hip_dit_stack_set_block": ([_vp, _i] + [_vp] * 9, _i),
        "iro_hip_dit_stack_step": ([_vp, _vp, _vp, _i, _i], _i),
        "iro_hip_dit_stack_bytes": ([_vp], C.c_size_t),
        "iro_hip_dit_stack_buffers": ([_vp] + [C.POINTER(_vp)] * 6, _i),
        "iro_hip_dit_stack_destroy": ([_vp], None),
        "iro_hip_selfcheck_silu": ([_vp, C.POINTER(C.c_ulonglong), C.POINTER(C.c_ulonglong)], _i),
        "iro_hip_dit_stack_use_graph": ([_vp, _i], _i),
        "iro_hip_dit_stack_use_persistent": ([_vp, _i], _i),
        "iro_hip_dit_stack_set_layer_f32": ([_vp, _i, C.POINTER(DiTLayerF32)], _i),
        "iro_hip_dit_stack_set_head": ([_vp, C.POINTER(DiTHead)], _i),
        "iro_hip_dit_sampler_step": ([_vp, _vp, _vp, _i, _i, _vp, _i, _i, _i, _i, C.c_float,
                                      C.c_float, C.c_float, C.c_float, _vp], _i),
        "iro_hip_dit_stack_block_forward": ([_vp, _i, _vp, _i, _i, _vp, _vp, _vp, _vp, C.c_float,
                                             _vp, _vp, _vp], _i),
        "iro_hip_dit_adaln_apply": ([_vp, _vp, _i, _i, _i, _vp, _vp, C.c_float, _vp], _i),
        "iro_hip_dit_qk_norm_rope": ([_vp, _vp, _vp, _vp, _vp, _i, _i, _i, C.c_float], _i),
        "iro_hip_dit_head_rmsnorm": ([_vp, _vp, _vp, _i, _i, _i, C.c_float], _i),
        "iro_hip_dit_attn_context_create": ([_vp, _vp, _i, _i, _i, C.POINTER(_vp)], _i),
        "iro_hip_dit_adaln_params": ([_vp, _vp, _i, _i, _i, C.POINTER(_vp), _i, _vp], _i),
        "iro_hip_linear_f32": ([_vp, _vp, _i, _i, _vp, _i, _vp, _vp], _i),
        "iro_hip_rmsnorm_f32": ([_vp, _vp, _i, _i, _vp, C.c_float, _vp], _i),
        "iro_hip_euler_update": ([_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, C.c_float, C.c_float,
                                  C.c_float, C.c_float], _i),
        "iro_hip_selfcheck_tanhf": ([_vp, C.POINTER(C.c_ulonglong)], _i),
        "iro_hip_dit_attn_context_destroy": ([_vp], None),
        "iro_hip_dit_attention": ([_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, _vp], _i),
        "iro_hip_selfcheck_fp32": ([_vp, C.POINTER(C.c_ulonglong), C.POINTER(C.c_ulonglong)], _i),
        "iro_hip_profile_enable": ([_vp, _i], _i),
        "iro_hip_profile_reset": ([_vp], _i),
        "iro_hip_profile_kinds": ([], _i),
        "iro_hip_profile_read": ([_vp, _i, C.POINTER(C.c_char_p), C.POINTER(C.c_longlong),
                                  C.POINTER(C.c_double), C.POINTER(C.c_double),
                                  C.POINTER(C.c_double)], _i),
        "iro_hip_selfcheck": ([_vp], _i),
        "iro_hip_snake": ([_vp, _vp, _i, _i, _vp, _vp], _i),
        "iro_hip_silu": ([_vp, _vp, _vp, C.c_longlong], _i),
        "iro_hip_gated_residual": ([_vp, _vp, _vp, _i, _vp, _i, _i, _i], _i),
        "iro_hip_dit_condition": ([_vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _vp], _i),
        "iro_hip_dit_stack_set_int8_mask": ([_vp, _i], _i),
        "iro_hip_dit_stack_get_int8_mask": ([_vp], _i),
        "iro_hip_dit_stack_set_runs": ([_vp, _i], _i),
        "iro_hip_selfcheck_inject_fault": ([_i], _i),
        "iro_hip_selfcheck_codes": ([_vp, C.POINTER(C.c_ulonglong)], _i),
        "iro_hip_snake_bias": ([_vp, _vp, _i, _i, _vp, _vp, _vp], _i),
        "iro_hip_selfcheck_sincosf": ([_vp, C.POINTER(C.c_ulonglong),
                                       C.POINTER(C.c_ulonglong)], _i),
        "iro_hip_dacvae_residual_int8": ([_vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i,
                                          _i, _vp], _i),
        "iro_hip_dacvae_create": ([_vp, C.POINTER(DACVAEDecoderF32), C.POINTER(_vp)], _i),
        "iro_hip_dacvae_int8_bytes": ([_vp], C.c_size_t),
        "iro_hip_dacvae_destroy": ([_vp], None),
        "iro_hip_dacvae_output_frames": ([_vp, _i], _i),
        "iro_hip_dacvae_decode_int8": ([_vp, _vp, _i, _i, _i, _vp], _i),
        "iro_hip_backend_name": ([_vp], C.c_char_p),
        # ops.h drop-in
        "iro_int8_weight_quantize": ([_vp, _vp, _i, _i], _i),
        "iro_int8_weight_quantize_transposed": ([_vp, _vp, _i, _i], _i),
        "iro_int8_weight_free": ([_vp], None),
        "iro_int8_weight_bytes": ([_vp], C.c_size_t),
        "iro_int8_quantize_rows": ([_vp, _i, _i, _vp, _vp, _vp], None),
        "iro_int8_quantize_rows_residual": ([_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp],
                                            None),
        "iro_int8_linear": ([_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp], None),
        "iro_int8_linear_ex": ([_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i], None),
        "iro_int8_fast_available": ([], _i),
        "iro_int8_prepare_backend": ([], C.c_char_p),
        "iro_int8_selfcheck": ([], _i),
        "iro_int8_last_error": ([], _i),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


class HipError(RuntimeError):
    pass


def _ptr(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


class DeviceArray:
    """A device allocation with a numpy shape/dtype; freed with its context."""

    def __init__(self, ctx: "Context", shape, dtype):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in np.atleast_1d(shape))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = C.c_void_p()
        ctx._check(ctx.lib.iro_hip_alloc(ctx.h, max(self.nbytes, 1), C.byref(p)), "alloc")
        self.ptr = p.value
        ctx._arrays.append(self)

    @property
    def vp(self):
        return C.c_void_p(self.ptr)

    def upload(self, host):
        host = np.ascontiguousarray(host, dtype=self.dtype)
        assert host.nbytes == self.nbytes, (host.shape, self.shape)
        self.ctx._check(self.ctx.lib.iro_hip_upload(self.ctx.h, self.vp, _ptr(host), self.nbytes),
                        "upload")
        return self

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        self.ctx._check(self.ctx.lib.iro_hip_download(self.ctx.h, _ptr(out), self.vp, self.nbytes),
                        "download")
        return out

    def free(self):
        if self.ptr:
            self.ctx.lib.iro_hip_free(self.ctx.h, self.vp)
            self.ptr = None

    def view(self, offset: int, shape) -> "DeviceView":
        """A window of this allocation from element `offset` (no ownership)."""
        v = DeviceView(self.ctx, shape, self.dtype, self.ptr + offset * self.dtype.itemsize)
        assert offset >= 0 and offset * self.dtype.itemsize + v.nbytes <= self.nbytes
        return v


class DeviceView(DeviceArray):
    """A non-owning window into a DeviceArray (freed with its parent)."""

    def __init__(self, ctx: "Context", shape, dtype, ptr: int):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in np.atleast_1d(shape))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = ptr

    def free(self):
        self.ptr = None


class AttnContext:
    """A device joined-key layout (iro_hip_dit_attn_context_create); destroy it
    before its Context is closed."""

    def __init__(self, ctx: "Context", h, B: int, C_: int):
        self.ctx, self.h, self.B, self.C = ctx, h, B, C_

    def destroy(self):
        if self.h:
            self.ctx.lib.iro_hip_dit_attn_context_destroy(self.h)
            self.h = None


ST_DTYPES = ["F32", "F16", "BF16", "I64", "I32", "I16", "I8", "U8", "BOOL"]
_ST_NP = {"F32": np.float32, "F16": np.float16, "I64": np.int64, "I32": np.int32,
          "I16": np.int16, "I8": np.int8, "U8": np.uint8, "BOOL": np.bool_}


class StError(RuntimeError):
    pass


class Safetensors:
    """A safetensors checkpoint through iro_hip_st_* (mmapped; no device)."""

    def __init__(self, path: str):
        self.lib = load()
        h = C.c_void_p()
        if self.lib.iro_hip_st_open(os.fsencode(path), C.byref(h)) != 0:
            raise StError(self.lib.iro_hip_st_last_error().decode(errors="replace"))
        self.h = h

    def names(self) -> list[str]:
        return [self.lib.iro_hip_st_name(self.h, i).decode()
                for i in range(self.lib.iro_hip_st_count(self.h))]

    def info(self, name: str):
        """(dtype name, shape, address, nbytes) of a tensor."""
        dt, nd = C.c_int(), C.c_int()
        shape = (C.c_uint64 * 8)()
        data, nb = C.c_void_p(), C.c_uint64()
        if self.lib.iro_hip_st_tensor(self.h, name.encode(), C.byref(dt), C.byref(nd), shape,
                                      C.byref(data), C.byref(nb)) != 0:
            raise KeyError(name)
        return ST_DTYPES[dt.value], tuple(shape[i] for i in range(nd.value)), data.value, nb.value

    def bytes(self, name: str) -> bytes:
        _, _, addr, nb = self.info(name)
        return C.string_at(addr, nb) if nb else b""

    def array(self, name: str) -> np.ndarray:
        dt, shape, _, _ = self.info(name)
        raw = self.bytes(name)
        if dt == "BF16":
            u = np.frombuffer(raw, np.uint16).astype(np.uint32) << 16
            return u.view(np.float32).reshape(shape)
        return np.frombuffer(raw, _ST_NP[dt]).reshape(shape)

    def meta(self, key: str):
        v = self.lib.iro_hip_st_meta(self.h, key.encode())
        return v.decode() if v is not None else None

    def close(self):
        if self.h:
            self.lib.iro_hip_st_close(self.h)
            self.h = None


class Weight:
    def __init__(self, ctx: "Context", handle: int):
        self.ctx = ctx
        self.h = C.c_void_p(handle)
        n, k = C.c_int(), C.c_int()
        ctx.lib.iro_hip_weight_dims(self.h, C.byref(n), C.byref(k))
        self.N, self.K = n.value, k.value

    def export(self):
        q = np.empty((self.N, self.K), np.int8)
        s = np.empty(self.N, np.float32)
        cs = np.empty(self.N, np.int32)
        self.ctx._check(self.ctx.lib.iro_hip_weight_export(self.ctx.h, self.h, _ptr(q), _ptr(s),
                                                           _ptr(cs)), "weight_export")
        return q, s, cs

    def nbytes(self):
        return self.ctx.lib.iro_hip_weight_bytes(self.h)

    def destroy(self):
        if self.h:
            self.ctx.lib.iro_hip_weight_destroy(self.h)
            self.h = None


class Context:
    """One HIP device context (stream, convention, workspace)."""

    def __init__(self, device: int = 0, convention: int = STRICT):
        self.lib = load()
        h = C.c_void_p()
        rc = self.lib.iro_hip_create(device, convention, C.byref(h))
        if rc != 0 or not h.value:
            raise HipError("iro_hip_create failed (no usable gfx950 device or selfcheck failed)")
        self.h = h
        self.convention = convention
        self._arrays: list[DeviceArray] = []
        self._weights: list[Weight] = []

    # -- plumbing --------------------------------------------------------------
    def _check(self, rc, what):
        if rc != 0:
            msg = self.lib.iro_hip_error(self.h).decode(errors="replace")
            self.lib.iro_hip_clear_error(self.h)
            raise HipError(f"{what}: {msg}")

    def release_all(self):
        """Free every array and weight made through this context so far."""
        for w in self._weights:
            w.destroy()
        for a in self._arrays:
            a.free()
        self._weights.clear()
        self._arrays.clear()

    def close(self):
        for w in self._weights:
            w.destroy()
        for a in self._arrays:
            a.free()
        self._weights.clear()
        self._arrays.clear()
        if self.h:
            self.lib.iro_hip_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def sync(self):
        self._check(self.lib.iro_hip_sync(self.h), "sync")

    def set_gemm_tile(self, ti: int, tj: int):
        self._check(self.lib.iro_hip_set_gemm_tile(self.h, ti, tj), "set_gemm_tile")

    def backend(self) -> str:
        return self.lib.iro_hip_backend_name(self.h).decode()

    def empty(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def to_device(self, host) -> DeviceArray:
        host = np.ascontiguousarray(host)
        return DeviceArray(self, host.shape, host.dtype).upload(host)

    def fill(self, arr: DeviceArray, value: int = 0):
        self._check(self.lib.iro_hip_fill(self.h, arr.vp, value, arr.nbytes), "fill")

    def copy(self, dst: DeviceArray, src: DeviceArray):
        if dst.nbytes != src.nbytes:
            raise ValueError("copy: size mismatch")
        self._check(self.lib.iro_hip_copy(self.h, dst.vp, src.vp, src.nbytes), "copy")

    def selfcheck(self) -> int:
        return self.lib.iro_hip_selfcheck(self.h)

    def selfcheck_fp32(self):
        """(sqrtf digest, 1/x digest) over every float input."""
        d, r = C.c_ulonglong(0), C.c_ulonglong(0)
        self._check(self.lib.iro_hip_selfcheck_fp32(self.h, C.byref(d), C.byref(r)),
                    "selfcheck_fp32")
        return int(d.value), int(r.value)

    def selfcheck_codes(self) -> int:
        """Float inputs whose packed code differs from clamp(rint(v), 0, 255)."""
        m = C.c_ulonglong(0)
        self._check(self.lib.iro_hip_selfcheck_codes(self.h, C.byref(m)), "selfcheck_codes")
        return int(m.value)

    def selfcheck_silu(self):
        """(expf digest over every float input, fast-division mismatches)."""
        d, m = C.c_ulonglong(0), C.c_ulonglong(0)
        self._check(self.lib.iro_hip_selfcheck_silu(self.h, C.byref(d), C.byref(m)),
                    "selfcheck_silu")
        return int(d.value), int(m.value)

    # -- events --------------------------------------------------------------------
    def event(self):
        e = C.c_void_p()
        if self.lib.iro_hip_event_create(C.byref(e)) != 0:
            raise HipError("event_create")
        return e

    def record(self, ev):
        self._check(self.lib.iro_hip_event_record(self.h, ev), "event_record")

    def elapsed_ms(self, e0, e1) -> float:
        ms = C.c_float()
        if self.lib.iro_hip_event_elapsed_ms(e0, e1, C.byref(ms)) != 0:
            raise HipError("event_elapsed")
        return ms.value

    # -- weights ---------------------------------------------------------------------
    def weight(self, w_dev: DeviceArray, N: int, K: int, transposed: bool = False) -> Weight:
        h = C.c_void_p()
        fn = (self.lib.iro_hip_weight_create_transposed if transposed
              else self.lib.iro_hip_weight_create)
        self._check(fn(self.h, w_dev.vp, N, K, C.byref(h)), "weight_create")
        w = Weight(self, h.value)
        self._weights.append(w)
        return w

    def dit_adaln_apply(self, x: DeviceArray, B: int, S: int, D: int, shift: DeviceArray,
                        scale: DeviceArray, eps: float, h: DeviceArray):
        self._check(self.lib.iro_hip_dit_adaln_apply(self.h, x.vp, B, S, D, shift.vp, scale.vp,
                                                     eps, h.vp), "dit_adaln_apply")

    def dit_qk_norm_rope(self, q: DeviceArray, q_weight: DeviceArray, k: DeviceArray,
                         k_weight: DeviceArray, B: int, S: int, D: int, eps: float):
        """dit.c:638-706 in place on q, k [B*S, D]."""
        self._check(self.lib.iro_hip_dit_qk_norm_rope(self.h, q.vp, q_weight.vp, k.vp,
                                                      k_weight.vp, B, S, D, eps),
                    "dit_qk_norm_rope")

    def dit_head_rmsnorm(self, x: DeviceArray, weight: DeviceArray, B: int, S: int, D: int,
                         eps: float):
        """dit.c:619-636 in place on x [B*S, D]."""
        self._check(self.lib.iro_hip_dit_head_rmsnorm(self.h, x.vp, weight.vp, B, S, D, eps),
                    "dit_head_rmsnorm")

    def dit_adaln_params(self, cond: DeviceArray, B: int, D: int, R: int, weights,
                         out: DeviceArray):
        """dit.c:543-588: out [len(weights) // 9, 3, B, D] from cond [B, 3D]."""
        n = len(weights) // 9
        arr = (_vp * len(weights))(*[w.vp for w in weights])
        self._check(self.lib.iro_hip_dit_adaln_params(self.h, cond.vp, B, D, R, arr, n, out.vp),
                    "dit_adaln_params")

    def linear_f32(self, x: DeviceArray, M: int, K: int, w: DeviceArray, N: int, bias, y):
        """ops.c:221-234: y [M, N] = x @ w^T (+ bias), K-order chains."""
        self._check(self.lib.iro_hip_linear_f32(self.h, x.vp, M, K, w.vp, N,
                                                None if bias is None else bias.vp, y.vp),
                    "linear_f32")

    def rmsnorm_f32(self, x: DeviceArray, M: int, D: int, w: DeviceArray, eps: float,
                    y: DeviceArray):
        """ops.c:738-747: y = (x * inv) * w."""
        self._check(self.lib.iro_hip_rmsnorm_f32(self.h, x.vp, M, D, w.vp, eps, y.vp),
                    "rmsnorm_f32")

    def euler_update(self, state: DeviceArray, velocity: DeviceArray, length: int, batch: int,
                     use_cfg: bool, rows, scales, dt: float):
        """sampler.c:281-297: state [length] += guided * dt in place; velocity
        [batch, length]; rows = (text, speaker, caption) unconditional rows,
        -1 when absent; scales the three CFG scales."""
        self._check(self.lib.iro_hip_euler_update(self.h, state.vp, velocity.vp, length, batch,
                                                  int(bool(use_cfg)), *[int(r) for r in rows],
                                                  *[float(x) for x in scales], float(dt)),
                    "euler_update")

    def selfcheck_tanhf(self) -> int:
        d = C.c_ulonglong(0)
        self._check(self.lib.iro_hip_selfcheck_tanhf(self.h, C.byref(d)), "selfcheck_tanhf")
        return int(d.value)

    def attn_context(self, mask, context_batch: int) -> "AttnContext":
        """The joined-key layout of mask [B, C] (host uint8) for dit_attention."""
        mask = np.ascontiguousarray(mask, np.uint8)
        B, Cn = mask.shape
        h = C.c_void_p()
        self._check(self.lib.iro_hip_dit_attn_context_create(self.h, _ptr(mask), B, Cn,
                                                             context_batch, C.byref(h)),
                    "dit_attn_context")
        return AttnContext(self, h.value, B, Cn)

    def dit_attention(self, actx: "AttnContext", q: DeviceArray, k: DeviceArray,
                      v: DeviceArray, gate: DeviceArray, B: int, S: int, D: int,
                      context_k: DeviceArray, context_v: DeviceArray, mix: DeviceArray):
        """dit.c:808-870: mix [B*S, D] from q, k, v, gate and the context rows."""
        self._check(self.lib.iro_hip_dit_attention(self.h, actx.h, q.vp, k.vp, v.vp, gate.vp, B,
                                                   S, D, context_k.vp, context_v.vp, mix.vp),
                    "dit_attention")

    def weight_from_st(self, st: Safetensors, name: str, transposed: bool = False) -> Weight:
        h = C.c_void_p()
        self._check(self.lib.iro_hip_weight_from_st(self.h, st.h, name.encode(), int(transposed),
                                                    C.byref(h)), "weight_from_st")
        w = Weight(self, h.value)
        self._weights.append(w)
        return w

    def weight_save(self, w: Weight, path: str):
        self._check(self.lib.iro_hip_weight_save(self.h, w.h, os.fsencode(path)), "weight_save")

    def weight_load(self, path: str) -> Weight:
        h = C.c_void_p()
        self._check(self.lib.iro_hip_weight_load(self.h, os.fsencode(path), C.byref(h)),
                    "weight_load")
        w = Weight(self, h.value)
        self._weights.append(w)
        return w

    def weight_fused(self, parts: list[DeviceArray], parts_N: list[int], K: int,
                     layout: int) -> Weight:
        h = C.c_void_p()
        arr = (C.c_void_p * len(parts))(*[p.ptr for p in parts])
        pn = (C.c_int * len(parts))(*parts_N)
        self._check(self.lib.iro_hip_weight_create_fused(self.h, arr, pn, len(parts), K, layout,
                                                         C.byref(h)), "weight_create_fused")
        w = Weight(self, h.value)
        self._weights.append(w)
        return w

    def weight_from_host(self, q, scale, colsum) -> Weight:
        q = np.ascontiguousarray(q, np.int8)
        N, K = q.shape
        h = C.c_void_p()
        self._check(self.lib.iro_hip_weight_from_host(
            self.h, _ptr(q), _ptr(np.ascontiguousarray(scale, np.float32)),
            _ptr(np.ascontiguousarray(colsum, np.int32)), N, K, C.byref(h)), "weight_from_host")
        w = Weight(self, h.value)
        self._weights.append(w)
        return w

    # -- ops (device arrays in, device arrays out) -----------------------------------
    def quantize_rows(self, x: DeviceArray, q, s, z):
        M, K = x.shape
        self._check(self.lib.iro_hip_quantize_rows(self.h, x.vp, M, K, q.vp, s.vp, z.vp),
                    "quantize_rows")

    def quantize_rows_residual(self, x, q1, s1, z1, r, q2, s2, z2):
        M, K = x.shape
        self._check(self.lib.iro_hip_quantize_rows_residual(
            self.h, x.vp, M, K, q1.vp, s1.vp, z1.vp, None if r is None else r.vp, q2.vp, s2.vp,
            z2.vp), "quantize_rows_residual")

    def linear_ex(self, q, s, z, w: Weight, bias, y, M, work=None, accumulate=False):
        self._check(self.lib.iro_hip_int8_linear_ex(
            self.h, q.vp, s.vp, z.vp, w.h, None if bias is None else bias.vp, y.vp, M,
            None if work is None else work.vp, int(bool(accumulate))), "int8_linear_ex")

    def linear_two_term(self, q1, s1, z1, q2, s2, z2, w: Weight, bias, y, M, accumulate=False):
        self._check(self.lib.iro_hip_int8_linear_two_term(
            self.h, q1.vp, s1.vp, z1.vp, q2.vp, s2.vp, z2.vp, w.h,
            None if bias is None else bias.vp, y.vp, M, int(bool(accumulate))),
            "int8_linear_two_term")

    def dit_qkvg(self, x, M, w, q, k, v, g, residual=False):
        self._check(self.lib.iro_hip_dit_qkvg(self.h, x.vp, M, w.h, q.vp, k.vp, v.vp, g.vp,
                                              int(bool(residual))), "dit_qkvg")

    def dit_linear_gated(self, mix, M, w, residual, out=None, x_res=None, gate=None, S=1):
        self._check(self.lib.iro_hip_dit_linear_gated(
            self.h, mix.vp, M, w.h, int(bool(residual)), None if out is None else out.vp,
            None if x_res is None else x_res.vp, None if gate is None else gate.vp, S),
            "dit_linear_gated")

    def dit_swiglu(self, h, M, w13, w2, residual_w13=False, residual_w2=True, hidden=None,
                   out=None, x_res=None, gate=None, S=1):
        self._check(self.lib.iro_hip_dit_swiglu(
            self.h, h.vp, M, w13.h, w2.h, int(bool(residual_w13)), int(bool(residual_w2)),
            None if hidden is None else hidden.vp, None if out is None else out.vp,
            None if x_res is None else x_res.vp, None if gate is None else gate.vp, S),
            "dit_swiglu")

    def conv1d(self, x, T, Cin, w, kernel, stride, dilation, padding, bias, residual, y):
        t_out = C.c_int()
        self._check(self.lib.iro_hip_conv1d_int8(
            self.h, x.vp, T, Cin, w.h, kernel, stride, dilation, padding,
            None if bias is None else bias.vp, int(bool(residual)), y.vp, C.byref(t_out)),
            "conv1d_int8")
        return t_out.value

    def convtranspose1d(self, x, T_in, Cin, w, Cout, kernel, stride, padding, output_padding,
                        bias, residual, y):
        """dacvae.c:696-795 int8 ConvTranspose1d (no snake); returns T_out."""
        t_out = C.c_int()
        self._check(self.lib.iro_hip_convtranspose1d_int8(
            self.h, x.vp, T_in, Cin, w.h, Cout, kernel, stride, padding, output_padding,
            None if bias is None else bias.vp, int(bool(residual)), y.vp, C.byref(t_out)),
            "convtranspose1d_int8")
        return t_out.value

    def conv1x1_skip(self, hidden, skip, T, w, bias, residual, out):
        """dacvae.c:974-1012: out = skip + conv1(hidden) + bias (int8)."""
        self._check(self.lib.iro_hip_conv1x1_skip_int8(
            self.h, hidden.vp, skip.vp, T, w.h, None if bias is None else bias.vp,
            int(bool(residual)), out.vp), "conv1x1_skip_int8")


    # -- fp32 pieces around the int8 linears -------------------------------------------
    def silu(self, x, n, gate=None):
        """ops.c:776-784 in place: x = silu(x) [* gate]."""
        self._check(self.lib.iro_hip_silu(self.h, x.vp, None if gate is None else gate.vp, n),
                    "silu")

    def gated_residual(self, x, gate, ldg, branch, M, D, S):
        """dit.c:1013-1020: x += gate[m / S] * branch."""
        self._check(self.lib.iro_hip_gated_residual(self.h, x.vp, gate.vp, ldg, branch.vp, M, D,
                                                    S), "gated_residual")

    def dit_condition(self, t, B, w0, w1, w2, tdim, D, cond_dim, cond):
        """iro_dit_condition (dit.c:488-530) into cond [B, cond_dim]."""
        self._check(self.lib.iro_hip_dit_condition(self.h, t.vp, B, w0.vp, w1.vp, w2.vp, tdim, D,
                                                   cond_dim, cond.vp), "dit_condition")

    # -- codec ---------------------------------------------------------------------------
    def snake(self, x, T, Cc, alpha, y):
        """iro_snake_forward (dacvae.c:830-857); y may be x."""
        self._check(self.lib.iro_hip_snake(self.h, x.vp, T, Cc, alpha.vp, y.vp), "snake")

    def snake_bias(self, x, T, Cc, bias, alpha, y):
        """snake_bias_forward (dacvae.c:910-931); y may be x."""
        self._check(self.lib.iro_hip_snake_bias(self.h, x.vp, T, Cc, bias.vp, alpha.vp, y.vp),
                    "snake_bias")

    def selfcheck_sincosf(self):
        """(sinf digest, cosf digest) over every float input."""
        a, b = C.c_ulonglong(0), C.c_ulonglong(0)
        self._check(self.lib.iro_hip_selfcheck_sincosf(self.h, C.byref(a), C.byref(b)),
                    "selfcheck_sincosf")
        return int(a.value), int(b.value)

    def dacvae_residual(self, x, T, Cc, conv0, alpha0, conv0_bias, alpha1, dilation, conv1,
                        conv1_bias, residual_conv7, residual_conv1, out):
        """run_residual_int8 (dacvae.c:934-1018)."""
        self._check(self.lib.iro_hip_dacvae_residual_int8(
            self.h, x.vp, T, Cc, conv0.h, alpha0.vp, conv0_bias.vp, alpha1.vp, dilation, conv1.h,
            conv1_bias.vp, int(bool(residual_conv7)), int(bool(residual_conv1)), out.vp),
            "dacvae_residual_int8")

    # -- profiler ----------------------------------------------------------------------
    def profile(self, on: bool):
        self._check(self.lib.iro_hip_profile_enable(self.h, int(bool(on))), "profile_enable")

    def profile_reset(self):
        self._check(self.lib.iro_hip_profile_reset(self.h), "profile_reset")

    def profile_read(self) -> dict:
        """{kind: (launches, total_ms, ops, bytes)} for kinds with launches."""
        out = {}
        for k in range(self.lib.iro_hip_profile_kinds()):
            name = C.c_char_p()
            n = C.c_longlong()
            ms, ops, by = C.c_double(), C.c_double(), C.c_double()
            self._check(self.lib.iro_hip_profile_read(self.h, k, C.byref(name), C.byref(n),
                                                      C.byref(ms), C.byref(ops), C.byref(by)),
                        "profile_read")
            if n.value:
                out[name.value.decode()] = (n.value, ms.value, ops.value, by.value)
        return out


class DiTStack:
    """The int8 linear stack of one Euler step (iro_hip_dit_stack_*)."""

    def __init__(self, ctx: Context, blocks: int, D: int, H: int, residual_mask: int = 8):
        self.ctx = ctx
        self.blocks, self.D, self.H = blocks, D, H
        h = C.c_void_p()
        ctx._check(ctx.lib.iro_hip_dit_stack_create(ctx.h, blocks, D, H, residual_mask,
                                                    C.byref(h)), "dit_stack_create")
        self.h = h

    def set_block(self, block, ada, wq, wk, wv, wgate, wo, w1, w3, w2):
        ctx = self.ctx
        ctx._check(ctx.lib.iro_hip_dit_stack_set_block(
            self.h, block, *[None if a is None else a.vp
                             for a in (ada, wq, wk, wv, wgate, wo, w1, w3, w2)]),
            "dit_stack_set_block")

    def buffers(self, B: int, S: int) -> dict:
        """Views of the last step's activation buffers (iro_hip_dit_stack_buffers):
        q, k, v, gate [B*S, D], hidden [B*S, H] and the modulation rows of every
        block, mod [B, blocks * P] (block b at column b * P, P = 6D rounded up
        to 256)."""
        ptrs = [C.c_void_p() for _ in range(6)]
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_buffers(self.h, *[C.byref(p) for p in ptrs]),
                        "dit_stack_buffers")
        M, D, H = B * S, self.D, self.H
        P = (6 * D + 255) // 256 * 256
        shapes = [(M, D)] * 4 + [(M, H), (B, self.blocks * P)]
        names = ["q", "k", "v", "gate", "hidden", "mod"]
        return {n: DeviceView(self.ctx, s, np.float32, p.value)
                for n, s, p in zip(names, shapes, ptrs)}

    def step(self, x: DeviceArray, cond: DeviceArray, B: int, S: int):
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_step(self.h, x.vp, cond.vp, B, S),
                        "dit_stack_step")

    def block_forward(self, block: int, x: DeviceArray, B: int, S: int, ada_attn: DeviceArray,
                      ada_mlp: DeviceArray, q_norm: DeviceArray, k_norm: DeviceArray, eps: float,
                      actx: "AttnContext", context_k: DeviceArray, context_v: DeviceArray):
        """dit.c:984-1040: one DiT block in place on x [B*S, D]."""
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_block_forward(
            self.h, block, x.vp, B, S, ada_attn.vp, ada_mlp.vp, q_norm.vp, k_norm.vp, eps,
            actx.h, context_k.vp, context_v.vp), "dit_block_forward")

    def set_layer_f32(self, layer: int, adaln, q_norm, k_norm, context_k, context_v):
        """Borrow layer's 18 adaLN arrays, head norms and cached context K/V."""
        p = DiTLayerF32((_vp * 18)(*[a.vp for a in adaln]), q_norm.vp, k_norm.vp, context_k.vp,
                        context_v.vp)
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_set_layer_f32(self.h, layer, C.byref(p)),
                        "dit_stack_set_layer_f32")

    def set_head(self, in_w, in_b, out_norm, out_w, out_b, latent: int, rank: int, eps: float):
        h = DiTHead(in_w.vp, in_b.vp, out_norm.vp, out_w.vp, out_b.vp, latent, rank, eps)
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_set_head(self.h, C.byref(h)),
                        "dit_stack_set_head")

    def sampler_step(self, state: DeviceArray, cond: DeviceArray, batch: int, S: int,
                     actx: "AttnContext", use_cfg: bool, rows, scales, dt: float,
                     velocity: DeviceArray):
        """sampler.c:259-297: one Euler step; state [S, latent] updated in place,
        velocity [batch*S, latent] receives the DiT output."""
        self.ctx._check(self.ctx.lib.iro_hip_dit_sampler_step(
            self.h, state.vp, cond.vp, batch, S, actx.h, int(bool(use_cfg)),
            *[int(r) for r in rows], *[float(x) for x in scales], float(dt), velocity.vp),
            "dit_sampler_step")

    def set_int8_mask(self, mask: int):
        """IRO_INT8_MASK (dit.c:273-291); before the first set_block."""
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_set_int8_mask(self.h, mask),
                        "dit_stack_set_int8_mask")

    def set_runs(self, runs: int):
        """Concurrent row runs of the stack step (0/1 off)."""
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_set_runs(self.h, runs),
                        "dit_stack_set_runs")

    def use_persistent(self, on: bool):
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_use_persistent(self.h, int(bool(on))),
                        "dit_stack_use_persistent")

    def use_graph(self, on: bool):
        self.ctx._check(self.ctx.lib.iro_hip_dit_stack_use_graph(self.h, int(bool(on))),
                        "dit_stack_use_graph")

    def nbytes(self):
        return self.ctx.lib.iro_hip_dit_stack_bytes(self.h)

    def destroy(self):
        if self.h:
            self.ctx.lib.iro_hip_dit_stack_destroy(self.h)
            self.h = None


class DACVAE:
    """The decoder's int8 weights and core (iro_hip_dacvae_*).  params: the
    fp32 device arrays, dict(initial_w, initial_b, stages=[dict(alpha, up_w,
    up_b, c_in, c_out, kernel, stride, padding, output_padding,
    residual=[dict(alpha0, w0, b0, alpha1, w1, b1, dil)] * 3)] * 4); they are
    borrowed and must outlive this object."""

    def __init__(self, ctx: Context, params: dict):
        self.ctx = ctx
        self._keep = params
        p = DACVAEDecoderF32()
        p.initial_weight = params["initial_w"].vp
        p.initial_bias = params["initial_b"].vp
        p.latent_channels = params["latent_channels"]
        p.channels = params["channels"]
        for i, st in enumerate(params["stages"]):
            d = p.stage[i]
            d.alpha, d.up_weight, d.up_bias = st["alpha"].vp, st["up_w"].vp, st["up_b"].vp
            for f in ("c_in", "c_out", "kernel", "stride", "padding", "output_padding"):
                setattr(d, f, st[f])
            for r, u in enumerate(st["residual"]):
                e = d.residual[r]
                e.alpha0, e.conv0_weight, e.conv0_bias = u["alpha0"].vp, u["w0"].vp, u["b0"].vp
                e.alpha1, e.conv1_weight, e.conv1_bias = u["alpha1"].vp, u["w1"].vp, u["b1"].vp
                e.dilation = u["dil"]
        h = C.c_void_p()
        ctx._check(ctx.lib.iro_hip_dacvae_create(ctx.h, C.byref(p), C.byref(h)), "dacvae_create")
        self.h = h

    def nbytes(self) -> int:
        return int(self.ctx.lib.iro_hip_dacvae_int8_bytes(self.h))

    def output_frames(self, frames: int) -> int:
        return int(self.ctx.lib.iro_hip_dacvae_output_frames(self.h, frames))

    def decode_int8(self, state, frames, out, residual_mask=12, residual_stages=8):
        self.ctx._check(self.ctx.lib.iro_hip_dacvae_decode_int8(
            self.h, state.vp, frames, residual_mask, residual_stages, out.vp),
            "dacvae_decode_int8")

    def destroy(self):
        if self.h:
            self.ctx.lib.iro_hip_dacvae_destroy(self.h)
            self.h = None


class _Int8Weight(C.Structure):
    # include/iro_int8_ops.h IroInt8Weight (ops.h:23-28)
    _fields_ = [("data", C.POINTER(C.c_int8)), ("scale", C.POINTER(C.c_float)),
                ("colsum", C.POINTER(C.c_int32)), ("N", C.c_int), ("K", C.c_int)]


class Ops:
    """The ops.h drop-in (host pointers), exactly as dit.c/dacvae.c call it."""

    def __init__(self):
        self.lib = load()

    def weight_quantize(self, w, transposed_shape=None):
        w = np.ascontiguousarray(w, np.float32)
        st = _Int8Weight()
        if transposed_shape is None:
            N, K = w.shape
            rc = self.lib.iro_int8_weight_quantize(C.byref(st), _ptr(w), N, K)
        else:
            N, K = transposed_shape
            rc = self.lib.iro_int8_weight_quantize_transposed(C.byref(st), _ptr(w), N, K)
        if rc != 0:
            raise HipError("iro_int8_weight_quantize failed")
        return st

    @staticmethod
    def weight_arrays(st):
        N, K = st.N, st.K
        return (np.ctypeslib.as_array(st.data, (N * K,)).reshape(N, K).copy(),
                np.ctypeslib.as_array(st.scale, (N,)).copy(),
                np.ctypeslib.as_array(st.colsum, (N,)).copy())

    def weight_free(self, st):
        self.lib.iro_int8_weight_free(C.byref(st))

    def weight_bytes(self, st):
        return self.lib.iro_int8_weight_bytes(C.byref(st))

    def quantize_rows(self, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        q = np.empty((M, K), np.uint8)
        s = np.empty(M, np.float32)
        z = np.empty(M, np.int32)
        self.lib.iro_int8_quantize_rows(_ptr(x), M, K, _ptr(q), _ptr(s), _ptr(z))
        return q, s, z

    def quantize_rows_residual(self, x):
        x = np.ascontiguousarray(x, np.float32)
        M, K = x.shape
        q1, q2 = np.empty((M, K), np.uint8), np.empty((M, K), np.uint8)
        r = np.empty((M, K), np.float32)
        s1, s2 = np.empty(M, np.float32), np.empty(M, np.float32)
        z1, z2 = np.empty(M, np.int32), np.empty(M, np.int32)
        self.lib.iro_int8_quantize_rows_residual(_ptr(x), M, K, _ptr(q1), _ptr(s1), _ptr(z1),
                                                 _ptr(r), _ptr(q2), _ptr(s2), _ptr(z2))
        return (q1, s1, z1), r, (q2, s2, z2)

    def linear_ex(self, q, s, z, st, bias=None, y=None, accumulate=False):
        q = np.ascontiguousarray(q, np.uint8)
        M = q.shape[0]
        N = st.N
        y = np.zeros((M, N), np.float32) if y is None else np.array(y, np.float32, copy=True)
        work = np.empty((M, N), np.int32)
        self.lib.iro_int8_linear_ex(_ptr(q), _ptr(np.ascontiguousarray(s, np.float32)),
                                    _ptr(np.ascontiguousarray(z, np.int32)), C.byref(st),
                                    None if bias is None else _ptr(np.ascontiguousarray(bias, np.float32)),
                                    _ptr(y), M, _ptr(work), int(bool(accumulate)))
        return y, work

    def selfcheck(self):
        return self.lib.iro_int8_selfcheck()

    def last_error(self):
        return self.lib.iro_int8_last_error()
