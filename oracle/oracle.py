"""ctypes binding of the CPU oracle (oracle/fa_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, where it is the checker (or the timed CPU
baseline), never the product path.

Functions
---------
fa_ggml(q, k, v, mask, scale, ..., acc_f32=False) -> float32 [B, Sq, Nh, DV]
    restatement of ggml's CPU flash_attn_ext (see fa_oracle.c header);
    acc_f32=True runs the same algorithm with an fp32 V accumulator.
fa_exact(q, k, v, mask, scale, ...) -> float64 [B, Sq, Nh, DV]
    fp64 two-pass softmax reference of the same op.
qk_norm_rope(q, k, v, q_w, k_w, pos, eps, base, clamp_v) -> (q, k, v) F32
    restatement of ggml's CPU rms_norm * weight + NEOX rope (+ V clamp).
qk_norm(x, w, eps) -> F32
    the same rms_norm * weight without RoPE (DiT cross-attention).
set_rows(dst, src, rows) -> skipped rows
    restatement of ggml's CPU set_rows (the KV-cache write), in place on dst.

Inputs are `HostTensor`s: raw host bytes plus ggml type / ne / nb, so the
oracle reads exactly the strided views the reference builds.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "build", "libfa_oracle.so")

F32, F16, Q8_0, BF16, I32, I64 = 0, 1, 8, 30, 26, 27


class _OraTensor(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
        ("data", ctypes.c_void_p),
    ]


@dataclass
class HostTensor:
    """A ggml-style view over a host byte buffer."""

    type: int
    ne: tuple
    nb: tuple
    buf: np.ndarray          # backing storage (any dtype), kept alive here
    offset: int = 0          # byte offset of element (0,0,0,0) in buf

    def ptr(self) -> int:
        return self.buf.ctypes.data + self.offset



_lib = None


def build() -> None:
    import subprocess

    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.POINTER(_OraTensor)
        L.ora_fa_ggml.argtypes = [P, P, P, P, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                  ctypes.c_void_p, ctypes.c_int]
        L.ora_fa_ggml.restype = ctypes.c_int
        L.ora_fa_ggml_ex.argtypes = [P, P, P, P, ctypes.c_float, ctypes.c_float, ctypes.c_float,
                                     ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        L.ora_fa_ggml_ex.restype = ctypes.c_int
        L.ora_fa_exact.argtypes = [P, P, P, P, ctypes.c_double, ctypes.c_double, ctypes.c_double,
                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        L.ora_fa_exact.restype = ctypes.c_int
        for name in ("ora_f32_to_f16", "ora_f32_to_bf16"):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        for name in ("ora_f16_to_f32", "ora_bf16_to_f32"):
            getattr(L, name).argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.ora_quantize_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        L.ora_dequantize_q8_0.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        for name in ("ora_dot_f16", "ora_dot_bf16", "ora_dot_q8_0"):
            getattr(L, name).argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]
            getattr(L, name).restype = ctypes.c_float
        L.ora_mad_f16.argtypes = [ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_float]
        L.ora_qk_norm_rope.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 5 + [ctypes.c_float] * 2 + \
            [ctypes.c_int] + [ctypes.c_void_p] * 3
        L.ora_qk_norm.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p]
        L.ora_qk_norm.restype = None
        L.ora_set_rows.argtypes = [P, P, P]
        L.ora_set_rows.restype = ctypes.c_int64
        L.ora_set_force_scalar.argtypes = [ctypes.c_int]
        L.ora_simd_available.restype = ctypes.c_int
        _lib = L
    return _lib


def _desc(t) -> _OraTensor:
    """Descriptor of any ggml-style host view (type, ne, nb, ptr())."""
    d = _OraTensor()
    d.type = int(t.type)
    for i in range(4):
        d.ne[i] = int(t.ne[i])
        d.nb[i] = int(t.nb[i])
    d.data = ctypes.c_void_p(int(t.ptr()))
    return d


def _threads(n_threads):
    if n_threads is None:
        n_threads = max(1, (os.cpu_count() or 2) // 2)
    return int(n_threads)


def _out_shape(q: HostTensor, v: HostTensor):
    return (int(q.ne[3]), int(q.ne[1]), int(q.ne[2]), int(v.ne[0]))


def fa_ggml(q, k, v, mask, scale, max_bias=0.0, softcap=0.0, n_threads=None, acc_f32=False) -> np.ndarray:
    """ggml CPU flash_attn_ext semantics.  acc_f32=False: as ggml runs it
    (fp16 running accumulator for F16 V); acc_f32=True: same algorithm with an
    fp32 accumulator."""
    out = np.zeros(_out_shape(q, v), dtype=np.float32)
    dq, dk, dv = _desc(q), _desc(k), _desc(v)
    dm = _desc(mask) if mask is not None else None
    rc = lib().ora_fa_ggml_ex(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv),
                              ctypes.byref(dm) if dm is not None else None,
                              scale, max_bias, softcap, int(bool(acc_f32)), out.ctypes.data,
                              _threads(n_threads))
    if rc:
        raise ValueError(f"ora_fa_ggml rejected the shapes (rc={rc})")
    return out


def fa_exact(q, k, v, mask, scale, max_bias=0.0, softcap=0.0, q_round=False,
             n_threads=None) -> np.ndarray:
    out = np.zeros(_out_shape(q, v), dtype=np.float64)
    dq, dk, dv = _desc(q), _desc(k), _desc(v)
    dm = _desc(mask) if mask is not None else None
    rc = lib().ora_fa_exact(ctypes.byref(dq), ctypes.byref(dk), ctypes.byref(dv),
                            ctypes.byref(dm) if dm is not None else None,
                            scale, max_bias, softcap, int(bool(q_round)), out.ctypes.data,
                            _threads(n_threads))
    if rc:
        raise ValueError(f"ora_fa_exact rejected the shapes (rc={rc})")
    return out


# -- codecs ------------------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().ora_f32_to_f16(x.ctypes.data, y.ctypes.data, x.size)
    return y


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().ora_f16_to_f32(h.ctypes.data, y.ctypes.data, h.size)
    return y


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().ora_f32_to_bf16(x.ctypes.data, y.ctypes.data, x.size)
    return y


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().ora_bf16_to_f32(h.ctypes.data, y.ctypes.data, h.size)
    return y


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % 32 == 0
    y = np.empty(x.size // 32 * 34, dtype=np.uint8)
    lib().ora_quantize_q8_0(x.ctypes.data, y.ctypes.data, x.size)
    return y


def dequantize_q8_0(y: np.ndarray, n: int) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.uint8)
    x = np.empty(n, dtype=np.float32)
    lib().ora_dequantize_q8_0(y.ctypes.data, x.ctypes.data, n)
    return x


# -- KV-cache write (GGML_OP_SET_ROWS) -----------------------------------------

def set_rows(dst: HostTensor, src: HostTensor, rows: HostTensor) -> int:
    """ggml set_rows on host views: converts src's F32 rows into dst (in
    place) at the rows that `rows` names; returns the number of rows skipped
    for an out-of-range id."""
    dd, ds, dr = _desc(dst), _desc(src), _desc(rows)
    n = lib().ora_set_rows(ctypes.byref(dd), ctypes.byref(ds), ctypes.byref(dr))
    if n < 0:
        raise ValueError("ora_set_rows rejected the shapes")
    return int(n)


# -- pre-attention work (rms_norm, NEOX rope) ----------------------------------

def qk_norm(x, w, eps):
    """x [..., 128] float32: rms_norm(x, eps) * w per row of 128, as ggml's
    CPU ops compute it (the QK-norm of DiT cross-attention, no RoPE)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    assert x.shape[-1] == 128 and w.shape == (128,)
    y = np.empty_like(x)
    lib().ora_qk_norm(x.ctypes.data, w.ctypes.data, x.size // 128, eps, y.ctypes.data)
    return y


def qk_norm_rope(q, k, v, q_w, k_w, pos, eps, freq_base, clamp_v=False):
    """q [B, S, Nh, 128], k/v [B, S, Nkv, 128] float32, pos [S] or [B, S]
    int32: returns the F32 rows ggml's ops produce before the 16-bit cast."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    q_w = np.ascontiguousarray(q_w, dtype=np.float32)
    k_w = np.ascontiguousarray(k_w, dtype=np.float32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    B, S, Nh, D = q.shape
    Nkv = k.shape[2]
    assert D == 128 and k.shape == (B, S, Nkv, 128) and v.shape == k.shape
    per_batch = int(pos.ndim == 2)
    qo, ko, vo = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    lib().ora_qk_norm_rope(q.ctypes.data, k.ctypes.data, v.ctypes.data, q_w.ctypes.data, k_w.ctypes.data,
                           pos.ctypes.data, per_batch, Nh, Nkv, S, B, eps, freq_base, int(bool(clamp_v)),
                           qo.ctypes.data, ko.ctypes.data, vo.ctypes.data)
    return qo, ko, vo
