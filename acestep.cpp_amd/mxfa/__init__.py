"""Python binding of libmxfa (the gfx950 flash-attention engine, C ABI in
include/mxfa.h).

It mirrors the reference's operator interface for this path:
``flash_attn_ext(q, k, v, mask, scale, max_bias, logit_softcap, prec)`` is
ggml_flash_attn_ext + ggml_flash_attn_ext_set_prec as acestep.cpp calls them
(src/qwen3-lm.h:465-469, :789-794; src/dit-graph.h:227-231, :348-352;
src/qwen3-enc.h:195-199), and ``supports`` is the backend's supports_op for
GGML_OP_FLASH_ATTN_EXT; ``set_rows`` / ``set_rows_supports`` do the same for
the KV-cache write before it (ggml_set_rows, src/qwen3-lm.h:453-454,
:776-777).  Tensors are ggml views: a type id, ne[4], nb[4] and
a device pointer (`DeviceView`).  Device memory and streams come from torch
(plumbing only); all arithmetic runs in the HIP kernels of libmxfa.so.

The library must exist (built by ``make -C acestep.cpp_amd`` or
``__graft_entry__.build()``); there is no fallback: importing this module
without it raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
from dataclasses import dataclass
from typing import Optional

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# MXFA_LIB names another build of the library (e.g. an instrumented one);
# the default is the in-tree build.
LIB_PATH = os.environ.get("MXFA_LIB") or os.path.join(_PKG_DIR, "lib", "libmxfa.so")

TYPE_F32, TYPE_F16, TYPE_Q8_0, TYPE_BF16 = 0, 1, 8, 30
TYPE_I32, TYPE_I64 = 26, 27
PREC_DEFAULT, PREC_F32 = 0, 10

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP, ERR_NOMEM = 0, -1, -2, -3, -4

# Symbols declared in include/mxfa.h.
EXPORTED_SYMBOLS = (
    "mxfa_supports",
    "mxfa_flash_attn_ext",
    "mxfa_supports_masked",
    "mxfa_flash_attn_ext_masked",
    "mxfa_flash_attn_ext_noalloc",
    "mxfa_reserve",
    "mxfa_graph_begin",
    "mxfa_graph_end",
    "mxfa_qk_norm_rope",
    "mxfa_qk_norm_rope_supports",
    "mxfa_set_rows_supports",
    "mxfa_set_rows",
    "mxfa_release",
    "mxfa_workspace_info",
    "mxfa_status_string",
    "mxfa_last_error",
    "mxfa_version",
    "mxfa_timing_enable",
    "mxfa_timing_read",
    "mxfa_timing_reset",
)


class MxfaTensor(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_size_t * 4),
        ("data", ctypes.c_void_p),
    ]


class MxfaParams(ctypes.Structure):
    _fields_ = [
        ("scale", ctypes.c_float),
        ("max_bias", ctypes.c_float),
        ("logit_softcap", ctypes.c_float),
        ("prec", ctypes.c_int32),
    ]


class MxfaNormRopeParams(ctypes.Structure):
    _fields_ = [("eps", ctypes.c_float), ("freq_base", ctypes.c_float), ("clamp_v", ctypes.c_int32)]


MASK_CAUSAL, MASK_WINDOW, MASK_LENGTHS, MASK_DEVICE = 1, 2, 4, 8


class MxfaMaskSpec(ctypes.Structure):
    _fields_ = [
        ("flags", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("pos0", ctypes.c_int64),
        ("n_lengths", ctypes.c_int32),
        ("lengths", ctypes.POINTER(ctypes.c_int32)),
        ("dev_pos0", ctypes.c_void_p),
    ]


def mask_spec(causal: bool = False, pos0: int = 0, window: Optional[int] = None, lengths=None,
              device_lengths=None, device_pos0=None):
    """A structured mask (mxfa_mask_spec).  Key j is live for query row i of
    batch b iff j < lengths[b % len(lengths)] (lengths given), j <= pos0 + i
    (causal), |pos0 + i - j| <= window (window given).  device_lengths /
    device_pos0: int32 torch tensors on the GPU read by the kernels at run
    time (MXFA_MASK_DEVICE) instead of host values fixed at the call."""
    sp = MxfaMaskSpec()
    dev = device_lengths is not None or device_pos0 is not None
    sp.flags = (MASK_CAUSAL if causal else 0) | (MASK_WINDOW if window is not None else 0) | \
        (MASK_LENGTHS if (lengths is not None or device_lengths is not None) else 0) | (MASK_DEVICE if dev else 0)
    sp.window = int(window or 0)
    sp.pos0 = int(pos0)
    if dev:
        keep = []
        if device_lengths is not None:
            sp.n_lengths = int(device_lengths.numel())
            sp.lengths = ctypes.cast(ctypes.c_void_p(int(device_lengths.data_ptr())), ctypes.POINTER(ctypes.c_int32))
            keep.append(device_lengths)
        if device_pos0 is not None:
            sp.dev_pos0 = int(device_pos0.data_ptr())
            keep.append(device_pos0)
        sp._keep = keep
        return sp
    if lengths is not None:
        arr = (ctypes.c_int32 * len(lengths))(*[int(x) for x in lengths])
        sp.n_lengths = len(lengths)
        sp.lengths = ctypes.cast(arr, ctypes.POINTER(ctypes.c_int32))
        sp._keep = arr   # the array lives as long as the spec
    return sp


class MxfaError(RuntimeError):
    def __init__(self, status: int, detail: str):
        super().__init__(f"mxfa status {status} ({status_string(status)}): {detail}")
        self.status = status
        self.detail = detail


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"libmxfa.so not built: {LIB_PATH} (run `make -C acestep.cpp_amd`)")
    # torch ships its own HIP runtime (torch/lib/libamdhip64.so, soname
    # libamdhip64.so.7) and loads it by path.  It must be in the process
    # before libmxfa.so, whose libamdhip64.so.7 dependency then resolves to
    # it: loaded the other way round, the process ends up with two HIP
    # runtimes (ROCm's and torch's) and torch's device calls crash.
    import torch  # noqa: F401

    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER(MxfaTensor)
    L.mxfa_supports.argtypes = [P, P, P, P, ctypes.POINTER(MxfaParams), P]
    L.mxfa_supports.restype = ctypes.c_int
    L.mxfa_flash_attn_ext.argtypes = [P, P, P, P, ctypes.POINTER(MxfaParams), P, ctypes.c_void_p]
    L.mxfa_flash_attn_ext.restype = ctypes.c_int
    L.mxfa_flash_attn_ext_noalloc.argtypes = [P, P, P, P, ctypes.POINTER(MxfaParams), P, ctypes.c_void_p]
    L.mxfa_flash_attn_ext_noalloc.restype = ctypes.c_int
    L.mxfa_qk_norm_rope.argtypes = [P, P, P, P, P, P, ctypes.POINTER(MxfaNormRopeParams), P, P, P, P,
                                    ctypes.c_void_p]
    L.mxfa_qk_norm_rope.restype = ctypes.c_int
    L.mxfa_qk_norm_rope_supports.argtypes = [P, P, P, P, P, P, ctypes.POINTER(MxfaNormRopeParams), P, P, P, P]
    L.mxfa_qk_norm_rope_supports.restype = ctypes.c_int
    L.mxfa_reserve.argtypes = [P, P, P, P, ctypes.POINTER(MxfaParams), ctypes.c_void_p]
    L.mxfa_reserve.restype = ctypes.c_int
    L.mxfa_graph_begin.argtypes = [ctypes.c_void_p]
    L.mxfa_graph_begin.restype = ctypes.c_int
    L.mxfa_graph_end.argtypes = [ctypes.c_void_p]
    L.mxfa_graph_end.restype = ctypes.c_int
    L.mxfa_set_rows_supports.argtypes = [P, P, P]
    L.mxfa_set_rows_supports.restype = ctypes.c_int
    L.mxfa_set_rows.argtypes = [P, P, P, ctypes.c_void_p]
    L.mxfa_set_rows.restype = ctypes.c_int
    L.mxfa_supports_masked.argtypes = [P, P, P, ctypes.POINTER(MxfaMaskSpec), ctypes.POINTER(MxfaParams), P]
    L.mxfa_supports_masked.restype = ctypes.c_int
    L.mxfa_flash_attn_ext_masked.argtypes = [P, P, P, ctypes.POINTER(MxfaMaskSpec), ctypes.POINTER(MxfaParams), P,
                                             ctypes.c_void_p]
    L.mxfa_flash_attn_ext_masked.restype = ctypes.c_int
    L.mxfa_release.argtypes = []
    L.mxfa_release.restype = None
    L.mxfa_workspace_info.argtypes = [ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]
    L.mxfa_workspace_info.restype = ctypes.c_int
    L.mxfa_status_string.argtypes = [ctypes.c_int]
    L.mxfa_status_string.restype = ctypes.c_char_p
    L.mxfa_last_error.argtypes = []
    L.mxfa_last_error.restype = ctypes.c_char_p
    L.mxfa_version.argtypes = []
    L.mxfa_version.restype = ctypes.c_int
    L.mxfa_timing_enable.argtypes = [ctypes.c_int]
    L.mxfa_timing_enable.restype = None
    L.mxfa_timing_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(ctypes.c_int64)]
    L.mxfa_timing_read.restype = ctypes.c_int
    L.mxfa_timing_reset.argtypes = []
    L.mxfa_timing_reset.restype = None
    return L


lib = _load()


def status_string(status: int) -> str:
    return lib.mxfa_status_string(int(status)).decode()


def last_error() -> str:
    return lib.mxfa_last_error().decode()


def version() -> int:
    return int(lib.mxfa_version())


@dataclass
class DeviceView:
    """A ggml-style tensor view over device memory."""

    type: int
    ne: tuple
    nb: tuple
    ptr: int                     # device address of element (0,0,0,0)
    owner: object = None         # keeps the backing allocation alive

    def desc(self) -> MxfaTensor:
        t = MxfaTensor()
        t.type = int(self.type)
        for i in range(4):
            t.ne[i] = int(self.ne[i])
            t.nb[i] = int(self.nb[i])
        t.data = ctypes.c_void_p(int(self.ptr)) if self.ptr else None
        return t


def _descs(q, k, v, mask, dst):
    dq, dk, dv = q.desc(), k.desc(), v.desc()
    dm = mask.desc() if mask is not None else None
    dd = dst.desc() if dst is not None else None
    ref = lambda d: ctypes.byref(d) if d is not None else None  # noqa: E731
    return (dq, dk, dv, dm, dd), (ref(dq), ref(dk), ref(dv), ref(dm), ref(dd))


def make_params(scale: float, max_bias: float = 0.0, logit_softcap: float = 0.0,
                prec: int = PREC_F32) -> MxfaParams:
    p = MxfaParams()
    p.scale, p.max_bias, p.logit_softcap, p.prec = float(scale), float(max_bias), float(logit_softcap), int(prec)
    return p


def supports(q, k, v, mask, scale, max_bias=0.0, logit_softcap=0.0, prec=PREC_F32, dst=None) -> bool:
    """supports_op: True when flash_attn_ext handles this combination."""
    keep, refs = _descs(q, k, v, mask, dst)
    p = make_params(scale, max_bias, logit_softcap, prec)
    return bool(lib.mxfa_supports(refs[0], refs[1], refs[2], refs[3], ctypes.byref(p), refs[4]))


def flash_attn_ext(q, k, v, mask, scale, max_bias=0.0, logit_softcap=0.0, prec=PREC_F32,
                   dst: Optional[DeviceView] = None, stream: Optional[int] = None) -> DeviceView:
    """GGML_OP_FLASH_ATTN_EXT on the GPU.  Returns the F32 [DV, Nh, Sq, B]
    output view (allocated with torch when `dst` is None).  Asynchronous on
    `stream` (default: torch's current stream).  Raises MxfaError on failure.
    """
    import torch

    if dst is None:
        DV, Nh, Sq, B = int(v.ne[0]), int(q.ne[2]), int(q.ne[1]), int(q.ne[3])
        out = torch.empty((B, Sq, Nh, DV), dtype=torch.float32, device="cuda")
        dst = DeviceView(TYPE_F32, (DV, Nh, Sq, B), (4, 4 * DV, 4 * DV * Nh, 4 * DV * Nh * Sq),
                         out.data_ptr(), out)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    keep, refs = _descs(q, k, v, mask, dst)
    p = make_params(scale, max_bias, logit_softcap, prec)
    rc = lib.mxfa_flash_attn_ext(refs[0], refs[1], refs[2], refs[3], ctypes.byref(p), refs[4],
                                 ctypes.c_void_p(int(stream)))
    if rc != OK:
        raise MxfaError(rc, last_error())
    return dst


def flash_attn_ext_noalloc(q, k, v, mask, scale, max_bias=0.0, logit_softcap=0.0, prec=PREC_F32,
                           dst: Optional[DeviceView] = None, stream: Optional[int] = None) -> DeviceView:
    """flash_attn_ext through mxfa_flash_attn_ext_noalloc: the same kernels
    with the split partials, tickets and mask classes in the library's fixed
    per-GPU scratch (no device allocation by the engine; `dst` is allocated
    here with torch when None)."""
    import torch

    if dst is None:
        dst = _out_view(q, v)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    keep, refs = _descs(q, k, v, mask, dst)
    p = make_params(scale, max_bias, logit_softcap, prec)
    rc = lib.mxfa_flash_attn_ext_noalloc(refs[0], refs[1], refs[2], refs[3], ctypes.byref(p), refs[4],
                                         ctypes.c_void_p(int(stream)))
    if rc != OK:
        raise MxfaError(rc, last_error())
    return dst


def qk_norm_rope(q, k, v, q_norm, k_norm, positions, eps, freq_base, q_out, k_out, v_out, rows=None,
                 clamp_v=False, stream: Optional[int] = None) -> None:
    """The pre-attention work of a layer in one kernel (mxfa_qk_norm_rope):
    QK-RMSNorm, NEOX RoPE, 16-bit cast of Q/K/V, K/V written into their
    cache rows.  All arguments are DeviceViews (rows may be None).
    positions=None: no RoPE (DiT cross-attention), and k/v may hold their
    own number of tokens."""
    import torch

    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    ds = [t.desc() if t is not None else None for t in (q, k, v, q_norm, k_norm, positions, q_out, k_out, v_out)]
    dr = rows.desc() if rows is not None else None
    p = MxfaNormRopeParams()
    p.eps, p.freq_base, p.clamp_v = float(eps), float(freq_base), int(bool(clamp_v))
    refs = [ctypes.byref(d) if d is not None else None for d in ds]
    rc = lib.mxfa_qk_norm_rope(refs[0], refs[1], refs[2], refs[3], refs[4], refs[5], ctypes.byref(p), refs[6],
                               refs[7], refs[8], ctypes.byref(dr) if dr is not None else None,
                               ctypes.c_void_p(int(stream)))
    if rc != OK:
        raise MxfaError(rc, last_error())


def reserve(q, k, v, mask, scale, max_bias=0.0, logit_softcap=0.0, prec=PREC_F32, stream=None) -> None:
    """Grows the engine's workspace for this call's shapes without launching
    anything, so that the call can then be captured into a HIP graph."""
    import torch

    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    keep, refs = _descs(q, k, v, mask, None)
    p = make_params(scale, max_bias, logit_softcap, prec)
    rc = lib.mxfa_reserve(refs[0], refs[1], refs[2], refs[3], ctypes.byref(p), ctypes.c_void_p(int(stream)))
    if rc != OK:
        raise MxfaError(rc, last_error())


def graph_begin(stream=None) -> None:
    """Starts one graph's computation on `stream` (mxfa_graph_begin): until
    the next call, FA calls on the stream that share a dense mask (same data
    pointer, shape and strides, same Sq and Skv) classify it once."""
    import torch

    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    rc = lib.mxfa_graph_begin(ctypes.c_void_p(int(stream)))
    if rc != OK:
        raise MxfaError(rc, last_error())


def graph_end(stream=None) -> None:
    """Ends the graph begun on `stream` (mxfa_graph_end): FA calls on it
    classify their masks per call again."""
    import torch

    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    rc = lib.mxfa_graph_end(ctypes.c_void_p(int(stream)))
    if rc != OK:
        raise MxfaError(rc, last_error())


@contextlib.contextmanager
def graph(stream=None):
    """with mxfa.graph(stream): ... -- the FA calls inside share their
    masks' classification (mxfa_graph_begin / mxfa_graph_end)."""
    graph_begin(stream)
    try:
        yield
    finally:
        graph_end(stream)


def set_rows_supports(dst, src, rows) -> bool:
    """supports_op for GGML_OP_SET_ROWS (node = dst view, src[0] = src,
    src[1] = rows)."""
    dd, ds, dr = dst.desc(), src.desc(), rows.desc()
    return bool(lib.mxfa_set_rows_supports(ctypes.byref(dd), ctypes.byref(ds), ctypes.byref(dr)))


def set_rows(dst: DeviceView, src: DeviceView, rows: DeviceView, stream: Optional[int] = None) -> DeviceView:
    """GGML_OP_SET_ROWS on the GPU, as ggml_set_rows(ctx, dst, src, rows) in
    the reference's KV-cache write (src/qwen3-lm.h:453-454, :776-777): the F32
    rows of `src` are converted to dst's type and written, in place, to the
    rows of `dst` that `rows` (I64 / I32) names.  Asynchronous on `stream`
    (default: torch's current stream).  Returns `dst`; raises MxfaError."""
    import torch

    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    dd, ds, dr = dst.desc(), src.desc(), rows.desc()
    rc = lib.mxfa_set_rows(ctypes.byref(dd), ctypes.byref(ds), ctypes.byref(dr), ctypes.c_void_p(int(stream)))
    if rc != OK:
        raise MxfaError(rc, last_error())
    return dst


def _out_view(q, v):
    import torch

    DV, Nh, Sq, B = int(v.ne[0]), int(q.ne[2]), int(q.ne[1]), int(q.ne[3])
    out = torch.empty((B, Sq, Nh, DV), dtype=torch.float32, device="cuda")
    return DeviceView(TYPE_F32, (DV, Nh, Sq, B), (4, 4 * DV, 4 * DV * Nh, 4 * DV * Nh * Sq), out.data_ptr(), out)


def supports_masked(q, k, v, spec, scale, max_bias=0.0, logit_softcap=0.0, prec=PREC_F32, dst=None) -> bool:
    """supports_op for a structured-mask call."""
    keep, refs = _descs(q, k, v, None, dst)
    p = make_params(scale, max_bias, logit_softcap, prec)
    return bool(lib.mxfa_supports_masked(refs[0], refs[1], refs[2], ctypes.byref(spec), ctypes.byref(p), refs[4]))


def flash_attn_ext_masked(q, k, v, spec, scale, max_bias=0.0, logit_softcap=0.0, prec=PREC_F32,
                          dst: Optional[DeviceView] = None, stream: Optional[int] = None) -> DeviceView:
    """flash_attn_ext with the mask given as metadata (`mask_spec(...)`):
    the result equals flash_attn_ext with the equivalent dense F16 mask."""
    import torch

    if dst is None:
        dst = _out_view(q, v)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    keep, refs = _descs(q, k, v, None, dst)
    p = make_params(scale, max_bias, logit_softcap, prec)
    rc = lib.mxfa_flash_attn_ext_masked(refs[0], refs[1], refs[2], ctypes.byref(spec), ctypes.byref(p), refs[4],
                                        ctypes.c_void_p(int(stream)))
    if rc != OK:
        raise MxfaError(rc, last_error())
    return dst


def release() -> None:
    lib.mxfa_release()


def workspace_info():
    """(live workspace bytes, outgrown buffers kept for earlier captures)."""
    live = ctypes.c_int64(0)
    ret = ctypes.c_int64(0)
    rc = lib.mxfa_workspace_info(ctypes.byref(live), ctypes.byref(ret))
    if rc != OK:
        raise MxfaError(rc, last_error())
    return live.value, ret.value


def timing_enable(on=True) -> None:
    """Profiling aid.  on = True / 1: bracket every engine kernel launch with
    HIP events; on = n > 1: run every launch n times back to back inside one
    event pair (counted as n launches: the kernel's own duration, without an
    event pair per launch); False / 0: off."""
    n = int(on) if not isinstance(on, bool) else int(on)
    lib.mxfa_timing_enable(max(0, n))


def timing_read(kernel: str):
    """(total_ms, launches) of one kernel family since the last reset."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    rc = lib.mxfa_timing_read(kernel.encode(), ctypes.byref(ms), ctypes.byref(n))
    if rc != OK:
        raise MxfaError(rc, last_error())
    return ms.value, n.value


def timing_reset() -> None:
    lib.mxfa_timing_reset()


def upload(view, device="cuda") -> DeviceView:
    """Copy a host view (any object with type/ne/nb/buf/offset) to the device,
    keeping its strides: the whole backing buffer is copied."""
    import numpy as np
    import torch

    buf = np.ascontiguousarray(view.buf).view(np.uint8).reshape(-1)
    t = torch.from_numpy(buf).to(device)
    return DeviceView(view.type, tuple(view.ne), tuple(view.nb), t.data_ptr() + int(view.offset), t)


def output_tensor(dst: DeviceView):
    """The torch tensor [B, Sq, Nh, DV] behind an output view."""
    return dst.owner
