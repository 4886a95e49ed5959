"""Host-side mirror of the reference decode datapath's operator interface.

The reference (allthingssecurity/qwen_fpga) exposes its decode datapath as HLS
C++ functions in ``namespace qwen`` (hls/src/*.hpp) plus the ``qwen_top`` decode
top and the ``run_hls`` CLI.  This module binds the MI355X C ABI
(``include/qh_decode.h``, implemented in ``libqh.so``) with ctypes and keeps the
same operator names and argument order:

    gemv_i8(y, w, scale, x, out, in)            hls/src/gemv.hpp:28
    rmsnorm(y, x, w, n, eps)                    hls/src/norm.hpp:13
    deltanet_layer(out, x, qkv_w, ...)          hls/src/deltanet.hpp:141
    Engine.decode_token(tok, want_logits)       hls/src/qwen_synth.hpp:39 qwen_top
    ...

Array arguments are torch tensors already on the GPU (``device="cuda"``); only
their data pointers cross the boundary.  ``Tensor`` mirrors the reference's
``qwen::Tensor`` view (types.hpp:51-56).  A non-zero status from the library is
raised as ``QHError``.  There is no CPU fallback: importing the ops without the
built library raises.
"""
from __future__ import annotations

import ctypes
import os
import re
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqh.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "qh_decode.h")

HIDDEN, N_LAYERS, INTER, VOCAB = 1024, 24, 3584, 248320
LH, LK, LV, CONV_DIM, CONV_K, Z_DIM = 16, 128, 128, 6144, 4, 2048
NH, NKV, HD, Q_PROJ, KV_PROJ, ROPE_DIM = 8, 2, 256, 4096, 512, 64
EPS = 1e-6
MODE_W8A16, MODE_W8A8 = 0, 1

QH_OK, QH_EINVAL, QH_ERANGE, QH_EIO, QH_EFORMAT, QH_ENOMEM, QH_ESTATE, QH_EDEVICE = 0, -1, -2, -3, -4, -5, -6, -7
EXEC_PERSISTENT, EXEC_GRAPH = 0, 1


class QHError(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        self.status = status
        msg = _lib().qh_strerror(status).decode() if _LIB is not None else str(status)
        super().__init__(f"{what}: status {status} ({msg})" if what else f"status {status} ({msg})")


class Tensor(ctypes.Structure):
    """qwen::Tensor (hls/src/types.hpp:51-56): int8 payload + per-row scales, or fp32."""

    _fields_ = [
        ("w_i8", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("w_f32", ctypes.c_void_p),
        ("out", ctypes.c_int),
        ("in_", ctypes.c_int),
    ]

    @staticmethod
    def i8(w, scale) -> "Tensor":
        out, inn = int(w.shape[0]), int(w.shape[1])
        _dev(w, "i8", out * inn, "Tensor.i8 w")
        _dev(scale, "f32", out, "Tensor.i8 scale")
        return Tensor(_ptr(w), _ptr(scale), None, out, inn)

    @staticmethod
    def f32(w) -> "Tensor":
        out, inn = int(w.shape[0]), int(w.shape[1])
        _dev(w, "f32", out * inn, "Tensor.f32 w")
        return Tensor(None, None, _ptr(w), out, inn)


_LIB: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return LIB_PATH


def _lib() -> ctypes.CDLL:
    """Load libqh.so (built by __graft_entry__.build()); fail loudly if absent."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
        # One HIP runtime per process.  torch ships its own libamdhip64 (and HSA
        # runtime) under the same soname that libqh.so needs: loaded first, it
        # satisfies libqh's dependency.  Loaded after libqh, it maps a second
        # runtime beside /opt/rocm's, and the one initialised second sees no
        # device.  So when torch is importable it is loaded before libqh.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = ctypes.CDLL(LIB_PATH)
        lib.qh_strerror.restype = ctypes.c_char_p
        lib.qh_blob_size.restype = ctypes.c_size_t
        lib.qh_layout_idx_text.restype = ctypes.c_size_t
        lib.qh_layout_idx_text.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
        lib.qh_synth_blob.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64]
        for n in ("qh_synth_fill_uniform", "qh_synth_fill_normal"):
            getattr(lib, n).argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_float,
                                        ctypes.c_float]
        lib.qh_synth_fill_i8.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64]
        lib.qh_engine_stream.restype = ctypes.c_void_p
        lib.qh_engine_stream.argtypes = [ctypes.c_void_p]
        lib.qh_engine_last_launch_ms.restype = ctypes.c_float
        lib.qh_engine_last_launch_ms.argtypes = [ctypes.c_void_p]
        lib.qh_engine_device_ptr.restype = ctypes.c_void_p
        lib.qh_engine_device_ptr.argtypes = [ctypes.c_void_p, ctypes.c_int]
        _LIB = lib
    return _LIB


def header_functions() -> list:
    """Names of every function the C ABI header declares."""
    text = open(HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qh_[a-z0-9_]+)\s*\(", text)))


def _ptr(t) -> Optional[int]:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    if isinstance(t, np.ndarray):
        return t.ctypes.data
    raise TypeError(f"cannot pass {type(t)} as a pointer")


_DTYPES = {"f32": ("float32",), "i8": ("int8",), "i32": ("int32",), "bf16": ("bfloat16", "int16", "uint16")}


def _dev(t, kind: str, n: int, what: str):
    """Checks a device-pointer argument before it reaches a kernel: a contiguous torch CUDA
    tensor of the expected dtype holding at least n elements (a host array or a short buffer
    would otherwise become a GPU page fault).  A _Ptr is a raw device address the caller
    vouches for and is passed unchecked; sizes and NULL pointers are the C ABI's to reject."""
    if t is None or isinstance(t, _Ptr):   # NULL: the C ABI rejects it where it is required
        return t
    if not hasattr(t, "is_cuda"):
        raise TypeError(f"{what}: expected a torch CUDA tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise TypeError(f"{what}: tensor is on {t.device}, not on the GPU")
    if str(t.dtype).rsplit(".", 1)[-1] not in _DTYPES[kind]:
        raise TypeError(f"{what}: dtype {t.dtype}, expected {'/'.join(_DTYPES[kind])}")
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor is not contiguous")
    if t.numel() < n:
        raise ValueError(f"{what}: {t.numel()} elements, the call needs {n}")
    return t


def _stream(stream) -> Optional[int]:
    if stream is None:
        try:
            import torch
            return torch.cuda.current_stream().cuda_stream or None
        except Exception:
            return None
    return getattr(stream, "cuda_stream", stream)


def _check(status: int, what: str) -> None:
    if status != QH_OK:
        raise QHError(status, what)


class _Ptr(int):
    """An already-resolved raw pointer (e.g. a stream handle); 0 means NULL."""

    def __new__(cls, v):
        return int.__new__(cls, v or 0)


def _call(name: str, *args) -> None:
    """Call a C ABI function: ints -> int, floats -> float, Tensor -> struct
    pointer, torch/numpy arrays -> data pointer, None -> NULL."""
    fn = getattr(_lib(), name)
    conv = []
    for a in args:
        if isinstance(a, _Ptr):
            conv.append(ctypes.c_void_p(int(a)) if int(a) else None)
        elif a is None:
            conv.append(None)
        elif isinstance(a, float):
            conv.append(ctypes.c_float(a))
        elif isinstance(a, Tensor):
            conv.append(ctypes.byref(a))
        elif isinstance(a, (bool, np.bool_, int, np.integer)):
            conv.append(ctypes.c_int(int(a)))
        else:
            conv.append(ctypes.c_void_p(_ptr(a)))
    _check(fn(*conv), name)


# ---------------------------------------------------------------- op level
# Integer sizes are passed as plain ints; pointers must be contiguous torch CUDA
# tensors of the right dtype and size (checked by _dev before the call).

def gemv_i8(y, w, scale, x, out: int, in_: int, stream=None):
    _call("qh_gemv_i8", _dev(y, "f32", out, "y"), _dev(w, "i8", out * in_, "w"), _dev(scale, "f32", out, "scale"),
          _dev(x, "f32", in_, "x"), out, in_, _Ptr(_stream(stream)))


def gemv_f32(y, w, x, out: int, in_: int, stream=None):
    _call("qh_gemv_f32", _dev(y, "f32", out, "y"), _dev(w, "f32", out * in_, "w"), _dev(x, "f32", in_, "x"),
          out, in_, _Ptr(_stream(stream)))


def row_dot_i8(result, w, scale, h, row: int, in_: int, stream=None):
    _call("qh_row_dot_i8", _dev(result, "f32", 1, "result"), _dev(w, "i8", (row + 1) * in_, "w"),
          _dev(scale, "f32", row + 1, "scale"), _dev(h, "f32", in_, "h"), row, in_, _Ptr(_stream(stream)))


def embed_row(h, w, scale, tok: int, in_: int, stream=None):
    _call("qh_embed_row", _dev(h, "f32", in_, "h"), _dev(w, "i8", (tok + 1) * in_, "w"),
          _dev(scale, "f32", tok + 1, "scale"), tok, in_, _Ptr(_stream(stream)))


def rmsnorm(y, x, w, n: int, eps: float = EPS, stream=None):
    _call("qh_rmsnorm", _dev(y, "f32", n, "y"), _dev(x, "f32", n, "x"), _dev(w, "f32", n, "w"), n, float(eps),
          _Ptr(_stream(stream)))


def rmsnorm_gated(y, x, w, z, n: int, eps: float = EPS, stream=None):
    _call("qh_rmsnorm_gated", _dev(y, "f32", n, "y"), _dev(x, "f32", n, "x"), _dev(w, "f32", n, "w"),
          _dev(z, "f32", n, "z"), n, float(eps), _Ptr(_stream(stream)))


def conv1d_step(out, in_ch, state, weight, stream=None):
    _call("qh_conv1d_step", _dev(out, "f32", CONV_DIM, "out"), _dev(in_ch, "f32", CONV_DIM, "in_ch"),
          _dev(state, "f32", CONV_DIM * 4, "state"), _dev(weight, "f32", CONV_DIM * 4, "weight"),
          _Ptr(_stream(stream)))


def rope_cos_sin(pos: int, cos_o, sin_o, stream=None):
    _call("qh_rope_cos_sin", pos, _dev(cos_o, "f32", 64, "cos"), _dev(sin_o, "f32", 64, "sin"),
          _Ptr(_stream(stream)))


def apply_rope(x, cos_, sin_, stream=None):
    _call("qh_apply_rope", _dev(x, "f32", 256, "x"), _dev(cos_, "f32", 64, "cos"), _dev(sin_, "f32", 64, "sin"),
          _Ptr(_stream(stream)))


def l2norm(v, n: int, stream=None):
    _call("qh_l2norm", _dev(v, "f32", n, "v"), n, _Ptr(_stream(stream)))


def delta_rule_head(q, k, v, g: float, beta: float, S, out, stream=None):
    _call("qh_delta_rule_head", _dev(q, "f32", 128, "q"), _dev(k, "f32", 128, "k"), _dev(v, "f32", 128, "v"),
          float(g), float(beta), _dev(S, "f32", 128 * 128, "S"), _dev(out, "f32", 128, "out"),
          _Ptr(_stream(stream)))


def delta_rule_layer(q, k, v, g, beta, S, out, stream=None):
    _call("qh_delta_rule_layer", _dev(q, "f32", 2048, "q"), _dev(k, "f32", 2048, "k"), _dev(v, "f32", 2048, "v"),
          _dev(g, "f32", 16, "g"), _dev(beta, "f32", 16, "beta"), _dev(S, "f32", 16 * 128 * 128, "S"),
          _dev(out, "f32", 2048, "out"), _Ptr(_stream(stream)))


def deltanet_step_workspace() -> int:
    """Bytes of device scratch qh_deltanet_step takes from its caller."""
    f = _lib().qh_deltanet_step_workspace
    f.restype = ctypes.c_size_t
    return int(f())


def deltanet_step(out, qkv, z, b, a, conv_w, A_log, dt_bias, gate_norm_w, rec, conv_state, workspace,
                  stream=None):
    """The DeltaNet recurrent step between the projections (deltanet.hpp:154-179; config C2):
    conv + SiLU, gates, l2norm, delta rule, per-head gated RMSNorm.  `workspace` is a device
    tensor of at least deltanet_step_workspace() bytes (256-byte aligned); nothing is allocated."""
    if not getattr(workspace, "is_cuda", False) or not workspace.is_contiguous():
        raise TypeError("workspace: a contiguous tensor on the GPU")
    nbytes = workspace.numel() * workspace.element_size()
    fn = _lib().qh_deltanet_step
    _check(fn(*[ctypes.c_void_p(_ptr(t)) for t in (
        _dev(out, "f32", 2048, "out"), _dev(qkv, "f32", CONV_DIM, "qkv"), _dev(z, "f32", 2048, "z"),
        _dev(b, "f32", 16, "b"), _dev(a, "f32", 16, "a"), _dev(conv_w, "f32", CONV_DIM * 4, "conv_w"),
        _dev(A_log, "f32", 16, "A_log"), _dev(dt_bias, "f32", 16, "dt_bias"),
        _dev(gate_norm_w, "f32", 128, "gate_norm_w"), _dev(rec, "f32", 16 * 128 * 128, "rec"),
        _dev(conv_state, "f32", CONV_DIM * 4, "conv_state"), workspace)],
        ctypes.c_size_t(nbytes), ctypes.c_void_p(_stream(stream) or 0) if _stream(stream) else None),
        "qh_deltanet_step")


def deltanet_layer(out, x, qkv_w: Tensor, z_w: Tensor, b_w: Tensor, a_w: Tensor, conv_w, A_log, dt_bias,
                   gate_norm_w, out_w: Tensor, rec, conv_state, w8a8: bool = False, stream=None):
    _call("qh_deltanet_layer_w8a8" if w8a8 else "qh_deltanet_layer", _dev(out, "f32", HIDDEN, "out"),
          _dev(x, "f32", HIDDEN, "x"), qkv_w, z_w, b_w, a_w, _dev(conv_w, "f32", CONV_DIM * 4, "conv_w"),
          _dev(A_log, "f32", 16, "A_log"), _dev(dt_bias, "f32", 16, "dt_bias"),
          _dev(gate_norm_w, "f32", 128, "gate_norm_w"), out_w, _dev(rec, "f32", 16 * 128 * 128, "rec"),
          _dev(conv_state, "f32", CONV_DIM * 4, "conv_state"), _Ptr(_stream(stream)))


def attention_layer(out, x, q_w: Tensor, k_w: Tensor, v_w: Tensor, o_w: Tensor, q_norm, k_norm, pos: int,
                    kcache, vcache, T: int, w8a8: bool = False, stream=None):
    n_kv = (max(T, 0) + 1) * 512
    _call("qh_attention_layer_w8a8" if w8a8 else "qh_attention_layer", _dev(out, "f32", HIDDEN, "out"),
          _dev(x, "f32", HIDDEN, "x"), q_w, k_w, v_w, o_w, _dev(q_norm, "f32", 256, "q_norm"),
          _dev(k_norm, "f32", 256, "k_norm"), pos, _dev(kcache, "f32", n_kv, "kcache"),
          _dev(vcache, "f32", n_kv, "vcache"), T, _Ptr(_stream(stream)))


def attention_layer_noalloc(out, x, q_w: Tensor, k_w: Tensor, v_w: Tensor, o_w: Tensor, q_norm, k_norm, pos: int,
                            kcache, vcache, T: int, w8a8: bool = False, stream=None):
    """attention_layer without any device allocation (the library's static scratch; T + 1 <= 65536)."""
    n_kv = (max(T, 0) + 1) * 512
    _call("qh_attention_layer_noalloc", _dev(out, "f32", HIDDEN, "out"), _dev(x, "f32", HIDDEN, "x"), q_w, k_w,
          v_w, o_w, _dev(q_norm, "f32", 256, "q_norm"), _dev(k_norm, "f32", 256, "k_norm"), pos,
          _dev(kcache, "f32", n_kv, "kcache"), _dev(vcache, "f32", n_kv, "vcache"), T,
          MODE_W8A8 if w8a8 else MODE_W8A16, _Ptr(_stream(stream)))


def mlp_layer(out, x, gate_w: Tensor, up_w: Tensor, down_w: Tensor, w8a8: bool = False, stream=None):
    _call("qh_mlp_layer_w8a8" if w8a8 else "qh_mlp_layer", _dev(out, "f32", HIDDEN, "out"),
          _dev(x, "f32", HIDDEN, "x"), gate_w, up_w, down_w, _Ptr(_stream(stream)))


def quant_act(xq, sx, x, n: int, stream=None):
    _call("qh_quant_act", _dev(xq, "i8", n, "xq"), _dev(sx, "f32", 1, "sx"), _dev(x, "f32", n, "x"), n,
          _Ptr(_stream(stream)))


def gemv_i8_w8a8(y, acc, w, scale, xq, sx, out: int, in_: int, stream=None):
    _call("qh_gemv_i8_w8a8", _dev(y, "f32", out, "y"), _dev(acc, "i32", out, "acc"),
          _dev(w, "i8", out * in_, "w"), _dev(scale, "f32", out, "scale"), _dev(xq, "i8", in_, "xq"),
          _dev(sx, "f32", 1, "sx"), out, in_, _Ptr(_stream(stream)))


def matvec_i8(y_q, acc, w, mult, xq, out: int, in_: int, shift: int = 16, outw: int = 16, stream=None):
    """rtl/matvec_i8.sv: int32 acc = w @ xq, y_q = (acc*mult + 2^(shift-1)) >>> shift in outw bits."""
    _call("qh_matvec_i8", _dev(y_q, "i32", out, "y_q"), _dev(acc, "i32", out, "acc"),
          _dev(w, "i8", out * in_, "w"), _dev(mult, "i32", out, "mult"), _dev(xq, "i8", in_, "xq"), out, in_,
          shift, outw, _Ptr(_stream(stream)))


def dequant_mult(sx: float, sw, outq: int = 14, shift: int = 16) -> np.ndarray:
    """Host-side fixed-point multipliers llround(sx*sw[o]*2^(outq+shift)) (rtl/tb/sim_matvec.cpp:36-41)."""
    sw = np.ascontiguousarray(sw, dtype=np.float32)
    mult = np.empty(sw.size, np.int32)
    _call("qh_dequant_mult", mult, float(sx), sw, int(sw.size), outq, shift)
    return mult


def quant_rows(q, scale, w, rows: int, cols: int, stream=None):
    """golden/quant.py:43-49 quant_rows on the device: per row s = amax/127 (1 if 0),
    q = rint(w/s) clipped to +-127.  ``w`` is fp32 [rows, cols] or the raw bits of a
    bfloat16 tensor (torch.bfloat16 / int16 / uint16), widened exactly on the device;
    q is int8 [rows, cols], scale fp32 [rows].  A row with a non-finite value gets
    scale NaN and q = 0."""
    bits16 = str(getattr(w, "dtype", "")).rsplit(".", 1)[-1] in ("bfloat16", "int16", "uint16")
    _call("qh_quant_rows_bf16" if bits16 else "qh_quant_rows", _dev(q, "i8", rows * cols, "q"),
          _dev(scale, "f32", rows, "scale"), _dev(w, "bf16" if bits16 else "f32", rows * cols, "w"), rows, cols,
          _Ptr(_stream(stream)))


# ---------------------------------------------------------------- layout / synthetic weights

def blob_size() -> int:
    return int(_lib().qh_blob_size())


def idx_text() -> str:
    lib = _lib()
    n = lib.qh_layout_idx_text(None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    lib.qh_layout_idx_text(buf, n + 1)
    return buf.value.decode()


def synth_blob(seed: int) -> np.ndarray:
    """The seeded synthetic model in the packed pack_weights.py layout (host bytes)."""
    n = blob_size()
    blob = np.empty(n, dtype=np.uint8)
    _check(_lib().qh_synth_blob(blob.ctypes.data, n, ctypes.c_uint64(seed)), "qh_synth_blob")
    return blob


def synth_i8(n: int, key: int) -> np.ndarray:
    a = np.empty(n, dtype=np.int8)
    _check(_lib().qh_synth_fill_i8(a.ctypes.data, n, ctypes.c_uint64(key)), "qh_synth_fill_i8")
    return a


def synth_uniform(n: int, key: int, lo: float, hi: float) -> np.ndarray:
    a = np.empty(n, dtype=np.float32)
    _check(_lib().qh_synth_fill_uniform(a.ctypes.data, n, ctypes.c_uint64(key), lo, hi), "fill_uniform")
    return a


def synth_normal(n: int, key: int, mean: float, std: float) -> np.ndarray:
    a = np.empty(n, dtype=np.float32)
    _check(_lib().qh_synth_fill_normal(a.ctypes.data, n, ctypes.c_uint64(key), mean, std), "fill_normal")
    return a


@dataclass
class Entry:
    """One weights.idx line (emit_weight_index.py:13-22)."""
    name: str
    off: int
    nbytes: int
    dtype: int
    soff: int
    snbytes: int
    out: int
    in_: int


def parse_idx(text: str) -> dict:
    ents = {}
    for line in text.splitlines():
        f = line.split()
        if len(f) != 8:
            continue
        ents[f[0]] = Entry(f[0], int(f[1]), int(f[2]), int(f[3]), int(f[4]), int(f[5]), int(f[6]), int(f[7]))
    return ents


# ---------------------------------------------------------------- engine (qwen_top)

class Engine:
    """The decode top on the device: embed -> 24 layers -> final norm -> tied head.

    Mirrors ``qwen_top(blob, state, tok, logits)`` (hls/src/qwen_synth.hpp:39-92)
    with the ``DecodeState`` (hls/src/state.hpp:18-35) owned by the engine.
    """

    def __init__(self, blob=None, *, path: Optional[str] = None, idx: Optional[str] = None,
                 max_ctx: int = 1024, mode: int = MODE_W8A16):
        lib = _lib()
        h = ctypes.c_void_p()
        if path is not None:
            st = lib.qh_engine_create(path.encode(), idx.encode() if idx else None, ctypes.c_int(max_ctx),
                                      ctypes.byref(h))
        else:
            arr = np.ascontiguousarray(blob, dtype=np.uint8)
            st = lib.qh_engine_create_from_memory(ctypes.c_void_p(arr.ctypes.data), ctypes.c_size_t(arr.size),
                                                  idx.encode() if idx else None, ctypes.c_int(max_ctx),
                                                  ctypes.byref(h))
        _check(st, "qh_engine_create")
        self._h = h
        self.max_ctx = max_ctx
        self.set_mode(mode)

    def close(self):
        if getattr(self, "_h", None):
            _lib().qh_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def set_mode(self, mode: int):
        _check(_lib().qh_engine_set_mode(self._h, ctypes.c_int(mode)), "qh_engine_set_mode")
        self.mode = mode

    def reset(self):
        _check(_lib().qh_engine_reset(self._h), "qh_engine_reset")

    def set_exec(self, exec_kind: int):
        """EXEC_PERSISTENT (one cooperative launch per call) or EXEC_GRAPH (a graph per token)."""
        _check(_lib().qh_engine_set_exec(self._h, ctypes.c_int(exec_kind)), "qh_engine_set_exec")

    @property
    def exec_kind(self) -> int:
        return int(_lib().qh_engine_get_exec(self._h))

    @property
    def exec_fallbacks(self) -> int:
        """Cooperative launches refused so far (each switched the engine to EXEC_GRAPH)."""
        return int(_lib().qh_engine_exec_fallbacks(self._h))

    def head_grid(self, exec_kind: int) -> int:
        """Workgroups the LM head runs on under an executor (row batch 4 b + w on wave w of workgroup b)."""
        r = _lib().qh_engine_head_grid(self._h, ctypes.c_int(exec_kind))
        if r < 0:
            raise QHError(r, "qh_engine_head_grid")
        return r

    @property
    def pos(self) -> int:
        return int(_lib().qh_engine_pos(self._h))

    def decode_token(self, tok: int, want_logits: bool = False):
        """qwen_top: returns (argmax, logits or None)."""
        am = ctypes.c_int()
        logits = np.empty(VOCAB, dtype=np.float32) if want_logits else None
        _check(_lib().qh_decode_token(self._h, ctypes.c_int(tok),
                                      ctypes.c_void_p(logits.ctypes.data) if want_logits else None,
                                      ctypes.byref(am)), "qh_decode_token")
        return int(am.value), logits

    def generate(self, prompt: Sequence[int], n_new: int, eos: int = -1) -> list:
        """The run_hls loop (run_hls.cpp:56-66), token feedback on the device."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32))
        out = np.empty(max(n_new, 1), dtype=np.int32)
        n = ctypes.c_int()
        _check(_lib().qh_generate(self._h, ctypes.c_void_p(p.ctypes.data), ctypes.c_int(p.size),
                                  ctypes.c_int(n_new), ctypes.c_int(eos), ctypes.c_void_p(out.ctypes.data),
                                  ctypes.byref(n)), "qh_generate")
        return out[: n.value].tolist()

    def forward_layers(self, l0: int, l1: int, h) -> None:
        """Layers [l0, l1) on a device hidden vector h (torch, in place)."""
        _check(_lib().qh_engine_forward_layers(self._h, ctypes.c_int(l0), ctypes.c_int(l1),
                                               ctypes.c_void_p(_ptr(h))), "qh_engine_forward_layers")

    def profile(self, n_steps: int):
        """(mean step ms, mean LM-head kernel ms) over n_steps stream-launched steps."""
        st, hd = ctypes.c_float(), ctypes.c_float()
        _check(_lib().qh_engine_profile(self._h, ctypes.c_int(n_steps), ctypes.byref(st), ctypes.byref(hd)),
               "qh_engine_profile")
        return float(st.value), float(hd.value)

    @property
    def stream(self) -> int:
        return int(_lib().qh_engine_stream(self._h) or 0)

    def device_ptr(self, which: int) -> int:
        return int(_lib().qh_engine_device_ptr(self._h, ctypes.c_int(which)) or 0)

    @property
    def last_argmax(self) -> int:
        return int(_lib().qh_engine_last_argmax(self._h))

    @property
    def last_launch_ms(self) -> float:
        """Duration of the last persistent-kernel launch (HIP events on the engine stream)."""
        return float(_lib().qh_engine_last_launch_ms(self._h))
