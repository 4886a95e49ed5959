"""ctypes bindings of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker.  Two libraries:

* ``liboracle.so`` (oracle.c): the C restatement of the reference datapath in
  the reference's own loop order (``ORDER_REF``) and in the device order of the
  gfx950 kernels (``ORDER_DEV``), in W8A16 and W8A8 modes.
* ``_ref/libqref.so``: the reference's hls/src kernels compiled from the
  headers where they lie (built by oracle/Makefile when /root/reference is
  present; the built file travels with the tree).  ``ref()`` returns None when
  it has not been built.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(_HERE, "liboracle.so")
REF_PATH = os.path.join(_HERE, "_ref", "libqref.so")

ORDER_REF, ORDER_DEV = 0, 1
W8A16, W8A8 = 0, 1

P = ctypes.c_void_p
I = ctypes.c_int
F = ctypes.c_float


class OrTensor(ctypes.Structure):
    """or_tensor / the reference Tensor view (hls/src/types.hpp:51-56)."""
    _fields_ = [("w_i8", P), ("scale", P), ("w_f32", P), ("out", I), ("in_", I)]


def ptr(a) -> Optional[int]:
    if a is None:
        return None
    return a.ctypes.data


def tensor_i8(w: np.ndarray, s: np.ndarray) -> OrTensor:
    return OrTensor(w.ctypes.data, s.ctypes.data, None, w.shape[0], w.shape[1])


def tensor_f32(w: np.ndarray) -> OrTensor:
    return OrTensor(None, None, w.ctypes.data, w.shape[0], w.shape[1])


_OR = None
_REF = None


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args


def lib():
    global _OR
    if _OR is None:
        if not os.path.exists(ORACLE_PATH):
            raise ImportError(f"{ORACLE_PATH} not built (make -C oracle)")
        L = ctypes.CDLL(ORACLE_PATH)
        T = ctypes.POINTER(OrTensor)
        _sig(L, "or_set_threads", None, [I])
        for n in ("or_silu", "or_sigmoid", "or_softplus", "or_expf"):
            _sig(L, n, F, [F, I])
        _sig(L, "or_dev_expf", F, [F])
        _sig(L, "or_dev_log1pf", F, [F])
        _sig(L, "or_gemv_i8", None, [P, P, P, P, I, I])
        _sig(L, "or_gemv_f32", None, [P, P, P, I, I])
        _sig(L, "or_row_dot_i8", F, [P, P, P, I, I])
        _sig(L, "or_embed_row", None, [P, P, P, I, I])
        _sig(L, "or_rmsnorm", None, [P, P, P, I, F])
        _sig(L, "or_rmsnorm_gated", None, [P, P, P, P, I, F])
        _sig(L, "or_conv1d_step", None, [P, P, P, P])
        _sig(L, "or_rope_cos_sin", None, [I, P, P])
        _sig(L, "or_apply_rope", None, [P, P, P])
        _sig(L, "or_l2norm", None, [P, I])
        _sig(L, "or_delta_rule_head", None, [P, P, P, F, F, P, P])
        _sig(L, "or_delta_rule_layer", None, [P, P, P, P, P, P, P])
        _sig(L, "or_quant_act", None, [P, P, P, I])
        _sig(L, "or_quant_act_markstein", None, [P, P, P, I])
        _sig(L, "or_quant_rows", None, [P, P, P, I, I])
        _sig(L, "or_matvec_fixed", None, [P, P, P, P, P, I, I, I, I])
        _sig(L, "or_dev_gemv_i8", None, [P, P, P, P, I, I])
        _sig(L, "or_dev_gemv_f32", None, [P, P, P, I, I])
        _sig(L, "or_dev_rmsnorm", None, [P, P, P, I, F])
        _sig(L, "or_dev_rmsnorm_gated", None, [P, P, P, P, I, F])
        _sig(L, "or_dev_l2norm", None, [P, I])
        _sig(L, "or_dev_conv1d_step", None, [P, P, P, P])
        _sig(L, "or_dev_delta_rule_head", None, [P, P, P, F, F, P, P])
        _sig(L, "or_dev_delta_rule_layer", None, [P, P, P, P, P, P, P])
        _sig(L, "or_gemv_w8a8", None, [P, P, P, P, P, F, I, I])
        _sig(L, "or_gemv_acc_i64", None, [P, P, P, I, I])
        _sig(L, "or_deltanet_layer", None, [P, P, T, T, T, T, P, P, P, P, T, P, P, I, I])
        _sig(L, "or_deltanet_step", None, [P, P, P, P, P, P, P, P, P, P, P, I])
        _sig(L, "or_attention_layer", None, [P, P, T, T, T, T, P, P, I, P, P, I, I, I])
        _sig(L, "or_mlp_layer", None, [P, P, T, T, T, I, I])
        _sig(L, "or_model_new", P, [P, ctypes.c_char_p, I])
        _sig(L, "or_model_free", None, [P])
        _sig(L, "or_model_reset", None, [P])
        _sig(L, "or_decode_token", I, [P, I, P, I, I])
        _sig(L, "or_forward_layers", None, [P, I, I, P, I, I])
        _sig(L, "or_model_pos", I, [P])
        for n in ("or_model_rec", "or_model_conv", "or_model_kcache", "or_model_vcache"):
            _sig(L, n, P, [P])
        _OR = L
    return _OR



def quant_rows(w: np.ndarray):
    """quant.py:43-49 quant_rows of an fp32 [rows, cols] array: (int8 q, fp32 scale)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(rows, np.float32)
    lib().or_quant_rows(q.ctypes.data, s.ctypes.data, w.ctypes.data, rows, cols)
    return q, s


def matvec_fixed(w: np.ndarray, xq: np.ndarray, mult: np.ndarray, shift: int = 16, outw: int = 16):
    """rtl/matvec_i8.sv on int8 w [out, in], int8 xq [in], int32 mult [out]: (y_q int32, acc int32)."""
    w = np.ascontiguousarray(w, dtype=np.int8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    mult = np.ascontiguousarray(mult, dtype=np.int32)
    out, in_ = w.shape
    yq = np.empty(out, np.int32)
    acc = np.empty(out, np.int32)
    lib().or_matvec_fixed(yq.ctypes.data, acc.ctypes.data, w.ctypes.data, mult.ctypes.data, xq.ctypes.data, out,
                          in_, shift, outw)
    return yq, acc


_REF_O3 = None
REF_O3_PATH = os.path.join(_HERE, "_ref", "libqref_o3.so")


def ref(o3: bool = False):
    """The compiled reference kernels (the reference's csim flags, -O2; with o3, the same
    sources built -O3), or None if oracle/_ref was not built."""
    global _REF, _REF_O3
    if o3:
        if _REF_O3 is None and os.path.exists(REF_O3_PATH):
            _REF_O3 = _ref_sigs(ctypes.CDLL(REF_O3_PATH))
        return _REF_O3
    if _REF is None and os.path.exists(REF_PATH):
        _REF = _ref_sigs(ctypes.CDLL(REF_PATH))
    return _REF


def _ref_sigs(L):
    if True:
        T = ctypes.POINTER(OrTensor)
        _sig(L, "ref_gemv_i8", None, [P, P, P, P, I, I])
        _sig(L, "ref_gemv_f32", None, [P, P, P, I, I])
        _sig(L, "ref_row_dot_i8", F, [P, P, P, I, I])
        _sig(L, "ref_embed_row", None, [P, P, P, I, I])
        _sig(L, "ref_rmsnorm", None, [P, P, P, I, F])
        _sig(L, "ref_rmsnorm_gated", None, [P, P, P, P, I, F])
        for n in ("ref_silu", "ref_sigmoid", "ref_softplus"):
            _sig(L, n, F, [F])
        _sig(L, "ref_conv1d_step", None, [P, P, P, P])
        _sig(L, "ref_rope_cos_sin", None, [I, P, P])
        _sig(L, "ref_apply_rope", None, [P, P, P])
        _sig(L, "ref_l2norm", None, [P, I])
        _sig(L, "ref_delta_rule_head", None, [P, P, P, F, F, P, P])
        _sig(L, "ref_delta_rule_layer", None, [P, P, P, P, P, P, P])
        _sig(L, "ref_deltanet_layer", None, [P, P, T, T, T, T, P, P, P, P, T, P, P])
        _sig(L, "ref_attention_layer", None, [P, P, T, T, T, T, P, P, I, P, P, I])
        _sig(L, "ref_mlp_layer", None, [P, P, T, T, T])
        _sig(L, "ref_state_new", P, [])
        _sig(L, "ref_state_free", None, [P])
        _sig(L, "ref_state_reset", None, [P])
        _sig(L, "ref_state_pos", I, [P])
        _sig(L, "ref_state_rec", P, [P])
        _sig(L, "ref_state_conv", P, [P])
        _sig(L, "ref_state_kc", P, [P, I])
        _sig(L, "ref_state_vc", P, [P, I])
        _sig(L, "ref_qwen_top", I, [P, P, I, P])
        _sig(L, "ref_decode_token", I, [P, ctypes.c_char_p, P, I, P])
        _sig(L, "ref_deltanet_step", None, [P] * 11)
    return L


class Model:
    """or_model: the whole-model restatement over a packed blob (qwen_top)."""

    def __init__(self, blob: np.ndarray, idx_text: str, max_ctx: int = 1024):
        self._blob = blob   # keep alive
        self._h = lib().or_model_new(blob.ctypes.data, idx_text.encode(), max_ctx)
        if not self._h:
            raise MemoryError("or_model_new failed")
        self.max_ctx = max_ctx

    def close(self):
        if self._h:
            lib().or_model_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def reset(self):
        lib().or_model_reset(self._h)

    def decode_token(self, tok: int, mode: int = W8A16, order: int = ORDER_REF, want_logits: bool = False):
        lg = np.empty(248320, dtype=np.float32) if want_logits else None
        am = lib().or_decode_token(self._h, tok, ptr(lg), mode, order)
        return am, lg

    def forward_layers(self, l0: int, l1: int, h: np.ndarray, mode: int = W8A16, order: int = ORDER_REF):
        lib().or_forward_layers(self._h, l0, l1, h.ctypes.data, mode, order)

    @property
    def pos(self) -> int:
        return lib().or_model_pos(self._h)

    def rec(self) -> np.ndarray:
        p = lib().or_model_rec(self._h)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (18, 16, 128, 128))

    def conv(self) -> np.ndarray:
        p = lib().or_model_conv(self._h)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (18, 6144, 4))

    def kcache(self) -> np.ndarray:
        p = lib().or_model_kcache(self._h)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (6, self.max_ctx, 512))

    def vcache(self) -> np.ndarray:
        p = lib().or_model_vcache(self._h)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (6, self.max_ctx, 512))


class RefModel:
    """The compiled reference decode top (qwen_top over its DecodeState)."""

    def __init__(self, blob: np.ndarray):
        r = ref()
        if r is None:
            raise ImportError("oracle/_ref/libqref.so not built")
        self._blob = blob
        self._st = r.ref_state_new()

    def close(self):
        if self._st:
            ref().ref_state_free(self._st)
            self._st = None

    def __del__(self):
        self.close()

    def reset(self):
        ref().ref_state_reset(self._st)

    def qwen_top(self, tok: int, want_logits: bool = False):
        lg = np.empty(248320, dtype=np.float32) if want_logits else None
        return ref().ref_qwen_top(self._blob.ctypes.data, self._st, tok, ptr(lg)), lg

    def decode_token(self, idx_text: str, tok: int, want_logits: bool = False):
        lg = np.empty(248320, dtype=np.float32) if want_logits else None
        return ref().ref_decode_token(self._blob.ctypes.data, idx_text.encode(), self._st, tok, ptr(lg)), lg

    @property
    def pos(self) -> int:
        return ref().ref_state_pos(self._st)

    def rec(self) -> np.ndarray:
        p = ref().ref_state_rec(self._st)
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_float)), (18, 16, 128, 128))
