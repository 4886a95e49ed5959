"""The CPU oracle against the reference's numpy golden model (golden/model.py).

The fixtures (tests/golden/numpy_*; written by tests/golden/make_golden_numpy.py
from the reference itself) pin what no compiled reference header can: the
golden's fp32 results in W8A16 (ACT_INT8 = False) and the W8A8 composition --
where model.py applies _qa (model.py:143, 191, 200, 230, 234, 237) and what
each GEMV computes from the quantised activation.

Per stage (identical inputs at every quantisation point):
  * act-quant: the oracle's (q, s) equal the golden's _qa codes and scale bit for bit;
  * every projection: int32 accumulators equal the int64 brute force, outputs within
    rtol 1e-4 (of the sum of |terms|) / atol 1e-5 elementwise of the golden's
    fake-quant BLAS product;
  * each mixer's fp32 path up to its last _qa (gated DeltaNet state and output, attention
    context, SwiGLU activation), read through a probe output projection (rows of the
    identity with unit scales): fp32 within tolerance (W8A16), int8 codes equal except
    at near-ties (W8A8);
  * the mixers' outputs, updated states and new cache rows (W8A16; state and cache rows
    also W8A8).
End to end: the oracle's decode (W8A16 and W8A8), teacher-forced on the golden's
token stream, meets golden_numpy.StreamCheck: its logits are as close to the
golden's as the golden's own are under another fp32 summation order.
"""
import os

import numpy as np
import pytest

import golden_numpy as gn
from conftest import assert_bitwise, assert_close

HAVE = all(os.path.exists(gn.stages_path(m)) for m in ("w8a16", "w8a8"))
pytestmark = pytest.mark.skipif(not HAVE, reason="numpy golden fixtures not generated")


def p(a):
    return a.ctypes.data


class Layer:
    """Host tensors of layer 0 (DeltaNet + MLP) and layer 3 (attention) as oracle views."""

    def __init__(self, orc, blob, entries):
        self.orc, self.blob, self.e = orc, blob, entries
        self.keep = []

    def i8(self, name):
        qw, s = gn.fake_quant_weights(self.blob, self.e[name])
        return qw, s

    def t(self, name):
        e = self.e[name]
        if e.dtype == 1:
            qw, s = self.i8(name)
            return self.orc.tensor_i8(qw, s)
        a = self.f32(name).reshape(e.out, e.in_)
        self.keep.append(a)
        return self.orc.tensor_f32(a)

    def f32(self, name):
        e = self.e[name]
        return self.blob[e.off:e.off + e.nbytes].view(np.float32)

    def probe(self, rows, in_dim, first):
        w, s, n = gn.probe_rows(rows, in_dim, first)
        self.keep += [w, s]
        return self.orc.tensor_i8(w, s), n


@pytest.fixture(scope="module")
def L(orc, blob, entries):
    return Layer(orc, blob, entries)


DN = "layers.0.linear_attn."
AT = "layers.3.self_attn."
ML = "layers.0.mlp."


def run_deltanet(orc, L, inp, mode, out_w=None):
    out = np.empty(1024, np.float32)
    rec, conv = inp["dn_rec"].copy(), inp["dn_conv"].copy()
    orc.lib().or_deltanet_layer(p(out), p(inp["dn_x"]), L.t(DN + "in_proj_qkv.weight"), L.t(DN + "in_proj_z.weight"),
                                L.t(DN + "in_proj_b.weight"), L.t(DN + "in_proj_a.weight"),
                                p(L.f32(DN + "conv1d.weight")), p(L.f32(DN + "A_log")), p(L.f32(DN + "dt_bias")),
                                p(L.f32(DN + "norm.weight")), out_w or L.t(DN + "out_proj.weight"), p(rec), p(conv),
                                mode, orc.ORDER_REF)
    return out, rec, conv


def run_attention(orc, L, inp, mode, out_w=None):
    T = gn.ATTN_T
    kc = np.zeros((T + 1, 512), np.float32)
    vc = np.zeros((T + 1, 512), np.float32)
    kc[:T] = inp["at_kc"].reshape(T, 512)
    vc[:T] = inp["at_vc"].reshape(T, 512)
    out = np.empty(1024, np.float32)
    orc.lib().or_attention_layer(p(out), p(inp["at_x"]), L.t(AT + "q_proj.weight"), L.t(AT + "k_proj.weight"),
                                 L.t(AT + "v_proj.weight"), out_w or L.t(AT + "o_proj.weight"),
                                 p(L.f32(AT + "q_norm.weight")), p(L.f32(AT + "k_norm.weight")), gn.ATTN_POS,
                                 p(kc), p(vc), T, mode, orc.ORDER_REF)
    return out, kc[T], vc[T]


def run_mlp(orc, L, inp, mode, out_w=None):
    out = np.empty(1024, np.float32)
    orc.lib().or_mlp_layer(p(out), p(inp["ml_x"]), L.t(ML + "gate_proj.weight"), L.t(ML + "up_proj.weight"),
                           out_w or L.t(ML + "down_proj.weight"), mode, orc.ORDER_REF)
    return out


def probed(run, L, in_dim):
    """The input vector of a mixer's output projection, read through probe projections."""
    parts = []
    for first in range(0, in_dim, 1024):
        w, n = L.probe(1024, in_dim, first)
        parts.append(run(w)[:n])
    return np.concatenate(parts)


def codes_of(y):
    """int8 codes from a W8A8 probe output y = float(code) * sx (|code| <= 127, the amax code = 127)."""
    sx = np.abs(y).max() / 127.0
    return np.rint(y / sx).astype(np.int32)


# ---------------------------------------------------------------- W8A16

def test_w8a16_projections(orc, L):
    fx, inp = gn.load_stages("w8a16")
    cases = [(DN + "in_proj_qkv.weight", inp["dn_x"], fx["dn_in_proj_qkv"]),
             (DN + "in_proj_z.weight", inp["dn_x"], fx["dn_in_proj_z"]),
             (DN + "out_proj.weight", fx["dn_qa1_in"], fx["dn_out_proj"]),
             (AT + "q_proj.weight", inp["at_x"], fx["at_q_proj"]),
             (AT + "k_proj.weight", inp["at_x"], fx["at_k_proj"]),
             (AT + "v_proj.weight", inp["at_x"], fx["at_v_proj"]),
             (AT + "o_proj.weight", fx["at_qa1_in"], fx["at_o_proj"]),
             (ML + "gate_proj.weight", inp["ml_x"], fx["ml_gate_proj"]),
             (ML + "up_proj.weight", inp["ml_x"], fx["ml_up_proj"]),
             (ML + "down_proj.weight", fx["ml_qa1_in"], fx["ml_down_proj"])]
    keys = ["dn_in_proj_qkv", "dn_in_proj_z", "dn_out_proj", "at_q_proj", "at_k_proj", "at_v_proj", "at_o_proj",
            "ml_gate_proj", "ml_up_proj", "ml_down_proj"]
    for (name, x, exp), key in zip(cases, keys):
        qw, s = L.i8(name)
        y = np.empty(qw.shape[0], np.float32)
        x = np.ascontiguousarray(x, np.float32)
        orc.lib().or_gemv_i8(p(y), p(qw), p(s), p(x), qw.shape[0], qw.shape[1])
        gn.assert_stage(y, exp, key, gn.dot_scale(qw, s, x), what=name)
    for name, key in ((DN + "in_proj_b.weight", "dn_in_proj_b"), (DN + "in_proj_a.weight", "dn_in_proj_a")):
        w = L.f32(name)
        y = np.empty(16, np.float32)
        orc.lib().or_gemv_f32(p(y), p(w), p(inp["dn_x"]), 16, 1024)
        gn.assert_stage(y, fx[key], key, np.abs(w.reshape(16, 1024).astype(np.float64)) @ np.abs(inp["dn_x"]),
                        what=name)


def check_conv(conv, fx, inp, L, x=None, mode="w8a16"):
    """conv history after the step (conv1d.hpp:22-36, model.py:153-154): columns 1..3 shifted
    down exactly, the new pre-conv sample (the qkv projection) in column 3."""
    assert_bitwise(conv[:, :3], fx["dn_conv_out"][:, :3], "conv history (shifted columns)")
    qw, sw = L.i8(DN + "in_proj_qkv.weight")
    x = inp["dn_x"] if x is None else x
    if mode == "w8a16":
        gn.assert_stage(conv[:, 3], fx["dn_conv_out"][:, 3], "dn_conv_out[:,3]", None, what="conv history (new column)")
    else:
        gn.assert_close_dot(conv[:, 3], fx["dn_conv_out"][:, 3], gn.dot_scale(qw, sw, x),
                            what="conv history (new column)")


def test_w8a16_deltanet(orc, L):
    fx, inp = gn.load_stages("w8a16")
    out, rec, conv = run_deltanet(orc, L, inp, orc.W8A16)
    qw, sw = L.i8(DN + "out_proj.weight")
    gn.assert_stage(out, fx["dn_out"], "dn_out", gn.dot_scale(qw, sw, fx["dn_qa1_in"]), what="deltanet out")
    assert_close(rec[gn.S_HEADS], fx["dn_S_out"], gn.RTOL, gn.ATOL, what="recurrent state")
    check_conv(conv, fx, inp, L)
    o = probed(lambda w: run_deltanet(orc, L, inp, orc.W8A16, w)[0], L, 2048)
    assert_close(o, fx["dn_qa1_in"], gn.RTOL, gn.ATOL, what="gated-norm output (out_proj input)")


def test_w8a16_attention(orc, L):
    fx, inp = gn.load_stages("w8a16")
    out, k_new, v_new = run_attention(orc, L, inp, orc.W8A16)
    qw, sw = L.i8(AT + "o_proj.weight")
    gn.assert_stage(out, fx["at_out"], "at_out", gn.dot_scale(qw, sw, fx["at_qa1_in"]), what="attention out")
    assert_close(k_new, fx["at_k_new"].reshape(-1), gn.RTOL, gn.ATOL, what="new K row")
    assert_close(v_new, fx["at_v_new"].reshape(-1), gn.RTOL, gn.ATOL, what="new V row")
    og = probed(lambda w: run_attention(orc, L, inp, orc.W8A16, w)[0], L, 2048)
    assert_close(og, fx["at_qa1_in"], gn.RTOL, gn.ATOL, what="gated context (o_proj input)")


def test_w8a16_mlp(orc, L):
    fx, inp = gn.load_stages("w8a16")
    qw, sw = L.i8(ML + "down_proj.weight")
    gn.assert_stage(run_mlp(orc, L, inp, orc.W8A16), fx["ml_out"], "ml_out", gn.dot_scale(qw, sw, fx["ml_qa1_in"]),
                    what="mlp out")
    act = probed(lambda w: run_mlp(orc, L, inp, orc.W8A16, w), L, 3584)
    gn.assert_stage(act, fx["ml_qa1_in"], "ml_qa1_in", None, what="SwiGLU activation (down input)")


# ---------------------------------------------------------------- W8A8

QA_POINTS = ("dn_qa0", "dn_qa1", "at_qa0", "at_qa1", "ml_qa0", "ml_qa1")


def test_w8a8_act_quant(orc):
    """or_quant_act on the golden's _qa inputs: codes and scale bit for bit (model.py:37-45)."""
    fx, _ = gn.load_stages("w8a8")
    for k in QA_POINTS:
        x = np.ascontiguousarray(fx[k + "_in"], np.float32)
        qv = np.empty(x.size, np.int8)
        s = np.empty(1, np.float32)
        orc.lib().or_quant_act(p(qv), p(s), p(x), x.size)
        assert np.array_equal(qv, fx[k + "_q"]), k
        assert_bitwise(s, np.atleast_1d(fx[k + "_s"]), k + " scale")


def w8a8_cases(fx):
    return [(DN + "in_proj_qkv.weight", "dn_qa0", fx["dn_in_proj_qkv"]),
            (DN + "in_proj_z.weight", "dn_qa0", fx["dn_in_proj_z"]),
            (DN + "out_proj.weight", "dn_qa1", fx["dn_out_proj"]),
            (AT + "q_proj.weight", "at_qa0", fx["at_q_proj"]),
            (AT + "k_proj.weight", "at_qa0", fx["at_k_proj"]),
            (AT + "v_proj.weight", "at_qa0", fx["at_v_proj"]),
            (AT + "o_proj.weight", "at_qa1", fx["at_o_proj"]),
            (ML + "gate_proj.weight", "ml_qa0", fx["ml_gate_proj"]),
            (ML + "up_proj.weight", "ml_qa0", fx["ml_up_proj"]),
            (ML + "down_proj.weight", "ml_qa1", fx["ml_down_proj"])]


def test_w8a8_projections(orc, L):
    """Golden codes in: exact int32 accumulators; float(acc)*sx*sw within tolerance of the
    golden's (q_w*s_w) @ (q_x*s_x) (export_gemv_tv.py:49-50 vs model.py:144-147)."""
    fx, _ = gn.load_stages("w8a8")
    for name, qa, exp in w8a8_cases(fx):
        qw, sw = L.i8(name)
        xq = np.ascontiguousarray(fx[qa + "_q"])
        y = np.empty(qw.shape[0], np.float32)
        acc = np.empty(qw.shape[0], np.int32)
        orc.lib().or_gemv_w8a8(p(y), p(acc), p(qw), p(sw), p(xq), float(fx[qa + "_s"]), qw.shape[0], qw.shape[1])
        brute = qw.astype(np.int64) @ xq.astype(np.int64)
        assert np.array_equal(acc.astype(np.int64), brute), name
        gn.assert_close_dot(y, exp, gn.dot_scale(qw, sw, xq.astype(np.float64) * float(fx[qa + "_s"])), what=name)
    xq = fx["dn_qa0_q"].astype(np.float32) * np.float32(fx["dn_qa0_s"])   # the gates take q*s (model.py:146-147)
    for name, key in ((DN + "in_proj_b.weight", "dn_in_proj_b"), (DN + "in_proj_a.weight", "dn_in_proj_a")):
        y = np.empty(16, np.float32)
        w = L.f32(name)
        orc.lib().or_gemv_f32(p(y), p(w), p(xq), 16, 1024)
        gn.assert_close_dot(y, fx[key], np.abs(w.reshape(16, 1024).astype(np.float64)) @ np.abs(xq), what=name)


def check_codes(y, fx, qa, what):
    ok, nd, nt = gn.codes_match(codes_of(y), fx[qa + "_q"], fx[qa + "_in"], fx[qa + "_s"])
    assert ok, f"{what}: {nd} codes differ outside the {nt} near-ties"


def test_w8a8_deltanet(orc, L):
    fx, inp = gn.load_stages("w8a8")
    _, rec, conv = run_deltanet(orc, L, inp, orc.W8A8)
    assert_close(rec[gn.S_HEADS], fx["dn_S_out"], gn.RTOL, gn.ATOL, what="recurrent state")
    check_conv(conv, fx, inp, L, fx["dn_qa0_q"].astype(np.float64) * float(fx["dn_qa0_s"]), mode="w8a8")
    y = probed(lambda w: run_deltanet(orc, L, inp, orc.W8A8, w)[0], L, 2048)
    check_codes(y, fx, "dn_qa1", "out_proj input codes")


def test_w8a8_attention(orc, L):
    fx, inp = gn.load_stages("w8a8")
    _, k_new, v_new = run_attention(orc, L, inp, orc.W8A8)
    assert_close(k_new, fx["at_k_new"].reshape(-1), gn.RTOL, gn.ATOL, what="new K row")
    assert_close(v_new, fx["at_v_new"].reshape(-1), gn.RTOL, gn.ATOL, what="new V row")
    y = probed(lambda w: run_attention(orc, L, inp, orc.W8A8, w)[0], L, 2048)
    check_codes(y, fx, "at_qa1", "o_proj input codes")


def test_w8a8_mlp(orc, L):
    fx, inp = gn.load_stages("w8a8")
    y = probed(lambda w: run_mlp(orc, L, inp, orc.W8A8, w), L, 3584)
    check_codes(y, fx, "ml_qa1", "down input codes")


# ---------------------------------------------------------------- whole decode

@pytest.mark.skipif(not os.path.exists(gn.stream_path("w8a8")), reason="golden stream not generated")
@pytest.mark.parametrize("mode", ["w8a16", "w8a8"])
def test_teacher_forced_stream(orc, blob, idx, mode):
    """The oracle's decode in the reference order, fed the golden's own token stream (the 64
    prompt ids and the first 64 greedy ones), against golden_numpy.StreamCheck."""
    g = gn.load_stream(mode)
    n = g["n_prompt"] + 64
    chk = gn.StreamCheck(g, n)
    m = orc.Model(blob, idx, max_ctx=n)
    try:
        for i in range(n):
            am, lg = m.decode_token(g["fed"][i], mode=orc.W8A8 if mode == "w8a8" else orc.W8A16,
                                    order=orc.ORDER_REF, want_logits=True)
            chk.step(i, am, lg)
        print(mode, chk.finish())
    finally:
        m.close()


@pytest.mark.skipif(not os.path.exists(gn.stream_path("w8a8")), reason="golden stream not generated")
@pytest.mark.parametrize("mode", ["w8a16", "w8a8"])
def test_numpy_restatement_equals_golden(blob, entries, mode):
    """oracle/numpy_golden.py (bench.py's CPU port of golden/model.py) reproduces the golden's
    logits bit for bit on the first steps of its stream (same numpy operations, same order)."""
    import oracle.numpy_golden as ng

    g = gn.load_stream(mode)
    m = ng.Golden(blob, entries, act_int8=mode == "w8a8")
    for i in range(12):
        lg = m.decode_step(g["fed"][i])
        assert int(np.argmax(lg)) == g["argmax"][i], f"step {i}"
        assert_bitwise(lg[g["top8_ids"][i]], np.array(g["top8_vals"][i], np.float32), f"top-8 logits step {i}")
