"""The HIP path against the reference's numpy golden model (golden/model.py).

The same per-stage checks as tests/test_golden_numpy.py (which pins the CPU
oracle), here through the C ABI on the MI355X -- every quantisation point fed
the golden's own int8 codes and scale:
  * qh_quant_act: codes and scale bit for bit at all six _qa points;
  * every projection (qh_gemv_i8 / qh_gemv_i8_w8a8 / qh_gemv_f32): int32
    accumulators exact (int64 brute force), outputs within rtol 1e-4 of the sum
    of |terms| / atol 1e-5 of the golden's fake-quant BLAS product;
  * the three layer ops: W8A16 outputs, updated DeltaNet state, conv history,
    new K/V rows; each mixer's last _qa input read through a probe output
    projection (fp32 within tolerance, W8A8 codes exact except at near-ties).
End to end, on the decode engine with both executors:
  * W8A16 and W8A8 teacher-forced on the golden's 576-token stream (64 prompt +
    512 greedy): golden_numpy.StreamCheck -- the logits as close to the golden's
    as the golden's own are under another fp32 summation order;
  * free-running greedy: the first divergence from the golden's stream, if any,
    falls on a step whose golden margin is within twice that spread.
"""
import os

import numpy as np
import pytest

import golden_numpy as gn
from conftest import assert_bitwise, assert_close

HAVE = all(os.path.exists(gn.stages_path(m)) for m in ("w8a16", "w8a8"))
pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not HAVE, reason="numpy golden fixtures not generated")]

DN = "layers.0.linear_attn."
AT = "layers.3.self_attn."
ML = "layers.0.mlp."


class Dev:
    """Device copies of the tensors of layers 0 and 3, and probe projections."""

    def __init__(self, q, torch, blob, entries):
        self.q, self.torch, self.blob, self.e = q, torch, blob, entries
        self.cache = {}

    def up(self, a):
        return self.torch.from_numpy(np.ascontiguousarray(a)).cuda()

    def host_i8(self, name):
        return gn.fake_quant_weights(self.blob, self.e[name])

    def f32(self, name):
        if name not in self.cache:
            e = self.e[name]
            self.cache[name] = self.up(self.blob[e.off:e.off + e.nbytes].view(np.float32))
        return self.cache[name]

    def t(self, name):
        e = self.e[name]
        key = ("tensor", name)
        if key not in self.cache:
            if e.dtype == 1:
                qw, s = self.host_i8(name)
                self.cache[key] = (self.up(qw), self.up(s))
            else:
                self.cache[key] = self.f32(name).view(e.out, e.in_)
        c = self.cache[key]
        return self.q.Tensor.i8(*c) if e.dtype == 1 else self.q.Tensor.f32(c)

    def probe(self, rows, in_dim, first):
        key = ("probe", rows, in_dim, first)
        if key not in self.cache:
            w, s, n = gn.probe_rows(rows, in_dim, first)
            self.cache[key] = (self.up(w), self.up(s), n)
        w, s, n = self.cache[key]
        return self.q.Tensor.i8(w, s), n


@pytest.fixture(scope="module")
def D(q, blob, entries, torch_cuda):
    return Dev(q, torch_cuda, blob, entries)


def host(t):
    return t.cpu().numpy()


def run_deltanet(D, inp, w8a8, out_w=None):
    q, torch = D.q, D.torch
    out = torch.empty(1024, device="cuda")
    rec, conv = D.up(inp["dn_rec"]), D.up(inp["dn_conv"])
    q.deltanet_layer(out, D.up(inp["dn_x"]), D.t(DN + "in_proj_qkv.weight"), D.t(DN + "in_proj_z.weight"),
                     D.t(DN + "in_proj_b.weight"), D.t(DN + "in_proj_a.weight"), D.f32(DN + "conv1d.weight"),
                     D.f32(DN + "A_log"), D.f32(DN + "dt_bias"), D.f32(DN + "norm.weight"),
                     out_w or D.t(DN + "out_proj.weight"), rec, conv, w8a8=w8a8)
    torch.cuda.synchronize()
    return host(out), host(rec), host(conv)


def run_attention(D, inp, w8a8, out_w=None):
    q, torch = D.q, D.torch
    T = gn.ATTN_T
    kc = np.zeros((T + 1, 512), np.float32)
    vc = np.zeros((T + 1, 512), np.float32)
    kc[:T] = inp["at_kc"].reshape(T, 512)
    vc[:T] = inp["at_vc"].reshape(T, 512)
    kd, vd = D.up(kc), D.up(vc)
    out = torch.empty(1024, device="cuda")
    q.attention_layer(out, D.up(inp["at_x"]), D.t(AT + "q_proj.weight"), D.t(AT + "k_proj.weight"),
                      D.t(AT + "v_proj.weight"), out_w or D.t(AT + "o_proj.weight"), D.f32(AT + "q_norm.weight"),
                      D.f32(AT + "k_norm.weight"), gn.ATTN_POS, kd, vd, T, w8a8=w8a8)
    torch.cuda.synchronize()
    return host(out), host(kd)[T], host(vd)[T]


def run_mlp(D, inp, w8a8, out_w=None):
    q, torch = D.q, D.torch
    out = torch.empty(1024, device="cuda")
    q.mlp_layer(out, D.up(inp["ml_x"]), D.t(ML + "gate_proj.weight"), D.t(ML + "up_proj.weight"),
                out_w or D.t(ML + "down_proj.weight"), w8a8=w8a8)
    torch.cuda.synchronize()
    return host(out)


def probed(run, D, in_dim):
    parts = []
    for first in range(0, in_dim, 1024):
        w, n = D.probe(1024, in_dim, first)
        parts.append(run(w)[:n])
    return np.concatenate(parts)


def codes_of(y):
    sx = np.abs(y).max() / 127.0
    return np.rint(y / sx).astype(np.int32)


def check_codes(y, fx, qa, what):
    ok, nd, nt = gn.codes_match(codes_of(y), fx[qa + "_q"], fx[qa + "_in"], fx[qa + "_s"])
    assert ok, f"{what}: {nd} codes differ outside the {nt} near-ties"


def check_conv(conv, fx, x, D, w8a8):
    assert_bitwise(conv[:, :3], fx["dn_conv_out"][:, :3], "conv history (shifted columns)")
    qw, sw = D.host_i8(DN + "in_proj_qkv.weight")
    if w8a8:
        gn.assert_close_dot(conv[:, 3], fx["dn_conv_out"][:, 3], gn.dot_scale(qw, sw, x), what="conv history (new)")
    else:
        gn.assert_stage(conv[:, 3], fx["dn_conv_out"][:, 3], "dn_conv_out[:,3]", None, what="conv history (new)")


# ---------------------------------------------------------------- per stage

def test_act_quant(q, D):
    fx, _ = gn.load_stages("w8a8")
    torch = D.torch
    for k in ("dn_qa0", "dn_qa1", "at_qa0", "at_qa1", "ml_qa0", "ml_qa1"):
        x = fx[k + "_in"]
        xq = torch.empty(x.size, dtype=torch.int8, device="cuda")
        sx = torch.empty(1, device="cuda")
        q.quant_act(xq, sx, D.up(x), x.size)
        torch.cuda.synchronize()
        assert np.array_equal(host(xq), fx[k + "_q"]), k
        assert_bitwise(host(sx), np.atleast_1d(fx[k + "_s"]), k + " scale")


@pytest.mark.parametrize("mode", ["w8a16", "w8a8"])
def test_projections(q, D, mode):
    fx, inp = gn.load_stages(mode)
    torch = D.torch
    w8a8 = mode == "w8a8"
    cases = [(DN + "in_proj_qkv.weight", "dn_qa0", inp["dn_x"], fx["dn_in_proj_qkv"]),
             (DN + "in_proj_z.weight", "dn_qa0", inp["dn_x"], fx["dn_in_proj_z"]),
             (DN + "out_proj.weight", "dn_qa1", fx["dn_qa1_in"], fx["dn_out_proj"]),
             (AT + "q_proj.weight", "at_qa0", inp["at_x"], fx["at_q_proj"]),
             (AT + "k_proj.weight", "at_qa0", inp["at_x"], fx["at_k_proj"]),
             (AT + "v_proj.weight", "at_qa0", inp["at_x"], fx["at_v_proj"]),
             (AT + "o_proj.weight", "at_qa1", fx["at_qa1_in"], fx["at_o_proj"]),
             (ML + "gate_proj.weight", "ml_qa0", inp["ml_x"], fx["ml_gate_proj"]),
             (ML + "up_proj.weight", "ml_qa0", inp["ml_x"], fx["ml_up_proj"]),
             (ML + "down_proj.weight", "ml_qa1", fx["ml_qa1_in"], fx["ml_down_proj"])]
    keys = ["dn_in_proj_qkv", "dn_in_proj_z", "dn_out_proj", "at_q_proj", "at_k_proj", "at_v_proj", "at_o_proj",
            "ml_gate_proj", "ml_up_proj", "ml_down_proj"]
    for (name, qa, x, exp), key in zip(cases, keys):
        qw, sw = D.host_i8(name)
        wd, sd = D.up(qw), D.up(sw)
        out, inn = qw.shape
        y = torch.empty(out, device="cuda")
        if w8a8:
            acc = torch.empty(out, dtype=torch.int32, device="cuda")
            xq = fx[qa + "_q"]
            q.gemv_i8_w8a8(y, acc, wd, sd, D.up(xq), D.up(np.atleast_1d(fx[qa + "_s"])), out, inn)
            torch.cuda.synchronize()
            assert np.array_equal(host(acc).astype(np.int64), qw.astype(np.int64) @ xq.astype(np.int64)), name
            xs = xq.astype(np.float64) * float(fx[qa + "_s"])
        else:
            q.gemv_i8(y, wd, sd, D.up(x), out, inn)
            torch.cuda.synchronize()
            xs = x
        if w8a8:
            gn.assert_close_dot(host(y), exp, gn.dot_scale(qw, sw, xs), what=f"{name} ({mode})")
        else:
            gn.assert_stage(host(y), exp, key, gn.dot_scale(qw, sw, xs), what=f"{name} ({mode})")
    xg = fx["dn_qa0_q"].astype(np.float32) * np.float32(fx["dn_qa0_s"]) if w8a8 else inp["dn_x"]
    for name, key in ((DN + "in_proj_b.weight", "dn_in_proj_b"), (DN + "in_proj_a.weight", "dn_in_proj_a")):
        y = torch.empty(16, device="cuda")
        q.gemv_f32(y, D.f32(name), D.up(xg), 16, 1024)
        torch.cuda.synchronize()
        w = D.blob[D.e[name].off:D.e[name].off + D.e[name].nbytes].view(np.float32).reshape(16, 1024)
        scale = np.abs(w.astype(np.float64)) @ np.abs(xg.astype(np.float64))
        if w8a8:
            gn.assert_close_dot(host(y), fx[key], scale, what=f"{name} ({mode})")
        else:
            gn.assert_stage(host(y), fx[key], key, scale, what=f"{name} ({mode})")


@pytest.mark.parametrize("mode", ["w8a16", "w8a8"])
def test_deltanet(D, mode):
    fx, inp = gn.load_stages(mode)
    w8a8 = mode == "w8a8"
    out, rec, conv = run_deltanet(D, inp, w8a8)
    assert_close(rec[gn.S_HEADS], fx["dn_S_out"], gn.RTOL, gn.ATOL, what="recurrent state")
    x = fx["dn_qa0_q"].astype(np.float64) * float(fx["dn_qa0_s"]) if w8a8 else inp["dn_x"]
    check_conv(conv, fx, x, D, w8a8)
    y = probed(lambda w: run_deltanet(D, inp, w8a8, w)[0], D, 2048)
    if w8a8:
        check_codes(y, fx, "dn_qa1", "out_proj input codes")
    else:
        assert_close(y, fx["dn_qa1_in"], gn.RTOL, gn.ATOL, what="gated-norm output (out_proj input)")
        qw, sw = D.host_i8(DN + "out_proj.weight")
        gn.assert_stage(out, fx["dn_out"], "dn_out", gn.dot_scale(qw, sw, fx["dn_qa1_in"]), what="deltanet out")


@pytest.mark.parametrize("mode", ["w8a16", "w8a8"])
def test_attention(D, mode):
    fx, inp = gn.load_stages(mode)
    w8a8 = mode == "w8a8"
    out, k_new, v_new = run_attention(D, inp, w8a8)
    assert_close(k_new, fx["at_k_new"].reshape(-1), gn.RTOL, gn.ATOL, what="new K row")
    assert_close(v_new, fx["at_v_new"].reshape(-1), gn.RTOL, gn.ATOL, what="new V row")
    y = probed(lambda w: run_attention(D, inp, w8a8, w)[0], D, 2048)
    if w8a8:
        check_codes(y, fx, "at_qa1", "o_proj input codes")
    else:
        assert_close(y, fx["at_qa1_in"], gn.RTOL, gn.ATOL, what="gated context (o_proj input)")
        qw, sw = D.host_i8(AT + "o_proj.weight")
        gn.assert_stage(out, fx["at_out"], "at_out", gn.dot_scale(qw, sw, fx["at_qa1_in"]), what="attention out")


@pytest.mark.parametrize("mode", ["w8a16", "w8a8"])
def test_mlp(D, mode):
    fx, inp = gn.load_stages(mode)
    w8a8 = mode == "w8a8"
    y = probed(lambda w: run_mlp(D, inp, w8a8, w), D, 3584)
    if w8a8:
        check_codes(y, fx, "ml_qa1", "down input codes")
    else:
        gn.assert_stage(y, fx["ml_qa1_in"], "ml_qa1_in", None, what="SwiGLU activation (down input)")
        qw, sw = D.host_i8(ML + "down_proj.weight")
        gn.assert_stage(run_mlp(D, inp, False), fx["ml_out"], "ml_out", gn.dot_scale(qw, sw, fx["ml_qa1_in"]),
                        what="mlp out")


# ---------------------------------------------------------------- whole decode

@pytest.fixture(scope="module")
def stream_engine(q, blob, torch_cuda):
    e = q.Engine(blob, max_ctx=576)
    yield e
    e.close()


@pytest.mark.parametrize("exec_kind", ["graph", "persistent"])
@pytest.mark.parametrize("mode", ["w8a16", "w8a8"])
def test_teacher_forced_stream(q, stream_engine, mode, exec_kind):
    """All 576 steps of the golden's stream fed token by token: golden_numpy.StreamCheck."""
    g = gn.load_stream(mode)
    e = stream_engine
    e.set_mode(q.MODE_W8A8 if mode == "w8a8" else q.MODE_W8A16)
    want = q.EXEC_GRAPH if exec_kind == "graph" else q.EXEC_PERSISTENT
    e.set_exec(want)
    e.reset()
    chk = gn.StreamCheck(g, len(g["fed"]))
    for i, tok in enumerate(g["fed"]):
        am, lg = e.decode_token(tok, want_logits=True)
        chk.step(i, am, lg)
    assert e.exec_kind == want
    print(mode, exec_kind, chk.finish())


@pytest.mark.parametrize("mode", ["w8a16", "w8a8"])
def test_free_running_stream(q, stream_engine, mode):
    """generate() on the persistent executor from the golden's prompt: its ids follow the golden's
    until a step whose golden top-2 margin is within twice that step's own order spread (the
    golden's logit difference between two summation orders at that step; W8A16: all 512 ids equal)."""
    g = gn.load_stream(mode)
    e = stream_engine
    e.set_mode(q.MODE_W8A8 if mode == "w8a8" else q.MODE_W8A16)
    e.set_exec(q.EXEC_PERSISTENT)
    e.reset()
    npr, nn = g["n_prompt"], g["n_new"]
    gen = e.generate(g["fed"][:npr], nn)
    golden = g["argmax"][npr - 1:npr - 1 + nn]
    assert e.exec_kind == q.EXEC_PERSISTENT, "generate() ran on the graph fallback"
    div = next((i for i, (a, b) in enumerate(zip(gen, golden)) if a != b), None)
    if div is not None:
        step = npr - 1 + div
        assert g["margin"][step] <= 2 * g["order_dev"][step], \
            f"diverged at generated token {div} where the golden margin {g['margin'][step]} exceeds twice " \
            f"that step's order spread {g['order_dev'][step]}"
    if mode == "w8a16":
        assert div is None
    print(f"{mode}: first divergence from the golden stream at generated token {div}")
