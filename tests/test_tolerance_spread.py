"""How far from the reference's numpy golden (golden/model.py) each golden stage lands, against the
north_star's literal tolerance, rtol 1e-4 / atol 1e-5 elementwise, for two implementations:

  device     the device-order twin (oracle.c ORDER_DEV), bit for bit the HIP path (the GPU tests
             compare them per op, per layer and per decode step);
  reference  the reference's own hls/src kernels, compiled from the headers where they lie
             (oracle/_ref, its csim flags) -- W8A16, the reference's arithmetic.

Per stage output: the largest elementwise relative error |a - b| / |b| (over |b| >= atol) and the
count of elements outside atol + rtol |b|.  Where the compiled reference meets the literal tolerance,
so must the device; the sum-|w x| bound of test_golden_numpy stays only for stages where the
reference's own pair (its sequential loops against the golden's BLAS) already exceeds it.  One
stage is a product of two reductions, the SwiGLU activation silu(gate) * up: each factor is held to
the literal tolerance (its projection row), and a product of two factors within rtol of theirs is
within 2 rtol of its own, so that stage is held to twice the literal tolerance.
Run with -s to see the table.
"""

PRODUCTS = {"ml_qa1_in"}   # silu(gate projection) * (up projection)
import numpy as np
import pytest

import golden_numpy as gn
from test_golden_numpy import AT, DN, HAVE, ML, L, p, probed  # noqa: F401 (L: fixture)

pytestmark = pytest.mark.skipif(not HAVE, reason="numpy golden fixtures not generated")


def spread(got, exp):
    """(max relative error, elements outside atol + rtol |b|, elements, max |a - b| / (atol + rtol |b|))"""
    got = np.asarray(got, np.float64).reshape(-1)
    exp = np.asarray(exp, np.float64).reshape(-1)
    err = np.abs(got - exp)
    big = np.abs(exp) >= gn.ATOL
    rel = float((err[big] / np.abs(exp[big])).max()) if big.any() else 0.0
    tol = gn.ATOL + gn.RTOL * np.abs(exp)
    return rel, int((err > tol).sum()), exp.size, float((err / tol).max())


def layers(orc, ref, L, inp, dev):
    """{stage: output} of the three golden stages (W8A16), device twin or compiled reference."""
    T, lib = gn.ATTN_T, orc.lib()

    def dn(out_w=None):
        out = np.empty(1024, np.float32)
        rec, conv = inp["dn_rec"].copy(), inp["dn_conv"].copy()
        args = (p(out), p(inp["dn_x"]), L.t(DN + "in_proj_qkv.weight"), L.t(DN + "in_proj_z.weight"),
                L.t(DN + "in_proj_b.weight"), L.t(DN + "in_proj_a.weight"), p(L.f32(DN + "conv1d.weight")),
                p(L.f32(DN + "A_log")), p(L.f32(DN + "dt_bias")), p(L.f32(DN + "norm.weight")),
                out_w or L.t(DN + "out_proj.weight"), p(rec), p(conv))
        if dev:
            lib.or_deltanet_layer(*args, orc.W8A16, orc.ORDER_DEV)
        else:
            ref.ref_deltanet_layer(*args)
        return out, rec, conv

    def at(out_w=None):
        kc = np.zeros((T + 1, 512), np.float32)
        vc = np.zeros((T + 1, 512), np.float32)
        kc[:T] = inp["at_kc"].reshape(T, 512)
        vc[:T] = inp["at_vc"].reshape(T, 512)
        out = np.empty(1024, np.float32)
        args = (p(out), p(inp["at_x"]), L.t(AT + "q_proj.weight"), L.t(AT + "k_proj.weight"),
                L.t(AT + "v_proj.weight"), out_w or L.t(AT + "o_proj.weight"), p(L.f32(AT + "q_norm.weight")),
                p(L.f32(AT + "k_norm.weight")), gn.ATTN_POS, p(kc), p(vc), T)
        if dev:
            lib.or_attention_layer(*args, orc.W8A16, orc.ORDER_DEV)
        else:
            ref.ref_attention_layer(*args)
        return out, kc[T], vc[T]

    def ml(out_w=None):
        out = np.empty(1024, np.float32)
        args = (p(out), p(inp["ml_x"]), L.t(ML + "gate_proj.weight"), L.t(ML + "up_proj.weight"),
                out_w or L.t(ML + "down_proj.weight"))
        if dev:
            lib.or_mlp_layer(*args, orc.W8A16, orc.ORDER_DEV)
        else:
            ref.ref_mlp_layer(*args)
        return out

    out, rec, conv = dn()
    a_out, k_new, v_new = at()
    return {"dn_out": out, "dn_S_out": rec[gn.S_HEADS], "dn_conv_out[:,3]": conv[:, 3],
            "dn_qa1_in": probed(lambda w: dn(w)[0], L, 2048),
            "at_out": a_out, "at_k_new": k_new, "at_v_new": v_new,
            "at_qa1_in": probed(lambda w: at(w)[0], L, 2048),
            "ml_out": ml(), "ml_qa1_in": probed(ml, L, 3584)}


def projections(orc, ref, L, fx, inp, dev):
    lib = orc.lib()
    out = {}
    for name, x, key in ((DN + "in_proj_qkv.weight", inp["dn_x"], "dn_in_proj_qkv"),
                         (DN + "in_proj_z.weight", inp["dn_x"], "dn_in_proj_z"),
                         (DN + "out_proj.weight", fx["dn_qa1_in"], "dn_out_proj"),
                         (AT + "q_proj.weight", inp["at_x"], "at_q_proj"),
                         (AT + "k_proj.weight", inp["at_x"], "at_k_proj"),
                         (AT + "v_proj.weight", inp["at_x"], "at_v_proj"),
                         (AT + "o_proj.weight", fx["at_qa1_in"], "at_o_proj"),
                         (ML + "gate_proj.weight", inp["ml_x"], "ml_gate_proj"),
                         (ML + "up_proj.weight", inp["ml_x"], "ml_up_proj"),
                         (ML + "down_proj.weight", fx["ml_qa1_in"], "ml_down_proj")):
        qw, s = L.i8(name)
        y = np.empty(qw.shape[0], np.float32)
        x = np.ascontiguousarray(x, np.float32)
        (lib.or_dev_gemv_i8 if dev else ref.ref_gemv_i8)(p(y), p(qw), p(s), p(x), qw.shape[0], qw.shape[1])
        out[key] = y
    for name, key in ((DN + "in_proj_b.weight", "dn_in_proj_b"), (DN + "in_proj_a.weight", "dn_in_proj_a")):
        y = np.empty(16, np.float32)
        (lib.or_dev_gemv_f32 if dev else ref.ref_gemv_f32)(p(y), p(L.f32(name)), p(inp["dn_x"]), 16, 1024)
        out[key] = y
    return out


def test_tolerance_spread_w8a16(orc, ref, L, capsys):
    fx, inp = gn.load_stages("w8a16")
    fx = dict(fx)
    fx["dn_conv_out[:,3]"] = fx["dn_conv_out"][:, 3]
    got = {}
    for dev in (True, False):
        got[dev] = dict(projections(orc, ref, L, fx, inp, dev), **layers(orc, ref, L, inp, dev))
    rows, bad = [], []
    for key in got[True]:
        d = spread(got[True][key], fx[key])
        r = spread(got[False][key], fx[key])
        rows.append(f"| {key} | {d[2]} | {d[0]:.2e} | {d[1]} | {d[3]:.2f} | {r[0]:.2e} | {r[1]} | {r[3]:.2f} |")
        limit = 2.0 if key in PRODUCTS else 1.0
        if r[1] == 0 and d[3] > limit:
            bad.append(f"{key}: the compiled reference meets rtol 1e-4 / atol 1e-5 but the device reaches "
                       f"{d[3]:.2f}x it (limit {limit}; {d[1]} elements outside, max rel {d[0]:.2e})")
    with capsys.disabled():
        print("\n| stage (W8A16) | elements | device max rel | device outside | device worst / tol |"
              " reference max rel | reference outside | reference worst / tol |")
        print("|---|---:|---:|---:|---:|---:|---:|---:|")
        print("\n".join(rows))
    assert not bad, "\n".join(bad)


@pytest.mark.parametrize("mode", ["w8a8"])
def test_tolerance_spread_w8a8(orc, L, mode, capsys):
    """W8A8 has no compiled reference (hls/src computes int8 x fp32): the device twin's spread against
    the golden's int8-activation path is reported, and pinned by test_golden_numpy's bounds."""
    fx, inp = gn.load_stages(mode)
    lib, T = orc.lib(), gn.ATTN_T
    out = np.empty(1024, np.float32)
    rec, conv = inp["dn_rec"].copy(), inp["dn_conv"].copy()
    lib.or_deltanet_layer(p(out), p(inp["dn_x"]), L.t(DN + "in_proj_qkv.weight"), L.t(DN + "in_proj_z.weight"),
                          L.t(DN + "in_proj_b.weight"), L.t(DN + "in_proj_a.weight"), p(L.f32(DN + "conv1d.weight")),
                          p(L.f32(DN + "A_log")), p(L.f32(DN + "dt_bias")), p(L.f32(DN + "norm.weight")),
                          L.t(DN + "out_proj.weight"), p(rec), p(conv), orc.W8A8, orc.ORDER_DEV)
    kc = np.zeros((T + 1, 512), np.float32)
    vc = np.zeros((T + 1, 512), np.float32)
    kc[:T] = inp["at_kc"].reshape(T, 512)
    vc[:T] = inp["at_vc"].reshape(T, 512)
    a_out = np.empty(1024, np.float32)
    lib.or_attention_layer(p(a_out), p(inp["at_x"]), L.t(AT + "q_proj.weight"), L.t(AT + "k_proj.weight"),
                           L.t(AT + "v_proj.weight"), L.t(AT + "o_proj.weight"), p(L.f32(AT + "q_norm.weight")),
                           p(L.f32(AT + "k_norm.weight")), gn.ATTN_POS, p(kc), p(vc), T, orc.W8A8, orc.ORDER_DEV)
    m_out = np.empty(1024, np.float32)
    lib.or_mlp_layer(p(m_out), p(inp["ml_x"]), L.t(ML + "gate_proj.weight"), L.t(ML + "up_proj.weight"),
                     L.t(ML + "down_proj.weight"), orc.W8A8, orc.ORDER_DEV)
    rows = []
    for key, g in (("dn_out", out), ("dn_S_out", rec[gn.S_HEADS]), ("at_out", a_out), ("at_k_new", kc[T]),
                   ("at_v_new", vc[T]), ("ml_out", m_out)):
        d = spread(g, fx[key])
        rows.append(f"| {key} | {d[2]} | {d[0]:.2e} | {d[1]} | {d[3]:.2f} |")
    with capsys.disabled():
        print("\n| stage (W8A8) | elements | device max rel | device outside | device worst / tol |")
        print("|---|---:|---:|---:|---:|")
        print("\n".join(rows))
