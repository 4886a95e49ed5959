"""Op-level parity on the MI355X through the C ABI (include/qh_decode.h).

Every op is compared (a) bit for bit with the device-order twin in
oracle/oracle.c (same algorithm, the kernels' fixed reduction order) and (b)
with the reference-order restatement -- itself bit-identical to the compiled
hls/src kernels -- within rtol 1e-4 / atol 1e-5 (tb_deltanet.cpp:91 uses 2e-5 for
the delta rule).  Integer work (int32 accumulators, act-quant) is bit-exact
against the oracle, an int64 brute force and the reference gemv_i8 itself.
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitwise, assert_close, assert_close_norm, rng

pytestmark = pytest.mark.gpu


def p(a):
    return a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


@pytest.fixture(scope="module")
def T(torch_cuda):
    torch = torch_cuda

    class Dev:
        @staticmethod
        def up(a):
            return torch.from_numpy(np.ascontiguousarray(a)).cuda()

        @staticmethod
        def down(t):
            torch.cuda.synchronize()
            return t.cpu().numpy()

        @staticmethod
        def empty(n, dtype=np.float32):
            return torch.empty(n, dtype={np.float32: torch.float32, np.int32: torch.int32,
                                         np.int8: torch.int8}[dtype], device="cuda")
    return Dev


# ------------------------------------------------------------------ GEMV

@pytest.mark.parametrize("out,inn", [(3584, 1024), (1024, 3584), (6144, 1024), (1024, 2048), (37, 1024)])
def test_gemv_i8_w8a16(q, orc, T, out, inn):
    r = rng(out * 7 + inn)
    w = r.integers(-127, 128, size=(out, inn)).astype(np.int8)
    s = f32(r.uniform(1e-3, 1e-2, out))
    x = f32(r.standard_normal(inn))
    y = T.empty(out)
    q.gemv_i8(y, T.up(w), T.up(s), T.up(x), out, inn)
    got = T.down(y)
    dev, ref = np.empty(out, np.float32), np.empty(out, np.float32)
    orc.lib().or_dev_gemv_i8(p(dev), p(w), p(s), p(x), out, inn)
    orc.lib().or_gemv_i8(p(ref), p(w), p(s), p(x), out, inn)
    assert_bitwise(got, dev, "gemv_i8 vs device twin")
    assert_close_norm(got, ref, 1e-5, what="gemv_i8 vs reference order")


@pytest.mark.parametrize("out,inn", [(3584, 1024), (1024, 3584), (6144, 1024)])
def test_gemv_w8a8_int32_exact(q, orc, ref, T, out, inn):
    """C1: x ~ N(0,1) quantized per tensor, int32 accumulate, dequant float(acc)*sx*sw."""
    r = rng(out + 3 * inn)
    w = r.integers(-127, 128, size=(out, inn)).astype(np.int8)
    sw = f32(r.uniform(1e-3, 1e-2, out))
    x = f32(r.standard_normal(inn))
    xq_d, sx_d = T.empty(inn, np.int8), T.empty(1)
    q.quant_act(xq_d, sx_d, T.up(x), inn)
    xq, sx = T.down(xq_d), T.down(sx_d)
    xq_o, sx_o = np.empty(inn, np.int8), np.empty(1, np.float32)
    orc.lib().or_quant_act(p(xq_o), p(sx_o), p(x), inn)
    np.testing.assert_array_equal(xq, xq_o)
    assert sx[0] == sx_o[0]
    y_d, acc_d = T.empty(out), T.empty(out, np.int32)
    q.gemv_i8_w8a8(y_d, acc_d, T.up(w), T.up(sw), xq_d, sx_d, out, inn)
    acc, y = T.down(acc_d), T.down(y_d)
    np.testing.assert_array_equal(acc.astype(np.int64), w.astype(np.int64) @ xq.astype(np.int64))
    yo, acco = np.empty(out, np.float32), np.empty(out, np.int32)
    orc.lib().or_gemv_w8a8(p(yo), p(acco), p(w), p(sw), p(xq), float(sx[0]), out, inn)
    np.testing.assert_array_equal(acc, acco)
    assert_bitwise(y, yo, "dequant")
    if inn == 1024:   # c-note 1: the unmodified hls gemv_i8 on float(xq), scale 1, is exact for K <= 1040
        yr, ones, xf = np.empty(out, np.float32), np.ones(out, np.float32), f32(xq)
        ref.ref_gemv_i8(p(yr), p(w), p(ones), p(xf), out, inn)
        np.testing.assert_array_equal(yr.astype(np.int64), acc.astype(np.int64))


def test_quant_act_edges(q, orc, T):
    r = rng(5)
    for x in (f32(r.standard_normal(3584) * 1e4), f32(np.zeros(1024)),
              f32([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.0, 0.0] * 2), f32(r.standard_normal(2048) * 1e-20)):
        n = x.size
        xq_d, sx_d = T.empty(n, np.int8), T.empty(1)
        q.quant_act(xq_d, sx_d, T.up(x), n)
        xq_o, sx_o = np.empty(n, np.int8), np.empty(1, np.float32)
        orc.lib().or_quant_act(p(xq_o), p(sx_o), p(x), n)
        np.testing.assert_array_equal(T.down(xq_d), xq_o)
        assert T.down(sx_d)[0] == sx_o[0]


def test_small_ops(q, orc, T):
    L = orc.lib()
    r = rng(9)
    w = f32(r.standard_normal((16, 1024)) / 32)
    x = f32(r.standard_normal(1024))
    y = T.empty(16)
    q.gemv_f32(y, T.up(w), T.up(x), 16, 1024)
    dev, ref = np.empty(16, np.float32), np.empty(16, np.float32)
    L.or_dev_gemv_f32(p(dev), p(w), p(x), 16, 1024)
    L.or_gemv_f32(p(ref), p(w), p(x), 16, 1024)
    assert_bitwise(T.down(y), dev, "gemv_f32")
    assert_close_norm(T.down(y), ref, 1e-5, what="gemv_f32 vs ref")
    E = r.integers(-127, 128, size=(300, 1024)).astype(np.int8)
    es = f32(r.uniform(1e-3, 1e-2, 300))
    Ed, esd, xd = T.up(E), T.up(es), T.up(x)
    for row in (0, 123, 299):
        res = T.empty(1)
        q.row_dot_i8(res, Ed, esd, xd, row, 1024)
        d1 = np.empty(1, np.float32)
        L.or_dev_gemv_i8(p(d1), p(E[row:row + 1]), p(es[row:row + 1]), p(x), 1, 1024)
        assert_bitwise(T.down(res), d1, "row_dot_i8")
        assert_close(T.down(res)[0], L.or_row_dot_i8(p(E), p(es), p(x), row, 1024), what="row_dot vs ref")
        h = T.empty(1024)
        q.embed_row(h, Ed, esd, row, 1024)
        ho = np.empty(1024, np.float32)
        L.or_embed_row(p(ho), p(E), p(es), row, 1024)
        assert_bitwise(T.down(h), ho, "embed_row")
    for n in (1024, 256, 128, 100):
        xx = f32(r.standard_normal(n) * 3)
        ww = f32(r.standard_normal(n) * 0.1)
        zz = f32(r.standard_normal(n))
        yd = T.empty(n)
        q.rmsnorm(yd, T.up(xx), T.up(ww), n, 1e-6)
        yo = np.empty(n, np.float32)
        L.or_dev_rmsnorm(p(yo), p(xx), p(ww), n, 1e-6)
        assert_bitwise(T.down(yd), yo, f"rmsnorm {n}")
        L.or_rmsnorm(p(yo), p(xx), p(ww), n, 1e-6)
        assert_close(T.down(yd), yo, what="rmsnorm vs ref")
        q.rmsnorm_gated(yd, T.up(xx), T.up(ww), T.up(zz), n, 1e-6)
        L.or_dev_rmsnorm_gated(p(yo), p(xx), p(ww), p(zz), n, 1e-6)
        assert_bitwise(T.down(yd), yo, f"rmsnorm_gated {n}")
        vd = T.up(xx)
        q.l2norm(vd, n)
        vo = xx.copy()
        L.or_dev_l2norm(p(vo), n)
        assert_bitwise(T.down(vd), vo, f"l2norm {n}")


def test_conv_and_rope(q, orc, T):
    L = orc.lib()
    r = rng(13)
    inp = f32(r.standard_normal(6144))
    st = f32(r.standard_normal((6144, 4)))
    w = f32(r.standard_normal((6144, 4)) * 0.5)
    out_d, st_d = T.empty(6144), T.up(st)
    q.conv1d_step(out_d, T.up(inp), st_d, T.up(w))
    so, oo = st.copy(), np.empty(6144, np.float32)
    L.or_dev_conv1d_step(p(oo), p(inp), p(so), p(w))
    assert_bitwise(T.down(out_d), oo, "conv out")
    assert_bitwise(T.down(st_d), so, "conv state")
    sr, orr = st.copy(), np.empty(6144, np.float32)
    L.or_conv1d_step(p(orr), p(inp), p(sr), p(w))
    assert_close_norm(T.down(out_d), orr, 1e-6, what="conv vs ref")
    for pos in (0, 1, 575, 32767):
        c_d, s_d = T.empty(64), T.empty(64)
        q.rope_cos_sin(pos, c_d, s_d)
        c, s = np.empty(64, np.float32), np.empty(64, np.float32)
        L.or_rope_cos_sin(pos, p(c), p(s))
        assert_bitwise(T.down(c_d), c, "cos")   # host table from the reference formula (powf/cosf/sinf)
        assert_bitwise(T.down(s_d), s, "sin")
        x = f32(r.standard_normal(256))
        xd = T.up(x)
        q.apply_rope(xd, c_d, s_d)
        L.or_apply_rope(p(x), p(c), p(s))
        assert_bitwise(T.down(xd), x, "apply_rope")


def _delta_inputs(seed):
    r = rng(seed)
    qq = f32(r.standard_normal((16, 128)))
    k = f32(r.standard_normal((16, 128)))
    qq = f32(qq / np.linalg.norm(qq, axis=1, keepdims=True) * np.float32(1 / np.sqrt(128)))
    k = f32(k / np.linalg.norm(k, axis=1, keepdims=True))
    v = f32(r.standard_normal((16, 128)))
    g = f32(-r.uniform(0.01, 2.0, 16))
    beta = f32(r.uniform(0.05, 0.95, 16))
    S = f32(r.standard_normal((16, 128, 128)) * 0.05)
    return qq, k, v, g, beta, S


def test_delta_rule(q, orc, T):
    L = orc.lib()
    qq, k, v, g, beta, S = _delta_inputs(17)
    S_d, o_d = T.up(S), T.empty(2048)
    q.delta_rule_layer(T.up(qq), T.up(k), T.up(v), T.up(g), T.up(beta), S_d, o_d)
    So, oo = S.copy(), np.empty((16, 128), np.float32)
    L.or_dev_delta_rule_layer(p(qq), p(k), p(v), p(g), p(beta), p(So), p(oo))
    assert_bitwise(T.down(o_d).reshape(16, 128), oo, "delta out")
    assert_bitwise(T.down(S_d).reshape(16, 128, 128), So, "delta S")
    Sr, orr = S.copy(), np.empty((16, 128), np.float32)
    L.or_delta_rule_layer(p(qq), p(k), p(v), p(g), p(beta), p(Sr), p(orr))
    assert_close(T.down(o_d).reshape(16, 128), orr, rtol=0, atol=2e-5, what="out vs ref (tb_deltanet tol)")
    assert_close(T.down(S_d).reshape(16, 128, 128), Sr, rtol=0, atol=2e-5, what="S vs ref")
    h = 5
    Sh_d, oh_d = T.up(S[h]), T.empty(128)
    q.delta_rule_head(T.up(qq[h]), T.up(k[h]), T.up(v[h]), float(g[h]), float(beta[h]), Sh_d, oh_d)
    assert_bitwise(T.down(oh_d), oo[h], "head out")
    assert_bitwise(T.down(Sh_d).reshape(128, 128), So[h], "head S")
