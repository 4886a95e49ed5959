"""The RTL's fixed-point matvec contract (rtl/matvec_i8.sv = gemv_i8.sv + dequant.sv) on the CPU:
the host-side multipliers (qh_dequant_mult, rtl/tb/sim_matvec.cpp:36-41), the oracle's
restatement pinned by closed forms and by Python's exact integers, the tv_gemv.bin format
(scripts/export_gemv_tv.py:62-72), and the reference bench's 4-LSB criterion on a case
built the way export_gemv_tv.py builds it (token 6511, layer 3 input norm, layer 3 k_proj)
from the seeded synthetic blob."""
import math

import numpy as np
import pytest

from qwen_fpga_amd import fixtures as fx


def llround(c: float) -> int:
    """C's llround: nearest integer, ties away from zero."""
    return int(math.copysign(math.floor(abs(c) + 0.5), c))


def rtl_yq(acc: int, mult: int, shift: int, outw: int) -> int:
    """dequant.sv in exact integers: (acc*mult + 2^(shift-1)) >>> shift, then the low outw bits."""
    y = (acc * mult + (1 << (shift - 1))) >> shift          # Python >> on negatives is floor
    return ((y + (1 << (outw - 1))) % (1 << outw)) - (1 << (outw - 1))


# ---------------------------------------------------------------- multipliers

def test_dequant_mult_closed_forms(q):
    two30 = 2.0 ** -30
    sw = np.array([1.0, 0.5, -0.5, 1.5, 2.5, 0.0, -2.5], np.float32) * np.float32(two30)
    # c = sx*sw*2^30 = 1, .5, -.5, 1.5, 2.5, 0, -2.5: ties go away from zero (not to even)
    assert q.dequant_mult(1.0, sw).tolist() == [1, 1, -1, 2, 3, 0, -3]
    assert q.dequant_mult(0.25, np.array([1.0], np.float32), outq=14, shift=16).tolist() == [1 << 28]


def test_dequant_mult_matches_double_formula(q):
    rng = np.random.default_rng(4)
    sw = (rng.random(512) * 1e-3).astype(np.float32)
    sx = float(np.float32(0.0123))
    for outq, shift in ((14, 16), (10, 12), (20, 8)):
        m = q.dequant_mult(sx, sw, outq=outq, shift=shift)
        exp = [llround(float(np.float64(np.float32(sx)) * np.float64(s)) * 2.0 ** (outq + shift)) for s in sw]
        assert m.tolist() == exp


def test_dequant_mult_range_and_arguments(q):
    with pytest.raises(q.QHError) as e:
        q.dequant_mult(1.0, np.array([2.0], np.float32))    # 2 * 2^30 = 2^31: beyond the 32-bit port
    assert e.value.status == q.QH_ERANGE
    assert q.dequant_mult(1.0, np.array([1.999999], np.float32)).tolist() == [llround(float(np.float32(1.999999)) * 2.0 ** 30)]
    for kw in ({"outq": 40, "shift": 30}, {"outq": 14, "shift": 0}, {"outq": -1, "shift": 16}):
        with pytest.raises(q.QHError):
            q.dequant_mult(1.0, np.array([1e-3], np.float32), **kw)


# ---------------------------------------------------------------- the oracle

def _single(a_vals, in_=16):
    """w rows with one non-zero weight a in column 0 and xq = e0: acc[o] = a_vals[o]."""
    w = np.zeros((len(a_vals), in_), np.int8)
    w[:, 0] = a_vals
    xq = np.zeros(in_, np.int8)
    xq[0] = 1
    return w, xq


def test_matvec_oracle_closed_forms(orc):
    w, xq = _single([3, -3, 125, 125, 0, -1])
    mult = np.array([1 << 15, 1 << 15, 20971520, 20971520, 12345, 1], np.int32)
    yq, acc = orc.matvec_fixed(w, xq, mult, shift=16, outw=16)
    assert acc.tolist() == [3, -3, 125, 125, 0, -1]
    # 1.5 -> 2 and -1.5 -> -1 (half up); 40000 wraps to 40000 - 65536 in 16 bits; -1/65536 -> 0
    assert yq.tolist() == [2, -1, -25536, -25536, 0, 0]
    yq32, _ = orc.matvec_fixed(w, xq, mult, shift=16, outw=32)
    assert yq32.tolist() == [2, -1, 40000, 40000, 0, 0]


@pytest.mark.parametrize("shift,outw", [(16, 16), (12, 32), (20, 16), (30, 24)])
def test_matvec_oracle_equals_exact_integers(orc, shift, outw):
    rng = np.random.default_rng(shift * 100 + outw)
    out, in_ = 96, 1024
    w = rng.integers(-127, 128, (out, in_), dtype=np.int8)
    xq = rng.integers(-127, 128, in_, dtype=np.int8)
    mult = rng.integers(-(1 << 31), (1 << 31) - 1, out, dtype=np.int64).astype(np.int32)
    mult[:4] = [0, 1, -1, (1 << 31) - 1]
    yq, acc = orc.matvec_fixed(w, xq, mult, shift=shift, outw=outw)
    acc_exact = w.astype(np.int64) @ xq.astype(np.int64)
    assert acc.tolist() == acc_exact.tolist()
    assert yq.tolist() == [rtl_yq(int(a), int(m), shift, outw) for a, m in zip(acc_exact, mult)]


# ---------------------------------------------------------------- tv_gemv.bin

def make_tv_gemv(orc, q, blob, entries, tok=6511, sw_scale=1.0):
    """export_gemv_tv.py:38-56 on the packed blob: embed token, layer-3 input norm (1+w),
    per-vector int8, layer-3 k_proj rows as packed; y = float(acc)*sx*sw.  sw_scale (a power
    of two, so y scales exactly) brings the synthetic outputs into the Q14 int16 range a real
    k_proj case has."""
    def f32(name):
        e = entries[name]
        return blob[e.off:e.off + e.nbytes].view(np.float32)

    emb = entries["embed_tokens.weight"]
    h = np.empty(1024, np.float32)
    L = orc.lib()
    L.or_embed_row(h.ctypes.data, blob[emb.off:].ctypes.data, blob[emb.soff:].ctypes.data, tok, 1024)
    hn = np.empty(1024, np.float32)
    L.or_rmsnorm(hn.ctypes.data, h.ctypes.data, np.ascontiguousarray(f32("layers.3.input_layernorm.weight")).ctypes.data,
                 1024, np.float32(1e-6))
    xq = np.empty(1024, np.int8)
    sx = np.empty(1, np.float32)
    L.or_quant_act(xq.ctypes.data, sx.ctypes.data, hn.ctypes.data, 1024)
    k = entries["layers.3.self_attn.k_proj.weight"]
    w = blob[k.off:k.off + k.nbytes].view(np.int8).reshape(k.out, k.in_).copy()
    sw = blob[k.soff:k.soff + k.snbytes].view(np.float32) * np.float32(sw_scale)
    acc = (w.astype(np.int64) @ xq.astype(np.int64)).astype(np.int32)
    y = acc.astype(np.float32) * np.float32(sx[0]) * sw
    return fx.GemvTv(xq, w, acc, float(sx[0]), sw, y)


def test_tv_gemv_roundtrip_and_size_check(orc, q, blob, entries, tmp_path):
    tv = make_tv_gemv(orc, q, blob, entries)
    p = str(tmp_path / "tv_gemv.bin")
    fx.write_tv_gemv(p, tv)
    assert (tmp_path / "tv_gemv.json").read_text() == '{"IN": 1024, "OUT": 512}'
    assert (tmp_path / "tv_gemv.bin").stat().st_size == 1024 + 512 * 1024 + 4 * 512 + 4 + 8 * 512
    r = fx.read_tv_gemv(p)
    for a, b in ((r.x, tv.x), (r.w, tv.w), (r.acc, tv.acc), (r.sw, tv.sw), (r.y, tv.y)):
        np.testing.assert_array_equal(a, b)
    assert r.sx == tv.sx
    with open(p, "ab") as f:
        f.write(b"\0")
    with pytest.raises(ValueError, match="needs"):
        fx.read_tv_gemv(p)


@pytest.mark.parametrize("sw_scale,outw", [(1 / 64, 16), (1.0, 32)], ids=["q14-int16", "q14-int32"])
def test_reference_criterion_holds_for_the_contract(orc, q, blob, entries, sw_scale, outw):
    """sim_matvec.cpp:78-86 on the oracle: Q14 within 4 LSB of round(y * 2^14), acc exact.
    The synthetic k_proj outputs reach ~70: in 16 bits they need the 1/64 scale, unscaled
    they need the widened output (OUTW 32, matvec_i8.sv:12)."""
    tv = make_tv_gemv(orc, q, blob, entries, sw_scale=sw_scale)
    assert np.abs(tv.y).max() * 16384 < 2.0 ** (outw - 1)
    mult = q.dequant_mult(tv.sx, tv.sw, outq=14, shift=16)
    yq, acc = orc.matvec_fixed(tv.w, tv.x, mult, shift=16, outw=outw)
    np.testing.assert_array_equal(acc, tv.acc)
    ref = np.array([llround(float(v) * 16384.0) for v in tv.y])
    assert np.abs(yq - ref).max() <= fx.MATVEC_LSB_TOL
    if outw == 32:   # the same case in 16 bits wraps wherever |y| >= 2
        y16, _ = orc.matvec_fixed(tv.w, tv.x, mult, shift=16, outw=16)
        assert y16.tolist() == [((v + 32768) % 65536) - 32768 for v in yq.tolist()]
        assert (np.abs(tv.y) >= 2).any()
