"""Readers / writers for the reference's own fixture files (qwen_fpga_amd.fixtures):
decode_ref.bin (scripts/export_decode_ref.py:47-53, hls/tb/tb_decode.cpp:73-82) and
tv_deltanet.bin (scripts/export_testvectors.py:55-60, hls/tb/tb_deltanet.cpp:57-71)."""
import numpy as np
import pytest

from conftest import rng
from qwen_fpga_amd import fixtures as fx


def test_tv_deltanet_layout_size():
    # artifacts/tv_deltanet.json: "total_bytes": 2130048, tensors q k v g beta S_in o_core S_out
    assert fx.TV_BYTES == 2130048
    assert fx.TV_ORDER == ("q", "k", "v", "g", "beta", "S_in", "o_core", "S_out")
    offs, o = {}, 0
    for n in fx.TV_ORDER:
        offs[n] = o
        o += 4 * int(np.prod(fx.TV_SHAPES[n]))
    # offsets of the reference's json (q 0, k 8192, v 16384, g 24576, beta 24640, S_in 24704, ...)
    assert (offs["k"], offs["v"], offs["g"], offs["beta"], offs["S_in"]) == (8192, 16384, 24576, 24640, 24704)
    assert offs["o_core"] == 24704 + 1048576 and offs["S_out"] == offs["o_core"] + 8192


def test_tv_deltanet_round_trip(tmp_path):
    r = rng(3)
    tv = {n: r.standard_normal(fx.TV_SHAPES[n]).astype(np.float32) for n in fx.TV_ORDER}
    p = tmp_path / "tv_deltanet.bin"
    fx.write_tv_deltanet(str(p), tv)
    assert p.stat().st_size == fx.TV_BYTES
    back = fx.read_tv_deltanet(str(p))
    for n in fx.TV_ORDER:
        assert np.array_equal(back[n], tv[n]), n
    raw = p.read_bytes()
    assert np.array_equal(np.frombuffer(raw[:4 * 2048], "<f4").reshape(16, 128), tv["q"])   # q first
    (tmp_path / "short.bin").write_bytes(raw[:-4])
    with pytest.raises(ValueError):
        fx.read_tv_deltanet(str(tmp_path / "short.bin"))


def test_decode_ref_round_trip(tmp_path):
    r = rng(5)
    n = 11
    fed = r.integers(0, fx.VOCAB, n)
    am = r.integers(0, fx.VOCAB, n)
    lg = r.standard_normal(fx.VOCAB).astype(np.float32)
    p = tmp_path / "decode_ref.bin"
    fx.write_decode_ref(str(p), fed, am, lg)
    assert p.stat().st_size == 4 + 8 * n + 4 * fx.VOCAB
    raw = p.read_bytes()
    assert int(np.frombuffer(raw[:4], "<i4")[0]) == n
    assert np.array_equal(np.frombuffer(raw[4:4 + 4 * n], "<i4"), fed)
    d = fx.read_decode_ref(str(p))
    assert np.array_equal(d.fed, fed) and np.array_equal(d.argmax, am) and np.array_equal(d.logits0, lg)
    (tmp_path / "long.bin").write_bytes(raw + b"\0\0\0\0")
    with pytest.raises(ValueError):
        fx.read_decode_ref(str(tmp_path / "long.bin"))


def test_tv_deltanet_from_the_oracle_passes_its_own_check(orc, tmp_path):
    """A fixture written from the reference-order delta rule reads back and, replayed through
    the same CPU rule, meets tb_deltanet's 2e-5 bound (checks the writer's tensor order)."""
    tv = make_tv_deltanet(orc, seed=9)
    p = tmp_path / "tv.bin"
    fx.write_tv_deltanet(str(p), tv)
    back = fx.read_tv_deltanet(str(p))
    S = back["S_in"].copy()
    out = np.empty((16, 128), np.float32)
    P = orc.ptr
    orc.lib().or_delta_rule_layer(P(back["q"]), P(back["k"]), P(back["v"]), P(back["g"]), P(back["beta"]), P(S), P(out))
    assert np.abs(out - back["o_core"]).max() < fx.DELTA_TOL
    assert np.abs(S - back["S_out"]).max() < fx.DELTA_TOL


def make_tv_deltanet(orc, seed: int) -> dict:
    """q, k l2-normalised (q also scaled by 1/sqrt(128)), like the exported fixture; a warm state."""
    r = rng(seed)
    q = r.standard_normal((16, 128)).astype(np.float32)
    k = r.standard_normal((16, 128)).astype(np.float32)
    q /= np.sqrt((q.astype(np.float64) ** 2).sum(1, keepdims=True) + 1e-6).astype(np.float32)
    k /= np.sqrt((k.astype(np.float64) ** 2).sum(1, keepdims=True) + 1e-6).astype(np.float32)
    q = (q * np.float32(1.0 / np.sqrt(128.0))).astype(np.float32)
    v = r.standard_normal((16, 128)).astype(np.float32)
    g = (-r.uniform(0.01, 2.0, 16)).astype(np.float32)
    beta = r.uniform(0.05, 0.95, 16).astype(np.float32)
    S_in = (0.05 * r.standard_normal((16, 128, 128))).astype(np.float32)
    S = S_in.copy()
    out = np.empty((16, 128), np.float32)
    P = orc.ptr
    orc.lib().or_delta_rule_layer(P(q), P(k), P(v), P(g), P(beta), P(S), P(out))
    return {"q": q, "k": k, "v": v, "g": g, "beta": beta, "S_in": S_in, "o_core": out, "S_out": S}
