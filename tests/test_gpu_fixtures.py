"""The reference's testbenches replayed on the MI355X: qh_tb_decode (hls/tb/tb_decode.cpp)
and qh_tb_deltanet (hls/tb/tb_deltanet.cpp) on fixture files in the reference's formats
(decode_ref.bin, tv_deltanet.bin), written here from the reference-order oracle, with the
reference testbenches' own pass criteria (argmax at every step and step-0 logits within
5e-2; delta rule within 2e-5)."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from qwen_fpga_amd import fixtures as fx
from test_fixtures import make_tv_deltanet

pytestmark = pytest.mark.gpu
BIN = os.path.join(ROOT, "qwen_fpga_amd", "bin")
FED = [11, 2222, 33333, 44, 248000, 5, 77, 77]


@pytest.fixture(scope="module")
def decode_ref_file(orc, blob, idx, tmp_path_factory):
    """decode_ref.bin from the reference-order oracle qwen_top (W8A16), plus the blob and idx."""
    d = tmp_path_factory.mktemp("decode_ref")
    m = orc.Model(blob, idx, max_ctx=len(FED))
    am, lg0 = [], None
    for i, t in enumerate(FED):
        a, lg = m.decode_token(t, mode=orc.W8A16, order=orc.ORDER_REF, want_logits=(i == 0))
        am.append(a)
        if i == 0:
            lg0 = lg
    m.close()
    fx.write_decode_ref(str(d / "decode_ref.bin"), FED, am, lg0)
    blob.tofile(str(d / "qwen35_int8.bin"))
    (d / "weights.idx").write_text(idx)
    return d


def test_tb_decode_cli(decode_ref_file):
    d = decode_ref_file
    for extra in ([], ["--persistent"]):
        r = subprocess.run([os.path.join(BIN, "qh_tb_decode"), str(d / "qwen35_int8.bin"), str(d / "weights.idx"),
                            str(d / "decode_ref.bin")] + extra, capture_output=True, text=True, timeout=180)
        assert r.returncode == 0, r.stdout + r.stderr
        assert "PASS" in r.stdout and "MISMATCH" not in r.stdout


def test_tb_decode_cli_fails_on_a_wrong_argmax(decode_ref_file, tmp_path):
    d = decode_ref_file
    ref = fx.read_decode_ref(str(d / "decode_ref.bin"))
    bad = ref.argmax.copy()
    bad[3] = (bad[3] + 1) % fx.VOCAB
    fx.write_decode_ref(str(tmp_path / "bad.bin"), ref.fed, bad, ref.logits0)
    r = subprocess.run([os.path.join(BIN, "qh_tb_decode"), str(d / "qwen35_int8.bin"), "-", str(tmp_path / "bad.bin")],
                       capture_output=True, text=True, timeout=180)
    assert r.returncode == 1 and "MISMATCH" in r.stdout and "FAIL" in r.stdout


def test_replay_decode_ref_python(q, decode_ref_file, blob, torch_cuda):
    ref = fx.read_decode_ref(str(decode_ref_file / "decode_ref.bin"))
    e = q.Engine(blob, max_ctx=len(FED))
    try:
        res = fx.replay_decode_ref(e, ref)
    finally:
        e.close()
    assert res["pass"], res
    assert res["mismatches"] == 0 and res["max_abs"] < 1e-3


def test_tb_deltanet_cli(orc, tmp_path):
    p = tmp_path / "tv_deltanet.bin"
    fx.write_tv_deltanet(str(p), make_tv_deltanet(orc, seed=11))
    r = subprocess.run([os.path.join(BIN, "qh_tb_deltanet"), str(p)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS" in r.stdout


def test_tb_deltanet_cli_fails_on_a_wrong_state(orc, tmp_path):
    tv = make_tv_deltanet(orc, seed=12)
    tv["S_out"] = tv["S_out"].copy()
    tv["S_out"][5, 7, 9] += 1e-3
    p = tmp_path / "tv_bad.bin"
    fx.write_tv_deltanet(str(p), tv)
    r = subprocess.run([os.path.join(BIN, "qh_tb_deltanet"), str(p)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "FAIL" in r.stdout


def test_replay_tv_deltanet_python(orc, torch_cuda):
    res = fx.replay_tv_deltanet(make_tv_deltanet(orc, seed=13))
    assert res["pass"], res
