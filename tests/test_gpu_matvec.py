"""qh_matvec_i8 (the RTL's gemv_i8 + dequant, rtl/matvec_i8.sv) on the MI355X against the
oracle bit for bit, and the qh_sim_matvec program (rtl/tb/sim_gemv.cpp + sim_matvec.cpp
criteria) on tv_gemv.bin files built like scripts/export_gemv_tv.py's."""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from qwen_fpga_amd import fixtures as fx
from test_matvec import make_tv_gemv

pytestmark = pytest.mark.gpu
SIM = os.path.join(ROOT, "qwen_fpga_amd", "bin", "qh_sim_matvec")


@pytest.mark.parametrize("out,in_,shift,outw", [(512, 1024, 16, 16), (1024, 2048, 16, 32), (100, 4096, 20, 16),
                                                (33, 16, 30, 24), (1024, 3584, 12, 32)])
def test_matvec_i8_matches_oracle(q, orc, torch_cuda, out, in_, shift, outw):
    torch = torch_cuda
    rng = np.random.default_rng(out + in_ + shift)
    w = rng.integers(-127, 128, (out, in_), dtype=np.int8)
    xq = rng.integers(-127, 128, in_, dtype=np.int8)
    mult = rng.integers(-(1 << 31), (1 << 31) - 1, out, dtype=np.int64).astype(np.int32)
    yq_o, acc_o = orc.matvec_fixed(w, xq, mult, shift=shift, outw=outw)
    dev = lambda a: torch.from_numpy(a).cuda()
    yq = torch.full((out,), 7, dtype=torch.int32, device="cuda")
    acc = torch.full((out,), 7, dtype=torch.int32, device="cuda")
    q.matvec_i8(yq, acc, dev(w), dev(mult), dev(xq), out, in_, shift=shift, outw=outw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_o)
    np.testing.assert_array_equal(yq.cpu().numpy(), yq_o)


def test_matvec_i8_rejects_bad_arguments(q, torch_cuda):
    torch = torch_cuda
    w = torch.zeros((8, 64), dtype=torch.int8, device="cuda")
    x = torch.zeros(64, dtype=torch.int8, device="cuda")
    m = torch.zeros(8, dtype=torch.int32, device="cuda")
    y = torch.zeros(8, dtype=torch.int32, device="cuda")
    for kw in ({"shift": 0}, {"shift": 63}, {"outw": 0}, {"outw": 33}):
        with pytest.raises(q.QHError):
            q.matvec_i8(y, y, w, m, x, 8, 64, **kw)
    with pytest.raises(q.QHError):
        q.matvec_i8(y, None, w, m, x, 8, 64)     # acc is required: the op keeps no buffers
    with pytest.raises(q.QHError):
        q.matvec_i8(y, y, w, m, x, 8, 60)        # in must be a multiple of 16


def _run(*args):
    return subprocess.run([SIM, *args], capture_output=True, text=True, timeout=120)


def test_sim_matvec_program(orc, q, blob, entries, tmp_path):
    p = str(tmp_path / "tv_gemv.bin")
    # a k_proj case in the Q14 int16 range: both reference criteria pass
    fx.write_tv_gemv(p, make_tv_gemv(orc, q, blob, entries, sw_scale=1 / 64))
    r = _run(p)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "PASS  gemv_i8" in r.stdout and "PASS  matvec_i8" in r.stdout
    # unscaled synthetic outputs (up to ~70) wrap in 16 bits, as the RTL bench would; 32 bits hold them
    tv = make_tv_gemv(orc, q, blob, entries)
    fx.write_tv_gemv(p, tv)
    r16 = _run(p)
    assert r16.returncode == 1 and "PASS  gemv_i8" in r16.stdout and r16.stdout.rstrip().endswith("FAIL")
    r32 = _run(p, "--outw", "32")
    assert r32.returncode == 0 and "PASS  matvec_i8" in r32.stdout, r32.stdout
    # a wrong reference accumulator is reported row by row
    tv.acc = tv.acc.copy()
    tv.acc[7] += 1
    fx.write_tv_gemv(p, tv)
    rb = _run(p, "--outw", "32")
    assert rb.returncode == 1 and "mismatch row 7" in rb.stdout
    # a truncated file is an input error
    with open(p, "r+b") as f:
        f.truncate(1000)
    assert _run(p).returncode == 2
