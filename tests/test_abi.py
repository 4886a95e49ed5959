"""The C ABI library loads, exports every declared entry point, and rejects bad
arguments on the host (CPU; nothing here launches device work)."""
import ctypes
import os
import subprocess

import pytest

from conftest import ROOT


def test_library_exports_every_header_function(q):
    names = q.header_functions()
    assert len(names) >= 38
    lib = q._lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_strerror(q):
    lib = q._lib()
    assert lib.qh_strerror(0) == b"ok"
    assert b"invalid" in lib.qh_strerror(q.QH_EINVAL)
    assert b"range" in lib.qh_strerror(q.QH_ERANGE)


@pytest.mark.parametrize("call", [
    lambda L, p: L.qh_gemv_i8(None, p, p, p, 8, 1024, None),
    lambda L, p: L.qh_gemv_i8(p, p, p, p, 8, 1000, None),      # in not a multiple of 16
    lambda L, p: L.qh_gemv_i8(p, p, p, p, 0, 1024, None),
    lambda L, p: L.qh_gemv_i8(p, p, p, p, 8, 8192, None),      # in beyond 4096
    lambda L, p: L.qh_gemv_f32(p, None, p, 8, 1024, None),
    lambda L, p: L.qh_rmsnorm(p, None, p, 1024, ctypes.c_float(1e-6), None),
    lambda L, p: L.qh_rmsnorm(p, p, p, 0, ctypes.c_float(1e-6), None),
    lambda L, p: L.qh_l2norm(None, 128, None),
    lambda L, p: L.qh_conv1d_step(p, p, None, p, None),
    lambda L, p: L.qh_quant_act(p, None, p, 16, None),
    lambda L, p: L.qh_gemv_i8_w8a8(p, None, p, p, p, None, 8, 1024, None),
    lambda L, p: L.qh_deltanet_layer(p, p, None, None, None, None, p, p, p, p, None, p, p, None),
    lambda L, p: L.qh_mlp_layer(p, p, None, None, None, None),
    lambda L, p: L.qh_engine_set_mode(None, 1),
    lambda L, p: L.qh_engine_reset(None),
    lambda L, p: L.qh_decode_token(None, 5, None, p),
])
def test_argument_errors(q, call):
    buf = ctypes.create_string_buffer(4096 + 16)
    p = ctypes.c_void_p((ctypes.addressof(buf) + 15) & ~15)   # aligned host stand-in, never dereferenced
    assert call(q._lib(), p) == q.QH_EINVAL


def test_range_errors(q):
    buf = ctypes.create_string_buffer(64)
    p = ctypes.c_void_p(ctypes.addressof(buf))
    L = q._lib()
    assert L.qh_embed_row(p, p, p, -1, 1024, None) == q.QH_ERANGE
    assert L.qh_rope_cos_sin(-3, p, p, None) == q.QH_ERANGE


def test_run_hls_cli_usage_and_missing_blob(tmp_path):
    exe = os.path.join(ROOT, "qwen_fpga_amd", "bin", "qh_run_hls")
    assert os.path.exists(exe), "CLI not built"
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 2 and "usage" in r.stderr
    ids = tmp_path / "ids.txt"
    ids.write_text("1 2 3\n")
    r = subprocess.run([exe, str(tmp_path / "missing.bin"), str(ids), "4"], capture_output=True, text=True)
    assert r.returncode == 2 and "engine" in r.stderr
    empty = tmp_path / "empty.txt"
    empty.write_text("")
    r = subprocess.run([exe, str(tmp_path / "missing.bin"), str(empty), "4"], capture_output=True, text=True)
    assert r.returncode == 2 and "no prompt ids" in r.stderr
