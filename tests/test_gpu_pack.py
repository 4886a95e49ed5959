"""Per-row weight quantisation on the MI355X and the packer end to end.

qh_quant_rows / qh_quant_rows_bf16 are compared bit for bit with the oracle's
quant_rows (golden/quant.py:43-49) on every code path of the kernel (rows held
in registers; the two-pass form for rows that are long, not a multiple of four
or misaligned), with exact ties, zero rows and non-finite rows.  The packer
turns a full-size synthetic snapshot (checkpoint names, bfloat16 values, an F32
A_log, vision and MTP tensors to drop) into the blob, manifest and weights.idx;
they must equal the reference's manifest and idx and the oracle's quantisation
of the widened weights, and the engine must decode the packed blob exactly as
the oracle does -- through the C ABI and through the qh_tb_decode testbench.
"""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, ROOT
from snapshot_util import bf16_bits, make_snapshot, reference_manifest
from qwen_fpga_amd import fixtures as fx
from qwen_fpga_amd import pack_weights as pw

pytestmark = pytest.mark.gpu


def _same_scales(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    return np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)])


def _rows(rng, rows, cols):
    """fp32 rows of bfloat16 values, with a zero row, an exact-tie row, a NaN row and an inf row."""
    w = (bf16_bits(rng, rows * cols, 119).astype(np.uint32) << 16).view(np.float32).reshape(rows, cols).copy()
    w[1] = 0.0
    w[2, :6] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5]
    w[2, 6:] = 0.25
    w[3, cols // 2] = np.nan
    w[4, 0] = -np.inf
    return w


@pytest.mark.parametrize("rows,cols,off", [(37, 1024, 0), (9, 3584, 0), (6, 2048, 0), (6, 1000, 0), (5, 5000, 0),
                                           (8, 1024, 1)],
                         ids=["1024", "3584", "2048", "1000-two-pass", "5000-two-pass", "misaligned"])
def test_quant_rows_matches_oracle(q, orc, torch_cuda, rows, cols, off):
    torch = torch_cuda
    rng = np.random.default_rng(rows * cols + off)
    w = _rows(rng, rows, cols)
    q_o, s_o = orc.quant_rows(w)
    # fp32 input; off shifts every pointer by one element (the two-pass form)
    buf = torch.zeros(rows * cols + 16, dtype=torch.float32, device="cuda")
    wd = buf[off:off + rows * cols].view(rows, cols)
    wd.copy_(torch.from_numpy(w))
    qb = torch.full((rows * cols + 16,), 99, dtype=torch.int8, device="cuda")
    qd = qb[off:off + rows * cols].view(rows, cols)
    sd = torch.empty(rows, dtype=torch.float32, device="cuda")
    q.quant_rows(qd, sd, wd, rows, cols)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(qd.cpu().numpy(), q_o)
    assert _same_scales(sd.cpu().numpy(), s_o)
    assert (qb[:off].cpu().numpy() == 99).all() and (qb[off + rows * cols:].cpu().numpy() == 99).all()
    # bfloat16 bits of the same values
    bits = (w.view(np.uint32) >> 16).astype(np.uint16)
    bbuf = torch.zeros(rows * cols + 16, dtype=torch.int16, device="cuda")
    bd = bbuf[off:off + rows * cols].view(rows, cols)
    bd.copy_(torch.from_numpy(bits.view(np.int16)))
    qd.fill_(99)
    q.quant_rows(qd, sd, bd, rows, cols)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(qd.cpu().numpy(), q_o)
    assert _same_scales(sd.cpu().numpy(), s_o)
    assert np.isnan(s_o[3]) and np.isnan(s_o[4]) and s_o[1] == 1.0 and s_o[2] == 1.0


def test_quant_rows_rejects_bad_arguments(q, torch_cuda):
    torch = torch_cuda
    w = torch.zeros((4, 8), device="cuda")
    qd = torch.empty((4, 8), dtype=torch.int8, device="cuda")
    sd = torch.empty(4, device="cuda")
    for args in ((qd, sd, w, 0, 8), (qd, sd, w, 4, 0), (None, sd, w, 4, 8), (qd, None, w, 4, 8)):
        with pytest.raises(q.QHError):
            q.quant_rows(*args)


# ---------------------------------------------------------------- the packer, end to end

FED = [11, 2222, 248000, 5, 77, 77]


@pytest.fixture(scope="module")
def packed(tmp_path_factory, torch_cuda):
    d = tmp_path_factory.mktemp("pack")
    snap = d / "snapshot"
    make_snapshot(str(snap), seed=5)
    out = d / "artifacts" / "qwen35_int8.bin"
    man = pw.pack(str(snap), str(out), check=False, verbose=False)
    return {"dir": d, "snap": str(snap), "blob": str(out), "idx": str(d / "artifacts" / "weights.idx"), "man": man}


def test_pack_outputs_equal_reference_layout(packed):
    ref = reference_manifest()
    with open(os.path.splitext(packed["blob"])[0] + ".manifest.json") as f:
        assert json.load(f) == ref == packed["man"]
    with open(packed["idx"]) as f, open(os.path.join(GOLDEN, "weights.idx")) as g:
        assert f.read() == g.read()
    assert os.path.getsize(packed["blob"]) == ref["total_bytes"]


def test_packed_blob_equals_oracle_quantisation(orc, packed):
    tensors = pw.scan_snapshot(packed["snap"])
    mm = np.memmap(packed["blob"], dtype=np.uint8, mode="r")
    end = 0
    for e in packed["man"]["tensors"]:
        assert not mm[end:e["offset"]].any(), f"padding before {e['name']}"
        w = pw.widen_f32(tensors[e["name"]])
        if e["dtype"] == "int8":
            q_o, s_o = orc.quant_rows(w)
            qb = np.frombuffer(mm[e["offset"]:e["offset"] + e["nbytes"]], dtype=np.int8).reshape(e["shape"])
            sb = np.frombuffer(mm[e["scale_offset"]:e["scale_offset"] + e["scale_nbytes"]], dtype="<f4")
            np.testing.assert_array_equal(qb, q_o, err_msg=e["name"])
            np.testing.assert_array_equal(sb, s_o, err_msg=e["name"])
            end = e["scale_offset"] + e["scale_nbytes"]
        else:
            got = np.frombuffer(mm[e["offset"]:e["offset"] + e["nbytes"]], dtype="<f4").reshape(e["shape"])
            np.testing.assert_array_equal(got, w, err_msg=e["name"])
            end = e["offset"] + e["nbytes"]
    assert end == len(mm)
    assert pw.check_blob(packed["blob"], packed["man"]["tensors"], tensors) == 0.0


@pytest.mark.parametrize("mode", [0, 1], ids=["w8a16", "w8a8"])
def test_engine_decodes_packed_blob_like_oracle(q, orc, packed, mode):
    blob = np.fromfile(packed["blob"], dtype=np.uint8)
    with open(packed["idx"]) as f:
        idx = f.read()
    m = orc.Model(blob, idx, max_ctx=len(FED))
    e = q.Engine(path=packed["blob"], idx=packed["idx"], max_ctx=len(FED), mode=mode)
    try:
        for step, tok in enumerate(FED):
            am, lg = e.decode_token(tok, want_logits=True)
            am_o, lg_o = m.decode_token(tok, mode=mode, order=orc.ORDER_DEV, want_logits=True)
            np.testing.assert_array_equal(lg.view(np.uint32), lg_o.view(np.uint32), err_msg=f"step {step}")
            assert am == am_o, (step, am, am_o)
    finally:
        e.close()
        m.close()


def test_tb_decode_on_packed_blob(orc, packed):
    """pack -> decode_ref.bin (reference order) -> qh_tb_decode, the reference's csim_decode flow."""
    blob = np.fromfile(packed["blob"], dtype=np.uint8)
    with open(packed["idx"]) as f:
        idx = f.read()
    m = orc.Model(blob, idx, max_ctx=len(FED))
    am, lg0 = [], None
    for i, t in enumerate(FED):
        a, lg = m.decode_token(t, mode=orc.W8A16, order=orc.ORDER_REF, want_logits=(i == 0))
        am.append(a)
        lg0 = lg if i == 0 else lg0
    m.close()
    ref = str(packed["dir"] / "artifacts" / "decode_ref.bin")
    fx.write_decode_ref(ref, FED, am, lg0)
    r = subprocess.run([os.path.join(ROOT, "qwen_fpga_amd", "bin", "qh_tb_decode"), packed["blob"], packed["idx"], ref],
                       capture_output=True, text=True, timeout=180)
    assert r.returncode == 0 and "PASS" in r.stdout, r.stdout + r.stderr


def test_run_hls_wrapper_on_packed_snapshot(q, packed, tmp_path, capsys):
    """run_hls.py's flow: tokenizer from the snapshot, blob packed on first use, qh_run_hls spawned."""
    from transformers import AutoTokenizer

    from qwen_fpga_amd import run_hls
    from snapshot_util import IM_END, IM_START, write_tokenizer

    write_tokenizer(packed["snap"])
    tok = AutoTokenizer.from_pretrained(packed["snap"])
    fresh = str(tmp_path / "artifacts")   # no blob yet: the wrapper packs it
    for raw, art, ids in ((True, os.path.dirname(packed["blob"]), [1, 2]),
                          (False, fresh, [IM_START, 3, 1, 2, IM_END, IM_START, 4])):
        rc = run_hls.main(["-p", "hello world", "-n", "6", "--snapshot", packed["snap"], "--artifacts", art]
                          + (["--raw"] if raw else []))
        out = capsys.readouterr().out
        assert rc == 0, out
        with open(os.path.join(art, "prompt_ids.txt")) as f:
            assert f.read() == " ".join(map(str, ids))
        e = q.Engine(path=packed["blob"], idx=packed["idx"], max_ctx=32)
        try:
            gen = e.generate(ids, 6, eos=IM_END)
        finally:
            e.close()
        assert out.split("answer   : ", 1)[1].split("\n", 1)[0] == tok.decode(gen)
    with open(os.path.join(fresh, "qwen35_int8.bin"), "rb") as f, open(packed["blob"], "rb") as g:
        assert f.read() == g.read()
