"""The packer (qwen_fpga_amd.pack_weights) and the quant_rows oracle, on the CPU.

The layout the packer plans is pinned to the reference's own artifacts: its
manifest (artifacts/qwen35_int8.manifest.json, copied to tests/golden) entry
for entry and its weights.idx byte for byte.  The quant_rows oracle
(golden/quant.py:43-49) is pinned by closed forms and by numpy's own float32
division and rint, an implementation independent of the C restatement.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN
from snapshot_util import PREFIX, bf16_bits, make_snapshot, reference_manifest, write_safetensors
from qwen_fpga_amd import pack_weights as pw


# ---------------------------------------------------------------- quant_rows oracle

def test_quant_rows_oracle_closed_forms(orc):
    w = np.array([[127.0, 63.5, -63.5, 0.5, -0.5, 1.5, -2.5, 0.0],   # s = 1: halves round to even
                  [0.0] * 8,                                          # amax 0: s = 1, q = 0
                  [-254.0, 1.0, 3.0, -3.0, 5.0, 0.0, 0.0, 0.0],       # s = 2
                  [1.0, np.nan, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],        # non-finite: s NaN, q 0
                  [np.inf, 1.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]], np.float32)
    q, s = orc.quant_rows(w)
    assert q[0].tolist() == [127, 64, -64, 0, 0, 2, -2, 0] and s[0] == 1.0
    assert not q[1].any() and s[1] == 1.0
    assert q[2].tolist() == [-127, 0, 2, -2, 2, 0, 0, 0] and s[2] == 2.0
    assert np.isnan(s[3]) and not q[3].any() and np.isnan(s[4]) and not q[4].any()


@pytest.mark.parametrize("rows,cols", [(7, 1024), (3, 3584), (5, 1000), (2, 4099)])
def test_quant_rows_oracle_equals_numpy_float32(orc, rows, cols):
    rng = np.random.default_rng(rows * cols)
    w = (bf16_bits(rng, rows * cols, 119).astype(np.uint32) << 16).view(np.float32).reshape(rows, cols)
    w[0, :8] = [0.5, 1.5, 2.5, -0.5, 0.25, 0.75, 0, 0]   # exact ties after the scale of row 0
    w[0, 8] = 127.0                                      # row 0: s = 1
    q, s = orc.quant_rows(w)
    amax = np.abs(w).max(axis=1)
    s_np = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q_np = np.rint(w / s_np[:, None]).clip(-127, 127).astype(np.int8)
    np.testing.assert_array_equal(s, s_np)
    np.testing.assert_array_equal(q, q_np)
    assert q[0, :6].tolist() == [0, 2, 2, 0, 0, 1]
    assert np.all(np.abs(q).max(axis=1) == 127)   # the row maximum maps to +-127


# ---------------------------------------------------------------- layout

def test_read_order_and_plan_equal_reference_manifest():
    man = reference_manifest()
    order = pw.read_order(man["config"])
    assert order == [t["name"] for t in man["tensors"]]
    entries, total = pw.plan(order, {t["name"]: tuple(t["shape"]) for t in man["tensors"]})
    assert entries == man["tensors"] and total == man["total_bytes"] == 758618112
    assert pw.manifest_json(man["config"], entries, total) == man


def test_quantised_tensors_are_the_reference_list():
    man = reference_manifest()
    for t in man["tensors"]:
        assert (t["dtype"] == "int8") == (pw.should_quant(t["name"]) and len(t["shape"]) == 2), t["name"]


def test_idx_text_equals_reference_weights_idx():
    man = reference_manifest()
    with open(os.path.join(GOLDEN, "weights.idx")) as f:
        assert pw.idx_text(man["tensors"]) == f.read()


def test_idx_text_equals_engine_layout(q):
    assert pw.idx_text(reference_manifest()["tensors"]) == q.idx_text()


# ---------------------------------------------------------------- snapshot reading

def test_scan_snapshot_names_dtypes_and_widening(tmp_path):
    rng = np.random.default_rng(3)
    bits = bf16_bits(rng, 6, 119)
    f32 = np.array([1.5, -2.0, 0.25], np.float32)
    write_safetensors(str(tmp_path / "a.safetensors"), [
        (PREFIX + "layers.0.mlp.up_proj.weight", "BF16", (2, 3), lambda: bits.astype("<u2").tobytes()),
        (PREFIX + "layers.0.linear_attn.A_log", "F32", (3,), lambda: f32.astype("<f4").tobytes()),
        ("model.visual.blocks.0.w", "BF16", (1, 2), lambda: b"\0" * 4),
        ("mtp.norm.weight", "BF16", (2,), lambda: b"\0" * 4),
    ])
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"text_config": {"hidden_size": 8}}, f)
    tensors = pw.scan_snapshot(str(tmp_path))
    assert sorted(tensors) == ["layers.0.linear_attn.A_log", "layers.0.mlp.up_proj.weight"]
    up = tensors["layers.0.mlp.up_proj.weight"]
    assert up.dtype == "BF16" and up.shape == (2, 3)
    # BF16 widening: the 16 bits become the high half of the fp32 (exact)
    w = pw.widen_f32(up)
    np.testing.assert_array_equal(w.view(np.uint32).ravel(), bits.astype(np.uint32) << 16)
    np.testing.assert_array_equal(pw.widen_f32(tensors["layers.0.linear_attn.A_log"]), f32)
    assert pw.load_config(str(tmp_path)) == {"hidden_size": 8}


def test_scan_snapshot_rejects_unknown_dtype_and_bad_sizes(tmp_path):
    write_safetensors(str(tmp_path / "a.safetensors"), [
        (PREFIX + "norm.weight", "BF16", (4,), lambda: b"\0" * 8)])
    p = str(tmp_path / "a.safetensors")
    raw = open(p, "rb").read()
    bad = raw.replace(b'"BF16"', b'"BOOL"')   # same length: a dtype the loader does not handle
    open(p, "wb").write(bad)
    with pytest.raises(ValueError, match="unhandled dtype"):
        pw.scan_snapshot(str(tmp_path))
    write_safetensors(p, [(PREFIX + "norm.weight", "BF16", (4,), lambda: b"\0" * 8)])
    t = pw.scan_snapshot(str(tmp_path))["norm.weight"]
    with pytest.raises(ValueError, match="needs"):
        pw._raw(t._replace(shape=(5,)))
    with pytest.raises(FileNotFoundError):
        pw.scan_snapshot(str(tmp_path / "nowhere"))


def test_find_snapshot(tmp_path):
    snap = tmp_path / "repo" / "snapshots" / "abc123"
    snap.mkdir(parents=True)
    (snap / "config.json").write_text("{}")
    assert pw.find_snapshot(str(tmp_path / "repo")) == str(snap)
    with pytest.raises(FileNotFoundError):
        pw.find_snapshot(str(tmp_path / "none"))


def test_pack_checks_names_and_shapes_before_the_gpu(q, tmp_path):
    # full-size snapshots whose data section is a hole: these checks read only headers
    snap = tmp_path / "snap"
    man = make_snapshot(str(snap), sparse=True)
    # one tensor missing, one extra: the reference's mismatch error
    tensors = [(PREFIX + t["name"], "BF16", tuple(t["shape"]), None) for t in man["tensors"][1:]]
    tensors.append((PREFIX + "lm_head.weight", "BF16", (4, 4), None))
    write_safetensors(str(snap / "model.safetensors"), tensors, sparse=True)
    with pytest.raises(SystemExit, match="do not match the packing order"):
        pw.pack(str(snap), str(tmp_path / "o2.bin"), verbose=False)
    # right names, a wrong shape: not the layout the engine reads
    tensors = [(PREFIX + t["name"], "BF16", tuple(t["shape"]), None) for t in man["tensors"]]
    tensors[1] = (tensors[1][0], "BF16", (6144, 512), None)
    write_safetensors(str(snap / "model.safetensors"), tensors, sparse=True)
    with pytest.raises(ValueError, match="layout"):
        pw.pack(str(snap), str(tmp_path / "o3.bin"), verbose=False)
    assert not (tmp_path / "o2.bin").exists() and not (tmp_path / "o3.bin").exists()


def test_pack_without_a_gpu_fails_loudly(q, tmp_path):
    import torch
    if torch.cuda.is_available():
        pytest.skip("checks the failure where no HIP device is visible")
    snap = tmp_path / "snap"
    make_snapshot(str(snap), sparse=True)
    with pytest.raises(RuntimeError, match="GPU"):
        pw.pack(str(snap), str(tmp_path / "out" / "qwen35_int8.bin"), verbose=False)
    assert not (tmp_path / "out" / "qwen35_int8.bin").exists()
