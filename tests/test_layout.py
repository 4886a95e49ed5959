"""Packed weight layout and the synthetic model (CPU).

The layout is pinned by the reference's committed artifacts: artifacts/weights.idx
(copied to tests/golden/weights.idx, all 320 lines) and the read-set header of
artifacts/access.txt ("471 ranges, 758248704 bytes").
"""
import hashlib
import os

import numpy as np

from conftest import GOLDEN


def test_idx_text_equals_reference_artifact(q):
    ref = open(os.path.join(GOLDEN, "weights.idx")).read()
    assert q.idx_text() == ref


def test_blob_size_is_manifest_total(q, entries):
    assert q.blob_size() == 758_618_112   # qwen35_int8.manifest.json total_bytes
    last = entries["embed_tokens.weight"]
    assert last.soff + last.snbytes == q.blob_size()


def test_read_set_matches_access_txt(entries):
    # emit_access.py:18-27: every payload plus every int8 scale block
    ranges = [(e.off, e.nbytes) for e in entries.values()]
    ranges += [(e.soff, e.snbytes) for e in entries.values() if e.dtype == 1]
    assert len(ranges) == 471
    assert sum(n for _, n in ranges) == 758_248_704


def test_alignment_and_scale_placement(entries):
    for e in entries.values():
        assert e.off % 4096 == 0, e.name
        if e.dtype == 1:
            assert e.soff == e.off + e.nbytes and e.snbytes == 4 * e.out, e.name
            assert e.in_ % 16 == 0, e.name   # 16-byte row chunks for the GEMV loads


def test_layer_schedule(entries):
    for layer in range(24):
        linear = f"layers.{layer}.linear_attn.in_proj_qkv.weight" in entries
        full = f"layers.{layer}.self_attn.q_proj.weight" in entries
        assert linear == (layer % 4 != 3) and full == (layer % 4 == 3)


def test_synthetic_blob_is_seeded_and_in_range(q, blob, entries):
    again = q.synth_blob(1234)
    assert hashlib.sha256(again.tobytes()).digest() == hashlib.sha256(blob.tobytes()).digest()
    other = q.synth_blob(1235)
    assert not np.array_equal(other[:1 << 20], blob[:1 << 20])

    def f32(name):
        e = entries[name]
        return blob[e.off:e.off + e.nbytes].view(np.float32)

    e = entries["layers.0.linear_attn.in_proj_qkv.weight"]
    w = blob[e.off:e.off + e.nbytes].view(np.int8)
    assert w.min() >= -127 and w.max() <= 127 and len(np.unique(w)) == 255
    s = blob[e.soff:e.soff + e.snbytes].view(np.float32)
    assert s.min() >= 1e-3 and s.max() <= 1e-2
    assert np.all(f32("layers.0.linear_attn.norm.weight") == 1.0)
    assert np.all(f32("layers.0.linear_attn.dt_bias") == 0.0)
    A = np.exp(f32("layers.0.linear_attn.A_log").astype(np.float64))
    assert A.min() >= 1.0 - 1e-6 and A.max() <= 16.0 + 1e-5
    # padding between tensors is zero
    e2 = entries["layers.0.linear_attn.in_proj_z.weight"]
    assert not blob[e.soff + e.snbytes:e2.off].any()


def test_engine_rejects_bad_inputs_before_touching_the_device(q, blob, idx):
    import ctypes

    lib = q._lib()
    h = ctypes.c_void_p()
    short = blob[:1 << 20]
    assert lib.qh_engine_create_from_memory(ctypes.c_void_p(short.ctypes.data), ctypes.c_size_t(short.size),
                                            None, 16, ctypes.byref(h)) == q.QH_EFORMAT
    bad = idx.replace("layers.5.mlp.up_proj.weight 120168448", "layers.5.mlp.up_proj.weight 120168449")
    assert lib.qh_engine_create_from_memory(ctypes.c_void_p(blob.ctypes.data), ctypes.c_size_t(blob.size),
                                            bad.encode(), 16, ctypes.byref(h)) == q.QH_EFORMAT
    trunc = "\n".join(idx.splitlines()[:300])
    assert lib.qh_engine_create_from_memory(ctypes.c_void_p(blob.ctypes.data), ctypes.c_size_t(blob.size),
                                            trunc.encode(), 16, ctypes.byref(h)) == q.QH_EFORMAT
    assert lib.qh_engine_create(b"/nonexistent/qwen35_int8.bin", None, 16, ctypes.byref(h)) == q.QH_EIO
