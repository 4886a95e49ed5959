"""Pack a Qwen3.5-0.8B text-LM snapshot into the int8 HBM blob the engine reads,
with the per-row weight quantisation on the MI355X.

    python -m qwen_fpga_amd.pack_weights [--snapshot DIR] [--out artifacts/qwen35_int8.bin]
                                          [--idx PATH] [--check]

The output is the reference's: the blob and ``<blob>.manifest.json`` of
scripts/pack_weights.py:50-114 and the ``weights.idx`` of
scripts/emit_weight_index.py:13-22.  Tensors follow the kernel read order
(pack_weights.py:27-47), each 4 KiB aligned; a tensor on the quantisation list
(golden/quant.py:21-39) is int8 [out, in] row-major followed by its fp32 [out]
per-row scales, every other tensor is fp32 as it is.  Weights are read from the
snapshot's ``*.safetensors`` the way golden/loader.py:41-75 reads them: the
vision tower (``model.visual.*``) and the MTP head (``mtp.*``) are dropped, the
``model.language_model.`` prefix is stripped, and BF16 is widened exactly (its
16 bits become the high half of an fp32).  A quantised tensor goes to the GPU
as it is stored (bfloat16 bits or fp32) and ``qh_quant_rows`` /
``qh_quant_rows_bf16`` produce its int8 rows and scales; there is no CPU
quantiser.  The blob's layout must be the one the engine reads: the emitted
idx is compared with the engine's own before anything is written.
"""
from __future__ import annotations

import argparse
import glob
import json
import os
import struct
import sys
from typing import Dict, List, NamedTuple, Optional

import numpy as np

ALIGN = 4096
DEFAULT_REPO = "~/.cache/huggingface/hub/models--Qwen--Qwen3.5-0.8B"

# golden/quant.py:21-33: the GEMV weights that carry the bandwidth
QUANT_SUFFIXES = (
    "in_proj_qkv.weight",
    "in_proj_z.weight",
    "linear_attn.out_proj.weight",
    "mlp.gate_proj.weight",
    "mlp.up_proj.weight",
    "mlp.down_proj.weight",
    "self_attn.q_proj.weight",
    "self_attn.k_proj.weight",
    "self_attn.v_proj.weight",
    "self_attn.o_proj.weight",
    "embed_tokens.weight",
)
# pack_weights.py:91-96: the config keys the manifest records
MANIFEST_CONFIG_KEYS = ("hidden_size", "num_hidden_layers", "layer_types", "head_dim", "num_attention_heads",
                        "num_key_value_heads", "intermediate_size", "vocab_size", "rms_norm_eps",
                        "linear_num_value_heads", "linear_key_head_dim", "linear_value_head_dim",
                        "linear_conv_kernel_dim", "rope_parameters")
_NP_DTYPES = {"F32": np.float32, "F16": np.float16, "I64": np.int64, "I32": np.int32}


def should_quant(name: str) -> bool:
    """A 2-D tensor with one of these suffixes is stored as per-row int8 (golden/quant.py:36-39)."""
    return any(name.endswith(s) for s in QUANT_SUFFIXES)


def find_snapshot(repo: str = DEFAULT_REPO) -> str:
    """The first snapshot directory with a config.json (golden/loader.py:22-26)."""
    hits = glob.glob(os.path.expanduser(f"{repo}/snapshots/*/config.json"))
    if not hits:
        raise FileNotFoundError(f"no snapshot with config.json under {repo}")
    return os.path.dirname(sorted(hits)[0])


def load_config(snapshot: str) -> dict:
    """config.json's text_config (golden/loader.py:78-80)."""
    with open(os.path.join(snapshot, "config.json")) as f:
        return json.load(f)["text_config"]


def read_order(cfg: dict) -> List[str]:
    """The order the decode kernels read the weights (pack_weights.py:27-47)."""
    order = []
    for i, kind in enumerate(cfg["layer_types"]):
        p = f"layers.{i}"
        order.append(f"{p}.input_layernorm.weight")
        if kind == "linear_attention":
            a = f"{p}.linear_attn"
            order += [f"{a}.in_proj_qkv.weight", f"{a}.in_proj_z.weight", f"{a}.in_proj_b.weight",
                      f"{a}.in_proj_a.weight", f"{a}.conv1d.weight", f"{a}.A_log", f"{a}.dt_bias",
                      f"{a}.norm.weight", f"{a}.out_proj.weight"]
        else:
            a = f"{p}.self_attn"
            order += [f"{a}.q_proj.weight", f"{a}.k_proj.weight", f"{a}.v_proj.weight", f"{a}.q_norm.weight",
                      f"{a}.k_norm.weight", f"{a}.o_proj.weight"]
        order.append(f"{p}.post_attention_layernorm.weight")
        order += [f"{p}.mlp.gate_proj.weight", f"{p}.mlp.up_proj.weight", f"{p}.mlp.down_proj.weight"]
    order += ["norm.weight", "embed_tokens.weight"]
    return order


class StTensor(NamedTuple):
    """One tensor of a safetensors file: where its bytes are and what they are."""
    path: str
    dtype: str          # safetensors dtype string ("BF16", "F32", ...)
    shape: tuple
    begin: int          # absolute byte offset of the data in the file
    end: int


def scan_snapshot(snapshot: str) -> Dict[str, StTensor]:
    """The text-LM tensors of every *.safetensors in the snapshot, by stripped name
    (golden/loader.py:41-64: headers parsed directly, vision and MTP tensors dropped)."""
    files = sorted(glob.glob(os.path.join(snapshot, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no .safetensors in {snapshot}")
    out: Dict[str, StTensor] = {}
    for path in files:
        with open(path, "rb") as f:
            hlen = struct.unpack("<Q", f.read(8))[0]
            hdr = json.loads(f.read(hlen))
        hdr.pop("__metadata__", None)
        base = 8 + hlen
        for name, meta in hdr.items():
            if name.startswith("model.visual") or name.startswith("mtp."):
                continue
            lo, hi = meta["data_offsets"]
            dt = meta["dtype"]
            if dt != "BF16" and dt not in _NP_DTYPES:
                raise ValueError(f"unhandled dtype {dt} for {name}")
            out[name.replace("model.language_model.", "")] = StTensor(path, dt, tuple(meta["shape"]), base + lo,
                                                                     base + hi)
    return out


def _raw(t: StTensor) -> np.ndarray:
    """The tensor's stored elements, memory-mapped (bfloat16 as uint16 bits)."""
    dt = np.dtype("<u2") if t.dtype == "BF16" else np.dtype(_NP_DTYPES[t.dtype]).newbyteorder("<")
    n = int(np.prod(t.shape)) if t.shape else 1
    if (t.end - t.begin) != n * dt.itemsize:
        raise ValueError(f"{t.path}: tensor of {t.end - t.begin} bytes, shape {t.shape} {t.dtype} needs "
                         f"{n * dt.itemsize}")
    return np.memmap(t.path, dtype=dt, mode="r", offset=t.begin, shape=(n,)).reshape(t.shape)


def widen_f32(t: StTensor) -> np.ndarray:
    """fp32 values of a stored tensor; BF16 is widened exactly (golden/loader.py:34-38)."""
    r = _raw(t)
    if t.dtype == "BF16":
        return (r.astype(np.uint32) << np.uint32(16)).view(np.float32)
    return np.asarray(r, dtype=np.float32)


def plan(order: List[str], shapes: Dict[str, tuple]) -> tuple:
    """Manifest entries (pack_weights.py:72-90) and the total size, without data."""
    entries, off = [], 0
    for name in order:
        shape = tuple(shapes[name])
        off += (-off) % ALIGN
        ent = {"name": name, "shape": list(shape), "offset": off}
        n = int(np.prod(shape)) if shape else 1
        if should_quant(name) and len(shape) == 2:
            ent["dtype"] = "int8"
            ent["nbytes"] = n
            ent["scale_offset"] = off + n
            ent["scale_nbytes"] = 4 * shape[0]
            off += n + 4 * shape[0]
        else:
            ent["dtype"] = "fp32"
            ent["nbytes"] = 4 * n
            off += 4 * n
        entries.append(ent)
    return entries, off


def idx_text(entries: List[dict]) -> str:
    """weights.idx: name off nbytes dtype(0 fp32 / 1 int8) scale_off scale_nbytes out in
    (scripts/emit_weight_index.py:13-22)."""
    lines = []
    for t in entries:
        sh = t["shape"]
        out_dim = sh[0] if len(sh) >= 1 else 0
        in_dim = sh[1] if len(sh) >= 2 else 0
        dtype = 1 if t["dtype"] == "int8" else 0
        lines.append(f"{t['name']} {t['offset']} {t['nbytes']} {dtype} {t.get('scale_offset', 0)} "
                     f"{t.get('scale_nbytes', 0)} {out_dim} {in_dim}\n")
    return "".join(lines)


def manifest_json(cfg: dict, entries: List[dict], total: int) -> dict:
    return {"config": {k: cfg[k] for k in MANIFEST_CONFIG_KEYS}, "align": ALIGN, "total_bytes": total,
            "tensors": entries}


def _device():
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("pack_weights quantises on the GPU: no HIP device is visible")
    return torch


def quant_tensor(t: StTensor, stream=None):
    """(int8 q [out, in], fp32 scale [out]) of a 2-D stored tensor, quantised on the GPU."""
    import qwen_fpga_amd as q

    torch = _device()
    rows, cols = t.shape
    r = _raw(t)
    # np.array: a writable host copy of the mapped bytes (bfloat16 as their int16 bits)
    if t.dtype == "BF16":
        w = torch.from_numpy(np.array(r).view(np.int16)).cuda()
    else:
        w = torch.from_numpy(np.array(r, dtype=np.float32)).cuda()
    qd = torch.empty((rows, cols), dtype=torch.int8, device="cuda")
    sd = torch.empty(rows, dtype=torch.float32, device="cuda")
    q.quant_rows(qd, sd, w, rows, cols, stream=stream)
    qh, sh = qd.cpu().numpy(), sd.cpu().numpy()
    if not np.all(np.isfinite(sh)):
        bad = int(np.flatnonzero(~np.isfinite(sh))[0])
        raise ValueError(f"{t.path}: row {bad} of a quantised tensor holds a NaN or an infinity")
    return qh, sh


def pack(snapshot: str, out: str, idx_path: Optional[str] = None, check: bool = False, verbose: bool = True) -> dict:
    """Write the blob, its manifest and weights.idx; return the manifest."""
    import qwen_fpga_amd as q

    cfg = load_config(snapshot)
    tensors = scan_snapshot(snapshot)
    order = read_order(cfg)
    missing = [k for k in order if k not in tensors]
    extra = [k for k in tensors if k not in order]
    if missing or extra:   # pack_weights.py:59-62
        raise SystemExit(f"the snapshot's tensors do not match the packing order: {len(missing)} absent "
                         f"(first {missing[:5]}), {len(extra)} not packed (first {extra[:5]})")
    entries, total = plan(order, {k: tensors[k].shape for k in order})
    idx = idx_text(entries)
    if idx != q.idx_text():
        raise ValueError("the snapshot's tensor shapes do not give the Qwen3.5-0.8B blob layout the engine reads")
    _device()

    if os.path.dirname(out):
        os.makedirs(os.path.dirname(out), exist_ok=True)
    with open(out, "wb") as f:
        for e in entries:
            t = tensors[e["name"]]
            if f.tell() != e["offset"]:
                f.write(b"\0" * (e["offset"] - f.tell()))
            if e["dtype"] == "int8":
                qh, sh = quant_tensor(t)
                f.write(qh.tobytes())
                f.write(sh.astype("<f4").tobytes())
            else:
                f.write(widen_f32(t).astype("<f4").tobytes())
        if f.tell() != total:
            raise RuntimeError(f"wrote {f.tell()} bytes, the layout has {total}")
    man = manifest_json(cfg, entries, total)
    mpath = os.path.splitext(out)[0] + ".manifest.json"
    with open(mpath, "w") as f:
        json.dump(man, f, indent=1)
    if idx_path is None:
        idx_path = os.path.join(os.path.dirname(out), "weights.idx")
    with open(idx_path, "w") as f:
        f.write(idx)
    if verbose:
        parts = {"int8 weights": sum(e["nbytes"] for e in entries if e["dtype"] == "int8"),
                 "row scales": sum(e.get("scale_nbytes", 0) for e in entries),
                 "fp32 tensors": sum(e["nbytes"] for e in entries if e["dtype"] == "fp32")}
        parts["alignment"] = total - sum(parts.values())
        print(f"{out}: {total:,} bytes in {len(entries)} tensors ("
              + ", ".join(f"{k} {v:,}" for k, v in parts.items()) + ")")
        print(f"{mpath}: manifest; {idx_path}: weight index")
    if check:
        worst = check_blob(out, entries, tensors)
        if verbose:
            print(f"  worst |packed - fakequant| = {worst:.3e}  {'OK' if worst == 0.0 else 'MISMATCH'}")
    return man


def check_blob(out: str, entries: List[dict], tensors: Dict[str, StTensor]) -> float:
    """Re-read the blob and compare every tensor with the snapshot: dequantised int8
    rows against a fresh device quantisation, fp32 tensors against the widened
    source (pack_weights.py:116-136).  Returns the worst absolute difference."""
    mm = np.memmap(out, dtype=np.uint8, mode="r")
    worst = 0.0
    for e in entries:
        t = tensors[e["name"]]
        if e["dtype"] == "int8":
            qb = np.frombuffer(mm[e["offset"]:e["offset"] + e["nbytes"]], dtype=np.int8).reshape(e["shape"])
            sb = np.frombuffer(mm[e["scale_offset"]:e["scale_offset"] + e["scale_nbytes"]], dtype="<f4")
            qq, ss = quant_tensor(t)
            d = float(np.abs(qb.astype(np.float32) * sb[:, None] - qq.astype(np.float32) * ss[:, None]).max())
        else:
            got = np.frombuffer(mm[e["offset"]:e["offset"] + e["nbytes"]], dtype="<f4").reshape(e["shape"])
            d = float(np.abs(got - widen_f32(t)).max()) if got.size else 0.0
        worst = max(worst, d)
    return worst


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="pack a Qwen3.5-0.8B snapshot into the int8 HBM blob")
    ap.add_argument("--snapshot", default=None, help=f"snapshot directory (default: the first under {DEFAULT_REPO})")
    ap.add_argument("--out", default="artifacts/qwen35_int8.bin")
    ap.add_argument("--idx", default=None, help="weights.idx path (default: next to the blob)")
    ap.add_argument("--check", action="store_true", help="re-read and verify round-trip")
    args = ap.parse_args(argv)
    snap = args.snapshot or find_snapshot()
    pack(snap, args.out, args.idx, check=args.check)
    return 0


if __name__ == "__main__":
    sys.exit(main())
