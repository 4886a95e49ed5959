"""Readers and writers for the reference's own test-vector files, and their
replay on the MI355X engine / op ABI.

* ``decode_ref.bin`` (scripts/export_decode_ref.py:47-53, read by
  hls/tb/tb_decode.cpp:73-82): int32 n, int32 fed[n], int32 argmax[n],
  float32 logits0[VOCAB] (the step-0 logits), little endian.  The reference
  testbench passes when every step's argmax matches and the step-0 logits are
  within 5e-2 (max |d|), tb_decode.cpp:104-109.
* ``tv_deltanet.bin`` (scripts/export_testvectors.py:55-60, read by
  hls/tb/tb_deltanet.cpp:57-71): float32 q, k, v [16][128] (q after l2norm and
  the 1/sqrt(128) scale), g, beta [16], S_in [16][128][128], o_core [16][128],
  S_out [16][128][128], one after another, 2,130,048 bytes.  The reference
  passes at max |d| < 2e-5 on o_core and S_out (tb_deltanet.cpp:88-91).

* ``tv_gemv.bin`` + ``tv_gemv.json`` (scripts/export_gemv_tv.py:62-72, read by
  rtl/tb/sim_gemv.cpp and sim_matvec.cpp): int8 x[IN], int8 w[OUT][IN], int32
  acc[OUT], float32 sx, float32 sw[OUT], float32 y[OUT] (y = float(acc)*sx*sw),
  with {"IN": 1024, "OUT": 512} in the json.  sim_gemv passes when every
  accumulator matches exactly; sim_matvec when the fixed-point output (SHIFT 16,
  OUTQ 14) is within 4 LSB of round(y * 2^14) (sim_matvec.cpp:78-86).

The same checks are the ``qh_tb_decode`` / ``qh_tb_deltanet`` / ``qh_sim_matvec``
programs in ``qwen_fpga_amd/bin``.
"""
import json
import os
from dataclasses import dataclass

import numpy as np

VOCAB = 248320
H, K, V = 16, 128, 128
TV_ORDER = ("q", "k", "v", "g", "beta", "S_in", "o_core", "S_out")
TV_SHAPES = {"q": (H, K), "k": (H, K), "v": (H, V), "g": (H,), "beta": (H,), "S_in": (H, K, V),
             "o_core": (H, V), "S_out": (H, K, V)}
TV_BYTES = 4 * sum(int(np.prod(s)) for s in TV_SHAPES.values())   # 2,130,048
DECODE_TOL = 5e-2   # step-0 logits, max |d| (tb_decode.cpp:109)
DELTA_TOL = 2e-5    # delta rule output and state, max |d| (tb_deltanet.cpp:89)
MATVEC_LSB_TOL = 4  # fixed-point output vs round(y * 2^OUTQ) (sim_matvec.cpp:82)


@dataclass
class DecodeRef:
    fed: np.ndarray      # int32 [n]
    argmax: np.ndarray   # int32 [n]
    logits0: np.ndarray  # float32 [VOCAB]


def read_decode_ref(path: str) -> DecodeRef:
    raw = np.fromfile(path, dtype=np.uint8)
    if raw.size < 4:
        raise ValueError(f"{path}: too short")
    n = int(raw[:4].view("<i4")[0])
    need = 4 + 8 * n + 4 * VOCAB
    if n <= 0 or raw.size != need:
        raise ValueError(f"{path}: {raw.size} bytes, n = {n} needs {need}")
    fed = raw[4:4 + 4 * n].view("<i4").astype(np.int32)
    am = raw[4 + 4 * n:4 + 8 * n].view("<i4").astype(np.int32)
    lg = raw[4 + 8 * n:].view("<f4").astype(np.float32)
    return DecodeRef(fed, am, lg)


def write_decode_ref(path: str, fed, argmax, logits0) -> None:
    fed = np.asarray(fed, dtype="<i4")
    argmax = np.asarray(argmax, dtype="<i4")
    logits0 = np.asarray(logits0, dtype="<f4")
    if fed.ndim != 1 or fed.shape != argmax.shape or logits0.shape != (VOCAB,):
        raise ValueError("fed and argmax must be [n], logits0 [VOCAB]")
    with open(path, "wb") as f:
        np.array([fed.size], "<i4").tofile(f)
        fed.tofile(f)
        argmax.tofile(f)
        logits0.tofile(f)


def read_tv_deltanet(path: str) -> dict:
    raw = np.fromfile(path, dtype="<f4")
    if raw.size * 4 != TV_BYTES:
        raise ValueError(f"{path}: {raw.size * 4} bytes, the layout needs {TV_BYTES}")
    out, o = {}, 0
    for name in TV_ORDER:
        n = int(np.prod(TV_SHAPES[name]))
        out[name] = raw[o:o + n].reshape(TV_SHAPES[name]).astype(np.float32)
        o += n
    return out


def write_tv_deltanet(path: str, tv: dict) -> None:
    with open(path, "wb") as f:
        for name in TV_ORDER:
            a = np.ascontiguousarray(tv[name], dtype="<f4")
            if a.shape != TV_SHAPES[name]:
                raise ValueError(f"{name}: shape {a.shape}, expected {TV_SHAPES[name]}")
            f.write(a.tobytes())


@dataclass
class GemvTv:
    x: np.ndarray      # int8 [IN]
    w: np.ndarray      # int8 [OUT, IN]
    acc: np.ndarray    # int32 [OUT]
    sx: float
    sw: np.ndarray     # float32 [OUT]
    y: np.ndarray      # float32 [OUT]


def read_tv_gemv(path: str) -> GemvTv:
    """tv_gemv.bin with its dimensions from the tv_gemv.json beside it (1024 x 512 without one)."""
    jpath = os.path.splitext(path)[0] + ".json"
    dims = {"IN": 1024, "OUT": 512}
    if os.path.exists(jpath):
        with open(jpath) as f:
            dims = json.load(f)
    n_in, n_out = int(dims["IN"]), int(dims["OUT"])
    raw = np.fromfile(path, dtype=np.uint8)
    need = n_in + n_out * n_in + 4 * n_out + 4 + 8 * n_out
    if raw.size != need:
        raise ValueError(f"{path}: {raw.size} bytes, IN={n_in} OUT={n_out} needs {need}")
    o = 0

    def take(n, dt):
        nonlocal o
        a = raw[o:o + n * np.dtype(dt).itemsize].view(dt)
        o += n * np.dtype(dt).itemsize
        return a

    x = take(n_in, "<i1").astype(np.int8)
    w = take(n_out * n_in, "<i1").astype(np.int8).reshape(n_out, n_in)
    acc = take(n_out, "<i4").astype(np.int32)
    sx = float(take(1, "<f4")[0])
    sw = take(n_out, "<f4").astype(np.float32)
    y = take(n_out, "<f4").astype(np.float32)
    return GemvTv(x, w, acc, sx, sw, y)


def write_tv_gemv(path: str, tv: GemvTv) -> None:
    n_out, n_in = tv.w.shape
    with open(path, "wb") as f:
        np.asarray(tv.x, "<i1").tofile(f)
        np.asarray(tv.w, "<i1").reshape(-1).tofile(f)
        np.asarray(tv.acc, "<i4").tofile(f)
        np.array([tv.sx], "<f4").tofile(f)
        np.asarray(tv.sw, "<f4").tofile(f)
        np.asarray(tv.y, "<f4").tofile(f)
    with open(os.path.splitext(path)[0] + ".json", "w") as f:
        json.dump({"IN": n_in, "OUT": n_out}, f)


def replay_decode_ref(engine, ref: DecodeRef) -> dict:
    """Decode ``ref.fed`` from a reset state; the tb_decode criteria."""
    engine.reset()
    am = []
    lg0 = None
    for i, tok in enumerate(ref.fed.tolist()):
        a, lg = engine.decode_token(int(tok), want_logits=(i == 0))
        am.append(a)
        if i == 0:
            lg0 = lg
    mism = int(np.sum(np.array(am) != ref.argmax))
    d = np.abs(lg0.astype(np.float64) - ref.logits0.astype(np.float64))
    return {"argmax": am, "mismatches": mism, "max_abs": float(d.max()), "mean_abs": float(d.mean()),
            "pass": mism == 0 and float(d.max()) < DECODE_TOL}


def replay_tv_deltanet(tv: dict, stream=None) -> dict:
    """Run qh_delta_rule_layer on (q, k, v, g, beta, S_in); the tb_deltanet criteria."""
    import torch

    import qwen_fpga_amd as q

    dev = torch.device("cuda")
    t = {k_: torch.from_numpy(np.ascontiguousarray(tv[k_])).to(dev) for k_ in ("q", "k", "v", "g", "beta")}
    S = torch.from_numpy(np.ascontiguousarray(tv["S_in"])).to(dev)
    out = torch.empty((H, V), dtype=torch.float32, device=dev)
    q.delta_rule_layer(t["q"], t["k"], t["v"], t["g"], t["beta"], S, out, stream=stream)
    torch.cuda.synchronize()
    do = float(np.abs(out.cpu().numpy().astype(np.float64) - tv["o_core"]).max())
    ds = float(np.abs(S.cpu().numpy().astype(np.float64) - tv["S_out"]).max())
    return {"max_abs_out": do, "max_abs_S": ds, "pass": do < DELTA_TOL and ds < DELTA_TOL}
