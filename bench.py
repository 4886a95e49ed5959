#!/usr/bin/env python3
"""Batch-1 decode throughput of the 24-layer int8 hybrid model on one MI355X.

Workload ("C5"): the full Qwen3.5-0.8B-shaped model
with seeded synthetic int8 weights in the packed pack_weights.py layout; a
64-token seeded prompt is fed through the recurrent path (untimed), then
`--steps` greedy decode steps are timed (default 512, so the KV cache grows to
576).  One "step" is one decode token: embed, 24 layers, final norm, the tied
248320x1024 int8 head and its on-device argmax, run by the persistent
kernel (default: one cooperative launch for all timed tokens, the token fed
back on the device) or, with --exec graph, replayed as a hipGraph per token.

Prints one JSON line with tok/s, the achieved HBM bandwidth per token against
the 8 TB/s MI355X peak, the roofline of the dominant kernel, and the reference
CPU path (the reference's hls/src decode top compiled natively, one core) on a
bounded sample.  The dominant kernel is the one the timed region launches: the
persistent kernel (its launch duration from HIP events on the engine stream
around the cooperative launch), or, with --exec graph, the LM head (in its
decode-step context, HIP events stamped at the kernel's own start and end).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_GBS = 8000.0          # MI355X HBM3E, AMD published
FLOOR_BYTES = 758_248_704  # int8 payload + scales + fp32 tensors read per token (artifacts/access.txt:1)
HEAD_BYTES = 248320 * 1024 + 248320 * 4 + 2 * 4096   # int8 rows + scales + h + final-norm gain


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "head_kernel_decode_c5_pmc_traffic.md")
PERSIST_TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "persist_kernel_decode_c5_pmc_traffic.md")


def profile_fields(path):
    """The `key: value` lines of a committed rocprofv3 summary (FETCH_SIZE + WRITE_SIZE, each
    scaled by a copy of known size; the counters cannot be read from inside this process)."""
    out = {}
    try:
        for line in open(path):
            if ":" in line and not line.startswith((" ", "|", "#", "`")):
                k, v = line.split(":", 1)
                if k and " " not in k.strip():
                    out[k.strip()] = v.strip()
    except OSError:
        pass
    return out


def source_hash():
    """Hash of the library's sources (qwen_fpga_amd/csrc, include/qh_decode.h): the build a
    committed counter summary was taken from."""
    import hashlib
    h = hashlib.sha256()
    d = os.path.join(ROOT, "qwen_fpga_amd", "csrc")
    names = sorted(n for n in os.listdir(d) if n.endswith((".hip", ".hpp", ".cpp", ".h")) or n == "Makefile")
    for n in names + ["../../include/qh_decode.h"]:
        with open(os.path.join(d, n), "rb") as f:
            h.update(n.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def traffic_of(path, workload, bytes_per_launch):
    """(traffic bytes per launch, source) from a committed counter summary, used only when it was
    taken on this workload and this build (source hash); otherwise (None, the reason)."""
    f = profile_fields(path)
    rel = os.path.relpath(path, ROOT)
    if "traffic_bytes_per_launch" not in f:
        return None, f"none: no counter summary ({rel})"
    if f.get("workload") != workload:
        return None, f"none: {rel} is of workload '{f.get('workload')}', this run '{workload}'"
    if f.get("source") != source_hash():
        return None, f"none: {rel} is of another build (source {f.get('source')}, this {source_hash()})"
    return int(f["traffic_bytes_per_launch"]), rel


def full_bytes(T: int) -> int:
    """Algorithmic bytes of one token with T cached positions: weights + DeltaNet
    state r/w + conv history r/w + KV read (T+1 rows) and write."""
    return 799_536_384 + 24_576 * (T + 1)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prompt", type=int, default=64)
    ap.add_argument("--mode", choices=["w8a8", "w8a16"], default="w8a8")
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--cpu-tokens", type=int, default=8, help="reference CPU decode sample (tokens)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the per-config C1-C4 op measurements")
    ap.add_argument("--configs-only", action="store_true",
                    help="only the C1-C4 section (with --no-c4: the workload of its committed kernel trace)")
    ap.add_argument("--no-c4", action="store_true", help="config section without C4 (no cooperative launch)")
    ap.add_argument("--profile-steps", type=int, default=16)
    ap.add_argument("--exec", dest="exec_kind", choices=["graph", "persistent"], default="persistent",
                    help="persistent: one cooperative launch runs every token, stages hand vectors over "
                         "through tagged buffers; graph: one hipGraph of per-stage kernels per token")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs batch-1 decode on a single MI355X "
              "(the independent unit is a whole sequence: one engine per GPU, no exchange)", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import qwen_fpga_amd as q

    torch.cuda.set_device(0)
    blob = q.synth_blob(args.seed)
    idx = q.idx_text()
    if args.configs_only:
        print(json.dumps({"configs": op_configs(q, torch, np, blob, idx, args.mode, not args.no_c4)}), flush=True)
        return 0
    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, q.VOCAB, size=args.prompt).astype(np.int32).tolist()
    mode = q.MODE_W8A8 if args.mode == "w8a8" else q.MODE_W8A16
    max_ctx = args.prompt + max(args.steps, args.warmup) + args.profile_steps + 2
    eng = q.Engine(blob, idx=idx, max_ctx=max_ctx, mode=mode)
    try:
        eng.set_exec(q.EXEC_PERSISTENT if args.exec_kind == "persistent" else q.EXEC_GRAPH)
    except q.QHError as exc:   # no cooperative launch on this device: the graph runs the same kernels
        print(f"persistent executor unavailable ({exc}); using the graph executor", file=sys.stderr)
        eng.set_exec(q.EXEC_GRAPH)

    # warmup: graph instantiation + a short run from a fresh state
    eng.reset()
    eng.generate(prompt, args.warmup)
    torch.cuda.synchronize()

    # timed: prefill (untimed), then exactly `steps` decode steps
    eng.reset()
    eng.generate(prompt, 0)
    cur = eng.last_argmax
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = eng.generate([cur], args.steps - 1)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    if len(out) != args.steps - 1:
        print(f"generated {len(out)} of {args.steps - 1} tokens", file=sys.stderr)
        return 1
    dt = t1 - t0
    tok_s = args.steps / dt
    T0 = args.prompt
    mean_full = sum(full_bytes(T0 + i) for i in range(args.steps)) / args.steps
    achieved_gbs = FLOOR_BYTES * tok_s / 1e9

    persistent = eng.exec_kind == q.EXEC_PERSISTENT
    if persistent:
        # the timed region is one cooperative launch of persist_kernel: its
        # algorithmic bytes (every token's weights, state and KV traffic) over the
        # launch duration from HIP events recorded around it on the engine stream
        launch_ms = eng.last_launch_ms
        launch_bytes = int(mean_full * args.steps)
        wl = f"steps={args.steps} prompt={args.prompt} warmup={args.warmup} mode={args.mode} exec=persistent"
        traffic, traffic_src = traffic_of(PERSIST_TRAFFIC_PROFILE, wl, launch_bytes)
        limiter = "latency of the 127 dependent all-to-all stage hand-overs per token and their post-arrival chains"
        if traffic:
            limiter += f" (HBM traffic {traffic / launch_bytes:.3f}x the algorithmic bytes)"
        roofline = {
            "kernel": "persist_kernel (every stage of every token in one cooperative launch)",
            # the only roofline of a ~2 op/B int8 GEMV datapath
            "bound": "hbm",
            "limiter": limiter,
            "achieved": round(launch_bytes / (launch_ms * 1e-3) / 1e9, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(launch_bytes / (launch_ms * 1e-3) / 1e9 / PEAK_GBS, 4),
            # FETCH_SIZE + WRITE_SIZE of this launch (committed summary of this workload and build)
            "traffic": traffic,
            "traffic_source": traffic_src,
            "duration_us": round(launch_ms * 1e3, 1),
            "bytes_per_launch": launch_bytes,
            "tokens_per_launch": args.steps,
        }
    else:
        # dominant kernel: the LM head inside each profiled step (after the 24 layers,
        # so its weights are not cache-resident), HIP events stamped at kernel start / end
        step_ms, head_ms = eng.profile(args.profile_steps)
        head_gbs = HEAD_BYTES / (head_ms * 1e-3) / 1e9
        roofline = {
            "kernel": "head_kernel (tied 248320x1024 int8 LM head + block argmax)",
            "bound": "hbm",
            "achieved": round(head_gbs, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(head_gbs / PEAK_GBS, 4),
            "traffic": traffic_of(TRAFFIC_PROFILE, f"graph head, steps={args.profile_steps}", HEAD_BYTES)[0],
            "traffic_source": traffic_of(TRAFFIC_PROFILE, f"graph head, steps={args.profile_steps}", HEAD_BYTES)[1],
            "duration_us": round(head_ms * 1e3, 2),
            "bytes_per_launch": HEAD_BYTES,
            "stream_step_ms": round(step_ms, 4),
        }

    line = {
        "metric": "batch-1 decode tok/s (24-layer int8) + achieved HBM GB/s vs peak",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * dt / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if mode == q.MODE_W8A8 else "int8xf32",
        "data": "synthetic (seeded random-init int8 weights in the pack_weights.py layout)",
        "config": {
            "workload": "C5: full 24-layer Qwen3.5-0.8B-shaped decode, batch 1, "
                        f"{args.prompt}-token prompt then {args.steps} greedy steps (KV to "
                        f"{args.prompt + args.steps})",
            "act_mode": args.mode,
            "exec": "persistent" if persistent else ("graph" if args.exec_kind == "graph" else "graph (fallback)"),
            "bytes_per_token_floor": FLOOR_BYTES,
            "bytes_per_token_full_mean": int(mean_full),
        },
        "achieved_hbm_gbs": round(achieved_gbs, 1),
        "achieved_hbm_gbs_full": round(mean_full * tok_s / 1e9, 1),
        "hbm_peak_gbs": PEAK_GBS,
        "frac_of_roofline": round(achieved_gbs / PEAK_GBS, 4),
        "roofline": roofline,
    }
    # the other activation mode on the same executor and workload (reported beside `value`)
    other = q.MODE_W8A16 if mode == q.MODE_W8A8 else q.MODE_W8A8
    eng.set_mode(other)
    eng.reset()
    eng.generate(prompt, 0)
    cur = eng.last_argmax
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eng.generate([cur], args.steps - 1)
    torch.cuda.synchronize()
    line["value_" + ("w8a16" if other == q.MODE_W8A16 else "w8a8")] = round(args.steps / (time.perf_counter() - t0), 2)
    eng.close()

    if not args.no_configs:
        line["configs"] = op_configs(q, torch, np, blob, idx, args.mode)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(blob, idx, prompt, args.cpu_tokens, args.mode)
    print(json.dumps(line), flush=True)
    return 0


def _timed(torch, fn, iters):
    """Median microseconds of one fn(i) call, from a pair of HIP events recorded right before
    and after it on the stream it runs on (the host enqueues slower than these kernels run,
    so timing a whole loop would time the host)."""
    s = torch.cuda.current_stream()
    fn()
    s.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for i, (a, b) in enumerate(ev):
        a.record(s)
        fn(i)
        b.record(s)
    s.synchronize()
    t = sorted(a.elapsed_time(b) * 1e3 for a, b in ev)
    return t[len(t) // 2]


def _rate(bytes_per_unit, us):
    gbs = bytes_per_unit / (us * 1e-6) / 1e9
    return {"us": round(us, 2), "bytes": int(bytes_per_unit), "gbs": round(gbs, 1), "frac": round(gbs / PEAK_GBS, 4)}


# The config section's timed phases, in order (prof_summary --phases); before each the GPU idles
# 0.2 s, so a kernel trace of `bench.py --configs-only` splits into exactly these phases.
CONFIG_PHASES = ["C1 3584x1024", "C1 1024x3584", "C1 6144x1024", "C2", "C3 T=512", "C3 T=4096", "C3 T=32768"]
CONFIG_PROFILE = os.path.join(ROOT, "profiles", "op_configs_c1_c3_kernel_trace.md")
ROTATE_BYTES = 300_000_000   # > the 256 MB Infinity Cache: no unit is served from it


def _gap(torch):
    torch.cuda.synchronize()
    time.sleep(0.2)


def config_profile():
    """{phase label: kernel us per call}, and the workload and source lines, of the committed
    summary of a kernel trace of this config section (CONFIG_PROFILE), or ({}, None, None)."""
    out, wl, src = {}, None, None
    try:
        for line in open(CONFIG_PROFILE):
            if line.startswith("workload:"):
                wl = line.split(":", 1)[1].strip()
            elif line.startswith("source:"):
                src = line.split(":", 1)[1].strip()
            elif line.startswith("config ") and "kernel_us_per_call" in line:
                label = line[len("config "):line.index(":")]
                out[label] = float(line.split("kernel_us_per_call")[1].split()[0])
    except OSError:
        pass
    return out, wl, src


def op_configs(q, torch, np, blob, idx, act_mode, with_c4=True):
    """BASELINE.json configs C1-C4, each unit's bytes the algorithmic count of the config
    (weights + scales + activations + state / cache traffic).  C1-C3 run the op-level C ABI with
    no allocation inside a timed call (C2 and C3 take their scratch from a workspace / the
    library's static array) and rotate through > 256 MB of weights, states and caches, so no
    call is served by the 256 MB Infinity Cache; `us` is a HIP-event pair around one op call
    (its launches included), `kernel_us` the op's kernel time per call from the committed kernel
    trace of this section (profiles/op_configs_c1_c3_kernel_trace.md).  C4 runs on the persistent
    executor: layers 0-3 inside the decode step, timed by the kernel's own stage clock."""
    dev = torch.device("cuda")
    w8a8 = act_mode == "w8a8"
    rng = np.random.default_rng(7)
    prof, prof_wl, prof_src = config_profile()
    workload = f"act_mode={act_mode} rotate_bytes={ROTATE_BYTES} phases={','.join(CONFIG_PHASES)}"
    matches = prof_wl == workload and prof_src == source_hash()
    out = {"workload": workload}

    def entry(label, nbytes, us, **kw):
        d = dict(_rate(nbytes, us), **kw)
        k = prof.get(label) if matches else None
        d["kernel_us"] = k
        if k:
            d["kernel_gbs"] = round(nbytes / (k * 1e-6) / 1e9, 1)
            d["kernel_frac"] = round(nbytes / (k * 1e-6) / 1e9 / PEAK_GBS, 4)
        d["kernel_source"] = ("profiles/op_configs_c1_c3_kernel_trace.md" if k else
                              "none: the committed kernel trace is of another workload or build" if prof else
                              "none: no committed kernel trace")
        return d

    # C1: int8 GEMV, W int8 U{-127..127}, scales U[1e-3,1e-2], x ~ N(0,1) quantised per tensor
    c1 = []
    for n, k in ((3584, 1024), (1024, 3584), (6144, 1024)):
        copies = -(-ROTATE_BYTES // (n * k))
        W = torch.from_numpy(q.synth_i8(copies * n * k, 11 + n)).to(dev).view(copies, n, k)
        sw = torch.from_numpy(q.synth_uniform(copies * n, 13 + n, 1e-3, 1e-2)).to(dev).view(copies, n)
        x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(dev)
        xq = torch.empty(k, dtype=torch.int8, device=dev)
        sx = torch.empty(1, device=dev)
        y = torch.empty(n, device=dev)
        q.quant_act(xq, sx, x, k)
        _gap(torch)
        if w8a8:
            us = _timed(torch, lambda i=0: q.gemv_i8_w8a8(y, None, W[i % copies], sw[i % copies], xq, sx, n, k), 200)
            nbytes = n * k + 4 * n + k + 4 + 4 * n
        else:
            us = _timed(torch, lambda i=0: q.gemv_i8(y, W[i % copies], sw[i % copies], x, n, k), 200)
            nbytes = n * k + 4 * n + 4 * k + 4 * n
        c1.append(entry(f"C1 {n}x{k}", nbytes, us, shape=f"{n}x{k}", copies=copies))
        del W, sw
    out["C1_gemv"] = c1

    # C2: the configured recurrent step (deltanet.hpp:154-179) from projected inputs: conv1d +
    # SiLU over qkv [6144] ~ N(0,1), gates from a, b ~ N(0,1), l2norm, the delta rule on a warm
    # state S ~ N(0, 0.05), per-head gated RMSNorm with z ~ N(0,1); layer 0's conv / gate / norm
    # weights.  Copies of S, the conv state and the conv weights rotate (> 256 MB).
    e = q.parse_idx(idx)
    pre = "layers.0.linear_attn."

    def f32w(name):
        t = e[name]
        return torch.from_numpy(blob[t.off:t.off + t.nbytes].view(np.float32).copy()).to(dev)

    per = 16 * 128 * 128 * 4 + 2 * 6144 * 4 * 4
    copies = -(-ROTATE_BYTES // per)
    S = torch.from_numpy((0.05 * rng.standard_normal((16, 128, 128))).astype(np.float32)).to(dev)
    S = S.unsqueeze(0).repeat(copies, 1, 1, 1)
    cst = torch.from_numpy(rng.standard_normal((6144, 4)).astype(np.float32)).to(dev).unsqueeze(0).repeat(copies, 1, 1)
    cw = f32w(pre + "conv1d.weight").view(1, 6144, 4).repeat(copies, 1, 1)
    A_log, dtb, nw = f32w(pre + "A_log"), f32w(pre + "dt_bias"), f32w(pre + "norm.weight")
    qkv = torch.from_numpy(rng.standard_normal(6144).astype(np.float32)).to(dev)
    z = torch.from_numpy(rng.standard_normal(2048).astype(np.float32)).to(dev)
    b = torch.from_numpy(rng.standard_normal(16).astype(np.float32)).to(dev)
    a = torch.from_numpy(rng.standard_normal(16).astype(np.float32)).to(dev)
    o = torch.empty(2048, device=dev)
    ws = torch.empty(q.deltanet_step_workspace(), dtype=torch.uint8, device=dev)
    _gap(torch)
    us = _timed(torch, lambda i=0: q.deltanet_step(o, qkv, z, b, a, cw[i % copies], A_log, dtb, nw, S[i % copies],
                                                   cst[i % copies], ws), 200)
    out["C2_deltanet_step"] = entry("C2", 2_384_640, us, copies=copies,
                                    ops="conv1d+SiLU+gates, l2norm+delta rule, gated RMSNorm (3 kernels)")
    del S, cst, cw

    # C3: the gated GQA attention layer (projections, QK-norm, RoPE, split-K softmax, gate, o_proj)
    # over an fp32 N(0,1) KV cache of T past tokens; KV caches and weight copies rotate (> 256 MB)
    p = "layers.3.self_attn."

    def up_i8(name):
        t = e[name]
        wq = blob[t.off:t.off + t.nbytes].view(np.int8).reshape(t.out, t.in_)
        return q.Tensor.i8(torch.from_numpy(wq.copy()).to(dev),
                           torch.from_numpy(blob[t.soff:t.soff + t.snbytes].view(np.float32).copy()).to(dev))

    wcopies = -(-ROTATE_BYTES // 7_364_608)
    keep = [[up_i8(p + n + "_proj.weight") for n in ("q", "k", "v", "o")] for _ in range(wcopies)]
    qn, kn = f32w(p + "q_norm.weight"), f32w(p + "k_norm.weight")
    xa = torch.from_numpy(rng.standard_normal(1024).astype(np.float32)).to(dev)
    ya = torch.empty(1024, device=dev)
    c3 = []
    for T in (512, 4096, 32768):
        kvc = max(2, -(-ROTATE_BYTES // ((T + 1) * 512 * 4 * 2)))
        kc = [torch.randn((T + 1) * 512, device=dev) for _ in range(kvc)]
        vc = [torch.randn((T + 1) * 512, device=dev) for _ in range(kvc)]
        _gap(torch)
        us = _timed(torch, lambda i=0: q.attention_layer_noalloc(ya, xa, *keep[i % wcopies], qn, kn, T, kc[i % kvc],
                                                                 vc[i % kvc], T, w8a8=w8a8), 50)
        c3.append(entry(f"C3 T={T}", 7_364_608 + 2_048 + 4_096 * T + 4_096, us, T=T, kv_copies=kvc,
                        weight_copies=wcopies))
        del kc, vc
    out["C3_attention"] = c3
    del keep
    if with_c4:
        out["C4_block"] = c4_persistent(q, torch, np, blob, idx, act_mode)
    return out


def c4_persistent(q, torch, np, blob, idx, act_mode, launches=8):
    """C4 on the persistent executor: layers 0-3 (3 DeltaNet + 1 attention layer, each with its
    MLP) inside the decode step.  Each launch decodes two tokens with the stage trace on; the
    unit is the second token's span from the end of the first token's last stage (the LM head)
    to the end of layer 3's down projection (program stage 20), on the kernel's s_memrealtime
    clock (100 MHz), after a 64-token prompt."""
    import tempfile
    from qwen_fpga_amd import stage_trace
    eng = q.Engine(blob, idx=idx, max_ctx=64 + 2 * launches + 8, mode=q.MODE_W8A8 if act_mode == "w8a8" else q.MODE_W8A16)
    spans = []
    try:
        eng.set_exec(q.EXEC_PERSISTENT)
        eng.reset()
        eng.generate(list(range(100, 164)), 0)
        fd, path = tempfile.mkstemp(suffix=".txt")
        os.close(fd)
        for _ in range(launches):
            os.environ["QH_TRACE_FILE"] = path
            try:
                eng.generate([eng.last_argmax], 2)
            finally:
                del os.environ["QH_TRACE_FILE"]
            spans.append(stage_trace.span_us(path, token=1, last_stage=20))
        os.unlink(path)
        T = eng.pos
    finally:
        eng.close()
    us = sorted(spans)[len(spans) // 2]
    return dict(_rate(90_709_888 + 4_096 * T, us), steps=launches, exec="persistent", T=T,
                note="kernel stage clock: layers 0-3 of the second traced token (program stages 0-20)")


def _blas_threads():
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads") for i in threadpool_info() if i.get("user_api") == "blas"]
        return int(n[0]) if n else 1
    except Exception:
        return int(os.environ.get("OPENBLAS_NUM_THREADS", "1"))


def cpu_baseline(blob, idx, prompt, ntok, act_mode):
    """The reference's CPU paths on this host, same synthetic model and prompt.  Primary
    (same activation mode as the GPU line): this repository's numpy restatement of the
    reference golden decode (golden/model.py; oracle/numpy_golden.py, pinned to fixtures the
    reference wrote), numpy's BLAS threads; the legs add the other mode and the reference's
    own hls/src decode top compiled natively (W8A16 only, one core)."""
    import oracle
    import oracle.numpy_golden as ng
    import qwen_fpga_amd as q

    entries = q.parse_idx(idx)
    legs = []
    for mode in (act_mode, "w8a16" if act_mode == "w8a8" else "w8a8"):
        g = ng.Golden(blob, entries, act_int8=mode == "w8a8")
        g.decode_step(int(prompt[0]))   # first touch of the weights
        g.reset()
        n = 2 * ntok
        t0 = time.perf_counter()
        for t in prompt[:n]:
            g.decode_step(int(t))
        dt = time.perf_counter() - t0
        legs.append({"value": round(n / dt, 3), "unit": "tok/s", "cores": _blas_threads(), "kind": "port",
                     "sample": f"{n} decode tokens from a fresh state, numpy golden decode restated "
                               f"(golden/model.py, {mode}; numpy BLAS threads, host nproc {os.cpu_count()})"})
        del g
    if oracle.ref() is not None:
        m = oracle.RefModel(blob)
        t0 = time.perf_counter()
        for t in prompt[:ntok]:
            m.qwen_top(int(t))
        dt = time.perf_counter() - t0
        legs.append({"value": round(ntok / dt, 4), "unit": "tok/s", "cores": 1, "kind": "reference",
                     "sample": f"{ntok} decode tokens from a fresh state, the reference hls/src qwen_top compiled "
                               f"-O2 -ffp-contract=off (csim build; w8a16)"})
    out = dict(legs[0])
    out["legs"] = legs[1:] + cpu_config_legs(blob, idx)
    return out


def cpu_config_legs(blob, idx):
    """BASELINE.json configs C1-C4 on one core, per unit: the reference's hls/src kernels
    (oracle/_ref, compiled from the headers where they lie) built -O3 (`value`) and with the
    reference's csim flags, -O2 (`value_o2`), both -ffp-contract=off, W8A16 (the reference's own
    arithmetic).  C3 at T = 32768 exceeds the reference's sc[8192] bound (attention.hpp:66): that
    unit runs this repository's C restatement in the reference order (oracle.c, -O3, one thread).
    Each unit is timed over a bounded sample (`calls`) after one untimed call."""
    import numpy as np
    import oracle
    import qwen_fpga_amd as q
    r3, r2 = oracle.ref(True), oracle.ref()
    if r3 is None or r2 is None:
        return []
    P = lambda a: a.ctypes.data
    rng = np.random.default_rng(3)
    f32 = lambda *shape: np.ascontiguousarray(rng.standard_normal(shape).astype(np.float32))
    entries = q.parse_idx(idx)

    def tensor(name):
        e = entries[name]
        if e.dtype == 1:
            w = blob[e.off:e.off + e.nbytes].view(np.int8).reshape(e.out, e.in_)
            return oracle.tensor_i8(w, blob[e.soff:e.soff + e.snbytes].view(np.float32)), w
        w = np.ascontiguousarray(blob[e.off:e.off + e.nbytes].view(np.float32))
        return (oracle.tensor_f32(w.reshape(e.out, e.in_)) if e.in_ > 1 and e.out * e.in_ == w.size else None), w

    def timed(fn, calls):
        fn()
        t0 = time.perf_counter()
        for _ in range(calls):
            fn()
        return (time.perf_counter() - t0) / calls * 1e6

    def leg(cfg, unit_bytes, calls, f3, f2=None, kind="reference", flags="-O3 / -O2 (value_o2)"):
        us3 = timed(f3, calls)
        d = {"config": cfg, "value": round(us3, 1), "unit": "us per unit", "cores": 1, "kind": kind,
             "bytes": int(unit_bytes), "gbs": round(unit_bytes / us3 / 1e3, 2), "calls": calls, "flags": flags}
        if f2 is not None:
            us2 = timed(f2, calls)
            d["value_o2"] = round(us2, 1)
        return d

    legs = []
    # C1: the reference gemv_i8 (gemv.hpp:28-42), int8 weights x fp32 activation, 4 rotating copies
    for n, k in ((3584, 1024), (1024, 3584), (6144, 1024)):
        W = [np.ascontiguousarray(q.synth_i8(n * k, 11 + n + c).reshape(n, k)) for c in range(4)]
        sw = q.synth_uniform(n, 13 + n, 1e-3, 1e-2)
        x, y = f32(k), np.empty(n, np.float32)
        it = [0]

        def mk(L):
            def f():
                it[0] += 1
                L.ref_gemv_i8(P(y), P(W[it[0] % 4]), P(sw), P(x), n, k)
            return f
        legs.append(leg(f"C1 {n}x{k}", n * k + 4 * n + 4 * k + 4 * n, 120, mk(r3), mk(r2)))
    # C2: the recurrent step from projected inputs (deltanet.hpp:154-179) on a warm state
    pre = "layers.0.linear_attn."
    cw, Al, dtb, nw = (tensor(pre + n)[1] for n in ("conv1d.weight", "A_log", "dt_bias", "norm.weight"))
    qkv, z, b, a = f32(6144), f32(2048), f32(16), f32(16)
    og = np.empty(2048, np.float32)
    rec, cs = f32(16 * 128 * 128) * np.float32(0.05), f32(6144 * 4)

    def step(L):
        return lambda: L.ref_deltanet_step(P(og), P(qkv), P(z), P(b), P(a), P(cw), P(Al), P(dtb), P(nw), P(rec), P(cs))
    legs.append(leg("C2", 2_384_640, 400, step(r3), step(r2)))
    # C3: the attention layer (attention.hpp:25-95) over an N(0,1) cache of T past tokens
    pa = "layers.3.self_attn."
    at = [tensor(pa + n + "_proj.weight")[0] for n in ("q", "k", "v", "o")]
    qn, kn = tensor(pa + "q_norm.weight")[1], tensor(pa + "k_norm.weight")[1]
    xa, ya = f32(1024), np.empty(1024, np.float32)
    for T, calls in ((512, 40), (4096, 12)):
        kc, vc = f32((T + 1) * 512), f32((T + 1) * 512)

        def att(L):
            return lambda: L.ref_attention_layer(P(ya), P(xa), *at, P(qn), P(kn), T, P(kc), P(vc), T)
        legs.append(leg(f"C3 T={T}", 7_364_608 + 2_048 + 4_096 * T + 4_096, calls, att(r3), att(r2)))
    T = 32768
    kc, vc = f32((T + 1) * 512), f32((T + 1) * 512)
    import ctypes
    os.environ["OMP_NUM_THREADS"] = "1"
    L = oracle.lib()
    try:   # one thread also if the OpenMP runtime started before this call
        ctypes.CDLL("libgomp.so.1").omp_set_num_threads(1)
    except OSError:
        pass
    legs.append(leg(f"C3 T={T}", 7_364_608 + 2_048 + 4_096 * T + 4_096, 2,
                    lambda: L.or_attention_layer(P(ya), P(xa), *at, P(qn), P(kn), T, P(kc), P(vc), T, oracle.W8A16,
                                                 oracle.ORDER_REF),
                    kind="port", flags="oracle.c -O3 -ffp-contract=off, reference order (beyond the reference's sc[8192])"))
    # C4: layers 0-3 (3 DeltaNet + 1 attention, each with its MLP) at T = 66 past tokens
    states = {}

    def block(Lr):
        st = states.setdefault(id(Lr), {
            "rec": [f32(16 * 128 * 128) * np.float32(0.05) for _ in range(3)], "conv": [f32(6144 * 4) for _ in range(3)],
            "kc": f32(67 * 512), "vc": f32(67 * 512)})
        h, t = f32(1024), np.empty(1024, np.float32)

        def run():
            for li in range(4):
                if li < 3:
                    pl = f"layers.{li}.linear_attn."
                    args = [tensor(pl + n)[0] for n in ("in_proj_qkv.weight", "in_proj_z.weight", "in_proj_b.weight",
                                                        "in_proj_a.weight")]
                    ws = [tensor(pl + n)[1] for n in ("conv1d.weight", "A_log", "dt_bias", "norm.weight")]
                    Lr.ref_deltanet_layer(P(t), P(h), *args, *[P(w) for w in ws], tensor(pl + "out_proj.weight")[0],
                                          P(st["rec"][li]), P(st["conv"][li]))
                else:
                    Lr.ref_attention_layer(P(t), P(h), *at, P(qn), P(kn), 66, P(st["kc"]), P(st["vc"]), 66)
                pm = f"layers.{li}.mlp."
                Lr.ref_mlp_layer(P(h), P(t), *[tensor(pm + n + "_proj.weight")[0] for n in ("gate", "up", "down")])
        return run
    legs.append(leg("C4", 90_709_888 + 4_096 * 66, 8, block(r3), block(r2)))
    return legs


if __name__ == "__main__":
    # A run that succeeds returns from the script instead of calling sys.exit(0): when
    # rocprofv3 profiles a process that made a cooperative launch, the process ends in a
    # segmentation fault inside exit(), in the libraries' exit handlers; on the normal-return
    # path the profiler's own exit handler writes its records before that, on the sys.exit
    # path after it (so the records were lost).  Nothing of this library runs at exit.
    rc = main()
    if rc:
        sys.exit(rc)
