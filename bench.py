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


def profile_value(path, key):
    """A figure from a committed rocprofv3 counter summary (FETCH_SIZE + WRITE_SIZE, each
    scaled by a copy of known size); the counters cannot be read from inside this process."""
    try:
        for line in open(path):
            if line.startswith(key + ":"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def head_traffic():
    return profile_value(TRAFFIC_PROFILE, "traffic_bytes_per_launch")


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
        per_tok = profile_value(PERSIST_TRAFFIC_PROFILE, "traffic_bytes_per_token")
        roofline = {
            "kernel": "persist_kernel (every stage of every token in one cooperative launch)",
            # the only roofline of a ~2 op/B int8 GEMV datapath; the counters show ~1.05x the
            # algorithmic bytes cross HBM, so the gap to it is latency (126 dependent all-to-all
            # hand-overs per token), not traffic
            "bound": "hbm",
            "limiter": "latency of the per-stage hand-overs and post-arrival chains (traffic 1.05x algorithmic)",
            "achieved": round(launch_bytes / (launch_ms * 1e-3) / 1e9, 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(launch_bytes / (launch_ms * 1e-3) / 1e9 / PEAK_GBS, 4),
            # FETCH_SIZE + WRITE_SIZE per token of a 64-token launch (committed summary) x tokens
            "traffic": per_tok * args.steps if per_tok else None,
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
            "traffic": head_traffic(),
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


def op_configs(q, torch, np, blob, idx, act_mode):
    """BASELINE.json configs C1-C4 on the op-level C ABI (the standalone kernels of the
    graph executor), each unit timed with HIP events on the stream it runs on; bytes per
    unit are the algorithmic counts of the configs (weights + scales + activations + state
    / cache traffic).  C1 rotates through > 256 MB of weight copies so that no call is
    served by the 256 MB Infinity Cache."""
    dev = torch.device("cuda")
    w8a8 = act_mode == "w8a8"
    rng = np.random.default_rng(7)
    out = {}

    # C1: int8 GEMV, W int8 U{-127..127}, scales U[1e-3,1e-2], x ~ N(0,1) quantised per tensor
    c1 = []
    for n, k in ((3584, 1024), (1024, 3584), (6144, 1024)):
        copies = -(-300_000_000 // (n * k))
        W = torch.from_numpy(q.synth_i8(copies * n * k, 11 + n)).to(dev).view(copies, n, k)
        sw = torch.from_numpy(q.synth_uniform(copies * n, 13 + n, 1e-3, 1e-2)).to(dev).view(copies, n)
        x = torch.from_numpy(rng.standard_normal(k).astype(np.float32)).to(dev)
        xq = torch.empty(k, dtype=torch.int8, device=dev)
        sx = torch.empty(1, device=dev)
        y = torch.empty(n, device=dev)
        q.quant_act(xq, sx, x, k)
        if w8a8:
            us = _timed(torch, lambda i=0: q.gemv_i8_w8a8(y, None, W[i % copies], sw[i % copies], xq, sx, n, k), 200)
            nbytes = n * k + 4 * n + k + 4 + 4 * n
        else:
            us = _timed(torch, lambda i=0: q.gemv_i8(y, W[i % copies], sw[i % copies], x, n, k), 200)
            nbytes = n * k + 4 * n + 4 * k + 4 * n
        c1.append(dict(shape=f"{n}x{k}", **_rate(nbytes, us)))
        del W, sw
    out["C1_gemv"] = c1

    # C2: the recurrent delta-rule step of 16 heads on a warm fp32 state S0 ~ N(0, 0.05),
    # q, k l2-normalised, beta = sigmoid(N(0,1)), g = -softplus(N(0,1)) * A, A ~ U[1,16]; 64 steps
    S = torch.from_numpy((0.05 * rng.standard_normal((16, 128, 128))).astype(np.float32)).to(dev)
    qkv = rng.standard_normal((3, 16, 128)).astype(np.float32)
    qkv[:2] /= np.linalg.norm(qkv[:2], axis=-1, keepdims=True)
    qd, kd, vd = (torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in qkv)
    beta = torch.from_numpy((1 / (1 + np.exp(-rng.standard_normal(16)))).astype(np.float32)).to(dev)
    g = torch.from_numpy((-np.log1p(np.exp(rng.standard_normal(16))) * rng.uniform(1, 16, 16)).astype(np.float32)).to(dev)
    o = torch.empty(16 * 128, device=dev)
    us = _timed(torch, lambda i=0: q.delta_rule_layer(qd, kd, vd, g, beta, S, o), 64)
    out["C2_delta_rule_step"] = dict(steps=64, **_rate(2 * 16 * 128 * 128 * 4 + 4 * 3 * 2048 + 4 * 32 + 4 * 2048, us))

    # C3: the gated GQA attention layer (projections, QK-norm, RoPE, split-K softmax, gate, o_proj)
    # over an fp32 N(0,1) KV cache of T past tokens
    e = q.parse_idx(idx)
    p = "layers.3.self_attn."

    def up_i8(name):
        t = e[name]
        wq = blob[t.off:t.off + t.nbytes].view(np.int8).reshape(t.out, t.in_)
        return q.Tensor.i8(torch.from_numpy(wq.copy()).to(dev),
                           torch.from_numpy(blob[t.soff:t.soff + t.snbytes].view(np.float32).copy()).to(dev))

    def up_f32(name):
        t = e[name]
        return torch.from_numpy(blob[t.off:t.off + t.nbytes].view(np.float32).copy()).to(dev)

    keep = [up_i8(p + n + "_proj.weight") for n in ("q", "k", "v", "o")]
    qn, kn = up_f32(p + "q_norm.weight"), up_f32(p + "k_norm.weight")
    xa = torch.from_numpy(rng.standard_normal(1024).astype(np.float32)).to(dev)
    ya = torch.empty(1024, device=dev)
    c3 = []
    for T in (512, 4096, 32768):
        kc = torch.randn((T + 1) * 512, device=dev)
        vc = torch.randn((T + 1) * 512, device=dev)
        us = _timed(torch, lambda i=0: q.attention_layer(ya, xa, *keep, qn, kn, T, kc, vc, T, w8a8=w8a8), 50)
        c3.append(dict(T=T, **_rate(7_364_608 + 2_048 + 4_096 * T + 4_096, us)))
        del kc, vc
    out["C3_attention"] = c3

    # C4: layers 0-3 (3 DeltaNet + 1 attention, each with its MLP) as the engine's per-stage
    # kernels, 128 decode steps on fresh hidden vectors ~ N(0,1)
    eng = q.Engine(blob, idx=idx, max_ctx=130, mode=q.MODE_W8A8 if w8a8 else q.MODE_W8A16)
    h = torch.from_numpy(rng.standard_normal(1024).astype(np.float32)).to(dev)
    eng.forward_layers(0, 4, h)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(128):
        eng.forward_layers(0, 4, h)
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) * 1e6 / 128
    eng.close()
    out["C4_block"] = dict(steps=128, note="host-timed per step (one synchronising call each)",
                           **_rate(90_709_888 + 4_096 * 66, us))
    return out


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
    out["legs"] = legs[1:]
    return out


if __name__ == "__main__":
    # A run that succeeds returns from the script instead of calling sys.exit(0): when
    # rocprofv3 profiles a process that made a cooperative launch, the process ends in a
    # segmentation fault inside exit(), in the libraries' exit handlers; on the normal-return
    # path the profiler's own exit handler writes its records before that, on the sys.exit
    # path after it (so the records were lost).  Nothing of this library runs at exit.
    rc = main()
    if rc:
        sys.exit(rc)
