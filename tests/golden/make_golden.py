"""Writes the committed decode fixtures from the reference's own decode top.

Runs the reference hls/src qwen_top (compiled from /root/reference into
oracle/_ref/libqref.so by oracle/Makefile) on the seeded synthetic model
(qwen_fpga_amd.synth_blob(seed), packed in the pack_weights.py layout) and
records, like hls/tb/tb_decode.cpp:93-100, the token fed and the argmax at
every step, plus a summary of the step-0 logits.  The fed stream is the
run_hls loop (hls/tb/run_hls.cpp:56-66): the prompt, then each greedy argmax.

    python tests/golden/make_golden.py --prompt 64 --new 512 --out tests/golden/decode_ref_c5.json

Only this container has /root/reference; the JSON travels, the reference does not.
"""
import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
import qwen_fpga_amd as q  # noqa: E402


def logits_summary(lg: np.ndarray) -> dict:
    order = np.argsort(-lg, kind="stable")[:16]
    return {
        "top16_ids": [int(i) for i in order],
        "top16_vals": [float(lg[i]) for i in order],
        "sum_f64": float(np.sum(lg, dtype=np.float64)),
        "sumsq_f64": float(np.sum(lg.astype(np.float64) ** 2)),
        "sha256": hashlib.sha256(lg.astype("<f4").tobytes()).hexdigest(),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--prompt", type=int, default=64)
    ap.add_argument("--new", type=int, default=512)
    ap.add_argument("--out", required=True)
    args = ap.parse_args()
    if oracle.ref() is None:
        raise SystemExit("oracle/_ref/libqref.so is not built (needs /root/reference)")
    blob = q.synth_blob(args.seed)
    rng = np.random.default_rng(args.seed)
    prompt = rng.integers(0, q.VOCAB, size=args.prompt).astype(np.int32).tolist()
    m = oracle.RefModel(blob)
    fed, am, summaries = [], [], {}
    t0 = time.time()
    cur = None
    steps = args.prompt + args.new
    for i in range(steps):
        tok = prompt[i] if i < args.prompt else cur
        want = i in (0, args.prompt - 1, steps - 1)
        a, lg = m.qwen_top(int(tok), want_logits=want)
        fed.append(int(tok))
        am.append(int(a))
        if want:
            summaries[str(i)] = logits_summary(lg)
        cur = a
        if (i + 1) % 32 == 0:
            print(f"step {i + 1}/{steps}  {time.time() - t0:.0f}s", flush=True)
    out = {
        "source": "reference hls/src qwen_top (hls/src/qwen_synth.hpp:39-92) compiled -O2 -ffp-contract=off",
        "mode": "W8A16 (int8 weights x fp32 activations, the csim datapath)",
        "seed": args.seed,
        "blob_sha256": hashlib.sha256(blob.tobytes()).hexdigest(),
        "n_prompt": args.prompt,
        "n_new": args.new,
        "fed": fed,
        "argmax": am,
        "logits": summaries,
    }
    with open(args.out, "w") as f:
        json.dump(out, f)
    print(f"wrote {args.out}: {steps} steps in {time.time() - t0:.0f}s")


if __name__ == "__main__":
    main()
