"""Per-stage timing of the persistent decode kernel (needs a GPU).

    python -m qwen_fpga_amd.stage_trace [--pos 305] [--mode w8a8|w8a16] [--out stage_trace.txt]

Builds the seeded synthetic model, generates greedily up to position ``pos``,
then decodes a few more tokens with ``QH_TRACE_FILE`` set: ``persist_kernel``
records ``s_memrealtime`` marks (100 MHz) per workgroup and stage for the first
two tokens of that launch and the engine writes them as text, one line per
(token, stage, workgroup).  The summary below is the second token's: per stage
kind, the mean stage time (from the last workgroup finishing the previous
stage to the last workgroup finishing this one) and, for the workgroup that
finished last, the time of each mark on the same clock.

Marks (slot: meaning) by stage kind, as the stage bodies record them:
  GEMV      0 entry, 3 first poll back, 4 complete after a repoll, 1 input in LDS,
            2 prologue done, 5 first batch's dot products, 6 first batch stored
  DeltaNet  0 entry, 1 q, k, v of the head received, 2 delta computed
  attention 0 entry, 1 q (and the new K/V rows) received, 2 softmax of the split done
  combine   0 entry, 1 all split partials folded
The last slot is the stage end on every workgroup.
"""
import argparse
import os
import warnings

import numpy as np

KIND_NAMES = {0: "GEMV in_proj 1x8", 8: "GEMV q,k,v 1x8", 9: "GEMV gate,up 1x8", 1: "GEMV out_proj (gated)",
              2: "GEMV o_proj", 3: "GEMV down", 4: "DeltaNet",
              5: "attention", 6: "combine", 7: "LM head + argmax"}
KIND_MARKS = {0: (1, 2, 5, 6), 8: (1, 2, 5, 6), 9: (1, 2, 5, 6), 1: (1, 2, 5, 6), 2: (1, 2, 5, 6), 3: (1, 2, 5, 6),
              4: (1, 2), 5: (1, 2), 6: (1,), 7: ()}
TICK_US = 0.01   # s_memrealtime runs at 100 MHz


def record(out: str, pos: int = 305, mode: str = "w8a8", seed: int = 1234) -> None:
    import qwen_fpga_amd as q

    n_prompt = 8
    if pos < n_prompt + 1:
        raise ValueError(f"pos must be > {n_prompt}")
    e = q.Engine(q.synth_blob(seed), idx=q.idx_text(), max_ctx=pos + 8,
                 mode=q.MODE_W8A8 if mode == "w8a8" else q.MODE_W8A16)
    try:
        e.set_exec(q.EXEC_PERSISTENT)
        e.reset()
        e.generate(list(range(100, 100 + n_prompt)), pos - n_prompt - 1)
        os.environ["QH_TRACE_FILE"] = out
        try:
            e.generate([e.last_argmax], 4)
        finally:
            del os.environ["QH_TRACE_FILE"]
    finally:
        e.close()


def summarise(path: str, token: int = 1) -> list:
    """Rows (kind, count, mean stage us, mean slowest-workgroup mark times us...) of one traced token."""
    with open(path) as f:
        hdr = f.readline()
    kinds = [int(x) for x in hdr.split("kinds:")[1].split()]
    d = np.loadtxt(path, dtype=np.float64, comments="#", ndmin=2)
    tok, st, blk = d[:, 0].astype(int), d[:, 1].astype(int), d[:, 2].astype(int)
    ns, nb, nslot = len(kinds), int(blk.max()) + 1, d.shape[1] - 3
    a = np.zeros((int(tok.max()) + 1, ns, nb, nslot))
    a[tok, st, blk] = d[:, 3:]
    if token < 1 or token >= a.shape[0]:
        raise ValueError("token must name a traced token after the first")
    end = a[token, :, :, nslot - 1].max(axis=1)
    prev = np.concatenate([[a[token - 1, -1, :, nslot - 1].max()], end[:-1]])
    per_kind = {}
    for i, kd in enumerate(kinds):
        last = int(np.argmax(a[token, i, :, nslot - 1]))
        marks = [(a[token, i, last, m] - prev[i]) * TICK_US if a[token, i, last, m] > 0 else np.nan
                 for m in KIND_MARKS.get(kd, ())]
        per_kind.setdefault(kd, []).append([(end[i] - prev[i]) * TICK_US] + marks)
    rows = []
    for kd in sorted(per_kind):
        r = np.array(per_kind[kd], dtype=np.float64)
        with warnings.catch_warnings():   # a mark no stage of the kind reached stays NaN
            warnings.simplefilter("ignore", RuntimeWarning)
            rows.append((kd, len(r)) + tuple(np.nanmean(r, axis=0).tolist()))
    return rows


def span_us(path: str, token: int = 1, last_stage: int = -1) -> float:
    """Microseconds from the end of token `token` - 1 (its last stage, on the workgroup that
    finished it last) to the end of stage `last_stage` of token `token`, on the kernel's clock."""
    d = np.loadtxt(path, dtype=np.float64, comments="#", ndmin=2)
    tok, st = d[:, 0].astype(int), d[:, 1].astype(int)
    end = d[:, -1]
    ns = st.max() + 1
    last = last_stage % ns
    t1 = end[(tok == token) & (st == last)].max()
    t0 = end[(tok == token - 1) & (st == ns - 1)].max()
    return (t1 - t0) * TICK_US


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--pos", type=int, default=305)
    ap.add_argument("--mode", choices=("w8a8", "w8a16"), default="w8a8")
    ap.add_argument("--out", default="stage_trace.txt")
    ap.add_argument("--summarise-only", action="store_true", help="summarise an existing trace file")
    args = ap.parse_args(argv)
    if not args.summarise_only:
        os.makedirs(os.path.dirname(os.path.abspath(args.out)), exist_ok=True)
        record(args.out, args.pos, args.mode)
    total = 0.0
    print(f"{'stage kind':18s} {'n':>3s} {'stage us':>9s}  slowest workgroup marks (us)")
    for kd, n, stage, *marks in summarise(args.out):
        total += n * stage
        print(f"{KIND_NAMES.get(kd, str(kd)):18s} {n:3d} {stage:9.2f}  " + " / ".join(f"{m:.2f}" for m in marks))
    print(f"token total {total:.1f} us")


if __name__ == "__main__":
    main()
