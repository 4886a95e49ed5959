"""Run a prompt through the MI355X decode engine: the reference's run_hls.py
(run_hls.py:41-91) with the engine in place of the HLS csim driver.

    python -m qwen_fpga_amd.run_hls -p "Explain what an FPGA is." -n 40 [--raw]
                                    [--snapshot DIR] [--artifacts DIR] [--w8a8] [--graph]

The prompt is tokenised with the checkpoint's own tokenizer (transformers'
AutoTokenizer from the snapshot directory; the chat template with the
generation prompt unless --raw, run_hls.py:53-66).  The int8 blob is packed
from the snapshot on first use (qwen_fpga_amd.pack_weights in place of
scripts/pack_weights.py, run_hls.py:29-37).  Generation is the qh_run_hls
program, spawned as the reference spawns its driver (run_hls.py:69-86): the
prompt ids in ``<artifacts>/prompt_ids.txt``, the generated ids on its stdout
(greedy, stopping before eos), its timing line on stderr.  The answer is the
tokenizer's decoding of the generated ids.
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
import time
from typing import List, Optional, Tuple

HERE = os.path.dirname(os.path.abspath(__file__))
DRIVER = os.path.join(HERE, "bin", "qh_run_hls")


def encode_prompt(tok, prompt: str, raw: bool) -> List[int]:
    """Prompt ids: raw completion, or the chat template with the generation prompt
    (run_hls.py:58-66)."""
    if raw:
        return [int(i) for i in tok(prompt)["input_ids"]]
    enc = tok.apply_chat_template([{"role": "user", "content": prompt}], add_generation_prompt=True, tokenize=True)
    if not isinstance(enc, (list, tuple)):
        enc = enc["input_ids"]
    flat = []
    for x in enc:   # a batch of one comes back nested
        if isinstance(x, (list, tuple)):
            flat.extend(int(i) for i in x)
        else:
            flat.append(int(x))
    return flat


def ensure_blob(artifacts: str, snapshot: Optional[str]) -> Tuple[str, str]:
    """The packed blob and its weights.idx under ``artifacts``, packed from the
    snapshot when the blob is missing."""
    blob = os.path.join(artifacts, "qwen35_int8.bin")
    idx = os.path.join(artifacts, "weights.idx")
    if not os.path.exists(blob) or not os.path.exists(idx):
        from qwen_fpga_amd import pack_weights

        print("packing int8 weights (one-time)...", flush=True)
        pack_weights.pack(snapshot or pack_weights.find_snapshot(), blob, idx, verbose=False)
    return blob, idx


def run_driver(blob: str, idx: str, ids: List[int], n_new: int, eos: int, ids_file: str, w8a8: bool = False,
               graph: bool = False) -> subprocess.CompletedProcess:
    """Write the prompt ids and run qh_run_hls on them."""
    if not os.path.exists(DRIVER):
        raise FileNotFoundError(f"{DRIVER} is not built (python -c 'import __graft_entry__ as g; g.build()')")
    with open(ids_file, "w") as f:
        f.write(" ".join(str(int(i)) for i in ids))
    cmd = [DRIVER, blob, ids_file, str(n_new), str(eos), "--idx", idx]
    if w8a8:
        cmd.append("--w8a8")
    if graph:
        cmd.append("--graph")
    return subprocess.run(cmd, capture_output=True, text=True)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="run a prompt through the MI355X int8 decode engine")
    ap.add_argument("-p", "--prompt", required=True)
    ap.add_argument("-n", "--n_new", type=int, default=40)
    ap.add_argument("--raw", action="store_true", help="raw completion; skip chat template")
    ap.add_argument("--snapshot", default=None, help="checkpoint snapshot (tokenizer; weights when packing)")
    ap.add_argument("--artifacts", default="artifacts", help="directory of the packed blob and weights.idx")
    ap.add_argument("--w8a8", action="store_true", help="int8 activations (golden/model.py ACT_INT8)")
    ap.add_argument("--graph", action="store_true", help="a graph launch per token instead of the persistent kernel")
    args = ap.parse_args(argv)

    from qwen_fpga_amd import pack_weights
    from transformers import AutoTokenizer

    snap = args.snapshot or pack_weights.find_snapshot()
    blob, idx = ensure_blob(args.artifacts, snap)
    tok = AutoTokenizer.from_pretrained(snap)
    ids = encode_prompt(tok, args.prompt, args.raw)
    eos = tok.eos_token_id if tok.eos_token_id is not None else -1

    print(f"\nprompt   : {args.prompt!r}  ({len(ids)} tokens)")
    print("datapath : MI355X int8 decode engine (qh_run_hls), int8 weights\n")
    print("answer   : ", end="", flush=True)
    t0 = time.perf_counter()
    out = run_driver(blob, idx, ids, args.n_new, eos, os.path.join(args.artifacts, "prompt_ids.txt"), args.w8a8,
                     args.graph)
    wall = time.perf_counter() - t0
    if out.returncode != 0:
        print("\n[driver error]\n" + out.stderr)
        return 1
    gen = [int(x) for x in out.stdout.split()] if out.stdout.strip() else []
    print(tok.decode(gen))
    print()
    sys.stderr.write(out.stderr)
    print(f"\n--- this ran on the MI355X: {len(gen)} tokens, {wall * 1000:.0f} ms including the engine load")
    return 0


if __name__ == "__main__":
    sys.exit(main())
