"""STREAM-style HBM probe on the GPU: confirms the achievable bandwidth of the
box (the roofline's denominator is MI355X's published 8 TB/s) and serves as
the known-size copy kernel that calibrates rocprofv3's FETCH_SIZE /
WRITE_SIZE counters (a copy of N bytes fetches N bytes and writes N bytes).

    python -m qwen_fpga_amd.hbm_stream [--mib 1024] [--iters 20]

Prints one JSON line: bytes per copy, mean copy time and GB/s (read + write).
The buffers are 4x the 256 MiB MALL by default, so the copy streams HBM.
"""
import argparse
import json


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--mib", type=int, default=1024, help="bytes copied per iteration, MiB")
    ap.add_argument("--iters", type=int, default=20)
    args = ap.parse_args()
    import torch

    n = args.mib * (1 << 20)
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.iters):
        dst.copy_(src)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.iters
    print(json.dumps({"bytes_per_copy": n, "copy_ms": round(ms, 4),
                      "copy_gbs_read_plus_write": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
