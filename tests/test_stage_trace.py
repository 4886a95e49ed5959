"""The per-stage trace summary (qwen_fpga_amd.stage_trace) on a hand-built trace file."""
from qwen_fpga_amd import stage_trace


def _write(path):
    # 2 tokens x 2 stages (kinds 0 = GEMV, 6 = combine) x 2 workgroups, 8 slots (last = stage end), ticks of 10 ns
    lines = ["# token stage block m0..m6 done (s_memrealtime ticks; 0 = not reached); 2 stages per token, kinds: 0 6"]
    t0 = 1000
    for tok in range(2):
        base = t0 + tok * 10000
        for st in range(2):
            sb = base + st * 1000
            for b in range(2):
                end = sb + 500 + 100 * b          # workgroup 1 finishes last
                m = [sb, sb + 200 + b, sb + 300 + b, sb + 100, 0, sb + 400 + b, sb + 450 + b, end] if st == 0 else \
                    [sb, sb + 250 + b, 0, 0, 0, 0, 0, end]
                lines.append(" ".join(str(x) for x in [tok, st, b] + m))
    path.write_text("\n".join(lines) + "\n")


def test_summary_times_from_previous_stage_end(tmp_path):
    p = tmp_path / "t.txt"
    _write(p)
    rows = {r[0]: r for r in stage_trace.summarise(str(p), token=1)}
    # token 1: stage 0 starts at 11000; the previous end is token 0's stage 1 end = 1000 + 1000 + 600 = 2600
    kd, n, stage, *marks = rows[0]
    assert n == 1 and abs(stage - (11600 - 2600) * 0.01) < 1e-9
    # slowest workgroup (1): slots 1, 2, 5, 6 at 11000 + 201, 301, 401, 451
    assert [round(m, 6) for m in marks] == [86.01, 87.01, 88.01, 88.51]
    kd, n, stage, fold = rows[6]
    assert abs(stage - (12600 - 11600) * 0.01) < 1e-9 and abs(fold - (12000 + 251 - 11600) * 0.01) < 1e-9


def test_unreached_marks_are_nan(tmp_path):
    p = tmp_path / "t.txt"
    _write(p)
    lines = p.read_text().splitlines()
    # token 1, stage 0, workgroup 1: clear "first batch stored" (slot 6)
    for i, l in enumerate(lines):
        f = l.split()
        if f[:3] == ["1", "0", "1"]:
            f[3 + 6] = "0"
            lines[i] = " ".join(f)
    p.write_text("\n".join(lines) + "\n")
    rows = {r[0]: r for r in stage_trace.summarise(str(p), token=1)}
    assert rows[0][-1] != rows[0][-1]   # NaN
