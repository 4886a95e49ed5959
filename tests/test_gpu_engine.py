"""Whole-model decode on the MI355X (qwen_top, hls/src/qwen_synth.hpp:39-92).

* bit for bit against the device-order twin of the oracle, logits and every
  recurrent / conv / KV state, in W8A16 and W8A8;
* the greedy argmax stream of the reference's own qwen_top (the committed
  fixture tests/golden/decode_ref_c5.json, written by make_golden.py from the
  compiled hls/src kernels): identical argmax at every one of 576 steps;
* the run_hls generation loop (hls/tb/run_hls.cpp:56-66) on the device against
  a host loop of decode_token calls, eos handling, context limits, reset;
* the benchmarked configuration (persistent executor, W8A8, 64 + 512 tokens in
  one launch) bit for bit against the twin; the argmax tie rule across
  workgroups; a forced hand-over give-up that every wave survives;
* layers [0, 4) as one block for 128 steps (C4), and the qh_run_hls CLI.
"""
import ctypes
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import GOLDEN, ROOT, assert_bitwise, assert_close, rng

pytestmark = pytest.mark.gpu


def _hip():
    for name in ("libamdhip64.so", "/opt/rocm/lib/libamdhip64.so"):
        try:
            h = ctypes.CDLL(name)
            h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
            return h
        except OSError:
            continue
    pytest.skip("libamdhip64 not loadable")


def d2h(ptr, shape):
    a = np.empty(shape, np.float32)
    assert _hip().hipMemcpy(a.ctypes.data, ptr, a.nbytes, 2) == 0   # hipMemcpyDeviceToHost
    return a


@pytest.fixture(scope="module")
def model(orc, blob, idx):
    m = orc.Model(blob, idx, max_ctx=64)
    yield m
    m.close()


@pytest.fixture(scope="module")
def engine(q, blob, torch_cuda):
    e = q.Engine(blob, max_ctx=64)
    yield e
    e.close()


@pytest.mark.parametrize("mode", [0, 1], ids=["w8a16", "w8a8"])
def test_decode_matches_device_twin(q, orc, engine, model, mode):
    engine.set_mode(mode)
    engine.reset()
    model.reset()
    toks = [17, 248319, 0, 5000, 123456, 77, 77, 248000]
    for step, tok in enumerate(toks):
        am, lg = engine.decode_token(tok, want_logits=True)
        am_o, lg_o = model.decode_token(tok, mode=mode, order=orc.ORDER_DEV, want_logits=True)
        assert_bitwise(lg, lg_o, f"logits step {step}")
        assert am == am_o == int(np.argmax(lg_o)), (step, am, am_o)
        assert engine.pos == model.pos == step + 1
    assert_bitwise(d2h(engine.device_ptr(1), (18, 16, 128, 128)), model.rec(), "recurrent state")
    assert_bitwise(d2h(engine.device_ptr(2), (18, 6144, 4)), model.conv(), "conv state")
    assert_bitwise(d2h(engine.device_ptr(3), (6, 64, 512))[:, :len(toks)], model.kcache()[:, :len(toks)], "k cache")
    assert_bitwise(d2h(engine.device_ptr(4), (6, 64, 512))[:, :len(toks)], model.vcache()[:, :len(toks)], "v cache")


@pytest.mark.parametrize("mode", [0, 1], ids=["w8a16", "w8a8"])
def test_persistent_equals_graph_path(q, engine, mode):
    """The persistent kernel (one launch, tagged hand-overs) and the per-stage graph give the same bits."""
    default = engine.exec_kind
    engine.set_mode(mode)
    toks = [5, 248319, 17, 0, 99999, 3]
    runs = []
    for ex in (q.EXEC_GRAPH, q.EXEC_PERSISTENT):
        engine.set_exec(ex)
        engine.reset()
        lg_all = [engine.decode_token(t, want_logits=True)[1] for t in toks]
        st = (d2h(engine.device_ptr(1), (18, 16, 128, 128)), d2h(engine.device_ptr(2), (18, 6144, 4)),
              d2h(engine.device_ptr(3), (6, 64, 512)), d2h(engine.device_ptr(4), (6, 64, 512)))
        engine.reset()
        gen = engine.generate([11, 2222, 33333], 20)
        runs.append((lg_all, st, gen, engine.pos))
    engine.set_exec(default)
    (lg_g, st_g, gen_g, pos_g), (lg_p, st_p, gen_p, pos_p) = runs
    for i, (a, b) in enumerate(zip(lg_g, lg_p)):
        assert_bitwise(b, a, f"logits step {i}")
    for name, a, b in zip(("rec", "conv", "k", "v"), st_g, st_p):
        assert_bitwise(b, a, name)
    assert gen_p == gen_g and pos_p == pos_g == 23


def test_persistent_equals_graph_path_long_context(q, blob):
    """Past 2048 cached positions the attention stages switch to the long-context splits: both
    executors, W8A8, an 8-token prompt then greedy decoding to 2078 positions, give the same
    tokens, the same K/V cache rows and the same logits at the last step."""
    n = 2080
    e = q.Engine(blob, max_ctx=n, mode=q.MODE_W8A8)
    try:
        runs = []
        for ex in (q.EXEC_GRAPH, q.EXEC_PERSISTENT):
            e.set_exec(ex)
            e.reset()
            gen = e.generate([11, 2222, 33333, 4, 5, 6, 7, 8], 2069)
            am, lg = e.decode_token(gen[-1], want_logits=True)
            runs.append((gen, am, lg, e.pos, d2h(e.device_ptr(3), (6, n, 512)), d2h(e.device_ptr(4), (6, n, 512))))
            assert e.exec_kind == ex
        (gen_g, am_g, lg_g, pos_g, k_g, v_g), (gen_p, am_p, lg_p, pos_p, k_p, v_p) = runs
        assert pos_g == pos_p == 2078
        assert gen_p == gen_g and am_p == am_g
        assert_bitwise(lg_p, lg_g, "logits at position 2078")
        assert_bitwise(k_p[:, :pos_p], k_g[:, :pos_g], "k cache")
        assert_bitwise(v_p[:, :pos_p], v_g[:, :pos_g], "v cache")
    finally:
        e.close()


def test_reset_restarts_the_sequence(engine):
    engine.set_mode(0)
    engine.reset()
    a1, l1 = engine.decode_token(42, want_logits=True)
    engine.decode_token(43)
    engine.reset()
    assert engine.pos == 0
    a2, l2 = engine.decode_token(42, want_logits=True)
    assert a1 == a2
    assert_bitwise(l1, l2, "after reset")


def test_generate_equals_host_loop(engine):
    """The device-side run_hls loop against decode_token driven from the host."""
    engine.set_mode(0)
    prompt = [11, 2222, 33333, 44]
    engine.reset()
    cur = None
    for t in prompt:
        cur, _ = engine.decode_token(t)
    gen = []
    for _ in range(12):
        gen.append(cur)
        cur, _ = engine.decode_token(cur)
    assert engine.pos == len(prompt) + 12
    engine.reset()
    dev = engine.generate(prompt, 12)
    assert dev == gen
    assert engine.pos == len(prompt) + 12
    # eos: run_hls stops before pushing the eos token, without running it
    eos = gen[5]
    first = gen.index(eos)
    engine.reset()
    assert engine.generate(prompt, 12, eos=eos) == gen[:first]
    assert engine.pos == len(prompt) + first
    engine.reset()
    assert engine.generate(prompt, 0) == []
    assert engine.pos == len(prompt)
    assert engine.last_argmax == gen[0]


def test_context_limit(q, blob, torch_cuda):
    e = q.Engine(blob, max_ctx=4)
    try:
        for t in range(4):
            e.decode_token(t)
        with pytest.raises(q.QHError) as ex:
            e.decode_token(5)
        assert ex.value.status == q.QH_ERANGE
        e.reset()
        with pytest.raises(q.QHError):
            e.generate([1, 2, 3], 2)     # 5 positions > 4
        assert e.generate([1, 2], 2) and e.pos == 4
        with pytest.raises(q.QHError):
            e.decode_token(248320)       # token out of the vocabulary
    finally:
        e.close()


@pytest.mark.parametrize("mode", [0, 1], ids=["w8a16", "w8a8"])
def test_forward_layers_block_c4(q, orc, blob, idx, torch_cuda, mode):
    """C4: layers [0, 4) = 3 DeltaNet + 1 attention, 128 decode steps, each on a fresh hidden
    vector ~ N(0, 1) (the states and the KV cache evolve); every output and the final states
    bit for bit against the device twin."""
    torch = torch_cuda
    n = 128
    e = q.Engine(blob, max_ctx=n, mode=mode)
    m = orc.Model(blob, idx, max_ctx=n)
    try:
        r = rng(404 + mode)
        for step in range(n):
            h = np.ascontiguousarray(r.standard_normal(1024), dtype=np.float32)
            hd = torch.from_numpy(h.copy()).cuda()
            e.forward_layers(0, 4, hd)
            ho = h.copy()
            m.forward_layers(0, 4, ho, mode=mode, order=orc.ORDER_DEV)
            assert_bitwise(hd.cpu().numpy(), ho, f"block output step {step}")
        assert e.pos == m.pos == n
        assert_bitwise(d2h(e.device_ptr(1), (18, 16, 128, 128))[:3], m.rec()[:3], "recurrent state")
        assert_bitwise(d2h(e.device_ptr(2), (18, 6144, 4))[:3], m.conv()[:3], "conv state")
        assert_bitwise(d2h(e.device_ptr(3), (6, n, 512))[0], m.kcache()[0], "k cache")
        assert_bitwise(d2h(e.device_ptr(4), (6, n, 512))[0], m.vcache()[0], "v cache")
    finally:
        e.close()
        m.close()


def test_persistent_full_c5_w8a8_vs_twin(q, orc, blob, idx, torch_cuda):
    """The benchmarked path at the benchmarked length: the persistent executor, W8A8, the C5
    prompt (64 seeded ids) and 512 greedy tokens in ONE launch (KV to 576, the multi-chunk
    combine past 512 positions), against the device twin: every generated id and, at the end,
    every recurrent / conv / KV buffer bit for bit; then the same stream token by token with
    the logits of chosen steps bit for bit."""
    npr, nn = 64, 512
    prompt = rng(1234).integers(0, q.VOCAB, size=npr).astype(np.int32).tolist()
    n = npr + nn
    keep = {0, 63, 64, 300, 511, 574}
    m = orc.Model(blob, idx, max_ctx=n)
    fed, twin_am, twin_lg = [], [], {}
    cur = None
    for i in range(n):   # the run_hls loop: prompt, then each argmax fed back (n passes in all)
        tok = prompt[i] if i < npr else cur
        cur, lg = m.decode_token(tok, mode=orc.W8A8, order=orc.ORDER_DEV, want_logits=i in keep)
        fed.append(tok)
        twin_am.append(cur)
        if i in keep:
            twin_lg[i] = lg
    e = q.Engine(blob, max_ctx=n, mode=q.MODE_W8A8)
    try:
        e.set_exec(q.EXEC_PERSISTENT)
        gen = e.generate(prompt, nn)
        assert e.exec_kind == q.EXEC_PERSISTENT, "the cooperative launch was refused"
        assert gen == twin_am[npr - 1:n - 1]
        assert e.pos == m.pos == n
        assert_bitwise(d2h(e.device_ptr(1), (18, 16, 128, 128)), m.rec(), "recurrent state")
        assert_bitwise(d2h(e.device_ptr(2), (18, 6144, 4)), m.conv(), "conv state")
        assert_bitwise(d2h(e.device_ptr(3), (6, n, 512)), m.kcache(), "k cache")
        assert_bitwise(d2h(e.device_ptr(4), (6, n, 512)), m.vcache(), "v cache")
        e.reset()
        for i, tok in enumerate(fed):
            am, lg = e.decode_token(tok, want_logits=i in keep)
            assert am == twin_am[i], f"step {i}: {am} vs twin {twin_am[i]}"
            if i in keep:
                assert_bitwise(lg, twin_lg[i], f"logits step {i}")
    finally:
        e.close()
        m.close()


@pytest.mark.parametrize("exec_kind", ["graph", "persistent"])
def test_argmax_tie_lowest_index_wins(q, orc, blob, idx, torch_cuda, exec_kind):
    """qwen_synth.hpp:81-88 / decoder.hpp:115: strict > from -1e30, so of equal logits the lowest
    index wins.  Row a (the argmax) of the tied embedding is copied to a lower row in another
    workgroup's range (that row must now win) and, separately, to a higher one (a must stay)."""
    tok = 17
    ex = q.EXEC_GRAPH if exec_kind == "graph" else q.EXEC_PERSISTENT
    e0 = q.Engine(blob, max_ctx=4)
    a, _ = e0.decode_token(tok)
    grid = e0.head_grid(ex)
    e0.close()
    emb = q.parse_idx(idx)["embed_tokens.weight"]
    stride = grid * 4   # head batches of 8 rows, one per wave, over this executor's workgroups of 4 waves

    def blk_of(r):
        return ((r // 8) % stride) // 4

    low = next(r for r in range(a // 3, a) if blk_of(r) != blk_of(a) and r != tok)
    high = next(r for r in range(a + (q.VOCAB - a) // 2, q.VOCAB) if blk_of(r) != blk_of(a) and r != tok)
    for other, want in ((low, low), (high, a)):
        b = blob.copy()
        row = slice(emb.off + a * 1024, emb.off + (a + 1) * 1024)
        b[emb.off + other * 1024:emb.off + (other + 1) * 1024] = b[row]
        b[emb.soff + 4 * other:emb.soff + 4 * other + 4] = b[emb.soff + 4 * a:emb.soff + 4 * a + 4]
        m = orc.Model(b, idx, max_ctx=4)
        am_t, lg_t = m.decode_token(tok, mode=orc.W8A16, order=orc.ORDER_DEV, want_logits=True)
        m.close()
        assert lg_t[other] == lg_t[a] and am_t == want
        e = q.Engine(b, max_ctx=4)
        try:
            e.set_exec(ex)
            am, lg = e.decode_token(tok, want_logits=True)
            assert e.exec_kind == ex
            assert lg[other] == lg[a], "tied rows must give identical logits"
            assert am == want, f"tie between {a} and {other}: argmax {am}, want {want}"
        finally:
            e.close()


def test_abort_exits_every_wave(q, blob, torch_cuda, monkeypatch):
    """A hand-over wait that gives up (forced from the host: QH_POLL_LIMIT=0 makes the first miss
    final) ends the launch with every workgroup leaving together: the call returns QH_EDEVICE,
    the engine refuses to decode until reset, and after the reset it decodes like a fresh one."""
    monkeypatch.setenv("QH_POLL_LIMIT", "0")
    e = q.Engine(blob, max_ctx=64)
    monkeypatch.delenv("QH_POLL_LIMIT")
    f = q.Engine(blob, max_ctx=64)
    try:
        e.set_exec(q.EXEC_PERSISTENT)
        with pytest.raises(q.QHError) as ex:
            e.generate([11, 2222, 33333, 44], 16)
        assert ex.value.status == q.QH_EDEVICE
        with pytest.raises(q.QHError) as ex:
            e.decode_token(5)
        assert ex.value.status == q.QH_ESTATE
        e.reset()
        e.set_exec(q.EXEC_GRAPH)   # the graph path has no hand-over waits
        f.set_exec(q.EXEC_GRAPH)
        a1, l1 = e.decode_token(5, want_logits=True)
        a2, l2 = f.decode_token(5, want_logits=True)
        assert a1 == a2
        assert_bitwise(l1, l2, "after reset")
    finally:
        e.close()
        f.close()


GOLD = os.path.join(GOLDEN, "decode_ref_c5.json")


@pytest.mark.skipif(not os.path.exists(GOLD), reason="golden decode fixture not generated")
@pytest.mark.parametrize("exec_kind", ["graph", "persistent"])
def test_reference_argmax_stream_c5(q, blob, exec_kind):
    """C5: 64-token prompt + 512 greedy tokens; argmax identical to the reference at every step,
    token by token and as one generate call, on both executors."""
    import hashlib

    g = json.load(open(GOLD))
    assert g["blob_sha256"] == hashlib.sha256(blob.tobytes()).hexdigest()
    n = len(g["fed"])
    e = q.Engine(blob, max_ctx=n)
    try:
        e.set_exec(q.EXEC_GRAPH if exec_kind == "graph" else q.EXEC_PERSISTENT)
        for i, tok in enumerate(g["fed"]):
            want = str(i) in g["logits"]
            am, lg = e.decode_token(tok, want_logits=want)
            assert am == g["argmax"][i], f"step {i}: {am} vs reference {g['argmax'][i]}"
            if want:
                s = g["logits"][str(i)]
                ids = np.array(s["top16_ids"])
                assert_close(lg[ids], np.array(s["top16_vals"]), rtol=1e-4, atol=1e-5, what=f"top16 step {i}")
                assert abs(np.sum(lg, dtype=np.float64) - s["sum_f64"]) <= 1e-4 * np.sqrt(s["sumsq_f64"]) * 20
        e.reset()
        npr = g["n_prompt"]
        gen = e.generate(g["fed"][:npr], g["n_new"])
        assert gen == g["argmax"][npr - 1:npr - 1 + g["n_new"]]
        assert e.exec_kind == (q.EXEC_GRAPH if exec_kind == "graph" else q.EXEC_PERSISTENT)
    finally:
        e.close()


def test_run_hls_cli(q, blob, idx, engine, tmp_path):
    exe = os.path.join(ROOT, "qwen_fpga_amd", "bin", "qh_run_hls")
    path = tmp_path / "qwen35_int8.bin"
    blob.tofile(path)
    ids = tmp_path / "ids.txt"
    ids.write_text("11 2222 33333 44\n")
    r = subprocess.run([exe, str(path), str(ids), "12"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    engine.set_mode(0)
    engine.reset()
    assert [int(t) for t in r.stdout.split()] == engine.generate([11, 2222, 33333, 44], 12)
    # the persistent kernel by default; the engine takes the graph path (same ids) when the
    # device refuses the cooperative launch, as it may while this test process holds the GPU
    assert "[mi355x]" in r.stderr and ("persistent kernel" in r.stderr or "graph per token" in r.stderr)
    rg = subprocess.run([exe, str(path), str(ids), "12", "--graph"], capture_output=True, text=True, timeout=120)
    assert rg.returncode == 0 and rg.stdout == r.stdout and "graph per token" in rg.stderr, rg.stderr
    (tmp_path / "w.idx").write_text(idx)
    r2 = subprocess.run([exe, str(path), str(ids), "12", "-1", "--w8a8", "--idx", str(tmp_path / "w.idx")],
                        capture_output=True, text=True, timeout=120)
    assert r2.returncode == 0, r2.stderr
    engine.set_mode(1)
    engine.reset()
    assert [int(t) for t in r2.stdout.split()] == engine.generate([11, 2222, 33333, 44], 12)


def test_tag_space_wrap(q, blob, torch_cuda, monkeypatch):
    """A persistent launch whose tags would run past 2^32 - 1 clears the tagged hand-over buffers
    and restarts the tags at 1 (qh_engine.hip run_persist).  Forced from the host by starting the
    tags just below the top (QH_TAG_START): the second of three launches wraps, and the ids,
    logits and every state buffer equal those of an engine whose tags start at 1."""
    top = 0xFFFFFFFF - 5000   # launch 1 needs 17 * 256 = 4352 tags, launch 2 another 10 * 256
    monkeypatch.setenv("QH_TAG_START", str(top))
    e = q.Engine(blob, max_ctx=64)
    monkeypatch.delenv("QH_TAG_START")
    f = q.Engine(blob, max_ctx=64)
    try:
        runs = []
        for eng in (e, f):
            eng.set_exec(q.EXEC_PERSISTENT)
            a = eng.generate([11, 2222, 33333, 44, 5, 6, 7, 8], 8)
            b = eng.generate([a[-1]], 8)
            am, lg = eng.decode_token(b[-1], want_logits=True)
            st = [d2h(eng.device_ptr(i), shp) for i, shp in
                  ((1, (18, 16, 128, 128)), (2, (18, 6144, 4)), (3, (6, 64, 512)), (4, (6, 64, 512)))]
            runs.append((a, b, am, lg, st))
        (a1, b1, m1, l1, s1), (a2, b2, m2, l2, s2) = runs
        assert a1 == a2 and b1 == b2 and m1 == m2
        assert_bitwise(l1, l2, "logits after the wrap")
        for x, y, what in zip(s1, s2, ("rec", "conv", "k cache", "v cache")):
            assert_bitwise(x, y, what)
    finally:
        e.close()
        f.close()
