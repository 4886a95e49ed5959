"""The run_hls wrapper (qwen_fpga_amd.run_hls, after the reference's run_hls.py) on the CPU:
prompt encoding with a checkpoint-style tokenizer, the ids file, the driver contract
and its failures.  The GPU run is in test_gpu_pack.py."""
import os

import pytest

from snapshot_util import IM_END, IM_START, make_snapshot, write_tokenizer
from qwen_fpga_amd import run_hls


@pytest.fixture(scope="module")
def snap(tmp_path_factory):
    d = tmp_path_factory.mktemp("snap")
    make_snapshot(str(d), sparse=True)   # config.json next to the tokenizer, as in a checkpoint
    write_tokenizer(str(d))
    return str(d)


@pytest.fixture(scope="module")
def tok(snap):
    from transformers import AutoTokenizer

    return AutoTokenizer.from_pretrained(snap)


def test_encode_prompt_raw_and_chat(tok):
    assert run_hls.encode_prompt(tok, "hello world", raw=True) == [1, 2]
    assert run_hls.encode_prompt(tok, "hello world", raw=False) == [IM_START, 3, 1, 2, IM_END, IM_START, 4]
    assert tok.eos_token_id == IM_END
    assert tok.decode([1, 2, 77]) == "hello world w77"


def test_driver_errors_are_reported(snap, tmp_path, capsys):
    # artifacts present but not a blob: qh_run_hls rejects it and main reports the driver error
    art = tmp_path / "artifacts"
    art.mkdir()
    (art / "qwen35_int8.bin").write_bytes(b"\0" * 4096)
    (art / "weights.idx").write_text("x 0 0 0 0 0 0 0\n")
    if not os.path.exists(run_hls.DRIVER):
        pytest.skip("qh_run_hls not built")
    rc = run_hls.main(["-p", "hello world", "-n", "4", "--raw", "--snapshot", snap, "--artifacts", str(art)])
    out = capsys.readouterr().out
    assert rc == 1 and "[driver error]" in out
    assert (art / "prompt_ids.txt").read_text() == "1 2"


def test_missing_driver(tmp_path, monkeypatch):
    monkeypatch.setattr(run_hls, "DRIVER", str(tmp_path / "nope"))
    with pytest.raises(FileNotFoundError, match="not built"):
        run_hls.run_driver("b", "i", [1], 1, -1, str(tmp_path / "ids.txt"))


def test_packs_on_first_use_and_needs_the_gpu(snap, tmp_path):
    import torch

    if torch.cuda.is_available():
        pytest.skip("checks the failure where no HIP device is visible")
    with pytest.raises(RuntimeError, match="GPU"):
        run_hls.ensure_blob(str(tmp_path / "artifacts"), snap)
