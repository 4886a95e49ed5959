"""Synthetic Hugging Face snapshots of the Qwen3.5-0.8B text LM for the packer tests.

A snapshot is ``config.json`` (``text_config`` = the config block of the reference's
qwen35_int8.manifest.json, plus two keys the packer must ignore) and one
``model.safetensors`` whose text tensors carry the checkpoint's names
(``model.language_model.<manifest name>``) and shapes, next to a vision and an MTP
tensor the packer must drop.  Values are bfloat16 bits drawn per tensor with a
bounded exponent (finite, weight-like magnitudes); ``A_log`` is stored as F32
(log of a value in [1, 16)), so both stored dtypes reach the packer.  With
``sparse=True`` the data section is a hole: the headers are complete and no
tensor bytes are written (for tests that never read the data).
"""
import json
import os
import struct

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MANIFEST = os.path.join(GOLDEN, "qwen35_int8.manifest.json")
PREFIX = "model.language_model."


def reference_manifest() -> dict:
    with open(MANIFEST) as f:
        return json.load(f)


def _exp_range(name: str, shape) -> int:
    """Lowest bfloat16 exponent field of a tensor's values (four consecutive binades)."""
    if "conv1d" in name:
        return 122   # |v| in [2^-5, 2^-1)
    if name.endswith("norm.weight") or name.endswith("dt_bias"):
        return 120   # [2^-7, 2^-3)
    return 119       # [2^-8, 2^-4): GEMV weights, embeddings, in_proj_a/b


def bf16_bits(rng, n: int, lo_exp: int) -> np.ndarray:
    """n bfloat16 bit patterns: random sign and mantissa, exponent lo_exp .. lo_exp + 3."""
    r = rng.integers(0, 1 << 32, size=(n + 1) // 2, dtype=np.uint32).view(np.uint16)[:n]
    return (r & np.uint16(0x807F)) | ((((r >> np.uint16(7)) & np.uint16(3)) + np.uint16(lo_exp)) << np.uint16(7))


def write_safetensors(path: str, tensors: list, sparse: bool = False) -> None:
    """tensors: [(name, dtype string, shape, producer)], producer() -> bytes of the data
    (not called when sparse)."""
    hdr, off = {"__metadata__": {"format": "pt"}}, 0
    sizes = {"BF16": 2, "F32": 4}
    for name, dt, shape, _ in tensors:
        n = int(np.prod(shape)) * sizes[dt]
        hdr[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + n]}
        off += n
    h = json.dumps(hdr).encode()
    h += b" " * ((-len(h)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        if sparse:
            f.truncate(8 + len(h) + off)
            return
        for _, _, _, produce in tensors:
            f.write(produce())


def make_snapshot(d: str, seed: int = 0, sparse: bool = False) -> dict:
    """Write a full-size synthetic snapshot into directory d; return the reference manifest."""
    os.makedirs(d, exist_ok=True)
    man = reference_manifest()
    cfg = dict(man["config"])
    cfg["model_type"] = "qwen3_5_text"
    cfg["tie_word_embeddings"] = True
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump({"text_config": cfg, "architectures": ["Qwen3_5ForConditionalGeneration"]}, f)
    rng = np.random.default_rng(seed)
    tensors = []
    for t in man["tensors"]:
        name, shape = t["name"], tuple(t["shape"])
        n = int(np.prod(shape))
        if name.endswith("A_log"):
            tensors.append((PREFIX + name, "F32", shape,
                            lambda n=n: np.log(rng.uniform(1.0, 16.0, n)).astype("<f4").tobytes()))
        else:
            tensors.append((PREFIX + name, "BF16", shape,
                            lambda n=n, e=_exp_range(name, shape): bf16_bits(rng, n, e).astype("<u2").tobytes()))
    # tensors outside the text LM, which the packer drops (golden/loader.py:55-57)
    tensors.append(("model.visual.patch_embed.proj.weight", "BF16", (8, 16),
                    lambda: bf16_bits(rng, 128, 119).astype("<u2").tobytes()))
    tensors.append(("mtp.fc.weight", "BF16", (4, 8), lambda: bf16_bits(rng, 32, 119).astype("<u2").tobytes()))
    write_safetensors(os.path.join(d, "model.safetensors"), tensors, sparse=sparse)
    return man


IM_START, IM_END = 248045, 248046   # chat markers; IM_END is the eos


def write_tokenizer(d: str) -> None:
    """A word-level tokenizer over all 248,320 ids, saved like a checkpoint's
    (tokenizer.json + tokenizer_config.json with a chat template): "hello" = 1,
    "world" = 2, "user" = 3, "assistant" = 4, the chat markers at 248045/248046,
    every other id a word "w<id>"; words are split on whitespace and decoding
    joins them with spaces."""
    from tokenizers import Tokenizer
    from tokenizers.models import WordLevel
    from tokenizers.pre_tokenizers import WhitespaceSplit
    from transformers import PreTrainedTokenizerFast

    vocab = {f"w{i}": i for i in range(248320)}
    special = {"<unk>": 0, "hello": 1, "world": 2, "user": 3, "assistant": 4, "<|im_start|>": IM_START,
               "<|im_end|>": IM_END}
    for w, i in special.items():
        vocab.pop(f"w{i}")
        vocab[w] = i
    tk = Tokenizer(WordLevel(vocab, unk_token="<unk>"))
    tk.pre_tokenizer = WhitespaceSplit()
    chat = ("{% for m in messages %}<|im_start|> {{ m['role'] }} {{ m['content'] }} <|im_end|> {% endfor %}"
            "{% if add_generation_prompt %}<|im_start|> assistant {% endif %}")
    fast = PreTrainedTokenizerFast(tokenizer_object=tk, unk_token="<unk>", eos_token="<|im_end|>")
    fast.chat_template = chat
    fast.save_pretrained(d)
