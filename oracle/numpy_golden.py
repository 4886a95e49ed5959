"""A numpy restatement of the reference's golden decode (golden/model.py) --
TEST INFRASTRUCTURE ONLY: imported by tests/ (which pin it to the fixtures the
reference itself wrote, tests/golden/numpy_*) and by bench.py's cpu_baseline
leg, where it is the CPU port the reference publishes a rate for (30-35 tok/s,
artifacts/generations.md:16-17).  Never part of the product.

Same datapath as model.py: fake-quantised weights (golden/quant.py:52-53,
q.astype(float32) * scale per row) times fp32 activations through numpy's BLAS;
in W8A8 mode every projection input goes through the per-vector absmax int8
round trip of model.py:37-45 (at model.py:143, 191, 200, 230, 234, 237, not the
LM head, model.py:267).  Each function cites the lines it follows.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
EPS = 1e-6
THETA = 1e7
N_LAYERS = 24
H_LIN, DK, DV = 16, 128, 128
NH, NKV, HD, ROT = 8, 2, 256, 64


def layer_kind(i: int) -> str:
    """[linear x3, full] x 6 (model.py:16)."""
    return "full" if i % 4 == 3 else "linear"


class Golden:
    """golden/model.py decode_step over a packed blob; `act_int8` selects model.py's ACT_INT8."""

    def __init__(self, blob: np.ndarray, entries: dict, act_int8: bool):
        self.act_int8 = act_int8
        self.W = {}
        for name, e in entries.items():
            raw = blob[e.off:e.off + e.nbytes]
            if e.dtype == 1:   # dequant_rows (quant.py:52-53)
                q = raw.view(np.int8).reshape(e.out, e.in_)
                s = blob[e.soff:e.soff + 4 * e.out].view(F32)
                self.W[name] = q.astype(F32) * s[:, None]
            else:
                a = raw.view(F32)
                self.W[name] = a.reshape(e.out, e.in_) if e.in_ > 1 else a.copy()
        j = np.arange(0, ROT, 2, dtype=F32)
        self.inv_freq = 1.0 / (THETA ** (j / ROT))          # model.py:117
        self.reset()

    def reset(self):
        """DecodeState.new (model.py:94-107)."""
        n_lin = sum(layer_kind(i) == "linear" for i in range(N_LAYERS))
        self.conv = np.zeros((n_lin, 3 * 2048, 4), F32)
        self.rec = np.zeros((n_lin, H_LIN, DK, DV), F32)
        self.kc = [np.zeros((0, NKV, HD), F32) for _ in range(N_LAYERS - n_lin)]
        self.vc = [np.zeros((0, NKV, HD), F32) for _ in range(N_LAYERS - n_lin)]
        self.pos = 0

    # ---- primitives (model.py:37-80)
    def qa(self, x):
        """model.py:37-45: per-vector symmetric int8 round trip (identity in W8A16)."""
        if not self.act_int8:
            return x
        m = np.abs(x).max()
        if m == 0:
            return x
        step = m / 127.0
        return np.rint(x / step).clip(-127, 127) * step

    @staticmethod
    def silu(x):
        with np.errstate(over="ignore"):   # exp(-x) = inf below x = -88 gives the limit -0
            return x / (1.0 + np.exp(-x, dtype=F32))

    @staticmethod
    def sigmoid(x):
        return 1.0 / (1.0 + np.exp(-x, dtype=F32))

    @staticmethod
    def softplus(x):
        return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))

    @staticmethod
    def rms(x, w):
        """(1 + w) RMSNorm over the last axis (model.py:63-75)."""
        ms = np.mean(x.astype(F32) ** 2, axis=-1, keepdims=True)
        return (x * (1.0 / np.sqrt(ms + EPS))) * (1.0 + w)

    @staticmethod
    def l2n(x):
        """model.py:78-80: eps inside the sqrt of the SUM."""
        return x * (1.0 / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + EPS))

    def rope(self, x):
        """Partial RoPE on dims 0..63 at self.pos (model.py:113-129)."""
        f = self.pos * self.inv_freq
        ang = np.concatenate([f, f])
        c, s = np.cos(ang).astype(F32), np.sin(ang).astype(F32)
        r, rest = x[..., :ROT], x[..., ROT:]
        rot_half = np.concatenate([-r[..., ROT // 2:], r[..., :ROT // 2]], axis=-1)
        return np.concatenate([r * c + rot_half * s, rest], axis=-1)

    # ---- mixers
    def deltanet(self, p, x, li):
        """model.py:135-191."""
        W = self.W
        xq = self.qa(x)
        pre = W[p + "in_proj_qkv.weight"] @ xq
        z = W[p + "in_proj_z.weight"] @ xq
        b = W[p + "in_proj_b.weight"] @ xq
        a = W[p + "in_proj_a.weight"] @ xq
        taps = W[p + "conv1d.weight"].reshape(-1, 4)
        win = np.concatenate([self.conv[li], pre[:, None]], axis=1)    # model.py:153-155
        self.conv[li] = win[:, 1:]
        qkv = self.silu(np.sum(win[:, 1:] * taps, axis=1))
        q, k, v = (qkv[i * 2048:(i + 1) * 2048].reshape(H_LIN, DK) for i in range(3))
        beta = self.sigmoid(b)
        g = -np.exp(W[p + "A_log"].astype(F32)) * self.softplus(a + W[p + "dt_bias"])
        q = self.l2n(q) * (DK ** -0.5)
        k = self.l2n(k)
        S = self.rec[li]                                               # model.py:174-178
        S *= np.exp(g)[:, None, None]
        delta = (v - np.einsum("hkv,hk->hv", S, k)) * beta[:, None]
        S += np.einsum("hk,hv->hkv", k, delta)
        o = np.einsum("hkv,hk->hv", S, q)
        ms = np.mean(o.astype(F32) ** 2, axis=-1, keepdims=True)      # model.py:185-189
        o = W[p + "norm.weight"] * (o * (1.0 / np.sqrt(ms + EPS)))
        o = o * self.silu(z.reshape(H_LIN, DV))
        return W[p + "out_proj.weight"] @ self.qa(o.reshape(-1))

    def attention(self, p, x, fi):
        """model.py:194-230."""
        W = self.W
        xq = self.qa(x)
        qg = (W[p + "q_proj.weight"] @ xq).reshape(NH, 2 * HD)
        q, gate = qg[:, :HD], qg[:, HD:].reshape(-1)
        q = self.rope(self.rms(q, W[p + "q_norm.weight"]))
        k = self.rope(self.rms((W[p + "k_proj.weight"] @ xq).reshape(NKV, HD), W[p + "k_norm.weight"]))
        v = (W[p + "v_proj.weight"] @ xq).reshape(NKV, HD)
        self.kc[fi] = np.concatenate([self.kc[fi], k[None]], axis=0)
        self.vc[fi] = np.concatenate([self.vc[fi], v[None]], axis=0)
        K = np.repeat(self.kc[fi], NH // NKV, axis=1)                  # kv head of query head h: h // 4
        V = np.repeat(self.vc[fi], NH // NKV, axis=1)
        sc = np.einsum("hd,thd->ht", q, K) * (HD ** -0.5)
        sc = sc - sc.max(-1, keepdims=True)
        w = np.exp(sc)
        w /= w.sum(-1, keepdims=True)
        o = np.einsum("ht,thd->hd", w, V).reshape(-1) * self.sigmoid(gate)
        return W[p + "o_proj.weight"] @ self.qa(o)

    def mlp(self, p, x):
        """model.py:233-237."""
        W = self.W
        xq = self.qa(x)
        act = self.silu(W[p + "gate_proj.weight"] @ xq) * (W[p + "up_proj.weight"] @ xq)
        return W[p + "down_proj.weight"] @ self.qa(act)

    def decode_step(self, tok: int) -> np.ndarray:
        """model.py:243-267: one token in, the logits out."""
        W = self.W
        h = W["embed_tokens.weight"][tok].copy()
        li = fi = 0
        for i in range(N_LAYERS):
            p = f"layers.{i}."
            x = self.rms(h, W[p + "input_layernorm.weight"])
            if layer_kind(i) == "linear":
                h = h + self.deltanet(p + "linear_attn.", x, li)
                li += 1
            else:
                h = h + self.attention(p + "self_attn.", x, fi)
                fi += 1
            h = h + self.mlp(p + "mlp.", self.rms(h, W[p + "post_attention_layernorm.weight"]))
        self.pos += 1
        return W["embed_tokens.weight"] @ self.rms(h, W["norm.weight"])
