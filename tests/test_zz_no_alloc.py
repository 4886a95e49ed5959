"""qh_attention_layer_noalloc: the attention layer op without any device allocation.

It runs the kernels of qh_attention_layer / qh_attention_layer_w8a8 with their
intermediate vectors in the library's file-scope device array instead of a
stream-ordered allocation.  Through the C ABI it must give the same bits as
the allocating entry point -- output and both cache rows -- on two calls in a
row, the second with a shorter context (the array keeps the first call's
contents), in both activation modes, on a long context (the split scheme above
2048 positions) and short ones; contexts beyond its maximum are refused.  The
device memory pool that stream-ordered allocations draw from shows no use during
its calls, and does during the allocating entry point's (the control).
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitwise, rng

pytestmark = pytest.mark.gpu

PRE = "layers.3.self_attn."


@pytest.fixture(scope="module")
def W(q, blob, entries, torch_cuda):
    torch = torch_cuda

    def up(a):
        return torch.from_numpy(np.ascontiguousarray(a)).cuda()

    dev = {}
    for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
        e = entries[PRE + name + ".weight"]
        w = blob[e.off:e.off + e.nbytes].view(np.int8).reshape(e.out, e.in_)
        s = blob[e.soff:e.soff + e.snbytes].view(np.float32)
        dev[name] = (up(w), up(s))
    for name in ("q_norm", "k_norm"):
        e = entries[PRE + name + ".weight"]
        dev[name] = up(blob[e.off:e.off + e.nbytes].view(np.float32))
    return torch, up, dev


def _run(q, W, fn, x, kc, vc, T, w8a8):
    torch, up, dev = W
    t = [q.Tensor.i8(*dev[n]) for n in ("q_proj", "k_proj", "v_proj", "o_proj")]
    out, kd, vd = torch.empty(1024, device="cuda"), up(kc), up(vc)
    fn(out, up(x), *t, dev["q_norm"], dev["k_norm"], T, kd, vd, T, w8a8=w8a8)
    torch.cuda.synchronize()
    return out.cpu().numpy(), kd.cpu().numpy(), vd.cpu().numpy()


class _Pool:
    """The current device's default memory pool (hipMallocAsync draws from it): its
    high-water mark of memory in use, reset to the current use."""
    USED_MEM_HIGH = 0x8   # hipMemPoolAttrUsedMemHigh

    def __init__(self, torch):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.pool = ctypes.c_void_p()
        assert self.hip.hipDeviceGetDefaultMemPool(ctypes.byref(self.pool), torch.cuda.current_device()) == 0

    def reset(self):
        zero = ctypes.c_uint64(0)
        assert self.hip.hipMemPoolSetAttribute(self.pool, self.USED_MEM_HIGH, ctypes.byref(zero)) == 0

    def used_high(self):
        v = ctypes.c_uint64(0)
        assert self.hip.hipMemPoolGetAttribute(self.pool, self.USED_MEM_HIGH, ctypes.byref(v)) == 0
        return v.value


@pytest.mark.parametrize("w8a8", [False, True], ids=["w8a16", "w8a8"])
def test_noalloc_equals_allocating_entry_point(q, W, w8a8):
    r = rng(5150 + w8a8)
    pool = _Pool(W[0])
    # the second and third calls are smaller: stale scratch from the first must not matter
    for T in (5000, 1000, 37):
        x = np.ascontiguousarray(r.standard_normal(1024), np.float32)
        kc = np.zeros((T + 1, 512), np.float32)
        vc = np.zeros((T + 1, 512), np.float32)
        kc[:T] = r.standard_normal((T, 512))
        vc[:T] = r.standard_normal((T, 512))
        pool.reset()
        ref = _run(q, W, q.attention_layer, x, kc, vc, T, w8a8)
        assert pool.used_high() > 0, "control: the allocating entry point draws from the pool"
        pool.reset()
        got = _run(q, W, q.attention_layer_noalloc, x, kc, vc, T, w8a8)
        assert pool.used_high() == 0, f"T={T}: the pool was used during the call that allocates nothing"
        for name, a, b in zip(("out", "k cache", "v cache"), got, ref):
            assert_bitwise(a, b, f"T={T} {name}")


def test_noalloc_refuses_contexts_beyond_its_scratch(q, W):
    torch, up, dev = W
    T = 65536   # T + 1 = 65537 positions > 65536
    kc = torch.zeros((T + 1) * 512, device="cuda")
    vc = torch.zeros((T + 1) * 512, device="cuda")
    t = [q.Tensor.i8(*dev[n]) for n in ("q_proj", "k_proj", "v_proj", "o_proj")]
    with pytest.raises(q.QHError) as ex:
        q.attention_layer_noalloc(torch.empty(1024, device="cuda"), torch.zeros(1024, device="cuda"), *t,
                                  dev["q_norm"], dev["k_norm"], T, kc, vc, T)
    assert ex.value.status == q.QH_ERANGE
    # the largest accepted context runs
    T = 65535
    out = torch.empty(1024, device="cuda")
    q.attention_layer_noalloc(out, torch.zeros(1024, device="cuda"), *t, dev["q_norm"], dev["k_norm"], T,
                              kc, vc, T)
    torch.cuda.synchronize()
    assert np.isfinite(out.cpu().numpy()).all()
