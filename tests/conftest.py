import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (parity through the C ABI on the device)")


@pytest.fixture(scope="session")
def q():
    import qwen_fpga_amd

    qwen_fpga_amd._lib()
    return qwen_fpga_amd


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib().or_set_threads(min(16, os.cpu_count() or 1))
    return oracle


@pytest.fixture(scope="session")
def ref(orc):
    r = orc.ref()
    if r is None:
        pytest.skip("oracle/_ref (the compiled reference kernels) is not built")
    return r


@pytest.fixture(scope="session")
def blob(q):
    return q.synth_blob(1234)


@pytest.fixture(scope="session")
def idx(q):
    return q.idx_text()


@pytest.fixture(scope="session")
def entries(q, idx):
    return q.parse_idx(idx)


@pytest.fixture(scope="session")
def torch_cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    torch.cuda.set_device(0)
    return torch


def rng(seed):
    return np.random.default_rng(seed)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitwise(got, exp, what=""):
    g, e = np.asarray(got, dtype=np.float32), np.asarray(exp, dtype=np.float32)
    assert g.shape == e.shape, (what, g.shape, e.shape)
    same = (bits(g) == bits(e)) | ((g == 0) & (e == 0))   # +0 and -0 compare equal
    if not same.all():
        i = int(np.flatnonzero(~same)[0])
        raise AssertionError(f"{what}: {int((~same).sum())} of {g.size} differ; first at {i}: "
                             f"{g.flat[i]!r} vs {e.flat[i]!r}")


def assert_close(got, exp, rtol=1e-4, atol=1e-5, what=""):
    g, e = np.asarray(got, dtype=np.float64), np.asarray(exp, dtype=np.float64)
    err = np.abs(g - e)
    bad = err > atol + rtol * np.abs(e)
    if bad.any():
        i = int(np.flatnonzero(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {g.size} outside rtol={rtol} atol={atol}; "
                             f"first at {i}: {g.flat[i]!r} vs {e.flat[i]!r}; max|d|={err.max():.3e}")


def assert_close_norm(got, exp, rel, what=""):
    """max |got - exp| <= rel * max |exp|: the reassociation bound for a vector whose
    elements come from long fp32 sums (immune to cancellation in single elements)."""
    g, e = np.asarray(got, dtype=np.float64), np.asarray(exp, dtype=np.float64)
    err = np.abs(g - e).max()
    scale = np.abs(e).max()
    if err > rel * scale:
        i = int(np.argmax(np.abs(g - e)))
        raise AssertionError(f"{what}: max|d|={err:.3e} > {rel:g} * max|exp|={scale:.3e}; at {i}: "
                             f"{g.flat[i]!r} vs {e.flat[i]!r}")
