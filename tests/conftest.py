"""Shared fixtures. `-m gpu` tests need a HIP device and the built libfl355.so;
everything else runs on the CPU (oracle pinning, host logic, ABI loading)."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libfl355.so")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o

    if not o._LIB_PATH.exists():
        o.build()
    o.lib()
    return o


@pytest.fixture(scope="session")
def fl():
    import __graft_entry__ as ge

    return ge.load_package()


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda:0")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def f16(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16)


def rand_qg(rng, T, n_heads=24, head_dim=256, q_scale=1 / 16):
    """A q|gate buffer [T, n_heads, 2*head_dim]: q ~ N(0,1) * q_scale, gate ~ N(0,1)."""
    qg = np.empty((T, n_heads, 2 * head_dim), np.float16)
    qg[..., :head_dim] = rng.standard_normal((T, n_heads, head_dim)) * q_scale
    qg[..., head_dim:] = rng.standard_normal((T, n_heads, head_dim))
    return qg


def rand_cache(rng, L, n_kv=4, head_dim=256):
    k = rng.standard_normal((L, n_kv, head_dim)).astype(np.float16)
    v = rng.standard_normal((L, n_kv, head_dim)).astype(np.float16)
    return k, v


def close(got, want, atol, rtol):
    """max |got - want| <= atol + rtol * |want|, elementwise; returns the worst
    (abs err, violation) for the failure message."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), "non-finite values"
    err = np.abs(got - want)
    bound = atol + rtol * np.abs(want)
    return float(err.max()), bool((err <= bound).all())


REL_MAX = 1e-2


def close_rel(got, want, atol, rtol, frac=REL_MAX):
    """close() and also max |got - want| <= frac * max |want|. A long-context
    attention output averages ~10^5 rows of V, so its values are ~1e-3 and the
    absolute bar alone passes an output that lost a whole split; the relative
    bar does not (tests/test_parity_bar.py shows which defects each bar
    rejects at these statistics)."""
    err, ok = close(got, want, atol, rtol)
    scale = float(np.abs(np.asarray(want, np.float64)).max())
    return err, ok and err <= frac * scale
