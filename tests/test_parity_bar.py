"""The long-context decode parity bar can fail: at the statistics of the GPU
decode tests (K, V ~ N(0, 1) fp16; q ~ N(0, 1) * q_scale; scale 1/16; a
sigmoid gate from N(0, 1) logits) an fp64 attention over ~95k rows is
compared with outputs carrying plausible kernel defects -- one of the 64
splits lost, one 32-row tile lost, every value scaled by 0.8 -- and
conftest.close_rel, the bar of tests/test_gpu_attention.py and
tests/test_gpu_q8.py, must reject each, while the exact output rounded to
fp16 passes. Where the scores are flat the absolute bar alone (max-abs 2e-3 /
rel 1e-2) accepts a lost split, which is why the relative bar exists.

The defects are planted in a CPU restatement here, never in a kernel. Split
ranges follow the batched decode's rule for a token of length L (St =
clamp(max(L / 256, min(L / 64, 32)), 1, 64) splits over its 32-row tiles,
tile-aligned), which cuts ~95k rows into 64 splits.
"""
import numpy as np
import pytest

from conftest import close, close_rel

ATOL, RTOL = 2e-3, 1e-2
TILE = 32
L = 95000
ROWS = 18            # T = 3 verify rows x 6 q heads of one kv head


def split_rows(seqlen, s, split_rows=256, split=64, floor=32):
    st = max(seqlen // split_rows, min(seqlen // 64, floor))
    st = max(1, min(st, split))
    nt = -(-seqlen // TILE)
    lo = nt * s // st * TILE
    hi = min(nt * (s + 1) // st * TILE, seqlen)
    return st, lo, hi


@pytest.fixture(scope="module")
def kv():
    rng = np.random.default_rng(95000)
    K = rng.standard_normal((L, 256)).astype(np.float16).astype(np.float64)
    V = rng.standard_normal((L, 256)).astype(np.float16).astype(np.float64)
    g = rng.standard_normal((ROWS, 256)).astype(np.float16).astype(np.float64)
    return rng, K, V, g


def attend(q, K, V, g, keep):
    s = (q @ K[keep].T) / 16.0
    s -= s.max(1, keepdims=True)
    p = np.exp(s)
    z = (p @ V[keep]) / p.sum(1, keepdims=True)
    return z / (1.0 + np.exp(-g))


@pytest.mark.parametrize("q_scale", [1 / 16, 1.0])
def test_relative_bar_rejects_planted_defects(kv, q_scale):
    rng, K, V, g = kv
    q = (rng.standard_normal((ROWS, 256)) * q_scale).astype(np.float16).astype(np.float64)
    every = np.ones(L, bool)
    want = attend(q, K, V, g, every)

    exact16 = want.astype(np.float16)
    assert close_rel(exact16, want, ATOL, RTOL)[1], "the exact output must pass"

    st, lo, hi = split_rows(L, 17)
    assert st == 64
    no_split = every.copy()
    no_split[lo:hi] = False
    lost_split = attend(q, K, V, g, no_split).astype(np.float16)
    no_tile = every.copy()
    no_tile[1000 * TILE:1001 * TILE] = False
    lost_tile = attend(q, K, V, g, no_tile).astype(np.float16)
    scaled = (0.8 * want).astype(np.float16)

    for name, bad in (("one split of 64 lost", lost_split), ("one 32-row tile lost", lost_tile),
                      ("0.8 z", scaled)):
        err, ok = close_rel(bad, want, ATOL, RTOL)
        print(f"q_scale {q_scale}: {name}: max|err| {err:.2e}, max|z| {np.abs(want).max():.2e}")
        assert not ok, f"q_scale {q_scale}: the bar accepts '{name}'"

    if q_scale < 1:
        # flat scores: the absolute bar alone accepts a lost split
        assert close(lost_split, want, ATOL, RTOL)[1]
