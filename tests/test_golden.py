"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) against the C oracle: every stored output is
recomputed from the stored inputs and must come out bit for bit, so a change
to the oracle that moves any value fails here (the fixtures were made after
the oracle was pinned by tests/test_oracle_*.py). Also checks the fixtures'
own invariants that need no oracle: the int8 bytes decode to values within
half a quantisation step, the zero L2-norm row stays zero, the reference's
known gate answers (kernels.cu:139-141)."""
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
SCALE = 256 ** -0.5
QS = 128 ** -0.5


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def same_bits(got, want):
    got, want = np.asarray(got), np.asarray(want)
    return got.dtype == want.dtype and got.shape == want.shape and \
        np.array_equal(got.view(np.uint8), want.view(np.uint8))


def recompute(orc, name, g):
    """The oracle's outputs from the fixture's stored inputs."""
    if name == "attn_decode":
        L = g["kc"].shape[0]
        return {"z": orc.attention_decode(g["qg"], g["kc"], g["vc"], int(g["pos0"]), max_pos=L,
                                          scale=SCALE)}
    if name == "attn_prefill":
        L, T = g["kc"].shape[0], g["qg"].shape[0]
        return {"z": orc.attention_prefill(g["qg"], g["kc"], g["vc"], q_pitch=512,
                                           pos0=int(g["pos0"]), max_pos=L, scale=SCALE, T=T)}
    if name == "kv8":
        L = g["k"].shape[0]
        kc8, vc8 = orc.kv8_buffer(L), orc.kv8_buffer(L)
        orc.kv_store_q8(g["k"], g["v"], kc8, vc8, 0, L, L)
        z = orc.attention_decode_q8(g["qg"], g["kc8"], g["vc8"], int(g["pos0"]), max_pos=L,
                                    scale=SCALE)
        return {"kc8": kc8, "vc8": vc8, "z": z}
    if name == "attn_prep":
        T, pos0 = g["qg"].shape[0], int(g["pos0"])
        kc = np.zeros((pos0 + T, 4, 256), np.float16)
        vc = np.zeros_like(kc)
        q, k = orc.attn_prep(g["qg"], g["k"], g["v"], g["wq"], g["wk"], kc, vc, pos0=pos0, T=T,
                             max_pos=pos0 + T)
        assert same_bits(kc[pos0:], k) and same_bits(vc[pos0:], g["v"])
        return {"q_out": q, "k_out": k}
    if name == "conv":
        T, dim = g["x"].shape
        y, st = orc.conv1d_causal(g["x"], g["w"], g["st"], dim=dim, T=T, pos0=int(g["pos0"]),
                                  row_stride=dim)
        return {"y": y, "st_out": st}
    if name == "norm_gates":
        T = g["x"].shape[0]
        y = orc.l2norm_scaled(g["x"], n=128, rows=8, pitch=128, eps=1e-6, scale=1.0, T=T)
        beta, decay = orc.gdn_scalars(g["a"], g["b"], g["A_log"], g["dt_bias"],
                                      T=g["a"].shape[0], n_heads=48)
        return {"y": y, "beta": beta, "decay": decay}
    if name == "scan":
        S = g["S0"].copy()
        y = orc.gdn_scan(g["q"], g["k"], g["v"], g["beta"], g["decay"], S, T=g["q"].shape[0],
                         n_kheads=1, n_vheads=3, qk_stride=128, v_stride=384, out_scale=QS)
        return {"S": S, "y": y}
    if name == "out_norm":
        return {"y": orc.rmsnorm_gated(g["o"], g["z"], g["w"], T=g["o"].shape[0])}
    raise KeyError(name)


NAMES = ["attn_decode", "attn_prefill", "kv8", "attn_prep", "conv", "norm_gates", "scan",
         "out_norm"]


def test_every_fixture_is_listed():
    assert sorted(p.stem for p in GOLDEN.glob("*.npz")) == sorted(NAMES)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(orc, name):
    g = load(name)
    for key, want in recompute(orc, name, g).items():
        assert same_bits(want, g[key]), f"{name}: {key} differs from the committed fixture"


def test_fixture_invariants(orc):
    # int8: every stored byte decodes to within half a step of its fp16 value
    g = load("kv8")
    L = g["k"].shape[0]
    for src, buf in (("k", "kc8"), ("v", "vc8")):
        vals, scales = orc.kv8_split(g[buf], L)
        x = g[src].astype(np.float64).reshape(L, 4, 8, 32)
        s = scales.astype(np.float64).reshape(L, 4, 8, 1)
        deq = vals.astype(np.float64).reshape(L, 4, 8, 32) * s
        assert np.all(np.abs(deq - x) <= 0.5 * s + 1e-12)
    # the zero row of the L2 norm stays zero; the others have unit norm
    g = load("norm_gates")
    y = g["y"].astype(np.float64).reshape(2, 8, 128)
    assert not y[1, 2].any()
    n = np.linalg.norm(y, axis=2)
    assert np.all(np.abs(np.delete(n.ravel(), 8 + 2) - 1) < 2e-3)
    # gdn_scalars' known answers (kernels.cu:139-141): x = -40 gives decay 1
    # (softplus ~ 0); x = 100 the softplus branch x itself
    A = np.exp(g["A_log"].astype(np.float64))
    x = g["a"][0, :2].astype(np.float64) + g["dt_bias"][:2]
    want = np.exp(-A[:2] * np.where(x > 20, x, np.log1p(np.exp(x))))
    assert np.allclose(g["decay"][0, :2], want, rtol=1e-5, atol=1e-7)
