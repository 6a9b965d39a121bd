"""Pinning the attention oracle (oracle/fl_oracle.c) on the CPU.

The reference ships no test vectors for this path (its tests/ and _build/
harnesses are absent), so each oracle function is pinned by what the
mathematics and the reference's stated invariants fix:
  * an independent numpy float64 brute force of causal GQA softmax attention
    (query (t, h) sees cache rows [0, pos0 + t] of kv head h // G,
    runtime.py:78-83, kernels.cu:690-707) -- the closed form;
  * known answers: a one-row context returns that v row; zero queries give
    the mean of the visible v rows; the GQA head map lights exactly the q
    heads of one kv head;
  * the reference's invariants: a verify row equals the T = 1 call at its
    position bit for bit (runtime.py:2062-2069), the merge is independent of
    the split count (kernels.cu:1387-1396), empty splits are (m=-1e30, d=0);
  * the gate is a SIGMOID (kernels.cu:1572-1578): gate logit 0 halves z.
"""
import numpy as np
import pytest

from conftest import close, f16, rand_cache, rand_qg

SCALE = 256 ** -0.5


def brute_force(qg, kc, vc, pos0, n_q=24, n_kv=4, hd=256):
    """numpy float64 causal GQA attention, no gate."""
    T = qg.shape[0]
    G = n_q // n_kv
    out = np.zeros((T, n_q, hd))
    q = qg[..., :hd].astype(np.float64)
    k = kc.astype(np.float64)
    v = vc.astype(np.float64)
    for t in range(T):
        n = pos0 + t + 1
        for h in range(n_q):
            s = k[:n, h // G] @ q[t, h] * SCALE
            p = np.exp(s - s.max())
            out[t, h] = p @ v[:n, h // G] / p.sum()
    return out


@pytest.mark.parametrize("L,T", [(1, 1), (5, 1), (33, 3), (300, 2), (700, 4)])
def test_exact_f64_is_the_brute_force(orc, rng, L, T):
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    pos0 = L - T
    want = brute_force(qg, kc, vc, pos0)
    got = orc.attention_exact(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    assert np.abs(got - want).max() < 1e-12


@pytest.mark.parametrize("L,T,split_rows,split", [(1, 1, 32, 32), (40, 1, 32, 32),
                                                  (97, 3, 32, 32), (1500, 2, 32, 32),
                                                  (1500, 3, 512, 64), (4096, 1, 64, 64)])
def test_split_decode_matches_closed_form(orc, rng, L, T, split_rows, split):
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    pos0 = L - T
    z = orc.attention_decode(qg, kc, vc, pos0, max_pos=L, scale=SCALE, split_rows=split_rows,
                             split=split, gate=False)
    want = orc.attention_exact(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    err, ok = close(z, want, 1e-3, 2e-3)
    assert ok, f"split decode vs float64: {err}"


def test_verify_row_equals_t1_call(orc, rng):
    """runtime.py:2062-2069: verify row t is bit-identical to the T=1 decode at pos0+t."""
    L = 2100
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, 3)
    pos0 = L - 3
    pv = orc.attention_split(qg, kc, vc, 0, 24, 4, 256, 512, pos0, L, SCALE, 32, 3, 32)
    for t in range(3):
        p1 = orc.attention_split(qg[t:t + 1], kc, vc, 0, 24, 4, 256, 512, pos0 + t, L, SCALE, 32,
                                 1, 32)
        for a, b in zip(pv, p1):
            assert np.array_equal(a[t:t + 1], b)


def test_empty_splits_and_split_count_independence(orc, rng):
    L = 70   # St = clamp(70 / 32, 1, 32) = 2
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, 1)
    pacc, pm, pd = orc.attention_split(qg, kc, vc, 0, 24, 4, 256, 512, L - 1, L, SCALE, 32, 1, 32)
    assert (pm[..., 2:] == np.float32(-1e30)).all() and (pd[..., 2:] == 0).all()
    assert (pacc[:, :, 2:] == 0).all()
    z_many = orc.attention_merge(pacc, pm, pd, 24, 256, 1, 32)
    p1 = orc.attention_split(qg, kc, vc, 0, 24, 4, 256, 512, L - 1, L, SCALE, 10 ** 6, 1, 1)
    z_one = orc.attention_merge(*p1, 24, 256, 1, 1)
    err, ok = close(z_many, z_one, 1e-3, 2e-3)
    assert ok, err


def test_one_row_context_returns_v(orc, rng):
    kc, vc = rand_cache(rng, 1)
    qg = rand_qg(rng, 1, q_scale=1.0)
    z = orc.attention_decode(qg, kc, vc, 0, max_pos=1, scale=SCALE, gate=False)
    for h in range(24):
        assert np.array_equal(z[0, h], vc[0, h // 6])


def test_zero_query_gives_mean_of_v(orc, rng):
    L = 257
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, 1)
    qg[..., :256] = 0
    z = orc.attention_decode(qg, kc, vc, L - 1, max_pos=L, scale=SCALE, gate=False)
    want = vc.astype(np.float64).mean(axis=0)
    for h in range(24):
        err, ok = close(z[0, h], want[h // 6], 1e-3, 2e-3)
        assert ok, err


def test_gqa_head_map(orc, rng):
    """q head h reads kv head h // 6: only kv head 2's V is non-zero."""
    L = 100
    kc, vc = rand_cache(rng, L)
    vc[:, [0, 1, 3]] = 0
    qg = rand_qg(rng, 1)
    z = orc.attention_decode(qg, kc, vc, L - 1, max_pos=L, scale=SCALE, gate=False)
    nz = [h for h in range(24) if np.abs(z[0, h].astype(np.float32)).max() > 0]
    assert nz == list(range(12, 18))


def test_gate_is_sigmoid(orc, rng):
    L = 50
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, 1)
    z0 = orc.attention_decode(qg, kc, vc, L - 1, max_pos=L, scale=SCALE, gate=False)
    for logit, factor in ((0.0, 0.5), (30.0, 1.0), (-30.0, 0.0)):
        qg[..., 256:] = logit
        z = orc.attention_decode(qg, kc, vc, L - 1, max_pos=L, scale=SCALE, gate=True)
        want = (z0.astype(np.float32) * np.float32(factor)).astype(np.float16)
        assert np.array_equal(z, want), logit


@pytest.mark.parametrize("T,pos0", [(8, 0), (13, 0), (40, 3), (130, 70)])
@pytest.mark.parametrize("pv_fp16", [False, True])
def test_prefill_matches_closed_form(orc, rng, T, pos0, pv_fp16):
    L = pos0 + T
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    z = orc.attention_prefill(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T,
                              pv_fp16=pv_fp16)
    want = orc.attention_exact(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    err, ok = close(z, want, 2e-3 if pv_fp16 else 1e-3, 1e-2 if pv_fp16 else 2e-3)
    assert ok, f"prefill vs float64: {err}"


def test_prefill_row_equals_decode_row(orc, rng):
    T, pos0 = 20, 45
    L = pos0 + T
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    zp = orc.attention_prefill(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    zd = orc.attention_decode(qg, kc, vc, pos0, max_pos=L, scale=SCALE, gate=False,
                              split=32, split_rows=32)
    err, ok = close(zp, zd, 1e-3, 4e-3)
    assert ok, err


def test_kv_store_positions(orc, rng):
    layers, max_pos, T, pos0, layer = 3, 40, 5, 17, 2
    kc = np.zeros((layers, max_pos, 4, 256), np.float16)
    vc = np.zeros_like(kc)
    k = rng.standard_normal((T, 4, 256)).astype(np.float16)
    v = rng.standard_normal((T, 4, 256)).astype(np.float16)
    orc.kv_store(k, v, kc, vc, layer, pos0, 4, 256, max_pos, T)
    assert np.array_equal(kc[layer, pos0:pos0 + T], k) and np.array_equal(vc[layer, pos0:pos0 + T], v)
    kc[layer, pos0:pos0 + T] = 0
    vc[layer, pos0:pos0 + T] = 0
    assert not kc.any() and not vc.any()


def test_f16_sat(orc):
    assert orc.f16_sat(1e6) == np.float16(65504)
    assert orc.f16_sat(-1e6) == np.float16(-65504)
    assert np.isnan(orc.f16_sat(float("nan")))
    for x in (0.1, 1 / 3, 65519.0, 6e-8, 3e-8, 2.98e-8, -1.5e-5, 1.0009765625 + 2 ** -11):
        assert orc.f16_sat(x) == np.float16(x), x


def test_attention_split_rejects_nothing_silently(orc, rng):
    """An all-equal-score context: the merged output is the plain mean of V
    (pins the natural-exp merge of partials with identical maxima)."""
    L = 1000
    kc = np.zeros((L, 4, 256), np.float16)
    vc = f16(rng.standard_normal((L, 4, 256)))
    qg = rand_qg(rng, 1)
    z = orc.attention_decode(qg, kc, vc, L - 1, max_pos=L, scale=SCALE, gate=False)
    err, ok = close(z[0], np.repeat(vc.astype(np.float64).mean(0), 6, axis=0), 1e-3, 2e-3)
    assert ok, err
