"""Pinning the attention-prep oracle (rmsnorm1p, rope_partial, attn_prep) on the CPU.

No reference vectors exist for these kernels; each is pinned by what the
mathematics fixes, with inputs chosen so a plausible mistake fails:
  * rmsnorm1p against a float64 closed form y = x / sqrt(mean(x^2) + eps) *
    (1 + w) (kernels.cu:241-272) -- on rows small enough that a SUM-space eps
    (l2norm_scaled's convention) or a missing "1 +" would be far off;
    a zero row gives zeros, not NaN (kernels.cu:250-251);
  * rope_partial against a float64 rotation of the NeoX pairs (j, j + 32)
    with frequency theta^(-2j / 64) over the ROTARY width (kernels.cu:
    401-406) -- interleaved pairs or a head_dim-wide frequency would fail;
    position 0 is the identity bit for bit; dims >= 64 are untouched bit for
    bit (kernels.cu:400); pair norms are preserved;
  * attn_prep is the composition the runtime launches (runtime.py:2797-2815):
    the cache rows are the roped k rows and the v rows, bit for bit.
"""
import numpy as np
import pytest

from conftest import f16


def ulp16(a, b):
    """max distance in fp16 units in the last place (same-sign finite values)."""
    ia = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    ib = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    return int(np.abs(ia - ib).max())


def rms_closed(x, w, eps):
    x = x.astype(np.float64)
    return x / np.sqrt((x ** 2).mean(-1, keepdims=True) + eps) * (1.0 + w.astype(np.float64))


@pytest.mark.parametrize("scale", [1.0, 1e-3])
def test_rmsnorm1p_closed_form(orc, rng, scale):
    T, rows = 3, 24
    x = f16(rng.standard_normal((T, rows, 512)) * scale)
    w = (rng.standard_normal(256) * 0.3).astype(np.float32)
    y = orc.rmsnorm1p(x, w, rows=rows, pitch=512, T=T, eps=1e-6)
    want = rms_closed(x[..., :256], w, 1e-6)
    assert ulp16(y[..., :256], f16(want)) <= 1
    assert np.array_equal(y[..., 256:], x[..., 256:])          # the gate half is not touched
    # a sum-space eps or (w instead of 1 + w) is far off on these rows
    wrong_eps = x[..., :256].astype(np.float64) / np.sqrt(
        (x[..., :256].astype(np.float64) ** 2).sum(-1, keepdims=True) + 1e-6) * (1 + w)
    assert np.abs(wrong_eps - want).max() > 0.1 * np.abs(want).max()
    wrong_w = rms_closed(x[..., :256], w - 1, 1e-6)
    assert np.abs(wrong_w - want).max() > 0.1 * np.abs(want).max()


def test_rmsnorm1p_zero_row(orc):
    x = np.zeros((1, 4, 256), np.float16)
    y = orc.rmsnorm1p(x, np.ones(256, np.float32), rows=4, pitch=256, T=1, eps=1e-6)
    assert np.isfinite(y.astype(np.float32)).all() and not y.any()


def rope_closed(x, pos, rope_dim=64, theta=1e7):
    """float64 NeoX rotation of one row of fp16 values."""
    y = x.astype(np.float64).copy()
    half = rope_dim // 2
    j = np.arange(half)
    ang = pos * theta ** (-2.0 * j / rope_dim)
    x0, x1 = y[:half].copy(), y[half:rope_dim].copy()
    y[:half] = x0 * np.cos(ang) - x1 * np.sin(ang)
    y[half:rope_dim] = x1 * np.cos(ang) + x0 * np.sin(ang)
    return y


@pytest.mark.parametrize("pos0", [0, 7, 100_000])
def test_rope_partial_closed_form(orc, rng, pos0):
    T = 3
    q = f16(rng.standard_normal((T, 24, 512)))
    k = f16(rng.standard_normal((T, 4, 256)))
    qr, kr = orc.rope_partial(q, k, n_q_heads=24, n_kv_heads=4, q_pitch=512, k_pitch=256,
                              pos0=pos0, T=T)
    assert np.array_equal(qr[..., 64:], q[..., 64:]) and np.array_equal(kr[..., 64:], k[..., 64:])
    worst = 0
    for t in range(T):
        for h in range(24):
            want = rope_closed(q[t, h, :256], pos0 + t)
            worst = max(worst, ulp16(qr[t, h, :64], f16(want[:64])))
        for h in range(4):
            want = rope_closed(k[t, h], pos0 + t)
            worst = max(worst, ulp16(kr[t, h, :64], f16(want[:64])))
    assert worst <= 1
    # norms of the (j, j + 32) pairs are kept (to fp16 rounding)
    n_in = q[..., :32].astype(np.float64) ** 2 + q[..., 32:64].astype(np.float64) ** 2
    n_out = qr[..., :32].astype(np.float64) ** 2 + qr[..., 32:64].astype(np.float64) ** 2
    assert np.allclose(n_in, n_out, rtol=5e-3, atol=1e-3)


def test_rope_partial_position0_identity_and_known_answer(orc):
    q = np.zeros((2, 1, 256), np.float16)
    q[:, 0, 0] = 1.0                       # pair j = 0 (frequency 1): x = (1, 0)
    q[:, 0, 31] = 1.0                      # pair j = 31
    k = q.copy()
    qr, _ = orc.rope_partial(q, k, n_q_heads=1, n_kv_heads=1, q_pitch=256, k_pitch=256,
                             pos0=0, T=2)
    assert np.array_equal(qr[0], q[0])     # position 0: identity, bit for bit
    # position 1, pair 0: (cos 1, sin 1) in slots 0 and 32
    assert qr[1, 0, 0] == np.float16(np.cos(1.0)) and qr[1, 0, 32] == np.float16(np.sin(1.0))
    # pair 31 rotates by theta^(-62/64) over the 64-wide rotary part, not 256
    a = 1e7 ** (-62 / 64)
    assert qr[1, 0, 31] == np.float16(np.cos(a)) and qr[1, 0, 63] == np.float16(np.sin(a))
    a_wrong = 1e7 ** (-62 / 256)
    assert np.float16(np.sin(a_wrong)) != qr[1, 0, 63]


def test_attn_prep_composition(orc, rng):
    T, pos0, max_pos = 4, 9, 16
    qg = f16(rng.standard_normal((T, 24, 512)))
    k = f16(rng.standard_normal((T, 4, 256)))
    v = f16(rng.standard_normal((T, 4, 256)))
    wq = (rng.standard_normal(256) * 0.2).astype(np.float32)
    wk = (rng.standard_normal(256) * 0.2).astype(np.float32)
    kc = np.zeros((max_pos, 4, 256), np.float16)
    vc = np.zeros_like(kc)
    qo, ko = orc.attn_prep(qg, k, v, wq, wk, kc, vc, pos0=pos0, T=T, max_pos=max_pos)
    assert np.array_equal(kc[pos0:pos0 + T], ko) and np.array_equal(vc[pos0:pos0 + T], v)
    assert not kc[:pos0].any() and not kc[pos0 + T:].any()
    assert np.array_equal(qo[..., 256:], qg[..., 256:])     # the gate half stays
    want = rope_closed(rms_closed(k[1, 2], wk, 1e-6).astype(np.float16), pos0 + 1)
    assert ulp16(ko[1, 2], f16(want)) <= 2
