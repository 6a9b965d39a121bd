"""Pinning the int8 KV cache oracle (oracle/fl_oracle.c) on the CPU.

The reference ships no vectors for its int8 path either; each function is
pinned by what the format and the mathematics fix:
  * kv_store_q8 (kernels.cu:486-520) against a numpy closed form of the
    format -- per 32 dims scale = f16(absmax / 127), value =
    clip(rint(x / scale), -127, 127), 0 where the scale is 0 -- on inputs
    where the plausible mistakes (absmax / 128, truncation instead of
    round-half-even, dividing by the unrounded scale) give different bytes;
    known answers: a block whose absmax is 127 has scale 1 and stores
    rint(x); a zero block stores scale 0 and zeros; the values sit at
    [pos][head][dim], the scales at byte max_pos * n_kv * 256 as
    [pos][head][block];
  * attention_dec_q8 + attention_dec_merge and attention_prefill_fh_q8
    against a numpy float64 brute force of causal GQA softmax attention over
    the exactly dequantized cache (byte * scale) -- the closed form;
  * the reference's invariants: a verify row equals the T = 1 call at its
    position bit for bit (runtime.py:2062-2069); the merged output does not
    depend on (tmin, smax) beyond rounding; splits s >= St are not written
    (kernels.cu:1107-1118); the merge's gate is a sigmoid.
"""
import numpy as np
import pytest

from conftest import close, f16, rand_qg

SCALE = 256 ** -0.5
LOG2E = 1.4426950408889634


def q8_closed(x):
    """numpy closed form of the int8 format: (values int8 like x, scales
    float16 [..., 8])."""
    xb = np.asarray(x, np.float16).astype(np.float32).reshape(*x.shape[:-1], -1, 32)
    a = np.abs(xb).max(-1)
    sh = (a / np.float32(127)).astype(np.float16)
    sc = sh.astype(np.float32)[..., None]
    with np.errstate(divide="ignore", invalid="ignore"):
        qv = np.where(sc > 0, np.clip(np.rint(xb / sc), -127, 127), 0)
    return qv.astype(np.int8).reshape(x.shape), sh


def rand_kv(rng, T, n_kv=4, hd=256, lo=-3.0, hi=2.0):
    """fp16 rows whose 32-dim blocks span magnitudes 10^lo .. 10^hi."""
    mag = 10.0 ** rng.uniform(lo, hi, (T, n_kv, hd // 32, 1))
    x = rng.standard_normal((T, n_kv, hd // 32, 32)) * mag
    return f16(x.reshape(T, n_kv, hd))


def deq(orc, buf, max_pos):
    vals, sc = orc.kv8_split(buf, max_pos)
    return vals.astype(np.float64) * np.repeat(sc.astype(np.float64), 32, axis=-1)


def brute(qg, kd, vd, pos0, n_q=24, n_kv=4, hd=256):
    T = qg.shape[0]
    G = n_q // n_kv
    out = np.zeros((T, n_q, hd))
    q = qg[..., :hd].astype(np.float64)
    for t in range(T):
        n = pos0 + t + 1
        for h in range(n_q):
            s = kd[:n, h // G] @ q[t, h] * SCALE
            p = np.exp(s - s.max())
            out[t, h] = p @ vd[:n, h // G] / p.sum()
    return out


def filled(orc, rng, L, max_pos=None):
    """int8 caches holding L random rows (block magnitudes 0.03 .. 3); returns
    (kc8, vc8, max_pos)."""
    max_pos = L if max_pos is None else max_pos
    kc8, vc8 = orc.kv8_buffer(max_pos), orc.kv8_buffer(max_pos)
    k, v = rand_kv(rng, L, lo=-1.5, hi=0.5), rand_kv(rng, L, lo=-1.5, hi=0.5)
    orc.kv_store_q8(k, v, kc8, vc8, 0, max_pos, L)
    return kc8, vc8, max_pos


def test_kv_store_q8_closed_form_and_layout(orc, rng):
    T, pos0, max_pos = 5, 3, 16
    k, v = rand_kv(rng, T), rand_kv(rng, T)
    k[0, 0, :32] = 0                                            # a zero block
    k[0, 1, :32] = f16(np.r_[127.0, -126.0, 2.5, 3.5, -4.5, 0.5, -0.5, 1.5, np.zeros(24)])
    kc8, vc8 = orc.kv8_buffer(max_pos), orc.kv8_buffer(max_pos)
    orc.kv_store_q8(k, v, kc8, vc8, pos0, max_pos, T)
    for x, buf in ((k, kc8), (v, vc8)):
        vals, sc = orc.kv8_split(buf, max_pos)
        want_v, want_s = q8_closed(x)
        assert np.array_equal(vals[pos0:pos0 + T], want_v)
        assert np.array_equal(sc[pos0:pos0 + T].view(np.uint16), want_s.view(np.uint16))
        assert not vals[:pos0].any() and not vals[pos0 + T:].any()
        assert not sc[:pos0].view(np.uint16).any() and not sc[pos0 + T:].view(np.uint16).any()
    vals, sc = orc.kv8_split(kc8, max_pos)
    assert sc[pos0, 0, 0] == 0 and not vals[pos0, 0, :32].any()
    # absmax 127: scale 1, rint with ties to even
    assert sc[pos0, 1, 0] == 1.0
    assert list(vals[pos0, 1, :8]) == [127, -126, 2, 4, -4, 0, 0, 2]


def test_kv_store_q8_rejects_plausible_mistakes(orc, rng):
    """The inputs above make each plausible mistake visible: the closed form is
    not satisfied by an absmax / 128 scale, truncation, or dividing by the
    unrounded absmax / 127."""
    x = rand_kv(rng, 64)
    good_v, good_s = q8_closed(x)
    xb = x.astype(np.float32).reshape(64, 4, 8, 32)
    a = np.abs(xb).max(-1, keepdims=True)
    s128 = (a / np.float32(128)).astype(np.float16).astype(np.float32)
    s127 = (a / np.float32(127)).astype(np.float16).astype(np.float32)
    raw = a / np.float32(127)
    with np.errstate(divide="ignore", invalid="ignore"):
        m1 = np.clip(np.rint(xb / s128), -127, 127)
        m2 = np.clip(np.trunc(xb / s127), -127, 127)
        m3 = np.clip(np.rint(xb / raw), -127, 127)
    for m in (m1, m2, m3):
        assert not np.array_equal(m.astype(np.int8).reshape(x.shape), good_v)
    kc8, vc8 = orc.kv8_buffer(64), orc.kv8_buffer(64)
    orc.kv_store_q8(x, x, kc8, vc8, 0, 64, 64)
    vals, sc = orc.kv8_split(kc8, 64)
    assert np.array_equal(vals, good_v) and np.array_equal(sc.view(np.uint16), good_s.view(np.uint16))
    # the dequantized value is within half a scale step of the input
    err = np.abs(deq(orc, kc8, 64) - x.astype(np.float64))
    step = np.repeat(sc.astype(np.float64), 32, axis=-1)
    assert (err <= 0.5 * step * (1 + 2e-3) + 1e-12).all()


@pytest.mark.parametrize("L,T", [(1, 1), (40, 2), (300, 3)])
def test_exact_f64_q8_is_the_brute_force(orc, rng, L, T):
    kc8, vc8, _ = filled(orc, rng, L)
    qg = rand_qg(rng, T)
    want = brute(qg, deq(orc, kc8, L), deq(orc, vc8, L), L - T)
    got = orc.attention_exact_q8(qg, kc8, vc8, q_pitch=512, pos0=L - T, max_pos=L, scale=SCALE, T=T)
    assert np.abs(got - want).max() < 1e-12


@pytest.mark.parametrize("L,T,tmin,smax", [(1, 1, 1, 28), (64, 1, 1, 28), (65, 2, 1, 28),
                                           (700, 3, 1, 28), (3000, 1, 1, 28), (3000, 3, 4, 8),
                                           (5000, 2, 1, 3)])
def test_dec_q8_matches_closed_form(orc, rng, L, T, tmin, smax):
    kc8, vc8, _ = filled(orc, rng, L, L + 5)
    qg = rand_qg(rng, T)
    pos0 = L - T
    z = orc.attention_decode_q8(qg, kc8, vc8, pos0, max_pos=L + 5, scale=SCALE, tmin=tmin,
                                smax=smax, gate=False)
    want = brute(qg, deq(orc, kc8, L + 5), deq(orc, vc8, L + 5), pos0)
    err, ok = close(z, want, 1e-3, 2e-3)
    assert ok, f"dec_q8 vs float64: {err}"


def test_dec_q8_verify_row_equals_t1_call(orc, rng):
    L, T = 2000, 3
    kc8, vc8, _ = filled(orc, rng, L)
    qg = rand_qg(rng, T)
    pos0 = L - T
    pa, pm, pd = orc.attention_dec_q8(qg, kc8, vc8, pos0=pos0, max_pos=L, sl2=SCALE * LOG2E, T=T)
    for t in range(T):
        a1, m1, d1 = orc.attention_dec_q8(qg[t:t + 1], kc8, vc8, pos0=pos0 + t, max_pos=L,
                                          sl2=SCALE * LOG2E, T=1)
        st = orc.dec_split_count(pos0 + t + 1, 1, 28)
        assert np.array_equal(pa[t, :, :st], a1[0, :, :st])
        assert np.array_equal(pm[t, :, :st], m1[0, :, :st])
        assert np.array_equal(pd[t, :, :st], d1[0, :, :st])
        assert np.isnan(pm[t, :, st:]).all()                     # not written


def test_dec_q8_split_independence(orc, rng):
    L, T = 4000, 2
    kc8, vc8, _ = filled(orc, rng, L)
    qg = rand_qg(rng, T)
    zs = [orc.attention_decode_q8(qg, kc8, vc8, L - T, max_pos=L, scale=SCALE, tmin=tm, smax=sm,
                                  gate=False)
          for tm, sm in ((1, 28), (1, 1), (2, 5), (8, 64))]
    for z in zs[1:]:
        err, ok = close(z, zs[0], 2e-3, 0)
        assert ok, err
    # (1, 28) and (1, 1) really split differently
    assert orc.dec_split_count(L, 1, 28) == 28 and orc.dec_split_count(L, 1, 1) == 1


def test_dec_merge_gate_is_sigmoid(orc, rng):
    L, T = 300, 2
    kc8, vc8, _ = filled(orc, rng, L)
    qg = rand_qg(rng, T)
    qg[..., 256:] = 0                                            # sigmoid(0) = 1/2
    z0 = orc.attention_decode_q8(qg, kc8, vc8, L - T, max_pos=L, scale=SCALE, gate=False)
    zg = orc.attention_decode_q8(qg, kc8, vc8, L - T, max_pos=L, scale=SCALE, gate=True)
    assert np.array_equal(zg, f16(z0.astype(np.float32) * np.float32(0.5)))


@pytest.mark.parametrize("T,pos0,pv_fp16", [(1, 0, False), (70, 0, False), (40, 100, True),
                                            (130, 37, False)])
def test_prefill_q8_matches_closed_form(orc, rng, T, pos0, pv_fp16):
    L = pos0 + T
    kc8, vc8, _ = filled(orc, rng, L)
    qg = rand_qg(rng, T)
    z = orc.attention_prefill_q8(qg, kc8, vc8, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T,
                                 pv_fp16=pv_fp16)
    want = brute(qg, deq(orc, kc8, L), deq(orc, vc8, L), pos0)
    err, ok = close(z, want, 1e-3, 2e-3)
    assert ok, f"prefill_q8 vs float64: {err}"
