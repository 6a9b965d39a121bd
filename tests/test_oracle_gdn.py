"""Pinning the Gated DeltaNet oracle (oracle/fl_oracle.c) on the CPU.

The reference ships no vectors; its kernel comments state what its
(absent) tests pinned, and the mathematics fixes the rest:
  * known answers of gdn_scalars (kernels.cu:139-141): exp(A_log) = 1e-3,
    x = 100 -> decay 0.904837; x = -40 -> 1.0; beta(0) = 0.5; the softplus
    threshold at exactly 20;
  * conv1d: a hand-computed closed form, zero history at pos0 == 0, chunk
    invariance 4+4 == 8 and 2+1 == 3 bit-exact (kernels.cu:135-138), T = 1 at
    pos0 > 0 leaves (s1, s2, x0) (kernels.cu:1620-1622), the verify-rows
    kernel == consecutive T = 1 calls;
  * l2norm: ||y|| = scale ||x|| / sqrt(||x||^2 + eps), zero row -> 0;
  * the delta rule: an independent numpy float64 recurrence; beta = 0 is a
    pure decay; decay = 1, beta = 1, unit k writes v exactly (S k = v);
    contraction over a long run; chunk invariance; checkpoints == the states
    the prefixes leave; the fused decode == conv -> l2norm -> gates -> scan
    bit for bit (kernels.cu:1903-1909 states that equality);
  * the chunked WY scan == the recurrence; chunk 1 is the recurrence.
"""
import numpy as np
import pytest

from conftest import close, f16

QS = 128 ** -0.5


def test_gdn_scalars_known_answers(orc):
    a = np.array([[100.0, -40.0, 0.0, 20.0, 20.0001]], np.float32)
    b = np.array([[0.0, 3.0, -3.0, 0.0, 0.0]], np.float32)
    A_log = np.array([np.log(1e-3), 0, 0, 0, 0], np.float32)
    dt = np.zeros(5, np.float32)
    beta, decay = orc.gdn_scalars(a, b, A_log, dt, T=1, n_heads=5)
    assert abs(decay[0, 0] - 0.904837) < 1e-6
    assert decay[0, 1] == 1.0
    assert abs(decay[0, 2] - np.exp(-np.log(2.0))) < 1e-6
    assert beta[0, 0] == 0.5
    assert abs(beta[0, 1] - 1 / (1 + np.exp(-3.0))) < 1e-7
    assert abs(beta[0, 2] - 1 / (1 + np.exp(3.0))) < 1e-7
    assert abs(decay[0, 3] - np.exp(-np.log1p(np.exp(20.0)))) < 1e-12
    assert abs(decay[0, 4] - np.exp(-20.0001)) < 1e-12
    a2 = a.copy()
    a2[0, 2] = 0.5
    dt2 = np.array([0, 0, 0.25, 0, 0], np.float32)
    _, d2 = orc.gdn_scalars(a2, b, A_log, dt2, T=1, n_heads=5)
    assert abs(d2[0, 2] - np.exp(-np.log1p(np.exp(0.75)))) < 1e-6   # softplus(a + dt_bias)


def test_det_expf_against_libm(orc):
    """The exp both the oracle and the kernels use for silu / sigmoid: within
    2 ulp of the correctly rounded value over the range the path sees."""
    xs = np.concatenate([np.linspace(-87, 88, 20001), np.linspace(-1, 1, 2001),
                         [0.0, -0.0, 1e-8, -1e-8, 20.0, -20.0, 0.5 * np.log(2)]]).astype(np.float32)
    got = np.array([orc.det_expf(x) for x in xs], np.float32)
    want = np.exp(xs.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - want) / ulp).max() <= 2.0
    assert orc.det_expf(100.0) == np.inf and orc.det_expf(-110.0) == 0.0


def test_conv1d_closed_form(orc):
    dim, T = 2, 3
    x = np.array([[1.0, -1.0], [2.0, 0.5], [-3.0, 4.0]], np.float16)
    w = np.array([[0.5, -1.0, 2.0, 0.25], [1.0, 1.0, 1.0, 1.0]], np.float16)
    st = np.array([[1.0, 2.0, 3.0], [-1.0, -2.0, -3.0]], np.float16)
    silu = lambda v: v / (1 + np.exp(-v))
    for pos0 in (0, 7):
        y, so = orc.conv1d_causal(x, w, st, dim=dim, T=T, pos0=pos0, row_stride=dim)
        E = np.concatenate([st.T.astype(np.float64) * (pos0 > 0), x.astype(np.float64)])
        for t in range(T):
            for d in range(dim):
                want = silu(sum(float(w[d, j]) * E[t + j, d] for j in range(4)))
                assert abs(float(y[t, d]) - want) <= 1e-3 * max(1, abs(want))
        assert np.array_equal(so, E[T:T + 3].T.astype(np.float16))


def _conv_inputs(rng, dim=64, T=8):
    x = rng.standard_normal((T, dim)).astype(np.float16)
    w = (rng.standard_normal((dim, 4)) * 0.5).astype(np.float16)
    st = rng.standard_normal((dim, 3)).astype(np.float16)
    return x, w, st


@pytest.mark.parametrize("split", [(4, 4), (2, 1), (1, 1, 1, 5), (3, 5)])
def test_conv1d_chunk_invariance(orc, rng, split):
    T = sum(split)
    x, w, st = _conv_inputs(rng, T=T)
    y_all, s_all = orc.conv1d_causal(x, w, st, dim=64, T=T, pos0=5, row_stride=64)
    s, t0, ys = st, 0, []
    for n in split:
        y, s = orc.conv1d_causal(x[t0:t0 + n], w, s, dim=64, T=n, pos0=5 + t0, row_stride=64)
        ys.append(y)
        t0 += n
    assert np.array_equal(np.concatenate(ys), y_all) and np.array_equal(s, s_all)


def test_conv1d_t1_state(orc, rng):
    x, w, st = _conv_inputs(rng, T=1)
    _, so = orc.conv1d_causal(x, w, st, dim=64, T=1, pos0=3, row_stride=64)
    assert np.array_equal(so, np.stack([st[:, 1], st[:, 2], x[0]], axis=1))


@pytest.mark.parametrize("T", [1, 2, 3])
def test_conv_rows_equals_t1_calls(orc, rng, T):
    x, w, st = _conv_inputs(rng, T=T)
    y, sts = orc.conv1d_causal_rows(x, w, st, dim=64, T=T, pos0=9, row_stride=64)
    s = st
    for t in range(T):
        y1, s = orc.conv1d_causal(x[t:t + 1], w, s, dim=64, T=1, pos0=9 + t, row_stride=64)
        assert np.array_equal(y1[0], y[t]) and np.array_equal(s, sts[t])


@pytest.mark.parametrize("n", [128, 64, 200, 1024])
def test_l2norm(orc, rng, n):
    """||y|| = scale ||x|| / sqrt(||x||^2 + eps) and each y_i = scale x_i / that
    denominator in fp64, within fp16 rounding; a zero row gives 0. Row lengths
    beyond the reference block's 128 threads make each thread sum several
    elements: a sum that dropped them fails the per-element bound."""
    x = rng.standard_normal((2, 3, n)).astype(np.float16)
    x[1, 2] = 0
    for scale in (1.0, QS):
        y = orc.l2norm_scaled(x, n=n, rows=3, pitch=n, eps=1e-6, scale=scale, T=2)
        x64 = x.astype(np.float64)
        xn = np.linalg.norm(x64, axis=-1)
        yn = np.linalg.norm(y.astype(np.float64), axis=-1)
        want = scale * xn / np.sqrt(xn ** 2 + 1e-6)
        assert np.abs(yn - want).max() < 2e-3 * scale
        ye = scale * x64 / np.sqrt(xn ** 2 + 1e-6)[..., None]
        assert np.abs(y.astype(np.float64) - ye).max() <= 2 ** -10 * np.abs(ye).max()
        assert not y[1, 2].any()


# --------------------------------------------------------------------------
# the delta rule
# --------------------------------------------------------------------------

def make_scan_inputs(rng, T, nk=2, nv=6, unit=True, S_scale=0.02):
    K = V = 128
    q = rng.standard_normal((T, nk, K))
    k = rng.standard_normal((T, nk, K))
    if unit:
        q /= np.linalg.norm(q, axis=-1, keepdims=True)
        k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((T, nv, V))
    beta = 1 / (1 + np.exp(-rng.standard_normal((T, nv))))
    decay = np.exp(-np.log1p(np.exp(rng.standard_normal((T, nv)))))
    S0 = rng.standard_normal((nv, V, K)) * S_scale
    return (q.astype(np.float16), k.astype(np.float16), v.astype(np.float16),
            beta.astype(np.float32), decay.astype(np.float32), S0.astype(np.float32))


def numpy_recurrence(q, k, v, beta, decay, S0, group, out_scale=QS):
    """float64 restatement of kernels.cu:1755-1766, independent of the C code."""
    T, nv = beta.shape
    S = S0.astype(np.float64).copy()
    y = np.zeros((T, nv, 128))
    for t in range(T):
        for h in range(nv):
            kk = k[t, h // group].astype(np.float64)
            qq = q[t, h // group].astype(np.float64)
            S[h] *= decay[t, h]
            d = beta[t, h] * (v[t, h].astype(np.float64) - S[h] @ kk)
            S[h] += np.outer(d, kk)
            y[t, h] = (S[h] @ qq) * out_scale
    return y, S


def run_scan(orc, q, k, v, beta, decay, S, ck=None, ck_step=0):
    T, nk, K = q.shape
    nv = v.shape[1]
    return orc.gdn_scan(q, k, v, beta, decay, S, T=T, n_kheads=nk, n_vheads=nv,
                        qk_stride=nk * K, v_stride=nv * 128, out_scale=QS, group=nv // nk,
                        ck=ck, ck_step=ck_step).reshape(T, nv, 128)


def test_scan_matches_float64_recurrence(orc, rng):
    q, k, v, beta, decay, S0 = make_scan_inputs(rng, 64)
    S = S0.copy()
    y = run_scan(orc, q, k, v, beta, decay, S)
    y64, S64 = numpy_recurrence(q, k, v, beta, decay, S0, 3)
    err, ok = close(y, y64, 1e-3, 2e-3)
    assert ok, err
    assert np.abs(S - S64).max() / np.abs(S64).max() < 1e-5


def test_scan_single_token_special_cases(orc, rng):
    q, k, v, beta, decay, S0 = make_scan_inputs(rng, 1)
    # beta = 0: a pure decay
    S = S0.copy()
    run_scan(orc, q, k, v, np.zeros_like(beta), decay, S)
    assert np.allclose(S, S0 * decay[0][:, None, None], rtol=1e-6, atol=0)
    # decay = 1, beta = 1, unit k: the update writes v exactly along k (S k = v)
    S = S0.copy()
    run_scan(orc, q, k, v, np.ones_like(beta), np.ones_like(decay), S)
    for h in range(6):
        sk = S[h].astype(np.float64) @ k[0, h // 3].astype(np.float64)
        kn = np.linalg.norm(k[0, h // 3].astype(np.float64)) ** 2   # 1 up to fp16 rounding
        want = v[0, h].astype(np.float64) + (kn - 1) * (
            v[0, h].astype(np.float64) - S0[h].astype(np.float64) @ k[0, h // 3])
        assert np.abs(sk - want).max() < 2e-5


def test_scan_contraction(orc, rng):
    q, k, v, beta, decay, S0 = make_scan_inputs(rng, 512, S_scale=5.0)
    S = S0.copy()
    run_scan(orc, q, k, v, beta, np.ones_like(decay), S)
    assert np.isfinite(S).all()
    # |S|_F is bounded: each step is a contraction plus beta |v| |k|
    assert np.linalg.norm(S[0]) < np.linalg.norm(S0[0]) + 512 * np.abs(v).max() * np.sqrt(128)


def test_scan_chunk_invariance_and_checkpoints(orc, rng):
    q, k, v, beta, decay, S0 = make_scan_inputs(rng, 8)
    S8 = S0.copy()
    ck = np.zeros((7, 6, 128, 128), np.float32)
    y8 = run_scan(orc, q, k, v, beta, decay, S8, ck=ck, ck_step=6 * 128 * 128)
    S = S0.copy()
    ya = run_scan(orc, q[:4], k[:4], v[:4], beta[:4], decay[:4], S)
    yb = run_scan(orc, q[4:], k[4:], v[4:], beta[4:], decay[4:], S)
    assert np.array_equal(np.concatenate([ya, yb]), y8) and np.array_equal(S, S8)
    S = S0.copy()
    for t in range(7):
        run_scan(orc, q[t:t + 1], k[t:t + 1], v[t:t + 1], beta[t:t + 1], decay[t:t + 1], S)
        assert np.array_equal(S, ck[t])


def _decode_inputs(rng, T, nk=16, nv=48):
    row = 2 * nk * 128 + nv * 128
    c = rng.standard_normal((T, row)).astype(np.float16)
    a = rng.standard_normal((T, nv)).astype(np.float32)
    b = rng.standard_normal((T, nv)).astype(np.float32)
    A_log = (rng.standard_normal(nv) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(nv) * 0.5).astype(np.float32)
    S0 = (rng.standard_normal((nv, 128, 128)) * 0.02).astype(np.float32)
    return c, a, b, A_log, dt, S0


@pytest.mark.parametrize("T", [1, 3])
def test_fused_decode_equals_unfused(orc, rng, T):
    """gdn_scan_rows_f == l2norm_scaled -> gdn_scalars -> gdn_scan, bit for bit."""
    c, a, b, A_log, dt, S0 = _decode_inputs(rng, T)
    S1 = S0.copy()
    ck = np.zeros((max(T - 1, 1), 48, 128, 128), np.float32)
    y1 = orc.gdn_decode(c, S1, a, b, A_log, dt, T=T, out_scale=QS, ck=ck, ck_step=48 * 128 * 128)
    ln = orc.l2norm_scaled(c, n=128, rows=80, pitch=128, eps=1e-6, scale=1.0, T=T)
    beta, decay = orc.gdn_scalars(a, b, A_log, dt, T=T, n_heads=48)
    S2 = S0.copy()
    ck2 = np.zeros_like(ck)
    y2 = orc.gdn_scan(ln[:, :2048], ln[:, 2048:4096], c[:, 4096:], beta, decay, S2, T=T,
                      qk_stride=10240, v_stride=10240, out_scale=QS, ck=ck2,
                      ck_step=48 * 128 * 128)
    assert np.array_equal(y1, y2) and np.array_equal(S1, S2) and np.array_equal(ck, ck2)


def test_fused_conv_decode_equals_conv_then_decode(orc, rng):
    c, a, b, A_log, dt, S0 = _decode_inputs(rng, 1)
    w = (rng.standard_normal((10240, 4)) * 0.5).astype(np.float16)
    st = rng.standard_normal((10240, 3)).astype(np.float16)
    for pos0 in (0, 11):
        S1 = S0.copy()
        so1 = np.zeros_like(st)
        y1 = orc.gdn_decode(None, S1, a, b, A_log, dt, T=1, out_scale=QS, cx=c, cw=w, cst_in=st,
                            cst_out=so1, pos0=pos0)
        cc, so2 = orc.conv1d_causal(c, w, st, dim=10240, T=1, pos0=pos0, row_stride=10240)
        S2 = S0.copy()
        y2 = orc.gdn_decode(cc, S2, a, b, A_log, dt, T=1, out_scale=QS)
        assert np.array_equal(y1, y2) and np.array_equal(S1, S2) and np.array_equal(so1, so2)


@pytest.mark.parametrize("T,chunk", [(64, 64), (200, 64), (37, 16), (9, 1)])
def test_chunked_equals_recurrence(orc, rng, T, chunk):
    q, k, v, beta, decay, S0 = make_scan_inputs(rng, T)
    S_r = S0.copy()
    y_r = run_scan(orc, q, k, v, beta, decay, S_r)
    S_c = S0.copy()
    y_c = orc.gdn_chunked(q, k, v, beta, decay, S_c, T=T, n_kheads=2, n_vheads=6,
                          qk_stride=256, v_stride=768, out_scale=QS, group=3,
                          chunk=chunk).reshape(T, 6, 128)
    err, ok = close(y_c, y_r, 1e-3, 2e-3)
    assert ok, err
    assert np.abs(S_c - S_r).max() / np.abs(S_r).max() < 1e-5


def test_chunked_beta_zero_is_decay(orc, rng):
    q, k, v, beta, decay, S0 = make_scan_inputs(rng, 70)
    S = S0.copy()
    orc.gdn_chunked(q, k, v, np.zeros_like(beta), decay, S, T=70, n_kheads=2, n_vheads=6,
                    qk_stride=256, v_stride=768, out_scale=QS, group=3, chunk=64)
    want = S0.astype(np.float64) * np.prod(decay.astype(np.float64), axis=0)[:, None, None]
    assert np.abs(S - want).max() <= 1e-6 * np.abs(S0).max()


# ---------------------------------------------------------------------------
# rmsnorm_gated (kernels.cu:321-358): plain gamma, norm before the gate
# ---------------------------------------------------------------------------

def test_rmsnorm_gated_closed_form(orc, rng):
    T, rows = 3, 48
    o = f16(rng.standard_normal((T, rows, 128)) * 0.3)
    z = f16(rng.standard_normal((T, rows, 128)) * 2)
    w = (1 + rng.standard_normal(128) * 0.2).astype(np.float32)
    y = orc.rmsnorm_gated(o, z, w, T=T).astype(np.float64)
    of, zf = o.astype(np.float64), z.astype(np.float64)
    silu = zf / (1 + np.exp(-zf))
    want = of / np.sqrt((of ** 2).mean(-1, keepdims=True) + 1e-6) * w * silu
    assert np.abs(y - want).max() <= 2e-3 * np.abs(want).max()
    # (1 + w) instead of w, or the norm over o * silu(z), are far off
    wrong_w = of / np.sqrt((of ** 2).mean(-1, keepdims=True) + 1e-6) * (1 + w) * silu
    g = of * silu
    wrong_gate = g / np.sqrt((g ** 2).mean(-1, keepdims=True) + 1e-6) * w
    for wrong in (wrong_w, wrong_gate):
        assert np.abs(wrong - want).max() > 0.1 * np.abs(want).max()


def test_rmsnorm_gated_zero_gate_and_zero_row(orc):
    o = np.ones((1, 2, 128), np.float16)
    z = np.zeros((1, 2, 128), np.float16)          # silu(0) = 0
    y = orc.rmsnorm_gated(o, z, np.ones(128, np.float32), rows=2, T=1)
    assert not y.any()
    o0 = np.zeros((1, 2, 128), np.float16)          # zero row: no NaN
    y0 = orc.rmsnorm_gated(o0, np.ones((1, 2, 128), np.float16), np.ones(128, np.float32), rows=2, T=1)
    assert np.isfinite(y0.astype(np.float32)).all() and not y0.any()
