"""The PyTorch fp32 CPU implementation (oracle/torch_ref.py, bench.py's CPU
baseline) agrees with the C oracle on the same inputs.

torch sums in its own fp32 order and uses its own exp, so an fp32 value that
is then rounded to fp16 (a normalised q / k element, a conv output) can land
one fp16 ulp away from the oracle's; such a flip moves the fp32 state by
~|delta| * ulp(k) after one step (~2e-4 of max |S|). The state bound for this
baseline is therefore 1e-3, not the parity bar the kernels are held to."""
import numpy as np
import torch

from conftest import close, rand_cache, rand_qg
from oracle import torch_ref as tr

SCALE = 256 ** -0.5
QS = 128 ** -0.5


def test_attention_decode(orc, rng):
    L, T = 900, 3
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    z = tr.attention_decode(torch.from_numpy(qg), torch.from_numpy(kc), torch.from_numpy(vc),
                            L - T, SCALE)
    want = orc.attention_decode(qg, kc, vc, L - T, max_pos=L, scale=SCALE)
    err, ok = close(z.numpy(), want, 2e-3, 1e-2)
    assert ok, err


def test_attention_prefill(orc, rng):
    T, pos0 = 150, 20
    L = pos0 + T
    kc, vc = rand_cache(rng, L)
    q = rand_qg(rng, T)[..., :256].copy()
    z = tr.attention_prefill(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc),
                             pos0, SCALE, block=64)
    want = orc.attention_exact(q, kc, vc, q_pitch=256, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    err, ok = close(z.numpy(), want, 2e-3, 1e-2)
    assert ok, err
    part = tr.attention_prefill(torch.from_numpy(q), torch.from_numpy(kc), torch.from_numpy(vc),
                                pos0, SCALE, rows=slice(100, 130))
    assert torch.equal(part, z[100:130]) or np.abs(part.float().numpy() - z[100:130].float().numpy()).max() < 2e-3


def test_gdn_decode_step(orc, rng):
    B = 2
    x = rng.standard_normal((B, 10240)).astype(np.float16)
    w = (rng.standard_normal((10240, 4)) * 0.5).astype(np.float16)
    st = rng.standard_normal((B, 10240, 3)).astype(np.float16)
    S0 = (rng.standard_normal((B, 48, 128, 128)) * 0.02).astype(np.float32)
    a = rng.standard_normal((B, 48)).astype(np.float32)
    b = rng.standard_normal((B, 48)).astype(np.float32)
    A_log = (rng.standard_normal(48) * 0.3).astype(np.float32)
    dt = (rng.standard_normal(48) * 0.3).astype(np.float32)
    S_t = torch.from_numpy(S0.copy())
    y, so = tr.gdn_decode_step(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(st),
                               S_t, torch.from_numpy(a), torch.from_numpy(b),
                               torch.from_numpy(A_log), torch.from_numpy(dt), pos0=3)
    for i in range(B):
        S_r = S0[i].copy()
        so_r = np.zeros((10240, 3), np.float16)
        y_r = orc.gdn_decode(None, S_r, a[i:i + 1], b[i:i + 1], A_log, dt, T=1, out_scale=QS,
                             cx=x[i:i + 1], cw=w, cst_in=st[i], cst_out=so_r, pos0=3)
        err, ok = close(y[i].numpy(), y_r[0], 2e-3, 1e-2)
        assert ok, err
        assert np.abs(S_t[i].numpy() - S_r).max() / np.abs(S_r).max() < 1e-3
        assert np.array_equal(so[i].numpy(), so_r)


def test_gdn_recurrence_and_chunked(orc, rng):
    T, nk, nv = 100, 2, 6
    q = rng.standard_normal((T, nk, 128))
    k = rng.standard_normal((T, nk, 128))
    q = (q / np.linalg.norm(q, axis=-1, keepdims=True)).astype(np.float16)
    k = (k / np.linalg.norm(k, axis=-1, keepdims=True)).astype(np.float16)
    v = rng.standard_normal((T, nv, 128)).astype(np.float16)
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, nv))))).astype(np.float32)
    decay = np.exp(-np.log1p(np.exp(rng.standard_normal((T, nv))))).astype(np.float32)
    S0 = (rng.standard_normal((nv, 128, 128)) * 0.02).astype(np.float32)
    S_r = S0.copy()
    y_r = orc.gdn_scan(q, k, v, beta, decay, S_r, T=T, n_kheads=nk, n_vheads=nv,
                       qk_stride=nk * 128, v_stride=nv * 128, out_scale=QS, group=3)
    args = [torch.from_numpy(a) for a in (q, k, v, beta, decay)]
    S1 = torch.from_numpy(S0.copy())
    y1 = tr.gdn_recurrence(*args, S1)
    S2 = torch.from_numpy(S0.copy())
    y2 = tr.gdn_chunked(*args, S2)
    for y, S in ((y1, S1), (y2, S2)):
        err, ok = close(y.numpy(), y_r, 2e-3, 1e-2)
        assert ok, err
        assert np.abs(S.numpy() - S_r).max() / np.abs(S_r).max() < 1e-4
