"""The HIP path on the committed golden fixtures (tests/golden/*.npz, the C
oracle's outputs on seeded inputs; tests/test_golden.py pins them to the
oracle), through the op layer and the C ABI, at the bars the other GPU tests
use: attention max-abs 2e-3 / rel 1e-2 and max|err| <= 1e-2 max|want|; the
int8 store and the KV rows bit for bit; prep, conv, norms <= 1 fp16 ulp and
the conv state bit for bit; gates within 2e-7 (beta) / 2e-6 rel (decay); the
delta-rule state rel <= 1e-4 and y within the attention bar -- for the
recurrent scan and for the chunked scan, both against the recurrence."""
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import close, close_rel

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
ATOL, RTOL = 2e-3, 1e-2
STATE_RTOL = 1e-4


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def dev_(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def ulps(a, b):
    ai = np.asarray(a).view(np.int16).astype(np.int32)
    bi = np.asarray(b).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return int(np.abs(ai - bi).max())


def rel(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / np.abs(want).max())


def test_golden_attn_decode(fl, dev):
    g = load("attn_decode")
    z = fl.ops.attn_decode(dev_(g["qg"][None], dev), [dev_(g["kc"], dev)], [dev_(g["vc"], dev)],
                           [int(g["pos0"])])
    torch.cuda.synchronize()
    err, ok = close_rel(z[0].cpu().numpy(), g["z"], ATOL, RTOL)
    assert ok, f"max|err| {err}"


def test_golden_attn_prefill(fl, dev):
    g = load("attn_prefill")
    z = fl.ops.attention_prefill(dev_(g["qg"], dev), dev_(g["kc"], dev), dev_(g["vc"], dev),
                                 pos0=int(g["pos0"]))
    torch.cuda.synchronize()
    err, ok = close_rel(z.cpu().numpy(), g["z"], ATOL, RTOL)
    assert ok, f"max|err| {err}"


def test_golden_kv8_store_and_decode(fl, dev):
    g = load("kv8")
    L = g["k"].shape[0]
    kd, vd = fl.ops.kv8_cache(L), fl.ops.kv8_cache(L)
    fl.ops.kv_store_q8(dev_(g["k"], dev), dev_(g["v"], dev), kd, vd, pos0=0, max_pos=L)
    z = fl.ops.attn_decode_q8(dev_(g["qg"][None], dev), [kd], [vd], [int(g["pos0"])], [L])
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), g["kc8"]) and np.array_equal(vd.cpu().numpy(),
                                                                          g["vc8"])
    err, ok = close_rel(z[0].cpu().numpy(), g["z"], ATOL, RTOL)
    assert ok, f"max|err| {err}"


def test_golden_attn_prep(fl, dev):
    g = load("attn_prep")
    T, pos0 = g["qg"].shape[0], int(g["pos0"])
    qd, kd, vd = dev_(g["qg"], dev), dev_(g["k"], dev), dev_(g["v"], dev)
    kc = torch.zeros((pos0 + T, 4, 256), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    fl.ops.attn_prep(qd, kd, vd, dev_(g["wq"], dev), dev_(g["wk"], dev), kc, vc, pos0=pos0)
    torch.cuda.synchronize()
    q, k = qd.cpu().numpy(), kd.cpu().numpy()
    assert ulps(q, g["q_out"]) <= 1 and ulps(k, g["k_out"]) <= 1
    assert np.array_equal(kc.cpu().numpy()[pos0:], k)
    assert np.array_equal(vc.cpu().numpy()[pos0:], g["v"])


def test_golden_conv(fl, dev):
    g = load("conv")
    T, dim = g["x"].shape
    y = torch.zeros((T, dim), dtype=torch.float16, device=dev)
    so = torch.empty(g["st"].shape, dtype=torch.float16, device=dev)
    fl.ops.conv1d_causal(dev_(g["x"], dev), dev_(g["w"], dev), dev_(g["st"], dev), y, so,
                         dim=dim, T=T, pos0=int(g["pos0"]), row_stride=dim)
    torch.cuda.synchronize()
    assert ulps(y.cpu().numpy(), g["y"]) <= 1
    assert np.array_equal(so.cpu().numpy(), g["st_out"])


def test_golden_norm_and_gates(fl, dev):
    g = load("norm_gates")
    T = g["x"].shape[0]
    y = torch.zeros(g["x"].shape, dtype=torch.float16, device=dev)
    fl.ops.l2norm_scaled(dev_(g["x"], dev), y, rows=8, T=T)
    Tg = g["a"].shape[0]
    beta = torch.empty((Tg, 48), dtype=torch.float32, device=dev)
    decay = torch.empty_like(beta)
    fl.ops.gdn_scalars(dev_(g["a"], dev), dev_(g["b"], dev), dev_(g["A_log"], dev),
                       dev_(g["dt_bias"], dev), beta, decay, T=Tg)
    torch.cuda.synchronize()
    assert ulps(y.cpu().numpy(), g["y"]) <= 1
    assert np.abs(beta.cpu().numpy() - g["beta"]).max() <= 2e-7
    assert np.abs(decay.cpu().numpy() - g["decay"]).max() / g["decay"].max() <= 2e-6


@pytest.mark.parametrize("form", ["recurrent", "chunked"])
def test_golden_scan(fl, dev, form):
    g = load("scan")
    T = g["q"].shape[0]
    q, k, v = dev_(g["q"], dev), dev_(g["k"], dev), dev_(g["v"], dev)
    beta, decay = dev_(g["beta"], dev), dev_(g["decay"], dev)
    S = dev_(g["S0"], dev)
    geo = dict(T=T, n_kheads=1, n_vheads=3, qk_stride=128, v_stride=384)
    if form == "recurrent":
        y = torch.empty((T, 384), dtype=torch.float16, device=dev)
        fl.ops.gdn_scan(q, k, v, beta, decay, S, y, **geo)
    else:
        y = fl.ops.gdn_prefill_chunked(q, k, v, beta, decay, S, **geo)
    torch.cuda.synchronize()
    assert rel(S.cpu().numpy(), g["S"]) <= STATE_RTOL
    err, ok = close(y.cpu().numpy(), g["y"], ATOL, RTOL)
    assert ok, f"{form}: max|dy| {err}"


def test_golden_out_norm(fl, dev):
    g = load("out_norm")
    y = fl.ops.rmsnorm_gated(dev_(g["o"], dev), dev_(g["z"], dev), dev_(g["w"], dev),
                             T=g["o"].shape[0])
    torch.cuda.synchronize()
    assert ulps(y.cpu().numpy(), g["y"]) <= 1
