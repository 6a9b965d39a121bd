"""Seeded random shapes through the HIP path against the oracle: the shapes a
hand-picked list misses (ragged lengths, one-row contexts, capacities beyond
the length, batches of up to 10 sequences at unrelated positions, forced KV
splits from 1 to 9, verify rows 1..5, scan lengths 1..300, GDN decode batches
of up to 12 with the conv fused or verify rows with checkpoints, the fused
attention prep at positions up to ~200k, conv1d over odd channel counts and
widths 1..8). Each case prints
its shape before it runs, and every comparison uses the attention bar with the
relative-to-max check, the state bar for the scans."""
import numpy as np
import pytest
import torch

from conftest import close, close_rel, rand_cache, rand_qg

pytestmark = pytest.mark.gpu

SCALE = 256 ** -0.5
QS = 128 ** -0.5
ATOL, RTOL = 2e-3, 1e-2
ROW, NV = 10240, 48


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("seed", range(6))
def test_random_decode_batches(fl, dev, orc, seed):
    rng = np.random.default_rng(1000 + seed)
    for case in range(4):
        B = int(rng.integers(1, 11))
        T = int(rng.integers(1, 6))
        lens = [int(x) for x in rng.integers(T, 3001, size=B)]
        caps = [L + int(rng.integers(0, 41)) for L in lens]
        print(f"seed {seed} case {case}: B={B} T={T} lens={lens}", flush=True)
        caches = [rand_cache(rng, cap) for cap in caps]
        qg = np.stack([rand_qg(rng, T, q_scale=float(rng.choice([1 / 16, 0.5]))) for _ in range(B)])
        pos0s = [L - T for L in lens]
        z = fl.ops.attn_decode(to_dev(qg, dev), [to_dev(c[0], dev) for c in caches],
                               [to_dev(c[1], dev) for c in caches], pos0s)
        torch.cuda.synchronize()
        zh = z.cpu().numpy()
        for b in range(B):
            want = orc.attention_decode(qg[b], caches[b][0], caches[b][1], pos0s[b],
                                        max_pos=caps[b], scale=SCALE)
            err, ok = close_rel(zh[b], want, ATOL, RTOL)
            assert ok, f"seed {seed} case {case} sequence {b}: max|err| {err}"


@pytest.mark.parametrize("seed", range(3))
def test_random_decode_q8_batches(fl, dev, orc, seed):
    from test_gpu_q8 import oracle_cache

    rng = np.random.default_rng(2000 + seed)
    for case in range(3):
        B = int(rng.integers(1, 9))
        T = int(rng.integers(1, 6))
        lens = [int(x) for x in rng.integers(T, 3001, size=B)]
        caps = [L + int(rng.integers(0, 41)) for L in lens]
        print(f"seed {seed} case {case}: B={B} T={T} lens={lens}", flush=True)
        caches = [oracle_cache(orc, rng, L, cap) for L, cap in zip(lens, caps)]
        qg = np.stack([rand_qg(rng, T) for _ in range(B)])
        pos0s = [L - T for L in lens]
        kd, vd = [], []
        for (k, v, _, _), L, cap in zip(caches, lens, caps):
            a, b_ = fl.ops.kv8_cache(cap), fl.ops.kv8_cache(cap)
            fl.ops.kv_store_q8(to_dev(k, dev), to_dev(v, dev), a, b_, pos0=0, max_pos=cap)
            kd.append(a), vd.append(b_)
        z = fl.ops.attn_decode_q8(to_dev(qg, dev), kd, vd, pos0s, caps)
        torch.cuda.synchronize()
        zh = z.cpu().numpy()
        for b in range(B):
            want = orc.attention_decode_q8(qg[b], caches[b][2], caches[b][3], pos0s[b],
                                           max_pos=caps[b], scale=SCALE)
            err, ok = close_rel(zh[b], want, ATOL, RTOL)
            assert ok, f"seed {seed} case {case} sequence {b}: max|err| {err}"


@pytest.mark.parametrize("seed", range(4))
def test_random_prefill(fl, dev, orc, seed):
    rng = np.random.default_rng(3000 + seed)
    for case in range(4):
        T = int(rng.integers(1, 301))
        pos0 = int(rng.integers(0, 2001))
        cap = pos0 + T + int(rng.integers(0, 33))
        split = [None, 1, int(rng.integers(2, 10))][int(rng.integers(0, 3))]
        print(f"seed {seed} case {case}: T={T} pos0={pos0} cap={cap} split={split}", flush=True)
        k, v = rand_cache(rng, cap)
        qg = rand_qg(rng, T, q_scale=float(rng.choice([1 / 16, 0.5])))
        z = fl.ops.attention_prefill(to_dev(qg, dev), to_dev(k, dev), to_dev(v, dev), pos0=pos0,
                                     split=split)
        torch.cuda.synchronize()
        want = orc.attention_prefill(qg, k, v, q_pitch=512, pos0=pos0, max_pos=cap, scale=SCALE,
                                     T=T)
        err, ok = close_rel(z.cpu().numpy(), want, ATOL, RTOL)
        assert ok, f"seed {seed} case {case}: max|err| {err}"


@pytest.mark.parametrize("seed", range(2))
def test_random_prefill_q8(fl, dev, orc, seed):
    from test_gpu_q8 import oracle_cache

    rng = np.random.default_rng(4000 + seed)
    for case in range(3):
        T = int(rng.integers(1, 301))
        pos0 = int(rng.integers(0, 2001))
        cap = pos0 + T + int(rng.integers(0, 33))
        split = [None, 1, int(rng.integers(2, 10))][int(rng.integers(0, 3))]
        print(f"seed {seed} case {case}: T={T} pos0={pos0} cap={cap} split={split}", flush=True)
        k, v, kc8, vc8 = oracle_cache(orc, rng, pos0 + T, cap)
        qg = rand_qg(rng, T)
        kd, vd = fl.ops.kv8_cache(cap), fl.ops.kv8_cache(cap)
        fl.ops.kv_store_q8(to_dev(k, dev), to_dev(v, dev), kd, vd, pos0=0, max_pos=cap)
        z = fl.ops.attention_prefill_q8(to_dev(qg, dev), kd, vd, pos0=pos0, max_pos=cap,
                                        split=split)
        torch.cuda.synchronize()
        want = orc.attention_prefill_q8(qg, kc8, vc8, q_pitch=512, pos0=pos0, max_pos=cap,
                                        scale=SCALE, T=T)
        err, ok = close_rel(z.cpu().numpy(), want, ATOL, RTOL)
        assert ok, f"seed {seed} case {case}: max|err| {err}"


@pytest.mark.parametrize("seed", range(3))
def test_random_scans(fl, dev, orc, seed):
    rng = np.random.default_rng(5000 + seed)
    for case in range(3):
        T = int(rng.integers(1, 301))
        print(f"seed {seed} case {case}: T={T}", flush=True)
        c = rng.standard_normal((T, ROW)).astype(np.float16)
        ln = c.copy()
        qk = c[:, :4096].astype(np.float64).reshape(T, 32, 128)
        ln[:, :4096] = (qk / np.linalg.norm(qk, axis=-1, keepdims=True)).reshape(T, 4096)
        beta = (1 / (1 + np.exp(-rng.standard_normal((T, NV)) * 2))).astype(np.float32)
        decay = np.exp(-np.log1p(np.exp(rng.standard_normal((T, NV)) * 2))).astype(np.float32)
        S0 = (rng.standard_normal((NV, 128, 128)) * float(rng.choice([0.0, 0.02, 0.5]))).astype(
            np.float32)
        S_r = S0.copy()
        y_r = orc.gdn_scan(ln[:, :2048], ln[:, 2048:4096], ln[:, 4096:], beta, decay, S_r, T=T,
                           qk_stride=ROW, v_stride=ROW, out_scale=QS)
        lnd = to_dev(ln, dev)
        for form in ("recurrent", "chunked"):
            S = to_dev(S0, dev)
            if form == "recurrent":
                y = torch.empty((T, NV * 128), dtype=torch.float16, device=dev)
                fl.ops.gdn_scan(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:],
                                to_dev(beta, dev), to_dev(decay, dev), S, y, T=T)
            else:
                y = fl.ops.gdn_prefill_chunked(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:],
                                               to_dev(beta, dev), to_dev(decay, dev), S, T=T)
            torch.cuda.synchronize()
            Sh = S.cpu().numpy().astype(np.float64)
            rel = float(np.abs(Sh - S_r).max() / max(np.abs(S_r).max(), 1e-30))
            assert rel <= 1e-4, f"seed {seed} case {case} {form}: state rel {rel:.2e}"
            err, ok = close(y.cpu().numpy(), y_r, ATOL, RTOL)
            assert ok, f"seed {seed} case {case} {form}: max|dy| {err}"


@pytest.mark.parametrize("seed", range(3))
def test_random_gdn_decode(fl, dev, orc, seed):
    """The fused GDN decode over random batches: T = 1 with the conv fused
    (the plain decode step) or T = 2..3 verify rows after the conv rows, with
    checkpoints, at random positions and gates, each sequence against the
    oracle."""
    rng = np.random.default_rng(6000 + seed)
    for case in range(3):
        B = int(rng.integers(1, 13))
        T = int(rng.integers(1, 4))
        pos0s = [int(x) for x in rng.integers(0, 5000, size=B)]
        print(f"seed {seed} case {case}: B={B} T={T} pos0s={pos0s}", flush=True)
        w = (rng.standard_normal((ROW, 4)) * 0.5).astype(np.float16)
        A_log = (rng.standard_normal(NV) * 0.3).astype(np.float32)
        dt = (rng.standard_normal(NV) * 0.3).astype(np.float32)
        x = rng.standard_normal((B, T, ROW)).astype(np.float16)
        a = rng.standard_normal((B, T, NV)).astype(np.float32)
        bb = rng.standard_normal((B, T, NV)).astype(np.float32)
        S0 = (rng.standard_normal((B, NV, 128, 128)) * 0.02).astype(np.float32)
        st = rng.standard_normal((B, ROW, 3)).astype(np.float16)
        S_d = [to_dev(S0[b], dev) for b in range(B)]
        wd, Ad, dtd = to_dev(w, dev), to_dev(A_log, dev), to_dev(dt, dev)
        if T == 1:
            rin = [to_dev(st[b], dev) for b in range(B)]
            rout = [torch.empty((ROW, 3), dtype=torch.float16, device=dev) for _ in range(B)]
            y = fl.ops.gdn_decode(to_dev(x, dev), S_d, to_dev(a, dev), to_dev(bb, dev), Ad, dtd,
                                  T=1, pos0s=pos0s, conv_fused=True, conv_w=wd, cst_in=rin,
                                  cst_out=rout)
            cks = None
        else:
            c = torch.empty((B, T, ROW), dtype=torch.float16, device=dev)
            for b in range(B):
                sts = [torch.empty((ROW, 3), dtype=torch.float16, device=dev) for _ in range(3)]
                fl.ops.conv1d_causal_rows(to_dev(x[b], dev), wd, to_dev(st[b], dev), c[b],
                                          *sts[:T], T=T, pos0=pos0s[b])
            cks = [torch.zeros((T - 1, NV, 128, 128), dtype=torch.float32, device=dev)
                   for _ in range(B)]
            y = fl.ops.gdn_decode(c, S_d, to_dev(a, dev), to_dev(bb, dev), Ad, dtd, T=T,
                                  pos0s=pos0s, ck=cks, ck_step=NV * 128 * 128)
        torch.cuda.synchronize()
        yh = y.cpu().numpy()
        for b in range(B):
            S_r = S0[b].copy()
            if T == 1:
                ring = np.zeros((ROW, 3), np.float16)
                y_r = orc.gdn_decode(None, S_r, a[b], bb[b], A_log, dt, T=1, out_scale=QS,
                                     cx=x[b], cw=w, cst_in=st[b], cst_out=ring, pos0=pos0s[b])
                assert np.array_equal(rout[b].cpu().numpy(), ring), f"case {case} ring {b}"
            else:
                y_c, _ = orc.conv1d_causal_rows(x[b], w, st[b], dim=ROW, T=T, pos0=pos0s[b],
                                                row_stride=ROW)
                ck_r = np.zeros((T - 1, NV, 128, 128), np.float32)
                y_r = orc.gdn_decode(y_c, S_r, a[b], bb[b], A_log, dt, T=T, out_scale=QS,
                                     ck=ck_r, ck_step=NV * 128 * 128)
                ckh = cks[b].cpu().numpy().astype(np.float64)
                assert np.abs(ckh - ck_r).max() / np.abs(ck_r).max() <= 1e-4, f"case {case} ck {b}"
            Sh = S_d[b].cpu().numpy().astype(np.float64)
            assert np.abs(Sh - S_r).max() / np.abs(S_r).max() <= 1e-4, f"case {case} state {b}"
            err, ok = close(yh[b], y_r, ATOL, RTOL)
            assert ok, f"seed {seed} case {case} sequence {b}: max|dy| {err}"


def _ulps(a, b):
    ai = np.asarray(a).view(np.int16).astype(np.int32)
    bi = np.asarray(b).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return int(np.abs(ai - bi).max())


@pytest.mark.parametrize("seed", range(2))
def test_random_attn_prep(fl, dev, orc, seed):
    """The fused prep (norms, partial RoPE, KV store; fp16 and int8 caches) at
    random positions up to ~200k and 1..64 tokens: q and k within 1 fp16 ulp of
    the oracle, the cache rows (int8: values and scales) bit for bit, nothing
    written outside them."""
    rng = np.random.default_rng(7000 + seed)
    for case in range(4):
        T = int(rng.integers(1, 65))
        pos0 = int(rng.integers(0, 200000))
        cap = pos0 + T + int(rng.integers(0, 9))
        kv8 = bool(case & 1)
        print(f"seed {seed} case {case}: T={T} pos0={pos0} kv8={kv8}", flush=True)
        qg = rng.standard_normal((T, 24, 512)).astype(np.float16)
        k = (rng.standard_normal((T, 4, 256)) * 3).astype(np.float16)
        v = rng.standard_normal((T, 4, 256)).astype(np.float16)
        wq = (rng.standard_normal(256) * 0.2).astype(np.float32)
        wk = (rng.standard_normal(256) * 0.2).astype(np.float32)
        qd, kd, vd = to_dev(qg, dev), to_dev(k, dev), to_dev(v, dev)
        if kv8:
            kc, vc = orc.kv8_buffer(cap), orc.kv8_buffer(cap)
            q_o, k_o = orc.attn_prep_q8(qg, k, v, wq, wk, kc, vc, pos0=pos0, T=T, max_pos=cap)
            kcd, vcd = fl.ops.kv8_cache(cap), fl.ops.kv8_cache(cap)
            fl.ops.attn_prep_q8(qd, kd, vd, to_dev(wq, dev), to_dev(wk, dev), kcd, vcd,
                                pos0=pos0, max_pos=cap)
        else:
            kc = np.zeros((cap, 4, 256), np.float16)
            vc = np.zeros_like(kc)
            q_o, k_o = orc.attn_prep(qg, k, v, wq, wk, kc, vc, pos0=pos0, T=T, max_pos=cap)
            kcd = torch.zeros((cap, 4, 256), dtype=torch.float16, device=dev)
            vcd = torch.zeros_like(kcd)
            fl.ops.attn_prep(qd, kd, vd, to_dev(wq, dev), to_dev(wk, dev), kcd, vcd, pos0=pos0)
        torch.cuda.synchronize()
        assert _ulps(qd.cpu().numpy(), q_o) <= 1 and _ulps(kd.cpu().numpy(), k_o) <= 1, case
        assert np.array_equal(kcd.cpu().numpy(), kc) and np.array_equal(vcd.cpu().numpy(), vc), \
            f"seed {seed} case {case}: cache bytes"


@pytest.mark.parametrize("seed", range(2))
def test_random_conv(fl, dev, orc, seed):
    """conv1d_causal over random channel counts (multiples of 8 and not),
    widths 1..8, lengths and positions: y within 1 fp16 ulp of the oracle, the
    new state bit for bit."""
    rng = np.random.default_rng(8000 + seed)
    for case in range(4):
        dim = int(rng.choice([8, 64, 1000, 2048, 6144, 10240, 333]))
        width = int(rng.integers(1, 9))
        T = int(rng.integers(1, 70))
        pos0 = int(rng.integers(0, 50))
        stride = dim + int(rng.choice([0, 8, 16]))
        print(f"seed {seed} case {case}: dim={dim} width={width} T={T} pos0={pos0}", flush=True)
        x = rng.standard_normal((T, stride)).astype(np.float16)
        w = (rng.standard_normal((dim, width)) * 0.5).astype(np.float16)
        st = rng.standard_normal((dim, width - 1) if width > 1 else (8,)).astype(np.float16)
        y = torch.zeros((T, stride), dtype=torch.float16, device=dev)
        so = torch.empty(st.shape, dtype=torch.float16, device=dev)
        fl.ops.conv1d_causal(to_dev(x, dev), to_dev(w, dev), to_dev(st, dev), y, so, dim=dim,
                             T=T, pos0=pos0, row_stride=stride, width=width)
        torch.cuda.synchronize()
        y_r, so_r = orc.conv1d_causal(x, w, st, dim=dim, T=T, pos0=pos0, row_stride=stride,
                                      width=width)
        assert _ulps(y.cpu().numpy()[:, :dim], y_r[:, :dim]) <= 1, f"seed {seed} case {case}"
        if width > 1:
            assert np.array_equal(so.cpu().numpy(), so_r), f"seed {seed} case {case}: state"
