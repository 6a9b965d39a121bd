"""Attention prep on the GPU through the C ABI against the oracle: rmsnorm1p,
rope_partial and the fused attn_prep (q / k norms + partial RoPE + KV store).
Both sides round products and sums separately and use correctly rounded sqrt /
divide and fp64 sincos, so the fp16 outputs are expected bit for bit; the bar
written here is <= 1 fp16 ulp (a last-bit fp64 pow / sincos difference between
the device's and libm's may move one), with the count of differing values
printed. The KV cache rows must equal the kernel's own roped k / v bit for bit,
and the fused launch must equal the unfused sequence bit for bit."""
import numpy as np
import pytest
import torch

from conftest import f16

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def ulp16(a, b):
    ia = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    ib = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    d = np.abs(ia - ib)
    return int(d.max()), int((d > 0).sum())


@pytest.mark.parametrize("T", [1, 3, 257])
def test_rmsnorm1p_vs_oracle(fl, dev, orc, rng, T):
    x = f16(rng.standard_normal((T, 24, 512)) * rng.uniform(0.01, 10))
    w = (rng.standard_normal(256) * 0.3).astype(np.float32)
    want = orc.rmsnorm1p(x, w, rows=24, pitch=512, T=T)
    xd = to_dev(x, dev)
    yd = torch.zeros_like(xd)
    fl.ops.rmsnorm1p(xd, to_dev(w, dev), yd, rows=24, pitch=512)   # out of place
    fl.ops.rmsnorm1p(xd, to_dev(w, dev), rows=24, pitch=512)       # in place
    torch.cuda.synchronize()
    got, got_ip = yd.cpu().numpy(), xd.cpu().numpy()
    m, n = ulp16(got[..., :256], want[..., :256])
    print(f"rmsnorm1p T={T}: max {m} ulp, {n} values differ")
    assert m <= 1
    assert np.array_equal(got_ip[..., :256], got[..., :256])
    assert np.array_equal(got_ip[..., 256:], x[..., 256:])         # gate half untouched
    assert not got[..., 256:].any()                                 # out of place writes 256 only


@pytest.mark.parametrize("T,pos0", [(1, 0), (3, 4097), (64, 100_000)])
def test_rope_partial_vs_oracle(fl, dev, orc, rng, T, pos0):
    q = f16(rng.standard_normal((T, 24, 512)))
    k = f16(rng.standard_normal((T, 4, 256)))
    wq, wk = orc.rope_partial(q, k, n_q_heads=24, n_kv_heads=4, q_pitch=512, k_pitch=256,
                              pos0=pos0, T=T)
    qd, kd = to_dev(q, dev), to_dev(k, dev)
    fl.ops.rope_partial(qd, kd, pos0=pos0)
    torch.cuda.synchronize()
    gq, gk = qd.cpu().numpy(), kd.cpu().numpy()
    mq, nq = ulp16(gq, wq)
    mk, nk = ulp16(gk, wk)
    print(f"rope_partial T={T} pos0={pos0}: q max {mq} ulp ({nq} differ), k max {mk} ({nk})")
    assert mq <= 1 and mk <= 1
    assert np.array_equal(gq[..., 64:], q[..., 64:]) and np.array_equal(gk[..., 64:], k[..., 64:])


@pytest.mark.parametrize("T,pos0", [(1, 4095), (3, 100), (2048, 0)])
def test_attn_prep_vs_oracle_and_unfused(fl, dev, orc, rng, T, pos0):
    max_pos = pos0 + T + 5
    qg = f16(rng.standard_normal((T, 24, 512)))
    k = f16(rng.standard_normal((T, 4, 256)) * 3)
    v = f16(rng.standard_normal((T, 4, 256)))
    wq = (rng.standard_normal(256) * 0.2).astype(np.float32)
    wk = (rng.standard_normal(256) * 0.2).astype(np.float32)
    kc = np.zeros((max_pos, 4, 256), np.float16)
    vc = np.zeros_like(kc)
    wq_o, wk_o = orc.attn_prep(qg, k, v, wq, wk, kc, vc, pos0=pos0, T=T, max_pos=max_pos)
    # fused
    qd, kd, vd = to_dev(qg, dev), to_dev(k, dev), to_dev(v, dev)
    kcd = torch.zeros((max_pos, 4, 256), dtype=torch.float16, device=dev)
    vcd = torch.zeros_like(kcd)
    wqd, wkd = to_dev(wq, dev), to_dev(wk, dev)
    fl.ops.attn_prep(qd, kd, vd, wqd, wkd, kcd, vcd, pos0=pos0)
    # unfused: rmsnorm1p x2, rope_partial, kv_store
    qu, ku = to_dev(qg, dev), to_dev(k, dev)
    kcu = torch.zeros_like(kcd)
    vcu = torch.zeros_like(kcd)
    fl.ops.rmsnorm1p(qu, wqd, rows=24, pitch=512)
    fl.ops.rmsnorm1p(ku, wkd, rows=4, pitch=256)
    fl.ops.rope_partial(qu, ku, pos0=pos0)
    fl.ops.kv_store(ku, vd, kcu, vcu, pos0=pos0)
    torch.cuda.synchronize()
    gq, gk, gkc, gvc = (t.cpu().numpy() for t in (qd, kd, kcd, vcd))
    assert np.array_equal(gq, qu.cpu().numpy()) and np.array_equal(gk, ku.cpu().numpy())
    assert np.array_equal(gkc, kcu.cpu().numpy()) and np.array_equal(gvc, vcu.cpu().numpy())
    mq, nq = ulp16(gq, wq_o)
    mk, nk = ulp16(gk, wk_o)
    print(f"attn_prep T={T} pos0={pos0}: q max {mq} ulp ({nq} differ), k max {mk} ({nk})")
    assert mq <= 1 and mk <= 1
    assert np.array_equal(gkc[pos0:pos0 + T], gk) and np.array_equal(gvc[pos0:pos0 + T], v)
    assert not gkc[:pos0].any() and not gkc[pos0 + T:].any()


def test_attn_prep_bad_geometry(fl, dev):
    q = torch.zeros((2, 24, 512), dtype=torch.float16, device=dev)
    k = torch.zeros((2, 4, 256), dtype=torch.float16, device=dev)
    w = torch.zeros(256, dtype=torch.float32, device=dev)
    kc = torch.zeros((4, 4, 256), dtype=torch.float16, device=dev)
    with pytest.raises(ValueError):       # pos0 + T beyond the cache
        fl.ops.attn_prep(q, k, k, w, w, kc, kc, pos0=3)
    with pytest.raises(ValueError):       # odd rotary width
        fl.ops.rope_partial(q, k, pos0=0, rope_dim=63)


@pytest.mark.parametrize("kv8", [False, True])
def test_attn_prep_rows_equals_a_prep_a_row(fl, dev, rng, kv8):
    """fl_attn_prep_rows (a batched decode step's rows, one launch) against
    one attn_prep (attn_prep_q8) call a row, bit for bit: q and k rewritten
    in place and each row's K / V stored in its own cache at its own
    position -- caches of different capacities, positions from 0 to deep in
    a prompt, five rows -- and nothing else of the caches touched."""
    caps = [64, 4096, 100000, 32, 2048]
    pos = [0, 4095, 99999, 17, 1000]
    B = len(caps)
    qg = f16(rng.standard_normal((B, 24, 512)))
    k = f16(rng.standard_normal((B, 4, 256)) * 2)
    v = f16(rng.standard_normal((B, 4, 256)))
    wq = to_dev((rng.standard_normal(256) * 0.2).astype(np.float32), dev)
    wk = to_dev((rng.standard_normal(256) * 0.2).astype(np.float32), dev)

    def caches():
        if kv8:
            return [fl.ops.kv8_cache(c) for c in caps], [fl.ops.kv8_cache(c) for c in caps]
        return ([torch.full((c, 4, 256), 3.0, dtype=torch.float16, device=dev) for c in caps],
                [torch.full((c, 4, 256), -2.0, dtype=torch.float16, device=dev) for c in caps])

    kb, vb = caches()
    qd, kd, vd = to_dev(qg, dev), to_dev(k, dev), to_dev(v, dev)
    fl.ops.attn_prep_rows(qd, kd, vd, wq, wk, kb, vb, pos, caps, kv8=kv8)
    ks, vs = caches()
    q1, k1 = to_dev(qg, dev), to_dev(k, dev)
    for b in range(B):
        if kv8:
            fl.ops.attn_prep_q8(q1[b:b + 1], k1[b:b + 1], vd[b:b + 1], wq, wk, ks[b], vs[b],
                                pos0=pos[b], max_pos=caps[b], T=1)
        else:
            fl.ops.attn_prep(q1[b:b + 1], k1[b:b + 1], vd[b:b + 1], wq, wk, ks[b], vs[b],
                             pos0=pos[b], T=1)
    torch.cuda.synchronize()
    assert torch.equal(qd, q1) and torch.equal(kd, k1)
    for b in range(B):
        assert torch.equal(kb[b], ks[b]) and torch.equal(vb[b], vs[b]), b
    with pytest.raises(ValueError):                       # a position past its capacity
        fl.ops.attn_prep_rows(qd, kd, vd, wq, wk, kb, vb, [0, 4096, 0, 0, 0], caps, kv8=kv8)
