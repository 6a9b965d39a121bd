"""GPU parity of the full-attention path against the CPU oracle.

Bar: attention outputs within max-abs 2e-3 / rel 1e-2 of the reference math
in fp16; the KV store bit-exact. Size-independent properties at the
benchmark's full sizes: a verify row equals the T = 1 call at its position
bit for bit, a batched call equals per-sequence calls bit for bit, the split
count does not change the result beyond rounding.
"""
import numpy as np
import pytest
import torch

from conftest import close_rel, rand_cache, rand_qg

pytestmark = pytest.mark.gpu

SCALE = 256 ** -0.5
ATOL, RTOL = 2e-3, 1e-2


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_kv_store_bit_exact(fl, dev, rng):
    layers, max_pos, T, pos0, layer = 3, 300, 37, 200, 1
    kc = torch.zeros((layers, max_pos, 4, 256), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    k = rng.standard_normal((T, 4, 256)).astype(np.float16)
    v = rng.standard_normal((T, 4, 256)).astype(np.float16)
    fl.ops.kv_store(to_dev(k, dev), to_dev(v, dev), kc, vc, layer=layer, pos0=pos0)
    torch.cuda.synchronize()
    kh, vh = kc.cpu().numpy(), vc.cpu().numpy()
    assert np.array_equal(kh[layer, pos0:pos0 + T], k) and np.array_equal(vh[layer, pos0:pos0 + T], v)
    kh[layer, pos0:pos0 + T] = 0
    vh[layer, pos0:pos0 + T] = 0
    assert not kh.any() and not vh.any()
    with pytest.raises(ValueError):
        fl.ops.kv_store(to_dev(k, dev), to_dev(v, dev), kc, vc, layer=layer, pos0=max_pos - 3)


@pytest.mark.parametrize("L,T", [(1, 1), (2, 2), (31, 1), (32, 1), (33, 3), (100, 4),
                                 (1000, 3), (4096, 1), (5000, 2)])
def test_split_and_merge_vs_oracle(fl, dev, orc, rng, L, T):
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    pos0 = L - T
    split = 8
    kd, vd, qd = to_dev(kc, dev), to_dev(vc, dev), to_dev(qg, dev)
    pacc = torch.empty((T, 24, split, 256), dtype=torch.float32, device=dev)
    pm = torch.empty((T, 24, split), dtype=torch.float32, device=dev)
    pd = torch.empty_like(pm)
    z = torch.empty((T, 24, 256), dtype=torch.float16, device=dev)
    fl.ops.attention_split_gqa(qd, kd, vd, pacc, pm, pd, pos0=pos0, split_rows=64, T=T, split=split)
    fl.ops.attention_merge(pacc, pm, pd, z, T=T, split=split, gate=qd)
    torch.cuda.synchronize()
    want = orc.attention_decode(qg, kc, vc, pos0, max_pos=L, scale=SCALE)
    err, ok = close_rel(z.cpu().numpy(), want, ATOL, RTOL)
    assert ok, f"L={L} T={T}: max|err| {err}"


@pytest.mark.parametrize("Lmax,q_scale", [(8192, 1 / 16), (32768, 1 / 16), (102400, 1 / 16),
                                           (102400, 1.0)])
def test_config2_decode_verify_vs_oracle(fl, dev, orc, Lmax, q_scale):
    """Config 2: B=4, T=3 verify rows, lengths seeded-uniform in [0.9 Lmax, Lmax].
    Bar: max-abs 2e-3 / rel 1e-2 and max|err| <= 1e-2 max|want|; at ~100k the
    second rejects one lost split of 64 or one lost 32-row tile, which the first
    alone accepts (tests/test_parity_bar.py). q_scale 1 gives scores of std 1
    (peaked softmax) where config 2's q / 16 gives a nearly flat one."""
    rng = np.random.default_rng(Lmax + int(q_scale * 16))
    B, T = 4, 3
    lens = rng.integers(int(np.ceil(0.9 * Lmax)), Lmax + 1, size=B)
    caches = [rand_cache(rng, int(L)) for L in lens]
    qg = np.stack([rand_qg(rng, T, q_scale=q_scale) for _ in range(B)])
    pos0s = [int(L) - T for L in lens]
    z = fl.ops.attn_decode(to_dev(qg, dev), [to_dev(c[0], dev) for c in caches],
                           [to_dev(c[1], dev) for c in caches], pos0s)
    torch.cuda.synchronize()
    zh = z.cpu().numpy()
    for b in range(B):
        want = orc.attention_decode(qg[b], caches[b][0], caches[b][1], pos0s[b],
                                    max_pos=int(lens[b]), scale=SCALE)
        err, ok = close_rel(zh[b], want, ATOL, RTOL)
        print(f"Lmax={Lmax} q_scale={q_scale} seq {b}: max|err| {err:.2e} "
              f"max|want| {np.abs(want).max():.2e}")
        assert ok, f"Lmax={Lmax} seq {b} (L={lens[b]}): max|err| {err}"


@pytest.mark.parametrize("L", [40000, 2050, 8450])
def test_verify_rows_equal_t1_calls_bit_exact(fl, dev, rng, L):
    """Each row of a T = 4 verify equals the T = 1 call at its position, bit for
    bit -- also where the rows' split counts differ: lengths 2047..2050 cross
    the 64-row floor's 31 -> 32 splits, 8447..8450 the 256-row rule's 32 -> 33."""
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, 4)
    kd, vd = to_dev(kc, dev), to_dev(vc, dev)
    pos0 = L - 4
    zv = fl.ops.attn_decode(to_dev(qg[None], dev), [kd], [vd], [pos0])
    for t in range(4):
        z1 = fl.ops.attn_decode(to_dev(qg[None, t:t + 1], dev), [kd], [vd], [pos0 + t])
        assert torch.equal(zv[0, t], z1[0, 0]), t


def test_batched_equals_single_bit_exact(fl, dev, rng):
    """The length-only split rule (split_rows > 0): a batched call gives every
    sequence the bits of its own single call. The default grid rule sizes the
    split to the batch, so there a sequence's values may differ in the last
    bits from its single call's; both stay within the attention bar of the
    oracle and of each other."""
    lens = [3000, 17, 9000, 1]
    caches = [rand_cache(rng, L) for L in lens]
    qg = np.stack([rand_qg(rng, 1) for _ in lens])
    ks = [to_dev(c[0], dev) for c in caches]
    vs = [to_dev(c[1], dev) for c in caches]
    sr = fl.geometry.SPLIT_ROWS
    zb = fl.ops.attn_decode(to_dev(qg, dev), ks, vs, [L - 1 for L in lens], split_rows=sr)
    zg = fl.ops.attn_decode(to_dev(qg, dev), ks, vs, [L - 1 for L in lens])
    for b, L in enumerate(lens):
        z1 = fl.ops.attn_decode(to_dev(qg[b:b + 1], dev), [ks[b]], [vs[b]], [L - 1], split_rows=sr)
        assert torch.equal(zb[b], z1[0]), b
        g1 = fl.ops.attn_decode(to_dev(qg[b:b + 1], dev), [ks[b]], [vs[b]], [L - 1])
        for got in (zg[b], g1[0]):
            err, ok = close_rel(got.cpu().numpy(), z1[0].cpu().numpy().astype(np.float64), ATOL,
                                RTOL)
            assert ok, f"seq {b}: grid rule against the length rule {err}"


def test_split_count_independence(fl, dev, orc, rng):
    """4 splits and 300 splits of the same ~20k rows agree with each other and
    with the oracle, within the relative bar (a split lost or counted twice
    moves z by ~1/4 of its own size at 4 splits)."""
    L = 20000
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, 2)
    kd, vd, qd = to_dev(kc, dev), to_dev(vc, dev), to_dev(qg[None], dev)
    za = fl.ops.attn_decode(qd, [kd], [vd], [L - 2], split_rows=32, split=4)
    zb = fl.ops.attn_decode(qd, [kd], [vd], [L - 2], split_rows=64, split=300)
    err, ok = close_rel(za.cpu().numpy(), zb.cpu().numpy().astype(np.float64), 1e-3, 1e-2)
    assert ok, err
    want = orc.attention_decode(qg, kc, vc, L - 2, max_pos=L, scale=SCALE)
    for name, z in (("4 splits", za), ("300 splits", zb)):
        err, ok = close_rel(z[0].cpu().numpy(), want, ATOL, RTOL)
        assert ok, (name, err)


def test_gate_is_sigmoid(fl, dev, rng):
    L = 700
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, 1)
    kd, vd = to_dev(kc, dev), to_dev(vc, dev)
    z0 = fl.ops.attn_decode(to_dev(qg[None], dev), [kd], [vd], [L - 1], gate=False)
    qg[..., 256:] = 0.0
    zg = fl.ops.attn_decode(to_dev(qg[None], dev), [kd], [vd], [L - 1], gate=True)
    want = (z0.float() * 0.5).half()
    assert torch.equal(zg, want)


@pytest.mark.parametrize("T", [1, 37])
def test_attn_gate_layouts(fl, dev, rng, T):
    """fl_attn_gate over the runtime's layout (z pitch 256, the gate at 256 of
    a 512-wide q | gate row: 8 elements a lane) and over pitches that take the
    element-a-thread kernel (z pitch 260, gate pitch 516 at 258) gives the
    same bits, within fp16 rounding of f16(z * sigmoid(g)) in fp32, and
    leaves the rest of each row untouched."""
    z = (rng.standard_normal((T, 24, 256)) * 2).astype(np.float16)
    g = (rng.standard_normal((T, 24, 256)) * 4).astype(np.float16)
    g[0, 0, :4] = [0.0, 30.0, -30.0, 88.0]
    outs = []
    for zp, gp, goff in ((256, 512, 256), (260, 516, 258)):
        zb = np.full((T, 24, zp), 5.0, np.float16)
        zb[..., :256] = z
        gb = np.zeros((T, 24, gp), np.float16)
        gb[..., goff:goff + 256] = g
        zd = torch.from_numpy(zb).to(dev)
        fl.ops.attn_gate(zd, torch.from_numpy(gb).to(dev), z_pitch=zp, g_pitch=gp, g_off=goff,
                         T=T)
        torch.cuda.synchronize()
        zh = zd.cpu().numpy()
        assert (zh[..., 256:] == 5.0).all()
        outs.append(zh[..., :256])
    assert np.array_equal(outs[0].view(np.int16), outs[1].view(np.int16))
    want = (z.astype(np.float32) / (1 + np.exp(-g.astype(np.float32)))).astype(np.float16)
    err, ok = close_rel(outs[0], want.astype(np.float64), ATOL, RTOL)
    assert ok, err


def test_decode_rejects_bad_geometry(fl, dev, rng):
    kc, vc = rand_cache(rng, 64)
    kd, vd = to_dev(kc, dev), to_dev(vc, dev)
    qg = to_dev(rand_qg(rng, 6)[None], dev)       # 6 tokens x 6 heads = 36 > 32 columns
    with pytest.raises(ValueError):
        fl.ops.attn_decode(qg, [kd], [vd], [10])
    with pytest.raises(ValueError):                # pos0 + T beyond the cache
        fl.ops.attn_decode(to_dev(rand_qg(rng, 1)[None], dev), [kd], [vd], [64])


# --------------------------------------------------------------------------
# prefill
# --------------------------------------------------------------------------

@pytest.mark.parametrize("T,pos0", [(1, 0), (8, 0), (13, 0), (40, 3), (300, 0), (129, 1000),
                                    (1024, 1000), (2048, 0)])
def test_prefill_vs_oracle(fl, dev, orc, rng, T, pos0):
    L = pos0 + T
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    # the new rows arrive through the fused kv_store; older rows are already cached
    kd = torch.zeros((L, 4, 256), dtype=torch.float16, device=dev)
    vd = torch.zeros_like(kd)
    kd[:pos0] = to_dev(kc[:pos0], dev)
    vd[:pos0] = to_dev(vc[:pos0], dev)
    z = fl.ops.attention_prefill(to_dev(qg, dev), kd, vd, pos0=pos0,
                                 k_new=to_dev(kc[pos0:], dev), v_new=to_dev(vc[pos0:], dev))
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), kc) and np.array_equal(vd.cpu().numpy(), vc)
    want = orc.attention_prefill(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    err, ok = close_rel(z.cpu().numpy(), want, ATOL, RTOL)
    assert ok, f"T={T} pos0={pos0}: max|err| {err}"


@pytest.mark.parametrize("T,pos0", [(512, 0), (300, 200)])
def test_prefill_growing_scores(fl, dev, orc, rng, T, pos0):
    """Scores that climb along the sequence (a sawtooth of up to ~11 log2 units a
    64-row tile), so a column's running max keeps moving after its first tile and
    the O / l rescale path runs, against the oracle's running-max restatement."""
    L = pos0 + T
    kc, vc = rand_cache(rng, L)
    pos = np.arange(L)
    ramp = (0.12 * (pos % 384)).astype(np.float32)            # q.k * scale ~ ramp (natural units)
    kc = (kc.astype(np.float32) * 0.25 + ramp[:, None, None]).astype(np.float16)
    qg = rand_qg(rng, T)
    qg[..., :256] = (1 / 16 + 0.01 * rng.standard_normal((T, 24, 256))).astype(np.float16)
    kd = torch.from_numpy(kc).to(dev)
    vd = torch.from_numpy(vc).to(dev)
    z = fl.ops.attention_prefill(to_dev(qg, dev), kd, vd, pos0=pos0)
    torch.cuda.synchronize()
    want = orc.attention_prefill(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    err, ok = close_rel(z.cpu().numpy(), want, ATOL, RTOL)
    assert ok, f"T={T} pos0={pos0}: max|err| {err}"


def test_prefill_config3_scaling_full_rows_2k(fl, dev, orc):
    """Config 3's own scaling at 2k: q ~ N(0,1)/16 pre-scaled and scale 1 in
    the kernel (scores of std 1, a peaked softmax), every row of every head
    against the C oracle."""
    L = 2048
    rng = np.random.default_rng(2048)
    kc, vc = rand_cache(rng, L)
    q = (rng.standard_normal((L, 24, 256)) / 16).astype(np.float16)
    kd = torch.zeros((L, 4, 256), dtype=torch.float16, device=dev)
    vd = torch.zeros_like(kd)
    z = fl.ops.attention_prefill(to_dev(q, dev), kd, vd, pos0=0, scale=1.0,
                                 k_new=to_dev(kc, dev), v_new=to_dev(vc, dev))
    torch.cuda.synchronize()
    want = orc.attention_prefill(q, kc, vc, q_pitch=256, pos0=0, max_pos=L, scale=1.0, T=L)
    err, ok = close_rel(z.cpu().numpy(), want, ATOL, RTOL)
    assert ok, f"max|err| {err}"


@pytest.mark.parametrize("L", [8192, 32768])
def test_prefill_config3_full_rows(fl, dev, L):
    """Config 3 at full size, every row of every head: the kernel against
    oracle/torch_ref.attention_prefill (fp32 matmuls, P rounded to fp16 as
    the reference does; pinned to the C oracle by tests/test_oracle_torch.py)
    run on the GPU, so each of the XCD-mapped row tiles is checked."""
    from oracle import torch_ref as tr

    g = torch.Generator(device=dev).manual_seed(L)
    q = (torch.randn((L, 24, 256), generator=g, device=dev) / 16).half()
    k = torch.randn((L, 4, 256), generator=g, device=dev).half()
    v = torch.randn((L, 4, 256), generator=g, device=dev).half()
    kd = torch.zeros_like(k)
    vd = torch.zeros_like(v)
    z = fl.ops.attention_prefill(q, kd, vd, pos0=0, scale=1.0, k_new=k, v_new=v)
    torch.cuda.synchronize()
    assert torch.equal(kd, k) and torch.equal(vd, v)
    want = tr.attention_prefill(q, k, v, 0, 1.0, block=256)
    err = (z.float() - want.float()).abs()
    bound = ATOL + RTOL * want.float().abs()
    bad = int((err > bound).sum())
    print(f"config 3 L={L}: all {L * 24} rows, max|err| {float(err.max()):.2e}, "
          f"{bad} elements over the bar")
    assert torch.isfinite(z.float()).all()
    assert bad == 0, f"L={L}: max|err| {float(err.max())}"
    assert float(err.max()) <= 1e-2 * float(want.float().abs().max())


@pytest.mark.parametrize("L", [8192, 32768])
def test_prefill_config3_sampled_rows(fl, dev, orc, L):
    """Config 3 at full size: q pre-scaled by 1/16 (scale 1 in the kernel); sampled
    rows against the float64 closed form, every row finite."""
    rng = np.random.default_rng(L)
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, L)
    q = np.ascontiguousarray(qg[..., :256])
    kd = torch.zeros((L, 4, 256), dtype=torch.float16, device=dev)
    vd = torch.zeros_like(kd)
    z = fl.ops.attention_prefill(to_dev(q, dev), kd, vd, pos0=0, scale=1.0,
                                 k_new=to_dev(kc, dev), v_new=to_dev(vc, dev))
    torch.cuda.synchronize()
    zh = z.cpu().numpy()
    assert np.isfinite(zh.astype(np.float32)).all()
    for t in sorted({0, 1, 63, 64, 127, L // 2 + 5, L - 2, L - 1,
                     *rng.integers(0, L, 4).tolist()}):
        want = orc.attention_exact(q[t:t + 1], kc, vc, q_pitch=256, pos0=t, max_pos=L,
                                   scale=1.0, T=1)
        err, ok = close_rel(zh[t:t + 1], want, ATOL, RTOL)
        assert ok, f"L={L} row {t}: max|err| {err}"


@pytest.mark.parametrize("n_kv,G,T", [(8, 3, 300), (1, 24, 256), (1, 24, 300), (3, 8, 200),
                                       (8, 3, 5600), (2, 12, 5632), (2, 12, 5600)])
def test_prefill_kv_head_counts(fl, dev, orc, n_kv, G, T):
    """Other kv-head counts and GQA group sizes, on both prefill kernels and
    both workgroup orders (row tiles spread over the XCDs by kv head when the
    head count divides 8 and the tiles split evenly, the plain grid order
    otherwise): every row against the oracle for the short prompts, sampled
    rows against the float64 closed form for the long ones."""
    n_q = n_kv * G
    rng = np.random.default_rng(1000 * n_kv + T)
    kc = rng.standard_normal((T, n_kv, 256)).astype(np.float16)
    vc = rng.standard_normal((T, n_kv, 256)).astype(np.float16)
    q = (rng.standard_normal((T, n_q, 256)) / 16).astype(np.float16)
    kd = torch.zeros((T, n_kv, 256), dtype=torch.float16, device=dev)
    vd = torch.zeros_like(kd)
    z = fl.ops.attention_prefill(to_dev(q, dev), kd, vd, pos0=0, scale=1.0, n_q_heads=n_q,
                                 n_kv_heads=n_kv, k_new=to_dev(kc, dev), v_new=to_dev(vc, dev))
    torch.cuda.synchronize()
    zh = z.cpu().numpy()
    assert np.isfinite(zh.astype(np.float32)).all()
    if T <= 512:
        want = orc.attention_prefill(q, kc, vc, n_q_heads=n_q, n_kv_heads=n_kv, q_pitch=256,
                                     pos0=0, max_pos=T, scale=1.0, T=T)
        err, ok = close_rel(zh, want, ATOL, RTOL)
        assert ok, f"n_kv={n_kv} T={T}: max|err| {err}"
        return
    for t in sorted({0, 1, 85, 86, T // 2, T - 2, T - 1, *rng.integers(0, T, 4).tolist()}):
        want = orc.attention_exact(q[t:t + 1], kc, vc, n_q_heads=n_q, n_kv_heads=n_kv,
                                   q_pitch=256, pos0=t, max_pos=T, scale=1.0, T=1)
        err, ok = close_rel(zh[t:t + 1], want, ATOL, RTOL)
        assert ok, f"n_kv={n_kv} T={T} row {t}: max|err| {err}"


@pytest.mark.parametrize("T,pos0,ramp", [(6000, 0, False), (5800, 700, True), (4100, 0, False)])
def test_prefill_long_sampled_rows(fl, dev, orc, T, pos0, ramp):
    """Prompts long enough for the 64-rows-a-wave prefill kernel (at least 384
    workgroups of 256 (token, head) rows): a ragged last workgroup, pos0 > 0,
    and (ramp) scores that climb along the sequence so the lazy O / l rescale
    runs on later tiles; sampled rows against the float64 closed form."""
    L = pos0 + T
    rng = np.random.default_rng(T)
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    if ramp:
        pos = np.arange(L)
        kc = (kc.astype(np.float32) * 0.25 + (0.12 * (pos % 384))[:, None, None]).astype(np.float16)
        qg[..., :256] = (1 / 16 + 0.01 * rng.standard_normal((T, 24, 256))).astype(np.float16)
    kd = torch.from_numpy(kc).to(dev)
    vd = torch.from_numpy(vc).to(dev)
    z = fl.ops.attention_prefill(to_dev(qg, dev), kd, vd, pos0=pos0)
    torch.cuda.synchronize()
    zh = z.cpu().numpy()
    assert np.isfinite(zh.astype(np.float32)).all()
    for t in sorted({0, 1, 5, 42, 43, 255, 256, T // 2, T - 43, T - 2, T - 1,
                     *rng.integers(0, T, 5).tolist()}):
        want = orc.attention_exact(qg[t:t + 1], kc, vc, q_pitch=512, pos0=pos0 + t, max_pos=L,
                                   scale=SCALE, T=1)
        err, ok = close_rel(zh[t:t + 1], want, ATOL, RTOL)
        assert ok, f"T={T} pos0={pos0} row {t}: max|err| {err}"

# --------------------------------------------------------------------------
# prefill with a KV split (attention_prefill_fh's gridDim.z + attention_merge_fh)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("T,pos0,split", [(300, 500, 2), (300, 500, 3), (129, 1000, 7),
                                          (40, 3, 4), (1, 70, 5), (700, 0, 16)])
def test_prefill_kv_split_vs_oracle(fl, dev, orc, rng, T, pos0, split):
    """Forced KV splits (the 128-row kernel's) against the C oracle, every
    row: splits that leave some workgroups' shares empty (40 tokens from pos0
    3 are one or two 64-row tiles for 4 splits; 16 splits of a fresh
    700-token prompt), one query token, and the fused kv_store in front."""
    L = pos0 + T
    kc, vc = rand_cache(rng, L)
    qg = rand_qg(rng, T)
    kd = torch.zeros((L, 4, 256), dtype=torch.float16, device=dev)
    vd = torch.zeros_like(kd)
    kd[:pos0] = to_dev(kc[:pos0], dev)
    vd[:pos0] = to_dev(vc[:pos0], dev)
    z = fl.ops.attention_prefill(to_dev(qg, dev), kd, vd, pos0=pos0, split=split,
                                 k_new=to_dev(kc[pos0:], dev), v_new=to_dev(vc[pos0:], dev))
    torch.cuda.synchronize()
    assert np.array_equal(kd.cpu().numpy(), kc) and np.array_equal(vd.cpu().numpy(), vc)
    want = orc.attention_prefill(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    err, ok = close_rel(z.cpu().numpy(), want, ATOL, RTOL)
    assert ok, f"T={T} pos0={pos0} split={split}: max|err| {err}"


@pytest.mark.parametrize("T,pos0,split", [(683, 16000, 5), (700, 15700, 16)])
def test_prefill_r64_kv_split_vs_fp32(fl, dev, T, pos0, split):
    """The 64-rows-a-wave kernel's KV split (>= 64 workgroups of 256 rows and
    >= 16384 cache rows): 683 tokens leave 2 rows in the last row tile, 16
    splits of 16400 rows leave some shares of the first row tiles' ranges
    short. Every row against oracle/torch_ref.attention_prefill (fp32 on the
    GPU) and the unsplit call, the attention bar."""
    from oracle import torch_ref as tr

    L = pos0 + T
    g = torch.Generator(device=dev).manual_seed(T + split)
    q = (torch.randn((T, 24, 256), generator=g, device=dev) / 16).half()
    kd = torch.randn((L, 4, 256), generator=g, device=dev).half()
    vd = torch.randn((L, 4, 256), generator=g, device=dev).half()
    z = fl.ops.attention_prefill(q, kd, vd, pos0=pos0, scale=1.0, split=split)
    z1 = fl.ops.attention_prefill(q, kd, vd, pos0=pos0, scale=1.0, split=1)
    want = tr.attention_prefill(q, kd, vd, pos0, 1.0, block=256)
    torch.cuda.synchronize()
    for name, got in ((f"split {split}", z), ("split 1", z1)):
        err = (got.float() - want.float()).abs()
        bad = int((err > ATOL + RTOL * want.float().abs()).sum())
        assert torch.isfinite(got.float()).all() and bad == 0, (name, float(err.max()))
        assert float(err.max()) <= 1e-2 * float(want.float().abs().max()), name


def test_prefill_kv_split_chunk_deep_in_prompt(fl, dev):
    """The reference's own prefill shape: a 1024-token chunk (MAX_CHUNK,
    runtime.py:196) at pos0 = 98000, where the 256-row workgroups (96) are
    fewer than the CUs and the policy splits the KV range 8 ways (768
    workgroups of the 64-rows-a-wave kernel). Every row against
    oracle/torch_ref.attention_prefill (fp32 on the GPU), and the unsplit call
    (the 128-row kernel) within the same bar."""
    from oracle import torch_ref as tr

    T, pos0 = 1024, 98000
    assert fl.ops.prefill_split_count(T, pos0) == 8
    L = pos0 + T
    g = torch.Generator(device=dev).manual_seed(98)
    q = (torch.randn((T, 24, 256), generator=g, device=dev) / 16).half()
    kd = torch.randn((L, 4, 256), generator=g, device=dev).half()
    vd = torch.randn((L, 4, 256), generator=g, device=dev).half()
    z = fl.ops.attention_prefill(q, kd, vd, pos0=pos0, scale=1.0)
    z1 = fl.ops.attention_prefill(q, kd, vd, pos0=pos0, scale=1.0, split=1)
    want = tr.attention_prefill(q, kd, vd, pos0, 1.0, block=256)
    torch.cuda.synchronize()
    scale_out = float(want.float().abs().max())
    for name, got in (("split 8", z), ("split 1", z1)):
        err = (got.float() - want.float()).abs()
        bad = int((err > ATOL + RTOL * want.float().abs()).sum())
        print(f"T={T} pos0={pos0} {name}: max|err| {float(err.max()):.2e} "
              f"(max|z| {scale_out:.2e}), {bad} over the bar")
        assert torch.isfinite(got.float()).all() and bad == 0, name
        # outputs average ~99k values (|z| ~ 1e-2), so the absolute bar alone
        # is loose: a tile range lost or counted twice moves z by ~1/4 of itself
        assert float(err.max()) <= 1e-2 * scale_out, name


@pytest.mark.parametrize("kind", ["decode", "decode_q8", "prefill", "prefill_split"])
def test_peaked_scores_vs_oracle(fl, dev, orc, rng, kind):
    """Scores of std ~30 (q ~ N(0,1) x 2 at scale 1/16): every row's softmax is
    dominated by a few keys, its running max moves by far more than the lazy
    rescale's 2^8 threshold several times, and P spans the whole fp16 range.
    Decode / verify (fp16 and int8 caches) and the causal prefill, unsplit and
    KV-split, against the oracle, to the attention bar and 1e-2 max|want|."""
    from test_gpu_q8 import oracle_cache

    L, T = 2000, 3 if kind.startswith("decode") else 200
    pos0 = L - T
    if kind == "decode_q8":
        k, v, kc8, vc8 = oracle_cache(orc, rng, L, L)
    else:
        k, v = rand_cache(rng, L)
    qg = rand_qg(rng, T, q_scale=2.0)
    if kind == "decode":
        z = fl.ops.attn_decode(to_dev(qg[None], dev), [to_dev(k, dev)], [to_dev(v, dev)],
                               [pos0])[0]
        want = orc.attention_decode(qg, k, v, pos0, max_pos=L, scale=SCALE)
    elif kind == "decode_q8":
        kd, vd = fl.ops.kv8_cache(L), fl.ops.kv8_cache(L)
        fl.ops.kv_store_q8(to_dev(k, dev), to_dev(v, dev), kd, vd, pos0=0, max_pos=L)
        z = fl.ops.attn_decode_q8(to_dev(qg[None], dev), [kd], [vd], [pos0], [L])[0]
        want = orc.attention_decode_q8(qg, kc8, vc8, pos0, max_pos=L, scale=SCALE)
    else:
        split = 4 if kind == "prefill_split" else 1
        z = fl.ops.attention_prefill(to_dev(qg, dev), to_dev(k, dev), to_dev(v, dev),
                                     pos0=pos0, split=split)
        want = orc.attention_prefill(qg, k, v, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE,
                                     T=T)
    torch.cuda.synchronize()
    zh = z.cpu().numpy()
    assert np.isfinite(zh.astype(np.float32)).all()
    err, ok = close_rel(zh, want, ATOL, RTOL)
    assert ok, f"{kind}: max|err| {err}"


@pytest.mark.parametrize("T,pos0,split", [(200, 700, 3), (64, 100, 6)])
def test_prefill_q8_kv_split_vs_oracle(fl, dev, orc, rng, T, pos0, split):
    """The KV split over the int8 cache (attention_prefill_fh_q8 with
    gridDim.z > 1) against the C oracle's int8 prefill, every row."""
    from test_gpu_q8 import oracle_cache

    L = pos0 + T
    k, v, kc8, vc8 = oracle_cache(orc, rng, L, L)
    qg = rand_qg(rng, T)
    kd, vd = fl.ops.kv8_cache(L), fl.ops.kv8_cache(L)
    fl.ops.kv_store_q8(to_dev(k, dev), to_dev(v, dev), kd, vd, pos0=0, max_pos=L)
    z = fl.ops.attention_prefill_q8(to_dev(qg, dev), kd, vd, pos0=pos0, max_pos=L, split=split)
    torch.cuda.synchronize()
    want = orc.attention_prefill_q8(qg, kc8, vc8, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE,
                                    T=T)
    err, ok = close_rel(z.cpu().numpy(), want, ATOL, RTOL)
    assert ok, f"T={T} pos0={pos0} split={split}: max|err| {err}"


@pytest.mark.parametrize("head_dim,z_pitch,split,T", [(256, 256, 4, 300), (128, 128, 13, 7),
                                                      (64, 72, 9, 5), (256, 258, 8, 3)])
def test_merge_layouts_vs_oracle(fl, dev, orc, rng, head_dim, z_pitch, split, T):
    """fl_attention_merge on random partials (empty ones among them) against
    the oracle's merge: the wavefront-a-row kernel for head_dim <= 256 and a
    pitch of 4 halves (head_dim 128 and 64 leave lanes without dims; 9 and 13
    splits a partial batch of 8), the block-a-row kernel for an odd pitch
    (258). Bar: the attention bar and 1e-2 max|want|."""
    H = 24
    pacc = rng.standard_normal((T, H, split, head_dim)).astype(np.float32)
    pm = (rng.standard_normal((T, H, split)) * 3).astype(np.float32)
    pd = rng.uniform(0.5, 4.0, (T, H, split)).astype(np.float32)
    pm[:, :, 1::3] = -1e30                       # empty partials: m = -1e30, d = 0, acc = 0
    pd[:, :, 1::3] = 0
    pacc[:, :, 1::3] = 0
    want = orc.attention_merge(pacc, pm, pd, H, head_dim, T, split, z_pitch=z_pitch)
    z = torch.zeros((T, H, z_pitch), dtype=torch.float16, device=dev)
    fl.ops.attention_merge(to_dev(pacc, dev), to_dev(pm, dev), to_dev(pd, dev), z,
                           head_dim=head_dim, z_pitch=z_pitch, T=T, split=split)
    torch.cuda.synchronize()
    got = z.cpu().numpy()
    err, ok = close_rel(got[..., :head_dim], want[..., :head_dim], ATOL, RTOL)
    assert ok and err <= 1e-2 * float(np.abs(want[..., :head_dim].astype(np.float32)).max()), err
    assert not got[..., head_dim:].any(), "wrote past head_dim"


# the KV-split prefills' merge carries the gate; the unsplit ones run the gate
# after them: split 3 of the 128-row kernel, the 64-rows-a-wave kernel's own
# split (683 tokens at 16000), the unsplit 128-row and long-prompt kernels,
# and over an int8 cache its split, an unsplit call and a staged long prompt
@pytest.mark.parametrize("kv8,T,pos0,split,splits", [
    (False, 300, 500, 3, True), (False, 683, 16000, None, True), (False, 300, 500, 1, False),
    (False, 4096, 0, None, False), (True, 300, 500, 3, True), (True, 1024, 8000, None, True),
    (True, 300, 500, 1, False), (True, 4096, 512, None, False)])
def test_prefill_gated_equals_prefill_then_gate(fl, dev, kv8, T, pos0, split, splits):
    """fl_attention_prefill_gated (the layer's attention output: the gate half
    of each head's q | gate row applied in the KV-split merge, or by
    attn_gate after an unsplit prefill) against the prefill then attn_gate,
    bit for bit."""
    L = pos0 + T
    if split is None:
        count = (fl.ops.prefill_split_count_q8 if kv8 else fl.ops.prefill_split_count)(T, pos0)
        assert (count > 1) == splits, count
    g = torch.Generator(device=dev).manual_seed(T + pos0)
    qg = torch.randn((T, 24, 512), generator=g, device=dev)
    qg[..., :256] /= 16
    qg = qg.half()
    k = torch.randn((L, 4, 256), generator=g, device=dev).half()
    v = torch.randn((L, 4, 256), generator=g, device=dev).half()
    if kv8:
        kd, vd = fl.ops.kv8_cache(L), fl.ops.kv8_cache(L)
        fl.ops.kv_store_q8(k, v, kd, vd, pos0=0, max_pos=L)

        def run(gated):
            return fl.ops.attention_prefill_q8(qg, kd, vd, pos0=pos0, max_pos=L, split=split,
                                               gated=gated)
    else:
        def run(gated):
            return fl.ops.attention_prefill(qg, k, v, pos0=pos0, split=split, gated=gated)
    zg = run(True)
    z = run(False)
    fl.ops.attn_gate(z, qg, T=T)
    torch.cuda.synchronize()
    assert torch.isfinite(zg.float()).all()
    assert torch.equal(zg, z), f"kv8={kv8} T={T} pos0={pos0} split={split}"
