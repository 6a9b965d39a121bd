"""GPU parity of the Gated DeltaNet path against the CPU oracle.

Bar: GDN recurrent state within rel 1e-4 (fp32) after 1024
decode steps (config 1); outputs y within max-abs 2e-3 / rel 1e-2 (fp16);
conv states bit-exact (they are fp16 copies of inputs). The chunked WY scan
(config 4) against the step-by-step recurrence.
"""
import numpy as np
import pytest
import torch

from conftest import close

pytestmark = pytest.mark.gpu

QS = 128 ** -0.5
ROW = 10240
NV, NK = 48, 16
STATE_RTOL = 1e-4


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rel_err(got, want):
    return float(np.abs(np.asarray(got, np.float64) - want).max() / np.abs(want).max())


def ulp16_diff(a, b):
    ai = a.view(np.int16).astype(np.int32)
    bi = b.view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return int(np.abs(ai - bi).max())


def _conv_case(fl, dev, orc, rng, *, T, pos0, dim=ROW, stride=None, width=4):
    """One conv call on the GPU and in the oracle: (y, st_out) of each."""
    stride = dim if stride is None else stride
    x = rng.standard_normal((T, stride)).astype(np.float16)
    w = (rng.standard_normal((dim, width)) * 0.5).astype(np.float16)
    # width 1 keeps no history: one-element placeholders stand in for the state
    st = rng.standard_normal((dim, width - 1) if width > 1 else (8,)).astype(np.float16)
    y = torch.zeros((T, stride), dtype=torch.float16, device=dev)
    so = torch.empty(st.shape, dtype=torch.float16, device=dev)
    fl.ops.conv1d_causal(to_dev(x, dev), to_dev(w, dev), to_dev(st, dev), y, so, dim=dim, T=T,
                         pos0=pos0, row_stride=stride, width=width)
    torch.cuda.synchronize()
    y_r, so_r = orc.conv1d_causal(x, w, st, dim=dim, T=T, pos0=pos0, row_stride=stride,
                                  width=width)
    if width == 1:
        so, so_r = np.zeros(0, np.float16), np.zeros(0, np.float16)
    else:
        so = so.cpu().numpy()
    return y.cpu().numpy()[:, :dim], so, y_r[:, :dim], so_r


# token counts around the 4-token block a lane walks at width 4: 1, 2
# (shorter than the 3 frames of history: the new state mixes old frames and
# new ones), a block and one past it, many blocks with a ragged last one, and
# long calls (1700, 4000: a thousand blocks down each lane's channels).
@pytest.mark.parametrize("T,pos0", [(1, 0), (1, 9), (2, 5), (5, 0), (8, 3), (16, 1), (17, 2),
                                    (64, 100), (333, 7), (1700, 4), (4000, 9)])
def test_conv1d_vs_oracle(fl, dev, orc, rng, T, pos0):
    y, so, y_r, so_r = _conv_case(fl, dev, orc, rng, T=T, pos0=pos0)
    assert np.array_equal(so, so_r)
    assert ulp16_diff(y, y_r) <= 1


# both lane layouts (8 channels a lane with 16-byte rows; a channel a lane for
# an odd row stride / channel count) and every supported width
@pytest.mark.parametrize("width", [1, 2, 3, 5, 6, 8])
@pytest.mark.parametrize("layout", ["vec", "lane"])
@pytest.mark.parametrize("T,pos0", [(2, 3), (21, 0)])
def test_conv1d_widths_and_layouts(fl, dev, orc, rng, width, layout, T, pos0):
    dim, stride = (1024, 1032) if layout == "vec" else (1001, 1003)
    y, so, y_r, so_r = _conv_case(fl, dev, orc, rng, T=T, pos0=pos0, dim=dim, stride=stride,
                                  width=width)
    assert np.array_equal(so, so_r)
    assert ulp16_diff(y, y_r) <= 1


def test_conv1d_segment_view_and_chunk_invariance(fl, dev, orc, rng):
    """The v segment of a q|k|v row (a view 4096 channels in, row stride
    10240), and the reference's chunk invariance (kernels.cu:135-138): 7
    tokens then 13 from the state the first call left equal the 20-token call,
    y and the state bit for bit."""
    T = 20
    x = rng.standard_normal((T, ROW)).astype(np.float16)
    w = (rng.standard_normal((6144, 4)) * 0.5).astype(np.float16)
    st = rng.standard_normal((6144, 3)).astype(np.float16)
    xd, wd, sd = to_dev(x, dev), to_dev(w, dev), to_dev(st, dev)
    y = torch.zeros((T, ROW), dtype=torch.float16, device=dev)
    so = torch.empty((6144, 3), dtype=torch.float16, device=dev)
    fl.ops.conv1d_causal(xd[:, 4096:], wd, sd, y[:, 4096:], so, dim=6144, T=T, pos0=5)
    y2 = torch.zeros_like(y)
    mid = torch.empty_like(so)
    so2 = torch.empty_like(so)
    fl.ops.conv1d_causal(xd[:7, 4096:], wd, sd, y2[:7, 4096:], mid, dim=6144, T=7, pos0=5)
    fl.ops.conv1d_causal(xd[7:, 4096:], wd, mid, y2[7:, 4096:], so2, dim=6144, T=13, pos0=12)
    torch.cuda.synchronize()
    assert torch.equal(y, y2) and torch.equal(so, so2)
    assert (y[:, :4096] == 0).all(), "wrote outside the segment"
    y_r, so_r = orc.conv1d_causal(x[:, 4096:].copy(), w, st, dim=6144, T=T, pos0=5,
                                  row_stride=6144)
    assert np.array_equal(so.cpu().numpy(), so_r)
    assert ulp16_diff(y.cpu().numpy()[:, 4096:], y_r) <= 1


@pytest.mark.parametrize("T,pos0,layout", [(1, 4, "vec"), (2, 4, "vec"), (3, 4, "vec"),
                                           (3, 0, "vec"), (3, 4, "lane")])
def test_conv_rows_vs_oracle(fl, dev, orc, rng, T, pos0, layout):
    dim, stride = (ROW, ROW) if layout == "vec" else (1001, 1003)
    x = rng.standard_normal((T, stride)).astype(np.float16)
    w = (rng.standard_normal((dim, 4)) * 0.5).astype(np.float16)
    st = rng.standard_normal((dim, 3)).astype(np.float16)
    y = torch.zeros((T, stride), dtype=torch.float16, device=dev)
    sts = [torch.empty((dim, 3), dtype=torch.float16, device=dev) for _ in range(3)]
    fl.ops.conv1d_causal_rows(to_dev(x, dev), to_dev(w, dev), to_dev(st, dev), y, *sts[:T], T=T,
                              pos0=pos0, dim=dim, row_stride=stride)
    torch.cuda.synchronize()
    y_r, sts_r = orc.conv1d_causal_rows(x, w, st, dim=dim, T=T, pos0=pos0, row_stride=stride)
    assert ulp16_diff(y.cpu().numpy()[:, :dim], y_r[:, :dim]) <= 1
    for t in range(T):
        assert np.array_equal(sts[t].cpu().numpy(), sts_r[t])


def test_conv_rows_state_in_place(fl, dev, orc, rng):
    """Row 0's state may be written over st_in (kernels.cu:1681-1685): every
    lane reads its channels' frames before it writes them."""
    T = 3
    x = rng.standard_normal((T, ROW)).astype(np.float16)
    w = (rng.standard_normal((ROW, 4)) * 0.5).astype(np.float16)
    st = rng.standard_normal((ROW, 3)).astype(np.float16)
    y = torch.empty((T, ROW), dtype=torch.float16, device=dev)
    s0 = to_dev(st, dev)
    s1 = torch.empty_like(s0)
    s2 = torch.empty_like(s0)
    fl.ops.conv1d_causal_rows(to_dev(x, dev), to_dev(w, dev), s0, y, s0, s1, s2, T=T, pos0=9)
    torch.cuda.synchronize()
    y_r, sts_r = orc.conv1d_causal_rows(x, w, st, dim=ROW, T=T, pos0=9, row_stride=ROW)
    assert ulp16_diff(y.cpu().numpy(), y_r) <= 1
    for got, want in zip((s0, s1, s2), sts_r):
        assert np.array_equal(got.cpu().numpy(), want)


def test_l2norm_and_gates_vs_oracle(fl, dev, orc, rng):
    T = 5
    x = rng.standard_normal((T, ROW)).astype(np.float16)
    x[2, 128:256] = 0
    y = torch.zeros((T, ROW), dtype=torch.float16, device=dev)
    fl.ops.l2norm_scaled(to_dev(x, dev), y, rows=80, T=T)
    a = (rng.standard_normal((T, NV)) * 5).astype(np.float32)
    a[0, :4] = [100.0, -40.0, 20.0, 20.0001]
    b = rng.standard_normal((T, NV)).astype(np.float32)
    A_log = rng.standard_normal(NV).astype(np.float32)
    dt = rng.standard_normal(NV).astype(np.float32)
    beta = torch.empty((T, NV), dtype=torch.float32, device=dev)
    decay = torch.empty_like(beta)
    fl.ops.gdn_scalars(to_dev(a, dev), to_dev(b, dev), to_dev(A_log, dev), to_dev(dt, dev),
                       beta, decay, T=T)
    torch.cuda.synchronize()
    y_r = orc.l2norm_scaled(x, n=128, rows=80, pitch=128, eps=1e-6, scale=1.0, T=T)
    assert ulp16_diff(y.cpu().numpy(), y_r) <= 1
    b_r, d_r = orc.gdn_scalars(a, b, A_log, dt, T=T, n_heads=NV)
    assert np.abs(beta.cpu().numpy() - b_r).max() <= 2e-7
    assert np.abs(decay.cpu().numpy() - d_r).max() / d_r.max() <= 2e-6


@pytest.mark.parametrize("T", [1, 37, 300])
def test_l2norm_strided_equals_full_rows(fl, dev, rng, T):
    """fl_l2norm_scaled_strided over the q and k rows (32 of a token's 80
    head-sized rows, the GDN prefill's use) gives the bits fl_l2norm_scaled
    gives them over all 80, and leaves the other 48 rows untouched; 37 x 32
    rows leave the last wave ragged."""
    x = torch.from_numpy((rng.standard_normal((T, 80, 128)) * 0.8).astype(np.float16)).to(dev)
    full = torch.empty_like(x)
    fl.ops.l2norm_scaled(x, full, rows=80, T=T)
    part = torch.full_like(x, 5.0)
    fl.ops.l2norm_scaled_strided(x, part, rows=32, token_stride=80 * 128, T=T)
    torch.cuda.synchronize()
    assert torch.equal(part[:, :32].view(torch.int16), full[:, :32].view(torch.int16))
    assert (part[:, 32:] == 5.0).all()


@pytest.mark.parametrize("T,rows", [(7, 3), (5, 80), (1, 1)])
def test_l2norm_row_layouts(fl, dev, orc, rng, T, rows):
    """Rows at 16-byte-aligned pitch 136 (16 lanes a row, 4 rows a wave) and
    at pitch 130 (a workgroup a row) give the same bits, the oracle's within
    1 ulp, leave the padding after each row untouched, and run in place;
    row counts that leave a wave's last rows empty."""
    x = (rng.standard_normal((T, rows, 128)) * 3).astype(np.float16)
    x[0, 0, :] = 0
    want = orc.l2norm_scaled(x.reshape(T, rows * 128), n=128, rows=rows, pitch=128, eps=1e-6,
                             scale=0.5, T=T).reshape(T, rows, 128)
    outs = []
    for pitch in (136, 130):
        xp = np.zeros((T, rows, pitch), np.float16)
        xp[..., :128] = x
        y = torch.full((T, rows, pitch), 7.0, dtype=torch.float16, device=dev)
        fl.ops.l2norm_scaled(torch.from_numpy(xp).to(dev), y, rows=rows, pitch=pitch,
                             scale=0.5, T=T)
        torch.cuda.synchronize()
        yh = y.cpu().numpy()
        assert (yh[..., 128:] == 7.0).all(), f"pitch {pitch}: wrote past the row"
        outs.append(yh[..., :128])
    assert np.array_equal(outs[0].view(np.int16), outs[1].view(np.int16))
    assert ulp16_diff(outs[0], want) <= 1
    xi = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    fl.ops.l2norm_scaled(xi, xi, rows=rows, scale=0.5, T=T)
    torch.cuda.synchronize()
    assert np.array_equal(xi.cpu().numpy().view(np.int16), outs[0].view(np.int16))


@pytest.mark.parametrize("n,pitch,rows,T", [(64, 64, 3, 5), (200, 203, 2, 4), (1024, 1024, 1, 3),
                                             (129, 129, 7, 1)])
def test_l2norm_other_row_lengths(fl, dev, orc, rng, n, pitch, rows, T):
    """Row lengths other than 128 (one wavefront a row): within 1 ulp of the
    oracle's block order (thread v sums x[v], x[v + 128], ...; warp trees;
    (r0 + r2) + (r1 + r3)), the padding after each row untouched, in place
    the same bits."""
    x = (rng.standard_normal((T, rows, pitch)) * 2).astype(np.float16)
    x[0, 0, :] = 0
    want = orc.l2norm_scaled(x.reshape(T, rows * pitch), n=n, rows=rows, pitch=pitch, eps=1e-6,
                             scale=0.75, T=T).reshape(T, rows, pitch)
    y = torch.full((T, rows, pitch), 7.0, dtype=torch.float16, device=dev)
    fl.ops.l2norm_scaled(torch.from_numpy(x).to(dev), y, n=n, rows=rows, pitch=pitch, scale=0.75,
                         T=T)
    xi = torch.from_numpy(x).to(dev)
    fl.ops.l2norm_scaled(xi, xi, n=n, rows=rows, pitch=pitch, scale=0.75, T=T)
    torch.cuda.synchronize()
    yh = y.cpu().numpy()
    assert (yh[..., n:] == 7.0).all()
    assert ulp16_diff(yh[..., :n], want[..., :n]) <= 1
    assert not yh[0, 0, :n].any()
    assert np.array_equal(xi.cpu().numpy()[..., :n].view(np.int16), yh[..., :n].view(np.int16))


def _scan_inputs(rng, T):
    c = rng.standard_normal((T, ROW)).astype(np.float16)
    ln = np.zeros_like(c)
    for t in range(T):
        for r in range(32):
            seg = c[t, 128 * r:128 * r + 128].astype(np.float64)
            ln[t, 128 * r:128 * r + 128] = seg / np.linalg.norm(seg)
    ln[:, 4096:] = c[:, 4096:]
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, NV))))).astype(np.float32)
    decay = np.exp(-np.log1p(np.exp(rng.standard_normal((T, NV))))).astype(np.float32)
    S0 = (rng.standard_normal((NV, 128, 128)) * 0.02).astype(np.float32)
    return ln, beta, decay, S0


@pytest.mark.parametrize("T", [1, 3, 40, 101])
def test_gdn_scan_vs_oracle(fl, dev, orc, rng, T):
    ln, beta, decay, S0 = _scan_inputs(rng, T)
    lnd = to_dev(ln, dev)
    S = to_dev(S0, dev)
    ck = torch.zeros((max(T - 1, 1), NV, 128, 128), dtype=torch.float32, device=dev)
    y = torch.empty((T, NV * 128), dtype=torch.float16, device=dev)
    fl.ops.gdn_scan(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:], to_dev(beta, dev),
                    to_dev(decay, dev), S, y, T=T, ck=ck, ck_step=NV * 128 * 128)
    torch.cuda.synchronize()
    S_r = S0.copy()
    ck_r = np.zeros((max(T - 1, 1), NV, 128, 128), np.float32)
    y_r = orc.gdn_scan(ln[:, :2048], ln[:, 2048:4096], ln[:, 4096:], beta, decay, S_r, T=T,
                       qk_stride=ROW, v_stride=ROW, out_scale=QS, ck=ck_r, ck_step=NV * 128 * 128)
    Sh = S.cpu().numpy()
    print(f"gdn_scan T={T}: state bit-exact {np.array_equal(Sh, S_r)}, "
          f"rel {rel_err(Sh, S_r):.2e}, y ulps {ulp16_diff(y.cpu().numpy(), y_r)}")
    assert rel_err(Sh, S_r) <= STATE_RTOL
    err, ok = close(y.cpu().numpy(), y_r, 2e-3, 1e-2)
    assert ok, err
    if T > 1:
        assert rel_err(ck.cpu().numpy(), ck_r) <= STATE_RTOL


def _decode_weights(rng):
    w = (rng.standard_normal((ROW, 4)) * 0.5).astype(np.float16)
    A_log = np.zeros(NV, np.float32)
    dt = np.zeros(NV, np.float32)
    return w, A_log, dt


def test_config1_decode_1024_steps_vs_oracle(fl, dev, orc):
    """Config 1: B=4, S0 ~ N(0, 0.02), conv fused, fp16 conv ring, 1024 steps;
    the fp32 state within rel 1e-4 of the oracle's after the last step."""
    rng = np.random.default_rng(1)
    B, steps = 4, 1024
    w, A_log, dt = _decode_weights(rng)
    S0 = (rng.standard_normal((B, NV, 128, 128)) * 0.02).astype(np.float32)
    wd, Ad, dtd = to_dev(w, dev), to_dev(A_log, dev), to_dev(dt, dev)
    S_d = [to_dev(S0[b], dev) for b in range(B)]
    ring = [[torch.zeros((ROW, 3), dtype=torch.float16, device=dev) for _ in range(2)]
            for _ in range(B)]
    S_r = [S0[b].copy() for b in range(B)]
    ring_r = [[np.zeros((ROW, 3), np.float16) for _ in range(2)] for _ in range(B)]
    worst_y = 0.0
    for step in range(steps):
        x = rng.standard_normal((B, 1, ROW)).astype(np.float16)
        a = rng.standard_normal((B, 1, NV)).astype(np.float32)
        bb = rng.standard_normal((B, 1, NV)).astype(np.float32)
        ph = step & 1
        y = fl.ops.gdn_decode(to_dev(x, dev), S_d, to_dev(a, dev), to_dev(bb, dev), Ad, dtd, T=1,
                              pos0s=[step] * B, conv_fused=True, conv_w=wd,
                              cst_in=[ring[b][ph] for b in range(B)],
                              cst_out=[ring[b][ph ^ 1] for b in range(B)])
        yh = y.cpu().numpy()
        for b in range(B):
            y_r = orc.gdn_decode(None, S_r[b], a[b], bb[b], A_log, dt, T=1, out_scale=QS,
                                 cx=x[b], cw=w, cst_in=ring_r[b][ph], cst_out=ring_r[b][ph ^ 1],
                                 pos0=step)
            worst_y = max(worst_y, float(np.abs(yh[b].astype(np.float64) - y_r).max()))
    worst_s = max(rel_err(S_d[b].cpu().numpy(), S_r[b]) for b in range(B))
    for b in range(B):
        assert np.array_equal(ring[b][0].cpu().numpy(), ring_r[b][0])
    print(f"config 1: 1024 steps, state rel {worst_s:.2e}, max|dy| {worst_y:.2e}")
    assert worst_s <= STATE_RTOL
    assert worst_y <= 2e-3


@pytest.mark.parametrize("T", [1, 3])
def test_fused_decode_equals_unfused_bit_exact(fl, dev, rng, T):
    """The fused decode (norms, gates and delta rule in one launch) against the
    unfused launches on the GPU -- l2norm_scaled, gdn_scalars, gdn_scan -- on
    the same conv output: y and the state bit for bit. The unfused l2norm adds
    the sums of squares in the reference's block_reduce_sum order, so this
    pins the fused kernel's in-wave norm to that order."""
    B = 2
    c = (rng.standard_normal((B, T, ROW)) * 2).astype(np.float16)
    c[1, 0, 2048:2176] = 0                                   # a zero k row
    a = rng.standard_normal((B, T, NV)).astype(np.float32)
    bb = rng.standard_normal((B, T, NV)).astype(np.float32)
    A_log = (rng.standard_normal(NV) * 0.3).astype(np.float32)
    dt = (rng.standard_normal(NV) * 0.3).astype(np.float32)
    S0 = (rng.standard_normal((B, NV, 128, 128)) * 0.02).astype(np.float32)
    Sf = [to_dev(S0[i], dev) for i in range(B)]
    yf = fl.ops.gdn_decode(to_dev(c, dev), Sf, to_dev(a, dev), to_dev(bb, dev), to_dev(A_log, dev),
                           to_dev(dt, dev), T=T, pos0s=[7] * B)
    for i in range(B):
        cd = to_dev(c[i], dev)
        ln = cd.clone()
        for t in range(T):
            fl.ops.l2norm_scaled(cd[t], ln[t], rows=32, T=1)
        beta = torch.empty((T, NV), dtype=torch.float32, device=dev)
        decay = torch.empty_like(beta)
        fl.ops.gdn_scalars(to_dev(a[i], dev), to_dev(bb[i], dev), to_dev(A_log, dev),
                           to_dev(dt, dev), beta, decay, T=T)
        Su = to_dev(S0[i], dev)
        yu = torch.empty((T, NV * 128), dtype=torch.float16, device=dev)
        fl.ops.gdn_scan(ln[:, :2048], ln[:, 2048:4096], ln[:, 4096:], beta, decay, Su, yu, T=T)
        torch.cuda.synchronize()
        assert torch.equal(yf[i], yu), f"seq {i}: y differs"
        assert torch.equal(Sf[i], Su), f"seq {i}: state differs"


def test_verify_t3_checkpoints_and_rollback(fl, dev, orc, rng):
    """MTP verify (runtime.py:3017-3053): conv rows then the fused scan with
    checkpoints; each checkpoint equals the state after that many T=1 steps."""
    T = 3
    w, A_log, dt = _decode_weights(rng)
    A_log[:] = rng.standard_normal(NV) * 0.3
    x = rng.standard_normal((1, T, ROW)).astype(np.float16)
    st = rng.standard_normal((ROW, 3)).astype(np.float16)
    a = rng.standard_normal((1, T, NV)).astype(np.float32)
    bb = rng.standard_normal((1, T, NV)).astype(np.float32)
    S0 = (rng.standard_normal((NV, 128, 128)) * 0.02).astype(np.float32)
    c = torch.empty((1, T, ROW), dtype=torch.float16, device=dev)
    sts = [torch.empty((ROW, 3), dtype=torch.float16, device=dev) for _ in range(3)]
    fl.ops.conv1d_causal_rows(to_dev(x[0], dev), to_dev(w, dev), to_dev(st, dev), c[0], *sts,
                              T=T, pos0=20)
    S = to_dev(S0, dev)
    ck = torch.zeros((T - 1, NV, 128, 128), dtype=torch.float32, device=dev)
    y = fl.ops.gdn_decode(c, [S], to_dev(a, dev), to_dev(bb, dev), to_dev(A_log, dev),
                          to_dev(dt, dev), T=T, pos0s=[20], ck=[ck], ck_step=NV * 128 * 128)
    # T = 1 steps on the GPU from the same start: checkpoint t == state after t+1 steps
    S1 = to_dev(S0, dev)
    for t in range(T):
        y1 = fl.ops.gdn_decode(c[:, t:t + 1].contiguous(), [S1], to_dev(a[:, t:t + 1], dev),
                               to_dev(bb[:, t:t + 1], dev), to_dev(A_log, dev), to_dev(dt, dev),
                               T=1, pos0s=[20 + t])
        assert torch.equal(y1[0, 0], y[0, t])
        want = S1 if t == T - 1 else ck[t]
        assert torch.equal(S1, want), t
    torch.cuda.synchronize()
    # and against the oracle
    S_r = S0.copy()
    y_c, _ = orc.conv1d_causal_rows(x[0], w, st, dim=ROW, T=T, pos0=20, row_stride=ROW)
    ck_r = np.zeros((T - 1, NV, 128, 128), np.float32)
    y_r = orc.gdn_decode(y_c, S_r, a[0], bb[0], A_log, dt, T=T, out_scale=QS, ck=ck_r,
                         ck_step=NV * 128 * 128)
    assert rel_err(S.cpu().numpy(), S_r) <= STATE_RTOL
    assert rel_err(ck.cpu().numpy(), ck_r) <= STATE_RTOL
    err, ok = close(y[0].cpu().numpy(), y_r, 2e-3, 1e-2)
    assert ok, err


@pytest.mark.parametrize("T", [1, 37, 64, 200, 8192])
def test_chunked_vs_recurrence(fl, dev, orc, T):
    """Config 4 (T = 8192) and ragged lengths: the chunked WY scan against the
    oracle's step-by-step recurrence on the same fp16 inputs."""
    rng = np.random.default_rng(T)
    ln, beta, decay, S0 = _scan_inputs(rng, T)
    lnd = to_dev(ln, dev)
    S = to_dev(S0, dev)
    y = fl.ops.gdn_prefill_chunked(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:],
                                   to_dev(beta, dev), to_dev(decay, dev), S, T=T)
    torch.cuda.synchronize()
    S_r = S0.copy()
    y_r = orc.gdn_scan(ln[:, :2048], ln[:, 2048:4096], ln[:, 4096:], beta, decay, S_r, T=T,
                       qk_stride=ROW, v_stride=ROW, out_scale=QS)
    Sh = S.cpu().numpy()
    print(f"chunked T={T}: state rel {rel_err(Sh, S_r):.2e}")
    assert rel_err(Sh, S_r) <= STATE_RTOL
    err, ok = close(y.cpu().numpy(), y_r, 2e-3, 1e-2)
    assert ok, f"T={T}: max|dy| {err}"
    # y against each (token, head) row's RMS, beyond one fp16 ulp of rounding:
    # the gated norm after the scan divides every row by its RMS, so an output
    # error inside y's own tolerance but large in a row whose terms cancel
    # would surface there. Emulated: fp32 products <= 1.3e-3, products on
    # split fp16 halves <= 2e-4, the output on one fp16 pass 1.6e-3 - 5.3e-3.
    yg = y.cpu().numpy().reshape(T, NV, 128).astype(np.float64)
    yr = y_r.reshape(T, NV, 128).astype(np.float64)
    rms = np.sqrt((yr ** 2).mean(axis=-1, keepdims=True)) + 1e-30
    beyond = float((np.maximum(np.abs(yg - yr) - 2.0 ** -10 * np.abs(yr), 0) / rms).max())
    print(f"chunked T={T}: y error against the row RMS beyond 1 ulp {beyond:.2e}")
    assert beyond <= 1.5e-3, f"T={T}: y error against the row RMS {beyond:.2e}"


def test_chunked_degenerate_chunks_vs_recurrence(fl, dev, orc):
    """Chunks whose operands vanish: tokens 64-127 with q = 0 (their M o QK^T
    block is zero) and tokens 192-255 with beta = 0 (their Delta is zero):
    the output's accumulator scale, chosen from Delta, once overflowed there
    and saturated y. Against the oracle's recurrence, as the other chunked
    cases."""
    T = 300
    rng = np.random.default_rng(300)
    ln, beta, decay, S0 = _scan_inputs(rng, T)
    ln[64:128, :2048] = 0
    beta[192:256] = 0
    lnd = to_dev(ln, dev)
    S = to_dev(S0, dev)
    y = fl.ops.gdn_prefill_chunked(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:],
                                   to_dev(beta, dev), to_dev(decay, dev), S, T=T)
    torch.cuda.synchronize()
    S_r = S0.copy()
    y_r = orc.gdn_scan(ln[:, :2048], ln[:, 2048:4096], ln[:, 4096:], beta, decay, S_r, T=T,
                       qk_stride=ROW, v_stride=ROW, out_scale=QS)
    assert rel_err(S.cpu().numpy(), S_r) <= STATE_RTOL
    yh = y.cpu().numpy()
    assert np.isfinite(yh.astype(np.float32)).all()
    err, ok = close(yh, y_r, 2e-3, 1e-2)
    assert ok, f"max|dy| {err}"


@pytest.mark.parametrize("regime", ["strong", "zero", "none", "mixed"])
def test_scans_extreme_decay_vs_recurrence(fl, dev, orc, regime):
    """Decay at its ends, for the recurrent and the chunked scan against the
    oracle's recurrence over 200 tokens: 'strong' ~e^-12 a token (the in-chunk
    ratios e^{g_i - g_j} underflow to 0 after a few tokens and the state is
    all but erased every step), 'zero' exactly 0 for a third of the tokens
    (the chunked form's log takes FLT_MIN there), 'none' exactly 1, 'mixed'
    alternating heads of strong and none with beta also at 0 and 1 for some
    tokens."""
    T = 200
    rng = np.random.default_rng({"strong": 11, "zero": 14, "none": 12, "mixed": 13}[regime])
    ln, beta, decay, S0 = _scan_inputs(rng, T)
    if regime == "strong":
        decay[:] = np.exp(-rng.uniform(10, 14, decay.shape)).astype(np.float32)
    elif regime == "zero":
        decay[::3] = 0.0
    elif regime == "none":
        decay[:] = 1.0
    else:
        decay[:, 0::2] = np.exp(-rng.uniform(10, 14, decay[:, 0::2].shape)).astype(np.float32)
        decay[:, 1::2] = 1.0
        beta[::7] = 0.0
        beta[3::11] = 1.0
    S_r = S0.copy()
    y_r = orc.gdn_scan(ln[:, :2048], ln[:, 2048:4096], ln[:, 4096:], beta, decay, S_r, T=T,
                       qk_stride=ROW, v_stride=ROW, out_scale=QS)
    lnd = to_dev(ln, dev)
    for form in ("recurrent", "chunked"):
        S = to_dev(S0, dev)
        if form == "recurrent":
            y = torch.empty((T, NV * 128), dtype=torch.float16, device=dev)
            fl.ops.gdn_scan(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:], to_dev(beta, dev),
                            to_dev(decay, dev), S, y, T=T)
        else:
            y = fl.ops.gdn_prefill_chunked(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:],
                                           to_dev(beta, dev), to_dev(decay, dev), S, T=T)
        torch.cuda.synchronize()
        yh, Sh = y.cpu().numpy(), S.cpu().numpy()
        assert np.isfinite(yh.astype(np.float32)).all() and np.isfinite(Sh).all(), form
        assert rel_err(Sh, S_r) <= STATE_RTOL, f"{regime} {form}: state rel {rel_err(Sh, S_r):.2e}"
        err, ok = close(yh, y_r, 2e-3, 1e-2)
        assert ok, f"{regime} {form}: max|dy| {err}"


def test_decode_beta_zero_is_pure_decay(fl, dev, rng):
    """Config 1's shape (B = 4, 48 v heads, conv fused) with b = -1000, so
    beta = 1 / (1 + e^1000) = 0 exactly: every state is decay * S_0 (one fp32
    product, bit for bit) with decay the gates kernel's value for the same
    inputs."""
    B = 4
    w, A_log, dt = _decode_weights(rng)
    S0 = (rng.standard_normal((B, NV, 128, 128)) * 0.02).astype(np.float32)
    S_d = [to_dev(S0[b], dev) for b in range(B)]
    x = rng.standard_normal((B, 1, ROW)).astype(np.float16)
    a = rng.standard_normal((B, 1, NV)).astype(np.float32)
    bb = np.full((B, 1, NV), -1000.0, np.float32)
    rings = [[torch.zeros((ROW, 3), dtype=torch.float16, device=dev) for _ in range(2)]
             for _ in range(B)]
    fl.ops.gdn_decode(to_dev(x, dev), S_d, to_dev(a, dev), to_dev(bb, dev), to_dev(A_log, dev),
                      to_dev(dt, dev), T=1, pos0s=[5] * B, conv_fused=True, conv_w=to_dev(w, dev),
                      cst_in=[r[0] for r in rings], cst_out=[r[1] for r in rings])
    beta = torch.empty((B, NV), dtype=torch.float32, device=dev)
    decay = torch.empty_like(beta)
    fl.ops.gdn_scalars(to_dev(a[:, 0], dev), to_dev(bb[:, 0], dev), to_dev(A_log, dev),
                       to_dev(dt, dev), beta, decay, T=B)
    torch.cuda.synchronize()
    assert not beta.cpu().numpy().any()
    dh = decay.cpu().numpy()
    for b in range(B):
        want = (dh[b][:, None, None] * S0[b]).astype(np.float32)
        assert np.array_equal(S_d[b].cpu().numpy(), want), f"sequence {b}"


# the 16-lanes-a-row kernel takes calls of >= 8192 rows with 16-byte aligned
# rows: 171 x 48 = 8208 and 8193 x 1 rows reach it with a ragged last wave
# (8208 % 16 == 0 but 8193 % 16 == 1; 8211 = 1173 x 7 leaves 3 rows in the last
# wave); the small cases keep the wave-a-row kernel on both pitches
@pytest.mark.parametrize("T,rows", [(1, 48), (3, 5), (7, 48), (171, 48), (8193, 1),
                                    (1173, 7)])
def test_rmsnorm_gated_row_layouts(fl, dev, orc, rng, T, rows):
    """Rows 16-byte aligned (pitch 136: from 8192 rows up, 16 lanes a row and
    4 rows a wave) and not (pitch 130: a wave a row) give the same bits, the
    oracle's, and leave the padding after each row untouched; row counts that
    leave a wave's last rows empty."""
    o = (rng.standard_normal((T, rows, 128)) * 0.7).astype(np.float16)
    z = (rng.standard_normal((T, rows, 128)) * 2).astype(np.float16)
    w = (1 + rng.standard_normal(128) * 0.2).astype(np.float32)
    want = orc.rmsnorm_gated(o, z, w, rows=rows, T=T)
    wd = torch.from_numpy(w).to(dev)
    outs = []
    for pitch in (136, 130):
        op = np.zeros((T, rows, pitch), np.float16)
        zp = np.zeros((T, rows, pitch), np.float16)
        op[..., :128], zp[..., :128] = o, z
        y = torch.full((T, rows, pitch), 7.0, dtype=torch.float16, device=dev)
        fl.ops.rmsnorm_gated(torch.from_numpy(op).to(dev), torch.from_numpy(zp).to(dev), wd, y,
                             T=T, rows=rows, pitch=pitch)
        torch.cuda.synchronize()
        yh = y.cpu().numpy()
        assert (yh[..., 128:] == 7.0).all(), f"pitch {pitch}: wrote past the row"
        outs.append(yh[..., :128])
    assert np.array_equal(outs[0].view(np.int16), outs[1].view(np.int16))
    d = np.abs(outs[0].view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    assert d.max() <= 1, f"max {d.max()} ulp"


@pytest.mark.parametrize("T", [1, 4, 1000])
def test_rmsnorm_gated_vs_oracle(fl, dev, orc, rng, T):
    """The GDN output norm through the C ABI: same operations and order as the
    oracle (deterministic exp in silu), so bit for bit; the bar is 1 fp16 ulp."""
    o = (rng.standard_normal((T, 48, 128)) * rng.uniform(0.01, 3)).astype(np.float16)
    z = (rng.standard_normal((T, 48, 128)) * 2).astype(np.float16)
    w = (1 + rng.standard_normal(128) * 0.2).astype(np.float32)
    want = orc.rmsnorm_gated(o, z, w, T=T)
    y = fl.ops.rmsnorm_gated(torch.from_numpy(o).to(dev), torch.from_numpy(z).to(dev),
                             torch.from_numpy(w).to(dev))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    d = np.abs(got.view(np.int16).astype(np.int32) - want.view(np.int16).astype(np.int32))
    print(f"rmsnorm_gated T={T}: max {d.max()} ulp, {(d > 0).sum()} values differ")
    assert d.max() <= 1


@pytest.mark.parametrize("B", [1, 4, 7])
def test_decode_normed_equals_decode_then_norm(fl, dev, orc, rng, B):
    """The one-launch decode step + output norm against the pair it replaces
    (gdn_decode with the conv fused, then rmsnorm_gated) over three steps in
    a row: the normed output, the state and both conv rings bit for bit.
    Sequences start at pos0 0 (no history) and past it; with B = 7 the gate
    and the output rows carry padding, which must stay untouched. Step 0 is
    also checked against the oracle's pair."""
    w, A_log, dt = _decode_weights(rng)
    A_log = (rng.standard_normal(NV) * 0.3).astype(np.float32)
    dt = (rng.standard_normal(NV) * 0.3).astype(np.float32)
    nw = (1 + rng.standard_normal(128) * 0.2).astype(np.float32)
    width = NV * 128
    zp, yp = (width + 64, width + 32) if B == 7 else (width, width)
    S0 = (rng.standard_normal((B, NV, 128, 128)) * 0.02).astype(np.float32)
    ring0 = rng.standard_normal((B, ROW, 3)).astype(np.float16)
    starts = [0 if b % 2 == 0 else 9 + b for b in range(B)]
    wd, Ad, dtd, nwd = to_dev(w, dev), to_dev(A_log, dev), to_dev(dt, dev), to_dev(nw, dev)
    Sf = [to_dev(S0[b], dev) for b in range(B)]
    Su = [to_dev(S0[b], dev) for b in range(B)]
    rf = [[to_dev(ring0[b], dev), torch.zeros((ROW, 3), dtype=torch.float16, device=dev)]
          for b in range(B)]
    ru = [[r[0].clone(), r[1].clone()] for r in rf]
    for step in range(3):
        x = rng.standard_normal((B, ROW)).astype(np.float16)
        a = rng.standard_normal((B, NV)).astype(np.float32)
        bb = rng.standard_normal((B, NV)).astype(np.float32)
        z = np.zeros((B, zp), np.float16)
        z[:, :width] = rng.standard_normal((B, width)) * 2
        xd, ad, bd, zd = to_dev(x, dev), to_dev(a, dev), to_dev(bb, dev), to_dev(z, dev)
        ph = step & 1
        pos = [s + step for s in starts]
        yf = torch.full((B, yp), 7.0, dtype=torch.float16, device=dev)
        fl.ops.gdn_decode_normed(xd, Sf, ad, bd, Ad, dtd, zd[:, :width], nwd, yf[:, :width],
                                 pos0s=pos, conv_w=wd, cst_in=[r[ph] for r in rf],
                                 cst_out=[r[ph ^ 1] for r in rf])
        yu = fl.ops.gdn_decode(xd[:, None], Su, ad[:, None], bd[:, None], Ad, dtd, T=1,
                               pos0s=pos, conv_fused=True, conv_w=wd,
                               cst_in=[r[ph] for r in ru], cst_out=[r[ph ^ 1] for r in ru])
        zc = zd[:, :width].contiguous()
        yn = fl.ops.rmsnorm_gated(yu.view(B, NV, 128), zc, nwd, T=B)
        torch.cuda.synchronize()
        yh = yf.cpu().numpy()
        assert (yh[:, width:] == 7.0).all(), f"step {step}: wrote into the row padding"
        assert torch.equal(yf[:, :width], yn.view(B, width)), f"step {step}: y differs"
        for b in range(B):
            assert torch.equal(Sf[b], Su[b]), f"step {step}, seq {b}: state differs"
            assert torch.equal(rf[b][ph ^ 1], ru[b][ph ^ 1]), f"step {step}, seq {b}: ring"
        if step == 0:
            for b in range(B):
                ring_r = [ring0[b].copy(), np.zeros((ROW, 3), np.float16)]
                y_r = orc.gdn_decode(None, S0[b].copy(), a[b:b + 1], bb[b:b + 1], A_log, dt,
                                     T=1, out_scale=QS, cx=x[b], cw=w, cst_in=ring_r[0],
                                     cst_out=ring_r[1], pos0=pos[b])
                want = orc.rmsnorm_gated(y_r.reshape(1, NV, 128), z[b:b + 1, :width], nw, T=1)
                err, ok = close(yh[b, :width], want.reshape(-1), 2e-2, 2e-2)
                assert ok, f"seq {b} against the oracle: max |dy| {err}"


@pytest.mark.parametrize("T,ab_stride", [(1, 48), (100, 48), (1024, 56)])
def test_chunked_logits_equals_gates_then_scan(fl, dev, rng, T, ab_stride):
    """The chunked scan forming beta and decay from the logits itself against
    gdn_scalars then the scan on its output: y and the state bit for bit
    (strong and weak decays, logits past softplus's x = 20 switch, a padded
    logit row)."""
    ln = (rng.standard_normal((T, ROW)) * 0.5).astype(np.float16)
    a = (rng.standard_normal((T, ab_stride)) * 4).astype(np.float32)
    a[:, 0] = 25.0                                       # softplus(x) = x branch
    bb = (rng.standard_normal((T, ab_stride)) * 3).astype(np.float32)
    A_log = (rng.standard_normal(NV) * 0.5).astype(np.float32)
    dt = (rng.standard_normal(NV) * 0.5).astype(np.float32)
    S0 = (rng.standard_normal((NV, 128, 128)) * 0.05).astype(np.float32)
    lnd, ad, bd = to_dev(ln, dev), to_dev(a, dev), to_dev(bb, dev)
    Ad, dtd = to_dev(A_log, dev), to_dev(dt, dev)
    S1, S2 = to_dev(S0, dev), to_dev(S0, dev)
    y1 = fl.ops.gdn_prefill_chunked_logits(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:], ad, bd,
                                           Ad, dtd, S1, T=T, ab_stride=ab_stride)
    beta = torch.empty((T, NV), dtype=torch.float32, device=dev)
    decay = torch.empty_like(beta)
    fl.ops.gdn_scalars(ad, bd, Ad, dtd, beta, decay, T=T, a_stride=ab_stride, b_stride=ab_stride)
    y2 = fl.ops.gdn_prefill_chunked(lnd[:, :2048], lnd[:, 2048:4096], lnd[:, 4096:], beta, decay,
                                    S2, T=T)
    torch.cuda.synchronize()
    assert torch.isfinite(y1.float()).all()
    assert torch.equal(y1, y2), f"T={T}: y differs"
    assert torch.equal(S1, S2), f"T={T}: state differs"


@pytest.mark.parametrize("B,T", [(1, 3), (1, 2), (3, 3)])
def test_verify_normed_equals_verify_then_norm(fl, dev, rng, B, T):
    """A verify round's rows through the one-launch step + output norm (the
    conv rows done before it) against gdn_decode over the same rows with
    checkpoints, then rmsnorm_gated: the normed rows, the final state and
    every checkpoint bit for bit."""
    A_log = (rng.standard_normal(NV) * 0.3).astype(np.float32)
    dt = (rng.standard_normal(NV) * 0.3).astype(np.float32)
    nw = (1 + rng.standard_normal(128) * 0.2).astype(np.float32)
    width = NV * 128
    c = (rng.standard_normal((B * T, ROW)) * 2).astype(np.float16)
    a = rng.standard_normal((B * T, NV)).astype(np.float32)
    bb = rng.standard_normal((B * T, NV)).astype(np.float32)
    z = (rng.standard_normal((B * T, width)) * 2).astype(np.float16)
    S0 = (rng.standard_normal((B, NV, 128, 128)) * 0.02).astype(np.float32)
    cd, ad, bd, zd = to_dev(c, dev), to_dev(a, dev), to_dev(bb, dev), to_dev(z, dev)
    Ad, dtd, nwd = to_dev(A_log, dev), to_dev(dt, dev), to_dev(nw, dev)
    state = NV * 128 * 128
    Sf = [to_dev(S0[i], dev) for i in range(B)]
    Su = [to_dev(S0[i], dev) for i in range(B)]
    ckf = [torch.full((max(T - 1, 1), NV, 128, 128), 9.0, device=dev) for _ in range(B)]
    cku = [t.clone() for t in ckf]
    yf = fl.ops.gdn_decode_normed(cd, Sf, ad, bd, Ad, dtd, zd, nwd, pos0s=[50] * B, T=T,
                                  conv_fused=False, ck=ckf, ck_step=state)
    yu = fl.ops.gdn_decode(cd.view(B, T, ROW), Su, ad.view(B, T, NV), bd.view(B, T, NV), Ad, dtd,
                           T=T, pos0s=[50] * B, ck=cku, ck_step=state)
    yn = fl.ops.rmsnorm_gated(yu.view(B * T, NV, 128), zd, nwd, T=B * T)
    torch.cuda.synchronize()
    assert torch.equal(yf, yn.view(B * T, width)), "normed rows differ"
    for i in range(B):
        assert torch.equal(Sf[i], Su[i]), f"seq {i}: state differs"
        assert torch.equal(ckf[i], cku[i]), f"seq {i}: checkpoints differ"
