"""The layer runtime on the GPU against the oracle, over the model's 64-layer
schedule (48 GDN, 16 full attention) with synthetic per-layer projections:
a prefill chunk, decode steps, an MTP verify that keeps two of three rows and
one that keeps one of two, and a batched decode of two sequences. Each
layer's output is held to the attention tolerance, the recurrent states to
rel 1e-4, the conv rings and the KV caches (prep's RoPE'd k, v) bit for bit.

The oracle side runs the reference's launch sequence per layer
(runtime.py:2780-2863 / 2961-3112): attn_prep then decode attention with the
gate, or prefill attention then attn_gate; the T = 1 fused conv + delta rule,
or conv1d_causal + l2norm_scaled + gdn_scalars + gdn_scan; rmsnorm_gated. A
verify's kept rows are checked against T = 1 steps, the property the
reference's MTP round relies on (runtime.py:2062-2069)."""
import numpy as np
import pytest
import torch

from conftest import close

pytestmark = pytest.mark.gpu

QS = 128 ** -0.5
ATTN_SCALE = 256 ** -0.5
ATOL, RTOL = 2e-3, 1e-2


def _np(t):
    return t.detach().cpu().numpy()


class Inputs:
    """Seeded projections for one forward of T rows of every layer."""

    def __init__(self, layer_types, T, seed):
        rng = np.random.default_rng(seed)
        self.T = T
        self.d = {}
        for i, kind in enumerate(layer_types):
            if kind == "full_attention":
                self.d[i] = (rng.standard_normal((T, 24, 512)).astype(np.float16),
                             rng.standard_normal((T, 4, 256)).astype(np.float16),
                             rng.standard_normal((T, 4, 256)).astype(np.float16))
            else:
                self.d[i] = (rng.standard_normal((T, 10240)).astype(np.float16),
                             (rng.standard_normal((T, 48, 128)) * 2).astype(np.float16),
                             rng.standard_normal((T, 48)).astype(np.float32),
                             rng.standard_normal((T, 48)).astype(np.float32))

    def rows(self, lo, hi):
        out = Inputs.__new__(Inputs)
        out.T = hi - lo
        out.d = {i: tuple(np.ascontiguousarray(a[lo:hi]) for a in v) for i, v in self.d.items()}
        return out


class GpuProj:
    """The Projections seam: hands the seeded inputs to the runtime as device
    tensors and keeps each layer's output."""

    def __init__(self, inp, dev):
        self.inp, self.dev, self.out = inp, dev, {}

    def _t(self, a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)

    def full_attn_in(self, layer, T):
        assert T == self.inp.T
        return tuple(self._t(a) for a in self.inp.d[layer])

    def gdn_in(self, layer, T):
        assert T == self.inp.T
        return tuple(self._t(a) for a in self.inp.d[layer])

    def layer_out(self, layer, out):
        self.out[layer] = _np(out)


class OracleStack:
    """The same layers on the CPU oracle, one sequence; kv8: int8 caches (the
    reference's attn_prep_q8 and int8 attention, runtime.py:2907-2959)."""

    def __init__(self, orc, rt, cap, kv8=False):
        self.orc, self.rt, self.cap, self.kv8 = orc, rt, cap, kv8
        self.w = {i: tuple(_np(t) for t in (w.q_norm, w.k_norm)) if i in rt.full_ord else
                  tuple(_np(t) for t in (w.conv_w, w.A_log, w.dt_bias, w.norm_w))
                  for i, w in rt.w.items()}
        self.S = {g: np.zeros((48, 128, 128), np.float32) for g in rt.gdn_ord.values()}
        self.conv = {g: [np.zeros((10240, 3), np.float16) for _ in range(2)]
                     for g in rt.gdn_ord.values()}
        buf = (lambda: orc.kv8_buffer(cap)) if kv8 else \
            (lambda: np.zeros((cap, 4, 256), np.float16))
        self.kc = {li: buf() for li in rt.full_ord.values()}
        self.vc = {li: buf() for li in rt.full_ord.values()}
        self.n, self.phase = 0, 0

    def step(self, inp):
        orc, T, pos0, out = self.orc, inp.T, self.n, {}
        for i, kind in enumerate(self.rt.layer_types):
            if kind == "full_attention":
                li = self.rt.full_ord[i]
                qg, k, v = (a.copy() for a in inp.d[i])
                wq, wk = self.w[i]
                prep = orc.attn_prep_q8 if self.kv8 else orc.attn_prep
                qr, _ = prep(qg, k, v, wq, wk, self.kc[li], self.vc[li], pos0=pos0, T=T,
                             max_pos=self.cap)
                if T <= 4:
                    dec = orc.attention_decode_q8 if self.kv8 else orc.attention_decode
                    z = dec(qr, self.kc[li], self.vc[li], pos0, max_pos=self.cap,
                            scale=ATTN_SCALE)
                else:
                    pre = orc.attention_prefill_q8 if self.kv8 else orc.attention_prefill
                    z = pre(qr, self.kc[li], self.vc[li], q_pitch=512, pos0=pos0,
                            max_pos=self.cap, scale=ATTN_SCALE, T=T)
                    orc.attn_gate(z, qr, 24, 256, 256, 512, 256, T)
                out[i] = z
            else:
                g = self.rt.gdn_ord[i]
                qkv, zg, a, b = inp.d[i]
                cw, A_log, dt, nw = self.w[i]
                cin, cout = self.conv[g][self.phase], self.conv[g][self.phase ^ 1]
                if T == 1:
                    y = orc.gdn_decode(None, self.S[g], a, b, A_log, dt, T=1, out_scale=QS,
                                       cx=qkv, cw=cw, cst_in=cin, cst_out=cout, pos0=pos0)
                else:
                    c, so = orc.conv1d_causal(qkv, cw, cin, dim=10240, T=T, pos0=pos0,
                                              row_stride=10240)
                    cout[...] = so
                    ln = orc.l2norm_scaled(c, n=128, rows=80, pitch=128, eps=1e-6, scale=1.0, T=T)
                    beta, decay = orc.gdn_scalars(a, b, A_log, dt, T=T, n_heads=48)
                    y = orc.gdn_scan(ln[:, :2048], ln[:, 2048:4096], c[:, 4096:], beta, decay,
                                     self.S[g], T=T, qk_stride=10240, v_stride=10240,
                                     out_scale=QS)
                out[i] = orc.rmsnorm_gated(y.reshape(T, 48, 128), zg, nw, T=T)
        self.n += T
        self.phase ^= 1
        return out


def _check_outputs(got, want, what, rows=None):
    for i in want:
        g = got[i] if rows is None else got[i][rows]
        err, ok = close(g, want[i], ATOL, RTOL)
        assert ok, f"{what}: layer {i} max|err| {err}"


def _check_state(rt, st, ref, what):
    worst = 0.0
    for g in ref.S:
        gs = _np(st.s[g]).astype(np.float64)
        worst = max(worst, float(np.abs(gs - ref.S[g]).max() / np.abs(ref.S[g]).max()))
        assert np.array_equal(_np(st.conv[st.phase, g]), ref.conv[g][ref.phase]), \
            f"{what}: conv ring of GDN layer {g}"
    assert worst <= 1e-4, f"{what}: recurrent state rel {worst:.2e}"
    n = len(st.tokens)
    assert n == ref.n
    for li in ref.kc:
        for name, got, want in (("K", st.kk[li], ref.kc[li]), ("V", st.kv[li], ref.vc[li])):
            if ref.kv8:   # values and block scales, each buffer at its own capacity
                gv, gs = ref.orc.kv8_split(_np(got), st.lcap[li])
                wv, ws = ref.orc.kv8_split(want, ref.cap)
                same = np.array_equal(gv[:n], wv[:n]) and \
                    np.array_equal(gs[:n].view(np.int16), ws[:n].view(np.int16))
            else:
                same = np.array_equal(_np(got[:n]), want[:n])
            assert same, f"{what}: {name} of layer {li}"
    print(f"{what}: {n} positions, state rel {worst:.2e}")


def test_runtime_stack_prefill_decode_verify(fl, dev, orc):
    rt_mod = fl.runtime
    rt = rt_mod.HybridRuntime(rt_mod.random_weights(seed=5), device=dev)
    st = rt.new_state()
    ref = OracleStack(orc, rt, cap=128)
    types = rt.layer_types

    # a prefill chunk (chunked WY scan, causal prefill attention)
    inp = Inputs(types, 40, seed=1)
    p = GpuProj(inp, dev)
    rt.forward(st, p, list(range(100, 140)))
    torch.cuda.synchronize()
    _check_outputs(p.out, ref.step(inp), "prefill 40")
    _check_state(rt, st, ref, "after prefill")

    # two decode steps (the fused conv + delta rule, split-K attention)
    for s in range(2):
        inp = Inputs(types, 1, seed=10 + s)
        p = GpuProj(inp, dev)
        rt.forward(st, p, [200 + s])
        torch.cuda.synchronize()
        _check_outputs(p.out, ref.step(inp), f"decode {s}")
    _check_state(rt, st, ref, "after decode")

    # a verify of 3 rows keeping 2: rows 0 and 1 equal T = 1 steps
    inp = Inputs(types, 3, seed=20)
    p = GpuProj(inp, dev)
    rt.forward(st, p, [300, 301, 302], verify=True)
    rt.accept_verify(st, [300, 301, 302], kept=2)
    torch.cuda.synchronize()
    for r in range(2):
        _check_outputs(p.out, ref.step(inp.rows(r, r + 1)), f"verify row {r}", rows=slice(r, r + 1))
    _check_state(rt, st, ref, "after verify, 2 of 3 kept")

    # a verify of 2 rows keeping 1 (the reject)
    inp = Inputs(types, 2, seed=30)
    p = GpuProj(inp, dev)
    rt.forward(st, p, [400, 401], verify=True)
    rt.accept_verify(st, [400, 401], kept=1)
    torch.cuda.synchronize()
    _check_outputs(p.out, ref.step(inp.rows(0, 1)), "verify reject row 0", rows=slice(0, 1))
    _check_state(rt, st, ref, "after verify, 1 of 2 kept")

    # and a decode step on from there
    inp = Inputs(types, 1, seed=40)
    p = GpuProj(inp, dev)
    rt.forward(st, p, [500])
    torch.cuda.synchronize()
    _check_outputs(p.out, ref.step(inp), "decode after reject")
    _check_state(rt, st, ref, "final")


@pytest.mark.parametrize("kv8", [False, True])
def test_runtime_stack_continuation_prefill(fl, dev, orc, kv8):
    """A prompt fed as two prefills, the reference's sub-chunked prompt in
    small (runtime.py:1939-1966): 40 tokens, then 200 at pos0 40 -- the GDN
    layers' chunked scan over chunks of 64 + 64 + 64 + 8 from the state the
    first call left, the conv ring carried across the calls; the attention
    layers' prefill over the 40 rows already cached -- then two decode steps,
    each against the oracle stack. fp16 and int8 caches; the runtime's caches
    grow from 64 to 256 positions between the calls (int8: values and scales
    moved as two regions)."""
    rt_mod = fl.runtime
    rt = rt_mod.HybridRuntime(rt_mod.random_weights(seed=7), device=dev, kv8=kv8)
    st = rt.new_state()
    ref = OracleStack(orc, rt, cap=256, kv8=kv8)
    types = rt.layer_types
    for T, seed, what in ((40, 60, "prefill 40"), (200, 61, "prefill 200 at pos0 40")):
        inp = Inputs(types, T, seed=seed)
        p = GpuProj(inp, dev)
        pos = len(st.tokens)
        rt.forward(st, p, list(range(pos, pos + T)))
        torch.cuda.synchronize()
        _check_outputs(p.out, ref.step(inp), what)
        _check_state(rt, st, ref, what)
    assert min(st.lcap) == 256
    for s in range(2):
        inp = Inputs(types, 1, seed=62 + s)
        p = GpuProj(inp, dev)
        rt.forward(st, p, [600 + s])
        torch.cuda.synchronize()
        _check_outputs(p.out, ref.step(inp), f"decode {s}")
    _check_state(rt, st, ref, "after decode")


@pytest.mark.parametrize("rule", ["length", "grid"])
@pytest.mark.parametrize("kv8", [False, True])
def test_runtime_batched_decode_equals_single(fl, dev, kv8, rule):
    """forward_batch over two sequences at different positions gives each the
    state its own single-sequence step gives, bit for bit, and the same
    outputs: bit for bit under the length-only split rule; under the default
    grid rule (the split sized to the batch) the attention layers' outputs
    within the attention bar and every other output bit for bit."""
    rt_mod = fl.runtime
    sr = fl.geometry.SPLIT_ROWS if rule == "length" else fl.geometry.DEC_SPLIT_ROWS
    rt = rt_mod.HybridRuntime(rt_mod.random_weights(seed=6), device=dev, kv8=kv8, split_rows=sr)
    types = rt.layer_types
    a, b = rt.new_state(), rt.new_state()
    rt.forward(a, GpuProj(Inputs(types, 20, seed=2), dev), list(range(20)))
    rt.forward(b, GpuProj(Inputs(types, 7, seed=3), dev), list(range(7)))
    a1, b1 = rt.clone_state(a), rt.clone_state(b)
    ia, ib = Inputs(types, 1, seed=50), Inputs(types, 1, seed=51)
    both = Inputs.__new__(Inputs)
    both.T = 2
    both.d = {i: tuple(np.concatenate([x, y]) for x, y in zip(ia.d[i], ib.d[i])) for i in ia.d}
    pb = GpuProj(both, dev)
    rt.forward_batch([a, b], pb, [7, 8])
    pa, pb1 = GpuProj(ia, dev), GpuProj(ib, dev)
    rt.forward(a1, pa, [7])
    rt.forward(b1, pb1, [8])
    torch.cuda.synchronize()
    for i in pb.out:
        for got, want in ((pb.out[i][0:1], pa.out[i]), (pb.out[i][1:2], pb1.out[i])):
            if rule == "grid" and types[i] == "full_attention":
                err, ok = close(got, want, ATOL, RTOL)
                assert ok, (i, err)
            else:
                assert np.array_equal(got.view(np.int16), want.view(np.int16)), i
    for x, y in ((a, a1), (b, b1)):
        assert x.tokens == y.tokens and x.phase == y.phase
        assert torch.equal(x.s, y.s) and torch.equal(x.conv, y.conv)
        for u, w in zip(x.kk + x.kv, y.kk + y.kv):
            assert torch.equal(u, w)
