"""The engine-facing backend's step() on the GPU, over the model's 64-layer
schedule, against the oracle's layer stack (tests/test_gpu_runtime.py's
OracleStack: the reference's launch sequence per layer on the CPU oracle).

One sequence is driven through step() as the engine drives it: a 40-token
prompt cut into sub-chunks (max_chunk 16 here, so three forwards at pos0 0,
16, 32; the reference's MAX_CHUNK = 1024, runtime.py:1939-1966), decode
steps, speculative rounds -- K = 2 accepting both drafts, then one, then
none; K = 1 accepting and rejecting (runtime.py:2033-2215) -- and then a
batched decode beside a second sequence (runtime.py:1793-1838). Every
forward the backend ran is replayed on the oracle: prefill sub-chunks and
decode rows as they ran, a verify's kept rows as the T = 1 steps they must
equal. Each layer's output is held to the attention tolerance, the final
recurrent states to rel 1e-4, conv rings and KV caches bit for bit. The
synthetic head makes greedy decoding follow a known chain, so the token
stream itself checks the rounds' bookkeeping."""
import numpy as np
import pytest
import torch

from test_gpu_runtime import ATOL, RTOL, OracleStack, _np
from conftest import close

pytestmark = pytest.mark.gpu


class Ctx:
    def cancelled(self):
        return False


class Script:
    """The drafter's proposals, round by round: 'truth' (the chain), 'one'
    (first right, second wrong), 'none' (first wrong), 'k1' (one right
    draft), 'k1x' (one wrong draft)."""

    def __init__(self):
        self.plan = []

    def __call__(self, context, n, truth):
        mode = self.plan.pop(0) if self.plan else "truth"
        wrong = lambda t: t % 200 + 1     # noqa: E731  (never t itself)
        if mode == "truth":
            return truth
        if mode == "one":
            return [truth[0], wrong(truth[1])]
        if mode == "none":
            return [wrong(truth[0]), truth[1]]
        if mode == "k1":
            return truth[:1]
        return [wrong(truth[0])]


def _instrument(runtime):
    """Log every forward the layer runtime runs and every verify outcome."""
    rt, log = runtime.rt, []
    fwd, fb, acc = rt.forward, rt.forward_batch, rt.accept_verify

    def forward(st, proj, tokens, verify=False):
        log.append(("fwd", st, proj, len(st.tokens), verify))
        return fwd(st, proj, tokens, verify)

    def forward_batch(states, proj, tokens):
        log.append(("batch", list(states), proj, [len(s.tokens) for s in states], False))
        return fb(states, proj, tokens)

    def accept_verify(st, tokens, kept):
        log.append(("accept", st, None, kept, False))
        return acc(st, tokens, kept)

    rt.forward, rt.forward_batch, rt.accept_verify = forward, forward_batch, accept_verify
    return log


def _inputs(proj, rows, layer_types):
    """The oracle's numpy inputs of rows [lo, hi) of a forward's projections."""
    lo, hi = rows
    class Inp:
        pass
    inp = Inp()
    inp.T = hi - lo
    inp.d = {}
    T = len(proj.tokens)
    for i, kind in enumerate(layer_types):
        parts = proj.full_attn_in(i, T) if kind == "full_attention" else proj.gdn_in(i, T)
        inp.d[i] = tuple(np.ascontiguousarray(_np(p)[lo:hi]) for p in parts)
    return inp


def _compare(proj, rows, out_rows, want, what):
    for i in want:
        got = _np(proj.out[i])[out_rows[0]:out_rows[1]]
        err, ok = close(got, want[i], ATOL, RTOL)
        assert ok, f"{what}: layer {i} max|err| {err}"


def _replay(log, refs, layer_types):
    """Replay the logged forwards on the oracle stacks (one per sequence)."""
    n = 0
    for k, (kind, st, proj, pos, verify) in enumerate(log):
        if kind == "fwd" and not verify:
            ref = refs[id(st)]
            T = len(proj.tokens)
            assert pos == ref.n
            want = ref.step(_inputs(proj, (0, T), layer_types))
            _compare(proj, (0, T), (0, T), want, f"forward {k} (T={T}, pos0={pos})")
            n += 1
        elif kind == "fwd":
            kept = log[k + 1][3]
            assert log[k + 1][0] == "accept"
            ref = refs[id(st)]
            for r in range(kept):
                want = ref.step(_inputs(proj, (r, r + 1), layer_types))
                _compare(proj, (r, r + 1), (r, r + 1), want,
                         f"verify {k} row {r} of {len(proj.tokens)} (kept {kept})")
            n += 1
        elif kind == "batch":
            for r, s in enumerate(st):
                want = refs[id(s)].step(_inputs(proj, (r, r + 1), layer_types))
                _compare(proj, (r, r + 1), (r, r + 1), want, f"batch {k} row {r}")
            n += 1
    return n


def _check_state(seq, ref, what):
    worst = 0.0
    for g in ref.S:
        gs = _np(seq.s[g]).astype(np.float64)
        worst = max(worst, float(np.abs(gs - ref.S[g]).max() / np.abs(ref.S[g]).max()))
        assert np.array_equal(_np(seq.conv[seq.phase, g]), ref.conv[g][ref.phase]), \
            f"{what}: conv ring of GDN layer {g}"
    assert worst <= 1e-4, f"{what}: recurrent state rel {worst:.2e}"
    n = len(seq.tokens)
    assert n == ref.n, (what, n, ref.n)
    for li in ref.kc:
        assert np.array_equal(_np(seq.kk[li][:n]), ref.kc[li][:n]), f"{what}: K of layer {li}"
        assert np.array_equal(_np(seq.kv[li][:n]), ref.vc[li][:n]), f"{what}: V of layer {li}"
    print(f"{what}: {n} positions, state rel {worst:.2e}")


def _chain_ok(pkg, stream, start_tok, start_pos):
    tok, pos = start_tok, start_pos
    for t in stream:
        assert t == pkg.successor(tok, pos), (t, tok, pos)
        tok, pos = t, pos + 1


def test_step_prefill_decode_rounds_batch_vs_oracle(fl, dev, orc):
    be = fl.backend
    script = Script()
    pkg = be.SyntheticPackage(seed=3, kv8=False, device=dev, draft_fn=script)
    runtime = be.create(pkg, device=dev, max_chunk=16)
    runtime.open("")
    log = _instrument(runtime)
    greedy = be.SamplingSpec(temperature=0.0)
    ctx = Ctx()

    a = runtime.new_state()
    refs = {id(a.seq): OracleStack(orc, runtime.rt, cap=128)}
    prompt = [int(x) for x in np.random.default_rng(0).integers(1, 256, 40)]
    stream = []
    r = runtime.step([be.StepItem(a, prompt, greedy)], ctx)[0]
    assert r.forwarded_tokens == 40
    stream.append(r.token)
    assert [e[3] for e in log if e[0] == "fwd"] == [0, 16, 32]       # three sub-chunks
    for _ in range(2):                                                # plain decode steps
        stream.append(runtime.step([be.StepItem(a, [], greedy)], ctx)[0].token)

    runtime.set_speculative(True)
    stream.append(runtime.step([be.StepItem(a, [], greedy)], ctx)[0].token)  # drafts appear
    script.plan = ["one", "none", "k1", "k1x", "truth"]
    handed = []
    for _ in range(12):
        res = runtime.step([be.StepItem(a, [], greedy)], ctx)[0]
        handed.append(res.forwarded)
        stream.append(res.token)
    assert runtime.mtp_rounds >= 5 and runtime.mtp_reject >= 2 and runtime.mtp_accept >= 3
    assert False in handed                       # an accepted round's queued token
    _chain_ok(pkg, stream, prompt[-1], 39)

    while a.out:                                 # hand out what a round still holds
        stream.append(runtime.step([be.StepItem(a, [], greedy)], ctx)[0].token)
    # a second sequence, then one batched decode of both (speculation off)
    runtime.set_speculative(False)
    b = runtime.new_state()
    refs[id(b.seq)] = OracleStack(orc, runtime.rt, cap=128)
    runtime.step([be.StepItem(b, prompt[:7], greedy)], ctx)
    res = runtime.step([be.StepItem(a, [], greedy), be.StepItem(b, [], greedy)], ctx)
    assert log[-1][0] == "batch"
    stream.append(res[0].token)
    _chain_ok(pkg, stream, prompt[-1], 39)
    torch.cuda.synchronize()

    n = _replay(log, refs, runtime.rt.layer_types)
    print(f"replayed {n} forwards; rounds {runtime.mtp_rounds}, accepted "
          f"{runtime.mtp_accept}, rejected {runtime.mtp_reject}")
    _check_state(a.seq, refs[id(a.seq)], "sequence a")
    _check_state(b.seq, refs[id(b.seq)], "sequence b")


def test_step_int8_cache_follows_the_chain(fl, dev):
    """The same flow over the int8 KV cache (the reference's shipped format):
    every step's token follows the synthetic chain, a prompt past MAX_CHUNK
    (1030 tokens: sub-chunks of 1024 and 6) included, and the state export
    round-trips."""
    be = fl.backend
    types = ("linear_attention",) * 3 + ("full_attention",)
    pkg = be.SyntheticPackage(seed=4, kv8=True, device=dev, layer_types=types)
    runtime = be.create(pkg, device=dev)
    runtime.open("")
    log = _instrument(runtime)
    greedy = be.SamplingSpec(temperature=0.0)
    a = runtime.new_state()
    prompt = [int(x) for x in np.random.default_rng(1).integers(1, 256, 1030)]
    stream = [runtime.step([be.StepItem(a, prompt, greedy)], Ctx())[0].token]
    assert [e[3] for e in log if e[0] == "fwd"] == [0, 1024]
    runtime.set_speculative(True)
    for _ in range(8):
        stream.append(runtime.step([be.StepItem(a, [], greedy)], Ctx())[0].token)
    _chain_ok(pkg, stream, prompt[-1], 1029)
    assert runtime.mtp_accept >= 1
    c = runtime.clone_state(a)
    assert c.seq.tokens == a.seq.tokens[:len(c.seq.tokens)]
    for _ in range(3):
        stream.append(runtime.step([be.StepItem(a, [], greedy)], Ctx())[0].token)
    _chain_ok(pkg, stream, prompt[-1], 1029)
