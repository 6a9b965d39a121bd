"""The engine-facing backend's contract on the CPU (no kernel runs: every
refusal below happens before a forward): create() exposes the 13 methods of
footless/sdk.py:172-186; open() reports the reference's facts (max_batch 4,
34,816 cache bytes a token for the int8 format, model/footless/manifest:13);
step() refuses an oversized batch, a state twice in one batch, a freed state,
an empty step with nothing to sample and a context past max_context
(runtime.py:1729-1735, 1890-1900); a cancelled step forwards nothing; a
refused budget claim leaves every state as it was (runtime.py:1738-1748).
States live in host memory here (device "cpu") over a 4-layer schedule."""
import pytest

TYPES = ("linear_attention", "linear_attention", "linear_attention", "full_attention")


class Ctx:
    def __init__(self, cancel=False):
        self.cancel = cancel

    def cancelled(self):
        return self.cancel


class Ledger:
    """Accounting that refuses claims past `limit` bytes outstanding."""

    def __init__(self, be, limit):
        self.be, self.limit, self.held = be, limit, 0

    def claim(self, n):
        if self.held + n > self.limit:
            raise self.be.BudgetRefused(f"{n} B over the budget")
        self.held += n

        class C:
            nbytes = n
        return C()

    def release(self, c):
        self.held -= c.nbytes

    def available(self):
        return self.limit - self.held


class Services:
    def __init__(self, acc):
        self.accounting = acc

    @staticmethod
    def log(level, msg):
        pass


@pytest.fixture
def be(fl):
    return fl.backend


def _open(be, kv8=True, services=None):
    pkg = be.SyntheticPackage(layer_types=TYPES, kv8=kv8, device="cpu", vocab=64)
    rt = be.create(pkg, device="cpu")
    facts = rt.open("", services)
    return rt, facts


def test_create_exposes_the_runtime_methods(be):
    rt = be.create()
    for name in be.RUNTIME_METHODS:
        assert callable(getattr(rt, name)), name
    assert len(be.RUNTIME_METHODS) == 13


@pytest.mark.parametrize("kv8,row", [(True, 34816), (False, 65536)])
def test_open_facts(be, kv8, row):
    rt, facts = _open(be, kv8)
    # 16 full-attention layers in the model; this 4-layer schedule has 1
    assert facts.cache_bytes_per_token == row // 16
    assert facts.max_batch == 4 and facts.max_context == 102400
    assert "speculative" in facts.capabilities and facts.stop_tokens == [0]


def test_step_refuses_contract_violations(be):
    rt, _ = _open(be)
    spec = be.SamplingSpec(temperature=0.0)
    states = [rt.new_state() for _ in range(5)]
    with pytest.raises(be.ContractError, match="max_batch"):
        rt.step([be.StepItem(s, [1], spec) for s in states], Ctx())
    with pytest.raises(be.ContractError, match="more than once"):
        rt.step([be.StepItem(states[0], [1]), be.StepItem(states[0], [2])], Ctx())
    with pytest.raises(be.ContractError, match="nothing to forward"):
        rt.step([be.StepItem(states[1], [], spec)], Ctx())
    with pytest.raises(be.ContractError, match="max_context"):
        rt.step([be.StepItem(states[2], [1] * 102401, spec)], Ctx())
    rt.free_state(states[3])
    with pytest.raises(be.ContractError, match="freed"):
        rt.step([be.StepItem(states[3], [1], spec)], Ctx())
    for s in states[:3] + states[4:]:
        assert s.seq.tokens == [] and s.seq.cap == 0


def test_cancelled_step_forwards_nothing(be):
    rt, _ = _open(be)
    s = rt.new_state()
    res = rt.step([be.StepItem(s, [5, 6, 7], be.SamplingSpec(temperature=0.0))], Ctx(True))
    assert res[0].token is None and res[0].finished
    assert s.seq.tokens == [] and s.seq.cap == 0


def test_refused_growth_moves_nothing(be):
    """A claim refused while the step makes room raises BudgetRefused before
    any forward, leaving capacity, tokens and claims as they were."""
    rt0, _ = _open(be)
    base = rt0._bytes(0)
    led = Ledger(be, 2 * base + 4096)      # two fresh states fit; no KV room for either
    rt, _ = _open(be, services=Services(led))
    a, b = rt.new_state(), rt.new_state()
    held = led.held
    with pytest.raises(be.BudgetRefused):
        rt.step([be.StepItem(a, [1, 2]), be.StepItem(b, [3])], Ctx())
    assert led.held == held
    assert a.seq.cap == 0 and b.seq.cap == 0 and a.seq.tokens == [] and b.seq.tokens == []
    rt.free_state(a)
    rt.free_state(b)
    assert led.held == 0


def test_text_verbs(be):
    rt, _ = _open(be)
    ids = rt.encode("héllo")
    assert rt.decode(ids) == "héllo"
    chat = rt.chat([{"role": "user", "content": "hi"}])
    assert rt.decode(chat).endswith("<assistant>")


def test_truncate_and_state_bytes(be):
    rt, _ = _open(be)
    s = rt.new_state()
    assert rt.state_nbytes(s) == rt.rt.s_bytes + 2 * rt.rt.conv_bytes
    s.seq.tokens = [1, 2, 3]
    s.seq.fed = 3
    rt.truncate_state(s, 1)
    assert s.seq.replay == [1] and s.seq.tokens == [1] and not s.seq.s.any()
    with pytest.raises(be.ContractError):
        rt.truncate_state(s, -1)
