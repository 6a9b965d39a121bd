"""The engine-facing backend over the hot path: `create()` returns a runtime
with the 13 methods of the engine's Runtime protocol (footless/sdk.py:136-186,
`RUNTIME_METHODS`, checked by engine.load_runtime, engine.py:985-999) -- the
role model/footless/cuda_sm60/runtime.py's CudaRuntime plays for that
backend (open 576-644, the state verbs 1017-1405, step 1729-1966, the MTP
rounds 2033-2246, create 3999-4002).

What runs here: every layer of every forward through `HybridRuntime`
(runtime.py of this package, the HIP kernels of libfl355); the step's
contract around it -- the batch checks, every state's room claimed before
anything moves, cancellation, prompts cut into MAX_CHUNK sub-chunks with the
conv phase flipped per sub-chunk, decode rows of several sequences in one
batched forward, and the speculative verify rounds (K = 1: [p, d]; K = 2:
[p, d1, d2]) that keep the longest accepted prefix and roll the recurrent
and conv state back to the checkpoint after the last kept row.

What the model package supplies (`ModelPackage`): the weights of the hot
path's layers, the projections between them (embedding, EXL3 projections,
MLP), the LM head, the sampler, the tokenizer and the drafter -- the
reference backend's other kernels and host code, outside this path.
`SyntheticPackage` is a seeded stand-in for all of them (there is no
checkpoint or tokenizer here): tests and the bench drive the backend through
it, and a real package plugs in at `create(package)`.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Protocol, Sequence

import numpy as np
import torch

from . import state_blob
from .runtime import LAYER_TYPES, MTP_K, HybridRuntime, Projections, SeqState, random_weights

# The engine's contract types when the engine is installed; otherwise these
# mirrors of footless/sdk.py's (same names, fields and meaning), which the
# engine's own objects satisfy attribute for attribute.
try:                                                    # pragma: no cover - engine absent here
    from footless.sdk import (BudgetRefused, ContractError, Facts, SamplingSpec,  # type: ignore
                              StepResult)
except ImportError:
    class ContractError(Exception):
        """A contract violation (sdk.py:14-15)."""

    class BudgetRefused(ContractError):
        """A claim the budget could not admit (sdk.py:18-19)."""

    @dataclass(frozen=True)
    class Facts:
        """Load-time truths (sdk.py:22-37)."""
        cache_bytes_per_token: int
        max_batch: int
        max_context: int
        capabilities: list
        stop_tokens: list
        thinking_markers: list = field(default_factory=list)
        thinking_open_at_start: bool = False
        thinking_levels: list = field(default_factory=list)
        default_sampling: Any = None

    @dataclass(frozen=True)
    class SamplingSpec:
        """What the engine's sampling policy asks of one row (sdk.py:40-65)."""
        temperature: float = 0.8
        top_k: int = 40
        top_p: float = 0.95
        min_p: float = 0.0
        logprobs: int = 0
        seed: int | None = None
        repetition_penalty: float = 1.0
        presence_penalty: float = 0.0
        frequency_penalty: float = 0.0

    @dataclass
    class StepResult:
        """One item's outcome (sdk.py:75-96)."""
        token: int | None
        finished: bool
        top_logprobs: list | None = None
        forwarded: bool = True
        forwarded_tokens: int = 0


@dataclass
class StepItem:
    """sdk.py:68-72: a state, the tokens fed (empty: decode) and the sampling
    (None: a prefill chunk that samples nothing)."""
    state: Any
    input_tokens: list
    sampling: Any = None


RUNTIME_METHODS = ("open", "close", "new_state", "clone_state", "truncate_state", "state_nbytes",
                   "export_state", "import_state", "free_state", "encode", "decode", "chat",
                   "step")                              # sdk.py:172-186

MAX_BATCH = 4                                           # runtime.py:138
MAX_CHUNK = 1024                                        # runtime.py:196
VOCAB_ROW = state_blob.VOCAB                            # the state's logits row (runtime.py:1020)


class ModelPackage(Protocol):
    """The model package's side of the backend: what the reference's
    CudaRuntime does besides the attention / GDN layers."""

    kv8: bool                 # the KV cache format (the package manifest's, runtime.py:123-132)
    stop_tokens: Sequence[int]
    vocab: int

    def layer_types(self) -> Sequence[str]:
        """config.json's `layer_types` (runtime.py:654-665)."""

    def weights(self, layer_types: Sequence[str], device) -> dict:
        """FullWeights / GdnWeights a layer (runtime.py's FullWeights, GdnWeights)."""

    def projections(self, tokens: Sequence[int], positions: Sequence[int], device) -> Projections:
        """The Projections of one forward of these rows (row r: token
        tokens[r] at position positions[r]); layer_out chains the hidden."""

    def logits(self, proj: Projections) -> torch.Tensor:
        """[rows, vocab] float32 logits of the forward `proj` served."""

    def sample(self, row: torch.Tensor, spec, prompt_ids: list, output_ids: list) -> int:
        """One token from one logits row under `spec` (the package's sampler)."""

    def sampler_state(self, spec) -> Any:
        """The draw stream's position for `spec`, to undo draws a verify drops."""

    def restore_sampler(self, spec, state: Any) -> None: ...

    def draft(self, context: Sequence[int], n: int) -> list:
        """Up to n drafted tokens following `context` (the drafter)."""

    def encode(self, text: str) -> list: ...

    def decode(self, tokens: Sequence[int]) -> str: ...

    def chat(self, messages: list, thinking: bool = True, level: str | None = None) -> list: ...


class _Ledger:
    """Accounting when the engine hands none: admits every claim."""

    class _Claim:
        def __init__(self, nbytes):
            self.nbytes = nbytes

    def claim(self, nbytes):
        return self._Claim(nbytes)

    def release(self, claim):
        pass

    def available(self):
        return 1 << 62


class _Services:
    def __init__(self):
        self.accounting = _Ledger()

    @staticmethod
    def log(level, msg):
        pass


class EngineState:
    """A sequence as the engine holds it: the layer runtime's SeqState plus
    the budget claim and the speculative bookkeeping -- `out`, tokens a round
    verified and not yet handed out (the deepest is the next forward's
    input); `drafts`, the drafter's tokens for the next round; `rb_tag`, the
    verify after which the rows past the handed ones can still be undone."""

    __slots__ = ("seq", "claim", "out", "drafts", "rb_tag")

    def __init__(self, seq: SeqState):
        self.seq = seq
        self.claim = None
        self.out: list[int] = []
        self.drafts: list[int] = []
        self.rb_tag = -1

    @property
    def tokens(self) -> list:
        return self.seq.tokens


class RocmRuntime:
    """The Runtime protocol over HybridRuntime on one MI355X."""

    def __init__(self, package: ModelPackage | None = None, *, device="cuda",
                 max_chunk: int = MAX_CHUNK, max_batch: int = MAX_BATCH) -> None:
        self._package = package
        self.device = torch.device(device)
        self.max_chunk = int(max_chunk)
        self.max_batch = int(max_batch)
        self.pkg: ModelPackage | None = None
        self.rt: HybridRuntime | None = None
        self.services = None
        self.mtp_on = False
        self.verify_tag = 0
        self.mtp_rounds = self.mtp_accept = self.mtp_reject = 0

    # -- lifecycle (sdk.py:139-142; runtime.py:576-644, 1427-1440) ----------

    def open(self, model_dir: str, services=None) -> Facts:
        self.services = services if services is not None else _Services()
        self.pkg = self._package or SyntheticPackage.from_dir(model_dir, device=self.device)
        types = tuple(self.pkg.layer_types())
        self.rt = HybridRuntime(self.pkg.weights(types, self.device), layer_types=types,
                                kv8=bool(self.pkg.kv8), device=self.device, mtp_k=MTP_K)
        self.mtp_on = False
        return Facts(cache_bytes_per_token=self.rt.n_full * 2 * self.rt.kv_row_bytes(),
                     max_batch=self.max_batch, max_context=self.rt.max_context,
                     capabilities=["speculative"], stop_tokens=list(self.pkg.stop_tokens))

    def close(self) -> None:
        self.rt = None
        self.pkg = None

    def set_speculative(self, enabled: bool = True) -> None:
        """The optional verb (runtime.py:2578-2608): speculation on or off;
        the verify checkpoints are allocated on the first switch on."""
        if enabled:
            self.rt._ensure_verify_buffers()
        self.mtp_on = bool(enabled)

    # -- text (sdk.py:160-166) ------------------------------------------------

    def encode(self, text: str) -> list:
        return list(self.pkg.encode(text))

    def decode(self, tokens: list) -> str:
        return self.pkg.decode(tokens)

    def chat(self, messages: list, thinking: bool = True, level: str | None = None) -> list:
        return list(self.pkg.chat(messages, thinking, level))

    # -- budget --------------------------------------------------------------

    def _bytes(self, cap: int) -> int:
        """What a state of KV capacity `cap` holds on the device
        (runtime.py:1150-1162's sum for these buffers)."""
        rt = self.rt
        return (rt.s_bytes + 2 * rt.conv_bytes + VOCAB_ROW * 2
                + cap * 2 * rt.n_full * rt.kv_row_bytes())

    def _reclaim(self, es: EngineState, nbytes: int) -> None:
        """One claim of `nbytes` for the state; a refusal leaves the old one."""
        acc = self.services.accounting
        old = es.claim
        if old is not None:
            acc.release(old)
            es.claim = None
        try:
            es.claim = acc.claim(nbytes)
        except BudgetRefused:
            if old is not None:
                es.claim = acc.claim(old.nbytes)
            raise

    def _grow(self, es: EngineState, need: int) -> None:
        """KV room for `need` positions on the capacity ladder, claimed first
        (runtime.py:1363-1405)."""
        seq = es.seq
        if need <= seq.cap:
            return
        if need > self.rt.max_context:
            raise ContractError(f"context {need} exceeds max_context {self.rt.max_context}")
        self._reclaim(es, self._bytes(state_blob.next_cap(need)))
        self.rt.grow(seq, need)

    # -- state verbs (sdk.py:145-157; runtime.py:1017-1060, 1221-1405) ------

    def _claimed(self, nbytes: int, make) -> EngineState:
        """A state built by `make()` under a claim of `nbytes`, taken before
        the device is asked; a failure releases it."""
        acc = self.services.accounting
        claim = acc.claim(nbytes)
        try:
            es = EngineState(make())
        except BaseException:
            acc.release(claim)
            raise
        es.claim = claim
        if es.seq.logits is None:
            es.seq.logits = torch.full((VOCAB_ROW,), -65504.0, dtype=torch.float16,
                                       device=self.device)
        return es

    def new_state(self) -> EngineState:
        return self._claimed(self._bytes(0), self.rt.new_state)

    def clone_state(self, es: EngineState) -> EngineState:
        self._live(es)
        c = self._claimed(self._bytes(es.seq.cap), lambda: self.rt.clone_state(es.seq))
        c.out, c.drafts, c.rb_tag = list(es.out), list(es.drafts), es.rb_tag
        self._unforward(c)          # a clone is what a cache keeps: nothing forwarded unhanded
        return c

    def truncate_state(self, es: EngineState, n_tokens: int) -> None:
        self._live(es)
        seq = es.seq
        if 0 <= n_tokens < seq.logical() and n_tokens == len(seq.tokens) - 1:
            self._unforward(es)     # a K = 2 round's extra row, undone for free
        below = 0 <= n_tokens < len(seq.tokens)
        try:
            self.rt.truncate_state(seq, n_tokens)
        except ValueError as e:
            raise ContractError(str(e)) from None
        if below:
            es.out, es.drafts, es.rb_tag = [], [], -1

    def state_nbytes(self, es: EngineState) -> int:
        return self.rt.state_nbytes(es.seq)

    def export_state(self, es: EngineState) -> bytes:
        self._live(es)
        return self.rt.export_state(es.seq)

    def import_state(self, blob: bytes) -> EngineState:
        cap = json.loads(blob[4:4 + int.from_bytes(blob[:4], "little")]).get("cap", 0)
        return self._claimed(self._bytes(cap), lambda: self.rt.import_state(blob))

    def free_state(self, es: EngineState) -> None:
        if es.claim is not None:
            self.services.accounting.release(es.claim)
            es.claim = None
        if es.seq.s is not None:
            self.rt.free_state(es.seq)
        es.out, es.drafts = [], []

    @staticmethod
    def _live(es: EngineState) -> None:
        if es.seq.s is None:
            raise ContractError("state was freed")

    # -- the step (sdk.py:168-169; runtime.py:1729-1767) -------------------

    def step(self, batch: Sequence, ctx) -> list:
        if len(batch) > self.max_batch:
            raise ContractError(f"batch of {len(batch)} exceeds max_batch {self.max_batch}")
        if len({id(item.state) for item in batch}) != len(batch):
            raise ContractError("a state appears more than once in one batch")
        cancelled = ctx.cancelled()
        if not cancelled:
            for item in batch:      # every state's room first: a refusal moves nothing
                need = self._need(item)
                if need:
                    self._grow(item.state, need)
        out: list = [None] * len(batch)
        rows = []
        for k, item in enumerate(batch):
            if cancelled or ctx.cancelled():
                out[k] = StepResult(None, True)
            elif self._joins_rows(item):
                rows.append(k)
            else:
                out[k] = self._step_one(item)
        if len(rows) == 1:
            out[rows[0]] = self._step_one(batch[rows[0]])
        elif rows:
            for k, res in zip(rows, self._step_rows([batch[k] for k in rows])):
                out[k] = res
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)     # step is synchronous to its caller
        return out

    def _need(self, item) -> int:
        """Positions the item's state must hold for this step, 0 when it
        forwards nothing or asks past max_context (runtime.py:1769-1781)."""
        es: EngineState = item.state
        seq = es.seq
        if seq.s is None or (self.mtp_on and es.out and not item.input_tokens):
            return 0
        n = len(seq.tokens) + (seq.pending is not None) + len(item.input_tokens)
        if n == len(seq.tokens) or n > self.rt.max_context:
            return 0
        if self.mtp_on and item.sampling is not None:
            n = min(n + 1 + self.rt.mtp_k, self.rt.max_context)
        return n

    def _joins_rows(self, item) -> bool:
        """A decode row of a batched forward (runtime.py:1783-1791)?"""
        es: EngineState = item.state
        seq = es.seq
        return (seq.s is not None and item.sampling is not None and not item.input_tokens
                and seq.pending is not None and not seq.replay
                and not (self.mtp_on and es.out)
                and len(seq.tokens) + 1 <= self.rt.max_context)

    def _forward(self, es: EngineState, tokens: list, *, verify: bool = False,
                 want: bool = False):
        """One forward of `tokens` at the state's next position; the rows'
        logits when `want`."""
        seq = es.seq
        pos0 = len(seq.tokens)
        fed = seq.fed
        proj = self.pkg.projections(tokens, list(range(pos0, pos0 + len(tokens))), self.device)
        self.rt.forward(seq, proj, tokens, verify=verify)
        seq.fed = fed
        # the state's logits row is fp16 (runtime.py:1020): every draw reads that
        return self.pkg.logits(proj).half() if want else None

    def _keep_logits(self, seq: SeqState, row: torch.Tensor) -> None:
        n = row.numel()
        seq.logits[:n].copy_(row.to(torch.float16))
        seq.has_logits = True

    def _pen_ctx(self, seq: SeqState):
        """(prompt ids, output ids): `fed` splits the forwarded tokens."""
        return list(seq.tokens[:seq.fed]), list(seq.tokens[seq.fed:])

    def _draft(self, es: EngineState, after: int) -> None:
        if self.mtp_on:
            es.drafts = list(self.pkg.draft(list(es.seq.tokens) + [after], self.rt.mtp_k))

    def _step_one(self, item) -> StepResult:
        """One sequence's step (runtime.py:1850-1966)."""
        es: EngineState = item.state
        seq = es.seq
        self._live(es)
        if self.mtp_on and es.out:
            if not item.input_tokens:       # a token a round verified earlier: no forward
                return StepResult(es.out.pop(0), False, forwarded=False)
            # a new prompt behind a queued tail: the tail was never handed out
            self._unforward(es)
            es.out, es.drafts = [], []
            seq.pending = None
        inputs = list(item.input_tokens)
        carried = seq.pending is not None
        if carried:
            inputs.insert(0, seq.pending)
        replay = list(seq.replay) if seq.replay else None
        if replay:
            inputs = replay + inputs
        pos0 = len(seq.tokens) - (len(replay) if replay else 0)
        if not inputs and item.sampling is not None and not seq.has_logits:
            raise ContractError("nothing to forward: empty step with no pending token and no "
                                "logits carried by the state")
        if pos0 + len(inputs) > self.rt.max_context:
            raise ContractError(f"state would reach {pos0 + len(inputs)} tokens, "
                                f"max_context {self.rt.max_context}")
        # a prompt feed starts a request: all that came before is prompt
        fed = len(seq.tokens) if item.input_tokens else seq.fed
        fed_add = len(item.input_tokens) + (1 if carried and item.input_tokens else 0)
        seq.pending = None
        if replay:
            self.rt.take_replay(seq)
        want_round = (self.mtp_on and item.sampling is not None and len(inputs) == 1
                      and not replay and bool(es.drafts)
                      and pos0 + 2 <= self.rt.max_context)
        have = seq.has_logits and not inputs
        if inputs and not want_round:
            self._grow(es, pos0 + len(inputs))
            for start in range(0, len(inputs), self.max_chunk):
                chunk = inputs[start:start + self.max_chunk]
                want = start + len(chunk) == len(inputs) and item.sampling is not None
                rows = self._forward(es, chunk, want=want)
                if want:
                    self._keep_logits(seq, rows[-1])
                    have = True
            seq.fed = fed + fed_add
        token, finished = None, False
        if item.sampling is not None:
            if want_round:
                token = self._round(es, item, inputs[0], pos0, fed, fed_add)
            else:
                if not have:
                    raise ContractError("no logits to sample: the step forwarded nothing")
                token = self.pkg.sample(seq.logits[:self.pkg.vocab], item.sampling,
                                        *self._pen_ctx(seq))
                if inputs:
                    self._draft(es, token)
            finished = token in self.pkg.stop_tokens
            seq.pending = es.out[-1] if es.out else token
        return StepResult(token, finished, forwarded_tokens=len(inputs))

    def _round(self, es: EngineState, item, p: int, pos0: int, fed: int, fed_add: int) -> int:
        """A speculative round (runtime.py:2033-2215): ONE verify forward of
        [p, d1(, d2)] at pos0; row r samples the token at pos0 + r + 1. The
        longest prefix of drafts the rows confirm is kept (a stop token caps
        it); the recurrence and conv state fall back to the checkpoint after
        the last kept row, the draws past it are undone, and a round that
        keeps nothing re-draws row 0's token from the round's first draw. The
        kept tokens are queued in `out`; the first is returned."""
        seq, spec, rt = es.seq, item.sampling, self.rt
        k = 2 if (len(es.drafts) >= 2 and rt.mtp_k >= 2
                  and pos0 + 3 <= rt.max_context) else 1
        drafts = es.drafts[:k]
        rows = [p] + drafts
        self._grow(es, pos0 + len(rows) + 1)
        st0 = self.pkg.sampler_state(spec)
        logits = self._forward(es, rows, verify=True, want=True)
        self.verify_tag += 1
        self.mtp_rounds += 1
        p_ids, o_ids = self._pen_ctx(seq)
        out0 = o_ids + [p]
        draws, marks = [], []
        for r in range(len(rows)):
            marks.append(self.pkg.sampler_state(spec))
            draws.append(self.pkg.sample(logits[r], spec, p_ids, out0 + draws))
        j = 0
        while j < k and draws[j] == drafts[j] and draws[j] not in self.pkg.stop_tokens:
            j += 1
        rt.accept_verify(seq, rows, j + 1)
        seq.fed = fed + fed_add
        if j == 0:
            self.mtp_reject += 1
            self.pkg.restore_sampler(spec, st0)
            token = self.pkg.sample(logits[0], spec, *self._pen_ctx(seq))
            self._keep_logits(seq, logits[0])
            es.out = [token]
        else:
            self.mtp_accept += 1
            if j + 1 < len(rows):
                self.pkg.restore_sampler(spec, marks[j + 1])
            self._keep_logits(seq, logits[j])
            es.out = draws[:j + 1]
            es.rb_tag = self.verify_tag if j == 2 else -1
        self._draft(es, es.out[-1])
        return es.out.pop(0)

    def _unforward(self, es: EngineState) -> bool:
        """Undo the row a K = 2 round forwarded ahead of the engine
        (runtime.py:2217-2246): while two of its tokens wait and no verify has
        run since, the checkpoint after row 1 and the other conv buffer are
        the state without it, and that row's token becomes the pending one."""
        seq, rt = es.seq, self.rt
        if (len(es.out) < 2 or es.rb_tag != self.verify_tag or rt.snap_s is None
                or not seq.tokens):
            return False
        seq.s.copy_(rt.snap_s[1])
        seq.phase ^= 1
        seq.pending = seq.tokens[-1]
        seq.tokens = seq.tokens[:-1]
        seq.fed = min(seq.fed, len(seq.tokens))
        es.out, es.drafts, es.rb_tag = [], [], -1
        return True

    def _step_rows(self, items) -> list:
        """One token for each of several sequences from one batched forward of
        their pending tokens (runtime.py:1793-1838); batched rows do not
        speculate."""
        states = [item.state for item in items]
        for es in states:
            self._live(es)
            self._grow(es, len(es.seq.tokens) + 1)
        seqs = [es.seq for es in states]
        tokens = [s.pending for s in seqs]
        fed = [s.fed for s in seqs]
        pos = [len(s.tokens) for s in seqs]
        proj = self.pkg.projections(tokens, pos, self.device)
        self.rt.forward_batch(seqs, proj, tokens)
        logits = self.pkg.logits(proj).half()
        out = []
        for r, (item, es) in enumerate(zip(items, states)):
            seq = es.seq
            seq.fed = fed[r]
            self._keep_logits(seq, logits[r])
            token = self.pkg.sample(logits[r], item.sampling, *self._pen_ctx(seq))
            seq.pending = token
            es.drafts = []
            out.append(StepResult(token, token in self.pkg.stop_tokens, forwarded_tokens=1))
        return out


def create(package: ModelPackage | None = None, **kw) -> RocmRuntime:
    """runtime.py:3999-4002: the backend object the engine opens."""
    return RocmRuntime(package, **kw)


# ---------------------------------------------------------------------------
# A seeded stand-in for the model package
# ---------------------------------------------------------------------------

class _SynthProj:
    """Projections of one forward: a row's inputs are a function of its
    (token, position) only -- a token table plus a position table, rotated by
    a per-layer amount -- so the same row gets the same inputs however the
    rows are grouped (sub-chunks, a verify, a batch)."""

    def __init__(self, pkg: "SyntheticPackage", tokens, positions, device):
        self.tokens = [int(t) for t in tokens]
        self.positions = [int(q) for q in positions]
        t = torch.as_tensor(self.tokens, dtype=torch.long, device=device)
        p = torch.as_tensor([q % pkg.n_pos for q in self.positions], dtype=torch.long,
                            device=device)
        self.base = pkg.tok_table[t] + pkg.pos_table[p]
        self.out: dict[int, torch.Tensor] = {}

    def _row(self, layer: int) -> torch.Tensor:
        return torch.roll(self.base, shifts=997 * (layer + 1), dims=1)

    def full_attn_in(self, layer, T):
        x = self._row(layer)
        return (x[:, :12288].reshape(T, 24, 512).contiguous(),
                x[:, 12288:13312].reshape(T, 4, 256).contiguous(),
                x[:, 13312:14336].reshape(T, 4, 256).contiguous())

    def gdn_in(self, layer, T):
        x = self._row(layer)
        return (x[:, :10240].contiguous(),
                (x[:, 10240:16384] * 2).reshape(T, 48, 128).contiguous(),
                x[:, 16384:16432].float().contiguous(),
                x[:, 16432:16480].float().contiguous())

    def layer_out(self, layer, out):
        self.out[layer] = out


class SyntheticPackage:
    """Seeded weights, projections, an LM head, a sampler, a byte tokenizer
    and a drafter of the model's shapes, standing in for the model package.

    The head reads the last full-attention and the last GDN layer's outputs
    through a random projection and adds a large bias on one token, a fixed
    function of the row's (token, position) -- `successor` -- so greedy
    decoding follows a known chain while the logits still carry every layer's
    arithmetic. The drafter proposes that chain, except where `draft_fn`
    (given (context, n, truth)) says otherwise: tests make it propose wrong
    tokens to drive rejections."""

    D = 16480
    n_pos = 61

    def __init__(self, *, seed: int = 0, vocab: int = 256, layer_types=LAYER_TYPES,
                 kv8: bool = True, device="cuda", stop_tokens=(0,), draft_fn=None) -> None:
        self.seed, self.vocab, self.kv8 = seed, vocab, kv8
        self.types = tuple(layer_types)
        self.stop_tokens = list(stop_tokens)
        self.draft_fn = draft_fn
        g = torch.Generator().manual_seed(seed + 1)
        self.tok_table = torch.randn((vocab, self.D), generator=g).half().to(device)
        self.pos_table = (torch.randn((self.n_pos, self.D), generator=g) * 0.5).half().to(device)
        self.last_full = max(i for i, t in enumerate(self.types) if t == "full_attention")
        self.last_gdn = max(i for i, t in enumerate(self.types) if t != "full_attention")
        self.head_full = (torch.randn((24 * 256, vocab), generator=g) / 80).to(device)
        self.head_gdn = (torch.randn((48 * 128, vocab), generator=g) / 80).to(device)
        self._rngs: dict = {}

    @classmethod
    def from_dir(cls, model_dir, device="cuda") -> "SyntheticPackage":
        """Layer schedule and KV format from the package's config.json
        (text_config.layer_types, kv_cache "int8" | "fp16") when present."""
        kw = {}
        path = Path(model_dir) / "config.json" if model_dir else None
        if path is not None and path.is_file():
            cfg = json.loads(path.read_text())
            tc = cfg.get("text_config", cfg)
            if "layer_types" in tc:
                kw["layer_types"] = tuple(tc["layer_types"])
            if "kv_cache" in cfg:
                kw["kv8"] = cfg["kv_cache"] == "int8"
            if "seed" in cfg:
                kw["seed"] = int(cfg["seed"])
        return cls(device=device, **kw)

    def layer_types(self):
        return self.types

    def weights(self, layer_types, device):
        return random_weights(layer_types, seed=self.seed, device=device)

    def projections(self, tokens, positions, device):
        return _SynthProj(self, tokens, positions, device)

    def successor(self, token: int, pos: int) -> int:
        return (token * 31 + pos * 7) % (self.vocab - 1) + 1

    def logits(self, proj: _SynthProj) -> torch.Tensor:
        T = len(proj.tokens)
        zf = proj.out[self.last_full].float().reshape(T, -1)
        yg = proj.out[self.last_gdn].float().reshape(T, -1)
        lg = zf @ self.head_full + yg @ self.head_gdn
        succ = [self.successor(t, q) for t, q in zip(proj.tokens, proj.positions)]
        lg[torch.arange(T, device=lg.device), torch.as_tensor(succ, device=lg.device)] += 30.0
        return lg

    def _rng(self, spec) -> np.random.Generator:
        key = getattr(spec, "seed", None)
        if key not in self._rngs:
            self._rngs[key] = np.random.default_rng(0 if key is None else key)
        return self._rngs[key]

    def sample(self, row, spec, prompt_ids, output_ids) -> int:
        x = row.detach().float().cpu().numpy()[:self.vocab].astype(np.float64)
        temp = float(getattr(spec, "temperature", 0.0))
        if temp <= 0:
            return int(np.argmax(x))
        top_k = int(getattr(spec, "top_k", 0)) or self.vocab
        idx = np.argsort(-x)[:top_k]
        w = np.exp((x[idx] - x[idx[0]]) / temp)
        return int(idx[self._rng(spec).choice(len(idx), p=w / w.sum())])

    def sampler_state(self, spec):
        return self._rng(spec).bit_generator.state

    def restore_sampler(self, spec, state) -> None:
        self._rng(spec).bit_generator.state = state

    def draft(self, context, n):
        pos = len(context) - 1
        truth, tok = [], context[-1]
        for i in range(n):
            tok = self.successor(tok, pos + i)
            truth.append(tok)
        return list(self.draft_fn(list(context), n, truth)) if self.draft_fn else truth

    def encode(self, text: str) -> list:
        return list(text.encode("utf-8"))

    def decode(self, tokens) -> str:
        return bytes(int(t) for t in tokens if 0 < int(t) < 256).decode("utf-8", errors="replace")

    def chat(self, messages, thinking: bool = True, level=None) -> list:
        text = "".join(f"<{m['role']}>{m['content']}\n" for m in messages) + "<assistant>"
        return self.encode(text)
