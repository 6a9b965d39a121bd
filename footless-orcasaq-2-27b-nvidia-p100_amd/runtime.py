"""Layer-level runtime over libfl355: the reference backend's per-sequence
device state and its full-attention / Gated DeltaNet layer steps
(model/footless/cuda_sm60/runtime.py), on one MI355X.

Covered (reference line ranges):

* a sequence's device state (`_State`, runtime.py:459-501): the recurrent
  state of every GDN layer, the conv ring ping-pong and its phase, one K and
  one V buffer per full-attention layer grown on the capacity ladder
  (`_grow` 1363-1405, `_next_cap` 1209-1219), fp16 or the int8 format;
* the state verbs `new_state`, `clone_state`, `truncate_state`,
  `state_nbytes`, `export_state`, `import_state`, `free_state`
  (1017-1060, 1221-1335; the engine's names, `sdk.py:136-186`);
* the layer steps over the projections a caller hands in: `_full_attn`
  (2780-2863: q / k norm, RoPE and KV store, decode / verify or prefill
  attention, the sigmoid gate) and `_gdn` (2961-3112: causal conv, the fused
  decode or verify step with its per-row checkpoints, the chunked prefill
  scan, the gated output norm);
* the batched decode of several sequences (`_full_attn_rows`, `_gdn_rows`,
  2865-2878 / 3114-3146): one attention launch and one GDN launch a layer for
  every sequence;
* the MTP verify round's keep-or-roll-back of the recurrent and conv state
  (`_mtp_round`, `_mtp_round2`, 2033-2246).

Not covered: the embedding, the EXL3 trellis projections and the MLP between
the layers, the LM head, the sampler and the tokenizer -- the backend's other
kernels, outside this hot path. `forward` takes each layer's projections from
a `Projections` object and hands the layer's output back to it: the seam where
those kernels plug in.

Every layer step runs the HIP kernels of libfl355 through `ops`; this module
only owns buffers and the order of the calls.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Protocol, Sequence

import torch

from . import ops, state_blob
from .geometry import (DEC_SPLIT_ROWS, GDN_K, GDN_K_HEADS, GDN_V, GDN_V_HEADS, HEAD_DIM,
                       N_KV, QKV_ROWS, SPLIT_T_MAX, kv8_nbytes)

F16, F32 = torch.float16, torch.float32

N_LAYERS = 64
# The package's layer schedule (config.json `layer_types`, read at
# runtime.py:654-665): every fourth layer is full attention, the rest GDN.
LAYER_TYPES = tuple("full_attention" if (i + 1) % 4 == 0 else "linear_attention"
                    for i in range(N_LAYERS))
MAX_CONTEXT = state_blob.MAX_CONTEXT
MTP_K = 2            # drafts a verify round carries: rows T = MTP_K + 1


class Projections(Protocol):
    """Where the layers' inputs come from and their outputs go (the EXL3
    projections, norms and MLP of the reference sit behind this)."""

    def full_attn_in(self, layer: int, T: int):
        """(qg [T, 24, 512], k [T, 4, 256], v [T, 4, 256]) fp16 for layer `layer`:
        the q | gate, k and v projections of its T rows."""

    def gdn_in(self, layer: int, T: int):
        """(qkv [T, 10240] fp16, z [T, 48, 128] fp16, a [T, 48] f32, b [T, 48] f32):
        the q|k|v row, the output gate and the two gate logits."""

    def layer_out(self, layer: int, out: torch.Tensor) -> None:
        """The layer's result: z [T, 24, 256] (attention, gated) or
        yn [T, 48, 128] (GDN, normed), fp16."""


@dataclass
class FullWeights:
    """One full-attention layer's weights on the hot path: the Gemma RMSNorm
    gammas of q and k (fp32 [256], applied as 1 + w)."""
    q_norm: torch.Tensor
    k_norm: torch.Tensor


@dataclass
class GdnWeights:
    """One GDN layer's weights on the hot path: the depthwise conv taps
    (fp16 [10240, 4], tap 0 oldest), A_log and dt_bias (fp32 [48]) and the
    output norm's gamma (fp32 [128])."""
    conv_w: torch.Tensor
    A_log: torch.Tensor
    dt_bias: torch.Tensor
    norm_w: torch.Tensor


class SeqState:
    """One sequence's cache. `tokens` are the positions the KV cache and the
    recurrences cover; `replay` a prefix the recurrence no longer matches
    after a truncate (re-forwarded from position 0 by the next prefill)."""

    __slots__ = ("tokens", "fed", "pending", "replay", "s", "conv", "phase", "kk", "kv",
                 "lcap", "cap", "logits", "has_logits")

    def __init__(self) -> None:
        self.tokens: list[int] = []
        self.fed = 0
        self.pending: int | None = None
        self.replay: list[int] | None = None
        self.s: torch.Tensor | None = None        # [G, 48, 128, 128] f32
        self.conv: torch.Tensor | None = None     # [2, G, 10240, 3] f16, ping-pong
        self.phase = 0
        self.kk: list[torch.Tensor] | None = None
        self.kv: list[torch.Tensor] | None = None
        self.lcap: list[int] | None = None
        self.cap = 0
        self.logits: torch.Tensor | None = None
        self.has_logits = False

    def logical(self) -> int:
        return len(self.tokens) + (1 if self.pending is not None else 0)


class HybridRuntime:
    """The hot-path half of a ROCm backend for the hybrid model.

    layer_types: the schedule (full attention or linear attention a layer);
    weights: per layer index, FullWeights or GdnWeights; kv8: the int8 KV
    format (the reference's shipped default) instead of fp16; split_rows: the
    decode attention's split rule (0: sized to the grid, so a sequence's
    attention values in a batch may differ in the last bits from its own
    single step's; > 0: the length-only rule, batched == single bit for bit)."""

    def __init__(self, weights: dict, *, layer_types: Sequence[str] = LAYER_TYPES,
                 kv8: bool = False, device="cuda", max_context: int = MAX_CONTEXT,
                 mtp_k: int = MTP_K, split_rows: int = DEC_SPLIT_ROWS) -> None:
        self.split_rows = split_rows
        self.layer_types = tuple(layer_types)
        self.full_ord = {i: k for k, i in enumerate(
            j for j, t in enumerate(self.layer_types) if t == "full_attention")}
        self.gdn_ord = {i: k for k, i in enumerate(
            j for j, t in enumerate(self.layer_types) if t != "full_attention")}
        for i in range(len(self.layer_types)):
            want = FullWeights if i in self.full_ord else GdnWeights
            if not isinstance(weights.get(i), want):
                raise ValueError(f"layer {i} needs {want.__name__}")
        self.w = weights
        self.kv8 = kv8
        self.device = torch.device(device)
        self.max_context = max_context
        self.mtp_k = mtp_k
        self.n_gdn = len(self.gdn_ord)
        self.n_full = len(self.full_ord)
        # verify checkpoints of every GDN layer (the state after rows 0 ..
        # mtp_k - 1) and the spare conv buffer of the last row: per runtime,
        # as the reference's snap_s / snap_c (runtime.py:2600-2605)
        self.snap_s = None
        self.snap_c = None
        self.verify_T = 0
        self._verify_pos0 = -1

    # -- sizes ---------------------------------------------------------------

    @property
    def layer_s_elems(self) -> int:
        return GDN_V_HEADS * GDN_V * GDN_K

    @property
    def s_bytes(self) -> int:
        return self.n_gdn * self.layer_s_elems * 4

    @property
    def conv_bytes(self) -> int:
        return self.n_gdn * QKV_ROWS * 3 * 2

    def kv_row_bytes(self) -> int:
        return state_blob.kv_row_bytes(self.kv8)

    # -- state verbs ---------------------------------------------------------

    def new_state(self) -> SeqState:
        st = SeqState()
        st.s = torch.zeros((self.n_gdn, GDN_V_HEADS, GDN_V, GDN_K), dtype=F32,
                           device=self.device)
        st.conv = torch.zeros((2, self.n_gdn, QKV_ROWS, 3), dtype=F16, device=self.device)
        return st

    def _kv_buffer(self, cap: int) -> torch.Tensor:
        if self.kv8:
            return torch.zeros(kv8_nbytes(cap), dtype=torch.int8, device=self.device)
        return torch.zeros((cap, N_KV, HEAD_DIM), dtype=F16, device=self.device)

    def _kv_copy(self, dst: torch.Tensor, dst_cap: int, src: torch.Tensor, src_cap: int,
                 rows: int) -> None:
        """The first `rows` positions of a layer's K (or V) buffer into one of
        another capacity; int8 buffers move their values and their block
        scales as two regions (runtime.py:1184-1194)."""
        if not self.kv8:
            dst[:rows].copy_(src[:rows])
            return
        vals = N_KV * HEAD_DIM
        dst[:rows * vals].copy_(src[:rows * vals])
        srow = self.kv_row_bytes() - vals
        dst[dst_cap * vals:dst_cap * vals + rows * srow].copy_(
            src[src_cap * vals:src_cap * vals + rows * srow])

    def grow(self, st: SeqState, need: int) -> None:
        """Room for `need` positions in every full-attention layer, on the
        reference's ladder; a layer's rows move to its new buffers."""
        if need <= st.cap:
            return
        if need > self.max_context:
            raise ValueError(f"context {need} exceeds max_context {self.max_context}")
        cap = state_blob.next_cap(need)
        if st.kk is None:
            st.kk, st.kv, st.lcap = [None] * self.n_full, [None] * self.n_full, [0] * self.n_full
        for li in range(self.n_full):
            old = st.lcap[li]
            if old >= cap:
                continue
            k, v = self._kv_buffer(cap), self._kv_buffer(cap)
            if old:
                self._kv_copy(k, cap, st.kk[li], old, old)
                self._kv_copy(v, cap, st.kv[li], old, old)
            st.kk[li], st.kv[li], st.lcap[li] = k, v, cap
        st.cap = min(st.lcap) if st.lcap else cap   # a schedule without attention layers

    def clone_state(self, st: SeqState) -> SeqState:
        c = SeqState()
        c.tokens = list(st.tokens)
        c.fed = st.fed
        c.pending = st.pending
        c.replay = None if st.replay is None else list(st.replay)
        c.phase = st.phase
        c.s = st.s.clone()
        c.conv = st.conv.clone()
        c.has_logits = st.has_logits
        c.logits = None if st.logits is None else st.logits.clone()
        if st.kk is not None:
            c.kk = [b.clone() for b in st.kk]
            c.kv = [b.clone() for b in st.kv]
            c.lcap = list(st.lcap)
            c.cap = st.cap
        return c

    def truncate_state(self, st: SeqState, n_tokens: int) -> None:
        """Keep the first n_tokens as a fresh state fed them would: the KV
        cache shrinks for free (position-addressable); the recurrences cannot
        drop a tail, so below the cached count they are zeroed and the kept
        ids recorded as a replay (runtime.py:1221-1262)."""
        if n_tokens < 0:
            raise ValueError(f"truncate to a negative count {n_tokens}")
        if n_tokens >= st.logical():
            st.fed = len(st.tokens)
            return
        if n_tokens == len(st.tokens):
            st.pending = None
            st.fed = n_tokens
            return
        st.replay = list(st.tokens[:n_tokens]) or None
        st.tokens = st.tokens[:n_tokens]
        st.fed = n_tokens
        st.pending = None
        st.has_logits = False
        st.s.zero_()
        st.conv.zero_()

    def state_nbytes(self, st: SeqState) -> int:
        return (self.s_bytes + 2 * self.conv_bytes
                + st.cap * 2 * self.n_full * self.kv_row_bytes())

    def export_state(self, st: SeqState) -> bytes:
        """The reference's blob (runtime.py:1267-1296); the model's geometry
        (48 GDN, 16 full-attention layers) only, as the format fixes it."""
        self._check_model_geometry()
        meta = {"tokens": st.tokens, "fed": st.fed, "pending": st.pending,
                "replay": st.replay, "phase": st.phase}
        return state_blob.export_state(meta, st.s, (st.conv[0], st.conv[1]),
                                       st.logits if st.has_logits else None,
                                       st.kk or (), st.kv or (), st.lcap or (), st.cap, self.kv8)

    def import_state(self, blob: bytes) -> SeqState:
        self._check_model_geometry()
        d = state_blob.import_state(blob, self.device, self.kv8)
        st = SeqState()
        m = d["meta"]
        st.tokens, st.fed, st.pending = list(m["tokens"]), m["fed"], m["pending"]
        st.replay, st.phase = m["replay"], m["phase"]
        st.s = d["S"].contiguous()
        st.conv = torch.stack(list(d["conv"])).contiguous()
        st.logits = d["logits"]
        st.has_logits = d["logits"] is not None
        if d["cap"]:
            as_kv = (lambda t: t.view(torch.int8)) if self.kv8 else (lambda t: t)
            st.kk, st.kv = [as_kv(t) for t in d["kk"]], [as_kv(t) for t in d["kv"]]
            st.lcap = [d["cap"]] * self.n_full
            st.cap = d["cap"]
        return st

    def free_state(self, st: SeqState) -> None:
        st.s = st.conv = st.logits = None
        st.kk = st.kv = st.lcap = None
        st.cap = 0
        st.tokens = []

    def _check_model_geometry(self) -> None:
        if self.n_gdn != state_blob.GDN_LAYERS or self.n_full != state_blob.FULL_LAYERS:
            raise ValueError("the state blob format is the model's: 48 GDN and 16 "
                             "full-attention layers")

    # -- layer steps ---------------------------------------------------------

    def _full_attn(self, st: SeqState, i: int, qg, k, v, T: int, pos0: int) -> torch.Tensor:
        """runtime.py:2780-2863 for one sequence: prep (norms, RoPE, KV store)
        then the decode / verify attention (T <= SPLIT_T_MAX, every row the
        T = 1 call's at its position) or the causal prefill, gated."""
        li = self.full_ord[i]
        wt = self.w[i]
        kc, vc, lcap = st.kk[li], st.kv[li], st.lcap[li]
        if self.kv8:
            ops.attn_prep_q8(qg, k, v, wt.q_norm, wt.k_norm, kc, vc, pos0=pos0, max_pos=lcap, T=T)
        else:
            ops.attn_prep(qg, k, v, wt.q_norm, wt.k_norm, kc, vc, pos0=pos0, T=T)
        if T <= SPLIT_T_MAX:
            if self.kv8:
                return ops.attn_decode_q8(qg[None], [kc], [vc], [pos0], [lcap],
                                          split_rows=self.split_rows)[0]
            return ops.attn_decode(qg[None], [kc], [vc], [pos0], split_rows=self.split_rows)[0]
        # gated by the gate half of each head's q | gate row (in the merge when
        # the KV is split)
        if self.kv8:
            return ops.attention_prefill_q8(qg, kc, vc, pos0=pos0, max_pos=lcap, gated=True)
        return ops.attention_prefill(qg, kc, vc, pos0=pos0, gated=True)

    def _gdn(self, st: SeqState, i: int, qkv, zg, a, b, T: int, pos0: int,
             verify: bool) -> torch.Tensor:
        """runtime.py:2961-3112 for one sequence. Decode (T = 1): one launch
        runs the conv (conv[phase] -> conv[phase ^ 1]), the fused step and the
        gated output norm. Verify (T <= 1 + mtp_k): the conv rows leave row
        0's state in place in conv[phase], row 1's in conv[phase ^ 1], row 2's
        in the spare; the fused step keeps the recurrent state after each row
        but the last as a checkpoint; then the gated output norm. Prefill:
        conv over the chunk, the q / k L2 norm, the chunked WY scan with the
        gates, then the gated output norm."""
        g = self.gdn_ord[i]
        wt = self.w[i]
        S = st.s[g]
        cin, cout = st.conv[st.phase, g], st.conv[st.phase ^ 1, g]
        if T == 1 and not verify:   # the step and its output norm, one launch
            return ops.gdn_decode_normed(qkv, [S], a, b, wt.A_log, wt.dt_bias, zg, wt.norm_w,
                                         pos0s=[pos0], conv_w=wt.conv_w, cst_in=[cin],
                                         cst_out=[cout]).view(1, GDN_V_HEADS, GDN_V)
        c = torch.empty_like(qkv)
        if verify:
            # the one-launch step + norm gives one sequence's rows 48 workgroups
            # (a v head each): slower here than the 192 of the step alone
            ops.conv1d_causal_rows(qkv, wt.conv_w, cin, c, cin, cout, self.snap_c[g], T=T,
                                   pos0=pos0)
            y = ops.gdn_decode(c[None], [S], a[None], b[None], wt.A_log, wt.dt_bias, T=T,
                               pos0s=[pos0], ck=[self.snap_s[0, g]],
                               ck_step=self.n_gdn * self.layer_s_elems)[0]
            return ops.rmsnorm_gated(y.view(T, GDN_V_HEADS, GDN_V), zg, wt.norm_w, T=T)
        ops.conv1d_causal(qkv, wt.conv_w, cin, c, cout, T=T, pos0=pos0)
        # the L2 norm of the q and k head rows (the reference launches it over
        # all 80 head-sized rows of the conv'd row, runtime.py:3070, and reads
        # back only these 32: the same bits for them)
        ln = torch.empty_like(c)
        ops.l2norm_scaled_strided(c, ln, rows=2 * GDN_K_HEADS, token_stride=QKV_ROWS, T=T)
        # the gates formed from a, b inside the scan (gdn_scalars' values)
        qn, kn = GDN_K_HEADS * GDN_K, 2 * GDN_K_HEADS * GDN_K
        y = ops.gdn_prefill_chunked_logits(ln[:, :qn], ln[:, qn:kn], c[:, kn:], a, b, wt.A_log,
                                           wt.dt_bias, S, T=T)
        return ops.rmsnorm_gated(y.view(T, GDN_V_HEADS, GDN_V), zg, wt.norm_w, T=T)

    def _ensure_verify_buffers(self) -> None:
        if self.snap_s is None:
            self.snap_s = torch.empty((max(1, self.mtp_k), self.n_gdn, GDN_V_HEADS, GDN_V, GDN_K),
                                      dtype=F32, device=self.device)
            self.snap_c = torch.empty((self.n_gdn, QKV_ROWS, 3), dtype=F16, device=self.device)

    def forward(self, st: SeqState, proj: Projections, tokens: Sequence[int],
                verify: bool = False) -> None:
        """One forward of `tokens` (their ids are bookkeeping here; the
        projections stand for their embedding) through every layer, at the
        state's next position. A plain step appends them and flips the conv
        phase; a verify (2 <= T <= 1 + mtp_k) leaves both to accept_verify."""
        T = len(tokens)
        if T < 1:
            raise ValueError("forward of no tokens")
        if st.replay:
            raise ValueError("the state holds a replay: forward the replayed prefix first "
                             "(take_replay)")
        pos0 = len(st.tokens)
        if verify:
            if not 2 <= T <= 1 + self.mtp_k:
                raise ValueError(f"a verify carries 2..{1 + self.mtp_k} rows")
            self._ensure_verify_buffers()
        self.grow(st, pos0 + T)
        for i, kind in enumerate(self.layer_types):
            if kind == "full_attention":
                qg, k, v = proj.full_attn_in(i, T)
                out = self._full_attn(st, i, qg, k, v, T, pos0)
            else:
                qkv, zg, a, b = proj.gdn_in(i, T)
                out = self._gdn(st, i, qkv, zg, a, b, T, pos0, verify)
            proj.layer_out(i, out)
        if verify:
            self.verify_T, self._verify_pos0 = T, pos0
            return
        st.tokens.extend(int(t) for t in tokens)
        st.fed = len(st.tokens)
        st.phase ^= 1

    def accept_verify(self, st: SeqState, tokens: Sequence[int], kept: int) -> None:
        """Keep the first `kept` rows (1 <= kept <= T) of the verify forward
        just run on `st` (runtime.py:2105-2130 for T = 2, 2181-2215 for T = 3):
        all kept -- the recurrence is already final, the conv state after the
        last row is adopted (T = 2: the other phase buffer; T = 3: the spare);
        kept = 2 of 3 -- the checkpoint after row 1 and the other phase
        buffer; kept = 1 -- the checkpoint after row 0, and row 0's conv state
        already sits in conv[phase]. KV rows past the kept ones are dead."""
        T = self.verify_T
        if T == 0 or len(st.tokens) != self._verify_pos0 or len(tokens) != T:
            raise ValueError("accept_verify follows a verify forward of the same rows")
        if not 1 <= kept <= T:
            raise ValueError(f"kept must be in 1..{T}")
        if kept < T:
            st.s.copy_(self.snap_s[kept - 1])
        if kept == T and T == 3:
            st.conv[st.phase].copy_(self.snap_c)
        elif kept == 2:
            st.phase ^= 1
        st.tokens.extend(int(t) for t in tokens[:kept])
        st.fed = len(st.tokens)
        self.verify_T = 0

    def take_replay(self, st: SeqState) -> list[int]:
        """The prefix a truncate left to re-forward (then forward it as a
        prefill from position 0), clearing the mark."""
        r = st.replay or []
        st.replay = None
        st.tokens = []
        st.fed = 0
        return r

    # -- batched decode --------------------------------------------------------

    def forward_batch(self, states: Sequence[SeqState], proj: Projections,
                      tokens: Sequence[int]) -> None:
        """One decode step of several sequences (one token each), as
        `_step_rows` runs it: per full-attention layer one launch of every
        row's prep into its own cache, then one attention launch over all
        rows; per GDN layer one fused conv + delta-rule + output-norm launch
        over all rows. `proj` hands the B rows stacked ([B, ...] where
        forward takes [T, ...])."""
        B = len(states)
        if B != len(tokens) or B < 1:
            raise ValueError("one token a sequence")
        pos0s = []
        for st in states:
            if st.replay:
                raise ValueError("a state holds a replay")
            pos0s.append(len(st.tokens))
            self.grow(st, len(st.tokens) + 1)
        for i, kind in enumerate(self.layer_types):
            if kind == "full_attention":
                li, wt = self.full_ord[i], self.w[i]
                qg, k, v = proj.full_attn_in(i, B)
                kcs = [st.kk[li] for st in states]
                vcs = [st.kv[li] for st in states]
                # every row's prep into its own cache, one launch (the same values
                # as a prep a row)
                ops.attn_prep_rows(qg, k, v, wt.q_norm, wt.k_norm, kcs, vcs, pos0s,
                                   [st.lcap[li] for st in states], kv8=self.kv8)
                if self.kv8:
                    z = ops.attn_decode_q8(qg[:, None], kcs, vcs, pos0s,
                                           [st.lcap[li] for st in states],
                                           split_rows=self.split_rows)
                else:
                    z = ops.attn_decode(qg[:, None], kcs, vcs, pos0s, split_rows=self.split_rows)
                proj.layer_out(i, z[:, 0])
            else:
                g, wt = self.gdn_ord[i], self.w[i]
                qkv, zg, a, b = proj.gdn_in(i, B)
                yn = ops.gdn_decode_normed(qkv, [st.s[g] for st in states], a, b, wt.A_log,
                                           wt.dt_bias, zg, wt.norm_w, pos0s=pos0s,
                                           conv_w=wt.conv_w,
                                           cst_in=[st.conv[st.phase, g] for st in states],
                                           cst_out=[st.conv[st.phase ^ 1, g] for st in states])
                proj.layer_out(i, yn.view(B, GDN_V_HEADS, GDN_V))
        for st, t in zip(states, tokens):
            st.tokens.append(int(t))
            st.fed = len(st.tokens)
            st.phase ^= 1


# The engine-facing verbs of the Runtime protocol (footless/sdk.py:172-186)
# that this module implements; open / close / encode / decode / chat / step
# bind the model package, tokenizer and sampler, outside the hot path.
STATE_VERBS = ("new_state", "clone_state", "truncate_state", "state_nbytes", "export_state",
               "import_state", "free_state")


def random_weights(layer_types: Sequence[str] = LAYER_TYPES, *, seed: int = 0,
                   device="cuda") -> dict:
    """Synthetic layer weights of the model's shapes (there is no checkpoint
    to load here): norm gammas ~ N(0, 0.1), conv taps ~ N(0, 0.5), A_log and
    dt_bias ~ N(0, 0.3)."""
    g = torch.Generator().manual_seed(seed)
    out = {}
    for i, t in enumerate(layer_types):
        if t == "full_attention":
            out[i] = FullWeights((torch.randn(HEAD_DIM, generator=g) * 0.1).to(device),
                                 (torch.randn(HEAD_DIM, generator=g) * 0.1).to(device))
        else:
            out[i] = GdnWeights((torch.randn((QKV_ROWS, 4), generator=g) * 0.5).half().to(device),
                                (torch.randn(GDN_V_HEADS, generator=g) * 0.3).to(device),
                                (torch.randn(GDN_V_HEADS, generator=g) * 0.3).to(device),
                                (1 + torch.randn(GDN_V, generator=g) * 0.2).to(device))
    return out
