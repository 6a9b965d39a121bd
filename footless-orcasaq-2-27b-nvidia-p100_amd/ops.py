"""The hot-path op surface over libfl355 (PyTorch-ROCm tensors in, HIP kernels out).

Each function carries the name of the reference kernel it replaces and that
kernel's argument meaning (model/footless/cuda_sm60/kernels.cu); the grid the
reference's host computed (runtime.py) becomes the `T` / `split` arguments.
Buffers are torch tensors on the current HIP device; launches go on torch's
current stream. Views into a larger row buffer (q / k / v inside the
10240-wide q|k|v row, q inside the q|gate row) are passed as tensors whose
data pointer is the view's start, with the row stride given explicitly, as
the reference passed an offset pointer and a stride.

Errors: where a reference kernel returned without writing on a geometry it
does not handle (kernels.cu:22-28), these raise ValueError before anything
is launched. Every tensor's storage is checked to cover the rows the kernel
will touch.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .geometry import (ATTN_SCALE, DEC_SMAX, DEC_SPLIT_ROWS, DEC_TMIN, GATE_OFF, GDN_CHUNK,
                       GDN_GROUP, GDN_K, GDN_K_HEADS, GDN_NORM_EPS, GDN_V, GDN_V_HEADS, HEAD_DIM,
                       L2_EPS, LOG2E, N_HEADS, N_KV, NORM_EPS, Q_PITCH, Q_SCALE, QKV_ROWS, ROPE_DIM,
                       ROPE_THETA, SPLIT_MAX, SPLIT_ROWS, kv8_nbytes)

F16, F32, I8 = torch.float16, torch.float32, torch.int8


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor | None, dtype, name: str, span: int = 0):
    """Device pointer of `t` after checking dtype / device and that its
    storage holds `span` elements from its start."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if t.device.type != "cuda":
        raise ValueError(f"{name}: must be a GPU tensor (got {t.device})")
    if span:
        st = t.untyped_storage()
        have = (st.nbytes() - (t.data_ptr() - st.data_ptr())) // t.element_size()
        if have < span:
            raise ValueError(f"{name}: storage holds {have} elements from its start, "
                             f"the call touches {span}")
    return t.data_ptr()


def _contig(t: torch.Tensor, name: str):
    if not t.is_contiguous():
        raise ValueError(f"{name}: must be contiguous")


# ---------------------------------------------------------------------------
# full attention
# ---------------------------------------------------------------------------

def kv_store(k, v, kcache, vcache, *, layer: int = 0, pos0: int, T: int | None = None,
             n_kv_heads: int = N_KV, head_dim: int = HEAD_DIM, max_pos: int | None = None):
    """kernels.cu:465-484 (runtime.py:2813-2815): k, v [T, n_kv, head_dim] fp16
    into rows pos0.. of kcache / vcache [layers?, max_pos, n_kv, head_dim]."""
    T = k.shape[0] if T is None else T
    max_pos = kcache.shape[-3] if max_pos is None else max_pos
    row = n_kv_heads * head_dim
    _contig(k, "k"), _contig(v, "v"), _contig(kcache, "kcache"), _contig(vcache, "vcache")
    _lib.call("fl_kv_store", _ptr(k, F16, "k", T * row), _ptr(v, F16, "v", T * row),
              _ptr(kcache, F16, "kcache", (layer + 1) * max_pos * row),
              _ptr(vcache, F16, "vcache", (layer + 1) * max_pos * row),
              layer, pos0, T, n_kv_heads, head_dim, max_pos, _stream())


def rmsnorm1p(x, w, y=None, *, rows: int, pitch: int, T: int | None = None, n: int = HEAD_DIM,
              eps: float = NORM_EPS):
    """kernels.cu:241-272 (runtime.py:2797-2801): per-row Gemma RMSNorm of
    [T, rows] rows `pitch` halves apart (q inside the q|gate buffer: rows =
    n_q_heads, pitch = 512), weight w [n] fp32; y = x (in place) by default."""
    T = x.shape[0] if T is None else T
    y = x if y is None else y
    span = T * rows * pitch
    _lib.call("fl_rmsnorm1p", _ptr(x, F16, "x", span), _ptr(w, F32, "w", n),
              _ptr(y, F16, "y", span), n, rows, pitch, T, float(eps), _stream())
    return y


def rope_partial(q, k, *, pos0: int, T: int | None = None, n_q_heads: int = N_HEADS,
                 n_kv_heads: int = N_KV, head_dim: int = HEAD_DIM, rope_dim: int = ROPE_DIM,
                 q_pitch: int = Q_PITCH, k_pitch: int = HEAD_DIM, theta: float = ROPE_THETA):
    """kernels.cu:422-455 (runtime.py:2809-2812): partial NeoX RoPE in place on
    q [T, n_q_heads, q_pitch] and k [T, n_kv_heads, k_pitch] fp16."""
    T = q.shape[0] if T is None else T
    _lib.call("fl_rope_partial", _ptr(q, F16, "q", T * n_q_heads * q_pitch),
              _ptr(k, F16, "k", T * n_kv_heads * k_pitch), n_q_heads, n_kv_heads, head_dim,
              rope_dim, q_pitch, k_pitch, pos0, T, float(theta), _stream())


def attn_prep(qg, k, v, wq, wk, kcache, vcache, *, pos0: int, T: int | None = None,
              layer: int = 0, n_q_heads: int = N_HEADS, n_kv_heads: int = N_KV,
              head_dim: int = HEAD_DIM, q_pitch: int = Q_PITCH, max_pos: int | None = None,
              rope_dim: int = ROPE_DIM, theta: float = ROPE_THETA, eps: float = NORM_EPS):
    """runtime.py:2797-2815 in one launch: rmsnorm1p of q (inside qg) and k,
    rope_partial of both (both rewritten in place), and the roped k and v
    [T, n_kv, head_dim] stored at cache rows pos0 + t (kv_store)."""
    T = qg.shape[0] if T is None else T
    max_pos = kcache.shape[-3] if max_pos is None else max_pos
    row = n_kv_heads * head_dim
    _lib.call("fl_attn_prep", _ptr(qg, F16, "qg", T * n_q_heads * q_pitch), q_pitch,
              _ptr(k, F16, "k", T * row), _ptr(v, F16, "v", T * row),
              _ptr(wq, F32, "wq", head_dim), _ptr(wk, F32, "wk", head_dim),
              _ptr(kcache, F16, "kcache", (layer + 1) * max_pos * row),
              _ptr(vcache, F16, "vcache", (layer + 1) * max_pos * row), layer, n_q_heads,
              n_kv_heads, head_dim, pos0, max_pos, T, rope_dim, float(theta), float(eps),
              _stream())


def attention_split_gqa(q, kcache, vcache, pacc, pm, pd, *, layer: int = 0,
                        n_q_heads: int = N_HEADS, n_kv_heads: int = N_KV,
                        head_dim: int = HEAD_DIM, q_pitch: int = Q_PITCH, pos0: int,
                        max_pos: int | None = None, scale: float = ATTN_SCALE,
                        split_rows: int = SPLIT_ROWS, T: int, split: int = SPLIT_MAX):
    """kernels.cu:820-835 (runtime.py:2830-2837): split partials of T tokens at
    pos0.. -- pacc [T, n_q_heads, split, head_dim], pm / pd [T, n_q_heads, split]
    fp32, pm in natural-log units. The per-token split rule is geometry.py's."""
    max_pos = kcache.shape[-3] if max_pos is None else max_pos
    row = n_kv_heads * head_dim
    parts = T * n_q_heads * split
    _lib.call("fl_attention_split_gqa",
              _ptr(q, F16, "q", (T - 1) * n_q_heads * q_pitch + n_q_heads * q_pitch),
              _ptr(kcache, F16, "kcache", (layer + 1) * max_pos * row),
              _ptr(vcache, F16, "vcache", (layer + 1) * max_pos * row),
              _ptr(pacc, F32, "pacc", parts * head_dim), _ptr(pm, F32, "pm", parts),
              _ptr(pd, F32, "pd", parts), layer, n_q_heads, n_kv_heads, head_dim, q_pitch, pos0,
              max_pos, float(scale), split_rows, T, split, _stream())


def attention_merge(pacc, pm, pd, z, *, n_q_heads: int = N_HEADS, head_dim: int = HEAD_DIM,
                    z_pitch: int = HEAD_DIM, T: int, split: int, gate=None,
                    g_pitch: int = Q_PITCH, g_off: int = GATE_OFF):
    """kernels.cu:1398-1424 (runtime.py:2844-2846), with attn_gate
    (kernels.cu:1585-1600) fused when `gate` (a q|gate buffer view) is given."""
    parts = T * n_q_heads * split
    _lib.call("fl_attention_merge", _ptr(pacc, F32, "pacc", parts * head_dim),
              _ptr(pm, F32, "pm", parts), _ptr(pd, F32, "pd", parts),
              _ptr(z, F16, "z", T * n_q_heads * z_pitch), n_q_heads, head_dim, z_pitch, T, split,
              _ptr(gate, F16, "gate", T * n_q_heads * g_pitch), g_pitch, g_off, _stream())


def attn_gate(z, g, *, n_heads: int = N_HEADS, head_dim: int = HEAD_DIM,
              z_pitch: int = HEAD_DIM, g_pitch: int = Q_PITCH, g_off: int = GATE_OFF, T: int):
    """kernels.cu:1585-1600 (runtime.py:2860-2862): z = f16_sat(z * sigmoid(g))."""
    _lib.call("fl_attn_gate", _ptr(z, F16, "z", T * n_heads * z_pitch),
              _ptr(g, F16, "g", T * n_heads * g_pitch), n_heads, head_dim, z_pitch, g_pitch,
              g_off, T, _stream())


def attn_decode_work_bytes(B: int, T: int, n_q_heads: int = N_HEADS, head_dim: int = HEAD_DIM,
                           split: int = SPLIT_MAX) -> int:
    return int(_lib.lib().fl_attn_decode_work_bytes(B, T, n_q_heads, head_dim, split))


def attn_decode(qg, kcaches, vcaches, pos0s, *, z=None, gate: bool = True,
                n_kv_heads: int = N_KV, scale: float = ATTN_SCALE,
                split_rows: int = DEC_SPLIT_ROWS, split: int = SPLIT_MAX, work=None):
    """The decode / MTP-verify attention block of B sequences (runtime.py:
    2828-2862 and the per-sequence loop of 2865-2878): split partials + merge
    + sigmoid gate. qg [B, T, n_q_heads, q_pitch] fp16 with q | gate per head;
    kcaches / vcaches: per-sequence layer caches [cap, n_kv, head_dim] fp16;
    pos0s: each sequence's first query position. split_rows: 0 (default) the
    library's grid-sized split, > 0 the length-only rule (geometry.py).
    Returns z [B, T, n_q_heads, head_dim] fp16."""
    B, T, n_q_heads, q_pitch = qg.shape
    head_dim = kcaches[0].shape[-1]
    _contig(qg, "qg")
    if z is None:
        z = torch.empty((B, T, n_q_heads, head_dim), dtype=F16, device=qg.device)
    need = attn_decode_work_bytes(B, T, n_q_heads, head_dim, split)
    if work is None:
        work = torch.empty(need, dtype=torch.uint8, device=qg.device)
    if len(kcaches) != B or len(vcaches) != B or len(pos0s) != B:
        raise ValueError("one cache pair and one pos0 per sequence")
    caps = []
    for b in range(B):
        for name, c in (("kcache", kcaches[b]), ("vcache", vcaches[b])):
            _contig(c, name)
            _ptr(c, F16, name, c.shape[-3] * n_kv_heads * head_dim)
        caps.append(kcaches[b].shape[-3])
    _lib.call("fl_attn_decode", _ptr(qg, F16, "qg", B * T * n_q_heads * q_pitch), q_pitch,
              _lib.ptr_array([c.data_ptr() for c in kcaches]),
              _lib.ptr_array([c.data_ptr() for c in vcaches]), _lib.int_array(pos0s),
              _lib.int_array(caps), B, T, n_q_heads, n_kv_heads, head_dim, float(scale),
              split_rows, split, qg.data_ptr() if gate else None, q_pitch, GATE_OFF if gate else 0,
              _ptr(z, F16, "z", B * T * n_q_heads * head_dim), z.shape[-1],
              _ptr(work, torch.uint8, "work", need), work.numel(), _stream())
    return z


def attn_decode_noalloc(qg, kcaches, vcaches, pos0s, z, *, gate: bool = True,
                        n_kv_heads: int = N_KV, scale: float = ATTN_SCALE,
                        split_rows: int = SPLIT_ROWS, split: int = SPLIT_MAX):
    """attn_decode without a work buffer (fl_attn_decode_noalloc): the partials
    live in the library's static per-GPU array, so nothing is allocated; z
    [B, T, n_q_heads, head_dim] fp16 must be given. Calls that overlap on one
    GPU race on that array."""
    B, T, n_q_heads, q_pitch = qg.shape
    head_dim = kcaches[0].shape[-1]
    _contig(qg, "qg")
    if len(kcaches) != B or len(vcaches) != B or len(pos0s) != B:
        raise ValueError("one cache pair and one pos0 per sequence")
    for b in range(B):
        for name, c in (("kcache", kcaches[b]), ("vcache", vcaches[b])):
            _contig(c, name)
            _ptr(c, F16, name, c.shape[-3] * n_kv_heads * head_dim)
    _lib.call("fl_attn_decode_noalloc", _ptr(qg, F16, "qg", B * T * n_q_heads * q_pitch), q_pitch,
              _lib.ptr_array([c.data_ptr() for c in kcaches]),
              _lib.ptr_array([c.data_ptr() for c in vcaches]), _lib.int_array(pos0s),
              _lib.int_array([c.shape[-3] for c in kcaches]), B, T, n_q_heads, n_kv_heads,
              head_dim, float(scale), split_rows, split, qg.data_ptr() if gate else None, q_pitch,
              GATE_OFF if gate else 0, _ptr(z, F16, "z", B * T * n_q_heads * head_dim),
              z.shape[-1], _stream())
    return z


def attention_prefill(q, kcache, vcache, *, pos0: int, T: int | None = None, z=None,
                      k_new=None, v_new=None, layer: int = 0, n_q_heads: int = N_HEADS,
                      n_kv_heads: int = N_KV, q_pitch: int | None = None,
                      scale: float = ATTN_SCALE, max_pos: int | None = None,
                      split: int | None = None, work=None, gated: bool = False):
    """attention_prefill_fh + attention_merge_fh (kernels.cu:2461-2807, host
    _attn_fh runtime.py:2943-2959), with kv_store (kernels.cu:465-484) of
    k_new / v_new [T, n_kv, head_dim] fused in front when given. q [T,
    n_q_heads, q_pitch] fp16 (q first in a head's row). split: the KV split
    (None: prefill_split_count's choice; a split > 1 leaves partials in `work`,
    a uint8 tensor, allocated here unless given). gated: attn_gate applied too
    (kernels.cu:1585-1600, runtime.py:2860-2862), the gate the second half of
    each head's q row -- in the merge when the KV is split. Returns z [T,
    n_q_heads, head_dim] fp16."""
    T = q.shape[0] if T is None else T
    q_pitch = q.shape[-1] if q_pitch is None else q_pitch
    head_dim = kcache.shape[-1]
    max_pos = kcache.shape[-3] if max_pos is None else max_pos
    row = n_kv_heads * head_dim
    if z is None:
        z = torch.empty((T, n_q_heads, head_dim), dtype=F16, device=q.device)
    split, work = _prefill_split(T, pos0, n_q_heads, n_kv_heads, head_dim, split, work, q.device)
    args = (_ptr(q, F16, "q", T * n_q_heads * q_pitch), q_pitch,
            _ptr(k_new, F16, "k_new", T * row), _ptr(v_new, F16, "v_new", T * row),
            _ptr(kcache, F16, "kcache", (layer + 1) * max_pos * row),
            _ptr(vcache, F16, "vcache", (layer + 1) * max_pos * row), layer, n_q_heads,
            n_kv_heads, head_dim, pos0, max_pos, float(scale), T)
    zargs = (_ptr(z, F16, "z", T * n_q_heads * z.shape[-1]), z.shape[-1])
    if gated:
        _prefill_gated(args, 0, split, zargs, work)
    elif split == 1:
        _lib.call("fl_attention_prefill", *args, *zargs, _stream())
    else:
        _lib.call("fl_attention_prefill_kv", *args, split, *zargs,
                  _ptr(work, torch.uint8, "work", work.numel()), work.numel(), _stream())
    return z


def _prefill_gated(args, q8: int, split: int, zargs, work):
    """fl_attention_prefill_gated over the (q .. T) arguments of the ungated
    entry points (layer is args[6]; the cache flag goes after it)."""
    wp = _ptr(work, torch.uint8, "work", work.numel()) if work is not None else None
    _lib.call("fl_attention_prefill_gated", *args[:7], q8, *args[7:], split, *zargs, wp,
              work.numel() if work is not None else 0, _stream())


def prefill_split_count(T: int, pos0: int, n_q_heads: int = N_HEADS,
                        n_kv_heads: int = N_KV) -> int:
    """The KV split the prefill takes for T queries at pos0 (runtime.py:
    2932-2941's role): 1 unless the 128-row workgroups are too few for the
    CUs (the 64-rows-a-wave kernel's split from 64 workgroups of 256 rows
    and 16384 cache rows, the 128-row kernel's otherwise). The int8 prefill
    takes prefill_split_count_q8's."""
    return int(_lib.lib().fl_attention_prefill_split_count(T, pos0, n_q_heads, n_kv_heads))


def prefill_split_count_q8(T: int, pos0: int, n_q_heads: int = N_HEADS,
                           n_kv_heads: int = N_KV) -> int:
    """prefill_split_count for an int8 cache: the 128-row int8 kernel's split
    (what fl_attention_prefill_kv_q8 takes for split 0)."""
    return int(_lib.lib().fl_attention_prefill_split_count_q8(T, pos0, n_q_heads, n_kv_heads))


def _prefill_split(T, pos0, n_q_heads, n_kv_heads, head_dim, split, work, device, q8=False):
    if split is None:
        split = (prefill_split_count_q8 if q8 else prefill_split_count)(T, pos0, n_q_heads,
                                                                          n_kv_heads)
    if split > 1 and work is None:
        need = int(_lib.lib().fl_attention_prefill_work_bytes(T, n_q_heads, head_dim, split))
        work = torch.empty(need, dtype=torch.uint8, device=device)
    return split, work


# ---------------------------------------------------------------------------
# int8 KV cache (kernels.cu:486-520's format): one flat int8 buffer a layer
# and K / V of kv8_nbytes(max_pos) bytes -- the values [max_pos, n_kv, 256],
# then the fp16 scales [max_pos, n_kv, 8]. A flat buffer carries no shape, so
# these take max_pos explicitly.
# ---------------------------------------------------------------------------

def kv8_cache(max_pos: int, n_kv_heads: int = N_KV, head_dim: int = HEAD_DIM, device="cuda"):
    """A zeroed int8 cache buffer of capacity max_pos."""
    return torch.zeros(kv8_nbytes(max_pos, n_kv_heads, head_dim), dtype=I8, device=device)


def _kv8(c, name, max_pos, n_kv_heads, head_dim):
    _contig(c, name)
    return _ptr(c, I8, name, kv8_nbytes(max_pos, n_kv_heads, head_dim))


def kv_store_q8(k, v, kcache, vcache, *, pos0: int, max_pos: int, T: int | None = None,
                n_kv_heads: int = N_KV, head_dim: int = HEAD_DIM):
    """kernels.cu:486-520 (runtime.py:2813-2815 with KV8): k, v [T, n_kv,
    head_dim] fp16 quantized into positions pos0.. of the int8 buffers."""
    T = k.shape[0] if T is None else T
    row = n_kv_heads * head_dim
    _contig(k, "k"), _contig(v, "v")
    _lib.call("fl_kv_store_q8", _ptr(k, F16, "k", T * row), _ptr(v, F16, "v", T * row),
              _kv8(kcache, "kcache", max_pos, n_kv_heads, head_dim),
              _kv8(vcache, "vcache", max_pos, n_kv_heads, head_dim), 0, pos0, T, n_kv_heads,
              head_dim, max_pos, _stream())


def attn_prep_q8(qg, k, v, wq, wk, kcache, vcache, *, pos0: int, max_pos: int,
                 T: int | None = None, n_q_heads: int = N_HEADS, n_kv_heads: int = N_KV,
                 head_dim: int = HEAD_DIM, q_pitch: int = Q_PITCH, rope_dim: int = ROPE_DIM,
                 theta: float = ROPE_THETA, eps: float = NORM_EPS):
    """attn_prep_q8 (kernels.cu:837-908, runtime.py:2922-2930): attn_prep with
    the int8 store."""
    T = qg.shape[0] if T is None else T
    row = n_kv_heads * head_dim
    _lib.call("fl_attn_prep_q8", _ptr(qg, F16, "qg", T * n_q_heads * q_pitch), q_pitch,
              _ptr(k, F16, "k", T * row), _ptr(v, F16, "v", T * row),
              _ptr(wq, F32, "wq", head_dim), _ptr(wk, F32, "wk", head_dim),
              _kv8(kcache, "kcache", max_pos, n_kv_heads, head_dim),
              _kv8(vcache, "vcache", max_pos, n_kv_heads, head_dim), 0, n_q_heads, n_kv_heads,
              head_dim, pos0, max_pos, T, rope_dim, float(theta), float(eps), _stream())


def attn_prep_rows(qg, k, v, wq, wk, kcaches, vcaches, pos, caps, *, kv8: bool,
                   n_q_heads: int = N_HEADS, n_kv_heads: int = N_KV, head_dim: int = HEAD_DIM,
                   q_pitch: int = Q_PITCH, rope_dim: int = ROPE_DIM, theta: float = ROPE_THETA,
                   eps: float = NORM_EPS):
    """The prep of a batched decode step's rows in one launch (the per-row
    attn_prep / attn_prep_q8 calls of runtime.py:2873-2876): row b of qg [B,
    n_q_heads, q_pitch], k / v [B, n_kv, head_dim] into kcaches[b] /
    vcaches[b] (capacity caps[b]; fp16 [cap, n_kv, head_dim] or, kv8, the
    int8 buffers) at position pos[b]."""
    B = qg.shape[0]
    row = n_kv_heads * head_dim
    if not (len(kcaches) == len(vcaches) == len(pos) == len(caps) == B):
        raise ValueError("one cache pair, position and capacity per row")
    for b in range(B):
        for name, c in (("kcache", kcaches[b]), ("vcache", vcaches[b])):
            if kv8:
                _kv8(c, name, caps[b], n_kv_heads, head_dim)
            else:
                _contig(c, name)
                _ptr(c, F16, name, caps[b] * row)
    _lib.call("fl_attn_prep_rows", _ptr(qg, F16, "qg", B * n_q_heads * q_pitch), q_pitch,
              _ptr(k, F16, "k", B * row), _ptr(v, F16, "v", B * row),
              _ptr(wq, F32, "wq", head_dim), _ptr(wk, F32, "wk", head_dim),
              _lib.ptr_array([c.data_ptr() for c in kcaches]),
              _lib.ptr_array([c.data_ptr() for c in vcaches]), _lib.int_array(pos),
              _lib.int_array(caps), B, int(bool(kv8)), n_q_heads, n_kv_heads, head_dim, rope_dim,
              float(theta), float(eps), _stream())


def attention_split_gqa_q8(q, kcache, vcache, pacc, pm, pd, *, pos0: int, max_pos: int, T: int,
                           n_q_heads: int = N_HEADS, n_kv_heads: int = N_KV,
                           head_dim: int = HEAD_DIM, q_pitch: int = Q_PITCH,
                           scale: float = ATTN_SCALE, split_rows: int = SPLIT_ROWS,
                           split: int = SPLIT_MAX):
    """kernels.cu:910-1047: attention_split_gqa's partials over an int8 cache."""
    parts = T * n_q_heads * split
    _lib.call("fl_attention_split_gqa_q8", _ptr(q, F16, "q", T * n_q_heads * q_pitch),
              _kv8(kcache, "kcache", max_pos, n_kv_heads, head_dim),
              _kv8(vcache, "vcache", max_pos, n_kv_heads, head_dim),
              _ptr(pacc, F32, "pacc", parts * head_dim), _ptr(pm, F32, "pm", parts),
              _ptr(pd, F32, "pd", parts), 0, n_q_heads, n_kv_heads, head_dim, q_pitch, pos0,
              max_pos, float(scale), split_rows, T, split, _stream())


def attention_dec_q8(q, kcache, vcache, pacc, pm, pd, *, pos0: int, max_pos: int, T: int,
                     n_q_heads: int = N_HEADS, n_kv_heads: int = N_KV, q_pitch: int = Q_PITCH,
                     sl2: float = ATTN_SCALE * LOG2E, tmin: int = DEC_TMIN,
                     smax: int = DEC_SMAX):
    """kernels.cu:1049-1335 (runtime.py:2907-2916): int8 decode partials of T
    tokens -- pacc [T, n_q_heads, smax, 256], pm (log2 units) / pd [T,
    n_q_heads, smax]; only each token's first St splits are written."""
    parts = T * n_q_heads * smax
    _lib.call("fl_attention_dec_q8", _ptr(q, F16, "q", T * n_q_heads * q_pitch),
              _kv8(kcache, "kcache", max_pos, n_kv_heads, HEAD_DIM),
              _kv8(vcache, "vcache", max_pos, n_kv_heads, HEAD_DIM),
              _ptr(pacc, F32, "pacc", parts * HEAD_DIM), _ptr(pm, F32, "pm", parts),
              _ptr(pd, F32, "pd", parts), n_q_heads, n_kv_heads, q_pitch, pos0, max_pos,
              float(sl2), tmin, smax, T, _stream())


def attention_dec_merge(pacc, pm, pd, z, *, pos0: int, T: int, n_q_heads: int = N_HEADS,
                        z_pitch: int = HEAD_DIM, tmin: int = DEC_TMIN, smax: int = DEC_SMAX,
                        gate=None, g_pitch: int = Q_PITCH, g_off: int = GATE_OFF):
    """kernels.cu:1336-1385 (runtime.py:2917-2920): the merge of
    attention_dec_q8's partials, with the sigmoid gate when `gate` is given."""
    parts = T * n_q_heads * smax
    _lib.call("fl_attention_dec_merge", _ptr(pacc, F32, "pacc", parts * HEAD_DIM),
              _ptr(pm, F32, "pm", parts), _ptr(pd, F32, "pd", parts),
              _ptr(z, F16, "z", T * n_q_heads * z_pitch), n_q_heads, z_pitch, pos0, tmin, smax,
              T, _ptr(gate, F16, "gate", T * n_q_heads * g_pitch), g_pitch, g_off, _stream())


def attn_decode_q8(qg, kcaches, vcaches, pos0s, caps, *, z=None, gate: bool = True,
                   n_kv_heads: int = N_KV, scale: float = ATTN_SCALE,
                   split_rows: int = DEC_SPLIT_ROWS, split: int = SPLIT_MAX, work=None):
    """attn_decode over int8 caches: kcaches / vcaches per-sequence int8 buffers
    of capacities caps. Returns z [B, T, n_q_heads, 256] fp16."""
    B, T, n_q_heads, q_pitch = qg.shape
    _contig(qg, "qg")
    if z is None:
        z = torch.empty((B, T, n_q_heads, HEAD_DIM), dtype=F16, device=qg.device)
    need = attn_decode_work_bytes(B, T, n_q_heads, HEAD_DIM, split)
    if work is None:
        work = torch.empty(need, dtype=torch.uint8, device=qg.device)
    if not (len(kcaches) == len(vcaches) == len(pos0s) == len(caps) == B):
        raise ValueError("one cache pair, pos0 and capacity per sequence")
    for b in range(B):
        _kv8(kcaches[b], "kcache", caps[b], n_kv_heads, HEAD_DIM)
        _kv8(vcaches[b], "vcache", caps[b], n_kv_heads, HEAD_DIM)
    _lib.call("fl_attn_decode_q8", _ptr(qg, F16, "qg", B * T * n_q_heads * q_pitch), q_pitch,
              _lib.ptr_array([c.data_ptr() for c in kcaches]),
              _lib.ptr_array([c.data_ptr() for c in vcaches]), _lib.int_array(pos0s),
              _lib.int_array(caps), B, T, n_q_heads, n_kv_heads, HEAD_DIM, float(scale),
              split_rows, split, qg.data_ptr() if gate else None, q_pitch, GATE_OFF if gate else 0,
              _ptr(z, F16, "z", B * T * n_q_heads * HEAD_DIM), z.shape[-1],
              _ptr(work, torch.uint8, "work", need), work.numel(), _stream())
    return z


def attention_prefill_q8(q, kcache, vcache, *, pos0: int, max_pos: int, T: int | None = None,
                         z=None, k_new=None, v_new=None, n_q_heads: int = N_HEADS,
                         n_kv_heads: int = N_KV, q_pitch: int | None = None,
                         scale: float = ATTN_SCALE, split: int | None = None, work=None,
                         gated: bool = False):
    """attention_prefill_fh_q8 (kernels.cu:2778-2786) over an int8 cache, with
    kv_store_q8 of k_new / v_new fused in front when given. Long prompts run
    the fp16 long-prompt kernel on an fp16 copy of the cache rows made first
    (in `work`, allocated here when not given or too small). gated: as
    attention_prefill's."""
    T = q.shape[0] if T is None else T
    q_pitch = q.shape[-1] if q_pitch is None else q_pitch
    row = n_kv_heads * HEAD_DIM
    if z is None:
        z = torch.empty((T, n_q_heads, HEAD_DIM), dtype=F16, device=q.device)
    split, work = _prefill_split(T, pos0, n_q_heads, n_kv_heads, HEAD_DIM, split, work, q.device,
                                 q8=True)
    args = (_ptr(q, F16, "q", T * n_q_heads * q_pitch), q_pitch,
            _ptr(k_new, F16, "k_new", T * row), _ptr(v_new, F16, "v_new", T * row),
            _kv8(kcache, "kcache", max_pos, n_kv_heads, HEAD_DIM),
            _kv8(vcache, "vcache", max_pos, n_kv_heads, HEAD_DIM), 0, n_q_heads, n_kv_heads,
            HEAD_DIM, pos0, max_pos, float(scale), T)
    zargs = (_ptr(z, F16, "z", T * n_q_heads * z.shape[-1]), z.shape[-1])
    stage = 0
    if split == 1:
        stage = int(_lib.lib().fl_attention_prefill_q8_stage_bytes(T, pos0, n_q_heads, n_kv_heads,
                                                                   HEAD_DIM))
    if split == 1 and stage > 0 and (work is None or work.numel() < stage):
        work = torch.empty(stage, dtype=torch.uint8, device=q.device)
    if gated:
        _prefill_gated(args, 1, split, zargs, work)
    elif split == 1 and stage > 0:
        _lib.call("fl_attention_prefill_kv_q8", *args, 1, *zargs,
                  _ptr(work, torch.uint8, "work", stage), work.numel(), _stream())
    elif split == 1:
        _lib.call("fl_attention_prefill_q8", *args, *zargs, _stream())
    else:
        _lib.call("fl_attention_prefill_kv_q8", *args, split, *zargs,
                  _ptr(work, torch.uint8, "work", work.numel()), work.numel(), _stream())
    return z


# ---------------------------------------------------------------------------
# Gated DeltaNet
# ---------------------------------------------------------------------------

def conv1d_causal(x, w, st_in, y, st_out, *, dim: int = QKV_ROWS, T: int, pos0: int,
                  row_stride: int = QKV_ROWS, width: int = 4):
    """kernels.cu:1634-1679 (runtime.py:3035-3038). st_in and st_out distinct."""
    _lib.call("fl_conv1d_causal", _ptr(x, F16, "x", (T - 1) * row_stride + dim),
              _ptr(w, F16, "w", dim * width), _ptr(st_in, F16, "st_in", dim * (width - 1)),
              _ptr(y, F16, "y", (T - 1) * row_stride + dim),
              _ptr(st_out, F16, "st_out", dim * (width - 1)), dim, T, pos0, row_stride, width,
              _stream())


def conv1d_causal_rows(x, w, st_in, y, st0, st1=None, st2=None, *, dim: int = QKV_ROWS, T: int,
                       pos0: int, row_stride: int = QKV_ROWS):
    """kernels.cu:1686-1714 (runtime.py:3021-3026): verify rows T <= 3, the
    state after row t into st_t."""
    n = (T - 1) * row_stride + dim
    _lib.call("fl_conv1d_causal_rows", _ptr(x, F16, "x", n), _ptr(w, F16, "w", dim * 4),
              _ptr(st_in, F16, "st_in", dim * 3), _ptr(y, F16, "y", n),
              _ptr(st0, F16, "st0", dim * 3), _ptr(st1, F16, "st1", dim * 3),
              _ptr(st2, F16, "st2", dim * 3), dim, T, pos0, row_stride, _stream())


def l2norm_scaled(x, y, *, n: int = GDN_K, rows: int, pitch: int = GDN_K, eps: float = L2_EPS,
                  scale: float = 1.0, T: int):
    """kernels.cu:373-391 (runtime.py:3070-3071)."""
    span = (T * rows - 1) * pitch + n
    _lib.call("fl_l2norm_scaled", _ptr(x, F16, "x", span), _ptr(y, F16, "y", span), n, rows,
              pitch, float(eps), float(scale), T, _stream())


def l2norm_scaled_strided(x, y, *, rows: int, token_stride: int, pitch: int = GDN_K,
                          eps: float = L2_EPS, scale: float = 1.0, T: int):
    """l2norm_scaled (n = 128) over the first `rows` head-sized rows of each
    token, token t starting at element t * token_stride (no reference
    counterpart: the GDN prefill needs only the q and k rows of the 80 the
    reference normalises, runtime.py:3068-3072); the other rows of y are not
    written."""
    span = (T - 1) * token_stride + (rows - 1) * pitch + GDN_K
    _lib.call("fl_l2norm_scaled_strided", _ptr(x, F16, "x", span), _ptr(y, F16, "y", span), rows,
              pitch, int(token_stride), float(eps), float(scale), T, _stream())


def rmsnorm_gated(o, z, w, y=None, *, T: int | None = None, rows: int = GDN_V_HEADS,
                  n: int = GDN_V, pitch: int = GDN_V, eps: float = GDN_NORM_EPS):
    """kernels.cu:335-358 (runtime.py:3063-3065): the GDN output norm
    y = f16((o / rms(o) * w) * silu(z)) over [T, rows, pitch] fp16 rows, w [n]
    fp32 (plain gamma). Returns y (new unless given)."""
    T = o.shape[0] if T is None else T
    span = T * rows * pitch
    y = torch.empty_like(o) if y is None else y
    _lib.call("fl_rmsnorm_gated", _ptr(o, F16, "o", span), _ptr(z, F16, "z", span),
              _ptr(w, F32, "w", n), _ptr(y, F16, "y", span), n, rows, pitch, T, float(eps),
              _stream())
    return y


def gdn_scalars(a, b, A_log, dt_bias, beta, decay, *, T: int, n_heads: int = GDN_V_HEADS,
                a_stride: int | None = None, b_stride: int | None = None):
    """kernels.cu:1732-1748 (runtime.py:3072-3076)."""
    a_stride = n_heads if a_stride is None else a_stride
    b_stride = n_heads if b_stride is None else b_stride
    _lib.call("fl_gdn_scalars", _ptr(a, F32, "a", (T - 1) * a_stride + n_heads),
              _ptr(b, F32, "b", (T - 1) * b_stride + n_heads), _ptr(A_log, F32, "A_log", n_heads),
              _ptr(dt_bias, F32, "dt_bias", n_heads), _ptr(beta, F32, "beta", T * n_heads),
              _ptr(decay, F32, "decay", T * n_heads), T, n_heads, a_stride, b_stride, _stream())


def gdn_scan(q, k, v, beta, decay, S, y, *, T: int, n_kheads: int = GDN_K_HEADS,
             n_vheads: int = GDN_V_HEADS, K: int = GDN_K, V: int = GDN_V,
             qk_stride: int = QKV_ROWS, v_stride: int = QKV_ROWS, y_stride: int | None = None,
             out_scale: float = Q_SCALE, group: int = GDN_GROUP, ck=None, ck_step: int = 0):
    """gdn_scan_rows / gdn_scan (kernels.cu:2831-2914, 1794-1901; runtime.py:
    3094-3108): the delta rule over T tokens, S [n_vheads, V, K] fp32 in place;
    ck (optional) receives the state after every token but the last at
    ck + t * ck_step."""
    y_stride = n_vheads * V if y_stride is None else y_stride
    _contig(S, "S")
    if ck is not None:
        _contig(ck, "ck")
    _lib.call("fl_gdn_scan", _ptr(q, F16, "q", (T - 1) * qk_stride + n_kheads * K),
              _ptr(k, F16, "k", (T - 1) * qk_stride + n_kheads * K),
              _ptr(v, F16, "v", (T - 1) * v_stride + n_vheads * V),
              _ptr(beta, F32, "beta", T * n_vheads), _ptr(decay, F32, "decay", T * n_vheads),
              _ptr(S, F32, "S", n_vheads * V * K),
              _ptr(y, F16, "y", (T - 1) * y_stride + n_vheads * V), T, n_kheads, n_vheads, K, V,
              qk_stride, v_stride, y_stride, float(out_scale), group,
              _ptr(ck, F32, "ck", max(T - 2, 0) * ck_step + n_vheads * V * K) if ck is not None
              else None, ck_step, _stream())


def gdn_decode(x, S, a, b, A_log, dt_bias, y=None, *, T: int, pos0s, conv_fused: bool = False,
               conv_w=None, cst_in=None, cst_out=None, ck=None, ck_step: int = 0,
               n_kheads: int = GDN_K_HEADS, n_vheads: int = GDN_V_HEADS, K: int = GDN_K,
               V: int = GDN_V, x_stride: int = QKV_ROWS, ab_stride: int = GDN_V_HEADS,
               out_scale: float = Q_SCALE, l2eps: float = L2_EPS):
    """gdn_scan_rows_f (+ gdn_conv1) for B sequences (kernels.cu:2916-3070;
    runtime.py:3040-3053 and the per-row loop 3131-3142). x [B, T, x_stride]
    fp16: the raw q|k|v projection row when conv_fused (T == 1, the conv runs
    in the kernel from cst_in[b] into cst_out[b]), else the conv output.
    S: list of B states [n_vheads, V, K] fp32 updated in place; a, b [B, T,
    ab_stride] fp32; ck: optional list of B checkpoint buffers. Returns y
    [B, T, n_vheads * V] fp16."""
    B = len(S)
    _contig(x, "x"), _contig(a, "a"), _contig(b, "b")
    if y is None:
        y = torch.empty((B, T, n_vheads * V), dtype=F16, device=x.device)
    state = n_vheads * V * K
    s_ptrs = [_ptr(s, F32, "S[b]", state) for s in S]
    ci = co = None
    if conv_fused:
        if cst_in is None or cst_out is None or conv_w is None:
            raise ValueError("conv_fused needs conv_w, cst_in and cst_out")
        ci = _lib.ptr_array([_ptr(c, F16, "cst_in[b]", x_stride * 3) for c in cst_in])
        co = _lib.ptr_array([_ptr(c, F16, "cst_out[b]", x_stride * 3) for c in cst_out])
    ck_arr = None
    if ck is not None:
        ck_arr = _lib.ptr_array([_ptr(c, F32, "ck[b]", max(T - 2, 0) * ck_step + state)
                                 if c is not None else None for c in ck])
    _lib.call("fl_gdn_decode", _ptr(x, F16, "x", B * T * x_stride), x_stride,
              1 if conv_fused else 0, _ptr(conv_w, F16, "conv_w", x_stride * 4), ci, co,
              _lib.int_array(pos0s), _ptr(a, F32, "a", B * T * ab_stride),
              _ptr(b, F32, "b", B * T * ab_stride), ab_stride, _ptr(A_log, F32, "A_log", n_vheads),
              _ptr(dt_bias, F32, "dt_bias", n_vheads), _lib.ptr_array(s_ptrs),
              _ptr(y, F16, "y", B * T * y.shape[-1]), y.shape[-1], ck_arr, ck_step, B, T,
              n_kheads, n_vheads, K, V, float(out_scale), float(l2eps), _stream())
    return y


def gdn_decode_normed(x, S, a, b, A_log, dt_bias, z, norm_w, y=None, *, pos0s, T: int = 1,
                      conv_fused: bool = True, conv_w=None, cst_in=None, cst_out=None, ck=None,
                      ck_step: int = 0, n_kheads: int = GDN_K_HEADS,
                      n_vheads: int = GDN_V_HEADS, K: int = GDN_K, V: int = GDN_V,
                      x_stride: int = QKV_ROWS, ab_stride: int = GDN_V_HEADS,
                      out_scale: float = Q_SCALE, l2eps: float = L2_EPS,
                      norm_eps: float = GDN_NORM_EPS):
    """A decode step or a verify round of B sequences and its output norm in
    one launch (gdn_scan_rows_f, kernels.cu:2916-3070, then rmsnorm_gated,
    kernels.cu:335-358, as runtime.py:3040-3053 / 3131-3142 and 3063-3065
    run them): the values gdn_decode followed by rmsnorm_gated give. x [B * T,
    x_stride] fp16 -- the raw q|k|v rows when conv_fused (T == 1, the conv
    from cst_in[b] into cst_out[b]), else the conv output; z [B * T, n_vheads
    * V] fp16 (rows at z's stride); S: list of B states; a, b [B * T,
    ab_stride] fp32; ck: optional list of B checkpoint buffers (a verify's
    state after every row but the last, at ck + t * ck_step). Returns y [B *
    T, n_vheads * V] fp16 (new unless given)."""
    B = len(S)
    rows = B * T
    _contig(x, "x"), _contig(a, "a"), _contig(b, "b")
    width = n_vheads * V
    if y is None:
        y = torch.empty((rows, width), dtype=F16, device=x.device)
    # one row a (sequence, token), the heads contiguous inside it (view raises if not)
    z_pitch, y_pitch = z.view(rows, width).stride(0), y.view(rows, width).stride(0)
    state = n_vheads * V * K
    ci = co = None
    if conv_fused:
        if cst_in is None or cst_out is None or conv_w is None:
            raise ValueError("conv_fused needs conv_w, cst_in and cst_out")
        ci = _lib.ptr_array([_ptr(c, F16, "cst_in[b]", x_stride * 3) for c in cst_in])
        co = _lib.ptr_array([_ptr(c, F16, "cst_out[b]", x_stride * 3) for c in cst_out])
    ck_arr = None
    if ck is not None:
        ck_arr = _lib.ptr_array([_ptr(c, F32, "ck[b]", max(T - 2, 0) * ck_step + state)
                                 if c is not None else None for c in ck])
    _lib.call("fl_gdn_decode_normed", _ptr(x, F16, "x", rows * x_stride), x_stride,
              1 if conv_fused else 0, _ptr(conv_w, F16, "conv_w", x_stride * 4), ci, co,
              _lib.int_array(pos0s), _ptr(a, F32, "a", rows * ab_stride),
              _ptr(b, F32, "b", rows * ab_stride), ab_stride,
              _ptr(A_log, F32, "A_log", n_vheads), _ptr(dt_bias, F32, "dt_bias", n_vheads),
              _lib.ptr_array([_ptr(s, F32, "S[b]", state) for s in S]), ck_arr, ck_step,
              _ptr(z, F16, "z", (rows - 1) * z_pitch + width), z_pitch,
              _ptr(norm_w, F32, "norm_w", V), _ptr(y, F16, "y", (rows - 1) * y_pitch + width),
              y_pitch, B, T, n_kheads, n_vheads, K, V, float(out_scale), float(l2eps),
              float(norm_eps), _stream())
    return y


def gdn_chunked_work_bytes(T: int, n_vheads: int = GDN_V_HEADS, K: int = GDN_K, V: int = GDN_V,
                           chunk: int = GDN_CHUNK) -> int:
    return int(_lib.lib().fl_gdn_chunked_work_bytes(T, n_vheads, K, V, chunk))


def gdn_prefill_chunked(q, k, v, beta, decay, S, y=None, *, T: int, n_kheads: int = GDN_K_HEADS,
                        n_vheads: int = GDN_V_HEADS, K: int = GDN_K, V: int = GDN_V,
                        qk_stride: int = QKV_ROWS, v_stride: int = QKV_ROWS,
                        out_scale: float = Q_SCALE, group: int = GDN_GROUP,
                        chunk: int = GDN_CHUNK, work=None):
    """The chunked WY/UT scan (not in the reference; replaces gdn_scan_rows
    for prefill, runtime.py:3094-3100): same arguments and results as
    gdn_scan. Returns y [T, n_vheads * V] fp16."""
    _contig(S, "S")
    if y is None:
        y = torch.empty((T, n_vheads * V), dtype=F16, device=q.device)
    need = gdn_chunked_work_bytes(T, n_vheads, K, V, chunk)
    if work is None:
        work = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.call("fl_gdn_prefill_chunked", _ptr(q, F16, "q", (T - 1) * qk_stride + n_kheads * K),
              _ptr(k, F16, "k", (T - 1) * qk_stride + n_kheads * K),
              _ptr(v, F16, "v", (T - 1) * v_stride + n_vheads * V),
              _ptr(beta, F32, "beta", T * n_vheads), _ptr(decay, F32, "decay", T * n_vheads),
              _ptr(S, F32, "S", n_vheads * V * K),
              _ptr(y, F16, "y", (T - 1) * y.shape[-1] + n_vheads * V), T, n_kheads, n_vheads, K,
              V, qk_stride, v_stride, y.shape[-1], float(out_scale), group, chunk,
              _ptr(work, torch.uint8, "work", need), work.numel(), _stream())
    return y


def gdn_prefill_chunked_logits(q, k, v, a, b, A_log, dt_bias, S, y=None, *, T: int,
                               ab_stride: int = GDN_V_HEADS, n_kheads: int = GDN_K_HEADS,
                               n_vheads: int = GDN_V_HEADS, K: int = GDN_K, V: int = GDN_V,
                               qk_stride: int = QKV_ROWS, v_stride: int = QKV_ROWS,
                               out_scale: float = Q_SCALE, group: int = GDN_GROUP,
                               chunk: int = GDN_CHUNK, work=None):
    """gdn_scalars then gdn_prefill_chunked in one call (runtime.py:3072-3076,
    3094-3100): the scan forms beta and decay from the logits a, b [T,
    ab_stride] fp32 itself, the values gdn_scalars writes. Returns y [T,
    n_vheads * V] fp16."""
    _contig(S, "S")
    if y is None:
        y = torch.empty((T, n_vheads * V), dtype=F16, device=q.device)
    need = gdn_chunked_work_bytes(T, n_vheads, K, V, chunk)
    if work is None:
        work = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.call("fl_gdn_prefill_chunked_logits",
              _ptr(q, F16, "q", (T - 1) * qk_stride + n_kheads * K),
              _ptr(k, F16, "k", (T - 1) * qk_stride + n_kheads * K),
              _ptr(v, F16, "v", (T - 1) * v_stride + n_vheads * V),
              _ptr(a, F32, "a", (T - 1) * ab_stride + n_vheads),
              _ptr(b, F32, "b", (T - 1) * ab_stride + n_vheads), ab_stride,
              _ptr(A_log, F32, "A_log", n_vheads), _ptr(dt_bias, F32, "dt_bias", n_vheads),
              _ptr(S, F32, "S", n_vheads * V * K),
              _ptr(y, F16, "y", (T - 1) * y.shape[-1] + n_vheads * V), T, n_kheads, n_vheads, K,
              V, qk_stride, v_stride, y.shape[-1], float(out_scale), group, chunk,
              _ptr(work, torch.uint8, "work", need), work.numel(), _stream())
    return y
