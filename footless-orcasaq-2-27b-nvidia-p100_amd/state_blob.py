"""A sequence's state as bytes: the export / import format of the reference
runtime (model/footless/cuda_sm60/runtime.py:1267-1329), over this build's
device buffers.

Layout, little-endian, in this order:

* ``uint32 n`` and ``n`` bytes of JSON ``{"tokens", "fed", "pending",
  "replay", "cap", "phase"}`` (keys in that order, ``json.dumps`` defaults);
* the GDN recurrent state of every GDN layer, ``[48][48][128][128]`` fp32
  (``GDN_S_BYTES``, runtime.py:180-181);
* the two conv ping-pong buffers, each ``[48][10240][3]`` fp16
  (``GDN_CONV_BYTES``, runtime.py:182-184);
* ``uint32 has_logits``, then the last logits row ``[VOCAB]`` fp16 if set;
* if ``cap``: for the K buffers, then the V buffers, of the 16 full-attention
  layers, the first ``cap`` positions of each, as a buffer of exactly ``cap``
  positions holds them (runtime.py:1196-1206). fp16: ``[cap][4][256]`` fp16.
  int8: ``[cap][4][256]`` int8 values, then ``[cap][4][8]`` fp16 block scales
  (a buffer of capacity ``lcap`` keeps its scales at byte ``lcap * 1024``).

This is host-side plumbing (device <-> host copies); the arithmetic of the
path is in libfl355.
"""
from __future__ import annotations

import json
import struct

import torch

GDN_LAYERS = 48
FULL_LAYERS = 16
VOCAB = 248320
GDN_S_SHAPE = (GDN_LAYERS, 48, 128, 128)
CONV_SHAPE = (GDN_LAYERS, 10240, 3)
GDN_S_BYTES = GDN_LAYERS * 48 * 128 * 128 * 4
GDN_CONV_BYTES = GDN_LAYERS * 3 * 10240 * 2
KV_VALUES = 4 * 256                       # values a position and layer, k or v
KV_GROW_STEP = 4096
MAX_CONTEXT = 102400


def next_cap(need: int) -> int:
    """The KV capacity reserved for `need` positions (runtime.py:1209-1219):
    doubling from 32 up to KV_GROW_STEP, then whole steps of it, at most
    MAX_CONTEXT. An exported cap is always a value of this ladder."""
    c = 32
    while c < need and c < KV_GROW_STEP:
        c *= 2
    if c < need:
        c = -(-need // KV_GROW_STEP) * KV_GROW_STEP
    return min(c, MAX_CONTEXT)


def kv_row_bytes(kv8: bool) -> int:
    """Bytes a position takes in one layer's K (or V) buffer (runtime.py:127-129)."""
    return KV_VALUES + 4 * (256 // 32) * 2 if kv8 else KV_VALUES * 2


def _host_bytes(t: torch.Tensor, nbytes: int | None = None) -> bytes:
    b = t.detach().contiguous().view(torch.uint8).reshape(-1)
    if nbytes is not None:
        b = b[:nbytes]
    return b.cpu().numpy().tobytes()


def _kv_rows(buf: torch.Tensor, lcap: int, rows: int, kv8: bool) -> bytes:
    """The first `rows` positions of one layer's buffer of capacity `lcap`."""
    raw = buf.detach().contiguous().view(torch.uint8).reshape(-1)
    if not kv8:
        return raw[:rows * kv_row_bytes(False)].cpu().numpy().tobytes()
    scales = raw[lcap * KV_VALUES:]
    return (raw[:rows * KV_VALUES].cpu().numpy().tobytes()
            + scales[:rows * (kv_row_bytes(True) - KV_VALUES)].cpu().numpy().tobytes())


def export_state(meta: dict, S: torch.Tensor, conv: tuple[torch.Tensor, torch.Tensor],
                 logits: torch.Tensor | None = None, kk=(), kv=(), lcap=(), cap: int = 0,
                 kv8: bool = False) -> bytes:
    """Serialise a state. `meta` carries tokens, fed, pending, replay and phase;
    S [48, 48, 128, 128] fp32; conv two [48, 10240, 3] fp16; logits [VOCAB] fp16
    or None; kk / kv the 16 layers' K / V buffers with capacities `lcap`,
    exported up to `cap` positions."""
    if tuple(S.shape) != GDN_S_SHAPE or S.dtype != torch.float32:
        raise ValueError(f"S must be {GDN_S_SHAPE} float32")
    if len(conv) != 2 or any(tuple(c.shape) != CONV_SHAPE or c.dtype != torch.float16
                             for c in conv):
        raise ValueError(f"conv must be two {CONV_SHAPE} float16 buffers")
    head = json.dumps({"tokens": list(meta["tokens"]), "fed": meta["fed"],
                       "pending": meta["pending"], "replay": meta["replay"], "cap": cap,
                       "phase": meta["phase"]}).encode()
    out = bytearray(struct.pack("<I", len(head)) + head)
    out += _host_bytes(S)
    out += _host_bytes(conv[0])
    out += _host_bytes(conv[1])
    out += struct.pack("<I", 1 if logits is not None else 0)
    if logits is not None:
        if logits.numel() != VOCAB or logits.dtype != torch.float16:
            raise ValueError("logits must be VOCAB float16 values")
        out += _host_bytes(logits)
    if cap:
        if len(kk) != FULL_LAYERS or len(kv) != FULL_LAYERS or len(lcap) != FULL_LAYERS:
            raise ValueError("kk, kv and lcap need the 16 full-attention layers")
        for bufs in (kk, kv):
            for buf, lc in zip(bufs, lcap):
                if lc < cap:
                    raise ValueError(f"a layer's capacity {lc} is below cap {cap}")
                out += _kv_rows(buf, lc, cap, kv8)
    return bytes(out)


def import_state(blob: bytes, device, kv8: bool = False) -> dict:
    """Parse a blob into device tensors: {"meta", "S", "conv", "logits", "kk",
    "kv", "cap"}; the K / V buffers come back with capacity exactly `cap`
    (fp16: [cap, 4, 256] float16; int8: flat uint8 of cap * row bytes).
    As in runtime.py:1279-1329, bytes after the last K / V row are not read;
    a blob shorter than its header declares raises ValueError."""
    n = struct.unpack("<I", blob[:4])[0]
    head = json.loads(blob[4:4 + n])
    off = 4 + n

    def take(nbytes):
        nonlocal off
        if off + nbytes > len(blob):
            raise ValueError("blob is shorter than its header declares")
        part = blob[off:off + nbytes]
        off += nbytes
        return torch.frombuffer(bytearray(part), dtype=torch.uint8)

    S = take(GDN_S_BYTES).view(torch.float32).reshape(GDN_S_SHAPE).to(device)
    conv = tuple(take(GDN_CONV_BYTES).view(torch.float16).reshape(CONV_SHAPE).to(device)
                 for _ in range(2))
    has_logits = struct.unpack("<I", blob[off:off + 4])[0] == 1
    off += 4
    logits = take(VOCAB * 2).view(torch.float16).to(device) if has_logits else None
    cap = head["cap"]
    kk, kv = [], []
    if cap:
        # runtime.py:1305-1323: a cap the ladder does not reproduce is a
        # foreign blob whose rows would be read at the wrong stride
        if next_cap(cap) != cap:
            raise ValueError(f"blob declares cap {cap}, which reserves {next_cap(cap)} positions")
        row = cap * kv_row_bytes(kv8)
        for bufs in (kk, kv):
            for _ in range(FULL_LAYERS):
                raw = take(row)
                bufs.append((raw if kv8 else raw.view(torch.float16).reshape(cap, 4, 256))
                            .to(device))
    meta = {k: head[k] for k in ("tokens", "fed", "pending", "replay", "phase")}
    return {"meta": meta, "S": S, "conv": conv, "logits": logits, "kk": kk, "kv": kv,
            "cap": cap}
