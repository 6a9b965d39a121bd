"""The state blob (runtime.py:1267-1329) on the CPU: byte layout restated from
the reference's export code, round trips, int8 KV buffers whose capacity
exceeds the exported cap (scales read from byte lcap * 1024), bad blobs."""
import json
import struct

import numpy as np
import pytest
import torch


@pytest.fixture(scope="module")
def sb(fl):
    return fl.state_blob


def make_state(sb, cap, lcap, kv8, seed=0, logits=True):
    g = torch.Generator().manual_seed(seed)
    S = torch.randn(sb.GDN_S_SHAPE, generator=g)
    conv = tuple(torch.randn(sb.CONV_SHAPE, generator=g).half() for _ in range(2))
    lg = torch.randn(sb.VOCAB, generator=g).half() if logits else None
    row = sb.kv_row_bytes(kv8)
    if kv8:
        kk = [torch.randint(0, 256, (lc * row,), generator=g, dtype=torch.uint8) for lc in lcap]
        kv = [torch.randint(0, 256, (lc * row,), generator=g, dtype=torch.uint8) for lc in lcap]
    else:
        kk = [torch.randn((lc, 4, 256), generator=g).half() for lc in lcap]
        kv = [torch.randn((lc, 4, 256), generator=g).half() for lc in lcap]
    meta = {"tokens": [5, 6, 7], "fed": 3, "pending": None, "replay": None, "phase": "decode"}
    return meta, S, conv, lg, kk, kv


def test_layout_matches_the_reference_order(sb):
    cap = 8
    meta, S, conv, lg, kk, kv = make_state(sb, cap, [8] * 16, kv8=False)
    blob = sb.export_state(meta, S, conv, lg, kk, kv, [8] * 16, cap)
    head = json.dumps({"tokens": [5, 6, 7], "fed": 3, "pending": None, "replay": None,
                       "cap": cap, "phase": "decode"}).encode()
    assert blob[:4] == struct.pack("<I", len(head)) and blob[4:4 + len(head)] == head
    off = 4 + len(head)
    assert blob[off:off + 16] == S.numpy().tobytes()[:16]
    off += sb.GDN_S_BYTES
    assert blob[off:off + sb.GDN_CONV_BYTES] == conv[0].numpy().tobytes()
    off += 2 * sb.GDN_CONV_BYTES
    assert blob[off:off + 4] == struct.pack("<I", 1)
    off += 4 + sb.VOCAB * 2
    assert blob[off:off + cap * 2048] == kk[0].numpy().tobytes()
    assert len(blob) == off + 2 * 16 * cap * 2048


@pytest.mark.parametrize("kv8", [False, True])
def test_round_trip(sb, kv8):
    cap, lcap = 64, [128] * 16          # buffers larger than the exported cap
    meta, S, conv, lg, kk, kv = make_state(sb, cap, lcap, kv8, seed=1)
    blob = sb.export_state(meta, S, conv, lg, kk, kv, lcap, cap, kv8=kv8)
    st = sb.import_state(blob, "cpu", kv8=kv8)
    assert st["meta"] == meta and st["cap"] == cap
    assert torch.equal(st["S"], S) and torch.equal(st["conv"][1], conv[1])
    assert torch.equal(st["logits"], lg)
    row = sb.kv_row_bytes(kv8)
    for got, src in zip(st["kk"], kk):
        raw = src.contiguous().view(torch.uint8).reshape(-1)
        if kv8:   # values of the first cap rows, then their scales from byte lcap * 1024
            want = torch.cat([raw[:cap * 1024], raw[128 * 1024:128 * 1024 + cap * (row - 1024)]])
            assert torch.equal(got, want)
        else:
            assert torch.equal(got, src[:cap])
    # a re-export of the imported state is the same bytes
    again = sb.export_state(st["meta"], st["S"], st["conv"], st["logits"], st["kk"], st["kv"],
                            [cap] * 16, cap, kv8=kv8)
    assert again == blob


def test_no_kv_no_logits_and_bad_blobs(sb):
    meta, S, conv, _, _, _ = make_state(sb, 0, [], kv8=False, logits=False)
    blob = sb.export_state(meta, S, conv)
    st = sb.import_state(blob, "cpu")
    assert st["logits"] is None and st["kk"] == [] and st["cap"] == 0
    with pytest.raises(ValueError):
        sb.import_state(blob[:-5], "cpu")                # truncated
    assert sb.import_state(blob + b"\0", "cpu")["cap"] == 0   # trailing bytes are not read


def test_capacity_ladder(sb):
    # runtime.py:1209-1219: doubling from 32 to 4096, then steps of 4096, capped
    assert [sb.next_cap(n) for n in (1, 32, 33, 4096, 4097, 100_000, 102_400)] == \
        [32, 32, 64, 4096, 8192, 102_400, 102_400]
    meta, S, conv, _, kk, kv = make_state(sb, 48, [48] * 16, kv8=False, logits=False)
    blob = sb.export_state(meta, S, conv, None, kk, kv, [48] * 16, 48)
    with pytest.raises(ValueError, match="reserves 64"):
        sb.import_state(blob, "cpu")                     # 48 is not a ladder capacity
    with pytest.raises(ValueError):
        sb.export_state(meta, S[:1], conv)               # wrong state shape
