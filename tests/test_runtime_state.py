"""The layer runtime's state verbs on the CPU (no kernel runs): the reference
runtime's semantics for growth, clone, truncate, size, export / import and the
verify round's keep-or-roll-back bookkeeping (model/footless/cuda_sm60/
runtime.py:1017-1060, 1209-1335, 1363-1405, 2105-2215)."""
import pytest
import torch

import __graft_entry__ as ge

fl = ge.load_package()
rt_mod = fl.runtime
SMALL = ("linear_attention", "linear_attention", "full_attention", "linear_attention",
         "full_attention")


def small_rt(kv8=False, layer_types=SMALL):
    return rt_mod.HybridRuntime(rt_mod.random_weights(layer_types, device="cpu"),
                                layer_types=layer_types, kv8=kv8, device="cpu")


def test_layer_schedule_and_sizes():
    assert len(rt_mod.LAYER_TYPES) == 64
    assert sum(t == "full_attention" for t in rt_mod.LAYER_TYPES) == 16
    assert rt_mod.LAYER_TYPES[3] == "full_attention" and rt_mod.LAYER_TYPES[0] != "full_attention"
    rt = small_rt()
    st = rt.new_state()
    assert st.s.shape == (3, 48, 128, 128) and st.s.dtype == torch.float32
    assert st.conv.shape == (2, 3, 10240, 3) and st.cap == 0
    rt.grow(st, 100)
    assert st.cap == 128 and st.lcap == [128, 128]          # the doubling ladder
    assert rt.state_nbytes(st) == 3 * 48 * 128 * 128 * 4 + 2 * 3 * 10240 * 3 * 2 + 128 * 2 * 2 * 2048
    with pytest.raises(ValueError):
        rt.grow(st, rt_mod.MAX_CONTEXT + 1)


@pytest.mark.parametrize("kv8", [False, True])
def test_grow_keeps_rows_and_int8_scales(kv8):
    """Growing moves every cached row: fp16 rows, and for the int8 format the
    values and the block scales (whose region starts at cap * 1024 bytes, so
    it moves with the capacity)."""
    rt = small_rt(kv8)
    st = rt.new_state()
    rt.grow(st, 40)
    g = torch.Generator().manual_seed(0)
    for li in range(2):
        if kv8:
            st.kk[li].copy_(torch.randint(-127, 128, st.kk[li].shape, generator=g,
                                          dtype=torch.int8))
        else:
            st.kk[li].copy_(torch.randn(st.kk[li].shape, generator=g).half())
    before = [b.clone() for b in st.kk]
    old = st.cap
    rt.grow(st, 5000)
    assert st.cap == 8192
    for li in range(2):
        if kv8:
            vals = 4 * 256
            assert torch.equal(st.kk[li][:old * vals], before[li][:old * vals])
            srow = 4 * 8 * 2
            assert torch.equal(st.kk[li][st.cap * vals:st.cap * vals + old * srow],
                               before[li][old * vals:old * vals + old * srow])
        else:
            assert torch.equal(st.kk[li][:old], before[li])


def test_clone_is_independent_and_truncate_replays():
    rt = small_rt()
    st = rt.new_state()
    rt.grow(st, 10)
    st.tokens = [5, 6, 7, 8]
    st.fed = 4
    st.s.fill_(1.5)
    st.conv.fill_(2.0)
    st.phase = 1
    c = rt.clone_state(st)
    assert c.tokens == st.tokens and c.phase == 1 and torch.equal(c.s, st.s)
    c.s.zero_()
    assert float(st.s.max()) == 1.5                      # no shared storage
    # truncate at or beyond the logical length only moves `fed`
    rt.truncate_state(st, 9)
    assert st.tokens == [5, 6, 7, 8] and st.replay is None
    # below: the recurrences restart, the kept ids become a replay
    rt.truncate_state(st, 2)
    assert st.tokens == [5, 6] and st.replay == [5, 6] and st.fed == 2
    assert float(st.s.abs().max()) == 0.0 and float(st.conv.abs().max()) == 0.0
    assert rt.take_replay(st) == [5, 6] and st.tokens == [] and st.replay is None
    # to zero: a fresh state, nothing to replay
    c2 = rt.clone_state(c)
    rt.truncate_state(c2, 0)
    assert c2.replay is None and c2.tokens == []


def test_export_import_round_trip_model_geometry():
    """The reference's blob at the model's geometry (48 GDN, 16 full layers)."""
    rt = rt_mod.HybridRuntime(rt_mod.random_weights(device="cpu"), device="cpu")
    st = rt.new_state()
    rt.grow(st, 33)                                       # cap 64
    g = torch.Generator().manual_seed(3)
    st.s.copy_(torch.randn(st.s.shape, generator=g))
    st.conv.copy_(torch.randn(st.conv.shape, generator=g).half())
    for b in st.kk + st.kv:
        b.copy_(torch.randn(b.shape, generator=g).half())
    st.tokens, st.fed, st.phase = list(range(33)), 33, 1
    blob = rt.export_state(st)
    back = rt.import_state(blob)
    assert back.tokens == st.tokens and back.phase == 1 and back.cap == 64
    assert torch.equal(back.s, st.s) and torch.equal(back.conv, st.conv)
    for a, b in zip(back.kk + back.kv, st.kk + st.kv):
        assert torch.equal(a, b)
    assert rt.export_state(back) == blob
    with pytest.raises(ValueError):
        small_rt().export_state(small_rt().new_state())   # not the model's geometry


@pytest.mark.parametrize("T,kept", [(2, 2), (2, 1), (3, 3), (3, 2), (3, 1)])
def test_accept_verify_bookkeeping(T, kept):
    """Which recurrent state and conv buffer a verify round keeps: all rows --
    the final state, and the conv state after the last row (T = 2: the other
    phase buffer; T = 3: the spare); two of three -- the checkpoint after row
    1 and the other phase buffer; one -- the checkpoint after row 0 and the
    conv state row 0 left in place."""
    rt = small_rt()
    st = rt.new_state()
    st.tokens, st.phase = [1, 2, 3], 0
    rt._ensure_verify_buffers()
    st.s.fill_(9.0)                                       # the state after the last row
    rt.snap_s[0].fill_(1.0)                               # after row 0
    rt.snap_s[1].fill_(2.0)                               # after row 1
    st.conv[0].fill_(10.0)                                # row 0's conv state (in place)
    st.conv[1].fill_(11.0)                                # row 1's
    rt.snap_c.fill_(12.0)                                 # row 2's
    rt.verify_T, rt._verify_pos0 = T, 3
    rt.accept_verify(st, [7, 8, 9][:T], kept)
    assert st.tokens == [1, 2, 3] + [7, 8, 9][:kept]
    want_s = 9.0 if kept == T else float(kept)
    assert float(st.s.min()) == float(st.s.max()) == want_s
    live = float(st.conv[st.phase].max())
    assert live == {1: 10.0, 2: 11.0, 3: 12.0}[kept]
    with pytest.raises(ValueError):                       # only once a verify
        rt.accept_verify(st, [7, 8, 9][:T], kept)
