"""fl_attn_decode_noalloc, the decode / verify attention entry point that
allocates nothing (its partials live in a static device array), against
fl_attn_decode with a caller work buffer: the same kernels, so the outputs
agree bit for bit. Two calls in a row, the second smaller than the first, so
stale partials of the first call cannot leak into the second."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _caches(rng, lens, dev):
    ks = [torch.from_numpy(rng.standard_normal((L, 4, 256)).astype(np.float16)).to(dev)
          for L in lens]
    vs = [torch.from_numpy(rng.standard_normal((L, 4, 256)).astype(np.float16)).to(dev)
          for L in lens]
    return ks, vs


def _noalloc(fl, qg, ks, vs, pos0s, z):
    lib, g = fl._lib, fl.geometry
    B, T, H, qp = qg.shape
    lib.call("fl_attn_decode_noalloc", qg.data_ptr(), qp,
             lib.ptr_array([k.data_ptr() for k in ks]), lib.ptr_array([v.data_ptr() for v in vs]),
             lib.int_array(pos0s), lib.int_array([k.shape[0] for k in ks]), B, T, H, 4, 256,
             float(g.ATTN_SCALE), g.DEC_SPLIT_ROWS, g.SPLIT_MAX, qg.data_ptr(), qp, g.GATE_OFF,
             z.data_ptr(), 256, torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("seed", [0])
def test_noalloc_decode_matches_work_buffer_entry_point(fl, dev, seed):
    rng = np.random.default_rng(seed)
    cases = [([8100, 7950, 8192, 7900], 3),    # config 2's shape at 8k: 19 MB of partials
             ([1500, 700], 1)]                 # then a smaller call
    for lens, T in cases:
        ks, vs = _caches(rng, lens, dev)
        B = len(lens)
        qg = rng.standard_normal((B, T, 24, 512)).astype(np.float16)
        qg[..., :256] /= 16
        qg = torch.from_numpy(qg).to(dev)
        pos0s = [L - T for L in lens]
        z = torch.full((B, T, 24, 256), 3.0, dtype=torch.float16, device=dev)
        _noalloc(fl, qg, ks, vs, pos0s, z)
        want = fl.ops.attn_decode(qg, ks, vs, pos0s)
        torch.cuda.synchronize()
        print(f"noalloc B={B} T={T} lens={lens}: bit-exact {torch.equal(z, want)}")
        assert torch.isfinite(z.float()).all()
        assert torch.equal(z, want)


def _case(rng, lens, T, dev):
    ks, vs = _caches(rng, lens, dev)
    qg = rng.standard_normal((len(lens), T, 24, 512)).astype(np.float16)
    qg[..., :256] /= 16
    return ks, vs, torch.from_numpy(qg).to(dev), [L - T for L in lens]


def test_noalloc_refuses_calls_beyond_its_scratch(fl, dev):
    """B = 8, T = 3 at 64 splits needs ~38 MB of partials, more than the
    32 MiB array: FL_ESCRATCH, nothing launched, the output left as it was."""
    lib = fl._lib.lib()
    need = lib.fl_attn_decode_work_bytes(8, 3, 24, 256, fl.geometry.SPLIT_MAX)
    assert need > lib.fl_attn_decode_noalloc_max_bytes() == 32 << 20
    ks, vs, qg, pos0s = _case(np.random.default_rng(5), [64] * 8, 3, dev)
    z = torch.full((8, 3, 24, 256), 3.0, dtype=torch.float16, device=dev)
    with pytest.raises(fl._lib.FlError) as e:
        _noalloc(fl, qg, ks, vs, pos0s, z)
    assert e.value.status == fl._lib.FL_ESCRATCH
    torch.cuda.synchronize()
    assert bool((z == 3.0).all())


def test_noalloc_under_graph_capture(fl, dev):
    """The entry point captured into a HIP graph (torch.cuda.CUDAGraph) and
    replayed three times, with new q | gate values copied in and eager work on
    the stream between the replays: every replay equals fl_attn_decode on the
    same inputs bit for bit."""
    rng = np.random.default_rng(7)
    ks, vs, qg, pos0s = _case(rng, [3000, 2900], 3, dev)
    z = torch.zeros((2, 3, 24, 256), dtype=torch.float16, device=dev)
    _noalloc(fl, qg, ks, vs, pos0s, z)          # the device's scratch address is looked up here
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _noalloc(fl, qg, ks, vs, pos0s, z)
    for r in range(3):
        new = rng.standard_normal(tuple(qg.shape)).astype(np.float16)
        new[..., :256] /= 16
        qg.copy_(torch.from_numpy(new))
        z.fill_(7.0)
        g.replay()
        want = fl.ops.attn_decode(qg, ks, vs, pos0s)
        torch.cuda.synchronize()
        assert torch.equal(z, want), r


_FRESH = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import __graft_entry__ as ge
from tests.test_zz_no_alloc import _case, _noalloc
fl = ge.load_package()
dev = torch.device("cuda:0")
ks, vs, qg, pos0s = _case(np.random.default_rng(9), [2000, 1900, 2100], 2, dev)
z = torch.zeros((3, 2, 24, 256), dtype=torch.float16, device=dev)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):      # the process's first call of the entry point
    _noalloc(fl, qg, ks, vs, pos0s, z)
for r in range(2):
    z.fill_(7.0)
    g.replay()
    want = fl.ops.attn_decode(qg, ks, vs, pos0s)
    torch.cuda.synchronize()
    assert torch.equal(z, want), r
print("fresh-process capture: ok", flush=True)
"""


def test_noalloc_first_call_under_graph_capture(fl, dev):
    """In a fresh process the first call of the entry point (which looks up
    the device's scratch address) is made under graph capture, then replayed
    and checked against fl_attn_decode bit for bit."""
    import subprocess
    import sys
    from pathlib import Path

    repo = Path(__file__).resolve().parent.parent
    res = subprocess.run([sys.executable, "-c", _FRESH, str(repo)], capture_output=True,
                         text=True, timeout=110, cwd=str(repo))
    print(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0 and "ok" in res.stdout
