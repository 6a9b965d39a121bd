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
             float(g.ATTN_SCALE), g.SPLIT_ROWS, g.SPLIT_MAX, qg.data_ptr(), qp, g.GATE_OFF,
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
