"""Write the golden fixtures in this directory: small seeded inputs and the C
oracle's outputs (oracle/fl_oracle.c through oracle/oracle.py) for each row
of the path -- decode / verify attention with its gate, causal prefill, the
int8 store and int8 decode, the fused attention prep, conv1d, the L2 norm,
the gates, the delta-rule scan (its result is also what the chunked scan must
reproduce) and the gated output norm.

The reference ships no vectors for this path, so these are the oracle's own,
made after the oracle was pinned by the closed forms, known answers and
invariants of tests/test_oracle_*.py. tests/test_golden.py regenerates every
output from the stored inputs and requires the same bits (the oracle has not
drifted); tests/test_gpu_golden.py runs the HIP path on the stored inputs.

Run from the repository root: python tests/golden/make_golden.py
Each fixture is an .npz of plain arrays (no pickled objects)."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import oracle as orc  # noqa: E402

SCALE = 256 ** -0.5          # the model's attention scale (head_dim 256)
QS = 128 ** -0.5             # the GDN output scale (d_k 128)


def f16(a):
    return np.ascontiguousarray(a, dtype=np.float16)


def qgate(rng, T):
    """q | gate rows [T, 24, 512]: q ~ N(0,1)/16 (config 2's scaling), gate N(0,1)."""
    qg = np.empty((T, 24, 512), np.float16)
    qg[..., :256] = rng.standard_normal((T, 24, 256)) / 16
    qg[..., 256:] = rng.standard_normal((T, 24, 256))
    return qg


def attn_decode(rng):
    """Three verify rows at the end of a 64-row fp16 cache: split partials,
    merge and sigmoid gate (kernels.cu:682-835, 1387-1424, 1572-1600)."""
    L, T = 64, 3
    kc = f16(rng.standard_normal((L, 4, 256)))
    vc = f16(rng.standard_normal((L, 4, 256)))
    qg = qgate(rng, T)
    z = orc.attention_decode(qg, kc, vc, L - T, max_pos=L, scale=SCALE)
    return {"qg": qg, "kc": kc, "vc": vc, "pos0": np.int64(L - T), "z": z}


def attn_prefill(rng):
    """16 causal rows from pos0 40 over a 56-row cache (kernels.cu:2461-2786)."""
    L, T, pos0 = 56, 16, 40
    kc = f16(rng.standard_normal((L, 4, 256)))
    vc = f16(rng.standard_normal((L, 4, 256)))
    qg = qgate(rng, T)
    z = orc.attention_prefill(qg, kc, vc, q_pitch=512, pos0=pos0, max_pos=L, scale=SCALE, T=T)
    return {"qg": qg, "kc": kc, "vc": vc, "pos0": np.int64(pos0), "z": z}


def kv8(rng):
    """40 rows stored into the int8 format (values, then fp16 per-32 scales;
    kernels.cu:486-520), then two decode rows over it with the reference's
    int8 split rule and gated merge (kernels.cu:1049-1385)."""
    L, T = 40, 2
    k = f16(rng.uniform(-1.5, 0.5, (L, 4, 256)))
    v = f16(rng.uniform(-1.5, 0.5, (L, 4, 256)))
    k[3, 1, 32:64] = 0                       # an all-zero scale block
    kc8, vc8 = orc.kv8_buffer(L), orc.kv8_buffer(L)
    orc.kv_store_q8(k, v, kc8, vc8, 0, L, L)
    qg = qgate(rng, T)
    z = orc.attention_decode_q8(qg, kc8, vc8, L - T, max_pos=L, scale=SCALE)
    return {"k": k, "v": v, "kc8": kc8, "vc8": vc8, "qg": qg, "pos0": np.int64(L - T), "z": z}


def attn_prep(rng):
    """q / k Gemma RMSNorm, partial NeoX RoPE at positions 1000.. and the KV
    store (kernels.cu:241-272, 397-455, 465-484; runtime.py:2797-2815)."""
    T, pos0 = 3, 1000
    max_pos = pos0 + T
    qg = f16(rng.standard_normal((T, 24, 512)))
    k = f16(rng.standard_normal((T, 4, 256)) * 3)
    v = f16(rng.standard_normal((T, 4, 256)))
    wq = (rng.standard_normal(256) * 0.2).astype(np.float32)
    wk = (rng.standard_normal(256) * 0.2).astype(np.float32)
    kc = np.zeros((max_pos, 4, 256), np.float16)
    vc = np.zeros_like(kc)
    q_out, k_out = orc.attn_prep(qg, k, v, wq, wk, kc, vc, pos0=pos0, T=T, max_pos=max_pos)
    return {"qg": qg, "k": k, "v": v, "wq": wq, "wk": wk, "pos0": np.int64(pos0),
            "q_out": q_out, "k_out": k_out}


def conv(rng):
    """Five tokens of the causal width-4 conv from position 3 over 256
    channels, silu applied, and the 3-frame state after them
    (kernels.cu:1634-1679)."""
    T, pos0, dim = 5, 3, 256
    x = f16(rng.standard_normal((T, dim)))
    w = f16(rng.standard_normal((dim, 4)) * 0.5)
    st = f16(rng.standard_normal((dim, 3)))
    y, st_out = orc.conv1d_causal(x, w, st, dim=dim, T=T, pos0=pos0, row_stride=dim)
    return {"x": x, "w": w, "st": st, "pos0": np.int64(pos0), "y": y, "st_out": st_out}


def norm_gates(rng):
    """l2norm_scaled over 8 head rows a token, one of them zero
    (kernels.cu:373-391), and the gates with the reference's known inputs
    (softplus branch at x = 100 and -40; kernels.cu:1732-1748)."""
    T = 2
    x = f16(rng.standard_normal((T, 8 * 128)))
    x[1, 256:384] = 0
    y = orc.l2norm_scaled(x, n=128, rows=8, pitch=128, eps=1e-6, scale=1.0, T=T)
    a = (rng.standard_normal((3, 48)) * 5).astype(np.float32)
    a[0, :2] = [100.0, -40.0]
    b = rng.standard_normal((3, 48)).astype(np.float32)
    A_log = rng.standard_normal(48).astype(np.float32)
    dt = rng.standard_normal(48).astype(np.float32)
    beta, decay = orc.gdn_scalars(a, b, A_log, dt, T=3, n_heads=48)
    return {"x": x, "y": y, "a": a, "b": b, "A_log": A_log, "dt_bias": dt, "beta": beta,
            "decay": decay}


def scan(rng):
    """The delta rule over 100 tokens for one k head and its three v heads
    (kernels.cu:1794-1901, 2831-2914): unit-L2 q / k rows, gates in (0, 1),
    S0 ~ N(0, 0.02). 100 tokens are one full 64-token chunk and a ragged one
    for the chunked form."""
    T = 100
    q = rng.standard_normal((T, 128))
    k = rng.standard_normal((T, 128))
    q = f16(q / np.linalg.norm(q, axis=1, keepdims=True))
    k = f16(k / np.linalg.norm(k, axis=1, keepdims=True))
    v = f16(rng.standard_normal((T, 3 * 128)))
    beta = (1 / (1 + np.exp(-rng.standard_normal((T, 3))))).astype(np.float32)
    decay = np.exp(-np.log1p(np.exp(rng.standard_normal((T, 3))))).astype(np.float32)
    S0 = (rng.standard_normal((3, 128, 128)) * 0.02).astype(np.float32)
    S = S0.copy()
    y = orc.gdn_scan(q, k, v, beta, decay, S, T=T, n_kheads=1, n_vheads=3, qk_stride=128,
                     v_stride=384, out_scale=QS)
    return {"q": q, "k": k, "v": v, "beta": beta, "decay": decay, "S0": S0, "S": S, "y": y}


def out_norm(rng):
    """The GDN output norm y = f16(o / rms(o) * w * silu(z)) over 48 rows of
    two tokens (kernels.cu:321-358)."""
    T = 2
    o = f16(rng.standard_normal((T, 48, 128)) * 0.7)
    z = f16(rng.standard_normal((T, 48, 128)) * 2)
    w = (1 + rng.standard_normal(128) * 0.2).astype(np.float32)
    y = orc.rmsnorm_gated(o, z, w, T=T)
    return {"o": o, "z": z, "w": w, "y": y}


FIXTURES = {
    "attn_decode": attn_decode,
    "attn_prefill": attn_prefill,
    "kv8": kv8,
    "attn_prep": attn_prep,
    "conv": conv,
    "norm_gates": norm_gates,
    "scan": scan,
    "out_norm": out_norm,
}


def make(name: str) -> dict:
    """The fixture's arrays, from its own seed."""
    seed = sum(ord(c) * 31 ** i for i, c in enumerate(name)) % (2 ** 32)
    return FIXTURES[name](np.random.default_rng(seed))


def main() -> None:
    for name in FIXTURES:
        arrays = make(name)
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        size = (HERE / f"{name}.npz").stat().st_size
        print(f"{name}.npz: {len(arrays)} arrays, {size} bytes")


if __name__ == "__main__":
    main()
