"""PyTorch fp32 CPU implementation of the hot path (test infrastructure / CPU
baseline only).

The same ops as the reference kernels (model/footless/cuda_sm60/kernels.cu),
vectorised over sequences and heads in fp32 with the reference's fp16
rounding points, for running on the host's cores: bench.py's CPU baseline
is this module, timed. tests/test_oracle_torch.py checks it
against the C oracle (fl_oracle.c). Never imported by the product.
"""
from __future__ import annotations

import math

import torch

F16, F32 = torch.float16, torch.float32


def r16(x: torch.Tensor) -> torch.Tensor:
    """fp16 store with the range pinned to +-65504 (kernels.cu:187-195), back to fp32."""
    return x.clamp(-65504.0, 65504.0).to(F16).to(F32)


# ---------------------------------------------------------------------------
# full attention
# ---------------------------------------------------------------------------

def attention_decode(qg: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int,
                     scale: float, gate: bool = True, head_dim: int = 256) -> torch.Tensor:
    """Decode / verify rows of one sequence (kernels.cu:682-835 + 1398-1424 +
    1585-1600): qg [T, 24, 512] fp16, caches [L, 4, 256] fp16, token t sees
    rows [0, pos0 + t]. Returns z [T, 24, 256] fp16."""
    T, H, _ = qg.shape
    n_kv = kc.shape[1]
    G = H // n_kv
    n = pos0 + T
    q = qg[..., :head_dim].to(F32).view(T, n_kv, G, head_dim)
    k = kc[:n].to(F32).permute(1, 0, 2)               # [kv, n, d]
    v = vc[:n].to(F32).permute(1, 0, 2)
    s = torch.einsum("tkgd,knd->tkgn", q, k) * scale  # [T, kv, G, n]
    pos = torch.arange(n)
    mask = pos[None, :] > (pos0 + torch.arange(T))[:, None]   # [T, n]
    s = s.masked_fill(mask[:, None, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1)
    z = torch.einsum("tkgn,knd->tkgd", p, v).reshape(T, H, head_dim)
    z = r16(z)
    if gate:
        z = r16(z * torch.sigmoid(qg[..., head_dim:].to(F32)))
    return z.to(F16)


def attention_prefill(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int,
                      scale: float, rows: slice | None = None, block: int = 512) -> torch.Tensor:
    """Causal GQA prefill (kernels.cu:2461-2807): q [T, 24, d] fp16, query t
    at position pos0 + t. `rows` limits the computed query rows (a bounded
    CPU sample). P is rounded to fp16 before P V, as the reference does.
    Runs on whatever device the tensors are on (fp32 matmuls over contiguous
    operands, blocks of `block` query rows)."""
    T, H, d = q.shape
    n_kv = kc.shape[1]
    G = H // n_kv
    dev = q.device
    rows = rows or slice(0, T)
    t_idx = torch.arange(T, device=dev)[rows]
    out = torch.empty((len(t_idx), H, d), dtype=F16, device=dev)
    for b0 in range(0, len(t_idx), block):
        tb = t_idx[b0:b0 + block]
        nb = len(tb)
        n = pos0 + int(tb[-1]) + 1
        # [kv, nb * G, d] query rows of each kv head; [kv, d, n] keys; [kv, n, d] values
        qb = q[tb].to(F32).view(nb, n_kv, G, d).permute(1, 0, 2, 3).reshape(n_kv, nb * G, d)
        kt = kc[:n].to(F32).permute(1, 2, 0).contiguous()
        v = vc[:n].to(F32).permute(1, 0, 2).contiguous()
        s = torch.matmul(qb.contiguous(), kt) * scale                    # [kv, nb * G, n]
        qpos = (pos0 + tb).repeat_interleave(G)                           # row (t, g) -> t
        mask = torch.arange(n, device=dev)[None, :] > qpos[:, None]
        s = s.masked_fill(mask[None], float("-inf"))
        m = s.amax(dim=-1, keepdim=True)
        p = torch.exp(s - m)
        l = p.sum(dim=-1, keepdim=True)
        o = torch.matmul(r16(p), v) / l                                    # [kv, nb * G, d]
        out[b0:b0 + nb] = r16(o).view(n_kv, nb, G, d).permute(1, 0, 2, 3).reshape(nb, H, d) \
            .to(F16)
    return out


# ---------------------------------------------------------------------------
# Gated DeltaNet
# ---------------------------------------------------------------------------

def gdn_decode_step(x: torch.Tensor, w: torch.Tensor, st_in: torch.Tensor, S: torch.Tensor,
                    a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor,
                    pos0: int, n_kheads: int = 16, K: int = 128, V: int = 128,
                    out_scale: float = 128 ** -0.5, l2eps: float = 1e-6):
    """One fused decode step of B sequences (kernels.cu:2916-3070 with the
    conv folded in): x [B, 10240] fp16 raw q|k|v rows, w [10240, 4] fp16,
    st_in [B, 10240, 3] fp16, S [B, 48, V, K] fp32 (updated in place),
    a, b [B, 48] fp32. Returns (y [B, 48*V] fp16, st_out [B, 10240, 3] fp16)."""
    B = x.shape[0]
    nv = S.shape[1]
    group = nv // n_kheads
    st = st_in.to(F32) * (1.0 if pos0 > 0 else 0.0)
    E = torch.cat([st, x.to(F32)[..., None]], dim=-1)          # [B, C, 4], tap 0 oldest
    acc = (E * w.to(F32)[None]).sum(-1)
    c = r16(acc * torch.sigmoid(acc))                           # silu, fp16
    st_out = E[..., 1:].to(F16)
    q = c[:, :n_kheads * K].view(B, n_kheads, K)
    k = c[:, n_kheads * K:2 * n_kheads * K].view(B, n_kheads, K)
    v = c[:, 2 * n_kheads * K:].view(B, nv, V)
    q = r16(q / torch.sqrt((q * q).sum(-1, keepdim=True) + l2eps))
    k = r16(k / torch.sqrt((k * k).sum(-1, keepdim=True) + l2eps))
    q = q.repeat_interleave(group, dim=1)                       # [B, nv, K]
    k = k.repeat_interleave(group, dim=1)
    beta = torch.sigmoid(b)
    xx = a + dt_bias
    sp = torch.where(xx <= 20.0, torch.log1p(torch.exp(xx.clamp(max=20.0))), xx)
    decay = torch.exp(-torch.exp(A_log) * sp)
    S.mul_(decay[..., None, None])
    m = torch.einsum("bhvk,bhk->bhv", S, k)
    delta = beta[..., None] * (v - m)
    S.add_(delta[..., :, None] * k[..., None, :])
    o = torch.einsum("bhvk,bhk->bhv", S, q)
    y = r16(o * out_scale).to(F16).reshape(B, nv * V)
    return y, st_out


def gdn_recurrence(q, k, v, beta, decay, S, group: int = 3, out_scale: float = 128 ** -0.5):
    """The delta rule token by token (kernels.cu:1755-1766): q, k [T, nk, K]
    fp16, v [T, nv, V] fp16, beta / decay [T, nv] fp32, S [nv, V, K] fp32 in
    place. Returns y [T, nv*V] fp16."""
    T = q.shape[0]
    nv = v.shape[1]
    ys = []
    qf = q.to(F32).repeat_interleave(group, dim=1)
    kf = k.to(F32).repeat_interleave(group, dim=1)
    vf = v.to(F32)
    for t in range(T):
        S.mul_(decay[t][:, None, None])
        m = torch.einsum("hvk,hk->hv", S, kf[t])
        delta = beta[t][:, None] * (vf[t] - m)
        S.add_(delta[:, :, None] * kf[t][:, None, :])
        ys.append(r16(torch.einsum("hvk,hk->hv", S, qf[t]) * out_scale).to(F16).reshape(nv * 128))
    return torch.stack(ys)


def gdn_chunked(q, k, v, beta, decay, S, group: int = 3, chunk: int = 64,
                out_scale: float = 128 ** -0.5):
    """The chunked WY/UT form of gdn_recurrence in fp32 (see the GPU kernel's
    header for the algebra). Same arguments and result."""
    T = q.shape[0]
    nv = v.shape[1]
    qf = q.to(F32).repeat_interleave(group, dim=1).transpose(0, 1)   # [nv, T, K]
    kf = k.to(F32).repeat_interleave(group, dim=1).transpose(0, 1)
    vf = v.to(F32).transpose(0, 1)                                   # [nv, T, V]
    y = torch.empty((T, nv, 128), dtype=F16)
    for c0 in range(0, T, chunk):
        n = min(chunk, T - c0)
        sl = slice(c0, c0 + n)
        Kc, Qc, Vc = kf[:, sl], qf[:, sl], vf[:, sl]
        bc = beta[sl].transpose(0, 1)                                # [nv, n]
        g = torch.cumsum(torch.log(decay[sl].clamp_min(1e-38)), dim=0).transpose(0, 1)
        diff = g[:, :, None] - g[:, None, :]
        tri = torch.tril(torch.ones(n, n, dtype=torch.bool))
        ratio = torch.where(tri, torch.exp(diff.masked_fill(~tri, 0.0)), torch.zeros(()))
        A = (bc[:, :, None] * ratio * (Kc @ Kc.transpose(1, 2))).tril(-1)
        eye = torch.eye(n).expand(nv, n, n)
        W = torch.linalg.solve_triangular(eye + A, (bc * torch.exp(g))[..., None] * Kc,
                                          upper=False, unitriangular=True)
        U = torch.linalg.solve_triangular(eye + A, bc[..., None] * Vc, upper=False,
                                          unitriangular=True)
        D = U - W @ S.transpose(1, 2)
        O = torch.exp(g)[..., None] * (Qc @ S.transpose(1, 2)) + (ratio * (Qc @ Kc.transpose(1, 2))) @ D
        y[sl] = r16(O * out_scale).to(F16).transpose(0, 1)
        gC = g[:, -1]
        S.mul_(torch.exp(gC)[:, None, None])
        S.add_(D.transpose(1, 2) @ (torch.exp(gC[:, None] - g)[..., None] * Kc))
    return y.reshape(T, nv * 128)


def threads() -> int:
    return torch.get_num_threads()


def set_threads(n: int | None = None) -> int:
    import os

    torch.set_num_threads(n or os.cpu_count() or 1)
    return torch.get_num_threads()


__all__ = ["attention_decode", "attention_prefill", "gdn_decode_step", "gdn_recurrence",
           "gdn_chunked", "threads", "set_threads", "math"]
