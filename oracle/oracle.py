"""CPU ORACLE wrapper (test infrastructure only).

numpy front end over ``liboracle.so`` (``fl_oracle.c``), the scalar C
restatement of the reference's attention / Gated DeltaNet kernels
(``model/footless/cuda_sm60/kernels.cu``). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this module, and only as the checker: the product path never calls it.

fp16 tensors are numpy ``float16`` arrays (passed to C as their uint16 bits);
fp32 tensors are ``float32`` arrays. Every function allocates its outputs and
returns them, except where the reference kernel updates a buffer in place
(``S`` of the GDN scans, the caches of ``kv_store``), which these functions
also update in place.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double
_LL = ctypes.c_longlong


def build(force: bool = False) -> Path:
    """Compile liboracle.so with the committed Makefile (gcc)."""
    import subprocess

    if force or not _LIB_PATH.exists() or (
            _LIB_PATH.stat().st_mtime < (_HERE / "fl_oracle.c").stat().st_mtime):
        subprocess.run(["make", "-s", "-B", "-C", str(_HERE), "liboracle.so"], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        sigs = {
            "orc_kv_store": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I],
            "orc_rmsnorm1p": [_P, _P, _P, _I, _I, _I, _I, _F],
            "orc_rope_partial": [_P, _P, _I, _I, _I, _I, _I, _I, _I, _D],
            "orc_rmsnorm_gated": [_P, _P, _P, _P, _I, _I, _I, _I, _F],
            "orc_attention_split": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _I],
            "orc_attention_merge": [_P, _P, _P, _P, _I, _I, _I, _I, _I],
            "orc_attn_gate": [_P, _P, _I, _I, _I, _I, _I, _I],
            "orc_attention_prefill": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I],
            "orc_attention_exact_f64": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _D, _I],
            "orc_kv_store_q8": [_P, _P, _P, _P, _I, _I, _I, _I, _I],
            "orc_attention_dec_q8": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _I],
            "orc_attention_dec_merge": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _I, _I],
            "orc_attention_prefill_q8": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I],
            "orc_attention_exact_f64_q8": [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _D, _I],
            "orc_conv1d_causal": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I],
            "orc_conv1d_causal_rows": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I],
            "orc_l2norm_scaled": [_P, _P, _I, _I, _I, _F, _F, _I],
            "orc_gdn_scalars": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I],
            "orc_gdn_scan": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _LL],
            "orc_gdn_decode": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _P, _LL,
                               _P, _P, _P, _P, _I, _F, _P, _P, _P, _P, _I],
            "orc_gdn_chunked": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _I, _I],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _I if name in ("orc_gdn_scan", "orc_gdn_decode", "orc_gdn_chunked") else None
        L.orc_dec_split_count.argtypes = [_I, _I, _I]
        L.orc_dec_split_count.restype = _I
        L.orc_f16_sat.argtypes = [_F]
        L.orc_f16_sat.restype = ctypes.c_uint16
        L.orc_det_expf.argtypes = [_F]
        L.orc_det_expf.restype = _F
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _h(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16)


def _rows(a, dtype=np.float16):
    """Pointer to a row view (inner dimension contiguous, any row stride):
    the reference's offset pointer + explicit stride. Never copies."""
    a = np.asarray(a)
    if a.dtype != dtype:
        raise TypeError(f"expected {np.dtype(dtype).name}, got {a.dtype}")
    if a.strides[-1] != a.itemsize:
        raise ValueError("row views must be contiguous along the last axis")
    return a.ctypes.data


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# --------------------------------------------------------------------------
# full attention
# --------------------------------------------------------------------------

def kv_store(k, v, kcache, vcache, layer, pos0, n_kv_heads, head_dim, max_pos, T):
    """kernels.cu:465-484. Updates kcache / vcache (float16) in place."""
    k, v = _h(k), _h(v)
    lib().orc_kv_store(_p(k), _p(v), _p(kcache), _p(vcache), layer, pos0, n_kv_heads,
                       head_dim, max_pos, T)


def rmsnorm1p(x, w, *, n=256, rows, pitch, T, eps=1e-6):
    """kernels.cu:241-272 over [T][rows] rows `pitch` halves apart; returns a new
    float16 array shaped like x (the elements past n of each pitch copied)."""
    x = _h(x)
    y = x.copy()
    lib().orc_rmsnorm1p(_p(x), _p(_f(w)), _p(y), n, rows, pitch, T, eps)
    return y


def rope_partial(q, k, *, n_q_heads, n_kv_heads, rope_dim=64, q_pitch, k_pitch, pos0, T,
                 theta=1e7):
    """kernels.cu:422-455; returns new (q, k) float16 arrays."""
    q, k = _h(q).copy(), _h(k).copy()
    lib().orc_rope_partial(_p(q), _p(k), n_q_heads, n_kv_heads, rope_dim, q_pitch, k_pitch,
                           pos0, T, float(theta))
    return q, k


def attn_prep(qg, k, v, wq, wk, kcache, vcache, *, pos0, T, n_q_heads=24, n_kv_heads=4,
              head_dim=256, q_pitch=512, layer=0, max_pos, rope_dim=64, theta=1e7, eps=1e-6):
    """The sequence runtime.py:2797-2815 launches: rmsnorm1p of q (inside qg)
    and of k, rope_partial of both, kv_store of the roped k and v. Returns
    (qg, k) as new arrays; kcache / vcache (float16) are updated in place."""
    qn = rmsnorm1p(qg, wq, n=head_dim, rows=n_q_heads, pitch=q_pitch, T=T, eps=eps)
    kn = rmsnorm1p(k, wk, n=head_dim, rows=n_kv_heads, pitch=head_dim, T=T, eps=eps)
    qr, kr = rope_partial(qn, kn, n_q_heads=n_q_heads, n_kv_heads=n_kv_heads, rope_dim=rope_dim,
                          q_pitch=q_pitch, k_pitch=head_dim, pos0=pos0, T=T, theta=theta)
    kv_store(kr, v, kcache, vcache, layer, pos0, n_kv_heads, head_dim, max_pos, T)
    return qr, kr


def attention_split(q, kcache, vcache, layer, n_q_heads, n_kv_heads, head_dim, q_pitch,
                    pos0, max_pos, scale, split_rows, T, split):
    """kernels.cu:522-835. Returns (pacc [T,H,split,D], pm [T,H,split], pd)."""
    q = _h(q)
    pacc = np.zeros((T, n_q_heads, split, head_dim), np.float32)
    pm = np.zeros((T, n_q_heads, split), np.float32)
    pd = np.zeros((T, n_q_heads, split), np.float32)
    lib().orc_attention_split(_p(q), _p(kcache), _p(vcache), _p(pacc), _p(pm), _p(pd), layer,
                              n_q_heads, n_kv_heads, head_dim, q_pitch, pos0, max_pos,
                              float(scale), split_rows, T, split)
    return pacc, pm, pd


def attention_merge(pacc, pm, pd, n_q_heads, head_dim, T, split, z_pitch=None):
    """kernels.cu:1398-1424. Returns z [T, n_q_heads, z_pitch] float16."""
    z_pitch = head_dim if z_pitch is None else z_pitch
    z = np.zeros((T, n_q_heads, z_pitch), np.float16)
    lib().orc_attention_merge(_p(_f(pacc)), _p(_f(pm)), _p(_f(pd)), _p(z), n_q_heads,
                              head_dim, z_pitch, T, split)
    return z


def attn_gate(z, g, n_heads, head_dim, z_pitch, g_pitch, g_off, T):
    """kernels.cu:1585-1600, in place on z (float16)."""
    lib().orc_attn_gate(_p(z), _p(_h(g)), n_heads, head_dim, z_pitch, g_pitch, g_off, T)


def attention_decode(qg, kcache, vcache, pos0, *, n_q_heads=24, n_kv_heads=4, head_dim=256,
                     q_pitch=512, max_pos, scale, split_rows=32, split=32, layer=0,
                     gate=True, g_off=256):
    """The decode / verify attention block of _full_attn (runtime.py:2828-2862):
    attention_split_gqa -> attention_merge -> attn_gate over one sequence's
    cache. qg [T, n_q_heads, q_pitch] float16 (q | gate per head). Returns
    z [T, n_q_heads, head_dim] float16."""
    qg = _h(qg)
    T = qg.shape[0]
    pacc, pm, pd = attention_split(qg, kcache, vcache, layer, n_q_heads, n_kv_heads, head_dim,
                                   q_pitch, pos0, max_pos, scale, split_rows, T, split)
    z = attention_merge(pacc, pm, pd, n_q_heads, head_dim, T, split)
    if gate:
        attn_gate(z, qg, n_q_heads, head_dim, head_dim, q_pitch, g_off, T)
    return z


def attention_prefill(q, kcache, vcache, *, layer=0, n_q_heads=24, n_kv_heads=4, head_dim=256,
                      q_pitch, pos0, max_pos, scale, T, pv_fp16=False):
    """kernels.cu:2461-2807 (KV split 1). Returns z [T, n_q_heads, head_dim] float16."""
    q = _h(q)
    z = np.zeros((T, n_q_heads, head_dim), np.float16)
    lib().orc_attention_prefill(_p(q), _p(kcache), _p(vcache), _p(z), layer, n_q_heads,
                                n_kv_heads, head_dim, q_pitch, head_dim, pos0, max_pos,
                                float(scale), T, 1 if pv_fp16 else 0)
    return z


def attention_exact(q, kcache, vcache, *, layer=0, n_q_heads=24, n_kv_heads=4, head_dim=256,
                    q_pitch, pos0, max_pos, scale, T):
    """Closed form: causal GQA softmax attention in float64."""
    q = _h(q)
    out = np.zeros((T, n_q_heads, head_dim), np.float64)
    lib().orc_attention_exact_f64(_p(q), _p(kcache), _p(vcache), _p(out), layer, n_q_heads,
                                  n_kv_heads, head_dim, q_pitch, pos0, max_pos, float(scale), T)
    return out


# --------------------------------------------------------------------------
# int8 KV cache
# --------------------------------------------------------------------------

def kv8_buffer(max_pos, n_kv_heads=4, head_dim=256):
    """An empty int8 cache buffer of capacity max_pos: values, then fp16 scales
    (kernels.cu:486-490), as flat int8."""
    return np.zeros(max_pos * n_kv_heads * (head_dim + 2 * head_dim // 32), np.int8)


def kv8_split(buf, max_pos, n_kv_heads=4, head_dim=256):
    """(values [max_pos, n_kv, head_dim] int8, scales [max_pos, n_kv, head_dim/32]
    float16) views of an int8 cache buffer."""
    nv = max_pos * n_kv_heads * head_dim
    vals = buf[:nv].reshape(max_pos, n_kv_heads, head_dim)
    scales = buf[nv:].view(np.float16).reshape(max_pos, n_kv_heads, head_dim // 32)
    return vals, scales


def kv_store_q8(k, v, kcache, vcache, pos0, max_pos, T, n_kv_heads=4, head_dim=256):
    """kernels.cu:486-520. Updates the int8 buffers kcache / vcache in place."""
    k, v = _h(k), _h(v)
    assert kcache.dtype == np.int8 and vcache.dtype == np.int8
    lib().orc_kv_store_q8(_p(k), _p(v), _p(kcache), _p(vcache), pos0, n_kv_heads, head_dim,
                          max_pos, T)


def attn_prep_q8(qg, k, v, wq, wk, kcache, vcache, *, pos0, T, max_pos, n_q_heads=24,
                 n_kv_heads=4, head_dim=256, q_pitch=512, rope_dim=64, theta=1e7, eps=1e-6):
    """attn_prep_q8 (kernels.cu:837-908): rmsnorm1p, rope_partial, kv_store_q8.
    Returns (qg, k) as new arrays; the int8 buffers are updated in place."""
    qn = rmsnorm1p(qg, wq, n=head_dim, rows=n_q_heads, pitch=q_pitch, T=T, eps=eps)
    kn = rmsnorm1p(k, wk, n=head_dim, rows=n_kv_heads, pitch=head_dim, T=T, eps=eps)
    qr, kr = rope_partial(qn, kn, n_q_heads=n_q_heads, n_kv_heads=n_kv_heads, rope_dim=rope_dim,
                          q_pitch=q_pitch, k_pitch=head_dim, pos0=pos0, T=T, theta=theta)
    kv_store_q8(kr, v, kcache, vcache, pos0, max_pos, T, n_kv_heads, head_dim)
    return qr, kr


def dec_split_count(length, tmin, smax):
    return lib().orc_dec_split_count(length, tmin, smax)


def attention_dec_q8(q, kcache, vcache, *, pos0, max_pos, sl2, tmin=1, smax=28, T,
                     n_q_heads=24, n_kv_heads=4, q_pitch=512):
    """kernels.cu:1049-1335. Returns (pacc [T,H,smax,256], pm, pd); partials the
    reference does not write stay NaN."""
    q = _h(q)
    pacc = np.full((T, n_q_heads, smax, 256), np.nan, np.float32)
    pm = np.full((T, n_q_heads, smax), np.nan, np.float32)
    pd = np.full((T, n_q_heads, smax), np.nan, np.float32)
    lib().orc_attention_dec_q8(_p(q), _p(kcache), _p(vcache), _p(pacc), _p(pm), _p(pd),
                               n_q_heads, n_kv_heads, q_pitch, pos0, max_pos, float(sl2), tmin,
                               smax, T)
    return pacc, pm, pd


def attention_dec_merge(pacc, pm, pd, *, pos0, tmin=1, smax=28, T, n_q_heads=24, gate=None,
                        g_pitch=512, g_off=256):
    """kernels.cu:1336-1385 (the _gate form when gate is given). Returns z
    [T, n_q_heads, 256] float16."""
    z = np.zeros((T, n_q_heads, 256), np.float16)
    g = None if gate is None else _h(gate)
    lib().orc_attention_dec_merge(_p(_f(pacc)), _p(_f(pm)), _p(_f(pd)), _p(z), n_q_heads, 256,
                                  pos0, tmin, smax, T, _p(g), g_pitch, g_off)
    return z


def attention_decode_q8(qg, kcache, vcache, pos0, *, max_pos, scale, tmin=1, smax=28,
                        n_q_heads=24, n_kv_heads=4, q_pitch=512, gate=True, g_off=256):
    """_attn_dec with the gate (runtime.py:2907-2920): attention_dec_q8 then
    attention_dec_merge_gate over one sequence's int8 cache. Returns z
    [T, n_q_heads, 256] float16."""
    qg = _h(qg)
    T = qg.shape[0]
    pacc, pm, pd = attention_dec_q8(qg, kcache, vcache, pos0=pos0, max_pos=max_pos,
                                    sl2=scale * 1.4426950408889634, tmin=tmin, smax=smax, T=T,
                                    n_q_heads=n_q_heads, n_kv_heads=n_kv_heads, q_pitch=q_pitch)
    return attention_dec_merge(pacc, pm, pd, pos0=pos0, tmin=tmin, smax=smax, T=T,
                               n_q_heads=n_q_heads, gate=qg if gate else None, g_pitch=q_pitch,
                               g_off=g_off)


def attention_prefill_q8(q, kcache, vcache, *, n_q_heads=24, n_kv_heads=4, head_dim=256,
                         q_pitch, pos0, max_pos, scale, T, pv_fp16=False):
    """kernels.cu:2778-2786 (KV split 1). Returns z [T, n_q_heads, head_dim] float16."""
    q = _h(q)
    z = np.zeros((T, n_q_heads, head_dim), np.float16)
    lib().orc_attention_prefill_q8(_p(q), _p(kcache), _p(vcache), _p(z), n_q_heads, n_kv_heads,
                                   head_dim, q_pitch, head_dim, pos0, max_pos, float(scale), T,
                                   1 if pv_fp16 else 0)
    return z


def attention_exact_q8(q, kcache, vcache, *, n_q_heads=24, n_kv_heads=4, head_dim=256, q_pitch,
                       pos0, max_pos, scale, T):
    """Closed form over an int8 cache (values dequantized exactly), float64."""
    q = _h(q)
    out = np.zeros((T, n_q_heads, head_dim), np.float64)
    lib().orc_attention_exact_f64_q8(_p(q), _p(kcache), _p(vcache), _p(out), n_q_heads,
                                     n_kv_heads, head_dim, q_pitch, pos0, max_pos, float(scale), T)
    return out


# --------------------------------------------------------------------------
# Gated DeltaNet
# --------------------------------------------------------------------------

def conv1d_causal(x, w, st_in, *, dim, T, pos0, row_stride, width=4):
    """kernels.cu:1634-1679. Returns (y like x, st_out [dim, width-1])."""
    x, w, st_in = _h(x), _h(w), _h(st_in)
    y = np.zeros_like(x)
    st_out = np.zeros_like(st_in)
    lib().orc_conv1d_causal(_p(x), _p(w), _p(st_in), _p(y), _p(st_out), dim, T, pos0,
                            row_stride, width)
    return y, st_out


def conv1d_causal_rows(x, w, st_in, *, dim, T, pos0, row_stride):
    """kernels.cu:1686-1714. Returns (y, [st0, st1, st2][:T])."""
    x, w, st_in = _h(x), _h(w), _h(st_in)
    y = np.zeros_like(x)
    sts = [np.zeros_like(st_in) for _ in range(3)]
    lib().orc_conv1d_causal_rows(_p(x), _p(w), _p(st_in), _p(y), _p(sts[0]), _p(sts[1]),
                                 _p(sts[2]), dim, T, pos0, row_stride)
    return y, sts[:T]


def l2norm_scaled(x, *, n, rows, pitch, eps, scale, T):
    """kernels.cu:373-391. Returns y like x (only the n-wide rows written)."""
    x = _h(x)
    y = np.zeros_like(x)
    lib().orc_l2norm_scaled(_p(x), _p(y), n, rows, pitch, float(eps), float(scale), T)
    return y


def rmsnorm_gated(o, z, w, *, n=128, rows=48, pitch=128, T, eps=1e-6):
    """kernels.cu:335-358 over [T][rows] rows of `pitch` halves; returns y."""
    o, z = _h(o), _h(z)
    y = np.zeros_like(o)
    lib().orc_rmsnorm_gated(_p(o), _p(z), _p(_f(w)), _p(y), n, rows, pitch, T, eps)
    return y


def gdn_scalars(a, b, A_log, dt_bias, *, T, n_heads, a_stride=None, b_stride=None):
    """kernels.cu:1732-1748. Returns (beta [T, n_heads], decay [T, n_heads])."""
    a, b, A_log, dt_bias = _f(a), _f(b), _f(A_log), _f(dt_bias)
    beta = np.zeros((T, n_heads), np.float32)
    decay = np.zeros((T, n_heads), np.float32)
    lib().orc_gdn_scalars(_p(a), _p(b), _p(A_log), _p(dt_bias), _p(beta), _p(decay), T,
                          n_heads, a_stride or n_heads, b_stride or n_heads)
    return beta, decay


def gdn_scan(q, k, v, beta, decay, S, *, T, n_kheads=16, n_vheads=48, K=128, V=128,
             qk_stride, v_stride, y_stride=None, out_scale, group=3, ck=None, ck_step=0):
    """kernels.cu:1794-1901 / 2831-2914. S (float32 [n_vheads, V, K]) in place.
    q, k, v are row views (float16, rows at qk_stride / v_stride elements).
    Returns y [T, y_stride] float16."""
    y_stride = n_vheads * V if y_stride is None else y_stride
    y = np.zeros((T, y_stride), np.float16)
    rc = lib().orc_gdn_scan(_rows(q), _rows(k), _rows(v), _p(_f(beta)), _p(_f(decay)),
                            _p(S), _p(y), T, n_kheads, n_vheads, K, V, qk_stride, v_stride,
                            y_stride, float(out_scale), group, _p(ck), ck_step)
    assert rc == 0, "orc_gdn_scan rejected the geometry"
    return y


def gdn_decode(c, S, a, b, A_log, dt_bias, *, T, n_kheads=16, n_vheads=48, K=128, V=128,
               row=10240, out_scale, group=3, ab_stride=48, l2eps=1e-6, ck=None, ck_step=0,
               cx=None, cw=None, cst_in=None, cst_out=None, pos0=0):
    """kernels.cu:2943-3070 (gdn_scan_rows_f). `c` the conv'd q|k|v rows
    [T, row] (ignored when cx is given: the raw row, conv fused, T = 1).
    S in place; cst_out (conv fused) in place. Returns y [T, n_vheads*V]."""
    y = np.zeros((T, n_vheads * V), np.float16)
    c = _h(c) if c is not None else _h(cx)
    # the reference's offsets into the q|k|v row (runtime.py:3044-3045): q at c,
    # k at c + n_kheads*K elements, v at c + 2*n_kheads*K (2 bytes an element)
    base = c.ctypes.data
    rc = lib().orc_gdn_decode(base, base + 2 * n_kheads * K, base + 2 * 2 * n_kheads * K,
                              _p(S), _p(y), T, n_kheads, n_vheads, K, V, row, row,
                              n_vheads * V, float(out_scale), group, _p(ck), ck_step,
                              _p(_f(a)), _p(_f(b)), _p(_f(A_log)), _p(_f(dt_bias)), ab_stride,
                              float(l2eps), _p(_h(cx)) if cx is not None else None,
                              _p(_h(cw)) if cw is not None else None,
                              _p(_h(cst_in)) if cst_in is not None else None,
                              _p(cst_out), pos0)
    assert rc == 0, "orc_gdn_decode rejected the geometry"
    return y


def gdn_chunked(q, k, v, beta, decay, S, *, T, n_kheads=16, n_vheads=48, K=128, V=128,
                qk_stride, v_stride, out_scale, group=3, chunk=64):
    """The chunked WY/UT scan (not in the reference), in float64. S in place.
    Returns y [T, n_vheads*V] float16."""
    y = np.zeros((T, n_vheads * V), np.float16)
    rc = lib().orc_gdn_chunked(_rows(q), _rows(k), _rows(v), _p(_f(beta)), _p(_f(decay)),
                               _p(S), _p(y), T, n_kheads, n_vheads, K, V, qk_stride, v_stride,
                               n_vheads * V, float(out_scale), group, chunk)
    assert rc == 0, "orc_gdn_chunked rejected the geometry"
    return y


def det_expf(x: float) -> float:
    return lib().orc_det_expf(float(x))


def f16_sat(x: float) -> np.float16:
    bits = lib().orc_f16_sat(float(x))
    return np.array([bits], np.uint16).view(np.float16)[0]


__all__ = [n for n in dir() if not n.startswith("_")]
del os
