// Gated DeltaNet decode / recurrent path for gfx950: causal conv1d, the q/k
// L2 norm, the beta / decay gates, the gated delta rule, and the fused
// batched decode step.
//
// Reference behaviour restated (model/footless/cuda_sm60/kernels.cu):
//   conv1d_causal        1606-1679  E = [state | x], y = silu(w . E), state tail
//   conv1d_causal_rows   1681-1714  verify rows with a state per row
//   l2norm_scaled         360-391   y = x / sqrt(sum x^2 + eps) * scale
//   gdn_scalars          1716-1748  beta = sigmoid(b), decay = exp(-e^A softplus)
//   gdn_scan(_rows)      1750-1901, 2809-2914   the delta rule, S in place
//   gdn_scan_rows_f      2943-3070  the fused decode / verify step
//
// State layout: S [n_vheads][V rows][K cols] fp32, a head is 64 KiB. The
// delta-rule kernels give a state row 8 lanes (16 columns a lane = four
// float4 at columns c0 + 32j, c0 = 4 (lane % 8)), so each 8-lane group reads
// a row's 128 contiguous bytes per load and the row's dot products reduce
// inside the group with DPP (quad_perm xor 1, xor 2, then the half-row
// mirror); a wavefront holds 8 rows. The rows' state stays in registers for
// the whole call: loaded once, stored once.
#include "fl_common.hpp"

#pragma clang fp contract(off)

#include "gdn_gates.hpp"

namespace {

constexpr int GR_ROWS = 32;       // state rows a workgroup
constexpr int GR_THREADS = 256;   // 8 lanes a row
constexpr int GR_K = 128;

// Sum over the 8 lanes of a row group; every lane gets the same bits.
__device__ __forceinline__ float row8_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
    return v;
}

// Sum of squares over a 128-thread row in the reference's order (kernels.cu:
// 214-227, block_reduce_sum over 4 warps of 32): a tree inside each 32-lane
// half of the wavefront (lane 0 of the half ends with the warp's sum), the
// four warp sums then combined as (r0 + r2) + (r1 + r3). `red` holds 8 floats;
// `w0` is the first of the row's four 32-lane warps. Every thread gets the
// total. Matching the order keeps the fp16-rounded normalised values
// identical to the oracle's.
__device__ __forceinline__ float warp32_tree(float v) {
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v += lane_xor(v, o);
    return v;
}

// One token of the delta rule on a lane's 16 columns (`reg`), with k and q
// (fp32 values of fp16 numbers) at columns c0 + 32j + 0..3: delta_update
// updates the state, delta_out returns the row's output o = S_new . q
// (identical in the 8 lanes of the row). The dots run in two chains (even /
// odd register) summed, then over the row's lanes -- the reference's
// gdn_scan_rows order (kernels.cu:2866-2905).
__device__ __forceinline__ void delta_update(float (&reg)[16], const float* kk, float vt, float bt,
                                             float dt) {
    float m0 = 0.f, m1 = 0.f;
#pragma unroll
    for (int c = 0; c < 16; c += 2) {
        reg[c] = reg[c] * dt;
        reg[c + 1] = reg[c + 1] * dt;
        m0 = fmaf(reg[c], kk[c], m0);
        m1 = fmaf(reg[c + 1], kk[c + 1], m1);
    }
    const float m = row8_sum(m0 + m1);
    const float delta = bt * (vt - m);
#pragma unroll
    for (int c = 0; c < 16; ++c) reg[c] = fmaf(delta, kk[c], reg[c]);
}

__device__ __forceinline__ float delta_out(const float (&reg)[16], const float* qq) {
    float o0 = 0.f, o1 = 0.f;
#pragma unroll
    for (int c = 0; c < 16; c += 2) {
        o0 = fmaf(reg[c], qq[c], o0);
        o1 = fmaf(reg[c + 1], qq[c + 1], o1);
    }
    return row8_sum(o0 + o1);
}

__device__ __forceinline__ float delta_rule_token(float (&reg)[16], const float* kk,
                                                  const float* qq, float vt, float bt, float dt) {
    delta_update(reg, kk, vt, bt, dt);
    return delta_out(reg, qq);
}

__device__ __forceinline__ void load_row16(float (&reg)[16], const float* src) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f32x4 v4 = *(const f32x4*)(src + 32 * j);
        reg[4 * j] = v4[0];
        reg[4 * j + 1] = v4[1];
        reg[4 * j + 2] = v4[2];
        reg[4 * j + 3] = v4[3];
    }
}

__device__ __forceinline__ void store_row16(float* dst, const float (&reg)[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
        *(f32x4*)(dst + 32 * j) = (f32x4){reg[4 * j], reg[4 * j + 1], reg[4 * j + 2], reg[4 * j + 3]};
}

// gather a lane's 16 columns of a staged 128-wide fp32 row
__device__ __forceinline__ void gather16(float (&dst)[16], const float* row, int c0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f32x4 v4 = *(const f32x4*)(row + c0 + 32 * j);
        dst[4 * j] = v4[0];
        dst[4 * j + 1] = v4[1];
        dst[4 * j + 2] = v4[2];
        dst[4 * j + 3] = v4[3];
    }
}

// ---------------------------------------------------------------------------
// Causal conv over a run of tokens (a8) and a verify's rows (a9): one
// "sliding window" kernel. A lane owns CPL adjacent channels -- 8 (one
// 16-byte load of a token's row, one 16-byte store of y) when the layout
// allows it, else 1 -- and a block of TB consecutive tokens. It requests
// all of its block's rows first, then slides a register window of the W - 1
// previous frames down them, so each x value is read from HBM once (a
// block's W - 1 leading frames are the previous block's last rows, which L2
// already holds) instead of once per tap. A workgroup is one wavefront:
// 64 CPL channels of one token block; blockIdx.y is the token block.
//
// The taps add oldest first from zero (acc = fma(w_j, E_j, acc)), the order
// the reference's per-channel loop uses (kernels.cu:1659-1668), so y and the
// frames match its values bit for bit. E = [the stored W - 1 frames (zero at
// pos0 == 0) | x]: the window of block t0 starts as E[t0 .. t0 + W - 2] and
// after the call's last token is E[T .. T + W - 2], the new stored state.
// ROWS (a verify, T <= 3): the window after token t goes to the t-th state
// buffer, and a frame entering the window is rounded by f16_sat first, as the
// reference's row form does (kernels.cu:1704-1711).
// ---------------------------------------------------------------------------
// Tokens a lane: CONV_TB (the window's W - 1 history frames come from the
// rows before the block, so at least W - 1: 8 for widths 6..8), halved to 2
// for widths up to 3 while the grid has fewer than CONV_WAVES_PER_SIMD waves
// a SIMD. A lane's work is its block's silu chain (~36 vector instructions a
// token and channel), and a wave keeps its SIMD busy on its own, so a call
// takes as long as the SIMD with the most waves, and a short block keeps the
// grid even: at 10240 channels (W = 4) blocks of 16 / 8 / 4 tokens measured
// 25 / 17 / 17 us at T = 1024 (16 tokens: 1280 waves for 1024 SIMDs, a
// quarter of them running two in turn), 28.5 / 28.5 / 26.3 at 2048 and
// 96 / 91 / 91 at 8192.
constexpr int CONV_TB = 4;
constexpr int CONV_TB_MIN = 2;
constexpr int CONV_WAVES_PER_SIMD = 4;
constexpr int CONV_WMAX = 8;      // widths 1 .. 8

template <int CPL> struct ConvVec;
template <> struct ConvVec<8> { typedef f16x8 type; };
template <> struct ConvVec<1> { typedef f16 type; };

template <int CPL>
__device__ __forceinline__ float cv_get(const typename ConvVec<CPL>::type& v, int i) {
    if constexpr (CPL == 8) return (float)v[i];
    else return (float)v;
}
template <int CPL>
__device__ __forceinline__ void cv_set(typename ConvVec<CPL>::type& v, int i, f16 h) {
    if constexpr (CPL == 8) v[i] = h;
    else v = h;
}

// N consecutive fp16 values at p as floats: N / 8 16-byte loads when VEC
// (N a multiple of 8, p 16-byte aligned), else N 2-byte loads.
template <int N, bool VEC>
__device__ __forceinline__ void halves_in(float (&f)[N], const f16* p) {
    if constexpr (VEC) {
        static_assert(N % 8 == 0, "whole vectors");
#pragma unroll
        for (int m = 0; m < N / 8; ++m) {
            const f16x8 v = *(const f16x8*)(p + 8 * m);
#pragma unroll
            for (int i = 0; i < 8; ++i) f[8 * m + i] = (float)v[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) f[i] = (float)p[i];
    }
}

// The window [frame][channel] stored as the state layout [channel][frame].
template <int H, int CPL>
__device__ __forceinline__ void frames_out(f16* p, const float (&win)[H][CPL]) {
    if constexpr (CPL == 8) {
#pragma unroll
        for (int m = 0; m < H; ++m) {
            f16x8 v;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int flat = 8 * m + i;   // channel flat / H, frame flat % H
                v[i] = f16_sat(win[flat % H][flat / H]);
            }
            *(f16x8*)(p + 8 * m) = v;
        }
    } else {
#pragma unroll
        for (int j = 0; j < H; ++j) p[j] = f16_sat(win[j][0]);
    }
}

struct ConvStates {
    f16* st[3];   // the new state (st[0]), or a verify's one state a row
};

template <int W, int CPL, bool ROWS, int TB>
__global__ void __launch_bounds__(64)
conv_window_kernel(const f16* __restrict__ x, const f16* __restrict__ w, const f16* st_in,
                   f16* __restrict__ y, ConvStates outs, int dim, int T, int pos0,
                   int row_stride) {
    typedef typename ConvVec<CPL>::type vec;
    constexpr bool VEC = CPL == 8;
    constexpr int H = W - 1;          // frames of history
    constexpr int HW = H > 0 ? H : 1;
    static_assert(TB >= H, "a block's leading frames are the previous block's rows");
    constexpr int NTOK = ROWS ? 3 : TB;   // a verify has at most 3 rows
    const int d = (blockIdx.x * 64 + threadIdx.x) * CPL;
    if (d >= dim) return;
    const int t0 = blockIdx.y * TB;
    const int nt = min(NTOK, T - t0);
    // the block's rows, all requested before any arithmetic (a row past the
    // call re-reads the last one and is not used)
    vec xr[NTOK];
#pragma unroll
    for (int i = 0; i < NTOK; ++i)
        xr[i] = *(const vec*)(x + (size_t)min(t0 + i, T - 1) * row_stride + d);
    float taps[CPL * W];   // [channel][tap]
    halves_in<CPL * W, VEC>(taps, w + (size_t)d * W);
    float win[HW][CPL];
    if constexpr (H > 0) {
        if (t0 == 0) {
            float hist[CPL * H];   // [channel][frame]
            halves_in<CPL * H, VEC>(hist, st_in + (size_t)d * H);
            const bool keep = pos0 > 0;
#pragma unroll
            for (int j = 0; j < H; ++j)
#pragma unroll
                for (int c = 0; c < CPL; ++c) win[j][c] = keep ? hist[c * H + j] : 0.f;
        } else {
#pragma unroll
            for (int j = 0; j < H; ++j) {
                const vec r = *(const vec*)(x + (size_t)(t0 - H + j) * row_stride + d);
#pragma unroll
                for (int c = 0; c < CPL; ++c) win[j][c] = cv_get<CPL>(r, c);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NTOK; ++i) {
        if (i >= nt) continue;   // uniform; keeps the trip count constant (full unroll)
        vec out;
        float xf[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            xf[c] = cv_get<CPL>(xr[i], c);
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < H; ++j) acc = fmaf(taps[c * W + j], win[j][c], acc);
            acc = fmaf(taps[c * W + H], xf[c], acc);
            cv_set<CPL>(out, c, f16_sat(silu_f(acc)));
        }
        *(vec*)(y + (size_t)(t0 + i) * row_stride + d) = out;
        if constexpr (H > 0) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
#pragma unroll
                for (int j = 0; j + 1 < H; ++j) win[j][c] = win[j + 1][c];
                win[H - 1][c] = ROWS ? (float)f16_sat(xf[c]) : xf[c];
            }
            if constexpr (ROWS) frames_out<H, CPL>(outs.st[i] + (size_t)d * H, win);
        }
    }
    if constexpr (!ROWS && H > 0)
        if (t0 + nt == T) frames_out<H, CPL>(outs.st[0] + (size_t)d * H, win);
}

// The block length for a call: CONV_TB, or the smallest power of two >= W - 1
// where that is longer; then halved while the grid is short of
// CONV_WAVES_PER_SIMD waves a SIMD and the block stays >= max(2, W - 1).
int conv_tb(int W, int T, int channel_waves, int n_cu) {
    const long long want = (long long)CONV_WAVES_PER_SIMD * 4 * n_cu;
    int tb = CONV_TB;
    while (tb < W - 1) tb *= 2;
    while (tb / 2 >= CONV_TB_MIN && tb / 2 >= W - 1 &&
           (long long)channel_waves * ((T + tb - 1) / tb) < want)
        tb /= 2;
    return tb;
}

template <int W, int CPL, int TB>
void conv_launch_tb(bool rows, int tok_blocks, const f16* x, const f16* w, const f16* st_in,
                    f16* y, ConvStates outs, int dim, int T, int pos0, int row_stride,
                    hipStream_t stream) {
    const dim3 grid((dim + 64 * CPL - 1) / (64 * CPL), tok_blocks);
    if constexpr (TB >= W - 1) {
        if (rows) {   // the verify form: width 4, one block of CONV_TB (T <= 3)
            static_assert(CONV_TB >= 3, "a verify's rows are one block");
            if constexpr (W == 4 && TB == CONV_TB)
                hipLaunchKernelGGL((conv_window_kernel<W, CPL, true, TB>), grid, dim3(64), 0,
                                   stream, x, w, st_in, y, outs, dim, T, pos0, row_stride);
        } else {
            hipLaunchKernelGGL((conv_window_kernel<W, CPL, false, TB>), grid, dim3(64), 0, stream,
                               x, w, st_in, y, outs, dim, T, pos0, row_stride);
        }
    }
}

template <int W>
void conv_launch(bool vec, bool rows, int tb, const f16* x, const f16* w, const f16* st_in,
                 f16* y, ConvStates outs, int dim, int T, int pos0, int row_stride,
                 hipStream_t stream) {
    const int blocks = (T + tb - 1) / tb;
#define FL_CONV_TB(TBv)                                                                        \
    case TBv:                                                                                  \
        if (vec)                                                                               \
            conv_launch_tb<W, 8, TBv>(rows, blocks, x, w, st_in, y, outs, dim, T, pos0,        \
                                      row_stride, stream);                                     \
        else                                                                                   \
            conv_launch_tb<W, 1, TBv>(rows, blocks, x, w, st_in, y, outs, dim, T, pos0,        \
                                      row_stride, stream);                                     \
        break;
    switch (tb) {
        FL_CONV_TB(8) FL_CONV_TB(4) FL_CONV_TB(2)
        default: break;
    }
#undef FL_CONV_TB
}

// ---------------------------------------------------------------------------
// L2 norm for any row length n <= 1024 and pitch (the layouts the 16-lane row
// kernel below does not take): one wavefront a row, four rows a workgroup, no
// LDS and no barrier. The reference's 128-thread block (kernels.cu:373-391)
// lets thread v sum x[v], x[v + 128], ... in order, reduces each warp by a
// shuffle-down tree and combines the warp sums as (r0 + r2) + (r1 + r3).
// Lane l here runs two of those threads, l and l + 64, as two running sums;
// the warp trees become butterflies inside each 32-lane half (a lane and its
// partner add the same two values, a + b == b + a, so every lane ends with
// its half's tree sum), after which a lane below 32 holds r0 and r2, a lane
// above r1 and r3; their sums meet in one exchange at distance 32. The same
// additions in the same order, so the bits of the row kernel and the oracle.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
l2norm_wave_kernel(const f16* __restrict__ x, f16* __restrict__ y, int n, int rows, int pitch,
                   int n_rows, float eps, float scale) {
    const int lane = threadIdx.x & 63;
    const int rid = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (rid >= n_rows) return;                        // wave-uniform
    const size_t off = (size_t)rid * pitch;           // rid = t rows + r
    const f16* xr = x + off;
    f16* yr = y + off;
    float lo = 0.f, hi = 0.f;                         // threads `lane` and `lane + 64`
    for (int i = lane; i < n; i += 128) {
        const float a = (float)xr[i];
        lo = fmaf(a, a, lo);
        if (i + 64 < n) {
            const float b = (float)xr[i + 64];
            hi = fmaf(b, b, hi);
        }
    }
    lo = warp32_tree(lo);                             // r0 (lanes < 32) or r1
    hi = warp32_tree(hi);                             // r2 or r3
    const float pair = lo + hi;
    const float den = sqrtf((pair + lane_xor(pair, 32)) + eps);
    for (int i = lane; i < n; i += 64) yr[i] = f16_sat(((float)xr[i] / den) * scale);
}

// ---------------------------------------------------------------------------
// gates
// ---------------------------------------------------------------------------
__global__ void gdn_scalars_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                   const float* __restrict__ A_log,
                                   const float* __restrict__ dt_bias, float* __restrict__ beta,
                                   float* __restrict__ decay, int n_heads, int a_stride,
                                   int b_stride) {
    const int t = blockIdx.y;
    const int h = blockIdx.x * blockDim.x + threadIdx.x;
    if (h >= n_heads) return;
    beta[(size_t)t * n_heads + h] = gdn_beta(b[(size_t)t * b_stride + h]);
    decay[(size_t)t * n_heads + h] = gdn_decay(a[(size_t)t * a_stride + h] + dt_bias[h], A_log[h]);
}

// ---------------------------------------------------------------------------
// The delta rule over T tokens (a12): one wavefront per 8 state rows of a v
// head, no LDS and no barrier. Each lane reads the operands of its own
// columns straight from global memory -- k and q at columns c0 + 32 j + 0..3
// (four 8-byte loads each; the 16 wavefronts of a head share them in L2), its
// row's v, the head's beta and decay -- SCAN_AHEAD tokens before it computes
// with them, from a ring of registers, so the loads of later tokens are in
// flight under the dependent chain of the current one. The rows' state stays
// in registers from the first token to the last. Workgroups are mapped so
// that the row blocks of neighbouring v heads (which read the same k / q
// rows) run on one XCD, i.e. share one L2.
// grid n_vheads * V / 8 workgroups of 64.
// ---------------------------------------------------------------------------
constexpr int SCAN_AHEAD = 4;

struct ScanOps {
    f16x4 k[4], q[4];
    float v, beta, decay;
};

// 0, in a VGPR the compiler cannot see through: an index plus this makes a
// uniform load a vector load (scalar loads complete out of order, so waiting
// for one would also wait for every later-issued scalar load)
__device__ __forceinline__ int opaque_zero() {
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    return z;
}

__device__ __forceinline__ ScanOps scan_fetch(const f16* __restrict__ q, const f16* __restrict__ k,
                                              const f16* __restrict__ v,
                                              const float* __restrict__ beta,
                                              const float* __restrict__ decay, int t,
                                              size_t qk_off, size_t v_off, int hv_vz,
                                              int qk_stride, int v_stride, int n_vheads) {
    ScanOps o;
    const size_t qk = (size_t)t * qk_stride + qk_off;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        o.k[j] = *(const f16x4*)(k + qk + 32 * j);
        o.q[j] = *(const f16x4*)(q + qk + 32 * j);
    }
    o.v = (float)v[(size_t)t * v_stride + v_off];
    o.beta = beta[(size_t)t * n_vheads + hv_vz];
    o.decay = decay[(size_t)t * n_vheads + hv_vz];
    return o;
}

__global__ void __launch_bounds__(64)
gdn_scan_kernel(const f16* __restrict__ q, const f16* __restrict__ k, const f16* __restrict__ v,
                const float* __restrict__ beta, const float* __restrict__ decay,
                float* __restrict__ S, f16* __restrict__ y, int T, int n_vheads, int V,
                int qk_stride, int v_stride, int y_stride, float out_scale, int group,
                float* __restrict__ Ck, long long ck_step) {
    const int rbs = V / 8;   // row blocks a head
    const int nb = n_vheads * rbs;
    int blk = blockIdx.x;
    if (nb % 8 == 0) blk = (blk % 8) * (nb / 8) + blk / 8;   // XCD blk % 8 takes a run of heads
    const int hv = blk / rbs, rb = blk - hv * rbs;
    const int lane = threadIdx.x, c0 = 4 * (lane & 7);
    const int vi = rb * 8 + (lane >> 3);
    const size_t row = (size_t)hv * V + vi;
    float* Srow = S + row * GR_K + c0;
    const size_t qk_off = (size_t)(hv / group) * GR_K + c0;
    const int hv_vz = hv + opaque_zero();
    float reg[16];
    load_row16(reg, Srow);
    ScanOps ring[SCAN_AHEAD];
#pragma unroll
    for (int i = 0; i < SCAN_AHEAD; ++i)
        ring[i] = scan_fetch(q, k, v, beta, decay, min(i, T - 1), qk_off, row, hv_vz, qk_stride,
                             v_stride, n_vheads);
    for (int t0 = 0; t0 < T; t0 += SCAN_AHEAD) {
#pragma unroll
        for (int i = 0; i < SCAN_AHEAD; ++i) {
            const int t = t0 + i;
            if (t >= T) break;
            const ScanOps cur = ring[i];
            ring[i] = scan_fetch(q, k, v, beta, decay, min(t + SCAN_AHEAD, T - 1), qk_off, row,
                                 hv_vz, qk_stride, v_stride, n_vheads);
            float kk[16], qq[16];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    kk[4 * j + e] = (float)cur.k[j][e];
                    qq[4 * j + e] = (float)cur.q[j][e];
                }
            delta_update(reg, kk, cur.v, cur.beta, cur.decay);
            if (Ck != nullptr && t < T - 1) store_row16(Ck + (size_t)t * ck_step + row * GR_K + c0, reg);
            const float o = delta_out(reg, qq);
            if (c0 == 0) y[(size_t)t * y_stride + row] = f16_sat(o * out_scale);
        }
    }
    store_row16(Srow, reg);
}

// ---------------------------------------------------------------------------
// the fused decode / verify step of B sequences.
// grid (V / 32, n_vheads, B), block 256.
// ---------------------------------------------------------------------------
struct GdnSeqs {
    float* S[FL_MAX_SEQS];
    const f16* cst_in[FL_MAX_SEQS];
    f16* cst_out[FL_MAX_SEQS];
    float* Ck[FL_MAX_SEQS];
    int pos0[FL_MAX_SEQS];
};

__device__ __forceinline__ void load_row16_nt(float (&reg)[16], const float* src) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f32x4 v4 = __builtin_nontemporal_load((const f32x4*)(src + 32 * j));
        reg[4 * j] = v4[0];
        reg[4 * j + 1] = v4[1];
        reg[4 * j + 2] = v4[2];
        reg[4 * j + 3] = v4[3];
    }
}

__device__ __forceinline__ void store_row16_nt(float* dst, const float (&reg)[16]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
        __builtin_nontemporal_store((f32x4){reg[4 * j], reg[4 * j + 1], reg[4 * j + 2], reg[4 * j + 3]},
                                    (f32x4*)(dst + 32 * j));
}

// warp32_tree's value at lanes 0 and 32 (other lanes: partial sums) without
// LDS-pipe exchanges: lane i pairs with i + 16 (v_permlane16_swap, gfx950:
// with both operands v it returns rows (0, 0, 2, 2) and (1, 1, 3, 3) of v, so
// their sum at lane i of rows 0 and 2 is v[i] + v[i + 16]), then with i + 8,
// 4, 2, 1 inside its 16-lane row (DPP row_shl, a VALU operand modifier). At
// lanes 0 and 32 these are the pairs of the xor tree (x ^ d == x + d there),
// added in the same order.
template <int D>
__device__ __forceinline__ float dpp_shl(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + D, 0xF, 0xF, true));
}
__device__ __forceinline__ float warp32_tree_lane0(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    v += dpp_shl<8>(v);
    v += dpp_shl<4>(v);
    v += dpp_shl<2>(v);
    v += dpp_shl<1>(v);
    return v;
}

// conv1_ch split in two so the loads can be issued ahead of the state's: the
// raw fp16 values are kept until conv1_apply, after the state loads are
// issued, so no wait for them lands in front of those loads.
struct ConvIn {
    f16 h0, h1, h2, x;
    f16x4 w;
};

// The ring is read unconditionally (the buffer is always there) and zeroed
// by a select in conv1_apply when pos0 == 0: a load under a branch would be
// waited for inside the branch, one HBM round trip after another.
__device__ __forceinline__ ConvIn conv1_load(const f16* __restrict__ x, const f16* __restrict__ w,
                                             const f16* __restrict__ st_in, int d) {
    ConvIn c;
    const f16* st = st_in + (size_t)d * 3;
    c.h0 = st[0];
    c.h1 = st[1];
    c.h2 = st[2];
    c.x = x[d];
    c.w = *(const f16x4*)(w + (size_t)d * 4);
    return c;
}

// conv1d_causal at T = 1 for channel d (width 4, kernels.cu:1634-1679 /
// 2916-2941; the history is zero when pos0 == 0): the fp16-rounded silu
// output.
__device__ __forceinline__ float conv1_apply(const ConvIn& c, bool hist) {
    const float s0 = hist ? (float)c.h0 : 0.f;
    const float s1 = hist ? (float)c.h1 : 0.f;
    const float s2 = hist ? (float)c.h2 : 0.f;
    const float xv = (float)c.x;
    float acc = 0.f;
    acc = fmaf((float)c.w[0], s0, acc);
    acc = fmaf((float)c.w[1], s1, acc);
    acc = fmaf((float)c.w[2], s2, acc);
    acc = fmaf((float)c.w[3], xv, acc);
    return (float)f16_sat(silu_f(acc));
}

// ... and its new state (s1, s2, x) into the ring. Stored at the kernel's
// end: vector memory operations complete in order for the wait counter, so
// a store issued behind the state's loads would make every later wait (the
// barrier's for the gate loads included) wait for those loads too.
__device__ __forceinline__ void conv1_ring_store(const ConvIn& c, bool hist, f16* st_out, int d) {
    f16* so = st_out + (size_t)d * 3;
    so[0] = f16_sat(hist ? (float)c.h1 : 0.f);
    so[1] = f16_sat(hist ? (float)c.h2 : 0.f);
    so[2] = f16_sat((float)c.x);
}

// The decode / verify step: a workgroup of 4 wavefronts owns 32 state rows
// of one v head (8 lanes a row, 8 rows a wave). Per token every thread
// convolves (or reads) one q / k channel of the row's k head (k: threads
// 0-127, q: 128-255) and one of the 32 rows' v channels, and each wave sums
// the squares of its 64 q / k values as two 32-lane trees (the reference's
// warp sums); one wave keeps the v values, another forms the two gates --
// barrier -- every thread normalises its own channel into LDS -- barrier --
// and every wave runs the delta rule on its 8 rows. The kernel is a chain of
// short dependent steps between the state's load and its store, so the
// per-wave instruction count on that chain is what was cut: the gates (a
// dozen transcendental-unit instructions) and the v values once a workgroup
// instead of once a wave, the norm's trees ahead of the first barrier. The
// state is stored as soon as it is updated, before the output's reduction.
// (Measured and not kept: two rows a thread.) Token 0's conv / gate inputs
// are issued before the state's loads so the prologue computes while the
// state streams in; the state is read and written with non-temporal loads /
// stores (once a step).
template <bool CONV>
__global__ void __launch_bounds__(GR_THREADS)
gdn_decode_kernel(const f16* __restrict__ x, int x_stride, const f16* __restrict__ conv_w,
                  GdnSeqs seqs, const float* __restrict__ ga, const float* __restrict__ gb,
                  int ab_stride, const float* __restrict__ A_log,
                  const float* __restrict__ dt_bias, f16* __restrict__ y, int y_stride,
                  long long ck_step, int T, int n_kheads, int n_vheads, int V, float out_scale,
                  float l2eps, int group, int delay_loads) {
    __shared__ __attribute__((aligned(16))) float ssq[8];   // k's, q's 32-channel sums of squares
    __shared__ __attribute__((aligned(16))) float snorm[2 * GR_K];         // k | q, normalised
    __shared__ float sv[GR_ROWS];   // the rows' v values
    __shared__ float sg[2];         // beta, decay
    const int rb = blockIdx.x, hv = blockIdx.y, b = blockIdx.z;
    // this sequence's kernel-argument values in one scalar round, ahead of
    // every vector load (each later scalar load would be one more round trip
    // on the way to the state stores)
    float* const Sb = seqs.S[b];
    const f16* const cst_in = seqs.cst_in[b];
    f16* const cst_out = seqs.cst_out[b];
    float* const Ck = seqs.Ck[b];
    const int pos0 = seqs.pos0[b];
    asm volatile("" ::"s"(Sb), "s"(cst_in), "s"(cst_out), "s"(Ck), "s"(pos0), "s"(x), "s"(conv_w),
                 "s"(ga), "s"(gb), "s"(A_log), "s"(dt_bias), "s"(x_stride), "s"(ab_stride), "s"(T),
                 "s"(n_kheads), "s"(V), "s"(group), "s"(y), "s"(y_stride), "s"(out_scale),
                 "s"(l2eps), "s"(ck_step), "s"(delay_loads));
    __builtin_amdgcn_sched_barrier(0);
    const int hk = hv / group;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ri = tid >> 3, c0 = 4 * (tid & 7);
    const int vi = rb * GR_ROWS + ri;
    float* Srow = Sb + ((size_t)hv * V + vi) * GR_K + c0;
    const int half_ = tid >> 7, i = tid & 127;
    const int ch = (half_ ? hk * GR_K : n_kheads * GR_K + hk * GR_K) + i;   // q | k channel
    // the per-head gates and the 32 rows' v channels are formed once a
    // workgroup, by one wave each (which two varies with the block, spreading
    // that work over the SIMDs), and handed over at the barrier
    const int gw = (rb + hv + b) & 3, vw = gw ^ 2;
    const bool vkeep = w == vw && lane < GR_ROWS;
    const int ch_v = 2 * n_kheads * GR_K + hv * V + rb * GR_ROWS + (lane & 31);
    // token 0's inputs first, then the state: the prologue runs while S streams
    // in. The per-head gate inputs are uniform but read with vector loads (an
    // opaque zero in the index): they then queue in order ahead of the state
    // loads, where a scalar load's wait (lgkmcnt, out of order) would also
    // wait for every kernel-argument load issued after it.
    ConvIn cq, cv;
    const f16* x0 = x + (size_t)b * T * x_stride;
    if constexpr (CONV) {
        cq = conv1_load(x0, conv_w, cst_in, ch);
        cv = conv1_load(x0, conv_w, cst_in, ch_v);
    } else {
        cq.x = x0[ch];
        cv.x = x0[ch_v];
    }
    const int vz = opaque_zero();
    const float dtb = dt_bias[hv + vz], A = A_log[hv + vz];
    const size_t ab0 = (size_t)b * T * ab_stride + hv + vz;
    const float ga0 = ga[ab0], gb0 = gb[ab0];
    // The state loads wait ~512 clocks behind the small loads above when the
    // host asks (delay_loads: grids of 2 to 3 workgroups a CU, all resident and
    // dispatched at once): issued at once, the first workgroups' state reads
    // (16 KiB each) queue ahead of the later ones' conv inputs, which head the
    // chain to every store. Measured at s_sleep 4..16 (B = 4): 8 and 9 best.
    if (delay_loads) __builtin_amdgcn_s_sleep(8);
    __builtin_amdgcn_sched_barrier(0);
    float reg[16];
    load_row16_nt(reg, Srow);
    __builtin_amdgcn_sched_barrier(0);
    // one token; token 0 is peeled so that nothing of its conversions is
    // hoisted in front of the state loads
    auto token = [&](int t, float a_t, float b_t) {
        const size_t bt_row = (size_t)b * T + t;
        // every wave convolves a v channel beside its q / k one (independent
        // chains, interleaved); wave vw keeps them
        float xv, v_;
        if constexpr (CONV) {
            xv = conv1_apply(cq, pos0 > 0);
            v_ = conv1_apply(cv, pos0 > 0);
        } else {
            xv = (float)cq.x;
            v_ = (float)cv.x;
        }
        // the sums of squares of this wave's 64 values as two 32-lane trees:
        // lanes 0 and 32 hold the reference's warp sums r0, r1 (wave 0) and
        // r2, r3 (wave 1) of k, the same of q in waves 2 and 3
        const float tr = warp32_tree_lane0(xv * xv);
        if ((lane & 31) == 0) ssq[tid >> 5] = tr;
        if (vkeep) sv[lane] = v_;
        if (w == gw) {
            const float bt_ = gdn_beta(b_t);
            const float dt_ = gdn_decay(a_t + dtb, A);
            if (lane == 0) {
                sg[0] = bt_;
                sg[1] = dt_;
            }
        }
        __syncthreads();
        const float vt = sv[ri], bt = sg[0], dt = sg[1];
        // the norms, the reference's order (r0 + r2) + (r1 + r3): every thread
        // normalises its own channel (snorm is [k | q] as the channels are
        // laid over the threads); a second barrier
        const f32x4 r = *(const f32x4*)&ssq[4 * (w >> 1)];
        const float den = sqrtf(((r[0] + r[2]) + (r[1] + r[3])) + l2eps);
        snorm[tid] = (float)f16_sat(xv / den);
        __syncthreads();
        float kk[16], qq[16];
        gather16(kk, snorm, c0);
        gather16(qq, snorm + GR_K, c0);
        // nothing of the delta rule (its S *= decay first) above this point:
        // the state's wait would otherwise land inside the norms
        __builtin_amdgcn_sched_barrier(0);
        delta_update(reg, kk, vt, bt, dt);
        // the state (or its checkpoint) leaves ahead of the output's reduction
        if (t == T - 1)
            store_row16_nt(Srow, reg);
        else if (Ck != nullptr)
            store_row16_nt(Ck + (size_t)t * ck_step + ((size_t)hv * V + vi) * GR_K + c0, reg);
        const float o = delta_out(reg, qq);
        if (c0 == 0) y[bt_row * y_stride + (size_t)hv * V + vi] = f16_sat(o * out_scale);
    };
    token(0, ga0, gb0);
    for (int t = 1; t < T; ++t) {   // verify rows (conv_fused is T == 1 only)
        __syncthreads();   // ssq, sv and sg are rewritten by this token
        const size_t bt_row = (size_t)b * T + t;
        const f16* xr = x + bt_row * x_stride;
        cq.x = xr[ch];
        cv.x = xr[ch_v];
        token(t, ga[bt_row * ab_stride + hv + vz], gb[bt_row * ab_stride + hv + vz]);
    }
    if constexpr (CONV) {   // T == 1
        if ((hv % group) == 0 && rb == 0)   // one workgroup stores the q / k channels' ring
            conv1_ring_store(cq, pos0 > 0, cst_out, ch);
        if (vkeep) conv1_ring_store(cv, pos0 > 0, cst_out, ch_v);
    }
}

// The GDN output norm, RMSNormGated (kernels.cu:321-358, launched at
// runtime.py:3063-3065 / 3109-3111): y = f16((o * rsqrt(mean(o^2) + eps) * w) *
// silu(z)) -- plain gamma w (not 1 + w), mean-space eps, the norm over o alone
// with the gate applied after it, one 128-long w for every v head. A wave a
// row of 128: lane l holds o[2l], o[2l + 1] (one 4-byte load), so the
// reference's warp w' (elements 32 w'..32 w' + 31) is lanes 16 w'..16 w' + 15
// and its __shfl_down tree over offsets 16, 8, 4, 2, 1 is lane exchanges at
// distance 8, 4, 2, 1 then the in-lane pair; the 4 warp sums combine as
// block_reduce_sum does, (r0 + r2) + (r1 + r3).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// One row's norm from a wave holding it two values a lane (x0 = o[2l], x1 =
// o[2l + 1], z0 / z1 and w0 / w1 the gate and gamma there): the row's output
// at the lane's two places.
__device__ __forceinline__ f16x2 gated_rms_pair(float x0, float x1, float z0, float z1, float w0,
                                                float w1, float eps) {
    float s0 = fmaf(x0, x0, 0.f), s1 = fmaf(x1, x1, 0.f);
#pragma unroll
    for (int d = 8; d > 0; d >>= 1) {
        s0 += lane_xor(s0, d);
        s1 += lane_xor(s1, d);
    }
    const float ws = s0 + s1;   // lane 16 w': warp w''s total
    auto at = [](float v, int src) {
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
    };
    const float ss = (at(ws, 0) + at(ws, 32)) + (at(ws, 16) + at(ws, 48));
    const float inv = 1.f / sqrtf(ss / (float)GR_K + eps);
    return (f16x2){f16_sat(x0 * inv * w0 * silu_f(z0)), f16_sat(x1 * inv * w1 * silu_f(z1))};
}

__global__ void __launch_bounds__(GR_THREADS)
rmsnorm_gated_kernel(const f16* __restrict__ o, const f16* __restrict__ z,
                     const float* __restrict__ w, f16* __restrict__ y, int rows, int pitch,
                     int n_rows, float eps) {
    const int lane = threadIdx.x & 63;
    const int rid = blockIdx.x * (GR_THREADS / 64) + (threadIdx.x >> 6);
    if (rid >= n_rows) return;   // whole wavefronts; no workgroup barrier
    const int t = rid / rows, r = rid - t * rows;
    const size_t base = ((size_t)t * rows + r) * pitch + 2 * lane;
    const f16x2 ov = *(const f16x2*)(o + base);
    const f16x2 zv = *(const f16x2*)(z + base);
    *(f16x2*)(y + base) = gated_rms_pair((float)ov[0], (float)ov[1], (float)zv[0], (float)zv[1],
                                         w[2 * lane], w[2 * lane + 1], eps);
}

// A decode step (T = 1, the conv in the kernel) or a verify's rows (T <= 3,
// the conv rows done before it, a checkpoint of the state after every row but
// the last) with the output norm after every row, in one launch: a workgroup
// owns a whole v head (128 rows, 8 lanes a row, 16 waves), so the norm over
// the head's 128 outputs is a reduction inside the workgroup instead of a
// second launch. Per row: waves 0-1 convolve (or read) and sum the squares of
// the k head's channels, waves 2-3 the q head's, waves 4-5 the head's 128 v
// channels, wave 6 forms the gates -- barrier -- the k / q channels are
// normalised into LDS -- barrier -- every wave runs the delta rule on its 8
// rows and stores them (or their checkpoint), the rows' outputs (rounded to
// fp16, the value the unfused step writes) go to LDS -- barrier -- wave 0 runs
// the norm on them (gated_rms_pair, the unfused norm's arithmetic) and writes
// the head's 128 normed values while the others start the next row (that
// barrier also ends every read of the row's LDS values). Every value equals
// the unfused pair's bit for bit. One workgroup a head and sequence: 48 B
// workgroups, so below B = 5 a CU holds at most one; the small inputs are
// issued ahead of the state as in gdn_decode_kernel.
constexpr int GN_ROWS = 128;                  // the v head's rows
constexpr int GN_THREADS = 8 * GN_ROWS;       // 8 lanes a row

template <bool CONV>
__global__ void __launch_bounds__(GN_THREADS)
gdn_decode_normed_kernel(const f16* __restrict__ x, int x_stride, const f16* __restrict__ conv_w,
                         GdnSeqs seqs, const float* __restrict__ ga, const float* __restrict__ gb,
                         int ab_stride, const float* __restrict__ A_log,
                         const float* __restrict__ dt_bias, const f16* __restrict__ z,
                         int z_pitch, const float* __restrict__ norm_w, f16* __restrict__ y,
                         int y_pitch, long long ck_step, int T, int n_kheads, float out_scale,
                         float l2eps, float norm_eps, int group) {
    __shared__ __attribute__((aligned(16))) float ssq[8];   // k's, q's 32-channel sums of squares
    __shared__ __attribute__((aligned(16))) float snorm[2 * GR_K];   // k | q, normalised
    __shared__ float sv[GN_ROWS];                                    // the head's v values
    __shared__ float sg[2];                                          // beta, decay
    __shared__ __attribute__((aligned(16))) float so[GN_ROWS];       // the rows' fp16 outputs
    const int hv = blockIdx.x, b = blockIdx.y;
    float* const Sb = seqs.S[b];
    const f16* const cst_in = seqs.cst_in[b];
    f16* const cst_out = seqs.cst_out[b];
    float* const Ck = seqs.Ck[b];
    const int pos0 = seqs.pos0[b];
    asm volatile("" ::"s"(Sb), "s"(cst_in), "s"(cst_out), "s"(Ck), "s"(pos0), "s"(x), "s"(conv_w),
                 "s"(ga), "s"(gb), "s"(A_log), "s"(dt_bias), "s"(x_stride), "s"(ab_stride), "s"(z),
                 "s"(z_pitch), "s"(norm_w), "s"(y), "s"(y_pitch), "s"(n_kheads), "s"(group),
                 "s"(out_scale), "s"(l2eps), "s"(norm_eps), "s"(ck_step), "s"(T));
    __builtin_amdgcn_sched_barrier(0);
    const int hk = hv / group;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ri = tid >> 3, c0 = 4 * (tid & 7);
    const size_t srow = ((size_t)hv * GN_ROWS + ri) * GR_K + c0;
    float* Srow = Sb + srow;
    // waves 0-5: channel i of the k | q | v heads (uniform per wave)
    const int role = w >> 1, i = tid & 127;
    const int ch = role == 0   ? n_kheads * GR_K + hk * GR_K + i
                   : role == 1 ? hk * GR_K + i
                               : 2 * n_kheads * GR_K + hv * GN_ROWS + i;
    const bool conv_wave = w < 6;
    const size_t bt0 = (size_t)b * T;   // the sequence's first row
    const f16* x0 = x + bt0 * x_stride;
    ConvIn cc;
    if (conv_wave) {
        if constexpr (CONV) cc = conv1_load(x0, conv_w, cst_in, ch);
        else cc.x = x0[ch];
    }
    const int vz = opaque_zero();
    const float dtb = dt_bias[hv + vz], A = A_log[hv + vz];
    const size_t ab0 = bt0 * ab_stride + hv + vz;
    const float ga0 = ga[ab0], gb0 = gb[ab0];
    f16x2 zv = {};
    float nw0 = 0.f, nw1 = 0.f;
    if (w == 0) {
        zv = *(const f16x2*)(z + bt0 * z_pitch + (size_t)hv * GN_ROWS + 2 * lane);
        nw0 = norm_w[2 * lane];
        nw1 = norm_w[2 * lane + 1];
    }
    __builtin_amdgcn_sched_barrier(0);
    float reg[16];
    load_row16_nt(reg, Srow);
    __builtin_amdgcn_sched_barrier(0);
    auto row = [&](int t, float a_t, float b_t) {
        const size_t bt = bt0 + t;
        float xv = 0.f;
        if (conv_wave) {
            if constexpr (CONV) xv = conv1_apply(cc, pos0 > 0);
            else xv = (float)cc.x;
            if (role < 2) {
                const float tr = warp32_tree_lane0(xv * xv);
                if ((lane & 31) == 0) ssq[tid >> 5] = tr;
            } else {
                sv[i] = xv;
            }
        } else if (w == 6) {
            const float bt_ = gdn_beta(b_t);
            const float dt_ = gdn_decay(a_t + dtb, A);
            if (lane == 0) {
                sg[0] = bt_;
                sg[1] = dt_;
            }
        }
        __syncthreads();
        if (role < 2) {   // the reference's order (r0 + r2) + (r1 + r3)
            const f32x4 r = *(const f32x4*)&ssq[4 * role];
            const float den = sqrtf(((r[0] + r[2]) + (r[1] + r[3])) + l2eps);
            snorm[tid] = (float)f16_sat(xv / den);
        }
        __syncthreads();
        const float vt = sv[ri], bet = sg[0], dec = sg[1];
        float kk[16], qq[16];
        gather16(kk, snorm, c0);
        gather16(qq, snorm + GR_K, c0);
        __builtin_amdgcn_sched_barrier(0);
        delta_update(reg, kk, vt, bet, dec);
        if (t == T - 1)
            store_row16_nt(Srow, reg);
        else if (Ck != nullptr)
            store_row16_nt(Ck + (size_t)t * ck_step + srow, reg);
        const float o = delta_out(reg, qq);
        if (c0 == 0) so[ri] = (float)f16_sat(o * out_scale);
        __syncthreads();
        if (w == 0) {
            const float x0v = so[2 * lane], x1v = so[2 * lane + 1];
            *(f16x2*)(y + bt * y_pitch + (size_t)hv * GN_ROWS + 2 * lane) =
                gated_rms_pair(x0v, x1v, (float)zv[0], (float)zv[1], nw0, nw1, norm_eps);
        }
    };
    row(0, ga0, gb0);
    for (int t = 1; t < T; ++t) {   // verify rows (the conv in the kernel is T == 1 only)
        const size_t bt = bt0 + t;
        if (conv_wave) cc.x = x[bt * x_stride + ch];
        if (w == 0) zv = *(const f16x2*)(z + bt * z_pitch + (size_t)hv * GN_ROWS + 2 * lane);
        row(t, ga[bt * ab_stride + hv + vz], gb[bt * ab_stride + hv + vz]);
    }
    if constexpr (CONV) {   // T == 1
        if (conv_wave && (role == 2 || hv % group == 0))   // one v head a k head stores its ring
            conv1_ring_store(cc, pos0 > 0, cst_out, ch);
    }
}

// The same norm, 16-byte aligned rows: 16 lanes a row (lane j of the row holds
// o[8 j .. 8 j + 7], one 16-byte load), 4 rows a wave per pass and GR_PASSES
// passes (all loads issued first), so a wave carries 4 GR_PASSES rows.
// The reference's warp w' is lanes 4 w' .. 4 w' + 3 of the row; its
// __shfl_down tree over offsets 16, 8, 4, 2, 1 is lane exchanges at distance
// 2 and 1 (butterflies: a + b == b + a, so every lane holds the tree's lane-0
// sum bit for bit) then the in-lane pairs (i, i + 4), (i, i + 2), (0, 1); the
// warp sums combine as (r0 + r2) + (r1 + r3) by exchanges at distance 8, 4.
// Passes a wave: 1, 2 and 4 measured alike at T = 8192 (48 rows a token,
// 74 us against 111 us for a wave a row), 1 best at T = 1024 (11.4 / 12.7 /
// 14.2 us against 15.5).
constexpr int GR_PASSES = 1;
// the 16-lanes-a-row kernel from this many rows up: below, a wave a row keeps
// more waves on a decode step's few rows (T = 4, 192 rows: 2.0 us, against
// 3.7 us at 8 rows a wave)
constexpr long long GR_ROWS_MIN = 8192;
// v of lane l ^ 1 / l ^ 2 (DPP quad permutes [1 0 3 2] / [2 3 0 1])
__device__ __forceinline__ float dpp_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}
__global__ void __launch_bounds__(GR_THREADS)
rmsnorm_gated_rows_kernel(const f16* __restrict__ o, const f16* __restrict__ z,
                          const float* __restrict__ w, f16* __restrict__ y, int rows, int pitch,
                          int n_rows, float eps) {
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int wave = blockIdx.x * (GR_THREADS / 64) + (threadIdx.x >> 6);
    typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
    f16x8v ov[GR_PASSES], zv[GR_PASSES];
    size_t base[GR_PASSES];
    bool ok[GR_PASSES];
#pragma unroll
    for (int p = 0; p < GR_PASSES; ++p) {
        const int rid = (wave * GR_PASSES + p) * 4 + (lane >> 4);
        ok[p] = rid < n_rows;
        const int rr = ok[p] ? rid : n_rows - 1;
        const int t = rr / rows, r = rr - t * rows;
        base[p] = ((size_t)t * rows + r) * pitch + 8 * j;
        ov[p] = *(const f16x8v*)(o + base[p]);
        zv[p] = *(const f16x8v*)(z + base[p]);
    }
    const f32x4 w0 = *(const f32x4*)(w + 8 * j), w1 = *(const f32x4*)(w + 8 * j + 4);
    const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
#pragma unroll
    for (int p = 0; p < GR_PASSES; ++p) {
        float x[8], sq[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            x[i] = (float)ov[p][i];
            sq[i] = x[i] * x[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) sq[i] += dpp_xor2(sq[i]);   // offset 16
#pragma unroll
        for (int i = 0; i < 8; ++i) sq[i] += dpp_xor1(sq[i]);   // offset 8
        float t4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) t4[i] = sq[i] + sq[i + 4];        // offset 4
        const float t2a = t4[0] + t4[2], t2b = t4[1] + t4[3];         // offset 2
        float ss = t2a + t2b;                                          // offset 1: warp sum
        ss += lane_xor(ss, 8);                                         // r0 + r2, r1 + r3
        ss += lane_xor(ss, 4);                                         // (r0 + r2) + (r1 + r3)
        const float inv = 1.f / sqrtf(ss / (float)GR_K + eps);
        f16x8v out;
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = f16_sat(x[i] * inv * wv[i] * silu_f((float)zv[p][i]));
        if (ok[p]) *(f16x8v*)(y + base[p]) = out;
    }
}

// l2norm_scaled on 128-element rows at 16-byte-aligned pitch: 16 lanes a row
// (lane j of the row holds x[8 j .. 8 j + 7], one 16-byte load), 4 rows a
// wave. The reference's block of 128 threads sums the squares by warp
// (elements 32 w'.. 32 w' + 31, a __shfl_down tree over offsets 16, 8, 4, 2,
// 1) and then (r0 + r2) + (r1 + r3) (kernels.cu:373-391): here warp w' is
// lanes 4 w'.. 4 w' + 3, offsets 16 and 8 are the lane exchanges at distance
// 2 and 1 (butterflies: every lane of the four holds the tree's sum, a + b ==
// b + a), 4, 2, 1 the in-lane pairs, and the warp sums combine by exchanges
// at distance 8 and 4 -- the same additions in the same order, so the same
// bits as the one-row-a-wavefront kernel above.
constexpr int L2_ROWS_PER_WG = (GR_THREADS / 64) * 4;
__global__ void __launch_bounds__(GR_THREADS)
l2norm_rows_kernel(const f16* __restrict__ x, f16* __restrict__ y, int rows, int pitch,
                   long long tstride, int n_rows, float eps, float scale) {
    typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int rid = (blockIdx.x * (GR_THREADS / 64) + (threadIdx.x >> 6)) * 4 + (lane >> 4);
    const bool ok = rid < n_rows;
    const int rr = ok ? rid : n_rows - 1;   // rows past the end read the last, store nothing
    const int t = rr / rows, r = rr - t * rows;
    // tstride: elements between tokens' first rows (rows * pitch when a
    // token's rows are all normalised)
    const size_t base = (size_t)t * tstride + (size_t)r * pitch + 8 * j;
    const f16x8v xv = *(const f16x8v*)(x + base);
    float xf[8], sq[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        xf[i] = (float)xv[i];
        sq[i] = fmaf(xf[i], xf[i], 0.f);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) sq[i] += dpp_xor2(sq[i]);   // offset 16
#pragma unroll
    for (int i = 0; i < 8; ++i) sq[i] += dpp_xor1(sq[i]);   // offset 8
    float t4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) t4[i] = sq[i] + sq[i + 4];        // offset 4
    const float t2a = t4[0] + t4[2], t2b = t4[1] + t4[3];         // offset 2
    float ss = t2a + t2b;                                          // offset 1: warp sum
    ss += lane_xor(ss, 8);                                         // r0 + r2, r1 + r3
    ss += lane_xor(ss, 4);                                         // (r0 + r2) + (r1 + r3)
    const float den = sqrtf(ss + eps);
    f16x8v out;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = f16_sat((xf[i] / den) * scale);
    if (ok) *(f16x8v*)(y + base) = out;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The current device's compute-unit count, looked up once per device.
int gdn_cu_count() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

}  // namespace

extern "C" {

// The 8-channel (16-byte) form needs every row, tap set and state of a lane's
// channels on 16-byte boundaries: dim and row_stride multiples of 8 and the
// five buffers 16-byte aligned; anything else takes the channel-a-lane form.
static bool conv_vec_ok(const void* x, const void* w, const void* st_in, const void* y,
                        const f16* const* st, int n_st, int dim, int row_stride) {
    bool ok = dim % 8 == 0 && row_stride % 8 == 0 && aligned16(x) && aligned16(w) &&
              aligned16(st_in) && aligned16(y);
    for (int i = 0; i < n_st; ++i) ok = ok && aligned16(st[i]);
    return ok;
}

static int conv_dispatch(const void* x, const void* w, const void* st_in, void* y,
                         ConvStates outs, int n_st, bool rows, int dim, int T, int pos0,
                         int row_stride, int width, hipStream_t stream) {
    const f16* sts[3] = {outs.st[0], outs.st[1], outs.st[2]};
    const bool vec = conv_vec_ok(x, w, st_in, y, sts, n_st, dim, row_stride);
    const int cpl = vec ? 8 : 1;
    // a verify (T <= 3) is one block whatever its length
    const int tb = rows ? CONV_TB : conv_tb(width, T, (dim + 64 * cpl - 1) / (64 * cpl),
                                            gdn_cu_count());
    const f16 *xp = (const f16*)x, *wp = (const f16*)w, *sp = (const f16*)st_in;
    f16* yp = (f16*)y;
    switch (width) {
#define FL_CONV_W(Wd) \
    case Wd: conv_launch<Wd>(vec, rows, tb, xp, wp, sp, yp, outs, dim, T, pos0, row_stride, stream); break;
        FL_CONV_W(1) FL_CONV_W(2) FL_CONV_W(3) FL_CONV_W(4)
        FL_CONV_W(5) FL_CONV_W(6) FL_CONV_W(7) FL_CONV_W(8)
#undef FL_CONV_W
        default: return fl::einval("1 <= width <= 8");
    }
    return fl::check_launch(rows ? "conv1d_causal_rows" : "conv1d_causal");
}

int fl_conv1d_causal(const void* x, const void* w, const void* st_in, void* y, void* st_out,
                     int dim, int T, int pos0, int row_stride, int width, fl_stream_t stream) {
    FL_REQUIRE(x && w && st_in && y && st_out, "null pointer");
    FL_REQUIRE(st_in != st_out, "st_in and st_out must be distinct buffers");
    FL_REQUIRE(dim >= 1 && T >= 1 && pos0 >= 0 && row_stride >= dim, "dim, T, pos0, row_stride");
    FL_REQUIRE(width >= 1 && width <= CONV_WMAX, "1 <= width <= 8");
    ConvStates outs = {{(f16*)st_out, nullptr, nullptr}};
    return conv_dispatch(x, w, st_in, y, outs, 1, false, dim, T, pos0, row_stride, width,
                         (hipStream_t)stream);
}

int fl_conv1d_causal_rows(const void* x, const void* w, const void* st_in, void* y, void* st0,
                          void* st1, void* st2, int dim, int T, int pos0, int row_stride,
                          fl_stream_t stream) {
    FL_REQUIRE(x && w && st_in && y, "null pointer");
    FL_REQUIRE(T >= 1 && T <= 3, "1 <= T <= 3");
    FL_REQUIRE(st0 && (T < 2 || st1) && (T < 3 || st2), "a state buffer per row");
    FL_REQUIRE(dim >= 1 && pos0 >= 0 && row_stride >= dim, "dim, pos0, row_stride");
    ConvStates outs = {{(f16*)st0, (f16*)st1, (f16*)st2}};
    return conv_dispatch(x, w, st_in, y, outs, T, true, dim, T, pos0, row_stride, 4,
                         (hipStream_t)stream);
}

int fl_l2norm_scaled(const void* x, void* y, int n, int rows, int pitch, float eps, float scale,
                     int T, fl_stream_t stream) {
    FL_REQUIRE(x && y, "null pointer");
    FL_REQUIRE(n >= 1 && n <= 1024 && pitch >= n && rows >= 1 && T >= 1, "n, rows, pitch, T");
    const long long n_rows = (long long)rows * T;
    if (n == GR_K && pitch % 8 == 0 && aligned16(x) && aligned16(y) && n_rows < (1ll << 31)) {
        const long long wgs = (n_rows + L2_ROWS_PER_WG - 1) / L2_ROWS_PER_WG;
        hipLaunchKernelGGL(l2norm_rows_kernel, dim3((unsigned)wgs), dim3(GR_THREADS), 0,
                           (hipStream_t)stream, (const f16*)x, (f16*)y, rows, pitch,
                           (long long)rows * pitch, (int)n_rows, eps, scale);
    } else {
        FL_REQUIRE(n_rows < (1ll << 31), "rows * T < 2^31");
        hipLaunchKernelGGL(l2norm_wave_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0,
                           (hipStream_t)stream, (const f16*)x, (f16*)y, n, rows, pitch,
                           (int)n_rows, eps, scale);
    }
    return fl::check_launch("l2norm_scaled");
}

int fl_l2norm_scaled_strided(const void* x, void* y, int rows, int pitch,
                             long long token_stride, float eps, float scale, int T,
                             fl_stream_t stream) {
    FL_REQUIRE(x && y, "null pointer");
    FL_REQUIRE(rows >= 1 && T >= 1 && pitch >= GR_K && pitch % 8 == 0, "rows, T, pitch");
    FL_REQUIRE(token_stride >= (long long)rows * pitch && token_stride % 8 == 0,
               "token_stride >= rows * pitch, a multiple of 8");
    FL_REQUIRE(aligned16(x) && aligned16(y), "16-byte aligned x / y");
    const long long n_rows = (long long)rows * T;
    FL_REQUIRE(n_rows < (1ll << 31), "rows * T < 2^31");
    const long long wgs = (n_rows + L2_ROWS_PER_WG - 1) / L2_ROWS_PER_WG;
    hipLaunchKernelGGL(l2norm_rows_kernel, dim3((unsigned)wgs), dim3(GR_THREADS), 0,
                       (hipStream_t)stream, (const f16*)x, (f16*)y, rows, pitch, token_stride,
                       (int)n_rows, eps, scale);
    return fl::check_launch("l2norm_scaled_strided");
}

int fl_gdn_scalars(const float* a, const float* b, const float* A_log, const float* dt_bias,
                   float* beta, float* decay, int T, int n_heads, int a_stride, int b_stride,
                   fl_stream_t stream) {
    FL_REQUIRE(a && b && A_log && dt_bias && beta && decay, "null pointer");
    FL_REQUIRE(T >= 1 && n_heads >= 1 && a_stride >= n_heads && b_stride >= n_heads,
               "T, n_heads, strides");
    hipLaunchKernelGGL(gdn_scalars_kernel, dim3((n_heads + 255) / 256, T), dim3(256), 0,
                       (hipStream_t)stream, a, b, A_log, dt_bias, beta, decay, n_heads, a_stride,
                       b_stride);
    return fl::check_launch("gdn_scalars");
}

int fl_gdn_scan(const void* q, const void* k, const void* v, const float* beta,
                const float* decay, float* S, void* y, int T, int n_kheads, int n_vheads, int K,
                int V, int qk_stride, int v_stride, int y_stride, float out_scale, int group,
                float* Ck, long long ck_step, fl_stream_t stream) {
    FL_REQUIRE(q && k && v && beta && decay && S && y, "null pointer");
    FL_REQUIRE(K == GR_K, "K must be 128");
    FL_REQUIRE(V >= 8 && V % 8 == 0, "V % 8 == 0");
    FL_REQUIRE(group >= 1 && n_vheads >= 1 && (n_vheads - 1) / group < n_kheads,
               "n_vheads / group <= n_kheads");
    FL_REQUIRE(T >= 1, "T >= 1");
    FL_REQUIRE(aligned16(S) && (Ck == nullptr || (aligned16(Ck) && ck_step % 4 == 0)),
               "16-byte aligned S / Ck");
    FL_REQUIRE(((uintptr_t)q & 7u) == 0 && ((uintptr_t)k & 7u) == 0 && qk_stride % 4 == 0,
               "8-byte aligned q / k rows (qk_stride % 4 == 0)");
    hipLaunchKernelGGL(gdn_scan_kernel, dim3(n_vheads * (V / 8)), dim3(64), 0,
                       (hipStream_t)stream, (const f16*)q, (const f16*)k, (const f16*)v, beta,
                       decay, S, (f16*)y, T, n_vheads, V, qk_stride, v_stride, y_stride,
                       out_scale, group, Ck, ck_step);
    return fl::check_launch("gdn_scan");
}

int fl_gdn_decode(const void* x, int x_stride, int conv_fused, const void* conv_w,
                  const void* const* cst_in, void* const* cst_out, const int* pos0,
                  const float* a, const float* b, int ab_stride, const float* A_log,
                  const float* dt_bias, float* const* S, void* y, int y_stride, float* const* Ck,
                  long long ck_step, int B, int T, int n_kheads, int n_vheads, int K, int V,
                  float out_scale, float l2eps, fl_stream_t stream) {
    FL_REQUIRE(x && a && b && A_log && dt_bias && S && y && pos0, "null pointer");
    FL_REQUIRE(B >= 1 && B <= FL_MAX_SEQS, "1 <= B <= FL_MAX_SEQS");
    FL_REQUIRE(T >= 1 && T <= 3, "1 <= T <= 3");
    FL_REQUIRE(K == GR_K, "K must be 128");
    FL_REQUIRE(V >= GR_ROWS && V % GR_ROWS == 0, "V % 32 == 0");
    FL_REQUIRE(n_kheads >= 1 && n_vheads % n_kheads == 0, "n_vheads % n_kheads == 0");
    FL_REQUIRE(x_stride >= 2 * n_kheads * K + n_vheads * V, "x_stride covers q|k|v");
    FL_REQUIRE(ab_stride >= n_vheads && y_stride >= n_vheads * V, "ab_stride, y_stride");
    FL_REQUIRE(!conv_fused || (T == 1 && conv_w && cst_in && cst_out), "conv_fused: T == 1 and "
               "conv_w, cst_in, cst_out");
    GdnSeqs seqs = {};
    for (int i = 0; i < B; ++i) {
        FL_REQUIRE(S[i] && aligned16(S[i]), "16-byte aligned S[b]");
        seqs.S[i] = S[i];
        seqs.pos0[i] = pos0[i];
        FL_REQUIRE(pos0[i] >= 0, "pos0 >= 0");
        if (conv_fused) {
            FL_REQUIRE(cst_in[i] && cst_out[i] && cst_in[i] != cst_out[i],
                       "cst_in[b], cst_out[b] distinct");
            seqs.cst_in[i] = (const f16*)cst_in[i];
            seqs.cst_out[i] = (f16*)cst_out[i];
        }
        if (Ck != nullptr && Ck[i] != nullptr) {
            FL_REQUIRE(aligned16(Ck[i]) && ck_step % 4 == 0, "16-byte aligned Ck");
            seqs.Ck[i] = Ck[i];
        }
    }
    const dim3 grid(V / GR_ROWS, n_vheads, B);
    // the state loads held behind the small ones for grids of 2 to 3
    // workgroups a CU (B = 3, 4 at 48 v heads on 256 CUs: 5.96 / 6.33 us a
    // step against 6.07 / 6.63 without); beyond that the delay costs (B = 5..8:
    // ~0.1 us a step), below it changes nothing
    const long long wgs = (long long)grid.x * grid.y * grid.z;
    const int cus = gdn_cu_count();
    const int delay = wgs >= 2LL * cus && wgs <= 3LL * cus;
    if (conv_fused)
        hipLaunchKernelGGL(gdn_decode_kernel<true>, grid, dim3(GR_THREADS), 0, (hipStream_t)stream,
                           (const f16*)x, x_stride, (const f16*)conv_w, seqs, a, b, ab_stride,
                           A_log, dt_bias, (f16*)y, y_stride, ck_step, T, n_kheads, n_vheads, V,
                           out_scale, l2eps, n_vheads / n_kheads, delay);
    else
        hipLaunchKernelGGL(gdn_decode_kernel<false>, grid, dim3(GR_THREADS), 0,
                           (hipStream_t)stream, (const f16*)x, x_stride, (const f16*)conv_w, seqs,
                           a, b, ab_stride, A_log, dt_bias, (f16*)y, y_stride, ck_step, T,
                           n_kheads, n_vheads, V, out_scale, l2eps, n_vheads / n_kheads, delay);
    return fl::check_launch("gdn_decode");
}

int fl_gdn_decode_normed(const void* x, int x_stride, int conv_fused, const void* conv_w,
                         const void* const* cst_in, void* const* cst_out, const int* pos0,
                         const float* a, const float* b, int ab_stride, const float* A_log,
                         const float* dt_bias, float* const* S, float* const* Ck,
                         long long ck_step, const void* z, int z_pitch, const float* norm_w,
                         void* y, int y_pitch, int B, int T, int n_kheads, int n_vheads, int K,
                         int V, float out_scale, float l2eps, float norm_eps,
                         fl_stream_t stream) {
    FL_REQUIRE(x && pos0 && a && b && A_log && dt_bias && S && z && norm_w && y, "null pointer");
    FL_REQUIRE(B >= 1 && B <= FL_MAX_SEQS, "1 <= B <= FL_MAX_SEQS");
    FL_REQUIRE(T >= 1 && T <= 3, "1 <= T <= 3");
    FL_REQUIRE(K == GR_K && V == GN_ROWS, "K and V must be 128");
    FL_REQUIRE(n_kheads >= 1 && n_vheads >= 1 && n_vheads % n_kheads == 0,
               "n_vheads % n_kheads == 0");
    FL_REQUIRE(x_stride >= 2 * n_kheads * K + n_vheads * V, "x_stride covers q|k|v");
    FL_REQUIRE(ab_stride >= n_vheads, "ab_stride >= n_vheads");
    FL_REQUIRE(z_pitch >= n_vheads * V && y_pitch >= n_vheads * V && z_pitch % 2 == 0 &&
                   y_pitch % 2 == 0,
               "z_pitch, y_pitch >= n_vheads * V and even");
    FL_REQUIRE(((uintptr_t)z & 3u) == 0 && ((uintptr_t)y & 3u) == 0 && ((uintptr_t)norm_w & 7u) == 0,
               "aligned z, y, norm_w");
    FL_REQUIRE(norm_eps >= 0.f, "norm_eps >= 0");
    FL_REQUIRE(!conv_fused || (T == 1 && conv_w && cst_in && cst_out), "conv_fused: T == 1 and "
               "conv_w, cst_in, cst_out");
    GdnSeqs seqs = {};
    for (int i = 0; i < B; ++i) {
        FL_REQUIRE(S[i] && aligned16(S[i]), "16-byte aligned S[b]");
        FL_REQUIRE(pos0[i] >= 0, "pos0 >= 0");
        seqs.S[i] = S[i];
        seqs.pos0[i] = pos0[i];
        if (conv_fused) {
            FL_REQUIRE(cst_in[i] && cst_out[i] && cst_in[i] != cst_out[i],
                       "cst_in[b], cst_out[b] distinct");
            seqs.cst_in[i] = (const f16*)cst_in[i];
            seqs.cst_out[i] = (f16*)cst_out[i];
        }
        if (Ck != nullptr && Ck[i] != nullptr) {
            FL_REQUIRE(aligned16(Ck[i]) && ck_step % 4 == 0, "16-byte aligned Ck");
            seqs.Ck[i] = Ck[i];
        }
    }
    const int group = n_vheads / n_kheads;
    if (conv_fused)
        hipLaunchKernelGGL(gdn_decode_normed_kernel<true>, dim3(n_vheads, B), dim3(GN_THREADS), 0,
                           (hipStream_t)stream, (const f16*)x, x_stride, (const f16*)conv_w, seqs,
                           a, b, ab_stride, A_log, dt_bias, (const f16*)z, z_pitch, norm_w,
                           (f16*)y, y_pitch, ck_step, T, n_kheads, out_scale, l2eps, norm_eps,
                           group);
    else
        hipLaunchKernelGGL(gdn_decode_normed_kernel<false>, dim3(n_vheads, B), dim3(GN_THREADS), 0,
                           (hipStream_t)stream, (const f16*)x, x_stride, (const f16*)conv_w, seqs,
                           a, b, ab_stride, A_log, dt_bias, (const f16*)z, z_pitch, norm_w,
                           (f16*)y, y_pitch, ck_step, T, n_kheads, out_scale, l2eps, norm_eps,
                           group);
    return fl::check_launch("gdn_decode_normed");
}


int fl_rmsnorm_gated(const void* o, const void* z, const float* w, void* y, int n, int rows,
                     int pitch, int T, float eps, fl_stream_t stream) {
    FL_REQUIRE(o && z && w && y, "null pointer");
    FL_REQUIRE(n == GR_K, "n must be 128 (the GDN v head dim)");
    FL_REQUIRE(rows >= 1 && T >= 1 && pitch >= n && eps >= 0.f, "rows, T >= 1, pitch >= n");
    FL_REQUIRE(pitch % 2 == 0 && ((uintptr_t)o & 3u) == 0 && ((uintptr_t)z & 3u) == 0 &&
                   ((uintptr_t)y & 3u) == 0 && ((uintptr_t)w & 7u) == 0,
               "pitch % 2, aligned o, z, y, w");
    const long long n_rows = (long long)rows * T;
    const int waves = GR_THREADS / 64;
    if (n_rows >= GR_ROWS_MIN && pitch % 8 == 0 && aligned16(o) && aligned16(z) && aligned16(y) &&
        aligned16(w)) {
        const long long rows_wg = 4LL * GR_PASSES * waves;
        hipLaunchKernelGGL(rmsnorm_gated_rows_kernel, dim3((unsigned)((n_rows + rows_wg - 1) / rows_wg)),
                           dim3(GR_THREADS), 0, (hipStream_t)stream, (const f16*)o, (const f16*)z, w,
                           (f16*)y, rows, pitch, (int)n_rows, eps);
        return fl::check_launch("rmsnorm_gated");
    }
    hipLaunchKernelGGL(rmsnorm_gated_kernel, dim3((unsigned)((n_rows + waves - 1) / waves)),
                       dim3(GR_THREADS), 0, (hipStream_t)stream, (const f16*)o, (const f16*)z, w,
                       (f16*)y, rows, pitch, (int)n_rows, eps);
    return fl::check_launch("rmsnorm_gated");
}

}  // extern "C"
