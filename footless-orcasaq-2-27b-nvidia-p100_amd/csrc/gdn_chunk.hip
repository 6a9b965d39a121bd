// Chunked (WY / UT transform) Gated DeltaNet prefill on gfx950.
//
// Not in the reference: it runs the delta rule sequentially over a prefill
// (gdn_scan_rows, kernels.cu:2809-2914) and names the chunked scan as the
// undone optimisation (kernels.cu:1788-1791). This computes the same
// recurrence (S *= decay; delta = beta (v - S k); S += delta k^T; o = S q)
// chunk by chunk. For a chunk of C = 64 tokens with start state S0 [V][K] and
// g_i the in-chunk prefix sum of log(decay):
//   A[i][j] = beta_i e^{g_i - g_j} (k_i . k_j), j < i          (strictly lower)
//   T = (I + A)^-1                                              (unit lower)
//   X = K S0^T,  Y = diag(beta) (V - diag(e^g) X)               (C x V)
//   Delta = T Y
//   O   = diag(e^g) Q S0^T + (M o Q K^T) Delta,  M[i][j] = e^{g_i - g_j}, j <= i
//   S_C = e^{g_C} S0 + Delta^T diag(e^{g_C - g}) K
// (Delta = U - W S0^T with W = T diag(beta e^g) K and U = T diag(beta) V is
// the same product grouped otherwise; this grouping keeps only T and M o QK^T
// in the workspace and feeds K, Q and V, exact in fp16, straight to the
// matrix cores.) The decay ratios are formed as e^{g_i - g_j} with j <= i
// (never 1 / gamma_j, which overflows over a chunk of strong decay).
//
// Two launches. chunk_prep_kernel, every (chunk, v head) in parallel: K K^T
// and Q K^T of the v head's k head on MFMA (the three v heads of a k head
// each form them: one workgroup walking the three in turn measured 5 us
// slower at 8k), then the prefix sums, A, T in fp32 by blocks of 16 (the
// diagonal blocks by forward substitution, the others on fp32 MFMA), the
// gates, and T and M o QK^T written as fp16 MFMA operands.
// chunk_state_kernel: a state wavefront per 16 state rows (v) of a v head,
// all 128 k columns of them in fp32 registers, sequential over the chunks; a
// paired output wavefront takes its Q S0^T and Delta through LDS a chunk later,
// forms O and stores y, and issues the HBM -> LDS copies of the operands one
// chunk ahead, so the state chain carries only its own products.
//
// Precision. Every product runs on v_mfma_f32_16x16x32_f16 (fp16 inputs,
// fp32 accumulate: the product of two fp16 values is exact in fp32). K, Q and
// V are fp16 data. An fp32 operand x of the recurrence's products (the state,
// Y, T, the decayed Delta) is scaled by a power of two 2^s chosen from its
// block's maximum (max |x| 2^s in [128, 256); a block is T or M o QK^T whole,
// and one state row, i.e. one column of a B operand, for the state, Y and
// Delta) and split x 2^s = hi + lo, both fp16: two MFMAs (hi, lo) against an
// exact operand, three (hi.hi, hi.lo, lo.hi) between two split operands, which
// leaves an error of ~2^-22 of the block's maximum, fp32's order. The output's products need it too: one fp16
// pass leaves y within its own tolerance, but its two terms cancel in places
// and the gated norm that follows divides each head's row by its RMS (7e-3 of
// the row's RMS against 2e-3 for fp32 products). Emulated in numpy before the
// kernels were written, on the test's inputs: the state within 1.2e-6 of the
// sequential recurrence after 8192 tokens and y as close as with all-fp32
// products.
//
// MFMA operand layout (v_mfma_f32_16x16x32_f16, lane l = 16 g + i): the A
// operand of rows r0 .. r0 + 15 and a 32-wide k-step at k0 holds, in lane l,
// row r0 + i at k = k0 + kap(g, e), e = 0..7, kap(g, e) = 4 g + e (e < 4) or
// 16 + 4 g + (e - 4); the B operand holds column c0 + i at the same k. The
// result holds, in lane l, rows 4 g + r (r = 0..3) of column i. The matrix
// core pairs A and B by (lane group, slot), so any k order the two share is
// the same product; with kap, the results of two consecutive 16-row blocks
// are, as they stand in the registers, the B operand of the next product
// over those 32 rows: the state, X, Y and Delta never move between lanes.
#include "fl_common.hpp"

#include <mutex>

#pragma clang fp contract(off)

#include "gdn_gates.hpp"

namespace {

constexpr int CK_C = 64;       // tokens a chunk
constexpr int CK_K = 128;      // key dim
constexpr int CK_V = 128;      // value dim

// Workspace block of one (chunk, v head), bytes: T and M o QK^T, each as hi
// and lo fp16 A operands [6 blocks][64 lanes][8] (6 KiB each; block f is row
// block mb = f, k-step 0 for f < 4, and mb = f - 2, k-step 1 for f = 4, 5: both
// matrices are lower triangular, so rows 0..31 take nothing from k-step 1),
// then beta, e^{g} and e^{g_C - g} [64] f32 (beta 0 past the chunk's last
// token), then e^{g_C}, 2^-tau and 2^-kappa (T's and M o QK^T's scales).
constexpr int CK_NF = 6;
__host__ __device__ constexpr int f_mb(int f) { return f < 4 ? f : f - 2; }
__host__ __device__ constexpr int f_kq(int f) { return f < 4 ? 0 : 1; }
constexpr int WS_OP = CK_NF * 1024;
constexpr int WS_T_HI = 0, WS_T_LO = WS_OP, WS_Q_HI = 2 * WS_OP, WS_Q_LO = 3 * WS_OP,
              WS_BETA = 4 * WS_OP, WS_EG = WS_BETA + 256, WS_DK = WS_BETA + 512,
              WS_SC = WS_BETA + 768;
constexpr int CK_BLK = WS_BETA + 1024;

typedef __attribute__((address_space(3))) const f16x4 lds_f16x4;
typedef __attribute__((address_space(3))) const f16x8 lds_f16x8;
typedef __attribute__((address_space(3))) const f32x4 lds_f32x4;

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// max over the 64 lanes, on every lane: quad exchanges and row rotations by
// 4 and 8 (DPP), then v_permlane16_swap and v_permlane32_swap
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_xor1(v));
    v = fmaxf(v, dpp_xor2(v));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true)));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return pair32_max(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}

// max over the lanes l, l ^ 16, l ^ 32 and l ^ 48, the four lane groups that
// hold one column of an MFMA B operand (or result): v_permlane16_swap with
// both operands v returns v of the lane pair (l, l ^ 16), then
// v_permlane32_swap the pair (l, l ^ 32)
__device__ __forceinline__ float col_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return pair32_max(fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])));
}

// The power of two s with m s in [2^P, 2^(P+1)) for a block maximum m >= 0
// (from m's exponent field; at most 2^126, so 1 / s stays normal); inv = 1 / s.
template <int P>
__device__ __forceinline__ float pow2_scale(float m, float& inv) {
    const int e = (int)((__float_as_uint(m) >> 23) & 0xff);
    const int se = min(254 + P - e, 253);
    inv = __uint_as_float((uint32_t)(254 - se) << 23);
    return __uint_as_float((uint32_t)se << 23);
}

// 1 / x for a power of two x = 2^e with -126 <= e <= 126, exactly
__device__ __forceinline__ float pow2_inv(float x) {
    return __uint_as_float((254u - (__float_as_uint(x) >> 23)) << 23);
}

// x s = hi + lo, both fp16 (round to nearest), for two values into packed
// halves: v_fma_mix rounds x s (exact: s is a power of two) and x s - hi
// (exact in fp32: hi is x s to 11 bits) to fp16 once each, reading hi back as
// an fp16 source, so a value costs two instructions
__device__ __forceinline__ void split2(float x0, float x1, float s, uint32_t& hi, uint32_t& lo) {
    uint32_t h, e;
    asm("v_fma_mixlo_f16 %0, %1, %2, 0" : "=v"(h) : "v"(x0), "v"(s));
    asm("v_fma_mixhi_f16 %0, %1, %2, 0" : "+v"(h) : "v"(x1), "v"(s));
    asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,0,1]" : "=v"(e) : "v"(x0), "v"(s), "v"(h));
    asm("v_fma_mixhi_f16 %0, %1, %2, -%3 op_sel:[0,0,1] op_sel_hi:[0,0,1]"
        : "+v"(e) : "v"(x1), "v"(s), "v"(h));
    hi = h;
    lo = e;
}

// the B operand of a k-step from the accumulators a (slots 0..3) and b
// (slots 4..7), scaled by s and split
__device__ __forceinline__ void split8(f32x4 a, f32x4 b, float s, f16x8& hi, f16x8& lo) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    uint32_t h0, h1, h2, h3, l0, l1, l2, l3;
    split2(a[0], a[1], s, h0, l0);
    split2(a[2], a[3], s, h1, l1);
    split2(b[0], b[1], s, h2, l2);
    split2(b[2], b[3], s, h3, l3);
    hi = __builtin_bit_cast(f16x8, (u32x4){h0, h1, h2, h3});
    lo = __builtin_bit_cast(f16x8, (u32x4){l0, l1, l2, l3});
}

// ---------------------------------------------------------------------------
// chunk_prep_kernel: one workgroup of 4 waves a (chunk, v head)
// ---------------------------------------------------------------------------
constexpr int PK_P = CK_K + 8;   // f16 pitch of staged K / Q rows
constexpr int PA_P = CK_C + 4;   // f32 pitch of the A / T and M o QK^T rows
static_assert(CK_C * PA_P * 4 == CK_C * PK_P * 2, "A / QKm reuse the K / Q storage");

__device__ __forceinline__ float safe_log(float d) { return logf(fmaxf(d, 1.17549435e-38f)); }

// an empty use: the value is loaded unconditionally (every address read is in
// bounds), instead of the load being moved under the select that keeps it
__device__ __forceinline__ void keep(float& v) { asm volatile("" : "+v"(v)); }

// v_mfma_f32_16x16x4_f32, lane l = 16 g + i: A holds X[i][g], B holds Y[g][i],
// the result Z[4 g + r][i] in slot r
__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// T's block (bi, bj), bi > bj, from the blocks of T already in sA (kept
// transposed above the diagonal, the diagonal blocks D with their zeros):
// S = sum_k A_{bi,k} T_{k,bj} (k-step s takes k = 16 k + 4 s + g), then
// T_{bi,bj} = -D_bi S with S's result slots as the B operand as they stand
// (k-step s pairs lane group g with S's row 4 g + s, so D is read at column
// 4 g + s)
__device__ __forceinline__ void t_block(float (*sA)[CK_C + 4], int bi, int bj, int lane) {
    const int g = lane >> 4, i = lane & 15;
    f32x4 sm = (f32x4)(0.f);
    for (int kb = bj; kb < bi; ++kb) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kk = 4 * s + g;
            const float a = sA[16 * bi + i][16 * kb + kk];
            // T_{kb,bj}[kk][i]: transposed at sA[16 bj + i][16 kb + kk] (D's
            // zeros above its diagonal are stored)
            sm = mfma4(a, sA[16 * bj + i][16 * kb + kk], sm);
        }
    }
    f32x4 t = (f32x4)(0.f);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const int kk = 4 * g + s;
        t = mfma4(sA[16 * bi + kk][16 * bi + i], sm[s], t);   // D_bi[i][kk], transposed
    }
    *(f32x4*)&sA[16 * bj + i][16 * bi + 4 * g] = -t;
}


// inclusive prefix sum over the 64 lanes of a wavefront: DPP row shifts by 1,
// 2, 4 and 8 (zero fill at the row start), then the row totals carried by
// row_bcast:15 and row_bcast:31
__device__ __forceinline__ float wave_prefix_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));
    return v;
}

// The gates the prep reads: beta and decay [T][n_vheads] (gdn_scalars'
// output), or, LOGITS, the logits a and b [T][ab_stride] with A_log and
// dt_bias, from which a lane forms its token's beta and decay itself (the
// gates kernel's functions: the same values).
struct PrepGates {
    const float* beta;     // or a
    const float* decay;    // or b
    const float* A_log;
    const float* dt_bias;
    int stride;            // n_vheads, or ab_stride
};

// One workgroup of 4 waves a (chunk, v head), a grid of chunks x v heads: it
// loads its k head's K and Q rows of the chunk, forms K K^T and Q K^T (wave w
// the 32 x 32 block (w / 2, w % 2)), then its v head's A, T and M o QK^T from
// them with that head's gates, into the head's block of the workspace.
template <bool LOGITS>
__global__ void __launch_bounds__(256)
chunk_prep_kernel(const f16* __restrict__ q, const f16* __restrict__ k, const PrepGates gates,
                  int T, int n_vheads, int qk_stride, int group, char* __restrict__ work) {
    __shared__ __attribute__((aligned(16))) char smem[2 * CK_C * PK_P * 2];
    __shared__ float sG[CK_C], sB[CK_C], sRed[8];
    f16(*sK)[PK_P] = (f16(*)[PK_P])smem;
    f16(*sQ)[PK_P] = (f16(*)[PK_P])(smem + CK_C * PK_P * 2);
    float(*sA)[PA_P] = (float(*)[PA_P])smem;                     // after the products
    float(*sM)[PA_P] = (float(*)[PA_P])(smem + CK_C * PA_P * 4);

    const int c = blockIdx.x, hv_blk = blockIdx.y, hk = hv_blk / group;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ql = lane & 31, hh = lane >> 5;
    const int t0 = c * CK_C;
    const int n = min(CK_C, T - t0);
    const int hv0 = hv_blk;

    // Every global load issued up front and unconditionally, rows clamped to
    // the chunk's last token, past-the-end rows zeroed by a select: K and Q
    // (4 rows x 16 B a thread), the first v head's beta and decay.
    f16x8 kv8[4], qv8[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int idx = tid + 256 * m, i = idx >> 4, c8 = (idx & 15) * 8;
        const size_t off = (size_t)(t0 + min(i, n - 1)) * qk_stride + (size_t)hk * CK_K + c8;
        kv8[m] = *(const f16x8*)(k + off);
        qv8[m] = *(const f16x8*)(q + off);
    }
    const size_t gt = (size_t)(t0 + min(lane, n - 1)) * gates.stride + hv0;
    float dec, bet;
    if constexpr (LOGITS) {
        const float av = gates.beta[gt], bv = gates.decay[gt];
        const float dtb = gates.dt_bias[hv0], A = gates.A_log[hv0];
        dec = gdn_decay(av + dtb, A);
        bet = gdn_beta(bv);
    } else {
        dec = gates.decay[gt];
        bet = gates.beta[gt];
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int idx = tid + 256 * m, i = idx >> 4, c8 = (idx & 15) * 8;
        *(f16x8*)&sK[i][c8] = i < n ? kv8[m] : (f16x8)(0);
        *(f16x8*)&sQ[i][c8] = i < n ? qv8[m] : (f16x8)(0);
    }
    __syncthreads();

    // K K^T and Q K^T: wave w the 32 x 32 block (bi, bj), kept in registers
    const int bi = w >> 1, bj = w & 1;
    f32x16 kk = (f32x16)(0.f), qk = (f32x16)(0.f);
#pragma unroll
    for (int ks = 0; ks < CK_K / 16; ++ks) {
        const f16x8 bk = *(const f16x8*)&sK[32 * bj + ql][16 * ks + 8 * hh];
        const f16x8 ak = *(const f16x8*)&sK[32 * bi + ql][16 * ks + 8 * hh];
        const f16x8 aq = *(const f16x8*)&sQ[32 * bi + ql][16 * ks + 8 * hh];
        kk = __builtin_amdgcn_mfma_f32_32x32x16_f16(ak, bk, kk, 0, 0, 0);
        qk = __builtin_amdgcn_mfma_f32_32x32x16_f16(aq, bk, qk, 0, 0, 0);
    }

    {
        const int hv = hv0;
        char* blk = work + ((size_t)c * n_vheads + hv) * CK_BLK;
        // this head's gates (decay 1 and beta 0 past the end: g stays at the
        // last token's), the in-chunk prefix sums of log decay on wave 0
        if (w == 0) {
            const float gs = wave_prefix_sum(lane < n ? safe_log(dec) : 0.f);
            sG[lane] = gs;
            sB[lane] = lane < n ? bet : 0.f;
        }
        __syncthreads();   // the gates in; every K / Q read (or T / M o QK^T
                           // read of the previous head) done

        // A = strictly lower beta_i e^{g_i - g_j} k_i.k_j and M o QK^T. The
        // 32 x 32 block above the diagonal (wave 1) is left alone: nothing
        // reads M there, and T's blocks below the diagonal are written there
        // (transposed) before anything reads it
        if (bi >= bj) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = 32 * bi + 8 * (r >> 2) + 4 * hh + (r & 3);
                const int j = 32 * bj + ql;
                // e^{g_i - g_j}, taken for every pair (above the diagonal it may
                // be inf, and is not selected)
                const float ratio = fast_exp2((sG[i] - sG[j]) * FL_LOG2E);
                sA[i][j] = j < i ? sB[i] * ratio * kk[r] : 0.f;
                sM[i][j] = j <= i ? ratio * qk[r] : 0.f;
            }
        }
        __syncthreads();

        // T = (I + A)^-1 by blocks of 16, in fp32: T_ii = D_i = (I + A_ii)^-1
        // by forward substitution (wave i, lane j solving column j), then, a
        // block diagonal at a time, T_ij = -D_i sum_{k = j .. i-1} A_ik T_kj on
        // fp32 MFMA. T is kept transposed in sA's upper triangle
        // (T_ij[a][b] at sA[16 j + b][16 i + a]), clear of A below the diagonal.
        if (lane < 16) {
            const int o = 16 * w, j = lane;
            float xd[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float a0 = i == j ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
                for (int m = 0; m < i; ++m) {
                    if (m & 1)
                        a1 = fmaf(-sA[o + i][o + m], xd[m], a1);
                    else
                        a0 = fmaf(-sA[o + i][o + m], xd[m], a0);
                }
                xd[i] = a0 + a1;
            }
            // every element, the zeros above D_w's diagonal included: they land
            // on A_ww, which the remaining steps do not read
#pragma unroll
            for (int i = 0; i < 16; ++i) sA[o + j][o + i] = xd[i];
        }
        __syncthreads();
#pragma unroll
        for (int lv = 1; lv < 4; ++lv) {
            if (w < 4 - lv) t_block(sA, w + lv, w, lane);
            __syncthreads();
        }

        // the scales: block maxima of |T| and |M o QK^T| over their lower
        // triangles, a row of each a pass (the lanes along it: no bank
        // conflicts). sA[r][c] holds T[c][r] where c >= r (A's values below)
        float mt = 0.f, mq = 0.f;
#pragma unroll
        for (int m = 0; m < CK_C * CK_C / 256; ++m) {
            const int idx = tid + 256 * m, r = idx >> 6, c = idx & 63;
            float tv = sA[r][c];
            keep(tv);
            mt = fmaxf(mt, c >= r ? fabsf(tv) : 0.f);
            float qv = sM[r][c];
            keep(qv);
            mq = fmaxf(mq, c <= r ? fabsf(qv) : 0.f);
        }
        mt = wave_max(mt);
        mq = wave_max(mq);
        if (lane == 0) {
            sRed[w] = mt;
            sRed[4 + w] = mq;
        }
        __syncthreads();
        mt = fmaxf(fmaxf(sRed[0], sRed[1]), fmaxf(sRed[2], sRed[3]));
        mq = fmaxf(fmaxf(sRed[4], sRed[5]), fmaxf(sRed[6], sRed[7]));
        float t_inv, q_inv;
        const float t_sc = pow2_scale<7>(mt, t_inv);
        const float q_sc = pow2_scale<7>(mq, q_inv);

        // the operands: slot (T or M o QK^T; block f, lane l = 16 g + i) holds
        // row 16 mb + i at columns 32 kq + kap(g, e), its hi and lo halves
        // 6 KiB apart
        // (which matrix a pass takes is the same for a whole wave: 6 blocks x
        // 64 lanes of T, then 6 of M o QK^T, over 3 passes of 256 threads)
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            const int s = tid + 256 * m;
            const bool isq = s >= CK_NF * 64;
            const int f = (s % (CK_NF * 64)) >> 6, l = s & 63;
            const int g = l >> 4, row = 16 * f_mb(f) + (l & 15), kq = f_kq(f);
            float xs[8];
            if (isq) {   // M o QK^T[row][32 kq + kap(g, e)]: two row segments of 4
                const f32x4 a = *(const f32x4*)&sM[row][32 * kq + 4 * g];
                const f32x4 b = *(const f32x4*)&sM[row][32 * kq + 16 + 4 * g];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xs[e] = a[e] * q_sc;
                    xs[4 + e] = b[e] * q_sc;
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int col = 32 * kq + (e < 4 ? 4 * g + e : 12 + 4 * g + e);
                    float ta = sA[col][row];   // T[row][col], transposed
                    keep(ta);
                    xs[e] = (row >= col ? ta : 0.f) * t_sc;
                }
            }
            f16x8 hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const f16 h = (f16)xs[e];
                hi[e] = h;
                lo[e] = (f16)(xs[e] - (float)h);
            }
            char* dst = blk + (isq ? WS_Q_HI : WS_T_HI) + (f * 64 + l) * 16;
            *(f16x8*)dst = hi;
            *(f16x8*)(dst + WS_OP) = lo;
        }
        if (tid < CK_C) {
            const float gC = sG[CK_C - 1];
            ((float*)(blk + WS_BETA))[tid] = sB[tid];
            ((float*)(blk + WS_EG))[tid] = expf(sG[tid]);
            ((float*)(blk + WS_DK))[tid] = expf(gC - sG[tid]);
            if (tid < 4)
                ((float*)(blk + WS_SC))[tid] =
                    tid == 0 ? expf(gC) : tid == 1 ? t_inv : tid == 2 ? q_inv : 0.f;
        }
    }
}

// ---------------------------------------------------------------------------
// chunk_state_kernel: 32 state rows (v) of a v head a workgroup, 4 wavefronts.
// Waves 0 and 1 (state waves) each hold 16 rows of S and run the recurrence's
// chain: X = K S^T and Q S^T, Y, Delta = T Y, the state update. Waves 2 and 3
// (output waves) each take a state wave's Q S^T and Delta a chunk later, form
// O and store y, and issue every HBM -> LDS copy, so the state waves' chain
// carries neither.
// ---------------------------------------------------------------------------
constexpr int CS_ROWS = 32;   // state rows (v) a workgroup
// A stage (the state waves' operands of a chunk): K and Q rows [64][256 B]
// (16-byte chunk c of row r at c ^ (r & 15)), V columns [64][CS_ROWS] fp16,
// T's hi / lo operands and the gates KiB (workspace bytes 0 .. 16 KiB and
// 32 .. 33 KiB, as in HBM)
constexpr int SA_K = 0, SA_Q = 16384, SA_V = 32768, SA_T = SA_V + CK_C * CS_ROWS * 2,
              SA_G = SA_T + 2 * WS_OP, SA_BYTES = SA_G + 1024;
// B stage (the output waves'): M o QK^T's hi / lo operands (workspace bytes
// 16 .. 32 KiB) and the gates KiB
constexpr int SB_Q = 0, SB_G = 2 * WS_OP, SB_BYTES = SB_G + 1024;
// offsets in the gates KiB: beta, e^g, e^{g_C - g} [64] f32, then e^{g_C},
// 2^-tau, 2^-kappa
constexpr int G_BETA = WS_BETA - WS_BETA, G_EG = WS_EG - WS_BETA, G_DK = WS_DK - WS_BETA,
              G_SC = WS_SC - WS_BETA;
static_assert(WS_T_LO == WS_T_HI + WS_OP && WS_Q_HI == WS_T_LO + WS_OP &&
                  WS_Q_LO == WS_Q_HI + WS_OP && WS_BETA == WS_Q_LO + WS_OP &&
                  CK_BLK == WS_BETA + 1024 && WS_OP % 2048 == 0,
              "workspace block: T, then M o QK^T, then the gates KiB, whole copy pairs");
// LDS: two A stages, two B stages, the hand-over (each state wave's Q S^T
// 2^-s and Delta, [8][64 lanes] f32x4) and each output wave's y tile
// [64 tokens][16 rows] fp16
constexpr int L_A = 0, L_B = 2 * SA_BYTES, L_X = L_B + 2 * SB_BYTES, X_WAVE = 8 * 64 * 16,
              L_Y = L_X + 2 * X_WAVE, CS_LDS = L_Y + 2 * CK_C * 16 * 2;
static_assert(CS_LDS <= 160 * 1024, "the state pass's LDS fits 160 KiB");
// y stores an output wave issues a chunk, after that chunk's copies
constexpr int CS_NSTORE = 2;

typedef __attribute__((address_space(3))) f32x4 lds_f32x4w;
typedef __attribute__((address_space(3))) f16 lds_f16w;

// Per-lane source offsets of output wave wb's copies of a 64-token chunk (the
// base is scalar): K / Q copy n (n = 2 j + wb) brings rows 4 n .. 4 n + 3,
// lane -> row 8 j + rr, rr = 4 wb + lane / 16, and 16-byte chunk
// (lane % 16) ^ (row & 15), row & 15 = rr + 8 (j & 1); V copy n rows
// 16 n + lane / 4, 16 bytes (lane % 4) of the workgroup's 64-byte slice; a
// workspace copy 16 bytes a lane.
struct CsOff {
    uint32_t kq[2], v, w;
};
__device__ __forceinline__ CsOff cs_offsets(int qk_bytes, int v_bytes, int wb, int lane) {
    const int rr = 4 * wb + (lane >> 4), p = lane & 15;
    return {{(uint32_t)(rr * qk_bytes + 16 * (p ^ rr)),
             (uint32_t)(rr * qk_bytes + 16 * (p ^ (rr + 8)))},
            (uint32_t)((lane >> 2) * v_bytes + 16 * (lane & 3)), (uint32_t)(16 * lane)};
}

// Output wave wb's half of the copies of chunk c's A stage into dst: 8 K, 8 Q,
// 2 V and 6 T copies, and (wb = 0) the gates KiB. Rows past the last token
// repeat it (beta is 0 there).
__device__ __forceinline__ void cs_copy_a(uint32_t dst, const char* kb, const char* qb,
                                          const char* vb, const char* wk, int t0, int T,
                                          int qk_bytes, int v_bytes, int wb, int lane,
                                          const CsOff& o) {
    if (T - t0 >= CK_C) {
        const char* kt = kb + (size_t)t0 * qk_bytes;
        const char* qt = qb + (size_t)t0 * qk_bytes;
        const char* vt = vb + (size_t)t0 * v_bytes;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = 2 * j + wb;
            copy16(kt + (size_t)(8 * j) * qk_bytes, o.kq[j & 1], dst + SA_K + 1024 * n);
            copy16(qt + (size_t)(8 * j) * qk_bytes, o.kq[j & 1], dst + SA_Q + 1024 * n);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = 2 * j + wb;
            copy16(vt + (size_t)(16 * n) * v_bytes, o.v, dst + SA_V + 1024 * n);
        }
    } else {
        const int last = T - t0 - 1;
        const int rr = 4 * wb + (lane >> 4), p = lane & 15;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int n = 2 * j + wb, r = 8 * j + rr;
            const size_t ro = (size_t)(t0 + min(r, last)) * qk_bytes + 16 * (p ^ (r & 15));
            copy16_v(kb + ro, __builtin_amdgcn_readfirstlane(dst + SA_K + 1024 * n));
            copy16_v(qb + ro, __builtin_amdgcn_readfirstlane(dst + SA_Q + 1024 * n));
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int n = 2 * j + wb, r = 16 * n + (lane >> 2);
            copy16_v(vb + (size_t)(t0 + min(r, last)) * v_bytes + 16 * (lane & 3),
                     __builtin_amdgcn_readfirstlane(dst + SA_V + 1024 * n));
        }
    }
#pragma unroll
    for (int j = 0; j < WS_OP / 1024; ++j) {
        const int n = 2 * j + wb;
        copy16(wk + WS_T_HI + 1024 * n, o.w, dst + SA_T + 1024 * n);
    }
    if (wb == 0) copy16(wk + WS_BETA, o.w, dst + SA_G);
}

// Output wave wb's half of the copies of chunk c's B stage: 6 M o QK^T copies
// and (wb = 1) the gates KiB.
__device__ __forceinline__ void cs_copy_b(uint32_t dst, const char* wk, int wb, const CsOff& o) {
#pragma unroll
    for (int j = 0; j < WS_OP / 1024; ++j) {
        const int n = 2 * j + wb;
        copy16(wk + WS_Q_HI + 1024 * n, o.w, dst + SB_Q + 1024 * n);
    }
    if (wb == 1) copy16(wk + WS_BETA, o.w, dst + SB_G);
}

// The lane's parts of the swizzled K / Q row addresses, fixed for the kernel:
// the A operand of X = K S^T (or Q S^T) for row block mb, k-step js holds row
// 16 mb + i at k = 32 js + kap(g, e), two 8-byte reads at 16-byte chunks
// (4 js + 2 h + (g >> 1)) ^ i, h = 0, 1 (row & 15 = i for every mb; mb adds
// 16 rows = 4096 bytes)
__device__ __forceinline__ void row_offsets(int g, int i, uint32_t (&ro)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
        ro[j] = i * 256 + 8 * (g & 1) + 16 * ((2 * j + (g >> 1)) ^ i);
}
// stage base (scalar) + lane part, once a chunk: an opaque vector sum, so the
// constant parts of each read (row block, K or Q, k step) stay in the LDS
// instruction's offset field instead of each read adding its own base
__device__ __forceinline__ uint32_t lane_addr(uint32_t sbase, uint32_t lane_part) {
    uint32_t r;
    asm("v_add_u32 %0, %1, %2" : "=v"(r) : "s"(sbase), "v"(lane_part));
    return r;
}
__device__ __forceinline__ f16x8 row_frag(const uint32_t (&ra)[8], uint32_t off, int mb, int js) {
    const f16x4 a = *(volatile lds_f16x4*)(uintptr_t)(ra[2 * js] + off + 4096 * mb);
    const f16x4 b = *(volatile lds_f16x4*)(uintptr_t)(ra[2 * js + 1] + off + 4096 * mb);
    return (f16x8){a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// A operand of K^T Delta' for k rows 16 kb .., token step kq: lane 16 g + i
// gets K[32 kq + kap(g, e)][16 kb + i] by two transposed reads (each: the
// group's 16 lanes read a 4-row x 16-column block, lane i addressing row
// r = 32 kq + 4 g + i / 4 (+ 16), columns 4 (i % 4) .., and receiving column
// i of the four rows). r & 15 = 4 g + i / 4 for both reads and every kq, so the
// lane's part of the address is fixed per kb; kq and the second read add
// 8192 and 4096 bytes.
__device__ __forceinline__ void col_offsets(int g, int i, uint32_t (&co)[8]) {
    const int rr = 4 * g + (i >> 2);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
        co[kb] = rr * 256 + 16 * ((2 * kb + ((i & 3) >> 1)) ^ rr) + 8 * (i & 1);
}
__device__ __forceinline__ f16x8 col_frag(const uint32_t (&ca)[8], int kb, int kq) {
    const uint32_t a0 = ca[kb] + SA_K + 8192 * kq;
    const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)a0);
    const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)(a0 + 4096));
    const f16x4 ah = __builtin_bit_cast(f16x4, a), bh = __builtin_bit_cast(f16x4, b);
    return (f16x8){ah[0], ah[1], ah[2], ah[3], bh[0], bh[1], bh[2], bh[3]};
}

// A state wave: 16 rows v0 .. v0 + 15 of the state, chunk after chunk.
// Barriers (every wave of the workgroup passes the same sequence): E(-1),
// then per chunk c: M(c-1) (the output wave has read the hand-over of c-1),
// E(c) (the hand-over of c written; A stage c free for the copies of c + 2).
__device__ __forceinline__ void cs_state_wave(float* __restrict__ S, uint32_t lds0, int hv, int v0,
                                              int wa, int g, int i, int l, int n_chunks) {
    uint32_t ro[8], co[8];
    row_offsets(g, i, ro);
    col_offsets(g, i, co);
    // the state, st[kb][r] = S[v0 + i][16 kb + 4 g + r]: the result layout of
    // the 16 x 16 blocks of S^T
    float* Sv = S + ((size_t)hv * CK_V + v0 + i) * CK_K + 4 * g;
    f32x4 st[8];
#pragma unroll
    for (int kb8 = 0; kb8 < 8; ++kb8) st[kb8] = *(const f32x4*)(Sv + 16 * kb8);
    tile_done();   // E(-1): stages 0 and 1 landed
    for (int c = 0; c < n_chunks; ++c) {
        const uint32_t sb = lds0 + L_A + (c & 1) * SA_BYTES;
        const uint32_t sg = sb + SA_G;
        uint32_t ra[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) ra[j] = lane_addr(sb, ro[j]);
        // Each phase's LDS operands are read a phase ahead, behind a
        // scheduling fence, so no phase waits on LDS latency. First X's K
        // fragments, which do not wait for the state.
        f16x8 kx[4][4];
#pragma unroll
        for (int js = 0; js < 4; ++js)
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) kx[js][mb] = row_frag(ra, SA_K, mb, js);
        const f32x4 sc = *(lds_f32x4*)(uintptr_t)(sg + G_SC);   // e^{g_C}, 2^-tau, 2^-kappa
        __builtin_amdgcn_sched_barrier(0);

        // the state, scaled and split: B operands of the four k-steps
        float ms = 0.f;
#pragma unroll
        for (int kb8 = 0; kb8 < 8; ++kb8)
#pragma unroll
            for (int r = 0; r < 4; ++r) ms = fmaxf(ms, fabsf(st[kb8][r]));
        float s_inv;
        const float s_sc = pow2_scale<7>(col_max(ms), s_inv);
        f16x8 sh[4], sl[4];
#pragma unroll
        for (int js = 0; js < 4; ++js) split8(st[2 * js], st[2 * js + 1], s_sc, sh[js], sl[js]);
        __builtin_amdgcn_sched_barrier(0);

        // Y's inputs and Q S^T's first fragments, then X = K S^T (two
        // passes), 64 tokens x 16 rows, on four accumulators
        f16x4 vv[4];
        f32x4 be[4], eg[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const int tok = 16 * mb + 4 * g;
            const int vr = tok + (i >> 2);
            vv[mb] = __builtin_bit_cast(
                f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)(
                           sb + SA_V + vr * (CS_ROWS * 2) + 32 * wa + 8 * (i & 3))));
            be[mb] = *(lds_f32x4*)(uintptr_t)(sg + G_BETA + 4 * tok);
            eg[mb] = *(lds_f32x4*)(uintptr_t)(sg + G_EG + 4 * tok);
        }
        f16x8 qa[2][4];
#pragma unroll
        for (int m2 = 0; m2 < 4; ++m2) qa[0][m2] = row_frag(ra, SA_Q, m2, 0);
        f32x4 x[4], qs[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) x[mb] = qs[mb] = (f32x4)(0.f);
#pragma unroll
        for (int js = 0; js < 4; ++js) {
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) x[mb] = mfma16(kx[js][mb], sh[js], x[mb]);
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) x[mb] = mfma16(kx[js][mb], sl[js], x[mb]);
        }
        __builtin_amdgcn_sched_barrier(0);

        // T's operands for Delta; then Q S^T, which only the output wave
        // needs, issued between the blocks of Y = beta (V - e^g X) (tokens
        // 16 mb + 4 g + r, column v0 + i), its next fragments read a k-step
        // ahead
        f16x8 th[CK_NF], tl[CK_NF];
#pragma unroll
        for (int f = 0; f < CK_NF; ++f) {
            const uint32_t fo = (f * 64 + l) * 16;
            th[f] = *(lds_f16x8*)(uintptr_t)(sb + SA_T + fo);
            tl[f] = *(lds_f16x8*)(uintptr_t)(sb + SA_T + WS_OP + fo);
        }
        f32x4 yv[4];
        float my = 0.f;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            if (mb < 3) {
#pragma unroll
                for (int m2 = 0; m2 < 4; ++m2) qa[(mb + 1) & 1][m2] = row_frag(ra, SA_Q, m2, mb + 1);
            }
#pragma unroll
            for (int m2 = 0; m2 < 4; ++m2) qs[m2] = mfma16(qa[mb & 1][m2], sh[mb], qs[m2]);
#pragma unroll
            for (int m2 = 0; m2 < 4; ++m2) qs[m2] = mfma16(qa[mb & 1][m2], sl[mb], qs[m2]);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                yv[mb][r] = be[mb][r] * fmaf(-(eg[mb][r] * s_inv), x[mb][r], (float)vv[mb][r]);
                my = fmaxf(my, fabsf(yv[mb][r]));
            }
        }
        float y_inv;
        const float y_sc = pow2_scale<7>(col_max(my), y_inv);
        f16x8 yh[2], yl[2];
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) split8(yv[2 * kq], yv[2 * kq + 1], y_sc, yh[kq], yl[kq]);
        __builtin_amdgcn_sched_barrier(0);

        // the state update's first K^T fragments and the decays; then
        // Delta = T Y (three passes; T is zero above the diagonal, so rows
        // 0..31 take no columns 32..63)
        uint32_t ca[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) ca[j] = lane_addr(sb, co[j]);
        f16x8 kt[2][2][4];
#pragma unroll
        for (int kq = 0; kq < 2; ++kq)
#pragma unroll
            for (int b = 0; b < 4; ++b) kt[0][kq][b] = col_frag(ca, b, kq);
        f32x4 dk[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
            dk[mb] = *(lds_f32x4*)(uintptr_t)(sg + G_DK + 4 * (16 * mb + 4 * g));
        f32x4 dl[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) dl[mb] = (f32x4)(0.f);
#pragma unroll
        for (int f = 0; f < CK_NF; ++f) {
            const int mb = f_mb(f), kq = f_kq(f);
            dl[mb] = mfma16(th[f], yh[kq], dl[mb]);
        }
#pragma unroll
        for (int f = 0; f < CK_NF; ++f) {
            const int mb = f_mb(f), kq = f_kq(f);
            dl[mb] = mfma16(th[f], yl[kq], dl[mb]);
        }
#pragma unroll
        for (int f = 0; f < CK_NF; ++f) {
            const int mb = f_mb(f), kq = f_kq(f);
            dl[mb] = mfma16(tl[f], yh[kq], dl[mb]);
        }
        __builtin_amdgcn_sched_barrier(0);

        // the second half's K^T fragments; Delta' = e^{g_C - g} Delta for
        // the state update, scaled and split
#pragma unroll
        for (int kq = 0; kq < 2; ++kq)
#pragma unroll
            for (int b = 0; b < 4; ++b) kt[1][kq][b] = col_frag(ca, 4 + b, kq);
        const float d_un = sc[1] * y_inv;
        float md = 0.f;
        f32x4 dp[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                dl[mb][r] *= d_un;
                dp[mb][r] = dk[mb][r] * dl[mb][r];
                md = fmaxf(md, fabsf(dp[mb][r]));
            }
        }
        float p_inv;
        const float p_sc = pow2_scale<7>(col_max(md), p_inv);
        f16x8 ph[2], pl[2];
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) split8(dp[2 * kq], dp[2 * kq + 1], p_sc, ph[kq], pl[kq]);

        // S^T = e^{g_C} S^T + K^T Delta' (K exact: two passes), in two halves
        // of 4 k blocks
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f32x4 u[4];
#pragma unroll
            for (int b = 0; b < 4; ++b) u[b] = (f32x4)(0.f);
#pragma unroll
            for (int kq = 0; kq < 2; ++kq) {
#pragma unroll
                for (int b = 0; b < 4; ++b) u[b] = mfma16(kt[h][kq][b], ph[kq], u[b]);
#pragma unroll
                for (int b = 0; b < 4; ++b) u[b] = mfma16(kt[h][kq][b], pl[kq], u[b]);
            }
#pragma unroll
            for (int b = 0; b < 4; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    st[4 * h + b][r] = fmaf(u[b][r], p_inv, sc[0] * st[4 * h + b][r]);
        }
        __builtin_amdgcn_sched_barrier(0);

        // hand Q S0^T and Delta to the output wave (after it has read the
        // previous chunk's)
        tile_done();   // M(c-1)
        const uint32_t xo = lds0 + L_X + wa * X_WAVE + l * 16;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            *(lds_f32x4w*)(uintptr_t)(xo + 1024 * mb) = qs[mb] * s_inv;
            *(lds_f32x4w*)(uintptr_t)(xo + 1024 * (4 + mb)) = dl[mb];
        }
        tile_done();   // E(c)
    }
#pragma unroll
    for (int kb8 = 0; kb8 < 8; ++kb8) *(f32x4*)(Sv + 16 * kb8) = st[kb8];
}

// An output wave: the paired state wave's rows, a chunk behind it. y at token
// t = 16 mb + 4 g + r, row v0 + i: O = e^g Q S0^T + (M o QK^T) Delta (three
// passes), accumulated scaled by 2^(kappa + eps). Barriers: E(-1), M(-1), then
// per chunk c: E(c), and M(c) but for the last chunk.
__device__ __forceinline__ void cs_output_wave(const f16* q, const f16* k, const f16* v,
                                               f16* __restrict__ y, const char* work,
                                               uint32_t lds0, int T, int n_vheads, int hv, int hk,
                                               int vw0, int v0, int wb, int g, int i, int l,
                                               int n_chunks, int qk_bytes, int v_bytes,
                                               int y_stride, float out_scale) {
    const char* kb = uniform_ptr((const char*)(k + (size_t)hk * CK_K));
    const char* qb = uniform_ptr((const char*)(q + (size_t)hk * CK_K));
    const char* vb = uniform_ptr((const char*)(v + (size_t)hv * CK_V + vw0));
    auto wblock = [&](int c) {
        return uniform_ptr(work + ((size_t)c * n_vheads + hv) * CK_BLK);
    };
    const CsOff off = cs_offsets(qk_bytes, v_bytes, wb, l);
    auto copy_a = [&](int c) {
        cs_copy_a(lds0 + L_A + (c & 1) * SA_BYTES, kb, qb, vb, wblock(c), c * CK_C, T, qk_bytes,
                  v_bytes, wb, l, off);
    };
    auto copy_b = [&](int c) { cs_copy_b(lds0 + L_B + (c & 1) * SB_BYTES, wblock(c), wb, off); };
    copy_a(0);
    copy_b(0);
    if (n_chunks > 1) copy_a(1);
    WAIT_VMCNT(0);
    tile_done();   // E(-1)
    tile_done();   // M(-1)
    const uint32_t yt = lds0 + L_Y + wb * (CK_C * 32);
    for (int c = 0; c < n_chunks; ++c) {
        // this wave's copies for chunk c (B stage) and c + 1 (A stage) landed;
        // only this wave's y stores of chunk c - 1 were issued after them
        WAIT_VMCNT(CS_NSTORE);
        tile_done();   // E(c)
        if (c + 2 < n_chunks) copy_a(c + 2);
        if (c + 1 < n_chunks) copy_b(c + 1);
        const uint32_t xo = lds0 + L_X + wb * X_WAVE + l * 16;
        const uint32_t sbb = lds0 + L_B + (c & 1) * SB_BYTES;
        f32x4 qs[4], dl[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            qs[mb] = *(lds_f32x4*)(uintptr_t)(xo + 1024 * mb);
            dl[mb] = *(lds_f32x4*)(uintptr_t)(xo + 1024 * (4 + mb));
        }
        const f32x4 sc = *(lds_f32x4*)(uintptr_t)(sbb + SB_G + G_SC);
        float mo = 0.f;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) mo = fmaxf(mo, fabsf(dl[mb][r]));
        float o_inv;
        float o_sc = pow2_scale<7>(col_max(mo), o_inv);
        // o_up below brings e^g Q S0^T into the accumulator's scale. Chosen
        // from Delta alone, that scale overflows it for a zero (or nearly
        // zero) Delta row -- a chunk with beta = 0 throughout -- or a zero M o
        // QK^T block (2^-kappa = 2^-126): at most 2^64 2^-kappa, where
        // Delta's own term is below 2^-40 of y
        const float o_cap = 0x1p64f * sc[2];
        if (o_sc > o_cap) {
            o_sc = o_cap;
            o_inv = pow2_inv(o_cap);
        }
        f16x8 oh[2], ol[2];
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) split8(dl[2 * kq], dl[2 * kq + 1], o_sc, oh[kq], ol[kq]);
        const float o_un = sc[2] * o_inv;
        const float o_up = o_sc * __builtin_amdgcn_rcpf(sc[2]);   // 1 / o_un: powers of two, exact
        f32x4 o[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const f32x4 eg = *(lds_f32x4*)(uintptr_t)(sbb + SB_G + G_EG + 4 * (16 * mb + 4 * g));
#pragma unroll
            for (int r = 0; r < 4; ++r) o[mb][r] = eg[r] * qs[mb][r] * o_up;
        }
        f16x8 qh[CK_NF], ql[CK_NF];
#pragma unroll
        for (int f = 0; f < CK_NF; ++f) {
            const uint32_t fo = (f * 64 + l) * 16;
            qh[f] = *(lds_f16x8*)(uintptr_t)(sbb + SB_Q + fo);
            ql[f] = *(lds_f16x8*)(uintptr_t)(sbb + SB_Q + WS_OP + fo);
        }
#pragma unroll
        for (int f = 0; f < CK_NF; ++f) o[f_mb(f)] = mfma16(qh[f], oh[f_kq(f)], o[f_mb(f)]);
#pragma unroll
        for (int f = 0; f < CK_NF; ++f) o[f_mb(f)] = mfma16(qh[f], ol[f_kq(f)], o[f_mb(f)]);
#pragma unroll
        for (int f = 0; f < CK_NF; ++f) o[f_mb(f)] = mfma16(ql[f], oh[f_kq(f)], o[f_mb(f)]);
        // y through this wave's LDS tile: element (token 16 mb + 4 g + r, row
        // i) in, then lane l stores token l's 16 rows (32 bytes) with two
        // 16-byte stores
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                *(lds_f16w*)(uintptr_t)(yt + (16 * mb + 4 * g + r) * 32 + 2 * i) =
                    f16_sat(o[mb][r] * o_un * out_scale);
        const f16x8 y0 = *(lds_f16x8*)(uintptr_t)(yt + l * 32);
        const f16x8 y1 = *(lds_f16x8*)(uintptr_t)(yt + l * 32 + 16);
        const int t0 = c * CK_C;
        if (T - t0 >= CK_C || l < T - t0) {
            f16* yo = y + (size_t)(t0 + l) * y_stride + (size_t)hv * CK_V + v0;
            *(f16x8*)yo = y0;
            *(f16x8*)(yo + 8) = y1;
        }
        if (c + 1 < n_chunks) tile_done();   // M(c)
    }
}

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
chunk_state_kernel(const f16* __restrict__ q, const f16* __restrict__ k,
                   const f16* __restrict__ v, float* __restrict__ S, f16* __restrict__ y, int T,
                   int n_vheads, int qk_stride, int v_stride, int y_stride, float out_scale,
                   int group, const char* __restrict__ work) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    // a v head's workgroups are n_vheads apart in the flat id, so with
    // n_vheads a multiple of 8 (48 here) they land on one XCD (dispatch goes
    // round robin over the 8) and share its L2
    const int hv = blockIdx.x % n_vheads, part = blockIdx.x / n_vheads, hk = hv / group;
    const int l = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = l >> 4, i = l & 15;
    const int vw0 = part * CS_ROWS;
    const uint32_t lds0 = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)smem);
    const int n_chunks = (T + CK_C - 1) / CK_C;
    if (w < 2)
        cs_state_wave(S, lds0, hv, vw0 + 16 * w, w, g, i, l, n_chunks);
    else
        cs_output_wave(q, k, v, y, work, lds0, T, n_vheads, hv, hk, vw0, vw0 + 16 * (w - 2),
                       w - 2, g, i, l, n_chunks, 2 * qk_stride, 2 * v_stride, y_stride, out_scale);
}

// The state pass's dynamic LDS is above the 64 KiB default: raised once per
// device (a mutex: callers may come from several threads).
std::mutex g_cs_mu;
constexpr int CS_MAX_DEVICES = 64;
bool g_cs_done[CS_MAX_DEVICES];

int raise_state_lds_limit() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= CS_MAX_DEVICES) {
        fl::set_error("gdn_chunk_state: no current device below index %d", CS_MAX_DEVICES);
        return FL_ELAUNCH;
    }
    std::lock_guard<std::mutex> lock(g_cs_mu);
    if (g_cs_done[dev]) return FL_OK;
    if (hipFuncSetAttribute((const void*)chunk_state_kernel,
                            hipFuncAttributeMaxDynamicSharedMemorySize, CS_LDS) != hipSuccess) {
        fl::set_error("gdn_chunk_state: cannot raise the dynamic LDS limit to %d bytes", CS_LDS);
        return FL_ELAUNCH;
    }
    g_cs_done[dev] = true;
    return FL_OK;
}

}  // namespace

extern "C" {

size_t fl_gdn_chunked_work_bytes(int T, int n_vheads, int K, int V, int chunk) {
    if (T < 1 || n_vheads < 1 || K != CK_K || V != CK_V || chunk != CK_C) return 0;
    const size_t n_chunks = (size_t)(T + CK_C - 1) / CK_C;
    return n_chunks * n_vheads * CK_BLK;
}

}  // extern "C"

namespace {

int prefill_chunked(const void* q, const void* k, const void* v, const PrepGates& gates,
                    bool logits, float* S, void* y, int T, int n_kheads, int n_vheads, int K,
                    int V, int qk_stride, int v_stride, int y_stride, float out_scale, int group,
                    int chunk, void* work, size_t work_bytes, fl_stream_t stream) {
    FL_REQUIRE(q && k && v && gates.beta && gates.decay && S && y && work, "null pointer");
    FL_REQUIRE(!logits || (gates.A_log && gates.dt_bias && gates.stride >= n_vheads),
               "A_log, dt_bias; ab_stride >= n_vheads");
    FL_REQUIRE(K == CK_K && V == CK_V, "K == V == 128");
    FL_REQUIRE(chunk == CK_C, "chunk == 64");
    FL_REQUIRE(T >= 1, "T >= 1");
    FL_REQUIRE(group >= 1 && (n_vheads - 1) / group < n_kheads, "n_vheads / group <= n_kheads");
    FL_REQUIRE(qk_stride % 8 == 0 && v_stride % 8 == 0 && ((uintptr_t)q & 15u) == 0 &&
                   ((uintptr_t)k & 15u) == 0 && ((uintptr_t)v & 15u) == 0,
               "16-byte aligned q / k / v rows");
    FL_REQUIRE(((uintptr_t)S & 15u) == 0 && ((uintptr_t)work & 15u) == 0 &&
                   ((uintptr_t)y & 15u) == 0 && y_stride % 8 == 0,
               "16-byte aligned S, work and y rows");
    const size_t need = fl_gdn_chunked_work_bytes(T, n_vheads, K, V, chunk);
    if (work_bytes < need) {
        fl::set_error("work: %zu bytes, fl_gdn_chunked_work_bytes asks %zu", work_bytes, need);
        return FL_ESCRATCH;
    }
    const int n_chunks = (T + CK_C - 1) / CK_C;
    if (logits)
        hipLaunchKernelGGL(chunk_prep_kernel<true>, dim3(n_chunks, n_vheads), dim3(256), 0,
                           (hipStream_t)stream, (const f16*)q, (const f16*)k, gates, T, n_vheads,
                           qk_stride, group, (char*)work);
    else
        hipLaunchKernelGGL(chunk_prep_kernel<false>, dim3(n_chunks, n_vheads), dim3(256), 0,
                           (hipStream_t)stream, (const f16*)q, (const f16*)k, gates, T, n_vheads,
                           qk_stride, group, (char*)work);
    int rc = fl::check_launch("gdn_chunk_prep");
    if (rc) return rc;
    rc = raise_state_lds_limit();
    if (rc) return rc;
    hipLaunchKernelGGL(chunk_state_kernel, dim3(n_vheads * (CK_V / CS_ROWS)), dim3(256),
                       CS_LDS, (hipStream_t)stream, (const f16*)q, (const f16*)k, (const f16*)v, S,
                       (f16*)y, T, n_vheads, qk_stride, v_stride, y_stride, out_scale, group,
                       (const char*)work);
    return fl::check_launch("gdn_chunk_state");
}

}  // namespace

extern "C" {

int fl_gdn_prefill_chunked(const void* q, const void* k, const void* v, const float* beta,
                           const float* decay, float* S, void* y, int T, int n_kheads,
                           int n_vheads, int K, int V, int qk_stride, int v_stride, int y_stride,
                           float out_scale, int group, int chunk, void* work, size_t work_bytes,
                           fl_stream_t stream) {
    return prefill_chunked(q, k, v, PrepGates{beta, decay, nullptr, nullptr, n_vheads}, false, S,
                           y, T, n_kheads, n_vheads, K, V, qk_stride, v_stride, y_stride,
                           out_scale, group, chunk, work, work_bytes, stream);
}

int fl_gdn_prefill_chunked_logits(const void* q, const void* k, const void* v, const float* a,
                                  const float* b, int ab_stride, const float* A_log,
                                  const float* dt_bias, float* S, void* y, int T, int n_kheads,
                                  int n_vheads, int K, int V, int qk_stride, int v_stride,
                                  int y_stride, float out_scale, int group, int chunk, void* work,
                                  size_t work_bytes, fl_stream_t stream) {
    return prefill_chunked(q, k, v, PrepGates{a, b, A_log, dt_bias, ab_stride}, true, S, y, T,
                           n_kheads, n_vheads, K, V, qk_stride, v_stride, y_stride, out_scale,
                           group, chunk, work, work_bytes, stream);
}

}  // extern "C"
