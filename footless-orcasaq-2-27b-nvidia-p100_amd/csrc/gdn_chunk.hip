// Chunked (WY / UT transform) Gated DeltaNet prefill on gfx950.
//
// Not in the reference: it runs the delta rule sequentially over a prefill
// (gdn_scan_rows, kernels.cu:2809-2914) and names the chunked scan as the
// undone optimisation (kernels.cu:1788-1791). This computes the same
// recurrence (S *= decay; delta = beta (v - S k); S += delta k^T; o = S q)
// chunk by chunk. For a chunk of C tokens with start state S0 [V][K], g_i the
// in-chunk prefix sum of log(decay):
//   A[i][j] = beta_i e^{g_i - g_j} (k_i . k_j), j < i      (strictly lower)
//   (I + A) W = diag(beta e^{g}) K,  (I + A) U = diag(beta) V   (forward subst.)
//   Delta = U - W S0^T                                       (C x V)
//   O     = diag(e^{g}) Q S0^T + (M o Q K^T) Delta,  M[i][j] = e^{g_i - g_j}, j <= i
//   S_C   = e^{g_C} S0 + Delta^T diag(e^{g_C - g_j}) K
// The decay ratios are formed as e^{g_i - g_j} with j <= i (never 1 / gamma_j,
// which overflows over a chunk of strong decay).
//
// Two launches: chunk_prep (every (chunk, v head) in parallel: Q K^T and K K^T
// on MFMA, W and U by forward substitution in fp32, into the caller's
// workspace), then chunk_state (one workgroup per (v head, 32 state rows),
// sequential over the chunks with the rows in registers, fp32 throughout).
#include "fl_common.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int CK_C = 64;       // tokens a chunk
constexpr int CK_K = 128;      // key dim
constexpr int CK_V = 128;      // value dim
constexpr int CK_ROWS = 32;    // state rows a chunk_state workgroup
constexpr int CK_KP = CK_K + 8;   // f16 pitch of staged K / Q rows
constexpr int CK_AP = 68;      // f32 pitch of the A matrix rows

// workspace block of one (chunk, v head): W [C][K], U [C][V], QKm [C][C], G [C]
constexpr size_t CK_BLK = (size_t)CK_C * CK_K + (size_t)CK_C * CK_V + (size_t)CK_C * CK_C + CK_C;

__device__ __forceinline__ float safe_log(float d) { return logf(fmaxf(d, 1.17549435e-38f)); }

__global__ void __launch_bounds__(256)
chunk_prep_kernel(const f16* __restrict__ q, const f16* __restrict__ k, const f16* __restrict__ v,
                  const float* __restrict__ beta, const float* __restrict__ decay, int T,
                  int n_vheads, int qk_stride, int v_stride, int group, float* __restrict__ work) {
    __shared__ __attribute__((aligned(16))) f16 sK[CK_C][CK_KP];
    __shared__ __attribute__((aligned(16))) f16 sQ[CK_C][CK_KP];
    __shared__ __attribute__((aligned(16))) float sA[CK_C][CK_AP];
    __shared__ float sG[CK_C], sB[CK_C];

    const int c = blockIdx.x, hv = blockIdx.y, hk = hv / group;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ql = lane & 31, hh = lane >> 5;
    const int t0 = c * CK_C;
    const int n = min(CK_C, T - t0);
    float* blk = work + ((size_t)c * n_vheads + hv) * CK_BLK;
    float* Wg = blk;
    float* Ug = Wg + CK_C * CK_K;
    float* QKg = Ug + CK_C * CK_V;
    float* Gg = QKg + CK_C * CK_C;

    // stage K, Q (padding rows zero)
    for (int idx = tid; idx < CK_C * (CK_K / 8); idx += 256) {
        const int i = idx >> 4, c8 = (idx & 15) * 8;
        f16x8 kv8 = (f16x8)(0), qv8 = (f16x8)(0);
        if (i < n) {
            kv8 = *(const f16x8*)(k + (size_t)(t0 + i) * qk_stride + (size_t)hk * CK_K + c8);
            qv8 = *(const f16x8*)(q + (size_t)(t0 + i) * qk_stride + (size_t)hk * CK_K + c8);
        }
        *(f16x8*)&sK[i][c8] = kv8;
        *(f16x8*)&sQ[i][c8] = qv8;
    }
    if (tid < CK_C) {
        sG[tid] = tid < n ? safe_log(decay[(size_t)(t0 + tid) * n_vheads + hv]) : 0.f;
        sB[tid] = tid < n ? beta[(size_t)(t0 + tid) * n_vheads + hv] : 0.f;
    }
    __syncthreads();
    if (tid == 0) {
        float a = 0.f;
        for (int i = 0; i < CK_C; ++i) {
            a += sG[i];
            sG[i] = a;
        }
    }
    __syncthreads();

    // K K^T and Q K^T: wave w takes the 32x32 block (bi, bj)
    {
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
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int i = 32 * bi + 8 * (r >> 2) + 4 * hh + (r & 3);
            const int j = 32 * bj + ql;
            const float ratio = j <= i ? expf(sG[i] - sG[j]) : 0.f;
            sA[i][j] = j < i ? sB[i] * ratio * kk[r] : 0.f;
            QKg[(size_t)i * CK_C + j] = j <= i ? ratio * qk[r] : 0.f;
        }
    }
    __syncthreads();

    // forward substitution: thread c < 128 solves column c of W, c >= 128 of U
    {
        const bool isW = tid < CK_K;
        const int col = isW ? tid : tid - CK_K;
        float x[CK_C];
#pragma unroll
        for (int i = 0; i < CK_C; ++i) {
            float rhs = 0.f;
            if (i < n) {
                if (isW)
                    rhs = sB[i] * expf(sG[i]) * (float)sK[i][col];
                else
                    rhs = sB[i] * (float)v[(size_t)(t0 + i) * v_stride + (size_t)hv * CK_V + col];
            }
            x[i] = rhs;
        }
#pragma unroll
        for (int i = 1; i < CK_C; ++i) {
            float acc = x[i];
#pragma unroll
            for (int j = 0; j < i; j += 4) {
                const f32x4 a4 = *(const f32x4*)&sA[i][j];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (j + e < i) acc = fmaf(-a4[e], x[j + e], acc);
            }
            x[i] = acc;
        }
        float* dst = isW ? Wg : Ug;
#pragma unroll
        for (int i = 0; i < CK_C; ++i) dst[(size_t)i * CK_K + col] = x[i];
    }
    if (tid < CK_C) Gg[tid] = sG[tid];
}

__global__ void __launch_bounds__(256)
chunk_state_kernel(const f16* __restrict__ q, const f16* __restrict__ k, float* __restrict__ S,
                   f16* __restrict__ y, int T, int n_vheads, int qk_stride, int y_stride,
                   float out_scale, int group, const float* __restrict__ work) {
    __shared__ __attribute__((aligned(16))) float sW[CK_C][CK_K];
    __shared__ __attribute__((aligned(16))) float sKf[CK_C][CK_K];
    __shared__ __attribute__((aligned(16))) float sQf[CK_C][CK_K];
    __shared__ __attribute__((aligned(16))) float sQK[CK_C][CK_C];
    __shared__ float sU[CK_C][CK_ROWS];
    __shared__ float sG[CK_C];

    const int rb = blockIdx.x, hv = blockIdx.y, hk = hv / group;
    const int tid = threadIdx.x, ri = tid >> 3, c0 = 4 * (tid & 7);
    const int vi = rb * CK_ROWS + ri;
    float* Srow = S + ((size_t)hv * CK_V + vi) * CK_K + c0;
    float reg[16];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const f32x4 v4 = *(const f32x4*)(Srow + 32 * j);
        reg[4 * j] = v4[0]; reg[4 * j + 1] = v4[1]; reg[4 * j + 2] = v4[2]; reg[4 * j + 3] = v4[3];
    }
    const int n_chunks = (T + CK_C - 1) / CK_C;
    for (int c = 0; c < n_chunks; ++c) {
        const int t0 = c * CK_C;
        const int n = min(CK_C, T - t0);
        const float* blk = work + ((size_t)c * n_vheads + hv) * CK_BLK;
        const float* Wg = blk;
        const float* Ug = Wg + CK_C * CK_K;
        const float* QKg = Ug + CK_C * CK_V;
        const float* Gg = QKg + CK_C * CK_C;
        __syncthreads();   // the previous chunk's reads are done
        for (int idx = tid; idx < CK_C * CK_K / 4; idx += 256) {
            const int i = idx >> 5, c4 = (idx & 31) * 4;
            *(f32x4*)&sW[i][c4] = *(const f32x4*)(Wg + (size_t)i * CK_K + c4);
            f16x4 kh = (f16x4)(0), qh = (f16x4)(0);
            if (i < n) {
                kh = *(const f16x4*)(k + (size_t)(t0 + i) * qk_stride + (size_t)hk * CK_K + c4);
                qh = *(const f16x4*)(q + (size_t)(t0 + i) * qk_stride + (size_t)hk * CK_K + c4);
            }
            *(f32x4*)&sKf[i][c4] = (f32x4){(float)kh[0], (float)kh[1], (float)kh[2], (float)kh[3]};
            *(f32x4*)&sQf[i][c4] = (f32x4){(float)qh[0], (float)qh[1], (float)qh[2], (float)qh[3]};
        }
        for (int idx = tid; idx < CK_C * CK_C / 4; idx += 256) {
            const int i = idx >> 4, c4 = (idx & 15) * 4;
            *(f32x4*)&sQK[i][c4] = *(const f32x4*)(QKg + (size_t)i * CK_C + c4);
        }
        for (int idx = tid; idx < CK_C * CK_ROWS; idx += 256) {
            const int i = idx >> 5, r = idx & 31;
            sU[i][r] = Ug[(size_t)i * CK_V + rb * CK_ROWS + r];
        }
        if (tid < CK_C) sG[tid] = Gg[tid];
        __syncthreads();

        // Delta_i = U_i - W_i . S_row and (Q S0^T)_i, every lane of the row
        float dl[CK_C];
        float qs[CK_C];
#pragma unroll
        for (int i = 0; i < CK_C; ++i) {
            float pw = 0.f, pq = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 w4 = *(const f32x4*)&sW[i][c0 + 32 * j];
                const f32x4 q4 = *(const f32x4*)&sQf[i][c0 + 32 * j];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pw = fmaf(w4[e], reg[4 * j + e], pw);
                    pq = fmaf(q4[e], reg[4 * j + e], pq);
                }
            }
            // sum over the row's 8 lanes (quad xor 1, xor 2, half-row mirror)
            pw += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(pw), 0xB1, 0xF, 0xF, true));
            pq += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(pq), 0xB1, 0xF, 0xF, true));
            pw += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(pw), 0x4E, 0xF, 0xF, true));
            pq += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(pq), 0x4E, 0xF, 0xF, true));
            pw += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(pw), 0x141, 0xF, 0xF, true));
            pq += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(pq), 0x141, 0xF, 0xF, true));
            dl[i] = sU[i][ri] - pw;
            qs[i] = pq;
        }
        // outputs
#pragma unroll
        for (int i = 0; i < CK_C; ++i) {
            float acc = expf(sG[i]) * qs[i];
#pragma unroll
            for (int j = 0; j <= i; ++j) acc = fmaf(sQK[i][j], dl[j], acc);
            if (c0 == 0 && i < n) y[(size_t)(t0 + i) * y_stride + (size_t)hv * CK_V + vi] = f16_sat(acc * out_scale);
        }
        // state: S = e^{g_C} S + sum_j Delta_j e^{g_C - g_j} k_j
        const float gC = sG[CK_C - 1];
        const float eC = expf(gC);
#pragma unroll
        for (int e = 0; e < 16; ++e) reg[e] = reg[e] * eC;
#pragma unroll
        for (int j = 0; j < CK_C; ++j) {
            const float coef = dl[j] * expf(gC - sG[j]);
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const f32x4 k4 = *(const f32x4*)&sKf[j][c0 + 32 * jj];
#pragma unroll
                for (int e = 0; e < 4; ++e) reg[4 * jj + e] = fmaf(coef, k4[e], reg[4 * jj + e]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        *(f32x4*)(Srow + 32 * j) = (f32x4){reg[4 * j], reg[4 * j + 1], reg[4 * j + 2], reg[4 * j + 3]};
}

}  // namespace

extern "C" {

size_t fl_gdn_chunked_work_bytes(int T, int n_vheads, int K, int V, int chunk) {
    if (T < 1 || n_vheads < 1 || K != CK_K || V != CK_V || chunk != CK_C) return 0;
    const size_t n_chunks = (size_t)(T + CK_C - 1) / CK_C;
    return n_chunks * n_vheads * CK_BLK * sizeof(float);
}

int fl_gdn_prefill_chunked(const void* q, const void* k, const void* v, const float* beta,
                           const float* decay, float* S, void* y, int T, int n_kheads,
                           int n_vheads, int K, int V, int qk_stride, int v_stride, int y_stride,
                           float out_scale, int group, int chunk, void* work, size_t work_bytes,
                           fl_stream_t stream) {
    FL_REQUIRE(q && k && v && beta && decay && S && y && work, "null pointer");
    FL_REQUIRE(K == CK_K && V == CK_V, "K == V == 128");
    FL_REQUIRE(chunk == CK_C, "chunk == 64");
    FL_REQUIRE(T >= 1, "T >= 1");
    FL_REQUIRE(group >= 1 && (n_vheads - 1) / group < n_kheads, "n_vheads / group <= n_kheads");
    FL_REQUIRE(qk_stride % 8 == 0 && ((uintptr_t)q & 15u) == 0 && ((uintptr_t)k & 15u) == 0,
               "16-byte aligned q / k rows");
    FL_REQUIRE(((uintptr_t)S & 15u) == 0 && ((uintptr_t)work & 15u) == 0, "16-byte aligned S, work");
    const size_t need = fl_gdn_chunked_work_bytes(T, n_vheads, K, V, chunk);
    if (work_bytes < need) {
        fl::set_error("work: %zu bytes, fl_gdn_chunked_work_bytes asks %zu", work_bytes, need);
        return FL_ESCRATCH;
    }
    const int n_chunks = (T + CK_C - 1) / CK_C;
    hipLaunchKernelGGL(chunk_prep_kernel, dim3(n_chunks, n_vheads), dim3(256), 0,
                       (hipStream_t)stream, (const f16*)q, (const f16*)k, (const f16*)v, beta,
                       decay, T, n_vheads, qk_stride, v_stride, group, (float*)work);
    int rc = fl::check_launch("gdn_chunk_prep");
    if (rc) return rc;
    hipLaunchKernelGGL(chunk_state_kernel, dim3(CK_V / CK_ROWS, n_vheads), dim3(256), 0,
                       (hipStream_t)stream, (const f16*)q, (const f16*)k, S, (f16*)y, T, n_vheads,
                       qk_stride, y_stride, out_scale, group, (const float*)work);
    return fl::check_launch("gdn_chunk_state");
}

}  // extern "C"
