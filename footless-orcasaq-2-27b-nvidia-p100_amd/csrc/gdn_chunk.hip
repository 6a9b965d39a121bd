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
// workspace), then chunk_state (one workgroup per (v head, 64 state rows),
// sequential over the chunks with the state in MFMA accumulators; fp32 MFMA
// (v_mfma_f32_16x16x4_f32) for the three products of a chunk).
#include "fl_common.hpp"

#pragma clang fp contract(off)

namespace {

constexpr int CK_C = 64;       // tokens a chunk
constexpr int CK_K = 128;      // key dim
constexpr int CK_V = 128;      // value dim
constexpr int CK_KP = CK_K + 8;   // f16 pitch of staged K / Q rows
constexpr int CK_AP = 68;      // f32 pitch of the A matrix rows

// workspace block of one (chunk, v head): W [C][K], U^T [V][C], QKm [C][C], then
// G [C] (in-chunk prefix sums of log decay), e^{G} [C], e^{G_last - G} [C]
constexpr size_t CK_BLK = (size_t)CK_C * CK_K + (size_t)CK_C * CK_V + (size_t)CK_C * CK_C + 3 * CK_C;

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
        if (isW) {
#pragma unroll
            for (int i = 0; i < CK_C; ++i) Wg[(size_t)i * CK_K + col] = x[i];
        } else {   // U transposed: a v row's 64 tokens contiguous
#pragma unroll
            for (int i = 0; i < CK_C; i += 4)
                *(f32x4*)(Ug + (size_t)col * CK_C + i) = (f32x4){x[i], x[i + 1], x[i + 2], x[i + 3]};
        }
    }
    if (tid < CK_C) {
        Gg[tid] = sG[tid];
        Gg[CK_C + tid] = expf(sG[tid]);
        Gg[2 * CK_C + tid] = expf(sG[CK_C - 1] - sG[tid]);
    }
}

// The state pass. A workgroup of 4 waves owns 64 state rows (v) of one v
// head, 16 a wave; a wave keeps its slice of S^T (128 k x 16 v) in 32 fp32
// MFMA accumulators (block mb of 16 k rows, lane l: k = 16 mb + 4 (l/16) + r,
// v = v0 + l%16 -- the D layout of v_mfma_f32_16x16x4_f32). Per chunk:
//   A: P = W S^T, QS = Q S^T              [64 tok x 16 v], 256 MFMA
//      Delta = U - P
//   B: O = e^{g} o QS + QKm Delta         causal blocks only, 40 MFMA
//   C: S^T = e^{g_C} S^T + Kd^T Delta     Kd^T[k][j] = e^{g_C - g_j} k_j[k], 128 MFMA
// The k-step order of each product is permuted so that its B operand is an
// accumulator register of the previous product: step (kq, r) takes k (or the
// token) 16 kq + 4 (l/16) + r, which is register r of block kq. W, QKm, Q and
// K are staged in LDS with row pitches that keep the operand reads on
// distinct banks; Kd^T is read with ds_read_b64_tr_b16 from K's rows.
constexpr int CS_ROWS = 64;          // state rows a workgroup
constexpr int CS_WP = CK_K + 4;      // f32 pitch of staged W rows
constexpr int CS_QKP = CK_C + 4;     // f32 pitch of staged QKm rows
constexpr int CS_QP = CK_K + 8;      // f16 pitch of staged Q rows
constexpr int CS_KP = CK_K + 16;     // f16 pitch of staged K rows
constexpr int CS_OFF_QK = CK_C * CS_WP * 4;
constexpr int CS_OFF_Q = CS_OFF_QK + CK_C * CS_QKP * 4;
constexpr int CS_OFF_K = CS_OFF_Q + CK_C * CS_QP * 2;
constexpr int CS_OFF_G = CS_OFF_K + CK_C * CS_KP * 2;
constexpr int CS_LDS = CS_OFF_G + 3 * CK_C * 4;   // G, e^{G}, e^{G_last - G}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__global__ void __launch_bounds__(256)
chunk_state_kernel(const f16* __restrict__ q, const f16* __restrict__ k, float* __restrict__ S,
                   f16* __restrict__ y, int T, int n_vheads, int qk_stride, int y_stride,
                   float out_scale, int group, const float* __restrict__ work) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    float* sW = (float*)smem;
    float* sQK = (float*)(smem + CS_OFF_QK);
    f16* sQ = (f16*)(smem + CS_OFF_Q);
    f16* sK = (f16*)(smem + CS_OFF_K);
    float* sG = (float*)(smem + CS_OFF_G);

    const int rb = blockIdx.x, hv = blockIdx.y, hk = hv / group;
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6;
    const int m = l & 15, kk = l >> 4;
    const int v0 = rb * CS_ROWS + 16 * w;
    float* Sv = S + ((size_t)hv * CK_V + v0 + m) * CK_K + 4 * kk;   // S[v0 + m][4 kk ...]

    f32x4 st[8];   // S^T block mb: rows k = 16 mb + 4 kk + r, column v0 + m
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) st[mb] = *(const f32x4*)(Sv + 16 * mb);

    // A chunk's operands are loaded into registers one chunk ahead (while the
    // previous chunk computes) and written to LDS after its end barrier.
    // Thread tid stages W rows i = tid / 32 + 8 j (f32x4 at column 4 (tid % 32)),
    // QKm rows tid / 16 + 16 j, Q / K rows tid / 16 + 16 j (f16x8 at 8 (tid % 16)).
    f32x4 pw[8], pqk[4];
    f16x8 pq[4], pk[4];
    float pg[3] = {0.f, 0.f, 0.f};
    f32x4 pu[4];
    auto prefetch = [&](int c) {
        const int t0 = c * CK_C;
        const int n = min(CK_C, T - t0);
        const float* blk = work + ((size_t)c * n_vheads + hv) * CK_BLK;
        const float* Wg = blk;
        const float* UTg = Wg + CK_C * CK_K;
        const float* QKg = UTg + CK_C * CK_V;
        const float* Gg = QKg + CK_C * CK_C;
#pragma unroll
        for (int j = 0; j < 8; ++j)
            pw[j] = *(const f32x4*)(Wg + (size_t)((tid >> 5) + 8 * j) * CK_K + 4 * (tid & 31));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = (tid >> 4) + 16 * j;
            pqk[j] = *(const f32x4*)(QKg + (size_t)i * CK_C + 4 * (tid & 15));
            pk[j] = pq[j] = (f16x8)(0);
            if (i < n) {
                const size_t off = (size_t)(t0 + i) * qk_stride + (size_t)hk * CK_K + 8 * (tid & 15);
                pk[j] = *(const f16x8*)(k + off);
                pq[j] = *(const f16x8*)(q + off);
            }
        }
        if (tid < CK_C) {
            pg[0] = Gg[tid];
            pg[1] = Gg[CK_C + tid];
            pg[2] = Gg[2 * CK_C + tid];
        }
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
            pu[mb] = *(const f32x4*)(UTg + (size_t)(v0 + m) * CK_C + 16 * mb + 4 * kk);
    };
    auto commit = [&]() {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            *(f32x4*)&sW[((tid >> 5) + 8 * j) * CS_WP + 4 * (tid & 31)] = pw[j];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = (tid >> 4) + 16 * j;
            *(f32x4*)&sQK[i * CS_QKP + 4 * (tid & 15)] = pqk[j];
            *(f16x8*)&sK[i * CS_KP + 8 * (tid & 15)] = pk[j];
            *(f16x8*)&sQ[i * CS_QP + 8 * (tid & 15)] = pq[j];
        }
        if (tid < CK_C) {
            sG[tid] = pg[0];
            sG[CK_C + tid] = pg[1];
            sG[2 * CK_C + tid] = pg[2];
        }
    };

    const int n_chunks = (T + CK_C - 1) / CK_C;
    prefetch(0);
    commit();
    for (int c = 0; c < n_chunks; ++c) {
        const int t0 = c * CK_C;
        const int n = min(CK_C, T - t0);
        const f32x4 u[4] = {pu[0], pu[1], pu[2], pu[3]};   // U rows tok = 16 mb + 4 kk + r
        __syncthreads();   // chunk c is in LDS
        if (c + 1 < n_chunks) prefetch(c + 1);

        // A: P = W S^T and QS = Q S^T
        f32x4 p[4], qs[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) p[mb] = qs[mb] = (f32x4)(0.f);
#pragma unroll
        for (int kq = 0; kq < 8; ++kq) {
            f32x4 wf[4], qf[4];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                wf[mb] = *(const f32x4*)&sW[(16 * mb + m) * CS_WP + 16 * kq + 4 * kk];
                const f16x4 qh = *(const f16x4*)&sQ[(16 * mb + m) * CS_QP + 16 * kq + 4 * kk];
                qf[mb] = (f32x4){(float)qh[0], (float)qh[1], (float)qh[2], (float)qh[3]};
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    p[mb] = mfma4(wf[mb][r], st[kq][r], p[mb]);
                    qs[mb] = mfma4(qf[mb][r], st[kq][r], qs[mb]);
                }
        }
        f32x4 d[4];   // Delta rows tok = 16 mb + 4 kk + r, column v0 + m
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) d[mb] = u[mb] - p[mb];

        // B: O = e^{g} o QS + QKm Delta (QKm is zero above the diagonal: blocks kq <= mb)
        f32x4 o[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) o[mb][r] = sG[CK_C + 16 * mb + 4 * kk + r] * qs[mb][r];
#pragma unroll
            for (int kq = 0; kq <= mb; ++kq) {
                const f32x4 af = *(const f32x4*)&sQK[(16 * mb + m) * CS_QKP + 16 * kq + 4 * kk];
#pragma unroll
                for (int r = 0; r < 4; ++r) o[mb] = mfma4(af[r], d[kq][r], o[mb]);
            }
        }
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * mb + 4 * kk + r;
                if (i < n)
                    y[(size_t)(t0 + i) * y_stride + (size_t)hv * CK_V + v0 + m] =
                        f16_sat(o[mb][r] * out_scale);
            }

        // C: S^T = e^{g_C} S^T + Kd^T Delta
        const float eC = sG[CK_C + CK_C - 1];
        float dk[4][4];   // e^{g_C - g_tok}, tok = 16 kq + 4 kk + r
#pragma unroll
        for (int kq = 0; kq < 4; ++kq)
#pragma unroll
            for (int r = 0; r < 4; ++r) dk[kq][r] = sG[2 * CK_C + 16 * kq + 4 * kk + r];
        typedef __attribute__((address_space(3))) const char lds_char;
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) st[mb] *= eC;
#pragma unroll
        for (int kq = 0; kq < 4; ++kq) {
            // lane m of group kk receives K[16 kq + 4 kk + e][16 mb + m], e = 0..3
            const int row = 16 * kq + 4 * kk + (m >> 2);
            f32x4 ka[8];
#pragma unroll
            for (int mb = 0; mb < 8; ++mb) {
                const s16x4 kt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)((lds_char*)sK + 2 * (row * CS_KP + 16 * mb + 4 * (m & 3))));
                const f16x4 kh = __builtin_bit_cast(f16x4, kt);
#pragma unroll
                for (int r = 0; r < 4; ++r) ka[mb][r] = (float)kh[r] * dk[kq][r];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int mb = 0; mb < 8; ++mb) st[mb] = mfma4(ka[mb][r], d[kq][r], st[mb]);
        }
        __syncthreads();   // chunk c's LDS reads are done
        if (c + 1 < n_chunks) commit();
    }
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) *(f32x4*)(Sv + 16 * mb) = st[mb];
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
    static bool lds_attr_set = false;   // above the 64 KiB default of dynamic LDS
    if (!lds_attr_set) {
        if (hipFuncSetAttribute((const void*)chunk_state_kernel,
                                hipFuncAttributeMaxDynamicSharedMemorySize, CS_LDS) != hipSuccess) {
            fl::set_error("gdn_chunk_state: cannot raise the dynamic LDS limit to %d bytes", CS_LDS);
            return FL_ELAUNCH;
        }
        lds_attr_set = true;
    }
    hipLaunchKernelGGL(chunk_state_kernel, dim3(CK_V / CS_ROWS, n_vheads), dim3(256), CS_LDS,
                       (hipStream_t)stream, (const f16*)q, (const f16*)k, S, (f16*)y, T, n_vheads,
                       qk_stride, y_stride, out_scale, group, (const float*)work);
    return fl::check_launch("gdn_chunk_state");
}

}  // extern "C"
