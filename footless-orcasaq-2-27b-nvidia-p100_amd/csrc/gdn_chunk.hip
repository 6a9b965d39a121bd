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
// workspace), then chunk_state (one workgroup per (v head, 16 state rows),
// sequential over the chunks with the state in MFMA accumulators spread over
// four waves; fp32 MFMA (v_mfma_f32_16x16x4_f32) for the three products of a
// chunk).
#include "fl_common.hpp"

#include <mutex>

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
    __shared__ float sG[CK_C], sB[CK_C], sEG[CK_C];

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

    // Every global load of the chunk is issued up front and unconditionally,
    // rows clamped to the chunk's last token, past-the-end rows then zeroed
    // by a select: a load under a branch is waited for inside it, one HBM
    // round trip after another.
    // K, Q (4 rows x 16 B a thread), the gates, and this thread's v column
    // (U threads, tid >= 128: column tid - 128, every token)
    f16x8 kv8[4], qv8[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int idx = tid + 256 * m, i = idx >> 4, c8 = (idx & 15) * 8;
        const size_t off = (size_t)(t0 + min(i, n - 1)) * qk_stride + (size_t)hk * CK_K + c8;
        kv8[m] = *(const f16x8*)(k + off);
        qv8[m] = *(const f16x8*)(q + off);
    }
    const int tg = min(tid & (CK_C - 1), n - 1);
    const float dec = decay[(size_t)(t0 + tg) * n_vheads + hv];
    const float bet = beta[(size_t)(t0 + tg) * n_vheads + hv];
    const bool isW = tid < CK_K;
    const int col = isW ? tid : tid - CK_K;
    f16 vcol[CK_C];
#pragma unroll
    for (int i = 0; i < CK_C; ++i)
        vcol[i] = v[(size_t)(t0 + min(i, n - 1)) * v_stride + (size_t)hv * CK_V + col];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const int idx = tid + 256 * m, i = idx >> 4, c8 = (idx & 15) * 8;
        *(f16x8*)&sK[i][c8] = i < n ? kv8[m] : (f16x8)(0);
        *(f16x8*)&sQ[i][c8] = i < n ? qv8[m] : (f16x8)(0);
    }
    if (tid < CK_C) {
        sG[tid] = tid < n ? safe_log(dec) : 0.f;
        sB[tid] = tid < n ? bet : 0.f;
    }
    __syncthreads();
    if (tid == 0) {   // the in-chunk prefix sums of log decay, in token order
        float g[CK_C];
#pragma unroll
        for (int i = 0; i < CK_C; ++i) g[i] = sG[i];
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < CK_C; ++i) {
            a += g[i];
            sG[i] = a;
        }
    }
    __syncthreads();
    if (tid < CK_C) sEG[tid] = expf(sG[tid]);   // read after the next barrier

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
    // (sB and the staged K rows are zero past the chunk end; v by select)
    {
        float x[CK_C];
#pragma unroll
        for (int i = 0; i < CK_C; ++i)
            x[i] = isW ? sB[i] * sEG[i] * (float)sK[i][col] : (i < n ? sB[i] * (float)vcol[i] : 0.f);
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
        Gg[CK_C + tid] = sEG[tid];
        Gg[2 * CK_C + tid] = expf(sG[CK_C - 1] - sG[tid]);
    }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// The state pass, with the state's k columns split over the 4 waves of a
// workgroup (four waves on each sequential chain, a quarter of its MFMAs
// each). A workgroup owns 16 state rows (v) of one v head; wave w the k
// range [32 w, 32 w + 32) of them, as two 16 x 16 blocks of S^T in the D
// layout of v_mfma_f32_16x16x4_f32 (block kb, lane l: k = 32 w + 16 kb +
// 4 (l / 16) + r, v = v0 + l % 16). Per chunk:
//   A: the wave's partials P_w = W[:, k_w] S^T[k_w, :] and QS_w = Q[:, k_w]
//      S^T[k_w, :] (64 tokens x 16 v, 64 MFMA) into LDS; one barrier;
//      every wave adds the four partials of P in wave order: Delta = U - P
//   B: wave w's token block of O = e^{g} o QS + QKm Delta (QS summed the
//      same way), the causal blocks only
//   C: its k range of S^T = e^{g_C} S^T + Kd^T Delta (32 MFMA; Kd^T read
//      from this wave's K slice in LDS with ds_read_b64_tr_b16)
// Every operand is read by one wave only (W, Q and K by k range, QKm by
// token block; U and the decay factors by all four), straight from the
// workspace into registers: W and Q of the next chunk are requested after
// phase A, the rest after phase C, so each load has half a chunk to land.
// The partial buffers alternate between chunks (one barrier a chunk).
constexpr int CS_ROWS = 16;                       // state rows (v) a workgroup
constexpr int CS_PART = 2 * 4 * 4 * 64;           // f32x4 of one parity: [wave][P | QS][mb][lane]
constexpr int CS_KSLICE = 64 * 64;                // bytes of one wave's K slice (64 tok x 32 k f16)
constexpr int CS_LDS = 2 * CS_PART * 16 + 4 * CS_KSLICE;   // 64 KiB + 16 KiB

__global__ void __launch_bounds__(256, 2)   // two workgroups a CU: <= 256 registers a lane
chunk_state_kernel(const f16* __restrict__ q, const f16* __restrict__ k, float* __restrict__ S,
                   f16* __restrict__ y, int T, int n_vheads, int qk_stride, int y_stride,
                   float out_scale, int group, const float* __restrict__ work) {
    extern __shared__ __attribute__((aligned(16))) char smem[];
    f32x4* part = (f32x4*)smem;
    // grid (v heads, row blocks): the workgroups of a v head, which read the
    // same W / QKm / K of every chunk, are dispatched n_vheads apart and so,
    // with n_vheads a multiple of 8 (48 here), land on one XCD (dispatch goes
    // round robin over the 8) and share its L2
    const int hv = blockIdx.x, rb = blockIdx.y, hk = hv / group;
    const int tid = threadIdx.x, l = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m = l & 15, kk = l >> 4;
    const int v0 = rb * CS_ROWS, k0 = 32 * w;
    char* ksl = smem + 2 * CS_PART * 16 + w * CS_KSLICE;   // this wave's K slice
    typedef __attribute__((address_space(3))) const char lds_char;
    const uint32_t ksl_lds = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)ksl);

    float* Sv = S + ((size_t)hv * CK_V + v0 + m) * CK_K + k0 + 4 * kk;   // S[v0 + m][k0 + 4 kk ..]
    f32x4 st[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) st[kb] = *(const f32x4*)(Sv + 16 * kb);

    // operands of a chunk
    f32x4 wf[4][2];    // W[16 mb + m][k0 + 16 kq + 4 kk ..]
    f16x4 qf[4][2];    // Q[t0 + 16 mb + m][k0 + 16 kq + 4 kk ..]
    f32x4 qkm[4];      // QKm[16 w + m][16 kq + 4 kk ..]
    f32x4 u[4];        // U^T[v0 + m][16 mb + 4 kk ..]
    f32x4 dk[4];       // e^{g_C - g}[16 kq + 4 kk ..]
    f32x4 eg;          // e^{g}[16 w + 4 kk ..]
    float eC;          // e^{g_C}
    f16x8 kv[4];       // K slice staging: 16-byte chunk l + 64 j of the wave's [64 tok][32 k]
    auto blk_of = [&](int c) { return work + ((size_t)c * n_vheads + hv) * CK_BLK; };
    auto load_wq = [&](int c) {
        const int t0 = c * CK_C;
        const int n = min(CK_C, T - t0);
        const float* Wg = blk_of(c);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int kq = 0; kq < 2; ++kq) {
                wf[mb][kq] = *(const f32x4*)(Wg + (size_t)(16 * mb + m) * CK_K + k0 + 16 * kq + 4 * kk);
                const int i = 16 * mb + m;   // row clamped, zeroed by select (no branch)
                const f16x4 qv = *(const f16x4*)(q + (size_t)(t0 + min(i, n - 1)) * qk_stride +
                                                 (size_t)hk * CK_K + k0 + 16 * kq + 4 * kk);
                qf[mb][kq] = i < n ? qv : (f16x4)(0);
            }
    };
    auto load_rest = [&](int c) {
        const int t0 = c * CK_C;
        const int n = min(CK_C, T - t0);
        const float* Wg = blk_of(c);
        const float* UTg = Wg + CK_C * CK_K;
        const float* QKg = UTg + CK_C * CK_V;
        const float* Gg = QKg + CK_C * CK_C;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            qkm[j] = *(const f32x4*)(QKg + (size_t)(16 * w + m) * CK_C + 16 * j + 4 * kk);
            u[j] = *(const f32x4*)(UTg + (size_t)(v0 + m) * CK_C + 16 * j + 4 * kk);
            dk[j] = *(const f32x4*)(Gg + 2 * CK_C + 16 * j + 4 * kk);
        }
        eg = *(const f32x4*)(Gg + CK_C + 16 * w + 4 * kk);
        eC = Gg[2 * CK_C - 1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int idx = l + 64 * j, row = idx >> 2, c16 = idx & 3;
            const f16x8 kr = *(const f16x8*)(k + (size_t)(t0 + min(row, n - 1)) * qk_stride +
                                             (size_t)hk * CK_K + k0 + 8 * c16);
            kv[j] = row < n ? kr : (f16x8)(0);
        }
    };
    // the K slice into LDS: row r's 32-byte half kb at kb ^ ((r / 4) % 2), so
    // the transposed reads of phase C hit 16 distinct 32-byte bank groups
    auto stage_k = [&]() {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int idx = l + 64 * j, row = idx >> 2, c16 = idx & 3;
            const int pos = row * 64 + 32 * ((c16 >> 1) ^ ((row >> 2) & 1)) + 16 * (c16 & 1);
            *(f16x8*)(ksl + pos) = kv[j];
        }
    };

    const int n_chunks = (T + CK_C - 1) / CK_C;
    load_wq(0);
    load_rest(0);
    for (int c = 0; c < n_chunks; ++c) {
        const int t0 = c * CK_C;
        const int n = min(CK_C, T - t0);
        const int par = c & 1;

        // A: this wave's partials of P = W S^T and QS = Q S^T
        f32x4 p[4], qs[4];
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) p[mb] = qs[mb] = (f32x4)(0.f);
#pragma unroll
        for (int kq = 0; kq < 2; ++kq)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int mb = 0; mb < 4; ++mb) {
                    p[mb] = mfma4(wf[mb][kq][r], st[kq][r], p[mb]);
                    qs[mb] = mfma4((float)qf[mb][kq][r], st[kq][r], qs[mb]);
                }
        load_wq(min(c + 1, n_chunks - 1));   // unconditional: see load_rest below
        f32x4* mine = part + par * (CS_PART) + w * (2 * 4 * 64);
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            mine[mb * 64 + l] = p[mb];
            mine[4 * 64 + mb * 64 + l] = qs[mb];
        }
        stage_k();   // this wave's own region: its reads of the previous slice came before
        // The partials are LDS writes: wait for those alone, then the barrier
        // (__syncthreads would first drain vmcnt, i.e. wait for the next
        // chunk's W / Q loads just issued and the y stores, every chunk).
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        const f32x4* all = part + par * (CS_PART);
        f32x4 d[4];   // Delta rows tok = 16 mb + 4 kk + r, column v0 + m
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            f32x4 s = all[mb * 64 + l];
#pragma unroll
            for (int ww = 1; ww < 4; ++ww) s += all[ww * (2 * 4 * 64) + mb * 64 + l];
            d[mb] = u[mb] - s;
        }
        f32x4 qsw = all[4 * 64 + w * 64 + l];   // this wave's token block of QS
#pragma unroll
        for (int ww = 1; ww < 4; ++ww) qsw += all[ww * (2 * 4 * 64) + 4 * 64 + w * 64 + l];

        // B: O for tokens 16 w .. 16 w + 15
        f32x4 o;
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = eg[r] * qsw[r];
#pragma unroll
        for (int kq = 0; kq < 4; ++kq) {
            if (kq > w) break;   // QKm is zero above the diagonal
#pragma unroll
            for (int r = 0; r < 4; ++r) o = mfma4(qkm[kq][r], d[kq][r], o);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = 16 * w + 4 * kk + r;
            if (i < n)
                y[(size_t)(t0 + i) * y_stride + (size_t)hv * CK_V + v0 + m] = f16_sat(o[r] * out_scale);
        }

        // C: S^T = e^{g_C} S^T + Kd^T Delta over this wave's k range
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) st[kb] *= eC;
#pragma unroll
        for (int kq = 0; kq < 4; ++kq) {
            // lane m of group kk receives K[16 kq + 4 kk + e][k0 + 16 kb + m], e = 0..3
            const int row = 16 * kq + 4 * kk + (m >> 2);
            f32x4 ka[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int pos = row * 64 + 32 * (kb ^ ((row >> 2) & 1)) + 8 * (m & 3);
                const s16x4 kt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4*)((lds_char*)(uintptr_t)ksl_lds + pos));
                const f16x4 kh = __builtin_bit_cast(f16x4, kt);
#pragma unroll
                for (int r = 0; r < 4; ++r) ka[kb][r] = (float)kh[r] * dk[kq][r];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) st[kb] = mfma4(ka[kb][r], d[kq][r], st[kb]);
        }
        // Unconditional (the last chunk re-reads its own operands): under a
        // branch the compiler's wait for the K slice before the barrier could
        // not count the loads issued after it and drained them all.
        load_rest(min(c + 1, n_chunks - 1));
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) *(f32x4*)(Sv + 16 * kb) = st[kb];
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
    rc = raise_state_lds_limit();
    if (rc) return rc;
    hipLaunchKernelGGL(chunk_state_kernel, dim3(n_vheads, CK_V / CS_ROWS), dim3(256), CS_LDS,
                       (hipStream_t)stream, (const f16*)q, (const f16*)k, S, (f16*)y, T, n_vheads,
                       qk_stride, y_stride, out_scale, group, (const float*)work);
    return fl::check_launch("gdn_chunk_state");
}

}  // extern "C"
