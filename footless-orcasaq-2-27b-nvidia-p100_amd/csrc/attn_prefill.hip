// Causal GQA prefill attention over the fp16 KV cache on gfx950 MFMA.
//
// Reference behaviour restated: attention_prefill_fh (kernels.cu:2461-2786)
// and its host call _attn_fh (runtime.py:2943-2959): rows are (token, q head)
// pairs of ONE kv head, token-major (row = t * G + g), so the G = 6 q heads of
// a kv head share every K / V tile; query (t, h) sees cache rows
// [0, pos0 + t]; online softmax in exp2 with the scale folded in; P rounded
// to fp16 for the P V product; z = f16_sat(o / l). The heaviest (latest) row
// tiles launch first (kernels.cu:2522).
//
// Kernel design: a workgroup owns 128 rows (4 wavefronts x 32) of one kv
// head and walks the causal KV range in 64-row tiles staged in LDS (K as
// rows, V transposed to [d][kv]). Per wave and tile:
//   S^T (64 kv x 32 rows) = K Q^T      32 MFMA 32x32x16 f16 (Q in registers)
//   online softmax per query column     one lane pair holds a column
//   O^T (256 d x 32 rows) += V^T P^T    32 MFMA, P straight from the S^T
//                                       accumulators (KV order permuted to
//                                       match, V^T read with it)
// fp32 accumulation throughout; O^T lives in 128 accumulator registers.
#include "fl_common.hpp"

namespace {

constexpr int PF_WAVES = 4;
constexpr int PF_THREADS = 64 * PF_WAVES;
constexpr int PF_BQ = 32 * PF_WAVES;   // rows a workgroup
constexpr int PF_BK = 64;              // kv rows a tile
constexpr int PF_HD = 256;
constexpr int PK_PITCH = PF_HD + 8;    // halves per staged K row (528 B)
constexpr int PV_PITCH = PF_BK + 8;    // halves per staged V^T row (144 B)

__global__ void __launch_bounds__(PF_THREADS)
attn_prefill_kernel(const f16* __restrict__ q, int q_pitch, const f16* __restrict__ kc,
                    const f16* __restrict__ vc, f16* __restrict__ z, int z_pitch, int n_q_heads,
                    int n_kv, int pos0, int T, float sl2, int n_row_tiles) {
    __shared__ __attribute__((aligned(16))) f16 sK[PF_BK][PK_PITCH];
    __shared__ __attribute__((aligned(16))) f16 sVt[PF_HD][PV_PITCH];

    const int tile = n_row_tiles - 1 - (int)blockIdx.x;   // heaviest first
    const int h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ql = lane & 31, hh = lane >> 5;
    const int G = n_q_heads / n_kv;
    const int RT = T * G;
    const int R0 = tile * PF_BQ;
    const int row = R0 + 32 * w + ql;
    const bool rvalid = row < RT;
    const int t = rvalid ? row / G : 0;
    const int g = rvalid ? row - t * G : 0;
    const int qpos = rvalid ? pos0 + t : -1;
    const int wlast = min(R0 + 32 * w + 31, RT - 1);
    const int wqmax = wlast >= R0 + 32 * w ? pos0 + wlast / G : -1;   // the wave's last query position
    const int blast = min(R0 + PF_BQ - 1, RT - 1);
    const int kv_end = pos0 + blast / G + 1;                          // rows any query here sees

    f16x8 qreg[16];   // Q[row][128 hh + 8 ks + 0..7]
    {
        const f16* qrow = q + ((size_t)t * n_q_heads + h * G + g) * q_pitch + 128 * hh;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qreg[ks] = rvalid ? *(const f16x8*)(qrow + 8 * ks) : (f16x8)(0);
    }
    f32x16 o[8];
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) o[mb] = (f32x16)(0.f);
    float m_run = -1e30f, l_run = 0.f;

    const size_t rs = (size_t)n_kv * PF_HD;
    const f16* kb = kc + (size_t)h * PF_HD;
    const f16* vb = vc + (size_t)h * PF_HD;

    for (int kv0 = 0; kv0 < kv_end; kv0 += PF_BK) {
        // ---- stage K (rows) and V (transposed) ----
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int idx = tid + PF_THREADS * i;
            const int r = idx >> 5, c = idx & 31;
            const int kv = kv0 + r;
            const f16x8 val = kv < kv_end ? *(const f16x8*)(kb + (size_t)kv * rs + 8 * c) : (f16x8)(0);
            *(f16x8*)&sK[r][8 * c] = val;
        }
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            const int rbase = 4 * (tid & 15);
            const int dblk = 8 * (tid >> 4) + 128 * pass;
            f16x8 vv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int kv = kv0 + rbase + i;
                vv[i] = kv < kv_end ? *(const f16x8*)(vb + (size_t)kv * rs + dblk) : (f16x8)(0);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e)
                *(f16x4*)&sVt[dblk + e][rbase] = (f16x4){vv[0][e], vv[1][e], vv[2][e], vv[3][e]};
        }
        __syncthreads();

        if (kv0 <= wqmax) {
            f32x16 s0 = (f32x16)(0.f), s1 = (f32x16)(0.f);
#pragma unroll
            for (int ks = 0; ks < 16; ++ks) {
                const f16x8 a0 = *(const f16x8*)&sK[ql][128 * hh + 8 * ks];
                const f16x8 a1 = *(const f16x8*)&sK[32 + ql][128 * hh + 8 * ks];
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qreg[ks], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qreg[ks], s1, 0, 0, 0);
            }
            float sc[32];
            float mt = -INFINITY;
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const int kvr = kv0 + 8 * (rr >> 2) + 4 * hh + (rr & 3);
                sc[rr] = kvr <= qpos ? s0[rr] * sl2 : -INFINITY;
                sc[16 + rr] = kvr + 32 <= qpos ? s1[rr] * sl2 : -INFINITY;
                mt = fmaxf(mt, fmaxf(sc[rr], sc[16 + rr]));
            }
            mt = fmaxf(mt, lane_xor(mt, 32));
            const float m_new = fmaxf(m_run, mt);
            const float corr = fast_exp2(m_run - m_new);
            float psum = 0.f;
            f16x8 pk[4];
#pragma unroll
            for (int rr = 0; rr < 32; ++rr) {
                const float p = fast_exp2(sc[rr] - m_new);
                psum += p;
                pk[rr >> 3][rr & 7] = (f16)p;
            }
            psum += lane_xor(psum, 32);
            l_run = l_run * corr + psum;
            m_run = m_new;
#pragma unroll
            for (int mb = 0; mb < 8; ++mb) o[mb] *= corr;
#pragma unroll
            for (int kq = 0; kq < 4; ++kq) {
                const int kb0 = 32 * (kq >> 1) + 16 * (kq & 1) + 4 * hh;
#pragma unroll
                for (int mb = 0; mb < 8; ++mb) {
                    const f16x4 lo4 = *(const f16x4*)&sVt[32 * mb + ql][kb0];
                    const f16x4 hi4 = *(const f16x4*)&sVt[32 * mb + ql][kb0 + 8];
                    const f16x8 a = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                    o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pk[kq], o[mb], 0, 0, 0);
                }
            }
        }
        __syncthreads();
    }

    if (rvalid) {
        const float inv = 1.f / l_run;
        f16* zrow = z + ((size_t)t * n_q_heads + h * G + g) * z_pitch + 4 * hh;
#pragma unroll
        for (int mb = 0; mb < 8; ++mb)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                *(f16x4*)(zrow + 32 * mb + 8 * r4) =
                    (f16x4){f16_sat(o[mb][4 * r4] * inv), f16_sat(o[mb][4 * r4 + 1] * inv),
                            f16_sat(o[mb][4 * r4 + 2] * inv), f16_sat(o[mb][4 * r4 + 3] * inv)};
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" int fl_attention_prefill(const void* q, int q_pitch, const void* k_new,
                                    const void* v_new, void* kcache, void* vcache, int layer,
                                    int n_q_heads, int n_kv_heads, int head_dim, int pos0,
                                    int max_pos, float scale, int T, void* z, int z_pitch,
                                    fl_stream_t stream) {
    FL_REQUIRE(q && kcache && vcache && z, "null pointer");
    FL_REQUIRE(head_dim == PF_HD, "head_dim must be 256");
    FL_REQUIRE(n_kv_heads > 0 && n_q_heads > 0 && n_q_heads % n_kv_heads == 0,
               "n_q_heads % n_kv_heads");
    FL_REQUIRE(T >= 1 && pos0 >= 0 && layer >= 0 && pos0 + T <= max_pos, "pos0 + T <= max_pos");
    FL_REQUIRE(q_pitch >= head_dim && q_pitch % 8 == 0 && z_pitch >= head_dim && z_pitch % 4 == 0,
               "q_pitch, z_pitch");
    FL_REQUIRE((k_new == nullptr) == (v_new == nullptr), "k_new and v_new together");
    FL_REQUIRE(aligned16(q) && aligned16(kcache) && aligned16(vcache) && ((uintptr_t)z & 7u) == 0,
               "aligned buffers");
    if (k_new != nullptr) {
        const int rc = fl_kv_store(k_new, v_new, kcache, vcache, layer, pos0, T, n_kv_heads,
                                   head_dim, max_pos, stream);
        if (rc) return rc;
    }
    const size_t off = (size_t)layer * max_pos * n_kv_heads * head_dim;
    const int rows = T * (n_q_heads / n_kv_heads);
    const int n_row_tiles = (rows + PF_BQ - 1) / PF_BQ;
    hipLaunchKernelGGL(attn_prefill_kernel, dim3(n_row_tiles, n_kv_heads), dim3(PF_THREADS), 0,
                       (hipStream_t)stream, (const f16*)q, q_pitch, (const f16*)kcache + off,
                       (const f16*)vcache + off, (f16*)z, z_pitch, n_q_heads, n_kv_heads, pos0, T,
                       scale * FL_LOG2E, n_row_tiles);
    return fl::check_launch("attn_prefill");
}
