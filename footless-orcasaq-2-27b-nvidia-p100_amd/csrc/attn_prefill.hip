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
// head and walks the causal KV range in 64-row tiles. Per wave and tile:
//   S^T (64 kv x 32 rows) = K Q^T      32 MFMA 32x32x16 f16 (Q in registers)
//   online softmax per query column     one lane pair holds a column
//   O^T (256 d x 32 rows) += V^T P^T    32 MFMA, P straight from the S^T
//                                       accumulators (KV order permuted to
//                                       match, V^T read with it)
// fp32 accumulation throughout; O^T lives in 128 accumulator registers.
// K and V tiles stay in their cache layout ([kv][256] rows) and are copied
// HBM -> LDS by global_load_lds (no registers), two stages deep: the copy of
// tile j+1 runs while tile j is computed. Rows are XOR-swizzled in 16-byte
// chunks (chunk c of row r at c ^ (r % 8)) to spread LDS banks. The V^T
// operand is read with ds_read_b64_tr_b16: in each 16-lane group, lane j
// points at row kb + j/4, columns n0 + 4 (j%4)..+3 of the tile, and lane i
// receives V[kb..kb+3][n0 + i] -- four kv rows of one output dim.
#include "fl_common.hpp"

namespace {

constexpr int PF_WAVES = 4;
constexpr int PF_THREADS = 64 * PF_WAVES;
constexpr int PF_BQ = 32 * PF_WAVES;   // rows a workgroup
constexpr int PF_BK = 64;              // kv rows a tile
constexpr int PF_HD = 256;
constexpr int ROW_B = PF_HD * 2;       // bytes a K / V row
constexpr int TILE_B = PF_BK * ROW_B;  // 32 KiB
constexpr int STAGE_B = 2 * TILE_B;    // K then V

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// byte offset of 16-byte chunk c (0..31) of tile row r
__device__ __forceinline__ int swz(int r, int c) { return r * ROW_B + ((c ^ (r & 7)) << 4); }

// s_waitcnt vmcnt(n) (n < 64), every other counter left alone
#define WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0F70)

// A workgroup barrier that is also a compiler memory barrier but adds no
// s_waitcnt: __syncthreads() would drain vmcnt, i.e. wait for the next tile's
// copies too. The copies a barrier must cover are waited for explicitly
// (WAIT_VMCNT), and every LDS read of a tile has been consumed by an MFMA
// before the barrier that lets the tile be overwritten.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Issue the copy of one 64-row K tile and V tile into an LDS stage: 64 KiB as
// 64 wave instructions of 1 KiB (two rows each), 16 a wave. Rows past kv_end
// read row kv_end - 1 (in bounds; masked by the causal mask, p = 0).
__device__ __forceinline__ void issue_tile(char* stage, const f16* __restrict__ kb,
                                           const f16* __restrict__ vb, size_t rs, int kv0,
                                           int kv_end, int w, int lane) {
#pragma unroll
    for (int n = 0; n < 8; ++n) {
        const int r = 16 * w + 2 * n + (lane >> 5);
        const int c = (lane & 31) ^ (r & 7);
        const int kv = min(kv0 + r, kv_end - 1);
        const size_t off = (size_t)kv * rs + 8 * c;
        __builtin_amdgcn_global_load_lds((const void*)(kb + off),
                                         (lds_void*)(stage + (16 * w + 2 * n) * ROW_B), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((const void*)(vb + off),
                                         (lds_void*)(stage + TILE_B + (16 * w + 2 * n) * ROW_B), 16,
                                         0, 0);
    }
}

__global__ void __launch_bounds__(PF_THREADS)
attn_prefill_kernel(const f16* __restrict__ q, int q_pitch, const f16* __restrict__ kc,
                    const f16* __restrict__ vc, f16* __restrict__ z, int z_pitch, int n_q_heads,
                    int n_kv, int pos0, int T, float sl2, int n_row_tiles) {
    extern __shared__ __attribute__((aligned(16))) char smem[];

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
    const int n_tiles = (kv_end + PF_BK - 1) / PF_BK;

    const size_t rs = (size_t)n_kv * PF_HD;
    const f16* kb = kc + (size_t)h * PF_HD;
    const f16* vb = vc + (size_t)h * PF_HD;

    issue_tile(smem, kb, vb, rs, 0, kv_end, w, lane);

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

    // the ds_read_b64_tr_b16 source coordinates of this lane for V^T block mb:
    // row kb0 + (lane%16)/4, columns 32 mb + 16 ((lane%32)/16) + 4 (lane%4)
    const int tr_r = (lane & 15) >> 2;
    const int tr_d = 16 * ((lane & 31) >> 4) + 4 * (lane & 3);

    for (int j = 0; j < n_tiles; ++j) {
        char* cur = smem + (j & 1) * STAGE_B;
        if (j + 1 < n_tiles) {
            issue_tile(smem + ((j + 1) & 1) * STAGE_B, kb, vb, rs, (j + 1) * PF_BK, kv_end, w, lane);
            WAIT_VMCNT(16);   // this tile's 16 copies done, the next tile's in flight
        } else {
            WAIT_VMCNT(0);
        }
        lds_barrier();
        const int kv0 = j * PF_BK;
        if (kv0 <= wqmax) {
            const char* K = cur;
            const char* Vt = cur + TILE_B;
            f32x16 s0 = (f32x16)(0.f), s1 = (f32x16)(0.f);
#pragma unroll
            for (int ks = 0; ks < 16; ++ks) {
                const f16x8 a0 = *(const f16x8*)(K + swz(ql, 16 * hh + ks));
                const f16x8 a1 = *(const f16x8*)(K + swz(32 + ql, 16 * hh + ks));
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
                const int r0 = 16 * kq + 4 * hh + tr_r;
#pragma unroll
                for (int mb = 0; mb < 8; ++mb) {
                    const int d = 32 * mb + tr_d;
                    const int off = ((d & 7) << 1);
                    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(Vt + swz(r0, d >> 3) + off));
                    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_s16x4*)(Vt + swz(r0 + 8, d >> 3) + off));
                    const f16x4 lf = __builtin_bit_cast(f16x4, lo);
                    const f16x4 hf = __builtin_bit_cast(f16x4, hi);
                    const f16x8 a = {lf[0], lf[1], lf[2], lf[3], hf[0], hf[1], hf[2], hf[3]};
                    o[mb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pk[kq], o[mb], 0, 0, 0);
                }
            }
        }
        lds_barrier();   // this stage is refilled two tiles on
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
    static bool lds_attr_set = false;   // 128 KiB of dynamic LDS is above the default limit
    if (!lds_attr_set) {
        if (hipFuncSetAttribute((const void*)attn_prefill_kernel,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 2 * STAGE_B) !=
            hipSuccess) {
            fl::set_error("attn_prefill: cannot raise the dynamic LDS limit to %d bytes",
                          2 * STAGE_B);
            return FL_ELAUNCH;
        }
        lds_attr_set = true;
    }
    const size_t off = (size_t)layer * max_pos * n_kv_heads * head_dim;
    const int rows = T * (n_q_heads / n_kv_heads);
    const int n_row_tiles = (rows + PF_BQ - 1) / PF_BQ;
    hipLaunchKernelGGL(attn_prefill_kernel, dim3(n_row_tiles, n_kv_heads), dim3(PF_THREADS),
                       2 * STAGE_B,
                       (hipStream_t)stream, (const f16*)q, q_pitch, (const f16*)kcache + off,
                       (const f16*)vcache + off, (f16*)z, z_pitch, n_q_heads, n_kv_heads, pos0, T,
                       scale * FL_LOG2E, n_row_tiles);
    return fl::check_launch("attn_prefill");
}
