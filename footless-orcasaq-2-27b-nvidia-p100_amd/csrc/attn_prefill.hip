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
// chunks: chunk c of row r sits at c ^ sw(r), sw(r) = 4 (r % 4) + (r / 4) % 4,
// which keeps both the K reads (16 consecutive rows, one chunk) and the V^T
// reads (8 consecutive rows, 4 chunks) on 16 distinct 16-byte slots of the
// 256-byte bank window (measured on gfx950: 1.3x the K read rate and 1.8x the
// transposed read rate of a c ^ (r % 8) swizzle). The V^T
// operand is read with ds_read_b64_tr_b16: in each 16-lane group, lane j
// points at row kb + j/4, columns n0 + 4 (j%4)..+3 of the tile, and lane i
// receives V[kb..kb+3][n0 + i] -- four kv rows of one output dim.
//
// Over the int8 cache (attention_prefill_fh_q8, kernels.cu:2778-2786) the
// tiles reach LDS through registers instead: each thread loads 64 bytes of a
// K row and of a V row of the next tile (and their two block scales) while
// the current tile is computed, then writes them as fp16(byte * scale) into
// the other stage, in the same swizzled layout, so the compute is the fp16
// kernel's. The reference dequantizes V the same way; its K stays fp32
// (byte * scale exact), here it is rounded to fp16 once.
#include "fl_common.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace {

constexpr int PF_WAVES = 4;
constexpr int PF_THREADS = 64 * PF_WAVES;
constexpr int PF_BQ = 32 * PF_WAVES;   // rows a workgroup
constexpr int PF_BK = 64;              // kv rows a tile
constexpr int PF_HD = 256;
constexpr int ROW_B = PF_HD * 2;       // bytes a K / V row
constexpr int TILE_B = PF_BK * ROW_B;  // 32 KiB
constexpr int LDS_B = 4 * TILE_B;      // K stage 0 | K stage 1 | V stage 0 | V stage 1
constexpr int V_OFF = 2 * TILE_B;
// A column's running max only moves when a tile's max exceeds it by more
// than this (log2 units): P = 2^(s - m) stays <= 256, exact in fp16 range,
// and the O / l rescale is skipped on almost every tile.
constexpr float RESCALE_LOG2 = 8.f;

// the chunk swizzle of tile row r: chunk c is stored at c ^ sw(r)
__device__ __forceinline__ int sw(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// The O^T accumulators live in AGPRs and are touched only through the asm
// below. With compiler-generated MFMAs O would be either in VGPRs (leaving no
// registers to read LDS ahead) or, in AGPRs, given a VGPR home because of the
// rare rescale and copied out of the accumulators on every tile. Hazards the
// compiler cannot see inside asm are covered here: s_nop 2 before each MFMA
// (a VALU write of an A / B operand needs two wait states before the MFMA
// reads it; without them the MFMA reads the register's previous contents),
// s_nop 2 between a VALU result and v_accvgpr_write of it, and acc_settle()
// before the accumulators are read (an MFMA result must leave the pipeline
// before v_accvgpr_read; 24 wait states cover the 8-pass MFMA). MFMAs that
// accumulate into the same registers back to back need no wait states.
__device__ __forceinline__ void acc_zero(f32x16& acc, const f16x8& zero) {
    asm volatile("s_nop 2\n\tv_mfma_f32_32x32x16_f16 %0, %1, %1, 0" : "=a"(acc) : "v"(zero));
}
__device__ __forceinline__ void acc_mfma(f32x16& acc, const f16x8& a, const f16x8& b) {
    asm("s_nop 2\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void acc_settle(f32x16 (&o)[8]) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+a"(o[0]), "+a"(o[1]), "+a"(o[2]), "+a"(o[3]), "+a"(o[4]), "+a"(o[5]),
                   "+a"(o[6]), "+a"(o[7]));
}
// a0..a3 *= c, on accumulator registers
__device__ __forceinline__ void scale4_acc(float& a0, float& a1, float& a2, float& a3, float c) {
    float t0, t1;
    asm volatile(
        "v_accvgpr_read_b32 %4, %0\n\t"
        "v_accvgpr_read_b32 %5, %1\n\t"
        "v_mul_f32 %4, %4, %6\n\t"
        "v_mul_f32 %5, %5, %6\n\t"
        "s_nop 2\n\t"
        "v_accvgpr_write_b32 %0, %4\n\t"
        "v_accvgpr_write_b32 %1, %5\n\t"
        "v_accvgpr_read_b32 %4, %2\n\t"
        "v_accvgpr_read_b32 %5, %3\n\t"
        "v_mul_f32 %4, %4, %6\n\t"
        "v_mul_f32 %5, %5, %6\n\t"
        "s_nop 2\n\t"
        "v_accvgpr_write_b32 %2, %4\n\t"
        "v_accvgpr_write_b32 %3, %5"
        : "+a"(a0), "+a"(a1), "+a"(a2), "+a"(a3), "=&v"(t0), "=&v"(t1)
        : "v"(c));
}
__device__ __forceinline__ void acc_scale(f32x16 (&o)[8], float c) {
    acc_settle(o);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            float x0 = o[mb][e], x1 = o[mb][e + 1], x2 = o[mb][e + 2], x3 = o[mb][e + 3];
            scale4_acc(x0, x1, x2, x3, c);
            o[mb][e] = x0;
            o[mb][e + 1] = x1;
            o[mb][e + 2] = x2;
            o[mb][e + 3] = x3;
        }
}

// O^T[mb] += V^T P^T for the 16 kv rows of step KQ, output blocks 4 HALF..+3.
// b[2 u + s] is this lane's LDS offset for output block 4 HALF + u, row pair
// member s (the swizzle makes it depend on u and s); the rest is a constant,
// +8 KiB per 16 kv rows and +256 B for the upper four output blocks.
template <int KQ, int HALF>
__device__ __forceinline__ void pv_step(f32x16 (&o)[8], const f16x8& pk, const char* lds,
                                        const uint32_t (&b)[8]) {
    constexpr int IMM = 16 * ROW_B * KQ + 256 * HALF;
    typedef __attribute__((address_space(3))) const char lds_char;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)((lds_char*)lds + b[2 * u] + IMM));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s16x4*)((lds_char*)lds + b[2 * u + 1] + IMM));
        const f16x4 lf = __builtin_bit_cast(f16x4, lo);
        const f16x4 hf = __builtin_bit_cast(f16x4, hi);
        const f16x8 av = {lf[0], lf[1], lf[2], lf[3], hf[0], hf[1], hf[2], hf[3]};
        acc_mfma(o[4 * HALF + u], av, pk);
    }
}

// Issue the copy of one 64-row K tile and V tile into LDS stage st: 64 KiB as
// 64 wave instructions of 1 KiB (two rows each), 16 a wave. Wave w copies
// rows 16 w .. 16 w + 15; lane l of the n-th instruction row 16 w + 2 n +
// l / 32, source chunk (l % 32) ^ sw(row), so the tile lands swizzled. The
// row base is wave-uniform (a scalar address), the lane part the per-lane
// offset loff[n]. On the last tile rows past kv_end read row
// kv_end - 1 instead (in bounds; masked by the causal mask, p = 0).
__device__ __forceinline__ void issue_tile(uint32_t lds_base, int st, const char* kb,
                                           const char* vb, uint32_t rsb, int kv0, int kv_end,
                                           int w, int lane, const uint32_t (&loff)[8]) {
    const uint32_t dst0 = lds_base + st * TILE_B + 16 * w * ROW_B;
    if (kv0 + PF_BK <= kv_end) {
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const size_t rb = (size_t)(kv0 + 16 * w + 2 * n) * rsb;
            const uint32_t dst = dst0 + 2 * n * ROW_B;
            copy16(kb + rb, loff[n], dst);
            copy16(vb + rb, loff[n], dst + V_OFF);
        }
    } else {
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const int r = 16 * w + 2 * n + (lane >> 5);
            const int c = (lane & 31) ^ sw(r);
            const int kv = min(kv0 + r, kv_end - 1);
            const size_t off = (size_t)kv * rsb + 16 * c;
            const uint32_t dst = dst0 + 2 * n * ROW_B;
            copy16_v(kb + off, dst);
            copy16_v(vb + off, dst + V_OFF);
        }
    }
}


// The workgroup's (row tile, kv head), heaviest row tiles first. Workgroups
// go to the 8 XCDs round-robin by flat id, and each XCD has its own L2: when
// the kv heads divide 8 and every XCD gets the same number of workgroups,
// XCDs 8 / n_kv * h .. + 8 / n_kv - 1 take all of kv head h's row tiles, so
// an L2 serves one head's K / V prefix instead of all of them (8k prompt:
// ~10 % faster than blockIdx.x / blockIdx.y; the output is identical).
__device__ __forceinline__ void xcd_tile(int n_row_tiles, int n_kv, int& tile, int& h) {
    const int per = 8 % n_kv == 0 ? 8 / n_kv : 0;
    if (per > 0 && n_row_tiles % per == 0) {
        const int id = blockIdx.x + blockIdx.y * gridDim.x;
        const int xcd = id & 7, slot = id >> 3;
        h = xcd / per;
        tile = n_row_tiles - 1 - (slot * per + xcd % per);
    } else {
        tile = n_row_tiles - 1 - (int)blockIdx.x;
        h = blockIdx.y;
    }
}

// One int8 tile row quarter in flight: thread tid holds bytes 64 (tid % 4) ..
// + 63 of K and V row tid / 4 and the two scales of those 64 dims.
struct PfRawQ8 {
    u32x4 k[4], v[4];
    uint32_t ks, vs;
};

// 8 bytes (two dwords) to 8 halves fp16(byte * s)
__device__ __forceinline__ f16x8 deq8(uint32_t a, uint32_t b, f16 s) {
    const f16x2 s2 = {s, s};
    const f16x4 lo = q8_deq4(a, s2), hi = q8_deq4(b, s2);
    return (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// The KV-split form's partials (attention_prefill_fh with gridDim.z > 1,
// kernels.cu:2461-2486 / 2763): split s of a workgroup walks tiles
// [n_tiles s / n, n_tiles (s + 1) / n) of its causal range and leaves, per
// (token, q head), the unnormalised O in pacc [T][heads][n][256], the running
// max in natural-log units in pm and the sum in pd ([T][heads][n]) -- the
// decode partials' layout, so attn_merge_kernel combines them. A split with no
// tile writes the empty partial (m = -1e30, d = 0, O = 0).
struct PfSplit {
    float* pacc;
    float* pm;
    float* pd;
    int n;
};

// Q8: kc / vc are int8 values, ksc / vsc their scales (unused for fp16).
// SPLIT: blockIdx.z is the KV split and the result goes to `sp`, not z.
template <bool Q8, bool SPLIT>
__global__ void __launch_bounds__(PF_THREADS)
attn_prefill_kernel(const f16* __restrict__ q, int q_pitch, const void* __restrict__ kc,
                    const void* __restrict__ vc, const f16* __restrict__ ksc,
                    const f16* __restrict__ vsc, f16* __restrict__ z, int z_pitch, int n_q_heads,
                    int n_kv, int pos0, int T, float sl2, int n_row_tiles, PfSplit sp) {
    extern __shared__ __attribute__((aligned(16))) char smem[];

    int tile, h;
    xcd_tile(n_row_tiles, n_kv, tile, h);
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int G = n_q_heads / n_kv;
    const int RT = T * G;
    const int R0 = tile * PF_BQ;
    const int row = R0 + 32 * w + ql;
    const bool rvalid = row < RT;
    const int t = rvalid ? row / G : 0;
    const int g = rvalid ? row - t * G : 0;
    const int qpos = rvalid ? pos0 + t : -1;
    // Workgroup / wave scalars, marked uniform: the integer divisions are VALU
    // code, and a VGPR-held bound would turn the copy issue into a divergent
    // branch with its scalar base address in VGPRs.
    const int wfirst = R0 + 32 * w;
    const int wlast = min(wfirst + 31, RT - 1);
    const int wqmax = __builtin_amdgcn_readfirstlane(wlast >= wfirst ? pos0 + wlast / G : -1);
    const int wqmin = __builtin_amdgcn_readfirstlane(pos0 + wfirst / G);   // first query position
    const int blast = min(R0 + PF_BQ - 1, RT - 1);
    const int kv_end = __builtin_amdgcn_readfirstlane(pos0 + blast / G + 1);   // rows seen here
    const int n_tiles = (kv_end + PF_BK - 1) / PF_BK;
    // this workgroup's tiles [j_lo, j_hi): all of them, or split s's share
    const int s_idx = SPLIT ? (int)blockIdx.z : 0;
    // (uniform: the divisions are VALU code, and the copies need scalar bases)
    const int j_lo = SPLIT ? __builtin_amdgcn_readfirstlane(n_tiles * s_idx / sp.n) : 0;
    const int j_hi = SPLIT ? __builtin_amdgcn_readfirstlane(n_tiles * (s_idx + 1) / sp.n) : n_tiles;
    if constexpr (SPLIT) {
        if (j_lo == j_hi) {   // an empty split (uniform: the whole workgroup leaves here)
            if (rvalid) {
                const size_t part = ((size_t)t * n_q_heads + h * G + g) * sp.n + s_idx;
                float* acc = sp.pacc + part * PF_HD + 4 * hh;
#pragma unroll
                for (int i = 0; i < 32; ++i) *(f32x4*)(acc + 8 * i) = (f32x4)(0.f);
                if (hh == 0) {
                    sp.pm[part] = -1e30f;
                    sp.pd[part] = 0.f;
                }
            }
            return;
        }
    }

    const uint32_t rsb = (uint32_t)n_kv * ROW_B;   // bytes between cache rows
    const char* kb = uniform_ptr((const char*)((const f16*)kc + (size_t)h * PF_HD));
    const char* vb = uniform_ptr((const char*)((const f16*)vc + (size_t)h * PF_HD));
    uint32_t loff[8];
#pragma unroll
    for (int n = 0; n < 8; ++n)
        loff[n] = (lane >> 5) * rsb + 16 * ((lane & 31) ^ sw(2 * n + (lane >> 5)));
    const uint32_t lds_base = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)smem);

    // int8 staging: this thread's row and quarter of a tile
    const int qr = tid >> 2, qc = tid & 3;
    const char* kb8 = (const char*)kc + (size_t)h * PF_HD + 64 * qc;
    const char* vb8 = (const char*)vc + (size_t)h * PF_HD + 64 * qc;
    const size_t rs8 = (size_t)n_kv * PF_HD;   // bytes between int8 rows
    PfRawQ8 raw;
    // rows past kv_end read row kv_end - 1 (in bounds; masked, p = 0)
    auto q8_load = [&](int kv0) {
        const int kv = min(kv0 + qr, kv_end - 1);
        const u32x4* ks = (const u32x4*)(kb8 + (size_t)kv * rs8);
        const u32x4* vs = (const u32x4*)(vb8 + (size_t)kv * rs8);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            raw.k[i] = ks[i];
            raw.v[i] = __builtin_nontemporal_load(vs + i);
        }
        const size_t so = ((size_t)kv * n_kv + h) * 8 + 2 * qc;
        raw.ks = *(const uint32_t*)(ksc + so);
        raw.vs = *(const uint32_t*)(vsc + so);
    };
    // into LDS stage st: chunk 8 qc + i of row qr at (8 qc + i) ^ sw(qr)
    auto q8_store = [&](int st) {
        char* kd = smem + st * TILE_B + qr * ROW_B;
        const f16x2 ks2 = __builtin_bit_cast(f16x2, raw.ks), vs2 = __builtin_bit_cast(f16x2, raw.vs);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int off = 16 * ((8 * qc + i) ^ sw(qr));
            const u32x4 kw = raw.k[i >> 1], vw = raw.v[i >> 1];
            *(f16x8*)(kd + off) = (i & 1) ? deq8(kw.z, kw.w, ks2[i >> 2]) : deq8(kw.x, kw.y, ks2[i >> 2]);
            *(f16x8*)(kd + V_OFF + off) =
                (i & 1) ? deq8(vw.z, vw.w, vs2[i >> 2]) : deq8(vw.x, vw.y, vs2[i >> 2]);
        }
    };

    if constexpr (Q8)
        q8_load(j_lo * PF_BK);
    else
        issue_tile(lds_base, 0, kb, vb, rsb, j_lo * PF_BK, kv_end, w, lane, loff);

    f16x8 qreg[16];   // Q[row][128 hh + 8 ks + 0..7]
    {
        const f16* qrow = q + ((size_t)t * n_q_heads + h * G + g) * q_pitch + 128 * hh;
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) qreg[ks] = rvalid ? *(const f16x8*)(qrow + 8 * ks) : (f16x8)(0);
    }
    // Wait for Q (and tile 0) here: left to the compiler, the wait for Q lands
    // inside the tile loop as vmcnt(0) -- on every tile, and on the next tile's
    // copy with it.
    WAIT_VMCNT(0);
    if constexpr (Q8) {
        q8_store(0);
        tile_done();
    }
    f32x16 o[8];
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) acc_zero(o[mb], (f16x8)(0));
    float m_run = -1e30f, l_run = 0.f;

    // K operand, k-step ks: row ql (and 32 + ql, +16 KiB) chunk 16 hh + ks,
    // stored at 16 hh + (ks ^ sw(ql)): the byte offset is koff ^ 16 ks.
    const uint32_t koff = ql * ROW_B + 256 * hh + 16 * sw(ql);
    // V^T operand (ds_read_b64_tr_b16): this lane points at tile row
    // 16 kq + 4 hh + tr_r + 8 s, output dims 32 mb + tr_d .. + 3. With
    // mb = 4 mh + u and sw(row) = 4 tr_r + hh + 2 s that is chunk
    // 16 mh + 4 (u ^ tr_r) + (tr_d / 8 ^ (hh + 2 s)): one offset per (u, s),
    // 8 KiB kq + 256 mh as the immediate.
    const int tr_r = (lane & 15) >> 2;
    const int tr_d = 16 * ((lane & 31) >> 4) + 4 * (lane & 3);
    uint32_t troff[8];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
            troff[2 * u + s2] = (4 * hh + tr_r + 8 * s2) * ROW_B + 64 * (u ^ tr_r) +
                                16 * ((tr_d >> 3) ^ (hh + 2 * s2)) + 2 * (tr_d & 7);

    typedef __attribute__((address_space(3))) const f16x8 lds_f16x8;
    typedef __attribute__((address_space(3))) const char lds_char;
    for (int j = j_lo; j < j_hi; ++j) {
        const int st = (j - j_lo) & 1;
        if constexpr (Q8) {
            if (j + 1 < j_hi) q8_load((j + 1) * PF_BK);   // in registers during the math
        } else {
            if (j + 1 < j_hi) {
                issue_tile(lds_base, st ^ 1, kb, vb, rsb, (j + 1) * PF_BK, kv_end, w, lane, loff);
                WAIT_VMCNT(16);   // this tile's 16 copies done, the next tile's in flight
            } else {
                WAIT_VMCNT(0);
            }
            tile_ready();
        }
        const int kv0 = j * PF_BK;
        if (kv0 <= wqmax) {
            const uint32_t kst = koff + st * TILE_B;
            f32x16 s0 = (f32x16)(0.f), s1 = (f32x16)(0.f);
            // K fragments read KPF k-steps ahead of their MFMAs
            constexpr int KPF = 3;
            f16x8 ka0[KPF], ka1[KPF];
#pragma unroll
            for (int ks = 0; ks < KPF; ++ks) {
                lds_char* ka = (lds_char*)smem + (kst ^ (16 * ks));
                ka0[ks] = *(lds_f16x8*)ka;
                ka1[ks] = *(lds_f16x8*)(ka + 32 * ROW_B);
            }
#pragma unroll
            for (int ks = 0; ks < 16; ++ks) {
                const f16x8 a0 = ka0[ks % KPF], a1 = ka1[ks % KPF];
                if (ks + KPF < 16) {
                    lds_char* ka = (lds_char*)smem + (kst ^ (16 * (ks + KPF)));
                    ka0[ks % KPF] = *(lds_f16x8*)ka;
                    ka1[ks % KPF] = *(lds_f16x8*)(ka + 32 * ROW_B);
                }
                s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qreg[ks], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qreg[ks], s1, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead (the scheduler sinks them)
            }
            // raw scores; the causal mask only on tiles that cross the diagonal
            float sc[32];
            if (kv0 + PF_BK - 1 <= wqmin) {
#pragma unroll
                for (int rr = 0; rr < 16; ++rr) {
                    sc[rr] = s0[rr];
                    sc[16 + rr] = s1[rr];
                }
            } else {
                // score rr of s0 is kv row kv0 + 8 (rr / 4) + 4 hh + rr % 4 (s1:
                // + 32); it is visible when that row <= qpos
                const int lim = qpos - kv0 - 4 * hh;
#pragma unroll
                for (int rr = 0; rr < 16; ++rr) {
                    const int d = 8 * (rr >> 2) + (rr & 3);
                    sc[rr] = d <= lim ? s0[rr] : -INFINITY;
                    sc[16 + rr] = d + 32 <= lim ? s1[rr] : -INFINITY;
                }
            }
            float mt = sc[0];
#pragma unroll
            for (int rr = 1; rr < 32; ++rr) mt = fmaxf(mt, sc[rr]);
            mt = pair32_max(mt) * sl2;
            if (__any(mt > m_run + RESCALE_LOG2)) {   // always on a wave's first tile, rarely after
                const float m_new = fmaxf(m_run, mt);
                const float corr = fast_exp2(m_run - m_new);
                m_run = m_new;
                l_run *= corr;
                acc_scale(o, corr);
            }
            float psum = 0.f;
            f16x8 pk[4];
#pragma unroll
            for (int rr = 0; rr < 32; ++rr) {
                const float p = fast_exp2(fmaf(sc[rr], sl2, -m_run));
                psum += p;
                pk[rr >> 3][rr & 7] = (f16)p;
            }
            l_run += pair32_sum(psum);
            const char* vt = smem + V_OFF + st * TILE_B;
            pv_step<0, 0>(o, pk[0], vt, troff);
            pv_step<0, 1>(o, pk[0], vt, troff);
            pv_step<1, 0>(o, pk[1], vt, troff);
            pv_step<1, 1>(o, pk[1], vt, troff);
            pv_step<2, 0>(o, pk[2], vt, troff);
            pv_step<2, 1>(o, pk[2], vt, troff);
            pv_step<3, 0>(o, pk[3], vt, troff);
            pv_step<3, 1>(o, pk[3], vt, troff);
        }
        if constexpr (Q8) {
            // the other stage's last readers passed the previous barrier
            if (j + 1 < j_hi) q8_store(st ^ 1);
        }
        tile_done();   // this stage is refilled two tiles on
    }

    acc_settle(o);
    if constexpr (SPLIT) {
        if (rvalid) {
            // dims 32 mb + 8 r4 + 4 hh + 0..3 of O, unnormalised; m in natural-log units
            const size_t part = ((size_t)t * n_q_heads + h * G + g) * sp.n + s_idx;
            float* acc = sp.pacc + part * PF_HD + 4 * hh;
#pragma unroll
            for (int mb = 0; mb < 8; ++mb)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    *(f32x4*)(acc + 32 * mb + 8 * r4) =
                        (f32x4){o[mb][4 * r4], o[mb][4 * r4 + 1], o[mb][4 * r4 + 2],
                                o[mb][4 * r4 + 3]};
            if (hh == 0) {
                sp.pm[part] = l_run > 0.f ? m_run * FL_LN2 : -1e30f;
                sp.pd[part] = l_run;
            }
        }
        return;
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

// One HBM -> LDS copy of 16 bytes a lane to LDS dst + IMM (+ 16 lane). m0 is
// set inside the asm from a wave-uniform base and an immediate, so the
// compiler keeps no per-copy LDS addresses in SGPRs (it would otherwise hoist
// all of them out of the tile loop); the asm declares m0 as its output.
template <int IMM>
__device__ __forceinline__ void copy16_at(const char* sbase, uint32_t voff, uint32_t dst) {
    uint32_t m0v;
    asm volatile("s_add_u32 m0, %3, %4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 : "={m0}"(m0v)
                 : "v"(voff), "s"(sbase), "s"(dst), "i"(IMM));
}

// ---------------------------------------------------------------------------
// fp16 cache, long prompts: 64 query rows a wave. A workgroup owns 256 rows
// (4 waves x 64) of one kv head and walks the causal KV range in 32-row
// tiles. Per wave and tile the 64 rows are two 32-column MFMA blocks (nb = 0,
// 1) that share every K and V fragment read from LDS:
//   S^T (32 kv x 64 rows) = K Q^T      16 k-steps x 2 MFMA 32x32x16 (one
//                                       K fragment per k-step, Q in
//                                       registers)
//   online softmax per query column     as attn_prefill_kernel, per block
//   O^T (256 d x 64 rows) += V^T P^T    8 dim blocks x 2 k-steps x 2 MFMA
//                                       (one V^T fragment per pair)
// so a wave reads 32 KiB of K and V from LDS per 64 MFMAs (attn_prefill_
// kernel: 64 KiB) and the workgroup copies 32 KiB from HBM per 256 x 32 query
// x key pairs (there: 64 KiB per 128 x 64). O^T is 256 AGPRs (all of them),
// Q^T 128 VGPRs. Tiles are copied HBM -> LDS by global_load_lds, R64_DIST
// tiles ahead of the one computed, into R64_NST = R64_DIST + 1 stages of 32
// KiB (K | V), with the swizzle of attn_prefill_kernel. Same arithmetic as
// attn_prefill_kernel (fp32 scores, exp2 with the scale folded in, the
// lazy rescale, P rounded to fp16); 32-row tiles move the rescale points,
// so the two kernels agree to rounding, not bit for bit.
// ---------------------------------------------------------------------------
constexpr int R64_BQ = 256;                 // rows a workgroup
constexpr int R64_BK = 32;                  // kv rows a tile
constexpr int R64_TILE = R64_BK * ROW_B;    // 16 KiB: K (or V) of a tile
constexpr int R64_STAGE = 2 * R64_TILE;     // K | V
// Tiles copied ahead and K fragments read ahead: 2, 3 and 4 tiles and 2, 3
// and 4 k-steps measured the same within noise at 8k and 32k.
constexpr int R64_DIST = 3;
constexpr int R64_KPF = 3;
constexpr int R64_NST = R64_DIST + 1;
constexpr int R64_LDS = R64_NST * R64_STAGE;   // 128 KiB at R64_DIST 3
static_assert(R64_LDS <= 160 * 1024, "R64_DIST: LDS <= 160 KiB");
constexpr int R64_COPIES = 8;               // copy instructions a wave a tile (4 K + 4 V)
// the r64 kernel from this many workgroups up (T >= 4096 at 24 / 4 heads).
// Same-box A/B, r64 against the 128-row kernel: 192 workgroups (T = 2048)
// 156 against 100 us, 384 (T = 4096) 289-299 against 297-315 us, 480 (T =
// 5120) 378 against 410-422 us.
constexpr int R64_MIN_WGS = 384;

// Persistent launch: one workgroup a CU, each walking the row tiles of its
// bin, heaviest first. A CU runs one 128 KiB-LDS workgroup at a time, and
// the hardware hands an XCD's workgroups round-robin to its 4 shader engines
// in launch order, a workgroup waiting for a CU of its own engine and the
// ones behind it waiting for it; with 3 row tiles a CU (T = 8192) that left
// 12 % of the CU time idle, the heavier tiles stranded behind the lighter.
// The host balances the bins (kv tiles walked + a fixed cost a row tile).
// Plan layout: v[0 .. bins] = offsets of each bin's list in the row-tile
// indices at v[bins + 1 ..].
constexpr int R64_PLAN_MAX = 1024;     // bins + 1 + row tiles a kv head: 2 KiB of arguments
constexpr int R64_ITEM_COST = 5;       // a row tile's fixed cost in kv tiles (Q, pipeline fill, z)
struct R64Plan {
    uint16_t v[R64_PLAN_MAX];
};

// Copy tile kv0 (K and V, 32 rows each) into the stage at dst: wave w copies
// rows 8 w .. 8 w + 7, two a copy instruction (as issue_rows: loff[n] = this
// lane's source offset from row 8 w, row 2 n + lane / 32, swizzled chunk).
__device__ __forceinline__ void r64_issue(uint32_t dst, const char* kb, const char* vb,
                                          uint32_t rsb, int kv0, int kv_end, int w, int lane,
                                          const uint32_t (&loff)[4]) {
    const uint32_t d0 = __builtin_amdgcn_readfirstlane(dst + 8 * w * ROW_B);
    if (kv0 + R64_BK <= kv_end) {
        const size_t ro = (size_t)(kv0 + 8 * w) * rsb;
        const char* kr = kb + ro;
        const char* vr = vb + ro;
        copy16_at<0 * ROW_B>(kr, loff[0], d0);
        copy16_at<2 * ROW_B>(kr, loff[1], d0);
        copy16_at<4 * ROW_B>(kr, loff[2], d0);
        copy16_at<6 * ROW_B>(kr, loff[3], d0);
        copy16_at<R64_TILE + 0 * ROW_B>(vr, loff[0], d0);
        copy16_at<R64_TILE + 2 * ROW_B>(vr, loff[1], d0);
        copy16_at<R64_TILE + 4 * ROW_B>(vr, loff[2], d0);
        copy16_at<R64_TILE + 6 * ROW_B>(vr, loff[3], d0);
    } else {
        uint32_t vo[4];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            const int r = 8 * w + 2 * n + (lane >> 5);
            const int c = (lane & 31) ^ sw(r);
            vo[n] = (uint32_t)min(kv0 + r, kv_end - 1) * rsb + 16 * c;
        }
        copy16_at<0 * ROW_B>(kb, vo[0], d0);
        copy16_at<2 * ROW_B>(kb, vo[1], d0);
        copy16_at<4 * ROW_B>(kb, vo[2], d0);
        copy16_at<6 * ROW_B>(kb, vo[3], d0);
        copy16_at<R64_TILE + 0 * ROW_B>(vb, vo[0], d0);
        copy16_at<R64_TILE + 2 * ROW_B>(vb, vo[1], d0);
        copy16_at<R64_TILE + 4 * ROW_B>(vb, vo[2], d0);
        copy16_at<R64_TILE + 6 * ROW_B>(vb, vo[3], d0);
    }
}

// Softmax of one 32-column block of a tile (one query column per lane pair,
// 16 of its 32 scores a lane): the masked scores (diag: the tile crosses this
// wave's diagonal; score r is kv row 8 (r / 4) + 4 hh + r % 4 of the tile,
// kept when that is <= lim), the running max / sum update with the lazy
// rescale of this block's O^T, and P in fp16 (pk[kq] = scores 8 kq .. + 7,
// the B operand of the PV k-step kq).
__device__ __forceinline__ void r64_softmax(f32x16& s, bool diag, int lim, float sl2,
                                            float& m_run, float& l_run, f32x16 (&o)[8],
                                            f16x8 (&pk)[2]) {
    if (diag) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 8 * (r >> 2) + (r & 3) <= lim ? s[r] : -INFINITY;
    }
    float mt = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
    mt = pair32_max(mt) * sl2;
    if (__any(mt > m_run + RESCALE_LOG2)) {   // always on a wave's first tile, rarely after
        const float m_new = fmaxf(m_run, mt);
        const float corr = fast_exp2(m_run - m_new);
        m_run = m_new;
        l_run *= corr;
        acc_scale(o, corr);
    }
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float p = fast_exp2(fmaf(s[r], sl2, -m_run));
        psum += p;
        pk[r >> 3][r & 7] = (f16)p;
    }
    l_run += pair32_sum(psum);
}

// The 8 V^T fragments (ds_read_b64_tr_b16) of PV step n: k-step kq = n / 2
// (kv rows 16 kq ..), dim blocks 4 (n % 2) .. + 3; b: this lane's offsets
// (the troff of attn_prefill_kernel).
__device__ __forceinline__ void r64_vfrags(s16x4 (&vb)[8], const char* vt,
                                           const uint32_t (&b)[8], int n) {
    const int imm = 16 * ROW_B * (n >> 1) + 256 * (n & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i)
        vb[i] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vt + b[i] + imm));
}

// SPLIT: blockIdx.z is the KV split (tile grid only, bins == 0): the
// workgroup walks tiles [n s / S, n (s + 1) / S) of its causal range (n
// tiles) and leaves the partials in `sp`, as attn_prefill_kernel<Q8, true>.
template <bool SPLIT>
__global__ void __launch_bounds__(PF_THREADS)
attn_prefill_r64_kernel(const f16* __restrict__ q, int q_pitch, const f16* __restrict__ kc,
                        const f16* __restrict__ vc, f16* __restrict__ z, int z_pitch,
                        int n_q_heads, int n_kv, int pos0, int T, float sl2, int n_row_tiles,
                        int bins, const R64Plan plan, PfSplit sp) {
    extern __shared__ __attribute__((aligned(16))) char smem[];

    // This workgroup's row tiles: one, of a grid of row tiles x kv heads
    // (bins == 0), or the list of its bin, of a grid of one workgroup a CU.
    int h, tile = 0, item0 = 0, n_items = 1;
    if (bins == 0) {
        xcd_tile(n_row_tiles, n_kv, tile, h);
    } else {
        const int id = blockIdx.x, xcd = id & 7, per = 8 / n_kv;
        h = xcd / per;
        const int bin = (id >> 3) * per + xcd % per;
        item0 = plan.v[bin];
        n_items = plan.v[bin + 1] - item0;
    }
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ql = lane & 31, hh = lane >> 5;
    const int G = n_q_heads / n_kv;
    const int RT = T * G;
    const uint32_t rsb = (uint32_t)n_kv * ROW_B;
    const char* kb = uniform_ptr((const char*)(kc + (size_t)h * PF_HD));
    const char* vb = uniform_ptr((const char*)(vc + (size_t)h * PF_HD));
    uint32_t loff[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
        const int r = 2 * n + (lane >> 5);   // row from 8 w
        loff[n] = r * rsb + 16 * ((lane & 31) ^ sw(8 * w + r));
    }
    const uint32_t lds_base = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)smem);
    // K operand of k-step ks: tile row ql, chunk 16 hh + ks, at 16 hh + (ks ^ sw(ql))
    const uint32_t koff = ql * ROW_B + 256 * hh + 16 * sw(ql);
    const int tr_r = (lane & 15) >> 2;
    const int tr_d = 16 * ((lane & 31) >> 4) + 4 * (lane & 3);
    uint32_t troff[8];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
            troff[2 * u + s2] = (4 * hh + tr_r + 8 * s2) * ROW_B + 64 * (u ^ tr_r) +
                                16 * ((tr_d >> 3) ^ (hh + 2 * s2)) + 2 * (tr_d & 7);

    for (int it = 0; it < n_items; ++it) {
        if (bins != 0) tile = __builtin_amdgcn_readfirstlane(plan.v[bins + 1 + item0 + it]);
        if (it > 0) tile_done();   // every wave is done with the previous row tile's stages
        const int R0 = tile * R64_BQ;
        // this lane's two query rows (columns of the two MFMA blocks)
        int row[2], t[2], g[2], qpos[2];
        bool rvalid[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            row[nb] = R0 + 64 * w + 32 * nb + ql;
            rvalid[nb] = row[nb] < RT;
            t[nb] = rvalid[nb] ? row[nb] / G : 0;
            g[nb] = rvalid[nb] ? row[nb] - t[nb] * G : 0;
            qpos[nb] = rvalid[nb] ? pos0 + t[nb] : -1;
        }
        const int wfirst = R0 + 64 * w;
        const int wlast = min(wfirst + 63, RT - 1);
        const int wqmax = __builtin_amdgcn_readfirstlane(wlast >= wfirst ? pos0 + wlast / G : -1);
        const int wqmin = __builtin_amdgcn_readfirstlane(pos0 + wfirst / G);
        const int blast = min(R0 + R64_BQ - 1, RT - 1);
        const int kv_end = __builtin_amdgcn_readfirstlane(pos0 + blast / G + 1);
        // this item's tiles [j_lo, j_lo + n_tiles): all, or split s's share
        const int n_all = (kv_end + R64_BK - 1) / R64_BK;
        const int s_idx = SPLIT ? (int)blockIdx.z : 0;
        const int j_lo = SPLIT ? __builtin_amdgcn_readfirstlane(n_all * s_idx / sp.n) : 0;
        const int n_tiles =
            SPLIT ? __builtin_amdgcn_readfirstlane(n_all * (s_idx + 1) / sp.n) - j_lo : n_all;
        if constexpr (SPLIT) {
            if (n_tiles == 0) {   // an empty split: the empty partial (uniform exit)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    if (!rvalid[nb]) continue;
                    const size_t part = ((size_t)t[nb] * n_q_heads + h * G + g[nb]) * sp.n + s_idx;
                    float* acc = sp.pacc + part * PF_HD + 4 * hh;
#pragma unroll
                    for (int i = 0; i < 32; ++i) *(f32x4*)(acc + 8 * i) = (f32x4)(0.f);
                    if (hh == 0) {
                        sp.pm[part] = -1e30f;
                        sp.pd[part] = 0.f;
                    }
                }
                continue;
            }
        }


#pragma unroll
        for (int d = 0; d < R64_DIST; ++d)
            if (d < n_tiles)
                r64_issue(lds_base + d * R64_STAGE, kb, vb, rsb, (j_lo + d) * R64_BK, kv_end, w,
                          lane, loff);

        f16x8 qreg[2][16];   // Q[row nb][128 hh + 8 ks + 0..7]
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const f16* qrow = q + ((size_t)t[nb] * n_q_heads + h * G + g[nb]) * q_pitch + 128 * hh;
#pragma unroll
            for (int ks = 0; ks < 16; ++ks)
                qreg[nb][ks] = rvalid[nb] ? *(const f16x8*)(qrow + 8 * ks) : (f16x8)(0);
        }
        WAIT_VMCNT(0);   // Q and the first tiles: the wait left to the compiler lands in the loop

        f32x16 o[2][8];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int mb = 0; mb < 8; ++mb) acc_zero(o[nb][mb], (f16x8)(0));
        float m_run[2] = {-1e30f, -1e30f}, l_run[2] = {0.f, 0.f};

        typedef __attribute__((address_space(3))) const f16x8 lds_f16x8;
        typedef __attribute__((address_space(3))) const char lds_char;
        int st = 0;   // stage of tile j
        for (int j = 0; j < n_tiles; ++j) {
            // tile j landed: the copies of the min(DIST - 1, n_tiles - 1 - j)
            // tiles issued after it may still be in flight
            const int ahead = min(R64_DIST - 1, n_tiles - 1 - j);
            if (ahead >= 3) WAIT_VMCNT(3 * R64_COPIES);
            else if (ahead == 2) WAIT_VMCNT(2 * R64_COPIES);
            else if (ahead == 1) WAIT_VMCNT(R64_COPIES);
            else WAIT_VMCNT(0);
            tile_done();   // every wave is past tile j - 1: its stage can be refilled
            if (j + R64_DIST < n_tiles) {
                const int sn = st == 0 ? R64_NST - 1 : st - 1;   // (j + DIST) % NST == (j - 1) % NST
                r64_issue(lds_base + sn * R64_STAGE, kb, vb, rsb, (j_lo + j + R64_DIST) * R64_BK,
                          kv_end, w, lane, loff);
            }
            const int kv0 = (j_lo + j) * R64_BK;
            if (kv0 <= wqmax) {
                const uint32_t kst = koff + st * R64_STAGE;
                f32x16 s[2] = {(f32x16)(0.f), (f32x16)(0.f)};
                constexpr int KPF = R64_KPF;
                f16x8 ka[KPF];
#pragma unroll
                for (int ks = 0; ks < KPF; ++ks) ka[ks] = *(lds_f16x8*)((lds_char*)smem + (kst ^ (16 * ks)));
#pragma unroll
                for (int ks = 0; ks < 16; ++ks) {
                    const f16x8 a = ka[ks % KPF];
                    if (ks + KPF < 16)
                        ka[ks % KPF] = *(lds_f16x8*)((lds_char*)smem + (kst ^ (16 * (ks + KPF))));
                    s[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qreg[0][ks], s[0], 0, 0, 0);
                    s[1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qreg[1][ks], s[1], 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead
                }
                const bool diag = kv0 + R64_BK - 1 > wqmin;   // wave-uniform
                f16x8 pk[2][2];
                r64_softmax(s[0], diag, qpos[0] - kv0 - 4 * hh, sl2, m_run[0], l_run[0], o[0], pk[0]);
                r64_softmax(s[1], diag, qpos[1] - kv0 - 4 * hh, sl2, m_run[1], l_run[1], o[1], pk[1]);
                // O^T += V^T P^T: 4 steps (kq, dim half) of 4 fragments x 2 blocks,
                // the next step's fragments read under this step's MFMAs
                const char* vt = smem + st * R64_STAGE + R64_TILE;
                s16x4 vf[2][8];
                r64_vfrags(vf[0], vt, troff, 0);
#pragma unroll
                for (int n = 0; n < 4; ++n) {
                    if (n + 1 < 4) r64_vfrags(vf[(n + 1) & 1], vt, troff, n + 1);
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const f16x4 lf = __builtin_bit_cast(f16x4, vf[n & 1][2 * u]);
                        const f16x4 hf = __builtin_bit_cast(f16x4, vf[n & 1][2 * u + 1]);
                        const f16x8 av = {lf[0], lf[1], lf[2], lf[3], hf[0], hf[1], hf[2], hf[3]};
                        acc_mfma(o[0][4 * (n & 1) + u], av, pk[0][n >> 1]);
                        acc_mfma(o[1][4 * (n & 1) + u], av, pk[1][n >> 1]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            st = st == R64_NST - 1 ? 0 : st + 1;
        }

        acc_settle(o[0]);
        acc_settle(o[1]);
        if constexpr (SPLIT) {
            // dims 32 mb + 8 r4 + 4 hh + 0..3 of O, unnormalised; m in natural-log units
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                if (!rvalid[nb]) continue;
                const size_t part = ((size_t)t[nb] * n_q_heads + h * G + g[nb]) * sp.n + s_idx;
                float* acc = sp.pacc + part * PF_HD + 4 * hh;
#pragma unroll
                for (int mb = 0; mb < 8; ++mb)
#pragma unroll
                    for (int r4 = 0; r4 < 4; ++r4)
                        *(f32x4*)(acc + 32 * mb + 8 * r4) =
                            (f32x4){o[nb][mb][4 * r4], o[nb][mb][4 * r4 + 1], o[nb][mb][4 * r4 + 2],
                                    o[nb][mb][4 * r4 + 3]};
                if (hh == 0) {
                    sp.pm[part] = l_run[nb] > 0.f ? m_run[nb] * FL_LN2 : -1e30f;
                    sp.pd[part] = l_run[nb];
                }
            }
            continue;
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            if (!rvalid[nb]) continue;
            const float inv = 1.f / l_run[nb];
            f16* zrow = z + ((size_t)t[nb] * n_q_heads + h * G + g[nb]) * z_pitch + 4 * hh;
#pragma unroll
            for (int mb = 0; mb < 8; ++mb)
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4)
                    *(f16x4*)(zrow + 32 * mb + 8 * r4) = (f16x4){
                        f16_sat(o[nb][mb][4 * r4] * inv), f16_sat(o[nb][mb][4 * r4 + 1] * inv),
                        f16_sat(o[nb][mb][4 * r4 + 2] * inv), f16_sat(o[nb][mb][4 * r4 + 3] * inv)};
        }
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Dynamic LDS above the default limit, raised once per device for each
// prefill kernel, and the device's CU count (a mutex: callers may come from
// several threads).
std::mutex g_lds_mu;
constexpr int PF_MAX_DEVICES = 64;
bool g_lds_done[PF_MAX_DEVICES];
int g_cus[PF_MAX_DEVICES];

int prefill_device_setup(int& n_cu) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= PF_MAX_DEVICES) {
        fl::set_error("attn_prefill: no current device below index %d", PF_MAX_DEVICES);
        return FL_ELAUNCH;
    }
    std::lock_guard<std::mutex> lock(g_lds_mu);
    if (g_lds_done[dev]) {
        n_cu = g_cus[dev];
        return FL_OK;
    }
    const void* fns[] = {(const void*)attn_prefill_kernel<false, false>,
                         (const void*)attn_prefill_kernel<false, true>,
                         (const void*)attn_prefill_kernel<true, false>,
                         (const void*)attn_prefill_kernel<true, true>};
    for (const void* f : fns)
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, LDS_B) !=
            hipSuccess) {
            fl::set_error("attn_prefill: cannot raise the dynamic LDS limit to %d bytes", LDS_B);
            return FL_ELAUNCH;
        }
    const void* fns64[] = {(const void*)attn_prefill_r64_kernel<false>,
                           (const void*)attn_prefill_r64_kernel<true>};
    for (const void* f : fns64)
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, R64_LDS) !=
            hipSuccess) {
            fl::set_error("attn_prefill: cannot raise the dynamic LDS limit to %d bytes", R64_LDS);
            return FL_ELAUNCH;
        }
    if (hipDeviceGetAttribute(&g_cus[dev], hipDeviceAttributeMultiprocessorCount, dev) !=
        hipSuccess) {
        fl::set_error("attn_prefill: cannot read the CU count of device %d", dev);
        return FL_ELAUNCH;
    }
    g_lds_done[dev] = true;
    n_cu = g_cus[dev];
    return FL_OK;
}

// The persistent plan of the r64 kernel for T rows from pos0 (G query heads a
// kv head) on n_cu CUs: bins = n_cu / n_kv bins a kv head (a kv head's row
// tiles on 8 / n_kv XCDs). A row tile's weight is the kv tiles it walks +
// R64_ITEM_COST; the heaviest go first, each to the lightest bin; then, for
// each pair of bins, the single move or swap that best closes their gap, and
// last single moves and swaps off the heaviest bin while they lower its
// load. Returns the
// entries used (bins + 1 + row tiles), 0 where the grid of row tiles x kv
// heads is launched instead: a kv-head count that does not divide the 8 XCDs,
// no more row tiles than bins, or a plan over R64_PLAN_MAX entries.
int r64_build_plan(int T, int pos0, int G, int n_kv, int n_cu, R64Plan& plan) {
    if (T < 1 || pos0 < 0 || G < 1 || n_kv < 1 || 8 % n_kv != 0 || n_cu < 8 || n_cu % 8 != 0)
        return 0;
    const int RT = T * G;
    const int N = (RT + R64_BQ - 1) / R64_BQ;
    const int bins = n_cu / n_kv;
    if (N <= bins || bins + 1 + N > R64_PLAN_MAX) return 0;
    std::vector<int> wt(N);
    for (int t = 0; t < N; ++t) {
        const int kv_end = pos0 + std::min(t * R64_BQ + R64_BQ - 1, RT - 1) / G + 1;
        wt[t] = (kv_end + R64_BK - 1) / R64_BK + R64_ITEM_COST;
    }
    std::vector<int> order(N);
    for (int t = 0; t < N; ++t) order[t] = N - 1 - t;   // weights grow with t
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return wt[a] > wt[b]; });
    std::vector<std::vector<int>> bin(bins);
    std::vector<long long> load(bins, 0);
    for (int t : order) {
        int lo = 0;
        for (int b = 1; b < bins; ++b)
            if (load[b] < load[lo]) lo = b;
        bin[lo].push_back(t);
        load[lo] += wt[t];
    }
    auto move = [&](int a, int xa, int b, int yb) {   // bin[a][xa] to b, bin[b][yb] (if >= 0) to a
        const int tx = bin[a][xa];
        bin[a].erase(bin[a].begin() + xa);
        load[a] -= wt[tx];
        if (yb >= 0) {
            const int ty = bin[b][yb];
            bin[b].erase(bin[b].begin() + yb);
            load[b] -= wt[ty];
            bin[a].push_back(ty);
            load[a] += wt[ty];
        }
        bin[b].push_back(tx);
        load[b] += wt[tx];
    };
    long long total = 0;
    int wmax = 0;
    for (int t = 0; t < N; ++t) total += wt[t], wmax = std::max(wmax, wt[t]);
    const long long bound = std::max<long long>((total + bins - 1) / bins, wmax);
    // pairs of a bin above and one below the mean (unless within 0.2 % of the
    // bound already): the move or swap that best closes their gap
    for (int round = 0; round < 16 && *std::max_element(load.begin(), load.end()) > bound + bound / 500;
         ++round) {
        bool changed = false;
        for (int a = 0; a < bins; ++a)
            for (int b = 0; b < bins; ++b) {
                const long long gap = load[a] - load[b];
                if (gap <= 0 || load[a] * bins < total || load[b] * bins > total) continue;
                long long best = gap;
                int bx = -1, by = -1;
                for (int x = 0; x < (int)bin[a].size(); ++x) {
                    const int wx = wt[bin[a][x]];
                    if (std::llabs(gap - 2 * wx) < best) best = std::llabs(gap - 2 * wx), bx = x, by = -1;
                    for (int y = 0; y < (int)bin[b].size(); ++y) {
                        const int d = wx - wt[bin[b][y]];
                        if (d > 0 && std::llabs(gap - 2 * d) < best)
                            best = std::llabs(gap - 2 * d), bx = x, by = y;
                    }
                }
                if (bx >= 0) move(a, bx, b, by), changed = true;
            }
        if (!changed) break;
    }
    // then single moves and swaps off the heaviest bin, to the same 0.2 %
    for (int iter = 0; iter < 4 * N; ++iter) {
        int hi = 0;
        for (int b = 1; b < bins; ++b)
            if (load[b] > load[hi]) hi = b;
        if (load[hi] <= bound + bound / 500) break;
        long long best = load[hi];
        int bx = -1, by = -1, blo = -1;   // move bin[hi][bx] to blo (by < 0) or swap it with bin[blo][by]
        for (int lo = 0; lo < bins; ++lo) {
            if (lo == hi) continue;
            for (int x = 0; x < (int)bin[hi].size(); ++x) {
                const int wx = wt[bin[hi][x]];
                const long long mv = std::max(load[hi] - wx, load[lo] + wx);
                if (mv < best) best = mv, bx = x, by = -1, blo = lo;
                for (int y = 0; y < (int)bin[lo].size(); ++y) {
                    const int d = wx - wt[bin[lo][y]];
                    if (d <= 0) continue;
                    const long long sv = std::max(load[hi] - d, load[lo] + d);
                    if (sv < best) best = sv, bx = x, by = y, blo = lo;
                }
            }
        }
        if (bx < 0) break;
        move(hi, bx, blo, by);
    }
    int k = bins + 1;
    for (int b = 0; b < bins; ++b) {
        std::stable_sort(bin[b].begin(), bin[b].end(), [&](int a, int c) { return wt[a] > wt[c]; });
        plan.v[b] = (uint16_t)(k - bins - 1);
        for (int t : bin[b]) plan.v[k++] = (uint16_t)t;
    }
    plan.v[bins] = (uint16_t)(k - bins - 1);
    return k;
}

// r64_build_plan, kept for the last few shapes (a serving loop repeats its
// chunk shapes); copied out under the lock.
struct R64PlanEntry {
    int T, pos0, G, n_kv, n_cu, used;
    R64Plan plan;
};
constexpr int R64_PLAN_CACHE = 8;
std::mutex g_plan_mu;
R64PlanEntry g_plan_cache[R64_PLAN_CACHE];
int g_plan_fill, g_plan_next;

int r64_plan(int T, int pos0, int G, int n_kv, int n_cu, R64Plan& plan) {
    {
        std::lock_guard<std::mutex> lock(g_plan_mu);
        for (int i = 0; i < g_plan_fill; ++i) {
            const R64PlanEntry& e = g_plan_cache[i];
            if (e.T == T && e.pos0 == pos0 && e.G == G && e.n_kv == n_kv && e.n_cu == n_cu) {
                plan = e.plan;
                return e.used;
            }
        }
    }
    const int used = r64_build_plan(T, pos0, G, n_kv, n_cu, plan);
    std::lock_guard<std::mutex> lock(g_plan_mu);
    R64PlanEntry& e = g_plan_cache[g_plan_next];
    e = {T, pos0, G, n_kv, n_cu, used, plan};
    g_plan_next = (g_plan_next + 1) % R64_PLAN_CACHE;
    g_plan_fill = std::min(g_plan_fill + 1, R64_PLAN_CACHE);
    return used;
}

// The 64-rows-a-wave kernel takes a call once there are enough 256-row
// workgroups to fill the chip twice over.
bool use_r64(int T, int n_q_heads, int n_kv_heads) {
    const int rows = T * (n_q_heads / n_kv_heads);
    return (rows + R64_BQ - 1) / R64_BQ * n_kv_heads >= R64_MIN_WGS;
}

constexpr int PF_SPLIT_MAX = 16;
constexpr int PF_CUS = 256;         // MI355X: 256 CUs, one 128 KiB-LDS workgroup each
constexpr int PF_SPLIT_OVH = 2;     // a split's fixed cost in tile units: prologue, partials, merge
// The 64-rows-a-wave kernel takes a KV split (fp16 caches) from this many
// 256-row workgroups a split and a causal range of this many rows (a chunk
// deep in a prompt); a split's fixed cost there, in its 32-row tiles.
// Same-box A/B at T = 1024, the 128-row kernel's split against it: pos0 0
// 49 against 82 us, 1024 116 / 121, 3072 and 8000 equal, 30000 836 / 776,
// 98000 2716 / 2264.
constexpr int R64_SPLIT_MIN_WGS = 64;
constexpr int R64_SPLIT_MIN_ROWS = 16384;
constexpr int R64_SPLIT_OVH = 4;

bool use_r64_split(int T, int pos0, int n_q_heads, int n_kv_heads) {
    const int rows = T * (n_q_heads / n_kv_heads);
    return (rows + R64_BQ - 1) / R64_BQ * n_kv_heads >= R64_SPLIT_MIN_WGS &&
           (long long)pos0 + T >= R64_SPLIT_MIN_ROWS;
}

// The count S minimising (rounds of one workgroup a CU) x (tiles a split
// walks + a split's fixed cost), S <= PF_SPLIT_MAX.
int best_split(int wgs, int nkt, int ovh) {
    int best = 1;
    long long best_cost = -1;
    for (int S = 1; S <= PF_SPLIT_MAX && S <= nkt; ++S) {
        const long long rounds = ((long long)wgs * S + PF_CUS - 1) / PF_CUS;
        const long long cost = rounds * ((nkt + S - 1) / S + ovh);
        if (best_cost < 0 || cost < best_cost) {
            best_cost = cost;
            best = S;
        }
    }
    return best;
}

// The KV split of a prefill call whose 128-row workgroups are too few to
// fill the CUs (a short chunk deep into a long prompt, runtime.py:196 /
// 2932-2941), by best_split over the kernel that runs: fp16 caches with at least
// R64_SPLIT_MIN_WGS 256-row workgroups and R64_SPLIT_MIN_ROWS rows take the
// 64-rows-a-wave kernel's split (a 1024-token chunk at 24 / 4 heads from
// pos0 15360: 96 workgroups a split), the rest the 128-row kernel's. 1 where the unsplit 64-rows-a-wave kernel runs or the
// 128-row grid already fills the chip.
int split_policy(int T, int pos0, int n_q_heads, int n_kv_heads, bool q8 = false) {
    if (T < 1 || pos0 < 0 || n_kv_heads < 1 || n_q_heads % n_kv_heads != 0) return 1;
    if (use_r64(T, n_q_heads, n_kv_heads)) return 1;
    const int G = n_q_heads / n_kv_heads;
    const int wgs = n_kv_heads * ((T * G + PF_BQ - 1) / PF_BQ);
    if (wgs >= PF_CUS) return 1;   // e.g. a fresh 2k prompt: 384 workgroups, unsplit
    if (!q8 && use_r64_split(T, pos0, n_q_heads, n_kv_heads)) {
        const int wgs64 = n_kv_heads * ((T * G + R64_BQ - 1) / R64_BQ);
        return best_split(wgs64, (pos0 + T + R64_BK - 1) / R64_BK, R64_SPLIT_OVH);
    }
    return best_split(wgs, (pos0 + T + PF_BK - 1) / PF_BK, PF_SPLIT_OVH);
}

// The int8 cache's rows [0, rows) as fp16(byte * scale), the values the int8
// kernel builds in LDS, into a staging copy [rows][n_kv][256] of K then V:
// thread i converts 16-byte chunk i of a K row and of a V row (16 values of
// one 32-value scale block) into two 16-byte stores each. HBM-bound; the
// long prefill then runs the 64-rows-a-wave kernel on the copy.
__global__ void __launch_bounds__(256)
q8_stage_kernel(const uint4* __restrict__ kc, const uint4* __restrict__ vc,
                const f16* __restrict__ ksc, const f16* __restrict__ vsc, f16x8* __restrict__ ko,
                f16x8* __restrict__ vo, int n_chunks) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_chunks) return;
    const uint4 kb = kc[i], vb = vc[i];
    const f16 ks = ksc[i >> 1], vs = vsc[i >> 1];   // 16 chunks, 8 scales a row of 256
    ko[2 * i] = deq8(kb.x, kb.y, ks);
    ko[2 * i + 1] = deq8(kb.z, kb.w, ks);
    vo[2 * i] = deq8(vb.x, vb.y, vs);
    vo[2 * i + 1] = deq8(vb.z, vb.w, vs);
}

// Bytes of that staging copy for a long prefill over an int8 cache (the rows
// [0, pos0 + T) every query reads, fp16 K and V), 0 where the 64-rows-a-wave
// kernel does not run (short prompts, the KV-split chunk).
size_t q8_stage_bytes(int T, int pos0, int n_q_heads, int n_kv_heads, int head_dim) {
    if (T < 1 || pos0 < 0 || n_kv_heads < 1 || n_q_heads < 1 || n_q_heads % n_kv_heads != 0 ||
        head_dim != PF_HD)
        return 0;
    if (split_policy(T, pos0, n_q_heads, n_kv_heads) != 1 || !use_r64(T, n_q_heads, n_kv_heads))
        return 0;
    return 2 * (size_t)(pos0 + T) * n_kv_heads * head_dim * sizeof(f16);
}

size_t split_work_bytes(int T, int n_q_heads, int head_dim, int split) {
    return (size_t)T * n_q_heads * split * ((size_t)head_dim * 4 + 8);
}

// gated: z *= sigmoid(gate) after the attention (attn_gate), the gate being
// the second half of each head's q row (q | gate rows, q_pitch >= 2 head_dim):
// applied by the merge when the KV is split, else by fl_attn_gate after it.
template <bool Q8>
int prefill(const void* q, int q_pitch, const void* k_new, const void* v_new, void* kcache,
            void* vcache, int layer, int n_q_heads, int n_kv_heads, int head_dim, int pos0,
            int max_pos, float scale, int T, void* z, int z_pitch, int split, void* work,
            size_t work_bytes, fl_stream_t stream, bool gated = false) {
    FL_REQUIRE(q && kcache && vcache && z, "null pointer");
    FL_REQUIRE(!gated || q_pitch >= 2 * head_dim, "gated: q_pitch >= 2 head_dim (q | gate rows)");
    const void* gate = gated ? q : nullptr;
    auto gate_after = [&](int rc_) {
        if (rc_ || !gated) return rc_;
        return fl_attn_gate(z, q, n_q_heads, head_dim, z_pitch, q_pitch, head_dim, T, stream);
    };
    FL_REQUIRE(head_dim == PF_HD, "head_dim must be 256");
    FL_REQUIRE(n_kv_heads > 0 && n_q_heads > 0 && n_q_heads % n_kv_heads == 0,
               "n_q_heads % n_kv_heads");
    FL_REQUIRE(T >= 1 && pos0 >= 0 && layer >= 0 && pos0 + T <= max_pos, "pos0 + T <= max_pos");
    FL_REQUIRE(!Q8 || layer == 0, "an int8 cache is one buffer a layer: layer must be 0");
    FL_REQUIRE(q_pitch >= head_dim && q_pitch % 8 == 0 && z_pitch >= head_dim && z_pitch % 4 == 0,
               "q_pitch, z_pitch");
    FL_REQUIRE((k_new == nullptr) == (v_new == nullptr), "k_new and v_new together");
    FL_REQUIRE(aligned16(q) && aligned16(kcache) && aligned16(vcache) && ((uintptr_t)z & 7u) == 0,
               "aligned buffers");
    FL_REQUIRE(split >= 1 && split <= 1024, "1 <= split <= 1024");
    if (split > 1) {
        FL_REQUIRE(work != nullptr && aligned16(work), "16-byte aligned work for a split");
        if (work_bytes < split_work_bytes(T, n_q_heads, head_dim, split)) {
            fl::set_error("work: %zu bytes, fl_attention_prefill_work_bytes asks %zu", work_bytes,
                          split_work_bytes(T, n_q_heads, head_dim, split));
            return FL_ESCRATCH;
        }
    }
    if (k_new != nullptr) {
        const int rc = Q8 ? fl_kv_store_q8(k_new, v_new, kcache, vcache, layer, pos0, T,
                                           n_kv_heads, head_dim, max_pos, stream)
                          : fl_kv_store(k_new, v_new, kcache, vcache, layer, pos0, T, n_kv_heads,
                                        head_dim, max_pos, stream);
        if (rc) return rc;
    }
    int n_cu = 0;
    int rc = prefill_device_setup(n_cu);
    if (rc) return rc;
    const void* kc;
    const void* vc;
    const f16* ksc = nullptr;
    const f16* vsc = nullptr;
    if (Q8) {
        const size_t vals = (size_t)max_pos * n_kv_heads * head_dim;   // scales follow
        kc = kcache;
        vc = vcache;
        ksc = (const f16*)((const char*)kcache + vals);
        vsc = (const f16*)((const char*)vcache + vals);
    } else {
        const size_t off = (size_t)layer * max_pos * n_kv_heads * head_dim;
        kc = (const f16*)kcache + off;
        vc = (const f16*)vcache + off;
    }
    const int rows = T * (n_q_heads / n_kv_heads);
    const int r64_tiles = (rows + R64_BQ - 1) / R64_BQ;
    // over an int8 cache with room in `work` for the fp16 staging copy: stage,
    // then the fp16 path below on the copy
    const size_t stage = Q8 && split == 1 ? q8_stage_bytes(T, pos0, n_q_heads, n_kv_heads, head_dim)
                                          : 0;
    const bool staged = stage > 0 && work != nullptr && aligned16(work) && work_bytes >= stage;
    if (staged) {
        const size_t cache_rows = (size_t)(pos0 + T) * n_kv_heads;
        const int n_chunks = (int)(cache_rows * (PF_HD / 16));
        f16* ko = (f16*)work;
        f16* vo = ko + cache_rows * PF_HD;
        hipLaunchKernelGGL(q8_stage_kernel, dim3((n_chunks + 255) / 256), dim3(256), 0,
                           (hipStream_t)stream, (const uint4*)kc, (const uint4*)vc, ksc, vsc,
                           (f16x8*)ko, (f16x8*)vo, n_chunks);
        rc = fl::check_launch("attn_prefill q8 staging");
        if (rc) return rc;
        kc = ko;
        vc = vo;
    }
    if ((!Q8 || staged) && split == 1 && use_r64(T, n_q_heads, n_kv_heads)) {
        R64Plan plan;
        const int G = n_q_heads / n_kv_heads;
        const int bins = r64_plan(T, pos0, G, n_kv_heads, n_cu, plan) > 0 ? n_cu / n_kv_heads : 0;
        const dim3 grid = bins > 0 ? dim3(n_cu) : dim3(r64_tiles, n_kv_heads);
        hipLaunchKernelGGL(attn_prefill_r64_kernel<false>, grid, dim3(PF_THREADS), R64_LDS,
                           (hipStream_t)stream, (const f16*)q, q_pitch, (const f16*)kc,
                           (const f16*)vc, (f16*)z, z_pitch, n_q_heads, n_kv_heads, pos0, T,
                           scale * FL_LOG2E, r64_tiles, bins, plan,
                           PfSplit{nullptr, nullptr, nullptr, 1});
        return gate_after(fl::check_launch("attn_prefill_r64"));
    }
    if (!Q8 && split > 1 && use_r64_split(T, pos0, n_q_heads, n_kv_heads)) {
        const size_t parts = (size_t)T * n_q_heads * split;
        PfSplit sp = {(float*)work, nullptr, nullptr, split};
        sp.pm = sp.pacc + parts * PF_HD;
        sp.pd = sp.pm + parts;
        R64Plan plan;
        plan.v[0] = 0;
        hipLaunchKernelGGL(attn_prefill_r64_kernel<true>, dim3(r64_tiles, n_kv_heads, split),
                           dim3(PF_THREADS), R64_LDS, (hipStream_t)stream, (const f16*)q, q_pitch,
                           (const f16*)kc, (const f16*)vc, (f16*)z, z_pitch, n_q_heads,
                           n_kv_heads, pos0, T, scale * FL_LOG2E, r64_tiles, 0, plan, sp);
        rc = fl::check_launch("attn_prefill_r64 (kv split)");
        if (rc) return rc;
        return fl_attention_merge(sp.pacc, sp.pm, sp.pd, z, n_q_heads, head_dim, z_pitch, T,
                                  split, gate, q_pitch, head_dim, stream);
    }
    const int n_row_tiles = (rows + PF_BQ - 1) / PF_BQ;
    if (split == 1) {
        hipLaunchKernelGGL((attn_prefill_kernel<Q8, false>), dim3(n_row_tiles, n_kv_heads),
                           dim3(PF_THREADS), LDS_B, (hipStream_t)stream, (const f16*)q, q_pitch,
                           kc, vc, ksc, vsc, (f16*)z, z_pitch, n_q_heads, n_kv_heads, pos0, T,
                           scale * FL_LOG2E, n_row_tiles, PfSplit{nullptr, nullptr, nullptr, 1});
        return gate_after(fl::check_launch("attn_prefill"));
    }
    const size_t parts = (size_t)T * n_q_heads * split;
    PfSplit sp = {(float*)work, nullptr, nullptr, split};
    sp.pm = sp.pacc + parts * PF_HD;
    sp.pd = sp.pm + parts;
    hipLaunchKernelGGL((attn_prefill_kernel<Q8, true>), dim3(n_row_tiles, n_kv_heads, split),
                       dim3(PF_THREADS), LDS_B, (hipStream_t)stream, (const f16*)q, q_pitch, kc,
                       vc, ksc, vsc, (f16*)z, z_pitch, n_q_heads, n_kv_heads, pos0, T,
                       scale * FL_LOG2E, n_row_tiles, sp);
    rc = fl::check_launch("attn_prefill (kv split)");
    if (rc) return rc;
    return fl_attention_merge(sp.pacc, sp.pm, sp.pd, z, n_q_heads, head_dim, z_pitch, T, split,
                              gate, q_pitch, head_dim, stream);
}

}  // namespace

extern "C" int fl_attention_prefill(const void* q, int q_pitch, const void* k_new,
                                    const void* v_new, void* kcache, void* vcache, int layer,
                                    int n_q_heads, int n_kv_heads, int head_dim, int pos0,
                                    int max_pos, float scale, int T, void* z, int z_pitch,
                                    fl_stream_t stream) {
    return prefill<false>(q, q_pitch, k_new, v_new, kcache, vcache, layer, n_q_heads, n_kv_heads,
                          head_dim, pos0, max_pos, scale, T, z, z_pitch, 1, nullptr, 0, stream);
}

extern "C" int fl_attention_prefill_q8(const void* q, int q_pitch, const void* k_new,
                                       const void* v_new, void* kcache, void* vcache, int layer,
                                       int n_q_heads, int n_kv_heads, int head_dim, int pos0,
                                       int max_pos, float scale, int T, void* z, int z_pitch,
                                       fl_stream_t stream) {
    return prefill<true>(q, q_pitch, k_new, v_new, kcache, vcache, layer, n_q_heads, n_kv_heads,
                         head_dim, pos0, max_pos, scale, T, z, z_pitch, 1, nullptr, 0, stream);
}

extern "C" int fl_attention_prefill_plan(int T, int pos0, int n_q_heads, int n_kv_heads,
                                         int n_cu, unsigned short* out, int cap) {
    if (n_kv_heads < 1 || n_q_heads < 1 || n_q_heads % n_kv_heads != 0) return 0;
    if (split_policy(T, pos0, n_q_heads, n_kv_heads) != 1 ||
        !use_r64(T, n_q_heads, n_kv_heads))
        return 0;
    R64Plan plan;
    const int used = r64_build_plan(T, pos0, n_q_heads / n_kv_heads, n_kv_heads, n_cu, plan);
    if (out != nullptr)
        for (int i = 0; i < used && i < cap; ++i) out[i] = plan.v[i];
    return used;
}

extern "C" int fl_attention_prefill_split_count(int T, int pos0, int n_q_heads, int n_kv_heads) {
    return split_policy(T, pos0, n_q_heads, n_kv_heads);
}

extern "C" int fl_attention_prefill_split_count_q8(int T, int pos0, int n_q_heads,
                                                   int n_kv_heads) {
    return split_policy(T, pos0, n_q_heads, n_kv_heads, true);
}

extern "C" size_t fl_attention_prefill_q8_stage_bytes(int T, int pos0, int n_q_heads,
                                                     int n_kv_heads, int head_dim) {
    return q8_stage_bytes(T, pos0, n_q_heads, n_kv_heads, head_dim);
}

extern "C" size_t fl_attention_prefill_work_bytes(int T, int n_q_heads, int head_dim, int split) {
    if (T < 1 || n_q_heads < 1 || head_dim < 1 || split < 1) return 0;
    return split > 1 ? split_work_bytes(T, n_q_heads, head_dim, split) : 0;
}

extern "C" int fl_attention_prefill_kv(const void* q, int q_pitch, const void* k_new,
                                       const void* v_new, void* kcache, void* vcache, int layer,
                                       int n_q_heads, int n_kv_heads, int head_dim, int pos0,
                                       int max_pos, float scale, int T, int split, void* z,
                                       int z_pitch, void* work, size_t work_bytes,
                                       fl_stream_t stream) {
    if (split == 0) split = split_policy(T, pos0, n_q_heads, n_kv_heads);
    return prefill<false>(q, q_pitch, k_new, v_new, kcache, vcache, layer, n_q_heads, n_kv_heads,
                          head_dim, pos0, max_pos, scale, T, z, z_pitch, split, work, work_bytes,
                          stream);
}

extern "C" int fl_attention_prefill_gated(const void* q, int q_pitch, const void* k_new,
                                          const void* v_new, void* kcache, void* vcache,
                                          int layer, int q8, int n_q_heads, int n_kv_heads,
                                          int head_dim, int pos0, int max_pos, float scale, int T,
                                          int split, void* z, int z_pitch, void* work,
                                          size_t work_bytes, fl_stream_t stream) {
    if (split == 0) split = split_policy(T, pos0, n_q_heads, n_kv_heads, q8 != 0);
    if (q8)
        return prefill<true>(q, q_pitch, k_new, v_new, kcache, vcache, layer, n_q_heads,
                             n_kv_heads, head_dim, pos0, max_pos, scale, T, z, z_pitch, split, work,
                             work_bytes, stream, true);
    return prefill<false>(q, q_pitch, k_new, v_new, kcache, vcache, layer, n_q_heads, n_kv_heads,
                          head_dim, pos0, max_pos, scale, T, z, z_pitch, split, work, work_bytes,
                          stream, true);
}

extern "C" int fl_attention_prefill_kv_q8(const void* q, int q_pitch, const void* k_new,
                                          const void* v_new, void* kcache, void* vcache,
                                          int layer, int n_q_heads, int n_kv_heads, int head_dim,
                                          int pos0, int max_pos, float scale, int T, int split,
                                          void* z, int z_pitch, void* work, size_t work_bytes,
                                          fl_stream_t stream) {
    if (split == 0) split = split_policy(T, pos0, n_q_heads, n_kv_heads, true);
    return prefill<true>(q, q_pitch, k_new, v_new, kcache, vcache, layer, n_q_heads, n_kv_heads,
                         head_dim, pos0, max_pos, scale, T, z, z_pitch, split, work, work_bytes,
                         stream);
}
