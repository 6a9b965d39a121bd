// Full-attention decode / MTP-verify path for gfx950: the fp16 KV store, the
// split-K flash-decode partials on MFMA, and the merge with the fused sigmoid
// output gate.
//
// Reference behaviour restated (model/footless/cuda_sm60/kernels.cu):
//   kv_store              465-484   rows pos0+t of a [max_pos][n_kv][256] cache
//   attention_split_gqa   682-835   split partials (m, d, acc), per-token split
//   attention_merge       1387-1424 M = max m, z = sum e acc / sum e d, f16_sat
//   attn_gate             1572-1600 z = f16_sat(z * sigmoid(gate))
//   kv_store_q8           486-520   the int8 cache format (values, then fp16
//                                   scales of 32-dim blocks)
//   attention_split_gqa_q8 910-1047 the split partials over the int8 cache
//   attention_dec_q8      1049-1335 int8 decode partials, 64-row tiles split
//                                   by (tmin, smax), pm in log2 units
//   attention_dec_merge   1336-1385 their merge (+ the gate), exp2
//
// Decode kernel design (one workgroup = one (sequence, kv head, split)):
//   * The query rows of a kv head -- T tokens x G = 6 q heads, token-major,
//     padded to 32 -- are the N columns of a 32x32x16 f16 MFMA; the split's
//     KV rows stream through it in 32-row tiles as the M rows.
//   * The 4 wavefronts split the head dimension: wave w owns d in [64w, 64w+64).
//     For S^T = K Q^T each wave contracts its 64 dims (4 MFMAs) and the four
//     partial 32x32 score tiles are summed through LDS in a fixed order, so
//     every wave holds the identical full score tile; for O^T = V^T P^T each
//     wave produces its own 64 output dims (2 MFMA blocks), so there is no
//     cross-wave merge of O at the end.
//   * The S^T accumulator layout puts one query column in each lane pair
//     (lane l and l^32), so the online-softmax max / sum is a 16-value
//     in-lane reduction plus one lane exchange, and the probabilities P are
//     already the B operand of the PV MFMA (the KV order inside a 16-row
//     k-step is permuted to match; V is read with the same permutation).
//   * K goes straight from HBM into MFMA A-operand registers (a lane reads 64
//     contiguous bytes of its row); V is loaded with 128-byte row segments per
//     8 lanes and transposed into a per-wave LDS slice. The next tile's loads
//     are issued before the current tile's math.
//   * Over the int8 cache the same kernel runs on dequantized tiles: a lane
//     loads its K / V bytes (half the fp16 bytes) and one dword of scales,
//     and each value becomes fp16(byte * scale) in registers -- the
//     reference's prefill dequantizes V the same way (kernels.cu:2500-2509);
//     its decode keeps byte * scale in fp32, so scores and outputs differ
//     from it by fp16 rounding, far below the int8 format's own error. An
//     int8 row of a kv head is two 128-byte lines, so the int8 tiles split
//     the work otherwise: wave w takes 16 rows and 128 dims (S^T on 16x16x32
//     MFMAs, two partials a score summed through LDS) and reads whole lines;
//     its V^T lands in the owning waves' LDS slices (double-buffered). Grids
//     of at most one workgroup a CU copy the int8 tiles HBM -> LDS instead.
//   * Tiles are 32-row aligned in absolute position and every tile a token's
//     range does not cover is an exact no-op for that token (masked scores,
//     p = 0, corr = 1), so a token's partial is the same bits whichever other
//     tokens share the launch: a verify row equals the T = 1 call at its
//     position (the reference asserts this, runtime.py:2062-2069).
#include "fl_common.hpp"

#include <mutex>

#include <limits.h>
#include <type_traits>

namespace {

constexpr int DEC_TILE = 32;
constexpr int DEC_HD = 256;
constexpr int DEC_WAVES = 4;
constexpr int DEC_THREADS = 64 * DEC_WAVES;
constexpr int VT_PITCH = 40;   // halves per d row of the transposed V slice (32 + 8 pad)
// the int8 layout's pitch: its V^T writes (8 d rows 8 apart x 4 kv groups a
// store) spread over 32 banks at 18 dwords a row, 8 at 20
constexpr int VT_PITCH_Q8 = 36;
constexpr float RESCALE_LOG2 = 8.f;
#ifndef DEC_NBUF
#define DEC_NBUF 2                // register tile buffers (prefetch depth + 1)
#endif
#ifndef DEC_NT_V
#define DEC_NT_V true             // V rows streamed with non-temporal loads
#endif

struct DecSeqs {
    const f16* k[FL_MAX_SEQS];    // int8 caches: the values, as bytes
    const f16* v[FL_MAX_SEQS];
    const f16* ks[FL_MAX_SEQS];   // int8 caches: the scales (unused for fp16)
    const f16* vs[FL_MAX_SEQS];
    int pos0[FL_MAX_SEQS];
};

// Token range of split s for a token of length `seqlen`: St = clamp(seqlen /
// split_rows, 1, split) splits over its nt = ceil(seqlen / 32) tiles, split s
// taking tiles [nt s / St, nt (s+1) / St) (the reference's per-token rule,
// kernels.cu:535-544, on tile boundaries). Empty (lo == hi == 0) for s >= St.
// With floor_splits > 0 a token gets at least min(seqlen / 64, floor_splits)
// splits (still at most `split`): short contexts are cut into 64-row splits
// up to that floor, so they spread over more CUs; longer ones keep
// split_rows rows a split, so the partials stay a small part of the bytes.
// Either way St is a function of the token's own length.
constexpr int DEC_FINE_ROWS = 64;

__host__ __device__ __forceinline__ int split_count(int seqlen, int split_rows, int split,
                                                    int floor_splits) {
    int st = seqlen / split_rows;
    const int fine = seqlen / DEC_FINE_ROWS;
    const int lo = fine < floor_splits ? fine : floor_splits;
    st = st > lo ? st : lo;
    return st < 1 ? 1 : (st > split ? split : st);
}

__host__ __device__ __forceinline__ void split_range(int seqlen, int s, int split_rows, int split,
                                                     int floor_splits, int& lo, int& hi) {
    const int st = split_count(seqlen, split_rows, split, floor_splits);
    if (s >= st) {
        lo = 0;
        hi = 0;
        return;
    }
    // nt (s + 1) < 2^32 (split_math_fits): 32-bit unsigned products
    const unsigned nt = (unsigned)(seqlen + DEC_TILE - 1) / DEC_TILE;
    const int t0 = (int)(nt * (unsigned)s / (unsigned)st);
    const int t1 = (int)(nt * (unsigned)(s + 1) / (unsigned)st);
    lo = t0 * DEC_TILE;
    hi = t1 * DEC_TILE < seqlen ? t1 * DEC_TILE : seqlen;
}

// The int8 decode's rule (attention_dec_q8, kernels.cu:1107-1118): a token of
// length len has nkt = ceil(len / 64) tiles of 64 rows, St = min(smax,
// ceil(nkt / tmin)) splits, split s taking tiles [nkt s / St, nkt (s+1) / St).
// Splits s >= St are not written (the merge reads the first St).
__host__ __device__ __forceinline__ int dec_split_count(int len, int tmin, int smax) {
    const int nkt = (len + 63) / 64;
    const int st = (nkt + tmin - 1) / tmin;
    return st > smax ? smax : st;
}

__host__ __device__ __forceinline__ void dec_split_range(int len, int s, int tmin, int smax,
                                                         int& lo, int& hi) {
    const int st = dec_split_count(len, tmin, smax);
    if (s >= st) {
        lo = 0;
        hi = 0;
        return;
    }
    const unsigned nkt = (unsigned)(len + 63) / 64;   // nkt (s + 1) < 2^32
    lo = (int)(nkt * (unsigned)s / (unsigned)st) * 64;
    const int e = (int)(nkt * (unsigned)(s + 1) / (unsigned)st) * 64;
    hi = e < len ? e : len;
}

// ---------------------------------------------------------------------------
// kv_store: 16-byte copies, one lane per 8 halves of a (token, kv head) row.
// ---------------------------------------------------------------------------
__global__ void kv_store_kernel(const uint4* __restrict__ k, const uint4* __restrict__ v,
                                uint4* __restrict__ kc, uint4* __restrict__ vc, size_t layer_off,
                                int pos0, int T, int row_u4) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * row_u4) return;
    const int t = i / row_u4;
    const size_t dst = layer_off + (size_t)(pos0 + t) * row_u4 + (i - t * row_u4);
    kc[dst] = k[i];
    vc[dst] = v[i];
}

// kv_store_q8: a wavefront a (token, kv head) row, 4 elements a lane.
__global__ void __launch_bounds__(256)
kv_store_q8_kernel(const f16* __restrict__ k, const f16* __restrict__ v, signed char* __restrict__ kc,
                   signed char* __restrict__ vc, f16* __restrict__ ksc, f16* __restrict__ vsc,
                   int pos0, int T, int n_kv) {
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);   // wave-uniform
    if (row >= T * n_kv) return;
    const int lane = threadIdx.x & 63;
    const int t = row / n_kv, h = row - t * n_kv;
    const size_t src = (size_t)row * DEC_HD + 4 * lane;
    const size_t dst = (size_t)(pos0 + t) * n_kv + h;
    q8_store_row(*(const f16x4*)(k + src), kc + dst * DEC_HD, ksc + dst * 8, lane);
    q8_store_row(*(const f16x4*)(v + src), vc + dst * DEC_HD, vsc + dst * 8, lane);
}

// ---------------------------------------------------------------------------
// split partials
// ---------------------------------------------------------------------------
struct DecTileRegs {
    f16x8 k[4];   // K[row ql][64w + 32hh + 8ks + 0..7], ks = 0..3
    f16x8 v[4];   // V[row 4(l&7) + i][64w + 8(l>>3) + 0..7], i = 0..3
};

// int8 tiles use their own split of the work (the int8 layout): wave w
// takes kv rows 16 (w & 1) .. + 15 and dims 128 (w >> 1) .. + 127, so each
// wave reads whole 128-byte lines of its K and V rows (4 lanes a K row, 16
// lanes a V row), where the fp16 layout reads each line in two halves from
// two waves. In DecTileRegs, lane l = 16 g + i:
//   k[ks] = K[row 16 (w & 1) + i][128 (w >> 1) + 32 g + 8 ks + 0..7]
//   v[i'] = V[row 16 (w & 1) + 4 (l & 3) + i'][128 (w >> 1) + 8 (l >> 2) + 0..7]
// One int8 tile in flight: the same elements as bytes, plus one dword of
// scales a lane -- rows 16 (w & 1) + (l & 15), blocks 4 (w >> 1) + 2 ((l >>
// 4) & 1) + 0, 1; K for l < 32, V above.
struct DecTileQ8 {
    u32x4 k[2];
    u32x2 v[4];
    uint32_t sc;
};

template <bool NT_V>
__device__ __forceinline__ void dec_load_tile(DecTileQ8& r, const char* __restrict__ kbase,
                                              const char* __restrict__ vbase,
                                              const f16* __restrict__ ksb,
                                              const f16* __restrict__ vsb, size_t row_stride,
                                              int j, int uhi, int lane, int w) {
    const int hh = lane >> 5;
    const uint32_t rs = (uint32_t)row_stride;   // bytes between rows; caches < 2 GiB
    const int r0 = j * DEC_TILE + 16 * (w & 1), cb = 128 * (w >> 1);
    const uint32_t krow = (uint32_t)min(r0 + (lane & 15), uhi - 1);
    const u32x4* src = (const u32x4*)(kbase + (krow * rs + cb + 32 * ((lane >> 4) & 3)));
    r.k[0] = src[0];
    r.k[1] = src[1];
    const char* sb = (const char*)(hh ? vsb : ksb);
    r.sc = *(const uint32_t*)(sb + (krow * (rs / 16) + 2 * (4 * (w >> 1) + 2 * ((lane >> 4) & 1))));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t vrow = (uint32_t)min(r0 + 4 * (lane & 3) + i, uhi - 1);
        const u32x2* vsrc = (const u32x2*)(vbase + (vrow * rs + cb + 8 * (lane >> 2)));
        r.v[i] = NT_V ? __builtin_nontemporal_load(vsrc) : *vsrc;
    }
}

// The int8 tile as the fp16 tile the MFMAs read: fp16(byte * scale).
__device__ __forceinline__ DecTileRegs dec_dequant(const DecTileQ8& q, int lane) {
    DecTileRegs r;
    // K: row (l & 15), block 4 (w >> 1) + l / 16 -- lane (l & 15) + 16 (l / 32)'s
    // dword, half (l / 16) & 1; V row 4 (l & 3) + i, the same block -- lane 32 + that
    const int bh = (lane >> 4) & 1, bl = 16 * (lane >> 5);
    const uint32_t kp = (uint32_t)__builtin_amdgcn_ds_bpermute(((lane & 15) + bl) << 2, (int)q.sc);
    const f16 ksh = __builtin_bit_cast(f16x2, kp)[bh];
    const f16x2 ks2 = {ksh, ksh};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const u32x4 b = q.k[ks >> 1];
        const f16x4 lo = q8_deq4((ks & 1) ? b.z : b.x, ks2);
        const f16x4 hi = q8_deq4((ks & 1) ? b.w : b.y, ks2);
        r.k[ks] = (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t vp = (uint32_t)__builtin_amdgcn_ds_bpermute(
            (32 + bl + 4 * (lane & 3) + i) << 2, (int)q.sc);
        const f16 vsh = __builtin_bit_cast(f16x2, vp)[bh];
        const f16x2 vs2 = {vsh, vsh};
        const f16x4 lo = q8_deq4(q.v[i].x, vs2);
        const f16x4 hi = q8_deq4(q.v[i].y, vs2);
        r.v[i] = (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    return r;
}

// int8 tiles are copied HBM -> LDS (global_load_lds) into stages of
// Q8_STAGE_B bytes: K rows [32][256] at Q8_K_OFF, V rows at Q8_V_OFF, then
// one 1 KiB block of scales a wave at Q8_S_OFF + 1024 w -- the tile's 32 rows
// of K scales (16 bytes a row: the 8 blocks) and then its 32 rows of V scales
// (every wave copies them all, for its own reads). A row's 16-byte chunk c is stored at c ^ q8_sw(row): a copy
// instruction reads 4 whole rows (16 lanes a row, each 128-byte line from
// one instruction), and the fragment reads below hit distinct banks -- the K
// operand (one row a lane, 16 rows at one chunk) and the V slice (rows 4k + i,
// k = 0..7, at chunks c and c ^ 1, 8 bytes a lane).
constexpr int Q8_K_OFF = 0;
constexpr int Q8_V_OFF = DEC_TILE * DEC_HD;
constexpr int Q8_S_OFF = 2 * DEC_TILE * DEC_HD;
constexpr int Q8_STAGE_B = Q8_S_OFF + DEC_WAVES * 1024;   // 20 KiB
constexpr int Q8_COPIES = 5;   // copy instructions a wave a tile (2 K, 2 V, scales)

__device__ __forceinline__ int q8_sw(int r) {
    return (r & 1) | (((r >> 2) & 3) << 1) | ((((r >> 1) ^ (r >> 4)) & 1) << 3);
}

typedef __attribute__((address_space(3))) const char lds_cchar;

// Copy tile jt (rows past uhi clamped to uhi - 1) into the stage at LDS
// address sb: wave w copies rows 8w .. 8w + 7 of K and V and its own scales.
// copy_off[c]: this lane's offset in row 8w + 4c + lane / 16 (its swizzled
// chunk); sc: this lane's scale row 0 (K for lanes < 32, V above).
__device__ __forceinline__ void q8_issue(uint32_t sb, const char* kb, const char* vb,
                                         const char* sc, uint32_t rs, int jt, int uhi, int w,
                                         int lane, const uint32_t (&copy_off)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint32_t row = (uint32_t)min(jt * DEC_TILE + 8 * w + 4 * c + (lane >> 4), uhi - 1);
        const uint32_t lds = __builtin_amdgcn_readfirstlane(sb + (8 * w + 4 * c) * DEC_HD);
        copy16(kb, row * rs + copy_off[c], lds + Q8_K_OFF);
        copy16(vb, row * rs + copy_off[c], lds + Q8_V_OFF);
    }
    const uint32_t srow = (uint32_t)min(jt * DEC_TILE + (lane & 31), uhi - 1);
    copy16_v(sc + (size_t)srow * (rs / 16), __builtin_amdgcn_readfirstlane(sb + Q8_S_OFF + 1024 * w));
}

// The staged int8 tile as the fp16 tile the MFMAs read (DecTileRegs):
// fp16(byte * scale), each value once.
__device__ __forceinline__ DecTileRegs q8_stage_tile(lds_cchar* S, int lane, int w) {
    DecTileRegs r;
    typedef __attribute__((address_space(3))) const u32x4 lds_u32x4;
    typedef __attribute__((address_space(3))) const u32x2 lds_u32x2;
    typedef __attribute__((address_space(3))) const f16 lds_f16;
    // the int8 layout: K row 16 (w & 1) + (l & 15), chunks 8 (w >> 1) + 2 (l /
    // 16) + 0, 1; V rows 16 (w & 1) + 4 (l & 3) + i, chunk 8 (w >> 1) + l / 8,
    // half (l / 4) & 1; scales of block 4 (w >> 1) + l / 16
    const int kr = 16 * (w & 1) + (lane & 15), kc = 8 * (w >> 1) + 2 * (lane >> 4);
    lds_cchar* krow = S + Q8_K_OFF + kr * DEC_HD;
    const u32x4 k0 = *(lds_u32x4*)(krow + 16 * (kc ^ q8_sw(kr)));
    const u32x4 k1 = *(lds_u32x4*)(krow + 16 * ((kc + 1) ^ q8_sw(kr)));
    lds_cchar* scl = S + Q8_S_OFF + 1024 * w + 2 * (4 * (w >> 1) + (lane >> 4));
    const f16 ksh = *(lds_f16*)(scl + 16 * kr);
    const f16x2 ks2 = {ksh, ksh};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const u32x4 b = ks < 2 ? k0 : k1;
        const f16x4 lo = q8_deq4((ks & 1) ? b.z : b.x, ks2);
        const f16x4 hi = q8_deq4((ks & 1) ? b.w : b.y, ks2);
        r.k[ks] = (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    const int vr = 16 * (w & 1) + 4 * (lane & 3), vc = 8 * (w >> 1) + (lane >> 3),
              vhalf = 8 * ((lane >> 2) & 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x2 bv =
            *(lds_u32x2*)(S + Q8_V_OFF + (vr + i) * DEC_HD + 16 * (vc ^ q8_sw(vr + i)) + vhalf);
        const f16 vsh = *(lds_f16*)(scl + 16 * (32 + vr + i));
        const f16x2 vs2 = {vsh, vsh};
        const f16x4 lo = q8_deq4(bv.x, vs2);
        const f16x4 hi = q8_deq4(bv.y, vs2);
        r.v[i] = (f16x8){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
    return r;
}

template <bool NT_V>
__device__ __forceinline__ void dec_load_tile(DecTileRegs& r, const f16* __restrict__ kbase,
                                              const f16* __restrict__ vbase, size_t row_stride,
                                              int j, int uhi, int lane, int w) {
    const int ql = lane & 31, hh = lane >> 5;
    const uint32_t rs = (uint32_t)row_stride * 2;   // bytes between rows; caches < 2 GiB
    const char* kb = (const char*)kbase;
    const char* vb = (const char*)vbase;
    const uint32_t krow = (uint32_t)min(j * DEC_TILE + ql, uhi - 1);
    const f16x8* src = (const f16x8*)(kb + (krow * rs + 2 * (64 * w + 32 * hh)));
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) r.k[ks] = src[ks];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t vrow = (uint32_t)min(j * DEC_TILE + 4 * (lane & 7) + i, uhi - 1);
        const f16x8* vsrc = (const f16x8*)(vb + (vrow * rs + 2 * (64 * w + 8 * (lane >> 3))));
        r.v[i] = NT_V ? __builtin_nontemporal_load(vsrc) : *vsrc;
    }
}

// Workgroup barrier after this wave's LDS writes, without the vmcnt drain of
// __syncthreads(): the next tiles' loads stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Q8: the caches are int8 (DecSeqs k / v the values, ks / vs the scales).
// DEC: attention_dec_q8's split rule and partials -- (split, split_rows) are
// (smax, tmin), pm in log2 units, no partial written for s >= St; otherwise
// attention_split_gqa's -- pm in natural-log units, empty partials written.
template <int NBUF, bool NT_V, bool Q8, bool DEC, bool STAGE>
__global__ void __launch_bounds__(DEC_THREADS)
attn_decode_split_kernel(const f16* __restrict__ qg, DecSeqs seqs, float* __restrict__ pacc,
                         float* __restrict__ pm, float* __restrict__ pd, int n_q_heads,
                         int n_kv, int q_pitch, int T, int split, int split_rows,
                         int split_floor, float sl2) {
    // partial scores: 4 writers a row (fp16 layout: a wave's 64 dims) or 2
    // (int8 layout: a wave's 128 dims of 16 rows); V^T in the owner wave's
    // region, double-buffered in the int8 layout (written across waves)
    constexpr int SP_W = Q8 ? 2 : DEC_WAVES;
    constexpr int VTP = Q8 ? VT_PITCH_Q8 : VT_PITCH;
    __shared__ __attribute__((aligned(16))) f32x4 s_part[2][SP_W][4][64];
    __shared__ __attribute__((aligned(16))) f16 s_vt[Q8 ? 2 : 1][DEC_WAVES][64][VTP];
    __shared__ __attribute__((aligned(16))) char s_stage[STAGE ? NBUF * Q8_STAGE_B : 16];

    const int s = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int hh = lane >> 5, ql = lane & 31;
    const int G = n_q_heads / n_kv;
    const int R = T * G;
    const int pos0 = seqs.pos0[b];
    const size_t row_stride = (size_t)n_kv * DEC_HD;   // elements (bytes for int8)
    const f16* kbase = seqs.k[b] + (size_t)h * DEC_HD;
    const f16* vbase = seqs.v[b] + (size_t)h * DEC_HD;
    const char* kbase8 = (const char*)seqs.k[b] + (size_t)h * DEC_HD;
    const char* vbase8 = (const char*)seqs.v[b] + (size_t)h * DEC_HD;
    const f16* ksb = Q8 ? seqs.ks[b] + (size_t)h * 8 : nullptr;
    const f16* vsb = Q8 ? seqs.vs[b] + (size_t)h * 8 : nullptr;
    auto range = [&](int len, int& lo, int& hi) {
        if constexpr (DEC)
            dec_split_range(len, s, split_rows, split, lo, hi);
        else
            split_range(len, s, split_rows, split, split_floor, lo, hi);
    };

    // the union of the launch's tokens' ranges for this split
    int ulo = INT_MAX, uhi = 0;
    for (int t = 0; t < T; ++t) {
        int lo, hi;
        range(pos0 + t + 1, lo, hi);
        if (hi > lo) {
            ulo = lo < ulo ? lo : ulo;
            uhi = hi > uhi ? hi : uhi;
        }
    }
    // this lane's query column: token tq, q head h*G + gq
    const bool qvalid = ql < R;
    const int tq = qvalid ? ql / G : 0;
    const int gq = qvalid ? ql - tq * G : 0;
    int qlo = 0, qhi = 0;
    if (qvalid) range(pos0 + tq + 1, qlo, qhi);

    // fp16 layout: qreg[ks] = Q[column ql][64 w + 32 hh + 8 ks + 0..7]; int8
    // layout: qreg[4 nb + ks] = Q[column 16 nb + (l & 15)][128 (w >> 1) + 32 (l
    // / 16) + 8 ks + 0..7], the B operand of the 16x16x32 products
    f16x8 qreg[Q8 ? 8 : 4];
    auto load_q = [&] {
        if constexpr (Q8) {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int c = 16 * nb + (lane & 15);
                const bool ok = c < R;
                const int t = ok ? c / G : 0, g = ok ? c - t * G : 0;
                const f16* qrow = qg + (((size_t)b * T + t) * n_q_heads + h * G + g) * q_pitch +
                                  128 * (w >> 1) + 32 * (lane >> 4);
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    qreg[4 * nb + ks] = ok ? *(const f16x8*)(qrow + 8 * ks) : (f16x8)(0);
            }
        } else {
            const f16* qrow = qg + (((size_t)b * T + tq) * n_q_heads + h * G + gq) * q_pitch + 64 * w + 32 * hh;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) qreg[ks] = qvalid ? *(const f16x8*)(qrow + 8 * ks) : (f16x8)(0);
        }
    };
    if constexpr (!STAGE) load_q();

    f32x16 o0 = (f32x16)(0.f), o1 = (f32x16)(0.f);
    float m_run = -1e30f, l_run = 0.f;

    // at_barrier: run before the mid-tile barrier (pre) and after it (post)
    auto body = [&](const DecTileRegs& r, int j, auto&& pre, auto&& post) {
        const int buf = j & 1;
        const int vb = Q8 ? buf : 0;
        if constexpr (Q8) {
            // partial scores of 16 rows x 32 columns over this wave's 128 dims
            // (16x16x32: lane 16 g + i holds rows 4 g .. + 3 of column i), stored
            // where the 32x32 layout below reads rows 8 r4 + 4 hh .. + 3 of
            // column ql: r4 = 2 (w & 1) + g / 2, hh = g & 1
            f32x4 c0 = (f32x4)(0.f), c1 = (f32x4)(0.f);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.k[ks], qreg[ks], c0, 0, 0, 0);
                c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.k[ks], qreg[4 + ks], c1, 0, 0, 0);
            }
            const int g = lane >> 4, lp = (lane & 15) + 32 * (g & 1);
            s_part[buf][w >> 1][2 * (w & 1) + (g >> 1)][lp] = c0;
            s_part[buf][w >> 1][2 * (w & 1) + (g >> 1)][lp + 16] = c1;
            // V slice, transposed to [d][kv] in the region of the wave that
            // owns dims 64 w' .. (w' = 2 (w >> 1) + l / 32)
            const int own = 2 * (w >> 1) + (lane >> 5), d0 = 8 * ((lane >> 2) & 7);
            const int kv0 = 16 * (w & 1) + 4 * (lane & 3);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const f16x4 col = {r.v[0][e], r.v[1][e], r.v[2][e], r.v[3][e]};
                *(f16x4*)&s_vt[vb][own][d0 + e][kv0] = col;
            }
        } else {
            // partial scores of this wave's 64 dims
            f32x16 sacc = (f32x16)(0.f);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(r.k[ks], qreg[ks], sacc, 0, 0, 0);
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                s_part[buf][w][r4][lane] =
                    (f32x4){sacc[4 * r4], sacc[4 * r4 + 1], sacc[4 * r4 + 2], sacc[4 * r4 + 3]};
            // V slice, transposed to [d][kv] in this wave's LDS region
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const f16x4 col = {r.v[0][e], r.v[1][e], r.v[2][e], r.v[3][e]};
                *(f16x4*)&s_vt[0][w][8 * (lane >> 3) + e][4 * (lane & 7)] = col;
            }
        }
        pre();
        lds_barrier();
        post();
        // full scores, summed in wave order
        float sc[16];
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            f32x4 t4;
            if constexpr (Q8) {
                t4 = s_part[buf][0][r4][lane] + s_part[buf][1][r4][lane];
            } else {
                const f32x4 a0 = s_part[buf][0][r4][lane], a1 = s_part[buf][1][r4][lane];
                const f32x4 a2 = s_part[buf][2][r4][lane], a3 = s_part[buf][3][r4][lane];
                t4 = ((a0 + a1) + a2) + a3;
            }
            sc[4 * r4] = t4[0];
            sc[4 * r4 + 1] = t4[1];
            sc[4 * r4 + 2] = t4[2];
            sc[4 * r4 + 3] = t4[3];
        }
        // online softmax of this lane's column over the tile's 32 rows. The
        // range mask only runs when some column's range ends inside the tile.
        const int r0 = j * DEC_TILE;
        const bool inside = !qvalid || (r0 >= qlo && r0 + DEC_TILE <= qhi);
        if (!__all(inside)) {
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const int row = r0 + 8 * (rr >> 2) + 4 * hh + (rr & 3);
                sc[rr] = (row >= qlo && row < qhi) ? sc[rr] : -INFINITY;
            }
        }
        float mt = sc[0];
#pragma unroll
        for (int rr = 1; rr < 16; ++rr) mt = fmaxf(mt, sc[rr]);
        mt = pair32_max(mt) * sl2;
        // A column's running max moves only when the tile's max exceeds it by
        // more than RESCALE_LOG2: p <= 2^RESCALE_LOG2 stays exact in fp16 range
        // and O / l are rescaled on few tiles. The decision is the column's own
        // (corr = 1 exactly for the others), so a token's values do not depend
        // on the other tokens in the launch.
        const bool grow = mt > m_run + RESCALE_LOG2;
        if (__any(grow)) {
            const float m_new = grow ? mt : m_run;
            const float corr = fast_exp2(m_run - m_new);
            m_run = m_new;
            l_run *= corr;
            o0 *= corr;
            o1 *= corr;
        }
        float psum = 0.f;
        f16x8 pk0, pk1;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            const float p = fast_exp2(fmaf(sc[rr], sl2, -m_run));
            psum += p;
            if (rr < 8) pk0[rr] = (f16)p;
            else pk1[rr - 8] = (f16)p;
        }
        l_run += pair32_sum(psum);
        // O^T += V^T P^T over the tile's two 16-row k-steps
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const f16x8 pb = ks ? pk1 : pk0;
            {
                const f16x4 lo4 = *(const f16x4*)&s_vt[vb][w][ql][16 * ks + 4 * hh];
                const f16x4 hi4 = *(const f16x4*)&s_vt[vb][w][ql][16 * ks + 8 + 4 * hh];
                const f16x8 a = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                o0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o0, 0, 0, 0);
            }
            {
                const f16x4 lo4 = *(const f16x4*)&s_vt[vb][w][32 + ql][16 * ks + 4 * hh];
                const f16x4 hi4 = *(const f16x4*)&s_vt[vb][w][32 + ql][16 * ks + 8 + 4 * hh];
                const f16x8 a = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                o1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb, o1, 0, 0, 0);
            }
        }
    };

    auto none = [] {};
    if constexpr (STAGE) {
        static_assert(Q8, "the staged tiles are int8");
        if (uhi > ulo) {
            // NBUF stages, copied NBUF - 1 tiles ahead of the one computed.
            // Tile j's copies are waited for (each wave its own, then the
            // mid-tile barrier of tile j - 1) before tile j is read; stage j
            // is refilled after tile j's barrier, when every wave is past
            // reading it. Copies past the last tile re-copy it (clamped), so
            // every wave issues Q8_COPIES a tile and the waits are constants.
            const int j0 = ulo / DEC_TILE;
            const int j1 = (uhi + DEC_TILE - 1) / DEC_TILE;
            const uint32_t rs = (uint32_t)row_stride;   // bytes between rows; caches < 2 GiB
            const char* kb = uniform_ptr(kbase8);
            const char* vb = uniform_ptr(vbase8);
            const char* sc = (const char*)(hh ? vsb : ksb);
            uint32_t copy_off[2];
#pragma unroll
            for (int c = 0; c < 2; ++c)
                copy_off[c] = 16 * ((lane & 15) ^ q8_sw(8 * w + 4 * c + (lane >> 4)));
            const uint32_t stage0 = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) char*)s_stage);
#pragma unroll
            for (int p = 0; p < NBUF; ++p)
                q8_issue(stage0 + p * Q8_STAGE_B, kb, vb, sc, rs, j0 + p, uhi, w, lane, copy_off);
            // q after the copies, then one wait for all of them: the compiler
            // does not see the copies, so a wait it placed for q would land in
            // the loop and drain every tile's copies
            asm volatile("" ::: "memory");
            load_q();
            WAIT_VMCNT(0);
            tile_ready();
            int st = 0;
            for (int j = j0; j < j1; ++j) {
                const DecTileRegs r = q8_stage_tile((lds_cchar*)s_stage + st * Q8_STAGE_B, lane, w);
                const int sn = st;
                body(r, j, [] { WAIT_VMCNT((NBUF - 2) * Q8_COPIES); },
                     [&] {
                         q8_issue(stage0 + sn * Q8_STAGE_B, kb, vb, sc, rs, j + NBUF, uhi, w, lane,
                                  copy_off);
                     });
                st = st == NBUF - 1 ? 0 : st + 1;
            }
            WAIT_VMCNT(0);   // no copy into LDS outlives the workgroup
        }
    } else if (uhi > ulo) {
        // NBUF register tile buffers: the loads of tile j + NBUF - 1 are issued
        // before the math of tile j. Every load is issued unconditionally (rows
        // and tiles clamped into the range: a row past uhi reads row uhi - 1,
        // masked to p = 0; a tile past the end re-reads the last one), so the
        // compiler's wait before tile j's math counts exactly the loads of the
        // tiles behind it instead of draining them all.
        typedef typename std::conditional<Q8, DecTileQ8, DecTileRegs>::type Raw;
        auto load = [&](Raw& r, int j) {
            if constexpr (Q8)
                dec_load_tile<NT_V>(r, kbase8, vbase8, ksb, vsb, row_stride, j, uhi, lane, w);
            else
                dec_load_tile<NT_V>(r, kbase, vbase, row_stride, j, uhi, lane, w);
        };
        const int j0 = ulo / DEC_TILE;
        const int j1 = (uhi + DEC_TILE - 1) / DEC_TILE;
        Raw rbuf[NBUF];
#pragma unroll
        for (int p = 0; p < NBUF - 1; ++p) load(rbuf[p], min(j0 + p, j1 - 1));
        for (int j = j0; j < j1; j += NBUF) {
#pragma unroll
            for (int u = 0; u < NBUF; ++u) {
                const int jj = j + u;
                load(rbuf[(u + NBUF - 1) % NBUF], min(jj + NBUF - 1, j1 - 1));
                if (jj < j1) {
                    if constexpr (Q8)
                        body(dec_dequant(rbuf[u], lane), jj, none, none);
                    else
                        body(rbuf[u], jj, none, none);
                }
            }
        }
    }

    if (qvalid && (!DEC || qhi > qlo)) {
        const size_t part = (((size_t)b * T + tq) * n_q_heads + h * G + gq) * split + s;
        float* dst = pacc + part * DEC_HD + 64 * w + 4 * hh;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            *(f32x4*)(dst + 8 * r4) = (f32x4){o0[4 * r4], o0[4 * r4 + 1], o0[4 * r4 + 2], o0[4 * r4 + 3]};
            *(f32x4*)(dst + 32 + 8 * r4) =
                (f32x4){o1[4 * r4], o1[4 * r4 + 1], o1[4 * r4 + 2], o1[4 * r4 + 3]};
        }
        if (w == 0 && hh == 0) {
            if constexpr (DEC)
                pm[part] = m_run;
            else
                pm[part] = l_run > 0.f ? m_run * FL_LN2 : -1e30f;
            pd[part] = l_run;
        }
    }
}

// ---------------------------------------------------------------------------
// merge (+ gate): attention_merge (kernels.cu:1387-1424) with attn_gate
// (kernels.cu:1572-1600) fused. z = f16_sat(sum_s e_s acc_s / sum_s e_s d_s),
// e_s = e^(m_s - M) with M = max_s m_s, then z = f16_sat(z * sigmoid(g)).
// One block of 256 threads a (row, q head), one pass over the partials:
// thread tid owns the float4 of dims 4c..4c+3 (c = tid % C, C = head_dim / 4)
// for the splits s = j, j + J, ... (j = tid / C, J = 256 / C), read in
// batches of eight with every load issued before any is used (indices past
// the last split clamped, their values replaced by an empty partial). Each
// thread weighs its splits by e^(m_s - M_j) against its own running max M_j
// (rescaled when a batch raises it); the J group sums are then weighed by
// e^(M_j - M) and added in j order through LDS. The gate is read before the
// partials. Empty partials (m = -1e30, d = 0, acc = 0) contribute exact
// zeros, so the result does not depend on how many empty splits follow a
// token's own.
// ---------------------------------------------------------------------------
constexpr int MG_THREADS = 256;
constexpr int MG_BATCH = 8;

//
// DEC: attention_dec_merge's contract (kernels.cu:1336-1385) -- pm in log2
// units and only the first St = dec_split_count(pos0 + row + 1, tmin,
// split) partials of a row written (the rest are never read); otherwise pm
// in natural-log units and all `split` partials read.
template <bool DEC>
__global__ void __launch_bounds__(MG_THREADS)
attn_merge_kernel(const float* __restrict__ pacc, const float* __restrict__ pm,
                  const float* __restrict__ pd, f16* __restrict__ z,
                  const f16* __restrict__ gate, int n_q_heads, int head_dim, int z_pitch,
                  int g_pitch, int g_off, int split, int pos0, int tmin) {
    __shared__ f32x4 s_num[MG_THREADS];
    __shared__ float s_den[MG_THREADS];
    __shared__ float s_mx[MG_THREADS];
    const int head = blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
    const int C = head_dim >> 2, J = MG_THREADS / C;
    const int c = tid % C, j = tid / C;
    const size_t rh = (size_t)row * n_q_heads + head;
    const size_t p0 = rh * split;
    const float* pmr = pm + p0;
    const float* pdr = pd + p0;
    const int ns = DEC ? dec_split_count(pos0 + row + 1, tmin, split) : split;
    const float units = DEC ? 1.f : FL_LOG2E;   // m_s to log2 units

    float gv[4] = {0.f, 0.f, 0.f, 0.f};
    if (gate != nullptr && tid < C) {
        const f16* gr = gate + rh * g_pitch + g_off + 4 * tid;
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e] = (float)gr[e];
    }

    f32x4 num = (f32x4)(0.f);
    float den = 0.f, M = -1e30f;
    if (j < J) {
        const f32x4* acc = (const f32x4*)(pacc + p0 * head_dim) + c;
        for (int s = j; s < ns; s += MG_BATCH * J) {
            float mv[MG_BATCH], dv[MG_BATCH];
            f32x4 av[MG_BATCH];
#pragma unroll
            for (int u = 0; u < MG_BATCH; ++u) {
                const int si = min(s + u * J, ns - 1);
                mv[u] = pmr[si];
                dv[u] = pdr[si];
                av[u] = acc[(size_t)si * C];
            }
            float bm = M;
#pragma unroll
            for (int u = 0; u < MG_BATCH; ++u) {
                const bool ok = s + u * J < ns;
                mv[u] = ok ? mv[u] : -1e30f;
                dv[u] = ok ? dv[u] : 0.f;
                av[u] = ok ? av[u] : (f32x4)(0.f);
                bm = fmaxf(bm, mv[u]);
            }
            if (bm > M) {
                const float corr = fast_exp2((M - bm) * units);
                num *= corr;
                den *= corr;
                M = bm;
            }
#pragma unroll
            for (int u = 0; u < MG_BATCH; ++u) {
                const float e = fast_exp2((mv[u] - M) * units);
                num[0] = fmaf(e, av[u][0], num[0]);
                num[1] = fmaf(e, av[u][1], num[1]);
                num[2] = fmaf(e, av[u][2], num[2]);
                num[3] = fmaf(e, av[u][3], num[3]);
                den = fmaf(e, dv[u], den);
            }
        }
    }
    s_num[tid] = num;
    s_den[tid] = den;
    s_mx[tid] = M;
    __syncthreads();
    if (tid < C) {
        float Mg = s_mx[tid];
        for (int jj = 1; jj < J; ++jj) Mg = fmaxf(Mg, s_mx[jj * C + tid]);
        f32x4 n = (f32x4)(0.f);
        float dsum = 0.f;
        for (int jj = 0; jj < J; ++jj) {
            const float e = fast_exp2((s_mx[jj * C + tid] - Mg) * units);
            const f32x4 o = s_num[jj * C + tid];
            n[0] = fmaf(e, o[0], n[0]);
            n[1] = fmaf(e, o[1], n[1]);
            n[2] = fmaf(e, o[2], n[2]);
            n[3] = fmaf(e, o[3], n[3]);
            dsum = fmaf(e, s_den[jj * C + tid], dsum);
        }
        const float inv = 1.f / dsum;
        f16* zr = z + rh * z_pitch + 4 * tid;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            f16 zv = f16_sat(n[e] * inv);
            if (gate != nullptr) zv = f16_sat((float)zv * sigmoid_f(gv[e]));
            zr[e] = zv;
        }
    }
}

// The same merge for fl_attention_merge's callers (the KV-split prefill: T up
// to a chunk of 1024 tokens, so T x 24 (row, head) pairs of a few splits
// each): one wavefront a pair, lane l holding dims 4 l .. 4 l + 3 (head_dim
// <= 256), four pairs a workgroup, no LDS and no barrier. The splits are read
// in batches of eight, every load issued before any is used, and weighed by
// e^(m_s - M) against the running max M, rescaled when a batch raises it --
// attn_merge_kernel's arithmetic with one running max instead of J (the J
// group sums' order differs, so the two agree to rounding). A block a pair
// spent most of its time on its barrier and LDS exchange: a 1024-token
// chunk's 4 splits (101 MB of partials) took 39 us that way, 17 us this way.
constexpr int MR_PAIRS = 4;   // (row, head) pairs a workgroup, one a wave
__global__ void __launch_bounds__(64 * MR_PAIRS)
attn_merge_rows_kernel(const float* __restrict__ pacc, const float* __restrict__ pm,
                       const float* __restrict__ pd, f16* __restrict__ z,
                       const f16* __restrict__ gate, int n_q_heads, int head_dim, int z_pitch,
                       int g_pitch, int g_off, int split, long long n_pairs) {
    const int lane = threadIdx.x & 63;
    const long long rh = (long long)blockIdx.x * MR_PAIRS + (threadIdx.x >> 6);
    if (rh >= n_pairs) return;                            // wave-uniform
    const int C = head_dim >> 2;
    const bool on = lane < C;
    const int c = on ? lane : 0;                          // idle lanes read dims 0..3
    const size_t p0 = (size_t)rh * split;
    const float* pmr = pm + p0;
    const float* pdr = pd + p0;
    const f32x4* acc = (const f32x4*)(pacc + p0 * head_dim) + c;

    float gv[4] = {0.f, 0.f, 0.f, 0.f};
    if (gate != nullptr) {
        const f16* gr = gate + (size_t)rh * g_pitch + g_off + 4 * c;
#pragma unroll
        for (int e = 0; e < 4; ++e) gv[e] = (float)gr[e];
    }
    f32x4 num = (f32x4)(0.f);
    float den = 0.f, M = -1e30f;
    for (int s = 0; s < split; s += MG_BATCH) {
        float mv[MG_BATCH], dv[MG_BATCH];
        f32x4 av[MG_BATCH];
#pragma unroll
        for (int u = 0; u < MG_BATCH; ++u) {
            const int si = min(s + u, split - 1);
            mv[u] = pmr[si];
            dv[u] = pdr[si];
            av[u] = acc[(size_t)si * C];
        }
        float bm = M;
#pragma unroll
        for (int u = 0; u < MG_BATCH; ++u) {
            const bool ok = s + u < split;
            mv[u] = ok ? mv[u] : -1e30f;
            dv[u] = ok ? dv[u] : 0.f;
            av[u] = ok ? av[u] : (f32x4)(0.f);
            bm = fmaxf(bm, mv[u]);
        }
        if (bm > M) {
            const float corr = fast_exp2((M - bm) * FL_LOG2E);
            num *= corr;
            den *= corr;
            M = bm;
        }
#pragma unroll
        for (int u = 0; u < MG_BATCH; ++u) {
            const float e = fast_exp2((mv[u] - M) * FL_LOG2E);
            num[0] = fmaf(e, av[u][0], num[0]);
            num[1] = fmaf(e, av[u][1], num[1]);
            num[2] = fmaf(e, av[u][2], num[2]);
            num[3] = fmaf(e, av[u][3], num[3]);
            den = fmaf(e, dv[u], den);
        }
    }
    if (!on) return;
    const float inv = 1.f / den;
    f16x4 out;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f16 zv = f16_sat(num[e] * inv);
        if (gate != nullptr) zv = f16_sat((float)zv * sigmoid_f(gv[e]));
        out[e] = zv;
    }
    *(f16x4*)(z + (size_t)rh * z_pitch + 4 * c) = out;
}

// The output gate for layouts the 8-a-lane kernel below does not take (odd
// head_dim, pitches or offsets, unaligned buffers): one wavefront a (token,
// head) row, lane l taking elements l, l + 64, ... of it, with the same
// sigmoid_f and roundings.
__global__ void __launch_bounds__(64)
attn_gate_row_kernel(f16* __restrict__ z, const f16* __restrict__ g, int head_dim, int z_pitch,
                     int g_pitch, int g_off) {
    const size_t row = blockIdx.x;                      // token n_heads + head
    f16* zr = z + row * z_pitch;
    const f16* gr = g + row * g_pitch + g_off;
    for (int d = threadIdx.x; d < head_dim; d += 64)
        zr[d] = f16_sat((float)zr[d] * sigmoid_f((float)gr[d]));
}

// The gate with 8 elements a lane (one 16-byte load of z and of g, one store
// of z), for head_dim, the pitches and g_off multiples of 8 and 16-byte
// aligned z / g: the same sigmoid_f and roundings as attn_gate_row_kernel,
// so the same bits. chunks = T n_heads head_dim / 8 lanes in all.
__global__ void __launch_bounds__(256)
attn_gate_vec_kernel(f16* __restrict__ z, const f16* __restrict__ g, int n_heads, int head_dim,
                     int z_pitch, int g_pitch, int g_off, long long chunks) {
    const long long c = (long long)blockIdx.x * 256 + threadIdx.x;
    if (c >= chunks) return;
    const int per_row = head_dim >> 3;
    const long long row = c / per_row;                  // (token, head)
    const int d = (int)(c - row * per_row) * 8;
    f16x8* zp = (f16x8*)(z + row * z_pitch + d);
    const f16x8 gv = *(const f16x8*)(g + row * g_pitch + g_off + d);
    f16x8 zv = *zp;
#pragma unroll
    for (int e = 0; e < 8; ++e) zv[e] = f16_sat((float)zv[e] * sigmoid_f((float)gv[e]));
    *zp = zv;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The batched decode's split floor (split_count): on MI355X a 4k-row B = 1
// decode with 16 splits of 256 rows leaves 192 of 256 CUs idle; 32 splits of
// 64-128 rows run it 1.3x faster, while 4-sequence verify launches at 8k and
// beyond keep their 256-row splits (more splits there cost more in partial
// traffic than the wider grid gains).
#ifndef DEC_SPLIT_FLOOR
#define DEC_SPLIT_FLOOR 32
#endif

// int8 register tiles: 2 buffers (168 VGPRs, three waves a SIMD) -- in the
// int8 layout 3 buffers (two waves a SIMD) measured 83.4 / 30.9 us at ~32k /
// ~8k against 77.5 / 28.0, 4 and 5 slower still
#ifndef DEC_NBUF_Q8
#define DEC_NBUF_Q8 2
#endif

// int8 grids of at most one workgroup a CU take the LDS-staged tiles (2
// stages of Q8_STAGE_B: 92 KiB of LDS, one workgroup a CU): whole-line
// copies and no registers held by tiles in flight. Measured on MI355X: the
// per-sequence launches of attention_dec_q8 (112 workgroups, ~100k rows
// each) 478 against 525 us a step for the register tiles; B = 1 at 4k-16k
// within 3 % of them (12.2 at 4k either way); larger grids keep the register
// tiles, whose workgroups (three a CU) overlap each other's barriers (B = 4,
// T = 3 at ~8k / ~100k: 33.3 / 223 us against 34.4 / 235 staged, measured
// before the int8 layout). Both give the same bits.
constexpr int DEC_STAGE_MAX_WGS = 256;
constexpr int DEC_NBUF_STAGE = 2;

// grid_split blocks a (sequence, kv head); `split` the partials' stride;
// split_floor the floor of split_count (0: the reference's rule).
template <bool Q8, bool DEC>
int launch_split(const f16* qg, const DecSeqs& seqs, float* pacc, float* pm, float* pd, int B,
                 int T, int n_q_heads, int n_kv, int q_pitch, int grid_split, int split,
                 int split_rows, float sl2, hipStream_t stream, int split_floor = 0) {
    dim3 grid(grid_split, n_kv, B);
    if (Q8 && (long long)grid_split * n_kv * B <= DEC_STAGE_MAX_WGS)
        hipLaunchKernelGGL((attn_decode_split_kernel<DEC_NBUF_STAGE, false, true, DEC, true>),
                           grid, dim3(DEC_THREADS), 0, stream, qg, seqs, pacc, pm, pd, n_q_heads,
                           n_kv, q_pitch, T, split, split_rows, split_floor, sl2);
    else
        hipLaunchKernelGGL((attn_decode_split_kernel<Q8 ? DEC_NBUF_Q8 : DEC_NBUF, DEC_NT_V, Q8, DEC,
                                                     false>),
                           grid, dim3(DEC_THREADS), 0, stream, qg, seqs, pacc, pm, pd, n_q_heads,
                           n_kv, q_pitch, T, split, split_rows, split_floor, sl2);
    return fl::check_launch("attn_decode_split");
}

// sequence b over an int8 cache of capacity max_pos (scales after the values)
void set_q8_seq(DecSeqs& seqs, int b, const void* kc, const void* vc, int max_pos, int n_kv,
                int pos0) {
    const size_t vals = (size_t)max_pos * n_kv * DEC_HD;
    seqs.k[b] = (const f16*)kc;
    seqs.v[b] = (const f16*)vc;
    seqs.ks[b] = (const f16*)((const char*)kc + vals);
    seqs.vs[b] = (const f16*)((const char*)vc + vals);
    seqs.pos0[b] = pos0;
}

// The kernels address a cache row with a 32-bit byte offset from the layer's
// (or sequence's) base.
bool cache_fits(int max_pos, int n_kv, int bytes_per_elem) {
    return (uint64_t)max_pos * n_kv * DEC_HD * bytes_per_elem < (1ull << 31);
}

// The split ranges are formed with 32-bit unsigned products of a token's
// tile count and a split index.
bool split_math_fits(int max_pos, int split) {
    return (uint64_t)(max_pos / DEC_TILE + 1) * (uint64_t)(split + 1) < (1ull << 32);
}

int check_decode_geometry(int T, int n_q_heads, int n_kv, int head_dim, int q_pitch, int split,
                          int split_rows) {
    FL_REQUIRE(head_dim == DEC_HD, "head_dim must be 256");
    FL_REQUIRE(n_kv > 0 && n_q_heads > 0 && n_q_heads % n_kv == 0, "n_q_heads % n_kv_heads");
    FL_REQUIRE(T >= 1 && T * (n_q_heads / n_kv) <= 32, "T * (n_q_heads / n_kv_heads) <= 32");
    FL_REQUIRE(q_pitch >= head_dim && q_pitch % 8 == 0, "q_pitch >= head_dim, multiple of 8");
    FL_REQUIRE(split >= 1 && split <= 65535, "split in [1, 65535]");
    FL_REQUIRE(split_rows >= DEC_TILE, "split_rows >= 32");
    return FL_OK;
}

// The current device's compute-unit count, looked up once per device.
int dec_cu_count() {
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

// split_rows 0, the grid rule: S = floor(W / (B n_kv)) splits a token (at
// least 1, at most `split`), W one workgroup a CU over fp16 caches and two
// over int8 ones, fewer where the token's length leaves under 64 rows a
// split. Swept at B = 1..16 and ~8k..~100k (forced split counts,
// graph-timed): the fp16 kernel is fastest at one workgroup a CU (B = 4 at
// ~32k: 16 splits 85.3 us, 32: 88.9, 64: 91.4; B = 1 at ~8k: 64 splits
// 14.4 us, 32: 16.7), the int8 kernel, with three waves a SIMD, at two (B =
// 4 at ~32k: 32 splits 67.8 us, 16: 73.4, 64: 69.1). The optimum is sharp and
// a partial second round costs more than idle CUs (B = 4, T = 3 at ~8k / ~100k:
// 14 splits 30.5 / 260.8 us, 16: 29.2 / 244.6, 18: 40.8 / 341.9), hence the
// floor. A token's split count then depends on B as well as its length, so a
// batched call's values can differ in the last bits from single calls';
// split_rows > 0 keeps the length-only rule.
constexpr int DEC_GRID_RULE = 0;

void grid_rule(bool q8, int B, int n_kv, int split, int& rows, int& smax, int& floor_splits) {
    const int W = (q8 ? 2 : 1) * dec_cu_count();
    const int S = W / (B * n_kv);
    smax = S < 1 ? 1 : (S > split ? split : S);
    rows = DEC_FINE_ROWS;
    floor_splits = 0;
}

template <bool Q8>
int attn_decode_batched(const void* qg, int q_pitch, const void* const* kcache,
                        const void* const* vcache, const int* pos0, const int* cap, int B, int T,
                        int n_q_heads, int n_kv_heads, int head_dim, float scale, int split_rows,
                        int split, const void* gate, int g_pitch, int g_off, void* z, int z_pitch,
                        void* work, size_t work_bytes, fl_stream_t stream) {
    int rc = check_decode_geometry(T, n_q_heads, n_kv_heads, head_dim, q_pitch, split,
                                   split_rows == DEC_GRID_RULE ? DEC_TILE : split_rows);
    if (rc) return rc;
    FL_REQUIRE(B >= 1 && B <= FL_MAX_SEQS, "1 <= B <= FL_MAX_SEQS");
    FL_REQUIRE(qg && kcache && vcache && pos0 && cap && z && work, "null pointer");
    int rows = split_rows, smax = split, floor_splits = DEC_SPLIT_FLOOR;
    if (split_rows == DEC_GRID_RULE) grid_rule(Q8, B, n_kv_heads, split, rows, smax, floor_splits);
    FL_REQUIRE(z_pitch >= head_dim, "z_pitch >= head_dim");
    FL_REQUIRE(gate == nullptr || g_off + head_dim <= g_pitch, "g_off + head_dim <= g_pitch");
    FL_REQUIRE(aligned16(qg) && aligned16(work), "16-byte aligned qg / work");
    if (work_bytes < fl_attn_decode_work_bytes(B, T, n_q_heads, head_dim, split)) {
        fl::set_error("work: %zu bytes, fl_attn_decode_work_bytes asks %zu", work_bytes,
                      fl_attn_decode_work_bytes(B, T, n_q_heads, head_dim, split));
        return FL_ESCRATCH;
    }
    DecSeqs seqs = {};
    int grid_split = 1;
    for (int b = 0; b < B; ++b) {
        FL_REQUIRE(kcache[b] && vcache[b], "null cache pointer");
        FL_REQUIRE(aligned16(kcache[b]) && aligned16(vcache[b]), "16-byte aligned caches");
        FL_REQUIRE(pos0[b] >= 0 && pos0[b] + T <= cap[b], "pos0[b] + T <= cap[b]");
        FL_REQUIRE(cache_fits(cap[b], n_kv_heads, Q8 ? 1 : 2), "a cache of at most 2 GiB");
        FL_REQUIRE(split_math_fits(cap[b], split), "(cap / 32 + 1) * (split + 1) < 2^32");
        if (Q8)
            set_q8_seq(seqs, b, kcache[b], vcache[b], cap[b], n_kv_heads, pos0[b]);
        else {
            seqs.k[b] = (const f16*)kcache[b];
            seqs.v[b] = (const f16*)vcache[b];
            seqs.pos0[b] = pos0[b];
        }
        const int st = split_count(pos0[b] + T, rows, smax, floor_splits);
        grid_split = st > grid_split ? st : grid_split;
    }
    const size_t parts = (size_t)B * T * n_q_heads * grid_split;
    float* pacc = (float*)work;
    float* pm = pacc + parts * head_dim;
    float* pd = pm + parts;
    rc = launch_split<Q8, false>((const f16*)qg, seqs, pacc, pm, pd, B, T, n_q_heads, n_kv_heads,
                                 q_pitch, grid_split, grid_split, rows, scale * FL_LOG2E,
                                 (hipStream_t)stream, floor_splits);
    if (rc) return rc;
    hipLaunchKernelGGL(attn_merge_kernel<false>, dim3(n_q_heads, B * T), dim3(MG_THREADS), 0,
                       (hipStream_t)stream, pacc, pm, pd, (f16*)z, (const f16*)gate, n_q_heads,
                       head_dim, z_pitch, g_pitch, g_off, grid_split, 0, 1);
    return fl::check_launch("attn_merge");
}

}  // namespace

// ---------------------------------------------------------------------------
// Partials of fl_attn_decode_noalloc: one array a GPU (every device that
// loads the library holds its own copy until the process ends), shared by
// every call of that entry point on the device. The split kernel writes every
// partial slot the merge reads (empty splits included), so nothing here has
// to start at zero; two calls that overlap on one GPU race on it.
// ---------------------------------------------------------------------------
constexpr size_t DEC_SCRATCH_BYTES = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[DEC_SCRATCH_BYTES];

namespace {
constexpr int DEC_SCRATCH_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[DEC_SCRATCH_DEVICES];   // `scratch`'s address on each device

// The device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept: the array's name is a host-side
// stand-in, never a device address.
int scratch_on_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        fl::set_error("hipGetDevice: %s", hipGetErrorString(e));
        return FL_ELAUNCH;
    }
    FL_REQUIRE(dev >= 0 && dev < DEC_SCRATCH_DEVICES, "device index < 64");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            fl::set_error("hipGetSymbolAddress(scratch) on device %d: %s", dev,
                          hipGetErrorString(e));
            return FL_ELAUNCH;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return FL_OK;
}
}  // namespace

extern "C" {

int fl_kv_store(const void* k, const void* v, void* kcache, void* vcache, int layer, int pos0,
                int T, int n_kv_heads, int head_dim, int max_pos, fl_stream_t stream) {
    FL_REQUIRE(k && v && kcache && vcache, "null pointer");
    FL_REQUIRE(T >= 0 && pos0 >= 0 && layer >= 0, "T, pos0, layer >= 0");
    FL_REQUIRE(head_dim % 8 == 0 && n_kv_heads > 0, "head_dim % 8 == 0");
    FL_REQUIRE(pos0 + T <= max_pos, "pos0 + T <= max_pos");
    FL_REQUIRE(aligned16(k) && aligned16(v) && aligned16(kcache) && aligned16(vcache),
               "16-byte aligned buffers");
    if (T == 0) return FL_OK;
    const int row_u4 = n_kv_heads * head_dim / 8;
    const size_t layer_off = (size_t)layer * max_pos * row_u4;
    const int n = T * row_u4;
    hipLaunchKernelGGL(kv_store_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint4*)k, (const uint4*)v, (uint4*)kcache, (uint4*)vcache, layer_off,
                       pos0, T, row_u4);
    return fl::check_launch("kv_store");
}

int fl_attention_split_gqa(const void* q, const void* kcache, const void* vcache, float* pacc,
                           float* pm, float* pd, int layer, int n_q_heads, int n_kv_heads,
                           int head_dim, int q_pitch, int pos0, int max_pos, float scale,
                           int split_rows, int T, int split, fl_stream_t stream) {
    int rc = check_decode_geometry(T, n_q_heads, n_kv_heads, head_dim, q_pitch, split, split_rows);
    if (rc) return rc;
    FL_REQUIRE(q && kcache && vcache && pacc && pm && pd, "null pointer");
    FL_REQUIRE(pos0 >= 0 && layer >= 0 && pos0 + T <= max_pos, "pos0 + T <= max_pos");
    FL_REQUIRE(cache_fits(max_pos, n_kv_heads, 2), "a layer cache of at most 2 GiB");
    FL_REQUIRE(split_math_fits(max_pos, split), "(max_pos / 32 + 1) * (split + 1) < 2^32");
    FL_REQUIRE(aligned16(q) && aligned16(kcache) && aligned16(vcache) && aligned16(pacc),
               "16-byte aligned buffers");
    DecSeqs seqs = {};
    const size_t off = (size_t)layer * max_pos * n_kv_heads * head_dim;
    seqs.k[0] = (const f16*)kcache + off;
    seqs.v[0] = (const f16*)vcache + off;
    seqs.pos0[0] = pos0;
    return launch_split<false, false>((const f16*)q, seqs, pacc, pm, pd, 1, T, n_q_heads,
                                      n_kv_heads, q_pitch, split, split, split_rows,
                                      scale * FL_LOG2E, (hipStream_t)stream);
}

int fl_attention_split_gqa_q8(const void* q, const void* kcache, const void* vcache, float* pacc,
                              float* pm, float* pd, int layer, int n_q_heads, int n_kv_heads,
                              int head_dim, int q_pitch, int pos0, int max_pos, float scale,
                              int split_rows, int T, int split, fl_stream_t stream) {
    int rc = check_decode_geometry(T, n_q_heads, n_kv_heads, head_dim, q_pitch, split, split_rows);
    if (rc) return rc;
    FL_REQUIRE(q && kcache && vcache && pacc && pm && pd, "null pointer");
    FL_REQUIRE(layer == 0, "an int8 cache is one buffer a layer: layer must be 0");
    FL_REQUIRE(pos0 >= 0 && pos0 + T <= max_pos, "pos0 + T <= max_pos");
    FL_REQUIRE(cache_fits(max_pos, n_kv_heads, 1), "a cache of at most 2 GiB");
    FL_REQUIRE(split_math_fits(max_pos, split), "(max_pos / 32 + 1) * (split + 1) < 2^32");
    FL_REQUIRE(aligned16(q) && aligned16(kcache) && aligned16(vcache) && aligned16(pacc),
               "16-byte aligned buffers");
    DecSeqs seqs = {};
    set_q8_seq(seqs, 0, kcache, vcache, max_pos, n_kv_heads, pos0);
    return launch_split<true, false>((const f16*)q, seqs, pacc, pm, pd, 1, T, n_q_heads,
                                     n_kv_heads, q_pitch, split, split, split_rows,
                                     scale * FL_LOG2E, (hipStream_t)stream);
}

int fl_attention_dec_q8(const void* q, const void* kcache, const void* vcache, float* pacc,
                        float* pm, float* pd, int n_q_heads, int n_kv_heads, int q_pitch, int pos0,
                        int max_pos, float sl2, int tmin, int smax, int T, fl_stream_t stream) {
    int rc = check_decode_geometry(T, n_q_heads, n_kv_heads, DEC_HD, q_pitch, smax, DEC_TILE);
    if (rc) return rc;
    FL_REQUIRE(q && kcache && vcache && pacc && pm && pd, "null pointer");
    FL_REQUIRE(tmin >= 1, "tmin >= 1");
    FL_REQUIRE(pos0 >= 0 && pos0 + T <= max_pos, "pos0 + T <= max_pos");
    FL_REQUIRE(cache_fits(max_pos, n_kv_heads, 1), "a cache of at most 2 GiB");
    FL_REQUIRE(split_math_fits(max_pos, smax), "(max_pos / 32 + 1) * (smax + 1) < 2^32");
    FL_REQUIRE(aligned16(q) && aligned16(kcache) && aligned16(vcache) && aligned16(pacc),
               "16-byte aligned buffers");
    DecSeqs seqs = {};
    set_q8_seq(seqs, 0, kcache, vcache, max_pos, n_kv_heads, pos0);
    // the last token is the longest: its split count is the widest
    const int grid_split = dec_split_count(pos0 + T, tmin, smax);
    return launch_split<true, true>((const f16*)q, seqs, pacc, pm, pd, 1, T, n_q_heads, n_kv_heads,
                                    q_pitch, grid_split, smax, tmin, sl2, (hipStream_t)stream);
}

int fl_attention_dec_merge(const float* pacc, const float* pm, const float* pd, void* z,
                           int n_q_heads, int z_pitch, int pos0, int tmin, int smax, int T,
                           const void* gate, int g_pitch, int g_off, fl_stream_t stream) {
    FL_REQUIRE(pacc && pm && pd && z, "null pointer");
    FL_REQUIRE(n_q_heads >= 1 && T >= 1 && pos0 >= 0, "n_q_heads, T >= 1, pos0 >= 0");
    FL_REQUIRE(tmin >= 1 && smax >= 1 && z_pitch >= DEC_HD, "tmin, smax >= 1, z_pitch >= 256");
    FL_REQUIRE(gate == nullptr || g_off + DEC_HD <= g_pitch, "g_off + 256 <= g_pitch");
    FL_REQUIRE(aligned16(pacc), "16-byte aligned pacc");
    hipLaunchKernelGGL(attn_merge_kernel<true>, dim3(n_q_heads, T), dim3(MG_THREADS), 0,
                       (hipStream_t)stream, pacc, pm, pd, (f16*)z, (const f16*)gate, n_q_heads,
                       DEC_HD, z_pitch, g_pitch, g_off, smax, pos0, tmin);
    return fl::check_launch("attn_dec_merge");
}

int fl_kv_store_q8(const void* k, const void* v, void* kcache, void* vcache, int layer, int pos0,
                   int T, int n_kv_heads, int head_dim, int max_pos, fl_stream_t stream) {
    FL_REQUIRE(k && v && kcache && vcache, "null pointer");
    FL_REQUIRE(layer == 0, "an int8 cache is one buffer a layer: layer must be 0");
    FL_REQUIRE(head_dim == DEC_HD, "head_dim must be 256");
    FL_REQUIRE(T >= 0 && pos0 >= 0 && n_kv_heads > 0 && pos0 + T <= max_pos, "pos0 + T <= max_pos");
    FL_REQUIRE(((uintptr_t)k & 7u) == 0 && ((uintptr_t)v & 7u) == 0 &&
                   ((uintptr_t)kcache & 3u) == 0 && ((uintptr_t)vcache & 3u) == 0,
               "8-byte aligned k, v; 4-byte aligned caches");
    if (T == 0) return FL_OK;
    const size_t vals = (size_t)max_pos * n_kv_heads * DEC_HD;
    const int rows = T * n_kv_heads;
    hipLaunchKernelGGL(kv_store_q8_kernel, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                       (const f16*)k, (const f16*)v, (signed char*)kcache, (signed char*)vcache,
                       (f16*)((char*)kcache + vals), (f16*)((char*)vcache + vals), pos0, T,
                       n_kv_heads);
    return fl::check_launch("kv_store_q8");
}

int fl_attention_merge(const float* pacc, const float* pm, const float* pd, void* z,
                       int n_q_heads, int head_dim, int z_pitch, int T, int split,
                       const void* gate, int g_pitch, int g_off, fl_stream_t stream) {
    FL_REQUIRE(pacc && pm && pd && z, "null pointer");
    FL_REQUIRE(head_dim >= 4 && head_dim <= 4 * MG_THREADS && head_dim % 4 == 0 &&
                   z_pitch >= head_dim,
               "head_dim a multiple of 4 in [4, 1024], z_pitch >= head_dim");
    FL_REQUIRE(T >= 1 && split >= 1 && n_q_heads >= 1, "T, split, n_q_heads >= 1");
    FL_REQUIRE(gate == nullptr || g_off + head_dim <= g_pitch, "g_off + head_dim <= g_pitch");
    FL_REQUIRE(aligned16(pacc), "16-byte aligned pacc");
    if (head_dim <= 256 && z_pitch % 4 == 0 && ((uintptr_t)z & 7u) == 0) {
        const long long pairs = (long long)T * n_q_heads;
        hipLaunchKernelGGL(attn_merge_rows_kernel, dim3((unsigned)((pairs + MR_PAIRS - 1) / MR_PAIRS)),
                           dim3(64 * MR_PAIRS), 0, (hipStream_t)stream, pacc, pm, pd, (f16*)z,
                           (const f16*)gate, n_q_heads, head_dim, z_pitch, g_pitch, g_off, split,
                           pairs);
        return fl::check_launch("attn_merge_rows");
    }
    hipLaunchKernelGGL(attn_merge_kernel<false>, dim3(n_q_heads, T), dim3(MG_THREADS), 0,
                       (hipStream_t)stream, pacc, pm, pd, (f16*)z, (const f16*)gate, n_q_heads,
                       head_dim, z_pitch, g_pitch, g_off, split, 0, 1);
    return fl::check_launch("attn_merge");
}

int fl_attn_gate(void* z, const void* g, int n_heads, int head_dim, int z_pitch, int g_pitch,
                 int g_off, int T, fl_stream_t stream) {
    FL_REQUIRE(z && g, "null pointer");
    FL_REQUIRE(T >= 1 && n_heads >= 1 && head_dim >= 1, "T, n_heads, head_dim >= 1");
    FL_REQUIRE(z_pitch >= head_dim && g_off + head_dim <= g_pitch, "pitches");
    if (head_dim % 8 == 0 && z_pitch % 8 == 0 && g_pitch % 8 == 0 && g_off % 8 == 0 &&
        aligned16(z) && aligned16(g)) {
        const long long chunks = (long long)T * n_heads * (head_dim / 8);
        hipLaunchKernelGGL(attn_gate_vec_kernel, dim3((unsigned)((chunks + 255) / 256)),
                           dim3(256), 0, (hipStream_t)stream, (f16*)z, (const f16*)g, n_heads,
                           head_dim, z_pitch, g_pitch, g_off, chunks);
    } else {
        const long long rows = (long long)T * n_heads;
        FL_REQUIRE(rows < (1ll << 31), "T * n_heads < 2^31");
        hipLaunchKernelGGL(attn_gate_row_kernel, dim3((unsigned)rows), dim3(64), 0,
                           (hipStream_t)stream, (f16*)z, (const f16*)g, head_dim, z_pitch,
                           g_pitch, g_off);
    }
    return fl::check_launch("attn_gate");
}

size_t fl_attn_decode_work_bytes(int B, int T, int n_q_heads, int head_dim, int split) {
    if (B < 1 || T < 1 || n_q_heads < 1 || head_dim < 1 || split < 1) return 0;
    const size_t parts = (size_t)B * T * n_q_heads * split;
    const size_t acc = parts * head_dim * sizeof(float);
    return acc + 2 * parts * sizeof(float);
}

int fl_attn_decode(const void* qg, int q_pitch, const void* const* kcache,
                   const void* const* vcache, const int* pos0, const int* cap, int B, int T,
                   int n_q_heads, int n_kv_heads, int head_dim, float scale, int split_rows,
                   int split, const void* gate, int g_pitch, int g_off, void* z, int z_pitch,
                   void* work, size_t work_bytes, fl_stream_t stream) {
    return attn_decode_batched<false>(qg, q_pitch, kcache, vcache, pos0, cap, B, T, n_q_heads,
                                      n_kv_heads, head_dim, scale, split_rows, split, gate,
                                      g_pitch, g_off, z, z_pitch, work, work_bytes, stream);
}

int fl_attn_decode_noalloc(const void* qg, int q_pitch, const void* const* kcache,
                           const void* const* vcache, const int* pos0, const int* cap, int B,
                           int T, int n_q_heads, int n_kv_heads, int head_dim, float scale,
                           int split_rows, int split, const void* gate, int g_pitch, int g_off,
                           void* z, int z_pitch, fl_stream_t stream) {
    const size_t need = fl_attn_decode_work_bytes(B, T, n_q_heads, head_dim, split);
    if (need > DEC_SCRATCH_BYTES) {
        fl::set_error("fl_attn_decode_noalloc: B %d x T %d x %d heads x %d splits need %zu bytes of "
                      "partials; the static scratch holds %zu (use fl_attn_decode with a work "
                      "buffer)", B, T, n_q_heads, split, need, DEC_SCRATCH_BYTES);
        return FL_ESCRATCH;
    }
    void* ptr = nullptr;
    const int rc = scratch_on_current_device(&ptr);
    if (rc) return rc;
    return attn_decode_batched<false>(qg, q_pitch, kcache, vcache, pos0, cap, B, T, n_q_heads,
                                      n_kv_heads, head_dim, scale, split_rows, split, gate,
                                      g_pitch, g_off, z, z_pitch, ptr, DEC_SCRATCH_BYTES, stream);
}

size_t fl_attn_decode_noalloc_max_bytes(void) { return DEC_SCRATCH_BYTES; }

int fl_attn_decode_q8(const void* qg, int q_pitch, const void* const* kcache,
                      const void* const* vcache, const int* pos0, const int* cap, int B, int T,
                      int n_q_heads, int n_kv_heads, int head_dim, float scale, int split_rows,
                      int split, const void* gate, int g_pitch, int g_off, void* z, int z_pitch,
                      void* work, size_t work_bytes, fl_stream_t stream) {
    return attn_decode_batched<true>(qg, q_pitch, kcache, vcache, pos0, cap, B, T, n_q_heads,
                                     n_kv_heads, head_dim, scale, split_rows, split, gate,
                                     g_pitch, g_off, z, z_pitch, work, work_bytes, stream);
}

}  // extern "C"
