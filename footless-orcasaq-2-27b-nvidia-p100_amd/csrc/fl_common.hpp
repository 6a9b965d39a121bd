// Shared device helpers and host-side error plumbing for libfl355 (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "fl355.h"

typedef _Float16 f16;
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define FL_LOG2E 1.4426950408889634f
#define FL_LN2 0.6931471805599453f

// fp16 store with the range pinned to the largest finite magnitude (NaN kept):
// the reference's f16_sat (kernels.cu:187-195). The float -> half conversion
// is the hardware's round-to-nearest-even.
__device__ __forceinline__ f16 f16_sat(float v) {
    return (f16)(v != v ? v : fminf(fmaxf(v, -65504.f), 65504.f));
}

// exp(x) from IEEE operations only, so the CPU oracle (which carries the same
// routine) rounds every value the same way: Cody-Waite reduction x = n ln2 + r
// with ln2 split in two (the high part has trailing zero bits, so n * hi is
// exact), |r| <= ln2 / 2, then the degree-7 Taylor polynomial of e^r (the
// truncation error r^8 / 8! is below 0.1 ulp) and the exact scaling by 2^n.
// Accuracy ~1 ulp. Used where an fp32 result is rounded to fp16 and fed back
// into the recurrence (the conv's silu), so a last-bit difference from a
// platform exp cannot flip an fp16 value between the kernels and the oracle.
__device__ __forceinline__ float det_expf(float x) {
#pragma clang fp contract(off)
    if (x > 88.72f) return INFINITY;
    if (x < -103.98f) return 0.f;
    const float n = rintf(x * 1.44269504f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.4286068203094173e-06f, r);
    float p = 1.f / 5040.f;
    p = fmaf(p, r, 1.f / 720.f);
    p = fmaf(p, r, 1.f / 120.f);
    p = fmaf(p, r, 1.f / 24.f);
    p = fmaf(p, r, 1.f / 6.f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.f);
    p = fmaf(p, r, 1.f);
    return ldexpf(p, (int)n);
}

// sigmoid / silu with the correctly rounded divide (hipcc's default for `/`,
// as kernels.cu:229-235 asks with __fdiv_rn) over det_expf.
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + det_expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x / (1.f + det_expf(-x)); }

// exp2 on the hardware transcendental unit (v_exp_f32); -inf -> 0.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Lane exchange within a wavefront of 64 (ds_bpermute, no LDS traffic).
__device__ __forceinline__ float lane_xor(float v, int mask) {
    const int lane = __lane_id();
    return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

// max / sum of v over the lane pair (l, l ^ 32) on every lane, with one
// v_permlane32_swap (gfx950, a VALU operation) instead of an LDS-pipe lane
// exchange: with both operands v it returns (v[0..31], v[0..31]) and
// (v[32..63], v[32..63]), so lane l gets v[l % 32] and v[l % 32 + 32];
// max and + are symmetric, the result equals v op lane_xor(v, 32) bit for
// bit.
__device__ __forceinline__ float pair32_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_sum(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Lane exchanges at distance 1 and 2 inside each group of 4 lanes (DPP quad
// permutes, no LDS).
__device__ __forceinline__ float dpp_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// s_waitcnt vmcnt(n) (n < 64), every other counter left alone
#define WAIT_VMCNT(n) __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0F70)

// Workgroup barriers that are compiler memory barriers but add no vmcnt
// wait: __syncthreads() would drain vmcnt, i.e. wait for the next tile's
// copies too. tile_ready follows the explicit WAIT_VMCNT for this tile's
// copies; tile_done also waits for this wave's outstanding LDS reads, so no
// read of a stage can still be in flight when the copy that refills it is
// issued after the barrier.
__device__ __forceinline__ void tile_ready() { asm volatile("s_barrier" ::: "memory"); }
__device__ __forceinline__ void tile_done() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// One 16-byte-a-lane HBM -> LDS copy (global_load_lds_dwordx4): lane l's 16
// bytes land at LDS m0 + 16 l. Issued as asm so that the compiler does not
// track it as an LDS write in flight: it would otherwise drain vmcnt (wait for
// the next tile's copies) before every LDS read it cannot prove disjoint. The
// copies are waited for explicitly (WAIT_VMCNT + tile_ready). The s_nop is the
// wait state between the m0 write and its use by the copy.
__device__ __forceinline__ void copy16(const char* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds));
}
__device__ __forceinline__ void copy16_v(const char* vptr, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(vptr), "{m0}"(lds));
}
// p as a wave-uniform (scalar) value: the copies take their row base in SGPRs
__device__ __forceinline__ const char* uniform_ptr(const char* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const char*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// ---------------------------------------------------------------------------
// int8 KV cache format (kernels.cu:486-520): one buffer a layer of capacity
// max_pos, values [max_pos][n_kv][256] int8, then the scales
// [max_pos][n_kv][8] fp16 at byte max_pos * n_kv * 256. A 32-dim block shares
// the fp16 scale absmax / 127 and stores rint(x / scale) in [-127, 127]
// (0 where the scale is 0).
// ---------------------------------------------------------------------------
constexpr int Q8_BLOCK = 32;

__device__ __forceinline__ f16 q8_scale(float absmax) { return (f16)(absmax / 127.0f); }

__device__ __forceinline__ int q8_value(float x, float scale) {
    return scale > 0.f ? (int)fminf(fmaxf(rintf(x / scale), -127.f), 127.f) : 0;
}

// One 256-wide row held 4 consecutive elements a lane (lane l: dims 4l..4l+3,
// so a 32-dim block is 8 lanes) stored in the int8 format: its 256 values at
// `vals`, its 8 scales at `scales`. The block max is exact in any order.
__device__ __forceinline__ void q8_store_row(f16x4 y, signed char* vals, f16* scales, int lane) {
    float a = fmaxf(fmaxf(fabsf((float)y[0]), fabsf((float)y[1])),
                    fmaxf(fabsf((float)y[2]), fabsf((float)y[3])));
    a = fmaxf(a, lane_xor(a, 4));
    a = fmaxf(a, dpp_xor2(a));
    a = fmaxf(a, dpp_xor1(a));
    const f16 sh = q8_scale(a);
    const float sc = (float)sh;
    uint32_t packed = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) packed |= (uint32_t)(q8_value((float)y[c], sc) & 0xff) << (8 * c);
    *(uint32_t*)(vals + 4 * lane) = packed;
    if ((lane & 7) == 0) scales[lane >> 3] = sh;
}

typedef f16 f16x2 __attribute__((ext_vector_type(2)));

// Four int8 (one dword, byte 0 first) to fp16(byte * s): each byte is made an
// exact fp16 by placing (byte + 128) in the mantissa of 1024 (0x64XX is
// 1024 + XX) and subtracting 1152; the product with the scale rounds once.
__device__ __forceinline__ f16x4 q8_deq4(uint32_t b, f16x2 s2) {
    const uint32_t u = b ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const f16x2 off = {(f16)1152.f, (f16)1152.f};
    const f16x2 a = (__builtin_bit_cast(f16x2, lo) - off) * s2;
    const f16x2 c = (__builtin_bit_cast(f16x2, hi) - off) * s2;
    return (f16x4){a[0], a[1], c[0], c[1]};
}

// ---------------------------------------------------------------------------
// host side: status + thread-local detail message
// ---------------------------------------------------------------------------
namespace fl {
void set_error(const char* fmt, ...);
inline int einval(const char* what) {
    set_error("invalid argument: %s", what);
    return FL_EINVAL;
}
int check_launch(const char* kernel);
}  // namespace fl

#define FL_REQUIRE(cond, msg) \
    do {                      \
        if (!(cond)) return fl::einval(msg); \
    } while (0)
