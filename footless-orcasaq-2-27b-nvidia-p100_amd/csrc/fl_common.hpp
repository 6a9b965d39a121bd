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
