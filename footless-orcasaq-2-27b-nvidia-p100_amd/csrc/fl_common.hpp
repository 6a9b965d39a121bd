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

// sigmoid / silu with the correctly rounded divide (hipcc's default for `/`)
// and the accurate expf (kernels.cu:229-235 uses a precise divide as well).
__device__ __forceinline__ float sigmoid_f(float x) { return 1.f / (1.f + expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x / (1.f + expf(-x)); }

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
