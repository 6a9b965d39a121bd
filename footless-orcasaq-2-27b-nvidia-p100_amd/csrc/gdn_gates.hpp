// The Gated DeltaNet gates, shared by the decode step (gdn.hip) and the
// chunked prefill's prep (gdn_chunk.hip): one definition, so the two paths
// form the same bits from the same logits.
#pragma once

#include "fl_common.hpp"

namespace {

// e^x built as the reference's __expf builds it: 2^(x log2 e) on the
// transcendental unit (v_exp_f32, 1 ulp).
__device__ __forceinline__ float hw_expf(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504f); }

// log1p(e) for e >= 0 from the hardware log2 (v_log_f32) with Goldberg's
// correction: u = 1 + e is rounded, and log(u) * e / (u - 1) cancels that
// rounding (log1p(e) = e to working precision where u == 1).
__device__ __forceinline__ float log1p_pos(float e) {
    const float u = 1.f + e, d = u - 1.f;
    return d == 0.f ? e : __builtin_amdgcn_logf(u) * 0.693147181f * (e * __builtin_amdgcn_rcpf(d));
}

// The gates (kernels.cu:1732-1748): beta = sigmoid(b) with a correctly
// rounded divide, decay = exp(-e^A softplus(a + dt_bias)), softplus =
// log1p(e^x) up to x = 20 and x above. The exponentials and the log run on the
// transcendental unit; against the fp64 values the worst error is ~1e-7 on
// beta and ~4e-7 on decay, inside the reference's own (4.6e-7 and 5.6e-6
// relative, kernels.cu:139), with a dozen dependent instructions instead of
// three libm calls in series. (The conv's silu keeps det_expf: its output is
// rounded to fp16, and with the transcendental unit's exponential an fp16
// flip now and then moved config 1's state after 1024 steps from 4e-8 to 4e-5
// of the oracle's, within the 1e-4 bar but too close to it.)
__device__ __forceinline__ float gdn_beta(float b) { return 1.f / (1.f + hw_expf(-b)); }
__device__ __forceinline__ float gdn_decay(float a_dt, float A) {
    const float sp = a_dt <= 20.f ? log1p_pos(hw_expf(a_dt)) : a_dt;
    return hw_expf(-hw_expf(A) * sp);
}

}  // namespace
