// The full-attention layer's preparation between its projections and the
// attention: per-head Gemma RMSNorm of q and k, partial NeoX RoPE, and the
// fp16 KV cache store -- fused, or as the separate steps.
//
// Reference behaviour restated (kernels.cu, host runtime.py:2797-2815):
//   rmsnorm1p (kernels.cu:241-272): y = f16(x * rsqrt(sum(x^2) / n + eps) * (1 + w)),
//     mean-space eps, the sum in block_reduce_sum's order (kernels.cu:214-227);
//     q is normalised inside the q|gate buffer (pitch 2 head_dim), k packed.
//   rope_partial (kernels.cu:397-455): pairs (j, j + rope_dim / 2) of the first
//     rope_dim dims rotate by pos * theta^(-2j / rope_dim), the frequency and
//     angle and sincos in fp64, cos / sin rounded to fp32, the pair products
//     in fp32 on the fp16-rounded normed values; dims past rope_dim are not
//     touched.
//   kv_store (kernels.cu:457-484): the roped k row and the v row to position
//     pos0 + t of the layer's cache.
//   attn_prep_q8 (kernels.cu:837-908): the same fused, with kv_store_q8's int8
//     store (kernels.cu:486-520) in place of kv_store.
//
// One workgroup a (token, group of 4 RPW heads), a wavefront RPW rows (all
// loaded before any is processed). The rotation's cos / sin depend only on
// (position, pair), so the workgroup computes the rope_dim / 2 pairs once
// into LDS: the fp64 frequencies theta^(-2j / rope_dim), which do not depend
// on the position, formed once on the host (std::pow) and passed in the
// kernel arguments, the angle and its sincos in fp64, as the reference does
// for every row. A lane holds 4 consecutive
// elements of a row (one 8-byte load): the reference's warp w' (elements
// 32 w'..32 w' + 31) is lanes 8 w'..8 w' + 7, and its __shfl_down tree over
// offsets 16, 8, 4, 2, 1 becomes lane exchanges at distance 4, 2, 1 followed
// by the in-lane pairs (c, c + 2) and (0, 1) -- the same additions in the same
// order. The 8 warp sums are then combined as block_reduce_sum's second stage.
#include "fl_common.hpp"

#include <cmath>
#include <mutex>

// Products and sums round separately (no fma contraction), as the oracle's
// restatement does, so the two agree bit for bit.
#pragma clang fp contract(off)

namespace {

constexpr int PR_HD = 256;
constexpr int PR_WAVES = 4;
constexpr int PR_MAXPAIRS = PR_HD / 2;

// The rotation's frequencies theta^(-2j / rope_dim), j < rope_dim / 2, in
// fp64: they do not depend on the position, so the host forms them once per
// (theta, rope_dim) and they ride in the kernel arguments.
struct RopeFreqs {
    double f[PR_MAXPAIRS];
};

// The rows of a batched decode step, each its own sequence's: row t goes to
// cache kc[t] / vc[t] (capacity max_pos[t]) at position pos[t].
struct PrepRows {
    void* kc[FL_MAX_SEQS];
    void* vc[FL_MAX_SEQS];
    int pos[FL_MAX_SEQS];
    int max_pos[FL_MAX_SEQS];
};

// flags: bit 0 norm, bit 1 rope, bit 2 KV store (k rows and their v rows),
// bit 3 the store in the int8 format (caches of capacity max_pos); RPW rows a
// wavefront. ROWS: token t is row t of a batched decode step, its position,
// cache and capacity from `rows` (pos0, kc, vc and max_pos unused).
template <int FLAGS, int RPW, bool ROWS = false>
__global__ void __launch_bounds__(64 * PR_WAVES)
attn_prep_kernel(const f16* q, f16* qo, int q_pitch, f16* k, int k_pitch,
                 const f16* __restrict__ v, const float* __restrict__ wq,
                 const float* __restrict__ wk, void* __restrict__ kc_, void* __restrict__ vc_,
                 int n_q_heads, int n_kv_heads, int pos0, int max_pos_, int rope_dim,
                 const RopeFreqs freqs, float eps, const PrepRows rows) {
    __shared__ float scs[PR_MAXPAIRS], ssn[PR_MAXPAIRS];
    __shared__ __attribute__((aligned(16))) f16 srow[PR_WAVES][PR_HD];
    constexpr bool NORM = FLAGS & 1, ROPE = FLAGS & 2, STORE = FLAGS & 4, Q8 = FLAGS & 8;
    const int t = blockIdx.x, hd0 = blockIdx.y * PR_WAVES * RPW;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int pos = ROWS ? rows.pos[t] : pos0 + t;
    void* const kc = ROWS ? rows.kc[t] : kc_;
    void* const vc = ROWS ? rows.vc[t] : vc_;
    const int max_pos = ROWS ? rows.max_pos[t] : max_pos_;
    const int half_r = rope_dim >> 1;
    if (ROPE) {
        for (int j = threadIdx.x; j < half_r; j += 64 * PR_WAVES) {
            const double ang = (double)pos * freqs.f[j];
            double sn, cs;
            sincos(ang, &sn, &cs);
            scs[j] = (float)cs;
            ssn[j] = (float)sn;
        }
        __syncthreads();
    }
    const int heads = n_q_heads + n_kv_heads;
    f16x4 yin[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int hd = hd0 + w + PR_WAVES * r;
        if (hd >= heads) break;
        const bool is_q = hd < n_q_heads;
        const size_t roff = is_q ? ((size_t)t * n_q_heads + hd) * q_pitch
                                 : ((size_t)t * n_kv_heads + hd - n_q_heads) * k_pitch;
        yin[r] = *(const f16x4*)((is_q ? q : k) + roff + 4 * lane);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int hd = hd0 + w + PR_WAVES * r;
        if (hd >= heads) break;
        const bool is_q = hd < n_q_heads;
        const int h = is_q ? hd : hd - n_q_heads;
        const size_t roff = is_q ? ((size_t)t * n_q_heads + h) * q_pitch
                                 : ((size_t)t * n_kv_heads + h) * k_pitch;
        f16* orow = is_q ? qo + roff : k + roff;   // q rows may go elsewhere; k in place
        f16x4 y = yin[r];
        if (NORM) {
            float x[4], sq[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                x[c] = (float)y[c];
                sq[c] = fmaf(x[c], x[c], 0.f);
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                sq[c] += lane_xor(sq[c], 4);   // offset 16
                sq[c] += dpp_xor2(sq[c]);      // offset 8
                sq[c] += dpp_xor1(sq[c]);      // offset 4
            }
            const float ws = (sq[0] + sq[2]) + (sq[1] + sq[3]);   // offsets 2, 1: lane 8 w' = warp w'
            auto at = [](float val, int src) {
                return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(val), src));
            };
            const float r0 = at(ws, 0), r1 = at(ws, 8), r2 = at(ws, 16), r3 = at(ws, 24);
            const float r4 = at(ws, 32), r5 = at(ws, 40), r6 = at(ws, 48), r7 = at(ws, 56);
            const float ss = ((r0 + r4) + (r2 + r6)) + ((r1 + r5) + (r3 + r7));
            const float inv = 1.f / sqrtf(ss / (float)PR_HD + eps);
            const f32x4 w4 = *(const f32x4*)((is_q ? wq : wk) + 4 * lane);
#pragma unroll
            for (int c = 0; c < 4; ++c) y[c] = f16_sat(x[c] * inv * (1.f + w4[c]));
        }
        if (ROPE) {
            f16* sr = srow[w];
            *(f16x4*)(sr + 4 * lane) = y;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            for (int j = lane; j < half_r; j += 64) {
                const float cf = scs[j], sf = ssn[j];
                const float x0 = (float)sr[j];
                const float x1 = (float)sr[j + half_r];
                sr[j] = f16_sat(x0 * cf - x1 * sf);
                sr[j + half_r] = f16_sat(x1 * cf + x0 * sf);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            y = *(const f16x4*)(sr + 4 * lane);
            // the slice is rewritten by the wave's next row only after every
            // lane has read it back (in-order LDS within the wave)
        }
        if (NORM || ROPE) *(f16x4*)(orow + 4 * lane) = y;
        if (STORE && !is_q) {
            const f16x4 vin = *(const f16x4*)(v + ((size_t)t * n_kv_heads + h) * PR_HD + 4 * lane);
            const size_t crow = (size_t)pos * n_kv_heads + h;
            if constexpr (Q8) {
                const size_t vals = (size_t)max_pos * n_kv_heads * PR_HD;   // scales follow
                q8_store_row(y, (signed char*)kc + crow * PR_HD,
                             (f16*)((signed char*)kc + vals) + crow * 8, lane);
                q8_store_row(vin, (signed char*)vc + crow * PR_HD,
                             (f16*)((signed char*)vc + vals) + crow * 8, lane);
            } else {
                *(f16x4*)((f16*)kc + crow * PR_HD + 4 * lane) = y;
                *(f16x4*)((f16*)vc + crow * PR_HD + 4 * lane) = vin;
            }
        }
    }
}

// Small T: a row a wavefront (more workgroups to spread a decode step's few
// rows); large T: 7 rows a wavefront -- a token's 28 heads in one workgroup,
// its cos / sin computed once (measured at T = 8192: 2 rows a wave 118 us,
// 7 rows a wave 97 us, the fp64 sincos per workgroup being the difference).
// theta^(-2j / rope_dim) for j < rope_dim / 2; the last (theta, rope_dim)'s
// are kept (a mutex: callers may come from several threads).
std::mutex g_freq_mu;
float g_freq_theta = 0.f;
int g_freq_dim = 0;
RopeFreqs g_freqs;
void rope_freqs(float theta, int rope_dim, RopeFreqs& out) {
    std::lock_guard<std::mutex> lock(g_freq_mu);
    if (theta != g_freq_theta || rope_dim != g_freq_dim) {
        for (int j = 0; j < rope_dim / 2; ++j)
            g_freqs.f[j] = std::pow((double)theta, -2.0 * (double)j / (double)rope_dim);
        g_freq_theta = theta;
        g_freq_dim = rope_dim;
    }
    out = g_freqs;
}

template <int FLAGS>
int launch_prep(const f16* q, f16* qo, int q_pitch, f16* k, int k_pitch, const f16* v,
                const float* wq, const float* wk, void* kc, void* vc, int n_q_heads, int n_kv_heads,
                int pos0, int max_pos, int T, int rope_dim, float theta, float eps,
                fl_stream_t stream) {
    const int heads = n_q_heads + n_kv_heads;
    RopeFreqs freqs = {};
    if (FLAGS & 2) rope_freqs(theta, rope_dim, freqs);
    if (T < 256) {
        hipLaunchKernelGGL((attn_prep_kernel<FLAGS, 1>),
                           dim3(T, (heads + PR_WAVES - 1) / PR_WAVES), dim3(64 * PR_WAVES), 0,
                           (hipStream_t)stream, q, qo, q_pitch, k, k_pitch, v, wq, wk, kc, vc,
                           n_q_heads, n_kv_heads, pos0, max_pos, rope_dim, freqs, eps,
                           PrepRows{});
    } else {
        hipLaunchKernelGGL((attn_prep_kernel<FLAGS, 7>),
                           dim3(T, (heads + 7 * PR_WAVES - 1) / (7 * PR_WAVES)),
                           dim3(64 * PR_WAVES), 0, (hipStream_t)stream, q, qo, q_pitch, k,
                           k_pitch, v, wq, wk, kc, vc, n_q_heads, n_kv_heads, pos0, max_pos,
                           rope_dim, freqs, eps, PrepRows{});
    }
    return fl::check_launch("attn_prep");
}


bool al(const void* p, unsigned a) { return ((uintptr_t)p & (a - 1)) == 0; }

int check_prep(const void* qg, const void* k, const void* v, const float* wq, const float* wk,
               const void* kcache, const void* vcache, int q_pitch, int n_q_heads,
               int n_kv_heads, int head_dim, int pos0, int max_pos, int T, int rope_dim,
               float eps) {
    FL_REQUIRE(qg && k && v && wq && wk && kcache && vcache, "null pointer");
    FL_REQUIRE(head_dim == PR_HD, "head_dim must be 256");
    FL_REQUIRE(rope_dim > 0 && rope_dim <= head_dim && (rope_dim & 1) == 0,
               "0 < rope_dim <= head_dim, even");
    FL_REQUIRE(n_q_heads >= 1 && n_kv_heads >= 1 && n_q_heads % n_kv_heads == 0,
               "n_q_heads % n_kv_heads");
    FL_REQUIRE(T >= 1 && pos0 >= 0 && pos0 + T <= max_pos, "pos0 + T <= max_pos");
    FL_REQUIRE(q_pitch >= head_dim && eps >= 0.f, "q_pitch >= head_dim");
    FL_REQUIRE(q_pitch % 4 == 0 && al(qg, 8) && al(k, 8) && al(v, 8) && al(wq, 16) && al(wk, 16),
               "q_pitch % 4, aligned qg, k, v, weights");
    return FL_OK;
}

}  // namespace

extern "C" {

int fl_rmsnorm1p(const void* x, const float* w, void* y, int n, int rows, int pitch, int T,
                 float eps, fl_stream_t stream) {
    FL_REQUIRE(x && w && y, "null pointer");
    FL_REQUIRE(n == PR_HD, "n must be 256 (the per-head q / k norm)");
    FL_REQUIRE(rows >= 1 && T >= 1 && pitch >= n && eps >= 0.f, "rows, T >= 1, pitch >= n");
    FL_REQUIRE(pitch % 4 == 0 && al(x, 8) && al(y, 8) && al(w, 16), "pitch % 4, aligned x, y, w");
    // the rows of one tensor run as the kernel's "q" heads, none as "k"
    return launch_prep<1>((const f16*)x, (f16*)y, pitch, nullptr, 0, nullptr, w, nullptr, nullptr,
                          nullptr, rows, 0, 0, 0, T, 0, 0.f, eps, stream);
}

int fl_rope_partial(void* q, void* k, int n_q_heads, int n_kv_heads, int head_dim, int rope_dim,
                    int q_pitch, int k_pitch, int pos0, int T, float theta,
                    fl_stream_t stream) {
    FL_REQUIRE(q && k, "null pointer");
    FL_REQUIRE(head_dim == PR_HD, "head_dim must be 256");
    FL_REQUIRE(rope_dim > 0 && rope_dim <= head_dim && (rope_dim & 1) == 0,
               "0 < rope_dim <= head_dim, even");
    FL_REQUIRE(n_q_heads >= 1 && n_kv_heads >= 1 && T >= 1 && pos0 >= 0, "heads, T, pos0");
    FL_REQUIRE(q_pitch >= head_dim && k_pitch >= head_dim, "pitches");
    FL_REQUIRE(q_pitch % 4 == 0 && k_pitch % 4 == 0 && al(q, 8) && al(k, 8), "pitch % 4, aligned q, k");
    return launch_prep<2>((const f16*)q, (f16*)q, q_pitch, (f16*)k, k_pitch, nullptr, nullptr,
                          nullptr, nullptr, nullptr, n_q_heads, n_kv_heads, pos0, 0, T, rope_dim,
                          theta, 0.f, stream);
}

int fl_attn_prep(void* qg, int q_pitch, void* k, const void* v, const float* wq, const float* wk,
                 void* kcache, void* vcache, int layer, int n_q_heads, int n_kv_heads,
                 int head_dim, int pos0, int max_pos, int T, int rope_dim, float theta, float eps,
                 fl_stream_t stream) {
    int rc = check_prep(qg, k, v, wq, wk, kcache, vcache, q_pitch, n_q_heads, n_kv_heads,
                        head_dim, pos0, max_pos, T, rope_dim, eps);
    if (rc) return rc;
    FL_REQUIRE(layer >= 0 && al(kcache, 8) && al(vcache, 8), "layer >= 0, 8-byte aligned caches");
    const size_t off = (size_t)layer * max_pos * n_kv_heads * head_dim;
    return launch_prep<7>((const f16*)qg, (f16*)qg, q_pitch, (f16*)k, head_dim, (const f16*)v, wq, wk,
                          (f16*)kcache + off, (f16*)vcache + off, n_q_heads, n_kv_heads, pos0,
                          max_pos, T, rope_dim, theta, eps, stream);
}

int fl_attn_prep_q8(void* qg, int q_pitch, void* k, const void* v, const float* wq,
                    const float* wk, void* kcache, void* vcache, int layer, int n_q_heads,
                    int n_kv_heads, int head_dim, int pos0, int max_pos, int T, int rope_dim,
                    float theta, float eps, fl_stream_t stream) {
    int rc = check_prep(qg, k, v, wq, wk, kcache, vcache, q_pitch, n_q_heads, n_kv_heads,
                        head_dim, pos0, max_pos, T, rope_dim, eps);
    if (rc) return rc;
    FL_REQUIRE(layer == 0, "an int8 cache is one buffer a layer: layer must be 0");
    FL_REQUIRE(al(kcache, 4) && al(vcache, 4), "4-byte aligned caches");
    return launch_prep<15>((const f16*)qg, (f16*)qg, q_pitch, (f16*)k, head_dim, (const f16*)v, wq,
                           wk, kcache, vcache, n_q_heads, n_kv_heads, pos0, max_pos, T, rope_dim,
                           theta, eps, stream);
}

int fl_attn_prep_rows(void* qg, int q_pitch, void* k, const void* v, const float* wq,
                      const float* wk, void* const* kcaches, void* const* vcaches,
                      const int* pos, const int* max_pos, int B, int q8, int n_q_heads,
                      int n_kv_heads, int head_dim, int rope_dim, float theta, float eps,
                      fl_stream_t stream) {
    FL_REQUIRE(kcaches && vcaches && pos && max_pos, "null pointer");
    FL_REQUIRE(B >= 1 && B <= FL_MAX_SEQS, "1 <= B <= FL_MAX_SEQS");
    PrepRows rows = {};
    for (int b = 0; b < B; ++b) {
        const int rc = check_prep(qg, k, v, wq, wk, kcaches[b], vcaches[b], q_pitch, n_q_heads,
                                  n_kv_heads, head_dim, pos[b], max_pos[b], 1, rope_dim, eps);
        if (rc) return rc;
        FL_REQUIRE(q8 ? al(kcaches[b], 4) && al(vcaches[b], 4)
                      : al(kcaches[b], 8) && al(vcaches[b], 8), "aligned caches");
        rows.kc[b] = kcaches[b];
        rows.vc[b] = vcaches[b];
        rows.pos[b] = pos[b];
        rows.max_pos[b] = max_pos[b];
    }
    RopeFreqs freqs = {};
    rope_freqs(theta, rope_dim, freqs);
    const dim3 grid(B, (n_q_heads + n_kv_heads + PR_WAVES - 1) / PR_WAVES);
    if (q8)
        hipLaunchKernelGGL((attn_prep_kernel<15, 1, true>), grid, dim3(64 * PR_WAVES), 0,
                           (hipStream_t)stream, (const f16*)qg, (f16*)qg, q_pitch, (f16*)k,
                           head_dim, (const f16*)v, wq, wk, nullptr, nullptr, n_q_heads,
                           n_kv_heads, 0, 0, rope_dim, freqs, eps, rows);
    else
        hipLaunchKernelGGL((attn_prep_kernel<7, 1, true>), grid, dim3(64 * PR_WAVES), 0,
                           (hipStream_t)stream, (const f16*)qg, (f16*)qg, q_pitch, (f16*)k,
                           head_dim, (const f16*)v, wq, wk, nullptr, nullptr, n_q_heads,
                           n_kv_heads, 0, 0, rope_dim, freqs, eps, rows);
    return fl::check_launch("attn_prep_rows");
}

}  // extern "C"
