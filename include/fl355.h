/*
 * fl355.h -- C ABI of libfl355.so, the MI355X (gfx950) implementation of the
 * footless attention / Gated DeltaNet hot path.
 *
 * Every entry point takes raw device pointers, plain integers / floats and a
 * HIP stream, enqueues its kernels on that stream and returns an int status
 * (FL_OK = 0). Where the reference kernel returned without writing on a
 * geometry it could not handle (model/footless/cuda_sm60/kernels.cu:22-28),
 * these entry points enqueue nothing and return FL_EINVAL; fl_last_error()
 * then names the argument. The caller owns every buffer (weights, caches,
 * states, scratch), as the reference's runtime does (runtime.py:886-967);
 * no entry point allocates device memory.
 *
 * Storage types: "f16" = IEEE binary16 (uint16_t bits), "f32" = float.
 * Each declaration names the reference launch it replaces: the kernel
 * (kernels.cu:line) and the runtime call site (runtime.py:line) that a
 * maintainer rebinds through a ctypes binding of this header.
 */
#ifndef FL355_H
#define FL355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* fl_stream_t; /* hipStream_t; NULL = default stream */

#define FL_OK 0
#define FL_EINVAL 1   /* geometry / argument the kernels do not support */
#define FL_ELAUNCH 2  /* the HIP runtime refused a launch */
#define FL_ESCRATCH 3 /* caller scratch smaller than *_work_bytes asked for */

#define FL_MAX_SEQS 16 /* sequences one batched decode call carries */

int fl_abi_version(void);
const char* fl_strerror(int status);
/* Detail of the last failure on the calling thread ("" if none). */
const char* fl_last_error(void);

/* ---- KV store -------------------------------------------------------------
 * kv_store: k, v [T][n_kv_heads][head_dim] f16 -> cache rows pos0 + t of a
 * position-addressable [layers][max_pos][n_kv_heads][head_dim] f16 cache.
 * Replaces kernels.cu:465-484 kv_store, launched at runtime.py:2813-2815.
 * Differs: pos0 + T > max_pos is FL_EINVAL (the reference skipped the rows). */
int fl_kv_store(const void* k, const void* v, void* kcache, void* vcache, int layer,
                int pos0, int T, int n_kv_heads, int head_dim, int max_pos,
                fl_stream_t stream);

/* ---- attention prep ---------------------------------------------------------
 * rmsnorm1p: per-row Gemma RMSNorm, y = f16(x * rsqrt(sum(x^2) / n + eps) *
 * (1 + w[i])), rows [T][rows] at `pitch` f16 apart (q: rows = n_q_heads,
 * pitch = 2 head_dim inside the q|gate buffer; k: rows = n_kv_heads, pitch =
 * head_dim); x == y (in place) allowed. The sum of squares in the reference
 * block reduction's order. Replaces kernels.cu:241-272 rmsnorm1p, launched at
 * runtime.py:2797-2801 (via _rms, runtime.py:2747-2748). Supported: n == 256. */
int fl_rmsnorm1p(const void* x, const float* w, void* y, int n, int rows, int pitch, int T,
                 float eps, fl_stream_t stream);

/* rope_partial: partial NeoX RoPE in place on q [T][n_q_heads][q_pitch] and
 * k [T][n_kv_heads][k_pitch] f16 at positions pos0 + t: pairs (j, j +
 * rope_dim / 2), j < rope_dim / 2, rotate by (pos0 + t) * theta^(-2j /
 * rope_dim), frequency, angle and sincos in fp64; dims >= rope_dim untouched.
 * Replaces kernels.cu:422-455 rope_partial, launched at runtime.py:2809-2812.
 * Supported: head_dim == 256, rope_dim even, <= head_dim. */
int fl_rope_partial(void* q, void* k, int n_q_heads, int n_kv_heads, int head_dim, int rope_dim,
                    int q_pitch, int k_pitch, int pos0, int T, float theta, fl_stream_t stream);

/* attn_prep: rmsnorm1p of q (inside qg, q_pitch) with wq and of k with wk,
 * rope_partial of both, then the roped k and v rows [T][n_kv_heads][head_dim]
 * stored at cache positions pos0 + t of `layer` -- the sequence
 * runtime.py:2797-2815 launches (rmsnorm1p x2, rope_partial, kv_store) as one
 * launch, the same values (the reference's own fused form is its int8-cache
 * attn_prep_q8, kernels.cu:837-908, runtime.py:2922-2930). q and k are
 * rewritten in place, as there. Supported: head_dim == 256. */
int fl_attn_prep(void* qg, int q_pitch, void* k, const void* v, const float* wq, const float* wk,
                 void* kcache, void* vcache, int layer, int n_q_heads, int n_kv_heads,
                 int head_dim, int pos0, int max_pos, int T, int rope_dim, float theta, float eps,
                 fl_stream_t stream);

/* ---- decode attention: split partials -------------------------------------
 * attention_split_gqa for one sequence: split-K flash-decode partials of T
 * query tokens at positions pos0..pos0+T-1 (token t attends rows
 * [0, pos0 + t]), q [T][n_q_heads][q_pitch] f16 (q = first head_dim of a
 * head's row), q head h reads kv head h / (n_q_heads / n_kv_heads).
 * Token t's split count is St = clamp((pos0+t+1) / split_rows, 1, split);
 * split s covers the 32-row tiles [nt*s/St, nt*(s+1)/St) of its nt =
 * ceil(seqlen/32) tiles; s >= St writes an empty partial (m = -1e30, d = 0).
 * Outputs pacc [T][n_q_heads][split][head_dim] f32, pm / pd
 * [T][n_q_heads][split] f32, pm in natural-log units of the scaled score
 * (the reference's partial contract, kernels.cu:93-99).
 * Replaces kernels.cu:820-835 (+ 522-680), runtime.py:2830-2837.
 * Supported: head_dim == 256, T * n_q_heads / n_kv_heads <= 32,
 * split_rows >= 32, a layer cache under 2 GiB and (max_pos / 32 + 1) *
 * (split + 1) < 2^32. */
int fl_attention_split_gqa(const void* q, const void* kcache, const void* vcache,
                           float* pacc, float* pm, float* pd, int layer, int n_q_heads,
                           int n_kv_heads, int head_dim, int q_pitch, int pos0, int max_pos,
                           float scale, int split_rows, int T, int split,
                           fl_stream_t stream);

/* ---- decode attention: merge + gate ---------------------------------------
 * attention_merge (+ attn_gate when gate != NULL): z[t][h][:] =
 * f16_sat(sum_s e_s acc_s / sum_s e_s d_s), e_s = exp(m_s - max m), then
 * z = f16_sat(z * sigmoid(gate[t][h][g_off + d])) with gate rows of g_pitch
 * per head. z is written at z_pitch per head. head_dim is a multiple of 4
 * up to 1024; pacc is 16-byte aligned.
 * Replaces kernels.cu:1398-1424 (runtime.py:2844-2846) and kernels.cu:
 * 1585-1600 (runtime.py:2860-2862); the fused form of kernels.cu:1342-1385. */
int fl_attention_merge(const float* pacc, const float* pm, const float* pd, void* z,
                       int n_q_heads, int head_dim, int z_pitch, int T, int split,
                       const void* gate, int g_pitch, int g_off, fl_stream_t stream);

/* The output gate alone: z = f16_sat(z * sigmoid(g)), kernels.cu:1585-1600. */
int fl_attn_gate(void* z, const void* g, int n_heads, int head_dim, int z_pitch,
                 int g_pitch, int g_off, int T, fl_stream_t stream);

/* ---- decode attention, batched --------------------------------------------
 * The decode / MTP-verify attention of B sequences in two launches: the
 * split partials of every (sequence, kv head, split) and the gated merge.
 * qg [B][T][n_q_heads][q_pitch] f16, q at offset 0 of a head's row and the
 * gate at g_off (gate may be NULL: no gate); kcache[b] / vcache[b] host
 * arrays of B device pointers to each sequence's layer cache
 * [cap[b]][n_kv_heads][head_dim] f16; pos0[b], cap[b] host arrays.
 * z [B][T][n_q_heads][z_pitch] f16. work: caller scratch of at least
 * fl_attn_decode_work_bytes(B, T, n_q_heads, head_dim, split) bytes.
 * A token of length len gets clamp(max(len / split_rows, min(len / 64, 32)),
 * 1, split) splits: the reference's rule (kernels.cu:535-544) with a floor of
 * 64-row splits for short contexts, up to 32 of them.
 * split_rows 0 sizes the split to the grid instead: S = floor(W / (B *
 * n_kv_heads)) (>= 1) splits a token, W the device's CU count (fp16 caches) or
 * twice it (int8), at most `split`, and at most len / 64 (>= 1) for a token
 * of length len -- faster for every batch size measured, at the price that a
 * token's values then depend on B (in the last bits: the partials' number).
 * Either way each token's values equal a T = 1 call at its own position with
 * the same B, bit for bit (runtime.py:2062-2069); with split_rows > 0 they
 * equal single-sequence calls too.
 * Replaces the per-sequence loop of runtime.py:2865-2878 / 2828-2862. */
size_t fl_attn_decode_work_bytes(int B, int T, int n_q_heads, int head_dim, int split);
int fl_attn_decode(const void* qg, int q_pitch, const void* const* kcache,
                   const void* const* vcache, const int* pos0, const int* cap, int B, int T,
                   int n_q_heads, int n_kv_heads, int head_dim, float scale, int split_rows,
                   int split, const void* gate, int g_pitch, int g_off, void* z, int z_pitch,
                   void* work, size_t work_bytes, fl_stream_t stream);

/* ---- prefill attention ----------------------------------------------------
 * Causal GQA prefill attention of T tokens at pos0.. over one layer cache
 * [max_pos][n_kv_heads][head_dim] f16: query (t, h) attends rows
 * [0, pos0 + t] of kv head h / G, z [T][n_q_heads][z_pitch] f16.
 * k_new / v_new [T][n_kv_heads][head_dim] f16, when not NULL, are first
 * stored into cache rows pos0.. (the fused kv_store).
 * Replaces kernels.cu:2768-2807 attention_prefill_fh (+ merge_fh) launched
 * by runtime.py:2943-2959 (and kv_store at runtime.py:2813-2815).
 * `scale` multiplies q.k (the reference passes sl2 = scale * log2 e).
 * Supported: head_dim == 256, pos0 + T <= max_pos. */
int fl_attention_prefill(const void* q, int q_pitch, const void* k_new, const void* v_new,
                         void* kcache, void* vcache, int layer, int n_q_heads, int n_kv_heads,
                         int head_dim, int pos0, int max_pos, float scale, int T, void* z,
                         int z_pitch, fl_stream_t stream);

/* Long fp16 prefills (the 256-row-workgroup kernel) launch one workgroup a CU,
 * each walking a host-balanced list of 256-row tiles of one kv head. The plan
 * for n_cu CUs: out[0 .. bins] = offsets of each bin's list in the row-tile
 * indices at out[bins + 1 ..] (bins = n_cu / n_kv_heads; bin b runs on the
 * workgroups whose XCD serves kv head b / (n_cu / n_kv_heads)). Returns the
 * entries (bins + 1 + row tiles; at most `cap` written), 0 where the call
 * launches a grid of row tiles x kv heads instead. No reference counterpart:
 * a query of this library's launch, for tests and tuning. */
int fl_attention_prefill_plan(int T, int pos0, int n_q_heads, int n_kv_heads, int n_cu,
                              unsigned short* out, int cap);

/* ---- int8 KV cache --------------------------------------------------------
 * The reference's int8 cache format (kernels.cu:486-520, runtime.py:119-132),
 * one buffer a layer and K / V: for capacity max_pos, the values
 * [max_pos][n_kv_heads][256] int8, then the scales [max_pos][n_kv_heads][8]
 * f16 at byte max_pos * n_kv_heads * 256 (256 + 16 bytes a position and kv
 * head; 1088 for the model's 4 kv heads). A 32-dim block shares the scale
 * f16(absmax / 127) and stores rint(x / scale) clamped to [-127, 127], 0 where
 * the scale is 0. `layer` must be 0 (one buffer a layer), head_dim 256.
 * The attention entry points read fp16(byte * scale) -- one rounding of the
 * product, where the reference's decode kept it in fp32. */

/* kv_store_q8: k, v [T][n_kv_heads][256] f16 into positions pos0 + t.
 * Replaces kernels.cu:486-520 kv_store_q8, launched at runtime.py:2813-2815,
 * 2895-2897, 3247-3249. Differs: pos0 + T > max_pos is FL_EINVAL. */
int fl_kv_store_q8(const void* k, const void* v, void* kcache, void* vcache, int layer,
                   int pos0, int T, int n_kv_heads, int head_dim, int max_pos,
                   fl_stream_t stream);

/* attn_prep_q8: fl_attn_prep with the int8 store -- q / k norms, rope and
 * kv_store_q8 in one launch, the same values as the separate steps.
 * Replaces kernels.cu:837-908 attn_prep_q8, launched at runtime.py:2922-2930. */
int fl_attn_prep_q8(void* qg, int q_pitch, void* k, const void* v, const float* wq,
                    const float* wk, void* kcache, void* vcache, int layer, int n_q_heads,
                    int n_kv_heads, int head_dim, int pos0, int max_pos, int T, int rope_dim,
                    float theta, float eps, fl_stream_t stream);

/* The prep of a batched decode step's B rows (T = 1 each), every row into its
 * own sequence's cache: row b of qg [B][n_q_heads][q_pitch], k / v
 * [B][n_kv_heads][head_dim] goes to kcaches[b] / vcaches[b] (host arrays of
 * device pointers; capacity max_pos[b]) at position pos[b], fp16 caches
 * ([max_pos][n_kv_heads][head_dim], layer 0) or, with q8, the int8 format --
 * the same values fl_attn_prep / fl_attn_prep_q8 give each row alone, in one
 * launch. Replaces the per-row _attn_prep calls of _full_attn_rows
 * (runtime.py:2873-2876). B <= FL_MAX_SEQS. */
int fl_attn_prep_rows(void* qg, int q_pitch, void* k, const void* v, const float* wq,
                      const float* wk, void* const* kcaches, void* const* vcaches,
                      const int* pos, const int* max_pos, int B, int q8, int n_q_heads,
                      int n_kv_heads, int head_dim, int rope_dim, float theta, float eps,
                      fl_stream_t stream);

/* attention_split_gqa_q8: fl_attention_split_gqa over an int8 cache (the same
 * split rule and partials). Replaces kernels.cu:910-1047, launched at
 * runtime.py:2832-2837 with KV8. */
int fl_attention_split_gqa_q8(const void* q, const void* kcache, const void* vcache,
                              float* pacc, float* pm, float* pd, int layer, int n_q_heads,
                              int n_kv_heads, int head_dim, int q_pitch, int pos0, int max_pos,
                              float scale, int split_rows, int T, int split,
                              fl_stream_t stream);

/* attention_dec_q8: decode partials of T tokens at pos0.. over an int8 cache.
 * Token t (length len = pos0 + t + 1) has nkt = ceil(len / 64) tiles of 64
 * rows and St = min(smax, ceil(nkt / tmin)) splits; split s covers tiles
 * [nkt*s/St, nkt*(s+1)/St). Writes pacc [T][n_q_heads][smax][256] f32,
 * pm / pd [T][n_q_heads][smax] f32 for s < St only, pm in log2 units
 * (sl2 = scale * log2 e multiplies q.k). Each token's partials equal the
 * T = 1 call's at its position, bit for bit.
 * Replaces kernels.cu:1049-1335 attention_dec_q8, runtime.py:2907-2916.
 * Supported: head_dim 256, T * n_q_heads / n_kv_heads <= 32. */
int fl_attention_dec_q8(const void* q, const void* kcache, const void* vcache, float* pacc,
                        float* pm, float* pd, int n_q_heads, int n_kv_heads, int q_pitch,
                        int pos0, int max_pos, float sl2, int tmin, int smax, int T,
                        fl_stream_t stream);

/* attention_dec_merge (+ gate when gate != NULL): z = f16_sat(sum_s 2^(m_s -
 * M) acc_s / sum_s 2^(m_s - M) d_s) over token t's first St partials, then
 * z = f16_sat(z * sigmoid(gate[t][h][g_off + d])). z [T][n_q_heads][z_pitch].
 * pacc 16-byte aligned. Replaces kernels.cu:1336-1385 attention_dec_merge /
 * _gate, runtime.py:2917-2920. */
int fl_attention_dec_merge(const float* pacc, const float* pm, const float* pd, void* z,
                           int n_q_heads, int z_pitch, int pos0, int tmin, int smax, int T,
                           const void* gate, int g_pitch, int g_off, fl_stream_t stream);

/* fl_attn_decode over int8 caches of capacities cap[b] (same arguments, work
 * from fl_attn_decode_work_bytes). Replaces the per-sequence _attn_dec loop of
 * runtime.py:2865-2878 (the batched _step_rows path, runtime.py:1784-1860). */
int fl_attn_decode_q8(const void* qg, int q_pitch, const void* const* kcache,
                      const void* const* vcache, const int* pos0, const int* cap, int B, int T,
                      int n_q_heads, int n_kv_heads, int head_dim, float scale, int split_rows,
                      int split, const void* gate, int g_pitch, int g_off, void* z, int z_pitch,
                      void* work, size_t work_bytes, fl_stream_t stream);

/* fl_attn_decode without a work buffer: the partials live in a static device
 * array of fl_attn_decode_noalloc_max_bytes() (32 MiB) bytes per GPU, so the
 * call allocates nothing (no hipMalloc / hipFree, no allocating library
 * routine). No counterpart in the reference: it is for callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation. Refuses (FL_ESCRATCH) a call whose
 * fl_attn_decode_work_bytes(B, T, n_q_heads, head_dim, split) exceeds the
 * array; B = 4, T = 3, 24 heads, 64 splits take 19 MB. Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU race. */
int fl_attn_decode_noalloc(const void* qg, int q_pitch, const void* const* kcache,
                           const void* const* vcache, const int* pos0, const int* cap, int B,
                           int T, int n_q_heads, int n_kv_heads, int head_dim, float scale,
                           int split_rows, int split, const void* gate, int g_pitch, int g_off,
                           void* z, int z_pitch, fl_stream_t stream);
size_t fl_attn_decode_noalloc_max_bytes(void);

/* The prefill with a KV split (attention_prefill_fh with gridDim.z = S and
 * attention_merge_fh, kernels.cu:2461-2486 / 2763 / 2788-2807; split chosen by
 * _fh_split, runtime.py:2932-2959): split s of every workgroup walks a share
 * of its causal KV tiles and leaves partials in `work` (the reference's `pt`
 * arena: pacc [T][n_q_heads][S][head_dim], pm (natural log) and pd
 * [T][n_q_heads][S], f32); one merge writes z. For calls whose workgroups
 * are too few to fill the CUs -- a 1024-token chunk deep into a long prompt
 * (runtime.py:196): the 64-rows-a-wave kernel splits from 64 workgroups of
 * 256 rows and 16384 cache rows (fp16 caches), the 128-row kernel otherwise
 * and over int8 caches.
 * split 0: fl_attention_prefill_split_count's choice; split 1:
 * fl_attention_prefill (no work needed). */
int fl_attention_prefill_split_count(int T, int pos0, int n_q_heads, int n_kv_heads);
/* The same choice for an int8 cache (_fh_split's role for
 * attention_prefill_fh_q8, runtime.py:2932-2941): always the 128-row int8
 * kernel's split, what fl_attention_prefill_kv_q8 takes for split 0. */
int fl_attention_prefill_split_count_q8(int T, int pos0, int n_q_heads, int n_kv_heads);
size_t fl_attention_prefill_work_bytes(int T, int n_q_heads, int head_dim, int split);
int fl_attention_prefill_kv(const void* q, int q_pitch, const void* k_new, const void* v_new,
                            void* kcache, void* vcache, int layer, int n_q_heads, int n_kv_heads,
                            int head_dim, int pos0, int max_pos, float scale, int T, int split,
                            void* z, int z_pitch, void* work, size_t work_bytes,
                            fl_stream_t stream);
/* ... over an int8 cache (attention_prefill_fh_q8, kernels.cu:2778-2786).
 * With split 1 and `work` of at least fl_attention_prefill_q8_stage_bytes
 * bytes (nonzero for long prompts), the rows [0, pos0 + T) are first
 * converted to fp16 (byte * scale, the values the int8 kernel forms) into
 * `work`, and the long-prompt fp16 kernel runs on that copy. */
size_t fl_attention_prefill_q8_stage_bytes(int T, int pos0, int n_q_heads, int n_kv_heads,
                                           int head_dim);
int fl_attention_prefill_kv_q8(const void* q, int q_pitch, const void* k_new, const void* v_new,
                               void* kcache, void* vcache, int layer, int n_q_heads,
                               int n_kv_heads, int head_dim, int pos0, int max_pos, float scale,
                               int T, int split, void* z, int z_pitch, void* work,
                               size_t work_bytes, fl_stream_t stream);
/* A prefill chunk's attention output as the layer uses it: the prefill
 * (fl_attention_prefill_kv, or fl_attention_prefill_kv_q8 when q8 != 0; split
 * 0 takes that cache's split count) followed by attn_gate, z = f16_sat(z *
 * sigmoid(gate)), the gate being the second half of each head's q row (q |
 * gate rows of q_pitch >= 2*head_dim halves, the reference's qg buffer).
 * When the KV is split the gate rides in the merge (one launch fewer); the
 * values are the pair's bit for bit. Replaces the sequence _attn_fh then
 * attn_gate, runtime.py:2943-2959 then 2860-2862 (kernels.cu:2461-2807,
 * 1585-1600). */
int fl_attention_prefill_gated(const void* q, int q_pitch, const void* k_new, const void* v_new,
                               void* kcache, void* vcache, int layer, int q8, int n_q_heads,
                               int n_kv_heads, int head_dim, int pos0, int max_pos, float scale,
                               int T, int split, void* z, int z_pitch, void* work,
                               size_t work_bytes, fl_stream_t stream);

/* fl_attention_prefill over an int8 cache (k_new / v_new, when given, are
 * stored first with kv_store_q8). Replaces kernels.cu:2778-2786
 * attention_prefill_fh_q8 (+ merge_fh), launched by runtime.py:2943-2959. */
int fl_attention_prefill_q8(const void* q, int q_pitch, const void* k_new, const void* v_new,
                            void* kcache, void* vcache, int layer, int n_q_heads,
                            int n_kv_heads, int head_dim, int pos0, int max_pos, float scale,
                            int T, void* z, int z_pitch, fl_stream_t stream);

/* ---- causal conv ----------------------------------------------------------
 * conv1d_causal over `dim` channels of rows x [T][row_stride] f16: E =
 * [st_in (width-1 frames, ZERO if pos0 == 0) | x], y[t][d] =
 * f16_sat(silu(sum_j w[d][j] E[t+j])), st_out = last width-1 frames of E.
 * w [dim][width] f16, states [dim][width-1] f16; st_in != st_out; y must not
 * overlap x; 1 <= width <= 8. 16-byte loads and stores when dim and
 * row_stride are multiples of 8 and every buffer is 16-byte aligned.
 * Replaces kernels.cu:1634-1679, runtime.py:3035-3038. */
int fl_conv1d_causal(const void* x, const void* w, const void* st_in, void* y, void* st_out,
                     int dim, int T, int pos0, int row_stride, int width, fl_stream_t stream);

/* conv1d_causal_rows: T <= 3 verify rows, the state after row t into st_t
 * (st0 may be st_in). Replaces kernels.cu:1686-1714, runtime.py:3021-3026. */
int fl_conv1d_causal_rows(const void* x, const void* w, const void* st_in, void* y, void* st0,
                          void* st1, void* st2, int dim, int T, int pos0, int row_stride,
                          fl_stream_t stream);

/* ---- L2 norm --------------------------------------------------------------
 * l2norm_scaled: y = f16_sat((x / sqrt(sum x^2 + eps)) * scale) per row of n
 * (n <= 1024), rows [T][rows][pitch] f16.
 * Replaces kernels.cu:373-391, runtime.py:3070-3071. */
int fl_l2norm_scaled(const void* x, void* y, int n, int rows, int pitch, float eps, float scale,
                     int T, fl_stream_t stream);
/* No counterpart in the reference: l2norm_scaled (n = 128) over the first
 * `rows` rows of each token, token t's rows starting at t * token_stride
 * elements -- for callers that need only some of a token's rows (the GDN
 * prefill reads back q and k, 32 of the 80 head-sized rows the reference
 * normalises, runtime.py:3068-3072). The same bits as fl_l2norm_scaled for
 * those rows; the others are not touched. pitch and token_stride multiples
 * of 8, x / y 16-byte aligned. */
int fl_l2norm_scaled_strided(const void* x, void* y, int rows, int pitch, long long token_stride,
                             float eps, float scale, int T, fl_stream_t stream);

/* ---- GDN gates ------------------------------------------------------------
 * gdn_scalars: beta = sigmoid(b), decay = exp(-exp(A_log[h]) *
 * softplus(a + dt_bias[h])), softplus threshold 20. a, b [T][stride] f32;
 * beta, decay [T][n_heads] f32. Replaces kernels.cu:1732-1748,
 * runtime.py:3072-3076. */
int fl_gdn_scalars(const float* a, const float* b, const float* A_log, const float* dt_bias,
                   float* beta, float* decay, int T, int n_heads, int a_stride, int b_stride,
                   fl_stream_t stream);

/* ---- GDN recurrent scan ---------------------------------------------------
 * The gated delta rule over T tokens, S [n_vheads][V][K] f32 in place:
 *   S *= decay; m = S k; delta = beta (v - m); S += delta k^T;
 *   y = f16_sat((S q) * out_scale)
 * q, k rows at qk_stride (head hk at hk*K), v at v_stride, y at y_stride;
 * v-head hv reads q/k head hv / group. Ck (nullable): the state after every
 * token but the last at Ck + t*ck_step floats.
 * Replaces kernels.cu:2831-2914 gdn_scan_rows (runtime.py:3094-3100) and
 * kernels.cu:1794-1901 gdn_scan (runtime.py:3102-3108). K == 128, V % 8 == 0,
 * q and k 8-byte aligned with qk_stride % 4 == 0. */
int fl_gdn_scan(const void* q, const void* k, const void* v, const float* beta,
                const float* decay, float* S, void* y, int T, int n_kheads, int n_vheads,
                int K, int V, int qk_stride, int v_stride, int y_stride, float out_scale,
                int group, float* Ck, long long ck_step, fl_stream_t stream);

/* ---- GDN fused decode / verify --------------------------------------------
 * The fused GDN decode / verify step of B sequences (T <= 3): the gates
 * (gdn_scalars), the L2 norm of q and k (l2norm_scaled, eps l2eps, fp16-rounded, scale 1),
 * and the delta rule (gdn_scan_rows) with checkpoints, in one launch. With
 * conv_fused = 1 (T == 1 only) x is the RAW q|k|v projection row and the
 * conv (conv1d_causal, width 4) runs in the kernel from cst_in[b] into cst_out[b]
 * (distinct buffers); with conv_fused = 0 x is the conv output.
 * x [B][T][x_stride] f16 with q at channel 0, k at n_kheads*K, v at
 * 2*n_kheads*K; conv_w [x channels][4] f16; a, b [B][T][ab_stride] f32;
 * A_log, dt_bias [n_vheads] f32; S[b] [n_vheads][V][K] f32 in place;
 * y [B][T][y_stride] f16; Ck[b] (nullable) as in fl_gdn_scan. Host arrays
 * S, cst_in, cst_out, Ck, pos0 hold one entry per sequence.
 * Replaces kernels.cu:2954-3070 gdn_scan_rows_f (+ gdn_conv1 2916-2941),
 * runtime.py:3040-3053 and the per-row loop runtime.py:3131-3142.
 * K == 128, V % 32 == 0, B <= FL_MAX_SEQS. */
int fl_gdn_decode(const void* x, int x_stride, int conv_fused, const void* conv_w,
                  const void* const* cst_in, void* const* cst_out, const int* pos0,
                  const float* a, const float* b, int ab_stride, const float* A_log,
                  const float* dt_bias, float* const* S, void* y, int y_stride,
                  float* const* Ck, long long ck_step, int B, int T, int n_kheads,
                  int n_vheads, int K, int V, float out_scale, float l2eps,
                  fl_stream_t stream);

/* ---- GDN output norm ----------------------------------------------------------
 * rmsnorm_gated: y = f16((o * rsqrt(sum(o^2) / n + eps) * w) * silu(z)) over
 * rows [T][rows] of `pitch` halves (o, z, y alike), w [n] f32 shared by every
 * row -- plain gamma, the norm over o before the gate. silu's exp is the
 * deterministic one the GDN kernels use. Replaces kernels.cu:335-358
 * rmsnorm_gated, launched at runtime.py:3063-3065 and 3109-3111.
 * Supported: n == 128. */
int fl_rmsnorm_gated(const void* o, const void* z, const float* w, void* y, int n, int rows,
                     int pitch, int T, float eps, fl_stream_t stream);

/* ---- GDN decode / verify step with its output norm --------------------------
 * fl_gdn_decode (T <= 3 rows a sequence; conv_fused = 1 at T == 1, else x is
 * the conv output and Ck receives the per-row checkpoints) followed by
 * fl_rmsnorm_gated over every output row, in one launch: y[b][t] =
 * rmsnorm_gated(the step's output row, z[b][t], norm_w), bit for bit the
 * pair's values; the step's own fp16 output is not written. z [B][T][z_pitch]
 * f16 (the gate, head hv at hv*V), y [B][T][y_pitch] f16; the other arguments
 * as fl_gdn_decode's (cst_in / cst_out and conv_w only read when conv_fused).
 * Replaces the pair kernels.cu:2954-3070 gdn_scan_rows_f (+ gdn_conv1
 * 2916-2941) then kernels.cu:335-358 rmsnorm_gated as a decode step or a
 * verify round runs them (runtime.py:3040-3053 / 3131-3142, then 3063-3065 /
 * 3143-3145). One workgroup a (sequence, v head): the pair is faster where B
 * is small and T > 1 (one sequence's verify rows: 14.3 against 13.2 us a
 * layer with the conv rows), the one launch where B * n_vheads workgroups
 * fill the CUs or T == 1 (B = 1..8 decode steps: 5.0 against 6.0 .. 11.7
 * against 13.3 us). K == V == 128, B <= FL_MAX_SEQS; z and y 4-byte aligned,
 * even pitches, norm_w 8-byte aligned. */
int fl_gdn_decode_normed(const void* x, int x_stride, int conv_fused, const void* conv_w,
                         const void* const* cst_in, void* const* cst_out, const int* pos0,
                         const float* a, const float* b, int ab_stride, const float* A_log,
                         const float* dt_bias, float* const* S, float* const* Ck,
                         long long ck_step, const void* z, int z_pitch, const float* norm_w,
                         void* y, int y_pitch, int B, int T, int n_kheads, int n_vheads, int K,
                         int V, float out_scale, float l2eps, float norm_eps,
                         fl_stream_t stream);

/* ---- GDN chunked prefill --------------------------------------------------
 * Chunked (WY / UT transform) GDN prefill: the same recurrence as
 * fl_gdn_scan over T tokens in chunks of `chunk` tokens, fp32 state carried
 * between chunks; S in place, y as fl_gdn_scan. NOT in the reference (the
 * reference runs gdn_scan sequentially and names the chunked scan as undone,
 * kernels.cu:1788-1791); it replaces that call (runtime.py:3094-3100) for
 * prefill. work: caller scratch of fl_gdn_chunked_work_bytes(...) bytes (per
 * chunk and v head 25,600: T = (I + A)^-1 and the decayed Q K^T of the WY form
 * as fp16 hi / lo MFMA operands of their nonzero blocks, and the gates). chunk == 64, K == V == 128; q, k, v, S,
 * work and the rows of y (y_stride % 8 == 0) 16-byte aligned. */
size_t fl_gdn_chunked_work_bytes(int T, int n_vheads, int K, int V, int chunk);
int fl_gdn_prefill_chunked(const void* q, const void* k, const void* v, const float* beta,
                           const float* decay, float* S, void* y, int T, int n_kheads,
                           int n_vheads, int K, int V, int qk_stride, int v_stride,
                           int y_stride, float out_scale, int group, int chunk, void* work,
                           size_t work_bytes, fl_stream_t stream);
/* fl_gdn_prefill_chunked with the gates formed from their logits inside it:
 * beta = sigmoid(b), decay = exp(-e^A_log softplus(a + dt_bias)), the values
 * fl_gdn_scalars writes, so the pair gdn_scalars then the scan
 * (runtime.py:3072-3076, 3094-3100) is one call and no beta / decay buffers:
 * a, b [T][ab_stride] f32 (head hv at hv), A_log, dt_bias [n_vheads] f32;
 * the rest as fl_gdn_prefill_chunked. The same values bit for bit. */
int fl_gdn_prefill_chunked_logits(const void* q, const void* k, const void* v, const float* a,
                                  const float* b, int ab_stride, const float* A_log,
                                  const float* dt_bias, float* S, void* y, int T, int n_kheads,
                                  int n_vheads, int K, int V, int qk_stride, int v_stride,
                                  int y_stride, float out_scale, int group, int chunk, void* work,
                                  size_t work_bytes, fl_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FL355_H */
