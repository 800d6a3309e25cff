/*
 * ecf8_llm.h -- C ABI of the consumer kernels in libecf8.so: the
 * block-scaled FP8 linear that reads decoded weights, and the fused
 * kernels of a Qwen3-shaped decoder layer around it.
 *
 * None of these entry points replaces a reference interface one to one.
 * The reference runs its decoded weights through transformers' FP8Linear
 * (fine-grained FP8: weights e4m3fn with fp32 scales per 128x128 block,
 * activations quantized per 1x128 group, transformers
 * integrations/finegrained_fp8.py:182-350), inside the forward that
 * dfloat/run/run.py:84-155 hooks.  These kernels are that consumer on
 * gfx950, so a compressed model and its uncompressed FP8 original can be
 * run and timed end to end by one engine.
 *
 * Conventions as in ecf8.h: device pointers, stream as void*, ECF8_*
 * status, asynchronous, no allocation.  bf16 tensors are passed as void*
 * (2-byte elements); fp8 tensors are e4m3fn bytes.  All deterministic.
 */
#ifndef ECF8_LLM_H
#define ECF8_LLM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ECF8_LINEAR_MAX_SEGS 3

/*
 * FP8 operand layouts.  Quantized activations (every aq / out_q below) are
 * always in the tile layout; weights may be in either:
 *   ECF8_WEIGHT_ROWS   e4m3fn [rows, K] row-major (the checkpoint's layout,
 *                      and the decoder's output);
 *   ECF8_WEIGHT_TILES  the tile layout.
 * Tile layout of an [R, K] e4m3fn matrix (K a multiple of 128, rows padded
 * to a multiple of 16): for each 16-row tile t and 128-column group kg one
 * 2048-byte block at ((t * K/128) + kg) * 2048, in the order the lanes of
 * v_mfma_f32_16x16x32_fp8_fp8 take their operands -- lane l = 16 g + r
 * holds bytes [16 g, +16) of the tile's row r at block byte 16 l, and bytes
 * [64 + 16 g, +16) at 1024 + 16 l -- so each 16-byte load of a wave reads
 * 1 KB contiguous.  The pad rows of the last tile are never read into a
 * stored output.  Activation scales stay row-major fp32 [M, K/128].
 */
#define ECF8_WEIGHT_ROWS 0
#define ECF8_WEIGHT_TILES 1

/* One weight matrix of a (possibly fused) linear: weight e4m3fn [n, K]
 * (16-byte aligned) in weight_layout, weight_scale fp32 [n/128, K/128];
 * its outputs go to columns [out_col, out_col + n) of the output. */
typedef struct ecf8_linear_seg {
  const void *weight;
  const float *weight_scale;
  int64_t n;
  int64_t out_col;
  int64_t weight_layout; /* ECF8_WEIGHT_ROWS or ECF8_WEIGHT_TILES */
} ecf8_linear_seg;

/*
 * out[m, seg.out_col + j] (bf16, row stride ldo) =
 *   sum_g (sum_{k in g} aq[m, k] * w[j, k]) * as[m, g] * ws[j/128, g]
 * for each of n_segs (1..3) segments, e.g. q/k/v or gate/up in one launch.
 * aq: e4m3fn [M, K] in the tile layout (16-byte aligned, ceil(M/16) * 16
 * rows), as: fp32 [M, K/128].  K and every seg.n must be multiples of 128.
 */
int ecf8_fp8_linear(const void *aq, const float *as, int64_t M, int64_t K,
                    const ecf8_linear_seg *segs, int n_segs, void *out, int64_t ldo,
                    void *stream);

/*
 * Residual add + RMSNorm over rows of K = 4096 or 2048:
 *   residual[m] += x[m]  (x bf16 [M, K], or NULL for no add; residual fp32)
 *   y = residual[m] * rsqrt(mean(residual[m]^2) + eps) * weight  (bf16 weight)
 * y goes to out_bf16 (bf16 [M, K]) and/or, quantized, to out_q (e4m3fn
 * [M, K], tile layout) + out_scale (fp32 [M, K/128]); with both, the
 * quantized form is
 * that of the bf16-rounded y (what ecf8_act_quant of out_bf16 gives).
 */
int ecf8_rmsnorm(const void *x, float *residual, const void *weight, float eps, int64_t M,
                 int64_t K, void *out_q, float *out_scale, void *out_bf16, void *stream);

/* h = silu(gate) * up for gate_up bf16 [M, 2I] (gate in columns [0, I)),
 * quantized to out_q e4m3fn [M, I] (tile layout) + out_scale fp32
 * [M, I/128].
 * I must be a multiple of 128. */
int ecf8_silu_mul_quant(const void *gate_up, int64_t M, int64_t I, void *out_q,
                        float *out_scale, void *stream);

/* bf16 [M, K] -> e4m3fn (tile layout) + fp32 scale per 1x128 group
 * (scale = amax/448, 1 for an all-zero group; q =
 * round_nearest_even(x / scale)).  K must be a multiple of 128. */
int ecf8_act_quant(const void *x, int64_t M, int64_t K, void *out_q, float *out_scale,
                   void *stream);

/*
 * For the fused projection output qkv bf16 [B*T, (Hq + 2*Hkv) * 128]
 * (q heads, then k heads, then v heads), token t of sequence b at position
 * p = pos[0] + t (pos: device int32):
 *   q, k: RMSNorm over the head (bf16 weights q_norm / k_norm [128]), then
 *         the rotary embedding, rotate-half form, cos_t/sin_t fp32 [Lmax, 64];
 *   q -> q_out bf16 [B, Hq, T, 128];
 *   k, v -> k_cache / v_cache bf16 [B, Hkv, Lmax, 128] at position p.
 * Tokens whose p falls outside [0, Lmax) are skipped.
 */
int ecf8_qk_norm_rope(const void *qkv, int64_t B, int64_t T, int Hq, int Hkv, const void *q_norm,
                      const void *k_norm, float eps, const float *cos_t, const float *sin_t,
                      const int *pos, int64_t Lmax, void *q_out, void *k_cache, void *v_cache,
                      void *stream);

/* out bf16 [n, k] = weight e4m3fn [n, k] x weight_scale fp32 [n/128, k/128]
 * (per 128x128 block), rounded to nearest even: the weights of a linear
 * whose activations are too many rows for the small-M kernel, handed to a
 * library bf16 GEMM.  n and k multiples of 128. */
int ecf8_dequant_fp8_block(const void *weight, const float *weight_scale, int64_t n, int64_t k,
                           void *out, void *stream);

/* fp32 elements of the work buffer ecf8_decode_attention and
 * ecf8_decode_attention_fused need. */
int64_t ecf8_attention_work_floats(int64_t B, int Hq, int64_t Lmax);

/*
 * Attention of one new token per sequence (q bf16 [B, Hq, 128], scaled by
 * 1/sqrt(128)) over cached positions [0, pos[0]] (pos: device int32, the
 * new token's position, already written to the caches), grouped-query with
 * Hq = 4 * Hkv or 8 * Hkv.  The result per (b, head) is quantized as one 128-group:
 * out_q e4m3fn [B, Hq*128] (tile layout), out_scale fp32 [B, Hq]; out_bf16 (optional,
 * bf16 [B, Hq*128]) receives the unquantized result.
 */
int ecf8_decode_attention(const void *q, const void *k_cache, const void *v_cache, const int *pos,
                          int64_t B, int Hq, int Hkv, int64_t Lmax, float *work,
                          int64_t work_floats, void *out_q, float *out_scale, void *out_bf16,
                          void *stream);

/*
 * ecf8_qk_norm_rope (T = 1) folded into ecf8_decode_attention, with the
 * same arithmetic and results: q comes from the projection output qkv
 * bf16 [B, (Hq + 2*Hkv) * 128] through the per-head norm and rotary
 * embedding at position pos[0], and the workgroup whose split holds pos[0]
 * writes the new token's k and v to the caches before reading them.  Two
 * launches (the split kernel and the merge) instead of three.
 */
int ecf8_decode_attention_fused(const void *qkv, int64_t B, int Hq, int Hkv, const void *q_norm,
                                const void *k_norm, float eps, const float *cos_t,
                                const float *sin_t, const int *pos, int64_t Lmax, void *k_cache,
                                void *v_cache, float *work, int64_t work_floats, void *out_q,
                                float *out_scale, void *out_bf16, void *stream);

/* ---------------------------------------------------------------- MoE
 * The routed-expert MLP of a Qwen3-MoE-shaped layer
 * (transformers' Qwen3MoeSparseMoeBlock: softmax router, top-k experts,
 * weights renormalized to sum 1), whose experts are the compressed blocks
 * model.layers.N.mlp.experts.E of the reference's qwen3moe patterns
 * (dfloat/const.py:15-21).  No entry point replaces a reference interface:
 * the reference runs transformers' own MoE forward over hooked experts.
 */

/* Router: logits fp32 [M, E] (a work buffer the caller owns) = x [M, H]
 * (bf16) . router_w [E, H]^T (bf16) with fp32 products, softmax over E,
 * the top_k largest probabilities (ties to the lower expert), renormalized
 * to sum 1: topk_idx int32 [M, top_k] (descending probability), topk_w
 * fp32 [M, top_k].  Two launches.  H a multiple of 512; E <= 256;
 * top_k <= 16; M <= 65536. */
int ecf8_moe_route(const void *x, const void *router_w, int64_t M, int64_t H, int E, int top_k,
                   float *logits, int *topk_idx, float *topk_w, void *stream);

/* Group the P = M * top_k (token, expert) pairs by expert (P <= 8192,
 * E <= 256): expert e's pairs take sorted positions [offsets[e],
 * offsets[e + 1]) in token order (offsets int32 [E + 1]); pair_tok int32
 * [P] / pair_w fp32 [P]: token and weight of each sorted position;
 * pair_pos int32 [P]: sorted position of pair (m, k) at m * top_k + k;
 * active int32 [E]: the experts with pairs, increasing, n_active int32 [1]
 * of them; select (optional) int32 [E]: 1 where an expert has pairs, the
 * flags ecf8_decode_batched_select takes. */
int ecf8_moe_group(const int *topk_idx, const float *topk_w, int64_t M, int top_k, int E,
                   int *offsets, int *active, int *n_active, int *pair_tok, float *pair_w,
                   int *pair_pos, int *select, void *stream);

/* Grouped FP8 linear over the active experts (offsets / active / n_active
 * from ecf8_moe_group, all device memory):
 *   out[q, s * seg_n + j] = linear(aq[row(q)], weights[e * n_segs + s])[j]
 * for every sorted position q of expert e, with the block-scaled math of
 * ecf8_fp8_linear; row(q) = row_of[q] (e.g. pair_tok: gather the token's
 * activation row) or q when row_of is NULL (aq in the tile layout).
 * weights / weight_scales are device arrays of n_experts * n_segs
 * addresses (e4m3fn [seg_n, K] in weight_layout, and fp32 [seg_n/128,
 * K/128]); active entries must be < n_experts.  The grid covers every
 * expert and idle slots exit, so the launch can be captured in a graph.
 * Each output sums its K groups over three waves when K/128 = 6, four when
 * K/128 <= ECF8_MOE_FOUR_WAVE_GROUPS, else eight (wave w takes groups w,
 * w + waves, ...), then the waves in order. */
#define ECF8_MOE_FOUR_WAVE_GROUPS 16
int ecf8_moe_linear(const void *aq, const float *as, const int *row_of, const int *offsets,
                    const int *active, const int *n_active, int n_experts,
                    const void *const *weights, const float *const *weight_scales, int n_segs,
                    int64_t seg_n, int64_t K, int weight_layout, void *out, int64_t ldo,
                    void *stream);

/* out bf16 [M, H] = sum_k pair_w[q] * down[q, :] (down bf16, row stride
 * ldd) over q = pair_pos[m * top_k + k], k in order, accumulated in fp32. */
int ecf8_moe_combine(const void *down, int64_t ldd, const int *pair_pos, const float *pair_w,
                     int64_t M, int top_k, int64_t H, void *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* ECF8_LLM_H */
