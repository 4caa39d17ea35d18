/*
 * CPU oracle for the EXL3 MoE decode path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's arithmetic (muyouming/exl3-server),
 * used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
 * the checker and the CPU baseline. Nothing in the product links or calls it:
 * the HIP library under exl3-server_amd/ is self-contained and fails loudly
 * when it is not built.
 *
 * Every function cites the reference lines it restates. Integer and byte work
 * (codebooks, ring windows, permutation, routing selection, run grouping) is
 * restated bit-for-bit; floating-point work keeps the reference's rounding
 * points (f16 RNE at the same places) and accumulates in f64 where the
 * reference's own association is an unpinned MLX/Metal internal.
 *
 * How each function is pinned (checks that a plausible mistake would fail):
 *   or_f16_from_double   exhaustive round trip over all 65536 f16 patterns,
 *                        midpoints between neighbours (ties-to-even), the
 *                        overflow/underflow edges, numpy.float16 as a second
 *                        implementation (tests/test_oracle.py)
 *   or_codebook_lut      golden hashes + samples written from the reference's
 *                        own exl3.cpp (tests/golden/), closed-form ranges
 *   or_decode_inner      golden outputs from the reference's decode_inner, and
 *                        a bit-by-bit brute-force restatement of the ring
 *                        window (or_tile_state_bruteforce)
 *   or_reconstruct       golden outputs from the reference's reconstruct, and
 *                        the Sylvester identity H.H = 128 I
 *   or_had_pre/post      explicit Sylvester-matrix products in f64 (rounding
 *                        points checked by construction on exact inputs)
 *   or_router_logits     numpy f64 h . W^T on a non-square layer, with the
 *                        transposed weight layout shown to be far off
 *   or_route             the reference test's known answers (moe_test.cpp
 *                        (a)/(b)) and brute-force subset search on tiny E
 *   or_moe_runs          hand-worked sort/run cases and the (g)/(h) geometries
 *   or_moe_layer         f64 textbook restatement on dequantised weights
 *   or_hc_prepare        column sums of the Sinkhorn output (the last normalisation)
 *                        equal 1, stream-permutation equivariance, invariance of
 *                        post/comb under scaling the streams (the RMS
 *                        normalisation), the N = 1 closed form
 *   or_rms_norm          scale invariance and unit mean square before the weight
 *   or_hc_mix            the N = 1 closed form and linearity in each input
 */
#ifndef EXL3_ORACLE_H
#define EXL3_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Codebook ids follow the reference (exl3.h:28): 0 = 3inst, 1 = mcg, 2 = mul1. */

double or_f16_to_double(uint16_t h);
uint16_t or_f16_from_double(double x);
uint16_t or_codebook_value(uint16_t state, int cb);
void or_codebook_lut(int cb, uint16_t *lut /* 65536 */);
/* GEMV weight values: mode 0 = the reference's f16 weights (default); mode 1 = for
 * mcg/3inst the exact sum of the masked hash word's two f16 halves, before the
 * reference's f16 rounding (mul1 unchanged). Affects or_matmul_raw and everything built
 * on it (linear, layer); decode/reconstruct always give the reference's bits. */
void or_set_gemv_mode(int exact_halves);
int or_get_gemv_mode(void);
float or_codebook_halves_sum(uint16_t state, int cb);

/* 16-bit state of stream position p in one tile (fast 64-bit window form and
 * a bit-by-bit form used to pin it). */
uint16_t or_tile_state(const uint16_t *tile_words, int K, int p);
uint16_t or_tile_state_bruteforce(const uint16_t *tile_words, int K, int p);
/* Stream position -> row-major element (row * 16 + col) inside a 16x16 tile. */
int or_tile_perm(int p);

/* W_hat (rotated basis) f16 row-major [in, out]. Returns 0, or -1 on bad geometry. */
int or_decode_inner(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb,
                    uint16_t *w_hat, int threads);
/* W = diag(suh) H W_hat H diag(svh) / 128, one f16 rounding. Returns 0 / -1. */
int or_reconstruct(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb,
                   const uint16_t *suh, const uint16_t *svh, uint16_t *w, int threads);

/* Hadamard steps of the trellis linear (f16 in/out, f32 butterflies). */
void or_had_pre(const uint16_t *x, int64_t rows, int64_t n, const uint16_t *suh, uint16_t *xhat);
void or_had_post(const float *yhat, int64_t rows, int64_t n, const uint16_t *svh, uint16_t *y);
void or_had_post_f64(const double *yhat, int64_t rows, int64_t n, const uint16_t *svh,
                     uint16_t *y);

/* yhat[r][n] = sum_k xhat[r][k] * W_hat[k][n], decoding on the fly, f64. */
int or_matmul_raw(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb,
                  const uint16_t *xhat, int64_t rows, double *yhat, int threads);

/* y = trellis_linear(x): had_pre -> f64 GEMV -> had_post. */
int or_trellis_linear(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb,
                      const uint16_t *suh, const uint16_t *svh, const uint16_t *x, int64_t rows,
                      uint16_t *y, int threads);

/* One linear of the layer: trellis (trellis != NULL) or plain f16 (in, out). */
typedef struct {
  const uint16_t *trellis; /* u16 words (in/16, out/16, 16K), or NULL */
  const uint16_t *suh;     /* f16 [in] */
  const uint16_t *svh;     /* f16 [out] */
  const uint16_t *dense;   /* f16 (in, out) row-major when trellis == NULL */
  int32_t in, out, K, cb;
} or_linear;

typedef struct {
  int32_t hidden, inter, n_experts, top_k, n_group, topk_group, norm_topk_prob, has_shared;
  float routed_scaling_factor, swiglu_limit;
} or_moe_cfg;

/* Router on f64 logits (N, E). Writes idx (N, top_k) in descending
 * scores-for-choice order (ties -> lower expert id) and weights (N, top_k). */
int or_route(const double *logits, const float *bias, int64_t N, const or_moe_cfg *cfg,
             int32_t *idx, double *weights);
/* logits = f32(h) . f32(router_w)^T accumulated in f64. */
void or_router_logits(const uint16_t *h, int64_t N, const uint16_t *router_w, int E, int H,
                      double *logits);

/* Expert-order dispatch (glm5_moe.cpp:158-200, 236-255): pairs sorted stably by
 * expert; perm[rank * N + row] = sorted position; runs = maximal equal-expert
 * spans. Returns the number of runs. run_expert/run_off/run_len have room for N*K. */
int or_moe_runs(const int32_t *idx, int64_t N, int K, int32_t *sorted_expert,
                int32_t *sorted_row, int32_t *sorted_rank, int32_t *perm, int32_t *run_expert,
                int32_t *run_off, int32_t *run_len);

/* The whole layer (moe_layer / moe_layer_rows semantics). experts has 3*E
 * entries (gate, up, down per expert); shared has 3 entries or is NULL.
 * Outputs f16 (N, H); optionally the routing (idx, weights as f64). */
int or_moe_layer(const or_moe_cfg *cfg, const or_linear *experts, const or_linear *shared,
                 const uint16_t *router_w, const float *bias, const uint16_t *h, int64_t N,
                 uint16_t *out, int32_t *idx_out, double *w_out, int threads);

/* The same layer with routing supplied by the caller (idx, weights), so the
 * expert arithmetic can be checked independently of near-tie selection. */
int or_moe_layer_routed(const or_moe_cfg *cfg, const or_linear *experts,
                        const or_linear *shared, const uint16_t *h, int64_t N,
                        const int32_t *idx, const double *weights, uint16_t *out, int threads);

/* ------------------------------------------------------------------------- */
/* The steps either side of the MoE in batch_step (glm5_forward.cpp:434-438):  */
/* g5_hc_prepare (glm5_hc.cpp:242-340), rms_norm (glm5_attn.cpp:12-22) and     */
/* g5_hc_mix (glm5_hc.cpp:342-355). f64 arithmetic with the reference's f16    */
/* rounding points: the collapsed stream, the normalised row before its weight */
/* multiply and after it, and the mix's product, matmul and sum.               */
/* ------------------------------------------------------------------------- */

/* streams (P, N, D) f16; fn (W, N*D) f32 with W = (2+N)*N, base (W), scale (3).
 * Outputs: collapsed (P, D) f16, post (P, N) and comb (P, N, N) in f64. */
void or_hc_prepare(const uint16_t *streams, int64_t P, int N, int D, const float *fn,
                   const float *base, const float *scale, int iters, double eps,
                   uint16_t *collapsed, double *post, double *comb);
/* y = f16(f16(x * rsqrt(mean(x^2) + eps)) * w), x (P, D) f16, w (D) f16. */
void or_rms_norm(const uint16_t *x, int64_t P, int D, const uint16_t *w, double eps, uint16_t *y);
/* out[p][n][d] = f16(f16(f16(post[p][n]) * b[p][d]) + f16(sum_m f16(comb[p][m][n]) *
 * residual[p][m][d])), all f16 (the reference runs g5_hc_mix in block_out's dtype). */
void or_hc_mix(const uint16_t *block_out, const double *post, const double *comb,
               const uint16_t *residual, int64_t P, int N, int D, uint16_t *out);

#ifdef __cplusplus
}
#endif

#endif
