/*
 * exl3_moe.h -- C ABI of the MI355X (gfx950) EXL3 trellis / GLM-5 MoE decode library.
 *
 * Drop-in boundary for the reference's trellis_gemm.h / glm5_moe.h call surface
 * (muyouming/exl3-server): the same EXL3 tensors (.trellis words, .suh/.svh f16
 * scales, K bits, codebook) and the same (rows, hidden) f16 activations in, the same
 * f16 results out. Plain pointers and sizes only; every device pointer is caller-owned
 * HIP device memory; every call is asynchronous on the given stream (a hipStream_t,
 * NULL = the default stream) unless stated otherwise.
 *
 * Errors: every entry point returns an exl3_status; exl3_last_error() describes the
 * last failure on the calling thread. Nothing is thrown across the ABI. Shape and
 * geometry errors are detected on the host before any kernel is launched.
 *
 * Threading: calls are thread-safe for distinct streams, also on one handle from
 * several threads. A workspace must not be used by two in-flight calls at once (it
 * holds that call's routing, dispatch table and intermediate activations).
 */
#ifndef EXL3_MOE_H
#define EXL3_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *exl3_stream_t; /* hipStream_t */

typedef enum {
  EXL3_OK = 0,
  EXL3_ERR_INVALID = 1,     /* bad argument, shape or geometry */
  EXL3_ERR_UNSUPPORTED = 2, /* valid input outside what this build implements */
  EXL3_ERR_WORKSPACE = 3,   /* workspace missing or smaller than the size query */
  EXL3_ERR_HIP = 4,         /* a HIP runtime call failed */
} exl3_status;

/* Codebook ids as the reference (exl3.h:28; loader glm5.cpp:303). */
typedef enum { EXL3_CB_3INST = 0, EXL3_CB_MCG = 1, EXL3_CB_MUL1 = 2 } exl3_codebook;

/* One EXL3 trellis tensor. Replaces TrellisWeight (trellis_gemm.h:21-48).
 * `trellis` is the on-disk (in/16, out/16, 16*K) int16 array as bytes: tile
 * (tk, tn) starts at byte (tk*(out/16) + tn)*32*K and holds 8*K little-endian
 * 32-bit ring words. The base must be 4-byte aligned (the reference's unaligned
 * byte path, trellis_gemm.cpp:311-316, is a loader concern: use exl3_trellis_pack).
 * in/out must be multiples of 128 (Hadamard blocks); 1 <= K <= 8. */
typedef struct {
  const void *trellis;  /* device */
  const uint16_t *suh;  /* device f16 [in_features] */
  const uint16_t *svh;  /* device f16 [out_features] */
  int32_t in_features;
  int32_t out_features;
  int32_t K;
  int32_t codebook;     /* exl3_codebook */
} exl3_trellis_desc;

/* A linear of the MoE: trellis, or plain f16 (in, out) row-major when dense != NULL.
 * Replaces G5Linear (glm5.h:41-49; biases are not used by the MoE). */
typedef struct {
  exl3_trellis_desc tw;    /* used when dense == NULL */
  const uint16_t *dense;   /* device f16 (in_features, out_features) or NULL */
  int32_t in_features;
  int32_t out_features;
} exl3_linear_desc;

/* MoE fields of ModelConfig (model.h:47-53, 68-69; parsed model.cpp:138-144,160-161). */
typedef struct {
  int32_t hidden_size;
  int32_t moe_intermediate_size;
  int32_t n_routed_experts;
  int32_t num_experts_per_tok;
  int32_t n_group;          /* routing groups (1 = none) */
  int32_t topk_group;       /* groups kept */
  int32_t norm_topk_prob;   /* bool */
  float routed_scaling_factor;
  float swiglu_limit;       /* gate <= L, up in [-L, L] before SwiGLU, always (L = f16 of
                               this; as glm5_moe.cpp:70-71, a limit of 0 zeroes it) */
} exl3_moe_config;

/* The MoE weights of one layer. Replaces G5Layer's MoE members (glm5.h:104-110):
 * experts[3*e + {0,1,2}] = gate, up, down of expert e (host array of descriptors
 * pointing at device tensors), shared[0..2] = shared expert gate/up/down or NULL,
 * router_w = gate.weight (E, hidden) f16, router_bias = e_score_correction_bias (E) f32. */
typedef struct {
  const exl3_linear_desc *experts;  /* host array, 3 * n_routed_experts entries */
  const exl3_linear_desc *shared;   /* host array of 3, or NULL */
  const uint16_t *router_w;         /* device f16 (E, hidden) */
  const float *router_bias;         /* device f32 (E) */
} exl3_moe_layer_desc;

/* The weights an mcg/3inst GEMV multiplies (exl3_tuning.weight_form). A weight of these
 * codebooks is the sum of the two f16 halves of its masked hash word (exl3.cpp:36-42).
 * mul1 has one form (one f16 fma per weight, trellis_gemm.cpp:336-345). */
typedef enum {
  /* Default. Each weight rounded to f16 once, half(lo + hi), exactly the value the
   * reference's QMV multiplies (trellis_gemm.cpp:348-356) and the bits of
   * exl3_trellis_decode. */
  EXL3_FORM_REFERENCE = 0,
  /* Opt-in. x*lo + x*hi summed in f32, without the f16 rounding of lo + hi: one VALU
   * instruction per weight less and twice the MFMAs. Outputs differ from the reference's
   * by the weights' f16 rounding (at most 2^-11 of each weight); a SwiGLU clamp that
   * cuts large gate/up outputs can amplify that to percents of the output RMS. */
  EXL3_FORM_HALVES = 1
} exl3_weight_form;

/* Scheduling knobs. Mirrors TrellisTuning (trellis_gemm.h:137-145): rows_per_pass is
 * the linear's token rows per MFMA pass (the reference's mb; 1..16), mat_min_rows and
 * mat_max_rows the reference's staged-path window (0 = off / no cap), reported by
 * exl3_trellis_path_info. Every pass runs on the matrix cores here, so the staged
 * window only labels calls. None of these three changes an output bit (the k-split
 * partition is a function of the tensor shape only). weight_form (no counterpart in
 * the reference, whose Metal QMV has the reference form only) selects the mcg/3inst
 * weights: EXL3_FORM_REFERENCE (0, the default) or EXL3_FORM_HALVES. */
typedef struct {
  int32_t rows_per_pass;  /* 0 = auto: min(rows, 16), one MFMA pass */
  int32_t mat_min_rows;   /* calls of >= this many rows count as staged (default 16) */
  int32_t mat_max_rows;   /* 0 = no cap */
  int32_t weight_form;    /* exl3_weight_form */
} exl3_tuning;

/* What a trellis linear at `rows` rows will do. Mirrors TrellisPathInfo
 * (trellis_gemm.h:154-162). passes = weight streams per call. */
typedef struct {
  int32_t staged;
  int32_t rows_per_block;
  int32_t pad_rows;
  int32_t passes;
  int32_t splits;
  int32_t tiles_per_workgroup;
} exl3_path_info;

/* Per-layer dispatch statistics. Mirrors MoeRowsDiag (glm5_moe.h:112-122) plus the
 * run-length histogram the reference prints under EXL3_MOE_RUNS_DEBUG
 * (glm5_moe.cpp:288-295). Collected only while enabled (it synchronises the stream
 * after each layer call to read the device-side run table). */
typedef struct {
  int64_t calls;
  int64_t pairs;
  int64_t runs;
  int64_t distinct_experts;
  int64_t staged_runs;
  int64_t streamed_bytes;
  int64_t shared_bytes;
  int64_t run_hist[65];  /* run_hist[r] = runs of r rows (r >= 64 counted at 64) */
} exl3_moe_diag;

/* Per-stage GPU time of the layer calls made while timing is enabled (HIP events on
 * the call's stream around each stage; the call synchronises its stream at the end).
 * The counterpart of the reference's Glm5Profile / moe_bench stage timing
 * (glm5_forward.h:53-66, moe_bench.cpp:444-462). Bytes are the EXL3 trellis bytes of
 * the distinct experts each call streamed (each expert counted once per call). */
typedef struct {
  int64_t calls;
  double router_ms;     /* logits + top-k routing + expert-order dispatch */
  double gate_up_ms;    /* (input rotation +) routed gate|up (+ f16 shared gate/up) */
  double down_ms;       /* routed SwiGLU + down (+ f16 shared SwiGLU and down) */
  double combine_ms;    /* (a trellis shared expert on the caller's stream +) combine */
  double total_ms;
  int64_t gate_up_trellis_bytes;
  int64_t down_trellis_bytes;
} exl3_moe_timing;

typedef struct exl3_moe_layer_s *exl3_moe_layer_t;

/* ---- library ------------------------------------------------------------------ */

const char *exl3_last_error(void);
/* Version of this ABI (bumped on any incompatible change). */
int32_t exl3_abi_version(void);

/* Replaces trellis_set_tuning / trellis_get_tuning (trellis_gemm.h:144-145). */
exl3_status exl3_set_tuning(const exl3_tuning *t);
exl3_status exl3_get_tuning(exl3_tuning *t);
/* Replaces trellis_path_info (trellis_gemm.h:162). */
exl3_status exl3_trellis_path_info(const exl3_trellis_desc *w, int64_t rows,
                                   exl3_path_info *info);

/* ---- single trellis tensor ---------------------------------------------------- */

/* Copy on-disk words (host, (k_tiles, n_tiles, 16K) int16) to a 4-byte-aligned device
 * buffer of k_tiles*n_tiles*32*K bytes. Replaces trellis_pack (trellis_gemm.h:64). */
exl3_status exl3_trellis_pack(const uint16_t *words16_host, int32_t k_tiles, int32_t n_tiles,
                              int32_t K, void *dst_device, exl3_stream_t stream);

/* W_hat, the decoded rotated-basis weight, f16 row-major [in, out]. Bit-exact with
 * exl3::decode_inner (exl3.h:44; exl3.cpp:109-125). Only needs in/out % 16 == 0. */
exl3_status exl3_trellis_decode(const exl3_trellis_desc *w, uint16_t *w_hat,
                                exl3_stream_t stream);

/* W = diag(suh) H W_hat H diag(svh) / 128, f16 [in, out]. Bit-exact with
 * exl3::reconstruct (exl3.h:48; exl3.cpp:152-209). */
exl3_status exl3_trellis_reconstruct(const exl3_trellis_desc *w, uint16_t *w_out,
                                     exl3_stream_t stream);

/* One Hadamard step of the linear. Replaces trellis_hadamard (trellis_gemm.h:77-78):
 *   pre  (x_f16 != NULL): y = f16(H128(f32(x) * f32(s)) / sqrt(128))
 *   post (x_f32 != NULL): y = f16(H128(f32(f16(x))) / sqrt(128) * f32(s))
 * Exactly one of x_f16 / x_f32 is non-NULL. x is (rows, n), s is f16 [n] or, when
 * stacked > 0, `stacked` member vectors [stacked, n] with rows/stacked rows each. */
exl3_status exl3_trellis_hadamard(const uint16_t *x_f16, const float *x_f32, int64_t rows,
                                  int32_t n, const uint16_t *s, int32_t stacked, uint16_t *y,
                                  exl3_stream_t stream);

/* Workspace bytes for exl3_trellis_matmul_raw / exl3_trellis_linear(_grouped) on
 * n_members members of w's shape at `rows` rows. */
size_t exl3_trellis_workspace_size(const exl3_trellis_desc *w, int64_t rows, int32_t n_members);

/* yhat = xhat @ W_hat (f32, (rows, out)); xhat already rotated. Replaces
 * trellis_matmul_raw (trellis_gemm.h:68). */
exl3_status exl3_trellis_matmul_raw(const exl3_trellis_desc *w, const uint16_t *xhat,
                                    int64_t rows, float *yhat, void *workspace,
                                    size_t workspace_bytes, exl3_stream_t stream);

/* y = x @ W, f16 (rows, in) -> f16 (rows, out). Replaces trellis_linear
 * (trellis_gemm.h:51; trellis_gemm.cpp:1157-1197). */
exl3_status exl3_trellis_linear(const exl3_trellis_desc *w, const uint16_t *x, int64_t rows,
                                uint16_t *y, void *workspace, size_t workspace_bytes,
                                exl3_stream_t stream);

/* n linears of one shape in one launch, no member cap. members: host array of n.
 * x is (n, rows, in) (x_shared = 0, replaces trellis_linear_group_rows) or one
 * (rows, in) block shared by every member (x_shared = 1, replaces
 * trellis_linear_group); y is (n, rows, out). suh_stack/svh_stack, when non-NULL,
 * are device (n, in)/(n, out) f16 stacks used instead of the members' own scales
 * (replaces the *_scaled forms, trellis_gemm.h:102-106). Bit-identical to n calls
 * of exl3_trellis_linear. */
exl3_status exl3_trellis_linear_grouped(const exl3_trellis_desc *members, int32_t n,
                                        const uint16_t *x, int64_t rows, int32_t x_shared,
                                        const uint16_t *suh_stack, const uint16_t *svh_stack,
                                        uint16_t *y, void *workspace, size_t workspace_bytes,
                                        exl3_stream_t stream);

/* ---- MoE layer ---------------------------------------------------------------- */

/* Validates a layer (every expert of a projection class must share shape, K and
 * codebook; moe_prep_of, glm5_moe.cpp:430-486) and uploads its device-resident
 * expert table (pointer and scale tables, the G5MoePrep equivalent). Synchronous.
 * Trellis words and the router are referenced, not copied. Copied into device memory
 * the layer owns (so these must hold their final values at this call): every expert's
 * suh/svh, stacked by expert like G5MoePrep (glm5_moe.cpp:430-486), and an f16 shared
 * expert, transposed to (out, in) for the matrix cores (3 * hidden * SI f16). A layer
 * with a trellis shared expert also owns a second stream (default priority): calls of
 * 65 rows or more run the shared expert on it, forked from and joined back into the
 * caller's stream within the call. */
exl3_status exl3_moe_layer_create(const exl3_moe_layer_desc *desc, const exl3_moe_config *cfg,
                                  exl3_moe_layer_t *out);
exl3_status exl3_moe_layer_destroy(exl3_moe_layer_t layer);

/* Workspace bytes for a call with `rows` (= B * L) token rows; 0 when rows <= 0 or
 * rows exceeds one call's limit (2^24 / num_experts_per_tok). */
size_t exl3_moe_workspace_size(exl3_moe_layer_t layer, int64_t rows);

/* Router only: weights (rows, top_k) f32 and ids (rows, top_k) i32 from h (rows, hidden)
 * f16. Replaces the logits matmul + moe_topk_route (glm5_moe.cpp:16-60, 127-130).
 * Ids are in descending scores-for-choice order (ties: lower id first). */
exl3_status exl3_moe_route(exl3_moe_layer_t layer, const uint16_t *h, int64_t rows,
                           float *weights, int32_t *ids, void *workspace,
                           size_t workspace_bytes, exl3_stream_t stream);

/* Routing from caller logits (rows, n_experts) f32 and bias (n_experts) f32, no layer
 * handle. Replaces moe_topk_route (glm5_moe.h:29-31; glm5_moe.cpp:16-60): sigmoid
 * scores, bias used for selection only, optional group limit (n_group/topk_group:
 * group score = sum of its top-2 biased scores), top_k by biased score (ties: lower
 * id), weights = un-biased scores, normalised when norm_topk_prob, times
 * routed_scaling_factor. Only the routing fields of cfg are read. */
exl3_status exl3_moe_topk_route(const float *logits, const float *bias, int64_t rows,
                                const exl3_moe_config *cfg, float *weights, int32_t *ids,
                                exl3_stream_t stream);

/* The whole routed + shared MoE block: out (B, L, hidden) f16 from h (B, L, hidden)
 * f16. Replaces moe_layer (glm5_moe.h:35) and moe_layer_rows (glm5_moe.h:97); no host
 * round trip: routing, dispatch and every expert launch stay on the device. */
exl3_status exl3_moe_layer(exl3_moe_layer_t layer, const uint16_t *h, int64_t B, int64_t L,
                           uint16_t *out, void *workspace, size_t workspace_bytes,
                           exl3_stream_t stream);

/* Allocation-free form of exl3_moe_layer: no counterpart in the reference. It is for
 * callers that cannot allocate device memory (code under HIP graph capture, serving
 * loops that forbid hipMalloc): the workspace is a file-scope device array of the
 * library, exl3_moe_scratch_capacity() bytes (32 MiB; enough for the GLM-5 MoE layer up
 * to 30 token rows per call), one per GPU, held until the process ends. It calls no
 * hipMalloc/hipFree. Calls whose exl3_moe_workspace_size() is larger return
 * EXL3_ERR_UNSUPPORTED. Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (on different streams or threads, or different layers) race, so serialise
 * them. Stage timing and diagnostics are not collected on this path. Outputs are
 * bit-identical to exl3_moe_layer's. */
exl3_status exl3_moe_layer_noalloc(exl3_moe_layer_t layer, const uint16_t *h, int64_t B, int64_t L,
                                   uint16_t *out, exl3_stream_t stream);
size_t exl3_moe_scratch_capacity(void);

/* Stage timing (exl3_moe_timing); enabling it makes each layer call synchronous. The
 * stage events belong to the handle: timed calls must not overlap (one caller at a
 * time while timing is on). */
exl3_status exl3_moe_timing_enable(exl3_moe_layer_t layer, int32_t enabled);
exl3_status exl3_moe_timing_get(exl3_moe_layer_t layer, exl3_moe_timing *out);
exl3_status exl3_moe_timing_reset(exl3_moe_layer_t layer);

/* The handle's own copy of the tuning knobs (TrellisTuning, trellis_gemm.h:137-145,
 * which the reference keeps process-global). It starts as exl3_get_tuning() at
 * exl3_moe_layer_create; its mat_min_rows/mat_max_rows window decides which runs the
 * diagnostics count as staged, and its weight_form the weights of the mcg/3inst expert
 * GEMVs (the only knob that changes output bits). Rejected (EXL3_ERR_INVALID) for a
 * weight_form outside exl3_weight_form. Not to be changed while a call on the handle
 * is being enqueued. */
exl3_status exl3_moe_set_tuning(exl3_moe_layer_t layer, const exl3_tuning *t);
exl3_status exl3_moe_get_tuning(exl3_moe_layer_t layer, exl3_tuning *t);

/* MoeRowsDiag equivalents (glm5_moe.h:121-122). staged_runs counts runs whose row
 * count lies in the handle's staged window; streamed_bytes counts each run's expert
 * bytes once per weight pass (passes of min(rows, 16) rows, or of 64 rows in calls of
 * 65 rows or more). */
exl3_status exl3_moe_diag_enable(exl3_moe_layer_t layer, int32_t enabled);
exl3_status exl3_moe_diag_get(exl3_moe_layer_t layer, exl3_moe_diag *out);
exl3_status exl3_moe_diag_reset(exl3_moe_layer_t layer);

/* ---------------------------------------------------------------------------------
 * The steps either side of the MoE in the GLM-5 batch step (glm5_forward.cpp:434-438):
 * hyper-connection prepare, RMSNorm, the MoE, hyper-connection mix.
 * --------------------------------------------------------------------------------- */

/* One hyper-connection site (G5Layer hc_ffn_* / hc_attn_*, glm5.h:79-82; config
 * hc_mult, hc_sinkhorn_iters, hc_eps, model.h:65-67). fn is (W, mult*hidden) f32 with
 * W = (2 + mult) * mult, stored (out, in) as F.linear's weight; base (W) f32; scale (3)
 * f32. mult 1..8 (the reference's fused kernel takes 1..4 and its MLX expression any
 * count; GLM-5 uses 4). */
typedef struct {
  int32_t mult;
  int32_t sinkhorn_iters;
  float eps;
  const float *fn;     /* device, 16-byte aligned */
  const float *base;   /* device */
  const float *scale;  /* device */
} exl3_hc_site;

/* Replaces g5_hc_prepare (glm5_hc.cpp:242-340) and, when norm_w != NULL, the rms_norm of
 * its collapsed stream that follows it (glm5_attn.cpp:12-22; glm5_forward.cpp:435-436).
 * streams (P, mult, hidden) f16 (8-byte aligned) -> out (P, hidden) f16: the collapsed
 * stream sum_n pre[n] * streams[n], or rms_norm(collapsed) * norm_w; post (P, mult) and
 * comb (P, mult, mult) f32 as the reference returns them. The workspace holds k-split
 * partials (exl3_hc_workspace_size). Requires mult * hidden % 64 == 0, hidden even and <= 8192. */
size_t exl3_hc_workspace_size(int32_t mult, int32_t hidden, int64_t P);
exl3_status exl3_hc_prepare(const exl3_hc_site *hc, const uint16_t *streams, int64_t P, int32_t hidden,
                            const uint16_t *norm_w, float norm_eps, uint16_t *out, float *post, float *comb,
                            void *workspace, size_t workspace_bytes, exl3_stream_t stream);
/* Replaces rms_norm (glm5_attn.cpp:12-22): y = f16(f16(x * rsqrt(mean(x^2) + eps)) * w),
 * f32 statistics; x, y (P, hidden) f16, w (hidden) f16, 4-byte aligned; hidden even,
 * <= 8192. */
exl3_status exl3_rms_norm(const uint16_t *x, int64_t P, int32_t hidden, const uint16_t *w, float eps,
                          uint16_t *y, exl3_stream_t stream);
/* Replaces g5_hc_mix (glm5_hc.cpp:342-355): out[p][n] = post[p][n] * block_out[p] +
 * sum_m comb[p][m][n] * residual[p][m], in f16 as the reference (block_out's dtype). */
exl3_status exl3_hc_mix(const uint16_t *block_out, const float *post, const float *comb, const uint16_t *residual,
                        int64_t P, int32_t mult, int32_t hidden, uint16_t *out, exl3_stream_t stream);

/* The MLP sub-block of a GLM-5 MoE layer in one call (glm5_forward.cpp:434-438):
 * f = g5_hc_prepare(streams, hc); h = rms_norm(f.collapsed, norm_w, norm_eps);
 * out = moe_layer_rows(h); streams_out = g5_hc_mix(out, f.post, f.comb, streams).
 * Two launches before the MoE's own (the prepare's projection partials, then its
 * finalize with the RMSNorm fused), and the mix fused into the MoE's combine. streams /
 * streams_out (P, mult, hidden) f16 (distinct buffers). Bit-identical to the separate
 * calls exl3_hc_prepare + exl3_moe_layer + exl3_hc_mix. */
size_t exl3_moe_block_workspace_size(exl3_moe_layer_t layer, int32_t hc_mult, int64_t P);
exl3_status exl3_moe_block(exl3_moe_layer_t layer, const exl3_hc_site *hc, const uint16_t *norm_w, float norm_eps,
                           const uint16_t *streams, int64_t P, uint16_t *streams_out, void *workspace,
                           size_t workspace_bytes, exl3_stream_t stream);

/* ---------------------------------------------------------------------------------
 * Safetensors shards and the EXL3 MoE layer loader. Replaces SafetensorsFile
 * (safetensors.h:23-70: header parse + mmap) and the MoE part of load_glm5
 * (glm5.cpp:284-376 load_linear, 503-518 the layer's keys). Host-only calls except
 * exl3_moe_layer_load, which allocates and fills device memory.
 * --------------------------------------------------------------------------------- */
typedef enum {
  EXL3_ST_F16 = 0, EXL3_ST_BF16 = 1, EXL3_ST_F32 = 2, EXL3_ST_I16 = 3, EXL3_ST_I32 = 4,
  EXL3_ST_U8 = 5, EXL3_ST_I8 = 6, EXL3_ST_I64 = 7, EXL3_ST_F64 = 8, EXL3_ST_U16 = 9,
  EXL3_ST_U32 = 10, EXL3_ST_BOOL = 11
} exl3_st_dtype;

/* One tensor of a shard (STTensor, safetensors.h:14-21). offset is relative to the data
 * section, file_offset = header_len + offset is the byte position in the file. */
typedef struct {
  int32_t dtype; /* exl3_st_dtype */
  int32_t ndim;
  int64_t shape[8];
  int64_t offset;
  int64_t nbytes;
  int64_t file_offset;
} exl3_st_tensor;

typedef struct exl3_st_file_s *exl3_st_file_t;

/* Parse the header (8-byte little-endian length, JSON) and map the file read-only. The
 * reference's consistency checks apply: dtype size x element count = byte count, and the
 * data lies inside the file. */
exl3_status exl3_st_open(const char *path, exl3_st_file_t *out);
exl3_status exl3_st_close(exl3_st_file_t f);
int64_t exl3_st_header_len(exl3_st_file_t f);  /* 8 + JSON length */
int32_t exl3_st_count(exl3_st_file_t f);
exl3_status exl3_st_tensor_at(exl3_st_file_t f, int32_t i, exl3_st_tensor *info, const char **name);
exl3_status exl3_st_find(exl3_st_file_t f, const char *name, exl3_st_tensor *info);
const void *exl3_st_data(exl3_st_file_t f, const char *name);  /* host pointer into the map */

/* Load one GLM-5 MoE layer from EXL3 shards: `prefix` is the layer's "...mlp." key
 * prefix; the keys are experts.{e}.{gate,up,down}_proj.{trellis,suh,svh,mul1|mcg},
 * shared_experts.* (trellis or a plain f16 .weight, stored (out, in)), gate.weight (E,
 * hidden) f16 and gate.e_score_correction_bias (E) f32. The codebook of a linear is mul1
 * when its .mul1 marker exists, else mcg when .mcg exists, else 3inst (glm5.cpp:303).
 * Every shard's needed byte range is copied to the device once, keeping the file's
 * alignment modulo 4: a trellis tensor at a 4-byte-aligned file position is used in
 * place (the reference's zero-copy view, glm5.cpp:333-347); the others are repacked on
 * the device into aligned buffers (glm5.cpp:349-352, trellis_gemm.cpp:311-316). The
 * returned handle owns all device memory of the layer (exl3_moe_layer_destroy frees
 * it); the call synchronises `stream`. */
exl3_status exl3_moe_layer_load(const char *const *shard_paths, int32_t n_shards, const char *prefix,
                                const exl3_moe_config *cfg, exl3_moe_layer_t *out_layer,
                                exl3_stream_t stream);
/* The MLP sub-block's own tensors of one decoder layer, so that exl3_moe_block can run
 * from shards. Replaces the loads of l.post_norm and l.hc_ffn_* in load_decoder_layer
 * (glm5.cpp:409-415). layer_prefix is the decoder layer's key prefix ("model.layers.N.");
 * the keys are post_attention_layernorm.weight (hidden), hc_ffn_fn ((2 + mult) * mult,
 * mult * hidden), hc_ffn_base ((2 + mult) * mult) and hc_ffn_scale (3), converted as the
 * reference's load_any (glm5.cpp:205-281): the norm weight to f16 (F16 as stored, BF16
 * widened to f32 and rounded once to f16, F32 rounded to f16, both to nearest even), the
 * hc tensors to f32 (F32 as stored, F16 widened, BF16 through that same f16 value). The
 * caller sets site->mult, sinkhorn_iters and eps (the model's hc_mult, hc_sinkhorn_iters,
 * hc_eps); the call fills site->fn/base/scale and *norm_w with device pointers into
 * memory `layer` owns (freed by exl3_moe_layer_destroy). Synchronises `stream`. */
exl3_status exl3_moe_layer_load_block(exl3_moe_layer_t layer, const char *const *shard_paths, int32_t n_shards,
                                      const char *layer_prefix, exl3_hc_site *site, const uint16_t **norm_w,
                                      exl3_stream_t stream);
/* For a loaded layer: trellis tensors used in place and repacked (0, 0 otherwise). */
exl3_status exl3_moe_layer_load_info(exl3_moe_layer_t layer, int64_t *in_place, int64_t *repacked);

#ifdef __cplusplus
}
#endif

#endif /* EXL3_MOE_H */
