/*
 * CPU oracle for the EXL3 MoE decode path -- TEST INFRASTRUCTURE ONLY.
 * See exl3_oracle.h for what each function restates and how it is pinned.
 *
 * Reference files (muyouming/exl3-server): src/fp16.h, src/exl3.cpp,
 * src/trellis_gemm.cpp (Hadamard kernel rounding points), src/glm5_moe.cpp.
 */
#include "exl3_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* Minimal parallel-for: `threads` workers pull indices from an atomic counter */
/* (the scheme of the reference's util.h:55-74).                              */
/* ------------------------------------------------------------------------- */

typedef void (*or_task_fn)(void *ctx, int64_t i);

typedef struct {
  or_task_fn fn;
  void *ctx;
  int64_t n;
  atomic_llong next;
} or_pool;

static void *or_worker(void *arg) {
  or_pool *p = (or_pool *)arg;
  for (;;) {
    int64_t i = atomic_fetch_add(&p->next, 1);
    if (i >= p->n) break;
    p->fn(p->ctx, i);
  }
  return NULL;
}

static void or_parallel_for(int64_t n, int threads, or_task_fn fn, void *ctx) {
  if (n <= 0) return;
  if (threads <= 1 || n == 1) {
    for (int64_t i = 0; i < n; ++i) fn(ctx, i);
    return;
  }
  if (threads > 256) threads = 256;
  or_pool p;
  p.fn = fn;
  p.ctx = ctx;
  p.n = n;
  atomic_init(&p.next, 0);
  pthread_t tid[256];
  int started = 0;
  for (int t = 1; t < threads; ++t)
    if (pthread_create(&tid[started], NULL, or_worker, &p) == 0) ++started;
  or_worker(&p);
  for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
}

/* ------------------------------------------------------------------------- */
/* IEEE binary16 <-> double (reference fp16.h:18-64).                          */
/* ------------------------------------------------------------------------- */

double or_f16_to_double(uint16_t h) {
  const int sign = h >> 15, e = (h >> 10) & 31, m = h & 1023;
  double v;
  if (e == 0)
    v = ldexp((double)m, -24);
  else if (e == 31)
    v = m ? NAN : INFINITY;
  else
    v = ldexp((double)(1024 + m), e - 25);
  return sign ? -v : v;
}

/* Round to nearest, ties to even. NaN -> 0x7e00, |x| that rounds past 65504 -> inf. */
uint16_t or_f16_from_double(double x) {
  if (isnan(x)) return 0x7e00;
  const uint16_t sign = signbit(x) ? 0x8000 : 0;
  double a = fabs(x);
  if (isinf(a)) return sign | 0x7c00;
  if (a == 0.0) return sign;
  int e2;
  (void)frexp(a, &e2); /* a in [2^(e2-1), 2^e2) */
  int e = e2 - 1;      /* a = m * 2^e, m in [1, 2) */
  if (e > 15) return sign | 0x7c00;
  if (e >= -14) {
    /* 10 fraction bits: q = a * 2^(10-e) in [1024, 2048). rint is RNE in the
     * default rounding mode; the multiply by a power of two is exact. */
    double q = rint(ldexp(a, 10 - e));
    if (q >= 2048.0) {
      q = 1024.0;
      e += 1;
      if (e > 15) return sign | 0x7c00;
    }
    return (uint16_t)(sign | ((uint16_t)(e + 15) << 10) | (uint16_t)((int)q - 1024));
  }
  /* Subnormal: multiples of 2^-24; q == 1024 is the smallest normal (0x0400). */
  double q = rint(ldexp(a, 24));
  return (uint16_t)(sign | (uint16_t)q);
}

/* ------------------------------------------------------------------------- */
/* Procedural codebooks (reference exl3.cpp:21-42, GPU form trellis_gemm.cpp   */
/* :333-356). All intermediate values are exact in double, so one RNE here is  */
/* the single rounding of the fused half arithmetic.                           */
/* ------------------------------------------------------------------------- */

uint16_t or_codebook_value(uint16_t state, int cb) {
  const uint32_t s = state;
  if (cb == 2) { /* mul1 */
    const uint32_t x = s * 0x83DCD12Du;
    const uint32_t bytesum = (x & 0xffu) + ((x >> 8) & 0xffu) + ((x >> 16) & 0xffu) + (x >> 24);
    const double v = or_f16_to_double((uint16_t)(0x6400u + bytesum));
    return or_f16_from_double(v * or_f16_to_double(0x1eee) + or_f16_to_double(0xc931));
  }
  uint32_t x = (cb == 1) ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
  x = (x & 0x8fff8fffu) ^ 0x3b603b60u;
  return or_f16_from_double(or_f16_to_double((uint16_t)(x & 0xffffu)) +
                            or_f16_to_double((uint16_t)(x >> 16)));
}

static uint16_t g_lut[3][65536];
static pthread_once_t g_lut_once = PTHREAD_ONCE_INIT;

static void or_build_luts(void) {
  for (int cb = 0; cb < 3; ++cb)
    for (uint32_t s = 0; s < 65536u; ++s) g_lut[cb][s] = or_codebook_value((uint16_t)s, cb);
}

static const uint16_t *or_lut(int cb) {
  pthread_once(&g_lut_once, or_build_luts);
  return g_lut[cb];
}

void or_codebook_lut(int cb, uint16_t *lut) { memcpy(lut, or_lut(cb), sizeof(uint16_t) * 65536); }

/* The GEMV's weight values, as f32. Mode 0: the reference's f16 weights. Mode 1
 * ("exact halves"): for mcg and 3inst the exact sum lo + hi of the masked hash word's two
 * f16 halves (exact in f32: both halves lie in [2^-3, 2), so the sum needs at most 15
 * significant bits), i.e. the weight before the reference's f16 rounding of lo + hi
 * (trellis_gemm.cpp:348-356). That is the value a GEMV that feeds both halves to its
 * multiply-accumulate uses; mul1 is unchanged. */
static float g_lutf[2][3][65536];
static pthread_once_t g_lutf_once = PTHREAD_ONCE_INIT;
static int g_gemv_mode = 0;

float or_codebook_halves_sum(uint16_t state, int cb) {
  const uint32_t s = state;
  uint32_t x = (cb == 1) ? s * 0xCBAC1FEDu : s * 89226354u + 64248484u;
  x = (x & 0x8fff8fffu) ^ 0x3b603b60u;
  return (float)(or_f16_to_double((uint16_t)(x & 0xffffu)) + or_f16_to_double((uint16_t)(x >> 16)));
}

static void or_build_lutf(void) {
  for (int cb = 0; cb < 3; ++cb)
    for (uint32_t st = 0; st < 65536u; ++st) {
      const float ref = (float)or_f16_to_double(or_lut(cb)[st]);
      g_lutf[0][cb][st] = ref;
      g_lutf[1][cb][st] = cb == 2 ? ref : or_codebook_halves_sum((uint16_t)st, cb);
    }
}

static const float *or_lutf(int cb) {
  pthread_once(&g_lutf_once, or_build_lutf);
  return g_lutf[g_gemv_mode][cb];
}

void or_set_gemv_mode(int exact_halves) { g_gemv_mode = exact_halves ? 1 : 0; }
int or_get_gemv_mode(void) { return g_gemv_mode; }

/* ------------------------------------------------------------------------- */
/* Tile bitstream (reference exl3.cpp:55-107; format comment exl3.h:11-16).    */
/* One tile is 16*K stored u16; ring word i = s[2i] | s[2i+1] << 16 (8K words, */
/* 256K bits). Ring bit b is bit 31 - (b mod 32) of word (b / 32) mod 8K, i.e. */
/* MSB first. Position p's state is the 16 ring bits ending (exclusive) at     */
/* bit (p + 1) * K, read as a big-endian number.                               */
/* ------------------------------------------------------------------------- */

static inline uint32_t or_ring_word(const uint16_t *tile_words, int K, int64_t i) {
  const int64_t nw = 8 * (int64_t)K;
  i %= nw;
  if (i < 0) i += nw;
  return (uint32_t)tile_words[2 * i] | ((uint32_t)tile_words[2 * i + 1] << 16);
}

uint16_t or_tile_state(const uint16_t *tile_words, int K, int p) {
  const int64_t last_bit = (int64_t)(p + 1) * K - 1; /* ring bit holding the state's LSB */
  const int64_t last = last_bit / 32;
  const uint64_t pair = ((uint64_t)or_ring_word(tile_words, K, last - 1) << 32) |
                        (uint64_t)or_ring_word(tile_words, K, last);
  return (uint16_t)(pair >> (31 - (last_bit % 32)));
}

uint16_t or_tile_state_bruteforce(const uint16_t *tile_words, int K, int p) {
  const int64_t ring = 256 * (int64_t)K;
  uint32_t st = 0;
  for (int j = 0; j < 16; ++j) {
    int64_t b = ((int64_t)(p + 1) * K - 16 + j) % ring;
    if (b < 0) b += ring;
    const uint32_t w = or_ring_word(tile_words, K, b / 32);
    st = (st << 1) | ((w >> (31 - (b % 32))) & 1u);
  }
  return (uint16_t)st;
}

/* Tensor-core permutation (reference exl3.cpp:81-99): p = L*8 + i with L the
 * 32-lane index; row = 2*(L%4) + {0,1,8,9}[i%4], col = L/4 + 8*(i/4). */
int or_tile_perm(int p) {
  static const int rsel[4] = {0, 1, 8, 9};
  const int L = p >> 3, i = p & 7;
  const int row = 2 * (L & 3) + rsel[i & 3];
  const int col = (L >> 2) + 8 * (i >> 2);
  return row * 16 + col;
}

static void or_decode_tile(const uint16_t *tile_words, int K, const uint16_t *lut, uint16_t *dst,
                           int64_t stride) {
  for (int p = 0; p < 256; ++p) {
    const int e = or_tile_perm(p);
    dst[(int64_t)(e >> 4) * stride + (e & 15)] = lut[or_tile_state(tile_words, K, p)];
  }
}

/* Decode one tile to f32 [16][16] (row = k, col = n) through a table of weight values. */
static void or_decode_tile_f(const uint16_t *tile_words, int K, const float *lutf, float out[256]) {
  for (int p = 0; p < 256; ++p) out[or_tile_perm(p)] = lutf[or_tile_state(tile_words, K, p)];
}

typedef struct {
  const uint16_t *trellis;
  int64_t in, out;
  int K;
  const uint16_t *lut;
  uint16_t *dst;
} or_decode_ctx;

static void or_decode_task(void *vctx, int64_t idx) {
  or_decode_ctx *c = (or_decode_ctx *)vctx;
  const int64_t tiles_n = c->out / 16;
  const int64_t tk = idx / tiles_n, tn = idx % tiles_n;
  or_decode_tile(c->trellis + idx * 16 * c->K, c->K, c->lut, c->dst + tk * 16 * c->out + tn * 16,
                 c->out);
}

int or_decode_inner(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb,
                    uint16_t *w_hat, int threads) {
  if (in <= 0 || out <= 0 || in % 16 || out % 16 || K < 1 || K > 8 || cb < 0 || cb > 2) return -1;
  or_decode_ctx c = {trellis, in, out, K, or_lut(cb), w_hat};
  or_parallel_for((in / 16) * (out / 16), threads, or_decode_task, &c);
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Hadamard (Sylvester, 128-blocks). Stage order len = 1, 2, ..., 64 with      */
/* (x[j], x[j+len]) -> (a + b, a - b) in f32: the order of reference           */
/* exl3.cpp:140-150 and of the GPU kernel trellis_gemm.cpp:387-396, so every   */
/* output is the same f32 association.                                         */
/* ------------------------------------------------------------------------- */

static const float kHadScaleF = 1.0f / 11.313708498984761f; /* 1/sqrt(128) in f32 */

static void or_fwht128(float *x) {
  for (int len = 1; len < 128; len <<= 1)
    for (int i = 0; i < 128; i += 2 * len)
      for (int j = i; j < i + len; ++j) {
        const float a = x[j], b = x[j + len];
        x[j] = a + b;
        x[j + len] = a - b;
      }
}

/* Reference reconstruct: exl3.cpp:152-209. */
typedef struct {
  uint16_t *w;
  int64_t out;
  const uint16_t *suh, *svh;
} or_rot_ctx;

static void or_rot_task(void *vctx, int64_t b) {
  or_rot_ctx *c = (or_rot_ctx *)vctx;
  const int64_t out = c->out;
  float *buf = (float *)malloc(sizeof(float) * 128 * (size_t)out);
  uint16_t *base = c->w + b * 128 * out;
  for (int64_t i = 0; i < 128 * out; ++i) buf[i] = (float)or_f16_to_double(base[i]);
  /* left: butterflies across the 128 rows of the block */
  for (int len = 1; len < 128; len <<= 1)
    for (int i = 0; i < 128; i += 2 * len)
      for (int j = i; j < i + len; ++j) {
        float *ra = buf + (int64_t)j * out, *rb = buf + (int64_t)(j + len) * out;
        for (int64_t col = 0; col < out; ++col) {
          const float a = ra[col], d = rb[col];
          ra[col] = a + d;
          rb[col] = a - d;
        }
      }
  for (int i = 0; i < 128; ++i) {
    const float s = (float)or_f16_to_double(c->suh[b * 128 + i]) * kHadScaleF;
    float *r = buf + (int64_t)i * out;
    for (int64_t col = 0; col < out; ++col) r[col] *= s;
  }
  /* right: per row and 128-column segment, butterfly then the column scale */
  for (int i = 0; i < 128; ++i) {
    float *r = buf + (int64_t)i * out;
    for (int64_t cb = 0; cb < out / 128; ++cb) {
      float *seg = r + cb * 128;
      or_fwht128(seg);
      for (int j = 0; j < 128; ++j) {
        const float s = (float)or_f16_to_double(c->svh[cb * 128 + j]) * kHadScaleF;
        seg[j] *= s;
      }
    }
    for (int64_t col = 0; col < out; ++col)
      base[(int64_t)i * out + col] = or_f16_from_double((double)r[col]);
  }
  free(buf);
}

int or_reconstruct(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb,
                   const uint16_t *suh, const uint16_t *svh, uint16_t *w, int threads) {
  if (in <= 0 || out <= 0 || in % 128 || out % 128) return -1;
  if (or_decode_inner(trellis, in, out, K, cb, w, threads)) return -1;
  or_rot_ctx c = {w, out, suh, svh};
  or_parallel_for(in / 128, threads, or_rot_task, &c);
  return 0;
}

/* Input side (trellis_gemm.cpp:383-399 with HAD_PRE=1):
 *   xhat = f16( fwht(f32(x) * f32(suh)) * (1/sqrt 128) ) */
void or_had_pre(const uint16_t *x, int64_t rows, int64_t n, const uint16_t *suh, uint16_t *xhat) {
  float buf[128];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t blk = 0; blk < n / 128; ++blk) {
      const int64_t o = r * n + blk * 128;
      for (int t = 0; t < 128; ++t)
        buf[t] = (float)or_f16_to_double(x[o + t]) * (float)or_f16_to_double(suh[blk * 128 + t]);
      or_fwht128(buf);
      for (int t = 0; t < 128; ++t) xhat[o + t] = or_f16_from_double((double)(buf[t] * kHadScaleF));
    }
}

/* Output side (HAD_PRE=0): y = f16( fwht(f32(f16(yhat))) * (1/sqrt 128) * f32(svh) ),
 * the two multiplies rounded separately in f32. */
void or_had_post(const float *yhat, int64_t rows, int64_t n, const uint16_t *svh, uint16_t *y) {
  float buf[128];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t blk = 0; blk < n / 128; ++blk) {
      const int64_t o = r * n + blk * 128;
      for (int t = 0; t < 128; ++t)
        buf[t] = (float)or_f16_to_double(or_f16_from_double((double)yhat[o + t]));
      or_fwht128(buf);
      for (int t = 0; t < 128; ++t) {
        float v = buf[t] * kHadScaleF;
        v = v * (float)or_f16_to_double(svh[blk * 128 + t]);
        y[o + t] = or_f16_from_double((double)v);
      }
    }
}

void or_had_post_f64(const double *yhat, int64_t rows, int64_t n, const uint16_t *svh,
                     uint16_t *y) {
  float buf[128];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t blk = 0; blk < n / 128; ++blk) {
      const int64_t o = r * n + blk * 128;
      for (int t = 0; t < 128; ++t)
        buf[t] = (float)or_f16_to_double(or_f16_from_double(yhat[o + t]));
      or_fwht128(buf);
      for (int t = 0; t < 128; ++t) {
        float v = buf[t] * kHadScaleF;
        v = v * (float)or_f16_to_double(svh[blk * 128 + t]);
        y[o + t] = or_f16_from_double((double)v);
      }
    }
}

/* ------------------------------------------------------------------------- */
/* GEMV with on-the-fly decode, f64 accumulation.                              */
/* ------------------------------------------------------------------------- */

typedef struct {
  const uint16_t *trellis;
  int64_t in, out, rows;
  int K;
  const float *lutf;
  const uint16_t *xhat;
  double *yhat;
} or_mm_ctx;

/* One task = one output tile column (tn) over every k-tile, so each task owns
 * its outputs and no reduction across threads is needed. */
static void or_mm_task(void *vctx, int64_t tn) {
  or_mm_ctx *c = (or_mm_ctx *)vctx;
  const int64_t tiles_n = c->out / 16, tiles_k = c->in / 16;
  float w[256];
  for (int64_t r = 0; r < c->rows; ++r)
    for (int col = 0; col < 16; ++col) c->yhat[r * c->out + tn * 16 + col] = 0.0;
  for (int64_t tk = 0; tk < tiles_k; ++tk) {
    or_decode_tile_f(c->trellis + (tk * tiles_n + tn) * 16 * c->K, c->K, c->lutf, w);
    for (int64_t r = 0; r < c->rows; ++r) {
      const uint16_t *xr = c->xhat + r * c->in + tk * 16;
      double *yr = c->yhat + r * c->out + tn * 16;
      for (int k = 0; k < 16; ++k) {
        const double xv = or_f16_to_double(xr[k]);
        if (xv == 0.0) continue;
        for (int col = 0; col < 16; ++col) yr[col] += xv * (double)w[k * 16 + col];
      }
    }
  }
}

int or_matmul_raw(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb,
                  const uint16_t *xhat, int64_t rows, double *yhat, int threads) {
  if (in <= 0 || out <= 0 || in % 16 || out % 16 || K < 1 || K > 8 || cb < 0 || cb > 2) return -1;
  or_mm_ctx c = {trellis, in, out, rows, K, or_lutf(cb), xhat, yhat};
  or_parallel_for(out / 16, threads, or_mm_task, &c);
  return 0;
}

int or_trellis_linear(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb,
                      const uint16_t *suh, const uint16_t *svh, const uint16_t *x, int64_t rows,
                      uint16_t *y, int threads) {
  if (in % 128 || out % 128) return -1;
  uint16_t *xhat = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(rows * in));
  double *yhat = (double *)malloc(sizeof(double) * (size_t)(rows * out));
  or_had_pre(x, rows, in, suh, xhat);
  int rc = or_matmul_raw(trellis, in, out, K, cb, xhat, rows, yhat, threads);
  if (rc == 0) or_had_post_f64(yhat, rows, out, svh, y);
  free(xhat);
  free(yhat);
  return rc;
}

/* ------------------------------------------------------------------------- */
/* Router (reference glm5_moe.cpp:16-60, HF Glm5NextTextTopkRouter.forward).   */
/* ------------------------------------------------------------------------- */

void or_router_logits(const uint16_t *h, int64_t N, const uint16_t *router_w, int E, int H,
                      double *logits) {
  for (int64_t t = 0; t < N; ++t)
    for (int e = 0; e < E; ++e) {
      double acc = 0.0;
      for (int k = 0; k < H; ++k)
        acc += or_f16_to_double(h[t * H + k]) * or_f16_to_double(router_w[(int64_t)e * H + k]);
      logits[t * E + e] = acc;
    }
}

/* Index order for "descending value, ties to the lower index". */
static int or_better(double va, int a, double vb, int b) { return va > vb || (va == vb && a < b); }

int or_route(const double *logits, const float *bias, int64_t N, const or_moe_cfg *cfg,
             int32_t *idx, double *weights) {
  const int E = cfg->n_experts, K = cfg->top_k;
  const int ng = cfg->n_group > 1 ? cfg->n_group : 1;
  int tg = cfg->topk_group > 0 ? cfg->topk_group : 1;
  if (tg > ng) tg = ng;
  if (E <= 0 || K <= 0 || K > E || E % ng) return -1;
  const int gsize = E / ng;
  double *sc = (double *)malloc(sizeof(double) * (size_t)E);
  double *sfc = (double *)malloc(sizeof(double) * (size_t)E);
  double *gs = (double *)malloc(sizeof(double) * (size_t)ng);
  char *keep = (char *)malloc((size_t)E);
  char *taken = (char *)malloc((size_t)E);
  for (int64_t t = 0; t < N; ++t) {
    for (int e = 0; e < E; ++e) {
      sc[e] = 1.0 / (1.0 + exp(-logits[t * E + e]));
      sfc[e] = sc[e] + (double)bias[e];
    }
    /* group score: sum of the group's top-2 scores_for_choice (top-1 if 1 wide) */
    for (int g = 0; g < ng; ++g) {
      double m1 = -INFINITY, m2 = -INFINITY;
      for (int j = 0; j < gsize; ++j) {
        const double v = sfc[g * gsize + j];
        if (v > m1) {
          m2 = m1;
          m1 = v;
        } else if (v > m2) {
          m2 = v;
        }
      }
      gs[g] = gsize >= 2 ? m1 + m2 : m1;
    }
    memset(keep, 0, (size_t)E);
    for (int i = 0; i < tg; ++i) {
      int best = -1;
      for (int g = 0; g < ng; ++g) {
        if (keep[g * gsize]) continue;
        if (best < 0 || or_better(gs[g], g, gs[best], best)) best = g;
      }
      for (int j = 0; j < gsize; ++j) keep[best * gsize + j] = 1;
    }
    memset(taken, 0, (size_t)E);
    double denom = 0.0;
    for (int k = 0; k < K; ++k) {
      int best = -1;
      for (int e = 0; e < E; ++e) {
        if (taken[e]) continue;
        const double v = keep[e] ? sfc[e] : -INFINITY;
        const double vb = best >= 0 ? (keep[best] ? sfc[best] : -INFINITY) : 0.0;
        if (best < 0 || or_better(v, e, vb, best)) best = e;
      }
      taken[best] = 1;
      idx[t * K + k] = best;
      weights[t * K + k] = sc[best];
      denom += sc[best];
    }
    for (int k = 0; k < K; ++k) {
      double w = weights[t * K + k];
      if (cfg->norm_topk_prob) w /= (denom + 1e-20);
      weights[t * K + k] = w * (double)cfg->routed_scaling_factor;
    }
  }
  free(sc);
  free(sfc);
  free(gs);
  free(keep);
  free(taken);
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Expert-order dispatch (reference glm5_moe.cpp:158-200, 236-255).            */
/* ------------------------------------------------------------------------- */

int or_moe_runs(const int32_t *idx, int64_t N, int K, int32_t *sorted_expert,
                int32_t *sorted_row, int32_t *sorted_rank, int32_t *perm, int32_t *run_expert,
                int32_t *run_off, int32_t *run_len) {
  const int64_t P = N * K;
  /* stable counting sort by expert id over the (row, rank) visiting order */
  int32_t maxe = 0;
  for (int64_t p = 0; p < P; ++p)
    if (idx[p] > maxe) maxe = idx[p];
  int64_t *cnt = (int64_t *)calloc((size_t)maxe + 2, sizeof(int64_t));
  for (int64_t p = 0; p < P; ++p) cnt[idx[p] + 1]++;
  for (int32_t e = 0; e <= maxe; ++e) cnt[e + 1] += cnt[e];
  for (int64_t b = 0; b < N; ++b)
    for (int k = 0; k < K; ++k) {
      const int32_t e = idx[b * K + k];
      const int64_t pos = cnt[e]++;
      sorted_expert[pos] = e;
      sorted_row[pos] = (int32_t)b;
      sorted_rank[pos] = k;
      perm[(int64_t)k * N + b] = (int32_t)pos;
    }
  free(cnt);
  int runs = 0;
  for (int64_t p = 0; p < P;) {
    int64_t q = p;
    while (q < P && sorted_expert[q] == sorted_expert[p]) ++q;
    run_expert[runs] = sorted_expert[p];
    run_off[runs] = (int32_t)p;
    run_len[runs] = (int32_t)(q - p);
    ++runs;
    p = q;
  }
  return runs;
}

/* ------------------------------------------------------------------------- */
/* The layer (reference glm5_moe.cpp:66-74 swiglu, 112-417 rows path, 490-660). */
/* ------------------------------------------------------------------------- */

/* g5_linear (glm5_kda.cpp:119-123): trellis_linear, or f16 matmul rounded once. */
static void or_linear_apply(const or_linear *l, const uint16_t *x, int64_t rows, uint16_t *y) {
  if (l->trellis) {
    or_trellis_linear(l->trellis, l->in, l->out, l->K, l->cb, l->suh, l->svh, x, rows, y, 1);
    return;
  }
  double *acc = (double *)calloc((size_t)(rows * l->out), sizeof(double));
  for (int64_t r = 0; r < rows; ++r)
    for (int k = 0; k < l->in; ++k) {
      const double xv = or_f16_to_double(x[r * l->in + k]);
      if (xv == 0.0) continue;
      const uint16_t *wr = l->dense + (int64_t)k * l->out;
      double *ar = acc + r * l->out;
      for (int n = 0; n < l->out; ++n) ar[n] += xv * or_f16_to_double(wr[n]);
    }
  for (int64_t i = 0; i < rows * l->out; ++i) y[i] = or_f16_from_double(acc[i]);
  free(acc);
}

/* silu(min(gate, L)) * clamp(up, -L, L) in f16 op-by-op (each MLX op rounds to
 * f16), then the down projection. */
static void or_swiglu(const or_linear *g, const or_linear *u, const or_linear *d,
                      const uint16_t *x, int64_t rows, float limit, uint16_t *y) {
  const int I = g->out;
  uint16_t *gate = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(rows * I));
  uint16_t *up = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(rows * I));
  or_linear_apply(g, x, rows, gate);
  or_linear_apply(u, x, rows, up);
  const double L = or_f16_to_double(or_f16_from_double((double)limit));
  for (int64_t i = 0; i < rows * I; ++i) {
    double gv = or_f16_to_double(gate[i]);
    double uv = or_f16_to_double(up[i]);
    if (gv > L) gv = L;   /* mx::clip(gate, none, L) */
    if (uv < -L) uv = -L; /* mx::clip(up, -L, L): the lower bound, then the upper */
    if (uv > L) uv = L;
    const double sig = or_f16_to_double(or_f16_from_double(1.0 / (1.0 + exp(-gv))));
    const double act = or_f16_to_double(or_f16_from_double(gv * sig));
    gate[i] = or_f16_from_double(act * uv);
  }
  or_linear_apply(d, gate, rows, y);
  free(gate);
  free(up);
}

typedef struct {
  const or_moe_cfg *cfg;
  const or_linear *experts;
  const uint16_t *h;
  int64_t N;
  const int32_t *sorted_row;
  const int32_t *run_expert, *run_off, *run_len;
  uint16_t *ysorted; /* (P, H) f16, sorted-pair order */
} or_layer_ctx;

static void or_layer_task(void *vctx, int64_t r) {
  or_layer_ctx *c = (or_layer_ctx *)vctx;
  const int H = c->cfg->hidden;
  const int e = c->run_expert[r], off = c->run_off[r], n = c->run_len[r];
  uint16_t *xr = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)n * H);
  for (int i = 0; i < n; ++i)
    memcpy(xr + (int64_t)i * H, c->h + (int64_t)c->sorted_row[off + i] * H, sizeof(uint16_t) * H);
  or_swiglu(&c->experts[3 * e], &c->experts[3 * e + 1], &c->experts[3 * e + 2], xr, n,
            c->cfg->swiglu_limit, c->ysorted + (int64_t)off * H);
  free(xr);
}

int or_moe_layer_routed(const or_moe_cfg *cfg, const or_linear *experts,
                        const or_linear *shared, const uint16_t *h, int64_t N,
                        const int32_t *idx, const double *weights, uint16_t *out, int threads) {
  const int H = cfg->hidden, K = cfg->top_k;
  const int64_t P = N * K;
  int32_t *se = (int32_t *)malloc(sizeof(int32_t) * (size_t)P * 7);
  int32_t *sr = se + P, *sk = se + 2 * P, *perm = se + 3 * P, *re = se + 4 * P, *ro = se + 5 * P,
          *rl = se + 6 * P;
  const int runs = or_moe_runs(idx, N, K, se, sr, sk, perm, re, ro, rl);
  uint16_t *ys = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(P * H));
  or_layer_ctx c = {cfg, experts, h, N, sr, re, ro, rl, ys};
  or_parallel_for(runs, threads, or_layer_task, &c);
  uint16_t *sh = NULL;
  if (shared && cfg->has_shared) {
    sh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)(N * H));
    or_swiglu(&shared[0], &shared[1], &shared[2], h, N, cfg->swiglu_limit, sh);
  }
  /* routed = sum_k f16(f32(y_k) * f32(w_k)) (rank order, summed exactly then
   * rounded once), out = f16(routed + shared) */
  for (int64_t b = 0; b < N; ++b)
    for (int col = 0; col < H; ++col) {
      double acc = 0.0;
      for (int k = 0; k < K; ++k) {
        const int64_t pos = perm[(int64_t)k * N + b];
        const float yv = (float)or_f16_to_double(ys[pos * H + col]);
        const float wv = (float)weights[b * K + k];
        acc += or_f16_to_double(or_f16_from_double((double)(yv * wv)));
      }
      double routed = or_f16_to_double(or_f16_from_double(acc));
      if (sh) routed += or_f16_to_double(sh[b * H + col]);
      out[b * H + col] = or_f16_from_double(routed);
    }
  free(sh);
  free(ys);
  free(se);
  return 0;
}

int or_moe_layer(const or_moe_cfg *cfg, const or_linear *experts, const or_linear *shared,
                 const uint16_t *router_w, const float *bias, const uint16_t *h, int64_t N,
                 uint16_t *out, int32_t *idx_out, double *w_out, int threads) {
  const int E = cfg->n_experts, K = cfg->top_k, H = cfg->hidden;
  double *logits = (double *)malloc(sizeof(double) * (size_t)(N * E));
  int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)(N * K));
  double *w = (double *)malloc(sizeof(double) * (size_t)(N * K));
  or_router_logits(h, N, router_w, E, H, logits);
  int rc = or_route(logits, bias, N, cfg, idx, w);
  if (rc == 0) rc = or_moe_layer_routed(cfg, experts, shared, h, N, idx, w, out, threads);
  if (idx_out) memcpy(idx_out, idx, sizeof(int32_t) * (size_t)(N * K));
  if (w_out) memcpy(w_out, w, sizeof(double) * (size_t)(N * K));
  free(logits);
  free(idx);
  free(w);
  return rc;
}

/* ------------------------------------------------------------------------- */
/* Hyper-connection prepare / mix and RMSNorm (glm5_hc.cpp:242-355,           */
/* glm5_attn.cpp:12-22).                                                       */
/* ------------------------------------------------------------------------- */

static double or_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

void or_hc_prepare(const uint16_t *streams, int64_t P, int N, int D, const float *fn,
                   const float *base, const float *scale, int iters, double eps,
                   uint16_t *collapsed, double *post, double *comb) {
  const int W = (2 + N) * N;
  const int64_t ND = (int64_t)N * D;
  double *w = (double *)malloc(sizeof(double) * (size_t)W);
  double *c = (double *)malloc(sizeof(double) * (size_t)N * N);
  double *pre = (double *)malloc(sizeof(double) * (size_t)N);
  for (int64_t p = 0; p < P; ++p) {
    const uint16_t *s = streams + p * ND;
    /* 300-301: unweighted RMSNorm over the N*D axis */
    double ss = 0.0;
    for (int64_t i = 0; i < ND; ++i) {
      const double v = or_f16_to_double(s[i]);
      ss += v * v;
    }
    const double rms = 1.0 / sqrt(ss / (double)ND + eps);
    /* 303: x @ fn^T, fn stored (out, in) */
    for (int j = 0; j < W; ++j) {
      double acc = 0.0;
      for (int64_t i = 0; i < ND; ++i) acc += or_f16_to_double(s[i]) * rms * (double)fn[(int64_t)j * ND + i];
      w[j] = acc;
    }
    /* 313-315 */
    for (int n = 0; n < N; ++n) {
      pre[n] = or_sigmoid(w[n] * scale[0] + base[n]) + eps;
      post[p * N + n] = 2.0 * or_sigmoid(w[N + n] * scale[1] + base[N + n]);
    }
    for (int i = 0; i < N; ++i) {
      double m = -INFINITY;
      for (int j = 0; j < N; ++j) {
        const double z = w[2 * N + i * N + j] * scale[2] + base[2 * N + i * N + j];
        c[i * N + j] = z;
        if (z > m) m = z;
      }
      double t = 0.0;
      for (int j = 0; j < N; ++j) {
        c[i * N + j] = exp(c[i * N + j] - m);
        t += c[i * N + j];
      }
      for (int j = 0; j < N; ++j) c[i * N + j] = c[i * N + j] / t + eps;
    }
    /* 321-324: Sinkhorn, sums over axis -2 (columns) then (iters-1) x (rows, columns) */
    for (int j = 0; j < N; ++j) {
      double cs = 0.0;
      for (int i = 0; i < N; ++i) cs += c[i * N + j];
      for (int i = 0; i < N; ++i) c[i * N + j] /= (cs + eps);
    }
    for (int it = 0; it < iters - 1; ++it) {
      for (int i = 0; i < N; ++i) {
        double rs = 0.0;
        for (int j = 0; j < N; ++j) rs += c[i * N + j];
        for (int j = 0; j < N; ++j) c[i * N + j] /= (rs + eps);
      }
      for (int j = 0; j < N; ++j) {
        double cs = 0.0;
        for (int i = 0; i < N; ++i) cs += c[i * N + j];
        for (int i = 0; i < N; ++i) c[i * N + j] /= (cs + eps);
      }
    }
    for (int k = 0; k < N * N; ++k) comb[p * N * N + k] = c[k];
    /* 328: collapsed = sum_n pre[n] * streams[n], in the streams' dtype */
    for (int d = 0; d < D; ++d) {
      double a = 0.0;
      for (int n = 0; n < N; ++n) a += pre[n] * or_f16_to_double(s[(int64_t)n * D + d]);
      collapsed[p * D + d] = or_f16_from_double(a);
    }
  }
  free(w);
  free(c);
  free(pre);
}

void or_rms_norm(const uint16_t *x, int64_t P, int D, const uint16_t *w, double eps, uint16_t *y) {
  for (int64_t p = 0; p < P; ++p) {
    double ss = 0.0;
    for (int d = 0; d < D; ++d) {
      const double v = or_f16_to_double(x[p * D + d]);
      ss += v * v;
    }
    const double r = 1.0 / sqrt(ss / (double)D + eps);
    for (int d = 0; d < D; ++d) {
      const double n = or_f16_to_double(or_f16_from_double(or_f16_to_double(x[p * D + d]) * r));
      y[p * D + d] = or_f16_from_double(n * or_f16_to_double(w[d]));
    }
  }
}

void or_hc_mix(const uint16_t *block_out, const double *post, const double *comb,
               const uint16_t *residual, int64_t P, int N, int D, uint16_t *out) {
  for (int64_t p = 0; p < P; ++p)
    for (int n = 0; n < N; ++n) {
      const double pn = or_f16_to_double(or_f16_from_double(post[p * N + n]));
      for (int d = 0; d < D; ++d) {
        const double a = or_f16_to_double(or_f16_from_double(pn * or_f16_to_double(block_out[p * D + d])));
        double r = 0.0;
        for (int m = 0; m < N; ++m)
          r += or_f16_to_double(or_f16_from_double(comb[(p * N + m) * N + n])) *
               or_f16_to_double(residual[(p * N + m) * (int64_t)D + d]);
        const double b = or_f16_to_double(or_f16_from_double(r));
        out[(p * N + n) * (int64_t)D + d] = or_f16_from_double(a + b);
      }
    }
}
