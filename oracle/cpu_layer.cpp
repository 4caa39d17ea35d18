/*
 * CPU baseline of the EXL3 MoE layer -- MEASUREMENT INFRASTRUCTURE ONLY.
 *
 * bench.py's cpu_baseline leg times this next to the GPU; tests/ check it against the
 * oracle. The product (exl3-server_amd/) never loads it.
 *
 * The same layer as or_moe_layer (reference glm5_moe.cpp:112-417), computed the way a
 * fast CPU implementation would: f32 arithmetic with the reference's f16 rounding
 * points, AVX2/FMA/F16C, one worker thread per core pulling work items from an atomic
 * counter (the scheme of the reference's util.h:55-74), and on-the-fly codebook decode
 * through a 65536-entry value table, as the reference's CPU decode does (exl3.cpp:101-107).
 *
 * Identity with the oracle, where it is required (weights and routing):
 *  - the value table is the oracle's (or_codebook_lut), and the ring window / tile
 *    permutation are the oracle's formulas (or_tile_state, or_tile_perm), so cpu_decode
 *    is bit-identical to or_decode_inner (checked by tests and by bench.py);
 *  - router logits are f64 sums in the oracle's order (compiled without contraction,
 *    so bit-identical to or_router_logits), and selection and dispatch are the oracle's
 *    own or_route / or_moe_runs.
 * The expert GEMVs accumulate in f32 (the oracle in f64), so outputs agree within the
 * layer tolerance, not bit for bit.
 */
#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

extern "C" {
#include "exl3_oracle.h"
}

namespace {

// ---------------------------------------------------------------------------------
// A persistent pool: run(n, fn) calls fn(0..n-1) on the workers and the caller.
// ---------------------------------------------------------------------------------
class Pool {
 public:
  ~Pool() { stop_workers(); }

  void run(int threads, int64_t n, const std::function<void(int64_t)> &fn) {
    if (threads <= 1 || n <= 1) {
      for (int64_t i = 0; i < n; ++i) fn(i);
      return;
    }
    std::lock_guard<std::mutex> call(call_mu_);  // one job at a time
    ensure(threads - 1);
    {
      std::lock_guard<std::mutex> l(mu_);
      fn_ = &fn;
      n_ = n;
      next_.store(0);
      active_ = (int)workers_.size();
      ++gen_;
    }
    cv_.notify_all();
    drain();
    std::unique_lock<std::mutex> l(mu_);
    done_.wait(l, [&] { return active_ == 0; });
  }

 private:
  void ensure(int n) {
    if ((int)workers_.size() == n) return;
    stop_workers();
    stop_ = false;
    for (int i = 0; i < n; ++i) workers_.emplace_back([this, g = gen_] { loop(g); });
  }
  void stop_workers() {
    {
      std::lock_guard<std::mutex> l(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto &t : workers_) t.join();
    workers_.clear();
  }
  void loop(uint64_t seen) {
    for (;;) {
      {
        std::unique_lock<std::mutex> l(mu_);
        cv_.wait(l, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
      }
      drain();
      std::lock_guard<std::mutex> l(mu_);
      if (--active_ == 0) done_.notify_one();
    }
  }
  void drain() {
    for (;;) {
      const int64_t i = next_.fetch_add(1);
      if (i >= n_) return;
      (*fn_)(i);
    }
  }

  std::mutex call_mu_, mu_;
  std::condition_variable cv_, done_;
  std::vector<std::thread> workers_;
  const std::function<void(int64_t)> *fn_ = nullptr;
  int64_t n_ = 0;
  std::atomic<int64_t> next_{0};
  int active_ = 0;
  uint64_t gen_ = 0;
  bool stop_ = false;
};

Pool &pool() {
  static Pool p;
  return p;
}

// ---------------------------------------------------------------------------------
// f16 helpers (F16C: hardware RNE conversions, subnormals included)
// ---------------------------------------------------------------------------------
inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
inline uint16_t f2h(float f) { return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }
inline float f16r(float f) { return h2f(f2h(f)); }

constexpr float kHadScale = 1.0f / 11.313708498984761f;

// Tables: codebook values as f32 (the oracle's f16 values), tile permutation.
struct Tables {
  float lut[3][65536];
  uint16_t perm[256];
  Tables() {
    std::vector<uint16_t> l(65536);
    for (int cb = 0; cb < 3; ++cb) {
      or_codebook_lut(cb, l.data());
      for (int s = 0; s < 65536; ++s) lut[cb][s] = h2f(l[s]);
    }
    for (int p = 0; p < 256; ++p) perm[p] = (uint16_t)or_tile_perm(p);
  }
};

const Tables &tables() {
  static const Tables *t = new Tables();
  return *t;
}

// One 16x16 tile: w[k * 16 + n] for the tile's 8K ring words (MSB first; position p's
// state is the 16 ring bits ending at bit (p + 1) * K). ext[0] holds the last ring word
// so that the windows of the first positions wrap.
inline void decode_tile(const uint16_t *tw, int K, const float *lut, const uint16_t *perm, float *w) {
  uint32_t ext[8 * 8 + 1];
  const int nw = 8 * K;
  for (int i = 0; i < nw; ++i) ext[i + 1] = (uint32_t)tw[2 * i] | ((uint32_t)tw[2 * i + 1] << 16);
  ext[0] = ext[nw];
  for (int p = 0; p < 256; ++p) {
    const int lb = (p + 1) * K + 31;  // the state's last bit, in ext's bit numbering
    const int j = lb >> 5;
    const uint64_t pair = ((uint64_t)ext[j - 1] << 32) | ext[j];
    w[perm[p]] = lut[(uint16_t)(pair >> (31 - (lb & 31)))];
  }
}

void fwht128(float *x) {
  for (int len = 1; len < 128; len <<= 1)
    for (int i = 0; i < 128; i += 2 * len)
      for (int j = i; j < i + len; ++j) {
        const float a = x[j], b = x[j + len];
        x[j] = a + b;
        x[j + len] = a - b;
      }
}

// xhat = f16(fwht(f32(x) * f32(s)) / sqrt(128)) as f32 values; x given as f32 f16-values.
void had_pre(const float *x, int n, const uint16_t *s, float *xhat) {
  float buf[128];
  for (int b = 0; b < n / 128; ++b) {
    for (int t = 0; t < 128; ++t) buf[t] = x[b * 128 + t] * h2f(s[b * 128 + t]);
    fwht128(buf);
    for (int t = 0; t < 128; ++t) xhat[b * 128 + t] = f16r(buf[t] * kHadScale);
  }
}

// y = f16((fwht(f32(f16(yhat))) / sqrt(128)) * f32(s)) as f32 values.
void had_post(const float *yhat, int n, const uint16_t *s, float *y) {
  float buf[128];
  for (int b = 0; b < n / 128; ++b) {
    for (int t = 0; t < 128; ++t) buf[t] = f16r(yhat[b * 128 + t]);
    fwht128(buf);
    for (int t = 0; t < 128; ++t) y[b * 128 + t] = f16r((buf[t] * kHadScale) * h2f(s[b * 128 + t]));
  }
}

constexpr int kColBlock = 64;  // output columns per work item (4 tiles)
constexpr int kMaxRows = 16;   // rows per accumulator block

// yhat[r][c] for columns [c0, c0 + 64) of a trellis linear, rows x[r] (f32, stride in).
void trellis_cols(const or_linear &L, const float *x, int64_t rows, int c0, float *y, int64_t ystride) {
  const Tables &T = tables();
  const float *lut = T.lut[L.cb];
  const int tiles_n = L.out / 16, tiles_k = L.in / 16;
  alignas(32) float w[256];
  for (int64_t r0 = 0; r0 < rows; r0 += kMaxRows) {
    const int nr = (int)std::min<int64_t>(kMaxRows, rows - r0);
    for (int tn = c0 / 16; tn < (c0 + kColBlock) / 16 && tn < tiles_n; ++tn) {
      __m256 acc[kMaxRows][2];
      for (int r = 0; r < nr; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
      for (int tk = 0; tk < tiles_k; ++tk) {
        decode_tile(L.trellis + ((int64_t)tk * tiles_n + tn) * 16 * L.K, L.K, lut, T.perm, w);
        for (int r = 0; r < nr; ++r) {
          const float *xr = x + (r0 + r) * L.in + tk * 16;
          __m256 a0 = acc[r][0], a1 = acc[r][1];
          for (int k = 0; k < 16; ++k) {
            const __m256 xv = _mm256_set1_ps(xr[k]);
            a0 = _mm256_fmadd_ps(xv, _mm256_load_ps(w + k * 16), a0);
            a1 = _mm256_fmadd_ps(xv, _mm256_load_ps(w + k * 16 + 8), a1);
          }
          acc[r][0] = a0;
          acc[r][1] = a1;
        }
      }
      for (int r = 0; r < nr; ++r) {
        _mm256_storeu_ps(y + (r0 + r) * ystride + tn * 16, acc[r][0]);
        _mm256_storeu_ps(y + (r0 + r) * ystride + tn * 16 + 8, acc[r][1]);
      }
    }
  }
}

// The same columns of a plain f16 linear (dense (in, out) row-major), rounded to f16.
void dense_cols(const or_linear &L, const float *x, int64_t rows, int c0, float *y, int64_t ystride) {
  const int c1 = std::min(c0 + kColBlock, L.out);
  for (int64_t r0 = 0; r0 < rows; r0 += kMaxRows) {
    const int nr = (int)std::min<int64_t>(kMaxRows, rows - r0);
    for (int c = c0; c < c1; c += 16) {
      __m256 acc[kMaxRows][2];
      for (int r = 0; r < nr; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
      for (int k = 0; k < L.in; ++k) {
        const uint16_t *wr = L.dense + (int64_t)k * L.out + c;
        const __m256 w0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)wr));
        const __m256 w1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(wr + 8)));
        for (int r = 0; r < nr; ++r) {
          const __m256 xv = _mm256_set1_ps(x[(r0 + r) * L.in + k]);
          acc[r][0] = _mm256_fmadd_ps(xv, w0, acc[r][0]);
          acc[r][1] = _mm256_fmadd_ps(xv, w1, acc[r][1]);
        }
      }
      for (int r = 0; r < nr; ++r) {
        alignas(32) float t[16];
        _mm256_store_ps(t, acc[r][0]);
        _mm256_store_ps(t + 8, acc[r][1]);
        for (int i = 0; i < 16; ++i) y[(r0 + r) * ystride + c + i] = f16r(t[i]);
      }
    }
  }
}

inline int col_blocks(int out) { return (out + kColBlock - 1) / kColBlock; }

// silu(min(g, L)) * clamp(u, -L, L), each op rounded to f16 (glm5_moe.cpp:66-74).
inline float swiglu(float g, float u, float L) {
  if (g > L) g = L;
  if (u < -L) u = -L;
  if (u > L) u = L;
  const float sig = f16r(1.0f / (1.0f + std::exp(-g)));
  return f16r(f16r(g * sig) * u);
}

// One expert (or the shared expert) applied to n rows: the buffers of its part of the
// call. Trellis projections take Hadamard-rotated inputs; plain ones the rows as they are.
struct Unit {
  const or_linear *lin;  // gate, up, down
  int64_t n;             // rows
  const float *x;        // (n, H) f32 input rows (f16 values)
  float *xg, *xu;        // (n, H) rotated inputs for gate / up (trellis) -- or unused
  float *yg, *yu;        // (n, I) gate / up GEMV outputs (raw for trellis, f16 for dense)
  float *xd;             // (n, I) down input (rotated for trellis)
  float *yd;             // (n, H) down GEMV output
  float *y;              // (n, H) the unit's f16 output values
};

}  // namespace

extern "C" {

/* Decode a trellis tensor through the baseline's table and ring window (bit-identical
 * to or_decode_inner by construction; tests check it). w_hat (in, out) f16. */
int cpu_decode(const uint16_t *trellis, int64_t in, int64_t out, int K, int cb, uint16_t *w_hat, int threads) {
  if (in <= 0 || out <= 0 || in % 16 || out % 16 || K < 1 || K > 8 || cb < 0 || cb > 2) return -1;
  const Tables &T = tables();
  const int64_t tiles_n = out / 16;
  pool().run(threads, (in / 16) * tiles_n, [&](int64_t t) {
    alignas(32) float w[256];
    decode_tile(trellis + t * 16 * K, K, T.lut[cb], T.perm, w);
    const int64_t tk = t / tiles_n, tn = t % tiles_n;
    for (int k = 0; k < 16; ++k)
      for (int c = 0; c < 16; ++c) w_hat[(tk * 16 + k) * out + tn * 16 + c] = f2h(w[k * 16 + c]);
  });
  return 0;
}

/* Router logits in f64 in the oracle's summation order, over the pool. */
void cpu_router_logits(const uint16_t *h, int64_t N, const uint16_t *router_w, int E, int H, double *logits,
                       int threads) {
  pool().run(threads, N * E, [&](int64_t i) {
    const int64_t t = i / E, e = i % E;
    double acc = 0.0;
    for (int k = 0; k < H; ++k) acc += (double)h2f(h[t * H + k]) * (double)h2f(router_w[e * H + k]);
    logits[i] = acc;
  });
}

/* The layer: routing (f64, the oracle's selection and dispatch), then every expert
 * product in f32 over the pool. Same arguments as or_moe_layer; idx_out optional. */
int cpu_moe_layer(const or_moe_cfg *cfg, const or_linear *experts, const or_linear *shared, const uint16_t *router_w,
                  const float *bias, const uint16_t *h, int64_t N, uint16_t *out, int32_t *idx_out, int threads) {
  const int E = cfg->n_experts, K = cfg->top_k, H = cfg->hidden;
  const int64_t P = N * K;
  if (N <= 0 || H % 128) return -1;
  std::vector<double> logits((size_t)(N * E)), wts((size_t)P);
  std::vector<int32_t> idx((size_t)P), se((size_t)P * 7);
  cpu_router_logits(h, N, router_w, E, H, logits.data(), threads);
  if (or_route(logits.data(), bias, N, cfg, idx.data(), wts.data())) return -1;
  int32_t *sr = se.data() + P, *sk = se.data() + 2 * P, *perm = se.data() + 3 * P, *re = se.data() + 4 * P,
          *ro = se.data() + 5 * P, *rl = se.data() + 6 * P;
  const int runs = or_moe_runs(idx.data(), N, K, se.data(), sr, sk, perm, re, ro, rl);
  if (idx_out) std::memcpy(idx_out, idx.data(), sizeof(int32_t) * (size_t)P);

  // units: the runs in sorted-pair order, then the shared expert over all N rows
  const bool has_shared = shared && cfg->has_shared;
  const int64_t I = cfg->inter, SI = has_shared ? shared[0].out : 0;
  const int64_t rows_all = P + (has_shared ? N : 0);
  const int64_t Imax = std::max<int64_t>(I, SI);
  std::vector<float> xs((size_t)(rows_all * H)), xg((size_t)(rows_all * H)), xu((size_t)(rows_all * H));
  std::vector<float> yg((size_t)(rows_all * Imax)), yu((size_t)(rows_all * Imax)), xd((size_t)(rows_all * Imax));
  std::vector<float> yd((size_t)(rows_all * H)), ys((size_t)(rows_all * H));
  std::vector<Unit> units;
  for (int r = 0; r < runs + (has_shared ? 1 : 0); ++r) {
    const bool sh = r == runs;
    const int64_t off = sh ? P : ro[r], n = sh ? N : rl[r];
    Unit u{sh ? shared : &experts[3 * (int64_t)re[r]], n, &xs[off * H], &xg[off * H], &xu[off * H],
           &yg[off * Imax], &yu[off * Imax], &xd[off * Imax], &yd[off * H], &ys[off * H]};
    for (int64_t i = 0; i < n; ++i) {
      const int64_t row = sh ? i : sr[off + i];
      for (int c = 0; c < H; ++c) xs[(off + i) * H + c] = h2f(h[row * H + c]);
    }
    units.push_back(u);
  }
  const int U = (int)units.size();
  auto width = [&](const Unit &u) { return u.lin[0].out; };
  // rotated inputs of gate and up, per (unit, projection)
  pool().run(threads, 2 * (int64_t)U, [&](int64_t t) {
    const Unit &u = units[t / 2];
    const or_linear &L = u.lin[t % 2];
    if (!L.trellis) return;
    float *dst = t % 2 ? u.xu : u.xg;
    for (int64_t i = 0; i < u.n; ++i) had_pre(u.x + i * H, H, L.suh, dst + i * H);
  });
  // gate / up GEMVs, per (unit, projection, 64-column block)
  std::vector<int64_t> first(U + 1, 0);
  for (int i = 0; i < U; ++i) first[i + 1] = first[i] + 2 * col_blocks(width(units[i]));
  pool().run(threads, first[U], [&](int64_t t) {
    int i = 0;
    while (first[i + 1] <= t) ++i;
    const Unit &u = units[i];
    const int64_t j = t - first[i], nb = col_blocks(width(u));
    const int proj = (int)(j / nb), c0 = (int)(j % nb) * kColBlock;
    const or_linear &L = u.lin[proj];
    float *y = proj ? u.yu : u.yg;
    if (L.trellis)
      trellis_cols(L, proj ? u.xu : u.xg, u.n, c0, y, Imax);
    else
      dense_cols(L, u.x, u.n, c0, y, Imax);
  });
  // SwiGLU and the down projection's rotated input, per unit
  pool().run(threads, U, [&](int64_t t) {
    const Unit &u = units[t];
    const int w = width(u);
    const float Lim = f16r(cfg->swiglu_limit);
    std::vector<float> g(w), v(w), a(w);
    for (int64_t i = 0; i < u.n; ++i) {
      if (u.lin[0].trellis) {
        had_post(u.yg + i * Imax, w, u.lin[0].svh, g.data());
        had_post(u.yu + i * Imax, w, u.lin[1].svh, v.data());
      } else {
        std::memcpy(g.data(), u.yg + i * Imax, sizeof(float) * w);
        std::memcpy(v.data(), u.yu + i * Imax, sizeof(float) * w);
      }
      for (int c = 0; c < w; ++c) a[c] = swiglu(g[c], v[c], Lim);
      if (u.lin[2].trellis)
        had_pre(a.data(), w, u.lin[2].suh, u.xd + i * Imax);
      else
        std::memcpy(u.xd + i * Imax, a.data(), sizeof(float) * w);
    }
  });
  // down GEMVs, per (unit, 64-column block)
  const int nbh = col_blocks(H);
  pool().run(threads, (int64_t)U * nbh, [&](int64_t t) {
    const Unit &u = units[t / nbh];
    const int c0 = (int)(t % nbh) * kColBlock;
    const or_linear &L = u.lin[2];
    if (L.trellis)
      trellis_cols(L, u.xd, u.n, c0, u.yd, H);
    else
      dense_cols(L, u.xd, u.n, c0, u.yd, H);
  });
  pool().run(threads, U, [&](int64_t t) {
    const Unit &u = units[t];
    for (int64_t i = 0; i < u.n; ++i) {
      if (u.lin[2].trellis)
        had_post(u.yd + i * H, H, u.lin[2].svh, u.y + i * H);
      else
        std::memcpy(u.y + i * H, u.yd + i * H, sizeof(float) * H);
    }
  });
  // combine: f16(sum_k f16(y_k * w_k)) + shared, per (row, column block)
  pool().run(threads, N * nbh, [&](int64_t t) {
    const int64_t b = t / nbh;
    const int c0 = (int)(t % nbh) * kColBlock, c1 = std::min(c0 + kColBlock, H);
    for (int c = c0; c < c1; ++c) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k) {
        const int64_t pos = perm[(int64_t)k * N + b];
        acc += f16r(ys[pos * H + c] * (float)wts[b * K + k]);
      }
      float routed = f16r(acc);
      if (has_shared) routed += ys[(P + b) * H + c];
      out[b * H + c] = f2h(routed);
    }
  });
  return 0;
}

}  // extern "C"
