/*
 * cpu_ref.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the arithmetic of laya-js' CPU backend
 * (backend-cpu, a re-export of the un-vendored npm module
 * @johnhenry/math-plus-tensor-cpu@0.3.0 / math-plus-tensor-core@0.2.1, see
 * packages/backend-cpu/src/index.ts:12-15) for the ops on the ModernBERT
 * encoder path, plus the quantized-format producer of
 * packages/laya/src/quant.ts.  Storage is f32; GEMMs and reductions
 * accumulate in f64 ("packed f64 panels", backend-cpu/src/index.ts:12-13).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker / the timed CPU baseline.  The
 * product (laya-js_amd/) never links or calls it.
 *
 * Parity pins (each checked by tests/test_oracle.py):
 *   linear        ops.json linear/{bias,nobias}; brute-force numpy f64 dot
 *   layernorm     ops.json layerNorm/{wb,w,none}; numpy closed form
 *   rope          ops.json rope/base{10000,160000}; rotation-norm invariant
 *   sdpa          ops.json sdpa/{full,sliding,nomask}; uniform-attention
 *                 closed form (q = 0 gives the masked mean of v)
 *   gelu/geglu    ops.json gelu/erf, geglu; libm erf values from
 *                 backend-cpu/test/backend.test.ts:56-73
 *   embedding     ops.json embedding
 *   meanpool      ops.json meanPool
 *   dequant       ops-quantized.json (20 quantizedLinear + 6
 *                 quantizedEmbedding cases)
 *   quantize      laya/test/quant.test.ts invariants: range-fit error
 *                 <= scale/2, refit never increases squared error, the
 *                 exact 16-level nibble layout, all-zero rows
 *   masks         ops.json sdpa masks (window 16), as
 *                 modernbert/test/modernbert.test.ts:52-63 does
 *   encoder       tiny activations.json, every stage at 1e-5
 *   f16 / bf16    every binary16 pattern decoded as numpy does and rounded
 *                 back to itself; every bfloat16 pattern unchanged, halfway
 *                 points to even, one ulp either side to the nearer value,
 *                 overflow to inf; torch's bfloat16 RNE on random values
 *   f16 storage   encoder_forward(dtype="f16"): layer 0 equals the pinned
 *                 ops composed with an f16 rounding after each, bit for
 *                 bit; every stage f16-valued and within 2e-2 of the tiny
 *                 activations
 *   decision head (cpu_ref.py) tiny activations.json type_emb_added,
 *                 head.layers.0/1, logits and act at 1e-5; masked logits
 *                 exactly -1e4
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ f16 */

/* Round-to-nearest-even double -> IEEE binary16 bits (subnormals, overflow to
 * inf).  JS `Float16Array` stores follow this rule (laya/src/quant.ts:79-81). */
uint16_t cr_f64_to_f16(double x) {
  uint16_t sign = 0;
  if (signbit(x)) { sign = 0x8000; x = -x; }
  if (isnan(x)) return sign | 0x7e00;
  if (isinf(x)) return sign | 0x7c00;
  if (x == 0.0) return sign;
  int e;
  double m = frexp(x, &e); /* x = m * 2^e, m in [0.5, 1) */
  /* binary16: normal exponent range e-1 in [-14, 15] */
  int exp16 = e - 1;
  if (exp16 < -14) {
    /* subnormal: value = n * 2^-24 */
    double n = ldexp(x, 24);
    double r = nearbyint(n); /* default rounding mode is to-nearest-even */
    if (r >= 1024.0) return sign | 0x0400; /* rounds up to the smallest normal */
    return sign | (uint16_t)r;
  }
  /* normal: significand with 10 fraction bits */
  double sig = ldexp(m, 11); /* in [1024, 2048) */
  double r = nearbyint(sig);
  if (r >= 2048.0) { r = 1024.0; exp16 += 1; }
  if (exp16 > 15) return sign | 0x7c00;
  return sign | (uint16_t)((exp16 + 15) << 10) | ((uint16_t)r - 1024);
}

double cr_f16_to_f64(uint16_t h) {
  int s = h >> 15, e = (h >> 10) & 31, f = h & 1023;
  double v;
  if (e == 0) v = ldexp((double)f, -24);
  else if (e == 31) v = f ? NAN : INFINITY;
  else v = ldexp((double)(f + 1024), e - 25);
  return s ? -v : v;
}

/* Round-to-nearest-even f32 -> bf16 bits (tensor-backend/src/host.ts:63-69). */
uint16_t cr_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  return (uint16_t)(((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) & 0xffffu);
}

/* Rounds an f32 array through f16 (or bf16) storage and back, in place. */
void cr_round_f16(float* x, int64_t n) {
  for (int64_t i = 0; i < n; i++) x[i] = (float)cr_f16_to_f64(cr_f64_to_f16((double)x[i]));
}
void cr_round_bf16(float* x, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    uint32_t u = (uint32_t)cr_f32_to_bf16(x[i]) << 16;
    memcpy(&x[i], &u, 4);
  }
}
void cr_f16_bits_to_f32(const uint16_t* h, float* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = (float)cr_f16_to_f64(h[i]);
}
void cr_f32_to_f16_bits(const float* x, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) out[i] = cr_f64_to_f16((double)x[i]);
}

int cr_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ------------------------------------------------------------------ linear */

/* Sum of the four lanes. */
static inline double hsum4(__m256d v) {
  __m128d lo = _mm256_castpd256_pd128(v), hi = _mm256_extractf128_pd(v, 1);
  lo = _mm_add_pd(lo, hi);
  return _mm_cvtsd_f64(_mm_add_sd(lo, _mm_unpackhi_pd(lo, lo)));
}

/* Dot products of up to 4 rows of a with up to 4 rows of b (f64, length K):
 * out[r][c] = sum_k a[r][k] b[c][k], accumulated in four f64 lanes over k
 * (k mod 4), then the lanes and the k tail in order.  Rows past ra / cb
 * alias row 0 and are not stored. */
static void dot4x4(const double* const* a, int ra, const double* const* b, int cb, int64_t K, double out[4][4]) {
  __m256d acc[4][4];
  for (int r = 0; r < 4; r++)
    for (int c = 0; c < 4; c++) acc[r][c] = _mm256_setzero_pd();
  int64_t k = 0;
  for (; k + 4 <= K; k += 4) {
    __m256d av[4], bv[4];
    for (int r = 0; r < 4; r++) av[r] = _mm256_loadu_pd(a[r] + k);
    for (int c = 0; c < 4; c++) bv[c] = _mm256_loadu_pd(b[c] + k);
    for (int r = 0; r < 4; r++)
      for (int c = 0; c < 4; c++) acc[r][c] = _mm256_fmadd_pd(av[r], bv[c], acc[r][c]);
  }
  for (int r = 0; r < ra; r++)
    for (int c = 0; c < cb; c++) {
      double v = hsum4(acc[r][c]);
      for (int64_t t = k; t < K; t++) v += a[r][t] * b[c][t];
      out[r][c] = v;
    }
}

/* y[M,N] = x[M,K] . w[N,K]^T (+ b[N]); f64 accumulation (every f32 product
 * is exact in f64), one f32 rounding.  Backend.linear,
 * tensor-backend/src/index.ts:211-215. */
void cr_linear(const float* x, const float* w, const float* b, float* y, int64_t M, int64_t N, int64_t K) {
  double* wd = (double*)malloc(sizeof(double) * (size_t)(N * K + 1));
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < N * K; i++) wd[i] = (double)w[i];
  const int64_t RB = 4;
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t r0 = 0; r0 < M; r0 += RB) {
    int ra = (int)(r0 + RB < M ? RB : M - r0);
    double* xd = (double*)malloc(sizeof(double) * (size_t)(RB * K + 1));
    const double* xr[4];
    for (int r = 0; r < 4; r++) {
      xr[r] = xd + (r < ra ? r : 0) * K;
      if (r < ra)
        for (int64_t k = 0; k < K; k++) xd[r * K + k] = (double)x[(r0 + r) * K + k];
    }
    for (int64_t n0 = 0; n0 < N; n0 += 4) {
      int cb = (int)(n0 + 4 < N ? 4 : N - n0);
      const double* wr[4];
      for (int c = 0; c < 4; c++) wr[c] = wd + (n0 + (c < cb ? c : 0)) * K;
      double out[4][4];
      dot4x4(xr, ra, wr, cb, K, out);
      for (int r = 0; r < ra; r++)
        for (int c = 0; c < cb; c++) y[(r0 + r) * N + n0 + c] = (float)(out[r][c] + (b ? (double)b[n0 + c] : 0.0));
    }
    free(xd);
  }
  free(wd);
}

/* ------------------------------------------------------------------ norms */

/* LayerNorm over the last axis, two-pass f64 statistics; w and b may be NULL.
 * Backend.layerNorm, tensor-backend/src/index.ts:216-217. */
void cr_layernorm(const float* x, const float* w, const float* b, float* y, int64_t rows, int64_t D, double eps) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    const float* xr = x + r * D;
    double mean = 0, var = 0;
    for (int64_t i = 0; i < D; i++) mean += xr[i];
    mean /= (double)D;
    for (int64_t i = 0; i < D; i++) { double d = xr[i] - mean; var += d * d; }
    var /= (double)D;
    double rstd = 1.0 / sqrt(var + eps);
    for (int64_t i = 0; i < D; i++) {
      double v = (xr[i] - mean) * rstd;
      if (w) v *= (double)w[i];
      if (b) v += (double)b[i];
      y[r * D + i] = (float)v;
    }
  }
}

/* ------------------------------------------------------------------ rope */

/* cos/sin tables [L, D/2] under the f32 angle rule the CPU backend uses
 * (restated in packages/backend-webgpu/src/backend.ts:1185-1195):
 * inv_i = f32(2^f32(-f32(i/half) * f32(log2 base))), theta = f32(l * inv_i),
 * cos/sin evaluated in f64 and stored as f32. */
void cr_rope_table(int64_t L, int64_t D, double base, float* cosT, float* sinT) {
  int64_t half = D / 2;
  float lb = (float)log2(base);
  for (int64_t i = 0; i < half; i++) {
    float frac = (float)((double)i / (double)half);
    float ex = (float)(-(double)frac * (double)lb);
    float inv = (float)exp2((double)ex);
    for (int64_t l = 0; l < L; l++) {
      float th = (float)((double)l * (double)inv);
      cosT[l * half + i] = (float)cos((double)th);
      sinT[l * half + i] = (float)sin((double)th);
    }
  }
}

/* Split-half (NeoX) rotary embedding on x [BH, L, D] contiguous, positions
 * 0..L-1.  Backend.rope, tensor-backend/src/index.ts:225-229. */
void cr_rope(const float* x, float* y, int64_t BH, int64_t L, int64_t D, double base) {
  int64_t half = D / 2;
  float* c = (float*)malloc(sizeof(float) * (size_t)(L * half));
  float* s = (float*)malloc(sizeof(float) * (size_t)(L * half));
  cr_rope_table(L, D, base, c, s);
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < BH * L; r++) {
    int64_t l = r % L;
    const float* xr = x + r * D;
    float* yr = y + r * D;
    for (int64_t i = 0; i < half; i++) {
      double cc = c[l * half + i], ss = s[l * half + i];
      double x0 = xr[i], x1 = xr[i + half];
      yr[i] = (float)(x0 * cc - x1 * ss);
      yr[i + half] = (float)(x0 * ss + x1 * cc);
    }
  }
  free(c);
  free(s);
}

/* ------------------------------------------------------------------ sdpa */

/* softmax(q k^T * scale, masked) v for q [B,H,Lq,D], k/v [B,H,Lk,D]
 * (contiguous) and a bool mask addressed by element strides ms[4] over
 * [B,H,Lq,Lk] (0 = broadcast; mask NULL = no mask).  f64 softmax.
 * Backend.sdpa, tensor-backend/src/index.ts:230-237. */
void cr_sdpa(const float* q, const float* k, const float* v, const uint8_t* mask, const int64_t* ms, float* o,
             int64_t B, int64_t H, int64_t Lq, int64_t Lk, int64_t D, double scale) {
  const int64_t nkv = B * H * Lk * D;
  double* kd = (double*)malloc(sizeof(double) * (size_t)(nkv + 1));
  double* vd = (double*)malloc(sizeof(double) * (size_t)(nkv + 1));
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < nkv; t++) {
    kd[t] = (double)k[t];
    vd[t] = (double)v[t];
  }
#pragma omp parallel for schedule(static) collapse(2)
  for (int64_t bh = 0; bh < B * H; bh++) {
    for (int64_t i = 0; i < Lq; i++) {
      int64_t bb = bh / H, hh = bh % H;
      const float* qi = q + (bh * Lq + i) * D;
      double* p = (double*)malloc(sizeof(double) * (size_t)(Lk + 2 * D + 8));
      int64_t* vis = (int64_t*)malloc(sizeof(int64_t) * (size_t)(Lk + 1));
      double* qd = p + Lk;   /* q row in f64 */
      double* acc = qd + D;  /* output row accumulator */
      for (int64_t d = 0; d < D; d++) qd[d] = (double)qi[d];
      int64_t nv = 0;
      for (int64_t j = 0; j < Lk; j++) {
        p[j] = -INFINITY;
        if (!mask || mask[bb * ms[0] + hh * ms[1] + i * ms[2] + j * ms[3]]) vis[nv++] = j;
      }
      const double* qa[4] = {qd, qd, qd, qd};
      double mx = -INFINITY;
      for (int64_t t = 0; t < nv; t += 4) {  /* four visible keys at a time */
        int cb = (int)(t + 4 < nv ? 4 : nv - t);
        const double* ka[4];
        for (int c = 0; c < 4; c++) ka[c] = kd + (bh * Lk + vis[t + (c < cb ? c : 0)]) * D;
        double s[4][4];
        dot4x4(qa, 1, ka, cb, D, s);
        for (int c = 0; c < cb; c++) {
          double sc = s[0][c] * scale;
          p[vis[t + c]] = sc;
          if (sc > mx) mx = sc;
        }
      }
      double sum = 0;
      for (int64_t j = 0; j < Lk; j++) { p[j] = p[j] == -INFINITY ? 0.0 : exp(p[j] - mx); sum += p[j]; }
      /* sum_j p_j v_j, in key order for every d */
      for (int64_t d = 0; d < D; d++) acc[d] = 0.0;
      for (int64_t j = 0; j < Lk; j++) {
        if (p[j] == 0.0) continue;
        const double pj = p[j];
        const double* vj = vd + (bh * Lk + j) * D;
        for (int64_t d = 0; d < D; d++) acc[d] += pj * vj[d];
      }
      for (int64_t d = 0; d < D; d++) o[(bh * Lq + i) * D + d] = (float)(acc[d] / sum);
      free(vis);
      free(p);
    }
  }
  free(kd);
  free(vd);
}

/* ------------------------------------------------------------------ gelu */

/* Exact-erf GELU 0.5 x (1 + erf(x / sqrt 2)) in f64 (Backend.gelu,
 * tensor-backend/src/index.ts:197-198). */
void cr_gelu(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    double v = x[i];
    y[i] = (float)(0.5 * v * (1.0 + erf(v / sqrt(2.0))));
  }
}

void cr_erf(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; i++) y[i] = (float)erf((double)x[i]);
}

/* gelu(value) * gate with [value, gate] = split(x, 2, -1)
 * (compose.ts:86-93); x [rows, 2F] -> y [rows, F]. */
void cr_geglu(const float* x, float* y, int64_t rows, int64_t F) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t j = 0; j < F; j++) {
      double v = x[r * 2 * F + j], g = x[r * 2 * F + F + j];
      double gl = (double)(float)(0.5 * v * (1.0 + erf(v / sqrt(2.0))));
      y[r * F + j] = (float)(gl * g);
    }
  }
}

/* ------------------------------------------------------------------ gathers */

/* Row gather table [V, D] by ids [n] -> out [n, D] (Backend.embedding). */
void cr_embedding(const float* table, int64_t V, int64_t D, const int32_t* ids, int64_t n, float* out) {
  for (int64_t r = 0; r < n; r++) {
    int64_t id = ids[r];
    if (id < 0) id = 0;
    if (id >= V) id = V - 1;
    memcpy(out + r * D, table + id * D, sizeof(float) * (size_t)D);
  }
}

/* Masked mean over axis 1 in f64: x [B,L,D], mask [B,L] -> [B,D]; an empty
 * row divides by max(n, 1) (compose.ts:96-105). */
void cr_meanpool(const float* x, const uint8_t* mask, int64_t B, int64_t L, int64_t D, float* out) {
  for (int64_t b = 0; b < B; b++) {
    double n = 0;
    for (int64_t l = 0; l < L; l++) n += mask[b * L + l] ? 1 : 0;
    if (n < 1) n = 1;
    for (int64_t d = 0; d < D; d++) {
      double s = 0;
      for (int64_t l = 0; l < L; l++) if (mask[b * L + l]) s += x[(b * L + l) * D + d];
      out[b * D + d] = (float)(s / n);
    }
  }
}

/* ------------------------------------------------------------------ quantized */

/* Compose-layout dequantization (compose.ts:379-398): q values [R, K] as
 * integers, scales/biases [R, G] as f32; w = f32(f32(q * s) + b), the two
 * f32 roundings the composed mul + add perform. */
void cr_dequant_compose(const int32_t* q, const float* scales, const float* biases, int64_t R, int64_t K, int64_t group,
                        float* out) {
  int64_t G = (K + group - 1) / group;
  for (int64_t r = 0; r < R; r++) {
    for (int64_t j = 0; j < K; j++) {
      float s = scales[r * G + j / group];
      float v = (float)q[r * K + j] * s;
      if (biases) v = v + biases[r * G + j / group];
      out[r * K + j] = v;
    }
  }
}

/* Host dequantization as laya's loader does it (quant.ts:189-243):
 * fl16(q * s + b) rounded once from the exact value. */
void cr_dequant_exact_f16(const int32_t* q, const float* scales, const float* biases, int64_t R, int64_t K, int64_t group,
                          uint16_t* out) {
  int64_t G = (K + group - 1) / group;
  for (int64_t r = 0; r < R; r++) {
    for (int64_t j = 0; j < K; j++) {
      double v = (double)q[r * K + j] * (double)scales[r * G + j / group];
      if (biases) v += (double)biases[r * G + j / group];
      out[r * K + j] = cr_f64_to_f16(v);
    }
  }
}

/* JS Math.round: nearest integer, ties toward +inf (quant.ts:139). */
static double js_round(double x) {
  double f = floor(x);
  return (x - f >= 0.5) ? f + 1.0 : f;
}

static double to_f16(double x) { return cr_f16_to_f64(cr_f64_to_f16(x)); }

/* quant.ts:135-146 */
static double q_assign(const double* w, int32_t* q, int64_t n, double s, double b, int qmin, int qmax) {
  double err = 0;
  int ok = s > 0 && isfinite(s);
  for (int64_t k = 0; k < n; k++) {
    double v = ok ? js_round((w[k] - b) / s) : 0;
    v = v < qmin ? qmin : v > qmax ? qmax : v;
    q[k] = (int32_t)v;
    double d = w[k] - (v * (ok ? s : 0) + b);
    err += d * d;
  }
  return err;
}

/* quant.ts:148-165 */
static void fit_symmetric(const double* w, int32_t* cur, int32_t* best, int64_t n, int steps, double* os, double* ob) {
  double amax = 0;
  for (int64_t k = 0; k < n; k++) amax = fmax(amax, fabs(w[k]));
  double s = to_f16(amax / 127);
  double bestErr = q_assign(w, best, n, s, 0, -127, 127), bestS = s;
  for (int it = 0; it < steps; it++) {
    double num = 0, den = 0;
    for (int64_t k = 0; k < n; k++) { num += best[k] * w[k]; den += (double)best[k] * best[k]; }
    if (den == 0) break;
    s = to_f16(num / den);
    double err = q_assign(w, cur, n, s, 0, -127, 127);
    if (!(err < bestErr)) break;
    bestErr = err; bestS = s;
    memcpy(best, cur, sizeof(int32_t) * (size_t)n);
  }
  *os = bestS;
  *ob = 0;
}

/* quant.ts:167-187 */
static void fit_affine(const double* w, int32_t* cur, int32_t* best, int64_t n, int steps, double* os, double* ob) {
  double lo = INFINITY, hi = -INFINITY;
  for (int64_t k = 0; k < n; k++) { lo = fmin(lo, w[k]); hi = fmax(hi, w[k]); }
  double b = to_f16(lo), s = to_f16((hi - b) / 15);
  double bestErr = q_assign(w, best, n, s, b, 0, 15), bestS = s, bestB = b;
  for (int it = 0; it < steps; it++) {
    double sq = 0, sw = 0, sqq = 0, sqw = 0;
    for (int64_t k = 0; k < n; k++) {
      sq += best[k]; sw += w[k]; sqq += (double)best[k] * best[k]; sqw += best[k] * w[k];
    }
    double den = (double)n * sqq - sq * sq;
    if (den == 0) break;
    s = to_f16(((double)n * sqw - sq * sw) / den);
    b = to_f16((sw - s * sq) / (double)n);
    double err = q_assign(w, cur, n, s, b, 0, 15);
    if (!(err < bestErr)) break;
    bestErr = err; bestS = s; bestB = b;
    memcpy(best, cur, sizeof(int32_t) * (size_t)n);
  }
  *os = bestS;
  *ob = bestB;
}

/* quantizeMatrix (quant.ts:96-129): values [rows, cols] -> q [rows, cols]
 * (int32), scales/biases [rows, cols/group] as f16 bits.  Returns 0, or -1
 * on a bad shape.  refine_steps = 8 for the q4 default, 0 for q8. */
int cr_quantize_matrix(const float* values, int64_t rows, int64_t cols, int bits, int64_t group, int refine_steps,
                       int32_t* q, uint16_t* scales, uint16_t* biases) {
  if ((bits != 8 && bits != 4) || group <= 0 || cols % group) return -1;
  if (bits == 4 && (cols % 2 || group % 2)) return -1;
  int64_t G = cols / group;
  double* w = (double*)malloc(sizeof(double) * (size_t)group);
  int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)group);
  int32_t* best = (int32_t*)malloc(sizeof(int32_t) * (size_t)group);
  for (int64_t r = 0; r < rows; r++) {
    for (int64_t gi = 0; gi < G; gi++) {
      int64_t start = r * cols + gi * group;
      for (int64_t k = 0; k < group; k++) w[k] = (double)values[start + k];
      double s, b;
      if (bits == 8) fit_symmetric(w, cur, best, group, refine_steps, &s, &b);
      else fit_affine(w, cur, best, group, refine_steps, &s, &b);
      scales[r * G + gi] = cr_f64_to_f16(s);
      if (bits == 4 && biases) biases[r * G + gi] = cr_f64_to_f16(b);
      memcpy(q + start, best, sizeof(int32_t) * (size_t)group);
    }
  }
  free(w); free(cur); free(best);
  return 0;
}

/* ------------------------------------------------------------------ masks */

/* attentionMasks (modernbert/src/index.ts:240-259): full [B,L] = valid;
 * sliding [B,L,L] = (|i-j| <= window/2 OR query i padded) AND valid[j]. */
void cr_attention_masks(const uint8_t* valid, int64_t B, int64_t L, int64_t window, uint8_t* full, uint8_t* sliding) {
  int64_t half = window / 2;
  for (int64_t b = 0; b < B; b++) {
    for (int64_t j = 0; j < L; j++) full[b * L + j] = valid[b * L + j] ? 1 : 0;
    for (int64_t i = 0; i < L; i++) {
      int padq = !valid[b * L + i];
      for (int64_t j = 0; j < L; j++) {
        int64_t d = i > j ? i - j : j - i;
        sliding[(b * L + i) * L + j] = full[b * L + j] && (padq || d <= half) ? 1 : 0;
      }
    }
  }
}
