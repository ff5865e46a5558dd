/* CPU oracle for the MXFP4 matmul path — TEST INFRASTRUCTURE ONLY (see mxoracle.h). */
#include "mxoracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ rng */

/* crates/kern-test/src/workload.rs:18-24 */
uint64_t mxo_splitmix64_next(uint64_t* state) {
  *state += 0x9E3779B97F4A7C15ull;
  uint64_t z = *state;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t mxo_splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t s = seed + i * 0x9E3779B97F4A7C15ull;
  return mxo_splitmix64_next(&s);
}

double mxo_normal_at(uint64_t seed, uint64_t i) {
  double u1 = (double)(mxo_splitmix64_at(seed, 2 * i) >> 11) * 0x1p-53;
  double u2 = (double)(mxo_splitmix64_at(seed, 2 * i + 1) >> 11) * 0x1p-53;
  return sqrt(-2.0 * log(1.0 - u1)) * cos(2.0 * M_PI * u2);
}

/* --------------------------------------------------------------- codecs */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* probe.py:24 E2M1 = [0, .5, 1, 1.5, 2, 3, 4, 6]; probe.py:30 sign = bit 3 */
float mxo_e2m1_decode(uint8_t nibble) {
  static const float t[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  float v = t[nibble & 7];
  return (nibble & 8) ? -v : v;
}

/* values.rs:18-24: 255 is NaN, else 2^(c-127) */
float mxo_e8m0_decode(uint8_t code) {
  if (code == 255) return NAN;
  return (float)ldexp(1.0, (int)code - 127);
}

/* values.rs:117-135 */
uint8_t mxo_e8m0_encode(double v) {
  if (!isfinite(v) || v < 0.0) return 255;
  if (v <= ldexp(1.0, -127)) return 0;
  if (v >= ldexp(1.0, 127)) return 254;
  int e;
  double m = frexp(v, &e); /* v = m * 2^e, m in [0.5, 1) */
  (void)m;
  int exponent = e - 1; /* floor(log2 v) */
  uint8_t code = (uint8_t)(exponent + 127);
  double mid = 1.5 * ldexp(1.0, exponent);
  if (v > mid || (v == mid && (code % 2) != 0)) return (uint8_t)(code + 1);
  return code;
}

/* values.rs:81-89 */
float mxo_e4m3_decode(uint8_t b) {
  float sign = (b & 0x80) ? -1.f : 1.f;
  int exp = (b >> 3) & 0xf;
  int man = b & 7;
  if (exp == 0xf && man == 7) return NAN;
  if (exp == 0) return sign * (float)ldexp(man / 8.0, -6);
  return sign * (float)ldexp(1.0 + man / 8.0, exp - 7);
}

/* values.rs:91-113 (kept to document that its rounding is half away from zero) */
uint8_t mxo_e4m3_encode_values_rs(double v) {
  if (isnan(v)) return 0x7f;
  uint8_t sign = signbit(v) ? 0x80 : 0;
  double a = fmin(fabs(v), 448.0);
  if (a < ldexp(1.0, -9)) return sign;
  int exp = (int)floor(log2(a));
  if (exp < -6) {
    double man = round(a / ldexp(1.0, -6) * 8.0);
    uint8_t m = (uint8_t)man;
    return sign | (m > 7 ? 7 : m);
  }
  double man = round((a / ldexp(1.0, exp) - 1.0) * 8.0);
  if (man >= 8.0) { exp += 1; man = 0.0; }
  int e = exp + 7;
  if (e < 0) e = 0;
  if (e > 15) e = 15;
  uint8_t m = (uint8_t)man;
  if (e == 15 && m == 7) return sign | 0x7e;
  return sign | (uint8_t)(e << 3) | m;
}

/* RNE of an unsigned significand shifted right by s (s >= 1). */
static uint32_t rne_shift(uint32_t mant, int s) {
  if (s >= 32) return 0;
  uint32_t q = mant >> s;
  uint32_t rem = mant & ((1u << s) - 1u);
  uint32_t half = 1u << (s - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return q;
}

uint8_t mxo_e4m3_encode_rne(uint32_t bits, int shift) {
  uint8_t sign = (uint8_t)((bits >> 24) & 0x80);
  uint32_t a = bits & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7f;
  if (a == 0x7f800000u) return sign | 0x7e;
  if (a == 0) return sign;
  int E = (int)(a >> 23);
  uint32_t mant;
  int e;
  if (E == 0) { /* f32 subnormal: normalise */
    mant = a & 0x7fffffu;
    e = -126;
    while (!(mant & 0x800000u)) { mant <<= 1; e -= 1; }
  } else {
    mant = (a & 0x7fffffu) | 0x800000u;
    e = E - 127;
  }
  e += shift; /* value = mant * 2^(e - 23) */
  if (e >= -6) {
    uint32_t r = rne_shift(mant, 20); /* 4-bit significand, in [8, 16] */
    if (r == 16) { r = 8; e += 1; }
    int ef = e + 7;
    if (ef > 15 || (ef == 15 && r - 8 == 7)) return sign | 0x7e;
    return sign | (uint8_t)(ef << 3) | (uint8_t)(r - 8);
  }
  /* subnormal e4m3: units of 2^-9; value / 2^-9 = mant * 2^(e - 23 + 9) */
  int s = 14 - e; /* >= 21 */
  uint32_t q = rne_shift(mant, s); /* 0..8; 8 is the smallest normal (code 0x08) */
  return sign | (uint8_t)q;
}

float mxo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t mxo_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

uint8_t mxo_e4m3_from_f32(float v) { return mxo_e4m3_encode_rne(f2u(v), 0); }

void mxo_e4m3_from_f32_array(const float* v, int64_t n, uint8_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = mxo_e4m3_encode_rne(f2u(v[i]), 0);
}

void mxo_quant_blocks_f32(const float* v, int64_t nblocks, uint8_t* q, uint8_t* sf) {
  for (int64_t b = 0; b < nblocks; ++b) sf[b] = mxo_quant_block32_f32(v + 32 * b, q + 32 * b);
}

/* ------------------------------------------------------------ quantizer */

/* floor(log2 |x|) of a finite nonzero f32 given its bits */
static int floor_log2_bits(uint32_t a) {
  int E = (int)(a >> 23);
  if (E > 0) return E - 127;
  uint32_t m = a & 0x7fffffu;
  int p = 31 - __builtin_clz(m);
  return p - 149;
}

uint8_t mxo_quant_block32_f32(const float* v, uint8_t* q) {
  uint32_t amax = 0;
  int nonfinite = 0;
  for (int i = 0; i < 32; ++i) {
    uint32_t a = f2u(v[i]) & 0x7fffffffu;
    if (a >= 0x7f800000u) nonfinite = 1;
    if (a > amax) amax = a;
  }
  if (nonfinite) {
    for (int i = 0; i < 32; ++i) q[i] = (uint8_t)(((f2u(v[i]) >> 24) & 0x80) | 0x7f);
    return 255;
  }
  int code = 0;
  if (amax != 0) {
    code = floor_log2_bits(amax) - 8 + 127;
    if (code < 0) code = 0;
    if (code > 254) code = 254;
  }
  for (int i = 0; i < 32; ++i) q[i] = mxo_e4m3_encode_rne(f2u(v[i]), 127 - code);
  return (uint8_t)code;
}

void mxo_quant_mxfp8(const uint16_t* x, int64_t T, int64_t K, uint8_t* q, uint8_t* sf) {
  float blk[32];
  for (int64_t t = 0; t < T; ++t)
    for (int64_t b = 0; b < K / 32; ++b) {
      for (int i = 0; i < 32; ++i) blk[i] = mxo_bf16_to_f32(x[t * K + b * 32 + i]);
      sf[t * (K / 32) + b] = mxo_quant_block32_f32(blk, q + t * K + b * 32);
    }
}

/* --------------------------------------------------------------- repack */

int64_t mxo_w_src_row(int64_t R, int64_t rows, int gated) {
  if (!gated) return R;
  int64_t half = rows / 2;
  int64_t j = R % 4;
  int64_t n = 8 * (R / 16) + 2 * ((R % 16) / 4) + (j & 1);
  return j < 2 ? half + n : n; /* gate = second half (w1), up = first half (w3) */
}

int64_t mxo_w_offset(int64_t R, int64_t kbyte, int64_t rows, int64_t row_bytes) {
  (void)rows;
  int64_t KT = row_bytes / 64;
  int64_t kt = kbyte / 64, g = (kbyte % 64) / 16, b = kbyte % 16;
  return ((R / 16) * KT + kt) * 1024 + (16 * g + R % 16) * 16 + b;
}

int64_t mxo_sf_offset(int64_t R, int64_t kblock, int64_t rows, int64_t sf_cols) {
  (void)rows;
  int64_t KG = sf_cols / 16;
  int64_t kg = kblock / 16, j = (kblock % 16) / 4, g = kblock % 4;
  return ((R / 16) * KG + kg) * 256 + (16 * g + R % 16) * 4 + j;
}

void mxo_w_shuffle(const uint8_t* raw, uint8_t* out, int64_t E, int64_t rows, int64_t row_bytes, int gated) {
  int64_t per = rows * row_bytes;
  for (int64_t e = 0; e < E; ++e)
    for (int64_t R = 0; R < rows; ++R) {
      const uint8_t* src = raw + e * per + mxo_w_src_row(R, rows, gated) * row_bytes;
      for (int64_t kb = 0; kb < row_bytes; ++kb) out[e * per + mxo_w_offset(R, kb, rows, row_bytes)] = src[kb];
    }
}

void mxo_w_unshuffle(const uint8_t* in, uint8_t* raw, int64_t E, int64_t rows, int64_t row_bytes, int gated) {
  int64_t per = rows * row_bytes;
  for (int64_t e = 0; e < E; ++e)
    for (int64_t R = 0; R < rows; ++R) {
      uint8_t* dst = raw + e * per + mxo_w_src_row(R, rows, gated) * row_bytes;
      for (int64_t kb = 0; kb < row_bytes; ++kb) dst[kb] = in[e * per + mxo_w_offset(R, kb, rows, row_bytes)];
    }
}

void mxo_sf_shuffle(const uint8_t* raw, uint8_t* out, int64_t E, int64_t rows, int64_t sf_cols, int gated) {
  int64_t per = rows * sf_cols;
  for (int64_t e = 0; e < E; ++e)
    for (int64_t R = 0; R < rows; ++R) {
      const uint8_t* src = raw + e * per + mxo_w_src_row(R, rows, gated) * sf_cols;
      for (int64_t b = 0; b < sf_cols; ++b) out[e * per + mxo_sf_offset(R, b, rows, sf_cols)] = src[b];
    }
}

void mxo_sf_unshuffle(const uint8_t* in, uint8_t* raw, int64_t E, int64_t rows, int64_t sf_cols, int gated) {
  int64_t per = rows * sf_cols;
  for (int64_t e = 0; e < E; ++e)
    for (int64_t R = 0; R < rows; ++R) {
      uint8_t* dst = raw + e * per + mxo_w_src_row(R, rows, gated) * sf_cols;
      for (int64_t b = 0; b < sf_cols; ++b) dst[b] = in[e * per + mxo_sf_offset(R, b, rows, sf_cols)];
    }
}

int64_t mxo_r128c4_offset(int64_t r, int64_t b, int64_t kblocks) {
  int64_t kb4 = (kblocks + 3) / 4;
  return 512 * ((r / 128) * kb4 + b / 4) + (r % 32) * 16 + ((r % 128) / 32) * 4 + b % 4;
}

int64_t mxo_r128c4_size(int64_t rows, int64_t kblocks) { return ((rows + 127) / 128) * 512 * ((kblocks + 3) / 4); }

/* --------------------------------------------------------------- dequant */

void mxo_deq_fp4(const uint8_t* w, const uint8_t* sf, int64_t N, int64_t K, float* out) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      uint8_t byte = w[n * (K / 2) + k / 2];
      uint8_t nib = (k & 1) ? (byte >> 4) : (byte & 15);
      out[n * K + k] = mxo_e2m1_decode(nib) * mxo_e8m0_decode(sf[n * (K / 32) + k / 32]);
    }
}

void mxo_deq_fp8(const uint8_t* q, const uint8_t* sf, int64_t T, int64_t K, float* out) {
  for (int64_t t = 0; t < T; ++t)
    for (int64_t k = 0; k < K; ++k)
      out[t * K + k] = mxo_e4m3_decode(q[t * K + k]) * mxo_e8m0_decode(sf[t * (K / 32) + k / 32]);
}

/* ------------------------------------------------------- threaded helper */

typedef void (*row_fn)(void* ctx, int64_t lo, int64_t hi);
typedef struct { row_fn fn; void* ctx; int64_t lo, hi; } span_t;
static void* span_run(void* p) { span_t* s = (span_t*)p; s->fn(s->ctx, s->lo, s->hi); return NULL; }

static void parallel_rows(row_fn fn, void* ctx, int64_t n, int nthreads) {
  if (nthreads <= 1 || n < 2) { fn(ctx, 0, n); return; }
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  span_t sp[256];
  int64_t per = (n + nthreads - 1) / nthreads;
  int used = 0;
  for (int i = 0; i < nthreads; ++i) {
    int64_t lo = i * per, hi = lo + per < n ? lo + per : n;
    if (lo >= hi) break;
    sp[i].fn = fn; sp[i].ctx = ctx; sp[i].lo = lo; sp[i].hi = hi;
    pthread_create(&th[i], NULL, span_run, &sp[i]);
    used++;
  }
  for (int i = 0; i < used; ++i) pthread_join(th[i], NULL);
}

/* ------------------------------------------------------------------ GEMM */

typedef struct { const float *X, *W; int64_t T, N, K; float* C; } gemm_ctx;
static void gemm_rows(void* p, int64_t lo, int64_t hi) {
  gemm_ctx* c = (gemm_ctx*)p;
  for (int64_t t = lo; t < hi; ++t)
    for (int64_t n = 0; n < c->N; ++n) {
      const float* x = c->X + t * c->K;
      const float* w = c->W + n * c->K;
      float acc = 0.f;
      for (int64_t k = 0; k < c->K; ++k) acc += x[k] * w[k];
      c->C[t * c->N + n] = acc;
    }
}

void mxo_gemm_f32(const float* X, const float* W, int64_t T, int64_t N, int64_t K, float* C, int nthreads) {
  gemm_ctx c = {X, W, T, N, K, C};
  parallel_rows(gemm_rows, &c, T, nthreads);
}

typedef struct { const uint16_t* x; const uint8_t *w, *sf; int64_t M, N, K; uint16_t* y; float* yf; } gemv_ctx;
static void gemv_rows(void* p, int64_t lo, int64_t hi) {
  gemv_ctx* c = (gemv_ctx*)p;
  int64_t K = c->K;
  float* wrow = (float*)malloc(sizeof(float) * K);
  for (int64_t n = lo; n < hi; ++n) {
    for (int64_t k = 0; k < K; ++k) {
      uint8_t byte = c->w[n * (K / 2) + k / 2];
      uint8_t nib = (k & 1) ? (byte >> 4) : (byte & 15);
      wrow[k] = mxo_e2m1_decode(nib) * mxo_e8m0_decode(c->sf[n * (K / 32) + k / 32]);
    }
    for (int64_t t = 0; t < c->M; ++t) {
      float acc = 0.f;
      const uint16_t* x = c->x + t * K;
      for (int64_t k = 0; k < K; ++k) acc += mxo_bf16_to_f32(x[k]) * wrow[k];
      if (c->yf) c->yf[t * c->N + n] = acc;
      if (c->y) c->y[t * c->N + n] = mxo_f32_to_bf16(acc);
    }
  }
  free(wrow);
}

void mxo_gemv_w4a16(const uint16_t* x, const uint8_t* w, const uint8_t* sf, int64_t M, int64_t N, int64_t K,
                    uint16_t* y, float* y_f32, int nthreads) {
  gemv_ctx c = {x, w, sf, M, N, K, y, y_f32};
  parallel_rows(gemv_rows, &c, N, nthreads);
}

/* ------------------------------------------------------------ activations */

float mxo_situ(float g, float u, float alpha, float beta) {
  float sg = 1.0f / (1.0f + expf(-g));
  return alpha * tanhf(g / alpha) * sg * beta * tanhf(u / beta);
}

void mxo_silu_mul_bf16(const uint16_t* in, int64_t T, int64_t d, uint16_t* out) {
  for (int64_t t = 0; t < T; ++t)
    for (int64_t i = 0; i < d; ++i) {
      float g = mxo_bf16_to_f32(in[t * 2 * d + i]);
      float u = mxo_bf16_to_f32(in[t * 2 * d + d + i]);
      float s = mxo_bf16_to_f32(mxo_f32_to_bf16(g / (1.0f + expf(-g))));
      out[t * d + i] = mxo_f32_to_bf16(s * u);
    }
}

/* MoE finalize (tools/trtllm-bmm/probe.py:100-110: index_add of the weighted FC2 rows of each token):
 * y[t][h] = sum_j w[t][j] * fc2[e2p[t*topk + j]][h], j ascending, f32 fused multiply-adds, rows with
 * e2p < 0 (non-local experts) skipped. gamma == NULL: out = bf16(y). Otherwise the norm of op
 * moe_finalize_rms: out = bf16(y * (1 / sqrt(ss / H + eps)) * gamma), ss = sum of y^2 over the row in
 * column order (f32 FMAs). */
void mxo_moe_finalize(const uint16_t* fc2, const int32_t* e2p, const float* w, const uint16_t* gamma, int64_t T,
                      int64_t H, int topk, float eps, uint16_t* out) {
  float* y = (float*)malloc(sizeof(float) * (size_t)H);
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t h = 0; h < H; ++h) y[h] = 0.f;
    for (int j = 0; j < topk; ++j) {
      int32_t row = e2p[t * topk + j];
      float wj = w[t * topk + j];
      if (row < 0) continue;
      for (int64_t h = 0; h < H; ++h) y[h] = fmaf(wj, mxo_bf16_to_f32(fc2[(int64_t)row * H + h]), y[h]);
    }
    if (!gamma) {
      for (int64_t h = 0; h < H; ++h) out[t * H + h] = mxo_f32_to_bf16(y[h]);
      continue;
    }
    float ss = 0.f;
    for (int64_t h = 0; h < H; ++h) ss = fmaf(y[h], y[h], ss);
    float r = 1.0f / sqrtf(ss / (float)H + eps);
    for (int64_t h = 0; h < H; ++h) out[t * H + h] = mxo_f32_to_bf16(y[h] * r * mxo_bf16_to_f32(gamma[h]));
  }
  free(y);
}

/* weight_prep's RoPE cache (tools/kernels-src/weight_prep.cu:9-13, :37-47): inv = 1 / base^(2j/(2 half)),
 * angle = r * inv, all in f32, cos/sin rounded to bf16 at [r*stride + j]. */
void mxo_rope_table(uint16_t* cos_t, uint16_t* sin_t, int64_t rows, int64_t half, int64_t stride, float base) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t j = 0; j < half; ++j) {
      float inv = 1.0f / powf(base, (float)(2 * j) / (float)(2 * half));
      float angle = (float)r * inv;
      cos_t[r * stride + j] = mxo_f32_to_bf16(cosf(angle));
      sin_t[r * stride + j] = mxo_f32_to_bf16(sinf(angle));
    }
}

/* Linear [rows][kblocks] e8m0 scales from the 128x4 tiled layout (mxo_r128c4_offset). */
void mxo_r128c4_gather(const uint8_t* tiled, int64_t rows, int64_t kblocks, uint8_t* linear) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t b = 0; b < kblocks; ++b) linear[r * kblocks + b] = tiled[mxo_r128c4_offset(r, b, kblocks)];
}

/* --------------------------------------------------------------- routing */

int64_t mxo_max_ctas(int64_t tokens, int topk, int experts, int tile) {
  int64_t expanded = tokens * topk;
  int64_t filled = experts < expanded ? experts : expanded;
  return filled + (expanded - filled) / tile;
}

void mxo_routing(const int32_t* topk_idx, int64_t T, int topk, int local_start, int E_local, int tile,
                 int32_t* counts, int32_t* cta_batch, int32_t* cta_limit, int32_t* num_non_exiting,
                 int32_t* total_padded, int32_t* route_map, int32_t* exp2perm) {
  int64_t n = T * topk;
  for (int e = 0; e < 2 * E_local; ++e) counts[e] = 0;
  for (int64_t i = 0; i < n; ++i) {
    int e = topk_idx[i] - local_start;
    if (e >= 0 && e < E_local) counts[e]++;
  }
  int32_t slots = 0;
  for (int e = 0; e < E_local; ++e) {
    counts[E_local + e] = slots;
    int32_t ns = (counts[e] + tile - 1) / tile;
    for (int32_t s = 0; s < ns; ++s) {
      int32_t lim1 = (slots + s + 1) * tile;
      int32_t lim2 = slots * tile + counts[e];
      cta_batch[slots + s] = e;
      cta_limit[slots + s] = lim1 < lim2 ? lim1 : lim2;
    }
    slots += ns;
  }
  num_non_exiting[0] = slots;
  total_padded[0] = slots * tile;
  for (int64_t p = 0; p < (int64_t)slots * tile; ++p) route_map[p] = -1;
  int32_t* fill = (int32_t*)calloc((size_t)(E_local > 0 ? E_local : 1), sizeof(int32_t));
  for (int64_t i = 0; i < n; ++i) {
    int e = topk_idx[i] - local_start;
    if (e >= 0 && e < E_local) {
      int32_t p = counts[E_local + e] * tile + fill[e]++;
      exp2perm[i] = p;
      route_map[p] = (int32_t)(i / topk);
    } else {
      exp2perm[i] = -1;
    }
  }
  free(fill);
}

/* ------------------------------------------------------- grouped GEMMs */

/* dequantised repacked weight row R of one expert */
static void deq_repacked_row(const uint8_t* a, const uint8_t* sf_a, int64_t rows, int64_t k, int64_t R, float* out) {
  int64_t rb = k / 2, sc = k / 32;
  for (int64_t kk = 0; kk < k; ++kk) {
    uint8_t byte = a[mxo_w_offset(R, kk / 2, rows, rb)];
    uint8_t nib = (kk & 1) ? (byte >> 4) : (byte & 15);
    out[kk] = mxo_e2m1_decode(nib) * mxo_e8m0_decode(sf_a[mxo_sf_offset(R, kk / 32, rows, sc)]);
  }
}

static float dot_f32(const float* a, const float* b, int64_t k) {
  float acc = 0.f;
  for (int64_t i = 0; i < k; ++i) acc += a[i] * b[i];
  return acc;
}

typedef struct {
  const uint8_t *a, *sf_a, *b, *sf_b;
  int sf_b_r128c4;
  int64_t rows_b;
  uint16_t* c;
  float* acc_out;
  const int32_t *cta_batch, *cta_limit;
  int64_t m, k;
  int tile;
} fc2_ctx;

static void fc2_slots(void* p, int64_t lo, int64_t hi) {
  fc2_ctx* c = (fc2_ctx*)p;
  int64_t m = c->m, k = c->k;
  float* w = (float*)malloc(sizeof(float) * k);
  float* x = (float*)malloc(sizeof(float) * k * c->tile);
  for (int64_t s = lo; s < hi; ++s) {
    int64_t e = c->cta_batch[s];
    int64_t r0 = s * c->tile, r1 = c->cta_limit[s];
    const uint8_t* ae = c->a + e * m * (k / 2);
    const uint8_t* se = c->sf_a + e * m * (k / 32);
    for (int64_t pr = r0; pr < r1; ++pr)
      for (int64_t kk = 0; kk < k; ++kk) {
        int64_t so = c->sf_b_r128c4 ? mxo_r128c4_offset(pr, kk / 32, k / 32) : pr * (k / 32) + kk / 32;
        x[(pr - r0) * k + kk] = mxo_e4m3_decode(c->b[pr * k + kk]) * mxo_e8m0_decode(c->sf_b[so]);
      }
    for (int64_t n = 0; n < m; ++n) {
      deq_repacked_row(ae, se, m, k, n, w);
      for (int64_t pr = r0; pr < r1; ++pr) {
        float acc = dot_f32(x + (pr - r0) * k, w, k);
        if (c->acc_out) c->acc_out[pr * m + n] = acc;
        c->c[pr * m + n] = mxo_f32_to_bf16(acc);
      }
    }
  }
  free(w);
  free(x);
}

void mxo_fc2(const uint8_t* a, const uint8_t* sf_a, const uint8_t* b, const uint8_t* sf_b, int sf_b_r128c4,
             int64_t rows_b, uint16_t* c, float* acc_out, const int32_t* num_non_exiting,
             const int32_t* cta_batch, const int32_t* cta_limit, int64_t m, int64_t k, int tile, int nthreads) {
  fc2_ctx ctx = {a, sf_a, b, sf_b, sf_b_r128c4, rows_b, c, acc_out, cta_batch, cta_limit, m, k, tile};
  parallel_rows(fc2_slots, &ctx, num_non_exiting[0], nthreads);
}

typedef struct {
  const uint8_t *a, *sf_a, *b, *sf_b;
  uint8_t *c, *sf_c;
  int64_t padded_rows;
  const int32_t* route_map;
  const float *alpha, *beta;
  float* dbg;
  const int32_t *cta_batch, *cta_limit;
  int64_t m, k;
  int tile;
} fc1_ctx;

static void fc1_slots(void* p, int64_t lo, int64_t hi) {
  fc1_ctx* c = (fc1_ctx*)p;
  int64_t m = c->m, k = c->k, half = m / 2, tile = c->tile;
  float* wg = (float*)malloc(sizeof(float) * k);
  float* wu = (float*)malloc(sizeof(float) * k);
  float* x = (float*)malloc(sizeof(float) * k * tile);
  float* h = (float*)malloc(sizeof(float) * half * tile);
  for (int64_t s = lo; s < hi; ++s) {
    int64_t e = c->cta_batch[s];
    int64_t r0 = s * tile, r1 = c->cta_limit[s];
    const uint8_t* ae = c->a + e * m * (k / 2);
    const uint8_t* se = c->sf_a + e * m * (k / 32);
    for (int64_t pr = r0; pr < r1; ++pr) {
      int64_t tok = c->route_map[pr];
      for (int64_t kk = 0; kk < k; ++kk)
        x[(pr - r0) * k + kk] =
            mxo_e4m3_decode(c->b[tok * k + kk]) * mxo_e8m0_decode(c->sf_b[tok * (k / 32) + kk / 32]);
    }
    for (int64_t n = 0; n < half; ++n) {
      int64_t Rg = 16 * (n / 8) + 4 * ((n % 8) / 2) + (n % 2); /* gate row; the up row is Rg + 2 */
      deq_repacked_row(ae, se, m, k, Rg, wg);
      deq_repacked_row(ae, se, m, k, Rg + 2, wu);
      for (int64_t pr = r0; pr < r1; ++pr) {
        float g = dot_f32(x + (pr - r0) * k, wg, k), u = dot_f32(x + (pr - r0) * k, wu, k);
        float hv = mxo_situ(g, u, c->alpha[e], c->beta[e]);
        h[(pr - r0) * half + n] = hv;
        if (c->dbg) {
          c->dbg[(pr * 3 + 0) * half + n] = g;
          c->dbg[(pr * 3 + 1) * half + n] = u;
          c->dbg[(pr * 3 + 2) * half + n] = hv;
        }
      }
    }
    for (int64_t pr = r0; pr < r1; ++pr)
      for (int64_t blk = 0; blk < half / 32; ++blk)
        c->sf_c[mxo_r128c4_offset(pr, blk, half / 32)] =
            mxo_quant_block32_f32(h + (pr - r0) * half + blk * 32, c->c + pr * half + blk * 32);
  }
  free(wg); free(wu); free(x); free(h);
}

void mxo_fc1(const uint8_t* a, const uint8_t* sf_a, const uint8_t* b, const uint8_t* sf_b, uint8_t* c,
             uint8_t* sf_c, int64_t padded_rows, const int32_t* route_map, const float* alpha, const float* beta,
             float* dbg, const int32_t* num_non_exiting, const int32_t* cta_batch, const int32_t* cta_limit,
             int64_t m, int64_t k, int tile, int nthreads) {
  fc1_ctx ctx = {a, sf_a, b, sf_b, c, sf_c, padded_rows, route_map, alpha, beta, dbg, cta_batch, cta_limit, m, k, tile};
  parallel_rows(fc1_slots, &ctx, num_non_exiting[0], nthreads);
}

typedef struct {
  const uint8_t *a, *sf_a, *b, *sf_b;
  int64_t T, m, k;
  float d_scale;
  uint8_t* c;
  float* acc_out;
} pt_ctx;

static void pt_rows(void* p, int64_t lo, int64_t hi) {
  pt_ctx* c = (pt_ctx*)p;
  int64_t m = c->m, k = c->k;
  float* x = (float*)malloc(sizeof(float) * k);
  float* w = (float*)malloc(sizeof(float) * k * 16);
  for (int64_t n0 = 0; n0 < m; n0 += 16) {
    for (int i = 0; i < 16; ++i) deq_repacked_row(c->a, c->sf_a, m, k, n0 + i, w + i * k);
    for (int64_t t = lo; t < hi; ++t) {
      for (int64_t kk = 0; kk < k; ++kk)
        x[kk] = mxo_e4m3_decode(c->b[t * k + kk]) * mxo_e8m0_decode(c->sf_b[t * (k / 32) + kk / 32]);
      for (int i = 0; i < 16; ++i) {
        float acc = dot_f32(x, w + i * k, k);
        if (c->acc_out) c->acc_out[t * m + n0 + i] = acc;
        c->c[t * m + n0 + i] = mxo_e4m3_from_f32(acc * c->d_scale);
      }
    }
  }
  free(x);
  free(w);
}

void mxo_gemm_e4m3_pt(const uint8_t* a, const uint8_t* sf_a, const uint8_t* b, const uint8_t* sf_b, int64_t T,
                      int64_t m, int64_t k, float d_scale, uint8_t* c, float* acc_out, int nthreads) {
  pt_ctx ctx = {a, sf_a, b, sf_b, T, m, k, d_scale, c, acc_out};
  parallel_rows(pt_rows, &ctx, T, nthreads);
}
