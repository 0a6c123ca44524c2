/* CPU oracle: plain-C restatement of the reference qpack x86 CPU path for the Llama token loop.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT (see oracle.h).  Built by oracle/Makefile into oracle/liboracle.so.
 *
 * Pinning (what checks each part; the tests live in tests/test_oracle.py):
 *   - f16 conversion, quantisation, int32 block / group sums: closed forms and brute force in numpy (exact integers);
 *   - rows_q8 / rows_q4 / matvec / matmul / rmsnorm / exp / silu: bit-identical to the reference compiled from its own
 *     sources (oracle/_ref/libqpref.so) on seeded inputs, and to golden vectors in tests/golden/;
 *   - the full model (step / prefill / greedy): bit-identical logits and identical greedy streams against
 *     oracle/_ref/libqpref.so on seeded synthetic QPACK2 files, and against the golden fixtures;
 *   - the rANS codec: byte-identical blobs to the reference encoder and identical decodes of the reference's blobs
 *     (oracle/_ref/libqpref.so), golden blobs in tests/golden/, and the round trip decode(encode(x)) == x.
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

void or_set_threads(int n) { if (n > 0) omp_set_num_threads(n); }

/* Evaluation-order variants (OR_ORD_* bits, 0 = the reference's orders).  They exist to measure which float-order
 * difference between the HIP path and the reference decides a greedy token: each bit swaps one reference order for the
 * HIP path's (or, for attention, for float64 arithmetic standing in for "another order"). */
static int g_order = 0;
void or_set_order(int flags) { g_order = flags; }

/* ------------------------------------------------------------------ fp16 */
uint16_t or_f32_to_f16(float f) {
  uint32_t x; memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 rounds to infinity */
  if (ax < 0x38800000u) {                                     /* below 2^-14: subnormal half, unit 2^-24 */
    const int e = (int)(ax >> 23);
    if (e < 102) return (uint16_t)sign;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u; const int sh = 126 - e;
    uint32_t q = m >> sh; const uint32_t rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t h = (ax - (112u << 23)) >> 13; const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}
float or_f16_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u; uint32_t m = h & 1023u, f;
  if (e == 0) {
    if (!m) f = s;
    else { int e2 = -1; do { e2++; m <<= 1; } while (!(m & 1024u)); m &= 1023u; f = s | ((uint32_t)(127 - 15 - e2) << 23) | (m << 13); }
  } else if (e == 31) f = s | 0x7f800000u | (m << 13);
  else f = s | ((e + 112u) << 23) | (m << 13);
  float r; memcpy(&r, &f, 4); return r;
}

/* hsum256 (/root/reference/src/kernels_x86.cpp:18-21): ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)) */
static float hsum8(const float v[8]) {
  const float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
  return (a0 + a2) + (a1 + a3);
}

/* ------------------------------------------------------------------ activation quantisation */
/* quant_rows for one row (/root/reference/src/kernels.cpp:17-31): per 128-column block mx = max |x|,
 * isx = mx > 0 ? 32767 / mx : 0, scale = mx / 32767, q = lrintf(x * isx) */
void or_quant_act(const float *x, int cols, int16_t *xq, float *bs) {
  const int nb = (cols + OR_QB - 1) / OR_QB;
  for (int k = 0; k < nb; k++) {
    const int c0 = k * OR_QB, c1 = c0 + OR_QB < cols ? c0 + OR_QB : cols; float mx = 0;
    for (int c = c0; c < c1; c++) { const float a = fabsf(x[c]); if (mx < a) mx = a; }
    const float isx = mx > 0 ? OR_ACT_MAX / mx : 0.f; bs[k] = mx / OR_ACT_MAX;
    for (int c = c0; c < c1; c++) xq[c] = (int16_t)lrintf(x[c] * isx);
  }
}

/* ------------------------------------------------------------------ integer accumulators */
void or_block_sums_q8(const int8_t *Q, int rows, int cols, const int16_t *xq, int32_t *out) {
  const int nb = cols / OR_QB;
  #pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++)
    for (int b = 0; b < nb; b++) {
      const int8_t *q = Q + (int64_t)r * cols + b * OR_QB; const int16_t *x = xq + b * OR_QB; int32_t s = 0;
      for (int c = 0; c < OR_QB; c++) s += (int32_t)q[c] * (int32_t)x[c];
      out[(int64_t)r * nb + b] = s;
    }
}
/* q4 group g of 16 bytes: byte j = column j (low nibble) and column j + 16 (high nibble), each stored as q + 8
 * (/root/reference/src/kernels_x86.cpp:73-80, QPACK2.md table) */
void or_group_sums_q4(const uint8_t *Q, int rows, int cols, const int16_t *xq, int32_t *out) {
  const int G = cols / 32;
  #pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++)
    for (int g = 0; g < G; g++) {
      const uint8_t *q = Q + (int64_t)r * (cols / 2) + 16 * g; const int16_t *x = xq + 32 * g; int32_t s = 0;
      for (int j = 0; j < 16; j++) s += ((int32_t)(q[j] & 15) - 8) * x[j] + ((int32_t)(q[j] >> 4) - 8) * x[j + 16];
      out[(int64_t)r * G + g] = s;
    }
}

/* ------------------------------------------------------------------ row kernels */
/* rows_q8 (kernels_x86.cpp:55-71): per block an exact int32 sum, acc = fma(bs[b], (float)isum, acc) in block order,
 * y = acc * scale[r]; columns past the last full block: tail = fma(q, x, tail), acc = fma(bs[nb], tail, acc) */
static float row_q8(const int8_t *q, float scale, const int16_t *xq, const float *bs, int cols) {
  const int nb = cols / OR_QB; float acc = 0;
  for (int b = 0; b < nb; b++) {
    int32_t s = 0; const int8_t *qb = q + b * OR_QB; const int16_t *xb = xq + b * OR_QB;
    for (int c = 0; c < OR_QB; c++) s += (int32_t)qb[c] * xb[c];
    acc = fmaf(bs[b], (float)s, acc);
  }
  if (nb * OR_QB < cols) {
    float tail = 0; for (int c = nb * OR_QB; c < cols; c++) tail = fmaf((float)q[c], (float)xq[c], tail);
    acc = fmaf(bs[nb], tail, acc);
  }
  return acc * scale;
}
void or_rows_q8(const int8_t *Q, const float *scale, const int16_t *xq, const float *bs, float *y, int rows, int cols) {
  #pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++) y[r] = row_q8(Q + (int64_t)r * cols, scale[r], xq, bs, cols);
}
/* the int32 value of AVX2 lane l (0..7) of one q4 group: columns 2l, 2l+1 (low nibbles) and 16+2l, 17+2l (high
 * nibbles) -- _mm256_madd_epi16 pairs (kernels_x86.cpp:89-91) */
static int32_t q4_lane(const uint8_t *g16, const int16_t *x, int l) {
  const uint8_t b0 = g16[2 * l], b1 = g16[2 * l + 1];
  return ((int32_t)(b0 & 15) - 8) * x[2 * l] + ((int32_t)(b1 & 15) - 8) * x[2 * l + 1] +
         ((int32_t)(b0 >> 4) - 8) * x[16 + 2 * l] + ((int32_t)(b1 >> 4) - 8) * x[17 + 2 * l];
}
/* rows_q4 (kernels_x86.cpp:81-106): comb[g] = f16(s[g]) * bs[g >> 2]; 8-lane accumulators, even groups -> a0,
 * odd groups -> a1 (an odd last group -> a0), lane = fma((float)lane_sum, comb, lane); y = hsum(a0 + a1) */
static float row_q4(const uint8_t *q, const uint16_t *s, const int16_t *xq, const float *bs, int cols) {
  const int G = cols / 32; float a0[8] = {0}, a1[8] = {0}, t[8];
  int k = 0;
  for (; k + 2 <= G; k += 2) {
    const float c0 = or_f16_to_f32(s[k]) * bs[k >> 2], c1 = or_f16_to_f32(s[k + 1]) * bs[(k + 1) >> 2];
    for (int l = 0; l < 8; l++) {
      a0[l] = fmaf((float)q4_lane(q + 16 * k, xq + 32 * k, l), c0, a0[l]);
      a1[l] = fmaf((float)q4_lane(q + 16 * k + 16, xq + 32 * k + 32, l), c1, a1[l]);
    }
  }
  for (; k < G; k++) {
    const float c0 = or_f16_to_f32(s[k]) * bs[k >> 2];
    for (int l = 0; l < 8; l++) a0[l] = fmaf((float)q4_lane(q + 16 * k, xq + 32 * k, l), c0, a0[l]);
  }
  for (int l = 0; l < 8; l++) t[l] = a0[l] + a1[l];
  return hsum8(t);
}
void or_rows_q4(const uint8_t *Q, const uint16_t *S, const int16_t *xq, const float *bs, float *y, int rows, int cols) {
  const int G = cols / 32;
  #pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++) y[r] = row_q4(Q + (int64_t)r * (cols / 2), S + (int64_t)r * G, xq, bs, cols);
}
/* q1 (kernels_x86.cpp:167-203): column 128g + c of a row is bit c (LSB first) of the group's 16 bytes, +1 when set,
 * -1 when clear.  row_q1_nt: lane l (of 8) of group g sums columns 16i + 2l and 16i + 2l + 1 (i = 0..7) exactly;
 * f_l = fma((float)lane, f16(scale_g) * bs[g], f_l); y = hsum(f).  A partial last group reads activations past cols
 * as 0. */
static int q1_sign(const uint8_t *g16, int c) { return (g16[c >> 3] >> (c & 7)) & 1 ? 1 : -1; }
static float row_q1(const uint8_t *q, const uint16_t *s, const int16_t *xq, const float *bs, int cols) {
  const int G = (cols + 127) / 128; float f[8] = {0};
  for (int g = 0; g < G; g++) {
    const float cb = or_f16_to_f32(s[g]) * bs[g];
    for (int l = 0; l < 8; l++) {
      int32_t a = 0;
      for (int i = 0; i < 8; i++)
        for (int t = 0; t < 2; t++) {
          const int c = 16 * i + 2 * l + t, col = 128 * g + c;
          a += q1_sign(q + 16 * g, c) * (col < cols ? (int32_t)xq[col] : 0);
        }
      f[l] = fmaf((float)a, cb, f[l]);
    }
  }
  return hsum8(f);
}
void or_rows_q1(const uint8_t *Q, const uint16_t *S, const int16_t *xq, const float *bs, float *y, int rows, int cols) {
  const int G = (cols + 127) / 128;
  #pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++) y[r] = row_q1(Q + (int64_t)r * G * 16, S + (int64_t)r * G, xq, bs, cols);
}
void or_group_sums_q1(const uint8_t *Q, int rows, int cols, const int16_t *xq, int32_t *out) {
  const int G = (cols + 127) / 128;
  for (int r = 0; r < rows; r++)
    for (int g = 0; g < G; g++) {
      int32_t a = 0;
      for (int c = 0; c < 128 && 128 * g + c < cols; c++) a += q1_sign(Q + ((int64_t)r * G + g) * 16, c) * xq[128 * g + c];
      out[(int64_t)r * G + g] = a;
    }
}

/* rows_f32 (kernels_x86.cpp:26-38): four 8-lane FMA accumulators over 32-column steps, hsum of their sum, scalar tail */
static float row_f32(const float *w, const float *x, int cols) {
  float a[4][8] = {{0}}; int c = 0;
  for (; c + 32 <= cols; c += 32)
    for (int u = 0; u < 4; u++) for (int l = 0; l < 8; l++) a[u][l] = fmaf(w[c + 8 * u + l], x[c + 8 * u + l], a[u][l]);
  float t[8]; for (int l = 0; l < 8; l++) t[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
  float s = hsum8(t); for (; c < cols; c++) s = fmaf(w[c], x[c], s);
  return s;
}

void or_matvec(const or_mat *W, const float *x, float *y) {
  const int rows = W->rows, cols = W->cols;
  if (W->kind == OR_F32) {
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) y[r] = row_f32((const float *)W->q + (int64_t)r * cols, x, cols);
    return;
  }
  const int nb = (cols + OR_QB - 1) / OR_QB;
  int16_t *xq = (int16_t *)malloc(sizeof(int16_t) * (size_t)cols); float *bs = (float *)malloc(sizeof(float) * (size_t)nb);
  or_quant_act(x, cols, xq, bs);
  if (W->kind == OR_Q8) or_rows_q8((const int8_t *)W->q, (const float *)W->s, xq, bs, y, rows, cols);
  else if (W->kind == OR_Q1) or_rows_q1((const uint8_t *)W->q, (const uint16_t *)W->s, xq, bs, y, rows, cols);
  else or_rows_q4((const uint8_t *)W->q, (const uint16_t *)W->s, xq, bs, y, rows, cols);
  free(xq); free(bs);
}

/* mm_q8 lane arithmetic (kernels_x86.cpp:287-334) for one (row, vector) with vector index < B - B % 4: lane l of a
 * 128-column block sums columns 16s + 2l, 16s + 2l + 1 (s = 0..7); f_l = fma((float)lane, bs[block], f_l);
 * y = hsum(f) * scale */
static float mm_row_q8(const int8_t *q, float scale, const int16_t *xq, const float *bs, int cols) {
  const int nb = cols / OR_QB; float f[8] = {0};
  for (int k = 0; k < nb; k++) {
    for (int l = 0; l < 8; l++) {
      int32_t a = 0;
      for (int s = 0; s < 8; s++) {
        const int c = k * OR_QB + 16 * s + 2 * l;
        a += (int32_t)q[c] * xq[c] + (int32_t)q[c + 1] * xq[c + 1];
      }
      f[l] = fmaf((float)a, bs[k], f[l]);
    }
  }
  return hsum8(f) * scale;
}
/* mm_q4 lane arithmetic (kernels_x86.cpp:345-371) for vector index < B - B % 4: one 8-lane accumulator over all groups,
 * comb = f16(s[g]) * bs[g >> 2]; y = hsum(f) */
static float mm_row_q4(const uint8_t *q, const uint16_t *s, const int16_t *xq, const float *bs, int cols) {
  const int G = cols / 32; float f[8] = {0};
  for (int k = 0; k < G; k++) {
    const float cb = or_f16_to_f32(s[k]) * bs[k >> 2];
    for (int l = 0; l < 8; l++) f[l] = fmaf((float)q4_lane(q + 16 * k, xq + 32 * k, l), cb, f[l]);
  }
  return hsum8(f);
}
/* matmul (kernels.cpp:97-143) without ExactBatches: B == 1 -> matvec; otherwise every vector quantised, the vectors
 * [0, B - B % 4) take the tiled lane arithmetic and the rest the row kernel (kernels_x86.cpp:313, :334, :368) */
void or_matmul(const or_mat *W, const float *X, int B, float *Y) {
  const int rows = W->rows, cols = W->cols;
  if (B == 1) { or_matvec(W, X, Y); return; }
  if (W->kind == OR_F32) { for (int b = 0; b < B; b++) or_matvec(W, X + (size_t)b * cols, Y + (size_t)b * rows); return; }
  const int nb = (cols + OR_QB - 1) / OR_QB, B4 = B - B % 4;
  int16_t *xq = (int16_t *)malloc(sizeof(int16_t) * (size_t)B * cols); float *bs = (float *)malloc(sizeof(float) * (size_t)B * nb);
  for (int b = 0; b < B; b++) or_quant_act(X + (size_t)b * cols, cols, xq + (size_t)b * cols, bs + (size_t)b * nb);
  #pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++)
    for (int b = 0; b < B; b++) {
      const int16_t *xb = xq + (size_t)b * cols; const float *sb = bs + (size_t)b * nb; float v;
      if (W->kind == OR_Q8) {
        const int8_t *q = (const int8_t *)W->q + (int64_t)r * cols; const float sc = ((const float *)W->s)[r];
        v = (b < B4 && cols % OR_QB == 0 && !(g_order & OR_ORD_ROWS_PREFILL)) ? mm_row_q8(q, sc, xb, sb, cols) : row_q8(q, sc, xb, sb, cols);
      } else if (W->kind == OR_Q1) {   /* mm_q1 -> row_q1_multi: the row kernel's arithmetic for every vector */
        const int G = (cols + 127) / 128;
        v = row_q1((const uint8_t *)W->q + (int64_t)r * G * 16, (const uint16_t *)W->s + (int64_t)r * G, xb, sb, cols);
      } else {
        const uint8_t *q = (const uint8_t *)W->q + (int64_t)r * (cols / 2); const uint16_t *s = (const uint16_t *)W->s + (int64_t)r * (cols / 32);
        v = (b < B4 && !(g_order & OR_ORD_ROWS_PREFILL)) ? mm_row_q4(q, s, xb, sb, cols) : row_q4(q, s, xb, sb, cols);
      }
      Y[(size_t)b * rows + r] = v;
    }
  free(xq); free(bs);
}

/* ------------------------------------------------------------------ elementwise */
/* rmsnorm (kernels.cpp:184-189) as g++ vectorises it: the squares of the first n - n % 4 elements are rounded products
 * summed in order, the last n % 4 are fused (ss = fma(x, x, ss)); inv = 1 / sqrt(ss / n + eps); out = x * inv * w */
/* the HIP prologue's order (act.hpp): per 128-column block, 8 lanes fma-sum 16 columns each in order, then
 * ((l0+l1)+(l2+l3)) + ((l7+l6)+(l5+l4)) by DPP; the block sums b[0..255] (zero past nb) enter a 64-lane wave as
 * (b[l]+b[l+64]) + (b[l+128]+b[l+192]) and a butterfly over xor 32, 16, .., 1 gives lane 0's total */
static float tree_ss(const float *x, int n) {
  const int nb = n / OR_QB; float bsum[256] = {0}, v[64];
  for (int b = 0; b < nb; b++) {
    float l[8];
    for (int j = 0; j < 8; j++) { float t = 0; for (int k = 0; k < 16; k++) { const float a = x[b * OR_QB + 16 * j + k]; t = fmaf(a, a, t); } l[j] = t; }
    float p[8]; for (int j = 0; j < 8; j++) p[j] = l[j] + l[j ^ 1];
    float q[8]; for (int j = 0; j < 8; j++) q[j] = p[j] + p[j ^ 2];
    bsum[b] = q[0] + q[7];
  }
  for (int i = 0; i < 64; i++) v[i] = (bsum[i] + bsum[i + 64]) + (bsum[i + 128] + bsum[i + 192]);
  for (int o = 32; o > 0; o >>= 1) { float w[64]; for (int i = 0; i < 64; i++) w[i] = v[i] + v[i ^ o]; memcpy(v, w, sizeof v); }
  return v[0];
}
void or_rmsnorm(const float *x, const float *w, int n, float eps, float *out) {
  if ((g_order & OR_ORD_TREE_NORM) && n % OR_QB == 0 && n <= 256 * OR_QB) {
    const float inv = 1.f / sqrtf(tree_ss(x, n) / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
    return;
  }
  float ss = 0; const int nv = n - n % 4;
  for (int i = 0; i < nv; i++) { const float p = x[i] * x[i]; ss = ss + p; }
  for (int i = nv; i < n; i++) ss = fmaf(x[i], x[i], ss);
  const float inv = 1.f / sqrtf(ss / (float)n + eps);
  for (int i = 0; i < n; i++) out[i] = x[i] * inv * w[i];
}
/* exp256, one lane (kernels_x86.cpp:406-417): clamp to [-87, 88], k = rint(x * log2 e), Cody-Waite reduction with
 * 0.693359375 and -2.12194440e-4, degree-6 polynomial, times 2^k */
static float exp_lane(float x) {
  x = x > -87.f ? x : -87.f; x = 88.f > x ? x : 88.f;
  const float k = nearbyintf(x * 1.44269504088896341f);
  const float r = fmaf(-k, 0.693359375f, fmaf(-k, -2.12194440e-4f, x));
  float p = 1.9875691500e-4f;
  p = fmaf(p, r, 1.3981999507e-3f); p = fmaf(p, r, 8.3334519073e-3f); p = fmaf(p, r, 4.1665795894e-2f);
  p = fmaf(p, r, 1.6666665459e-1f); p = fmaf(p, r, 5.0000001201e-1f);
  p = fmaf(p * r, r, r + 1.f);
  const int32_t e = ((int32_t)k + 127) << 23; float s; memcpy(&s, &e, 4);
  return p * s;
}
/* exp_v (kernels_x86.cpp:418-421): exp256 on every full group of 8 from the start, libm expf on the tail */
static float or_expf(float x) { return (g_order & OR_ORD_EXP_F64) ? (float)exp((double)x) : expf(x); }
void or_exp_v(const float *x, float *y, int n) {
  int i = 0; for (; i + 8 <= n; i += 8) for (int l = 0; l < 8; l++) y[i + l] = exp_lane(x[i + l]);
  for (; i < n; i++) y[i] = or_expf(x[i]);
}
/* silu_mul (kernels_x86.cpp:427-434): g = g / (1 + exp(0 - g)) * u, exp256 on full groups of 8, expf on the tail */
void or_silu_mul(float *g, const float *u, int n) {
  int i = 0;
  for (; i + 8 <= n; i += 8) for (int l = 0; l < 8; l++) { const float v = g[i + l]; g[i + l] = v / (1.f + exp_lane(0.f - v)) * u[i + l]; }
  for (; i < n; i++) g[i] = g[i] / (1.f + expf(-g[i])) * u[i];
}
/* row_f32 (kernels.cpp:146-162): q8 row -> q * scale, q4 row -> (nibble - 8) * f16 scale, f32 copy */
void or_row_f32(const or_mat *W, int r, float *out) {
  const int n = W->cols;
  if (W->kind == OR_F32) { memcpy(out, (const float *)W->q + (int64_t)r * n, 4 * (size_t)n); return; }
  if (W->kind == OR_Q8) {
    const int8_t *q = (const int8_t *)W->q + (int64_t)r * n; const float s = ((const float *)W->s)[r];
    for (int i = 0; i < n; i++) out[i] = q[i] * s;
    return;
  }
  const uint8_t *q = (const uint8_t *)W->q + (int64_t)r * (n / 2); const uint16_t *s = (const uint16_t *)W->s + (int64_t)r * (n / 32);
  for (int k = 0; k < n / 32; k++) {
    const float sc = or_f16_to_f32(s[k]);
    for (int j = 0; j < 16; j++) { const uint8_t b = q[16 * k + j]; out[32 * k + j] = ((int)(b & 15) - 8) * sc; out[32 * k + j + 16] = ((int)(b >> 4) - 8) * sc; }
  }
}

/* attention helpers: dot_f16 (kernels_x86.cpp:453-462) and axpy_f16 (:463-467) */
static float dot_f16(const float *a, const uint16_t *b, int n) {
  float s0[8] = {0}, s1[8] = {0}; int i = 0;
  for (; i + 16 <= n; i += 16)
    for (int l = 0; l < 8; l++) { s0[l] = fmaf(a[i + l], or_f16_to_f32(b[i + l]), s0[l]); s1[l] = fmaf(a[i + 8 + l], or_f16_to_f32(b[i + 8 + l]), s1[l]); }
  for (; i + 8 <= n; i += 8) for (int l = 0; l < 8; l++) s0[l] = fmaf(a[i + l], or_f16_to_f32(b[i + l]), s0[l]);
  float t[8]; for (int l = 0; l < 8; l++) t[l] = s0[l] + s1[l];
  float s = hsum8(t); for (; i < n; i++) s = fmaf(a[i], or_f16_to_f32(b[i]), s);
  return s;
}
static void axpy_f16(float a, const uint16_t *x, float *y, int n) { for (int i = 0; i < n; i++) y[i] = fmaf(a, or_f16_to_f32(x[i]), y[i]); }

/* ------------------------------------------------------------------ model */
struct or_model {
  or_cfg c; or_mat embed, head; const float *fnorm; or_layer *layers;
  uint16_t *kc, *vc; double *inv; int pos, kvd;
  float *x, *xn, *q, *k, *v, *att, *o, *g, *u, *part;
  size_t part_cap;
};

or_model *or_create(const or_cfg *cfg, const or_mat *embed, const or_mat *head, const float *final_norm, const or_layer *layers) {
  or_model *m = (or_model *)calloc(1, sizeof *m);
  m->c = *cfg; m->embed = *embed; m->head = cfg->tied ? *embed : *head; m->fnorm = final_norm;
  m->layers = (or_layer *)malloc(sizeof(or_layer) * (size_t)cfg->L); memcpy(m->layers, layers, sizeof(or_layer) * (size_t)cfg->L);
  m->kvd = cfg->nkv * cfg->hd;
  const size_t kv = (size_t)cfg->L * cfg->ctx * m->kvd;
  m->kc = (uint16_t *)calloc(kv, 2); m->vc = (uint16_t *)calloc(kv, 2);
  m->inv = (double *)malloc(sizeof(double) * (size_t)(cfg->hd / 2));
  for (int i = 0; i < cfg->hd / 2; i++) m->inv[i] = 1.0 / pow(cfg->theta, (2.0 * i) / cfg->hd);   /* model_llama.cpp:39 */
  const int qd = cfg->nh * cfg->hd;
  m->x = (float *)calloc((size_t)cfg->d, 4); m->xn = (float *)calloc((size_t)cfg->d, 4); m->q = (float *)calloc((size_t)qd, 4);
  m->k = (float *)calloc((size_t)m->kvd, 4); m->v = (float *)calloc((size_t)m->kvd, 4); m->att = (float *)calloc((size_t)qd, 4);
  m->o = (float *)calloc((size_t)cfg->d, 4); m->g = (float *)calloc((size_t)cfg->ff, 4); m->u = (float *)calloc((size_t)cfg->ff, 4);
  return m;
}
void or_free(or_model *m) {
  if (!m) return;
  free(m->layers); free(m->kc); free(m->vc); free(m->inv); free(m->x); free(m->xn); free(m->q); free(m->k); free(m->v);
  free(m->att); free(m->o); free(m->g); free(m->u); free(m->part); free(m);
}
void or_reset(or_model *m) { m->pos = 0; }
int or_pos(const or_model *m) { return m->pos; }
int or_set_pos(or_model *m, int pos) { if (pos < 0 || pos > m->c.ctx) return -1; m->pos = pos; return 0; }
uint16_t *or_kcache(or_model *m) { return m->kc; }
uint16_t *or_vcache(or_model *m) { return m->vc; }

/* rotate-half RoPE as g++ contracts it (model_llama.cpp:176, :88): v[i] = fma(a, cs, -(b * sn)),
 * v[i + half] = fma(b, cs, a * sn) */
static void rope(float *vec, const float *cs, const float *sn, int half) {
  for (int i = 0; i < half; i++) {
    const float a = vec[i], b = vec[i + half];
    vec[i] = fmaf(a, cs[i], -(b * sn[i])); vec[i + half] = fmaf(b, cs[i], a * sn[i]);
  }
}
static void rope_tables(const or_model *m, int pos, float *cs, float *sn) {
  for (int i = 0; i < m->c.hd / 2; i++) { const double a = pos * m->inv[i]; cs[i] = (float)cos(a); sn[i] = (float)sin(a); }
}

/* decode attention (model_llama.cpp:134-166): items (kv group g, 64-position chunk c); scores_tpl (kernels_x86.cpp:474-486),
 * chunk max / exp_v / sum, values_tpl (:487-496), then the chunks merged in order per head */
/* one query head over cache positions [0, T) of kv group g in float64, rounded to float at the end */
static void attn_head_f64(const float *qh, const uint16_t *kl, const uint16_t *vl, int T, int g, int hd, int kvd, float *out) {
  double *sc = (double *)malloc(8 * (size_t)T), mx = -1e300, sum = 0, o[256] = {0};
  for (int t = 0; t < T; t++) {
    double s = 0; for (int i = 0; i < hd; i++) s += (double)qh[i] * or_f16_to_f32(kl[(size_t)t * kvd + g * hd + i]);
    sc[t] = s / sqrt((double)hd); if (sc[t] > mx) mx = sc[t];
  }
  for (int t = 0; t < T; t++) { sc[t] = exp(sc[t] - mx); sum += sc[t]; }
  for (int t = 0; t < T; t++) for (int i = 0; i < hd; i++) o[i] += sc[t] * or_f16_to_f32(vl[(size_t)t * kvd + g * hd + i]);
  for (int i = 0; i < hd; i++) out[i] = (float)(o[i] / sum);
  free(sc);
}
static void attend_f64(or_model *m, const uint16_t *kl, const uint16_t *vl, const float *q, int T, float *out) {
  const int nh = m->c.nh, rep = nh / m->c.nkv, hd = m->c.hd;
  #pragma omp parallel for schedule(dynamic, 1)
  for (int h = 0; h < nh; h++) attn_head_f64(q + h * hd, kl, vl, T, h / rep, hd, m->kvd, out + h * hd);
}
static void attend(or_model *m, const uint16_t *kl, const uint16_t *vl, const float *q, int T, float *out) {
  if (g_order & OR_ORD_ATTN_F64) { attend_f64(m, kl, vl, q, T, out); return; }
  const int C = 64, nc = (T + C - 1) / C, nh = m->c.nh, rep = nh / m->c.nkv, hd = m->c.hd, kvd = m->kvd;
  const float scl = 1.f / sqrtf((float)hd);
  const size_t need = (size_t)nh * nc * (hd + 2);
  if (m->part_cap < need) { free(m->part); m->part = (float *)malloc(4 * need); m->part_cap = need; }
  float *part = m->part; const int items = m->c.nkv * nc;
  #pragma omp parallel for schedule(dynamic, 1)
  for (int w = 0; w < items; w++) {
    float sc[16 * 64];   /* rep <= 16 */
    const int g = w / nc, c = w % nc, t0 = c * C, t1 = t0 + C < T ? t0 + C : T, n = t1 - t0;
    for (int t = t0; t < t1; t++) {
      const uint16_t *kk = kl + (size_t)t * kvd + g * hd;
      for (int j = 0; j < rep; j++) {
        const float *qj = q + (g * rep + j) * hd; float a0[8], a1[8];
        for (int l = 0; l < 8; l++) { a0[l] = qj[l] * or_f16_to_f32(kk[l]); a1[l] = qj[8 + l] * or_f16_to_f32(kk[8 + l]); }
        for (int i = 2; i < hd / 8; i += 2)
          for (int l = 0; l < 8; l++) {
            a0[l] = fmaf(qj[8 * i + l], or_f16_to_f32(kk[8 * i + l]), a0[l]);
            a1[l] = fmaf(qj[8 * i + 8 + l], or_f16_to_f32(kk[8 * i + 8 + l]), a1[l]);
          }
        float a[8]; for (int l = 0; l < 8; l++) a[l] = a0[l] + a1[l];
        sc[j * C + (t - t0)] = hsum8(a) * scl;
      }
    }
    for (int j = 0; j < rep; j++) {
      float *sj = sc + j * C, mx = -1e30f;
      for (int t = 0; t < n; t++) if (mx < sj[t]) mx = sj[t];
      for (int t = 0; t < n; t++) sj[t] -= mx;
      or_exp_v(sj, sj, n); float sum = 0; for (int t = 0; t < n; t++) sum += sj[t];
      float *pp = part + ((size_t)(g * rep + j) * nc + c) * (hd + 2); pp[0] = mx; pp[1] = sum; memset(pp + 2, 0, 4 * (size_t)hd);
    }
    for (int t = t0; t < t1; t++) {
      const uint16_t *vv = vl + (size_t)t * kvd + g * hd;
      for (int j = 0; j < rep; j++) {
        float *o = part + ((size_t)(g * rep + j) * nc + c) * (hd + 2) + 2; const float wgt = sc[j * C + (t - t0)];
        for (int i = 0; i < hd; i++) o[i] = fmaf(wgt, or_f16_to_f32(vv[i]), o[i]);
      }
    }
  }
  for (int h = 0; h < nh; h++) {
    const float *ph = part + (size_t)h * nc * (hd + 2); float M = -1e30f;
    for (int c = 0; c < nc; c++) if (M < ph[(size_t)c * (hd + 2)]) M = ph[(size_t)c * (hd + 2)];
    float *o = out + h * hd, L = 0; memset(o, 0, 4 * (size_t)hd);
    for (int c = 0; c < nc; c++) {
      const float *pc = ph + (size_t)c * (hd + 2); const float f = or_expf(pc[0] - M);
      L = fmaf(pc[1], f, L);
      for (int i = 0; i < hd; i++) o[i] = fmaf(f, pc[2 + i], o[i]);
    }
    const float il = 1.f / L; for (int i = 0; i < hd; i++) o[i] *= il;
  }
}

static void head_out(or_model *m, int want, float *out) {
  or_rmsnorm(m->x, m->fnorm, m->c.d, m->c.eps, m->xn);
  if (want == 2) { memcpy(out, m->xn, 4 * (size_t)m->c.d); return; }
  or_matvec(&m->head, m->xn, out);
}

int or_step(or_model *m, int tok, int want, float *out) {
  const or_cfg *c = &m->c;
  if (m->pos >= c->ctx || tok < 0 || tok >= c->V) return -1;
  or_row_f32(&m->embed, tok, m->x);
  const int half = c->hd / 2, T = m->pos + 1, qd = c->nh * c->hd, kvd = m->kvd;
  float cs[256], sn[256]; rope_tables(m, m->pos, cs, sn);
  for (int l = 0; l < c->L; l++) {
    const or_layer *ly = &m->layers[l];
    or_rmsnorm(m->x, ly->attn_norm, c->d, c->eps, m->xn);
    or_matvec(&ly->wq, m->xn, m->q); or_matvec(&ly->wk, m->xn, m->k); or_matvec(&ly->wv, m->xn, m->v);
    if (ly->bq) {
      for (int i = 0; i < qd; i++) m->q[i] += ly->bq[i];
      for (int i = 0; i < kvd; i++) { m->k[i] += ly->bk[i]; m->v[i] += ly->bv[i]; }
    }
    for (int h = 0; h < c->nh; h++) rope(m->q + h * c->hd, cs, sn, half);
    for (int g = 0; g < c->nkv; g++) rope(m->k + g * c->hd, cs, sn, half);
    uint16_t *kl = m->kc + (size_t)l * c->ctx * kvd, *vl = m->vc + (size_t)l * c->ctx * kvd;
    for (int i = 0; i < kvd; i++) { kl[(size_t)m->pos * kvd + i] = or_f32_to_f16(m->k[i]); vl[(size_t)m->pos * kvd + i] = or_f32_to_f16(m->v[i]); }
    attend(m, kl, vl, m->q, T, m->att);
    or_matvec(&ly->wo, m->att, m->o);
    for (int i = 0; i < c->d; i++) m->x[i] += m->o[i];
    or_rmsnorm(m->x, ly->ffn_norm, c->d, c->eps, m->xn);
    or_matvec(&ly->wg, m->xn, m->g); or_matvec(&ly->wu, m->xn, m->u);
    or_silu_mul(m->g, m->u, c->ff);
    or_matvec(&ly->wd, m->g, m->o);
    for (int i = 0; i < c->d; i++) m->x[i] += m->o[i];
  }
  m->pos++;
  if (want) head_out(m, want, out);
  return 0;
}

/* prompt batches of PB = 64 tokens (model_llama.cpp:66-130): matrix x matrix products through or_matmul, full causal
 * softmax per (token, head) with dot_f16 / exp_v / axpy_f16 */
int or_prefill(or_model *m, const int *toks, int n, int want, float *out) {
  if (n == 1) return or_step(m, toks[0], want, out);
  const or_cfg *c = &m->c; const int PB = 64, half = c->hd / 2, rep = c->nh / c->nkv, qd = c->nh * c->hd, kvd = m->kvd, d = c->d, ff = c->ff, hd = c->hd;
  if (m->pos + n > c->ctx) return -1;
  for (int i = 0; i < n; i++) if (toks[i] < 0 || toks[i] >= c->V) return -1;
  const float scl = 1.f / sqrtf((float)hd);
  float *X = (float *)malloc(4 * (size_t)PB * d), *XN = (float *)malloc(4 * (size_t)PB * d), *Q = (float *)malloc(4 * (size_t)PB * qd);
  float *K = (float *)malloc(4 * (size_t)PB * kvd), *V = (float *)malloc(4 * (size_t)PB * kvd), *A = (float *)malloc(4 * (size_t)PB * qd);
  float *O = (float *)malloc(4 * (size_t)PB * d), *Gt = (float *)malloc(4 * (size_t)PB * ff), *U = (float *)malloc(4 * (size_t)PB * ff);
  for (int s0 = 0; s0 < n; s0 += PB) {
    const int B = n - s0 < PB ? n - s0 : PB, p0 = m->pos;
    for (int i = 0; i < B; i++) or_row_f32(&m->embed, toks[s0 + i], X + (size_t)i * d);
    for (int l = 0; l < c->L; l++) {
      const or_layer *ly = &m->layers[l];
      for (int i = 0; i < B; i++) or_rmsnorm(X + (size_t)i * d, ly->attn_norm, d, c->eps, XN + (size_t)i * d);
      or_matmul(&ly->wq, XN, B, Q); or_matmul(&ly->wk, XN, B, K); or_matmul(&ly->wv, XN, B, V);
      uint16_t *kl = m->kc + (size_t)l * c->ctx * kvd, *vl = m->vc + (size_t)l * c->ctx * kvd;
      for (int i = 0; i < B; i++) {
        float *q = Q + (size_t)i * qd, *k = K + (size_t)i * kvd, *v = V + (size_t)i * kvd;
        if (ly->bq) { for (int j = 0; j < qd; j++) q[j] += ly->bq[j]; for (int j = 0; j < kvd; j++) { k[j] += ly->bk[j]; v[j] += ly->bv[j]; } }
        float cs[256], sn[256]; rope_tables(m, p0 + i, cs, sn);
        for (int h = 0; h < c->nh; h++) rope(q + h * hd, cs, sn, half);
        for (int g = 0; g < c->nkv; g++) rope(k + g * hd, cs, sn, half);
        for (int j = 0; j < kvd; j++) { kl[(size_t)(p0 + i) * kvd + j] = or_f32_to_f16(k[j]); vl[(size_t)(p0 + i) * kvd + j] = or_f32_to_f16(v[j]); }
      }
      #pragma omp parallel for schedule(dynamic, 1)
      for (int w = 0; w < B * c->nh; w++) {
        const int i = w / c->nh, h = w % c->nh, T = p0 + i + 1, g = h / rep;
        const float *qh = Q + (size_t)i * qd + h * hd; float mx = -1e30f;
        if (g_order & OR_ORD_ATTN_F64) { attn_head_f64(qh, kl, vl, T, g, hd, kvd, A + (size_t)i * qd + h * hd); continue; }
        float *sc = (float *)malloc(4 * (size_t)T);
        for (int t = 0; t < T; t++) { float s = dot_f16(qh, kl + (size_t)t * kvd + g * hd, hd); s *= scl; sc[t] = s; if (mx < s) mx = s; }
        float sum = 0; for (int t = 0; t < T; t++) sc[t] -= mx;
        or_exp_v(sc, sc, T); for (int t = 0; t < T; t++) sum += sc[t];
        float *o = A + (size_t)i * qd + h * hd; memset(o, 0, 4 * (size_t)hd); const float inv = 1.f / sum;
        for (int t = 0; t < T; t++) axpy_f16(sc[t] * inv, vl + (size_t)t * kvd + g * hd, o, hd);
        free(sc);
      }
      or_matmul(&ly->wo, A, B, O);
      for (size_t j = 0; j < (size_t)B * d; j++) X[j] += O[j];
      for (int i = 0; i < B; i++) or_rmsnorm(X + (size_t)i * d, ly->ffn_norm, d, c->eps, XN + (size_t)i * d);
      or_matmul(&ly->wg, XN, B, Gt); or_matmul(&ly->wu, XN, B, U);
      or_silu_mul(Gt, U, B * ff);
      or_matmul(&ly->wd, Gt, B, O);
      for (size_t j = 0; j < (size_t)B * d; j++) X[j] += O[j];
    }
    m->pos += B;
    if (s0 + PB >= n) memcpy(m->x, X + (size_t)((n - 1) % PB) * d, 4 * (size_t)d);
  }
  free(X); free(XN); free(Q); free(K); free(V); free(A); free(O); free(Gt); free(U);
  if (want) head_out(m, want, out);
  return 0;
}

/* greedy_run (qpack.h:143-149): token i+1 = argmax of the logits after token i, strict '>' so the lowest id wins ties */
int or_greedy(or_model *m, int tok, int n, int *out) {
  float *l = (float *)malloc(4 * (size_t)m->c.V);
  for (int i = 0; i < n; i++) {
    if (or_step(m, tok, 1, l)) { free(l); return -1; }
    int b = 0; for (int v = 1; v < m->c.V; v++) if (l[v] > l[b]) b = v;
    out[i] = tok = b;
  }
  free(l);
  return n;
}

/* ------------------------------------------------------------------ sampler candidates
 * top_m + the sort of Sampler::dist (/root/reference/src/sampler.cpp:12-27, :41-42): the M largest logits in the order
 * value descending, lower index first among equal values.  Same steps as the reference: all V candidates when
 * M >= V / 4; otherwise the first min(V, 4 M + 8) entries, cut to M (the threshold = the smallest kept value), then a
 * scan of the rest for entries strictly above the threshold (scan_gt, kernels_x86.cpp:498-506), cut again whenever more
 * than 4 M are held, a last cut to M, and the sort.  The cuts keep the M first entries of the same total order the
 * sort uses, which is what nth_element + resize keeps. */
typedef struct { int i; float v; } or_cand;
static int cand_cmp(const void *pa, const void *pb) {
  const or_cand *a = (const or_cand *)pa, *b = (const or_cand *)pb;
  if (a->v > b->v) return -1;
  if (b->v > a->v) return 1;
  return a->i < b->i ? -1 : (a->i > b->i);
}
int or_top_m(const float *x, int V, int M, int *idx, float *val) {
  if (V <= 0 || M < 1 || M > V) return -1;
  or_cand *c = (or_cand *)malloc(sizeof(or_cand) * (size_t)(M >= V / 4 ? V : 4 * M + 8 + 4096));
  int n = 0;
  if (M >= V / 4) {
    for (int v = 0; v < V; v++) { c[n].i = v; c[n].v = x[v]; n++; }
  } else {
    const int init = V < 4 * M + 8 ? V : 4 * M + 8;
    for (int v = 0; v < init; v++) { c[n].i = v; c[n].v = x[v]; n++; }
    qsort(c, (size_t)n, sizeof *c, cand_cmp); n = M; float thr = c[M - 1].v;
    for (int v0 = init; v0 < V; v0 += 4096) {
      const int v1 = v0 + 4096 < V ? v0 + 4096 : V;
      for (int v = v0; v < v1; v++) if (x[v] > thr) { c[n].i = v; c[n].v = x[v]; n++; }
      if (n > 4 * M) { qsort(c, (size_t)n, sizeof *c, cand_cmp); n = M; thr = c[M - 1].v; }
    }
  }
  qsort(c, (size_t)n, sizeof *c, cand_cmp);
  for (int k = 0; k < M; k++) { idx[k] = c[k].i; val[k] = c[k].v; }
  free(c);
  return 0;
}

/* ------------------------------------------------------------------ QPACK3 rANS (/root/reference/include/qpack/rans.h)
 * Static per-plane model: 12-bit frequencies summing to 4096, four interleaved 32-bit states (symbol i uses state i & 3),
 * byte-wise renormalisation into [2^23, 2^31).  The encoder walks the symbols backwards and the bytes are stored in
 * decode order, after the four final states. */
#define RANS_PBITS 12u
#define RANS_PSCALE (1u << RANS_PBITS)
#define RANS_L (1u << 23)

static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static void wr32(uint8_t *p, uint32_t v) { for (int i = 0; i < 4; i++) p[i] = (uint8_t)(v >> (8 * i)); }

/* rans.h:23-37: f = floor(h * 4096 / n), at least 1 for a present symbol; the most frequent symbol (first on ties) takes
 * the rest; when the rest is < 1 the largest frequency (first on ties) is decremented until the sum is 4096 */
int or_rans_freqs(const uint8_t *sym, int64_t n, int nsym, uint32_t *f) {
  uint64_t h[256] = {0};
  for (int64_t i = 0; i < n; i++) h[sym[i]]++;
  for (int i = 0; i < nsym; i++) f[i] = 0;
  if (n == 0) { f[0] = RANS_PSCALE; return 0; }
  int64_t sum = 0; int big = 0;
  for (int i = 0; i < nsym; i++) {
    if (!h[i]) continue;
    uint32_t v = (uint32_t)((h[i] * RANS_PSCALE) / (uint64_t)n);
    f[i] = v ? v : 1;
    sum += f[i];
    if (h[i] > h[big]) big = i;
  }
  const int64_t rest = (int64_t)f[big] + RANS_PSCALE - sum;
  if (rest >= 1) { f[big] = (uint32_t)rest; return 0; }
  for (int64_t d = sum - RANS_PSCALE; d > 0; d--) {
    int m = 0;
    for (int i = 1; i < nsym; i++) if (f[i] > f[m]) m = i;
    if (f[m] <= 1) return OR_RANS_NORMALISE;
    f[m]--;
  }
  return 0;
}

/* one coded plane: u32 comp_len | u16 f[nsym] | u32 state[4] | bytes (rans.h:38-49) */
static int64_t encode_plane(const uint8_t *sym, int64_t n, int nsym, uint8_t *out, int64_t cap) {
  uint32_t f[256], c[257];
  int e = or_rans_freqs(sym, n, nsym, f);
  if (e) return e;
  c[0] = 0;
  for (int i = 0; i < nsym; i++) c[i + 1] = c[i] + f[i];
  /* renormalisation bytes are produced last-first; at most 2 per symbol plus 16 for the final states */
  uint8_t *rev = (uint8_t *)malloc((size_t)(2 * n + 16));
  if (!rev) return OR_RANS_CAPACITY;
  int64_t nr = 0;
  uint32_t x[4] = {RANS_L, RANS_L, RANS_L, RANS_L};
  for (int64_t i = n - 1; i >= 0; i--) {
    uint32_t *st = &x[i & 3];
    const uint32_t s = sym[i], fr = f[s], xmax = ((RANS_L >> RANS_PBITS) << 8) * fr;
    while (*st >= xmax) { rev[nr++] = (uint8_t)*st; *st >>= 8; }
    *st = ((*st / fr) << RANS_PBITS) + (*st % fr) + c[s];
  }
  const int64_t total = 4 + 2 * nsym + 16 + nr;
  if (total > cap) { free(rev); return OR_RANS_CAPACITY; }
  uint8_t *o = out + 4;
  for (int i = 0; i < nsym; i++) { *o++ = (uint8_t)f[i]; *o++ = (uint8_t)(f[i] >> 8); }
  for (int i = 0; i < 4; i++) { wr32(o, x[i]); o += 4; }
  for (int64_t k = nr - 1; k >= 0; k--) *o++ = rev[k];
  free(rev);
  wr32(out, (uint32_t)(total - 4));
  return total;
}

int64_t or_rans_encode(const uint8_t *raw, int64_t n, int codec, int planes, uint8_t *out, int64_t cap) {
  if (cap < 6) return OR_RANS_CAPACITY;
  if (!((codec == 2 && planes == 1) || (codec == 1 && planes >= 1 && planes <= 4))) return OR_RANS_BAD_CODEC;
  out[0] = (uint8_t)codec; out[1] = (uint8_t)planes; wr32(out + 2, (uint32_t)n);
  int64_t pos = 6;
  if (codec == 2) {   /* each byte -> low nibble, then high nibble */
    uint8_t *s = (uint8_t *)malloc((size_t)(2 * n + 1));
    if (!s) return OR_RANS_CAPACITY;
    for (int64_t i = 0; i < n; i++) { s[2 * i] = raw[i] & 15; s[2 * i + 1] = raw[i] >> 4; }
    const int64_t r = encode_plane(s, 2 * n, 16, out + pos, cap - pos);
    free(s);
    if (r < 0) return r;
    pos += r;
  } else {            /* plane k = raw[k], raw[k + planes], ... */
    uint8_t *s = (uint8_t *)malloc((size_t)(n / planes + 1));
    if (!s) return OR_RANS_CAPACITY;
    for (int k = 0; k < planes; k++) {
      int64_t m = 0;
      for (int64_t i = k; i < n; i += planes) s[m++] = raw[i];
      const int64_t r = encode_plane(s, m, 256, out + pos, cap - pos);
      if (r < 0) { free(s); return r; }
      pos += r;
    }
    free(s);
  }
  return pos;
}

/* one plane (rans.h:53-71): symbol i -> out[(i * stride + phase)] (bytes) or its nibble i & 1 of out[i >> 1] (nibbles);
 * returns the bytes consumed */
static int64_t decode_plane(const uint8_t *p, int64_t avail, int nsym, int64_t n, uint8_t *out, int stride, int phase,
                            int nibbles) {
  if (avail < 4) return OR_RANS_TRUNCATED;
  const uint32_t cl = rd32(p);
  if ((int64_t)cl + 4 > avail || cl < 2u * (uint32_t)nsym + 16) return OR_RANS_TRUNCATED_PLANE;
  const uint8_t *q = p + 4, *end = p + 4 + cl;
  uint32_t f[256], c[257];
  c[0] = 0;
  for (int i = 0; i < nsym; i++) { f[i] = (uint32_t)q[2 * i] | ((uint32_t)q[2 * i + 1] << 8); c[i + 1] = c[i] + f[i]; }
  if (c[nsym] != RANS_PSCALE) return OR_RANS_BAD_TABLE;
  q += 2 * nsym;
  /* the symbol of a slot m is the s with c[s] <= m < c[s + 1] */
  uint8_t slot[RANS_PSCALE];
  for (int s = 0; s < nsym; s++) for (uint32_t k = c[s]; k < c[s + 1]; k++) slot[k] = (uint8_t)s;
  uint32_t x[4];
  for (int i = 0; i < 4; i++) { x[i] = rd32(q); q += 4; }
  for (int64_t i = 0; i < n; i++) {
    uint32_t *st = &x[i & 3];
    const uint32_t m = *st & (RANS_PSCALE - 1), s = slot[m];
    *st = f[s] * (*st >> RANS_PBITS) + m - c[s];
    while (*st < RANS_L) {
      if (q >= end) return OR_RANS_OVERRUN;
      *st = (*st << 8) | *q++;
    }
    if (nibbles) out[i >> 1] |= (uint8_t)(s << (4 * (i & 1)));
    else out[i * stride + phase] = (uint8_t)s;
  }
  return (int64_t)cl + 4;
}

int64_t or_rans_raw_size(const uint8_t *p, int64_t len) {
  if (len < 6) return OR_RANS_SHORT;
  return rd32(p + 2);
}

int or_rans_decode(const uint8_t *p, int64_t len, uint8_t *out, int64_t cap) {
  if (len >= 1 && p[0] == 3) {   /* chunked: u8 3 | u8 0 | u32 raw_len | u32 chunk_raw | u32 nchunks | u32 comp_len[] | chunks */
    if (len < 14) return OR_RANS_SHORT_CHUNKED;
    const int64_t cr = rd32(p + 6), nc = rd32(p + 10);
    int64_t pos = 14 + 4 * nc;
    if (pos > len) return OR_RANS_TRUNCATED_TABLE;
    for (int64_t i = 0; i < nc; i++) {
      const int64_t cl = rd32(p + 14 + 4 * i);
      if (pos + cl > len) return OR_RANS_TRUNCATED_CHUNK;
      if (i * cr > cap) return OR_RANS_CAPACITY;
      const int r = or_rans_decode(p + pos, cl, out + i * cr, cap - i * cr);
      if (r) return r;
      pos += cl;
    }
    return 0;
  }
  const int64_t n = or_rans_raw_size(p, len);
  if (n < 0) return (int)n;
  if (n > cap) return OR_RANS_CAPACITY;
  const int codec = p[0], planes = p[1];
  int64_t pos = 6;
  if (codec == 2) {
    memset(out, 0, (size_t)n);
    const int64_t r = decode_plane(p + pos, len - pos, 16, 2 * n, out, 1, 0, 1);
    return r < 0 ? (int)r : 0;
  }
  if (codec == 1 && planes >= 1 && planes <= 4) {
    for (int k = 0; k < planes; k++) {
      const int64_t cnt = (n + planes - 1 - k) / planes;
      const int64_t r = decode_plane(p + pos, len - pos, 256, cnt, out, planes, k, 0);
      if (r < 0) return (int)r;
      pos += r;
    }
    return 0;
  }
  return OR_RANS_BAD_CODEC;
}
