// Reference-order kernels: the token loop with every floating-point operation in the order, and with the rounding, of
// the reference's x86 CPU path, so logits, caches and greedy streams come out bit-identical to qp::Llama's.  They serve
// the model's reference-order mode (HipLlama::set_order(1)); the default mode's kernels keep their own, faster orders.
//
// What the default kernels already do in the reference's order and is reused as is: the activation quantisation and
// rows_q8 (the decode matvec: exact int32 block sums, fma chain in block order), the epilogues (bias, residual,
// silu(gate) * up with exp256, the head's argmax), RoPE and the fp16 cache rows.  What is here:
//   - RMSNorm with the reference's sequential sum of squares (/root/reference/src/kernels.cpp:184-189);
//   - decode attention over 64-position chunks with its per-chunk softmax and ordered merge
//     (/root/reference/src/model_llama.cpp:134-166, scores_tpl / values_tpl at /root/reference/src/kernels_x86.cpp:474-496);
//   - prompt attention per (token, head) with a full-row softmax (/root/reference/src/model_llama.cpp:95-105, dot_f16 /
//     axpy_f16 at /root/reference/src/kernels_x86.cpp:453-467);
//   - the prompt's matrix products in mm_q8 / mm_q4 lane order for the first B - B % 4 vectors of each 64-token batch
//     and rows_q8 / rows_q4 order for the rest (/root/reference/src/kernels_x86.cpp:55-106, :287-371), and the q4
//     matvec in rows_q4 order;
//   - exp256 on groups of 8 and the C library's expf on the tails (libm_expf.hpp).
// These kernels favour plain one-thread-per-output loops over speed: the mode exists to check greedy identity.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "launch.hpp"
#include "libm_expf.hpp"

#pragma clang fp contract(off)

namespace qph {

// hsum256 of /root/reference/src/kernels_x86.cpp:18-21 over eight lane values
__device__ __forceinline__ float ex_hsum8(const float v[8]) {
  const float a0 = v[0] + v[4], a1 = v[1] + v[5], a2 = v[2] + v[6], a3 = v[3] + v[7];
  return (a0 + a2) + (a1 + a3);
}
__device__ __forceinline__ float h2f(uint16_t h) { return half_bits_to_float(h); }

// ------------------------------------------------------------------ RMSNorm, sequential sum of squares
// rmsnorm (kernels.cpp:184-189) as g++ -O3 -mfma compiles it: the squares of the first n - n % 4 elements are rounded
// products added in order, the last n % 4 are fused (ss = fma(x, x, ss)); inv = 1 / sqrt(ss / n + eps);
// out = x * inv * w.  One workgroup per row; the chain runs in one thread.
__global__ __launch_bounds__(256) void k_ex_rmsnorm(const float *x, int ldx, const float *w, int n, float eps, float *out, int ldo) {
  extern __shared__ __align__(16) float sq[];
  __shared__ float inv_s;
  const float *xr = x + (size_t)blockIdx.x * ldx;
  const int nv = n - n % 4;
  for (int i = threadIdx.x; i < nv; i += blockDim.x) { const float v = xr[i]; sq[i] = v * v; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float ss = 0.f;
    int i = 0;
    for (; i + 32 <= nv; i += 32) {
      float4 p[8];
#pragma unroll
      for (int k = 0; k < 8; k++) p[k] = *(const float4 *)(sq + i + 4 * k);
#pragma unroll
      for (int k = 0; k < 8; k++) { ss = ss + p[k].x; ss = ss + p[k].y; ss = ss + p[k].z; ss = ss + p[k].w; }
    }
    for (; i < nv; i++) ss = ss + sq[i];
    for (; i < n; i++) ss = __builtin_fmaf(xr[i], xr[i], ss);
    inv_s = 1.f / sqrtf(ss / (float)n + eps);
  }
  __syncthreads();
  const float inv = inv_s;
  float *o = out + (size_t)blockIdx.x * ldo;
  for (int i = threadIdx.x; i < n; i += blockDim.x) o[i] = xr[i] * inv * w[i];
}
hipError_t launch_ex_rmsnorm(const float *x, int ldx, const float *w, int n, float eps, float *out, int ldo, int rows,
                             hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  if (n <= 0 || n > 32768) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ex_rmsnorm, dim3(rows), dim3(256), 4 * (size_t)n, st, x, ldx, w, n, eps, out, ldo);
  return hipGetLastError();
}

// ------------------------------------------------------------------ decode: RoPE and the fp16 cache rows
// the step's RoPE (model_llama.cpp:172-183, the fma forms g++ contracts it to) on q into qr and on k, then k and v
// rounded to fp16 into the cache row of position ctl->pos
__global__ __launch_bounds__(256) void k_ex_rope(ExRopeArgs a) {
  const int pos = a.ctl->pos, half = a.hd / 2, kvd = a.nkv * a.hd;
  const float *cs = a.cos_t + (size_t)pos * half, *sn = a.sin_t + (size_t)pos * half;
  for (int e = threadIdx.x; e < a.nh * half; e += blockDim.x) {
    const int h = e / half, i = e % half;
    const float x0 = a.q[h * a.hd + i], x1 = a.q[h * a.hd + i + half];
    a.qr[h * a.hd + i] = __builtin_fmaf(x0, cs[i], -(x1 * sn[i]));
    a.qr[h * a.hd + i + half] = __builtin_fmaf(x1, cs[i], x0 * sn[i]);
  }
  uint16_t *kr = a.kc + (size_t)pos * kvd, *vr = a.vc + (size_t)pos * kvd;
  for (int e = threadIdx.x; e < a.nkv * half; e += blockDim.x) {
    const int g = e / half, i = e % half;
    const float x0 = a.k[g * a.hd + i], x1 = a.k[g * a.hd + i + half];
    kr[g * a.hd + i] = f32_to_half_bits(__builtin_fmaf(x0, cs[i], -(x1 * sn[i])));
    kr[g * a.hd + i + half] = f32_to_half_bits(__builtin_fmaf(x1, cs[i], x0 * sn[i]));
  }
  for (int e = threadIdx.x; e < kvd; e += blockDim.x) vr[e] = float_to_half_bits(a.v[e]);
}
hipError_t launch_ex_rope(const ExRopeArgs &a, hipStream_t st) {
  hipLaunchKernelGGL(k_ex_rope, dim3(1), dim3(256), 0, st, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ decode attention, reference order
// exp_v (kernels_x86.cpp:418-421) over v[0, n) in place: exp256 on every full group of 8 from the start, expf on the tail
__device__ __forceinline__ float ex_exp_v(float x, int t, int n) { return t < n - n % 8 ? exp_poly(x) : libm_expf(x); }

// one workgroup per item (kv group g = blockIdx.x, chunk c = blockIdx.y of 64 positions), attend()'s item body
// (model_llama.cpp:139-156): scores of the group's rep heads (scores_tpl: lane products of dims 0..15, fma over the
// next pairs of 8-dim steps, a0 + a1, hsum, times 1 / sqrt(hd)); per head the chunk max, x - max, exp_v, the sum in
// order; values_tpl: o = fma(p_t, v_t, o) over the chunk's positions in order.  Partials part[h][c][2 + hd] with
// (max, sum) first; chunks past the context exit.
template <int HD>
__global__ __launch_bounds__(256) void k_ex_attn_part(ExAttnArgs a) {
  constexpr int C = 64;
  __shared__ float qs[8][HD];
  __shared__ float sc[8][C];
  const int T = a.ctl->pos + 1, nc = (T + C - 1) / C, g = blockIdx.x, c = blockIdx.y;
  if (c >= nc) return;
  const int rep = a.nh / a.nkv, kvd = a.nkv * HD, t0 = c * C, n = min(C, T - t0);
  for (int e = threadIdx.x; e < rep * HD; e += blockDim.x) qs[e / HD][e % HD] = a.qr[(size_t)g * rep * HD + e];
  __syncthreads();
  const float scl = 1.f / sqrtf((float)HD);
  for (int e = threadIdx.x; e < rep * C; e += blockDim.x) {
    const int j = e / C, t = e % C;
    if (t >= n) continue;
    const uint16_t *kk = a.kc + (size_t)(t0 + t) * kvd + g * HD;
    const float *qj = qs[j];
    float a0[8], a1[8];
#pragma unroll
    for (int l = 0; l < 8; l++) { a0[l] = qj[l] * h2f(kk[l]); a1[l] = qj[8 + l] * h2f(kk[8 + l]); }
#pragma unroll
    for (int i = 2; i < HD / 8; i += 2)
#pragma unroll
      for (int l = 0; l < 8; l++) {
        a0[l] = __builtin_fmaf(qj[8 * i + l], h2f(kk[8 * i + l]), a0[l]);
        a1[l] = __builtin_fmaf(qj[8 * i + 8 + l], h2f(kk[8 * i + 8 + l]), a1[l]);
      }
    float s8[8];
#pragma unroll
    for (int l = 0; l < 8; l++) s8[l] = a0[l] + a1[l];
    sc[j][t] = ex_hsum8(s8) * scl;
  }
  __syncthreads();
  if (threadIdx.x < rep) {
    const int j = threadIdx.x;
    float mx = -1e30f;
    for (int t = 0; t < n; t++) mx = mx < sc[j][t] ? sc[j][t] : mx;
    float sum = 0.f;
    for (int t = 0; t < n; t++) { const float e = ex_exp_v(sc[j][t] - mx, t, n); sc[j][t] = e; sum = sum + e; }
    float *pp = a.part + ((size_t)(g * rep + j) * a.ncmax + c) * (HD + 2);
    pp[0] = mx; pp[1] = sum;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < rep * HD; e += blockDim.x) {
    const int j = e / HD, i = e % HD;
    const uint16_t *vv = a.vc + (size_t)t0 * kvd + g * HD + i;
    float o = 0.f;
    for (int t = 0; t < n; t++) o = __builtin_fmaf(sc[j][t], h2f(vv[(size_t)t * kvd]), o);
    a.part[((size_t)(g * rep + j) * a.ncmax + c) * (HD + 2) + 2 + i] = o;
  }
}
// the merge (model_llama.cpp:159-165): M = max of the chunk maxima; in chunk order f = expf(m_c - M), L = fma(l_c, f, L),
// o = fma(f, o_c, o); out = o * (1 / L).  One workgroup per query head, one thread per dim.
template <int HD>
__global__ __launch_bounds__(HD) void k_ex_attn_merge(ExAttnArgs a) {
  const int T = a.ctl->pos + 1, nc = (T + 63) / 64, h = blockIdx.x, i = threadIdx.x;
  const float *ph = a.part + (size_t)h * a.ncmax * (HD + 2);
  float M = -1e30f;
  for (int c = 0; c < nc; c++) { const float m = ph[(size_t)c * (HD + 2)]; M = M < m ? m : M; }
  float o = 0.f, L = 0.f;
  for (int c = 0; c < nc; c++) {
    const float *pc = ph + (size_t)c * (HD + 2);
    const float f = libm_expf(pc[0] - M);
    L = __builtin_fmaf(pc[1], f, L);
    o = __builtin_fmaf(f, pc[2 + i], o);
  }
  const float il = 1.f / L;
  a.att[(size_t)h * HD + i] = o * il;
}
hipError_t launch_ex_attention(const ExAttnArgs &a, hipStream_t st) {
  if (a.nh % a.nkv || a.nh / a.nkv > 8 || a.ncmax < 1) return hipErrorInvalidValue;
  if (a.hd == 64) {
    hipLaunchKernelGGL(k_ex_attn_part<64>, dim3(a.nkv, a.ncmax), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_ex_attn_merge<64>, dim3(a.nh), dim3(64), 0, st, a);
  } else if (a.hd == 128) {
    hipLaunchKernelGGL(k_ex_attn_part<128>, dim3(a.nkv, a.ncmax), dim3(256), 0, st, a);
    hipLaunchKernelGGL(k_ex_attn_merge<128>, dim3(a.nh), dim3(128), 0, st, a);
  } else return hipErrorInvalidValue;
  return hipGetLastError();
}

// ------------------------------------------------------------------ prompt attention, reference order
// token i = blockIdx.y (position p0 + i), head h = blockIdx.x over cache positions [0, p0 + i]: s_t = dot_f16(q, k_t)
// (two 8-lane fma chains over 16-dim steps from zero, their sum, hsum) times 1 / sqrt(hd); x - max; exp_v over the row;
// the sum in order; o = fma(p_t * (1 / sum), v_t, o) in position order (model_llama.cpp:95-105).
template <int HD>
__global__ __launch_bounds__(256) void k_ex_pf_attn(ExPfAttnArgs a) {
  extern __shared__ __align__(16) float srow[];
  __shared__ float qs[HD];
  __shared__ float red[256];
  const int h = blockIdx.x, i = blockIdx.y, T = a.p0 + i + 1, rep = a.nh / a.nkv, g = h / rep, kvd = a.nkv * HD;
  const float *qh = a.q + (size_t)i * a.ldq + h * HD;
  for (int e = threadIdx.x; e < HD; e += blockDim.x) qs[e] = qh[e];
  __syncthreads();
  const float scl = 1.f / sqrtf((float)HD);
  float mx = -1e30f;
  for (int t = threadIdx.x; t < T; t += blockDim.x) {
    const uint16_t *kk = a.kc + (size_t)t * kvd + g * HD;
    float s0[8], s1[8];
#pragma unroll
    for (int l = 0; l < 8; l++) { s0[l] = 0.f; s1[l] = 0.f; }
#pragma unroll
    for (int d = 0; d < HD; d += 16)
#pragma unroll
      for (int l = 0; l < 8; l++) {
        s0[l] = __builtin_fmaf(qs[d + l], h2f(kk[d + l]), s0[l]);
        s1[l] = __builtin_fmaf(qs[d + 8 + l], h2f(kk[d + 8 + l]), s1[l]);
      }
    float s8[8];
#pragma unroll
    for (int l = 0; l < 8; l++) s8[l] = s0[l] + s1[l];
    float s = ex_hsum8(s8);
    s = s * scl;
    srow[t] = s;
    mx = mx < s ? s : mx;
  }
  red[threadIdx.x] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    float m = -1e30f;
    for (int k = 0; k < (int)blockDim.x; k++) m = m < red[k] ? red[k] : m;
    red[0] = m;
  }
  __syncthreads();
  mx = red[0];
  for (int t = threadIdx.x; t < T; t += blockDim.x) srow[t] = ex_exp_v(srow[t] - mx, t, T);
  __syncthreads();
  __shared__ float inv_s;
  if (threadIdx.x == 0) {
    float sum = 0.f;
    for (int t = 0; t < T; t++) sum = sum + srow[t];
    inv_s = 1.f / sum;
  }
  __syncthreads();
  const float inv = inv_s;
  for (int d = threadIdx.x; d < HD; d += blockDim.x) {
    const uint16_t *vv = a.vc + g * HD + d;
    float o = 0.f;
    for (int t = 0; t < T; t++) o = __builtin_fmaf(srow[t] * inv, h2f(vv[(size_t)t * kvd]), o);
    a.att[(size_t)i * a.lda + h * HD + d] = o;
  }
}
hipError_t launch_ex_pf_attn(const ExPfAttnArgs &a, int B, hipStream_t st) {
  if (B <= 0) return hipSuccess;
  if (a.nh % a.nkv) return hipErrorInvalidValue;
  const size_t lds = 4 * (size_t)(a.p0 + B);
  if (lds > 128 * 1024) return hipErrorInvalidValue;
  if (a.hd == 64) hipLaunchKernelGGL(k_ex_pf_attn<64>, dim3(a.nh, B), dim3(256), lds, st, a);
  else if (a.hd == 128) hipLaunchKernelGGL(k_ex_pf_attn<128>, dim3(a.nh, B), dim3(256), lds, st, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

// ------------------------------------------------------------------ matrix products, reference order
// the int16 activation of column c from the quantiser's planes (hi = q >> 8, lo = (q & 255) - 128)
__device__ __forceinline__ int ex_act(const int8_t *xh, const int8_t *xl, int c) { return (int)xh[c] * 256 + (int)xl[c] + 128; }

// mm_q8 (kernels_x86.cpp:287-334) for one (row, vector): lane l of each 128-column block sums columns 16 s + 2 l and
// 16 s + 2 l + 1 (s = 0..7) exactly; f_l = fma((float)lane, bs[block], f_l) in block order; y = hsum(f) * scale
__device__ float ex_mm_q8(const int8_t *w, const int8_t *xh, const int8_t *xl, const float *bs, int cols, float scale) {
  float f[8];
#pragma unroll
  for (int l = 0; l < 8; l++) f[l] = 0.f;
  for (int k = 0; k < cols / kQB; k++) {
#pragma unroll
    for (int l = 0; l < 8; l++) {
      int s = 0;
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int c = k * kQB + 16 * u + 2 * l;
        s += (int)w[c] * ex_act(xh, xl, c) + (int)w[c + 1] * ex_act(xh, xl, c + 1);
      }
      f[l] = __builtin_fmaf((float)s, bs[k], f[l]);
    }
  }
  return ex_hsum8(f) * scale;
}
// rows_q8 (kernels_x86.cpp:55-71): the exact int32 sum of each block, acc = fma(bs, (float)sum, acc), y = acc * scale
__device__ float ex_row_q8(const int8_t *w, const int8_t *xh, const int8_t *xl, const float *bs, int cols, float scale) {
  float acc = 0.f;
  for (int k = 0; k < cols / kQB; k++) {
    int s = 0;
    for (int c = k * kQB; c < (k + 1) * kQB; c++) s += (int)w[c] * ex_act(xh, xl, c);
    acc = __builtin_fmaf(bs[k], (float)s, acc);
  }
  return acc * scale;
}
// AVX2 lane l (0..7) of one q4 group of 16 bytes: columns 2l, 2l + 1 (low nibbles) and 16 + 2l, 17 + 2l (high nibbles),
// each nibble - 8 (kernels_x86.cpp:81-91)
__device__ __forceinline__ int ex_q4_lane(const uint8_t *g16, const int8_t *xh, const int8_t *xl, int c0, int l) {
  const uint8_t b0 = g16[2 * l], b1 = g16[2 * l + 1];
  return ((int)(b0 & 15) - 8) * ex_act(xh, xl, c0 + 2 * l) + ((int)(b1 & 15) - 8) * ex_act(xh, xl, c0 + 2 * l + 1) +
         ((int)(b0 >> 4) - 8) * ex_act(xh, xl, c0 + 16 + 2 * l) + ((int)(b1 >> 4) - 8) * ex_act(xh, xl, c0 + 17 + 2 * l);
}
// rows_q4 (kernels_x86.cpp:81-106): comb_g = f16(s_g) * bs[g / 4]; even groups into lane accumulators a0, odd into a1
// (an odd last group into a0), lane = fma((float)lane_sum, comb, lane); y = hsum(a0 + a1)
__device__ float ex_row_q4(const uint8_t *q, const uint16_t *s, const int8_t *xh, const int8_t *xl, const float *bs, int cols) {
  const int G = cols / 32;
  float a0[8], a1[8];
#pragma unroll
  for (int l = 0; l < 8; l++) { a0[l] = 0.f; a1[l] = 0.f; }
  int k = 0;
  for (; k + 2 <= G; k += 2) {
    const float c0 = h2f(s[k]) * bs[k >> 2], c1 = h2f(s[k + 1]) * bs[(k + 1) >> 2];
#pragma unroll
    for (int l = 0; l < 8; l++) {
      a0[l] = __builtin_fmaf((float)ex_q4_lane(q + 16 * k, xh, xl, 32 * k, l), c0, a0[l]);
      a1[l] = __builtin_fmaf((float)ex_q4_lane(q + 16 * k + 16, xh, xl, 32 * k + 32, l), c1, a1[l]);
    }
  }
  for (; k < G; k++) {
    const float c0 = h2f(s[k]) * bs[k >> 2];
#pragma unroll
    for (int l = 0; l < 8; l++) a0[l] = __builtin_fmaf((float)ex_q4_lane(q + 16 * k, xh, xl, 32 * k, l), c0, a0[l]);
  }
  float t[8];
#pragma unroll
  for (int l = 0; l < 8; l++) t[l] = a0[l] + a1[l];
  return ex_hsum8(t);
}
// mm_q4 (kernels_x86.cpp:345-371): one 8-lane accumulator over all groups, comb = f16(s_g) * bs[g / 4]; y = hsum(f)
__device__ float ex_mm_q4(const uint8_t *q, const uint16_t *s, const int8_t *xh, const int8_t *xl, const float *bs, int cols) {
  float f[8];
#pragma unroll
  for (int l = 0; l < 8; l++) f[l] = 0.f;
  for (int k = 0; k < cols / 32; k++) {
    const float cb = h2f(s[k]) * bs[k >> 2];
#pragma unroll
    for (int l = 0; l < 8; l++) f[l] = __builtin_fmaf((float)ex_q4_lane(q + 16 * k, xh, xl, 32 * k, l), cb, f[l]);
  }
  return ex_hsum8(f);
}

// rows_q1 / mm_q1 (kernels_x86.cpp:163-211: every q1 entry point runs row_q1_nt, so a vector's result does not depend
// on its batch): per 128-column group, AVX2 lane l's exact sum over columns 16 i + 2 l and 16 i + 2 l + 1 (i = 0..7) of
// (+1 for a set sign bit, -1 for a clear one) x the activation; lane = fma((float)sum, f16(scale) * bs[g], lane) in group
// order; y = hsum(lanes).  cols % 128 == 0 (the q1 matrices this model takes)
__device__ float ex_row_q1(const uint8_t *q, const uint16_t *s, const int8_t *xh, const int8_t *xl, const float *bs, int cols) {
  float f[8];
#pragma unroll
  for (int l = 0; l < 8; l++) f[l] = 0.f;
  for (int g = 0; g < cols / kQB; g++) {
    const uint8_t *gb = q + 16 * g;
    const float cb = h2f(s[g]) * bs[g];
#pragma unroll
    for (int l = 0; l < 8; l++) {
      int sum = 0;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int c = 16 * i + 2 * l;   // bits c and c + 1 of the group: byte c / 8, bits c % 8 and c % 8 + 1
        const int b0 = (gb[c >> 3] >> (c & 7)) & 1, b1 = (gb[(c + 1) >> 3] >> ((c + 1) & 7)) & 1;
        sum += (2 * b0 - 1) * ex_act(xh, xl, kQB * g + c) + (2 * b1 - 1) * ex_act(xh, xl, kQB * g + c + 1);
      }
      f[l] = __builtin_fmaf((float)sum, cb, f[l]);
    }
  }
  return ex_hsum8(f);
}

// Y[t][r] (+ bias[r]; or Y[t][r] += when resid) for rows r of one q8 / q4 / q1 matrix and the batch's quantised vectors; the
// vectors t < mm_below take the tiled order (mm_q8 / mm_q4), the others the row order.  A workgroup takes 256 / tt rows
// x tt vectors (tt = 1 for a single vector).
__global__ __launch_bounds__(256) void k_ex_gemm(ExGemmArgs a) {
  const int tt = a.tt, r = blockIdx.x * (256 / tt) + (int)threadIdx.x / tt, t = blockIdx.y * tt + (int)threadIdx.x % tt;
  if (r >= a.rows || t >= a.ntok) return;
  const int8_t *xh = a.xh + (size_t)t * a.ldq, *xl = a.xl + (size_t)t * a.ldq;
  const float *bs = a.xb + (size_t)t * a.ldb;
  float y;
  if (a.kind == MK_Q8) {
    const int8_t *w = (const int8_t *)a.w + (size_t)r * a.cols;
    const float sc = a.scale[r];
    y = t < a.mm_below ? ex_mm_q8(w, xh, xl, bs, a.cols, sc) : ex_row_q8(w, xh, xl, bs, a.cols, sc);
  } else if (a.kind == MK_Q4) {
    const uint8_t *q = (const uint8_t *)a.w + (size_t)r * (a.cols / 2);
    const uint16_t *s = a.s16 + (size_t)r * (a.cols / 32);
    y = t < a.mm_below ? ex_mm_q4(q, s, xh, xl, bs, a.cols) : ex_row_q4(q, s, xh, xl, bs, a.cols);
  } else {
    y = ex_row_q1((const uint8_t *)a.w + (size_t)r * (a.cols / 8), a.s16 + (size_t)r * (a.cols / kQB), xh, xl, bs, a.cols);
  }
  float *out = a.y + (size_t)t * a.ldy + r;
  if (a.bias) y = y + a.bias[r];
  if (a.resid) *out = *out + y;
  else *out = y;
}
hipError_t launch_ex_gemm(const ExGemmArgs &a, hipStream_t st) {
  if (a.ntok <= 0 || a.rows <= 0) return hipSuccess;
  if ((a.kind != MK_Q8 && a.kind != MK_Q4 && a.kind != MK_Q1) || a.cols % kQB || (a.tt != 1 && a.tt != 16))
    return hipErrorInvalidValue;
  const int rpb = 256 / a.tt;
  hipLaunchKernelGGL(k_ex_gemm, dim3((a.rows + rpb - 1) / rpb, (a.ntok + a.tt - 1) / a.tt), dim3(256), 0, st, a);
  return hipGetLastError();
}

// the greedy pick's per-workgroup partials from a logits vector (a head product that is not the argmax matvec): part b
// of n holds the (largest value, lowest index among equals) of its chunk, the strict > scan of qpack.h:143-149
__global__ __launch_bounds__(256) void k_ex_argmax_parts(const float *x, int V, float2 *amax) {
  const int per = (V + gridDim.x - 1) / gridDim.x, i0 = blockIdx.x * per, i1 = min(V, i0 + per);
  float bv = -INFINITY; int bi = 0x7fffffff;
  for (int i = i0 + (int)threadIdx.x; i < i1; i += blockDim.x)
    if (x[i] > bv || (x[i] == bv && i < bi)) { bv = x[i]; bi = i; }
  __shared__ float sv[256]; __shared__ int si[256];
  sv[threadIdx.x] = bv; si[threadIdx.x] = bi;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 256; k++)
      if (sv[k] > bv || (sv[k] == bv && si[k] < bi)) { bv = sv[k]; bi = si[k]; }
    amax[blockIdx.x] = make_float2(bv, __builtin_bit_cast(float, bi));
  }
}
hipError_t launch_ex_argmax_parts(const float *x, int V, float2 *amax, int nparts, hipStream_t st) {
  if (V <= 0 || nparts <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_ex_argmax_parts, dim3(nparts), dim3(256), 0, st, x, V, amax);
  return hipGetLastError();
}

// silu_mul (kernels_x86.cpp:427-434) on rows of n values (n % 8 == 0 at every configuration; a tail takes expf):
// g = g / (1 + exp256(0 - g)) * u
__global__ __launch_bounds__(256) void k_ex_silu(float *g, const float *u, int n, int ld, int rows) {
  const int row = blockIdx.y;
  float *gr = g + (size_t)row * ld; const float *ur = u + (size_t)row * ld;
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
    const float v = gr[i];
    const float e = i < n - n % 8 ? exp_poly(0.f - v) : libm_expf(-v);
    gr[i] = v / (1.f + e) * ur[i];
  }
}
hipError_t launch_ex_silu(float *g, const float *u, int n, int ld, int rows, hipStream_t st) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_ex_silu, dim3((n + 255) / 256, rows), dim3(256), 0, st, g, u, n, ld, rows);
  return hipGetLastError();
}

}  // namespace qph
