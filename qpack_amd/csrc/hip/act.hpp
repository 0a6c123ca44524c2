// Activation prologue shared by the decode matvec and the prefill quantiser: RMSNorm (optional) and quant_rows'
// per-128-column int16 quantisation, built in LDS as two byte planes.  One implementation, so a prompt token's
// activation is bit-identical to the decode step's.
#pragma once
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "launch.hpp"

namespace qph {

// ------------------------------------------------------------------ LDS activation layout
struct ActView {
  int8_t *xh;    // [cols] high bytes (signed)
  uint8_t *xl;   // [cols] low bytes (unsigned)
  float *bs;     // [nb] block scales
  int *lsum;     // [nb] sum of the low bytes per 128-column block
  int *gsum;     // [cols / 32] sum of q per 32-column group
  float *red;    // [32] reduction scratch (16 wave partials, argmax values and indices)
  int *sums;     // [waves][slots][nbp] q8 block sums
  int nbp;
};

__host__ __device__ inline int round_up(int a, int b) { return (a + b - 1) / b * b; }

__device__ inline ActView act_view(char *smem, int cols) {
  ActView v; const int nb = cols / kQB, G = cols / 32;
  v.nbp = round_up(nb, 4);
  v.xh = (int8_t *)smem;
  v.xl = (uint8_t *)(smem + cols);
  v.bs = (float *)(smem + 2 * cols);
  v.lsum = (int *)(v.bs + v.nbp);
  v.gsum = v.lsum + v.nbp;
  v.red = (float *)(v.gsum + round_up(G, 4));
  v.sums = (int *)(v.red + 32);
  return v;
}
// The activation prologue in two halves, so its global reads are issued before the weight prefetch (a wave's loads
// return in order: a read issued after the prefetch would wait for all of it).
//   act_load:   eight lanes own a 128-column block, 16 columns each (two passes cover up to 2 x blockDim.x / 8 blocks);
//               x (and the RMSNorm weight) go to registers.
//   act_build:  optional RMSNorm, then quant_rows' arithmetic (/root/reference/src/kernels.cpp:17-31): mx = max |v|,
//               isx = mx > 0 ? 32767 / mx : 0, bs = mx / 32767, q = rint(v * isx); written to LDS as byte planes.
// The sum of squares is taken per 128-column block (each lane fma-sums its 16 columns in order, the 8 lanes add with
// DPP), then wave 0 adds the block sums in a fixed tree: the same value for every workgroup size.  (The reference sums
// sequentially, kernels.cpp:185; the order differs.)
struct ActRegs {
  float4 x[2][4];
  float4 w[2][4];
};
// PRO_NORM_SUM: the input is x + y, y the sum of np <= kMaxParts partial vectors `pstride` floats apart, and workgroup
// 0 stores that input to xsum.  When the workgroup has at least two threads per 16-column piece, nsets = min(np,
// threads / pieces) sets of `pieces` threads share the partials (set s adds parts s, s + nsets, ... in order; sets
// 1 .. nsets - 1 hand their sums to set 0 through scr, [nsets - 1][cols] floats), so every load goes out at once:
// y = (S_0 + S_1) + ... ; otherwise the owners add the parts one by one, y = ((p_0 + p_1) + p_2) + ...
constexpr int kMaxParts = 8;
__host__ __device__ inline int act_part_sets(int cols, int threads, int np) {
  const int pieces = cols / kQB * 8;
  return 2 * pieces <= threads ? (np < threads / pieces ? np : threads / pieces) : 1;
}
__device__ __forceinline__ void f4add(float4 &a, const float4 &b) { a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w; }
// sets path (act_part_sets >= 2, one pass): thread t % pieces owns columns 16 (t % pieces) .. + 15 (the set-0 thread)
__device__ inline void act_load_sum_sets(const float *x, const float *w, int cols, ActRegs &r, const float *part, int np,
                                         size_t pstride, float *xsum, float *scr, int nsets) {
  const int pieces = cols / kQB * 8, t = threadIdx.x, set = t / pieces, c0 = (t % pieces) * 16;
  if (set == 0)
#pragma unroll
    for (int k = 0; k < 4; k++) { r.x[0][k] = *(const float4 *)(x + c0 + 4 * k); r.w[0][k] = *(const float4 *)(w + c0 + 4 * k); }
  float4 y[4];
  if (set < nsets) {
    constexpr int Q = kMaxParts / 2;   // parts per set (nsets >= 2)
    float4 v[Q][4];
#pragma unroll
    for (int q = 0; q < Q; q++)
      if (set + q * nsets < np)
#pragma unroll
        for (int k = 0; k < 4; k++) v[q][k] = *(const float4 *)(part + (set + q * nsets) * pstride + c0 + 4 * k);
#pragma unroll
    for (int k = 0; k < 4; k++) y[k] = v[0][k];
#pragma unroll
    for (int q = 1; q < Q; q++)
      if (set + q * nsets < np)
#pragma unroll
        for (int k = 0; k < 4; k++) f4add(y[k], v[q][k]);
    if (set > 0)
#pragma unroll
      for (int k = 0; k < 4; k++) *(float4 *)(scr + (set - 1) * cols + c0 + 4 * k) = y[k];
  }
  __syncthreads();
  if (set == 0) {
    for (int s = 1; s < nsets; s++)
#pragma unroll
      for (int k = 0; k < 4; k++) f4add(y[k], *(const float4 *)(scr + (s - 1) * cols + c0 + 4 * k));
#pragma unroll
    for (int k = 0; k < 4; k++) {
      f4add(r.x[0][k], y[k]);
      if (blockIdx.x == 0) *(float4 *)(xsum + c0 + 4 * k) = r.x[0][k];
    }
  }
  __syncthreads();   // scr is the block-sum area act_build uses next
}

template <int PRO>
__device__ __forceinline__ void act_load(const float *x, const float *w, int cols, ActRegs &r, const float *part = nullptr,
                                         int np = 0, size_t pstride = 0, float *xsum = nullptr, float *scr = nullptr) {
  const int nb = cols / kQB, per = (int)blockDim.x / 8, sub = threadIdx.x & 7;
  if (PRO == PRO_NORM_SUM) {
    const int nsets = act_part_sets(cols, (int)blockDim.x, np);
    if (nsets >= 2) { act_load_sum_sets(x, w, cols, r, part, np, pstride, xsum, scr, nsets); return; }
  }
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int b = p * per + (int)(threadIdx.x >> 3);
    if (b < nb) {
      const int c0 = b * kQB + sub * 16;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        r.x[p][k] = *(const float4 *)(x + c0 + 4 * k);
        if (PRO != PRO_QUANT) r.w[p][k] = *(const float4 *)(w + c0 + 4 * k);
      }
    }
  }
  if (PRO == PRO_NORM_SUM)   // the owners add the parts one by one
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int b = p * per + (int)(threadIdx.x >> 3);
      if (b < nb) {
        const int c0 = b * kQB + sub * 16;
        float4 y[4];
#pragma unroll
        for (int k = 0; k < 4; k++) y[k] = *(const float4 *)(part + c0 + 4 * k);
        for (int j = 1; j < np; j++)
#pragma unroll
          for (int k = 0; k < 4; k++) f4add(y[k], *(const float4 *)(part + j * pstride + c0 + 4 * k));
#pragma unroll
        for (int k = 0; k < 4; k++) {
          f4add(r.x[p][k], y[k]);
          if (blockIdx.x == 0) *(float4 *)(xsum + c0 + 4 * k) = r.x[p][k];
        }
      }
    }
}
__device__ __forceinline__ float f4get(const float4 &v, int j) { return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w)); }

// CM (chunk-major, the q1 kernels): the 16-column piece k of 128-column block b is stored at byte (k * nb + b) * 16 of
// each plane instead of b * 128 + 16 k, so lanes that own consecutive blocks read consecutive 16-byte pieces (the
// row-major layout puts them 128 bytes apart: every lane in the same LDS banks).
template <int PRO, bool CM = false>
__device__ void act_build(const ActRegs &r, float eps, int cols, const ActView &a) {
  const int nb = cols / kQB, per = (int)blockDim.x / 8, sub = threadIdx.x & 7;
  float inv = 1.f;
  if (PRO != PRO_QUANT) {
    float *bss = (float *)a.sums;   // block sums of squares; the sums area is free until the main loop
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const int b = p * per + (int)(threadIdx.x >> 3);
      if (b < nb) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 16; k++) { const float v = f4get(r.x[p][k >> 2], k & 3); s = __builtin_fmaf(v, v, s); }
        s += dpp_f<kDppQuadXor1>(s);
        s += dpp_f<kDppQuadXor2>(s);
        s += dpp_f<kDppHalfMirror>(s);
        if (sub == 0) bss[b] = s;
      }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      float v[4];
#pragma unroll
      for (int k = 0; k < 4; k++) { const int b = (int)threadIdx.x + 64 * k; v[k] = b < nb ? bss[b] : 0.f; }
      const float t = wave_sum((v[0] + v[1]) + (v[2] + v[3]));
      if (threadIdx.x == 0) a.red[0] = 1.f / sqrtf(t / (float)cols + eps);
    }
    __syncthreads();
    inv = a.red[0];
  }
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const int b = p * per + (int)(threadIdx.x >> 3);
    if (b < nb) {
      const int c0 = b * kQB + sub * 16;
      float v[16];
#pragma unroll
      for (int k = 0; k < 16; k++) {
        v[k] = f4get(r.x[p][k >> 2], k & 3);
        if (PRO != PRO_QUANT) v[k] = v[k] * inv * f4get(r.w[p][k >> 2], k & 3);
      }
      float m = 0;
#pragma unroll
      for (int k = 0; k < 16; k++) m = fmaxf(m, fabsf(v[k]));
      m = max8_f(m);
      const float isx = m > 0 ? kActMax / m : 0.f;
      if (sub == 0) a.bs[b] = m / kActMax;
      uint32_t hw[4], lw[4]; int ls = 0, gs = 0;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t hh = 0, ll = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int q = (int)__builtin_rintf(v[4 * k + j] * isx);
          hh |= (uint32_t)((q >> 8) & 0xff) << (8 * j);
          ll |= (uint32_t)(q & 0xff) << (8 * j);
          ls += q & 0xff; gs += q;
        }
        hw[k] = hh; lw[k] = ll;
      }
      const int at = CM ? (sub * nb + b) * 16 : c0;
      *(uint4 *)(a.xh + at) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      *(uint4 *)(a.xl + at) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
      ls = sum8_i(ls);
      if (sub == 0) a.lsum[b] = ls;
      gs += dpp_i<kDppQuadXor1>(gs);
      if ((sub & 1) == 0) a.gsum[c0 / 32] = gs;
    }
  }
  __syncthreads();
}

// row `tok` of the embedding as f32 (row_f32, /root/reference/src/kernels.cpp:146-182): q8 q * scale, q4 nibble - 8 times
// its group's fp16 scale, f32 copied; out-of-range ids are clamped (the host validates them first)
__device__ inline void embed_row(const DMat &e, int tok, float *x, int tid, int nthreads) {
  tok = tok < 0 ? 0 : (tok >= e.rows ? e.rows - 1 : tok);
  const int n = e.cols;
  if (e.kind == MK_Q8) {   // 16 columns per thread and step (n is a multiple of 128): one 16-byte load, four float4 stores
    const int8_t *q = (const int8_t *)e.q + (size_t)tok * n; const float s = ((const float *)e.s)[tok];
    for (int c = 16 * tid; c < n; c += 16 * nthreads) {
      const int4 v = *(const int4 *)(q + c);
      const int w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int k = 0; k < 4; k++)
        *(float4 *)(x + c + 4 * k) = make_float4((float)(int8_t)(w[k] & 255) * s, (float)(int8_t)((w[k] >> 8) & 255) * s,
                                                 (float)(int8_t)((w[k] >> 16) & 255) * s, (float)(int8_t)(w[k] >> 24) * s);
    }
  } else if (e.kind == MK_Q4) {
    const uint8_t *q = (const uint8_t *)e.q + (size_t)tok * (n / 2); const uint16_t *s = (const uint16_t *)e.s + (size_t)tok * (n / 32);
    for (int i = tid; i < n / 2; i += nthreads) {
      const int g = i / 16, j = i % 16; const float sc = half_bits_to_float(s[g]); const uint8_t b = q[i];
      x[32 * g + j] = (float)((int)(b & 15) - 8) * sc; x[32 * g + j + 16] = (float)((int)(b >> 4) - 8) * sc;
    }
  } else if (e.kind == MK_Q1) {   // row_f32 of a q1 row (kernels.cpp:162-166): (2 bit - 1) * scale
    const uint8_t *q = (const uint8_t *)e.q + (size_t)tok * (n / 8); const uint16_t *s = (const uint16_t *)e.s + (size_t)tok * (n / 128);
    for (int i = tid; i < n; i += nthreads) x[i] = ((q[i >> 3] >> (i & 7)) & 1 ? 1.f : -1.f) * half_bits_to_float(s[i >> 7]);
  } else {
    const float *q = (const float *)e.q + (size_t)tok * n;
    for (int i = tid; i < n; i += nthreads) x[i] = q[i];
  }
}

}  // namespace qph
