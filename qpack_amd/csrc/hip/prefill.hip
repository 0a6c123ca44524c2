// gfx950 kernels of the batched prompt path (qp::Model::prefill, /root/reference/src/model_llama.cpp:66-130).
//
// A prompt chunk of B tokens turns every projection into a matrix product Y[B, rows] = X[B, cols] W^T, the one
// compute-bound step of the token loop, done on the int8 matrix cores:
//   - each token's activation is quantised exactly as in decode (the shared prologue of act.hpp: RMSNorm optional,
//     then quant_rows' int16 per 128-column block) and stored as two int8 planes, hi = q >> 8 and lo = (q & 255) - 128,
//     so q = 256 hi + lo + 128;
//   - v_mfma_i32_16x16x64_i8 multiplies weight rows by each plane; per 128-column block
//         isum = 256 (W . hi) + (W . lo) + 128 sum(W)
//     is the exact int32 accumulator of rows_q8 / mm_q8 (/root/reference/src/kernels_x86.cpp:55-71, 287-340);
//   - the float epilogue replays rows_q8's order per (row, token): acc = fma(bs[token][b], (float)isum_b, acc) over
//     blocks in order, y = acc * scale[row]; every prompt token's projection is therefore bit-identical to a decode
//     step's (the reference's own batched mm_q8 sums lane partials in another float order, within the logit tolerance).
#include "act.hpp"
#include "launch.hpp"

namespace qph {

typedef int v4i __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ embeddings of a token batch
__global__ __launch_bounds__(256) void k_pf_embed(DMat e, const int *toks, float *X, int ldx) {
  embed_row(e, toks[blockIdx.x], X + (size_t)blockIdx.x * ldx, threadIdx.x, blockDim.x);
}
hipError_t launch_pf_embed(const DMat &embed, const int *toks, int B, float *X, int ldx, hipStream_t st) {
  if (B <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_pf_embed, dim3(B), dim3(256), 0, st, embed, toks, X, ldx);
  return hipGetLastError();
}

// ------------------------------------------------------------------ per-token quantisation into int8 planes
// one workgroup per token: the decode prologue (act_load / act_build) builds the planes in LDS, then they are copied
// out: XH = q >> 8, XL = (q & 255) - 128 (the unsigned low byte with its top bit flipped), XB = block scales
template <int PRO>
__global__ __launch_bounds__(1024) void k_pf_quant(PfQuantArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int t = blockIdx.x, cols = a.cols, nb = cols / kQB;
  const ActView av = act_view(smem, cols);
  ActRegs ar;
  act_load<PRO>(a.x + (size_t)t * a.ldx, a.norm_w, cols, ar);
  act_build<PRO>(ar, a.eps, cols, av);
  int8_t *xh = a.xh + (size_t)t * a.ldq, *xl = a.xl + (size_t)t * a.ldq;
  for (int c = threadIdx.x * 16; c < cols; c += blockDim.x * 16) {
    const uint4 h = *(const uint4 *)(av.xh + c), l = *(const uint4 *)(av.xl + c);
    *(uint4 *)(xh + c) = h;
    *(uint4 *)(xl + c) = make_uint4(l.x ^ 0x80808080u, l.y ^ 0x80808080u, l.z ^ 0x80808080u, l.w ^ 0x80808080u);
  }
  for (int b = threadIdx.x; b < nb; b += blockDim.x) a.xb[(size_t)t * a.ldb + b] = av.bs[b];
}
hipError_t launch_pf_quant(int pro, const PfQuantArgs &a, int B, hipStream_t st) {
  if (B <= 0) return hipSuccess;
  if (a.cols % kQB || a.cols > 32768 || a.ldq % 16) return hipErrorInvalidValue;
  const size_t lds = mv_lds_bytes(a.cols, 16, 0);
  if (pro == PRO_NORM) hipLaunchKernelGGL(k_pf_quant<PRO_NORM>, dim3(B), dim3(1024), lds, st, a);
  else hipLaunchKernelGGL(k_pf_quant<PRO_QUANT>, dim3(B), dim3(1024), lds, st, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ int8 MFMA matrix product (q8 weights)
// Workgroup tile: 128 weight rows x 128 tokens, 4 waves in a 2 x 2 grid of 64 x 64, each a 4 x 4 grid of 16 x 16
// MFMA tiles.  K advances one 128-column block at a time (two 64-deep MFMA steps per plane) through double-buffered
// LDS: weight rows [128][144 B] (16 B padding per row keeps 16-lane fragment reads conflict-free), the two activation
// planes [128][144 B] each, the block's row sums of W and the tokens' block scales.
//   fragments (v_mfma_i32_16x16x64_i8): lane l reads A = W[row l % 16][16 (l / 16) + 0..15] and B = plane[token l % 16]
//   [16 (l / 16) + 0..15] - the same k set for A and B; C lane l holds rows 4 (l / 16) + 0..3 of token l % 16.
constexpr int kGM = 128, kGN = 128, kGS = 144;
size_t gemm_lds_bytes() { return (size_t)2 * (kGM + 2 * kGN) * kGS + 2 * kGM * 4 + 2 * kGN * 4; }

__global__ __launch_bounds__(256) void k_gemm_q8(GemmArgs a) {
  extern __shared__ __align__(16) char smem[];
  int8_t *sw = (int8_t *)smem;                        // [2][kGM][kGS]
  int8_t *sh = sw + 2 * kGM * kGS;                     // [2][kGN][kGS]
  int8_t *sl = sh + 2 * kGN * kGS;                     // [2][kGN][kGS]
  int *ssum = (int *)(sl + 2 * kGN * kGS);             // [2][kGM] row sums of W over the block
  float *sbs = (float *)(ssum + 2 * kGM);              // [2][kGN] block scale of each token
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1, lr = lane & 15, lg = lane >> 4;
  const int r0 = blockIdx.y * kGM, t0 = blockIdx.x * kGN;
  const int nb = a.cols / kQB;

  // global -> registers: 4 x 16 B of weights, 4 x 16 B of each plane per thread (row / token tid / 8 + 32 j,
  // 16-byte segment tid % 8), and one block scale (tid < 128)
  v4i gw[4], gh[4], gl[4];
  float gb = 0.f;
  const int seg = tid & 7;
  auto gload = [&](int kb) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int row = (tid >> 3) + 32 * j;
      const int r = r0 + row, t = t0 + row;
      const v4i z = {0, 0, 0, 0};
      gw[j] = r < a.rows ? *(const v4i *)(a.w + (size_t)r * a.cols + kb * kQB + seg * 16) : z;
      gh[j] = t < a.ntok ? *(const v4i *)(a.xh + (size_t)t * a.ldq + kb * kQB + seg * 16) : z;
      gl[j] = t < a.ntok ? *(const v4i *)(a.xl + (size_t)t * a.ldq + kb * kQB + seg * 16) : z;
    }
    if (tid < kGN) gb = t0 + tid < a.ntok ? a.xb[(size_t)(t0 + tid) * a.ldb + kb] : 0.f;
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int row = (tid >> 3) + 32 * j;
      *(v4i *)(sw + ((size_t)buf * kGM + row) * kGS + seg * 16) = gw[j];
      *(v4i *)(sh + ((size_t)buf * kGN + row) * kGS + seg * 16) = gh[j];
      *(v4i *)(sl + ((size_t)buf * kGN + row) * kGS + seg * 16) = gl[j];
      int s = __builtin_amdgcn_sdot4(gw[j].x, 0x01010101, 0, false);
      s = __builtin_amdgcn_sdot4(gw[j].y, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(gw[j].z, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(gw[j].w, 0x01010101, s, false);
      s = sum8_i(s);   // the 8 segments of the row sit in 8 consecutive lanes
      if (seg == 0) ssum[buf * kGM + row] = s;
    }
    if (tid < kGN) sbs[buf * kGN + tid] = gb;
  };

  float acc[4][4][4];
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 4; ni++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[mi][ni][i] = 0.f;

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kb = 0; kb < nb; kb++) {
    const int buf = kb & 1;
    if (kb + 1 < nb) gload(kb + 1);
    v4i ch[4][4], cl[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < 4; ni++) { ch[mi][ni] = (v4i){0, 0, 0, 0}; cl[mi][ni] = (v4i){0, 0, 0, 0}; }
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      v4i A[4];
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
        A[mi] = *(const v4i *)(sw + ((size_t)buf * kGM + wr * 64 + mi * 16 + lr) * kGS + ks * 64 + lg * 16);
#pragma unroll
      for (int ni = 0; ni < 4; ni++) {
        const size_t o = ((size_t)buf * kGN + wc * 64 + ni * 16 + lr) * kGS + ks * 64 + lg * 16;
        const v4i bh = *(const v4i *)(sh + o), bl = *(const v4i *)(sl + o);
#pragma unroll
        for (int mi = 0; mi < 4; mi++) {
          ch[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mi], bh, ch[mi][ni], 0, 0, 0);
          cl[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[mi], bl, cl[mi][ni], 0, 0, 0);
        }
      }
    }
    // the block's exact int32 sums, then rows_q8's fma step
#pragma unroll
    for (int mi = 0; mi < 4; mi++) {
      int ws[4];
#pragma unroll
      for (int i = 0; i < 4; i++) ws[i] = 128 * ssum[buf * kGM + wr * 64 + mi * 16 + 4 * lg + i];
#pragma unroll
      for (int ni = 0; ni < 4; ni++) {
        const float b = sbs[buf * kGN + wc * 64 + ni * 16 + lr];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int isum = ch[mi][ni][i] * 256 + cl[mi][ni][i] + ws[i];
          acc[mi][ni][i] = __builtin_fmaf(b, (float)isum, acc[mi][ni][i]);
        }
      }
    }
    if (kb + 1 < nb) sstore(buf ^ 1);
    __syncthreads();
  }
  // y = acc * scale (+ bias), or y += (residual stream)
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 4; ni++) {
      const int t = t0 + wc * 64 + ni * 16 + lr;
      if (t >= a.ntok) continue;
      float *yt = a.y + (size_t)t * a.ldy;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = r0 + wr * 64 + mi * 16 + 4 * lg + i;
        if (r >= a.rows) continue;
        float v = acc[mi][ni][i] * a.scale[r];
        if (a.resid) yt[r] = yt[r] + v;
        else { if (a.bias) v = v + a.bias[r]; yt[r] = v; }
      }
    }
}

hipError_t launch_gemm(const GemmArgs &a, hipStream_t st) {
  if (a.ntok <= 0) return hipSuccess;
  if (a.cols % kQB || a.rows <= 0 || a.ldq % 16 || a.ldq < a.cols || a.ldb < a.cols / kQB) return hipErrorInvalidValue;
  const dim3 grid((a.ntok + kGN - 1) / kGN, (a.rows + kGM - 1) / kGM);
  hipLaunchKernelGGL(k_gemm_q8, grid, dim3(256), gemm_lds_bytes(), st, a);
  return hipGetLastError();
}

}  // namespace qph
