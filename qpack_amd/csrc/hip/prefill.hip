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
#include <math.h>
#include <stdlib.h>

#include <algorithm>

#include "act.hpp"
#include "launch.hpp"

namespace qph {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

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
  if (a.xbt)
    for (int b = threadIdx.x; b < nb; b += blockDim.x) a.xbt[(size_t)b * a.ldbt + t] = av.bs[b];
  if (a.xg)   // sum of q per 32-column group (the q4 product's nibble-offset correction)
    for (int g = threadIdx.x; g < cols / 32; g += blockDim.x) a.xg[(size_t)t * a.ldg + g] = av.gsum[g];
}
hipError_t launch_pf_quant(int pro, const PfQuantArgs &a, int B, hipStream_t st) {
  if (B <= 0) return hipSuccess;
  if (a.cols % kQB || a.cols > 32768 || a.ldq % 16) return hipErrorInvalidValue;
  const size_t lds = mv_lds_bytes(a.cols, 16, 0);
  // the fewest threads whose two act_load passes cover the row (8 per 128-column block and pass): small workgroups,
  // so several tokens' load -> reduce -> store chains overlap on a CU
  const int nb = a.cols / kQB, threads = std::min(1024, std::max(256, (4 * nb + 63) / 64 * 64));
  if (pro == PRO_NORM) hipLaunchKernelGGL(k_pf_quant<PRO_NORM>, dim3(B), dim3(threads), lds, st, a);
  else hipLaunchKernelGGL(k_pf_quant<PRO_QUANT>, dim3(B), dim3(threads), lds, st, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ int8 MFMA matrix product (q8 weights)
// Workgroup tile: 128 weight rows x 128 tokens, 8 waves (two per SIMD, so one wave's fp32 epilogue overlaps the other's
// matrix-core work) in a 2 x 4 grid of 64 rows x 32 tokens, each a 4 x 2 grid of 16 x 16 MFMA tiles.  K advances one
// 128-column block at a time (two 64-deep MFMA steps per plane).  Operands reach LDS by direct global->LDS loads
// (global_load_lds_dwordx4: a wave instruction lands 64 x 16 B contiguously) in a 3-stage ring, so two blocks are
// always in flight while one is multiplied; no operand passes through registers.
//   stage layout: weights, hi plane, lo plane, each [128 rows][128 B] with the 16-byte segments XOR-swizzled
//   (physical segment = segment ^ (row & 7)) so 16-lane fragment reads hit distinct banks; the tokens' block scales;
//   the weight rows' block sums (precomputed once per matrix, k_rowsum_q8).
//   fragments (v_mfma_i32_16x16x64_i8): lane l reads A = W[row l % 16][16 (l / 16) + 0..15] and B = plane[token l % 16]
//   [16 (l / 16) + 0..15] - the same k set for A and B; C lane l holds rows 4 (l / 16) + 0..3 of token l % 16.
// Rows or tokens past the end load a clamped (valid) address; their results are never stored.
constexpr int kGM = 128, kGN = 128, kGStages = 3, kGWaves = 8;
constexpr int kGStage = 3 * 128 * 128 + 128 * 4 + 128 * 4;   // bytes per stage
size_t gemm_lds_bytes() { return (size_t)kGStages * kGStage; }

// LDS reads of DMA-filled stages, kept out of the compiler's sight: it cannot tell which stage a DMA fills and would
// otherwise wait for every load in flight before each read.  The results are only valid after the explicit lgkmcnt
// wait that takes them as operands, so no use can be scheduled before it.
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)(const lds_void_t *)p; }
__device__ __forceinline__ v4i lds_read16(uint32_t addr) {
  v4i r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
__device__ __forceinline__ float lds_read4(uint32_t addr) {
  float r;
  asm volatile("ds_read_b32 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}
// the same with a constant byte offset folded into the instruction
template <int OFF>
__device__ __forceinline__ v4i lds_read16o(uint32_t addr) {
  v4i r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int OFF>
__device__ __forceinline__ float lds_read4o(uint32_t addr) {
  float r;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// 128 x the sum of each weight row over each 128-column block, block-major: out[block][ws_pitch(rows)] (exact int32;
// isum = 256 hi + lo + 128 sum(W))
__global__ __launch_bounds__(256) void k_rowsum_q8(const int8_t *w, int rows, int cols, int *out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * (cols / kQB)) return;
  const int row = (int)(i % rows), blk = (int)(i / rows);
  const v4i *p = (const v4i *)(w + (size_t)row * cols + (size_t)blk * kQB);
  int s = 0;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const v4i v = p[k];
    s = __builtin_amdgcn_sdot4(v.x, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(v.y, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(v.z, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(v.w, 0x01010101, s, false);
  }
  out[(size_t)blk * ws_pitch(rows) + row] = 128 * s;
}
hipError_t launch_rowsum_q8(const int8_t *w, int rows, int cols, int *out, hipStream_t st) {
  if (cols % kQB || rows <= 0) return hipErrorInvalidValue;
  const int64_t n = (int64_t)rows * (cols / kQB);
  hipLaunchKernelGGL(k_rowsum_q8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, rows, cols, out);
  return hipGetLastError();
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.f + exp_poly(0.f - g)) * u; }   // kernels_x86.cpp:427-431
// silu_mul's first half: silu_mul(g, u) == silu_f(g) * u, the same operations in the same order
__device__ __forceinline__ float silu_f(float g) { return g / (1.f + exp_poly(0.f - g)); }

// rows rb .. rb + 3 of token row yt (the MFMA C layout gives a lane four consecutive rows of one token): y = v (* row
// scale when `scaled`), then y += the residual, y = that + bias, or y = silu(gate) * that; one 16-byte access where the
// rows are in range and the token rows 16-byte aligned
__device__ __forceinline__ void gemm_store4(const GemmArgs &a, float *yt, int rb, float4 v, bool scaled) {
  const float *gt = a.gate ? a.gate + (yt - a.y) : nullptr;   // the gate's token row
  if (rb + 3 < a.rows && (a.ldy & 3) == 0) {
    if (scaled) { const float4 s = *(const float4 *)(a.scale + rb); v.x = v.x * s.x; v.y = v.y * s.y; v.z = v.z * s.z; v.w = v.w * s.w; }
    if (gt) {
      const float4 g = *(const float4 *)(gt + rb);
      v = make_float4(silu_mul(g.x, v.x), silu_mul(g.y, v.y), silu_mul(g.z, v.z), silu_mul(g.w, v.w));
    } else if (a.resid) {
      const float4 o = *(const float4 *)(yt + rb);
      v = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
    } else if (a.bias) {
      const float4 b = *(const float4 *)(a.bias + rb);
      v = make_float4(v.x + b.x, v.y + b.y, v.z + b.z, v.w + b.w);
    }
    *(float4 *)(yt + rb) = v;
    return;
  }
  const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = rb + i;
    if (r >= a.rows) continue;
    float x = scaled ? vv[i] * a.scale[r] : vv[i];
    if (gt) yt[r] = silu_mul(gt[r], x);
    else if (a.resid) yt[r] = yt[r] + x;
    else { if (a.bias) x = x + a.bias[r]; yt[r] = x; }
  }
}

// multi-matrix launches: row tile r0 / rt of the grid -> the matrix it belongs to (wave-uniform), whose fields replace
// the launch's; returns the tile's first row within that matrix
__device__ __forceinline__ int gemm_segment(GemmArgs &a, int r0, int rt) {
  if (a.nseg < 2) return r0;
  const int tile = r0 / rt;
  int base = 0, first = 0;
  bool found = false;
#pragma unroll
  for (int s = 0; s < kGemmMaxSeg; s++) {   // constant indices: the segment table stays in kernel-argument memory
    if (!found && s < a.nseg) {
      const GemmSeg &g = a.seg[s];
      const int nt = (g.rows + rt - 1) / rt;
      if (tile < base + nt || s == a.nseg - 1) {
        a.w = g.w; a.scale = g.scale; a.wsum = g.wsum; a.q4ns = g.q4ns; a.q4sc = g.q4sc;
        a.bias = g.bias; a.y = g.y; a.rows = g.rows; a.ldy = g.ldy;
        first = base; found = true;
      }
      base += nt;
    }
  }
  return (tile - first) * rt;
}

__global__ __launch_bounds__(512) void k_gemm_q8(GemmArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 2, wc = wave & 3, lr = lane & 15, lg = lane >> 4;
  // XCD-aware tile order: workgroups are dealt to the 8 XCDs round-robin (linear id % 8).  When the token tiles split
  // evenly over the XCDs, XCD x owns its eighth of them over all weight rows: its activation planes (a few MiB) stay in
  // its L2 while the weights stream past from the last-level cache.  Otherwise XCD x owns the x-th eighth of the tiles
  // in row-major order (token tile fastest), so a weight tile is reused from L2 by the token tiles that need it.
  // paired (a.w2): the tile's 128 weight rows are 64 rows of the gate matrix (waves 0-3) and the same 64 rows of the
  // up matrix (waves 4-7)
  const bool paired = a.w2 != nullptr;
  const int RT = paired ? kGM / 2 : kGM;   // output rows per tile
  int r0, t0;
  {
    const int ntt = gridDim.x, nrt = gridDim.y, n = ntt * nrt, lin = blockIdx.y * gridDim.x + blockIdx.x;
    const int xcd = lin & 7, k = lin >> 3;
    if (ntt % 8 == 0) {
      // each XCD: ntt / 8 token tiles x all nrt row tiles = n / 8 tiles, exactly its share of the round-robin
      const int tn = ntt >> 3;
      r0 = (k / tn) * RT; t0 = (xcd * tn + k % tn) * kGN;
    } else {
      const int base = n >> 3, rem = n & 7;
      const int tile = xcd * base + min(xcd, rem) + k;
      r0 = (tile / ntt) * RT; t0 = (tile % ntt) * kGN;
    }
  }
  r0 = gemm_segment(a, r0 + a.tile0 * RT, RT);
  const int nb = a.cols / kQB;

  // this lane's DMA sources.  Per stage the 48 1-KiB row groups (16 each of weights, hi plane, lo plane; 8 rows per
  // group) go 6 to a wave; the lane fetches the 16-byte segment that belongs at physical position lane % 8 of its row.
  const int drow = lane >> 3, dseg = (lane & 7) ^ drow;
  const int8_t *src[6];
  int dst[6];
#pragma unroll
  for (int j = 0; j < 6; j++) {
    const int q = wave * 6 + j, m = q >> 4, row = 8 * (q & 15) + drow;
    dst[j] = m * 128 * 128 + 8 * (q & 15) * 128;
    if (m == 0) {
      const int8_t *wm = paired && row >= 64 ? a.w2 : a.w;
      src[j] = wm + (size_t)min(r0 + (paired ? (row & 63) : row), a.rows - 1) * a.cols + dseg * 16;
    } else {
      src[j] = (m == 1 ? a.xh : a.xl) + (size_t)min(t0 + row, a.ntok - 1) * a.ldq + dseg * 16;
    }
  }
  // one 4-byte load per wave and stage: waves 0 / 1 (and 4 / 5) the block scales of tokens 64 (w & 1) + lane, waves
  // 2 / 3 (and 6 / 7) the block sums of rows 64 (w & 1) + lane - duplicates write identical bytes to the same slot,
  // so every wave issues the same number of loads
  const int half = wave & 1;
  const bool sums = (wave & 2) != 0;
  const int *wsm = paired && half ? a.wsum2 : a.wsum;
  const char *esrc = sums ? (const char *)(wsm + min(r0 + (paired ? 0 : 64 * half) + lane, a.rows - 1))
                          : (const char *)(a.xb + (size_t)min(t0 + 64 * half + lane, a.ntok - 1) * a.ldb);
  const size_t estep = sums ? 4 * (size_t)ws_pitch(a.rows) : 4;   // bytes per block
  const int edst = 3 * 128 * 128 + (sums ? 512 : 0) + 256 * half;
  auto issue = [&](int kb) {
    char *st = smem + (size_t)(kb % kGStages) * kGStage;
#pragma unroll
    for (int j = 0; j < 6; j++) dma16(src[j] + kb * kQB, st + dst[j]);
    dma4(esrc + kb * estep, st + edst);
  };

  float acc[4][2][4];
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[mi][ni][i] = 0.f;

  // per-lane LDS offsets within a stage.  Fragment rows (and tokens) 16 apart share the swizzle (row & 7), so the
  // mi / ni / plane steps are constant offsets folded into the reads: per block only the stage base is added.
  //   A[mi] of step ks: W row wr 64 + 16 mi + lr, segment 4 ks + lg; B[ni] likewise for token wc 32 + 16 ni + lr
  uint32_t aoff[2], boff[2];
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    const int seg = ks * 4 + lg, row = wr * 64 + lr, tok = wc * 32 + lr;
    aoff[ks] = row * 128 + ((seg ^ (row & 7)) << 4);
    boff[ks] = 128 * 128 + tok * 128 + ((seg ^ (tok & 7)) << 4);
  }
  const uint32_t soff = 3 * 128 * 128 + 512 + 4 * (wr * 64 + 4 * lg);   // row block sums, + 64 mi
  const uint32_t toff = 3 * 128 * 128 + 4 * (wc * 32 + lr);             // token block scales, + 64 ni
  const uint32_t sbase = lds_addr(smem);

  // software pipeline: block kb's MFMAs are issued while block kb - 1's epilogue (its exact int32 sums -> rows_q8's
  // fma step) runs on the vector ALU - independent work the matrix cores and the VALU overlap
  auto epilogue_half = [&](const v4i (&pch)[4][2], const v4i (&pcl)[4][2], const float (&pbs)[2], int ni) {
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int isum = pch[mi][ni][i] * 256 + pcl[mi][ni][i];   // the lo accumulator started at 128 sum(W)
        acc[mi][ni][i] = __builtin_fmaf(pbs[ni], (float)isum, acc[mi][ni][i]);
      }
  };
  // block kb into (ch, cl, bsc); the previous block's (pch, pcl, pbs) epilogue under its MFMAs when `prev`
  auto block = [&](int kb, v4i (&ch)[4][2], v4i (&cl)[4][2], float (&bsc)[2], const v4i (&pch)[4][2],
                   const v4i (&pcl)[4][2], const float (&pbs)[2], bool prev) {
    // this wave's loads of block kb have landed (block kb + 1's 7 may still be in flight), then everyone's
    if (kb + 1 < nb) asm volatile("s_waitcnt vmcnt(7)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (kb + 2 < nb) issue(kb + 2);   // into the stage everyone finished reading in the previous iteration
    const uint32_t st = sbase + (uint32_t)((kb % kGStages) * kGStage);
    // both steps' fragments are read up front; step 1's land while step 0 multiplies
    v4i A[2][4], BH[2][2], BL[2][2];
    v4i wsv[4];
    {
      const uint32_t pa = st + aoff[0], pb = st + boff[0], ps = st + soff, pt = st + toff;
      A[0][0] = lds_read16o<0>(pa); A[0][1] = lds_read16o<2048>(pa); A[0][2] = lds_read16o<4096>(pa); A[0][3] = lds_read16o<6144>(pa);
      BH[0][0] = lds_read16o<0>(pb); BH[0][1] = lds_read16o<2048>(pb);
      BL[0][0] = lds_read16o<16384>(pb); BL[0][1] = lds_read16o<16384 + 2048>(pb);
      wsv[0] = lds_read16o<0>(ps); wsv[1] = lds_read16o<64>(ps); wsv[2] = lds_read16o<128>(ps); wsv[3] = lds_read16o<192>(ps);
      bsc[0] = lds_read4o<0>(pt); bsc[1] = lds_read4o<64>(pt);
    }
    {
      const uint32_t pa = st + aoff[1], pb = st + boff[1];
      A[1][0] = lds_read16o<0>(pa); A[1][1] = lds_read16o<2048>(pa); A[1][2] = lds_read16o<4096>(pa); A[1][3] = lds_read16o<6144>(pa);
      BH[1][0] = lds_read16o<0>(pb); BH[1][1] = lds_read16o<2048>(pb);
      BL[1][0] = lds_read16o<16384>(pb); BL[1][1] = lds_read16o<16384 + 2048>(pb);
    }
    // LDS reads complete in order: 8 outstanding = step 1's
    asm volatile("s_waitcnt lgkmcnt(8)"
                 : "+v"(A[0][0]), "+v"(A[0][1]), "+v"(A[0][2]), "+v"(A[0][3]), "+v"(BH[0][0]), "+v"(BH[0][1]),
                   "+v"(BL[0][0]), "+v"(BL[0][1]), "+v"(bsc[0]), "+v"(bsc[1]), "+v"(wsv[0]), "+v"(wsv[1]), "+v"(wsv[2]),
                   "+v"(wsv[3]));
    // the block's row sums start the lo accumulators (isum = 256 hi + lo + 128 sum(W)); hi starts at zero
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++) { ch[mi][ni] = (v4i){0, 0, 0, 0}; cl[mi][ni] = wsv[mi]; }
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      if (ks == 1)
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(A[1][0]), "+v"(A[1][1]), "+v"(A[1][2]), "+v"(A[1][3]), "+v"(BH[1][0]), "+v"(BH[1][1]),
                       "+v"(BL[1][0]), "+v"(BL[1][1]));
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int mi = 0; mi < 4; mi++) {
          ch[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ks][mi], BH[ks][ni], ch[mi][ni], 0, 0, 0);
          cl[mi][ni] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[ks][mi], BL[ks][ni], cl[mi][ni], 0, 0, 0);
        }
      if (prev) epilogue_half(pch, pcl, pbs, ks);   // half of the previous block's epilogue under each step's MFMAs
    }
  };
  v4i ch[4][2], cl[4][2], pch[4][2], pcl[4][2];
  float bsc[2], pbs[2];
  issue(0);
  if (nb > 1) issue(1);
  for (int kb = 0; kb < nb; kb++) {
    block(kb, ch, cl, bsc, pch, pcl, pbs, kb > 0);
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++) { pch[mi][ni] = ch[mi][ni]; pcl[mi][ni] = cl[mi][ni]; }
    pbs[0] = bsc[0]; pbs[1] = bsc[1];
  }
  epilogue_half(pch, pcl, pbs, 0);
  epilogue_half(pch, pcl, pbs, 1);
  if (paired) {
    // the gate waves hand gate = acc * scale to the up waves through LDS ([128 tokens][64 rows] floats over the
    // stages, free once everyone is past the loop; rows padded to 68 floats so a lane group's 16-byte accesses 68
    // floats apart spread over the banks); they store y = silu(gate) * (acc * scale2)
    constexpr int GXS = 68;
    __syncthreads();
    float *gx = (float *)smem;
    auto scaled = [&](const float *sc, int mi, int ni) {
      float4 v = make_float4(acc[mi][ni][0], acc[mi][ni][1], acc[mi][ni][2], acc[mi][ni][3]);
      const int rb = r0 + mi * 16 + 4 * lg;
      v.x = v.x * sc[min(rb, a.rows - 1)]; v.y = v.y * sc[min(rb + 1, a.rows - 1)];
      v.z = v.z * sc[min(rb + 2, a.rows - 1)]; v.w = v.w * sc[min(rb + 3, a.rows - 1)];
      return v;
    };
    if (wr == 0)
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) *(float4 *)(gx + (wc * 32 + ni * 16 + lr) * GXS + mi * 16 + 4 * lg) = scaled(a.scale, mi, ni);
    __syncthreads();
    if (wr == 1)
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) {
          const int t = t0 + wc * 32 + ni * 16 + lr;
          if (t >= a.ntok) continue;
          const float4 g = *(const float4 *)(gx + (wc * 32 + ni * 16 + lr) * GXS + mi * 16 + 4 * lg);
          const float4 u = scaled(a.scale2, mi, ni);
          const float h[4] = {silu_mul(g.x, u.x), silu_mul(g.y, u.y), silu_mul(g.z, u.z), silu_mul(g.w, u.w)};
          float *yt = a.y + (size_t)t * a.ldy;
          const int rb = r0 + mi * 16 + 4 * lg;
          if (rb + 3 < a.rows && (a.ldy & 3) == 0) *(float4 *)(yt + rb) = make_float4(h[0], h[1], h[2], h[3]);
          else
#pragma unroll
            for (int i = 0; i < 4; i++) if (rb + i < a.rows) yt[rb + i] = h[i];
        }
    return;
  }
  // y = acc * scale (+ bias), or y += (residual stream)
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
      const int t = t0 + wc * 32 + ni * 16 + lr;
      if (t >= a.ntok) continue;
      gemm_store4(a, a.y + (size_t)t * a.ldy, r0 + wr * 64 + mi * 16 + 4 * lg,
                  make_float4(acc[mi][ni][0], acc[mi][ni][1], acc[mi][ni][2], acc[mi][ni][3]), true);
    }
}

// ------------------------------------------------------------------ int8 MFMA matrix product (q8), 32 x 32 tiles
// Workgroup tile: 256 weight rows x 128 tokens, 8 waves (two per SIMD) in a 4 x 2 grid of 64 rows x 64 tokens, each a
// 2 x 2 grid of v_mfma_i32_32x32x32_i8 tiles.  Per 128-column block a tile's one int32 accumulator T takes the hi plane
// over the block's four 32-deep steps, then T = 256 T + 128 sum(W) (one shift-add), then the lo plane on top: T is the
// block's exact isum = 256 hi + lo + 128 sum(W), and acc = fma(bs, (float) T, acc) is rows_q8's fp32 step - the same
// arithmetic, bit for bit, as the 16 x 16 product and the decode matrix-vector product.
// K advances in 64-column stages through a 4-slot ring of direct global->LDS loads, two stages ahead.
//   stage: weights [256 rows][64 B], hi plane [128 tokens][64 B], lo plane likewise, the rows' block sums [256] and the
//   tokens' block scales [128] of the stage's block.  The four 16-byte segments of a 64-byte row are XOR-swizzled by
//   (row bit 2, row bit 1 ^ row bit 3), so the 32 rows of a fragment read spread over the 64 banks.
//   fragments: lane l reads A = W[row l % 32][16 (l / 32) + 0..15] and B = plane[token l % 32][16 (l / 32) + 0..15]
//   within the 32-deep step; C lane l holds rows 8 (r / 4) + 4 (l / 32) + r % 4 (r = 0..15) of token l % 32.
constexpr int kG2M = 256, kG2N = 128, kG2Slots = 2, kG2Waves = 8;
// stage = one 128-column block: the rows' block sums [256] and the tokens' block scales [128] first (small constant
// offsets for their reads), then weights [256 rows][128 B], hi plane [128 tokens][128 B], lo plane likewise
constexpr int kG2WS = 0, kG2BS = 1024, kG2W = 2048, kG2XH = kG2W + 256 * 128, kG2XL = kG2XH + 128 * 128;
constexpr int kG2Stage = kG2XL + 128 * 128;   // 67584 bytes (the block scales' second 512 bytes unused)
constexpr int kG2GX = 132;                    // gate hand-off row pitch (floats)
size_t gemm2_lds_bytes() { return (size_t)kG2Slots * kG2Stage; }
static_assert(kG2N * kG2GX * 4 + 2 * kG2N * 4 <= kG2Slots * kG2Stage, "gate hand-off and block maxima fit in the ring");
static_assert(kG2XL + 4096 + 16 < 65536, "fragment offsets fit the ds_read offset field");

// physical 16-byte segment of logical segment s in 128-byte row r: s ^ g2_swz(r).  The 8 rows of a 128-byte (32-bank)
// read phase and the 8 same-parity rows of a 256-byte (64-bank) phase all land on distinct segments.
__device__ __forceinline__ int g2_swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }

#define G2_WAIT(n, ...) asm volatile("s_waitcnt lgkmcnt(" #n ")" : __VA_ARGS__)

__global__ __launch_bounds__(512) void k_gemm2_q8(GemmArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 1, wc = wave & 1;   // rows 64 wr, tokens 64 wc of the tile
  const bool paired = a.w2 != nullptr;       // rows 0-127 of the tile from the gate matrix, 128-255 the same up rows
  const int RT = paired ? kG2M / 2 : kG2M;
  int r0, t0;
  {
    // XCD-aware tile order, as in the 16 x 16 product
    const int ntt = gridDim.x, nrt = gridDim.y, n = ntt * nrt, lin = blockIdx.y * gridDim.x + blockIdx.x;
    const int xcd = lin & 7, k = lin >> 3;
    if (ntt % 8 == 0) {
      const int tn = ntt >> 3;
      r0 = (k / tn) * RT; t0 = (xcd * tn + k % tn) * kG2N;
    } else {
      const int base = n >> 3, rem = n & 7;
      const int tile = xcd * base + min(xcd, rem) + k;
      r0 = (tile / ntt) * RT; t0 = (tile % ntt) * kG2N;
    }
  }
  r0 = gemm_segment(a, r0 + a.tile0 * RT, RT);
  const int nb = a.cols / kQB;

  // DMA sources: 64 1-KiB row groups per stage (32 of weights, 16 per plane; 8 rows of 128 B each), 8 to a wave; the
  // lane fetches the logical segment that belongs at physical segment lane % 8 of row lane / 8
  const int8_t *src[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int q = wave * 8 + j, row = 8 * (q & 31) + (lane >> 3), seg = (lane & 7) ^ g2_swz(row);
    if (q < 32) {
      const int8_t *wm = paired && row >= 128 ? a.w2 : a.w;
      src[j] = wm + (size_t)min(r0 + (paired ? (row & 127) : row), a.rows - 1) * a.cols + seg * 16;
    } else {
      const int tok = row & 127;
      src[j] = (q < 48 ? a.xh : a.xl) + (size_t)min(t0 + tok, a.ntok - 1) * a.ldq + seg * 16;
    }
  }
  // with each block: wave 0 the tile's 256 row sums (16 bytes = 4 rows a lane), wave 1 the 128 token scales (lanes
  // 32-63 repeat lanes 0-31 into the unused half), both from the block-major copies
  const int pitch = ws_pitch(a.rows);
  const char *esrc = nullptr;
  size_t estep = 0;
  if (wave == 0) {
    const int row = 4 * lane;
    const int *wsm = paired && row >= 128 ? a.wsum2 : a.wsum;
    esrc = (const char *)(wsm + min(r0 + (paired ? (row & 127) : row), pitch - 4));
    estep = 4 * (size_t)pitch;
  } else if (wave == 1) {
    esrc = (const char *)(a.xbt + min(t0 + 4 * (lane & 31), a.ldbt - 4));
    estep = 4 * (size_t)a.ldbt;
  }
  auto issue = [&](int b) {
    char *st = smem + (size_t)(b % kG2Slots) * kG2Stage;
#pragma unroll
    for (int j = 0; j < 8; j++) dma16(src[j] + kQB * b, st + kG2W + (wave * 8 + j) * 1024);
    if (wave < 2) dma16(esrc + b * estep, st + (wave ? kG2BS : kG2WS));
  };

  // per-lane LDS offsets of step ks: fragment row / token lane % 32, logical segment 2 ks + lane / 32, swizzled
  const int fr = lane & 31, fh = lane >> 5, fsw = g2_swz(fr);
  uint32_t ra[4], rb[4];
#pragma unroll
  for (int ks = 0; ks < 4; ks++) {
    const uint32_t o = fr * 128 + (((2 * ks + fh) ^ fsw) << 4);
    ra[ks] = kG2W + 64 * wr * 128 + o;   // + 4096 mi
    rb[ks] = 64 * wc * 128 + o;          // + plane + 4096 ni
  }
  const uint32_t rws = kG2WS + (64 * wr + 4 * fh) * 4;   // + 128 mi + 32 j
  const uint32_t rbs = kG2BS + (64 * wc + fr) * 4;       // + 128 ni
  const uint32_t sbase = lds_addr(smem);

  float acc[2][2][16];
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[mi][ni][r] = 0.f;
  const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  v16i T[2][2] = {{zero, zero}, {zero, zero}};
  v4i A0[4], A1[4], w0, w1, w2, w3, x0, x1, x2, x3;
  [[maybe_unused]] v4i f0a, f0b, f1a, f1b;   // the other schedules' fragment pairs
  [[maybe_unused]] v4i f2a, f2b;   // the staggered-halves schedule's third fragment pair
  [[maybe_unused]] v4i bq[4];   // the eighths / pairs schedules' token fragments (rolling)
  float nb0 = 0.f, nb1 = 0.f, pb1 = 0.f;   // token scales of this block / of the previous one
  [[maybe_unused]] float pb0 = 0.f;

  // one block per iteration: it has landed (every wave's loads: the barrier), every wave is done with the previous
  // block, whose slot now takes the next one
  issue(0);
  for (int b = 0; b < nb; b++) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (!(a.dbg & 4)) __builtin_amdgcn_s_barrier();
    if (b + 1 < nb && !(a.dbg & 2)) issue(b + 1);
    const uint32_t st = sbase + (uint32_t)((b % kG2Slots) * kG2Stage);
    if (a.dbg & 1) continue;
#include "gemm2_loop.inc"
    pb0 = nb0; pb1 = nb1;
  }
  // the last block's deferred fp32 steps (the loop runs them under the next block's first MFMAs)
#define G2_TAIL
#include "gemm2_loop.inc"
#undef G2_TAIL

  if (paired) {
    // the gate waves (rows 0-127) hand silu(gate), gate = acc * scale, to the up waves through LDS ([128 tokens][132
    // floats] over the ring, free once everyone is past the loop); the up waves form h = silu(gate) * (acc * scale2)
    // (silu_mul's operations, split between the two wave groups) and store it,
    // or (a.oh) quantise it: the tile's 128 rows are one 128-column block of each token's h, so the block max needs
    // only this workgroup (the two up waves of a token column meet in LDS)
    __syncthreads();
    float *gx = (float *)smem;
    float *red = gx + kG2N * kG2GX;   // [2 up waves][128 tokens] block maxima
    auto scaled = [&](const float *sc, int rb, const float *v) {
      float4 o;
      if (rb + 3 < a.rows) {
        const float4 s = *(const float4 *)(sc + rb);
        o = make_float4(v[0] * s.x, v[1] * s.y, v[2] * s.z, v[3] * s.w);
      } else {
        o = make_float4(v[0] * sc[min(rb, a.rows - 1)], v[1] * sc[min(rb + 1, a.rows - 1)], v[2] * sc[min(rb + 2, a.rows - 1)],
                        v[3] * sc[min(rb + 3, a.rows - 1)]);
      }
      return o;
    };
    if (wr < 2)
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int lrow = 64 * wr + 32 * mi + 8 * j + 4 * fh, tok = 64 * wc + 32 * ni + fr;
            const float4 g = scaled(a.scale, r0 + lrow, &acc[mi][ni][4 * j]);
            *(float4 *)(gx + tok * kG2GX + lrow) = make_float4(silu_f(g.x), silu_f(g.y), silu_f(g.z), silu_f(g.w));
          }
    __syncthreads();
    if (wr >= 2) {
      // h in place of the up accumulators
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
          for (int j = 0; j < 4; j++) {
            const int lrow = 64 * (wr - 2) + 32 * mi + 8 * j + 4 * fh, tok = 64 * wc + 32 * ni + fr;
            const float4 g = *(const float4 *)(gx + tok * kG2GX + lrow);
            const float4 u = scaled(a.scale2, r0 + lrow, &acc[mi][ni][4 * j]);
            acc[mi][ni][4 * j] = g.x * u.x; acc[mi][ni][4 * j + 1] = g.y * u.y;   // g = silu(gate), from the gate waves
            acc[mi][ni][4 * j + 2] = g.z * u.z; acc[mi][ni][4 * j + 3] = g.w * u.w;
          }
    }
    if (!a.oh) {
      if (wr >= 2)
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
          for (int ni = 0; ni < 2; ni++) {
            const int t = t0 + 64 * wc + 32 * ni + fr;
            if (t >= a.ntok) continue;
            float *yt = a.y + (size_t)t * a.ldy;
#pragma unroll
            for (int j = 0; j < 4; j++) {
              const int rb = r0 + 64 * (wr - 2) + 32 * mi + 8 * j + 4 * fh;
              const float *h = &acc[mi][ni][4 * j];
              if (rb + 3 < a.rows && (a.ldy & 3) == 0) *(float4 *)(yt + rb) = make_float4(h[0], h[1], h[2], h[3]);
              else
#pragma unroll
                for (int i = 0; i < 4; i++) if (rb + i < a.rows) yt[rb + i] = h[i];
            }
          }
      return;
    }
    // quantise (quant_rows, kernels.cpp:17-31, as k_pf_quant: mx = max |h| over the block, isx = mx > 0 ? 32767 / mx
    // : 0, bs = mx / 32767, q = rint(h * isx), planes hi = q >> 8, lo = (q & 255) ^ 0x80)
    if (wr >= 2)
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
        float m = 0.f;
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
          for (int r = 0; r < 16; r++) m = fmaxf(m, fabsf(acc[mi][ni][r]));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        if (fh == 0) red[(wr - 2) * kG2N + 64 * wc + 32 * ni + fr] = m;
      }
    __syncthreads();
    if (wr < 2) return;
    const int blk = r0 / kQB;
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
      const int tok = 64 * wc + 32 * ni + fr, t = t0 + tok;
      if (t >= a.ntok) continue;
      const float m = fmaxf(red[tok], red[kG2N + tok]);
      const float isx = m > 0 ? kActMax / m : 0.f;
      if (wr == 2 && fh == 0) {
        const float bs = m / kActMax;
        a.ob[(size_t)t * a.ldb + blk] = bs;
        a.obt[(size_t)blk * a.ldbt + t] = bs;
      }
      int8_t *oh = a.oh + (size_t)t * a.ldq, *ol = a.ol + (size_t)t * a.ldq;
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int rb = r0 + 64 * (wr - 2) + 32 * mi + 8 * j + 4 * fh;
          uint32_t hh = 0, ll = 0;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int q = (int)__builtin_rintf(acc[mi][ni][4 * j + i] * isx);
            hh |= (uint32_t)((q >> 8) & 0xff) << (8 * i);
            ll |= (uint32_t)((q & 0xff) ^ 0x80) << (8 * i);
          }
          *(uint32_t *)(oh + rb) = hh;
          *(uint32_t *)(ol + rb) = ll;
        }
    }
    return;
  }
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
      const int t = t0 + 64 * wc + 32 * ni + fr;
      if (t >= a.ntok) continue;
#pragma unroll
      for (int j = 0; j < 4; j++)
        gemm_store4(a, a.y + (size_t)t * a.ldy, r0 + 64 * wr + 32 * mi + 8 * j + 4 * fh,
                    make_float4(acc[mi][ni][4 * j], acc[mi][ni][4 * j + 1], acc[mi][ni][4 * j + 2], acc[mi][ni][4 * j + 3]), true);
    }
}

// ------------------------------------------------------------------ int8 MFMA matrix product (q4 weights)
// The q8 product's tile, waves, stages and DMA ring, for q4 rows (byte j of a 32-column group holds column j in the low
// nibble and column j + 16 in the high one; an fp16 scale per row and group).  Each group gets its exact int32 sum on
// v_mfma_i32_16x16x32_i8 (one 32-deep step per plane): lane l's 8 A bytes are the low (l / 16 < 2) or high nibbles of
// packed bytes 8 (l / 16 & 1) + 0..7 - unsigned 0..15 - against the planes' columns 8 (l / 16) + 0..7, and
//     isum_g = 256 (nib . hi) + (nib . lo) + 128 sum(nib) - 8 sum(q)       (w = nib - 8, q = 256 hi + lo + 128)
// with sum(nib) per (row, group) precomputed (k_q4_prep, together with the f32 scales, group-major) and sum(q) per
// (token, group) from the quantiser.  Float step: blk = sum_g fma(scale_g, (float)isum_g), acc = fma(bs, blk, acc) per
// block - another order than rows_q4's 8-lane partials, within the logit tolerance like the decode q4 path.
//   stage: packed weights [128][64 B] (segments swizzled ^ (row & 3)), hi / lo planes as in the q8 product, block
//   scales [128 tokens], sum(q) [128 tokens][4], sum(nib) [4][128 rows], weight scales [4][128 rows] f32.
constexpr int kG4Stage = 128 * 64 + 2 * 128 * 128 + 512 + 2048 + 2048 + 2048;

// per (block, group, row): sum of the row's nibbles over the group and its fp16 scale as f32, group-major within a
// block: out_ns[(b * 4 + g) * rows + r], out_sc likewise
__global__ __launch_bounds__(256) void k_q4_prep(const uint8_t *w, const uint16_t *sc, int rows, int cols, int *out_ns,
                                                 float *out_sc) {
  const int G = cols / 32;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)rows * G) return;
  const int r = (int)(i / G), g = (int)(i % G);
  const v4i v = *(const v4i *)(w + (size_t)r * (cols / 2) + 16 * g);
  int s = 0;
  const int words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    s = __builtin_amdgcn_sdot4(words[k] & 0x0f0f0f0f, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4((words[k] >> 4) & 0x0f0f0f0f, 0x01010101, s, false);
  }
  const size_t o = ((size_t)(g >> 2) * 4 + (g & 3)) * rows + r;
  out_ns[o] = s;
  out_sc[o] = half_bits_to_float(sc[(size_t)r * G + g]);
}
hipError_t launch_q4_prep(const uint8_t *w, const uint16_t *sc, int rows, int cols, int *out_ns, float *out_sc,
                          hipStream_t st) {
  if (cols % kQB || rows <= 0) return hipErrorInvalidValue;
  const int64_t n = (int64_t)rows * (cols / 32);
  hipLaunchKernelGGL(k_q4_prep, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, sc, rows, cols, out_ns, out_sc);
  return hipGetLastError();
}

__device__ __forceinline__ uint2 lds_read8(uint32_t addr) {
  uint2 r;
  asm volatile("ds_read_b64 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

__global__ __launch_bounds__(512) void k_gemm_q4(GemmArgs a) {
  extern __shared__ __align__(16) char smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 2, wc = wave & 3, lr = lane & 15, lg = lane >> 4;
  int r0, t0;
  {
    const int ntt = gridDim.x, n = gridDim.x * gridDim.y, lin = blockIdx.y * gridDim.x + blockIdx.x;
    const int xcd = lin & 7, k = lin >> 3;
    if (ntt % 8 == 0) {
      const int tn = ntt >> 3;
      r0 = (k / tn) * kGM; t0 = (xcd * tn + k % tn) * kGN;
    } else {
      const int base = n >> 3, rem = n & 7;
      const int tile = xcd * base + min(xcd, rem) + k;
      r0 = (tile / ntt) * kGM; t0 = (tile % ntt) * kGN;
    }
  }
  r0 = gemm_segment(a, r0 + a.tile0 * kGM, kGM);
  const int nb = a.cols / kQB, rb = a.cols / 2;   // packed bytes per row
  // DMA jobs per stage (64 wave instructions, 8 per wave; jobs 60..63 repeat 0..3 byte for byte):
  //   0..7 packed weights (16 rows x 64 B each), 8..23 hi plane, 24..39 lo plane (8 rows x 128 B each),
  //   40..47 sum(nib) and 48..55 scales (64 rows of one group each, 4 B per lane), 56..57 sum(q) (64 tokens x 16 B),
  //   58..59 block scales (64 tokens x 4 B)
  const char *src[8];
  int dst[8], bytes[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    int q = wave * 8 + j;
    if (q >= 60) q -= 60;
    if (q < 8) {
      const int row = 16 * q + (lane >> 2), seg = (lane & 3) ^ (row & 3);
      src[j] = (const char *)a.w + (size_t)min(r0 + row, a.rows - 1) * rb + seg * 16;
      dst[j] = 16 * q * 64; bytes[j] = 16;
    } else if (q < 40) {
      const int m = q < 24 ? 0 : 1, qq = (q - 8) & 15, row = 8 * qq + (lane >> 3), seg = (lane & 7) ^ (lane >> 3);
      src[j] = (const char *)(m == 0 ? a.xh : a.xl) + (size_t)min(t0 + row, a.ntok - 1) * a.ldq + seg * 16;
      dst[j] = 128 * 64 + m * 128 * 128 + 8 * qq * 128; bytes[j] = 16;
    } else if (q < 56) {
      const int which = q < 48 ? 0 : 1, qq = (q - 40) & 7, g = qq >> 1, row = 64 * (qq & 1) + lane;
      // group-major per block: element (kb * 4 + g) * rows + row; the block offset is added at issue time
      const char *base = which == 0 ? (const char *)a.q4ns : (const char *)a.q4sc;
      src[j] = base + 4 * ((size_t)g * a.rows + min(r0 + row, a.rows - 1));
      dst[j] = 128 * 64 + 2 * 128 * 128 + 512 + 2048 + which * 2048 + g * 512 + (qq & 1) * 256; bytes[j] = 4;
    } else if (q < 58) {
      const int tok = 64 * (q - 56) + lane;
      src[j] = (const char *)(a.xg + (size_t)min(t0 + tok, a.ntok - 1) * a.ldg);
      dst[j] = 128 * 64 + 2 * 128 * 128 + 512 + 64 * 16 * (q - 56); bytes[j] = 16;
    } else {
      const int tok = 64 * (q - 58) + lane;
      src[j] = (const char *)(a.xb + (size_t)min(t0 + tok, a.ntok - 1) * a.ldb);
      dst[j] = 128 * 64 + 2 * 128 * 128 + 256 * (q - 58); bytes[j] = 4;
    }
  }
  auto issue = [&](int kb) {
    char *st = smem + (size_t)(kb % kGStages) * kG4Stage;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      int q = wave * 8 + j;
      if (q >= 60) q -= 60;
      size_t adv;
      if (q < 8) adv = (size_t)kb * 64;                                     // packed row bytes of the block
      else if (q < 40) adv = (size_t)kb * kQB;                              // plane bytes of the block
      else if (q < 56) adv = (size_t)kb * 4 * a.rows * 4;                   // group-major block of 4 x rows
      else if (q < 58) adv = (size_t)kb * 16;                               // 4 groups of sum(q)
      else adv = (size_t)kb * 4;                                            // one block scale
      if (bytes[j] == 16) dma16(src[j] + adv, st + dst[j]);
      else dma4(src[j] + adv, st + dst[j]);
    }
  };

  float acc[4][2][4];
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[mi][ni][i] = 0.f;

  issue(0);
  if (nb > 1) issue(1);
  for (int kb = 0; kb < nb; kb++) {
    if (kb + 1 < nb) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (kb + 2 < nb) issue(kb + 2);
    const uint32_t st = lds_addr(smem + (size_t)(kb % kGStages) * kG4Stage);
    const uint32_t sw = st, sh = st + 128 * 64, sl = sh + 128 * 128, sbs = sl + 128 * 128, sgq = sbs + 512,
                   sns = sgq + 2048, ssc = sns + 2048;
    // per-lane block data: the tokens' block scales and sum(q) of the 4 groups
    float bsc[2]; v4i gq[2];
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
      const int tok = wc * 32 + ni * 16 + lr;
      bsc[ni] = lds_read4(sbs + 4 * tok);
      gq[ni] = lds_read16(sgq + 16 * tok);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(bsc[0]), "+v"(bsc[1]), "+v"(gq[0]), "+v"(gq[1]));
    float blk[4][2][4];
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int i = 0; i < 4; i++) blk[mi][ni][i] = 0.f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      long A[4], BH[2], BL[2];
      v4i ns[4], scv[4];
#pragma unroll
      for (int mi = 0; mi < 4; mi++) {
        const int row = wr * 64 + mi * 16 + lr;
        const uint2 v = lds_read8(sw + row * 64 + ((g ^ (row & 3)) << 4) + 8 * (lg & 1));
        A[mi] = (long)v.x | ((long)v.y << 32);   // raw bytes; nibbles extracted after the wait
        const int r4 = wr * 64 + mi * 16 + 4 * lg;
        ns[mi] = lds_read16(sns + 4 * (g * 128 + r4));
        scv[mi] = lds_read16(ssc + 4 * (g * 128 + r4));
      }
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
        const int tok = wc * 32 + ni * 16 + lr;
        const uint32_t o = tok * 128 + (((2 * g + (lg >> 1)) ^ (tok & 7)) << 4) + 8 * (lg & 1);
        const uint2 h = lds_read8(sh + o), l = lds_read8(sl + o);
        BH[ni] = (long)h.x | ((long)h.y << 32);
        BL[ni] = (long)l.x | ((long)l.y << 32);
      }
      asm volatile("s_waitcnt lgkmcnt(0)"
                   : "+v"(A[0]), "+v"(A[1]), "+v"(A[2]), "+v"(A[3]), "+v"(BH[0]), "+v"(BH[1]), "+v"(BL[0]), "+v"(BL[1]),
                     "+v"(ns[0]), "+v"(ns[1]), "+v"(ns[2]), "+v"(ns[3]), "+v"(scv[0]), "+v"(scv[1]), "+v"(scv[2]),
                     "+v"(scv[3]));
#pragma unroll
      for (int mi = 0; mi < 4; mi++) {   // low nibbles for k 0..15 of the group, high nibbles for 16..31
        const uint32_t lo = (uint32_t)A[mi], hi = (uint32_t)((unsigned long)A[mi] >> 32);
        const uint32_t x0 = lg < 2 ? lo & 0x0f0f0f0fu : (lo >> 4) & 0x0f0f0f0fu;
        const uint32_t x1 = lg < 2 ? hi & 0x0f0f0f0fu : (hi >> 4) & 0x0f0f0f0fu;
        A[mi] = (long)x0 | ((long)x1 << 32);
      }
#pragma unroll
      for (int mi = 0; mi < 4; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) {
          v4i ch = {0, 0, 0, 0};
          v4i cl = ns[mi] * 128 - gq[ni][g] * 8;
          ch = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[mi], BH[ni], ch, 0, 0, 0);
          cl = __builtin_amdgcn_mfma_i32_16x16x32_i8(A[mi], BL[ni], cl, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int isum = ch[i] * 256 + cl[i];
            const int sbits = scv[mi][i];   // copied out first: this compiler lowers a bit_cast of a vector-element
                                            // lvalue to a read of element 0
            blk[mi][ni][i] = __builtin_fmaf(__builtin_bit_cast(float, sbits), (float)isum, blk[mi][ni][i]);
          }
        }
    }
#pragma unroll
    for (int mi = 0; mi < 4; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[mi][ni][i] = __builtin_fmaf(bsc[ni], blk[mi][ni][i], acc[mi][ni][i]);
  }
#pragma unroll
  for (int mi = 0; mi < 4; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
      const int t = t0 + wc * 32 + ni * 16 + lr;
      if (t >= a.ntok) continue;
      gemm_store4(a, a.y + (size_t)t * a.ldy, r0 + wr * 64 + mi * 16 + 4 * lg,
                  make_float4(acc[mi][ni][0], acc[mi][ni][1], acc[mi][ni][2], acc[mi][ni][3]), false);
    }
}

// q8: which product kernel.  A 32 x 32 workgroup does twice a 16 x 16 one's work in ~1.45 x its time (C4 shapes on
// MI355X: 2 x 14336 x 4096 578 vs 707 us, 4096 x 4096 173 vs 215, 6144 x 4096 152 vs 160), so it wins unless its fewer,
// larger workgroups leave CUs idle: ceil(n2 / CUs) x 1.45 against ceil(2 n2 / CUs) rounds (n2 = its workgroup count).
// QPH_GEMM=1 / 2 forces the 32 x 32 / 16 x 16 kernel.
static int gemm_forced() {   // QPH_GEMM, read per launch: tests switch it between calls
  const char *fe = getenv("QPH_GEMM");
  const int f = fe ? atoi(fe) : 0;
  return f == 1 || f == 2 ? f : 0;
}
static int gemm_cus() {
  if (const char *e = getenv("QPH_GEMM_CUS")) return std::max(1, atoi(e));   // test hook: the choice for another CU count
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 256;
    return std::max(1, n);
  }();
  return cus;
}
static double gemm_rounds(long wgs) { return (double)((wgs + gemm_cus() - 1) / gemm_cus()); }
constexpr double kG2Cost = 1.45;   // a 32 x 32 round in 16 x 16 rounds
static bool gemm_use_32x32(int row_tiles32, int token_tiles32) {
  if (const int f = gemm_forced()) return f == 1;
  const long n2 = (long)row_tiles32 * token_tiles32;
  return gemm_rounds(n2) * kG2Cost < gemm_rounds(2 * n2);
}

// row tiles of a launch for a tile height (a gate / up pair: half-height tiles of each matrix)
static int gemm_row_tiles(const GemmArgs &a, bool big) {
  const int rt = big ? (a.w2 ? kG2M / 2 : kG2M) : (a.w2 ? kGM / 2 : kGM);
  if (a.nseg < 2) return (a.rows + rt - 1) / rt;
  int t = 0;
  for (int s = 0; s < a.nseg && s < kGemmMaxSeg; s++) t += (a.seg[s].rows + rt - 1) / rt;
  return t;
}
bool gemm_uses_32x32(const GemmArgs &a) {
  return a.kind == MK_Q8 && a.xbt && a.ntok > 0 && gemm_use_32x32(gemm_row_tiles(a, true), (a.ntok + kG2N - 1) / kG2N);
}

hipError_t launch_gemm(const GemmArgs &a0, hipStream_t st) {
  if (a0.ntok <= 0) return hipSuccess;
  GemmArgs a = a0;
  { static const int dbg = [] { const char *e = getenv("QPH_G2_DBG"); return e ? atoi(e) : 0; }(); a.dbg = dbg; }
  if (a0.tile0) return hipErrorInvalidValue;   // set only here
  const bool big = gemm_uses_32x32(a0);
  const int tiles = gemm_row_tiles(a0, big);
  if (a.oh && (!big || !a.w2 || a.rows % kQB || !a.ol || !a.ob || !a.obt || a.ldbt % 4 || a.ldbt < a.ntok))
    return hipErrorInvalidValue;   // quantised output: the 32 x 32 kernel's gate / up pair, whole 128-row blocks
  if (a.nseg > 1) {
    // the first matrix also stands in the launch's own fields, so the checks below cover every segment's pointers
    if (a.nseg > kGemmMaxSeg || a.w2 || a.resid || a.gate) return hipErrorInvalidValue;
    for (int s = 0; s < a.nseg; s++) {
      const GemmSeg &g = a.seg[s];
      if (g.rows <= 0 || !g.w || !g.scale || !g.y || (a.kind == MK_Q8 ? !g.wsum : (!g.q4ns || !g.q4sc))) return hipErrorInvalidValue;
    }
    const GemmSeg &g = a.seg[0];
    a.w = g.w; a.scale = g.scale; a.wsum = g.wsum; a.q4ns = g.q4ns; a.q4sc = g.q4sc; a.bias = g.bias; a.y = g.y;
    a.rows = g.rows; a.ldy = g.ldy;
  } else {
    a.nseg = 0;
  }
  if (a.cols % kQB || a.rows <= 0 || a.ldq % 16 || a.ldq < a.cols || a.ldb < a.cols / kQB) return hipErrorInvalidValue;
  const dim3 grid((a.ntok + (big ? kG2N : kGN) - 1) / (big ? kG2N : kGN), tiles);
  if (a.w2 && (a.kind != MK_Q8 || !a.scale2 || !a.wsum2 || a.resid || a.bias || a.gate)) return hipErrorInvalidValue;
  if (a.kind == MK_Q8) {
    if (!a.wsum) return hipErrorInvalidValue;
    if (big && (!a.xbt || a.ldbt % 4 || a.ldbt < a.ntok)) return hipErrorInvalidValue;
    // a segment launch whose 32 x 32 grid would end in a part-filled round: its first segments on the 32 x 32 kernel,
    // the rest on the 16 x 16 one, when that takes fewer rounds (C4 q / k / v: q alone fills one 32 x 32 round, k + v
    // one 16 x 16 round)
    int split = 0, t32 = 0, t16 = 0, t16_0 = 0;
    if (big && a.nseg > 1 && a.tile0 == 0 && !gemm_forced()) {
      const int tt = grid.x;
      double best = gemm_rounds((long)tiles * tt) * kG2Cost;
      for (int s = 1; s < a.nseg; s++) {
        int f32 = 0, f16 = 0, r16 = 0;
        for (int i = 0; i < a.nseg; i++) {
          if (i < s) { f32 += (a.seg[i].rows + kG2M - 1) / kG2M; f16 += (a.seg[i].rows + kGM - 1) / kGM; }
          else r16 += (a.seg[i].rows + kGM - 1) / kGM;
        }
        const double c = gemm_rounds((long)f32 * tt) * kG2Cost + gemm_rounds((long)r16 * tt);
        if (c < best) { best = c; split = s; t32 = f32; t16 = r16; t16_0 = f16; }
      }
    }
    if (split) {
      hipLaunchKernelGGL(k_gemm2_q8, dim3(grid.x, t32), dim3(64 * kG2Waves), gemm2_lds_bytes(), st, a);
      GemmArgs b = a;
      b.tile0 = t16_0;
      hipLaunchKernelGGL(k_gemm_q8, dim3(grid.x, t16), dim3(64 * kGWaves), gemm_lds_bytes(), st, b);
    } else if (big) {
      hipLaunchKernelGGL(k_gemm2_q8, grid, dim3(64 * kG2Waves), gemm2_lds_bytes(), st, a);
    } else {
      hipLaunchKernelGGL(k_gemm_q8, grid, dim3(64 * kGWaves), gemm_lds_bytes(), st, a);
    }
  } else if (a.kind == MK_Q4) {
    if (!a.q4ns || !a.q4sc || !a.xg || a.ldg < a.cols / 32 || a.ldg % 4) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_gemm_q4, grid, dim3(64 * kGWaves), (size_t)kGStages * kG4Stage, st, a);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ RoPE and the fp16 cache rows of a token batch
// token t sits at position p0 + t: q heads and k groups rotate (rotate-half with the reference's contraction,
// model_llama.cpp:86-90), k and v go to the layer's caches as fp16 (to_f16, kernels_x86.cpp:449-452)
__global__ __launch_bounds__(256) void k_pf_rope(PfRopeArgs a) {
  const int t = blockIdx.x, pos = a.p0 + t, half = a.hd / 2, kvd = a.nkv * a.hd;
  const float *cs = a.cos_t + (size_t)pos * half, *sn = a.sin_t + (size_t)pos * half;
  float *q = a.q + (size_t)t * a.ldq;
  for (int e = threadIdx.x; e < (a.skip_q ? 0 : a.nh * half); e += blockDim.x) {
    const int h = e / half, i = e % half;
    float *qh = q + h * a.hd; const float x0 = qh[i], x1 = qh[i + half];
    qh[i] = __builtin_fmaf(x0, cs[i], -(x1 * sn[i]));
    qh[i + half] = __builtin_fmaf(x1, cs[i], x0 * sn[i]);
  }
  const float *k = a.k + (size_t)t * a.ldk, *v = a.v + (size_t)t * a.ldk;
  uint16_t *kr = a.kc + (size_t)pos * kvd, *vr = a.vc + (size_t)pos * kvd;
  for (int e = threadIdx.x; e < a.nkv * half; e += blockDim.x) {
    const int g = e / half, i = e % half;
    const float x0 = k[g * a.hd + i], x1 = k[g * a.hd + i + half];
    kr[g * a.hd + i] = f32_to_half_bits(__builtin_fmaf(x0, cs[i], -(x1 * sn[i])));
    kr[g * a.hd + i + half] = f32_to_half_bits(__builtin_fmaf(x1, cs[i], x0 * sn[i]));
  }
  for (int e = threadIdx.x; e < kvd; e += blockDim.x) vr[e] = float_to_half_bits(v[e]);
}
hipError_t launch_pf_rope(const PfRopeArgs &a, int B, hipStream_t st) {
  if (B <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_pf_rope, dim3(B), dim3(256), 0, st, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ causal attention of a token batch (f16 MFMA)
// Token t (position P = p0 + t) attends to cache positions [0, P] - the prompt path of model_llama.cpp:95-105.
// A wave owns one unit = (16-token tile, query head); a workgroup's 8 waves share the kv group and stream its cache in
// 32-position blocks through LDS (K as stored, V transposed), with an online softmax per token:
//   scores  S^T[p][t] = K[p] . q[t] on v_mfma_f32_16x16x32_f16: A = K rows (exact fp16), B = q^T; q is fp32, so it
//           enters as hi + lo halves (hi = f16(q), lo = f16(q - hi)) - two MFMAs, products exact, fp32 accumulation;
//           q is pre-scaled by log2(e) / sqrt(hd) (the reference's 1 / sqrt(hd), in base-2 units);
//   values  O^T[d][t] += V^T[d][p] P^T[p][t], P split into hi + lo halves the same way; the C layout of S^T
//           (lane l: token l % 16, positions 4 (l / 16) + i of each 16-block) is the B layout the value MFMA needs once
//           its k index runs over those 8 positions, so P never leaves the registers;
//   softmax each lane keeps its token's running max and sum (reduced over the 4 lanes holding that token); the
//           exponentials are the hardware exp2 (v_exp_f32, ~1 ulp) instead of the reference's exp256 polynomial
//           (kernels_x86.cpp:406-417): a float-order difference within the logit tolerance, like the rest of this
//           kernel's order (the reference-order mode has its own kernel, k_ex_pf_attn).
constexpr int kPfKB = 64;      // cache positions per block (two 32-deep value steps)
constexpr int kPfAttnWaves = 8;   // units (16-token tile, query head) per workgroup, one per wave: they share the K / V
template <int HD>
__global__ __launch_bounds__(kPfAttnWaves * 64) void k_pf_attn(PfAttnArgs a) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  // KS: K rows of HD / 2 + 8 dwords. A b128 LDS read serves 16 lanes a cycle from 64 banks, the 16 being four 4-lane
  // groups of one 32-lane half with lane bit 4 = bit 2 ^ bit 3 (or its complement; measured with bank-conflict counters
  // on gfx950); the K fragment reads below (lanes: row lr, quad lg) then cover 16 distinct bank quads per cycle, where
  // the HD / 2 + 4 stride put rows lr and lr + 1 one quad apart and collided (3.5 conflict cycles per read).
  // VS: transposed V rows of 36 dwords (see the V stores)
  constexpr int KS = HD + 16, VS = kPfKB + 8, DT = HD / 16;
  constexpr int NH = kPfKB / 32, NM = kPfKB / 16;              // 32-position value steps, 16-position score tiles
  constexpr int NT = kPfAttnWaves * 64;
  constexpr int NPC = kPfKB * (HD / 8);                        // 16-byte pieces of K (and of V) per block
  constexpr int NP = (NPC + NT - 1) / NT;                      // ... per thread
  static_assert(NPC % NT == 0, "every thread holds NP whole pieces (the shuffles below see whole waves)");
  __shared__ __align__(16) uint16_t ks[kPfKB * KS];
  __shared__ __align__(16) uint16_t vt[HD * VS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 15, lg = lane >> 4;
  // longest first over all kv groups: workgroup L (in dispatch order) takes the (L / ngroups)-th last token tiles of
  // group L % ngroups, so the first workgroups on the CUs are the ones that stream the most of the cache and the short
  // ones fill in behind them (causal work grows with the tile index)
  const int L = blockIdx.y * gridDim.x + blockIdx.x;
  const int bx = gridDim.x - 1 - L / gridDim.y, g = L % gridDim.y;
  const int rep = a.nh / a.nkv, kvd = a.nkv * HD;
  const int ntiles = (a.ntok + 15) / 16, nunits = ntiles * rep;
  const int u = bx * kPfAttnWaves + wave;
  const bool live = u < nunits;
  const int tile = live ? u / rep : 0, head = g * rep + (live ? u % rep : 0);
  const int t = tile * 16 + lr;                        // this lane's token
  const bool tok_ok = live && t < a.ntok;
  const int ptok = a.p0 + t;                           // its position: attends to [0, ptok]
  const int wave_last = live ? a.p0 + min(tile * 16 + 15, a.ntok - 1) : -1;
  // the workgroup streams up to its last live unit's last token
  const int ulast = min(bx * kPfAttnWaves + kPfAttnWaves - 1, nunits - 1);
  const int wg_last = a.p0 + min((ulast / rep) * 16 + 15, a.ntok - 1);
  const int nkb = wg_last / kPfKB + 1;

  // q^T fragments: lane holds q[t][32 s + 8 lg + 0..7] as hi / lo halves, pre-scaled by log2(e) / sqrt(hd) so the
  // scores come out in base-2 units for the hardware exp2 (v_exp_f32)
  const float qscale = 1.4426950408889634f / sqrtf((float)HD);
  h8 qh[HD / 32], ql[HD / 32];
  {
    const float *qt = a.q + (size_t)(tok_ok ? t : 0) * a.ldq + head * HD;
    float qv[HD / 32][8];
#pragma unroll
    for (int s = 0; s < HD / 32; s++)
#pragma unroll
      for (int j = 0; j < 8; j++) qv[s][j] = tok_ok ? qt[32 * s + 8 * lg + j] : 0.f;
    if (a.cos_t) {
      // RoPE here (k_pf_rope's arithmetic): dims d and d + hd / 2 of a rotate-half pair sit in this lane's steps s and
      // s + hd / 64
      const int pos = tok_ok ? ptok : 0;   // tokens past the batch: any row of the table (their q is 0)
      const float *cs = a.cos_t + (size_t)pos * (HD / 2), *sn = a.sin_t + (size_t)pos * (HD / 2);
#pragma unroll
      for (int s = 0; s < HD / 64; s++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int i = 32 * s + 8 * lg + j;
          const float x0 = qv[s][j], x1 = qv[s + HD / 64][j], c = cs[i], si = sn[i];
          qv[s][j] = __builtin_fmaf(x0, c, -(x1 * si));
          qv[s + HD / 64][j] = __builtin_fmaf(x1, c, x0 * si);
        }
    }
#pragma unroll
    for (int s = 0; s < HD / 32; s++) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float x = qv[s][j] * qscale;
        const _Float16 h = (_Float16)x;
        qh[s][j] = h; ql[s][j] = (_Float16)(x - (float)h);
      }
    }
  }
  f4 o[DT];
#pragma unroll
  for (int d = 0; d < DT; d++) o[d] = (f4){0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  const uint16_t *kg = a.kc + g * HD, *vg = a.vc + g * HD;

  // piece c = tid + NT i of a block: a wave holds 8 positions x 8 dim octets (each position's 128 bytes in 8 adjacent
  // lanes, one cache line), HD / 64 waves side by side cover a position's dims; the next block's pieces are loaded
  // while the current one is computed (named registers, not an array: a two-entry array indexed in the rolled-up loop
  // ended in scratch)
  static_assert(NP == 1 || NP == 2, "one or two pieces per thread");
  constexpr int WPO = HD / 64;   // waves per 8-position group
  auto piece_pos = [&](int c) { return ((c >> 6) / WPO) * 8 + ((c & 63) >> 3); };
  auto piece_dim = [&](int c) { return (((c >> 6) % WPO) * 8 + (c & 7)) * 8; };
  uint4 kr0, vr0, kr1, vr1;
  auto load_piece = [&](int pb, int i, uint4 &k, uint4 &v) {
    const int c = tid + NT * i, pos = pb + piece_pos(c), d0 = piece_dim(c);
    const int pc = pos <= wg_last ? pos : wg_last;   // rows past the last one re-read it (masked out)
    k = *(const uint4 *)(kg + (size_t)pc * kvd + d0);
    v = *(const uint4 *)(vg + (size_t)pc * kvd + d0);
  };
  auto load_block = [&](int pb) {
    load_piece(pb, 0, kr0, vr0);
    if (NP == 2) load_piece(pb, 1, kr1, vr1);
  };
  // K as stored; V transposed: the lane 8 away holds position p ^ 1 with the same dims, the two swap halves so the
  // even-position lane owns dims d0 .. d0 + 3 and the odd one d0 + 4 .. d0 + 7 of both positions, and each writes
  // four (p even, p odd) pairs as 32-bit words
  auto store_piece = [&](int i, const uint4 &k, const uint4 &vrr) {
    const int c = tid + NT * i, p = piece_pos(c), d0 = piece_dim(c);
    *(uint4 *)(ks + p * KS + d0) = k;
    const uint32_t vv[4] = {vrr.x, vrr.y, vrr.z, vrr.w};
    const bool ev = (p & 1) == 0;
    const uint32_t rx = xchg8_u32(ev ? vv[2] : vv[0]);
    const uint32_t ry = xchg8_u32(ev ? vv[3] : vv[1]);
    const uint32_t ox = ev ? vv[0] : vv[2], oy = ev ? vv[1] : vv[3];
    const uint32_t lo_x = ev ? ox : rx, hi_x = ev ? rx : ox, lo_y = ev ? oy : ry, hi_y = ev ? ry : oy;
    // dword (p / 2) of the row, XOR 2 (row / 8 mod 8) (even, so the pairs the reads take stay adjacent; a lane's rows
    // d0 .. d0 + 7 share it). gfx950 serves b32 LDS accesses 32 lanes a cycle from 32 banks and b64 ones 32 lanes a
    // cycle from 64 banks (measured): with 36-dword rows, 8 positions x 8 octets per wave and this swizzle both these
    // stores and the V^T fragment reads below are conflict-free; 4 positions x 16 octets per wave put a 32-lane
    // phase's stores on 16 banks (every lane the same dword column, every address even)
    const int sw = 2 * ((d0 >> 3) & 7);
    uint32_t *w = (uint32_t *)(vt + (d0 + (ev ? 0 : 4)) * VS) + ((p >> 1) ^ sw);
    w[0] = (lo_x & 0xffffu) | (hi_x << 16);
    w[VS / 2] = (lo_x >> 16) | (hi_x & 0xffff0000u);
    w[VS] = (lo_y & 0xffffu) | (hi_y << 16);
    w[3 * VS / 2] = (lo_y >> 16) | (hi_y & 0xffff0000u);
  };
  load_block(0);
  for (int kb = 0; kb < nkb; kb++) {
    const int pb = kb * kPfKB;
    __syncthreads();   // the previous block's LDS reads are done
    store_piece(0, kr0, vr0);
    if (NP == 2) store_piece(1, kr1, vr1);
    __syncthreads();
    if (kb + 1 < nkb) load_block(pb + kPfKB);
    if (!live || pb > wave_last) continue;
    // scores of the block's 16-position tiles
    f4 sc[NM];
#pragma unroll
    for (int mt = 0; mt < NM; mt++) {
      sc[mt] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < HD / 32; s++) {
        const h8 kf = *(const h8 *)(ks + (mt * 16 + lr) * KS + 32 * s + 8 * lg);
        sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[s], sc[mt], 0, 0, 0);
        sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[s], sc[mt], 0, 0, 0);
      }
    }
    // online softmax for token t over positions pb + 16 mt + 4 lg + i
    float sv[4 * NM], bm = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < NM; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int p = pb + 16 * mt + 4 * lg + i;
        const float x = (tok_ok && p <= ptok) ? sc[mt][i] : -INFINITY;
        sv[4 * mt + i] = x; bm = fmaxf(bm, x);
      }
    bm = pair_max16(bm);
    bm = pair_max32(bm);
    const float mn = fmaxf(m, bm);
    // exp2 of -inf is 0: masked scores need no select; a token with no valid position yet (only tokens past the
    // batch, never stored) keeps mn = -inf, replaced by 0 so no -inf - -inf appears
    const float mz = mn == -INFINITY ? 0.f : mn;
    const float corr = __builtin_amdgcn_exp2f(m - mz);
    float rs = 0.f;
    h8 ph[NH], pl[NH];   // value step hs: positions 32 hs + 4 lg + 0..3 and 32 hs + 16 + 4 lg + 0..3
#pragma unroll
    for (int j = 0; j < 4 * NM; j++) {
      const float pv = __builtin_amdgcn_exp2f(sv[j] - mz);
      rs += pv;
      const _Float16 h = (_Float16)pv;
      ph[j / 8][j % 8] = h; pl[j / 8][j % 8] = (_Float16)(pv - (float)h);
    }
    rs = pair_sum16(rs);
    rs = pair_sum32(rs);
    l = l * corr + rs;
    m = mn;
#pragma unroll
    for (int d = 0; d < DT; d++) {
      o[d] *= corr;
      // V^T fragment of step hs: dim 16 d + lr, positions 32 hs + 4 lg + 0..3 and 32 hs + 16 + 4 lg + 0..3 (the k order
      // of ph / pl); the writes' swizzle XORs the low four bits of the dword index only
      const int row = 16 * d + lr, sw = 2 * ((row >> 3) & 7);
      const uint32_t *vr = (const uint32_t *)(vt + row * VS);
#pragma unroll
      for (int hs = 0; hs < NH; hs++) {
        const uint2 v0 = *(const uint2 *)(vr + 16 * hs + ((2 * lg) ^ sw)), v1 = *(const uint2 *)(vr + 16 * hs + ((8 + 2 * lg) ^ sw));
        const uint4 vv = make_uint4(v0.x, v0.y, v1.x, v1.y);
        const h8 vf = __builtin_bit_cast(h8, vv);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, ph[hs], o[d], 0, 0, 0);
        o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[hs], o[d], 0, 0, 0);
      }
    }
  }
  if (!tok_ok) return;   // a token's four lanes (lr, l ^ 16, l ^ 32, l ^ 48) leave together
  const float inv = 1.f / l;
  if (HD == kQB && a.oh) {
    // quantise the head (one 128-column block; quant_rows as k_pf_quant: mx = max |v|, isx = mx > 0 ? 32767 / mx : 0,
    // bs = mx / 32767, q = rint(v * isx), planes hi = q >> 8, lo = (q & 255) ^ 0x80)
    float v[DT][4], mx = 0.f;
#pragma unroll
    for (int d = 0; d < DT; d++)
#pragma unroll
      for (int i = 0; i < 4; i++) { v[d][i] = o[d][i] * inv; mx = fmaxf(mx, fabsf(v[d][i])); }
    mx = pair_max16(mx);
    mx = pair_max32(mx);
    const float isx = mx > 0 ? kActMax / mx : 0.f;
    if (lg == 0) {
      const float bs = mx / kActMax;
      a.ob[(size_t)t * a.ldb + head] = bs;
      a.obt[(size_t)head * a.ldbt + t] = bs;
    }
    int8_t *oh = a.oh + (size_t)t * a.ldo + head * HD, *ol = a.ol + (size_t)t * a.ldo + head * HD;
#pragma unroll
    for (int d = 0; d < DT; d++) {
      uint32_t hh = 0, ll = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int q = (int)__builtin_rintf(v[d][i] * isx);
        hh |= (uint32_t)((q >> 8) & 0xff) << (8 * i);
        ll |= (uint32_t)((q & 0xff) ^ 0x80) << (8 * i);
      }
      *(uint32_t *)(oh + 16 * d + 4 * lg) = hh;
      *(uint32_t *)(ol + 16 * d + 4 * lg) = ll;
    }
    return;
  }
  float *out = a.att + (size_t)t * a.lda + head * HD;
#pragma unroll
  for (int d = 0; d < DT; d++)
    *(float4 *)(out + 16 * d + 4 * lg) = make_float4(o[d][0] * inv, o[d][1] * inv, o[d][2] * inv, o[d][3] * inv);
}
hipError_t launch_pf_attn(const PfAttnArgs &a, hipStream_t st) {
  if (a.ntok <= 0) return hipSuccess;
  if (a.nh % a.nkv || (a.hd != 64 && a.hd != 128) || a.lda % 4 || (a.cos_t && !a.sin_t)) return hipErrorInvalidValue;
  if (a.oh && (a.hd != kQB || !a.ol || !a.ob || !a.obt || a.ldo % 4 || a.ldbt < a.ntok)) return hipErrorInvalidValue;
  const int units = (a.ntok + 15) / 16 * (a.nh / a.nkv);
  const dim3 grid((units + kPfAttnWaves - 1) / kPfAttnWaves, a.nkv);
  if (a.hd == 128) hipLaunchKernelGGL(k_pf_attn<128>, grid, dim3(kPfAttnWaves * 64), 0, st, a);
  else hipLaunchKernelGGL(k_pf_attn<64>, grid, dim3(kPfAttnWaves * 64), 0, st, a);
  return hipGetLastError();
}

// ------------------------------------------------------------------ SwiGLU of a token batch
// g = silu(g) * u in place (silu_mul with exp256, kernels_x86.cpp:427-431, the decode epilogue's arithmetic)
}  // namespace qph
