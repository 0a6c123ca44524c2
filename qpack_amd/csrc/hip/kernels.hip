// gfx950 kernels of the qpack Llama decode step.
//
// Matvec (the HBM-bound hot path): y = W x with W int8 (q8, f32 row scale) or int4 (q4, fp16 scale per 32 columns) and
// x quantised to int16 per 128-column block exactly as quant_rows does (/root/reference/src/kernels.cpp:17-31).
//   - Each workgroup first builds the activation in LDS as two byte planes, h = q >> 8 (signed) and l = q & 255
//     (unsigned), so one 4-byte weight word costs one v_dot4_i32_i8 (w . h) and one v_dot4_u32_u8 ((w ^ 0x80) . l):
//     w . q = 256 (w . h) + (w + 128) . l - 128 sum(l)   (q8)     nib . q = 256 (nib . h) + nib . l   (q4, nib = q + 8)
//     Every int32 accumulator is therefore exact and equal to the reference's _mm256_madd_epi16 sums.
//   - Weights stream once, coalesced: lane i of a wave reads bytes [16 i, 16 i + 16) of each 1 KiB row chunk.
//   - q8: the eight lanes of a 128-column block are summed with DPP; the block sums go to LDS as (float)isum and one
//     lane per row replays rows_q8's float epilogue in block order (acc = fma(bs[b], (float)isum, acc); y = acc * scale,
//     kernels_x86.cpp:57-69), so q8 rows are bit-identical to the reference given the same activation.
//   - q4: one lane owns one 32-column group (16 bytes); per-group exact int32 sums, fma with f16(scale) * bs in the lane,
//     then a fixed-order wave reduction (float order differs from rows_q4's 8-lane split: within the logit tolerance).
// The prologue optionally fuses RMSNorm (PRO_NORM); epilogues fuse bias, residual add, SwiGLU and the argmax partials.
#include <math.h>

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "act.hpp"
#include "launch.hpp"

namespace qph {

constexpr int kThreads = 256;

// LDS of the matvec kernel: activation planes, block scales / low-byte sums, group sums, reduction scratch, and per wave
// `per_wave` ints of block sums (q8) or unit values (q4) - at least nbp in total (the RMSNorm block sums use it first)
size_t mv_lds_bytes(int cols, int waves, int per_wave) {
  const int nb = cols / kQB, G = cols / 32, nbp = round_up(nb, 4);
  const size_t sums = std::max<size_t>((size_t)waves * per_wave, (size_t)nbp);
  return (size_t)2 * cols + 4 * (size_t)nbp * 2 + 4 * (size_t)round_up(G, 4) + 32 * 4 + 4 * sums;
}


// ------------------------------------------------------------------ streaming matvec
// one 16-byte weight load: global_load_dwordx4 with the nontemporal hint (the weights stream through once per token;
// the hint keeps them from displacing the activations and the kv cache in the caches - C3 decode 461 -> 473 tok/s)
__device__ __forceinline__ uint4 ld16(const void *p) {
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load((const v4u *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float lane_bcast(float v, int lane) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane)); }
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }
// (max, lowest index) over the wave, in every lane: the butterfly of wave_max (partners lane ^ 32, ^ 16 by permlane
// swaps, ^ 8, ^ 4 by row rotations, ^ 2, ^ 1 by quad permutations), each step keeping the better of the pair - a total
// order, so both lanes of a pair keep the same (value, index), which the rotation by 4 relies on
__device__ __forceinline__ void wave_argmax(float &v, int &i) {
  auto pick = [&](float ov, int oi) { if (better(ov, oi, v, i)) { v = ov; i = oi; } };
  {
    float a, b, c, d;
    swap32(v, a, b); swap32(__builtin_bit_cast(float, i), c, d);
    v = a; i = __builtin_bit_cast(int, c); pick(b, __builtin_bit_cast(int, d));
  }
  {
    float a, b, c, d;
    swap16(v, a, b); swap16(__builtin_bit_cast(float, i), c, d);
    v = a; i = __builtin_bit_cast(int, c); pick(b, __builtin_bit_cast(int, d));
  }
  pick(dpp_f<kDppRowRor8>(v), dpp_i<kDppRowRor8>(i));
  pick(dpp_f<kDppRowRor4>(v), dpp_i<kDppRowRor4>(i));
  pick(dpp_f<kDppQuadXor2>(v), dpp_i<kDppQuadXor2>(i));
  pick(dpp_f<kDppQuadXor1>(v), dpp_i<kDppQuadXor1>(i));
}

// A unit is NS rows of one segment (EPI_SWIGLU: row r of the gate and of the up matrix).  Waves own units
// round-robin and stream them chunk by chunk (1 KiB of every row of the unit per step: lane i reads bytes [16 i, 16 i + 16)).
template <int NS>
struct UnitGeo {
  const uint8_t *p[NS];     // row bytes (clamped rows)
  const uint16_t *sp[NS];   // q4 / q1 fp16 scale rows
  const float *sc[NS];      // q8 row scale
  int row[NS];              // output rows (may be >= rows: computed, not stored)
  int rows, seg, kind, nch, rowbytes;
};

template <int EPI, int NS>
__device__ __forceinline__ UnitGeo<NS> unit_geo(const MvArgs &a, int u, int cols) {
  UnitGeo<NS> g;
  int seg = 0;
  if (EPI != EPI_SWIGLU && a.nseg > 1 && u >= a.seg_tile0[1]) seg = (a.nseg > 2 && u >= a.seg_tile0[2]) ? 2 : 1;
  const DMat m0 = seg == 0 ? a.m[0] : (seg == 1 ? a.m[1] : a.m[2]);
  const int u0 = seg == 0 ? a.seg_tile0[0] : (seg == 1 ? a.seg_tile0[1] : a.seg_tile0[2]);
  g.seg = seg; g.kind = m0.kind; g.rows = m0.rows;
  g.rowbytes = m0.kind == MK_Q8 ? cols : m0.kind == MK_Q4 ? cols / 2 : cols / 8;
  const int sgroups = m0.kind == MK_Q1 ? cols / 128 : cols / 32;   // fp16 scales per row (q4, q1)
  g.nch = (g.rowbytes + 1023) >> 10;
  const bool rope = EPI == EPI_STORE && NS == 2 && (seg == 0 ? a.rope[0] : (seg == 1 ? a.rope[1] : a.rope[2]));
  const int H = a.hd / 2;
#pragma unroll
  for (int s = 0; s < NS; s++) {
    const DMat m = (EPI == EPI_SWIGLU && s == 1) ? a.m[1] : m0;
    const int lu = u - u0;
    const int r = EPI == EPI_SWIGLU ? lu : (rope ? (lu / H) * a.hd + lu % H + s * H : lu * NS + s);
    g.row[s] = r;
    const int rc = r < m.rows ? r : m.rows - 1;
    g.p[s] = (const uint8_t *)m.q + (size_t)rc * g.rowbytes;
    g.sp[s] = (const uint16_t *)m.s + (size_t)rc * sgroups;
    g.sc[s] = (const float *)m.s + rc;
  }
  return g;
}

// row pointers of unit u (NS rows of one segment; EPI_SWIGLU: row u of the gate and of the up matrix)
template <int EPI, int NS>
__device__ __forceinline__ void unit_rows(const MvArgs &a, int u, int cols, const uint8_t *(&p)[NS], const uint16_t *(&sp)[NS]) {
  const UnitGeo<NS> g = unit_geo<EPI, NS>(a, u, cols);
#pragma unroll
  for (int s = 0; s < NS; s++) { p[s] = g.p[s]; sp[s] = g.sp[s]; }
}

// The matvec kernel.  Per wave: a ring of D prefetched steps (one 1 KiB chunk of each of the unit's NS rows per step,
// issued right after the activation reads so streaming starts at launch), and a main loop whose only vector memory
// operations are those unconditional prefetch loads: a wave's loads return in order, and any other load or store in
// the loop would make the compiler wait for the whole ring.  Block sums (q8) and unit results (q4) go to LDS; the
// fp32 chains, scales and stores run after the loop, one lane per (unit, row).
template <int PRO, int EPI, int NS, int KIND, bool DBG>
__global__ __launch_bounds__(1024) void k_matvec(MvArgs a) {
  // ring slots per wave (a slot: one 1 KiB chunk of each of the unit's NS rows); measured with the nontemporal weight
  // loads, same box, C3 / C5 greedy tok/s: 8 / NS 486 / 480, 6 / NS 494 / 499, (4, 2) 510 / 519, (3, 2) 513 / 525,
  // (2, 2) 512 / 524, (3, 1) 499 / 517 - more loads in flight per wave only queue behind each other
  constexpr int D = NS == 1 ? 3 : 2;
  extern __shared__ __align__(16) char smem[];
  const int WAVES = (int)blockDim.x >> 6;
  const int cols = a.m[0].cols, G = cols / 32, nb = cols / kQB;
  const ActView av = act_view(smem, cols);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int Wg = gridDim.x * WAVES, gw = wave * gridDim.x + blockIdx.x;
  // the wave's weight kind, its index among the waves of that kind (W of them) and its units [ub, ub + U): one kind per
  // launch, or (MK_MIX) the first mix_w8 waves over the q8 segments' units and the rest over the q4 units
  const bool mq8 = KIND == MK_MIX && gw < a.mix_w8;
  const bool isq8 = KIND == MK_Q8 || mq8, isq1 = KIND == MK_Q1, isq4 = KIND == MK_Q4 || (KIND == MK_MIX && !mq8);
  const int W = KIND != MK_MIX ? Wg : (mq8 ? a.mix_w8 : Wg - a.mix_w8);
  const int gk = KIND != MK_MIX || mq8 ? gw : gw - a.mix_w8;
  const int ub = KIND != MK_MIX || mq8 ? 0 : a.mix_u8;
  const int U = (KIND != MK_MIX ? a.seg_tile0[a.nseg] : (mq8 ? a.mix_u8 : a.seg_tile0[a.nseg])) - ub;
  const int nmine = gk < U ? (U - gk + W - 1) / W : 0;
  const int rowbytes = isq8 ? cols : isq4 ? cols / 2 : cols / 8;
  const int GS = isq1 ? cols / 128 : G;   // the scale group a lane's 16 bytes belong to: 32 (q4) or 128 (q1) columns
  const int nch = (rowbytes + 1023) >> 10;
  const int total = nmine * nch;
  // per-wave LDS: q8 block sums [upw][NS][nbp] ints, q4 / q1 unit values [upw][NS] floats (MK_MIX: the q8 size for all)
  int *wsum = av.sums + wave * (a.upw * NS * (KIND == MK_Q8 || KIND == MK_MIX ? av.nbp : 1));
  float *wval = (float *)wsum;

  ActRegs ar;
  const int dm = a.dbg_mode;
  uint64_t ts0 = 0, ts1 = 0, ts2 = 0;
  if (a.stamps) ts0 = __builtin_amdgcn_s_memrealtime();
  const int pos = EPI == EPI_STORE && NS == 2 && a.ctl ? a.ctl->pos : 0;   // RoPE / cache position
  if (!(dm & 2)) act_load<PRO>(a.x, a.norm_w, cols, ar, a.part, a.nparts, a.pstride, a.xsum, (float *)av.sums);

  uint4 wr[D][NS];
  uint16_t sr[D][NS];
  int pi = 0, pc = 0;
  const uint8_t *pp[NS]; const uint16_t *psp[NS];
  unit_rows<EPI, NS>(a, ub + (nmine ? gk : 0), cols, pp, psp);
  auto issue = [&](uint4 (&w)[NS], uint16_t (&sv)[NS]) {
    // past the wave's last unit every lane re-reads the same 16 bytes (one cache line, no HBM traffic)
    const bool live = pi < nmine;
    const int off = pc * 1024 + lane * 16, grp = pc * 64 + lane;
    const int offc = !live ? 0 : (off < rowbytes ? off : rowbytes - 16);
    const int grpc = !live ? 0 : (grp < GS ? grp : GS - 1);
#pragma unroll
    for (int s = 0; s < NS; s++) {
      w[s] = ld16(pp[s] + offc);
      if (!isq8) sv[s] = psp[s][grpc];
    }
    if (live && ++pc == nch) { pc = 0; if (++pi < nmine) unit_rows<EPI, NS>(a, ub + gk + pi * W, cols, pp, psp); }
  };
#pragma unroll
  for (int k = 0; k < D; k++) issue(wr[k], sr[k]);

  if (!(dm & 2)) act_build<PRO, KIND == MK_Q1>(ar, a.eps, cols, av);
  else __syncthreads();
  if (a.stamps) ts1 = __builtin_amdgcn_s_memrealtime();
  if (DBG && blockIdx.x == 0) {
    for (int c = threadIdx.x; c < cols; c += blockDim.x) {
      const int at = KIND == MK_Q1 ? (((c & 127) >> 4) * nb + (c >> 7)) * 16 + (c & 15) : c;   // q1: chunk-major planes
      if (a.dbg_xq) a.dbg_xq[c] = (int16_t)(((int)av.xh[at] << 8) | av.xl[at]);
    }
    for (int b = threadIdx.x; b < nb; b += blockDim.x)
      if (a.dbg_bs) a.dbg_bs[b] = av.bs[b];
  }

  int ci = 0, cc = 0;
  float acc[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) acc[s] = 0.f;
  for (int t0 = 0; t0 < total; t0 += D) {
#pragma unroll
    for (int k = 0; k < D; k++) {
      // consume slot k, then refill it: the load reuses the slot's registers (taking a copy first and loading
      // before the use would need new registers and a copy per slot at the loop edge, which waits for the whole ring)
      const uint4 (&cur)[NS] = wr[k]; const uint16_t (&curs)[NS] = sr[k];
      if (t0 + k < total) {
        if (dm & 1) {
#pragma unroll
          for (int s = 0; s < NS; s++) acc[s] += (float)(cur[s].x ^ cur[s].y ^ cur[s].z ^ cur[s].w);
        } else if (isq8) {
          const int col = cc * 1024 + lane * 16;
          const bool act = col < cols;
          const int colc = act ? col : cols - 16;
          const uint4 h = *(const uint4 *)(av.xh + colc);
          const uint4 l = *(const uint4 *)(av.xl + colc);
#pragma unroll
          for (int s = 0; s < NS; s++) {
            const uint4 ww = cur[s];
            int A = __builtin_amdgcn_sdot4((int)ww.x, (int)h.x, 0, false);
            A = __builtin_amdgcn_sdot4((int)ww.y, (int)h.y, A, false);
            A = __builtin_amdgcn_sdot4((int)ww.z, (int)h.z, A, false);
            A = __builtin_amdgcn_sdot4((int)ww.w, (int)h.w, A, false);
            uint32_t B = __builtin_amdgcn_udot4(ww.x ^ 0x80808080u, l.x, 0u, false);
            B = __builtin_amdgcn_udot4(ww.y ^ 0x80808080u, l.y, B, false);
            B = __builtin_amdgcn_udot4(ww.z ^ 0x80808080u, l.z, B, false);
            B = __builtin_amdgcn_udot4(ww.w ^ 0x80808080u, l.w, B, false);
            const int p = sum8_i(A * 256 + (int)B);
            if (act && (lane & 7) == 0) {   // the block sum, as the float the chain takes (DBG: the int, for the hook)
              const int b = cc * 8 + (lane >> 3);
              const int isum = p - 128 * av.lsum[b];
              if (DBG) wsum[(ci * NS + s) * av.nbp + b] = isum;
              else ((float *)wsum)[(ci * NS + s) * av.nbp + b] = (float)isum;
            }
          }
        } else if (isq1) {
          // one lane = one 128-column group: sign bit c of its 16 bytes is column 128 g + c (+1 set, -1 clear).
          // Each nibble becomes four byte masks (bit k -> byte k: nib * 0x204081 & 0x01010101), dotted with the high
          // and low activation planes: S = sum of x over the set bits, exact; the group's dot product is 2 S - sum(x).
          const int g = cc * 64 + lane;
          const bool act = g < GS;
          const int gc = act ? g : GS - 1;
          // chunk-major activation planes (act_build<PRO, true>): piece k of group gc at (k * nb + gc) * 16
          const uint4 *hp = (const uint4 *)(av.xh + 16 * gc), *lp = (const uint4 *)(av.xl + 16 * gc);
          const int4 gs4 = *(const int4 *)(av.gsum + 4 * gc);
          const int xsum = gs4.x + gs4.y + gs4.z + gs4.w;
          const float bsg = av.bs[gc];
#pragma unroll
          for (int s = 0; s < NS; s++) {
            const uint32_t wd[4] = {cur[s].x, cur[s].y, cur[s].z, cur[s].w};
            int A[4] = {0, 0, 0, 0}; uint32_t B[4] = {0, 0, 0, 0};   // per dword: 4 chains of 8, integer sums
#pragma unroll
            for (int j = 0; j < 4; j++) {          // 32 columns per dword
#pragma unroll
              for (int hh = 0; hh < 2; hh++) {     // 16 columns per activation load
                const uint4 h = hp[(2 * j + hh) * nb], l = lp[(2 * j + hh) * nb];
                const uint32_t hx[4] = {h.x, h.y, h.z, h.w}, lx[4] = {l.x, l.y, l.z, l.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                  const uint32_t nib = (wd[j] >> (16 * hh + 4 * k)) & 15u;
                  const uint32_t msk = (nib * 0x204081u) & 0x01010101u;
                  A[j] = __builtin_amdgcn_sdot4((int)msk, (int)hx[k], A[j], false);
                  B[j] = __builtin_amdgcn_udot4(msk, lx[k], B[j], false);
                }
              }
            }
            const int isum = 2 * ((A[0] + A[1] + A[2] + A[3]) * 256 + (int)(B[0] + B[1] + B[2] + B[3])) - xsum;
            if (DBG && act && a.dbg_sums) {
              const UnitGeo<NS> og = unit_geo<EPI, NS>(a, ub + gk + ci * W, cols);
              if (og.seg == 0 && og.row[s] < og.rows) a.dbg_sums[(size_t)og.row[s] * GS + g] = isum;
            }
            if (act) acc[s] = __builtin_fmaf(half_bits_to_float(curs[s]) * bsg, (float)isum, acc[s]);
          }
        } else {
          const int g = cc * 64 + lane;
          const bool act = g < G;
          const int gc = act ? g : G - 1;
          const uint4 h0 = *(const uint4 *)(av.xh + 32 * gc), h1 = *(const uint4 *)(av.xh + 32 * gc + 16);
          const uint4 l0 = *(const uint4 *)(av.xl + 32 * gc), l1 = *(const uint4 *)(av.xl + 32 * gc + 16);
          const int hx[8] = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
          const uint32_t lx[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
          const int corr = 8 * av.gsum[gc];
          const float bsg = av.bs[gc >> 2];
#pragma unroll
          for (int s = 0; s < NS; s++) {
            const uint32_t wd[4] = {cur[s].x, cur[s].y, cur[s].z, cur[s].w};
            // low and high nibbles in separate accumulators: four dependent chains of 4 instead of two of 8 (integer
            // sums, so the result is the same)
            int A0 = 0, A1 = 0; uint32_t B0 = 0, B1 = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
              const uint32_t lo = wd[j] & 0x0f0f0f0fu, hi = (wd[j] >> 4) & 0x0f0f0f0fu;
              A0 = __builtin_amdgcn_sdot4((int)lo, hx[j], A0, false);
              A1 = __builtin_amdgcn_sdot4((int)hi, hx[4 + j], A1, false);
              B0 = __builtin_amdgcn_udot4(lo, lx[j], B0, false);
              B1 = __builtin_amdgcn_udot4(hi, lx[4 + j], B1, false);
            }
            const int isum = (A0 + A1) * 256 + (int)(B0 + B1) - corr;
            if (DBG && act && a.dbg_sums) {
              const UnitGeo<NS> og = unit_geo<EPI, NS>(a, ub + gk + ci * W, cols);
              if (og.seg == 0 && og.row[s] < og.rows) a.dbg_sums[(size_t)og.row[s] * G + g] = isum;
            }
            if (act) acc[s] = __builtin_fmaf(half_bits_to_float(curs[s]) * bsg, (float)isum, acc[s]);
          }
        }
        if (++cc == nch) {   // unit complete: q4 / q1 values to LDS (LDS and cross-lane ops only inside the loop)
          if (!isq8) {
#pragma unroll
            for (int s = 0; s < NS; s++) {
              const float v = wave_sum_dpp(acc[s]);
              if (lane == 0) wval[ci * NS + s] = v;
              acc[s] = 0.f;
            }
          }
          cc = 0; ci++;
        }
      }
      issue(wr[k], sr[k]);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (a.stamps) ts2 = __builtin_amdgcn_s_memrealtime();
  if (dm & 4) return;   // timing: no epilogue

  // epilogue: lane j finishes (unit j / NS, row slot j % NS); with the split chain, lanes lpr j .. lpr j + lpr - 1 do
  // (lpr lanes per row: 8, or 4 / 2 where the wave's rows need more lanes)
  const int nrows = nmine * NS;
  const bool split = !DBG && (EPI == EPI_RESID || EPI == EPI_SWIGLU) && KIND == MK_Q8 && a.split_chain && nrows <= kWave / 2;
  const int lpr = !split ? 1 : nrows <= kWave / 8 ? 8 : nrows <= kWave / 4 ? 4 : 2;
  const int lsh = lpr == 8 ? 3 : lpr == 4 ? 2 : lpr == 2 ? 1 : 0, part = lane & (lpr - 1);
  float best_v = -INFINITY; int best_i = 0x7fffffff;
  for (int j0 = 0; j0 < nrows; j0 += kWave / lpr) {
    const int j = j0 + (lane >> lsh), u = j / NS, s = j % NS;
    const bool live = j < nrows;
    const UnitGeo<NS> og = unit_geo<EPI, NS>(a, ub + gk + (live ? u : 0) * W, cols);
    int row = og.row[0]; const float *scl = og.sc[0];
#pragma unroll
    for (int t = 1; t < NS; t++) if (s == t) { row = og.row[t]; scl = og.sc[t]; }
    float v = 0.f;
    // the row scale and the residual are loaded before the chain, so their round trips overlap it
    const bool store = live && row < og.rows && part == 0;
    const float sc_pre = live && isq8 ? *scl : 0.f;
    float res_pre = 0.f;
    if (EPI == EPI_RESID && store) res_pre = a.resid_in ? a.resid_in[row] : a.out[0][row];
    if (split) {
      // blocks [part nbk, (part + 1) nbk) chained in order (nbk: 1 / lpr of the blocks rounded up to whole float4
      // reads), then the lane partials summed pairwise: ((c0 + c1) + (c2 + c3)) + ((c4 + c5) + (c6 + c7)) for lpr 8
      const int nbk = ((nb + 4 * lpr - 1) / (4 * lpr)) * 4, b0 = min(nb, part * nbk), b1 = min(nb, b0 + nbk);
      const float *sf = (const float *)(wsum + ((live ? u : 0) * NS + s) * av.nbp);
      float ch = 0.f;
      int b = b0;
      for (; b + 4 <= b1; b += 4) {
        const float4 sv = *(const float4 *)(sf + b), bv = *(const float4 *)(av.bs + b);
        ch = __builtin_fmaf(bv.x, sv.x, ch); ch = __builtin_fmaf(bv.y, sv.y, ch);
        ch = __builtin_fmaf(bv.z, sv.z, ch); ch = __builtin_fmaf(bv.w, sv.w, ch);
      }
      for (; b < b1; b++) ch = __builtin_fmaf(av.bs[b], sf[b], ch);
      // the lane partials summed over lanes l ^ 1, l ^ 2 (quad permutations) and l + 4, which is l ^ 4 in the lanes
      // that keep the row's value (part 0): DPP, the same sums as xor shuffles without the LDS crossbar
      if (lpr > 1) ch += dpp_f<kDppQuadXor1>(ch);
      if (lpr > 2) ch += dpp_f<kDppQuadXor2>(ch);
      if (lpr > 4) ch += dpp_f<kDppRowShl4>(ch);
      v = ch * sc_pre;
    } else if (live) {
      if (isq8) {
        const int *ss = wsum + (u * NS + s) * av.nbp;
        const float *sf = (const float *)ss;
        float ch = 0.f;   // rows_q8's block order; LDS read 16 blocks at a time so the chain is not latency-bound
        int b = 0;
        for (; b + 16 <= nb; b += 16) {
          float4 sv[4], bv[4];
#pragma unroll
          for (int q = 0; q < 4; q++) {
            if (DBG) { const int4 t = *(const int4 *)(ss + b + 4 * q); sv[q] = make_float4((float)t.x, (float)t.y, (float)t.z, (float)t.w); }
            else sv[q] = *(const float4 *)(sf + b + 4 * q);
            bv[q] = *(const float4 *)(av.bs + b + 4 * q);
          }
#pragma unroll
          for (int q = 0; q < 4; q++) {
            ch = __builtin_fmaf(bv[q].x, sv[q].x, ch); ch = __builtin_fmaf(bv[q].y, sv[q].y, ch);
            ch = __builtin_fmaf(bv[q].z, sv[q].z, ch); ch = __builtin_fmaf(bv[q].w, sv[q].w, ch);
          }
        }
        for (; b < nb; b++) ch = __builtin_fmaf(av.bs[b], DBG ? (float)ss[b] : sf[b], ch);
        v = ch * sc_pre;
        if (DBG && a.dbg_sums && og.seg == 0 && row < og.rows)
          for (int b = 0; b < nb; b++) a.dbg_sums[(size_t)row * nb + b] = ss[b];
      } else {
        v = wval[u * NS + s];
      }
    }
    if (EPI == EPI_STORE && NS == 2 && a.ctl) {
      // RoPE of q / k rows (the partner row of the pair sits in the next lane) and the fp16 cache rows
      const int sg = og.seg;
      const float *const bias_seg = sg == 0 ? a.bias[0] : (sg == 1 ? a.bias[1] : a.bias[2]);
      float y = v;
      if (store && bias_seg) y = y + bias_seg[row];
      const float yo = dpp_f<kDppQuadXor1>(y);   // the pair's other row, lane ^ 1
      const bool rope = sg == 0 ? a.rope[0] : (sg == 1 ? a.rope[1] : a.rope[2]);
      uint16_t *const cache = sg == 0 ? a.cache[0] : (sg == 1 ? a.cache[1] : a.cache[2]);
      if (store) {
        if (rope) {
          const int H = a.hd / 2, i = row % H;
          const float cs = a.cos_t[(size_t)pos * H + i], sn = a.sin_t[(size_t)pos * H + i];
          y = s == 0 ? __builtin_fmaf(y, cs, -(yo * sn)) : __builtin_fmaf(y, cs, yo * sn);
        }
        (sg == 0 ? a.out[0] : (sg == 1 ? a.out[1] : a.out[2]))[row] = y;
        if (cache) cache[(size_t)pos * a.cache_ld + row] = f32_to_half_bits(y);
        uint16_t *const q16 = sg == 0 ? a.q16[0] : (sg == 1 ? a.q16[1] : a.q16[2]);
        if (q16) {   // the attention's MFMA operand halves: hi = f16(y), lo = f16(y - hi)
          const _Float16 h = (_Float16)y;
          q16[row] = __builtin_bit_cast(uint16_t, h);
          q16[og.rows + row] = __builtin_bit_cast(uint16_t, (_Float16)(y - (float)h));
        }
      }
    } else if (EPI == EPI_SWIGLU) {
      // slot 1 (up) sits lpr lanes after slot 0 (gate): lane ^ lpr for the gate lanes that store (part 0)
      const float up = lpr == 1 ? dpp_f<kDppQuadXor1>(v) : lpr == 2 ? dpp_f<kDppQuadXor2>(v)
                     : lpr == 4 ? dpp_f<kDppRowShl4>(v) : dpp_f<kDppRowRor8>(v);
      if (store && s == 0) a.out[0][row] = v / (1.f + exp_poly(0.f - v)) * up;   // silu_mul, kernels_x86.cpp:427-431
    } else if (store) {
      float *const out_seg = og.seg == 0 ? a.out[0] : (og.seg == 1 ? a.out[1] : a.out[2]);
      const float *const bias_seg = og.seg == 0 ? a.bias[0] : (og.seg == 1 ? a.bias[1] : a.bias[2]);
      if (EPI == EPI_STORE) { float y = v; if (bias_seg) y = y + bias_seg[row]; out_seg[row] = y; }
      else if (EPI == EPI_RESID) a.out[0][row] = res_pre + v;
      else { a.out[0][row] = v; if (better(v, row, best_v, best_i)) { best_v = v; best_i = row; } }
    }
  }
  if (EPI == EPI_ARGMAX) {
    wave_argmax(best_v, best_i);
    __syncthreads();
    float *rv = av.red; int *ri = (int *)(av.red + 16);
    if (lane == 0) { rv[wave] = best_v; ri[wave] = best_i; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = rv[0]; int bi = ri[0];
      for (int w = 1; w < WAVES; w++) if (better(rv[w], ri[w], bv, bi)) { bv = rv[w]; bi = ri[w]; }
      a.amax[blockIdx.x] = make_float2(bv, __builtin_bit_cast(float, bi));
    }
  }
  if (a.stamps && lane == 0) {   // measurement: per wave, realtime at start, after the prologue, after the loop, at the end
    uint64_t *o = a.stamps + 4 * ((size_t)blockIdx.x * WAVES + wave);
    o[0] = ts0; o[1] = ts1; o[2] = ts2; o[3] = __builtin_amdgcn_s_memrealtime();
  }
}

// rows per unit: SwiGLU units are one gate/up row pair; large matrices stream 2 rows per unit (the activation LDS reads
// serve both), small ones 1 row so every wave gets an equal share
static int mv_ns(const MvArgs &a, int epi, int waves) {
  if (epi == EPI_SWIGLU || (epi == EPI_STORE && a.ctl)) return 2;   // SwiGLU pairs; RoPE pairs (q / k / v)
  int rows = 0;
  for (int s = 0; s < a.nseg; s++) rows += a.m[s].rows;
  return rows >= 4 * waves ? 2 : 1;
}
int mv_tile_rows(int epi) { return epi == EPI_SWIGLU ? 1 : 2; }
void mv_plan(MvArgs &a, int epi) {
  // unit prefix per segment for 2-row units; launch_matvec re-plans when it picks 1-row units
  const int ns = epi == EPI_SWIGLU ? 1 : 2; int t = 0;
  const int nseg = epi == EPI_SWIGLU ? 1 : a.nseg;
  for (int s = 0; s < nseg; s++) { a.seg_tile0[s] = t; t += (a.m[s].rows + ns - 1) / ns; }
  a.seg_tile0[nseg] = t;
  if (epi == EPI_SWIGLU) a.nseg = 1;
}

// Launch shape: every CU gets one workgroup of `w` waves and every wave the same number of units, where possible:
// units per CU upc = ceil(U / cus); w = the largest divisor of upc in [4, 16] (16 when there is none).
template <int PRO, int EPI, int NS, int KIND>
static hipError_t launch_mv_t(MvArgs a, int grid_cap, hipStream_t st) {
  if (EPI != EPI_SWIGLU) {
    int t = 0;
    for (int s = 0; s < a.nseg; s++) { a.seg_tile0[s] = t; t += (a.m[s].rows + NS - 1) / NS; }
    a.seg_tile0[a.nseg] = t;
  }
  const int units = a.seg_tile0[a.nseg], cus = g_mv_config.cus;
  const int upc = (units + cus - 1) / cus;
  // at most 8 waves per workgroup for gate / up and the head, 16 for the rest (same-box sweep, C3 greedy: 16
  // everywhere 513.9 tok/s, 8 for gate / up and head 521.7, 12 for all 521.1, 6 or 4 for gate / up and head ~467)
  constexpr int WM = EPI == EPI_SWIGLU || EPI == EPI_ARGMAX ? 8 : 16;
  int w = upc <= WM ? upc : WM;
  if (upc > WM) for (int c = WM; c >= 4; c--) if (upc % c == 0) { w = c; break; }
  int u = (upc + w - 1) / w;                                        // units per wave
  const int cols = a.m[0].cols;
  if (cols / kQB > 2 * w * 8) { w = 16; u = (upc + 15) / 16; }     // the prologue covers 2 x (threads / 8) blocks
  int grid = (units + w * u - 1) / (w * u);
  // units are dealt round-robin over all the launch's waves, so a grid short of the CU count (units per CU with no
  // divisor in 4..16) only leaves CUs idle: one workgroup per CU then
  if (grid < cus && units >= cus) grid = cus;
  if (grid > grid_cap) return hipErrorInvalidValue;
  // a wave may own one unit more than u when the grid rounds: size the per-wave LDS for ceil(units / waves)
  const int waves = grid * w;
  if (a.stamps && a.stamp_waves > 0 && waves > a.stamp_waves) a.stamps = nullptr;
  a.upw = (units + waves - 1) / waves;
  if (KIND == MK_MIX) {
    // q8 segments first: their units [0, u8) go to the first w8 waves, w8 in proportion to their bytes
    int n8 = 0;
    while (n8 < a.nseg && a.m[n8].kind == MK_Q8) n8++;
    const int u8 = a.seg_tile0[n8];
    double b8 = 0, b4 = 0;
    for (int s = 0; s < a.nseg; s++) (s < n8 ? b8 : b4) += (double)a.m[s].rows * (s < n8 ? cols : cols / 2);
    if (n8 == 0 || n8 == a.nseg || waves < 2) return hipErrorInvalidValue;
    int w8 = (int)(waves * b8 / (b8 + b4) + 0.5);
    w8 = w8 < 1 ? 1 : (w8 > waves - 1 ? waves - 1 : w8);
    a.mix_w8 = w8; a.mix_u8 = u8;
    const int up8 = (u8 + w8 - 1) / w8, up4 = (units - u8 + (waves - w8) - 1) / (waves - w8);
    a.upw = up8 > up4 ? up8 : up4;
  }
  const int nbp = ((cols / kQB) + 3) / 4 * 4;
  size_t lds = mv_lds_bytes(cols, w, a.upw * NS * (KIND == MK_Q8 || KIND == MK_MIX ? nbp : 1));
  if (PRO == PRO_NORM_SUM) {   // the partial sets' hand-over area at the sums offset
    if (a.nparts < 1 || a.nparts > kMaxParts) return hipErrorInvalidValue;
    const int ns = act_part_sets(cols, w * 64, a.nparts);
    lds = std::max(lds, mv_lds_bytes(cols, w, 0) - 4 * (size_t)nbp + 4 * (size_t)(ns - 1) * cols);
  }
  if (lds > 160 * 1024) return hipErrorInvalidValue;
  if (a.plan_only) return hipSuccess;
  const bool dbg = a.dbg_sums || a.dbg_xq || a.dbg_bs;
  if (dbg) {
    if (PRO != PRO_QUANT || EPI != EPI_STORE || KIND == MK_MIX) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_matvec<PRO_QUANT, EPI_STORE, NS, KIND, true>), dim3(grid), dim3(w * 64), lds, st, a);
  } else {
    hipLaunchKernelGGL((k_matvec<PRO, EPI, NS, KIND, false>), dim3(grid), dim3(w * 64), lds, st, a);
  }
  return hipGetLastError();
}
template <int KIND>
static hipError_t launch_mv_k(int pro, int epi, const MvArgs &a, int ns, int grid_cap, hipStream_t st) {
#define QPH_MV(P, E) \
  if (pro == P && epi == E) return ns == 2 ? launch_mv_t<P, E, 2, KIND>(a, grid_cap, st) : launch_mv_t<P, E, 1, KIND>(a, grid_cap, st);
  QPH_MV(PRO_QUANT, EPI_STORE) QPH_MV(PRO_QUANT, EPI_RESID) QPH_MV(PRO_NORM, EPI_STORE) QPH_MV(PRO_NORM, EPI_ARGMAX)
  QPH_MV(PRO_QUANT, EPI_ARGMAX)
#undef QPH_MV
  if (pro == PRO_NORM && epi == EPI_SWIGLU) return launch_mv_t<PRO_NORM, EPI_SWIGLU, 2, KIND>(a, grid_cap, st);
  if (pro == PRO_NORM_SUM && epi == EPI_SWIGLU) return launch_mv_t<PRO_NORM_SUM, EPI_SWIGLU, 2, KIND>(a, grid_cap, st);
  return hipErrorInvalidValue;
}
MvConfig g_mv_config;
// grid_cap: the most workgroups one launch may use (EPI_ARGMAX writes one (max, index) partial per workgroup).
// Segments of q8 and q4 (q4m: q4 wq / wk with a q8 wv) go out as one MK_MIX launch of the stored-output kernels, where
// each wave streams one kind; other mixes (q1) as one launch per kind.
hipError_t launch_matvec(int pro, int epi, const MvArgs &a, int grid_cap, hipStream_t st) {
  const int cols = a.m[0].cols;
  if (cols % kQB || cols > 32768) return hipErrorInvalidValue;
  if (a.ctl) {   // RoPE / cache rows: the decode q / k / v launch
    if (epi != EPI_STORE || a.hd < 2 || a.hd % 2 || !a.cos_t || !a.sin_t) return hipErrorInvalidValue;
    for (int s = 0; s < a.nseg; s++)
      if ((a.rope[s] && a.m[s].rows % a.hd) || (!a.rope[s] && a.m[s].rows % 2)) return hipErrorInvalidValue;
  }
  const int nseg = epi == EPI_SWIGLU ? 1 : a.nseg;
  bool has8 = false, has4 = false, has1 = false;
  for (int s = 0; s < nseg; s++) { has8 |= a.m[s].kind == MK_Q8; has4 |= a.m[s].kind == MK_Q4; has1 |= a.m[s].kind == MK_Q1; }
  const bool dbg = a.dbg_sums || a.dbg_xq || a.dbg_bs;
  if (has8 && has4 && !has1 && epi == EPI_STORE && !dbg && !getenv("QPH_MV_NOMIX")) {
    MvArgs b = a; b.nseg = 0;
    for (int k : {(int)MK_Q8, (int)MK_Q4})
      for (int s = 0; s < nseg; s++)
        if (a.m[s].kind == k) {
          b.m[b.nseg] = a.m[s]; b.out[b.nseg] = a.out[s]; b.bias[b.nseg] = a.bias[s];
          b.rope[b.nseg] = a.rope[s]; b.cache[b.nseg] = a.cache[s]; b.q16[b.nseg] = a.q16[s]; b.nseg++;
        }
    const int ns = mv_ns(b, epi, g_mv_config.cus * 16);
    if (pro == PRO_NORM) return ns == 2 ? launch_mv_t<PRO_NORM, EPI_STORE, 2, MK_MIX>(b, grid_cap, st)
                                        : launch_mv_t<PRO_NORM, EPI_STORE, 1, MK_MIX>(b, grid_cap, st);
    return ns == 2 ? launch_mv_t<PRO_QUANT, EPI_STORE, 2, MK_MIX>(b, grid_cap, st)
                   : launch_mv_t<PRO_QUANT, EPI_STORE, 1, MK_MIX>(b, grid_cap, st);
  }
  for (int k : {(int)MK_Q8, (int)MK_Q4, (int)MK_Q1}) {
    MvArgs b = a; b.nseg = 0;
    for (int s = 0; s < nseg; s++)
      if (a.m[s].kind == k) {
        b.m[b.nseg] = a.m[s]; b.out[b.nseg] = a.out[s]; b.bias[b.nseg] = a.bias[s];
        b.rope[b.nseg] = a.rope[s]; b.cache[b.nseg] = a.cache[s]; b.q16[b.nseg] = a.q16[s]; b.nseg++;
      }
    if (!b.nseg) continue;
    if (epi == EPI_SWIGLU) { b.m[1] = a.m[1]; b.nseg = 1; b.seg_tile0[0] = 0; b.seg_tile0[1] = a.m[0].rows; }
    if (b.nseg != nseg && (b.dbg_sums || epi == EPI_ARGMAX)) return hipErrorInvalidValue;
    const int ns = mv_ns(b, epi, g_mv_config.cus * 16);
    const hipError_t e = k == MK_Q8 ? launch_mv_k<MK_Q8>(pro, epi, b, ns, grid_cap, st)
                         : k == MK_Q4 ? launch_mv_k<MK_Q4>(pro, epi, b, ns, grid_cap, st)
                                      : launch_mv_k<MK_Q1>(pro, epi, b, ns, grid_cap, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// ------------------------------------------------------------------ embedding, norm
__global__ __launch_bounds__(kThreads) void k_embed(DMat e, const Ctl *ctl, float *x) { embed_row(e, ctl->tok, x, threadIdx.x, kThreads); }
hipError_t launch_embed(const DMat &embed, const Ctl *ctl, float *x, hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(1), dim3(kThreads), 0, st, embed, ctl, x);
  return hipGetLastError();
}

// out = RMSNorm(x) * w with the PRO_NORM prologue's arithmetic (same inverse norm, same products)
__global__ __launch_bounds__(1024) void k_rmsnorm(const float *x, const float *w, int n, float eps, float *out) {
  extern __shared__ __align__(16) char smem[];
  const ActView av = act_view(smem, n);
  ActRegs ar;
  act_load<PRO_NORM>(x, w, n, ar);
  act_build<PRO_NORM>(ar, eps, n, av);
  const float inv = av.red[0];
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * inv * w[i];
}
hipError_t launch_rmsnorm(const float *x, const float *w, int n, float eps, float *out, hipStream_t st) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(1024), mv_lds_bytes(n, 16, 0), st, x, w, n, eps, out);
  return hipGetLastError();
}

// ------------------------------------------------------------------ decode attention (split-K over the context)
// grid (kv group g, split s), 8 waves.  The number of active splits follows the context: while every wave needs at
// most one 32-position block (T <= 256) one workgroup per kv group does everything and no cross-workgroup merge is
// needed; beyond that S_eff = min(grid.y, ceil(T / 64)) splits.  Split s takes positions [s T / S_eff, (s + 1) T /
// S_eff); the waves take contiguous runs of whole blocks, streamed straight from HBM with the next block's loads in
// flight.
// The queries arrive rotated and the current position's k / v rows are already in the cache: the q / k / v matvec's
// epilogue applies RoPE and writes the fp16 rows (EPI_STORE with MvArgs::rope / cache).
// Per wave (MFMA, see attn_split): scores S^T = K q^T, an online softmax per head, values O^T += V^T P^T; the wave
// partials merge in LDS; with several splits the last one to finish (a per-group counter, which that workgroup
// resets) merges the split partials in split order - the merge of model_llama.cpp:160-165:
// M = max m, L = sum l e^(m - M), out = sum o e^(m - M) * (1 / L).
constexpr int kAttnMaxSplits = 64, kAttnParMerge = 16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// the waves of a split -> its [m, l, o]: S == 1 writes the normalised heads to a.att, otherwise the unnormalised
// output and (max, sum) to a.part (waves 0 .. nact - 1 hold positions; ored rows HS floats apart)
// S == 1 with an Epi other than AttnNoEpi: epi(j, i, v) takes the normalised dims i .. i + 3 of head j instead of
// the store (thread e takes column e: REP * HD / 4 threads, whole 32-lane groups per 128 columns)
struct AttnNoEpi { __device__ void operator()(int, int, float4) const {} };
template <int HD, int REP, int NW, int HS, typename Epi = AttnNoEpi>
__device__ __forceinline__ void attn_wave_merge(const AttnArgs &a, int g, int s, int S, int ys, int nact,
                                                const float (*wm)[REP], const float (*wl)[REP], const float *ored,
                                                int ows, float *lout, const Epi &epi = Epi()) {
  // per head: M = max over the waves, wave factors e^(m_w - M), L = sum l_w e^(m_w - M).  Each wave that sums output
  // columns (thread e takes column e; REP * HD / 4 <= 4 x 64 columns) forms them itself - a wave holds every (wave w,
  // head j) pair, lane 8 w + j (NW, REP <= 8), reduces over w with exchanges of lanes 8, 16 and 32 apart and keeps
  // them in its own LDS copy - so only a wave-level fence, no workgroup barrier, stands before the sums
  static_assert(NW <= 8, "one lane per (wave, head)");
  constexpr int NMW = (REP * HD / 4 + 63) / 64;   // waves with columns
  static_assert(NMW <= NW, "every column has a thread");
  __shared__ float fwv[NMW][NW][REP], mlv[NMW][REP][2];
  const int mwv = threadIdx.x >> 6;
  if (mwv >= NMW) return;
  {
    const int w = (threadIdx.x & 63) >> 3, j = threadIdx.x & 7;
    const bool on = w < nact && j < REP;
    const float mw = on ? wm[w][j] : -INFINITY, lw = on ? wl[w][j] : 0.f;
    float M = mw;
    M = fmaxf(M, xchg8_f(M)); M = pair_max16(M); M = pair_max32(M);
    const float f = mw == -INFINITY ? 0.f : expf(mw - M);
    float L = lw * f;
    L += xchg8_f(L); L = pair_sum16(L); L = pair_sum32(L);
    if (on) fwv[mwv][w][j] = f;
    if (w == 0 && j < REP) { mlv[mwv][j][0] = M; mlv[mwv][j][1] = L; }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // 4 dims per thread: float4 reads of the padded rows, one 16-byte store
  {
    const int e = threadIdx.x;
    if (e >= REP * HD / 4) return;
    const int j = e / (HD / 4), i = 4 * (e % (HD / 4));
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int w = 0; w < nact; w++) {
      const float f = fwv[mwv][w][j];
      const float4 x = *(const float4 *)(ored + w * ows + j * HS + i);
      O.x = __builtin_fmaf(f, x.x, O.x); O.y = __builtin_fmaf(f, x.y, O.y);
      O.z = __builtin_fmaf(f, x.z, O.z); O.w = __builtin_fmaf(f, x.w, O.w);
    }
    const float M = mlv[mwv][j][0], L = mlv[mwv][j][1];
    if (S == 1) {
      const float li = 1.f / L;
      const float4 y = make_float4(O.x * li, O.y * li, O.z * li, O.w * li);
      if constexpr (!std::is_same<Epi, AttnNoEpi>::value) {
        epi(j, i, y);
      } else {
        float *dst = lout ? lout + j * HD + i : a.att + (size_t)(g * REP + j) * HD + i;
        *(float4 *)dst = y;
      }
    } else {
      // coherent (sc1) stores: the merging workgroup may sit on another XCD, and this avoids an L2 writeback; the
      // caller's s_waitcnt vmcnt(0) before the arrival counter covers them.
      // Layout: unnormalised outputs [nh][splits][HD], then (max, sum) pairs [nh][splits][2]
      const size_t hs = (size_t)(g * REP + j) * ys + s;
      if (i == 0) {
        float *ml = a.part + (size_t)a.nh * ys * HD + 2 * hs;
        __hip_atomic_store(ml, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ml + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      const f32x4 v = {O.x, O.y, O.z, O.w};
      asm volatile("global_store_dwordx4 %0, %1, off sc1" ::"v"(a.part + hs * HD + i), "v"(v) : "memory");
    }
  }
}

// Split s of S of kv group g (ys = the partial buffer's split stride).  Each wave streams its positions in 32-position
// blocks with the next block's K and V loads in flight (K in two register sets, alternating):
//   scores  S^T[p][h] = K[p] . q[h] on v_mfma_f32_16x16x32_f16: A = K rows as stored (exact fp16, loaded straight
//           from the cache in the A layout), B = q^T with the group's REP heads as columns; q (fp32, RoPE applied)
//           enters as hi + lo halves (hi = f16(q), lo = f16(q - hi)) - two MFMAs, exact products, fp32 sums;
//           scaled by 1/sqrt(hd) like attend() (model_llama.cpp:137-146);
//   softmax online per head column: lane l holds head l % 16 at positions 4 (l / 16) + i of each 16-row tile;
//   values  O^T[d][h] += V^T[d][p] P^T[p][h]; V lands in a per-wave LDS tile as stored (positions x dims) and the
//           A operand comes out of it transposed by the LDS read; P (hi + lo halves) stays in registers: the C layout
//           of the two score tiles is the B layout once the k index runs over positions {4 (l / 16) + i} and
//           {16 + 4 (l / 16) + i}.
constexpr int kAttnMfWaves = 8, kAttnMfBlk = 32;
template <int HD>
struct MfK {   // K of one 32-position block in the A layout: [2 tiles][HD / 32] 16-byte pieces
  static constexpr int KS = HD / 32;
  u32x4 k[2][KS];
};
// rows at or past te (the cache allocation) read row te - 1 instead
template <int HD>
__device__ __forceinline__ void mf_load_k(const uint16_t *kc, int kvd, int g, int tb, int te, int lane, MfK<HD> &b) {
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int mt = 0; mt < 2; mt++) {
    const int t = tb + 16 * mt + lr, tc = t < te ? t : te - 1;
#pragma unroll
    for (int s = 0; s < MfK<HD>::KS; s++) b.k[mt][s] = *(const u32x4 *)(kc + (size_t)tc * kvd + g * HD + 32 * s + 8 * lg);
  }
}
// V of one block goes to LDS as stored - [32 positions][HD] fp16, rows of HD * 2 bytes - by direct-to-LDS loads (no
// registers), and the PV product reads its A fragments (V^T: dims x positions) with ds_read_b64_tr_b16.  The 16-byte
// segment c of row p sits at segment c ^ vswz(p), so the 8 rows of a 32-lane transpose read (positions 4 lg + r / 4
// over two lane groups) cover all 64 banks: 2 (p & 7) at 256-byte rows, 2 ((p >> 1) & 3) at 128-byte rows (the row's
// parity picks the bank half)
template <int HD>
__device__ __forceinline__ int vswz(int p) { return HD == 128 ? 2 * (p & 7) : 2 * ((p >> 1) & 3); }
// rows at or past te (the cache allocation) read row te - 1 instead.  buf: the wave's 32 x HD tile (wave-uniform)
template <int HD>
__device__ __forceinline__ void mf_dma_v(const uint16_t *vc, int kvd, int g, int tb, int te, int lane, uint16_t *buf) {
  constexpr int SEG = HD / 8, RPI = 64 / SEG;   // 16-byte segments per row; rows per 1 KiB load instruction
  const int r = lane / SEG, sp = lane % SEG;
#pragma unroll
  for (int q = 0; q < kAttnMfBlk / RPI; q++) {
    const int p = q * RPI + r, t = tb + p, tc = t < te ? t : te - 1;
    // lane l writes bytes [16 l, 16 l + 16) of the instruction's 1 KiB: row q RPI + r, segment position sp
    dma16(vc + (size_t)tc * kvd + g * HD + 8 * (sp ^ vswz<HD>(p)), buf + q * RPI * HD);
  }
}

// lout: with S == 1, the normalised heads go to this LDS array [REP][HD] instead of a.att; mid() runs once the waves'
// partials are in LDS, before their merge (the block loop's registers are free by then).  ONE: S == 1 is known before
// the position is: each wave's first block (positions 32 w ..) is loaded before ctl->pos arrives.
struct AttnNoMid { __device__ void operator()() const {} };
template <int HD, int REP, bool ONE = false, typename Mid = AttnNoMid, typename Epi = AttnNoEpi>
__device__ void attn_split(const AttnArgs &a, int g, int s, int S, int ys, float *lout = nullptr, const Mid &mid = Mid(),
                           const Epi &epi = Epi()) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  typedef float f4 __attribute__((ext_vector_type(4)));
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef short s8 __attribute__((ext_vector_type(8)));
  typedef __attribute__((address_space(3))) s4 lds_s4;
  constexpr int NW = kAttnMfWaves, KS = MfK<HD>::KS, DT = HD / 16;
  constexpr int QS = HD + 4;
  __shared__ float wm[NW][REP], wl[NW][REP];
  __shared__ __align__(16) uint16_t vt[NW][kAttnMfBlk * HD];   // each wave's V block as stored (swizzled segments)
  // a wave's (unnormalised) output rows go into its own V tile once its block loop is done: [REP][QS] floats
  static_assert(REP * QS * 4 <= kAttnMfBlk * HD * 2, "the output rows fit in the wave's V tile");
  constexpr int OWS = kAttnMfBlk * HD / 2;   // floats between two waves' output rows
  const int kvd = a.nkv * HD;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
  uint16_t *vw = vt[wave];
  MfK<HD> ka, kb;
  const int pos_s = ctl_pos_issue(a.ctl);
  // positions past the context or the split are loaded from rows below a.ctx (in the allocation) and masked: their
  // scores become -inf and their V rows zero.  ONE: the first a.early waves (all when 0) load their first block now;
  // the host sets a.early to the blocks the step's context can need, so no wave loads a block past it
  const bool early = ONE && (a.early <= 0 || wave < a.early);
  if (early) {
    mf_dma_v<HD>(a.vc, kvd, g, kAttnMfBlk * wave, a.ctx, lane, vw);
    mf_load_k<HD>(a.kc, kvd, g, kAttnMfBlk * wave, a.ctx, lane, ka);
  }
  // q^T fragments straight from the q / k / v epilogue's fp16 planes (hi = f16(q), lo = f16(q - hi)): lane holds head
  // lr (zero past REP), dims 32 k + 8 lg + 0..7
  h8 qh[KS], ql[KS];
  {
    // only the lanes of the group's REP heads load (the other columns are zero): 16 / REP times fewer requests
    const uint16_t *qp = a.q16 + (size_t)(g * REP + (lr < REP ? lr : 0)) * HD + 8 * lg;
#pragma unroll
    for (int k = 0; k < KS; k++) {
      u32x4 h = (u32x4){0u, 0u, 0u, 0u}, lo = h;
      if (lr < REP) { h = *(const u32x4 *)(qp + 32 * k); lo = *(const u32x4 *)(qp + (size_t)a.nh * HD + 32 * k); }
      qh[k] = __builtin_bit_cast(h8, h); ql[k] = __builtin_bit_cast(h8, lo);
    }
  }
  const int pos = ctl_pos_wait(pos_s), T = pos + 1;
  const int t0 = (int)((int64_t)s * T / S), t1 = (int)((int64_t)(s + 1) * T / S);
  // wave w takes blocks w, w + NW, ... of the split's 32-position blocks (waves without a block idle)
  const int nblk = (t1 - t0 + kAttnMfBlk - 1) / kAttnMfBlk, nact = min(nblk, NW);
  if (!early && wave < nblk) {
    mf_dma_v<HD>(a.vc, kvd, g, t0 + kAttnMfBlk * wave, a.ctx, lane, vw);
    mf_load_k<HD>(a.kc, kvd, g, t0 + kAttnMfBlk * wave, a.ctx, lane, ka);
  }
  const float scl = 1.f / sqrtf((float)HD);
  f4 o[DT];
#pragma unroll
  for (int d = 0; d < DT; d++) o[d] = (f4){0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  // one block: wait for its V (in LDS) and K (registers), read the V^T fragments, issue the next block's loads into
  // the same LDS tile and the other K set, then the scores, the softmax and the PV product
  auto block = [&](MfK<HD> &kcur, MfK<HD> &knxt, int tb) {
    // the block's K registers and V tile: its K loads were issued after the V tile's, so the compiler's wait for K
    // (forced here by a use of every K register, which it sees; an s_waitcnt in asm it would not) covers V too
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
      for (int k = 0; k < KS; k++) asm volatile("" ::"v"(kcur.k[mt][k]));
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (tb + kAttnMfBlk > t1) {
      // rows past the split become zeros: their probabilities are 0, but 0 x a stale NaN would not be
      constexpr int SEG = HD / 8, RPI = 64 / SEG;
#pragma unroll
      for (int q = 0; q < kAttnMfBlk / RPI; q++) {
        const int p = q * RPI + lane / SEG;
        if (tb + p >= t1) *(u32x4 *)(vw + p * HD + 8 * (lane % SEG)) = (u32x4){0u, 0u, 0u, 0u};
      }
    }
    // V^T fragment of tile d: dim 16 d + lr, positions 4 lg + 0..3 and 16 + 4 lg + 0..3 (the k order of ph / pl).
    // ds_read_b64_tr_b16 hands lane i of a 16-lane group element i % 4 of the 4 values that lane 4 j + i / 4
    // addresses, as its element j: so source lane r addresses row 4 lg + r / 4 (+ 16), dims 16 d + 4 (r % 4) .. + 3
    h8 vf[DT];
    {
      const int pr = 4 * lg + (lr >> 2), dq = 4 * (lr & 3), sw = vswz<HD>(pr);   // rows pr and pr + 16: same swizzle
#pragma unroll
      for (int d = 0; d < DT; d++) {
        const int off = 8 * (((16 * d + dq) >> 3) ^ sw) + (dq & 4);
        const s4 x0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(vw + pr * HD + off));
        const s4 x1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)(vw + (pr + 16) * HD + off));
        vf[d] = __builtin_bit_cast(h8, (s8)__builtin_shufflevector(x0, x1, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
    if (tb + NW * kAttnMfBlk < t1) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the tile's reads are done before the DMA rewrites it
      mf_dma_v<HD>(a.vc, kvd, g, tb + NW * kAttnMfBlk, a.ctx, lane, vw);
      mf_load_k<HD>(a.kc, kvd, g, tb + NW * kAttnMfBlk, a.ctx, lane, knxt);
    }
    // scores of the two 16-position tiles
    f4 sc[2];
#pragma unroll
    for (int mt = 0; mt < 2; mt++) {
      sc[mt] = (f4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < KS; k++) {
        const h8 kf = __builtin_bit_cast(h8, kcur.k[mt][k]);
        sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[k], sc[mt], 0, 0, 0);
        sc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[k], sc[mt], 0, 0, 0);
      }
    }
    // online softmax of head lr over this block's positions
    float sv[8], bm = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float x = tb + 16 * mt + 4 * lg + i < t1 ? sc[mt][i] * scl : -INFINITY;
        sv[4 * mt + i] = x; bm = fmaxf(bm, x);
      }
    bm = pair_max16(bm);
    bm = pair_max32(bm);
    // e^(x - mn) as the hardware exp2 of (x - mn) log2(e) (v_exp_f32, one instruction against ~20 for expf; the
    // default order's attention is held to the logit tolerance - the reference-order kernels keep glibc's expf)
    constexpr float kL2E = 1.44269504088896340736f;
    const float mn = fmaxf(m, bm);
    const float corr = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m - mn) * kL2E);
    float rs = 0.f;
    h8 ph, pl;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float pv = sv[j] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((sv[j] - mn) * kL2E);
      rs += pv;
      const _Float16 h = (_Float16)pv;
      ph[j] = h; pl[j] = (_Float16)(pv - (float)h);
    }
    rs = pair_sum16(rs);
    rs = pair_sum32(rs);
    l = l * corr + rs;
    m = mn;
#pragma unroll
    for (int d = 0; d < DT; d++) {
      o[d] *= corr;
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[d], ph, o[d], 0, 0, 0);
      o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf[d], pl, o[d], 0, 0, 0);
    }
  };
  for (int tb = t0 + kAttnMfBlk * wave; tb < t1; tb += 2 * NW * kAttnMfBlk) {
    block(ka, kb, tb);
    if (tb + NW * kAttnMfBlk >= t1) break;
    block(kb, ka, tb + NW * kAttnMfBlk);
  }
  // a wave without a block may still have its early loads in flight: they land before its tile is reused
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // this wave's (m, l, o) -> LDS (its own V tile, free now): lane holds head lr, dims 16 d + 4 lg + i
  float *ored = (float *)&vt[0][0];
  if (lr < REP) {
    if (lg == 0) { wm[wave][lr] = m; wl[wave][lr] = l; }
#pragma unroll
    for (int d = 0; d < DT; d++)
      *(float4 *)(ored + wave * OWS + lr * QS + 16 * d + 4 * lg) = make_float4(o[d][0], o[d][1], o[d][2], o[d][3]);
  }
  mid();
  __syncthreads();
  attn_wave_merge<HD, REP, NW, QS, Epi>(a, g, s, S, ys, nact, wm, wl, ored, OWS, lout, epi);
}

// One workgroup merges every head of group g over S < kAttnParMerge splits, in one round of loads: P threads share
// each (head, 4 dims) column of partials, split c going to thread c mod P, and issue all their coherent 16-byte loads
// at once, together with wave j's loads of head j's (m, l) pairs (one split per lane); wave j then forms head j's
// factors e^(m_c - M) and 1 / L, and the column sums go through LDS.
template <int HD, int REP, int NW>
__device__ void attn_merge_all(const AttnArgs &a, int g, int S) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  auto cload = [](const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  constexpr int NC = REP * HD / 4;                            // output columns of 4 dims
  constexpr int P = NW * 64 / NC >= 4 ? 4 : (NW * 64 / NC >= 2 ? 2 : 1);
  constexpr int K = (kAttnParMerge - 1 + P - 1) / P;          // loads per thread
  __shared__ float fw[REP][kAttnParMerge], linv[REP];
  __shared__ float4 opart[NW * 64];
  const float *ml = a.part + (size_t)a.nh * gridDim.y * HD + 2 * (size_t)g * REP * gridDim.y;
  const int e = threadIdx.x % NC, part = threadIdx.x / NC;
  const int j = e / (HD / 4), i4 = e % (HD / 4);
  f32x4 v[K];
  if (part < P) {
    const float4 *ph = (const float4 *)(a.part + ((size_t)(g * REP + j) * gridDim.y) * HD) + i4;
#pragma unroll
    for (int k = 0; k < K; k++) {   // clamped in range; unused ones are not summed
      const int c = part + k * P < S ? part + k * P : 0;
      asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v[k]) : "v"(ph + (size_t)c * (HD / 4)));
    }
  }
  if (wave < REP) {
    const bool on = lane < S;
    const float *mp = ml + 2 * ((size_t)wave * gridDim.y + lane);
    const float2 mv = on ? make_float2(cload(mp), cload(mp + 1)) : make_float2(-INFINITY, 0.f);
    const float M = wave_max(mv.x);
    const float f = on && mv.x != -INFINITY ? expf(mv.x - M) : 0.f;
    const float L = wave_sum(mv.y * f);
    if (on) fw[wave][lane] = f;
    if (lane == 0) linv[wave] = 1.f / L;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int k = 0; k < K; k++) asm volatile("" : "+v"(v[k]));   // the values are used only after the wait
  __syncthreads();
  float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
  if (part < P) {
#pragma unroll
    for (int k = 0; k < K; k++)
      if (part + k * P < S) {
        const float f = fw[j][part + k * P];
        O.x = __builtin_fmaf(f, v[k][0], O.x); O.y = __builtin_fmaf(f, v[k][1], O.y);
        O.z = __builtin_fmaf(f, v[k][2], O.z); O.w = __builtin_fmaf(f, v[k][3], O.w);
      }
    opart[threadIdx.x] = O;
  }
  __syncthreads();
  if (threadIdx.x < NC) {
    for (int q = 1; q < P; q++) {
      const float4 t = opart[q * NC + threadIdx.x];
      O.x += t.x; O.y += t.y; O.z += t.z; O.w += t.w;
    }
    const float li = linv[j];
    *(float4 *)(a.att + (size_t)(g * REP + j) * HD + 4 * i4) = make_float4(O.x * li, O.y * li, O.z * li, O.w * li);
  }
}

// Merger r of MG merges heads r, r + MG, ... of group g over the S splits.  Per head: thread t takes column t % (HD / 4)
// of 4 dims and the splits t / (HD / 4) + (NW * 256 / HD) k, all its loads issued at once; wave 0 also reduces M and L
// over the splits (one split per lane).  late: the wait for the other splits ran out (the outputs are then NaN).
template <int HD, int REP, int NW>
__device__ void attn_merge_heads(const AttnArgs &a, int g, int S, int r, int MG, bool late, int ys) {
  constexpr int NCOL = HD / 4, NGRP = NW * 64 / NCOL, PER = (kAttnMaxSplits + NGRP - 1) / NGRP;
  __shared__ float Ms, Linv;
  __shared__ float4 opart[NGRP][NCOL];
  const int col = threadIdx.x % NCOL, grp = threadIdx.x / NCOL;
  const float *mlb = a.part + (size_t)a.nh * ys * HD;
  for (int j = r; j < REP; j += MG) {
    const size_t hs0 = (size_t)(g * REP + j) * ys;
    f32x4 v[PER];
    float2 mlk[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) {   // coherent loads (clamped in range; unused ones are not summed)
      const int c = grp + NGRP * k < S ? grp + NGRP * k : 0;
      const float4 *ph = (const float4 *)(a.part + (hs0 + c) * HD) + col;
      asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v[k]) : "v"(ph));
      mlk[k] = make_float2(__hip_atomic_load(mlb + 2 * (hs0 + c), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                           __hip_atomic_load(mlb + 2 * (hs0 + c) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
    if (threadIdx.x < 64) {
      const bool on = threadIdx.x < S;
      const float m = on ? __hip_atomic_load(mlb + 2 * (hs0 + threadIdx.x), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -INFINITY;
      const float l = on ? __hip_atomic_load(mlb + 2 * (hs0 + threadIdx.x) + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0.f;
      const float M = wave_max(m);
      const float L = wave_sum(on && m != -INFINITY ? l * expf(m - M) : 0.f);
      if (threadIdx.x == 0) { Ms = M; Linv = 1.f / L; }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int k = 0; k < PER; k++) asm volatile("" : "+v"(v[k]));   // the values are used only after the wait
    __syncthreads();
    const float M = Ms;
    float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < PER; k++)
      if (grp + NGRP * k < S) {
        const float f = mlk[k].x == -INFINITY ? 0.f : expf(mlk[k].x - M);
        O.x = __builtin_fmaf(f, v[k][0], O.x); O.y = __builtin_fmaf(f, v[k][1], O.y);
        O.z = __builtin_fmaf(f, v[k][2], O.z); O.w = __builtin_fmaf(f, v[k][3], O.w);
      }
    opart[grp][col] = O;
    __syncthreads();
    if (threadIdx.x < NCOL) {
      for (int q = 1; q < NGRP; q++) {
        const float4 t = opart[q][threadIdx.x];
        O.x += t.x; O.y += t.y; O.z += t.z; O.w += t.w;
      }
      const float li = late ? __builtin_nanf("") : Linv;   // a wait that ran out leaves NaN, never stale values
      *(float4 *)(a.att + (size_t)(g * REP + j) * HD + 4 * threadIdx.x) = make_float4(O.x * li, O.y * li, O.z * li, O.w * li);
    }
    __syncthreads();
  }
}

template <int HD, int REP>
__global__ __launch_bounds__(kAttnMfWaves * 64) void k_attention(AttnArgs a) {
  constexpr int NW = kAttnMfWaves;
  const int pos = a.ctl->pos, T = pos + 1, g = blockIdx.x, s = blockIdx.y;
  // one workgroup per kv group while the group's K and V are at most 64 KiB (a CU streams ~55 GB/s: 128 positions at
  // head dim 128, 256 at 64); beyond that up to 64 splits of >= 64 positions
  const int smax = a.single_max > 0 ? a.single_max : kAttnMfBlk * NW * 64 / HD, sp = a.split_pos > 0 ? a.split_pos : 64;
  const int S = T <= smax ? 1 : min((int)gridDim.y, (T + sp - 1) / sp);
  if (s >= S) return;
  uint64_t st0 = 0, st1 = 0, st2 = 0;   // measurement (a.stamps): start, partials stored, rank known
  if (a.stamps) st0 = __builtin_amdgcn_s_memrealtime();
  attn_split<HD, REP>(a, g, s, S, gridDim.y);
  if (S == 1 || (a.merge_sep && S >= a.merge_sep)) return;   // merge_sep: k_attn_merge merges (the next launch)
  // this thread's coherent stores have completed before the workgroup's counter bump
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (a.stamps) st1 = __builtin_amdgcn_s_memrealtime();
  auto stamp = [&](int merger) {
    if (a.stamps && threadIdx.x == 0) {
      uint64_t *o = a.stamps + 5 * ((size_t)blockIdx.y * gridDim.x + blockIdx.x);
      o[0] = st0; o[1] = st1; o[2] = st2; o[3] = __builtin_amdgcn_s_memrealtime(); o[4] = merger;
    }
  };
  // (With AttnArgs::merge_sep - the default from 16 splits - the splits returned above and k_attn_merge merges.)
  // The last MG splits to arrive merge the S partials of the group's heads (model_llama.cpp:160-165: M = max m_c,
  // f_c = exp(m_c - M), L = sum l_c f_c, O = sum f_c o_c / L): from kAttnParMerge splits up MG = min(REP, S), head j
  // by merger j % MG, each head's loads in one round; below, the merge is short and the last arrival does it alone
  // (MG = 1, all heads in one round of loads).  Counter
  // a.counters[g] counts arrivals, a.counters[nkv + g] mergers done waiting; the last of those resets both for the next
  // launch (a lone merger resets the arrivals at once).  A merger waits for the arrivals behind it: those splits are already resident or wait only for workgroups
  // that finish without waiting (at most nh mergers wait at any time), and the wait is bounded.
  __shared__ int rank, late;
  int *arrive = a.counters + g, *done = a.counters + a.nkv + g;
  const int MG = S >= kAttnParMerge ? min(REP, S) : 1;
  if (threadIdx.x == 0) {
    const int r = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - (S - MG);
    if (MG == 1 && r == 0) __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int spins = 0;
    const int lim = a.spin_limit > 0 ? a.spin_limit : (1 << 22);
    if (r >= 0 && r < MG - 1)
      while (__hip_atomic_load(arrive, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < S && ++spins < lim)
        __builtin_amdgcn_s_sleep(1);
    rank = r < 0 ? -1 : r;
    late = spins >= lim || (a.force_late && r >= 0 && r < MG - 1);
    if (late && a.status) *(volatile int *)a.status = 1;   // the step's outputs are invalid: the host raises an error
  }
  __syncthreads();
  if (a.stamps) st2 = __builtin_amdgcn_s_memrealtime();
  const int r = rank;
  if (r < 0) { stamp(0); return; }
  // The partials were written through to memory by other workgroups before their counter bumps; they are read with
  // coherent loads (no acquire fence: that is an L2 invalidate, far slower).
  if (S < kAttnParMerge) {
    attn_merge_all<HD, REP, NW>(a, g, S);
    stamp(1);
    return;
  }
  // this merger no longer reads the arrivals; the round trip overlaps the merge
  const int d = threadIdx.x == 0 ? __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
  attn_merge_heads<HD, REP, NW>(a, g, S, r, MG, late, gridDim.y);
  if (threadIdx.x == 0 && d == MG - 1) {
    __hip_atomic_store(done, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  stamp(1);
}

// The merge of k_attention's splits as a launch of its own (AttnArgs::merge_sep: contexts of at least merge_sep
// splits): workgroup (g, j) merges head j of group g over the S splits the previous launch stored - the kernel
// boundary orders the partials before their loads, in place of the arrival counters and the mergers' wait.
template <int HD, int REP>
__global__ __launch_bounds__(kAttnMfWaves * 64) void k_attn_merge(AttnArgs a) {
  const int pos = a.ctl->pos, T = pos + 1;
  const int smax = a.single_max > 0 ? a.single_max : kAttnMfBlk * kAttnMfWaves * 64 / HD, sp = a.split_pos > 0 ? a.split_pos : 64;
  const int S = T <= smax ? 1 : min(a.max_chunks, (T + sp - 1) / sp);
  if (S < a.merge_sep || S == 1) return;   // k_attention merged in-kernel (or had one split)
  attn_merge_heads<HD, REP, kAttnMfWaves>(a, blockIdx.x, S, blockIdx.y, REP, false, a.max_chunks);
}

int attn_long_merge_min(int hd, int single_max, int split_pos, int max_chunks, int min_splits) {
  const int smax = single_max > 0 ? single_max : kAttnMfBlk * kAttnMfWaves * 64 / hd, sp = split_pos > 0 ? split_pos : 64;
  if (min_splits < 2 || max_chunks < min_splits) return 0;
  return std::max(smax + 1, (min_splits - 1) * sp + 1);   // S = min(max_chunks, ceil(T / sp)) >= min_splits
}

hipError_t launch_attention(const AttnArgs &a, hipStream_t st) {
  if (a.nh % a.nkv || a.nh / a.nkv > 8 || a.max_chunks < 1 || a.max_chunks > kAttnMaxSplits) return hipErrorInvalidValue;
  const dim3 grid(a.nkv, a.max_chunks);
  const int rep = a.nh / a.nkv;
#define QPH_ATT(HD, R)                                                                                              \
  if (a.hd == HD && rep == R) {                                                                                     \
    hipLaunchKernelGGL((k_attention<HD, R>), grid, dim3(kAttnMfWaves * 64), 0, st, a);                              \
    if (a.merge_sep) hipLaunchKernelGGL((k_attn_merge<HD, R>), dim3(a.nkv, R), dim3(kAttnMfWaves * 64), 0, st, a);   \
    return hipGetLastError();                                                                                       \
  }
  QPH_ATT(64, 1) QPH_ATT(64, 2) QPH_ATT(64, 3) QPH_ATT(64, 4) QPH_ATT(64, 5) QPH_ATT(64, 6) QPH_ATT(64, 7) QPH_ATT(64, 8)
  QPH_ATT(128, 1) QPH_ATT(128, 2) QPH_ATT(128, 3) QPH_ATT(128, 4) QPH_ATT(128, 5) QPH_ATT(128, 6) QPH_ATT(128, 7) QPH_ATT(128, 8)
#undef QPH_ATT
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------------ decode attention fused with the wo product
// Workgroup (kv group g, row chunk c) of grid (nkv, rc), 8 waves:
//   1. computes the group's attention over the whole context with attn_split (one split, output to LDS);
//   2. once the waves' partials are in LDS (before their merge) issues the loads of its wo tile - rows [c R, c R + R)
//      x the group's columns [g CG, g CG + CG), CG = REP * HD - into registers (NL 16-byte pieces per thread; piece
//      p = thread + 512 i is row p / (CG / 16), bytes 16 (p % (CG / 16)) of the row's slice);
//   3. quantises the REP * HD outputs with quant_rows' arithmetic, every 128 columns one block (act_build's
//      expressions: the same planes and scales as the wo matvec's prologue builds from att for these blocks);
//   4. forms the exact int32 block sums (the matvec's two-plane dot products and 8-lane sums) and, one thread per row,
//      rows_q8's fp32 chain over the group's blocks, acc = fma(bs[b], sum[b], acc) (kernels_x86.cpp:57-69), times the
//      row scale: part[g][row].  No workgroup waits for another; the next kernel sums the groups' parts.
constexpr int kAwoMaxGroups = 8;    // kv groups the last arrival adds up (AwoArgs::counters)
template <int HD, int REP, int NL>
__global__ __launch_bounds__(kAttnMfWaves * 64) void k_attn_wo(AttnArgs a, AwoArgs w) {
  constexpr int NT = kAttnMfWaves * 64, CG = REP * HD, PPR = CG / 16, NBG = CG / kQB;
  static_assert(CG % kQB == 0, "a group's columns are whole quantisation blocks");
  __shared__ __align__(16) int8_t xh[CG];
  __shared__ __align__(16) uint8_t xl[CG];
  __shared__ float bsl[NBG];
  __shared__ int lsl[NBG];
  __shared__ int isl[NT * NL / 8];   // block sums [row in tile][NBG]
  const int g = blockIdx.x, c = blockIdx.y, d = w.wo.rows, cols = w.wo.cols;
  const int r0 = c * w.R, R = min(w.R, d - r0);
  const int8_t *wq = (const int8_t *)w.wo.q + (size_t)g * CG;
  uint64_t t0 = 0, t1 = 0, t2 = 0, tm = 0;
  if (w.stamps) t0 = __builtin_amdgcn_s_memrealtime();
  uint4 wr[NL];
  // the first row of each thread (threadIdx.x < R): its scale and, for the last arrival, its residual, loaded with the
  // tile so that they are in registers by the epilogue (loaded there, each was a memory round trip on its path)
  const float *wsc = (const float *)w.wo.s;
  float rsc = 0.f, xpre = 0.f;
  auto issue = [&]() {
    if (w.stamps) tm = __builtin_amdgcn_s_memrealtime();
    if ((int)threadIdx.x < R) {
      rsc = wsc[r0 + threadIdx.x];
      if (w.counters) xpre = w.x[r0 + threadIdx.x];   // this launch changes x only in the last arrival, below
    }
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int p = threadIdx.x + NT * i, lr = p / PPR, c16 = p % PPR;
      const int row = lr < R ? r0 + lr : r0;   // past the tile: row r0 (< d: chunks are never empty), not used
      wr[i] = ld16(wq + (size_t)row * cols + 16 * c16);
    }
  };
  // the merge hands each thread 4 normalised dims; a 128-column block is 32 lanes, which quantise it with
  // quant_rows' arithmetic (act_build's expressions: max |v| over the block, isx = 32767 / max, q = rint(v isx),
  // planes hi = q >> 8 and lo = q & 255, the block's sum of lo) straight into the planes the products read
  auto quant = [&](int j, int i, float4 v) {
    const int c0 = j * HD + i, b = c0 / kQB;
    const float m = max32_f(fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    const float isx = m > 0 ? kActMax / m : 0.f;
    const float vv[4] = {v.x, v.y, v.z, v.w};
    uint32_t hh = 0, ll = 0; int ls = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int q = (int)__builtin_rintf(vv[k] * isx);
      hh |= (uint32_t)((q >> 8) & 0xff) << (8 * k);
      ll |= (uint32_t)(q & 0xff) << (8 * k);
      ls += q & 0xff;
    }
    *(uint32_t *)(xh + c0) = hh;
    *(uint32_t *)(xl + c0) = ll;
    ls = sum32_i(ls);
    if ((c0 & (kQB - 1)) == 0) { bsl[b] = m / kActMax; lsl[b] = ls; }
  };
  attn_split<HD, REP, true, decltype(issue), decltype(quant)>(a, g, 0, 1, 1, nullptr, issue, quant);
  if (w.stamps) t1 = __builtin_amdgcn_s_memrealtime();
  __syncthreads();
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    const int p = threadIdx.x + NT * i, lr = p / PPR, c16 = p % PPR;
    const uint4 h = *(const uint4 *)(xh + 16 * c16), l = *(const uint4 *)(xl + 16 * c16);
    const uint4 ww = wr[i];
    int A = __builtin_amdgcn_sdot4((int)ww.x, (int)h.x, 0, false);
    A = __builtin_amdgcn_sdot4((int)ww.y, (int)h.y, A, false);
    A = __builtin_amdgcn_sdot4((int)ww.z, (int)h.z, A, false);
    A = __builtin_amdgcn_sdot4((int)ww.w, (int)h.w, A, false);
    uint32_t B = __builtin_amdgcn_udot4(ww.x ^ 0x80808080u, l.x, 0u, false);
    B = __builtin_amdgcn_udot4(ww.y ^ 0x80808080u, l.y, B, false);
    B = __builtin_amdgcn_udot4(ww.z ^ 0x80808080u, l.z, B, false);
    B = __builtin_amdgcn_udot4(ww.w ^ 0x80808080u, l.w, B, false);
    const int sum = sum8_i(A * 256 + (int)B);
    if ((lane & 7) == 0 && lr < R) isl[lr * NBG + (c16 >> 3)] = sum - 128 * lsl[c16 >> 3];
  }
  __syncthreads();
  if (w.stamps) t2 = __builtin_amdgcn_s_memrealtime();
  for (int lr = threadIdx.x; lr < R; lr += NT) {
    float ch = 0.f;
#pragma unroll
    for (int b = 0; b < NBG; b++) ch = __builtin_fmaf(bsl[b], (float)isl[lr * NBG + b], ch);
    const int row = r0 + lr;
    const float y = ch * (lr == (int)threadIdx.x ? rsc : wsc[row]);
    float *dst = w.part + (size_t)g * d + row;
    if (w.counters) asm volatile("global_store_dword %0, %1, off sc1" ::"v"(dst), "v"(y) : "memory");
    else *dst = y;
  }
  if (w.counters) {
    // the last of the nkv groups to arrive adds their parts to the residual stream:
    // x[row] += ((p_0 + p_1) + ...) + p_{nkv-1}.  The parts went through to memory (coherent stores, drained before the
    // counter bump) and are read back with coherent loads; the last arrival resets the counter for the next launch.
    // With one row per thread (R <= NT) the arrivals are per wave - counter [c][wave] for rows [64 wave, 64 wave + 64)
    // of the chunk - so no workgroup barrier sits between a wave's stores and its hand-off; else per workgroup.
    auto add_parts = [&](int lr, float xp) {
      const int row = r0 + lr, ng = (int)gridDim.x;
      float p[kAwoMaxGroups];
#pragma unroll
      for (int j = 0; j < kAwoMaxGroups; j++) {   // clamped in range; unused ones are not summed
        const float *src = w.part + (size_t)(j < ng ? j : 0) * d + row;
        asm volatile("global_load_dword %0, %1, off sc1" : "=v"(p[j]) : "v"(src));
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int j = 0; j < kAwoMaxGroups; j++) asm volatile("" : "+v"(p[j]));   // used only after the wait
      float y = p[0];
#pragma unroll
      for (int j = 1; j < kAwoMaxGroups; j++)
        if (j < ng) y += p[j];
      w.x[row] = xp + y;
    };
    if (R <= NT) {
      const int wv = threadIdx.x >> 6;
      if (64 * wv < R) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's part stores have completed
        int *cnt = w.counters + c * kAttnMfWaves + wv;
        int n = 0;
        if (lane == 0) n = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        n = __builtin_amdgcn_readfirstlane(n);
        if (n == (int)gridDim.x - 1) {
          if (lane == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if ((int)threadIdx.x < R) add_parts(threadIdx.x, xpre);
        }
      }
    } else {
      __shared__ int last;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (threadIdx.x == 0) {
        int *cnt = w.counters + c * kAttnMfWaves;
        const int n = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = n == (int)gridDim.x - 1;
        if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (last)
        for (int lr = threadIdx.x; lr < R; lr += NT) add_parts(lr, lr == (int)threadIdx.x ? xpre : w.x[r0 + lr]);
    }
  }
  if (w.stamps && threadIdx.x == 0) {
    uint64_t *o = w.stamps + 5 * (blockIdx.y * gridDim.x + blockIdx.x);
    o[0] = t0; o[1] = tm; o[2] = t1; o[3] = t2; o[4] = __builtin_amdgcn_s_memrealtime();
  }
}

bool attn_wo_fits(int hd, int nh, int nkv, const DMat &wo, int cus, int *rc, int *nl) {
  if (wo.kind != MK_Q8 || nkv > kAwoMaxGroups || nh % nkv || (hd != 64 && hd != 128)) return false;
  const int rep = nh / nkv, cg = rep * hd;
  if (cg % kQB || rep > 8 || wo.cols != nh * hd || wo.rows < 1) return false;
  // about one workgroup per CU; every chunk non-empty (rc = ceil(rows / R))
  for (int c = std::max(1, std::min(wo.rows, cus / nkv)); c <= wo.rows; c++) {
    const int R = (wo.rows + c - 1) / c, pieces = R * (cg / 16), need = (pieces + kAttnMfWaves * 64 - 1) / (kAttnMfWaves * 64);
    if (need <= 16) { *rc = (wo.rows + R - 1) / R; *nl = need <= 4 ? 4 : need <= 8 ? 8 : 16; return true; }
  }
  return false;
}

hipError_t launch_attn_wo(const AttnArgs &a, AwoArgs w, hipStream_t st) {
  int rc = 0, nl = 0;
  if (!attn_wo_fits(a.hd, a.nh, a.nkv, w.wo, g_mv_config.cus, &rc, &nl)) return hipErrorInvalidValue;
  w.R = (w.wo.rows + rc - 1) / rc;
  if ((size_t)(rc - 1) * w.R >= (size_t)w.wo.rows) return hipErrorInvalidValue;
  const dim3 grid(a.nkv, rc);
  const int rep = a.nh / a.nkv;
#define QPH_AWO(HD, R, NL)                                                                                          \
  if (a.hd == HD && rep == R && nl == NL) {                                                                         \
    hipLaunchKernelGGL((k_attn_wo<HD, R, NL>), grid, dim3(kAttnMfWaves * 64), 0, st, a, w);                         \
    return hipGetLastError();                                                                                       \
  }
#define QPH_AWO3(HD, R) QPH_AWO(HD, R, 4) QPH_AWO(HD, R, 8) QPH_AWO(HD, R, 16)
  QPH_AWO3(64, 2) QPH_AWO3(64, 4) QPH_AWO3(64, 6) QPH_AWO3(64, 8)
  QPH_AWO3(128, 1) QPH_AWO3(128, 2) QPH_AWO3(128, 3) QPH_AWO3(128, 4) QPH_AWO3(128, 5) QPH_AWO3(128, 6) QPH_AWO3(128, 7) QPH_AWO3(128, 8)
#undef QPH_AWO3
#undef QPH_AWO
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------------ every group's attention + whole wo rows
// For models whose kv groups are not whole 128-column blocks (C1: 7 heads of 64 per group) at contexts where the
// attention runs one split per group: workgroup c of rc computes every group's attention in turn (attn_split, one
// split, into LDS), quantises the whole attention vector (the wo matvec prologue's blocks), loads wo rows
// [cR, cR + R) whole - issued while the last group's partials merge - and finishes them as the wo matvec does: the
// exact int32 block sums, rows_q8's fp32 chain over all blocks in order (kernels_x86.cpp:57-69), the row scale and
// x[row] += y.  The same arithmetic as k_attention with one split per group followed by the wo matvec, bit for bit;
// the next kernels are unchanged.
constexpr int kAwoRowsMaxCols = 2048, kAwoRowsMaxGroups = 2;
template <int HD, int REP, int NL>
__global__ __launch_bounds__(kAttnMfWaves * 64) void k_attn_wo_rows(AttnArgs a, AwoArgs w) {
  constexpr int NT = kAttnMfWaves * 64;
  __shared__ __align__(16) float ao[kAwoRowsMaxCols];
  __shared__ __align__(16) int8_t xh[kAwoRowsMaxCols];
  __shared__ __align__(16) uint8_t xl[kAwoRowsMaxCols];
  __shared__ float bsl[kAwoRowsMaxCols / kQB];
  __shared__ int lsl[kAwoRowsMaxCols / kQB];
  __shared__ int isl[NT * NL / 8];   // block sums [row in tile][nb]
  const int c = blockIdx.x, d = w.wo.rows, cols = w.wo.cols, nb = cols / kQB, ppr = cols / 16;
  const int r0 = c * w.R, R = min(w.R, d - r0);
  const int8_t *wq = (const int8_t *)w.wo.q;
  uint4 wr[NL];
  auto issue = [&]() {
#pragma unroll
    for (int i = 0; i < NL; i++) {
      const int p = threadIdx.x + NT * i, lr = p / ppr, c16 = p % ppr;
      const int row = lr < R ? r0 + lr : r0;   // past the tile: row r0 (chunks are never empty), not used
      wr[i] = ld16(wq + (size_t)row * cols + 16 * c16);
    }
  };
  bool last = false;
  auto mid = [&]() { if (last) issue(); };   // one attn_split instantiation (its LDS arrays are per instantiation)
  for (int g = 0; g < a.nkv; g++) {
    last = g + 1 == a.nkv;
    attn_split<HD, REP, true>(a, g, 0, 1, 1, ao + g * REP * HD, mid);
    __syncthreads();
  }
  if (threadIdx.x < 8 * nb) {   // eight lanes per block, 16 columns each (act_build's arithmetic)
    const int b = threadIdx.x >> 3, sub = threadIdx.x & 7, c0 = b * kQB + sub * 16;
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const float4 t = *(const float4 *)(ao + c0 + 4 * k);
      v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w;
    }
    float m = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) m = fmaxf(m, fabsf(v[k]));
    m = max8_f(m);
    const float isx = m > 0 ? kActMax / m : 0.f;
    if (sub == 0) bsl[b] = m / kActMax;
    uint32_t hw[4], lw[4]; int ls = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      uint32_t hh = 0, ll = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int q = (int)__builtin_rintf(v[4 * k + j] * isx);
        hh |= (uint32_t)((q >> 8) & 0xff) << (8 * j);
        ll |= (uint32_t)(q & 0xff) << (8 * j);
        ls += q & 0xff;
      }
      hw[k] = hh; lw[k] = ll;
    }
    *(uint4 *)(xh + c0) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    *(uint4 *)(xl + c0) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    ls = sum8_i(ls);
    if (sub == 0) lsl[b] = ls;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < NL; i++) {
    const int p = threadIdx.x + NT * i, lr = p / ppr, c16 = p % ppr;
    const uint4 h = *(const uint4 *)(xh + 16 * c16), l = *(const uint4 *)(xl + 16 * c16);
    const uint4 ww = wr[i];
    int A = __builtin_amdgcn_sdot4((int)ww.x, (int)h.x, 0, false);
    A = __builtin_amdgcn_sdot4((int)ww.y, (int)h.y, A, false);
    A = __builtin_amdgcn_sdot4((int)ww.z, (int)h.z, A, false);
    A = __builtin_amdgcn_sdot4((int)ww.w, (int)h.w, A, false);
    uint32_t B = __builtin_amdgcn_udot4(ww.x ^ 0x80808080u, l.x, 0u, false);
    B = __builtin_amdgcn_udot4(ww.y ^ 0x80808080u, l.y, B, false);
    B = __builtin_amdgcn_udot4(ww.z ^ 0x80808080u, l.z, B, false);
    B = __builtin_amdgcn_udot4(ww.w ^ 0x80808080u, l.w, B, false);
    const int sum = sum8_i(A * 256 + (int)B);
    if ((lane & 7) == 0 && lr < R) isl[lr * nb + (c16 >> 3)] = sum - 128 * lsl[c16 >> 3];
  }
  __syncthreads();
  for (int lr = threadIdx.x; lr < R; lr += NT) {
    float ch = 0.f;
    for (int b = 0; b < nb; b++) ch = __builtin_fmaf(bsl[b], (float)isl[lr * nb + b], ch);
    const int row = r0 + lr;
    float y = ch * ((const float *)w.wo.s)[row];
    asm volatile("" : "+v"(y));   // y rounded on its own, then added (rows_q8's y, then x += y): no fma contraction
    w.x[row] = w.x[row] + y;
  }
}

int attn_single_max(int hd) { return kAttnMfBlk * kAttnMfWaves * 64 / hd; }

bool attn_wo_rows_fits(int hd, int nh, int nkv, const DMat &wo, int cus, int *rc, int *nl) {
  if (wo.kind != MK_Q8 || nh % nkv || hd != 64 || nkv > kAwoRowsMaxGroups) return false;
  const int rep = nh / nkv, cols = nh * hd;
  if (rep > 8 || wo.cols != cols || cols % kQB || cols > kAwoRowsMaxCols || wo.rows < 1) return false;
  const int c = std::max(1, std::min(wo.rows, cus)), R = (wo.rows + c - 1) / c, pieces = R * (cols / 16);
  const int need = (pieces + kAttnMfWaves * 64 - 1) / (kAttnMfWaves * 64);
  if (need > 4) return false;
  *rc = (wo.rows + R - 1) / R; *nl = need <= 1 ? 1 : need <= 2 ? 2 : 4;
  return true;
}

hipError_t launch_attn_wo_rows(const AttnArgs &a, AwoArgs w, hipStream_t st) {
  int rc = 0, nl = 0;
  if (!attn_wo_rows_fits(a.hd, a.nh, a.nkv, w.wo, g_mv_config.cus, &rc, &nl) || !w.x) return hipErrorInvalidValue;
  w.R = (w.wo.rows + rc - 1) / rc;
  if ((size_t)(rc - 1) * w.R >= (size_t)w.wo.rows) return hipErrorInvalidValue;
  const int rep = a.nh / a.nkv;
#define QPH_AWR(HD, R, NL)                                                                                          \
  if (a.hd == HD && rep == R && nl == NL) {                                                                         \
    hipLaunchKernelGGL((k_attn_wo_rows<HD, R, NL>), dim3(rc), dim3(kAttnMfWaves * 64), 0, st, a, w);                \
    return hipGetLastError();                                                                                       \
  }
#define QPH_AWR3(HD, R) QPH_AWR(HD, R, 1) QPH_AWR(HD, R, 2) QPH_AWR(HD, R, 4)
  // head dim 64 only: at 128 a group's heads are always whole 128-column blocks (k_attn_wo takes the model)
  QPH_AWR3(64, 1) QPH_AWR3(64, 2) QPH_AWR3(64, 3) QPH_AWR3(64, 4) QPH_AWR3(64, 5) QPH_AWR3(64, 6) QPH_AWR3(64, 7)
  QPH_AWR3(64, 8)
#undef QPH_AWR3
#undef QPH_AWR
  return hipErrorInvalidValue;
}

// ------------------------------------------------------------------ greedy pick
// embed (optional, greedy runs): the chosen token's embedding row also goes to x - the next step's input, so the
// next greedy step needs no embedding launch of its own
__global__ __launch_bounds__(kThreads) void k_argmax_finish(const float2 *amax, int n, Ctl *ctl, int *out_tokens, DMat embed,
                                                            float *x) {
  constexpr int NW = kThreads / kWave;
  __shared__ float bv_s[NW]; __shared__ int bi_s[NW]; __shared__ int tok_s;
  float bv = -INFINITY; int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const float v = amax[i].x; const int idx = __builtin_bit_cast(int, amax[i].y);
    if (better(v, idx, bv, bi)) { bv = v; bi = idx; }
  }
  // strict > with the lower index winning ties is associative: the wave butterfly, then the wave results in order
  wave_argmax(bv, bi);
  if ((threadIdx.x & (kWave - 1)) == 0) { bv_s[threadIdx.x / kWave] = bv; bi_s[threadIdx.x / kWave] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < NW; w++) if (better(bv_s[w], bi_s[w], bv_s[0], bi_s[0])) { bv_s[0] = bv_s[w]; bi_s[0] = bi_s[w]; }
    int t = bi_s[0]; if (t == 0x7fffffff) t = 0;
    out_tokens[ctl->n_out] = t;
    ctl->tok = t; ctl->pos = ctl->pos + 1; ctl->n_out = ctl->n_out + 1;
    tok_s = t;
  }
  if (x) {
    __syncthreads();
    embed_row(embed, tok_s, x, threadIdx.x, kThreads);
  }
}
hipError_t launch_argmax_finish(const float2 *amax, int n, Ctl *ctl, int *out_tokens, hipStream_t st, const DMat *embed,
                                float *x) {
  hipLaunchKernelGGL(k_argmax_finish, dim3(1), dim3(kThreads), 0, st, amax, n, ctl, out_tokens, embed ? *embed : DMat{},
                     embed ? x : nullptr);
  return hipGetLastError();
}

// ------------------------------------------------------------------ calibration copy
__global__ __launch_bounds__(256) void k_copy(const u32x4 *src, u32x4 *dst, size_t n16) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}
hipError_t launch_copy(const void *src, void *dst, size_t n16, hipStream_t st) {
  hipLaunchKernelGGL(k_copy, dim3(4096), dim3(256), 0, st, (const u32x4 *)src, (u32x4 *)dst, n16);
  return hipGetLastError();
}

}  // namespace qph
