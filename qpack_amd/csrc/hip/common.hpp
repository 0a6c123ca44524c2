// Shared device-side definitions of the gfx950 token-loop kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qph {

constexpr int kQB = 128;            // activation block (/root/reference/src/kernels_impl.h:13)
constexpr float kActMax = 32767.f;  // x86 kActMax (/root/reference/src/kernels_impl.h:19)
constexpr int kWave = 64;

enum MatKind : int { MK_F32 = 0, MK_Q8 = 1, MK_Q4 = 2, MK_Q1 = 3 };
constexpr int MK_MIX = 9;   // a matvec launch over q8 and q4 segments (each wave streams one kind)

// a weight matrix resident in HBM, row-major as in the QPACK2 file
struct DMat {
  const void *q;       // q8: int8 [rows, cols]; q4: u8 [rows, cols / 2]; q1: sign bits u8 [rows, cols / 8]; f32: float
  const void *s;       // q8: f32 [rows]; q4: fp16 [rows, cols / 32]; q1: fp16 [rows, cols / 128]
  int rows, cols, kind;
  // layer matrices on the batched prompt path: q8 row sums per 128-column block [rows, cols / 128]; q4 nibble sums and
  // f32 scales per (block, group, row), group-major within each block
  const int *rs;
  const int *q4ns;
  const float *q4sc;
};

// device-resident decode control block: the token to embed, its position, and the greedy output cursor
struct Ctl {   // pos at byte offset 4 (ctl_pos_issue)
  int tok;
  int pos;
  int n_out;   // greedy tokens written so far in this run
  int pad;
};
// ctl->pos read through the scalar data cache: ctl_pos_issue sends the load, the value is valid after ctl_pos_wait.  A
// vector load of it would return in order behind every vector load the wave issued before it, and the wave would wait
// for all of them to learn the position.
__device__ __forceinline__ int ctl_pos_issue(const Ctl *c) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x4" : "=s"(v) : "s"(c));
  return v;
}
__device__ __forceinline__ int ctl_pos_wait(int v) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(v)::"memory");
  return v;
}


__device__ __forceinline__ float half_bits_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t float_to_half_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
// an fp32 result rounded to fp32 first and then to fp16, like the reference's to_f16 of a stored float vector
// (kernels_x86.cpp:449-452): without the barrier the compiler fuses an fma feeding the conversion into v_fma_mix, which
// rounds once, straight to fp16 (a different fp16 value when the fp32 result sits next to an fp16 midpoint)
__device__ __forceinline__ uint16_t f32_to_half_bits(float f) {
  asm volatile("" : "+v"(f));
  return float_to_half_bits(f);
}

// exp256 of /root/reference/src/kernels_x86.cpp:406-417 for one lane: clamp to [-87, 88], k = rint(x log2 e),
// two-constant reduction, degree-6 polynomial, scale by 2^k.  Written with explicit fmaf so it is bit-identical.
__device__ __forceinline__ float exp_poly(float x) {
  x = x > -87.f ? x : -87.f;
  x = 88.f > x ? x : 88.f;
  const float k = __builtin_rintf(x * 1.44269504088896341f);
  const float r = __builtin_fmaf(-k, 0.693359375f, __builtin_fmaf(-k, -2.12194440e-4f, x));
  float p = 1.9875691500e-4f;
  p = __builtin_fmaf(p, r, 1.3981999507e-3f);
  p = __builtin_fmaf(p, r, 8.3334519073e-3f);
  p = __builtin_fmaf(p, r, 4.1665795894e-2f);
  p = __builtin_fmaf(p, r, 1.6666665459e-1f);
  p = __builtin_fmaf(p, r, 5.0000001201e-1f);
  p = __builtin_fmaf(p * r, r, r + 1.f);
  const int e = ((int)k + 127) << 23;
  return p * __builtin_bit_cast(float, e);
}

// DPP cross-lane moves (bound_ctrl, full row / bank masks)
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true); }
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) { return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, true)); }
constexpr int kDppQuadXor1 = 0xb1;       // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4e;       // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;    // row_half_mirror: lane i <-> 7 - i within 8 lanes
constexpr int kDppMirror = 0x140;        // row_mirror: lane i <-> 15 - i within 16 lanes
constexpr int kDppRowShl4 = 0x104;       // row_shl:4: lane i reads lane i + 4 of its 16-lane row (0 past the row)
constexpr int kDppRowRor8 = 0x128;       // row_ror:8: lane i reads lane i ^ 8 of its 16-lane row
constexpr int kDppRowRor4 = 0x124;       // row_ror:4: lane i reads lane (i + 4) mod 16 of its row

// sum over aligned groups of 8 lanes, result in every lane of the group (exact for integers)
__device__ __forceinline__ int sum8_i(int v) {
  v += dpp_i<kDppQuadXor1>(v);
  v += dpp_i<kDppQuadXor2>(v);
  v += dpp_i<kDppHalfMirror>(v);
  return v;
}
__device__ __forceinline__ float max8_f(float v) {
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  return v;
}

// full-wave sum without LDS traffic (for loops that stream memory): DPP sums over each 16-lane row, then the four row
// sums in order ((r0 + r1) + (r2 + r3)); the value in every lane (the row sums are read as scalars)
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_f<kDppQuadXor1>(v);
  v += dpp_f<kDppQuadXor2>(v);
  v += dpp_f<kDppHalfMirror>(v);
  v += dpp_f<kDppMirror>(v);
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)), r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)), r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

// exchanges with lane ^ 8, ^ 16, ^ 32 as VALU instructions (__shfl_xor goes through the LDS crossbar, ds_bpermute):
// lane ^ 8 is a DPP rotation by 8 inside each 16-lane row; the gfx950 v_permlane16_swap / v_permlane32_swap of a
// value and a copy of it leave, in some order, the lane's own value and that of lane ^ 16 (^ 32) in the two registers -
// a max or a sum of the two is the pair's, the same bits as with the shuffle (both operations are commutative).  The
// swaps are written as asm: clang's builtins for them (ROCm 7.2) lost the second result once inlined (both read as the
// first); s_nop 1 on either side covers the VALU hazards the compiler inserted itself around the builtin.
__device__ __forceinline__ uint32_t xchg8_u32(uint32_t v) { return __builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, false); }
__device__ __forceinline__ void swap16(float v, float &a, float &b) {
  a = v; b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float v, float &a, float &b) {
  a = v; b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ int pair_sum16_i(int v) {
  int a = v, b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return a + b;
}
__device__ __forceinline__ float pair_max16(float v) { float a, b; swap16(v, a, b); return fmaxf(a, b); }
__device__ __forceinline__ float pair_max32(float v) { float a, b; swap32(v, a, b); return fmaxf(a, b); }
__device__ __forceinline__ float pair_sum16(float v) { float a, b; swap16(v, a, b); return a + b; }
__device__ __forceinline__ float pair_sum32(float v) { float a, b; swap32(v, a, b); return a + b; }

// max / integer sum over aligned groups of 32 lanes, in every lane of the group: 8-lane steps, the row mirror, then
// the two rows of the half
__device__ __forceinline__ float max32_f(float v) {
  v = max8_f(v);
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  return pair_max16(v);
}
__device__ __forceinline__ int sum32_i(int v) {
  v = sum8_i(v);
  v += dpp_i<kDppMirror>(v);
  return pair_sum16_i(v);
}
__device__ __forceinline__ float xchg8_f(float v) { return __builtin_bit_cast(float, xchg8_u32(__builtin_bit_cast(uint32_t, v))); }

// full-wave butterfly reductions, partners lane ^ 32, ^ 16, ^ 8, ^ 4, ^ 2, ^ 1 in that order (the same sums as xor
// shuffles), each exchange a VALU instruction: the permlane swaps, DPP row rotations by 8 and by 4 (after the ^ 8 step
// lanes i and i ^ 8 hold equal values, so lane i + 4 within the row stands for lane i ^ 4), quad permutations
__device__ __forceinline__ float wave_sum(float v) {
  v = pair_sum32(v);
  v = pair_sum16(v);
  v += dpp_f<kDppRowRor8>(v);
  v += dpp_f<kDppRowRor4>(v);
  v += dpp_f<kDppQuadXor2>(v);
  v += dpp_f<kDppQuadXor1>(v);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  v = pair_max32(v);
  v = pair_max16(v);
  v = fmaxf(v, dpp_f<kDppRowRor8>(v));
  v = fmaxf(v, dpp_f<kDppRowRor4>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f<kDppQuadXor1>(v));
  return v;
}

// direct global -> LDS loads (global_load_lds_dwordx4 / _dword): the wave's lanes land 16 (4) bytes each, contiguously
// from the wave-uniform LDS base, in lane order; they count in vmcnt like any other load
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;
__device__ __forceinline__ void dma16(const void *g, void *lds_wave_base) {
  __builtin_amdgcn_global_load_lds((glb_void_t *)g, (lds_void_t *)lds_wave_base, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void *g, void *lds_wave_base) {
  __builtin_amdgcn_global_load_lds((glb_void_t *)g, (lds_void_t *)lds_wave_base, 4, 0, 0);
}
}  // namespace qph
