// Host-side launchers of the gfx950 token-loop kernels (implemented in kernels.hip).
#pragma once
#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "common.hpp"

// host code: throw on a failed HIP call
#define QPH_CK(x)                                                                                           \
  do {                                                                                                      \
    hipError_t e_ = (x);                                                                                    \
    if (e_ != hipSuccess) throw std::runtime_error(std::string("hip: ") + hipGetErrorString(e_) + " at " + #x); \
  } while (0)

namespace qph {

// how a matvec kernel builds its int16 activation vector in LDS
enum Prologue : int {
  PRO_QUANT = 0,   // quantise x as is (wo input, down input, test hook)
  PRO_NORM = 1,    // RMSNorm(x) * w, then quantise (qkv, gate/up, output head)
  PRO_NORM_SUM = 2,   // the same on x + the sum of nparts partial vectors (gate/up after the fused attention + wo)
};
// what a matvec kernel does with each finished row value y = W x
enum Epilogue : int {
  EPI_STORE = 0,    // out[seg][row] = y (+ bias[seg][row])          up to 3 segments (q / k / v)
  EPI_RESID = 1,    // out[0][row] = in[row] + y, in = resid_in or out[0] (wo, down: residual stream)
  EPI_SWIGLU = 2,   // out[0][row] = silu(y_gate) * y_up            (segments 0 = gate, 1 = up, same rows)
  EPI_ARGMAX = 3,   // out[0][row] = y and one (max, index) per workgroup into amax (output head)
};

struct MvArgs {
  DMat m[3];
  int nseg;
  int seg_tile0[4];       // first tile of each segment (prefix sums), seg_tile0[nseg] = total tiles
  const float *x;         // input vector [cols]
  const float *norm_w;    // PRO_NORM weights [cols]
  float eps;
  float *out[3];
  const float *bias[3];
  float2 *amax;           // EPI_ARGMAX: one (value, index-as-float-bits) per workgroup
  int32_t *dbg_sums;      // optional: exact int32 accumulators [rows, cols/128] (q8) or [rows, cols/32] (q4), segment 0
  int16_t *dbg_xq;        // optional: the quantised activation (workgroup 0 writes it)
  float *dbg_bs;          // optional: the activation block scales
  int dbg_mode;           // measurement only: bit 0 skips the dot products, bit 1 skips the activation prologue, bit 2 the epilogue
  int upw;                // set by the launcher: the most units one wave owns (sizes the per-wave LDS)
  // set by the launcher for one launch over q8 and q4 segments (MK_MIX): the q8 segments come first, their units are
  // [0, mix_u8), and waves gw < mix_w8 take them; the other waves take the q4 units
  int mix_w8, mix_u8;
  // PRO_NORM_SUM: partial vectors part[j * pstride + c], j < nparts (added to x in order); workgroup 0 stores the sum
  const float *part; int nparts; size_t pstride; float *xsum;
  int plan_only;   // launch_matvec checks the launch (shape, LDS) and returns without enqueueing it
  uint64_t *stamps;   // measurement only (optional): per wave 4 realtime stamps (start, prologue done, loop done, end)
  int stamp_waves;    // with stamps: the waves they have room for (0: any); a larger launch runs without stamps
  const float *resid_in;   // EPI_RESID: the residual input when it is not out[0]
  // EPI_STORE (q / k / v of the decode step; needs 2-row units): segment s with rope[s] pairs rows i and i + hd / 2 of
  // each head in a unit and rotates them after the bias (model_llama.cpp:176: a' = fma(a, cos, -(b sin)),
  // b' = fma(b, cos, a sin), tables at position ctl->pos); a segment with cache[s] also writes its (rotated) row as
  // fp16 into cache[s] at position ctl->pos (row stride cache_ld)
  int rope[3];
  uint16_t *cache[3];
  int cache_ld, hd;
  const float *cos_t, *sin_t;
  const Ctl *ctl;
  uint16_t *q16[3];   // optional per segment (q): its rotated rows also as fp16 hi [rows] then lo = f16(y - hi) [rows]
  // EPI_RESID / EPI_SWIGLU, q8, at most 32 rows per wave (the decode step's down and gate / up products): 8, 4 or 2
  // lanes per row (as the wave's rows allow) each chain a contiguous share of the blocks, then a fixed pairwise sum -
  // another fp32 order than rows_q8's single chain (the int32 block sums stay exact), a fraction of its dependent
  // latency (down at the 8B shape: a 112-block chain)
  int split_chain;
};

// The matvec kernel runs one workgroup of up to 16 waves per CU; every wave streams its own units of 1 or 2 rows
// (2 slots: EPI_SWIGLU pairs the gate and up rows).  `cus` is the device's CU count.
struct MvConfig {
  int cus = 256;
};
extern MvConfig g_mv_config;
constexpr int kMvMaxWaves = 16;
constexpr int kMvSlots = 2;
int mv_tile_rows(int epi);
size_t mv_lds_bytes(int cols, int waves, int per_wave);
// fills seg_tile0 from the segment row counts
void mv_plan(MvArgs &a, int epi);
// grid_cap: the most workgroups (EPI_ARGMAX writes one (max, index) partial per workgroup launched)
hipError_t launch_matvec(int pro, int epi, const MvArgs &a, int grid_cap, hipStream_t st);

// the M largest (index, value) pairs of x[n] (device), value descending and the lower index first among equal values
// (sampler.cpp:12-27), into idx[M] / val[M] (device); scratch buf_a / buf_b of topk_scratch_keys(n, M) keys each
constexpr int kTopkMax = 512;
size_t topk_scratch_keys(int n, int M);
hipError_t launch_topk(const float *x, int n, int M, uint64_t *buf_a, uint64_t *buf_b, int *idx, float *val,
                       hipStream_t st);
// the same with the key buffers in a file-scope device array (no allocation): n <= 262144; device pointers; enqueued on st
hipError_t launch_topk_noalloc(const float *x, int n, int M, int *idx, float *val, hipStream_t st);

// x[0..d) = row ctl->tok of the embedding (row_f32 semantics, /root/reference/src/kernels.cpp:146-162)
hipError_t launch_embed(const DMat &embed, const Ctl *ctl, float *x, hipStream_t st);
// out = RMSNorm(x) * w (single workgroup; identical arithmetic to the PRO_NORM prologue)
hipError_t launch_rmsnorm(const float *x, const float *w, int n, float eps, float *out, hipStream_t st);

struct AttnArgs {
  const float *q;              // this step's queries, RoPE applied (the q / k / v matvec's epilogue)
  const uint16_t *q16;         // the same as fp16 hi [nh * hd] then lo [nh * hd] halves (MvArgs::q16)
  int ctx;                     // positions allocated in the caches (loads stay below it)
  uint16_t *kc, *vc;           // this layer's fp16 caches [ctx][kvd], the current position's rows already written
  const Ctl *ctl;
  float *part;                 // unnormalised outputs [nh][splits][hd], then (max, sum) [nh][splits][2]
  int *counters;               // [2 nkv] zero: arrivals and finished mergers per group; the last merger resets both
  float *att;                  // output [nh * hd]
  int nh, nkv, hd;
  int max_chunks;              // splits S of the context per kv group (grid.y)
  int single_max;              // contexts up to this many positions run one split per group (0: 64 KiB of K and V)
  int split_pos;               // beyond: S = min(max_chunks, ceil(T / split_pos)) (0: 64)
  int *status;                 // optional (host-visible): set to 1 when a merger's bounded wait for the partials ran out
  int spin_limit;              // the bound of that wait in polls (0: 1 << 22)
  int force_late;              // test hook: every merger that would wait gives up at once (the error path, forced)
  int early;                   // one-split kernels (k_attn_wo, k_attn_wo_rows): the waves that load their first block before
                               // the context is known (0: all); the others load theirs, if they have one, once it is
  int merge_sep;               // > 1: contexts of at least this many splits only store their partials and a second
                               // launch (k_attn_merge, one workgroup per head) merges them
  uint64_t *stamps;            // measurement only (optional): per workgroup of k_attention 5 words - realtime at start,
                               // partials stored, merge rank known, end, and 1 if it merged
};
hipError_t launch_attention(const AttnArgs &a, hipStream_t st);
// the shortest context from which every decode step runs at least min_splits splits per kv group (the
// separate-merge form, AttnArgs::merge_sep), 0 when no context does
int attn_long_merge_min(int hd, int single_max, int split_pos, int max_chunks, int min_splits);
// Decode attention fused with the wo product (q8 wo, REP * hd a multiple of 128): grid (nkv, rc); workgroup (g, c)
// computes kv group g's attention over the whole context (no splits) and, for wo rows [c R, c R + R), the product over
// the group's columns: part[g][row] = (rows_q8's fp32 block chain over the group's blocks) * scale[row].  The next
// kernel adds x + sum_g part[g] in group order (PRO_NORM_SUM).  The attention's part / counters / max_chunks fields are
// unused.
struct AwoArgs {
  DMat wo;      // q8 [d][nh * hd]
  float *part;  // [nkv][d] per-group partial products
  float *x;     // k_attn_wo_rows, and k_attn_wo with counters: the residual stream [d] (x += wo . att)
  int *counters;   // k_attn_wo: [row chunks][8] arrival counters (per wave of the chunk's rows, or [c][0] per
                   // workgroup), zero before the first launch (each launch leaves them zero); when set, the last
                   // arrival adds the group parts to x, else the next kernel does
  int R;        // rows per chunk (set by the launcher)
  uint64_t *stamps;   // measurement only (optional): per workgroup realtime at start, after the attention, after the
                      // weights arrived, at the end
};
// whether the fused kernel takes this shape; rc = row chunks (grid.y), nl = 16-byte weight pieces per thread
bool attn_wo_fits(int hd, int nh, int nkv, const DMat &wo, int cus, int *rc, int *nl);
hipError_t launch_attn_wo(const AttnArgs &a, AwoArgs w, hipStream_t st);
// Every group's attention (one split each) and whole wo rows with the residual add, for q8 wo with at most 2 kv groups
// and nh * hd <= 2048 (groups that are not whole 128-column blocks, e.g. 7 heads of 64): grid rc; bit-identical to
// k_attention with one split per group followed by the wo matvec (EPI_RESID)
bool attn_wo_rows_fits(int hd, int nh, int nkv, const DMat &wo, int cus, int *rc, int *nl);
// the longest context k_attention runs as one split per kv group by default (64 KiB of K and V per group)
int attn_single_max(int hd);
hipError_t launch_attn_wo_rows(const AttnArgs &a, AwoArgs w, hipStream_t st);

// greedy pick over the head's per-workgroup (max, index) pairs; advances ctl (tok = pick, pos += 1, n_out += 1) and
// writes the pick to out_tokens[ctl->n_out]
// dst[0..n16) = src[0..n16) in 16-byte words (counter calibration)
hipError_t launch_copy(const void *src, void *dst, size_t n16, hipStream_t st);

// embed / x (optional): also write the chosen token's embedding row to x (the next greedy step's input)
hipError_t launch_argmax_finish(const float2 *amax, int n, Ctl *ctl, int *out_tokens, hipStream_t st,
                                const DMat *embed = nullptr, float *x = nullptr);

// ---- batched prompt path (prefill.hip)
// embeddings of B token ids (device array) into X[B][ldx]
hipError_t launch_pf_embed(const DMat &embed, const int *toks, int B, float *X, int ldx, hipStream_t st);
// per-token quantisation: X[t] (optionally RMSNorm(X[t]) * norm_w) -> int8 planes xh = q >> 8, xl = (q & 255) - 128
// [B][ldq] and block scales xb [B][ldb]; the decode prologue's arithmetic
struct PfQuantArgs {
  const float *x; int ldx;
  const float *norm_w; float eps;
  int cols;
  int8_t *xh, *xl; int ldq;
  float *xb; int ldb;
  float *xbt; int ldbt;   // optional: the block scales block-major [cols / 128][ldbt]
  int *xg; int ldg;   // optional: sum of q per 32-column group [B][ldg] (the q4 product needs it)
};
hipError_t launch_pf_quant(int pro, const PfQuantArgs &a, int B, hipStream_t st);
// Y[t][r] = the row's dot product with token t's quantised activation (+ bias[r]), or Y[t][r] += that when resid.
//   kind MK_Q8: w int8 [rows][cols], scale f32 [rows], wsum = row sums per 128-column block [rows][ldw] (launch_rowsum_q8)
//   kind MK_Q4: w packed q4 [rows][cols / 2], q4ns / q4sc = per-group nibble sums and f32 scales, group-major per block
//               (launch_q4_prep), and the activation's group sums xg [ntok][ldg] (launch_pf_quant)
// one matrix of a multi-matrix product launch (GemmArgs::nseg > 1): its own weights, scales, bias and output
struct GemmSeg {
  const int8_t *w; const float *scale; const int *wsum; const int *q4ns; const float *q4sc;
  const float *bias; float *y; int rows, ldy;
};
constexpr int kGemmMaxSeg = 3;
struct GemmArgs {
  int kind;
  const int8_t *w; const float *scale; int rows, cols;
  const int *wsum;   // q8: 128 x the row sums per 128-column block (k_rowsum_q8), [cols / 128][ws_pitch(rows)]
  const int *q4ns; const float *q4sc;
  const int *xg; int ldg;
  const int8_t *xh, *xl; const float *xb; int ntok, ldq, ldb;
  const float *xbt; int ldbt;   // q8: the block scales again, block-major [cols / 128][ldbt] (ldbt % 4 == 0, >= ntok)
  float *y; int ldy;
  const float *bias;
  int resid;
  // optional, same layout as y: y = silu(gate) * product (SwiGLU on the up product; gate may be y itself)
  const float *gate;
  // optional (q8): a second matrix of the same shape (the up matrix, with w / scale / wsum the gate's): one launch
  // computes both products for each 64-row tile and stores only y = silu(gate product) * (up product)
  const int8_t *w2; const float *scale2; const int *wsum2;
  // optional (with w2, 32 x 32 kernel only, rows % 128 == 0): instead of y, the SwiGLU output quantised for the next
  // product - planes oh / ol [ntok][ldq], block scales ob [ntok][ldb] and obt [rows / 128][ldbt] (the quantiser's
  // arithmetic: every 128-row tile of the pair is one quantisation block of each token)
  int8_t *oh, *ol; float *ob, *obt;
  // optional: nseg (2 .. kGemmMaxSeg) matrices of this kind and column count over the same activations (q / k / v), the
  // segment fields replacing w / scale / wsum / q4ns / q4sc / bias / y / ldy / rows; each starts on a fresh row tile
  int nseg;
  GemmSeg seg[kGemmMaxSeg];
  int tile0;   // first row tile of this launch (a launch split over the two q8 kernels; set by launch_gemm)
  int dbg;   // measurement switches of the 32 x 32 q8 kernel (QPH_G2_DBG; results are wrong when set): 1 no compute,
             // 2 no loads after the first block, 4 no barriers
};
size_t gemm_lds_bytes();
// row pitch of the block-major row sums: rows rounded up to 64 (16-byte loads of 4 rows stay inside a block's run)
__host__ __device__ inline int ws_pitch(int rows) { return (rows + 63) & ~63; }
// out[row][block] = sum of W[row] over each 128-column block
hipError_t launch_rowsum_q8(const int8_t *w, int rows, int cols, int *out, hipStream_t st);
// q4 rows: per (block, group, row) the sum of the nibbles and the f32 scale, group-major within each 128-column block
hipError_t launch_q4_prep(const uint8_t *w, const uint16_t *sc, int rows, int cols, int *out_ns, float *out_sc, hipStream_t st);
hipError_t launch_gemm(const GemmArgs &a, hipStream_t st);
// whether launch_gemm runs this q8 launch on the 32 x 32 kernel (the one that can quantise a SwiGLU pair's output)
bool gemm_uses_32x32(const GemmArgs &a);
// token t of the batch at position p0 + t: RoPE on q [t][ldq] (in place) and k, fp16 k / v rows into the caches
struct PfRopeArgs {
  float *q; int ldq;
  const float *k, *v; int ldk;
  const float *cos_t, *sin_t;
  uint16_t *kc, *vc;
  int p0, nh, nkv, hd;
  int skip_q;   // q is rotated by the attention kernel instead
};
hipError_t launch_pf_rope(const PfRopeArgs &a, int B, hipStream_t st);
// causal attention of the batch's (rotated) queries over cache positions [0, p0 + t] -> att [t][lda]
struct PfAttnArgs {
  const float *q; int ldq;
  const uint16_t *kc, *vc;
  float *att; int lda;
  int ntok, p0, nh, nkv, hd;
  // optional: q not yet rotated - the kernel applies RoPE (k_pf_rope's arithmetic) as it loads q
  const float *cos_t, *sin_t;
  // optional (hd 128, one head = one 128-column block): the output quantised for the wo product instead of att -
  // planes oh / ol [ntok][ldo], block scales ob [ntok][ldb] and obt [nh][ldbt] (the quantiser's arithmetic)
  int8_t *oh, *ol; float *ob, *obt; int ldo, ldb, ldbt;
};
hipError_t launch_pf_attn(const PfAttnArgs &a, hipStream_t st);

// ---- reference-order mode (exact.hip): the reference CPU path's float orders, bit-identical results
// RMSNorm of `rows` vectors [ldx] with the sequential sum of squares, out [ldo]
hipError_t launch_ex_rmsnorm(const float *x, int ldx, const float *w, int n, float eps, float *out, int ldo, int rows,
                             hipStream_t st);
// decode RoPE: q -> qr rotated; k rotated and v, as fp16, into the cache row ctl->pos
struct ExRopeArgs {
  const float *q, *k, *v;
  float *qr;
  const float *cos_t, *sin_t;
  const Ctl *ctl;
  uint16_t *kc, *vc;
  int nh, nkv, hd;
};
hipError_t launch_ex_rope(const ExRopeArgs &a, hipStream_t st);
// decode attention over 64-position chunks (partials [nh][ncmax][hd + 2]) and their ordered merge into att [nh * hd]
struct ExAttnArgs {
  const float *qr;
  const uint16_t *kc, *vc;
  const Ctl *ctl;
  float *part;
  float *att;
  int nh, nkv, hd, ncmax;
};
hipError_t launch_ex_attention(const ExAttnArgs &a, hipStream_t st);
// prompt attention: the batch's rotated queries q [B][ldq] at positions p0 .. p0 + B - 1 -> att [B][lda]
struct ExPfAttnArgs {
  const float *q; int ldq;
  const uint16_t *kc, *vc;
  float *att; int lda;
  int p0, nh, nkv, hd;
};
hipError_t launch_ex_pf_attn(const ExPfAttnArgs &a, int B, hipStream_t st);
// y [ntok][ldy] = W x_t (+ bias; or += when resid) over the quantiser's planes; vectors t < mm_below in mm_q8 / mm_q4
// order, the rest in rows_q8 / rows_q4 order; tt = vectors per workgroup tile (1 or 16)
struct ExGemmArgs {
  int kind;
  const void *w; const float *scale; const uint16_t *s16;
  int rows, cols;
  const int8_t *xh, *xl; int ldq;
  const float *xb; int ldb;
  int ntok, mm_below, tt;
  float *y; int ldy;
  const float *bias;
  int resid;
};
hipError_t launch_ex_gemm(const ExGemmArgs &a, hipStream_t st);
// per-workgroup (max, lowest index) partials of logits x[V] into amax[nparts] (what the argmax matvec leaves for
// k_argmax_finish)
hipError_t launch_ex_argmax_parts(const float *x, int V, float2 *amax, int nparts, hipStream_t st);
// g = silu(g) * u on rows of n values
hipError_t launch_ex_silu(float *g, const float *u, int n, int ld, int rows, hipStream_t st);

// QPACK3 rANS decode (hip/rans_decode.hip): one task per coded plane, one wave per task
struct RansTaskDev {
  const uint8_t *plane;   // the plane's u32 comp_len field (device)
  uint8_t *out;           // output byte of symbol 0 (device)
  int64_t n;              // symbols
  uint32_t comp_len;      // bytes after the comp_len field
  int nsym, stride, nibbles;
};
struct RansState {   // a plane's decoder between launches
  uint32_t st[4];
  uint64_t q;   // stream offset from the 16-byte aligned address at or below the first stream byte
  int64_t s0;   // symbols decoded
};
// decode every plane as far as its first `avail` bytes (from the comp_len field) allow (state[].s0 = -1 before the
// first launch)
hipError_t launch_rans(const RansTaskDev *tasks, int ntasks, int *status, RansState *state, uint64_t avail, hipStream_t st);
struct RansTiming {
  int planes = 0, rounds = 0;
  uint64_t coded = 0, raw = 0;
  float upload_ms = 0, decode_ms = 0, total_ms = 0;
};
// Coded blobs (host memory) with their device destinations: run() plans the planes (throwing on malformed headers),
// uploads the coded bytes into one staging buffer and decodes them there, waits, and throws on a stream overrun.
// round_bytes > 0 streams the upload: round r brings bytes [r R, (r + 1) R) of every plane (R = round_bytes) on a copy
// stream, and a decode launch after each round takes every plane as far as its uploaded bytes allow, so the decode
// runs under the upload; 0: the whole upload, then one launch.
class RansBatch {
 public:
  void add(const uint8_t *blob, size_t len, void *out, size_t out_cap);
  void run(hipStream_t st, RansTiming *tm = nullptr, uint64_t round_bytes = 0);
  // the round size loads use: QPH_RANS_ROUND (bytes; 0 = no streaming), else 512 KiB
  static uint64_t default_round();
  bool empty() const { return items_.empty(); }

 private:
  struct Item { const uint8_t *blob; size_t len; uint8_t *out; size_t stage_off; };
  std::vector<Item> items_;
  size_t coded_ = 0;
  uint64_t raw_ = 0;
};

}  // namespace qph
