// QPACK3 rANS decode in HBM (the format of /root/reference/include/qpack/rans.h; the reference decodes on the CPU at
// load, /root/reference/src/container.cpp:94-121).
//
// A coded plane is one sequential stream: its four interleaved states share one byte stream, so symbol i + 1's bytes
// start where symbol i's end and a plane decodes in order.  The parallelism is across planes (16 MiB chunks of large
// blobs, the blobs themselves), so the kernel runs one decoding wave per plane and spends that wave on the plane's
// latency chain; a second wave of the workgroup keeps its stream ring filled and stores its symbols.  A wave issues
// about one instruction per 5-6 cycles and an LDS read returns after ~85, so a group's instruction count and its table
// read's exposed latency are the whole cost:
//   - the decode table sits in LDS: per 12-bit slot m the frequency and m - cum as two 16-bit entries, so the state
//     update freq * (x >> 12) + (m - cum) is one multiply-add on the two loaded values; the symbol table is read only
//     when a step's output leaves (the slots wait in registers, then in LDS);
//   - lanes 0..3 hold states 0..3 and decode the group of four symbols 4g .. 4g + 3 together: each lane needs 0, 1 or 2
//     renormalisation bytes; two ballots (x < 2^23, x < 2^15) give every lane its byte offset in the stream (mbcnt of
//     both below the lane) and the group's total (their popcount); the bytes come from an unaligned 8-byte window of the
//     stream, picked out with one byte permute, and the renormalised state is a second byte permute of x and them;
//   - the coded stream is staged in an 8 KiB LDS ring by 1 KiB coalesced loads, at least 2 KiB ahead of the decoder;
//   - the output leaves as 8-byte (bytes) or 4-byte (nibbles) stores of all 64 lanes of the second wave per step;
//   - a launch can stop a plane between steps and a later one resume it (RansState), so the decode runs under the
//     upload of the coded bytes (RansBatch::run).
// The decoded bytes equal rans::decode's (bit-exact); a stream that needs a byte past its plane's end reports an
// overrun, where the reference throws "rans: stream overrun".
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <stdexcept>
#include <vector>

#include "../host/rans.hpp"
#include "launch.hpp"

namespace qph {

constexpr int kRansRing = 8192;    // LDS stream ring (bytes)
constexpr int kRansBlk = 1024;     // one load: 64 lanes x 16 bytes
constexpr int kRansStep = 512;     // symbols between ring refills / output flushes (at most 2 bytes each)
constexpr int kRansAhead = 4096;   // a refill is issued while fewer bytes than this are loaded past the read position

__device__ __forceinline__ uint32_t rd_u8(const uint8_t *p) { return *p; }
// LDS layout (one array, so it starts at LDS address 0 - checked - and the loop's LDS instructions take the tables'
// addresses as immediate offsets):
// ring (+ a copy of its first 16 bytes, so a window never wraps) | tables [3][4096] u16: slot m's freq, m - cum, symbol
// | slot staging, two steps (each group's 2m, 16 bits per symbol) | cumulative frequencies | the decoder's offset
constexpr int kLdsTab = kRansRing + 16, kLdsSlots = kLdsTab + 3 * 2 * rans::kProbScale;
constexpr int kLdsCum = kLdsSlots + 2 * 2 * kRansStep, kLdsQ = kLdsCum + 4 * 260, kLdsBytes = kLdsQ + 16;

// One launch decodes every plane as far as `avail` allows: the bytes of each plane from its comp_len field up to
// avail are in HBM (all of them when avail >= 4 + comp_len).  A step of 512 symbols starts only while its bytes (at
// most 2 per symbol, plus the 8-byte window) are there; a plane that stops keeps its four states, stream offset and
// symbol count in `state` for the next launch, which rebuilds its table and ring from them.  A plane starts (states
// from its header) in the first launch that has its whole header; state[].s0 < 0 marks one not started.
//
// Two waves per plane: wave 0 decodes and touches no global memory inside the step loop; wave 1 keeps the ring filled
// and stores the previous step's symbols.  A wave with a global load in flight had the compiler wait for it
// (vmcnt(0)) at the head of the group loop, next to the loop's LDS asm - a stall at every step; in wave 0 that wait
// now finds nothing outstanding.  The waves meet at one barrier per step: the decoder's stream offset goes to LDS,
// the slot staging alternates between two buffers, and the ring runs at least 2 KiB ahead of the decoder.
__global__ __launch_bounds__(128) void k_rans_decode(const RansTaskDev *tasks, int *status, RansState *state, uint64_t avail) {
  __shared__ __align__(16) uint8_t lds[kLdsBytes];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)lds;
  if (lds0 != 0) { if (threadIdx.x == 0) status[blockIdx.x] = 2; return; }
  uint32_t *const ring = (uint32_t *)lds;
  uint16_t *const tfq = (uint16_t *)(lds + kLdsTab), *const tbi = tfq + rans::kProbScale, *const tsym = tbi + rans::kProbScale;
  uint32_t *const cum = (uint32_t *)(lds + kLdsCum);
  uint32_t *const qsh = (uint32_t *)(lds + kLdsQ);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const RansTaskDev t = tasks[blockIdx.x];
  RansState *const S = state + blockIdx.x;
  const int64_t n = t.n;
  const int nsym = t.nsym;
  const bool first = S->s0 < 0;
  if (first && avail < 4ull + 2 * nsym + 16) return;   // the header is not all in HBM yet
  int64_t s0 = first ? 0 : S->s0;
  if (!first && s0 >= n) return;   // done in an earlier launch

  // stream bytes: offsets are counted from `base`, the 16-byte aligned address at or below the first stream byte
  const uint8_t *sp = t.plane + 4 + 2 * nsym + 16;
  const uint8_t *base = (const uint8_t *)((uintptr_t)sp & ~(uintptr_t)15);
  const uint64_t end_off = (uint64_t)(t.plane + 4 + t.comp_len - base);
  // stream offsets below lim are in HBM (the whole plane: no limit, an overrunning stream reads on and is reported)
  const bool whole = avail >= 4ull + t.comp_len;
  const uint64_t lim = whole ? ~0ull : (uint64_t)(t.plane + avail - base);
  uint64_t q = first ? (uint64_t)(sp - base) : S->q;
  // loads stop at the plane's end (the bytes past it only feed a stream that has overrun, reported below); the ring
  // is filled from the block holding q (bytes loaded past lim are never used in this launch)
  const uint64_t load_max = (end_off + 15) & ~(uint64_t)15;
  uint64_t issued = q & ~(uint64_t)(kRansBlk - 1);
  auto ring_put = [&](uint64_t at, const uint4 &v) {
    const uint32_t o = (uint32_t)(at + 16 * lane) & (kRansRing - 1);
    *(uint4 *)((uint8_t *)ring + o) = v;
    if (o == 0) *(uint4 *)((uint8_t *)ring + kRansRing) = v;
  };
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  auto gload = [&](uint64_t at) {
    const u32x4 v = *(const __attribute__((address_space(1))) u32x4 *)(uintptr_t)(base + std::min(at, load_max) + 16 * lane);
    return make_uint4(v.x, v.y, v.z, v.w);
  };
  // refill (wave 1): the blocks from `issued` while fewer than kRansAhead bytes are loaded past the decoder
  auto refill = [&]() {
    uint4 v[kRansAhead / kRansBlk];
    int k = 0;
#pragma unroll
    for (int j = 0; j < kRansAhead / kRansBlk; j++)
      if ((int64_t)(issued + (uint64_t)j * kRansBlk) - (int64_t)q < kRansAhead) { v[j] = gload(issued + (uint64_t)j * kRansBlk); k = j + 1; }
#pragma unroll
    for (int j = 0; j < kRansAhead / kRansBlk; j++)
      if (j < k) ring_put(issued + (uint64_t)j * kRansBlk, v[j]);
    issued += (uint64_t)k * kRansBlk;
  };

  uint32_t st = 0;
  if (wave == 0) {
    if (lane < 4) {
      if (first) {
        const uint8_t *xs = t.plane + 4 + 2 * nsym + 4 * lane;
        st = rd_u8(xs) | (rd_u8(xs + 1) << 8) | (rd_u8(xs + 2) << 16) | (rd_u8(xs + 3) << 24);
      } else {
        st = S->st[lane];
      }
    }
    // cumulative frequencies: lane l sums symbols [l * per, (l + 1) * per), then an exclusive scan over the lanes
    const uint8_t *fq = t.plane + 4;
    const int per = nsym / 64 ? nsym / 64 : 1;
    uint32_t fl[4] = {0, 0, 0, 0}, own = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int s = lane * per + k;
      if (k < per && s < nsym) { fl[k] = rd_u8(fq + 2 * s) | (rd_u8(fq + 2 * s + 1) << 8); own += fl[k]; }
    }
    uint32_t incl = own;
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t v = __shfl_up(incl, o, 64);
      if (lane >= o) incl += v;
    }
    uint32_t run = incl - own;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int s = lane * per + k;
      if (k < per && s < nsym) { cum[s] = run; run += fl[k]; }
    }
    if (lane == 0) cum[nsym] = rans::kProbScale;
  } else {
    refill();   // the ring's first kRansAhead bytes, under the table build
  }
  __syncthreads();
  // table (both waves): thread i fills slots [32 i, 32 i + 32): the symbol of slot m is the s with cum[s] <= m < cum[s + 1]
  {
    const uint32_t m0 = threadIdx.x * 32;
    int lo = 0, hi = nsym - 1;   // largest s with cum[s] <= m0
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (cum[mid] <= m0) lo = mid; else hi = mid - 1;
    }
    int s = lo;
    for (uint32_t m = m0; m < m0 + 32; m++) {
      while (cum[s + 1] <= m) s++;
      tfq[m] = (uint16_t)(cum[s + 1] - cum[s]);   // <= 4096
      tbi[m] = (uint16_t)(m - cum[s]);
      tsym[m] = (uint16_t)s;
    }
  }
  __syncthreads();

  // flush (wave 1): lane l owns symbols [8 l, 8 l + 8) of a step: batch l / 2, entries 2 (l & 1) and 2 (l & 1) + 1 of
  // the four lanes' slots, mapped to symbols through the symbol table
  typedef __attribute__((address_space(1))) uint8_t glb_u8;
  auto flush = [&](int64_t fs0, int ng, int buf) {
    const int i0 = 8 * lane;
    if (i0 < ng) {
      const uint8_t *const sl = lds + kLdsSlots + 2 * kRansStep * buf + 32 * (lane >> 1) + 4 * (lane & 1);
      const uint8_t *const tsy = lds + kLdsTab + 4 * rans::kProbScale;
      uint2 v = {0, 0};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t pr = *(const uint32_t *)(sl + 8 * j);   // slots of symbols 8 l + j and 8 l + 4 + j
        v.x |= (uint32_t)*(const uint16_t *)(tsy + (pr & 0xffff)) << (8 * j);
        v.y |= (uint32_t)*(const uint16_t *)(tsy + (pr >> 16)) << (8 * j);
      }
      const int64_t gi = fs0 + i0;
      auto byte = [&](int k) { return (uint8_t)((k < 4 ? v.x : v.y) >> (8 * (k & 3))); };
      if (t.nibbles) {
        const uint32_t b = (v.x & 0x0f) | ((v.x >> 4) & 0xf0) | ((v.x >> 8) & 0x0f00) | ((v.x >> 12) & 0xf000) |
                           ((v.y & 0x0f) << 16) | ((v.y << 12) & 0xf00000) | ((v.y & 0x0f0000) << 8) | ((v.y << 4) & 0xf0000000);
        glb_u8 *o = (glb_u8 *)(uintptr_t)(t.out + gi / 2);
        if (i0 + 8 <= ng && !((uintptr_t)o & 3)) *(__attribute__((address_space(1))) uint32_t *)o = b;
        else for (int k = 0; k < 4 && 2 * k < ng - i0; k++) o[k] = (uint8_t)(b >> (8 * k));
      } else if (t.stride == 1) {
        glb_u8 *o = (glb_u8 *)(uintptr_t)(t.out + gi);
        if (i0 + 8 <= ng && !((uintptr_t)o & 7)) {   // wide stores where aligned (always, for 16 MiB chunks)
          *(__attribute__((address_space(1))) uint32_t *)o = v.x;
          *(__attribute__((address_space(1))) uint32_t *)(o + 4) = v.y;
        } else {
          for (int k = 0; k < 8 && k < ng - i0; k++) o[k] = byte(k);
        }
      } else {
        glb_u8 *o = (glb_u8 *)(uintptr_t)t.out;
        for (int k = 0; k < 8 && i0 + k < ng; k++) o[(gi + k) * t.stride] = byte(k);
      }
    }
  };

  // the step loop, run by both waves with the same s0 and q (q from the decoder through LDS after every step)
  int prev_ng = 0, buf = 0;
  for (;; s0 += kRansStep, buf ^= 1) {
    const bool go = s0 < n && q + 2 * kRansStep + 8 <= lim;   // this step's bytes are all in HBM
    const int ng = go ? (int)std::min<int64_t>(kRansStep, n - s0) : 0;
    if (wave == 1) {
      if (prev_ng) flush(s0 - kRansStep, prev_ng, buf ^ 1);
      if (go) refill();
    } else if (go && lane < 4) {
      // the groups run on lanes 0..3 alone (the ballots then hold just the four states' bits).  A single wave
      // issues about one instruction per 5-6 cycles (measured), so a group costs its instruction count plus the
      // table reads' exposed latency; the stream offset lives in a VGPR (two v_bcnt per group, the window address
      // without a copy).  Every LDS access of the loop is written out with its waits.  A group issues its two table
      // reads (freq, m - cum) first; in their latency it adds the previous group's byte counts to the stream offset
      // and reads its window there; it waits for the table (lgkmcnt(1)), and for the window just before the bytes
      // are picked out of it (lgkmcnt(0)).  Only the table reads and the state's own arithmetic are on the chain from
      // one group to the next.  The symbols are not read here: each group's slot (as 2m, the table offset) stays in
      // a register, four groups leave in one 8-byte store, and wave 1 maps the slots to symbols.
      uint32_t qv = (uint32_t)q;
      asm volatile("" : "+v"(qv));
      uint32_t b1p = 0, b2p = 0;   // the previous group's renormalisation ballots
      // one group of four symbols, returning its slots; MASKED: the step's last group may hold fewer (lanes past it
      // keep their state)
      auto group = [&](int g, auto masked) {
        const uint32_t a = (st & (rans::kProbScale - 1)) << 1;
        uint32_t fq, bi;
        uint2 win;
        asm volatile("ds_read_u16 %0, %2 offset:%3\n\tds_read_u16 %1, %2 offset:%4"
                     : "=&v"(fq), "=&v"(bi) : "v"(a), "i"(kLdsTab), "i"(kLdsTab + 2 * rans::kProbScale));
        asm volatile("v_bcnt_u32_b32 %0, %1, %0\n\tv_bcnt_u32_b32 %0, %2, %0" : "+v"(qv) : "s"(b1p), "s"(b2p));
        asm volatile("ds_read_b64 %0, %1" : "=v"(win) : "v"(qv & (kRansRing - 1)));   // stream bytes qv .. qv + 7
        const uint32_t hs = st >> rans::kProbBits;
        asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(fq), "+v"(bi) : "v"(hs));
        __builtin_assume(fq <= (uint32_t)rans::kProbScale); __builtin_assume(bi < (uint32_t)rans::kProbScale);
        __builtin_assume(hs < (1u << 20));
        uint32_t x = fq * hs + bi;   // freq <= 2^12, x >> 12 < 2^20: one 24-bit multiply-add
        // renormalisation bytes: 2 below 2^15, 1 below 2^23 (x >= 2^11 and < 2^31 here).  Each count is a ballot; a
        // lane's byte offset is the bits of both ballots below it (mbcnt), the group's total their popcount
        const bool c1 = x < (1u << 23), c2 = x < (1u << 15);
        uint32_t b1 = (uint32_t)__builtin_amdgcn_ballot_w64(c1), b2 = (uint32_t)__builtin_amdgcn_ballot_w64(c2);
        const uint32_t lm = decltype(masked)::value ? (1u << (ng - g)) - 1u : 0xfu;
        if (decltype(masked)::value) { b1 &= lm; b2 &= lm; }
        const uint32_t excl = __builtin_amdgcn_mbcnt_lo(b2, __builtin_amdgcn_mbcnt_lo(b1, 0u));
        const uint32_t sel = excl * 0x101u + 0x0c0c0001u;
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(win) : "v"(sel));
        // the lane's bytes b0 = window[excl], b1 = window[excl + 1] into bytes 1, 0 of w (v_perm; selector 0x0c
        // gives 0), then the renormalised state is a byte permutation of x and w: x, x << 8 | b0, x << 16 | b0 << 8 | b1
        const uint32_t w = __builtin_amdgcn_perm(win.y, win.x, sel);
        x = __builtin_amdgcn_perm(x, w, c1 ? (c2 ? 0x05040100u : 0x06050401u) : 0x07060504u);
        if (decltype(masked)::value) {
          const uint32_t keep = (uint32_t)0 - ((lm >> lane) & 1u);
          st = (x & keep) | (st & ~keep);
        } else {
          st = x;
        }
        b1p = b1; b2p = b2;
        return a;
      };
      // slot staging: groups 4k .. 4k + 3 of the step form batch k; lane j stores its four slots at
      // 32 k + 8 j of the step's buffer (symbol 4 g + j of the step is batch g / 4, lane j, entry g % 4)
      uint32_t sp = kLdsSlots + 2 * kRansStep * buf + 8 * lane;
      const int nfull = ng & ~3;
      int g = 0;
      for (; g + 16 <= nfull; g += 16) {
        const uint32_t a0 = group(g, std::false_type{}), a1 = group(g + 4, std::false_type{});
        const uint32_t a2 = group(g + 8, std::false_type{}), a3 = group(g + 12, std::false_type{});
        asm volatile("ds_write_b64 %0, %1" : : "v"(sp), "v"(make_uint2(a0 | (a1 << 16), a2 | (a3 << 16))));
        sp += 32;
      }
      // the plane's last step: up to three more full groups and a partial one, one 16-bit store each
      for (int e = 0; g < ng; g += 4, e += 2) {
        const uint32_t a = g < nfull ? group(g, std::false_type{}) : group(g, std::true_type{});
        asm volatile("ds_write_b16 %0, %1" : : "v"(sp + e), "v"(a));
      }
      asm volatile("v_bcnt_u32_b32 %0, %1, %0\n\tv_bcnt_u32_b32 %0, %2, %0\n\ts_waitcnt lgkmcnt(0)" : "+v"(qv) : "s"(b1p), "s"(b2p) : "memory");
      if (lane == 0) qsh[buf] = qv;   // two slots: wave 1 reads this one after the barrier, before the next write to it
    }
    if (!go) break;
    __syncthreads();
    q = (uint64_t)qsh[buf];
    prev_ng = ng;
  }
  if (wave == 0) {
    if (lane < 4) S->st[lane] = st;
    if (lane == 0) {
      S->q = q; S->s0 = s0;
      if (s0 >= n) status[blockIdx.x] = q > end_off ? 1 : 0;
    }
  }
}

hipError_t launch_rans(const RansTaskDev *tasks, int ntasks, int *status, RansState *state, uint64_t avail, hipStream_t st) {
  if (ntasks <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_rans_decode, dim3(ntasks), dim3(128), 0, st, tasks, status, state, avail);
  return hipGetLastError();
}

// ------------------------------------------------------------------ host side: many blobs, one staging buffer
void RansBatch::add(const uint8_t *blob, size_t len, void *out, size_t out_cap) {
  const uint64_t raw = rans::raw_size(blob, len);
  if (raw > out_cap) throw std::runtime_error("rans: decoded size exceeds the destination");
  items_.push_back({blob, len, (uint8_t *)out, coded_});
  coded_ += (len + 15) & ~(size_t)15;
  raw_ += raw;
}

// a wave reads up to kRansAhead + kRansBlk bytes from the block holding its stream offset, and at most kRansBlk + 16
// past its plane's end
static constexpr size_t kRansSlack = kRansAhead + 2 * kRansBlk + 64;

uint64_t RansBatch::default_round() {
  const char *e = getenv("QPH_RANS_ROUND");
  return e ? (uint64_t)strtoull(e, nullptr, 10) : (uint64_t)1 << 19;   // C3: 0.45 s load (1 MiB 0.47, 2 MiB 0.49)
}

void RansBatch::run(hipStream_t st, RansTiming *tm, uint64_t round_bytes) {
  if (items_.empty()) return;
  struct Seg { const uint8_t *src; size_t off, len; };   // a plane's bytes: host source, staging offset
  std::vector<RansTaskDev> tasks;
  std::vector<Seg> segs;
  for (const Item &it : items_)
    for (const rans::PlaneTask &p : rans::plan(it.blob, it.len)) {
      RansTaskDev d{};
      d.plane = (const uint8_t *)(uintptr_t)(it.stage_off + p.hdr);   // rebased onto the staging buffer below
      d.out = it.out + p.out_off;
      d.n = p.n; d.comp_len = p.comp_len; d.nsym = p.nsym; d.stride = p.stride; d.nibbles = p.nibbles ? 1 : 0;
      tasks.push_back(d);
      segs.push_back({it.blob + p.hdr, it.stage_off + p.hdr, 4 + (size_t)p.comp_len});
    }
  // longest planes first, so the last waves to start are short ones
  std::stable_sort(tasks.begin(), tasks.end(), [](const RansTaskDev &a, const RansTaskDev &b) { return a.n > b.n; });
  size_t longest = 0;
  for (const Seg &g : segs) longest = std::max(longest, g.len);
  const int rounds = round_bytes ? (int)std::max<uint64_t>(1, (longest + round_bytes - 1) / round_bytes) : 1;
  uint8_t *stage = nullptr; RansTaskDev *dt = nullptr; int *dst = nullptr; RansState *dstate = nullptr;
  hipStream_t up = nullptr;
  std::vector<hipEvent_t> ev(rounds, nullptr);
  hipEvent_t e[4] = {};
  auto cleanup = [&] {
    // an error can come between launches: every copy and decode launch already queued finishes before the buffers go
    if (up) (void)hipStreamSynchronize(up);
    (void)hipStreamSynchronize(st);
    if (stage) (void)hipFree(stage);
    if (dt) (void)hipFree(dt);
    if (dst) (void)hipFree(dst);
    if (dstate) (void)hipFree(dstate);
    for (hipEvent_t &x : e) if (x) (void)hipEventDestroy(x);
    for (hipEvent_t &x : ev) if (x) (void)hipEventDestroy(x);
    if (up) (void)hipStreamDestroy(up);
  };
  try {
    auto ck = [](hipError_t r, const char *what) { if (r != hipSuccess) throw std::runtime_error(std::string("rans: ") + what + ": " + hipGetErrorString(r)); };
    for (hipEvent_t &x : e) ck(hipEventCreate(&x), "event");
    for (hipEvent_t &x : ev) ck(hipEventCreateWithFlags(&x, hipEventDisableTiming), "event");
    ck(hipStreamCreateWithFlags(&up, hipStreamNonBlocking), "copy stream");
    ck(hipMalloc(&stage, coded_ + kRansSlack), "staging allocation");
    ck(hipMalloc(&dt, tasks.size() * sizeof(RansTaskDev) + 1), "task allocation");
    ck(hipMalloc(&dst, tasks.size() * sizeof(int) + 4), "status allocation");
    ck(hipMalloc(&dstate, tasks.size() * sizeof(RansState) + 8), "state allocation");
    for (RansTaskDev &d : tasks) d.plane = stage + (uintptr_t)d.plane;
    // the task table, the status words and the staging slack go first, on the decode stream
    ck(hipMemcpyAsync(dt, tasks.data(), tasks.size() * sizeof(RansTaskDev), hipMemcpyHostToDevice, st), "task upload");
    ck(hipMemsetAsync(dst, 0, tasks.size() * sizeof(int), st), "status clear");
    ck(hipMemsetAsync(dstate, 0xff, tasks.size() * sizeof(RansState), st), "state clear");   // s0 = -1: not started
    ck(hipMemsetAsync(stage + coded_, 0, kRansSlack, st), "staging clear");
    ck(hipEventRecord(e[0], up), "event");
    for (int r = 0; r < rounds; r++) {
      const uint64_t lo = rounds == 1 ? 0 : (uint64_t)r * round_bytes, hi = rounds == 1 ? ~0ull : lo + round_bytes;
      for (const Seg &g : segs)
        if (lo < g.len) {
          const size_t n = (size_t)std::min<uint64_t>(g.len, hi) - (size_t)lo;
          ck(hipMemcpyAsync(stage + g.off + lo, g.src + lo, n, hipMemcpyHostToDevice, up), "upload");
        }
      ck(hipEventRecord(ev[r], up), "event");
      if (r == rounds - 1) ck(hipEventRecord(e[1], up), "event");
      ck(hipStreamWaitEvent(st, ev[r], 0), "stream wait");
      if (r == 0) ck(hipEventRecord(e[2], st), "event");
      ck(launch_rans(dt, (int)tasks.size(), dst, dstate, r == rounds - 1 ? ~0ull : hi, st), "decode launch");
    }
    ck(hipEventRecord(e[3], st), "event");
    std::vector<int> status(tasks.size());
    ck(hipMemcpyAsync(status.data(), dst, status.size() * sizeof(int), hipMemcpyDeviceToHost, st), "status copy");
    ck(hipStreamSynchronize(st), "decode");
    for (int s : status) {
      if (s == 2) throw std::runtime_error("rans: decoder LDS layout (the ring must start at LDS address 0)");
      if (s) throw std::runtime_error("rans: stream overrun");
    }
    if (tm) {
      tm->planes = (int)tasks.size(); tm->rounds = rounds; tm->coded = coded_; tm->raw = raw_;
      ck(hipEventElapsedTime(&tm->upload_ms, e[0], e[1]), "event");
      ck(hipEventElapsedTime(&tm->decode_ms, e[2], e[3]), "event");
      ck(hipEventElapsedTime(&tm->total_ms, e[0], e[3]), "event");
    }
  } catch (...) { cleanup(); items_.clear(); coded_ = raw_ = 0; throw; }
  cleanup();
  items_.clear(); coded_ = raw_ = 0;
}

}  // namespace qph
