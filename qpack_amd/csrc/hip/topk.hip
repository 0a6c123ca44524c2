// Device top-M of a logits vector: the M largest (index, value) pairs in the sampler's order - value descending, the
// lower index first among equal values (top_m and the sort in Sampler::dist, /root/reference/src/sampler.cpp:12-27 and
// :41-42).  The host then applies its penalties / temperature / top-p to those M candidates, so it receives M pairs
// instead of V floats.
//
// Each pair is one 64-bit key whose ascending order is the sampler's order: the high word is the complement of the
// value's order-preserving unsigned image, the low word the index.  Rounds: every workgroup bitonic-sorts a chunk of
// 4096 keys in LDS and keeps its first M; the survivors form the next round's input, until one chunk is left, whose
// first M keys are the result.
#include <mutex>

#include "launch.hpp"

namespace qph {

constexpr int kTopkChunk = 4096, kTopkThreads = 1024;

__device__ __forceinline__ uint64_t topk_key(float v, int i) {
  // -0 compares equal to +0 (the index then decides, as in the sampler's comparison), so it takes +0's key
  const uint32_t b = v == 0.f ? 0u : __builtin_bit_cast(uint32_t, v);
  const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);   // ascending with the float value
  return ((uint64_t)(~k) << 32) | (uint32_t)i;
}
__device__ __forceinline__ float topk_val(uint64_t key) {
  const uint32_t k = ~(uint32_t)(key >> 32);
  return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// one chunk of n input keys (from x when keys_in is null) -> its M smallest keys at out + chunk * M, or, in the last
// round (idx != null, one chunk), decoded into idx[M] / val[M]
__global__ __launch_bounds__(kTopkThreads) void k_topk_chunk(const float *x, const uint64_t *keys_in, int n, int M,
                                                             uint64_t *out, int *idx, float *val) {
  __shared__ uint64_t s[kTopkChunk];
  const int tid = threadIdx.x, base = blockIdx.x * kTopkChunk;
#pragma unroll
  for (int j = 0; j < kTopkChunk / kTopkThreads; j++) {
    const int e = base + tid + j * kTopkThreads;
    s[tid + j * kTopkThreads] = e < n ? (keys_in ? keys_in[e] : topk_key(x[e], e)) : ~0ull;   // padding sorts last
  }
  __syncthreads();
  // bitonic sort, ascending: each thread owns the compare-exchanges of pairs (i, i ^ j) with i < i ^ j
  for (int k = 2; k <= kTopkChunk; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
#pragma unroll
      for (int q = 0; q < kTopkChunk / 2 / kTopkThreads; q++) {
        const int t = tid + q * kTopkThreads;                 // pair number
        const int i = 2 * t - (t & (j - 1));                  // lower element: bit j of i clear
        const int p = i + j;
        const bool up = (i & k) == 0;
        const uint64_t a = s[i], b = s[p];
        if ((a > b) == up) { s[i] = b; s[p] = a; }
      }
      __syncthreads();
    }
  for (int e = tid; e < M; e += kTopkThreads) {
    if (idx) { idx[e] = (int)(uint32_t)s[e]; val[e] = topk_val(s[e]); }
    else out[(size_t)blockIdx.x * M + e] = s[e];
  }
}

size_t topk_scratch_keys(int n, int M) { return (size_t)((n + kTopkChunk - 1) / kTopkChunk) * (size_t)M; }

hipError_t launch_topk(const float *x, int n, int M, uint64_t *buf_a, uint64_t *buf_b, int *idx, float *val,
                       hipStream_t st) {
  if (n <= 0 || M < 1 || M > kTopkMax || M > n) return hipErrorInvalidValue;
  const uint64_t *in = nullptr;
  uint64_t *out = buf_a, *spare = buf_b;
  int len = n;
  for (;;) {
    const int chunks = (len + kTopkChunk - 1) / kTopkChunk;
    const bool last = chunks == 1;
    hipLaunchKernelGGL(k_topk_chunk, dim3(chunks), dim3(kTopkThreads), 0, st, in ? nullptr : x, in, len, M, out,
                       last ? idx : nullptr, last ? val : nullptr);
    if (last) break;
    len = chunks * M;   // survivors (M per chunk; M <= kTopkChunk / 8, so every round shrinks the input 8 times or more)
    in = out;
    std::swap(out, spare);
  }
  return hipGetLastError();
}

// ---- the top-M without allocation (qph_topk_noalloc): the key buffers live in a file-scope device array, one copy per
// GPU, held until the process ends.  Its address comes from hipGetSymbolAddress once per device, with that device
// current (the array's name in host code is only a stand-in: passed to a kernel it would fault).  Calls that overlap
// on one GPU share the array and race; the array keeps the last call's keys (every round writes what the next reads,
// so nothing needs clearing).
constexpr int kTopkNoAllocMaxN = 262144;
constexpr size_t kTopkNoAllocKeys = (size_t)(kTopkNoAllocMaxN / kTopkChunk) * kTopkMax;   // per buffer: 32768 keys
static __device__ __align__(256) uint64_t scratch[2 * kTopkNoAllocKeys];                  // 512 KiB per GPU

static uint64_t *scratch_ptr(int dev) {
  static std::mutex mu;
  static uint64_t *ptrs[64] = {};
  if (dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
    ptrs[dev] = (uint64_t *)p;
  }
  return ptrs[dev];
}

hipError_t launch_topk_noalloc(const float *x, int n, int M, int *idx, float *val, hipStream_t st) {
  if (n <= 0 || n > kTopkNoAllocMaxN || M < 1 || M > kTopkMax || M > n) return hipErrorInvalidValue;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  uint64_t *base = scratch_ptr(dev);
  if (!base) return hipErrorInvalidSymbol;
  return launch_topk(x, n, M, base, base + kTopkNoAllocKeys, idx, val, st);
}

}  // namespace qph
