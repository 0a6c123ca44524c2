// QPACK3 static rANS: the host half.  The bulk decode runs on the GPU (hip/rans_decode.hip); the host parses each coded blob's
// headers into decode tasks (one per coded plane), validating them as the reference decoder does, and writes QPACK3
// files (the packer used to build coded inputs).
//
// Blob format (/root/reference/include/qpack/rans.h:1-8 and :115-124, /root/reference/QPACK2.md:30-51), little endian:
//   plain:   u8 codec (1 bytes, 2 nibbles) | u8 planes | u32 raw_len | per plane: u32 comp_len | u16 freq[nsym] | u32 state[4] | bytes
//   chunked: u8 3 | u8 0 | u32 raw_len | u32 chunk_raw | u32 nchunks | u32 comp_len[nchunks] | nchunks plain blobs
// codec 1: byte i of the raw data is symbol i / planes of plane i % planes (256-ary); codec 2: one plane, byte i = symbols
// 2i (low nibble) and 2i + 1 (high nibble), 16-ary.  12-bit frequencies summing to 4096, four interleaved 32-bit states
// (symbol i uses state i & 3), bytewise renormalisation into [2^23, 2^31).
#pragma once
#include <cstdint>
#include <string>
#include <vector>

namespace qph {
namespace rans {

constexpr uint32_t kProbBits = 12, kProbScale = 1u << kProbBits, kL = 1u << 23;

// one coded plane: decode n symbols from the plane whose comp_len field sits at byte `hdr` of the blob, into the raw
// output at `out_off` (codec 1: symbol i -> byte out_off + i * stride; codec 2: symbol i -> nibble i & 1 of byte
// out_off + i / 2)
struct PlaneTask {
  uint64_t hdr;       // offset of the plane's comp_len within the blob
  uint32_t comp_len;  // bytes after the comp_len field
  int nsym;           // 256 (codec 1) or 16 (codec 2)
  int64_t n;          // symbols
  uint64_t out_off;   // first output byte within the blob's raw data
  int stride;         // codec 1: planes; codec 2: 1
  bool nibbles;
};

// raw (decoded) length of a plain or chunked blob (rans.h:75)
uint64_t raw_size(const uint8_t *p, size_t len);
// the planes of a plain or chunked blob, checked as rans.h:53-62 / :94-113 check them (truncation, comp_len bounds,
// frequency sums, codec); throws std::runtime_error with the reference's messages.  The one check left to the decoder is
// the stream overrun (rans.h:66), which depends on the symbols.
std::vector<PlaneTask> plan(const uint8_t *p, size_t len);

// raw bytes -> a plain codec 1 / 2 blob (rans.h:21-49, :81-93)
std::vector<uint8_t> encode(const uint8_t *raw, size_t n, int codec, int planes);
// a chunked blob of the given chunks (rans.h:117-122)
std::vector<uint8_t> assemble_chunked(size_t n, size_t chunk_raw, const std::vector<std::vector<uint8_t>> &chunks);

// qpack-pack in out (all classes, /root/reference/tools/qpack-pack.cpp:43-84): QPACK2 -> QPACK3 with every q4 / q8 /
// scale / f16 / f32 blob coded (16 MiB chunks above 32 MiB) where that makes it smaller.  Returns the coded blob count.
int pack(const std::string &src, const std::string &dst, int threads);

}  // namespace rans
}  // namespace qph
