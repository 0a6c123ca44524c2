// QPACK1 / QPACK2 single-file containers: a read-only mmap view and a streaming writer.
//
// On-disk layout (the reference format, /root/reference/QPACK2.md:6-12, reader /root/reference/src/container.cpp:22-90):
//   magic "QPACK1\0\0" | "QPACK2\0\0" (8 bytes), count u32, pad u32,
//   count x { name[56] NUL-padded, offset u64, length u64 }, blobs each aligned to 64 bytes.
// manifest.json lists the tensors ({name, shape, kind, blob, scale, group}); config.json holds the model config.
// Tensor kinds read here: f32, f16 (1-D f16 is widened to f32 at load, as the reference does), q8, q4, q1 (2-D,
// cols % 128 == 0).
// QPACK3 (/root/reference/QPACK2.md:30-51): the blobs named in the manifest's "encoded" list hold rANS streams.  Unlike
// the reference Container, which decodes them on the CPU at load (/root/reference/src/container.cpp:94-121), this view
// leaves them coded: a tensor records the coded lengths, and the model decodes them in HBM (hip/rans_decode.hip).
#pragma once
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "json.hpp"

namespace qph {

enum class Kind { F32, F16, Q8, Q4, Q1 };

struct TensorView {
  std::string name;
  std::vector<int64_t> shape;
  Kind kind = Kind::F32;
  const void *data = nullptr;    // q8: int8 [rows, cols]; q4: u8 [rows, cols / 2]; q1: sign bits [rows, cols / 8]; f32 / f16
  const void *scale = nullptr;   // q8: f32 [rows]; q4: f16 [rows, cols / 32]; q1: f16 [rows, cols / 128]
  uint64_t data_coded = 0;       // QPACK3: > 0 when `data` is a rANS blob of this many bytes
  uint64_t scale_coded = 0;      // QPACK3: > 0 when `scale` is a rANS blob of this many bytes
  int64_t rows() const { return shape.empty() ? 0 : shape[0]; }
  int64_t cols() const {
    if (shape.size() == 1) return shape[0];
    int64_t c = 1; for (size_t i = 1; i < shape.size(); i++) c *= shape[i];
    return c;
  }
  int64_t numel() const { int64_t n = 1; for (auto s : shape) n *= s; return n; }
};

class Container {
 public:
  explicit Container(const std::string &path);
  ~Container();
  Container(const Container &) = delete;
  Container &operator=(const Container &) = delete;
  int version() const { return version_; }
  const JNode &config() const { return config_; }
  const JNode &manifest() const { return manifest_; }
  bool has_blob(const std::string &n) const { return toc_.count(n) > 0; }
  bool is_coded(const std::string &n) const { return coded_.count(n) > 0; }
  std::vector<std::string> blob_names() const;                    // in file order
  const uint8_t *blob(const std::string &n, size_t *len) const;   // throws when absent
  const TensorView *get(const std::string &n) const;              // nullptr when absent
  const TensorView &at(const std::string &n) const;               // throws when absent
  size_t file_size() const { return size_; }

 private:
  int fd_ = -1;
  uint8_t *map_ = nullptr;
  size_t size_ = 0;
  int version_ = 0;
  std::map<std::string, std::pair<uint64_t, uint64_t>> toc_;
  std::map<std::string, bool> coded_;
  JNode manifest_, config_;
  std::map<std::string, TensorView> tensors_;
  std::vector<std::vector<float>> widened_;   // storage of 1-D f16 tensors converted to f32
};

// Streaming writer: the table of contents is laid out from a plan of (blob name, byte length) first, then blobs are
// appended in plan order, so multi-GB files are written without holding them in memory.
class ContainerWriter {
 public:
  ContainerWriter(const std::string &path, const std::vector<std::pair<std::string, uint64_t>> &plan, const char magic[8]);
  ~ContainerWriter();
  void write(const std::string &name, const void *data, uint64_t len);   // must follow the plan order and lengths
  void close();

 private:
  FILE *f_ = nullptr;
  std::vector<std::pair<std::string, uint64_t>> plan_;
  std::vector<uint64_t> offs_;
  size_t next_ = 0;
  uint64_t pos_ = 0;
  std::string path_;
};

}  // namespace qph
