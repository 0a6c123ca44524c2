#include "container.hpp"

#include "rans.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdio>
#include <cstring>
#include <stdexcept>

namespace qph {

namespace {

// file layout constants of the QPACK container: 16-byte header (magic, entry count, reserved), 72-byte table entries
// (NUL-padded name, offset, length), blobs placed on 64-byte boundaries
constexpr size_t kHeaderBytes = 16, kEntryBytes = 72, kNameBytes = 56;
constexpr uint64_t kBlobAlign = 64;

uint64_t le_u64(const uint8_t *p) { uint64_t v = 0; for (int i = 7; i >= 0; i--) v = (v << 8) | p[i]; return v; }
uint32_t le_u32(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
void put_u32(std::vector<uint8_t> &o, uint32_t v) { for (int i = 0; i < 4; i++) o.push_back((uint8_t)(v >> (8 * i))); }
void put_u64(std::vector<uint8_t> &o, uint64_t v) { for (int i = 0; i < 8; i++) o.push_back((uint8_t)(v >> (8 * i))); }
uint64_t align_up(uint64_t v) { return (v + kBlobAlign - 1) / kBlobAlign * kBlobAlign; }

// 1, 2 or 3 for the magics "QPACK1\0\0" .. "QPACK3\0\0"; 0 for anything else
int container_version(const uint8_t *p) {
  static const char stem[5] = {'Q', 'P', 'A', 'C', 'K'};
  for (int i = 0; i < 5; i++) if (p[i] != (uint8_t)stem[i]) return 0;
  if (p[6] || p[7] || p[5] < '1' || p[5] > '3') return 0;
  return p[5] - '0';
}

float f16_value(const uint8_t *p) { uint16_t h = (uint16_t)(p[0] | p[1] << 8); return (float)__builtin_bit_cast(_Float16, h); }

}  // namespace

Container::Container(const std::string &path) {
  fd_ = open(path.c_str(), O_RDONLY);
  if (fd_ < 0) throw std::runtime_error("qpack: cannot open " + path + ": " + strerror(errno));
  struct stat st{};
  if (fstat(fd_, &st) != 0) throw std::runtime_error("qpack: cannot stat " + path + ": " + strerror(errno));
  size_ = (size_t)st.st_size;
  if (size_ < kHeaderBytes) throw std::runtime_error("qpack: " + path + " is too short to be a QPACK container");
  void *m = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
  if (m == MAP_FAILED) throw std::runtime_error("qpack: cannot map " + path + ": " + strerror(errno));
  map_ = (uint8_t *)m;
  version_ = container_version(map_);
  if (!version_) throw std::runtime_error("qpack: " + path + " is not a QPACK container (bad magic)");
  const uint32_t entries = le_u32(map_ + 8);
  if (kHeaderBytes + (uint64_t)kEntryBytes * entries > size_)
    throw std::runtime_error("qpack: " + path + ": the table of contents runs past the end of the file");
  for (uint32_t i = 0; i < entries; i++) {
    const uint8_t *e = map_ + kHeaderBytes + (size_t)kEntryBytes * i;
    size_t nl = 0;
    while (nl < kNameBytes && e[nl]) nl++;
    const std::string name((const char *)e, nl);
    const uint64_t off = le_u64(e + kNameBytes), len = le_u64(e + kNameBytes + 8);
    if (off > size_ || len > size_ - off)
      throw std::runtime_error("qpack: " + path + ": the table of contents points outside the file (" + name + ")");
    toc_[name] = {off, len};
  }
  auto parse = [&](const char *name) { size_t l; const uint8_t *p = blob(name, &l); return JNode::read((const char *)p, l); };
  manifest_ = parse("manifest.json");
  config_ = parse("config.json");
  for (const JNode &e : manifest_.get("encoded").items()) {
    if (!toc_.count(e.text())) throw std::runtime_error("qpack: coded blob " + e.text() + " is not in the file");
    coded_[e.text()] = true;
  }
  // length of blob b as the loader sees it: the raw length behind a coded blob (its header carries it, chunked or not)
  auto open_blob = [&](const std::string &b, const void **p, uint64_t *coded) -> uint64_t {
    size_t l;
    *p = blob(b, &l);
    if (!coded_.count(b)) return l;
    *coded = l;
    return rans::raw_size((const uint8_t *)*p, l);
  };
  for (const JNode &e : manifest_.get("tensors").items()) {
    TensorView t;
    t.name = e.get("name").text();
    for (const JNode &s : e.get("shape").items()) t.shape.push_back(s.int_or(0));
    const std::string &kind = e.get("kind").text();
    const uint64_t len = open_blob(e.get("blob").text(), &t.data, &t.data_coded);
    const int64_t rows = t.rows(), cols = t.cols();
    auto short_blob = [&]() { return std::runtime_error("qpack: tensor " + t.name + " (" + kind + "): blob shorter than its shape"); };
    auto scale_blob = [&]() { return open_blob(e.get("scale").text(), &t.scale, &t.scale_coded); };
    auto group_of = [&](int64_t want) {
      if (e.get("group").int_or(want) != want) throw std::runtime_error("qpack: tensor " + t.name + ": only groups of " + std::to_string(want) + " are read");
      if (t.shape.size() != 2 || cols % want) throw std::runtime_error("qpack: tensor " + t.name + " must be 2-D with a whole number of groups per row");
    };
    if (kind == "f32") {
      t.kind = Kind::F32;
      if (len < 4ull * t.numel()) throw short_blob();
    } else if (kind == "f16") {
      t.kind = Kind::F16;
      if (len < 2ull * t.numel()) throw short_blob();
      if (t.shape.size() != 2) {   // vectors (norms, biases) are used as f32
        if (t.data_coded) throw std::runtime_error("qpack: tensor " + t.name + ": a coded f16 vector is not read by the HIP loader");
        std::vector<float> wide((size_t)t.numel());
        const uint8_t *src = (const uint8_t *)t.data;
        for (size_t i = 0; i < wide.size(); i++) wide[i] = f16_value(src + 2 * i);
        widened_.push_back(std::move(wide));
        t.data = widened_.back().data();
        t.kind = Kind::F32;
      }
    } else if (kind == "q8") {
      t.kind = Kind::Q8;
      if (t.shape.size() != 2) throw std::runtime_error("qpack: tensor " + t.name + " (q8) must be 2-D");
      if (len < (uint64_t)(rows * cols) || scale_blob() < 4ull * rows) throw short_blob();
    } else if (kind == "q4") {
      t.kind = Kind::Q4;
      group_of(32);
      if (len < (uint64_t)(rows * cols / 2) || scale_blob() < 2ull * rows * (cols / 32)) throw short_blob();
    } else if (kind == "q1") {   // /root/reference/QPACK2.md:18; whole 128-column groups on the GPU path
      t.kind = Kind::Q1;
      group_of(128);
      if (len < (uint64_t)(rows * cols / 8) || scale_blob() < 2ull * rows * (cols / 128)) throw short_blob();
    } else {
      throw std::runtime_error("qpack: tensor " + t.name + ": kind '" + kind + "' is not read by the HIP loader");
    }
    tensors_[t.name] = std::move(t);
  }
}

Container::~Container() {
  if (map_) munmap(map_, size_);
  if (fd_ >= 0) ::close(fd_);
}

const uint8_t *Container::blob(const std::string &n, size_t *len) const {
  auto it = toc_.find(n);
  if (it == toc_.end()) throw std::runtime_error("qpack: the file has no blob " + n);
  if (len) *len = it->second.second;
  return map_ + it->second.first;
}
std::vector<std::string> Container::blob_names() const {   // in the order the blobs lie in the file
  std::vector<const std::pair<const std::string, std::pair<uint64_t, uint64_t>> *> e;
  for (const auto &kv : toc_) e.push_back(&kv);
  std::stable_sort(e.begin(), e.end(), [](auto *a, auto *b) { return a->second.first < b->second.first; });
  std::vector<std::string> names;
  for (auto *x : e) names.push_back(x->first);
  return names;
}
const TensorView *Container::get(const std::string &n) const { auto it = tensors_.find(n); return it == tensors_.end() ? nullptr : &it->second; }
const TensorView &Container::at(const std::string &n) const {
  const TensorView *t = get(n);
  if (!t) throw std::runtime_error("qpack: the model has no tensor " + n);
  return *t;
}

ContainerWriter::ContainerWriter(const std::string &path, const std::vector<std::pair<std::string, uint64_t>> &plan, const char magic[8])
    : plan_(plan), path_(path) {
  std::vector<uint8_t> head(magic, magic + 8);
  put_u32(head, (uint32_t)plan.size());
  put_u32(head, 0);
  uint64_t at = align_up(kHeaderBytes + kEntryBytes * plan.size());
  for (const auto &b : plan) {
    if (b.first.size() >= kNameBytes) throw std::runtime_error("qpack: blob name longer than 55 bytes: " + b.first);
    head.insert(head.end(), b.first.begin(), b.first.end());
    head.resize(head.size() + (kNameBytes - b.first.size()), 0);
    put_u64(head, at);
    put_u64(head, b.second);
    offs_.push_back(at);
    at = align_up(at + b.second);
  }
  f_ = fopen(path.c_str(), "wb");
  if (!f_) throw std::runtime_error("qpack: cannot create " + path + ": " + strerror(errno));
  if (fwrite(head.data(), 1, head.size(), f_) != head.size()) throw std::runtime_error("qpack: short write to " + path);
  pos_ = head.size();
}
ContainerWriter::~ContainerWriter() { if (f_) fclose(f_); }
void ContainerWriter::write(const std::string &name, const void *data, uint64_t len) {
  if (next_ >= plan_.size() || plan_[next_].first != name || plan_[next_].second != len)
    throw std::runtime_error("qpack: writer: blob " + name + " does not follow the planned order and size");
  const std::vector<char> fill((size_t)(offs_[next_] - pos_), 0);   // zeros up to the blob's aligned offset
  if (!fill.empty() && fwrite(fill.data(), 1, fill.size(), f_) != fill.size()) throw std::runtime_error("qpack: short write to " + path_);
  if (len && fwrite(data, 1, len, f_) != len) throw std::runtime_error("qpack: short write to " + path_);
  pos_ = offs_[next_] + len;
  next_++;
}
void ContainerWriter::close() {
  if (next_ != plan_.size()) throw std::runtime_error("qpack: writer: " + path_ + " closed with blobs missing");
  const int rc = f_ ? fclose(f_) : 0;
  f_ = nullptr;
  if (rc != 0) throw std::runtime_error("qpack: short write to " + path_);
}

}  // namespace qph
