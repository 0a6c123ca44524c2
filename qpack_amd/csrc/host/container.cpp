#include "container.hpp"

#include "rans.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <stdexcept>

namespace qph {

static float half_to_float(uint16_t h) { _Float16 v; memcpy(&v, &h, 2); return (float)v; }

Container::Container(const std::string &path) {
  fd_ = open(path.c_str(), O_RDONLY);
  if (fd_ < 0) throw std::runtime_error("cannot open " + path);
  struct stat st;
  if (fstat(fd_, &st) != 0) throw std::runtime_error("cannot stat " + path);
  size_ = (size_t)st.st_size;
  if (size_ < 16) throw std::runtime_error("not a QPACK file: " + path);
  map_ = (uint8_t *)mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
  if (map_ == MAP_FAILED) { map_ = nullptr; throw std::runtime_error("mmap failed: " + path); }
  if (!memcmp(map_, "QPACK1\0\0", 8)) version_ = 1;
  else if (!memcmp(map_, "QPACK2\0\0", 8)) version_ = 2;
  else if (!memcmp(map_, "QPACK3\0\0", 8)) version_ = 3;
  else throw std::runtime_error("not a QPACK1/QPACK2/QPACK3 file: " + path);
  uint32_t n; memcpy(&n, map_ + 8, 4);
  if (16 + 72ull * n > size_) throw std::runtime_error("corrupt table of contents: " + path);
  for (uint32_t i = 0; i < n; i++) {
    const uint8_t *e = map_ + 16 + 72ull * i;
    const std::string name((const char *)e, strnlen((const char *)e, 56));
    uint64_t off, len; memcpy(&off, e + 56, 8); memcpy(&len, e + 64, 8);
    if (off > size_ || len > size_ - off) throw std::runtime_error("corrupt table of contents: " + name);
    toc_[name] = {off, len};
  }
  auto json_blob = [&](const char *b) { size_t l; const uint8_t *p = blob(b, &l); return Json::parse((const char *)p, l); };
  manifest_ = json_blob("manifest.json");
  config_ = json_blob("config.json");
  for (const Json &e : manifest_["encoded"].arr) {
    if (!toc_.count(e.string())) throw std::runtime_error("missing blob " + e.string());
    coded_[e.string()] = true;
  }
  // a coded blob's length check uses its raw length (the u32 after codec and planes, the same for chunked blobs)
  auto view = [&](const std::string &b, const void **p, uint64_t *coded) {
    size_t l; *p = blob(b, &l);
    if (!coded_.count(b)) return (uint64_t)l;
    *coded = l;
    return (uint64_t)rans::raw_size((const uint8_t *)*p, l);
  };
  for (const Json &e : manifest_["tensors"].arr) {
    TensorView t; t.name = e["name"].string();
    for (const Json &s : e["shape"].arr) t.shape.push_back(s.integer(0));
    const std::string &kind = e["kind"].string();
    const uint64_t len = view(e["blob"].string(), &t.data, &t.data_coded);
    const int64_t rows = t.rows(), cols = t.cols(); uint64_t sl = 0;
    if (kind == "f32") {
      t.kind = Kind::F32;
      if (len < 4ull * t.numel()) throw std::runtime_error("tensor " + t.name + ": blob too short");
    } else if (kind == "f16") {
      t.kind = Kind::F16;
      if (len < 2ull * t.numel()) throw std::runtime_error("tensor " + t.name + ": blob too short");
      if (t.shape.size() != 2 && t.data_coded) throw std::runtime_error("tensor " + t.name + ": a coded f16 vector is not read by the HIP loader");
      if (t.shape.size() != 2) {   // norms / biases: widened to f32 once
        std::vector<float> w((size_t)t.numel());
        for (size_t i = 0; i < w.size(); i++) { uint16_t h; memcpy(&h, (const uint8_t *)t.data + 2 * i, 2); w[i] = half_to_float(h); }
        widened_.push_back(std::move(w)); t.data = widened_.back().data(); t.kind = Kind::F32;
      }
    } else if (kind == "q8") {
      t.kind = Kind::Q8; sl = view(e["scale"].string(), &t.scale, &t.scale_coded);
      if (t.shape.size() != 2 || len < (size_t)(rows * cols) || sl < 4ull * rows) throw std::runtime_error("q8 tensor " + t.name + ": bad shape or blob size");
    } else if (kind == "q4") {
      t.kind = Kind::Q4; sl = view(e["scale"].string(), &t.scale, &t.scale_coded);
      if (e["group"].integer(32) != 32) throw std::runtime_error("q4 tensor " + t.name + ": only group 32 is supported");
      if (t.shape.size() != 2 || cols % 32) throw std::runtime_error("q4 tensor " + t.name + ": 2-D with cols % 32 == 0 required");
      if (len < (size_t)(rows * cols / 2) || sl < 2ull * rows * (cols / 32)) throw std::runtime_error("q4 tensor " + t.name + ": blob too short");
    } else if (kind == "q1") {   // /root/reference/QPACK2.md:18; the GPU path needs whole 128-column groups
      t.kind = Kind::Q1; sl = view(e["scale"].string(), &t.scale, &t.scale_coded);
      if (e["group"].integer(128) != 128) throw std::runtime_error("q1 tensor " + t.name + ": only group 128 is supported");
      if (t.shape.size() != 2 || cols % 128) throw std::runtime_error("q1 tensor " + t.name + ": 2-D with cols % 128 == 0 required");
      if (len < (size_t)(rows * cols / 8) || sl < 2ull * rows * (cols / 128)) throw std::runtime_error("q1 tensor " + t.name + ": blob too short");
    } else throw std::runtime_error("tensor " + t.name + ": kind '" + kind + "' is not supported by the HIP loader");
    tensors_[t.name] = std::move(t);
  }
}

Container::~Container() {
  if (map_) munmap(map_, size_);
  if (fd_ >= 0) ::close(fd_);
}

const uint8_t *Container::blob(const std::string &n, size_t *len) const {
  auto it = toc_.find(n);
  if (it == toc_.end()) throw std::runtime_error("missing blob " + n);
  if (len) *len = it->second.second;
  return map_ + it->second.first;
}
std::vector<std::string> Container::blob_names() const {
  std::vector<std::pair<uint64_t, std::string>> v;
  for (auto &kv : toc_) v.push_back({kv.second.first, kv.first});
  std::sort(v.begin(), v.end());
  std::vector<std::string> o;
  for (auto &x : v) o.push_back(x.second);
  return o;
}
const TensorView *Container::get(const std::string &n) const { auto it = tensors_.find(n); return it == tensors_.end() ? nullptr : &it->second; }
const TensorView &Container::at(const std::string &n) const {
  const TensorView *t = get(n);
  if (!t) throw std::runtime_error("missing tensor " + n);
  return *t;
}

static const uint64_t kAlign = 64;

ContainerWriter::ContainerWriter(const std::string &path, const std::vector<std::pair<std::string, uint64_t>> &plan, const char magic[8])
    : plan_(plan), path_(path) {
  uint64_t off = (16 + 72 * plan.size() + kAlign - 1) / kAlign * kAlign;
  std::string head(magic, 8); const uint32_t n = (uint32_t)plan.size(), pad = 0;
  head.append((const char *)&n, 4); head.append((const char *)&pad, 4);
  for (auto &b : plan) {
    if (b.first.size() > 55) throw std::runtime_error("blob name too long: " + b.first);
    std::string nm = b.first; nm.resize(56, '\0');
    head += nm; head.append((const char *)&off, 8); head.append((const char *)&b.second, 8);
    offs_.push_back(off); off = (off + b.second + kAlign - 1) / kAlign * kAlign;
  }
  f_ = fopen(path.c_str(), "wb");
  if (!f_) throw std::runtime_error("cannot write " + path);
  if (fwrite(head.data(), 1, head.size(), f_) != head.size()) throw std::runtime_error("write failed: " + path);
  pos_ = head.size();
}
ContainerWriter::~ContainerWriter() { if (f_) fclose(f_); }
void ContainerWriter::write(const std::string &name, const void *data, uint64_t len) {
  if (next_ >= plan_.size() || plan_[next_].first != name || plan_[next_].second != len)
    throw std::runtime_error("container writer: blob " + name + " out of plan order");
  static const char zeros[kAlign] = {};
  const uint64_t gap = offs_[next_] - pos_;
  if (gap && fwrite(zeros, 1, gap, f_) != gap) throw std::runtime_error("write failed: " + path_);
  if (len && fwrite(data, 1, len, f_) != len) throw std::runtime_error("write failed: " + path_);
  pos_ = offs_[next_] + len; next_++;
}
void ContainerWriter::close() {
  if (next_ != plan_.size()) throw std::runtime_error("container writer: " + path_ + " closed before all blobs were written");
  if (f_ && fclose(f_) != 0) { f_ = nullptr; throw std::runtime_error("write failed: " + path_); }
  f_ = nullptr;
}

}  // namespace qph
