#include "rans.hpp"

#include <algorithm>
#include <atomic>
#include <cstring>
#include <map>
#include <stdexcept>
#include <thread>

#include "container.hpp"

namespace qph {
namespace rans {

static uint32_t get32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static void put32(std::vector<uint8_t> &o, uint32_t v) { for (int i = 0; i < 4; i++) o.push_back((uint8_t)(v >> (8 * i))); }

uint64_t raw_size(const uint8_t *p, size_t len) {
  if (len < 6) throw std::runtime_error("rans: short blob");
  return get32(p + 2);
}

// one plain blob at p[0, len) whose raw output starts at out_base; hdr offsets are relative to `origin`
static void plan_plain(const uint8_t *origin, const uint8_t *p, size_t len, uint64_t out_base, std::vector<PlaneTask> &t) {
  const uint64_t n = raw_size(p, len);
  const int codec = p[0], planes = p[1];
  auto plane = [&](size_t pos, int nsym, uint64_t cnt, uint64_t off, int stride, bool nib) -> size_t {
    const size_t avail = len - pos;
    if (avail < 4) throw std::runtime_error("rans: truncated");
    const uint32_t cl = get32(p + pos);
    if ((size_t)cl + 4 > avail || cl < 2u * nsym + 16) throw std::runtime_error("rans: truncated plane");
    uint32_t sum = 0;
    for (int i = 0; i < nsym; i++) sum += (uint32_t)p[pos + 4 + 2 * i] | ((uint32_t)p[pos + 5 + 2 * i] << 8);
    if (sum != kProbScale) throw std::runtime_error("rans: bad frequency table");
    if (cnt) t.push_back({(uint64_t)(p + pos - origin), cl, nsym, (int64_t)cnt, off, stride, nib});
    return (size_t)cl + 4;
  };
  size_t pos = 6;
  if (codec == 2) {
    plane(pos, 16, 2 * n, out_base, 1, true);
  } else if (codec == 1 && planes >= 1 && planes <= 4) {
    for (int k = 0; k < planes; k++) pos += plane(pos, 256, (n + planes - 1 - k) / planes, out_base + k, planes, false);
  } else {
    throw std::runtime_error("rans: unknown codec");
  }
}

std::vector<PlaneTask> plan(const uint8_t *p, size_t len) {
  std::vector<PlaneTask> t;
  if (len >= 1 && p[0] == 3) {
    if (len < 14) throw std::runtime_error("rans: short chunked blob");
    const uint64_t cr = get32(p + 6), nc = get32(p + 10);
    size_t pos = 14 + 4 * nc;
    if (pos > len) throw std::runtime_error("rans: truncated chunk table");
    const uint64_t n = get32(p + 2);
    for (uint64_t i = 0; i < nc; i++) {
      const size_t cl = get32(p + 14 + 4 * i);
      if (pos + cl > len) throw std::runtime_error("rans: truncated chunk");
      // a chunk writing past the blob's raw length would write past the caller's buffer (the reference trusts it)
      if (i * cr + raw_size(p + pos, cl) > n) throw std::runtime_error("rans: chunk beyond the raw length");
      plan_plain(p, p + pos, cl, i * cr, t);
      pos += cl;
    }
  } else {
    plan_plain(p, p, len, 0, t);
  }
  return t;
}

// the encoder's 12-bit table (rans.h:23-37): floor(h * 4096 / n), at least 1 for a present symbol; the most frequent
// symbol (first on ties) absorbs the difference, or, when that would leave it below 1, the largest frequency (first on
// ties) is decremented until the total is 4096
static void freqs(const uint8_t *sym, size_t n, int nsym, uint32_t *f) {
  uint64_t h[256] = {};
  for (size_t i = 0; i < n; i++) h[sym[i]]++;
  std::fill(f, f + nsym, 0u);
  if (n == 0) { f[0] = kProbScale; return; }
  int64_t sum = 0; int big = 0;
  for (int i = 0; i < nsym; i++) {
    if (!h[i]) continue;
    const uint32_t v = (uint32_t)(h[i] * kProbScale / n);
    f[i] = std::max(v, 1u); sum += f[i];
    if (h[i] > h[big]) big = i;
  }
  const int64_t rest = (int64_t)f[big] + kProbScale - sum;
  if (rest >= 1) { f[big] = (uint32_t)rest; return; }
  for (int64_t d = sum - kProbScale; d > 0; d--) {
    int m = 0;
    for (int i = 1; i < nsym; i++) if (f[i] > f[m]) m = i;
    if (f[m] <= 1) throw std::runtime_error("rans: cannot normalise frequencies");
    f[m]--;
  }
}

static void encode_plane(const std::vector<uint8_t> &sym, int nsym, std::vector<uint8_t> &o) {
  uint32_t f[256], c[257];
  freqs(sym.data(), sym.size(), nsym, f);
  c[0] = 0;
  for (int i = 0; i < nsym; i++) c[i + 1] = c[i] + f[i];
  std::vector<uint8_t> tail;   // renormalisation bytes, produced last-first
  tail.reserve(sym.size() + 16);
  uint32_t x[4] = {kL, kL, kL, kL};
  for (size_t i = sym.size(); i-- > 0;) {
    uint32_t &st = x[i & 3];
    const uint32_t s = sym[i], fr = f[s], xmax = ((kL >> kProbBits) << 8) * fr;
    while (st >= xmax) { tail.push_back((uint8_t)st); st >>= 8; }
    st = ((st / fr) << kProbBits) + (st % fr) + c[s];
  }
  const size_t at = o.size();
  put32(o, 0);
  for (int i = 0; i < nsym; i++) { o.push_back((uint8_t)f[i]); o.push_back((uint8_t)(f[i] >> 8)); }
  for (uint32_t v : x) put32(o, v);
  o.insert(o.end(), tail.rbegin(), tail.rend());
  const uint32_t cl = (uint32_t)(o.size() - at - 4);
  for (int i = 0; i < 4; i++) o[at + i] = (uint8_t)(cl >> (8 * i));
}

std::vector<uint8_t> encode(const uint8_t *raw, size_t n, int codec, int planes) {
  std::vector<uint8_t> o = {(uint8_t)codec, (uint8_t)planes};
  put32(o, (uint32_t)n);
  if (codec == 2) {
    std::vector<uint8_t> s(2 * n);
    for (size_t i = 0; i < n; i++) { s[2 * i] = raw[i] & 15; s[2 * i + 1] = raw[i] >> 4; }
    encode_plane(s, 16, o);
  } else if (codec == 1 && planes >= 1 && planes <= 4) {
    for (int k = 0; k < planes; k++) {
      std::vector<uint8_t> s;
      s.reserve(n / planes + 1);
      for (size_t i = k; i < n; i += planes) s.push_back(raw[i]);
      encode_plane(s, 256, o);
    }
  } else {
    throw std::runtime_error("rans: unknown codec");
  }
  return o;
}

std::vector<uint8_t> assemble_chunked(size_t n, size_t chunk_raw, const std::vector<std::vector<uint8_t>> &chunks) {
  std::vector<uint8_t> o = {3, 0};
  put32(o, (uint32_t)n); put32(o, (uint32_t)chunk_raw); put32(o, (uint32_t)chunks.size());
  for (auto &c : chunks) put32(o, (uint32_t)c.size());
  for (auto &c : chunks) o.insert(o.end(), c.begin(), c.end());
  return o;
}

int pack(const std::string &src_path, const std::string &dst_path, int threads) {
  Container src(src_path);
  if (src.version() != 2) throw std::runtime_error(src_path + ": pack needs a QPACK2 file");
  struct Plan { int codec, planes; };
  std::map<std::string, Plan> plan;   // qpack-pack's classes, all selected (tools/qpack-pack.cpp:43-53)
  for (const JNode &e : src.manifest().get("tensors").items()) {
    const std::string &k = e.get("kind").text(), &b = e.get("blob").text();
    if (k == "q4") { plan[b] = {2, 1}; plan[e.get("scale").text()] = {1, 2}; }
    else if (k == "q8") plan[b] = {1, 1};
    else if (k == "mxfp4") { plan[b] = {1, 1}; plan[e.get("scale").text()] = {1, 1}; }
    else if (k == "q1" || k == "q8g") { plan[b] = {1, 1}; plan[e.get("scale").text()] = {1, 2}; }
    else if (k == "f16") plan[b] = {1, 2};
    else if (k == "f32") plan[b] = {1, 4};
  }
  const size_t kThresh = 32u << 20, kChunk = 16u << 20;
  const std::vector<std::string> names = src.blob_names();
  struct Job { size_t blob; size_t off, len; std::vector<uint8_t> out; };
  std::vector<Job> jobs;
  std::vector<std::pair<size_t, size_t>> range(names.size(), {0, 0});   // blob -> [first job, end)
  for (size_t i = 0; i < names.size(); i++) {
    size_t len; src.blob(names[i], &len);
    if (!plan.count(names[i]) || names[i] == "manifest.json" || !len) continue;
    range[i].first = jobs.size();
    if (len > kThresh) for (size_t o = 0; o < len; o += kChunk) jobs.push_back({i, o, std::min(kChunk, len - o), {}});
    else jobs.push_back({i, 0, len, {}});
    range[i].second = jobs.size();
  }
  std::atomic<size_t> next{0};
  std::vector<std::string> errs(std::max(1, threads));
  std::vector<std::thread> th;
  for (int t = 0; t < std::max(1, threads); t++)
    th.emplace_back([&, t] {
      try {
        for (size_t j; (j = next++) < jobs.size();) {
          Job &jb = jobs[j];
          const Plan &pl = plan[names[jb.blob]];
          jb.out = encode(src.blob(names[jb.blob], nullptr) + jb.off, jb.len, pl.codec, pl.planes);
        }
      } catch (std::exception &e) { errs[t] = e.what(); }
    });
  for (auto &x : th) x.join();
  for (auto &e : errs) if (!e.empty()) throw std::runtime_error("pack: " + e);
  std::vector<std::vector<uint8_t>> coded(names.size());
  JNode enc = JNode(JNode::List{});
  for (size_t i = 0; i < names.size(); i++) {
    if (range[i].first == range[i].second) continue;
    size_t len; src.blob(names[i], &len);
    std::vector<uint8_t> c;
    if (len > kThresh) {
      std::vector<std::vector<uint8_t>> ch;
      for (size_t j = range[i].first; j < range[i].second; j++) ch.push_back(std::move(jobs[j].out));
      c = assemble_chunked(len, kChunk, ch);
    } else {
      c = std::move(jobs[range[i].first].out);
    }
    if (c.size() < len) { coded[i] = std::move(c); enc.append(JNode(names[i])); }   // blobs that do not shrink stay raw
  }
  JNode man = src.manifest();
  man.put("encoded", enc);
  man.put("format", "QPACK3");
  const std::string mtext = man.serialize();
  std::vector<std::pair<std::string, uint64_t>> layout;
  for (size_t i = 0; i < names.size(); i++) {
    size_t len; src.blob(names[i], &len);
    layout.push_back({names[i], names[i] == "manifest.json" ? mtext.size() : !coded[i].empty() ? coded[i].size() : len});
  }
  ContainerWriter w(dst_path, layout, "QPACK3\0\0");
  for (size_t i = 0; i < names.size(); i++) {
    size_t len; const uint8_t *p = src.blob(names[i], &len);
    if (names[i] == "manifest.json") w.write(names[i], mtext.data(), mtext.size());
    else if (!coded[i].empty()) w.write(names[i], coded[i].data(), coded[i].size());
    else w.write(names[i], p, len);
  }
  w.close();
  return (int)enc.size();
}

}  // namespace rans
}  // namespace qph
