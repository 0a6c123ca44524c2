// Seeded synthetic Llama-family models written as QPACK2 files (random init: there are no checkpoints offline).
//
// Weights: N(0, std) from a counter-based generator, so every element is a pure function of (seed, tensor index,
// element index) and the file is identical for any thread count:
//   h = mix64(seed, tensor, pair index); u1 = (hi32(h) + 0.5) / 2^32, u2 = lo32(h) / 2^32;
//   Box-Muller in double: r = sqrt(-2 ln u1), element 2p = r cos(2 pi u2), element 2p + 1 = r sin(2 pi u2); w = (float)(std * n).
// Quantisation rules:
//   q8 - per row s = max|w| / 127 (1 for an all-zero row), q = clamp(nearbyint(w / s), -127, 127): the rule of
//        /root/reference/tools/qpack-quantize.cpp:327-339 and python/qpack/container.py:90-95;
//   q4 - per 32-column group s = fp16(max|w| / 7), q = clamp(lrintf(w / s), -8, 7) stored as q + 8 in the QPACK2 q4 layout
//        (byte j = column j low nibble, column j + 16 high nibble).  This absmax scale is this build's choice; the
//        reference's own writer searches the scale by squared error (qpack-quantize.cpp:34-58).  Kernels read both alike.
//   q1 - per 128-column group: bit c (LSB first in 16 bytes) = (w >= 0), scale = fp16(mean |w|): q1_group without
//        calibration (qpack-quantize.cpp:80-85).
// Which matrices: q8 everything; q4 the layer matrices (q4m_alt: wv and even layers' w_down in q8; more_bits: the
// quantiser's q4m policy, qpack-quantize.cpp:67-74; q4_head: embed / lm_head q4 too); mlp_q1: w_gate / w_up / w_down
// in q1 (with more_bits the policy's downs stay q8, its q1m).
// Norm weights are 1.0; biases are N(0, std) f32.  Tensor names follow /root/reference/python/qpack/convert_llama.py:5-11.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "container.hpp"
#include "synth.hpp"

namespace qph {

static inline uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// elements [i0, i1) (i0 even) of tensor `tid` as float N(0, std)
static void normals(uint64_t seed, uint64_t tid, int64_t i0, int64_t i1, float sd, float *out) {
  const uint64_t key = mix64(seed ^ mix64(tid + 0x51ed270b27e3a1c5ull));
  for (int64_t i = i0; i < i1; i += 2) {
    const uint64_t h = mix64(key ^ (uint64_t)(i >> 1) * 0xd6e8feb86659fd93ull);
    const double u1 = ((double)(h >> 32) + 0.5) * (1.0 / 4294967296.0), u2 = (double)(h & 0xffffffffull) * (1.0 / 4294967296.0);
    const double r = std::sqrt(-2.0 * std::log(u1)), a = 6.283185307179586476925286766559 * u2;
    out[i - i0] = (float)(sd * r * std::cos(a));
    if (i + 1 < i1) out[i + 1 - i0] = (float)(sd * r * std::sin(a));
  }
}

static void parallel_rows(int64_t rows, int threads, const std::function<void(int64_t, int64_t)> &f) {
  if (threads <= 1 || rows < 64) { f(0, rows); return; }
  std::vector<std::thread> th; const int64_t chunk = (rows + threads - 1) / threads;
  for (int t = 0; t < threads; t++) {
    const int64_t a = t * chunk, b = std::min(rows, a + chunk);
    if (a < b) th.emplace_back([=, &f] { f(a, b); });
  }
  for (auto &t : th) t.join();
}

static uint16_t to_half(float f) { const _Float16 h = (_Float16)f; uint16_t u; memcpy(&u, &h, 2); return u; }
static float from_half(uint16_t u) { _Float16 h; memcpy(&h, &u, 2); return (float)h; }

enum class Q { F32, Q8, Q4, Q1 };

// tools/qpack-quantize.cpp:67-74 (without --q4m-last-half): wv, and the w_down of layers i < n/8, i >= 7n/8 or with
// (i - n/8) % 3 == 2
static bool more_bits(const std::string &tail, int i, int n) {
  if (tail == "wv") return true;
  if (tail != "w_down") return false;
  return i < n / 8 || i >= 7 * n / 8 || (i - n / 8) % 3 == 2;
}
struct Plan { std::string name; std::vector<int64_t> shape; Q q; bool ones; uint64_t tid; };

void synth_write(const SynthSpec &s, const std::string &path, int threads) {
  if (s.hidden <= 0 || s.layers <= 0 || s.heads <= 0 || s.kv_heads <= 0 || s.head_dim <= 0 || s.ffn <= 0 || s.vocab <= 0)
    throw std::runtime_error("synth: all dimensions must be positive");
  if (s.heads % s.kv_heads) throw std::runtime_error("synth: heads must be a multiple of kv_heads");
  if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
  const int64_t d = s.hidden, qd = (int64_t)s.heads * s.head_dim, kvd = (int64_t)s.kv_heads * s.head_dim, ff = s.ffn, V = s.vocab;
  std::vector<Plan> ts; uint64_t tid = 0;
  auto add = [&](const std::string &n, std::vector<int64_t> sh, Q q, bool ones = false) { ts.push_back({n, sh, q, ones, tid++}); };
  const Q lq = s.q4 ? Q::Q4 : Q::Q8;
  const Q hq = s.q4 && s.q4_head ? Q::Q4 : Q::Q8;
  add("embed", {V, d}, hq);
  if (!s.tied) add("lm_head", {V, d}, hq);
  // a layer matrix's kind: q1 for the MLP (mlp_q1), q8 where a policy keeps more bits, else the layers' kind
  auto kind = [&](const std::string &tail, int l) {
    if (s.mlp_q1 && (tail == "w_gate" || tail == "w_up" || tail == "w_down")) return s.more_bits && more_bits(tail, l, s.layers) ? Q::Q8 : Q::Q1;
    if (!s.q4) return Q::Q8;
    if (s.more_bits) return more_bits(tail, l, s.layers) ? Q::Q8 : Q::Q4;
    if (s.q4m_alt && (tail == "wv" || (tail == "w_down" && l % 2 == 0))) return Q::Q8;
    return Q::Q4;
  };
  add("final_norm", {d}, Q::F32, true);
  for (int l = 0; l < s.layers; l++) {
    const std::string p = "layers." + std::to_string(l) + ".";
    add(p + "attn_norm", {d}, Q::F32, true); add(p + "ffn_norm", {d}, Q::F32, true);
    add(p + "wq", {qd, d}, kind("wq", l)); add(p + "wk", {kvd, d}, kind("wk", l));
    add(p + "wv", {kvd, d}, kind("wv", l));
    add(p + "wo", {d, qd}, kind("wo", l));
    if (s.qkv_bias) { add(p + "bq", {qd}, Q::F32); add(p + "bk", {kvd}, Q::F32); add(p + "bv", {kvd}, Q::F32); }
    add(p + "w_gate", {ff, d}, kind("w_gate", l)); add(p + "w_up", {ff, d}, kind("w_up", l));
    add(p + "w_down", {d, ff}, kind("w_down", l));
  }
  (void)lq;
  for (auto &t : ts) if (t.q == Q::Q4 && t.shape[1] % 32) throw std::runtime_error("synth: q4 tensor " + t.name + " needs cols % 32 == 0");
  for (auto &t : ts) if (t.q == Q::Q1 && t.shape[1] % 128) throw std::runtime_error("synth: q1 tensor " + t.name + " needs cols % 128 == 0");

  JNode man = JNode(JNode::Fields{}), tl = JNode(JNode::List{});
  std::vector<std::pair<std::string, uint64_t>> plan;
  for (size_t k = 0; k < ts.size(); k++) {
    const Plan &t = ts[k]; char bid[16]; snprintf(bid, sizeof bid, "w%04zu", k);
    JNode e = JNode(JNode::Fields{}); e.put("name", t.name);
    JNode sh = JNode(JNode::List{}); for (auto v : t.shape) sh.append(JNode((int64_t)v)); e.put("shape", sh); e.put("dtype", "float32");
    const int64_t rows = t.shape[0], cols = t.shape.size() > 1 ? t.shape[1] : 1;
    if (t.q == Q::F32) { e.put("kind", "f32"); e.put("blob", std::string(bid) + ".f32"); plan.push_back({std::string(bid) + ".f32", 4ull * rows * cols}); }
    else if (t.q == Q::Q8) {
      e.put("kind", "q8"); e.put("blob", std::string(bid) + ".q8"); e.put("scale", std::string(bid) + ".scale");
      plan.push_back({std::string(bid) + ".q8", (uint64_t)(rows * cols)}); plan.push_back({std::string(bid) + ".scale", 4ull * rows});
    } else if (t.q == Q::Q1) {
      e.put("kind", "q1"); e.put("blob", std::string(bid) + ".q1"); e.put("scale", std::string(bid) + ".scale"); e.put("group", 128);
      plan.push_back({std::string(bid) + ".q1", (uint64_t)(rows * cols / 8)}); plan.push_back({std::string(bid) + ".scale", 2ull * rows * (cols / 128)});
    } else {
      e.put("kind", "q4"); e.put("blob", std::string(bid) + ".q4"); e.put("scale", std::string(bid) + ".scale"); e.put("group", 32);
      plan.push_back({std::string(bid) + ".q4", (uint64_t)(rows * cols / 2)}); plan.push_back({std::string(bid) + ".scale", 2ull * rows * (cols / 32)});
    }
    tl.append(e);
  }
  man.put("format", "QPACK2");
  man.put("quant", s.mlp_q1 ? (s.more_bits ? "q1m" : "q1") : s.q4 ? (s.q4m_alt || s.more_bits ? "q4m" : "q4") : "q8");
  man.put("tensors", tl);
  {
    JNode syn = JNode(JNode::Fields{});
    syn.put("seed", JNode((int64_t)s.seed));
    syn.put("std", JNode((double)s.std));
    man.put("synthetic", syn);
  }
  JNode cfg = JNode(JNode::Fields{});
  cfg.put("arch", "llama"); cfg.put("model_type", s.model_type[0] ? s.model_type : "llama");
  cfg.put("hidden_size", JNode(d)); cfg.put("num_hidden_layers", s.layers); cfg.put("num_attention_heads", s.heads);
  cfg.put("num_key_value_heads", s.kv_heads); cfg.put("head_dim", s.head_dim); cfg.put("intermediate_size", JNode(ff));
  cfg.put("vocab_size", JNode(V)); cfg.put("rope_theta", s.rope_theta); cfg.put("max_position_embeddings", s.max_pos);
  cfg.put("rms_norm_eps", (double)s.rms_eps); cfg.put("tie_embeddings", (bool)s.tied); cfg.put("qkv_bias", (bool)s.qkv_bias);
  const std::string mj = man.serialize(), cj = cfg.serialize();
  plan.insert(plan.begin(), {"config.json", cj.size()});
  plan.insert(plan.begin(), {"manifest.json", mj.size()});

  ContainerWriter w(path, plan, "QPACK2\0\0");
  w.write("manifest.json", mj.data(), mj.size());
  w.write("config.json", cj.data(), cj.size());
  size_t pi = 2;
  for (const Plan &t : ts) {
    const int64_t rows = t.shape[0], cols = t.shape.size() > 1 ? t.shape[1] : 1;
    if (t.q == Q::F32) {
      std::vector<float> v((size_t)(rows * cols));
      if (t.ones) std::fill(v.begin(), v.end(), 1.f); else normals(s.seed, t.tid, 0, rows * cols, s.std, v.data());
      w.write(plan[pi].first, v.data(), plan[pi].second); pi++;
    } else if (t.q == Q::Q8) {
      std::vector<int8_t> q((size_t)(rows * cols)); std::vector<float> sc((size_t)rows);
      parallel_rows(rows, threads, [&](int64_t a, int64_t b) {
        std::vector<float> row((size_t)cols);
        for (int64_t r = a; r < b; r++) {
          normals(s.seed, t.tid, r * cols, (r + 1) * cols, s.std, row.data());
          float mx = 0; for (float v : row) mx = std::max(mx, std::fabs(v));
          float sr = mx / 127.f; if (sr == 0) sr = 1.f;
          for (int64_t c = 0; c < cols; c++) q[(size_t)(r * cols + c)] = (int8_t)std::max(-127, std::min(127, (int)std::nearbyint(row[(size_t)c] / sr)));
          sc[(size_t)r] = sr;
        }
      });
      w.write(plan[pi].first, q.data(), plan[pi].second); pi++;
      w.write(plan[pi].first, sc.data(), plan[pi].second); pi++;
    } else if (t.q == Q::Q1) {
      const int64_t G = cols / 128;
      std::vector<uint8_t> q((size_t)(rows * cols / 8)); std::vector<uint16_t> sc((size_t)(rows * G));
      parallel_rows(rows, threads, [&](int64_t a, int64_t b) {
        std::vector<float> row((size_t)cols);
        for (int64_t r = a; r < b; r++) {
          normals(s.seed, t.tid, r * cols, (r + 1) * cols, s.std, row.data());
          for (int64_t g = 0; g < G; g++) {
            const float *wg = row.data() + 128 * g; double num = 0;
            uint8_t *o = q.data() + (size_t)((r * G + g) * 16);
            memset(o, 0, 16);
            for (int i = 0; i < 128; i++) { num += std::fabs(wg[i]); if (wg[i] >= 0) o[i >> 3] |= (uint8_t)(1 << (i & 7)); }
            sc[(size_t)(r * G + g)] = to_half((float)(num / 128.0));
          }
        }
      });
      w.write(plan[pi].first, q.data(), plan[pi].second); pi++;
      w.write(plan[pi].first, sc.data(), plan[pi].second); pi++;
    } else {
      const int64_t G = cols / 32;
      std::vector<uint8_t> q((size_t)(rows * cols / 2)); std::vector<uint16_t> sc((size_t)(rows * G));
      parallel_rows(rows, threads, [&](int64_t a, int64_t b) {
        std::vector<float> row((size_t)cols);
        for (int64_t r = a; r < b; r++) {
          normals(s.seed, t.tid, r * cols, (r + 1) * cols, s.std, row.data());
          for (int64_t g = 0; g < G; g++) {
            const float *wg = row.data() + 32 * g; float amax = 0; int qv[32];
            for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(wg[i]));
            uint16_t h = 0;
            if (amax > 0) {
              h = to_half(amax / 7.f); const float sh = from_half(h);
              for (int i = 0; i < 32; i++) qv[i] = std::max(-8, std::min(7, (int)std::lrintf(wg[i] / sh)));
            } else for (int i = 0; i < 32; i++) qv[i] = 0;
            uint8_t *o = q.data() + (size_t)(r * (cols / 2) + 16 * g);
            for (int j = 0; j < 16; j++) o[j] = (uint8_t)((qv[j] + 8) | ((qv[j + 16] + 8) << 4));
            sc[(size_t)(r * G + g)] = h;
          }
        }
      });
      w.write(plan[pi].first, q.data(), plan[pi].second); pi++;
      w.write(plan[pi].first, sc.data(), plan[pi].second); pi++;
    }
  }
  w.close();
}

}  // namespace qph
