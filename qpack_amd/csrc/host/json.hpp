// Minimal JSON value for QPACK manifests and model configs (manifest.json / config.json blobs).
// Objects keep insertion order so a written manifest reads back in the same order.
#pragma once
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace qph {

struct Json {
  enum Type { Null, Bool, Num, Str, Arr, Obj } type = Null;
  bool b = false;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;

  Json() = default;
  Json(bool v) : type(Bool), b(v) {}
  Json(int v) : type(Num), num(v) {}
  Json(int64_t v) : type(Num), num((double)v) {}
  Json(double v) : type(Num), num(v) {}
  Json(const char *s) : type(Str), str(s) {}
  Json(std::string s) : type(Str), str(std::move(s)) {}
  static Json array() { Json j; j.type = Arr; return j; }
  static Json object() { Json j; j.type = Obj; return j; }

  const Json *find(const std::string &k) const;
  const Json &operator[](const std::string &k) const;   // a Null value when absent
  Json &set(const std::string &k, Json v);
  void push(Json v) { type = Arr; arr.push_back(std::move(v)); }

  double number(double def) const { return type == Num ? num : def; }
  int64_t integer(int64_t def) const { return type == Num ? (int64_t)num : def; }
  bool boolean(bool def) const { return type == Bool ? b : def; }
  const std::string &string() const;

  static Json parse(const char *p, size_t n);   // throws std::runtime_error on malformed input
  std::string dump() const;
};

}  // namespace qph
