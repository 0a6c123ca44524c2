#include "json.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <stdexcept>

namespace qph {

static const Json kNullJson;
static const std::string kEmptyStr;

const Json *Json::find(const std::string &k) const {
  if (type != Obj) return nullptr;
  for (auto &kv : obj) if (kv.first == k) return &kv.second;
  return nullptr;
}
const Json &Json::operator[](const std::string &k) const { const Json *j = find(k); return j ? *j : kNullJson; }
Json &Json::set(const std::string &k, Json v) {
  if (type != Obj) { type = Obj; obj.clear(); }
  for (auto &kv : obj) if (kv.first == k) { kv.second = std::move(v); return kv.second; }
  obj.emplace_back(k, std::move(v));
  return obj.back().second;
}
const std::string &Json::string() const { return type == Str ? str : kEmptyStr; }

namespace {
class Parser {
 public:
  Parser(const char *p, size_t n) : p_(p), e_(p + n) {}
  Json document() {
    Json v = value(0); ws();
    if (p_ != e_) fail("trailing characters");
    return v;
  }

 private:
  const char *p_, *e_;
  [[noreturn]] void fail(const char *what) { throw std::runtime_error(std::string("json: ") + what); }
  void ws() { while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++; }
  bool eat(char c) { ws(); if (p_ < e_ && *p_ == c) { p_++; return true; } return false; }
  void expect(char c) { if (!eat(c)) fail("unexpected character"); }
  bool word(const char *w) {
    const char *q = p_; for (; *w; w++, q++) if (q >= e_ || *q != *w) return false;
    p_ = q; return true;
  }
  static void utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) out += (char)cp;
    else if (cp < 0x800) { out += (char)(0xC0 | (cp >> 6)); out += (char)(0x80 | (cp & 63)); }
    else if (cp < 0x10000) { out += (char)(0xE0 | (cp >> 12)); out += (char)(0x80 | ((cp >> 6) & 63)); out += (char)(0x80 | (cp & 63)); }
    else { out += (char)(0xF0 | (cp >> 18)); out += (char)(0x80 | ((cp >> 12) & 63)); out += (char)(0x80 | ((cp >> 6) & 63)); out += (char)(0x80 | (cp & 63)); }
  }
  uint32_t hex4() {
    if (e_ - p_ < 4) fail("short \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; i++) {
      const char c = *p_++; v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }
  std::string text() {
    std::string s;
    for (;;) {
      if (p_ >= e_) fail("unterminated string");
      const char c = *p_++;
      if (c == '"') return s;
      if (c != '\\') { s += c; continue; }
      if (p_ >= e_) fail("bad escape");
      const char x = *p_++;
      switch (x) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && e_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            p_ += 2; const uint32_t lo = hex4(); cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(s, cp); break;
        }
        default: fail("bad escape");
      }
    }
  }
  Json value(int depth) {
    if (depth > 64) fail("nesting too deep");
    ws();
    if (p_ >= e_) fail("unexpected end");
    const char c = *p_;
    if (c == '{') {
      p_++; Json o = Json::object();
      if (eat('}')) return o;
      do { ws(); expect('"'); std::string k = text(); expect(':'); o.obj.emplace_back(std::move(k), value(depth + 1)); } while (eat(','));
      expect('}'); return o;
    }
    if (c == '[') {
      p_++; Json a = Json::array();
      if (eat(']')) return a;
      do a.arr.push_back(value(depth + 1)); while (eat(','));
      expect(']'); return a;
    }
    if (c == '"') { p_++; return Json(text()); }
    if (word("true")) return Json(true);
    if (word("false")) return Json(false);
    if (word("null")) return Json();
    char *end = nullptr; const std::string tok(p_, (size_t)std::min<ptrdiff_t>(e_ - p_, 64));
    const double v = strtod(tok.c_str(), &end);
    if (end == tok.c_str()) fail("bad value");
    p_ += end - tok.c_str();
    return Json(v);
  }
};

void dump_to(const Json &j, std::string &o) {
  switch (j.type) {
    case Json::Null: o += "null"; break;
    case Json::Bool: o += j.b ? "true" : "false"; break;
    case Json::Num: {
      char buf[40];
      if (std::isfinite(j.num) && j.num == std::floor(j.num) && std::fabs(j.num) < 9e15) snprintf(buf, sizeof buf, "%lld", (long long)j.num);
      else snprintf(buf, sizeof buf, "%.17g", j.num);
      o += buf; break;
    }
    case Json::Str:
      o += '"';
      for (unsigned char ch : j.str) {
        if (ch == '"') o += "\\\""; else if (ch == '\\') o += "\\\\"; else if (ch == '\n') o += "\\n";
        else if (ch < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", ch); o += b; }
        else o += (char)ch;
      }
      o += '"'; break;
    case Json::Arr:
      o += '[';
      for (size_t i = 0; i < j.arr.size(); i++) { if (i) o += ','; dump_to(j.arr[i], o); }
      o += ']'; break;
    case Json::Obj:
      o += '{';
      for (size_t i = 0; i < j.obj.size(); i++) {
        if (i) o += ',';
        dump_to(Json(j.obj[i].first), o); o += ':'; dump_to(j.obj[i].second, o);
      }
      o += '}'; break;
  }
}
}  // namespace

Json Json::parse(const char *p, size_t n) { return Parser(p, n).document(); }
std::string Json::dump() const { std::string o; dump_to(*this, o); return o; }

}  // namespace qph
