#include "json.hpp"

#include <charconv>
#include <clocale>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <locale.h>
#include <stdexcept>

namespace qph {

namespace {

const JNode kNullNode;
const JNode::List kNoItems;
const std::string kNoText;

// recursive-descent reader over [p, end); depth-limited so hostile input cannot exhaust the stack
class Reader {
 public:
  Reader(const char *p, size_t n) : begin_(p), p_(p), end_(p + n) {}

  JNode document() {
    JNode v = value(0);
    blank();
    if (p_ != end_) fail("text after the document");
    return v;
  }

 private:
  const char *begin_, *p_, *end_;

  [[noreturn]] void fail(const char *what) const {
    throw std::runtime_error(std::string("JSON: ") + what + " at offset " + std::to_string(p_ - begin_));
  }
  void blank() { while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++; }
  bool eat(char c) { blank(); if (p_ < end_ && *p_ == c) { p_++; return true; } return false; }
  void expect(char c, const char *what) { if (!eat(c)) fail(what); }
  bool word(const char *w) {
    size_t n = 0;
    while (w[n]) n++;
    if ((size_t)(end_ - p_) < n) return false;
    for (size_t i = 0; i < n; i++) if (p_[i] != w[i]) return false;
    p_ += n;
    return true;
  }

  JNode value(int depth) {
    if (depth > 64) fail("nesting too deep");
    blank();
    if (p_ >= end_) fail("unexpected end of text");
    switch (*p_) {
      case '{': return fields(depth);
      case '[': return list(depth);
      case '"': return JNode(text());
      case 't': if (word("true")) return JNode(true); break;
      case 'f': if (word("false")) return JNode(false); break;
      case 'n': if (word("null")) return JNode(); break;
      default: return JNode(number());
    }
    fail("unknown literal");
  }

  JNode fields(int depth) {
    p_++;   // '{'
    JNode::Fields f;
    if (eat('}')) return JNode(std::move(f));
    do {
      blank();
      if (p_ >= end_ || *p_ != '"') fail("expected a member name");
      std::string k = text();
      expect(':', "expected ':' after a member name");
      f.emplace_back(std::move(k), value(depth + 1));
    } while (eat(','));
    expect('}', "expected ',' or '}' in an object");
    return JNode(std::move(f));
  }

  JNode list(int depth) {
    p_++;   // '['
    JNode::List l;
    if (eat(']')) return JNode(std::move(l));
    do l.push_back(value(depth + 1));
    while (eat(','));
    expect(']', "expected ',' or ']' in an array");
    return JNode(std::move(l));
  }

  double number() {
    // the JSON number grammar, checked here; the conversion is std::from_chars, which ignores the process's locale
    // (strtod would read "1.5" as 1 under a comma-decimal LC_NUMERIC)
    const char *s = p_;
    if (p_ < end_ && *p_ == '-') p_++;
    auto digits = [&] { const char *d = p_; while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++; return p_ > d; };
    if (!digits()) fail("malformed number");
    if (p_ < end_ && *p_ == '.') { p_++; if (!digits()) fail("malformed number"); }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      p_++;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) p_++;
      if (!digits()) fail("malformed number");
    }
    double v = 0;
    const auto r = std::from_chars(s, p_, v);
    if (r.ec == std::errc::result_out_of_range) {   // overflow or underflow: strtod's result, in the "C" locale
      static const locale_t c_loc = newlocale(LC_ALL_MASK, "C", (locale_t)0);
      return strtod_l(std::string(s, p_).c_str(), nullptr, c_loc);
    }
    if (r.ec != std::errc() || r.ptr != p_) fail("malformed number");
    return v;
  }

  unsigned hex4() {
    if (end_ - p_ < 4) fail("short \\u escape");
    unsigned v = 0;
    for (int i = 0; i < 4; i++, p_++) {
      const char c = *p_;
      const unsigned d = c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10 : c >= 'A' && c <= 'F' ? c - 'A' + 10 : 99;
      if (d > 15) fail("bad hex digit in \\u escape");
      v = v * 16 + d;
    }
    return v;
  }

  static void put_utf8(std::string &s, unsigned cp) {
    if (cp < 0x80) { s += (char)cp; return; }
    if (cp < 0x800) { s += (char)(0xc0 | cp >> 6); s += (char)(0x80 | (cp & 0x3f)); return; }
    if (cp < 0x10000) { s += (char)(0xe0 | cp >> 12); s += (char)(0x80 | ((cp >> 6) & 0x3f)); s += (char)(0x80 | (cp & 0x3f)); return; }
    s += (char)(0xf0 | cp >> 18); s += (char)(0x80 | ((cp >> 12) & 0x3f));
    s += (char)(0x80 | ((cp >> 6) & 0x3f)); s += (char)(0x80 | (cp & 0x3f));
  }

  std::string text() {
    p_++;   // opening quote
    std::string s;
    while (true) {
      if (p_ >= end_) fail("unterminated string");
      const char c = *p_++;
      if (c == '"') return s;
      if ((unsigned char)c < 0x20) fail("control character in a string");
      if (c != '\\') { s += c; continue; }
      if (p_ >= end_) fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': case '\\': case '/': s += e; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          unsigned cp = hex4();
          if (cp >= 0xd800 && cp < 0xdc00) {   // a high surrogate must pair with a low one
            if (!word("\\u")) fail("unpaired surrogate");
            const unsigned lo = hex4();
            if (lo < 0xdc00 || lo >= 0xe000) fail("unpaired surrogate");
            cp = 0x10000 + ((cp - 0xd800) << 10 | (lo - 0xdc00));
          }
          put_utf8(s, cp);
          break;
        }
        default: fail("unknown escape");
      }
    }
  }
};

void write_text(std::string &out, const std::string &s) {
  out += '"';
  for (const char c : s) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if ((unsigned char)c < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", (unsigned)(unsigned char)c); out += b; }
        else out += c;
    }
  }
  out += '"';
}

void write_number(std::string &out, double v) {
  char b[40];
  if (!std::isfinite(v)) { out += "null"; return; }   // JSON has no inf / nan
  if (v == std::floor(v) && std::fabs(v) < 9007199254740992.0) snprintf(b, sizeof b, "%.0f", v);
  else snprintf(b, sizeof b, "%.17g", v);   // round-trips every double
  out += b;
}

}  // namespace

const JNode *JNode::find(std::string_view key) const {
  const Fields *f = std::get_if<Fields>(&v_);
  if (!f) return nullptr;
  for (const auto &kv : *f) if (kv.first == key) return &kv.second;
  return nullptr;
}
const JNode &JNode::get(std::string_view key) const { const JNode *n = find(key); return n ? *n : kNullNode; }
const JNode::List &JNode::items() const { const List *l = std::get_if<List>(&v_); return l ? *l : kNoItems; }
size_t JNode::size() const {
  if (const List *l = std::get_if<List>(&v_)) return l->size();
  if (const Fields *f = std::get_if<Fields>(&v_)) return f->size();
  return 0;
}
const std::string &JNode::text() const { const std::string *s = std::get_if<std::string>(&v_); return s ? *s : kNoText; }

JNode &JNode::put(std::string key, JNode v) {
  if (is_null()) v_ = Fields{};
  Fields *f = std::get_if<Fields>(&v_);
  if (!f) throw std::runtime_error("JSON: put on a node that is not an object");
  for (auto &kv : *f)
    if (kv.first == key) { kv.second = std::move(v); return kv.second; }
  f->emplace_back(std::move(key), std::move(v));
  return f->back().second;
}
JNode &JNode::append(JNode v) {
  if (is_null()) v_ = List{};
  List *l = std::get_if<List>(&v_);
  if (!l) throw std::runtime_error("JSON: append on a node that is not an array");
  l->push_back(std::move(v));
  return l->back();
}

void JNode::write_to(std::string &out) const {
  switch (v_.index()) {
    case 0: out += "null"; break;
    case 1: out += std::get<bool>(v_) ? "true" : "false"; break;
    case 2: write_number(out, std::get<double>(v_)); break;
    case 3: write_text(out, std::get<std::string>(v_)); break;
    case 4: {
      out += '[';
      bool first = true;
      for (const JNode &n : std::get<List>(v_)) { if (!first) out += ','; first = false; n.write_to(out); }
      out += ']';
      break;
    }
    default: {
      out += '{';
      bool first = true;
      for (const auto &kv : std::get<Fields>(v_)) {
        if (!first) out += ',';
        first = false;
        write_text(out, kv.first);
        out += ':';
        kv.second.write_to(out);
      }
      out += '}';
    }
  }
}
std::string JNode::serialize() const { std::string s; write_to(s); return s; }
JNode JNode::read(const char *text, size_t n) { return Reader(text, n).document(); }

}  // namespace qph
