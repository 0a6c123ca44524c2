// JNode: a JSON document tree for the two small text blobs of a QPACK container (config.json, manifest.json) and for
// the manifests this library writes (synthetic models, QPACK3 packing).
//
// One std::variant holds the node: null, bool, number (double), text, list, or fields.  Fields are a vector of
// (key, node) pairs rather than a map because a written manifest must list its members, and its tensors, in the order
// they were added.  Lookups on the wrong kind of node return neutral values (a null node, an empty list, the caller's
// default), so reading optional config keys needs no checks; malformed text throws std::runtime_error from read().
#pragma once
#include <cstdint>
#include <string>
#include <string_view>
#include <utility>
#include <variant>
#include <vector>

namespace qph {

class JNode {
 public:
  using List = std::vector<JNode>;
  using Fields = std::vector<std::pair<std::string, JNode>>;

  JNode() = default;
  JNode(bool v) : v_(v) {}
  JNode(int v) : v_((double)v) {}
  JNode(int64_t v) : v_((double)v) {}
  JNode(uint64_t v) : v_((double)v) {}
  JNode(double v) : v_(v) {}
  JNode(const char *s) : v_(std::string(s)) {}
  JNode(std::string s) : v_(std::move(s)) {}
  JNode(List l) : v_(std::move(l)) {}
  JNode(Fields f) : v_(std::move(f)) {}

  bool is_null() const { return v_.index() == 0; }
  bool is_list() const { return std::holds_alternative<List>(v_); }
  bool is_fields() const { return std::holds_alternative<Fields>(v_); }

  // member `key` of an object node: nullptr (find) or a null node (get) when absent
  const JNode *find(std::string_view key) const;
  const JNode &get(std::string_view key) const;
  // elements of a list node (an empty list for any other node)
  const List &items() const;
  size_t size() const;

  double num_or(double def) const { const double *d = std::get_if<double>(&v_); return d ? *d : def; }
  int64_t int_or(int64_t def) const { const double *d = std::get_if<double>(&v_); return d ? (int64_t)*d : def; }
  bool bool_or(bool def) const { const bool *b = std::get_if<bool>(&v_); return b ? *b : def; }
  const std::string &text() const;   // an empty string for a non-text node

  // builders: put replaces an existing member or appends one (a null node becomes an object); append adds a list element
  JNode &put(std::string key, JNode v);
  JNode &append(JNode v);

  std::string serialize() const;
  static JNode read(const char *text, size_t n);

 private:
  std::variant<std::monostate, bool, double, std::string, List, Fields> v_;
  void write_to(std::string &out) const;
};

}  // namespace qph
