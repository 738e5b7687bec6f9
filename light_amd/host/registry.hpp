// registry.hpp -- Light's operator dispatch table (internal/registry/registry.go:12-82).
//
// A kernel is registered once per Key{Op, Dev, DType}; a duplicate registration is a
// programming error (Go panics; here std::logic_error).  Lookup of a missing key fails
// with an Error for which IsKernelNotFound() holds ("registry: kernel not found: K").
#pragma once

#include <functional>
#include <map>
#include <optional>
#include <string>
#include <vector>

#include "light.hpp"

namespace light {

struct Key {
  std::string op;
  DeviceKind dev;
  DType dtype;
  std::string str() const;  // "op/Kind/DType" (Key.String)
  bool operator<(const Key &o) const;
  bool operator==(const Key &o) const { return op == o.op && dev == o.dev && dtype == o.dtype; }
};

// Scalar attributes: Light's Attrs map[string]any holds ints and bools on this path.
struct Attr {
  int64_t i = 0;
  bool is_bool = false;
  static Attr Int(int64_t v) { return Attr{v, false}; }
  static Attr Bool(bool b) { return Attr{b ? 1 : 0, true}; }
};

// registry.Context: inputs (optional ones absent), the pre-allocated output, attrs.
struct Context {
  std::vector<std::optional<Tensor>> inputs;
  Tensor output;
  std::map<std::string, Attr> attrs;
  const Tensor &in(size_t i) const { return *inputs.at(i); }
  bool has(size_t i) const { return i < inputs.size() && inputs[i].has_value(); }
  int64_t attr(const std::string &k) const;
};

using Kernel = std::function<void(Context &)>;  // throws Error on failure

void Register(const Key &k, Kernel fn);
Kernel Lookup(const Key &k);
std::vector<Key> Registered();

}  // namespace light
