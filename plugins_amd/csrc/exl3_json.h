// exl3_json.h -- a small JSON reader for the quantization blocks and model
// configs the boundary's claims/validate entries inspect (the reference
// parses them with std.json: turboexl3_ds41/config.zig:13-17,
// turboexl3_qwen38/config.zig:18-28,69-105).  Values are parsed into a tree;
// malformed text yields an invalid root.
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

namespace exl3 {

struct Json {
  enum Kind { INVALID, NUL, BOOL, NUMBER, STRING, ARRAY, OBJECT };
  Kind kind = INVALID;
  bool b = false;
  double num = 0.0;
  bool integral = false;  // the number was written without fraction or exponent
  std::string str;
  std::vector<Json> arr;
  std::map<std::string, Json> obj;

  bool valid() const { return kind != INVALID; }
  bool is_object() const { return kind == OBJECT; }
  // Member lookup; nullptr when absent or not an object.
  const Json *get(const std::string &k) const {
    if (kind != OBJECT) return nullptr;
    auto it = obj.find(k);
    return it == obj.end() ? nullptr : &it->second;
  }
  bool is_string(const char *s) const { return kind == STRING && str == s; }

  static Json parse(const char *p, size_t n);
};

}  // namespace exl3
