// exl3_json.cpp -- recursive-descent JSON reader (RFC 8259 subset: no
// surrogate-pair validation beyond decoding \uXXXX to UTF-8).
#include "exl3_json.h"

#include <cstdlib>
#include <cstring>

namespace exl3 {
namespace {

struct Reader {
  const char *p;
  const char *end;
  int depth = 0;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char *s) {
    size_t n = std::strlen(s);
    if ((size_t)(end - p) < n || std::memcmp(p, s, n) != 0) return false;
    p += n;
    return true;
  }
  static void utf8(std::string &out, unsigned cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool string(std::string &out) {
    if (p >= end || *p != '"') return false;
    ++p;
    while (p < end && *p != '"') {
      unsigned char ch = (unsigned char)*p;
      if (ch < 0x20) return false;
      if (ch == '\\') {
        ++p;
        if (p >= end) return false;
        switch (*p) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            if (end - p < 5) return false;
            unsigned cp = 0;
            for (int i = 1; i <= 4; ++i) {
              char h = p[i];
              cp <<= 4;
              if (h >= '0' && h <= '9') cp |= (unsigned)(h - '0');
              else if (h >= 'a' && h <= 'f') cp |= (unsigned)(h - 'a' + 10);
              else if (h >= 'A' && h <= 'F') cp |= (unsigned)(h - 'A' + 10);
              else return false;
            }
            utf8(out, cp);
            p += 4;
            break;
          }
          default: return false;
        }
        ++p;
      } else {
        out += (char)ch;
        ++p;
      }
    }
    if (p >= end) return false;
    ++p;
    return true;
  }
  bool number(Json &j) {
    const char *s = p;
    bool integral = true;
    if (p < end && *p == '-') ++p;
    if (p >= end) return false;
    if (*p == '0') {
      ++p;
    } else if (*p >= '1' && *p <= '9') {
      while (p < end && *p >= '0' && *p <= '9') ++p;
    } else {
      return false;
    }
    if (p < end && *p == '.') {
      integral = false;
      ++p;
      if (p >= end || !(*p >= '0' && *p <= '9')) return false;
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    if (p < end && (*p == 'e' || *p == 'E')) {
      integral = false;
      ++p;
      if (p < end && (*p == '+' || *p == '-')) ++p;
      if (p >= end || !(*p >= '0' && *p <= '9')) return false;
      while (p < end && *p >= '0' && *p <= '9') ++p;
    }
    std::string text(s, p);
    j.kind = Json::NUMBER;
    j.num = std::strtod(text.c_str(), nullptr);
    j.integral = integral;
    return true;
  }
  bool value(Json &j) {
    if (++depth > 256) return false;
    ws();
    if (p >= end) return false;
    bool ok = true;
    switch (*p) {
      case '{': {
        ++p;
        j.kind = Json::OBJECT;
        ws();
        if (p < end && *p == '}') {
          ++p;
          break;
        }
        for (;;) {
          ws();
          std::string key;
          if (!string(key)) return false;
          ws();
          if (p >= end || *p != ':') return false;
          ++p;
          Json v;
          if (!value(v)) return false;
          j.obj[key] = std::move(v);
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == '}') {
            ++p;
            break;
          }
          return false;
        }
        break;
      }
      case '[': {
        ++p;
        j.kind = Json::ARRAY;
        ws();
        if (p < end && *p == ']') {
          ++p;
          break;
        }
        for (;;) {
          Json v;
          if (!value(v)) return false;
          j.arr.push_back(std::move(v));
          ws();
          if (p < end && *p == ',') {
            ++p;
            continue;
          }
          if (p < end && *p == ']') {
            ++p;
            break;
          }
          return false;
        }
        break;
      }
      case '"':
        j.kind = Json::STRING;
        ok = string(j.str);
        break;
      case 't':
        ok = lit("true");
        j.kind = Json::BOOL;
        j.b = true;
        break;
      case 'f':
        ok = lit("false");
        j.kind = Json::BOOL;
        break;
      case 'n':
        ok = lit("null");
        j.kind = Json::NUL;
        break;
      default:
        ok = number(j);
    }
    --depth;
    return ok;
  }
};

}  // namespace

Json Json::parse(const char *p, size_t n) {
  Json j;
  if (p == nullptr) return j;
  Reader r{p, p + n};
  if (!r.value(j)) return Json{};
  r.ws();
  if (r.p != r.end) return Json{};
  return j;
}

}  // namespace exl3
