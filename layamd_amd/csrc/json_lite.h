// Small JSON reader for the checkpoint's config files and the safetensors header.
// Supports objects, arrays, strings (with \uXXXX escapes kept as UTF-8), numbers, true/false/null.
#pragma once
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace laya {

struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;   // keeps file order

  bool has(const std::string& k) const { return find(k) != nullptr; }
  const JVal* find(const std::string& k) const {
    if (kind != Obj) return nullptr;
    for (auto& kv : obj) if (kv.first == k) return &kv.second;
    return nullptr;
  }
  const JVal& operator[](const std::string& k) const {
    const JVal* v = find(k);
    if (!v) throw std::runtime_error("json: missing key " + k);
    return *v;
  }
  double num_or(const std::string& k, double d) const { const JVal* v = find(k); return v && v->kind == Num ? v->num : d; }
  int int_or(const std::string& k, int d) const { return (int)num_or(k, d); }
  std::string str_or(const std::string& k, const std::string& d) const {
    const JVal* v = find(k); return v && v->kind == Str ? v->str : d;
  }
};

class JParser {
 public:
  explicit JParser(const char* s, size_t n) : p_(s), e_(s + n) {}
  JVal parse() { JVal v = value(); ws(); if (p_ != e_) fail("trailing characters"); return v; }

 private:
  const char* p_; const char* e_;
  [[noreturn]] void fail(const char* m) { throw std::runtime_error(std::string("json: ") + m); }
  void ws() { while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_; }
  bool lit(const char* w) { size_t n = strlen(w); if ((size_t)(e_ - p_) >= n && !memcmp(p_, w, n)) { p_ += n; return true; } return false; }
  static void utf8(std::string& o, unsigned cp) {
    if (cp < 0x80) o += (char)cp;
    else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3F)); }
    else if (cp < 0x10000) { o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
    else { o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3F)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
  }
  unsigned hex4() {
    if (e_ - p_ < 4) fail("bad \\u escape");
    unsigned v = 0;
    for (int i = 0; i < 4; i++) {
      char c = *p_++; v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0'; else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10; else fail("bad hex digit");
    }
    return v;
  }
  std::string string() {
    if (*p_ != '"') fail("expected string");
    ++p_; std::string o;
    while (p_ < e_ && *p_ != '"') {
      char c = *p_++;
      if (c != '\\') { o += c; continue; }
      if (p_ >= e_) fail("bad escape");
      char x = *p_++;
      switch (x) {
        case '"': o += '"'; break; case '\\': o += '\\'; break; case '/': o += '/'; break;
        case 'b': o += '\b'; break; case 'f': o += '\f'; break; case 'n': o += '\n'; break;
        case 'r': o += '\r'; break; case 't': o += '\t'; break;
        case 'u': {
          unsigned cp = hex4();
          if (cp >= 0xD800 && cp < 0xDC00 && e_ - p_ >= 6 && p_[0] == '\\' && p_[1] == 'u') {
            p_ += 2; unsigned lo = hex4(); cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(o, cp); break;
        }
        default: fail("bad escape");
      }
    }
    if (p_ >= e_) fail("unterminated string");
    ++p_;
    return o;
  }
  JVal value() {
    ws();
    if (p_ >= e_) fail("unexpected end");
    JVal v;
    char c = *p_;
    if (c == '{') {
      v.kind = JVal::Obj; ++p_; ws();
      if (p_ < e_ && *p_ == '}') { ++p_; return v; }
      for (;;) {
        ws(); std::string k = string(); ws();
        if (p_ >= e_ || *p_ != ':') fail("expected ':'");
        ++p_;
        v.obj.emplace_back(std::move(k), value());
        ws();
        if (p_ < e_ && *p_ == ',') { ++p_; continue; }
        if (p_ < e_ && *p_ == '}') { ++p_; return v; }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = JVal::Arr; ++p_; ws();
      if (p_ < e_ && *p_ == ']') { ++p_; return v; }
      for (;;) {
        v.arr.push_back(value()); ws();
        if (p_ < e_ && *p_ == ',') { ++p_; continue; }
        if (p_ < e_ && *p_ == ']') { ++p_; return v; }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') { v.kind = JVal::Str; v.str = string(); return v; }
    if (lit("true")) { v.kind = JVal::Bool; v.b = true; return v; }
    if (lit("false")) { v.kind = JVal::Bool; v.b = false; return v; }
    if (lit("null")) { v.kind = JVal::Null; return v; }
    if (c == '-' || (c >= '0' && c <= '9')) {
      std::string tok;
      while (p_ < e_ && (strchr("+-.eE", *p_) || (*p_ >= '0' && *p_ <= '9'))) tok += *p_++;
      char* end = nullptr;
      v.kind = JVal::Num; v.num = strtod(tok.c_str(), &end);
      if (!end || *end) fail("bad number");
      return v;
    }
    fail("unexpected character");
  }
};

inline JVal json_parse(const std::string& s) { return JParser(s.data(), s.size()).parse(); }

}  // namespace laya
