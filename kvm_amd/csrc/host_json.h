// Host-side helpers shared by the command-line runners (kvm_exec, kvm_run): a minimal JSON reader for bundle
// metadata and manifests, file readers, and the buffer initialisation a bundle's metadata declares.
#pragma once
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>
#include "../../include/kvm_exec.h"

namespace kvmh {

// ---------------------------------------------------------------------------------------------- minimal JSON
struct Json {
  enum T { NUL, B, N, S, A, O } t = NUL;
  double n = 0; bool b = false; std::string s; std::vector<Json> a; std::vector<std::pair<std::string, Json>> o;
  const Json* get(const std::string& k) const { for (auto& kv : o) if (kv.first == k) return &kv.second; return nullptr; }
  const Json& need(const std::string& k) const { const Json* j = get(k); if (!j) throw std::runtime_error("metadata: missing key " + k); return *j; }
  double num(const std::string& k, double d) const { const Json* j = get(k); return j && j->t == N ? j->n : d; }
};
struct Parser {
  const std::string& s; size_t p = 0;
  explicit Parser(const std::string& x) : s(x) {}
  void ws() { while (p < s.size() && isspace((unsigned char)s[p])) ++p; }
  Json parse() {
    ws(); Json j;
    if (p >= s.size()) throw std::runtime_error("json: unexpected end");
    char c = s[p];
    if (c == '{') { ++p; j.t = Json::O; ws(); if (s[p] == '}') { ++p; return j; }
      for (;;) { ws(); std::string k = str(); ws(); if (s[p++] != ':') throw std::runtime_error("json: ':' expected"); j.o.push_back({k, parse()}); ws();
        if (s[p] == ',') { ++p; continue; } if (s[p] == '}') { ++p; return j; } throw std::runtime_error("json: ',' or '}' expected"); } }
    if (c == '[') { ++p; j.t = Json::A; ws(); if (s[p] == ']') { ++p; return j; }
      for (;;) { j.a.push_back(parse()); ws(); if (s[p] == ',') { ++p; continue; } if (s[p] == ']') { ++p; return j; } throw std::runtime_error("json: ',' or ']' expected"); } }
    if (c == '"') { j.t = Json::S; j.s = str(); return j; }
    if (!s.compare(p, 4, "true")) { p += 4; j.t = Json::B; j.b = true; return j; }
    if (!s.compare(p, 5, "false")) { p += 5; j.t = Json::B; return j; }
    if (!s.compare(p, 4, "null")) { p += 4; return j; }
    if (!s.compare(p, 8, "Infinity")) { p += 8; j.t = Json::N; j.n = INFINITY; return j; }
    if (!s.compare(p, 9, "-Infinity")) { p += 9; j.t = Json::N; j.n = -INFINITY; return j; }
    if (!s.compare(p, 3, "NaN")) { p += 3; j.t = Json::N; j.n = NAN; return j; }
    char* e; j.n = strtod(s.c_str() + p, &e); if (e == s.c_str() + p) throw std::runtime_error("json: bad value");
    j.s = s.substr(p, (e - s.c_str()) - p); p = e - s.c_str(); j.t = Json::N; return j;
  }
  std::string str() {
    if (s[p] != '"') throw std::runtime_error("json: string expected");
    std::string out; ++p;
    while (p < s.size() && s[p] != '"') {
      if (s[p] != '\\') { out += s[p++]; continue; }
      ++p; const char c = s[p++];
      if (c == 'u') { unsigned cp = hex4();
        if (cp >= 0xD800 && cp < 0xDC00 && !s.compare(p, 2, "\\u")) { p += 2; cp = 0x10000 + ((cp - 0xD800) << 10) + (hex4() - 0xDC00); }
        utf8(out, cp); }
      else out += c == 'n' ? '\n' : c == 't' ? '\t' : c == 'r' ? '\r' : c == 'b' ? '\b' : c == 'f' ? '\f' : c;
    }
    if (p >= s.size()) throw std::runtime_error("json: unterminated string");
    ++p; return out;
  }
  unsigned hex4() {
    if (p + 4 > s.size()) throw std::runtime_error("json: bad \\u escape");
    const unsigned v = (unsigned)std::stoul(s.substr(p, 4), nullptr, 16); p += 4; return v;
  }
  static void utf8(std::string& o, unsigned cp) {
    if (cp < 0x80) o += (char)cp;
    else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3F)); }
    else if (cp < 0x10000) { o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
    else { o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3F)); o += (char)(0x80 | ((cp >> 6) & 0x3F)); o += (char)(0x80 | (cp & 0x3F)); }
  }
};
inline std::string read_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary); if (!f) throw std::runtime_error("cannot read " + path);
  std::stringstream ss; ss << f.rdbuf(); return ss.str();
}
template <class T> std::vector<T> read_bin(const std::string& path) {
  std::string d = read_file(path); std::vector<T> v(d.size() / sizeof(T)); memcpy(v.data(), d.data(), v.size() * sizeof(T)); return v;
}

// f32 -> bf16 storage bits, round to nearest even (reference: mvm_exec.cu:1607); NaN stays NaN, infinities stay.
inline uint16_t bf16_rne(float f) {
  uint32_t u; memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Adds the buffer a bundle's metadata entry `jb` declares (dims, dtype and init: fill / values / seeded / file, files
// relative to `dir`); returns its index. The reference refuses a values array or file of the wrong size the same way.
inline int add_buffer_from_meta(KvmExec* ex, const Json& jb, const std::string& dir) {
  int rows = (int)jb.num("rows", 1), cols = (int)jb.num("cols", 1), dt = (int)jb.num("dtype", 0);
  const Json& in = jb.need("init"); std::string kind = in.need("kind").s;
      KvmInit init{}; std::vector<float> vf; std::vector<int32_t> vi; std::vector<uint16_t> vh; std::string raw;
      if (kind == "fill") { init.kind = KVM_INIT_FILL; init.value = (float)in.need("value").n; }
      else if (kind == "values") {
        init.kind = KVM_INIT_VALUES; const auto& vals = in.need("values").a;
        if ((long long)vals.size() != (long long)rows * cols)   // the reference refuses a short or long array the same way
          throw std::runtime_error("buffer " + jb.need("name").s + ": buffer init size " + std::to_string(vals.size()) + " != " +
                                   std::to_string((long long)rows * cols));
        if (dt == 1) { for (auto& v : vals) vi.push_back((int32_t)v.n); init.values = vi.data(); }
        else if (dt == 2) { for (auto& v : vals) vh.push_back(bf16_rne((float)v.n)); init.values = vh.data(); }
        else { for (auto& v : vals) vf.push_back((float)v.n); init.values = vf.data(); }
      } else if (kind == "seeded") {
        init.kind = KVM_INIT_SEEDED; init.seed = strtoull(in.need("seed").s.c_str(), nullptr, 10); init.draws = (int)in.need("draws").n;
        init.bias = (float)in.need("bias").n; init.coef = (float)in.need("coef").n;
      } else if (kind == "file") {
        init.kind = KVM_INIT_VALUES; raw = read_file(dir + "/" + in.need("path").s);
        const size_t want = (size_t)rows * cols * (dt == 2 ? 2 : 4);
        if (raw.size() != want)
          throw std::runtime_error("buffer " + jb.need("name").s + ": buffer init size " + std::to_string(raw.size()) + " bytes != " + std::to_string(want));
        init.values = raw.data();
      }
      else throw std::runtime_error("unknown init kind " + kind);
  const int idx = kvm_add_buffer(ex, rows, cols, dt, &init);
  if (idx < 0) throw std::runtime_error(std::string("add_buffer: ") + kvm_last_error(ex));
  return idx;
}

}  // namespace kvmh
