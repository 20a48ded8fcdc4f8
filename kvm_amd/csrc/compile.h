// Workload JSON -> ABI-v2 task bundle, in C++: the counterpart of the reference's bundle compiler (reference:
// runtime/compile_workload.py:452-713) and of this repository's Python restatement (kvm_amd/compiler.py), with
// byte-identical output for the same workload: tasks.bin (64-byte descriptors), successors.bin (int32 CSR),
// args.bin (int32 words, f32 as IEEE bits) and metadata.json (the same keys, order and text as Python's
// json.dump(indent=2)).
//
// Semantics (the reference's):
//   * every `publishes` task numbers its variable's next version in declaration order;
//   * each read waits for its version; reads beyond a task's first waiting read get a `noop` gate task inserted just
//     before the task;
//   * an `exact` read of version N adds a write-after-read edge to the publisher of N + 1;
//   * the first publisher of a variable with base version > 0 waits for the live head;
//   * the graph must be acyclic, every variable's publishers totally ordered, and no task may wait for a publisher
//     ordered after it.
#pragma once
#include <algorithm>
#include <cmath>
#include <charconv>
#include <cstdint>
#include <cstring>
#include <map>
#include <set>
#include <stdexcept>
#include <string>
#include <sys/stat.h>
#include <vector>
#include "../../include/mvm_task_abi.h"
#include "host_json.h"

namespace kvmc {

using kvmh::Json;

struct CompileError : std::runtime_error { using std::runtime_error::runtime_error; };
inline void need(bool ok, const std::string& msg) { if (!ok) throw CompileError(msg); }

constexpr int kExtIdMin = 300;    // this executor's own operator pack: listed in operator_ids only when used
constexpr double kF32Max = 3.4028234663852886e38;

struct Arg { std::string name, type; bool optional; };
struct Op { std::string name; int id; std::vector<Arg> args; };

// The registries in mvm_ops_list.inc order.
inline const std::vector<Op>& registry() {
  static std::vector<Op> ops;
  if (ops.empty()) {
    struct Raw { const char* name; int id; const char* sig; };
    static const Raw raw[] = {
#define X(n, id, sig) {#n, id, sig},
#include "../../include/mvm_ops_list.inc"
#undef X
    };
    for (const Raw& r : raw) {
      Op o{r.name, r.id, {}};
      std::string s(r.sig);
      size_t p = 0;
      while (p < s.size()) {
        size_t e = s.find(',', p); if (e == std::string::npos) e = s.size();
        const std::string item = s.substr(p, e - p);
        const size_t c = item.find(':');
        std::string ty = item.substr(c + 1);
        const bool opt = ty == "buf?";
        if (opt) ty = "buf";
        o.args.push_back(Arg{item.substr(0, c), ty, opt});
        p = e + 1;
      }
      ops.push_back(o);
    }
  }
  return ops;
}

// ---------------------------------------------------------------------------------------------- JSON output
// A value tree written as Python's json.dump(value, indent=2) writes it (ensure_ascii, shortest-repr floats).
struct Val {
  enum T { NUL, INT, FLT, STR, ARR, OBJ } t = NUL;
  long long i = 0; double f = 0; std::string s;
  std::vector<Val> a; std::vector<std::pair<std::string, Val>> o;
  static Val null() { return Val{}; }
  static Val num(long long v) { Val x; x.t = INT; x.i = v; return x; }
  static Val flt(double v) { Val x; x.t = FLT; x.f = v; return x; }
  static Val str(const std::string& v) { Val x; x.t = STR; x.s = v; return x; }
  static Val arr() { Val x; x.t = ARR; return x; }
  static Val obj() { Val x; x.t = OBJ; return x; }
  Val& add(const std::string& k, Val v) { o.push_back({k, std::move(v)}); return *this; }
  Val& push(Val v) { a.push_back(std::move(v)); return *this; }
};

// Python's repr of a finite double: the shortest digits that round-trip; fixed notation for decimal exponents in
// [-4, 16), else d.ddde[+-]XX.
inline std::string py_float(double v) {
  if (v == 0) return std::signbit(v) ? "-0.0" : "0.0";
  char buf[64];
  auto r = std::to_chars(buf, buf + sizeof buf, v, std::chars_format::scientific);
  std::string sc(buf, r.ptr);
  bool neg = sc[0] == '-';
  if (neg) sc = sc.substr(1);
  const size_t e = sc.find('e');
  std::string mant = sc.substr(0, e), digits;
  for (char c : mant) if (c != '.') digits += c;
  const int ex = std::stoi(sc.substr(e + 1));
  std::string out;
  if (ex >= -4 && ex < 16) {
    if (ex >= 0) {
      std::string ip = digits.substr(0, std::min<size_t>(digits.size(), ex + 1));
      while ((int)ip.size() < ex + 1) ip += '0';
      std::string fp = (int)digits.size() > ex + 1 ? digits.substr(ex + 1) : "0";
      out = ip + "." + fp;
    } else {
      out = "0." + std::string(-ex - 1, '0') + digits;
    }
  } else {
    out = digits.substr(0, 1);
    if (digits.size() > 1) out += "." + digits.substr(1);
    char eb[16];
    snprintf(eb, sizeof eb, "e%c%02d", ex < 0 ? '-' : '+', std::abs(ex));
    out += eb;
  }
  return neg ? "-" + out : out;
}

inline void json_str(std::string& out, const std::string& s) {
  out += '"';
  for (size_t i = 0; i < s.size();) {
    const unsigned char c = (unsigned char)s[i];
    if (c == '"') { out += "\\\""; ++i; }
    else if (c == '\\') { out += "\\\\"; ++i; }
    else if (c == '\n') { out += "\\n"; ++i; }
    else if (c == '\r') { out += "\\r"; ++i; }
    else if (c == '\t') { out += "\\t"; ++i; }
    else if (c == '\b') { out += "\\b"; ++i; }
    else if (c == '\f') { out += "\\f"; ++i; }
    else if (c < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", c); out += b; ++i; }
    else if (c < 0x80) { out += (char)c; ++i; }
    else {   // UTF-8 sequence -> \uXXXX (surrogate pairs above the BMP), as ensure_ascii does
      unsigned cp = 0; int n = 0;
      if ((c & 0xE0) == 0xC0) { cp = c & 0x1F; n = 1; } else if ((c & 0xF0) == 0xE0) { cp = c & 0x0F; n = 2; } else { cp = c & 0x07; n = 3; }
      for (int k = 1; k <= n && i + k < s.size(); ++k) cp = (cp << 6) | ((unsigned char)s[i + k] & 0x3F);
      i += n + 1;
      char b[16];
      if (cp >= 0x10000) { cp -= 0x10000; snprintf(b, sizeof b, "\\u%04x\\u%04x", 0xD800 + (cp >> 10), 0xDC00 + (cp & 0x3FF)); }
      else snprintf(b, sizeof b, "\\u%04x", cp);
      out += b;
    }
  }
  out += '"';
}

inline void json_write(std::string& out, const Val& v, int ind) {
  const std::string pad(ind + 2, ' '), end(ind, ' ');
  switch (v.t) {
    case Val::NUL: out += "null"; break;
    case Val::INT: out += std::to_string(v.i); break;
    case Val::FLT: out += py_float(v.f); break;
    case Val::STR: json_str(out, v.s); break;
    case Val::ARR:
      if (v.a.empty()) { out += "[]"; break; }
      out += "[\n";
      for (size_t k = 0; k < v.a.size(); ++k) { out += pad; json_write(out, v.a[k], ind + 2); out += k + 1 < v.a.size() ? ",\n" : "\n"; }
      out += end + "]";
      break;
    case Val::OBJ:
      if (v.o.empty()) { out += "{}"; break; }
      out += "{\n";
      for (size_t k = 0; k < v.o.size(); ++k) {
        out += pad; json_str(out, v.o[k].first); out += ": "; json_write(out, v.o[k].second, ind + 2);
        out += k + 1 < v.o.size() ? ",\n" : "\n";
      }
      out += end + "}";
      break;
  }
}

// ---------------------------------------------------------------------------------------------- input checks
inline bool is_int_literal(const Json& j) {
  return j.t == Json::N && std::isfinite(j.n) && j.s.find_first_of(".eE") == std::string::npos;
}
inline long long int_literal(const Json& j, const std::string& where) {
  long long v = 0;
  auto r = std::from_chars(j.s.data(), j.s.data() + j.s.size(), v);
  need(r.ec == std::errc() && r.ptr == j.s.data() + j.s.size(), where + ": integer out of range");
  return v;
}
inline float to_f32(double v) { return (float)v; }
inline double num_f32(const Json& x, const std::string& where) {
  need(x.t == Json::N, where + ": expected a number");
  need(std::isfinite(x.n) && std::fabs(x.n) <= kF32Max, where + ": " + x.s + " is not a finite float32");
  return (double)to_f32(x.n);
}
inline long long num_i32(const Json& x, const std::string& where) {
  if (x.t == Json::B) return x.b ? 1 : 0;     // a JSON bool is a Python int
  need(x.t == Json::N && std::fabs(x.n) < 9.2e18 && std::isfinite(x.n) && x.n == std::floor(x.n), where + ": integer expected");
  const long long v = is_int_literal(x) ? int_literal(x, where) : (long long)x.n;
  need(v >= INT32_MIN && v <= INT32_MAX, where + ": " + std::to_string(v) + " overflows int32");
  return v;
}
inline double bf16_of(double f) {
  float x = (float)f;
  if (std::isnan(x) || std::isinf(x)) return f;
  uint32_t u; std::memcpy(&u, &x, 4);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  std::memcpy(&x, &u, 4);
  return (double)x;
}

struct Buffer { std::string name; int index, rows, cols, dtype; Val init; };
struct Read { std::string var, policy; int version, wait_ver; bool waits, implicit = false; int gate = -1; };
struct Task {
  std::string name; int graph; const Op* op; std::vector<int32_t> words;
  int priority = 0, deadline_us = -1;
  std::vector<int> after;
  std::string publishes;
  std::vector<std::tuple<std::string, std::string, int>> decl_reads;
  std::vector<Read> reads;
  std::string wait_var; int wait_ver = 0; bool has_wait = false;
  std::string pub_var; int pub_ver = 0; bool has_pub = false;
  bool gate = false;
};

struct Bundle {
  std::vector<std::string> files;     // relative paths of `file` initial values (copied in beside the bundle)
  std::vector<MvmTaskDesc> tasks;
  std::vector<int32_t> succ, args;
  std::string metadata;     // the metadata.json text, newline-terminated
};

inline Val make_init(const std::string& where, const Json* init, long long n, const std::string& dtype, const std::string* data_dir) {
  Json fill_default;
  if (!init) return Val::obj().add("kind", Val::str("fill")).add("value", dtype == "i32" ? Val::num(0) : Val::flt(0.0));
  need(init->t == Json::O && init->get("kind"), where + ": init needs a kind");
  auto conv = [&](const Json& x) -> Val {
    if (dtype == "i32") return Val::num(num_i32(x, where));
    if (dtype == "bf16") return Val::flt(bf16_of(num_f32(x, where)));
    return Val::flt(num_f32(x, where));
  };
  const std::string& k = init->need("kind").s;
  if (k == "fill") return Val::obj().add("kind", Val::str("fill")).add("value", conv(init->need("value")));
  if (k == "values") {
    const Json& vals = init->need("values");
    need(vals.t == Json::A && (long long)vals.a.size() == n, where + ": init.values needs " + std::to_string(n) + " numbers");
    Val arr = Val::arr();
    for (auto& x : vals.a) arr.push(conv(x));
    return Val::obj().add("kind", Val::str("values")).add("values", std::move(arr));
  }
  if (k == "seeded") {
    need(dtype == "f32", where + ": seeded init needs dtype f32");
    const Json& seed = init->need("seed");
    need(is_int_literal(seed), where + ": seed must be in [0, 2^63)");
    const long long sv = int_literal(seed, where);
    need(sv >= 0, where + ": seed must be in [0, 2^63)");
    const std::string dist = init->get("dist") ? init->need("dist").s : "normal";
    const double scale = num_f32(init->need("scale"), where);
    need(scale >= 0, where + ": scale must be >= 0");
    int draws; double bias, coef;
    if (dist == "uniform") { draws = 1; bias = 0.5; coef = (double)to_f32(2.0 * scale); }
    else if (dist == "normal") { draws = 4; bias = 2.0; coef = (double)to_f32(scale * std::sqrt(3.0)); }
    else throw CompileError("unknown dist '" + dist + "'");
    return Val::obj().add("kind", Val::str("seeded")).add("seed", Val::num(sv)).add("scale", Val::flt(scale)).add("dist", Val::str(dist))
        .add("draws", Val::num(draws)).add("bias", Val::flt(bias)).add("coef", Val::flt(coef));
  }
  if (k == "file") {
    const Json& p = init->need("path");
    need(p.t == Json::S && !p.s.empty() && p.s[0] != '/' && p.s.find('\\') == std::string::npos, where + ": bad init.path");
    std::vector<std::string> parts;
    size_t q = 0;
    while (q <= p.s.size()) {
      size_t e = p.s.find('/', q); if (e == std::string::npos) e = p.s.size();
      const std::string part = p.s.substr(q, e - q);
      need(part != "..", where + ": bad init.path");
      if (!part.empty() && part != ".") parts.push_back(part);
      q = e + 1;
    }
    std::string norm;
    for (size_t i = 0; i < parts.size(); ++i) norm += (i ? "/" : "") + parts[i];
    if (norm.empty()) norm = ".";
    if (data_dir) {     // validated when the data directory is known (reference: runtime/compile_workload.py:237-241)
      const std::string f = *data_dir + "/" + p.s;
      struct stat st;
      need(stat(f.c_str(), &st) == 0 && S_ISREG(st.st_mode), where + ": init file '" + f + "' not found");
      const long long want = (dtype == "bf16" ? 2 : 4) * n;
      need((long long)st.st_size == want, where + ": init file '" + p.s + "' has " + std::to_string((long long)st.st_size) +
                                              " bytes, expected " + std::to_string(want));
    }
    return Val::obj().add("kind", Val::str("file")).add("path", Val::str(norm));
  }
  throw CompileError(where + ": unknown init kind '" + k + "'");
}

inline std::vector<int32_t> make_args(const std::string& where, const Op& op, const Json* raw, const std::map<std::string, Buffer>& buffers) {
  Json empty; empty.t = Json::O;
  if (!raw) raw = &empty;
  need(raw->t == Json::O, where + ": args must be an object");
  std::set<std::string> want, got;
  for (auto& a : op.args) want.insert(a.name);
  for (auto& kv : raw->o) got.insert(kv.first);
  need(want == got && got.size() == raw->o.size(), where + ": op " + op.name + " takes other arguments");
  std::vector<int32_t> words;
  for (auto& a : op.args) {
    const Json& v = *raw->get(a.name);
    if (a.type == "buf") {
      if (v.t == Json::NUL) { need(a.optional, where + ": " + a.name + " is a required buffer"); words.push_back(-1); }
      else {
        need(v.t == Json::S && buffers.count(v.s), where + ": " + a.name + ": unknown buffer");
        words.push_back(buffers.at(v.s).index);
      }
    } else if (a.type == "i32") {
      need(is_int_literal(v), where + ": " + a.name + ": int32 expected");
      const long long x = int_literal(v, where);
      need(x >= INT32_MIN && x <= INT32_MAX, where + ": " + a.name + ": int32 expected");
      words.push_back((int32_t)x);
    } else {
      need(v.t == Json::N, where + ": " + a.name + ": number expected");
      const float f = (float)v.n;
      need(!(std::isinf(f) && !std::isinf(v.n)), where + ": " + a.name + ": " + v.s + " overflows float32");
      int32_t w; std::memcpy(&w, &f, 4);
      need(((w >> 23) & 0xFF) != 0xFF, where + ": " + a.name + ": non-finite value");
      words.push_back(w);
    }
  }
  return words;
}

// ---------------------------------------------------------------------------------------------- graph helpers
struct Csr { std::vector<int> off, succ, indeg; };
inline Csr make_csr(const std::vector<std::vector<int>>& preds) {
  const int n = (int)preds.size();
  std::vector<std::vector<int>> outs(n);
  for (int i = 0; i < n; ++i) for (int p : preds[i]) outs[p].push_back(i);
  Csr c; c.off.push_back(0);
  for (auto& o : outs) { c.succ.insert(c.succ.end(), o.begin(), o.end()); c.off.push_back((int)c.succ.size()); }
  for (auto& p : preds) c.indeg.push_back((int)p.size());
  return c;
}
inline bool topo(const Csr& c, std::vector<int>& pos) {
  const int n = (int)c.indeg.size();
  std::vector<int> rem = c.indeg, order;
  for (int i = 0; i < n; ++i) if (!rem[i]) order.push_back(i);
  for (size_t h = 0; h < order.size(); ++h) {
    const int i = order[h];
    for (int k = c.off[i]; k < c.off[i + 1]; ++k) if (--rem[c.succ[k]] == 0) order.push_back(c.succ[k]);
  }
  if ((int)order.size() != n) return false;
  pos.assign(n, 0);
  for (int p = 0; p < n; ++p) pos[order[p]] = p;
  return true;
}
inline bool reaches(const Csr& c, const std::vector<int>& pos, int a, int b) {
  if (a == b) return true;
  if (pos[a] > pos[b]) return false;
  std::vector<int> stack{a};
  std::set<int> seen{a};
  while (!stack.empty()) {
    const int i = stack.back(); stack.pop_back();
    for (int k = c.off[i]; k < c.off[i + 1]; ++k) {
      const int j = c.succ[k];
      if (j == b) return true;
      if (!seen.count(j) && pos[j] < pos[b]) { seen.insert(j); stack.push_back(j); }
    }
  }
  return false;
}

// ---------------------------------------------------------------------------------------------- compile
// data_dir: where `file` initial values are read from (checked here); null leaves them unchecked.
inline Bundle compile(const Json& spec, const std::map<std::string, int>& base_versions, const std::string* data_dir = nullptr) {
  const auto& reg = registry();
  std::map<std::string, const Op*> ops;
  for (auto& o : reg) ops[o.name] = &o;
  need(spec.t == Json::O && spec.get("graphs"), "workload: keys are variables, buffers, graphs (graphs required)");
  for (auto& kv : spec.o) need(kv.first == "variables" || kv.first == "buffers" || kv.first == "graphs", "workload: keys are variables, buffers, graphs (graphs required)");
  std::vector<std::string> vnames;
  if (const Json* v = spec.get("variables")) for (auto& x : v->a) vnames.push_back(x.s);
  need(std::set<std::string>(vnames.begin(), vnames.end()).size() == vnames.size(), "duplicate variable names");
  for (auto& kv : base_versions) need(std::find(vnames.begin(), vnames.end(), kv.first) != vnames.end(), "base_versions names undeclared variables");
  struct Var { int id, base, final_; };
  std::map<std::string, Var> vars;
  for (size_t i = 0; i < vnames.size(); ++i) {
    const int b = base_versions.count(vnames[i]) ? base_versions.at(vnames[i]) : 0;
    vars[vnames[i]] = Var{(int)i, b, b};
  }
  std::map<std::string, Buffer> buffers;
  std::vector<std::string> border;
  if (const Json* bl = spec.get("buffers"))
    for (auto& d : bl->a) {
      const std::string& name = d.need("name").s;
      need(!buffers.count(name), "duplicate buffer '" + name + "'");
      const Json* jr = d.get("rows"); const Json* jc = d.get("cols"); const Json* jd = d.get("dtype");
      need((!jr || is_int_literal(*jr)) && (!jc || is_int_literal(*jc)), "buffer '" + name + "': bad shape");
      const long long rows = jr ? int_literal(*jr, name) : 1, cols = jc ? int_literal(*jc, name) : 1;
      need(rows >= 1 && cols >= 1 && rows * cols <= INT32_MAX, "buffer '" + name + "': bad shape");
      const std::string dt = jd ? jd->s : "f32";
      need(dt == "f32" || dt == "i32" || dt == "bf16", "buffer '" + name + "': bad dtype '" + dt + "'");
      Buffer b{name, (int)buffers.size(), (int)rows, (int)cols, dt == "i32" ? 1 : dt == "bf16" ? 2 : 0,
               make_init("buffer '" + name + "'", d.get("init"), rows * cols, dt, data_dir)};
      buffers[name] = b;
      border.push_back(name);
    }
  std::vector<Task> decls;
  const auto& graphs = spec.need("graphs").a;
  for (size_t gi = 0; gi < graphs.size(); ++gi) {
    const Json& g = graphs[gi];
    const Json* gn = g.get("name");
    need(gn && gn->t == Json::S && !gn->s.empty() && gn->s.find('/') == std::string::npos, "graphs[" + std::to_string(gi) + "]: bad name");
    const std::string gname = gn->s;
    const int base = (int)decls.size();
    std::map<std::string, int> index;
    const auto& ts = g.need("tasks").a;
    for (size_t ti = 0; ti < ts.size(); ++ti) {
      const std::string id = ts[ti].need("id").s;
      need(!index.count(id), "graph '" + gname + "': duplicate task id '" + id + "'");
      index[id] = base + (int)ti;
    }
    for (auto& t : ts) {
      const std::string where = gname + "/" + t.need("id").s;
      auto op = ops.find(t.need("op").s);
      need(op != ops.end(), where + ": unknown op '" + t.need("op").s + "'");
      Task k;
      k.name = where; k.graph = (int)gi; k.op = op->second;
      k.words = make_args(where, *op->second, t.get("args"), buffers);
      if (const Json* af = t.get("after"))
        for (auto& x : af->a) {
          auto it = index.find(x.s);
          need(it != index.end(), where + ": after names unknown task '" + x.s + "'");
          k.after.push_back(it->second);
        }
      need(std::set<int>(k.after.begin(), k.after.end()).size() == k.after.size() &&
               std::find(k.after.begin(), k.after.end(), (int)decls.size()) == k.after.end(), where + ": bad after list");
      if (const Json* p = t.get("publishes")) if (p->t != Json::NUL) {
        need(p->t == Json::S && vars.count(p->s), where + ": publishes undeclared variable");
        k.publishes = p->s;
      }
      if (const Json* rs = t.get("reads"))
        for (auto& r : rs->a) {
          const Json* rv = r.get("var"); const Json* rp = r.get("policy"); const Json* rn = r.get("version");
          need(rv && rv->t == Json::S && vars.count(rv->s) && rp && (rp->s == "exact" || rp->s == "at_least") && rn && is_int_literal(*rn) &&
                   int_literal(*rn, where) >= 0, where + ": bad read");
          for (auto& x : k.decl_reads) need(std::get<0>(x) != rv->s, where + ": reads '" + rv->s + "' twice");
          k.decl_reads.push_back({rv->s, rp->s, (int)int_literal(*rn, where)});
        }
      if (const Json* pr = t.get("priority")) { need(is_int_literal(*pr), where + ": priority must be an integer"); k.priority = (int)int_literal(*pr, where); }
      if (const Json* dl = t.get("deadline_us")) { need(is_int_literal(*dl), where + ": deadline_us must be an integer"); k.deadline_us = (int)int_literal(*dl, where); }
      decls.push_back(k);
    }
  }
  // versions
  std::map<std::string, std::vector<int>> pubs;
  for (auto& v : vnames) pubs[v];
  for (size_t i = 0; i < decls.size(); ++i) {
    Task& t = decls[i];
    if (!t.publishes.empty()) {
      Var& v = vars[t.publishes];
      ++v.final_;
      pubs[t.publishes].push_back((int)i);
      t.has_pub = true; t.pub_var = t.publishes; t.pub_ver = v.final_;
    }
  }
  std::map<std::string, std::map<int, int>> by_ver;
  for (auto& kv : pubs) for (size_t k = 0; k < kv.second.size(); ++k) by_ver[kv.first][vars[kv.first].base + (int)k + 1] = kv.second[k];
  std::vector<std::pair<int, int>> exact_edges;
  for (size_t i = 0; i < decls.size(); ++i) {
    Task& t = decls[i];
    for (auto& dr : t.decl_reads) {
      const std::string& var = std::get<0>(dr); const std::string& pol = std::get<1>(dr); const int n = std::get<2>(dr);
      const Var& v = vars[var];
      if (pol == "exact") need(n >= v.base, t.name + ": exact read of '" + var + "' at " + std::to_string(n) + " is stale (base " + std::to_string(v.base) + ")");
      if (n > v.base) need(by_ver[var].count(n), t.name + ": read of '" + var + "' at " + std::to_string(n) + " can never be satisfied");
      auto nx = by_ver[var].find(n + 1);
      if (pol == "exact" && nx != by_ver[var].end() && nx->second != (int)i) exact_edges.push_back({(int)i, nx->second});
      t.reads.push_back(Read{var, pol, n, n, n > 0});
    }
  }
  for (auto& vn : vnames) {
    const auto& ix = pubs[vn];
    const int b = vars[vn].base;
    if (!ix.empty() && b > 0) {
      Task& t = decls[ix[0]];
      Read* own = nullptr;
      for (auto& r : t.reads) if (r.var == vn) { own = &r; break; }
      if (own) own->wait_ver = std::max(own->wait_ver, b);
      else { Read r{vn, "at_least", b, b, true}; r.implicit = true; t.reads.push_back(r); }
    }
  }
  // gates and edges
  const Op* noop = ops.at("noop");
  std::vector<Task> tasks;
  std::vector<int> final_(decls.size(), 0);
  std::map<int, std::vector<int>> gates_of;
  for (size_t i = 0; i < decls.size(); ++i) {
    Task& t = decls[i];
    std::vector<Read*> waiting;
    for (auto& r : t.reads) if (r.waits) waiting.push_back(&r);
    for (size_t k = 1; k < waiting.size(); ++k) {
      Task g;
      g.name = "__gate/" + t.name + "/" + std::to_string(k); g.graph = t.graph; g.op = noop; g.priority = t.priority; g.deadline_us = t.deadline_us;
      g.gate = true; g.has_wait = true; g.wait_var = waiting[k]->var; g.wait_ver = waiting[k]->wait_ver;
      waiting[k]->gate = (int)tasks.size();
      gates_of[(int)i].push_back((int)tasks.size());
      tasks.push_back(g);
    }
    final_[i] = (int)tasks.size();
    if (!waiting.empty()) { t.has_wait = true; t.wait_var = waiting[0]->var; t.wait_ver = waiting[0]->wait_ver; }
    tasks.push_back(t);
  }
  std::vector<std::vector<int>> preds(tasks.size());
  for (size_t i = 0; i < decls.size(); ++i) {
    auto& p = preds[final_[i]];
    if (gates_of.count((int)i)) p = gates_of[(int)i];
    for (int j : decls[i].after) p.push_back(final_[j]);
  }
  for (auto& e : exact_edges) {
    auto& p = preds[final_[e.second]];
    if (std::find(p.begin(), p.end(), final_[e.first]) == p.end()) p.push_back(final_[e.first]);
  }
  const Csr c = make_csr(preds);
  std::vector<int> pos;
  need(topo(c, pos), "dependency cycle (possibly through an exact read's write-after-read edge)");
  for (auto& vn : vnames) {
    const auto& ix = pubs[vn];
    for (size_t k = 1; k < ix.size(); ++k)
      need(reaches(c, pos, final_[ix[k - 1]], final_[ix[k]]), "unordered publishers of '" + vn + "': " + decls[ix[k - 1]].name + ", " + decls[ix[k]].name);
  }
  for (size_t i = 0; i < decls.size(); ++i)
    for (auto& r : decls[i].reads)
      if (r.wait_ver > vars[r.var].base) {
        const int p = by_ver[r.var][r.wait_ver];
        need(!reaches(c, pos, final_[i], final_[p]), decls[i].name + ": waits for a publisher ordered after it (deadlock)");
      }
  // pack
  Bundle out;
  for (auto& n : border)
    if (buffers.at(n).init.o[0].second.s == "file") out.files.push_back(buffers.at(n).init.o[1].second.s);
  std::set<std::string> used;
  for (auto& t : tasks) used.insert(t.op->name);
  for (size_t i = 0; i < tasks.size(); ++i) {
    const Task& t = tasks[i];
    MvmTaskDesc d{};
    d.op_id = t.op->id; d.succ_off = c.off[i]; d.succ_cnt = c.off[i + 1] - c.off[i]; d.indegree = c.indeg[i];
    d.priority = t.priority; d.deadline_us = t.deadline_us; d.args_off = (int)out.args.size(); d.args_words = (int)t.words.size();
    d.wait_var = t.has_wait ? vars[t.wait_var].id : -1; d.wait_ver = t.has_wait ? t.wait_ver : 0;
    d.pub_var = t.has_pub ? vars[t.pub_var].id : -1; d.pub_ver = t.has_pub ? t.pub_ver : 0;
    d.workload_id = t.graph;
    out.tasks.push_back(d);
    out.args.insert(out.args.end(), t.words.begin(), t.words.end());
  }
  out.succ = c.succ;
  Val meta = Val::obj();
  meta.add("abi_version", Val::num(MVM_ABI_VERSION)).add("task_count", Val::num((long long)tasks.size()))
      .add("edge_count", Val::num((long long)c.succ.size())).add("args_words", Val::num((long long)out.args.size()));
  Val names = Val::arr(); for (auto& t : tasks) names.push(Val::str(t.name));
  meta.add("task_names", std::move(names));
  Val ready = Val::arr(); for (size_t i = 0; i < tasks.size(); ++i) if (!c.indeg[i]) ready.push(Val::num((long long)i));
  meta.add("initial_ready", std::move(ready));
  Val opids = Val::obj(); for (auto& o : reg) if (o.id < kExtIdMin || used.count(o.name)) opids.add(o.name, Val::num(o.id));
  meta.add("operator_ids", std::move(opids));
  Val bufs = Val::arr();
  for (auto& n : border) {
    const Buffer& b = buffers.at(n);
    bufs.push(Val::obj().add("name", Val::str(b.name)).add("index", Val::num(b.index)).add("rows", Val::num(b.rows))
                  .add("cols", Val::num(b.cols)).add("dtype", Val::num(b.dtype)).add("init", b.init));
  }
  meta.add("buffers", std::move(bufs));
  Val jv = Val::arr(); for (auto& n : vnames) jv.push(Val::obj().add("name", Val::str(n)).add("id", Val::num(vars[n].id)).add("base_version", Val::num(vars[n].base)));
  meta.add("variables", std::move(jv));
  Val jp = Val::arr();
  for (size_t i = 0; i < tasks.size(); ++i)
    if (tasks[i].has_pub) jp.push(Val::obj().add("task", Val::num((long long)i)).add("name", Val::str(tasks[i].name))
                                      .add("var", Val::num(vars[tasks[i].pub_var].id)).add("version", Val::num(tasks[i].pub_ver)));
  meta.add("publishers", std::move(jp));
  Val jr = Val::arr();
  for (size_t i = 0; i < tasks.size(); ++i) {
    if (tasks[i].gate) continue;
    for (auto& r : tasks[i].reads) {
      if (r.implicit) continue;
      jr.push(Val::obj().add("task", Val::num((long long)i)).add("name", Val::str(tasks[i].name)).add("var", Val::num(vars[r.var].id))
                  .add("policy", Val::str(r.policy)).add("version", Val::num(r.version))
                  .add("observed", r.policy == "exact" ? Val::num(r.version) : Val::null()).add("gate", r.gate >= 0 ? Val::num(r.gate) : Val::null()));
    }
  }
  meta.add("reads", std::move(jr));
  Val jf = Val::obj(); for (auto& n : vnames) jf.add(n, Val::num(vars[n].final_));
  meta.add("final_versions", std::move(jf));
  json_write(out.metadata, meta, 0);
  out.metadata += "\n";
  return out;
}

}  // namespace kvmc
