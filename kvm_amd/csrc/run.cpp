// kvm_run: the manifest runner, counterpart of the reference's demo runner (reference: demo/mvm_run.cu). It reads a
// demo directory (MANIFEST.json plus compiled ABI-v2 bundles) and runs every admission it lists on ONE persistent
// kernel in stream mode, with no knowledge of the models: buffers, version variables, admission order and conditions
// all come from the manifest.
//
//   kvm_run DEMO_DIR [--out DIR] [--dump REGEX] [--windows N] [--blocks N] [--timeout-s N] [--check-only] [--quiet]
//
// Manifest semantics (the reference's, restated): `buffers` are allocated once, initialised from their owner
// workload's bundle, and shared by name across bundles; an admission starts when its time (at_us) has come, every
// `after_bundles` entry has completed, each `when` condition holds for the LIVE version of its variable, and, for every
// variable it publishes, the live version equals the base it was compiled for while no other admission in flight
// publishes it. Several admissions may be in flight. A bundle compiled for other base versions is shifted (every wait
// and publish of a published variable moved by the difference) when it reads no such variable by absolute version; an
// admission without a bundle directory reuses the last bundle of its workload, shifted. Everything that can be checked
// without a GPU is checked first: the manifest's shape, a serial simulation of the version flow (cycles, conditions no
// order reaches), and every bundle against the global buffer table.
//
// Output (--out): summary.json (per admission: tasks, windows, submit / completion times, live versions at
// completion; final versions), and DIR/<buffer>.bin for buffers matching --dump (f32 widened, i32 raw). Prints
// "OK: d/a tasks, X ms, N admissions" or "FAIL: ..." and exits 0 / 1 (2 for usage errors).
#include <algorithm>
#include <chrono>
#include <climits>
#include <cstdarg>
#include <map>
#include <memory>
#include <regex>
#include <set>
#include <sys/stat.h>
#include <ftw.h>
#include <thread>
#include <unistd.h>
#include "../../include/kvm_exec.h"
#include "compile.h"
#include "host_json.h"

using namespace kvmh;

namespace {

struct ManifestError : std::runtime_error { using std::runtime_error::runtime_error; };
[[noreturn]] void fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void fail(const char* fmt, ...) {
  char b[2048];
  va_list ap; va_start(ap, fmt); vsnprintf(b, sizeof b, fmt, ap); va_end(ap);
  throw ManifestError(b);
}

// ---------------------------------------------------------------------------------------------- strict accessors
const Json& member(const Json& o, const char* k, const std::string& where) {
  if (o.t != Json::O) fail("%s: expected an object", where.c_str());
  const Json* j = o.get(k);
  if (!j) fail("%s: missing key '%s'", where.c_str(), k);
  return *j;
}
long long as_int(const Json& j, const std::string& where, long long lo = LLONG_MIN / 2, long long hi = LLONG_MAX / 2) {
  if (j.t != Json::N || j.n != std::floor(j.n) || !std::isfinite(j.n)) fail("%s: expected an integer", where.c_str());
  if (j.n < (double)lo || j.n > (double)hi) fail("%s: %.17g outside [%lld, %lld]", where.c_str(), j.n, lo, hi);
  return (long long)j.n;
}
const std::string& as_str(const Json& j, const std::string& where) {
  if (j.t != Json::S || j.s.empty()) fail("%s: expected a non-empty string", where.c_str());
  return j.s;
}
const std::vector<Json>& as_arr(const Json& j, const std::string& where) {
  if (j.t != Json::A) fail("%s: expected an array", where.c_str());
  return j.a;
}
bool is_null(const Json* j) { return !j || j->t == Json::NUL; }
const std::string& as_rel_path(const Json& j, const std::string& where) {
  const std::string& s = as_str(j, where);
  if (s[0] == '/' || s.find("..") != std::string::npos) fail("%s: '%s' must be a relative path without '..'", where.c_str(), s.c_str());
  return s;
}
typedef std::map<std::string, long long> VerMap;
VerMap as_versions(const Json* j, const std::string& where) {
  VerMap m;
  if (is_null(j)) return m;
  if (j->t != Json::O) fail("%s: expected an object of variable -> version", where.c_str());
  for (auto& kv : j->o) m[kv.first] = as_int(kv.second, where + "." + kv.first, 0, INT_MAX / 2);
  return m;
}

// ---------------------------------------------------------------------------------------------- manifest model
struct Cond { std::string var; long long mn = 0, mx = LLONG_MAX; };
struct Workload { std::string name, file, cls; long long tasks = 0, edges = 0; int priority = 0; std::vector<std::string> variables; };
struct Admission {
  std::string name, workload, bundle_dir, compile_workload, compile_data_dir;
  std::vector<std::string> after;
  std::vector<Cond> when;
  long long at_us = -1;
  VerMap base, publishes;
};
struct BufDecl { std::string name; int rows = 0, cols = 0, dtype = 0; std::string owner; };
struct ClassDecl { std::string name; std::map<std::string, long long> params; };
struct Manifest {
  std::string root;
  std::vector<Workload> workloads; std::map<std::string, int> wl_idx;
  std::vector<Admission> adms; std::map<std::string, int> adm_idx;
  std::vector<BufDecl> buffers; std::map<std::string, int> buf_idx;
  std::vector<std::string> vars; std::map<std::string, int> var_idx;
  std::vector<ClassDecl> classes;
  int var_id(const std::string& n, const std::string& where) const {
    auto it = var_idx.find(n);
    if (it == var_idx.end()) fail("%s: version variable '%s' is not declared by any workload", where.c_str(), n.c_str());
    return it->second;
  }
};

const char* const kClassKeys[] = {"weight", "min_cta", "max_cta", "bw_cta", "urgent_us"};

Manifest parse_manifest(const std::string& root) {
  Manifest m; m.root = root;
  Json j = Parser(read_file(root + "/MANIFEST.json")).parse();
  if (as_int(member(j, "manifest_version", "manifest"), "manifest_version") != 1) fail("manifest_version must be 1");
  const Json& jw = member(j, "workloads", "manifest");
  if (jw.t != Json::O || jw.o.empty()) fail("workloads: expected a non-empty object");
  auto class_of = [&](const std::string& c) {
    for (size_t i = 0; i < m.classes.size(); ++i) if (m.classes[i].name == c) return (int)i;
    m.classes.push_back(ClassDecl{c, {}});
    return (int)m.classes.size() - 1;
  };
  if (const Json* jc = j.get("classes")) {
    if (jc->t != Json::O) fail("classes: expected an object");
    for (auto& kv : jc->o) {
      const int c = class_of(kv.first);
      if (kv.second.t != Json::O) fail("classes.%s: expected an object", kv.first.c_str());
      for (auto& pk : kv.second.o) {
        if (std::none_of(std::begin(kClassKeys), std::end(kClassKeys), [&](const char* k) { return pk.first == k; }))
          fail("classes.%s: unknown scheduler parameter '%s' (weight, min_cta, max_cta, bw_cta, urgent_us)", kv.first.c_str(), pk.first.c_str());
        const long long v = as_int(pk.second, "classes." + kv.first + "." + pk.first, 0, INT_MAX);
        if (pk.first == "weight" && v < 1) fail("classes.%s.weight must be >= 1", kv.first.c_str());
        m.classes[c].params[pk.first] = v;
      }
    }
  }
  for (auto& kv : jw.o) {
    const std::string where = "workloads." + kv.first;
    Workload w; w.name = kv.first;
    w.file = as_rel_path(member(kv.second, "file", where), where + ".file");
    w.tasks = as_int(member(kv.second, "tasks", where), where + ".tasks", 1, INT_MAX);
    w.edges = as_int(member(kv.second, "edges", where), where + ".edges", 0, INT_MAX);
    w.priority = (int)as_int(member(kv.second, "priority", where), where + ".priority", 0, 1 << 20);
    w.cls = kv.second.get("class") ? as_str(*kv.second.get("class"), where + ".class") : "default";
    if (const Json* v = kv.second.get("variables"))
      for (auto& x : as_arr(*v, where + ".variables")) w.variables.push_back(as_str(x, where + ".variables[]"));
    if (const Json* rq = kv.second.get("requirements"))
      if (const Json* rs = rq->get("resources"))
        if (!as_arr(*rs, where + ".requirements.resources").empty())
          fail("%s needs host resources, which this runner does not provide (the game pack is out of scope)", where.c_str());
    class_of(w.cls);
    for (auto& v : w.variables) if (!m.var_idx.count(v)) { m.var_idx[v] = (int)m.vars.size(); m.vars.push_back(v); }
    m.wl_idx[w.name] = (int)m.workloads.size();
    m.workloads.push_back(w);
  }
  const Json& jb = member(j, "buffers", "manifest");
  if (jb.t != Json::O) fail("buffers: expected an object");
  for (auto& kv : jb.o) {
    const std::string where = "buffers." + kv.first;
    BufDecl b; b.name = kv.first;
    b.rows = (int)as_int(member(kv.second, "rows", where), where + ".rows", 1, INT_MAX);
    b.cols = (int)as_int(member(kv.second, "cols", where), where + ".cols", 1, INT_MAX);
    const std::string& dt = as_str(member(kv.second, "dtype", where), where + ".dtype");
    if (dt != "f32" && dt != "i32" && dt != "bf16") fail("%s.dtype: '%s' is not f32, i32 or bf16", where.c_str(), dt.c_str());
    b.dtype = dt == "i32" ? 1 : dt == "bf16" ? 2 : 0;
    b.owner = as_str(member(kv.second, "owner", where), where + ".owner");
    if (!m.wl_idx.count(b.owner)) fail("%s.owner: unknown workload '%s'", where.c_str(), b.owner.c_str());
    if ((long long)b.rows * b.cols > (1ll << 31) - 1) fail("%s: %d x %d elements overflow", where.c_str(), b.rows, b.cols);
    m.buf_idx[b.name] = (int)m.buffers.size();
    m.buffers.push_back(b);
  }
  const auto& arr = as_arr(member(j, "admissions", "manifest"), "admissions");
  if (arr.empty()) fail("admissions: empty");
  for (size_t i = 0; i < arr.size(); ++i) {
    const Json& x = arr[i];
    const std::string where = "admissions[" + std::to_string(i) + "]";
    Admission a;
    a.name = as_str(member(x, "name", where), where + ".name");
    if (m.adm_idx.count(a.name)) fail("%s: duplicate admission name '%s'", where.c_str(), a.name.c_str());
    a.workload = as_str(member(x, "workload", where), where + ".workload");
    auto wi = m.wl_idx.find(a.workload);
    if (wi == m.wl_idx.end()) fail("%s (%s): unknown workload '%s'", where.c_str(), a.name.c_str(), a.workload.c_str());
    const std::string w2 = "admission " + a.name;
    if (const Json* v = x.get("after_bundles")) for (auto& s : as_arr(*v, w2 + ".after_bundles")) a.after.push_back(as_str(s, w2 + ".after_bundles[]"));
    if (const Json* v = x.get("when"))
      for (auto& c : as_arr(*v, w2 + ".when")) {
        Cond cd;
        cd.var = as_str(member(c, "var", w2 + ".when[]"), w2 + ".when.var");
        cd.mn = as_int(member(c, "min", w2 + ".when[]"), w2 + ".when.min", 0, INT_MAX / 2);
        if (const Json* mx = c.get("max")) {
          cd.mx = as_int(*mx, w2 + ".when.max", 0, INT_MAX / 2);
          if (cd.mx < cd.mn) fail("%s: when %s has max %lld < min %lld (can never hold)", w2.c_str(), cd.var.c_str(), cd.mx, cd.mn);
        }
        a.when.push_back(cd);
      }
    if (const Json* t = x.get("at_us")) if (!is_null(t)) a.at_us = as_int(*t, w2 + ".at_us", 0, 1ll << 50);
    a.base = as_versions(x.get("base_versions"), w2 + ".base_versions");
    a.publishes = as_versions(x.get("publishes"), w2 + ".publishes");
    if (const Json* bd = x.get("bundle_dir")) if (!is_null(bd)) a.bundle_dir = as_rel_path(*bd, w2 + ".bundle_dir");
    if (const Json* cp = x.get("compile")) if (!is_null(cp)) {
      a.compile_workload = as_rel_path(member(*cp, "workload", w2 + ".compile"), w2 + ".compile.workload");
      a.compile_data_dir = cp->get("data_dir") ? as_rel_path(*cp->get("data_dir"), w2 + ".compile.data_dir") : ".";
      as_versions(cp->get("base_versions"), w2 + ".compile.base_versions");   // checked; the admission's own base is used
    }
    const Workload& w = m.workloads[wi->second];
    auto declared = [&](const std::string& v) { return std::find(w.variables.begin(), w.variables.end(), v) != w.variables.end(); };
    for (auto& kv : a.publishes) {
      m.var_id(kv.first, w2 + ".publishes");
      if (!declared(kv.first)) fail("%s publishes '%s', which its workload does not declare", w2.c_str(), kv.first.c_str());
      if (!a.base.count(kv.first)) fail("%s publishes '%s' but has no base version for it", w2.c_str(), kv.first.c_str());
    }
    for (auto& kv : a.base) m.var_id(kv.first, w2 + ".base_versions");
    for (auto& c : a.when) m.var_id(c.var, w2 + ".when");
    m.adm_idx[a.name] = (int)m.adms.size();
    m.adms.push_back(a);
  }
  for (auto& a : m.adms)
    for (auto& d : a.after) {
      if (!m.adm_idx.count(d)) fail("admission %s: after_bundles names unknown admission '%s'", a.name.c_str(), d.c_str());
      if (d == a.name) fail("admission %s waits for itself", a.name.c_str());
    }
  for (auto& b : m.buffers)
    if (std::none_of(m.adms.begin(), m.adms.end(), [&](const Admission& a) { return a.workload == b.owner; }))
      fail("buffer %s: owner workload '%s' has no admission", b.name.c_str(), b.owner.c_str());
  return m;
}

// ---------------------------------------------------------------------------------------------- serial simulation
bool conds_hold(const Admission& a, const std::vector<long long>& live, const Manifest& m) {
  for (auto& c : a.when) {
    const long long v = live[m.var_idx.at(c.var)];
    if (v < c.mn || v > c.mx) return false;
  }
  return true;
}
// One admission at a time, the first (in manifest order) whose conditions hold, time conditions ignored; a
// publishing admission moves its variables from its base to the published versions. Fails with the reason for every
// admission that no order reaches.
std::vector<std::string> simulate(const Manifest& m) {
  std::vector<long long> live(m.vars.size(), 0);
  std::vector<char> done(m.adms.size(), 0);
  std::vector<std::string> order;
  for (size_t left = m.adms.size(); left > 0; --left) {
    int pick = -1;
    for (size_t i = 0; i < m.adms.size() && pick < 0; ++i) {
      const Admission& a = m.adms[i];
      if (done[i]) continue;
      bool ok = conds_hold(a, live, m);
      for (auto& d : a.after) ok = ok && done[m.adm_idx.at(d)];
      for (auto& kv : a.publishes) ok = ok && live[m.var_idx.at(kv.first)] == a.base.at(kv.first);
      if (ok) pick = (int)i;
    }
    if (pick < 0) {
      std::string why;
      for (size_t i = 0; i < m.adms.size(); ++i) {
        if (done[i]) continue;
        const Admission& a = m.adms[i];
        why += "\n  " + a.name + ":";
        for (auto& d : a.after) if (!done[m.adm_idx.at(d)]) why += " waits for bundle " + d + ";";
        for (auto& c : a.when) {
          const long long v = live[m.var_idx.at(c.var)];
          if (v < c.mn || v > c.mx)
            why += " needs " + c.var + " in [" + std::to_string(c.mn) + "," + (c.mx == LLONG_MAX ? "inf" : std::to_string(c.mx)) + "] but it is " + std::to_string(v) + ";";
        }
        for (auto& kv : a.publishes) {
          const long long v = live[m.var_idx.at(kv.first)];
          if (v != a.base.at(kv.first)) why += " compiled for " + kv.first + "=" + std::to_string(a.base.at(kv.first)) + " but the flow gives " + std::to_string(v) + ";";
        }
      }
      fail("the manifest cannot complete (%zu of %zu admissions run in the serial simulation):%s", order.size(), m.adms.size(), why.c_str());
    }
    done[pick] = 1;
    order.push_back(m.adms[pick].name);
    for (auto& kv : m.adms[pick].publishes) live[m.var_idx.at(kv.first)] = kv.second;
  }
  return order;
}

// ---------------------------------------------------------------------------------------------- bundles
struct Bundle {
  std::vector<MvmTaskDesc> t; std::vector<int32_t> s, a;
  Json meta; std::string dir;
  std::map<int, std::string> var_name;   // local id -> name
  VerMap var_base;                       // variable -> base version the bundle was compiled for
  std::map<int, std::string> buf_name;   // local index -> name
};

Bundle read_bundle(const std::string& dir) {
  Bundle r; r.dir = dir;
  r.meta = Parser(read_file(dir + "/metadata.json")).parse();
  if (as_int(member(r.meta, "abi_version", dir), dir + ".abi_version") != MVM_ABI_VERSION) fail("%s: abi_version is not %d", dir.c_str(), MVM_ABI_VERSION);
  const long long nt = as_int(member(r.meta, "task_count", dir), dir + ".task_count", 1, INT_MAX);
  const long long ne = as_int(member(r.meta, "edge_count", dir), dir + ".edge_count", 0, INT_MAX);
  const long long nw = as_int(member(r.meta, "args_words", dir), dir + ".args_words", 0, INT_MAX);
  r.t = read_bin<MvmTaskDesc>(dir + "/tasks.bin");
  r.s = read_bin<int32_t>(dir + "/successors.bin");
  r.a = read_bin<int32_t>(dir + "/args.bin");
  if ((long long)r.t.size() != nt || (long long)r.s.size() != ne || (long long)r.a.size() != nw) fail("%s: binary files do not match the metadata counts", dir.c_str());
  for (auto& v : as_arr(member(r.meta, "variables", dir), dir + ".variables")) {
    const std::string& nm = as_str(member(v, "name", dir), dir + ".variables.name");
    r.var_name[(int)as_int(member(v, "id", dir), dir + ".variables.id", 0, 1 << 20)] = nm;
    r.var_base[nm] = as_int(member(v, "base_version", dir), dir + ".variables.base_version", 0, INT_MAX / 2);
  }
  const auto& bufs = as_arr(member(r.meta, "buffers", dir), dir + ".buffers");
  for (size_t i = 0; i < bufs.size(); ++i) {
    const Json* ix = bufs[i].get("index");
    r.buf_name[ix ? (int)as_int(*ix, dir + ".buffers.index", 0, 1 << 24) : (int)i] = as_str(member(bufs[i], "name", dir), dir + ".buffers.name");
  }
  return r;
}

// Version shift: a bundle compiled with base b for a variable it publishes is the same program with every wait and
// publish of that variable moved by (target - b), valid when no read of that variable is by absolute version (the
// metadata lists the reads). Returns "" when applied, else the reason it does not apply.
std::string rebase(Bundle& r, const VerMap& to) {
  std::map<int, long long> shift;
  for (auto& kv : r.var_name) {
    bool published = false;
    for (auto& t : r.t) if (t.pub_var == kv.first) { published = true; break; }
    if (!published) continue;
    auto f = r.var_base.find(kv.second);
    auto g = to.find(kv.second);
    if (f == r.var_base.end() || g == to.end()) return "no base version for published variable " + kv.second;
    if (g->second == f->second) continue;
    if (const Json* reads = r.meta.get("reads"))
      for (auto& rd : reads->a)
        if (rd.get("var") && (int)rd.get("var")->n == kv.first) return "the bundle reads " + kv.second + " by absolute version";
    shift[kv.first] = g->second - f->second;
  }
  for (auto& kv : shift) r.var_base[r.var_name.at(kv.first)] = to.at(r.var_name.at(kv.first));
  for (auto& t : r.t) {
    auto p = shift.find(t.pub_var);
    if (t.pub_var >= 0 && p != shift.end()) { t.pub_ver += (int)p->second; if (t.pub_ver < 1) return "shifted publish version below 1"; }
    auto w = shift.find(t.wait_var);
    if (t.wait_var >= 0 && w != shift.end()) { t.wait_ver += (int)w->second; if (t.wait_ver < 0) return "shifted wait version below 0"; }
  }
  return "";
}

// Buffer-argument positions of every registry operator.
const std::map<int, std::vector<std::pair<bool, bool>>>& registry_args() {   // id -> per argument (is buffer, optional)
  static std::map<int, std::vector<std::pair<bool, bool>>> m;
  if (m.empty()) {
    struct Op { int id; const char* sig; };
    static const Op ops[] = {
#define X(n, id, sig) {id, sig},
#include "../../include/mvm_ops_list.inc"
#undef X
    };
    for (const Op& o : ops) {
      std::vector<std::pair<bool, bool>> v;
      std::string s(o.sig);
      size_t p = 0;
      while (p < s.size()) {
        size_t e = s.find(',', p); if (e == std::string::npos) e = s.size();
        const std::string ty = s.substr(s.find(':', p) + 1, e - s.find(':', p) - 1);
        v.push_back({ty == "buf" || ty == "buf?", ty == "buf?"});
        p = e + 1;
      }
      m[o.id] = v;
    }
  }
  return m;
}

// Local buffer and variable ids to the manifest's global tables.
void remap(Bundle& r, const Manifest& m, const std::string& what) {
  std::map<int, int> bmap, vmap;
  for (auto& kv : r.buf_name) {
    auto it = m.buf_idx.find(kv.second);
    if (it == m.buf_idx.end()) fail("%s: buffer '%s' is not in manifest.buffers", what.c_str(), kv.second.c_str());
    bmap[kv.first] = it->second;
  }
  for (auto& kv : r.var_name) vmap[kv.first] = m.var_id(kv.second, what);
  const auto& reg = registry_args();
  for (size_t i = 0; i < r.t.size(); ++i) {
    MvmTaskDesc& t = r.t[i];
    auto op = reg.find(t.op_id);
    if (op == reg.end()) fail("%s: task %zu: op id %d is not in the operator registry", what.c_str(), i, t.op_id);
    if (t.args_words != (int)op->second.size() || t.args_off < 0 || (long long)t.args_off + t.args_words > (long long)r.a.size())
      fail("%s: task %zu: bad argument range", what.c_str(), i);
    for (int k = 0; k < t.args_words; ++k) {
      if (!op->second[k].first) continue;
      int32_t& w = r.a[t.args_off + k];
      if (w == -1 && op->second[k].second) continue;
      auto it = bmap.find(w);
      if (it == bmap.end()) fail("%s: task %zu arg %d: local buffer index %d is not in the bundle's buffer table", what.c_str(), i, k, w);
      w = it->second;
    }
    for (int32_t* v : {&t.wait_var, &t.pub_var}) {
      if (*v < 0) continue;
      auto it = vmap.find(*v);
      if (it == vmap.end()) fail("%s: task %zu: local version variable %d is not declared in the bundle", what.c_str(), i, *v);
      *v = it->second;
    }
  }
}

// ---------------------------------------------------------------------------------------------- the run
struct Options {
  std::string root, out, dump;
  int windows = 4, blocks = 0, timeout_s = 120;
  bool check_only = false, quiet = false;
};

enum class St { PENDING, SUBMITTED, DONE, FAILED };
struct Runtime {
  St st = St::PENDING;
  std::vector<long long> wids;
  int tasks = 0;
  std::string how;
  double t_submit = -1, t_done = -1;
  std::vector<int> live_done;
};

class Runner {
 public:
  Runner(Manifest m, Options o) : m_(std::move(m)), o_(std::move(o)) {}

  int run() {
    order_ = simulate(m_);
    load_bundles();
    if (o_.check_only) {
      printf("OK: manifest, %zu bundles and the version flow are consistent (serial order %s ... %s)\n", m_.adms.size(), order_.front().c_str(), order_.back().c_str());
      return 0;
    }
    if (!o_.out.empty()) mkdir(o_.out.c_str(), 0755);
    KvmConfig cfg; kvm_config_default(&cfg);
    size_t max_t = 1, max_e = 1;
    for (auto& b : bundles_) { max_t = std::max(max_t, b->t.size()); max_e = std::max(max_e, b->s.size()); }
    int wt = 256;
    while ((size_t)wt < max_t && wt < (1 << 16)) wt <<= 1;
    cfg_tasks_ = wt;                                    // a bundle above a window streams in windows
    cfg_edges_ = (int)std::min<size_t>(std::max<size_t>(max_e, 1024), (size_t)1 << 22);
    cfg.window_cap = o_.windows; cfg.window_tasks = cfg_tasks_; cfg.window_edges = cfg_edges_;
    cfg.num_vars = std::max<int>(1, (int)m_.vars.size());
    cfg.blocks = o_.blocks; cfg.trace_on = 0;
    cfg.timeout_us = (unsigned long long)o_.timeout_s * 1000000ull;
    cfg.backpressure_ms = o_.timeout_s * 1000;
    ex_.reset(kvm_create(&cfg));
    if (!ex_) fail("kvm_create: %s", kvm_last_error(nullptr));
    allocate_buffers();
    if (kvm_start(ex_.get()) < 0) fail("kvm_start: %s", kvm_last_error(ex_.get()));
    t0_ = std::chrono::steady_clock::now();
    bool ok = loop();
    kvm_close(ex_.get());
    KvmResult r{};
    const int frc = kvm_finish(ex_.get(), &r);
    ok = ok && frc == 0 && r.err_code == 0;
    if (r.err_code && !o_.quiet) fprintf(stderr, "device error %d at task %d (a=%d b=%d)\n", r.err_code, r.err_slot, r.err_a, r.err_b);
    if (!errors_.empty() && !o_.quiet) fprintf(stderr, "%s", errors_.c_str());
    if (!o_.out.empty()) { write_summary(r, ok); dump_buffers(); }
    printf("%s: %d/%d tasks, %.3f ms, %zu admissions\n", ok ? "OK" : "FAIL", r.done, r.admitted, r.kernel_ms, m_.adms.size());
    return ok ? 0 : 1;
  }

 private:
  Manifest m_; Options o_;
  std::unique_ptr<KvmExec, void (*)(KvmExec*)> ex_{nullptr, kvm_destroy};
  std::vector<std::unique_ptr<Bundle>> bundles_;   // per admission, remapped
  std::vector<std::string> how_;
  std::vector<Runtime> rt_;
  std::vector<std::string> order_;
  std::chrono::steady_clock::time_point t0_;
  std::string errors_;
  long long next_wid_ = 0;                            // window ids are consecutive: this runner is the only submitter
  int cfg_tasks_ = 0, cfg_edges_ = 0;                 // window slot size

  double now_us() const { return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0_).count(); }
  bool exists(const std::string& f) const { struct stat sb; return stat(f.c_str(), &sb) == 0; }

  std::vector<std::string> scratch_;                  // directories of bundles compiled on demand (removed at exit)

  // Compiles an admission's workload file in-process (the same compiler as kvm_compile) for the admission's base
  // versions into a scratch directory, so `file` initial values sit beside the bundle like a precompiled one's.
  Bundle compile_admission(const Admission& a) {
    if (a.compile_workload.empty()) fail("admission %s: no usable bundle and no compile entry", a.name.c_str());
    char tmpl[] = "/tmp/kvm_run_compile.XXXXXX";
    if (!mkdtemp(tmpl)) fail("admission %s: cannot create a scratch directory", a.name.c_str());
    scratch_.push_back(tmpl);
    const std::string data_dir = m_.root + "/" + a.compile_data_dir, out = std::string(tmpl);
    std::map<std::string, int> base;
    for (auto& kv : a.base) base[kv.first] = (int)kv.second;
    try {
      const std::string text = read_file(m_.root + "/" + a.compile_workload);
      const kvmc::Bundle b = kvmc::compile(Parser(text).parse(), base, &data_dir);
      auto put = [&](const std::string& f, const void* p, size_t n) {
        FILE* fp = fopen((out + "/" + f).c_str(), "wb");
        if (!fp || (n && fwrite(p, 1, n, fp) != n) || fclose(fp) != 0) fail("admission %s: cannot write %s", a.name.c_str(), f.c_str());
      };
      for (const std::string& f : b.files) {     // the file's directories, then the file
        for (size_t k = f.find('/'); k != std::string::npos; k = f.find('/', k + 1)) mkdir((out + "/" + f.substr(0, k)).c_str(), 0777);
        const std::string d = read_file(data_dir + "/" + f);
        put(f, d.data(), d.size());
      }
      put("tasks.bin", b.tasks.data(), b.tasks.size() * sizeof(MvmTaskDesc));
      put("successors.bin", b.succ.data(), b.succ.size() * 4);
      put("args.bin", b.args.data(), b.args.size() * 4);
      put("metadata.json", b.metadata.data(), b.metadata.size());
    } catch (const ManifestError&) {
      throw;
    } catch (const std::exception& e) {
      fail("admission %s: compiling %s: %s", a.name.c_str(), a.compile_workload.c_str(), e.what());
    }
    return read_bundle(out);
  }

 public:
  ~Runner() {
    for (auto& d : scratch_)
      nftw(d.c_str(), [](const char* p, const struct stat*, int, struct FTW*) { return remove(p); }, 16, FTW_DEPTH | FTW_PHYS);
  }

 private:
  // Each admission's bundle, the first of: its own directory, the last bundle of the same workload, a compile of its
  // workload file (the `compile` entry); the first two shifted when compiled for other base versions and skipped
  // when no shift applies. Then remapped onto the global tables and validated against them.
  void load_bundles() {
    std::map<std::string, Bundle> last;   // workload -> last loaded bundle (local ids)
    std::vector<MvmBuf> table;
    for (auto& b : m_.buffers) table.push_back(MvmBuf{nullptr, b.rows, b.cols, b.cols, b.dtype, {0, 0}});
    for (auto& a : m_.adms) {
      Bundle r;
      std::string how;
      bool have = false;
      auto needs_shift = [&](const Bundle& b) {
        for (auto& kv : a.publishes) { auto f = b.var_base.find(kv.first); if (f == b.var_base.end() || f->second != a.base.at(kv.first)) return true; }
        return false;
      };
      std::string why_not;
      auto try_shift = [&](Bundle& t, const char* what) {
        if (!needs_shift(t)) { how = what; return true; }
        const std::string why = rebase(t, a.base);
        if (why.empty()) { how = std::string(what) + ", versions shifted"; return true; }
        why_not += std::string(" the ") + what + " bundle cannot be shifted to its base versions:" + why + ";";
        return false;
      };
      if (!a.bundle_dir.empty() && exists(m_.root + "/" + a.bundle_dir + "/metadata.json")) {
        Bundle t = read_bundle(m_.root + "/" + a.bundle_dir);
        if (try_shift(t, "precompiled")) { r = std::move(t); have = true; }
      }
      if (!have && last.count(a.workload)) {
        Bundle t = last.at(a.workload);
        if (try_shift(t, "previous bundle of the workload")) { r = std::move(t); have = true; }
      }
      if (!have && !a.compile_workload.empty()) { r = compile_admission(a); how = "compiled on demand"; have = true; }
      if (!have)
        fail("admission %s: no bundle (bundle_dir '%s' missing or unusable, no usable earlier bundle of workload %s, no compile entry);%s",
             a.name.c_str(), a.bundle_dir.c_str(), a.workload.c_str(), why_not.c_str());
      last[a.workload] = r;
      remap(r, m_, "admission " + a.name);
      char err[1024] = {0};
      if (kvm_validate(r.t.data(), (int)r.t.size(), r.s.data(), (int)r.s.size(), r.a.data(), (int)r.a.size(), table.data(), (int)table.size(),
                       std::max<int>(1, (int)m_.vars.size()), err, sizeof err) < 0)
        fail("admission %s: %s", a.name.c_str(), err);
      bundles_.push_back(std::make_unique<Bundle>(std::move(r)));
      how_.push_back(how);
    }
  }

  // Buffers are fixed at launch: each initialised from the bundle of the first admission of its owner workload.
  void allocate_buffers() {
    for (size_t bi = 0; bi < m_.buffers.size(); ++bi) {
      const BufDecl& b = m_.buffers[bi];
      size_t ai = 0;
      while (m_.adms[ai].workload != b.owner) ++ai;
      const Bundle& own = *bundles_[ai];
      const Json* decl = nullptr;
      for (auto& jb : own.meta.need("buffers").a) if (jb.get("name") && jb.get("name")->s == b.name) { decl = &jb; break; }
      if (!decl) fail("buffer %s: its owner workload %s has no such buffer in its bundle", b.name.c_str(), b.owner.c_str());
      const int rows = (int)decl->num("rows", 0), cols = (int)decl->num("cols", 0), dtype = (int)decl->num("dtype", 0);
      if (rows != b.rows || cols != b.cols || dtype != b.dtype)
        fail("buffer %s: manifest says %dx%d dtype %d, owner bundle %dx%d dtype %d", b.name.c_str(), b.rows, b.cols, b.dtype, rows, cols, dtype);
      if (add_buffer_from_meta(ex_.get(), *decl, own.dir) != (int)bi) fail("buffer %s: index mismatch", b.name.c_str());
    }
  }

  bool windows_done(const Runtime& r) const {
    for (long long w : r.wids) if (kvm_window_done(ex_.get(), w) != 1) return false;
    return true;
  }

  void submit(size_t i) {
    Runtime& r = rt_[i];
    const Bundle& b = *bundles_[i];
    const int nt = (int)b.t.size(), ne = (int)b.s.size();
    r.tasks = nt;
    r.how = how_[i];
    int rc;
    if (nt <= cfg_tasks_ && ne <= cfg_edges_) {
      rc = kvm_submit(ex_.get(), b.t.data(), nt, b.s.data(), ne, b.a.data(), (int)b.a.size());
      if (rc >= 0) { r.wids.push_back(next_wid_++); }
    } else {
      rc = kvm_submit_stream(ex_.get(), b.t.data(), nt, b.s.data(), ne, b.a.data(), (int)b.a.size(), 0, o_.timeout_s * 1000);
      if (rc >= 0) for (int k = 0; k < rc; ++k) r.wids.push_back(next_wid_++);
    }
    if (rc < 0) {
      errors_ += m_.adms[i].name + ": submit failed: " + kvm_last_error(ex_.get()) + "\n";
      r.st = St::FAILED;
      return;
    }
    r.t_submit = now_us();
    r.st = St::SUBMITTED;
  }

  bool loop() {
    rt_.assign(m_.adms.size(), Runtime{});
    const size_t nv = std::max<size_t>(1, m_.vars.size());
    std::vector<int> live(nv, 0);
    size_t done = 0;
    while (done < m_.adms.size()) {
      if (now_us() > o_.timeout_s * 1e6) { errors_ += "the manifest did not complete within --timeout-s\n"; return false; }
      if (kvm_live_versions(ex_.get(), live.data(), (int)nv) < 0) { errors_ += std::string("live versions: ") + kvm_last_error(ex_.get()) + "\n"; return false; }
      for (size_t i = 0; i < m_.adms.size(); ++i) {
        Runtime& r = rt_[i];
        if (r.st == St::SUBMITTED && windows_done(r)) {
          r.st = St::DONE; r.t_done = now_us(); r.live_done = live; ++done;
          if (!o_.quiet) fprintf(stderr, "[%9.0f us] done %-16s %6d tasks\n", r.t_done, m_.adms[i].name.c_str(), r.tasks);
        }
        if (r.st == St::FAILED) return false;
      }
      for (size_t i = 0; i < m_.adms.size(); ++i) {
        if (rt_[i].st != St::PENDING) continue;
        const Admission& a = m_.adms[i];
        bool elig = a.at_us < 0 || now_us() >= (double)a.at_us;
        for (auto& d : a.after) elig = elig && rt_[m_.adm_idx.at(d)].st == St::DONE;
        for (auto& c : a.when) {
          const int v = live[m_.var_idx.at(c.var)];
          if (v > c.mx) { errors_ += a.name + ": version window passed (" + c.var + "=" + std::to_string(v) + " > max " + std::to_string(c.mx) + ")\n"; return false; }
          elig = elig && v >= c.mn;
        }
        for (auto& kv : a.publishes) {
          const int v = live[m_.var_idx.at(kv.first)], base = (int)a.base.at(kv.first);
          if (v > base) { errors_ += a.name + ": compiled for " + kv.first + "=" + std::to_string(base) + " but the live version is already " + std::to_string(v) + "\n"; return false; }
          elig = elig && v == base;
          for (size_t j = 0; j < m_.adms.size() && elig; ++j)   // one publisher of a variable in flight
            if (j != i && rt_[j].st == St::SUBMITTED && m_.adms[j].publishes.count(kv.first)) elig = false;
        }
        if (elig) {
          submit(i);
          if (rt_[i].st == St::FAILED) return false;
          if (!o_.quiet) fprintf(stderr, "[%9.0f us] admit %-15s %6d tasks (%s)\n", rt_[i].t_submit, a.name.c_str(), rt_[i].tasks, rt_[i].how.c_str());
        }
      }
      std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    return true;
  }

  void write_summary(const KvmResult& r, bool ok) {
    FILE* f = fopen((o_.out + "/summary.json").c_str(), "w");
    if (!f) { errors_ += "cannot write summary.json\n"; return; }
    fprintf(f, "{\"ok\": %s, \"done\": %d, \"admitted\": %d, \"kernel_ms\": %.3f, \"serial_order\": [", ok ? "true" : "false", r.done, r.admitted, r.kernel_ms);
    for (size_t i = 0; i < order_.size(); ++i) fprintf(f, "%s\"%s\"", i ? ", " : "", order_[i].c_str());
    fprintf(f, "], \"admissions\": [");
    for (size_t i = 0; i < m_.adms.size(); ++i) {
      const Runtime& t = rt_[i];
      fprintf(f, "%s{\"name\": \"%s\", \"workload\": \"%s\", \"tasks\": %d, \"windows\": %zu, \"how\": \"%s\", \"submitted_us\": %.1f, \"done_us\": %.1f, \"versions_at_done\": {",
              i ? ", " : "", m_.adms[i].name.c_str(), m_.adms[i].workload.c_str(), t.tasks, t.wids.size(), t.how.c_str(), t.t_submit, t.t_done);
      for (size_t v = 0; v < m_.vars.size() && v < t.live_done.size(); ++v) fprintf(f, "%s\"%s\": %d", v ? ", " : "", m_.vars[v].c_str(), t.live_done[v]);
      fprintf(f, "}}");
    }
    std::vector<int32_t> ver(std::max<size_t>(1, m_.vars.size()));
    kvm_versions(ex_.get(), ver.data(), (int)ver.size());
    fprintf(f, "], \"versions\": {");
    for (size_t v = 0; v < m_.vars.size(); ++v) fprintf(f, "%s\"%s\": %d", v ? ", " : "", m_.vars[v].c_str(), ver[v]);
    fprintf(f, "}}\n");
    fclose(f);
  }

  void dump_buffers() {
    if (o_.dump.empty()) return;
    std::regex re;
    try { re = std::regex(o_.dump); } catch (const std::regex_error& e) { errors_ += std::string("--dump: bad regex: ") + e.what() + "\n"; return; }
    for (size_t i = 0; i < m_.buffers.size(); ++i) {
      if (!std::regex_search(m_.buffers[i].name, re)) continue;
      const size_t n = (size_t)m_.buffers[i].rows * m_.buffers[i].cols;
      std::vector<float> v(n);
      if (kvm_read_buffer(ex_.get(), (int)i, v.data(), n) < 0) { errors_ += "dump " + m_.buffers[i].name + ": " + kvm_last_error(ex_.get()) + "\n"; continue; }
      FILE* f = fopen((o_.out + "/" + m_.buffers[i].name + ".bin").c_str(), "wb");
      if (!f || fwrite(v.data(), 4, n, f) != n) errors_ += "cannot write the dump of " + m_.buffers[i].name + "\n";
      if (f) fclose(f);
    }
  }
};

void usage() {
  fprintf(stderr, "usage: kvm_run DEMO_DIR [--out DIR] [--dump REGEX] [--windows N] [--blocks N] [--timeout-s N] [--check-only] [--quiet]\n"
                  "  runs every admission of DEMO_DIR/MANIFEST.json on one persistent kernel (stream mode)\n");
}

}  // namespace

int main(int argc, char** argv) {
  Options o;
  for (int i = 1; i < argc; ++i) {
    std::string a = argv[i];
    auto next = [&]() -> const char* { if (i + 1 >= argc) { usage(); exit(2); } return argv[++i]; };
    if (a == "--out") o.out = next();
    else if (a == "--dump") o.dump = next();
    else if (a == "--windows") o.windows = atoi(next());
    else if (a == "--blocks") o.blocks = atoi(next());
    else if (a == "--timeout-s") o.timeout_s = atoi(next());
    else if (a == "--check-only") o.check_only = true;
    else if (a == "--quiet") o.quiet = true;
    else if (a[0] == '-') { usage(); return 2; }
    else if (o.root.empty()) o.root = a;
    else { usage(); return 2; }
  }
  if (o.root.empty() || o.windows < 1 || o.timeout_s < 1) { usage(); return 2; }
  try {
    Runner r(parse_manifest(o.root), o);
    return r.run();
  } catch (const std::exception& e) {
    fprintf(stderr, "kvm_run: %s\n", e.what());
    printf("FAIL: %s\n", e.what());
    return 1;
  }
}
