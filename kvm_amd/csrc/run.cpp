// kvm_run: runs a demo directory (MANIFEST.json plus ABI-v2 bundles) on ONE persistent kernel in stream mode. It is
// the counterpart of the reference's demo runner (reference: demo/mvm_run.cu; manifest writer and CPU runner:
// frontend/mvmfe/demo.py, frontend/mvmfe/run_manifest.py). The runner knows nothing about models: buffers, version
// variables and the admission order come from the manifest.
//
//   kvm_run DEMO_DIR [--out DIR] [--dump REGEX] [--windows N] [--blocks N] [--timeout-s N]
//                    [--sched off|global|static|dynamic] [--shares a,b,..] [--check-only] [--quiet]
//
// The rules this runner applies (the manifest format's, frontend/mvmfe/demo.py:136-152):
//   * every `buffers` entry is one device allocation, initialised from the bundle of its owner workload and shared by
//     name by every bundle that names it;
//   * an admission may be submitted when its `at_us` has passed, every admission in its `after_bundles` has finished,
//     the live version of each `when` variable lies in [min, max], and, for every variable in its `publishes`, the
//     live version equals the admission's base version and no other admission publishing it is in flight;
//   * an admission that completes has advanced each published variable BY `publishes[var]`:
//     live after completion = base + publishes[var] (demo.py:136, mvm_run.cu:262);
//   * a bundle compiled for other base versions runs shifted (its waits and publications of a published variable
//     move by the difference) when it reads that variable by no absolute version;
//   * scheduler classes: one per class name, the `classes` entries first (their parameters: weight, min_cta, max_cta,
//     bw_cta, urgent_us), then each workload's `class` (default "default") not declared there; every task of an
//     admission runs in its workload's class (its workload_id). --sched dynamic (the default) applies them with the
//     device's class scheduler, static splits the workers by --shares, off and global run first-come first-served
//     (reference: demo/mvm_run.cu, class_id / apply_class_param and --sched).
// Before the GPU is touched the runner checks the manifest's shape, checks every bundle against the global tables
// (including that what it publishes is what its admission declares), and runs the version flow serially (one
// admission at a time, the first in manifest order whose gate is open; time ignored).
//
// --out DIR writes summary.json (per admission: tasks, windows, submission and completion times, live versions at
// completion; final versions) and DIR/<buffer>.bin for the buffers --dump matches (f32 values; i32 raw). The last
// stdout line is "OK: d/a tasks, X ms, N admissions" or "FAIL: <reason>"; exit 0 / 1, 2 for usage errors.
#include <algorithm>
#include <chrono>
#include <climits>
#include <ftw.h>
#include <map>
#include <memory>
#include <regex>
#include <set>
#include <sys/stat.h>
#include <thread>
#include <unistd.h>
#include "../../include/kvm_exec.h"
#include "compile.h"
#include "host_json.h"

using namespace kvmh;

namespace {

// ================================================================================================ reading the manifest
// Every problem the runner finds before launch is a ManifestProblem whose text starts with where it was found, as a
// JSON path ("$.admissions[2].when[0].min") or the name of the object concerned.
struct ManifestProblem : std::runtime_error { using std::runtime_error::runtime_error; };
[[noreturn]] void refuse(const std::string& where, const std::string& what) { throw ManifestProblem(where + ": " + what); }

// A position in a parsed JSON document, carrying its path so that every typed read can say where it failed.
class Node {
 public:
  Node(const Json* j, std::string path) : j_(j), path_(std::move(path)) {}
  const std::string& path() const { return path_; }
  bool given() const { return j_ && j_->t != Json::NUL; }
  bool is_object() const { return j_ && j_->t == Json::O; }

  Node field(const std::string& key) const {      // a member that must be there
    const Node n = opt(key);
    if (!n.j_) refuse(path_, "the key \"" + key + "\" is required");
    return n;
  }
  Node opt(const std::string& key) const {        // a member that may be absent (given() is false then)
    if (!is_object()) refuse(path_, "must be a JSON object");
    return Node(j_->get(key), path_ + "." + key);
  }
  std::vector<std::pair<std::string, Node>> members() const {
    if (!is_object()) refuse(path_, "must be a JSON object");
    std::vector<std::pair<std::string, Node>> v;
    for (auto& kv : j_->o) v.emplace_back(kv.first, Node(&kv.second, path_ + "." + kv.first));
    return v;
  }
  std::vector<Node> items() const {
    if (!j_ || j_->t != Json::A) refuse(path_, "must be a JSON array");
    std::vector<Node> v;
    for (size_t i = 0; i < j_->a.size(); ++i) v.emplace_back(&j_->a[i], path_ + "[" + std::to_string(i) + "]");
    return v;
  }
  long long whole(long long lo, long long hi) const {
    if (!j_ || j_->t != Json::N || !std::isfinite(j_->n) || std::floor(j_->n) != j_->n) refuse(path_, "must be a whole number");
    if (j_->n < (double)lo || j_->n > (double)hi)
      refuse(path_, "is " + std::to_string((long long)j_->n) + ", allowed " + std::to_string(lo) + " .. " + std::to_string(hi));
    return (long long)j_->n;
  }
  std::string text() const {
    if (!j_ || j_->t != Json::S || j_->s.empty()) refuse(path_, "must be a non-empty string");
    return j_->s;
  }
  std::string inner_path() const {                // a file or directory inside the demo directory
    const std::string s = text();
    if (s[0] == '/' || s.find("..") != std::string::npos) refuse(path_, "\"" + s + "\" leaves the demo directory (relative path without '..' required)");
    return s;
  }

 private:
  const Json* j_;
  std::string path_;
};

constexpr long long kMaxVersion = INT_MAX / 2;

struct Window { int var; long long lo, hi; };           // a `when` entry: lo <= live[var] <= hi
struct VarVersion { int var; long long v; };

struct WorkloadDecl { std::string name, cls; int cls_id = 0; std::vector<int> vars; };
struct BufferDecl { std::string name, owner; int rows, cols, dtype; };
struct AdmissionDecl {
  std::string name;
  int workload = -1;
  std::vector<int> after;                               // admissions that must have finished
  std::vector<Window> when;
  long long at_us = -1;                                 // -1: no time condition
  std::vector<VarVersion> base;                         // versions the bundle was compiled for
  std::vector<VarVersion> advance;                      // `publishes`: increments applied at completion
  std::string bundle_dir, compile_file, compile_data;
  long long base_of(int var) const { for (auto& b : base) if (b.var == var) return b.v; return -1; }
  bool publishes(int var) const { for (auto& p : advance) if (p.var == var) return true; return false; }
};

// The manifest with every name resolved to an index.
struct Plan {
  std::string root;
  std::vector<std::string> vars;
  std::vector<WorkloadDecl> workloads;
  std::vector<BufferDecl> buffers;
  std::vector<AdmissionDecl> adms;
  std::vector<std::string> class_names;                 // class ids: declared classes, then workloads' classes
  std::vector<std::map<std::string, long long>> class_params;
  int class_id(const std::string& n) {
    for (size_t i = 0; i < class_names.size(); ++i) if (class_names[i] == n) return (int)i;
    class_names.push_back(n);
    class_params.emplace_back();
    return (int)class_names.size() - 1;
  }

  static int find(const std::vector<std::string>& names, const std::string& n) {
    auto it = std::find(names.begin(), names.end(), n);
    return it == names.end() ? -1 : (int)(it - names.begin());
  }
  int var(const std::string& n) const { return find(vars, n); }
  int buffer(const std::string& n) const { for (size_t i = 0; i < buffers.size(); ++i) if (buffers[i].name == n) return (int)i; return -1; }
  int workload(const std::string& n) const { for (size_t i = 0; i < workloads.size(); ++i) if (workloads[i].name == n) return (int)i; return -1; }
  int admission(const std::string& n) const { for (size_t i = 0; i < adms.size(); ++i) if (adms[i].name == n) return (int)i; return -1; }
};

const char* const kClassParams[] = {"weight", "min_cta", "max_cta", "bw_cta", "urgent_us"};

std::vector<VarVersion> read_versions(const Node& n, const Plan& p, bool positive) {
  std::vector<VarVersion> out;
  if (!n.given()) return out;
  for (auto& [name, v] : n.members()) {
    const int id = p.var(name);
    if (id < 0) refuse(v.path(), "\"" + name + "\" is not a variable any workload declares");
    out.push_back({id, v.whole(positive ? 1 : 0, kMaxVersion)});
  }
  return out;
}

Plan read_plan(const std::string& root) {
  Plan p;
  p.root = root;
  const Json doc = Parser(read_file(root + "/MANIFEST.json")).parse();
  const Node top(&doc, "$");
  if (top.field("manifest_version").whole(LLONG_MIN / 2, LLONG_MAX / 2) != 1)
    refuse("$.manifest_version", "this runner reads manifest_version 1");

  if (const Node cls = top.opt("classes"); cls.given())
    for (auto& [cname, params] : cls.members()) {
      auto& dst = p.class_params[p.class_id(cname)];
      for (auto& [key, val] : params.members()) {
        bool known = false;
        for (const char* k : kClassParams) known = known || key == k;
        if (!known) refuse(val.path(), "\"" + key + "\" is not a scheduler class parameter (weight, min_cta, max_cta, bw_cta, urgent_us)");
        dst[key] = val.whole(key == "weight" ? 1 : 0, INT_MAX);
      }
    }

  const auto wls = top.field("workloads").members();
  if (wls.empty()) refuse("$.workloads", "declares no workload");
  for (auto& [wname, w] : wls) {
    WorkloadDecl d;
    d.name = wname;
    w.field("file").inner_path();
    w.field("tasks").whole(1, INT_MAX);
    w.field("edges").whole(0, INT_MAX);
    w.field("priority").whole(0, 1 << 20);
    d.cls = w.opt("class").given() ? w.opt("class").text() : "default";
    d.cls_id = p.class_id(d.cls);
    if (p.class_names.size() > KVM_MAX_CLASSES) refuse(w.path(), "more than " + std::to_string(KVM_MAX_CLASSES) + " scheduler classes");
    if (const Node vs = w.opt("variables"); vs.given())
      for (const Node& v : vs.items()) {
        const std::string vn = v.text();
        int id = p.var(vn);
        if (id < 0) { id = (int)p.vars.size(); p.vars.push_back(vn); }
        d.vars.push_back(id);
      }
    if (const Node req = w.opt("requirements"); req.given())
      if (const Node res = req.opt("resources"); res.given() && !res.items().empty())
        refuse(res.path(), "host resources are not provided by this runner (the game pack is not part of this build)");
    p.workloads.push_back(d);
  }

  for (auto& [bname, b] : top.field("buffers").members()) {
    BufferDecl d;
    d.name = bname;
    d.rows = (int)b.field("rows").whole(1, INT_MAX);
    d.cols = (int)b.field("cols").whole(1, INT_MAX);
    const std::string dt = b.field("dtype").text();
    d.dtype = dt == "f32" ? 0 : dt == "i32" ? 1 : dt == "bf16" ? 2 : -1;
    if (d.dtype < 0) refuse(b.path() + ".dtype", "\"" + dt + "\" is not one of f32, i32, bf16");
    if ((long long)d.rows * d.cols > (long long)INT_MAX) refuse(b.path(), "more than 2^31-1 elements");
    d.owner = b.field("owner").text();
    if (p.workload(d.owner) < 0) refuse(b.path() + ".owner", "no workload is called \"" + d.owner + "\"");
    p.buffers.push_back(d);
  }

  const std::vector<Node> list = top.field("admissions").items();
  if (list.empty()) refuse("$.admissions", "lists no admission");
  std::vector<std::vector<std::string>> after_names(list.size());
  for (size_t i = 0; i < list.size(); ++i) {
    const Node& x = list[i];
    AdmissionDecl a;
    a.name = x.field("name").text();
    if (p.admission(a.name) >= 0) refuse(x.path() + ".name", "\"" + a.name + "\" names an earlier admission too");
    const std::string wl = x.field("workload").text();
    a.workload = p.workload(wl);
    if (a.workload < 0) refuse(x.path() + ".workload", "no workload is called \"" + wl + "\"");
    if (const Node ab = x.opt("after_bundles"); ab.given()) for (const Node& n : ab.items()) after_names[i].push_back(n.text());
    if (const Node wh = x.opt("when"); wh.given())
      for (const Node& c : wh.items()) {
        const std::string vn = c.field("var").text();
        Window win{p.var(vn), c.field("min").whole(0, kMaxVersion), LLONG_MAX};
        if (win.var < 0) refuse(c.path() + ".var", "\"" + vn + "\" is not a variable any workload declares");
        if (c.opt("max").given()) win.hi = c.opt("max").whole(0, kMaxVersion);
        if (win.hi < win.lo) refuse(c.path(), "max " + std::to_string(win.hi) + " below min " + std::to_string(win.lo) + ": the window is empty");
        a.when.push_back(win);
      }
    if (const Node t = x.opt("at_us"); t.given()) a.at_us = t.whole(0, 1ll << 50);
    a.base = read_versions(x.opt("base_versions"), p, false);
    a.advance = read_versions(x.opt("publishes"), p, true);
    if (const Node bd = x.opt("bundle_dir"); bd.given()) a.bundle_dir = bd.inner_path();
    if (const Node cp = x.opt("compile"); cp.given()) {
      a.compile_file = cp.field("workload").inner_path();
      a.compile_data = cp.opt("data_dir").given() ? cp.opt("data_dir").inner_path() : ".";
      read_versions(cp.opt("base_versions"), p, false);    // shape-checked; the admission's own base versions are used
    }
    const WorkloadDecl& w = p.workloads[a.workload];
    for (const VarVersion& pv : a.advance) {
      const std::string& vn = p.vars[pv.var];
      if (std::find(w.vars.begin(), w.vars.end(), pv.var) == w.vars.end())
        refuse(x.path() + ".publishes." + vn, "workload \"" + w.name + "\" does not declare the variable");
      if (a.base_of(pv.var) < 0) refuse(x.path() + ".publishes." + vn, "a published variable needs an entry in base_versions");
    }
    p.adms.push_back(a);
  }
  for (size_t i = 0; i < list.size(); ++i)
    for (const std::string& n : after_names[i]) {
      const int j = p.admission(n);
      if (j < 0) refuse(list[i].path() + ".after_bundles", "no admission is called \"" + n + "\"");
      if (j == (int)i) refuse(list[i].path() + ".after_bundles", "the admission lists itself");
      p.adms[i].after.push_back(j);
    }
  for (const BufferDecl& b : p.buffers) {
    const int w = p.workload(b.owner);
    if (std::none_of(p.adms.begin(), p.adms.end(), [&](const AdmissionDecl& a) { return a.workload == w; }))
      refuse("$.buffers." + b.name, "its owner \"" + b.owner + "\" is never admitted, so nothing initialises it");
  }
  return p;
}

// ================================================================================================ the admission gate
// The state the gate looks at. `now_us` < 0 ignores time conditions (the dry run).
struct Flow {
  std::vector<long long> live;        // per variable
  std::vector<char> finished, in_flight;
  double now_us = -1;
};

struct Gate {
  bool open = true;                   // may be submitted now
  bool dead = false;                  // can never open again (a window passed, or a base version overtaken)
  std::string why;                    // what keeps it closed
  void close(const std::string& r, bool fatal = false) { open = false; dead = dead || fatal; why += (why.empty() ? "" : "; ") + r; }
};

// One gate for the dry run and the live loop, so both apply exactly the same rules.
Gate gate(const Plan& p, int ai, const Flow& f) {
  const AdmissionDecl& a = p.adms[ai];
  Gate g;
  if (f.now_us >= 0 && a.at_us >= 0 && f.now_us < (double)a.at_us) g.close("starts at " + std::to_string(a.at_us) + " us");
  for (int d : a.after)
    if (!f.finished[d]) g.close("after " + p.adms[d].name);
  for (const Window& w : a.when) {
    const long long v = f.live[w.var];
    if (v < w.lo || v > w.hi)
      g.close(p.vars[w.var] + " is " + std::to_string(v) + ", window [" + std::to_string(w.lo) + ", " +
              (w.hi == LLONG_MAX ? std::string("any") : std::to_string(w.hi)) + "]", v > w.hi);
  }
  for (const VarVersion& pv : a.advance) {
    const long long v = f.live[pv.var], b = a.base_of(pv.var);
    if (v != b) g.close("built for " + p.vars[pv.var] + " = " + std::to_string(b) + ", live " + std::to_string(v), v > b);
    for (size_t j = 0; j < p.adms.size(); ++j)
      if ((int)j != ai && f.in_flight[j] && p.adms[j].publishes(pv.var)) { g.close(p.vars[pv.var] + " is being published by " + p.adms[j].name); break; }
  }
  return g;
}

void complete(const Plan& p, int ai, Flow& f) {
  for (const VarVersion& pv : p.adms[ai].advance) f.live[pv.var] += pv.v;
  f.finished[ai] = 1;
}

// Serial run of the version flow: repeatedly the first admission (manifest order) whose gate is open. Returns the
// order, or refuses with every waiting admission's reason when the flow gets stuck.
std::vector<int> dry_run(const Plan& p) {
  Flow f;
  f.live.assign(p.vars.size(), 0);
  f.finished.assign(p.adms.size(), 0);
  f.in_flight.assign(p.adms.size(), 0);
  std::vector<int> order;
  while (order.size() < p.adms.size()) {
    int next = -1;
    for (size_t i = 0; i < p.adms.size() && next < 0; ++i)
      if (!f.finished[i] && gate(p, (int)i, f).open) next = (int)i;
    if (next < 0) {
      std::string stuck;
      for (size_t i = 0; i < p.adms.size(); ++i)
        if (!f.finished[i]) stuck += "\n  " + p.adms[i].name + ": " + gate(p, (int)i, f).why;
      refuse("version flow", "stuck after " + std::to_string(order.size()) + " of " + std::to_string(p.adms.size()) +
                             " admissions in the serial order; waiting:" + stuck);
    }
    order.push_back(next);
    complete(p, next, f);
  }
  return order;
}

// ================================================================================================ bundles
// One bundle as read from disk, with its local buffer and variable tables.
struct Program {
  std::string dir;
  Json meta;
  std::vector<MvmTaskDesc> tasks;
  std::vector<int32_t> succ, args;
  std::map<int, std::string> local_var;          // local variable id -> name
  std::map<std::string, long long> built_for;    // variable name -> base version the bundle was compiled with
  std::map<int, std::string> local_buf;          // local buffer index -> name
  std::string origin;                            // how the runner obtained it (summary.json)
};

Program load_program(const std::string& dir) {
  Program g;
  g.dir = dir;
  g.meta = Parser(read_file(dir + "/metadata.json")).parse();
  const Node m(&g.meta, dir + "/metadata.json");
  if (m.field("abi_version").whole(0, INT_MAX) != MVM_ABI_VERSION) refuse(m.path(), "abi_version is not " + std::to_string(MVM_ABI_VERSION));
  const long long nt = m.field("task_count").whole(1, INT_MAX), ne = m.field("edge_count").whole(0, INT_MAX), nw = m.field("args_words").whole(0, INT_MAX);
  g.tasks = read_bin<MvmTaskDesc>(dir + "/tasks.bin");
  g.succ = read_bin<int32_t>(dir + "/successors.bin");
  g.args = read_bin<int32_t>(dir + "/args.bin");
  if ((long long)g.tasks.size() != nt || (long long)g.succ.size() != ne || (long long)g.args.size() != nw)
    refuse(dir, "tasks.bin / successors.bin / args.bin sizes disagree with task_count / edge_count / args_words");
  for (const Node& v : m.field("variables").items()) {
    const std::string name = v.field("name").text();
    g.local_var[(int)v.field("id").whole(0, 1 << 20)] = name;
    g.built_for[name] = v.field("base_version").whole(0, kMaxVersion);
  }
  const std::vector<Node> bufs = m.field("buffers").items();
  for (size_t i = 0; i < bufs.size(); ++i) {
    const int idx = bufs[i].opt("index").given() ? (int)bufs[i].opt("index").whole(0, 1 << 24) : (int)i;
    g.local_buf[idx] = bufs[i].field("name").text();
  }
  return g;
}

// Local variable ids a bundle publishes (some task has pub_var = id).
std::set<int> published_ids(const Program& g) {
  std::set<int> s;
  for (const MvmTaskDesc& t : g.tasks) if (t.pub_var >= 0) s.insert(t.pub_var);
  return s;
}

// Moves every wait and publication of the variables the bundle publishes from the base it was built for to the
// admission's base. Returns an empty string when done, else why the bundle cannot be moved (it then stays as is).
std::string shift_to(Program& g, const std::map<std::string, long long>& target) {
  std::map<int, long long> delta;
  std::set<int> absolute_reads;
  if (const Json* reads = g.meta.get("reads"))
    for (const Json& r : reads->a) if (const Json* v = r.get("var")) absolute_reads.insert((int)v->n);
  for (int id : published_ids(g)) {
    auto nm = g.local_var.find(id);
    if (nm == g.local_var.end()) return "a task publishes undeclared local variable " + std::to_string(id);
    auto want = target.find(nm->second);
    if (want == target.end()) return "no base version given for published variable " + nm->second;
    const long long d = want->second - g.built_for[nm->second];
    if (d == 0) continue;
    if (absolute_reads.count(id)) return nm->second + " is read at an absolute version inside the bundle";
    delta[id] = d;
  }
  std::vector<MvmTaskDesc> moved = g.tasks;
  for (MvmTaskDesc& t : moved) {
    if (auto it = delta.find(t.pub_var); t.pub_var >= 0 && it != delta.end()) {
      t.pub_ver += (int)it->second;
      if (t.pub_ver < 1) return "a publication would move below version 1";
    }
    if (auto it = delta.find(t.wait_var); t.wait_var >= 0 && it != delta.end()) {
      t.wait_ver += (int)it->second;
      if (t.wait_ver < 0) return "a wait would move below version 0";
    }
  }
  g.tasks.swap(moved);
  for (auto& [id, d] : delta) g.built_for[g.local_var[id]] += d;
  return "";
}

// The admission's declared publications against the bundle: each published variable's last version must be its base
// plus the declared increment, and a bundle may publish nothing its admission does not declare (the runner's
// in-flight exclusion and the version flow rest on that).
void check_publications(const Program& g, const AdmissionDecl& a, const Plan& p) {
  std::map<std::string, int> last;
  for (const MvmTaskDesc& t : g.tasks)
    if (t.pub_var >= 0) {
      const std::string& n = g.local_var.at(t.pub_var);
      last[n] = std::max(last.count(n) ? last[n] : 0, (int)t.pub_ver);
    }
  for (auto& [name, top] : last) {
    const int id = p.var(name);
    if (id < 0 || !a.publishes(id)) refuse("admission " + a.name, "its bundle publishes " + name + ", which the admission's publishes does not declare");
  }
  for (const VarVersion& pv : a.advance) {
    const std::string& name = p.vars[pv.var];
    const long long want = a.base_of(pv.var) + pv.v;
    auto it = last.find(name);
    if (it == last.end()) refuse("admission " + a.name, "declares publishes " + name + " +" + std::to_string(pv.v) + " but its bundle publishes no version of it");
    if (it->second != want)
      refuse("admission " + a.name, "its bundle leaves " + name + " at " + std::to_string(it->second) + ", the manifest says " +
                                        std::to_string(a.base_of(pv.var)) + " + " + std::to_string(pv.v) + " = " + std::to_string(want));
  }
}

// Operator id -> which argument words are buffer indices (first) and which of those may be -1 (second), from the
// registry signatures.
const std::map<int, std::vector<std::pair<bool, bool>>>& buffer_slots() {
  static const std::map<int, std::vector<std::pair<bool, bool>>> table = [] {
    std::map<int, std::vector<std::pair<bool, bool>>> m;
    struct Sig { int id; const char* sig; };
    static const Sig sigs[] = {
#define X(n, id, sig) {id, sig},
#include "../../include/mvm_ops_list.inc"
#undef X
    };
    for (const Sig& s : sigs) {
      auto& v = m[s.id];
      std::string rest(s.sig);
      while (!rest.empty()) {
        const size_t comma = rest.find(',');
        const std::string item = rest.substr(0, comma);
        const std::string type = item.substr(item.find(':') + 1);
        v.push_back({type == "buf" || type == "buf?", type == "buf?"});
        rest = comma == std::string::npos ? "" : rest.substr(comma + 1);
      }
    }
    return m;
  }();
  return table;
}

// Rewrites the bundle's local buffer and variable ids into the manifest's global tables.
void bind_globals(Program& g, const Plan& p, const std::string& who) {
  std::map<int, int> buf, var;
  for (auto& [local, name] : g.local_buf) {
    buf[local] = p.buffer(name);
    if (buf[local] < 0) refuse(who, "bundle buffer \"" + name + "\" is not declared in $.buffers");
  }
  for (auto& [local, name] : g.local_var) {
    var[local] = p.var(name);
    if (var[local] < 0) refuse(who, "bundle variable \"" + name + "\" is not declared by any workload");
  }
  const auto& slots = buffer_slots();
  for (size_t i = 0; i < g.tasks.size(); ++i) {
    MvmTaskDesc& t = g.tasks[i];
    const std::string at = who + ", task " + std::to_string(i);
    auto op = slots.find(t.op_id);
    if (op == slots.end()) refuse(at, "operator id " + std::to_string(t.op_id) + " is not in the registry");
    if (t.args_words != (int)op->second.size() || t.args_off < 0 || (long long)t.args_off + t.args_words > (long long)g.args.size())
      refuse(at, "argument words outside args.bin or not the operator's arity");
    for (int k = 0; k < t.args_words; ++k) {
      if (!op->second[k].first) continue;
      int32_t& w = g.args[t.args_off + k];
      if (w == -1 && op->second[k].second) continue;
      auto it = buf.find(w);
      if (it == buf.end()) refuse(at, "argument " + std::to_string(k) + " names local buffer " + std::to_string(w) + ", absent from the bundle's table");
      w = it->second;
    }
    for (int32_t* v : {&t.wait_var, &t.pub_var}) {
      if (*v < 0) continue;
      auto it = var.find(*v);
      if (it == var.end()) refuse(at, "local variable " + std::to_string(*v) + " is not in the bundle's table");
      *v = it->second;
    }
  }
}

// ================================================================================================ the run
struct Options {
  std::string root, out, dump, sched = "dynamic";
  std::vector<int> shares;
  int windows = 4, blocks = 0, timeout_s = 120;
  bool check_only = false, quiet = false;
};

enum class Phase { WAITING, RUNNING, FINISHED, FAILED };
struct Track {
  Phase phase = Phase::WAITING;
  std::vector<long long> windows;     // window ids of its submission
  double submitted_us = -1, done_us = -1;
  std::vector<int32_t> live_at_done;
};

class ManifestRun {
 public:
  ManifestRun(Plan p, Options o) : p_(std::move(p)), o_(std::move(o)) {}
  ~ManifestRun() {
    for (const std::string& d : scratch_dirs_)
      nftw(d.c_str(), [](const char* f, const struct stat*, int, struct FTW*) { return remove(f); }, 16, FTW_DEPTH | FTW_PHYS);
  }

  int go() {
    if (o_.sched == "static" && o_.shares.size() != p_.class_names.size())
      refuse("--shares", "--sched static needs one share per class (" + std::to_string(p_.class_names.size()) + " classes)");
    prepare_programs();
    order_ = dry_run(p_);
    if (o_.check_only) {
      printf("OK: %zu admissions, bundles and version flow consistent; serial order %s",
             p_.adms.size(), p_.adms[order_.front()].name.c_str());
      for (size_t i = 1; i < order_.size(); ++i) printf(" %s", p_.adms[order_[i]].name.c_str());
      printf("\n");
      return 0;
    }
    if (!o_.out.empty()) mkdir(o_.out.c_str(), 0755);
    launch();
    const bool drove = drive();
    kvm_close(ex_.get());
    KvmResult r{};
    const bool ok = drove && kvm_finish(ex_.get(), &r) == 0 && r.err_code == 0;
    if (r.err_code && !o_.quiet) fprintf(stderr, "device error %d at task %d (a=%d b=%d)\n", r.err_code, r.err_slot, r.err_a, r.err_b);
    if (!problems_.empty() && !o_.quiet) fprintf(stderr, "%s", problems_.c_str());
    if (!o_.out.empty()) { write_summary(r, ok); write_dumps(); }
    printf("%s: %d/%d tasks, %.3f ms, %zu admissions\n", ok ? "OK" : "FAIL", r.done, r.admitted, r.kernel_ms, p_.adms.size());
    return ok ? 0 : 1;
  }

 private:
  Plan p_;
  Options o_;
  std::vector<int> order_;
  std::vector<Program> progs_;                   // per admission, bound to the global tables
  std::vector<Track> track_;
  std::vector<std::string> scratch_dirs_;
  std::unique_ptr<KvmExec, void (*)(KvmExec*)> ex_{nullptr, kvm_destroy};
  std::chrono::steady_clock::time_point t0_;
  std::string problems_;
  long long window_serial_ = 0;                  // the runner is the only submitter, so window ids are consecutive
  int slot_tasks_ = 0, slot_edges_ = 0;

  double elapsed_us() const { return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0_).count(); }
  static bool has_file(const std::string& f) { struct stat sb; return stat(f.c_str(), &sb) == 0; }

  // Compiles the admission's workload file for its base versions (the compiler kvm_compile links) into a scratch
  // directory that receives the data files its `file` inits name, then loads it like a precompiled bundle.
  Program compile_for(const AdmissionDecl& a) {
    char dir_t[] = "/tmp/kvm_run_bundle.XXXXXX";
    if (!mkdtemp(dir_t)) refuse("admission " + a.name, "no scratch directory for the on-demand compile");
    const std::string dir = dir_t, data = p_.root + "/" + a.compile_data;
    scratch_dirs_.push_back(dir);
    std::map<std::string, int> base;
    for (const VarVersion& b : a.base) base[p_.vars[b.var]] = (int)b.v;
    auto save = [&](const std::string& rel, const void* bytes, size_t n) {
      for (size_t k = rel.find('/'); k != std::string::npos; k = rel.find('/', k + 1)) mkdir((dir + "/" + rel.substr(0, k)).c_str(), 0777);
      FILE* fp = fopen((dir + "/" + rel).c_str(), "wb");
      const bool good = fp && (n == 0 || fwrite(bytes, 1, n, fp) == n);
      if (fp && fclose(fp) != 0) refuse("admission " + a.name, "writing " + rel + " failed");
      if (!good) refuse("admission " + a.name, "writing " + rel + " failed");
    };
    try {
      const kvmc::Bundle b = kvmc::compile(Parser(read_file(p_.root + "/" + a.compile_file)).parse(), base, &data);
      for (const std::string& f : b.files) { const std::string bytes = read_file(data + "/" + f); save(f, bytes.data(), bytes.size()); }
      save("tasks.bin", b.tasks.data(), b.tasks.size() * sizeof(MvmTaskDesc));
      save("successors.bin", b.succ.data(), b.succ.size() * sizeof(int32_t));
      save("args.bin", b.args.data(), b.args.size() * sizeof(int32_t));
      save("metadata.json", b.metadata.data(), b.metadata.size());
    } catch (const ManifestProblem&) {
      throw;
    } catch (const std::exception& e) {
      refuse("admission " + a.name, "compiling " + a.compile_file + " failed: " + e.what());
    }
    Program g = load_program(dir);
    g.origin = "compiled on demand";
    return g;
  }

  // A bundle per admission: its bundle_dir, else the workload's previous bundle, each moved to the admission's base
  // versions when it was built for others; else a compile of its `compile` entry. Then checked and bound.
  void prepare_programs() {
    std::map<int, Program> previous;             // workload -> last bundle before binding
    std::vector<MvmBuf> table;
    for (const BufferDecl& b : p_.buffers) table.push_back(MvmBuf{nullptr, b.rows, b.cols, b.cols, b.dtype, {0, 0}});
    for (const AdmissionDecl& a : p_.adms) {
      const std::string who = "admission " + a.name;
      std::map<std::string, long long> target;
      for (const VarVersion& b : a.base) target[p_.vars[b.var]] = b.v;
      std::vector<std::string> tried;
      auto usable = [&](Program& g, const std::string& label) {
        const std::string why = shift_to(g, target);
        if (!why.empty()) { tried.push_back(label + ": " + why); return false; }
        return true;
      };
      Program g;
      bool have = false;
      if (!a.bundle_dir.empty() && has_file(p_.root + "/" + a.bundle_dir + "/metadata.json")) {
        Program c = load_program(p_.root + "/" + a.bundle_dir);
        const auto before = c.built_for;
        if (usable(c, a.bundle_dir)) { g = std::move(c); g.origin = g.built_for == before ? "bundle_dir" : "bundle_dir, versions moved"; have = true; }
      }
      if (!have && previous.count(a.workload)) {
        Program c = previous.at(a.workload);
        const auto before = c.built_for;
        if (usable(c, "previous bundle of " + p_.workloads[a.workload].name)) {
          g = std::move(c);
          g.origin = g.built_for == before ? "reused" : "reused, versions moved";
          have = true;
        }
      }
      if (!have && !a.compile_file.empty()) { g = compile_for(a); have = true; }
      if (!have) {
        std::string detail;
        for (const std::string& t : tried) detail += " [" + t + "]";
        refuse(who, "no bundle: bundle_dir absent or unusable, no usable earlier bundle of its workload, no compile entry" + detail);
      }
      check_publications(g, a, p_);
      for (MvmTaskDesc& t : g.tasks) t.workload_id = p_.workloads[a.workload].cls_id;   // the scheduler class
      previous[a.workload] = g;
      bind_globals(g, p_, who);
      char err[1024] = {0};
      if (kvm_validate(g.tasks.data(), (int)g.tasks.size(), g.succ.data(), (int)g.succ.size(), g.args.data(), (int)g.args.size(),
                       table.data(), (int)table.size(), std::max<int>(1, (int)p_.vars.size()), err, sizeof err) < 0)
        refuse(who, err);
      progs_.push_back(std::move(g));
    }
  }

  // Creates the executor in stream mode (window slots sized to the largest bundle, up to 64K tasks; larger bundles
  // stream through several windows), allocates and initialises every manifest buffer from its owner's first bundle,
  // and starts the kernel.
  bool classes_on() const { return o_.sched == "dynamic" || o_.sched == "static"; }

  void launch() {
    size_t most_tasks = 1, most_edges = 1;
    for (const Program& g : progs_) { most_tasks = std::max(most_tasks, g.tasks.size()); most_edges = std::max(most_edges, g.succ.size()); }
    slot_tasks_ = 256;
    while ((size_t)slot_tasks_ < most_tasks && slot_tasks_ < (1 << 16)) slot_tasks_ *= 2;
    slot_edges_ = (int)std::min<size_t>(std::max<size_t>(most_edges, 1024), (size_t)1 << 22);
    KvmConfig cfg;
    kvm_config_default(&cfg);
    cfg.window_cap = o_.windows;
    cfg.window_tasks = slot_tasks_;
    cfg.window_edges = slot_edges_;
    cfg.num_vars = std::max<int>(1, (int)p_.vars.size());
    cfg.blocks = o_.blocks;
    cfg.trace_on = 0;
    cfg.timeout_us = (unsigned long long)o_.timeout_s * 1000000ull;
    cfg.backpressure_ms = o_.timeout_s * 1000;
    ex_.reset(kvm_create(&cfg));
    if (!ex_) refuse("executor", std::string("kvm_create: ") + kvm_last_error(nullptr));
    for (size_t bi = 0; bi < p_.buffers.size(); ++bi) {
      const BufferDecl& b = p_.buffers[bi];
      const int owner = p_.workload(b.owner);
      size_t ai = 0;
      while (p_.adms[ai].workload != owner) ++ai;
      const Json* decl = nullptr;
      for (const Json& jb : progs_[ai].meta.need("buffers").a)
        if (const Json* n = jb.get("name"); n && n->s == b.name) { decl = &jb; break; }
      if (!decl) refuse("$.buffers." + b.name, "the bundle of owner " + b.owner + " does not declare it");
      const int rows = (int)decl->num("rows", 0), cols = (int)decl->num("cols", 0), dt = (int)decl->num("dtype", 0);
      if (rows != b.rows || cols != b.cols || dt != b.dtype)
        refuse("$.buffers." + b.name, "manifest " + std::to_string(b.rows) + "x" + std::to_string(b.cols) + " dtype " + std::to_string(b.dtype) +
                                      ", owner bundle " + std::to_string(rows) + "x" + std::to_string(cols) + " dtype " + std::to_string(dt));
      if (add_buffer_from_meta(ex_.get(), *decl, progs_[ai].dir) != (int)bi) refuse("$.buffers." + b.name, "buffer index out of step");
    }
    if (classes_on()) {
      std::vector<KvmClassParams> cp(p_.class_names.size());
      for (size_t c = 0; c < cp.size(); ++c) {
        const auto& m = p_.class_params[c];
        auto get = [&](const char* k, int d) { auto it = m.find(k); return it == m.end() ? d : (int)it->second; };
        cp[c] = KvmClassParams{get("weight", 1), get("min_cta", 0), get("max_cta", KVM_UNLIMITED), get("urgent_us", 0),
                               o_.sched == "static" ? o_.shares[c] : 1, get("bw_cta", KVM_UNLIMITED), 0};
      }
      if (kvm_set_classes(ex_.get(), o_.sched == "static" ? KVM_SCHED_STATIC : KVM_SCHED_DYNAMIC, cp.data(), (int)cp.size()) < 0)
        refuse("$.classes", std::string("kvm_set_classes: ") + kvm_last_error(ex_.get()));
    }
    if (kvm_start(ex_.get()) < 0) refuse("executor", std::string("kvm_start: ") + kvm_last_error(ex_.get()));
    t0_ = std::chrono::steady_clock::now();
  }

  bool submit(int ai) {
    const Program& g = progs_[ai];
    Track& tr = track_[ai];
    const int nt = (int)g.tasks.size(), ne = (int)g.succ.size(), na = (int)g.args.size();
    int rc;
    if (nt <= slot_tasks_ && ne <= slot_edges_) {
      rc = kvm_submit(ex_.get(), g.tasks.data(), nt, g.succ.data(), ne, g.args.data(), na);
      if (rc >= 0) tr.windows.push_back(window_serial_++);
    } else {
      rc = kvm_submit_stream(ex_.get(), g.tasks.data(), nt, g.succ.data(), ne, g.args.data(), na, 0, o_.timeout_s * 1000);
      for (int k = 0; k < rc; ++k) tr.windows.push_back(window_serial_++);
    }
    if (rc < 0) {
      problems_ += p_.adms[ai].name + ": submission refused: " + kvm_last_error(ex_.get()) + "\n";
      tr.phase = Phase::FAILED;
      return false;
    }
    tr.submitted_us = elapsed_us();
    tr.phase = Phase::RUNNING;
    if (!o_.quiet) fprintf(stderr, "[%10.0f us] submit %-16s %7d tasks (%s)\n", tr.submitted_us, p_.adms[ai].name.c_str(), nt, g.origin.c_str());
    return true;
  }

  // Polls the device's live versions and window completion marks, retires finished admissions and submits every
  // admission whose gate opens (manifest order within one poll), until all have finished or something fails.
  bool drive() {
    track_.assign(p_.adms.size(), Track{});
    const int nv = std::max<int>(1, (int)p_.vars.size());
    std::vector<int32_t> live(nv, 0);
    Flow f;
    f.finished.assign(p_.adms.size(), 0);
    f.in_flight.assign(p_.adms.size(), 0);
    size_t left = p_.adms.size();
    while (left > 0) {
      if (elapsed_us() > o_.timeout_s * 1e6) { problems_ += "not finished within --timeout-s\n"; return false; }
      if (kvm_live_versions(ex_.get(), live.data(), nv) < 0) { problems_ += std::string("live versions: ") + kvm_last_error(ex_.get()) + "\n"; return false; }
      for (size_t i = 0; i < p_.adms.size(); ++i) {
        Track& tr = track_[i];
        if (tr.phase != Phase::RUNNING) continue;
        bool all = true;
        for (long long w : tr.windows) all = all && kvm_window_done(ex_.get(), w) == 1;
        if (!all) continue;
        tr.phase = Phase::FINISHED;
        tr.done_us = elapsed_us();
        tr.live_at_done = live;
        f.finished[i] = 1;
        f.in_flight[i] = 0;
        --left;
        if (!o_.quiet) fprintf(stderr, "[%10.0f us] done   %-16s\n", tr.done_us, p_.adms[i].name.c_str());
      }
      f.live.assign(live.begin(), live.begin() + p_.vars.size());
      f.now_us = elapsed_us();
      for (size_t i = 0; i < p_.adms.size(); ++i) {
        if (track_[i].phase != Phase::WAITING) continue;
        const Gate g = gate(p_, (int)i, f);
        if (g.dead) { problems_ += p_.adms[i].name + " can no longer be admitted: " + g.why + "\n"; return false; }
        if (!g.open) continue;
        if (!submit((int)i)) return false;
        f.in_flight[i] = 1;
      }
      std::this_thread::sleep_for(std::chrono::microseconds(50));
    }
    return true;
  }

  void write_summary(const KvmResult& r, bool ok) {
    FILE* f = fopen((o_.out + "/summary.json").c_str(), "w");
    if (!f) { problems_ += "cannot write summary.json\n"; return; }
    std::vector<KvmClassStats> cs(p_.class_names.size());
    const int ncs = classes_on() ? kvm_class_stats(ex_.get(), cs.data(), (int)cs.size()) : 0;
    auto versions = [&](const std::vector<int32_t>& v) {
      fprintf(f, "{");
      for (size_t k = 0; k < p_.vars.size() && k < v.size(); ++k) fprintf(f, "%s\"%s\": %d", k ? ", " : "", p_.vars[k].c_str(), v[k]);
      fprintf(f, "}");
    };
    fprintf(f, "{\"ok\": %s, \"done\": %d, \"admitted\": %d, \"kernel_ms\": %.3f,\n \"serial_order\": [", ok ? "true" : "false", r.done, r.admitted, r.kernel_ms);
    for (size_t i = 0; i < order_.size(); ++i) fprintf(f, "%s\"%s\"", i ? ", " : "", p_.adms[order_[i]].name.c_str());
    fprintf(f, "],\n \"admissions\": [");
    for (size_t i = 0; i < p_.adms.size(); ++i) {
      const Track& t = track_[i];
      fprintf(f, "%s\n  {\"name\": \"%s\", \"workload\": \"%s\", \"tasks\": %zu, \"windows\": %zu, \"how\": \"%s\", \"submitted_us\": %.1f, \"done_us\": %.1f, \"versions_at_done\": ",
              i ? "," : "", p_.adms[i].name.c_str(), p_.workloads[p_.adms[i].workload].name.c_str(), progs_[i].tasks.size(), t.windows.size(),
              progs_[i].origin.c_str(), t.submitted_us, t.done_us);
      versions(t.live_at_done);
      fprintf(f, "}");
    }
    std::vector<int32_t> fin(std::max<size_t>(1, p_.vars.size()));
    kvm_versions(ex_.get(), fin.data(), (int)fin.size());
    fprintf(f, "],\n \"sched\": \"%s\", \"classes\": [", o_.sched.c_str());
    for (size_t c = 0; c < p_.class_names.size(); ++c) {
      fprintf(f, "%s{\"name\": \"%s\"", c ? ", " : "", p_.class_names[c].c_str());
      if ((int)c < ncs) fprintf(f, ", \"tasks\": %llu, \"max_running\": %d, \"missed\": %llu", (unsigned long long)cs[c].tasks, cs[c].max_running,
                                (unsigned long long)cs[c].missed);
      fprintf(f, "}");
    }
    fprintf(f, "],\n \"versions\": ");
    versions(fin);
    fprintf(f, "}\n");
    fclose(f);
  }

  void write_dumps() {
    if (o_.dump.empty()) return;
    std::regex pick;
    try { pick = std::regex(o_.dump); } catch (const std::regex_error& e) { problems_ += std::string("--dump: ") + e.what() + "\n"; return; }
    for (size_t i = 0; i < p_.buffers.size(); ++i) {
      if (!std::regex_search(p_.buffers[i].name, pick)) continue;
      const size_t n = (size_t)p_.buffers[i].rows * p_.buffers[i].cols;
      std::vector<float> v(n);
      if (kvm_read_buffer(ex_.get(), (int)i, v.data(), n) < 0) { problems_ += "dump " + p_.buffers[i].name + ": " + kvm_last_error(ex_.get()) + "\n"; continue; }
      FILE* f = fopen((o_.out + "/" + p_.buffers[i].name + ".bin").c_str(), "wb");
      if (!f || fwrite(v.data(), sizeof(float), n, f) != n) problems_ += "cannot write the dump of " + p_.buffers[i].name + "\n";
      if (f) fclose(f);
    }
  }
};

int usage() {
  fprintf(stderr,
          "usage: kvm_run DEMO_DIR [--out DIR] [--dump REGEX] [--windows N] [--blocks N] [--timeout-s N]\n"
          "               [--sched off|global|static|dynamic] [--shares a,b,..] [--check-only] [--quiet]\n"
          "  runs every admission of DEMO_DIR/MANIFEST.json on one persistent kernel (stream mode)\n"
          "  --sched MODE  dynamic (default): one scheduler class per manifest class; static: workers split by --shares\n"
          "                (one per class); off / global: first-come first-served\n");
  return 2;
}

}  // namespace

int main(int argc, char** argv) {
  Options o;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    const bool has_value = i + 1 < argc;
    if (a == "--check-only") o.check_only = true;
    else if (a == "--quiet") o.quiet = true;
    else if (a[0] == '-' && !has_value) return usage();
    else if (a == "--out") o.out = argv[++i];
    else if (a == "--dump") o.dump = argv[++i];
    else if (a == "--windows") o.windows = atoi(argv[++i]);
    else if (a == "--blocks") o.blocks = atoi(argv[++i]);
    else if (a == "--timeout-s") o.timeout_s = atoi(argv[++i]);
    else if (a == "--sched") o.sched = argv[++i];
    else if (a == "--shares") {
      std::string v = argv[++i];
      for (size_t pos = 0; pos <= v.size();) {
        const size_t e = std::min(v.find(',', pos), v.size());
        const int x = atoi(v.substr(pos, e - pos).c_str());
        if (x < 1) return usage();
        o.shares.push_back(x);
        pos = e + 1;
      }
    }
    else if (a[0] == '-' || !o.root.empty()) return usage();
    else o.root = a;
  }
  if (o.root.empty() || o.windows < 1 || o.timeout_s < 1 || (o.sched != "off" && o.sched != "global" && o.sched != "static" && o.sched != "dynamic")) return usage();
  try {
    ManifestRun run(read_plan(o.root), o);
    return run.go();
  } catch (const std::exception& e) {
    fprintf(stderr, "kvm_run: %s\n", e.what());
    printf("FAIL: %s\n", e.what());
    return 1;
  }
}
