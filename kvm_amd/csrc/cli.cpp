// kvm_exec: command-line runner of ABI-v2 bundles on one MI355X, the counterpart of the reference's `mvm_exec` CLI
// (reference: mvm_exec.cu:1962-2315). Prints "OK: d/a tasks, X ms[, golden match]" or "FAIL: ..." and exits 0 / 1
// (2 for usage errors).
//
//   kvm_exec [--golden [--golden-tol R] [--golden-tol-bf16 R]] [--dump-bin DIR i,j,..] [--trace-csv FILE] [--repeat N] [--timeout-s N]
//            [--blocks N] [--no-trace] [--quiet] [--check-ops] [--sched global|static|dynamic --classes N --weights a,b,..
//            --min a,b,.. --max a,b,.. --urgent-us a,b,.. --shares a,b,..] bundle_dir...
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>
#include "../../include/kvm_exec.h"
#include "host_json.h"

using namespace kvmh;

static void usage() {
  fprintf(stderr, "usage: kvm_exec [options] bundle_dir...\n"
                  "  --golden [--golden-tol R] [--golden-tol-bf16 R]   compare with <bundle_dir>/golden.json (one bundle): buffers (relative\n"
                  "                              L2; bf16-storage buffers by the second tolerance, default 1e-2), versions, reads\n"
                  "  --dump-bin DIR i,j,..       write buffers (widened to f32 / raw i32) to DIR/<index>.bin\n"
                  "  --trace-csv FILE            per-task timeline   --repeat N   run the graph N times (timed)   --timeout-s N\n"
                  "  --dump-buffers              print every buffer (reference text format)\n"
                  "  --path auto|dynamic|static  scheduler: per-worker static programs, ready queues, or chosen from the graph (default auto)\n"
                  "  --blocks N   --no-trace   --quiet   --check-ops\n"
                  "  --sched global|static|dynamic --classes N   scheduler classes (a task's class is its workload_id); per class, comma\n"
                  "    lists: --weights, --min (reservation), --max (cap), --bw-cta (bandwidth-bound cap), --urgent-us (EDF window),\n"
                  "    --shares (static split), --op-affinity (1 = op affinity); --arbiter --bw-limit N (global bandwidth-bound cap),\n"
                  "    --no-guarantee, --no-inherit, --affinity-us N (task affinity window)\n");
}

int main(int argc, char** argv) {
  std::vector<std::string> dirs; bool golden = false, quiet = false, trace = true, dump_text = false; float tol = 1e-6f, tol_bf16 = 1e-2f;
  const char* csv = nullptr; std::string dump_dir; std::vector<int> dump_idx; int repeat = 1, blocks = 0, path = KVM_PATH_AUTO; long long timeout_s = 20;
  int sched = KVM_SCHED_GLOBAL, nclasses = 1, sflags = KVM_SCHED_F_GUARANTEE | KVM_SCHED_F_INHERIT, bw_limit = KVM_UNLIMITED, affinity_us = 0;
  std::vector<KvmClassParams> cls(KVM_MAX_CLASSES, KvmClassParams{1, 0, KVM_UNLIMITED, 0, 1, KVM_UNLIMITED, 0});
  // a comma list of integers into field f of classes 0, 1, ...
  auto list = [&](const char* v, int KvmClassParams::*f) {
    int c = 0;
    for (const char* p = v; *p && c < KVM_MAX_CLASSES; ++c) {
      char* e; const long x = strtol(p, &e, 10);
      if (e == p) return false;
      cls[c].*f = (int)x;
      p = *e == ',' ? e + 1 : e;
    }
    return true;
  };
  for (int i = 1; i < argc; ++i) {
    std::string a = argv[i];
    auto next = [&]() -> const char* { if (i + 1 >= argc) { usage(); exit(2); } return argv[++i]; };
    if (a == "--golden") golden = true;
    else if (a == "--dump-buffers") dump_text = true;
    else if (a == "--golden-tol") tol = (float)atof(next());
    else if (a == "--golden-tol-bf16") tol_bf16 = (float)atof(next());
    else if (a == "--trace-csv") csv = next();
    else if (a == "--repeat") repeat = atoi(next());
    else if (a == "--timeout-s") timeout_s = atoll(next());
    else if (a == "--blocks") blocks = atoi(next());
    else if (a == "--no-trace") trace = false;
    else if (a == "--path") {
      std::string p = next();
      if (p == "auto") path = KVM_PATH_AUTO; else if (p == "dynamic") path = KVM_PATH_DYNAMIC; else if (p == "static") path = KVM_PATH_STATIC;
      else { usage(); return 2; }
    }
    else if (a == "--quiet") quiet = true;
    else if (a == "--sched") {
      const std::string m = next();
      if (m == "global") sched = KVM_SCHED_GLOBAL; else if (m == "static") sched = KVM_SCHED_STATIC; else if (m == "dynamic") sched = KVM_SCHED_DYNAMIC;
      else { usage(); return 2; }
    }
    else if (a == "--classes") { nclasses = atoi(next()); if (nclasses < 1 || nclasses > KVM_MAX_CLASSES) { usage(); return 2; } }
    else if (a == "--weights") { if (!list(next(), &KvmClassParams::weight)) { usage(); return 2; } }
    else if (a == "--min") { if (!list(next(), &KvmClassParams::min_cta)) { usage(); return 2; } }
    else if (a == "--max") { if (!list(next(), &KvmClassParams::max_cta)) { usage(); return 2; } }
    else if (a == "--urgent-us") { if (!list(next(), &KvmClassParams::urgent_us)) { usage(); return 2; } }
    else if (a == "--shares") { if (!list(next(), &KvmClassParams::share)) { usage(); return 2; } }
    else if (a == "--bw-cta") { if (!list(next(), &KvmClassParams::bw_cta)) { usage(); return 2; } }
    else if (a == "--op-affinity") {
      if (!list(next(), &KvmClassParams::flags)) { usage(); return 2; }
      for (auto& c : cls) c.flags = c.flags ? KVM_CLASS_OPAFF : 0;
    }
    else if (a == "--affinity-us") affinity_us = atoi(next());
    else if (a == "--arbiter") sflags |= KVM_SCHED_F_ARBITER;
    else if (a == "--bw-limit") bw_limit = atoi(next());
    else if (a == "--no-guarantee") sflags &= ~KVM_SCHED_F_GUARANTEE;
    else if (a == "--no-inherit") sflags &= ~KVM_SCHED_F_INHERIT;
    else if (a == "--dump-bin") { dump_dir = next(); for (char* p = (char*)next(); *p;) { char* e; long v = strtol(p, &e, 10); if (e == p) { usage(); return 2; } dump_idx.push_back((int)v); p = *e == ',' ? e + 1 : e; } }
    else if (a == "--check-ops") { for (int id = 0; id < 400; ++id) if (const char* n = kvm_op_name(id)) printf("%3d %s\n", id, n); return 0; }
    else if (a[0] == '-') { usage(); return 2; }
    else dirs.push_back(a);
  }
  if (dirs.empty() || repeat < 1) { usage(); return 2; }
  try {
    std::vector<Json> metas;
    int nvars = 1;
    for (auto& d : dirs) {
      metas.push_back(Parser(read_file(d + "/metadata.json")).parse());
      if ((int)metas.back().num("abi_version", -1) != MVM_ABI_VERSION) throw std::runtime_error(d + ": abi_version is not 2");
      nvars = std::max(nvars, (int)metas.back().need("variables").a.size());
    }
    KvmConfig cfg; kvm_config_default(&cfg);
    cfg.num_vars = nvars; cfg.trace_on = (trace || golden || csv) ? 1 : 0; cfg.timeout_us = (unsigned long long)timeout_s * 1000000ull; cfg.blocks = blocks; cfg.path = path;
    std::unique_ptr<KvmExec, void (*)(KvmExec*)> ex(kvm_create(&cfg), kvm_destroy);
    if (!ex) throw std::runtime_error(std::string("kvm_create: ") + kvm_last_error(nullptr));
    // buffers: the first bundle declares them; later bundles must name the same table (the reference's shared buffer model)
    std::vector<std::string> names;
    for (auto& jb : metas[0].need("buffers").a) {
      add_buffer_from_meta(ex.get(), jb, dirs[0]);
      names.push_back(jb.need("name").s);
    }
    for (auto& jv : metas[0].need("variables").a) kvm_set_version(ex.get(), (int)jv.num("id", 0), (int)jv.num("base_version", 0));
    for (size_t k = 0; k < dirs.size(); ++k) {
      auto t = read_bin<MvmTaskDesc>(dirs[k] + "/tasks.bin");
      auto s = read_bin<int32_t>(dirs[k] + "/successors.bin");
      auto a = read_bin<int32_t>(dirs[k] + "/args.bin");
      if ((int)t.size() != (int)metas[k].num("task_count", -1)) throw std::runtime_error(dirs[k] + ": tasks.bin does not match task_count");
      if (kvm_submit(ex.get(), t.data(), (int)t.size(), s.data(), (int)s.size(), a.data(), (int)a.size()) < 0)
        throw std::runtime_error(dirs[k] + ": submit: " + kvm_last_error(ex.get()));
    }
    if (sched != KVM_SCHED_GLOBAL && (kvm_set_classes(ex.get(), sched, cls.data(), nclasses) < 0 ||
                                      kvm_set_sched_flags(ex.get(), sflags, bw_limit) < 0 || kvm_set_affinity(ex.get(), affinity_us) < 0))
      throw std::runtime_error(kvm_last_error(ex.get()));
    KvmResult r{}; float ms = 0;
    if (repeat == 1) { if (kvm_start(ex.get()) < 0) throw std::runtime_error(kvm_last_error(ex.get())); }
    else if (kvm_run_timed(ex.get(), repeat, &ms) < 0) throw std::runtime_error(kvm_last_error(ex.get()));
    kvm_finish(ex.get(), &r);
    if (repeat > 1) r.kernel_ms = ms / repeat;
    if (r.err_code && !quiet) fprintf(stderr, "device error %d at task %d (a=%d b=%d)\n", r.err_code, r.err_slot, r.err_a, r.err_b);
    int bad = 0;
    std::vector<KvmTrace> tr;
    if (cfg.trace_on) { tr.resize(kvm_ntasks(ex.get())); kvm_trace(ex.get(), tr.data(), (int)tr.size()); }
    if (golden && r.err_code == 0) {
      if (dirs.size() != 1) throw std::runtime_error("--golden needs exactly one bundle");
      Json g = Parser(read_file(dirs[0] + "/golden.json")).parse();
      float worst = 0;
      for (auto& kv : g.need("buffers").o) {
        int idx = -1; for (size_t i = 0; i < names.size(); ++i) if (names[i] == kv.first) idx = (int)i;
        if (idx < 0) { ++bad; continue; }
        size_t n = kv.second.a.size(); std::vector<float> got(n);
        if (kvm_read_buffer(ex.get(), idx, got.data(), n) < 0) { ++bad; continue; }
        const int bdt = kvm_buffer_dtype(ex.get(), idx);
        bool is_int = bdt == 1; double num = 0, den = 0;
        const float btol = bdt == 2 ? tol_bf16 : tol;   // bf16 storage: a stored value may round to the neighbouring bf16
        for (size_t i = 0; i < n; ++i) {
          if (is_int) { int32_t gi; memcpy(&gi, &got[i], 4); if (gi != (int32_t)kv.second.a[i].n) ++bad; continue; }
          double w = kv.second.a[i].n, d = got[i] - w; num += d * d; den += w * w;
        }
        float rel = (float)(std::sqrt(num) / std::max(1e-30, std::sqrt(den))); worst = std::max(worst, rel);
        if (rel > btol) { if (!quiet) fprintf(stderr, "golden: buffer %s relative L2 %.3g > %.3g\n", kv.first.c_str(), rel, btol); ++bad; }
      }
      std::vector<int32_t> ver(nvars); kvm_versions(ex.get(), ver.data(), nvars);
      std::map<std::string, int> vid; for (auto& jv : metas[0].need("variables").a) vid[jv.need("name").s] = (int)jv.num("id", 0);
      for (auto& kv : g.need("versions").o) if (ver[vid[kv.first]] != (int)kv.second.n) { ++bad; if (!quiet) fprintf(stderr, "golden: version %s\n", kv.first.c_str()); }
      std::map<std::pair<int, int>, int> pub;   // (variable, version) -> publishing task
      for (auto& jp : metas[0].need("publishers").a) pub[{(int)jp.num("var", -1), (int)jp.num("version", -1)}] = (int)jp.num("task", -1);
      for (auto& jr : metas[0].need("reads").a) {   // the task carrying each read's wait saw an admissible version
        int task = (int)jr.num("task", -1), slot = task; const Json* gate = jr.get("gate"); if (gate && gate->t == Json::N) slot = (int)gate->n;
        int var = (int)jr.num("var", -1), want = (int)jr.num("version", 0); bool exact = jr.need("policy").s == "exact";
        const KvmTrace& t = tr[slot];
        bool ok;
        if (t.ver0 < 0) {   // a read of the initial version carries no wait: it held if the next publisher started after it
          auto nx = pub.find({var, want + 1});
          ok = want == 0 && (!exact || nx == pub.end() || tr[nx->second].start >= tr[task].end);
        } else ok = t.ver0 >= want && (!exact || (t.ver0 == want && t.ver1 == want));
        if (!ok && !quiet) fprintf(stderr, "golden: read %s of variable %d at version %d not admissible\n", jr.need("name").s.c_str(), var, want);
        bad += !ok;
      }
      if (!quiet) fprintf(stderr, "golden: worst buffer relative L2 %.3g (tolerance %.3g)\n", worst, tol);
    }
    if (csv) {
      FILE* f = fopen(csv, "w");
      if (f) { fprintf(f, "task,start,end,block,xcc,ver0,ver1,exec_count\n");
        for (size_t i = 0; i < tr.size(); ++i) fprintf(f, "%zu,%llu,%llu,%d,%d,%d,%d,%d\n", i, tr[i].start, tr[i].end, tr[i].block, tr[i].xcc, tr[i].ver0, tr[i].ver1, tr[i].exec_count);
        fclose(f); }
    }
    // text dump of every buffer, one line each, in the reference CLI's format (mvm_exec.cu:2298): raw 4-byte elements
    // printed as floats (an i32 buffer's bits reinterpreted), bf16 storage widened to fp32
    if (dump_text)
      for (int idx = 0; idx < kvm_nbufs(ex.get()); ++idx) {
        const Json& jb = metas[0].need("buffers").a[idx];
        size_t n = (size_t)jb.num("rows", 1) * (size_t)jb.num("cols", 1);
        std::vector<float> v(n); kvm_read_buffer(ex.get(), idx, v.data(), n);
        printf("buffer %d:", idx);
        for (float x : v) printf(" %.9g", x);
        printf("\n");
      }
    for (int idx : dump_idx) {
      if (idx < 0 || idx >= kvm_nbufs(ex.get())) { fprintf(stderr, "--dump-bin: buffer %d out of range\n", idx); return 2; }
      int dt = kvm_buffer_dtype(ex.get(), idx);
      const Json& jb = metas[0].need("buffers").a[idx];
      size_t n = (size_t)jb.num("rows", 1) * (size_t)jb.num("cols", 1);
      std::vector<float> v(n); kvm_read_buffer(ex.get(), idx, v.data(), n); (void)dt;
      FILE* f = fopen((dump_dir + "/" + std::to_string(idx) + ".bin").c_str(), "wb");
      if (!f || fwrite(v.data(), 4, n, f) != n) { fprintf(stderr, "--dump-bin: cannot write\n"); return 2; }
      fclose(f);
    }
    bool pass = r.err_code == 0 && bad == 0;
    printf("%s: %d/%d tasks, %.3f ms (%s path)%s\n", pass ? "OK" : "FAIL", r.done, r.admitted, r.kernel_ms, kvm_path(ex.get()) == KVM_PATH_STATIC ? "static" : "dynamic", golden ? (bad ? ", golden MISMATCH" : ", golden match") : "");
    if (sched != KVM_SCHED_GLOBAL && !quiet) {   // per-class report (reference: mvm_exec.cu:1842-1860)
      std::vector<KvmClassStats> st(nclasses);
      const int m = kvm_class_stats(ex.get(), st.data(), nclasses);
      for (int c = 0; c < m; ++c)
        printf("class %d: %llu tasks, busy %.3f ms, %llu reserved starts, %llu urgent starts, %llu missed deadlines, max running %d\n", c,
               st[c].tasks, st[c].busy_ticks / 1e5, st[c].resv_starts, st[c].urgent_starts, st[c].missed, st[c].max_running);
    }
    return pass ? 0 : 1;
  } catch (const std::exception& e) {
    fprintf(stderr, "kvm_exec: %s\n", e.what());
    return 1;
  }
}
