// kvm_compile: workload JSON -> task bundle directory (reference: runtime/compile_workload.py:715-760, its command
// line). Usage: kvm_compile WORKLOAD.json OUT_DIR [--base-versions var=N,...]... [--data-dir DIR]. `file` initial
// values are read from DIR (default: the workload file's directory), checked for size and copied into OUT_DIR under
// their relative path. Exit 0 on success; 2 with the compile error on stderr (nothing is written then).
#include <sys/stat.h>
#include <cerrno>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include "compile.h"

static void write_bytes(const std::string& path, const void* p, size_t n) {
  FILE* f = fopen(path.c_str(), "wb");
  if (!f) throw std::runtime_error("cannot write " + path);
  const bool ok = (n == 0 || fwrite(p, 1, n, f) == n);
  if (fclose(f) != 0 || !ok) throw std::runtime_error("cannot write " + path);
}

static void copy_file(const std::string& src, const std::string& dst) {
  const std::string d = kvmh::read_file(src);
  write_bytes(dst, d.data(), d.size());
}

static std::string real_or_self(const std::string& p) {
  char buf[4096];
  return realpath(p.c_str(), buf) ? std::string(buf) : p;
}

static void make_dirs(const std::string& d) {
  for (size_t i = 1; i <= d.size(); ++i)
    if (i == d.size() || d[i] == '/') {
      const std::string part = d.substr(0, i);
      if (mkdir(part.c_str(), 0777) != 0 && errno != EEXIST) throw std::runtime_error("cannot create " + part);
    }
}

int main(int argc, char** argv) {
  std::vector<std::string> pos;
  std::string base_arg, data_dir;
  bool have_dir = false;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--base-versions" && i + 1 < argc) base_arg += std::string(",") + argv[++i];
    else if (a.rfind("--base-versions=", 0) == 0) base_arg += "," + a.substr(16);
    else if (a == "--data-dir" && i + 1 < argc) { data_dir = argv[++i]; have_dir = true; }
    else if (a == "-h" || a == "--help") { printf("usage: kvm_compile WORKLOAD.json OUT_DIR [--base-versions var=N,...] [--data-dir DIR]\n"); return 0; }
    else pos.push_back(a);
  }
  if (pos.size() != 2) { fprintf(stderr, "usage: kvm_compile WORKLOAD.json OUT_DIR [--base-versions var=N,...]\n"); return 2; }
  try {
    std::map<std::string, int> base;
    size_t p = 0;
    while (p < base_arg.size()) {
      size_t e = base_arg.find(',', p); if (e == std::string::npos) e = base_arg.size();
      const std::string item = base_arg.substr(p, e - p);
      if (!item.empty()) {
        const size_t eq = item.find('=');
        if (eq == std::string::npos) throw kvmc::CompileError("--base-versions: var=N expected, got '" + item + "'");
        base[item.substr(0, eq)] = std::stoi(item.substr(eq + 1));
      }
      p = e + 1;
    }
    const std::string text = kvmh::read_file(pos[0]);
    kvmh::Parser parser(text);
    const kvmh::Json spec = parser.parse();
    if (!have_dir) {
      const std::string w = real_or_self(pos[0]);
      const size_t sl = w.rfind('/');
      data_dir = sl == std::string::npos ? "." : w.substr(0, std::max<size_t>(sl, 1));
    }
    const kvmc::Bundle b = kvmc::compile(spec, base, &data_dir);
    make_dirs(pos[1]);
    for (const std::string& f : b.files) {
      const std::string src = data_dir + "/" + f, dst = pos[1] + "/" + f;
      if (real_or_self(src) == real_or_self(dst)) continue;
      const size_t sl = dst.rfind('/');
      make_dirs(dst.substr(0, sl));
      copy_file(src, dst);
    }
    write_bytes(pos[1] + "/tasks.bin", b.tasks.data(), b.tasks.size() * sizeof(MvmTaskDesc));
    write_bytes(pos[1] + "/successors.bin", b.succ.data(), b.succ.size() * 4);
    write_bytes(pos[1] + "/args.bin", b.args.data(), b.args.size() * 4);
    write_bytes(pos[1] + "/metadata.json", b.metadata.data(), b.metadata.size());
  } catch (const std::exception& e) {
    fprintf(stderr, "kvm_compile: %s\n", e.what());
    return 2;
  }
  return 0;
}
