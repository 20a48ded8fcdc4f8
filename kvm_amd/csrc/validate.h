// Host-side bundle validation: descriptor ranges, operator arity, dependency counts, acyclicity, buffer indices and
// dtypes, and every operator's operand extents (the element ranges it will touch). A bundle that passes cannot make
// an operator read or write outside its buffers, apart from data-dependent indices (token ids, KV lengths), which the
// operators check on the device. Extent rules follow the reference's (runtime/ref_gpt.py, ref_extra.py `extents`).
#pragma once
#include <cstring>
#include <string>
#include <vector>
#include <initializer_list>
#include <algorithm>
#include "../../include/mvm_task_abi.h"
#include "../../include/kvm_exec.h"

namespace kvmv {

struct OpSig { const char* name; int id; const char* sig; };
static const OpSig kRegistry[] = {
#define X(n, id, sig) {#n, id, sig},
#include "../../include/mvm_ops_list.inc"
#undef X
};

struct ArgInfo { std::string name; int type; bool opt; };   // type 0 buf, 1 i32, 2 f32
static std::vector<ArgInfo> parse_sig(const char* s) {
  std::vector<ArgInfo> out;
  std::string str(s);
  size_t p = 0;
  while (p < str.size()) {
    size_t e = str.find(',', p); if (e == std::string::npos) e = str.size();
    std::string item = str.substr(p, e - p);
    size_t c = item.find(':');
    std::string nm = item.substr(0, c), ty = item.substr(c + 1);
    out.push_back({nm, ty == "i32" ? 1 : ty == "f32" ? 2 : 0, ty == "buf?"});
    p = e + 1;
  }
  return out;
}
static const OpSig* find_op(int id) { for (const OpSig& o : kRegistry) if (o.id == id) return &o; return nullptr; }

// Operators this executor runs (the rest of the registry ids exist for id-space compatibility only).
static bool implemented(int id) {
  static const int ids[] = {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 32, 33, 34, 35, 36, 37, 38, 39, 40, 41, 42, 43, 44, 45, 46, 47, 48, 49, 50,
                            51, 52, 53, 54, 55, 56, 57, 58, 59, 60, 61, 62, 63, 96, 97, 98, 99, 100, 101, 102, 103, 104, 113, 114, 115,
                            116, 117, 118, 120, 121, 122, 123, 126, 127, 134, 135, 136, 300, 301, 302, 303, 304, 305, 306, 308, 309, 310, 311};
  for (int i : ids) if (i == id) return true;
  return false;
}

struct Check {
  const MvmBuf* bufs; int nbufs; const int32_t* a; std::vector<ArgInfo> args; std::string err; std::string op;
  int idx(const char* n) const { for (size_t i = 0; i < args.size(); ++i) if (args[i].name == n) return (int)i; return -1; }
  int I(const char* n) const { return a[idx(n)]; }
  float F(const char* n) const { float f; memcpy(&f, &a[idx(n)], 4); return f; }
  const MvmBuf* B(const char* n) const { int w = a[idx(n)]; return w < 0 ? nullptr : &bufs[w]; }
  bool need(bool c, const char* m) { if (!c && err.empty()) err = op + ": " + m; return c; }
  // rows x cols extent (buffer must have >= r rows and >= c cols); absent optional buffers pass
  void ext(const char* n, long long r, long long c) {
    const MvmBuf* b = B(n); if (!b) return;
    if (!(b->rows >= r && b->cols >= c)) need(false, (std::string("buffer '") + n + "' too small: needs " + std::to_string(r) + "x" + std::to_string(c)).c_str());
  }
  void extn(const char* n, long long cnt) {
    const MvmBuf* b = B(n); if (!b) return;
    if (!((long long)b->rows * b->cols >= cnt)) need(false, (std::string("buffer '") + n + "' too small: needs " + std::to_string(cnt) + " elements").c_str());
  }
  void range(long long lo, long long hi) { need(0 <= lo && lo <= hi, "bad range"); }
};

// dtype classes of buffer arguments: 'i' int32, 'a' any (f32 / bf16 storage; i32 where the op moves raw words), else f32
static char arg_class(int op, const std::string& n) {
  auto in = [&](std::initializer_list<const char*> l) { for (const char* s : l) if (n == s) return true; return false; };
  switch (op) {
    case 1: return 'a';   // copy moves raw 4-byte words
    case 32: return in({"ids"}) ? 'i' : in({"out"}) ? 'a' : 'f';
    case 33: return in({"ids"}) ? 'i' : 'f';
    case 35: case 36: return in({"x", "out"}) ? 'a' : 'f';
    case 37: case 38: return in({"x", "dy", "dx"}) ? 'a' : 'f';
    case 309: return in({"x", "dy", "dx", "res"}) ? 'a' : 'f';
    case 39: return in({"x", "dy"}) ? 'a' : 'f';
    case 40: return 'f';
    case 41: return in({"x", "dy", "dx"}) ? 'a' : 'f';
    case 42: return in({"a", "b", "out"}) ? 'a' : 'f';
    case 43: case 44: return in({"pos"}) ? 'i' : in({"x", "out"}) ? 'a' : 'f';
    case 45: return in({"q", "k", "v", "o"}) ? 'a' : 'f';
    case 46: return in({"o", "do"}) ? 'a' : 'f';
    case 47: return in({"q", "k", "v", "do", "dq"}) ? 'a' : 'f';
    case 48: return in({"q", "k", "v", "do", "dk", "dv"}) ? 'a' : 'f';
    case 49: return in({"lens"}) ? 'i' : 'a';
    case 50: return in({"lens"}) ? 'i' : in({"q", "kc", "vc", "o"}) ? 'a' : 'f';
    case 51: case 52: return in({"tgt"}) ? 'i' : in({"logits"}) ? 'a' : 'f';
    case 53: case 127: return in({"tgt"}) ? 'i' : in({"logits", "dlogits"}) ? 'a' : 'f';
    case 54: case 115: return in({"step"}) ? 'i' : 'f';
    case 305: return in({"step"}) ? 'i' : in({"sh"}) ? 'a' : 'f';
    case 57: return in({"out", "ctr"}) ? 'i' : 'f';
    case 58: return in({"out"}) ? 'i' : 'f';
    case 59: return 'a';
    case 60: return 'i';
    case 61: return in({"x"}) ? 'a' : 'f';
    case 62: return in({"step"}) ? 'i' : 'a';
    case 63: case 102: case 103: case 104: return in({"idx"}) ? 'i' : 'f';
    case 98: return 'a';
    case 113: return 'a';
    case 114: case 122: case 304: return in({"bias"}) ? 'f' : 'a';
    case 308: return in({"bias", "delta"}) ? 'f' : 'a';
    case 116: return in({"step"}) ? 'i' : 'f';
    case 134: return in({"gamma"}) ? 'f' : 'a';
    case 135: return in({"lens"}) ? 'i' : in({"part"}) ? 'f' : 'a';
    case 306: return in({"lens"}) ? 'i' : in({"part", "qgamma", "kgamma"}) ? 'f' : 'a';
    case 310: return in({"lens", "cnt"}) ? 'i' : in({"part", "qgamma", "kgamma"}) ? 'f' : 'a';
    case 136: return in({"o"}) ? 'a' : 'f';
    case 300: return in({"x", "out"}) ? 'a' : 'f';
    case 301: return in({"gamma"}) ? 'f' : 'a';
    case 311: return in({"gamma"}) ? 'f' : 'a';
    case 302: return in({"bias"}) ? 'f' : 'a';
    case 303: return in({"out"}) ? 'a' : 'f';
    default: return 'f';
  }
}

static bool attn_hd(int hd) { return hd == 16 || hd == 32 || hd == 64 || hd == 128; }

// Operand extents of one task; mirrors the reference's extent functions for the ops implemented here.
static void extents(int op, Check& k) {
  auto flat = [&](std::initializer_list<const char*> names, const char* lo, const char* hi) {
    k.range(k.I(lo), k.I(hi)); for (const char* n : names) k.extn(n, k.I(hi));
  };
  switch (op) {
    case 0: case 10: break;
    case 1: k.need(k.I("n") >= 1, "n >= 1"); k.extn("src", k.I("n")); k.extn("dst", k.I("n")); break;
    case 2: k.need(k.I("n") >= 1, "n >= 1"); for (const char* n : {"a", "b", "out"}) k.extn(n, k.I("n")); break;
    case 3: case 4: k.need(k.I("n") >= 1, "n >= 1"); k.extn("x", k.I("n")); k.extn("out", k.I("n")); break;
    case 5: k.need(k.I("n") >= 1, "n >= 1"); k.extn("w", k.I("n")); k.extn("g", k.I("n")); break;
    case 6: k.need(k.I("n") >= 1, "n >= 1"); k.extn("x", k.I("n")); k.extn("w", 1); k.extn("out", k.I("n")); break;
    case 7: k.need(k.I("n") >= 1, "n >= 1"); for (const char* n : {"pred", "target", "x"}) k.extn(n, k.I("n")); k.extn("loss", 1); k.extn("grad", 1); break;
    case 8: { int m = k.I("m"), n = k.I("n"), kk = k.I("k"); k.need(m >= 1 && n >= 1 && kk >= 1, "m,n,k >= 1");
      k.extn("a", (long long)m * kk); k.extn("b", (long long)kk * n); k.extn("out", (long long)m * n); break; }
    case 9: k.need(k.I("n") >= 1, "n >= 1"); k.extn("x", k.I("n")); break;
    case 32: { int r0 = k.I("r0"), r1 = k.I("r1"), T = k.I("T"), d = k.I("d"); k.range(r0, r1); k.need(T > 0 && d > 0, "bad T/d");
      k.extn("ids", r1); k.ext("wte", 0, d); k.ext("wpe", T, d); k.ext("out", r1, d); break; }
    case 33: { int N = k.I("N"), v0 = k.I("v0"), v1 = k.I("v1"), d = k.I("d"); k.need(N >= 0 && 0 <= v0 && v0 <= v1 && d > 0, "bad N/v0/v1/d");
      k.need(k.B("ids") || k.I("mod") > 0, "ids absent needs mod > 0");
      k.extn("ids", N); k.ext("dout", N, d); k.ext("dtab", v1, d); break; }
    case 308: { const int M = k.I("M"), N = k.I("N"), K = k.I("K"), m0 = k.I("m0"), n0 = k.I("n0"), T = k.I("T"), H = k.I("H");
      k.need(M > 0 && N > 0 && K > 0 && M % 128 == 0 && N % 256 == 0 && m0 % 128 == 0 && n0 % 256 == 0 && m0 < M && n0 < N,
             "needs whole 128 x 256 tiles (M % 128, N % 256, m0, n0 on tile boundaries)");
      k.need((k.I("flags") & ~3) == 0 && !k.B("bias") && !k.B("res") && !k.B("pre"), "plain epilogue only (flags 1 / 2, no bias, res, pre)");
      k.need(k.I("hd") == 64 && T > 0 && H > 0 && N == H * 64, "needs 64-column heads covering N");
      const MvmBuf* ob = k.B("out"); const MvmBuf* o = k.B("o");
      k.need(ob && o && ob->dtype == 2 && o->dtype == 2 && o->cols % 8 == 0, "out and o must be bf16 storage");
      const int fl = k.I("flags");
      k.ext("a", fl & 1 ? K : M, fl & 1 ? M : K); k.ext("b", fl & 2 ? N : K, fl & 2 ? K : N); k.ext("out", M, N); k.ext("o", M, N);
      k.extn("delta", (long long)((M - 1) / T + 1) * H * T); break; }
    case 34: case 114: case 122: case 304: {
      int M = k.I("M"), N = k.I("N"), K = k.I("K"), fl = k.I("flags"), m0 = k.I("m0"), n0 = k.I("n0");
      k.need(M > 0 && N > 0 && K > 0 && 0 <= m0 && m0 < M && 0 <= n0 && n0 < N, "bad M/N/K/m0/n0");
      k.need((fl & ~(127 | 256 | 512 | 1024)) == 0 && !((fl & 32) && (fl & 64)) && !((fl & 256) && (fl & 1024)), "unsupported flags");
      if (fl & 512) k.need(k.B("pre") && !k.B("bias") && !k.B("res") && !(fl & (4 | 8 | 128)), "flag 512 needs pre and refuses bias, res, 4, 8, 128");
      k.ext("a", fl & 1 ? K : M, fl & 1 ? M : K); k.ext("b", fl & 2 ? N : K, fl & 2 ? K : N); k.ext("out", M, N);
      k.extn("bias", N); k.ext("res", M, N); k.ext("pre", M, N); break; }
    case 35: case 36: { int r0 = k.I("r0"), r1 = k.I("r1"), d = k.I("d"); k.range(r0, r1); k.need(d > 0, "d > 0");
      k.ext("x", r1, d); k.extn("gamma", d); k.ext("out", r1, d); k.extn("rstd", r1);
      if (op == 35) { k.extn("beta", d); k.extn("mean", r1); } break; }
    case 309: { int r0 = k.I("r0"), r1 = k.I("r1"), d = k.I("d"); k.range(r0, r1); k.need(d > 0, "d > 0");
      k.ext("x", r1, d); k.ext("dy", r1, d); k.extn("gamma", d); k.extn("rstd", r1); k.extn("mean", r1); k.ext("dx", r1, d); k.ext("res", r1, d); break; }
    case 37: case 38: { int r0 = k.I("r0"), r1 = k.I("r1"), d = k.I("d"); k.range(r0, r1); k.need(d > 0, "d > 0");
      k.ext("x", r1, d); k.ext("dy", r1, d); k.extn("gamma", d); k.extn("rstd", r1); k.ext("dx", r1, d); if (op == 37) k.extn("mean", r1); break; }
    case 39: { int R = k.I("R"), d = k.I("d"), c0 = k.I("c0"), c1 = k.I("c1"); k.need(R >= 0 && 0 <= c0 && c0 <= c1 && c1 <= d, "bad R/c0/c1/d");
      k.ext("x", R, d); k.ext("dy", R, d); k.extn("mean", R); k.extn("rstd", R); k.extn("dgamma", d); k.extn("dbeta", d); break; }
    case 40: flat({"x", "out"}, "e0", "e1"); break;
    case 41: flat({"x", "dy", "dx"}, "e0", "e1"); break;
    case 42: flat({"a", "b", "out"}, "e0", "e1"); break;
    case 123: flat({"w", "g"}, "e0", "e1"); break;
    case 126: flat({"x", "out"}, "e0", "e1"); break;
    case 43: case 44: { int r0 = k.I("r0"), r1 = k.I("r1"), T = k.I("T"), H = k.I("H"), hd = k.I("hd"); k.range(r0, r1);
      k.need(T > 0 && H > 0 && hd > 0 && hd % 2 == 0, "bad T/H/hd"); k.ext("x", r1, (long long)H * hd); k.ext("out", r1, (long long)H * hd); k.extn("pos", 1); break; }
    case 45: case 47: {
      int b = k.I("b"), h = k.I("h"), q0 = k.I("q0"), T = k.I("T"), H = k.I("H"), Hkv = k.I("Hkv"), hd = k.I("hd");
      k.need(attn_hd(hd), "hd not in 16/32/64/128");
      k.need(T > 0 && H > 0 && Hkv > 0 && H % Hkv == 0 && b >= 0 && q0 >= 0 && q0 < T && 0 <= h && h < H, "bad T/H/Hkv/b/q0/h");
      long long R = (long long)(b + 1) * T;
      k.ext("q", R, (long long)H * hd); k.ext("k", R, (long long)Hkv * hd); k.ext("v", R, (long long)Hkv * hd);
      if (op == 45) { k.ext("o", R, (long long)H * hd); k.extn("lse", R * H); }
      else { k.ext("do", R, (long long)H * hd); k.extn("lse", R * H); k.extn("delta", R * H); k.ext("dq", R, (long long)H * hd); }
      break; }
    case 46: { int r0 = k.I("r0"), r1 = k.I("r1"), T = k.I("T"), H = k.I("H"), hd = k.I("hd"); k.range(r0, r1); k.need(T > 0 && H > 0 && hd > 0, "bad T/H/hd");
      k.ext("o", r1, (long long)H * hd); k.ext("do", r1, (long long)H * hd); k.extn("delta", (long long)((r1 + T - 1) / T) * H * T); break; }
    case 48: { int b = k.I("b"), kvh = k.I("kvh"), k0 = k.I("k0"), T = k.I("T"), H = k.I("H"), hd = k.I("hd");
      k.need(attn_hd(hd), "hd not in 16/32/64/128");
      k.need(T > 0 && H > 0 && b >= 0 && 0 <= k0 && k0 < T && kvh >= 0, "bad T/H/b/k0/kvh");
      const MvmBuf* kb = k.B("k");
      if (kb) k.need(kb->cols % hd == 0 && kb->cols / hd > 0 && H % (kb->cols / hd) == 0, "k.cols must be Hkv*hd with H % Hkv == 0");
      long long R = (long long)(b + 1) * T;
      k.ext("q", R, (long long)H * hd); k.ext("do", R, (long long)H * hd); k.extn("lse", R * H); k.extn("delta", R * H);
      for (const char* n : {"k", "v", "dk", "dv"}) k.ext(n, R, (long long)(kvh + 1) * hd); break; }
    case 49: { int b0 = k.I("b0"), b1 = k.I("b1"), nn = k.I("n_new"), Hkv = k.I("Hkv"), hd = k.I("hd"), Tm = k.I("Tmax"); k.range(b0, b1);
      k.need(nn > 0 && Hkv > 0 && hd > 0 && Tm > 0, "bad n_new/Hkv/hd/Tmax");
      k.ext("knew", (long long)b1 * nn, (long long)Hkv * hd); k.ext("vnew", (long long)b1 * nn, (long long)Hkv * hd);
      k.ext("kc", (long long)b1 * Hkv * Tm, hd); k.ext("vc", (long long)b1 * Hkv * Tm, hd); k.extn("lens", b1); break; }
    case 50: { int b = k.I("b"), h = k.I("h"), H = k.I("H"), Hkv = k.I("Hkv"), hd = k.I("hd"), Tm = k.I("Tmax");
      k.need(b >= 0 && 0 <= h && h < H && Hkv > 0 && H % Hkv == 0 && Tm > 0 && hd > 0 && hd <= 128, "bad b/h/H/Hkv/hd/Tmax");
      k.need((128 + Tm + 16) * 4 <= 128 * 1024, "Tmax too large for one task's LDS");
      long long n = b + 1; k.ext("q", n, (long long)H * hd); k.ext("kc", n * Hkv * Tm, hd); k.ext("vc", n * Hkv * Tm, hd); k.extn("lens", n); k.ext("o", n, (long long)H * hd); break; }
    case 51: { int r0 = k.I("r0"), r1 = k.I("r1"), V = k.I("V"); k.range(r0, r1); k.need(V > 0, "V > 0");
      k.ext("logits", r1, V); k.extn("tgt", r1); k.extn("rowloss", r1); k.extn("lse", r1); break; }
    case 52: { int N = k.I("N"); k.need(N >= 0, "N >= 0"); k.extn("rowloss", N); k.extn("tgt", N); k.extn("loss", 2); break; }
    case 53: { int r0 = k.I("r0"), r1 = k.I("r1"), V = k.I("V"); k.range(r0, r1); k.need(V > 0, "V > 0");
      k.ext("logits", r1, V); k.extn("tgt", r1); k.extn("lse", r1); k.extn("loss", 2); k.ext("dlogits", r1, V); break; }
    case 127: { int r0 = k.I("r0"), r1 = k.I("r1"), V = k.I("V"); k.range(r0, r1); k.need(V > 0 && k.I("ignore") == -1 && k.I("N") > 0, "bad V/ignore/N");
      k.ext("logits", r1, V); k.extn("tgt", r1); k.extn("rowloss", r1); k.extn("lse", r1); k.ext("dlogits", r1, V); break; }
    case 305: flat({"p", "g", "m", "v", "sh"}, "e0", "e1"); k.extn("gscale", 1); k.extn("step", 1); break;
    case 54: case 115: flat({"p", "g", "m", "v"}, "e0", "e1"); k.extn("gscale", 1); k.extn("step", 1); if (op == 115) k.extn("lr", 1); break;
    case 55: k.range(k.I("e0"), k.I("e1")); k.need(k.I("slot") >= 0, "slot >= 0"); k.extn("g", k.I("e1")); k.extn("partial", k.I("slot") + 1); break;
    case 56: k.need(k.I("nslots") >= 0, "nslots >= 0"); k.extn("partial", k.I("nslots")); k.extn("out", 2); break;
    case 57: case 58: { int r0 = k.I("r0"), r1 = k.I("r1"), V = k.I("V"); k.range(r0, r1); k.need(V > 0, "V > 0");
      k.ext("logits", r1, V); k.extn("out", r1); if (op == 57) k.extn("ctr", 1); break; }
    case 59: flat({"x"}, "e0", "e1"); break;
    case 60: flat({"x"}, "i0", "i1"); break;
    case 61: { int R = k.I("R"), c0 = k.I("c0"), c1 = k.I("c1"); k.need(R >= 0 && 0 <= c0 && c0 <= c1, "bad R/c0/c1"); k.ext("x", R, c1); k.extn("out", c1); break; }
    case 62: { k.range(k.I("i0"), k.I("i1")); k.extn("step", 1); k.extn("dst", k.I("i1"));
      const MvmBuf* s = k.B("src"); const MvmBuf* d = k.B("dst"); if (s && d) k.need((s->dtype == 1) == (d->dtype == 1) && s->dtype != 2 && d->dtype != 2, "src/dst must share a 4-byte dtype"); break; }
    case 63: { int r0 = k.I("r0"), r1 = k.I("r1"), d = k.I("d"); k.range(r0, r1); k.need(d > 0, "d > 0"); k.ext("src", 0, d); k.extn("idx", r1); k.ext("dst", r1, d); break; }
    case 96: k.need(k.I("kind") >= 0 && k.I("kind") <= 3, "kind 0..3"); flat({"x", "out"}, "e0", "e1"); break;
    case 97: k.need(k.I("kind") >= 0 && k.I("kind") <= 3, "kind 0..3"); flat({"x", "dy", "dx"}, "e0", "e1"); break;
    case 98: flat({"gate", "up", "out"}, "e0", "e1"); break;
    case 99: flat({"gate", "up", "dy", "dgate", "dup"}, "e0", "e1"); break;
    case 100: { k.range(k.I("r0"), k.I("r1")); k.need(k.I("d") > 0, "d > 0"); k.ext("x", k.I("r1"), k.I("d")); k.ext("out", k.I("r1"), k.I("d")); break; }
    case 101: { k.range(k.I("r0"), k.I("r1")); k.need(k.I("d") > 0, "d > 0"); for (const char* n : {"p", "dp", "dx"}) k.ext(n, k.I("r1"), k.I("d")); break; }
    case 102: { int r1 = k.I("r1"), d = k.I("d"), i0 = k.I("idx0"); k.range(k.I("r0"), r1); k.need(d > 0 && i0 >= 0, "bad d/idx0");
      k.ext("src", 0, d); k.extn("idx", (long long)i0 + r1); k.extn("scale", (long long)i0 + r1); k.ext("dst", r1, d); break; }
    case 103: { int N = k.I("N"), v0 = k.I("v0"), v1 = k.I("v1"), d = k.I("d"), i0 = k.I("idx0"); k.need(N >= 0 && 0 <= v0 && v0 <= v1 && d > 0 && i0 >= 0, "bad N/v0/v1/d");
      k.ext("src", N, d); k.extn("idx", (long long)i0 + N); k.extn("scale", (long long)i0 + N); k.ext("dst", v1, d); break; }
    case 104: { int r1 = k.I("r1"), d = k.I("d"), i0 = k.I("idx0"); k.range(k.I("r0"), r1); k.need(d > 0 && i0 >= 0, "bad d/idx0");
      k.ext("a", 0, d); k.ext("b", r1, d); k.extn("idx", (long long)i0 + r1); k.extn("out", (long long)i0 + r1); break; }
    case 113: flat({"x", "out"}, "e0", "e1"); break;
    case 116: k.need(k.I("kind") >= 0 && k.I("kind") <= 2, "kind 0..2"); k.extn("step", 1); k.extn("lr", 1); break;
    case 117: flat({"x", "out"}, "e0", "e1"); break;
    case 118: { int r1 = k.I("r1"), T = k.I("T"), d = k.I("d"); k.range(k.I("r0"), r1); k.need(T > 0 && d > 0, "bad T/d");
      k.ext("x", r1, d); k.ext("pos", T, d); k.ext("out", r1, d); break; }
    case 120: case 121: { int M = k.I("M"), N = k.I("N"), K = k.I("K"), fl = k.I("flags"), m0 = k.I("m0"), n0 = k.I("n0");
      k.need(M > 0 && N > 0 && K > 0 && 0 <= m0 && m0 < M && 0 <= n0 && n0 < N, "bad M/N/K/m0/n0");
      k.need((fl & ~(19 | 96)) == 0 && !((fl & 32) && (fl & 64)), "unsupported flags");
      k.ext("a", fl & 1 ? K : M, fl & 1 ? M : K); k.ext("b", fl & 2 ? N : K, fl & 2 ? K : N);
      for (const char* n : {"out", "gate", "up", "dgate", "dup"}) if (k.idx(n) >= 0) k.ext(n, M, N); break; }
    case 134: { int n0 = k.I("n0"), n1 = k.I("n1"), K = k.I("K"), pro = k.I("pro");
      k.need(0 <= n0 && n0 < n1 && K > 0 && K % 8 == 0 && pro >= 0 && pro <= 2, "bad range, K or pro");
      k.need((2 * K + 64) * 4 <= 128 * 1024, "K too large for one task's LDS");
      k.extn("x", K); k.extn("x2", K); k.extn("gamma", K); k.ext("w", n1, K); k.ext("out", 1, n1); k.ext("res", 1, n1);
      if (pro == 1) k.need(k.B("gamma") != nullptr, "pro 1 needs gamma");
      if (pro == 2) k.need(k.B("x2") != nullptr, "pro 2 needs x2");
      const MvmBuf* w = k.B("w"); if (w) k.need(w->dtype == 2 && w->cols % 8 == 0, "w must be bf16 storage with cols % 8 == 0");
      break; }
    case 310: { const int S = k.I("S"), H = k.I("H"), Hkv = k.I("Hkv"), b = k.I("b");
      k.need(Hkv > 0 && b >= 0 && (long long)(H / Hkv) * (S + 1) * 4 <= 128 * 1024, "G*(S+1) too large for one task's LDS");
      k.ext("o", (long long)b + 1, (long long)H * 128); k.extn("cnt", ((long long)b + 1) * Hkv); }
      [[fallthrough]];
    case 306: { const MvmBuf* kc = k.B("kc"); const MvmBuf* vc = k.B("vc"); const int H = k.I("H"), Hkv = k.I("Hkv");
      k.need(k.I("hd") == 128 && kc && vc && kc->dtype == 2 && vc->dtype == 2 && Hkv > 0 && H % Hkv == 0 &&
             (H / Hkv == 1 || H / Hkv == 2 || H / Hkv == 4 || H / Hkv == 8) && (k.I("flags") == 1 || k.I("flags") == 3),
             "needs hd 128, bf16 kc/vc, H/Hkv in {1,2,4,8} and flags 1 or 3");
      k.extn("qgamma", 128); k.extn("kgamma", 128); }
      [[fallthrough]];
    case 135: { int b = k.I("b"), kvh = k.I("kvh"), s = k.I("s"), S = k.I("S"), H = k.I("H"), Hkv = k.I("Hkv"), hd = k.I("hd"), Tm = k.I("Tmax"), fl = k.I("flags");
      k.need(b >= 0 && Hkv > 0 && H % Hkv == 0 && 0 <= kvh && kvh < Hkv && 0 <= s && s < S && Tm > 0, "bad b/kvh/s/S/H/Hkv/Tmax");
      k.need(0 < hd && hd <= 128 && hd % 8 == 0 && H / Hkv <= 8, "hd must be a multiple of 8 up to 128, H/Hkv <= 8");
      k.need(fl == 0 || fl == 1 || fl == 3, "flags must be 0, 1 or 3");
      long long n = b + 1; k.ext("q", n, (long long)H * hd); k.ext("kc", n * Hkv * Tm, hd); k.ext("vc", n * Hkv * Tm, hd); k.extn("lens", n);
      k.ext("part", n * S * H, hd + 2);
      if (fl & 1) { k.need(k.B("knew") && k.B("vnew"), "flag 1 needs knew and vnew"); k.ext("knew", n, (long long)Hkv * hd); k.ext("vnew", n, (long long)Hkv * hd); }
      const MvmBuf* kc = k.B("kc"); if (kc && kc->dtype == 2) k.need(kc->cols % 8 == 0, "bf16 kc needs cols % 8 == 0");
      break; }
    case 136: { int b = k.I("b"), h0 = k.I("h0"), h1 = k.I("h1"), S = k.I("S"), H = k.I("H"), hd = k.I("hd");
      k.need(b >= 0 && 0 <= h0 && h0 < h1 && h1 <= H && S > 0 && hd > 0, "bad b/h0/h1/S/H/hd");
      k.need((long long)(h1 - h0) * (S + 1) * 4 <= 128 * 1024, "(h1-h0)*(S+1) too large for one task's LDS");
      long long n = b + 1; k.ext("part", n * S * H, hd + 2); k.ext("o", n, (long long)H * hd); break; }
    case 301: { int n0 = k.I("n0"), n1 = k.I("n1"), K = k.I("K"), M = k.I("M"), pro = k.I("pro");
      k.need(0 <= n0 && n0 < n1 && K > 0 && K % 64 == 0 && 1 <= M && M <= 16 && pro >= 0 && pro <= 2, "bad range, K (% 64), M (1..16) or pro");
      k.ext("x", M, K); k.ext("x2", M, K); k.extn("gamma", K); k.ext("w", n1, K); k.ext("out", M, n1); k.ext("res", M, n1);
      if (pro == 1) k.need(k.B("gamma") != nullptr, "pro 1 needs gamma");
      if (pro == 2) k.need(k.B("x2") != nullptr, "pro 2 needs x2");
      const MvmBuf* w = k.B("w"); if (w) k.need(w->dtype == 2 && w->cols % 8 == 0, "w must be bf16 storage with cols % 8 == 0");
      break; }
    case 311: { int n0 = k.I("n0"), n1 = k.I("n1"), K = k.I("K"), M = k.I("M");
      k.need(0 <= n0 && n0 < n1 && K > 0 && K % 256 == 0 && 1 <= M && M <= 16, "bad range, K (% 256) or M (1..16)");
      k.ext("x", M, K); k.extn("gamma", K); k.ext("wg", n1, K); k.ext("wu", n1, K); k.ext("out", M, n1);
      const MvmBuf* wg = k.B("wg"); const MvmBuf* wu = k.B("wu"); const MvmBuf* x = k.B("x"); const MvmBuf* o = k.B("out");
      if (wg && wu) k.need(wg->dtype == 2 && wu->dtype == 2 && wg->cols % 8 == 0 && wg->rows == wu->rows && wg->cols == wu->cols,
                           "wg and wu must be bf16 storage of one shape with cols % 8 == 0");
      if (x && o) k.need(x->dtype != 1 && o->dtype != 1 && x->cols % 4 == 0, "x and out must be f32 or bf16, x cols % 4 == 0");
      break; }
    case 302: {
      int M = k.I("M"), N = k.I("N"), K = k.I("K"), fl = k.I("flags"), m0 = k.I("m0"), n0 = k.I("n0"), k0 = k.I("k0"), om0 = k.I("om0");
      k.need(M > 0 && N > 0 && K > 0 && 0 <= m0 && m0 < M && 0 <= n0 && n0 < N && k0 >= 0 && om0 >= 0, "bad M/N/K/m0/n0/k0/om0");
      k.need((fl & ~(1 | 2 | 4 | 32 | 64)) == 0, "flags: only 1, 2, 4, 32, 64");
      k.need(!k.B("bias") && !k.B("res") && !k.B("pre"), "bias, res and pre must be absent");
      const long long k1 = (long long)k0 + K;
      k.ext("a", fl & 1 ? k1 : M, fl & 1 ? M : k1); k.ext("b", fl & 2 ? N : k1, fl & 2 ? k1 : N); k.ext("out", (long long)om0 + M, N); break; }
    case 303: { int M = k.I("M"), N = k.I("N"), S = k.I("S"), r0 = k.I("r0"), r1 = k.I("r1");
      k.need(M > 0 && N > 0 && S > 0 && 0 <= r0 && r0 <= r1 && r1 <= M, "bad M/N/S/r0/r1");
      k.ext("part", (long long)(S - 1) * M + r1, N); k.ext("out", r1, N); break; }
    case 300: { int r1 = k.I("r1"), H = k.I("H"), hd = k.I("hd"); k.range(k.I("r0"), r1); k.need(H > 0 && hd > 0, "bad H/hd");
      k.ext("x", r1, (long long)H * hd); k.ext("out", r1, (long long)H * hd); k.extn("gamma", hd); break; }
    default: k.need(false, "no extent rule");
  }
}

}  // namespace kvmv

static const char* kvm_registry_name(int id) { const kvmv::OpSig* o = kvmv::find_op(id); return o ? o->name : nullptr; }

// Version waits that the bundle itself must satisfy (reference check: mvm_exec.cu:179-205). A task waiting for
// version w of variable v can only start after every in-bundle publisher of v with pub_ver <= w has finished (versions
// advance one step at a time). Those implied edges are added to the dependency graph through one virtual node per
// published (variable, version): publisher -> node(v, k), node(v, k_prev) -> node(v, k) for the next lower published
// version, and node(v, k*) -> waiter for the highest published k* <= w. The graph is O(tasks + edges + publishers)
// and must stay acyclic, else some task can never run. Waits above every in-bundle publication depend on the outside
// (base versions, other bundles) and add no edge.
static bool version_waits_acyclic(const MvmTaskDesc* t, int n, const int32_t* succ, std::string* why) {
  std::vector<std::pair<long long, int>> pubs;   // ((var << 32) | ver, publisher)
  for (int i = 0; i < n; ++i) if (t[i].pub_var >= 0) pubs.push_back({((long long)t[i].pub_var << 32) | (unsigned)t[i].pub_ver, i});
  if (pubs.empty()) return true;
  for (int i = 0; i < n; ++i)
    if (t[i].wait_var >= 0 && t[i].wait_var == t[i].pub_var && t[i].pub_ver <= t[i].wait_ver) {
      *why = "task " + std::to_string(i) + ": waits for version " + std::to_string(t[i].wait_ver) + " of variable " +
             std::to_string(t[i].wait_var) + " that it publishes itself";
      return false;
    }
  std::sort(pubs.begin(), pubs.end());
  std::vector<long long> key;                     // distinct published (var, ver), ascending: virtual node n + j
  std::vector<int> node_of(pubs.size());
  for (size_t k = 0; k < pubs.size(); ++k) {
    if (key.empty() || key.back() != pubs[k].first) key.push_back(pubs[k].first);
    node_of[k] = (int)key.size() - 1;
  }
  const int nv = (int)key.size(), N = n + nv;
  std::vector<std::vector<int>> extra(N);          // implied edges only; the bundle's own edges are read from succ
  for (size_t k = 0; k < pubs.size(); ++k) extra[pubs[k].second].push_back(n + node_of[k]);
  for (int j = 1; j < nv; ++j) if ((key[j] >> 32) == (key[j - 1] >> 32)) extra[n + j - 1].push_back(n + j);
  for (int i = 0; i < n; ++i) {
    if (t[i].wait_var < 0) continue;
    const long long want = ((long long)t[i].wait_var << 32) | (unsigned)t[i].wait_ver;
    auto it = std::upper_bound(key.begin(), key.end(), want);   // first key above the wanted version
    if (it == key.begin()) continue;
    --it;
    if ((*it >> 32) != t[i].wait_var) continue;    // no in-bundle publication of this variable at or below w
    extra[n + (int)(it - key.begin())].push_back(i);
  }
  std::vector<int> deg(N, 0), st;
  for (int i = 0; i < n; ++i) for (int k = 0; k < t[i].succ_cnt; ++k) ++deg[succ[t[i].succ_off + k]];
  for (int u = 0; u < N; ++u) for (int v : extra[u]) ++deg[v];
  for (int u = 0; u < N; ++u) if (!deg[u]) st.push_back(u);
  int seen = 0;
  while (!st.empty()) {
    const int u = st.back(); st.pop_back(); ++seen;
    if (u < n) for (int k = 0; k < t[u].succ_cnt; ++k) { const int v = succ[t[u].succ_off + k]; if (--deg[v] == 0) st.push_back(v); }
    for (int v : extra[u]) if (--deg[v] == 0) st.push_back(v);
  }
  if (seen != N) { *why = "version-wait cycle: a task waits for a version that only a task depending on it can publish"; return false; }
  return true;
}

// Whole-bundle validation: descriptors, arity, edges, indegrees, acyclicity, buffer arguments, extents.
static bool kvm_validate_bundle(const MvmTaskDesc* t, int n, const int32_t* succ, int ne, const int32_t* args, int na,
                                const MvmBuf* bufs, int nbufs, int nvars, std::string* why) {
  using namespace kvmv;
  auto bad = [&](int i, const std::string& m) { *why = "task " + std::to_string(i) + ": " + m; return false; };
  std::vector<int> indeg(n, 0);
  for (int i = 0; i < n; ++i) {
    const MvmTaskDesc& d = t[i];
    const OpSig* o = find_op(d.op_id);
    if (!o) return bad(i, "op_id " + std::to_string(d.op_id) + " not in the registry");
    if (!implemented(d.op_id)) return bad(i, std::string("operator ") + o->name + " is not run by this executor");
    std::vector<ArgInfo> sig = parse_sig(o->sig);
    if (d.args_words != (int)sig.size()) return bad(i, "args_words != arity of " + std::string(o->name));
    if (d.args_words > KVM_MAX_ARGS) return bad(i, "more argument words than a task's LDS argument block holds");
    if (d.succ_off < 0 || d.succ_cnt < 0 || (long long)d.succ_off + d.succ_cnt > ne) return bad(i, "successor range outside the bundle");
    if (d.args_off < 0 || (long long)d.args_off + d.args_words > na) return bad(i, "argument range outside the bundle");
    if (d.indegree < 0) return bad(i, "negative indegree");
    if (d.wait_var < -1 || d.wait_var >= nvars || d.pub_var < -1 || d.pub_var >= nvars) return bad(i, "version variable out of range");
    if (d.pub_var >= 0 && d.pub_ver < 1) return bad(i, "pub_ver must be >= 1");
    if (d.wait_var >= 0 && d.wait_ver < 0) return bad(i, "wait_ver must be >= 0");
    if (d.priority < 0 || d.priority >= KVM_PRIORITIES) return bad(i, "priority " + std::to_string(d.priority) + " outside [0, " + std::to_string(KVM_PRIORITIES - 1) + "]");
    if (d.deadline_us < -1) return bad(i, "deadline_us must be -1 (none) or >= 0");
    for (int k = 0; k < d.succ_cnt; ++k) {
      int s = succ[d.succ_off + k];
      if (s < 0 || s >= n || s == i) return bad(i, "successor index out of range");
      ++indeg[s];
    }
    const int32_t* a = args + d.args_off;
    for (size_t k = 0; k < sig.size(); ++k) {
      if (sig[k].type != 0) continue;
      int w = a[k];
      if (w == -1 && sig[k].opt) continue;
      if (w < 0 || w >= nbufs) return bad(i, std::string(o->name) + " arg '" + sig[k].name + "': buffer index out of range");
      char cls = arg_class(d.op_id, sig[k].name);
      int dt = bufs[w].dtype;
      if (cls == 'i' && dt != 1) return bad(i, std::string(o->name) + " arg '" + sig[k].name + "' needs an i32 buffer");
      if (cls == 'f' && dt != 0) return bad(i, std::string(o->name) + " arg '" + sig[k].name + "' needs an f32 buffer");
      if (d.op_id == 1 && dt == 2) return bad(i, "copy moves 4-byte words: bf16 buffers are refused");
      if (cls == 'a' && dt == 1 && d.op_id != 1 && d.op_id != 59 && d.op_id != 62) return bad(i, std::string(o->name) + " arg '" + sig[k].name + "' must be f32 or bf16");
    }
    Check c{bufs, nbufs, a, sig, "", o->name};
    extents(d.op_id, c);
    if (!c.err.empty()) return bad(i, c.err);
  }
  for (int i = 0; i < n; ++i) if (indeg[i] != t[i].indegree) return bad(i, "indegree differs from the number of in-bundle predecessors");
  std::vector<int> rem(indeg), q; q.reserve(n);
  for (int i = 0; i < n; ++i) if (rem[i] == 0) q.push_back(i);
  for (size_t h = 0; h < q.size(); ++h) { const MvmTaskDesc& d = t[q[h]]; for (int k = 0; k < d.succ_cnt; ++k) if (--rem[succ[d.succ_off + k]] == 0) q.push_back(succ[d.succ_off + k]); }
  if ((int)q.size() != n) { *why = "dependency cycle"; return false; }
  return version_waits_acyclic(t, n, succ, why);
}
