// CPU ORACLE — test infrastructure only. Nothing in the product path (kvm_amd/) links or calls this file; it is
// built for tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker.
//
// A restatement, in C++, of the reference's CPU path:
//   * the deterministic bundle interpreter (reference: runtime/workload_vm.py:45-286; deterministic pick = highest
//     priority, then lowest task index, :128-129; version publish and exact/at_least checks, :168-202);
//   * the operator semantics of runtime/ref_ops.py (core ops: every result rounded to f32, ascending order),
//     runtime/ref_gpt.py and runtime/ref_extra.py (double intermediates, sums left to right as Python's sum() does,
//     libm transcendentals, one f32 rounding per stored value), including the bf16-storage variants
//     (ref_extra.py:560-612: a value stored to a bf16 buffer is rounded to bf16, nearest even).
// Buffers are host arrays: f32 and bf16 buffers as float (bf16 buffers hold bf16-representable values), i32 as int32.
//
// Parity pins (tests/test_oracle.py): the reference VM's own final buffers for every case in tests/golden (bit-exact),
// the SplitMix64 vectors of the reference (tests/golden/data/initgen_vectors.txt), and closed forms.
// Deliberate difference: matmul_tile_bf16 with a bf16-storage output and a 128x128 / 256x128 tile flag rounds every
// stored element (as the reference's device does); the reference's CPU model rounds only the first 64x64 of such a
// tile (ref_extra.py:317-323). No workload here uses that combination.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <chrono>
#include <functional>
#include <set>
#include <thread>
#include <mutex>
#include <condition_variable>
#include <string>
#include <vector>

extern "C" {
#include "../include/mvm_task_abi.h"
}

namespace {

struct OBuf { void* p; int32_t rows, cols, dtype; };   // dtype 0 f32, 1 i32, 2 bf16 (held as float)

struct Fail { std::string msg; };
[[noreturn]] void fail(const std::string& m) { throw Fail{m}; }
inline void need(bool c, const char* m) { if (!c) fail(m); }

inline float f32(double x) { return (float)x; }
inline float bf16r(float x) {
  if (std::isnan(x) || std::isinf(x)) return x;
  uint32_t u; memcpy(&u, &x, 4);
  u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  float r; memcpy(&r, &u, 4); return r;
}

// Typed view of a buffer argument. ld() widens; st() rounds to bf16 when the buffer is bf16 storage.
struct V {
  float* f = nullptr; int32_t* i = nullptr; int rows = 0, cols = 0, dtype = 0;
  bool ok() const { return f || i; }
  long long n() const { return (long long)rows * cols; }
  double ld(long long k) const { return f[k]; }
  double at(long long r, long long c) const { return f[r * cols + c]; }
  void st(long long k, double v) const { float x = f32(v); f[k] = dtype == 2 ? bf16r(x) : x; }
  void stf(long long k, float x) const { f[k] = dtype == 2 ? bf16r(x) : x; }
};

struct Ctx {
  OBuf* bufs; int nbufs;
  const int32_t* a;
  V buf(int k, bool opt = false) const {
    int idx = a[k];
    if (idx == -1 && opt) return V{};
    if (idx < 0 || idx >= nbufs) fail("buffer index out of range");
    OBuf& b = bufs[idx];
    V v; v.rows = b.rows; v.cols = b.cols; v.dtype = b.dtype;
    if (b.dtype == 1) v.i = (int32_t*)b.p; else v.f = (float*)b.p;
    return v;
  }
  int i(int k) const { return a[k]; }
  float fl(int k) const { float x; memcpy(&x, &a[k], 4); return x; }
};

// ------------------------------------------------------------------------------------------- helpers
inline double gelu(double x) { return 0.5 * x * (1.0 + std::tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))); }
inline double gelu_grad(double x) {
  double t = std::tanh(0.7978845608028654 * (x + 0.044715 * x * x * x));
  return 0.5 * (1 + t) + 0.5 * x * (1 - t * t) * 0.7978845608028654 * (1 + 3 * 0.044715 * x * x);
}
inline double sig(double x) { return x >= 0 ? 1.0 / (1.0 + std::exp(-x)) : std::exp(x) / (1.0 + std::exp(x)); }
inline double silu(double x) { return x * sig(x); }
inline double silu_d(double x) { double s = sig(x); return s * (1.0 + x * (1.0 - s)); }
inline long long pymod(long long a, long long b) { long long r = a % b; return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r; }
inline long long pyfloordiv(long long a, long long b) { long long q = a / b; if ((a % b != 0) && ((a < 0) != (b < 0))) --q; return q; }
inline int token(int i, int n) { if (i < 0 || i >= n) fail("token id out of range"); return i; }

// ------------------------------------------------------------------------------------------- core ops (ref_ops.py)
void op_copy(const Ctx& c) { V s = c.buf(0), d = c.buf(1); int n = c.i(2);
  for (int k = 0; k < n; ++k) { if (d.i) d.i[k] = s.i[k]; else d.f[k] = s.f[k]; } }
void op_add(const Ctx& c) { V a = c.buf(0), b = c.buf(1), o = c.buf(2); int n = c.i(3);
  for (int k = 0; k < n; ++k) o.f[k] = f32((double)a.f[k] + b.f[k]); }
void op_scale(const Ctx& c) { V x = c.buf(0), o = c.buf(1); float al = c.fl(2); int n = c.i(3);
  for (int k = 0; k < n; ++k) o.f[k] = f32((double)x.f[k] * al); }
void op_relu(const Ctx& c) { V x = c.buf(0), o = c.buf(1); int n = c.i(2);
  for (int k = 0; k < n; ++k) o.f[k] = x.f[k] > 0 ? x.f[k] : 0.0f; }
void op_sgd(const Ctx& c) { V w = c.buf(0), g = c.buf(1); float lr = c.fl(2); int n = c.i(3);
  for (int k = 0; k < n; ++k) w.f[k] = f32((double)w.f[k] - (double)f32((double)lr * g.f[k])); }
void op_predict(const Ctx& c) { V x = c.buf(0), w = c.buf(1), o = c.buf(2); int n = c.i(3);
  for (int k = 0; k < n; ++k) o.f[k] = f32((double)w.f[0] * x.f[k]); }
void op_mse_grad(const Ctx& c) {
  V p = c.buf(0), t = c.buf(1), x = c.buf(2), l = c.buf(3), g = c.buf(4); int n = c.i(5);
  float la = 0, ga = 0;
  for (int k = 0; k < n; ++k) {
    float d = f32((double)p.f[k] - t.f[k]);
    la = f32((double)la + (double)f32((double)d * d));
    ga = f32((double)ga + (double)f32((double)f32(2.0 * d) * x.f[k]));
  }
  l.f[0] = f32((double)la / n); g.f[0] = f32((double)ga / n);
}
void op_matmul(const Ctx& c) {
  V a = c.buf(0), b = c.buf(1), o = c.buf(2); int m = c.i(3), n = c.i(4), k = c.i(5);
  std::vector<float> out((size_t)m * n);
  for (int i = 0; i < m; ++i) for (int j = 0; j < n; ++j) {
    float acc = 0;
    for (int p = 0; p < k; ++p) acc = f32((double)acc + (double)f32((double)a.f[i * k + p] * b.f[p * n + j]));
    out[(size_t)i * n + j] = acc;
  }
  memcpy(o.f, out.data(), out.size() * 4);
}
void op_fill(const Ctx& c) { V x = c.buf(0); float v = c.fl(1); int n = c.i(2); for (int k = 0; k < n; ++k) x.f[k] = v; }

// ------------------------------------------------------------------------------------------- GPT ops (ref_gpt.py)
void op_embedding_fwd(const Ctx& c) {   // ref_gpt.py:43-52
  V ids = c.buf(0), wte = c.buf(1), wpe = c.buf(2, true), out = c.buf(3);
  int r0 = c.i(4), r1 = c.i(5), T = c.i(6), d = c.i(7);
  for (int r = r0; r < r1; ++r) {
    int i = token(ids.i[r], wte.rows);
    for (int k = 0; k < d; ++k) {
      double v = wte.at(i, k);
      if (wpe.ok()) v = f32(v + wpe.at(pymod(r, T), k));
      out.st((long long)r * out.cols + k, v);
    }
  }
}
void op_embedding_bwd(const Ctx& c) {   // ref_gpt.py:55-65
  V ids = c.buf(0, true), dout = c.buf(1), dt = c.buf(2);
  int N = c.i(3), mod = c.i(4), v0 = c.i(5), v1 = c.i(6), d = c.i(7), acc = c.i(8);
  need(ids.ok() || mod > 0, "embedding_bwd: ids absent needs mod > 0");
  for (int key = v0; key < v1; ++key) {
    long long base = (long long)key * dt.cols;
    if (!acc) for (int k = 0; k < d; ++k) dt.f[base + k] = 0.0f;
    auto addrow = [&](int r) { for (int k = 0; k < d; ++k) dt.f[base + k] = f32((double)dt.f[base + k] + dout.at(r, k)); };
    if (ids.ok()) { for (int r = 0; r < N; ++r) if (ids.i[r] == key) addrow(r); }
    else for (int r = key; r < N; r += mod) addrow(r);
  }
}
int tile_m(int fl) { return fl & 64 ? 256 : fl & 32 ? 128 : 64; }
int tile_n(int fl) { return fl & 64 ? 128 : fl & 32 ? 128 : 64; }
// matmul_tile (ref_gpt.py:69-95); round_ops: operands rounded to bf16 first (matmul_tile_bf16, ref_extra.py:312-323)
// The reference's tile product: acc = f32(acc + f32(a * b)) over k in order, per output element
// (ref_gpt.py:69-103). Computed in float: f32(a * b) of two floats is the float product (their exact product fits a
// double), and f32(double(acc) + double(p)) is the float sum (double rounding is innocuous for one addition), so the
// float loop below gives the same bits. Each output column keeps its own k-ordered chain; the loop runs over the
// tile's columns innermost (independent chains, which the compiler may vectorise without reassociating anything).
static void tile_product(int m0, int m1, int n0, int n1, int k0, int K, const std::function<float(int, int)>& opA,
                         const std::function<float(int, int)>& opB, std::vector<float>& acc) {
  const int nn = n1 - n0;
  std::vector<float> Bt((size_t)K * nn), arow(K);
  for (int k = 0; k < K; ++k) for (int n = 0; n < nn; ++n) Bt[(size_t)k * nn + n] = opB(n0 + n, k0 + k);
  acc.assign((size_t)(m1 - m0) * nn, 0.0f);
  for (int m = m0; m < m1; ++m) {
    for (int k = 0; k < K; ++k) arow[k] = opA(m, k0 + k);
    float* __restrict__ out = &acc[(size_t)(m - m0) * nn];
    for (int k = 0; k < K; ++k) {
      const float a = arow[k];
      const float* __restrict__ b = &Bt[(size_t)k * nn];
      for (int n = 0; n < nn; ++n) out[n] = out[n] + a * b[n];
    }
  }
}

void mm_tile(const Ctx& c, bool bf16ops, int tm_override = 0) {
  V A = c.buf(0), B = c.buf(1), out = c.buf(2), bias = c.buf(3, true), res = c.buf(4, true), pre = c.buf(5, true);
  int m0 = c.i(6), n0 = c.i(7), M = c.i(8), N = c.i(9), K = c.i(10), fl = c.i(11); float alpha = c.fl(12);
  int ta = fl & 1, tb = fl & 2, accum = fl & 4, ge = fl & 8, dg = fl & 512;
  need(!dg || (pre.ok() && !bias.ok() && !res.ok() && !accum && !ge && !(fl & 128)), "matmul_tile: flag 512 needs pre and refuses bias, res, 4, 8, 128");
  int tm = tm_override ? tm_override : tile_m(fl), tn = tm_override ? tm_override : tile_n(fl);
  auto opA = [&](int m, int k) -> float { float x = ta ? A.f[(long long)k * A.cols + m] : A.f[(long long)m * A.cols + k]; return bf16ops ? bf16r(x) : x; };
  auto opB = [&](int n, int k) -> float { float y = tb ? B.f[(long long)n * B.cols + k] : B.f[(long long)k * B.cols + n]; return bf16ops ? bf16r(y) : y; };
  const int m1 = std::min(m0 + tm, M), n1 = std::min(n0 + tn, N);
  if (m0 >= m1 || n0 >= n1) return;
  std::vector<float> accv;
  tile_product(m0, m1, n0, n1, 0, K, opA, opB, accv);
  for (int m = m0; m < m1; ++m)
    for (int n = n0; n < n1; ++n) {
      float acc = accv[(size_t)(m - m0) * (n1 - n0) + (n - n0)];
      float v = f32((double)acc * alpha);
      if (bias.ok()) v = f32((double)v + bias.f[n]);
      if (dg) v = f32((double)v * gelu_grad(pre.at(m, n)));
      else {
        if (pre.ok()) pre.stf((long long)m * pre.cols + n, v);
        if (ge) v = f32(gelu(v));
      }
      if (res.ok()) v = f32((double)v + res.at(m, n));
      long long o = (long long)m * out.cols + n;
      out.stf(o, accum ? f32((double)out.f[o] + v) : v);
    }
}
void op_matmul_tile(const Ctx& c) { mm_tile(c, false); }

template <bool RMS> void norm_fwd(const Ctx& c) {   // ref_gpt.py:107-120
  V x = c.buf(0), g = c.buf(1), be, out, mean, rstd; int k = 2;
  if (!RMS) be = c.buf(k++);
  out = c.buf(k++); if (!RMS) mean = c.buf(k++); rstd = c.buf(k++);
  int r0 = c.i(k), r1 = c.i(k + 1), d = c.i(k + 2); float eps = c.fl(k + 3);
  std::vector<double> row(d);
  for (int r = r0; r < r1; ++r) {
    for (int j = 0; j < d; ++j) row[j] = x.at(r, j);
    double mu = 0.0;
    if (!RMS) { double s = 0; for (double v : row) s += v; mu = s / d; }
    double ss = 0; for (double v : row) ss += (v - mu) * (v - mu);
    float rs = f32(1.0 / std::sqrt(ss / d + eps));
    for (int j = 0; j < d; ++j) out.st((long long)r * out.cols + j, (row[j] - mu) * rs * g.f[j] + (RMS ? 0.0 : (double)be.f[j]));
    rstd.f[r] = rs;
    if (!RMS) mean.f[r] = f32(mu);
  }
}
// res (this executor's op 309): the accumulated term read from res instead of dx.
template <bool RMS> void norm_bwd_dx(const Ctx& c, bool res_op = false) {   // ref_gpt.py:131-144
  V x = c.buf(0), dy = c.buf(1), g = c.buf(2), mean, rstd, dx, res; int k = 3;
  if (!RMS) mean = c.buf(k++);
  rstd = c.buf(k++); dx = c.buf(k++);
  if (res_op) res = c.buf(k++);
  int r0 = c.i(k), r1 = c.i(k + 1), d = c.i(k + 2), acc = res_op ? 1 : c.i(k + 3);
  std::vector<double> gs(d), xh(d);
  for (int r = r0; r < r1; ++r) {
    double mu = RMS ? 0.0 : mean.f[r], rs = rstd.f[r];
    for (int j = 0; j < d; ++j) { gs[j] = dy.at(r, j) * g.f[j]; xh[j] = (x.at(r, j) - mu) * rs; }
    double s1 = 0.0;
    if (!RMS) { double s = 0; for (double v : gs) s += v; s1 = s / d; }
    double s2 = 0; for (int j = 0; j < d; ++j) s2 += gs[j] * xh[j];
    s2 /= d;
    for (int j = 0; j < d; ++j) {
      float v = f32(rs * (gs[j] - s1 - xh[j] * s2));
      long long o = (long long)r * dx.cols + j;
      const double prev = res_op ? (double)res.f[(long long)r * res.cols + j] : (double)dx.f[o];
      dx.st(o, acc ? (double)f32(prev + v) : (double)v);
    }
  }
}
void op_layernorm_bwd_dx(const Ctx& c) { norm_bwd_dx<false>(c); }
void op_rmsnorm_bwd_dx(const Ctx& c) { norm_bwd_dx<true>(c); }
void op_layernorm_bwd_dx_res(const Ctx& c) { norm_bwd_dx<false>(c, true); }   // this executor's op 309
void op_norm_bwd_params(const Ctx& c) {   // ref_gpt.py:147-159
  V x = c.buf(0), dy = c.buf(1), mean = c.buf(2, true), rstd = c.buf(3), dg = c.buf(4), db = c.buf(5, true);
  int R = c.i(6), c0 = c.i(8), c1 = c.i(9), acc = c.i(10);
  for (int j = c0; j < c1; ++j) {
    double sg = 0, sb = 0;
    for (int r = 0; r < R; ++r) {
      double g = dy.at(r, j);
      sg += g * (x.at(r, j) - (mean.ok() ? (double)mean.f[r] : 0.0)) * rstd.f[r];
      sb += g;
    }
    dg.f[j] = acc ? f32((double)dg.f[j] + sg) : f32(sg);
    if (db.ok()) db.f[j] = acc ? f32((double)db.f[j] + sb) : f32(sb);
  }
}
void op_colsum(const Ctx& c) {   // ref_gpt.py:167-173
  V x = c.buf(0), out = c.buf(1); int R = c.i(2), c0 = c.i(3), c1 = c.i(4), acc = c.i(5);
  for (int j = c0; j < c1; ++j) {
    float s = 0; for (int r = 0; r < R; ++r) s = f32((double)s + x.at(r, j));
    out.f[j] = acc ? f32((double)out.f[j] + s) : s;
  }
}
void op_gelu_fwd(const Ctx& c) { V x = c.buf(0), o = c.buf(1); for (int k = c.i(2); k < c.i(3); ++k) o.st(k, gelu(x.f[k])); }
void op_gelu_bwd(const Ctx& c) { V x = c.buf(0), dy = c.buf(1), dx = c.buf(2); int acc = c.i(5);
  for (int k = c.i(3); k < c.i(4); ++k) { float v = f32((double)dy.f[k] * gelu_grad(x.f[k])); dx.st(k, acc ? (double)f32((double)dx.f[k] + v) : (double)v); } }
void op_residual_add(const Ctx& c) { V a = c.buf(0), b = c.buf(1), o = c.buf(2);
  for (int k = c.i(3); k < c.i(4); ++k) o.st(k, (double)a.f[k] + b.f[k]); }
void op_sgd_range(const Ctx& c) { V w = c.buf(0), g = c.buf(1); float lr = c.fl(2);
  for (int k = c.i(3); k < c.i(4); ++k) w.f[k] = f32((double)w.f[k] - (double)f32((double)lr * g.f[k])); }
void op_round_tf32(const Ctx& c) { V x = c.buf(0), o = c.buf(1);
  for (int k = c.i(2); k < c.i(3); ++k) { uint32_t u; memcpy(&u, &x.f[k], 4); if ((u & 0x7fffffffu) <= 0x7f800000u) u += 0x1000u; u &= 0xffffe000u; memcpy(&o.f[k], &u, 4); } }
void op_zero_buf(const Ctx& c) { V x = c.buf(0); for (int k = c.i(1); k < c.i(2); ++k) { if (x.i) x.i[k] = 0; else x.f[k] = 0.0f; } }
void op_counter_inc(const Ctx& c) { V x = c.buf(0); for (int k = c.i(1); k < c.i(2); ++k) x.i[k] = (int32_t)(uint32_t)((uint32_t)x.i[k] + (uint32_t)c.i(3)); }

inline float rope_ang(long long p, int i, int hd, float theta) {
  return f32((double)f32((double)p) * (double)f32(std::pow((double)theta, -(double)f32((double)(2 * i)) / hd)));
}
template <int SIGN> void op_rope(const Ctx& c) {   // ref_gpt.py:250-262
  V x = c.buf(0), out = c.buf(1), pos = c.buf(2, true);
  int r0 = c.i(3), r1 = c.i(4), T = c.i(5), H = c.i(6), hd = c.i(7); float th = c.fl(8);
  long long p0 = pos.ok() ? pos.i[0] : 0; int half = hd / 2;
  for (int r = r0; r < r1; ++r) for (int h = 0; h < H; ++h) for (int i = 0; i < half; ++i) {
    float ang = rope_ang(pymod(r, T) + p0, i, hd, th);
    double s = SIGN * (double)f32(std::sin((double)ang)), co = f32(std::cos((double)ang));
    double x1 = x.at(r, h * hd + i), x2 = x.at(r, h * hd + i + half);
    out.st((long long)r * out.cols + h * hd + i, x1 * co - x2 * s);
    out.st((long long)r * out.cols + h * hd + i + half, x1 * s + x2 * co);
  }
}

const int ATTN_ROWS = 128;
void op_attn_fwd(const Ctx& c) {   // ref_gpt.py:279-291
  V q = c.buf(0), k = c.buf(1), v = c.buf(2), o = c.buf(3), lse = c.buf(4);
  int bb = c.i(5), h = c.i(6), q0 = c.i(7), T = c.i(8), H = c.i(9), Hkv = c.i(10), hd = c.i(11); float sc = c.fl(12);
  need(hd == 16 || hd == 32 || hd == 64 || hd == 128, "attention: bad hd");
  int kvh = h / (H / Hkv);
  std::vector<double> s, p;
  for (int gq = q0; gq < std::min(q0 + ATTN_ROWS, T); ++gq) {
    s.assign(gq + 1, 0); p.assign(gq + 1, 0);
    for (int j = 0; j <= gq; ++j) { double a = 0; for (int cc = 0; cc < hd; ++cc) a += q.at((long long)bb * T + gq, h * hd + cc) * k.at((long long)bb * T + j, kvh * hd + cc); s[j] = a * sc; }
    double m = s[0]; for (double x : s) if (x > m) m = x;
    double l = 0; for (int j = 0; j <= gq; ++j) { p[j] = std::exp(s[j] - m); l += p[j]; }
    for (int cc = 0; cc < hd; ++cc) { double a = 0; for (int j = 0; j <= gq; ++j) a += p[j] * v.at((long long)bb * T + j, kvh * hd + cc);
      o.st(((long long)bb * T + gq) * o.cols + h * hd + cc, a / l); }
    lse.f[((long long)bb * H + h) * T + gq] = f32(m + std::log(l));
  }
}
void op_attn_bwd_delta(const Ctx& c) {   // ref_gpt.py:301-305
  V o = c.buf(0), d = c.buf(1), delta = c.buf(2); int r0 = c.i(3), r1 = c.i(4), T = c.i(5), H = c.i(6), hd = c.i(7);
  for (int r = r0; r < r1; ++r) for (int h = 0; h < H; ++h) {
    double a = 0; for (int cc = 0; cc < hd; ++cc) a += o.at(r, h * hd + cc) * d.at(r, h * hd + cc);
    delta.f[((long long)(r / T) * H + h) * T + r % T] = f32(a);
  }
}
void op_attn_bwd_dq(const Ctx& c) {   // ref_gpt.py:315-330
  V q = c.buf(0), k = c.buf(1), v = c.buf(2), d = c.buf(3), lse = c.buf(4), delta = c.buf(5), dq = c.buf(6);
  int bb = c.i(7), h = c.i(8), q0 = c.i(9), T = c.i(10), H = c.i(11), Hkv = c.i(12), hd = c.i(13); float sc = c.fl(14);
  int kvh = h / (H / Hkv);
  std::vector<double> acc(hd);
  for (int gq = q0; gq < std::min(q0 + ATTN_ROWS, T); ++gq) {
    double li = lse.f[((long long)bb * H + h) * T + gq], di = delta.f[((long long)bb * H + h) * T + gq];
    std::fill(acc.begin(), acc.end(), 0.0);
    long long qr = (long long)bb * T + gq;
    for (int j = 0; j <= gq; ++j) {
      long long kr = (long long)bb * T + j;
      double s = 0, dp = 0;
      for (int cc = 0; cc < hd; ++cc) s += q.at(qr, h * hd + cc) * k.at(kr, kvh * hd + cc);
      for (int cc = 0; cc < hd; ++cc) dp += d.at(qr, h * hd + cc) * v.at(kr, kvh * hd + cc);
      double ds = std::exp(s * sc - li) * (dp - di);
      for (int cc = 0; cc < hd; ++cc) acc[cc] += ds * k.at(kr, kvh * hd + cc);
    }
    for (int cc = 0; cc < hd; ++cc) dq.st(qr * dq.cols + h * hd + cc, acc[cc] * sc);
  }
}
void op_attn_bwd_dkv(const Ctx& c) {   // ref_gpt.py:333-352
  V q = c.buf(0), k = c.buf(1), v = c.buf(2), d = c.buf(3), lse = c.buf(4), delta = c.buf(5), dk = c.buf(6), dv = c.buf(7);
  int bb = c.i(8), kvh = c.i(9), k0 = c.i(10), T = c.i(11), H = c.i(12), hd = c.i(13); float sc = c.fl(14);
  int G = H / (k.cols / hd);
  std::vector<double> sk(hd), sv(hd);
  for (int gk = k0; gk < std::min(k0 + ATTN_ROWS, T); ++gk) {
    std::fill(sk.begin(), sk.end(), 0.0); std::fill(sv.begin(), sv.end(), 0.0);
    long long kr = (long long)bb * T + gk;
    for (int h = kvh * G; h < (kvh + 1) * G; ++h)
      for (int gq = gk; gq < T; ++gq) {
        double li = lse.f[((long long)bb * H + h) * T + gq], di = delta.f[((long long)bb * H + h) * T + gq];
        long long qr = (long long)bb * T + gq;
        double s = 0, dp = 0;
        for (int cc = 0; cc < hd; ++cc) s += q.at(qr, h * hd + cc) * k.at(kr, kvh * hd + cc);
        for (int cc = 0; cc < hd; ++cc) dp += d.at(qr, h * hd + cc) * v.at(kr, kvh * hd + cc);
        double p = std::exp(s * sc - li);
        for (int cc = 0; cc < hd; ++cc) { sv[cc] += p * d.at(qr, h * hd + cc); sk[cc] += p * (dp - di) * q.at(qr, h * hd + cc); }
      }
    for (int cc = 0; cc < hd; ++cc) { dk.st(kr * dk.cols + kvh * hd + cc, sk[cc] * sc); dv.st(kr * dv.cols + kvh * hd + cc, sv[cc]); }
  }
}
void op_kv_append(const Ctx& c) {   // ref_gpt.py:367-380
  V kn = c.buf(0), vn = c.buf(1), kc = c.buf(2), vc = c.buf(3), lens = c.buf(4);
  int b0 = c.i(5), b1 = c.i(6), nn = c.i(7), Hkv = c.i(8), hd = c.i(9), Tmax = c.i(10);
  for (int b = b0; b < b1; ++b) if (lens.i[b] < 0 || lens.i[b] + nn > Tmax) fail("kv_append: length exceeds Tmax");
  for (int b = b0; b < b1; ++b) for (int t = 0; t < nn; ++t) for (int h = 0; h < Hkv; ++h) {
    long long row = ((long long)b * Hkv + h) * Tmax + lens.i[b] + t;
    for (int cc = 0; cc < hd; ++cc) { kc.st(row * kc.cols + cc, kn.at((long long)b * nn + t, h * hd + cc)); vc.st(row * vc.cols + cc, vn.at((long long)b * nn + t, h * hd + cc)); }
  }
}
void op_attn_decode(const Ctx& c) {   // ref_gpt.py:391-404
  V q = c.buf(0), kc = c.buf(1), vc = c.buf(2), lens = c.buf(3), o = c.buf(4);
  int bb = c.i(5), h = c.i(6), H = c.i(7), Hkv = c.i(8), hd = c.i(9), Tmax = c.i(10); float sc = c.fl(11);
  int n = lens.i[bb] + 1;
  if (lens.i[bb] < 0 || n > Tmax) fail("attn_decode: length exceeds Tmax");
  long long base = ((long long)bb * Hkv + h / (H / Hkv)) * Tmax;
  std::vector<double> s(n), p(n);
  for (int j = 0; j < n; ++j) { double a = 0; for (int cc = 0; cc < hd; ++cc) a += q.at(bb, h * hd + cc) * kc.at(base + j, cc); s[j] = a * sc; }
  double m = s[0]; for (double x : s) if (x > m) m = x;
  double l = 0; for (int j = 0; j < n; ++j) { p[j] = std::exp(s[j] - m); l += p[j]; }
  for (int cc = 0; cc < hd; ++cc) { double a = 0; for (int j = 0; j < n; ++j) a += p[j] * vc.at(base + j, cc); o.st((long long)bb * o.cols + h * hd + cc, a / l); }
}
void ce_fwd(const Ctx& c, V lg, V tg, V rl, V ls, int r0, int r1, int Vn, int ignore) {   // ref_gpt.py:414-426
  for (int r = r0; r < r1; ++r) {
    int t = tg.i[r];
    if (t == ignore) { rl.f[r] = ls.f[r] = 0.0f; continue; }
    token(t, Vn);
    double m = lg.at(r, 0); for (int j = 1; j < Vn; ++j) if (lg.at(r, j) > m) m = lg.at(r, j);
    double s = 0; for (int j = 0; j < Vn; ++j) s += std::exp(lg.at(r, j) - m);
    double l = m + std::log(s);
    ls.f[r] = f32(l); rl.f[r] = f32(l - lg.at(r, t));
  }
}
void ce_bwd(V lg, V tg, V ls, V dl, int r0, int r1, int Vn, int ignore, float f) {   // ref_gpt.py:440-448
  for (int r = r0; r < r1; ++r) {
    int t = tg.i[r];
    if (t != ignore) token(t, Vn);
    for (int j = 0; j < Vn; ++j)
      dl.st((long long)r * dl.cols + j, t == ignore ? 0.0 : (double)f32((std::exp(lg.at(r, j) - ls.f[r]) - (j == t ? 1.0 : 0.0)) * f));
  }
}
void op_softmax_ce_fwd(const Ctx& c) { ce_fwd(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.i(4), c.i(5), c.i(6), c.i(7)); }
void op_softmax_ce_reduce(const Ctx& c) {   // ref_gpt.py:429-437
  V rl = c.buf(0), tg = c.buf(1), loss = c.buf(2); int N = c.i(3), ignore = c.i(4);
  double s = 0; int cnt = 0;
  for (int r = 0; r < N; ++r) if (tg.i[r] != ignore) { s += rl.f[r]; ++cnt; }
  loss.f[0] = cnt ? f32(s / cnt) : 0.0f; loss.f[1] = cnt ? f32(1.0 / cnt) : 0.0f;
}
void op_softmax_ce_bwd(const Ctx& c) {
  V loss = c.buf(3);
  ce_bwd(c.buf(0), c.buf(1), c.buf(2), c.buf(4), c.i(5), c.i(6), c.i(7), c.i(8), f32((double)loss.f[1] * c.fl(9)));
}
void op_softmax_ce_fused(const Ctx& c) {   // ref_gpt.py:451-453
  V lg = c.buf(0), tg = c.buf(1), rl = c.buf(2), ls = c.buf(3), dl = c.buf(4);
  int r0 = c.i(5), r1 = c.i(6), Vn = c.i(7), ig = c.i(8), N = c.i(9); float sc = c.fl(10);
  need(Vn > 0 && ig == -1 && N > 0, "softmax_ce_fused: bad V/ignore/N");
  ce_fwd(c, lg, tg, rl, ls, r0, r1, Vn, ig);
  ce_bwd(lg, tg, ls, dl, r0, r1, Vn, ig, f32((double)f32(1.0 / N) * sc));
}
void adamw(V p, V g, V m, V v, V gs, V st, int e0, int e1, float lr, float b1, float b2, float eps, float wd, V sh = V()) {   // ref_gpt.py:457-471
  int t = st.i[0];
  if (t < 1) fail("adamw: step counter < 1");
  double gsc = gs.ok() ? (double)gs.f[0] : 1.0;
  float bc1 = f32(1.0 - (double)f32(std::pow((double)b1, (double)t))), bc2 = f32(1.0 - (double)f32(std::pow((double)b2, (double)t)));
  for (int i = e0; i < e1; ++i) {
    float gi = f32(g.f[i] * gsc);
    float mi = f32((double)f32((double)b1 * m.f[i]) + (double)f32((double)f32(1.0 - b1) * gi));
    float vi = f32((double)f32((double)b2 * v.f[i]) + (double)f32((double)f32((double)f32(1.0 - b2) * gi) * gi));
    m.f[i] = mi; v.f[i] = vi;
    float decay = f32((double)f32((double)lr * wd) * p.f[i]);
    float step = f32((double)f32((double)lr * (double)f32((double)mi / bc1)) / (double)f32((double)f32(std::sqrt((double)f32((double)vi / bc2))) + eps));
    p.f[i] = f32((double)f32((double)p.f[i] - decay) - step);
    if (sh.ok()) sh.f[i] = bf16r(p.f[i]);
  }
}
void op_adamw(const Ctx& c) { adamw(c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4, true), c.buf(5), c.i(6), c.i(7), c.fl(8), c.fl(9), c.fl(10), c.fl(11), c.fl(12)); }
void op_adamw_bf16(const Ctx& c) {   // this executor's op 305: adamw, then the bf16 copy of the new weight
  adamw(c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4, true), c.buf(5), c.i(6), c.i(7), c.fl(8), c.fl(9), c.fl(10), c.fl(11), c.fl(12), c.buf(13));
}
void op_adamw_lr(const Ctx& c) { V lr = c.buf(8); adamw(c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4, true), c.buf(5), c.i(6), c.i(7), lr.f[0], c.fl(9), c.fl(10), c.fl(11), c.fl(12)); }
void op_gradnorm_partial(const Ctx& c) { V g = c.buf(0), part = c.buf(1); double s = 0;
  for (int i = c.i(3); i < c.i(4); ++i) s += (double)g.f[i] * g.f[i];
  part.f[c.i(2)] = f32(s); }
void op_gradnorm_finish(const Ctx& c) {   // ref_gpt.py:478-482
  V part = c.buf(0), out = c.buf(2); int ns = c.i(1); float mx = c.fl(3);
  double s = 0; for (int i = 0; i < ns; ++i) s += part.f[i];
  float n = f32(std::sqrt(s));
  if (mx > 0) { float x = f32((double)mx / (double)f32((double)n + (double)f32(1e-6))); out.f[0] = x < 1.0f ? x : 1.0f; }
  else out.f[0] = 1.0f;
  out.f[1] = n;
}
// Philox-4x32-10 (Salmon et al. 2011), the sampling uniform of ref_gpt.py:486-498
void philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c[0], p1 = (uint64_t)0xCD9E8D57u * c[2];
    uint32_t n0 = (uint32_t)(p1 >> 32) ^ c[1] ^ k0, n1 = (uint32_t)p1, n2 = (uint32_t)(p0 >> 32) ^ c[3] ^ k1, n3 = (uint32_t)p0;
    c[0] = n0; c[1] = n1; c[2] = n2; c[3] = n3;
    k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
  }
}
double philox_uniform(int seed, int ctr, int row) {
  uint32_t c[4] = {(uint32_t)row, (uint32_t)ctr, 0, 0};
  philox(c, (uint32_t)seed, 0x9E3779B9u);
  return (double)(c[0] >> 8) * (1.0 / 16777216.0);
}
uint32_t order_key(float x) { uint32_t b; memcpy(&b, &x, 4); return b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u); }
int argmax_row(const float* row, int Vn) {
  double bv = -INFINITY; int bi = 0x7FFFFFFF;
  for (int j = 0; j < Vn; ++j) { double x = row[j]; if (x > bv || (x == bv && j < bi)) { bv = x; bi = j; } }
  return bi == 0x7FFFFFFF ? 0 : bi;
}
void op_sample(const Ctx& c) {   // ref_gpt.py:515-540
  V lg = c.buf(0), out = c.buf(1), ctr = c.buf(2, true);
  int r0 = c.i(3), r1 = c.i(4), Vn = c.i(5); float temp = c.fl(6); int topk = c.i(7), seed = c.i(8);
  int cv = ctr.ok() ? ctr.i[0] : 0;
  std::vector<uint32_t> keys(Vn); std::vector<double> w(Vn); std::vector<char> has(Vn);
  for (int r = r0; r < r1; ++r) {
    const float* row = lg.f + (long long)r * lg.cols;
    if (temp <= 0) { out.i[r] = argmax_row(row, Vn); continue; }
    double mx = -INFINITY; for (int j = 0; j < Vn; ++j) if (row[j] == row[j] && row[j] > mx) mx = row[j];
    uint32_t thr = 0;
    if (topk > 0 && topk < Vn) { for (int j = 0; j < Vn; ++j) keys[j] = order_key(row[j]); std::sort(keys.begin(), keys.end(), std::greater<uint32_t>()); thr = keys[topk - 1]; }
    for (int j = 0; j < Vn; ++j) { has[j] = row[j] == row[j] && order_key(row[j]) >= thr; w[j] = has[j] ? std::exp((double)f32((double)row[j] - mx) / temp) : 0.0; }
    double total = 0; for (int j = 0; j < Vn; ++j) total += has[j] ? w[j] : 0.0;
    double target = philox_uniform(seed, cv, r) * total, run = 0; int pick = -1, last = -1;
    for (int j = 0; j < Vn; ++j) if (has[j]) { run += w[j]; last = j; if (run > target) { pick = j; break; } }
    out.i[r] = pick >= 0 ? pick : std::max(last, 0);
  }
}
void op_argmax(const Ctx& c) { V lg = c.buf(0), out = c.buf(1); for (int r = c.i(2); r < c.i(3); ++r) out.i[r] = argmax_row(lg.f + (long long)r * lg.cols, c.i(4)); }
void op_select_window(const Ctx& c) {   // ref_gpt.py:543-548
  V src = c.buf(0), step = c.buf(1), dst = c.buf(2); int i0 = c.i(3), i1 = c.i(4), stride = c.i(5), off = c.i(6);
  long long base = (long long)step.i[0] * stride + off;
  if (base < 0 || base + i1 > src.n()) fail("select_window: window outside src");
  for (int i = i0; i < i1; ++i) { if (dst.i) dst.i[i] = src.i[base + i]; else dst.f[i] = src.f[base + i]; }
}
void op_gather_rows(const Ctx& c) { V src = c.buf(0), idx = c.buf(1), dst = c.buf(2); int d = c.i(5);
  for (int r = c.i(3); r < c.i(4); ++r) { int i = token(idx.i[r], src.rows); for (int k = 0; k < d; ++k) dst.f[(long long)r * dst.cols + k] = src.f[(long long)i * src.cols + k]; } }

// ------------------------------------------------------------------------------------------- extra ops (ref_extra.py)
double act_f(int kind, double x) { switch (kind) { case 0: return x > 0 ? x : 0.0; case 1: return silu(x); case 2: return std::tanh(x); default: return sig(x); } }
double act_d(int kind, double x) { switch (kind) { case 0: return x > 0 ? 1.0 : 0.0; case 1: return silu_d(x); case 2: { double t = std::tanh(x); return 1.0 - t * t; } default: return sig(x) * (1.0 - sig(x)); } }
void op_act_fwd(const Ctx& c) { V x = c.buf(0), o = c.buf(1); int kind = c.i(2); need(kind >= 0 && kind <= 3, "act: kind");
  for (int k = c.i(3); k < c.i(4); ++k) o.f[k] = f32(act_f(kind, x.f[k])); }
void op_act_bwd(const Ctx& c) { V x = c.buf(0), dy = c.buf(1), dx = c.buf(2); int kind = c.i(3), acc = c.i(6); need(kind >= 0 && kind <= 3, "act: kind");
  for (int k = c.i(4); k < c.i(5); ++k) { float v = f32((double)dy.f[k] * act_d(kind, x.f[k])); dx.f[k] = acc ? f32((double)dx.f[k] + v) : v; } }
void op_silu_mul_fwd(const Ctx& c) { V g = c.buf(0), u = c.buf(1), o = c.buf(2);
  for (int k = c.i(3); k < c.i(4); ++k) o.st(k, silu(g.f[k]) * u.f[k]); }
void op_silu_mul_bwd(const Ctx& c) { V g = c.buf(0), u = c.buf(1), dy = c.buf(2), dg = c.buf(3), du = c.buf(4); int acc = c.i(7);
  for (int k = c.i(5); k < c.i(6); ++k) {
    float vg = f32((double)dy.f[k] * (double)f32((double)u.f[k] * silu_d(g.f[k]))), vu = f32((double)dy.f[k] * silu(g.f[k]));
    dg.f[k] = acc ? f32((double)dg.f[k] + vg) : vg; du.f[k] = acc ? f32((double)du.f[k] + vu) : vu;
  } }
void op_softmax_rows_fwd(const Ctx& c) { V x = c.buf(0), o = c.buf(1); int d = c.i(4); float sc = c.fl(5); std::vector<double> e(d);
  for (int r = c.i(2); r < c.i(3); ++r) {
    double m = -INFINITY; for (int j = 0; j < d; ++j) { e[j] = x.at(r, j) * sc; if (j == 0 || e[j] > m) m = e[j]; }
    double z = 0; for (int j = 0; j < d; ++j) { e[j] = std::exp(e[j] - m); z += e[j]; }
    for (int j = 0; j < d; ++j) o.f[(long long)r * o.cols + j] = f32(e[j] / z);
  } }
void op_softmax_rows_bwd(const Ctx& c) { V p = c.buf(0), dp = c.buf(1), dx = c.buf(2); int d = c.i(5), acc = c.i(7); float sc = c.fl(6);
  for (int r = c.i(3); r < c.i(4); ++r) {
    double dot = 0; for (int j = 0; j < d; ++j) dot += p.at(r, j) * dp.at(r, j);
    for (int j = 0; j < d; ++j) { float v = f32(sc * p.at(r, j) * (dp.at(r, j) - dot)); long long o = (long long)r * dx.cols + j; dx.f[o] = acc ? f32((double)dx.f[o] + v) : v; }
  } }
void op_gather_rows_scaled(const Ctx& c) { V src = c.buf(0), idx = c.buf(1), sc = c.buf(2, true), dst = c.buf(3);
  int d = c.i(6), acc = c.i(7), i0 = c.i(8);
  for (int r = c.i(4); r < c.i(5); ++r) { int j = idx.i[i0 + r]; double s = sc.ok() ? (double)sc.f[i0 + r] : 1.0;
    for (int k = 0; k < d; ++k) { float v = (j >= 0 && j < src.rows) ? f32(s * src.at(j, k)) : 0.0f; long long o = (long long)r * dst.cols + k; dst.f[o] = acc ? f32((double)dst.f[o] + v) : v; } } }
void op_scatter_add_rows(const Ctx& c) { V src = c.buf(0), idx = c.buf(1), sc = c.buf(2, true), dst = c.buf(3);
  int N = c.i(4), d = c.i(7), acc = c.i(8), i0 = c.i(9); std::vector<float> a(d);
  for (int v = c.i(5); v < c.i(6); ++v) { std::fill(a.begin(), a.end(), 0.0f);
    for (int r = 0; r < N; ++r) if (idx.i[i0 + r] == v) { double s = sc.ok() ? (double)sc.f[i0 + r] : 1.0; for (int k = 0; k < d; ++k) a[k] = f32((double)a[k] + (double)f32(s * src.at(r, k))); }
    for (int k = 0; k < d; ++k) { long long o = (long long)v * dst.cols + k; dst.f[o] = acc ? f32((double)dst.f[o] + a[k]) : a[k]; } } }
void op_row_dot(const Ctx& c) { V A = c.buf(0), B = c.buf(1), idx = c.buf(2, true), out = c.buf(3); int d = c.i(6), acc = c.i(7), i0 = c.i(8);
  for (int r = c.i(4); r < c.i(5); ++r) { int j = idx.ok() ? idx.i[i0 + r] : r; float v = 0.0f;
    if (j >= 0 && j < A.rows) { double s = 0; for (int k = 0; k < d; ++k) s += A.at(j, k) * B.at(r, k); v = f32(s); }
    out.f[i0 + r] = acc ? f32((double)out.f[i0 + r] + v) : v; } }
void op_round_bf16(const Ctx& c) { V x = c.buf(0), o = c.buf(1); for (int k = c.i(2); k < c.i(3); ++k) o.f[k] = bf16r(x.f[k]); }
void op_matmul_tile_bf16(const Ctx& c) { mm_tile(c, true); }
void op_matmul_mma_bf16(const Ctx& c) {   // the 128x256 tile = eight 64x64 bf16 tiles (ref_extra.py:326-331)
  int32_t a[13]; memcpy(a, c.a, sizeof a);
  Ctx sub = c; sub.a = a;
  for (int dm : {0, 64}) for (int dn : {0, 64, 128, 192}) {
    a[6] = c.a[6] + dm; a[7] = c.a[7] + dn; a[11] = c.a[11] & ~(32 | 64);
    if (a[6] < c.a[8] && a[7] < c.a[9]) mm_tile(sub, true, 64);
  }
}
void op_matmul_mma_bf16_256(const Ctx& c) {   // this executor's op 304: op 122 with a 256x256 tile (sixteen 64x64 tiles)
  int32_t a[13]; memcpy(a, c.a, sizeof a);
  Ctx sub = c; sub.a = a;
  for (int dm = 0; dm < 256; dm += 64) for (int dn = 0; dn < 256; dn += 64) {
    a[6] = c.a[6] + dm; a[7] = c.a[7] + dn; a[11] = c.a[11] & ~(32 | 64);
    if (a[6] < c.a[8] && a[7] < c.a[9]) mm_tile(sub, true, 64);
  }
}
// This executor's op 302: op 122's 128x256 tile (flag 64: a 256x256 tile) over k in [k0, k0 + K), written to output
// row om0 + m; plain epilogue (alpha, optional accumulate).
void op_matmul_mma_bf16_kr(const Ctx& c) {
  V A = c.buf(0), B = c.buf(1), out = c.buf(2);
  int m0 = c.i(6), n0 = c.i(7), M = c.i(8), N = c.i(9), K = c.i(10), fl = c.i(11), k0 = c.i(13), om0 = c.i(14); float alpha = c.fl(12);
  need((fl & ~(1 | 2 | 4 | 32 | 64)) == 0 && c.a[3] == -1 && c.a[4] == -1 && c.a[5] == -1 && k0 >= 0 && om0 >= 0,
       "matmul_mma_bf16_kr: flags / epilogue / k0 / om0");
  int ta = fl & 1, tb = fl & 2, accum = fl & 4;
  auto opA = [&](int m, int k) -> float { return bf16r(ta ? A.f[(long long)k * A.cols + m] : A.f[(long long)m * A.cols + k]); };
  auto opB = [&](int n, int k) -> float { return bf16r(tb ? B.f[(long long)n * B.cols + k] : B.f[(long long)k * B.cols + n]); };
  const int m1 = std::min(m0 + (fl & 64 ? 256 : 128), M), n1 = std::min(n0 + 256, N);
  if (m0 >= m1 || n0 >= n1) return;
  std::vector<float> accv;
  tile_product(m0, m1, n0, n1, k0, K, opA, opB, accv);
  for (int m = m0; m < m1; ++m)
    for (int n = n0; n < n1; ++n) {
      float acc = accv[(size_t)(m - m0) * (n1 - n0) + (n - n0)];
      float v = f32((double)acc * alpha);
      long long o = (long long)(om0 + m) * out.cols + n;
      out.stf(o, accum ? f32((double)out.f[o] + v) : v);
    }
}
// This executor's op 303: out[r, c] = sum over s in order of part[s*M + r, c].
void op_matmul_mma_bf16_delta(const Ctx& c) {   // this executor's op 308: op 122's tile, then op 46 over the tile's rows and heads
  op_matmul_mma_bf16(c);
  V out = c.buf(2), o = c.buf(13), dl = c.buf(14);
  const int m0 = c.i(6), n0 = c.i(7), M = c.i(8), N = c.i(9), T = c.i(15), H = c.i(16), hd = c.i(17);
  for (int m = m0; m < std::min(m0 + 128, M); ++m)
    for (int h = n0 / hd; h < std::min(n0 + 256, N) / hd; ++h) {
      double a = 0; for (int cc = 0; cc < hd; ++cc) a += o.at(m, h * hd + cc) * out.at(m, h * hd + cc);
      dl.f[((long long)(m / T) * H + h) * T + m % T] = f32(a);
    }
}
void op_splitk_reduce(const Ctx& c) {
  V part = c.buf(0), out = c.buf(1); int M = c.i(2), N = c.i(3), S = c.i(4), r0 = c.i(5), r1 = c.i(6);
  need(M > 0 && N > 0 && S > 0 && 0 <= r0 && r0 <= r1 && r1 <= M, "splitk_reduce: args");
  for (int r = r0; r < r1; ++r)
    for (int col = 0; col < N; ++col) {
      float t = part.f[(long long)r * part.cols + col];
      for (int s = 1; s < S; ++s) t = f32((double)t + part.f[((long long)s * M + r) * part.cols + col]);
      out.stf((long long)r * out.cols + col, t);
    }
}
void op_lr_schedule(const Ctx& c) {   // ref_extra.py:339-345
  V st = c.buf(0), lr = c.buf(1); int kind = c.i(2); float base = c.fl(3); int wu = c.i(4), tot = c.i(5); float mr = c.fl(6);
  need(kind >= 0 && kind <= 2, "lr_schedule: kind");
  int t = st.i[0];
  double warm = (wu > 0 && t <= wu) ? (double)t / wu : 1.0;
  double prog = std::min(std::max((double)(t - wu) / std::max(tot - wu, 1), 0.0), 1.0);
  double f = kind == 0 ? 1.0 : kind == 1 ? mr + (1 - (double)mr) * 0.5 * (1 + std::cos(M_PI * prog)) : 1.0 - (1 - (double)mr) * prog;
  lr.f[0] = f32((double)base * warm * f);
}
void op_scale_flat(const Ctx& c) { V x = c.buf(0), o = c.buf(1); float al = c.fl(2); for (int k = c.i(3); k < c.i(4); ++k) o.f[k] = f32((double)al * x.f[k]); }
void op_add_rowtile(const Ctx& c) { V x = c.buf(0), pos = c.buf(1), o = c.buf(2); int T = c.i(5), d = c.i(6);
  for (int r = c.i(3); r < c.i(4); ++r) for (int k = 0; k < d; ++k) o.f[(long long)r * o.cols + k] = f32(x.at(r, k) + pos.at(pymod(r, T), k)); }
void op_matmul_tile_silu_mul(const Ctx& c) {   // ref_extra.py:372-379
  V A = c.buf(0), B = c.buf(1), out = c.buf(2), gate = c.buf(3), up = c.buf(4);
  int m0 = c.i(5), n0 = c.i(6), M = c.i(7), N = c.i(8), K = c.i(9), fl = c.i(10); float alpha = c.fl(11);
  need((fl & ~(19 | 96)) == 0 && !((fl & 32) && (fl & 64)), "matmul_tile_silu_mul: flags");
  int ta = fl & 1, tb = fl & 2, tm = tile_m(fl), tn = tile_n(fl);
  for (int m = m0; m < std::min(m0 + tm, M); ++m) for (int n = n0; n < std::min(n0 + tn, N); ++n) {
    float acc = 0;
    for (int k = 0; k < K; ++k) acc = f32((double)acc + (double)f32((double)(ta ? A.f[(long long)k * A.cols + m] : A.f[(long long)m * A.cols + k]) * (double)(tb ? B.f[(long long)n * B.cols + k] : B.f[(long long)k * B.cols + n])));
    up.f[(long long)m * up.cols + n] = f32((double)acc * alpha);
  }
  for (int m = m0; m < std::min(m0 + tm, M); ++m) for (int n = n0; n < std::min(n0 + tn, N); ++n)
    out.f[(long long)m * out.cols + n] = f32(silu(gate.at(m, n)) * up.at(m, n));
}
void op_matmul_tile_silu_mul_bwd(const Ctx& c) {   // ref_extra.py:382-390
  V A = c.buf(0), B = c.buf(1), gate = c.buf(2), up = c.buf(3), dg = c.buf(4), du = c.buf(5);
  int m0 = c.i(6), n0 = c.i(7), M = c.i(8), N = c.i(9), K = c.i(10), fl = c.i(11); float alpha = c.fl(12);
  need((fl & ~(19 | 96)) == 0 && !((fl & 32) && (fl & 64)), "matmul_tile_silu_mul_bwd: flags");
  int ta = fl & 1, tb = fl & 2, tm = tile_m(fl), tn = tile_n(fl);
  for (int m = m0; m < std::min(m0 + tm, M); ++m) for (int n = n0; n < std::min(n0 + tn, N); ++n) {
    float acc = 0;
    for (int k = 0; k < K; ++k) acc = f32((double)acc + (double)f32((double)(ta ? A.f[(long long)k * A.cols + m] : A.f[(long long)m * A.cols + k]) * (double)(tb ? B.f[(long long)n * B.cols + k] : B.f[(long long)k * B.cols + n])));
    dg.f[(long long)m * dg.cols + n] = f32((double)acc * alpha);
  }
  for (int m = m0; m < std::min(m0 + tm, M); ++m) for (int n = n0; n < std::min(n0 + tn, N); ++n) {
    long long o = (long long)m * dg.cols + n; double dh = dg.f[o];
    dg.f[o] = f32(dh * (double)f32(up.at(m, n) * silu_d(gate.at(m, n))));
    du.f[(long long)m * du.cols + n] = f32(dh * silu(gate.at(m, n)));
  }
}
void op_gemv_bf16(const Ctx& c) {   // ref_extra.py:399-418
  V x = c.buf(0), x2 = c.buf(1, true), g = c.buf(2, true), w = c.buf(3), out = c.buf(4), res = c.buf(5, true);
  int n0 = c.i(6), n1 = c.i(7), K = c.i(8), pro = c.i(9); float eps = c.fl(10);
  need(0 <= n0 && n0 < n1 && K > 0 && K % 8 == 0 && pro >= 0 && pro <= 2, "gemv_bf16: bad range, K or pro");
  std::vector<double> v(K);
  if (pro == 1) {
    double ss = 0; for (int k = 0; k < K; ++k) ss += (double)x.f[k] * x.f[k];
    float rs = f32(1.0 / std::sqrt(ss / K + eps));
    for (int k = 0; k < K; ++k) v[k] = bf16r(f32((double)x.f[k] * rs * g.f[k]));
  } else if (pro == 2) { for (int k = 0; k < K; ++k) v[k] = bf16r(f32(silu(x.f[k]) * x2.f[k])); }
  else for (int k = 0; k < K; ++k) v[k] = bf16r(x.f[k]);
  for (int n = n0; n < n1; ++n) {
    double y = 0; for (int k = 0; k < K; ++k) y += v[k] * w.at(n, k);
    out.st(n, (double)f32(y + (res.ok() ? (double)res.f[n] : 0.0)));
  }
}
const float ATTN_EMPTY_M = -3.4028234663852886e38f;
void rope_pair(double x1, double x2, long long p0, int i, int hd, float th, float& y1, float& y2) {
  float ang = rope_ang(p0, i, hd, th);
  double s = f32(std::sin((double)ang)), co = f32(std::cos((double)ang));
  y1 = f32(x1 * co - x2 * s); y2 = f32(x1 * s + x2 * co);
}
// Per-head RMSNorm of one head slice, as op_head_rmsnorm computes it: f32(f32(x * rs) * gamma), rs from a double sum.
static void head_norm(std::vector<double>& x, const V& g, float eps) {
  const int hd = (int)x.size();
  double ss = 0; for (double v : x) ss += (double)f32(v) * f32(v);
  const float rs = f32(1.0 / std::sqrt(ss / hd + eps));
  for (int k = 0; k < hd; ++k) x[k] = f32((double)f32(f32(x[k]) * rs) * g.f[k]);
}
// attn_decode_part; with qg / kg (op 306) the query heads and the new key are head-normalised first.
static void attn_decode_part_impl(const Ctx& c, V qg, V kg, float eps) {   // ref_extra.py:441-479
  V q = c.buf(0), kc = c.buf(1), vc = c.buf(2), lens = c.buf(3), part = c.buf(4), kn = c.buf(5, true), vn = c.buf(6, true);
  int bb = c.i(7), kvh = c.i(8), s = c.i(9), S = c.i(10), H = c.i(11), Hkv = c.i(12), hd = c.i(13), Tmax = c.i(14);
  float sc = c.fl(15), th = c.fl(16); int fl = c.i(17);
  need(fl == 0 || fl == 1 || fl == 3, "attn_decode_part: flags");
  int n = lens.i[bb] + 1;
  if (lens.i[bb] < 0 || n > Tmax) fail("attn_decode_part: length exceeds Tmax");
  int chunk = (n + S - 1) / S, j0 = s * chunk, j1 = std::min(n, s * chunk + chunk);
  int G = H / Hkv, half = hd / 2; long long base = ((long long)bb * Hkv + kvh) * Tmax, p0 = lens.i[bb];
  if ((fl & 1) && j0 <= n - 1 && n - 1 < j1) {
    long long row = (base + n - 1) * kc.cols;
    std::vector<double> kv(hd);
    for (int cc = 0; cc < hd; ++cc) kv[cc] = kn.at(bb, kvh * hd + cc);
    if (kg.ok()) head_norm(kv, kg, eps);
    for (int i = 0; i < half; ++i) { float y1, y2; rope_pair(kv[i], kv[i + half], p0, i, hd, th, y1, y2); kc.stf(row + i, y1); kc.stf(row + i + half, y2); }
    long long vrow = (base + n - 1) * vc.cols;
    for (int cc = 0; cc < hd; ++cc) vc.stf(vrow + cc, (float)vn.at(bb, kvh * hd + cc));
  }
  std::vector<double> qv(hd), sc_(std::max(0, j1 - j0)), p(std::max(0, j1 - j0));
  for (int g = 0; g < G; ++g) {
    int h = kvh * G + g;
    for (int cc = 0; cc < hd; ++cc) qv[cc] = q.at(bb, h * hd + cc);
    if (qg.ok()) head_norm(qv, qg, eps);
    if (fl & 1) for (int i = 0; i < half; ++i) { float y1, y2; rope_pair(qv[i], qv[i + half], p0, i, hd, th, y1, y2);
      if (fl & 2) { y1 = bf16r(y1); y2 = bf16r(y2); } qv[i] = y1; qv[i + half] = y2; }
    long long row = (((long long)bb * S + s) * H + h) * part.cols;
    if (j1 <= j0) { for (int cc = 0; cc < hd; ++cc) part.f[row + cc] = 0.0f; part.f[row + hd] = ATTN_EMPTY_M; part.f[row + hd + 1] = 0.0f; continue; }
    for (int j = j0; j < j1; ++j) { double a = 0; for (int cc = 0; cc < hd; ++cc) a += qv[cc] * kc.at(base + j, cc); sc_[j - j0] = a * sc; }
    double m = sc_[0]; for (int j = 1; j < j1 - j0; ++j) if (sc_[j] > m) m = sc_[j];
    double l = 0; for (int j = 0; j < j1 - j0; ++j) { p[j] = std::exp(sc_[j] - m); }
    for (int cc = 0; cc < hd; ++cc) { double a = 0; for (int j = 0; j < j1 - j0; ++j) a += p[j] * vc.at(base + j0 + j, cc); part.f[row + cc] = f32(a); }
    for (int j = 0; j < j1 - j0; ++j) l += p[j];
    part.f[row + hd] = f32(m); part.f[row + hd + 1] = f32(l);
  }
}
void op_attn_decode_part(const Ctx& c) { attn_decode_part_impl(c, V(), V(), 0.f); }
void op_attn_decode_part_qkn(const Ctx& c) {   // this executor's op 306: op 135 after op 300's per-head norm of q and the new key
  need(c.i(17) == 1 || c.i(17) == 3, "attn_decode_part_qkn: flags");
  attn_decode_part_impl(c, c.buf(18), c.buf(19), c.fl(20));
}
static void merge_heads(const V& part, const V& o, int bb, int h0, int h1, int S, int H, int hd) {   // ref_extra.py:487-498
  for (int h = h0; h < h1; ++h) {
    std::vector<long long> live;
    for (int s = 0; s < S; ++s) { long long r = (((long long)bb * S + s) * H + h) * part.cols; if (part.f[r + hd + 1] > 0.0f) live.push_back(r); }
    if (live.empty()) fail("attn_decode_merge: no live split");
    double M = part.f[live[0] + hd]; for (long long r : live) if (part.f[r + hd] > M) M = part.f[r + hd];
    std::vector<double> e; double L = 0;
    for (long long r : live) e.push_back(std::exp(part.f[r + hd] - M));
    for (size_t i = 0; i < live.size(); ++i) L += e[i] * part.f[live[i] + hd + 1];
    for (int cc = 0; cc < hd; ++cc) { double a = 0; for (size_t i = 0; i < live.size(); ++i) a += e[i] * part.f[live[i] + cc];
      o.stf((long long)bb * o.cols + h * hd + cc, f32(a / L)); }
  }
}
void op_attn_decode_merge(const Ctx& c) {
  merge_heads(c.buf(0), c.buf(1), c.i(2), c.i(3), c.i(4), c.i(5), c.i(6), c.i(7));
}
// This executor's op 310: op 306, then the split that completes last among the S splits of (b, kvh) (counted in cnt,
// under a lock when the VM runs tasks on several threads) merges that kv head's G query heads as op 136 and resets
// the count.
void op_attn_decode_part_merge(const Ctx& c) {
  op_attn_decode_part_qkn(c);
  static std::mutex mu;
  const int bb = c.i(7), kvh = c.i(8), S = c.i(10), H = c.i(11), Hkv = c.i(12), hd = c.i(13);
  V cnt = c.buf(22);
  bool last;
  {
    std::lock_guard<std::mutex> lk(mu);
    int32_t& k = cnt.i[(long long)bb * Hkv + kvh];
    if (k < 0 || k >= S) fail("attn_decode_part_merge: split count out of range");
    last = ++k == S;
    if (last) k = 0;
  }
  if (last) merge_heads(c.buf(4), c.buf(21), bb, kvh * (H / Hkv), (kvh + 1) * (H / Hkv), S, H, hd);
}
void op_head_rmsnorm(const Ctx& c) {   // this executor's own op: RMSNorm over each head slice (no reference counterpart)
  V x = c.buf(0), g = c.buf(1), o = c.buf(2); int r0 = c.i(3), r1 = c.i(4), H = c.i(5), hd = c.i(6); float eps = c.fl(7);
  for (int r = r0; r < r1; ++r) for (int h = 0; h < H; ++h) {
    double ss = 0; for (int k = 0; k < hd; ++k) { double v = x.at(r, h * hd + k); ss += v * v; }
    float rs = f32(1.0 / std::sqrt(ss / hd + eps));
    for (int k = 0; k < hd; ++k) { long long i = (long long)r * o.cols + h * hd + k; o.st(i, (double)f32(x.at(r, h * hd + k) * rs) * g.f[k]); }
  }
}

void op_gemv_bf16_rows(const Ctx& c) {   // this executor's op 301: gemv_bf16 for M rows sharing one weight stream
  V x = c.buf(0), x2 = c.buf(1, true), g = c.buf(2, true), w = c.buf(3), out = c.buf(4), res = c.buf(5, true);
  int n0 = c.i(6), n1 = c.i(7), K = c.i(8), M = c.i(9), pro = c.i(10); float eps = c.fl(11);
  need(0 <= n0 && n0 < n1 && K > 0 && K % 64 == 0 && M >= 1 && M <= 16 && pro >= 0 && pro <= 2, "gemv_bf16_rows: bad args");
  std::vector<double> v(K);
  for (int m = 0; m < M; ++m) {
    if (pro == 1) {
      double ss = 0; for (int k = 0; k < K; ++k) ss += x.at(m, k) * x.at(m, k);
      float rs = f32(1.0 / std::sqrt(ss / K + eps));
      for (int k = 0; k < K; ++k) v[k] = bf16r(f32(x.at(m, k) * rs * g.f[k]));
    } else if (pro == 2) { for (int k = 0; k < K; ++k) v[k] = bf16r(f32(silu(x.at(m, k)) * x2.at(m, k))); }
    else for (int k = 0; k < K; ++k) v[k] = bf16r((float)x.at(m, k));
    for (int n = n0; n < n1; ++n) {
      double y = 0; for (int k = 0; k < K; ++k) y += v[k] * w.at(n, k);
      out.st((long long)m * out.cols + n, (double)f32(y + (res.ok() ? res.at(m, n) : 0.0)));
    }
  }
}

// This executor's op 311: op 301 with pro 1 on the rows of wg and of wu (the two sums of a row n rounded to f32 as
// op 301 stores them), then out = silu(g) * u rounded once as out stores it (the down projection's pro 2 prologue /
// op 98 on the stored gate and up values).
void op_gemv_swiglu(const Ctx& c) {
  V x = c.buf(0), g = c.buf(1), wg = c.buf(2), wu = c.buf(3), out = c.buf(4);
  int n0 = c.i(5), n1 = c.i(6), K = c.i(7), M = c.i(8); float eps = c.fl(9);
  need(0 <= n0 && n0 < n1 && K > 0 && K % 256 == 0 && M >= 1 && M <= 16, "gemv_swiglu: bad args");
  std::vector<double> v(K);
  for (int m = 0; m < M; ++m) {
    double ss = 0; for (int k = 0; k < K; ++k) ss += x.at(m, k) * x.at(m, k);
    float rs = f32(1.0 / std::sqrt(ss / K + eps));
    for (int k = 0; k < K; ++k) v[k] = bf16r(f32(x.at(m, k) * rs * g.f[k]));
    for (int n = n0; n < n1; ++n) {
      double yg = 0, yu = 0;
      for (int k = 0; k < K; ++k) { yg += v[k] * wg.at(n, k); yu += v[k] * wu.at(n, k); }
      const float gf = f32(yg), uf = f32(yu);
      out.st((long long)m * out.cols + n, silu(gf) * uf);
    }
  }
}

typedef void (*OpFn)(const Ctx&);
struct OpEnt { int id; OpFn fn; };
const OpEnt kOps[] = {
  {0, [](const Ctx&) {}}, {1, op_copy}, {2, op_add}, {3, op_scale}, {4, op_relu}, {5, op_sgd}, {6, op_predict}, {7, op_mse_grad},
  {8, op_matmul}, {9, op_fill}, {10, [](const Ctx&) {}},
  {32, op_embedding_fwd}, {33, op_embedding_bwd}, {34, op_matmul_tile}, {35, norm_fwd<false>}, {36, norm_fwd<true>},
  {37, op_layernorm_bwd_dx}, {38, op_rmsnorm_bwd_dx}, {309, op_layernorm_bwd_dx_res}, {39, op_norm_bwd_params}, {40, op_gelu_fwd}, {41, op_gelu_bwd},
  {42, op_residual_add}, {123, op_sgd_range}, {43, op_rope<1>}, {44, op_rope<-1>}, {45, op_attn_fwd}, {46, op_attn_bwd_delta},
  {47, op_attn_bwd_dq}, {48, op_attn_bwd_dkv}, {49, op_kv_append}, {50, op_attn_decode}, {51, op_softmax_ce_fwd},
  {52, op_softmax_ce_reduce}, {53, op_softmax_ce_bwd}, {127, op_softmax_ce_fused}, {54, op_adamw}, {55, op_gradnorm_partial},
  {56, op_gradnorm_finish}, {57, op_sample}, {58, op_argmax}, {59, op_zero_buf}, {60, op_counter_inc}, {61, op_colsum},
  {62, op_select_window}, {63, op_gather_rows}, {126, op_round_tf32},
  {96, op_act_fwd}, {97, op_act_bwd}, {98, op_silu_mul_fwd}, {99, op_silu_mul_bwd}, {100, op_softmax_rows_fwd},
  {101, op_softmax_rows_bwd}, {102, op_gather_rows_scaled}, {103, op_scatter_add_rows}, {104, op_row_dot},
  {113, op_round_bf16}, {114, op_matmul_tile_bf16}, {122, op_matmul_mma_bf16}, {134, op_gemv_bf16},
  {135, op_attn_decode_part}, {136, op_attn_decode_merge}, {115, op_adamw_lr}, {116, op_lr_schedule}, {117, op_scale_flat},
  {118, op_add_rowtile}, {120, op_matmul_tile_silu_mul}, {121, op_matmul_tile_silu_mul_bwd}, {300, op_head_rmsnorm}, {301, op_gemv_bf16_rows}, {311, op_gemv_swiglu}, {302, op_matmul_mma_bf16_kr}, {303, op_splitk_reduce}, {304, op_matmul_mma_bf16_256}, {305, op_adamw_bf16}, {306, op_attn_decode_part_qkn}, {310, op_attn_decode_part_merge}, {308, op_matmul_mma_bf16_delta},
};
OpFn find_op(int id) { for (const OpEnt& e : kOps) if (e.id == id) return e.fn; return nullptr; }

}  // namespace

extern "C" {

typedef struct OrcBuf { void* p; int32_t rows, cols, dtype; } OrcBuf;
typedef struct OrcRead { int32_t task, var, policy, version; } OrcRead;   // policy 0 exact, 1 at_least

// Runs one bundle to completion in the reference VM's deterministic order. Returns 0 on success, else 1 with `err` set.
// order[i] = the i-th task run; observed[r] = version of reads[r].var when reads[r].task started.
int orc_run(const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs,
            OrcBuf* bufs, int nbufs, int32_t* versions, int nvars, const OrcRead* reads, int nreads, int32_t* observed,
            int32_t* order, int limit, float* dur_us, char* err, int errlen) {
  std::vector<int> indeg(ntasks);
  std::vector<std::vector<int>> reads_of(ntasks);
  for (int r = 0; r < nreads; ++r) if (reads[r].task >= 0 && reads[r].task < ntasks) reads_of[reads[r].task].push_back(r);
  std::set<std::pair<long long, int>> ready;                // key (-priority, index): begin() = deterministic pick
  std::vector<std::vector<int>> parked(nvars > 0 ? nvars : 1);   // released but waiting on a version
  auto key = [&](int t) { return std::make_pair(-(long long)tasks[t].priority, t); };
  auto release = [&](int t) {
    const MvmTaskDesc& d = tasks[t];
    if (d.wait_var >= 0 && versions[d.wait_var] < d.wait_ver) parked[d.wait_var].push_back(t);
    else ready.insert(key(t));
  };
  int cur = -1, done = 0;
  try {
    for (int t = 0; t < ntasks; ++t) {
      const MvmTaskDesc& d = tasks[t];
      if (d.succ_off < 0 || d.succ_cnt < 0 || d.succ_off + d.succ_cnt > nedges || d.args_off < 0 || d.args_off + d.args_words > nargs)
        fail("task descriptor out of range");
      if (d.wait_var >= nvars || d.pub_var >= nvars) fail("version variable out of range");
      indeg[t] = d.indegree;
    }
    for (int t = 0; t < ntasks; ++t) if (indeg[t] == 0) release(t);
    while (done < ntasks && (limit <= 0 || done < limit)) {
      if (ready.empty()) fail("deadlock: no runnable task");
      cur = ready.begin()->second;
      ready.erase(ready.begin());
      const MvmTaskDesc& d = tasks[cur];
      for (int r : reads_of[cur]) {
        int seen = versions[reads[r].var];
        observed[r] = seen;
        if (reads[r].policy == 0 ? seen != reads[r].version : seen < reads[r].version) fail("read version violated");
      }
      OpFn fn = find_op(d.op_id);
      if (!fn) fail("operator not supported by the oracle");
      Ctx c{(OBuf*)bufs, nbufs, args + d.args_off};
      auto t0 = std::chrono::steady_clock::now();
      fn(c);
      if (dur_us) dur_us[cur] = std::chrono::duration<float, std::micro>(std::chrono::steady_clock::now() - t0).count();
      order[done++] = cur;
      if (d.pub_var >= 0) {
        if (versions[d.pub_var] + 1 != d.pub_ver) fail("publish order broken");
        versions[d.pub_var] = d.pub_ver;
        std::vector<int> w; w.swap(parked[d.pub_var]);
        for (int t : w) release(t);
      }
      for (int k = 0; k < d.succ_cnt; ++k) { int s = succ[d.succ_off + k]; if (--indeg[s] == 0) release(s); }
    }
  } catch (const Fail& f) {
    snprintf(err, errlen, "task %d: %s", cur, f.msg.c_str());
    return 1;
  }
  return 0;
}

// The same VM with `threads` workers (the reference's Runtime(workers=N), workload_vm.py:46): every ready task may run
// beside the others, since a valid graph orders every conflicting pair of accesses by an edge or a version wait. Picks
// follow the same (priority, index) rule under one lock; operators run outside it. Results do not depend on the
// interleaving (each output has one writer per phase); `order` records completion order and `observed` the version
// each read saw at its task's start. threads <= 1 runs orc_run.
int orc_run_mt(const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs,
               OrcBuf* bufs, int nbufs, int32_t* versions, int nvars, const OrcRead* reads, int nreads, int32_t* observed,
               int32_t* order, float* dur_us, int threads, char* err, int errlen) {
  if (threads <= 1) return orc_run(tasks, ntasks, succ, nedges, args, nargs, bufs, nbufs, versions, nvars, reads, nreads, observed, order, 0, dur_us, err, errlen);
  std::vector<int> indeg(ntasks);
  std::vector<std::vector<int>> reads_of(ntasks);
  for (int r = 0; r < nreads; ++r) if (reads[r].task >= 0 && reads[r].task < ntasks) reads_of[reads[r].task].push_back(r);
  std::set<std::pair<long long, int>> ready;
  std::vector<std::vector<int>> parked(nvars > 0 ? nvars : 1);
  auto key = [&](int t) { return std::make_pair(-(long long)tasks[t].priority, t); };
  auto release = [&](int t) {
    const MvmTaskDesc& d = tasks[t];
    if (d.wait_var >= 0 && versions[d.wait_var] < d.wait_ver) parked[d.wait_var].push_back(t);
    else ready.insert(key(t));
  };
  for (int t = 0; t < ntasks; ++t) {
    const MvmTaskDesc& d = tasks[t];
    if (d.succ_off < 0 || d.succ_cnt < 0 || d.succ_off + d.succ_cnt > nedges || d.args_off < 0 || d.args_off + d.args_words > nargs ||
        d.wait_var >= nvars || d.pub_var >= nvars) { snprintf(err, errlen, "task %d: descriptor out of range", t); return 1; }
    indeg[t] = d.indegree;
  }
  for (int t = 0; t < ntasks; ++t) if (indeg[t] == 0) release(t);
  std::mutex mu;
  std::condition_variable cv;
  int done = 0, running = 0;
  bool failed = false;
  std::string why;
  auto worker = [&]() {
    std::unique_lock<std::mutex> lk(mu);
    for (;;) {
      cv.wait(lk, [&] { return failed || done == ntasks || !ready.empty() || running == 0; });
      if (failed || done == ntasks) return;
      if (ready.empty()) { failed = true; why = "deadlock: no runnable task"; cv.notify_all(); return; }
      const int cur = ready.begin()->second;
      ready.erase(ready.begin());
      const MvmTaskDesc& d = tasks[cur];
      for (int r : reads_of[cur]) {
        int seen = versions[reads[r].var];
        observed[r] = seen;
        if (reads[r].policy == 0 ? seen != reads[r].version : seen < reads[r].version) { failed = true; why = "task " + std::to_string(cur) + ": read version violated"; }
      }
      OpFn fn = find_op(d.op_id);
      if (!fn) { failed = true; why = "task " + std::to_string(cur) + ": operator not supported by the oracle"; }
      if (failed) { cv.notify_all(); return; }
      ++running;
      lk.unlock();
      std::string msg;
      auto t0 = std::chrono::steady_clock::now();
      try { Ctx c{(OBuf*)bufs, nbufs, args + d.args_off}; fn(c); } catch (const Fail& f) { msg = f.msg; }
      const float us = std::chrono::duration<float, std::micro>(std::chrono::steady_clock::now() - t0).count();
      lk.lock();
      --running;
      if (dur_us) dur_us[cur] = us;
      if (!msg.empty()) { failed = true; why = "task " + std::to_string(cur) + ": " + msg; cv.notify_all(); return; }
      order[done++] = cur;
      if (d.pub_var >= 0) {
        if (versions[d.pub_var] + 1 != d.pub_ver) { failed = true; why = "task " + std::to_string(cur) + ": publish order broken"; cv.notify_all(); return; }
        versions[d.pub_var] = d.pub_ver;
        std::vector<int> w; w.swap(parked[d.pub_var]);
        for (int t : w) release(t);
      }
      for (int k = 0; k < d.succ_cnt; ++k) { int sx = succ[d.succ_off + k]; if (--indeg[sx] == 0) release(sx); }
      cv.notify_all();
    }
  };
  std::vector<std::thread> pool;
  for (int i = 0; i < threads; ++i) pool.emplace_back(worker);
  for (auto& th : pool) th.join();
  if (failed) { snprintf(err, errlen, "%s", why.c_str()); return 1; }
  return 0;
}

// Single-op entry for tests: runs one operator on explicit buffers.
int orc_op(int op_id, const int32_t* args, OrcBuf* bufs, int nbufs, char* err, int errlen) {
  OpFn fn = find_op(op_id);
  if (!fn) { snprintf(err, errlen, "unknown op %d", op_id); return 1; }
  try { Ctx c{(OBuf*)bufs, nbufs, args}; fn(c); }
  catch (const Fail& f) { snprintf(err, errlen, "%s", f.msg.c_str()); return 1; }
  return 0;
}

// SplitMix64 seeded value (runtime/initgen.py:49-58), for the tests' known-answer check.
// The same values rounded to bf16 (nearest even on the bits; the executor's bf16 seeded weights), as float.
void orc_seeded(float* out, long long n, unsigned long long seed, int draws, float bias, float coef);
void orc_seeded_bf16(float* out, long long n, unsigned long long seed, int draws, float bias, float coef) {
  orc_seeded(out, n, seed, draws, bias, coef);
  auto rnd = [&](long long i0, long long i1) { for (long long i = i0; i < i1; ++i) out[i] = bf16r(out[i]); };
  const int nt = n >= (1ll << 22) ? (int)std::min<unsigned>(16u, std::max(1u, std::thread::hardware_concurrency())) : 1;
  std::vector<std::thread> pool;
  for (int t = 0; t < nt; ++t) pool.emplace_back(rnd, n * t / nt, n * (t + 1) / nt);
  for (auto& th : pool) th.join();
}
void orc_seeded(float* out, long long n, unsigned long long seed, int draws, float bias, float coef) {
  auto u = [&](unsigned long long j) {
    unsigned long long z = seed + (j + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull; z = (z ^ (z >> 27)) * 0x94D049BB133111EBull; z ^= z >> 31;
    return (float)(z >> 40) * (1.0f / 16777216.0f);
  };
  auto fill = [&](long long i0, long long i1) {
    for (long long i = i0; i < i1; ++i) {
      float acc = draws == 1 ? u(i) : (u(i * 4) + u(i * 4 + 1)) + (u(i * 4 + 2) + u(i * 4 + 3));
      out[i] = (acc - bias) * coef;
    }
  };
  // counter-based: every element is a function of its index alone, so large fills split over threads
  const int nt = n >= (1ll << 22) ? (int)std::min<unsigned>(16u, std::max(1u, std::thread::hardware_concurrency())) : 1;
  std::vector<std::thread> pool;
  for (int t = 0; t < nt; ++t) pool.emplace_back(fill, n * t / nt, n * (t + 1) / nt);
  for (auto& th : pool) th.join();
}

}  // extern "C"
