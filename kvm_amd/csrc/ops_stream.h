// Bandwidth-bound operators in streaming form: 16-byte loads, several loads in flight per lane, rows held in registers
// between the passes that need them, and reductions in a fixed order (so results are reproducible run to run).
// Each op_*_fast returns false when the shape or alignment is outside what it handles; the caller then runs the
// element-wise body in ops_basic.h (same semantics).
#pragma once
#include "common.h"
#include "ops_basic.h"
#include "ops_gemm.h"

namespace kvm {

// 8 consecutive elements at flat offset o (o % 8 == 0) of a bf16 or f32 view, widened to f32.
__device__ __forceinline__ void ld8(const View& X, long long o, float (&v)[8]) {
  if (X.dtype == 2) {
    const u16x8_t h = *(const GLOBAL u16x8_t*)(X.h() + o);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = bf2f(h[i]);
  } else {
    const f32x4n a = *(const GLOBAL f32x4n*)(X.f() + o), b = *(const GLOBAL f32x4n*)(X.f() + o + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}
__device__ __forceinline__ void st8(const View& X, long long o, const float (&v)[8]) {
  if (X.dtype == 2) {
    if (X.n() * 2 < 0x7fffffffll) {
      const u32x4_t w = {(uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16), (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16),
                         (uint32_t)f2bf(v[4]) | ((uint32_t)f2bf(v[5]) << 16), (uint32_t)f2bf(v[6]) | ((uint32_t)f2bf(v[7]) << 16)};
      stwt_buf(wt_rsrc(X.p, X.n() * 2), (int)o * 2, __builtin_bit_cast(f32x4n, w));
    } else {
      stwt_bf4(X.h() + o, v[0], v[1], v[2], v[3]);
      stwt_bf4(X.h() + o + 4, v[4], v[5], v[6], v[7]);
    }
  } else if (X.n() * 4 < 0x7fffffffll) {
    const __amdgpu_buffer_rsrc_t r = wt_rsrc(X.p, X.n() * 4);
    stwt_buf(r, (int)o * 4, f32x4n{v[0], v[1], v[2], v[3]});
    stwt_buf(r, (int)o * 4 + 16, f32x4n{v[4], v[5], v[6], v[7]});
  } else {
    stwt_f4(X.f() + o, f32x4n{v[0], v[1], v[2], v[3]});
    stwt_f4(X.f() + o + 4, f32x4n{v[4], v[5], v[6], v[7]});
  }
}
// ld8 with the storage type as a template parameter (no dtype test between a batch of loads).
template <bool BF> __device__ __forceinline__ void ld8t(const View& X, long long o, float (&v)[8]) {
  if constexpr (BF) {
    const u16x8_t h = *(const GLOBAL u16x8_t*)(X.h() + o);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = bf2f(h[i]);
  } else {
    const f32x4n a = *(const GLOBAL f32x4n*)(X.f() + o), b = *(const GLOBAL f32x4n*)(X.f() + o + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[i + 4] = b[i]; }
  }
}
__device__ __forceinline__ bool vec8_ok(const View& X) { return X.dtype != 1 && (X.cols % 8) == 0; }
__device__ __forceinline__ bool vec4_ok(const View& X) { return X.dtype != 1 && (X.cols % 4) == 0; }
// Within reach of 32-bit byte offsets (buffer loads).
__device__ __forceinline__ bool off32_ok(const View& X) { return (long long)X.rows * X.cols * 4 < 0x7fffffffll; }

// Embedding lookup (registry op 32): out[r] = wte[ids[r]] (+ wpe[r % T]), 8-column vectors, each wave's RPW rows
// and both tables loaded before any is used; storage types as template parameters (no dtype test per vector).
template <bool BW, bool BP, int NV>
__device__ __forceinline__ void emb_rows(const Ctx& c, const View& ids, const View& wte, const View& wpe, const View& out, int r0, int r1, int T, int d) {
  constexpr int RPW = NV == 1 ? 4 : NV == 2 ? 2 : 1;
  const bool hp = wpe.ok();
  for (int rb = r0 + wave() * RPW; rb < r1; rb += KVM_WAVES * RPW) {
    int id[RPW];
    float a[RPW][NV][8], b[RPW][NV][8];
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int r = min(rb + q, r1 - 1);
      const int t = ids.i()[r];
      id[q] = t;
      const int tc = (t < 0 || t >= wte.rows) ? 0 : t;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int col = min(8 * (lane() + 64 * i), d - 8);
        ld8t<BW>(wte, (long long)tc * wte.cols + col, a[q][i]);
        if (hp) ld8t<BP>(wpe, (long long)(r % T) * wpe.cols + col, b[q][i]);
      }
    }
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int r = rb + q;
      if (r >= r1) break;
      const bool bad = id[q] < 0 || id[q] >= wte.rows;
      if (bad && lane() == 0) c.fail(KVM_ERR_OP_TOKEN, r, id[q]);
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int col = 8 * (lane() + 64 * i);
        if (col >= d) break;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = bad ? 0.f : (hp ? a[q][i][e] + b[q][i][e] : a[q][i][e]);
        st8(out, (long long)r * out.cols + col, v);
      }
    }
  }
}
__device__ __noinline__ bool op_embedding_fwd_fast(const Ctx& c) {
  const View ids = c.buf(0), wte = c.buf(1), wpe = c.buf(2), out = c.buf(3);
  const int r0 = c.i(4), r1 = c.i(5), T = c.i(6), d = c.i(7);
  if (d % 8 || d > 4096 || !vec8_ok(wte) || !vec8_ok(out) || (wpe.ok() && (!vec8_ok(wpe) || wpe.dtype != wte.dtype)) || T <= 0) return false;
  const bool bw = wte.dtype == 2;
  const int nv = (d + 511) / 512;
  if (nv > 4) {   // rows up to 4096 wide (a decode step's token rows): one row per wave, 8 vectors per lane in flight
    if (bw) emb_rows<true, true, 8>(c, ids, wte, wpe, out, r0, r1, T, d); else emb_rows<false, false, 8>(c, ids, wte, wpe, out, r0, r1, T, d);
    return true;
  }
  if (nv == 1) { if (bw) emb_rows<true, true, 1>(c, ids, wte, wpe, out, r0, r1, T, d); else emb_rows<false, false, 1>(c, ids, wte, wpe, out, r0, r1, T, d); }
  else if (nv == 2) { if (bw) emb_rows<true, true, 2>(c, ids, wte, wpe, out, r0, r1, T, d); else emb_rows<false, false, 2>(c, ids, wte, wpe, out, r0, r1, T, d); }
  else { if (bw) emb_rows<true, true, 4>(c, ids, wte, wpe, out, r0, r1, T, d); else emb_rows<false, false, 4>(c, ids, wte, wpe, out, r0, r1, T, d); }
  return true;
}

// ---------------------------------------------------------------------------------------------- flat elementwise ops
// out[i] = f(in_0[i], .., in_{NIN-1}[i]) over flat [e0, e1) for f32 views: groups of 4 elements, NB groups per thread
// loaded before any is used (a load / store round trip per element otherwise serialises the loop: write-through
// stores and loads share one counter), elements outside the 16-byte grid one by one. In-place use (an input is the
// output) is fine: each element is read and written by the same thread.
template <int NIN, class F>
__device__ __forceinline__ void flat_map(const View (&in)[NIN], const View& out, long long e0, long long e1, F f) {
  constexpr int NB = 8;
  const long long a0 = min((e0 + 3) & ~3ll, e1), a1 = max(a0, e1 & ~3ll);
  auto one = [&](long long i) {
    float x[NIN];
#pragma unroll
    for (int k = 0; k < NIN; ++k) x[k] = in[k].f()[i];
    stwt32(out.f() + i, f(x));
  };
  for (long long i = e0 + tid(); i < a0; i += KVM_THREADS) one(i);
  for (long long i = a1 + tid(); i < e1; i += KVM_THREADS) one(i);
  const long long q1 = a1 / 4;
  const bool bo = out.n() * 4 < 0x7fffffffll;
  const __amdgpu_buffer_rsrc_t ro = wt_rsrc(out.p, bo ? out.n() * 4 : 0);
  for (long long q = a0 / 4 + tid(); q < q1; q += NB * KVM_THREADS) {
    f32x4n v[NB][NIN];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const long long qq = min(q + (long long)u * KVM_THREADS, q1 - 1);
#pragma unroll
      for (int k = 0; k < NIN; ++k) v[u][k] = ((const GLOBAL f32x4n*)in[k].f())[qq];
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const long long qq = q + (long long)u * KVM_THREADS;
      if (qq >= q1) break;
      f32x4n r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float x[NIN];
#pragma unroll
        for (int k = 0; k < NIN; ++k) x[k] = v[u][k][j];
        r[j] = f(x);
      }
      if (bo) stwt_buf(ro, (int)(qq * 16), r);
      else stwt_f4(out.f() + 4 * qq, r);
    }
  }
}
__device__ __forceinline__ bool all_f32(const View& a, const View& b = View{nullptr, 0, 0, 0}, const View& c = View{nullptr, 0, 0, 0}) {
  return a.dtype == 0 && (!b.ok() || b.dtype == 0) && (!c.ok() || c.dtype == 0);
}
__device__ __noinline__ bool op_act_fwd_fast(const Ctx& c) {
  const View x = c.buf(0), o = c.buf(1);
  const int kind = c.i(2);
  if (!all_f32(x, o)) return false;
  const View in[1] = {x};
  flat_map(in, o, c.i(3), c.i(4), [kind](const float (&v)[1]) { return act_f(kind, v[0]); });
  return true;
}
__device__ __noinline__ bool op_act_bwd_fast(const Ctx& c) {
  const View x = c.buf(0), dy = c.buf(1), dx = c.buf(2);
  const int kind = c.i(3), acc = c.i(6);
  if (!all_f32(x, dy, dx)) return false;
  if (acc) {
    const View in[3] = {x, dy, dx};
    flat_map(in, dx, c.i(4), c.i(5), [kind](const float (&v)[3]) { return v[2] + v[1] * act_d(kind, v[0]); });
  } else {
    const View in[2] = {x, dy};
    flat_map(in, dx, c.i(4), c.i(5), [kind](const float (&v)[2]) { return v[1] * act_d(kind, v[0]); });
  }
  return true;
}
__device__ __noinline__ bool op_scale_flat_fast(const Ctx& c) {
  const View x = c.buf(0), o = c.buf(1);
  const float al = c.f(2);
  if (!all_f32(x, o)) return false;
  const View in[1] = {x};
  flat_map(in, o, c.i(3), c.i(4), [al](const float (&v)[1]) { return al * v[0]; });
  return true;
}
__device__ __noinline__ bool op_relu_fast(const Ctx& c) {
  const View x = c.buf(0), o = c.buf(1);
  if (!all_f32(x, o)) return false;
  const View in[1] = {x};
  flat_map(in, o, 0, c.i(2), [](const float (&v)[1]) { return v[0] > 0.f ? v[0] : 0.f; });
  return true;
}
__device__ __noinline__ bool op_add_fast(const Ctx& c) {
  const View a = c.buf(0), b = c.buf(1), o = c.buf(2);
  if (!all_f32(a, b, o)) return false;
  const View in[2] = {a, b};
  flat_map(in, o, 0, c.i(3), [](const float (&v)[2]) { return v[0] + v[1]; });
  return true;
}
__device__ __noinline__ bool op_scale_fast(const Ctx& c) {
  const View x = c.buf(0), o = c.buf(1);
  const float al = c.f(2);
  if (!all_f32(x, o)) return false;
  const View in[1] = {x};
  flat_map(in, o, 0, c.i(3), [al](const float (&v)[1]) { return v[0] * al; });
  return true;
}

// silu(gate) * up over [e0, e1) (registry op 104): groups of 8 elements, four groups in flight per thread.
__device__ __noinline__ bool op_silu_mul_fwd_fast(const Ctx& c) {
  const View g = c.buf(0), u = c.buf(1), o = c.buf(2);
  const long long e0 = c.i(3), e1 = c.i(4);
  if (!vec8_ok(g) || !vec8_ok(u) || !vec8_ok(o) || (e0 % 8) || (e1 % 8)) return false;
  const long long n8 = (e1 - e0) / 8;
  for (long long q0 = tid(); q0 < n8; q0 += 4 * KVM_THREADS) {
    float gv[4][8], uv[4][8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const long long q = min(q0 + k * KVM_THREADS, n8 - 1);
      ld8(g, e0 + 8 * q, gv[k]); ld8(u, e0 + 8 * q, uv[k]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (q0 + k * KVM_THREADS >= n8) break;
      float r[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = silu_f(gv[k][i]) * uv[k][i];
      st8(o, e0 + 8 * (q0 + k * KVM_THREADS), r);
    }
  }
  return true;
}

// ---------------------------------------------------------------------------------------------- column reductions
// Column sums over rows [0, R) for 64-column chunks: 8 lanes cover 64 columns of one row (8 columns each), so 32 row
// slots run side by side; slot s takes rows s, s+32, ... (ascending, CR_UNROLL rows in flight) and the 32 slot partials
// are added in slot order through LDS.
// The CR_UNROLL rows of a step are loaded (at clamped row indices, no branch between the loads) before any is
// used; rows past R then add nothing. The storage type is a template parameter, so there is no dtype test per row.
constexpr int CR_UNROLL = 8;
// Column sums of x over rows [0, R) at columns col .. col+7 for row slot `slot` (rows slot, slot+32, ...).
template <bool BF> __device__ __forceinline__ void col_sum8(const View& x, int R, int col, int slot, float (&a)[8]) {
  for (int r0 = slot; r0 < R; r0 += 32 * CR_UNROLL) {
    float v[CR_UNROLL][8];
#pragma unroll
    for (int u = 0; u < CR_UNROLL; ++u) ld8t<BF>(x, (long long)min(r0 + 32 * u, R - 1) * x.cols + col, v[u]);
#pragma unroll
    for (int u = 0; u < CR_UNROLL; ++u) {
      const bool in = r0 + 32 * u < R;
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] += in ? v[u][i] : 0.f;
    }
  }
}
// dgamma / dbeta partials: sum_r dy (x - mean_r) rstd_r and sum_r dy, same row order.
template <bool BX, bool BY> __device__ __forceinline__ void col_norm8(const View& x, const View& dy, const View& mean, const View& rstd, int R,
                                                                     int col, int slot, float (&sg)[8], float (&sb)[8]) {
  const bool hm = mean.ok();
  for (int r0 = slot; r0 < R; r0 += 32 * CR_UNROLL) {
    float xv[CR_UNROLL][8], gv[CR_UNROLL][8], mu[CR_UNROLL], rs[CR_UNROLL];
#pragma unroll
    for (int u = 0; u < CR_UNROLL; ++u) {
      const int r = min(r0 + 32 * u, R - 1);
      ld8t<BX>(x, (long long)r * x.cols + col, xv[u]);
      ld8t<BY>(dy, (long long)r * dy.cols + col, gv[u]);
      mu[u] = hm ? mean.f()[r] : 0.f;
      rs[u] = rstd.f()[r];
    }
#pragma unroll
    for (int u = 0; u < CR_UNROLL; ++u) {
      const bool in = r0 + 32 * u < R;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        sg[i] += in ? gv[u][i] * (xv[u][i] - mu[u]) * rs[u] : 0.f;
        sb[i] += in ? gv[u][i] : 0.f;
      }
    }
  }
}
// Adds the 32 slot partials (LDS, [32][64] per quantity) in slot order; thread t < W gets column t's total.
__device__ __forceinline__ float slot_total(const LDS float* part, int t) {
  float s = 0.f;
#pragma unroll 8
  for (int k = 0; k < 32; ++k) s += part[k * 64 + t];
  return s;
}

__device__ __noinline__ bool op_colsum_fast(const Ctx& c) {
  const View x = c.buf(0), out = c.buf(1);
  const int R = c.i(2), c0 = c.i(3), c1 = c.i(4), acc = c.i(5);
  if (!vec8_ok(x) || (c0 % 8) || ((c1 - c0) % 8)) return false;
  LDS float* part = (LDS float*)c.smem;
  for (int cb = c0; cb < c1; cb += 64) {
    const int W = min(64, c1 - cb);
    const int vi = tid() & 7, slot = tid() >> 3;
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (vi * 8 < W) { if (x.dtype == 2) col_sum8<true>(x, R, cb + vi * 8, slot, a); else col_sum8<false>(x, R, cb + vi * 8, slot, a); }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) part[slot * 64 + vi * 8 + i] = a[i];
    __syncthreads();
    if (tid() < W) {
      const float s = slot_total(part, tid());
      stwt32(out.f() + (cb + tid()), acc ? out.f()[cb + tid()] + s : s);
    }
  }
  return true;
}

// dgamma = sum_r dy * (x - mean) * rstd, dbeta = sum_r dy (registry op 39).
__device__ __noinline__ bool op_norm_bwd_params_fast(const Ctx& c) {
  const View x = c.buf(0), dy = c.buf(1), mean = c.buf(2), rstd = c.buf(3), dg = c.buf(4), db = c.buf(5);
  const int R = c.i(6), c0 = c.i(8), c1 = c.i(9), acc = c.i(10);
  if (!vec8_ok(x) || !vec8_ok(dy) || (c0 % 8) || ((c1 - c0) % 8)) return false;
  LDS float* part = (LDS float*)c.smem;
  for (int cb = c0; cb < c1; cb += 64) {
    const int W = min(64, c1 - cb);
    const int vi = tid() & 7, slot = tid() >> 3;
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, b[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (vi * 8 < W) {
      const int col = cb + vi * 8;
      if (x.dtype == 2) { if (dy.dtype == 2) col_norm8<true, true>(x, dy, mean, rstd, R, col, slot, a, b); else col_norm8<true, false>(x, dy, mean, rstd, R, col, slot, a, b); }
      else { if (dy.dtype == 2) col_norm8<false, true>(x, dy, mean, rstd, R, col, slot, a, b); else col_norm8<false, false>(x, dy, mean, rstd, R, col, slot, a, b); }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 8; ++i) { part[slot * 64 + vi * 8 + i] = a[i]; part[2048 + slot * 64 + vi * 8 + i] = b[i]; }
    __syncthreads();
    if (tid() < W) {
      const int j = cb + tid();
      const float sg = slot_total(part, tid());
      stwt32(dg.f() + j, acc ? dg.f()[j] + sg : sg);
      if (db.ok()) { const float sb = slot_total(part + 2048, tid()); stwt32(db.f() + j, acc ? db.f()[j] + sb : sb); }
    }
  }
  return true;
}

// ---------------------------------------------------------------------------------------------- row normalisation
// One wave per row, the row in registers (NV 4-element vectors per lane, d = 256 * NV), rows of a wave loaded before
// any is reduced (RPW rows at a time) so their loads overlap.
template <int NV, bool RMS> __device__ __noinline__ void norm_fwd_rows(const View& x_, const View& g_, const View& be_, const View& out_,
                                                          const View& mean_, const View& rstd_, int r0, int r1, int d, float eps) {
  // Register copies of the views, and all of a wave's row loads issued together through branch-free buffer loads
  // (rows past r1 re-read the last row): by-reference views and dtype branches would each add a full memory wait.
  const View x = uniform_view(x_), g = uniform_view(g_), be = uniform_view(be_), out = uniform_view(out_), mean = uniform_view(mean_),
             rstd = uniform_view(rstd_);
  // Rows per wave whose loads are in flight together: at d 768 (NV 3) six, so that a task's ~21 rows need one round
  // of loads (GPT-162M 8.90 -> 8.83 ms against four; eight measured 8.86).
  constexpr int RPW = NV >= 8 ? 1 : NV >= 4 ? 2 : NV == 3 ? 6 : 4;
  Ld4 lx;
  lx.init(x);
  float gv[NV][4], bv[NV][4];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const f32x4n t = *(const GLOBAL f32x4n*)(g.f() + 4 * (lane() + 64 * i));
    gv[i][0] = t.x; gv[i][1] = t.y; gv[i][2] = t.z; gv[i][3] = t.w;
    const f32x4n u = RMS ? f32x4n{0.f, 0.f, 0.f, 0.f} : *(const GLOBAL f32x4n*)(be.f() + 4 * (lane() + 64 * i));
    bv[i][0] = u.x; bv[i][1] = u.y; bv[i][2] = u.z; bv[i][3] = u.w;
  }
  for (int rb = r0 + wave() * RPW; rb < r1; rb += KVM_WAVES * RPW) {
    u32x4_t raw[RPW][NV];
#pragma unroll
    for (int q = 0; q < RPW; ++q)
#pragma unroll
      for (int i = 0; i < NV; ++i) raw[q][i] = lx.raw(min(rb + q, r1 - 1) * x.cols + 4 * (lane() + 64 * i));
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int r = rb + q;
      f32x4n v[NV];
#pragma unroll
      for (int i = 0; i < NV; ++i) v[i] = lx.cvt(raw[q][i]);
      float mu = 0.f;
      if (!RMS) {
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
        mu = wave_sum(s) / (float)d;
      }
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const f32x4n t = v[i] - mu;
        ss += (t.x * t.x + t.y * t.y) + (t.z * t.z + t.w * t.w);
      }
      const float rs = 1.f / sqrtf(wave_sum(ss) / (float)d + eps);
      if (r < r1) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          f32x4n o;
          o.x = (v[i].x - mu) * rs * gv[i][0] + bv[i][0]; o.y = (v[i].y - mu) * rs * gv[i][1] + bv[i][1];
          o.z = (v[i].z - mu) * rs * gv[i][2] + bv[i][2]; o.w = (v[i].w - mu) * rs * gv[i][3] + bv[i][3];
          st4(out, (long long)r * out.cols + 4 * (lane() + 64 * i), o);
        }
        if (lane() == 0) { stwt32(rstd.f() + r, rs); if (!RMS) stwt32(mean.f() + r, mu); }
      }
    }
  }
}
template <bool RMS> __device__ __noinline__ bool op_norm_fwd_fast(const Ctx& c) {
  int k = 0; View x = c.buf(k++), g = c.buf(k++), be; if (!RMS) be = c.buf(k++);
  View out = c.buf(k++), mean; if (!RMS) mean = c.buf(k++);
  View rstd = c.buf(k++);
  const int r0 = c.i(k), r1 = c.i(k + 1), d = c.i(k + 2); const float eps = c.f(k + 3);
  if (d % 256 || d > 4096 || !vec4_ok(x) || !vec4_ok(out) || g.dtype != 0 || (!RMS && be.dtype != 0) || !off32_ok(x)) return false;
  switch (d / 256) {
    case 1: norm_fwd_rows<1, RMS>(x, g, be, out, mean, rstd, r0, r1, d, eps); break;
    case 2: norm_fwd_rows<2, RMS>(x, g, be, out, mean, rstd, r0, r1, d, eps); break;
    case 3: norm_fwd_rows<3, RMS>(x, g, be, out, mean, rstd, r0, r1, d, eps); break;
    case 4: norm_fwd_rows<4, RMS>(x, g, be, out, mean, rstd, r0, r1, d, eps); break;
    case 8: norm_fwd_rows<8, RMS>(x, g, be, out, mean, rstd, r0, r1, d, eps); break;
    case 16: norm_fwd_rows<16, RMS>(x, g, be, out, mean, rstd, r0, r1, d, eps); break;
    default: return false;
  }
  return true;
}

// dx = rstd * (dy*g - mean(dy*g) - xhat * mean(dy*g*xhat)) (+ dx when acc) (registry ops 37, 38).
// src: the accumulated term (dx itself for op 37 with acc, the residual gradient for op 309); unused when acc is 0.
template <int NV, bool RMS> __device__ __noinline__ void norm_bwd_rows(const View& x_, const View& dy_, const View& g_, const View& mean_,
                                                          const View& rstd_, const View& dx_, const View& src_, int r0, int r1, int d, int acc) {
  // As norm_fwd_rows: register copies of the views; x, dy, the accumulated dx and the row statistics of all of a
  // wave's rows are loaded together before any of them is used.
  const View x = uniform_view(x_), dy = uniform_view(dy_), g = uniform_view(g_), mean = uniform_view(mean_), rstd = uniform_view(rstd_),
             dx = uniform_view(dx_), src = uniform_view(src_);
  constexpr int RPW = NV >= 8 ? 1 : NV >= 4 ? 2 : 4;
  Ld4 lx, ly, ld;
  lx.init(x); ly.init(dy); ld.init(src, acc != 0);
  float gv[NV][4];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const f32x4n t = *(const GLOBAL f32x4n*)(g.f() + 4 * (lane() + 64 * i));
    gv[i][0] = t.x; gv[i][1] = t.y; gv[i][2] = t.z; gv[i][3] = t.w;
  }
  for (int rb = r0 + wave() * RPW; rb < r1; rb += KVM_WAVES * RPW) {
    u32x4_t rx[RPW][NV], ry[RPW][NV], rd[RPW][NV];
    float mu[RPW], rs[RPW];
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int rr = min(rb + q, r1 - 1);
      mu[q] = RMS ? 0.f : mean.f()[rr];
      rs[q] = rstd.f()[rr];
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        rx[q][i] = lx.raw(rr * x.cols + 4 * (lane() + 64 * i));
        ry[q][i] = ly.raw(rr * dy.cols + 4 * (lane() + 64 * i));
        rd[q][i] = ld.raw(rr * src.cols + 4 * (lane() + 64 * i));
      }
    }
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
      const int r = rb + q;
      float s1 = 0.f, s2 = 0.f;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const f32x4n xv = lx.cvt(rx[q][i]), gy = ly.cvt(ry[q][i]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float gs = gy[e] * gv[i][e];
          s1 += gs; s2 += gs * (xv[e] - mu[q]) * rs[q];
        }
      }
      s1 = RMS ? 0.f : wave_sum(s1) / (float)d;
      s2 = wave_sum(s2) / (float)d;
      if (r < r1) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          const f32x4n xv = lx.cvt(rx[q][i]), gy = ly.cvt(ry[q][i]);
          f32x4n res;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float gs = gy[e] * gv[i][e], xh = (xv[e] - mu[q]) * rs[q];
            res[e] = rs[q] * (gs - s1 - xh * s2);
          }
          res += ld.cvt(rd[q][i]);                  // zero unless accumulating
          st4(dx, (long long)r * dx.cols + 4 * (lane() + 64 * i), res);
        }
      }
    }
  }
}
template <bool RMS> __device__ bool norm_bwd_dispatch(const View& x, const View& dy, const View& g, const View& mean, const View& rstd,
                                                     const View& dx, const View& src, int r0, int r1, int d, int acc) {
  if (d % 256 || d > 4096 || !vec4_ok(x) || !vec4_ok(dy) || !vec4_ok(dx) || (acc && !vec4_ok(src)) || g.dtype != 0 || !off32_ok(x) ||
      !off32_ok(dy) || !off32_ok(dx) || (acc && !off32_ok(src))) return false;
  switch (d / 256) {
    case 1: norm_bwd_rows<1, RMS>(x, dy, g, mean, rstd, dx, src, r0, r1, d, acc); break;
    case 2: norm_bwd_rows<2, RMS>(x, dy, g, mean, rstd, dx, src, r0, r1, d, acc); break;
    case 3: norm_bwd_rows<3, RMS>(x, dy, g, mean, rstd, dx, src, r0, r1, d, acc); break;
    case 4: norm_bwd_rows<4, RMS>(x, dy, g, mean, rstd, dx, src, r0, r1, d, acc); break;
    case 8: norm_bwd_rows<8, RMS>(x, dy, g, mean, rstd, dx, src, r0, r1, d, acc); break;
    case 16: norm_bwd_rows<16, RMS>(x, dy, g, mean, rstd, dx, src, r0, r1, d, acc); break;
    default: return false;
  }
  return true;
}
// Op 309: dx = res + the LayerNorm input gradient.
__device__ __noinline__ bool op_norm_bwd_dx_res_fast(const Ctx& c) {
  return norm_bwd_dispatch<false>(c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4), c.buf(5), c.buf(6), c.i(7), c.i(8), c.i(9), 1);
}
template <bool RMS> __device__ __noinline__ bool op_norm_bwd_dx_fast(const Ctx& c) {
  int k = 0; View x = c.buf(k++), dy = c.buf(k++), g = c.buf(k++), mean; if (!RMS) mean = c.buf(k++);
  View rstd = c.buf(k++), dx = c.buf(k++);
  return norm_bwd_dispatch<RMS>(x, dy, g, mean, rstd, dx, dx, c.i(k), c.i(k + 1), c.i(k + 2), c.i(k + 3));
}

// ---------------------------------------------------------------------------------------------- cross entropy
// One wave per row: pass 1 streams the logits in 8-element vectors (4 in flight per lane) with a per-lane online
// max / sum, combined across the wave; pass 2 writes dlogits = (softmax - onehot) * f. Same results as ce_rows up to
// fp32 reassociation.
constexpr float LOG2E = 1.4426950408889634f, LN2 = 0.6931471805599453f;
// Block-per-row form for bf16 logits: the whole row (V <= 2048 * NR) is loaded into registers with every load in
// flight at once (thread t holds the 8-element vectors t, t + 256, ...), the row max and the exp-sum are reduced over
// the block in a fixed order (lanes by xor steps, then the four waves in order), and dlogits is written from the same
// registers, so each row is read from memory once. The exponentials are the hardware exp2 (arguments are <= 0, so
// only results below the normal range, probabilities under 2^-126, can differ from exp2f).
__device__ __forceinline__ float bfl(unsigned short h) { return __uint_as_float((unsigned)h << 16); }
template <typename F> __device__ __forceinline__ float block_reduce(LDS float* red, float v, F op) {
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o, 64));
  __syncthreads();                                   // the previous use of red is done
  if (lane() == 0) red[wave()] = v;
  __syncthreads();
  return op(op(red[0], red[1]), op(red[2], red[3]));
}
template <int NR>
__device__ __noinline__ void ce_rows_block(const Ctx& c, const View& lg_, const View& tg_, const View& rl_, const View& ls_, const View& dl_, int r0,
                                           int r1, int V, int ignore, float f, bool fwd, bool bwd) {
  // Register copies: fields of by-reference views would be re-read from memory with a full vmcnt wait each time,
  // which also waits for every store in flight.
  const View lg = uniform_view(lg_), tg = uniform_view(tg_), rl = uniform_view(rl_), ls = uniform_view(ls_), dl = uniform_view(dl_);
  LDS float* red = (LDS float*)c.smem;
  // Rows pipelined when the row fits in LDS: after its reductions each thread parks its own vectors of row r in LDS
  // (read back only by the same thread, so no barrier), the loads of row r + 1 go into the registers, and dlogits of
  // row r is written from LDS while they are in flight.
  constexpr bool PIPE = 64 + NR * 256 * 16 <= KVM_LDS_BYTES;
  LDS u16x8_t* park = (LDS u16x8_t*)(c.smem + 64);
  const int nv = V / 8, t8 = tid();
  u16x8_t v[NR];
  auto load_row = [&](int r) {
    const GLOBAL u16x8_t* row = (const GLOBAL u16x8_t*)(lg.h() + (long long)r * lg.cols);
#pragma unroll
    for (int u = 0; u < NR; ++u) v[u] = row[min(t8 + 256 * u, nv - 1)];         // unconditional: all in flight
  };
  auto write_grad = [&](int r, int t, bool ign, float lse, auto get) {
    if (ign) {                                       // ignored row: zeros (a uniform branch, outside the element loop)
      const long long ob = (long long)r * dl.cols;
      const float z[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int j = t8; j < nv; j += 256) st8(dl, ob + 8 * j, z);
      return;
    }
    const long long ob = (long long)r * dl.cols;
    // softmax * f as one exponential: exp2(x log2 e - (lse log2 e - log2 f)); the target's -f is applied by the one
    // lane holding it.
    if (!(f > 0.f)) {                                // other scales: (softmax - onehot) * f as written
      const float l2 = lse * LOG2E;
#pragma unroll
      for (int u = 0; u < NR; ++u) {
        const int j = t8 + 256 * u;
        if (j < nv) {
          const u16x8_t x = get(u);
          float o[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = (__builtin_amdgcn_exp2f(bfl(x[i]) * LOG2E - l2) - (8 * j + i == t ? 1.f : 0.f)) * f;
          st8(dl, ob + 8 * j, o);
        }
      }
      return;
    }
    const float l2 = lse * LOG2E - log2f(f);
#pragma unroll
    for (int u = 0; u < NR; ++u) {
      const int j = t8 + 256 * u;
      if (j < nv) {
        const u16x8_t x = get(u);
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = __builtin_amdgcn_exp2f(bfl(x[i]) * LOG2E - l2);
        if (j == (t >> 3))
#pragma unroll
          for (int i = 0; i < 8; ++i) if (i == (t & 7)) o[i] -= f;
        st8(dl, ob + 8 * j, o);
      }
    }
  };
  if (r0 < r1) load_row(r0);
  for (int r = r0; r < r1; ++r) {
    const int t = __builtin_amdgcn_readfirstlane(tg.i()[r]);   // uniform: tests on it are scalar branches
    const bool ign = t == ignore, bad = !ign && (t < 0 || t >= V);
    if (bad && tid() == 0) c.fail(KVM_ERR_OP_TOKEN, r, t);
    float lse = 0.f;
    if (fwd && !ign && !bad) {
      float m = -INFINITY;
#pragma unroll
      for (int u = 0; u < NR; ++u)
        if (t8 + 256 * u < nv)
#pragma unroll
          for (int i = 0; i < 8; ++i) m = fmaxf(m, bfl(v[u][i]));
      m = block_reduce(red, m, [](float a, float b) { return fmaxf(a, b); });
      const float ml2 = m * LOG2E;
      float s = 0.f;
#pragma unroll
      for (int u = 0; u < NR; ++u)
        if (t8 + 256 * u < nv)
#pragma unroll
          for (int i = 0; i < 8; ++i) s += __builtin_amdgcn_exp2f(bfl(v[u][i]) * LOG2E - ml2);
      s = block_reduce(red, s, [](float a, float b) { return a + b; });
      lse = (ml2 + log2f(s)) * LN2;
      if (tid() == 0) stwt32(ls.f() + r, lse);
      if (t8 == (t >> 3) % 256) {                    // the thread holding the target logit (element t % 8 of vector t / 8)
        float xt = 0.f;
#pragma unroll
        for (int u = 0; u < NR; ++u)
          if (u == (t >> 3) / 256)
#pragma unroll
            for (int i = 0; i < 8; ++i) if (i == (t & 7)) xt = bfl(v[u][i]);
        stwt32(rl.f() + r, lse - xt);
      }
    } else if (fwd && ign) {
      if (tid() == 0) { stwt32(ls.f() + r, 0.f); stwt32(rl.f() + r, 0.f); }
    } else if (!fwd && !bad) {
      lse = ls.f()[r];
    }
    // lse is uniform; taking it into a scalar register here completes its load (bwd-only form) before the next
    // row's loads are issued, so the gradient pass below waits for none of them.
    lse = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(lse)));
    const bool grad = bwd && !bad;
    if constexpr (PIPE) {
      if (grad)
#pragma unroll
        for (int u = 0; u < NR; ++u) park[u * 256 + t8] = v[u];
      if (r + 1 < r1) load_row(r + 1);
      if (grad) write_grad(r, t, ign, lse, [&](int u) { return park[u * 256 + t8]; });
    } else {
      if (grad) write_grad(r, t, ign, lse, [&](int u) { return v[u]; });
      if (r + 1 < r1) load_row(r + 1);
    }
  }
}

__device__ __noinline__ bool ce_rows_fast(const Ctx& c, View lg, View tg, View rl, View ls, View dl, int r0, int r1, int V, int ignore, float f, bool fwd, bool bwd) {
  if (!vec8_ok(lg) || (V % 8) || (bwd && !vec8_ok(dl))) return false;
  const int nv = V / 8;
  if (lg.dtype == 2 && nv <= 256 * 32) {
    const int nr = (nv + 255) / 256;
    if (nr <= 4) ce_rows_block<4>(c, lg, tg, rl, ls, dl, r0, r1, V, ignore, f, fwd, bwd);
    else if (nr <= 8) ce_rows_block<8>(c, lg, tg, rl, ls, dl, r0, r1, V, ignore, f, fwd, bwd);
    else if (nr <= 16) ce_rows_block<16>(c, lg, tg, rl, ls, dl, r0, r1, V, ignore, f, fwd, bwd);
    else if (nr <= 25) ce_rows_block<25>(c, lg, tg, rl, ls, dl, r0, r1, V, ignore, f, fwd, bwd);
    else ce_rows_block<32>(c, lg, tg, rl, ls, dl, r0, r1, V, ignore, f, fwd, bwd);
    return true;
  }
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    const int t = tg.i()[r];
    const bool ign = t == ignore;
    if (!ign && (t < 0 || t >= V)) { if (lane() == 0) c.fail(KVM_ERR_OP_TOKEN, r, t); continue; }
    const long long base = (long long)r * lg.cols;
    float lse;
    if (fwd) {
      if (ign) { if (lane() == 0) { stwt32(rl.f() + r, 0.f); stwt32(ls.f() + r, 0.f); } lse = 0.f; }
      else {
        float m = -INFINITY, s = 0.f;            // log2 domain
        for (int j0 = lane(); j0 < nv; j0 += 64 * 4) {
          float v[4][8];
#pragma unroll
          for (int u = 0; u < 4; ++u) if (j0 + 64 * u < nv) ld8(lg, base + 8 * (j0 + 64 * u), v[u]);
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (j0 + 64 * u >= nv) break;
            float bm = v[u][0];
#pragma unroll
            for (int i = 1; i < 8; ++i) bm = fmaxf(bm, v[u][i]);
            const float nm = fmaxf(m, bm * LOG2E);
            float a = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) a += exp2f(v[u][i] * LOG2E - nm);
            s = s * exp2f(m - nm) + a;
            m = nm;
          }
        }
        for (int o = 32; o > 0; o >>= 1) {
          const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64), nm = fmaxf(m, m2);
          s = (nm == -INFINITY) ? 0.f : s * exp2f(m - nm) + s2 * exp2f(m2 - nm);
          m = nm;
        }
        lse = (m + log2f(s)) * LN2;
        if (lane() == 0) { stwt32(ls.f() + r, lse); stwt32(rl.f() + r, lse - lg.at(r, t)); }
      }
    } else lse = ls.f()[r];
    if (bwd) {
      const long long ob = (long long)r * dl.cols;
      const float l2 = lse * LOG2E;
      for (int j0 = lane(); j0 < nv; j0 += 64 * 4) {
        float v[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) if (j0 + 64 * u < nv && !ign) ld8(lg, base + 8 * (j0 + 64 * u), v[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = j0 + 64 * u;
          if (j >= nv) break;
          float o[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = ign ? 0.f : (exp2f(v[u][i] * LOG2E - l2) - (8 * j + i == t ? 1.f : 0.f)) * f;
          st8(dl, ob + 8 * j, o);
        }
      }
    }
  }
  return true;
}

// ---------------------------------------------------------------------------------------------- flat streams
// f32 <-> bf16 storage conversion / copy over [e0, e1) (registry op 113): aligned 8-element vectors in the middle.
__device__ __noinline__ bool op_round_bf16_fast(const Ctx& c) {
  const View x = c.buf(0), o = c.buf(1);
  const long long e0 = c.i(2), e1 = c.i(3);
  if (x.dtype == 1 || o.dtype == 1) return false;
  const long long a0 = min(e1, (e0 + 7) & ~7ll), a1 = max(a0, e1 & ~7ll);
  auto one = [&](long long k) { const float v = x.ld(k); if (o.dtype == 2) stwt16(o.h() + k, f2bf(v)); else stwt32(o.f() + k, x.dtype == 2 ? v : round_bf(v)); };
  for (long long k = e0 + tid(); k < a0; k += KVM_THREADS) one(k);
  for (long long k = a1 + tid(); k < e1; k += KVM_THREADS) one(k);
  const long long n8 = (a1 - a0) / 8;
  for (long long q0 = tid(); q0 < n8; q0 += 4 * KVM_THREADS) {
    float v[4][8];
#pragma unroll
    for (int u = 0; u < 4; ++u) if (q0 + u * KVM_THREADS < n8) ld8(x, a0 + 8 * (q0 + u * KVM_THREADS), v[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long q = q0 + u * KVM_THREADS;
      if (q >= n8) break;
      if (o.dtype == 0 && x.dtype == 0)
#pragma unroll
        for (int i = 0; i < 8; ++i) v[u][i] = round_bf(v[u][i]);
      st8(o, a0 + 8 * q, v[u]);
    }
  }
  return true;
}

// Sum of squares of g[e0, e1) in double (registry op 55), 4 vectors in flight per lane.
__device__ __noinline__ bool op_gradnorm_partial_fast(const Ctx& c) {
  const View g = c.buf(0), part = c.buf(1);
  const long long e0 = c.i(3), e1 = c.i(4);
  if (g.dtype != 0) return false;
  __shared__ double red[KVM_WAVES];
  const long long a0 = min(e1, (e0 + 3) & ~3ll), a1 = max(a0, e1 & ~3ll);
  double s = 0.0;
  for (long long k = e0 + tid(); k < a0; k += KVM_THREADS) { const double v = g.f()[k]; s += v * v; }
  for (long long k = a1 + tid(); k < e1; k += KVM_THREADS) { const double v = g.f()[k]; s += v * v; }
  const long long n4 = (a1 - a0) / 4;
  const GLOBAL f32x4n* p = (const GLOBAL f32x4n*)(g.f() + a0);
  double t[4] = {0.0, 0.0, 0.0, 0.0};
  for (long long q0 = tid(); q0 < n4; q0 += 4 * KVM_THREADS) {
    f32x4n v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) if (q0 + u * KVM_THREADS < n4) v[u] = p[q0 + u * KVM_THREADS];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (q0 + u * KVM_THREADS < n4) t[u] += ((double)v[u].x * v[u].x + (double)v[u].y * v[u].y) + ((double)v[u].z * v[u].z + (double)v[u].w * v[u].w);
  }
  s += (t[0] + t[1]) + (t[2] + t[3]);
  s = block_sum_d(s, red);
  if (tid() == 0) stwt32(part.f() + (c.i(2)), (float)s);
  return true;
}

// delta[b, h, t] = sum over the head's columns of o * do (registry op 46): one wave per row, each head's hd columns
// on hd/4 lanes (reduced with lane exchanges inside the group); NV 4-element vectors per lane (row width 256 * NV).
template <int NV> __device__ __noinline__ void delta_rows(const View& o, const View& d, const View& delta, int r0, int r1, int T, int H, int hd) {
  const int gl = hd / 4;
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    f32x4n a[NV], b[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) { a[i] = ld4(o, (long long)r * o.cols + 4 * (lane() + 64 * i)); b[i] = ld4(d, (long long)r * d.cols + 4 * (lane() + 64 * i)); }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      float s = (a[i].x * b[i].x + a[i].y * b[i].y) + (a[i].z * b[i].z + a[i].w * b[i].w);
      for (int x = 1; x < gl; x <<= 1) s += __shfl_xor(s, x, 64);
      const int col = 4 * (lane() + 64 * i);
      if ((lane() & (gl - 1)) == 0) stwt32(delta.f() + (((long long)(r / T) * H + col / hd) * T + r % T), s);
    }
  }
}
__device__ __noinline__ bool op_attn_bwd_delta_fast(const Ctx& c) {
  const View o = c.buf(0), d = c.buf(1), delta = c.buf(2);
  const int r0 = c.i(3), r1 = c.i(4), T = c.i(5), H = c.i(6), hd = c.i(7);
  const int W = H * hd, gl = hd / 4;
  if (hd % 4 || (gl & (gl - 1)) || gl > 64 || W % 256 || !vec4_ok(o) || !vec4_ok(d)) return false;
  switch (W / 256) {
    case 1: delta_rows<1>(o, d, delta, r0, r1, T, H, hd); break;
    case 2: delta_rows<2>(o, d, delta, r0, r1, T, H, hd); break;
    case 3: delta_rows<3>(o, d, delta, r0, r1, T, H, hd); break;
    case 4: delta_rows<4>(o, d, delta, r0, r1, T, H, hd); break;
    case 8: delta_rows<8>(o, d, delta, r0, r1, T, H, hd); break;
    case 16: delta_rows<16>(o, d, delta, r0, r1, T, H, hd); break;
    default: return false;
  }
  return true;
}

// Cross-entropy entry points (ops 51, 53, 127): the streaming rows when the logits allow, else ce_rows.
__device__ __noinline__ void op_softmax_ce_fwd_any(const Ctx& c) {
  View n{};
  if (!ce_rows_fast(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), n, c.i(4), c.i(5), c.i(6), c.i(7), 0.f, true, false)) op_softmax_ce_fwd(c);
}
__device__ __noinline__ void op_softmax_ce_bwd_any(const Ctx& c) {
  View n{};
  const float f = c.buf(3).f()[1] * c.f(9);
  if (!ce_rows_fast(c, c.buf(0), c.buf(1), n, c.buf(2), c.buf(4), c.i(5), c.i(6), c.i(7), c.i(8), f, false, true)) op_softmax_ce_bwd(c);
}
// Cross entropy for small vocabularies (V <= 32, f32 logits and gradient: classifier heads): one row per lane, the row's
// logits loaded together into registers, then max, sum of exponentials, lse, loss and gradient as in ce_rows.
constexpr int CE_SMALL_V = 32;
__device__ bool ce_rows_small(const Ctx& c, View lg, View tg, View rl, View ls, View dl, int r0, int r1, int V, int ignore, float f) {
  if (V > CE_SMALL_V || V < 1 || lg.dtype != 0 || dl.dtype != 0) return false;
  for (int r = r0 + tid(); r < r1; r += KVM_THREADS) {
    const int t = tg.i()[r];
    const bool ign = t == ignore;
    if (!ign && (t < 0 || t >= V)) { c.fail(KVM_ERR_OP_TOKEN, r, t); continue; }
    const GLOBAL float* row = lg.f() + (long long)r * lg.cols;
    float x[CE_SMALL_V];
#pragma unroll
    for (int j = 0; j < CE_SMALL_V; ++j) x[j] = row[j < V ? j : V - 1];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < CE_SMALL_V; ++j) if (j < V) m = fmaxf(m, x[j]);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < CE_SMALL_V; ++j) if (j < V) s += __expf(x[j] - m);
    const float lse = ign ? 0.f : m + logf(s);
    float xt = 0.f;                          // the target's logit, without indexing the register array at run time
#pragma unroll
    for (int j = 0; j < CE_SMALL_V; ++j) if (j == t) xt = x[j];
    stwt32(ls.f() + r, lse);
    stwt32(rl.f() + r, ign ? 0.f : lse - xt);
    GLOBAL float* d = dl.f() + (long long)r * dl.cols;
#pragma unroll
    for (int j = 0; j < CE_SMALL_V; ++j)
      if (j < V) stwt32(d + j, ign ? 0.f : (__expf(x[j] - lse) - (j == t ? 1.f : 0.f)) * f);
  }
  return true;
}

__device__ __noinline__ void op_softmax_ce_fused_any(const Ctx& c) {
  const float f = (float)(1.0 / c.i(9)) * c.f(10);
  if (ce_rows_small(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4), c.i(5), c.i(6), c.i(7), c.i(8), f)) return;
  if (!ce_rows_fast(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4), c.i(5), c.i(6), c.i(7), c.i(8), f, true, true)) op_softmax_ce_fused(c);
}

}  // namespace kvm

namespace kvm {
// Op 303: out[r, c] = sum over s = 0..S-1, in order, of part[s*M + r, c] for rows [r0, r1) and columns [0, N). Each
// thread takes 4 columns of one row and keeps the S partial loads of that piece in flight together (S <= 16 in the
// vector form; larger S and unaligned shapes take the scalar loop).
__device__ __noinline__ void op_splitk_reduce(const Ctx& c) {
  const View part = c.buf(0), out = c.buf(1);
  const int M = c.i(2), N = c.i(3), S = c.i(4), r0 = c.i(5), r1 = c.i(6);
  const long long pc = part.cols, oc = out.cols;
  if (S <= 16 && (N & 3) == 0 && (pc & 3) == 0 && (oc & 3) == 0 && part.dtype == 0) {
    const int q = N / 4;
    const long long n = (long long)(r1 - r0) * q;
    for (long long e = tid(); e < n; e += KVM_THREADS) {
      const int r = r0 + (int)(e / q), col = 4 * (int)(e % q);
      f32x4n v[16];
#pragma unroll
      for (int s = 0; s < 16; ++s)
        if (s < S) v[s] = *(const GLOBAL f32x4n*)(part.f() + ((long long)s * M + r) * pc + col);
      f32x4n t = v[0];
#pragma unroll
      for (int s = 1; s < 16; ++s)
        if (s < S) t += v[s];
      st4(out, (long long)r * oc + col, t);
    }
    return;
  }
  for (long long e = tid(); e < (long long)(r1 - r0) * N; e += KVM_THREADS) {
    const int r = r0 + (int)(e / N), col = (int)(e % N);
    float t = part.ld((long long)r * pc + col);
    for (int s = 1; s < S; ++s) t += part.ld(((long long)s * M + r) * pc + col);
    out.st((long long)r * oc + col, t);
  }
}
}  // namespace kvm

namespace kvm {
// Embedding backward with token ids (registry op 33): dtab[key] += dout[r] for the rows r whose id falls in this
// task's key range [v0, v1). The ids are read 4096 at a time with all loads in flight, the matching rows are compacted
// into an LDS list in ascending row order (wave ballots, then the four waves in order), and only those rows are added,
// row after row in that order (the reference's summation order), 256 columns per pass.
__device__ __noinline__ bool op_embedding_bwd_fast(const Ctx& c) {
  const View ids = uniform_view(c.buf(0)), dout = uniform_view(c.buf(1)), dt = uniform_view(c.buf(2));
  const int N = c.i(3), v0 = c.i(5), v1 = c.i(6), d = c.i(7), acc = c.i(8);
  if (!ids.ok() || dt.dtype != 0 || N > 16384) return false;
  LDS int* list = (LDS int*)c.smem;                 // [N] matching rows
  LDS int* wcnt = list + 16384;                      // [4]
  if (!acc)
    for (long long e = tid(); e < (long long)(v1 - v0) * d; e += KVM_THREADS) stwt32(dt.f() + ((long long)(v0 + e / d) * dt.cols + e % d), 0.f);
  int nm = 0;
  for (int s0 = 0; s0 < N; s0 += 16 * KVM_THREADS) {
    int key[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) key[u] = ids.i()[min(s0 + u * KVM_THREADS + tid(), N - 1)];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int r = s0 + u * KVM_THREADS + tid();
      const bool hit = r < N && key[u] >= v0 && key[u] < v1;
      const unsigned long long bal = __ballot(hit);
      __syncthreads();                                 // the previous round's counts are consumed
      if (lane() == 0) wcnt[wave()] = __popcll(bal);
      __syncthreads();
      int off = nm;
      for (int w = 0; w < wave(); ++w) off += wcnt[w];
      if (hit) list[off + __popcll(bal & ((1ull << lane()) - 1ull))] = r;
      nm += (wcnt[0] + wcnt[1]) + (wcnt[2] + wcnt[3]);
    }
  }
  __syncthreads();
  for (int i = 0; i < nm; ++i) {
    const int r = list[i], k = ids.i()[r];
    for (int col = tid(); col < d; col += KVM_THREADS) stwt32(dt.f() + ((long long)k * dt.cols + col), dt.f()[(long long)k * dt.cols + col] + (dout.at(r, col)));
  }
  return true;
}
}  // namespace kvm
