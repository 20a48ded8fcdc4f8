// Operator bodies of the core, GPT and extra packs that are not GEMM or attention tiles. Each runs on one
// workgroup of 256 threads; every output element has one writer and a fixed summation order, so results are
// reproducible run to run. Semantics: the registry comments in include/mvm_ops*.def (reference: runtime/ref_ops.py,
// ref_gpt.py, ref_extra.py). Arithmetic is f32 (wider where noted); bf16-storage outputs are rounded once.
#pragma once
#include "common.h"

namespace kvm {

// Flat loop over [e0, e1) with 4-way unrolled coalesced access.
#define FLAT_FOR(i, e0, e1) for (long long i = (long long)(e0) + tid(); i < (long long)(e1); i += KVM_THREADS)

// ---------------------------------------------------------------------------------------------- core pack
__device__ __noinline__ void op_copy(const Ctx& c) { View s = c.buf(0), d = c.buf(1); FLAT_FOR(k, 0, c.i(2)) stwt32i(d.i() + k, s.i()[k]); }
__device__ __noinline__ void op_add(const Ctx& c) { View a = c.buf(0), b = c.buf(1), o = c.buf(2); FLAT_FOR(k, 0, c.i(3)) stwt32(o.f() + k, a.f()[k] + b.f()[k]); }
__device__ __noinline__ void op_scale(const Ctx& c) { View x = c.buf(0), o = c.buf(1); float al = c.f(2); FLAT_FOR(k, 0, c.i(3)) stwt32(o.f() + k, x.f()[k] * al); }
__device__ __noinline__ void op_relu(const Ctx& c) { View x = c.buf(0), o = c.buf(1); FLAT_FOR(k, 0, c.i(2)) { float v = x.f()[k]; stwt32(o.f() + k, v > 0.f ? v : 0.f); } }
__device__ __noinline__ void op_sgd(const Ctx& c) { View w = c.buf(0), g = c.buf(1); float lr = c.f(2); FLAT_FOR(k, 0, c.i(3)) stwt32(w.f() + k, w.f()[k] - __fmul_rn(lr, g.f()[k])); }
__device__ __noinline__ void op_predict(const Ctx& c) { View x = c.buf(0), w = c.buf(1), o = c.buf(2); float s = w.f()[0]; FLAT_FOR(k, 0, c.i(3)) stwt32(o.f() + k, s * x.f()[k]); }
__device__ __noinline__ void op_mse_grad(const Ctx& c) {   // sequential f32 accumulation, as the reference (ref_ops.py:46-54)
  View p = c.buf(0), t = c.buf(1), x = c.buf(2), l = c.buf(3), g = c.buf(4); int n = c.i(5);
  if (tid() == 0) {
    float la = 0.f, ga = 0.f;
    for (int k = 0; k < n; ++k) {
      float d = p.f()[k] - t.f()[k];
      la = la + __fmul_rn(d, d);
      ga = ga + __fmul_rn(2.f * d, x.f()[k]);
    }
    stwt32(l.f() + 0, la / (float)n); stwt32(g.f() + 0, ga / (float)n);
  }
}
__device__ __noinline__ void op_matmul(const Ctx& c) {   // small fp32 GEMM, sequential k (ref_ops.py:57-66)
  View a = c.buf(0), b = c.buf(1), o = c.buf(2); int m = c.i(3), n = c.i(4), k = c.i(5);
  for (int e = tid(); e < m * n; e += KVM_THREADS) {
    int i = e / n, j = e % n; float acc = 0.f;
    for (int p = 0; p < k; ++p) acc = acc + __fmul_rn(a.f()[i * k + p], b.f()[p * n + j]);
    stwt32(o.f() + e, acc);
  }
}
__device__ __noinline__ void op_fill(const Ctx& c) { View x = c.buf(0); float v = c.f(1); FLAT_FOR(k, 0, c.i(2)) stwt32(x.f() + k, v); }
__device__ __noinline__ void op_spin(const Ctx& c) {
  if (tid() == 0) { unsigned long long t0 = wall_clock64(), n = (unsigned long long)c.i(0) * 100ull; while (wall_clock64() - t0 < n) __builtin_amdgcn_s_sleep(2); }
}

// ---------------------------------------------------------------------------------------------- elementwise
// tanh-GELU through the identity 0.5 (1 + tanh(u)) = sigmoid(2u): gelu(x) = x / (1 + 2^(-2 log2(e) u)) with
// u = sqrt(2/pi) (x + 0.044715 x^3), one hardware exp2 and one reciprocal (absolute error below 1e-6 of the tanh
// form in f32; an epilogue of the GEMM tiles, where half the instructions of the tanh form made it VALU-bound).
// For x -> -inf the exponential overflows to inf and the result is -0; for x -> +inf it is x.
__device__ __forceinline__ float gelu_sig(float x, float x2) {
  const float t = fmaf(0.044715f * x2, x, x);                            // x + 0.044715 x^3
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-2.302208198144325f * t));   // sigmoid(2 sqrt(2/pi) t)
}
__device__ __forceinline__ float gelu_f(float x) { return x * gelu_sig(x, x * x); }
// d/dx x s(x) = s + x s (1 - s) 2 sqrt(2/pi) (1 + 3 * 0.044715 x^2), s = sigmoid(2u).
__device__ __forceinline__ float gelu_grad_f(float x) {
  const float x2 = x * x, s = gelu_sig(x, x2);
  return fmaf((x * s) * (1.f - s), fmaf(0.21406444881780076f, x2, 1.5957691216057308f), s);
}
__device__ __forceinline__ float sigmoid_f(float x) { return x >= 0.f ? 1.f / (1.f + __expf(-x)) : __expf(x) / (1.f + __expf(x)); }
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }
__device__ __forceinline__ float silu_d_f(float x) { float s = sigmoid_f(x); return s * (1.f + x * (1.f - s)); }

__device__ __noinline__ void op_gelu_fwd(const Ctx& c) { View x = c.buf(0), o = c.buf(1); FLAT_FOR(k, c.i(2), c.i(3)) o.st(k, gelu_f(x.ld(k))); }
__device__ __noinline__ void op_gelu_bwd(const Ctx& c) {
  View x = c.buf(0), dy = c.buf(1), dx = c.buf(2); int acc = c.i(5);
  FLAT_FOR(k, c.i(3), c.i(4)) { float v = dy.ld(k) * gelu_grad_f(x.ld(k)); dx.st(k, acc ? dx.ld(k) + v : v); }
}
__device__ __noinline__ void op_residual_add(const Ctx& c) { View a = c.buf(0), b = c.buf(1), o = c.buf(2); FLAT_FOR(k, c.i(3), c.i(4)) o.st(k, a.ld(k) + b.ld(k)); }
__device__ __noinline__ void op_sgd_range(const Ctx& c) { View w = c.buf(0), g = c.buf(1); float lr = c.f(2); FLAT_FOR(k, c.i(3), c.i(4)) stwt32(w.f() + k, w.f()[k] - __fmul_rn(lr, g.f()[k])); }
__device__ __noinline__ void op_round_tf32(const Ctx& c) {
  View x = c.buf(0), o = c.buf(1);
  FLAT_FOR(k, c.i(2), c.i(3)) { uint32_t u = __float_as_uint(x.f()[k]); if ((u & 0x7fffffffu) <= 0x7f800000u) u += 0x1000u; stwt32(o.f() + k, __uint_as_float(u & 0xffffe000u)); }
}
__device__ __noinline__ void op_zero_buf(const Ctx& c) {
  View x = c.buf(0);
  if (x.dtype == 2) { FLAT_FOR(k, c.i(1), c.i(2)) stwt16(x.h() + k, 0); }
  else FLAT_FOR(k, c.i(1), c.i(2)) stwt32i(x.i() + k, 0);
}
__device__ __noinline__ void op_counter_inc(const Ctx& c) { View x = c.buf(0); FLAT_FOR(k, c.i(1), c.i(2)) stwt32i(x.i() + k, (int)((unsigned)x.i()[k] + (unsigned)c.i(3))); }
__device__ __noinline__ void op_round_bf16(const Ctx& c) {   // f32<->bf16 storage conversion (or f32->f32 emulation)
  View x = c.buf(0), o = c.buf(1);
  if (x.dtype == 2 && o.dtype == 2) { FLAT_FOR(k, c.i(2), c.i(3)) stwt16(o.h() + k, x.h()[k]); return; }
  FLAT_FOR(k, c.i(2), c.i(3)) { float v = x.ld(k); if (o.dtype == 2) stwt16(o.h() + k, f2bf(v)); else stwt32(o.f() + k, round_bf(v)); }
}
__device__ __forceinline__ float act_f(int kind, float x) {
  switch (kind) { case 0: return x > 0.f ? x : 0.f; case 1: return silu_f(x); case 2: return tanhf(x); default: return sigmoid_f(x); }
}
__device__ __forceinline__ float act_d(int kind, float x) {
  switch (kind) { case 0: return x > 0.f ? 1.f : 0.f; case 1: return silu_d_f(x); case 2: { float t = tanhf(x); return 1.f - t * t; }
    default: { float s = sigmoid_f(x); return s * (1.f - s); } }
}
__device__ __noinline__ void op_act_fwd(const Ctx& c) { View x = c.buf(0), o = c.buf(1); int kind = c.i(2); FLAT_FOR(k, c.i(3), c.i(4)) stwt32(o.f() + k, act_f(kind, x.f()[k])); }
__device__ __noinline__ void op_act_bwd(const Ctx& c) {
  View x = c.buf(0), dy = c.buf(1), dx = c.buf(2); int kind = c.i(3), acc = c.i(6);
  FLAT_FOR(k, c.i(4), c.i(5)) { float v = dy.f()[k] * act_d(kind, x.f()[k]); stwt32(dx.f() + k, acc ? dx.f()[k] + v : v); }
}
__device__ __noinline__ void op_silu_mul_fwd(const Ctx& c) { View g = c.buf(0), u = c.buf(1), o = c.buf(2); FLAT_FOR(k, c.i(3), c.i(4)) o.st(k, silu_f(g.ld(k)) * u.ld(k)); }
__device__ __noinline__ void op_silu_mul_bwd(const Ctx& c) {
  View g = c.buf(0), u = c.buf(1), dy = c.buf(2), dg = c.buf(3), du = c.buf(4); int acc = c.i(7);
  FLAT_FOR(k, c.i(5), c.i(6)) {
    float gv = g.f()[k], vg = dy.f()[k] * (u.f()[k] * silu_d_f(gv)), vu = dy.f()[k] * silu_f(gv);
    stwt32(dg.f() + k, acc ? dg.f()[k] + vg : vg); stwt32(du.f() + k, acc ? du.f()[k] + vu : vu);
  }
}
__device__ __noinline__ void op_scale_flat(const Ctx& c) { View x = c.buf(0), o = c.buf(1); float al = c.f(2); FLAT_FOR(k, c.i(3), c.i(4)) stwt32(o.f() + k, al * x.f()[k]); }
__device__ __noinline__ void op_add_rowtile(const Ctx& c) {
  View x = c.buf(0), pos = c.buf(1), o = c.buf(2); int r0 = c.i(3), r1 = c.i(4), T = c.i(5), d = c.i(6);
  for (long long e = tid(); e < (long long)(r1 - r0) * d; e += KVM_THREADS) {
    int r = r0 + (int)(e / d), k = (int)(e % d);
    stwt32(o.f() + ((long long)r * o.cols + k), x.f()[(long long)r * x.cols + k] + pos.f()[(long long)(r % T) * pos.cols + k]);
  }
}

// ---------------------------------------------------------------------------------------------- embeddings
__device__ __noinline__ void op_embedding_fwd(const Ctx& c) {
  View ids = c.buf(0), wte = c.buf(1), wpe = c.buf(2), out = c.buf(3);
  int r0 = c.i(4), r1 = c.i(5), T = c.i(6), d = c.i(7);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    int id = ids.i()[r];
    bool bad = id < 0 || id >= wte.rows;
    if (bad && lane() == 0) c.fail(KVM_ERR_OP_TOKEN, r, id);
    for (int k = lane(); k < d; k += 64) {
      float v = bad ? 0.f : wte.at(id, k);
      if (wpe.ok() && !bad) v += wpe.at(r % T, k);
      out.st((long long)r * out.cols + k, v);
    }
  }
}
// dtab[key,:] (+)= sum of dout rows with that key, rows ascending. Each thread owns columns; rows in order.
// Table gradient rows [v0, v1): each row gets its matching output-gradient rows added in ascending r (the reference's
// order). With ids, the waves first scan the ids in parallel (wave w takes the w-th quarter of r, a 64-id ballot at a
// time) into an LDS list of the matching r in ascending order, and the in-order updates then run over the matches
// only. Without ids (positions: rows key, key + mod, ...) each wave owns whole table rows and sums them in registers.
__device__ __noinline__ void op_embedding_bwd(const Ctx& c) {
  View ids = c.buf(0), dout = c.buf(1), dt = c.buf(2);
  int N = c.i(3), mod = c.i(4), v0 = c.i(5), v1 = c.i(6), d = c.i(7), acc = c.i(8);
  if (!ids.ok()) {
    for (int key = v0 + wave(); key < v1; key += KVM_WAVES)
      for (int k = lane(); k < d; k += 64) {
        auto* o = dt.f() + ((long long)key * dt.cols + k);
        float s = acc ? *o : 0.f;
        for (int r = key; r < N; r += mod) s += dout.at(r, k);
        stwt32(o, s);
      }
    return;
  }
  if (!acc) for (long long e = tid(); e < (long long)(v1 - v0) * d; e += KVM_THREADS) stwt32(dt.f() + ((long long)(v0 + e / d) * dt.cols + e % d), 0.f);
  const int Q = (N + KVM_WAVES - 1) / KVM_WAVES;
  if (2ll * N * 4 + 64 <= KVM_LDS_BYTES) {
    LDS int* mr = (LDS int*)c.smem;          // [KVM_WAVES][Q]: matching r, per wave in ascending order
    LDS int* mk = mr + KVM_WAVES * Q;        // their keys
    LDS int* cnt = mk + KVM_WAVES * Q;       // [KVM_WAVES]
    const int w = wave(), l = lane(), r1 = min(N, (w + 1) * Q);
    int n = 0;
    for (int r0 = w * Q; r0 < r1; r0 += 64) {
      const int r = r0 + l;
      const int key = r < r1 ? ids.i()[r] : -1;
      const bool m = key >= v0 && key < v1;
      const unsigned long long bal = __ballot(m);
      if (m) {
        const int at = n + __popcll(bal & ((1ull << l) - 1));
        mr[w * Q + at] = r; mk[w * Q + at] = key;
      }
      n += __popcll(bal);
    }
    if (l == 0) cnt[w] = n;
    __syncthreads();
    for (int ww = 0; ww < KVM_WAVES; ++ww) {
      const int nw = cnt[ww];
      for (int i = 0; i < nw; ++i) {
        const int r = mr[ww * Q + i], key = mk[ww * Q + i];
        for (int k = tid(); k < d; k += KVM_THREADS) {
          auto* o = dt.f() + ((long long)key * dt.cols + k);
          stwt32(o, *o + dout.at(r, k));
        }
      }
    }
    return;
  }
  __syncthreads();
  for (int r = 0; r < N; ++r) {
    int key = ids.i()[r];
    if (key < v0 || key >= v1) continue;
    for (int k = tid(); k < d; k += KVM_THREADS) stwt32(dt.f() + ((long long)key * dt.cols + k), dt.f()[(long long)key * dt.cols + k] + (dout.at(r, k)));
  }
}
__device__ __noinline__ void op_gather_rows(const Ctx& c) {
  View src = c.buf(0), idx = c.buf(1), dst = c.buf(2); int r0 = c.i(3), r1 = c.i(4), d = c.i(5);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    int j = idx.i()[r]; bool bad = j < 0 || j >= src.rows;
    if (bad && lane() == 0) c.fail(KVM_ERR_OP_TOKEN, r, j);
    for (int k = lane(); k < d; k += 64) stwt32(dst.f() + ((long long)r * dst.cols + k), bad ? 0.f : src.f()[(long long)j * src.cols + k]);
  }
}
__device__ __noinline__ void op_select_window(const Ctx& c) {
  View src = c.buf(0), step = c.buf(1), dst = c.buf(2); int i0 = c.i(3), i1 = c.i(4), stride = c.i(5), off = c.i(6);
  long long base = (long long)step.i()[0] * stride + off;
  if (base < 0 || base + i1 > src.n()) { if (tid() == 0) c.fail(KVM_ERR_OP_RANGE, (int)base, i1); return; }
  FLAT_FOR(k, i0, i1) stwt32i(dst.i() + k, src.i()[base + k]);
}
__device__ __noinline__ void op_gather_rows_scaled(const Ctx& c) {
  View src = c.buf(0), idx = c.buf(1), sc = c.buf(2), dst = c.buf(3); int r0 = c.i(4), r1 = c.i(5), d = c.i(6), acc = c.i(7), i0 = c.i(8);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    int j = idx.i()[i0 + r]; float s = sc.ok() ? sc.f()[i0 + r] : 1.f; bool ok = j >= 0 && j < src.rows;
    for (int k = lane(); k < d; k += 64) {
      float v = ok ? s * src.f()[(long long)j * src.cols + k] : 0.f; long long o = (long long)r * dst.cols + k;
      stwt32(dst.f() + o, acc ? dst.f()[o] + v : v);
    }
  }
}
__device__ __noinline__ void op_scatter_add_rows(const Ctx& c) {
  View src = c.buf(0), idx = c.buf(1), sc = c.buf(2), dst = c.buf(3);
  int N = c.i(4), v0 = c.i(5), v1 = c.i(6), d = c.i(7), acc = c.i(8), i0 = c.i(9);
  for (int v = v0; v < v1; ++v)
    for (int k = tid(); k < d; k += KVM_THREADS) {
      float a = 0.f;
      for (int r = 0; r < N; ++r) if (idx.i()[i0 + r] == v) a += (sc.ok() ? sc.f()[i0 + r] : 1.f) * src.f()[(long long)r * src.cols + k];
      long long o = (long long)v * dst.cols + k; stwt32(dst.f() + o, acc ? dst.f()[o] + a : a);
    }
}
__device__ __noinline__ void op_row_dot(const Ctx& c) {
  View A = c.buf(0), B = c.buf(1), idx = c.buf(2), out = c.buf(3); int r0 = c.i(4), r1 = c.i(5), d = c.i(6), acc = c.i(7), i0 = c.i(8);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    int j = idx.ok() ? idx.i()[i0 + r] : r; bool ok = j >= 0 && j < A.rows;
    float s = 0.f;
    if (ok) for (int k = lane(); k < d; k += 64) s += A.f()[(long long)j * A.cols + k] * B.f()[(long long)r * B.cols + k];
    s = wave_sum(s);
    if (lane() == 0) stwt32(out.f() + (i0 + r), acc ? out.f()[i0 + r] + s : s);
  }
}

// ---------------------------------------------------------------------------------------------- normalisation
// One wave per row; row statistics in f32 with a two-pass (mean, then centred square) reduction.
template <bool RMS> __device__ __noinline__ void op_norm_fwd(const Ctx& c) {
  int k = 0; View x = c.buf(k++), g = c.buf(k++), be; if (!RMS) be = c.buf(k++);
  View out = c.buf(k++), mean; if (!RMS) mean = c.buf(k++);
  View rstd = c.buf(k++);
  int r0 = c.i(k), r1 = c.i(k + 1), d = c.i(k + 2); float eps = c.f(k + 3);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    float mu = 0.f;
    if (!RMS) { float s = 0.f; for (int j = lane(); j < d; j += 64) s += x.at(r, j); mu = wave_sum(s) / (float)d; }
    float ss = 0.f; for (int j = lane(); j < d; j += 64) { float v = x.at(r, j) - mu; ss += v * v; }
    float rs = 1.f / sqrtf(wave_sum(ss) / (float)d + eps);
    for (int j = lane(); j < d; j += 64) out.st((long long)r * out.cols + j, (x.at(r, j) - mu) * rs * g.f()[j] + (RMS ? 0.f : be.f()[j]));
    if (lane() == 0) { stwt32(rstd.f() + r, rs); if (!RMS) stwt32(mean.f() + r, mu); }
  }
}
// Op 309 (element-wise form): dx = res + the LayerNorm input gradient.
__device__ __noinline__ void op_norm_bwd_dx_res(const Ctx& c) {
  View x = c.buf(0), dy = c.buf(1), g = c.buf(2), mean = c.buf(3), rstd = c.buf(4), dx = c.buf(5), res = c.buf(6);
  int r0 = c.i(7), r1 = c.i(8), d = c.i(9);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    float mu = mean.f()[r], rs = rstd.f()[r], s1 = 0.f, s2 = 0.f;
    for (int j = lane(); j < d; j += 64) { float gs = dy.at(r, j) * g.f()[j]; s1 += gs; s2 += gs * (x.at(r, j) - mu) * rs; }
    s1 = wave_sum(s1) / (float)d; s2 = wave_sum(s2) / (float)d;
    for (int j = lane(); j < d; j += 64) {
      float gs = dy.at(r, j) * g.f()[j], xh = (x.at(r, j) - mu) * rs, v = rs * (gs - s1 - xh * s2);
      dx.st((long long)r * dx.cols + j, res.at(r, j) + v);
    }
  }
}
template <bool RMS> __device__ __noinline__ void op_norm_bwd_dx(const Ctx& c) {
  int k = 0; View x = c.buf(k++), dy = c.buf(k++), g = c.buf(k++), mean; if (!RMS) mean = c.buf(k++);
  View rstd = c.buf(k++), dx = c.buf(k++);
  int r0 = c.i(k), r1 = c.i(k + 1), d = c.i(k + 2), acc = c.i(k + 3);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    float mu = RMS ? 0.f : mean.f()[r], rs = rstd.f()[r], s1 = 0.f, s2 = 0.f;
    for (int j = lane(); j < d; j += 64) { float gs = dy.at(r, j) * g.f()[j]; s1 += gs; s2 += gs * (x.at(r, j) - mu) * rs; }
    s1 = RMS ? 0.f : wave_sum(s1) / (float)d; s2 = wave_sum(s2) / (float)d;
    for (int j = lane(); j < d; j += 64) {
      float gs = dy.at(r, j) * g.f()[j], xh = (x.at(r, j) - mu) * rs, v = rs * (gs - s1 - xh * s2);
      long long o = (long long)r * dx.cols + j;
      dx.st(o, acc ? dx.ld(o) + v : v);
    }
  }
}
// dgamma/dbeta column sums over all rows ascending; each thread owns a column, rows read coalesced across threads.
__device__ __noinline__ void op_norm_bwd_params(const Ctx& c) {
  View x = c.buf(0), dy = c.buf(1), mean = c.buf(2), rstd = c.buf(3), dg = c.buf(4), db = c.buf(5);
  int R = c.i(6), c0 = c.i(8), c1 = c.i(9), acc = c.i(10);
  for (int j = c0 + tid(); j < c1; j += KVM_THREADS) {
    float sg = 0.f, sb = 0.f;
    for (int r = 0; r < R; ++r) { float gv = dy.at(r, j); sg += gv * (x.at(r, j) - (mean.ok() ? mean.f()[r] : 0.f)) * rstd.f()[r]; sb += gv; }
    stwt32(dg.f() + j, acc ? dg.f()[j] + sg : sg);
    if (db.ok()) stwt32(db.f() + j, acc ? db.f()[j] + sb : sb);
  }
}
// Columns in groups of 16, each summed by 16 row slots (slot k takes rows k, k + 16, ..., four loads in flight) whose
// partials are then added in slot order: a column of R rows costs R / 16 dependent steps instead of R.
__device__ __noinline__ void op_colsum(const Ctx& c) {
  View x = c.buf(0), out = c.buf(1); int R = c.i(2), c0 = c.i(3), c1 = c.i(4), acc = c.i(5);
  LDS float* part = (LDS float*)c.smem;                 // [16 slots][16 columns]
  const int cj = tid() & 15, slot = tid() >> 4;
  for (int cb = c0; cb < c1; cb += 16) {
    const int j = cb + cj;
    float s = 0.f;
    if (j < c1) {
      int r = slot;
      for (; r + 48 < R; r += 64) {
        const float a0 = x.at(r, j), a1 = x.at(r + 16, j), a2 = x.at(r + 32, j), a3 = x.at(r + 48, j);
        s += a0; s += a1; s += a2; s += a3;
      }
      for (; r < R; r += 16) s += x.at(r, j);
    }
    __syncthreads();                                    // the previous group's partials are read
    part[slot * 16 + cj] = s;
    __syncthreads();
    if (tid() < 16 && j < c1) {
      float t = 0.f;
      for (int k = 0; k < 16; ++k) t += part[k * 16 + tid()];
      stwt32(out.f() + j, acc ? out.f()[j] + t : t);
    }
  }
}
__device__ __noinline__ void op_head_rmsnorm(const Ctx& c) {   // RMSNorm per head slice of hd columns (Qwen3 q/k norm)
  View x = c.buf(0), g = c.buf(1), o = c.buf(2); int r0 = c.i(3), r1 = c.i(4), H = c.i(5), hd = c.i(6); float eps = c.f(7);
  for (int rh = r0 * H + wave(); rh < r1 * H; rh += KVM_WAVES) {
    int r = rh / H, h = rh % H; float ss = 0.f;
    for (int k = lane(); k < hd; k += 64) { float v = x.at(r, h * hd + k); ss += v * v; }
    float rs = 1.f / sqrtf(wave_sum(ss) / (float)hd + eps);
    for (int k = lane(); k < hd; k += 64) o.st((long long)r * o.cols + h * hd + k, (x.at(r, h * hd + k) * rs) * g.f()[k]);
  }
}

// ---------------------------------------------------------------------------------------------- RoPE
__device__ __forceinline__ void rope_sc(long long p, int i, int hd, float theta, float& s, float& co) {
  float inv = powf(theta, -(float)(2 * i) / (float)hd);
  float ang = (float)p * inv;
  sincosf(ang, &s, &co);
}
// The rotation angle with the reference's rounding steps: the inverse frequency theta^(-2i/hd) evaluated in double
// (as exp(x * ln theta), ln theta passed in) and rounded to f32, the angle rounded to f32 from the double product (an
// f32 powf can be an ulp off, which at positions in the thousands moves the angle by ~1e-4); sin and cos of that f32
// angle in f32.
__device__ __forceinline__ void rope_sc_ref(long long p, int i, int hd, double ln_theta, float& s, float& co) {
  const float inv = (float)exp(-(double)(float)(2 * i) / hd * ln_theta);
  const float ang = (float)((double)(float)p * (double)inv);
  sincosf(ang, &s, &co);
}
template <int SIGN> __device__ __noinline__ void op_rope(const Ctx& c) {
  View x = c.buf(0), out = c.buf(1), pos = c.buf(2); int r0 = c.i(3), r1 = c.i(4), T = c.i(5), H = c.i(6), hd = c.i(7); float th = c.f(8);
  long long p0 = pos.ok() ? pos.i()[0] : 0; int half = hd / 2;
  for (long long e = tid(); e < (long long)(r1 - r0) * H * half; e += KVM_THREADS) {
    int i = (int)(e % half); long long rh = e / half; int h = (int)(rh % H), r = r0 + (int)(rh / H);
    float s, co; rope_sc((r % T) + p0, i, hd, th, s, co); s *= (float)SIGN;
    float x1 = x.at(r, h * hd + i), x2 = x.at(r, h * hd + i + half);
    out.st((long long)r * out.cols + h * hd + i, x1 * co - x2 * s);
    out.st((long long)r * out.cols + h * hd + i + half, x1 * s + x2 * co);
  }
}

// ---------------------------------------------------------------------------------------------- softmax / loss
__device__ __noinline__ void op_softmax_rows_fwd(const Ctx& c) {
  View x = c.buf(0), o = c.buf(1); int r0 = c.i(2), r1 = c.i(3), d = c.i(4); float sc = c.f(5);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    float m = -INFINITY; for (int j = lane(); j < d; j += 64) m = fmaxf(m, x.at(r, j) * sc);
    m = wave_max(m);
    float z = 0.f; for (int j = lane(); j < d; j += 64) z += __expf(x.at(r, j) * sc - m);
    z = wave_sum(z);
    for (int j = lane(); j < d; j += 64) stwt32(o.f() + ((long long)r * o.cols + j), __expf(x.at(r, j) * sc - m) / z);
  }
}
__device__ __noinline__ void op_softmax_rows_bwd(const Ctx& c) {
  View p = c.buf(0), dp = c.buf(1), dx = c.buf(2); int r0 = c.i(3), r1 = c.i(4), d = c.i(5), acc = c.i(7); float sc = c.f(6);
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    float dot = 0.f; for (int j = lane(); j < d; j += 64) dot += p.at(r, j) * dp.at(r, j);
    dot = wave_sum(dot);
    for (int j = lane(); j < d; j += 64) { float v = sc * p.at(r, j) * (dp.at(r, j) - dot); long long o = (long long)r * dx.cols + j; stwt32(dx.f() + o, acc ? dx.f()[o] + v : v); }
  }
}
// Cross entropy over rows [r0, r1): one wave per row, online max/sum in one pass over the logits, then the gradient.
__device__ void ce_rows(const Ctx& c, View lg, View tg, View rl, View ls, View dl, int r0, int r1, int V, int ignore, float f, bool fwd, bool bwd) {
  for (int r = r0 + wave(); r < r1; r += KVM_WAVES) {
    int t = tg.i()[r];
    bool ign = t == ignore;
    if (!ign && (t < 0 || t >= V)) { if (lane() == 0) c.fail(KVM_ERR_OP_TOKEN, r, t); continue; }
    float lse;
    if (fwd) {
      if (ign) { if (lane() == 0) { stwt32(rl.f() + r, 0.f); stwt32(ls.f() + r, 0.f); } lse = 0.f; }
      else {
        float m = -INFINITY, s = 0.f;
        for (int j = lane(); j < V; j += 64) { float v = lg.at(r, j); float nm = fmaxf(m, v); s = s * __expf(m - nm) + __expf(v - nm); m = nm; }
        for (int o = 32; o > 0; o >>= 1) {
          float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64), nm = fmaxf(m, m2);
          s = (nm == -INFINITY) ? 0.f : s * __expf(m - nm) + s2 * __expf(m2 - nm); m = nm;
        }
        lse = m + logf(s);
        if (lane() == 0) { stwt32(ls.f() + r, lse); stwt32(rl.f() + r, lse - lg.at(r, t)); }
      }
    } else lse = ls.f()[r];
    if (bwd) for (int j = lane(); j < V; j += 64)
      dl.st((long long)r * dl.cols + j, ign ? 0.f : (__expf(lg.at(r, j) - lse) - (j == t ? 1.f : 0.f)) * f);
  }
}
__device__ __noinline__ void op_softmax_ce_fwd(const Ctx& c) { View n{}; ce_rows(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), n, c.i(4), c.i(5), c.i(6), c.i(7), 0.f, true, false); }
__device__ __noinline__ void op_softmax_ce_reduce(const Ctx& c) {
  View rl = c.buf(0), tg = c.buf(1), loss = c.buf(2); int N = c.i(3), ig = c.i(4);
  __shared__ double red[KVM_WAVES]; __shared__ float redc[KVM_WAVES];
  double s = 0.0; float cnt = 0.f;
  for (int r = tid(); r < N; r += KVM_THREADS) if (tg.i()[r] != ig) { s += rl.f()[r]; cnt += 1.f; }
  s = block_sum_d(s, red); cnt = block_sum(cnt, redc);
  if (tid() == 0) { int n = (int)cnt; stwt32(loss.f() + 0, n ? (float)(s / n) : 0.f); stwt32(loss.f() + 1, n ? (float)(1.0 / n) : 0.f); }
}
__device__ __noinline__ void op_softmax_ce_bwd(const Ctx& c) {
  View n{}; float f = c.buf(3).f()[1] * c.f(9);
  ce_rows(c, c.buf(0), c.buf(1), n, c.buf(2), c.buf(4), c.i(5), c.i(6), c.i(7), c.i(8), f, false, true);
}
__device__ __noinline__ void op_softmax_ce_fused(const Ctx& c) {
  float f = (float)(1.0 / c.i(9)) * c.f(10);
  ce_rows(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4), c.i(5), c.i(6), c.i(7), c.i(8), f, true, true);
}

// ---------------------------------------------------------------------------------------------- optimizer
// AdamW in the reference's f32 step order (ref_gpt.py:457-471), 128-bit vectorised where the range allows.
__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, float gsc, float b1, float b2, float lr, float eps, float wd,
                                           float bc1, float bc2) {
  float gi = g * gsc;
  m = __fadd_rn(__fmul_rn(b1, m), __fmul_rn(1.f - b1, gi));
  v = __fadd_rn(__fmul_rn(b2, v), __fmul_rn(__fmul_rn(1.f - b2, gi), gi));
  float decay = __fmul_rn(__fmul_rn(lr, wd), p);
  float step = __fdiv_rn(__fmul_rn(lr, __fdiv_rn(m, bc1)), __fadd_rn(__fsqrt_rn(__fdiv_rn(v, bc2)), eps));
  p = __fsub_rn(__fsub_rn(p, decay), step);
}
// sh (optional, op 305): the updated weight rounded to bf16 (or its f32 emulation when sh is f32), as op 113 would write it.
__device__ void adamw_body(const Ctx& c, View p, View g, View m, View v, View gs, View st, int e0, int e1, float lr, float b1, float b2, float eps, float wd,
                           View sh = View{nullptr, 0, 0, 0}) {
  int t = st.i()[0];
  if (t < 1) { if (tid() == 0) c.fail(KVM_ERR_OP_RANGE, t, 0); return; }
  float gsc = gs.ok() ? gs.f()[0] : 1.f;
  float bc1 = 1.f - (float)pow((double)b1, (double)t), bc2 = 1.f - (float)pow((double)b2, (double)t);
  const int shk = sh.ok() ? (sh.dtype == 2 ? 2 : 1) : 0;    // 0 none, 1 f32 emulation, 2 bf16 storage
  long long a0 = ((long long)e0 + 3) & ~3ll, a1 = (long long)e1 & ~3ll;
  if (a0 > a1) { a0 = e1; a1 = e1; }
  auto one = [&](long long i) {
    float pp = p.f()[i], mm = m.f()[i], vv = v.f()[i];
    adamw_elem(pp, g.f()[i], mm, vv, gsc, b1, b2, lr, eps, wd, bc1, bc2);
    stwt32(p.f() + i, pp); stwt32(m.f() + i, mm); stwt32(v.f() + i, vv);
    if (shk == 2) stwt16(sh.h() + i, f2bf(pp)); else if (shk == 1) stwt32(sh.f() + i, round_bf(pp));
  };
  for (long long i = e0 + tid(); i < a0; i += KVM_THREADS) one(i);
  for (long long i = a1 + tid(); i < e1; i += KVM_THREADS) one(i);
  GLOBAL f32x4n* P = (GLOBAL f32x4n*)p.f(); const GLOBAL f32x4n* G = (const GLOBAL f32x4n*)g.f(); GLOBAL f32x4n* M = (GLOBAL f32x4n*)m.f(); GLOBAL f32x4n* Vv = (GLOBAL f32x4n*)v.f();
  // 16-byte groups are stored through buffer descriptors (one write-through instruction each) when the ranges
  // fit 32-bit byte offsets
  const bool bo = (long long)e1 * 4 < 0x7fffffffll;
  const __amdgpu_buffer_rsrc_t rp = wt_rsrc(p.p, 4ll * e1), rm = wt_rsrc(m.p, 4ll * e1), rv = wt_rsrc(v.p, 4ll * e1);
  auto upd = [&](long long q, f32x4n pp, f32x4n gg, f32x4n mm, f32x4n vv) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float a = pp[j], b = mm[j], d = vv[j];
      adamw_elem(a, gg[j], b, d, gsc, b1, b2, lr, eps, wd, bc1, bc2);
      pp[j] = a; mm[j] = b; vv[j] = d;
    }
    if (bo) { stwt_buf(rp, (int)q * 16, pp); stwt_buf(rm, (int)q * 16, mm); stwt_buf(rv, (int)q * 16, vv); }
    else { stwt_f4((GLOBAL float*)(P + q), pp); stwt_f4((GLOBAL float*)(M + q), mm); stwt_f4((GLOBAL float*)(Vv + q), vv); }
    if (shk == 2) {
      stwt_bf4(sh.h() + 4 * q, pp[0], pp[1], pp[2], pp[3]);
    } else if (shk == 1) {
      f32x4n r; for (int j = 0; j < 4; ++j) r[j] = round_bf(pp[j]);
      stwt_f4(sh.f() + 4 * q, r);
    }
  };
  // four 16-byte groups per thread per pass: sixteen loads in flight before the first update (the loads of a pass
  // wait for the previous pass's write-through stores, so fewer, larger passes)
  constexpr int NG = 4;
  long long q = a0 / 4 + tid(), qe = a1 / 4;
  for (; q + (NG - 1) * KVM_THREADS < qe; q += NG * KVM_THREADS) {
    f32x4n pv[NG], gv[NG], mv[NG], vv[NG];
#pragma unroll
    for (int u = 0; u < NG; ++u) {
      const long long r = q + u * KVM_THREADS;
      pv[u] = P[r]; gv[u] = G[r]; mv[u] = M[r]; vv[u] = Vv[r];
    }
#pragma unroll
    for (int u = 0; u < NG; ++u) upd(q + u * KVM_THREADS, pv[u], gv[u], mv[u], vv[u]);
  }
  for (; q < qe; q += KVM_THREADS) upd(q, P[q], G[q], M[q], Vv[q]);
}
__device__ __noinline__ void op_adamw(const Ctx& c) { adamw_body(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4), c.buf(5), c.i(6), c.i(7), c.f(8), c.f(9), c.f(10), c.f(11), c.f(12)); }
__device__ __noinline__ void op_adamw_bf16(const Ctx& c) { adamw_body(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4), c.buf(5), c.i(6), c.i(7), c.f(8), c.f(9), c.f(10), c.f(11), c.f(12), c.buf(13)); }
__device__ __noinline__ void op_adamw_lr(const Ctx& c) { adamw_body(c, c.buf(0), c.buf(1), c.buf(2), c.buf(3), c.buf(4), c.buf(5), c.i(6), c.i(7), c.buf(8).f()[0], c.f(9), c.f(10), c.f(11), c.f(12)); }
__device__ __noinline__ void op_gradnorm_partial(const Ctx& c) {
  View g = c.buf(0), part = c.buf(1); __shared__ double red[KVM_WAVES];
  double s = 0.0; FLAT_FOR(i, c.i(3), c.i(4)) { double x = g.f()[i]; s += x * x; }
  s = block_sum_d(s, red);
  if (tid() == 0) stwt32(part.f() + (c.i(2)), (float)s);
}
__device__ __noinline__ void op_gradnorm_finish(const Ctx& c) {
  View part = c.buf(0), out = c.buf(2); int ns = c.i(1); float mx = c.f(3);
  // Sum in double: each thread adds a strided subset, then a fixed tree over the threads. The order differs from a
  // serial sum only in the last bits of the double, far below the rounding of the float norm computed from it.
  __shared__ double red[KVM_WAVES];
  double s = 0.0;
  for (int i = tid(); i < ns; i += KVM_THREADS) s += part.f()[i];
  s = block_sum_d(s, red);
  if (tid() == 0) {
    float n = (float)sqrt(s);
    stwt32(out.f() + 0, mx > 0.f ? fminf(1.f, mx / (n + 1e-6f)) : 1.f);
    stwt32(out.f() + 1, n);
  }
}
__device__ __noinline__ void op_lr_schedule(const Ctx& c) {
  View st = c.buf(0), lr = c.buf(1); int kind = c.i(2); float base = c.f(3); int wu = c.i(4), tot = c.i(5); float mr = c.f(6);
  if (tid() == 0) {
    int t = st.i()[0];
    double warm = (wu > 0 && t <= wu) ? (double)t / wu : 1.0;
    double prog = fmin(fmax((double)(t - wu) / (double)max(tot - wu, 1), 0.0), 1.0);
    double f = kind == 0 ? 1.0 : kind == 1 ? mr + (1.0 - mr) * 0.5 * (1.0 + cos(M_PI * prog)) : 1.0 - (1.0 - mr) * prog;
    stwt32(lr.f() + 0, (float)(base * warm * f));
  }
}

// ---------------------------------------------------------------------------------------------- token selection
__device__ __forceinline__ uint32_t order_key(float x) { uint32_t b = __float_as_uint(x); return b ^ ((b >> 31) ? 0xFFFFFFFFu : 0x80000000u); }
// Row argmax: largest value, lowest index on ties; NaN never wins (all-NaN row -> 0).
template <class PF, class PI> __device__ int row_argmax(const View& lg, int r, int V, PF redv, PI redi) {
  float bv = -INFINITY; int bi = 0x7FFFFFFF;
  auto take = [&](float x, int j) { if (x > bv || (x == bv && j < bi)) { bv = x; bi = j; } };
  int j0 = 0;
  if (lg.dtype == 0 && (lg.cols % 4) == 0 && V <= lg.cols) {
    // f32 rows: 16-byte loads, NB of them in flight per thread before any is compared (a scalar load per step
    // serialises a 150k-wide row on load latency). The tie rule makes the visiting order irrelevant.
    constexpr int NB = 16;
    const GLOBAL f32x4n* row = (const GLOBAL f32x4n*)(lg.f() + (long long)r * lg.cols);
    const int nq = V / 4;
    for (int q = tid(); q < nq; q += NB * KVM_THREADS) {
      f32x4n v[NB];
#pragma unroll
      for (int u = 0; u < NB; ++u) v[u] = row[min(q + u * KVM_THREADS, nq - 1)];
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int qq = q + u * KVM_THREADS;
        if (qq < nq) {
#pragma unroll
          for (int e = 0; e < 4; ++e) take(v[u][e], 4 * qq + e);
        }
      }
    }
    j0 = nq * 4;
  }
  for (int j = j0 + tid(); j < V; j += KVM_THREADS) take(lg.at(r, j), j);
  for (int o = 32; o > 0; o >>= 1) {
    float v2 = __shfl_xor(bv, o, 64); int i2 = __shfl_xor(bi, o, 64);
    if (v2 > bv || (v2 == bv && i2 < bi)) { bv = v2; bi = i2; }
  }
  __syncthreads();
  if (lane() == 0) { redv[wave()] = bv; redi[wave()] = bi; }
  __syncthreads();
  bv = redv[0]; bi = redi[0];
  for (int w = 1; w < KVM_WAVES; ++w) if (redv[w] > bv || (redv[w] == bv && redi[w] < bi)) { bv = redv[w]; bi = redi[w]; }
  return bi == 0x7FFFFFFF ? 0 : bi;
}
__device__ __noinline__ void op_argmax(const Ctx& c) {
  View lg = c.buf(0), out = c.buf(1); int r0 = c.i(2), r1 = c.i(3), V = c.i(4);
  __shared__ float rv[KVM_WAVES]; __shared__ int ri[KVM_WAVES];
  for (int r = r0; r < r1; ++r) { int a = row_argmax(lg, r, V, rv, ri); if (tid() == 0) stwt32i(out.i() + r, a); }
}
__device__ void philox10(uint32_t c[4], uint32_t k0, uint32_t k1) {
  for (int r = 0; r < 10; ++r) {
    uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0], hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
    uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
    k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
  }
}
// Sampling (registry text of op 57): temperature softmax over the top-k, inverse CDF in index order, Philox uniform.
// Serial per row on thread 0 after a parallel threshold search; sampling is off the hot path.
__device__ __noinline__ void op_sample(const Ctx& c) {
  View lg = c.buf(0), out = c.buf(1), ctr = c.buf(2); int r0 = c.i(3), r1 = c.i(4), V = c.i(5); float temp = c.f(6); int topk = c.i(7), seed = c.i(8);
  __shared__ float rv[KVM_WAVES]; __shared__ int ri[KVM_WAVES]; __shared__ uint32_t s_thr;
  int cv = ctr.ok() ? ctr.i()[0] : 0;
  for (int r = r0; r < r1; ++r) {
    if (temp <= 0.f) { int a = row_argmax(lg, r, V, rv, ri); if (tid() == 0) stwt32i(out.i() + r, a); continue; }
    if (tid() == 0) {
      uint32_t thr = 0;
      if (topk > 0 && topk < V) {   // k-th largest order key by bitwise binary search on the count of keys >= candidate
        uint32_t lo = 0;
        for (int bit = 31; bit >= 0; --bit) {
          uint32_t cand = lo | (1u << bit); int cnt = 0;
          for (int j = 0; j < V; ++j) cnt += order_key(lg.at(r, j)) >= cand;
          if (cnt >= topk) lo = cand;
        }
        thr = lo;
      }
      s_thr = thr;
      float mx = -INFINITY; for (int j = 0; j < V; ++j) { float x = lg.at(r, j); if (x == x && x > mx) mx = x; }
      double total = 0.0;
      for (int j = 0; j < V; ++j) { float x = lg.at(r, j); if (x == x && order_key(x) >= thr) total += exp((double)(x - mx) / temp); }
      uint32_t cc[4] = {(uint32_t)r, (uint32_t)cv, 0u, 0u}; philox10(cc, (uint32_t)seed, 0x9E3779B9u);
      double target = (double)(cc[0] >> 8) * (1.0 / 16777216.0) * total, run = 0.0; int pick = -1, last = -1;
      for (int j = 0; j < V; ++j) { float x = lg.at(r, j); if (x == x && order_key(x) >= thr) { run += exp((double)(x - mx) / temp); last = j; if (run > target) { pick = j; break; } } }
      stwt32i(out.i() + r, pick >= 0 ? pick : max(last, 0));
    }
    __syncthreads();
  }
  (void)s_thr;
}

// ---------------------------------------------------------------------------------------------- KV cache
__device__ __noinline__ void op_kv_append(const Ctx& c) {
  View kn = c.buf(0), vn = c.buf(1), kc = c.buf(2), vc = c.buf(3), lens = c.buf(4);
  int b0 = c.i(5), b1 = c.i(6), nn = c.i(7), Hkv = c.i(8), hd = c.i(9), Tmax = c.i(10);
  for (int b = b0; b < b1; ++b) { int L = lens.i()[b]; if (L < 0 || L + nn > Tmax) { if (tid() == 0) c.fail(KVM_ERR_OP_KVLEN, b, L); return; } }
  long long per = (long long)nn * Hkv * hd;
  for (long long e = tid(); e < (long long)(b1 - b0) * per; e += KVM_THREADS) {
    int b = b0 + (int)(e / per); long long r = e % per; int t = (int)(r / (Hkv * hd)), h = (int)((r / hd) % Hkv), k = (int)(r % hd);
    long long row = ((long long)b * Hkv + h) * Tmax + lens.i()[b] + t;
    kc.st(row * kc.cols + k, kn.at((long long)b * nn + t, h * hd + k));
    vc.st(row * vc.cols + k, vn.at((long long)b * nn + t, h * hd + k));
  }
}

}  // namespace kvm
