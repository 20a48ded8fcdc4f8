// Decode GEMVs: the bandwidth-bound weight streams of one decode step. The weight matrix w is bf16 [N, K] (row n holds
// output n's K weights), read exactly once per task with 16-byte loads and many loads in flight per lane; the
// prologue vector v = bf16(prologue(x)) sits in LDS. Sums are fp32 in a fixed order.
#pragma once
#include "common.h"
#include "ops_basic.h"

namespace kvm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// v[k] for one row: pro 0 x, 1 x*rstd*gamma (rstd of the whole row), 2 silu(x)*x2; rounded to bf16 (registry op 134).
// Copies n floats (f32 buffer, 16-byte aligned, n % 4 == 0) to LDS with all of a thread's loads issued together;
// the generic per-element loop otherwise runs one load round trip per element.
__device__ void stage_f32(LDS float* dst, const GLOBAL float* src, int n) {
  const GLOBAL f32x4n* sv = (const GLOBAL f32x4n*)src;
  for (int q0 = tid(); q0 < n / 4; q0 += 4 * KVM_THREADS) {
    f32x4n t[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) if (q0 + u * KVM_THREADS < n / 4) t[u] = sv[q0 + u * KVM_THREADS];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 4; ++u) if (q0 + u * KVM_THREADS < n / 4) *(LDS f32x4n*)(dst + 4 * (q0 + u * KVM_THREADS)) = t[u];
  }
}
__device__ __forceinline__ void stage_view(LDS float* dst, const View& v, long long off, int n) {
  if (v.dtype == 0 && (n & 3) == 0 && (off & 3) == 0) stage_f32(dst, v.f() + off, n);
  else for (int k = tid(); k < n; k += KVM_THREADS) dst[k] = v.ld(off + k);
}

// v = bf16(prologue(x)) into vs[0..K): x (and gamma or x2) are staged in LDS first (vs and vs + K), then combined.
// `red` must leave room for 2*K floats after vs.
__device__ void prologue_row(LDS float* vs, const View& x, const View& x2, const View& g, long long xoff, int K, int pro, float eps, LDS float* red) {
  LDS float* aux = vs + K;
  stage_view(vs, x, xoff, K);
  if (pro == 1) stage_view(aux, g, 0, K);
  else if (pro == 2) stage_view(aux, x2, xoff, K);
  __syncthreads();
  if (pro == 1) {
    float ss = 0.f; for (int k = tid(); k < K; k += KVM_THREADS) { float a = vs[k]; ss += a * a; }
    ss = block_sum(ss, red);
    float rs = 1.f / sqrtf(ss / (float)K + eps);
    for (int k = tid(); k < K; k += KVM_THREADS) vs[k] = round_bf(vs[k] * rs * aux[k]);
  } else if (pro == 2) {
    for (int k = tid(); k < K; k += KVM_THREADS) vs[k] = round_bf(silu_f(vs[k]) * aux[k]);
  } else for (int k = tid(); k < K; k += KVM_THREADS) vs[k] = round_bf(vs[k]);
  __syncthreads();
}

__device__ __forceinline__ float dot8(const u16x8_t w, const LDS float* v) {
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) a = fmaf(bf2f(w[i]), v[i], a);
  return a;
}

// Registry op 134. Each wave owns two weight rows at a time and keeps 16 loads of 16 bytes in flight per lane.
__device__ __noinline__ void op_gemv_bf16(const Ctx& c) {
  View x = c.buf(0), x2 = c.buf(1), g = c.buf(2), w = c.buf(3), out = c.buf(4), res = c.buf(5);
  int n0 = c.i(6), n1 = c.i(7), K = c.i(8), pro = c.i(9); float eps = c.f(10);
  LDS float* vs = (LDS float*)c.smem; LDS float* red = vs + 2 * K;
  const int l = lane(), nv = K / 8;
  // Work items: (row pair, 512-vector chunk of the row). Each wave walks its items with two register buffers: the
  // loads of item i+1 are issued before item i is multiplied, so 32 loads of 16 bytes stay in flight per lane.
  // The weights do not depend on x, so the first item's loads are issued before the prologue runs.
  const int chunks = (nv + 511) / 512, npairs = (n1 - n0 + 1) / 2;
  const int nitems = ((npairs - wave() + KVM_WAVES - 1) / KVM_WAVES) * chunks;   // items of this wave
  u16x8_t bufA[16], bufB[16];
  auto issue = [&](int it, u16x8_t* b) {
    const int pr = wave() + (it / chunks) * KVM_WAVES, ch = it % chunks;
    const int row = n0 + 2 * pr, row2 = min(row + 1, n1 - 1);
    const GLOBAL u16x8_t* r0 = (const GLOBAL u16x8_t*)(w.h() + (long long)row * w.cols);
    const GLOBAL u16x8_t* r1 = (const GLOBAL u16x8_t*)(w.h() + (long long)row2 * w.cols);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int qq = min(ch * 512 + l + i * 64, nv - 1);
      b[i] = __builtin_nontemporal_load(&r0[qq]); b[8 + i] = __builtin_nontemporal_load(&r1[qq]);
    }
  };
  float a0 = 0.f, a1 = 0.f;
  auto consume = [&](int it, const u16x8_t* cur) {
    const int ch = it % chunks;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = ch * 512 + l + i * 64;
      if (q < nv) { a0 += dot8(cur[i], vs + q * 8); a1 += dot8(cur[8 + i], vs + q * 8); }
    }
    if (ch == chunks - 1) {           // row pair complete
      const int n = n0 + 2 * (wave() + (it / chunks) * KVM_WAVES);
      a0 = wave_sum(a0); a1 = wave_sum(a1);
      if (l == 0) {
        out.st(n, a0 + (res.ok() ? res.ld(n) : 0.f));
        if (n + 1 < n1) out.st(n + 1, a1 + (res.ok() ? res.ld(n + 1) : 0.f));
      }
      a0 = a1 = 0.f;
    }
  };
  if (nitems > 0) issue(0, bufA);
  __builtin_amdgcn_sched_barrier(0);
  prologue_row(vs, x, x2, g, 0, K, pro, eps, red);
  for (int it = 0; it < nitems; it += 2) {   // two items per trip so the buffers are named statically
    if (it + 1 < nitems) issue(it + 1, bufB);
    __builtin_amdgcn_sched_barrier(0);
    consume(it, bufA);
    if (it + 1 >= nitems) break;
    if (it + 2 < nitems) issue(it + 2, bufA);
    __builtin_amdgcn_sched_barrier(0);
    consume(it + 1, bufB);
  }
}

// Registry op 301 (this executor's pack): M <= 16 rows of activations against 16 weight rows at a time on the
// MFMA units (v_mfma_f32_16x16x32_bf16): A = v (M rows, zero-padded to 16) from LDS, B = the weight rows, loaded
// straight from HBM into the operand registers. Each lane loads 32 contiguous bytes of one weight row per two MFMA
// steps, so four lanes cover a 128-byte line; A uses the same k permutation, which leaves the dot products unchanged.
// The four waves split K into quarters and their 16x16 partial tiles are summed in LDS (fixed order).
constexpr int ROWS_KC = 2048;   // K chunk whose prologue vectors are staged in LDS at once
__device__ __noinline__ void op_gemv_bf16_rows(const Ctx& c) {
  View x = c.buf(0), x2 = c.buf(1), g = c.buf(2), w = c.buf(3), out = c.buf(4), res = c.buf(5);
  int n0 = c.i(6), n1 = c.i(7), K = c.i(8), M = c.i(9), pro = c.i(10); float eps = c.f(11);
  LDS uint16_t* vs = (LDS uint16_t*)c.smem;              // [16][ROWS_KC + 8] bf16
  constexpr int VST = ROWS_KC + 8;
  LDS float* rstd = (LDS float*)(c.smem + 16 * VST * 2); // [16]
  LDS float* part = rstd + 16;                           // [4][16][16] partial tiles
  const int l = lane(), wv = wave();
  if (pro == 1) {                                        // per-row rstd over the full K
    for (int m = wv; m < M; m += KVM_WAVES) {
      float ss = 0.f; for (int k = l; k < K; k += 64) { float a = x.at(m, k); ss += a * a; }
      ss = wave_sum(ss);
      if (l == 0) rstd[m] = 1.f / sqrtf(ss / (float)K + eps);
    }
  }
  for (int nb = n0; nb < n1; nb += 16) {
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    const int nrow = min(nb + (l & 15), n1 - 1);         // rows past n1 repeat the last row; their results are dropped
    const GLOBAL uint16_t* wr = w.h() + (long long)nrow * w.cols;
    for (int kc = 0; kc < K; kc += ROWS_KC) {
      const int kn = min(ROWS_KC, K - kc);
      __syncthreads();
      for (int e = tid(); e < 16 * kn; e += KVM_THREADS) {
        int m = e / kn, k = e % kn;
        float v = 0.f;
        if (m < M) {
          float xv = x.at(m, kc + k);
          v = pro == 1 ? xv * rstd[m] * g.f()[kc + k] : pro == 2 ? silu_f(xv) * x2.at(m, kc + k) : xv;
        }
        vs[m * VST + k] = f2bf(v);
      }
      __syncthreads();
      // 64-k steps round-robin over the four waves (wave wv takes steps wv, wv+4, ...): two MFMAs per step
      const int nsteps = kn / 64, gk = (l >> 4) * 16;
      const LDS uint16_t* va = vs + (l & 15) * VST;
      int s = wv;
      for (; s + 12 < nsteps; s += 16) {
        u16x8_t b[8];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const GLOBAL u16x8_t* p = (const GLOBAL u16x8_t*)(wr + kc + (s + 4 * u) * 64 + gk);
          b[2 * u] = __builtin_nontemporal_load(p); b[2 * u + 1] = __builtin_nontemporal_load(p + 1);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int k = (s + 4 * u) * 64 + gk;
          u16x8_t a0 = *(const LDS u16x8_t*)(va + k), a1 = *(const LDS u16x8_t*)(va + k + 8);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8_t)a0, (bf16x8_t)b[2 * u], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8_t)a1, (bf16x8_t)b[2 * u + 1], acc, 0, 0, 0);
        }
      }
      for (; s < nsteps; s += 4) {
        const int k = s * 64 + gk;
        const GLOBAL u16x8_t* p = (const GLOBAL u16x8_t*)(wr + kc + k);
        u16x8_t b0 = p[0], b1 = p[1];
        u16x8_t a0 = *(const LDS u16x8_t*)(va + k), a1 = *(const LDS u16x8_t*)(va + k + 8);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8_t)a0, (bf16x8_t)b0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8_t)a1, (bf16x8_t)b1, acc, 0, 0, 0);
      }
    }
    // D[m][n]: lane holds m = 4*(l/16) + i, n = l % 16
#pragma unroll
    for (int i = 0; i < 4; ++i) part[(wv * 16 + 4 * (l >> 4) + i) * 16 + (l & 15)] = acc[i];
    __syncthreads();
    for (int e = tid(); e < 16 * 16; e += KVM_THREADS) {
      int m = e / 16, nn = e % 16, n = nb + nn;
      if (m < M && n < n1) {
        float s = (part[m * 16 + nn] + part[(16 + m) * 16 + nn]) + (part[(32 + m) * 16 + nn] + part[(48 + m) * 16 + nn]);
        long long o = (long long)m * out.cols + n;
        out.st(o, s + (res.ok() ? res.at(m, n) : 0.f));
      }
    }
  }
}

}  // namespace kvm
