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
__device__ __noinline__ void op_gemv_bf16_simt(const Ctx& c) {
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
__device__ __noinline__ void op_gemv_bf16_rows_simt(const Ctx& c) {
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


// ---------------------------------------------------------------------------------------------- streaming GEMV
// out[m, n] = sum_k v[m, k] * w[n, k] (+ res[m, n]) for M <= 16 rows of activations (op 134 with M = 1, and op 301),
// v = bf16(prologue(x)). The weight stream is the whole cost, so it is shaped for HBM:
//   * each wave streams one quarter of K. A 64-k step covers 16 weight rows: lane l loads 32 contiguous bytes of row
//     l % 16 (16 lanes cover 16 rows, the 4 lane groups cover the 64 k, so every 128-byte line is read whole) straight
//     into the registers that two v_mfma_f32_16x16x32_bf16 take as their B operand; the activation rows are the A
//     operand (rows >= M read as zero). Both operands take k in the same lane-group order, so the dot products are
//     unchanged;
//   * the weight loads are issued from inline assembly into a ring of GV_RING register pairs, GV_RING steps ahead,
//     and each step waits with an explicit vmcnt tied to the registers it consumes: the compiler's own wait placement
//     (which drains all loads at any branch) never sees them. Every step issues exactly two loads (past the end a
//     re-read of a line just streamed), so the wait count is a constant, and the ring is drained before it goes out of
//     scope;
//   * the first steps' loads are requested before v is staged, which does not depend on the weights;
//   * v is staged as bf16 [M][KC + 8] in LDS once per K chunk, with the activation loads batched; each wave adds its
//     partial 16x16 tiles into its own LDS region, and the four regions are summed in wave order at the end (fixed
//     order).
constexpr int GV_SB = 8;           // activation vectors per thread per staging batch (all in flight)
constexpr int GV_GRP = 8;          // 16-row blocks whose partial tiles are kept in LDS at once (a group re-stages v)
#ifndef KVM_GV_RING
#define KVM_GV_RING 4
#endif
constexpr int GV_RING = KVM_GV_RING;   // 64-k steps in flight per wave (2 KiB each): deeper rings measured slower

__device__ __forceinline__ float gv_pro(int pro, float xv, float x2v, float gv, float rs) {
  return pro == 1 ? xv * rs * gv : pro == 2 ? silu_f(xv) * x2v : xv;
}

// RMSNorm statistics of the M rows of x over all of K: each wave takes two rows at a time, and every load of a batch
// (RU 16-byte vectors of each of the two rows per lane) is in flight before any is used.
template <int RU> __device__ __forceinline__ void gv_rstd(const Ld4& lx, int xc, int M, int K, float eps, LDS float* rstd) {
  const int l = lane(), wv = wave();
  for (int m0 = wv; m0 < M; m0 += 2 * KVM_WAVES) {
    const int mb = m0 + KVM_WAVES, mbc = mb < M ? mb : m0;
    float sa = 0.f, sb = 0.f;
    for (int k0 = 0; k0 < K; k0 += 256 * RU) {
      f32x4n ta[RU], tb[RU];
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const int kk = min(k0 + 4 * l + 256 * u, K - 4);
        ta[u] = lx.get(m0 * xc + kk);
        tb[u] = lx.get(mbc * xc + kk);
      }
#pragma unroll
      for (int u = 0; u < RU; ++u)
        if (k0 + 4 * l + 256 * u < K) {
          sa += (ta[u].x * ta[u].x + ta[u].y * ta[u].y) + (ta[u].z * ta[u].z + ta[u].w * ta[u].w);
          sb += (tb[u].x * tb[u].x + tb[u].y * tb[u].y) + (tb[u].z * tb[u].z + tb[u].w * tb[u].w);
        }
    }
    sa = wave_sum(sa);
    sb = wave_sum(sb);
    if (l == 0) {
      rstd[m0] = 1.f / sqrtf(sa / (float)K + eps);
      if (mb < M) rstd[mb] = 1.f / sqrtf(sb / (float)K + eps);
    }
  }
}
// v = bf16(prologue(x)) for columns [kc, kc + kn) of the M rows: batches of SB vectors per thread, each batch's loads
// (x, and x2 for the SwiGLU prologue or gamma for the RMSNorm one; nothing for an absent operand) issued first.
template <int PRO, int SB>
__device__ __forceinline__ void gv_stage(const Ld4& lx, const Ld4& la, int xc, int ac, int M, int kc, int kn, int VS, LDS uint16_t* vs,
                                         const LDS float* rstd) {
  const int q4 = kn / 4, nel = M * q4;
  for (int e0 = tid(); e0 < nel; e0 += SB * KVM_THREADS) {
    f32x4n xv[SB], av[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int e = min(e0 + u * KVM_THREADS, nel - 1), m = e / q4, k = kc + 4 * (e % q4);
      xv[u] = lx.get(m * xc + k);
      if constexpr (PRO == 2) av[u] = la.get(m * ac + k);
      else if constexpr (PRO == 1) av[u] = la.get(k);
    }
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int e = e0 + u * KVM_THREADS;
      if (e < nel) {
        const int m = e / q4, k = 4 * (e % q4);
        const float rs = PRO == 1 ? rstd[m] : 0.f;
        const f32x4n a = PRO != 0 ? av[u] : f32x4n{0.f, 0.f, 0.f, 0.f};
        *(LDS u16x4_t*)(vs + m * VS + k) = u16x4_t{f2bf(gv_pro(PRO, xv[u].x, a.x, a.x, rs)), f2bf(gv_pro(PRO, xv[u].y, a.y, a.y, rs)),
                                                  f2bf(gv_pro(PRO, xv[u].z, a.z, a.z, rs)), f2bf(gv_pro(PRO, xv[u].w, a.w, a.w, rs))};
      }
    }
  }
}

// K chunk staged in LDS at once: all of K when M rows of it fit in GV_VS_MAX (then one chunk, one continuous weight
// stream), else the largest of 4096 / 2048 / 1024 that divides K.
// LDS left for the staged activations [M][KC + 8] next to the row statistics and the partial tiles.
constexpr long long GV_VS_MAX = KVM_LDS_BYTES - 4ll * GV_GRP * 256 * 4 - 128;
__device__ __forceinline__ int gv_kc(int K, int M) {
  if ((long long)M * (K + 8) * 2 <= GV_VS_MAX) return K;
  for (int kc = 4096; kc >= 256; kc >>= 1)
    if (K % kc == 0 && (long long)M * (kc + 8) * 2 <= GV_VS_MAX) return kc;
  return 256;
}

// Shapes the stream form takes: K a multiple of 256 (each wave a whole number of 64-k steps) made of equal chunks,
// 16-byte aligned rows.
__device__ __forceinline__ bool gemv_stream_ok(const View& x, const View& x2, const View& w, const View& out, int K, int M, int pro) {
  const int KC = gv_kc(K, M);
  return M >= 1 && M <= 16 && K % 256 == 0 && K % KC == 0 && w.dtype == 2 && (w.cols % 8) == 0 && x.dtype != 1 &&
         (x.cols % 4) == 0 && (pro != 2 || (x2.ok() && x2.dtype != 1 && (x2.cols % 4) == 0)) && out.dtype != 1 &&
         (long long)w.rows * w.cols * 2 < 0x7fffffffll && (long long)x.rows * x.cols * 4 < 0x7fffffffll &&
         (!x2.ok() || (long long)x2.rows * x2.cols * 4 < 0x7fffffffll);
}

// 32 bytes of weights into registers, invisible to the compiler's wait tracking.
__device__ __forceinline__ void gv_load(u16x8_t& a, u16x8_t& b, i32x4_t rs, int off) {
  asm volatile("buffer_load_dwordx4 %0, %2, %3, 0 offen\n\tbuffer_load_dwordx4 %1, %2, %3, 0 offen offset:16"
               : "=v"(a), "=v"(b) : "v"(off), "s"(rs));
}
// vmcnt(N), tied to the registers about to be read so that their uses stay after it.
template <int N> __device__ __forceinline__ void gv_wait(u16x8_t& a, u16x8_t& b) {
  asm volatile("s_waitcnt vmcnt(%2)" : "+v"(a), "+v"(b) : "n"(N));
}

__device__ __noinline__ void gemv_stream(const Ctx& c, int M, int pro, float eps) {
  const View x = uniform_view(c.buf(0)), x2 = uniform_view(c.buf(1)), g = uniform_view(c.buf(2)), w = uniform_view(c.buf(3));
  const View out = uniform_view(c.buf(4)), res = uniform_view(c.buf(5));
  const int n0 = rfl(c.i(6)), n1 = rfl(c.i(7)), K = rfl(c.i(8));
  const int KC = gv_kc(K, M), VS = KC + 8;
  LDS uint16_t* vs = (LDS uint16_t*)c.smem;                                    // [M][VS]
  LDS float* rstd = (LDS float*)(c.smem + ((M * VS * 2 + 15) & ~15));          // [16]
  LDS float* part = rstd + 16;                                                  // [4][GV_GRP][256]
  const int l = lane(), wv = wave(), nrows = n1 - n0, nrb = (nrows + 15) / 16, rowb = w.cols * 2;
#ifdef KVM_GEMM_PROF
  unsigned long long pt[8] = {(unsigned long long)wall_clock64(), 0, 0, 0, 0, 0, 0, 0};
#endif
  const i32x4_t rw = dma_rsrc((const void*)(w.h() + (long long)n0 * w.cols), ((long long)w.rows - n0) * w.cols * 2);
  Ld4 lx, lx2, lg;
  lx.init(x); lx2.init(x2); lg.init(g);
  const bool arow = (l & 15) < M;
  const LDS uint16_t* va = vs + (arow ? (l & 15) : 0) * VS + 16 * (l >> 4);   // rows >= M read row 0 and are zeroed
  bool rstd_done = pro != 1;
  u16x8_t wb[GV_RING][2];
  for (int g0 = 0; g0 < nrb; g0 += GV_GRP) {
    const int ng = min(GV_GRP, nrb - g0);
    for (int kc = 0; kc < K; kc += KC) {
      const int kn = min(KC, K - kc), kq = kn / 4, ns = kq / 64, T = ng * ns;
      // byte offset of this lane's 32 bytes in step 0 of row block rb (rows past n1 repeat the last; dropped below)
      auto row_base = [&](int rb) { return min((g0 + rb) * 16 + (l & 15), nrows - 1) * rowb + (kc + wv * kq) * 2 + 32 * (l >> 4); };
      // issue cursor: step it = (irb, ist)
      int irb = 0, ist = 0, ibase = row_base(0);
      const int dummy = ibase;
      auto issue_next = [&](u16x8_t& a, u16x8_t& b) {
        const bool live = irb < ng;
        gv_load(a, b, rw, live ? ibase + ist * 128 : dummy);
        if (live && ++ist == ns) { ist = 0; ++irb; if (irb < ng) ibase = row_base(irb); }
      };
#pragma unroll
      for (int j = 0; j < GV_RING; ++j) issue_next(wb[j][0], wb[j][1]);     // weights first: they do not wait for x
      if (!rstd_done) {                                                          // rstd of each row over all of K
        gv_rstd<8>(lx, x.cols, M, K, eps, rstd);
        rstd_done = true;
      }
      if (kc == 0) for (int e = l; e < ng * 256; e += 64) part[(wv * GV_GRP) * 256 + e] = 0.f;
      __syncthreads();                                                          // rstd ready; the previous chunk's readers are done
      if (pro == 1) gv_stage<1, 8>(lx, lg, x.cols, 0, M, kc, kn, VS, vs, rstd);          // v = bf16(prologue(x)), this chunk
      else if (pro == 2) gv_stage<2, 8>(lx, lx2, x.cols, x2.cols, M, kc, kn, VS, vs, rstd);
      else gv_stage<0, 16>(lx, lx, x.cols, 0, M, kc, kn, VS, vs, rstd);
      __syncthreads();
#ifdef KVM_GEMM_PROF
      if (g0 == 0) pt[1] = wall_clock64();
#endif
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      int crb = 0, cst = 0;
      const LDS uint16_t* vk = va + wv * kq;
      for (int t0 = 0; t0 < T; t0 += GV_RING) {
#pragma unroll
        for (int j = 0; j < GV_RING; ++j) {
          if (t0 + j < T) {
            gv_wait<2 * (GV_RING - 1)>(wb[j][0], wb[j][1]);                  // this step's two loads have landed
            const u16x8_t a0 = *(const LDS u16x8_t*)(vk + cst * 64), a1 = *(const LDS u16x8_t*)(vk + cst * 64 + 8);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8_t)(arow ? a0 : u16x8_t{}), (bf16x8_t)wb[j][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8_t)(arow ? a1 : u16x8_t{}), (bf16x8_t)wb[j][1], acc, 0, 0, 0);
            issue_next(wb[j][0], wb[j][1]);
            if (++cst == ns) {        // row block finished for this chunk: D[m][n], lane holds m = 4*(l/16) + i, n = l % 16
              LDS float* pp = part + (wv * GV_GRP + crb) * 256 + 4 * (l >> 4) * 16 + (l & 15);
#pragma unroll
              for (int i = 0; i < 4; ++i) pp[i * 16] += acc[i];
              acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
              cst = 0; ++crb;
            }
          }
        }
      }
#pragma unroll
      for (int j = 0; j < GV_RING; ++j) gv_wait<0>(wb[j][0], wb[j][1]);      // the ring's trailing re-reads have landed
    }
#ifdef KVM_GEMM_PROF
    if (g0 == 0) pt[2] = wall_clock64();
#endif
    __syncthreads();
#ifdef KVM_GEMM_PROF
    if (g0 == 0) pt[3] = wall_clock64();
#endif
    for (int e = tid(); e < ng * 16 * M; e += KVM_THREADS) {                   // sum the four waves' tiles, in wave order
      const int rb = e / (16 * M), m = (e / 16) % M, nn = e % 16, n = n0 + (g0 + rb) * 16 + nn;
      if (n >= n1) continue;
      const int q = rb * 256 + m * 16 + nn;
      const float s = (part[q] + part[GV_GRP * 256 + q]) + (part[2 * GV_GRP * 256 + q] + part[3 * GV_GRP * 256 + q]);
      out.st((long long)m * out.cols + n, s + (res.ok() ? res.ld((long long)m * res.cols + n) : 0.f));
    }
    __syncthreads();
  }
#ifdef KVM_GEMM_PROF
  pt[4] = wall_clock64();
  __syncthreads();
  if (tid() == 0 && out.dtype == 0) { unsigned long long* o = (unsigned long long*)(out.f() + n0); for (int i = 0; i < 5; ++i) o[i] = pt[i]; o[5] = g_prof[blockIdx.x][6]; }
#endif
}

__device__ __noinline__ void op_gemv_bf16(const Ctx& c) {
  const View x = c.buf(0), x2 = c.buf(1), w = c.buf(3), out = c.buf(4);
  if (gemv_stream_ok(x, x2, w, out, c.i(8), 1, c.i(9))) gemv_stream(c, 1, c.i(9), c.f(10));
  else op_gemv_bf16_simt(c);
}
__device__ __noinline__ void op_gemv_bf16_rows(const Ctx& c) {
  const View x = c.buf(0), x2 = c.buf(1), w = c.buf(3), out = c.buf(4);
  if (gemv_stream_ok(x, x2, w, out, c.i(8), c.i(9), c.i(10))) gemv_stream(c, c.i(9), c.i(10), c.f(11));
  else op_gemv_bf16_rows_simt(c);
}

}  // namespace kvm
