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
//   * each wave streams one quarter of K. A 64-k step covers 16 weight rows: two direct HBM -> LDS loads per wave
//     (buffer_load_dwordx4 ... lds), the first bringing bytes 0-63 of each row's 128-byte step segment, the second
//     bytes 64-127 (lane l: row l % 16, 16 bytes at 16 (l / 16) of its half), so each load reads 16 whole 64-byte
//     runs. Lane l then reads its own two 16-byte pieces back as the B operands of two v_mfma_f32_16x16x32_bf16; the
//     activation rows are the A operand in the same k order (rows >= M read as zero), so the dot products are unchanged;
//   * the loads land in a ring of R step slots per wave in LDS (R up to 12: 24 KiB in flight per wave, 96 KiB per CU,
//     where registers held 8 KiB per wave), issued R steps ahead across row blocks, K chunks and row groups. Each step
//     waits with an explicit vmcnt for its own two loads (every step issues exactly two, past the end two loads
//     outside the descriptor's range, which touch no memory), and the compiler never sees the ring;
//   * the first R steps do not depend on the task's inputs: they are requested before v is staged, and on the static
//     path before the task even waits for its predecessors (gemv_prefetch, when the host found the weight buffer
//     read-only in the graph);
//   * v is staged as bf16 [M][KC + 8] in LDS once per K chunk, with the activation loads batched; each wave adds its
//     partial 16 x M tiles into its own LDS region, and the four regions are summed in wave order at the end (fixed
//     order).
constexpr int GV_SB = 8;           // activation vectors per thread per staging batch (all in flight)
constexpr int GV_GRP = 8;          // 16-row blocks whose partial tiles are kept in LDS at once (a group re-stages v)
constexpr int GV_STEP = 2048;      // one wave's 64-k step of 16 rows: 64 lanes x 32 bytes

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
// One row's RMSNorm prologue over all of K in one round trip (the batch-1 decode form): each thread loads its NV
// 16-byte vectors of x and gamma at once, the sum of squares is reduced over the workgroup (wave sums, then the four
// in order through `red`), and v = bf16(x * rstd * gamma) is written to vs. K / 4 <= NV * KVM_THREADS.
template <int NV> __device__ __forceinline__ void gv_stage_rms1(const Ld4& lx, const Ld4& lg, int K, float eps, LDS uint16_t* vs, LDS float* red) {
  const int q4 = K / 4;
  f32x4n xv[NV], gv[NV];
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int e = min(tid() + u * KVM_THREADS, q4 - 1);
    xv[u] = lx.get(4 * e);
    gv[u] = lg.get(4 * e);
  }
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < NV; ++u)
    if (tid() + u * KVM_THREADS < q4) ss += (xv[u].x * xv[u].x + xv[u].y * xv[u].y) + (xv[u].z * xv[u].z + xv[u].w * xv[u].w);
  ss = wave_sum(ss);
  if (lane() == 0) red[wave()] = ss;
  __syncthreads();
  const float rs = 1.f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)K + eps);
#pragma unroll
  for (int u = 0; u < NV; ++u) {
    const int e = tid() + u * KVM_THREADS;
    if (e < q4)
      *(LDS u16x4_t*)(vs + 4 * e) = u16x4_t{f2bf(xv[u].x * rs * gv[u].x), f2bf(xv[u].y * rs * gv[u].y), f2bf(xv[u].z * rs * gv[u].z),
                                           f2bf(xv[u].w * rs * gv[u].w)};
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

// LDS geometry of one call with a ring of R steps per wave: [ring: 4 waves x R steps][v: M x (KC + 8) bf16]
// [rstd: 16 f32][partials: 4 x GV_GRP x M x 16 f32]. KC is all of K when it fits, else the largest of 4096 .. 256
// dividing K that does.
struct GvGeo { int KC, VS, vs_off, rstd_off, part_off; };
__device__ __forceinline__ GvGeo gv_geo(int K, int M, int R) {
  auto fits = [&](int kc) {
    return R * KVM_WAVES * GV_STEP + ((M * (kc + 8) * 2 + 15) & ~15) + 64 + KVM_WAVES * GV_GRP * M * 16 * 4 <= KVM_LDS_BYTES;
  };
  int KC = 256;
  if (fits(K)) KC = K;
  else
    for (int kc = 4096; kc >= 512; kc >>= 1)
      if (K % kc == 0 && fits(kc)) { KC = kc; break; }
  GvGeo g;
  g.KC = KC; g.VS = KC + 8;
  g.vs_off = R * KVM_WAVES * GV_STEP;
  g.rstd_off = g.vs_off + ((M * g.VS * 2 + 15) & ~15);
  g.part_off = g.rstd_off + 64;
  return g;
}
// Ring depth: GV_R steps per wave (8 KiB per wave: in the steady state the stream is not latency bound with more);
// a ring filled before the dependency wait is deeper for one-row GEMVs, so that more of the task's weights arrive during
// the wait. Batched rows keep 4 steps: their activations then fit LDS whole and are staged once instead of per K chunk
// (batch-8 decode 7.21 vs 7.27 ms with 8 steps).
#ifndef KVM_GV_R
#define KVM_GV_R 4
#endif
constexpr int GV_R = KVM_GV_R;
#ifndef KVM_GV_PRE
#define KVM_GV_PRE 0
#endif
__device__ __forceinline__ int gv_pre_ring(int M) { return KVM_GV_PRE ? KVM_GV_PRE : M <= 4 ? 12 : 4; }

// Shapes the stream form takes: K a multiple of 256 (each wave a whole number of 64-k steps), M <= 16, 16-byte
// aligned rows, byte offsets inside 31 bits.
__device__ __forceinline__ bool gemv_stream_ok(const View& x, const View& x2, const View& w, const View& out, int K, int M, int pro) {
  return M >= 1 && M <= 16 && K % 256 == 0 && w.dtype == 2 && (w.cols % 8) == 0 && x.dtype != 1 &&
         (x.cols % 4) == 0 && (pro != 2 || (x2.ok() && x2.dtype != 1 && (x2.cols % 4) == 0)) && out.dtype != 1 &&
         (long long)w.rows * w.cols * 2 < 0x7fff0000ll && (long long)x.rows * x.cols * 4 < 0x7fffffffll &&
         (!x2.ok() || (long long)x2.rows * x2.cols * 4 < 0x7fffffffll);
}

// One wave's weight stream: a wave-uniform issue cursor over (row group, K chunk, row block, step) and the ring slot
// it fills next.
// DUAL (the fused SwiGLU GEMV): two matrices of one shape, whose row blocks alternate in the stream: block 2j holds
// rows n0 + 16j .. +16 of w, block 2j + 1 the same rows of w2.
template <bool DUAL = false> struct GvStream {
  i32x4_t rw, rw2;
  int nrows, nrb, rowb, K, KC, ns, koff;
  int g0, kc, rb, st, islot;
  __device__ __forceinline__ void init(const View& w, int n0, int n1, int K_, int KC_, const View* w2 = nullptr) {
    nrows = rfl(n1 - n0); nrb = rfl(((nrows + 15) / 16) * (DUAL ? 2 : 1)); rowb = rfl(w.cols * 2); K = rfl(K_); KC = rfl(KC_); ns = KC / 256;
    koff = rfl(wave() * (KC / 4) * 2);
    rw = dma_rsrc((const void*)(w.h() + (long long)n0 * w.cols), ((long long)w.rows - n0) * w.cols * 2);
    if constexpr (DUAL) rw2 = dma_rsrc((const void*)(w2->h() + (long long)n0 * w2->cols), ((long long)w2->rows - n0) * w2->cols * 2);
    g0 = kc = rb = st = islot = 0;
  }
  __device__ __forceinline__ void advance() {
    if (g0 >= nrb) return;
    if (++st == ns) {
      st = 0;
      if (++rb == min(GV_GRP, nrb - g0)) { rb = 0; kc += KC; if (kc == K) { kc = 0; g0 += GV_GRP; } }
    }
    g0 = rfl(g0); kc = rfl(kc); rb = rfl(rb); st = rfl(st);
  }
  // Requests the next step into its ring slot (past the end: two loads beyond the descriptor's range).
  template <int R> __device__ __forceinline__ void issue(LDS char* ring) {
    LDS char* dst = ring + islot * GV_STEP;
    if constexpr (DUAL) {
      const int vb = g0 + rb;
      const int row = min((vb >> 1) * 16 + (lane() & 15), nrows - 1);
      const int off = g0 < nrb ? row * rowb + kc * 2 + koff + st * 128 + 16 * (lane() >> 4) : 0x7fff0000;
      const bool up = rfl(vb & 1) != 0;                                         // wave-uniform: the descriptor stays scalar
      const i32x4_t r = {rfl(up ? rw2[0] : rw[0]), rfl(up ? rw2[1] : rw[1]), rfl(up ? rw2[2] : rw[2]), rfl(up ? rw2[3] : rw[3])};
      dma16(r, off, 0, dst);
      dma16(r, off + 64, 0, dst + 1024);
    } else {
      const int row = min((g0 + rb) * 16 + (lane() & 15), nrows - 1);
      const int off = g0 < nrb ? row * rowb + kc * 2 + koff + st * 128 + 16 * (lane() >> 4) : 0x7fff0000;
      dma16(rw, off, 0, dst);
      dma16(rw, off + 64, 0, dst + 1024);
    }
    islot = islot + 1 == R ? 0 : islot + 1;
    advance();
  }
  template <int R> __device__ __forceinline__ void skip() { islot = islot + 1 == R ? 0 : islot + 1; advance(); }
};

// The first steps of every wave's stream, into the ring of a task that will run with c.pre set. Called by all four
// waves with the task's record in c (op 134 or 301) before its dependencies are met; it reads only the weights and
// writes only the ring.
template <int R, bool DUAL = false>
__device__ __forceinline__ void gemv_prefetch_r(const View& w, int n0, int n1, int K, int M, LDS char* smem, const View* w2 = nullptr) {
  GvStream<DUAL> ws;
  ws.init(w, n0, n1, K, gv_geo(K, M, R).KC, w2);
  LDS char* ring = smem + wave() * R * GV_STEP;
#pragma unroll
  for (int j = 0; j < R; ++j) ws.template issue<R>(ring);
}
// Op 311's stream form: op 301's shapes with pro 1, both matrices bf16 of one shape.
__device__ __forceinline__ bool gemv_swiglu_ok(const Ctx& c) {
  const View wg = c.buf(2), wu = c.buf(3);
  return gemv_stream_ok(c.buf(0), View{nullptr, 0, 0, 0}, wg, c.buf(4), c.i(7), c.i(8), 1) && wu.dtype == 2 && wu.rows == wg.rows &&
         wu.cols == wg.cols;
}
__device__ __noinline__ void gemv_prefetch(const Ctx& c, int op) {
  if (op == 311) {
    if (!gemv_swiglu_ok(c)) return;
    const View wg = uniform_view(c.buf(2)), wu = uniform_view(c.buf(3));
    const int M = rfl(c.i(8)), K = rfl(c.i(7)), n0 = rfl(c.i(5)), n1 = rfl(c.i(6)), R = gv_pre_ring(M);
    if (R == 12) gemv_prefetch_r<12, true>(wg, n0, n1, K, M, c.smem, &wu);
    else if (R == 8) gemv_prefetch_r<8, true>(wg, n0, n1, K, M, c.smem, &wu);
    else gemv_prefetch_r<4, true>(wg, n0, n1, K, M, c.smem, &wu);
    return;
  }
  const View x = c.buf(0), x2 = c.buf(1), w = uniform_view(c.buf(3)), out = c.buf(4);
  const bool rows = op == 301;
  const int M = rfl(rows ? c.i(9) : 1), pro = rows ? c.i(10) : c.i(9), K = rfl(c.i(8)), n0 = rfl(c.i(6)), n1 = rfl(c.i(7));
  if (!gemv_stream_ok(x, x2, w, out, K, M, pro)) return;
  const int R = gv_pre_ring(M);
  if (R == 12) gemv_prefetch_r<12>(w, n0, n1, K, M, c.smem);
  else if (R == 8) gemv_prefetch_r<8>(w, n0, n1, K, M, c.smem);
  else gemv_prefetch_r<4>(w, n0, n1, K, M, c.smem);
}

// The streaming GEMV of ops 134 / 301; DUAL: op 311 (x, gamma, wg, wu, out, n0, n1, K, M, eps), whose output row n is
// silu(g) * u with g and u the sums of its gate and up row blocks.
template <int R, bool DUAL = false> __device__ __forceinline__ void gemv_body(const Ctx& c, int M_, int pro_, float eps) {
  const int M = rfl(M_), pro = DUAL ? 1 : rfl(pro_);                            // function arguments arrive in VGPRs
  constexpr int BX = 0, BX2 = 1, BG = DUAL ? 1 : 2, BW = DUAL ? 2 : 3, BO = 4, IA = DUAL ? 5 : 6;
  const View x = uniform_view(c.buf(BX)), x2 = DUAL ? View{nullptr, 0, 0, 0} : uniform_view(c.buf(BX2)), g = uniform_view(c.buf(BG));
  const View w = uniform_view(c.buf(BW)), w2 = DUAL ? uniform_view(c.buf(3)) : View{nullptr, 0, 0, 0};
  const View out = uniform_view(c.buf(BO)), res = DUAL ? View{nullptr, 0, 0, 0} : uniform_view(c.buf(5));
  const int n0 = rfl(c.i(IA)), n1 = rfl(c.i(IA + 1)), K = rfl(c.i(IA + 2));
  const GvGeo geo = gv_geo(K, M, R);
  const int KC = geo.KC, VS = geo.VS, PM = 16 * M;
  LDS uint16_t* vs = (LDS uint16_t*)(c.smem + geo.vs_off);                     // [M][VS]
  LDS float* rstd = (LDS float*)(c.smem + geo.rstd_off);                       // [16]
  LDS float* part = (LDS float*)(c.smem + geo.part_off);                       // [4][GV_GRP][M][16]
  const int l = lane(), wv = wave(), nrows = n1 - n0, nrb = ((nrows + 15) / 16) * (DUAL ? 2 : 1);   // stream row blocks
  LDS char* ring = c.smem + wv * R * GV_STEP;
  GvStream<DUAL> ws;
  ws.init(w, n0, n1, K, KC, &w2);
  if (rfl(c.pre)) {
#pragma unroll
    for (int j = 0; j < R; ++j) ws.template skip<R>();                           // issued before the dependency wait
  } else {
#pragma unroll
    for (int j = 0; j < R; ++j) ws.template issue<R>(ring);                     // weights first: they do not wait for x
  }
  Ld4 lx, lx2, lg;
  lx.init(x); lx2.init(x2); lg.init(g);
  const bool arow = (l & 15) < M;
  const LDS uint16_t* va = vs + (arow ? (l & 15) : 0) * VS + 8 * (l >> 4);     // rows >= M read row 0 and are zeroed
  const LDS char* rl = ring + 16 * l;
  // With KC == K the staged v covers all of K and serves every row group. A single row with the RMSNorm prologue
  // is then staged in one pass (statistics and v from the same loads).
  const bool once = KC == K, rms1 = once && pro == 1 && M == 1 && K / 4 <= 4 * KVM_THREADS;
  if (rms1) gv_stage_rms1<4>(lx, lg, K, eps, vs, rstd + 4);
  else if (pro == 1) gv_rstd<8>(lx, x.cols, M, K, eps, rstd);                   // rstd of each row over all of K
  int cslot = 0;                                                                // ring slot of the next step consumed
  for (int g0 = 0; g0 < nrb; g0 += GV_GRP) {
    const int ng = min(GV_GRP, nrb - g0);
    for (int e = l; e < ng * PM; e += 64) part[(wv * GV_GRP) * PM + e] = 0.f;
    for (int kc = 0; kc < K; kc += KC) {
      const int kq = KC / 4, ns = kq / 64;
      __syncthreads();                                                          // rstd ready; the previous chunk's readers are done
      if (!rms1 && (!once || g0 == 0)) {                                        // v = bf16(prologue(x)), this chunk
        if (pro == 1) gv_stage<1, GV_SB>(lx, lg, x.cols, 0, M, kc, KC, VS, vs, rstd);
        else if (pro == 2) gv_stage<2, GV_SB>(lx, lx2, x.cols, x2.cols, M, kc, KC, VS, vs, rstd);
        else gv_stage<0, 2 * GV_SB>(lx, lx, x.cols, 0, M, kc, KC, VS, vs, rstd);
      }
      __syncthreads();
      const LDS uint16_t* vk = va + wv * kq;
      // One flat loop over the group's steps (row block rb, step st): a nested loop's header is where the compiler
      // places a full vmcnt wait, which would drain the ring once per row block.
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      int rb = 0, st = 0;
      for (int tt = 0; tt < ng * ns; ++tt) {
        wait_vm_c<2 * (R - 1)>();                                               // this step's two loads have landed
        const LDS char* slot = rl + cslot * GV_STEP;
        const u16x8_t w0 = *(const LDS u16x8_t*)slot, w1 = *(const LDS u16x8_t*)(slot + 1024);
        const u16x8_t a0 = *(const LDS u16x8_t*)(vk + st * 64), a1 = *(const LDS u16x8_t*)(vk + st * 64 + 32);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8_t)(arow ? a0 : u16x8_t{}), (bf16x8_t)w0, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16((bf16x8_t)(arow ? a1 : u16x8_t{}), (bf16x8_t)w1, acc, 0, 0, 0);
        wait_lds();                                                             // the slot's reads are done before it is refilled
        ws.template issue<R>(ring);
        cslot = cslot + 1 == R ? 0 : cslot + 1;
        if (++st == ns) {           // row block done. D[m][n]: lane holds m = 4 (l / 16) + i, n = l % 16; m >= M padding
          LDS float* pp = part + (wv * GV_GRP + rb) * PM + (l & 15);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = 4 * (l >> 4) + i;
            if (m < M) pp[m * 16] += acc[i];
          }
          acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
          st = 0; ++rb;
        }
      }
    }
    __syncthreads();
    if constexpr (DUAL) {                                                      // block pairs (gate, up): silu(g) u
      for (int e = tid(); e < (ng >> 1) * PM; e += KVM_THREADS) {
        const int rp = e / PM, m = (e / 16) % M, nn = e % 16, n = n0 + ((g0 >> 1) + rp) * 16 + nn;
        if (n >= n1) continue;
        const int eg = 2 * rp * PM + e % PM, eu = eg + PM;
        const float sg = (part[eg] + part[GV_GRP * PM + eg]) + (part[2 * GV_GRP * PM + eg] + part[3 * GV_GRP * PM + eg]);
        const float su = (part[eu] + part[GV_GRP * PM + eu]) + (part[2 * GV_GRP * PM + eu] + part[3 * GV_GRP * PM + eu]);
        out.st((long long)m * out.cols + n, silu_f(sg) * su);
      }
    } else {
      for (int e = tid(); e < ng * PM; e += KVM_THREADS) {                     // sum the four waves' tiles, in wave order
        const int rb = e / PM, m = (e / 16) % M, nn = e % 16, n = n0 + (g0 + rb) * 16 + nn;
        if (n >= n1) continue;
        const float s = (part[e] + part[GV_GRP * PM + e]) + (part[2 * GV_GRP * PM + e] + part[3 * GV_GRP * PM + e]);
        out.st((long long)m * out.cols + n, s + (res.ok() ? res.ld((long long)m * res.cols + n) : 0.f));
      }
    }
    if (g0 + GV_GRP < nrb) __syncthreads();                                    // the sums are read before the tiles are cleared
  }
  wait_vm_c<0>();                                                               // the ring's trailing loads have landed
}
template <int R, bool DUAL = false> __device__ __noinline__ void gemv_stream_r(const Ctx& c, int M, int pro, float eps) {
  gemv_body<R, DUAL>(c, M, pro, eps);
}
template <bool DUAL = false> __device__ __noinline__ void gemv_stream(const Ctx& c, int M, int pro, float eps) {
  if (!rfl(c.pre)) gemv_stream_r<GV_R, DUAL>(c, M, pro, eps);
  else {
    const int R = gv_pre_ring(rfl(M));
    if (R == 12) gemv_stream_r<12, DUAL>(c, M, pro, eps);
    else if (R == 8) gemv_stream_r<8, DUAL>(c, M, pro, eps);
    else gemv_stream_r<4, DUAL>(c, M, pro, eps);
  }
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

// Op 311 (this executor's fused SwiGLU GEMV): out[m, n] = silu(g) * u for n in [n0, n1), g / u the RMSNorm-prologue
// GEMV sums of row n of wg / wu (each exactly as op 301 with pro 1 computes it), rounded once as out stores. The
// validator admits only the stream form's shapes.
__device__ __noinline__ void op_gemv_swiglu(const Ctx& c) {
  if (gemv_swiglu_ok(c)) gemv_stream<true>(c, c.i(8), 1, c.f(9));
  else c.fail(KVM_ERR_OP_SHAPE, c.i(7), c.i(8));
}

}  // namespace kvm
