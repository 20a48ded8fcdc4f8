// GEMM tile operators: C tile at (m0, n0) of alpha*op(A)*op(B) with the registry's epilogue
// (bias -> pre -> gelu | dgelu -> res -> accumulate; reference: runtime/ref_gpt.py:69-95, include/mvm_ops_gpt.def op 34).
//   * matmul_tile (f32): exact fp32 SIMT FMA tiles. CDNA4 has no TF32, so flags 16 / 256 / 1024 give the same exact-fp32
//     products (more accurate than the reference's 1xTF32 default).
//   * matmul_tile_bf16 / matmul_mma_bf16: bf16 operands on the MFMA units (v_mfma_f32_32x32x16_bf16), fp32 accumulation,
//     one RNE rounding per stored bf16 value. Operands are staged through LDS in [row][k] layout so each lane feeds the
//     MFMA with one 16-byte LDS read; the next K slab is fetched from HBM into registers while the current one is
//     multiplied (double-buffered LDS).
#pragma once
#include "common.h"
#include "ops_basic.h"

namespace kvm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------------------------- epilogue
struct Epi {
  View out, bias, res, pre; float alpha; int accum, ge, dg;
  __device__ void put(int m, int n, float acc) const {
    float v = acc * alpha;
    if (bias.ok()) v += bias.f()[n];
    if (dg) v *= gelu_grad_f(pre.at(m, n));
    else {
      if (pre.ok()) pre.st((long long)m * pre.cols + n, v);
      if (ge) v = gelu_f(v);
    }
    if (res.ok()) v += res.at(m, n);
    long long o = (long long)m * out.cols + n;
    out.st(o, accum ? out.ld(o) + v : v);
  }
};

// ---------------------------------------------------------------------------------------------- fp32 SIMT tile
// 64x64 output block, 256 threads x (4x4) outputs, K in slabs of 16 through LDS. Operand access handles both
// storage orders; accumulation is fp32 FMA in increasing k.
__device__ void f32_block(const Ctx& c, View A, View B, int ta, int tb, int m0, int n0, int M, int N, int K, const Epi& e, bool bf16ops,
                          LDS float* out_tile /* optional: write raw alpha*acc here [64*64] instead of the epilogue */) {
  LDS float* As = (LDS float*)c.smem;    // [16][65]
  LDS float* Bs = As + 16 * 65;          // [16][65]
  int tx = tid() % 16, ty = tid() / 16;  // thread owns rows ty*4.., cols tx*4..
  float acc[4][4] = {};
  for (int k0 = 0; k0 < K; k0 += 16) {
    __syncthreads();
    for (int e2 = tid(); e2 < 16 * 64; e2 += KVM_THREADS) {
      int kk = e2 / 64, mm = e2 % 64, m = m0 + mm, k = k0 + kk;
      float a = (m < M && k < K) ? (ta ? A.at(k, m) : A.at(m, k)) : 0.f;
      int n = n0 + mm;
      float b = (n < N && k < K) ? (tb ? B.at(n, k) : B.at(k, n)) : 0.f;
      if (bf16ops) { a = round_bf(a); b = round_bf(b); }
      As[kk * 65 + mm] = a; Bs[kk * 65 + mm] = b;
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < 16; ++kk) {
      float a[4], b[4];
      for (int i = 0; i < 4; ++i) { a[i] = As[kk * 65 + ty * 4 + i]; b[i] = Bs[kk * 65 + tx * 4 + i]; }
      for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
  }
  for (int i = 0; i < 4; ++i) for (int j = 0; j < 4; ++j) {
    int m = m0 + ty * 4 + i, n = n0 + tx * 4 + j;
    if (m < M && n < N) {
      if (out_tile) out_tile[(ty * 4 + i) * 64 + tx * 4 + j] = acc[i][j] * e.alpha;
      else e.put(m, n, acc[i][j]);
    }
  }
  __syncthreads();
}

__device__ __forceinline__ int tile_m(int fl) { return fl & 64 ? 256 : fl & 32 ? 128 : 64; }
__device__ __forceinline__ int tile_n(int fl) { return (fl & 96) ? 128 : 64; }

__device__ __noinline__ void op_matmul_tile(const Ctx& c) {
  View A = c.buf(0), B = c.buf(1);
  int m0 = c.i(6), n0 = c.i(7), M = c.i(8), N = c.i(9), K = c.i(10), fl = c.i(11);
  Epi e{c.buf(2), c.buf(3), c.buf(4), c.buf(5), c.f(12), fl & 4, fl & 8, fl & 512};
  int tm = tile_m(fl), tn = tile_n(fl);
  for (int dm = 0; dm < tm; dm += 64) for (int dn = 0; dn < tn; dn += 64)
    if (m0 + dm < M && n0 + dn < N) f32_block(c, A, B, fl & 1, fl & 2, m0 + dm, n0 + dn, M, N, K, e, false, nullptr);
}

// SwiGLU epilogue wrappers: the raw tile lands in LDS, then the elementwise pass (registry ops 120 / 121).
__device__ __noinline__ void op_matmul_tile_silu_mul(const Ctx& c) {
  View A = c.buf(0), B = c.buf(1), out = c.buf(2), gate = c.buf(3), up = c.buf(4);
  int m0 = c.i(5), n0 = c.i(6), M = c.i(7), N = c.i(8), K = c.i(9), fl = c.i(10);
  Epi e{}; e.alpha = c.f(11);
  LDS float* t = (LDS float*)(c.smem + 32 * 1024);
  for (int dm = 0; dm < tile_m(fl); dm += 64) for (int dn = 0; dn < tile_n(fl); dn += 64) {
    int bm = m0 + dm, bn = n0 + dn;
    if (bm >= M || bn >= N) continue;
    f32_block(c, A, B, fl & 1, fl & 2, bm, bn, M, N, K, e, false, t);
    for (int q = tid(); q < 64 * 64; q += KVM_THREADS) {
      int m = bm + q / 64, n = bn + q % 64;
      if (m < M && n < N) { float u = t[q]; up.f()[(long long)m * up.cols + n] = u; out.f()[(long long)m * out.cols + n] = silu_f(gate.at(m, n)) * u; }
    }
    __syncthreads();
  }
}
__device__ __noinline__ void op_matmul_tile_silu_mul_bwd(const Ctx& c) {
  View A = c.buf(0), B = c.buf(1), gate = c.buf(2), up = c.buf(3), dg = c.buf(4), du = c.buf(5);
  int m0 = c.i(6), n0 = c.i(7), M = c.i(8), N = c.i(9), K = c.i(10), fl = c.i(11);
  Epi e{}; e.alpha = c.f(12);
  LDS float* t = (LDS float*)(c.smem + 32 * 1024);
  for (int dm = 0; dm < tile_m(fl); dm += 64) for (int dn = 0; dn < tile_n(fl); dn += 64) {
    int bm = m0 + dm, bn = n0 + dn;
    if (bm >= M || bn >= N) continue;
    f32_block(c, A, B, fl & 1, fl & 2, bm, bn, M, N, K, e, false, t);
    for (int q = tid(); q < 64 * 64; q += KVM_THREADS) {
      int m = bm + q / 64, n = bn + q % 64;
      if (m < M && n < N) {
        float dh = t[q], g = gate.at(m, n);
        dg.f()[(long long)m * dg.cols + n] = dh * (up.at(m, n) * silu_d_f(g));
        du.f()[(long long)m * du.cols + n] = dh * silu_f(g);
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------- bf16 MFMA engine
// Loads 8 consecutive elements (along the operand's contiguous dimension) as bf16 bits; out-of-range -> 0.
__device__ __forceinline__ u16x8_t load8(const View& X, long long base, int valid) {
  u16x8_t r;
  if (valid >= 8 && (base & 7) == 0) {
    if (X.dtype == 2) return *(const GLOBAL u16x8_t*)(X.h() + base);
    const GLOBAL f32x4n* p = (const GLOBAL f32x4n*)(X.f() + base);
    f32x4n a = p[0], b = p[1];
    r[0] = f2bf(a.x); r[1] = f2bf(a.y); r[2] = f2bf(a.z); r[3] = f2bf(a.w);
    r[4] = f2bf(b.x); r[5] = f2bf(b.y); r[6] = f2bf(b.z); r[7] = f2bf(b.w);
    return r;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = i < valid ? (X.dtype == 2 ? X.h()[base + i] : f2bf(X.f()[base + i])) : (uint16_t)0;
  return r;
}

// One operand tile of R rows x KT k values, staged to LDS as [row][k] with a padded row stride.
//   trans == 0: element (r, k) at X[r*ld + k] (k contiguous): thread vectors run along k, one 16-byte LDS store each.
//   trans == 1: element (r, k) at X[k*ld + r] (r contiguous): a vector holds 8 consecutive rows at one k; consecutive
//     lanes take consecutive k so the eight 2-byte LDS stores of a vector hit consecutive addresses (no bank
//     conflicts), at the price of 16-byte global loads from different rows (each 128-byte line is still read whole by
//     the tile).
// `fast` (uniform per task): bf16 storage, 16-byte aligned rows, the whole tile in range: every load is
// unconditional, so all of a thread's loads are in flight together.
template <int R, int KT> struct Stage {
  static constexpr int STRIDE = KT + 8;                   // elements; +16 B per row spreads rows over LDS banks
  static constexpr int VEC = R * KT / 8;                  // 8-element vectors per tile
  static constexpr int PER = (VEC + KVM_THREADS - 1) / KVM_THREADS;
  u16x8_t v[PER];
  __device__ void fetch(const View& X, int trans, int r0, int rows, int k0, int K, bool fast) {
    if (fast) {
      const GLOBAL uint16_t* base = X.h();
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int idx = tid() + q * KVM_THREADS;
        if (VEC % KVM_THREADS != 0 && idx >= VEC) break;
        if (!trans) {
          const int row = idx / (KT / 8), kv = idx % (KT / 8);
          v[q] = *(const GLOBAL u16x8_t*)(base + (long long)(r0 + row) * X.cols + k0 + kv * 8);
        } else {
          const int k = idx % KT, rv = idx / KT;
          v[q] = *(const GLOBAL u16x8_t*)(base + (long long)(k0 + k) * X.cols + r0 + rv * 8);
        }
      }
      return;
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      int idx = tid() + q * KVM_THREADS;
      if (idx >= VEC) break;
      if (!trans) {
        int row = idx / (KT / 8), kv = idx % (KT / 8), r = r0 + row, k = k0 + kv * 8;
        int valid = (r < rows) ? min(8, K - k) : 0;
        v[q] = load8(X, (long long)r * X.cols + k, valid);
      } else {
        int k = idx % KT, rv = idx / KT, kk = k0 + k, r = r0 + rv * 8;
        int valid = (kk < K) ? min(8, rows - r) : 0;
        v[q] = load8(X, (long long)kk * X.cols + r, valid);
      }
    }
  }
  __device__ void store(LDS uint16_t* lds, int trans) const {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      int idx = tid() + q * KVM_THREADS;
      if (VEC % KVM_THREADS != 0 && idx >= VEC) break;
      if (!trans) {
        int row = idx / (KT / 8), kv = idx % (KT / 8);
        *(LDS u16x8_t*)(lds + row * STRIDE + kv * 8) = v[q];
      } else {
        int k = idx % KT, rv = idx / KT;
#pragma unroll
        for (int i = 0; i < 8; ++i) lds[(rv * 8 + i) * STRIDE + k] = v[q][i];
      }
    }
  }
};

// Whether an operand tile can take the unconditional fast path (see Stage).
__device__ __forceinline__ bool fast_operand(const View& X, int trans, int r0, int R, int rows, int K, int KT) {
  if (X.dtype != 2 || (X.cols & 7) || (((uintptr_t)X.p) & 15) || (K % KT)) return false;
  return r0 + R <= rows && (!trans || (r0 & 7) == 0);
}

// TM x TN output tile at (m0, n0); waves in a 2 x 2 grid, each owning (TM/2) x (TN/2) as 32x32 MFMA blocks.
template <int TM, int TN> __device__ __noinline__ void mfma_tile(const Ctx& c, View A, View B, int ta, int tb, int m0, int n0, int M, int N,
                                                                  int K, const Epi& e) {
  constexpr int KT = 32, WM = TM / 2, WN = TN / 2, BM = WM / 32, BN = WN / 32;
  typedef Stage<TM, KT> SA;
  typedef Stage<TN, KT> SB;
  LDS uint16_t* lA[2] = {(LDS uint16_t*)c.smem, (LDS uint16_t*)c.smem + TM * SA::STRIDE};
  LDS uint16_t* lB[2] = {lA[1] + TM * SA::STRIDE, lA[1] + TM * SA::STRIDE + TN * SB::STRIDE};
  const int wm0 = (wave() >> 1) * WM, wn0 = (wave() & 1) * WN, l = lane();
  const bool fa = fast_operand(A, ta, m0, TM, M, K, KT), fb = fast_operand(B, !tb, n0, TN, N, K, KT);
  f32x16 acc[BM][BN];
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j) acc[i][j] = f32x16{};
  SA sa; SB sb;
  sa.fetch(A, ta, m0, M, 0, K, fa);
  sb.fetch(B, !tb, n0, N, 0, K, fb);
  __syncthreads();                        // LDS may still be read by the previous tile / task
  sa.store(lA[0], ta); sb.store(lB[0], !tb);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < K; k0 += KT) {
    bool more = k0 + KT < K;
    if (more) { sa.fetch(A, ta, m0, M, k0 + KT, K, fa); sb.fetch(B, !tb, n0, N, k0 + KT, K, fb); }
    __builtin_amdgcn_sched_barrier(0);     // the next slab's loads are in flight during this slab's MFMAs
#pragma unroll
    for (int kk = 0; kk < KT; kk += 16) {
      bf16x8 af[BM], bfr[BN];
#pragma unroll
      for (int i = 0; i < BM; ++i) af[i] = *(const LDS bf16x8*)(lA[buf] + (wm0 + i * 32 + (l & 31)) * SA::STRIDE + kk + (l >> 5) * 8);
#pragma unroll
      for (int j = 0; j < BN; ++j) bfr[j] = *(const LDS bf16x8*)(lB[buf] + (wn0 + j * 32 + (l & 31)) * SB::STRIDE + kk + (l >> 5) * 8);
#pragma unroll
      for (int i = 0; i < BM; ++i)
#pragma unroll
        for (int j = 0; j < BN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) { sa.store(lA[buf ^ 1], ta); sb.store(lB[buf ^ 1], !tb); }
    __syncthreads();
    buf ^= 1;
  }
  // D layout of a 32x32 block: column = lane % 32, row = 8*(r/4) + 4*(lane/32) + r%4 for accumulator register r.
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int m = m0 + wm0 + i * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3), n = n0 + wn0 + j * 32 + (l & 31);
        if (m < M && n < N) e.put(m, n, acc[i][j][r]);
      }
}

// Note on operand orientation: the LDS tile of B is [n][k]. B stored [N,K] (flag 2) is read row-contiguous (trans 0 in
// Stage terms); B stored [K,N] is read column-wise (trans 1).
__device__ __noinline__ void op_matmul_tile_bf16(const Ctx& c) {
  View A = c.buf(0), B = c.buf(1);
  int m0 = c.i(6), n0 = c.i(7), M = c.i(8), N = c.i(9), K = c.i(10), fl = c.i(11);
  Epi e{c.buf(2), c.buf(3), c.buf(4), c.buf(5), c.f(12), fl & 4, fl & 8, fl & 512};
  if (fl & 64) mfma_tile<256, 128>(c, A, B, fl & 1, (fl & 2) != 0, m0, n0, M, N, K, e);
  else if (fl & 32) mfma_tile<128, 128>(c, A, B, fl & 1, (fl & 2) != 0, m0, n0, M, N, K, e);
  else mfma_tile<64, 64>(c, A, B, fl & 1, (fl & 2) != 0, m0, n0, M, N, K, e);
}
__device__ __noinline__ void op_matmul_mma_bf16(const Ctx& c) {
  View A = c.buf(0), B = c.buf(1);
  int m0 = c.i(6), n0 = c.i(7), M = c.i(8), N = c.i(9), K = c.i(10), fl = c.i(11);
  Epi e{c.buf(2), c.buf(3), c.buf(4), c.buf(5), c.f(12), fl & 4, fl & 8, fl & 512};
  mfma_tile<128, 256>(c, A, B, fl & 1, (fl & 2) != 0, m0, n0, M, N, K, e);
}

}  // namespace kvm
