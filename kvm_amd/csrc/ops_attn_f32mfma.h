// Causal flash attention on the MFMA units for f32 storage (registry ops 45, 47, 48; reference semantics:
// runtime/ref_gpt.py:279-364), with v_mfma_f32_32x32x2f32: every product is an exact f32 product accumulated in f32,
// the same arithmetic class as the SIMT bodies in ops_attn.h, which take the shapes this form does not (T not a
// multiple of 64, hd other than 32 / 64 / 128, head slices not 16-byte aligned).
//
// The scheme is the bf16 form's (ops_attn_mfma.h), "transposed space": S^T = K Q^T puts the softmax axis on the
// MFMA's row axis, so lane l owns query (or key) l % 32 and the accumulator register r holds row 8 (r / 4) + 4 (l / 32)
// + r % 4 of its 32-row block. With k = 2 per instruction:
//   * the products over the head dimension give lane half g = l / 32 the dims g hd/2 .. g hd/2 + hd/2 - 1 (a dot
//     product does not depend on the order of its terms): the register operand (Q, dO, K or V of the lane's own row)
//     is hd/2 floats per lane, and the LDS operand is read 4 dims at a time (one 16-byte read per 4 MFMAs);
//   * the products over the softmax axis (P V, dS K, ...) take the accumulator registers themselves as the B operand:
//     step r pairs the rows 8 (r / 4) + r % 4 (lanes 0-31) and + 4 (lanes 32-63), and the A operand is one float per
//     lane, read from the staged block at (that row, dim l % 32).
// Blocks of 64 rows go from HBM straight into LDS (buffer_load ... lds), FA_NS stages (2 at hd 128). A row's 16-byte
// units are XOR-swizzled by row: 8 consecutive rows read at one unit (the 16-byte reads) are conflict-free, and rows
// r and r + 4 (the two halves of a one-float read) land on different banks from hd 64 up.
#pragma once
#include "common.h"
#include "ops_gemm.h"
#include "ops_attn_mfma.h"

namespace kvm {

template <int HD> struct FaF {
  static constexpr int UPR = HD / 4;                                   // 16-byte units per row
  static constexpr int NL = FA_KB * HD * 4 / 1024 / KVM_WAVES;         // direct loads per thread per 64-row block
  static constexpr int NS = HD <= 64 ? FA_NS : 2;                      // stages
  static_assert(NL >= 1 && NS * 2 * FA_KB * HD * 4 <= KVM_LDS_BYTES, "hd");
  __device__ static __forceinline__ int swz(int row) { return UPR >= 16 ? ((row & 7) ^ (((row >> 2) & 1) << 3)) : (row & 7); }
  __device__ static __forceinline__ int at(int row, int col) { return row * HD + 4 * ((col >> 2) ^ swz(row)) + (col & 3); }
  // Direct loads of rows [row0, row0 + 64), columns [c0, c0 + HD) of an f32 matrix with `cols` columns (descriptor rs).
  __device__ static __forceinline__ void issue(LDS float* dst, i32x4_t rs, int row0, int cols, int c0) {
#pragma unroll
    for (int q = 0; q < NL; ++q) {
      const int b = q * KVM_WAVES + wave(), u = 64 * b + lane(), row = u / UPR, pos = u % UPR;
      dma16(rs, ((row0 + row) * cols + c0 + 4 * (pos ^ swz(row))) * 4, 0, dst + b * 256);
    }
  }
  // S-type product over the head dims: acc += A (32 staged rows rb.., dims of lane half g) x B (the lane's register row).
  __device__ static __forceinline__ void dot(f32x16& acc, const LDS float* s, int rb, const float (&reg)[HD / 2]) {
    const int l = lane(), g = l >> 5, r = rb + (l & 31);
#pragma unroll
    for (int s4 = 0; s4 < HD / 8; ++s4) {
      const f32x4n a = *(const LDS f32x4n*)(s + at(r, g * (HD / 2) + 4 * s4));
#pragma unroll
      for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t], reg[4 * s4 + t], acc, 0, 0, 0);
    }
  }
  // Product over 32 staged rows rb.. (the accumulator's row order): acc (dims db.. x lane rows) += staged^T x w.
  __device__ static __forceinline__ void axpy(f32x16& acc, const LDS float* s, int rb, int db, const f32x16& wv) {
    const int l = lane(), g = l >> 5, d = db + (l & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = rb + 8 * (r >> 2) + 4 * g + (r & 3);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(s[at(row, d)], wv[r], acc, 0, 0, 0);
    }
  }
};

__device__ __forceinline__ bool fa_ok_f32(const View& x, int T) {
  return x.ok() && x.dtype == 0 && (x.cols % 4) == 0 && (long long)T * x.cols * 4 < 0x7fffffffll;
}

// Forward for 128 queries of head h: lane l of wave w owns query q0 + 32 w + l % 32.
template <int HD> __device__ __noinline__ void attn_fwd_f32mfma(const Ctx& c) {
  typedef FaF<HD> L;
  constexpr int NDB = HD / 32, HH = HD / 2, NS = L::NS, ST = 2 * FA_KB * HD;
  const View q = uview(c, 0), k = uview(c, 1), v = uview(c, 2), o = uview(c, 3), lse = uview(c, 4);
  const int bb = rfl(c.i(5)), h = rfl(c.i(6)), q0 = rfl(c.i(7)), T = rfl(c.i(8)), H = rfl(c.i(9)), Hkv = rfl(c.i(10));
  const float sl2 = __int_as_float(rfl(__float_as_int(c.f(12)))) * 1.4426950408889634f;   // scale * log2(e)
  const int w = wave(), l = lane(), g = l >> 5, qi = l & 31;
  const int qrow = q0 + 32 * w + qi, kvh = h / (H / Hkv);
  const bool qok = qrow < T;
  float qf[HH];
#pragma unroll
  for (int s4 = 0; s4 < HH / 4; ++s4) {
    const f32x4n x = qok ? *(const GLOBAL f32x4n*)(q.f() + ((long long)bb * T + qrow) * q.cols + h * HD + g * HH + 4 * s4) : f32x4n{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t) qf[4 * s4 + t] = x[t];
  }
  const int kend = min(T, q0 + 128), nkb = (kend + FA_KB - 1) / FA_KB;
  const int wlast = min(T - 1, q0 + 32 * w + 31);
  const i32x4_t rk = dma_rsrc((const void*)(k.f() + (long long)bb * T * k.cols), (long long)T * k.cols * 4);
  const i32x4_t rv = dma_rsrc((const void*)(v.f() + (long long)bb * T * v.cols), (long long)T * v.cols * 4);
  LDS float* lds = (LDS float*)c.smem;
  f32x16 oacc[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) oacc[d] = f32x16{};
  float m = -INFINITY, lsum = 0.f;
  __syncthreads();                                         // the previous task may still read this LDS
#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < nkb) { L::issue(lds + p * ST, rk, p * FA_KB, k.cols, kvh * HD); L::issue(lds + p * ST + FA_KB * HD, rv, p * FA_KB, v.cols, kvh * HD); }
  for (int kb = 0; kb < nkb; ++kb) {
    wait_vm(min(NS - 2, nkb - 1 - kb) * 2 * L::NL);
    __syncthreads();
    if (kb + NS - 1 < nkb) {
      LDS float* nb = lds + ((kb + NS - 1) % NS) * ST;
      L::issue(nb, rk, (kb + NS - 1) * FA_KB, k.cols, kvh * HD);
      L::issue(nb + FA_KB * HD, rv, (kb + NS - 1) * FA_KB, v.cols, kvh * HD);
    }
    if (kb * FA_KB > wlast) continue;                      // every key of the block is after this wave's queries
    const LDS float* Ks = lds + (kb % NS) * ST;
    const LDS float* Vs = Ks + FA_KB * HD;
    f32x16 s[2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) { s[sb] = f32x16{}; L::dot(s[sb], Ks, sb * 32, qf); }
    float mloc = -INFINITY;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb * FA_KB + sb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        const float x = key > qrow ? -INFINITY : s[sb][r] * sl2;
        s[sb][r] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float mn = fmaxf(m, mloc), f = __builtin_amdgcn_exp2f(m - mn);
    float ps = 0.f;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) { s[sb][r] = __builtin_amdgcn_exp2f(s[sb][r] - mn); ps += s[sb][r]; }
    ps += __shfl_xor(ps, 32, 64);
    lsum = lsum * f + ps;
    m = mn;
#pragma unroll
    for (int d = 0; d < NDB; ++d) {
      oacc[d] *= f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) L::axpy(oacc[d], Vs, sb * 32, d * 32, s[sb]);
    }
  }
  if (qok) {
    const float inv = 1.f / lsum;
    GLOBAL float* orow = o.f() + ((long long)bb * T + qrow) * o.cols + h * HD + 4 * g;
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        stwt_f4(orow + d * 32 + 8 * rq, f32x4n{oacc[d][4 * rq] * inv, oacc[d][4 * rq + 1] * inv, oacc[d][4 * rq + 2] * inv, oacc[d][4 * rq + 3] * inv});
    if (g == 0) stwt32(lse.f() + (((long long)bb * H + h) * T + qrow), (m + log2f(lsum)) * 0.6931471805599453f);
  }
}

// dQ for 128 queries of head h (op 47): S^T = K Q^T, dP^T = V dO^T, P^T = exp(S^T scale - lse), dS^T = P^T (dP^T -
// delta), dQ^T += K^T dS^T, dq = scale dQ.
template <int HD> __device__ __noinline__ void attn_dq_f32mfma(const Ctx& c) {
  typedef FaF<HD> L;
  constexpr int NDB = HD / 32, HH = HD / 2, NS = L::NS, ST = 2 * FA_KB * HD;
  const View q = uview(c, 0), k = uview(c, 1), v = uview(c, 2), dO = uview(c, 3), lse = uview(c, 4), delta = uview(c, 5), dq = uview(c, 6);
  const int bb = rfl(c.i(7)), h = rfl(c.i(8)), q0 = rfl(c.i(9)), T = rfl(c.i(10)), H = rfl(c.i(11)), Hkv = rfl(c.i(12));
  const float sc = __int_as_float(rfl(__float_as_int(c.f(14)))), sl2 = sc * 1.4426950408889634f;
  const int w = wave(), l = lane(), g = l >> 5, qi = l & 31;
  const int qrow = q0 + 32 * w + qi, kvh = h / (H / Hkv);
  const bool qok = qrow < T;
  const long long grow = (long long)bb * T + qrow;
  float qf[HH], df[HH];
#pragma unroll
  for (int s4 = 0; s4 < HH / 4; ++s4) {
    const f32x4n z = f32x4n{0.f, 0.f, 0.f, 0.f};
    const f32x4n x = qok ? *(const GLOBAL f32x4n*)(q.f() + grow * q.cols + h * HD + g * HH + 4 * s4) : z;
    const f32x4n y = qok ? *(const GLOBAL f32x4n*)(dO.f() + grow * dO.cols + h * HD + g * HH + 4 * s4) : z;
#pragma unroll
    for (int t = 0; t < 4; ++t) { qf[4 * s4 + t] = x[t]; df[4 * s4 + t] = y[t]; }
  }
  const float l2 = qok ? lse.f()[((long long)bb * H + h) * T + qrow] * 1.4426950408889634f : 0.f;
  const float di = qok ? delta.f()[((long long)bb * H + h) * T + qrow] : 0.f;
  const int kend = min(T, q0 + 128), nkb = (kend + FA_KB - 1) / FA_KB;
  const int wlast = min(T - 1, q0 + 32 * w + 31);
  const i32x4_t rk = dma_rsrc((const void*)(k.f() + (long long)bb * T * k.cols), (long long)T * k.cols * 4);
  const i32x4_t rv = dma_rsrc((const void*)(v.f() + (long long)bb * T * v.cols), (long long)T * v.cols * 4);
  LDS float* lds = (LDS float*)c.smem;
  f32x16 acc[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) acc[d] = f32x16{};
  __syncthreads();
#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < nkb) { L::issue(lds + p * ST, rk, p * FA_KB, k.cols, kvh * HD); L::issue(lds + p * ST + FA_KB * HD, rv, p * FA_KB, v.cols, kvh * HD); }
  for (int kb = 0; kb < nkb; ++kb) {
    wait_vm(min(NS - 2, nkb - 1 - kb) * 2 * L::NL);
    __syncthreads();
    if (kb + NS - 1 < nkb) {
      LDS float* nb = lds + ((kb + NS - 1) % NS) * ST;
      L::issue(nb, rk, (kb + NS - 1) * FA_KB, k.cols, kvh * HD);
      L::issue(nb + FA_KB * HD, rv, (kb + NS - 1) * FA_KB, v.cols, kvh * HD);
    }
    if (kb * FA_KB > wlast) continue;
    const LDS float* Ks = lds + (kb % NS) * ST;
    const LDS float* Vs = Ks + FA_KB * HD;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      f32x16 sv = f32x16{}, dp = f32x16{};
      L::dot(sv, Ks, sb * 32, qf);
      L::dot(dp, Vs, sb * 32, df);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kb * FA_KB + sb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        const float pr = key > qrow ? 0.f : __builtin_amdgcn_exp2f(sv[r] * sl2 - l2);
        sv[r] = pr * (dp[r] - di);
      }
#pragma unroll
      for (int d = 0; d < NDB; ++d) L::axpy(acc[d], Ks, sb * 32, d * 32, sv);
    }
  }
  if (qok) {
    GLOBAL float* orow = dq.f() + grow * dq.cols + h * HD + 4 * g;
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        stwt_f4(orow + d * 32 + 8 * rq, f32x4n{acc[d][4 * rq] * sc, acc[d][4 * rq + 1] * sc, acc[d][4 * rq + 2] * sc, acc[d][4 * rq + 3] * sc});
  }
}

// dK / dV for 128 keys of kv head kvh (op 48), summed over the heads of its GQA group and every later query: lane l of
// wave w owns key k0 + 32 w + l % 32. S = Q K^T, dP = dO V^T (Q, dO staged; K, V in registers), P = exp(S scale -
// lse[q]), dS = P (dP - delta[q]), dV^T += dO^T P, dK^T += Q^T dS, dk = scale dK. The staged queries' lse / delta go
// to LDS by one 8-lane direct load per wave.
template <int HD> __device__ __noinline__ void attn_dkv_f32mfma(const Ctx& c) {
  typedef FaF<HD> L;
  constexpr int NDB = HD / 32, HH = HD / 2, NS = L::NS, BK = FA_KB * HD, ST = 2 * BK + 2 * FA_KB;   // + lse, delta
  static_assert(NS * ST * 4 <= KVM_LDS_BYTES, "LDS");
  const View q = uview(c, 0), k = uview(c, 1), v = uview(c, 2), dO = uview(c, 3), lse = uview(c, 4), delta = uview(c, 5);
  const View dk = uview(c, 6), dv = uview(c, 7);
  const int bb = rfl(c.i(8)), kvh = rfl(c.i(9)), k0 = rfl(c.i(10)), T = rfl(c.i(11)), H = rfl(c.i(12));
  const float sc = __int_as_float(rfl(__float_as_int(c.f(14)))), sl2 = sc * 1.4426950408889634f;
  const int G = H / (k.cols / HD);
  const int w = wave(), l = lane(), g = l >> 5, ki = l & 31;
  const int krow = k0 + 32 * w + ki;
  const bool kok = krow < T;
  const long long grow = (long long)bb * T + krow;
  float kf[HH], vf[HH];
#pragma unroll
  for (int s4 = 0; s4 < HH / 4; ++s4) {
    const f32x4n z = f32x4n{0.f, 0.f, 0.f, 0.f};
    const f32x4n x = kok ? *(const GLOBAL f32x4n*)(k.f() + grow * k.cols + kvh * HD + g * HH + 4 * s4) : z;
    const f32x4n y = kok ? *(const GLOBAL f32x4n*)(v.f() + grow * v.cols + kvh * HD + g * HH + 4 * s4) : z;
#pragma unroll
    for (int t = 0; t < 4; ++t) { kf[4 * s4 + t] = x[t]; vf[4 * s4 + t] = y[t]; }
  }
  const int qb0 = k0 / FA_KB, nqb = (T + FA_KB - 1) / FA_KB - qb0, nit = G * nqb;
  const int wfirst = k0 + 32 * w;
  const i32x4_t rq = dma_rsrc((const void*)(q.f() + (long long)bb * T * q.cols), (long long)T * q.cols * 4);
  const i32x4_t rd = dma_rsrc((const void*)(dO.f() + (long long)bb * T * dO.cols), (long long)T * dO.cols * 4);
  LDS float* lds = (LDS float*)c.smem;
  auto issue = [&](int it) {
    const int hh = kvh * G + it / nqb, qb = qb0 + it % nqb;
    LDS float* d = lds + (it % NS) * ST;
    L::issue(d, rq, qb * FA_KB, q.cols, hh * HD);
    L::issue(d + BK, rd, qb * FA_KB, dO.cols, hh * HD);
    const View& src = w < 2 ? lse : delta;              // waves 0, 1: lse[0:32], [32:64]; waves 2, 3: delta
    const i32x4_t rs = dma_rsrc((const void*)(src.f() + ((long long)bb * H + hh) * T), (long long)T * 4);
    if (l < 8) dma16(rs, (qb * FA_KB + 32 * (w & 1) + 4 * l) * 4, 0, d + 2 * BK + (w >> 1) * FA_KB + (w & 1) * 32);
  };
  f32x16 adk[NDB], adv[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) { adk[d] = f32x16{}; adv[d] = f32x16{}; }
  constexpr int NLS = 2 * L::NL + 1;
  __syncthreads();
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) if (p < nit) issue(p);
  for (int it = 0; it < nit; ++it) {
    wait_vm(min(NS - 2, nit - 1 - it) * NLS);
    __syncthreads();
    if (it + NS - 1 < nit) issue(it + NS - 1);
    const int qb = qb0 + it % nqb;
    if (qb * FA_KB + FA_KB - 1 < wfirst) continue;          // every query of the block is before this wave's keys
    const LDS float* Qs = lds + (it % NS) * ST;
    const LDS float* Ds = Qs + BK;
    const LDS float* Ls = Qs + 2 * BK;
    const LDS float* Es = Ls + FA_KB;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      f32x16 sv = f32x16{}, dp = f32x16{};
      L::dot(sv, Qs, sb * 32, kf);
      L::dot(dp, Ds, sb * 32, vf);
      f32x16 ds;
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int ql = sb * 32 + 8 * i4 + 4 * g;            // first of 4 consecutive queries in this register group
        const f32x4n lq = *(const LDS f32x4n*)(Ls + ql), eq = *(const LDS f32x4n*)(Es + ql);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 4 * i4 + j, qq = qb * FA_KB + ql + j;
          const float pr = qq < krow ? 0.f : __builtin_amdgcn_exp2f(sv[r] * sl2 - lq[j] * 1.4426950408889634f);
          sv[r] = pr;
          ds[r] = pr * (dp[r] - eq[j]);
        }
      }
#pragma unroll
      for (int d = 0; d < NDB; ++d) {
        L::axpy(adv[d], Ds, sb * 32, d * 32, sv);
        L::axpy(adk[d], Qs, sb * 32, d * 32, ds);
      }
    }
  }
  if (kok) {
    GLOBAL float* kr = dk.f() + grow * dk.cols + kvh * HD + 4 * g;
    GLOBAL float* vr = dv.f() + grow * dv.cols + kvh * HD + 4 * g;
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        stwt_f4(kr + d * 32 + 8 * rq, f32x4n{adk[d][4 * rq] * sc, adk[d][4 * rq + 1] * sc, adk[d][4 * rq + 2] * sc, adk[d][4 * rq + 3] * sc});
        stwt_f4(vr + d * 32 + 8 * rq, f32x4n{adv[d][4 * rq], adv[d][4 * rq + 1], adv[d][4 * rq + 2], adv[d][4 * rq + 3]});
      }
  }
}

}  // namespace kvm
