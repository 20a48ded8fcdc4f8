// Causal flash attention on the MFMA units for bf16 storage (registry ops 45, 47, 48; reference semantics:
// runtime/ref_gpt.py:279-364). Used when q, k, v, do, o, dq, dk, dv are bf16 storage with 16-byte aligned head
// slices, lse / delta are f32, T is a multiple of 64 and hd is 32, 64 or 128; other cases run the fp32 SIMT bodies
// in ops_attn.h.
//
// Scheme ("transposed space"): every product is computed with the reduction axis of the softmax on the MFMA's row
// axis, so that each lane owns one query (forward, dQ) or one key (dK/dV):
//   * S^T = K Q^T with v_mfma_f32_32x32x16_bf16 (A = 32 key rows, B = 32 query rows, k = head dim). The accumulator
//     holds D[key][query] with lane l owning query l % 32 and keys 8*(r/4) + 4*(l/32) + r%4 of its 32-key block:
//     the softmax statistics of a query live in lanes l and l ^ 32, combined with one lane exchange.
//   * O^T += V^T P^T: the bf16-rounded P^T accumulator registers are used directly as the B operand; the key order
//     inside each 16-key MFMA step is the one those registers already have (keys 0-3, 8-11 in lanes 0-31 and 4-7,
//     12-15 in lanes 32-63), and V^T is read in the same key order with LDS transpose reads. A dot product does not
//     depend on the order of its terms, so the permutation is free.
//   * O^T's accumulator has lane l owning query l % 32 again, so the online-softmax rescale is one multiply per
//     register and the output store is 4 consecutive head-dim elements per lane.
// Softmax exponentials are the hardware exp2 (v_exp_f32): every argument is <= 0 (a score minus the running max or the
// row's log-sum-exp), where it differs from the library exp2f only by flushing results below 2^-126 to zero.
// K/V (or Q/dO) blocks of 64 rows go from HBM straight into LDS (buffer_load ... lds), FA_NS stages deep. Each block
// is kept in one of two swizzled layouts: "kc" for MFMA operands read along the head dim (ds_read_b128), "tr" for
// operands read across rows (ds_read_b64_tr_b16); see ops_gemm.h for the transpose-read semantics.
#pragma once
#include "common.h"
#include "ops_gemm.h"

namespace kvm {

constexpr int FA_KB = 64;      // rows (keys or queries) per stage
constexpr int FA_NS = 3;       // stages (prefetch distance FA_NS - 1)

template <int HD> struct FaL {
  static constexpr int UPR = HD / 8;                       // 16-byte units per row
  static constexpr int NL = FA_KB * HD * 2 / 1024 / KVM_WAVES;   // direct loads per thread per 64-row block
  static_assert(NL >= 1, "hd");
  // kc layout: 16 consecutive rows reading one unit hit every bank once
  __device__ static __forceinline__ int kswz(int row) { return (row / (16 / UPR)) % UPR; }
  // tr layout: 4 consecutive rows (row % 4 == 0) x 32 bytes per 16-lane group, 32 lanes per pass, conflict-free
  __device__ static __forceinline__ int tswz(int row) { return UPR >= 16 ? 4 * (row & 3) : UPR == 8 ? 4 * ((row >> 1) & 1) : 0; }
  __device__ static __forceinline__ int kc(int row, int unit) { return row * HD + 8 * (unit ^ kswz(row)); }
  __device__ static __forceinline__ int tr(int row, int col) { return row * HD + 8 * ((col >> 3) ^ tswz(row)) + (col & 7); }
  // Direct loads of rows [row0, row0 + 64), columns [c0, c0 + HD) of a bf16 matrix with `cols` columns (buffer
  // descriptor rs) into dst in the kc (TRL false) or tr (TRL true) layout.
  template <bool TRL> __device__ static __forceinline__ void issue(LDS uint16_t* dst, i32x4_t rs, int row0, int cols, int c0) {
#pragma unroll
    for (int q = 0; q < NL; ++q) {
      const int b = q * KVM_WAVES + wave(), u = 64 * b + lane(), row = u / UPR, ph = u % UPR;
      const int lu = ph ^ (TRL ? tswz(row) : kswz(row));
      dma16(rs, ((row0 + row) * cols + c0 + 8 * lu) * 2, 0, dst + b * 512);
    }
  }
  // MFMA operand from the kc layout: 8 values of row rb + l % 32 at head-dim chunk kk*2 + l/32.
  __device__ static __forceinline__ bf16x8 frag_kc(const LDS uint16_t* s, int rb, int kk) {
    const int l = lane(), r = rb + (l & 31);
    return *(const LDS bf16x8*)(s + kc(r, kk * 2 + (l >> 5)));
  }
  // MFMA operand from the tr layout, rows = head dims db..db+31 (lane l: dim db + l % 32), k = 16 block rows starting
  // at `base` in the accumulator key order: lanes 0-31 rows base+0..3, base+8..11; lanes 32-63 rows base+4..7,
  // base+12..15.
  __device__ static __forceinline__ bf16x8 frag_tr(const LDS uint16_t* s, int db, int base) {
    const int l = lane(), G = l >> 4, i = l & 15;
    const int row = base + 4 * (G >> 1) + (i >> 2), col = db + 16 * (G & 1) + 4 * (i & 3);
    const LDS uint16_t* p0 = s + tr(row, col);
    const s16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS s16x4_t*)p0);
    const s16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS s16x4_t*)(p0 + 8 * HD));
    typedef short s16x8_t __attribute__((ext_vector_type(8)));
    return (bf16x8)__builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
  }
};

__device__ __forceinline__ bf16x8 pack_bf16(const float* p) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)p[i];
  return r;
}

__device__ __forceinline__ View uview(const Ctx& c, int k) { return uniform_view(c.buf(k)); }

// Whether a bf16 view's head slices can be read as 16-byte vectors through a buffer descriptor of T rows.
__device__ __forceinline__ bool fa_ok(const View& x, int T) {
  return x.ok() && x.dtype == 2 && (x.cols % 8) == 0 && (long long)T * x.cols * 2 < 0x7fffffffll;
}

// Forward for 128 queries of head h (op 45): lane l of wave w owns query q0 + 32w + l%32. Per 64-key block kb:
// S^T = K Q^T, P^T = exp2(S^T * scale * log2(e) - m), O^T += V^T P^T, with a running maximum m per query.
//   * Software pipeline over blocks: iteration kb computes the scores of block kb + 1 and then the softmax and P V of
//     block kb, so the MFMAs of the next scores and the VALU work of the current softmax are independent and the
//     scheduler interleaves them (one wave per SIMD: nothing else hides either). FA_FNS stages of K/V in LDS; the
//     buffer a new block loads into held block kb - 1, which every wave finished before the barrier of iteration kb.
//   * The causal mask is applied only in blocks that reach past the wave's first query.
//   * Lazy rescaling: m moves (and O, l are rescaled) only when a query's block maximum exceeds m by more than 8 (in
//     log2 units); P values are then at most 2^8, which fp32 sums and bf16 P hold with the same relative rounding. The
//     result O / l and the log-sum-exp m + log2(l) do not depend on which m was used.
constexpr int FA_FNS = 4;
template <int HD> __device__ __noinline__ void attn_fwd_mfma(const Ctx& c) {
  typedef FaL<HD> L;
  constexpr int NKK = HD / 16, NDB = HD / 32, NS = FA_FNS;
  const View q = uview(c, 0), k = uview(c, 1), v = uview(c, 2), o = uview(c, 3), lse = uview(c, 4);
  const int bb = rfl(c.i(5)), h = rfl(c.i(6)), q0 = rfl(c.i(7)), T = rfl(c.i(8)), H = rfl(c.i(9)), Hkv = rfl(c.i(10));
  const float sl2 = __int_as_float(rfl(__float_as_int(c.f(12)))) * 1.4426950408889634f;   // scale * log2(e)
  const int w = wave(), l = lane(), g = l >> 5, qi = l & 31;
  const int qrow = q0 + 32 * w + qi, kvh = h / (H / Hkv);
  const bool qok = qrow < T;
  bf16x8 qf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk)
    qf[kk] = qok ? *(const GLOBAL bf16x8*)(q.h() + ((long long)bb * T + qrow) * q.cols + h * HD + kk * 16 + 8 * g) : bf16x8{};
  const int kend = min(T, q0 + 128), nkb = (kend + FA_KB - 1) / FA_KB;
  const int wfirst = rfl(q0 + 32 * w), wlast = rfl(min(T - 1, wfirst + 31));   // wave-uniform
  const i32x4_t rk = dma_rsrc((const void*)(k.h() + (long long)bb * T * k.cols), (long long)T * k.cols * 2);
  const i32x4_t rv = dma_rsrc((const void*)(v.h() + (long long)bb * T * v.cols), (long long)T * v.cols * 2);
  LDS uint16_t* lds = (LDS uint16_t*)c.smem;
  constexpr int ST = 2 * FA_KB * HD;                       // elements per stage: K then V
  static_assert(NS * ST * 2 <= KVM_LDS_BYTES, "LDS");
  auto issue = [&](int blk) {
    LDS uint16_t* d = lds + (blk % NS) * ST;
    L::template issue<false>(d, rk, blk * FA_KB, k.cols, kvh * HD);
    L::template issue<true>(d + FA_KB * HD, rv, blk * FA_KB, v.cols, kvh * HD);
  };
  auto scores = [&](int blk, f32x16 (&s)[2]) {
    const LDS uint16_t* Ks = lds + (blk % NS) * ST;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      s[sb] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) s[sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(L::frag_kc(Ks, sb * 32, kk), qf[kk], s[sb], 0, 0, 0);
    }
  };
  f32x16 oacc[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) oacc[d] = f32x16{};
  float m = -INFINITY, lsum = 0.f;                         // m in units of scale * log2(e) * score
  // One iteration: wait for block kb + 1, issue block kb + NS - 1, then (unless every key of block kb is after this
  // wave's queries) the mask of a diagonal block and the rescale, each behind a wave-uniform branch, and one
  // straight-line part: the fragment reads of block kb + 1's K and block kb's V, the softmax of kb, the scores of kb + 1
  // and P V of kb. The scores of kb + 1 are computed even where the wave does not use them (its last block), so that
  // the part has no branch and the scheduler can place the VALU softmax between the MFMAs. The barrier and the loads
  // are outside every per-wave condition.
  auto step = [&](int kb, f32x16 (&sc)[2], f32x16 (&sn)[2]) {
    if (kb + 1 < nkb) wait_vm(min(NS - 3, nkb - 2 - kb) * 2 * L::NL);
    __syncthreads();
    if (kb + NS - 1 < nkb) issue(kb + NS - 1);
    if (kb * FA_KB > wlast) return;                        // every key of the block is after this wave's queries
    if (kb * FA_KB + FA_KB - 1 > wfirst) {                 // a diagonal block: mask keys after each query
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (kb * FA_KB + sb * 32 + 8 * (r >> 2) + 4 * g + (r & 3) > qrow) sc[sb][r] = -INFINITY;
    }
    float mx = sc[0][0];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[sb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * sl2;
    if (__ballot(mx > m + 8.f)) {                          // wave-uniform: some query's maximum moved far enough
      const float mn = fmaxf(m, mx), f = __builtin_amdgcn_exp2f(m - mn);
      lsum *= f;
#pragma unroll
      for (int d = 0; d < NDB; ++d) oacc[d] *= f;
      m = mn;
    }
    const LDS uint16_t* Kn = lds + ((kb + 1) % NS) * ST;
    const LDS uint16_t* Vs = lds + (kb % NS) * ST + FA_KB * HD;
    bf16x8 kfr[2][NKK], vfr[NDB][2][2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) kfr[sb][kk] = L::frag_kc(Kn, sb * 32, kk);
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int t = 0; t < 2; ++t) vfr[d][sb][t] = L::frag_tr(Vs, d * 32, sb * 32 + 16 * t);
    float ps = 0.f;
    bf16x8 pf[2][2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) { pv[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[sb][8 * t + i], sl2, -m)); ps += pv[i]; }
        pf[sb][t] = pack_bf16(pv);
      }
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      sn[sb] = f32x16{};
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) sn[sb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfr[sb][kk], qf[kk], sn[sb], 0, 0, 0);
    }
    lsum += ps + __shfl_xor(ps, 32, 64);
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int t = 0; t < 2; ++t) oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vfr[d][sb][t], pf[sb][t], oacc[d], 0, 0, 0);
  };
  __syncthreads();                                         // the previous task may still read this LDS
#pragma unroll
  for (int p = 0; p < NS - 1; ++p)
    if (p < nkb) issue(p);
  wait_vm(min(NS - 2, nkb - 1) * 2 * L::NL);
  __syncthreads();
  f32x16 sa[2], sb2[2];
  scores(0, sa);                                           // block 0 holds key 0 <= every query of the task
  int kb = 0;
  for (; kb + 1 < nkb; kb += 2) { step(kb, sa, sb2); step(kb + 1, sb2, sa); }
  if (kb < nkb) step(kb, sa, sb2);
  if (qok) {
    const float inv = 1.f / lsum;
    GLOBAL uint16_t* orow = o.h() + ((long long)bb * T + qrow) * o.cols + h * HD + 4 * g;
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        stwt_bf4(orow + d * 32 + 8 * rq, oacc[d][4 * rq] * inv, oacc[d][4 * rq + 1] * inv, oacc[d][4 * rq + 2] * inv, oacc[d][4 * rq + 3] * inv);
    if (g == 0) stwt32(lse.f() + (((long long)bb * H + h) * T + qrow), (m + log2f(lsum)) * 0.6931471805599453f);
  }
}


// dQ for 128 queries of head h (op 47): lane l of wave w owns query q0 + 32w + l%32.
//   S^T = K Q^T, dP^T = V dO^T (K, V from kc LDS copies; Q, dO in registers), P^T = exp(S^T*scale - lse),
//   dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T (K^T from a tr LDS copy), dq = scale * dQ.
template <int HD> __device__ __noinline__ void attn_dq_mfma(const Ctx& c) {
  typedef FaL<HD> L;
  constexpr int NKK = HD / 16, NDB = HD / 32, BK = FA_KB * HD, ST = 3 * BK;
  const View q = uview(c, 0), k = uview(c, 1), v = uview(c, 2), dO = uview(c, 3), lse = uview(c, 4), delta = uview(c, 5), dq = uview(c, 6);
  const int bb = rfl(c.i(7)), h = rfl(c.i(8)), q0 = rfl(c.i(9)), T = rfl(c.i(10)), H = rfl(c.i(11)), Hkv = rfl(c.i(12));
  const float sc = __int_as_float(rfl(__float_as_int(c.f(14)))), sl2 = sc * 1.4426950408889634f;
  const int w = wave(), l = lane(), g = l >> 5, qi = l & 31;
  const int qrow = q0 + 32 * w + qi, kvh = h / (H / Hkv);
  const bool qok = qrow < T;
  const long long grow = (long long)bb * T + qrow;
  bf16x8 qf[NKK], df[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    qf[kk] = qok ? *(const GLOBAL bf16x8*)(q.h() + grow * q.cols + h * HD + kk * 16 + 8 * g) : bf16x8{};
    df[kk] = qok ? *(const GLOBAL bf16x8*)(dO.h() + grow * dO.cols + h * HD + kk * 16 + 8 * g) : bf16x8{};
  }
  const float l2 = qok ? lse.f()[((long long)bb * H + h) * T + qrow] * 1.4426950408889634f : 0.f;
  const float di = qok ? delta.f()[((long long)bb * H + h) * T + qrow] : 0.f;
  const int kend = min(T, q0 + 128), nkb = (kend + FA_KB - 1) / FA_KB;
  const int wlast = min(T - 1, q0 + 32 * w + 31);
  const i32x4_t rk = dma_rsrc((const void*)(k.h() + (long long)bb * T * k.cols), (long long)T * k.cols * 2);
  const i32x4_t rv = dma_rsrc((const void*)(v.h() + (long long)bb * T * v.cols), (long long)T * v.cols * 2);
  LDS uint16_t* lds = (LDS uint16_t*)c.smem;
  auto issue = [&](int blk) {
    LDS uint16_t* d = lds + (blk % FA_NS) * ST;
    L::template issue<false>(d, rk, blk * FA_KB, k.cols, kvh * HD);
    L::template issue<true>(d + BK, rk, blk * FA_KB, k.cols, kvh * HD);
    L::template issue<false>(d + 2 * BK, rv, blk * FA_KB, v.cols, kvh * HD);
  };
  f32x16 acc[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) acc[d] = f32x16{};
  __syncthreads();
#pragma unroll
  for (int p = 0; p < FA_NS - 1; ++p) if (p < nkb) issue(p);
  for (int kb = 0; kb < nkb; ++kb) {
    wait_vm(min(FA_NS - 2, nkb - 1 - kb) * 3 * L::NL);
    __syncthreads();
    if (kb + FA_NS - 1 < nkb) issue(kb + FA_NS - 1);
    if (kb * FA_KB > wlast) continue;
    const LDS uint16_t* Kc = lds + (kb % FA_NS) * ST;
    const LDS uint16_t* Kt = Kc + BK;
    const LDS uint16_t* Vc = Kc + 2 * BK;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      f32x16 sv = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        sv = __builtin_amdgcn_mfma_f32_32x32x16_bf16(L::frag_kc(Kc, sb * 32, kk), qf[kk], sv, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(L::frag_kc(Vc, sb * 32, kk), df[kk], dp, 0, 0, 0);
      }
      bf16x8 dsf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float d8[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = 8 * t + i, key = kb * FA_KB + sb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
          const float pr = key > qrow ? 0.f : __builtin_amdgcn_exp2f(sv[r] * sl2 - l2);
          d8[i] = pr * (dp[r] - di);
        }
        dsf[t] = pack_bf16(d8);
      }
#pragma unroll
      for (int d = 0; d < NDB; ++d)
#pragma unroll
        for (int t = 0; t < 2; ++t) acc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(L::frag_tr(Kt, d * 32, sb * 32 + 16 * t), dsf[t], acc[d], 0, 0, 0);
    }
  }
  if (qok) {
    GLOBAL uint16_t* orow = dq.h() + grow * dq.cols + h * HD + 4 * g;
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        stwt_bf4(orow + d * 32 + 8 * rq, acc[d][4 * rq] * sc, acc[d][4 * rq + 1] * sc, acc[d][4 * rq + 2] * sc, acc[d][4 * rq + 3] * sc);
  }
}

// dK / dV for 128 keys of kv head kvh (op 48), summed over the heads of its GQA group and every later query: lane l
// of wave w owns key k0 + 32w + l%32.
//   S = Q K^T, dP = dO V^T (Q, dO from kc LDS copies; K, V in registers), P = exp(S*scale - lse[q]),
//   dS = P (dP - delta[q]), dV^T += dO^T P, dK^T += Q^T dS (dO^T, Q^T from tr LDS copies), dk = scale * dK.
// lse / delta of the staged 64 queries are loaded into LDS by one 8-lane direct load per wave.
template <int HD> __device__ __noinline__ void attn_dkv_mfma(const Ctx& c) {
  typedef FaL<HD> L;
  constexpr int NKK = HD / 16, NDB = HD / 32, BK = FA_KB * HD, ST = 4 * BK + 2 * FA_KB * 2;   // + lse, delta (f32)
  const View q = uview(c, 0), k = uview(c, 1), v = uview(c, 2), dO = uview(c, 3), lse = uview(c, 4), delta = uview(c, 5);
  const View dk = uview(c, 6), dv = uview(c, 7);
  const int bb = rfl(c.i(8)), kvh = rfl(c.i(9)), k0 = rfl(c.i(10)), T = rfl(c.i(11)), H = rfl(c.i(12));
  const float sc = __int_as_float(rfl(__float_as_int(c.f(14)))), sl2 = sc * 1.4426950408889634f;
  const int G = H / (k.cols / HD);
  const int w = wave(), l = lane(), g = l >> 5, ki = l & 31;
  const int krow = k0 + 32 * w + ki;
  const bool kok = krow < T;
  const long long grow = (long long)bb * T + krow;
  bf16x8 kf[NKK], vf[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; ++kk) {
    kf[kk] = kok ? *(const GLOBAL bf16x8*)(k.h() + grow * k.cols + kvh * HD + kk * 16 + 8 * g) : bf16x8{};
    vf[kk] = kok ? *(const GLOBAL bf16x8*)(v.h() + grow * v.cols + kvh * HD + kk * 16 + 8 * g) : bf16x8{};
  }
  const int qb0 = k0 / FA_KB, nqb = (T + FA_KB - 1) / FA_KB - qb0, nit = G * nqb;
  const int wfirst = k0 + 32 * w;                          // this wave's first key: queries before it see none of its keys
  const i32x4_t rq = dma_rsrc((const void*)(q.h() + (long long)bb * T * q.cols), (long long)T * q.cols * 2);
  const i32x4_t rd = dma_rsrc((const void*)(dO.h() + (long long)bb * T * dO.cols), (long long)T * dO.cols * 2);
  LDS uint16_t* lds = (LDS uint16_t*)c.smem;
  auto issue = [&](int it) {
    const int hh = kvh * G + it / nqb, qb = qb0 + it % nqb;
    LDS uint16_t* d = lds + (it % FA_NS) * ST;
    L::template issue<false>(d, rq, qb * FA_KB, q.cols, hh * HD);
    L::template issue<true>(d + BK, rq, qb * FA_KB, q.cols, hh * HD);
    L::template issue<false>(d + 2 * BK, rd, qb * FA_KB, dO.cols, hh * HD);
    L::template issue<true>(d + 3 * BK, rd, qb * FA_KB, dO.cols, hh * HD);
    // lse / delta: wave 0, 1 -> lse[0:32], [32:64]; wave 2, 3 -> delta; 8 lanes x 16 bytes each
    const View& src = w < 2 ? lse : delta;
    const i32x4_t rs = dma_rsrc((const void*)(src.f() + ((long long)bb * H + hh) * T), (long long)T * 4);
    if (l < 8)
      dma16(rs, (qb * FA_KB + 32 * (w & 1) + 4 * l) * 4, 0, d + 4 * BK + (w >> 1) * 128 + (w & 1) * 64);
  };
  f32x16 adk[NDB], adv[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) { adk[d] = f32x16{}; adv[d] = f32x16{}; }
  constexpr int NLS = 4 * L::NL + 1;
  __syncthreads();
#pragma unroll
  for (int p = 0; p < FA_NS - 1; ++p) if (p < nit) issue(p);
  for (int it = 0; it < nit; ++it) {
    wait_vm(min(FA_NS - 2, nit - 1 - it) * NLS);
    __syncthreads();
    if (it + FA_NS - 1 < nit) issue(it + FA_NS - 1);
    const int qb = qb0 + it % nqb;
    if (qb * FA_KB + FA_KB - 1 < wfirst) continue;          // every query of the block is before this wave's keys
    const LDS uint16_t* Qc = lds + (it % FA_NS) * ST;
    const LDS uint16_t* Qt = Qc + BK;
    const LDS uint16_t* Dc = Qc + 2 * BK;
    const LDS uint16_t* Dt = Qc + 3 * BK;
    const LDS float* Ls = (const LDS float*)(Qc + 4 * BK);
    const LDS float* Es = Ls + FA_KB;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      f32x16 sv = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int kk = 0; kk < NKK; ++kk) {
        sv = __builtin_amdgcn_mfma_f32_32x32x16_bf16(L::frag_kc(Qc, sb * 32, kk), kf[kk], sv, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(L::frag_kc(Dc, sb * 32, kk), vf[kk], dp, 0, 0, 0);
      }
      bf16x8 pf[2], dsf[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        float p8[8], d8[8];
#pragma unroll
        for (int i4 = 0; i4 < 2; ++i4) {
          const int ql = sb * 32 + 8 * (2 * t + i4) + 4 * g;      // first of 4 consecutive queries in this register group
          const f32x4n lq = *(const LDS f32x4n*)(Ls + ql), eq = *(const LDS f32x4n*)(Es + ql);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 8 * t + 4 * i4 + j, qq = qb * FA_KB + ql + j;
            const float pr = qq < krow ? 0.f : __builtin_amdgcn_exp2f(sv[r] * sl2 - lq[j] * 1.4426950408889634f);
            p8[4 * i4 + j] = pr;
            d8[4 * i4 + j] = pr * (dp[r] - eq[j]);
          }
        }
        pf[t] = pack_bf16(p8);
        dsf[t] = pack_bf16(d8);
      }
#pragma unroll
      for (int d = 0; d < NDB; ++d)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          adv[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(L::frag_tr(Dt, d * 32, sb * 32 + 16 * t), pf[t], adv[d], 0, 0, 0);
          adk[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(L::frag_tr(Qt, d * 32, sb * 32 + 16 * t), dsf[t], adk[d], 0, 0, 0);
        }
    }
  }
  if (kok) {
    GLOBAL uint16_t* kr = dk.h() + grow * dk.cols + kvh * HD + 4 * g;
    GLOBAL uint16_t* vr = dv.h() + grow * dv.cols + kvh * HD + 4 * g;
#pragma unroll
    for (int d = 0; d < NDB; ++d)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        stwt_bf4(kr + d * 32 + 8 * rq, adk[d][4 * rq] * sc, adk[d][4 * rq + 1] * sc, adk[d][4 * rq + 2] * sc, adk[d][4 * rq + 3] * sc);
        stwt_bf4(vr + d * 32 + 8 * rq, adv[d][4 * rq], adv[d][4 * rq + 1], adv[d][4 * rq + 2], adv[d][4 * rq + 3]);
      }
  }
}

}  // namespace kvm
