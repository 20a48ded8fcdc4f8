// Attention and decode operators (registry ops 45-50, 134-136). Layouts: activations [B*T, H*hd]; lse/delta at
// (b*H+h)*T+t; KV cache [B*Hkv*Tmax, hd]. Causal tasks cover 128 rows (reference: runtime/ref_gpt.py:13, 279-364).
// Softmax statistics are fp32 with the online (running max) form; lse is the natural log.
#pragma once
#include "common.h"
#include "ops_basic.h"
#include "ops_attn_mfma.h"
#include "ops_attn_f32mfma.h"

namespace kvm {

constexpr int ATTN_ROWS = 128;
constexpr int ATTN_KT = 32;     // keys (or queries) staged per LDS slab

// Stages rows [r0, r0+n) of column block [c0, c0+HD) of X into LDS as fp32 [n][HD+1] (zero rows past `valid`).
// All of a thread's 16-byte loads are issued before any is converted (bf16 or f32 storage, 16-byte aligned columns).
template <int HD> __device__ __forceinline__ void stage_rows(LDS float* dst, const View& X, long long r0, int n, int valid, int c0) {
  constexpr int S = HD + 1;
  if (X.dtype == 2 && (X.cols & 7) == 0 && (c0 & 7) == 0) {
    constexpr int VPR = HD / 8;                        // 16-byte vectors per row
    const int nv = n * VPR;
    for (int base = 0; base < nv; base += 4 * KVM_THREADS) {
      u16x8_t t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = base + u * KVM_THREADS + tid(), r = e / VPR;
        if (e < nv && r < valid) t[u] = *(const GLOBAL u16x8_t*)(X.h() + (r0 + r) * X.cols + c0 + (e % VPR) * 8);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = base + u * KVM_THREADS + tid(), r = e / VPR, k = (e % VPR) * 8;
        if (e < nv)
#pragma unroll
          for (int i = 0; i < 8; ++i) dst[r * S + k + i] = r < valid ? bf2f(t[u][i]) : 0.f;
      }
    }
  } else if (X.dtype == 0 && (X.cols & 3) == 0 && (c0 & 3) == 0) {
    constexpr int VPR = HD / 4;
    const int nv = n * VPR;
    for (int base = 0; base < nv; base += 4 * KVM_THREADS) {
      f32x4n t[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = base + u * KVM_THREADS + tid(), r = e / VPR;
        if (e < nv && r < valid) t[u] = *(const GLOBAL f32x4n*)(X.f() + (r0 + r) * X.cols + c0 + (e % VPR) * 4);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = base + u * KVM_THREADS + tid(), r = e / VPR, k = (e % VPR) * 4;
        if (e < nv)
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[r * S + k + i] = r < valid ? t[u][i] : 0.f;
      }
    }
  } else {
    for (int e = tid(); e < n * HD; e += KVM_THREADS) {
      int r = e / HD, k = e % HD;
      dst[r * S + k] = r < valid ? X.at(r0 + r, c0 + k) : 0.f;
    }
  }
}

// N consecutive values of row r of X from column c0 (zeros when !on): 16-byte loads, all issued before any is
// converted, when the storage and alignment allow (a per-element load with its dtype test waits for each load alone).
template <int N> __device__ __forceinline__ void load_row_part(const View& X, long long r, int c0, bool on, float (&out)[N]) {
  const long long o = r * X.cols + c0;
  if (on && N % 4 == 0 && X.dtype == 0 && (X.cols & 3) == 0 && (c0 & 3) == 0) {
    f32x4n t[N / 4];
#pragma unroll
    for (int u = 0; u < N / 4; ++u) t[u] = *(const GLOBAL f32x4n*)(X.f() + o + 4 * u);
#pragma unroll
    for (int u = 0; u < N / 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) out[4 * u + i] = t[u][i];
  } else if (on && N % 8 == 0 && X.dtype == 2 && (X.cols & 7) == 0 && (c0 & 7) == 0) {
    u16x8_t t[N / 8];
#pragma unroll
    for (int u = 0; u < N / 8; ++u) t[u] = *(const GLOBAL u16x8_t*)(X.h() + o + 8 * u);
#pragma unroll
    for (int u = 0; u < N / 8; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) out[8 * u + i] = bf2f(t[u][i]);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = on ? X.ld(o + i) : 0.f;
  }
}

// Two threads per query row: thread pair (2*row, 2*row+1) splits the head dimension in halves; dot products combine
// with one lane swap. HD is a template parameter so the per-thread halves live in registers.
template <int HD> __device__ __noinline__ void attn_fwd_t(const Ctx& c) {
  constexpr int HALF = HD / 2, S = HD + 1;
  View q = c.buf(0), k = c.buf(1), v = c.buf(2), o = c.buf(3), lse = c.buf(4);
  int bb = c.i(5), h = c.i(6), q0 = c.i(7), T = c.i(8), H = c.i(9), Hkv = c.i(10); float sc = c.f(12);
  int kvh = h / (H / Hkv), row = tid() >> 1, part = tid() & 1;
  int gq = q0 + row; bool active = gq < T;
  LDS float* Ks = (LDS float*)c.smem; LDS float* Vs = Ks + ATTN_KT * S;
  float qr[HALF], acc[HALF];
  load_row_part<HALF>(q, (long long)bb * T + gq, h * HD + part * HALF, active, qr);
#pragma unroll
  for (int i = 0; i < HALF; ++i) { qr[i] *= sc; acc[i] = 0.f; }
  float m = -INFINITY, l = 0.f;
  int last = min(q0 + ATTN_ROWS, T);     // keys [0, last) can matter to this task
  for (int j0 = 0; j0 < last; j0 += ATTN_KT) {
    int nv = min(ATTN_KT, last - j0);
    __syncthreads();
    stage_rows<HD>(Ks, k, (long long)bb * T + j0, ATTN_KT, nv, kvh * HD);
    stage_rows<HD>(Vs, v, (long long)bb * T + j0, ATTN_KT, nv, kvh * HD);
    __syncthreads();
    const int jmax = min(nv, gq - j0 + 1);   // causal: keys j <= gq
    for (int jj = 0; jj < nv; ++jj) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < HALF; ++i) s += qr[i] * Ks[jj * S + part * HALF + i];
      s += __shfl_xor(s, 1, 64);
      if (!active || jj >= jmax) continue;
      float nm = fmaxf(m, s), f = __expf(m - nm), p = __expf(s - nm);
      l = l * f + p;
#pragma unroll
      for (int i = 0; i < HALF; ++i) acc[i] = acc[i] * f + p * Vs[jj * S + part * HALF + i];
      m = nm;
    }
  }
  if (active) {
    float inv = 1.f / l;
#pragma unroll
    for (int i = 0; i < HALF; ++i) o.st(((long long)bb * T + gq) * o.cols + h * HD + part * HALF + i, acc[i] * inv);
    if (part == 0) stwt32(lse.f() + (((long long)bb * H + h) * T + gq), m + logf(l));
  }
}
__device__ __noinline__ void op_attn_fwd(const Ctx& c) {
  const int hd = c.i(11), T = c.i(8);
  if ((hd == 32 || hd == 64 || hd == 128) && T % FA_KB == 0 && fa_ok(c.buf(0), T) && fa_ok(c.buf(1), T) && fa_ok(c.buf(2), T) &&
      fa_ok(c.buf(3), T) && c.buf(4).dtype == 0) {
    if (hd == 64) attn_fwd_mfma<64>(c); else if (hd == 128) attn_fwd_mfma<128>(c); else attn_fwd_mfma<32>(c);
    return;
  }
  if ((hd == 32 || hd == 64 || hd == 128) && T % FA_KB == 0 && fa_ok_f32(c.buf(0), T) && fa_ok_f32(c.buf(1), T) && fa_ok_f32(c.buf(2), T) &&
      fa_ok_f32(c.buf(3), T) && c.buf(4).dtype == 0) {
    if (hd == 64) attn_fwd_f32mfma<64>(c); else if (hd == 128) attn_fwd_f32mfma<128>(c); else attn_fwd_f32mfma<32>(c);
    return;
  }
  switch (c.i(11)) { case 16: attn_fwd_t<16>(c); break; case 32: attn_fwd_t<32>(c); break; case 64: attn_fwd_t<64>(c); break; default: attn_fwd_t<128>(c); }
}

__device__ __noinline__ void op_attn_bwd_delta(const Ctx& c) {
  View o = c.buf(0), d = c.buf(1), delta = c.buf(2); int r0 = c.i(3), r1 = c.i(4), T = c.i(5), H = c.i(6), hd = c.i(7);
  for (int rh = r0 * H + wave(); rh < r1 * H; rh += KVM_WAVES) {
    int r = rh / H, h = rh % H; float s = 0.f;
    for (int k = lane(); k < hd; k += 64) s += o.at(r, h * hd + k) * d.at(r, h * hd + k);
    s = wave_sum(s);
    if (lane() == 0) stwt32(delta.f() + (((long long)(r / T) * H + h) * T + r % T), s);
  }
}

template <int HD> __device__ __noinline__ void attn_dq_t(const Ctx& c) {
  constexpr int HALF = HD / 2, S = HD + 1;
  View q = c.buf(0), k = c.buf(1), v = c.buf(2), d = c.buf(3), lse = c.buf(4), delta = c.buf(5), dq = c.buf(6);
  int bb = c.i(7), h = c.i(8), q0 = c.i(9), T = c.i(10), H = c.i(11), Hkv = c.i(12); float sc = c.f(14);
  int kvh = h / (H / Hkv), row = tid() >> 1, part = tid() & 1;
  int gq = q0 + row; bool active = gq < T;
  LDS float* Ks = (LDS float*)c.smem; LDS float* Vs = Ks + ATTN_KT * S;
  float qr[HALF], dr[HALF], acc[HALF];
  long long qrow = (long long)bb * T + gq;
  load_row_part<HALF>(q, qrow, h * HD + part * HALF, active, qr);
  load_row_part<HALF>(d, qrow, h * HD + part * HALF, active, dr);
#pragma unroll
  for (int i = 0; i < HALF; ++i) acc[i] = 0.f;
  float li = active ? lse.f()[((long long)bb * H + h) * T + gq] : 0.f, di = active ? delta.f()[((long long)bb * H + h) * T + gq] : 0.f;
  int last = min(q0 + ATTN_ROWS, T);
  for (int j0 = 0; j0 < last; j0 += ATTN_KT) {
    int nv = min(ATTN_KT, last - j0);
    __syncthreads();
    stage_rows<HD>(Ks, k, (long long)bb * T + j0, ATTN_KT, nv, kvh * HD);
    stage_rows<HD>(Vs, v, (long long)bb * T + j0, ATTN_KT, nv, kvh * HD);
    __syncthreads();
    const int jmax = min(nv, gq - j0 + 1);
    for (int jj = 0; jj < nv; ++jj) {
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int i = 0; i < HALF; ++i) { s += qr[i] * Ks[jj * S + part * HALF + i]; dp += dr[i] * Vs[jj * S + part * HALF + i]; }
      s += __shfl_xor(s, 1, 64); dp += __shfl_xor(dp, 1, 64);
      if (!active || jj >= jmax) continue;
      float ds = __expf(s * sc - li) * (dp - di);
#pragma unroll
      for (int i = 0; i < HALF; ++i) acc[i] += ds * Ks[jj * S + part * HALF + i];
    }
  }
  if (active)
#pragma unroll
    for (int i = 0; i < HALF; ++i) dq.st(qrow * dq.cols + h * HD + part * HALF + i, acc[i] * sc);
}
__device__ __noinline__ void op_attn_bwd_dq(const Ctx& c) {
  const int hd = c.i(13), T = c.i(10);
  if ((hd == 32 || hd == 64) && T % FA_KB == 0 && fa_ok(c.buf(0), T) && fa_ok(c.buf(1), T) && fa_ok(c.buf(2), T) && fa_ok(c.buf(3), T) &&
      fa_ok(c.buf(6), T) && c.buf(4).dtype == 0 && c.buf(5).dtype == 0) {
    if (hd == 64) attn_dq_mfma<64>(c); else attn_dq_mfma<32>(c);
    return;
  }
  if ((hd == 32 || hd == 64) && T % FA_KB == 0 && fa_ok_f32(c.buf(0), T) && fa_ok_f32(c.buf(1), T) && fa_ok_f32(c.buf(2), T) &&
      fa_ok_f32(c.buf(3), T) && fa_ok_f32(c.buf(6), T) && c.buf(4).dtype == 0 && c.buf(5).dtype == 0) {
    if (hd == 64) attn_dq_f32mfma<64>(c); else attn_dq_f32mfma<32>(c);
    return;
  }
  switch (c.i(13)) { case 16: attn_dq_t<16>(c); break; case 32: attn_dq_t<32>(c); break; case 64: attn_dq_t<64>(c); break; default: attn_dq_t<128>(c); }
}

// dK/dV for 128 keys of kv head kvh: sums over the GQA group's heads and every later query, fixed order.
template <int HD> __device__ __noinline__ void attn_dkv_t(const Ctx& c) {
  constexpr int HALF = HD / 2, S = HD + 1;
  View q = c.buf(0), k = c.buf(1), v = c.buf(2), d = c.buf(3), lse = c.buf(4), delta = c.buf(5), dk = c.buf(6), dv = c.buf(7);
  int bb = c.i(8), kvh = c.i(9), k0 = c.i(10), T = c.i(11), H = c.i(12); float sc = c.f(14);
  int G = H / (k.cols / HD), row = tid() >> 1, part = tid() & 1;
  int gk = k0 + row; bool active = gk < T;
  LDS float* Qs = (LDS float*)c.smem; LDS float* Ds = Qs + ATTN_KT * S; LDS float* Ls = Ds + ATTN_KT * S; LDS float* Es = Ls + ATTN_KT;
  long long krow = (long long)bb * T + gk;
  float kr[HALF], vr[HALF], sk[HALF], sv[HALF];
  load_row_part<HALF>(k, krow, kvh * HD + part * HALF, active, kr);
  load_row_part<HALF>(v, krow, kvh * HD + part * HALF, active, vr);
#pragma unroll
  for (int i = 0; i < HALF; ++i) sk[i] = sv[i] = 0.f;
  for (int h = kvh * G; h < (kvh + 1) * G; ++h)
    for (int j0 = k0; j0 < T; j0 += ATTN_KT) {   // queries before k0 never see these keys
      int nv = min(ATTN_KT, T - j0);
      __syncthreads();
      stage_rows<HD>(Qs, q, (long long)bb * T + j0, ATTN_KT, nv, h * HD);
      stage_rows<HD>(Ds, d, (long long)bb * T + j0, ATTN_KT, nv, h * HD);
      for (int e = tid(); e < ATTN_KT; e += KVM_THREADS) {
        Ls[e] = e < nv ? lse.f()[((long long)bb * H + h) * T + j0 + e] : 0.f;
        Es[e] = e < nv ? delta.f()[((long long)bb * H + h) * T + j0 + e] : 0.f;
      }
      __syncthreads();
      const int jmin = max(0, gk - j0);      // causal: queries j >= gk
      for (int jj = 0; jj < nv; ++jj) {
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int i = 0; i < HALF; ++i) { s += Qs[jj * S + part * HALF + i] * kr[i]; dp += Ds[jj * S + part * HALF + i] * vr[i]; }
        s += __shfl_xor(s, 1, 64); dp += __shfl_xor(dp, 1, 64);
        if (!active || jj < jmin) continue;
        float p = __expf(s * sc - Ls[jj]), w = p * (dp - Es[jj]);
#pragma unroll
        for (int i = 0; i < HALF; ++i) { sv[i] += p * Ds[jj * S + part * HALF + i]; sk[i] += w * Qs[jj * S + part * HALF + i]; }
      }
    }
  if (active)
#pragma unroll
    for (int i = 0; i < HALF; ++i) {
      dk.st(krow * dk.cols + kvh * HD + part * HALF + i, sk[i] * sc);
      dv.st(krow * dv.cols + kvh * HD + part * HALF + i, sv[i]);
    }
}
__device__ __noinline__ void op_attn_bwd_dkv(const Ctx& c) {
  const int hd = c.i(13), T = c.i(11);
  if ((hd == 32 || hd == 64) && T % FA_KB == 0 && fa_ok(c.buf(0), T) && fa_ok(c.buf(1), T) && fa_ok(c.buf(2), T) && fa_ok(c.buf(3), T) &&
      fa_ok(c.buf(6), T) && fa_ok(c.buf(7), T) && c.buf(4).dtype == 0 && c.buf(5).dtype == 0) {
    if (hd == 64) attn_dkv_mfma<64>(c); else attn_dkv_mfma<32>(c);
    return;
  }
  if ((hd == 32 || hd == 64) && T % FA_KB == 0 && fa_ok_f32(c.buf(0), T) && fa_ok_f32(c.buf(1), T) && fa_ok_f32(c.buf(2), T) &&
      fa_ok_f32(c.buf(3), T) && fa_ok_f32(c.buf(6), T) && fa_ok_f32(c.buf(7), T) && c.buf(4).dtype == 0 && c.buf(5).dtype == 0) {
    if (hd == 64) attn_dkv_f32mfma<64>(c); else attn_dkv_f32mfma<32>(c);
    return;
  }
  switch (c.i(13)) { case 16: attn_dkv_t<16>(c); break; case 32: attn_dkv_t<32>(c); break; case 64: attn_dkv_t<64>(c); break; default: attn_dkv_t<128>(c); }
}

// ---------------------------------------------------------------------------------------------- decode
// One query row per (b, h) over cache positions [0, lens[b]] (registry op 50).
__device__ __noinline__ void op_attn_decode(const Ctx& c) {
  View q = c.buf(0), kc = c.buf(1), vc = c.buf(2), lens = c.buf(3), o = c.buf(4);
  int bb = c.i(5), h = c.i(6), H = c.i(7), Hkv = c.i(8), hd = c.i(9), Tmax = c.i(10); float sc = c.f(11);
  int n = lens.i()[bb] + 1;
  if (n < 1 || n > Tmax) { if (tid() == 0) c.fail(KVM_ERR_OP_KVLEN, bb, n - 1); return; }
  long long base = ((long long)bb * Hkv + h / (H / Hkv)) * Tmax;
  LDS float* qs = (LDS float*)c.smem; LDS float* s = qs + 128; LDS float* red = s + n;
  for (int k = tid(); k < hd; k += KVM_THREADS) qs[k] = q.at(bb, h * hd + k);
  __syncthreads();
  float mx = -INFINITY;
  for (int j = tid(); j < n; j += KVM_THREADS) { float a = 0.f; for (int k = 0; k < hd; ++k) a += qs[k] * kc.at(base + j, k); s[j] = a * sc; mx = fmaxf(mx, s[j]); }
  mx = block_max(mx, red);
  float l = 0.f;
  for (int j = tid(); j < n; j += KVM_THREADS) { s[j] = __expf(s[j] - mx); l += s[j]; }
  l = block_sum(l, red + 4);
  for (int k = tid(); k < hd; k += KVM_THREADS) {
    float a = 0.f; for (int j = 0; j < n; ++j) a += s[j] * vc.at(base + j, k);
    o.st((long long)bb * o.cols + h * hd + k, a / l);
  }
}

constexpr float ATTN_EMPTY_M = -3.4028234663852886e38f;

// Split-context decode attention (registry op 135): one task = (sequence b, kv head, split s) for the whole GQA group,
// so each K/V row of the split is read once for G query heads. Keys go through LDS in chunks of 64 (16-byte loads,
// all issued before use), with an online softmax across chunks. Optional fused RoPE of q and the new key, and the KV
// append of the new token by the split that holds it (flags 1, 3).
constexpr int DEC_KC = 64;
__device__ __noinline__ void op_attn_decode_part(const Ctx& c) {
  View q = c.buf(0), kc = c.buf(1), vc = c.buf(2), lens = c.buf(3), part = c.buf(4), kn = c.buf(5), vn = c.buf(6);
  int bb = c.i(7), kvh = c.i(8), s = c.i(9), S = c.i(10), H = c.i(11), Hkv = c.i(12), hd = c.i(13), Tmax = c.i(14);
  float sc = c.f(15), th = c.f(16); int fl = c.i(17);
  int L = lens.i()[bb], n = L + 1;
  if (L < 0 || n > Tmax) { if (tid() == 0) c.fail(KVM_ERR_OP_KVLEN, bb, L); return; }
  int chunk = (n + S - 1) / S, j0 = s * chunk, j1 = min(n, j0 + chunk), nk = max(0, j1 - j0);
  const int G = H / Hkv, half = hd / 2, HS = hd + 1;
  long long base = ((long long)bb * Hkv + kvh) * Tmax;
  LDS float* qs = (LDS float*)c.smem;          // [G][hd]
  LDS float* Ks = qs + 8 * 128;                // [DEC_KC][hd+1]
  LDS float* Vs = Ks + DEC_KC * 129;           // [DEC_KC][hd+1]
  LDS float* P = Vs + DEC_KC * 129;            // [G][DEC_KC]
  LDS float* st = P + 8 * DEC_KC;              // m_run[8], l_run[8], f[8]
  for (int e = tid(); e < G * hd; e += KVM_THREADS) qs[e] = q.at(bb, (kvh * G + e / hd) * hd + e % hd);
  if (tid() < 8) { st[tid()] = -INFINITY; st[8 + tid()] = 0.f; st[16 + tid()] = 1.f; }
  __syncthreads();
  if (fl & 1) {
    for (int e = tid(); e < G * half; e += KVM_THREADS) {
      int g = e / half, i = e % half; float sn, co; rope_sc(L, i, hd, th, sn, co);
      float x1 = qs[g * hd + i], x2 = qs[g * hd + i + half], y1 = x1 * co - x2 * sn, y2 = x1 * sn + x2 * co;
      if (fl & 2) { y1 = round_bf(y1); y2 = round_bf(y2); }
      qs[g * hd + i] = y1; qs[g * hd + i + half] = y2;
    }
    if (j0 <= n - 1 && n - 1 < j1) {      // this split holds the new key: write it (rotated) and its value first
      long long row = base + n - 1;
      for (int i = tid(); i < half; i += KVM_THREADS) {
        float sn, co; rope_sc(L, i, hd, th, sn, co);
        float x1 = kn.at(bb, kvh * hd + i), x2 = kn.at(bb, kvh * hd + i + half);
        kc.st(row * kc.cols + i, x1 * co - x2 * sn); kc.st(row * kc.cols + i + half, x1 * sn + x2 * co);
      }
      for (int k = tid(); k < hd; k += KVM_THREADS) vc.st(row * vc.cols + k, vn.at(bb, kvh * hd + k));
    }
    __syncthreads();
  }
  if (nk == 0) {
    for (int e = tid(); e < G * (hd + 2); e += KVM_THREADS) {
      int g = e / (hd + 2), k = e % (hd + 2); long long r = (((long long)bb * S + s) * H + kvh * G + g) * part.cols;
      stwt32(part.f() + (r + k), k < hd ? 0.f : (k == hd ? ATTN_EMPTY_M : 0.f));
    }
    return;
  }
  // outputs (g, k) owned by this thread: e = tid, tid + 256, ... over G*hd
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const int nvec = hd / 8;
  for (int c0 = 0; c0 < nk; c0 += DEC_KC) {
    const int cn = min(DEC_KC, nk - c0);
    __syncthreads();
    // stage K and V rows [j0+c0, j0+c0+cn): 16-byte loads, all issued before they are converted into LDS
    if (kc.dtype == 2 && vc.dtype == 2) {
      u16x8_t kv[4], vv[4]; int idx[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        idx[u] = tid() + u * KVM_THREADS;
        int j = idx[u] / nvec, v8 = idx[u] % nvec;
        if (idx[u] < cn * nvec) {
          kv[u] = *(const GLOBAL u16x8_t*)(kc.h() + (base + j0 + c0 + j) * kc.cols + v8 * 8);
          vv[u] = *(const GLOBAL u16x8_t*)(vc.h() + (base + j0 + c0 + j) * vc.cols + v8 * 8);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (idx[u] >= cn * nvec) continue;
        int j = idx[u] / nvec, v8 = idx[u] % nvec;
#pragma unroll
        for (int i = 0; i < 8; ++i) { Ks[j * HS + v8 * 8 + i] = bf2f(kv[u][i]); Vs[j * HS + v8 * 8 + i] = bf2f(vv[u][i]); }
      }
      for (int e = 4 * KVM_THREADS + tid(); e < cn * nvec; e += KVM_THREADS) {   // hd*DEC_KC beyond 4 vectors/thread
        int j = e / nvec, v8 = e % nvec;
        u16x8_t a = *(const GLOBAL u16x8_t*)(kc.h() + (base + j0 + c0 + j) * kc.cols + v8 * 8);
        u16x8_t b2 = *(const GLOBAL u16x8_t*)(vc.h() + (base + j0 + c0 + j) * vc.cols + v8 * 8);
        for (int i = 0; i < 8; ++i) { Ks[j * HS + v8 * 8 + i] = bf2f(a[i]); Vs[j * HS + v8 * 8 + i] = bf2f(b2[i]); }
      }
    } else {
      for (int e = tid(); e < cn * hd; e += KVM_THREADS) {
        int j = e / hd, k = e % hd;
        Ks[j * HS + k] = kc.ld((base + j0 + c0 + j) * kc.cols + k); Vs[j * HS + k] = vc.ld((base + j0 + c0 + j) * vc.cols + k);
      }
    }
    __syncthreads();
    for (int e = tid(); e < G * DEC_KC; e += KVM_THREADS) {     // scores of this chunk
      int g = e / DEC_KC, j = e % DEC_KC; float a = -INFINITY;
      if (j < cn) { a = 0.f; for (int k = 0; k < hd; ++k) a += qs[g * hd + k] * Ks[j * HS + k]; a *= sc; }
      P[g * DEC_KC + j] = a;
    }
    __syncthreads();
    for (int g = wave(); g < G; g += KVM_WAVES) {                 // online softmax update per head
      float v = lane() < DEC_KC ? P[g * DEC_KC + lane()] : -INFINITY;
      float cm = wave_max(v), mo = st[g], mn = fmaxf(mo, cm);
      float p = lane() < cn ? __expf(v - mn) : 0.f;
      if (lane() < DEC_KC) P[g * DEC_KC + lane()] = p;
      float ps = wave_sum(p);
      if (lane() == 0) { float f = __expf(mo - mn); st[16 + g] = f; st[8 + g] = st[8 + g] * f + ps; st[g] = mn; }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      int e = tid() + u * KVM_THREADS;
      if (e >= G * hd) break;
      int g = e / hd, k = e % hd; float a = acc[u] * st[16 + g];
      for (int j = 0; j < cn; ++j) a += P[g * DEC_KC + j] * Vs[j * HS + k];
      acc[u] = a;
    }
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    int e = tid() + u * KVM_THREADS;
    if (e >= G * hd) break;
    int g = e / hd, k = e % hd;
    long long r = (((long long)bb * S + s) * H + kvh * G + g) * part.cols;
    stwt32(part.f() + (r + k), acc[u]);
    if (k == 0) { stwt32(part.f() + (r + hd), st[g]); stwt32(part.f() + (r + hd + 1), st[8 + g]); }
  }
}
// Streaming form of op 135 for bf16 caches with hd = 128: the split's tokens go in blocks of 160 (40 per wave). Lane l
// owns head dimensions 8 * (l % 16) .. + 8 of token slot l / 16, so each of the 10 rounds of a wave covers 4 tokens, and
// the K and V rows of a block arrive with 16-byte loads that are all in flight together. Scores are dot products
// against the (rotated, scale-folded) query held in registers, summed over the 16 lanes of a token; the block max and
// exp-sum are reduced over the workgroup in a fixed order; P V accumulates in the same layout and is reduced over the
// token slots, then over the waves in order. Blocks after the first rescale the running sums (online softmax).
// Sum over the 16 lanes of a DPP row, every lane receiving it: four rotate-and-add steps (row_ror 8, 4, 2, 1), all in
// registers (a lane shuffle goes through the LDS crossbar).
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x128, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x124, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x122, 0xf, 0xf, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x121, 0xf, 0xf, false));
  return v;
}
// Op 308: the 128 x 256 tile of op 122 (plain epilogue, bf16 output), then, from the tile still staged in LDS, the
// attention backward statistic of its four 64-column heads: per row, each lane takes its 4 columns (bf16-rounded as
// stored) times o, and the 16 lanes of a head (one DPP row) are summed.
__device__ __noinline__ void mma_delta_tail(const Ctx& c);
__device__ __noinline__ void op_matmul_mma_bf16_delta(const Ctx& c) {
  mfma_tile<128, 256>(c);                                  // leaves the f32 tile staged in LDS (one 128 KiB half)
  mma_delta_tail(c);
}
__device__ __noinline__ void mma_delta_tail(const Ctx& c) {
  const GemmArgs g = gemm_args(c);
  const View o = uniform_view(c.buf(13)), dl = uniform_view(c.buf(14));
  const int T = rfl(c.i(15)), H = rfl(c.i(16));
  constexpr int TN = 256, NB = 8;
  const LDS float* et = (const LDS float*)c.smem;
  const int ch = lane(), w = wave(), n = g.n0 + 4 * ch, head = n / 64;
  Ld4 lo;
  lo.init(o);
  for (int r0 = w; r0 < 128; r0 += KVM_WAVES * NB) {
    u32x4_t raw[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) raw[u] = lo.raw((g.m0 + r0 + KVM_WAVES * u) * o.cols + n);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int r = r0 + KVM_WAVES * u, m = g.m0 + r;
      const f32x4n a = *(const LDS f32x4n*)(et + r * TN + 4 * (ch ^ epi_swz<TN>(r)));
      const f32x4n ov = lo.cvt(raw[u]);
      float p = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) p += round_bf(a[e] * g.e.alpha) * ov[e];
      p = row16_sum(p);
      if ((ch & 15) == 0) stwt32(dl.f() + (((long long)(m / T) * H + head) * T + m % T), p);
    }
  }
}
// Geometry of the streaming split: 160 tokens per block, staged in LDS as [token slot][128] bf16 rows, K then V
// (a block's slot k holds row min(k, nk - 1) of the split), then the block statistics and the rotation table. The
// P V partials alias the staging after the last block.
constexpr int ATT_DR = 10, ATT_DB = 4 * KVM_WAVES * ATT_DR, ATT_HD = 128;
constexpr int ATT_KV_BYTES = ATT_DB * ATT_HD * 2, ATT_RED_OFF = 2 * ATT_KV_BYTES, ATT_ROT_OFF = ATT_RED_OFF + 64 * 4;
static_assert(ATT_ROT_OFF + 128 * 4 <= KVM_LDS_BYTES && 16 * 8 * ATT_HD * 4 <= 2 * ATT_KV_BYTES, "decode attention LDS map");
// The split's token range [j0, j0 + nk) of the n = L + 1 tokens (L = lens[b]); false when L is out of range.
__device__ __forceinline__ bool attn_split(const Ctx& c, int& L, int& j0, int& nk) {
  const View lens = c.buf(3);
  const int bb = c.i(7), s = c.i(9), S = c.i(10), Tmax = c.i(14);
  L = lens.i()[bb];
  const int n = L + 1;
  if (L < 0 || n > Tmax) return false;
  const int chunk = (n + S - 1) / S;
  j0 = s * chunk;
  nk = max(0, min(n, j0 + chunk) - j0);
  return true;
}
// The rotation table of position L: sin, then cos, of the 64 angles (threads 0..63).
__device__ __forceinline__ void attn_rot_table(int L, float theta, LDS float* rot) {
  if (tid() < 64) { float sn, co; rope_sc_ref(L, tid(), ATT_HD, log((double)theta), sn, co); rot[tid()] = sn; rot[64 + tid()] = co; }
}
// Op 135 takes the streaming form for bf16 caches at hd 128 with G in {1, 2, 4, 8}; op 306 always (validated).
__device__ __forceinline__ bool attn_fast_ok(const Ctx& c, int op) {
  if (op == 306 || op == 310) return true;
  const View kc = c.buf(1), vc = c.buf(2);
  const int H = c.i(11), Hkv = c.i(12), G = Hkv > 0 ? H / Hkv : 0;
  return kc.dtype == 2 && vc.dtype == 2 && c.i(13) == 128 && (kc.cols % 8) == 0 && (vc.cols % 8) == 0 && (G == 1 || G == 2 || G == 4 || G == 8);
}
// A long split on the MFMA units (the batched decode graph's splits hold ~1,000 tokens; a one-row split's ~130 stay on
// the VALU form below, whose block pipeline suits it). Each wave streams its own contiguous quarter of the split in
// chunks of 16 tokens, K and V rows direct from HBM into a per-wave 3-stage LDS ring (16-byte units XOR-swizzled by
// token), with its own flash-softmax state; the four waves' states are combined at the end.
//   scores: v_mfma_f32_16x16x32_bf16, A = 16 K rows (tokens x hd), B = the query block (hd x 16 rows): rows 0..G-1 are
//   the bf16 rounding of the query heads, rows G..2G-1 the bf16 rounding of the remainder, so score = D[row g] +
//   D[row g + G] is the product with the f32 query to ~2^-16 (K is bf16 already: every product is exact in f32).
//   P V: v_mfma_f32_16x16x16_bf16, A = P (16 rows x 16 tokens, again hi rows and remainder rows; the scores' output
//   registers are already the A operand's layout: lane = row, 4 registers = 4 consecutive tokens), B = V rows read
//   transposed (ds_read_b64_tr_b16), 8 blocks of 16 head dims.
// The partial (unnormalised P V, max, sum) has op 135's format and meaning; the query block comes in LDS at ATT_MQ_OFF
// ([G][128] f32, rotated, normalised and scaled).
#ifndef ATT_MNS_V
#define ATT_MNS_V 3
#endif
constexpr int ATT_MCH = 16, ATT_MNS = ATT_MNS_V, ATT_MSB = ATT_MCH * ATT_HD * 2;   // tokens per chunk, ring stages, bytes per operand per stage
constexpr int ATT_MQ_OFF = KVM_LDS_BYTES - 8 * ATT_HD * 4;                // query block [8][128] f32 at the end of the LDS
constexpr int ATT_MFMA_MIN = 256;                                          // splits longer than this take the MFMA form
static_assert(KVM_WAVES * ATT_MNS * 2 * ATT_MSB <= ATT_MQ_OFF && KVM_WAVES * (16 * ATT_HD + 16) * 4 <= ATT_MQ_OFF, "decode MFMA LDS map");
// Before the dependency wait of a streaming split that will run with c.pre set (all four waves, the task's record in
// c): its first block's K and V rows go to the staging direct from HBM (loads in flight through the wait) and the
// rotation table is computed. The cache rows read here are written only by earlier launches, except the split's own
// new row, which the task itself writes into the staging after these loads have landed. The lengths are written
// only after the last layer's splits.
__device__ __noinline__ void attn_prefetch(const Ctx& c, int op) {
  if (!attn_fast_ok(c, op)) return;
  int L, j0, nk;
  if (!attn_split(c, L, j0, nk) || nk == 0) return;
  const View kc = uniform_view(c.buf(1)), vc = uniform_view(c.buf(2));
  const int bb = c.i(7), kvh = c.i(8), Hkv = c.i(12), Tmax = c.i(14);
  const long long row0 = ((long long)bb * Hkv + kvh) * Tmax + j0;
  const i32x4_t rk = dma_rsrc((const void*)(kc.h() + row0 * kc.cols), (long long)nk * kc.cols * 2);
  const i32x4_t rv = dma_rsrc((const void*)(vc.h() + row0 * vc.cols), (long long)nk * vc.cols * 2);
  const int l = lane(), w = wave(), ts = l >> 4, d0 = 8 * (l & 15);
  LDS uint16_t* Ks = (LDS uint16_t*)c.smem;
  LDS uint16_t* Vs = Ks + ATT_DB * ATT_HD;
#pragma unroll
  for (int i = 0; i < ATT_DR; ++i) {
    const int slot = w * 4 * ATT_DR + 4 * i, row = min(slot + ts, nk - 1);
    dma16(rk, (row * kc.cols + d0) * 2, 0, Ks + slot * ATT_HD);
    dma16(rv, (row * vc.cols + d0) * 2, 0, Vs + slot * ATT_HD);
  }
  if (c.i(17) & 1) attn_rot_table(L, c.f(16), (LDS float*)(c.smem + ATT_ROT_OFF));
}
// qkn (op 306): the query heads and the new key are RMS-normalised per head first (gamma args 18 / 19, eps arg 20).
// c.pre: attn_prefetch ran before the wait (block 0 staged, rotation table ready).
__device__ __forceinline__ void attn_merge(const View& part, const View& o, int bb, int h0, int h1, int S, int H, int hd, LDS char* smem);
// The merge of op 136 for the G query heads h0.. of one kv head at hd 128, latency-bound (a few KB per split):
// wave w takes heads w, w + 4, ...; lane l owns dimensions 2l, 2l + 1. Each lane requests its two values of 16
// splits at once (8-byte loads, all in flight), while lanes 0..S-1 hold the splits' (m, l) and the split weights
// e_s = exp(m_s - max m) over live splits (l > 0) are formed and broadcast from them. Sums in split order, as op 136.
template <int G> __device__ __forceinline__ void attn_merge_g(const View& part, const View& o, int bb, int h0, int S, int H) {
  constexpr int hd = ATT_HD, SB = 16;
  const int l = lane(), cols = part.cols;
  for (int g = wave(); g < G; g += KVM_WAVES) {
    const int h = h0 + g;
    const GLOBAL float* base = part.f() + (((long long)bb * S) * H + h) * cols;
    const long long step = (long long)H * cols;
    float M = -INFINITY;
    for (int s = l; s < S; s += 64) if (base[s * step + hd + 1] > 0.f) M = fmaxf(M, base[s * step + hd]);
    M = wave_max(M);
    float den = 0.f, a0 = 0.f, a1 = 0.f;
    for (int s0 = 0; s0 < S; s0 += 64) {
      float e = 0.f;
      if (s0 + l < S) {
        const float ll = base[(s0 + l) * step + hd + 1];
        e = ll > 0.f ? __expf(base[(s0 + l) * step + hd] - M) : 0.f;
        den += e * ll;
      }
      for (int s1 = 0; s1 < 64 && s0 + s1 < S; s1 += SB) {
        typedef float f2v __attribute__((ext_vector_type(2)));
        f2v v[SB];
#pragma unroll
        for (int i = 0; i < SB; ++i) {
          const int s = min(s0 + s1 + i, S - 1);
          v[i] = *(const GLOBAL f2v*)(base + s * step + 2 * l);
        }
#pragma unroll
        for (int i = 0; i < SB; ++i) {
          const float w = __shfl(e, s1 + i, 64);
          if (s0 + s1 + i < S) { a0 += w * v[i].x; a1 += w * v[i].y; }
        }
      }
    }
    const float inv = 1.f / wave_sum(den);
    o.st((long long)bb * o.cols + h * hd + 2 * l, a0 * inv);
    o.st((long long)bb * o.cols + h * hd + 2 * l + 1, a1 * inv);
  }
}
// Op 310's completion: this split's partials are made agent-visible (write-through stores, waited for) before it counts
// itself; the split that counts last acquires and merges the kv head's G query heads (op 136), then resets the count.
template <int G> __device__ __forceinline__ void attn_arrive(const Ctx& c, int bb, int kvh, int S, int H, int Hkv) {
  const View part = uniform_view(c.buf(4)), o = uniform_view(c.buf(21)), cnt = uniform_view(c.buf(22));
  LDS int* flag = (LDS int*)(c.smem + ATT_RED_OFF);
  wait_stores();
  __syncthreads();
  if (tid() == 0) *flag = add_relaxed((int*)(cnt.i() + ((long long)bb * Hkv + kvh)), 1);
  __syncthreads();
  const int old = *flag;
  if (old < 0 || old >= S) { if (tid() == 0) c.fail(KVM_ERR_OP_RANGE, bb * Hkv + kvh, old); return; }
  if (old != S - 1) return;
  fence_acquire();                                      // the other splits' partials, stored before their counts
  attn_merge_g<G>(part, o, bb, kvh * G, S, H);
  if (tid() == 0) st_relaxed((int*)(cnt.i() + ((long long)bb * Hkv + kvh)), 0);
}
template <int G> __device__ __noinline__ void attn_split_mfma(const Ctx& c, int j0, int nk) {
  static_assert(2 * G <= 16, "query rows");
  constexpr int hd = ATT_HD, CH = ATT_MCH, NS = ATT_MNS, SB = ATT_MSB;
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const View kc = uniform_view(c.buf(1)), vc = uniform_view(c.buf(2)), part = uniform_view(c.buf(4));
  const int bb = c.i(7), kvh = c.i(8), s = c.i(9), S = c.i(10), H = c.i(11), Hkv = c.i(12), Tmax = c.i(14);
  const long long row0 = ((long long)bb * Hkv + kvh) * Tmax + j0;
  const i32x4_t rk = dma_rsrc((const void*)(kc.h() + row0 * kc.cols), (long long)nk * kc.cols * 2);
  const i32x4_t rv = dma_rsrc((const void*)(vc.h() + row0 * vc.cols), (long long)nk * vc.cols * 2);
  const int l = lane(), w = wave(), n = l & 15, qq = l >> 4;
  // the query block as the B operand: lane (n, qq) holds row n, head dims 32 kk + 8 qq .. + 7
  const LDS float* qs = (const LDS float*)(c.smem + ATT_MQ_OFF);
  bf16x8 qb[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = n < 2 * G ? qs[(n % G) * hd + 32 * kk + 8 * qq + e] : 0.f;
      const __bf16 hi = (__bf16)x;
      qb[kk][e] = n < G ? hi : (__bf16)(x - (float)hi);
    }
  __syncthreads();                                         // every wave has its query block: the rings may overwrite it
  LDS char* ring = c.smem + w * NS * 2 * SB;
  const int nch = (nk + CH - 1) / CH, per = (nch + KVM_WAVES - 1) / KVM_WAVES, c0 = min(nch, w * per), c1 = min(nch, c0 + per);
  // chunk ch into stage slot: 4 loads of K and 4 of V per lane; lane (n, qq) of load i fills token 4 i + qq, unit
  // position n with the row's 16-byte unit n ^ token
  auto issue = [&](int ch, int slot) {
    LDS char* st = ring + slot * 2 * SB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 4 * i + qq, tok = min(ch * CH + t, nk - 1), u = n ^ t;
      dma16(rk, (tok * kc.cols + 8 * u) * 2, 0, st + i * 1024);
      dma16(rv, (tok * vc.cols + 8 * u) * 2, 0, st + SB + i * 1024);
    }
  };
  f32x4n o[8];
#pragma unroll
  for (int hb = 0; hb < 8; ++hb) o[hb] = f32x4n{0.f, 0.f, 0.f, 0.f};
  float mrun = -INFINITY, lrun = 0.f;
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) if (c0 + p < c1) issue(c0 + p, p);
  for (int ch = c0; ch < c1; ++ch) {
    const int k = ch - c0;
    if (ch + NS - 1 < c1) { wait_lds(); issue(ch + NS - 1, (k + NS - 1) % NS); }
    wait_vm(8 * min(NS - 1, c1 - 1 - ch));               // this chunk's loads have landed
    const LDS char* Ks = ring + (k % NS) * 2 * SB;
    const LDS char* Vs = Ks + SB;
    f32x4n d = f32x4n{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const bf16x8 a = *(const LDS bf16x8*)(Ks + n * 256 + (((4 * kk + qq) ^ n) * 16));
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[kk], d, 0, 0, 0);
    }
    // lane (n, qq), register i: row n, token 16 ch + 4 qq + i
    float sc4[4], bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = d[i] + __shfl_xor(d[i], G, 64);
      sc4[i] = (n < 2 * G && ch * CH + 4 * qq + i < nk) ? x : -INFINITY;
      bm = fmaxf(bm, sc4[i]);
    }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(mrun, bm);
    const float f = mn == -INFINITY ? 1.f : __expf(mrun - mn);
    float ps = 0.f;
    s16x4 pa;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = sc4[i] == -INFINITY ? 0.f : __expf(sc4[i] - mn);
      ps += p;
      const __bf16 hi = (__bf16)p, v = n < G ? hi : (__bf16)(p - (float)hi);
      pa[i] = __builtin_bit_cast(short, v);
    }
    lrun = lrun * f + ps;
    mrun = mn;
    if (__ballot(f != 1.f)) {                             // rescale: output register i of lane group qq is row 4 qq + i
      float fh[G];
#pragma unroll
      for (int g = 0; g < G; ++g) fh[g] = __shfl(f, g, 64);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * qq + i;
        float fr = 1.f;
#pragma unroll
        for (int g = 0; g < G; ++g) if (r % G == g && r < 2 * G) fr = fh[g];
#pragma unroll
        for (int hb = 0; hb < 8; ++hb) o[hb][i] *= fr;
      }
    }
    const int t = 4 * qq + (n >> 2);                       // transposed read: token row of this lane's 8 bytes
#pragma unroll
    for (int hb = 0; hb < 8; ++hb) {
      const int dd = hb * 16 + 4 * (n & 3);
      const LDS char* pv = Vs + t * 256 + (((dd >> 3) ^ t) * 16) + (dd & 7) * 2;
      const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS s16x4*)pv);
      o[hb] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pa, b, o[hb], 0, 0, 0);
    }
  }
  // per wave: rows of P V (16 x 128), and the max and sum of each head
  float lsum = lrun + __shfl_xor(lrun, 16, 64);           // over the four lane groups (their tokens)
  lsum += __shfl_xor(lsum, 32, 64);
  wait_vm_c<0>();
  __syncthreads();                                         // every wave is past its ring: the state goes over it
  LDS float* ow = (LDS float*)c.smem + w * (16 * hd + 16);
#pragma unroll
  for (int hb = 0; hb < 8; ++hb)
#pragma unroll
    for (int i = 0; i < 4; ++i) ow[(4 * qq + i) * hd + hb * 16 + n] = o[hb][i];
  if (qq == 0 && n < G) { ow[16 * hd + n] = mrun; ow[16 * hd + 8 + n] = lsum; }
  __syncthreads();
  for (int e = tid(); e < G * hd; e += KVM_THREADS) {
    const int g = e / hd, dd = e % hd;
    float M = -INFINITY;
#pragma unroll
    for (int v = 0; v < KVM_WAVES; ++v) M = fmaxf(M, ((const LDS float*)c.smem)[v * (16 * hd + 16) + 16 * hd + g]);
    float acc = 0.f, ls = 0.f;
#pragma unroll
    for (int v = 0; v < KVM_WAVES; ++v) {
      const LDS float* x = (const LDS float*)c.smem + v * (16 * hd + 16);
      const float mv = x[16 * hd + g], ew = mv == -INFINITY ? 0.f : __expf(mv - M);
      acc += ew * (x[g * hd + dd] + x[(g + G) * hd + dd]);
      ls += ew * x[16 * hd + 8 + g];
    }
    const long long r = (((long long)bb * S + s) * H + kvh * G + g) * part.cols;
    stwt32(part.f() + (r + dd), acc);
    if (dd == 0) { stwt32(part.f() + (r + hd), M); stwt32(part.f() + (r + hd + 1), ls); }
  }
}
// LONG: long splits may take the MFMA form (a call site the batch-1 static kernel is built without: its register
// allocation spills with it).
template <int G, bool LONG = true>
__device__ __forceinline__ void attn_part_body(const Ctx& c, bool qkn, bool merge = false) {
  const View q = uniform_view(c.buf(0)), kc = uniform_view(c.buf(1)), vc = uniform_view(c.buf(2)), lens = uniform_view(c.buf(3));
  const View part = uniform_view(c.buf(4)), kn = uniform_view(c.buf(5)), vn = uniform_view(c.buf(6));
  const int bb = c.i(7), kvh = c.i(8), s = c.i(9), S = c.i(10), H = c.i(11), Hkv = c.i(12), Tmax = c.i(14);
  const float sc = c.f(15), th = c.f(16);
  const int fl = c.i(17);
  constexpr int hd = ATT_HD, half = 64;
  constexpr int DR = ATT_DR, DB = ATT_DB;               // rounds of 4 tokens per wave; tokens per block (160)
  int L, j0, nk;
  if (!attn_split(c, L, j0, nk)) { if (tid() == 0) c.fail(KVM_ERR_OP_KVLEN, bb, lens.i()[bb]); return; }
  const int n = L + 1, j1 = j0 + nk;
  const bool pre = rfl(c.pre) && nk > 0;                // block 0 and the rotation table staged before the wait
  const bool mf = LONG && nk > ATT_MFMA_MIN;            // a long split: the MFMA form (its staged block 0 unused)
  const long long base = ((long long)bb * Hkv + kvh) * Tmax;
  const int l = lane(), w = wave(), cb = l & 15, ts = l >> 4, d0 = 8 * cb;
  LDS uint16_t* Ks = (LDS uint16_t*)c.smem;             // [DB][hd] block 0 K rows (prefetched), then V rows
  LDS uint16_t* Vs = Ks + DB * hd;
  LDS float* red = (LDS float*)(c.smem + ATT_RED_OFF);  // [4 waves][G] block max / sum
  LDS float* racc = (LDS float*)c.smem;                 // [16 token slots][G][hd] P V partials, after the last block
  LDS float* rot = (LDS float*)(c.smem + ATT_ROT_OFF);  // [half] sin, [half] cos of this position's angles
  // query (rotated when flag 1, rounded to bf16 when flag 2), times the score scale. This lane's 8 dimensions and their
  // rotation partners (d -+ 64) are loaded as vectors, every load before any use.
  float qr[G][8], qp[G][8];
  const bool qv = (q.cols % 8) == 0 && q.dtype != 1;
  if (qv && q.dtype == 2) {
    u16x8_t a[G], b2[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const long long qo = (long long)bb * q.cols + (long long)(kvh * G + g) * hd;
      a[g] = *(const GLOBAL u16x8_t*)(q.h() + qo + d0);
      b2[g] = *(const GLOBAL u16x8_t*)(q.h() + qo + (d0 ^ half));
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) { qr[g][e] = bf2f(a[g][e]); qp[g][e] = bf2f(b2[g][e]); }
  } else if (qv && q.dtype == 0) {                     // f32: four 16-byte loads per head, all issued before any use
    f32x4n a[G][2], b2[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const long long qo = (long long)bb * q.cols + (long long)(kvh * G + g) * hd;
      const GLOBAL f32x4n* pa = (const GLOBAL f32x4n*)(q.f() + qo + d0);
      const GLOBAL f32x4n* pb = (const GLOBAL f32x4n*)(q.f() + qo + (d0 ^ half));
      a[g][0] = pa[0]; a[g][1] = pa[1]; b2[g][0] = pb[0]; b2[g][1] = pb[1];
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) { qr[g][e] = a[g][e >> 2][e & 3]; qp[g][e] = b2[g][e >> 2][e & 3]; }
  } else {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const long long qo = (long long)bb * q.cols + (long long)(kvh * G + g) * hd;
#pragma unroll
      for (int e = 0; e < 8; ++e) { qr[g][e] = q.ld(qo + d0 + e); qp[g][e] = q.ld(qo + (d0 ^ half) + e); }
    }
  }
  if (qkn) {                                           // per-head RMSNorm: the 16 lanes of a DPP row hold one head's 128 dims
    const View qg = uniform_view(c.buf(18));
    const float eps = c.f(20);
    float gq[8], gp[8];
    const GLOBAL f32x4n* ga = (const GLOBAL f32x4n*)(qg.f() + d0);        // gamma: f32, 128 values (validated)
    const GLOBAL f32x4n* gb = (const GLOBAL f32x4n*)(qg.f() + (d0 ^ half));
    const f32x4n g0 = ga[0], g1 = ga[1], p0 = gb[0], p1 = gb[1];
#pragma unroll
    for (int e = 0; e < 4; ++e) { gq[e] = g0[e]; gq[e + 4] = g1[e]; gp[e] = p0[e]; gp[e + 4] = p1[e]; }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += qr[g][e] * qr[g][e];
      const float rs = 1.f / sqrtf(row16_sum(ss) / (float)hd + eps);
#pragma unroll
      for (int e = 0; e < 8; ++e) { qr[g][e] = (qr[g][e] * rs) * gq[e]; qp[g][e] = (qp[g][e] * rs) * gp[e]; }
    }
  }
  // the rotation table (computed while the query loads are in flight)
  if (fl & 1) {
    if (!pre) attn_rot_table(L, th, rot);
    __syncthreads();
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = d0 + e;
      float x = qr[g][e];
      if (fl & 1) {
        const double sn = rot[d % half], co = rot[half + d % half], y = qp[g][e];
        x = d < half ? (float)((double)x * co - y * sn) : (float)(y * sn + (double)x * co);
        if (fl & 2) x = round_bf(x);
      }
      qr[g][e] = x * sc;
    }
  if (pre) {                                            // the staged block has landed (every wave's own loads), for all waves
    wait_vm_c<0>();
    __syncthreads();
  }
  if ((fl & 1) && j0 <= n - 1 && n - 1 < j1) {          // this split holds the new key: store it (rotated) and its value
    const long long row = base + n - 1;
    const int srow = n - 1 - j0;                         // its staging slot, when staged (block 0, prefetched)
    const bool stage = pre && srow < DB;
    if (tid() < half) {                                  // wave 0: one lane per rotation pair
      const int i = tid();
      const double sn = rot[i], co = rot[half + i];
      float k1 = kn.at(bb, kvh * hd + i), k2 = kn.at(bb, kvh * hd + i + half);
      if (qkn) {
        const View kg = uniform_view(c.buf(19));
        const float rs = 1.f / sqrtf(wave_sum(k1 * k1 + k2 * k2) / (float)hd + c.f(20));
        k1 = (k1 * rs) * kg.f()[i]; k2 = (k2 * rs) * kg.f()[i + half];
      }
      const double x1 = k1, x2 = k2;
      const float r1 = (float)(x1 * co - x2 * sn), r2 = (float)(x1 * sn + x2 * co);
      kc.st(row * kc.cols + i, r1); kc.st(row * kc.cols + i + half, r2);
      if (stage) { Ks[srow * hd + i] = f2bf(r1); Ks[srow * hd + i + half] = f2bf(r2); }
    }
    for (int k = tid(); k < hd; k += KVM_THREADS) {
      const float v = vn.at(bb, kvh * hd + k);
      vc.st(row * vc.cols + k, v);
      if (stage) Vs[srow * hd + k] = f2bf(v);
    }
  }
  __syncthreads();                                      // the new row is stored before any block reads it
  if (nk == 0) {
    for (int e = tid(); e < G * (hd + 2); e += KVM_THREADS) {
      const int g = e / (hd + 2), k = e % (hd + 2);
      const long long r = (((long long)bb * S + s) * H + kvh * G + g) * part.cols;
      stwt32(part.f() + (r + k), k < hd ? 0.f : (k == hd ? ATTN_EMPTY_M : 0.f));
    }
    if (merge) attn_arrive<G>(c, bb, kvh, S, H, Hkv);
    return;
  }
  if (mf) {                                             // the MFMA form, the query block through LDS
    if (w == 0 && ts == 0)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) ((LDS float*)(c.smem + ATT_MQ_OFF))[g * hd + d0 + e] = qr[g][e];
    wait_stores();                                      // the new row is in L2 before the direct loads
    __syncthreads();
    attn_split_mfma<G>(c, j0, nk);
    if (merge) attn_arrive<G>(c, bb, kvh, S, H, Hkv);
    return;
  }
  float mrun[G], lrun[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    mrun[g] = -INFINITY; lrun[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }
  // K and V rows of a block in registers. The next block's K rows are requested once this block's scores are done
  // (under its softmax and P V), its V rows once this block's P V is done (under the next scores): the registers
  // each set occupies are free by then, so the pipeline costs no registers.
  u16x8_t kr[DR], vr[DR];
  auto load_k = [&](int b0) {
#pragma unroll
    for (int i = 0; i < DR; ++i) {
      const long long row = base + j0 + min(b0 + w * 4 * DR + 4 * i + ts, nk - 1);
      kr[i] = *(const GLOBAL u16x8_t*)(kc.h() + row * kc.cols + d0);
    }
  };
  auto load_v = [&](int b0) {
#pragma unroll
    for (int i = 0; i < DR; ++i) {
      const long long row = base + j0 + min(b0 + w * 4 * DR + 4 * i + ts, nk - 1);
      vr[i] = *(const GLOBAL u16x8_t*)(vc.h() + row * vc.cols + d0);
    }
  };
  if (pre) {
#pragma unroll
    for (int i = 0; i < DR; ++i) {
      const int slot = w * 4 * DR + 4 * i + ts;
      kr[i] = *(const LDS u16x8_t*)(Ks + slot * hd + d0);
      vr[i] = *(const LDS u16x8_t*)(Vs + slot * hd + d0);
    }
  } else {
    load_k(0);
    load_v(0);
  }
  for (int b0 = 0; b0 < nk; b0 += DB) {
    float sv[DR][G];
    float mb[G];
#pragma unroll
    for (int g = 0; g < G; ++g) mb[g] = -INFINITY;
#pragma unroll
    for (int i = 0; i < DR; ++i) {
      const bool live = b0 + w * 4 * DR + 4 * i + ts < nk;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a += qr[g][e] * bf2f(kr[i][e]);
        a = row16_sum(a);
        sv[i][g] = live ? a : -INFINITY;
        mb[g] = fmaxf(mb[g], sv[i][g]);
      }
    }
    const bool more = b0 + DB < nk;
    if (more) load_k(b0 + DB);
#pragma unroll
    for (int g = 0; g < G; ++g) { mb[g] = fmaxf(mb[g], __shfl_xor(mb[g], 16, 64)); mb[g] = fmaxf(mb[g], __shfl_xor(mb[g], 32, 64)); }
    __syncthreads();                                    // red is free
    if (l == 0)
#pragma unroll
      for (int g = 0; g < G; ++g) red[w * 8 + g] = mb[g];
    __syncthreads();
    float scale[G], ps[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m = fmaxf(fmaxf(red[g], red[8 + g]), fmaxf(red[16 + g], red[24 + g]));
      const float mn = fmaxf(mrun[g], m);
      scale[g] = __expf(mrun[g] - mn);                  // 0 on the first block
      mrun[g] = mn;
      ps[g] = 0.f;
    }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] *= scale[g];
#pragma unroll
    for (int i = 0; i < DR; ++i)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float p = __expf(sv[i][g] - mrun[g]);     // 0 for dead slots
        ps[g] += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] += p * bf2f(vr[i][e]);
      }
    if (more) load_v(b0 + DB);
#pragma unroll
    for (int g = 0; g < G; ++g) { ps[g] += __shfl_xor(ps[g], 16, 64); ps[g] += __shfl_xor(ps[g], 32, 64); }
    __syncthreads();
    if (l == 0)
#pragma unroll
      for (int g = 0; g < G; ++g) red[32 + w * 8 + g] = ps[g];
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) lrun[g] = lrun[g] * scale[g] + ((red[32 + g] + red[40 + g]) + (red[48 + g] + red[56 + g]));
  }
  // P V: the partial sums of the 16 token slots (4 per wave) through LDS, added in slot order
  __syncthreads();
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 8; ++e) racc[((w * 4 + ts) * G + g) * hd + d0 + e] = acc[g][e];
  __syncthreads();
  for (int e = tid(); e < G * hd; e += KVM_THREADS) {
    const int g = e / hd, k = e % hd;
    float t = 0.f;
#pragma unroll
    for (int q2 = 0; q2 < 16; ++q2) t += racc[(q2 * G + g) * hd + k];
    const long long r = (((long long)bb * S + s) * H + kvh * G + g) * part.cols;
    stwt32(part.f() + (r + k), t);
    if (k == 0) { stwt32(part.f() + (r + hd), mrun[g]); stwt32(part.f() + (r + hd + 1), lrun[g]); }
  }
  if (merge) attn_arrive<G>(c, bb, kvh, S, H, Hkv);
}
template <int G> __device__ __noinline__ void attn_decode_part_fast(const Ctx& c, bool qkn, bool merge = false) { attn_part_body<G>(c, qkn, merge); }
__device__ __noinline__ void op_attn_decode_part_any(const Ctx& c) {
  const View kc = c.buf(1), vc = c.buf(2);
  const int H = c.i(11), Hkv = c.i(12), hd = c.i(13), G = H / Hkv;
  const bool ok = kc.dtype == 2 && vc.dtype == 2 && hd == 128 && (kc.cols % 8) == 0 && (vc.cols % 8) == 0;
  if (ok && G == 4) attn_decode_part_fast<4>(c, false);
  else if (ok && G == 8) attn_decode_part_fast<8>(c, false);
  else if (ok && G == 2) attn_decode_part_fast<2>(c, false);
  else if (ok && G == 1) attn_decode_part_fast<1>(c, false);
  else op_attn_decode_part(c);
}
// Op 306 (validated to the streaming path's shapes: hd 128, bf16 caches, G in {1, 2, 4, 8}).
__device__ __noinline__ void op_attn_decode_part_qkn(const Ctx& c) {
  const int G = c.i(11) / c.i(12);
  if (G == 4) attn_decode_part_fast<4>(c, true);
  else if (G == 8) attn_decode_part_fast<8>(c, true);
  else if (G == 2) attn_decode_part_fast<2>(c, true);
  else attn_decode_part_fast<1>(c, true);
}

// Op 310 (validated as op 306): op 306, then the last split of its kv head merges the head's query heads.
__device__ __noinline__ void op_attn_decode_part_merge(const Ctx& c) {
  const int G = c.i(11) / c.i(12);
  if (G == 4) attn_decode_part_fast<4>(c, true, true);
  else if (G == 8) attn_decode_part_fast<8>(c, true, true);
  else if (G == 2) attn_decode_part_fast<2>(c, true, true);
  else attn_decode_part_fast<1>(c, true, true);
}

// Merge of the splits (registry op 136): per head, the split weights e_s = exp(m_s - max m) (live splits only) are
// computed once into LDS, then each output element is one pass over the splits.
__device__ __forceinline__ void attn_merge(const View& part, const View& o, int bb, int h0, int h1, int S, int H, int hd, LDS char* smem) {
  LDS float* w = (LDS float*)smem;        // [h1-h0][S] split weights, then [h1-h0] 1/denominator
  LDS float* inv = w + (h1 - h0) * S;
  for (int h = h0 + wave(); h < h1; h += KVM_WAVES) {
    float M = -INFINITY;
    for (int s = lane(); s < S; s += 64) { long long r = (((long long)bb * S + s) * H + h) * part.cols; if (part.f()[r + hd + 1] > 0.f) M = fmaxf(M, part.f()[r + hd]); }
    M = wave_max(M);
    float den = 0.f;
    for (int s = lane(); s < S; s += 64) {
      long long r = (((long long)bb * S + s) * H + h) * part.cols;
      float l = part.f()[r + hd + 1], e = l > 0.f ? __expf(part.f()[r + hd] - M) : 0.f;
      w[(h - h0) * S + s] = e; den += e * l;
    }
    den = wave_sum(den);
    if (lane() == 0) inv[h - h0] = 1.f / den;
  }
  __syncthreads();
  for (int e = tid(); e < (h1 - h0) * hd; e += KVM_THREADS) {
    int hh = e / hd, k = e % hd; float num = 0.f;
    const GLOBAL float* src = part.f() + (((long long)bb * S) * H + h0 + hh) * part.cols + k;
    const long long step = (long long)H * part.cols;
    int s = 0;
    for (; s + 8 <= S; s += 8) {                 // eight independent loads in flight
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = src[(s + i) * step];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; ++i) num += w[hh * S + s + i] * v[i];
    }
    for (; s < S; ++s) num += w[hh * S + s] * src[s * step];
    o.st((long long)bb * o.cols + (h0 + hh) * hd + k, num * inv[hh]);
  }
}

__device__ __forceinline__ void attn_merge_body(const Ctx& c) {
  attn_merge(c.buf(0), c.buf(1), c.i(2), c.i(3), c.i(4), c.i(5), c.i(6), c.i(7), c.smem);
}
__device__ __noinline__ void op_attn_decode_merge(const Ctx& c) { attn_merge_body(c); }

}  // namespace kvm
