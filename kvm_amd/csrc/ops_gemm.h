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
      if (m < M && n < N) { float u = t[q]; stwt32(up.f() + ((long long)m * up.cols + n), u); stwt32(out.f() + ((long long)m * out.cols + n), silu_f(gate.at(m, n)) * u); }
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
        stwt32(dg.f() + ((long long)m * dg.cols + n), dh * (up.at(m, n) * silu_d_f(g)));
        stwt32(du.f() + ((long long)m * du.cols + n), dh * silu_f(g));
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------------------------- bf16 MFMA engine
// Layout and schedule (one workgroup = four wave64s; waves in a 2 x 2 grid, each owning (TM/2) x (TN/2) of the tile):
//   * K advances in slabs of GK = 64. Each operand slab sits in LDS as [row][k] (row = m for A, n for B) with a row
//     stride of GS = 72 elements, and the eight 16-byte k-chunks of a row are XOR-swizzled by (row >> 4) & 7. With
//     that, the MFMA fragment reads (16 consecutive rows, one chunk) and the stores of transposed operands (16 row
//     groups, one chunk) both touch every LDS bank once.
//   * Operands stored k-contiguous are fetched as 16-byte row pieces (8 lanes read one 128-byte row segment) and
//     written to LDS unchanged. Operands stored row-contiguous ([K][rows]: A with flag 1, B without flag 2) are fetched
//     as 16-byte pieces along the rows (a wave reads whole 128-byte lines); each thread fetches KPT consecutive k rows
//     of one 8-row group and transposes them in registers, so it writes 8 rows x KPT k values with 8 LDS stores.
//   * Two LDS buffers: while slab s is multiplied, slab s+1 is already loaded into registers; it is written to the
//     other buffer afterwards and one barrier per slab separates the phases.
//   * MFMA v_mfma_f32_32x32x16_bf16 with the B fragment as the first source, so the accumulator holds D^T: each lane
//     owns 4 consecutive output columns of one row, and the epilogue reads and writes 4-element vectors.
typedef uint16_t u16x4_t __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
constexpr int GK = 64;
constexpr int GS = GK + 8;

// LDS element offset of k-chunk `ch` (8 k values) of tile row `row`.
__device__ __forceinline__ int gsw(int row, int ch) { return row * GS + ((ch ^ ((row >> 4) & 7)) << 3); }

// Element-wise form of load8 for tile edges (rows / K past the matrix, unaligned or short vectors).
__device__ __noinline__ u16x8_t load8_tail(const View& X, long long base, int valid) {
  u16x8_t r;
  for (int i = 0; i < 8; ++i) r[i] = i < valid ? (X.dtype == 2 ? X.h()[base + i] : f2bf(X.f()[base + i])) : (uint16_t)0;
  return r;
}
// 8 consecutive elements (along X's contiguous dimension) as bf16 bits; elements past `valid` read as 0.
__device__ __forceinline__ u16x8_t load8(const View& X, long long base, int valid) {
  if (valid >= 8 && (base & 7) == 0) {
    if (X.dtype == 2) return *(const GLOBAL u16x8_t*)(X.h() + base);
    const GLOBAL f32x4n* p = (const GLOBAL f32x4n*)(X.f() + base);
    f32x4n a = p[0], b = p[1];
    return u16x8_t{f2bf(a.x), f2bf(a.y), f2bf(a.z), f2bf(a.w), f2bf(b.x), f2bf(b.y), f2bf(b.z), f2bf(b.w)};
  }
  return load8_tail(X, base, valid);
}

// A view with every field made wave-uniform (scalar registers): the operand loads then address through buffer
// descriptors in SGPRs and nothing is re-read from memory inside the K loop.
__device__ __forceinline__ View uniform_view(const View& v) {
  const uint64_t p = (uint64_t)(uintptr_t)v.p;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p), hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(p >> 32));
  return View{(void*)(uintptr_t)(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(v.rows), __builtin_amdgcn_readfirstlane(v.cols),
              __builtin_amdgcn_readfirstlane(v.dtype)};
}
__device__ __forceinline__ Epi uniform_epi(const Epi& e) {
  return Epi{uniform_view(e.out), uniform_view(e.bias), uniform_view(e.res), uniform_view(e.pre),
             __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(e.alpha))), __builtin_amdgcn_readfirstlane(e.accum), __builtin_amdgcn_readfirstlane(e.ge),
             __builtin_amdgcn_readfirstlane(e.dg)};
}
// Raw buffer descriptor over `bytes` bytes from p (gfx9 word 3); loads past the range return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, long long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)min(bytes, 0x7fffffffll), 0x00020000);
}

// Direct HBM -> LDS loads (buffer_load_dwordx4 ... lds: lane l's 16 bytes land at M0 + 16 l). They are issued from
// inline assembly on purpose: the compiler tracks its own LDS-DMA loads and, lacking alias information, waits for all
// of them (vmcnt(0)) before any later LDS read, which drains every prefetch pipeline built on them. Code using dma16
// therefore orders its LDS reads itself, with wait_vm before reading a staged block and a barrier where other waves
// read it.
typedef int i32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4_t dma_rsrc(const void* p, long long bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)p;
  const long long nb = bytes < 0 ? 0 : min(bytes, 0x7fffffffll);
  return i32x4_t{__builtin_amdgcn_readfirstlane((int)(uint32_t)a), __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffff)),
                 __builtin_amdgcn_readfirstlane((int)nb), 0x00020000};
}
// 16 bytes per lane from rs + voff + soff into LDS at dst + 16 * lane (dst uniform across the wave).
__device__ __forceinline__ void dma16(i32x4_t rs, int voff, int soff, const LDS void* dst) {
  const int m = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)dst);
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" :: "s"(m), "v"(voff), "s"(rs), "s"(soff) : "memory", "m0");
}

// One operand slab: R tile rows x GK k values. NV 16-byte vectors per thread.
//   KC (k-contiguous, element (r, k) at X[r*cols + k]): vector q of a thread is row idx/8, k-chunk idx%8 with
//     idx = tid + 256q, so 8 lanes read one 128-byte row segment.
//   row-contiguous (element (r, k) at X[k*cols + r]): a thread takes rows 8*(tid % MV) .. +8 at k rows
//     KPT*(tid / MV) .. +KPT, so a wave reads whole lines along the rows.
// The fast path (bf16, whole tile inside the matrix, K a whole number of slabs) loads through a buffer descriptor
// with per-thread 32-bit offsets fixed for the task and a uniform per-slab offset.
template <int R> struct GTile {
  static constexpr int NV = R * GK / 8 / KVM_THREADS;    // R / 32
  static constexpr int KPT = NV;                         // row-contiguous operands: k rows per thread
  static constexpr int MV = R / 8;                       // row-contiguous operands: 8-row groups
  static_assert(NV >= 2 && KPT * (KVM_THREADS / MV) == GK, "tile shape");
  u16x8_t v[NV];
  __amdgpu_buffer_rsrc_t rs;
  int voff[NV];
  template <bool KC> __device__ __forceinline__ void init_fast(const View& X, int r0) {
    if constexpr (KC) {
      const GLOBAL uint16_t* base = X.h() + (long long)r0 * X.cols;
      rs = buf_rsrc((const void*)base, ((long long)X.rows - r0) * X.cols * 2);
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const int idx = tid() + q * KVM_THREADS;
        voff[q] = ((idx >> 3) * X.cols + (idx & 7) * 8) * 2;
      }
    } else {
      const GLOBAL uint16_t* base = X.h() + r0;
      rs = buf_rsrc((const void*)base, (long long)X.rows * X.cols * 2 - (long long)r0 * 2);
#pragma unroll
      for (int q = 0; q < NV; ++q) voff[q] = (((tid() / MV) * KPT + q) * X.cols + (tid() % MV) * 8) * 2;
    }
  }
  template <bool KC> __device__ __forceinline__ void fetch_fast(int k0, int cols) {
    const int so = KC ? k0 * 2 : k0 * cols * 2;
#pragma unroll
    for (int q = 0; q < NV; ++q) v[q] = (u16x8_t)__builtin_amdgcn_raw_buffer_load_b128(rs, voff[q], so, 0);
  }
  template <bool KC> __device__ __forceinline__ void fetch_any(const View& X, int r0, int rows, int k0, int K) {
    if constexpr (KC) {
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const int idx = tid() + q * KVM_THREADS, r = r0 + (idx >> 3), k = k0 + (idx & 7) * 8;
        v[q] = load8(X, (long long)r * X.cols + k, r < rows ? min(8, K - k) : 0);
      }
    } else {
      const int r = r0 + (tid() % MV) * 8, kb = k0 + (tid() / MV) * KPT;
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const int k = kb + q;
        v[q] = load8(X, (long long)k * X.cols + r, k < K ? min(8, rows - r) : 0);
      }
    }
  }
  template <bool FAST, bool KC> __device__ __forceinline__ void fetch(const View& X, int r0, int rows, int k0, int K) {
    if constexpr (FAST) fetch_fast<KC>(k0, X.cols);
    else fetch_any<KC>(X, r0, rows, k0, K);
  }
  template <bool KC> __device__ __forceinline__ void store(LDS uint16_t* lds) const {
    if constexpr (KC) {
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const int idx = tid() + q * KVM_THREADS;
        *(LDS u16x8_t*)(lds + gsw(idx >> 3, idx & 7)) = v[q];
      }
    } else {
      const int rg = (tid() % MV) * 8, kq = (tid() / MV) * KPT;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int o = gsw(rg + i, kq >> 3) + (kq & 7);
        if constexpr (KPT == 8) {
          u16x8_t w;
#pragma unroll
          for (int q = 0; q < 8; ++q) w[q] = v[q][i];
          *(LDS u16x8_t*)(lds + o) = w;
        } else if constexpr (KPT == 4) {
          u16x4_t w;
#pragma unroll
          for (int q = 0; q < 4; ++q) w[q] = v[q][i];
          *(LDS u16x4_t*)(lds + o) = w;
        } else {
          u16x2_t w;
          w[0] = v[0][i]; w[1] = v[1][i];
          *(LDS u16x2_t*)(lds + o) = w;
        }
      }
    }
  }
};

// 4 consecutive elements of a view at flat offset o (o % 4 == 0, cols % 4 == 0), widened to f32 / rounded on store.
__device__ __forceinline__ f32x4n ld4(const View& X, long long o) {
  if (X.dtype == 2) {
    const u16x4_t h = *(const GLOBAL u16x4_t*)(X.h() + o);
    return f32x4n{bf2f(h[0]), bf2f(h[1]), bf2f(h[2]), bf2f(h[3])};
  }
  return *(const GLOBAL f32x4n*)(X.f() + o);
}
__device__ __forceinline__ void st4(const View& X, long long o, f32x4n v) {
  if (X.dtype == 2) stwt_bf4(X.h() + o, v.x, v.y, v.z, v.w);
  else if (X.n() * 4 < 0x7fffffffll) stwt_buf(wt_rsrc(X.p, X.n() * 4), (int)o * 4, v);
  else stwt_f4(X.f() + o, v);
}

typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
// Four consecutive f32 or bf16 elements through a buffer descriptor: one 16-byte load either way (bf16 uses its
// first half), converted by selects, so a batch of these has no branches for the compiler to wait at.
struct Ld4 {
  __amdgpu_buffer_rsrc_t rs;
  int es;                              // element size: 4 (f32) or 2 (bf16)
  __device__ __forceinline__ void init(const View& v, bool use = true) {
    es = v.dtype == 2 ? 2 : 4;
    rs = v.ok() && use ? buf_rsrc((const void*)v.p, (long long)v.rows * v.cols * es) : buf_rsrc((const void*)v.p, 0);
  }
  __device__ __forceinline__ u32x4_t raw(int idx) const { return __builtin_amdgcn_raw_buffer_load_b128(rs, idx * es, 0, 0); }
  __device__ __forceinline__ f32x4n cvt(u32x4_t r) const {
    const bool h = es == 2;                      // selects, not a branch: a branch makes every load wait alone
    return f32x4n{__uint_as_float(h ? r.x << 16 : r.x), __uint_as_float(h ? r.x & 0xffff0000u : r.y),
                  __uint_as_float(h ? r.y << 16 : r.z), __uint_as_float(h ? r.y & 0xffff0000u : r.w)};
  }
  __device__ __forceinline__ f32x4n get(int idx) const { return cvt(raw(idx)); }
};

__device__ __noinline__ void epi_tail(Epi e, int N, int m, int n, f32x4n a) {
  for (int i = 0; i < 4 && n + i < N; ++i) e.put(m, n + i, a[i]);
}
// The arguments of a GEMM tile task (ops 114 and 122 share the layout a, b, out, bias, res, pre, m0, n0, M, N, K,
// flags, alpha), read from the dispatcher's LDS copies and made wave-uniform, so nothing is re-read from memory later.
struct GemmArgs { View A, B; Epi e; int m0, n0, M, N, K, fl; };
__device__ __forceinline__ int rfl(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ GemmArgs gemm_args(const Ctx& c) {
  const LDS View* vw = c.views;
  const LDS int32_t* a = c.a;
  auto V = [&](int k) {
    const View v = a[k] < 0 ? View{nullptr, 0, 0, 0} : View{vw[k].p, vw[k].rows, vw[k].cols, vw[k].dtype};
    return uniform_view(v);
  };
  const int fl = rfl(a[11]);
  GemmArgs g;
  g.A = V(0); g.B = V(1);
  g.e = Epi{V(2), V(3), V(4), V(5), __int_as_float(rfl(a[12])), fl & 4, fl & 8, fl & 512};
  g.m0 = rfl(a[6]); g.n0 = rfl(a[7]); g.M = rfl(a[8]); g.N = rfl(a[9]); g.K = rfl(a[10]); g.fl = fl;
  return g;
}

// Epilogue. The accumulators hold D^T: acc[i][j][r] is row m = l % 32 of block i, column 8*(r/4) + 4*(l/32) + r%4 of
// block j. The whole tile is staged in LDS as f32 (TM x TN floats, at most 128 KiB), its 16-byte column chunks XOR-
// swizzled by row so that both the accumulator writes (16 rows per phase, one chunk) and the row reads (one row, 16
// chunks) are conflict-free. The epilogue proper then runs as one out-of-line function per tile shape and output
// type: the accumulators are dead by then, so the call saves almost nothing, and its code exists once instead of once
// per operand orientation. There every lane owns a fixed 4-column piece (bias loaded once) and the waves take rows in
// turn, with the res / pre / previous-output loads of a batch of rows issued together through branch-free buffer
// loads; every row is stored as whole lines. Pieces that are not whole, aligned vectors take the scalar path.
// Rows of a wave whose second-operand loads (residual, pre-activation, previous output) are issued together, in the
// straight-line epilogues (KVM_EPI_NB) and the general one (KVM_EPI_NB2). Larger batches measured slower: the
// epilogue is an out-of-line function, and every register it uses beyond the caller-saved ones is saved and restored
// around each call.
#ifndef KVM_EPI_NB
#define KVM_EPI_NB 8
#endif
#ifndef KVM_EPI_NB2
#define KVM_EPI_NB2 4
#endif
template <int TN> __device__ __forceinline__ int epi_swz(int r) { return r & ((TN / 4 < 32 ? TN / 4 : 32) - 1); }

// Whole, aligned tile with one of the epilogues the GPT graphs use, as straight-line code: KIND 0 = (bias), 1 = bias +
// residual, 2 = accumulate into the output, 3 = times gelu'(pre), 4 = pre = bias-added value, out = gelu(pre).
// The second operand of kinds 1-3 is loaded raw for a batch of rows before any of them is used.
template <int TM, int TN, bool OBF, int KIND>
__device__ __forceinline__ void epi_rows(const Ctx& c, const GemmArgs& g) {
  constexpr int LPR = TN / 4, RPI = 64 / LPR, NI = TM / KVM_WAVES / RPI, NB = NI < KVM_EPI_NB ? NI : KVM_EPI_NB;
  const Epi& e = g.e;
  const LDS float* et = (const LDS float*)c.smem;
  const int l = lane(), w = wave(), ch = l % LPR, n = g.n0 + 4 * ch;
  Ld4 lb, lx;
  lb.init(e.bias);
  const View& xv = KIND == 1 ? e.res : KIND == 2 ? e.out : e.pre;
  lx.init(xv, KIND >= 1 && KIND <= 3);
  const f32x4n bv = lb.get(n);
  const __amdgpu_buffer_rsrc_t orsrc = wt_rsrc(e.out.p, (long long)g.M * e.out.cols * (OBF ? 2 : 4));   // output rows (small: < 2^31 bytes)
  const int xc = xv.cols;
  for (int k0 = 0; k0 < NI; k0 += NB) {
    u32x4_t raw[NB];
    f32x4n a[NB];
    if constexpr (KIND >= 1 && KIND <= 3) {
#pragma unroll
      for (int u = 0; u < NB; ++u) raw[u] = lx.raw((g.m0 + ((k0 + u) * KVM_WAVES + w) * RPI + l / LPR) * xc + n);
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int r = ((k0 + u) * KVM_WAVES + w) * RPI + l / LPR;
      a[u] = *(const LDS f32x4n*)(et + r * TN + 4 * (ch ^ epi_swz<TN>(r)));
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int m = g.m0 + ((k0 + u) * KVM_WAVES + w) * RPI + l / LPR;
      f32x4n v = a[u] * e.alpha + bv;
      if constexpr (KIND == 1 || KIND == 2) v += lx.cvt(raw[u]);
      if constexpr (KIND == 3) {
        const f32x4n p = lx.cvt(raw[u]);
        v.x *= gelu_grad_f(p.x); v.y *= gelu_grad_f(p.y); v.z *= gelu_grad_f(p.z); v.w *= gelu_grad_f(p.w);
      }
      if constexpr (KIND == 4) {
        st4(e.pre, (long long)m * e.pre.cols + n, v);
        v.x = gelu_f(v.x); v.y = gelu_f(v.y); v.z = gelu_f(v.z); v.w = gelu_f(v.w);
      }
      if constexpr (OBF) stwt_bf4_buf(orsrc, (m * e.out.cols + n) * 2, v);
      else stwt_buf(orsrc, (m * e.out.cols + n) * 4, v);
    }
  }
}

template <int TM, int TN, bool OBF>
__device__ __noinline__ void gemm_epilogue(const Ctx& c, int moff) {
  constexpr int LPR = TN / 4, RPI = 64 / LPR, NI = TM / KVM_WAVES / RPI;   // lanes per row, rows per instruction
  constexpr int NB = NI < KVM_EPI_NB2 ? NI : KVM_EPI_NB2;
  GemmArgs g = gemm_args(c);
  g.m0 += moff;                                          // the staged rows start at tile row moff
  const Epi& e = g.e;
  const LDS float* et = (const LDS float*)c.smem;
  const int l = lane(), w = wave(), ch = l % LPR, n = g.n0 + 4 * ch;
  const long long lim = 0x7fffffffll;
  const bool small = (long long)g.M * e.out.cols * 4 < lim && (long long)g.M * e.res.cols * 4 < lim && (long long)g.M * e.pre.cols * 4 < lim;
  const bool vec = (e.out.cols & 3) == 0 && (!e.res.ok() || (e.res.cols & 3) == 0) && (!e.pre.ok() || (e.pre.cols & 3) == 0);
  const bool fast = vec && small && n + 4 <= g.N;
  const bool dg = e.dg != 0, ge = e.ge != 0, spre = !dg && e.pre.ok(), loads = e.res.ok() || dg || e.accum;
  if (vec && small && g.m0 + TM <= g.M && g.n0 + TN <= g.N) {
    const bool res = e.res.ok(), acc = e.accum != 0;
    if (!res && !acc && !dg && !ge && !spre) { epi_rows<TM, TN, OBF, 0>(c, g); return; }
    if (res && !acc && !dg && !ge && !spre) { epi_rows<TM, TN, OBF, 1>(c, g); return; }
    if (!res && acc && !dg && !ge && !spre) { epi_rows<TM, TN, OBF, 2>(c, g); return; }
    if (!res && !acc && dg) { epi_rows<TM, TN, OBF, 3>(c, g); return; }
    if (!res && !acc && !dg && ge && spre) { epi_rows<TM, TN, OBF, 4>(c, g); return; }
  }
  Ld4 lb, lr, lp, lo;
  lb.init(e.bias); lr.init(e.res); lp.init(e.pre, dg); lo.init(e.out, e.accum != 0);
  const f32x4n bv = lb.get(n);
  const __amdgpu_buffer_rsrc_t orsrc = wt_rsrc(e.out.p, (long long)g.M * e.out.cols * 4);   // f32 output rows (small: < 2^31 bytes)
  for (int k0 = 0; k0 < NI; k0 += NB) {
    f32x4n rv[NB], pv[NB], ov[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) { rv[u] = f32x4n{0.f, 0.f, 0.f, 0.f}; pv[u] = rv[u]; ov[u] = rv[u]; }
    if (loads && small) {
#pragma unroll
      for (int u = 0; u < NB; ++u) {
        const int m = g.m0 + ((k0 + u) * KVM_WAVES + w) * RPI + l / LPR;
        rv[u] = lr.get(m * e.res.cols + n);
        pv[u] = lp.get(m * e.pre.cols + n);
        ov[u] = lo.get(m * e.out.cols + n);
      }
    }
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int r = ((k0 + u) * KVM_WAVES + w) * RPI + l / LPR, m = g.m0 + r;
      if (m >= g.M) continue;
      const f32x4n a = *(const LDS f32x4n*)(et + r * TN + 4 * (ch ^ epi_swz<TN>(r)));
      if (fast) {
        f32x4n v = a * e.alpha + bv;
        if (dg) {
          v.x *= gelu_grad_f(pv[u].x); v.y *= gelu_grad_f(pv[u].y); v.z *= gelu_grad_f(pv[u].z); v.w *= gelu_grad_f(pv[u].w);
        } else {
          if (spre) st4(e.pre, (long long)m * e.pre.cols + n, v);
          if (ge) { v.x = gelu_f(v.x); v.y = gelu_f(v.y); v.z = gelu_f(v.z); v.w = gelu_f(v.w); }
        }
        v += rv[u] + ov[u];
        if constexpr (OBF) stwt_bf4(e.out.h() + (long long)m * e.out.cols + n, v.x, v.y, v.z, v.w);
        else stwt_buf(orsrc, (m * e.out.cols + n) * 4, v);
      } else if (n < g.N) {
        epi_tail(e, g.N, m, n, a);
      }
    }
  }
}

// Stages the accumulators in LDS (see above) and runs the epilogue; a tile whose f32 copy exceeds the LDS budget
// (256 x 256) goes in two row halves, each staged by the two waves that own it.
template <int TM, int TN>
__device__ __forceinline__ void gemm_store(const Ctx& c, const f32x16 (&acc)[TM / 64][TN / 64], const GemmArgs& g) {
  constexpr int BM = TM / 64, BN = TN / 64, WM = TM / 2, WN = TN / 2;
  constexpr int NH = TM * TN * 4 <= KVM_LDS_BYTES ? 1 : 2, HM = TM / NH;
  static_assert(HM * TN * 4 <= KVM_LDS_BYTES && (NH == 1 || HM == WM), "LDS epilogue");
  const int wm0 = (wave() >> 1) * WM, wn0 = (wave() & 1) * WN, l = lane();
  LDS float* et = (LDS float*)c.smem;
#pragma unroll
  for (int h = 0; h < NH; ++h) {
    __syncthreads();                                       // operand stages / the previous half are no longer read
    if (NH == 1 || (wave() >> 1) == h) {
#pragma unroll
      for (int i = 0; i < BM; ++i) {
        const int r = (NH == 1 ? wm0 : 0) + i * 32 + (l & 31);
#pragma unroll
        for (int j = 0; j < BN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int chunk = (wn0 + j * 32 + 8 * q) / 4 + (l >> 5);
            *(LDS f32x4n*)(et + r * TN + 4 * (chunk ^ epi_swz<TN>(r))) = f32x4n{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          }
      }
    }
    __syncthreads();
    if (g.e.out.dtype == 2) gemm_epilogue<HM, TN, true>(c, h * HM);
    else gemm_epilogue<HM, TN, false>(c, h * HM);
  }
}

template <int TM, int TN, bool FAST, bool AKC, bool BKC>
__device__ __noinline__ void gemm_loop(const Ctx& c) {
  const GemmArgs g = gemm_args(c);
  const View& A = g.A; const View& B = g.B;
  const int m0 = g.m0, n0 = g.n0, M = g.M, N = g.N, K = g.K;
  constexpr int WM = TM / 2, WN = TN / 2, BM = WM / 32, BN = WN / 32;
  LDS uint16_t* lA0 = (LDS uint16_t*)c.smem;
  LDS uint16_t* lB0 = lA0 + TM * GS;
  LDS uint16_t* lA1 = lB0 + TN * GS;
  LDS uint16_t* lB1 = lA1 + TM * GS;
  const int wm0 = (wave() >> 1) * WM, wn0 = (wave() & 1) * WN, l = lane();
  f32x16 acc[BM][BN];
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j) acc[i][j] = f32x16{};
  GTile<TM> ga;
  GTile<TN> gb;
  if constexpr (FAST) { ga.template init_fast<AKC>(A, m0); gb.template init_fast<BKC>(B, n0); }
  ga.template fetch<FAST, AKC>(A, m0, M, 0, K);
  gb.template fetch<FAST, BKC>(B, n0, N, 0, K);
  __syncthreads();                         // the previous task may still read this LDS
  ga.template store<AKC>(lA0);
  gb.template store<BKC>(lB0);
  __syncthreads();
  const int nslab = (K + GK - 1) / GK;
  for (int s = 0; s < nslab; ++s) {
    LDS uint16_t* la = (s & 1) ? lA1 : lA0;
    LDS uint16_t* lb = (s & 1) ? lB1 : lB0;
    const bool more = s + 1 < nslab;
    if (more) {
      ga.template fetch<FAST, AKC>(A, m0, M, (s + 1) * GK, K);
      gb.template fetch<FAST, BKC>(B, n0, N, (s + 1) * GK, K);
    }
#pragma unroll
    for (int kk = 0; kk < GK / 16; ++kk) {
      const int ch = kk * 2 + (l >> 5);
      bf16x8 af[BM], bfr[BN];
#pragma unroll
      for (int i = 0; i < BM; ++i) af[i] = *(const LDS bf16x8*)(la + gsw(wm0 + i * 32 + (l & 31), ch));
#pragma unroll
      for (int j = 0; j < BN; ++j) bfr[j] = *(const LDS bf16x8*)(lb + gsw(wn0 + j * 32 + (l & 31), ch));
#pragma unroll
      for (int i = 0; i < BM; ++i)
#pragma unroll
        for (int j = 0; j < BN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (more) {
      ga.template store<AKC>((s & 1) ? lA0 : lA1);
      gb.template store<BKC>((s & 1) ? lB0 : lB1);
    }
    __syncthreads();
  }
  gemm_store<TM, TN>(c, acc, g);
}

// ---------------------------------------------------------------------------------------------- direct-to-LDS pipeline
// The path for whole bf16 tiles: operands go from HBM straight into LDS (buffer_load ... lds, 16 bytes per lane), so
// no registers stage them and DNS stages of DK k values are in flight at once (prefetch distance DNS-1). A wave's
// direct load writes 1 KiB of LDS, 16 bytes per lane in lane order; each lane picks its global source so that the
// LDS image comes out in the layouts below.
//   k-contiguous operand: [R][DK] bf16, 16-byte k-chunks XOR-swizzled by (row >> 2) & 3; fragments are one
//     ds_read_b128 per lane (16 rows of one chunk touch every bank once).
//   row-contiguous operand: [DK][R] bf16 (the global layout), 16-byte units XOR-swizzled per k row; fragments are two
//     ds_read_b64_tr_b16 per lane. That instruction, in each group of 16 lanes, hands lane i slot j the 16-bit value
//     at (address of lane 4j + i/4) + 2*(i%4): with lane i16 of a group addressing k row kb + i16/4 and rows
//     mb + 4*(i16%4) .. +3, lane i16 receives rows mb + i16 at k = kb .. kb+3, i.e. an MFMA operand (8 k values of one
//     row) from two reads.
constexpr int DK = 32;
// Stages in flight: 4 (3 ahead of the one being multiplied). Measured on 512 independent 128x256 tiles: 4 stages run
// K=768 tiles in 20.3 us against 23.9 with 5 (2.5 us less fixed cost, 0.44 instead of 0.48 us per stage), 3 stages in
// 27.9 us; GPT-162M step 9.56 -> 9.42 ms. A power of two also makes the stage index a mask.
constexpr int DNS = 4;

// s_waitcnt vmcnt(n) for a wave-uniform runtime n (other counters untouched); n above 30 waits for everything. The
// immediate must be a constant, so a (scalar) switch picks it; the wait is inline assembly with a memory clobber so
// that no LDS read of a dma16-staged block moves above it.
template <int N> __device__ __forceinline__ void wait_vm_c() { asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory"); }
__device__ __forceinline__ void wait_vm(int n) {
  switch (__builtin_amdgcn_readfirstlane(n)) {
#define KVM_WV(k) case k: wait_vm_c<k>(); break;
    KVM_WV(0) KVM_WV(1) KVM_WV(2) KVM_WV(3) KVM_WV(4) KVM_WV(5) KVM_WV(6) KVM_WV(7) KVM_WV(8) KVM_WV(9) KVM_WV(10) KVM_WV(11)
    KVM_WV(12) KVM_WV(13) KVM_WV(14) KVM_WV(15) KVM_WV(16) KVM_WV(17) KVM_WV(18) KVM_WV(19) KVM_WV(20) KVM_WV(21) KVM_WV(22)
    KVM_WV(23) KVM_WV(24) KVM_WV(25) KVM_WV(26) KVM_WV(27) KVM_WV(28) KVM_WV(29) KVM_WV(30)
#undef KVM_WV
    default: wait_vm_c<0>(); break;
  }
}
// lgkmcnt(0): this wave's LDS reads have returned (before a dma16 reuses the LDS they read).
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

typedef short s16x4_t __attribute__((ext_vector_type(4)));

template <int R, bool KC> struct DOp {
  static constexpr int BLK = R * DK * 2 / 1024;         // 1 KiB blocks per stage
  static constexpr int NL = BLK / KVM_WAVES;            // direct loads per thread per stage
  static constexpr int UPR = KC ? DK / 8 : R / 8;       // 16-byte units per LDS row
  static_assert(NL >= 1 && BLK % KVM_WAVES == 0, "tile shape");
  i32x4_t rs;
  int voff[NL];
  int sstep;
  unsigned m0w;                                         // LDS byte offset of this wave's first 1 KiB block (scalar)
  __device__ static __forceinline__ int kswz(int row) { return (row >> 2) & 3; }                       // k-contiguous
  __device__ static __forceinline__ int rswz(int k) { return R >= 128 ? 4 * (k & 3) : 4 * ((k >> 1) & 1); }  // row-contiguous
  __device__ __forceinline__ void init(const View& X, int r0) {
    m0w = (unsigned)__builtin_amdgcn_readfirstlane(wave()) * 1024u;
    if constexpr (KC) {
      rs = dma_rsrc((const void*)(X.h() + (long long)r0 * X.cols), ((long long)X.rows - r0) * X.cols * 2);
      sstep = DK * 2;
    } else {
      rs = dma_rsrc((const void*)(X.h() + r0), (long long)X.rows * X.cols * 2 - (long long)r0 * 2);
      sstep = DK * X.cols * 2;
    }
#pragma unroll
    for (int q = 0; q < NL; ++q) {
      const int u = 64 * (q * KVM_WAVES + wave()) + lane(), row = u / UPR, ph = u % UPR;
      if constexpr (KC) voff[q] = (row * X.cols + 8 * (ph ^ kswz(row))) * 2;
      else voff[q] = (row * X.cols + 8 * (ph ^ rswz(row))) * 2;
    }
  }
  // Direct loads of stage s (k0 = s*DK) into `lds` (this operand's region of one stage buffer); issue_one: load q only.
  // A stage at or past nst (a placeholder that keeps the count of loads in flight constant) loads from offset 2^31 and
  // up, past every descriptor's range: no memory access, the LDS bytes it writes are never read.
  // `lds` is the wave-uniform LDS byte address of the operand's region in the stage buffer: M0 is then computed with
  // scalar instructions only (a v_readfirstlane per load, with its hazard wait, measurably slows the MFMA stream).
  __device__ __forceinline__ void issue(unsigned lds, int s, int nst) const {
#pragma unroll
    for (int q = 0; q < NL; ++q) issue_one(lds, s, q, nst);
  }
  __device__ __forceinline__ void issue_one(unsigned lds, int s, int q, int nst) const {
    const unsigned m = lds + m0w + q * KVM_WAVES * 1024u;
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" :: "s"(m), "v"(voff[q]), "s"(rs),
                 "s"(s < nst ? s * sstep : (int)0x80000000) : "memory", "m0");
  }
  // MFMA operand for the 32 tile rows rb.. and k16 step kk: 8 bf16 of row rb + l%32 at k = 16kk + 8(l/32) ...
  __device__ __forceinline__ bf16x8 frag(const LDS uint16_t* lds, int rb, int kk) const {
    const int l = lane();
    if constexpr (KC) {
      const int r = rb + (l & 31), ch = kk * 2 + (l >> 5);
      return *(const LDS bf16x8*)(lds + r * DK + 8 * (ch ^ kswz(r)));
    } else {
      const int g = l >> 4, i = l & 15;
      const int k = kk * 16 + 8 * (g >> 1) + (i >> 2), m = rb + 16 * (g & 1) + 4 * (i & 3);
      const LDS uint16_t* p0 = lds + k * R + 8 * ((m >> 3) ^ rswz(k)) + (m & 7);
      const s16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS s16x4_t*)p0);
      const s16x4_t v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((LDS s16x4_t*)(p0 + 4 * R));
      typedef short s16x8_t __attribute__((ext_vector_type(8)));
      const s16x8_t v = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
      return (bf16x8)v;
    }
  }
};

template <int TM, int TN, bool AKC, bool BKC>
__device__ __forceinline__ void gemm_lds_b(const Ctx& c) {
  constexpr int WM = TM / 2, WN = TN / 2, BM = WM / 32, BN = WN / 32;
  constexpr int SA = TM * DK, SB = TN * DK, ST = SA + SB;    // elements per stage
  constexpr int NS = DNS * ST * 2 <= KVM_LDS_BYTES ? DNS : KVM_LDS_BYTES / (ST * 2);   // stages that fit in LDS
  static_assert(NS >= 3, "LDS");
  const GemmArgs g = gemm_args(c);
  const View& A = g.A; const View& B = g.B;
  const int m0 = g.m0, n0 = g.n0, K = g.K;
  LDS uint16_t* lds = (LDS uint16_t*)c.smem;
  const int wm0 = (wave() >> 1) * WM, wn0 = (wave() & 1) * WN;
  DOp<TM, AKC> da;
  DOp<TN, BKC> db;
  da.init(A, m0);
  db.init(B, n0);
  f32x16 acc[BM][BN];
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j) acc[i][j] = f32x16{};
  const int nst = K / DK;
  constexpr int NLS = DOp<TM, AKC>::NL + DOp<TN, BKC>::NL;  // direct loads per thread per stage
  // Every stage slot issues its direct loads, also past the last stage (placeholders, into a buffer no later stage
  // reads), so the number of loads in flight behind a stage is always the same and every wait is a constant vmcnt.
  __syncthreads();                                 // the previous task may still read this LDS
  const unsigned lb = (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)(uintptr_t)lds);   // LDS byte address
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) { da.issue(lb + p * ST * 2, p, nst); db.issue(lb + (p * ST + SA) * 2, p, nst); }
  // Software pipeline over stages, every instruction placed by hand (scheduling barriers around each MFMA): the compiler
  // otherwise sinks the fragment reads to just before the MFMAs that consume them (full LDS latency exposed at every
  // half) and issues the direct loads back to back (their issue stalls the wave's MFMA stream). Iteration s:
  //   half 0: the MFMAs of stage s's first k16 half, the fragment reads of its second half placed after its first
  //   MFMAs (as early as possible: they have the rest of the half to land);
  //   wait for stage s + 1 and barrier (every wave is then past stage s - 1, whose buffer the next loads reuse);
  //   half 1: the MFMAs of the second half; after its first ones the fragment reads of stage s + 1's first half, then
  //   the direct loads of stage s + NS - 1 (they have NS - 2 stages to land).
  // The last stage is peeled, so the loop body has no branch around LDS reads.
  constexpr int NF = BM + BN, NM = BM * BN;          // fragment reads / MFMAs per k16 half
  constexpr int NLA = DOp<TM, AKC>::NL;
  constexpr int PF = (NF + NM - 1) / NM, PX = (NF + NLS + NM - 1) / NM;   // reads / loads placed after each MFMA
  bf16x8 fa0[BM], fb0[BN], fa1[BM], fb1[BN];
  auto read_one = [&](const LDS uint16_t* st, int kk, int f, bf16x8 (&fa)[BM], bf16x8 (&fb)[BN]) {
    if (f < BM) fa[f] = da.frag(st, wm0 + f * 32, kk);
    else fb[f - BM] = db.frag(st + SA, wn0 + (f - BM) * 32, kk);
  };
  auto mfma_one = [&](int m, const bf16x8 (&fa)[BM], const bf16x8 (&fb)[BN]) {
    const int i = m / BN, j = m % BN;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[j], fa[i], acc[i][j], 0, 0, 0);
  };
  wait_vm_c<(NS - 2) * NLS>();                   // stage 0 has landed (NS - 2 stages were issued after it)
  __syncthreads();
#pragma unroll
  for (int f = 0; f < NF; ++f) read_one(lds, 0, f, fa0, fb0);
  for (int s = 0; s + 1 < nst; ++s) {
    const LDS uint16_t* la = lds + (s % NS) * ST;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      mfma_one(m, fa0, fb0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int f = m * PF; f < (m + 1) * PF && f < NF; ++f) read_one(la, 1, f, fa1, fb1);
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vm_c<(NS - 3) * NLS>();                 // this thread's loads of stage s + 1 have landed
    asm volatile("s_barrier" ::: "memory");        // ... everyone's
    const int sn = s + NS - 1;
    const unsigned nb = lb + ((s + NS - 1) % NS) * ST * 2;
    const LDS uint16_t* ln = lds + ((s + 1) % NS) * ST;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      mfma_one(m, fa1, fb1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int x = m * PX; x < (m + 1) * PX && x < NF + NLS; ++x) {
        if (x < NF) read_one(ln, 0, x, fa0, fb0);
        else if (x - NF < NLA) da.issue_one(nb, sn, x - NF, nst);
        else db.issue_one(nb + SA * 2, sn, x - NF - NLA, nst);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  {
    const LDS uint16_t* la = lds + ((nst - 1) % NS) * ST;
#pragma unroll
    for (int f = 0; f < NF; ++f) read_one(la, 1, f, fa1, fb1);
#pragma unroll
    for (int m = 0; m < NM; ++m) mfma_one(m, fa0, fb0);
#pragma unroll
    for (int m = 0; m < NM; ++m) mfma_one(m, fa1, fb1);
  }
  wait_vm_c<0>();                                  // the placeholder loads have written their LDS bytes
  gemm_store<TM, TN>(c, acc, g);
}
template <int TM, int TN, bool AKC, bool BKC>
__device__ __noinline__ void gemm_lds(const Ctx& c) { gemm_lds_b<TM, TN, AKC, BKC>(c); }

// Whether an operand slab sequence can use unconditional vector loads: bf16 storage, rows of whole 16-byte vectors,
// the tile's rows inside the matrix and K a whole number of slabs.
__device__ __forceinline__ bool gemm_fast_operand(const View& X, bool kc, int r0, int R, int rows, int K) {
  if (X.dtype != 2 || (X.cols & 7) || (K % DK) || r0 + R > rows) return false;
  if (kc) return (long long)R * X.cols * 2 + (long long)K * 2 < 0x7fffffffll;
  return (r0 & 7) == 0 && (long long)K * X.cols * 2 < 0x7fffffffll;    // buffer offsets are 32-bit
}

template <int TM, int TN> __device__ __forceinline__ void mfma_tile(const Ctx& c) {
  static_assert(2 * (TM + TN) * GS * 2 <= KVM_LDS_BYTES, "LDS");
  const GemmArgs g = gemm_args(c);
  const bool akc = !(g.fl & 1), bkc = (g.fl & 2) != 0;
  const bool fast = gemm_fast_operand(g.A, akc, g.m0, TM, g.M, g.K) && gemm_fast_operand(g.B, bkc, g.n0, TN, g.N, g.K);
  // One instantiation per operand orientation, so the slab prefetch is straight-line code (a runtime branch between
  // orientations makes the compiler wait for the loads of one operand before issuing the other's).
  if (fast) {
    if (akc) { if (bkc) gemm_lds<TM, TN, true, true>(c); else gemm_lds<TM, TN, true, false>(c); }
    else { if (bkc) gemm_lds<TM, TN, false, true>(c); else gemm_lds<TM, TN, false, false>(c); }
  } else {
    if (akc) { if (bkc) gemm_loop<TM, TN, false, true, true>(c); else gemm_loop<TM, TN, false, true, false>(c); }
    else { if (bkc) gemm_loop<TM, TN, false, false, true>(c); else gemm_loop<TM, TN, false, false, false>(c); }
  }
}

// ---------------------------------------------------------------------------------------------- fp32 MFMA engine
// matmul_tile (op 34) on the matrix cores: v_mfma_f32_32x32x2_f32, exact fp32 products with fp32 accumulation (CDNA4
// has no TF32; the reference's TF32 flags run as plain fp32). Four waves in a 2 x 2 grid, each owning (TM/2) x (TN/2)
// as 32 x 32 blocks. K advances in slabs of FKS = 16: both operands sit in LDS as [row][k] f32 (64-byte rows, 16-byte
// k-chunks XOR-swizzled by (row >> 2) & 3), double-buffered; the next slab is loaded into registers while the current
// one is multiplied. One ds_read_b128 per operand block gives a lane four k values: lanes 0-31 hold k 8q..8q+3 and
// lanes 32-63 k 8q+4..8q+7 of their row, and the four MFMAs of that read pair them up (which k each MFMA sums is a
// free choice as long as A and B agree). B is the MFMA's first source, so the accumulators hold D^T exactly as the
// bf16 engine's, and the tile leaves through the same LDS-staged epilogue (gemm_store).
constexpr int FKS = 16;
__device__ __forceinline__ int fsw(int row, int ch) { return row * FKS + 4 * (ch ^ ((row >> 2) & 3)); }

template <int R> struct FTile {
  static constexpr int NV = R * FKS / 4 / KVM_THREADS;   // float4 per thread per slab
  static_assert(NV >= 1, "tile shape");
  f32x4n v[NV];
  // Slab k0 of rows r0..r0+R of X: kc = element (r, k) at X[r*cols + k], else at X[k*cols + r]. Rows / k past the
  // matrix read as 0. vec: f32 storage with cols % 4 == 0 (every 4-aligned element index is a 16-byte load).
  __device__ __forceinline__ void fetch(const View& X, bool kc, bool vec, int r0, int rows, int k0, int K) {
#pragma unroll
    for (int q = 0; q < NV; ++q) {
      const int idx = tid() + q * KVM_THREADS;
      int r, k;
      if (kc) { r = r0 + (idx >> 2); k = k0 + 4 * (idx & 3); }       // 4 k of one row
      else { r = r0 + 4 * (idx % (R / 4)); k = k0 + idx / (R / 4); }   // 4 rows of one k
      const long long o = kc ? (long long)r * X.cols + k : (long long)k * X.cols + r;
      const bool whole = kc ? (r < rows && k + 4 <= K) : (k < K && r + 4 <= rows);
      if (vec && whole) v[q] = *(const GLOBAL f32x4n*)(X.f() + o);
      else {
        f32x4n t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool in = kc ? (r < rows && k + i < K) : (k < K && r + i < rows);
          if (in) t[i] = X.ld(o + i);
        }
        v[q] = t;
      }
    }
  }
  __device__ __forceinline__ void store(LDS float* lds, bool kc) const {
#pragma unroll
    for (int q = 0; q < NV; ++q) {
      const int idx = tid() + q * KVM_THREADS;
      if (kc) *(LDS f32x4n*)(lds + fsw(idx >> 2, idx & 3)) = v[q];
      else {
        const int r = 4 * (idx % (R / 4)), k = idx / (R / 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) lds[fsw(r + i, k >> 2) + (k & 3)] = v[q][i];
      }
    }
  }
};

template <int TM, int TN> __device__ __noinline__ void gemm_f32(const Ctx& c) {
  constexpr int WM = TM / 2, WN = TN / 2, BM = WM / 32, BN = WN / 32, ST = (TM + TN) * FKS;
  // Slabs move in batches of SB (all of a batch's loads in flight together, double-buffered in LDS): one global-load
  // latency per batch instead of per slab, which is what a small tile's short K loop is bound by.
  constexpr int NVA = FTile<TM>::NV, NVB = FTile<TN>::NV;
  constexpr int SB_REG = 16 / (NVA + NVB), SB_LDS = KVM_LDS_BYTES / 2 / (ST * 4);
  constexpr int SB = SB_REG < SB_LDS ? (SB_REG < 8 ? SB_REG : 8) : (SB_LDS < 8 ? SB_LDS : 8);
  static_assert(SB >= 1 && 2 * SB * ST * 4 <= KVM_LDS_BYTES && TM * TN * 4 <= KVM_LDS_BYTES, "LDS");
  const GemmArgs g = gemm_args(c);
  const View& A = g.A; const View& B = g.B;
  const bool akc = !(g.fl & 1), bkc = (g.fl & 2) != 0;
  const bool avec = A.dtype == 0 && (A.cols & 3) == 0, bvec = B.dtype == 0 && (B.cols & 3) == 0;
  const int wm0 = (wave() >> 1) * WM, wn0 = (wave() & 1) * WN, l = lane();
  LDS float* lds = (LDS float*)c.smem;
  f32x16 acc[BM][BN];
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j) acc[i][j] = f32x16{};
  FTile<TM> fa[SB];
  FTile<TN> fb[SB];
  auto fetch = [&](int bt) {
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      fa[u].fetch(A, akc, avec, g.m0, g.M, (bt * SB + u) * FKS, g.K);
      fb[u].fetch(B, bkc, bvec, g.n0, g.N, (bt * SB + u) * FKS, g.K);
    }
  };
  auto store = [&](int bt) {
    LDS float* base = lds + (bt & 1) * SB * ST;
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      fa[u].store(base + u * ST, akc);
      fb[u].store(base + u * ST + TM * FKS, bkc);
    }
  };
  const int nslab = (g.K + FKS - 1) / FKS, nbat = (nslab + SB - 1) / SB;
  fetch(0);
  __syncthreads();                         // the previous task may still read this LDS
  store(0);
  __syncthreads();
  for (int bt = 0; bt < nbat; ++bt) {
    const bool more = bt + 1 < nbat;
    if (more) fetch(bt + 1);
    const int ns = min(SB, nslab - bt * SB);
    for (int u = 0; u < ns; ++u) {
      const LDS float* la = lds + ((bt & 1) * SB + u) * ST;
      const LDS float* lb = la + TM * FKS;
#pragma unroll
      for (int q = 0; q < FKS / 8; ++q) {
        const int ch = 2 * q + (l >> 5);
        f32x4n av[BM], bv[BN];
#pragma unroll
        for (int i = 0; i < BM; ++i) av[i] = *(const LDS f32x4n*)(la + fsw(wm0 + i * 32 + (l & 31), ch));
#pragma unroll
        for (int j = 0; j < BN; ++j) bv[j] = *(const LDS f32x4n*)(lb + fsw(wn0 + j * 32 + (l & 31), ch));
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int i = 0; i < BM; ++i)
#pragma unroll
            for (int j = 0; j < BN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[j][t], av[i][t], acc[i][j], 0, 0, 0);
      }
    }
    if (more) store(bt + 1);
    __syncthreads();
  }
  gemm_store<TM, TN>(c, acc, g);
}

__device__ __noinline__ void op_matmul_tile_bf16(const Ctx& c) {
  const int fl = c.i(11);
  if (fl & 64) mfma_tile<256, 128>(c);
  else if (fl & 32) mfma_tile<128, 128>(c);
  else mfma_tile<64, 64>(c);
}
__device__ __noinline__ void op_matmul_mma_bf16(const Ctx& c) { mfma_tile<128, 256>(c); }
// Whole-tile shapes of a TM x TN tile with the direct-to-LDS main loop inlined into the caller (the persistent kernel):
// false when the tile needs the general path.
template <int TM, int TN> __device__ __forceinline__ bool gemm_tile_inline(const Ctx& c) {
  const GemmArgs g = gemm_args(c);
  const bool akc = !(g.fl & 1), bkc = (g.fl & 2) != 0;
  if (!gemm_fast_operand(g.A, akc, g.m0, TM, g.M, g.K) || !gemm_fast_operand(g.B, bkc, g.n0, TN, g.N, g.K)) return false;
  if (akc) { if (bkc) gemm_lds_b<TM, TN, true, true>(c); else gemm_lds_b<TM, TN, true, false>(c); }
  else { if (bkc) gemm_lds_b<TM, TN, false, true>(c); else gemm_lds_b<TM, TN, false, false>(c); }
  return true;
}
// Op 304: the 256x256 tile. Shapes outside the direct-to-LDS path (partial tiles, odd K, f32 operands) run as two
// 128x256 tiles, rows m0 and m0 + 128 (the second by advancing m0 in the task's LDS copy of its arguments).
__device__ __forceinline__ void tile_256(const Ctx& c) {
  const GemmArgs g = gemm_args(c);
  const bool akc = !(g.fl & 1), bkc = (g.fl & 2) != 0;
  if (gemm_fast_operand(g.A, akc, g.m0, 256, g.M, g.K) && gemm_fast_operand(g.B, bkc, g.n0, 256, g.N, g.K)) {
    if (akc) { if (bkc) gemm_lds<256, 256, true, true>(c); else gemm_lds<256, 256, true, false>(c); }
    else { if (bkc) gemm_lds<256, 256, false, true>(c); else gemm_lds<256, 256, false, false>(c); }
    return;
  }
  mfma_tile<128, 256>(c);
  if (g.m0 + 128 < g.M) {
    __syncthreads();                                     // every thread has read the arguments
    if (tid() == 0) ((LDS int32_t*)c.a)[6] = g.m0 + 128;
    __syncthreads();
    mfma_tile<128, 256>(c);
  }
}
__device__ __noinline__ void op_matmul_mma_bf16_256(const Ctx& c) { tile_256(c); }
// Op 302: op 122 over the K range [k0, k0 + K), written at output rows om0 + m; with flag 64 op 304's 256x256 tile
// (a quarter fewer operand bytes per output than 128x256). The task's buffer views (LDS copies made by the
// dispatcher) are narrowed in place to that K range and output row offset; the tile then runs unchanged.
__device__ __noinline__ void op_matmul_mma_bf16_kr(const Ctx& c) {
  if (tid() == 0) {
    LDS View* v = (LDS View*)c.views;
    const int fl = c.i(11), k0 = c.i(13), om0 = c.i(14);
    auto shift = [](LDS View& x, long long rows_off, long long elems) {
      const int es = x.dtype == 2 ? 2 : 4;
      x.p = (char*)x.p + elems * es;
      x.rows -= (int)rows_off;
    };
    if (fl & 1) shift(v[0], k0, (long long)k0 * v[0].cols); else shift(v[0], 0, k0);   // A [K, M] rows / [M, K] columns
    if (fl & 2) shift(v[1], 0, k0); else shift(v[1], k0, (long long)k0 * v[1].cols);   // B [N, K] columns / [K, N] rows
    shift(v[2], om0, (long long)om0 * v[2].cols);
  }
  __syncthreads();
  if (c.i(11) & 64) tile_256(c);
  else mfma_tile<128, 256>(c);
}

// The fp32 engine's pipelined form for whole tiles of f32 operands (16-byte aligned rows, K a multiple of 16): every
// slab goes from HBM straight into LDS (buffer_load ... lds), NS stages deep, so no slab passes through registers and
// the loads of NS - 1 slabs are always in flight behind the one being multiplied. A k-contiguous operand sits in LDS as
// [row][16 k] (the register-staged form's swizzled layout); a row-contiguous one as [16 k][R rows], read one k per
// ds_read_b32 (32 lanes: 128 contiguous bytes). Every stage slot issues its loads, also past the last slab (an offset
// past every descriptor's range: no memory access), so every wait is a constant vmcnt.
template <int R, bool KC> struct FOp {
  static constexpr int NL = R * FKS * 4 / 1024 / KVM_WAVES;   // direct loads per thread per slab
  static_assert(NL >= 1, "tile shape");
  i32x4_t rs;
  int voff[NL];
  int sstep;
  __device__ __forceinline__ void init(const View& X, int r0) {
    if constexpr (KC) {
      rs = dma_rsrc((const void*)(X.f() + (long long)r0 * X.cols), ((long long)X.rows - r0) * X.cols * 4);
      sstep = FKS * 4;
    } else {
      rs = dma_rsrc((const void*)(X.f() + r0), (long long)X.rows * X.cols * 4 - (long long)r0 * 4);
      sstep = FKS * X.cols * 4;
    }
#pragma unroll
    for (int q = 0; q < NL; ++q) {
      const int u = 64 * (q * KVM_WAVES + wave()) + lane();
      if constexpr (KC) { const int row = u >> 2, ch = (u & 3) ^ ((row >> 2) & 3); voff[q] = (row * X.cols + 4 * ch) * 4; }
      else { const int k = u / (R / 4), ph = u % (R / 4); voff[q] = (k * X.cols + 4 * ph) * 4; }
    }
  }
  __device__ __forceinline__ void issue(LDS float* lds, int s, int nst) const {
#pragma unroll
    for (int q = 0; q < NL; ++q) dma16(rs, voff[q], s < nst ? s * sstep : (int)0x80000000, lds + (q * KVM_WAVES + wave()) * 256);
  }
  // four k values (8q + 4 (l / 32) + t) of row rb + l % 32
  __device__ __forceinline__ f32x4n frag(const LDS float* lds, int rb, int q) const {
    const int l = lane(), r = rb + (l & 31), ch = 2 * q + (l >> 5);
    if constexpr (KC) return *(const LDS f32x4n*)(lds + fsw(r, ch));
    else return f32x4n{lds[(4 * ch) * R + r], lds[(4 * ch + 1) * R + r], lds[(4 * ch + 2) * R + r], lds[(4 * ch + 3) * R + r]};
  }
};

template <int TM, int TN, bool AKC, bool BKC> __device__ __forceinline__ void gemm_f32_lds_b(const Ctx& c) {
  constexpr int WM = TM / 2, WN = TN / 2, BM = WM / 32, BN = WN / 32, SA = TM * FKS, ST = (TM + TN) * FKS;
  constexpr int NS = ST * 4 * 6 <= KVM_LDS_BYTES ? 6 : KVM_LDS_BYTES / (ST * 4);
  static_assert(NS >= 3, "LDS");
  const GemmArgs g = gemm_args(c);
  const int wm0 = (wave() >> 1) * WM, wn0 = (wave() & 1) * WN;
  FOp<TM, AKC> da;
  FOp<TN, BKC> db;
  da.init(g.A, g.m0);
  db.init(g.B, g.n0);
  LDS float* lds = (LDS float*)c.smem;
  f32x16 acc[BM][BN];
#pragma unroll
  for (int i = 0; i < BM; ++i)
#pragma unroll
    for (int j = 0; j < BN; ++j) acc[i][j] = f32x16{};
  const int nst = g.K / FKS;
  constexpr int NLS = FOp<TM, AKC>::NL + FOp<TN, BKC>::NL;
  __syncthreads();                                 // the previous task may still read this LDS
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) { da.issue(lds + p * ST, p, nst); db.issue(lds + p * ST + SA, p, nst); }
  for (int s = 0; s < nst; ++s) {
    wait_vm_c<(NS - 2) * NLS>();                   // this thread's loads of slab s have landed
    __syncthreads();                               // ... everyone's, and every wave is past slab s - 1
    { const int sn = s + NS - 1; LDS float* nb = lds + (sn % NS) * ST; da.issue(nb, sn, nst); db.issue(nb + SA, sn, nst); }
    const LDS float* la = lds + (s % NS) * ST;
    const LDS float* lb = la + SA;
#pragma unroll
    for (int q = 0; q < FKS / 8; ++q) {
      f32x4n av[BM], bv[BN];
#pragma unroll
      for (int i = 0; i < BM; ++i) av[i] = da.frag(la, wm0 + i * 32, q);
#pragma unroll
      for (int j = 0; j < BN; ++j) bv[j] = db.frag(lb, wn0 + j * 32, q);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < BM; ++i)
#pragma unroll
          for (int j = 0; j < BN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(bv[j][t], av[i][t], acc[i][j], 0, 0, 0);
    }
  }
  wait_vm_c<0>();                                  // the placeholder loads have written their LDS bytes
  gemm_store<TM, TN>(c, acc, g);
}
template <int TM, int TN, bool AKC, bool BKC> __device__ __noinline__ void gemm_f32_lds(const Ctx& c) { gemm_f32_lds_b<TM, TN, AKC, BKC>(c); }

// Whether an f32 operand takes the pipelined form: f32 storage, 16-byte rows, the tile's rows inside the matrix, K a
// whole number of slabs, offsets within 32 bits.
__device__ __forceinline__ bool gemm_f32_fast_operand(const View& X, bool kc, int r0, int R, int rows, int K) {
  if (X.dtype != 0 || (X.cols & 3) || (K % FKS) || r0 + R > rows) return false;
  if (kc) return (long long)R * X.cols * 4 + (long long)K * 4 < 0x7fffffffll;
  return (r0 & 3) == 0 && (long long)K * X.cols * 4 < 0x7fffffffll;
}
template <int TM, int TN> __device__ __forceinline__ void f32_tile(const Ctx& c) {
  const GemmArgs g = gemm_args(c);
  const bool akc = !(g.fl & 1), bkc = (g.fl & 2) != 0;
  if (gemm_f32_fast_operand(g.A, akc, g.m0, TM, g.M, g.K) && gemm_f32_fast_operand(g.B, bkc, g.n0, TN, g.N, g.K)) {
    if (akc) { if (bkc) gemm_f32_lds<TM, TN, true, true>(c); else gemm_f32_lds<TM, TN, true, false>(c); }
    else { if (bkc) gemm_f32_lds<TM, TN, false, true>(c); else gemm_f32_lds<TM, TN, false, false>(c); }
    return;
  }
  gemm_f32<TM, TN>(c);
}

// The whole-tile fp32 form inlined into the caller (the persistent kernel); false when the tile needs the general path.
template <int TM, int TN> __device__ __forceinline__ bool f32_tile_inline(const Ctx& c) {
  const GemmArgs g = gemm_args(c);
  const bool akc = !(g.fl & 1), bkc = (g.fl & 2) != 0;
  if (!gemm_f32_fast_operand(g.A, akc, g.m0, TM, g.M, g.K) || !gemm_f32_fast_operand(g.B, bkc, g.n0, TN, g.N, g.K)) return false;
  if (akc) { if (bkc) gemm_f32_lds_b<TM, TN, true, true>(c); else gemm_f32_lds_b<TM, TN, true, false>(c); }
  else { if (bkc) gemm_f32_lds_b<TM, TN, false, true>(c); else gemm_f32_lds_b<TM, TN, false, false>(c); }
  return true;
}
// Op 34 on the fp32 MFMA engine: 64x64 tiles by default, 128x128 with flag 32, 256x128 with flag 64.
__device__ __noinline__ void op_matmul_tile(const Ctx& c) {
  const int fl = c.i(11);
#ifndef KVM_F32_REGSTAGE
  if (fl & 64) f32_tile<256, 128>(c);
  else if (fl & 32) f32_tile<128, 128>(c);
  else f32_tile<64, 64>(c);
#else
  if (fl & 64) gemm_f32<256, 128>(c);
  else if (fl & 32) gemm_f32<128, 128>(c);
  else gemm_f32<64, 64>(c);
#endif
}

}  // namespace kvm
