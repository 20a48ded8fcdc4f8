// Shared device/host definitions of the MI355X task-graph executor: error codes, device state, buffer views,
// bf16 conversion and the memory-ordering primitives the scheduler is built on.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/mvm_task_abi.h"
#include "../../include/kvm_exec.h"

typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));
// Address-space qualifiers: buffer data is global memory (addrspace 1), operator scratch is LDS (addrspace 3). Typing
// pointers this way makes the compiler emit global_/ds_ instructions instead of flat ones, so LDS traffic does not
// wait on outstanding HBM loads.
#define GLOBAL __attribute__((address_space(1)))
typedef float f32x4n __attribute__((ext_vector_type(4)));   // native 128-bit float vector (HIP's float4 is a class)
#define LDS __attribute__((address_space(3)))

#define KVM_THREADS 256          // every operator runs on one workgroup of 256 threads = four wave64s
#define KVM_WAVES (KVM_THREADS / 64)
#define KVM_MAX_ARGS 24
#define KVM_MAX_PRIVATE_BYTES 2048   // private segment per lane above which kvm_create refuses the kernel build
#define KVM_LDS_BYTES (128 * 1024)   // LDS one task may use (gfx950 has 160 KiB per CU; the executor keeps the rest)

// Device error codes. 0-20 keep the reference's numbering (reference: include/mvm_exec.cuh:148-164); operator
// argument errors are 1000+k with the k of the operator registries' conventions.
enum KvmErr {
  KVM_OK = 0, KVM_ERR_BAD_OP = 1, KVM_ERR_BAD_ARITY = 2, KVM_ERR_BAD_BUF_INDEX = 3, KVM_ERR_BAD_BUF = 4,
  KVM_ERR_BOUNDS = 5, KVM_ERR_BAD_VAR = 6, KVM_ERR_VERSION_GAP = 7, KVM_ERR_WAIT_VIOLATION = 8,
  KVM_ERR_DOUBLE_EXEC = 9, KVM_ERR_BAD_TASK = 11, KVM_ERR_TIMEOUT = 15, KVM_ERR_QUEUE_OVERFLOW = 16,
  KVM_ERR_BAD_CONFIG = 17,
  KVM_ERR_OP_BUF = 1001, KVM_ERR_OP_DTYPE = 1002, KVM_ERR_OP_RANGE = 1003, KVM_ERR_OP_SHAPE = 1004,
  KVM_ERR_OP_TOKEN = 1005, KVM_ERR_OP_KVLEN = 1006,
};

// Successor edges as uploaded to the device: the task index plus flag bits. KVM_EDGE_NOWAIT: the successor has no
// version wait (the predecessor whose decrement reaches zero enqueues it without reading its descriptor);
// KVM_EDGE_DIRECT: also exactly one predecessor (released by that predecessor without a counter).
#define KVM_EDGE_DIRECT (1 << 30)
#define KVM_EDGE_NOWAIT (1 << 29)
#define KVM_SF_PUB 1             // static path, per task: another worker waits for this task's program position
#define KVM_SF_PRE 2             // static path, per task: input-independent loads may be issued before the wait
#define KVM_EDGE_INDEX (KVM_EDGE_NOWAIT - 1)

struct KvmCounters {
  int err_code, err_slot, err_a, err_b;
  int pad[4];
};

// One ready queue. Head (consumer tickets) and tail (producer slots) sit on separate 128-byte lines.
#define KVM_MAX_QUEUES 8
#define KVM_PSTRIDE_MAX 16      // ints: 64 bytes between two static-path workers' progress words when padded
#define KVM_OPMASK_IDS 1024
struct KvmQueue {
  unsigned head; int pad0[31];
  int tail; int pad1[31];
};

// Streaming admission (stream mode, reference: the admitter and its windows, mvm_exec.cuh:820-1058). The persistent
// kernel runs while the host submits bundles: each bundle occupies one of `wcap` window slots (task slots
// [w * wtasks, (w + 1) * wtasks), successor slots [w * wedges, ...)). The host stages a window in pinned host memory
// (KvmHostWin + the arrays after it) and raises `submitted`; an idle worker takes the admission lock, copies the
// window into device memory, adds its tasks to the per-queue totals and releases its roots. The worker that finishes
// a window's last task writes its completion mark to host memory, after which the host may reuse the slot.
struct KvmHostCtl {                      // pinned, written by the host (submitted, closed) and the device (done_mark)
  long long submitted;                   // windows staged so far (window seq k lives in slot k % wcap)
  int closed;                            // no window follows the last one submitted
  int pad[13];
  long long done_mark[1];                // [wcap] seq + 1 of the last window completed in each slot (flexible)
};
struct KvmHostWin { int seq, ntasks, nedges, nroots; int qn[8]; int pad[4]; };   // per slot; qn: tasks per ready queue
struct KvmAdm {                          // device admission state
  int lock, next, fin, admitted;         // next: seq of the next window to admit; fin: closed and everything admitted
  int total[64];                         // tasks admitted per ready queue (tickets below it will be served); with
                                         // scheduler classes per (queue group, class) ring
  int pad[24];
};

// Everything the persistent kernel reads. One task graph per launch (the submitted bundles concatenated), or, in
// stream mode, the window slots.
// Scheduler classes (reference: MvmClsDev / MvmSchedDev, include/mvm_sched.h:80-111). A task's class is its
// workload_id. Per class: a parameter line written by the host at upload, a hot line (running workers, weighted
// virtual time charged ahead of time, the running-time estimate) and a statistics line; times in wall_clock64 ticks.
struct alignas(128) KvmClsDev {
  int weight, min_cta, max_cta, urgent_ticks, vt_mul, blk_lo, blk_hi, has_dl;   // vt_mul = 2^20 / weight
  int bw_cta, has_bw;              // cap on running bandwidth-bound tasks; the class has such tasks
  int opaff;                       // op affinity: a released task prefers the worker that last ran its operator
  int pad0[21];
  int running, bw_running;         // running tasks; of those, bandwidth-bound ones
  unsigned long long vtime;        // sum of (ticks run) * vt_mul: the class with the least is served first
  unsigned est;                    // running-time estimate of the class's tasks (moving average, ticks)
  int pad1[27];
  unsigned long long tasks, busy, resv_starts, urgent_starts, missed, boost_starts;
  int max_running;
  int pad2[19];
};
static_assert(sizeof(KvmClsDev) == 384, "class lines");
// (KVM_SCHED_F_* policy switches: include/kvm_exec.h)
#define KVM_OP_SLOTS 512          // operator ids below this have an op-affinity slot
#define KVM_HOW_BW 0x100          // pop_cls / cls_done only: the claimed task counts as bandwidth-bound (never traced)
struct KvmSchedDev {
  unsigned long long t0;           // launch time: task deadlines count from here
  int flags, bw_limit;             // KVM_SCHED_F_*; the global cap on running bandwidth-bound tasks (ARBITER)
  int boost;                       // classes boosted by inheritance (bit c), recomputed on every park / unpark
  int bw_total;                    // running bandwidth-bound tasks of all classes
  unsigned long long aff_ticks;    // task affinity window (0 off): a ready task is offered only to its preferred worker
  int pad[24];
  KvmClsDev cls[KVM_MAX_CLASSES];
};

struct KvmRec;
struct KvmDevState {
  const MvmTaskDesc* tasks;   // [ntasks]
  const KvmRec* recs;         // [ntasks] dispatch records (descriptor, argument words, buffer views)
  const int32_t* succ;        // [nedges] global task indices (| KVM_EDGE_NOWAIT, KVM_EDGE_DIRECT)
  int* indeg;                 // [ntasks] remaining predecessors
  int* ready;                 // ready cells: queue qi's i-th released task at ready[qoff[qi] + i], -1 until then
  KvmQueue* queues;           // [nq * nb]
  const int* qcount;          // [nq * nb] tasks that go through queue qi
  const int* qoff;            // [nq * nb] first cell of queue qi (FIFO mode: qi * qcap)
  // Priority mode (nb > 1 priority buckets, or aging): task t goes to queue tq[t] = (t % nq) * nb + bucket, bucket 0
  // holding the highest priority present in the graph. FIFO mode (nb == 1): queue t % nq, no table.
  const int* tq;              // [ntasks] or null
  const int* bucket_prio;     // [nb] priority of each bucket
  unsigned long long* ready_ts;   // [ntasks] release time (wall_clock64) when aging, else null
  int* done_blk;              // [grid] tasks finished per worker (summed by the host; no shared counter per task)
  int* state;                 // [ntasks] 0 not released, 1 parked on a version, 2 enqueued
  int* park_next;             // [ntasks] park list links
  int* version;               // [nvars]
  int* park_head;             // [nvars] park list heads, -1 empty
  KvmCounters* cnt;
  KvmTrace* trace;            // [ntasks] or null
  // Static path (kvm_static_kernel): worker w runs tasks sprog[sprog_off[w] .. sprog_off[w + 1]); task t first waits for
  // sprogress[sw[2k]] >= sw[2k + 1] for k in [swait_off[t], swait_off[t + 1]); after it, a task with KVM_SF_PUB in
  // sflag[t] stores its program position + 1 into sprogress[w]. KVM_SF_PRE: the task's input-independent loads may be
  // issued before the wait.
  const int* sprog_off;
  const int* sprog;
  const int* swait_off;
  const int* sw;
  const int* sflag;
  int* sprogress;            // [grid * KVM_PSTRIDE_MAX]: worker w's position at sprogress[w * pstride]
  int pstride;               // ints between two workers' positions: KVM_PSTRIDE_MAX (64 bytes each) or 1 (packed)
  int svariant;              // the static kernel's inlined operator set (kvm_static_kernel<V>)
  // Stream mode (stream != 0): FIFO queues of reused cells, ready64[q * qcap + (ticket & (qcap - 1))] = (round << 32) |
  // slot with round = ticket / qcap + 1 (0: empty); qcap a power of two above the slots' capacity.
  unsigned long long* ready64;
  KvmAdm* adm;
  KvmHostCtl* hctl;          // device address of the pinned control block
  int* hver;                 // device address of the pinned mirror of the version variables (stream mode), or null
  const char* hwin;          // device address of the pinned staging: KvmHostWin[wcap], then per slot recs, tasks, succ, roots
  int* win_left;             // [wcap] tasks of the slot's window not yet finished
  int* win_seq;              // [wcap] seq of the window in the slot
  unsigned long long* win_t0;   // [wcap] admission time of the slot's window (stream-mode deadlines count from it)
  int stream, wcap, wtasks, wedges;
  // Scheduler classes (ncls > 0): task t of class c = tasks[t].workload_id goes to queue ((t % nq) * ncls + c) * nb +
  // bucket; a worker's lane c * nb + b watches class c's bucket b. In stream mode nb = 1 and queue (t % nq) * ncls + c
  // is a ring of ready64 cells like the FIFO queues.
  KvmSchedDev* sched;
  int ncls;
  // Priority inheritance (classes on): pv[v * KVM_MAX_CLASSES + c] = tasks of class c parked on variable v; pubcls[v] =
  // classes with a task that publishes v; publist[0 .. npub) = the variables some task publishes. tbw[t] = 1: task t is
  // bandwidth-bound (counts against bw_cta / bw_limit).
  int* pv;
  int* pubcls;               // stream mode: or-ed in at admission (publist then lists every variable)
  const int* publist;
  unsigned char* tbw;        // stream mode: written at admission, per slot
  // Task affinity (classes on, an affinity window set): aff[t] = (ready time << 12) | (preferred worker + 1), written
  // before the task's cell is published; op_blk[op] = the worker that last finished a task of operator op (-1 none).
  unsigned long long* aff;
  int* op_blk;
  int npub;
  int ntasks, nvars, trace_on, nq, qcap, grid, nb, ncells;
  unsigned long long timeout_ticks;   // stall timeout in wall_clock64 ticks (100 MHz)
  unsigned long long aging_ticks;     // wall_clock64 ticks of waiting worth one priority level (0: strict priority)
};

// ---------------------------------------------------------------------------------------------- atomics
// Agent-scope release/acquire through the HIP atomic builtins: on gfx950 the compiler emits the L2 write-back /
// invalidate each XCD needs, so a release by a workgroup on one XCD is seen by an acquire on another.
__device__ __forceinline__ int ld_relaxed(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ unsigned ld_relaxed(const unsigned* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ int ld_acquire(const int* p) { return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_release(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_relaxed(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ int add_acqrel(int* p, int v) { return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ int add_relaxed(int* p, int v) { return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ unsigned add_relaxed(unsigned* p, unsigned v) { return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ bool cas_acqrel(int* p, int expect, int want) {
  return __hip_atomic_compare_exchange_strong(p, &expect, want, __ATOMIC_ACQ_REL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int xchg_acqrel(int* p, int v) { return __hip_atomic_exchange(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void fence_seqcst() { __atomic_thread_fence(__ATOMIC_SEQ_CST); }
__device__ __forceinline__ void fence_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }
__device__ __forceinline__ void fence_release() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); }


// ---------------------------------------------------------------------------------------------- bf16
__device__ __host__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
// float -> bf16, round to nearest even; NaN stays NaN (quiet bit set), inf stays inf.
// Round to nearest even, in hardware (v_cvt_pk_bf16_f32): one instruction instead of the integer rounding sequence.
// Finite values and infinities round exactly as (u + 0x7fff + ((u >> 16) & 1)) >> 16; NaNs stay NaN.
__device__ __forceinline__ uint16_t f2bf(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
__device__ __forceinline__ float round_bf(float x) { return bf2f(f2bf(x)); }

// Write-through global stores: the agent-scope form of a store (sc1, the encoding of an agent-scope relaxed atomic
// store), which is agent-visible once it completes, with no L2 write-back. A task of an operator whose every global
// store has this form is completed by waiting for the stores (vmcnt) instead of a release fence, whose L2 write-back
// costs microseconds per task on a chip with one L2 per XCD. Consumers still acquire (L1 / L2 invalidate) as usual.
__device__ __forceinline__ void stwt16(GLOBAL uint16_t* p, uint16_t v) { __hip_atomic_store((uint16_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void stwt32(GLOBAL float* p, float v) { __hip_atomic_store((float*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void stwt32i(GLOBAL int* p, int v) { __hip_atomic_store((int*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void stwt64(GLOBAL void* p, uint64_t v) { __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// 16 bytes as two 8-byte stores: every store stays visible to the compiler, whose wait counts must know about stores
// (on gfx950 loads and stores share vmcnt and complete out of order with respect to each other).
typedef uint64_t u64x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void stwt_f4(GLOBAL float* p, f32x4n v) {
  const u64x2_t u = __builtin_bit_cast(u64x2_t, v);
  stwt64(p, u.x); stwt64(p + 2, u.y);
}
// Two floats rounded to bf16 (round to nearest even, as f2bf) and packed, a in the low half: one v_cvt_pk_bf16_f32.
typedef float f32x2v_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v_t{a, b}, bf16x2v_t));
}
// Four bf16 values as one 8-byte write-through store.
__device__ __forceinline__ void stwt_bf4(GLOBAL uint16_t* p, float a, float b, float c, float d) {
  stwt64(p, (uint64_t)pk_bf2(a, b) | ((uint64_t)pk_bf2(c, d) << 32));
}
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
// 16-byte write-through stores through a buffer descriptor (cache policy SC1): one instruction, visible to the
// compiler. The descriptor covers [base, base + bytes) with bytes < 2^31; offsets are bytes from base.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wt_rsrc(const void* base, long long bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)(bytes < 0x7fffffffll ? bytes : 0x7fffffffll), 0x00020000);
}
__device__ __forceinline__ void stwt_buf(__amdgpu_buffer_rsrc_t r, int off, f32x4n v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), r, off, 0, 16 /* SC1 */);
}
// Four floats as bf16, one 8-byte write-through store through a buffer descriptor (32-bit offsets: no 64-bit address
// arithmetic per store).
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void stwt_bf4_buf(__amdgpu_buffer_rsrc_t r, int off, f32x4n v) {
  __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{pk_bf2(v.x, v.y), pk_bf2(v.z, v.w)}, r, off, 0, 16 /* SC1 */);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---------------------------------------------------------------------------------------------- views
// A buffer argument as an operator sees it. ld()/st() widen / round bf16 storage; f/i give typed raw pointers.
struct View {
  void* p; int rows, cols, dtype;
  __device__ bool ok() const { return p != nullptr; }
  __device__ GLOBAL float* f() const { return (GLOBAL float*)p; }
  __device__ GLOBAL int* i() const { return (GLOBAL int*)p; }
  __device__ GLOBAL uint16_t* h() const { return (GLOBAL uint16_t*)p; }
  __device__ float ld(long long k) const { return dtype == 2 ? bf2f(((const GLOBAL uint16_t*)p)[k]) : ((const GLOBAL float*)p)[k]; }
  __device__ float at(long long r, long long c) const { return ld(r * cols + c); }
  __device__ void st(long long k, float v) const { if (dtype == 2) stwt16((GLOBAL uint16_t*)p + k, f2bf(v)); else stwt32((GLOBAL float*)p + k, v); }
  __device__ long long n() const { return (long long)rows * cols; }
};

// A task's dispatch record, built on the host when the graph is uploaded (buffers are fixed by then): the descriptor,
// the argument words and, at every buffer argument's position, that buffer's view. A worker copies it to LDS with one
// parallel 16-byte load per thread instead of three dependent fetches (descriptor, then arguments, then the buffer
// table entries they name).
// The first KVM_REC_SUCC successor edges (device form, flag bits included) ride in the record, so the worker that
// completes the task signals them without a dependent load of the successor list (nsucc_rec of them; the rest, and
// all of them when nsucc_rec is 0, are read from the successor array).
#define KVM_REC_SUCC 64
struct KvmRec {
  MvmTaskDesc desc;
  int32_t args[KVM_MAX_ARGS];
  View views[KVM_MAX_ARGS];
  int32_t succ[KVM_REC_SUCC];
  int32_t nsucc_rec;
  int32_t pad[7];
};
static_assert(sizeof(View) == 24 && sizeof(KvmRec) == 1024, "record layout");
#define KVM_REC_VEC (int)(sizeof(KvmRec) / 16)
#define KVM_REC_VEC_OPS (int)(offsetof(KvmRec, succ) / 16)   // 16-byte pieces before the successors (all an operator reads)

// Byte offsets inside the pinned staging block of stream mode (host and device compute them alike).
struct KvmWinLayout {
  size_t meta, recs, tasks, succ, roots, total;
  __host__ __device__ KvmWinLayout(int wcap, int wtasks, int wedges) {
    auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
    meta = 0;
    recs = up((size_t)wcap * sizeof(KvmHostWin));
    tasks = up(recs + (size_t)wcap * wtasks * sizeof(KvmRec));
    succ = up(tasks + (size_t)wcap * wtasks * sizeof(MvmTaskDesc));
    roots = up(succ + (size_t)wcap * wedges * sizeof(int32_t));
    total = up(roots + (size_t)wcap * wtasks * sizeof(int32_t));
  }
};

struct Ctx {
  const LDS View* views;     // buffer arguments of the task, resolved from the buffer table by the dispatcher (in LDS)
  const LDS int32_t* a;      // argument words (in LDS)
  LDS char* smem;            // KVM_LDS_BYTES of LDS
  KvmCounters* cnt;
  int slot;
  int pre = 0;               // the task's first input-independent loads were issued before its dependency wait
  __device__ View buf(int k) const {
    if (a[k] < 0) return View{nullptr, 0, 0, 0};
    return View{views[k].p, views[k].rows, views[k].cols, views[k].dtype};
  }
  __device__ int i(int k) const { return a[k]; }
  __device__ float f(int k) const { return __int_as_float(a[k]); }
  // First error wins; the task then returns. Data-dependent errors only: argument shapes were validated on the host.
  __device__ void fail(int code, int x = 0, int y = 0) const {
    int zero = 0;
    if (__hip_atomic_compare_exchange_strong(&cnt->err_code, &zero, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      stwt32i((GLOBAL int*)&cnt->err_slot, slot); stwt32i((GLOBAL int*)&cnt->err_a, x); stwt32i((GLOBAL int*)&cnt->err_b, y);
    }
  }
};

__device__ __forceinline__ int tid() { return threadIdx.x; }
__device__ __forceinline__ int lane() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave() { return threadIdx.x >> 6; }

// Block-wide reductions over 256 threads (four wave64s), result returned to every thread. `red` = 4 floats of LDS.
__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
template <class P> __device__ __forceinline__ float block_sum(float v, P red) {
  v = wave_sum(v);
  __syncthreads();
  if (lane() == 0) red[wave()] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
template <class P> __device__ __forceinline__ float block_max(float v, P red) {
  v = wave_max(v);
  __syncthreads();
  if (lane() == 0) red[wave()] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ double wave_sum_d(double v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <class P> __device__ __forceinline__ double block_sum_d(double v, P red) {
  v = wave_sum_d(v);
  __syncthreads();
  if (lane() == 0) red[wave()] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
