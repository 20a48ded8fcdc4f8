// The persistent task-graph executor for MI355X (gfx950): device scheduler, operator dispatch and the C ABI host side.
//
// Device side (one workgroup of 256 threads per CU, all resident for the whole graph):
//   * Ready queues: every task is enqueued exactly once (by the last predecessor to finish, by a version publisher,
//     or at launch for roots), so a queue is a plain array of cells filled in enqueue order: enqueue takes the next
//     tail slot and stores the task index; a worker takes the next head ticket and waits for that cell. Task t always
//     goes to queue t % nq, so each queue knows how many tasks it will see, and a ticket past that count means the
//     queue is drained and the worker exits. No cell is ever reused: no ABA, no ring-capacity budget (reference
//     design for comparison: include/mvm_sched.cuh:115-374). There is one queue per XCD (workers of block b use queue
//     b % nq; the hardware places block b on XCD b % 8), so the ticket and tail atomics of a phase's tasks spread over
//     eight addresses instead of one.
//   * Dependencies: operators store only with write-through (agent-scope, sc1) stores, so after an operator each wave
//     waits for its own stores and the workgroup barrier orders them before wave 0 signals successors, with no
//     release fence (an agent-scope release writes the XCD's whole L2 back: microseconds per task). Wave 0
//     decrements successor counters (relaxed atomics) and enqueues the ones that reach zero; the worker that dequeues
//     a task acquires (agent scope: L1 and L2 invalidate) before running it.
//   * Versions: a task released with version[wait_var] < wait_ver is parked on the variable's lock-free list. The
//     publisher CASes version from pub_ver-1 to pub_ver (else VERSION_GAP), then takes the whole list and enqueues
//     what is now satisfied. Parker (push; seq_cst fence; re-read version) and publisher (CAS version; seq_cst fence;
//     exchange list) form a Dekker pair, and a per-task state CAS makes the enqueue unique.
//   * Errors: first error wins (CAS on err_code); every worker polls it while waiting and leaves. A stall timeout
//     (no task finished for timeout_ticks while a worker waits) ends the run with TIMEOUT instead of hanging.
#include <functional>
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <atomic>
#include <chrono>
#include <mutex>
#include <thread>
#include <vector>
#include "common.h"
#include "ops_basic.h"
#include "ops_gemm.h"
#include "ops_attn.h"
#include "ops_decode.h"
#include "ops_stream.h"
#include "validate.h"
#include "static_plan.h"

using namespace kvm;

// ---------------------------------------------------------------------------------------------- scheduler
__device__ __forceinline__ void queue_overflow(const KvmDevState& S) {
  int z = 0;   // cannot happen when every task is enqueued once; reported, never written out of bounds
  __hip_atomic_compare_exchange_strong(&S.cnt->err_code, &z, (int)KVM_ERR_QUEUE_OVERFLOW, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Host-memory (pinned, fine-grained) accesses of stream mode: system scope.
__device__ __forceinline__ long long ld_sys64(const long long* p) { return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM); }
__device__ __forceinline__ int ld_sys(const int* p) { return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM); }
__device__ __forceinline__ void st_sys64(long long* p, long long v) { __hip_atomic_store(p, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM); }
// Stream mode: cell of ticket `pos` of queue q, stamped with its round.
__device__ __forceinline__ void put_cell64(const KvmDevState& S, int q, unsigned pos, int t, bool release) {
  const unsigned long long v = ((unsigned long long)(pos / (unsigned)S.qcap + 1u) << 32) | (unsigned)t;
  unsigned long long* c = &S.ready64[(size_t)q * S.qcap + (pos & (unsigned)(S.qcap - 1))];
  if (release) __hip_atomic_store(c, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  else __hip_atomic_store(c, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Stream mode: the ring of task t (its queue group, and with scheduler classes its class within the group).
__device__ __forceinline__ int ring_of(const KvmDevState& S, int t) {
  return S.ncls ? (t % S.nq) * S.ncls + S.tasks[t].workload_id : t % S.nq;
}
// Deadlines count from the launch, in stream mode from the admission of the task's window.
__device__ __forceinline__ unsigned long long deadline_base(const KvmDevState& S, int t) {
  return S.stream ? S.win_t0[t / S.wtasks] : S.sched->t0;
}
// Stream mode: takes the admission lock when a window is staged and not admitted yet (or the host closed and fin is
// still down). Thread 0 / one lane only.
__device__ bool take_admission(const KvmDevState& S) {
  if (ld_relaxed(&S.adm->fin)) return false;
  const bool work = (long long)ld_relaxed(&S.adm->next) < ld_sys64(&S.hctl->submitted) || ld_sys(&S.hctl->closed);
  int z = 0;
  return work && ld_relaxed(&S.adm->lock) == 0 &&
         __hip_atomic_compare_exchange_strong(&S.adm->lock, &z, 1, __ATOMIC_ACQUIRE, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Task affinity (reference: mvm_sched.cuh, the cell's pref and mvm_sched_pref): a task released by a finishing task
// prefers the releasing worker (chain affinity), or, in a class with op affinity, the worker that last finished a task
// of its operator; roots prefer none. Recorded with the release time before the task's cell is published.
__device__ __forceinline__ void note_ready(const KvmDevState& S, int t, bool chain) {
  int pref = chain ? (int)blockIdx.x : -1;
  const MvmTaskDesc& d = S.tasks[t];
  if (chain && S.sched->cls[d.workload_id].opaff && d.op_id >= 0 && d.op_id < KVM_OP_SLOTS) {
    const int ob = ld_relaxed(&S.op_blk[d.op_id]);
    if (ob >= 0) pref = ob;
  }
  __hip_atomic_store(&S.aff[t], (wall_clock64() << 12) | (unsigned long long)(pref + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void enqueue(const KvmDevState& S, int t, bool chain = true) {
  if (S.aff) note_ready(S, t, chain);
  if (S.stream) {
    const int q = ring_of(S, t);
    put_cell64(S, q, (unsigned)add_relaxed(&S.queues[q].tail, 1), t, true);
    return;
  }
  if (S.tq) {   // priority mode: the task's (queue group, bucket) queue; its release time first when ready tasks age
    const int q = S.tq[t];
    if (S.ready_ts) __hip_atomic_store(&S.ready_ts[t], wall_clock64(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int pos = add_relaxed(&S.queues[q].tail, 1);
    if (pos >= S.qcount[q]) { queue_overflow(S); return; }
    st_release(&S.ready[S.qoff[q] + pos], t);
    return;
  }
  const int q = t % S.nq;
  int pos = add_relaxed(&S.queues[q].tail, 1);
  if (pos >= S.qcap) { queue_overflow(S); return; }
  st_release(&S.ready[q * S.qcap + pos], t);
}

// Priority inheritance (reference: the policy block's boost, include/mvm_sched.cuh:35-40 and 486-496, restated without a
// policy block): the classes boosted now, from the parked-waiter counts. wants[w] = the classes publishing a variable
// that a parked task of class w waits on; the boost is every wanted class, closed transitively (a boosted class's own
// parked tasks boost their publishers). Recomputed by whoever parks or unparks a task, and by idle workers of the class
// scheduler (a recomputation that raced with another park is repaired by the next idle poll).
__device__ int boost_mask(const KvmDevState& S) {
  const int nc = S.ncls;
  int wants[KVM_MAX_CLASSES] = {};
  for (int i = 0; i < S.npub; ++i) {
    const int v = S.publist[i], pc = S.pubcls[v];
    for (int w = 0; w < nc; ++w)
      if (ld_relaxed(&S.pv[v * KVM_MAX_CLASSES + w]) > 0) wants[w] |= pc & ~(1 << w);
  }
  int B = 0;
  for (int w = 0; w < nc; ++w) B |= wants[w];
  for (int it = 0; it < nc; ++it)
    for (int c = 0; c < nc; ++c) if ((B >> c) & 1) B |= wants[c];
  return B;
}
// A task of a class enters (+1) or leaves (-1) the parked state on `var`; the boost follows.
__device__ void park_count(const KvmDevState& S, int t, int var, int d) {
  if (!S.pv || !(S.sched->flags & KVM_SCHED_F_INHERIT)) return;
  const int c = S.tasks[t].workload_id;
  if (c < 0 || c >= S.ncls) return;
  add_relaxed(&S.pv[var * KVM_MAX_CLASSES + c], d);
  st_relaxed(&S.sched->boost, boost_mask(S));
}

__device__ void park(const KvmDevState& S, int t, int var, int want) {
  int* head = &S.park_head[var];
  int h = ld_relaxed(head);
  do { st_relaxed(&S.park_next[t], h); } while (!__hip_atomic_compare_exchange_strong(head, &h, t, __ATOMIC_ACQ_REL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  fence_seqcst();
  if (ld_acquire(&S.version[var]) >= want && cas_acqrel(&S.state[t], 1, 2)) { park_count(S, t, var, -1); enqueue(S, t); }
}

// A task whose predecessors have all finished: run it when its version wait holds, else park it.
// chain: released by a finishing task on this worker (false for roots).
__device__ void release(const KvmDevState& S, int t, bool chain = true) {
  const MvmTaskDesc& d = S.tasks[t];
  int var = d.wait_var;
  if (var < 0 || ld_acquire(&S.version[var]) >= d.wait_ver) { st_relaxed(&S.state[t], 2); enqueue(S, t, chain); return; }
  st_relaxed(&S.state[t], 1);
  park_count(S, t, var, 1);
  park(S, t, var, d.wait_ver);
}

__device__ void publish(const KvmDevState& S, int slot, int var, int ver) {
  int expect = ver - 1;
  if (!__hip_atomic_compare_exchange_strong(&S.version[var], &expect, ver, __ATOMIC_ACQ_REL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
    int z = 0;
    if (__hip_atomic_compare_exchange_strong(&S.cnt->err_code, &z, (int)KVM_ERR_VERSION_GAP, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
      S.cnt->err_slot = slot; S.cnt->err_a = expect; S.cnt->err_b = ver;
    }
    return;
  }
  if (S.hver) __hip_atomic_store(&S.hver[var], ver, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);   // host's live view
  fence_seqcst();
  int h = xchg_acqrel(&S.park_head[var], -1);
  while (h >= 0) {
    int nx = ld_relaxed(&S.park_next[h]);
    if (ld_relaxed(&S.state[h]) == 1) {
      int want = S.tasks[h].wait_ver;
      if (ld_acquire(&S.version[var]) >= want) { if (cas_acqrel(&S.state[h], 1, 2)) { park_count(S, h, var, -1); enqueue(S, h); } }
      else park(S, h, var, want);
    }
    h = nx;
  }
}

// Stall check of a waiting worker, every 4096 polls: has any worker finished a task since the last look? After
// timeout_ticks without one, the run ends with TIMEOUT (first error wins). Returns true when it fired.
__device__ bool stalled(const KvmDevState& S, unsigned long long& since, int& seen, int ticket) {
  int d = 0;
  for (int w = 0; w < S.grid; ++w) d += ld_relaxed(&S.done_blk[w]);
  unsigned long long now = wall_clock64();
  // stream mode: with every admitted task finished the device is waiting for the host, which is no stall
  if (S.stream && d >= ld_relaxed(&S.adm->admitted)) { seen = d; since = now; return false; }
  if (d != seen) { seen = d; since = now; return false; }
  if (now - since <= S.timeout_ticks) return false;
  int z = 0;
  if (__hip_atomic_compare_exchange_strong(&S.cnt->err_code, &z, (int)KVM_ERR_TIMEOUT, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
    S.cnt->err_slot = -1; S.cnt->err_a = ticket; S.cnt->err_b = d;
  }
  return true;
}

// Priority-mode pop, run by all 64 lanes of wave 0 (lane b watches bucket b of this worker's queue group; bucket 0 is
// the highest priority present). Strict priority: the lowest non-empty bucket wins; with aging, the largest
// priority * aging_ticks + time since release (reference rule: mvm_sched.cuh:155-220, score = priority * aging + age).
// A bucket's head is claimed with a CAS only while head < tail (the cell is reserved, so its store is imminent), so a
// head never passes the bucket's task count; the worker leaves when every bucket's head has reached its count.
// Returns the task, or -1 to leave (drained or error).
__device__ int pop_prio(const KvmDevState& S) {
  const int l = lane(), g = blockIdx.x % S.nq, qi = g * S.nb + l;
  const bool mine = l < S.nb;
  const int cnt = mine ? S.qcount[qi] : 0, off = mine ? S.qoff[qi] : 0;
  const unsigned long long boost = (mine && S.aging_ticks) ? (unsigned long long)S.bucket_prio[l] * S.aging_ticks : 0ull;
  unsigned long long since = wall_clock64();
  int seen = -1;
  for (unsigned polls = 0;; ++polls) {
    if (__shfl(ld_relaxed(&S.cnt->err_code), 0, 64) != 0) return -1;
    const int h = mine ? (int)ld_relaxed(&S.queues[qi].head) : 0;
    const int tl = mine ? ld_relaxed(&S.queues[qi].tail) : 0;
    if (__ballot(mine && h < cnt) == 0ull) return -1;
    bool avail = mine && h < tl && h < cnt;
    unsigned long long score = 0;
    if (S.aging_ticks) {
      int cell = avail ? ld_acquire(&S.ready[off + h]) : -1;
      avail = cell >= 0;
      if (avail) score = boost + (wall_clock64() - __hip_atomic_load(&S.ready_ts[cell], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
    const unsigned long long m = __ballot(avail);
    if (m) {
      int win = __ffsll((long long)m) - 1;
      if (S.aging_ticks) {
        unsigned long long best = avail ? score : 0ull;
        for (int o = 32; o > 0; o >>= 1) { unsigned long long y = __shfl_xor(best, o, 64); best = y > best ? y : best; }
        win = __ffsll((long long)__ballot(avail && score == best)) - 1;
      }
      int got = -1;
      if (l == win) {
        unsigned expect = (unsigned)h;
        if (__hip_atomic_compare_exchange_strong(&S.queues[qi].head, &expect, expect + 1u, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
          for (;;) {   // the enqueuer reserved this cell before we saw the tail: its store is in flight
            got = ld_relaxed(&S.ready[off + h]);
            if (got >= 0 || ld_relaxed(&S.cnt->err_code) != 0) break;
            __builtin_amdgcn_s_sleep(1);
          }
        }
      }
      got = __shfl(got, win, 64);
      if (got >= 0) { fence_acquire(); return got; }
      continue;   // lost the head to another worker: look again at once
    }
    __builtin_amdgcn_s_sleep(1);
    int fired = 0;
    if (l == 0 && (polls & 4095) == 4095) fired = stalled(S, since, seen, -1);
    if (__shfl(fired, 0, 64)) return -1;
  }
}

// Class-mode pop (scheduler classes on), by all 64 lanes of wave 0: lane c * nb + b watches bucket b of class c in
// this worker's queue group (reference policy: mvm_pop, mvm_sched.cuh:261-374; its tiers restated on one wave64
// that sees every class's buckets at once instead of deciding the class first and scanning it after). Each
// available bucket head gets a key (tier << 60 | order): tier 1 its class is below its reservation (order: running /
// min_cta), tier 2 its deadline is within the class's EDF window (order: slack), tier 3 the class's weighted virtual
// time. Classes at their cap offer nothing outside tier 1. The smallest key wins; inside the winning class the
// bucket rule of pop_prio applies (lowest bucket, or the largest aged score). The winner counts itself into its
// class's running workers before the head CAS, and gives the count back when capped or when the CAS loses, so the
// cap holds at every instant. Returns the task (how = KVM_TRACE_* start bits, est = the virtual-time charge taken,
// in ticks), or -1 to leave.
#define KVM_SLACKMAX (1ll << 40)
__device__ int pop_cls(const KvmDevState& S, int& how, unsigned& est) {
  const int l = lane(), g = blockIdx.x % S.nq, nb = S.nb, nc = S.ncls;
  const bool lane_ok = l < nc * nb;
  const int c = lane_ok ? l / nb : 0, b = lane_ok ? l % nb : 0;
  KvmClsDev* const K = S.sched->cls;
  const int flags = S.sched->flags, bw_limit = S.sched->bw_limit;
  const bool arb = (flags & KVM_SCHED_F_ARBITER) != 0, inherit = (flags & KVM_SCHED_F_INHERIT) != 0;
  const int mn = (flags & KVM_SCHED_F_GUARANTEE) ? K[c].min_cta : 0, mx = K[c].max_cta, urg = K[c].urgent_ticks, vt_mul = K[c].vt_mul;
  const int bwc = K[c].bw_cta;
  const bool bw_gate = K[c].has_bw != 0 && (bwc < KVM_UNLIMITED || arb);   // the head task's kind matters
  const bool mine = lane_ok && (int)blockIdx.x >= K[c].blk_lo && (int)blockIdx.x < K[c].blk_hi;
  const bool strm = S.stream != 0;
  const unsigned long long aff_ticks = S.aff ? S.sched->aff_ticks : 0ull;
  const bool need_cell = strm || S.aging_ticks != 0 || (urg > 0 && K[c].has_dl != 0) || bw_gate || aff_ticks != 0;
  const int qi = (g * nc + c) * nb + b;
  const int cnt = mine && !strm ? S.qcount[qi] : 0, off = mine && !strm ? S.qoff[qi] : 0;
  const unsigned long long boost = (mine && S.aging_ticks) ? (unsigned long long)S.bucket_prio[b] * S.aging_ticks : 0ull;
  const unsigned long long t0 = S.sched->t0;
  unsigned long long since = wall_clock64();
  int seen = -1;
  for (unsigned polls = 0;; ++polls) {
    if (__shfl(ld_relaxed(&S.cnt->err_code), 0, 64) != 0) return -1;
    const int h = mine ? (int)ld_relaxed(&S.queues[qi].head) : 0;
    bool avail;
    int cell = -1;
    if (strm) {   // a ring: the head cell is published when it carries the head's round; done once closed and drained
      if (ld_acquire(&S.adm->fin) && __ballot(mine && (unsigned)h < (unsigned)ld_relaxed(&S.adm->total[qi])) == 0ull) return -1;
      avail = false;
      if (mine) {
        const unsigned long long v = __hip_atomic_load(&S.ready64[(size_t)qi * S.qcap + ((unsigned)h & (unsigned)(S.qcap - 1))],
                                                       aff_ticks ? __ATOMIC_ACQUIRE : __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((unsigned)(v >> 32) == (unsigned)h / (unsigned)S.qcap + 1u) { cell = (int)(unsigned)v; avail = true; }
      }
    } else {
      const int tl = mine ? ld_relaxed(&S.queues[qi].tail) : 0;
      if (__ballot(mine && h < cnt) == 0ull) return -1;
      avail = mine && h < tl && h < cnt;
      if (avail && need_cell) { cell = ld_acquire(&S.ready[off + h]); avail = cell >= 0; }
    }
    int run_k = 0, bwr_k = 0;
    unsigned long long vt_k = 0;
    if (l < nc) {
      run_k = ld_relaxed(&K[l].running);
      bwr_k = ld_relaxed(&K[l].bw_running);
      vt_k = __hip_atomic_load(&K[l].vtime, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const int run = __shfl(run_k, c, 64), bwr = __shfl(bwr_k, c, 64);
    const unsigned long long vt = __shfl(vt_k, c, 64);
    const int boost = inherit ? __shfl(l == 0 ? ld_relaxed(&S.sched->boost) : 0, 0, 64) : 0;
    const int bwt = arb ? __shfl(l == 0 ? ld_relaxed(&S.sched->bw_total) : 0, 0, 64) : 0;
    const bool isbw = bw_gate && cell >= 0 && S.tbw[cell];
    const unsigned long long now = wall_clock64();
    if (avail && aff_ticks) {   // a head reserved for another worker within the affinity window is not offered here
      const unsigned long long a = __hip_atomic_load(&S.aff[cell], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int pref = (int)(a & 0xfffull) - 1;
      if (pref >= 0 && pref != (int)blockIdx.x && now - (a >> 12) < aff_ticks) avail = false;
    }
    unsigned long long key = ~0ull, score = 0;
    if (avail) {
      if ((boost >> c) & 1) key = (unsigned long long)run;                       // tier 0: inheritance, no caps
      else if (run < mn) key = (1ull << 60) | (((unsigned long long)run << 20) / (unsigned)(mn > 0 ? mn : 1));
      else if (run >= mx || (isbw && (bwr >= bwc || (arb && bwt >= bw_limit)))) avail = false;
      else {
        key = (3ull << 60) | (vt < (1ull << 60) ? vt : (1ull << 60) - 1);
        if (urg > 0 && cell >= 0) {
          const int dl = S.tasks[cell].deadline_us;
          if (dl >= 0) {
            long long slack = (long long)((strm ? S.win_t0[cell / S.wtasks] : t0) + (unsigned long long)dl * 100ull) - (long long)now;
            if (slack <= (long long)urg) {
              slack = slack < -KVM_SLACKMAX ? -KVM_SLACKMAX : slack > KVM_SLACKMAX ? KVM_SLACKMAX : slack;
              key = (2ull << 60) | (unsigned long long)(slack + KVM_SLACKMAX);
            }
          }
        }
      }
      if (avail && S.aging_ticks) score = boost + (now - __hip_atomic_load(&S.ready_ts[cell], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
    if (!avail) key = ~0ull;
    if (__ballot(avail)) {
      unsigned long long best = key;
      for (int o = 32; o > 0; o >>= 1) { const unsigned long long y = __shfl_xor(best, o, 64); best = y < best ? y : best; }
      unsigned long long wm = __ballot(avail && key == best);
      const int first = __ffsll((long long)wm) - 1, wc = first / nb;
      const unsigned long long cmask = nb >= 64 ? ~0ull : (((1ull << nb) - 1ull) << (wc * nb));
      wm &= cmask;                                 // equal keys across classes: the lower class
      const int tier = (int)(best >> 60);
      int win = first;
      if (tier != 2 && S.aging_ticks) {
        const bool cand = (wm >> l) & 1ull;
        unsigned long long bs = cand ? score : 0ull;
        for (int o = 32; o > 0; o >>= 1) { const unsigned long long y = __shfl_xor(bs, o, 64); bs = y > bs ? y : bs; }
        win = __ffsll((long long)__ballot(cand && score == bs)) - 1;
      }
      int got = -1;
      unsigned charge = 0;
      if (l == win) {
        KvmClsDev& k = K[c];
        // counts taken before the head CAS and given back when capped meanwhile or when the CAS loses: every cap holds
        // at every instant (tiers 0 and 1 override the caps but are counted)
        const int old = add_relaxed(&k.running, 1);
        const int oldbw = isbw ? add_relaxed(&k.bw_running, 1) : 0;
        const int oldt = isbw && arb ? add_relaxed(&S.sched->bw_total, 1) : 0;
        auto give_back = [&]() {
          add_relaxed(&k.running, -1);
          if (isbw) add_relaxed(&k.bw_running, -1);
          if (isbw && arb) add_relaxed(&S.sched->bw_total, -1);
        };
        if (tier >= 2 && (old >= mx || (isbw && (oldbw >= bwc || (arb && oldt >= bw_limit))))) give_back();   // capped meanwhile
        else {
          unsigned expect = (unsigned)h;
          if (__hip_atomic_compare_exchange_strong(&S.queues[qi].head, &expect, expect + 1u, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
            // ring: the cell read above is the head's (its round matched, and it cannot be reused before its task has
            // run, which needs this claim); counted queues: the enqueuer reserved the cell before we saw the tail
            if (strm) got = cell;
            else for (;;) {   // the enqueuer reserved this cell before we saw the tail: its store is in flight
              got = ld_relaxed(&S.ready[off + h]);
              if (got >= 0 || ld_relaxed(&S.cnt->err_code) != 0) break;
              __builtin_amdgcn_s_sleep(1);
            }
          }
          if (got < 0) give_back();
          else {
            __hip_atomic_fetch_max(&k.max_running, old + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            charge = __hip_atomic_load(&k.est, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(&k.vtime, (unsigned long long)charge * (unsigned)vt_mul, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
      got = __shfl(got, win, 64);
      if (got >= 0) {
        est = __shfl(charge, win, 64);
        how = (tier == 0 ? KVM_TRACE_BOOST : tier == 1 ? KVM_TRACE_RESV : tier == 2 ? KVM_TRACE_URGENT : 0) |
              (__shfl((int)isbw, win, 64) ? KVM_HOW_BW : 0);
        fence_acquire();
        return got;
      }
      continue;
    }
    __builtin_amdgcn_s_sleep(1);
    if (strm && (polls & 15) == 0 && __shfl((int)(l == 0 && take_admission(S)), 0, 64)) return -2;   // lock taken: admit
    int fired = 0;
    if (l == 0 && inherit && S.pv && (polls & 63) == 63) st_relaxed(&S.sched->boost, boost_mask(S));   // repair a raced boost
    if (l == 0 && (polls & 4095) == 4095) fired = stalled(S, since, seen, -1);
    if (__shfl(fired, 0, 64)) return -1;
  }
}

// Completion accounting of a class-mode task (thread 0): the worker leaves its class's running count, the
// virtual-time charge taken at the claim is corrected to the ticks run, the class's running-time estimate moves
// (a racy moving average, an estimate by design) and the statistics line counts the task. Returns the trace bits.
__device__ int cls_done(const KvmDevState& S, const MvmTaskDesc& d, int slot, int how, unsigned est, unsigned long long start) {
  KvmClsDev& k = S.sched->cls[d.workload_id];
  const unsigned long long end = wall_clock64(), run = end - start;
  if (S.op_blk && d.op_id >= 0 && d.op_id < KVM_OP_SLOTS) st_relaxed(&S.op_blk[d.op_id], (int)blockIdx.x);
  add_relaxed(&k.running, -1);
  if (how & KVM_HOW_BW) {
    add_relaxed(&k.bw_running, -1);
    if (S.sched->flags & KVM_SCHED_F_ARBITER) add_relaxed(&S.sched->bw_total, -1);
  }
  __hip_atomic_fetch_add(&k.vtime, (unsigned long long)(((long long)run - (long long)est) * (long long)k.vt_mul), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned r32 = run < 0xffffffffull ? (unsigned)run : 0xffffffffu;
  const unsigned old = __hip_atomic_load(&k.est, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&k.est, old ? (unsigned)(((unsigned long long)old * 7ull + r32) / 8ull) : r32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool missed = d.deadline_us >= 0 && end > deadline_base(S, slot) + (unsigned long long)d.deadline_us * 100ull;
  auto add64 = [](unsigned long long* p, unsigned long long v) { __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  add64(&k.tasks, 1ull);
  add64(&k.busy, run);
  if (how & KVM_TRACE_RESV) add64(&k.resv_starts, 1ull);
  if (how & KVM_TRACE_URGENT) add64(&k.urgent_starts, 1ull);
  if (how & KVM_TRACE_BOOST) add64(&k.boost_starts, 1ull);
  if (missed) add64(&k.missed, 1ull);
  return (how & ~KVM_HOW_BW) | (missed ? KVM_TRACE_MISSED : 0);
}

// Stream-mode admission, by the whole workgroup of the worker holding the admission lock: every window the host has
// staged since is copied from pinned host memory into its slot (records, descriptors, successors; counters and park
// links reset), its tasks are added to the per-queue totals and its roots are released, window by window in seq
// order. Then, once the host has closed and everything is admitted, fin is raised. Releases the lock.
__device__ void admit_windows(const KvmDevState& S) {
  __shared__ int s_go, s_seq;
  __shared__ int s_ring[KVM_MAX_QUEUES * KVM_MAX_CLASSES];   // with classes: the window's tasks per (group, class) ring
  const int t = threadIdx.x;
  const KvmWinLayout lay(S.wcap, S.wtasks, S.wedges);
  for (;;) {
    if (t == 0) {
      const long long sub = ld_sys64(&S.hctl->submitted);
      s_seq = ld_relaxed(&S.adm->next);
      s_go = s_seq < sub;
    }
    __syncthreads();
    if (!s_go) break;
    const int seq = s_seq, w = seq % S.wcap, base = w * S.wtasks;
    const KvmHostWin* hm = (const KvmHostWin*)(S.hwin + lay.meta) + w;
    const int n = ld_sys(&hm->ntasks), ne = ld_sys(&hm->nedges), nr = ld_sys(&hm->nroots);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "");    // the staged window (written before `submitted`) is visible
    const u32x4_t* hr = (const u32x4_t*)(S.hwin + lay.recs + (size_t)base * sizeof(KvmRec));
    u32x4_t* dr = (u32x4_t*)(const_cast<KvmRec*>(S.recs) + base);
    for (int k = t; k < n * KVM_REC_VEC; k += KVM_THREADS) dr[k] = hr[k];
    const u32x4_t* ht = (const u32x4_t*)(S.hwin + lay.tasks + (size_t)base * sizeof(MvmTaskDesc));
    u32x4_t* dt = (u32x4_t*)(const_cast<MvmTaskDesc*>(S.tasks) + base);
    for (int k = t; k < n * 4; k += KVM_THREADS) dt[k] = ht[k];
    const int32_t* hs = (const int32_t*)(S.hwin + lay.succ) + (size_t)w * S.wedges;
    int32_t* ds = const_cast<int32_t*>(S.succ) + (size_t)w * S.wedges;
    for (int k = t; k < ne; k += KVM_THREADS) ds[k] = hs[k];
    const MvmTaskDesc* htd = (const MvmTaskDesc*)(S.hwin + lay.tasks) + base;
    const int nring = S.nq * S.ncls;
    if (S.ncls) for (int k = t; k < nring; k += KVM_THREADS) s_ring[k] = 0;
    __syncthreads();
    for (int k = t; k < n; k += KVM_THREADS) {
      S.indeg[base + k] = htd[k].indegree;
      S.state[base + k] = 0;
      S.park_next[base + k] = -1;
      if (S.trace_on) { KvmTrace z = {}; z.ver0 = z.ver1 = -1; S.trace[base + k] = z; }
      if (S.ncls) {   // class of the task (validated on the host), its bandwidth flag (staged in reserved1), its publication
        const int cls = htd[k].workload_id, pv = htd[k].pub_var;
        atomicAdd(&s_ring[((base + k) % S.nq) * S.ncls + cls], 1);
        S.tbw[base + k] = (unsigned char)(htd[k].reserved1 & 1);
        if (pv >= 0) __hip_atomic_fetch_or(&S.pubcls[pv], 1 << cls, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (t == 0) {
      st_relaxed(&S.win_left[w], n);
      st_relaxed(&S.win_seq[w], seq);
      __hip_atomic_store(&S.win_t0[w], wall_clock64(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (S.ncls) for (int r = 0; r < nring; ++r) add_relaxed(&S.adm->total[r], s_ring[r]);
      else for (int q = 0; q < S.nq; ++q) add_relaxed(&S.adm->total[q], ld_sys(&hm->qn[q]));
      add_relaxed(&S.adm->admitted, n);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    }
    __syncthreads();
    const int32_t* hroot = (const int32_t*)(S.hwin + lay.roots) + base;
    for (int k = t; k < nr; k += KVM_THREADS) release(S, base + hroot[k], false);
    __syncthreads();
    if (t == 0) st_release(&S.adm->next, seq + 1);
    __syncthreads();
  }
  if (t == 0) {
    if (ld_sys(&S.hctl->closed) && (long long)ld_relaxed(&S.adm->next) == ld_sys64(&S.hctl->submitted)) st_release(&S.adm->fin, 1);
    st_release(&S.adm->lock, 0);
  }
  __syncthreads();
}

// Stream-mode dequeue by thread 0: the ticket held across calls (taken once, kept while the worker admits). Returns
// a task, -1 to leave (error, or closed with every ticket of this queue served), or -2 with the admission lock taken.
__device__ int stream_next(const KvmDevState& S, long long& held) {
  const int q = blockIdx.x % S.nq;
  if (held < 0) held = add_relaxed(&S.queues[q].head, 1u);
  const unsigned tk = (unsigned)held, round = tk / (unsigned)S.qcap + 1u;
  const unsigned long long* cell = &S.ready64[(size_t)q * S.qcap + (tk & (unsigned)(S.qcap - 1))];
  unsigned long long since = wall_clock64();
  int seen = -1;
  for (unsigned polls = 0;; ++polls) {
    const unsigned long long v = __hip_atomic_load(cell, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int err = ld_relaxed(&S.cnt->err_code);
    if ((unsigned)(v >> 32) == round) { fence_acquire(); held = -1; return (int)(unsigned)v; }
    if (err != 0) return -1;
    if (ld_relaxed(&S.adm->fin) && tk >= (unsigned)ld_relaxed(&S.adm->total[q])) return -1;
    if ((polls & 15) == 0 && take_admission(S)) return -2;
    __builtin_amdgcn_s_sleep(2);
    if ((polls & 4095) == 4095 && stalled(S, since, seen, (int)tk)) return -1;
  }
}

__device__ __forceinline__ int xcc_id() {
  // HW_REG_XCC_ID (hwreg 20), bits [3:0]: the XCD this wave runs on
  return __builtin_amdgcn_s_getreg((3 << 11) | 20) & 0xf;
}

__device__ void dispatch(int op, const Ctx& c) {
  switch (op) {
    case 0: break;
    case 1: op_copy(c); break;
    case 2: if (!op_add_fast(c)) op_add(c); break;
    case 3: if (!op_scale_fast(c)) op_scale(c); break;
    case 4: if (!op_relu_fast(c)) op_relu(c); break;
    case 5: op_sgd(c); break;
    case 6: op_predict(c); break;
    case 7: op_mse_grad(c); break;
    case 8: op_matmul(c); break;
    case 9: op_fill(c); break;
    case 10: op_spin(c); break;
    case 32: if (!op_embedding_fwd_fast(c)) op_embedding_fwd(c); break;
    case 33: if (!op_embedding_bwd_fast(c)) op_embedding_bwd(c); break;
    case 34: op_matmul_tile(c); break;
    case 35: if (!op_norm_fwd_fast<false>(c)) op_norm_fwd<false>(c); break;
    case 36: if (!op_norm_fwd_fast<true>(c)) op_norm_fwd<true>(c); break;
    case 37: if (!op_norm_bwd_dx_fast<false>(c)) op_norm_bwd_dx<false>(c); break;
    case 38: if (!op_norm_bwd_dx_fast<true>(c)) op_norm_bwd_dx<true>(c); break;
    case 39: if (!op_norm_bwd_params_fast(c)) op_norm_bwd_params(c); break;
    case 40: op_gelu_fwd(c); break;
    case 41: op_gelu_bwd(c); break;
    case 42: op_residual_add(c); break;
    case 43: op_rope<1>(c); break;
    case 44: op_rope<-1>(c); break;
    case 45: op_attn_fwd(c); break;
    case 46: if (!op_attn_bwd_delta_fast(c)) op_attn_bwd_delta(c); break;
    case 47: op_attn_bwd_dq(c); break;
    case 48: op_attn_bwd_dkv(c); break;
    case 49: op_kv_append(c); break;
    case 50: op_attn_decode(c); break;
    case 51: op_softmax_ce_fwd_any(c); break;
    case 52: op_softmax_ce_reduce(c); break;
    case 53: op_softmax_ce_bwd_any(c); break;
    case 54: op_adamw(c); break;
    case 55: if (!op_gradnorm_partial_fast(c)) op_gradnorm_partial(c); break;
    case 56: op_gradnorm_finish(c); break;
    case 57: op_sample(c); break;
    case 58: op_argmax(c); break;
    case 59: op_zero_buf(c); break;
    case 60: op_counter_inc(c); break;
    case 61: if (!op_colsum_fast(c)) op_colsum(c); break;
    case 62: op_select_window(c); break;
    case 63: op_gather_rows(c); break;
    case 96: if (!op_act_fwd_fast(c)) op_act_fwd(c); break;
    case 97: if (!op_act_bwd_fast(c)) op_act_bwd(c); break;
    case 98: if (!op_silu_mul_fwd_fast(c)) op_silu_mul_fwd(c); break;
    case 99: op_silu_mul_bwd(c); break;
    case 100: op_softmax_rows_fwd(c); break;
    case 101: op_softmax_rows_bwd(c); break;
    case 102: op_gather_rows_scaled(c); break;
    case 103: op_scatter_add_rows(c); break;
    case 104: op_row_dot(c); break;
    case 113: if (!op_round_bf16_fast(c)) op_round_bf16(c); break;
    case 114: op_matmul_tile_bf16(c); break;
    case 115: op_adamw_lr(c); break;
    case 116: op_lr_schedule(c); break;
    case 117: if (!op_scale_flat_fast(c)) op_scale_flat(c); break;
    case 118: op_add_rowtile(c); break;
    case 120: op_matmul_tile_silu_mul(c); break;
    case 121: op_matmul_tile_silu_mul_bwd(c); break;
    case 122: op_matmul_mma_bf16(c); break;
    case 123: op_sgd_range(c); break;
    case 126: op_round_tf32(c); break;
    case 127: op_softmax_ce_fused_any(c); break;
    case 134: op_gemv_bf16(c); break;
    case 135: op_attn_decode_part_any(c); break;
    case 306: op_attn_decode_part_qkn(c); break;
    case 310: op_attn_decode_part_merge(c); break;
    case 308: op_matmul_mma_bf16_delta(c); break;
    case 309: if (!op_norm_bwd_dx_res_fast(c)) op_norm_bwd_dx_res(c); break;
    case 136: op_attn_decode_merge(c); break;
    case 300: op_head_rmsnorm(c); break;
    case 301: op_gemv_bf16_rows(c); break;
    case 311: op_gemv_swiglu(c); break;
    case 302: op_matmul_mma_bf16_kr(c); break;
    case 303: op_splitk_reduce(c); break;
    case 304: op_matmul_mma_bf16_256(c); break;
    case 305: op_adamw_bf16(c); break;
    default: if (threadIdx.x == 0) c.fail(KVM_ERR_BAD_OP, op, 0);
  }
}

// Static-path wait on `cnt` (worker, need) pairs at ent, by the 64 lanes of one wave: each lane takes up to four
// entries per round of 256 and polls them together (their loads in flight at once), entries of the worker itself
// (program order) and set references (worker < 0) skipped. Gives up on an error anywhere or after timeout_ticks
// (TIMEOUT, first error wins). Returns true when it gave up (uniform across the wave).
__device__ bool static_wait(const KvmDevState& S, const int* ent, int cnt, int self, int slot) {
  const int l = lane();
  bool bad = false;
  for (int j0 = 0; j0 < cnt && !bad; j0 += 256) {
    int ww[4], need[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int j = j0 + l + 64 * u;
      ww[u] = j < cnt ? ent[2 * j] : -1;
      need[u] = j < cnt ? ent[2 * j + 1] : 0;
      if (ww[u] == self) ww[u] = -1;
    }
    const unsigned long long since = wall_clock64();
    for (unsigned polls = 0;; ++polls) {
      int have[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) have[u] = ww[u] >= 0 ? ld_relaxed(&S.sprogress[ww[u] * S.pstride]) : 0x7fffffff;
      bool mine = true;
#pragma unroll
      for (int u = 0; u < 4; ++u) mine = mine && have[u] >= need[u];
      if (__ballot(!mine) == 0ull) break;
      if (ld_relaxed(&S.cnt->err_code) != 0) { bad = true; break; }
      __builtin_amdgcn_s_sleep(1);
      if ((polls & 1023) == 1023 && wall_clock64() - since > S.timeout_ticks) {
        int z = 0;
        if (l == 0 && __hip_atomic_compare_exchange_strong(&S.cnt->err_code, &z, (int)KVM_ERR_TIMEOUT, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
          S.cnt->err_slot = slot; S.cnt->err_a = ww[0]; S.cnt->err_b = need[0];
        }
        bad = true;
        break;
      }
    }
  }
  return bad;
}

// The static path: worker w runs its program (the host plan) in order. Before a task, wave 0 waits for its cross-worker
// dependencies (lane k polls wait k: progress[worker] >= need) and acquires; after it, every wave waits for its own
// write-through stores and the barrier orders them before thread 0 publishes the program position, when another
// worker waits for this task. Version publications keep the dynamic path's CAS (a gap is still reported); no task
// parks, the plan orders every waiter after its publisher. A wait gives up after timeout_ticks (TIMEOUT) or when any
// worker reports an error, so every worker exits.
//
// V selects the operator bodies inlined into the worker loop (a call costs each task the callee-saved register spills
// and reloads of a large body, microseconds per task): 0 none, 1 batch-1 decode (one-row GEMV with the deep ring, the
// GQA-4 attention split), 2 batched decode (the 8-row GEMV, the GQA-4 attention split). One instantiation per set:
// each body's registers are allocated with only its set's other bodies (two GEMV ring depths in one kernel made both
// slower). The host picks V from the graph's operators.
template <int V>
__global__ __launch_bounds__(KVM_THREADS, 1) void kvm_static_kernel(KvmDevState S) {
  __shared__ __attribute__((aligned(16))) char smem[KVM_LDS_BYTES];
  __shared__ int s_go;
  __shared__ __attribute__((aligned(16))) KvmRec s_recs[2];
  const int t = threadIdx.x, w = blockIdx.x;
  const int p0 = S.sprog_off[w], p1 = S.sprog_off[w + 1];
  if (p0 < p1 && t < KVM_REC_VEC_OPS) ((LDS u32x4_t*)&s_recs[0])[t] = ((const u32x4_t*)(S.recs + S.sprog[p0]))[t];
  int next = p0 < p1 ? S.sprog[p0] : -1;
  __syncthreads();
  for (int i = p0; i < p1; ++i) {
    const int slot = next;
    KvmRec& s_rec = s_recs[(i - p0) & 1];
    // Records depend on nothing: wave 1 requests the next task's into the other buffer (direct to LDS) now; its
    // end-of-task store wait covers that load too.
    next = i + 1 < p1 ? S.sprog[i + 1] : -1;
    if (wave() == 1 && next >= 0 && lane() < KVM_REC_VEC_OPS)
      dma16(dma_rsrc(S.recs + next, sizeof(KvmRec)), 16 * lane(), 0, (const LDS void*)&s_recs[(i + 1 - p0) & 1]);
    const int sf = S.sflag[slot];
    // A decode GEMV whose weights no task writes requests its first weight steps before waiting (wave 0's share
    // lands before its first poll returns).
    Ctx c{(const LDS View*)s_rec.views, (const LDS int32_t*)s_rec.args, (LDS char*)smem, S.cnt, slot};
    if (sf & KVM_SF_PRE) {
      const int op = s_rec.desc.op_id;
      if (op == 134 || op == 301 || op == 311) gemv_prefetch(c, op);
      else attn_prefetch(c, op);
      c.pre = 1;
    }
    if (t < 64) {
      const int k0 = S.swait_off[slot], k1 = S.swait_off[slot + 1];
      const int err0 = ld_relaxed(&S.cnt->err_code);
      // the task's own list (set references skipped), then each referenced wait set (lanes of the reference
      // broadcast it in turn)
      bool bad = static_wait(S, S.sw + 2 * k0, k1 - k0, w, slot);
      for (int kb = k0; kb < k1 && !bad; kb += 64) {
        const int k = kb + t;
        unsigned long long refs = __ballot(k < k1 && S.sw[2 * k] < 0);
        while (refs && !bad) {
          const int kk = kb + __ffsll((long long)refs) - 1;
          refs &= refs - 1;
          bad = static_wait(S, S.sw + 2 * S.sw[2 * kk + 1], -1 - S.sw[2 * kk], w, slot);
        }
      }
      fence_acquire();                       // the publishers' stores are visible from here on
      if (t == 0) s_go = !bad && err0 == 0;
    }
    __syncthreads();
    if (!s_go) break;
    const MvmTaskDesc& d = s_rec.desc;
    const int pub_var = d.pub_var, pub_ver = d.pub_ver, wait_var = d.wait_var;   // s_rec is reloaded while thread 0 completes
    if (t == 0 && S.trace_on) {
      KvmTrace& tr = S.trace[slot];
      tr.start = wall_clock64();
      tr.block = w; tr.xcc = xcc_id();
      tr.ver0 = d.wait_var >= 0 ? ld_relaxed(&S.version[d.wait_var]) : -1;
      tr.exec_count += 1;
      if (d.wait_var >= 0 && tr.ver0 < d.wait_ver) {
        int z = 0;
        if (__hip_atomic_compare_exchange_strong(&S.cnt->err_code, &z, (int)KVM_ERR_WAIT_VIOLATION, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
          S.cnt->err_slot = slot;
      }
    }
    // The decode hot path's bodies are inlined here (no call: no callee-saved register spills and reloads per
    // task); every other operator goes through the dispatcher.
    const int op = d.op_id;
    // V 0 (the small fp32 training graphs): their 64x64 and 128x128 fp32 GEMM tiles inlined (tiny GPT 501 -> 484 us
    // per step; the dynamic kernel's 256x128 fp32 tile measured slower inlined, 98.4 vs 97.2 ms for GPT-355M).
    if (V == 0) {
      const int fl = op == 34 ? c.i(11) & 96 : -1;
      if (fl == 32 && f32_tile_inline<128, 128>(c)) {}
      else if (fl == 0 && f32_tile_inline<64, 64>(c)) {}
      else dispatch(op, c);
    }
    else {
      constexpr int GR = V == 1 ? 12 : 4;          // the set's GEMV ring depth
      // (the fused SwiGLU GEMV, op 311, runs through the dispatcher: inlined beside the others it made the kernel spill)
      const bool rows = op == 301, gv = (op == 134 || rows) && c.pre;
      const int gm = rows ? c.i(9) : 1, gpro = rows ? c.i(10) : c.i(9);
      if ((op == 306 || op == 310) && c.i(11) == 4 * c.i(12)) attn_part_body<4, V == 2>(c, true, op == 310);
      else if (gv && gv_pre_ring(gm) == GR && gemv_stream_ok(c.buf(0), c.buf(1), c.buf(3), c.buf(4), c.i(8), gm, gpro))
        gemv_body<GR>(c, gm, gpro, rows ? c.f(11) : c.f(10));
      else dispatch(op, c);
    }
    const bool pub_pos = (sf & KVM_SF_PUB) != 0;
    wait_stores();
    __syncthreads();
    if (t == 0) {
      if (S.trace_on) {
        KvmTrace& tr = S.trace[slot];
        tr.ver1 = wait_var >= 0 ? ld_relaxed(&S.version[wait_var]) : -1;
        tr.end = wall_clock64();
      }
      if (pub_var >= 0) publish(S, slot, pub_var, pub_ver);
      if (pub_pos) st_relaxed(&S.sprogress[w * S.pstride], i - p0 + 1);
      st_relaxed(&S.done_blk[w], i - p0 + 1);
    }
  }
  wait_stores();   // after an early exit: no direct-to-LDS load of a prefetch is still in flight when the workgroup ends
}

// Roots (tasks with no predecessors). Roots without a version wait go to fixed cells computed on the host (queue
// t % nq, in index order within the queue), written by all threads at once; the queue tails then start past them.
// Roots with a version wait are released one by one by thread 0 afterwards (they park until the version is published,
// or are enqueued behind the fixed cells when it already is).
// Instantiated here, ahead of the dynamic kernel: their place in the code object does not move with its code.
template __global__ void kvm_static_kernel<1>(KvmDevState);
template __global__ void kvm_static_kernel<2>(KvmDevState);
template __global__ void kvm_static_kernel<0>(KvmDevState);

__global__ __launch_bounds__(KVM_THREADS, 1) void kvm_exec_kernel(KvmDevState S) {
  __shared__ __attribute__((aligned(16))) char smem[KVM_LDS_BYTES];
  __shared__ int s_slot;
  // Two record buffers, alternating per task: wave 0 writes the next task's record while the other waves may still
  // read the finished task's successor edges.
  __shared__ __attribute__((aligned(16))) KvmRec s_recs[2];
  static_assert(KVM_REC_VEC <= 64, "one record piece per lane of wave 0");
  int cur = 0;
  const int t = threadIdx.x;
  int ndone = 0;              // tasks this worker finished (thread 0's count, stored after each task)
  long long held = -1;        // stream mode: thread 0's ticket, kept while it admits windows
  int how = 0;                // class mode (thread 0): start bits and virtual-time charge of the running task
  unsigned est = 0;
  unsigned long long t_start = 0;
  for (;;) {
    KvmRec& s_rec = s_recs[cur];
    MvmTaskDesc& s_desc = s_rec.desc;
    if (S.ncls) {   // class pop (-2 in stream mode: the admission lock was taken)
      if (wave() == 0) {
        const int slot = pop_cls(S, how, est);
        if (t == 0) { s_slot = slot == -2 ? -2 : ld_relaxed(&S.cnt->err_code) != 0 ? -1 : slot; t_start = wall_clock64(); }
      }
      __syncthreads();
      if (s_slot == -2) { admit_windows(S); continue; }
    } else if (S.stream) {
      if (t == 0) s_slot = stream_next(S, held);
      __syncthreads();
      if (s_slot == -2) { admit_windows(S); continue; }
    } else if (S.tq) {
      if (wave() == 0) {
        const int slot = pop_prio(S);
        if (t == 0) s_slot = ld_relaxed(&S.cnt->err_code) != 0 ? -1 : slot;
      }
    } else if (wave() == 0) {
      // FIFO mode: wave 0 takes the ticket (lane 0), polls the cell with every lane (one broadcast load), and pulls
      // the task's record into LDS itself (one 16-byte piece per lane), so one barrier hands the task to the block.
      const int q = blockIdx.x % S.nq;
      unsigned ticket = 0;
      if (t == 0) ticket = add_relaxed(&S.queues[q].head, 1u);
      ticket = __builtin_amdgcn_readfirstlane(ticket);
      int slot = -1;
      if (ticket < (unsigned)S.qcount[q]) {
        unsigned long long since = wall_clock64();
        int seen = -1, err = 0;
        for (unsigned polls = 0;; ++polls) {
          slot = __builtin_amdgcn_readfirstlane(ld_relaxed(&S.ready[q * S.qcap + ticket]));   // cell and error word in flight together
          err = __builtin_amdgcn_readfirstlane(ld_relaxed(&S.cnt->err_code));
          if (slot >= 0 || err != 0) break;
          __builtin_amdgcn_s_sleep(1);
          if ((polls & 4095) == 4095) {
            int st = 0;
            if (t == 0) st = stalled(S, since, seen, (int)ticket);
            if (__builtin_amdgcn_readfirstlane(st)) break;
          }
        }
        if (slot >= 0) fence_acquire();   // the enqueuer's release: predecessors' data is visible from here on
        if (err != 0) slot = -1;
      }
      if (slot >= 0 && t < KVM_REC_VEC) ((LDS u32x4_t*)&s_rec)[t] = ((const u32x4_t*)(S.recs + slot))[t];
      if (t == 0) s_slot = slot;
    }
    __syncthreads();
    const int slot = s_slot;
    if (slot < 0) break;
    if (S.stream || S.ncls || S.tq) {   // the other pop paths hand over only the slot: the record is loaded here
      if (t < KVM_REC_VEC) ((LDS u32x4_t*)&s_rec)[t] = ((const u32x4_t*)(S.recs + slot))[t];   // the whole record, one load per thread
      __syncthreads();
    }
    const int op = s_desc.op_id;
    if (t == 0 && S.trace_on) {
      KvmTrace& tr = S.trace[slot];
      tr.start = wall_clock64();
      tr.block = blockIdx.x; tr.xcc = xcc_id();
      tr.ver0 = s_desc.wait_var >= 0 ? ld_relaxed(&S.version[s_desc.wait_var]) : -1;
      tr.exec_count += 1;
      if (tr.exec_count > 1) {
        int z = 0;
        if (__hip_atomic_compare_exchange_strong(&S.cnt->err_code, &z, (int)KVM_ERR_DOUBLE_EXEC, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
          S.cnt->err_slot = slot;
      }
      if (s_desc.wait_var >= 0 && tr.ver0 < s_desc.wait_ver) {
        int z = 0;
        if (__hip_atomic_compare_exchange_strong(&S.cnt->err_code, &z, (int)KVM_ERR_WAIT_VIOLATION, __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
          S.cnt->err_slot = slot;
      }
    }
    Ctx c{(const LDS View*)s_rec.views, (const LDS int32_t*)s_rec.args, (LDS char*)smem, S.cnt, slot};
    // The 128x256 and 128x128 bf16 GEMM tiles (ops 122, 308, 114: most of a GPT step's tiles) run inlined here.
    // Called out of line, a body saves and restores the callee-saved registers it uses around every task (GPT-162M
    // 9.38 -> 9.15 ms with ops 122 / 308 inlined, 9.07 with op 114's 128x128 tiles too). The 256x256 tile (the
    // compiler fails on it inlined here) and the attention bodies (inlined, they push the kernel's private segment
    // past KVM_MAX_PRIVATE_BYTES) stay out of line.
    if ((op == 122 || op == 308) && gemm_tile_inline<128, 256>(c)) { if (op == 308) mma_delta_tail(c); } else
    if (op == 114 && (c.i(11) & 96) == 32 && gemm_tile_inline<128, 128>(c)) {} else
    dispatch(op, c);
    // Every operator stores through write-through (agent-scope) stores only, which tests/test_wt_stores.py checks
    // in the compiled code: once each wave has waited for its own stores, they are agent-visible, and the barrier
    // orders that before wave 0 signals successors. No release fence, so no L2 write-back per task.
    wait_stores();
    __syncthreads();
    // Completion. The task's stores are agent-visible (above). The first successor edges come from the record (in
    // LDS since dispatch), the rest from the successor array. Edges carry host-computed bits: KVM_EDGE_DIRECT means
    // the successor has this task as its only predecessor and no version wait, so it is released with no counter;
    // KVM_EDGE_NOWAIT that it has no version wait, so the decrement that reaches zero enqueues it with no descriptor
    // read. Other successors count down with a relaxed atomic; the decrement that reaches zero
    // acquires (fence) before releasing the task. Released tasks are enqueued in batches: per wave and per queue one
    // tail reservation (issued by lanes 0..nq-1 in parallel) and one relaxed cell store per task.
    const int nsucc = s_desc.succ_cnt;
    const int nwaves = nsucc > 64 ? KVM_WAVES : 1;
    if (wave() < nwaves) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      if (t == 0) {
        if (S.trace_on) {
          KvmTrace& tr = S.trace[slot];
          tr.ver1 = s_desc.wait_var >= 0 ? ld_relaxed(&S.version[s_desc.wait_var]) : -1;
          tr.end = wall_clock64();
        }
        if (s_desc.pub_var >= 0) publish(S, slot, s_desc.pub_var, s_desc.pub_ver);
      }
      const int l = lane();
      for (int base = wave() * 64; base < nsucc; base += nwaves * 64) {
        const int k = base + l;
        int s = -1; bool direct = false;
        if (k < nsucc) {
          const int e = k < s_rec.nsucc_rec ? s_rec.succ[k] : S.succ[s_desc.succ_off + k];
          s = e & KVM_EDGE_INDEX;
          if (e & KVM_EDGE_DIRECT) direct = true;
          else if (add_relaxed(&S.indeg[s], -1) == 1) {
            // Every predecessor made its stores agent-visible before its decrement, and the task that dequeues the
            // successor acquires (L1 / L2 invalidate) before reading them, so the plain enqueue needs no fence here;
            // the versioned path keeps its acquire-release.
            if (e & KVM_EDGE_NOWAIT) direct = true;
            else { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "agent"); release(S, s); }
          }
        }
        if (S.tq) {   // priority mode: lanes bound for the same queue share one tail reservation, in lane order
          const int myq = direct ? S.tq[s] : -1;
          if (direct) {
            st_relaxed(&S.state[s], 2);
            if (S.ready_ts) __hip_atomic_store(&S.ready_ts[s], wall_clock64(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (S.aff) note_ready(S, s, true);
          }
          unsigned long long todo = __ballot(direct);
          while (todo) {
            const int lead = __ffsll((long long)todo) - 1;
            const int q = __shfl(myq, lead, 64);
            const unsigned long long m = __ballot(direct && myq == q);
            int base_q = 0;
            if (l == lead) base_q = add_relaxed(&S.queues[q].tail, __popcll(m));
            base_q = __shfl(base_q, lead, 64);
            if (direct && myq == q) {
              const int pos = base_q + __popcll(m & ((1ull << l) - 1ull));
              if (pos >= S.qcount[q]) queue_overflow(S);
              else if (S.ready_ts || S.aff) st_release(&S.ready[S.qoff[q] + pos], s);   // release time / affinity before the cell
              else st_relaxed(&S.ready[S.qoff[q] + pos], s);
            }
            todo &= ~m;
          }
          continue;
        }
        const int sq = direct ? s % S.nq : -1;
        if (S.stream) {   // stream mode: one tail reservation per task, the cell stamped with its round
          if (direct) {
            const int r = ring_of(S, s);
            st_relaxed(&S.state[s], 2);
            if (S.aff) note_ready(S, s, true);
            put_cell64(S, r, (unsigned)add_relaxed(&S.queues[r].tail, 1), s, S.aff != nullptr);
          }
          continue;
        }
        int cnt_mine = 0;            // lane q < nq: how many of this round's tasks go to queue q
        for (int q = 0; q < S.nq; ++q) {
          const int c2 = __popcll(__ballot(sq == q));
          if (l == q) cnt_mine = c2;
        }
        int pos_mine = 0;
        if (l < S.nq && cnt_mine > 0) pos_mine = add_relaxed(&S.queues[l].tail, cnt_mine);
        // rank of this lane among the lanes bound for the same queue
        int rank = 0;
        for (int q = 0; q < S.nq; ++q) {
          const unsigned long long m2 = __ballot(sq == q);
          if (sq == q) rank = __popcll(m2 & ((1ull << l) - 1ull));
        }
        const int base_pos = __shfl(pos_mine, sq < 0 ? 0 : sq, 64);
        if (direct) {
          const int pos = base_pos + rank;
          if (pos < S.qcap) { st_relaxed(&S.state[s], 2); st_relaxed(&S.ready[sq * S.qcap + pos], s); }
          else queue_overflow(S);
        }
      }
    }
    if (t == 0) {
      if (S.ncls) {
        const int bits = cls_done(S, s_desc, slot, how, est, t_start);
        if (S.trace_on) S.trace[slot].how = bits;
      }
      st_relaxed(&S.done_blk[blockIdx.x], ++ndone);
      if (S.stream) {   // the slot's window: its last task marks it complete in host memory (the host may reuse it)
        const int w = slot / S.wtasks;
        if (add_acqrel(&S.win_left[w], -1) == 1) st_sys64(&S.hctl->done_mark[w], (long long)ld_relaxed(&S.win_seq[w]) + 1);
      }
    }
    cur ^= 1;
  }
}

// Launch-time state reset: counters, queue cells, park lists, versions; roots without a version wait go straight
// into the first queue cells in index order, roots with one go through release().
__global__ void kvm_reset_kernel(KvmDevState S, const int* base_versions) {
  int i = blockIdx.x * blockDim.x + threadIdx.x, stride = gridDim.x * blockDim.x;
  for (int k = i; k < S.ntasks; k += stride) {
    S.indeg[k] = S.tasks[k].indegree; S.state[k] = 0; S.park_next[k] = -1;
    if (S.trace_on) { KvmTrace z = {}; z.ver0 = z.ver1 = -1; S.trace[k] = z; }
  }
  for (long long k = i; k < (long long)S.ncells; k += stride) S.ready[k] = -1;
  for (int k = i; k < S.nvars; k += stride) { S.version[k] = base_versions[k]; S.park_head[k] = -1; }
  for (int k = i; k < S.grid; k += stride) { S.done_blk[k] = 0; if (S.sprogress) S.sprogress[k * S.pstride] = 0; }
  for (int k = i; k < S.nq * S.nb * (S.ncls ? S.ncls : 1); k += stride) { KvmQueue z = {}; S.queues[k] = z; }
  if (i == 0) { KvmCounters z = {}; *S.cnt = z; }
  if (S.ncls && i < S.ncls) {   // class hot and statistics lines; the parameter line stays as uploaded
    KvmClsDev& k = S.sched->cls[i];
    k.running = 0; k.bw_running = 0; k.vtime = 0; k.est = 200;   // 2 us until measured
    k.tasks = k.busy = k.resv_starts = k.urgent_starts = k.missed = k.boost_starts = 0; k.max_running = 0;
  }
  if (S.pv) for (int k = i; k < S.nvars * KVM_MAX_CLASSES; k += stride) S.pv[k] = 0;
  if (S.op_blk) for (int k = i; k < KVM_OP_SLOTS; k += stride) S.op_blk[k] = -1;
  if (S.ncls && i == 0) { S.sched->t0 = wall_clock64(); S.sched->boost = 0; S.sched->bw_total = 0; }
  if (S.stream) {
    for (long long k = i; k < (long long)S.nq * (S.ncls ? S.ncls : 1) * S.qcap; k += stride) S.ready64[k] = 0ull;
    for (int k = i; k < S.wcap; k += stride) { S.win_left[k] = 0; S.win_seq[k] = -1; S.win_t0[k] = 0ull; }
    if (S.ncls) for (int k = i; k < S.nvars; k += stride) S.pubcls[k] = 0;
    if (i == 0) { KvmAdm z = {}; *S.adm = z; }
  }
}
__global__ void kvm_seed_kernel(KvmDevState S, const int* roots, const int* root_cell, int nfixed, int nroots, const int* fixed_tail) {
  for (int r = threadIdx.x; r < nfixed; r += blockDim.x) {
    const int t = roots[r];
    if (S.ready_ts) S.ready_ts[t] = wall_clock64();
    if (S.aff) S.aff[t] = 0ull;   // no preferred worker
    S.ready[root_cell[r]] = t;
    S.state[t] = 2;
  }
  for (int q = threadIdx.x; q < S.nq * S.nb * (S.ncls ? S.ncls : 1); q += blockDim.x) S.queues[q].tail = fixed_tail[q];
  __syncthreads();
  if (threadIdx.x == 0)
    for (int r = nfixed; r < nroots; ++r) release(S, roots[r], false);
}

// ---------------------------------------------------------------------------------------------- init kernels
__device__ __forceinline__ float seeded_u(unsigned long long seed, unsigned long long j) {
  unsigned long long z = seed + (j + 1ull) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (float)(z >> 40) * (1.0f / 16777216.0f);
}
// SplitMix64 counter-based initialiser, one correctly rounded f32 operation per step (runtime/initgen.py:1-58).
__global__ void kvm_seeded_kernel(float* out, long long n, unsigned long long seed, int draws, float bias, float coef) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    float acc;
    if (draws == 1) acc = seeded_u(seed, i);
    else {
      unsigned long long j = (unsigned long long)i * 4ull;
      acc = __fadd_rn(__fadd_rn(seeded_u(seed, j), seeded_u(seed, j + 1)), __fadd_rn(seeded_u(seed, j + 2), seeded_u(seed, j + 3)));
    }
    out[i] = __fmul_rn(__fsub_rn(acc, bias), coef);
  }
}
// The same generator rounded once to bf16 storage (this executor's extension for bf16 weights; the bundle format
// keeps `seeded` for f32 buffers only).
__global__ void kvm_seeded_bf16_kernel(uint16_t* out, long long n, unsigned long long seed, int draws, float bias, float coef) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) {
    float acc;
    if (draws == 1) acc = seeded_u(seed, i);
    else {
      unsigned long long j = (unsigned long long)i * 4ull;
      acc = __fadd_rn(__fadd_rn(seeded_u(seed, j), seeded_u(seed, j + 1)), __fadd_rn(seeded_u(seed, j + 2), seeded_u(seed, j + 3)));
    }
    out[i] = f2bf(__fmul_rn(__fsub_rn(acc, bias), coef));
  }
}
__global__ void kvm_fill32_kernel(uint32_t* out, long long n, uint32_t v) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) out[i] = v;
}
__global__ void kvm_fill16_kernel(uint16_t* out, long long n, uint16_t v) {
  for (long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x) out[i] = v;
}

// ---------------------------------------------------------------------------------------------- host executor
static thread_local std::string g_err;

struct BufRec { void* p; int rows, cols, dtype; size_t bytes; };

// What a launch needs besides the device state: base versions to copy in and the root lists of the seed kernel.
struct LaunchArgs { int* base; const int* roots; const int* root_cell; const int* fixed_tail; int nfixed, nroots; };

struct KvmExec {
  KvmConfig cfg;
  int dev = 0, cus = 0, grid = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  std::vector<BufRec> bufs;
  std::vector<MvmTaskDesc> tasks;
  std::vector<int32_t> succ, args, roots;
  std::vector<int> base_versions;
  bool uploaded = false, launched = false;
  std::string err;
  // device memory of the placed graph (one hipMalloc each, freed by kvm_destroy)
  std::vector<void*> allocs;
  int path = -1;                           // the path launches use: KVM_PATH_DYNAMIC or KVM_PATH_STATIC (set at upload)
  // Static plans: splan keeps every task (traced launches: the trace is indexed by task); splan_d dissolves the
  // ordering no-ops (untraced launches). Their device arrays: sfull, sdis (the same arrays when nothing dissolves).
  kvms::Plan splan, splan_d;
  struct StaticDev { const int *prog_off = nullptr, *prog = nullptr, *wait_off = nullptr, *sw = nullptr, *flag = nullptr; int dissolved = 0; };
  StaticDev sfull, sdis;
  int last_dissolved = 0;                  // no-ops the last launch dissolved (counted as done)
  int trace_req = 1;                       // kvm_set_trace's last request (launches trace when the buffer exists and this is set)
  // stream mode
  bool streaming = false, closed = false;
  KvmHostCtl* hctl = nullptr;              // pinned control block (host address)
  int* hver = nullptr;                     // pinned mirror of the version variables (host address)
  char* hwin = nullptr;                    // pinned window staging (host address)
  long long seq = 0, stream_tasks = 0;     // windows and tasks submitted
  struct Pending { std::vector<MvmTaskDesc> t; std::vector<int32_t> s, a; };
  std::vector<Pending> pending;            // bundles submitted before kvm_start
  struct LaunchArgs L{};
  KvmDevState S{};
  // scheduler classes (kvm_set_classes, kvm_set_sched_flags)
  int sched_mode = KVM_SCHED_GLOBAL;
  std::vector<KvmClassParams> classes;
  int sched_flags = KVM_SCHED_F_GUARANTEE | KVM_SCHED_F_INHERIT, bw_limit = KVM_UNLIMITED;
  int affinity_us = 0;
};

#define HIPCK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { ex->err = std::string(#x) + ": " + hipGetErrorString(e_); return KVM_STATUS_HIP_ERROR; } } while (0)

static size_t elem_bytes(int dtype) { return dtype == 2 ? 2 : 4; }

// ---------------------------------------------------------------------------------------------- graph layout
// The host-side layout of one launch's task graph: dispatch records, device successor edges, ready-queue geometry
// (FIFO or priority buckets), root cells. Computed once per graph; placed into device memory by place_graph.
struct GraphPlan {
  int n = 0, nq = 1, qcap = 1, nb = 1, nqb = 1, ncells = 1, nfixed = 0;
  bool prio_mode = false;
  std::vector<int32_t> succ_dev;
  std::vector<KvmRec> recs;
  std::vector<int> qcount, qoff, tq, prios, roots, root_cell, fixed_tail;
};

// Buffer-argument positions of every registry operator (bit k: argument k is a buffer).
static const unsigned* op_buf_mask() {
  static unsigned m[KVM_OPMASK_IDS] = {};
  static bool done = false;
  if (!done) {
    for (const kvmv::OpSig& o : kvmv::kRegistry) {
      if (o.id < 0 || o.id >= KVM_OPMASK_IDS) continue;
      std::vector<kvmv::ArgInfo> a = kvmv::parse_sig(o.sig);
      for (size_t k = 0; k < a.size() && k < 32; ++k) if (a[k].type == 0) m[o.id] |= 1u << k;
    }
    done = true;
  }
  return m;
}
// A task's dispatch record: descriptor, argument words and the views of its buffer arguments.
static int32_t edge_flags(const MvmTaskDesc& d) {
  return d.wait_var < 0 ? (KVM_EDGE_NOWAIT | (d.indegree == 1 ? KVM_EDGE_DIRECT : 0)) : 0;
}
static void make_rec(const MvmTaskDesc& d, const int32_t* a, const std::vector<MvmBuf>& table, KvmRec& r) {
  std::memset(&r, 0, sizeof(r));
  r.desc = d;
  const unsigned mask = (unsigned)d.op_id < KVM_OPMASK_IDS ? op_buf_mask()[d.op_id] : 0u;
  for (int k = 0; k < d.args_words && k < KVM_MAX_ARGS; ++k) {
    const int w = a[k];
    r.args[k] = w;
    if (w >= 0 && ((mask >> k) & 1u)) r.views[k] = View{table[w].p, table[w].rows, table[w].cols, table[w].dtype};
  }
}

// ncls > 0: scheduler classes, the buckets split per class (task t's class is its workload_id); one_group: a single
// queue group (the class-partitioned mode, whose workers of one class must all see its buckets).
static void plan_graph(const std::vector<MvmTaskDesc>& tasks, const std::vector<int32_t>& succ, const std::vector<int32_t>& args,
                       const std::vector<MvmBuf>& table, const std::vector<int32_t>& roots, int grid, int aging_us, GraphPlan& g,
                       int ncls = 0, bool one_group = false) {
  const int n = (int)tasks.size();
  g.n = n;
  g.succ_dev = succ;
  for (auto& e : g.succ_dev) e |= edge_flags(tasks[e]);
  g.recs.assign(n, KvmRec{});
  for (int i = 0; i < n; ++i) {
    KvmRec& r = g.recs[i];
    make_rec(tasks[i], args.data() + tasks[i].args_off, table, r);
    r.nsucc_rec = std::min(tasks[i].succ_cnt, KVM_REC_SUCC);
    for (int k = 0; k < r.nsucc_rec; ++k) r.succ[k] = g.succ_dev[tasks[i].succ_off + k];
  }
  g.nq = one_group ? 1 : std::max(1, std::min(KVM_MAX_QUEUES, grid));
  g.qcap = (n + g.nq - 1) / g.nq;
  // Priority buckets: one per distinct priority in the graph, bucket 0 the highest. A graph with one priority and no
  // aging runs in FIFO mode (queue t % nq, fetch-add tickets); otherwise task t goes to queue (t % nq) * nb + bucket.
  g.prios.clear();
  for (const MvmTaskDesc& d : tasks) g.prios.push_back(d.priority);
  std::sort(g.prios.begin(), g.prios.end(), [](int a, int b) { return a > b; });
  g.prios.erase(std::unique(g.prios.begin(), g.prios.end()), g.prios.end());
  g.prio_mode = g.prios.size() > 1 || aging_us > 0 || ncls > 0;
  g.nb = g.prio_mode ? (int)g.prios.size() : 1;
  const int nc = ncls > 0 ? ncls : 1;
  g.nqb = g.nq * nc * g.nb;
  g.qcount.assign(g.nqb, 0); g.qoff.assign(g.nqb, 0); g.tq.clear();
  if (g.prio_mode) {
    int bucket_of[KVM_PRIORITIES];
    for (int b = 0; b < g.nb; ++b) bucket_of[g.prios[b]] = b;
    g.tq.resize(n);
    for (int t = 0; t < n; ++t) {
      const int c = ncls > 0 ? tasks[t].workload_id : 0;
      g.tq[t] = ((t % g.nq) * nc + c) * g.nb + bucket_of[tasks[t].priority];
      ++g.qcount[g.tq[t]];
    }
    for (int q = 1; q < g.nqb; ++q) g.qoff[q] = g.qoff[q - 1] + g.qcount[q - 1];
  } else {
    for (int t = 0; t < n; ++t) ++g.qcount[t % g.nq];
    for (int q = 0; q < g.nq; ++q) g.qoff[q] = q * g.qcap;
  }
  g.ncells = g.prio_mode ? n : g.nq * g.qcap;
  // roots: those without a version wait first (fixed ready cells, index order per queue), then those with one
  g.roots.clear(); g.root_cell.clear(); g.fixed_tail.assign(g.nqb, 0);
  std::vector<int> waiting;
  for (int t : roots) {
    if (tasks[t].wait_var < 0) {
      const int q = g.prio_mode ? g.tq[t] : t % g.nq;
      g.roots.push_back(t); g.root_cell.push_back(g.qoff[q] + g.fixed_tail[q]++);
    } else waiting.push_back(t);
  }
  g.nfixed = (int)g.roots.size();
  g.roots.insert(g.roots.end(), waiting.begin(), waiting.end());
}

// Places a planned graph into device memory obtained from `alloc(bytes)` (256-byte aligned, nullptr on failure),
// copies the host arrays in on `st` and waits for the copies; fills the device state and the launch arguments.
// With copy = false nothing is copied (a sizing pass over a counting allocator).
template <class Alloc>
static int place_graph(const GraphPlan& g, const std::vector<MvmTaskDesc>& tasks, int nv, int grid, bool trace, int aging_us,
                       unsigned long long timeout_us, Alloc&& alloc, hipStream_t st, KvmDevState& S, LaunchArgs& L, std::string& err,
                       bool copy = true) {
  hipError_t e = hipSuccess;
  auto put = [&](const void* host, size_t bytes) -> void* {
    void* d = alloc(std::max<size_t>(bytes, 4));
    if (!d) { if (err.empty()) err = "device memory for the task graph"; return nullptr; }
    if (copy && host && bytes && e == hipSuccess) e = hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, st);
    return d;
  };
  auto vec = [&](const auto& v) { return put(v.data(), v.size() * sizeof(v[0])); };
  const int n = g.n;
  S = KvmDevState{};
  S.recs = (const KvmRec*)vec(g.recs);
  S.tasks = (const MvmTaskDesc*)vec(tasks);
  S.succ = (const int32_t*)vec(g.succ_dev);
  S.indeg = (int*)put(nullptr, n * sizeof(int));
  S.ready = (int*)put(nullptr, (size_t)g.ncells * sizeof(int));
  S.queues = (KvmQueue*)put(nullptr, g.nqb * sizeof(KvmQueue));
  S.qcount = (const int*)vec(g.qcount);
  S.qoff = (const int*)vec(g.qoff);
  if (g.prio_mode) {
    S.tq = (const int*)vec(g.tq);
    S.bucket_prio = (const int*)vec(g.prios);
    if (aging_us > 0) S.ready_ts = (unsigned long long*)put(nullptr, n * sizeof(unsigned long long));
  }
  S.done_blk = (int*)put(nullptr, grid * sizeof(int));
  S.state = (int*)put(nullptr, n * sizeof(int));
  S.park_next = (int*)put(nullptr, n * sizeof(int));
  S.version = (int*)put(nullptr, nv * sizeof(int));
  S.park_head = (int*)put(nullptr, nv * sizeof(int));
  S.cnt = (KvmCounters*)put(nullptr, sizeof(KvmCounters));
  if (trace) S.trace = (KvmTrace*)put(nullptr, n * sizeof(KvmTrace));
  L.base = (int*)put(nullptr, nv * sizeof(int));
  L.roots = (const int*)vec(g.roots);
  L.root_cell = (const int*)vec(g.root_cell);
  L.fixed_tail = (const int*)vec(g.fixed_tail);
  L.nfixed = g.nfixed; L.nroots = (int)g.roots.size();
  if (!err.empty()) return KVM_STATUS_TOO_BIG;
  if (copy && e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) { err = std::string("graph upload: ") + hipGetErrorString(e); return KVM_STATUS_HIP_ERROR; }
  S.ntasks = n; S.nvars = nv; S.trace_on = trace ? 1 : 0;
  S.nq = g.nq; S.qcap = g.qcap; S.grid = grid; S.ncells = g.ncells; S.nb = g.nb;
  S.aging_ticks = aging_us > 0 ? (unsigned long long)aging_us * 100ull : 0ull;
  S.timeout_ticks = timeout_us * 100ull;   // wall_clock64 runs at 100 MHz on gfx950
  return 0;
}

// Every worker of a persistent kernel must be resident at once (a worker that never starts leaves its queue's tasks
// unrun and the others waiting): the grid is at most what the occupancy calculator admits per CU times the CUs.
// The workers' private segments (callee-saved registers of the operator calls) are backed by scratch for every
// resident wave; a kernel build whose segment grew to 2,096 bytes per lane stopped before its first task finished,
// while 1,328 runs, so builds above KVM_MAX_PRIVATE_BYTES per lane are refused rather than launched. Returns the
// co-resident worker capacity of the device, or -1 with the reason in err.
// The current device is the one asked about.
static int resident_capacity(int cus, std::string& err) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kvm_exec_kernel, KVM_THREADS, 0) != hipSuccess || per_cu < 1) {
    err = "the executor kernel does not fit on a CU (occupancy query)"; return -1;
  }
  for (const void* k : {(const void*)kvm_exec_kernel, (const void*)kvm_static_kernel<0>, (const void*)kvm_static_kernel<1>,
                        (const void*)kvm_static_kernel<2>}) {
    hipFuncAttributes fa{};
    if (hipFuncGetAttributes(&fa, k) != hipSuccess) { err = "hipFuncGetAttributes failed"; return -1; }
    if (fa.localSizeBytes > KVM_MAX_PRIVATE_BYTES) {
      err = "the executor kernel's private segment (" + std::to_string(fa.localSizeBytes) + " bytes per lane) exceeds " +
            std::to_string(KVM_MAX_PRIVATE_BYTES) + ": refusing a build whose workers may not all be resident";
      return -1;
    }
  }
  return per_cu * cus;
}

extern "C" {

void kvm_config_default(KvmConfig* c) {
  c->blocks = 0; c->trace_on = 1; c->num_vars = 64; c->timeout_us = 20ull * 1000000ull; c->device = 0; c->aging_us = 0;
  c->path = KVM_PATH_DYNAMIC;
  c->window_cap = 0; c->window_tasks = 0; c->window_edges = 0; c->backpressure_ms = 60000;
}

const char* kvm_last_error(const KvmExec* ex) { return ex ? ex->err.c_str() : g_err.c_str(); }

KvmExec* kvm_create(const KvmConfig* cfg) {
  KvmConfig c; kvm_config_default(&c);
  if (cfg) c = *cfg;
  if (c.num_vars < 1 || c.num_vars > (1 << 20)) { g_err = "num_vars out of range"; return nullptr; }
  if (c.aging_us < 0) { g_err = "aging_us must be >= 0"; return nullptr; }
  if (c.path < KVM_PATH_DYNAMIC || c.path > KVM_PATH_AUTO) { g_err = "path must be KVM_PATH_DYNAMIC, KVM_PATH_STATIC or KVM_PATH_AUTO"; return nullptr; }
  if (c.window_cap < 0 || c.window_cap > (1 << 16)) { g_err = "window_cap out of range"; return nullptr; }
  if (c.window_cap > 0) {
    if (c.window_tasks < 1 || c.window_edges < 0 || (long long)c.window_cap * c.window_tasks > (1ll << 26) ||
        (long long)c.window_cap * c.window_edges > (1ll << 28)) { g_err = "stream mode: window_tasks / window_edges out of range"; return nullptr; }
    if (c.path == KVM_PATH_STATIC) { g_err = "stream mode runs the dynamic path (a static plan needs the whole graph)"; return nullptr; }
    if (c.aging_us != 0) { g_err = "stream mode schedules FIFO: aging_us must be 0"; return nullptr; }
    if (c.backpressure_ms < 0) { g_err = "backpressure_ms must be >= 0"; return nullptr; }
  }
  if (hipSetDevice(c.device) != hipSuccess) { g_err = "hipSetDevice failed"; return nullptr; }
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, c.device) != hipSuccess) { g_err = "hipGetDeviceProperties failed"; return nullptr; }
  const int capacity = resident_capacity(p.multiProcessorCount, g_err);
  if (capacity < 0) return nullptr;
  if (c.blocks < 0 || c.blocks > capacity) {
    g_err = "blocks exceeds the co-resident capacity of the device (" + std::to_string(capacity) + ")"; return nullptr;
  }
  KvmExec* ex = new KvmExec();
  ex->cfg = c; ex->dev = c.device; ex->cus = p.multiProcessorCount;
  ex->grid = c.blocks > 0 ? c.blocks : ex->cus;
  ex->base_versions.assign(c.num_vars, 0);
  ex->streaming = c.window_cap > 0;
  if (hipStreamCreateWithFlags(&ex->stream, hipStreamNonBlocking) != hipSuccess || hipEventCreate(&ex->ev0) != hipSuccess ||
      hipEventCreate(&ex->ev1) != hipSuccess) { g_err = "stream/event creation failed"; delete ex; return nullptr; }
  return ex;
}

void kvm_destroy(KvmExec* ex) {
  if (!ex) return;
  hipSetDevice(ex->dev);
  if (ex->streaming && ex->hctl && !ex->closed) kvm_close(ex);   // the kernel ends once the admitted tasks finish
  if (ex->stream) hipStreamSynchronize(ex->stream);
  for (auto& b : ex->bufs) hipFree(b.p);
  for (void* q : ex->allocs) hipFree(q);
  if (ex->hctl) hipHostFree(ex->hctl);
  if (ex->hwin) hipHostFree(ex->hwin);
  if (ex->hver) hipHostFree(ex->hver);
  if (ex->ev0) hipEventDestroy(ex->ev0);
  if (ex->ev1) hipEventDestroy(ex->ev1);
  if (ex->stream) hipStreamDestroy(ex->stream);
  delete ex;
}

static void launch_fill(KvmExec* ex, BufRec& b, float value) {
  long long n = (long long)b.rows * b.cols;
  int grid = (int)std::min<long long>(4096, (n + 255) / 256);
  if (b.dtype == 2) {
    uint32_t u; memcpy(&u, &value, 4);
    uint32_t r = ((u & 0x7f800000u) == 0x7f800000u) ? (u >> 16) : ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    hipLaunchKernelGGL(kvm_fill16_kernel, dim3(grid), dim3(256), 0, ex->stream, (uint16_t*)b.p, n, (uint16_t)r);
  } else {
    uint32_t u;
    if (b.dtype == 1) { int32_t iv = (int32_t)value; memcpy(&u, &iv, 4); } else memcpy(&u, &value, 4);
    hipLaunchKernelGGL(kvm_fill32_kernel, dim3(grid), dim3(256), 0, ex->stream, (uint32_t*)b.p, n, u);
  }
}

int kvm_add_buffer(KvmExec* ex, int rows, int cols, int dtype, const KvmInit* init) {
  if (rows < 1 || cols < 1 || (long long)rows * cols > 0x7fffffffll || dtype < 0 || dtype > 2) { ex->err = "bad buffer shape or dtype"; return KVM_STATUS_INVALID; }
  if (ex->uploaded) { ex->err = "buffers must be added before kvm_start"; return KVM_STATUS_INVALID; }
  hipSetDevice(ex->dev);
  BufRec b{nullptr, rows, cols, dtype, (size_t)rows * cols * elem_bytes(dtype)};
  HIPCK(hipMalloc(&b.p, (b.bytes + 255) & ~(size_t)255));
  KvmInit z{}; if (!init) init = &z;
  switch (init->kind) {
    case KVM_INIT_ZERO: HIPCK(hipMemsetAsync(b.p, 0, b.bytes, ex->stream)); break;
    case KVM_INIT_FILL: launch_fill(ex, b, init->value); break;
    case KVM_INIT_VALUES: HIPCK(hipMemcpyAsync(b.p, init->values, b.bytes, hipMemcpyHostToDevice, ex->stream)); HIPCK(hipStreamSynchronize(ex->stream)); break;
    case KVM_INIT_SEEDED:
      if (dtype == 1) { hipFree(b.p); ex->err = "seeded init needs an f32 or bf16 buffer"; return KVM_STATUS_INVALID; }
      if (dtype == 2)
        hipLaunchKernelGGL(kvm_seeded_bf16_kernel, dim3(8192), dim3(256), 0, ex->stream, (uint16_t*)b.p, (long long)rows * cols, init->seed, init->draws, init->bias, init->coef);
      else
        hipLaunchKernelGGL(kvm_seeded_kernel, dim3(8192), dim3(256), 0, ex->stream, (float*)b.p, (long long)rows * cols, init->seed, init->draws, init->bias, init->coef);
      break;
    default: hipFree(b.p); ex->err = "unknown init kind"; return KVM_STATUS_INVALID;
  }
  HIPCK(hipGetLastError());
  ex->bufs.push_back(b);
  return (int)ex->bufs.size() - 1;
}

int kvm_nbufs(const KvmExec* ex) { return (int)ex->bufs.size(); }
int kvm_buffer_dtype(const KvmExec* ex, int idx) { return idx >= 0 && idx < (int)ex->bufs.size() ? ex->bufs[idx].dtype : KVM_STATUS_INVALID; }
void* kvm_buffer_device_ptr(const KvmExec* ex, int idx) { return idx >= 0 && idx < (int)ex->bufs.size() ? ex->bufs[idx].p : nullptr; }

int kvm_write_buffer(KvmExec* ex, int idx, const void* host, size_t bytes) {
  if (idx < 0 || idx >= (int)ex->bufs.size() || bytes != ex->bufs[idx].bytes) { ex->err = "kvm_write_buffer: bad index or size"; return KVM_STATUS_INVALID; }
  hipSetDevice(ex->dev);
  HIPCK(hipStreamSynchronize(ex->stream));
  HIPCK(hipMemcpy(ex->bufs[idx].p, host, bytes, hipMemcpyHostToDevice));
  return 0;
}

int kvm_read_raw(KvmExec* ex, int idx, void* out, size_t bytes) {
  if (idx < 0 || idx >= (int)ex->bufs.size() || bytes != ex->bufs[idx].bytes) { ex->err = "kvm_read_raw: bad index or size"; return KVM_STATUS_INVALID; }
  hipSetDevice(ex->dev);
  HIPCK(hipStreamSynchronize(ex->stream));
  HIPCK(hipMemcpy(out, ex->bufs[idx].p, bytes, hipMemcpyDeviceToHost));
  return 0;
}

int kvm_read_buffer(KvmExec* ex, int idx, float* out, size_t n) {
  if (idx < 0 || idx >= (int)ex->bufs.size() || n != (size_t)ex->bufs[idx].rows * ex->bufs[idx].cols) { ex->err = "kvm_read_buffer: bad index or size"; return KVM_STATUS_INVALID; }
  const BufRec& b = ex->bufs[idx];
  if (b.dtype != 2) return kvm_read_raw(ex, idx, out, b.bytes);
  std::vector<uint16_t> h(n);
  int rc = kvm_read_raw(ex, idx, h.data(), b.bytes);
  if (rc) return rc;
  for (size_t i = 0; i < n; ++i) { uint32_t u = (uint32_t)h[i] << 16; memcpy(&out[i], &u, 4); }
  return 0;
}

int kvm_set_version(KvmExec* ex, int var, int version) {
  if (var < 0 || var >= (int)ex->base_versions.size() || version < 0) { ex->err = "kvm_set_version: bad variable or version"; return KVM_STATUS_INVALID; }
  ex->base_versions[var] = version;
  return 0;
}

// ---------------------------------------------------------------------------------------------- stream mode (host)
static std::vector<MvmBuf> buf_table(const KvmExec* ex) {
  std::vector<MvmBuf> table(ex->bufs.size());
  for (size_t i = 0; i < table.size(); ++i) table[i] = MvmBuf{ex->bufs[i].p, ex->bufs[i].rows, ex->bufs[i].cols, ex->bufs[i].cols, ex->bufs[i].dtype, {0, 0}};
  return table;
}

static int upload_classes(KvmExec* ex, const std::function<void*(size_t)>& alloc, const unsigned char* has_dl, const unsigned char* has_bw,
                          const std::vector<int>& pubcls, const std::vector<unsigned char>& tbw, bool stream);
static bool task_is_bw(const MvmTaskDesc& d, const int32_t* a);

// Device window slots, pinned staging and control block; reset and launch of the persistent kernel. With scheduler
// classes each queue group holds one ring per class.
static int stream_launch(KvmExec* ex) {
  const KvmConfig& c = ex->cfg;
  const int cap = c.window_cap * c.window_tasks;
  auto alloc = [ex](size_t bytes) -> void* {
    void* d = nullptr;
    if (hipMalloc(&d, std::max<size_t>(bytes, 4)) != hipSuccess) return nullptr;
    ex->allocs.push_back(d);
    return d;
  };
  KvmDevState& S = ex->S;
  S = KvmDevState{};
  // one queue group when a task may be reserved for any worker (task affinity) or a class owns only some workers (the
  // static split): every worker sees every ring
  const bool one_group = ex->sched_mode == KVM_SCHED_STATIC || (ex->sched_mode != KVM_SCHED_GLOBAL && ex->affinity_us > 0);
  const int nq = one_group ? 1 : std::max(1, std::min(KVM_MAX_QUEUES, ex->grid));
  int qcap = 1;
  while (qcap < cap) qcap <<= 1;
  S.recs = (const KvmRec*)alloc((size_t)cap * sizeof(KvmRec));
  S.tasks = (const MvmTaskDesc*)alloc((size_t)cap * sizeof(MvmTaskDesc));
  S.succ = (const int32_t*)alloc((size_t)c.window_cap * std::max(1, c.window_edges) * sizeof(int32_t));
  S.indeg = (int*)alloc((size_t)cap * sizeof(int));
  S.state = (int*)alloc((size_t)cap * sizeof(int));
  S.park_next = (int*)alloc((size_t)cap * sizeof(int));
  if (c.trace_on) S.trace = (KvmTrace*)alloc((size_t)cap * sizeof(KvmTrace));
  const int ncls = ex->sched_mode != KVM_SCHED_GLOBAL ? (int)ex->classes.size() : 0, nring = nq * std::max(1, ncls);
  S.ready64 = (unsigned long long*)alloc((size_t)nring * qcap * sizeof(unsigned long long));
  S.queues = (KvmQueue*)alloc(nring * sizeof(KvmQueue));
  S.done_blk = (int*)alloc(ex->grid * sizeof(int));
  S.version = (int*)alloc(ex->base_versions.size() * sizeof(int));
  S.park_head = (int*)alloc(ex->base_versions.size() * sizeof(int));
  S.cnt = (KvmCounters*)alloc(sizeof(KvmCounters));
  S.adm = (KvmAdm*)alloc(sizeof(KvmAdm));
  S.win_left = (int*)alloc(c.window_cap * sizeof(int));
  S.win_seq = (int*)alloc(c.window_cap * sizeof(int));
  S.win_t0 = (unsigned long long*)alloc(c.window_cap * sizeof(unsigned long long));
  ex->L = LaunchArgs{};
  ex->L.base = (int*)alloc(ex->base_versions.size() * sizeof(int));
  if (!S.recs || !S.tasks || !S.succ || !S.indeg || !S.state || !S.park_next || (c.trace_on && !S.trace) || !S.ready64 || !S.queues ||
      !S.done_blk || !S.version || !S.park_head || !S.cnt || !S.adm || !S.win_left || !S.win_seq || !S.win_t0 || !ex->L.base) {
    ex->err = "stream mode: device memory for the window slots"; return KVM_STATUS_HIP_ERROR;
  }
  const KvmWinLayout lay(c.window_cap, c.window_tasks, c.window_edges);
  const size_t ctl_bytes = sizeof(KvmHostCtl) + (size_t)c.window_cap * sizeof(long long);
  HIPCK(hipHostMalloc((void**)&ex->hctl, ctl_bytes, hipHostMallocCoherent | hipHostMallocMapped));
  HIPCK(hipHostMalloc((void**)&ex->hwin, lay.total, hipHostMallocCoherent | hipHostMallocMapped));
  HIPCK(hipHostMalloc((void**)&ex->hver, ex->base_versions.size() * sizeof(int), hipHostMallocCoherent | hipHostMallocMapped));
  std::memcpy(ex->hver, ex->base_versions.data(), ex->base_versions.size() * sizeof(int));
  std::memset(ex->hctl, 0, ctl_bytes);
  std::memset(ex->hwin, 0, lay.meta + (size_t)c.window_cap * sizeof(KvmHostWin));
  void *dctl = nullptr, *dwin = nullptr;
  HIPCK(hipHostGetDevicePointer(&dctl, ex->hctl, 0));
  HIPCK(hipHostGetDevicePointer(&dwin, ex->hwin, 0));
  void* dver = nullptr;
  HIPCK(hipHostGetDevicePointer(&dver, ex->hver, 0));
  S.hctl = (KvmHostCtl*)dctl; S.hwin = (const char*)dwin; S.hver = (int*)dver;
  S.stream = 1; S.wcap = c.window_cap; S.wtasks = c.window_tasks; S.wedges = c.window_edges;
  S.ntasks = cap; S.nvars = (int)ex->base_versions.size(); S.trace_on = c.trace_on && ex->trace_req ? 1 : 0;
  S.nq = nq; S.qcap = qcap; S.grid = ex->grid; S.nb = 1; S.ncells = 0;
  S.timeout_ticks = c.timeout_us * 100ull;
  if (ncls) {   // deadlines and bandwidth caps may concern any class: their head cells are always inspected
    unsigned char hd[KVM_MAX_CLASSES] = {}, hb[KVM_MAX_CLASSES] = {};
    for (int k = 0; k < ncls; ++k) {
      hd[k] = ex->classes[k].urgent_us > 0;
      hb[k] = ex->classes[k].bw_cta < KVM_UNLIMITED || (ex->sched_flags & KVM_SCHED_F_ARBITER);
    }
    const std::vector<int> pubcls(ex->base_versions.size(), 0);
    const std::vector<unsigned char> tbw((size_t)cap, 0);
    if (int r = upload_classes(ex, alloc, hd, hb, pubcls, tbw, true)) return r;
  }
  ex->path = KVM_PATH_DYNAMIC;
  ex->uploaded = true;
  HIPCK(hipStreamSynchronize(ex->stream));   // buffer initialisation done
  HIPCK(hipMemcpyAsync(ex->L.base, ex->base_versions.data(), ex->base_versions.size() * sizeof(int), hipMemcpyHostToDevice, ex->stream));
  HIPCK(hipEventRecord(ex->ev0, ex->stream));
  hipLaunchKernelGGL(kvm_reset_kernel, dim3(1024), dim3(256), 0, ex->stream, S, (const int*)ex->L.base);
  hipLaunchKernelGGL(kvm_exec_kernel, dim3(ex->grid), dim3(KVM_THREADS), 0, ex->stream, S);
  HIPCK(hipGetLastError());
  HIPCK(hipEventRecord(ex->ev1, ex->stream));
  ex->launched = true;
  return 0;
}

// Stream mode with scheduler classes: every task of a bundle names a class (checked before anything is staged).
static int stream_class_check(KvmExec* ex, const MvmTaskDesc* tasks, int n) {
  const int ncls = ex->sched_mode != KVM_SCHED_GLOBAL ? (int)ex->classes.size() : 0;
  for (int i = 0; ncls && i < n; ++i)
    if (tasks[i].workload_id < 0 || tasks[i].workload_id >= ncls) {
      ex->err = "scheduler classes: task " + std::to_string(i) + " of the bundle has workload_id " + std::to_string(tasks[i].workload_id) +
                ", not a class in [0, " + std::to_string(ncls) + ")";
      return KVM_STATUS_INVALID;
    }
  return 0;
}

static bool stream_done_mark(const KvmExec* ex, long long wid) {
  return __atomic_load_n(&ex->hctl->done_mark[wid % ex->cfg.window_cap], __ATOMIC_ACQUIRE) >= wid + 1;
}

// Stages one validated bundle into the next window slot (waiting for it to be free) and publishes it. Returns the
// window id or a negative status.
static long long stream_stage(KvmExec* ex, const MvmTaskDesc* tasks, int n, const int32_t* succ, int ne, const int32_t* args) {
  const KvmConfig& c = ex->cfg;
  if (n > c.window_tasks || ne > c.window_edges) {
    ex->err = "stream mode: bundle of " + std::to_string(n) + " tasks / " + std::to_string(ne) + " edges exceeds a window (" +
              std::to_string(c.window_tasks) + " / " + std::to_string(c.window_edges) + ")";
    return KVM_STATUS_TOO_BIG;
  }
  const long long seq = ex->seq;
  const int w = (int)(seq % c.window_cap), base = w * c.window_tasks;
  if (seq >= c.window_cap) {   // the slot's previous window (seq - window_cap) must have finished
    const auto t0 = std::chrono::steady_clock::now();
    while (!stream_done_mark(ex, seq - c.window_cap)) {
      if (hipStreamQuery(ex->stream) == hipSuccess) { ex->err = "stream mode: the kernel ended (device error or stall) while windows were pending"; return KVM_STATUS_DEVICE_ERROR; }
      if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(c.backpressure_ms)) {
        ex->err = "stream mode: no window slot became free within " + std::to_string(c.backpressure_ms) + " ms (window " + std::to_string(seq - c.window_cap) + " not finished)";
        return KVM_STATUS_BACKPRESSURE_TIMEOUT;
      }
      std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
  }
  const KvmWinLayout lay(c.window_cap, c.window_tasks, c.window_edges);
  const std::vector<MvmBuf> table = buf_table(ex);
  KvmRec* recs = (KvmRec*)(ex->hwin + lay.recs) + base;
  MvmTaskDesc* td = (MvmTaskDesc*)(ex->hwin + lay.tasks) + base;
  int32_t* sd = (int32_t*)(ex->hwin + lay.succ) + (size_t)w * c.window_edges;
  int32_t* rt = (int32_t*)(ex->hwin + lay.roots) + base;
  KvmHostWin& m = *((KvmHostWin*)(ex->hwin + lay.meta) + w);
  int nroots = 0, qn[KVM_MAX_QUEUES] = {};
  const int nq = ex->S.nq, ncls = ex->S.ncls;
  for (int i = 0; i < n; ++i) {
    MvmTaskDesc d = tasks[i];
    d.succ_off += w * c.window_edges;
    d.reserved0 = base;
    d.reserved1 = ncls && task_is_bw(tasks[i], args + tasks[i].args_off) ? 1 : 0;   // the staged copy: bandwidth-bound
    td[i] = d;
    make_rec(d, args + tasks[i].args_off, table, recs[i]);
    if (d.indegree == 0) rt[nroots++] = i;
    ++qn[(base + i) % nq];
  }
  for (int e = 0; e < ne; ++e) {
    const int l = succ[e];
    sd[e] = (base + l) | edge_flags(tasks[l]);
  }
  m.seq = (int)seq; m.ntasks = n; m.nedges = ne; m.nroots = nroots;
  for (int q = 0; q < KVM_MAX_QUEUES; ++q) m.qn[q] = qn[q];
  std::atomic_thread_fence(std::memory_order_seq_cst);
  __atomic_store_n(&ex->hctl->submitted, seq + 1, __ATOMIC_SEQ_CST);
  ex->seq = seq + 1;
  ex->stream_tasks += n;
  return seq;
}

int kvm_close(KvmExec* ex) {
  if (!ex->streaming) { ex->err = "kvm_close: not in stream mode"; return KVM_STATUS_INVALID; }
  if (!ex->hctl) {   // never started: start (admits the pending bundles), then close
    if (int rc = kvm_start(ex)) return rc;
  }
  ex->closed = true;
  std::atomic_thread_fence(std::memory_order_seq_cst);
  __atomic_store_n(&ex->hctl->closed, 1, __ATOMIC_SEQ_CST);
  return 0;
}

int kvm_live_versions(KvmExec* ex, int32_t* out, int n) {
  if (!ex->streaming || !ex->hver || n < 0 || n > (int)ex->base_versions.size()) { ex->err = "kvm_live_versions: not started in stream mode, or n too large"; return KVM_STATUS_INVALID; }
  for (int i = 0; i < n; ++i) out[i] = __atomic_load_n(&ex->hver[i], __ATOMIC_ACQUIRE);
  return 0;
}

int kvm_window_done(KvmExec* ex, long long wid) {
  if (!ex->streaming || !ex->hctl || wid < 0 || wid >= ex->seq) { ex->err = "kvm_window_done: not a submitted window"; return KVM_STATUS_INVALID; }
  return stream_done_mark(ex, wid) ? 1 : 0;
}

int kvm_submit_stream(KvmExec* ex, const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args,
                      int nargs, int max_window_tasks, int timeout_ms) {
  if (!ex->streaming) { ex->err = "kvm_submit_stream: not in stream mode"; return KVM_STATUS_INVALID; }
  if (ex->closed) { ex->err = "kvm_submit_stream: closed"; return KVM_STATUS_CLOSED; }
  const std::vector<MvmBuf> table = buf_table(ex);
  std::string why;
  if (!kvm_validate_bundle(tasks, ntasks, succ, nedges, args, nargs, table.data(), (int)table.size(), (int)ex->base_versions.size(), &why)) {
    ex->err = why; return KVM_STATUS_INVALID;
  }
  if (int r = stream_class_check(ex, tasks, ntasks)) return r;
  for (int i = 0; i < ntasks; ++i)
    for (int k = 0; k < tasks[i].succ_cnt; ++k)
      if (succ[tasks[i].succ_off + k] <= i) {
        ex->err = "kvm_submit_stream: tasks must be in topological order (edge " + std::to_string(i) + " -> " + std::to_string(succ[tasks[i].succ_off + k]) + ")";
        return KVM_STATUS_INVALID;
      }
  if (!ex->hctl) { if (int rc = kvm_start(ex)) return rc; }
  const int cap = std::min(max_window_tasks > 0 ? max_window_tasks : ex->cfg.window_tasks, ex->cfg.window_tasks);
  // window boundaries: at most `cap` tasks and window_edges edges inside the window
  std::vector<int> lo{0};
  { int cnt = 0; long long edges = 0;
    for (int i = 0; i < ntasks; ++i) {
      int inside = 0;   // edges of task i that stay in its window if the window grows to hold it (counted pessimistically: all)
      inside = tasks[i].succ_cnt;
      if (cnt > 0 && (cnt >= cap || edges + inside > ex->cfg.window_edges)) { lo.push_back(i); cnt = 0; edges = 0; }
      ++cnt; edges += inside;
    }
    lo.push_back(ntasks); }
  const int nw = (int)lo.size() - 1;
  std::vector<int> win_of(ntasks);
  for (int k = 0; k < nw; ++k) for (int i = lo[k]; i < lo[k + 1]; ++i) win_of[i] = k;
  std::vector<std::vector<int>> needs(nw);
  { std::vector<int> last(nw, -1);
    for (int i = 0; i < ntasks; ++i) for (int k = 0; k < tasks[i].succ_cnt; ++k) {
      const int wt = win_of[succ[tasks[i].succ_off + k]], wi = win_of[i];
      if (wt != wi && last[wt] != wi) { last[wt] = wi; needs[wt].push_back(wi); }
    } }
  std::vector<long long> wid(nw, -1);
  for (int k = 0; k < nw; ++k) {
    for (int j : needs[k]) {
      const auto t0 = std::chrono::steady_clock::now();
      while (!stream_done_mark(ex, wid[j])) {
        if (hipStreamQuery(ex->stream) == hipSuccess) { ex->err = "kvm_submit_stream: the kernel ended while windows were pending"; return KVM_STATUS_DEVICE_ERROR; }
        if (std::chrono::steady_clock::now() - t0 > std::chrono::milliseconds(timeout_ms)) {
          ex->err = "kvm_submit_stream: window " + std::to_string(j) + " did not finish within " + std::to_string(timeout_ms) + " ms";
          return KVM_STATUS_BACKPRESSURE_TIMEOUT;
        }
        std::this_thread::sleep_for(std::chrono::microseconds(20));
      }
    }
    const int a = lo[k], z = lo[k + 1];
    std::vector<MvmTaskDesc> wt;
    std::vector<int32_t> ws, wa;
    for (int i = a; i < z; ++i) {
      MvmTaskDesc t = tasks[i];
      const int off = (int)ws.size();
      for (int e = 0; e < tasks[i].succ_cnt; ++e) { const int s2 = succ[tasks[i].succ_off + e]; if (s2 < z) ws.push_back(s2 - a); }
      t.succ_off = off; t.succ_cnt = (int)ws.size() - off; t.indegree = 0;
      t.args_off = (int)wa.size();
      wa.insert(wa.end(), args + tasks[i].args_off, args + tasks[i].args_off + t.args_words);
      wt.push_back(t);
    }
    for (int s2 : ws) ++wt[s2].indegree;
    const long long r = stream_stage(ex, wt.data(), (int)wt.size(), ws.data(), (int)ws.size(), wa.data());
    if (r < 0) return (int)r;
    wid[k] = r;
  }
  return nw;
}

int kvm_submit(KvmExec* ex, const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs) {
  if (ex->streaming) {
    if (ex->closed) { ex->err = "kvm_submit: closed"; return KVM_STATUS_CLOSED; }
    if (ntasks < 1 || nedges < 0 || nargs < 0) { ex->err = "empty bundle"; return KVM_STATUS_INVALID; }
    const std::vector<MvmBuf> table = buf_table(ex);
    std::string why;
    if (!kvm_validate_bundle(tasks, ntasks, succ, nedges, args, nargs, table.data(), (int)table.size(), (int)ex->base_versions.size(), &why)) {
      ex->err = why; return KVM_STATUS_INVALID;
    }
    if (ntasks > ex->cfg.window_tasks || nedges > ex->cfg.window_edges) {
      ex->err = "stream mode: bundle exceeds a window (" + std::to_string(ntasks) + " tasks, " + std::to_string(nedges) + " edges)";
      return KVM_STATUS_TOO_BIG;
    }
    if (int r = stream_class_check(ex, tasks, ntasks)) return r;
    if (!ex->hctl) {   // before start: kept, admitted in order at kvm_start
      ex->pending.push_back(KvmExec::Pending{std::vector<MvmTaskDesc>(tasks, tasks + ntasks), std::vector<int32_t>(succ, succ + nedges),
                                              std::vector<int32_t>(args, args + nargs)});
      return (int)(ex->pending.size() - 1);
    }
    const long long r = stream_stage(ex, tasks, ntasks, succ, nedges, args);
    return r < 0 ? (int)r : (int)std::min<long long>(r, 0x7fffffff);
  }
  if (ex->uploaded) { ex->err = "kvm_submit after kvm_start: this executor runs the bundles submitted before start"; return KVM_STATUS_CLOSED; }
  if (ntasks < 1 || nedges < 0 || nargs < 0) { ex->err = "empty bundle"; return KVM_STATUS_INVALID; }
  std::vector<MvmBuf> table(ex->bufs.size());
  for (size_t i = 0; i < table.size(); ++i) table[i] = MvmBuf{ex->bufs[i].p, ex->bufs[i].rows, ex->bufs[i].cols, ex->bufs[i].cols, ex->bufs[i].dtype, {0, 0}};
  std::string why;
  if (!kvm_validate_bundle(tasks, ntasks, succ, nedges, args, nargs, table.data(), (int)table.size(), (int)ex->base_versions.size(), &why)) {
    ex->err = why; return KVM_STATUS_INVALID;
  }
  if ((long long)ex->tasks.size() + ntasks > (1ll << 30)) { ex->err = "too many tasks"; return KVM_STATUS_TOO_BIG; }
  int tbase = (int)ex->tasks.size(), sbase = (int)ex->succ.size(), abase = (int)ex->args.size();
  for (int i = 0; i < ntasks; ++i) {
    MvmTaskDesc d = tasks[i];
    d.succ_off += sbase; d.args_off += abase; d.reserved0 = tbase;   // reserved0: the bundle's first global task index
    ex->tasks.push_back(d);
    if (d.indegree == 0) ex->roots.push_back(tbase + i);
  }
  for (int e = 0; e < nedges; ++e) ex->succ.push_back(succ[e] + tbase);
  ex->args.insert(ex->args.end(), args, args + nargs);
  return 0;
}

// Planning cost of a task in microseconds, for the static planner's list schedule. Fitted to per-task traces of the
// tiny GPT and the eight-MLP graph on MI355X: an fp32 GEMM tile costs about 9 us plus 1.55 us per MFLOP (least squares
// over 72,500 traced tiles), the bf16 MFMA tiles about 3 us plus their flops at 3 TFLOP/s per CU; the other operators
// take their traced medians (row norms and the fused cross entropy about 8 us, the layer-norm input gradient 15 us,
// elementwise activations 5.5 us, a no-op well under 1 us) and 3 us when not listed. The ratios set the plan's
// critical-path priorities and worker balance; the mean decides the auto path (KVM_STATIC_MAX_MEAN_US).
static double task_cost_us(const MvmTaskDesc& d, const int32_t* a) {
  const int op = d.op_id;
  if (op == 34 || op == 114 || op == 122 || op == 302 || op == 304 || op == 308) {
    const long long m0 = a[6], n0 = a[7], M = a[8], N = a[9], K = a[10], fl = a[11];
    int tm = 64, tn = 64;
    if (op == 122 || op == 308) { tm = 128; tn = 256; }
    else if (op == 304) { tm = 256; tn = 256; }
    else if (op == 302) { tm = fl & 64 ? 256 : 128; tn = 256; }
    else if (fl & 64) { tm = 256; tn = 128; }
    else if (fl & 32) { tm = tn = 128; }
    const double flops = 2.0 * (double)std::max(0ll, std::min(M, m0 + tm) - m0) * (double)std::max(0ll, std::min(N, n0 + tn) - n0) * (double)K;
    return op == 34 ? 9.0 + flops / 0.65e6 : 3.0 + flops / 3.0e6;
  }
  switch (op) {
    case 45: case 47: case 48: {   // q0 / k0 block of 128 rows against up to T keys: about T * 128 * hd * 4 flop
      const int T = op == 48 ? a[11] : a[8], hd = op == 48 ? a[13] : a[11];
      return 5.0 + 4.0 * 128.0 * (double)T * hd / 1.0e6;
    }
    case 0: return 0.7;                                              // noop
    case 37: return 15.0;                                            // layernorm_bwd_dx
    case 35: case 46: case 54: case 127: case 309: return 8.0;       // layernorm_fwd, attn_bwd_delta, adamw, softmax_ce_fused, layernorm_bwd_dx_res
    case 33: case 96: case 97: return 5.5;                           // embedding_bwd, act_fwd, act_bwd
    default: return 3.0;
  }
}

// Bytes a task streams when its operator is bandwidth-bound, else -1: the reference's scheduler cost table
// (include/mvm_ops_cost.inc: the operators it lists as BW, with its byte expressions over the argument words) for the
// operators implemented here, and this executor's AdamW with the bf16 copy (op 305). Operators it leaves out (GEMM tiles,
// attention, reductions, the decode GEMVs) count as not bandwidth-bound, as there. A BW task under 16 KiB is
// latency-bound (MVM_LAT_BYTES).
static long long task_bw_bytes(const MvmTaskDesc& d, const int32_t* a) {
  auto U = [&](int k) { return k < d.args_words ? (long long)(unsigned)a[k] : 0ll; };
  auto R = [&](int lo, int hi) { return std::max(0ll, U(hi) - U(lo)); };
  switch (d.op_id) {
    case 1: return 8 * U(2);                 // copy
    case 2: return 12 * U(3);                // add
    case 3: return 8 * U(3);                 // scale
    case 4: return 8 * U(2);                 // relu
    case 5: return 12 * U(3);                // sgd
    case 6: return 8 * U(3);                 // predict
    case 7: return 12 * U(5);                // mse_grad
    case 9: return 4 * U(2);                 // fill
    case 54: return 28 * R(6, 7);            // adamw
    case 305: return 30 * R(6, 7);           // adamw_bf16
    case 55: return 4 * R(3, 4);             // gradnorm_partial
    case 42: return 12 * R(3, 4);            // residual_add
    case 40: return 8 * R(2, 3);             // gelu_fwd
    case 41: return 12 * R(3, 4);            // gelu_bwd
    case 123: return 12 * R(3, 4);           // sgd_range
    case 126: return 8 * R(2, 3);            // round_tf32
    case 59: return 4 * R(1, 2);             // zero_buf
    case 32: return 8 * R(4, 5) * U(7);      // embedding_fwd
    case 51: return 4 * R(4, 5) * U(6);      // softmax_ce_fwd
    case 53: return 8 * R(5, 6) * U(7);      // softmax_ce_bwd
    default: return -1;
  }
}
static bool task_is_bw(const MvmTaskDesc& d, const int32_t* a) { return task_bw_bytes(d, a) >= 16384; }

// Static-path flags per task: KVM_SF_PUB, another worker waits for the task; KVM_SF_PRE, a decode GEMV (op 134 / 301)
// whose weight buffer no task of the graph writes (it appears in no argument slot other than the weights of such
// GEMVs), so its first weight loads may be issued before its dependencies are met, or a decode attention split whose
// caches appear only as the caches of splits.
static std::vector<int> static_flags(const KvmExec* ex, const kvms::Plan& P) {
  const int n = (int)ex->tasks.size(), nb = (int)ex->bufs.size();
  std::vector<char> other_use(nb, 0);
  std::vector<std::vector<kvmv::ArgInfo>> sigs(1024);
  for (int i = 0; i < n; ++i) {
    const MvmTaskDesc& d = ex->tasks[i];
    const int op = d.op_id;
    if (op < 0 || op >= 1024) continue;
    if (sigs[op].empty()) if (const kvmv::OpSig* o = kvmv::find_op(op)) sigs[op] = kvmv::parse_sig(o->sig);
    const int32_t* a = ex->args.data() + d.args_off;
    for (size_t k = 0; k < sigs[op].size() && (int)k < d.args_words; ++k)
      if (sigs[op][k].type == 0 && a[k] >= 0 && a[k] < nb && !((op == 134 || op == 301) && k == 3) && !(op == 311 && (k == 2 || k == 3)) &&
          !((op == 135 || op == 306 || op == 310) && (k == 1 || k == 2)))
        other_use[a[k]] = 1;
  }
  std::vector<int> f(n, 0);
  for (int i = 0; i < n; ++i) {
    const MvmTaskDesc& d = ex->tasks[i];
    if (P.publishes[i]) f[i] |= KVM_SF_PUB;
    if ((d.op_id == 134 || d.op_id == 301) && d.args_words > 3) {
      const int wb = ex->args[d.args_off + 3];
      if (wb >= 0 && wb < nb && !other_use[wb] && !getenv("KVM_NO_PREFETCH")) f[i] |= KVM_SF_PRE;
    }
    if (d.op_id == 311 && d.args_words > 3) {
      const int wg = ex->args[d.args_off + 2], wu = ex->args[d.args_off + 3];
      if (wg >= 0 && wg < nb && wu >= 0 && wu < nb && !other_use[wg] && !other_use[wu] && !getenv("KVM_NO_PREFETCH")) f[i] |= KVM_SF_PRE;
    }
    // A decode attention split whose caches only the splits use (each writes its own new row): its first block and
    // rotation table are staged before the wait.
    if ((d.op_id == 135 || d.op_id == 306 || d.op_id == 310) && d.args_words > 3) {
      const int kb = ex->args[d.args_off + 1], vb = ex->args[d.args_off + 2];
      if (kb >= 0 && kb < nb && vb >= 0 && vb < nb && kb != vb && !other_use[kb] && !other_use[vb] && !getenv("KVM_NO_PREFETCH") &&
          !getenv("KVM_NO_ATTN_PREFETCH"))
        f[i] |= KVM_SF_PRE;
    }
  }
  return f;
}

// The static kernel's inlined operator set for this graph: the one covering more of its decode GEMVs (the GQA-4
// attention split is in both).
static int static_variant(const KvmExec* ex) {
  long long deep = 0, rows8 = 0, attn4 = 0;
  for (const MvmTaskDesc& d : ex->tasks) {
    if (d.op_id == 134) ++deep;
    else if ((d.op_id == 306 || d.op_id == 310) && d.args_words > 12 && ex->args[d.args_off + 11] == 4 * ex->args[d.args_off + 12]) ++attn4;
    else if ((d.op_id == 301 && d.args_words > 9) || (d.op_id == 311 && d.args_words > 8)) {
      const int M = ex->args[d.args_off + (d.op_id == 301 ? 9 : 8)];
      if (M >= 1 && M <= 4) ++deep;
      else if (M >= 5 && M <= 8) ++rows8;
    }
  }
  return rows8 > deep ? 2 : deep > 0 || attn4 > 0 ? 1 : 0;
}

static int plan_static(KvmExec* ex, bool forced) {
  std::string why;
  if (!kvms::feasible(ex->tasks.data(), (int)ex->tasks.size(), ex->base_versions.data(), (int)ex->base_versions.size(), &why)) {
    if (forced) { ex->err = "static path: " + why; return KVM_STATUS_INVALID; }
    return 0;
  }
  std::vector<double> cost(ex->tasks.size());
  double total = 0;
  for (size_t i = 0; i < ex->tasks.size(); ++i) { cost[i] = task_cost_us(ex->tasks[i], ex->args.data() + ex->tasks[i].args_off); total += cost[i]; }
  if (!forced && total / (double)cost.size() > KVM_STATIC_MAX_MEAN_US) return 0;
  try {
    ex->splan_d = kvms::plan(ex->tasks.data(), (int)ex->tasks.size(), ex->succ.data(), cost, ex->grid, 1.5, true);
    if (ex->cfg.trace_on) {
      if (ex->splan_d.dissolved) ex->splan = kvms::plan(ex->tasks.data(), (int)ex->tasks.size(), ex->succ.data(), cost, ex->grid, 1.5, false);
      else ex->splan = ex->splan_d;
    }
  } catch (const std::exception& e) {
    ex->err = std::string("static path: ") + e.what();
    return KVM_STATUS_INVALID;
  }
  ex->path = KVM_PATH_STATIC;
  ex->S.svariant = static_variant(ex);
  // Progress words: one per 64 bytes for the general kernel (its tasks wait on a few workers each, and packed words
  // shared a line among 16-32 publishing workers: tiny GPT 477 -> 457 us per step), packed for the decode kernels (a
  // task there waits on a whole phase of up to 256 workers, whose packed words a poll reads in 8 lines: padded, decode
  // measured 0.5-1.4% slower).
  ex->S.pstride = ex->S.svariant == 0 ? KVM_PSTRIDE_MAX : 1;
  return 0;
}

// Scheduler classes on the device: the class parameter lines (the reset kernel clears the rest at every launch) and
// the inheritance and bandwidth state. Launch mode: has_dl / has_bw / pubcls / tbw from the submitted tasks. Stream
// mode: tbw per slot and pubcls start empty and are filled at admission; every variable is in the publication list.
static int upload_classes(KvmExec* ex, const std::function<void*(size_t)>& alloc, const unsigned char* has_dl, const unsigned char* has_bw,
                          const std::vector<int>& pubcls, const std::vector<unsigned char>& tbw, bool stream) {
  const int ncls = (int)ex->classes.size();
  KvmSchedDev h{};
  double tot = 0, acc = 0;
  for (auto& c : ex->classes) tot += c.share;
  for (int c = 0; c < ncls; ++c) {
    const KvmClassParams& p = ex->classes[c];
    KvmClsDev& k = h.cls[c];
    k.weight = p.weight; k.min_cta = p.min_cta; k.max_cta = p.max_cta;
    k.urgent_ticks = (int)std::min<long long>((long long)p.urgent_us * 100ll, 0x7fffffffll);
    k.vt_mul = (1 << 20) / p.weight; k.has_dl = has_dl[c];
    k.bw_cta = p.bw_cta; k.has_bw = has_bw[c]; k.opaff = (p.flags & KVM_CLASS_OPAFF) ? 1 : 0;
    k.blk_lo = 0; k.blk_hi = ex->grid;
    if (ex->sched_mode == KVM_SCHED_STATIC) {   // cumulative bounds, the last class takes the rest
      k.blk_lo = (int)(acc / tot * ex->grid + 0.5);
      acc += p.share;
      k.blk_hi = c + 1 == ncls ? ex->grid : (int)(acc / tot * ex->grid + 0.5);
      bool used = stream;   // stream mode: the tasks come later, every class needs a worker
      for (const MvmTaskDesc& d : ex->tasks) if (d.workload_id == c) { used = true; break; }
      if (used && k.blk_hi <= k.blk_lo) {
        ex->err = "scheduler classes: class " + std::to_string(c) + " gets no worker of " + std::to_string(ex->grid) + " (shares)";
        return KVM_STATUS_INVALID;
      }
    }
  }
  h.flags = ex->sched_mode == KVM_SCHED_DYNAMIC ? ex->sched_flags : 0;
  h.bw_limit = ex->bw_limit;
  h.aff_ticks = (unsigned long long)ex->affinity_us * 100ull;
  KvmSchedDev* d = (KvmSchedDev*)alloc(sizeof(KvmSchedDev));
  if (!d || hipMemcpy(d, &h, sizeof h, hipMemcpyHostToDevice) != hipSuccess) { ex->err = "scheduler classes: device memory"; return KVM_STATUS_HIP_ERROR; }
  ex->S.sched = d; ex->S.ncls = ncls;
  // inheritance: parked-waiter counts (cleared by the reset kernel), the publisher classes and the published variables
  std::vector<int> publist;   // stream mode: every variable (pubcls is or-ed in at admission)
  for (size_t v = 0; v < pubcls.size(); ++v) if (pubcls[v] || stream) publist.push_back((int)v);
  const size_t nv = std::max<size_t>(pubcls.size(), 1);
  int* pv = (int*)alloc(nv * KVM_MAX_CLASSES * sizeof(int));
  int* pc = (int*)alloc(nv * sizeof(int));
  int* pl = (int*)alloc(std::max<size_t>(publist.size(), 1) * sizeof(int));
  unsigned char* tb = (unsigned char*)alloc(std::max<size_t>(tbw.size(), 1));
  if (!pv || !pc || !pl || !tb || (!pubcls.empty() && hipMemcpy(pc, pubcls.data(), pubcls.size() * sizeof(int), hipMemcpyHostToDevice) != hipSuccess) ||
      (!publist.empty() && hipMemcpy(pl, publist.data(), publist.size() * sizeof(int), hipMemcpyHostToDevice) != hipSuccess) ||
      (!tbw.empty() && hipMemcpy(tb, tbw.data(), tbw.size(), hipMemcpyHostToDevice) != hipSuccess)) {
    ex->err = "scheduler classes: device memory"; return KVM_STATUS_HIP_ERROR;
  }
  ex->S.pv = pubcls.empty() ? nullptr : pv; ex->S.pubcls = pc; ex->S.publist = pl; ex->S.npub = (int)publist.size(); ex->S.tbw = tb;
  if (ex->affinity_us > 0) {   // per task slot: release time and preferred worker; per operator: the last worker
    ex->S.aff = (unsigned long long*)alloc(std::max<size_t>(tbw.size(), 1) * sizeof(unsigned long long));
    ex->S.op_blk = (int*)alloc(KVM_OP_SLOTS * sizeof(int));
    if (!ex->S.aff || !ex->S.op_blk) { ex->err = "scheduler classes: device memory"; return KVM_STATUS_HIP_ERROR; }
  }
  return 0;
}

static int do_upload(KvmExec* ex) {
  if (ex->tasks.empty()) { ex->err = "nothing submitted"; return KVM_STATUS_INVALID; }
  std::vector<MvmBuf> table(ex->bufs.size());
  for (size_t i = 0; i < table.size(); ++i) table[i] = MvmBuf{ex->bufs[i].p, ex->bufs[i].rows, ex->bufs[i].cols, ex->bufs[i].cols, ex->bufs[i].dtype, {0, 0}};
  const int ncls = ex->sched_mode != KVM_SCHED_GLOBAL ? (int)ex->classes.size() : 0;
  std::vector<unsigned char> has_dl(KVM_MAX_CLASSES, 0), has_bw(KVM_MAX_CLASSES, 0), tbw(ncls ? ex->tasks.size() : 0, 0);
  std::vector<int> pubcls(ex->base_versions.size(), 0);   // classes publishing each variable (inheritance)
  if (ncls) {   // every task names a class; the (class, priority) buckets fit one wave's lanes
    std::vector<char> seen(KVM_PRIORITIES, 0);
    int nprio = 0;
    for (size_t i = 0; i < ex->tasks.size(); ++i) {
      const MvmTaskDesc& d = ex->tasks[i];
      if (d.workload_id < 0 || d.workload_id >= ncls) {
        ex->err = "scheduler classes: task " + std::to_string(i) + " has workload_id " + std::to_string(d.workload_id) + ", not a class in [0, " +
                  std::to_string(ncls) + ")";
        return KVM_STATUS_INVALID;
      }
      if (!seen[d.priority]) { seen[d.priority] = 1; ++nprio; }
      if (d.deadline_us >= 0) has_dl[d.workload_id] = 1;
      tbw[i] = task_is_bw(d, ex->args.data() + d.args_off) ? 1 : 0;
      if (tbw[i]) has_bw[d.workload_id] = 1;
      if (d.pub_var >= 0 && d.pub_var < (int)pubcls.size()) pubcls[d.pub_var] |= 1 << d.workload_id;
    }
    if (nprio * ncls > 64) {
      ex->err = "scheduler classes: " + std::to_string(ncls) + " classes x " + std::to_string(nprio) + " distinct priorities exceed 64 ready buckets";
      return KVM_STATUS_INVALID;
    }
    if (ex->cfg.path == KVM_PATH_STATIC) { ex->err = "scheduler classes run on the dynamic path (path must be DYNAMIC or AUTO)"; return KVM_STATUS_INVALID; }
  }
  GraphPlan g;
  plan_graph(ex->tasks, ex->succ, ex->args, table, ex->roots, ex->grid, ex->cfg.aging_us, g, ncls,
             ex->sched_mode == KVM_SCHED_STATIC || (ncls && ex->affinity_us > 0));   // one group: every worker sees every queue
  auto alloc = [ex](size_t bytes) -> void* {
    void* d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return nullptr;
    ex->allocs.push_back(d);
    return d;
  };
  ex->err.clear();
  const int rc = place_graph(g, ex->tasks, (int)ex->base_versions.size(), ex->grid, ex->cfg.trace_on != 0, ex->cfg.aging_us,
                             ex->cfg.timeout_us, alloc, ex->stream, ex->S, ex->L, ex->err);
  if (rc) return rc == KVM_STATUS_TOO_BIG ? KVM_STATUS_HIP_ERROR : rc;
  ex->S.trace_on = ex->cfg.trace_on && ex->trace_req ? 1 : 0;   // a kvm_set_trace before the first launch holds
  ex->path = KVM_PATH_DYNAMIC;
  if (ncls) { if (int r = upload_classes(ex, alloc, has_dl.data(), has_bw.data(), pubcls, tbw, false)) return r; }
  if (ex->cfg.path != KVM_PATH_DYNAMIC && !ncls) {
    if (int r = plan_static(ex, ex->cfg.path == KVM_PATH_STATIC)) return r;
    if (ex->path == KVM_PATH_STATIC) {   // the plans' arrays next to the dynamic state (a later relaunch may use either)
      auto put = [&](const std::vector<int>& v) -> int* {
        void* d = alloc(std::max<size_t>(v.size(), 1) * sizeof(int));
        if (d && !v.empty() && hipMemcpy(d, v.data(), v.size() * sizeof(int), hipMemcpyHostToDevice) != hipSuccess) return nullptr;
        return (int*)d;
      };
      auto upload_plan = [&](const kvms::Plan& P, KvmExec::StaticDev& D) {
        std::vector<int> sw(2 * P.waits.size()), sflag = static_flags(ex, P);
        for (size_t k = 0; k < P.waits.size(); ++k) { sw[2 * k] = P.waits[k].worker; sw[2 * k + 1] = P.waits[k].need; }
        D.prog_off = put(P.prog_off); D.prog = put(P.prog); D.wait_off = put(P.wait_off); D.sw = put(sw); D.flag = put(sflag);
        D.dissolved = P.dissolved;
        return D.prog_off && D.prog && D.wait_off && D.sw && D.flag;
      };
      bool ok = upload_plan(ex->splan_d, ex->sdis);
      if (ex->cfg.trace_on) ok = ok && (ex->splan_d.dissolved ? upload_plan(ex->splan, ex->sfull) : (ex->sfull = ex->sdis, true));
      ex->S.sprogress = (int*)alloc(ex->grid * KVM_PSTRIDE_MAX * sizeof(int));
      if (!ok || !ex->S.sprogress) { ex->err = "static path: device memory"; return KVM_STATUS_HIP_ERROR; }
    }
  }
  ex->uploaded = true;
  return 0;
}

// Reset of the scheduler state, root seeding and the persistent kernel, on one stream.
static void launch_graph(const KvmDevState& S, const LaunchArgs& L, int grid, hipStream_t st, hipEvent_t before_exec, hipEvent_t after_exec,
                         bool static_path = false) {
  hipLaunchKernelGGL(kvm_reset_kernel, dim3(std::min(1024, (S.ntasks + 255) / 256 + 1)), dim3(256), 0, st, S, (const int*)L.base);
  if (!static_path) hipLaunchKernelGGL(kvm_seed_kernel, dim3(1), dim3(1024), 0, st, S, L.roots, L.root_cell, L.nfixed, L.nroots, L.fixed_tail);
  if (before_exec) hipEventRecord(before_exec, st);
  if (static_path) {
    if (S.svariant == 1) hipLaunchKernelGGL(kvm_static_kernel<1>, dim3(grid), dim3(KVM_THREADS), 0, st, S);
    else if (S.svariant == 2) hipLaunchKernelGGL(kvm_static_kernel<2>, dim3(grid), dim3(KVM_THREADS), 0, st, S);
    else hipLaunchKernelGGL(kvm_static_kernel<0>, dim3(grid), dim3(KVM_THREADS), 0, st, S);
  }
  else hipLaunchKernelGGL(kvm_exec_kernel, dim3(grid), dim3(KVM_THREADS), 0, st, S);
  if (after_exec) hipEventRecord(after_exec, st);
}

static int launch_once(KvmExec* ex, hipEvent_t before_exec = nullptr, hipEvent_t after_exec = nullptr) {
  HIPCK(hipMemcpyAsync(ex->L.base, ex->base_versions.data(), ex->base_versions.size() * sizeof(int), hipMemcpyHostToDevice, ex->stream));
  ex->last_dissolved = 0;
  if (ex->path == KVM_PATH_STATIC) {   // traced launches run every task; untraced ones the plan with the no-ops dissolved
    const KvmExec::StaticDev& D = ex->S.trace_on ? ex->sfull : ex->sdis;
    ex->S.sprog_off = D.prog_off; ex->S.sprog = D.prog; ex->S.swait_off = D.wait_off; ex->S.sw = D.sw; ex->S.sflag = D.flag;
    ex->last_dissolved = D.dissolved;
  }
  launch_graph(ex->S, ex->L, ex->grid, ex->stream, before_exec, after_exec, ex->path == KVM_PATH_STATIC);
  HIPCK(hipGetLastError());
  return 0;
}

int kvm_start(KvmExec* ex) {
  hipSetDevice(ex->dev);
  if (ex->streaming) {
    if (ex->hctl) { ex->err = "kvm_start: already started"; return KVM_STATUS_INVALID; }
    if (int rc = stream_launch(ex)) return rc;
    std::vector<KvmExec::Pending> p;
    p.swap(ex->pending);
    for (auto& b : p) {
      const long long r = stream_stage(ex, b.t.data(), (int)b.t.size(), b.s.data(), (int)b.s.size(), b.a.data());
      if (r < 0) return (int)r;
    }
    return 0;
  }
  if (!ex->uploaded) { int rc = do_upload(ex); if (rc) return rc; }
  HIPCK(hipStreamSynchronize(ex->stream));   // buffer initialisation done
  HIPCK(hipEventRecord(ex->ev0, ex->stream));
  int rc = launch_once(ex);
  if (rc) return rc;
  HIPCK(hipEventRecord(ex->ev1, ex->stream));
  ex->launched = true;
  return 0;
}

int kvm_relaunch(KvmExec* ex) {
  if (ex->streaming) { ex->err = "kvm_relaunch: stream mode runs one launch (submit more bundles instead)"; return KVM_STATUS_INVALID; }
  if (!ex->uploaded) return kvm_start(ex);
  hipSetDevice(ex->dev);
  HIPCK(hipEventRecord(ex->ev0, ex->stream));
  int rc = launch_once(ex);
  if (rc) return rc;
  HIPCK(hipEventRecord(ex->ev1, ex->stream));
  ex->launched = true;
  return 0;
}

int kvm_run_timed(KvmExec* ex, int n, float* ms) {
  if (ex->streaming) { ex->err = "kvm_run_timed: not in stream mode"; return KVM_STATUS_INVALID; }
  hipSetDevice(ex->dev);
  if (!ex->uploaded) { int rc = do_upload(ex); if (rc) return rc; }
  HIPCK(hipStreamSynchronize(ex->stream));
  HIPCK(hipEventRecord(ex->ev0, ex->stream));
  for (int i = 0; i < n; ++i) { int rc = launch_once(ex); if (rc) return rc; }
  HIPCK(hipEventRecord(ex->ev1, ex->stream));
  HIPCK(hipEventSynchronize(ex->ev1));
  HIPCK(hipEventElapsedTime(ms, ex->ev0, ex->ev1));
  ex->launched = true;
  return 0;
}

int kvm_run_timed_split(KvmExec* ex, int n, float* total_ms, float* exec_ms) {
  if (ex->streaming) { ex->err = "kvm_run_timed_split: not in stream mode"; return KVM_STATUS_INVALID; }
  hipSetDevice(ex->dev);
  if (n < 1) { ex->err = "kvm_run_timed_split: n < 1"; return KVM_STATUS_INVALID; }
  if (!ex->uploaded) { int rc = do_upload(ex); if (rc) return rc; }
  std::vector<hipEvent_t> ev(2 * n, nullptr);
  for (auto& e : ev) HIPCK(hipEventCreate(&e));
  HIPCK(hipStreamSynchronize(ex->stream));
  HIPCK(hipEventRecord(ex->ev0, ex->stream));
  int rc = 0;
  for (int i = 0; i < n && !rc; ++i) rc = launch_once(ex, ev[2 * i], ev[2 * i + 1]);
  HIPCK(hipEventRecord(ex->ev1, ex->stream));
  HIPCK(hipEventSynchronize(ex->ev1));
  float tot = 0.f, ex_sum = 0.f;
  if (!rc) {
    HIPCK(hipEventElapsedTime(&tot, ex->ev0, ex->ev1));
    for (int i = 0; i < n; ++i) { float t = 0.f; HIPCK(hipEventElapsedTime(&t, ev[2 * i], ev[2 * i + 1])); ex_sum += t; }
  }
  for (auto& e : ev) hipEventDestroy(e);
  if (rc) return rc;
  *total_ms = tot; *exec_ms = ex_sum;
  ex->launched = true;
  return 0;
}

int kvm_finish(KvmExec* ex, KvmResult* res) {
  hipSetDevice(ex->dev);
  if (ex->streaming && !ex->closed) { if (int rc = kvm_close(ex)) return rc; }
  HIPCK(hipStreamSynchronize(ex->stream));
  KvmCounters c{};
  int done = 0;
  if (ex->S.cnt) {
    HIPCK(hipMemcpy(&c, ex->S.cnt, sizeof c, hipMemcpyDeviceToHost));
    std::vector<int> per(ex->grid);
    HIPCK(hipMemcpy(per.data(), ex->S.done_blk, ex->grid * sizeof(int), hipMemcpyDeviceToHost));
    for (int d : per) done += d;
    if (!c.err_code) done += ex->last_dissolved;   // dissolved no-ops have no work: done once the run completes
  }
  float ms = 0.f;
  if (ex->launched) hipEventElapsedTime(&ms, ex->ev0, ex->ev1);
  if (res) {
    res->err_code = c.err_code; res->err_slot = c.err_slot; res->err_a = c.err_a; res->err_b = c.err_b;
    res->done = done; res->admitted = ex->streaming ? (int)ex->stream_tasks : (int)ex->tasks.size(); res->grid = ex->grid; res->kernel_ms = ms;
  }
  if (c.err_code) { ex->err = "device error " + std::to_string(c.err_code) + " at task " + std::to_string(c.err_slot); return KVM_STATUS_DEVICE_ERROR; }
  return 0;
}

int kvm_versions(KvmExec* ex, int32_t* out, int n) {
  if (!ex->S.version || n > (int)ex->base_versions.size()) { ex->err = "kvm_versions: not started or n too large"; return KVM_STATUS_INVALID; }
  HIPCK(hipStreamSynchronize(ex->stream));
  HIPCK(hipMemcpy(out, ex->S.version, n * sizeof(int), hipMemcpyDeviceToHost));
  return 0;
}

int kvm_trace(KvmExec* ex, KvmTrace* out, int n) {
  if (!ex->S.trace || n > kvm_ntasks(ex)) { ex->err = "kvm_trace: tracing off or n too large"; return KVM_STATUS_INVALID; }
  HIPCK(hipStreamSynchronize(ex->stream));
  HIPCK(hipMemcpy(out, ex->S.trace, n * sizeof(KvmTrace), hipMemcpyDeviceToHost));
  return 0;
}

int kvm_validate(const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs,
                 const MvmBuf* bufs, int nbufs, int nvars, char* err, int errlen) {
  std::string why;
  if (ntasks < 1) why = "empty bundle";
  else if (kvm_validate_bundle(tasks, ntasks, succ, nedges, args, nargs, bufs, nbufs, nvars, &why)) return 0;
  if (err && errlen > 0) snprintf(err, errlen, "%s", why.c_str());
  return KVM_STATUS_INVALID;
}

int kvm_ntasks(const KvmExec* ex) {   // stream mode: the task slots (window w's task i at w * window_tasks + i)
  return ex->streaming ? ex->cfg.window_cap * ex->cfg.window_tasks : (int)ex->tasks.size();
}

int kvm_set_classes(KvmExec* ex, int mode, const KvmClassParams* params, int nclasses) {
  if (ex->uploaded || ex->launched) { ex->err = "kvm_set_classes: before the first kvm_start"; return KVM_STATUS_INVALID; }
  if (mode == KVM_SCHED_GLOBAL) { ex->sched_mode = mode; ex->classes.clear(); return 0; }
  if (mode != KVM_SCHED_STATIC && mode != KVM_SCHED_DYNAMIC) { ex->err = "kvm_set_classes: mode must be KVM_SCHED_GLOBAL, _STATIC or _DYNAMIC"; return KVM_STATUS_INVALID; }
  if (!params || nclasses < 1 || nclasses > KVM_MAX_CLASSES) { ex->err = "kvm_set_classes: 1 to KVM_MAX_CLASSES classes"; return KVM_STATUS_INVALID; }
  for (int c = 0; c < nclasses; ++c) {
    const KvmClassParams& p = params[c];
    const std::string w = "kvm_set_classes: class " + std::to_string(c) + ": ";
    if (p.weight < 1 || p.weight > (1 << 20)) { ex->err = w + "weight must be in [1, 2^20]"; return KVM_STATUS_INVALID; }
    if (p.min_cta < 0) { ex->err = w + "min_cta must be >= 0"; return KVM_STATUS_INVALID; }
    if (p.max_cta < 0) { ex->err = w + "max_cta must be >= 0 (KVM_UNLIMITED for none)"; return KVM_STATUS_INVALID; }
    if (p.bw_cta < 0) { ex->err = w + "bw_cta must be >= 0 (KVM_UNLIMITED for none)"; return KVM_STATUS_INVALID; }
    if (p.urgent_us < 0) { ex->err = w + "urgent_us must be >= 0"; return KVM_STATUS_INVALID; }
    if (p.flags & ~KVM_CLASS_OPAFF) { ex->err = w + "unknown flags"; return KVM_STATUS_INVALID; }
    if (mode == KVM_SCHED_STATIC && p.share < 1) { ex->err = w + "share must be >= 1"; return KVM_STATUS_INVALID; }
  }
  ex->sched_mode = mode;
  ex->classes.assign(params, params + nclasses);
  return 0;
}

int kvm_set_sched_flags(KvmExec* ex, int flags, int bw_limit) {
  if (ex->uploaded || ex->launched) { ex->err = "kvm_set_sched_flags: before the first kvm_start"; return KVM_STATUS_INVALID; }
  if (flags & ~(KVM_SCHED_F_GUARANTEE | KVM_SCHED_F_INHERIT | KVM_SCHED_F_ARBITER)) { ex->err = "kvm_set_sched_flags: unknown flags"; return KVM_STATUS_INVALID; }
  if ((flags & KVM_SCHED_F_ARBITER) && bw_limit < 1) { ex->err = "kvm_set_sched_flags: bw_limit must be >= 1"; return KVM_STATUS_INVALID; }
  ex->sched_flags = flags;
  ex->bw_limit = bw_limit;
  return 0;
}

int kvm_set_affinity(KvmExec* ex, int affinity_us) {
  if (ex->uploaded || ex->launched) { ex->err = "kvm_set_affinity: before the first kvm_start"; return KVM_STATUS_INVALID; }
  if (affinity_us < 0 || affinity_us > 10000000) { ex->err = "kvm_set_affinity: affinity_us must be in [0, 10^7]"; return KVM_STATUS_INVALID; }
  ex->affinity_us = affinity_us;
  return 0;
}

int kvm_class_stats(KvmExec* ex, KvmClassStats* out, int n) {
  if (!ex->S.sched || !ex->launched) { ex->err = "kvm_class_stats: no launch with scheduler classes"; return KVM_STATUS_INVALID; }
  hipSetDevice(ex->dev);
  HIPCK(hipStreamSynchronize(ex->stream));
  std::vector<KvmClsDev> k(ex->S.ncls);
  HIPCK(hipMemcpy(k.data(), ex->S.sched->cls, k.size() * sizeof(KvmClsDev), hipMemcpyDeviceToHost));
  const int m = std::min(n, ex->S.ncls);
  for (int c = 0; c < m; ++c)
    out[c] = KvmClassStats{k[c].tasks, k[c].busy, k[c].resv_starts, k[c].urgent_starts, k[c].missed, k[c].max_running, 0, k[c].boost_starts};
  return m;
}

int kvm_path(const KvmExec* ex) { return ex ? ex->path : KVM_STATUS_INVALID; }

int kvm_static_plan(const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs,
                    int workers, int flags, int* worker_of, int* pos_of, int* nwaits, int* publishes, int* waits, int wait_cap,
                    double* stats, char* err, int errlen) {
  try {
    if (ntasks < 1 || workers < 1 || nedges < 0 || nargs < 0) throw std::invalid_argument("empty graph or no workers");
    std::vector<double> cost(ntasks);
    for (int i = 0; i < ntasks; ++i) {
      if (tasks[i].args_off < 0 || tasks[i].args_off + tasks[i].args_words > nargs || tasks[i].succ_off < 0 ||
          tasks[i].succ_off + tasks[i].succ_cnt > nedges) throw std::invalid_argument("task " + std::to_string(i) + ": range outside the bundle");
      for (int k = 0; k < tasks[i].succ_cnt; ++k) {
        const int s2 = succ[tasks[i].succ_off + k];
        if (s2 < 0 || s2 >= ntasks || s2 == i) throw std::invalid_argument("task " + std::to_string(i) + ": successor out of range");
      }
      cost[i] = task_cost_us(tasks[i], args + tasks[i].args_off);
    }
    const kvms::Plan P = kvms::plan(tasks, ntasks, succ, cost, workers, 1.5, (flags & KVM_PLAN_DISSOLVE) != 0);
    for (int i = 0; i < ntasks; ++i) {
      worker_of[i] = P.worker_of[i]; pos_of[i] = P.pos_of[i]; nwaits[i] = P.wait_off[i + 1] - P.wait_off[i]; publishes[i] = P.publishes[i];
    }
    if ((long long)P.waits.size() > wait_cap) throw std::invalid_argument("more waits than wait_cap");
    for (size_t k = 0; k < P.waits.size(); ++k) { waits[2 * k] = P.waits[k].worker; waits[2 * k + 1] = P.waits[k].need; }
    stats[0] = P.makespan_us; stats[1] = P.work_us; stats[2] = P.cross_edges; stats[3] = P.edges; stats[4] = P.dissolved;
    return 0;
  } catch (const std::exception& e) {
    if (err && errlen > 0) snprintf(err, errlen, "%s", e.what());
    return KVM_STATUS_INVALID;
  }
}

int kvm_set_trace(KvmExec* ex, int on) {
  if (on && !ex->cfg.trace_on) { ex->err = "kvm_set_trace: the executor was created without a trace buffer"; return KVM_STATUS_INVALID; }
  ex->trace_req = on ? 1 : 0;
  ex->S.trace_on = on ? 1 : 0;
  return 0;
}
int kvm_get_trace(const KvmExec* ex) {
  if (!ex) return KVM_STATUS_INVALID;
  return ex->uploaded || ex->streaming ? ex->S.trace_on : (ex->cfg.trace_on && ex->trace_req ? 1 : 0);   // the launch state once it exists
}

const char* kvm_op_name(int op_id) { return kvm_registry_name(op_id); }

// Plain copy, 16 bytes per lane, grid-stride: the reference dispatch for the HBM byte counters (reads n16 * 16 bytes,
// writes as many).
__global__ __launch_bounds__(256) void kvm_copy_probe_kernel(const f32x4n* __restrict__ src, f32x4n* __restrict__ dst, long long n16) {
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n16; i += (long long)gridDim.x * 256) dst[i] = src[i];
}
int kvm_copy_probe(long long bytes) {
  const long long n16 = bytes / 16;
  void *a = nullptr, *b = nullptr;
  if (n16 <= 0 || hipMalloc(&a, n16 * 16) != hipSuccess || hipMalloc(&b, n16 * 16) != hipSuccess) {
    if (a) hipFree(a);
    g_err = "kvm_copy_probe: bad size or hipMalloc failed";
    return KVM_STATUS_HIP_ERROR;
  }
  hipMemset(a, 0, n16 * 16);
  hipLaunchKernelGGL(kvm_copy_probe_kernel, dim3(2048), dim3(256), 0, 0, (const f32x4n*)a, (f32x4n*)b, n16);
  hipError_t e = hipDeviceSynchronize();
  hipFree(a); hipFree(b);
  if (e != hipSuccess) { g_err = hipGetErrorString(e); return KVM_STATUS_HIP_ERROR; }
  return 0;
}

// ---------------------------------------------------------------------------------------------- allocation-free run
// All device memory of kvm_run_noalloc's scheduler state and task graph: one file-scope array per GPU, held until the
// process ends. In host code `scratch` only names the symbol; its device address comes from hipGetSymbolAddress, once
// per device, and only that address is ever passed to kernels or copies.
static __device__ __align__(256) unsigned char scratch[KVM_NOALLOC_SCRATCH_BYTES];
#define KVM_MAX_DEVICES 64
static void* g_scratch_ptr[KVM_MAX_DEVICES];
static int g_scratch_cus[KVM_MAX_DEVICES];
static int g_scratch_cap[KVM_MAX_DEVICES];   // co-resident worker capacity (resident_capacity)
static std::mutex g_scratch_mu[KVM_MAX_DEVICES];

static int scratch_setup(int dev, std::string& err) {
  if (g_scratch_ptr[dev]) return 0;
  void* ptr = nullptr;
  hipError_t e = hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) { err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e); return KVM_STATUS_HIP_ERROR; }
  int cus = 0;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess || cus < 1) { err = "hipDeviceGetAttribute(multiprocessor count) failed"; return KVM_STATUS_HIP_ERROR; }
  const int cap = resident_capacity(cus, err);
  if (cap < 0) return KVM_STATUS_INVALID;
  g_scratch_cus[dev] = cus;
  g_scratch_cap[dev] = cap;
  g_scratch_ptr[dev] = ptr;
  return 0;
}

int kvm_run_noalloc(const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs,
                    const MvmBuf* bufs, int nbufs, int32_t* versions, int nvars, int blocks, unsigned long long timeout_us,
                    void* stream, KvmResult* res, char* errbuf, int errlen) {
  std::string err;
  auto fail = [&](int rc) { if (errbuf && errlen > 0) snprintf(errbuf, errlen, "%s", err.c_str()); return rc; };
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= KVM_MAX_DEVICES) { err = "no current HIP device"; return fail(KVM_STATUS_HIP_ERROR); }
  if (ntasks < 1 || nedges < 0 || nargs < 0 || nbufs < 0 || nvars < 1 || !versions || blocks < 0) { err = "bad sizes"; return fail(KVM_STATUS_INVALID); }
  if (!kvm_validate_bundle(tasks, ntasks, succ, nedges, args, nargs, bufs, nbufs, nvars, &err)) return fail(KVM_STATUS_INVALID);
  for (int i = 0; i < nbufs; ++i) if (!bufs[i].p) { err = "buffer " + std::to_string(i) + " has no device address"; return fail(KVM_STATUS_INVALID); }
  std::lock_guard<std::mutex> lock(g_scratch_mu[dev]);   // calls on one device in this process never overlap
  if (int rc = scratch_setup(dev, err)) return fail(rc);
  if (blocks > g_scratch_cap[dev]) {
    err = "blocks " + std::to_string(blocks) + " exceeds the co-resident capacity of the device (" + std::to_string(g_scratch_cap[dev]) + ")";
    return fail(KVM_STATUS_INVALID);
  }
  const int grid = blocks > 0 ? blocks : g_scratch_cus[dev];
  std::vector<MvmTaskDesc> tv(tasks, tasks + ntasks);
  std::vector<int32_t> sv(succ, succ + nedges), av(args, args + nargs), roots;
  for (int i = 0; i < ntasks; ++i) { tv[i].reserved0 = 0; if (tv[i].indegree == 0) roots.push_back(i); }
  std::vector<MvmBuf> table(bufs, bufs + nbufs);
  GraphPlan g;
  plan_graph(tv, sv, av, table, roots, grid, 0, g);
  unsigned char* base = (unsigned char*)g_scratch_ptr[dev];
  size_t used = 0;
  auto bump = [&](size_t bytes) -> void* {
    const size_t at = (used + 255) & ~(size_t)255;
    if (at + bytes > (size_t)KVM_NOALLOC_SCRATCH_BYTES) return nullptr;
    used = at + bytes;
    return base + at;
  };
  KvmDevState S; LaunchArgs L;
  hipStream_t st = (hipStream_t)stream;
  int rc = place_graph(g, tv, nvars, grid, false, 0, timeout_us, bump, st, S, L, err, false);   // sizing pass
  if (rc == KVM_STATUS_TOO_BIG) {
    err = "task graph needs more than the " + std::to_string(KVM_NOALLOC_SCRATCH_BYTES >> 20) + " MiB of kvm_run_noalloc's device scratch";
    return fail(KVM_STATUS_TOO_BIG);
  }
  used = 0;
  if ((rc = place_graph(g, tv, nvars, grid, false, 0, timeout_us, bump, st, S, L, err))) return fail(rc);
  hipError_t e = hipMemcpyAsync(L.base, versions, nvars * sizeof(int), hipMemcpyHostToDevice, st);
  if (e == hipSuccess) { launch_graph(S, L, grid, st, nullptr, nullptr); e = hipGetLastError(); }
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  KvmCounters c{};
  std::vector<int> per(grid);
  if (e == hipSuccess) e = hipMemcpyAsync(&c, S.cnt, sizeof c, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipMemcpyAsync(per.data(), S.done_blk, grid * sizeof(int), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipMemcpyAsync(versions, S.version, nvars * sizeof(int), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) { err = std::string("kvm_run_noalloc: ") + hipGetErrorString(e); return fail(KVM_STATUS_HIP_ERROR); }
  int done = 0;
  for (int d : per) done += d;
  if (res) {
    res->err_code = c.err_code; res->err_slot = c.err_slot; res->err_a = c.err_a; res->err_b = c.err_b;
    res->done = done; res->admitted = ntasks; res->grid = grid; res->kernel_ms = 0.f;
  }
  if (c.err_code) { err = "device error " + std::to_string(c.err_code) + " at task " + std::to_string(c.err_slot); return fail(KVM_STATUS_DEVICE_ERROR); }
  return 0;
}

int kvm_seeded_fill_test(unsigned long long seed, long long n, int draws, float bias, float coef, float* out) {
  float* d = nullptr;
  if (hipMalloc(&d, std::max<long long>(n, 1) * 4) != hipSuccess) { g_err = "hipMalloc failed"; return KVM_STATUS_HIP_ERROR; }
  hipLaunchKernelGGL(kvm_seeded_kernel, dim3(64), dim3(256), 0, 0, d, n, seed, draws, bias, coef);
  hipError_t e = hipMemcpy(out, d, n * 4, hipMemcpyDeviceToHost);
  hipFree(d);
  if (e != hipSuccess) { g_err = hipGetErrorString(e); return KVM_STATUS_HIP_ERROR; }
  return 0;
}

}  // extern "C"
