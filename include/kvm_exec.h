// C ABI of the MI355X persistent task-graph executor (libkvm_exec.so).
//
// It replaces the reference's host executor class MvmExec (reference: mvm_exec.cu:492-1560) for one GPU: the caller
// creates an executor, declares the buffer table, submits one or more ABI-v2 bundles, starts the persistent kernel and
// collects the result. Plain pointers and sizes only; every function returns 0 (or a non-negative index) on success
// and a negative KvmStatus on failure, with a message in kvm_last_error().
#ifndef KVM_EXEC_H
#define KVM_EXEC_H
#include <stddef.h>
#include <stdint.h>
#include "mvm_task_abi.h"

// Task priorities are 0..KVM_PRIORITIES-1, larger first among ready tasks (reference: MVM_NBUCKETS, mvm_exec.cuh:51-52).
#define KVM_PRIORITIES 32
// Scheduler classes (reference: MVM_MAX_CLS, MVM_UNLIMITED, include/mvm_sched.h:19-20).
#define KVM_MAX_CLASSES 8
#define KVM_UNLIMITED 0x7fffffff

#ifdef __cplusplus
extern "C" {
#endif

// Submit / call status (reference: MvmSubmit, mvm_exec.cu:410-413).
enum KvmStatus {
  KVM_STATUS_OK = 0, KVM_STATUS_BACKPRESSURE_TIMEOUT = -1, KVM_STATUS_TOO_BIG = -2, KVM_STATUS_DEVICE_ERROR = -3,
  KVM_STATUS_CLOSED = -4, KVM_STATUS_INVALID = -5, KVM_STATUS_HIP_ERROR = -6,
};

// Executor sizing and behaviour (reference: MvmConfig, mvm_exec.cu:367-408; the fields this executor uses).
typedef struct KvmConfig {
  int blocks;                  // persistent workgroups; 0 = one per CU
  int trace_on;                // 1: per-task timeline and execution witness (KvmTrace per task)
  int num_vars;                // version variables
  unsigned long long timeout_us;   // stall timeout: no task finished for this long while work is pending
  int device;                  // HIP device ordinal
  int aging_us;                // 0: strict priority among ready tasks; else a ready task gains one priority level per
                               //   aging_us of waiting (reference: MvmConfig::aging_us, mvm_exec.cu:375)
  int path;                    // KVM_PATH_*: dynamic scheduler, static per-worker programs, or chosen per graph
                               //   (reference: the --static / --dynamic path choice, mvm_exec.cu:2146-2164)
  // Stream mode (window_cap > 0; reference: live_cap / win_cap / succ_cap and submit while running, mvm_exec.cu:
  // 367-408, 742-889): kvm_start launches the persistent kernel at once and each kvm_submit admits one bundle into one
  // of window_cap window slots of window_tasks tasks and window_edges successor edges while it runs; a slot is reused
  // once its window has finished. Dynamic FIFO scheduling (no static path, no priority buckets).
  int window_cap;
  int window_tasks;
  int window_edges;
  int backpressure_ms;         // how long kvm_submit waits for a free window slot before KVM_STATUS_BACKPRESSURE_TIMEOUT
} KvmConfig;

// Execution paths. DYNAMIC: ready queues and dependency counters. STATIC: the graph is planned on the host into one
// program per worker (list scheduling), cross-worker dependencies are waits on progress watermarks (needs every
// version wait decided inside the graph). AUTO: STATIC when the graph allows it and its mean estimated task cost is at
// most KVM_STATIC_MAX_MEAN_US (short tasks, where queue and counter overheads dominate), else DYNAMIC. With the fitted
// task costs the graphs measured faster on the static path have means of 3-10 us (decode, tiny GPT, 8 MLPs) and those
// faster on the dynamic path 21 us and up (GPT-162M 22.3, 11.1 ms on the static path against 8.9 dynamic).
enum KvmPath { KVM_PATH_DYNAMIC = 0, KVM_PATH_STATIC = 1, KVM_PATH_AUTO = 2 };
#define KVM_STATIC_MAX_MEAN_US 15.0

// Buffer initialisation (reference: MvmInit, mvm_exec.cu:431-437).
enum KvmInitKind { KVM_INIT_ZERO = 0, KVM_INIT_FILL = 1, KVM_INIT_VALUES = 2, KVM_INIT_SEEDED = 3 };
typedef struct KvmInit {
  int kind;
  float value;                 // FILL (f32/bf16 value; i32 buffers take it as an integer)
  const void* values;          // VALUES: rows*cols elements in the buffer's dtype (bf16 as raw uint16)
  unsigned long long seed;     // SEEDED: SplitMix64 generator parameters as in the bundle metadata (bf16 buffers: each value
                               //   rounded once to bf16, this executor's extension for bf16 weights)
  int draws;
  float bias, coef;
} KvmInit;

// One task's timeline (reference: MvmTrace, mvm_exec.cuh:167-174). Times are wall_clock64 ticks (100 MHz).
typedef struct KvmTrace {
  unsigned long long start, end;
  int block, xcc, ver0, ver1;  // ver0/ver1: version of the task's wait variable at start / end (-1 none)
  int exec_count;              // times the task ran (the exactly-once witness)
  int how;                     // scheduler classes on: KVM_TRACE_* bits of how the task was started and ended
} KvmTrace;
// KvmTrace.how bits (reference: MVM_TRACE_MISSED / _RESV / _URGENT, include/mvm_sched.h:33-36).
#define KVM_TRACE_MISSED 1     // finished after its deadline
#define KVM_TRACE_RESV 2       // started while its class was below its reservation
#define KVM_TRACE_BOOST 4      // started under priority inheritance
#define KVM_TRACE_URGENT 8     // started by the deadline (EDF) tier

typedef struct KvmResult {
  int err_code, err_slot, err_a, err_b;   // first device error (0 none)
  int done, admitted, grid;
  float kernel_ms;
} KvmResult;

typedef struct KvmExec KvmExec;

void kvm_config_default(KvmConfig* cfg);
// Creates an executor on cfg->device. Returns NULL on failure (message in kvm_last_error(NULL)).
KvmExec* kvm_create(const KvmConfig* cfg);
void kvm_destroy(KvmExec* ex);
const char* kvm_last_error(const KvmExec* ex);

// Appends a buffer to the table (reference: MvmExec::add_buffer, mvm_exec.cu:582). dtype 0 f32, 1 i32, 2 bf16.
// Returns the buffer index (dense, ascending).
int kvm_add_buffer(KvmExec* ex, int rows, int cols, int dtype, const KvmInit* init);
int kvm_nbufs(const KvmExec* ex);
int kvm_buffer_dtype(const KvmExec* ex, int idx);
// Device address of a buffer (for callers that share it with their own kernels), or NULL.
void* kvm_buffer_device_ptr(const KvmExec* ex, int idx);
// Overwrites a buffer with host data of its own dtype (bytes = rows*cols*element size).
int kvm_write_buffer(KvmExec* ex, int idx, const void* host, size_t bytes);
// Reads a buffer widened to f32 (i32 buffers: raw int32 bit patterns) (reference: read_buffer, mvm_exec.cu:1542-1553).
int kvm_read_buffer(KvmExec* ex, int idx, float* out, size_t n);
// Reads a buffer in its own dtype (bf16 as uint16).
int kvm_read_raw(KvmExec* ex, int idx, void* out, size_t bytes);

// Sets a version variable's value before start (reference: set_version).
int kvm_set_version(KvmExec* ex, int var, int version);
// Adds one bundle (reference: MvmExec::submit, mvm_exec.cu:742): its tasks' successor indices are bundle-local.
// The host validates descriptors, arities, buffer indices/dtypes and operand extents; KVM_STATUS_INVALID on failure.
// Bundles submitted before kvm_start run in one launch and share state only through version variables. Stream mode:
// also while the kernel runs; returns the bundle's window id (>= 0), KVM_STATUS_TOO_BIG when it exceeds a window and
// KVM_STATUS_BACKPRESSURE_TIMEOUT when no slot frees up within backpressure_ms.
int kvm_submit(KvmExec* ex, const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges,
               const int32_t* args, int nargs);
// Uploads the task graph, resets the scheduler state and launches the persistent kernel (asynchronous). Stream mode:
// launches the kernel with empty window slots and admits the bundles submitted so far.
int kvm_start(KvmExec* ex);
// Stream mode: no bundle follows (reference: MvmExec::close, mvm_exec.cu:1505). The kernel ends once every admitted
// task has finished; kvm_finish closes first when the caller has not.
int kvm_close(KvmExec* ex);
// Stream mode: the version variables as the device has published them so far (a pinned mirror, readable while the
// kernel runs; reference: live_versions).
int kvm_live_versions(KvmExec* ex, int32_t* out, int n);
// Stream mode: 1 when window `wid` (the non-negative value kvm_submit returned) has finished, 0 when not yet.
int kvm_window_done(KvmExec* ex, long long wid);
// Stream mode: one bundle larger than a window, in consecutive windows of at most max_window_tasks tasks (0: the slot
// size). Task order must be topological (every edge to a higher index). Edges inside a window are device edges; a
// window with a predecessor in an earlier window is submitted once that window has finished (the host waits, up to
// timeout_ms per window). Returns the number of windows, or a negative status (reference: submit_stream,
// mvm_exec.cu:830-889).
int kvm_submit_stream(KvmExec* ex, const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges,
                      const int32_t* args, int nargs, int max_window_tasks, int timeout_ms);
// Waits for the launch, then fills `res` (reference: close/finish, mvm_exec.cu:1505-1540).
int kvm_finish(KvmExec* ex, KvmResult* res);
// Runs the whole submitted graph again on the current buffer contents (versions restart from their set values):
// reset + launch, asynchronous. Used for repeated training steps / decode tokens; kvm_finish collects it.
int kvm_relaunch(KvmExec* ex);
// Launches `n` back-to-back runs without host synchronisation in between and returns the elapsed milliseconds
// measured with HIP events around them (the timed region of the benchmark). Result of the last run via kvm_finish.
int kvm_run_timed(KvmExec* ex, int n, float* ms);
// As kvm_run_timed, and also the summed duration of the n persistent-kernel launches alone (HIP events on the
// executor's stream right before and after each launch, i.e. without the per-launch state reset). No counterpart in
// the reference; for benchmarks that report a kernel's own duration.
int kvm_run_timed_split(KvmExec* ex, int n, float* total_ms, float* exec_ms);

// Host-only validation of one bundle against a buffer table (shapes and dtypes in `bufs`; `p` unused): the checks
// kvm_submit runs. Returns 0 when valid, else KVM_STATUS_INVALID with the reason in `err`. Needs no GPU.
int kvm_validate(const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs,
                 const MvmBuf* bufs, int nbufs, int nvars, char* err, int errlen);

int kvm_versions(KvmExec* ex, int32_t* out, int n);
int kvm_trace(KvmExec* ex, KvmTrace* out, int n);
int kvm_ntasks(const KvmExec* ex);
// Turns the per-task trace on or off for the following launches (an executor created with trace_on keeps its trace
// buffer; tracing costs a read-modify-write at every task start). No counterpart in the reference, whose trace is
// fixed at creation; for benchmarks that time untraced runs and trace one more.
int kvm_set_trace(KvmExec* ex, int on);
// Whether the next launch traces (1) or not (0): the last kvm_set_trace, else the creation's trace_on. No counterpart
// in the reference (see kvm_set_trace).
int kvm_get_trace(const KvmExec* ex);
// Name of a registry operator id, or NULL (reference: --check-ops).
const char* kvm_op_name(int op_id);
// Fills `out` with n SplitMix64 seeded values on the device and copies them back (initialiser known-answer test).
int kvm_seeded_fill_test(unsigned long long seed, long long n, int draws, float bias, float coef, float* out);
// Copies `bytes` bytes between two fresh device buffers with a plain 16-byte-per-lane kernel and waits for it. No
// counterpart in the reference: a dispatch of known HBM traffic for calibrating byte counters (rocprofv3 FETCH_SIZE /
// WRITE_SIZE) against the executor's own dispatches.
int kvm_copy_probe(long long bytes);

// The static planner alone, on the host (no GPU): plans the bundle for `workers` workers exactly as KVM_PATH_STATIC does
// at upload (flags KVM_PLAN_DISSOLVE: as untraced launches do, with the ordering no-ops dissolved). Outputs
// (caller-sized): worker_of[ntasks], pos_of[ntasks] (index in the worker's program; both -1 for a dissolved no-op),
// nwaits[ntasks] (cross-worker waits kept after reduction), publishes[ntasks], and the waits as (worker, need) pairs in
// task order into waits[2 * wait_cap] (a task's waits follow the previous task's). A pair (-1 - count, start) is a
// reference to a dissolved no-op's wait set: the `count` pairs from pair index `start`, stored after every task's list.
// stats[5] = predicted makespan us, summed cost us, cross-worker edges, DAG edges, no-ops dissolved. Returns 0, or
// KVM_STATUS_INVALID (reason in err; also when the pairs exceed wait_cap). No counterpart in the reference as a C entry
// (its planner is mvm_static_plan, include/mvm_static.h; the dissolving transform mvm_dissolve_noops,
// mvm_exec.cu:212-296); for tests and tooling.
#define KVM_PLAN_DISSOLVE 1
int kvm_static_plan(const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs,
                    int workers, int flags, int* worker_of, int* pos_of, int* nwaits, int* publishes, int* waits, int wait_cap,
                    double* stats, char* err, int errlen);
// Scheduler classes (reference: MvmSchedCfg / MvmClassParams, include/mvm_sched.h:24-49, 112-121; the CLI's --sched,
// --classes, --weights, --min, --max, --urgent-us, --shares, mvm_exec.cu:1940-1952). A task's class is its
// workload_id (0 .. nclasses-1). Modes: KVM_SCHED_GLOBAL = off (one set of queues, the default). KVM_SCHED_DYNAMIC:
// per-class ready queues; a worker serves, in this order, a class below its reservation (running < min_cta), then a
// task whose deadline is within urgent_us (earliest deadline first; deadline_us counts from the launch), then the class
// with the least weighted worker-time (ticks run / weight) among those below their cap (running < max_cta). The cap is
// a hard bound on the class's concurrently running tasks outside its reservation. KVM_SCHED_STATIC: the workers are
// split among the classes in proportion to `share` and each serves only its own class. Priorities and aging order
// the tasks inside a class. Set before the first kvm_start; the launches run the dynamic path. In stream mode (the
// reference's admission path, where classes are the reason it exists) each class has one FIFO ring per queue group:
// priorities do not reorder tasks inside a class there, and deadline_us counts from the admission of the task's window.
enum KvmSchedMode { KVM_SCHED_GLOBAL = 0, KVM_SCHED_STATIC = 1, KVM_SCHED_DYNAMIC = 2 };
typedef struct KvmClassParams {
  int weight;                  // >= 1: relative share of worker-time among competing classes
  int min_cta;                 // reservation: workers the class is served first up to (0 none)
  int max_cta;                 // cap on running tasks (KVM_UNLIMITED none; 0: only reservations and inheritance start them)
  int urgent_us;               // EDF window: a ready task whose deadline is this close is served first (0 off)
  int share;                   // KVM_SCHED_STATIC: relative number of workers (>= 1)
  int bw_cta;                  // cap on the class's running bandwidth-bound tasks (KVM_UNLIMITED none)
  int flags;                   // KVM_CLASS_OPAFF: op affinity (with an affinity window, kvm_set_affinity)
} KvmClassParams;
// A task of the class released by a finishing task prefers the worker that last finished a task of its operator
// (warm code and caches) instead of the releasing worker (reference: MVM_CF_OPAFF, include/mvm_sched.h:34).
#define KVM_CLASS_OPAFF 2
int kvm_set_classes(KvmExec* ex, int mode, const KvmClassParams* params, int nclasses);
// Policy switches of KVM_SCHED_DYNAMIC (reference: MvmSchedParams.flags and MVM_SF_*, include/mvm_sched.h:26-33, default
// MVM_SF_DEFAULT = reservations + inheritance). KVM_SCHED_F_GUARANTEE: reservations are served first. KVM_SCHED_F_INHERIT:
// priority inheritance across version waits: while a task of class W is parked on a variable that a task of class C
// publishes, C is boosted (transitively: C's own parked tasks boost their publishers' classes); a boosted class is served
// before the reservations and ignores its caps, so a throttled publisher cannot hold a waiter back. KVM_SCHED_F_ARBITER:
// at most bw_limit bandwidth-bound tasks of all classes run at once outside reservations and boosts (the reference adapts
// this limit online from protected classes' queue waits; here it is fixed). A task is bandwidth-bound when its operator
// streams memory (the reference's cost table, include/mvm_ops_cost.inc, restated for the operators implemented here) and
// it moves at least 16 KiB. Default: GUARANTEE | INHERIT. Set before the first kvm_start.
#define KVM_SCHED_F_GUARANTEE 1
#define KVM_SCHED_F_INHERIT 2
#define KVM_SCHED_F_ARBITER 4
int kvm_set_sched_flags(KvmExec* ex, int flags, int bw_limit);
// Task affinity window of the class scheduler (reference: MvmSchedParams.affinity_us, include/mvm_sched.h:55): a ready
// task released by a finishing task is offered only to its preferred worker (the releasing one, or with
// KVM_CLASS_OPAFF the one that last ran its operator) for affinity_us after its release, then to every worker.
// Roots have no preferred worker. 0 (the default) = off. Set before the first kvm_start; with scheduler classes only. With
// a window the class queues form one group that every worker polls (no per-XCD queue groups), as in the reference.
int kvm_set_affinity(KvmExec* ex, int affinity_us);
// Per-class counters of the last launch (reference: MvmClassTele, include/mvm_sched.h:59-66). Times in
// wall_clock64 ticks (100 MHz).
typedef struct KvmClassStats {
  unsigned long long tasks, busy_ticks, resv_starts, urgent_starts, missed;
  int max_running, pad;
  unsigned long long boost_starts;   // tasks started under priority inheritance
} KvmClassStats;
int kvm_class_stats(KvmExec* ex, KvmClassStats* out, int n);

// The path a launch of this executor uses (KVM_PATH_DYNAMIC or KVM_PATH_STATIC; decided at the first start), or < 0.
int kvm_path(const KvmExec* ex);

// Device scratch of kvm_run_noalloc: one array per GPU the library runs on, held until the process ends.
#define KVM_NOALLOC_SCRATCH_BYTES (32u << 20)
// Runs one bundle to completion on the current HIP device without allocating device memory: no hipMalloc, hipFree or
// allocating library call. No counterpart in the reference; for callers that cannot allocate (code under HIP graph
// capture, serving loops, harnesses that forbid it). The caller owns the buffers: `bufs[i].p` are device addresses,
// rows/cols/dtype as in kvm_add_buffer. `versions` holds the nvars base versions on entry and the final versions on
// return. The scheduler state, queues and task graph live in the library's KVM_NOALLOC_SCRATCH_BYTES of scratch: a
// graph that needs more is refused with KVM_STATUS_TOO_BIG before anything runs. Validation as kvm_submit; tracing off.
// blocks 0 = one workgroup per CU; `stream` a hipStream_t or NULL (the null stream). Synchronous: returns after the
// run with `res` filled (kernel_ms 0). Every call on one GPU shares that GPU's scratch and clears what must start at
// zero; calls from one process are serialised per device, calls that overlap on one GPU from elsewhere would race.
int kvm_run_noalloc(const MvmTaskDesc* tasks, int ntasks, const int32_t* succ, int nedges, const int32_t* args, int nargs,
                    const MvmBuf* bufs, int nbufs, int32_t* versions, int nvars, int blocks, unsigned long long timeout_us,
                    void* stream, KvmResult* res, char* err, int errlen);

#ifdef __cplusplus
}
#endif
#endif
