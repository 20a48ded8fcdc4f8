#pragma once
// Task ABI, version 2: the binary contract between a bundle (tasks.bin / successors.bin / args.bin / metadata.json)
// and this executor. Identical in field order, width and meaning to the reference's descriptor
// (reference: include/mvm_task_abi.h:11-39) so bundles compiled for it run here unchanged.
// All fields are little-endian int32.
#include <stdint.h>

#define MVM_ABI_VERSION 2
#define MVM_NO_VAR (-1)

typedef struct MvmTaskDesc {
    int32_t op_id;        // operator id (mvm_ops*.def)
    int32_t succ_off;     // first successor in successors.bin (bundle-local task indices)
    int32_t succ_cnt;     // number of successors
    int32_t indegree;     // number of in-bundle predecessors
    int32_t priority;     // larger first among ready tasks (scheduling hint)
    int32_t deadline_us;  // -1 none (scheduling hint)
    int32_t args_off;     // first argument word in args.bin
    int32_t args_words;   // equals the operator's arity
    int32_t wait_var;     // MVM_NO_VAR, or run only once version[wait_var] >= wait_ver
    int32_t wait_ver;
    int32_t pub_var;      // MVM_NO_VAR, or on completion version[pub_var] goes from pub_ver-1 to pub_ver
    int32_t pub_ver;
    int32_t workload_id;  // graph index inside the workload (metrics only)
    int32_t flags;        // 0
    int32_t reserved0;
    int32_t reserved1;
} MvmTaskDesc;

// One entry of the device buffer table. Operators reach memory only through table indices in their arguments.
typedef struct MvmBuf {
    void*   p;
    int32_t rows, cols, ld;
    int32_t dtype;        // 0 f32, 1 i32, 2 bf16 storage (2 bytes per element)
    int32_t reserved[2];
} MvmBuf;

#ifdef __cplusplus
static_assert(sizeof(MvmTaskDesc) == 64, "task descriptor is 64 bytes");
static_assert(sizeof(MvmBuf) == 32, "buffer table entry is 32 bytes");
#endif
