// rt_shared.h — launch-shape constants that the kernels and the host runtime
// must agree on.  Plain C++ (no HIP types): included by the device sources
// and by runtime.cpp, so a grid and the kernel it launches cannot disagree.
#pragma once
#include <stdint.h>

// Decode attention: query heads per workgroup at a head size.  Head sizes 64
// and 128 take 1: a group of 7 query heads spreads over 7 workgroups per KV
// head and split, each thread's score chain one head long (0.5B step: 690 →
// 667 µs, 7B step: 1889 → 1846 µs against 8 and 4 heads per workgroup);
// head size 256 takes 8.
constexpr uint32_t rt_attn_gm(uint32_t head_dim) { return head_dim == 256 ? 8u : 1u; }
// Head groups of 256 threads per workgroup: one (groups share the query heads
// of their workgroup, so one head leaves one group; head size 256 is bound to
// one by its registers).
constexpr uint32_t rt_attn_hg(uint32_t) { return 1u; }
// The persistent step's attention phase runs RT_STEP_THREADS / 256 = 2 head
// groups, so its workgroups take 2 query heads (step 772 → 753 µs against 8).
constexpr uint32_t rt_step_attn_gm(uint32_t) { return 2u; }
// Multi-query (verify / prefill) attention on the matrix cores: the most
// waves a workgroup of 16 query columns may have at a head size.
constexpr uint32_t rt_attn_mq_wmax(uint32_t head_dim) { return head_dim == 256 ? 4u : 8u; }
// Key ranges of one column group merged by its last workgroup (at most).
constexpr uint32_t RT_ATTN_MQ_NSP_MAX = 8;
// LDS bytes of such a workgroup of w waves: per wave 16 columns × head_dim
// outputs + 16 maxima + 16 sums.
constexpr uint32_t rt_attn_mq_lds(uint32_t head_dim, uint32_t w) { return w * (16u * head_dim + 32u) * 4u; }

// Device scratch of the no-allocation entry points: one fixed array in the
// code object (k_scratch.hip), laid out as [arrival counters | activation
// workspace | K-split partial sums].
constexpr uint64_t RT_SCRATCH_BYTES = 4ull << 20;
constexpr uint64_t RT_SCRATCH_COUNTER_BYTES = 56ull << 10;  // as the context's counter area
constexpr uint64_t RT_SCRATCH_WS_OFF = 64ull << 10;
constexpr uint64_t RT_SCRATCH_WS_BYTES = 1ull << 20;
constexpr uint64_t RT_SCRATCH_PART_OFF = RT_SCRATCH_WS_OFF + RT_SCRATCH_WS_BYTES;
constexpr uint64_t RT_SCRATCH_PART_BYTES = RT_SCRATCH_BYTES - RT_SCRATCH_PART_OFF;

// Persistent decode step (k_step.hip): phase record size and the most
// workgroups a step grid may have.
constexpr uint32_t RT_STEP_PHASE_BYTES = 400;
constexpr uint32_t RT_STEP_MAX_WGS = 1024;
// threads per workgroup of the persistent step (its attention phase runs
// RT_STEP_THREADS / 256 head groups)
#define RT_STEP_THREADS 512
constexpr uint32_t RT_STEP_SYNC_BYTES = 2048;  // StepSync (k_step.hip)
constexpr uint32_t RT_STEP_STATUS_OFF = 1280;  // its status word
