// Host/device interface of the fused verification kernel (verify.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

constexpr int kMaxSpecLen = 128;  // reference MAX_SPEC_LEN, rejection_sampler.py:83
constexpr int kMaxQueues = 16;    // work queues of the split verify kernel
#ifndef MVSD_VERIFY_THREADS
#define MVSD_VERIFY_THREADS 512
#endif
constexpr int kVThreads = MVSD_VERIFY_THREADS;  // verify-kernel workgroup size
constexpr int kVWaves = kVThreads / 64;

// Kernel parameters, passed by value.  Pointers are device pointers; strides are in
// elements.  The workspace pointers are carved by the host from one caller buffer.
struct VerifyParams {
  int32_t* out;
  int64_t out_stride;
  const void* target;
  int64_t target_stride;
  const int32_t* target_rows;
  int64_t target_num_rows;
  const float* draft;
  int64_t draft_stride;
  const float* noise;
  int64_t noise_stride;
  const double* uniforms;
  const int32_t* draft_ids;
  const int32_t* cu;
  const int32_t* bonus;
  const float* temperature;
  const int32_t* recovered;
  const float* synth;
  int target_dtype;
  int all_greedy;
  int apply_temperature;
  int B;
  int P;
  int V;
  int max_spec_len;
  int chunk;  // vocab columns per task (a multiple of the sub-chunk)
  int nc;     // chunks per row
  int G;      // rows per group
  int lag;        // groups between a group's A-chunks and its B-chunks in ticket order
  int two_phase;  // the batch has random requests that need B-chunks
  bool target_aligned;
  bool draft_aligned;
  bool noise_aligned;
  // workspace
  int* ctrl;             // [0] ticket, [1] sticky spin-limit flag, [2] exit counter
  int* grp_off;          // [B + 1] exclusive scan of groups per request
  int4* grp_desc;        // [P] per group: request, first row, rows | groups << 8 | flags << 16,
                         //     bits of log2(e) / T   (flags: 1 greedy, 2 needs recovered scores)
  int* req_cnt;          // [B] finished tasks per request (zero between calls)
  // Work queues of the split kernel: request r belongs to queue r % nq, and workgroup w
  // serves queue w % nq (workgroups are dispatched round-robin over the XCDs, so a queue's
  // tasks share one L2).  qgi lists each queue's groups in request order.
  int nq;
  int* qticket;          // [nq] ticket counters
  int* qcount;           // [nq] groups per queue
  int* qoff;             // [nq] offset of each queue's list in qgi
  int* qgi;              // [groups] group indices, queue-major
  uint64_t* stat_slots;  // [P * nc] packed (chunk max, chunk sumexp); 0 = empty
  uint64_t* arg_slots;   // [P * nc] packed (chunk argmax value, index + 1); 0 = empty
};

struct VerifyPlan {
  int ept;    // elements per thread per row in one sub-chunk
  int g;      // rows per group
  int sub;    // columns per sub-chunk (threads * ept)
  int nsub;   // sub-chunks per row; upper bound of nc (sizes the workspace)
  int chunk;  // columns per task, a multiple of sub
  int nc;     // chunks per row
};

// groups = 0 gives the workspace-sizing plan (nc = nsub).  phases is 2 when the batch needs
// recovered scores (stats and score tasks per chunk), else 1; cap = resident workgroups.
VerifyPlan verify_plan(int target_dtype, int64_t vocab_size, int64_t groups, int phases, int cap);
// fused: the single-read kernel (one sub-chunk per task, scores computed by the workgroup that
// loaded the target chunk); otherwise the split kernel (stats tasks, then score tasks that
// re-read the target).
const void* verify_kernel_ptr(int target_dtype, bool fused, bool has_draft);
hipError_t launch_zero_fill(void* p, int64_t bytes, hipStream_t stream);
hipError_t launch_verify(const VerifyParams& params, int target_dtype, bool fused, int grid,
                         hipStream_t stream);

}  // namespace mvsd
