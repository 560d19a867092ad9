// Host/device interface of the fused verification kernel (verify.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

constexpr int kMaxSpecLen = 128;  // reference MAX_SPEC_LEN, rejection_sampler.py:83
constexpr int kMaxQueues = 16;    // work queues of the split verify kernel
constexpr int kMaxLdsRequests = 4096;  // requests whose group offsets fit the kernel's LDS
constexpr int kMaxFusedRequests = 2048;  // requests whose metadata fit the fused kernel's LDS
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
  int4* grp_desc;        // [P] per group: request, first row, rows | groups << 8 | flags << 16
                         //     | index within the request << 24, bits of log2(e) / T
                         //     (flags: 1 greedy, 2 needs recovered scores)
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
  uint64_t* arg_slots;   // [P * arg_stride] packed (chunk argmax value, index + 1); 0 = empty
  // Epilogue split of the split kernel: the score tasks of the last `lag` groups (whose steps
  // hold no stats tasks) cover half chunks, 2 * nc per row, so the final tasks are short.
  int split;
  // With the split, the score tasks of the last `quarter` groups (<= lag) cover quarter chunks,
  // 4 * nc per row, so the very last tasks are shorter still.
  int quarter;
  int arg_stride;  // arg slots per row: 4 * nc with quarters, 2 * nc with the split, else nc
  // Split kernel without the init kernel: every workgroup builds the requests' group offsets
  // in its own LDS and derives group descriptors from them (one queue, B <= kMaxLdsRequests);
  // grp_off / grp_desc are then unused.
  int lds_groups;
  // Sampling constraints (top-k / top-p per request, either may be null).  When set, the
  // constraints kernel writes one row mask per verify row, (A, B, J as bits, 0): entry i of
  // the row, raw value x, is masked iff x < A || (x < B && i <= J).
  const int64_t* top_k;  // [B]
  const float* top_p;    // [B]
  float4* masks;         // [P], null when no constraint applies
};

// Verify row j's row in the target tensor: target_rows[j] clamped to the tensor, or j.
__device__ inline int64_t target_row(const VerifyParams& p, int row) {
  if (!p.target_rows) return row;
  const int64_t t = p.target_rows[row];
  return t < 0 ? 0 : (t >= p.target_num_rows ? p.target_num_rows - 1 : t);
}

__device__ inline bool req_is_greedy(const VerifyParams& p, int r) {
  return p.all_greedy || p.temperature[r] == 0.f;
}

// Temperature applied to request r's rows: 1 unless apply_temperature; 0 (greedy) -> 1
// as expand_batch_to_tokens(replace_from=0, replace_to=1) does (rejection_sampler.py:553-559).
__device__ inline float req_temperature(const VerifyParams& p, int r) {
  if (!p.apply_temperature || p.all_greedy) return 1.f;
  const float t = p.temperature[r];
  return t == 0.f ? 1.f : t;
}

// Whether entry i (raw value x) of a row is masked by that row's constraints.
__device__ inline bool row_masked(const float4& m, float x, int i) {
  return (x < m.x) | ((x < m.y) & (i <= __float_as_int(m.z)));
}

struct VerifyPlan {
  int ept;    // elements per thread per row in one sub-chunk
  int g;      // rows per group
  int sub;    // columns per sub-chunk (threads * ept)
  int nsub;   // sub-chunks per row; upper bound of nc (sizes the workspace)
  int chunk;  // columns per task, a multiple of sub
  int nc;     // chunks per row
};

// Verify kernels: the split kernel (stats tasks, then score tasks that re-read the target) and
// the single-read fused kernel (one sub-chunk per task; the workgroup that loaded a target
// sub-chunk parks it in LDS and scores it once the row's statistics are complete).
constexpr int kModeSplit = 0;
constexpr int kModeFused = 1;
// The resident kernel: each task holds its target chunk in registers from the statistics to
// the scores, so every input byte is read once.
constexpr int kModeResident = 2;
// The parked kernel: long tasks whose target chunk is parked in LDS between the statistics and
// the scores, so every input byte is read once.
constexpr int kModeLds = 3;
constexpr int kModes = 4;

// groups = 0 gives the workspace-sizing plan (nc = nsub).  phases is 2 when the batch needs
// recovered scores (stats and score tasks per chunk), else 1; cap = resident workgroups.
VerifyPlan verify_plan(int target_dtype, int64_t vocab_size, int64_t groups, int phases, int cap);

// Chunking of the resident kernel: the fewest chunks of at most its per-task column count,
// balanced and aligned to 64 columns.
VerifyPlan verify_resident_plan(int target_dtype, int64_t vocab_size);
// Chunking of the parked kernel (chunks of its parked sub-chunk count) and the most requests
// whose metadata fit its LDS.
VerifyPlan verify_lds_plan(int target_dtype, int64_t vocab_size);
int lds_max_requests();

// masked: the variant that applies the row masks.
const void* verify_kernel_ptr(int target_dtype, int mode, bool has_draft, bool masked);
// Largest sub-chunks per row (nc) the fused kernel accepts (stats polls, FIFO bound).
int fused_max_chunks();
hipError_t launch_zero_fill(void* p, int64_t bytes, hipStream_t stream);
hipError_t launch_verify(const VerifyParams& params, int target_dtype, int mode, int grid,
                         hipStream_t stream);
// One workgroup per verify row: writes params.masks from top_k / top_p (constraints.hip).
hipError_t launch_constraints(const VerifyParams& params, int target_dtype, hipStream_t stream);
// Top-k / top-p masking in place on fp32 rows logits + r * stride, r < num_rows (one request
// per row, no temperature): masked entries become -inf.  top_k [num_rows] int64 or null;
// top_p [num_rows] fp32 or null.
hipError_t launch_topk_topp(float* logits, int64_t stride, const int64_t* top_k,
                            const float* top_p, int64_t num_rows, int64_t vocab_size,
                            hipStream_t stream);

}  // namespace mvsd
