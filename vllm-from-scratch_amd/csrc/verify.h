// Host/device interface of the verification kernel (verify.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvsd {

constexpr int kMaxSpecLen = 128;       // reference MAX_SPEC_LEN, rejection_sampler.py:83
constexpr int kMaxLaunchRequests = 4096;  // requests per verify launch (their tables live in LDS)
constexpr int kVThreads = 512;         // verify-kernel workgroup size
constexpr int kVWaves = kVThreads / 64;
constexpr int kSpinLimitDefault = 1 << 18;  // polls before a wait gives up (~0.3 s)
// Value written into every output entry of a call in which some wait gave up.
constexpr int32_t kPoison = INT32_MIN;
// The launch counters in VerifyParams::ctrl (ints), each on a 4 KiB page of its own.  Atomics on
// one line serialise, and with the three on one line the exit counts and flag reads at the end
// of a launch queued with the ticket claims of the last tasks (a 64-request fp32 batch measured
// 9 % slower).
constexpr int kCtrlTicket = 0;
constexpr int kCtrlFlag = 1024;
constexpr int kCtrlExit = 2048;
constexpr int kCtrlInts = 3072;

// Kernel parameters, passed by value.  Pointers are device pointers; strides are in
// elements.  One launch covers requests [r0, r0 + B) of the caller's batch: the request
// arrays (out, bonus, temperature, top_k, top_p, noise, cu) are offset by r0 on the host, and
// cu_prev points at cu[r0 - 1] (nullptr for r0 = 0).  Verify rows keep their batch-wide
// indices (P = rows of the whole batch).
struct VerifyParams {
  int32_t* out;
  int64_t out_stride;
  const void* target;
  int64_t target_stride;
  const int32_t* target_rows;
  int64_t target_num_rows;
  const void* draft;     // [P, V] draft probabilities (dtype draft_dtype), or null
  int64_t draft_stride;
  int draft_dtype;
  const float* noise;
  int64_t noise_stride;
  const double* uniforms;
  const int32_t* draft_ids;
  const int32_t* cu;
  const int32_t* cu_prev;
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
  int chunk;       // vocab columns per task (a multiple of the sub-chunk)
  int nc;          // chunks per row
  int G;           // rows per stats group
  int lag;         // stats units between a request's last stats unit and its score unit
  int tail_groups;  // stats groups at the end of the launch run in half-chunk tasks
  int spin_limit;  // polls before a wait gives up (0: every wait gives up at once)
  bool target_aligned;
  bool draft_aligned;
  bool noise_aligned;
  // workspace (every array is zero between calls)
  int* ctrl;             // [kCtrlTicket] ticket, [kCtrlFlag] wait-failure flag, [kCtrlExit] exits
  int* req_cnt;          // [B] started stats tasks per request
  int* score_cnt;        // [B] started score tasks per request
  int* decision;         // [B] first rejected position + 1, or K + 1 (all accepted)
  uint64_t* stat_slots;   // [P * 2 nc] per task of a row: packed (max, sum), or the argmax
                          // key of a greedy row; 0 = empty
  uint64_t* score_slots;  // [B * 2 nc] per score task: the rejected row's argmax key
  // Sampling constraints (top-k / top-p per request, either may be null).  When set, the
  // constraints kernel writes one row mask per verify row, (A, B, J as bits, 0): entry i of
  // the row, raw value x, is masked iff x < A || (x < B && i <= J).
  const int64_t* top_k;  // [B]
  const float* top_p;    // [B]
  float4* masks;         // [P], null when no constraint applies
  // Optional read-out [P, 3] of each random verify row as decided: raw max, sum of
  // exp2((x - max) log2(e) / T), and the fp32 probability of the draft token.
  float* debug_row_stats;
  // Rows the constraints kernel works on, heaviest first, as row + 1 (0 = no entry), written
  // by the plan kernel and cleared by the workgroup that takes each entry; null: every row.
  int* order;
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
  int ept;     // elements per thread per row in one sub-chunk
  int g;       // rows per stats group
  int sub;     // columns per sub-chunk (threads * ept)
  int nc_max;  // largest nc any plan for this vocabulary and batch size uses (sizes the workspace)
  int chunk;   // columns per task, a multiple of sub
  int nc;      // chunks per row
};

// units = stats groups + score units of the launch (0 gives the workspace-sizing plan);
// cap = resident workgroups; batch_rows = verify rows + requests of the call (the same value
// when sizing the workspace and when planning its launches: nc never exceeds nc_max);
// score_units: the launch has score units (random requests without supplied recovered ids).
VerifyPlan verify_plan(int target_dtype, int64_t vocab_size, int64_t units, int cap,
                       int64_t batch_rows, bool score_units);

// The verify kernel variant for a target dtype, draft dtype (-1: point-mass drafts) and
// sampling constraints.
const void* verify_kernel_ptr(int target_dtype, int draft_dtype, bool masked);
hipError_t launch_zero_fill(void* p, int64_t bytes, hipStream_t stream);
hipError_t launch_verify(const VerifyParams& params, int target_dtype, int grid,
                         hipStream_t stream);
// One workgroup per verify row: writes params.masks from top_k / top_p (constraints.hip).
// With params.order set, a plan kernel first writes the masks of the rows that need no work
// and lists the others heaviest first (random top-p, random top-k, greedy top-p).
hipError_t launch_constraints(const VerifyParams& params, int target_dtype, hipStream_t stream);
// Top-k / top-p masking in place on fp32 rows logits + r * stride, r < num_rows (one request
// per row, no temperature): masked entries become -inf.  top_k [num_rows] int64 or null;
// top_p [num_rows] fp32 or null.
hipError_t launch_topk_topp(float* logits, int64_t stride, const int64_t* top_k,
                            const float* top_p, int64_t num_rows, int64_t vocab_size,
                            hipStream_t stream);

}  // namespace mvsd
