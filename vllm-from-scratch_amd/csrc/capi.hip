// extern "C" entry points of libmvsd.so (declared in include/mvsd.h).
//
// Every function validates its arguments on the host, enqueues on the caller's stream and
// returns a status code; nothing here synchronises the host or allocates device memory.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "mvsd_device.h"
#include "rows.h"
#include "sampler.h"
#include "selftest.h"
#include "verify.h"
#include "logprobs.h"
#include "processors.h"

namespace {

thread_local int g_last_hip_error = 0;

int hip_status(hipError_t err) {
  if (err == hipSuccess) return MVSD_OK;
  g_last_hip_error = (int)err;
  return MVSD_E_HIP;
}

bool aligned16(const void* ptr, int64_t stride_bytes) {
  return ((uintptr_t)ptr % 16 == 0) && (stride_bytes % 16 == 0);
}

int elem_size(int dtype) {
  switch (dtype) {
    case MVSD_F32: return 4;
    case MVSD_BF16: return 2;
    case MVSD_F16: return 2;
    case MVSD_F64: return 8;
    case MVSD_I32: return 4;
    case MVSD_I64: return 8;
    case MVSD_U8: return 1;
    default: return 0;
  }
}

constexpr int kMaxDevices = 64;

// Resident-workgroup capacity of a verify kernel per device, dtype and kernel kind
// (CUs x occupancy).
int verify_capacity(int device, int dtype, int mode, bool has_draft, bool masked) {
  static std::mutex mu;
  static int cache[kMaxDevices][3][mvsd::kModes][4];
  if (device < 0 || device >= kMaxDevices || dtype < 0 || dtype > 2 || mode < 0 ||
      mode >= mvsd::kModes)
    return 0;
  std::lock_guard<std::mutex> lock(mu);
  int& slot = cache[device][dtype][mode][(masked ? 2 : 0) + (has_draft ? 1 : 0)];
  if (slot > 0) return slot;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return 0;
  const void* fn = mvsd::verify_kernel_ptr(dtype, mode, has_draft, masked);
  if (!fn) return 0;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, mvsd::kVThreads, 0) != hipSuccess)
    return 0;
  // The persistent kernels rely on every launched workgroup being resident, so the runtime's
  // figure is capped by an LDS estimate with a coarse (2 KiB) allocation granularity.
  hipFuncAttributes attr;
  int lds_cu = 0;
  if (hipFuncGetAttributes(&attr, fn) == hipSuccess &&
      hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device) ==
          hipSuccess &&
      attr.sharedSizeBytes > 0) {
    const int64_t granule = 2048;
    const int64_t per_block = ((int64_t)attr.sharedSizeBytes + granule - 1) / granule * granule;
    const int by_lds = (int)(lds_cu / per_block);
    if (by_lds < per_cu) per_cu = by_lds;
  }
  if (per_cu < 1) return 0;
  slot = cus * per_cu;
  return slot;
}

int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Workspace layout.  ctrl = {ticket, sticky spin-limit flag (byte offset 4), exit counter}.
struct WorkspaceLayout {
  int64_t ctrl, grp_off, grp_desc, req_cnt, queues, qgi, masks, stat_slots, arg_slots, total;
};

WorkspaceLayout verify_layout(int64_t B, int64_t P, int64_t nc) {
  WorkspaceLayout l;
  int64_t off = 0;
  l.ctrl = off;
  off = align_up(off + 3 * 4, 256);
  l.grp_off = off;
  off = align_up(off + (B + 1) * 4, 256);
  l.grp_desc = off;
  off = align_up(off + (P > 0 ? P : 1) * 16, 256);
  l.req_cnt = off;
  off = align_up(off + (B > 0 ? B : 1) * 4, 256);
  l.queues = off;  // qticket, qcount, qoff: kMaxQueues ints each
  off = align_up(off + 3 * mvsd::kMaxQueues * 4, 256);
  l.qgi = off;
  off = align_up(off + (P > 0 ? P : 1) * 4, 256);
  l.masks = off;  // row masks of the sampling constraints (zeroed again by the verify kernel)
  off = align_up(off + (P > 0 ? P : 1) * 16, 256);
  l.stat_slots = off;
  off = align_up(off + P * nc * 8, 256);
  l.arg_slots = off;
  off = align_up(off + P * nc * 8, 256);
  l.total = off;
  return l;
}

}  // namespace

namespace mvsd {
// Status of a HIP call for the entry points defined in other sources (MVSD_OK on success).
int record_hip_error(hipError_t err) { return hip_status(err); }
}  // namespace mvsd

extern "C" {

int mvsd_version(void) { return (0 << 16) | (1 << 8) | 0; }

const char* mvsd_status_string(int status) {
  switch (status) {
    case MVSD_OK: return "ok";
    case MVSD_E_INVALID: return "invalid argument";
    case MVSD_E_ALIGN: return "misaligned pointer or stride";
    case MVSD_E_WORKSPACE: return "workspace missing or too small";
    case MVSD_E_HIP: return "HIP runtime error";
    case MVSD_E_RANGE: return "size outside the supported range";
    default: return "unknown status";
  }
}

int mvsd_last_hip_error(void) { return g_last_hip_error; }

int mvsd_expand_batch_to_tokens(void* out, const void* x, int dtype, const int32_t* cu_num_tokens,
                                int64_t batch_size, int64_t num_tokens, double replace_from,
                                double replace_to, mvsd_stream_t stream) {
  if (batch_size < 0 || num_tokens < 0 || elem_size(dtype) == 0 || dtype == MVSD_BF16 ||
      dtype == MVSD_F16)
    return MVSD_E_INVALID;
  if (batch_size == 0) return MVSD_OK;
  if (!out || !x || !cu_num_tokens) return MVSD_E_INVALID;
  if (batch_size > 0x7fffffff) return MVSD_E_RANGE;
  return hip_status(mvsd::launch_expand(out, x, dtype, cu_num_tokens, batch_size, num_tokens,
                                        replace_from, replace_to, (hipStream_t)stream));
}

int64_t mvsd_rejection_workspace_bytes(int64_t batch_size, int64_t num_tokens, int64_t vocab_size,
                                       int target_dtype, int64_t max_spec_len) {
  (void)max_spec_len;
  if (batch_size < 0 || num_tokens < 0 || vocab_size <= 0) return -1;
  const mvsd::VerifyPlan plan = mvsd::verify_plan(target_dtype, vocab_size, 0, 1, 0);
  return verify_layout(batch_size, num_tokens, plan.nsub).total;
}

int mvsd_rejection_workspace_init(void* workspace, int64_t workspace_bytes, mvsd_stream_t stream) {
  if (!workspace || workspace_bytes < 0) return MVSD_E_INVALID;
  if ((uintptr_t)workspace % 256 != 0) return MVSD_E_ALIGN;
  return hip_status(mvsd::launch_zero_fill(workspace, workspace_bytes, (hipStream_t)stream));
}

int mvsd_rejection_sample(const mvsd_rejection_args* a, mvsd_stream_t stream) {
  if (!a) return MVSD_E_INVALID;
  const int64_t B = a->batch_size, P = a->num_tokens, V = a->vocab_size;
  if (B < 0 || P < 0 || V <= 0 || a->max_spec_len < 0) return MVSD_E_INVALID;
  if (a->max_spec_len > mvsd::kMaxSpecLen) return MVSD_E_RANGE;
  if (B > 0x7fffffff || P > 0x7fffffff || V > 0x7fffffff) return MVSD_E_RANGE;
  if (B == 0) return MVSD_OK;
  if (!a->output_token_ids || a->out_stride < a->max_spec_len + 1) return MVSD_E_INVALID;
  if (!a->cu_num_draft_tokens || !a->bonus_token_ids) return MVSD_E_INVALID;
  if (P > 0 && (!a->target_logits || !a->draft_token_ids)) return MVSD_E_INVALID;
  if (a->target_dtype != MVSD_F32 && a->target_dtype != MVSD_BF16 && a->target_dtype != MVSD_F16)
    return MVSD_E_INVALID;
  if (a->draft_probs && a->draft_dtype != MVSD_F32) return MVSD_E_INVALID;
  if (!a->all_greedy && !a->temperature) return MVSD_E_INVALID;
  if (P > 0 && a->target_stride < V) return MVSD_E_INVALID;
  if (P > 0 && a->target_rows && a->target_num_rows < 1) return MVSD_E_INVALID;
  if (a->draft_probs && a->draft_stride < V) return MVSD_E_INVALID;
  const bool need_uniforms = !a->all_greedy || a->synthetic_conditional_rates;
  if (P > 0 && need_uniforms && !a->uniform_probs) return MVSD_E_INVALID;
  const bool need_noise = !a->all_greedy && !a->recovered_token_ids;
  if (P > 0 && need_noise && (!a->exp_noise || a->noise_stride < V)) return MVSD_E_INVALID;

  // Slot arrays are sized for the most chunks any plan can use (nsub), so the layout does not
  // depend on the device.
  const mvsd::VerifyPlan size_plan = mvsd::verify_plan(a->target_dtype, V, 0, 1, 0);
  const WorkspaceLayout lay = verify_layout(B, P, size_plan.nsub);
  if (!a->workspace || a->workspace_bytes < lay.total) return MVSD_E_WORKSPACE;
  if ((uintptr_t)a->workspace % 256 != 0) return MVSD_E_ALIGN;

  // Kernel choice: the split kernel (stats tasks, then score tasks that re-read the target
  // chunk) by default.  MVSD_VERIFY_MODE=fused selects the single-read kernel when its
  // requirements hold: 16-byte loads (below), the request metadata in LDS
  // (B <= kMaxFusedRequests) and at most fused_max_chunks() sub-chunks per row.
  // MVSD_VERIFY_MODE=resident selects the register-resident kernel when its requirements
  // hold: 16-byte loads, B <= kMaxLdsRequests, and at least half as many resident workgroups
  // as chunks per row (its progress argument).  MVSD_VERIFY_MODE=lds selects the parked
  // kernel when B <= lds_max_requests() and more workgroups are resident than chunks per row.
  const int two_phase = (!a->all_greedy && !a->recovered_token_ids) ? 1 : 0;
  // Sampling constraints apply only when some request samples (rejection_sampler.py:549-550).
  const bool masked = !a->all_greedy && (a->top_k || a->top_p);
  int cap = 0;
  int kmode = mvsd::kModeSplit;
  if (P > 0) {
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess) return hip_status(err);
    // The fused kernel issues unconditional 16-byte loads: rows must be 16-byte aligned and
    // V a multiple of the vector width.
    const int esz = elem_size(a->target_dtype);
    const bool vec_ok = aligned16(a->target_logits, a->target_stride * esz) &&
                        aligned16(a->exp_noise, a->noise_stride * 4) &&
                        (!a->draft_probs || aligned16(a->draft_probs, a->draft_stride * 4)) &&
                        V % (16 / esz) == 0;
    const char* mode = getenv("MVSD_VERIFY_MODE");
    if (vec_ok && B <= mvsd::kMaxFusedRequests && size_plan.nsub <= mvsd::fused_max_chunks() &&
        mode && strcmp(mode, "fused") == 0) {
      const int fcap = verify_capacity(device, a->target_dtype, mvsd::kModeFused,
                                       a->draft_probs != nullptr, masked);
      if (fcap > 0) {
        kmode = mvsd::kModeFused;
        cap = fcap;
      }
    }
    if (vec_ok && B <= mvsd::kMaxLdsRequests && mode && strcmp(mode, "resident") == 0) {
      const int rcap = verify_capacity(device, a->target_dtype, mvsd::kModeResident,
                                       a->draft_probs != nullptr, masked);
      const mvsd::VerifyPlan rplan = mvsd::verify_resident_plan(a->target_dtype, V);
      if (rcap > 0 && rplan.nc <= size_plan.nsub && rplan.nc <= 2 * rcap) {
        kmode = mvsd::kModeResident;
        cap = rcap;
      }
    }
    if (B <= mvsd::lds_max_requests() && mode && strcmp(mode, "lds") == 0) {
      const int lcap = verify_capacity(device, a->target_dtype, mvsd::kModeLds,
                                       a->draft_probs != nullptr, masked);
      const mvsd::VerifyPlan lplan = mvsd::verify_lds_plan(a->target_dtype, V);
      if (lcap > 0 && lplan.nc <= size_plan.nsub && lplan.nc < lcap) {
        kmode = mvsd::kModeLds;
        cap = lcap;
      }
    }
    if (kmode == mvsd::kModeSplit)
      cap = verify_capacity(device, a->target_dtype, kmode, a->draft_probs != nullptr, masked);
    if (cap <= 0) return hip_status(hipErrorInvalidDevice);
  }
  // Upper bound on groups: min(P, B * ceil(max_spec_len / G)).
  int64_t groups = B * ((a->max_spec_len + size_plan.g - 1) / size_plan.g);
  if (groups > P) groups = P;
  mvsd::VerifyPlan plan = size_plan;
  if (kmode == mvsd::kModeSplit)
    plan = mvsd::verify_plan(a->target_dtype, V, groups > 0 ? groups : 1, two_phase ? 2 : 1, cap);
  else if (kmode == mvsd::kModeResident)
    plan = mvsd::verify_resident_plan(a->target_dtype, V);
  else if (kmode == mvsd::kModeLds)
    plan = mvsd::verify_lds_plan(a->target_dtype, V);

  char* ws = static_cast<char*>(a->workspace);
  mvsd::VerifyParams p;
  memset(&p, 0, sizeof(p));
  p.out = a->output_token_ids;
  p.out_stride = a->out_stride;
  p.target = a->target_logits;
  p.target_stride = a->target_stride;
  p.target_rows = a->target_rows;
  p.target_num_rows = a->target_num_rows;
  p.draft = static_cast<const float*>(a->draft_probs);
  p.draft_stride = a->draft_stride;
  p.noise = a->exp_noise;
  p.noise_stride = a->noise_stride;
  p.uniforms = a->uniform_probs;
  p.draft_ids = a->draft_token_ids;
  p.cu = a->cu_num_draft_tokens;
  p.bonus = a->bonus_token_ids;
  p.temperature = a->temperature;
  p.recovered = a->recovered_token_ids;
  p.synth = a->synthetic_conditional_rates;
  p.target_dtype = a->target_dtype;
  p.all_greedy = a->all_greedy ? 1 : 0;
  p.apply_temperature = a->apply_temperature ? 1 : 0;
  p.B = (int)B;
  p.P = (int)P;
  p.V = (int)V;
  p.max_spec_len = (int)a->max_spec_len;
  p.chunk = plan.chunk;
  p.nc = plan.nc;
  p.split = 0;
  p.arg_stride = plan.nc;
  p.G = plan.g;
  const int esz = elem_size(a->target_dtype);
  p.target_aligned = aligned16(a->target_logits, a->target_stride * esz);
  p.draft_aligned = a->draft_probs ? aligned16(a->draft_probs, a->draft_stride * 4) : false;
  p.noise_aligned = a->exp_noise ? aligned16(a->exp_noise, a->noise_stride * 4) : false;
  p.ctrl = reinterpret_cast<int*>(ws + lay.ctrl);
  p.grp_off = reinterpret_cast<int*>(ws + lay.grp_off);
  p.grp_desc = reinterpret_cast<int4*>(ws + lay.grp_desc);
  p.req_cnt = reinterpret_cast<int*>(ws + lay.req_cnt);
  p.qticket = reinterpret_cast<int*>(ws + lay.queues);
  p.qcount = p.qticket + mvsd::kMaxQueues;
  p.qoff = p.qcount + mvsd::kMaxQueues;
  p.qgi = reinterpret_cast<int*>(ws + lay.qgi);
  // Work queues (MVSD_VERIFY_QUEUES, 1..16; one per XCD gives each queue one L2).  One queue
  // measured fastest at the headline: the re-read is served by the Infinity Cache anyway.
  int nq = 1;
  if (const char* env = getenv("MVSD_VERIFY_QUEUES")) nq = atoi(env);
  p.nq = nq < 1 ? 1 : (nq > mvsd::kMaxQueues ? mvsd::kMaxQueues : nq);
  // Without the init kernel (group offsets built in each workgroup's LDS) when one queue
  // serves the batch and its requests fit (MVSD_VERIFY_LDS_GROUPS=0 keeps the init kernel).
  p.lds_groups = kmode == mvsd::kModeSplit && p.nq == 1 && B <= mvsd::kMaxLdsRequests && P > 0;
  if (const char* env = getenv("MVSD_VERIFY_LDS_GROUPS")) p.lds_groups = p.lds_groups && atoi(env) != 0;
  if (kmode != mvsd::kModeSplit) {
    p.nq = 1;  // one ticket; the group offsets always in LDS
    p.lds_groups = 1;
  }
  p.top_k = masked ? a->top_k : nullptr;
  p.top_p = masked ? a->top_p : nullptr;
  p.masks = masked ? reinterpret_cast<float4*>(ws + lay.masks) : nullptr;
  p.stat_slots = reinterpret_cast<uint64_t*>(ws + lay.stat_slots);
  p.arg_slots = reinterpret_cast<uint64_t*>(ws + lay.arg_slots);

  int grid = 0;
  if (P > 0) {
    int64_t tasks;
    if (kmode != mvsd::kModeSplit) {
      tasks = groups * plan.nc;
      grid = (int)(tasks < cap ? tasks : cap);
    } else {
      // Each queue is served by grid / nq workgroups.  A group's score chunks are claimed
      // `lag` groups after its stats chunks: enough for that queue's workgroups (each holding
      // a current and a prefetched ticket) to have finished the stats, and as few as possible
      // so that the score tasks re-read the target chunk while it is still cached (L2 or the
      // Infinity Cache).
      p.two_phase = two_phase;
      grid = cap / p.nq * p.nq;
      if (grid < p.nq) grid = p.nq;
      const int per_queue = grid / p.nq;
      int lag = (2 * per_queue + 2 * plan.nc - 1) / (2 * plan.nc) + 1;
      if (const char* env = getenv("MVSD_VERIFY_LAG")) lag = atoi(env);
      p.lag = lag < 1 ? 1 : (lag > 4096 ? 4096 : lag);
      const int64_t step = p.two_phase ? 2 * plan.nc : plan.nc;
      // Epilogue split (one queue): the score tasks of the last `lag` groups use the empty
      // stats slots of their steps as a second half-chunk task each (MVSD_VERIFY_SPLIT=0
      // turns it off).  MVSD_VERIFY_QUARTER=n runs the score tasks of the last n groups in
      // quarter chunks instead (off by default: no gain measured on MI355X, the end of the
      // launch is set by the last requests' finalisation rather than by the task length).
      p.split = p.two_phase && p.nq == 1 && 2 * plan.nc <= size_plan.nsub ? 1 : 0;
      if (const char* env = getenv("MVSD_VERIFY_SPLIT")) p.split = p.split && atoi(env) != 0;
      int quarter = 0;
      if (const char* env = getenv("MVSD_VERIFY_QUARTER")) quarter = atoi(env);
      p.quarter = p.split && 4 * plan.nc <= size_plan.nsub ? (quarter < 0 ? 0 : (quarter > p.lag ? p.lag : quarter)) : 0;
      if (p.split) p.arg_stride = (p.quarter > 0 ? 4 : 2) * plan.nc;
      tasks = (groups + (p.two_phase ? p.lag * p.nq : 0) + p.quarter) * step;
    }
    // every workgroup may claim up to three tickets past the last task
    if (tasks > 0x7fffffff - 4 * (int64_t)cap) return MVSD_E_RANGE;
  }
  return hip_status(mvsd::launch_verify(p, a->target_dtype, kmode, grid, (hipStream_t)stream));
}

int mvsd_apply_logits_processors(float* logits, int64_t stride, int64_t num_tokens,
                                 int64_t vocab_size, int64_t batch_size,
                                 const int32_t* cu_num_draft_tokens, const int32_t* spec_tokens,
                                 const int32_t* ent_off, const int32_t* ent_tok,
                                 const int32_t* ent_info, const float* presence,
                                 const float* frequency, const float* repetition,
                                 const int32_t* n_mask, const int32_t* stop_off,
                                 const int32_t* stop_tok, mvsd_stream_t stream) {
  if (num_tokens < 0 || batch_size < 0 || vocab_size <= 0) return MVSD_E_INVALID;
  if (num_tokens == 0 || batch_size == 0 || (!ent_off && !n_mask)) return MVSD_OK;
  if (num_tokens > 0x7fffffff || batch_size > 0x7fffffff || vocab_size > 0x7fffffff)
    return MVSD_E_RANGE;
  if (!logits || stride < vocab_size || !cu_num_draft_tokens) return MVSD_E_INVALID;
  if (ent_off && (!ent_tok || !ent_info || !spec_tokens)) return MVSD_E_INVALID;
  if (n_mask && (!stop_off || !stop_tok)) return MVSD_E_INVALID;
  mvsd::ProcessorParams p;
  p.logits = logits;
  p.stride = stride;
  p.P = (int)num_tokens;
  p.V = (int)vocab_size;
  p.B = (int)batch_size;
  p.cu = cu_num_draft_tokens;
  p.spec = spec_tokens;
  p.ent_off = ent_off;
  p.ent_tok = ent_tok;
  p.ent_info = ent_info;
  p.presence = presence;
  p.frequency = frequency;
  p.repetition = repetition;
  p.n_mask = n_mask;
  p.stop_off = stop_off;
  p.stop_tok = stop_tok;
  return hip_status(mvsd::launch_logits_processors(p, (hipStream_t)stream));
}

int mvsd_spec_logprobs(int32_t* ids, float* lps, int32_t* ranks, const float* target,
                       int64_t target_stride, const int32_t* target_rows, const float* bonus,
                       int64_t bonus_stride, const int32_t* cu_num_sampled_tokens,
                       const int32_t* sampled_token_ids, int64_t sampled_stride,
                       int64_t batch_size, int64_t num_tokens, int64_t vocab_size,
                       int64_t width, int64_t k, int logits_mode, mvsd_stream_t stream) {
  if (batch_size < 0 || num_tokens < 0 || vocab_size <= 0 || width < 0 || k < 0)
    return MVSD_E_INVALID;
  if (batch_size == 0 || width == 0) return MVSD_OK;
  if (k > mvsd::logprobs_max_k() || k > vocab_size) return MVSD_E_RANGE;
  if (batch_size * width > 0x7fffffff || num_tokens > 0x7fffffff || vocab_size > 0x7fffffff)
    return MVSD_E_RANGE;
  if (!ids || !lps || !ranks || !bonus || !cu_num_sampled_tokens || !sampled_token_ids)
    return MVSD_E_INVALID;
  if (num_tokens > 0 && (!target || target_stride < vocab_size)) return MVSD_E_INVALID;
  if (bonus_stride < vocab_size || sampled_stride < width) return MVSD_E_INVALID;
  mvsd::LogprobParams p;
  p.target = target;
  p.tstride = target_stride;
  p.target_rows = target_rows;
  p.bonus = bonus;
  p.bstride = bonus_stride;
  p.cu_sampled = cu_num_sampled_tokens;
  p.tokens = sampled_token_ids;
  p.tok_stride = sampled_stride;
  p.B = (int)batch_size;
  p.P = (int)num_tokens;
  p.V = (int)vocab_size;
  p.W = (int)width;
  p.k = (int)k;
  p.logits_mode = logits_mode ? 1 : 0;
  p.ids = ids;
  p.lps = lps;
  p.ranks = ranks;
  return hip_status(mvsd::launch_spec_logprobs(p, (hipStream_t)stream));
}

int mvsd_sampler_rows(int op, int32_t* ids, float* out, int64_t out_stride, float* x,
                      int64_t stride, const float* aux, int64_t aux_stride, int64_t num_rows,
                      int64_t vocab_size, mvsd_stream_t stream) {
  if (num_rows < 0 || vocab_size <= 0 || op < 0 || op > 3) return MVSD_E_INVALID;
  if (num_rows == 0) return MVSD_OK;
  if (num_rows > 0x7fffffff || vocab_size > 0x7fffffff) return MVSD_E_RANGE;
  if (!x || stride < vocab_size) return MVSD_E_INVALID;
  if ((op == mvsd::kSamplerArgmax || op == mvsd::kSamplerRace) && !ids) return MVSD_E_INVALID;
  if (op == mvsd::kSamplerMinP && !aux) return MVSD_E_INVALID;
  if (op == mvsd::kSamplerRace && (!aux || aux_stride < vocab_size)) return MVSD_E_INVALID;
  if (op == mvsd::kSamplerLogSoftmax && (!out || out_stride < vocab_size)) return MVSD_E_INVALID;
  return hip_status(mvsd::launch_sampler_rows(op, ids, out, out_stride, x, stride, aux,
                                              aux_stride, num_rows, vocab_size,
                                              (hipStream_t)stream));
}

int mvsd_selftest(int test, uint64_t* failures, mvsd_stream_t stream) {
  if (!failures) return MVSD_E_INVALID;
  unsigned long long* f = reinterpret_cast<unsigned long long*>(failures);
  if (test == 0) return hip_status(mvsd::launch_selftest_reciprocal(f, (hipStream_t)stream));
  if (test == 1) {
    // temperatures of the kind requests carry, both ends of the fast range, and divisors
    // outside it (IEEE path), plus 1 (greedy rows)
    static const float divisors[] = {1.0f, 0.3f, 0.8f, 1.5f, 0.7f, 1.0f / 3.0f, 0.9999999f,
                                     1.0000001f, 2.5f, 0.01f, 123.456f, 0x1p-20f, 0x1p20f,
                                     0x1.fffffep-21f, 3e-7f, 5e6f};
    return hip_status(mvsd::launch_selftest_division(
        divisors, (int)(sizeof(divisors) / sizeof(divisors[0])), f, (hipStream_t)stream));
  }
  return MVSD_E_INVALID;
}

int mvsd_sampling_masks(const mvsd_rejection_args* a, float* masks, mvsd_stream_t stream) {
  if (!a || !masks) return MVSD_E_INVALID;
  const int64_t B = a->batch_size, P = a->num_tokens, V = a->vocab_size;
  if (B < 0 || P < 0 || V <= 0) return MVSD_E_INVALID;
  if (B > 0x7fffffff || P > 0x7fffffff || V > 0x7fffffff) return MVSD_E_RANGE;
  if (P == 0) return MVSD_OK;
  if (!a->target_logits || !a->cu_num_draft_tokens) return MVSD_E_INVALID;
  if (a->target_dtype != MVSD_F32 && a->target_dtype != MVSD_BF16 && a->target_dtype != MVSD_F16)
    return MVSD_E_INVALID;
  if (!a->all_greedy && !a->temperature) return MVSD_E_INVALID;
  if (a->target_stride < V) return MVSD_E_INVALID;
  if (a->target_rows && a->target_num_rows < 1) return MVSD_E_INVALID;
  if ((uintptr_t)masks % 16 != 0) return MVSD_E_ALIGN;
  mvsd::VerifyParams p;
  memset(&p, 0, sizeof(p));
  p.target = a->target_logits;
  p.target_stride = a->target_stride;
  p.target_rows = a->target_rows;
  p.target_num_rows = a->target_num_rows;
  p.cu = a->cu_num_draft_tokens;
  p.temperature = a->temperature;
  p.target_dtype = a->target_dtype;
  p.all_greedy = a->all_greedy ? 1 : 0;
  p.apply_temperature = a->apply_temperature ? 1 : 0;
  p.B = (int)B;
  p.P = (int)P;
  p.V = (int)V;
  p.top_k = a->top_k;
  p.top_p = a->top_p;
  p.masks = reinterpret_cast<float4*>(masks);
  return hip_status(mvsd::launch_constraints(p, a->target_dtype, (hipStream_t)stream));
}

int mvsd_apply_top_k_top_p(float* logits, int64_t logits_stride, const int64_t* top_k,
                           const float* top_p, int64_t num_rows, int64_t vocab_size,
                           mvsd_stream_t stream) {
  if (num_rows < 0 || vocab_size <= 0) return MVSD_E_INVALID;
  if (num_rows == 0 || (!top_k && !top_p)) return MVSD_OK;
  if (!logits || logits_stride < vocab_size) return MVSD_E_INVALID;
  if (vocab_size > 0x7fffffff || num_rows > 0x7fffffff) return MVSD_E_RANGE;
  return hip_status(mvsd::launch_topk_topp(logits, logits_stride, top_k, top_p, num_rows,
                                           vocab_size, (hipStream_t)stream));
}

int mvsd_softmax_rows(float* probs, int64_t probs_stride, const void* logits, int dtype,
                      int64_t logits_stride, const float* temperature, int64_t num_rows,
                      int64_t vocab_size, mvsd_stream_t stream) {
  if (num_rows < 0 || vocab_size <= 0) return MVSD_E_INVALID;
  if (num_rows == 0) return MVSD_OK;
  if (!probs || !logits || probs_stride < vocab_size || logits_stride < vocab_size)
    return MVSD_E_INVALID;
  if (dtype != MVSD_F32 && dtype != MVSD_BF16 && dtype != MVSD_F16) return MVSD_E_INVALID;
  if (num_rows > 0x7fffffff) return MVSD_E_RANGE;
  return hip_status(mvsd::launch_softmax_rows(probs, probs_stride, logits, dtype, logits_stride,
                                              temperature, num_rows, vocab_size,
                                              (hipStream_t)stream));
}

int mvsd_sample_recovered_tokens(int32_t* recovered_token_ids, const int32_t* cu_num_draft_tokens,
                                 const int32_t* draft_token_ids, const float* draft_probs,
                                 int64_t draft_stride, const float* target_probs,
                                 int64_t target_stride, const float* exp_noise,
                                 int64_t noise_stride, int64_t batch_size, int64_t num_tokens,
                                 int64_t vocab_size, int64_t max_spec_len, mvsd_stream_t stream) {
  if (batch_size < 0 || num_tokens < 0 || vocab_size <= 0 || max_spec_len < 0)
    return MVSD_E_INVALID;
  if (batch_size == 0 || num_tokens == 0 || max_spec_len == 0) return MVSD_OK;
  if (!recovered_token_ids || !cu_num_draft_tokens || !draft_token_ids || !target_probs ||
      !exp_noise)
    return MVSD_E_INVALID;
  if (target_stride < vocab_size || noise_stride < vocab_size ||
      (draft_probs && draft_stride < vocab_size))
    return MVSD_E_INVALID;
  if (batch_size > 65535 * 1024LL || max_spec_len > 65535 || vocab_size > 0x7fffffff)
    return MVSD_E_RANGE;
  return hip_status(mvsd::launch_recovered(recovered_token_ids, cu_num_draft_tokens,
                                           draft_token_ids, draft_probs, draft_stride,
                                           target_probs, target_stride, exp_noise, noise_stride,
                                           batch_size, max_spec_len, vocab_size, num_tokens,
                                           (hipStream_t)stream));
}

int mvsd_ngram_valid_sampled(int32_t* next_token_ids, int32_t* counts, int32_t* valid_ids,
                             int64_t valid_stride, const int32_t* sampled,
                             int64_t sampled_stride, int64_t width, const uint8_t* discard,
                             const int32_t* token_ids, int64_t row_stride,
                             const int32_t* num_tokens, int64_t vocab_size, int64_t num_reqs,
                             mvsd_stream_t stream) {
  if (num_reqs < 0 || width < 0 || vocab_size < 0) return MVSD_E_INVALID;
  if (num_reqs == 0) return MVSD_OK;
  if (!next_token_ids || !counts || !valid_ids || !token_ids || !num_tokens) return MVSD_E_INVALID;
  if (width > 0 && !sampled) return MVSD_E_INVALID;
  if (valid_stride < width || sampled_stride < width || row_stride < 1) return MVSD_E_INVALID;
  if (vocab_size > 0x7fffffff || num_reqs > 0x7fffffff) return MVSD_E_RANGE;
  return hip_status(mvsd::launch_ngram_valid_sampled(
      next_token_ids, counts, valid_ids, valid_stride, sampled, sampled_stride, width, discard,
      token_ids, row_stride, num_tokens, (int32_t)vocab_size, num_reqs, (hipStream_t)stream));
}

int mvsd_ngram_propose(int32_t* drafts, int32_t* num_valid, int32_t* token_ids,
                       int64_t row_stride, int64_t max_seq_len, const int32_t* num_tokens,
                       const int32_t* new_tokens, int64_t new_tokens_stride,
                       int64_t max_new_tokens, const int32_t* new_counts,
                       const uint8_t* active, int gate_on_new_counts, int64_t num_reqs,
                       int32_t min_n, int32_t max_n, int32_t k, int cap_by_model_len,
                       int64_t max_model_len, mvsd_stream_t stream) {
  if (num_reqs < 0) return MVSD_E_INVALID;
  if (min_n < 1 || max_n < min_n || k < 1) return MVSD_E_INVALID;
  if (max_n > mvsd::kNgramMaxN || k > 256) return MVSD_E_RANGE;
  if (num_reqs == 0) return MVSD_OK;
  if (!drafts || !num_valid || !token_ids || !num_tokens) return MVSD_E_INVALID;
  if (max_seq_len < 0 || row_stride < max_seq_len) return MVSD_E_INVALID;
  if (row_stride > 0x7fffffff || num_reqs > 0x7fffffff) return MVSD_E_RANGE;
  if (new_tokens && (max_new_tokens < 0 || new_tokens_stride < max_new_tokens))
    return MVSD_E_INVALID;
  if (gate_on_new_counts && !new_counts) return MVSD_E_INVALID;
  mvsd::NgramParams p;
  p.drafts = drafts;
  p.num_valid = num_valid;
  p.tokens = token_ids;
  p.row_stride = row_stride;
  p.max_seq_len = max_seq_len;
  p.num_tokens = num_tokens;
  p.new_tokens = new_tokens;
  p.new_stride = new_tokens_stride;
  p.max_new = new_tokens ? max_new_tokens : 0;
  p.new_counts = new_counts;
  p.active = active;
  p.gate_on_new_counts = gate_on_new_counts ? 1 : 0;
  p.min_n = min_n;
  p.max_n = max_n;
  p.k = k;
  p.cap_by_model_len = cap_by_model_len ? 1 : 0;
  p.max_model_len = max_model_len;
  return hip_status(mvsd::launch_ngram(p, num_reqs, (hipStream_t)stream));
}

}  // extern "C"
