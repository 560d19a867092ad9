// extern "C" entry points of libmvsd.so (declared in include/mvsd.h).
//
// Every function validates its arguments on the host, enqueues on the caller's stream and
// returns a status code; nothing here synchronises the host or allocates device memory.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
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

// Size of the static scratch of mvsd_rejection_sample_static (include/mvsd.h).
constexpr int64_t kStaticScratchBytes = 16ll << 20;

// Polls before a verify-kernel wait gives up (mvsd_set_wait_limit).
std::atomic<int> g_wait_limit{mvsd::kSpinLimitDefault};

// Resident-workgroup capacity of the verify kernel variant per device (CUs x occupancy).
int verify_capacity(int device, int dtype, int draft_dtype, bool masked) {
  static std::mutex mu;
  static int cache[kMaxDevices][3][4][2];
  if (device < 0 || device >= kMaxDevices || dtype < 0 || dtype > 2 || draft_dtype < -1 ||
      draft_dtype > 2)
    return 0;
  std::lock_guard<std::mutex> lock(mu);
  int& slot = cache[device][dtype][draft_dtype + 1][masked ? 1 : 0];
  if (slot > 0) return slot;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return 0;
  const void* fn = mvsd::verify_kernel_ptr(dtype, draft_dtype, masked);
  if (!fn) return 0;
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, mvsd::kVThreads, 0) != hipSuccess)
    return 0;
  // The persistent kernel relies on every launched workgroup being resident, so the runtime's
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

// Workspace layout of the verify kernel for launches of at most Bl requests over P verify
// rows with at most nc chunks per row.  ctrl holds the launch counters (mvsd::kCtrlInts ints).
struct WorkspaceLayout {
  int64_t ctrl, req_cnt, score_cnt, decision, masks, order, stat_slots, score_slots, total;
};

WorkspaceLayout verify_layout(int64_t Bl, int64_t P, int64_t nc) {
  WorkspaceLayout l;
  int64_t off = 0;
  const int64_t b = Bl > 0 ? Bl : 1, rows = P > 0 ? P : 1;
  l.ctrl = off;
  off = align_up(off + mvsd::kCtrlInts * 4, 256);
  l.req_cnt = off;
  off = align_up(off + b * 4, 256);
  l.score_cnt = off;
  off = align_up(off + b * 4, 256);
  l.decision = off;
  off = align_up(off + b * 4, 256);
  l.masks = off;  // row masks of the sampling constraints (zeroed again by the verify kernel)
  off = align_up(off + rows * 16, 256);
  l.order = off;  // the constraints kernel's row plan (each entry cleared by its reader)
  off = align_up(off + rows * 4, 256);
  l.stat_slots = off;
  off = align_up(off + rows * 2 * nc * 8, 256);  // two slots per chunk (tail halves)
  l.score_slots = off;
  off = align_up(off + b * 2 * nc * 8, 256);
  l.total = off;
  return l;
}

int64_t launch_requests(int64_t B) {
  return B < mvsd::kMaxLaunchRequests ? B : mvsd::kMaxLaunchRequests;
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
    case MVSD_E_SCRATCH:
      return "the batch needs more scratch than the static scratch of "
             "mvsd_rejection_sample_static holds (see mvsd_rejection_static_scratch_bytes)";
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
  const mvsd::VerifyPlan plan = mvsd::verify_plan(target_dtype, vocab_size, 0, 0,
                                                  num_tokens + launch_requests(batch_size), true);
  return verify_layout(launch_requests(batch_size), num_tokens, plan.nc_max).total;
}

int mvsd_set_wait_limit(int polls) {
  const int prev = g_wait_limit.load();
  g_wait_limit.store(polls < 0 ? mvsd::kSpinLimitDefault : polls);
  return prev;
}

int mvsd_rejection_workspace_init(void* workspace, int64_t workspace_bytes, mvsd_stream_t stream) {
  if (!workspace || workspace_bytes < 0) return MVSD_E_INVALID;
  if ((uintptr_t)workspace % 256 != 0) return MVSD_E_ALIGN;
  return hip_status(mvsd::launch_zero_fill(workspace, workspace_bytes, (hipStream_t)stream));
}

}  // extern "C"

namespace {

// mvsd_rejection_sample with the workspace `ws` of `ws_bytes` bytes (the args' workspace fields
// are not read).
int rejection_sample_impl(const mvsd_rejection_args* a, void* ws_ptr, int64_t ws_bytes,
                          mvsd_stream_t stream) {
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
  if (a->draft_probs && a->draft_dtype != MVSD_F32 && a->draft_dtype != MVSD_BF16 &&
      a->draft_dtype != MVSD_F16)
    return MVSD_E_INVALID;
  if (!a->all_greedy && !a->temperature) return MVSD_E_INVALID;
  if (P > 0 && a->target_stride < V) return MVSD_E_INVALID;
  if (P > 0 && a->target_rows && a->target_num_rows < 1) return MVSD_E_INVALID;
  if (a->draft_probs && a->draft_stride < V) return MVSD_E_INVALID;
  const bool need_uniforms = !a->all_greedy || a->synthetic_conditional_rates;
  if (P > 0 && need_uniforms && !a->uniform_probs) return MVSD_E_INVALID;
  const bool need_noise = !a->all_greedy && !a->recovered_token_ids;
  if (P > 0 && need_noise && (!a->exp_noise || a->noise_stride < V)) return MVSD_E_INVALID;

  // Slot arrays are sized for the most chunks any plan can use, so the layout does not depend
  // on the device.
  const int64_t batch_rows = P + launch_requests(B);
  const mvsd::VerifyPlan size_plan = mvsd::verify_plan(a->target_dtype, V, 0, 0, batch_rows, true);
  const WorkspaceLayout lay = verify_layout(launch_requests(B), P, size_plan.nc_max);
  if (!ws_ptr || ws_bytes < lay.total) return MVSD_E_WORKSPACE;
  if ((uintptr_t)ws_ptr % 256 != 0) return MVSD_E_ALIGN;

  // Random requests with in-kernel recovered ids get score units (one per request).
  const bool scores = !a->all_greedy && !a->recovered_token_ids;
  // Sampling constraints apply only when some request samples (rejection_sampler.py:549-550).
  const bool masked = !a->all_greedy && (a->top_k || a->top_p);
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_status(err);
  const int draft_dtype = a->draft_probs ? a->draft_dtype : -1;
  const int cap = verify_capacity(device, a->target_dtype, draft_dtype, masked);
  if (cap <= 0) return hip_status(hipErrorInvalidDevice);

  char* ws = static_cast<char*>(ws_ptr);
  mvsd::VerifyParams p;
  memset(&p, 0, sizeof(p));
  p.out = a->output_token_ids;
  p.out_stride = a->out_stride;
  p.target = a->target_logits;
  p.target_stride = a->target_stride;
  p.target_rows = a->target_rows;
  p.target_num_rows = a->target_num_rows;
  p.draft = a->draft_probs;
  p.draft_stride = a->draft_stride;
  p.draft_dtype = draft_dtype;
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
  p.G = size_plan.g;
  p.spin_limit = g_wait_limit.load();
  const int esz = elem_size(a->target_dtype);
  p.target_aligned = aligned16(a->target_logits, a->target_stride * esz);
  p.draft_aligned =
      a->draft_probs ? aligned16(a->draft_probs, a->draft_stride * elem_size(draft_dtype)) : false;
  p.noise_aligned = a->exp_noise ? aligned16(a->exp_noise, a->noise_stride * 4) : false;
  p.ctrl = reinterpret_cast<int*>(ws + lay.ctrl);
  p.req_cnt = reinterpret_cast<int*>(ws + lay.req_cnt);
  p.score_cnt = reinterpret_cast<int*>(ws + lay.score_cnt);
  p.decision = reinterpret_cast<int*>(ws + lay.decision);
  p.top_k = masked ? a->top_k : nullptr;
  p.top_p = masked ? a->top_p : nullptr;
  p.masks = masked ? reinterpret_cast<float4*>(ws + lay.masks) : nullptr;
  p.order = masked ? reinterpret_cast<int*>(ws + lay.order) : nullptr;
  p.stat_slots = reinterpret_cast<uint64_t*>(ws + lay.stat_slots);
  p.score_slots = reinterpret_cast<uint64_t*>(ws + lay.score_slots);
  p.debug_row_stats = a->debug_row_stats;

  // The row masks of the whole batch, then one verify launch per kMaxLaunchRequests requests
  // (their tables live in LDS); the launches share the workspace, which each leaves zeroed.
  if (masked) {
    err = mvsd::launch_constraints(p, a->target_dtype, (hipStream_t)stream);
    if (err != hipSuccess) return hip_status(err);
  }
  const int groups_per_req = (int)((a->max_spec_len + size_plan.g - 1) / size_plan.g);
  for (int64_t r0 = 0; r0 < B; r0 += mvsd::kMaxLaunchRequests) {
    const int64_t Bl = launch_requests(B - r0);
    mvsd::VerifyParams q = p;
    q.B = (int)Bl;
    q.out = p.out + r0 * p.out_stride;
    q.bonus = p.bonus + r0;
    q.cu = p.cu + r0;
    q.cu_prev = r0 > 0 ? p.cu + r0 - 1 : nullptr;
    if (p.temperature) q.temperature = p.temperature + r0;
    if (p.noise) q.noise = p.noise + r0 * p.noise_stride;
    if (p.top_k) q.top_k = p.top_k + r0;
    if (p.top_p) q.top_p = p.top_p + r0;
    // Units: at most one stats unit per group and one score unit per random request.
    int64_t groups = Bl * groups_per_req;
    if (groups > P) groups = P;
    const int64_t units = groups + (scores ? Bl : 0);
    const mvsd::VerifyPlan plan = mvsd::verify_plan(a->target_dtype, V, units, cap, batch_rows, scores);
    q.chunk = plan.chunk;
    q.nc = plan.nc;
    int64_t grid = units * plan.nc;
    if (grid > cap) grid = cap;
    if (grid < 1) grid = 1;
    // A request's score unit comes `lag` stats units after its last one.  Each resident
    // workgroup holds two tickets, and a decision appears shortly after the request's last stats
    // task ends, so about three tickets per workgroup between the two (lag stats units and about
    // as many score units) let the score tasks find their decision published, while the
    // rejected row is still likely to be in the Infinity Cache.
    q.lag = (int)((3 * grid + 2 * plan.nc - 1) / (2 * plan.nc)) + 2;
    // The last groups' stats tasks and every score task after them cover half chunks, so
    // that the dependent decisions and scores at the end of the launch are short.  Half
    // tasks cost more per byte, so the tail groups hold about one half-chunk stats ticket per
    // two workgroups (a quarter of that, or none, measured 0.3-1.2 % slower on bf16 batches).
    q.tail_groups = (int)((grid + 4 * plan.nc - 1) / (4 * plan.nc));
    // A launch without score units whose tasks all start at once has no end to shorten: half
    // tasks there would only give some workgroups a second task.
    if (!scores && units * plan.nc <= cap) q.tail_groups = 0;
    // every workgroup may claim two tickets past the last task
    if (units * 2 * plan.nc > 0x7fffffff - 4 * grid) return MVSD_E_RANGE;
    err = mvsd::launch_verify(q, a->target_dtype, (int)grid, (hipStream_t)stream);
    if (err != hipSuccess) return hip_status(err);
  }
  return MVSD_OK;
}

// Static scratch of mvsd_rejection_sample_static: one per device that the library runs on, held
// until the process ends.  Host code never uses the array's name as an address: the device
// address comes from hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

struct StaticScratch {
  std::mutex mu;
  void* ptr[kMaxDevices] = {};
};

StaticScratch& static_scratch() {
  static StaticScratch s;
  return s;
}

// The calling thread's current device's scratch address; on the first call for a device also
// zero-fills the scratch with a kernel on `stream` (the verify workspace contract).
int static_scratch_for_current_device(void** out, hipStream_t stream) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_status(err);
  if (device < 0 || device >= kMaxDevices) return MVSD_E_RANGE;
  StaticScratch& st = static_scratch();
  std::lock_guard<std::mutex> lock(st.mu);
  if (!st.ptr[device]) {
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess) return hip_status(err);
    if (!ptr) return hip_status(hipErrorInvalidSymbol);
    err = mvsd::launch_zero_fill(ptr, kStaticScratchBytes, stream);
    if (err != hipSuccess) return hip_status(err);
    st.ptr[device] = ptr;
  }
  *out = st.ptr[device];
  return MVSD_OK;
}

}  // namespace

extern "C" {

int mvsd_rejection_sample(const mvsd_rejection_args* a, mvsd_stream_t stream) {
  if (!a) return MVSD_E_INVALID;
  return rejection_sample_impl(a, a->workspace, a->workspace_bytes, stream);
}

int64_t mvsd_rejection_static_scratch_bytes(void) { return kStaticScratchBytes; }

int mvsd_rejection_sample_static(const mvsd_rejection_args* a, mvsd_stream_t stream) {
  if (!a) return MVSD_E_INVALID;
  if (a->batch_size < 0 || a->num_tokens < 0 || a->vocab_size <= 0) return MVSD_E_INVALID;
  const int64_t need = mvsd_rejection_workspace_bytes(a->batch_size, a->num_tokens,
                                                      a->vocab_size, a->target_dtype,
                                                      a->max_spec_len);
  if (need < 0) return MVSD_E_INVALID;
  if (need > kStaticScratchBytes) return MVSD_E_SCRATCH;
  if (a->batch_size == 0) return MVSD_OK;
  void* ws = nullptr;
  const int st = static_scratch_for_current_device(&ws, (hipStream_t)stream);
  if (st != MVSD_OK) return st;
  return rejection_sample_impl(a, ws, kStaticScratchBytes, stream);
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
  if (k > vocab_size) return MVSD_E_RANGE;
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
  p.flat = 0;
  p.rank_raw = 0;
  p.ids = ids;
  p.lps = lps;
  p.ranks = ranks;
  return hip_status(mvsd::launch_spec_logprobs(p, (hipStream_t)stream));
}

int mvsd_topk_scores(int32_t* ids, float* scores, int32_t* ranks, const float* logits,
                     int64_t logits_stride, const int32_t* token_ids, int64_t num_rows,
                     int64_t vocab_size, int64_t k, int logits_mode, mvsd_stream_t stream) {
  if (num_rows < 0 || vocab_size <= 0 || k < 0) return MVSD_E_INVALID;
  if (num_rows == 0) return MVSD_OK;
  if (k > vocab_size) return MVSD_E_RANGE;
  if (num_rows > 0x7fffffff || vocab_size > 0x7fffffff) return MVSD_E_RANGE;
  if (!ids || !scores || !ranks || !logits || !token_ids || logits_stride < vocab_size)
    return MVSD_E_INVALID;
  mvsd::LogprobParams p{};
  p.bonus = logits;
  p.bstride = logits_stride;
  p.tokens = token_ids;
  p.B = (int)num_rows;
  p.W = 1;
  p.V = (int)vocab_size;
  p.k = (int)k;
  p.logits_mode = logits_mode ? 1 : 0;
  p.flat = 1;
  p.rank_raw = 1;
  p.ids = ids;
  p.lps = scores;
  p.ranks = ranks;
  return hip_status(mvsd::launch_spec_logprobs(p, (hipStream_t)stream));
}

int mvsd_sampler_rows(int op, int32_t* ids, float* out, int64_t out_stride, float* x,
                      int64_t stride, const float* aux, int64_t aux_stride, int64_t num_rows,
                      int64_t vocab_size, mvsd_stream_t stream) {
  // op 2 (the exponential race) is mvsd_sampler_race
  if (num_rows < 0 || vocab_size <= 0 || op < 0 || op > 3 || op == 2) return MVSD_E_INVALID;
  if (num_rows == 0) return MVSD_OK;
  if (num_rows > 0x7fffffff || vocab_size > 0x7fffffff) return MVSD_E_RANGE;
  if (!x || stride < vocab_size) return MVSD_E_INVALID;
  if (op == mvsd::kSamplerArgmax && !ids) return MVSD_E_INVALID;
  if (op == mvsd::kSamplerMinP && !aux) return MVSD_E_INVALID;
  if (op == mvsd::kSamplerLogSoftmax && (!out || out_stride < vocab_size)) return MVSD_E_INVALID;
  return hip_status(mvsd::launch_sampler_rows(op, ids, out, out_stride, x, stride, aux,
                                              aux_stride, num_rows, vocab_size,
                                              (hipStream_t)stream));
}

int64_t mvsd_sampler_race_workspace_bytes(int64_t num_rows, int64_t vocab_size) {
  if (num_rows < 0 || vocab_size <= 0) return MVSD_E_INVALID;
  return mvsd::sampler_race_workspace_bytes(num_rows, vocab_size);
}

int mvsd_sampler_race(int32_t* ids, const float* x, int64_t stride, const float* noise,
                      int64_t noise_stride, const float* temperature, int64_t num_rows,
                      int64_t vocab_size, void* workspace, int64_t workspace_bytes,
                      mvsd_stream_t stream) {
  // positive divisors only: no row is greedy (greedy_eps 0)
  if (!noise) return MVSD_E_INVALID;
  return mvsd_sampler_race_rows(ids, x, MVSD_F32, stride, nullptr, num_rows, noise,
                                noise_stride, temperature, 0.0f, num_rows, vocab_size,
                                workspace, workspace_bytes, stream);
}

int mvsd_sampler_race_rows(int32_t* ids, const void* x, int x_dtype, int64_t stride,
                           const int32_t* row_index, int64_t num_x_rows, const float* noise,
                           int64_t noise_stride, const float* temperature, float greedy_eps,
                           int64_t num_rows, int64_t vocab_size, void* workspace,
                           int64_t workspace_bytes, mvsd_stream_t stream) {
  if (num_rows < 0 || vocab_size <= 0) return MVSD_E_INVALID;
  if (num_rows == 0) return MVSD_OK;
  if (x_dtype != MVSD_F32 && x_dtype != MVSD_BF16 && x_dtype != MVSD_F16) return MVSD_E_INVALID;
  if (vocab_size > (int64_t)mvsd::kRaceChunk * mvsd::kRaceMaxChunks) return MVSD_E_RANGE;
  const int64_t nch = (vocab_size + mvsd::kRaceChunk - 1) / mvsd::kRaceChunk;
  if (num_rows * nch >= (1ll << 24)) return MVSD_E_RANGE;  // grid threads < 2^32
  if (!ids || !x || stride < vocab_size || (noise && noise_stride < vocab_size))
    return MVSD_E_INVALID;
  if (row_index ? num_x_rows <= 0 : num_x_rows < num_rows) return MVSD_E_INVALID;
  if (!(greedy_eps >= 0.0f)) return MVSD_E_INVALID;
  if (!workspace || workspace_bytes < mvsd::sampler_race_workspace_bytes(num_rows, vocab_size))
    return MVSD_E_WORKSPACE;
  return hip_status(mvsd::launch_sampler_race(ids, x, x_dtype, stride, row_index, num_x_rows,
                                              noise, noise_stride, temperature, greedy_eps,
                                              num_rows, vocab_size, workspace,
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
