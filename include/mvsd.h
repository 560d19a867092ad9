/*
 * mvsd.h — C ABI of the MI355X speculative-decoding verification library (libmvsd.so).
 *
 * Every entry point takes raw device pointers, element strides, dtype codes and a
 * hipStream_t, enqueues work on that stream, never synchronises the host and never
 * allocates device memory: scratch comes from a caller-owned workspace whose size is
 * returned by the matching *_workspace_bytes() query.  Each returns 0 on success or a
 * negative MVSD_E_* code; mvsd_status_string() turns a code into text.  A host-side
 * wrapper turns a non-zero code into an exception, the same pattern the reference uses
 * for its own ctypes-loaded kernels (minivllm/layers/ops/rms_norm_cuda.py:95-112,163-188).
 *
 * Row conventions follow the reference:
 *   - "verify rows" are the P = sum_i K_i draft positions, request-major
 *     (minivllm/spec_decode/metadata.py:31-39);
 *   - cu_num_draft_tokens is the inclusive prefix sum of K_i WITHOUT a leading 0
 *     (minivllm/spec_decode/metadata.py:49-52);
 *   - outputs are [B, max_spec_len + 1] int32 padded with -1
 *     (minivllm/sample/rejection_sampler.py:79,462-467).
 */
#ifndef MVSD_H_
#define MVSD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is an opaque pointer; callers pass torch.cuda.current_stream().cuda_stream. */
typedef void* mvsd_stream_t;

/* dtype codes for logits / probabilities / expanded values */
enum {
  MVSD_F32 = 0,
  MVSD_BF16 = 1,
  MVSD_F16 = 2,
  MVSD_F64 = 3,
  MVSD_I32 = 4,
  MVSD_I64 = 5,
  MVSD_U8 = 6
};

/* status codes */
enum {
  MVSD_OK = 0,
  MVSD_E_INVALID = -1,     /* bad argument (shape, null pointer, unsupported dtype) */
  MVSD_E_ALIGN = -2,       /* pointer/stride alignment the kernel needs is not met */
  MVSD_E_WORKSPACE = -3,   /* workspace missing or too small */
  MVSD_E_HIP = -4,         /* a HIP runtime call failed; see mvsd_last_hip_error() */
  MVSD_E_RANGE = -5,       /* a size exceeds what the kernel supports */
  MVSD_E_SCRATCH = -6      /* the static scratch is too small for the batch */
};

/* Library version, (major << 16) | (minor << 8) | patch. */
int mvsd_version(void);
/* Human-readable text of a status code. */
const char* mvsd_status_string(int status);
/* The hipError_t of the last failing HIP call in this thread (0 if none). */
int mvsd_last_hip_error(void);

/* ------------------------------------------------------------------------------------ */
/* expand_batch_to_tokens                                                                 */
/* Replaces: expand_batch_to_tokens + expand_kernel,                                     */
/*           minivllm/sample/rejection_sampler.py:574-597 and :826-847.                   */
/* out[j] = (x[i] == replace_from ? replace_to : x[i]) for every j in request i's range   */
/* [cu[i-1], cu[i]).  dtype in {F32, F64, I32, I64, U8}; out has x's dtype.               */
/* ------------------------------------------------------------------------------------ */
int mvsd_expand_batch_to_tokens(void* out, const void* x, int dtype,
                                const int32_t* cu_num_tokens, int64_t batch_size,
                                int64_t num_tokens, double replace_from, double replace_to,
                                mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* rejection_sample — fused verification of a whole batch, one persistent launch per 4096  */
/* requests.                                                                              */
/* Replaces: rejection_sample (minivllm/sample/rejection_sampler.py:414-534) together    */
/* with what it launches: target softmax (:502), target argmax (:485),                   */
/* rejection_greedy_sample_kernel (:678-740), sample_recovered_tokens + its kernel       */
/* (:627-670, :850-928) and rejection_random_sample_kernel (:744-822); and, when          */
/* apply_temperature != 0, the temperature divide of apply_sampling_constraints (:553-561)*/
/* that RejectionSampler.forward (:195-196) runs before it; and, when top_k or top_p is   */
/* given (and not all_greedy), the top-k / top-p masking of that function (:563-571,      */
/* minivllm/sample/ops/topk_topp_sampler.py:48-79) applied to the divided rows.           */
/*                                                                                        */
/* Request i is greedy iff all_greedy != 0 or temperature[i] == 0 (:469-473).            */
/* Random requests need exp_noise (one Exp(1) row per request, :648-655) unless           */
/* recovered_token_ids is given; uniform_probs is fp64 [P] (:600-624).                    */
/* ------------------------------------------------------------------------------------ */
typedef struct mvsd_rejection_args {
  /* output [batch_size, max_spec_len + 1] int32, row stride out_stride elements */
  int32_t* output_token_ids;
  int64_t out_stride;

  /* target logits: verify row j is at target_logits + target_rows[j] * target_stride
   * (target_rows == NULL means row j).  dtype F32, BF16 or F16; upcast to fp32 in-kernel. */
  const void* target_logits;
  int target_dtype;
  int64_t target_stride;
  const int32_t* target_rows;
  int64_t target_num_rows;              /* rows addressable from target_logits (indices are clamped) */

  /* draft probabilities [P, V], dtype F32, BF16 or F16 (upcast to fp32 in-kernel, as the
   * reference's kernels load them in their own dtype, :797-806, :882-890), or NULL for
   * point-mass drafts
   * (ngram: q[d] = 1, recovered distribution = p with the draft id removed, :793-795,:891-897) */
  const void* draft_probs;
  int draft_dtype;
  int64_t draft_stride;

  /* Exp(1) noise [batch_size, V] fp32, one row per request; may be NULL when every
   * request is greedy or recovered_token_ids is given */
  const float* exp_noise;
  int64_t noise_stride;

  const double* uniform_probs;          /* [P] fp64; may be NULL when all greedy and not synthetic */
  const int32_t* draft_token_ids;       /* [P] */
  const int32_t* cu_num_draft_tokens;   /* [batch_size], no leading 0 */
  const int32_t* bonus_token_ids;       /* [batch_size] */

  const float* temperature;             /* [batch_size] fp32, or NULL when all_greedy */
  int all_greedy;
  int apply_temperature;                /* 1: divide logits by T (T==0 -> 1) in-kernel */

  const int32_t* recovered_token_ids;   /* optional [P] override of the recovered ids */
  const float* synthetic_conditional_rates; /* optional [>= max_spec_len]; enables synthetic mode */

  int64_t batch_size;
  int64_t num_tokens;                   /* P */
  int64_t vocab_size;                   /* V */
  int64_t max_spec_len;                 /* <= 128 */

  void* workspace;                      /* >= mvsd_rejection_workspace_bytes(...) bytes */
  int64_t workspace_bytes;

  /* Optional per-request sampling constraints on the verify rows (NULL = none): keep the
   * top_k[i] largest values (k <= 0 or k >= V keeps all) and the smallest set of largest
   * values whose probability reaches top_p[i] (p >= 1 keeps all).  Masked entries get
   * probability 0 and are never a greedy argmax, as the reference's -inf does. */
  const int64_t* top_k;                 /* [batch_size] */
  const float* top_p;                   /* [batch_size] */

  /* Optional read-out (NULL = none), for tests and diagnostics; no counterpart in the
   * reference.  [num_tokens, 3] fp32: for each verify row of a random request, the row's raw
   * maximum M, its sum S of exp((x - M) / T) (as combined by the kernel), and the fp32
   * probability of the draft token that the acceptance test compared, p[d] =
   * exp(x_d / T - M / T) / S (0 where the sampling constraints mask d).  Rows of greedy
   * requests are not written. */
  float* debug_row_stats;
} mvsd_rejection_args;

/* Workspace contract: zero-filled before its first use (mvsd_rejection_workspace_init, or
 * any zeroed allocation); every call leaves it zero-filled again, also after a failed call.
 * One workspace must not be used by two calls that can run concurrently (different streams).
 * Sizes: the query below is monotone in every argument, so a workspace sized for the largest
 * batch serves smaller ones.
 *
 * Failure: the kernel's cross-workgroup waits are bounded (about 0.3 s of polling, see
 * mvsd_set_wait_limit).  When a wait gives up, every output entry of the requests whose
 * inputs were incomplete is set to MVSD_POISON (INT32_MIN, never a token id), and the
 * workspace is still returned to zero, so the next call is unaffected.  The caller detects
 * the failure on its existing device-to-host copy of the output (the reference's
 * parse_output, rejection_sampler.py:320); the Python layer raises RuntimeError there. */
#define MVSD_POISON ((int32_t)0x80000000)
int64_t mvsd_rejection_workspace_bytes(int64_t batch_size, int64_t num_tokens,
                                       int64_t vocab_size, int target_dtype,
                                       int64_t max_spec_len);
/* Zero-fill a workspace on `stream` with a kernel (no hipMemsetAsync). */
int mvsd_rejection_workspace_init(void* workspace, int64_t workspace_bytes, mvsd_stream_t stream);
/* Polls after which a wait inside mvsd_rejection_sample gives up, for calls made from now on
 * (process-wide; polls < 0 restores the default, 0 makes every wait give up at once so that
 * tests can exercise the failure path while every kernel still exits normally).  Returns the
 * previous limit.  No counterpart in the reference. */
int mvsd_set_wait_limit(int polls);
int mvsd_rejection_sample(const mvsd_rejection_args* args, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* rejection_sample_static — mvsd_rejection_sample without a workspace argument.           */
/* No counterpart in the reference: it is for callers that cannot allocate device memory  */
/* (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).   */
/* The workspace fields of *args are ignored; the scratch is a static device array of      */
/* mvsd_rejection_static_scratch_bytes() bytes (16 MiB) that the library holds on every    */
/* device it runs on until the process ends, zero-filled by a kernel on the first call for */
/* a device.  Nothing is allocated.  A batch whose mvsd_rejection_workspace_bytes(...)      */
/* exceeds the scratch returns MVSD_E_SCRATCH.  Every call on one device shares that        */
/* device's scratch, so calls that can overlap on one device (different streams) race.     */
/* Results, failure behaviour and everything else are those of mvsd_rejection_sample.      */
/* ------------------------------------------------------------------------------------ */
int64_t mvsd_rejection_static_scratch_bytes(void);
int mvsd_rejection_sample_static(const mvsd_rejection_args* args, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* sampling_masks — the per-row masks mvsd_rejection_sample applies for top_k / top_p.     */
/* Replaces: nothing directly; it exposes, as thresholds, what apply_sampling_constraints  */
/* (minivllm/sample/rejection_sampler.py:537-571) does to the verify rows.  Reads the      */
/* target, cu_num_draft_tokens, temperature / all_greedy / apply_temperature, top_k and    */
/* top_p fields of *args.  masks: [num_tokens, 4] fp32, 16-byte aligned; row j gets        */
/* (A, B, J as int bits, 0): entry i of verify row j, raw value x (before the temperature  */
/* divide), is masked iff x < A || (x < B && i <= J).  Rows without constraints get        */
/* (-inf, -inf, -1), and so do the rows of greedy requests whose argmax no mask can change */
/* (top-k never masks a maximum; top-p masks one only when the maximum is tied and the     */
/* entries below it hold at most 1 - p of the mass).                                        */
/* ------------------------------------------------------------------------------------ */
int mvsd_sampling_masks(const mvsd_rejection_args* args, float* masks, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* softmax_rows — probs[j, :] = softmax(logits[row_j, :] / t_j) in fp32.                 */
/* Replaces: target_logits.softmax(dim=-1, dtype=float32),                               */
/*           minivllm/sample/rejection_sampler.py:502.  temperature may be NULL (t = 1);  */
/* otherwise t_j = temperature[j] with 0 -> 1.                                            */
/* ------------------------------------------------------------------------------------ */
int mvsd_softmax_rows(float* probs, int64_t probs_stride, const void* logits, int dtype,
                      int64_t logits_stride, const float* temperature, int64_t num_rows,
                      int64_t vocab_size, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* sample_recovered_tokens — argmax_v max(p - q, 0) * (1 / E[req, v]) per verify row.    */
/* Replaces: sample_recovered_tokens + sample_recovered_tokens_kernel,                   */
/*           minivllm/sample/rejection_sampler.py:627-670 and :850-928 (noise supplied). */
/* draft_probs == NULL selects the point-mass form (p with the draft id masked).          */
/* ------------------------------------------------------------------------------------ */
int mvsd_sample_recovered_tokens(int32_t* recovered_token_ids, const int32_t* cu_num_draft_tokens,
                                 const int32_t* draft_token_ids, const float* draft_probs,
                                 int64_t draft_stride, const float* target_probs,
                                 int64_t target_stride, const float* exp_noise,
                                 int64_t noise_stride, int64_t batch_size, int64_t num_tokens,
                                 int64_t vocab_size, int64_t max_spec_len, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* apply_top_k_top_p — mask non-candidate logits to -inf, in place.                        */
/* Replaces: apply_top_k_top_p, minivllm/sample/ops/topk_topp_sampler.py:48-79, as called  */
/*           by apply_sampling_constraints (minivllm/sample/rejection_sampler.py:563-571). */
/* logits: fp32 rows at logits + r * logits_stride.  top_k [num_rows] int64 (NULL = none):  */
/* keep values >= the k-th largest (ties kept); k <= 0 or k >= V keeps the whole row.       */
/* top_p [num_rows] fp32 (NULL = none): over the top-k-masked row, mask the ascending       */
/* (value, then index) prefix whose cumulative softmax mass is <= 1 - p, never the largest  */
/* entry; p >= 1 masks nothing (the reference's p = 1 masks only entries whose fp32       */
/* probability underflows to 0).  Requires 1 <= V < 2^31.                                 */
/* ------------------------------------------------------------------------------------ */
int mvsd_apply_top_k_top_p(float* logits, int64_t logits_stride, const int64_t* top_k,
                           const float* top_p, int64_t num_rows, int64_t vocab_size,
                           mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* ngram_valid_sampled — the valid sampled tokens of one step, per request.               */
/* Replaces: NgramProposerGPU.update_token_ids_ngram                                     */
/*           (minivllm/spec_decode/ngram_proposer_gpu.py:247-290).                        */
/*                                                                                        */
/* sampled [num_reqs, width] int32 (row stride sampled_stride); discard [num_reqs] uint8  */
/* (NULL = keep all).  valid_ids [num_reqs, width] = sampled, or -1 for discarded rows.   */
/* counts[i] = #{j : valid_ids[i, j] != -1 and valid_ids[i, j] < vocab_size}.             */
/* next_token_ids[i] = valid_ids[i, counts[i] - 1] when counts[i] > 0, else               */
/* token_ids[i, max(num_tokens[i] - 1, 0)] (clamped to the row).                          */
/* ------------------------------------------------------------------------------------ */
int mvsd_ngram_valid_sampled(int32_t* next_token_ids, int32_t* counts, int32_t* valid_ids,
                             int64_t valid_stride, const int32_t* sampled,
                             int64_t sampled_stride, int64_t width, const uint8_t* discard,
                             const int32_t* token_ids, int64_t row_stride,
                             const int32_t* num_tokens, int64_t vocab_size, int64_t num_reqs,
                             mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* ngram_propose — prompt-lookup drafts for a batch of int32 token histories.            */
/* Replaces: NgramGPUKernel._find_first_and_extract_all_n_parallel + forward             */
/*           (minivllm/spec_decode/ngram_proposer_gpu.py:56-148) with the in-place       */
/*           history scatter of NgramProposerGPU.propose (:222-241) when new_tokens is   */
/*           given; and, with cap_by_model_len != 0, the CPU matcher                     */
/*           _find_longest_matched_ngram_and_propose_tokens                              */
/*           (minivllm/spec_decode/ngram_proposer.py:41-99) used by batch_propose        */
/*           (:152-184).                                                                  */
/*                                                                                        */
/* token_ids [num_reqs, row_stride] int32 (written in place when new_tokens != NULL).     */
/* num_tokens [num_reqs] int32 lengths (read only).  Row i is matched on length           */
/* L_i = num_tokens[i] + new_counts[i] (new_counts NULL -> 0), clamped to max_seq_len.    */
/* active [num_reqs] uint8 (NULL = all active): inactive rows get drafts of -1.          */
/* gate_on_new_counts != 0 additionally deactivates rows with new_counts[i] == 0 or       */
/* L_i < min_n (the combined_mask of NgramProposerGPU.propose, :239-241).                 */
/* GPU form (cap_by_model_len == 0): drafts [num_reqs, k] -1 padded, num_valid = count of */
/* leading valid drafts.  CPU form (cap_by_model_len != 0): k_i = min(k, max_model_len -  */
/* L_i); rows with L_i < min_n or k_i <= 0 give no drafts; num_valid = drafts copied.     */
/* Limits: 1 <= min_n <= max_n <= 32, 1 <= k <= 256, max_seq_len <= row_stride < 2^31.   */
/* ------------------------------------------------------------------------------------ */
int mvsd_ngram_propose(int32_t* drafts, int32_t* num_valid, int32_t* token_ids,
                       int64_t row_stride, int64_t max_seq_len, const int32_t* num_tokens,
                       const int32_t* new_tokens, int64_t new_tokens_stride,
                       int64_t max_new_tokens, const int32_t* new_counts,
                       const uint8_t* active, int gate_on_new_counts, int64_t num_reqs,
                       int32_t min_n, int32_t max_n, int32_t k, int cap_by_model_len,
                       int64_t max_model_len, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* apply_logits_processors — penalties and min_tokens of the verify rows, in place.        */
/* Replaces: RejectionSampler.apply_logits_processors / apply_penalties /                  */
/*           _combine_outputs_with_spec_tokens, minivllm/sample/rejection_sampler.py:338-406, */
/*           with apply_all_penalties, minivllm/sample/ops/penalties.py:51-72, and          */
/*           Sampler.apply_min_tokens_for_spec_decode, minivllm/sample/sampler.py:192-228.   */
/* logits: fp32 verify rows (num_tokens of them, request-major) at logits + j * stride.    */
/* Row j of request r (rows cu[r-1] .. cu[r]-1, cu without a leading 0) has the history    */
/* "committed output + spec_tokens of its request before row j".  Penalties (ent_off NULL:  */
/* none): ent_tok[ent_off[r] .. ent_off[r+1]) lists request r's distinct prompt, output and */
/* draft tokens, ent_info the committed output count | in_prompt << 31; for each listed    */
/* token t with count c (committed + earlier drafts equal to t):                           */
/*   if in_prompt or c > 0: x *= x > 0 ? 1 / repetition[r] : repetition[r];               */
/*   x -= frequency[r] * c;  x -= presence[r] * (c > 0)   (fp32, in this order).           */
/* presence / frequency / repetition [B] fp32, NULL = 0 / 0 / 1.  Then min_tokens (n_mask   */
/* NULL: none): the first n_mask[r] rows of request r get stop_tok[stop_off[r] ..          */
/* stop_off[r+1]) set to -inf.  Tokens outside [0, vocab_size) are skipped.                */
/* ------------------------------------------------------------------------------------ */
int mvsd_apply_logits_processors(float* logits, int64_t stride, int64_t num_tokens,
                                 int64_t vocab_size, int64_t batch_size,
                                 const int32_t* cu_num_draft_tokens, const int32_t* spec_tokens,
                                 const int32_t* ent_off, const int32_t* ent_tok,
                                 const int32_t* ent_info, const float* presence,
                                 const float* frequency, const float* repetition,
                                 const int32_t* n_mask, const int32_t* stop_off,
                                 const int32_t* stop_tok, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* spec_logprobs — logprobs of every output position of a verification step.              */
/* Replaces: RejectionSampler._get_logprobs_tensors, minivllm/sample/rejection_sampler.py: */
/*           229-300, with Sampler.compute_logprobs / gather_logprobs /                    */
/*           batched_count_greater_than, minivllm/sample/sampler.py:313-349.               */
/* Position (r, j), j < width, reads compact row start_r + j (clamped to num_tokens +      */
/* batch_size - 1), where the compact rows are each request's verify rows then its bonus   */
/* row and start_r = cu_num_sampled_tokens[r-1] (0 for r = 0; no leading 0 in the array).  */
/* Verify row v is target + t * target_stride with t = target_rows[v] (or v if NULL); the   */
/* bonus row of request q is bonus + q * bonus_stride; both fp32.  Token =                 */
/* sampled_token_ids[r * sampled_stride + j], -1 read as 0.  With lp(x) the fp32            */
/* log-softmax (x - max) - log(sum exp(x - max)) of the row (logits_mode != 0: lp(x) = x): */
/*   ids[n, 0] = token, lps[n, 0] = lp(x_token); ids / lps[n, 1 .. k] = the k largest lp    */
/*   by (value desc, index asc); ranks[n] = #{i : lp(x_i) >= lp(x_token)};                  */
/* n = r * width + j; ids / lps are [batch_size * width, k + 1].  0 <= k <= V.                */
/* ------------------------------------------------------------------------------------ */
int mvsd_spec_logprobs(int32_t* ids, float* lps, int32_t* ranks, const float* target,
                       int64_t target_stride, const int32_t* target_rows, const float* bonus,
                       int64_t bonus_stride, const int32_t* cu_num_sampled_tokens,
                       const int32_t* sampled_token_ids, int64_t sampled_stride,
                       int64_t batch_size, int64_t num_tokens, int64_t vocab_size,
                       int64_t width, int64_t k, int logits_mode, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* sampler_rows — row operations of the regular sampler on fp32 rows x + r * stride.       */
/* Replaces, in minivllm/sample/sampler.py: greedy_sample (:295-298, op 0: ids[r] = argmax */
/* of row r, NaN first, lowest index on ties), apply_min_p (:280-293, op 1: with p the      */
/* softmax of row r, entries with p < max(p) * aux[r] become -inf in place; aux[r] <= 0     */
/* leaves the row), compute_logprobs (:313-315, op 3: out row r = (x - max) - log(sum      */
/* exp(x - max))).  Op 2 is invalid: the exponential race is mvsd_sampler_race.            */
/* ------------------------------------------------------------------------------------ */
int mvsd_sampler_rows(int op, int32_t* ids, float* out, int64_t out_stride, float* x,
                      int64_t stride, const float* aux, int64_t aux_stride, int64_t num_rows,
                      int64_t vocab_size, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* sampler_race — random_sample, minivllm/sample/ops/topk_topp_sampler.py:82-90, with the  */
/* softmax before it (:73-80) and, when temperature is given, the temperature divide of    */
/* Sampler.sample (minivllm/sample/sampler.py:263-268) folded in: ids[r] = argmax over i of */
/* softmax(v)_i / noise[r][i] with v = fl(x[r][i] / temperature[r]) (or x[r][i] when       */
/* temperature is NULL).  The row's max and sum are common to its entries, so the argmax   */
/* is evaluated as that of v log2(e) - log2(noise[r][i]) in one pass; the keys differ from */
/* the reference's fp32 roundings of exp(v - M) / S / noise by a few ulps of |v| log2(e) + */
/* |log2 noise|, so only closer near-ties can pick another index.  A row the reference     */
/* maps to all-NaN probabilities (a NaN or +inf value, or every value -inf) gives 0; NaN   */
/* first, lowest index on ties.  temperature [num_rows] fp32 holds positive divisors (the  */
/* reference's safe temperatures: 1 for greedy rows).  Rows of 8192 columns are spread     */
/* over workgroups; workspace: >= mvsd_sampler_race_workspace_bytes(num_rows, V) bytes of   */
/* device memory, no initialisation needed.  V <= 8388608.                                  */
/* ------------------------------------------------------------------------------------ */
int64_t mvsd_sampler_race_workspace_bytes(int64_t num_rows, int64_t vocab_size);
int mvsd_sampler_race(int32_t* ids, const float* x, int64_t stride, const float* noise,
                      int64_t noise_stride, const float* temperature, int64_t num_rows,
                      int64_t vocab_size, void* workspace, int64_t workspace_bytes,
                      mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* sampler_race_rows — the bonus-row sampling of RejectionSampler.forward                  */
/* (minivllm/sample/rejection_sampler.py:169-181: logits[bonus_logits_indices] through      */
/* Sampler.forward, minivllm/sample/sampler.py:73-120, :243-278) when no logits processor, */
/* min_p, top-k or top-p applies: the race of mvsd_sampler_race on rows picked in place,   */
/* without the gather and the fp32 upcast.  Row r is x + row_index[r] * stride (row_index  */
/* clamped to [0, num_x_rows); NULL: x + r * stride, num_x_rows >= num_rows), x_dtype       */
/* MVSD_F32 / MVSD_BF16 / MVSD_F16, upcast exactly.  With temperature, a row whose          */
/* temperature is below greedy_eps (the reference's SAMPLING_EPS, 1e-5) is greedy: its id  */
/* is the argmax of the raw row (greedy_sample, sampler.py:295-298) and its noise row is    */
/* not read; the other rows race on fl(x / T).  noise NULL makes every row greedy.          */
/* Same workspace as mvsd_sampler_race.                                                     */
/* ------------------------------------------------------------------------------------ */
int mvsd_sampler_race_rows(int32_t* ids, const void* x, int x_dtype, int64_t stride,
                           const int32_t* row_index, int64_t num_x_rows, const float* noise,
                           int64_t noise_stride, const float* temperature, float greedy_eps,
                           int64_t num_rows, int64_t vocab_size, void* workspace,
                           int64_t workspace_bytes, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* selftest — on-device check of an arithmetic assumption of the kernels.  No counterpart   */
/* in the reference.  test 0: the FMA-corrected hardware reciprocal used for 1/E equals     */
/* IEEE fp32 division for every b in [2^-126, 2^126).  test 1: the corrected division x/T  */
/* used by the sampling-constraint kernel equals IEEE fp32 division for every float x at   */
/* sixteen divisors.  Adds the number of mismatches to *failures (a device uint64 the      */
/* caller zeroes).                                                                         */
/* ------------------------------------------------------------------------------------ */
int mvsd_selftest(int test, uint64_t* failures, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* v2_rejection_sample — the V2 model runner's verification, standard or block.          */
/* Replaces: rejection_sample (minivllm/worker/gpu/spec_decode/rejection_sampler_utils.py: */
/*           935-1201): _compute_local_logits_stats_kernel (:206-316),                    */
/*           _compute_cumulative_log_p_kernel (:318-384), _compute_local_residual_mass_     */
/*           kernel (:387-446), _rejection_kernel (:497-706), _resample_kernel (:709-866), */
/*           _insert_resampled_kernel (:869-932), and the counter draws of                  */
/*           minivllm/worker/gpu/sample/gumbel.py:72-131 (Philox4x32-10, as Triton's        */
/*           tl.randint4x / tl.rand).                                                       */
/* target_logits [num_logits, V] (F32/BF16/F16, already temperature-scaled, as the         */
/* reference assumes); draft_logits [states, K, V] pre-temperature or NULL; draft_sampled  */
/* [num_logits] int32 (entry j+1 is the draft at row j); cu_num_logits [num_reqs + 1]      */
/* int32 with a leading 0; pos [num_logits] int64; idx_mapping [num_reqs] and              */
/* expanded_idx_mapping / expanded_local_pos [num_logits] int32 (row j of request r has    */
/* state idx_mapping[r] and local position j - cu_num_logits[r], as the V2 runner builds   */
/* them); temperature [states] f32; seed [states] int64; synthetic_conditional_rates [K]   */
/* f32 or NULL.  use_block_verification selects block verification (Sun et al. 2024) for  */
/* random requests; it cannot be combined with synthetic rates (MVSD_E_INVALID).  Writes   */
/* sampled [num_reqs, >= K+1] int64 (entries at or past num_sampled[r] are left as they    */
/* were, or hold a rejected draft) and num_sampled [num_reqs] int32.  workspace:           */
/* mvsd_v2_workspace_bytes() bytes, 256-byte aligned, caller-owned, no initial contents    */
/* needed.  Draft ids >= V count as invalid (the reference does not check them); a request */
/* whose cu_num_logits span is empty, out of range or longer than K+1 gets num_sampled 0.  */
/* ------------------------------------------------------------------------------------ */
int64_t mvsd_v2_workspace_bytes(int64_t num_logits, int64_t num_reqs, int64_t vocab_size);

int mvsd_v2_rejection_sample(
    int64_t* sampled, int64_t sampled_stride, int32_t* num_sampled, const void* target_logits,
    int target_dtype, int64_t target_stride, int64_t num_logits, const void* draft_logits,
    int draft_dtype, int64_t draft_stride0, int64_t draft_stride1, const int32_t* draft_sampled,
    const int32_t* cu_num_logits, const int64_t* pos, const int32_t* idx_mapping,
    const int32_t* expanded_idx_mapping, const int32_t* expanded_local_pos,
    const float* temperature, const int64_t* seed, int64_t num_req_states, int64_t num_reqs,
    int64_t vocab_size, int32_t num_speculative_steps, const float* synthetic_conditional_rates,
    int use_fp64, int use_block_verification, void* workspace, int64_t workspace_bytes,
    mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* v2_flatten_sampled — the V2 sampled tokens, one per logits row.                         */
/* Replaces: flatten_sampled / _flatten_sampled_kernel (minivllm/worker/gpu/spec_decode/   */
/*           rejection_sampler.py:73-108).  Row cu_num_logits[r] + j of flat_sampled       */
/* [num_logits] int64 gets sampled[r * sampled_stride + j] for j < num_sampled[r]; every  */
/* other row (the rest of each request's rows, rows no request covers) gets 0, as after   */
/* the reference's zero fill.                                                              */
/* ------------------------------------------------------------------------------------ */
int mvsd_v2_flatten_sampled(int64_t* flat_sampled, const int64_t* sampled, int64_t sampled_stride,
                            const int32_t* num_sampled, const int32_t* cu_num_logits,
                            int64_t num_reqs, int64_t num_logits, mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* v2_num_sampled_and_rejected — per-request counts after a V2 verification.              */
/* Replaces: get_num_sampled_and_rejected (minivllm/worker/gpu/input_batch.py:507-553).   */
/* In place on num_sampled [num_reqs] int32; writes num_rejected [num_reqs] int32 =       */
/* (cu_num_logits[r+1] - cu_num_logits[r]) - num_sampled[r]; both 0 for a request still   */
/* prefilling (seq_lens[r] < prefill_len[idx_mapping[r]]).  seq_lens, cu_num_logits,       */
/* idx_mapping and prefill_len [num_req_states] are int32.                                 */
/* ------------------------------------------------------------------------------------ */
int mvsd_v2_num_sampled_and_rejected(int32_t* num_sampled, int32_t* num_rejected,
                                     const int32_t* seq_lens, const int32_t* cu_num_logits,
                                     const int32_t* idx_mapping, const int32_t* prefill_len,
                                     int64_t num_reqs, int64_t num_req_states,
                                     mvsd_stream_t stream);

/* ------------------------------------------------------------------------------------ */
/* topk_scores — logprobs of the V2 sampled tokens and of each row's top k.               */
/* Replaces: compute_topk_scores (minivllm/worker/gpu/sample/logprob.py:140-216), the      */
/* path without per-request logprob token ids, with _topk_log_softmax_kernel (:44-83) and  */
/* _ranks_kernel (:86-104).  Row n of logits [num_rows, V] fp32 (stride logits_stride),     */
/* token t = token_ids[n] (-1 read as 0):                                                  */
/*   ids[n, 0] = t; ids[n, 1 .. k] = the k largest raw logits by (value desc, index asc);  */
/*   scores[n, c] = the fp32 log-softmax (x - max) - log(sum exp(x - max)) at ids[n, c], or */
/*   the logit itself when logits_mode != 0;                                                */
/*   ranks[n] = #{i : x_i >= x_t} over the raw logits.                                      */
/* ids / scores are [num_rows, k + 1]; 0 <= k <= V.                                        */
/* ------------------------------------------------------------------------------------ */
int mvsd_topk_scores(int32_t* ids, float* scores, int32_t* ranks, const float* logits,
                     int64_t logits_stride, const int32_t* token_ids, int64_t num_rows,
                     int64_t vocab_size, int64_t k, int logits_mode, mvsd_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MVSD_H_ */
