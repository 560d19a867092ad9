/*
 * CPU oracle of the ngram prompt-lookup proposer — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this code, as the
 * checker or as the timed CPU baseline; the product library never links it.
 *
 * ngram_kmp   restates the reference CPU matcher line by line in C:
 *             minivllm/spec_decode/ngram_proposer.py:41-99 (reversed tokens, KMP lps capped at
 *             max_ngram, `>=` keeps the earliest original occurrence, k capped by
 *             max_model_len - total and by the tokens after the match).
 * ngram_brute is an independent definition used to pin it: for n from max_n down to min_n,
 *             scan window starts s = 0 .. len-n-1 and take the first s whose window equals
 *             the last n tokens; it also gives the device proposer's semantics
 *             (minivllm/spec_decode/ngram_proposer_gpu.py:56-128: no max_model_len cap,
 *             drafts -1 padded, valid = leading non -1 count).
 * Batch wrappers loop over rows of a [R, stride] int32 buffer.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Returns the number of drafts written to out (<= k). */
int ngram_kmp(const int32_t* origin, int64_t total, int min_ngram, int max_ngram,
              int64_t max_model_len, int k, int32_t* out) {
  if (total < min_ngram) return 0;
  int64_t kk = k;
  if (max_model_len - total < kk) kk = max_model_len - total;
  if (kk <= 0) return 0;
  /* tokens = origin[::-1] */
  int32_t* lps = (int32_t*)calloc((size_t)max_ngram, sizeof(int32_t));
  if (!lps) return -1;
#define TOK(i) (origin[total - 1 - (i)])
  int64_t longest = 0, position = 0, prev = 0, i = 1;
  while (i < total) {
    if (TOK(prev) == TOK(i)) {
      prev += 1;
      if (prev >= longest) {
        longest = prev;
        position = i;
      }
      if (i < max_ngram) lps[i] = (int32_t)prev;
      if (prev == max_ngram) prev = lps[max_ngram - 1];
      i += 1;
    } else if (prev != 0) {
      prev = lps[prev - 1];
    } else {
      i += 1;
    }
  }
#undef TOK
  free(lps);
  if (longest < min_ngram) return 0;
  int64_t start = total - 1 - position + longest;
  if (total - start < kk) kk = total - start;
  for (int64_t j = 0; j < kk; ++j) out[j] = origin[start + j];
  return (int)kk;
}

/* Earliest start of the longest matching n in [min_n, max_n]; -1 and *n_out = 0 if none. */
static int64_t brute_match(const int32_t* t, int64_t len, int min_n, int max_n, int* n_out) {
  for (int n = max_n; n >= min_n; --n) {
    for (int64_t s = 0; s + n <= len - 1; ++s) {
      int eq = 1;
      for (int j = 0; j < n && eq; ++j) eq = t[s + j] == t[len - n + j];
      if (eq) {
        *n_out = n;
        return s;
      }
    }
  }
  *n_out = 0;
  return -1;
}

/* Device semantics: out[0..k) -1 padded; returns the leading non -1 count. */
int ngram_brute_device(const int32_t* t, int64_t len, int min_n, int max_n, int k, int32_t* out) {
  int n = 0;
  int64_t s = brute_match(t, len, min_n, max_n, &n);
  for (int j = 0; j < k; ++j) out[j] = -1;
  if (s >= 0) {
    int64_t start = s + n;
    for (int j = 0; j < k && start + j < len; ++j) out[j] = t[start + j];
  }
  int valid = 0;
  while (valid < k && out[valid] != -1) ++valid;
  return valid;
}

/* CPU semantics via the brute-force match (for cross-checking ngram_kmp). */
int ngram_brute_cpu(const int32_t* t, int64_t len, int min_n, int max_n, int64_t max_model_len,
                    int k, int32_t* out) {
  if (len < min_n) return 0;
  int64_t kk = k;
  if (max_model_len - len < kk) kk = max_model_len - len;
  if (kk <= 0) return 0;
  int n = 0;
  int64_t s = brute_match(t, len, min_n, max_n, &n);
  if (s < 0) return 0;
  int64_t start = s + n;
  if (len - start < kk) kk = len - start;
  for (int64_t j = 0; j < kk; ++j) out[j] = t[start + j];
  return (int)kk;
}

/* Batch forms over a [R, stride] buffer; drafts [R, k] (-1 padded), counts [R]. */
void ngram_kmp_batch(const int32_t* tokens, int64_t stride, const int32_t* lens, int64_t rows,
                     int min_n, int max_n, int64_t max_model_len, int k, int32_t* drafts,
                     int32_t* counts) {
  for (int64_t r = 0; r < rows; ++r) {
    int32_t* d = drafts + r * k;
    for (int j = 0; j < k; ++j) d[j] = -1;
    counts[r] = ngram_kmp(tokens + r * stride, lens[r], min_n, max_n, max_model_len, k, d);
  }
}

void ngram_brute_device_batch(const int32_t* tokens, int64_t stride, const int32_t* lens,
                              int64_t rows, int min_n, int max_n, int k, int32_t* drafts,
                              int32_t* counts) {
  for (int64_t r = 0; r < rows; ++r)
    counts[r] = ngram_brute_device(tokens + r * stride, lens[r], min_n, max_n, k, drafts + r * k);
}
