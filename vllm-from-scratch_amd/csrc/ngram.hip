// Prompt-lookup (ngram) drafting, one workgroup per request.
//
// Semantics (both reference matchers agree on the match; see
// minivllm/spec_decode/ngram_proposer.py:41-99 and ngram_proposer_gpu.py:56-148):
//   For n in [min_n, max_n] find the earliest window tokens[s, s+n) equal to the last n
//   tokens with s + n <= L - 1 (at least one token follows the window); take the largest
//   n that has a match and propose tokens[s + n, s + n + k).
//
// Reformulated by window END e = s + n - 1 (0 <= e <= L - 2): let l(e) be the length of the
// common suffix of tokens[0..e] and tokens[0..L-1], capped at max_n.  A length-n window
// ending at e matches iff l(e) >= n, and for a fixed n the earliest start is the earliest
// end.  So one sweep over e computes l(e) from an LDS tile and keeps first_e[n] with an LDS
// atomicMin; the draft starts at first_e[best n] + 1.  Tiles are visited in order, and the
// sweep stops as soon as a max_n match is known (no later tile can give an earlier end).
#include "mvsd_device.h"
#include "rows.h"

namespace mvsd {

constexpr int kTile = 4096;
constexpr int kMaxDraft = 256;

__global__ __launch_bounds__(kThreads) void ngram_kernel(NgramParams p) {
  __shared__ int32_t s_tok[kTile + kNgramMaxN];
  __shared__ int32_t s_suf[kNgramMaxN];
  __shared__ int s_first[kNgramMaxN + 1];
  __shared__ int32_t s_draft[kMaxDraft];

  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  int32_t* row = p.tokens + (int64_t)r * p.row_stride;
  const int64_t base_len = p.num_tokens[r];
  const int cnt = p.new_counts ? p.new_counts[r] : 0;

  // 1) append this step's sampled tokens after the current length, in place
  //    (ngram_proposer_gpu.py:222-234): only the first `cnt` entries that are not -1 and
  //    fall inside the buffer are written.
  if (p.new_tokens) {
    for (int64_t j = tid; j < p.max_new; j += kThreads) {
      const int64_t pos = base_len + j;
      const int32_t tok = p.new_tokens[(int64_t)r * p.new_stride + j];
      if (j < cnt && tok != -1 && pos >= 0 && pos < p.max_seq_len) row[pos] = tok;
    }
  }
  __syncthreads();

  int64_t L = base_len + cnt;
  if (L < 0) L = 0;
  if (L > p.max_seq_len) L = p.max_seq_len;
  bool act = p.active ? p.active[r] != 0 : true;
  if (p.gate_on_new_counts) act = act && cnt > 0 && L >= p.min_n;
  int kk = p.k;
  if (p.cap_by_model_len) {
    // ngram_proposer.py:55-61
    const int64_t room = p.max_model_len - L;
    if (room < kk) kk = (int)(room < 0 ? 0 : room);
    if (L < p.min_n || kk <= 0) act = false;
  }

  const int max_n = p.max_n;
  const int min_n = p.min_n;
  if (tid <= max_n) s_first[tid] = INT_MAX;
  // the suffix is loaded with the first tile and stored after that tile's loads are issued,
  // so both take one memory round trip
  const bool has_suf = act && tid < max_n && tid < L;
  const int32_t suf = has_suf ? row[L - 1 - tid] : 0;
  if (!(act && L >= 2)) {
    if (has_suf) s_suf[tid] = suf;
    __syncthreads();
  }

  // the tile last loaded: tokens [tile_lo, tile_hi) at s_tok[tok - tile_lo]
  int64_t tile_lo = 0, tile_hi = 0;
  if (act && L >= 2) {
    const int halo = max_n - 1;
    for (int64_t t0 = 0; t0 <= L - 2; t0 += kTile) {
      const int64_t t1 = (t0 + kTile < L - 1) ? t0 + kTile : L - 1;  // ends e in [t0, t1)
      // tokens [t0 - halo, t1], the one after the last window too (a draft may start there)
      const int64_t span = t1 + 1 - t0 + halo;
      // every load of the tile is issued before any is stored, so the tile costs one memory
      // round trip instead of one per loop step
      constexpr int kPer = (kTile + kNgramMaxN + kThreads - 1) / kThreads;
      int32_t v[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int64_t i = tid + (int64_t)u * kThreads;
        const int64_t src = t0 - halo + i;
        v[u] = (i < span && src >= 0) ? row[src] : 0;
      }
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int64_t i = tid + (int64_t)u * kThreads;
        if (i < span) s_tok[i] = v[u];
      }
      if (t0 == 0 && has_suf) s_suf[tid] = suf;
      tile_lo = t0 - halo;
      tile_hi = t1 + 1;
      __syncthreads();
      for (int64_t e = t0 + tid; e < t1; e += kThreads) {
        int l = 0;
        while (l < max_n && e - l >= 0 && s_tok[e - l - t0 + halo] == s_suf[l]) ++l;
        for (int n = min_n; n <= l; ++n) atomicMin(&s_first[n], (int)e);
      }
      __syncthreads();
      const bool done = s_first[max_n] != INT_MAX;
      __syncthreads();
      if (done) break;
    }
  }

  // 2) pick the largest matching n and copy the draft
  if (tid == 0) {
    int start = -1;
    if (act) {
      for (int n = max_n; n >= min_n; --n) {
        if (s_first[n] != INT_MAX) {
          start = s_first[n] + 1;
          break;
        }
      }
    }
    s_first[0] = start;
  }
  __syncthreads();
  const int start = s_first[0];
  const int64_t avail = start >= 0 ? L - start : 0;
  const int64_t count = p.cap_by_model_len ? (avail < kk ? avail : kk) : avail;
  for (int j = tid; j < p.k; j += kThreads) {
    const int64_t pos = (int64_t)start + j;
    // from the last tile when it holds the token (every thread saw the same tile bounds)
    s_draft[j] = (start >= 0 && j < count)
                     ? (pos >= tile_lo && pos < tile_hi && pos >= 0 ? s_tok[pos - tile_lo] : row[pos])
                     : -1;
  }
  __syncthreads();
  if (tid == 0) {
    int nv = 0;
    if (p.cap_by_model_len) {
      nv = (int)(start >= 0 ? count : 0);
    } else {
      while (nv < p.k && s_draft[nv] != -1) ++nv;  // ngram_proposer_gpu.py:143-147
    }
    p.num_valid[r] = nv;
  }
  for (int j = tid; j < p.k; j += kThreads) p.drafts[(int64_t)r * p.k + j] = s_draft[j];
}

hipError_t launch_ngram(const NgramParams& p, int64_t num_reqs, hipStream_t stream) {
  if (num_reqs == 0) return hipSuccess;
  if (p.max_n > kNgramMaxN || p.k > kMaxDraft) return hipErrorInvalidValue;
  hipLaunchKernelGGL(ngram_kernel, dim3((unsigned)num_reqs), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

// Valid sampled tokens of one step, one thread per request
// (minivllm/spec_decode/ngram_proposer_gpu.py:247-290): a discarded request's row becomes -1;
// the count is the number of entries that are not -1 and below the vocabulary size; the next
// token is entry count - 1 of the row when the count is positive, else the history's token at
// max(num_tokens - 1, 0).
__global__ __launch_bounds__(256) void ngram_valid_sampled_kernel(
    int32_t* next_token_ids, int32_t* counts, int32_t* valid_ids, int64_t valid_stride,
    const int32_t* sampled, int64_t sampled_stride, int64_t width, const uint8_t* discard,
    const int32_t* token_ids, int64_t row_stride, const int32_t* num_tokens, int32_t vocab_size,
    int64_t num_reqs) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= num_reqs) return;
  const bool drop = discard && discard[r];
  const int32_t* src = sampled + r * sampled_stride;
  int32_t* dst = valid_ids + r * valid_stride;
  int count = 0;
  for (int64_t j = 0; j < width; ++j) {
    const int32_t v = drop ? -1 : src[j];
    dst[j] = v;
    count += (v != -1 && v < vocab_size) ? 1 : 0;
  }
  int32_t next;
  if (count > 0) {
    next = src[count - 1];  // count > 0 means the row was kept
  } else {
    // lengths beyond the row are clamped to its last column (the reference would raise)
    const int64_t n = num_tokens[r];
    next = token_ids[r * row_stride + (n > 1 ? (n - 1 < row_stride ? n - 1 : row_stride - 1) : 0)];
  }
  counts[r] = count;
  next_token_ids[r] = next;
}

hipError_t launch_ngram_valid_sampled(int32_t* next_token_ids, int32_t* counts,
                                      int32_t* valid_ids, int64_t valid_stride,
                                      const int32_t* sampled, int64_t sampled_stride,
                                      int64_t width, const uint8_t* discard,
                                      const int32_t* token_ids, int64_t row_stride,
                                      const int32_t* num_tokens, int32_t vocab_size,
                                      int64_t num_reqs, hipStream_t stream) {
  if (num_reqs == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((num_reqs + 255) / 256);
  hipLaunchKernelGGL(ngram_valid_sampled_kernel, dim3(blocks), dim3(256), 0, stream,
                     next_token_ids, counts, valid_ids, valid_stride, sampled, sampled_stride,
                     width, discard, token_ids, row_stride, num_tokens, vocab_size, num_reqs);
  return hipGetLastError();
}

}  // namespace mvsd
