// Speculative decoding bookkeeping on the device: prompt-lookup drafts and the
// acceptance of a verify step (no host synchronisation, graph-capturable).
//
// Restates engine/engine.py:955-977 (_spec_draft) and :979-1003 (_spec_step's
// acceptance, history scatter and position update). Like decode_finish
// (step.hip) the acceptance also embeds the next input row, so a plain step can
// follow a verify step directly.
#include "common.h"

namespace {

constexpr int SPEC_THREADS = 256;
constexpr int SPEC_MAX_T = 16;   // verify width T = k + 1 (the attention kernels take T <= 16)
constexpr int SPEC_MAX_N = 8;    // n-gram length

// One workgroup per sequence. L = pos[b] + 1 tokens of hist[b] are valid. The
// suffix hist[L-n .. L-1] (indices clamped at 0) is looked up in the history:
// the latest start i with i < L - n and hist[i .. i+n-1] == suffix wins (i = -1
// if none); the draft is hist[i+n .. i+n+k-1], indices clamped to [0, L-1].
// tok[b] = [hist[L-1], draft...] (T = k + 1 ids).
__global__ void __launch_bounds__(SPEC_THREADS) spec_draft_kernel(const int64_t* __restrict__ hist,
                                                                  const int32_t* __restrict__ pos, int cap, int k,
                                                                  int n, int64_t* __restrict__ tok) {
  const int b = blockIdx.x;
  const int64_t* h = hist + (long long)b * cap;
  const long long L = min((long long)cap, max(1ll, (long long)pos[b] + 1));
  int64_t suf[SPEC_MAX_N];
#pragma unroll
  for (int j = 0; j < SPEC_MAX_N; ++j) suf[j] = j < n ? h[max(0ll, L - n + j)] : 0;
  // Candidates i in [0, min(L - n, cap - n + 1)); each thread keeps its latest match.
  const long long iend = min(L - n, (long long)cap - n + 1);
  long long best = -1;
  for (long long i = threadIdx.x; i < iend; i += SPEC_THREADS) {
    bool match = true;
    for (int j = 0; j < n; ++j) match = match && (h[i + j] == suf[j]);
    if (match) best = i;
  }
  __shared__ long long s_best[SPEC_THREADS / 64];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) best = max(best, (long long)__shfl_xor(best, o, 64));
  if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    long long istar = -1;
    for (int w = 0; w < SPEC_THREADS / 64; ++w) istar = max(istar, s_best[w]);
    int64_t* out = tok + (long long)b * (k + 1);
    out[0] = h[L - 1];
    for (int j = 0; j < k; ++j) {
      long long src = istar + n + j;
      src = src < 0 ? 0 : (src > L - 1 ? L - 1 : src);
      out[1 + j] = h[src];
    }
  }
}

// One workgroup per sequence, after the verify step produced nxt[b*T + j] (the
// greedy token after tok[b, :j+1]). acc = leading j < k with nxt[b, j] ==
// tok[b, j+1]; adv = acc + 1, or 0 for a sequence that already produced its
// max_new_tokens ((L - s) >= ntarget: its state stays frozen). hist[b, L + j] =
// nxt[b, j] for j < adv (the other positions go to the dump slot cap - 1),
// pos[b] += adv; out_t[j, b] = nxt[b, j] and adv_out[b] = adv for the host; then
// h[b] = W[hist[b, pos[b]]] and psq[b] its per-16-column sums of squares (the
// input of a following plain step).
__global__ void __launch_bounds__(SPEC_THREADS) spec_accept_kernel(
    const int64_t* __restrict__ nxt, const int64_t* __restrict__ tok, int64_t* __restrict__ hist,
    int32_t* __restrict__ pos, const int64_t* __restrict__ s_buf, const int64_t* __restrict__ ntarget, int cap, int B,
    int T, int64_t* __restrict__ out_t, int64_t* __restrict__ adv_out, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ hrow, float* __restrict__ psq, long long V, int K) {
  const int b = blockIdx.x;
  __shared__ long long s_id;
  if (threadIdx.x == 0) {
    const int k = T - 1;
    const int64_t* nb = nxt + (long long)b * T;
    const int64_t* tb = tok + (long long)b * T;
    int acc = 0;
    while (acc < k && nb[acc] == tb[acc + 1]) ++acc;
    const long long L = (long long)pos[b] + 1;
    const bool done = (L - s_buf[0]) >= ntarget[0];
    const int adv = done ? 0 : acc + 1;
    int64_t* hb = hist + (long long)b * cap;
    for (int j = 0; j < T; ++j) {
      long long idx = j < adv ? L + j : (long long)cap - 1;
      idx = idx < 0 ? 0 : (idx >= cap ? cap - 1 : idx);
      hb[idx] = nb[j];
      out_t[(long long)j * B + b] = nb[j];
    }
    const long long p1 = (long long)pos[b] + adv;
    pos[b] = (int32_t)p1;
    adv_out[b] = adv;
    const long long pc = p1 < 0 ? 0 : (p1 >= cap ? cap - 1 : p1);
    s_id = hb[pc];
  }
  __syncthreads();
  embed_row_tiled(w, s_id, V, K, hrow + (long long)b * K, psq + (long long)b * (K / 16), threadIdx.x, SPEC_THREADS);
}

}  // namespace

extern "C" {

int qwen_spec_draft(const int64_t* hist, const int32_t* pos, int B, int cap, int k, int n, int64_t* tok_out,
                    hipStream_t stream) {
  if (!hist || !pos || !tok_out) return QWEN_ENULL;
  if (B < 0 || cap <= 0 || k < 1 || k + 1 > SPEC_MAX_T || n < 1 || n > SPEC_MAX_N || n > cap) return QWEN_EARG;
  if (B == 0) return QWEN_OK;
  spec_draft_kernel<<<B, SPEC_THREADS, 0, stream>>>(hist, pos, cap, k, n, tok_out);
  QWEN_RETURN_LAUNCH();
}

int qwen_spec_accept(const int64_t* nxt, const int64_t* tok, int64_t* hist, int32_t* pos, const int64_t* s_buf,
                     const int64_t* ntarget, int B, int cap, int T, int64_t* out_t, int64_t* adv_out,
                     const void* w_tiled, void* h, float* psq, long long V, int K, hipStream_t stream) {
  if (!nxt || !tok || !hist || !pos || !s_buf || !ntarget || !out_t || !adv_out || !w_tiled || !h || !psq)
    return QWEN_ENULL;
  if (B < 0 || cap <= 0 || T < 1 || T > SPEC_MAX_T || V <= 0 || V % 16 != 0 || K <= 0 || K % 32 != 0)
    return QWEN_EARG;
  if (B == 0) return QWEN_OK;
  spec_accept_kernel<<<B, SPEC_THREADS, 0, stream>>>(nxt, tok, hist, pos, s_buf, ntarget, cap, B, T, out_t, adv_out,
                                                     (const bf16_t*)w_tiled, (bf16_t*)h, psq, V, K);
  QWEN_RETURN_LAUNCH();
}

}  // extern "C"
