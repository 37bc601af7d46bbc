// Per-step token bookkeeping on the device (no host synchronisation).
//
// Restates the tail of engine/engine.py:941-953 (_plain_step after the model
// step) and the head of the next step (engine/engine.py:1101, the embedding of
// hist[pos]), fused into one launch that follows the LM head:
//   token[b]   = index held in row b's packed argmax key (its slots re-armed to zero)
//   hist[b, pos[b] + 1] = token[b] and pos[b] += 1, unless the sequence already
//   produced its max_new_tokens (frozen rows write to the dump slot cap-1 and
//   keep their position)
//   h[b, :]    = embedding row of hist[b, pos[b]] (the next step's input) and
//   psq[b, :]  = its per-16-column sums of squares (the next RMSNorm's statistics).
#include "common.h"

namespace {

constexpr int FIN_THREADS = 256;

__global__ void __launch_bounds__(FIN_THREADS) decode_finish_kernel(
    unsigned long long* __restrict__ amax, int64_t* __restrict__ next, int64_t* __restrict__ hist,
    int32_t* __restrict__ pos, const int64_t* __restrict__ s_buf, const int64_t* __restrict__ ntarget,
    const bf16_t* __restrict__ w, bf16_t* __restrict__ h, float* __restrict__ psq, int cap, long long V, int K) {
  const int b = blockIdx.x;
  // Every thread reads the state before thread 0 updates it.
  const unsigned long long key = argmax_key(amax, gridDim.x, b);
  const int64_t tok = (int64_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
  const long long p0 = pos[b];
  const long long L = p0 + 1;
  const bool done = (L - s_buf[0]) >= ntarget[0];
  const long long pc = p0 < 0 ? 0 : (p0 >= cap ? cap - 1 : p0);
  long long id = done ? hist[(long long)b * cap + pc] : tok;
  __syncthreads();
  if (threadIdx.x == 0) {
    long long idx = done ? (long long)(cap - 1) : L;
    idx = idx < 0 ? 0 : (idx >= cap ? cap - 1 : idx);
    hist[(long long)b * cap + idx] = tok;
    if (!done) pos[b] = (int32_t)L;
    next[b] = tok;
    argmax_rearm(amax, gridDim.x, b);
  }
  // Embedding gather from the tiled table (ids clamped into [0, V)).
  embed_row_tiled(w, id, V, K, h + (long long)b * K, psq + (long long)b * (K / 16), threadIdx.x, FIN_THREADS);
}

}  // namespace

extern "C" int qwen_decode_finish(unsigned long long* amax, int64_t* next, int64_t* hist, int32_t* pos,
                                  const int64_t* s_buf, const int64_t* ntarget, const void* w_tiled, void* h,
                                  float* psq, int B, int cap, long long V, int K, hipStream_t stream) {
  if (!amax || !next || !hist || !pos || !s_buf || !ntarget || !w_tiled || !h || !psq) return QWEN_ENULL;
  if (B < 0 || cap <= 0 || V <= 0 || V % 16 != 0 || K <= 0 || K % 32 != 0) return QWEN_EARG;
  if (B == 0) return QWEN_OK;
  decode_finish_kernel<<<B, FIN_THREADS, 0, stream>>>(amax, next, hist, pos, s_buf, ntarget, (const bf16_t*)w_tiled,
                                                      (bf16_t*)h, psq, cap, V, K);
  QWEN_RETURN_LAUNCH();
}
