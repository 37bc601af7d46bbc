// Per-step token bookkeeping on the device (no host synchronisation).
//
// Restates engine/engine.py:941-953 (_plain_step after the model step): the
// greedy token of sequence b goes to hist[b, pos[b] + 1] and pos[b] advances,
// unless the sequence already produced its max_new_tokens (frozen rows write
// to the dump slot and keep their position).
#include "common.h"

namespace {

__global__ void plain_update_kernel(const int64_t* __restrict__ next, int64_t* __restrict__ hist,
                                    int32_t* __restrict__ pos, const int64_t* __restrict__ s_buf,
                                    const int64_t* __restrict__ ntarget, int B, int cap) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const long long L = (long long)pos[b] + 1;
  const bool done = (L - s_buf[0]) >= ntarget[0];
  long long idx = done ? (long long)(cap - 1) : L;
  idx = idx < 0 ? 0 : (idx >= cap ? cap - 1 : idx);
  hist[(long long)b * cap + idx] = next[b];
  if (!done) pos[b] += 1;
}

}  // namespace

extern "C" int qwen_plain_update(const int64_t* next, int64_t* hist, int32_t* pos, const int64_t* s_buf,
                                 const int64_t* ntarget, int B, int cap, hipStream_t stream) {
  if (!next || !hist || !pos || !s_buf || !ntarget) return QWEN_ENULL;
  if (B < 0 || cap <= 0) return QWEN_EARG;
  if (B == 0) return QWEN_OK;
  plain_update_kernel<<<(B + 63) / 64, 64, 0, stream>>>(next, hist, pos, s_buf, ntarget, B, cap);
  QWEN_RETURN_LAUNCH();
}
