// The decode step's QK-norm + RoPE + KV write + GQA attention on the matrix cores: kernel
// wrappers, launchers and entry points (the kernel body and its design notes are in
// attention_mfma_impl.h).
#include "attention_mfma_impl.h"

#include <mutex>

namespace {

template <int MT, int WPG, bool KVC>
__global__ void __launch_bounds__(64 * WPG) __attribute__((amdgpu_waves_per_eu(1, 2)))
attn_mfma_kernel(MfmaAttnParams p) {  // LDS holds one workgroup per CU: at most two wavefronts per SIMD
  attn_mfma_body<MT, WPG, KVC, false>(p, blockIdx.x, blockIdx.y, QkvSync{});
}

template <int MT>
int launch_mfma(const MfmaAttnParams& p, int B, int waves, hipStream_t stream) {
  dim3 grid((unsigned)((long long)B * p.Nkv), p.S);
  if (waves == 4) {
    if (p.kv_cached) attn_mfma_kernel<MT, 4, true><<<grid, 256, 0, stream>>>(p);
    else attn_mfma_kernel<MT, 4, false><<<grid, 256, 0, stream>>>(p);
  } else if (waves == 8) {
    if (p.kv_cached) attn_mfma_kernel<MT, 8, true><<<grid, 512, 0, stream>>>(p);
    else attn_mfma_kernel<MT, 8, false><<<grid, 512, 0, stream>>>(p);
  } else {
    return QWEN_EARG;
  }
  QWEN_RETURN_LAUNCH();
}

// ---- the allocation-free variant's scratch: one array per GPU, for the split partials and
// arrival counters that qwen_attn_decode_mfma keeps in its caller's workspace. Host code never
// passes `scratch` itself to a kernel (in host code it names a host-side stand-in); it looks up
// each device's address once with hipGetSymbolAddress and uses that.
constexpr long long NOALLOC_SCRATCH_BYTES = 8ll << 20;   // QWEN_ATTN_NOALLOC_SCRATCH_BYTES
__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[MAX_DEVICES] = {};

// The current device's address of `scratch` (looked up on its first use there), or null.
void* device_scratch(int* status) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { *status = (int)e; return nullptr; }
  if (dev < 0 || dev >= MAX_DEVICES) { *status = QWEN_EARG; return nullptr; }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) { *status = e != hipSuccess ? (int)e : QWEN_ENULL; return nullptr; }
    g_scratch_ptr[dev] = ptr;
  }
  *status = QWEN_OK;
  return g_scratch_ptr[dev];
}

// Zero `n` 32-bit words (the arrival counters) with a kernel rather than hipMemsetAsync, so a
// caller may record the call into a HIP graph.
__global__ void __launch_bounds__(256) zero_words_kernel(unsigned* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace

extern "C" {

long long qwen_attn_mfma_workspace_bytes(int B, int T, int Nkv, int num_splits) {
  if (B <= 0 || T < 1 || T > 8 || Nkv <= 0 || num_splits < 1 || num_splits > MERGE_MAX) return 0;
  if (num_splits == 1) return 0;
  const long long bh = (long long)B * Nkv;
  return mfma_counter_bytes(bh) + bh * num_splits * mfma_rows(T) * (2 + MD) * (long long)sizeof(float);
}

int qwen_attn_decode_mfma_ex(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                             const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                             void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D,
                             int CAP, int P, float eps, float scale, int num_splits, int waves, int flags,
                             hipStream_t stream) {
  const int st = mfma_args_status(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out, B, T,
                                  Nq, Nkv, D, CAP, P, num_splits, waves, flags);
  if (st != QWEN_OK) return st;
  if (B == 0) return QWEN_OK;
  const long long need = qwen_attn_mfma_workspace_bytes(B, T, Nkv, num_splits);
  if (need > 0 && (!workspace || workspace_bytes < need)) return workspace ? QWEN_EWORKSPACE : QWEN_ENULL;
  MfmaAttnParams p{};
  p.qkv = (const bf16_t*)qkv;
  p.qnw = (const bf16_t*)q_norm_w;
  p.knw = (const bf16_t*)k_norm_w;
  p.cos_tab = (const bf16_t*)cos_tab;
  p.sin_tab = (const bf16_t*)sin_tab;
  p.pos = positions;
  p.kc = (bf16_t*)k_cache;
  p.vc = (bf16_t*)v_cache;
  p.out = (bf16_t*)out;
  const long long bh = (long long)B * Nkv;
  p.cnt = num_splits > 1 ? (unsigned*)workspace : nullptr;
  p.part = num_splits > 1 ? (float*)((char*)workspace + mfma_counter_bytes(bh)) : nullptr;
  p.T = T; p.Nkv = Nkv; p.CAP = CAP; p.P = P; p.S = num_splits;
  p.scale = scale; p.eps = eps;
  p.kv_cached = (flags & QWEN_ATTN_KV_CACHED) ? 1 : 0;
  return T <= 4 ? launch_mfma<1>(p, B, waves, stream) : launch_mfma<2>(p, B, waves, stream);
}

int qwen_attn_decode_mfma_noalloc(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                  const void* cos_tab, const void* sin_tab, const int32_t* positions, void* k_cache,
                                  void* v_cache, void* out, int B, int T, int Nq, int Nkv, int D, int CAP, int P,
                                  float eps, float scale, int num_splits, int waves, int flags, hipStream_t stream) {
  const int st = mfma_args_status(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out, B, T,
                                  Nq, Nkv, D, CAP, P, num_splits, waves, flags);
  if (st != QWEN_OK) return st;
  const long long need = qwen_attn_mfma_workspace_bytes(B, T, Nkv, num_splits);
  if (need > NOALLOC_SCRATCH_BYTES) return QWEN_ESCRATCH;
  if (need == 0 || B == 0)
    return qwen_attn_decode_mfma_ex(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out,
                                    nullptr, 0, B, T, Nq, Nkv, D, CAP, P, eps, scale, num_splits, waves, flags,
                                    stream);
  int status = QWEN_OK;
  void* ptr = device_scratch(&status);
  if (!ptr) return status;
  // the counters must start at zero (every launch re-arms them; cleared here all the same)
  const int words = (int)(mfma_counter_bytes((long long)B * Nkv) / 4);
  zero_words_kernel<<<(words + 255) / 256, 256, 0, stream>>>((unsigned*)ptr, words);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  return qwen_attn_decode_mfma_ex(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out, ptr,
                                  NOALLOC_SCRATCH_BYTES, B, T, Nq, Nkv, D, CAP, P, eps, scale, num_splits, waves,
                                  flags, stream);
}

int qwen_attn_decode_mfma(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                          const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                          void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D, int CAP,
                          int P, float eps, float scale, int num_splits, int waves, hipStream_t stream) {
  return qwen_attn_decode_mfma_ex(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out,
                                  workspace, workspace_bytes, B, T, Nq, Nkv, D, CAP, P, eps, scale, num_splits, waves,
                                  0, stream);
}

}  // extern "C"
