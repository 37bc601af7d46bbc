// Per-head QK RMSNorm + RoPE + KV-cache write.
//
// Operator semantics: engine/kernels/rope.py:169-226 and the rounding points of
// engine/kernels/torch_ref.py:94-162 (RMSNorm with the cast before the gain,
// then RoPE with three bf16 roundings: bf16(bf16(y*cos) + bf16(rot(y)*sin)),
// rot(y) = cat(-y[64:], y[:64])).
//
// One wavefront per (token, head). Lane l owns dims l and l + 64, which are
// exactly the two elements rotate_half pairs, so the rotation needs no lane
// exchange; the only cross-lane step is the 128-wide sum of squares.
#include "common.h"

namespace {

constexpr int HEADS_PER_BLOCK = 4;

__global__ void __launch_bounds__(64 * HEADS_PER_BLOCK) qk_norm_rope_cache_kernel(
    const bf16_t* __restrict__ qkv, const bf16_t* __restrict__ qw, const bf16_t* __restrict__ kw,
    const bf16_t* __restrict__ cos_tab, const bf16_t* __restrict__ sin_tab, const int32_t* __restrict__ positions,
    bf16_t* __restrict__ q_out, bf16_t* __restrict__ k_cache, bf16_t* __restrict__ v_cache,
    int T, int Nq, int Nkv, int CAP, int P, float eps) {
  constexpr int D = 128;
  const int lane = threadIdx.x & 63;
  const int head = blockIdx.y * HEADS_PER_BLOCK + (threadIdx.x >> 6);
  const int nheads = Nq + 2 * Nkv;
  if (head >= nheads) return;
  const long long m = blockIdx.x;
  const long long b = m / T;
  const long long t = m - b * T;
  const long long pos = (long long)positions[b] + t;
  if (pos < 0 || pos >= CAP || pos >= P) return;  // out-of-range slot: write nothing
  const bf16_t* src = qkv + m * (long long)nheads * D + (long long)head * D;
  const float x0 = bf2f(src[lane]);
  const float x1 = bf2f(src[lane + 64]);

  if (head >= Nq + Nkv) {  // V head: raw copy into the cache
    const long long kvh = head - Nq - Nkv;
    bf16_t* dst = v_cache + ((b * Nkv + kvh) * (long long)CAP + pos) * D;
    dst[lane] = src[lane];
    dst[lane + 64] = src[lane + 64];
    return;
  }
  const bf16_t* gain = head < Nq ? qw : kw;
  const float ss = wave_sum(add_rn(mul_rn(x0, x0), mul_rn(x1, x1)));
  const float rinv = 1.0f / sqrtf(ss / (float)D + eps);
  const float y0 = rbf(mul_rn(bf2f(gain[lane]), rbf(mul_rn(x0, rinv))));
  const float y1 = rbf(mul_rn(bf2f(gain[lane + 64]), rbf(mul_rn(x1, rinv))));
  const bf16_t* cr = cos_tab + pos * D;
  const bf16_t* sr = sin_tab + pos * D;
  const float c0 = bf2f(cr[lane]), c1 = bf2f(cr[lane + 64]);
  const float s0 = bf2f(sr[lane]), s1 = bf2f(sr[lane + 64]);
  const bf16_t o0 = f2bf(add_rn(rbf(mul_rn(y0, c0)), rbf(mul_rn(-y1, s0))));
  const bf16_t o1 = f2bf(add_rn(rbf(mul_rn(y1, c1)), rbf(mul_rn(y0, s1))));
  bf16_t* dst;
  if (head < Nq) {
    dst = q_out + (m * Nq + head) * (long long)D;
  } else {
    const long long kvh = head - Nq;
    dst = k_cache + ((b * Nkv + kvh) * (long long)CAP + pos) * D;
  }
  dst[lane] = o0;
  dst[lane + 64] = o1;
}

}  // namespace

extern "C" int qwen_qk_norm_rope_cache(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                       const void* cos_tab, const void* sin_tab, const int32_t* positions,
                                       void* q_out, void* k_cache, void* v_cache, int B, int T, int Nq, int Nkv,
                                       int D, int CAP, int P, float eps, hipStream_t stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !positions || !q_out || !k_cache || !v_cache)
    return QWEN_ENULL;
  if (D != 128 || B < 0 || T <= 0 || Nq <= 0 || Nkv <= 0 || CAP <= 0 || P <= 0) return QWEN_EARG;
  if ((long long)B * T == 0) return QWEN_OK;
  if ((long long)B * T > 0x7fffffffLL) return QWEN_EARG;
  const int nheads = Nq + 2 * Nkv;
  dim3 grid((unsigned)(B * T), (nheads + HEADS_PER_BLOCK - 1) / HEADS_PER_BLOCK);
  qk_norm_rope_cache_kernel<<<grid, 64 * HEADS_PER_BLOCK, 0, stream>>>(
      (const bf16_t*)qkv, (const bf16_t*)q_norm_w, (const bf16_t*)k_norm_w, (const bf16_t*)cos_tab,
      (const bf16_t*)sin_tab, positions, (bf16_t*)q_out, (bf16_t*)k_cache, (bf16_t*)v_cache, T, Nq, Nkv, CAP, P, eps);
  QWEN_RETURN_LAUNCH();
}
