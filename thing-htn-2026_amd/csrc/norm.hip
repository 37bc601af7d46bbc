// Standalone RMSNorm, residual-add + RMSNorm and SwiGLU kernels.
//
// These are the reference's unfused operators (engine/kernels/rmsnorm.py:77-131,
// engine/kernels/silu.py:68-92) with the rounding points of
// engine/kernels/torch_ref.py:47-88. The decode step fuses them into the GEMM
// prologues/epilogues (gemm.hip); these kernels serve the prefill path and the
// operator-level API.
#include "common.h"

namespace {

constexpr int NORM_THREADS = 256;

// Block-wide sum in a fixed order: wave butterflies, then wave 0 sums the
// per-wave results in index order.
__device__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = wave_sum(v);
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  const int nw = blockDim.x >> 6;
  for (int i = 0; i < nw; ++i) t += red[i];
  __syncthreads();
  return t;
}

// y = w * bf16(x * rsqrt(sum(x^2) / N + eps)); one row per block, N % 8 == 0.
// When r != nullptr the input row is h = bf16(x + r), which is stored to h_out.
__global__ void __launch_bounds__(NORM_THREADS) rms_norm_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ r, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ h_out, bf16_t* __restrict__ y, int N, float eps) {
  __shared__ float red[NORM_THREADS / 64];
  const size_t row = blockIdx.x;
  const uint4* xr = reinterpret_cast<const uint4*>(x + row * N);
  const uint4* rr = r ? reinterpret_cast<const uint4*>(r + row * N) : nullptr;
  const uint4* wr = reinterpret_cast<const uint4*>(w);
  uint4* hr = h_out ? reinterpret_cast<uint4*>(h_out + row * N) : nullptr;
  uint4* yr = reinterpret_cast<uint4*>(y + row * N);
  const int nchunk = N / 8;
  // Each thread keeps at most 4 chunks (N <= 8192) in registers between passes.
  // All chunks (and gains) are requested before any is used or any output is stored (the
  // outputs may alias the inputs, so a load after a store would wait for its own round trip);
  // chunks past the row re-read chunk 0 and are dropped.
  float v[4][8];
  uint4 xv[4], rv4[4], gv[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int ci = threadIdx.x + c * NORM_THREADS;
    const int cl = ci < nchunk ? ci : 0;
    xv[c] = xr[cl];
    if (rr) rv4[c] = rr[cl];
    gv[c] = wr[cl];
  }
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int ci = threadIdx.x + c * NORM_THREADS;
    if (ci < nchunk) {
      unpack8(xv[c], v[c]);
      if (rr) {
        float rv[8];
        unpack8(rv4[c], rv);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[c][e] = rbf(add_rn(v[c][e], rv[e]));
        hr[ci] = pack8(v[c]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = add_rn(ss, mul_rn(v[c][e], v[c][e]));
    }
  }
  const float total = block_sum(ss, red);
  const float rinv = rms_rinv(total, N, eps);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int ci = threadIdx.x + c * NORM_THREADS;
    if (ci < nchunk) {
      float g[8], o[8];
      unpack8(gv[c], g);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = mul_rn(g[e], rbf(mul_rn(v[c][e], rinv)));
      yr[ci] = pack8(o);
    }
  }
}

// out[m, i] = bf16(bf16(silu(g)) * u), g = gu[m, i], u = gu[m, I + i].
__global__ void __launch_bounds__(256) silu_mul_kernel(const bf16_t* __restrict__ gu, bf16_t* __restrict__ out,
                                                        int I, long long total) {
  const long long i = blockIdx.x * (long long)blockDim.x + threadIdx.x;
  if (i >= total) return;
  const long long m = i / I, c = i - m * I;
  const float g = bf2f(gu[m * 2 * I + c]);
  const float u = bf2f(gu[m * 2 * I + I + c]);
  const float s = rbf(g / (1.0f + expf(-g)));
  out[i] = f2bf(mul_rn(s, u));
}

// psq[m, u] = sum of squares of x[m, 16u .. 16u+15] (fp32 over the bf16 values):
// the per-16-column partials the normed projections read. One thread per 8
// values; the two threads of a 16-column unit are adjacent lanes.
__global__ void __launch_bounds__(256) sumsq16_kernel(const bf16_t* __restrict__ x, float* __restrict__ psq,
                                                       long long chunks) {
  const long long c = blockIdx.x * 256ll + threadIdx.x;
  float s = 0.f;
  if (c < chunks) {
    float f[8];
    unpack8(reinterpret_cast<const uint4*>(x)[c], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) s = add_rn(s, mul_rn(f[e], f[e]));
  }
  s += __shfl_xor(s, 1, 64);
  if (c < chunks && (c & 1) == 0) psq[c >> 1] = s;
}

}  // namespace

extern "C" {

// Partial sums of squares per 16 columns of a [M, K] bf16 matrix (K % 16 == 0).
int qwen_sumsq16(const void* x, float* psq, int M, int K, hipStream_t stream) {
  if (!x || !psq) return QWEN_ENULL;
  if (M < 0 || K <= 0 || K % 16 != 0) return QWEN_EARG;
  const long long chunks = (long long)M * (K / 8);
  if (chunks == 0) return QWEN_OK;
  const long long blocks = (chunks + 255) / 256;
  if (blocks > 0x7fffffffLL) return QWEN_EARG;
  sumsq16_kernel<<<(unsigned)blocks, 256, 0, stream>>>((const bf16_t*)x, psq, chunks);
  QWEN_RETURN_LAUNCH();
}

int qwen_rms_norm(const void* x, const void* w, void* y, int M, int N, float eps, hipStream_t stream) {
  if (!x || !w || !y) return QWEN_ENULL;
  if (M < 0 || N <= 0 || N % 8 != 0 || N > 8 * 4 * NORM_THREADS) return QWEN_EARG;
  if (M == 0) return QWEN_OK;
  rms_norm_kernel<<<M, NORM_THREADS, 0, stream>>>((const bf16_t*)x, nullptr, (const bf16_t*)w, nullptr,
                                                  (bf16_t*)y, N, eps);
  QWEN_RETURN_LAUNCH();
}

int qwen_add_rms_norm(const void* x, const void* r, const void* w, void* h, void* y, int M, int N, float eps,
                      hipStream_t stream) {
  if (!x || !r || !w || !h || !y) return QWEN_ENULL;
  if (M < 0 || N <= 0 || N % 8 != 0 || N > 8 * 4 * NORM_THREADS) return QWEN_EARG;
  if (M == 0) return QWEN_OK;
  rms_norm_kernel<<<M, NORM_THREADS, 0, stream>>>((const bf16_t*)x, (const bf16_t*)r, (const bf16_t*)w,
                                                  (bf16_t*)h, (bf16_t*)y, N, eps);
  QWEN_RETURN_LAUNCH();
}

int qwen_silu_mul(const void* gu, void* out, int M, int I, hipStream_t stream) {
  if (!gu || !out) return QWEN_ENULL;
  if (M < 0 || I <= 0) return QWEN_EARG;
  const long long total = (long long)M * I;
  if (total == 0) return QWEN_OK;
  const long long blocks = (total + 255) / 256;
  if (blocks > 0x7fffffffLL) return QWEN_EARG;
  silu_mul_kernel<<<(unsigned)blocks, 256, 0, stream>>>((const bf16_t*)gu, (bf16_t*)out, I, total);
  QWEN_RETURN_LAUNCH();
}

}  // extern "C"
