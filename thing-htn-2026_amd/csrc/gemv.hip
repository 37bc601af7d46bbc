// Balanced weight-streaming GEMV for the decode projections at M <= 2 rows (the kernel body
// and its design notes are in gemv_impl.h).
#include "gemv_impl.h"

namespace {

template <int M, int WAVES, bool NORM, int EPI>
__global__ void __launch_bounds__(64 * WAVES) gemv_kernel(GemvParams p) {
  extern __shared__ __align__(16) unsigned char gv_smem[];
  gemv_body<M, WAVES, NORM, EPI, false>(p, gv_smem, blockIdx.x, gridDim.x, nullptr);
}

template <int M, int WAVES, bool NORM, int EPI>
int launch_gemv(const GemvParams& p, int G, size_t lds, hipStream_t stream) {
  auto kern = gemv_kernel<M, WAVES, NORM, EPI>;
  static bool attr = false;  // one-time opt-in to more than 64 KB of dynamic LDS
  if (!attr) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
      return QWEN_EARG;
    attr = true;
  }
  kern<<<G, 64 * WAVES, lds, stream>>>(p);
  QWEN_RETURN_LAUNCH();
}

template <int M, int WAVES>
int dispatch_gemv(const GemvParams& p, bool norm, int epi, int G, size_t lds, hipStream_t stream) {
  if (norm) {
    if (epi == GEPI_STORE) return launch_gemv<M, WAVES, true, GEPI_STORE>(p, G, lds, stream);
    if (epi == GEPI_SWIGLU) return launch_gemv<M, WAVES, true, GEPI_SWIGLU>(p, G, lds, stream);
    if (epi == GEPI_ARGMAX) return launch_gemv<M, WAVES, true, GEPI_ARGMAX>(p, G, lds, stream);
    return QWEN_EARG;
  }
  if (epi == GEPI_STORE) return launch_gemv<M, WAVES, false, GEPI_STORE>(p, G, lds, stream);
  if (epi == GEPI_RES) return launch_gemv<M, WAVES, false, GEPI_RES>(p, G, lds, stream);
  return QWEN_EARG;
}

}  // namespace

extern "C" {

// Dynamic LDS bytes qwen_gemv needs for a launch shape (0 if the shape is unsupported).
long long qwen_gemv_lds_bytes(int M, int N, int K, int grid, int waves, int epi) {
  if (M < 1 || M > 2 || N <= 0 || K <= 0 || grid <= 0 || (waves != 8 && waves != 16)) return 0;
  if (epi < GEPI_STORE || epi > GEPI_ARGMAX) return 0;
  return (long long)gemv_lds_bytes(M, N, K, grid, waves, epi);
}

// epi: 0 store, 1 residual add (residual may alias out), 2 SwiGLU (w holds 2N rows: gate then
// up; out has N columns), 3 argmax into amax (out unused). norm_w == nullptr: no RMSNorm prologue.
int qwen_gemv_rowmap(const void* x, const void* w, void* out, int M, int N, int K, int ld_out, const void* norm_w,
                     float eps, const void* residual, int epi, unsigned long long* amax, const int32_t* row_map,
                     int groups, int grid, int waves, hipStream_t stream) {
  if (!x || !w) return QWEN_ENULL;
  if (row_map && epi != GEPI_STORE) return QWEN_EARG;
  if (groups < 1 || N % groups || grid % groups) return QWEN_EARG;
  if (M < 1 || M > 2 || N <= 0 || K <= 0 || K % GV_CHUNK != 0 || grid <= 0 || grid > 65536) return QWEN_EARG;
  if (waves != 8 && waves != 16) return QWEN_EARG;
  if (epi < GEPI_STORE || epi > GEPI_ARGMAX) return QWEN_EARG;
  if (epi == GEPI_ARGMAX ? !amax : !out) return QWEN_ENULL;
  if (epi == GEPI_RES && !residual) return QWEN_ENULL;
  if (epi != GEPI_ARGMAX && ld_out < N) return QWEN_EARG;
  const long long staged = (long long)M * (K / 8);   // 16-byte activation chunks staged per workgroup
  if (staged > (long long)(norm_w ? GV_XC_NORM : GV_XC_PLAIN) * 64 * waves) return QWEN_EARG;
  if ((epi == GEPI_SWIGLU || epi == GEPI_ARGMAX) && !norm_w) return QWEN_EARG;  // instantiated variants
  if (epi == GEPI_RES && norm_w) return QWEN_EARG;
  const size_t lds = gemv_lds_bytes(M, N, K, grid, waves, epi);
  if (lds > 160 * 1024) return QWEN_EARG;
  GemvParams p{(const bf16_t*)x, (const bf16_t*)w, (const bf16_t*)norm_w, (const bf16_t*)residual, (bf16_t*)out,
               amax, row_map, N, K, ld_out, eps, groups};
  if (M == 1) return waves == 16 ? dispatch_gemv<1, 16>(p, norm_w != nullptr, epi, grid, lds, stream)
                                 : dispatch_gemv<1, 8>(p, norm_w != nullptr, epi, grid, lds, stream);
  return waves == 16 ? dispatch_gemv<2, 16>(p, norm_w != nullptr, epi, grid, lds, stream)
                     : dispatch_gemv<2, 8>(p, norm_w != nullptr, epi, grid, lds, stream);
}

int qwen_gemv(const void* x, const void* w, void* out, int M, int N, int K, int ld_out, const void* norm_w, float eps,
              const void* residual, int epi, unsigned long long* amax, int grid, int waves, hipStream_t stream) {
  return qwen_gemv_rowmap(x, w, out, M, N, K, ld_out, norm_w, eps, residual, epi, amax, nullptr, 1, grid, waves,
                          stream);
}

}  // extern "C"
