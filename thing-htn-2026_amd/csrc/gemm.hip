// Weight-streaming skinny GEMM on MFMA for the decode projections (M <= 32 rows).
//
// out[M, N] = x[M, K] @ W[N, K]^T with bf16 operands, fp32 accumulation and
// one bf16 rounding (engine/kernels/gemm.py:12-15), plus the fused prologue /
// epilogues whose rounding points are fixed by engine/kernels/gemm_fused.py:5-19
// and :179-193:
//   NORM      : the A operand is RMSNorm(x) computed on the fly,
//               bf16(bf16(x * rsqrt(mean(x^2) + eps)) * gain)   (rmsnorm.py:91-102)
//   EPI_STORE : out = bf16(acc)
//   EPI_RES   : out = bf16(res + bf16(acc))      (residual add, in place allowed)
//   EPI_SWIGLU: out = bf16(bf16(silu(bf16(g))) * bf16(u)) for a gate/up tile pair
//   EPI_ARGMAX: logits = bf16(acc); per-row (max, lowest index) partials per
//               workgroup, reduced by argmax_finalize_kernel (LM head + argmax,
//               engine/engine.py:1119-1121).
//
// Weight layout ("MFMA-B tiles", written by weights.hip): W is cut into tiles
// of 16 rows x 32 k; tile (nt, kt) is 1 KB at offset (nt * K/32 + kt) * 512
// elements and lane l = 16*q + r of a wavefront owns the 16 bytes
// W[16*nt + r][32*kt + 8*q .. +8] at tile offset 8*l. One global_load_dwordx4
// per lane therefore reads a whole tile (1 KB contiguous) straight into the
// B-operand registers of v_mfma_f32_16x16x32_bf16, and the k-reduction
// happens inside the matrix core: no cross-lane shuffles, and the activation
// traffic does not grow with M. M <= 16 rows use one A fragment (rows past M
// are zero lanes), 17..32 rows use two.
//
// Work decomposition: one workgroup per "unit" of NTW adjacent n-tiles;
// its KSPLIT wavefronts split K into contiguous ranges and are reduced through
// LDS in a fixed order (deterministic), then wavefront 0 runs the epilogue.
#include "common.h"

namespace {

enum { EPI_STORE = 0, EPI_RES = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

struct GemmParams {
  const bf16_t* x;    // [M, K] row-major
  const bf16_t* w;    // MFMA-B tiled weight, N x K
  const bf16_t* nw;   // [K] RMSNorm gain (NORM)
  const bf16_t* res;  // [M, ld_out] residual (EPI_RES)
  bf16_t* out;        // [M, ld_out]
  float* pval;        // [units, M] argmax partial values (EPI_ARGMAX)
  int32_t* pidx;      // [units, M] argmax partial indices
  const float* psq_in;  // [M, K/16] partial sums of squares of x per 16 columns (NORM)
  float* psq_out;       // [M, N/16] same for the output rows (EPI_RES, may be null)
  int M, N, K, ld_out;
  float eps;
};

template <int MT, int NTW, int KSPLIT, bool NORM, int EPI>
__global__ void __launch_bounds__(64 * KSPLIT) skinny_gemm_kernel(GemmParams p) {
  constexpr int U = 8;  // k-steps (1 KB tiles per n-tile) loaded ahead per wavefront
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int unit = blockIdx.x;
  const int KT = p.K >> 5;
  const int kpw = (KT + KSPLIT - 1) / KSPLIT;
  const int k0 = min(KT, wave * kpw);
  const int k1 = min(KT, k0 + kpw);

  __shared__ f32x4_t red[KSPLIT > 1 ? KSPLIT * MT * NTW * 64 : 1];

  // Rows of the A operand this lane feeds: m = r + 16*mt. Rows past M read
  // row 0 (always valid) and are zeroed, so the loads need no branch.
  const bf16_t* xrow[MT];
  bool mval[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = r + 16 * mt;
    mval[mt] = m < p.M;
    xrow[mt] = p.x + (size_t)(mval[mt] ? m : 0) * p.K + 8 * q;
  }

  // RMSNorm statistics: the producer of x left one partial sum of squares per
  // 16 columns (rounded bf16 values, squared and summed in fp32). The four
  // lanes of a row each add a quarter of them in a fixed order, so every
  // workgroup derives bit-identical factors.
  float rinv[MT];
  if constexpr (NORM) {
    const int nu = p.K >> 4;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float* ps = p.psq_in + (size_t)(mval[mt] ? r + 16 * mt : 0) * nu;
      float s = 0.f;
      for (int u = q; u < nu; u += 4) s += ps[u];
      s += __shfl_xor(s, 16, 64);
      s += __shfl_xor(s, 32, 64);
      rinv[mt] = 1.0f / sqrtf(s / (float)p.K + p.eps);
    }
  }

  f32x4_t acc[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const uint4* wt = reinterpret_cast<const uint4*>(p.w);
  size_t wrow[NTW];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) wrow[nt] = (size_t)(unit * NTW + nt) * KT * 64 + lane;
  const uint4* nwp = reinterpret_cast<const uint4*>(p.nw);

  auto make_a = [&](uint4 raw, const uint4& gain, int mt) -> bf16x8_t {
    if (!mval[mt]) raw = make_uint4(0, 0, 0, 0);
    if constexpr (NORM) {
      float f[8], g[8], o[8];
      unpack8(raw, f);
      unpack8(gain, g);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = mul_rn(g[e], rbf(mul_rn(f[e], rinv[mt])));
      return as_bf16x8(pack8(o));
    } else {
      return as_bf16x8(raw);
    }
  };

  // Each batch issues all of its loads first (weights from HBM, activations and
  // gains from L2), then runs the MFMAs in arrival order. The last batch of a
  // range is padded by re-reading step k1-1 (a cache hit) with a zero A
  // operand, so there is no serial remainder loop.
  for (int kt = k0; kt < k1; kt += U) {
    uint4 bt[U][NTW], at[U][MT], gt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = min(kt + u, k1 - 1);
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) bt[u][nt] = wt[wrow[nt] + (size_t)kk * 64];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = min(kt + u, k1 - 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) at[u][mt] = *reinterpret_cast<const uint4*>(xrow[mt] + kk * 32);
      if constexpr (NORM) gt[u] = nwp[kk * 4 + q];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = kt + u < k1;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        bf16x8_t a = make_a(at[u][mt], gt[u], mt);
        if (!live) a = as_bf16x8(make_uint4(0, 0, 0, 0));
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(bt[u][nt]), acc[mt][nt], 0, 0, 0);
      }
    }
  }

  if constexpr (KSPLIT > 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) red[((wave * MT + mt) * NTW + nt) * 64 + lane] = acc[mt][nt];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        f32x4_t s = red[(mt * NTW + nt) * 64 + lane];
        for (int w = 1; w < KSPLIT; ++w) s += red[((w * MT + mt) * NTW + nt) * 64 + lane];
        acc[mt][nt] = s;
      }
  }

  // Epilogue. Lane (q, r) holds D[16*mt + 4*q + i][16*(unit*NTW + nt) + r].
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mt + 4 * q + i;
      if constexpr (EPI == EPI_ARGMAX) {
        float best = -INFINITY;
        int bidx = 0x7fffffff;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
          const float v = rbf(acc[mt][nt][i]);
          const int col = (unit * NTW + nt) * 16 + r;
          if (v > best) { best = v; bidx = col; }
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          const float ov = __shfl_xor(best, o, 64);
          const int oi = __shfl_xor(bidx, o, 64);
          if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
        }
        if (r == 0 && m < p.M) {
          p.pval[(size_t)unit * p.M + m] = best;
          p.pidx[(size_t)unit * p.M + m] = bidx;
        }
      } else {
        const bool mok = m < p.M;
        bf16_t* orow = p.out + (size_t)(mok ? m : 0) * p.ld_out;
        if constexpr (EPI == EPI_SWIGLU) {
          const float g = rbf(acc[mt][0][i]);
          const float u = rbf(acc[mt][1][i]);
          const float s = rbf(g / (1.0f + expf(-g)));
          if (mok) orow[unit * 16 + r] = f2bf(mul_rn(s, u));
        } else {
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt) {
            const int col = (unit * NTW + nt) * 16 + r;
            if constexpr (EPI == EPI_RES) {
              const float rv = mok ? bf2f(p.res[(size_t)m * p.ld_out + col]) : 0.f;
              const bf16_t o = f2bf(add_rn(rv, rbf(acc[mt][nt][i])));
              if (mok) orow[col] = o;
              if (p.psq_out) {  // partial sum of squares of the new row over these 16 columns
                const float v = bf2f(o);
                float sq = mul_rn(v, v);
                sq += __shfl_xor(sq, 1, 64);
                sq += __shfl_xor(sq, 2, 64);
                sq += __shfl_xor(sq, 4, 64);
                sq += __shfl_xor(sq, 8, 64);
                if (mok && r == 0) p.psq_out[(size_t)m * (p.N >> 4) + (col >> 4)] = sq;
              }
            } else {
              if (mok) orow[col] = f2bf(acc[mt][nt][i]);
            }
          }
        }
      }
    }
  }
}

// Reduce the per-workgroup (max, index) partials of one row: lowest index wins ties.
__global__ void __launch_bounds__(256) argmax_finalize_kernel(const float* __restrict__ pval,
                                                               const int32_t* __restrict__ pidx, int units, int M,
                                                               int64_t* __restrict__ out) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int m = blockIdx.x;
  float best = -INFINITY;
  int bidx = 0x7fffffff;
  for (int u = threadIdx.x; u < units; u += blockDim.x) {
    const float v = pval[(size_t)u * M + m];
    const int i = pidx[(size_t)u * M + m];
    if (v > best || (v == best && i < bidx)) { best = v; bidx = i; }
  }
  sv[threadIdx.x] = best;
  si[threadIdx.x] = bidx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      const float ov = sv[threadIdx.x + s];
      const int oi = si[threadIdx.x + s];
      if (ov > sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < si[threadIdx.x])) {
        sv[threadIdx.x] = ov;
        si[threadIdx.x] = oi;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[m] = si[0];
}

template <int MT, int NTW, int KSPLIT, bool NORM, int EPI>
hipError_t launch(const GemmParams& p, int units, hipStream_t stream) {
  skinny_gemm_kernel<MT, NTW, KSPLIT, NORM, EPI><<<units, 64 * KSPLIT, 0, stream>>>(p);
  return hipGetLastError();
}

// Dispatch over the instantiated (MT, NTW, KSPLIT) combinations.
template <bool NORM, int EPI>
int dispatch(const GemmParams& p, int units, int mt, int ntw, int ksplit, hipStream_t stream) {
#define QWEN_GEMM_CASE(MT_, NTW_, KS_) \
  if (mt == MT_ && ntw == NTW_ && ksplit == KS_) return qwen_status(launch<MT_, NTW_, KS_, NORM, EPI>(p, units, stream));
#define QWEN_GEMM_KS(MT_, NTW_) \
  QWEN_GEMM_CASE(MT_, NTW_, 1) QWEN_GEMM_CASE(MT_, NTW_, 2) QWEN_GEMM_CASE(MT_, NTW_, 4) QWEN_GEMM_CASE(MT_, NTW_, 8)
  if constexpr (EPI != EPI_SWIGLU) {
    QWEN_GEMM_KS(1, 1)
    QWEN_GEMM_CASE(1, 1, 16)
    QWEN_GEMM_KS(2, 1)
  }
  QWEN_GEMM_KS(1, 2)
  QWEN_GEMM_KS(2, 2)
#undef QWEN_GEMM_KS
#undef QWEN_GEMM_CASE
  return QWEN_EARG;
}

int check_common(const void* x, const void* w, int M, int N, int K, int ntw, int ksplit) {
  if (!x || !w) return QWEN_ENULL;
  if (M <= 0 || M > 32 || N <= 0 || K <= 0 || K % 32 != 0) return QWEN_EARG;
  if (ntw != 1 && ntw != 2) return QWEN_EARG;
  if (ksplit != 1 && ksplit != 2 && ksplit != 4 && ksplit != 8 && ksplit != 16) return QWEN_EARG;
  if (N % (16 * ntw) != 0) return QWEN_EARG;
  return QWEN_OK;
}

}  // namespace

extern "C" {

// epi: 0 = store, 1 = residual add (residual may alias out), 2 = SwiGLU pair
// (N counts gate + up rows; out has N/2 columns). norm_w == nullptr: no norm prologue.
int qwen_linear(const void* x, const void* w_tiled, void* out, int M, int N, int K, int ld_out, const void* norm_w,
                const float* psq_in, float eps, const void* residual, float* psq_out, int epi, int ntw, int ksplit,
                hipStream_t stream) {
  int st = check_common(x, w_tiled, M, N, K, ntw, ksplit);
  if (st) return st;
  if (!out) return QWEN_ENULL;
  if (epi == EPI_RES && !residual) return QWEN_ENULL;
  if (norm_w && !psq_in) return QWEN_ENULL;
  if (psq_out && (epi != EPI_RES || N % 16 != 0)) return QWEN_EARG;
  if (epi == EPI_SWIGLU && ntw != 2) return QWEN_EARG;
  if (epi < EPI_STORE || epi > EPI_SWIGLU) return QWEN_EARG;
  const int out_cols = epi == EPI_SWIGLU ? N / 2 : N;
  if (ld_out < out_cols) return QWEN_EARG;
  GemmParams p{(const bf16_t*)x, (const bf16_t*)w_tiled, (const bf16_t*)norm_w, (const bf16_t*)residual,
               (bf16_t*)out, nullptr, nullptr, psq_in, psq_out, M, N, K, ld_out, eps};
  const int units = N / (16 * ntw);
  const int mt = M > 16 ? 2 : 1;
  // Instantiated variants: norm+store (QKV), store (plain linear), residual
  // (O / down projections), norm+SwiGLU (gate/up).
  if (epi == EPI_STORE) return norm_w ? dispatch<true, EPI_STORE>(p, units, mt, ntw, ksplit, stream)
                                      : dispatch<false, EPI_STORE>(p, units, mt, ntw, ksplit, stream);
  if (epi == EPI_RES) return norm_w ? QWEN_EARG : dispatch<false, EPI_RES>(p, units, mt, ntw, ksplit, stream);
  return norm_w ? dispatch<true, EPI_SWIGLU>(p, units, mt, ntw, ksplit, stream) : QWEN_EARG;
}

long long qwen_argmax_workspace_bytes(int M, int N, int ntw) {
  if (M <= 0 || N <= 0 || (ntw != 1 && ntw != 2)) return 0;
  const long long units = N / (16 * ntw);
  return units * M * (long long)(sizeof(float) + sizeof(int32_t));
}

// Final RMSNorm (norm_w) + LM head GEMM + argmax over the bf16 logits,
// lowest index on ties. out_tok: [M] int64.
int qwen_lm_head_argmax(const void* x, const void* norm_w, const float* psq_in, float eps, const void* w_tiled, int M,
                        int N, int K, void* workspace, long long workspace_bytes, int64_t* out_tok, int ntw,
                        int ksplit, hipStream_t stream) {
  int st = check_common(x, w_tiled, M, N, K, ntw, ksplit);
  if (st) return st;
  if (!out_tok || !workspace || !norm_w || !psq_in) return QWEN_ENULL;
  if (workspace_bytes < qwen_argmax_workspace_bytes(M, N, ntw)) return QWEN_EWORKSPACE;
  const int units = N / (16 * ntw);
  float* pval = (float*)workspace;
  int32_t* pidx = (int32_t*)(pval + (size_t)units * M);
  GemmParams p{(const bf16_t*)x, (const bf16_t*)w_tiled, (const bf16_t*)norm_w, nullptr, nullptr, pval, pidx,
               psq_in, nullptr, M, N, K, 0, eps};
  const int mt = M > 16 ? 2 : 1;
  st = dispatch<true, EPI_ARGMAX>(p, units, mt, ntw, ksplit, stream);
  if (st) return st;
  argmax_finalize_kernel<<<M, 256, 0, stream>>>(pval, pidx, units, M, out_tok);
  QWEN_RETURN_LAUNCH();
}

}  // extern "C"
