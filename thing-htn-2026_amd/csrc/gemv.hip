// Balanced weight-streaming GEMV for the decode projections at M <= 2 rows.
//
// out[M, N] = x[M, K] @ W[N, K]^T, bf16 operands, fp32 accumulation, one bf16
// rounding (engine/kernels/gemm.py:12-15), with the fused RMSNorm prologue and
// residual / SwiGLU / argmax epilogues of engine/kernels/gemm_fused.py:5-19 and
// :179-193 (same rounding points as the MFMA kernels in gemm.hip).
//
// Why a second kernel for M <= 2: a decode projection at batch 1 is a pure
// weight stream, and one CU sustains only about 1/256 of the HBM bandwidth, so
// every CU must stream the same number of bytes. The MFMA kernels cut work into
// 16-row tiles, which leaves CUs idle for N = 2560 (160 tiles) and unbalanced
// for the others. Here workgroup g of G owns output rows [N*g/G, N*(g+1)/G) of
// the row-major weight ([N, K], HF nn.Linear layout; for SwiGLU [2N, K] =
// gate rows then up rows, and the workgroup owns gate row n and up row n), and
// the rows are reduced inside the workgroup, so no partial sum crosses
// workgroups. A workgroup's rows x (K / 512) chunks of 1 KB are cut into equal
// contiguous ranges, one per wavefront; every chunk is one 16-byte
// non-temporal load per lane (1 KB contiguous per wavefront instruction), with
// GV_DEPTH chunks in flight per wavefront. The activation rows are staged in
// LDS once per workgroup (normalised there when the prologue is RMSNorm, with
// the row statistics computed in the workgroup from the staged row itself), and
// each chunk is a 4 x v_dot2_f32_bf16 chain per row. Per-row partials of the
// wavefronts go to LDS and are summed in wavefront order (deterministic).
#include "common.h"

namespace {

enum { GEPI_STORE = 0, GEPI_RES = 1, GEPI_SWIGLU = 2, GEPI_ARGMAX = 3 };

constexpr int GV_CHUNK = 512;  // bf16 elements per row chunk: 1 KB, one wavefront load
constexpr int GV_DEPTH = 6;    // chunks in flight per wavefront
constexpr int GV_XC_NORM = 2;  // staged 16-byte activation chunks per thread: normed rows
constexpr int GV_XC_PLAIN = 5; // plain rows (down projection: K = 9728 at M = 2 over 512 threads)

typedef uint32_t gv_u32x4_t __attribute__((ext_vector_type(4)));

struct GemvParams {
  const bf16_t* x;      // [M, K] row-major
  const bf16_t* w;      // [N * PAIR, K] row-major
  const bf16_t* nw;     // [K] RMSNorm gain (NORM)
  const bf16_t* res;    // [M, ld_out] residual (GEPI_RES; may alias out)
  bf16_t* out;          // [M, ld_out]
  unsigned long long* amax;  // packed argmax keys (GEPI_ARGMAX, slot 0 of each row), zero before the launch
  const int32_t* rowmap;     // [N] output column of weight row i (GEPI_STORE; nullptr: column i)
  int N, K, ld_out;     // N = output columns (SwiGLU: gate/up row pairs)
  float eps;
};

__device__ __forceinline__ uint4 gv_load_nt(const uint4* p) {
  const gv_u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const gv_u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ uint32_t gv_ordered_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.x), __builtin_bit_cast(bf16x2_t, b.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.y), __builtin_bit_cast(bf16x2_t, b.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.z), __builtin_bit_cast(bf16x2_t, b.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.w), __builtin_bit_cast(bf16x2_t, b.w), acc, false);
  return acc;
}

// Dynamic LDS: x rows [M][K] bf16, then per-row wavefront partials [PR][WAVES][M] fp32,
// then the workgroup reduction scratch.
template <int M, int WAVES, bool NORM, int EPI>
__global__ void __launch_bounds__(64 * WAVES) gemv_kernel(GemvParams p) {
  extern __shared__ __align__(16) unsigned char gv_smem[];
  constexpr int NT = 64 * WAVES;
  constexpr int PAIR = EPI == GEPI_SWIGLU ? 2 : 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wavefront-uniform: scalar branches
  const int G = gridDim.x, g = blockIdx.x;
  const int K = p.K, KC = K / GV_CHUNK;
  const long long N = p.N;
  const int r0 = (int)(N * g / G), r1 = (int)(N * (g + 1) / G);
  const int R = r1 - r0;
  const int PR = R * PAIR;
  const int items = PR * KC;
  const int i0 = (int)((long long)items * wave / WAVES), i1 = (int)((long long)items * (wave + 1) / WAVES);

  bf16_t* xs = reinterpret_cast<bf16_t*>(gv_smem);
  float* part = reinterpret_cast<float*>(gv_smem + (size_t)M * K * 2);
  float* red = part + (size_t)PR * WAVES * M;  // [WAVES][M] (+ argmax scratch)

  // Issue cursor over this wavefront's chunks [i0, i1): (physical row ipr, chunk ic). Past the
  // range the loads read a dummy address inside the activation rows, which are cache-resident:
  // every load is issued unconditionally, so the compiler's wait counts stay exact, and no
  // dummy load reaches HBM.
  const int n = i1 - i0;
  const uint4* wb = reinterpret_cast<const uint4*>(p.w);
  const uint4* xb = reinterpret_cast<const uint4*>(p.x);
  int ipr = n > 0 ? i0 / KC : 0;
  int ic = n > 0 ? i0 - ipr * KC : 0;
  int left = n;
  auto wptr = [&]() -> const uint4* {
    if (left <= 0) return xb + lane;
    const long long row = (PAIR == 2 && ipr >= R) ? N + r0 + (ipr - R) : (long long)(r0 + ipr);
    return wb + ((row * K + (long long)ic * GV_CHUNK) >> 3) + lane;
  };
  auto advance = [&]() {
    if (left > 0) {
      --left;
      if (++ic == KC) { ic = 0; ++ipr; }
    }
  };

  uint4 buf[GV_DEPTH];
  auto issue = [&](int s) {
    buf[s] = gv_load_nt(wptr());
    advance();
  };

  // The activation rows are staged in LDS once per workgroup (normalised there with NORM):
  // this thread's XC 16-byte chunks (and gains) are requested before the weights, since
  // loads return in issue order and anything the staging needs that is requested after the
  // weight prefetch would wait for HBM. Chunks past the rows re-read the last one (issued
  // unconditionally, so the compiler's wait for them leaves the weights in flight).
  const int kc8 = K >> 3;
  const int nch = M * kc8;
  constexpr int XC = NORM ? GV_XC_NORM : GV_XC_PLAIN;
  gv_u32x4_t xv[XC], gv[NORM ? XC : 1];  // ext-vector registers (an array of uint4 would live in scratch)
#pragma unroll
  for (int q = 0; q < XC; ++q) {
    const int cq = min((int)threadIdx.x + q * NT, nch - 1);
    xv[q] = reinterpret_cast<const gv_u32x4_t*>(p.x)[cq];
    if constexpr (NORM) gv[q] = reinterpret_cast<const gv_u32x4_t*>(p.nw)[cq % kc8];
  }
#pragma unroll
  for (int s = 0; s < GV_DEPTH; ++s) issue(s);
  __builtin_amdgcn_sched_barrier(0);  // the staging below stays after the weight requests

  for (int j = threadIdx.x; j < PR * WAVES * M; j += NT) part[j] = 0.f;

  if constexpr (NORM) {
    // Normalised rows: fp32 sum of squares per row (threads in index order, then wavefronts
    // in order), rinv, then x <- bf16(bf16(x * rinv) * gain).
    float ss[M];
#pragma unroll
    for (int m = 0; m < M; ++m) ss[m] = 0.f;
#pragma unroll
    for (int q = 0; q < XC; ++q) {
      const int cidx = threadIdx.x + q * NT;
      if (cidx < nch) {
        float f[8], t = 0.f;
        unpack8(make_uint4(xv[q].x, xv[q].y, xv[q].z, xv[q].w), f);
#pragma unroll
        for (int e = 0; e < 8; ++e) t = add_rn(t, mul_rn(f[e], f[e]));
        const int m = cidx / kc8;
#pragma unroll
        for (int mm = 0; mm < M; ++mm) ss[mm] = add_rn(ss[mm], mm == m ? t : 0.f);
      }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = wave_sum_dpp(ss[m]);
      if (lane == 0) red[wave * M + m] = v;
    }
    __syncthreads();
    float rinv[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float t = 0.f;
      for (int w = 0; w < WAVES; ++w) t += red[w * M + m];
      rinv[m] = rms_rinv(t, K, p.eps);
    }
#pragma unroll
    for (int q = 0; q < XC; ++q) {
      const int cidx = threadIdx.x + q * NT;
      if (cidx < nch) {
        const int m = cidx / kc8;
        float f[8], gn[8], o[8];
        unpack8(make_uint4(xv[q].x, xv[q].y, xv[q].z, xv[q].w), f);
        unpack8(make_uint4(gv[q].x, gv[q].y, gv[q].z, gv[q].w), gn);
        float ri = rinv[0];
#pragma unroll
        for (int mm = 1; mm < M; ++mm) ri = mm == m ? rinv[mm] : ri;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = mul_rn(gn[e], rbf(mul_rn(f[e], ri)));
        reinterpret_cast<uint4*>(xs)[cidx] = pack8(o);
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < XC; ++q) {
      const int cidx = threadIdx.x + q * NT;
      if (cidx < nch) reinterpret_cast<gv_u32x4_t*>(xs)[cidx] = xv[q];
    }
  }
  __syncthreads();

  // Consume this wavefront's chunks with GV_DEPTH in flight, refilling each slot as it is consumed.
  float acc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) acc[m] = 0.f;
  int pr = n > 0 ? i0 / KC : 0;
  int c = n > 0 ? i0 - pr * KC : 0;
  auto flush = [&]() {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float v = wave_sum_dpp(acc[m]);
      if (lane == 0) part[((size_t)pr * WAVES + wave) * M + m] = v;
      acc[m] = 0.f;
    }
  };
  auto consume = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const uint4 xc = reinterpret_cast<const uint4*>(xs + (size_t)m * K + (size_t)c * GV_CHUNK)[lane];
      acc[m] = dot8(buf[s], xc, acc[m]);
    }
    if (++c == KC) {
      flush();
      c = 0;
      ++pr;
    }
  };
  // Groups of GV_DEPTH chunks: every group but the last is all real and refills its slots with
  // the next group (unconditional issues; past the range a dummy); the last group only consumes,
  // so a wavefront's end waits for no load it does not use.
  const int ng = (n + GV_DEPTH - 1) / GV_DEPTH;
  int grp = 0;
  for (; grp + 1 < ng; ++grp) {
#pragma unroll
    for (int s = 0; s < GV_DEPTH; ++s) {
      consume(s);
      issue(s);
    }
  }
  if (ng > 0) {
#pragma unroll
    for (int s = 0; s < GV_DEPTH; ++s)
      if (grp * GV_DEPTH + s < n) consume(s);
  }
  if (n > 0 && c != 0) flush();
  __syncthreads();

  // Epilogue: row sums in wavefront order.
  if constexpr (EPI == GEPI_ARGMAX) {
    // First-index argmax of bf16(logit) over this workgroup's rows, per output row m.
    float* bv = red;                                   // [WAVES][M] best values
    int* bi = reinterpret_cast<int*>(red + WAVES * M);  // [WAVES][M] best indices
#pragma unroll
    for (int m = 0; m < M; ++m) {
      float best = -INFINITY;
      int bidx = 0x7fffffff;
      for (int r = threadIdx.x; r < R; r += NT) {
        float v = 0.f;
        for (int w = 0; w < WAVES; ++w) v += part[((size_t)r * WAVES + w) * M + m];
        v = rbf(v);
        if (v > best) { best = v; bidx = r0 + r; }  // rows ascend per thread: first index kept on ties
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bidx, o, 64);
        if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
      }
      if (lane == 0) { bv[wave * M + m] = best; bi[wave * M + m] = bidx; }
    }
    __syncthreads();
    if (threadIdx.x < M && R > 0) {
      const int m = threadIdx.x;
      float best = -INFINITY;
      int bidx = 0x7fffffff;
      for (int w = 0; w < WAVES; ++w) {
        const float v = bv[w * M + m];
        const int i = bi[w * M + m];
        if (v > best || (v == best && i < bidx)) { best = v; bidx = i; }
      }
      const unsigned long long key =
          ((unsigned long long)gv_ordered_bits(best) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)bidx);
      __hip_atomic_fetch_max(p.amax + m, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  } else {
    for (int t = threadIdx.x; t < R * M; t += NT) {
      const int m = t / R, r = t - m * R;
      float v = 0.f;
      for (int w = 0; w < WAVES; ++w) v += part[((size_t)r * WAVES + w) * M + m];
      const size_t o = (size_t)m * p.ld_out + r0 + r;
      if constexpr (EPI == GEPI_STORE) {
        p.out[p.rowmap ? (size_t)m * p.ld_out + p.rowmap[r0 + r] : o] = f2bf(v);
      } else if constexpr (EPI == GEPI_RES) {
        p.out[o] = f2bf(add_rn(bf2f(p.res[o]), rbf(v)));
      } else {  // SwiGLU: gate row r, up row R + r
        float u = 0.f;
        for (int w = 0; w < WAVES; ++w) u += part[((size_t)(R + r) * WAVES + w) * M + m];
        const float gg = rbf(v);
        const float s = rbf(gg / (1.0f + expf(-gg)));
        p.out[o] = f2bf(mul_rn(s, rbf(u)));
      }
    }
  }
}

size_t gemv_lds_bytes(int M, int N, int K, int G, int waves, int epi) {
  const long long rows = (N + G - 1) / G + 1;
  const long long pr = rows * (epi == GEPI_SWIGLU ? 2 : 1);
  return (size_t)M * K * 2 + (size_t)(pr * waves * M) * 4 + (size_t)waves * M * 8;
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
                     int grid, int waves, hipStream_t stream) {
  if (!x || !w) return QWEN_ENULL;
  if (row_map && epi != GEPI_STORE) return QWEN_EARG;
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
               amax, row_map, N, K, ld_out, eps};
  if (M == 1) return waves == 16 ? dispatch_gemv<1, 16>(p, norm_w != nullptr, epi, grid, lds, stream)
                                 : dispatch_gemv<1, 8>(p, norm_w != nullptr, epi, grid, lds, stream);
  return waves == 16 ? dispatch_gemv<2, 16>(p, norm_w != nullptr, epi, grid, lds, stream)
                     : dispatch_gemv<2, 8>(p, norm_w != nullptr, epi, grid, lds, stream);
}

int qwen_gemv(const void* x, const void* w, void* out, int M, int N, int K, int ld_out, const void* norm_w, float eps,
              const void* residual, int epi, unsigned long long* amax, int grid, int waves, hipStream_t stream) {
  return qwen_gemv_rowmap(x, w, out, M, N, K, ld_out, norm_w, eps, residual, epi, amax, nullptr, grid, waves, stream);
}

}  // extern "C"
