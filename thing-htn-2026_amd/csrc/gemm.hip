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
//   EPI_ARGMAX: logits = bf16(acc); the row's (max logit, lowest index) is folded
//               into a packed 64-bit key with one atomicMax per row and workgroup
//               (LM head + argmax, engine/engine.py:1119-1121).
//
// Weight layout ("MFMA-B tiles", written by weights.hip): W is cut into tiles
// of 16 rows x 32 k; tile (nt, kt) is 1 KB at offset (nt * K/32 + kt) * 512
// elements and lane l = 16*q + r of a wavefront owns the 16 bytes
// W[16*nt + r][32*kt + 8*q .. +8] at tile offset 8*l. One global_load_dwordx4
// per lane therefore reads a whole tile (1 KB contiguous) straight into the
// B-operand registers of v_mfma_f32_16x16x32_bf16; the k-reduction happens in
// the matrix core. Weights are read with non-temporal loads: every byte is used
// once per step, and keeping it out of the memory-side cache raises the
// sustained HBM read rate on MI355X (measured 7.0 vs 6.2 TB/s for a plain
// streaming read). M <= 16 rows use one A fragment, 17..32 rows use two.
//
// Work decomposition: the N/16 n-tiles are grouped NTW per "unit"; each unit's
// K range is split over KS workgroups, and each workgroup's range over its WPG
// wavefronts. Wavefront partials are reduced through LDS in a fixed order.
// With KS > 1 every workgroup stores its fp32 partial with device-coherent
// (sc1) stores, then bumps the unit's arrival counter; the last arriver reads
// the KS partials back with sc1 loads, sums them in split order (so the result
// does not depend on arrival order), runs the epilogue and re-arms the counter
// to zero. No full-cache fences are needed because every value that crosses
// workgroups travels with device-scope stores and loads.
#include "common.h"

namespace {

enum { EPI_STORE = 0, EPI_RES = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };

// Split-K workspace: arrival counters for up to 16384 n-tile groups, then partials.
constexpr long long QWEN_LINEAR_COUNTER_BYTES = 65536;

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct GemmParams {
  const bf16_t* x;      // [M, K] row-major
  const bf16_t* w;      // MFMA-B tiled weight, N x K
  const bf16_t* nw;     // [K] RMSNorm gain (NORM)
  const bf16_t* res;    // [M, ld_out] residual (EPI_RES)
  bf16_t* out;          // [M, ld_out]
  unsigned long long* amax;  // [M] packed (logit, index) keys (EPI_ARGMAX), zero before the launch
  const float* psq_in;  // [M, K/16] partial sums of squares of x per 16 columns (NORM)
  float* psq_out;       // [M, N/16] same for the output rows (EPI_RES, may be null)
  f32x4_t* part;        // [units * KS][MT*NTW][64] split-K partials (KS > 1)
  unsigned* cnt;        // [units] arrival counters, zero between launches (KS > 1)
  int M, N, K, ld_out, ks;
  int piece_stride;     // partial slots per unit in `part` (ks for split-K, SK_PIECES for stream-K)
  float eps;
};

__device__ __forceinline__ uint4 load_nt(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Monotone map of an fp32 value onto uint32 (larger float -> larger integer).
__device__ __forceinline__ uint32_t ordered_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The A operand of one wavefront: rows m = r + 16*mt of x (rows past M read
// row 0, the same cache lines as a live row, and are zeroed, so the loads need
// no branch), and with NORM the RMSNorm factor of each row.
template <int MT, bool NORM>
struct AOperand {
  const bf16_t* xrow[MT];
  bool mval[MT];
  float rinv[MT];

  __device__ __forceinline__ void init(const GemmParams& p, int r, int q) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = r + 16 * mt;
      mval[mt] = m < p.M;
      xrow[mt] = p.x + (size_t)(mval[mt] ? m : 0) * p.K + 8 * q;
    }
  }

  // RMSNorm statistics: the producer of x left one partial sum of squares per
  // 16 columns (rounded bf16 values, squared and summed in fp32). The four
  // lanes of a row each add a contiguous quarter of them in a fixed order,
  // then the quarters are combined by a fixed butterfly, so every workgroup
  // derives bit-identical factors. The quarter is read with float4 loads that
  // are all issued by stats_load (before the first weights, so that waiting
  // for them does not wait for HBM) and added by stats_finish (out-of-range
  // slots add zero).
  static constexpr int MAXV = 10;  // float4 loads per lane: up to 40 partials (K <= 2560)
  f32x4_t sv[NORM ? MT : 1][MAXV];

  __device__ __forceinline__ bool stats_fast(const GemmParams& p) const {
    const int nu = p.K >> 4;
    return (nu & 15) == 0 && (nu >> 2) <= 4 * MAXV;
  }

  __device__ __forceinline__ void stats_load(const GemmParams& p, int r, int q) {
    if constexpr (NORM) {
      if (!stats_fast(p)) return;
      const int nu = p.K >> 4;
      const int per = nu >> 2;
      const int n4 = per >> 2;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float* ps = p.psq_in + (size_t)(mval[mt] ? r + 16 * mt : 0) * nu;
        const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(ps + q * per);
#pragma unroll
        for (int j = 0; j < MAXV; ++j) sv[mt][j] = p4[min(j, n4 - 1)];
      }
    }
  }

  __device__ __forceinline__ void stats_finish(const GemmParams& p, int r, int q) {
    if constexpr (NORM) {
      const int nu = p.K >> 4;
      const int per = nu >> 2;
      const bool fast = stats_fast(p);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float s = 0.f;
        if (fast) {
          const int n4 = per >> 2;
#pragma unroll
          for (int j = 0; j < MAXV; ++j) {
            const float keep = j < n4 ? 1.f : 0.f;
            s += sv[mt][j].x * keep;
            s += sv[mt][j].y * keep;
            s += sv[mt][j].z * keep;
            s += sv[mt][j].w * keep;
          }
        } else {
          const float* ps = p.psq_in + (size_t)(mval[mt] ? r + 16 * mt : 0) * nu;
          for (int u = q * per; u < (q + 1) * per; ++u) s += ps[u];
          if (nu & 3) {  // the last nu % 4 partials belong to lane q = 3
            for (int u = 4 * per; u < nu; ++u) s += q == 3 ? ps[u] : 0.f;
          }
        }
        s = xor32_sum(xor16_sum(s));  // the row's four quarters (lanes r, r + 16, r + 32, r + 48)
        rinv[mt] = rms_rinv(s, p.K, p.eps);
      }
    }
  }

  __device__ __forceinline__ void stats(const GemmParams& p, int r, int q) {
    stats_load(p, r, q);
    stats_finish(p, r, q);
  }

  // bf16x8 A fragment: raw x, or with NORM bf16(bf16(x * rinv) * gain).
  __device__ __forceinline__ bf16x8_t make(uint4 raw, const uint4& gain, int mt) const {
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
  }
};

// Software-pipelined accumulation of k-steps [k0, k1) of one n-tile group:
// a batch is U k-steps of loads (weights from HBM with non-temporal loads,
// activations and gains from L2); the next batch is issued before the current
// one is consumed, so two batches are in flight per wavefront. The steady-state
// issues are unconditional (a conditional issue makes the compiler's wait at the
// join count the batch just requested, which serialises the pipeline) and the
// last one or two batches form a separate tail. Within a batch, weight slots
// past k1 read a cache-resident dummy (the activation rows) and the activation
// slots re-read step k1-1; both meet a zero A operand. With `stats_after_first`
// the A operand's RMSNorm statistics are requested before the first weights and
// added once those are in flight.
template <int MT, int NTW, int U, bool NORM, typename AfterFirst>
__device__ __forceinline__ void accumulate(const GemmParams& p, AOperand<MT, NORM>& A, size_t unit, int k0, int k1,
                                           f32x4_t (&acc)[MT][NTW], int r, int q, int lane, bool stats_after_first,
                                           AfterFirst&& after_first) {
  const uint4* wt = reinterpret_cast<const uint4*>(p.w);
  const uint4* nwp = reinterpret_cast<const uint4*>(p.nw);
  const size_t KT = p.K >> 5;
  size_t wrow[NTW];
#pragma unroll
  for (int nt = 0; nt < NTW; ++nt) wrow[nt] = (unit * NTW + nt) * KT * 64 + lane;
  struct Batch {
    uint4 bt[U][NTW], at[U][MT], gt[U];
  };
  const uint4* dummy = reinterpret_cast<const uint4*>(p.x) + lane;
  auto issue = [&](Batch& b, int kt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = kt + u < k1;
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) b.bt[u][nt] = load_nt(live ? wt + wrow[nt] + (size_t)(kt + u) * 64 : dummy);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = min(kt + u, k1 - 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) b.at[u][mt] = *reinterpret_cast<const uint4*>(A.xrow[mt] + kk * 32);
      if constexpr (NORM) b.gt[u] = nwp[kk * 4 + q];
    }
  };
  auto consume = [&](const Batch& b, int kt) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool live = kt + u < k1;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        bf16x8_t a = A.make(b.at[u][mt], b.gt[u], mt);
        if (!live) a = as_bf16x8(make_uint4(0, 0, 0, 0));
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(b.bt[u][nt]), acc[mt][nt], 0, 0, 0);
      }
    }
  };
  Batch b0, b1;
  if (k0 >= k1) {
    if (stats_after_first) A.stats(p, r, q);
    after_first();
    return;
  }
  if (stats_after_first) A.stats_load(p, r, q);
  issue(b0, k0);
  if (stats_after_first) A.stats_finish(p, r, q);
  after_first();
  // Steady state: while at least two batches follow the current one, both issues are
  // unconditional; the last one or two batches are a separate (wavefront-uniform) tail, so
  // no batch is requested that is not consumed.
  int kt = k0;
  for (; kt + 2 * U < k1; kt += 2 * U) {
    issue(b1, kt + U);
    consume(b0, kt);
    issue(b0, kt + 2 * U);
    consume(b1, kt + U);
  }
  if (kt + U < k1) {
    issue(b1, kt + U);
    consume(b0, kt);
    consume(b1, kt + U);
  } else {
    consume(b0, kt);
  }
}

// Epilogue of one n-tile group (unit). Lane (q, r) holds D[16*mt + 4*q + i][16*(unit*NTW + nt) + r].
// Residual values of one unit's output tile (EPI_RES; empty otherwise), all requested before
// any is used (rows past M re-read row 0). The residual may alias the output, so loads placed
// between the epilogue's stores would each wait for their own round trip.
template <int MT, int NTW, int EPI>
struct ResRows {
  float v[EPI == EPI_RES ? MT : 1][4][EPI == EPI_RES ? NTW : 1];
  __device__ __forceinline__ void load(const GemmParams& p, long long unit, int lane) {
    if constexpr (EPI == EPI_RES) {
      const int r = lane & 15, q = lane >> 4;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = 16 * mt + 4 * q + i;
          const bf16_t* rrow = p.res + (size_t)(m < p.M ? m : 0) * p.ld_out;
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt) v[mt][i][nt] = bf2f(rrow[(unit * NTW + nt) * 16 + r]);
        }
    }
  }
};

template <int MT, int NTW, int EPI>
__device__ __forceinline__ void epilogue(const GemmParams& p, f32x4_t (&acc)[MT][NTW], long long unit, int lane,
                                         const ResRows<MT, NTW, EPI>& res) {
  const int r = lane & 15, q = lane >> 4;
  const auto& rv = res.v;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = 16 * mt + 4 * q + i;
      const bool mok = m < p.M;
      if constexpr (EPI == EPI_ARGMAX) {
        float best = -INFINITY;
        int bidx = 0x7fffffff;
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
          const float v = rbf(acc[mt][nt][i]);
          const int col = (int)(unit * NTW + nt) * 16 + r;
          if (v > best) { best = v; bidx = col; }
        }
        row16_argmax(best, bidx);  // over the 16 columns r of this row
        if (r == 0 && mok) {
          const unsigned long long key =
              ((unsigned long long)ordered_bits(best) << 32) | (unsigned long long)(0xffffffffu - (uint32_t)bidx);
          __hip_atomic_fetch_max(p.amax + (long long)(blockIdx.x % ARGMAX_SLOTS) * argmax_ld(p.M) + m, key,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        bf16_t* orow = p.out + (size_t)(mok ? m : 0) * p.ld_out;
        if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
          for (int j = 0; j < NTW / 2; ++j) {
            const float g = rbf(acc[mt][2 * j][i]);
            const float u = rbf(acc[mt][2 * j + 1][i]);
            const float s = rbf(g / (1.0f + expf(-g)));
            if (mok) orow[(unit * (NTW / 2) + j) * 16 + r] = f2bf(mul_rn(s, u));
          }
        } else {
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt) {
            const long long col = (unit * NTW + nt) * 16 + r;
            if constexpr (EPI == EPI_RES) {
              const bf16_t o = f2bf(add_rn(rv[mt][i][nt], rbf(acc[mt][nt][i])));
              if (mok) orow[col] = o;
              if (p.psq_out) {  // partial sum of squares of the new row over these 16 columns
                const float v = bf2f(o);
                const float sq = row16_sum(mul_rn(v, v));
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

template <int MT, int NTW, int EPI>
__device__ __forceinline__ void epilogue(const GemmParams& p, f32x4_t (&acc)[MT][NTW], long long unit, int lane) {
  ResRows<MT, NTW, EPI> res;
  res.load(p, unit, lane);
  epilogue<MT, NTW, EPI>(p, acc, unit, lane, res);
}

// Cross-workgroup completion of one unit: store this workgroup's partial as
// piece `slot` of `pieces` (device-coherent stores), count the arrival; the
// last arriver sums the pieces in slot order (its own from registers), runs
// the epilogue and re-arms the counter. Called by one whole wavefront. The residual rows
// (EPI_RES) are requested first, so that they arrive during the store / count round trips.
template <int MT, int NTW, int EPI, bool PRELOADED = false, int FSV = 32>
__device__ __forceinline__ void finish_split(const GemmParams& p, f32x4_t (&acc)[MT][NTW], long long unit, int slot,
                                             int pieces, int lane, ResRows<MT, NTW, EPI> res = {}) {
  // Small units request the residual before the hand-off; wide ones (where the residual, the
  // pieces and the sums together would spill) after the pieces, in the epilogue.
  constexpr bool EARLY = MT * NTW <= 4;
  if constexpr (!PRELOADED && EARLY) res.load(p, unit, lane);
  f32x4_t* base = p.part + (size_t)unit * p.piece_stride * MT * NTW * 64;
  const __amdgpu_buffer_rsrc_t prs = coherent_rsrc(base);  // this unit's pieces: [piece][mt][nt][lane]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) store16_dev(prs, (((slot * MT + mt) * NTW + nt) * 64 + lane) * 16, acc[mt][nt]);
  __builtin_amdgcn_s_waitcnt(0);  // partial stores complete before the arrival is counted
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  unsigned old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(p.cnt + unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);  // lane 0's (every lane is active here)
  if (old != (unsigned)(pieces - 1)) return;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  // Pieces are requested FS_BATCH at a time (one round trip per batch rather than per
  // piece) and summed in slot order.
  constexpr int FS_BATCH = MT * NTW * 4 >= FSV ? 1 : FSV / (MT * NTW * 4);  // at most FSV VGPRs in flight
  f32x4_t sum[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) sum[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < pieces; j0 += FS_BATCH) {
    f32x4_t v[FS_BATCH][MT][NTW];
#pragma unroll
    for (int jj = 0; jj < FS_BATCH; ++jj) {
      const int j = min(j0 + jj, pieces - 1);  // past the end: a valid piece, not added
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) v[jj][mt][nt] = load16_dev(prs, (((j * MT + mt) * NTW + nt) * 64 + lane) * 16);
    }
#pragma unroll
    for (int jj = 0; jj < FS_BATCH; ++jj) {
      const int j = j0 + jj;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
          if (j < pieces) sum[mt][nt] += (j == slot) ? acc[mt][nt] : v[jj][mt][nt];
        }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = sum[mt][nt];
  if (lane == 0) __hip_atomic_store(p.cnt + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if constexpr (PRELOADED || EARLY) epilogue<MT, NTW, EPI>(p, acc, unit, lane, res);
  else epilogue<MT, NTW, EPI>(p, acc, unit, lane);
}

template <int MT, int NTW, int WPG, bool NORM, int EPI>
__global__ void __launch_bounds__(64 * WPG) skinny_gemm_kernel(GemmParams p) {
  constexpr int U = NTW >= 4 ? 1 : 4 / NTW;  // k-steps per batch (4 KB of weights, 8 KB at NTW = 8); two in flight
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wavefront-uniform: scalar branches
  const int r = lane & 15, q = lane >> 4;
  const int KS = p.ks;
  const int unit = blockIdx.x / KS;
  const int ks = blockIdx.x - unit * KS;
  const int KT = p.K >> 5;
  const int nranges = KS * WPG;
  const int kpw = (KT + nranges - 1) / nranges;
  const int k0 = min(KT, (ks * WPG + wave) * kpw);
  const int k1 = min(KT, k0 + kpw);

  __shared__ f32x4_t red[WPG > 1 ? (WPG - 1) * MT * NTW * 64 : 1];
  __shared__ float srinv[MT * 16];

  // Residual rows of the output tile (EPI_RES, small units): requested before anything else,
  // unconditionally by every wavefront, so the epilogue (wavefront 0) has them without a
  // round trip of its own.
  constexpr bool PRE_RES = EPI == EPI_RES && MT * NTW <= 4 && WPG <= 8;  // (16 wavefronts: 128 VGPRs)
  ResRows<MT, NTW, EPI> res;
  if constexpr (PRE_RES) res.load(p, unit, lane);
  AOperand<MT, NORM> A;
  A.init(p, r, q);
  f32x4_t acc[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // RMSNorm factors: wavefront 0 derives them (the same per-wavefront code, so the same bits)
  // while every wavefront's first weights are in flight, and shares them through LDS.
  accumulate<MT, NTW, U, NORM>(p, A, (size_t)unit, k0, k1, acc, r, q, lane, NORM && wave == 0, [&]() {
    if constexpr (NORM) {
      if (wave == 0 && q == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) srinv[mt * 16 + r] = A.rinv[mt];
      }
      __syncthreads();
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) A.rinv[mt] = srinv[mt * 16 + r];
    }
  });

  // Wavefront partials -> wavefront 0, summed in wavefront order.
  if constexpr (WPG > 1) {
    if (wave > 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) red[(((wave - 1) * MT + mt) * NTW + nt) * 64 + lane] = acc[mt][nt];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt)
        for (int w = 1; w < WPG; ++w) acc[mt][nt] += red[(((w - 1) * MT + mt) * NTW + nt) * 64 + lane];
  }
  if constexpr (PRE_RES) {
    if (KS > 1) finish_split<MT, NTW, EPI, true, 64>(p, acc, unit, ks, KS, lane, res);  // split-K across workgroups
    else epilogue<MT, NTW, EPI>(p, acc, unit, lane, res);
  } else {
    if (KS > 1) finish_split<MT, NTW, EPI>(p, acc, unit, ks, KS, lane);
    else epilogue<MT, NTW, EPI>(p, acc, unit, lane);
  }
}

// Stream-K decomposition: exactly one workgroup per CU (gridDim.x = CU count;
// the LDS reservation keeps a second one off the CU). The units x K/32 weight
// tiles, unit-major, are cut into gridDim.x equal contiguous ranges, so every
// CU streams the same number of bytes; a CU's range is cut again into
// SK_WAVES equal pieces, one per wavefront, each touching at most two units.
// Units that lie entirely inside one CU's range are reduced through LDS (in
// wavefront order) and finished there; a unit shared by several CUs is
// finished by the last of them through finish_split (pieces in CU order), so
// results do not depend on timing.
constexpr int SK_WAVES = 8;
constexpr int SK_PIECES = 4;                 // CUs that may share one unit
constexpr int SK_LDS_BYTES = 96 * 1024;      // more than half of a CU's 160 KB

__device__ __forceinline__ long long sk_begin(long long T, int G, long long c) { return T * c / G; }

// CU whose range holds tile t.
__device__ __forceinline__ long long sk_owner(long long t, long long T, int G) {
  long long c = t * G / T;
  while (c > 0 && sk_begin(T, G, c) > t) --c;
  while (c + 1 < G && sk_begin(T, G, c + 1) <= t) ++c;
  return c;
}

template <int MT, int NTW, bool NORM, int EPI>
__global__ void __launch_bounds__(64 * SK_WAVES) sk_gemm_kernel(GemmParams p) {
  constexpr int U = (MT == 1 ? 8 : 4) / NTW;
  __shared__ f32x4_t red[SK_LDS_BYTES / 16];  // [wave][slot][mt][nt][lane]
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const long long KT = p.K >> 5;
  const long long units = p.N / (16 * NTW);
  const long long T = units * KT;
  const int G = gridDim.x;
  const long long c = blockIdx.x;
  const long long cs = sk_begin(T, G, c), ce = sk_begin(T, G, c + 1);
  auto wave_begin = [&](int w) { return cs + (ce - cs) * w / SK_WAVES; };
  const long long ws = wave_begin(wave), we = wave_begin(wave + 1);

  AOperand<MT, NORM> A;
  A.init(p, r, q);
  const long long u0 = ws / KT;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const long long u = u0 + s;
    const long long lo = max(ws, u * KT), hi = min(we, (u + 1) * KT);
    f32x4_t acc[MT][NTW];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    if (lo < hi) accumulate<MT, NTW, U, NORM>(p, A, (size_t)u, (int)(lo - u * KT), (int)(hi - u * KT), acc, r, q, lane, s == 0,
                                              [] {});
    else if (s == 0) A.stats(p, r, q);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) red[(((wave * 2 + s) * MT + mt) * NTW + nt) * 64 + lane] = acc[mt][nt];
  }
  __syncthreads();

  // Units of this CU: wavefront j reduces units U0 + j, U0 + j + SK_WAVES, ...
  if (ce <= cs) return;
  const long long U0 = cs / KT, U1 = (ce - 1) / KT;
  for (long long u = U0 + wave; u <= U1; u += SK_WAVES) {
    f32x4_t acc[MT][NTW];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int w = 0; w < SK_WAVES; ++w) {
      const long long a = wave_begin(w), b = wave_begin(w + 1);
      if (a >= b || b <= u * KT || a >= (u + 1) * KT) continue;  // wavefront w does not touch unit u
      const int s = (int)(u - a / KT);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] += red[(((w * 2 + s) * MT + mt) * NTW + nt) * 64 + lane];
    }
    if (u * KT >= cs && (u + 1) * KT <= ce) {
      epilogue<MT, NTW, EPI>(p, acc, u, lane);
    } else {
      const long long cf = sk_owner(u * KT, T, G), cl = sk_owner((u + 1) * KT - 1, T, G);
      finish_split<MT, NTW, EPI>(p, acc, u, (int)(c - cf), (int)(cl - cf + 1), lane);
    }
  }
}

// Rectangle decomposition with the A operand staged in LDS (M <= 32 rows).
//
// The (unit, k-step) plane -- units of 16*NTW weight rows, k-steps of 32 -- is
// cut into GN x GK rectangles (gridDim.x = GN*GK, normally the CU count), all
// the same size to within one unit (k-ranges are equal), so every CU streams
// the same weight bytes. Workgroup (gn, gk) stages its k-range of the A operand,
// x[0:M, 32*k0 : 32*k1], in LDS -- with NORM the RMSNorm is applied here, once
// per element -- then its WPG wavefronts stream equal contiguous pieces of the
// rectangle's tiles in unit-major order, reading A fragments from LDS (one
// activation read per workgroup instead of one per wavefront and tile).
//
// Staging is one straight-line round: wavefront w stages rows w and w + WPG
// (each lane up to RECT_CPL 16-byte chunks per row) and, with NORM, derives those
// rows' RMSNorm factors itself from the producer's per-16-column partial sums, so
// no barrier separates statistics and staging. The first weight batches are
// requested once the staged rows are stored (loads return in issue order, so
// earlier weight requests would hold the staging behind HBM). Staged rows hold the
// M real rows plus, when the 16-row tiles have padding rows, one zero row that
// those rows read: 16-byte chunk j of row m sits at chunk j ^ (m % 16) of its row,
// which keeps both the staging writes and the A-fragment reads (16 rows x one
// chunk each) free of bank conflicts.
//
// A piece is at most one unit long (the host checks units per rectangle <= WPG),
// so it touches at most two units: the first unit's sums are parked in registers
// when the second starts, at a tile index every lane of the wavefront knows, so
// the loop has no per-lane selects. Wavefront partials meet in LDS in wavefront order; with
// GK > 1 the GK rectangles of one unit column meet in finish_split (pieces in k
// order).
constexpr int RECT_LDS_MAX = 160 * 1024;
constexpr int RECT_RPW = 2;   // staged rows per wavefront (M <= 2 * WPG)
constexpr int RECT_CPL = 5;   // staged chunks per lane and row (k-range <= 80 k-steps)
constexpr int RECT_PPL = 4;   // RMSNorm partials per lane and row (K <= 4096 with NORM)

template <int MT, int NTW, int WPG, bool NORM, int EPI>
__global__ void __launch_bounds__(64 * WPG) rect_gemm_kernel(GemmParams p, int GN, int GK) {
  constexpr int U = 4 / NTW;  // tiles per batch (4 KB of weights); two batches in flight per wavefront
  extern __shared__ __align__(16) unsigned char rect_smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int NU = p.N / (16 * NTW);
  const int KT = p.K >> 5;
  const int gn = blockIdx.x / GK, gk = blockIdx.x - (blockIdx.x / GK) * GK;
  const int u0 = (int)((long long)NU * gn / GN), u1 = (int)((long long)NU * (gn + 1) / GN);
  const int k0 = (int)((long long)KT * gk / GK), k1 = (int)((long long)KT * (gk + 1) / GK);
  const int kc = k1 - k0, nun = u1 - u0, total = nun * kc;
  const int t0 = (int)((long long)total * wave / WPG), t1 = (int)((long long)total * (wave + 1) / WPG);
  const int rowe = kc * 32;  // bf16 per staged row
  bf16_t* xs = reinterpret_cast<bf16_t*>(rect_smem);

  // The wavefront's piece: n tiles of the (unit, k-step) plane in unit-major order, at most one
  // unit long. Its tiles 0 .. tb - 1 are k-steps kfirst .. of unit ufirst, tiles tb .. n - 1 are
  // k-steps 0 .. of unit ufirst + 1. Every quantity here is wavefront-uniform, so the tile
  // addresses are scalar; an empty piece points at the rectangle's first tile.
  const uint4* wt = reinterpret_cast<const uint4*>(p.w);
  const int n = t1 - t0;
  const int ufirst = n > 0 ? t0 / kc : 0;
  const int kfirst = n > 0 ? t0 - ufirst * kc : 0;
  const int tb = min(n, kc - kfirst);
  const size_t ustride = (size_t)NTW * KT * 64;  // 16-byte pieces per unit of the tiled weight
  const uint4* wA = wt + (size_t)(u0 + ufirst) * ustride + (size_t)(k0 + kfirst) * 64;
  const uint4* wB = wt + (size_t)min(u0 + ufirst + 1, NU - 1) * ustride + (size_t)k0 * 64;
  // Tile t of the piece; a tile at or past n (a partly used last batch) re-reads tile 0.
  auto tile_base = [&](int t) -> const uint4* {
    return t < tb ? wA + (size_t)t * 64 : (t < n ? wB + (size_t)(t - tb) * 64 : wA);
  };
  auto issue = [&](uint4 (&w)[U][NTW], int t) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const uint4* b = tile_base(t + i);
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) w[i][nt] = load_nt(b + (size_t)nt * KT * 64 + lane);
    }
  };

  // Staging loads first (every load unconditional: rows past M and chunks past the row
  // read row 0 / chunk 0 and are dropped), then the first two weight batches.
  const int cpr = kc * 4;  // 16-byte chunks per staged row
  const int nu = p.K >> 4;
  uint4 xv[RECT_RPW][RECT_CPL], gv[RECT_CPL];
  float pv[RECT_RPW][RECT_PPL];
#pragma unroll
  for (int i = 0; i < RECT_RPW; ++i) {
    const int m = wave + i * WPG;
    const size_t row = m < p.M ? (size_t)m : 0;
#pragma unroll
    for (int c = 0; c < RECT_CPL; ++c) {
      const int j = lane + 64 * c;
      xv[i][c] = *reinterpret_cast<const uint4*>(p.x + row * p.K + (size_t)k0 * 32 + (j < cpr ? j : 0) * 8);
    }
    if constexpr (NORM) {
#pragma unroll
      for (int u = 0; u < RECT_PPL; ++u) pv[i][u] = p.psq_in[row * nu + min(lane + 64 * u, nu - 1)];
    }
  }
  if constexpr (NORM) {
    const uint4* nwp = reinterpret_cast<const uint4*>(p.nw);
#pragma unroll
    for (int c = 0; c < RECT_CPL; ++c) {
      const int j = lane + 64 * c;
      gv[c] = nwp[k0 * 4 + (j < cpr ? j : 0)];
    }
  }

  const int nb = (n + U - 1) / U;
  uint4 b0[U][NTW], b1[U][NTW];
  // Normalise and store the staged rows (row m: RMSNorm factor from the K/16 partials,
  // summed lane-strided then by a fixed butterfly: identical in every workgroup). This
  // completes before the first weight batch is requested: loads return in issue order, so
  // a weight prefetch issued earlier holds the staging behind HBM. Measured on MI355X at
  // M = 32 (gate/up): staging done after 11 us with the prefetch first, 8 us with it after,
  // 9.9 us with it issued between the staging loads and the normalisation.
#pragma unroll
  for (int i = 0; i < RECT_RPW; ++i) {
    const int m = wave + i * WPG;
    float rinv = 1.f;
    if constexpr (NORM) {
      float sacc = 0.f;
#pragma unroll
      for (int u = 0; u < RECT_PPL; ++u) sacc += pv[i][u] * (lane + 64 * u < nu ? 1.f : 0.f);  // keeps every load used
      rinv = rms_rinv(wave_sum_dpp(sacc), p.K, p.eps);
    }
    if (m < p.M) {
#pragma unroll
      for (int c = 0; c < RECT_CPL; ++c) {
        const int j = lane + 64 * c;
        if (j < cpr) {
          uint4 v = xv[i][c];
          if constexpr (NORM) {
            float f[8], gg[8], o[8];
            unpack8(v, f);
            unpack8(gv[c], gg);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = mul_rn(gg[e], rbf(mul_rn(f[e], rinv)));
            v = pack8(o);
          }
          *reinterpret_cast<uint4*>(xs + m * rowe + (j ^ (m & 15)) * 8) = v;
        }
      }
    } else if (m == p.M && p.M < 16 * MT) {  // the zero row that A-fragment rows past M read
#pragma unroll
      for (int c = 0; c < RECT_CPL; ++c) {
        const int j = lane + 64 * c;
        if (j < cpr) *reinterpret_cast<uint4*>(xs + m * rowe + j * 8) = make_uint4(0, 0, 0, 0);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the weight requests below the staging
  // Both prologue batches unconditionally (an empty piece re-reads the rectangle's first
  // tile): every path then has the same loads in flight, so the compiler's wait for batch 0
  // leaves batch 1 in flight. They stream while the workgroup meets at the barrier.
  issue(b0, 0);
  issue(b1, U);
  __syncthreads();

  // A-fragment rows of this lane: rows past M read the zero row (row M).
  int abase[MT], asw[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int arow = 16 * mt + r < p.M ? 16 * mt + r : p.M;
    abase[mt] = arow * rowe;
    asw[mt] = arow & 15;
  }

  f32x4_t acc[MT][NTW], saved[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = saved[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Tile t: the unit switch (t == tb: the first unit's sums are parked) and a tile past the
  // piece (t >= n, skipped) are wavefront-uniform branches, so the sums see no selects.
  auto consume = [&](const uint4 (&w)[U][NTW], int t) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int tt = t + i;
      if (tt < n) {
        if (tt == tb) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) {
              saved[mt][nt] = acc[mt][nt];
              acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
        }
        const int kk = tt < tb ? kfirst + tt : tt - tb;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const bf16x8_t a = as_bf16x8(*reinterpret_cast<const uint4*>(xs + abase[mt] + (((kk * 4 + q) ^ asw[mt]) * 8)));
#pragma unroll
          for (int nt = 0; nt < NTW; ++nt)
            acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, as_bf16x8(w[i][nt]), acc[mt][nt], 0, 0, 0);
        }
      }
    }
  };
  int j = 0;
  for (; j + 3 < nb; j += 2) {  // batches j .. j+3 exist
    consume(b0, j * U);
    issue(b0, (j + 2) * U);
    consume(b1, (j + 1) * U);
    issue(b1, (j + 3) * U);
  }
  if (j < nb) consume(b0, j * U);
  if (j + 2 < nb) issue(b0, (j + 2) * U);
  if (j + 1 < nb) consume(b1, (j + 1) * U);
  if (j + 2 < nb) consume(b0, (j + 2) * U);

  // Wavefront partials -> LDS ([wave][slot][mt][nt][lane], aliasing the staged A), then per unit.
  __syncthreads();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(rect_smem);
  if (n > 0) {
    const bool two = tb < n;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) {
        red[(((wave * 2 + 0) * MT + mt) * NTW + nt) * 64 + lane] = two ? saved[mt][nt] : acc[mt][nt];
        if (two) red[(((wave * 2 + 1) * MT + mt) * NTW + nt) * 64 + lane] = acc[mt][nt];
      }
  }
  __syncthreads();
  for (int uu = wave; uu < nun; uu += WPG) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int w = 0; w < WPG; ++w) {
      const int a0 = (int)((long long)total * w / WPG), a1 = (int)((long long)total * (w + 1) / WPG);
      if (a0 >= a1) continue;
      const int wf = a0 / kc, wl = (a1 - 1) / kc;
      if (uu < wf || uu > wl) continue;
      const int slot = uu - wf;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) acc[mt][nt] += red[(((w * 2 + slot) * MT + mt) * NTW + nt) * 64 + lane];
    }
    if (GK > 1) finish_split<MT, NTW, EPI>(p, acc, u0 + uu, gk, GK, lane);
    else epilogue<MT, NTW, EPI>(p, acc, u0 + uu, lane);
  }
}

// token[m] = index held in row m's packed argmax key (the maximum over its slots); the slots
// are re-armed to zero.
__global__ void __launch_bounds__(64) argmax_extract_kernel(unsigned long long* __restrict__ amax, int M,
                                                            int64_t* __restrict__ out) {
  const int m = blockIdx.x * 64 + threadIdx.x;
  if (m >= M) return;
  const unsigned long long key = argmax_key(amax, M, m);
  out[m] = (int64_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
  argmax_rearm(amax, M, m);
}

template <int MT, int NTW, int WPG, bool NORM, int EPI>
hipError_t launch(const GemmParams& p, int grid, hipStream_t stream) {
  skinny_gemm_kernel<MT, NTW, WPG, NORM, EPI><<<grid, 64 * WPG, 0, stream>>>(p);
  return hipGetLastError();
}

template <int MT, int NTW, bool NORM, int EPI>
hipError_t launch_sk(const GemmParams& p, int grid, hipStream_t stream) {
  sk_gemm_kernel<MT, NTW, NORM, EPI><<<grid, 64 * SK_WAVES, 0, stream>>>(p);
  return hipGetLastError();
}

template <bool NORM, int EPI>
int dispatch_sk(const GemmParams& p, int grid, int mt, int ntw, hipStream_t stream) {
  if constexpr (EPI != EPI_SWIGLU) {
    if (mt == 1 && ntw == 1) return qwen_status(launch_sk<1, 1, NORM, EPI>(p, grid, stream));
    if (mt == 2 && ntw == 1) return qwen_status(launch_sk<2, 1, NORM, EPI>(p, grid, stream));
  }
  if (mt == 1 && ntw == 2) return qwen_status(launch_sk<1, 2, NORM, EPI>(p, grid, stream));
  if (mt == 2 && ntw == 2) return qwen_status(launch_sk<2, 2, NORM, EPI>(p, grid, stream));
  return QWEN_EARG;
}

int cu_count() { return device_cu_count(); }

// Stream-K applies when every CU gets at least one tile, a unit spans at most
// SK_PIECES CUs and a wavefront's share touches at most two units.
bool sk_fits(int N, int K, int ntw, int G) {
  if (G <= 0 || (ntw != 1 && ntw != 2)) return false;
  const long long KT = K / 32, units = N / (16 * ntw), T = units * KT;
  const long long lmin = T / G, lmax = (T + G - 1) / G;
  if (lmin < 1) return false;
  if ((KT - 1 + lmin - 1) / lmin + 1 > SK_PIECES) return false;
  return (lmax + SK_WAVES - 1) / SK_WAVES <= KT;
}

// Dispatch over the instantiated (MT, NTW, WPG) launch shapes. Shapes whose
// wavefront-reduction buffer would exceed 60 KB of LDS, or that would spill
// registers, are not built (the call returns QWEN_EARG).
template <bool NORM, int EPI>
int dispatch(const GemmParams& p, int grid, int mt, int ntw, int wpg, hipStream_t stream) {
#define QWEN_GEMM_CASE(MT_, NTW_, W_) \
  if (mt == MT_ && ntw == NTW_ && wpg == W_) return qwen_status(launch<MT_, NTW_, W_, NORM, EPI>(p, grid, stream));
#define QWEN_GEMM_W(MT_, NTW_) QWEN_GEMM_CASE(MT_, NTW_, 4) QWEN_GEMM_CASE(MT_, NTW_, 8)
  if constexpr (EPI != EPI_SWIGLU) {
    QWEN_GEMM_W(1, 1)
    QWEN_GEMM_W(2, 1)
  }
  QWEN_GEMM_W(1, 2)
  QWEN_GEMM_W(2, 2)
  QWEN_GEMM_W(1, 4)
  QWEN_GEMM_W(2, 4)
  QWEN_GEMM_W(1, 8)  // wider units share each activation load over 8 n-tiles
  QWEN_GEMM_W(2, 8)
  if constexpr (!NORM) {  // 16 wavefronts (128 VGPRs each) fit only without the norm prologue
    QWEN_GEMM_CASE(1, 1, 16)
    QWEN_GEMM_CASE(1, 2, 16)
    QWEN_GEMM_CASE(2, 2, 16)
  }
#undef QWEN_GEMM_W
#undef QWEN_GEMM_CASE
  return QWEN_EARG;
}

// Dynamic LDS of a rectangle launch: the M staged rows of a k-range, or the wavefront
// partials that later alias them, whichever is larger.
long long rect_lds_bytes(int M, int K, int ntw, int wpg, int gk) {
  const long long MT = M > 16 ? 2 : 1;
  const long long kc = (K / 32) / gk;
  const long long rows = M < 16 * MT ? M + 1 : M;  // plus the zero row when the tiles have padding rows
  const long long xs = rows * kc * 64;
  const long long red = (long long)wpg * 2 * MT * ntw * 64 * 16;
  return xs > red ? xs : red;
}

// A rectangle launch applies when every rectangle holds at least one unit and at most wpg
// units (a wavefront's piece touches at most two), the k-ranges are equal multiples of four
// k-steps of at most 4 * RECT_CPL * 16 / 4 (one staging round), every row has a staging
// wavefront, NORM rows have at most 64 * RECT_PPL partials, and the LDS fits.
bool rect_fits(int M, int N, int K, int ntw, int wpg, int gn, int gk, bool norm) {
  if (M < 1 || M > 32 || K % 32 != 0 || (ntw != 1 && ntw != 2) || (wpg != 8 && wpg != 16)) return false;
  if (N % (16 * ntw) != 0 || gn < 1 || gk < 1) return false;
  const long long NU = N / (16 * ntw), KT = K / 32;
  if (gn > NU || KT % (4 * gk) != 0) return false;
  const long long kc = KT / gk;
  if (kc * 4 > 64 * RECT_CPL) return false;
  if (M > RECT_RPW * wpg) return false;
  if (norm && K / 16 > 64 * RECT_PPL) return false;
  if ((NU + gn - 1) / gn > wpg) return false;
  if ((long long)gn * gk > 0x7fffffffLL || NU > QWEN_LINEAR_COUNTER_BYTES / 4) return false;
  return rect_lds_bytes(M, K, ntw, wpg, gk) <= RECT_LDS_MAX;
}

template <int MT, int NTW, int WPG, bool NORM, int EPI>
int launch_rect(const GemmParams& p, int gn, int gk, hipStream_t stream) {
  auto kern = rect_gemm_kernel<MT, NTW, WPG, NORM, EPI>;
  static bool attr = false;  // one-time opt-in to more than 64 KB of dynamic LDS
  if (!attr) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, RECT_LDS_MAX) != hipSuccess)
      return QWEN_EARG;
    attr = true;
  }
  const size_t lds = (size_t)rect_lds_bytes(p.M, p.K, NTW, WPG, gk);
  kern<<<gn * gk, 64 * WPG, lds, stream>>>(p, gn, gk);
  QWEN_RETURN_LAUNCH();
}

template <bool NORM, int EPI>
int dispatch_rect(const GemmParams& p, int gn, int gk, int ntw, int wpg, hipStream_t stream) {
  const int mt = p.M > 16 ? 2 : 1;
#define QWEN_RECT_CASE(MT_, NTW_, W_) \
  if (mt == MT_ && ntw == NTW_ && wpg == W_) return launch_rect<MT_, NTW_, W_, NORM, EPI>(p, gn, gk, stream);
  if constexpr (EPI != EPI_SWIGLU) {
    QWEN_RECT_CASE(1, 1, 8)
    QWEN_RECT_CASE(1, 1, 16)
    QWEN_RECT_CASE(2, 1, 8)
    QWEN_RECT_CASE(2, 1, 16)
  } else {
    QWEN_RECT_CASE(1, 2, 8)
    QWEN_RECT_CASE(1, 2, 16)
    QWEN_RECT_CASE(2, 2, 8)
    QWEN_RECT_CASE(2, 2, 16)
  }
#undef QWEN_RECT_CASE
  return QWEN_EARG;
}

int check_shape(const void* x, const void* w, int M, int N, int K, int ntw, int wpg, int ks) {
  if (!x || !w) return QWEN_ENULL;
  if (M <= 0 || M > 32 || N <= 0 || K <= 0 || K % 32 != 0) return QWEN_EARG;
  if (ntw != 1 && ntw != 2 && ntw != 4 && ntw != 8) return QWEN_EARG;
  if (wpg != 4 && wpg != 8 && wpg != 16) return QWEN_EARG;
  if (ntw >= 4 && wpg == 16) return QWEN_EARG;
  if (ks == 0) return (wpg == SK_WAVES && ntw <= 2) ? QWEN_OK : QWEN_EARG;  // stream-K
  if (ks < 1 || ks > 64 || ks * wpg > K / 32) return QWEN_EARG;  // every wavefront owns >= 1 k-step
  if (N % (16 * ntw) != 0) return QWEN_EARG;
  if ((long long)(N / (16 * ntw)) * ks > 0x7fffffffLL) return QWEN_EARG;
  return QWEN_OK;
}

}  // namespace

extern "C" {

long long qwen_linear_workspace_bytes(int M, int N, int ntw, int ks) {
  if (M <= 0 || M > 32 || N <= 0 || (ntw != 1 && ntw != 2 && ntw != 4 && ntw != 8) || ks < 0 ||
      N % (16 * ntw) != 0)
    return 0;
  if (ks == 1) return 0;
  const long long units = N / (16 * ntw);
  const long long mt = M > 16 ? 2 : 1;
  const long long pieces = ks == 0 ? SK_PIECES : ks;  // ks == 0: stream-K
  // A fixed counter region first (so GEMMs of any shape can share one
  // workspace without their partials landing on each other's counters),
  // then the partials.
  return QWEN_LINEAR_COUNTER_BYTES + units * pieces * mt * ntw * 64 * 16;
}

// epi: 0 = store, 1 = residual add (residual may alias out), 2 = SwiGLU pair
// (N counts gate + up rows; out has N/2 columns). norm_w == nullptr: no norm prologue.
int qwen_linear(const void* x, const void* w_tiled, void* out, int M, int N, int K, int ld_out, const void* norm_w,
                const float* psq_in, float eps, const void* residual, float* psq_out, int epi, int ntw, int wpg,
                int ks, void* workspace, long long workspace_bytes, hipStream_t stream) {
  int st = check_shape(x, w_tiled, M, N, K, ntw, wpg, ks);
  if (st) return st;
  if (!out) return QWEN_ENULL;
  if (epi == EPI_RES && !residual) return QWEN_ENULL;
  if (norm_w && !psq_in) return QWEN_ENULL;
  if (psq_out && (epi != EPI_RES || N % 16 != 0)) return QWEN_EARG;
  if (epi == EPI_SWIGLU && ntw < 2) return QWEN_EARG;
  if (epi < EPI_STORE || epi > EPI_SWIGLU) return QWEN_EARG;
  const int out_cols = epi == EPI_SWIGLU ? N / 2 : N;
  if (ld_out < out_cols) return QWEN_EARG;
  const long long need = qwen_linear_workspace_bytes(M, N, ntw, ks);
  if (need > 0 && (!workspace || workspace_bytes < need)) return workspace ? QWEN_EWORKSPACE : QWEN_ENULL;
  const int units = N / (16 * ntw);
  const int mt = M > 16 ? 2 : 1;
  if (units > QWEN_LINEAR_COUNTER_BYTES / 4) return QWEN_EARG;
  const bool split = ks != 1;
  unsigned* cnt = split ? (unsigned*)workspace : nullptr;
  f32x4_t* part = split ? (f32x4_t*)((char*)workspace + QWEN_LINEAR_COUNTER_BYTES) : nullptr;
  GemmParams p{(const bf16_t*)x, (const bf16_t*)w_tiled, (const bf16_t*)norm_w, (const bf16_t*)residual,
               (bf16_t*)out, nullptr, psq_in, psq_out, part, cnt, M, N, K, ld_out, ks, ks == 0 ? SK_PIECES : ks, eps};
  if (ks == 0) {  // stream-K: one workgroup per CU
    const int G = cu_count();
    if (!sk_fits(N, K, ntw, G)) return QWEN_EARG;
    if (epi == EPI_STORE) return norm_w ? dispatch_sk<true, EPI_STORE>(p, G, mt, ntw, stream)
                                        : dispatch_sk<false, EPI_STORE>(p, G, mt, ntw, stream);
    if (epi == EPI_RES) return norm_w ? QWEN_EARG : dispatch_sk<false, EPI_RES>(p, G, mt, ntw, stream);
    return norm_w ? dispatch_sk<true, EPI_SWIGLU>(p, G, mt, ntw, stream) : QWEN_EARG;
  }
  const int grid = units * ks;
  // Instantiated variants: norm+store (QKV), store (plain linear), residual
  // (O / down projections), norm+SwiGLU (gate/up).
  if (epi == EPI_STORE) return norm_w ? dispatch<true, EPI_STORE>(p, grid, mt, ntw, wpg, stream)
                                      : dispatch<false, EPI_STORE>(p, grid, mt, ntw, wpg, stream);
  if (epi == EPI_RES) return norm_w ? QWEN_EARG : dispatch<false, EPI_RES>(p, grid, mt, ntw, wpg, stream);
  return norm_w ? dispatch<true, EPI_SWIGLU>(p, grid, mt, ntw, wpg, stream) : QWEN_EARG;
}

// qwen_linear with the rectangle decomposition: gn x gk workgroups of wpg wavefronts
// (see rect_gemm_kernel). ntw = 2 for the SwiGLU pair epilogue, else 1. The workspace
// (gk > 1) is qwen_linear_workspace_bytes(M, N, ntw, gk) bytes.
int qwen_linear_rect(const void* x, const void* w_tiled, void* out, int M, int N, int K, int ld_out,
                     const void* norm_w, const float* psq_in, float eps, const void* residual, float* psq_out,
                     int epi, int ntw, int wpg, int gn, int gk, void* workspace, long long workspace_bytes,
                     hipStream_t stream) {
  if (!x || !w_tiled || !out) return QWEN_ENULL;
  if (!rect_fits(M, N, K, ntw, wpg, gn, gk, norm_w != nullptr)) return QWEN_EARG;
  if (epi == EPI_RES && !residual) return QWEN_ENULL;
  if (norm_w && !psq_in) return QWEN_ENULL;
  if (psq_out && (epi != EPI_RES || N % 16 != 0)) return QWEN_EARG;
  if (epi < EPI_STORE || epi > EPI_SWIGLU || (epi == EPI_SWIGLU) != (ntw == 2)) return QWEN_EARG;
  const int out_cols = epi == EPI_SWIGLU ? N / 2 : N;
  if (ld_out < out_cols) return QWEN_EARG;
  const long long need = gk > 1 ? qwen_linear_workspace_bytes(M, N, ntw, gk) : 0;
  if (need > 0 && (!workspace || workspace_bytes < need)) return workspace ? QWEN_EWORKSPACE : QWEN_ENULL;
  unsigned* cnt = gk > 1 ? (unsigned*)workspace : nullptr;
  f32x4_t* part = gk > 1 ? (f32x4_t*)((char*)workspace + QWEN_LINEAR_COUNTER_BYTES) : nullptr;
  GemmParams p{(const bf16_t*)x, (const bf16_t*)w_tiled, (const bf16_t*)norm_w, (const bf16_t*)residual,
               (bf16_t*)out, nullptr, psq_in, psq_out, part, cnt, M, N, K, ld_out, gk, gk, eps};
  if (epi == EPI_STORE) return norm_w ? dispatch_rect<true, EPI_STORE>(p, gn, gk, ntw, wpg, stream)
                                      : dispatch_rect<false, EPI_STORE>(p, gn, gk, ntw, wpg, stream);
  if (epi == EPI_RES) return norm_w ? QWEN_EARG : dispatch_rect<false, EPI_RES>(p, gn, gk, ntw, wpg, stream);
  return norm_w ? dispatch_rect<true, EPI_SWIGLU>(p, gn, gk, ntw, wpg, stream) : QWEN_EARG;
}

// Final RMSNorm (norm_w) + LM head GEMM + argmax over the bf16 logits, lowest
// index on ties. amax: [M] packed keys that must be zero before the call (the
// consumer, qwen_argmax_extract or qwen_decode_finish, re-arms them).
// With out_tok != nullptr the tokens are also extracted here (second kernel).
int qwen_lm_head_argmax(const void* x, const void* norm_w, const float* psq_in, float eps, const void* w_tiled, int M,
                        int N, int K, unsigned long long* amax, int64_t* out_tok, int ntw, int wpg,
                        hipStream_t stream) {
  int st = check_shape(x, w_tiled, M, N, K, ntw, wpg, 1);
  if (st) return st;
  if (!amax || !norm_w || !psq_in) return QWEN_ENULL;
  const int units = N / (16 * ntw);
  GemmParams p{(const bf16_t*)x, (const bf16_t*)w_tiled, (const bf16_t*)norm_w, nullptr, nullptr, amax, psq_in,
               nullptr, nullptr, nullptr, M, N, K, 0, 1, 1, eps};
  const int mt = M > 16 ? 2 : 1;
  st = dispatch<true, EPI_ARGMAX>(p, units, mt, ntw, wpg, stream);
  if (st || !out_tok) return st;
  argmax_extract_kernel<<<(M + 63) / 64, 64, 0, stream>>>(amax, M, out_tok);
  QWEN_RETURN_LAUNCH();
}

// out[m] = token index of amax[m]; re-arms amax[m] to zero.
int qwen_argmax_extract(unsigned long long* amax, int M, int64_t* out, hipStream_t stream) {
  if (!amax || !out) return QWEN_ENULL;
  if (M < 0) return QWEN_EARG;
  if (M == 0) return QWEN_OK;
  argmax_extract_kernel<<<(M + 63) / 64, 64, 0, stream>>>(amax, M, out);
  QWEN_RETURN_LAUNCH();
}

}  // extern "C"
