// Weight layout and initialisation kernels, and the embedding gather.
//
// A decode projection weight is the HF [N, K] matrix (engine/engine.py:209-227
// fuses q|k|v and gate|up along N) stored in MFMA-B tiles (see gemm.hip):
// tile (nt, kt) = rows 16nt..16nt+15, cols 32kt..32kt+31, 1 KB, lane l = 16q + r
// holding W[16nt + r][32kt + 8q .. +8]. With pair interleave (gate|up), tile
// 2p holds gate rows 16p.. and tile 2p+1 holds up rows 16p.. so the SwiGLU
// epilogue finds both halves in one workgroup.
//
// Random init follows the counter-based generator documented in the oracle
// (oracle/weights.py): element (row, col) of segment s is a function of
// (seed, tid[s], (row - start[s]) * K + col) only, so the tiled device copy
// and a host regeneration hold identical bits.
#include "common.h"

namespace {

struct Segments {
  int start[4];  // first composed row of each segment (ascending), start[0] = 0
  int tid[4];    // generator tensor id of each segment
  int nseg;
};

// Composed row held by tile row r of n-tile nt.
__device__ __forceinline__ long long tiled_row(long long nt, int r, int half_rows, int pair) {
  if (!pair) return nt * 16 + r;
  const long long pidx = nt >> 1;
  return (nt & 1) * (long long)half_rows + pidx * 16 + r;
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ bf16_t gen_elem(uint64_t seed, uint64_t tid, uint64_t idx, float scale) {
  const uint64_t z = splitmix64((seed << 52) | (tid << 32) | idx);
  const int s = (int)(z & 0xffff) + (int)((z >> 16) & 0xffff) + (int)((z >> 32) & 0xffff) + (int)(z >> 48) - 131070;
  return f2bf(mul_rn((float)s, scale));
}

// One thread per 16-byte chunk of the destination.
__global__ void __launch_bounds__(256) init_weight_kernel(bf16_t* __restrict__ dst, long long N, int K, int tiled,
                                                          int pair, Segments seg, uint64_t seed, float scale) {
  const long long c = blockIdx.x * 256ll + threadIdx.x;
  const long long KT = K / 32;
  if (c >= N * (K / 8)) return;
  long long row;
  int col;
  if (tiled) {
    const long long tile = c >> 6;
    const int lane = (int)(c & 63);
    const long long nt = tile / KT, kt = tile - nt * KT;
    row = tiled_row(nt, lane & 15, (int)(N / 2), pair);
    col = (int)(kt * 32 + 8 * (lane >> 4));
  } else {
    row = c / (K / 8);
    col = (int)(c - row * (K / 8)) * 8;
  }
  int s = 0;
  while (s + 1 < seg.nseg && row >= seg.start[s + 1]) ++s;
  const uint64_t base = (uint64_t)(row - seg.start[s]) * (uint64_t)K + (uint64_t)col;
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const bf16_t lo = gen_elem(seed, (uint64_t)seg.tid[s], base + 2 * e, scale);
    const bf16_t hi = gen_elem(seed, (uint64_t)seg.tid[s], base + 2 * e + 1, scale);
    w[e] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  reinterpret_cast<uint4*>(dst)[c] = make_uint4(w[0], w[1], w[2], w[3]);
}

// Row-major [N, K] -> MFMA-B tiles. One thread per destination 16-byte chunk.
__global__ void __launch_bounds__(256) tile_weight_kernel(const bf16_t* __restrict__ src, bf16_t* __restrict__ dst,
                                                          long long N, int K, int pair) {
  const long long c = blockIdx.x * 256ll + threadIdx.x;
  const long long KT = K / 32;
  if (c >= N * (K / 8)) return;
  const long long tile = c >> 6;
  const int lane = (int)(c & 63);
  const long long nt = tile / KT, kt = tile - nt * KT;
  const long long row = tiled_row(nt, lane & 15, (int)(N / 2), pair);
  const long long col = kt * 32 + 8 * (lane >> 4);
  reinterpret_cast<uint4*>(dst)[c] = *reinterpret_cast<const uint4*>(src + row * K + col);
}

// out[m, :] = W[tok[m], :] read from the tiled (tied embedding / LM head) weight.
// tok comes either from tok[m] or, for a decode step, from hist[m, pos[m]].
// With psq != null it also writes the per-16-column sums of squares of each
// row, which the first layer's normed QKV projection reads.
// Ids outside [0, V) are clamped so the gather stays in bounds (the host
// validates prompt ids before they reach the device).
__global__ void __launch_bounds__(256) embed_kernel(const int64_t* __restrict__ tok, const int64_t* __restrict__ hist,
                                                    const int32_t* __restrict__ pos, int cap,
                                                    const bf16_t* __restrict__ w, bf16_t* __restrict__ out,
                                                    float* __restrict__ psq, int M, long long V, int K) {
  const long long c0 = blockIdx.x * 256ll + threadIdx.x;
  const int kc = K / 8;
  const bool live = c0 < (long long)M * kc;
  const long long c = live ? c0 : 0;   // dead lanes redo chunk 0 so the pair shuffle stays uniform
  const int m = (int)(c / kc);
  const int chunk = (int)(c - (long long)m * kc);
  long long id;
  if (tok) {
    id = tok[m];
  } else {
    const int pm = min(max(pos[m], 0), cap - 1);
    id = hist[(long long)m * cap + pm];
  }
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);
  const long long KT = K / 32;
  const long long nt = id >> 4;
  const int r = (int)(id & 15);
  const int kt = chunk >> 2, q = chunk & 3;
  const long long src = ((nt * KT + kt) * 64 + q * 16 + r);
  const uint4 v = reinterpret_cast<const uint4*>(w)[src];
  if (live) reinterpret_cast<uint4*>(out)[c] = v;
  if (psq) {  // partial sums of squares per 16 columns (adjacent lane pairs), for the next RMSNorm
    float f[8], s = 0.f;
    unpack8(v, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) s = add_rn(s, mul_rn(f[e], f[e]));
    s += __shfl_xor(s, 1, 64);
    if (live && (c & 1) == 0) psq[c >> 1] = s;
  }
}

int grid_for(long long chunks, unsigned* blocks) {
  const long long b = (chunks + 255) / 256;
  if (b <= 0 || b > 0x7fffffffLL) return QWEN_EARG;
  *blocks = (unsigned)b;
  return QWEN_OK;
}

}  // namespace

extern "C" {

// Fill dst ([N, K], tiled or row-major) from the counter-based generator.
// seg_start/seg_tid: nseg (1..4) row segments of the composed matrix.
int qwen_init_weight(void* dst, long long N, int K, int tiled, int pair, const int* seg_start, const int* seg_tid,
                     int nseg, unsigned long long seed, float scale, hipStream_t stream) {
  if (!dst || !seg_start || !seg_tid) return QWEN_ENULL;
  if (N <= 0 || K <= 0 || K % 32 != 0 || N % 16 != 0 || nseg < 1 || nseg > 4 || seed >= 4096) return QWEN_EARG;
  if (pair && N % 32 != 0) return QWEN_EARG;
  Segments seg{};
  seg.nseg = nseg;
  for (int i = 0; i < nseg; ++i) {
    seg.start[i] = seg_start[i];
    seg.tid[i] = seg_tid[i];
    if (seg_tid[i] < 0 || seg_tid[i] >= (1 << 20)) return QWEN_EARG;
    if (i > 0 && seg_start[i] <= seg_start[i - 1]) return QWEN_EARG;
  }
  if (seg.start[0] != 0) return QWEN_EARG;
  unsigned blocks;
  if (grid_for(N * (K / 8), &blocks)) return QWEN_EARG;
  init_weight_kernel<<<blocks, 256, 0, stream>>>((bf16_t*)dst, N, K, tiled, pair, seg, seed, scale);
  QWEN_RETURN_LAUNCH();
}

int qwen_tile_weight(const void* src, void* dst, long long N, int K, int pair, hipStream_t stream) {
  if (!src || !dst) return QWEN_ENULL;
  if (N <= 0 || K <= 0 || K % 32 != 0 || N % 16 != 0 || (pair && N % 32 != 0)) return QWEN_EARG;
  unsigned blocks;
  if (grid_for(N * (K / 8), &blocks)) return QWEN_EARG;
  tile_weight_kernel<<<blocks, 256, 0, stream>>>((const bf16_t*)src, (bf16_t*)dst, N, K, pair);
  QWEN_RETURN_LAUNCH();
}

// Embedding gather from the tiled table. Either tok (M ids) or hist/pos
// (token hist[m, pos[m]] of each of M rows, row stride cap) must be given.
int qwen_embed(const int64_t* tok, const int64_t* hist, const int32_t* pos, int cap, const void* w_tiled, void* out,
               float* psq_out, int M, long long V, int K, hipStream_t stream) {
  if (!w_tiled || !out || (!tok && (!hist || !pos))) return QWEN_ENULL;
  if (M < 0 || V <= 0 || V % 16 != 0 || K <= 0 || K % 32 != 0 || (!tok && cap <= 0)) return QWEN_EARG;
  if (M == 0) return QWEN_OK;
  unsigned blocks;
  if (grid_for((long long)M * (K / 8), &blocks)) return QWEN_EARG;
  embed_kernel<<<blocks, 256, 0, stream>>>(tok, hist, pos, cap, (const bf16_t*)w_tiled, (bf16_t*)out, psq_out, M, V,
                                           K);
  QWEN_RETURN_LAUNCH();
}

}  // extern "C"
