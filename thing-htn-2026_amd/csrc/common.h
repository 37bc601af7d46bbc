// Shared device helpers for the Qwen3 decode kernels (gfx950 / CDNA4).
//
// bf16 values travel as raw 16-bit patterns (uint16_t). Conversions are done
// by hand so every rounding point is explicit: widening is exact (<< 16),
// narrowing is IEEE round-to-nearest-even on the fp32 bit pattern.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

#define QWEN_WAVE 64

// Status codes returned by every C-ABI entry point (0 = success). Positive
// values below 1000 are hipError_t codes from the launch.
enum {
  QWEN_OK = 0,
  QWEN_EARG = 1001,      // a size / shape argument is out of the supported range
  QWEN_ENULL = 1002,     // a required pointer is null
  QWEN_EWORKSPACE = 1003, // caller-provided workspace is too small
  QWEN_ESCRATCH = 1004    // the request needs more than an allocation-free entry point's fixed scratch
};

__device__ __forceinline__ float bf2f(bf16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

// fp32 -> bf16, round to nearest, ties to even (IEEE narrowing; on gfx950 the
// compiler emits the hardware v_cvt_pk_bf16_f32, two values per instruction).
__device__ __forceinline__ bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

// Two fp32 -> one dword of two bf16 (low half = a).
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// Packed argmax keys (monotone logit bits << 32 | ~index) of an M-row LM head are spread over
// ARGMAX_SLOTS slots per row: slot s of row m at s * argmax_ld(M) + m, so two slots are at least
// a 128-byte line apart. Workgroup g folds its rows' keys into slot g % ARGMAX_SLOTS, which
// spreads the launch's 64-bit atomicMax operations over ARGMAX_SLOTS addresses per row instead
// of one (same-address atomics serialise: ~25 us of a 194 us LM head at M = 32, measured); the
// consumers take the maximum over the slots and re-arm all of them to zero.
constexpr int ARGMAX_SLOTS = 8;
__host__ __device__ __forceinline__ int argmax_ld(int M) { return (M + 15) / 16 * 16; }
__device__ __forceinline__ unsigned long long argmax_key(const unsigned long long* amax, int M, int m) {
  unsigned long long k = 0;
#pragma unroll
  for (int s = 0; s < ARGMAX_SLOTS; ++s) {
    const unsigned long long v = amax[(long long)s * argmax_ld(M) + m];
    k = v > k ? v : k;
  }
  return k;
}
__device__ __forceinline__ void argmax_rearm(unsigned long long* amax, int M, int m) {
#pragma unroll
  for (int s = 0; s < ARGMAX_SLOTS; ++s) amax[(long long)s * argmax_ld(M) + m] = 0ull;
}

// Round an fp32 value to the nearest bf16 and return it widened again.
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// Product / sum with no contraction into an FMA: the reference rounds each
// square before summing it (and torch's CPU kernels do the same).
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }

// RMSNorm factor rsqrt(mean + eps) of a row of n values whose squares sum to sumsq. The mean
// is the fp32 sum times the fp32 reciprocal of n, as the reference's kernels compute it
// (engine/kernels/rmsnorm.py:87-88 passes inv_n = 1 / n_cols; gemm_fused.py:168 1 / K), not a
// division by n (up to 1 fp32 ulp apart for n = 2560); product and sum rounded one at a time.
__device__ __forceinline__ float rms_rinv(float sumsq, int n, float eps) {
  const float inv_n = __fdiv_rn(1.0f, (float)n);
  return 1.0f / sqrtf(add_rn(mul_rn(sumsq, inv_n), eps));
}

// Unpack 8 bf16 held in a uint4 (little-endian pairs) to fp32.
__device__ __forceinline__ void unpack8(const uint4& v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  return make_uint4(f2bf2(f[0], f[1]), f2bf2(f[2], f[3]), f2bf2(f[4], f[5]), f2bf2(f[6], f[7]));
}

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8_t, v); }

// Wave-wide sum / max with a fixed butterfly order (deterministic).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, QWEN_WAVE);
  return v;
}

// Lane permutations on DPP (VALU; no LDS round trip). The lanes a permutation reads from must
// be active: the row reductions below read across whole 16-lane rows, the 8-lane reduction of
// rope.hip within an 8-lane unit whose lanes return together.
template <int CTRL>
__device__ __forceinline__ float dpp_mov_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
// Sum over the 16 lanes of each DPP row (lanes 16 g .. 16 g + 15); every lane of the row ends
// with the sum. After the two quad steps all lanes of a quad hold the same value, so the
// mirrors add the same operands as lane ^ 4 and lane ^ 8 would: the result equals the xor
// butterfly (1, 2, 4, 8) bit for bit.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov_f<0xB1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_mov_f<0x4E>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_mov_f<0x141>(v);  // row_half_mirror
  v += dpp_mov_f<0x140>(v);  // row_mirror
  return v;
}
// Maximum over the 16 lanes of each DPP row on the same permutations (max is exact, so the
// order does not change the result).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov_f<0xB1>(v));
  v = fmaxf(v, dpp_mov_f<0x4E>(v));
  v = fmaxf(v, dpp_mov_f<0x141>(v));
  v = fmaxf(v, dpp_mov_f<0x140>(v));
  return v;
}
// (largest value, lowest index among equals) over the 16 lanes of each DPP row, on the same
// permutations; every lane of the row ends with the result. The combine is symmetric and
// associative for finite values, so the result does not depend on the order of the steps.
template <int CTRL>
__device__ __forceinline__ void argmax_dpp_step(float& best, int& bidx) {
  const float ov = dpp_mov_f<CTRL>(best);
  const int oi = dpp_mov_i<CTRL>(bidx);
  if (ov > best || (ov == best && oi < bidx)) { best = ov; bidx = oi; }
}
__device__ __forceinline__ void row16_argmax(float& best, int& bidx) {
  argmax_dpp_step<0xB1>(best, bidx);
  argmax_dpp_step<0x4E>(best, bidx);
  argmax_dpp_step<0x141>(best, bidx);
  argmax_dpp_step<0x140>(best, bidx);
}
// Combine lane l with lane l ^ 16 (rows 2g and 2g + 1) or l ^ 32 (the two halves) on the
// gfx950 lane-swap instructions (v_permlane16_swap / v_permlane32_swap: VALU, no LDS round
// trip). Called with the same value twice, the swap leaves the two lanes' values in the two
// results, so their sum (or maximum) equals v + __shfl_xor(v, 16 / 32) bit for bit (the
// addition is commutative). The compiler inserts the instructions' wait states.
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Wave-wide sum without LDS round trips: each 16-lane row is summed by row16_sum, then the
// four row sums are read out and added as (r0 + r1) + (r2 + r3). Fixed order (deterministic);
// the result is uniform across the wavefront.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = row16_sum(v);
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, QWEN_WAVE));
  return v;
}

// Row `id` (clamped into [0, V)) of a tiled [V, K] table -> hrow [K] bf16 and its
// per-16-column sums of squares psq_row [K/16] (the next RMSNorm's statistics).
// Called by a whole workgroup of `nthreads` threads (a multiple of 64).
// Tiled layout: element (n, k) sits in tile (n/16, k/32) at lane 16*((k%32)/8) + n%16.
__device__ __forceinline__ void embed_row_tiled(const bf16_t* __restrict__ w, long long id, long long V, int K,
                                                bf16_t* __restrict__ hrow, float* __restrict__ psq_row, int tid,
                                                int nthreads) {
  id = id < 0 ? 0 : (id >= V ? V - 1 : id);
  const long long KT = K / 32;
  const long long nt = id >> 4;
  const int r = (int)(id & 15);
  const int kc = K / 8;
  for (int c0 = 0; c0 < kc; c0 += nthreads) {
    const int cl = c0 + tid;
    const bool live = cl < kc;
    const int chunk = live ? cl : 0;  // dead lanes redo chunk 0 so the pair shuffle stays uniform
    const int kt = chunk >> 2, q = chunk & 3;
    const uint4 v = reinterpret_cast<const uint4*>(w)[(nt * KT + kt) * 64 + q * 16 + r];
    if (live) reinterpret_cast<uint4*>(hrow)[chunk] = v;
    float f[8], s = 0.f;
    unpack8(v, f);
#pragma unroll
    for (int e = 0; e < 8; ++e) s = add_rn(s, mul_rn(f[e], f[e]));
    s += __shfl_xor(s, 1, 64);
    if (live && (chunk & 1) == 0) psq_row[chunk >> 1] = s;
  }
}

// Device-coherent 16-byte accesses for cross-workgroup hand-offs: raw buffer loads / stores
// with the sc1 cache-policy bit, the same bit relaxed agent-scope atomics use (no cache flush;
// visible to the other XCDs' workgroups once the writer's vmcnt has drained). `off` is a byte
// offset below 2 GiB from `base`.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7ffffffe, 0x00020000);
}
__device__ __forceinline__ f32x4_t load16_dev(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16);
}
__device__ __forceinline__ void store16_dev(__amdgpu_buffer_rsrc_t r, int off, f32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 16);
}
__device__ __forceinline__ float load4_dev(__amdgpu_buffer_rsrc_t r, int off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 16));
}
__device__ __forceinline__ void store4_dev(__amdgpu_buffer_rsrc_t r, int off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 16);
}

static inline int qwen_status(hipError_t e) { return e == hipSuccess ? QWEN_OK : (int)e; }

// Compute units of the current device (cached per device and translation unit; 0 on error).
static inline int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

// Launch-status check used by every entry point: returns the launch error.
#define QWEN_RETURN_LAUNCH() return qwen_status(hipGetLastError())
