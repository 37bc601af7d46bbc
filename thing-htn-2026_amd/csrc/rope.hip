// Per-head QK RMSNorm + RoPE + KV-cache write.
//
// Operator semantics: engine/kernels/rope.py:169-226 and the rounding points of
// engine/kernels/torch_ref.py:94-162 (RMSNorm with the cast before the gain,
// then RoPE with three bf16 roundings: bf16(bf16(y*cos) + bf16(rot(y)*sin)),
// rot(y) = cat(-y[64:], y[:64])).
//
// Eight lanes per (token, head), 32 (token, head) units per 256-thread workgroup, numbered
// u = token * (Nq + 2 Nkv) + head so that unit u's input is the 256 contiguous bytes at
// qkv + u * D. Lane j of a unit owns dims 8j..8j+7 and 64+8j..64+8j+7: the pairs that
// rotate_half combines sit in the same lane, every load and store is 16 bytes wide, and
// the only cross-lane step is the sum of squares over the unit's 8 lanes (DPP, fixed order).
#include "common.h"

namespace {

constexpr int ROPE_LANES = 8;                          // lanes per (token, head)
constexpr int ROPE_UNITS = 256 / ROPE_LANES;           // units per workgroup

__global__ void __launch_bounds__(256) qk_norm_rope_cache_kernel(
    const bf16_t* __restrict__ qkv, const bf16_t* __restrict__ qw, const bf16_t* __restrict__ kw,
    const bf16_t* __restrict__ cos_tab, const bf16_t* __restrict__ sin_tab, const int32_t* __restrict__ positions,
    bf16_t* __restrict__ q_out, bf16_t* __restrict__ k_cache, bf16_t* __restrict__ v_cache,
    long long units, int T, int Nq, int Nkv, int CAP, int P, float eps) {
  constexpr int D = 128;
  const int j = threadIdx.x & (ROPE_LANES - 1);
  const long long u = (long long)blockIdx.x * ROPE_UNITS + (threadIdx.x / ROPE_LANES);
  if (u >= units) return;  // whole 8-lane units leave together
  const int nheads = Nq + 2 * Nkv;
  const long long m = u / nheads;
  const int head = (int)(u - m * nheads);
  const long long b = m / T;
  const long long t = m - b * T;
  const long long pos = (long long)positions[b] + t;
  if (pos < 0 || pos >= CAP || pos >= P) return;  // out-of-range slot: write nothing
  const bf16_t* src = qkv + u * D;
  const uint4 lo = *reinterpret_cast<const uint4*>(src + 8 * j);
  const uint4 hi = *reinterpret_cast<const uint4*>(src + 64 + 8 * j);

  if (head >= Nq + Nkv) {  // V head: raw copy into the cache
    const long long kvh = head - Nq - Nkv;
    bf16_t* dst = v_cache + ((b * Nkv + kvh) * (long long)CAP + pos) * D;
    *reinterpret_cast<uint4*>(dst + 8 * j) = lo;
    *reinterpret_cast<uint4*>(dst + 64 + 8 * j) = hi;
    return;
  }
  float xl[8], xh[8];
  unpack8(lo, xl);
  unpack8(hi, xh);
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) ss = add_rn(ss, add_rn(mul_rn(xl[i], xl[i]), mul_rn(xh[i], xh[i])));
  // Sum over the unit's 8 lanes: quad xor 1, quad xor 2, then the mirrored quad of the
  // 8-lane half row; every lane of the unit ends with the same value.
  ss += dpp_mov_f<0xB1>(ss);
  ss += dpp_mov_f<0x4E>(ss);
  ss += dpp_mov_f<0x141>(ss);
  const float rinv = rms_rinv(ss, D, eps);

  const bf16_t* gain = head < Nq ? qw : kw;
  float gl[8], gh[8], cl[8], ch[8], sl[8], sh[8];
  unpack8(*reinterpret_cast<const uint4*>(gain + 8 * j), gl);
  unpack8(*reinterpret_cast<const uint4*>(gain + 64 + 8 * j), gh);
  const bf16_t* cr = cos_tab + pos * D;
  const bf16_t* sr = sin_tab + pos * D;
  unpack8(*reinterpret_cast<const uint4*>(cr + 8 * j), cl);
  unpack8(*reinterpret_cast<const uint4*>(cr + 64 + 8 * j), ch);
  unpack8(*reinterpret_cast<const uint4*>(sr + 8 * j), sl);
  unpack8(*reinterpret_cast<const uint4*>(sr + 64 + 8 * j), sh);
  float ol[8], oh[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y0 = rbf(mul_rn(gl[i], rbf(mul_rn(xl[i], rinv))));
    const float y1 = rbf(mul_rn(gh[i], rbf(mul_rn(xh[i], rinv))));
    ol[i] = add_rn(rbf(mul_rn(y0, cl[i])), rbf(mul_rn(-y1, sl[i])));
    oh[i] = add_rn(rbf(mul_rn(y1, ch[i])), rbf(mul_rn(y0, sh[i])));
  }
  bf16_t* dst;
  if (head < Nq) {
    dst = q_out + (m * Nq + head) * (long long)D;
  } else {
    const long long kvh = head - Nq;
    dst = k_cache + ((b * Nkv + kvh) * (long long)CAP + pos) * D;
  }
  *reinterpret_cast<uint4*>(dst + 8 * j) = pack8(ol);
  *reinterpret_cast<uint4*>(dst + 64 + 8 * j) = pack8(oh);
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
  // Every tensor is read and written in 16-byte pieces.
  const void* ptrs[] = {qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, q_out, k_cache, v_cache};
  for (const void* p : ptrs)
    if ((uintptr_t)p % 16 != 0) return QWEN_EARG;
  const long long units = (long long)B * T * (Nq + 2 * Nkv);
  const long long blocks = (units + ROPE_UNITS - 1) / ROPE_UNITS;
  if (blocks > 0x7fffffffLL) return QWEN_EARG;
  qk_norm_rope_cache_kernel<<<(unsigned)blocks, ROPE_LANES * ROPE_UNITS, 0, stream>>>(
      (const bf16_t*)qkv, (const bf16_t*)q_norm_w, (const bf16_t*)k_norm_w, (const bf16_t*)cos_tab,
      (const bf16_t*)sin_tab, positions, (bf16_t*)q_out, (bf16_t*)k_cache, (bf16_t*)v_cache, units, T, Nq, Nkv, CAP,
      P, eps);
  QWEN_RETURN_LAUNCH();
}
