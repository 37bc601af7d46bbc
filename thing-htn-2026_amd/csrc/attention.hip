// GQA flash-decoding over a static KV cache, split-K over the context.
//
// Operator semantics: engine/kernels/attention.py:278-348 and
// engine/kernels/torch_ref.py:168-227. Query t of sequence b sees key j iff
// j < lengths[b] - (T-1-t); query head h reads KV head h / G; fp32 scores
// scaled after the dot; un-normalised probabilities rounded to bf16 for the
// PV product; fp32 row sums; LSE merge across splits; one final bf16 rounding.
//
// Work decomposition (CDNA4, 64-wide wavefronts):
//   grid (B*Nkv, S, T): one single-wavefront workgroup per (sequence, KV head,
//   context split, new query token t), G = 4 query heads per wavefront.
//   Inside a wavefront, lane = 8*slot + c: 8 key slots x 8 lanes per key.
//   Lane c of a slot owns dims [8c, 8c+8) and [64+8c, 64+8c+8), so one key
//   row (256 B) is read by its 8 lanes as 16 B loads and the 8 keys of one
//   load instruction are 2 KB of contiguous cache rows.
//   Each key slot runs its own online softmax over the keys it visits; the
//   8 slots are merged with a log-sum-exp butterfly at the end, and the
//   splits by attn_merge_kernel. A finite sentinel (-1e30) stands in for
//   -inf and invisible keys get p = 0 explicitly, so no inf - inf appears.
#include "common.h"

namespace {

constexpr float NEG_BIG = -1e30f;
constexpr int ATT_D = 128;
constexpr int KU = 2;                     // keys per slot per iteration
constexpr int KEYS_PER_ITER = 8 * KU;     // 8 slots

template <int G>
__global__ void __launch_bounds__(64) attn_partial_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k_cache, const bf16_t* __restrict__ v_cache,
    const int32_t* __restrict__ lengths, int len_add, float* __restrict__ part_ml, float* __restrict__ part_acc, int T,
    int Nkv, int CAP, int S, float scale) {
  const int lane = threadIdx.x;
  const int t = blockIdx.z;
  const int slot = lane >> 3, c = lane & 7;
  const long long bh = blockIdx.x;
  const long long b = bh / Nkv;
  const int kvh = (int)(bh - b * Nkv);
  const int split = blockIdx.y;
  const int Nq = Nkv * G;
  const int R = G * T;

  const int len = min(lengths[b] + len_add, CAP);  // never read past the cache
  int chunk = (len + S - 1) / S;
  chunk = (chunk + KEYS_PER_ITER - 1) / KEYS_PER_ITER * KEYS_PER_ITER;
  const int start = split * chunk;
  const int end = min(start + chunk, len);
  const int kend = min(end, len - (T - 1 - t));

  // q rows of this token: heads kvh*G + g, the lane's 16 dims, in fp32.
  float qf[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const bf16_t* qr = q + (((b * T + t) * Nq) + (long long)kvh * G + g) * ATT_D;
    unpack8(*reinterpret_cast<const uint4*>(qr + 8 * c), qf[g]);
    unpack8(*reinterpret_cast<const uint4*>(qr + 64 + 8 * c), qf[g] + 8);
  }
  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = NEG_BIG;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[g][e] = 0.f;
  }
  const bf16_t* kbase = k_cache + (bh * CAP) * ATT_D;
  const bf16_t* vbase = v_cache + (bh * CAP) * ATT_D;

  for (int base = start; base < kend; base += KEYS_PER_ITER) {
    uint4 kr[KU][2], vr[KU][2];
    bool valid[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int kk = base + u * 8 + slot;  // 8 consecutive keys per load instruction
      valid[u] = kk < kend;
      if (valid[u]) {
        const bf16_t* kp = kbase + (long long)kk * ATT_D;
        const bf16_t* vp = vbase + (long long)kk * ATT_D;
        kr[u][0] = *reinterpret_cast<const uint4*>(kp + 8 * c);
        kr[u][1] = *reinterpret_cast<const uint4*>(kp + 64 + 8 * c);
        vr[u][0] = *reinterpret_cast<const uint4*>(vp + 8 * c);
        vr[u][1] = *reinterpret_cast<const uint4*>(vp + 64 + 8 * c);
      } else {
        kr[u][0] = kr[u][1] = vr[u][0] = vr[u][1] = make_uint4(0, 0, 0, 0);
      }
    }
    float s[KU][G];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      float kf[16];
      unpack8(kr[u][0], kf);
      unpack8(kr[u][1], kf + 8);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) d = fmaf(qf[g][e], kf[e], d);
        d += __shfl_xor(d, 1, 64);
        d += __shfl_xor(d, 2, 64);
        d += __shfl_xor(d, 4, 64);
        s[u][g] = valid[u] ? d * scale : NEG_BIG;
      }
    }
    float vf[KU][16];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      unpack8(vr[u][0], vf[u]);
      unpack8(vr[u][1], vf[u] + 8);
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mn = m[g];
#pragma unroll
      for (int u = 0; u < KU; ++u) mn = fmaxf(mn, s[u][g]);
      const float alpha = __expf(m[g] - mn);
      float p[KU], psum = 0.f;
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        p[u] = valid[u] ? __expf(s[u][g] - mn) : 0.f;
        psum += p[u];
      }
      l[g] = l[g] * alpha + psum;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float a = acc[g][e] * alpha;
#pragma unroll
        for (int u = 0; u < KU; ++u) a = fmaf(rbf(p[u]), vf[u][e], a);
        acc[g][e] = a;
      }
      m[g] = mn;
    }
  }

  // Merge the 8 key slots of the wavefront (lanes differing in bits 3..5).
  const long long prow = (bh * S + split) * R + (long long)t * G;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float mx = m[g];
    mx = fmaxf(mx, __shfl_xor(mx, 8, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float w = __expf(m[g] - mx);
    float lw = l[g] * w;
    lw += __shfl_xor(lw, 8, 64);
    lw += __shfl_xor(lw, 16, 64);
    lw += __shfl_xor(lw, 32, 64);
    float o[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float a = acc[g][e] * w;
      a += __shfl_xor(a, 8, 64);
      a += __shfl_xor(a, 16, 64);
      a += __shfl_xor(a, 32, 64);
      o[e] = a;
    }
    if (slot == 0) {
      float* pa = part_acc + (prow + g) * ATT_D;
      *reinterpret_cast<float4*>(pa + 8 * c) = make_float4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<float4*>(pa + 8 * c + 4) = make_float4(o[4], o[5], o[6], o[7]);
      *reinterpret_cast<float4*>(pa + 64 + 8 * c) = make_float4(o[8], o[9], o[10], o[11]);
      *reinterpret_cast<float4*>(pa + 64 + 8 * c + 4) = make_float4(o[12], o[13], o[14], o[15]);
      if (c == 0) {
        part_ml[(prow + g) * 2] = mx;
        part_ml[(prow + g) * 2 + 1] = lw;
      }
    }
  }
}

// Merge the S split partials of one (b, kvh, row): grid (B*Nkv, G*T), 64 threads.
__global__ void __launch_bounds__(64) attn_merge_kernel(const float* __restrict__ part_ml,
                                                         const float* __restrict__ part_acc, bf16_t* __restrict__ out,
                                                         int T, int Nkv, int G, int S) {
  const int lane = threadIdx.x;
  const long long bh = blockIdx.x;
  const int r = blockIdx.y;
  const int R = G * T;
  const long long b = bh / Nkv;
  const int kvh = (int)(bh - b * Nkv);
  const int t = r / G, g = r - t * G;
  float mx = NEG_BIG;
  for (int s = 0; s < S; ++s) mx = fmaxf(mx, part_ml[((bh * S + s) * R + r) * 2]);
  float L = 0.f, a0 = 0.f, a1 = 0.f;
  for (int s = 0; s < S; ++s) {
    const long long pr = (bh * S + s) * R + r;
    const float w = __expf(part_ml[pr * 2] - mx);
    L += w * part_ml[pr * 2 + 1];
    a0 += w * part_acc[pr * ATT_D + lane];
    a1 += w * part_acc[pr * ATT_D + lane + 64];
  }
  const int Nq = Nkv * G;
  bf16_t* o = out + (((b * T + t) * Nq) + (long long)kvh * G + g) * ATT_D;
  o[lane] = f2bf(a0 / L);
  o[lane + 64] = f2bf(a1 / L);
}

}  // namespace

extern "C" {

long long qwen_attn_workspace_bytes(int B, int T, int Nq, int Nkv, int D, int num_splits) {
  if (B <= 0 || T <= 0 || Nkv <= 0 || Nq % Nkv != 0 || num_splits <= 0) return 0;
  const long long rows = (long long)B * Nkv * num_splits * (Nq / Nkv) * T;
  return rows * (2 + (long long)D) * (long long)sizeof(float);
}

int qwen_attn_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* lengths, int len_add,
                     void* out,
                     void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D, int CAP,
                     float scale, int num_splits, hipStream_t stream) {
  if (!q || !k_cache || !v_cache || !lengths || !out || !workspace) return QWEN_ENULL;
  if (D != ATT_D || Nkv <= 0 || Nq != 4 * Nkv || T <= 0 || T > 16 || B < 0 || CAP <= 0 || num_splits <= 0 ||
      num_splits > 1024)
    return QWEN_EARG;
  if (B == 0) return QWEN_OK;
  const long long need = qwen_attn_workspace_bytes(B, T, Nq, Nkv, D, num_splits);
  if (workspace_bytes < need) return QWEN_EWORKSPACE;
  const long long BH = (long long)B * Nkv;
  if (BH > 0x7fffffffLL) return QWEN_EARG;
  const int G = Nq / Nkv;
  const int R = G * T;
  // acc rows first (512 B each, so every float4 store is aligned), then (m, l) pairs.
  float* part_acc = (float*)workspace;
  float* part_ml = part_acc + BH * num_splits * R * ATT_D;
  attn_partial_kernel<4><<<dim3((unsigned)BH, num_splits, T), 64, 0, stream>>>(
      (const bf16_t*)q, (const bf16_t*)k_cache, (const bf16_t*)v_cache, lengths, len_add, part_ml, part_acc, T, Nkv, CAP,
      num_splits, scale);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return qwen_status(e);
  attn_merge_kernel<<<dim3((unsigned)BH, R), 64, 0, stream>>>(part_ml, part_acc, (bf16_t*)out, T, Nkv, G,
                                                              num_splits);
  QWEN_RETURN_LAUNCH();
}

}  // extern "C"
