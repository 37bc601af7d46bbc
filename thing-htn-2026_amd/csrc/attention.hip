// GQA flash-decoding over a static KV cache, split over the context.
//
// Operator semantics: engine/kernels/attention.py:278-348 and
// engine/kernels/torch_ref.py:168-227. Query t of sequence b sees key j iff
// j < len[b] - (T-1-t); query head h reads KV head h / G; fp32 scores scaled
// after the dot; un-normalised probabilities rounded to bf16 for the PV
// product; fp32 row sums; log-sum-exp merge of partial results; one final
// bf16 rounding.
//
// Two front ends share one kernel:
//   * qwen_attn_decode: the reference's attn_decode operator; q is given and
//     every key comes from the cache (len[b] = lengths[b] + len_add).
//   * qwen_attn_decode_fused: the decode step's QK-norm + RoPE + KV write fused
//     in front of the attention (engine/kernels/rope.py:169-226 semantics with
//     the rounding points of torch_ref.py:94-162). q is normalised and rotated
//     from the raw QKV projection; the T new keys at positions pos..pos+T-1
//     are normalised, rotated and consumed straight from the QKV rows, and the
//     workgroup of the last query writes them (and the raw V) into the cache.
//     No workgroup reads a cache slot that this launch writes.
//
// Work decomposition (CDNA4, 64-wide wavefronts):
//   grid (B*Nkv, S, T): one workgroup per (sequence, KV head, context split,
//   query token t); its WPG wavefronts split the split's keys further. Each
//   wavefront serves the G = 4 query heads of its KV head; lane = 8*slot + c:
//   8 key slots x 8 lanes per key. Lane c of a slot owns dims [8c, 8c+8) and
//   [64+8c, 64+8c+8) (the pairs rotate_half mixes), so one key row (256 B) is
//   read by its 8 lanes as 16 B loads and one load instruction covers 8
//   consecutive cache rows (2 KB). Each key slot runs its own online softmax;
//   slots merge by a log-sum-exp butterfly, wavefronts through LDS in
//   wavefront order, and with S > 1 the splits through the last-arriving
//   workgroup, which reads the partials back in split order (device-coherent
//   sc1 stores/loads, no cache flush). A finite sentinel (-1e30) stands in for
//   -inf and invisible keys get p = 0 explicitly, so no inf - inf appears.
#include "common.h"

namespace {

constexpr float NEG_BIG = -1e30f;
constexpr int ATT_D = 128;
constexpr int G = 4;                       // query heads per KV head
constexpr int KU = 2;                      // keys per slot per iteration
constexpr int KPI = 8 * KU;                // keys per wavefront iteration
constexpr int MERGE_BATCH = 8;             // split partials fetched in one round trip by the last arriver

struct AttnParams {
  const bf16_t* q;          // [B, T, Nq, D] (unfused)
  const bf16_t* qkv;        // [B*T, (Nq+2Nkv)*D] (fused)
  const bf16_t* qnw;        // [D] q_norm gain (fused)
  const bf16_t* knw;        // [D] k_norm gain (fused)
  const bf16_t* cos_tab;    // [P, D] (fused)
  const bf16_t* sin_tab;
  const int32_t* lens;      // unfused: lengths[b]; fused: positions[b]
  bf16_t* kc;               // [B, Nkv, CAP, D]
  bf16_t* vc;
  bf16_t* out;              // [B, T, Nq*D]
  float* part;              // [B*Nkv*T][S][G][2 + D] split partials (S > 1)
  unsigned* cnt;            // [B*Nkv*T] arrival counters, zero between launches (S > 1)
  int T, Nkv, CAP, P, S, len_add;
  float scale, eps;
};

__device__ __forceinline__ void store_dev(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// RMSNorm over one 128-wide head held as 16 values per lane by the 8 lanes of a
// slot (lanes differing in bits 0..2), then RoPE at table row `pos`:
// bf16(bf16(y*cos) + bf16(rot(y)*sin)), rot(y) = cat(-y[64:], y[:64]).
// x[0..7] are dims 8c.., x[8..15] are dims 64+8c... Returns bf16 values in f.
__device__ __forceinline__ void norm_rope_head(float* x, const bf16_t* gain, const bf16_t* cos_tab,
                                               const bf16_t* sin_tab, long long pos, int c, float eps) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) ss = add_rn(ss, mul_rn(x[e], x[e]));
  ss += __shfl_xor(ss, 1, 64);
  ss += __shfl_xor(ss, 2, 64);
  ss += __shfl_xor(ss, 4, 64);
  const float rinv = rms_rinv(ss, ATT_D, eps);
  float g[16], cs[16], sn[16];
  unpack8(*reinterpret_cast<const uint4*>(gain + 8 * c), g);
  unpack8(*reinterpret_cast<const uint4*>(gain + 64 + 8 * c), g + 8);
  unpack8(*reinterpret_cast<const uint4*>(cos_tab + pos * ATT_D + 8 * c), cs);
  unpack8(*reinterpret_cast<const uint4*>(cos_tab + pos * ATT_D + 64 + 8 * c), cs + 8);
  unpack8(*reinterpret_cast<const uint4*>(sin_tab + pos * ATT_D + 8 * c), sn);
  unpack8(*reinterpret_cast<const uint4*>(sin_tab + pos * ATT_D + 64 + 8 * c), sn + 8);
  float y[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) y[e] = rbf(mul_rn(g[e], rbf(mul_rn(x[e], rinv))));
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x[e] = rbf(add_rn(rbf(mul_rn(y[e], cs[e])), rbf(mul_rn(-y[e + 8], sn[e]))));
    x[e + 8] = rbf(add_rn(rbf(mul_rn(y[e + 8], cs[e + 8])), rbf(mul_rn(y[e], sn[e + 8]))));
  }
}

template <int WPG, bool FUSED>
__global__ void __launch_bounds__(64 * WPG) attn_kernel(AttnParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int slot = lane >> 3, c = lane & 7;
  const int t = blockIdx.z;
  const long long bh = blockIdx.x;
  const long long b = bh / p.Nkv;
  const int kvh = (int)(bh - b * p.Nkv);
  const int split = blockIdx.y;
  const int T = p.T;
  const int Nq = p.Nkv * G;
  const int nheads = Nq + 2 * p.Nkv;

  __shared__ float s_ml[WPG][G][2];
  __shared__ float s_acc[WPG][G][ATT_D];

  // Keys [0, len) exist; [newbeg, len) are this launch's new keys (fused only).
  long long pos0 = 0;
  int len, newbeg;
  if constexpr (FUSED) {
    pos0 = p.lens[b];
    len = (int)min((long long)p.CAP, max(0ll, pos0 + T));
    newbeg = (int)min((long long)len, max(0ll, pos0));
  } else {
    len = max(0, min(p.lens[b] + p.len_add, p.CAP));  // never outside [0, CAP)
    newbeg = len;
  }
  const int kend = len - (T - 1 - t);  // keys visible to query t
  int chunk = (len + p.S - 1) / p.S;
  chunk = (chunk + KPI - 1) / KPI * KPI;
  const int start = split * chunk;
  const int end = min(start + chunk, len);
  int wchunk = (chunk + WPG - 1) / WPG;
  wchunk = (wchunk + KPI - 1) / KPI * KPI;
  const int ws = min(end, start + wave * wchunk);
  const int we = min(end, ws + wchunk);

  const bf16_t* kbase = p.kc + (bh * p.CAP) * ATT_D;
  const bf16_t* vbase = p.vc + (bh * p.CAP) * ATT_D;
  const int wend = min(we, kend);  // this wavefront's visible keys [ws, wend)

  // Loads of one block of KPI keys: lane (slot, c) fetches 16 dims of key
  // base + 8u + slot. Keys below newbeg come from the cache, this launch's new
  // keys (fused) straight from the QKV rows (raw K, to be normed and rotated,
  // and raw V); keys past wend re-read key ws and are masked out.
  struct KV {
    uint4 k[KU][2], v[KU][2];
  };
  auto issue = [&](KV& r, int base) {
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int kk = base + u * 8 + slot;
      const long long j = kk < wend ? kk : ws;
      const bf16_t* kp;
      const bf16_t* vp;
      if (FUSED && j >= newbeg) {
        const bf16_t* row = p.qkv + (b * T + (j - pos0)) * nheads * ATT_D;
        kp = row + (long long)(Nq + kvh) * ATT_D;
        vp = row + (long long)(Nq + p.Nkv + kvh) * ATT_D;
      } else {
        kp = kbase + j * ATT_D;
        vp = vbase + j * ATT_D;
      }
      r.k[u][0] = *reinterpret_cast<const uint4*>(kp + 8 * c);
      r.k[u][1] = *reinterpret_cast<const uint4*>(kp + 64 + 8 * c);
      r.v[u][0] = *reinterpret_cast<const uint4*>(vp + 8 * c);
      r.v[u][1] = *reinterpret_cast<const uint4*>(vp + 64 + 8 * c);
    }
  };

  // The first NBUF blocks depend only on the position: they are in flight
  // before the q math starts. Eight-wavefront workgroups keep two blocks in
  // flight per wavefront (their registers are halved), smaller ones three.
  constexpr int NBUF = WPG >= 8 ? 2 : 3;
  KV r0, r1, r2;
  if (ws < wend) issue(r0, ws);
  if (ws + KPI < wend) issue(r1, ws + KPI);
  if constexpr (NBUF == 3) {
    if (ws + 2 * KPI < wend) issue(r2, ws + 2 * KPI);
  }

  // q rows of this token: heads kvh*G + g, the lane's 16 dims, kept as bf16
  // pairs for the v_dot2 score products (exact: the values are bf16).
  uint32_t qp[G][8];
  const long long m_row = b * T + t;
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const bf16_t* qr;
    if constexpr (FUSED) qr = p.qkv + m_row * nheads * ATT_D + (long long)(kvh * G + g) * ATT_D;
    else qr = p.q + ((m_row * Nq) + (long long)kvh * G + g) * ATT_D;
    const uint4 lo = *reinterpret_cast<const uint4*>(qr + 8 * c);
    const uint4 hi = *reinterpret_cast<const uint4*>(qr + 64 + 8 * c);
    if constexpr (FUSED) {
      float x[16];
      unpack8(lo, x);
      unpack8(hi, x + 8);
      const long long qpos = min((long long)p.P - 1, max(0ll, pos0 + t));
      norm_rope_head(x, p.qnw, p.cos_tab, p.sin_tab, qpos, c, p.eps);
      const uint4 a = pack8(x), bb = pack8(x + 8);
      qp[g][0] = a.x; qp[g][1] = a.y; qp[g][2] = a.z; qp[g][3] = a.w;
      qp[g][4] = bb.x; qp[g][5] = bb.y; qp[g][6] = bb.z; qp[g][7] = bb.w;
    } else {
      qp[g][0] = lo.x; qp[g][1] = lo.y; qp[g][2] = lo.z; qp[g][3] = lo.w;
      qp[g][4] = hi.x; qp[g][5] = hi.y; qp[g][6] = hi.z; qp[g][7] = hi.w;
    }
  }

  float m[G], l[G], acc[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = NEG_BIG;
    l[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[g][e] = 0.f;
  }
  const bool writer = FUSED && (t == T - 1);  // the last query's workgroup writes the new K/V

  // Online softmax over one block (KU keys per slot).
  auto consume = [&](KV& r, int base) {
    if constexpr (FUSED) {
      if (base + KPI > newbeg) {  // block holds new keys: norm + rotate them (block-uniform branch)
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const int kk = base + u * 8 + slot;
          const long long j = kk < wend ? kk : ws;
          float kf[16];
          unpack8(r.k[u][0], kf);
          unpack8(r.k[u][1], kf + 8);
          norm_rope_head(kf, p.knw, p.cos_tab, p.sin_tab, min((long long)p.P - 1, j), c, p.eps);
          if (j >= newbeg) {
            r.k[u][0] = pack8(kf);
            r.k[u][1] = pack8(kf + 8);
            if (writer && kk < wend) {
              bf16_t* kd = p.kc + (bh * p.CAP + j) * ATT_D;
              bf16_t* vd = p.vc + (bh * p.CAP + j) * ATT_D;
              *reinterpret_cast<uint4*>(kd + 8 * c) = r.k[u][0];
              *reinterpret_cast<uint4*>(kd + 64 + 8 * c) = r.k[u][1];
              *reinterpret_cast<uint4*>(vd + 8 * c) = r.v[u][0];
              *reinterpret_cast<uint4*>(vd + 64 + 8 * c) = r.v[u][1];
            }
          }
        }
      }
    }
    float s[KU][G];
    bool valid[KU];
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      valid[u] = base + u * 8 + slot < wend;
      const uint32_t kw[8] = {r.k[u][0].x, r.k[u][0].y, r.k[u][0].z, r.k[u][0].w,
                              r.k[u][1].x, r.k[u][1].y, r.k[u][1].z, r.k[u][1].w};
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qp[g][i]),
                                              __builtin_bit_cast(bf16x2_t, kw[i]), d, false);
        d += __shfl_xor(d, 1, 64);
        d += __shfl_xor(d, 2, 64);
        d += __shfl_xor(d, 4, 64);
        s[u][g] = valid[u] ? d * p.scale : NEG_BIG;
      }
    }
    // PV operands: the two keys of a slot paired per dimension, (V0[d], V1[d]) as a bf16x2,
    // so each head's update is one v_dot2_f32_bf16 per dimension (shared by the four heads).
    static_assert(KU == 2, "key pairing assumes two keys per slot");
    uint32_t vp[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t w0 = i < 4 ? (&r.v[0][0].x)[i] : (&r.v[0][1].x)[i - 4];
      const uint32_t w1 = i < 4 ? (&r.v[1][0].x)[i] : (&r.v[1][1].x)[i - 4];
      vp[2 * i] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);      // (V0[2i],   V1[2i])
      vp[2 * i + 1] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);  // (V0[2i+1], V1[2i+1])
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mn = m[g];
#pragma unroll
      for (int u = 0; u < KU; ++u) mn = fmaxf(mn, s[u][g]);
      const float alpha = __expf(m[g] - mn);
      float pb[KU], psum = 0.f;
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const float pr = valid[u] ? __expf(s[u][g] - mn) : 0.f;
        psum += pr;
        pb[u] = rbf(pr);  // P rounded to bf16 for the PV product
      }
      l[g] = l[g] * alpha + psum;
      // alpha is exactly 1 where no slot's running max moved: skip the (exact) no-op rescale
      // when that holds for the whole wavefront.
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[g][e] *= alpha;
      }
      const bf16x2_t pp = __builtin_bit_cast(
          bf16x2_t, (__float_as_uint(pb[0]) >> 16) | (__float_as_uint(pb[1]) & 0xffff0000u));  // exact: bf16 values
#pragma unroll
      for (int e = 0; e < 16; ++e)
        acc[g][e] = __builtin_amdgcn_fdot2_f32_bf16(pp, __builtin_bit_cast(bf16x2_t, vp[e]), acc[g][e], false);
      m[g] = mn;
    }
  };

  // Consume one block, refill its registers with the block NBUF ahead.
  for (int base = ws; base < wend; base += NBUF * KPI) {
    consume(r0, base);
    if (base + NBUF * KPI < wend) issue(r0, base + NBUF * KPI);
    if (base + KPI >= wend) break;
    consume(r1, base + KPI);
    if (base + (NBUF + 1) * KPI < wend) issue(r1, base + (NBUF + 1) * KPI);
    if constexpr (NBUF == 3) {
      if (base + 2 * KPI >= wend) break;
      consume(r2, base + 2 * KPI);
      if (base + 5 * KPI < wend) issue(r2, base + 5 * KPI);
    }
  }

  // Merge the 8 key slots of the wavefront (lanes differing in bits 3..5).
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
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      float a = acc[g][e] * w;
      a += __shfl_xor(a, 8, 64);
      a += __shfl_xor(a, 16, 64);
      a += __shfl_xor(a, 32, 64);
      acc[g][e] = a;
    }
    if (slot == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s_acc[wave][g][8 * c + e] = acc[g][e];
        s_acc[wave][g][64 + 8 * c + e] = acc[g][8 + e];
      }
      if (c == 0) {
        s_ml[wave][g][0] = mx;
        s_ml[wave][g][1] = lw;
      }
    }
  }
  __syncthreads();
  if (wave != 0) return;

  // Wavefront 0 merges the WPG wavefronts in order: lane -> head g = lane/16, dims 8*(lane%16)..+8.
  const int g = lane >> 4;
  const int d0 = (lane & 15) * 8;
  float M = NEG_BIG;
#pragma unroll
  for (int w = 0; w < WPG; ++w) M = fmaxf(M, s_ml[w][g][0]);
  float L = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < WPG; ++w) {
    const float sc = __expf(s_ml[w][g][0] - M);
    L += sc * s_ml[w][g][1];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] += sc * s_acc[w][g][d0 + e];
  }

  const long long row = bh * T + t;  // (b, kvh, t)
  bf16_t* dst = p.out + ((b * T + t) * Nq + (long long)kvh * G + g) * ATT_D + d0;
  if (p.S == 1) {
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = o[e] / L;
    *reinterpret_cast<uint4*>(dst) = pack8(r);
    return;
  }

  // Split partial -> device-coherent store; the last arriving split merges.
  constexpr int PW = 2 + ATT_D;
  float* mine = p.part + ((row * p.S + split) * G + g) * PW;
  if ((lane & 15) == 0) {
    store_dev(mine, M);
    store_dev(mine + 1, L);
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) store_dev(mine + 2 + d0 + e, o[e]);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  unsigned old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(p.cnt + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __shfl(old, 0, 64);
  if (old != (unsigned)(p.S - 1)) return;
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const float* all = p.part + (row * p.S * G + g) * PW;
  float LL = 0.f, oo[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (p.S <= MERGE_BATCH) {
    // Every split's partial requested at once (one round trip), merged in split order.
    float ms[MERGE_BATCH], ls[MERGE_BATCH], os[MERGE_BATCH][8];
#pragma unroll
    for (int s = 0; s < MERGE_BATCH; ++s) {
      const int sl = s < p.S ? s : split;  // slots past S repeat this split's own (ignored below)
      const float* ps = all + (long long)sl * G * PW;
      ms[s] = load_dev(ps);
      ls[s] = load_dev(ps + 1);
#pragma unroll
      for (int e = 0; e < 8; ++e) os[s][e] = load_dev(ps + 2 + d0 + e);
    }
    float MM = NEG_BIG;
#pragma unroll
    for (int s = 0; s < MERGE_BATCH; ++s)
      if (s < p.S) MM = fmaxf(MM, s == split ? M : ms[s]);
#pragma unroll
    for (int s = 0; s < MERGE_BATCH; ++s) {
      if (s < p.S) {
        const bool own = s == split;
        const float sc = __expf((own ? M : ms[s]) - MM);
        LL += sc * (own ? L : ls[s]);
#pragma unroll
        for (int e = 0; e < 8; ++e) oo[e] += sc * (own ? o[e] : os[s][e]);
      }
    }
  } else {
    float MM = NEG_BIG;
    for (int s = 0; s < p.S; ++s) MM = fmaxf(MM, s == split ? M : load_dev(all + (long long)s * G * PW));
    for (int s = 0; s < p.S; ++s) {
      const float* ps = all + (long long)s * G * PW;
      const bool own = s == split;
      const float sc = __expf((own ? M : load_dev(ps)) - MM);
      LL += sc * (own ? L : load_dev(ps + 1));
#pragma unroll
      for (int e = 0; e < 8; ++e) oo[e] += sc * (own ? o[e] : load_dev(ps + 2 + d0 + e));
    }
  }
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = oo[e] / LL;
  *reinterpret_cast<uint4*>(dst) = pack8(r);
  if (lane == 0) __hip_atomic_store(p.cnt + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool FUSED>
int launch_attn(const AttnParams& p, int B, int wpg, hipStream_t stream) {
  const long long BH = (long long)B * p.Nkv;
  dim3 grid((unsigned)BH, p.S, p.T);
  switch (wpg) {
    case 1: attn_kernel<1, FUSED><<<grid, 64, 0, stream>>>(p); break;
    case 2: attn_kernel<2, FUSED><<<grid, 128, 0, stream>>>(p); break;
    case 4: attn_kernel<4, FUSED><<<grid, 256, 0, stream>>>(p); break;
    case 8: attn_kernel<8, FUSED><<<grid, 512, 0, stream>>>(p); break;
    default: return QWEN_EARG;
  }
  QWEN_RETURN_LAUNCH();
}

long long counter_bytes(long long rows) { return (rows * 4 + 255) / 256 * 256; }

int check_attn(int B, int T, int Nq, int Nkv, int D, int CAP, int num_splits, int wpg) {
  if (D != ATT_D || Nkv <= 0 || Nq != G * Nkv || T <= 0 || T > 16 || B < 0 || CAP <= 0 || num_splits <= 0 ||
      num_splits > 1024)
    return QWEN_EARG;
  // up to 8 wavefronts: the kernel needs more than the 128 VGPRs a 16-wavefront workgroup leaves
  if (wpg != 1 && wpg != 2 && wpg != 4 && wpg != 8) return QWEN_EARG;
  if ((long long)B * Nkv > 0x7fffffffLL) return QWEN_EARG;
  return QWEN_OK;
}

}  // namespace

extern "C" {

long long qwen_attn_workspace_bytes(int B, int T, int Nq, int Nkv, int D, int num_splits) {
  if (B <= 0 || T <= 0 || Nkv <= 0 || Nq % Nkv != 0 || num_splits <= 0) return 0;
  if (num_splits == 1) return 0;
  const long long rows = (long long)B * Nkv * T;
  const long long part = rows * num_splits * (Nq / Nkv) * (2 + (long long)D) * (long long)sizeof(float);
  return counter_bytes(rows) + part;  // counters first: their offset does not depend on the split count
}

int qwen_attn_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* lengths, int len_add,
                     void* out, void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D,
                     int CAP, float scale, int num_splits, int wpg, hipStream_t stream) {
  if (!q || !k_cache || !v_cache || !lengths || !out) return QWEN_ENULL;
  int st = check_attn(B, T, Nq, Nkv, D, CAP, num_splits, wpg);
  if (st) return st;
  if (B == 0) return QWEN_OK;
  const long long need = qwen_attn_workspace_bytes(B, T, Nq, Nkv, D, num_splits);
  if (need > 0 && (!workspace || workspace_bytes < need)) return workspace ? QWEN_EWORKSPACE : QWEN_ENULL;
  const long long rows = (long long)B * Nkv * T;
  AttnParams p{};
  p.q = (const bf16_t*)q;
  p.lens = lengths;
  p.kc = (bf16_t*)k_cache;
  p.vc = (bf16_t*)v_cache;
  p.out = (bf16_t*)out;
  p.cnt = num_splits > 1 ? (unsigned*)workspace : nullptr;
  p.part = num_splits > 1 ? (float*)((char*)workspace + counter_bytes(rows)) : nullptr;
  p.T = T; p.Nkv = Nkv; p.CAP = CAP; p.P = 1; p.S = num_splits; p.len_add = len_add;
  p.scale = scale; p.eps = 0.f;
  return launch_attn<false>(p, B, wpg, stream);
}

int qwen_attn_decode_fused(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                           const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                           void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D, int CAP,
                           int P, float eps, float scale, int num_splits, int wpg, hipStream_t stream) {
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !positions || !k_cache || !v_cache || !out)
    return QWEN_ENULL;
  int st = check_attn(B, T, Nq, Nkv, D, CAP, num_splits, wpg);
  if (st) return st;
  if (P <= 0) return QWEN_EARG;
  if (B == 0) return QWEN_OK;
  const long long need = qwen_attn_workspace_bytes(B, T, Nq, Nkv, D, num_splits);
  if (need > 0 && (!workspace || workspace_bytes < need)) return workspace ? QWEN_EWORKSPACE : QWEN_ENULL;
  const long long rows = (long long)B * Nkv * T;
  AttnParams p{};
  p.qkv = (const bf16_t*)qkv;
  p.qnw = (const bf16_t*)q_norm_w;
  p.knw = (const bf16_t*)k_norm_w;
  p.cos_tab = (const bf16_t*)cos_tab;
  p.sin_tab = (const bf16_t*)sin_tab;
  p.lens = positions;
  p.kc = (bf16_t*)k_cache;
  p.vc = (bf16_t*)v_cache;
  p.out = (bf16_t*)out;
  p.cnt = num_splits > 1 ? (unsigned*)workspace : nullptr;
  p.part = num_splits > 1 ? (float*)((char*)workspace + counter_bytes(rows)) : nullptr;
  p.T = T; p.Nkv = Nkv; p.CAP = CAP; p.P = P; p.S = num_splits; p.len_add = 0;
  p.scale = scale; p.eps = eps;
  return launch_attn<true>(p, B, wpg, stream);
}

}  // extern "C"
