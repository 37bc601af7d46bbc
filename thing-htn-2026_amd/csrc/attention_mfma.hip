// The decode step's QK-norm + RoPE + KV write + GQA attention on the matrix cores.
//
// Same operator as qwen_attn_decode_fused (attention.hip): engine/kernels/rope.py:169-226
// followed by engine/kernels/attention.py:278-348, with the rounding points of
// torch_ref.py:94-227 — q and the T new keys are RMS-normed (gain after the bf16 cast),
// rotated with three bf16 roundings; scores are fp32 (q.k) * scale; the un-normalised
// probabilities are rounded to bf16 for the PV product; row sums stay fp32; one final
// bf16 rounding. Query t of a sequence sees key j iff j < pos + t + 1.
//
// Work decomposition (CDNA4): one workgroup per (sequence, KV head, context split) serves
// all R = T * 4 query rows of that KV head (the T query tokens x the 4 query heads), so
// each cache byte is read once for all of them. The grid is (KV head, split, sequence):
// workgroup kvh + Nkv * (split + S * b) runs on XCD kvh mod 8 (with Nkv = 8, head h's
// workgroups share XCD h with the M <= 2 QKV GEMV's workgroups that produce its rows). Its wavefronts split the split's keys
// into blocks of 32. Per block and wavefront:
//   S [16-row tiles x 32 keys] = Q K^T on v_mfma_f32_16x16x32_bf16: the A operand (Q) is
//     staged once in LDS; the B operand (K^T) is loaded straight from the cache, lane
//     (q, r) reading key r's 16 bytes at dims 32kt + 8q (contiguous rows of the cache);
//   online softmax in the accumulator layout (lane (q, r) holds rows 4q..4q+3 of key r);
//   P goes through LDS into the A layout of the PV product;
//   V [32 keys x 128 dims] is written to LDS (288-byte rows) and read back transposed by
//     ds_read_b64_tr_b16: in each 16-lane group, result lane L, element e comes from the
//     address of source lane 4e + L/4, element L%4 (probed on the MI355X), so source lane
//     s pointing at V[key0 + s/4][dim0 + 4(s%4)] yields V[key0 + e][dim0 + L] in lane L;
//   O [rows x 128 dims] += P V on the matrix cores (8 tiles of 16 dims).
// Wavefront results merge by log-sum-exp in LDS, splits through the last-arriving
// workgroup (device-coherent partials, as attention.hip). The new keys are normed,
// rotated and written to the cache by split 0's workgroup and consumed from LDS; no
// workgroup reads a cache slot this launch writes.
#include "common.h"

#include <mutex>
#include <type_traits>

namespace {

constexpr int MD = 128;          // head dim
constexpr int MG = 4;            // query heads per KV head
constexpr int MKB = 32;          // keys per block
constexpr int VROW = 144;        // bf16 per LDS row of V (288 B: 4-way banked transpose reads)
constexpr int MERGE_MAX = 8;     // splits merged in one round trip by the last arriver
constexpr float MNEG = -1e30f;

typedef short mv4i16 __attribute__((ext_vector_type(4)));
typedef unsigned mu32x4 __attribute__((ext_vector_type(4)));  // 16 bytes held as a vector (stays in VGPRs)
typedef __attribute__((address_space(3))) mv4i16 lds_mv4i16;

enum { QWEN_ATTN_KV_CACHED = 1 };  // qwen_attn_decode_mfma_ex flag

struct MfmaAttnParams {
  const bf16_t* qkv;      // [B*T, (Nq+2Nkv)*D]
  const bf16_t* qnw;      // [D]
  const bf16_t* knw;      // [D]
  const bf16_t* cos_tab;  // [P, D]
  const bf16_t* sin_tab;
  const int32_t* pos;     // [B]
  bf16_t* kc;             // [B, Nkv, CAP, D]
  bf16_t* vc;
  bf16_t* out;            // [B, T, Nq*D]
  float* part;            // [B*Nkv][S][MT*16][2 + D] split partials (S > 1)
  unsigned* cnt;          // [B*Nkv] arrival counters (S > 1), zero between launches
  int T, Nkv, CAP, P, S;
  float scale, eps;
  int kv_cached;          // launch the KVC = true kernel (cache-allocating K/V loads)
};

// Device-coherent (sc1) store / load of two adjacent fp32 values as one 64-bit access
// (q 8-byte aligned): half the instructions of per-float accesses on the split hand-off.
__device__ __forceinline__ void mstore2_dev(float* q, float a, float b) {
  const unsigned long long v = ((unsigned long long)__float_as_uint(b) << 32) | __float_as_uint(a);
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(q), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void mload2_dev(const float* q, float& a, float& b) {
  const unsigned long long v =
      __hip_atomic_load(reinterpret_cast<const unsigned long long*>(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  a = __uint_as_float((unsigned)v);
  b = __uint_as_float((unsigned)(v >> 32));
}

// Row reductions (row16_sum, row16_max: 16-lane DPP rows, no LDS round trip) are in common.h.

// One 128-wide head held as dims (c, c + 64) by lane c of a wavefront (x0, x1), with the
// gain (g0, g1) and the cos / sin table entries of its position already loaded: RMSNorm
// (gain after the bf16 cast) and RoPE, bf16(bf16(y cos) + bf16(rot(y) sin)).
__device__ __forceinline__ void mnorm_rope(float& x0, float& x1, float g0, float g1, float c0, float c1, float s0,
                                           float s1, float eps) {
  const float ss = wave_sum_dpp(add_rn(mul_rn(x0, x0), mul_rn(x1, x1)));
  const float rinv = rms_rinv(ss, MD, eps);
  const float y0 = rbf(mul_rn(g0, rbf(mul_rn(x0, rinv))));
  const float y1 = rbf(mul_rn(g1, rbf(mul_rn(x1, rinv))));
  x0 = rbf(add_rn(rbf(mul_rn(y0, c0)), rbf(mul_rn(-y1, s0))));
  x1 = rbf(add_rn(rbf(mul_rn(y1, c1)), rbf(mul_rn(y0, s1))));
}

template <int MT, int WPG>
struct MfmaSmem {
  bf16_t q[MT * 16][MD];                 // normed + rotated queries (rows past R are zero)
  bf16_t knew[MKB][MD];                  // the new keys (rows past T are zero)
  bf16_t vnew[MKB][VROW];                // the new values (rows past T are zero)
  union {
    struct {
      bf16_t v[WPG][MKB][VROW];          // each wavefront's current V block
      bf16_t pm[WPG][MT * 16][MKB];      // each wavefront's P tile
    } blk;
    float merge[WPG][MT * 16][MD + 4];   // per-wavefront O (16-byte aligned), then m, l for the merge
  } u;
  unsigned last;
};

// KVC: cached K / V read with ordinary (cache-allocating) loads instead of non-temporal ones.
template <int MT, int WPG, bool KVC>
__global__ void __launch_bounds__(64 * WPG) __attribute__((amdgpu_waves_per_eu(1, 2)))
attn_mfma_kernel(MfmaAttnParams p) {  // LDS holds one workgroup per CU: at most two wavefronts per SIMD
  __shared__ MfmaSmem<MT, WPG> sm;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qq = lane >> 4, rr = lane & 15;
  // Grid (Nkv, splits, B): the indices come straight from the workgroup id, so the position
  // load needs only the kernel arguments (one memory round trip before it, not two).
  const int kvh = blockIdx.x;
  const int split = blockIdx.y;
  const long long b = blockIdx.z;
  const long long bh = b * p.Nkv + kvh;
  const int T = p.T;
  const int R = T * MG;
  const int Nq = p.Nkv * MG;
  const int nheads = Nq + 2 * p.Nkv;
  const bf16_t* kbase = p.kc + bh * p.CAP * MD;
  const bf16_t* vbase = p.vc + bh * p.CAP * MD;

  // ---- prologue. Every load a wavefront needs is issued first (rows clamped to valid ones,
  // dropped later): the position-free ones, then those that need the position, then its first
  // cached block; then the RMSNorm + RoPE work: one memory round trip after the position's,
  // overlapped with the block's. Query row r (token r / 4, head r % 4) belongs to wavefront
  // r % WPG, new key t to wavefront WPG - 1 - t % WPG.
  constexpr int QPW = (MT * 16 + WPG - 1) / WPG;  // query rows per wavefront
  constexpr int KPW = (8 + WPG - 1) / WPG;        // new keys per wavefront (T <= 8)
  const bf16_t* ct = p.cos_tab;
  const bf16_t* st = p.sin_tab;
  // Prologue values: widened at the load with one query tile; with two they stay raw bf16 until
  // the block's loads are issued behind a scheduling barrier (below), since loads complete in
  // issue order and a gain load the compiler places after the block makes the RMSNorm wait for
  // the whole block (measured: c5 288.8 -> 291.2 verify steps/s; the same order costs c2 0.2 %).
  constexpr bool RAW = MT == 2;
  using PV = std::conditional_t<RAW, bf16_t, float>;
  auto ld = [](bf16_t v) -> PV { if constexpr (RAW) return v; else return bf2f(v); };
  auto fv = [](PV v) -> float { if constexpr (RAW) return bf2f(v); else return v; };
  // First the loads that need no position (this wavefront's q, k and v rows, the gains), so they
  // are in flight while the position arrives; then the table rows and the first cached block.
  PV qx[QPW][2], qcs[QPW][4], kx[KPW][2], kcs[KPW][4];
  bf16_t kv[KPW][2];
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int r = wave + i * WPG;
    const int rc = r < R ? r : 0;
    const int t = rc / MG, g = rc - t * MG;
    const bf16_t* qr = p.qkv + ((b * T + t) * nheads + (long long)(kvh * MG + g)) * MD;
    qx[i][0] = ld(qr[lane]);
    qx[i][1] = ld(qr[lane + 64]);
  }
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    const int t = (WPG - 1 - wave) + j * WPG;
    const int tc = t < T ? t : 0;
    const bf16_t* row = p.qkv + (b * T + tc) * nheads * MD;
    const bf16_t* kr = row + (long long)(Nq + kvh) * MD;
    const bf16_t* vrow = row + (long long)(Nq + p.Nkv + kvh) * MD;
    kx[j][0] = ld(kr[lane]);
    kx[j][1] = ld(kr[lane + 64]);
    kv[j][0] = vrow[lane];
    kv[j][1] = vrow[lane + 64];
  }
  const PV qg0r = ld(p.qnw[lane]), qg1r = ld(p.qnw[lane + 64]);
  const PV kg0r = ld(p.knw[lane]), kg1r = ld(p.knw[lane + 64]);
  __builtin_amdgcn_sched_barrier(0);  // the position is requested after these loads, in flight with them

  const long long pos0 = p.pos[b];
  const int nold = (int)min((long long)p.CAP, max(0ll, pos0));  // cached keys [0, nold)
  auto tab_row = [&](int t) { return min((long long)p.P - 1, max(0ll, pos0 + t)) * MD; };

  // ---- key partition: old keys in blocks of 32 over (split, wavefront); the new-key
  // block goes to the last wavefront of the last split.
  const int nblk = (nold + MKB - 1) / MKB;
  const int per_split = (nblk + p.S - 1) / p.S;
  const int sb0 = min(nblk, split * per_split), sb1 = min(nblk, sb0 + per_split);
  // Blocks are dealt to the wavefronts in turn (wavefront w: blocks sb0 + w, sb0 + w + WPG, ..):
  // the workgroup's K and V requests then form two contiguous streams rather than 2 * WPG.
  constexpr int BSTEP = WPG;
  const int wb0 = sb0 + wave, wb1 = sb1;  // this wavefront: blocks wb0, wb0 + BSTEP, .. < wb1
  const bool takes_new = split == p.S - 1 && wave == WPG - 1;

  // Loads of one cached block: K (B operand: lane (q, r) holds key 16 nt + r, dims 32 kt + 8 q ..)
  // and V rows (lane (q, r) holds key 4 i + q, dims 8 r ..), read with non-temporal loads
  // (each cached byte is read once per step; measured on MI355X: 7.0 vs 6.2 TB/s for a
  // plain streaming read). Keys past the split's range are masked.
  struct KVBlock {
    mu32x4 k[2][4], v[8];
  };
  // Keys at or past this split's range re-read slot 0 (a valid row every lane shares): a
  // wavefront's unconditional first load and its prefetches past its last block then cost no
  // HBM traffic and never touch a neighbouring split's blocks.
  const int kend = min(nold, sb1 * MKB);
  auto load_block = [&](KVBlock& d, int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int key = kb + 16 * nt + rr;
      const mu32x4* kp = reinterpret_cast<const mu32x4*>(kbase + (long long)(key < kend ? key : 0) * MD + 8 * qq);
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        if constexpr (KVC) d.k[nt][kt] = kp[4 * kt];
        else d.k[nt][kt] = __builtin_nontemporal_load(kp + 4 * kt);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = kb + 4 * i + qq;
      const mu32x4* vp = reinterpret_cast<const mu32x4*>(vbase + (long long)(key < kend ? key : 0) * MD + 8 * rr);
      if constexpr (KVC) d.v[i] = *vp;
      else d.v[i] = __builtin_nontemporal_load(vp);
    }
  };
  // Blocks in flight per wavefront: two where the registers allow it without spilling (one
  // 16-row query tile and four wavefronts: 228 VGPRs); otherwise one.
  constexpr int DEPTH = (MT == 1 && WPG == 4) ? 2 : 1;
  KVBlock blkA, blkB;

#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int r = wave + i * WPG;
    const int rc = r < R ? r : 0;
    const long long tr = tab_row(rc / MG);
    qcs[i][0] = ld(ct[tr + lane]);
    qcs[i][1] = ld(ct[tr + lane + 64]);
    qcs[i][2] = ld(st[tr + lane]);
    qcs[i][3] = ld(st[tr + lane + 64]);
  }
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    const int t = (WPG - 1 - wave) + j * WPG;
    const long long tr = tab_row(t < T ? t : 0);
    kcs[j][0] = ld(ct[tr + lane]);
    kcs[j][1] = ld(ct[tr + lane + 64]);
    kcs[j][2] = ld(st[tr + lane]);
    kcs[j][3] = ld(st[tr + lane + 64]);
  }
  if constexpr (RAW) __builtin_amdgcn_sched_barrier(0);
  load_block(blkA, wb0 * MKB);  // unconditional: a wavefront without blocks re-reads valid slots
  if constexpr (DEPTH == 2) load_block(blkB, (wb0 + BSTEP) * MKB);
  if constexpr (RAW) __builtin_amdgcn_sched_barrier(0);
  const float qg0 = fv(qg0r), qg1 = fv(qg1r), kg0 = fv(kg0r), kg1 = fv(kg1r);

  // Rows past R / T are computed too (on clamped inputs) and not stored: every load stays
  // used, so the compiler keeps them ahead of the block loads instead of sinking them into
  // the branches (which would make the first wait also wait for the block).
#pragma unroll
  for (int i = 0; i < QPW; ++i) {
    const int r = wave + i * WPG;
    float x0 = fv(qx[i][0]), x1 = fv(qx[i][1]);
    mnorm_rope(x0, x1, qg0, qg1, fv(qcs[i][0]), fv(qcs[i][1]), fv(qcs[i][2]), fv(qcs[i][3]), p.eps);
    if (r < R) {
      sm.q[r][lane] = f2bf(x0);
      sm.q[r][lane + 64] = f2bf(x1);
    }
  }
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    const int t = (WPG - 1 - wave) + j * WPG;
    float k0 = fv(kx[j][0]), k1 = fv(kx[j][1]);
    mnorm_rope(k0, k1, kg0, kg1, fv(kcs[j][0]), fv(kcs[j][1]), fv(kcs[j][2]), fv(kcs[j][3]), p.eps);
    if (t < T) {
      const long long slot = pos0 + t;
      if (split == 0 && slot >= 0 && slot < p.CAP) {  // one workgroup per (sequence, KV head) writes the cache
        bf16_t* kd = p.kc + (bh * p.CAP + slot) * MD;
        bf16_t* vd = p.vc + (bh * p.CAP + slot) * MD;
        kd[lane] = f2bf(k0);
        kd[lane + 64] = f2bf(k1);
        vd[lane] = kv[j][0];
        vd[lane + 64] = kv[j][1];
      }
      sm.knew[t][lane] = f2bf(k0);
      sm.knew[t][lane + 64] = f2bf(k1);
      sm.vnew[t][lane] = kv[j][0];
      sm.vnew[t][lane + 64] = kv[j][1];
    }
  }
  // Zero rows: query rows R .. 16 MT - 1 and new-key rows T .. 31 (16-byte stores).
  {
    const int zq = (MT * 16 - R) * (MD / 8), zk = (MKB - T) * (MD / 8);
    for (int z = threadIdx.x; z < zq + 2 * zk; z += 64 * WPG) {
      bf16_t* dst;
      if (z < zq) {
        dst = &sm.q[R + z / (MD / 8)][8 * (z % (MD / 8))];
      } else if (z < zq + zk) {
        const int y = z - zq;
        dst = &sm.knew[T + y / (MD / 8)][8 * (y % (MD / 8))];
      } else {
        const int y = z - zq - zk;
        dst = &sm.vnew[T + y / (MD / 8)][8 * (y % (MD / 8))];
      }
      *reinterpret_cast<uint4*>(dst) = make_uint4(0, 0, 0, 0);
    }
  }
  __syncthreads();

  // Q A-operand fragments: lane (q, r) holds Q[16 mt + r][32 kt + 8 q .. +8].
  bf16x8_t qa[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
      qa[mt][kt] = as_bf16x8(*reinterpret_cast<const uint4*>(&sm.q[mt * 16 + rr][32 * kt + 8 * qq]));

  float m[MT][4], l[MT][4];
  f32x4_t o[MT][8];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) { m[mt][i] = MNEG; l[mt][i] = 0.f; }
#pragma unroll
    for (int nd = 0; nd < 8; ++nd) o[mt][nd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  bf16_t* vl = &sm.u.blk.v[wave][0][0];
  bf16_t* pl = &sm.u.blk.pm[wave][0][0];

  // One block: S = Q K^T, online softmax, O = O * alpha + P V. `vsrc` holds the block's V
  // rows in LDS (VROW stride); `visible(nt, row)` masks keys.
  // Split in two so that a block's registers can take the next block's loads as soon as its
  // scores are computed: scores() reads K, finish() only the scores and the V rows in LDS.
  auto scores = [&](const mu32x4 (&kf)[2][4], f32x4_t (&s)[MT][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        s[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kt = 0; kt < 4; ++kt)
          s[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[mt][kt], __builtin_bit_cast(bf16x8_t, kf[nt][kt]), s[mt][nt], 0, 0, 0);
      }
  };
  auto finish = [&](f32x4_t (&s)[MT][2], const bf16_t* vsrc, auto&& visible) __attribute__((always_inline)) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float alpha[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = mt * 16 + 4 * qq + i;
        float sv[2];
        bool vis[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          vis[nt] = visible(nt, row);
          sv[nt] = vis[nt] ? s[mt][nt][i] * p.scale : MNEG;
        }
        const float mx = row16_max(fmaxf(sv[0], sv[1]));
        const float mn = fmaxf(m[mt][i], mx);
        alpha[i] = __expf(m[mt][i] - mn);
        float psum = 0.f;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const float pr = vis[nt] ? __expf(sv[nt] - mn) : 0.f;
          psum += pr;
          pl[(mt * 16 + 4 * qq + i) * MKB + 16 * nt + rr] = f2bf(pr);  // P rounded to bf16 for PV
        }
        l[mt][i] = l[mt][i] * alpha[i] + psum;
        m[mt][i] = mn;
      }
      if (__any(alpha[0] != 1.f || alpha[1] != 1.f || alpha[2] != 1.f || alpha[3] != 1.f)) {
#pragma unroll
        for (int nd = 0; nd < 8; ++nd)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[mt][nd][i] *= alpha[i];
      }
    }
    // P in the A layout: lane (q, r) takes P[16 mt + r][8 q .. +8]. The LDS round trip stays
    // within the wavefront (LDS instructions complete in issue order); the signal fence keeps
    // the compiler from moving these reads above the other lanes' writes.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    bf16x8_t pa[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) pa[mt] = as_bf16x8(*reinterpret_cast<const uint4*>(pl + (mt * 16 + rr) * MKB + 8 * qq));
    // V^T B operand by transpose reads: source lane s -> V[8q + s/4 (+4)][16 nd + 4 (s%4)].
    const bf16_t* vs = vsrc + (8 * qq + (rr >> 2)) * VROW + 4 * (rr & 3);
#pragma unroll
    for (int nd = 0; nd < 8; ++nd) {
      const mv4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_mv4i16*)(vs + 16 * nd));
      const mv4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_mv4i16*)(vs + 4 * VROW + 16 * nd));
      const uint4 vv = make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                  __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        o[mt][nd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[mt], as_bf16x8(vv), o[mt][nd], 0, 0, 0);
    }
  };
  auto process = [&](const mu32x4 (&kf)[2][4], const bf16_t* vsrc, auto&& visible) __attribute__((always_inline)) {
    f32x4_t s[MT][2];
    scores(kf, s);
    finish(s, vsrc, visible);
  };

  // One cached block: its V rows to this wavefront's LDS tile, then S / softmax / PV.
  auto run_block = [&](const KVBlock& d, int blk) __attribute__((always_inline)) {
    const int kb = blk * MKB;
    __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the previous block's transpose reads come first
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<mu32x4*>(vl + (4 * i + qq) * VROW + 8 * rr) = d.v[i];
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    process(d.k, vl, [&](int nt, int row) { return kb + 16 * nt + rr < nold && row < R; });
  };
  // The T new keys, from LDS (query row r, token r / 4, sees new key j iff j <= r / 4). With
  // one query tile and one block in flight their block runs first, in registers of its own,
  // while the wavefront's first cached block is still on its way from HBM; otherwise (no
  // registers to spare) it runs after the cached blocks, in theirs.
  auto run_new = [&](mu32x4 (&kf)[2][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
        kf[nt][kt] = *reinterpret_cast<const mu32x4*>(&sm.knew[16 * nt + rr][32 * kt + 8 * qq]);
    process(kf, &sm.vnew[0][0], [&](int nt, int row) {
      const int j = 16 * nt + rr;
      return j < T && row < R && j <= row / MG;
    });
  };
  constexpr bool NEW_FIRST = MT == 1 && DEPTH == 1;
  if constexpr (NEW_FIRST) {
    if (takes_new) {
      mu32x4 kn[2][4];
      run_new(kn);
    }
  }
  if constexpr (DEPTH == 2) {
    // Two blocks in flight: every load is unconditional (past the range: slot 0), so the
    // compiler's wait for one block leaves the other in flight.
    int blk = wb0;
    for (; blk + BSTEP < wb1; blk += 2 * BSTEP) {
      run_block(blkA, blk);
      load_block(blkA, (blk + 2 * BSTEP) * MKB);
      run_block(blkB, blk + BSTEP);
      load_block(blkB, (blk + 3 * BSTEP) * MKB);
    }
    if (blk < wb1) run_block(blkA, blk);
  } else {
    // One block in flight: the next block's loads go out once this block's V rows are in LDS
    // and its scores are computed (its registers are then free), ahead of the softmax and PV.
    for (int blk = wb0; blk < wb1; blk += BSTEP) {
      const int kb = blk * MKB;
      __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the previous block's transpose reads come first
#pragma unroll
      for (int i = 0; i < 8; ++i) *reinterpret_cast<mu32x4*>(vl + (4 * i + qq) * VROW + 8 * rr) = blkA.v[i];
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      f32x4_t s[MT][2];
      scores(blkA.k, s);
      if (blk + BSTEP < wb1) load_block(blkA, (blk + BSTEP) * MKB);
      finish(s, vl, [&](int nt, int row) { return kb + 16 * nt + rr < nold && row < R; });
    }
  }
  if constexpr (!NEW_FIRST) {
    if (takes_new) run_new(blkA.k);
  }

  // ---- merge: row sums over the 16 lanes of a group, then wavefronts in order through LDS
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      l[mt][i] = row16_sum(l[mt][i]);
    }
  __syncthreads();  // every wavefront is done with its V / P tiles (the merge area aliases them)
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = mt * 16 + 4 * qq + i;
      if (row < R) {  // padding rows of the tile are never read back
        float* mrow = sm.u.merge[wave][row];
        if (rr == 0) {
          mrow[MD] = m[mt][i];
          mrow[MD + 1] = l[mt][i];
        }
#pragma unroll
        for (int nd = 0; nd < 8; ++nd) mrow[16 * nd + rr] = o[mt][nd][i];
      }
    }
  __syncthreads();

  constexpr int NT = 64 * WPG;
  // Thread -> (row, 8-dim chunk) items of the R x 128 result; with at most NT elements (T = 1),
  // one element per thread, so the whole workgroup shares the combine instead of one wavefront
  // doing 8 elements per lane (the same operations in the same order per element: the results
  // are bit-identical).
  const int items = R * (MD / 8);
  const bool per_elem = R * MD <= NT;
  // Split partial of (bh, split): O [16 MT][MD] fp32 (16-byte aligned rows), then (m, l) per row.
  constexpr int PO = MT * 16 * MD, PSTRIDE = MT * 16 * (2 + MD);
  float* mine = p.part + (bh * p.S + split) * PSTRIDE;
  const __amdgpu_buffer_rsrc_t prs = coherent_rsrc(p.part + bh * p.S * PSTRIDE);
  if (per_elem) {
    const int it = threadIdx.x;
    if (it < R * MD) {
      const int row = it / MD, d = it - row * MD;
      f32x2_t ml[WPG];
      float ov[WPG];
#pragma unroll
      for (int w = 0; w < WPG; ++w) {
        const float* mrow = sm.u.merge[w][row];
        ml[w] = *reinterpret_cast<const f32x2_t*>(mrow + MD);
        ov[w] = mrow[d];
      }
      float M = MNEG;
#pragma unroll
      for (int w = 0; w < WPG; ++w) M = fmaxf(M, ml[w].x);
      float L = 0.f, acc = 0.f;
#pragma unroll
      for (int w = 0; w < WPG; ++w) {
        const float sc = __expf(ml[w].x - M);
        L += sc * ml[w].y;
        acc += sc * ov[w];
      }
      if (p.S == 1) {
        const int t = row / MG, g = row - t * MG;
        p.out[((b * T + t) * Nq + (long long)kvh * MG + g) * MD + d] = f2bf(acc / L);
      } else {
        if (d == 0) mstore2_dev(mine + PO + 2 * row, M, L);
        store4_dev(prs, (split * PSTRIDE + row * MD + d) * 4, acc);
      }
    }
  }
  for (int it = per_elem ? items : threadIdx.x; it < items; it += NT) {
    const int row = it / (MD / 8), d0 = (it - row * (MD / 8)) * 8;
    // every wavefront's (m, l) and 8 values requested at once (16-byte reads), then combined
    // in wavefront order
    f32x2_t ml[WPG];
    f32x4_t oa[WPG], ob[WPG];
#pragma unroll
    for (int w = 0; w < WPG; ++w) {
      const float* mrow = sm.u.merge[w][row];
      ml[w] = *reinterpret_cast<const f32x2_t*>(mrow + MD);
      oa[w] = *reinterpret_cast<const f32x4_t*>(mrow + d0);
      ob[w] = *reinterpret_cast<const f32x4_t*>(mrow + d0 + 4);
    }
    float M = MNEG;
#pragma unroll
    for (int w = 0; w < WPG; ++w) M = fmaxf(M, ml[w].x);
    float L = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < WPG; ++w) {
      const float sc = __expf(ml[w].x - M);
      L += sc * ml[w].y;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[e] += sc * oa[w][e];
        acc[e + 4] += sc * ob[w][e];
      }
    }
    if (p.S == 1) {
      const int t = row / MG, g = row - t * MG;
      float r8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) r8[e] = acc[e] / L;
      *reinterpret_cast<uint4*>(p.out + ((b * T + t) * Nq + (long long)kvh * MG + g) * MD + d0) = pack8(r8);
    } else {
      if (d0 == 0) mstore2_dev(mine + PO + 2 * row, M, L);
      const int ob = (split * PSTRIDE + row * MD + d0) * 4;
      store16_dev(prs, ob, f32x4_t{acc[0], acc[1], acc[2], acc[3]});
      store16_dev(prs, ob + 16, f32x4_t{acc[4], acc[5], acc[6], acc[7]});
    }
  }
  if (p.S == 1) return;

  // ---- splits: the last-arriving workgroup merges them in split order
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(p.cnt + bh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sm.last = old == (unsigned)(p.S - 1);
  }
  __syncthreads();
  if (!sm.last) return;
  const float* all = p.part + bh * p.S * PSTRIDE;
  if (per_elem) {
    const int it = threadIdx.x;
    if (it < R * MD) {
      const int row = it / MD, d = it - row * MD;
      // every split's (m, l) and value requested at once, merged in split order
      float ms[MERGE_MAX], ls[MERGE_MAX], os[MERGE_MAX];
#pragma unroll
      for (int j = 0; j < MERGE_MAX; ++j) {
        const int js = min(j, p.S - 1);
        mload2_dev(all + js * PSTRIDE + PO + 2 * row, ms[j], ls[j]);
        os[j] = load4_dev(prs, (js * PSTRIDE + row * MD + d) * 4);
      }
      float MM = MNEG;
#pragma unroll
      for (int j = 0; j < MERGE_MAX; ++j)
        if (j < p.S) MM = fmaxf(MM, ms[j]);
      float LL = 0.f, oo = 0.f;
#pragma unroll
      for (int j = 0; j < MERGE_MAX; ++j) {
        if (j < p.S) {
          const float sc = __expf(ms[j] - MM);
          LL += sc * ls[j];
          oo += sc * os[j];
        }
      }
      const int t = row / MG, g = row - t * MG;
      p.out[((b * T + t) * Nq + (long long)kvh * MG + g) * MD + d] = f2bf(oo / LL);
    }
  }
  for (int it = per_elem ? items : threadIdx.x; it < items; it += NT) {
    const int row = it / (MD / 8), d0 = (it - row * (MD / 8)) * 8;
    // every split's partial requested at once (S <= MERGE_MAX), merged in split order
    float ms[MERGE_MAX], ls[MERGE_MAX], os[MERGE_MAX][8];
#pragma unroll
    for (int j = 0; j < MERGE_MAX; ++j) {
      const int js = min(j, p.S - 1);
      mload2_dev(all + js * PSTRIDE + PO + 2 * row, ms[j], ls[j]);
      const int ob = (js * PSTRIDE + row * MD + d0) * 4;
      const f32x4_t lo = load16_dev(prs, ob), hi = load16_dev(prs, ob + 16);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        os[j][e] = lo[e];
        os[j][e + 4] = hi[e];
      }
    }
    float MM = MNEG;
#pragma unroll
    for (int j = 0; j < MERGE_MAX; ++j)
      if (j < p.S) MM = fmaxf(MM, ms[j]);
    float LL = 0.f, oo[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < MERGE_MAX; ++j) {
      if (j < p.S) {
        const float sc = __expf(ms[j] - MM);
        LL += sc * ls[j];
#pragma unroll
        for (int e = 0; e < 8; ++e) oo[e] += sc * os[j][e];
      }
    }
    const int t = row / MG, g = row - t * MG;
    float r8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) r8[e] = oo[e] / LL;
    *reinterpret_cast<uint4*>(p.out + ((b * T + t) * Nq + (long long)kvh * MG + g) * MD + d0) = pack8(r8);
  }
  if (threadIdx.x == 0) __hip_atomic_store(p.cnt + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

namespace {

long long mfma_counter_bytes(long long rows) { return (rows * 4 + 255) / 256 * 256; }

int mfma_rows(int T) { return T <= 4 ? 16 : 32; }

template <int MT>
int launch_mfma(const MfmaAttnParams& p, int B, int waves, hipStream_t stream) {
  dim3 grid((unsigned)p.Nkv, (unsigned)p.S, (unsigned)B);  // (KV head, split, sequence)
  if (waves == 4) {
    if (p.kv_cached) attn_mfma_kernel<MT, 4, true><<<grid, 256, 0, stream>>>(p);
    else attn_mfma_kernel<MT, 4, false><<<grid, 256, 0, stream>>>(p);
  } else if (waves == 8) {
    if (p.kv_cached) attn_mfma_kernel<MT, 8, true><<<grid, 512, 0, stream>>>(p);
    else attn_mfma_kernel<MT, 8, false><<<grid, 512, 0, stream>>>(p);
  } else {
    return QWEN_EARG;
  }
  QWEN_RETURN_LAUNCH();
}

// ---- the allocation-free variant's scratch: one array per GPU, for the split partials and
// arrival counters that qwen_attn_decode_mfma keeps in its caller's workspace. Host code never
// passes `scratch` itself to a kernel (in host code it names a host-side stand-in); it looks up
// each device's address once with hipGetSymbolAddress and uses that.
constexpr long long NOALLOC_SCRATCH_BYTES = 8ll << 20;   // QWEN_ATTN_NOALLOC_SCRATCH_BYTES
__device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[MAX_DEVICES] = {};

// The current device's address of `scratch` (looked up on its first use there), or null.
void* device_scratch(int* status) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { *status = (int)e; return nullptr; }
  if (dev < 0 || dev >= MAX_DEVICES) { *status = QWEN_EARG; return nullptr; }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) { *status = e != hipSuccess ? (int)e : QWEN_ENULL; return nullptr; }
    g_scratch_ptr[dev] = ptr;
  }
  *status = QWEN_OK;
  return g_scratch_ptr[dev];
}

// Zero `n` 32-bit words (the arrival counters) with a kernel rather than hipMemsetAsync, so a
// caller may record the call into a HIP graph.
__global__ void __launch_bounds__(256) zero_words_kernel(unsigned* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Argument checks shared by qwen_attn_decode_mfma_ex and the allocation-free variant (everything
// but the workspace), so that a refused call has launched nothing.
int mfma_args_status(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                     const void* sin_tab, const int32_t* positions, const void* k_cache, const void* v_cache,
                     const void* out, int B, int T, int Nq, int Nkv, int D, int CAP, int P, int num_splits, int waves,
                     int flags) {
  if (flags & ~QWEN_ATTN_KV_CACHED) return QWEN_EARG;
  if (!qkv || !q_norm_w || !k_norm_w || !cos_tab || !sin_tab || !positions || !k_cache || !v_cache || !out)
    return QWEN_ENULL;
  if (D != MD || Nkv <= 0 || Nq != MG * Nkv || T < 1 || T > 8 || B < 0 || CAP <= 0 || P <= 0) return QWEN_EARG;
  if (num_splits < 1 || num_splits > MERGE_MAX || (waves != 4 && waves != 8)) return QWEN_EARG;
  if ((long long)B * Nkv > 0x7fffffffLL || B > 65535) return QWEN_EARG;  // B is the grid's z extent
  return QWEN_OK;
}

}  // namespace

extern "C" {

long long qwen_attn_mfma_workspace_bytes(int B, int T, int Nkv, int num_splits) {
  if (B <= 0 || T < 1 || T > 8 || Nkv <= 0 || num_splits < 1 || num_splits > MERGE_MAX) return 0;
  if (num_splits == 1) return 0;
  const long long bh = (long long)B * Nkv;
  return mfma_counter_bytes(bh) + bh * num_splits * mfma_rows(T) * (2 + MD) * (long long)sizeof(float);
}

int qwen_attn_decode_mfma_ex(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                             const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                             void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D,
                             int CAP, int P, float eps, float scale, int num_splits, int waves, int flags,
                             hipStream_t stream) {
  const int st = mfma_args_status(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out, B, T,
                                  Nq, Nkv, D, CAP, P, num_splits, waves, flags);
  if (st != QWEN_OK) return st;
  if (B == 0) return QWEN_OK;
  const long long need = qwen_attn_mfma_workspace_bytes(B, T, Nkv, num_splits);
  if (need > 0 && (!workspace || workspace_bytes < need)) return workspace ? QWEN_EWORKSPACE : QWEN_ENULL;
  MfmaAttnParams p{};
  p.qkv = (const bf16_t*)qkv;
  p.qnw = (const bf16_t*)q_norm_w;
  p.knw = (const bf16_t*)k_norm_w;
  p.cos_tab = (const bf16_t*)cos_tab;
  p.sin_tab = (const bf16_t*)sin_tab;
  p.pos = positions;
  p.kc = (bf16_t*)k_cache;
  p.vc = (bf16_t*)v_cache;
  p.out = (bf16_t*)out;
  const long long bh = (long long)B * Nkv;
  p.cnt = num_splits > 1 ? (unsigned*)workspace : nullptr;
  p.part = num_splits > 1 ? (float*)((char*)workspace + mfma_counter_bytes(bh)) : nullptr;
  p.T = T; p.Nkv = Nkv; p.CAP = CAP; p.P = P; p.S = num_splits;
  p.scale = scale; p.eps = eps;
  p.kv_cached = (flags & QWEN_ATTN_KV_CACHED) ? 1 : 0;
  return T <= 4 ? launch_mfma<1>(p, B, waves, stream) : launch_mfma<2>(p, B, waves, stream);
}

int qwen_attn_decode_mfma_noalloc(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                  const void* cos_tab, const void* sin_tab, const int32_t* positions, void* k_cache,
                                  void* v_cache, void* out, int B, int T, int Nq, int Nkv, int D, int CAP, int P,
                                  float eps, float scale, int num_splits, int waves, int flags, hipStream_t stream) {
  const int st = mfma_args_status(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out, B, T,
                                  Nq, Nkv, D, CAP, P, num_splits, waves, flags);
  if (st != QWEN_OK) return st;
  const long long need = qwen_attn_mfma_workspace_bytes(B, T, Nkv, num_splits);
  if (need > NOALLOC_SCRATCH_BYTES) return QWEN_ESCRATCH;
  if (need == 0 || B == 0)
    return qwen_attn_decode_mfma_ex(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out,
                                    nullptr, 0, B, T, Nq, Nkv, D, CAP, P, eps, scale, num_splits, waves, flags,
                                    stream);
  int status = QWEN_OK;
  void* ptr = device_scratch(&status);
  if (!ptr) return status;
  // the counters must start at zero (every launch re-arms them; cleared here all the same)
  const int words = (int)(mfma_counter_bytes((long long)B * Nkv) / 4);
  zero_words_kernel<<<(words + 255) / 256, 256, 0, stream>>>((unsigned*)ptr, words);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  return qwen_attn_decode_mfma_ex(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out, ptr,
                                  NOALLOC_SCRATCH_BYTES, B, T, Nq, Nkv, D, CAP, P, eps, scale, num_splits, waves,
                                  flags, stream);
}

int qwen_attn_decode_mfma(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                          const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                          void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D, int CAP,
                          int P, float eps, float scale, int num_splits, int waves, hipStream_t stream) {
  return qwen_attn_decode_mfma_ex(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out,
                                  workspace, workspace_bytes, B, T, Nq, Nkv, D, CAP, P, eps, scale, num_splits, waves,
                                  0, stream);
}

}  // extern "C"
