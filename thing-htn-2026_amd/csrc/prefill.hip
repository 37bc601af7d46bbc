// Prompt-forward kernels: the projection GEMM over many rows and causal flash attention.
//
// The reference's prompt forward (engine/engine.py:1181-1221) runs cuBLAS GEMMs and SDPA
// over B x S rows. Here the prompt goes through in position chunks of all sequences; per
// layer these two kernels do the heavy work (norms, RoPE + cache write and the first-token
// LM head are the decode path's kernels):
//
// pf_gemm_kernel<EPI>: out[M, N] = A[M, K] @ W[N, K]^T with bf16 operands, fp32
//   accumulation and one bf16 rounding (engine/kernels/gemm.py:12-15), and the fused
//   epilogues of the decode projections (engine/kernels/gemm_fused.py:5-19):
//     STORE : out = bf16(acc)
//     RES   : out = bf16(res + bf16(acc))              (residual may alias out)
//     SWIGLU: out = bf16(bf16(silu(bf16(g))) * bf16(u)) for a pair-interleaved gate|up weight
//   W is in the MFMA-B tile layout (weights.hip): tile (nt, kt) = 16 rows x 32 k, 1 KB,
//   lane l = 16 q + r holding W[16 nt + r][32 kt + 8 q .. +8], i.e. exactly the B operand of
//   v_mfma_f32_16x16x32_bf16, so B fragments are one 16-byte load per lane with no LDS.
//   A workgroup (4 wavefronts) computes a 256-row x 128-column tile; wavefront (wm, wn)
//   owns rows 128 wm .. +128 and n-tiles 4 wn .. +4 (8 x 4 accumulator tiles). A is staged
//   through LDS in k-steps of 64 (double buffered, 16-byte chunk c of row r at slot
//   c ^ (r % 8), so the A-fragment reads of 8 consecutive rows hit 8 different bank groups);
//   the next k-step's A and B loads are issued before the current one's MFMAs. Workgroups
//   walk the tile grid in groups of 8 row tiles per column tile, so the 8 workgroups that
//   share a weight column tile run at the same time (one per XCD) and each XCD keeps one
//   A row tile in its L2. The epilogue stages each wavefront's tile in LDS as bf16 and
//   writes 16-byte chunks.
//
// pf_attn_kernel: causal GQA attention of the T queries of a chunk (positions p0 + t) over
//   the cache slots [0, p0 + t] (engine/engine.py:1123-1179's SDPA, with the decode
//   attention's rounding points, engine/kernels/torch_ref.py:168-227: fp32 scores times
//   scale, probabilities rounded to bf16 for the value product, fp32 row sums, one final
//   rounding). One workgroup per (sequence, KV head, 16 query tokens) holds the 64 query
//   rows (16 tokens x the 4 heads of the group); wavefront w owns tokens 4w .. 4w + 3. K and
//   V blocks of 64 keys are staged in LDS once per workgroup (double buffered, padded rows)
//   and shared by the 4 wavefronts: S = Q K^T and O += P V on the matrix cores, online
//   softmax in the accumulator layout, V^T fragments by ds_read_b64_tr_b16 (as in
//   attention_mfma.hip). Workgroups with the most keys are launched first.
//
// The large shapes take the wide forms, each described at its definition below:
// pf_gemm_wide_kernel (N a multiple of 256: persistent 256 x 256 tiles, both operands by
// direct global -> LDS loads) and pf_attn_wide_kernel (chunks of more than 16 tokens: 32
// query tokens per 4-wavefront workgroup, two workgroups per CU).
#include "common.h"

namespace {

enum { PEPI_STORE = 0, PEPI_RES = 1, PEPI_SWIGLU = 2 };

constexpr int PBM = 256;   // rows of A per workgroup
constexpr int PBN = 128;   // weight rows (output columns before SwiGLU) per workgroup
constexpr int PBK = 64;    // k per pipeline stage
constexpr int PGM = 8;     // row tiles per group of the tile walk

// 16 bytes held as a native vector: arrays of these stay in VGPRs (an array of the HIP uint4
// struct is placed in scratch memory, and every load into it then waits at its store).
typedef unsigned pv4 __attribute__((ext_vector_type(4)));

struct PfGemmParams {
  const bf16_t* a;    // [M, K] row-major
  const bf16_t* w;    // tiled [N, K]
  const bf16_t* res;  // [M, ldo] (RES; may alias out)
  bf16_t* out;        // [M, ldo]
  int M, N, K, ldo;
  int mtiles, ntiles;
};

template <int EPI>
__global__ void __launch_bounds__(256, 2) pf_gemm_kernel(PfGemmParams p) {
  __shared__ uint4 lds[2 * PBM * (PBK / 8)];  // 64 KB: A double buffer, then the epilogue tiles
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int qq = lane >> 4, rr = lane & 15;

  // tile walk: groups of PGM row tiles; inside a group the row tile varies fastest
  const int id = blockIdx.x;
  const int per_group = PGM * p.ntiles;
  const int grp = id / per_group;
  const int rem = id - grp * per_group;
  const int gsz = min(PGM, p.mtiles - grp * PGM);
  const int mt = grp * PGM + rem % gsz;
  const int ntile = rem / gsz;
  const long long m0 = (long long)mt * PBM;
  const int KT = p.K / 32, KB = p.K / PBK;
  const int nt0 = ntile * (PBN / 16) + wn * 4;  // this wavefront's first n-tile

  // A staging: thread -> 16-byte column chunk ac of rows (tid >> 3) + 32 i (rows past M
  // re-read row M - 1 and are never stored)
  const int ac = tid & 7;
  // (M * K < 2^31 is checked by the host: element offsets fit in 32 bits)
  const bf16_t* abase = p.a + ac * 8;
  int aoff[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) aoff[i] = (int)min(m0 + (tid >> 3) + 32 * i, (long long)p.M - 1) * p.K;
  pv4 ast[8];
  auto load_a = [&](int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) ast[i] = *reinterpret_cast<const pv4*>(abase + aoff[i] + kb * PBK);
  };
  auto store_a = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = (tid >> 3) + 32 * i;
      *reinterpret_cast<pv4*>(&lds[buf * (PBM * 8) + row * 8 + (ac ^ (row & 7))]) = ast[i];
    }
  };
  const pv4* wb = reinterpret_cast<const pv4*>(p.w) + (long long)nt0 * KT * 64 + lane;
  pv4 bcur[4][2], bnext[4][2];
  auto load_b = [&](pv4 (&d)[4][2], int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) d[j][kt] = wb[((long long)j * KT + kb * 2 + kt) * 64];
  };

  f32x4_t acc[8][4];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[mb][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  load_a(0);
  load_b(bcur, 0);
  store_a(0);
  __syncthreads();
  for (int kb = 0; kb < KB; ++kb) {
    // next stage's loads first (the last iteration re-reads its own stage: in bounds, unused)
    const int kn = kb + 1 < KB ? kb + 1 : kb;
    load_a(kn);
    load_b(bnext, kn);
    const uint4* abuf = lds + (kb & 1) * (PBM * 8);
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const int row = wm * 128 + mb * 16 + rr;
        const bf16x8_t af = as_bf16x8(abuf[row * 8 + ((kt * 4 + qq) ^ (row & 7))]);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[mb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, __builtin_bit_cast(bf16x8_t, bcur[j][kt]),
                                                               acc[mb][j], 0, 0, 0);
      }
    }
    store_a((kb + 1) & 1);  // buffer last read one iteration ago (behind the barrier below)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) bcur[j][kt] = bnext[j][kt];
    __syncthreads();
  }

  // ---- epilogue: wavefront tile -> bf16 in LDS (rows of 8 chunks of 16 bytes, chunk c of
  // row r at slot c ^ (r % 8)), then 16-byte stores.
  // Accumulator layout: acc[mb][j][i] = D[16 mb + 4 qq + i][16 j + rr] of the wavefront tile.
  constexpr int OCOLS = EPI == PEPI_SWIGLU ? 32 : 64;  // output columns per wavefront
  constexpr int CPR = OCOLS / 8;                        // 16-byte chunks per row
  bf16_t* tile = reinterpret_cast<bf16_t*>(lds + wave * 1024);  // 16 KB per wavefront
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = mb * 16 + 4 * qq + i;
      if constexpr (EPI == PEPI_SWIGLU) {
#pragma unroll
        for (int pj = 0; pj < 2; ++pj) {
          const float g = rbf(acc[mb][2 * pj][i]);
          const float u = rbf(acc[mb][2 * pj + 1][i]);
          const float s = rbf(g / (1.0f + expf(-g)));
          const int col = pj * 16 + rr;
          tile[row * 64 + (((col >> 3) ^ (row & 7)) << 3) + (col & 7)] = f2bf(mul_rn(s, u));
        }
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int col = j * 16 + rr;
          tile[row * 64 + (((col >> 3) ^ (row & 7)) << 3) + (col & 7)] = f2bf(acc[mb][j][i]);
        }
      }
    }
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wavefront's LDS writes are done
  __builtin_amdgcn_wave_barrier();
  const long long col0 = EPI == PEPI_SWIGLU ? (long long)(nt0 / 2) * 16 : (long long)nt0 * 16;
#pragma unroll 4
  for (int c = lane; c < 128 * CPR; c += 64) {
    const int row = c / CPR, ch = c - row * CPR;
    const long long grow = m0 + wm * 128 + row;
    const uint4 v = *reinterpret_cast<const uint4*>(tile + row * 64 + ((ch ^ (row & 7)) << 3));
    if (grow < p.M) {
      bf16_t* dst = p.out + grow * p.ldo + col0 + ch * 8;
      if constexpr (EPI == PEPI_RES) {
        const uint4 rv = *reinterpret_cast<const uint4*>(p.res + grow * p.ldo + col0 + ch * 8);
        float a[8], r[8];
        unpack8(v, a);
        unpack8(rv, r);
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = add_rn(r[e], a[e]);
        *reinterpret_cast<uint4*>(dst) = pack8(a);
      } else {
        *reinterpret_cast<uint4*>(dst) = v;
      }
    }
  }
}


// Wide form of the prompt GEMM (qwen_gemm for N a multiple of 256): a workgroup of WV
// wavefronts computes a 256-row x 256-column tile, wavefront (wm, wn) a 128-row x 512 / WV-column
// part (8 x 32 / WV accumulator tiles). With WV = 8 (the launched form) that is 128 registers
// of accumulators and two wavefronts per SIMD, so one wavefront's LDS reads and load issues
// run under the other's MFMAs (measured against WV = 4, 128 x 128 parts in the AGPRs and one
// wavefront per SIMD: gate/up 1137 -> 1176, down 1031 -> 1092, QKV 1069 -> 1053, O 1044 -> 1018
// TFLOP/s). Both operands are staged in LDS per k-step of 64 (double buffered, 2 x 64 KB): A rows
// as in pf_gemm_kernel (16-byte chunk c of row r at slot c ^ (r % 8)), W as its 1 KB MFMA tiles
// in their global order. Per k-step and CU that is 64 KB from L2 for 8.4 MFLOP, half of
// pf_gemm_kernel's traffic per flop. The product is computed transposed, D^T = W X^T: a weight tile is the MFMA's A
// operand as it stands (lane (q, r): row r, k 8 q ..) and an A-row fragment its B operand, so
// lane (q, r) of accumulator tile (mb, nb) holds D[16 mb + r][16 nb + 4 q + i], four adjacent
// output columns of one row: the epilogue writes them as one 8-byte store (SwiGLU pairs the
// gate and up tiles 2 p, 2 p + 1 of the pair-interleaved weight element by element).
// Direct global -> LDS load of 16 bytes per lane: lane l's bytes land at LDS byte address
// `lds_addr` + 16 l (lds_addr wavefront-uniform, held in M0). Written as inline assembly so that
// the compiler does not treat it as an LDS store: it would otherwise make every later LDS read
// wait for all such loads. The caller therefore waits for them itself (lds_dma_wait) before
// the barrier after which they are read; waits the compiler places for its own loads stay
// correct, only more conservative (loads complete in issue order). s_nop covers the M0 write ->
// LDS-DMA hazard.
__device__ __forceinline__ void lds_dma16(const void* gptr, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(gptr), "s"(lds_addr)
               : "memory", "m0");
}
__device__ __forceinline__ void lds_dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// The same load with a wavefront-uniform base in SGPRs and a 32-bit per-lane byte offset (the
// instruction's saddr form): no 64-bit address arithmetic per load.
__device__ __forceinline__ void lds_dma16_so(const void* sbase, unsigned voff, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds_addr)
               : "memory", "m0");
}

constexpr int PWM = 256;   // rows per workgroup
constexpr int PWN = 256;   // weight rows (output columns before SwiGLU) per workgroup
constexpr int PWG = 4;     // row tiles per group of the wide kernel's tile walk
constexpr int PWV = 8;     // wavefronts of the wide kernel (two per SIMD, 128 x 64 quadrants each)

template <int EPI, int WV>
__global__ void __launch_bounds__(64 * WV, 1) pf_gemm_wide_kernel(PfGemmParams p) {
  constexpr int NB = 32 / WV;        // 16-column accumulator tiles per wavefront (8 or 4)
  constexpr int PAIRS = 32 / WV;     // (A block, W tile) direct loads per wavefront and stage
  __shared__ pv4 lds[2 * (PWM + PWN) * (PBK / 8)];  // [stage][A: 256 rows x 8 chunks | W: 32 tiles x 64 lanes]
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int qq = lane >> 4, rr = lane & 15;

  // Persistent tile walk: gridDim.x = 8 s workgroups, workgroup g on XCD g % 8 (one per CU).
  // XCD x owns the contiguous run of logical tiles [x * ceil(T / 8), ...); its s workgroups take
  // them s at a time (workgroup g: run positions g / 8, g / 8 + s, ...). Logical tiles go in
  // groups of PWG row tiles, the row tile fastest, so the tiles an XCD works on at one time
  // form a block of PWG row tiles x s / PWG column tiles and share A and W k-slabs in its L2.
  // A workgroup keeps its CU from tile to tile: the next tile's first k-step is loaded while the
  // current tile's last one computes, and the current tile's output stores drain while the next
  // tile's MFMAs run (no workgroup turnover, no chip-wide burst of epilogue stores).
  const int tiles = p.mtiles * p.ntiles;
  const int per_xcd = (tiles + 7) / 8;
  const int xcd = (int)(blockIdx.x & 7), slot = (int)(blockIdx.x >> 3), nslots = (int)(gridDim.x >> 3);
  const int KT = p.K / 32, KB = p.K / PBK;
  auto tile_at = [&](int step, long long& m0, int& nt0) -> bool {
    const int j = slot + step * nslots;
    const int lt = xcd * per_xcd + j;
    if (j >= per_xcd || lt >= tiles) return false;
    const int gsize = PWG * p.ntiles;
    const int grp = lt / gsize;
    const int rem = lt - grp * gsize;
    const int gsz = min(PWG, p.mtiles - grp * PWG);
    m0 = (long long)(grp * PWG + rem % gsz) * PWM;
    nt0 = (rem / gsz) * (PWN / 16);  // the tile's first weight n-tile
    return true;
  };

  // Staging by direct global -> LDS loads (16 bytes per lane; one instruction fills 1 KB of LDS,
  // lane l at byte 16 l): wavefront w fills A blocks 8 w .. 8 w + 7 (block b = rows 8 b .. 8 b + 7;
  // lane l loads chunk (l % 8) ^ (l / 8) of row 8 b + l / 8, which lands in the swizzled slot
  // l % 8 of that row) and W tiles 8 w .. 8 w + 7 of the k-step (tile t = 2 j + kt, stored as
  // in memory). Rows past M re-read row M - 1 and are never stored. No staging registers.
  // (M * K < 2^31 is checked by the host.)
  // Addresses are formed per load from the tile's origin (m0, nt0), both wavefront-uniform:
  // arrays of per-tile offsets kept across the tile loop would live in scratch memory.
  const int achunk = ((lane & 7) ^ (lane >> 3)) * 8;
  const int arow = wave * PAIRS * 8 + (lane >> 3);  // + 8 i: this lane's row of A block PAIRS wave + i
  const pv4* wlane = reinterpret_cast<const pv4*>(p.w) + lane;
  // LDS byte address of stage 0 (stage 1 follows it)
  const unsigned lds0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) pv4*)lds;
  // Loads i of a stage (i < PAIRS): the wavefront's A block PAIRS wave + i and W tile PAIRS wave + i.
  auto issue_pair = [&](long long m0, int nt0, int kb, int buf, int i) __attribute__((always_inline)) {
    const unsigned sb = lds0 + buf * ((PWM + PWN) * 8 * 16);
    const long long row = min(m0 + arow + 8 * i, (long long)p.M - 1);
    lds_dma16(p.a + (int)row * p.K + achunk + kb * PBK, sb + (wave * PAIRS + i) * 1024);
    const int t = wave * PAIRS + i;
    lds_dma16(wlane + ((long long)(nt0 + (t >> 1)) * KT + kb * 2 + (t & 1)) * 64, sb + (PWM * 8 + t * 64) * 16);
  };
  auto issue = [&](long long m0, int nt0, int kb, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PAIRS; ++i) issue_pair(m0, nt0, kb, buf, i);
  };

  f32x4_t acc[8][NB];

  // One k-step on stage `buf`: the first half k-step's 16 fragments (8 W, 8 A-row) are read,
  // then the half's MFMAs run in groups of 8 (one A-row fragment each). After each group two of
  // the second half's fragments are requested, so the LDS reads overlap the matrix cores and no
  // wait needs more than 15 LDS requests outstanding (the counter's limit), and two of the
  // following stage's 16 direct loads go out (that stage was last read one k-step ago): issued
  // back to back, 64 loads of 1 KB per CU hold each wavefront at issue while the address unit
  // works through them (measured: the k-step then takes 1.6x its MFMA time), spread out they run
  // under the MFMAs. The scheduling barriers pin that order.
  auto kstep = [&](int buf, bool nload, long long nm0, int nnt0, int nkb) __attribute__((always_inline)) {
    const pv4* cur = lds + buf * ((PWM + PWN) * 8);
    auto wfrag = [&](int kt, int nb) { return __builtin_bit_cast(bf16x8_t, cur[PWM * 8 + ((wn * NB + nb) * 2 + kt) * 64 + lane]); };
    auto xfrag = [&](int kt, int mb) {
      const int row = wm * 128 + mb * 16 + rr;
      return __builtin_bit_cast(bf16x8_t, cur[row * 8 + ((kt * 4 + qq) ^ (row & 7))]);
    };
    bf16x8_t w0[NB], x0[8], w1[NB], x1[8];
#pragma unroll
    for (int j = 0; j < NB; ++j) w0[j] = wfrag(0, j);
#pragma unroll
    for (int j = 0; j < 8; ++j) x0[j] = xfrag(0, j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w0[nb], x0[mb], acc[mb][nb], 0, 0, 0);
      if (mb < NB) w1[mb] = wfrag(1, mb);
      x1[mb] = xfrag(1, mb);
      if (nload && mb < PAIRS) issue_pair(nm0, nnt0, nkb, buf ^ 1, mb);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w1[nb], x1[mb], acc[mb][nb], 0, 0, 0);
    }
    // The MFMAs only touch registers, so the scheduler may sink them below the barrier and the
    // wait for the loads issued above; this keeps them ahead (they run while the loads fly).
    __builtin_amdgcn_sched_barrier(0);
    lds_dma_wait();  // this wavefront's loads have landed in LDS ...
    __syncthreads();  // ... and, past the barrier, every wavefront's
  };

  // Epilogue of the tile at (m0, nt0): lane (q, r) of accumulator tile (mb, nb) holds
  // D[16 mb + r][16 nb + 4 q + i] of the wavefront's quadrant; four adjacent columns -> one
  // 8-byte store.
  auto epilogue = [&](long long m0, int nt0) __attribute__((always_inline)) {
  #pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const long long grow = m0 + wm * 128 + mb * 16 + rr;
      if (grow >= p.M) continue;
      if constexpr (EPI == PEPI_SWIGLU) {
  #pragma unroll
        for (int pj = 0; pj < NB / 2; ++pj) {
          float o[4];
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float g = rbf(acc[mb][2 * pj][i]);
            const float u = rbf(acc[mb][2 * pj + 1][i]);
            const float sg = rbf(g / (1.0f + expf(-g)));
            o[i] = mul_rn(sg, u);
          }
          const long long col = (long long)(nt0 / 2 + wn * (NB / 2) + pj) * 16 + 4 * qq;
          *reinterpret_cast<uint2*>(p.out + grow * p.ldo + col) = make_uint2(f2bf2(o[0], o[1]), f2bf2(o[2], o[3]));
        }
      } else {
  #pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const long long col = (long long)(nt0 + wn * NB + nb) * 16 + 4 * qq;
          float o[4];
  #pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = acc[mb][nb][i];
          if constexpr (EPI == PEPI_RES) {
            const uint2 rv = *reinterpret_cast<const uint2*>(p.res + grow * p.ldo + col);
  #pragma unroll
            for (int i = 0; i < 4; ++i) {
              const uint32_t w2 = i < 2 ? rv.x : rv.y;
              const float r = __uint_as_float((i & 1) ? (w2 & 0xffff0000u) : (w2 << 16));
              o[i] = add_rn(r, rbf(o[i]));
            }
          }
          *reinterpret_cast<uint2*>(p.out + grow * p.ldo + col) = make_uint2(f2bf2(o[0], o[1]), f2bf2(o[2], o[3]));
        }
      }
    }
  };

  long long m0;
  int nt0;
  if (!tile_at(0, m0, nt0)) return;
  issue(m0, nt0, 0, 0);
  lds_dma_wait();
  __syncthreads();
  int buf = 0;
  for (int step = 0;; ++step) {
    long long m1 = 0;
    int nt1 = 0;
    const bool more = tile_at(step + 1, m1, nt1);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb + 1 < KB; ++kb) {  // the next stage is this tile's k-step kb + 1
      kstep(buf, true, m0, nt0, kb + 1);
      buf ^= 1;
    }
    kstep(buf, more, m1, nt1, 0);  // last k-step: the next stage is the next tile's first
    buf ^= 1;
    epilogue(m0, nt0);
    if (!more) break;
    m0 = m1;
    nt0 = nt1;
  }
}

// ------------------------------------------------------------------ causal flash attention
constexpr int AD = 128;      // head dim
constexpr int AG = 4;        // query heads per KV head
constexpr int AQ = 16;       // query tokens per workgroup
constexpr int AKB = 64;      // keys per block
constexpr int AKROW = 136;   // bf16 per LDS row of K (272 B)
constexpr int AVROW = 144;   // bf16 per LDS row of V (288 B: banked transpose reads)
constexpr float ANEG = -1e30f;

typedef short av4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) av4i16 lds_av4i16;

struct PfAttnParams {
  const bf16_t* q;   // [B, T, Nq, D] (normed + rotated)
  const bf16_t* kc;  // [B, Nkv, CAP, D]
  const bf16_t* vc;
  bf16_t* out;       // [B, T, Nq * D]
  int T, Nkv, CAP, p0, qblocks;
  long long bh_count;
  float scale;
};

struct PfAttnSmem {
  bf16_t k[2][AKB][AKROW];
  bf16_t v[2][AKB][AVROW];
  bf16_t pm[4][16][AKB];
};

__global__ void __launch_bounds__(256, 2) pf_attn_kernel(PfAttnParams p) {
  __shared__ PfAttnSmem sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qq = lane >> 4, rr = lane & 15;
  // heaviest query blocks first
  const long long id = blockIdx.x;
  const int qb = p.qblocks - 1 - (int)(id / p.bh_count);
  const long long bh = id % p.bh_count;
  const long long b = bh / p.Nkv;
  const int kvh = (int)(bh - b * p.Nkv);
  const int T = p.T, Nq = p.Nkv * AG;
  const int t_lo = qb * AQ;
  const int kmax = p.p0 + min(T, t_lo + AQ);  // keys [0, kmax) are visible to some query here
  const int nblk = (kmax + AKB - 1) / AKB;
  const bf16_t* kbase = p.kc + bh * (long long)p.CAP * AD;
  const bf16_t* vbase = p.vc + bh * (long long)p.CAP * AD;

  // Q A-operand fragments: lane (q, r) holds row r of this wavefront's tile (token
  // 4 wave + r / 4, head r % 4), dims 32 kt + 8 q .. +8. Tokens past T re-read token T - 1.
  bf16x8_t qa[4];
  {
    const int t = min(t_lo + 4 * wave + (rr >> 2), T - 1);
    const bf16_t* qr = p.q + (((b * T + t) * Nq) + kvh * AG + (rr & 3)) * (long long)AD + 8 * qq;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) qa[kt] = as_bf16x8(*reinterpret_cast<const uint4*>(qr + 32 * kt));
  }
  // accumulator rows 4 qq + i: token t_lo + 4 wave + qq, head i; its last visible key
  const int my_tok = t_lo + 4 * wave + qq;
  const int my_last = p.p0 + my_tok;

  // K / V staging: thread -> 16-byte chunk c of keys (tid >> 4) + 16 i (keys past kmax are
  // read from slot 0 and their V rows zeroed, so a stale or non-finite slot never enters)
  const int sc = tid & 15;
  pv4 kst[4], vst[4];
  auto load_kv = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = blk * AKB + (tid >> 4) + 16 * i;
      const long long off = (long long)(key < kmax ? key : 0) * AD + sc * 8;
      kst[i] = *reinterpret_cast<const pv4*>(kbase + off);
      vst[i] = *reinterpret_cast<const pv4*>(vbase + off);
    }
  };
  auto store_kv = [&](int buf, int blk) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kr = (tid >> 4) + 16 * i;
      const bool live = blk * AKB + kr < kmax;
      *reinterpret_cast<pv4*>(&sm.k[buf][kr][sc * 8]) = kst[i];
      *reinterpret_cast<pv4*>(&sm.v[buf][kr][sc * 8]) = live ? vst[i] : pv4{0u, 0u, 0u, 0u};
    }
  };

  float m[4], l[4];
  f32x4_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) { m[i] = ANEG; l[i] = 0.f; }
#pragma unroll
  for (int nd = 0; nd < 8; ++nd) o[nd] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  bf16_t* pl = &sm.pm[wave][0][0];

  load_kv(0);
  store_kv(0, 0);
  __syncthreads();
  for (int blk = 0; blk < nblk; ++blk) {
    const int nb = blk + 1 < nblk ? blk + 1 : blk;
    load_kv(nb);
    const int buf = blk & 1;
    const int kb0 = blk * AKB;
    // S = Q K^T for 4 tiles of 16 keys: lane (q, r) takes key 16 nt + r, dims 32 kt + 8 q ..
    f32x4_t s[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      s[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const uint4 kf = *reinterpret_cast<const uint4*>(&sm.k[buf][16 * nt + rr][32 * kt + 8 * qq]);
        s[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[kt], as_bf16x8(kf), s[nt], 0, 0, 0);
      }
    }
    // online softmax (rows 4 qq + i share the token, so one causal limit per lane)
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float sv[4];
      float mx = ANEG;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const bool vis = kb0 + 16 * nt + rr <= my_last;
        sv[nt] = vis ? s[nt][i] * p.scale : ANEG;
        mx = fmaxf(mx, sv[nt]);
      }
      mx = row16_max(mx);
      const float mn = fmaxf(m[i], mx);
      alpha[i] = __expf(m[i] - mn);
      float psum = 0.f;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        const float pr = sv[nt] > ANEG ? __expf(sv[nt] - mn) : 0.f;
        psum += pr;
        pl[(4 * qq + i) * AKB + 16 * nt + rr] = f2bf(pr);  // P rounded to bf16 for PV
      }
      l[i] = l[i] * alpha[i] + psum;
      m[i] = mn;
    }
#pragma unroll
    for (int nd = 0; nd < 8; ++nd)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[nd][i] *= alpha[i];
    // P in the A layout (lane (q, r): row r, keys 32 kk + 8 q ..); the round trip stays inside
    // the wavefront (LDS instructions complete in order)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    bf16x8_t pa[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) pa[kk] = as_bf16x8(*reinterpret_cast<const uint4*>(pl + rr * AKB + 32 * kk + 8 * qq));
    // O += P V: V^T fragments by transpose reads, source lane s -> V[8 q + s / 4 (+4)][16 nd + 4 (s % 4)]
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const bf16_t* vs = &sm.v[buf][32 * kk + 8 * qq + (rr >> 2)][4 * (rr & 3)];
#pragma unroll
      for (int nd = 0; nd < 8; ++nd) {
        const av4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_av4i16*)(vs + 16 * nd));
        const av4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_av4i16*)(vs + 4 * AVROW + 16 * nd));
        const uint4 vv = make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                    __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y);
        o[nd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[kk], as_bf16x8(vv), o[nd], 0, 0, 0);
      }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    store_kv(buf ^ 1, nb);  // buffer last read one iteration ago (behind the barrier below)
    __syncthreads();
  }

  // ---- normalise and write: the wavefront's 16 rows x 128 dims through LDS (bf16), 16-byte stores
#pragma unroll
  for (int i = 0; i < 4; ++i) l[i] = row16_sum(l[i]);
  bf16_t* ot = &sm.k[0][0][0] + wave * 16 * AKROW;  // 16 rows of 272 B per wavefront
#pragma unroll
  for (int nd = 0; nd < 8; ++nd)
#pragma unroll
    for (int i = 0; i < 4; ++i) ot[(4 * qq + i) * AKROW + 16 * nd + rr] = f2bf(o[nd][i] / l[i]);
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int c = lane + 64 * it;        // 16 rows x 16 chunks
    const int row = c >> 4, ch = c & 15;
    const int t = t_lo + 4 * wave + (row >> 2);
    if (t < T) {
      const uint4 v = *reinterpret_cast<const uint4*>(ot + row * AKROW + ch * 8);
      bf16_t* dst = p.out + ((b * T + t) * Nq + kvh * AG + (row & 3)) * (long long)AD + ch * 8;
      *reinterpret_cast<uint4*>(dst) = v;
    }
  }
}


// Wide form of the prompt attention (qwen_attn_prefill for chunks of more than 16 tokens):
// 4 wavefronts x 2 query tiles per workgroup, i.e. 32 query tokens x the 4 heads of the GQA group
// = 128 query rows over the same 64-key K / V block in LDS. Wavefront w owns tokens 8 w .. 8 w + 7
// (tile mt: tokens 8 w + 4 mt .. + 3), so every K fragment read from LDS feeds both tiles' MFMAs
// and each staged K / V byte serves twice as many query rows as in pf_attn_kernel. Two
// workgroups share a CU (64 KB of LDS each), so the two wavefronts on a SIMD belong to different
// workgroups with their own barriers and drift apart: one's softmax runs under the other's MFMAs
// (measured on MI355X at the 32 x 512-token chunks: 2-3 % faster than one 8-wavefront
// workgroup of 64 tokens per CU, 20 % on the first chunk).
constexpr int AW2 = 4;               // wavefronts per workgroup
constexpr int AQ2 = AW2 * 2 * 4;     // query tokens per workgroup (2 tiles of 4 tokens per wavefront)
constexpr int AGPW = AKB / 4 / AW2;  // 4-row groups of a K / V block staged by each wavefront

// The score tiles are computed transposed, S^T = K Q^T (K as the MFMA's A operand, Q^T as B).
// Lane (q, r) then holds query r's scores for keys 16 nt + 4 q + i, which is already the
// B-operand layout of O^T += V^T P^T once the k-slots of the PV product are ordered
// (32 kk + 4 q + j, 32 kk + 16 + 4 q + j): P goes from the score accumulators into the PV MFMA
// through packed bf16 conversions, with no LDS round trip, and the V^T fragments are transposed
// LDS reads in that same key order. Softmax state is one (m, l) per lane and tile; a query's 64
// scores sit on 4 lanes (r, r + 16, r + 32, r + 48), so a block maximum is 15 in-lane maxima and
// 2 cross-lane steps. The causal mask is applied only to blocks that reach past the wavefront's
// first token. exp(x - m) is evaluated as exp2((x - m) log2 e) with scale folded in, and the
// rescale factor as exp2((m_old - m_new) scale log2 e), exactly 1 when the maximum is unchanged:
// a block that is fully masked for a query leaves that query's state bit for bit as it was, so
// the result does not depend on how many such blocks a workgroup walks. Rounding points as
// pf_attn_kernel (P rounded to bf16 for PV, l from the unrounded P, O normalised in fp32, then
// rounded). exp2 is the hardware v_exp_f32: a P below 2^-126 of the block maximum flushes to 0,
// far under bf16's resolution of the row sum.
__device__ __forceinline__ float xlane_max4(float v) { return xor32_max(xor16_max(v)); }
__device__ __forceinline__ float xlane_sum4(float v) { return xor32_sum(xor16_sum(v)); }

__global__ void __launch_bounds__(AW2 * 64, 2) pf_attn_wide_kernel(PfAttnParams p) {
  // K / V blocks in 256-byte rows with no padding (direct-to-LDS loads fill 1 KB runs), swizzled
  // so that the fragment reads stay conflict-free: K's 16-byte chunk c of key row r at c ^ (r % 16)
  // (the S^T operand reads 16 rows of one chunk), V's 32-byte block j of row r at j ^ (r % 8) (a
  // transposed read takes 8 bytes from 4 consecutive rows of one block, two groups of lanes at
  // once take rows 4 apart).
  __shared__ union {
    struct {
      pv4 k[2][AKB][16];
      pv4 v[2][AKB][16];
    } kv;
    bf16_t ot[AW2][32][AKROW];       // output staging: 32 rows per wavefront
  } sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qq = lane >> 4, rr = lane & 15;
  // Launch order: workgroup g runs on XCD g % 8 and takes logical item (g % 8) * ceil(G / 8) +
  // g / 8, so each XCD walks a contiguous run of items; an item is (head group bh, query block),
  // all query blocks of a head group consecutive, heaviest first. The workgroups that read the
  // same K / V (every query block of one head group) then run at the same time on one XCD and
  // stream its blocks in step, through that XCD's L2, instead of each reading them from HBM in
  // a different round.
  const long long G = p.bh_count * p.qblocks;
  const long long per_xcd = (G + 7) / 8;
  const long long item = (long long)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  if (item >= G) return;
  const long long bh = item / p.qblocks;
  const int qb = p.qblocks - 1 - (int)(item - bh * p.qblocks);
  const long long b = bh / p.Nkv;
  const int kvh = (int)(bh - b * p.Nkv);
  const int T = p.T, Nq = p.Nkv * AG;
  const int t_lo = qb * AQ2;
  const int kmax = p.p0 + min(T, t_lo + AQ2);  // keys [0, kmax) are visible to some query here
  const int nblk = (kmax + AKB - 1) / AKB;
  const bf16_t* kbase = p.kc + bh * (long long)p.CAP * AD;
  const bf16_t* vbase = p.vc + bh * (long long)p.CAP * AD;

  // Q^T B-operand fragments: lane (q, r) of tile mt holds query r (token 8 wave + 4 mt + r / 4,
  // head r % 4), dims 32 kt + 8 q .. +8. Tokens past T re-read token T - 1.
  bf16x8_t qb8[2][4];
  int my_last[2];                    // last key visible to this lane's query, per tile
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const int tq = t_lo + 8 * wave + 4 * mt + (rr >> 2);
    const bf16_t* qr = p.q + (((b * T + min(tq, T - 1)) * Nq) + kvh * AG + (rr & 3)) * (long long)AD + 8 * qq;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) qb8[mt][kt] = as_bf16x8(*reinterpret_cast<const uint4*>(qr + 32 * kt));
    my_last[mt] = p.p0 + tq;
  }
  const int wave_first = p.p0 + t_lo + 8 * wave;  // every query of the wavefront sees keys <= this
  const float c = p.scale * 1.4426950408889634f;  // scale * log2(e)

  // K / V staging by direct global -> LDS loads: wavefront w fills key rows 16 w .. 16 w + 15
  // of a block (four 1 KB runs of 4 rows each for K and for V). Lane l lands at row
  // 4 (AGPW w + i) + l / 16, physical chunk l % 16, so it loads the logical chunk the swizzle
  // puts there. Keys past kmax read slot kmax - 1, one of this chunk's keys (written before the
  // attention runs, so finite), and every query weighs them with P = 0 exactly: a stale or
  // non-finite slot never enters.
  const int srow = lane >> 4, spc = lane & 15;
  const unsigned lds_k = (unsigned)(uintptr_t)(__attribute__((address_space(3))) pv4*)&sm.kv.k[0][0][0];
  const unsigned lds_v = (unsigned)(uintptr_t)(__attribute__((address_space(3))) pv4*)&sm.kv.v[0][0][0];
  // (K and V are issued separately, so a block's eight loads per wavefront do not go out in one
  // burst)
  // A lane's byte offset within a block is the same for every block: row r's logical chunk,
  // r * 256 + chunk * 16, added to the block's address in the scalar base. In the
  // workgroup's last block, if it reaches past kmax, rows at or past kmax read row kmax - 1
  // instead (still within the block, so every offset stays below 16 KB whatever the cache
  // capacity).
  unsigned koff[AGPW], voff[AGPW];
#pragma unroll
  for (int i = 0; i < AGPW; ++i) {
    const int r = 4 * (AGPW * wave + i) + srow;
    koff[i] = (unsigned)(r * 256 + (spc ^ (r & 15)) * 16);                          // logical K chunk
    voff[i] = (unsigned)(r * 256 + (2 * ((spc >> 1) ^ (r & 7)) + (spc & 1)) * 16);  // V chunk
  }
  auto issue_kv = [&](int blk, int buf, bool k) __attribute__((always_inline)) {
    const bf16_t* sb = (k ? kbase : vbase) + (long long)blk * AKB * AD;
    const unsigned lds0 = (k ? lds_k : lds_v) + (unsigned)((buf * AKB + 4 * AGPW * wave) * 256);
    if ((blk + 1) * AKB <= kmax) {
#pragma unroll
      for (int i = 0; i < AGPW; ++i) lds_dma16_so(sb, k ? koff[i] : voff[i], lds0 + i * 1024);
    } else {
      const int last = kmax - 1 - blk * AKB;   // last row of the block below kmax (>= 0)
#pragma unroll
      for (int i = 0; i < AGPW; ++i) {
        const int r = 4 * (AGPW * wave + i) + srow;   // row of the block
        const unsigned off = k ? koff[i] : voff[i];
        lds_dma16_so(sb, r <= last ? off : off - (unsigned)((r - last) * 256), lds0 + i * 1024);
      }
    }
  };

  float m[2] = {ANEG, ANEG}, l[2] = {0.f, 0.f};
  f32x4_t o[2][8];                   // O^T: lane (q, r) holds dims 16 nd + 4 q + i of query r
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nd = 0; nd < 8; ++nd) o[mt][nd] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  issue_kv(0, 0, true);
  issue_kv(0, 0, false);
  lds_dma_wait();
  __syncthreads();
  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1;
    const bool more = blk + 1 < nblk;
    if (more) issue_kv(blk + 1, buf ^ 1, true);  // that buffer was last read one block ago
    const int kb0 = blk * AKB;
    // S^T for 4 tiles of 16 keys: A = K rows 16 nt + r, dims 32 kt + 8 q (one LDS read per
    // (nt, kt), both query tiles)
    f32x4_t st[2][4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      st[0][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      st[1][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const uint4 kf = __builtin_bit_cast(uint4, sm.kv.k[buf][16 * nt + rr][(4 * kt + qq) ^ rr]);
        st[0][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf), qb8[0][kt], st[0][nt], 0, 0, 0);
        st[1][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kf), qb8[1][kt], st[1][nt], 0, 0, 0);
      }
    }
    if (more) issue_kv(blk + 1, buf ^ 1, false);
    if (kb0 + AKB - 1 > wave_first) {  // block reaches past some query's last key: mask
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (kb0 + 16 * nt + 4 * qq + i > my_last[mt]) st[mt][nt][i] = ANEG;
    }
    // online softmax per tile (one query per lane); P^T as packed bf16 B fragments
    uint4 pb[2][2];
    float alpha[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      float mx = st[mt][0][0];
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, st[mt][nt][i]);
      mx = xlane_max4(mx);
      const float mn = fmaxf(m[mt], mx);
      const float mc = mn * c;
      alpha[mt] = __builtin_amdgcn_exp2f((m[mt] - mn) * c);  // 1 exactly if mn == m
      float pr[4][4];
      float psum = 0.f;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pr[nt][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[mt][nt][i], c, -mc));  // masked: 0
          psum += pr[nt][i];
        }
      l[mt] = l[mt] * alpha[mt] + psum;
      m[mt] = mn;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        pb[mt][kk] = make_uint4(f2bf2(pr[2 * kk][0], pr[2 * kk][1]), f2bf2(pr[2 * kk][2], pr[2 * kk][3]),
                                f2bf2(pr[2 * kk + 1][0], pr[2 * kk + 1][1]), f2bf2(pr[2 * kk + 1][2], pr[2 * kk + 1][3]));
    }
    // rescale O only when some query's maximum moved (alpha is exactly 1 otherwise)
    if (__builtin_amdgcn_ballot_w64(alpha[0] != 1.f || alpha[1] != 1.f) != 0) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nd = 0; nd < 8; ++nd)
#pragma unroll
          for (int i = 0; i < 4; ++i) o[mt][nd][i] *= alpha[mt];
    }
    // O^T += V^T P^T: A = V^T rows (dims) 16 nd + r, k-slots j -> key 32 kk + 4 q + j (lo) and
    // 32 kk + 16 + 4 q + j (hi), by transpose reads of 4 keys x 16 dims (source lane s ->
    // V[32 kk + 4 q + s / 4 (+16)][16 nd + 4 (s % 4)]), one read pair per (kk, nd) for both tiles
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      // row 32 kk + 4 q + r / 4 (+ 16), 8 bytes at column 16 nd + 4 (r % 4) of its swizzled block
      const int vr = 32 * kk + 4 * qq + (rr >> 2);
      const bf16_t* vlo = reinterpret_cast<const bf16_t*>(&sm.kv.v[buf][vr][0]) + 4 * (rr & 3);
      const bf16_t* vhi = reinterpret_cast<const bf16_t*>(&sm.kv.v[buf][vr + 16][0]) + 4 * (rr & 3);
#pragma unroll
      for (int nd = 0; nd < 8; ++nd) {
        const av4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_av4i16*)(vlo + 16 * (nd ^ (vr & 7))));
        const av4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_av4i16*)(vhi + 16 * (nd ^ ((vr + 16) & 7))));
        const uint4 vv = make_uint4(__builtin_bit_cast(uint2, lo).x, __builtin_bit_cast(uint2, lo).y,
                                    __builtin_bit_cast(uint2, hi).x, __builtin_bit_cast(uint2, hi).y);
        o[0][nd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(vv), as_bf16x8(pb[0][kk]), o[0][nd], 0, 0, 0);
        o[1][nd] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(vv), as_bf16x8(pb[1][kk]), o[1][nd], 0, 0, 0);
      }
    }
    lds_dma_wait();  // this wavefront's next-block loads have landed ...
    __syncthreads();  // ... and, past the barrier, every wavefront's
  }

  // ---- normalise and write: rows 16 mt + r (query r of tile mt) x 128 dims through LDS (bf16,
  // 4 dims per 8-byte store), then 16-byte global stores (the K / V buffers are free: every
  // wavefront passed the loop's last barrier)
  bf16_t* ot = &sm.ot[wave][0][0];
#pragma unroll
  for (int mt = 0; mt < 2; ++mt) {
    const float inv = 1.f / xlane_sum4(l[mt]);
#pragma unroll
    for (int nd = 0; nd < 8; ++nd)
      *reinterpret_cast<uint2*>(ot + (16 * mt + rr) * AKROW + 16 * nd + 4 * qq) =
          make_uint2(f2bf2(o[mt][nd][0] * inv, o[mt][nd][1] * inv), f2bf2(o[mt][nd][2] * inv, o[mt][nd][3] * inv));
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int cidx = lane + 64 * it;     // 32 rows x 16 chunks
    const int row = cidx >> 4, ch = cidx & 15;
    const int t = t_lo + 8 * wave + (row >> 2);
    if (t < T) {
      const uint4 v = *reinterpret_cast<const uint4*>(ot + row * AKROW + ch * 8);
      bf16_t* dst = p.out + ((b * T + t) * Nq + kvh * AG + (row & 3)) * (long long)AD + ch * 8;
      *reinterpret_cast<uint4*>(dst) = v;
    }
  }
}
}  // namespace

extern "C" {

int qwen_gemm(const void* a, const void* w_tiled, void* out, int M, int N, int K, int ld_out, const void* residual,
              int epi, hipStream_t stream) {
  if (!a || !w_tiled || !out) return QWEN_ENULL;
  if (M < 0 || N <= 0 || K <= 0 || N % PBN || K % PBK || epi < PEPI_STORE || epi > PEPI_SWIGLU) return QWEN_EARG;
  const int ncols = epi == PEPI_SWIGLU ? N / 2 : N;
  if (ld_out < ncols || ld_out % 8) return QWEN_EARG;
  if (epi == PEPI_RES && !residual) return QWEN_ENULL;
  if (M == 0) return QWEN_OK;
  if ((long long)M * K >= 0x7fffffffLL) return QWEN_EARG;
  PfGemmParams p{};
  p.a = (const bf16_t*)a;
  p.w = (const bf16_t*)w_tiled;
  p.res = (const bf16_t*)residual;
  p.out = (bf16_t*)out;
  p.M = M; p.N = N; p.K = K; p.ldo = ld_out;
  const bool wide = N % PWN == 0;
  p.mtiles = (M + (wide ? PWM : PBM) - 1) / (wide ? PWM : PBM);
  p.ntiles = N / (wide ? PWN : PBN);
  long long blocks = (long long)p.mtiles * p.ntiles;
  if (blocks > 0x7fffffffLL) return QWEN_EARG;
  if (wide) {  // persistent: one workgroup per CU (8 per XCD round), at most one per tile of an XCD's run
    const long long per_xcd = (blocks + 7) / 8;
    blocks = 8 * std::min<long long>(per_xcd, std::max(1, device_cu_count() / 8));
  }
  const dim3 grid((unsigned)blocks);
  if (wide) {
    if (epi == PEPI_STORE) pf_gemm_wide_kernel<PEPI_STORE, PWV><<<grid, 64 * PWV, 0, stream>>>(p);
    else if (epi == PEPI_RES) pf_gemm_wide_kernel<PEPI_RES, PWV><<<grid, 64 * PWV, 0, stream>>>(p);
    else pf_gemm_wide_kernel<PEPI_SWIGLU, PWV><<<grid, 64 * PWV, 0, stream>>>(p);
    QWEN_RETURN_LAUNCH();
  }
  if (epi == PEPI_STORE) pf_gemm_kernel<PEPI_STORE><<<grid, 256, 0, stream>>>(p);
  else if (epi == PEPI_RES) pf_gemm_kernel<PEPI_RES><<<grid, 256, 0, stream>>>(p);
  else pf_gemm_kernel<PEPI_SWIGLU><<<grid, 256, 0, stream>>>(p);
  QWEN_RETURN_LAUNCH();
}

int qwen_attn_prefill(const void* q, const void* k_cache, const void* v_cache, void* out, int B, int T, int Nq,
                      int Nkv, int D, int CAP, int p0, float scale, hipStream_t stream) {
  if (!q || !k_cache || !v_cache || !out) return QWEN_ENULL;
  if (D != AD || Nkv <= 0 || Nq != AG * Nkv || B < 0 || T < 0 || p0 < 0 || CAP <= 0) return QWEN_EARG;
  if ((long long)p0 + T > CAP) return QWEN_EARG;
  if (B == 0 || T == 0) return QWEN_OK;
  PfAttnParams p{};
  p.q = (const bf16_t*)q;
  p.kc = (const bf16_t*)k_cache;
  p.vc = (const bf16_t*)v_cache;
  p.out = (bf16_t*)out;
  p.T = T; p.Nkv = Nkv; p.CAP = CAP; p.p0 = p0;
  const bool wide = T > AQ;   // one 16-token workgroup per head group suffices for short chunks
  p.qblocks = wide ? (T + AQ2 - 1) / AQ2 : (T + AQ - 1) / AQ;
  p.bh_count = (long long)B * Nkv;
  p.scale = scale;
  const long long blocks = p.bh_count * p.qblocks;
  if (blocks > 0x7fffffffLL) return QWEN_EARG;
  if (wide) pf_attn_wide_kernel<<<dim3((unsigned)((blocks + 7) / 8 * 8)), AW2 * 64, 0, stream>>>(p);  // 8 equal runs
  else pf_attn_kernel<<<dim3((unsigned)blocks), 256, 0, stream>>>(p);
  QWEN_RETURN_LAUNCH();
}

}  // extern "C"
