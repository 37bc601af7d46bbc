// The decode step's QKV projection and attention in one launch, for M <= 2 rows (T = 1).
//
// Same operators as the two launches they replace: the RMSNorm + QKV GEMV over the head-major
// QKV weight (qwen_gemv_rowmap with 8 row groups; engine/engine.py:1104-1108) and the matrix-
// core decode attention with QK-norm, RoPE and the K/V write (qwen_attn_decode_mfma;
// engine/engine.py:1110-1113). The arithmetic, rounding points and summation orders are those
// of the two kernels (their bodies are compiled in here), so the results are bit-identical.
//
// Grid: exactly 256 workgroups, one per CU, so all are resident at once (the static attention
// LDS plus the GEMV's staging keep one workgroup per CU). Workgroups [0, na) are the attention
// workgroups, na = B * Nkv * splits, number w serving (sequence, KV head) w mod (B * Nkv) and
// split w / (B * Nkv); the other 256 - na project the QKV rows, 8 row groups of (256 - na) / 8
// workgroups. Workgroup i runs on XCD i mod 8 and na is a multiple of 8, so with Nkv = 8 the
// attention workgroups of KV head h and the projection workgroups of head group h (its q, k
// and v rows) share XCD h, and the rows pass through that XCD's L2. An attention workgroup
// first requests everything that does not depend on the projection (RoPE table rows, gains,
// its first cached K / V block), then waits until its head group's projection workgroups have
// stored their rows and raised their generation flags (QkvSync: a bounded wait that sets an
// error word on expiry), reads the rows from the L2 and finishes as the standalone kernel
// does. The attention workgroups check that the producers they waited for ran on their own XCD
// (the producers record their XCC ids) and set the error word otherwise, so a dispatch that
// breaks the placement cannot pass unnoticed.
// Projection workgroups never wait, so the launch completes whatever the dispatch order.
//
// Measured on Qwen3-4B at B = 1 (36 layers, median per layer): the projection's last row is
// stored 7.7 us after the launch starts, the waits end at 11.5 us (a flag poll is one L2 round
// trip, ~1.9 us while the projection streams its weights; sc0|nt, sc1 and invalidate-then-load
// polls all measure the same), and the launch ends at 15.4 us. That is longer than the two
// launches it replaces, so the engine uses it only when asked to.
#include "gemv_impl.h"
#include "attention_mfma_impl.h"

extern "C" long long qwen_attn_mfma_workspace_bytes(int B, int T, int Nkv, int num_splits);

namespace {

constexpr int QA_GRID = 256;            // workgroups of a launch: one per CU of an MI355X
constexpr int QA_GROUPS = 8;            // KV head groups = XCDs
constexpr long long QA_SYNC_BYTES = 4096;  // pflag[256], cflag[64], pxcc[256], err (the workspace's last 4 KB)
constexpr int QA_SPIN = 1 << 18;        // polls before a wait gives up (a poll is about one L2 round trip: ~0.2 s)

template <int M, bool KVC>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2)))
qkv_attn_kernel(GemvParams gp, MfmaAttnParams ap, QkvSync qs, int na) {
  extern __shared__ __align__(16) unsigned char gv_smem[];
  const int w = blockIdx.x;
  if (w < na) {
    const int nbh = M * ap.Nkv;
    attn_mfma_body<1, 8, KVC, true>(ap, w % nbh, w / nbh, qs);
  } else {
    gemv_body<M, 8, true, GEPI_STORE, true>(gp, gv_smem, w - na, QA_GRID - na, &qs);
  }
}

long long qa_attn_bytes(int B, int Nkv, int S) {
  const long long a = qwen_attn_mfma_workspace_bytes(B, 1, Nkv, S);
  return (a + 255) / 256 * 256;
}

}  // namespace

extern "C" {

long long qwen_qkv_attn_workspace_bytes(int B, int Nkv, int num_splits) {
  if (B < 1 || B > 2 || Nkv != QA_GROUPS || num_splits < 1 || num_splits > MERGE_MAX) return 0;
  if ((long long)B * Nkv * num_splits > 64) return 0;
  return qa_attn_bytes(B, Nkv, num_splits) + QA_SYNC_BYTES;
}

int qwen_qkv_attn_decode(const void* x, const void* w_qkv, const void* ln1, const int32_t* row_map, float eps,
                         void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                         const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                         void* workspace, long long workspace_bytes, int B, int H, int Nq, int Nkv, int D, int CAP,
                         int P, float scale, int num_splits, int flags, hipStream_t stream) {
  if (!x || !w_qkv || !ln1 || !row_map || !qkv || !workspace) return QWEN_ENULL;
  if (flags & ~QWEN_ATTN_KV_CACHED) return QWEN_EARG;
  if (B < 1 || B > 2 || Nkv != QA_GROUPS || Nq != MG * Nkv || D != MD) return QWEN_EARG;
  if (H <= 0 || H % GV_CHUNK || (long long)B * (H / 8) > (long long)GV_XC_NORM * 64 * 8) return QWEN_EARG;
  const long long need = qwen_qkv_attn_workspace_bytes(B, Nkv, num_splits);
  if (need == 0) return QWEN_EARG;
  if (workspace_bytes < need) return QWEN_EWORKSPACE;
  const int st = mfma_args_status(qkv, q_norm_w, k_norm_w, cos_tab, sin_tab, positions, k_cache, v_cache, out, B, 1,
                                  Nq, Nkv, D, CAP, P, num_splits, 8, flags);
  if (st != QWEN_OK) return st;
  const int N = (Nq + 2 * Nkv) * D;
  const int na = B * Nkv * num_splits;
  const int G = QA_GRID - na;
  const size_t lds = gemv_lds_bytes(B, N, H, G, 8, GEPI_STORE);

  GemvParams gp{(const bf16_t*)x, (const bf16_t*)w_qkv, (const bf16_t*)ln1, nullptr, (bf16_t*)qkv, nullptr, row_map,
                N, H, N, eps, QA_GROUPS};
  MfmaAttnParams ap{};
  ap.qkv = (const bf16_t*)qkv;
  ap.qnw = (const bf16_t*)q_norm_w;
  ap.knw = (const bf16_t*)k_norm_w;
  ap.cos_tab = (const bf16_t*)cos_tab;
  ap.sin_tab = (const bf16_t*)sin_tab;
  ap.pos = positions;
  ap.kc = (bf16_t*)k_cache;
  ap.vc = (bf16_t*)v_cache;
  ap.out = (bf16_t*)out;
  const long long bh = (long long)B * Nkv;
  ap.cnt = num_splits > 1 ? (unsigned*)workspace : nullptr;
  ap.part = num_splits > 1 ? (float*)((char*)workspace + mfma_counter_bytes(bh)) : nullptr;
  ap.T = 1; ap.Nkv = Nkv; ap.CAP = CAP; ap.P = P; ap.S = num_splits;
  ap.scale = scale; ap.eps = eps;
  ap.kv_cached = (flags & QWEN_ATTN_KV_CACHED) ? 1 : 0;
  unsigned* sync = (unsigned*)((char*)workspace + qa_attn_bytes(B, Nkv, num_splits));
  const QkvSync qs{sync, sync + QA_GRID, sync + QA_GRID + 64, sync + 2 * QA_GRID + 64, G / QA_GROUPS, QA_SPIN};

  if (B == 1) {
    if (ap.kv_cached) qkv_attn_kernel<1, true><<<QA_GRID, 512, lds, stream>>>(gp, ap, qs, na);
    else qkv_attn_kernel<1, false><<<QA_GRID, 512, lds, stream>>>(gp, ap, qs, na);
  } else {
    if (ap.kv_cached) qkv_attn_kernel<2, true><<<QA_GRID, 512, lds, stream>>>(gp, ap, qs, na);
    else qkv_attn_kernel<2, false><<<QA_GRID, 512, lds, stream>>>(gp, ap, qs, na);
  }
  QWEN_RETURN_LAUNCH();
}

}  // extern "C"
