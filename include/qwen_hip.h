/*
 * C ABI of libqwen_hip.so: the MI355X (gfx950) kernels behind the Qwen3-4B
 * greedy-decode engine.
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated otherwise; bf16 tensors
 *     are raw 16-bit patterns, row-major and contiguous.
 *   - Every entry point enqueues work on `stream` and returns immediately; it
 *     never allocates, frees or synchronises, so it can be recorded into a
 *     HIP graph. Return value: 0 on success, 1001 (bad size/shape argument),
 *     1002 (null pointer), 1003 (workspace too small), 1004 (request larger
 *     than an allocation-free entry point's fixed scratch), otherwise the
 *     hipError_t of the failed launch.
 *   - "Tiled" weights use the MFMA-B tile layout written by
 *     qwen_tile_weight / qwen_init_weight: tile (nt, kt) of 16 rows x 32
 *     columns is 1 KB at element offset (nt * K/32 + kt) * 512, and lane
 *     l = 16*q + r of a tile holds W[16*nt + r][32*kt + 8*q .. +8].
 *
 * Each declaration names the reference interface it replaces
 * (paths relative to the reference repository).
 */
#ifndef QWEN_HIP_H
#define QWEN_HIP_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* rms_norm(x, w, eps) -> y.  x, y: [M, N] bf16; w: [N] bf16; N % 8 == 0, N <= 8192.
 * Replaces engine/kernels/rmsnorm.py:141-167 (rms_norm) / torch_ref.py:47-58. */
int qwen_rms_norm(const void* x, const void* w, void* y, int M, int N, float eps, hipStream_t stream);

/* add_rms_norm(x, r, w, eps) -> (h, y): h = bf16(x + r), y = rms_norm(h).
 * Replaces engine/kernels/rmsnorm.py:170-207 (add_rms_norm) / torch_ref.py:61-68. */
int qwen_add_rms_norm(const void* x, const void* r, const void* w, void* h, void* y, int M, int N, float eps,
                      hipStream_t stream);

/* silu_mul(gu [M, 2I]) -> out [M, I] = bf16(bf16(silu(gate)) * up).
 * Replaces engine/kernels/silu.py:95-125 (silu_mul) / torch_ref.py:74-88. */
int qwen_silu_mul(const void* gu, void* out, int M, int I, hipStream_t stream);

/* qk_norm_rope_cache(qkv [B*T, (Nq+2Nkv)*D], q_norm_w [D], k_norm_w [D], eps, cos/sin [P, D],
 * positions [B] int32, T, k_cache/v_cache [B, Nkv, CAP, D]) -> q_out [B, T, Nq, D];
 * writes K (normed + RoPE) and V at slots positions[b] + t (P = rows of the cos/sin tables;
 * a slot outside [0, min(CAP, P)) is skipped, never written). D must be 128, and every
 * tensor pointer 16-byte aligned (QWEN_EARG otherwise).
 * Replaces engine/kernels/rope.py:169-226 (qk_norm_rope_cache) / torch_ref.py:107-162. */
int qwen_qk_norm_rope_cache(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                            const void* sin_tab, const int32_t* positions, void* q_out, void* k_cache, void* v_cache,
                            int B, int T, int Nq, int Nkv, int D, int CAP, int P, float eps, hipStream_t stream);

/* Workspace bytes for qwen_attn_decode / qwen_attn_decode_fused with the given split count
 * (0 for num_splits == 1). The workspace holds the split partials and one arrival counter per
 * (sequence, KV head, query); it must be zero before its first use and every launch leaves the
 * counters at zero again, so one buffer serves any number of launches on one stream. */
long long qwen_attn_workspace_bytes(int B, int T, int Nq, int Nkv, int D, int num_splits);

/* attn_decode(q [B, T, Nq, D], caches [B, Nkv, CAP, D], lengths [B] int32, scale, num_splits)
 * -> out [B, T, Nq*D]. The valid length of sequence b is lengths[b] + len_add (len_add = 0
 * gives the reference semantics). Nq == 4 * Nkv, D == 128, 1 <= T <= 16; waves (1|2|4|8)
 * wavefronts per workgroup split each context split further.
 * Replaces engine/kernels/attention.py:278-348 (attn_decode) / torch_ref.py:168-227. */
int qwen_attn_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* lengths, int len_add,
                     void* out, void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D,
                     int CAP, float scale, int num_splits, int waves, hipStream_t stream);

/* The decode step's qk_norm_rope_cache + attn_decode in one launch: q heads are RMS-normed
 * (q_norm_w) and rotated from qkv [B*T, (Nq+2Nkv)*D]; the T new keys at positions[b] + t are
 * normed (k_norm_w), rotated and consumed from qkv and, with the raw V, written to the caches;
 * lengths are positions[b] + T. cos/sin: [P, D] bf16 tables.
 * Replaces engine/kernels/rope.py:169-226 followed by engine/kernels/attention.py:278-348
 * (the two ops of engine/engine.py:1110-1113). */
int qwen_attn_decode_fused(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                           const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                           void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D, int CAP,
                           int P, float eps, float scale, int num_splits, int waves, hipStream_t stream);

/* Workspace bytes for qwen_attn_decode_mfma with the given split count (0 for num_splits == 1):
 * one arrival counter per (sequence, KV head) and the split partials. Same life cycle as
 * qwen_attn_workspace_bytes: zero before first use, every launch re-arms the counters. */
long long qwen_attn_mfma_workspace_bytes(int B, int T, int Nkv, int num_splits);

/* qwen_attn_decode_fused on the matrix cores: same operator, arguments and effects, for
 * 1 <= T <= 8, 1 <= num_splits <= 8 and B <= 65535. One workgroup per (KV head, split, sequence) serves
 * all T * 4 query rows of the KV head (each cache byte read once per launch); QK^T and PV run
 * on v_mfma_f32_16x16x32_bf16; waves (4|8) wavefronts split each context split further.
 * Replaces engine/kernels/rope.py:169-226 followed by engine/kernels/attention.py:278-348
 * (the two ops of engine/engine.py:1110-1113). */
int qwen_attn_decode_mfma(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                          const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                          void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D, int CAP,
                          int P, float eps, float scale, int num_splits, int waves, hipStream_t stream);

/* qwen_attn_decode_mfma with launch flags (flags == 0 is exactly that entry point). Bit 0
 * (QWEN_ATTN_KV_CACHED): read the cached keys and values with ordinary, cache-allocating loads
 * instead of non-temporal ones, for a whole KV cache small enough to stay in the Infinity
 * Cache between steps. Other bits are rejected. Results do not depend on the flags. No
 * reference counterpart (a load-policy choice). */
int qwen_attn_decode_mfma_ex(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                             const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache, void* out,
                             void* workspace, long long workspace_bytes, int B, int T, int Nq, int Nkv, int D,
                             int CAP, int P, float eps, float scale, int num_splits, int waves, int flags,
                             hipStream_t stream);

/* Fixed scratch of qwen_attn_decode_mfma_noalloc, per GPU (bytes). */
#define QWEN_ATTN_NOALLOC_SCRATCH_BYTES (8LL << 20)

/* qwen_attn_decode_mfma_ex without the workspace arguments: the split partials and arrival
 * counters live in a fixed device array of QWEN_ATTN_NOALLOC_SCRATCH_BYTES per GPU (held until
 * the process ends), so the call allocates nothing: no hipMalloc, hipFree or allocating library
 * routine, and its counters are cleared by a kernel (not hipMemsetAsync), so it may be recorded
 * into a HIP graph. A launch whose qwen_attn_mfma_workspace_bytes(B, T, Nkv, num_splits) exceeds
 * that size returns 1004 and launches nothing. Every call on one GPU shares its array: calls that
 * overlap on one GPU (on different streams) race. No counterpart in the reference; it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). */
int qwen_attn_decode_mfma_noalloc(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_tab,
                                  const void* sin_tab, const int32_t* positions, void* k_cache, void* v_cache,
                                  void* out, int B, int T, int Nq, int Nkv, int D, int CAP, int P, float eps,
                                  float scale, int num_splits, int waves, int flags, hipStream_t stream);

/* Per-16-column partial sums of squares of a [M, K] bf16 matrix: psq[m, u] =
 * sum_{j<16} x[m, 16u + j]^2 in fp32. These are the RMSNorm statistics the normed
 * projections consume (psq_in below). No reference counterpart: it is the first
 * half of the reference's RMSNorm (rmsnorm.py:91-93) split out so that producers
 * can emit it. */
int qwen_sumsq16(const void* x, float* psq, int M, int K, hipStream_t stream);

/* Workspace bytes for qwen_linear with ks > 1 (0 for ks == 1): split-K partials plus one
 * arrival counter per n-tile group; zero before first use, left at zero by every launch. */
long long qwen_linear_workspace_bytes(int M, int N, int ntw, int ks);

/* out = x @ W^T with optional RMSNorm prologue (norm_w != NULL; psq_in = x's
 * qwen_sumsq16 partials [M, K/16]) and epilogue
 * epi = 0 store, 1 residual add (out = bf16(residual + bf16(acc)); residual may alias out;
 * psq_out != NULL also writes the new rows' [M, N/16] partials),
 * 2 SwiGLU pair (W tiled with pair interleave; N = 2I rows; out has I columns).
 * x: [M, K] (M <= 32), W tiled [N, K]. Launch shape: ntw (1|2|4) n-tiles per workgroup,
 * waves (4|8|16) wavefronts per workgroup, ks k-splits across workgroups (ks > 1 needs the
 * workspace). Replaces the projections of engine/engine.py:1108-1118 (_mm / F.linear) and
 * engine/kernels/gemm_fused.py:136-173 (fused_linear). */
int qwen_linear(const void* x, const void* w_tiled, void* out, int M, int N, int K, int ld_out, const void* norm_w,
                const float* psq_in, float eps, const void* residual, float* psq_out, int epi, int ntw, int waves,
                int ks, void* workspace, long long workspace_bytes, hipStream_t stream);

/* qwen_linear for 1 <= M <= 32 with the rectangle decomposition: the (unit of 16*ntw weight
 * rows, k-step of 32) plane is cut into gn x gk equal rectangles, one workgroup of wpg (8|16)
 * wavefronts each; a workgroup stages its k-range of the (normed) activations in LDS once and
 * streams its rectangle's weight tiles. ntw = 2 exactly for the SwiGLU pair epilogue (epi 2),
 * else 1. Same operands, epilogues and rounding as qwen_linear; with gk > 1 the workspace is
 * qwen_linear_workspace_bytes(M, N, ntw, gk) bytes (counters re-armed by every launch).
 * Replaces engine/kernels/gemm_fused.py:136-173 (the fused projections of engine/engine.py:1103-1118). */
int qwen_linear_rect(const void* x, const void* w_tiled, void* out, int M, int N, int K, int ld_out,
                     const void* norm_w, const float* psq_in, float eps, const void* residual, float* psq_out,
                     int epi, int ntw, int wpg, int gn, int gk, void* workspace, long long workspace_bytes,
                     hipStream_t stream);

/* Dynamic LDS bytes of a qwen_gemv launch shape (0 = unsupported shape). */
long long qwen_gemv_lds_bytes(int M, int N, int K, int grid, int waves, int epi);

/* Balanced GEMV for M <= 2 rows over a ROW-MAJOR weight (HF nn.Linear layout [N, K]):
 * out = x @ W^T with optional RMSNorm prologue (norm_w != NULL; the row statistics are
 * computed in the kernel from x itself) and epilogue epi = 0 store, 1 residual add
 * (out = bf16(residual + bf16(acc)), residual may alias out), 2 SwiGLU (W = cat(gate, up)
 * rows [2N, K]; out = bf16(bf16(silu(bf16(g))) * bf16(u)), N columns), 3 argmax of the bf16
 * logits folded into slot 0 of row m's key in amax (the key buffer of qwen_lm_head_argmax,
 * QWEN_ARGMAX_KEYS(M) words; out unused).
 * Workgroup g of `grid` owns output rows [N*g/grid, N*(g+1)/grid), so every CU streams the
 * same bytes; K must be a multiple of 512; waves 8 or 16. Same operator contract as
 * qwen_linear / qwen_lm_head_argmax: replaces the projections of engine/engine.py:1108-1121
 * (_mm / F.linear, fused_linear of engine/kernels/gemm_fused.py:136-173, lm_head + argmax). */
int qwen_gemv(const void* x, const void* w, void* out, int M, int N, int K, int ld_out, const void* norm_w, float eps,
              const void* residual, int epi, unsigned long long* amax, int grid, int waves, hipStream_t stream);

/* qwen_gemv with the store epilogue (epi = 0) writing weight row i's output to column
 * row_map[i] (a permutation of [0, N), int32 on the device; row_map == NULL is qwen_gemv).
 * No reference counterpart: it lets a caller permute a weight's rows to choose which
 * workgroup, and so which XCD, produces each output column while the output keeps its
 * natural layout. */
int qwen_gemv_rowmap(const void* x, const void* w, void* out, int M, int N, int K, int ld_out, const void* norm_w,
                     float eps, const void* residual, int epi, unsigned long long* amax, const int32_t* row_map,
                     int grid, int waves, hipStream_t stream);

/* Packed argmax keys of an M-row LM head: QWEN_ARGMAX_SLOTS slots per row, slot s of row m at
 * amax[s * QWEN_ARGMAX_LD(M) + m] (uint64: monotone logit bits << 32 | ~index); the row's key
 * is the maximum over its slots. A key buffer holds QWEN_ARGMAX_KEYS(M) words, zero before a
 * producer runs; every consumer re-arms all slots of the rows it reads. */
#define QWEN_ARGMAX_SLOTS 8
#define QWEN_ARGMAX_LD(M) (((M) + 15) / 16 * 16)
#define QWEN_ARGMAX_KEYS(M) (QWEN_ARGMAX_SLOTS * QWEN_ARGMAX_LD(M))

/* Final RMSNorm + tied LM head + argmax over the bf16 logits (lowest index on ties):
 * token[m] = argmax_n bf16((rms_norm(x[m]) @ W^T)[n]); psq_in = x's qwen_sumsq16 partials.
 * The result is folded into the key buffer amax (QWEN_ARGMAX_KEYS(M) words, workgroup g
 * into slot g % QWEN_ARGMAX_SLOTS); with out_tok != NULL the tokens are extracted into out_tok
 * [M] int64 and amax re-armed, otherwise qwen_decode_finish / qwen_argmax_extract consume it.
 * Replaces engine/engine.py:1119-1121 (final add_rms_norm, lm_head _mm, argmax). */
int qwen_lm_head_argmax(const void* x, const void* norm_w, const float* psq_in, float eps, const void* w_tiled, int M,
                        int N, int K, unsigned long long* amax, int64_t* out_tok, int ntw, int waves,
                        hipStream_t stream);

/* out[m] = token index held in row m's key of amax (QWEN_ARGMAX_KEYS(M) words, from
 * qwen_lm_head_argmax or qwen_gemv); re-arms the key buffer to zero.
 * Replaces the argmax(-1) read-out of engine/engine.py:1121. */
int qwen_argmax_extract(unsigned long long* amax, int M, int64_t* out, hipStream_t stream);

/* Embedding gather from the tiled tied table: out[m] = W[tok[m]], or, with tok == NULL,
 * out[m] = W[hist[m, pos[m]]] (the decode step's token read, engine/engine.py:941-946).
 * psq_out != NULL also writes the rows' qwen_sumsq16 partials. Ids are clamped to [0, V).
 * Replaces F.embedding at engine/engine.py:1101. */
int qwen_embed(const int64_t* tok, const int64_t* hist, const int32_t* pos, int cap, const void* w_tiled, void* out,
               float* psq_out, int M, long long V, int K, hipStream_t stream);

/* Step tail after the LM head: token[b] = index held in row b's key of amax (QWEN_ARGMAX_KEYS(B)
 * words, re-armed to zero) -> next[b];
 * hist[b, pos[b]+1] = token[b], pos[b] += 1, frozen rows ((pos+1 - s_buf) >= ntarget) write slot
 * cap-1 and keep pos; then h[b] = W[hist[b, pos[b]]] from the tiled table and psq its
 * qwen_sumsq16 partials (the next step's input). Replaces the tail of engine/engine.py:941-953
 * (_plain_step) and the embedding of engine/engine.py:1101. */
int qwen_decode_finish(unsigned long long* amax, int64_t* next, int64_t* hist, int32_t* pos, const int64_t* s_buf,
                       const int64_t* ntarget, const void* w_tiled, void* h, float* psq, int B, int cap, long long V,
                       int K, hipStream_t stream);

/* Prompt-lookup draft for a speculative verify step: for each sequence b with L = pos[b] + 1
 * valid history tokens, the latest start i < L - n with hist[b, i..i+n-1] == hist[b, L-n..L-1]
 * (i = -1 if none) gives tok_out[b] = [hist[b, L-1], hist[b, clamp(i+n+j, 0, L-1)] for j < k]
 * ([B, k+1] int64). 1 <= k <= 15, 1 <= n <= 8. Replaces engine/engine.py:955-977 (_spec_draft). */
int qwen_spec_draft(const int64_t* hist, const int32_t* pos, int B, int cap, int k, int n, int64_t* tok_out,
                    hipStream_t stream);

/* Acceptance of a verify step of T = k+1 tokens: nxt [B*T] (greedy token after each fed prefix),
 * tok [B, T] (fed ids). adv[b] = 1 + (leading drafts equal to the model's tokens), 0 for rows that
 * already produced their tokens ((pos+1 - s_buf) >= ntarget); hist[b, pos[b]+1+j] = nxt[b, j] for
 * j < adv (other positions to the dump slot cap-1); pos[b] += adv; out_t [T, B] = nxt transposed;
 * then h[b] = W[hist[b, pos[b]]] from the tiled table and psq its qwen_sumsq16 partials (a plain
 * step may follow). Replaces engine/engine.py:994-1003 (the tail of _spec_step). */
int qwen_spec_accept(const int64_t* nxt, const int64_t* tok, int64_t* hist, int32_t* pos, const int64_t* s_buf,
                     const int64_t* ntarget, int B, int cap, int T, int64_t* out_t, int64_t* adv_out,
                     const void* w_tiled, void* h, float* psq, long long V, int K, hipStream_t stream);

/* Prompt-forward projection: out = x @ W^T for any M over a tiled weight, fp32 accumulation,
 * epilogue epi = 0 store (bf16(acc)), 1 residual add (out = bf16(residual + bf16(acc));
 * residual may alias out), 2 SwiGLU (pair-interleaved gate|up weight of N = 2I rows; out has
 * I columns: bf16(bf16(silu(bf16(g))) * bf16(u))). x: [M, K] row-major with M * K < 2^31;
 * N % 128 == 0, K % 64 == 0; out / residual: [M, ld_out], ld_out % 8 == 0.
 * Replaces the prompt forward's projections, engine/engine.py:1191-1221 (_mm / cuBLAS on
 * B*S rows) with the fused epilogues of engine/kernels/gemm_fused.py:136-173. */
int qwen_gemm(const void* x, const void* w_tiled, void* out, int M, int N, int K, int ld_out, const void* residual,
              int epi, hipStream_t stream);

/* Causal attention of a prompt chunk: q [B, T, Nq, D] (normed + rotated queries of positions
 * p0 .. p0 + T - 1 of every sequence), caches [B, Nkv, CAP, D] already holding those
 * positions' keys / values; query t sees slots [0, p0 + t]. out [B, T, Nq * D] bf16.
 * Nq == 4 * Nkv, D == 128, p0 + T <= CAP. Rounding points of the decode attention
 * (fp32 scores * scale, bf16 probabilities for PV, fp32 sums, one final rounding).
 * Replaces engine/engine.py:1123-1179 (_prefill_attention: SDPA flash, causal, GQA). */
int qwen_attn_prefill(const void* q, const void* k_cache, const void* v_cache, void* out, int B, int T, int Nq,
                      int Nkv, int D, int CAP, int p0, float scale, hipStream_t stream);

/* Row-major [N, K] bf16 -> tiled layout (pair = 1: gate|up interleave, tile 2p = rows
 * 16p.., tile 2p+1 = rows N/2 + 16p..). Replaces the weight fusion / layout step of
 * engine/engine.py:209-227 (the reference keeps row-major; this build re-lays for MFMA). */
int qwen_tile_weight(const void* src, void* dst, long long N, int K, int pair, hipStream_t stream);

/* Fill a [N, K] weight (tiled != 0: tiled layout) from the counter-based random-init
 * generator: nseg row segments starting at seg_start[i] (host array, ascending, first 0)
 * drawn from tensor ids seg_tid[i]; element = bf16(f32(IrwinHall4(splitmix64(seed<<52 |
 * tid<<32 | local_index)) - 131070) * scale). No reference counterpart: the benchmark
 * configs' "random-init weights from seed 0" (HF init would run on the host). */
int qwen_init_weight(void* dst, long long N, int K, int tiled, int pair, const int* seg_start, const int* seg_tid,
                     int nseg, unsigned long long seed, float scale, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_HIP_H */
