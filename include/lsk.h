/* liblsk: C ABI of the MI355X (gfx950) kernels behind the packed ragged LayerSkip-Llama forward.
 *
 * The reference (hsungo/thesis) is pure PyTorch; it has no native ABI.  Each entry point below
 * replaces the eager torch ops of one step of its hot path, cited as file:line of the reference.
 *
 * Conventions
 *   - dtype codes: LSK_DTYPE_F32 (0) and LSK_DTYPE_BF16 (1); bf16 is torch.bfloat16 storage.
 *   - All pointers are device pointers unless stated; the library never allocates or frees
 *     device memory: tensors and workspaces belong to the caller (the PyTorch caching allocator).
 *   - `stream` is a hipStream_t; every call is asynchronous on it, nothing synchronises inside.
 *   - Return value: 0 = ok, < 0 = argument error detected on the host before any launch
 *     (LSK_EARG, LSK_ESHAPE, LSK_EUNSUPPORTED, LSK_EWORKSPACE), > 0 = hipError_t of the launch.
 *     lsk_last_error() returns the message of the calling thread's last error.
 *   - Index arrays are int32 unless stated; token ids and sequence buffers are int64 (torch.long).
 */
#ifndef LSK_H_
#define LSK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LSK_ABI_VERSION 11

#define LSK_EPI_NONE 0     /* C = rnd(A W^T)                                   */
#define LSK_EPI_RESIDUAL 1 /* C = rnd(R + rnd(A W^T))                          */
#define LSK_EPI_SILU_MUL 2 /* C = rnd(rnd(silu(rnd(g))) * rnd(u)), [g;u] = A W^T */

#define LSK_ATTN_SPLIT 8192 /* KV positions per flash-decoding split of large bf16 caches */

const char* lsk_last_error(void);
int lsk_abi_version(void);

/* RMSNorm: out = w * (x * rsqrt(mean(x^2) + eps)).to(dtype).
 * Replaces common/model.py:153-156 (rms_norm), used at solutions/packed.py:175,183 and common/model.py:330. */
int lsk_rmsnorm(int dtype, const void* x, const void* w, void* out, int n_rows, int dim, float eps, long ldx,
                long ldo, void* stream);

/* RoPE of q and k + KV append: qkv [N, (Hq+2Hkv)D] -> q_out [N, Hq, D], k into the K cache (bf16
 * fragment-major [B, Hkv, S/32, D/16, 64, 8], fp32 [B, Hkv, S, D]) and v into the V cache at (rows[t], pos[t]).  The V cache is stored in 32-position blocks,
 * each block transposed: [B, Hkv, S/32, D, 32] (S a multiple of 64).  cos/sin tables: fp32 [tab_len, D] (device).
 * Replaces solutions/packed.py:176-181 (split, apply_rope, cache index_put) with
 * common/model.py:143-150 (apply_rope) and solutions/packed.py:106-107 (cos/sin gather + cast). */
int lsk_rope_append(int dtype, const void* qkv, void* q_out, void* kcache, void* vcache, const float* cos_tab,
                    const float* sin_tab, int tab_len, const int32_t* rows, const int32_t* pos, int n_tokens,
                    int n_heads, int n_kv_heads, int head_dim, int max_batch, int max_seq, void* stream);

/* KV append without RoPE: kcache[rows[t], :, pos[t]] = k[t]; V cache (rows[t], :, pos[t]) = v[t]
 * (K: bf16 fragment-major [B, Hkv, S/32, D/16, 64, 8] / fp32 [B, Hkv, S, D]; V blocked-transposed
 * [B, Hkv, S/32, D, 32]).  Replaces solutions/packed.py:180-181 and common/model.py:343-344. */
int lsk_kv_append(int dtype, const void* k, const void* v, void* kcache, void* vcache, const int32_t* rows,
                  const int32_t* pos, int n_tokens, int n_kv_heads, int head_dim, int max_batch, int max_seq,
                  void* stream);

/* Host-side planner for lsk_ragged_attn (host pointers, no GPU work).
 * blocks: int32 [nb][4] = {q_start, pos0, T, row}.  Writes work items int32 [n][8] (each <= rows_cap of a
 * block's T * group query rows over one KV split) and combine groups int32 [n][8]; `split` = KV positions per
 * split (LSK_ATTN_SPLIT for bf16; >= the longest context, e.g. 1<<30, for the unsplit fp32 path);
 * rows_cap = 16, 32 or 48 (lsk_attn_rows_cap; the outputs do not depend on it).  Mirrors the per-bucket
 * metadata of solutions/packed.py:109-138 (build_packed) without the dense masks. */
int lsk_attn_plan(const int32_t* blocks, int nb, int group, int split, int rows_cap, int32_t* works, int max_works,
                  int32_t* groups, int max_groups, int* n_works, int* n_groups, int* n_parts);

/* Rows per work item for a launch of these blocks over n_slots persistent workgroups (host only): 16, 32 or
 * 48, the cap with the smallest estimated time (latency-bound launches split a block's rows over more
 * workgroups, bandwidth-bound ones keep them together so the KV is read once); negative on bad arguments.
 * Has no reference counterpart (the reference runs one SDPA per bucket). */
int lsk_attn_rows_cap(const int32_t* blocks, int nb, int group, int split, int n_kv_heads, int head_dim,
                      int n_slots);

/* Static schedule of a plan's (work, KV head) items over n_slots persistent workgroups (host pointers):
 * longest first to the least-loaded slot.  Writes recs int32 [n_slots][n_rounds][8]: slot s's items in
 * processing order from round 0, each the work record with field 2 = nrows | kv_head << 8, padded with
 * all-zero records; n_rounds = the largest item count of a slot (recs == NULL: only n_rounds is written).
 * max_recs = capacity in records.  Has no reference counterpart (the reference runs one SDPA per bucket);
 * it only decides which workgroup computes an item, never the result. */
int lsk_attn_schedule(const int32_t* works, int n_works, int n_kv_heads, int n_slots, int32_t* recs, int max_recs,
                      int* n_rounds);

/* One packed segment's kernel metadata in one host call (no GPU work): blocks (rows, pos0, T; int64, nb of
 * them) already in packed order -> meta int32 [rows N][pos N][blocks nb*4][works nw*8][groups ng*8]
 * [recs n_slots*n_rounds*8], exactly what lsk_attn_rows_cap + lsk_attn_plan(split, cap) + lsk_attn_schedule
 * give, plus the token row / position expansion.  counts[11] = {N, n_works, n_groups, n_parts, n_rounds,
 * meta_len, kv_read, kv_read_padded, kv_gathered, attended (query, position) pairs, rows_cap}; the kv_* figures
 * are the reference's bucket accounting (bucketing 0 = "exact": runs of equal T, 1 = "pad": one bucket).
 * Blocks outside [0, max_batch) x [0, min(max_seq, rope_len)) are rejected with LSK_ESHAPE.  meta == NULL:
 * counts only; meta_cap too small: LSK_EWORKSPACE with counts written.  Replaces solutions/packed.py:81-139
 * (build_packed's ordering bookkeeping, metadata and accounting) for the native kernels. */
int lsk_pack_segment(const int64_t* rows, const int64_t* pos0, const int64_t* T, int nb, int group, int split,
                     int n_kv_heads, int head_dim, int n_slots, int bucketing, int max_batch, int max_seq,
                     int rope_len, int32_t* meta, long meta_cap, long* counts);

/* Workspace bytes for the split partials of a plan with n_parts partial slots. */
size_t lsk_attn_workspace_bytes(int n_parts, int n_kv_heads, int head_dim);

/* Ragged verify/decode attention: a query at position p of row r attends cache[r, :, 0..p].
 * q [N, Hq, D], K: bf16 fragment-major [B, Hkv, S/32, D/16, 64, 8] / fp32 [B, Hkv, S, D],
 * V blocked-transposed [B, Hkv, S/32, D, 32], out [N, Hq*D].  scale = 1/sqrt(D) for the reference's SDPA default.
 * bf16 runs n_slots persistent workgroups over the schedule records (recs, n_rounds); rows_cap is the cap the
 * plan was made with (16: one-tile kernel, Q in registers; 32 / 48: three-tile kernel, Q in LDS); the two
 * kernels give bitwise equal outputs.  fp32 reads works.
 * Replaces solutions/packed.py:142-166 (_attend: per-bucket gather + masked SDPA + scatter)
 * and common/model.py:352-364 (the padded path's masked SDPA). */
int lsk_ragged_attn(int dtype, const void* q, const void* kcache, const void* vcache, const int32_t* blocks,
                    const int32_t* works, int n_works, const int32_t* groups, int n_groups, int n_parts,
                    const int32_t* recs, int n_rounds, int n_slots, int rows_cap, void* out, int n_heads,
                    int n_kv_heads, int head_dim, int max_seq, float scale, void* workspace, size_t ws_bytes,
                    void* stream);

/* Allocation-free lsk_ragged_attn: the same arguments and outputs without the workspace.  The split partials live
 * in a static device array of LSK_ATTN_SCRATCH_BYTES per GPU (held until the process ends), so plans whose
 * partials need more (lsk_attn_workspace_bytes(n_parts, n_kv_heads, head_dim) > LSK_ATTN_SCRATCH_BYTES, about 170
 * partial slots at 8 KV heads x head_dim 128) are rejected with LSK_EWORKSPACE.  The current device must be the
 * stream's.  All calls on one GPU share its array: calls that overlap on one GPU (several streams or host
 * threads) race.  No hipMalloc / hipFree or other allocation happens inside.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). */
#define LSK_ATTN_SCRATCH_BYTES (32u << 20)
size_t lsk_ragged_attn_static_scratch_bytes(void);
int lsk_ragged_attn_static(int dtype, const void* q, const void* kcache, const void* vcache, const int32_t* blocks,
                           const int32_t* works, int n_works, const int32_t* groups, int n_groups, int n_parts,
                           const int32_t* recs, int n_rounds, int n_slots, int rows_cap, void* out, int n_heads,
                           int n_kv_heads, int head_dim, int max_seq, float scale, void* stream);

/* bf16 weight storage of the GEMMs: W [N, K] row-major (ldw) <-> fragment-major Wp (N*K elements, no
 * padding): fragment (g, j) = rows 16g..16g+15 x k 32j..32j+31 is 1 KiB, lane l's 8 elements being
 * W[16g + l%16][32j + 8(l/16) .. +7], fragments in [g][j] order.  N % 16 == 0, K % 32 == 0.
 * Pure copies (bit-exact both ways).  Has no reference counterpart: the reference keeps F.linear's
 * [out, in] tensors (common/model.py:259-276); the packed form is what lsk_gemm, lsk_gemm_partial,
 * lsk_head_argmax and the layer runner read for bf16, and unpacking restores the reference tensor. */
int lsk_pack_weight(const void* W, long ldw, void* Wp, int N, int K, void* stream);
int lsk_unpack_weight(const void* Wp, void* W, long ldw, int N, int K, void* stream);

/* GEMM C = epilogue(A W^T), A [M,K] (lda), W [N_w,K], C [M,N] (ldc), R residual [M,N] (ldr).
 * bf16: W is the packed storage (lsk_pack_weight) and ldw must equal K; fp32: W row-major with stride ldw.
 * For LSK_EPI_SILU_MUL, W has 2*ffn rows [gate; up] and N == ffn.
 * Replaces F.linear at solutions/packed.py:175 (wqkv), 182 (wo + residual), 183-185 (w13, silu*mul,
 * w2 + residual) and common/model.py:330 (lm_head). */
int lsk_gemm(int dtype, const void* A, long lda, const void* W, long ldw, void* C, long ldc, const void* R, long ldr,
             int M, int N, int K, int epilogue, int ffn, void* stream);

/* K-split plan of a bf16 weight shape (N rows x K): ks K slices (this fixes the per-element reduction
 * order) and ns, the 16-row-group tile width the rule is based on.  Chosen from (N, K) only, so the
 * reduction order never depends on the token count M; each launch picks its own tile width from M. */
int lsk_gemm_plan(int N, int K, int* ns_out, int* ks_out);

/* Configuration the wide-M tier (the bf16 GEMM path above 64 tokens) picks for a launch: cfg[4] = {ns (16-row
 * groups per tile; 0: the tier does not take the launch), blocks, 16-token groups per block, groups per wave}.
 * epilogue: LSK_EPI_*, or 3 = K-slice partials (lsk_gemm_partial), 4 = LM head + argmax, 5 = fused qkv + RoPE +
 * KV append; af: fragment-major A.  A query only (no launch): for tests and measurement tools to know which
 * kernel configuration a token count reaches.  Part of the lsk_gemm* family above (solutions/packed.py:175-185). */
int lsk_gemm_wide_config(int epilogue, int M, int N, int K, int ks, int af, int* cfg);

/* bf16 GEMM into fp32 K-slice partials (W packed, ldw == K): P[s][m][n] = sum over k in slice s of A[m][k] W[n][k], s < ks
 * (ks must equal lsk_gemm_plan's for this shape to keep the canonical reduction order; the consumer adds
 * the slices in order).  Replaces F.linear at solutions/packed.py:175 (wqkv), 182 (wo), 185 (w2). */
int lsk_gemm_partial(const void* A, long lda, const void* W, long ldw, float* P, int M, int N, int K, int ks,
                     void* stream);

/* Fragment-major A: A holds ceil(M/16)*16 rows x K in lsk_pack_weight's layout (16-token groups, each 16 x 32
 * block one 1 KiB fragment in lane order; the padding rows only reach discarded outputs).  These are the GEMM
 * launches lsk_forward_layers makes (its activations stay in that layout, so every row tile re-reads them as
 * contiguous 1 KiB); results are bitwise those of lsk_gemm_partial / lsk_gemm with the same values row-major.
 * lsk_gemm_silu_frag: w13 with the silu-mul epilogue, H [M, ffn] row-major (h_frag == 0, ldh = ffn) or
 * fragment-major (h_frag != 0, ceil(M/16)*16 rows).  No reference counterpart: the layer runner's internal
 * launches, exported so that measurements replay exactly those. */
int lsk_gemm_partial_frag(const void* A, const void* W, float* P, int M, int N, int K, int ks, void* stream);
int lsk_gemm_silu_frag(const void* A, const void* W, void* H, int h_frag, int M, int ffn, int K, void* stream);

/* LM head + greedy pick (W packed, ldw == K): out[dst_idx ? dst_idx[m] : m] = argmax_n rnd(A[m] . W[n]) (first index on ties),
 * optionally also storing the bf16 logits [M, ldl].  workspace >= lsk_head_workspace_bytes(M, N).
 * Replaces F.linear(.., lm_head) + .argmax(-1) (common/model.py:330, solutions/engine.py:255,352,463). */
size_t lsk_head_workspace_bytes(int M, int N);
int lsk_head_argmax(int dtype, const void* A, long lda, const void* W, long ldw, int M, int N, int K, void* logits,
                    long ldl, int64_t* out, const int64_t* dst_idx, void* workspace, size_t ws_bytes, void* stream);

/* Final norm + LM head + greedy pick in one call (bf16; W packed, ldw == K): out[dst_idx ? dst_idx[m] : m] =
 * argmax_n rnd(rmsnorm(h[m], norm_w, eps) . W[n]) (first index on ties), optionally storing the bf16 logits
 * [M, ldl].  Bitwise the same as lsk_rmsnorm followed by lsk_head_argmax; up to 64 rows the normalised rows
 * stay in the workspace in the GEMM's fragment order.  workspace >= lsk_head_norm_workspace_bytes(M, N, K).
 * Replaces LayerSkipLlama.head + .argmax(-1): F.linear(rms_norm(h, norm_w), lm_head_w) (common/model.py:329-330;
 * solutions/engine.py:255,352,463). */
size_t lsk_head_norm_workspace_bytes(int M, int N, int K);
int lsk_head_norm_argmax(int dtype, const void* h, long ldh, const void* norm_w, float eps, const void* W, long ldw,
                         int M, int N, int K, void* logits, long ldl, int64_t* out, const int64_t* dst_idx,
                         void* workspace, size_t ws_bytes, void* stream);

/* Residual add + RMSNorm: x_new = rnd(x + rnd(sum_{s<ks} P[s])) (ks = 0: x_new = x), stored to x_out when
 * non-NULL; out = rmsnorm(x_new, w) when out != NULL.  P: fp32 [ks][n_rows][dim].
 * Replaces `x + F.linear(...)` + rms_norm at solutions/packed.py:182-183, 185 + 175. */
int lsk_add_rmsnorm(int dtype, const void* x, long ldx, const float* partials, int ks, const void* w, float eps,
                    void* x_out, long ldxo, void* out, long ldo, int n_rows, int dim, void* stream);

/* Fused qkv projection + RoPE + KV append (bf16): replaces F.linear(x, wqkv) at solutions/packed.py:175 together
 * with apply_rope (common/model.py:143-150, solutions/packed.py:176-179) and the KV write (solutions/packed.py:
 * 180-181).  A: the normalised rows fragment-major (lsk_frag_off, ceil(M/16)*16 rows x K); W: lsk_pack_weight_qkv
 * storage.  Writes q_out [M, n_heads, head_dim] (rotated), the K cache (rotated) and the V cache at (rows[m],
 * pos[m]), with lsk_rope_append's arithmetic on rnd(the full-K sum).  head_dim % 32 == 0, max_seq % 32 == 0. */
int lsk_gemm_qkv_rope(const void* A, const void* W, int M, int n_heads, int n_kv_heads, int head_dim, int K,
                      void* q_out, void* kcache, void* vcache, const float* cos_tab, const float* sin_tab, int tab_len,
                      const int32_t* rows, const int32_t* pos, int max_batch, int max_seq, void* stream);

/* lsk_pack_weight for the fused [q; k; v] weight ((n_heads + 2 n_kv_heads) head_dim rows x K) that
 * lsk_gemm_qkv_rope reads: within each q and k head the 16-row groups are stored RoPE-paired (dims 16j..16j+15,
 * then their partners head_dim/2 + 16j ..), v rows in order.  Pure copies; unpacking restores the [out, in]
 * tensor (common/model.py:259-276).  No reference counterpart (storage format only). */
int lsk_pack_weight_qkv(const void* W, long ldw, void* Wp, int n_heads, int n_kv_heads, int head_dim, int K,
                        void* stream);
int lsk_unpack_weight_qkv(const void* Wp, void* W, long ldw, int n_heads, int n_kv_heads, int head_dim, int K,
                          void* stream);

/* lsk_rope_append reading qkv as rnd(sum_{s<ks} P[s]) from fp32 partials [ks][N][(Hq+2Hkv)D]. */
int lsk_rope_append_partial(int dtype, const float* partials, int ks, void* q_out, void* kcache, void* vcache,
                            const float* cos_tab, const float* sin_tab, int tab_len, const int32_t* rows,
                            const int32_t* pos, int n_tokens, int n_heads, int n_kv_heads, int head_dim,
                            int max_batch, int max_seq, void* stream);

/* Embedding gather with the engine's id assembly: out[t] = table[id_t],
 * id_t = (sel && sel[t] >= 0) ? seq_buf[sel[t]] : alt[t]  (int64 ids; out-of-range id -> zero row).
 * Replaces solutions/engine.py:345-346 (torch.where id assembly) + common/model.py:325-326 (F.embedding). */
int lsk_embed(const void* table, long vocab, long row_bytes, const int64_t* seq_buf, long seq_len,
              const int64_t* sel, const int64_t* alt, void* out, int n_tokens, void* stream);

/* Row copy dst[dst_idx[i]] = src[src_idx[i]] (int64 indices, NULL = identity).
 * Replaces the exit_h staging/gathers of solutions/engine.py:349-350 and 453-455. */
int lsk_copy_rows(void* dst, const int64_t* dst_idx, long n_dst, const void* src, const int64_t* src_idx, long n_src,
                  long row_bytes, int n, void* stream);

/* Row-wise argmax (first index on ties) of dtype logits [n_rows, ld]; out[dst_idx ? dst_idx[m] : m] (int64).
 * Replaces .argmax(-1) at solutions/engine.py:227,255,352,463,478. */
int lsk_argmax(int dtype, const void* logits, long ld, int n_rows, int vocab, int64_t* out, const int64_t* dst_idx,
               void* stream);

/* Greedy acceptance of nv verifiers (see the kernel comment); forced = optional per-verifier
 * acceptance override (-1 = natural).  Replaces solutions/engine.py:461-476 (dr / scatter_reduce amin /
 * last_tok / seq_buf write); kv_len (optional) receives the pointer rollback of solutions/engine.py:383. */
int lsk_greedy_accept(const int64_t* Yv, int64_t* seq_buf, int Dm1, const int32_t* slots, const int32_t* starts,
                      const int32_t* Ts, const int32_t* forced, int nv, int64_t* acc_out, int64_t* y_out,
                      int64_t* kv_len, void* stream);

/* M2 probe agreement: out[c] = number of verify tokens t with a correct prefix (jl[t] <= acc[blk[t]]) on which
 * candidate exit c's greedy token pred[c * nvt + t] equals the full model's Yv[t]; out[nc] = number of tokens
 * with a correct prefix.  int64 tokens and counts, int32 blk / jl.
 * Replaces the match counting of solutions/engine.py:491-514 (_probe_counts). */
int lsk_probe_matches(const int64_t* pred, const int64_t* Yv, const int64_t* acc, const int32_t* blk, const int32_t* jl,
                      int nc, int nvt, int64_t* out, void* stream);

/* Pointer rollback: kv_len[slots[j]] += accepted[j] + 1; moves no KV.
 * Replaces solutions/engine.py:381-384 (pos += a + 1; d = 0) for a device-resident length array. */
int lsk_kv_rollback(int64_t* kv_len, const int32_t* slots, const int64_t* accepted, int nv, void* stream);

/* No counterpart in the reference (it plans each step after the previous one's readback).  Moves the blocks of a
   decode segment that was planned before the previous step's acceptance was read back: every block in cache row
   vslots[j] was planned at the position it has if all vdrafts[j] drafts are accepted; accepted[j] (device, the
   greedy acceptance's acc_out) gives the actual one.  meta: the segment's metadata as lsk_pack_segment writes it
   (device; n_tokens, nb, n_works, n_groups from its counts, n_recs = n_slots * n_rounds); group = query heads per
   KV head.  Updates each token's position, each block's pos0 and the work records' pos0 / final kv_hi in place.
   The caller guarantees the move never changes a block's number of KV splits. */
int lsk_shift_segment_positions(int32_t* meta, int n_tokens, int nb, int n_works, int n_groups, int n_recs, int group,
                                const int64_t* accepted, const int32_t* vslots, const int32_t* vdrafts, int nv,
                                void* stream);

/* ---- native layer-range runner (solutions/packed.py:169-196, packed_layer / packed_layers) ----
 * A model handle holds host copies of per-layer device pointers (weights [out, in]: packed for bf16 --
 * wqkv in lsk_pack_weight_qkv storage, the others lsk_pack_weight; dim and head_dim multiples of 32 -- row-major
 * for fp32,
 * KV caches [B, Hkv, S, D], fp32 RoPE tables [tab_len, D]); it owns no device memory.
 * Returns a handle > 0, or a negative error code. */
long lsk_model_create(int dtype, int n_layers, int dim, int n_heads, int n_kv_heads, int head_dim, int ffn, int vocab,
                      float eps, const void* const* wqkv, const void* const* wo, const void* const* w13,
                      const void* const* w2, const void* const* attn_norm, const void* const* ffn_norm,
                      void* const* kcache, void* const* vcache, int max_batch, int max_seq, const float* cos_tab,
                      const float* sin_tab, int tab_len);
int lsk_model_destroy(long handle);

/* Workspace bytes lsk_forward_layers needs for n_tokens packed tokens and n_parts attention partial slots. */
size_t lsk_segment_workspace_bytes(long handle, int n_tokens, int n_parts);

/* Layers [start, end) over n_tokens packed tokens: x_out = layers(x_in) (x_in is not modified).
 * meta: device int32 [rows N][pos N][blocks nb*4][works n_works*8][groups n_groups*8]
 * [recs n_slots*n_rounds*8] (see lsk_attn_plan, lsk_attn_schedule); rows_cap as for lsk_ragged_attn.
 * capture: NULL or a host array of n_layers device pointers; capture[i] != NULL receives layer i's output
 * (solutions/packed.py:190-195).  Replaces packed_layers (solutions/packed.py:188-196). */
int lsk_forward_layers(long handle, const void* x_in, void* x_out, int n_tokens, int start, int end,
                       const int32_t* meta, int nb, int n_works, int n_groups, int n_parts, int n_rounds, int n_slots,
                       int rows_cap, void* workspace, size_t ws_bytes, void* const* capture, double attn_bytes,
                       double attn_flops, void* stream);

/* ---- optional per-launch profiling (no reference counterpart: measurement support) ----
 * When enabled, the layer runner (and callers using lsk_prof_start/stop around their own launches)
 * bracket each launch with HIP events on its stream, tagged with a class and the launch's algorithmic
 * bytes / flops.  lsk_prof_collect synchronises and returns per-class sums.  attn_bytes / attn_flops of
 * lsk_forward_layers are the per-layer algorithmic figures of the attention launch (profiling only). */
#define LSK_PROF_NORM 0
#define LSK_PROF_GEMM_QKV 1
#define LSK_PROF_ROPE 2
#define LSK_PROF_ATTN 3
#define LSK_PROF_GEMM_O 4
#define LSK_PROF_GEMM_W13 5
#define LSK_PROF_GEMM_W2 6
#define LSK_PROF_GEMM_HEAD 7
#define LSK_PROF_ARGMAX 8
#define LSK_PROF_GLUE 9
#define LSK_PROF_CLASSES 10
int lsk_prof_enable(int on);
int lsk_prof_start(int cls, double bytes, double flops, void* stream);
int lsk_prof_stop(void* stream);
int lsk_prof_collect(int n_classes, double* ms, double* bytes, double* flops, long* count);

#ifdef __cplusplus
}
#endif

#endif /* LSK_H_ */
