/*
 * symbiote_mi355x.h -- C ABI of the MI355X (gfx950) kernels behind the BailingMoeV2
 * (Ling-mini-2.0) decode hot path: paged GQA decode attention over a block-table KV cache,
 * and the MoE block (sigmoid/bias/group-limited router, token permute/unpermute, grouped
 * SwiGLU expert GEMMs, shared expert).
 *
 * Conventions (every entry point):
 *   - all tensor arguments are raw device pointers; sizes are plain ints;
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default stream);
 *   - the return value is a sym_status; on error sym_last_error() gives a message for the
 *     calling thread. No entry point throws, allocates device memory or synchronizes;
 *   - scratch memory is passed in by the caller (`workspace`, sized by the matching
 *     *_workspace_bytes query), so a whole decode step can be captured in a HIP graph;
 *   - bf16 tensors are raw uint16 bit patterns (torch.bfloat16 storage);
 *   - calls are stateless and may be issued from several host threads on distinct streams.
 *
 * Shapes follow the reference's device layouts:
 *   KV pools   [num_blocks, n_kv_heads, block_size, head_dim]   (ttnn_attention.py:116-137)
 *   page table [batch, max_blocks_per_seq] int32                (ttnn_attention.py:101-102)
 *   positions  [batch] int32: slot of the new token = tokens already cached for that sequence
 *              (the reference's cur_pos, ttnn_attention.py:2232-2306)
 *   expert weights stacked as gate_up [E(+1), 2*I, H] (gate rows first) and down
 *              [E(+1), H, I] (ttnn_moe.py:1596-1609); slot E holds the shared expert.
 */
#ifndef SYMBIOTE_MI355X_H
#define SYMBIOTE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  SYM_OK = 0,
  SYM_ERR_INVALID = 1,     /* bad argument: null pointer, size out of range */
  SYM_ERR_UNSUPPORTED = 2, /* shape the kernels do not implement (e.g. head_dim != 128) */
  SYM_ERR_WORKSPACE = 3,   /* workspace smaller than the *_workspace_bytes query */
  SYM_ERR_LAUNCH = 4       /* the HIP runtime rejected a launch */
} sym_status;

/* Message for the last non-zero status returned on the calling thread. */
const char* sym_last_error(void);
/* ABI revision; bumped on any signature change (2: workspace of the tiled grouped GEMMs). */
int sym_abi_version(void);

/* ---------------------------------------------------------------------------------------
 * RMSNorm over the last dim, bf16 in/out, fp32 statistics, with optional fused residual add.
 * Replaces the decoder layer's input_layernorm / post_attention_layernorm
 * (modeling_bailing_moe_v2.py:440-465; formula of DeepseekV2RMSNorm,
 * ttnn_normalization.py:54-68). If `residual` (bf16) is non-NULL, s = x + residual is written
 * to `residual_out` in fp32 (the layer's residual stream) and normalized; otherwise s = x.
 * out = bf16(weight * s * rsqrt(mean(s^2) + eps)). rows >= 1, cols % 8 == 0, cols <= 16384.
 */
int sym_rmsnorm_bf16(const void* x, const void* residual, const void* weight, int rows, int cols,
                     float eps, void* out, float* residual_out, void* stream);
/* sym_rmsnorm_bf16 with fp32 x (a projection's fp32 output, e.g. the attention's dense
 * projection at prefill size), so the layer's residual stream s = x + residual is formed
 * without rounding x to bf16 first. x and residual_out 16-byte aligned. */
int sym_rmsnorm_f32(const float* x, const void* residual, const void* weight, int rows, int cols,
                    float eps, void* out, float* residual_out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Skinny GEMM for the decode projections: out[M, N] = x[M, K] . w[N, K]^T (+ bias[N]).
 * Replaces the query_key_value and dense linears of TTNNBailingMoEAttention
 * (ttnn_attention.py:2324, 2459). x, w, bias bf16; fp32 accumulation; out bf16, or fp32 when
 * out_fp32 != 0. N % 16 == 0, K % 64 == 0; bias may be NULL.
 */
int sym_linear_bf16(const void* x, const void* w, const void* bias, int M, int N, int K,
                    void* out, int out_fp32, void* stream);

/* Projection with the RMSNorm of x fused in front (the decoder layer's input_layernorm,
 * modeling_bailing_moe_v2.py:440-442, feeding the query_key_value linear):
 *   out = bf16(x * rsqrt(mean(x^2) + eps) * gamma) . w^T (+ bias), gamma [K] bf16; the
 *   normalised operand is rounded to bf16 as a separate RMSNorm pass would.
 * Constraints as sym_linear_bf16.
 */
int sym_rmsnorm_linear_bf16(const void* x, const void* gamma, float eps, const void* w,
                            const void* bias, int M, int N, int K, void* out, int out_fp32,
                            void* stream);

/* Projection with the residual add fused behind (the dense linear plus the decoder layer's
 * first residual add, ttnn_attention.py:2459 and modeling_bailing_moe_v2.py:457-460):
 *   out [M, N] fp32 = x . w^T (+ bias) + residual (bf16 [M, N]), with no intermediate rounding;
 *   sumsq_parts [N/16, M] fp32: sum over each 16-column block of out's row of out^2, the
 *   statistics of the following RMSNorm (see sym_moe_router_logits_norm).
 * Constraints as sym_linear_bf16.
 */
int sym_linear_residual_bf16(const void* x, const void* w, const void* bias,
                             const void* residual, int M, int N, int K, float* out,
                             float* sumsq_parts, void* stream);

/* ---------------------------------------------------------------------------------------
 * Decode prologue: per-head QK RMSNorm, partial split-half RoPE, paged KV write.
 * Replaces TTNNBailingMoEAttention._forward_decode_paged's split / _apply_qk_norm / RoPE /
 * paged_update_on_device sequence (ttnn_attention.py:2329-2431).
 *   qkv        [B, (Hq + 2*Hkv) * 128] bf16, output of the fused query_key_value projection
 *   q_norm_w, k_norm_w [128] bf16 (ignored when use_qk_norm == 0)
 *   rope_cs    [max_pos, 2, rotary_dim/2] fp32: cos then sin of pos * inv_freq[i]
 *   q_out      [B, Hq, 128] bf16
 *   K and V of the new token are written at slot positions[b] of sequence b.
 * head_dim is 128; rotary_dim even, 0 < rotary_dim <= 128. Slots whose page-table entry is
 * outside [0, num_blocks) or whose position is >= max_pos are skipped.
 */
int sym_attn_decode_prologue(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                             const float* rope_cs, int max_pos, const int32_t* positions, int B,
                             int Hq, int Hkv, int head_dim, int rotary_dim, float eps,
                             int use_qk_norm, void* q_out, void* k_pool, void* v_pool,
                             const int32_t* block_tables, int max_blocks_per_seq, int block_size,
                             int num_blocks, void* stream);

/* Prefill prologue: the same per-token QK-norm + RoPE + paged KV write for T packed tokens of
 * several sequences (prefill branch of TTNNBailingMoEAttention, ttnn_attention.py:2153-2230;
 * paged_fill_on_device, 202-233): token t has position positions[t] and page-table row
 * seq_ids[t]; q -> q_out [T, Hq, 128]; k, v -> the pools and k_out / v_out [T, Hkv, 128]
 * (the operands of sym_prefill_attention). k_pool and v_pool may both be null: then only
 * k_out / v_out are written (an fp8 cache is filled from them by sym_paged_kv_fill_fp8).
 */
int sym_attn_prefill_prologue(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                              const float* rope_cs, int max_pos, const int32_t* positions,
                              const int32_t* seq_ids, int T, int Hq, int Hkv, int head_dim,
                              int rotary_dim, float eps, int use_qk_norm, void* q_out, void* k_out,
                              void* v_out, void* k_pool, void* v_pool, const int32_t* block_tables,
                              int max_blocks_per_seq, int block_size, int num_blocks, void* stream);

/* Causal GQA attention over packed sequences (prefill SDPA, ttnn_attention.py:2153-2230):
 *   q [T, Hq, 128], k, v [T, Hkv, 128] bf16, sequence s = rows cu_seqlens[s] .. cu_seqlens[s+1]-1
 *   at positions 0 .. L-1; out [T, Hq, 128] bf16 = softmax(q k^T * scale, causal) v within each
 *   sequence; max_seqlen >= every sequence length. fp32 accumulation, P rounded to bf16.
 */
int sym_prefill_attention(const void* q, const void* k, const void* v, const int32_t* cu_seqlens,
                          int n_seqs, int max_seqlen, int Hq, int Hkv, int head_dim, float scale,
                          void* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Paged KV write of one token per sequence: replaces TTNNPagedAttentionKVCache.
 * paged_update_on_device -> ttnn.experimental.paged_update_cache (ttnn_attention.py:235-269).
 *   k_new, v_new [B, Hkv, head_dim] bf16; slot = positions[b].
 */
int sym_paged_kv_write(const void* k_new, const void* v_new, void* k_pool, void* v_pool,
                       const int32_t* block_tables, const int32_t* positions, int B, int Hkv,
                       int head_dim, int block_size, int max_blocks_per_seq, int num_blocks,
                       void* stream);

/* ---------------------------------------------------------------------------------------
 * Paged prefill fill of one sequence: replaces paged_fill_on_device -> paged_fill_cache
 * (ttnn_attention.py:202-233). k, v [Hkv, S, head_dim] bf16 written at positions
 * start_pos .. start_pos+S-1 of sequence `batch_idx`.
 */
int sym_paged_kv_fill(const void* k, const void* v, void* k_pool, void* v_pool,
                      const int32_t* block_tables, int batch_idx, int start_pos, int S, int Hkv,
                      int head_dim, int block_size, int max_blocks_per_seq, int num_blocks,
                      void* stream);

/* ---------------------------------------------------------------------------------------
 * Paged GQA decode attention (split-K over the context, log-sum-exp merge).
 * Replaces TTNNPagedAttentionKVCache.paged_sdpa_decode ->
 * ttnn.transformer.paged_scaled_dot_product_attention_decode (ttnn_attention.py:288-329):
 *   out[b, h] = softmax(scale * q[b,h] . K[b, 0..positions[b]]^T) V[b, 0..positions[b]]
 * with kv head = h / (Hq/Hkv); K/V gathered through the page table; fp32 accumulation.
 *   q   [B, Hq, 128] bf16;  out [B, Hq, 128] bf16 (zero for a sequence with positions[b] < 0)
 *   max_context: attention length cap (normally max_blocks_per_seq * block_size); a sequence
 *   attends min(positions[b] + 1, max_context) slots.
 *   workspace: sym_paged_gqa_decode_workspace_bytes(...) bytes of per-split partial results
 *   (no initial contents needed). Calls that overlap in time must not share a workspace.
 * Hq/Hkv in {1,2,4,8}; head_dim 128.
 */
size_t sym_paged_gqa_decode_workspace_bytes(int B, int Hq, int head_dim, int max_context);
int sym_paged_gqa_decode(const void* q, const void* k_pool, const void* v_pool,
                         const int32_t* block_tables, const int32_t* positions, int B, int Hq,
                         int Hkv, int head_dim, int block_size, int max_blocks_per_seq,
                         int num_blocks, int max_context, float scale, void* workspace,
                         size_t workspace_bytes, void* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Allocation-free paged GQA decode. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same arguments, kernels and results as sym_paged_gqa_decode, without
 * the workspace: the per-split partial results live in a fixed 32 MiB device array inside the
 * library, one copy per GPU, held until the process ends. Calls whose
 * sym_paged_gqa_decode_workspace_bytes(B, Hq, head_dim, max_context) exceeds 32 MiB return
 * SYM_ERR_WORKSPACE (e.g. batch 32 x 16 heads fits up to 32 K tokens of max_context). The first
 * call on a device locates that device's copy (a runtime query, no allocation). Every call on a
 * GPU shares its copy: calls that overlap in time on one GPU (two streams, two host threads)
 * race. Nothing in it needs clearing between calls.
 */
int sym_paged_gqa_decode_noalloc(const void* q, const void* k_pool, const void* v_pool,
                                 const int32_t* block_tables, const int32_t* positions, int B,
                                 int Hq, int Hkv, int head_dim, int block_size,
                                 int max_blocks_per_seq, int num_blocks, int max_context,
                                 float scale, void* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Fused attention decode step: sym_attn_decode_prologue followed by sym_paged_gqa_decode in
 * one split kernel (+ the merge kernel). Replaces the QK-norm, RoPE, paged_update_cache and
 * paged SDPA decode of TTNNBailingMoEAttention._forward_decode_paged
 * (ttnn_attention.py:2329-2443). Every workgroup normalises and rotates its q heads from qkv;
 * the workgroup of each sequence's last split also normalises and rotates k, writes k and v into
 * the pools at positions[b] (as the prologue) and uses them for the new token directly.
 * Arguments as sym_attn_decode_prologue (qkv [B, (Hq+2Hkv)*head_dim]) and
 * sym_paged_gqa_decode (workspace, max_context, scale, out [B, Hq, head_dim]); results are
 * identical to the two calls in sequence.
 */
int sym_attn_decode_step(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                         const float* rope_cs, int max_pos, const int32_t* positions, int B, int Hq,
                         int Hkv, int head_dim, int rotary_dim, float eps, int use_qk_norm,
                         void* k_pool, void* v_pool, const int32_t* block_tables,
                         int max_blocks_per_seq, int block_size, int num_blocks, int max_context,
                         float scale, void* workspace, size_t workspace_bytes, void* out,
                         void* stream);

/* ---------------------------------------------------------------------------------------
 * fp8 KV cache (the "fp8-KV variant with kv_scales" of the paged decode). The K pool
 * [num_blocks, Hkv, block_size, 128] and the V pool [num_blocks, Hkv, 128, block_size] (dim-major
 * inside each (block, head): byte (d, slot) at d * block_size + slot, the operand layout of the
 * attention's P.V MFMA) hold OCP fp8 e4m3fn bytes; k_scale / v_scale [num_blocks, Hkv] fp32 hold
 * one power-of-two scale per (block, kv head); a stored value is byte value * scale. Appending tokens to a block: s_new = max(s_old, pow2_ceil(amax / 448))
 * (s_old = 0 for an empty block); when the scale grows, the block's earlier bytes c become
 * e4m3(value(c) * s_old / s_new); new tokens are e4m3(x / s_new) with x their bf16 values
 * (round to nearest even). block_size is a multiple of 8 dividing 256. The reference's cache is bf16
 * (TTNNPagedAttentionKVCache, ttnn_attention.py:116-137); the layout and page-table semantics
 * are the same.
 * sym_paged_kv_fill_fp8: appends tokens cu_seqlens[s] + i (i < L_s) of n_seqs sequences at
 *   positions start_pos[s] + i (start_pos null: 0) through page-table row seq_rows[s]
 *   (seq_rows null: row s) of a page table of page_table_rows rows
 *   (paged_fill_on_device / paged_update_on_device, ttnn_attention.py:202-269). The 128 bf16
 *   dims of token t, head g start at element t * tok_stride + g * head_stride of k / v
 *   ([T, Hkv, 128]: Hkv*128, 128; [Hkv, S, 128]: 128, S*128). A sequence whose start is
 *   negative, or whose row lies outside the page table, is skipped. max_seqlen >= every L_s.
 * sym_paged_gqa_decode_fp8 / sym_attn_decode_step_fp8: sym_paged_gqa_decode /
 *   sym_attn_decode_step over the fp8 pools (paged_sdpa_decode, ttnn_attention.py:288-329);
 *   same workspace. The step appends the new token's k and v by the rule above before the
 *   attention reads the pool.
 */
int sym_paged_kv_fill_fp8(const void* k, const void* v, long long tok_stride,
                          long long head_stride, const int32_t* cu_seqlens,
                          const int32_t* start_pos, const int32_t* seq_rows, int n_seqs,
                          int max_seqlen, int Hkv, int head_dim, void* k_pool, void* v_pool,
                          float* k_scale, float* v_scale, const int32_t* block_tables,
                          int page_table_rows, int max_blocks_per_seq, int block_size,
                          int num_blocks, void* stream);
int sym_paged_gqa_decode_fp8(const void* q, const void* k_pool, const void* v_pool,
                             const float* k_scale, const float* v_scale,
                             const int32_t* block_tables, const int32_t* positions, int B,
                             int Hq, int Hkv, int head_dim, int block_size,
                             int max_blocks_per_seq, int num_blocks, int max_context,
                             float scale, void* workspace, size_t workspace_bytes, void* out,
                             void* stream);
int sym_attn_decode_step_fp8(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                             const float* rope_cs, int max_pos, const int32_t* positions, int B,
                             int Hq, int Hkv, int head_dim, int rotary_dim, float eps,
                             int use_qk_norm, void* k_pool, void* v_pool, float* k_scale,
                             float* v_scale, const int32_t* block_tables,
                             int max_blocks_per_seq, int block_size, int num_blocks,
                             int max_context, float scale, void* workspace,
                             size_t workspace_bytes, void* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Router logits in fp32 (fp32 MFMA): replaces the fp32 gate GEMV of TTNNMoE.forward
 * (ttnn_moe.py:1438-1455; gate weight kept fp32, ttnn_moe.py:1542).
 *   x [T, H] bf16 (upcast exactly); w [E, H] fp32;
 *   parts [4, T, E] fp32: parts[q] = x[:, Hq] . w[:, Hq]^T over the q-th quarter of H.
 * The logits are ((parts[0] + parts[1]) + parts[2]) + parts[3], summed in that order by
 * sym_moe_route_permute (n_logit_parts = 4), so routing does not depend on launch order.
 * H % 512 == 0, E % 16 == 0.
 */
int sym_moe_router_logits(const void* x, const float* w, int T, int H, int E, float* parts,
                          void* stream);

/* The same router logits for prefill-size T, on bf16 MFMA tiles (128 x 256, the grouped down
 * projection's kernel):
 *   w_planes [3, E, H] bf16 with w = hi + mid + lo exactly (the fp32 gate weight split into
 *   three 8-bit-mantissa planes, e.g. hi = w with its low 16 bits cleared, mid likewise of
 *   w - hi, lo = w - hi - mid); x [T, H] bf16;
 *   parts [3, T, E] fp32: parts[z] = x . plane_z^T (each product exact in fp32), summed
 *   (parts[0] + parts[1]) + parts[2] by sym_moe_route_permute (n_logit_parts = 3).
 * H % 64 == 0, E % 16 == 0; x, w_planes and parts 16-byte aligned, x [T, H] and one plane
 * under 4 GB.
 */
int sym_moe_router_logits_split(const void* x, const void* w_planes, int T, int H, int E,
                                float* parts, void* stream);

/* Router logits with the post-attention RMSNorm fused in front (the decoder layer's
 * post_attention_layernorm, modeling_bailing_moe_v2.py:463-465, feeding TTNNMoE.forward):
 *   h [T, H] fp32 residual stream; ss_parts [n_ss, T] fp32 partial sums of squares of h's rows
 *   (sum over all n_ss gives sum_k h[t,k]^2; as written by sym_linear_residual_bf16);
 *   xn = bf16(h * rsqrt(sum/H + eps) * gamma) (gamma [H] bf16) is the operand of the logits, as
 *   sym_moe_router_logits on xn; when xn_out (bf16 [T, H]) is non-NULL it also receives xn,
 *   the input of the expert GEMMs.
 */
int sym_moe_router_logits_norm(const float* h, const float* ss_parts, int n_ss,
                               const void* gamma, float eps, const float* w, int T, int H, int E,
                               float* parts, void* xn_out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Fused MoE router + top-k + permute.
 * Replaces TTNNMoERouterDecode.forward (ttnn_moe.py:891-1024; torch form
 * Glm4MoeRouteTokenToExperts, ttnn_moe.py:413-436) and the dispatch/remap of
 * TTNNExperts.forward (ttnn_moe.py:1225-1245):
 *   logits = sum of the n_logit_parts arrays [n_logit_parts, T, E] (left to right);
 *   s = sigmoid(logits); c = s + bias; group score = sum of the two largest c in each group of
 *   E/n_group experts; keep the topk_group best groups; experts of other groups score 0.0;
 *   topk_idx = top_k experts by that score (ties: lower index first);
 *   topk_w = s[topk_idx], divided by (sum + 1e-20) when renormalize, times routed_scale.
 * Permute: assignments (t, k) sorted by (expert, token); expert_offsets is the exclusive
 * cumsum of expert_counts; sorted_tokens[row] = token of that row; inv_perm[t*top_k + k] =
 * row of assignment (t, k). When with_shared != 0, rows T*top_k .. T*top_k+T-1 hold every
 * token in order for the shared expert (stack slot E).
 * Segment list for the grouped GEMM: seg_expert/seg_offset/seg_count[0 .. *n_segments) list
 * the experts with at least one row in ascending order, then the shared expert.
 *   bias [E] fp32; E in {64,128,256,512}; E/n_group >= 2 and (E/n_group) % (E/64) == 0;
 *   top_k <= 32; topk_group <= n_group; 1 <= n_logit_parts <= 4.
 * Output sizes: topk_idx/topk_w/inv_perm [T*top_k]; expert_counts [E]; expert_offsets [E+1];
 * sorted_tokens [T*top_k + T]; seg_* [E+1]; n_segments [1].
 * Launches: routing (one wave per token), then the permute: one workgroup up to 2048 tokens
 * (state in LDS), else three launches over 256-token chunks (counts, per-expert scan, scatter)
 * with the same outputs bit for bit.
 * workspace: sym_moe_route_workspace_bytes(T, E) bytes (0 up to 2048 tokens, then
 * ceil(T/256) * E * 4: per-chunk counts; no initial contents needed); NULL / 0 when the query
 * gives 0. A smaller workspace returns SYM_ERR_WORKSPACE.
 */
size_t sym_moe_route_workspace_bytes(int T, int E);
int sym_moe_route_permute(const float* logits, int n_logit_parts, const float* bias, int T, int E,
                          int n_group, int topk_group, int top_k, float routed_scale,
                          int renormalize, int with_shared, int32_t* topk_idx, float* topk_w,
                          int32_t* expert_counts, int32_t* expert_offsets,
                          int32_t* sorted_tokens, int32_t* inv_perm, int32_t* seg_expert,
                          int32_t* seg_offset, int32_t* seg_count, int32_t* n_segments,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * Grouped SwiGLU expert GEMMs over the segment list of sym_moe_route_permute.
 * Replaces the three sparse_matmul calls + silu/mul of TTNNExperts.forward
 * (ttnn_moe.py:1250-1289) and the shared expert TTNNGlm4MoeMLP (ttnn_moe.py:656-675):
 *   for each segment s (expert e), row r in [seg_offset, seg_offset+seg_count):
 *     x_r = x[sorted_tokens[r]]
 *     h[r] = bf16(silu(x_r . Wg[e]^T) * (x_r . Wu[e]^T))     Wg = gate_up[e, :I], Wu = gate_up[e, I:]
 *     y[r] = h[r] . Wd[e]^T                                    (fp32)
 *   x [T, H] bf16; w_gate_up [E+1, 2I, H] bf16; w_down [E+1, H, I] bf16;
 *   h [rows, I] bf16 and y [rows, H] fp32 with rows = T*top_k (+T with a shared expert).
 * The segment list is read on the device; no host synchronization. H % 256 == 0, I % 64 == 0.
 * max_segments: the length of the segment list buffers (E+1).
 */
int sym_moe_grouped_swiglu(const void* x, int T, int H, int I, const int32_t* sorted_tokens,
                           const int32_t* seg_expert, const int32_t* seg_offset,
                           const int32_t* seg_count, const int32_t* n_segments, int max_segments,
                           const void* w_gate_up, const void* w_down, void* h, float* y,
                           void* stream);
/* The two halves of sym_moe_grouped_swiglu as separate launches: gate/up + SwiGLU -> h, then
 * down -> y (same arguments and layouts). */
int sym_moe_gate_up(const void* x, int T, int H, int I, const int32_t* sorted_tokens,
                    const int32_t* seg_expert, const int32_t* seg_offset, const int32_t* seg_count,
                    const int32_t* n_segments, int max_segments, const void* w_gate_up, void* h,
                    void* stream);
int sym_moe_down(const void* h, int T, int H, int I, const int32_t* seg_expert,
                 const int32_t* seg_offset, const int32_t* seg_count, const int32_t* n_segments,
                 int max_segments, const void* w_down, float* y, void* stream);
/* fp8 variants (the "_fp8 variant with w_scales" of the grouped SwiGLU; weight formats of
 * TTNNExperts.from_torch, ttnn_moe.py:1055-1078, stored as OCP fp8 e4m3fn): w_gate_up
 * [E+1, 2I, H] and w_down [E+1, H, I] are e4m3fn bytes with one fp32 scale per 128 x 128 block,
 * s_gate_up [E+1, 2I/128, H/128] and s_down [E+1, H/128, I/128]; weight = byte value * scale.
 * Dequantized inside the kernel (exact fp8 values on bf16 MFMA, block scale applied in fp32).
 * Other arguments and results as sym_moe_gate_up / sym_moe_down. H % 512 == 0, I % 128 == 0. */
int sym_moe_gate_up_fp8(const void* x, int T, int H, int I, const int32_t* sorted_tokens,
                        const int32_t* seg_expert, const int32_t* seg_offset,
                        const int32_t* seg_count, const int32_t* n_segments, int max_segments,
                        const void* w_gate_up, const float* s_gate_up, void* h, void* stream);
int sym_moe_down_fp8(const void* h, int T, int H, int I, const int32_t* seg_expert,
                     const int32_t* seg_offset, const int32_t* seg_count,
                     const int32_t* n_segments, int max_segments, const void* w_down,
                     const float* s_down, float* y, void* stream);

/* ---------------------------------------------------------------------------------------
 * Tiled GEMMs for prefill-size batches (MFMA-bound; 256 x 256 output tiles, 128 x 256 for the
 * grouped down projection over segment lists of more than 512 entries).
 * sym_gemm_bf16: out[M, N] = a[M, K] . w[N, K]^T (+ bias[N] bf16) (+ residual[M, N] fp32),
 *   bf16 out, or fp32 when out_fp32 != 0. Replaces the QKV / dense projections at sequence length
 *   > 1 (ttnn_attention.py:2001-2011, 2153-2230). N % 16 == 0, K % 64 == 0; a, w, out and
 *   residual 16-byte aligned, bias 8-byte aligned; a and w each under 4 GB.
 * sym_gemm_bf16_res_bf16: out[M, N] (fp32) = a . w^T (+ bias) + residual[M, N] (bf16), the sum
 *   taken in fp32 in the epilogue: the dense projection plus the decoder layer's first residual
 *   add at sequence length > 1 (ttnn_attention.py:2211-2230 dense, modeling_bailing_moe_v2.py:
 *   457-460 residual). Same shape rules as sym_gemm_bf16; residual 8-byte aligned.
 * sym_moe_gate_up_tiled / sym_moe_down_tiled: the grouped expert GEMMs of sym_moe_gate_up /
 *   sym_moe_down (same arguments and results; TTNNExperts.forward, ttnn_moe.py:1250-1289) for
 *   segments of many rows; rows = total rows of the segment list (T*top_k + T with the shared
 *   expert). y is fp32, or bf16 when y_bf16 != 0 (half the bytes written here and read back by
 *   sym_moe_unpermute_combine). H % 64 == 0, I % 64 == 0; x / h, the weights and h / y
 *   16-byte aligned; x, h and one expert's weights each under 4 GB.
 *   workspace: sym_moe_tiled_workspace_bytes() bytes (8 per-XCD tile counters), zeroed by the
 *   caller before its first use. With at most 512 segments the two kernels hand out their tiles
 *   from these counters, and every launch leaves them at zero again, so one workspace serves
 *   any number of stream-ordered launches (and graph replays). Launches that may overlap in time
 *   (on different streams) must use different workspaces. A smaller workspace returns
 *   SYM_ERR_WORKSPACE.
 */
size_t sym_moe_tiled_workspace_bytes(void);
int sym_gemm_bf16(const void* a, const void* w, const void* bias, const float* residual, int M,
                  int N, int K, void* out, int out_fp32, void* stream);
int sym_gemm_bf16_res_bf16(const void* a, const void* w, const void* bias, const void* residual,
                           int M, int N, int K, float* out, void* stream);
int sym_moe_gate_up_tiled(const void* x, int T, int H, int I, int rows,
                          const int32_t* sorted_tokens, const int32_t* seg_expert,
                          const int32_t* seg_offset, const int32_t* seg_count,
                          const int32_t* n_segments, int max_segments, const void* w_gate_up,
                          void* h, void* workspace, size_t workspace_bytes, void* stream);
int sym_moe_down_tiled(const void* h, int T, int H, int I, int rows, const int32_t* seg_expert,
                       const int32_t* seg_offset, const int32_t* seg_count,
                       const int32_t* n_segments, int max_segments, const void* w_down, void* y,
                       int y_bf16, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * Model ends of greedy generation (the embedding and final-norm swap of TTNNBailingMoeV2Model,
 * modeling_bailing_moe_v2.py:56-95 / 97-334; the lm_head linear; HF generate's greedy argmax,
 * taken on the device instead of the host).
 * sym_embedding_bf16: out[t] = table[ids[t]] ([T, H] rows of a [V, H] bf16 table); an id outside
 *   [0, V) gives a zero row. Also gathers rows of any [V, H] bf16 matrix (e.g. the last hidden
 *   row of each packed prompt). H % 8 == 0.
 * sym_lm_head_greedy: ids[b] = argmax_v x[b] . w[v] (x [B, H] bf16, already normalised; w [V, H]
 *   bf16; fp32 logits, never written; ties -> the lowest v). Workspace: the bytes
 *   sym_lm_head_greedy_workspace_bytes(B, V) returns. H % 256 == 0 (token rows are staged 256 columns at a time).
 * sym_greedy_advance: positions[b] += 1, then (history non-null) history[b][positions[b] -
 *   hist_base[b]] = ids[b] when that column lies in [0, hist_cols) -- the per-step bookkeeping of
 *   a captured decode step (positions and generated tokens stay on the device).
 */
int sym_embedding_bf16(const int32_t* ids, const void* table, int T, int H, int V, void* out,
                       void* stream);
size_t sym_lm_head_greedy_workspace_bytes(int B, int V);
int sym_lm_head_greedy(const void* x, const void* w, int B, int H, int V, void* workspace,
                       size_t workspace_bytes, int32_t* ids, void* stream);
int sym_greedy_advance(const int32_t* ids, int B, int32_t* positions, int32_t* history,
                       const int32_t* hist_base, int hist_cols, void* stream);

/* ---------------------------------------------------------------------------------------
 * Unpermute + weighted combine (+ shared expert, + residual).
 * Replaces all_to_all_combine + mul + sum(dim=0) (ttnn_moe.py:1307-1335), the shared-expert
 * add (ttnn_moe.py:1487-1490) and the decoder layer's residual add
 * (modeling_bailing_moe_v2.py:467-468):
 *   out[t] = bf16( sum_k topk_w[t,k] * y[inv_perm[t,k]]  (k ascending)
 *                  + (shared_row0 >= 0 ? y[shared_row0 + t] : 0)
 *                  + (residual ? residual[t] : 0) )
 *   y fp32, or bf16 when y_bf16 != 0 (widened exactly; the sum is fp32 either way);
 *   out [T, H] bf16; residual [T, H] fp32 (the residual stream) or NULL. H % 8 == 0.
 */
int sym_moe_unpermute_combine(const void* y, int y_bf16, const int32_t* inv_perm,
                              const float* topk_w, int T, int top_k, int H, int shared_row0,
                              const float* residual, void* out, void* stream);

/* ---------------------------------------------------------------------------------------
 * Streaming-read bandwidth probe (measurement only; no counterpart in the reference): reads
 * `bytes` (a multiple of 16) of `buf` once, with 2048 workgroups of 256 threads, 16 bytes per
 * thread per step; `sink` [1] is written only for one specific xor of the data.
 */
int sym_hbm_read_probe(const void* buf, size_t bytes, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SYMBIOTE_MI355X_H */
