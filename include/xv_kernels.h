/*
 * xv_kernels.h -- C ABI of the MI355X (gfx950) decode hot-path kernels.
 *
 * Every entry point takes raw device pointers, element strides (in elements,
 * not bytes) and sizes, launches on `stream`, never allocates, never
 * synchronises and never reads device memory on the host, so every call can
 * be recorded into a hipGraph.  The return value is a hipError_t: 0 on
 * success, hipErrorInvalidValue (1) for arguments the kernels do not support,
 * otherwise the launch error.  All activations are bf16 (raw 16-bit words),
 * arithmetic is fp32.
 *
 * Each declaration names the reference interface it replaces
 * (xixii421/xixi-vllm, paths relative to the repository root).
 */
#ifndef XV_KERNELS_H
#define XV_KERNELS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Human readable text for a code returned by any xv_* entry point. */
const char* xv_error_string(int code);

/* ABI version; bumped whenever a signature below changes. */
int xv_abi_version(void);

/*
 * KV store by slot mapping.
 * Replaces store_kvcache / _store_kvcache_kernel, src/compute/kv_ops.py:8-62.
 *   k_cache[slot[i], h, :] = key[i, h, :];  v_cache[slot[i], h, :] = value[i, h, :]
 *   for every i in [0, num_tokens) with slot[i] >= 0 (slot -1 is skipped, kv_ops.py:22-23).
 * key/value rows: element (i, h, d) at i*key_stride_tok + h*key_stride_head + d.
 * cache element of slot s = page*block_size + t, head h, dim d at
 * page*cache_page_stride + t*cache_tok_stride + h*cache_head_stride + d
 * (the reference pool [NB, BS, Hkv, D]; block_size 1 describes a flat
 * [num_slots, Hkv, D] view).  head_dim must be a multiple of 8 and all row
 * starts 16-byte aligned.
 */
int xv_store_kvcache(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                     const void* value, int64_t value_stride_tok, int64_t value_stride_head,
                     void* k_cache, void* v_cache,
                     int64_t cache_page_stride, int64_t cache_tok_stride, int64_t cache_head_stride,
                     int block_size, const int32_t* slot_mapping, int64_t num_tokens,
                     int num_kv_heads, int head_dim, hipStream_t stream);

/*
 * KV store into an fp8 (OCP e4m3fn) cache.  No counterpart in the reference,
 * whose pool holds the model dtype (src/compute/kv_pool.py:49-51): an optional
 * on-HBM format that halves the KV bytes the decode streams.  As
 * xv_store_kvcache, with each bf16 value x stored as e4m3fn(x * (1/scale))
 * (1/scale in fp32, one fp32 multiply, round to nearest even; a product past
 * the format's range, |p| > 464, becomes NaN, as torch's float8_e4m3fn cast
 * does), k_scale for key and v_scale for value, both finite and > 0.  Cache
 * strides are in elements (= bytes); cache rows and strides 8-byte aligned;
 * num_kv_heads * head_dim a multiple of 512.
 */
int xv_store_kvcache_fp8(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                         const void* value, int64_t value_stride_tok, int64_t value_stride_head,
                         void* k_cache, void* v_cache,
                         int64_t cache_page_stride, int64_t cache_tok_stride, int64_t cache_head_stride,
                         int block_size, const int32_t* slot_mapping, int64_t num_tokens,
                         int num_kv_heads, int head_dim, float k_scale, float v_scale, hipStream_t stream);

/*
 * Paged GQA decode attention (one query token per sequence, causal = attends
 * to every cached token including the one stored this step).
 * Replaces the decode branch of vllm::attention -> flash_attn_with_kvcache,
 * src/compute/layers/attention.py:91-99.
 *   q      : element (b, h, d) at b*q_stride_tok + h*q_stride_head + d   [B, Hq, D]
 *   caches : element (page, t, kvh, d) at page*page_stride + t*tok_stride + kvh*head_stride + d
 *   block_tables : int32 [B, bt_stride]; only the first ceil(seqlen/block_size) entries are read
 *   cache_seqlens: int32 [B]; 0 marks a padding row whose output is written as zeros
 *   out    : element (b, h, d) at b*out_stride_tok + h*D + d
 *   workspace: at least xv_paged_decode_workspace_size(...) bytes: per-segment
 *              partial counts, then partial outputs (bf16 rows; their
 *              log2-sum-exp in fp32) of sequences split across waves, merged by a
 *              second kernel.  No initial contents are required.  Calls
 *              sharing a workspace must be ordered on one stream.
 * Query head h reads kv head h / (Hq / Hkv).  scale multiplies q.k (1/sqrt(D) in the reference).
 * block_size is the tokens per cache block, any multiple of 16 (the
 * reference's default kvcache_block_size is 256, src/config.py:66-67): token t
 * of a sequence is row t % block_size of block block_tables[b][t / block_size],
 * max_blocks_per_seq counts blocks.
 * Supported: D == 128, Hq/Hkv in {1, 2, 4, 8} (batches above
 * 256 run as consecutive launches of 256 sequences on the same workspace),
 * head rows of 256 contiguous bytes with head_stride*(Hkv-1) + D <= tok_stride
 * or tok_stride == D (the reference's [page][token][head][d] pool, or a
 * [page][head][token][d] pool).  q, k_cache, v_cache 16-byte aligned and every
 * input stride a multiple of 8 elements (rows move by 16-byte LDS-DMA); out
 * 4-byte aligned with an even out_stride_tok.
 */
size_t xv_paged_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                      int max_blocks_per_seq, int block_size, int head_dim);
int xv_paged_decode_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                              const void* k_cache, const void* v_cache,
                              int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                              const int32_t* block_tables, int64_t bt_stride,
                              const int32_t* cache_seqlens,
                              void* out, int64_t out_stride_tok,
                              void* workspace, size_t workspace_bytes,
                              int batch, int num_q_heads, int num_kv_heads, int head_dim,
                              int block_size, int max_blocks_per_seq, float scale,
                              hipStream_t stream);

/*
 * xv_paged_decode_attention over an fp8 (OCP e4m3fn) cache written by
 * xv_store_kvcache_fp8.  No counterpart in the reference (its pool holds the
 * model dtype, src/compute/kv_pool.py:49-51): the on-HBM format option of the
 * KV pool, half the bytes per token.  Attends to K = k_cache * k_scale and
 * V = v_cache * v_scale (each fp8 value is exact in bf16; k_scale is folded
 * into the softmax scale, v_scale multiplies the output).  Cache strides are
 * in elements (= bytes) and multiples of 16; the same workspace as
 * xv_paged_decode_attention (xv_paged_decode_workspace_size).
 */
int xv_paged_decode_attention_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                  const void* k_cache, const void* v_cache,
                                  int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                  const int32_t* block_tables, int64_t bt_stride,
                                  const int32_t* cache_seqlens,
                                  void* out, int64_t out_stride_tok,
                                  void* workspace, size_t workspace_bytes,
                                  int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                  int block_size, int max_blocks_per_seq, float scale,
                                  float k_scale, float v_scale, hipStream_t stream);

/*
 * Chunked prefill over fp8 pages: every sequence's keys (cache rows 0 ..
 * cu_seqlens_k[b+1] - cu_seqlens_k[b] - 1 through its block table, the
 * cached prefix and this chunk, already stored) dequantized as
 * bf16(value * scale) into rows cu_seqlens_k[b] + t of k_out / v_out
 * ([T_k, Hkv, 128] at out_stride_tok), the varlen k/v that
 * xv_prefill_attention then reads.  No counterpart in the reference (fp8 pool
 * format); max_seqlen_k bounds every sequence's keys.  Cache strides in
 * elements (= bytes), multiples of 8.
 */
int xv_gather_kv_fp8(const void* k_cache, const void* v_cache, int64_t cache_page_stride,
                     int64_t cache_tok_stride, int64_t cache_head_stride, const int32_t* block_tables,
                     int64_t bt_stride, int block_size, const int32_t* cu_seqlens_k, int batch,
                     int max_seqlen_k, int num_kv_heads, int head_dim, float k_scale, float v_scale,
                     void* k_out, void* v_out, int64_t out_stride_tok, hipStream_t stream);

/*
 * Shared-prefix (cascade) decode attention: xv_paged_decode_attention for a
 * batch whose rows may share their first tokens' cache blocks, as a radix
 * prefix cache maps them (the reference's prefix index,
 * src/data/prefix/radix_index.py:20-129 with src/data/kv.py:40-119, shares
 * the blocks; its decode, attention.py:91-99, still reads them once per row).
 * Here each group's shared blocks are read once per kv head: a prefix pass
 * attends all of the group's query rows to them (MFMA, 16 rows per tile),
 * the per-row suffix runs through the decode kernels, and the merge combines
 * both by log-sum-exp.  Outputs equal xv_paged_decode_attention's up to
 * fp32 summation order.
 *   prefix_tokens[b]: tokens of row b covered by its group's prefix pass, a
 *     multiple of block_size (0: the row has no shared prefix); every row
 *     with prefix_tokens > 0 belongs to exactly one group, whose rows all have
 *     the same prefix_tokens and the same first prefix_tokens / block_size
 *     block ids; prefix_tokens[b] <= cache_seqlens[b] and
 *     <= max_prefix_blocks * block_size; max_prefix_blocks * block_size
 *     <= 1048576 (longer shared prefixes: hipErrorInvalidValue).
 *   group_info: int32 [num_groups][4], 16-byte aligned; group g's record is
 *     {first index into group_rows, number of rows, its first batch row,
 *     prefix_tokens of its rows}: the batch rows of group g are
 *     group_rows[info.x .. info.x + info.y), at most 128 / (Hq / Hkv) of
 *     them (further rows are not attended by the prefix pass: split larger
 *     groups), info.z == group_rows[info.x].  Empty groups (info.y == 0) are
 *     allowed, so a caller recording a graph can pass a fixed num_groups.
 *   workspace: xv_cascade_decode_workspace_size(batch, ...) bytes, 256-byte
 *     aligned; no initial contents.  batch <= 256.
 * Other arguments, supported shapes and errors as xv_paged_decode_attention.
 */
size_t xv_cascade_decode_workspace_size(int batch, int num_q_heads, int num_kv_heads,
                                        int max_blocks_per_seq, int block_size, int head_dim);
int xv_cascade_decode_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                const void* k_cache, const void* v_cache,
                                int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                const int32_t* block_tables, int64_t bt_stride,
                                const int32_t* cache_seqlens, const int32_t* prefix_tokens,
                                const int32_t* group_info, const int32_t* group_rows,
                                int num_groups, int max_prefix_blocks,
                                void* out, int64_t out_stride_tok,
                                void* workspace, size_t workspace_bytes,
                                int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                int block_size, int max_blocks_per_seq, float scale,
                                hipStream_t stream);

/*
 * xv_cascade_decode_attention over an fp8 (OCP e4m3fn) cache written by
 * xv_store_kvcache_fp8, scales as xv_paged_decode_attention_fp8 (k_scale
 * folded into the softmax scale, v_scale applied to the output).  No
 * counterpart in the reference (its pool holds bf16 pages only).
 */
int xv_cascade_decode_attention_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                    const void* k_cache, const void* v_cache,
                                    int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                    const int32_t* block_tables, int64_t bt_stride,
                                    const int32_t* cache_seqlens, const int32_t* prefix_tokens,
                                    const int32_t* group_info, const int32_t* group_rows,
                                    int num_groups, int max_prefix_blocks,
                                    void* out, int64_t out_stride_tok,
                                    void* workspace, size_t workspace_bytes,
                                    int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                    int block_size, int max_blocks_per_seq, float scale,
                                    float k_scale, float v_scale, hipStream_t stream);

/*
 * xv_paged_decode_attention without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture that must not
 * call hipMalloc, tight serving loops, harnesses that forbid allocation).  It
 * has no counterpart in the reference.  The workspace is a static device
 * array of 48 MiB that each GPU the library runs on holds until the process
 * ends; a call whose xv_paged_decode_workspace_size(batch, ...) exceeds it
 * returns hipErrorInvalidValue before touching the device.  Nothing is
 * allocated, freed or cleared (the kernels need no initial workspace
 * contents).  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (several streams or threads) race; order them on one
 * stream.  Arguments and results are those of xv_paged_decode_attention.
 */
int xv_paged_decode_attention_noalloc(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                                      const void* k_cache, const void* v_cache,
                                      int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                                      const int32_t* block_tables, int64_t bt_stride,
                                      const int32_t* cache_seqlens,
                                      void* out, int64_t out_stride_tok,
                                      int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                      int block_size, int max_blocks_per_seq, float scale,
                                      hipStream_t stream);

/*
 * Varlen causal prefill attention, optionally reading K/V through the paged
 * cache (chunked prefill / cached prefix).  Causal masking is bottom-right
 * aligned: query i of sequence b (of q_len_b queries) sees keys
 * j <= (k_len_b - q_len_b) + i.
 * Replaces the prefill branch of vllm::attention -> flash_attn_varlen_func,
 * src/compute/layers/attention.py:74-90.
 *   q   : element (tok, h, d) at tok*q_stride_tok + h*q_stride_head + d, tok in [0, cu_q[B])
 *   paged (block_tables != NULL): keys of sequence b are cache tokens 0..k_len_b-1
 *         gathered through block_tables like the decode kernel.
 *   dense (block_tables == NULL): key token j of sequence b is row cu_k[b]+j of k/v,
 *         element (row, kvh, d) at row*kv_stride_tok + kvh*kv_stride_head + d.
 *   out : element (tok, h, d) at tok*out_stride_tok + h*D + d.
 * Supported: D == 128, Hq/Hkv in {1, 2, 4, 8}, block_size a multiple of 16 when paged.
 * Rows move by 16-byte LDS-DMA: q, k, v, k_cache and v_cache 16-byte aligned,
 * every input stride a multiple of 8 elements; out 8-byte aligned with
 * out_stride_tok a multiple of 4 (hipErrorInvalidValue otherwise).
 */
int xv_prefill_attention(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                         const void* k, const void* v, int64_t kv_stride_tok, int64_t kv_stride_head,
                         const void* k_cache, const void* v_cache,
                         int64_t page_stride, int64_t tok_stride, int64_t head_stride,
                         const int32_t* block_tables, int64_t bt_stride,
                         const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                         void* out, int64_t out_stride_tok,
                         int batch, int max_seqlen_q, int num_q_heads, int num_kv_heads,
                         int head_dim, int block_size, float scale, hipStream_t stream);

/*
 * RMSNorm into a new buffer.
 * Replaces vllm::rmsnorm, src/compute/layers/ops.py:59-64 (flashinfer.norm.rmsnorm).
 *   out[r, :] = x[r, :] * rsqrt(mean(x[r, :]^2) + eps) * w
 * Row r = (o, i) with o in [0, n_outer), i in [0, n_inner); input row start
 * o*x_stride_outer + i*x_stride_inner (so [T, H, D] views of a fused qkv work
 * without a copy); output rows are contiguous (row r at r*hidden).
 * hidden must be a multiple of 8, at most 16384.
 */
int xv_rmsnorm(const void* x, int64_t x_stride_outer, int64_t x_stride_inner,
               const void* weight, void* out, int64_t n_outer, int64_t n_inner,
               int hidden, float eps, hipStream_t stream);

/*
 * In-place fused residual add + RMSNorm.
 * Replaces vllm::fused_add_rmsnorm, src/compute/layers/ops.py:72-79.
 *   s = x + residual (fp32);  residual <- bf16(s);  x <- bf16(s * rsqrt(mean(s^2)+eps) * w)
 */
int xv_fused_add_rmsnorm(void* x, int64_t x_stride, void* residual, int64_t residual_stride,
                         const void* weight, int64_t rows, int hidden, float eps,
                         hipStream_t stream);

/*
 * fused_add_rmsnorm whose x is the fp32 partial sums of a split-K GEMM.
 * Same contract as vllm::fused_add_rmsnorm (src/compute/layers/ops.py:72-79)
 * applied to x = bf16(sum_p parts[p]), the output of the unsplit GEMM that
 * feeds it (o_proj / down_proj, src/compute/models/qwen3.py:64,115, into the norms
 * of :150,:152 and the final norm); the normalised rows go to `out` instead of over x.
 *   part p of row r at parts + p*part_stride + r*row_stride (floats, both
 *   multiples of 4);  1 <= num_parts <= 8.
 *   s = bf16(sum parts) + residual (fp32);  residual <- bf16(s);
 *   out <- bf16(s * rsqrt(mean(s^2)+eps) * w)
 */
int xv_fused_add_rmsnorm_parts(const float* parts, int64_t part_stride, int64_t row_stride, int num_parts,
                               void* out, int64_t out_stride, void* residual, int64_t residual_stride,
                               const void* weight, int64_t rows, int hidden, float eps, hipStream_t stream);

/*
 * NeoX rotary embedding from an fp32 cos||sin table [max_pos, D] into new buffers.
 * Replaces vllm::rotary_embedding, src/compute/layers/ops.py:31-51
 * (flashinfer apply_rope_with_cos_sin_cache, is_neox=True) with the table of
 * build_cos_sin_cache, src/compute/layers/rotary.py:7-20.
 *   o[:D/2] = x1*cos - x2*sin;  o[D/2:] = x2*cos + x1*sin
 * q element (t, h, d) at t*q_stride_tok + h*q_stride_head + d; k likewise;
 * q_out [T, Hq, D] and k_out [T, Hkv, D] contiguous.  positions int64 [T].
 */
int xv_rotary_embedding(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                        const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                        const int64_t* positions, const float* cos_sin_cache,
                        void* q_out, void* k_out, int64_t num_tokens,
                        int num_q_heads, int num_kv_heads, int head_dim, hipStream_t stream);

/*
 * Qwen3 per-head q/k RMSNorm fused with NeoX RoPE (one pass over q and k).
 * Replaces Qwen3Attention._split_norm_rope, src/compute/models/qwen3.py:117-128
 * (vllm::rmsnorm on the q and k head views, then vllm::rotary_embedding).
 * The normed value is rounded to bf16 before the rotation, as the two
 * reference ops do.  Layouts as xv_rotary_embedding; q_weight/k_weight [D].
 */
int xv_qk_norm_rope(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                    const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                    const void* q_weight, const void* k_weight, float eps,
                    const int64_t* positions, const float* cos_sin_cache,
                    void* q_out, void* k_out, int64_t num_tokens,
                    int num_q_heads, int num_kv_heads, int head_dim, hipStream_t stream);

/*
 * Decode-step fusion of xv_qk_norm_rope with the KV store: q is normed and
 * rotated into q_out; k is normed, rotated and written, and v copied, straight
 * into the paged cache at slot_mapping[t] (slot -1 stores nothing), with the
 * cache addressing of xv_store_kvcache.  Replaces the pair
 * Qwen3Attention._split_norm_rope (src/compute/models/qwen3.py:117-128) +
 * store_kvcache (src/compute/kv_ops.py:35-62, called at attention.py:66-72).
 */
int xv_qk_norm_rope_store(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                          const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                          const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                          const void* q_weight, const void* k_weight, float eps,
                          const int64_t* positions, const float* cos_sin_cache, void* q_out,
                          void* k_cache, void* v_cache, int64_t cache_page_stride,
                          int64_t cache_tok_stride, int64_t cache_head_stride, int block_size,
                          const int32_t* slot_mapping, int64_t num_tokens, int num_q_heads,
                          int num_kv_heads, int head_dim, hipStream_t stream);
/* The same over an fp8 (e4m3fn) cache: the roped k (rounded to bf16) and v are
 * stored as e4m3fn(x * (1/scale)), as xv_store_kvcache_fp8 stores them.  No
 * counterpart in the reference (fp8 pool format). */
int xv_qk_norm_rope_store_fp8(const void* q, int64_t q_stride_tok, int64_t q_stride_head,
                              const void* k, int64_t k_stride_tok, int64_t k_stride_head,
                              const void* v, int64_t v_stride_tok, int64_t v_stride_head,
                              const void* q_weight, const void* k_weight, float eps,
                              const int64_t* positions, const float* cos_sin_cache, void* q_out,
                              void* k_cache, void* v_cache, int64_t cache_page_stride,
                              int64_t cache_tok_stride, int64_t cache_head_stride, int block_size,
                              const int32_t* slot_mapping, int64_t num_tokens, int num_q_heads,
                              int num_kv_heads, int head_dim, float k_scale, float v_scale,
                              hipStream_t stream);

/*
 * SiLU-and-mul.
 * Replaces vllm::silu_and_mul, src/compute/layers/ops.py:20-23 (gate first, up second).
 *   out[t, i] = silu(x[t, i]) * x[t, I + i]
 * x row t at t*x_stride, out row t at t*out_stride; inter_size multiple of 8.
 */
int xv_silu_and_mul(const void* x, int64_t x_stride, void* out, int64_t out_stride,
                    int64_t num_tokens, int inter_size, hipStream_t stream);

/*
 * Batched sampler over bf16 logits [B, V] (row b at b*logits_stride).
 * Replaces Sampler.forward, src/compute/sampler.py:27-119, and the greedy
 * ParallelLMHead.argmax, src/compute/layers/vocab_parallel.py:180-216.
 * Per row: temperature <= 1e-5 (or flag XV_SAMPLE_ALL_GREEDY) -> argmax of the
 *  logits, lowest index on ties.  Otherwise x = logit * (1/temperature); candidates
 * are ordered by descending x, ties by ascending id; the kept set is the
 * shortest prefix satisfying top-k (top_ks[b] < V), top-p (a candidate is
 * dropped when the mass strictly before it exceeds top_p of the top-k mass)
 * and min-p (dropped when its probability is below min_p times the largest);
 * the first candidate is always kept (with min_p above 1 it alone).  The
 * token is then drawn by inverse CDF over the kept set in ascending id order
 * with the explicit uniform uniforms[b] in [0, 1), masses in 2^-40 fixed
 * point (exact integer sums).  NaN logits of sampled rows have no mass; a row
 * whose scaled maximum is not finite (+inf or -inf, or past fp32's range)
 * has no mass anywhere and returns its first candidate.
 * flags: XV_SAMPLE_* bits mirroring the reference's host-side switches.
 * workspace: xv_sampler_workspace_size(B, V) bytes, zero-filled before its
 *   first use (each call leaves its greedy counters zero).  With it, all-greedy
 *   calls and calls of up to 512 rows spread each row over several workgroups
 *   (larger sampled batches take one workgroup per row, which fills the
 *   device); NULL selects one workgroup per row.  Both give identical ids.
 *   The size never decreases with B, and a workspace sized for B rows serves
 *   every later call of up to B rows, greedy or sampled, in any order (the
 *   greedy counters sit at the bottom, the sampled path's data at the top).
 *   Calls sharing a workspace must be ordered on one stream.
 */
#define XV_SAMPLE_ALL_GREEDY 1
#define XV_SAMPLE_USE_TOP_K  2
#define XV_SAMPLE_USE_TOP_P  4
#define XV_SAMPLE_USE_MIN_P  8
/* Every row's top_k is in [1, 64] (the reference's host-side max_top_k,
 * src/compute/batch.py:251, at most 64): with a workspace, a two-launch
 * top-k path that reads the logits once (batches whose B x 32 x 64 candidate
 * lists fit the workspace's sampled region: up to 4101 rows at V 151936).
 * Ids are the same with or without it; a row outside the bound is still
 * sampled exactly (one workgroup for that row). */
#define XV_SAMPLE_TOP_K_LE_64 16
size_t xv_sampler_workspace_size(int batch, int vocab);
int xv_sample(const void* logits, int64_t logits_stride, int batch, int vocab,
              const float* temperatures, const float* top_ps, const int32_t* top_ks,
              const float* min_ps, const float* uniforms, int flags,
              int64_t* out_ids, void* workspace, size_t workspace_bytes,
              hipStream_t stream);

/*
 * Weight-streaming GEMM of a decode batch: out = x[m, k] . w[n, k]^T, m <= 64,
 * bf16 operands, fp32 accumulate.  Replaces, for decode batches, the GEMMs
 * of Qwen3MLP.forward (src/compute/models/qwen3.py:62-64: gate_up_proj,
 * MergedColumnParallelLinear.forward src/compute/layers/linear.py:306, with
 * the SiLU-and-mul after it, activation.py:6-8; down_proj,
 * RowParallelLinear.forward linear.py:141) and o_proj (qwen3.py:115,
 * linear.py:141); prefill and larger batches keep them on hipBLASLt.
 *   w_packed  w in 16-row x 64-column tiles of 2 KB, row blocks outermost,
 *             tile (nb, sg): w[16 nb + l % 16][64 sg + 8 (l / 16) + e] at
 *             8 l + e and w[16 nb + l % 16][64 sg + 32 + 8 (l / 16) + e] at
 *             512 + 8 l + e (l < 64, e < 8); 16-byte aligned.
 *   x         row i at i * x_stride (a multiple of 8, >= k), 16-byte aligned.
 *   mode 0    bf16 out[m, n], row stride out_stride, 8-byte aligned.
 *   mode 1    fp32 partial products of K split `parts` ways: out[p][i][j] at
 *             p * part_stride + i * out_stride + j, 16-byte aligned, strides
 *             multiples of 4; their sum over p is the product.
 *   mode 2    w is the gate/up weight [2I, k] (gate rows first); bf16
 *             out[m, I] = silu(g) * u with g, u the two products rounded to bf16.
 *   col_tiles 16-row tiles per wave (1, 2 or 4; 2 or 4 in mode 2), waves 4 or 8:
 *             n a multiple of 16 col_tiles waves; k a multiple of 256 parts.
 */
int xv_dense_gemm(const void* x, int64_t x_stride, const void* w_packed, void* out, int64_t out_stride,
                  int64_t part_stride, int m, int n, int k, int mode, int col_tiles, int waves, int parts,
                  hipStream_t stream);

/*
 * Streaming copy of `bytes` (a multiple of 16; both pointers 16-byte aligned)
 * with non-temporal 16-byte loads and stores.  No counterpart in the
 * reference: a measurement yardstick for the HBM-bound kernels above (what a
 * plain read-once / write-once transfer of the same size reaches), used by
 * the benchmark.  shape 0: one 16-byte vector per thread; shape 1: a
 * 1024-workgroup grid-stride loop, four vectors per lane per round.
 */
int xv_stream_copy(const void* src, void* dst, int64_t bytes, int shape, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* XV_KERNELS_H */
