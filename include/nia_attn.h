/*
 * nia_attn.h - C ABI of the MI355X (gfx950) attention library for nano-inference.
 *
 * The library (libnia_attn.so) holds hand-written HIP kernels for the attention
 * hot path of nano-inference and nothing else.  Every entry point:
 *   - takes plain device pointers, sizes and element strides (no framework types);
 *   - enqueues its kernels on the caller's HIP stream (`stream`, a hipStream_t,
 *     NULL = the legacy default stream) and returns without synchronising;
 *   - returns NIA_OK (0) or a nonzero status; nia_error_string() names it.
 *     Status codes are returned for bad arguments before anything is launched,
 *     so a caller can fail one batch without tearing the process down.
 *   - allocates no device memory: outputs and scratch (`workspace`) belong to
 *     the caller (nia_paged_decode_noalloc uses a fixed array of the library's
 *     own instead, see there).
 *
 * Index dtypes follow the reference engine's metadata:
 *   slot_mapping int64 with -1 padding, block tables int32 zero-padded,
 *   context_lens int64 (src/nano_inference/engine/context_builder.py:121,154-159).
 * KV-cache layout is one layer's slice of the allocator's pool,
 *   [num_blocks, num_kv_heads, block_size, head_dim], contiguous
 *   (src/nano_inference/kv_cache/allocator.py:35-39, layers/attention.py:244-245).
 * Query head h reads KV head h / (num_heads / num_kv_heads)
 *   (repeat_interleave at src/nano_inference/layers/attention.py:310-314).
 *
 * The reference engine has no native code: every function below replaces a
 * sequence of PyTorch ops, cited per function.
 */
#ifndef NIA_ATTN_H
#define NIA_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types (`dtype` arguments) */
#define NIA_DTYPE_BF16 0
#define NIA_DTYPE_F32 1

/* causal modes (`causal` arguments of the prefill entry points) */
#define NIA_CAUSAL_NONE 0         /* every query row sees all k_len keys            */
#define NIA_CAUSAL_TOP_LEFT 1     /* row j sees keys [0, min(j + 1, k_len))         */
#define NIA_CAUSAL_BOTTOM_RIGHT 2 /* row j sees keys [0, k_len - q_len + j + 1)     */

/* status codes */
#define NIA_OK 0
#define NIA_ERR_INVALID_ARGUMENT 1 /* a null pointer, a negative size, a bad stride     */
#define NIA_ERR_UNSUPPORTED 2      /* a shape/dtype combination with no kernel         */
#define NIA_ERR_WORKSPACE 3        /* workspace missing or smaller than required       */
#define NIA_ERR_LAUNCH 4           /* the HIP runtime refused the kernel launch        */
#define NIA_ERR_MISALIGNED 5       /* a pointer or stride breaks 16-byte vector access */
#define NIA_ERR_SCRATCH_LIMIT 6    /* the call needs more than the library's fixed scratch */

/* Library ABI version; bumped whenever a signature below changes or an entry point is added. */
int32_t nia_abi_version(void);

/* Human-readable name of a status code (static storage, never NULL). */
const char* nia_error_string(int32_t status);

/*
 * KV-cache write: scatter the step's new K/V rows into their physical slots.
 * Replaces the per-token loop of src/nano_inference/layers/attention.py:267-278:
 *   for each token t with slot = slot_mapping[t] >= 0:
 *     k_cache[slot // block_size, :, slot % block_size, :] = k[t]   (same for v)
 * The copy is bit-exact (no conversion).  Tokens with slot < 0 are skipped, as
 * are slots >= num_blocks * block_size (the reference would raise; the Python
 * host layer validates when asked to).
 *   k, v          [num_tokens, num_kv_heads, head_dim] with element strides
 *                 (k_tok_stride, k_head_stride), (v_tok_stride, v_head_stride);
 *                 the last dimension is contiguous.
 *   slot_mapping  [num_tokens] int64 (the reference's (B, S_step) tensor flattened).
 */
int32_t nia_kv_write(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                     const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                     void* k_cache, void* v_cache, const int64_t* slot_mapping,
                     int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                     int32_t block_size, int64_t num_blocks, int32_t dtype, void* stream);

/*
 * Paged decode attention: one query token per sequence against its cached keys.
 * Replaces the decode branch of src/nano_inference/layers/attention.py:285-332
 * (block-table gather, GQA repeat_interleave, context-length mask, and
 * scaled_dot_product_attention at :12-50 with S_q = 1):
 *   out[b, h] = softmax(scale * q[b, h] . K[b, :L_b]^T) V[b, :L_b]
 * with L_b = context_lens[b] and key t of sequence b at block
 * block_tables[b, t / block_size], offset t % block_size.
 * Keys at t >= L_b are never read, so padded table entries (the reference reads
 * block 0 there and masks it) cannot affect the output.  Sequences with L_b <= 0
 * produce zeros.  Keys in blocks with ids outside [0, num_blocks) are skipped.
 *   q, out       [batch, num_heads, head_dim] with element strides (batch, head).
 *   block_tables [batch, bt_stride] int32, the first max_blocks_per_seq columns used.
 *   workspace    >= nia_paged_decode_workspace_size(...) bytes of device memory,
 *                256-byte aligned (partial results; nothing in it needs to be
 *                initialised).  Calls that overlap in time need workspaces of their
 *                own; calls issued one after another may share one.
 * Supported:
 *   dtype bf16 (fp32 softmax and accumulation): any block_size >= 1 (the reference's
 *     block size is a free integer, src/nano_inference/core/config.py:54), head_dim
 *     64, 80, 96 or 128, any num_heads / num_kv_heads, max_blocks_per_seq * block_size
 *     < 2^31.  Block sizes that are multiples of 4 run the key-range split kernels
 *     (groups of more than 16 query heads per KV head as several launches of at most 16
 *     heads each, which share the workspace one after another on the stream); other
 *     block sizes run the kernel of the f32 path below over bf16 rows (q . k in fp64;
 *     ~25x slower on the Qwen3-8B decode; no partials, so the workspace size is the
 *     256-byte header);
 *   dtype f32 (q . k summed in fp64): any block_size, head_dim 64, 80, 96 or 128, any
 *     num_heads / num_kv_heads.
 */
size_t nia_paged_decode_workspace_size(int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                       int32_t max_blocks_per_seq, int32_t block_size,
                                       int32_t head_dim, int32_t dtype);

int32_t nia_paged_decode(void* out, int64_t out_batch_stride, int64_t out_head_stride,
                         const void* q, int64_t q_batch_stride, int64_t q_head_stride,
                         const void* k_cache, const void* v_cache,
                         const int32_t* block_tables, int32_t bt_stride,
                         int32_t max_blocks_per_seq, const int64_t* context_lens,
                         int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                         int32_t head_dim, int32_t block_size, int64_t num_blocks,
                         float scale, void* workspace, size_t workspace_bytes,
                         int32_t dtype, void* stream);

/*
 * Paged decode that allocates nothing and takes no workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops and harnesses that forbid hipMalloc).  Same arguments,
 * kernels and results as nia_paged_decode (bf16 or f32 caches), with the workspace
 * replaced by a fixed array of NIA_DECODE_SCRATCH_BYTES in the library's device
 * memory (one per GPU, held until the process ends).  A call whose
 * nia_paged_decode_workspace_size(...) exceeds it returns NIA_ERR_SCRATCH_LIMIT before
 * anything is launched.  40 MiB holds every bf16 layout the split kernel takes (up to
 * 16 query heads per KV head at head_dim 128: 34.1 MB of partials) with 4 + 8 x
 * num_kv_heads bytes per sequence beside them, i.e. batches up to 115,000 sequences at 8
 * KV heads; fp32 calls need batch x num_heads x ceil(max_blocks / 32) x
 * (head_dim + 2) x 4 bytes (plus 256), so long fp32 batches can exceed it.  All calls
 * on one GPU share the array: calls that overlap in time on one GPU (other streams,
 * other threads) race.
 */
#define NIA_DECODE_SCRATCH_BYTES (40u << 20)

int32_t nia_paged_decode_noalloc(void* out, int64_t out_batch_stride, int64_t out_head_stride,
                                 const void* q, int64_t q_batch_stride, int64_t q_head_stride,
                                 const void* k_cache, const void* v_cache,
                                 const int32_t* block_tables, int32_t bt_stride,
                                 int32_t max_blocks_per_seq, const int64_t* context_lens,
                                 int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                 int32_t head_dim, int32_t block_size, int64_t num_blocks,
                                 float scale, int32_t dtype, void* stream);

/*
 * Varlen prefill attention over contiguous K/V (causal or not).
 * Replaces the prefill branch of src/nano_inference/layers/attention.py:281-284
 * with scaled_dot_product_attention (:12-50, causal triu at :33-38, padding
 * mask at :40-47), and the per-chunk loop of the vision tower
 * (src/nano_inference/layers/vision.py:190-208, is_causal=False).
 * Sequence s owns query rows [q_start[s], q_start[s] + q_len[s]) and key/value
 * rows [k_start[s], k_start[s] + k_len[s]); this covers the packed cu_seqlens
 * layout (q_start = cu[:-1]) and the reference's padded (B, S_max) layout
 * (q_start[s] = s * S_max).  Rows are visited by token index, so q/k/v/out are
 * [tokens, heads, head_dim] with element strides (tok, head).
 * Query rows that see no key produce zeros.
 *   max_q_len  upper bound of q_len[s] (sizes the grid; larger is allowed).
 * Supported: dtype bf16 (fp32 softmax and accumulation) or f32 (scores summed in fp64,
 * softmax and P V in fp32; rows and strides 16-byte aligned); head_dim 64, 80, 96 or
 * 128; num_heads % num_kv_heads == 0.
 */
int32_t nia_prefill(void* out, int64_t out_tok_stride, int64_t out_head_stride,
                    const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                    const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                    const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                    const int32_t* q_start, const int32_t* q_len,
                    const int32_t* k_start, const int32_t* k_len,
                    int32_t num_seqs, int32_t max_q_len, int32_t num_heads,
                    int32_t num_kv_heads, int32_t head_dim, float scale, int32_t causal,
                    int32_t dtype, void* stream);

/*
 * nia_prefill with an additive mask of any shape.  Replaces the general form of the
 * reference's mask at src/nano_inference/layers/attention.py:40-47, which adds any
 * broadcastable attention_mask (sliced to S_k) to the scaled scores before the fp32
 * softmax; nia_prefill covers the prefix masks the reference's own callers build
 * (context_builder.py:141-149 through :321-326) by key lengths.  mask is fp32, 16-byte
 * aligned; the value added to the scaled score of query row i (within its sequence) and
 * key j of sequence s and query head h is
 *     mask[s * mask_seq_stride + h * mask_head_stride + i * mask_q_stride + j]
 * (element strides, multiples of 4 and >= 0; 0 broadcasts), read for keys j < k_len[s]
 * and rows i < q_len[s] only; the library cannot see the mask's extent, so every such
 * element must lie inside it (the Python op checks the shape first).  -inf masks a key; the causal mode still applies.  A row
 * whose every key is masked produces zeros (the reference's softmax gives NaN there).
 * Same support as nia_prefill, except that bf16 K/V token strides must stay below 2^26
 * elements (else NIA_ERR_UNSUPPORTED); mask == NULL returns NIA_ERR_INVALID_ARGUMENT.
 */
int32_t nia_prefill_masked(void* out, int64_t out_tok_stride, int64_t out_head_stride,
                           const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                           const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                           const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                           const int32_t* q_start, const int32_t* q_len,
                           const int32_t* k_start, const int32_t* k_len,
                           int32_t num_seqs, int32_t max_q_len, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, float scale, int32_t causal,
                           int32_t dtype, const float* mask, int64_t mask_seq_stride,
                           int64_t mask_head_stride, int64_t mask_q_stride, void* stream);

/*
 * Chunked prefill over the paged KV cache.  Has no counterpart in the
 * reference, whose prefill ignores the cache (src/nano_inference/layers/
 * attention.py:281-284); it is the cache-reading generalisation of nia_prefill
 * that chunked prefill needs.  Sequence s has q_len[s] new query rows at
 * absolute positions context_lens[s] - q_len[s] + j (their K/V already written
 * by nia_kv_write) and reads its keys [0, context_lens[s]) through
 * block_tables exactly as nia_paged_decode does.  `causal` is normally
 * NIA_CAUSAL_BOTTOM_RIGHT; NIA_CAUSAL_NONE lets every row see the whole context.
 * Supported: head_dim 64, 80, 96 or 128; dtype bf16 or f32 with any block_size >= 1
 * and max_blocks_per_seq * block_size < 2^31 (keys in blocks outside [0, num_blocks)
 * are skipped).  bf16 block sizes >= 2 run the MFMA kernels (multiples of 4 stream rows
 * into LDS by DMA, 16-row groups of a block or, when 16 does not divide the block size,
 * 4-row groups; other sizes take register-staged loads, ~2.5x slower); bf16 block size
 * 1, and f32, run the f32 kernel (q . k in fp64, bf16 rows widened on load).
 */
int32_t nia_prefill_paged(void* out, int64_t out_tok_stride, int64_t out_head_stride,
                          const void* q, int64_t q_tok_stride, int64_t q_head_stride,
                          const void* k_cache, const void* v_cache,
                          const int32_t* block_tables, int32_t bt_stride,
                          int32_t max_blocks_per_seq, const int32_t* q_start,
                          const int32_t* q_len, const int64_t* context_lens,
                          int32_t num_seqs, int32_t max_q_len, int32_t num_heads,
                          int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                          int64_t num_blocks, float scale, int32_t causal, int32_t dtype,
                          void* stream);

/*
 * Fused QK-RMSNorm + RoPE / mRoPE + KV-cache write, in place on q and k.
 * Replaces the steps between the projections and attention in
 * src/nano_inference/layers/attention.py:254-278: q_norm / k_norm
 * (src/nano_inference/layers/norm.py:35-47), the rotary embedding
 * (src/nano_inference/layers/rotary.py:8-33, :104-130; 3-axis mRoPE :184-210) and
 * the cache write loop, with the same fp32 computation and the same rounding to
 * the model dtype after every PyTorch op (only the order of the RMSNorm sum of
 * squares differs, which can change the last bit of a value on a rounding boundary).
 *   q [num_tokens, num_heads, 128], k and v [num_tokens, num_kv_heads, 128] with
 *     element strides (tok, head); q and k are overwritten with their normalised,
 *     rotated values.
 *   q_norm_weight, k_norm_weight  [128] in the model dtype, or NULL for no QK norm
 *     (both are applied when given; eps as the reference module's).
 *   positions  [num_axes][num_tokens] int64 with axis stride pos_axis_stride:
 *     num_axes 1 = RoPE position ids, 3 = mRoPE (temporal, height, width), whose
 *     frequency i uses axis 0 for i < mrope_section0, axis 1 for
 *     i < mrope_section0 + mrope_section1, else axis 2.
 *   inv_freq  [64] fp32, the module's table (base^(-2i / 128)).
 *   k_cache, v_cache  one layer [num_blocks, num_kv_heads, block_size, 128], or NULL
 *     for no write; tokens whose slot_mapping entry is < 0 or >= num_blocks *
 *     block_size are not written (as nia_kv_write).
 * Supported: head_dim 128; dtype bf16 or f32.
 */
int32_t nia_qk_norm_rope_kv_write(void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                  void* k, int64_t k_tok_stride, int64_t k_head_stride,
                                  const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                                  const void* q_norm_weight, const void* k_norm_weight,
                                  float eps, const int64_t* positions,
                                  int64_t pos_axis_stride, int32_t num_axes,
                                  const float* inv_freq, int32_t mrope_section0,
                                  int32_t mrope_section1, void* k_cache, void* v_cache,
                                  const int64_t* slot_mapping, int32_t num_tokens,
                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                  int32_t block_size, int64_t num_blocks, int32_t dtype,
                                  void* stream);

/*
 * fp8 KV-cache format (no counterpart in the reference, whose caches hold the model
 * dtype, src/nano_inference/kv_cache/allocator.py:35-39): each (token, KV head) row
 * of head_dim values is stored as OCP float8 e4m3 codes (uint8; 4 exponent bits,
 * bias 7, max 448, torch.float8_e4m3fn) with one fp32 scale per row in
 * k_scale / v_scale [num_blocks, num_kv_heads, block_size]:
 *   scale = max_d |x_d| / 448,  code_d = e4m3(x_d / scale) (round to nearest even),
 *   x_d ~= code_d * scale;  a zero row stores scale 0 and zero codes.
 * Half the cache bytes of bf16, so paged decode reads half the bytes.
 */

/*
 * KV-cache write into fp8 caches: the loop of src/nano_inference/layers/
 * attention.py:267-278 with each row quantised as above.  k, v as nia_kv_write
 * (bf16 or f32 in `dtype`); k_cache, v_cache uint8 [num_blocks, num_kv_heads,
 * block_size, 128]; slots < 0 or >= num_blocks * block_size are skipped.
 * Supported: head_dim 128.
 */
int32_t nia_kv_write_fp8(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                         const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                         void* k_cache, void* v_cache, float* k_scale, float* v_scale,
                         const int64_t* slot_mapping, int32_t num_tokens, int32_t num_kv_heads,
                         int32_t head_dim, int32_t block_size, int64_t num_blocks, int32_t dtype,
                         void* stream);

/*
 * nia_qk_norm_rope_kv_write with fp8 caches: q and k are normalised and rotated in
 * place exactly as there, and the rotated k row and the v row are written to the
 * caches in the fp8 format above (k_cache, v_cache uint8; k_scale, v_scale fp32).
 */
int32_t nia_qk_norm_rope_kv_write_fp8(void* q, int64_t q_tok_stride, int64_t q_head_stride,
                                      void* k, int64_t k_tok_stride, int64_t k_head_stride,
                                      const void* v, int64_t v_tok_stride,
                                      int64_t v_head_stride, const void* q_norm_weight,
                                      const void* k_norm_weight, float eps,
                                      const int64_t* positions, int64_t pos_axis_stride,
                                      int32_t num_axes, const float* inv_freq,
                                      int32_t mrope_section0, int32_t mrope_section1,
                                      void* k_cache, void* v_cache, float* k_scale,
                                      float* v_scale, const int64_t* slot_mapping,
                                      int32_t num_tokens, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t head_dim,
                                      int32_t block_size, int64_t num_blocks, int32_t dtype,
                                      void* stream);

/*
 * Paged decode over fp8 caches: nia_paged_decode with k_cache / v_cache in the fp8
 * format above (uint8 codes, k_scale / v_scale fp32 [num_blocks, num_kv_heads,
 * block_size], 16-byte aligned, else NIA_ERR_MISALIGNED).  q and out are bf16; keys
 * are dequantised exactly as code * row scale (the code is widened to bf16 without
 * rounding, the scale multiplies the q . k score, and each softmax weight carries its
 * row's v scale).  Same workspace contract as nia_paged_decode (its size with dtype
 * NIA_DTYPE_BF16); head_dim 128, any block_size >= 1, any num_heads / num_kv_heads
 * (as nia_paged_decode).  Block sizes that are multiples of 16 run the split kernels
 * (a 16-key tile in one block); other sizes run the f32 path's kernel over rows
 * dequantised on load as code * row scale in fp32 (far slower).
 */
int32_t nia_paged_decode_fp8(void* out, int64_t out_batch_stride, int64_t out_head_stride,
                             const void* q, int64_t q_batch_stride, int64_t q_head_stride,
                             const void* k_cache, const void* v_cache, const float* k_scale,
                             const float* v_scale, const int32_t* block_tables,
                             int32_t bt_stride, int32_t max_blocks_per_seq,
                             const int64_t* context_lens, int32_t batch, int32_t num_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             int64_t num_blocks, float scale, void* workspace,
                             size_t workspace_bytes, void* stream);

/*
 * fp8 cache -> contiguous bf16 rows, for chunked prefill over an fp8 cache: the keys
 * [0, context_lens[s]) of sequence s, gathered through its block table as
 * nia_paged_decode reads them and dequantised (code * row scale, rounded to bf16),
 * land in rows s * seq_stride + t of out_k / out_v [batch * seq_stride][num_kv_heads]
 * [128] (seq_stride >= max_blocks_per_seq * block_size; rows past a context are not
 * written).  nia_prefill over those rows with k_start[s] = s * seq_stride and
 * NIA_CAUSAL_BOTTOM_RIGHT then gives nia_prefill_paged's result.
 */
int32_t nia_dequant_gather_fp8(const void* k_cache, const void* v_cache, const float* k_scale,
                               const float* v_scale, const int32_t* block_tables,
                               int32_t bt_stride, int32_t max_blocks_per_seq,
                               const int64_t* context_lens, int32_t batch, int32_t num_kv_heads,
                               int32_t head_dim, int32_t block_size, int64_t num_blocks,
                               void* out_k, void* out_v, int64_t seq_stride, void* stream);

/*
 * Step metadata: the padded model inputs and attention metadata of one engine
 * step, expanded on the device from a compact descriptor (one upload per step).
 * Replaces the loops of src/nano_inference/engine/context_builder.py:83-193
 * (input_ids, position_ids, context_lens, attention_mask, block tables, slot
 * mapping) and :18-81 (mRoPE positions).
 *   desc  int64, sections back to back:
 *     [batch][8] headers: step_len, start_pos, num_blocks, token_offset,
 *       block_offset, mrope_explicit e, mrope_offset, mrope_base c;
 *     [num_tokens] step token ids; [num_blocks] block ids; [num_mrope] explicit
 *       mRoPE rows (3 x e per sequence with e > 0).
 *   Outputs, i < batch, j < max_step:
 *     input_ids, position_ids, slot_mapping  [batch][max_step] int64
 *       (0, 0, -1 past step_len; a position past the block list uses the last
 *       block, as :176-189 does);
 *     context_lens, last_index  [batch] int64 (start + step_len, step_len - 1);
 *     attention_mask  [batch][max_total] bool, j < context_lens[i];
 *     block_tables  [batch][max_blocks] int32, zero-padded;
 *     mrope  [3][batch][max_step] int64 or NULL: explicit rows for j < e, then
 *       c + j - e up to step_len, 0 past it.
 * Descriptor reads are bounds-checked against the section lengths given.
 */
int32_t nia_step_metadata(const int64_t* desc, int64_t num_tokens, int64_t num_blocks,
                          int64_t num_mrope, int32_t batch, int32_t max_step,
                          int32_t max_total, int32_t max_blocks, int32_t block_size,
                          int64_t* input_ids, int64_t* position_ids, int64_t* slot_mapping,
                          int64_t* context_lens, int64_t* last_index, void* attention_mask,
                          int32_t* block_tables, int64_t* mrope, void* stream);

/*
 * Packed step metadata for batches that mix prefill chunks and decodes (no
 * counterpart in the reference, whose batches are all-prefill or all-decode,
 * src/nano_inference/scheduler/scheduler.py:176-230): the same expansion as
 * nia_step_metadata, with the step's tokens back to back instead of padded.
 *   desc  int64: [batch][8] headers (step_len, start_pos, num_blocks,
 *     token_offset, block_offset, out_offset, device_token_index, 0), then
 *     [num_tokens] token ids, then [num_blocks] block ids.
 *   A sequence with device_token_index >= 0 reads its step tokens from
 *   device_tokens[device_token_index + j] (tokens sampled on the device).
 *   Outputs: input_ids, position_ids, slot_mapping [num_rows] int64 at rows
 *     out_offset + j (num_rows = total step tokens; rows outside are not written); context_lens [batch] int64;
 *     last_index [batch] int64 (out_offset + step_len - 1); q_start, q_len
 *     [batch] int32 (out_offset, step_len: the varlen description nia_prefill_paged
 *     takes); block_tables [batch][max_blocks] int32, zero-padded.
 * Descriptor and device-token reads are bounds-checked against the lengths given.
 */
int32_t nia_step_metadata_packed(const int64_t* desc, int64_t num_tokens, int64_t num_blocks,
                                 const int64_t* device_tokens, int64_t num_device_tokens,
                                 int32_t batch, int64_t num_rows, int32_t max_step,
                                 int32_t max_blocks,
                                 int32_t block_size, int64_t* input_ids, int64_t* position_ids,
                                 int64_t* slot_mapping, int64_t* context_lens,
                                 int64_t* last_index, int32_t* q_start, int32_t* q_len,
                                 int32_t* block_tables, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NIA_ATTN_H */
