/*
 * slipstream_hip.h -- C ABI of the MI355X (gfx950) ragged paged-attention path.
 *
 * The shared library libslipstream_hip.so exports exactly the functions below.
 * Every entry point takes plain device pointers, element counts and element
 * strides, runs asynchronously on the HIP stream it is given (NULL = default
 * stream), never synchronises and never frees memory it did not allocate.
 * Outputs and workspaces are allocated by the caller.
 *
 * Return value: SS_OK (0) on success, otherwise one of the SS_ERR_* codes;
 * ss_status_string() names it and ss_last_error() gives the detail of the
 * most recent failure on the calling thread.
 *
 * Layout contract shared with the caller (reference: slipstream/core/types.py:23-29,
 * slipstream/memory/paged_cache.py:13-28):
 *   kv_cache  [num_layers, 2, num_blocks, block_size, num_kv_heads, head_dim]
 *   slot      = block * block_size + offset           (paged_cache.py:31-32)
 *   block_tables [batch, max_blocks] int32, -1 padded (paged_cache.py:57-68)
 *   seq_lens / context_lens [batch] int32: KV length after this step's tokens
 *   were reserved (paged_cache.py:39-41).
 * Callers pass the K plane and the V plane of one layer (kv_cache[layer, 0] and
 * kv_cache[layer, 1]) as two base pointers with one shared set of strides.
 */
#ifndef SLIPSTREAM_HIP_H
#define SLIPSTREAM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SS_OK 0
#define SS_ERR_INVALID 1     /* argument or shape error (Python raises ValueError)     */
#define SS_ERR_UNSUPPORTED 2 /* shape/dtype outside the kernels' tiles (RuntimeError)  */
#define SS_ERR_LAUNCH 3      /* HIP runtime error at launch                            */
#define SS_ERR_WORKSPACE 4   /* workspace too small                                    */

#define SS_DTYPE_F16 0
#define SS_DTYPE_BF16 1
#define SS_DTYPE_F32 2

const char* ss_status_string(int status);
const char* ss_last_error(void);
/* Library version, as major*10000 + minor*100 + patch. */
int ss_version(void);

/*
 * KV-cache slot-mapping scatter.
 * Replaces slipstream/kernels/reshape_and_cache.py:10-27 (dispatcher) whose
 * fast path is reshape_and_cache_triton (slipstream/kernels/triton_paged.py:209-258)
 * and whose oracle is reshape_and_cache_ref (slipstream/kernels/attention_ref.py:21-39).
 *
 * Token n (0 <= n < n_outer*n_inner) is k[n / n_inner, n % n_inner] with head
 * stride and unit dim stride, i.e. element (n, h, d) lives at
 *   k + (n / n_inner) * k_strides[0] + (n % n_inner) * k_strides[1] + h * k_strides[2] + d.
 * ([N, n_kv, D] input: n_outer = 1, n_inner = N; the reference's [B, n_kv, T, D]
 * input: n_outer = B, n_inner = T, strides (b, t, h) -- no copy is made.)
 * It is copied bit for bit to k_cache + blk*c_strides[0] + off*c_strides[1] + h*c_strides[2] + d
 * with blk = slot / block_size, off = slot % block_size, slot = slot_mapping[n].
 * Slots < 0 are skipped (triton_paged.py:70-71); slots >= num_slots are skipped
 * as well, so a bad slot never writes outside the pool.
 * elem_bytes is 2 (fp16/bf16) or 4 (fp32); strides are in elements.
 */
int ss_reshape_and_cache(const void* k, const void* v, void* k_cache, void* v_cache,
                         const int64_t* slot_mapping, int64_t n_outer, int64_t n_inner,
                         int n_kv, int head_dim, int block_size, int64_t num_slots,
                         const int64_t k_strides[3], const int64_t v_strides[3],
                         const int64_t c_strides[3], int elem_bytes, void* stream);

/*
 * Paged attention over block tables, padded form [B, n_q, Tq, D].
 * Replaces paged_attention_decode (slipstream/kernels/paged_attention.py:21-40)
 * and paged_attention_prefill (paged_attention.py:43-52); semantics of
 * paged_attention_ref (attention_ref.py:68-89) with eager_attention
 * (slipstream/models/layers/attention.py:64-88) and the edge rules of the Triton
 * kernel (triton_paged.py:133-206): query j of sequence b sits at absolute
 * position seq_lens[b] - Tq + j and sees keys [0, seq_lens[b] - Tq + j];
 * KV head of query head h is h / (n_q / n_kv); table entries < 0 (or >= num_blocks)
 * are masked; a query row with no visible key outputs zeros.
 *
 * q(b, h, t, d)   = q   + b*q_strides[0] + h*q_strides[1] + t*q_strides[2] + d
 * out(b, t, h, d) = out + b*o_strides[0] + t*o_strides[1] + h*o_strides[2] + d
 * cache element (blk, off, h, d) = cache + blk*c_strides[0] + off*c_strides[1] + h*c_strides[2] + d
 * block_tables(b, i) = block_tables[b * bt_stride + i]
 * dtype: SS_DTYPE_BF16, SS_DTYPE_F16 or SS_DTYPE_F32 (q, cache and out share it);
 * head_dim 1..256, block_size 1..1024 (the Triton decode's range, triton_paged.py:22-23,
 * 283-284: head_dim <= 256, block_size <= 128, any float dtype). bf16 / fp16 at head_dim
 * 64, 128 or 256 with power-of-two blocks of at least 4 tokens, 16-byte aligned planes
 * and strides that are multiples of 8 elements take the MFMA decode and prefill
 * kernels; every other call takes the general kernel (fp32 arithmetic, element strides).
 * workspace: device scratch of at least ss_paged_attention_workspace_size() bytes: the
 * split-K decode partials (sized by occupancy) and, when max_query_len * n_q / n_kv
 * exceeds 16 (prefill rows), the prefill work list (4 bytes per sequence and
 * 128-row query tile), so the size depends on batch and max_query_len then; the
 * general kernel's key-split partials (at most 2 x CUs x 16 x (head_dim + 2) x 4
 * bytes) fit inside the same size.
 */
int ss_paged_attention_workspace_size(int64_t batch, int n_q, int n_kv, int head_dim,
                                      int max_query_len, int dtype, int64_t* bytes);

int ss_paged_attention(const void* q, void* out, const void* k_cache, const void* v_cache,
                       const int32_t* block_tables, const int32_t* seq_lens, int64_t batch,
                       int n_q, int n_kv, int head_dim, int tq, int max_blocks, int block_size,
                       int64_t num_blocks, const int64_t q_strides[3], const int64_t o_strides[3],
                       const int64_t c_strides[3], int64_t bt_stride, float scale, int dtype,
                       void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Packed (varlen) paged attention: one token stream q [T, n_q, D] holding the
 * query tokens of all sequences back to back; sequence b owns tokens
 * [cu_seqlens[b], cu_seqlens[b+1]) and has context_lens[b] KV tokens after this
 * step's tokens were written. The reference has no packed entry: its engine
 * runs decodes as B x 1 (llm_engine.py:540-567) and each prefill chunk as its own
 * B = 1 call (llm_engine.py:508-538); this entry equals those per-sequence calls
 * concatenated. Rows with one query token per KV head group small enough for
 * the decode tile take the split-K decode kernel, the others the MFMA prefill
 * kernel, both inside this call.
 * q(t, h, d) = q + t*q_strides[0] + h*q_strides[1] + d; out likewise with o_strides.
 */
int ss_paged_attention_varlen(const void* q, void* out, const void* k_cache, const void* v_cache,
                              const int32_t* block_tables, const int32_t* cu_seqlens,
                              const int32_t* context_lens, int64_t batch, int64_t total_tokens,
                              int n_q, int n_kv, int head_dim, int max_query_len, int max_blocks,
                              int block_size, int64_t num_blocks, const int64_t q_strides[2],
                              const int64_t o_strides[2], const int64_t c_strides[3],
                              int64_t bt_stride, float scale, int dtype, void* workspace,
                              int64_t workspace_bytes, void* stream);

/*
 * ss_paged_attention_varlen without a workspace argument: the decode split-K partials
 * and the prefill work list live in a static device array of 64 MiB per GPU
 * (allocated when the library's code object loads on that GPU, held until the
 * process ends). No counterpart in the reference: it exists for callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. Same arguments, results and errors as ss_paged_attention_varlen
 * (same kernels, bit-identical output); a call whose scratch need
 * (ss_paged_attention_workspace_size) exceeds 64 MiB fails with SS_ERR_WORKSPACE
 * before any device work. Allocates nothing. Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (two streams without ordering) race; order
 * them on one stream. No part of the array must start at zero (every kernel writes
 * what it later reads within the call).
 */
int ss_paged_attention_varlen_noalloc(const void* q, void* out, const void* k_cache, const void* v_cache,
                                      const int32_t* block_tables, const int32_t* cu_seqlens,
                                      const int32_t* context_lens, int64_t batch, int64_t total_tokens,
                                      int n_q, int n_kv, int head_dim, int max_query_len, int max_blocks,
                                      int block_size, int64_t num_blocks, const int64_t q_strides[2],
                                      const int64_t o_strides[2], const int64_t c_strides[3],
                                      int64_t bt_stride, float scale, int dtype, void* stream);

/*
 * Device status word of the current GPU, OR-ed by the attention kernels when a
 * packed description breaks the caller's promises (SS_STATUS_* bits):
 *   SS_STATUS_QUERY_TOO_LONG  a sequence of ss_paged_attention_varlen had more query
 *     tokens than max_query_len covers; its uncovered rows were written as zeros;
 *   SS_STATUS_STREAM_OVERRUN  cu_seqlens ran past total_tokens (or backwards); the
 *     kernels clamped every sequence into [0, total_tokens);
 *   SS_STATUS_PREFIX_SHORT  a sequence of ss_paged_attention_shared_prefix had fewer
 *     KV tokens than the shared prefix; its suffix counted as empty (it attended the
 *     whole prefix).
 * The reference raises ValueError at such inputs (slipstream/models/layers/attention.py:44-45);
 * a device kernel cannot, so it writes defined values and reports here. Reads the
 * word on `stream` (after the work queued there), stores it in *flags and, when `clear`
 * is nonzero, clears it in the same atomic exchange, so no bit is lost to a race with
 * kernels on other streams; bits of work still running on other streams appear in a
 * later read.
 * No counterpart in the reference (its checks are synchronous host code).
 */
#define SS_STATUS_QUERY_TOO_LONG 1
#define SS_STATUS_STREAM_OVERRUN 2
#define SS_STATUS_PREFIX_SHORT 4
int ss_attention_status(int* flags, int clear, void* stream);

/*
 * Decode (one query token per sequence) for a batch whose block tables all begin
 * with the same prefix_blocks physical blocks, the tables a prefix-cache hit
 * produces (RadixPrefixCache.match / attach: slipstream/memory/prefix_cache.py:37-56,
 * block_manager.py:91-98). Same result as paged_attention_decode
 * (slipstream/kernels/paged_attention.py:21-40, ss_paged_attention with tq = 1) up to
 * rounding, but the shared prefix is read once for the whole batch: its chunks are
 * attended by every sequence's query rows together, the private suffixes by the
 * decode, and the parts merged by log-sum-exp weights (two kernel launches plus the
 * decode's merge).
 * Caller's promise: block_tables(b, i) == block_tables(0, i) for i < prefix_blocks
 * (not checked on the device; the prefix pass reads the first row) and
 * seq_lens[b] >= prefix_blocks * block_size for every b (a shorter sequence raises
 * SS_STATUS_PREFIX_SHORT, see ss_attention_status).
 * Batches with batch * n_q / n_kv <= 16, n_q / n_kv > 16, head_dim 256 or blocks of
 * fewer than 16 tokens run the plain decode path instead.
 * q(b, h, d) = q + b*q_strides[0] + h*q_strides[1] + d; out likewise with o_strides.
 * workspace: at least ss_paged_attention_shared_prefix_workspace_size() bytes (the
 * decode partials, the prefix parts and their log-sum-exp: S * batch * n_q * head_dim
 * elements, S ~ CU count / (query tiles * n_kv), and fp32 rows of the suffixes:
 * batch * n_q * (head_dim + 2) floats).
 */
int ss_paged_attention_shared_prefix_workspace_size(int64_t batch, int n_q, int n_kv, int head_dim,
                                                    int block_size, int prefix_blocks, int dtype,
                                                    int64_t* bytes);

int ss_paged_attention_shared_prefix(const void* q, void* out, const void* k_cache, const void* v_cache,
                                     const int32_t* block_tables, const int32_t* seq_lens, int64_t batch,
                                     int n_q, int n_kv, int head_dim, int max_blocks, int block_size,
                                     int64_t num_blocks, int prefix_blocks, const int64_t q_strides[2],
                                     const int64_t o_strides[2], const int64_t c_strides[3],
                                     int64_t bt_stride, float scale, int dtype, void* workspace,
                                     int64_t workspace_bytes, void* stream);

/*
 * W4A16 linear: out[m, :] = x[m, :] @ dequant(W)^T, no bias.
 * Replaces w4a16_gemm (slipstream/kernels/quant_gemm.py:23-42), whose body is
 * w4a16_gemm_ref (slipstream/kernels/quant_ref.py:119-133); weight format of
 * quant_ref.py:8-20,45-69,103-116:
 *   qweight [n, k/8] int32, row-major: nibble j of word w of row o is q[o, 8w + j]
 *           at bits 4j..4j+3 (two's-complement storage of the 32-bit pattern);
 *   scales  [n, k/group_size], dtype scale_dtype (SS_DTYPE_F16/BF16/F32), row-major;
 *   qzeros  [n, k/group_size] int32, row-major (values 0..15 as produced by
 *           quantize_w4a16; any int32 is accepted);
 *   w[o, c] = (q[o, c] - qzeros[o, c / group_size]) * scales[o, c / group_size].
 * x [m, k] with row stride x_stride (elements, unit column stride), dtype
 * act_dtype (SS_DTYPE_BF16/F16/F32); out [m, n] with row stride o_stride, same
 * dtype as x. Accumulation is fp32 with the exact dequantised weight.
 * group_size must be a positive multiple of 8 dividing k (else SS_ERR_INVALID,
 * quant_ref.py:38-42). bf16/fp16 activations with k % 128 == 0 and
 * group_size % 32 == 0 (16-byte aligned x rows and qweight, n*k/2 < 2^31, and
 * a per-workgroup scale table of 16 * (2*k/group_size + 2) floats within 64 KiB
 * of LDS: k/group_size <= 480 for m <= 16) take the MFMA kernels (m = 1: a
 * bandwidth GEMV; m >= 2 with group_size % 128 == 0: a tiled kernel that may
 * split K over workgroups); everything else a scalar fp32 kernel. The result
 * does not depend on timing: split-K partials are added in range order, by a
 * second kernel or (two ranges, n % 4 == 0) by the last range of each output tile
 * to finish, which a device-scope compare-and-swap on a tagged arrival word in
 * the workspace identifies; never by atomic adds.
 * workspace: ss_w4a16_workspace_size() reports the bytes of the split-K
 * partials (ranges * m * n floats) and the arrival words after them (8 bytes
 * per output tile); 0 when the plan does not split. Pass at least that many
 * bytes, 16-byte aligned, with any contents (each call tags its words, and the
 * last range leaves them zero); with less (or NULL, 0) the call still succeeds
 * on the untiled MFMA kernel, which needs no scratch. Calls that share one
 * workspace must be ordered on one stream.
 */
int ss_w4a16_workspace_size(int64_t m, int64_t n, int64_t k, int group_size, int act_dtype,
                            int64_t* bytes);

int ss_w4a16_gemm(const void* x, void* out, const int32_t* qweight, const void* scales,
                  const int32_t* qzeros, int64_t m, int64_t n, int64_t k, int group_size,
                  int64_t x_stride, int64_t o_stride, int act_dtype, int scale_dtype,
                  void* workspace, int64_t workspace_bytes, void* stream);

/*
 * KV page copies: for each pair i, page pairs[2i + 1] of dst <- page pairs[2i] of
 * src, in every plane p in [0, planes) (a plane is one (layer, K/V) of
 * kv_cache[L, 2, NB, ...], so planes = 2L for a contiguous cache). Page b of plane
 * p starts at base + p * plane_stride + b * block_stride (bytes) and is page_bytes
 * contiguous bytes (block_size * n_kv * head_dim * element size). pairs is a
 * device int64 array [n_pairs, 2]; pairs with an id outside [0, *_blocks) are
 * skipped. A byte copy, bit exact.
 *   dst == src: replaces copy_blocks_ref (slipstream/kernels/attention_ref.py:92-94),
 *     the copy-on-write copy of slipstream/memory/block_manager.py:297-298. All
 *     pairs of one call run at once: a destination that is also a source, or a
 *     repeated destination, makes the order matter -- split such lists into
 *     ordered calls (the Python wrapper does).
 *   one side a pinned host cache (hipHostMalloc, torch pin_memory): the swap
 *     copies of block_manager.py:196-200 (out) and :220-225 (in), read or written
 *     through the host memory's device mapping. Pageable host memory is
 *     SS_ERR_INVALID.
 */
int ss_copy_blocks(void* dst, const void* src, int64_t planes, int64_t dst_plane_stride,
                   int64_t dst_block_stride, int64_t dst_blocks, int64_t src_plane_stride,
                   int64_t src_block_stride, int64_t src_blocks, int64_t page_bytes,
                   const int64_t* pairs, int64_t n_pairs, void* stream);

/*
 * Rotary embedding of Q and K fused with the KV scatter: replaces
 * apply_rotary_pos_emb (slipstream/models/layers/rope.py:20-36) followed by
 * reshape_and_cache (slipstream/kernels/reshape_and_cache.py:10-27) as
 * Attention.forward runs them (slipstream/models/layers/attention.py:163,171-174);
 * the reference's fuse seam is slipstream/kernels/fused_rope.py:168-181.
 *   q_out[n, h]          = rope(q[n, h])            (h < n_q)
 *   k_cache[slot(n), h]  = rope(k[n, h])            (h < n_kv, slot(n) >= 0)
 *   v_cache[slot(n), h]  = v[n, h]
 * rope(x) = x * cos[n] + rotate_half(x) * sin[n], rotate_half(x) = cat(-x2, x1),
 * rounded as the reference's torch ops round: each product and the sum computed
 * in fp32 and rounded to dtype (no fused multiply-add for fp32) -- bit identical.
 * Token n = o * n_inner + i (o < n_outer, i < n_inner). Strides are in elements:
 * q/k/v/o strides are (outer, inner, head) with unit head_dim stride; cos/sin
 * strides are (outer, inner) with unit head_dim stride (0 broadcasts); c_strides
 * are the cache planes' (block, position, head) strides as for
 * ss_reshape_and_cache. Slots < 0 or >= num_slots are skipped. head_dim even;
 * dtype SS_DTYPE_BF16/F16/F32 for every tensor (cos/sin in the tensors' dtype,
 * as RotaryEmbedding returns them, rope.py:106).
 */
int ss_rope_and_cache(const void* q, const void* k, const void* v, const void* cos, const void* sin,
                      void* q_out, void* k_cache, void* v_cache, const int64_t* slot_mapping,
                      int64_t n_outer, int64_t n_inner, int n_q, int n_kv, int head_dim, int block_size,
                      int64_t num_slots, const int64_t q_strides[3], const int64_t k_strides[3],
                      const int64_t v_strides[3], const int64_t o_strides[3], const int64_t cos_strides[2],
                      const int64_t sin_strides[2], const int64_t c_strides[3], int dtype, void* stream);

/*
 * Packed-step metadata on the device: replaces the host-list building of
 * build_paged_forward (slipstream/memory/paged_cache.py:71-109) and the packed
 * description ss_paged_attention_varlen takes. From block_tables [batch, >= max_blocks]
 * (int32, row stride bt_stride, -1 padded), prior_lens [batch] (KV tokens before the
 * step) and query_lens [batch] (new tokens), all int32 on the device:
 *   cu_seqlens [batch + 1]  exclusive prefix sum of query_lens;
 *   context_lens [batch]    prior_lens + query_lens (the reference's seq_lens);
 *   slot_mapping [total_tokens] int64: token j of sequence b (position
 *     p = prior_lens[b] + j) -> table[b][p / block_size] * block_size + p % block_size,
 *     the slot BlockManagerImpl.append_slot hands out when earlier blocks are full
 *     (block_manager.py:141-159); -1 past the table or on a negative entry.
 * Negative lengths count as 0; tokens past total_tokens are not written, and entries
 * [sum(query_lens), total_tokens) of slot_mapping are set to -1 (skipped by the
 * scatter), so an over-sized slot_mapping never holds a stale slot. Nothing
 * is read back to the host, so a step built this way can be graph-captured.
 */
int ss_build_step_metadata(const int32_t* block_tables, int64_t bt_stride, int max_blocks,
                           const int32_t* prior_lens, const int32_t* query_lens, int batch,
                           int block_size, int32_t* cu_seqlens, int32_t* context_lens,
                           int64_t* slot_mapping, int64_t total_tokens, void* stream);

/*
 * RMSNorm with an optional residual add: replaces fused_rmsnorm
 * (slipstream/kernels/fused_rmsnorm.py:125-137) with the eager path's rounding
 * (rmsnorm.py:30-33, fused_rmsnorm.py:73-82): s = x + residual in dtype,
 * out = weight * dtype(s * rsqrt(mean(s^2) + eps)) with the variance in fp32.
 * x, residual (or NULL), out: [rows, cols] with row strides in elements; weight
 * [cols]. 16-byte aligned rows, cols a multiple of 8 (16-bit) or 4 (fp32);
 * otherwise SS_ERR_UNSUPPORTED. Rows of up to 2048 16-byte pieces are held in
 * registers; longer ones are read twice.
 */
int ss_rmsnorm(const void* x, const void* residual, const void* weight, void* out, int64_t rows, int cols,
               int64_t x_stride, int64_t r_stride, int64_t o_stride, float eps, int dtype, void* stream);

/*
 * SwiGLU: out = silu(gate) * up with the eager path's rounding (silu rounded to
 * dtype, then the product): replaces fused_swiglu (slipstream/kernels/fused_swiglu.py:72-79)
 * as MLP.forward runs it (slipstream/models/layers/mlp.py:37-40). [rows, cols], row
 * strides in elements, 16-byte aligned rows, cols a multiple of 8 (16-bit) or 4.
 */
int ss_swiglu(const void* gate, const void* up, void* out, int64_t rows, int cols, int64_t g_stride,
              int64_t u_stride, int64_t o_stride, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SLIPSTREAM_HIP_H */
