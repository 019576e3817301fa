/*
 * needle_amd.h -- C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * These operations replace the torch statement sequences of Needle's
 * needle/layers/attention.py:
 *
 *   ndl_kv_append       scatter new K/V rows into the block pool
 *                       (decode append attention.py:141-154, _write_kv :204-246)
 *   ndl_rope_kv_append  rotary embedding of q/k fused with that append
 *                       (_apply_rope :88, :277-288)
 *   ndl_paged_decode    one-query-per-sequence attention over block_table
 *                       (_decode_pytorch :291-310, dispatched from _decode :156-159;
 *                        also covers the FlashInfer wrapper :161-197)
 *   ndl_paged_decode_append  the decode append and that attention in one launch
 *                       (_decode :141-159)
 *   ndl_rope_paged_decode_append  the same with the rotary embedding of q and of the
 *                       new key row folded in (:88 then _decode :141-159)
 *   ndl_varlen_prefill  causal attention of packed varlen prompts, reading K/V
 *                       back through block_table
 *                       (_prefill_pytorch :120-134; FlashInfer path :109-118)
 *   ndl_rope_varlen_prefill  the same with the rotary embedding of q folded in
 *                       (q's half of :88, then :102-107)
 *   ndl_kv_block_copy   whole-block copies between pools for the KV swap
 *                       (needle/model/runner.py:175-192)
 *
 * and the decoder layer's elementwise work on either side of the attention
 * (needle/model/qwen2.py:52-65):
 *
 *   ndl_rms_norm        residual add + RMSNorm + weight product in one kernel
 *                       (qwen2.py:58-63, needle/layers/norm.py:14-17)
 *   ndl_silu_mul        silu(gate) * up of the SwiGLU MLP (needle/model/llama.py:36-37)
 *   ndl_greedy_argmax   the greedy sampler's argmax for a batch of logit rows
 *                       (needle/model/sampler.py:27-28)
 *
 * Conventions (every entry point):
 *   - Plain pointers to device memory, element counts and strides in ELEMENTS.
 *   - KV pool layout (needle/model/runner.py:65-78, attention.py:9-10):
 *       kv_cache[2][num_blocks][num_kv_heads][block_size][head_dim],
 *       plane 0 = K, plane 1 = V, both contiguous.
 *   - block_table is int32 [num_seqs][bt_row_stride], the first
 *     max_blocks_per_seq entries of each row are meaningful (runner.py:220-235).
 *   - context_lens[i] = tokens already in the cache before this call
 *     (runner.py:204-218).
 *   - Work is enqueued on `stream`; nothing synchronises with the host and
 *     nothing is allocated.  Scratch memory is passed in by the caller.
 *   - Return 0 on success or a negative NDL_ERR_* code.  Never aborts.
 *   - Block ids outside [0, num_blocks) are never dereferenced: append skips
 *     such rows and attention treats such blocks as empty (the reference
 *     raises an indexing error there instead).
 */
#ifndef NEEDLE_AMD_H
#define NEEDLE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same object as hipStream_t; declared here so callers need no HIP headers. */
typedef struct ihipStream_t* ndl_stream_t;

#define NDL_ABI_VERSION 8

enum ndl_status {
  NDL_OK = 0,
  NDL_ERR_INVALID_ARG = -1,   /* null pointer, negative size, inconsistent shape */
  NDL_ERR_UNSUPPORTED = -2,   /* dtype / head_dim / block_size / group size not built */
  NDL_ERR_WORKSPACE = -3,     /* workspace smaller than the *_workspace_bytes query */
  NDL_ERR_LAUNCH = -4,        /* the HIP runtime rejected a kernel launch */
  NDL_ERR_SCRATCH_LIMIT = -5, /* the shape needs more than NDL_DECODE_STATIC_SCRATCH_BYTES */
  NDL_ERR_CAPTURE = -6        /* a device's first allocation-free call made under capture */
};

/* Size of the per-device static scratch array of ndl_paged_decode_append_noalloc. */
#define NDL_DECODE_STATIC_SCRATCH_BYTES (16u << 20)

/* Element format of the pools and activations: the model dtypes the reference runs its
 * attention in (needle/args.py:80-84, resolved at :143-153).  Every entry point takes all
 * three; bf16 and fp16 run the MFMA kernels of the 16-bit formats, float32 its own kernels
 * (fp32 MFMA, fp32 probabilities) with the same split, masking and combine rules. */
enum ndl_dtype {
  NDL_DTYPE_BF16 = 0,
  NDL_DTYPE_F16 = 1,
  NDL_DTYPE_F32 = 2
};

/* ABI version of the loaded library (NDL_ABI_VERSION at build time). */
int ndl_abi_version(void);

/* Static, human-readable text for a status code. */
const char* ndl_strerror(int status);

/*
 * Scatter-append K/V rows into the paged pool.
 *
 * Replaces: needle/layers/attention.py:141-154 (decode: one token per sequence)
 *           needle/layers/attention.py:204-246 (_write_kv: packed varlen tokens)
 *
 * Token t of sequence i (cu_seqlens[i] <= t < cu_seqlens[i+1]) is written to
 *   p   = context_lens[i] + (t - cu_seqlens[i])
 *   col = min(p / block_size, max_blocks_per_seq - 1)       (attention.py:144,235)
 *   blk = block_table[i * bt_row_stride + col]               (attention.py:145,236)
 *   kv_cache[0][blk][h][p % block_size][:] = k[t][h][:]      (attention.py:153,245)
 *   kv_cache[1][blk][h][p % block_size][:] = v[t][h][:]      (attention.py:154,246)
 * for every kv head h.  cu_seqlens == NULL means one token per sequence
 * (t == i, num_tokens == num_seqs), which is the decode form.
 *
 * k, v: [num_tokens][num_kv_heads][head_dim], token stride k_tok_stride /
 * v_tok_stride elements, rows inside a token contiguous.  The copy is
 * bit-exact.  Any head_dim whose rows are whole 16-byte chunks is accepted (a multiple of 8
 * for bf16 and fp16, of 4 for float32).
 */
int ndl_kv_append(void* kv_cache, int64_t num_blocks, int num_kv_heads, int block_size,
                  int head_dim, int dtype,
                  const void* k, int64_t k_tok_stride,
                  const void* v, int64_t v_tok_stride,
                  const int32_t* block_table, int64_t bt_row_stride, int max_blocks_per_seq,
                  const int32_t* cu_seqlens, const int32_t* context_lens,
                  int num_seqs, int64_t num_tokens, ndl_stream_t stream);

/*
 * Rotary embedding of q and k fused with the K/V append.
 *
 * Replaces: needle/layers/attention.py:88 (_apply_rope, :277-288) followed by
 *           the append of attention.py:141-154 (decode) or :204-246 (_write_kv).
 *
 * For every token t and every element d < head_dim, with half = head_dim / 2,
 *   rot(x)[d] = -x[d + half] (d < half), x[d - half] (d >= half)
 *   y[d]      = r( r(x[d] * cos[t][d]) + r(rot(x)[d] * sin[t][d]) )
 * with r the rounding to the element format (bf16, fp16 or fp32, nearest even), which is the
 * reference's op-by-op rounding in the model dtype (bit-exact).  q rotated is
 * written to q_out [num_tokens][num_heads][head_dim] (contiguous); k rotated and
 * v unchanged go to the cache slot that ndl_kv_append would pick for token t
 * (same slot rule, same handling of out-of-range block ids).  cos/sin:
 * [num_tokens][head_dim] with token stride cs_tok_stride.  head_dim must be a
 * multiple of 16 (8 for float32).  q and q_out may both be NULL: then only k is rotated and
 * k, v appended (for ndl_rope_varlen_prefill, which rotates q itself).
 */
int ndl_rope_kv_append(void* q_out, const void* q, int64_t q_tok_stride,
                       const void* k, int64_t k_tok_stride,
                       const void* v, int64_t v_tok_stride,
                       const void* cos, const void* sin, int64_t cs_tok_stride,
                       void* kv_cache, int64_t num_blocks, int num_heads, int num_kv_heads,
                       int block_size, int head_dim, int dtype,
                       const int32_t* block_table, int64_t bt_row_stride, int max_blocks_per_seq,
                       const int32_t* cu_seqlens, const int32_t* context_lens,
                       int num_seqs, int64_t num_tokens, ndl_stream_t stream);

/*
 * Bytes of scratch ndl_paged_decode needs for this shape (a fixed function of the
 * arguments and the device, 0 for an invalid shape).  partition_tokens selects the
 * split: 0 lets the library choose; -1 asks for one workgroup per (kv head, sequence)
 * whose waves combine their pieces on chip (the workspace is then a nominal 256 bytes);
 * a positive multiple of 16 asks for the stream split with partition_tokens / 16 stream
 * slots per wave (a slot is one 16-token tile; each sequence starts with one empty slot).
 * Pass the same value to ndl_paged_decode.
 */
size_t ndl_paged_decode_workspace_bytes(int num_seqs, int num_heads, int num_kv_heads,
                                        int head_dim, int max_blocks_per_seq, int block_size,
                                        int partition_tokens);

/*
 * Paged decode attention, one query token per sequence.
 *
 * Replaces: needle/layers/attention.py:291-310 (_decode_pytorch) and the
 *           FlashInfer decode wrapper :161-197.
 *
 * For sequence i, L_i = min(context_lens[i] + 1, max_blocks_per_seq * block_size)
 * tokens are attended (attention.py:299-303: the token appended by this step is
 * included; a row of the table never yields more than its width).  Query head h
 * reads kv head h / (num_heads / num_kv_heads) (attention.py:304-306).
 *   out[i][h][:] = softmax(scale * q[i][h] . K_i^T) V_i            (:307-308)
 * q: [num_seqs][num_heads][head_dim], token stride q_tok_stride.
 * out: [num_seqs][num_heads][head_dim] contiguous.  fp32 accumulation.
 * L_i <= 0 gives zeros.  Supported: bf16, fp16 and float32, block_size 16 to 1024 (powers
 * of two), head_dim 64 or 128, num_heads / num_kv_heads in 1..16.  The workspace
 * (ndl_paged_decode_workspace_bytes) is required for bf16 and fp16; calls that share one
 * must not overlap.  float32 runs one workgroup per (kv head, sequence) whatever
 * partition_tokens asks for (the value is still checked) and uses no workspace.
 */
int ndl_paged_decode(void* out, const void* q, int64_t q_tok_stride,
                     const void* kv_cache, int64_t num_blocks,
                     const int32_t* block_table, int64_t bt_row_stride, int max_blocks_per_seq,
                     const int32_t* context_lens, int num_seqs,
                     int num_heads, int num_kv_heads, int head_dim, int block_size, int dtype,
                     float scale, int partition_tokens,
                     void* workspace, size_t workspace_bytes, ndl_stream_t stream);

/*
 * The decode step of Attention._decode in one launch: the append of the step's new
 * k/v rows and the paged attention that reads them.
 *
 * Replaces: needle/layers/attention.py:141-159 (the append :141-154, then the
 *           attention :156-159, _decode_pytorch :291-310).
 *
 * Same cache bytes and the same out as ndl_kv_append (cu_seqlens NULL: k/v row i is
 * sequence i's token at position context_lens[i]) followed by ndl_paged_decode with
 * the same arguments: the wave that attends a sequence's last block attends the new row
 * in place of the row it read, and the row is written to the cache within the same call
 * (by the attending workgroup when each sequence has its own; otherwise by the kernel
 * that merges the split sequences' partials, enqueued by the same call).  k, v:
 * [num_seqs][num_kv_heads][head_dim], token strides k_tok_stride / v_tok_stride
 * (multiples of 8, 16-byte aligned rows).  Requires that no block is attended by two sequences (BlockAllocator
 * hands every block to one sequence, block_allocator.py:37-56); the workspace is the
 * one ndl_paged_decode_workspace_bytes sizes.
 */
int ndl_paged_decode_append(void* out, const void* q, int64_t q_tok_stride,
                            const void* k, int64_t k_tok_stride,
                            const void* v, int64_t v_tok_stride,
                            void* kv_cache, int64_t num_blocks,
                            const int32_t* block_table, int64_t bt_row_stride,
                            int max_blocks_per_seq, const int32_t* context_lens, int num_seqs,
                            int num_heads, int num_kv_heads, int head_dim, int block_size,
                            int dtype, float scale, int partition_tokens,
                            void* workspace, size_t workspace_bytes, ndl_stream_t stream);

/*
 * The decode step of Attention.forward from RoPE on: the rotary embedding of q and of the
 * step's new key row, the append of the new k/v rows and the paged attention, in one
 * launch (plus the merge launch of the stream split).
 *
 * Replaces: needle/layers/attention.py:88 (_apply_rope :277-288 on the decode tokens)
 *           followed by _decode :141-159 (append :141-154, _decode_pytorch :291-310).
 *
 * q, k: as produced by the projections, NOT rotated.  cos/sin: [num_seqs][head_dim] rows
 * of the new tokens (the model's get_cos_sin(positions)), token stride cs_tok_stride.  The
 * rotation is ndl_rope_kv_append's, bit for bit (the reference's rounding op for op),
 * so the cache bytes and out equal those of ndl_rope_kv_append (decode form) followed by
 * ndl_paged_decode with the rotated q.  Everything else as ndl_paged_decode_append.
 */
int ndl_rope_paged_decode_append(void* out, const void* q, int64_t q_tok_stride,
                                 const void* k, int64_t k_tok_stride,
                                 const void* v, int64_t v_tok_stride,
                                 const void* cos, const void* sin, int64_t cs_tok_stride,
                                 void* kv_cache, int64_t num_blocks,
                                 const int32_t* block_table, int64_t bt_row_stride,
                                 int max_blocks_per_seq, const int32_t* context_lens,
                                 int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                                 int block_size, int dtype, float scale, int partition_tokens,
                                 void* workspace, size_t workspace_bytes, ndl_stream_t stream);

/*
 * ndl_paged_decode_append without a workspace argument and without any allocation.
 *
 * No counterpart in the reference: this entry point is for callers that cannot allocate
 * device memory at the call (code under HIP graph capture, serving loops that forbid
 * allocation).  It calls no hipMalloc/hipFree and no allocating library routine.  The
 * split-K partials live in a static device array of NDL_DECODE_STATIC_SCRATCH_BYTES
 * (16 MiB) per GPU, held until the process ends; a shape whose
 * ndl_paged_decode_workspace_bytes exceeds that returns NDL_ERR_SCRATCH_LIMIT (the
 * Llama-3-8B decode shapes need 5-9 MB).  Same arguments, kernels, cache bytes and out as
 * ndl_paged_decode_append.  All calls on one GPU share that GPU's array: calls that
 * overlap on one GPU (different streams, or different host threads without stream order
 * between them) race and may return wrong results; calls in stream order are safe.  The
 * first call on a device looks the array's address up (hipGetSymbolAddress) with that
 * device current; that lookup may load the library's code object, which allocates, so it
 * must not happen while `stream` is being captured: such a call returns NDL_ERR_CAPTURE
 * and enqueues nothing.  A call with num_seqs = 0 (pointers unused) does only the lookup,
 * so a caller that captures makes one before its first capture on each device.
 */
int ndl_paged_decode_append_noalloc(void* out, const void* q, int64_t q_tok_stride,
                                    const void* k, int64_t k_tok_stride,
                                    const void* v, int64_t v_tok_stride,
                                    void* kv_cache, int64_t num_blocks,
                                    const int32_t* block_table, int64_t bt_row_stride,
                                    int max_blocks_per_seq, const int32_t* context_lens,
                                    int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                                    int block_size, int dtype, float scale,
                                    int partition_tokens, ndl_stream_t stream);

/*
 * Varlen causal prefill attention over the paged cache.
 *
 * Replaces: needle/layers/attention.py:120-134 (_prefill_pytorch) and the
 *           FlashInfer prefill path :109-118.
 *
 * Query token t of sequence i sits at position p = context_lens[i] + (t - cu_seqlens[i])
 * and attends cache positions 0..p of sequence i, read through block_table
 * with the same column clamp as ndl_kv_append.  K/V of the new tokens must
 * already be in the cache (call ndl_kv_append first, as _prefill does at
 * attention.py:103).  With context_lens == 0 this is exactly the
 * reference's per-sequence causal SDPA (attention.py:132); with
 * context_lens > 0 the cached prefix is attended as well.
 * q: [num_tokens][num_heads][head_dim], token stride q_tok_stride.
 * out: [num_tokens][num_heads][head_dim] contiguous.
 * max_seqlen: host-known bound on cu_seqlens[i+1] - cu_seqlens[i].
 * max_context_len: host-known bound on context_lens[i] (0 for plain prefill).
 */
int ndl_varlen_prefill(void* out, const void* q, int64_t q_tok_stride,
                       const void* kv_cache, int64_t num_blocks,
                       const int32_t* block_table, int64_t bt_row_stride, int max_blocks_per_seq,
                       const int32_t* cu_seqlens, const int32_t* context_lens,
                       int num_seqs, int64_t num_tokens, int max_seqlen, int max_context_len,
                       int num_heads, int num_kv_heads, int head_dim, int block_size, int dtype,
                       float scale, ndl_stream_t stream);

/*
 * ndl_varlen_prefill on the raw (not yet rotated) q: each query row is rotated as the
 * kernel reads it, with the rounding of ndl_rope_kv_append, so out is bit-identical to
 * ndl_rope_kv_append (q_out) followed by ndl_varlen_prefill on q_out, and no rotated q
 * is written to or read back from memory.
 *
 * Replaces: needle/layers/attention.py:88 for q (_apply_rope, :277-288) together with
 *           _prefill's attention (:102-107, _prefill_pytorch :120-134).
 *
 * cos, sin: [num_tokens][head_dim] (the rows of each packed token, as
 * ndl_rope_kv_append takes them), token stride cs_tok_stride (a multiple of 8), 16-byte
 * aligned.  K/V of the new tokens must already be in the cache, rotated: call
 * ndl_rope_kv_append with q = q_out = NULL first.  Other arguments as ndl_varlen_prefill.
 */
int ndl_rope_varlen_prefill(void* out, const void* q, int64_t q_tok_stride,
                            const void* cos, const void* sin, int64_t cs_tok_stride,
                            const void* kv_cache, int64_t num_blocks,
                            const int32_t* block_table, int64_t bt_row_stride,
                            int max_blocks_per_seq, const int32_t* cu_seqlens,
                            const int32_t* context_lens, int num_seqs, int64_t num_tokens,
                            int max_seqlen, int max_context_len, int num_heads,
                            int num_kv_heads, int head_dim, int block_size, int dtype,
                            float scale, ndl_stream_t stream);

/*
 * Copy whole KV blocks between two sets of per-layer pools: the swap-out (GPU pool ->
 * pinned CPU pool) and swap-in (CPU pool -> GPU pool) copies of a preemption.
 *
 * Replaces: needle/model/runner.py:175-192 (_swap_kv_blocks: one copy per layer and block),
 *           fed by BlockAllocator.swap_out / swap_in (block_allocator.py:88-106).
 *
 * For every layer l < num_layers, pair j < num_pairs and plane p (K, V):
 *   dst_pools[l][p][dst_ids[j]][:][:][:] = src_pools[l][p][src_ids[j]][:][:][:]
 * Pools are [2][num_blocks][num_kv_heads][block_size][head_dim] (16-byte aligned), in
 * device memory or in pinned host memory (hipHostMalloc, torch pin_memory=True), which the
 * kernel reads or writes through its device mapping; other host memory is rejected
 * (NDL_ERR_INVALID_ARG) before any launch.  src_ids / dst_ids: int32 [num_pairs] in device
 * memory or pinned host memory.  A pair with an id outside its pool is skipped.  Pairs
 * must not write one destination block twice.  One launch for all layers;
 * num_layers <= 128.  bf16, fp16 or float32 (the copy is bit-exact in every format).
 */
int ndl_kv_block_copy(void* const* dst_pools, int64_t dst_num_blocks,
                      const void* const* src_pools, int64_t src_num_blocks,
                      int num_layers, int num_kv_heads, int block_size, int head_dim, int dtype,
                      const int32_t* src_ids, const int32_t* dst_ids, int num_pairs,
                      ndl_stream_t stream);

/*
 * RMSNorm of hidden-state rows, optionally after the residual add that precedes it.
 *
 * Replaces: needle/layers/norm.py:14-17 (RMSNorm.forward) and the residual adds of
 *           needle/model/qwen2.py:58 and :63 that feed the next RMSNorm (the layer's
 *           `residual + hidden_states`, then `residual = hidden_states` and the norm).
 *
 * residual == NULL:  out = weight * round(x * rsqrt(mean(x^2) + eps))
 * residual != NULL:  h = round(x + residual) is written to residual_out (which may be
 *                    residual itself), then out = weight * round(h * rsqrt(mean(h^2) + eps))
 * with the reference's roundings: the statistic in fp32 (sum of squares times 1/hidden),
 * the normalised value rounded to the dtype, the weight product rounded again.  x: rows of
 * `hidden` elements, row stride x_row_stride (a multiple of 8, >= hidden); residual,
 * residual_out, out: contiguous [rows][hidden]; weight: [hidden]; all in `dtype`, 16-byte
 * aligned.  hidden: a multiple of 8, at most 8192 (NDL_ERR_UNSUPPORTED otherwise).
 * out must not overlap x or residual.  rows == 0 is a no-op.
 */
int ndl_rms_norm(void* out, void* residual_out, const void* x, int64_t x_row_stride,
                 const void* residual, const void* weight, int64_t rows, int hidden,
                 float eps, int dtype, ndl_stream_t stream);

/*
 * The SwiGLU activation: out[r][i] = round(round(silu(gate[r][i])) * up[r][i]),
 * silu(g) = g / (1 + exp(-g)) in fp32, rounded to the dtype as torch's silu is, then the
 * product rounded again.
 *
 * Replaces: needle/model/llama.py:37 (F.silu(gate_proj(x)) * up_proj(x), two kernels).
 *
 * gate, up: rows of `intermediate` elements, row strides gate_row_stride / up_row_stride
 * (multiples of 8; the halves of one fused gate/up projection output are gate = p,
 * up = p + intermediate with both strides 2 * intermediate); out: contiguous
 * [rows][intermediate]; 16-byte aligned; intermediate a multiple of 8.
 */
int ndl_silu_mul(void* out, const void* gate, int64_t gate_row_stride, const void* up,
                 int64_t up_row_stride, int64_t rows, int intermediate, int dtype,
                 ndl_stream_t stream);

/*
 * Greedy sampling: out[r] = the index of the maximum of logits row r, in torch's argmax
 * order (a NaN is larger than every number and the first NaN wins; of equal maxima the
 * lowest index wins).
 *
 * Replaces: needle/model/sampler.py:27-28 (int(logit.argmax()) per greedy row, each with a
 *           host sync), for every row of the batch.
 *
 * logits: rows of `vocab` elements in `dtype`, row stride row_stride (a multiple of 8,
 * >= vocab), 16-byte aligned; rows <= 65535.  out: int32 [rows] (out_is_int64 = 0) or int64
 * [rows].  Long rows are scanned in slices by several workgroups whose partial results go
 * to `workspace` (ndl_greedy_argmax_workspace_bytes(rows, vocab) bytes, 4-byte aligned; 0
 * when one slice per row suffices, then workspace may be NULL), then a second launch picks
 * each row's best.  Calls that share a workspace must be ordered (one stream).  Records no
 * memset or allocation, so it can be captured in a HIP graph.
 */
size_t ndl_greedy_argmax_workspace_bytes(int64_t rows, int vocab);
int ndl_greedy_argmax(void* out, int out_is_int64, const void* logits, int64_t row_stride,
                      int64_t rows, int vocab, int dtype, void* workspace,
                      size_t workspace_bytes, ndl_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* NEEDLE_AMD_H */
