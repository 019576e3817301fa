// Scatter-append of new K/V rows into the paged pool.
//
// Reference: needle/layers/attention.py:141-154 (decode append) and
// attention.py:204-246 (_write_kv).  The reference derives the slot of every
// token with host round trips (context_lens.cpu(), a Python loop of aranges,
// repeat_interleave) and then issues 2*num_kv_heads index_put_ launches.
// Here one launch moves both planes: every thread copies one 16-byte chunk
// of one (token, kv head) row and derives the slot on the device.
#include "ndl_common.hpp"

namespace ndl {

// Largest i in [0, n) with cu[i] <= t (cu is non-decreasing, cu[0] == 0).
__device__ __forceinline__ int seq_of_token(const int32_t* __restrict__ cu, int n, int64_t t) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((int64_t)cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// grid.x covers num_tokens * num_kv_heads * chunks_per_row chunks, grid.y = plane (0 K, 1 V).
__global__ __launch_bounds__(256) void kv_append_kernel(
    u16* __restrict__ cache, int64_t plane_elems, int64_t num_blocks, int num_kv_heads,
    int block_size, int head_dim,
    const u16* __restrict__ k, int64_t k_tok_stride,
    const u16* __restrict__ v, int64_t v_tok_stride,
    const int32_t* __restrict__ block_table, int64_t bt_row_stride, int max_blocks,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ context_lens,
    int num_seqs, int64_t num_tokens) {
  const int chunks_per_row = head_dim >> 3;
  const int64_t chunk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = num_tokens * num_kv_heads * chunks_per_row;
  if (chunk >= total) return;
  const int plane = blockIdx.y;

  const int c = (int)(chunk % chunks_per_row);
  const int64_t row = chunk / chunks_per_row;
  const int h = (int)(row % num_kv_heads);
  const int64_t t = row / num_kv_heads;

  int i;
  int64_t p;
  if (cu_seqlens == nullptr) {
    i = (int)t;
    p = context_lens[i];
  } else {
    if (t >= (int64_t)cu_seqlens[num_seqs]) return;  // tokens past the packed batch
    i = seq_of_token(cu_seqlens, num_seqs, t);
    p = (int64_t)context_lens[i] + (t - cu_seqlens[i]);
  }
  if (p < 0) return;
  int64_t col = p / block_size;
  if (col > max_blocks - 1) col = max_blocks - 1;  // attention.py:144 / :235 clamp
  const int64_t blk = block_table[(int64_t)i * bt_row_stride + col];
  if (blk < 0 || blk >= num_blocks) return;
  const int off = (int)(p % block_size);

  const u16* src = (plane == 0 ? k + t * k_tok_stride : v + t * v_tok_stride)
                   + (int64_t)h * head_dim + c * 8;
  u16* dst = cache + plane * plane_elems
             + ((blk * num_kv_heads + h) * block_size + off) * (int64_t)head_dim + c * 8;
  st16(dst, ld16(src));
}

}  // namespace ndl

extern "C" int ndl_kv_append(void* kv_cache, int64_t num_blocks, int num_kv_heads, int block_size,
                             int head_dim, int dtype,
                             const void* k, int64_t k_tok_stride,
                             const void* v, int64_t v_tok_stride,
                             const int32_t* block_table, int64_t bt_row_stride,
                             int max_blocks_per_seq,
                             const int32_t* cu_seqlens, const int32_t* context_lens,
                             int num_seqs, int64_t num_tokens, ndl_stream_t stream) {
  using namespace ndl;
  if (dtype != NDL_DTYPE_BF16 && dtype != NDL_DTYPE_F16) return NDL_ERR_UNSUPPORTED;
  if (head_dim <= 0 || head_dim % 8 != 0 || block_size <= 0) return NDL_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_seqs < 0 || num_kv_heads <= 0 || num_blocks <= 0 ||
      max_blocks_per_seq <= 0 || bt_row_stride < max_blocks_per_seq)
    return NDL_ERR_INVALID_ARG;
  if (num_tokens == 0) return NDL_OK;
  if (!kv_cache || !k || !v || !block_table || !context_lens || num_seqs == 0)
    return NDL_ERR_INVALID_ARG;
  if (cu_seqlens == nullptr && num_tokens != num_seqs) return NDL_ERR_INVALID_ARG;
  if (k_tok_stride < (int64_t)num_kv_heads * head_dim ||
      v_tok_stride < (int64_t)num_kv_heads * head_dim)
    return NDL_ERR_INVALID_ARG;
  // 16-byte vector access needs 16-byte aligned rows.
  if (((uintptr_t)kv_cache | (uintptr_t)k | (uintptr_t)v) & 15u) return NDL_ERR_INVALID_ARG;
  if ((k_tok_stride | v_tok_stride) & 7) return NDL_ERR_INVALID_ARG;

  const int64_t plane_elems = num_blocks * num_kv_heads * (int64_t)block_size * head_dim;
  const int64_t total = num_tokens * num_kv_heads * (head_dim / 8);
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 0x7fffffff) return NDL_ERR_INVALID_ARG;
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)blocks, 2), dim3(threads), 0,
                     (hipStream_t)stream, (u16*)kv_cache, plane_elems, num_blocks, num_kv_heads,
                     block_size, head_dim, (const u16*)k, k_tok_stride, (const u16*)v,
                     v_tok_stride, block_table, bt_row_stride, max_blocks_per_seq, cu_seqlens,
                     context_lens, num_seqs, num_tokens);
  return check_launch();
}
