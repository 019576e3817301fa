// Fused rotary embedding + KV append.
//
// Reference: needle/layers/attention.py:88 with _apply_rope / _rotate_half
// (:277-288), followed by the decode append (:141-154) or _write_kv (:204-246).
// The reference runs ~8 elementwise kernels for RoPE on q and k, then the
// scatter; here one launch rotates q (written to q_out), rotates k and copies v
// straight into their cache slots.
//
// Rounding is the reference's, op for op, in the model dtype r (bf16, fp16 or fp32):
//   out[d] = r( r(x[d] * cos[d]) + r(rot(x)[d] * sin[d]) )
// with rot(x)[d] = -x[d + D/2] (d < D/2) or x[d - D/2] (d >= D/2); every
// product and the sum are formed in fp32 and rounded to the format, nearest even,
// exactly as torch does for bf16, fp16 and fp32 tensors.  The result is bit-identical to
// the reference's.  Sizes and offsets count 16-bit units (a float32 row of D elements is
// 2D units, its 16-byte chunks 4 elements; the entry point converts).
#include "ndl_common.hpp"

namespace ndl {

__device__ __forceinline__ int seq_of_token_rope(const int32_t* __restrict__ cu, int n,
                                                 int64_t t) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((int64_t)cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

struct RopeArgs {
  u16* q_out;
  const u16* q;
  int64_t q_tok_stride;
  const u16* k;
  int64_t k_tok_stride;
  const u16* v;
  int64_t v_tok_stride;
  const u16* cos;
  const u16* sin;
  int64_t cs_tok_stride;
  u16* cache;
  int64_t plane_elems;
  int64_t num_blocks;
  int num_heads;
  int num_kv_heads;
  int block_size;
  int head_dim;
  const int32_t* block_table;
  int64_t bt_row_stride;
  int max_blocks;
  const int32_t* cu_seqlens;
  const int32_t* context_lens;
  int num_seqs;
  int64_t num_tokens;
};

// Element offset in a plane of (token t, kv head 0)'s slot by the append's rule
// (attention.py:143-146, :224-237), or -1 when the slot is out of range.  t is
// wave-uniform, so these loads go through the scalar cache.
__device__ __forceinline__ int64_t kv_slot_row(const RopeArgs& a, int64_t t) {
  int i;
  int64_t p;
  if (a.cu_seqlens == nullptr) {
    i = (int)t;
    p = a.context_lens[i];
  } else {
    if (t >= (int64_t)a.cu_seqlens[a.num_seqs]) return -1;
    i = seq_of_token_rope(a.cu_seqlens, a.num_seqs, t);
    p = (int64_t)a.context_lens[i] + (t - a.cu_seqlens[i]);
  }
  if (p < 0) return -1;
  int64_t col = p / a.block_size;
  if (col > a.max_blocks - 1) col = a.max_blocks - 1;
  const int64_t blk = a.block_table[(int64_t)i * a.bt_row_stride + col];
  if (blk < 0 || blk >= a.num_blocks) return -1;
  return (blk * a.num_kv_heads * a.block_size + p % a.block_size) * (int64_t)a.head_dim;
}

// One wave per (token, round of 64 items).  A token's items are its (row, 8-element
// chunk of the first half) pairs: first the 2 * Hkv k and v rows (k rotated into the K
// plane, v copied into the V plane), then the H q rows (rotated into q_out).  Every wave
// runs one straight-line round: its loads go out first, then (k/v rounds) the slot
// lookup, which comes before any store of the kernel and so reads through the scalar
// cache.  Lanes past the last item load a valid item again and store nothing, so no
// divergent branch separates the loads.  (A lane chooses between two row bases at most:
// a three-way choice of pointers compiles to a lookup table in scratch memory.)
template <int FMT>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(RopeArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t w =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int D = a.head_dim, half = D >> 1, cph = half >> 3;  // chunks per half row
  const int H = a.num_heads, Hkv = a.num_kv_heads, bs = a.block_size;
  const int kv_items = 2 * Hkv * cph, q_items = H * cph;
  const int kv_rounds = (kv_items + 63) >> 6, rounds = kv_rounds + ((q_items + 63) >> 6);
  const int64_t t = w / rounds;
  const int r = (int)(w - t * rounds);
  if (t >= a.num_tokens) return;  // wave-uniform
  const u16* const cs = a.cos + t * a.cs_tok_stride;
  const u16* const sn = a.sin + t * a.cs_tok_stride;

  if (r < kv_rounds) {  // k / v rows
    const int item0 = 64 * r + lane;
    const bool live = item0 < kv_items;
    const int item = live ? item0 : kv_items - 1;
    const int row = item / cph, c = item - row * cph, d0 = 8 * c;
    const bool is_v = row >= Hkv;
    const int h = is_v ? row - Hkv : row;
    const u16* src = (is_v ? a.v + t * a.v_tok_stride : a.k + t * a.k_tok_stride) +
                     (int64_t)h * D;
    const u32x4 lo = ld16(src + d0), hi = ld16(src + d0 + half);
    const u32x4 clo = ld16(cs + d0), chi = ld16(cs + d0 + half);
    const u32x4 slo = ld16(sn + d0), shi = ld16(sn + d0 + half);
    const int64_t krow = kv_slot_row(a, t);
    u32x4 olo, ohi;
    rope16<FMT>(lo, hi, clo, chi, slo, shi, olo, ohi);
    if (is_v) {
      olo = lo;
      ohi = hi;
    }
    if (live && krow >= 0) {
      u16* const dst = a.cache + (is_v ? a.plane_elems : 0) + krow + (int64_t)h * bs * D;
      st16(dst + d0, olo);
      st16(dst + d0 + half, ohi);
    }
  } else {  // q rows
    const int item0 = 64 * (r - kv_rounds) + lane;
    const bool live = item0 < q_items;
    const int item = live ? item0 : q_items - 1;
    const int row = item / cph, c = item - row * cph, d0 = 8 * c;
    const u16* src = a.q + t * a.q_tok_stride + (int64_t)row * D;
    const u32x4 lo = ld16(src + d0), hi = ld16(src + d0 + half);
    const u32x4 clo = ld16(cs + d0), chi = ld16(cs + d0 + half);
    const u32x4 slo = ld16(sn + d0), shi = ld16(sn + d0 + half);
    u32x4 olo, ohi;
    rope16<FMT>(lo, hi, clo, chi, slo, shi, olo, ohi);
    if (live) {
      u16* const dst = a.q_out + (t * H + row) * (int64_t)D;
      st16(dst + d0, olo);
      st16(dst + d0 + half, ohi);
    }
  }
}

}  // namespace ndl

extern "C" int ndl_rope_kv_append(void* q_out, const void* q, int64_t q_tok_stride,
                                  const void* k, int64_t k_tok_stride, const void* v,
                                  int64_t v_tok_stride, const void* cos, const void* sin,
                                  int64_t cs_tok_stride, void* kv_cache, int64_t num_blocks,
                                  int num_heads, int num_kv_heads, int block_size, int head_dim,
                                  int dtype, const int32_t* block_table, int64_t bt_row_stride,
                                  int max_blocks_per_seq, const int32_t* cu_seqlens,
                                  const int32_t* context_lens, int num_seqs, int64_t num_tokens,
                                  ndl_stream_t stream) {
  using namespace ndl;
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  // halves of whole 16-byte chunks: a multiple of 16 16-bit elements or of 8 float32 ones
  if (head_dim <= 0 || head_dim % (dtype_is_f32(dtype) ? 8 : 16) != 0 || block_size <= 0)
    return NDL_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_seqs < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_blocks <= 0 ||
      max_blocks_per_seq <= 0 || bt_row_stride < max_blocks_per_seq)
    return NDL_ERR_INVALID_ARG;
  if (num_tokens == 0) return NDL_OK;
  if ((q_out == nullptr) != (q == nullptr)) return NDL_ERR_INVALID_ARG;  // both or neither
  if (!k || !v || !cos || !sin || !kv_cache || !block_table || !context_lens || num_seqs == 0)
    return NDL_ERR_INVALID_ARG;
  if (cu_seqlens == nullptr && num_tokens != num_seqs) return NDL_ERR_INVALID_ARG;
  if ((q != nullptr && q_tok_stride < (int64_t)num_heads * head_dim) ||
      k_tok_stride < (int64_t)num_kv_heads * head_dim ||
      v_tok_stride < (int64_t)num_kv_heads * head_dim || cs_tok_stride < head_dim)
    return NDL_ERR_INVALID_ARG;
  if (((uintptr_t)q_out | (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)cos |
       (uintptr_t)sin | (uintptr_t)kv_cache) & 15u)
    return NDL_ERR_INVALID_ARG;
  if ((q_tok_stride | k_tok_stride | v_tok_stride | cs_tok_stride) &
      (dtype_is_f32(dtype) ? 3 : 7))
    return NDL_ERR_INVALID_ARG;

  const int fmt = dtype_is_f32(dtype) ? kFmtF32 : dtype_is_f16(dtype) ? kFmtF16 : kFmtBF16;
  if (q == nullptr)  // k rotated and k, v appended: the append kernel with the rotation
    return launch_kv_append(kv_cache, num_blocks, num_kv_heads, block_size, head_dim, k,
                            k_tok_stride, v, v_tok_stride, block_table, bt_row_stride,
                            max_blocks_per_seq, cu_seqlens, context_lens, num_seqs, num_tokens,
                            cos, sin, cs_tok_stride, fmt, stream);
  if (fmt == kFmtF32) {   // the kernel counts 16-bit units
    head_dim *= 2;
    q_tok_stride *= 2;
    k_tok_stride *= 2;
    v_tok_stride *= 2;
    cs_tok_stride *= 2;
  }
  RopeArgs a;
  a.q_out = (u16*)q_out;
  a.q = (const u16*)q;
  a.q_tok_stride = q_tok_stride;
  a.k = (const u16*)k;
  a.k_tok_stride = k_tok_stride;
  a.v = (const u16*)v;
  a.v_tok_stride = v_tok_stride;
  a.cos = (const u16*)cos;
  a.sin = (const u16*)sin;
  a.cs_tok_stride = cs_tok_stride;
  a.cache = (u16*)kv_cache;
  a.plane_elems = num_blocks * num_kv_heads * (int64_t)block_size * head_dim;
  a.num_blocks = num_blocks;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.block_size = block_size;
  a.head_dim = head_dim;
  a.block_table = block_table;
  a.bt_row_stride = bt_row_stride;
  a.max_blocks = max_blocks_per_seq;
  a.cu_seqlens = cu_seqlens;
  a.context_lens = context_lens;
  a.num_seqs = num_seqs;
  a.num_tokens = num_tokens;
  // one wave per (token, round of 64 items), 4 per workgroup
  const int64_t cph = head_dim / 16;
  const int64_t rounds = (2 * num_kv_heads * cph + 63) / 64 + (num_heads * cph + 63) / 64;
  const int64_t blocks = (num_tokens * rounds + 3) / 4;
  if (blocks > 0x7fffffff) return NDL_ERR_INVALID_ARG;
  if (fmt == kFmtF32)
    hipLaunchKernelGGL(rope_kv_append_kernel<kFmtF32>, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, a);
  else if (fmt == kFmtF16)
    hipLaunchKernelGGL(rope_kv_append_kernel<kFmtF16>, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(rope_kv_append_kernel<kFmtBF16>, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, a);
  return check_launch();
}
