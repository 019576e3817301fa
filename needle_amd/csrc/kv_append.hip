// Scatter-append of new K/V rows into the paged pool.
//
// Reference: needle/layers/attention.py:141-154 (decode append) and
// attention.py:204-246 (_write_kv).  The reference derives the slot of every
// token with host round trips (context_lens.cpu(), a Python loop of aranges,
// repeat_interleave) and then issues 2*num_kv_heads index_put_ launches.
// Here one launch moves both planes: a wave derives the slots of its tokens on the
// device and its lanes copy the tokens' rows in 16-byte chunks.
#include "ndl_common.hpp"

namespace ndl {

// Largest i in [0, n) with cu[i] <= t (cu is non-decreasing, cu[0] == 0).  Called with
// a wave-uniform t, so its loads go through the scalar cache (and their own counter):
// they proceed while the wave's vector loads are in flight.
__device__ __forceinline__ int seq_of_token(const int32_t* __restrict__ cu, int n, int64_t t) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((int64_t)cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Tokens per wave at most (all of a wave's loads are issued before its slot lookups and
// its stores).
constexpr int kAppendMaxTokensPerWave = 4;
// Packed batches of at most this many sequences find their tokens' sequences with one
// vector load of cu_seqlens (lane l: boundary l) and a ballot.
constexpr int kAppendSmallSeqs = 63;

// One wave per group of TPW consecutive tokens.  The lanes copy a token's
// num_kv_heads * head_dim / 8 16-byte chunks of both planes (one 1 KiB instruction per
// plane when num_kv_heads * head_dim = 512).  The slot of a token is wave-uniform.
//   SMALL (cu_seqlens given, num_seqs <= kAppendSmallSeqs): lane l loads cu_seqlens[l] and
//     context_lens[l] with two vector loads issued before the rows, so they return first
//     (vector loads complete in issue order); a token's sequence is the number of
//     boundaries at or below it, less one (a ballot: the largest i with cu[i] <= t, empty
//     sequences included), its context length a readlane; only the table entries are
//     scalar loads, one per token, all in flight together.
//   otherwise: sequence by binary search over cu_seqlens (scalar loads, their own counter,
//     in flight while the rows load), or the token itself without cu_seqlens (decode).
// TPW is a template argument so that every wave issues the same loads and the compiler's
// vector-memory waits count them exactly; the last wave reloads its last valid token's
// row for the tokens past the end and stores nothing for them.
// ROPE: k is rotated on the way (the rotary embedding of ndl_rope_kv_append, rope8, from
// the token's cos/sin rows).  A lane then moves a chunk pair (c, c + head_dim/16) of one
// row, the rotation's operands: items are the k rows' pairs, then the v rows' pairs (copied
// unrotated), the same count as the chunks of one plane without ROPE.  FMT: the rotation's
// element format (Fmt); the plain copy is format-free.  Sizes and offsets count 16-bit
// units (a float32 row of D elements is 2D units; the launcher converts).
template <int TPW, bool SMALL, bool ROPE, int FMT = kFmtBF16>
__global__ __launch_bounds__(256) void kv_append_kernel(
    u16* __restrict__ cache, int64_t plane_elems, int64_t num_blocks, int num_kv_heads,
    int block_size, int head_dim,
    const u16* __restrict__ k, int64_t k_tok_stride,
    const u16* __restrict__ v, int64_t v_tok_stride,
    const int32_t* __restrict__ block_table, int64_t bt_row_stride, int max_blocks,
    const int32_t* __restrict__ cu_seqlens, const int32_t* __restrict__ context_lens,
    int num_seqs, int64_t num_tokens, const u16* __restrict__ rope_cos,
    const u16* __restrict__ rope_sin, int64_t rope_stride) {
  const int lane = threadIdx.x & 63;
  const int64_t wave_id =
      (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int64_t t0 = wave_id * TPW;
  const int cpr = head_dim >> 3;         // chunks per (token, kv head) row
  const int cpt = num_kv_heads * cpr;    // chunks per token and plane

  // SMALL: lane l's boundary cu_seqlens[l] (l <= num_seqs) and context length.
  int cu_l = 0, ctx_l = 0;
  if constexpr (SMALL) {
    cu_l = cu_seqlens[lane <= num_seqs ? lane : num_seqs];
    ctx_l = context_lens[lane < num_seqs ? lane : num_seqs - 1];
  }

  // Destination row (element offset in a plane) of each token, or -1 when it is skipped.
  int64_t dst_row[TPW];
  auto lookup = [&]() {
    int64_t packed;
    if constexpr (SMALL)
      packed = __builtin_amdgcn_readlane(cu_l, num_seqs);
    else
      packed = cu_seqlens == nullptr ? num_tokens : (int64_t)cu_seqlens[num_seqs];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      dst_row[u] = -1;
      const int64_t t = t0 + u;
      if (t >= num_tokens || t >= packed) continue;
      int i;
      int64_t p;
      if constexpr (SMALL) {
        const uint64_t m = __builtin_amdgcn_ballot_w64(lane <= num_seqs && (int64_t)cu_l <= t);
        i = __builtin_popcountll(m) - 1;
        if (i < 0 || i >= num_seqs) continue;   // only for a malformed cu_seqlens
        p = (int64_t)__builtin_amdgcn_readlane(ctx_l, i) +
            (t - __builtin_amdgcn_readlane(cu_l, i));
      } else if (cu_seqlens == nullptr) {
        i = (int)t;
        p = context_lens[i];
      } else {
        i = seq_of_token(cu_seqlens, num_seqs, t);
        p = (int64_t)context_lens[i] + (t - cu_seqlens[i]);
      }
      if (p < 0) continue;
      int64_t col = p / block_size;
      if (col > max_blocks - 1) col = max_blocks - 1;  // attention.py:144 / :235 clamp
      const int64_t blk = block_table[(int64_t)i * bt_row_stride + col];
      if (blk < 0 || blk >= num_blocks) continue;
      dst_row[u] = (blk * num_kv_heads * block_size + p % block_size) * (int64_t)head_dim;
    }
  };
  // Chunks r*64 .. r*64 + 63 of every token of the wave: all loads, then (round 0) the
  // slot lookups while the loads are in flight (the source rows depend only on the
  // token), then the stores.  Lanes past the row's chunks load its last chunk again (no
  // divergent branch around the loads, so they go out back to back) and store nothing.
  const int64_t t_last = num_tokens - 1;
  auto round = [&](const int r, const bool first) {
    const int cc0 = r * 64 + lane;
    const bool live = cc0 < cpt;
    const int cc = live ? cc0 : cpt - 1;
    const int h = cc / cpr, c = cc - h * cpr;
    const int64_t in_off = (int64_t)h * head_dim + c * 8;
    u32x4 kr[TPW], vr[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int64_t t = t0 + u < num_tokens ? t0 + u : t_last;
      kr[u] = ld16(k + t * k_tok_stride + in_off);
      vr[u] = ld16(v + t * v_tok_stride + in_off);
    }
    if (first) lookup();
    const int64_t out_off = ((int64_t)h * block_size) * head_dim + c * 8;
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      if (live && dst_row[u] >= 0) {
        st16(cache + dst_row[u] + out_off, kr[u]);
        st16(cache + plane_elems + dst_row[u] + out_off, vr[u]);
      }
    }
  };
  // ROPE rounds: item cc < cpt/2 is pair c of k row h, the rest the same pairs of v.
  const int half = cpr >> 1, pairs = cpt >> 1;
  auto rope_round = [&](const int r, const bool first) {
    const int cc0 = r * 64 + lane;
    const bool live = cc0 < cpt;
    const int cc = live ? cc0 : cpt - 1;
    const bool is_v = cc >= pairs;
    const int pi = is_v ? cc - pairs : cc;
    const int h = pi / half, c = pi - h * half;
    const u16* const src = is_v ? v : k;
    const int64_t src_stride = is_v ? v_tok_stride : k_tok_stride;
    const int64_t in_off = (int64_t)h * head_dim + c * 8;
    u32x4 xl[TPW], xh[TPW], cl[TPW], ch[TPW], sl[TPW], sh[TPW];
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int64_t t = t0 + u < num_tokens ? t0 + u : t_last;
      const u16* const x = src + t * src_stride + in_off;
      const u16* const cs = rope_cos + t * rope_stride + c * 8;
      const u16* const sn = rope_sin + t * rope_stride + c * 8;
      xl[u] = ld16(x);
      xh[u] = ld16(x + half * 8);
      cl[u] = ld16(cs);
      ch[u] = ld16(cs + half * 8);
      sl[u] = ld16(sn);
      sh[u] = ld16(sn + half * 8);
    }
    if (first) lookup();
    u16* const plane = cache + (is_v ? plane_elems : 0);
    const int64_t out_off = ((int64_t)h * block_size) * head_dim + c * 8;
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      u32x4 ol = xl[u], oh = xh[u];
      if (!is_v) rope16<FMT>(xl[u], xh[u], cl[u], ch[u], sl[u], sh[u], ol, oh);
      if (live && dst_row[u] >= 0) {
        st16(plane + dst_row[u] + out_off, ol);
        st16(plane + dst_row[u] + out_off + half * 8, oh);
      }
    }
  };
  if constexpr (ROPE) {
    rope_round(0, true);
    for (int r = 1; r < (cpt + 63) / 64; ++r) rope_round(r, false);
  } else {
    round(0, true);  // outside the loop: straight-line code, no waits between its loads
    for (int r = 1; r < (cpt + 63) / 64; ++r) round(r, false);
  }
}

// Shared by ndl_kv_append and the k-only form of ndl_rope_kv_append (rope_cos != nullptr:
// k rotated in format fmt; head_dim a multiple of 16).  head_dim and the strides count
// elements of format fmt.  Arguments are checked by the callers.
int launch_kv_append(void* kv_cache, int64_t num_blocks, int num_kv_heads, int block_size,
                     int head_dim, const void* k, int64_t k_tok_stride, const void* v,
                     int64_t v_tok_stride, const int32_t* block_table, int64_t bt_row_stride,
                     int max_blocks_per_seq, const int32_t* cu_seqlens,
                     const int32_t* context_lens, int num_seqs, int64_t num_tokens,
                     const void* rope_cos, const void* rope_sin, int64_t rope_stride,
                     int fmt, ndl_stream_t stream) {
  if (fmt == kFmtF32) {   // the kernel counts 16-bit units
    head_dim *= 2;
    k_tok_stride *= 2;
    v_tok_stride *= 2;
    rope_stride *= 2;
  }
  const int64_t plane_elems = num_blocks * num_kv_heads * (int64_t)block_size * head_dim;
  const bool small = cu_seqlens != nullptr && num_seqs <= kAppendSmallSeqs;
  const bool rope = rope_cos != nullptr;
  // As few tokens per wave as keep every wave resident at once (a second, partial round
  // of waves costs more than longer waves: 17,705 tokens of 4 x 128 went 13.3 us at 1
  // or 2 tokens per wave, 12.9 us at 3, 14.1 us at 4 on MI355X).
  int64_t resident = resident_workgroups((const void*)kv_append_kernel<1, false, false>, 256) * 4;
  if (resident <= 0) resident = 8192;
  int64_t tpw64 = (num_tokens + resident - 1) / resident;
  const int tpw = (int)(tpw64 < 1 ? 1 : tpw64 > kAppendMaxTokensPerWave ? kAppendMaxTokensPerWave
                                                                        : tpw64);
  const int64_t waves = (num_tokens + tpw - 1) / tpw;
  const int64_t blocks = (waves + 3) / 4;
  if (blocks > 0x7fffffff) return NDL_ERR_INVALID_ARG;
#define NDL_APPEND_FNS(S, R, F)                                                           \
  {(const void*)kv_append_kernel<1, S, R, F>, (const void*)kv_append_kernel<2, S, R, F>,  \
   (const void*)kv_append_kernel<3, S, R, F>, (const void*)kv_append_kernel<4, S, R, F>}
  // [copy, rotate bf16, rotate fp16, rotate fp32][small][tokens per wave - 1]
  const void* fns[4][2][kAppendMaxTokensPerWave] = {
      {NDL_APPEND_FNS(false, false, kFmtBF16), NDL_APPEND_FNS(true, false, kFmtBF16)},
      {NDL_APPEND_FNS(false, true, kFmtBF16), NDL_APPEND_FNS(true, true, kFmtBF16)},
      {NDL_APPEND_FNS(false, true, kFmtF16), NDL_APPEND_FNS(true, true, kFmtF16)},
      {NDL_APPEND_FNS(false, true, kFmtF32), NDL_APPEND_FNS(true, true, kFmtF32)}};
#undef NDL_APPEND_FNS
  u16* cache = (u16*)kv_cache;
  const u16* kp = (const u16*)k;
  const u16* vp = (const u16*)v;
  const u16* cp = (const u16*)rope_cos;
  const u16* sp = (const u16*)rope_sin;
  void* args[] = {&cache, (void*)&plane_elems, &num_blocks, &num_kv_heads, &block_size,
                  &head_dim, &kp, &k_tok_stride, &vp, &v_tok_stride, &block_table,
                  &bt_row_stride, &max_blocks_per_seq, &cu_seqlens, &context_lens, &num_seqs,
                  &num_tokens, &cp, &sp, &rope_stride};
  if (hipLaunchKernel(fns[rope ? 1 + fmt : 0][small ? 1 : 0][tpw - 1],
                      dim3((unsigned)blocks),
                      dim3(256), args, 0, (hipStream_t)stream) != hipSuccess) {
    (void)hipGetLastError();  // clear the error so that the next call's check sees its own
    return NDL_ERR_LAUNCH;
  }
  return check_launch();
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
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  // 16-byte rows: a multiple of 8 16-bit elements or of 4 float32 ones
  if (head_dim <= 0 || head_dim % (dtype_is_f32(dtype) ? 4 : 8) != 0 || block_size <= 0)
    return NDL_ERR_UNSUPPORTED;
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
  if ((k_tok_stride | v_tok_stride) & (dtype_is_f32(dtype) ? 3 : 7)) return NDL_ERR_INVALID_ARG;

  return launch_kv_append(kv_cache, num_blocks, num_kv_heads, block_size, head_dim, k,
                          k_tok_stride, v, v_tok_stride, block_table, bt_row_stride,
                          max_blocks_per_seq, cu_seqlens, context_lens, num_seqs, num_tokens,
                          nullptr, nullptr, 0, dtype_is_f32(dtype) ? kFmtF32 : kFmtBF16,
                          stream);
}
