// Varlen causal prefill attention over the paged cache in float32 (the reference's
// --dtype float32), gfx950.
//
// Reference: needle/layers/attention.py:120-134 (_prefill_pytorch) in a float32 model: per
// packed sequence, causal softmax(q K^T / sqrt(D)) V with the GQA group expanded, every op
// in fp32.  As ndl_varlen_prefill does for the 16-bit formats, K/V are read back through
// block_table after the append (attention.py:103), which also covers a cached prefix.
//
// One wave per (query head, 16 query rows); four waves per workgroup take consecutive row
// blocks of one head.  The tile math is the float32 decode's (paged_decode_f32.hip) with the
// N dimension holding the 16 query rows of one head instead of the heads of one token:
//   * S^T = K q^T on v_mfma_f32_16x16x4_f32: lane (i, kk) = (lane % 16, lane / 16) holds
//     K[key i][16 m + 4 kk + e] and q[row i][16 m + 4 kk + e];
//   * the accumulator holds keys 4 kk + r of row i in lane (i, kk), the B operand of
//     O^T = V^T P^T with V[4 kk + t][64 g + 4 i + e] as A, so lane (i, kk) ends with
//     O[row i][64 g + 16 kk + 4 r + e];
//   * online softmax in the exp2 domain, fp32 probabilities, row max and sum across the
//     four lanes of a row by two lane swaps.
// Causal masking per (key, row): key position <= ctx + row; keys past the block's range or
// in an invalid block are masked and their V rows cleared.  A tile past the table row reads
// the row's last tile, as the append's column clamp (attention.py:235) wrote it, and as
// the 16-bit kernel does.
#include "ndl_common.hpp"

namespace ndl {

constexpr int kPrefF32Waves = 4;
constexpr int kPrefF32Rows = 16 * kPrefF32Waves;   // query rows per workgroup

struct PrefillF32Args {
  float* out;
  const float* q;
  int64_t q_tok_stride;
  const float* kplane;
  const float* vplane;
  int64_t num_blocks;
  int num_kv_heads;
  const int32_t* block_table;
  int64_t bt_row_stride;
  int max_blocks;
  int tile_shift;   // log2(block_size / 16)
  const int32_t* cu_seqlens;
  const int32_t* context_lens;
  int64_t num_tokens;
  int num_heads;
  int group;
  float scale_log2;
  const float* rope_cos;   // null: q is already rotated
  const float* rope_sin;
  int64_t rope_stride;
};

__device__ __forceinline__ f32x4 ldf4p(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}

template <int D, bool ROPE>
__global__ __launch_bounds__(64 * kPrefF32Waves) void varlen_prefill_f32_kernel(PrefillF32Args a) {
  constexpr int QK = D / 16;
  constexpr int G = D / 64;
  static_assert(D == 64 || D == 128, "head_dim");
  const int head = blockIdx.x, seq = blockIdx.y;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int i16 = lane & 15, kk = lane >> 4;
  const int kvh = head / a.group;

  const int64_t tok0 = a.cu_seqlens[seq];
  int64_t tok1 = a.cu_seqlens[seq + 1];
  if (tok1 > a.num_tokens) tok1 = a.num_tokens;
  if (tok0 < 0 || tok1 <= tok0) return;
  const int n = (int)(tok1 - tok0);
  const int r0 = (int)blockIdx.z * kPrefF32Rows + 16 * wv;   // this wave's first row
  if (r0 >= n) return;   // no barriers in this kernel
  const int ctx0 = a.context_lens[seq];
  const int ctx = ctx0 < 0 ? 0 : ctx0;
  const int row = r0 + i16;                       // this lane's query row
  const bool row_ok = row < n;
  const int64_t qpos = (int64_t)ctx + row;        // its position in the sequence
  const int64_t kv_end = (int64_t)ctx + (r0 + 16 < n ? r0 + 16 : n);   // keys the wave reads
  const int ntk = (int)((kv_end + 15) >> 4);      // 16-key tiles
  const int tshift = a.tile_shift, tmask = (1 << tshift) - 1;
  const int64_t blk_stride = (int64_t)a.num_kv_heads * (16 << tshift) * D;
  const int64_t head_off = (int64_t)kvh * (16 << tshift) * D;

  // q^T operand of the lane's row (a row past the range reads the wave's first row)
  f32x4 qv[QK];
  {
    const int64_t t = tok0 + (row_ok ? row : r0);
    const float* qrow = a.q + t * a.q_tok_stride + (int64_t)head * D + 4 * kk;
#pragma unroll
    for (int m = 0; m < QK; ++m) qv[m] = ldf4p(qrow + 16 * m);
    if constexpr (ROPE) {
      const float* crow = a.rope_cos + t * a.rope_stride + 4 * kk;
      const float* srow = a.rope_sin + t * a.rope_stride + 4 * kk;
#pragma unroll
      for (int m = 0; m < QK / 2; ++m) {
        u32x4 lo, hi;
        rope4_f32(__builtin_bit_cast(u32x4, qv[m]), __builtin_bit_cast(u32x4, qv[m + QK / 2]),
                  __builtin_bit_cast(u32x4, ldf4p(crow + 16 * m)),
                  __builtin_bit_cast(u32x4, ldf4p(crow + 16 * (m + QK / 2))),
                  __builtin_bit_cast(u32x4, ldf4p(srow + 16 * m)),
                  __builtin_bit_cast(u32x4, ldf4p(srow + 16 * (m + QK / 2))), lo, hi);
        qv[m] = __builtin_bit_cast(f32x4, lo);
        qv[m + QK / 2] = __builtin_bit_cast(f32x4, hi);
      }
    }
  }

  struct Tile {
    f32x4 k[QK];
    f32x4 v[G][4];
    bool bad;
  };
  f32x4 acc[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[g][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf, l_run = 0.f;
  const int32_t* bt_row = a.block_table + (int64_t)seq * a.bt_row_stride;
  const int max_tiles = a.max_blocks << tshift;

  for (int w0 = 0; w0 < ntk; w0 += 64) {
    const int cnt = ntk - w0 < 64 ? ntk - w0 : 64;
    int tl = w0 + (lane < cnt ? lane : cnt - 1);
    if (tl > max_tiles - 1) tl = max_tiles - 1;   // the table row's clamp
    const int bt_lane = bt_row[tl >> tshift];
    asm volatile("" ::"v"(bt_lane));   // the ids are waited for once per window

    // live = false: a placeholder load (every lane reads the tile's first 16 bytes)
    auto load_tile = [&](int it, Tile& t, bool live) {
      const int itc = it < cnt ? it : cnt - 1;
      int64_t blk = __builtin_amdgcn_readlane(bt_lane, itc);
      int tix = w0 + itc;
      if (tix > max_tiles - 1) tix = max_tiles - 1;
      t.bad = blk < 0 || blk >= a.num_blocks;
      if (t.bad) blk = 0;
      const int64_t off = blk * blk_stride + head_off + (int64_t)(tix & tmask) * 16 * D;
      const float* kb = a.kplane + off + (live ? (int64_t)i16 * D + 4 * kk : 0);
      const float* vb = a.vplane + off + (live ? (int64_t)4 * kk * D + 4 * i16 : 0);
#pragma unroll
      for (int m = 0; m < QK; ++m) t.k[m] = ldf4p(kb + (live ? 16 * m : 0));
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) t.v[g][t4] = ldf4p(vb + (live ? t4 * D + 64 * g : 0));
    };
    auto compute = [&](int it, Tile& t) {
      const int64_t key0 = (int64_t)(w0 + it) * 16 + 4 * kk;
      f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < QK; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          st = __builtin_amdgcn_mfma_f32_16x16x4f32(t.k[m][e], qv[m][e], st, 0, 0, 0);
      // st[r]: key key0 + r for the lane's row
      float sc[4];
      float mt = kNegInf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t key = key0 + r;
        const bool in_range = !t.bad && key < kv_end;
        sc[r] = in_range && key <= qpos ? st[r] * a.scale_log2 : kNegInf;
        mt = fmaxf(mt, sc[r]);
        if (!in_range) {   // rows that may hold any bits (NaN * 0 = NaN): cleared
#pragma unroll
          for (int g = 0; g < G; ++g) t.v[g][r] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
      mt = max_xor32(max_xor16(mt));
      const float m_new = fmaxf(m_run, mt);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      float p[4];
      float ps = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = fast_exp2(sc[r] - m_use);
        ps += p[r];
      }
      l_run = l_run * alpha + ps;
      m_run = m_new;
      if (__ballot(alpha != 1.f)) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[g][e] *= alpha;
      }
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int t4 = 0; t4 < 4; ++t4)
            acc[g][e] = __builtin_amdgcn_mfma_f32_16x16x4f32(t.v[g][t4][e], p[t4], acc[g][e],
                                                             0, 0, 0);
    };
    Tile buf[2];
    load_tile(0, buf[0], true);
    for (int it = 0; it < cnt; it += 2) {
      load_tile(it + 1, buf[1], it + 1 < cnt);
      compute(it, buf[0]);
      load_tile(it + 2, buf[0], it + 2 < cnt);
      if (it + 1 < cnt) compute(it + 1, buf[1]);
    }
  }
  l_run = add_xor32(add_xor16(l_run));
  if (!row_ok) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  float* const dst = a.out + ((tok0 + row) * a.num_heads + head) * (int64_t)D + 16 * kk;
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<f32x4*>(dst + 64 * g + 4 * r) =
          f32x4{acc[g][0][r] * inv, acc[g][1][r] * inv, acc[g][2][r] * inv, acc[g][3][r] * inv};
}

int launch_prefill_f32(void* out, const void* q, int64_t q_tok_stride, const void* cos,
                       const void* sin, int64_t cs_tok_stride, const void* kv_cache,
                       int64_t num_blocks, const int32_t* block_table, int64_t bt_row_stride,
                       int max_blocks_per_seq, const int32_t* cu_seqlens,
                       const int32_t* context_lens, int num_seqs, int64_t num_tokens,
                       int max_seqlen, int max_context_len, int num_heads, int num_kv_heads,
                       int head_dim, int block_size, float scale, ndl_stream_t stream) {
  (void)max_context_len;
  if ((q_tok_stride & 3) || (cos != nullptr && (cs_tok_stride & 3))) return NDL_ERR_INVALID_ARG;
  const int64_t zb = ((int64_t)max_seqlen + kPrefF32Rows - 1) / kPrefF32Rows;
  if (num_seqs > 65535 || zb > 65535) return NDL_ERR_UNSUPPORTED;
  PrefillF32Args a;
  a.out = (float*)out;
  a.q = (const float*)q;
  a.q_tok_stride = q_tok_stride;
  a.kplane = (const float*)kv_cache;
  a.vplane = a.kplane + num_blocks * num_kv_heads * (int64_t)block_size * head_dim;
  a.num_blocks = num_blocks;
  a.num_kv_heads = num_kv_heads;
  a.block_table = block_table;
  a.bt_row_stride = bt_row_stride;
  a.max_blocks = max_blocks_per_seq;
  a.tile_shift = block_tile_shift(block_size);
  a.cu_seqlens = cu_seqlens;
  a.context_lens = context_lens;
  a.num_tokens = num_tokens;
  a.num_heads = num_heads;
  a.group = num_heads / num_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.rope_cos = (const float*)cos;
  a.rope_sin = (const float*)sin;
  a.rope_stride = cs_tok_stride;
  const bool rope = cos != nullptr;
  const void* fn = head_dim == 128
      ? (rope ? (const void*)varlen_prefill_f32_kernel<128, true>
              : (const void*)varlen_prefill_f32_kernel<128, false>)
      : (rope ? (const void*)varlen_prefill_f32_kernel<64, true>
              : (const void*)varlen_prefill_f32_kernel<64, false>);
  void* args[] = {&a};
  if (hipLaunchKernel(fn, dim3((unsigned)num_heads, (unsigned)num_seqs, (unsigned)zb),
                      dim3(64 * kPrefF32Waves), args, 0, (hipStream_t)stream) != hipSuccess) {
    (void)hipGetLastError();
    return NDL_ERR_LAUNCH;
  }
  return check_launch();
}

}  // namespace ndl
