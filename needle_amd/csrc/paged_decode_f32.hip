// Paged decode attention in float32 (the reference's --dtype float32), gfx950.
//
// Reference: needle/layers/attention.py:291-310 (_decode_pytorch) in a float32 model
// (needle/args.py:80-84, :143-153; runner.py:31-34, 75-78): per sequence gather K/V blocks,
// expand the GQA group, softmax(q K^T * scale) V, every op in fp32.
//
// One workgroup of kF32Waves waves per (kv head, sequence); wave w takes the sequence's
// 16-token tiles w, w + kF32Waves, ..; the waves combine their (m, l, acc) through LDS, as
// the 16-bit per-sequence split does.  The products run on v_mfma_f32_16x16x4_f32 (fp32
// operands, fp32 accumulation), the probabilities stay fp32:
//   * S^T = K q^T: M = the tile's 16 tokens, N = the g query heads (padded to 16),
//     K = head_dim in steps of 4.  Lane (i, kk) = (lane % 16, lane / 16) holds
//     K[token i][16 m + 4 kk + e] and q[head i][16 m + 4 kk + e] for m < D/16, e < 4 (one
//     16-byte load per m: 64 contiguous bytes of a row per four lanes); the k order inside
//     the contraction is immaterial as long as both operands use it.
//   * The S^T accumulator puts tokens 4 kk + r of head i in lane (i, kk), which is the B
//     operand (P^T) of O^T = V^T P^T with token 4 kk + t in k-step t: no lane exchange.  The
//     matching A operand is V[4 kk + t][64 g + 4 i + e] (a 16-byte load per (g, t): 256
//     contiguous bytes of a row per sixteen lanes), so O^T row i of group g, MFMA e is head
//     dim d = 64 g + 4 i + e, and lane (i, kk) ends with O[head i][64 g + 16 kk + 4 r + e].
//   * Online softmax in the exp2 domain (scale * log2 e folded), the row max and sum across
//     the four lanes of a head by two lane swaps; the accumulator is rescaled when a head's
//     max moves.
// The fused forms append the step's rows first with the append kernel (and rotate the new
// key there), then attend the pool; q is rotated as it is loaded.
#include "ndl_common.hpp"

namespace ndl {

constexpr int kF32Waves = 8;

struct DecodeF32Args {
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
  const int32_t* context_lens;
  int num_heads;
  int group;
  float scale_log2;
  const float* rope_cos;   // null: q is already rotated
  const float* rope_sin;
  int64_t rope_stride;
};

__device__ __forceinline__ f32x4 ldf4(const float* p) {
  return *reinterpret_cast<const f32x4*>(p);
}

template <int D, bool ROPE>
__global__ __launch_bounds__(64 * kF32Waves) void paged_decode_f32_kernel(DecodeF32Args a) {
  constexpr int NW = kF32Waves;
  constexpr int QK = D / 16;   // 16-byte pieces of a K row (and of q) per lane
  constexpr int G = D / 64;    // 64-wide head_dim groups of the PV product
  constexpr int E = D / 4;     // accumulator floats per lane
  constexpr int KPW = E / NW;  // accumulator floats per lane each wave finishes
  static_assert(D == 64 || D == 128, "head_dim");
  const int kvh = (int)(blockIdx.x % (unsigned)a.num_kv_heads);
  const int seq = (int)(blockIdx.x / (unsigned)a.num_kv_heads);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int i16 = lane & 15, kk = lane >> 4;
  const bool head_ok = i16 < a.group;
  const int head = kvh * a.group + i16;
  const int tshift = a.tile_shift, tmask = (1 << tshift) - 1;
  const int64_t blk_stride = (int64_t)a.num_kv_heads * (16 << tshift) * D;
  const int64_t head_off = (int64_t)kvh * (16 << tshift) * D;

  // attention.py:299: the step's token is attended; a table row holds W blocks at most
  int64_t L = (int64_t)a.context_lens[seq] + 1;
  const int64_t cap = (int64_t)a.max_blocks << (4 + tshift);
  if (L > cap) L = cap;
  const int nt = L <= 0 ? 0 : (int)((L + 15) >> 4);
  const int ntw = wv < nt ? (nt - wv + NW - 1) / NW : 0;   // this wave's tiles

  // q^T operand (lanes past the group read the group's first head and zero it)
  f32x4 qv[QK];
  {
    const float* qrow = a.q + (int64_t)seq * a.q_tok_stride +
                        (int64_t)(head_ok ? head : kvh * a.group) * D + 4 * kk;
#pragma unroll
    for (int m = 0; m < QK; ++m) qv[m] = ldf4(qrow + 16 * m);
    if constexpr (ROPE) {
      // element 16 m + 4 kk + e pairs with the same lane's piece m + QK / 2
      const float* crow = a.rope_cos + (int64_t)seq * a.rope_stride + 4 * kk;
      const float* srow = a.rope_sin + (int64_t)seq * a.rope_stride + 4 * kk;
#pragma unroll
      for (int m = 0; m < QK / 2; ++m) {
        u32x4 lo, hi;
        rope4_f32(__builtin_bit_cast(u32x4, qv[m]), __builtin_bit_cast(u32x4, qv[m + QK / 2]),
                  __builtin_bit_cast(u32x4, ldf4(crow + 16 * m)),
                  __builtin_bit_cast(u32x4, ldf4(crow + 16 * (m + QK / 2))),
                  __builtin_bit_cast(u32x4, ldf4(srow + 16 * m)),
                  __builtin_bit_cast(u32x4, ldf4(srow + 16 * (m + QK / 2))), lo, hi);
        qv[m] = __builtin_bit_cast(f32x4, lo);
        qv[m + QK / 2] = __builtin_bit_cast(f32x4, hi);
      }
    }
#pragma unroll
    for (int m = 0; m < QK; ++m) qv[m] = head_ok ? qv[m] : f32x4{0.f, 0.f, 0.f, 0.f};
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

  // The wave's tiles go in windows of 64 (lane l: the block id of the window's tile l).
  for (int w0 = 0; w0 < ntw; w0 += 64) {
    const int cnt = ntw - w0 < 64 ? ntw - w0 : 64;
    const int tl = wv + NW * (w0 + (lane < cnt ? lane : cnt - 1));   // the lane's tile
    const int bt_lane = bt_row[tl >> tshift];
    asm volatile("" ::"v"(bt_lane));   // the ids are waited for once per window

    // live = false: a placeholder of the same instructions (every lane reads the tile's
    // first 16 bytes), issued past the window's end so that every compute has the same
    // loads in flight behind it.
    auto load_tile = [&](int it, Tile& t, bool live) {
      const int itc = it < cnt ? it : cnt - 1;
      int64_t blk = __builtin_amdgcn_readlane(bt_lane, itc);
      t.bad = blk < 0 || blk >= a.num_blocks;
      if (t.bad) blk = 0;
      const int tix = wv + NW * (w0 + itc);
      const int64_t off = blk * blk_stride + head_off + (int64_t)(tix & tmask) * 16 * D;
      const float* kb = a.kplane + off + (live ? (int64_t)i16 * D + 4 * kk : 0);
      const float* vb = a.vplane + off + (live ? (int64_t)4 * kk * D + 4 * i16 : 0);
#pragma unroll
      for (int m = 0; m < QK; ++m) t.k[m] = ldf4(kb + (live ? 16 * m : 0));
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) t.v[g][t4] = ldf4(vb + (live ? t4 * D + 64 * g : 0));
    };
    auto compute = [&](int it, Tile& t) {
      const int tix = wv + NW * (w0 + it);
      f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < QK; ++m)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          st = __builtin_amdgcn_mfma_f32_16x16x4f32(t.k[m][e], qv[m][e], st, 0, 0, 0);
      // st[r]: token tix * 16 + 4 kk + r, head i16
      const int64_t pos0 = (int64_t)tix * 16 + 4 * kk;
      float sc[4];
      float mt = kNegInf;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = !t.bad && pos0 + r < L;
        sc[r] = ok ? st[r] * a.scale_log2 : kNegInf;
        mt = fmaxf(mt, sc[r]);
        // rows past the range may hold any bits (NaN * 0 = NaN): cleared
        if (!ok) {
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
    // A two-deep ring: one load per trip (placeholders past the window), compute behind it.
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

  // Combine over the waves (one barrier): wave w's m, l and accumulators into LDS, then
  // wave w sums elements w * KPW .. of every lane over the waves in a fixed order, each
  // term scaled by 2^(m_w - M) (products rounded before the sum).  Lane element
  // x = (4 g + r) * 4 + e holds O[head i16][64 g + 16 kk + 4 r + e].
  __shared__ __attribute__((aligned(16))) float sacc[NW * E * 64];
  __shared__ float sm[NW * 16], sl[NW * 16];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) sacc[(wv * E + (4 * g + r) * 4 + e) * 64 + lane] = acc[g][e][r];
  if (kk == 0) {
    sm[wv * 16 + i16] = m_run;
    sl[wv * 16 + i16] = l_run;
  }
  __syncthreads();
  if (!head_ok) return;
  float mw[NW];
  float mx = kNegInf;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    mw[w] = sm[w * 16 + i16];
    mx = fmaxf(mx, mw[w]);
  }
  float den = 0.f, o[KPW];
#pragma unroll
  for (int x = 0; x < KPW; ++x) o[x] = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float wt = mw[w] == kNegInf ? 0.f : fast_exp2(mw[w] - mx);
    den += __fmul_rn(sl[w * 16 + i16], wt);
#pragma unroll
    for (int x = 0; x < KPW; ++x) o[x] += __fmul_rn(sacc[(w * E + wv * KPW + x) * 64 + lane], wt);
  }
  const float inv = den > 0.f ? 1.f / den : 0.f;
  // elements wv * KPW .. + KPW: consecutive e of one (g, r)
  const int x0 = wv * KPW;
  const int g = x0 / 16, r = (x0 / 4) % 4, e0 = x0 % 4;
  float* const dst = a.out + ((int64_t)seq * a.num_heads + head) * D + 64 * g + 16 * kk + 4 * r + e0;
  if constexpr (KPW == 4) {
    *reinterpret_cast<f32x4*>(dst) = f32x4{o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv};
  } else {
    static_assert(KPW == 2, "elements per wave");
    *reinterpret_cast<f32x2*>(dst) = f32x2{o[0] * inv, o[1] * inv};
  }
}

int launch_decode_f32(void* out, const void* q, int64_t q_tok_stride, const void* k_new,
                      int64_t k_tok_stride, const void* v_new, int64_t v_tok_stride,
                      const void* cos, const void* sin, int64_t cs_tok_stride, void* kv_cache,
                      int64_t num_blocks, const int32_t* block_table, int64_t bt_row_stride,
                      int max_blocks_per_seq, const int32_t* context_lens, int num_seqs,
                      int num_heads, int num_kv_heads, int head_dim, int block_size, float scale,
                      ndl_stream_t stream) {
  if ((q_tok_stride & 3) || (cos != nullptr && (cs_tok_stride & 3))) return NDL_ERR_INVALID_ARG;
  if ((int64_t)num_seqs * num_kv_heads > 0x7fffffff) return NDL_ERR_UNSUPPORTED;
  if (k_new != nullptr) {   // the step's rows (k rotated with cos/sin) into the pool first
    const int rc = launch_kv_append(kv_cache, num_blocks, num_kv_heads, block_size, head_dim,
                                    k_new, k_tok_stride, v_new, v_tok_stride, block_table,
                                    bt_row_stride, max_blocks_per_seq, nullptr, context_lens,
                                    num_seqs, num_seqs, cos, sin, cs_tok_stride, kFmtF32, stream);
    if (rc != NDL_OK) return rc;
  }
  DecodeF32Args a;
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
  a.context_lens = context_lens;
  a.num_heads = num_heads;
  a.group = num_heads / num_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.rope_cos = (const float*)cos;
  a.rope_sin = (const float*)sin;
  a.rope_stride = cs_tok_stride;
  const bool rope = cos != nullptr;
  const void* fn = head_dim == 128
      ? (rope ? (const void*)paged_decode_f32_kernel<128, true>
              : (const void*)paged_decode_f32_kernel<128, false>)
      : (rope ? (const void*)paged_decode_f32_kernel<64, true>
              : (const void*)paged_decode_f32_kernel<64, false>);
  void* args[] = {&a};
  if (hipLaunchKernel(fn, dim3((unsigned)(num_seqs * num_kv_heads)), dim3(64 * kF32Waves), args,
                      0, (hipStream_t)stream) != hipSuccess) {
    (void)hipGetLastError();
    return NDL_ERR_LAUNCH;
  }
  return check_launch();
}

}  // namespace ndl
