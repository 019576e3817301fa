// Varlen causal prefill attention over the paged cache, gfx950 (CDNA4).
//
// Reference: needle/layers/attention.py:120-134 (_prefill_pytorch): per packed
// sequence, causal softmax(q K^T / sqrt(D)) V with the GQA group expanded.  The
// reference attends the fresh k/v; here K/V are read back through block_table
// after ndl_kv_append wrote them (attention.py:103 runs _write_kv first), which
// is the same data when context_lens == 0 and also covers a cached prefix.
//
// Design:
//   * One workgroup = 4 waves = 128 query rows of one (sequence, query head);
//     each wave owns 32 rows as two 16-column N-blocks of 16x16 MFMA tiles.
//   * K/V advance 32 tokens (two cache blocks) per step.  All 256 threads
//     fetch the step's K and V rows (whole 1 KiB row runs per load
//     instruction) into double-buffered LDS with a chunk swizzle; the next
//     step's global loads are in flight while the current step computes.
//   * S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (A = K rows from LDS, B = Q^T
//     held in registers).  Its accumulator layout is the B operand (P^T) of
//     O^T = V^T P^T on the same instruction with a 32-token contraction whose
//     k order interleaves the two blocks; V^T is assembled from LDS rows with
//     the head_dim permutation d = (D/16) * m + b, so no cross-lane traffic.
//   * fp32 online softmax (exp2, scale folded with log2 e); the causal mask is
//     applied only on tiles that reach past a wave's first query position.
//   * Query tiles are dispatched longest-first (the last tile of a sequence
//     has the most keys).
#include <type_traits>

#include "ndl_common.hpp"

namespace ndl {

constexpr int kPrefWaves = 4;
constexpr int kPrefRowsPerWave = 32;                          // two 16-row N-blocks
constexpr int kPrefBlockM = kPrefWaves * kPrefRowsPerWave;     // 128 query rows
constexpr int kPrefBlockN = 32;                               // keys per step (2 blocks)

struct PrefillArgs {
  u16* out;
  const u16* q;
  int64_t q_tok_stride;
  const u16* kplane;
  const u16* vplane;
  int64_t num_blocks;
  int num_kv_heads;
  const int32_t* block_table;
  int64_t bt_row_stride;
  int max_blocks;
  const int32_t* cu_seqlens;
  const int32_t* context_lens;
  int num_heads;
  int group;
  float scale_log2;
  int num_qtiles;
  int64_t num_tokens;
};

template <int D>
__device__ __forceinline__ int pref_swz(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}

template <int D>
__global__ __launch_bounds__(256) void varlen_prefill_kernel(PrefillArgs a) {
  constexpr int KS = D / 32;          // k-steps of the QK MFMA
  constexpr int DPL = D / 16;         // m-blocks of O^T (head_dim elements per lane per row)
  constexpr int CPR = D / 8;          // 16-byte chunks per row
  constexpr int NCH = 32 * CPR / 256; // chunks per thread per plane per step
  constexpr int NB = 2;               // N-blocks per wave

  __shared__ __attribute__((aligned(16))) u16 lk[2][32 * D];
  __shared__ __attribute__((aligned(16))) u16 lv[2][32 * D];

  const int head = blockIdx.x;
  const int qtile = a.num_qtiles - 1 - (int)blockIdx.y;  // longest tiles first
  const int seq = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane >> 4, c = lane & 15;

  // Rows past num_tokens are never touched, whatever cu_seqlens holds.
  const int64_t tok0 = a.cu_seqlens[seq];
  int64_t tok1 = a.cu_seqlens[seq + 1];
  if (tok1 > a.num_tokens) tok1 = a.num_tokens;
  if (tok0 < 0 || tok1 <= tok0) return;
  const int n = (int)(tok1 - tok0);
  const int row0 = qtile * kPrefBlockM;
  if (row0 >= n) return;
  const int ctx = a.context_lens[seq] < 0 ? 0 : a.context_lens[seq];
  const int kvh = head / a.group;
  const int kv_end = ctx + (row0 + kPrefBlockM < n ? row0 + kPrefBlockM : n);
  const int nsteps = (kv_end + kPrefBlockN - 1) / kPrefBlockN;

  const int wrow0 = row0 + wave * kPrefRowsPerWave;           // first row of this wave
  const int wlast = (wrow0 + kPrefRowsPerWave < n ? wrow0 + kPrefRowsPerWave : n) - 1;
  const bool wave_active = wrow0 < n;
  const int qpos_min = ctx + wrow0;                           // first query position
  const int qpos_max = ctx + wlast;                           // last query position

  // B operands of S^T = K Q^T: lane (j, c) supplies Q[row 16 nb + c][32 s + 8 j .. +8).
  bf16x8 qb[NB][KS];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int row = wrow0 + 16 * nb + c;
    const u16* qrow = a.q + (tok0 + row) * a.q_tok_stride + (int64_t)head * D + 8 * j;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      u32x4 w = row < n ? ld16(qrow + 32 * s) : u32x4{0u, 0u, 0u, 0u};
      qb[nb][s] = __builtin_bit_cast(bf16x8, w);
    }
  }

  const int64_t blk_stride = (int64_t)a.num_kv_heads * 16 * D;
  const int64_t head_off = (int64_t)kvh * 16 * D;
  const int32_t* bt_row = a.block_table + (int64_t)seq * a.bt_row_stride;

  auto block_id = [&](int col) -> int64_t {
    if (col > a.max_blocks - 1) col = a.max_blocks - 1;   // the append's column clamp
    return bt_row[col];
  };

  // Loader: chunk u of a step is row u / CPR (0..31), 16-byte chunk u % CPR.
  auto gload = [&](int step, u32x4 (&kr)[NCH], u32x4 (&vr)[NCH]) {
#pragma unroll
    for (int e = 0; e < NCH; ++e) {
      const int u = tid + 256 * e;
      const int r = u / CPR, ch = u % CPR;
      const int kp = step * kPrefBlockN + r;
      const int64_t blk = block_id(kp >> 4);
      if (kp < kv_end && blk >= 0 && blk < a.num_blocks) {
        const int64_t off = blk * blk_stride + head_off + (kp & 15) * D + 8 * ch;
        kr[e] = ldg16(a.kplane + off);
        vr[e] = ldg16(a.vplane + off);
      } else {  // past the range or an invalid id: zeros (masked below)
        kr[e] = u32x4{0u, 0u, 0u, 0u};
        vr[e] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  };
  auto sstore = [&](int buf, const u32x4 (&kr)[NCH], const u32x4 (&vr)[NCH]) {
#pragma unroll
    for (int e = 0; e < NCH; ++e) {
      const int u = tid + 256 * e;
      const int r = u / CPR, ch = u % CPR;
      const int o = r * D + 8 * (ch ^ pref_swz<D>(r));
      *reinterpret_cast<u32x4*>(&lk[buf][o]) = kr[e];
      *reinterpret_cast<u32x4*>(&lv[buf][o]) = vr[e];
    }
  };

  f32x4 acc[NB][DPL];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int b = 0; b < DPL; ++b) acc[nb][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[NB], lsum[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m[nb] = kNegInf;
    lsum[nb] = 0.f;
  }

  auto compute = [&](int step, int buf) {
    const int kv0 = step * kPrefBlockN;
    if (!wave_active || kv0 > qpos_max) return;  // every key of the step is in this wave's future
    const bool diag = kv0 + kPrefBlockN - 1 > qpos_min;
    // Keys of an invalid block are masked like future keys.
    const int64_t b0 = block_id(kv0 >> 4), b1 = block_id((kv0 >> 4) + 1);
    const bool bad0 = b0 < 0 || b0 >= a.num_blocks;
    const bool bad1 = b1 < 0 || b1 >= a.num_blocks;
    const bool masked = diag || bad0 || bad1;

    // S^T for the two blocks and both N-blocks.
    f32x4 st[2][NB];
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) st[blk][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const int r = 16 * blk + c;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(
            &lk[buf][r * D + 8 * ((j + 4 * s) ^ pref_swz<D>(r))]);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
          st[blk][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, ka), qb[nb][s], st[blk][nb], 0, 0, 0);
      }
    }

    // V rows of this lane: e = 4 blk + i -> key 16 blk + 4 j + i, head_dim DPL*c .. +DPL.
    using VT = typename std::conditional<D == 128, u32x4, u32x2>::type;
    VT vrow[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int r = 16 * (e >> 2) + 4 * j + (e & 3);
      if constexpr (D == 128) {
        vrow[e] = *reinterpret_cast<const u32x4*>(&lv[buf][r * D + 8 * (c ^ pref_swz<D>(r))]);
      } else {
        vrow[e] = *reinterpret_cast<const u32x2*>(
            &lv[buf][r * D + 8 * ((c >> 1) ^ pref_swz<D>(r)) + 4 * (c & 1)]);
      }
    }

    bf16x8 pb[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int qpos = ctx + wrow0 + 16 * nb + c;
      float sc[8];
      float mt = kNegInf;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int blk = e >> 2, i = e & 3;
        const int kp = kv0 + 16 * blk + 4 * j + i;
        bool ok = true;
        if (masked) ok = kp <= qpos && !(blk == 0 ? bad0 : bad1);
        sc[e] = ok ? st[blk][nb][i] * a.scale_log2 : kNegInf;
        mt = fmaxf(mt, sc[e]);
      }
      mt = fmaxf(mt, xor_shfl(mt, 16));
      mt = fmaxf(mt, xor_shfl(mt, 32));
      const float m_new = fmaxf(m[nb], mt);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      const float alpha = fast_exp2(m[nb] - m_use);
      float p[8];
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        p[e] = fast_exp2(sc[e] - m_use);
        ps += p[e];
      }
      lsum[nb] = lsum[nb] * alpha + ps;
      m[nb] = m_new;
#pragma unroll
      for (int b = 0; b < DPL; ++b) acc[nb][b] *= alpha;
      pb[nb] = __builtin_bit_cast(
          bf16x8, u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                        pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])});
    }

    // O^T += V^T P^T, one MFMA per (m-block, N-block).
#pragma unroll
    for (int b = 0; b < DPL; ++b) {
      uint32_t w[4];
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const uint32_t lo = vrow[2 * h][b >> 1], hi = vrow[2 * h + 1][b >> 1];
        w[h] = (b & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
      }
      const bf16x8 va = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[nb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[nb], acc[nb][b], 0, 0, 0);
    }
  };

  // Double-buffered main loop: global loads of step t+1 overlap the compute of step t.
  u32x4 kr[NCH], vr[NCH];
  gload(0, kr, vr);
  sstore(0, kr, vr);
  __syncthreads();
  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const bool more = step + 1 < nsteps;
    if (more) gload(step + 1, kr, vr);
    compute(step, buf);
    if (more) sstore(buf ^ 1, kr, vr);
    __syncthreads();
  }

  if (!wave_active) return;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    float l = lsum[nb];
    l += xor_shfl(l, 16);
    l += xor_shfl(l, 32);
    const int row = wrow0 + 16 * nb + c;
    if (row >= n) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    // acc[nb][b][i] holds O[row][d = DPL * (4 j + i) + b].
    u16* dst = a.out + ((tok0 + row) * a.num_heads + head) * (int64_t)D + DPL * 4 * j;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t w[DPL / 2];
#pragma unroll
      for (int b = 0; b < DPL; b += 2)
        w[b / 2] = pack_bf16x2(acc[nb][b][i] * inv, acc[nb][b + 1][i] * inv);
      if constexpr (DPL == 8)
        st16(dst + DPL * i, u32x4{w[0], w[1], w[2], w[3]});
      else
        *reinterpret_cast<u32x2*>(dst + DPL * i) = u32x2{w[0], w[1]};
    }
  }
}

}  // namespace ndl

extern "C" int ndl_varlen_prefill(void* out, const void* q, int64_t q_tok_stride,
                                  const void* kv_cache, int64_t num_blocks,
                                  const int32_t* block_table, int64_t bt_row_stride,
                                  int max_blocks_per_seq, const int32_t* cu_seqlens,
                                  const int32_t* context_lens, int num_seqs, int64_t num_tokens,
                                  int max_seqlen, int max_context_len, int num_heads,
                                  int num_kv_heads, int head_dim, int block_size, int dtype,
                                  float scale, ndl_stream_t stream) {
  using namespace ndl;
  if (dtype != NDL_DTYPE_BF16) return NDL_ERR_UNSUPPORTED;
  if (block_size != 16 || (head_dim != 64 && head_dim != 128)) return NDL_ERR_UNSUPPORTED;
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0)
    return NDL_ERR_INVALID_ARG;
  if (num_seqs < 0 || num_tokens < 0 || max_seqlen < 0 || max_context_len < 0 ||
      num_blocks <= 0 || max_blocks_per_seq <= 0 || bt_row_stride < max_blocks_per_seq ||
      q_tok_stride < (int64_t)num_heads * head_dim)
    return NDL_ERR_INVALID_ARG;
  if (num_seqs == 0 || num_tokens == 0 || max_seqlen == 0) return NDL_OK;
  if (!out || !q || !kv_cache || !block_table || !cu_seqlens || !context_lens)
    return NDL_ERR_INVALID_ARG;
  if (((uintptr_t)out | (uintptr_t)q | (uintptr_t)kv_cache) & 15u) return NDL_ERR_INVALID_ARG;
  if (q_tok_stride & 7) return NDL_ERR_INVALID_ARG;
  const int64_t qtiles = ((int64_t)max_seqlen + kPrefBlockM - 1) / kPrefBlockM;
  if (num_seqs > 65535 || qtiles > 65535) return NDL_ERR_UNSUPPORTED;
  (void)max_context_len;

  PrefillArgs a;
  a.out = (u16*)out;
  a.q = (const u16*)q;
  a.q_tok_stride = q_tok_stride;
  a.kplane = (const u16*)kv_cache;
  a.vplane = a.kplane + num_blocks * num_kv_heads * (int64_t)16 * head_dim;
  a.num_blocks = num_blocks;
  a.num_kv_heads = num_kv_heads;
  a.block_table = block_table;
  a.bt_row_stride = bt_row_stride;
  a.max_blocks = max_blocks_per_seq;
  a.cu_seqlens = cu_seqlens;
  a.context_lens = context_lens;
  a.num_heads = num_heads;
  a.group = num_heads / num_kv_heads;
  a.scale_log2 = scale * kLog2e;
  a.num_qtiles = (int)qtiles;
  a.num_tokens = num_tokens;

  const dim3 grid((unsigned)num_heads, (unsigned)qtiles, (unsigned)num_seqs);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(varlen_prefill_kernel<128>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(varlen_prefill_kernel<64>, grid, dim3(256), 0, s, a);
  return check_launch();
}
