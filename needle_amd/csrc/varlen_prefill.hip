// Varlen causal prefill attention over the paged cache, gfx950 (CDNA4).
//
// Reference: needle/layers/attention.py:120-134 (_prefill_pytorch): per packed
// sequence, causal softmax(q K^T / sqrt(D)) V with the GQA group expanded.  The
// reference attends the fresh k/v; here K/V are read back through block_table
// after ndl_kv_append wrote them (attention.py:103 runs _write_kv first), which
// is the same data when context_lens == 0 and also covers a cached prefix.
//
// Design:
//   * One workgroup = 8 waves = 128 query rows of one (sequence, query head);
//     each wave owns 16 rows as the N columns of 16x16 MFMA tiles (other
//     shapes are built for tuning: 4 waves x 16 or x 32 rows).
//   * K/V advance 32 tokens (two cache blocks) per step through a 4-stage LDS
//     ring filled by direct global->LDS loads (global_load_lds_dwordx4, no
//     register staging): each instruction reads whole rows, 1 KiB contiguous,
//     and lands them swizzled; three steps are in flight while one computes.
//   * S^T = K Q^T with v_mfma_f32_16x16x32_bf16 (A = K rows from LDS, B = Q^T
//     held in registers).  Its accumulator layout is the B operand (P^T) of
//     O^T = V^T P^T on the same instruction with a 32-token contraction whose
//     k order interleaves the two blocks; V^T is assembled from LDS rows with
//     the head_dim permutation d = (D/16) * m + b, so no cross-lane traffic.
//   * fp32 online softmax (exp2, scale folded with log2 e); the causal mask is
//     applied only on tiles that reach past a wave's first query position.
//   * Query tiles are dispatched longest-first (the last tile of a sequence
//     has the most keys).
#include <stdlib.h>

#include <type_traits>

#include "ndl_common.hpp"

namespace ndl {

constexpr int kPrefBlockN = 32;                               // keys per step (2 blocks)
constexpr int kPrefStages = 4;                                // LDS ring depth (steps)

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

// s_waitcnt vmcnt(N) with expcnt / lgkmcnt left unconstrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] at bits 15:14).
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier without the vmcnt(0) drain __syncthreads() implies: callers wait
// for exactly the loads they need first.  The memory clobber keeps the compiler from
// moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// One direct global->LDS load: lane L reads 16 bytes at gbase + lane_off (gbase
// wave-uniform) and they land at LDS byte lds_ptr + 16 * L.
// Issued from inline asm so the compiler does not order every later LDS read behind
// it (it cannot tell the ring's stages apart); the ring waits on vmcnt itself.
// M0 takes the LDS base; one wait state separates the M0 write from its use.  M0 is
// a reserved register, so clang ignores it in the clobber list: this is sound only
// while no other instruction in these kernels keeps a value in M0, which
// tests/test_isa_guards.py checks on the generated code.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void* gbase, uint32_t lane_off,
                                          const void* lds_ptr) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_ptr);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(base), "v"(lane_off), "s"(gbase)
               : "memory", "m0");
}
#pragma clang diagnostic pop

template <int D>
__device__ __forceinline__ int pref_swz(int r) {
  return D == 128 ? (r & 15) : ((r >> 1) & 7);
}

// NB 16-row N-blocks per wave, WAVES waves per workgroup: 16 * NB * WAVES query rows.
template <int D, int NB, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void varlen_prefill_kernel(PrefillArgs a) {
  constexpr int KS = D / 32;          // k-steps of the QK MFMA
  constexpr int DPL = D / 16;         // m-blocks of O^T (head_dim elements per lane per row)
  constexpr int CPR = D / 8;          // 16-byte chunks per row
  constexpr int kPrefRowsPerWave = 16 * NB;
  constexpr int kPrefBlockM = kPrefRowsPerWave * WAVES;
  constexpr int RPP = 512 / D;        // rows per 1 KiB piece (one direct load instruction)
  constexpr int PIECES = 32 / RPP;    // pieces per plane per step
  constexpr int IPW = 2 * PIECES / WAVES;  // direct load instructions per wave per step
  static_assert(IPW >= 1 && (2 * PIECES) % WAVES == 0, "load distribution");

  // Ring of kPrefStages steps; each stage holds 32 K rows and 32 V rows.
  __shared__ __attribute__((aligned(16))) u16 lk[kPrefStages][32 * D];
  __shared__ __attribute__((aligned(16))) u16 lv[kPrefStages][32 * D];

  const int head = blockIdx.x;
  const int qtile = a.num_qtiles - 1 - (int)blockIdx.y;  // longest tiles first
  const int seq = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, j = lane >> 4, c = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // provably wave-uniform

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
  // Retire the Q loads before the load ring starts, so that no wait inside the loop has
  // to cover them (the ring's own waits count only its direct loads).
  vm_wait<0>();

  const int64_t blk_stride = (int64_t)a.num_kv_heads * 16 * D;
  const int64_t head_off = (int64_t)kvh * 16 * D;
  const int32_t* bt_row = a.block_table + (int64_t)seq * a.bt_row_stride;

  // Block ids come from a 64-entry window of the table row held one per lane and are
  // read with readlane (uniform).  A window refill waits for every outstanding load
  // (a vector-memory wait cannot single one out); it happens once per 64 blocks.
  int win0 = -64, btw = 0;
  auto clamp_col = [&](int col) { return col > a.max_blocks - 1 ? a.max_blocks - 1 : col; };
  uint32_t badbits = 0;  // bit 2*stage + b: block b of that stage's step is not a valid id

  // Direct global->LDS loads.  Instruction p of a plane writes 1 KiB at piece p of the
  // stage (lane L -> byte 16 L), i.e. row p*RPP + L/CPR at 16-byte slot L%CPR.  The
  // slot must hold chunk slot ^ swz(row), so each lane fetches that chunk: every
  // instruction still reads RPP whole rows, all inside one cache block, so the block
  // base is uniform.  An invalid block id reads block 0 instead (always mapped); rows
  // past the range read whatever the table maps them to.  compute() masks both.
  auto issue = [&](int step) {
    const int stage = step % kPrefStages;
    const int c0 = clamp_col(2 * step), c1 = clamp_col(2 * step + 1);  // same 64-window
    if (c0 < win0 || c0 >= win0 + 64) {
      win0 = c0 & ~63;
      btw = win0 + lane < a.max_blocks ? bt_row[win0 + lane] : 0;
      vm_wait<0>();
    }
    const int64_t b0 = __builtin_amdgcn_readlane(btw, c0 - win0);
    const int64_t b1 = __builtin_amdgcn_readlane(btw, c1 - win0);
    const bool bad0 = b0 < 0 || b0 >= a.num_blocks, bad1 = b1 < 0 || b1 >= a.num_blocks;
    badbits = (badbits & ~(3u << (2 * stage))) | ((bad0 ? 1u : 0u) << (2 * stage)) |
              ((bad1 ? 2u : 0u) << (2 * stage));
#pragma unroll
    for (int e = 0; e < IPW; ++e) {
      const int u = wave * IPW + e;                     // instruction index in the step
      const bool vplane = u >= PIECES;
      const int piece = vplane ? u - PIECES : u;
      const int r0 = piece * RPP;                       // first row of the piece
      const int64_t blk = r0 < 16 ? (bad0 ? 0 : b0) : (bad1 ? 0 : b1);
      const int64_t row0 = blk * blk_stride + head_off + (int64_t)(r0 & 15) * D;
      const int r = r0 + lane / CPR;
      const uint32_t off = (uint32_t)(((lane / CPR) * D + 8 * ((lane % CPR) ^ pref_swz<D>(r))) * 2);
      if (vplane)
        lds_dma16(a.vplane + row0, off, &lv[stage][piece * 512]);
      else
        lds_dma16(a.kplane + row0, off, &lk[stage][piece * 512]);
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
    const bool bad0 = (badbits >> (2 * buf)) & 1u;
    const bool bad1 = (badbits >> (2 * buf + 1)) & 1u;
    const bool tail = kv0 + kPrefBlockN > kv_end;  // rows past the range hold stale bits
    const bool masked = diag || bad0 || bad1 || tail;

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
      if (masked) {  // stale rows may hold NaN bits: clear them (NaN * 0 = NaN)
        const int kp = kv0 + r;
        if (kp >= kv_end || ((e >> 2) ? bad1 : bad0)) vrow[e] = VT{};
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
        if (masked) ok = kp <= qpos && kp < kv_end && !(blk == 0 ? bad0 : bad1);
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
      if (__ballot(alpha != 1.f)) {  // rescale only when some row's max moved
#pragma unroll
        for (int b = 0; b < DPL; ++b) acc[nb][b] *= alpha;
      }
      pb[nb] = __builtin_bit_cast(
          bf16x8, u32x4{pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3]),
                        pack_bf16x2(p[4], p[5]), pack_bf16x2(p[6], p[7])});
    }

    // O^T += V^T P^T, one MFMA per (m-block, N-block).
#pragma unroll
    for (int b = 0; b < DPL; ++b) {
      uint32_t w[4];
#pragma unroll
      for (int h = 0; h < 4; ++h)
        w[h] = pack_halves(vrow[2 * h][b >> 1], vrow[2 * h + 1][b >> 1], b & 1);
      const bf16x8 va = __builtin_bit_cast(bf16x8, u32x4{w[0], w[1], w[2], w[3]});
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        acc[nb][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[nb], acc[nb][b], 0, 0, 0);
    }
  };

  // Main loop over a kPrefStages-deep ring: while step t computes, the direct loads of
  // steps t+1 .. t+kPrefStages-1 are in flight.  One barrier per step: it publishes
  // step t's loads and retires every wave's compute(t-1), whose stage step t reuses.
#pragma unroll
  for (int t = 0; t < kPrefStages - 1; ++t)
    if (t < nsteps) issue(t);
  for (int step = 0; step < nsteps; ++step) {
    // Loads issued after step's own: min(kPrefStages - 2, nsteps - 1 - step) steps.
    const int ahead = nsteps - 1 - step < kPrefStages - 2 ? nsteps - 1 - step : kPrefStages - 2;
    if (ahead >= 2) vm_wait<2 * IPW>();
    else if (ahead == 1) vm_wait<IPW>();
    else vm_wait<0>();
    lds_barrier();
    if (step + kPrefStages - 1 < nsteps) issue(step + kPrefStages - 1);
    compute(step, step % kPrefStages);
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

// Workgroup shape (see the launch below).  NDL_PREFILL_VARIANT overrides it for tuning.
inline int prefill_variant() {
  static const int v = [] {
    const char* e = getenv("NDL_PREFILL_VARIANT");
    const int x = e ? atoi(e) : 2;
    return (x >= 0 && x <= 2) ? x : 2;
  }();
  return v;
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
  const int variant = prefill_variant();
  const int block_m = variant == 0 ? 128 : variant == 1 ? 64 : 128;
  const int64_t qtiles = ((int64_t)max_seqlen + block_m - 1) / block_m;
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
  // variant 0: 4 waves x 32 rows; 1: 4 waves x 16 rows; 2: 8 waves x 16 rows.
  if (head_dim == 128) {
    if (variant == 1)
      hipLaunchKernelGGL((varlen_prefill_kernel<128, 1, 4>), grid, dim3(256), 0, s, a);
    else if (variant == 2)
      hipLaunchKernelGGL((varlen_prefill_kernel<128, 1, 8>), grid, dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((varlen_prefill_kernel<128, 2, 4>), grid, dim3(256), 0, s, a);
  } else {
    if (variant == 1)
      hipLaunchKernelGGL((varlen_prefill_kernel<64, 1, 4>), grid, dim3(256), 0, s, a);
    else if (variant == 2)
      hipLaunchKernelGGL((varlen_prefill_kernel<64, 1, 8>), grid, dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((varlen_prefill_kernel<64, 2, 4>), grid, dim3(256), 0, s, a);
  }
  return check_launch();
}
