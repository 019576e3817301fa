// Varlen causal prefill attention over the paged cache, gfx950 (CDNA4).
//
// Reference: needle/layers/attention.py:120-134 (_prefill_pytorch): per packed
// sequence, causal softmax(q K^T / sqrt(D)) V with the GQA group expanded.  The
// reference attends the fresh k/v; here K/V are read back through block_table
// after ndl_kv_append wrote them (attention.py:103 runs _write_kv first), which
// is the same data when context_lens == 0 and also covers a cached prefix.
//
// Design:
//   * The work of one (sequence, kv head) is a list of jobs, one per (query head of
//     the GQA group, 32-row query subtile), subtile-major: job j is head j % g of
//     subtile j / g.  A workgroup runs eight consecutive jobs, one per wave, so every
//     K/V tile staged in LDS serves eight jobs and each of the four SIMDs carries two
//     busy waves whatever g is (with one job per head, g = 7 would leave a SIMD half
//     idle).  The eight jobs span one or two subtiles when g >= 7 (more for smaller
//     groups); the workgroup walks the keys up to its last subtile's end and each
//     wave masks past its own rows.
//   * K/V advance 32 keys (two cache blocks) per step through an NS-stage LDS ring
//     filled by direct global->LDS loads (global_load_lds_dwordx4, no register
//     staging), 1 KiB per instruction: a K piece is whole rows (contiguous), landed
//     with a row-dependent 16-byte chunk swizzle; a V piece is 64 bytes of each of a
//     block's 16 rows.
//   * S^T = K Q^T on v_mfma_f32_32x32x16_bf16: A = K rows from LDS
//     (ds_read_b128), B = Q^T held in registers.  Lane l holds the scores of query
//     row l%32 for 16 of the 32 keys, so a row max needs one permlane32 swap.
//   * The S^T accumulator, rounded to bf16, is the B operand (P^T) of
//     O^T = V^T P^T on the same instruction with the k order
//     k = 8h + e -> key 16t + 4h + (e&3) + 8(e>>2); the matching V^T operand comes
//     straight from LDS through ds_read_b64_tr_b16 (4 keys x 16 head_dim columns
//     per 16 lanes), so P and V need no register shuffles.
//   * Software pipeline: QK of step t+1 is issued before the softmax of step t,
//     so the MFMA pipe works while the VALU computes exponentials.
//   * fp32 online softmax in the exp2 domain (scale * log2 e folded into one FMA);
//     the exponentials use the running max as it stands, and only a step whose
//     probabilities could exceed 2^kRescaleSlack (a lane's partial sum above it) or a
//     row's first attended step takes the exact path (row max, in-place O^T rescale,
//     exponentials again), so no row max is computed on most steps; the row sums add
//     the fp32 probabilities with v_add_f32 (no v_dot2: the dot unit shares the MFMA
//     pipe, while plain VALU instructions issue beside the MFMAs).
//   * Each step first issues its LDS reads and the QK MFMAs of the next step, which
//     depend on nothing else in it, then the ring upkeep, masking and softmax.
//   * Causal masking only on steps that reach past a wave's first query position;
//     query tiles are dispatched longest-first.
#include "ndl_common.hpp"

namespace ndl {

constexpr int kPrefKeys = 32;          // keys per step (two cache blocks)
constexpr int kPrefRows = 32;          // query rows per wave
constexpr int kPrefWaves = 8;          // waves (jobs) per workgroup
// Tile-list limits of the persistent launch (larger batches use one workgroup per tile).
constexpr int kPrefListSeqs = 8192;
constexpr int kPrefListLevels = 2048;
// exp2-domain growth of a row max tolerated before the accumulator is rescaled:
// probabilities stay <= 2^8, exact in bf16's exponent range and in fp32 sums.
constexpr float kRescaleSlack = 8.0f;
// A lane's partial sum of one step's probabilities above this takes the exact path.
constexpr float kGrowSum = 256.0f;   // 2^kRescaleSlack
static_assert(kGrowSum == (float)(1 << (int)kRescaleSlack), "growth bound is 2^slack");

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
  // Keys are read in 16-token tiles: a block (table column) holds 1 << tile_shift of them
  // (log2(block_size / 16)), so a table row of W columns holds max_tiles = W << tile_shift.
  int tile_shift;
  int max_tiles;
  const int32_t* cu_seqlens;
  const int32_t* context_lens;
  int num_heads;
  int group;          // query heads per kv head
  float scale_log2;
  int num_qtiles;
  int64_t num_tokens;
  int num_seqs;
  int persistent;     // 1: grid of resident workgroups walking the tile list
  // Rotary embedding of q (ROPE kernels): cos/sin rows of every packed token.
  const u16* rope_cos;
  const u16* rope_sin;
  int64_t rope_stride;
};

// One workgroup tile, looked up one tile ahead by the persistent walk: jobs
// 8 qtile .. 8 qtile + 7 of sequence seq, kv head kvh, with the sequence's cu_seqlens
// pair and context length as loaded (checked where they are used, so that the look-up
// does not wait for the loads).  seq < 0: no tile.
struct PrefTile {
  int seq, qtile, kvh;
  int tok0, tok1, ctx;
};

typedef __attribute__((ext_vector_type(4))) short i16x4v;

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
// wave-uniform) and they land at LDS byte address lds_addr + 16 * L (lds_addr uniform).
// Issued from inline asm so the compiler does not order every later LDS read behind
// it (it cannot tell the ring's stages apart); the ring waits on vmcnt itself.
// M0 takes the LDS base; one wait state separates the M0 write from its use.  M0 is
// a reserved register, so clang ignores it in the clobber list: this is sound only
// while no other instruction in these kernels keeps a value in M0, which
// tests/test_isa_guards.py checks on the generated code.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void* gbase, uint32_t lane_off,
                                          uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(lane_off), "s"(gbase)
               : "memory", "m0");
}
// The same with one dword per lane, landing at lds_addr + 4 * L.
__device__ __forceinline__ void lds_dma4(const void* gbase, uint32_t lane_off, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "v"(lane_off), "s"(gbase)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS byte address of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// 16-byte chunk swizzle of a staged K row (row index within the 32-row stage).
//   D = 128 (16 chunks per row): ((r & 3) << 2) | ((r >> 2) & 3)
//   D = 64  (8 chunks per row):  (((r >> 1) & 1) << 2) | ((r >> 2) & 3)
// Both keep the K operand read (16 consecutive rows at one chunk, ds_read_b128)
// conflict-free.
template <int D>
__device__ __forceinline__ int pref_swz(int r) {
  return D == 128 ? (((r & 3) << 2) | ((r >> 2) & 3)) : ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
}

// A compile-time int as a type, for the unrolled ring turn below.
template <int N>
struct Ic {
  static constexpr int value = N;
};
// f(Ic<J>{}) for J = J0 .. N-1 in order.
template <int J0, int N, class F>
__device__ __forceinline__ void unroll(F& f) {
  if constexpr (J0 < N) {
    f(Ic<J0>{});
    unroll<J0 + 1, N>(f);
  }
}

// Combine a value with the one held by lane l ^ 32 (v_permlane32_swap of a register
// with itself: one result holds the lower half's values, the other the upper half's).
__device__ __forceinline__ float half_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ROPE: q is the raw projection; each Q row is rotated as it is read into the operand
// registers (with the reference's rounding, rope8), from cos/sin rows of its token.
// F16: the elements are fp16 (else bf16).
template <int D, int NS, bool ROPE, bool F16>
__global__ __launch_bounds__(64 * kPrefWaves) void varlen_prefill_kernel(PrefillArgs a) {
  using T = Elt<F16>;
  using X8 = typename T::x8;
  constexpr int KS = D / 16;          // k-steps of the QK MFMA (16 head_dim each)
  constexpr int DT = D / 32;          // 32-wide head_dim tiles of O^T
  constexpr int CPR = D / 8;          // 16-byte chunks per row
  constexpr int RPP = 512 / D;        // rows per 1 KiB piece (one direct load)
  constexpr int PIECES = kPrefKeys / RPP;                 // pieces per plane per step
  constexpr int IPW = 2 * PIECES / kPrefWaves;            // direct loads per wave per step
  static_assert(IPW >= 1 && (2 * PIECES) % kPrefWaves == 0, "load distribution");
  static_assert(NS >= 5 && NS - 3 <= 6 && (NS - 3) * IPW < 64, "ring depth");
  static_assert(2 * NS - 3 >= kPrefWaves, "an output piece per wave");

  // Ring of NS steps; each stage holds 32 K rows and 32 V rows.
  __shared__ __attribute__((aligned(16))) u16 lk[NS][kPrefKeys * D];
  __shared__ __attribute__((aligned(16))) u16 lv[NS][kPrefKeys * D];
  __shared__ uint32_t lds_sink[64];   // destination of the L2 warm-up loads, never read
  __shared__ int32_t s_btw[64];       // first table window of the tile (prefetched)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // provably wave-uniform
  // The lane number through an empty asm: per-lane offsets computed from it stay where they
  // are used instead of being hoisted out of the tile loop (and kept live, in registers
  // the ring needs, or spilled).
  auto fresh_lane = [&] {
    int l = lane;
    asm volatile("" : "+v"(l));
    return l;
  };
  const int r32 = lane & 31, h = lane >> 5;

  // The look-up reads through the scalar cache (constant address space; the kernel never
  // writes these arrays): its waits count scalar loads only and never drain the ring's
  // direct loads.
  typedef const __attribute__((address_space(4))) int32_t* cptr;
  auto look_up = [&](int seq, int qtile, int kvh) {
    const cptr cu = (cptr)a.cu_seqlens, cl = (cptr)a.context_lens;
    return PrefTile{seq, qtile, kvh, cu[seq], cu[seq + 1], cl[seq]};
  };
  // First row of a tile's first job.
  auto first_row = [&](int qtile) { return qtile * kPrefWaves / a.group * kPrefRows; };
  // A tile's first token, rows and cached tokens; false if it has no rows.  Rows past
  // num_tokens are never touched, whatever cu_seqlens holds.
  auto bounds = [&](const PrefTile& t, int64_t& tok0, int& n, int& ctx) {
    if (t.seq < 0) return false;
    tok0 = t.tok0;
    const int64_t tok1 = t.tok1 < a.num_tokens ? (int64_t)t.tok1 : a.num_tokens;
    if (tok0 < 0 || tok1 <= tok0 || (int64_t)first_row(t.qtile) >= tok1 - tok0) return false;
    n = (int)(tok1 - tok0);
    ctx = t.ctx < 0 ? 0 : t.ctx;
    return true;
  };

  // One query tile (see PrefTile).  Every wave of the workgroup runs it together (it has
  // workgroup barriers).  ahead() resolves nx, the tile this workgroup takes next
  // (n == 0: none); it runs while the tile's first loads are in flight, and nx's Q rows
  // and table window are pulled into the L2 at the end of this tile.
  bool btw_next = false;
  auto tile = [&](const PrefTile& t, const PrefTile& nx, auto&& ahead) {
    const bool pre = btw_next;
    btw_next = false;
    int64_t tok0;
    int n, ctx;
    if (!bounds(t, tok0, n, ctx)) {
      ahead();
      return;
    }
    const int seq = t.seq, kvh = t.kvh;
    const int job0 = t.qtile * kPrefWaves;
    const int job = job0 + wave;
    const int sub = job / a.group;                               // this wave's subtile
    const int hg = job - sub * a.group;                          // head within the group
    const int head = kvh * a.group + hg;
    const int row0 = job0 / a.group * kPrefRows;                 // the tile's first row
    const int row_end = ((job0 + kPrefWaves - 1) / a.group + 1) * kPrefRows;
    const int kv_end = ctx + (row_end < n ? row_end : n);
    const int nsteps = (kv_end + kPrefKeys - 1) / kPrefKeys;

    const int wrow0 = sub * kPrefRows;                           // first row of this wave
    const bool wave_active = wrow0 < n;
    const int qpos_min = ctx + wrow0;
    const int qpos = ctx + wrow0 + r32;                          // this lane's query position
    // Position of this wave's last query row (-1: the wave has no rows).
    const int qpos_last = wave_active ? ctx + (wrow0 + kPrefRows <= n ? wrow0 + kPrefRows : n) - 1 : -1;

    const int tshift = a.tile_shift, tmask = (1 << tshift) - 1;
    const int32_t* bt_row = a.block_table + (int64_t)seq * a.bt_row_stride;
    // Block ids are int32; every id in [0, nb32) is a valid block.
    const uint32_t nb32 = a.num_blocks > 0x7fffffff ? 0x80000000u : (uint32_t)a.num_blocks;
    // Tile `sub` of block b, kv head kvh, starts at plane + kvh * bs * D + u * 16 * D with
    // u = b * Hkv * 2^shift + sub (the tile's index in units of 16 rows; u * 16 * D is
    // within the plane, so u fits 32 bits).
    const uint32_t units_per_blk = (uint32_t)a.num_kv_heads << tshift;

    // The tiles' block ids come from a 64-tile window of the table row, one tile per lane
    // (lane l: tile win0 + l, table column (win0 + l) >> shift), held as unit indices u
    // (an invalid id as block 0, with its lane's bit set in win_badm) and read with
    // readlane (uniform).  The first window goes out with the Q loads below and one wait
    // covers both; a later refill waits for every outstanding load (a vector-memory wait
    // cannot single one out); it happens once per 64 tiles.
    int win0 = 0;
    int btw = 0;
    uint64_t win_badm = 0;
    auto to_unit = [&](int raw, int t) {
      return (int)(((uint32_t)raw < nb32 ? (uint32_t)raw : 0u) * units_per_blk +
                   (uint32_t)(t & tmask));
    };
    if (!pre && wave == 0) {
      const int l = fresh_lane();
      lds_dma4(bt_row, 4u * (uint32_t)((l < a.max_tiles ? l : a.max_tiles - 1) >> tshift),
               lds_addr(s_btw));
      vm_wait<0>();
    }

    // B operand of S^T = K Q^T: lane l supplies Q[row l%32][16 s + 8 h .. + 8), read from
    // LDS at the ring start (below).  Loads issued after a step's (window refills) only
    // make a ring wait, which counts the direct loads issued after that step, wait longer,
    // never shorter: vector-memory loads complete in issue order.
    X8 qb[KS];

    // Every wave stages, per step, IPW of the PIECES / 2 pieces (1 KiB, one direct load
    // each) that block ld_blk of the step holds in plane ld_plane (K, V): pieces
    // ld_half * IPW + e of the block, so that no wave's issue time carries more loads
    // than another's (the step ends at a barrier).
    //   K piece: RPP rows, row-major, LDS slot L%CPR of row L/CPR holding chunk
    //     (L%CPR) ^ swz(row).
    //   V piece e of a block: its 16 rows at head_dim 32 e .. +32 ([row][32 d], 64 bytes
    //     per row): lane L -> row L/4, chunk 4 e + L%4.
    static_assert((PIECES / 2) % IPW == 0, "load distribution");
    const int ld_plane = wave >> 2, ld_blk = (wave >> 1) & 1, ld_half = wave & 1;
    const u16* ld_head = (ld_plane ? a.vplane : a.kplane) + ((int64_t)kvh << tshift) * 16 * D;
    uint32_t ld_off[IPW];
#pragma unroll
    for (int e = 0; e < IPW; ++e) {
      const int pe = ld_half * IPW + e;                     // piece within the block
      if (ld_plane == 0) {
        const int r0 = (ld_blk * (PIECES / 2) + pe) * RPP;  // first row of the piece (stage)
        const int r = r0 + lane / CPR;
        ld_off[e] = (uint32_t)((((r0 & 15) + lane / CPR) * D +
                                8 * ((lane % CPR) ^ pref_swz<D>(r))) * 2);
      } else {
        ld_off[e] = (uint32_t)(((lane >> 2) * D + 32 * pe + 8 * (lane & 3)) * 2);
      }
    }
    const uint32_t lds_k0 = lds_addr(&lk[0][0]), lds_v0 = lds_addr(&lv[0][0]);
    const uint32_t ld_lds =
        (ld_plane ? lds_v0 : lds_k0) + (ld_blk * (PIECES / 2) + ld_half * IPW) * 1024;

    auto clamp_col = [&](int col) { return col > a.max_tiles - 1 ? a.max_tiles - 1 : col; };
    // bit 2*stage + b: block b of that stage's step is not a valid id.  Every wave keeps
    // its own copy (all waves walk the same table window).
    uint32_t badbits = 0;

    // Stage `step` into ring slot `stage`: note its block validity and issue this wave's
    // direct loads of it.  An invalid block id reads block 0 instead (always mapped);
    // rows past the range read whatever the table maps them to.  The softmax masks both.
    // A window of the table with no invalid id (the normal case) sets no bits.
    auto stage_in = [&](int step, int stage) {
      const int c0 = clamp_col(2 * step), c1 = clamp_col(2 * step + 1);  // same 64-window
      if (c0 < win0 || c0 >= win0 + 64) {
        win0 = c0 & ~63;
        const int l = fresh_lane();
        const int raw = win0 + l < a.max_tiles ? bt_row[(win0 + l) >> tshift] : 0;
        vm_wait<0>();
        win_badm = __builtin_amdgcn_ballot_w64(win0 + lane < a.max_tiles &&
                                               (uint32_t)raw >= nb32);
        btw = to_unit(raw, win0 + l);
      }
      badbits &= ~(3u << (2 * stage));
      if (win_badm)
        badbits |= ((uint32_t)((win_badm >> (c0 - win0)) & 1u) |
                    ((uint32_t)((win_badm >> (c1 - win0)) & 1u) << 1)) << (2 * stage);
      const uint32_t u = (uint32_t)__builtin_amdgcn_readlane(btw, (ld_blk ? c1 : c0) - win0);
      const u16* base = ld_head + (int64_t)u * 16 * D;
      const uint32_t lds = ld_lds + (uint32_t)stage * (kPrefKeys * D * 2);
#pragma unroll
      for (int e = 0; e < IPW; ++e)
        lds_dma16(base, ld_off[e], lds + 1024 * e);
    };

    // Waits until this wave's loads of the step after the current one have landed:
    // `later` = steps issued after it.
    auto wait_loads = [&](int later) {
      switch (later) {
        case 0: vm_wait<0>(); break;
        case 1: vm_wait<IPW>(); break;
        case 2: vm_wait<2 * IPW>(); break;
        case 3: vm_wait<3 * IPW>(); break;
        case 4: vm_wait<4 * IPW>(); break;
        case 5: vm_wait<5 * IPW>(); break;
        default: vm_wait<6 * IPW>(); break;
      }
    };

    // Per-lane LDS element offsets of the operands inside a stage.
    //   K (A of S^T = K Q^T), k-step s: row l%32, chunk 2s + h.
    int koff[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) koff[s] = r32 * D + 8 * ((2 * s + h) ^ pref_swz<D>(r32));
    // V^T operand (k-step t, head_dim tile dt, half k): the V piece (t, dt) holds rows
    // 16t .. 16t+15 as [row][32 d]; lane (G = l/16, i = l%16) reads 4 elements of row
    // 8k + 4h + i/4 at head_dim 16 (G&1) + 4 (i%4), and ds_read_b64_tr_b16 hands lane i
    // column i of each of the 4 rows (keys 16t + 8k + 4h + x, x = 0..3).
    const int vlane = (4 * h + ((lane & 15) >> 2)) * 32 + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    f32x16 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f32x16{};
    float m_run = kNegInf;   // running max of this lane's row (exp2 domain)
    float l_run = 0.f;       // this lane's share of the row sum

    // K operands of one stage (read ahead of the MFMAs that use them).
    auto k_reads = [&](int stage, u32x4* ka) {
      const u16* kt = lk[stage];
#pragma unroll
      for (int s = 0; s < KS; ++s) ka[s] = *reinterpret_cast<const u32x4*>(&kt[koff[s]]);
    };
    // S^T of one step: st[r] = score of key 8(r/4) + 4h + r%4 for query row l%32.
    auto qk = [&](const u32x4* ka) {
      f32x16 st = {};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        st = T::mfma32x32x16(__builtin_bit_cast(X8, ka[s]), qb[s], st);
      return st;
    };
    // P = exp2(s * scale log2e - m) rounded to bf16 (the B operand of the PV product);
    // the row sum adds the fp32 values in a tree of v_add_f32.  (v_dot2_f32_bf16 on the
    // rounded pairs would take half the instructions, but the dot unit is the matrix
    // core's: each one holds the MFMA pipe for ~10 cycles, where plain VALU work runs
    // beside the MFMAs.)
    auto probs = [&](const f32x16& st, float m_use, uint32_t* pw, float& lsum) {
      float p[16];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        p[r] = fast_exp2(fmaf(st[r], a.scale_log2, -m_use));
        p[r + 1] = fast_exp2(fmaf(st[r + 1], a.scale_log2, -m_use));
        pw[r >> 1] = T::pack(p[r], p[r + 1]);
      }
#pragma unroll
      for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int i = 0; i < w; ++i) p[i] = p[i] + p[i + w];
      lsum += p[0];
    };
    // V^T operands of one step (all 16 transpose reads issued together, ahead of the
    // exponentials, so that no PV MFMA waits on LDS latency).
    auto v_reads = [&](int stage, X8* vop) {
      const u16* vt = lv[stage] + vlane;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const u16* piece = vt + (t * DT + dt) * 512;
          const i16x4v v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4v*)(piece));
          const i16x4v v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4v*)(piece + 8 * 32));
          const u32x2 w0 = __builtin_bit_cast(u32x2, v0), w1 = __builtin_bit_cast(u32x2, v1);
          vop[t * DT + dt] = __builtin_bit_cast(X8, u32x4{w0[0], w0[1], w1[0], w1[1]});
        }
    };
    // O^T += V^T P^T over the step's 32 keys.
    auto pv = [&](const X8* vop, const uint32_t* pw) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const X8 pb = __builtin_bit_cast(X8, u32x4{pw[4 * t], pw[4 * t + 1], pw[4 * t + 2],
                                                   pw[4 * t + 3]});
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          acc[dt] = T::mfma32x32x16(vop[t * DT + dt], pb, acc[dt]);
      }
    };

    // V rows past the range or in an invalid block may hold any bits, NaN included, and
    // NaN * 0 = NaN in the PV product: a step with such rows has them cleared in LDS once
    // its loads have landed (one barrier before its PV).  Only a workgroup's last step
    // and steps over invalid block ids need this.
    auto needs_vzero = [&](int step, int stage) {
      return step * kPrefKeys + kPrefKeys > kv_end || ((badbits >> (2 * stage)) & 3u) != 0;
    };
    auto zero_v = [&](int step, int stage) {
      const int kv0 = step * kPrefKeys;
      int valid[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int v = (badbits >> (2 * stage + t)) & 1u ? 0 : kv_end - (kv0 + 16 * t);
        valid[t] = v < 0 ? 0 : (v > 16 ? 16 : v);
      }
      // 16-byte chunk c of the stage's V plane: piece c / 64 (t = piece / DT), row (c % 64) / 4
      for (int c = tid; c < 2 * DT * 64; c += blockDim.x) {
        const int piece = c >> 6, row = (c & 63) >> 2;
        if (row >= valid[piece / DT]) st16(&lv[stage][c * 8], u32x4{0u, 0u, 0u, 0u});
      }
    };

    // The ring walks the steps two at a time (trip t: steps t, t + 1).  At the start of
    // a trip, steps up to min(t + NS - 3, nsteps - 1) have their loads issued and V rows
    // of steps up to t are cleared where needed.  A trip normally has one barrier, before
    // step t: it publishes steps t + 1 and t + 2 (K of step t + 2 is read by step t + 1),
    // retires every wave's reads of steps before t, whose slots then take steps
    // t + NS - 2 and t + NS - 1, and clears V rows of step t + 2.  A trip whose second step
    // has V rows to clear (the last step, steps over invalid block ids) takes a second
    // barrier before step t + 1 instead.
    //   kPair:  barrier publishing t + 1, t + 2; issues t + NS - 2, t + NS - 1
    //   kFirst: barrier publishing t + 1;        issues t + NS - 2, t + NS - 1
    //   kSecond (step t + 1): barrier publishing t + 2; also the last step of an odd
    //           count, whose loads the trip before waited for and whose V rows it
    //           cleared (the barrier publishes the clearing)
    //   kNone:  no barrier (second step of a paired trip)
    enum { kNone = 0, kPair = 1, kFirst = 2, kSecond = 3 };
    auto slot_after = [](int stage, int k) { return stage + k >= NS ? stage + k - NS : stage + k; };
    // Returns the last step the barrier publishes (`step` itself when there is none).
    auto sync = [&](int step, int mode) {
      const int lead = step + (mode == kPair ? 2 : 1);
      const int need = lead < nsteps - 1 ? lead : nsteps - 1;
      if (need > step) {
        // steps issued at the barrier before this one, counted from `step`
        const int ahead = step + (mode == kSecond ? NS - 2 : NS - 3);
        const int later = (ahead < nsteps - 1 ? ahead : nsteps - 1) - need;
        if (later == NS - 5) vm_wait<(NS - 5) * IPW>();   // a paired trip in full flow
        else wait_loads(later);
      }
      lds_barrier();
      return need;
    };
    auto upkeep = [&](int step, int stage, int need, int mode) {
      if (mode != kSecond) {
        if (step + NS - 2 < nsteps) stage_in(step + NS - 2, slot_after(stage, NS - 2));
        if (step + NS - 1 < nsteps) stage_in(step + NS - 1, slot_after(stage, NS - 1));
      }
      if (need > step) {
        const int ns = slot_after(stage, need - step);
        if (needs_vzero(need, ns)) zero_v(need, ns);
      }
    };

    // Softmax and PV of one step whose scores are st (may_mask false: the caller knows
    // the step needs no mask).
    auto finish = [&](int step, int stage, f32x16 st, const X8* vop, bool may_mask) {
      const int kv0 = step * kPrefKeys;
      const bool masked = kv0 + kPrefKeys - 1 > qpos_min || kv0 + kPrefKeys > kv_end ||
                          ((badbits >> (2 * stage)) & 3u) != 0;
      if (may_mask && masked) {
        // Element r holds key kv0 + 4h + o(r), o(r) = 8 (r/4) + r%4 (o < 16 exactly for
        // r < 8, the step's first block).  It is attended iff key <= qpos, key < kv_end and
        // its block is valid, i.e. o(r) <= one limit per lane and block: one compare each.
        const int base = kv0 + 4 * h;
        const int lim = min(qpos, kv_end - 1) - base;
        const int lim0 = (badbits >> (2 * stage)) & 1u ? -1 : lim;
        const int lim1 = (badbits >> (2 * stage + 1)) & 1u ? -1 : lim;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int o = 8 * (r >> 2) + (r & 3);
          st[r] = o <= (r < 8 ? lim0 : lim1) ? st[r] : kNegInf;
        }
      }
      // Exponentials against the running max as it stands.  A row whose max grew by
      // more than the slack has some p > 2^slack, so its lane's partial sum of the step
      // exceeds 2^slack; then (and while a row has no running max yet, i.e. at its first
      // attended step) the wave takes the exact path: row max, in-place rescale, the
      // exponentials again.  No row max is computed otherwise.  (A sum past the bound
      // without such a p only costs an early rescale.)
      uint32_t pw[8];
      float lstep = 0.f;
      probs(st, m_run == kNegInf ? 0.f : m_run, pw, lstep);
      const bool exact = !(lstep <= kGrowSum) || m_run == kNegInf;
      if (__builtin_amdgcn_ballot_w64(exact) != 0) {
        float m3[6];  // row max as a tree (three levels of 3-input max)
#pragma unroll
        for (int i = 0; i < 5; ++i) m3[i] = fmaxf(fmaxf(st[3 * i], st[3 * i + 1]), st[3 * i + 2]);
        m3[5] = st[15];
        float mx = fmaxf(fmaxf(fmaxf(m3[0], m3[1]), m3[2]), fmaxf(fmaxf(m3[3], m3[4]), m3[5]));
        mx = half_max(mx);
        const float m_new = fmaxf(m_run, mx * a.scale_log2);
        if (m_new != m_run) {
          // While m_run is -inf every probability so far was 0 (V rows that could hold
          // non-finite bits are cleared), so the accumulator and the sum are 0 and need no
          // rescale: a row's first attended step (every wave's first step of a tile)
          // skips it.
          if (m_run != kNegInf) {
            // The accumulator is scaled in place (tied asm operands: a plain multiply lets
            // the register allocator give the scaled accumulator new registers and copy it
            // back on every step).
            const float alpha = fast_exp2(m_run - m_new);
            // The compiler's hazard tracking does not look into inline asm: the first
            // multiply carries the wait state a VALU read of a transcendental's result
            // needs (without it, it reads the register's previous contents).
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
              for (int i = 0; i < 16; ++i) {
                if (t == 0 && i == 0)
                  asm volatile("s_nop 1\n\tv_mul_f32 %0, %0, %1" : "+v"(acc[t][i]) : "v"(alpha));
                else
                  asm volatile("v_mul_f32 %0, %0, %1" : "+v"(acc[t][i]) : "v"(alpha));
              }
            l_run *= alpha;
          }
          m_run = m_new;
        }
        lstep = 0.f;
        probs(st, m_run == kNegInf ? 0.f : m_run, pw, lstep);
      }
      l_run += lstep;
      pv(vop, pw);
    };

    // One step: QK(step + 1) and the softmax + PV of step, after the trip's barrier if
    // `mode` has one.  Masking (steps that reach past a wave's first query position, the
    // tail, invalid blocks) and the rare rescale are the only other branches.  QK of a
    // step past the last one reads a stale slot; its scores are never used.
    auto iteration = [&](int step, int stage, f32x16& st_cur, f32x16& st_next, int mode) {
      const int nstage = stage + 1 == NS ? 0 : stage + 1;
      int need = 0;
      if (mode != kNone) need = sync(step, mode);
      // The LDS reads (K of step + 1, V of this step) and the QK MFMAs of step + 1 depend on
      // nothing below, so they go out first: the matrix core runs while the ring upkeep,
      // the row max, the growth check and the exponentials of this step run.  The upkeep
      // writes only slots no wave reads before the next barrier: those of steps before
      // this one, and V of step `need`, read after it.
      // A step wholly past this wave's last query row (the last step of a tile whose
      // jobs span two subtiles, for the earlier subtile's waves; every step of a wave with
      // no rows) contributes nothing: its LDS reads, MFMAs and softmax are skipped (a
      // wave-uniform branch; the barriers and the loads stay).  QK of step + 1 is skipped
      // exactly when step + 1 will be.
      // (The V reads may follow the upkeep: it writes no slot of this step.)
      u32x4 ka[KS];
      X8 vop[2 * DT];
      if ((step + 1) * kPrefKeys <= qpos_last) {
        k_reads(nstage, ka);
        st_next = qk(ka);
      }
      if (mode != kNone) upkeep(step, stage, need, mode);
      if (step * kPrefKeys <= qpos_last) {
        v_reads(stage, vop);
        finish(step, stage, st_cur, vop, true);
      }
    };

    // Ring start: steps 0 .. NS-3 in flight before the first trip.  The first barrier
    // retires every wave's reads of the previous tile (persistent launch) before the slots
    // are refilled.  Steps 0 and 1 go out first.  The wave's Q rows are staged in one plane
    // of slots 2 .. 5, free until step 2 is staged (wave w: the K plane of slot 2 + w/2 for
    // even w, else its V plane), by whole-row direct loads (RPP rows per instruction, the K
    // pieces' row-dependent chunk swizzle), and read back in the operand layout: loading
    // the operand layout from memory directly (32 rows x 32 bytes per instruction) moves a
    // third of the bytes per cycle that whole rows do through the CU's memory path.  Rows
    // past the range load the wave's first row (the tile's first row for a wave with no
    // rows) and are zeroed when read.  The second barrier publishes steps 0 and 1 and
    // retires the Q reads; then steps 2 .. NS - 3 go out.
    static_assert(NS >= 2 + kPrefWaves / 2, "Q staging planes in slots 2 ..");
    lds_barrier();
    {
      const int l = fresh_lane();
      const int raw = l < a.max_tiles ? s_btw[l] : 0;
      win_badm = __builtin_amdgcn_ballot_w64(l < a.max_tiles && (uint32_t)raw >= nb32);
      btw = to_unit(raw, l);
    }
    stage_in(0, 0);
    if (nsteps > 1) stage_in(1, 1);
    u16* const qplane = (wave & 1) ? lv[2 + (wave >> 1)] : lk[2 + (wave >> 1)];
    {
      const u16* qbase = a.q + (tok0 + (wave_active ? wrow0 : 0)) * a.q_tok_stride +
                         (int64_t)head * D;
      const uint32_t ql = lds_addr(qplane);
#pragma unroll
      for (int e = 0; e < KS; ++e) {          // 32 rows x D x 2 bytes = KS pieces of 1 KiB
        const int r = e * RPP + lane / CPR;
        const int rr = wave_active && wrow0 + r < n ? r : 0;
        const int c = (lane % CPR) ^ pref_swz<D>(r);
        lds_dma16(qbase, (uint32_t)((rr * a.q_tok_stride + 8 * c) * 2), ql + 1024 * e);
      }
    }
    // Rotary embedding of the staged Q rows (ROPE).  Row r's element pairs (d, d + D/2) are
    // chunk pairs (p, p + KS), KS = D/16 pairs per row; lane l takes pair l % KS of rows
    // (64/KS) i + l / KS, i < KS/2, so that each cos/sin load instruction covers whole
    // 128-byte halves of rows (coalesced).  Those loads go out with the Q rows; once both
    // have landed the lane rotates its pairs in the wave's own Q plane (read, rope8, write
    // back: the wave's LDS accesses complete in order), and the operand layout is read
    // from the rotated rows below.  A row past the range reads the tile's first row of
    // cos/sin; its Q operand is zeroed when read.
    constexpr int RIPL = ROPE ? KS / 2 : 1;      // (row, pair) items per lane
    u32x4 rcos[RIPL][2], rsin[RIPL][2];
    if constexpr (ROPE) {
      const int l = fresh_lane();   // offsets computed here, not hoisted out of the tile loop
#pragma unroll
      for (int i = 0; i < RIPL; ++i) {
        const int row = (64 / KS) * i + l / KS, p = l % KS;
        const int rr = wave_active && wrow0 + row < n ? wrow0 + row : 0;
        const int64_t off = (tok0 + rr) * a.rope_stride + 8 * p;
        rcos[i][0] = ld16(a.rope_cos + off);
        rcos[i][1] = ld16(a.rope_cos + off + D / 2);
        rsin[i][0] = ld16(a.rope_sin + off);
        rsin[i][1] = ld16(a.rope_sin + off + D / 2);
      }
    }
    ahead();
    vm_wait<0>();   // this wave's Q rows (and cos/sin), and steps 0 and 1, landed
    if constexpr (ROPE) {
      const int l = fresh_lane();
#pragma unroll
      for (int i = 0; i < RIPL; ++i) {
        const int row = (64 / KS) * i + l / KS, p = l % KS;
        u16* const lo_at = qplane + row * D + 8 * (p ^ pref_swz<D>(row));
        u16* const hi_at = qplane + row * D + 8 * ((p + KS) ^ pref_swz<D>(row));
        u32x4 lo = *reinterpret_cast<const u32x4*>(lo_at);
        u32x4 hi = *reinterpret_cast<const u32x4*>(hi_at);
        u32x4 rlo, rhi;
        rope8<F16>(lo, hi, rcos[i][0], rcos[i][1], rsin[i][0], rsin[i][1], rlo, rhi);
        *reinterpret_cast<u32x4*>(lo_at) = rlo;
        *reinterpret_cast<u32x4*>(hi_at) = rhi;
      }
      __builtin_amdgcn_wave_barrier();
    }
    {
      const bool ok = wave_active && wrow0 + r32 < n;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(&qplane[koff[s]]);
        qb[s] = __builtin_bit_cast(X8, ok ? w : u32x4{0u, 0u, 0u, 0u});
      }
    }
    lds_barrier();
    if (nx.seq >= 0) {
      if (wave == 0) {
        const int l = fresh_lane();
        lds_dma4(a.block_table + (int64_t)nx.seq * a.bt_row_stride,
                 4u * (uint32_t)((l < a.max_tiles ? l : a.max_tiles - 1) >> tshift),
                 lds_addr(s_btw));
      }
      btw_next = true;
    }
#pragma unroll
    for (int t = 2; t < NS - 2; ++t)
      if (t < nsteps) stage_in(t, t);
    if (needs_vzero(0, 0)) zero_v(0, 0);
    f32x16 st0, st1;
    {
      u32x4 ka[KS];
      k_reads(0, ka);
      st0 = qk(ka);
    }
    int step = 0, stage = 0;

    // Unmasked trips: both steps' keys lie wholly below every wave's first query row (no
    // mask, full steps) and no block id in flight is invalid.  The ring protocol of a
    // paired trip below, with only the bookkeeping such a trip needs: a constant load
    // wait while the ring is in full flow, staging of the steps that exist, clearing of
    // step + 2 (the last step can be partial).
    {
      const int lim = (ctx + row0 + 1) / kPrefKeys - 1;   // t + 1 < steps below row0's first query
      // Issues step x into slot sl if it exists; the general path for a new table window,
      // a window with an invalid id, or a table row too short for the step.
      auto stage_fast = [&](int x, int sl) {
        if (x >= nsteps) return;
        const int c0 = 2 * x;
        if (c0 >= win0 + 64 || win_badm || c0 + 1 >= a.max_tiles) {
          stage_in(x, sl);
          return;
        }
        const uint32_t u = (uint32_t)__builtin_amdgcn_readlane(btw, c0 + ld_blk - win0);
        const u16* base = ld_head + (int64_t)u * 16 * D;
        const uint32_t lds = ld_lds + (uint32_t)sl * (kPrefKeys * D * 2);
#pragma unroll
        for (int e = 0; e < IPW; ++e)
          lds_dma16(base, ld_off[e], lds + 1024 * e);
      };
      constexpr uint32_t unit_bytes = 16 * D * 2;   // one 16-row tile of one kv head
      while (step < lim && badbits == 0) {
        // Fast trips: every per-trip check of the trip below holds for the whole run, so it
        // is tested once: both steps staged (step + NS - 2, step + NS - 1) exist and their
        // four tiles lie inside the current window and the table row (no clamp);
        // the window has no invalid id (badbits stays 0); step + 2 is a full step (no V
        // rows to clear); the ring is in full flow (a constant load wait).  What is left
        // per trip is the barrier, two block look-ups and their loads.
        if (!win_badm) {
          const int wcols = win0 + 64 < a.max_tiles ? win0 + 64 : a.max_tiles;
          int end = lim;
          if (nsteps - NS + 1 < end) end = nsteps - NS + 1;            // step + NS - 1 exists
          if (kv_end / kPrefKeys - 2 < end) end = kv_end / kPrefKeys - 2;   // step + 2 full
          if ((wcols - 2 * NS + 2) / 2 < end) end = (wcols - 2 * NS + 2) / 2;  // columns
          for (; step < end; step += 2) {
            const int stage1 = stage + 1 == NS ? 0 : stage + 1;
            const int stage2 = stage1 + 1 == NS ? 0 : stage1 + 1;
            vm_wait<(NS - 5) * IPW>();
            lds_barrier();
            u32x4 ka[KS];
            X8 vop[2 * DT];
            k_reads(stage1, ka);
            v_reads(stage, vop);
            st1 = qk(ka);
            {
              // This wave's tile of steps step + NS - 2 and step + NS - 1: tiles ci and
              // ci + 2 of the window.
              const int ci = 2 * (step + NS - 2) + ld_blk - win0;
              const uint32_t b0 = (uint32_t)__builtin_amdgcn_readlane(btw, ci);
              const uint32_t b1 = (uint32_t)__builtin_amdgcn_readlane(btw, ci + 2);
              const u16* base0 = (const u16*)((const char*)ld_head + (uint64_t)b0 * unit_bytes);
              const u16* base1 = (const u16*)((const char*)ld_head + (uint64_t)b1 * unit_bytes);
              const uint32_t l0 = ld_lds + (uint32_t)slot_after(stage, NS - 2) * (kPrefKeys * D * 2);
              const uint32_t l1 = ld_lds + (uint32_t)slot_after(stage, NS - 1) * (kPrefKeys * D * 2);
#pragma unroll
              for (int e = 0; e < IPW; ++e) lds_dma16(base0, ld_off[e], l0 + 1024 * e);
#pragma unroll
              for (int e = 0; e < IPW; ++e) lds_dma16(base1, ld_off[e], l1 + 1024 * e);
            }
            finish(step, stage, st0, vop, false);
            k_reads(stage2, ka);
            v_reads(stage1, vop);
            st0 = qk(ka);
            finish(step + 1, stage1, st1, vop, false);
            stage = stage2;
          }
          if (step >= lim) break;
        }
        const int stage1 = stage + 1 == NS ? 0 : stage + 1;
        const int stage2 = stage1 + 1 == NS ? 0 : stage1 + 1;
        // Loads of steps up to step + 2 (the last one at most) landed: steps issued after
        // it stay out, NS - 5 of them while the ring is in full flow.
        if (step + NS - 3 <= nsteps - 1) {
          vm_wait<(NS - 5) * IPW>();
        } else {
          const int need = step + 2 < nsteps - 1 ? step + 2 : nsteps - 1;
          wait_loads(nsteps - 1 - need);
        }
        lds_barrier();
        u32x4 ka[KS];
        X8 vop[2 * DT];
        k_reads(stage1, ka);
        v_reads(stage, vop);
        st1 = qk(ka);
        stage_fast(step + NS - 2, slot_after(stage, NS - 2));
        stage_fast(step + NS - 1, slot_after(stage, NS - 1));
        if (step + 2 < nsteps && needs_vzero(step + 2, stage2)) zero_v(step + 2, stage2);
        finish(step, stage, st0, vop, false);
        k_reads(stage2, ka);
        v_reads(stage1, vop);
        st0 = qk(ka);
        finish(step + 1, stage1, st1, vop, false);
        stage = stage2;
        step += 2;
      }
    }

    for (; step + 2 <= nsteps; step += 2) {
      const int stage1 = stage + 1 == NS ? 0 : stage + 1;
      const bool pair = !needs_vzero(step + 1, stage1);
      iteration(step, stage, st0, st1, pair ? kPair : kFirst);
      iteration(step + 1, stage1, st1, st0, pair ? kNone : kSecond);
      stage = stage1 + 1 == NS ? 0 : stage1 + 1;
    }
    if (step < nsteps) iteration(step, stage, st0, st1, kSecond);  // a barrier, no loads

    // Pull the next tile's Q rows of this wave and (wave 0) its table window into the
    // L2, after the ring's last wait: direct loads into a scratch LDS word per lane that
    // nothing reads, retired by the next tile's first wait.  Lane l touches row l / 2,
    // 128-byte half l % 2 of the row's head slice.
    if (btw_next && wave == 0) vm_wait<0>();
    int64_t ntok0;
    int nn, nctx;
    if (bounds(nx, ntok0, nn, nctx)) {
      const int njob = nx.qtile * kPrefWaves + wave;
      const int nsub = njob / a.group, nhg = njob - nsub * a.group;
      const int nrow0 = nsub * kPrefRows;
      if (nrow0 < nn) {
        const int l = fresh_lane();
        const int r = nrow0 + (l >> 1) < nn ? l >> 1 : 0;
        const u16* base = a.q + (ntok0 + nrow0) * a.q_tok_stride +
                          (int64_t)(nx.kvh * a.group + nhg) * D;
        lds_dma4(base, (uint32_t)(r * a.q_tok_stride * 2) + (D >= 128 ? (l & 1) * 128u : 0u),
                 lds_addr(lds_sink));
      }
    }

    if (!wave_active) return;
    const float l = half_sum(l_run);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    // The output tile (32 rows x D, the size of one K or V plane of a stage) goes through
    // an LDS piece no wave reads after the tile's last barrier, so that every store
    // covers whole rows.  After that barrier the waves read at most K of stage
    // nsteps - 1 and V of stages nsteps - 2 and nsteps - 1 (slots mod NS); wave w takes
    // the K plane of slot nsteps + w for w < NS - 1, else the V plane of slot
    // nsteps + w - (NS - 1).  Chunk c (16 bytes) of row r sits at chunk c ^ (r % CPR).
    u16* piece;
    {
      const int k = wave < NS - 1 ? wave : wave - (NS - 1);
      const int sl = (nsteps + k) % NS;
      piece = wave < NS - 1 ? lk[sl] : lv[sl];
    }
    // The lane number passes through an empty asm so that the offset arithmetic below
    // stays here instead of being hoisted out of the tile loop (and kept live, in
    // registers the ring needs).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int rr = ln & 31, hh = ln >> 5;
    // acc[dt][i] holds O[row rr][d = 32 dt + 8 (i/4) + 4 hh + i%4]: chunk 4 dt + i/4, half hh.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        *reinterpret_cast<u32x2*>(piece + rr * D + 8 * ((4 * dt + b) ^ (rr % CPR)) + 4 * hh) =
            u32x2{T::pack(acc[dt][4 * b] * inv, acc[dt][4 * b + 1] * inv),
                  T::pack(acc[dt][4 * b + 2] * inv, acc[dt][4 * b + 3] * inv)};
    // Lane L reads back chunk L % CPR of row 64 / CPR * i + L / CPR (the wave's own writes:
    // LDS accesses of one wave complete in order).
    __builtin_amdgcn_wave_barrier();
    constexpr int RPI = 64 / CPR;                     // rows per instruction
    const int c = ln % CPR;
    u32x4 ov[32 / RPI];
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int r = RPI * i + ln / CPR;
      ov[i] = *reinterpret_cast<const u32x4*>(piece + r * D + 8 * (c ^ (r % CPR)));
    }
    u16* dst = a.out + ((tok0 + wrow0 + ln / CPR) * a.num_heads + head) * (int64_t)D + 8 * c;
    const int64_t rstride = (int64_t)RPI * a.num_heads * D;   // elements per RPI rows
    if (wrow0 + 32 <= n) {
#pragma unroll
      for (int i = 0; i < 32 / RPI; ++i) *reinterpret_cast<u32x4*>(dst + i * rstride) = ov[i];
    } else {
#pragma unroll
      for (int i = 0; i < 32 / RPI; ++i)
        if (wrow0 + RPI * i + ln / CPR < n) *reinterpret_cast<u32x4*>(dst + i * rstride) = ov[i];
    }
  };  // tile

  if (!a.persistent) {
    tile(look_up(blockIdx.y, a.num_qtiles - 1 - (int)blockIdx.z, blockIdx.x),
         PrefTile{-1, 0, 0, 0, 0, 0}, [] {});
    return;
  }

  // Persistent launch: every workgroup builds the same tile list in LDS, longest tiles
  // first (level t = query tile index, from the last down to 0; within a level the
  // sequences that reach it, ascending, times the kv-head chunks), then takes items
  // w, 2G-1-w, 2G+w, 4G-1-w, ... (G workgroups).  Query tiles past max_seqlen are not
  // computed, as in the one-workgroup-per-tile launch.
  __shared__ uint16_t s_ntiles[kPrefListSeqs];
  __shared__ int s_cnt[kPrefListLevels];    // sequences with more than t tiles
  __shared__ int s_off[kPrefListLevels];    // items in the levels above t
  const int S = a.num_seqs, NQ = a.num_qtiles, KVC = a.num_kv_heads;
  for (int t = tid; t < NQ; t += blockDim.x) s_cnt[t] = 0;
  lds_barrier();
  for (int q = tid; q < S; q += blockDim.x) {
    const int64_t t0 = a.cu_seqlens[q];
    int64_t t1 = a.cu_seqlens[q + 1];
    if (t1 > a.num_tokens) t1 = a.num_tokens;
    int nt = 0;
    if (t0 >= 0 && t1 > t0) {
      const int64_t subs = (t1 - t0 + kPrefRows - 1) / kPrefRows;
      const int64_t x = (subs * a.group + kPrefWaves - 1) / kPrefWaves;
      nt = x > NQ ? NQ : (int)x;
    }
    s_ntiles[q] = (uint16_t)nt;
    if (nt > 0) atomicAdd(&s_cnt[nt - 1], 1);
  }
  lds_barrier();
  if (wave == 0) {  // suffix sums: s_cnt[t] = #seqs with ntiles > t; s_off[t] = items above t
    int run_cnt = 0, run_items = 0;
    for (int base = NQ - 1; base >= 0; base -= 64) {
      const int t = base - lane;
      const int hcount = t >= 0 ? s_cnt[t] : 0;
      // inclusive prefix over lanes 0..lane (descending t)
      int inc = hcount;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(inc, d, 64);
        if (lane >= d) inc += o;
      }
      const int cnt = run_cnt + inc;                 // seqs with ntiles > t
      int inc_items = cnt;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(inc_items, d, 64);
        if (lane >= d) inc_items += o;
      }
      if (t >= 0) {
        s_cnt[t] = cnt;
        s_off[t] = (run_items + inc_items - cnt) * KVC;
      }
      run_cnt = __shfl(cnt, 63, 64);
      run_items += __shfl(inc_items, 63, 64);
    }
  }
  lds_barrier();
  const int total = NQ > 0 ? s_off[0] + s_cnt[0] * KVC : 0;
  const int G = gridDim.x, w = blockIdx.x;
  int lvl = NQ - 1;
  int r = 0;
  // The item of the next round that has one, resolved (false: none left).
  auto next_item = [&](PrefTile& out) {
    for (; r * G < total; ++r) {
      const int j = (r & 1) ? r * G + (G - 1 - w) : r * G + w;
      if (j >= total) continue;
      // Level of item j (j only grows): the highest t <= lvl with
      // j < s_off[t] + s_cnt[t] * KVC (the items in levels >= t), 64 levels per look.
      for (;;) {
        const int t = lvl - lane;
        const uint64_t m = __builtin_amdgcn_ballot_w64(t >= 0 && j < s_off[t] + s_cnt[t] * KVC);
        if (m != 0) {
          lvl -= __builtin_ctzll(m);
          break;
        }
        lvl -= 64;
      }
      const int i = j - s_off[lvl];
      int rank = i / KVC;
      const int c = i - rank * KVC;
      int seq = -1;
      for (int base = 0; base < S && seq < 0; base += 64) {
        const int q = base + fresh_lane();
        const bool has = q < S && s_ntiles[q] > lvl;
        const uint64_t m = __builtin_amdgcn_ballot_w64(has);
        const int pc = __builtin_popcountll(m);
        if (rank < pc) {
          // the lane whose bit is set with `rank` set bits below it
          const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
          seq = base + __builtin_ctzll(__builtin_amdgcn_ballot_w64(has && below == rank));
        } else {
          rank -= pc;
        }
      }
      out = look_up(seq, lvl, c);
      ++r;
      return true;
    }
    return false;
  };
  // One tile ahead: each tile resolves the next one while its own first loads are out.
  PrefTile cur, nxt;
  bool have = next_item(cur), more = false;
  while (have) {
    tile(cur, nxt, [&] {
      more = next_item(nxt);
      if (!more) nxt.seq = -1;
    });
    cur = nxt;
    have = more;
  }
}

}  // namespace ndl

namespace ndl {

// Shared by both entry points; cos == nullptr: q is already rotated.
static int launch_prefill(void* out, const void* q, int64_t q_tok_stride, const void* cos,
                          const void* sin, int64_t cs_tok_stride, const void* kv_cache,
                          int64_t num_blocks, const int32_t* block_table, int64_t bt_row_stride,
                          int max_blocks_per_seq, const int32_t* cu_seqlens,
                          const int32_t* context_lens, int num_seqs, int64_t num_tokens,
                          int max_seqlen, int max_context_len, int num_heads, int num_kv_heads,
                          int head_dim, int block_size, int dtype, float scale,
                          ndl_stream_t stream) {
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  const int tshift = block_tile_shift(block_size);
  if (tshift < 0 || (head_dim != 64 && head_dim != 128)) return NDL_ERR_UNSUPPORTED;
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0)
    return NDL_ERR_INVALID_ARG;
  if (num_seqs < 0 || num_tokens < 0 || max_seqlen < 0 || max_context_len < 0 ||
      num_blocks <= 0 || max_blocks_per_seq <= 0 || bt_row_stride < max_blocks_per_seq ||
      q_tok_stride < (int64_t)num_heads * head_dim)
    return NDL_ERR_INVALID_ARG;
  if (((int64_t)max_blocks_per_seq << tshift) > 0x7fffffff) return NDL_ERR_UNSUPPORTED;
  const bool rope = cos != nullptr || sin != nullptr;
  if (rope && (cos == nullptr || sin == nullptr || cs_tok_stride < head_dim ||
               (cs_tok_stride & 7) || (((uintptr_t)cos | (uintptr_t)sin) & 15u)))
    return NDL_ERR_INVALID_ARG;
  if (num_seqs == 0 || num_tokens == 0 || max_seqlen == 0) return NDL_OK;
  if (!out || !q || !kv_cache || !block_table || !cu_seqlens || !context_lens)
    return NDL_ERR_INVALID_ARG;
  if (((uintptr_t)out | (uintptr_t)q | (uintptr_t)kv_cache) & 15u) return NDL_ERR_INVALID_ARG;
  if (q_tok_stride & 7) return NDL_ERR_INVALID_ARG;
  if (dtype_is_f32(dtype))
    return launch_prefill_f32(out, q, q_tok_stride, cos, sin, cs_tok_stride, kv_cache,
                              num_blocks, block_table, bt_row_stride, max_blocks_per_seq,
                              cu_seqlens, context_lens, num_seqs, num_tokens, max_seqlen,
                              max_context_len, num_heads, num_kv_heads, head_dim, block_size,
                              scale, stream);
  (void)max_context_len;

  const int group = num_heads / num_kv_heads;

  // Eight jobs (query head, 32-row subtile) per workgroup; a (sequence, kv head) pair has
  // group * ceil(rows / 32) jobs.
  const int waves = kPrefWaves;
  const int64_t qtiles = (((int64_t)max_seqlen + kPrefRows - 1) / kPrefRows * group +
                          kPrefWaves - 1) / kPrefWaves;
  const int64_t gx = num_kv_heads;
  if (num_seqs > 65535 || qtiles > 65535 || gx > 0x7fffffff) return NDL_ERR_UNSUPPORTED;

  PrefillArgs a;
  a.out = (u16*)out;
  a.q = (const u16*)q;
  a.q_tok_stride = q_tok_stride;
  a.kplane = (const u16*)kv_cache;
  a.vplane = a.kplane + num_blocks * num_kv_heads * (int64_t)block_size * head_dim;
  a.num_blocks = num_blocks;
  a.num_kv_heads = num_kv_heads;
  a.block_table = block_table;
  a.bt_row_stride = bt_row_stride;
  a.tile_shift = tshift;
  a.max_tiles = max_blocks_per_seq << tshift;
  a.cu_seqlens = cu_seqlens;
  a.context_lens = context_lens;
  a.num_heads = num_heads;
  a.group = group;
  a.scale_log2 = scale * kLog2e;
  a.num_qtiles = (int)qtiles;
  a.num_tokens = num_tokens;
  a.rope_cos = (const u16*)cos;
  a.rope_sin = (const u16*)sin;
  a.rope_stride = cs_tok_stride;

  hipStream_t s = (hipStream_t)stream;
  // Persistent launch (one resident workgroup per slot, walking the longest-first tile
  // list) unless the list would not fit in LDS.
  a.num_seqs = num_seqs;
  a.persistent = num_seqs <= kPrefListSeqs && qtiles <= kPrefListLevels &&
                 gx * (int64_t)num_seqs * qtiles < ((int64_t)1 << 31);
  // [f16][head_dim 128][rope]
  const void* const fns[2][2][2] = {
      {{(const void*)varlen_prefill_kernel<64, 8, false, false>,
        (const void*)varlen_prefill_kernel<64, 8, true, false>},
       {(const void*)varlen_prefill_kernel<128, 6, false, false>,
        (const void*)varlen_prefill_kernel<128, 6, true, false>}},
      {{(const void*)varlen_prefill_kernel<64, 8, false, true>,
        (const void*)varlen_prefill_kernel<64, 8, true, true>},
       {(const void*)varlen_prefill_kernel<128, 6, false, true>,
        (const void*)varlen_prefill_kernel<128, 6, true, true>}}};
  const void* fn = fns[dtype_is_f16(dtype) ? 1 : 0][head_dim == 128 ? 1 : 0][rope ? 1 : 0];
  dim3 grid((unsigned)gx, (unsigned)num_seqs, (unsigned)qtiles);
  if (a.persistent) {
    const int64_t slots = resident_workgroups(fn, 64 * waves);
    if (slots <= 0) return NDL_ERR_LAUNCH;
    const int64_t items = gx * (int64_t)num_seqs * qtiles;   // upper bound of the list
    grid = dim3((unsigned)(items < slots ? items : slots), 1, 1);
  }
  void* args[] = {&a};
  if (hipLaunchKernel(fn, grid, dim3(64 * waves), args, 0, s) != hipSuccess) {
    (void)hipGetLastError();  // clear the error so that the next call's check sees its own
    return NDL_ERR_LAUNCH;
  }
  return check_launch();
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
  return ndl::launch_prefill(out, q, q_tok_stride, nullptr, nullptr, 0, kv_cache, num_blocks,
                             block_table, bt_row_stride, max_blocks_per_seq, cu_seqlens,
                             context_lens, num_seqs, num_tokens, max_seqlen, max_context_len,
                             num_heads, num_kv_heads, head_dim, block_size, dtype, scale,
                             stream);
}

extern "C" int ndl_rope_varlen_prefill(void* out, const void* q, int64_t q_tok_stride,
                                       const void* cos, const void* sin, int64_t cs_tok_stride,
                                       const void* kv_cache, int64_t num_blocks,
                                       const int32_t* block_table, int64_t bt_row_stride,
                                       int max_blocks_per_seq, const int32_t* cu_seqlens,
                                       const int32_t* context_lens, int num_seqs,
                                       int64_t num_tokens, int max_seqlen, int max_context_len,
                                       int num_heads, int num_kv_heads, int head_dim,
                                       int block_size, int dtype, float scale,
                                       ndl_stream_t stream) {
  if (cos == nullptr || sin == nullptr) return NDL_ERR_INVALID_ARG;
  return ndl::launch_prefill(out, q, q_tok_stride, cos, sin, cs_tok_stride, kv_cache,
                             num_blocks, block_table, bt_row_stride, max_blocks_per_seq,
                             cu_seqlens, context_lens, num_seqs, num_tokens, max_seqlen,
                             max_context_len, num_heads, num_kv_heads, head_dim, block_size,
                             dtype, scale, stream);
}
