// Paged decode attention for gfx950 (CDNA4).
//
// Reference: needle/layers/attention.py:291-310 (_decode_pytorch): per
// sequence gather K/V blocks, expand the GQA group, softmax(q K^T * scale) V.
//
// Work split (stream-K): for each kv head, the 16-token tiles of all sequences are
// laid end to end, each sequence after one empty slot (sequence i owns slots
// P_i .. P_i + 1 + n_i, n_i = ceil(L_i / 16)), and wave s of the kv head takes the C
// consecutive slots s*C .. s*C + C, whatever sequences they belong to.  Every wave has
// about the same amount of K/V to stream (the empty slot stands for the cost of starting
// a sequence), so all of them run for the whole launch (a per-sequence split leaves the
// waves of short remainders idle while the long ones finish).  The (wave s, sequence i)
// piece of a sequence that spans waves leaves partial (m, l, unnormalised acc) in
// segment slot s + i of its kv head (unique: the waves and the sequences are both
// in stream order); a sequence inside one wave is written directly.  A wave finds
// its first sequence with a wave-parallel prefix scan of context_lens.
//
// Per tile (one wave64):
//   * The g query heads of a kv head are the N columns (padded to 16) of a
//     16x16 MFMA tile; the 16 tokens of one cache block are its M rows.
//     S^T = K . Q^T runs as head_dim/32 v_mfma_f32_16x16x32_bf16 steps; K is
//     fetched in row layout (1 KiB contiguous per load instruction), staged in a
//     swizzled 4 KiB LDS tile and read back in the A-operand layout.
//   * The S^T accumulator layout (lane 16j+c holds tokens 4j..4j+3 of head c)
//     is exactly the B operand layout of v_mfma_f32_16x16x16bf16_1k, so
//     P^T feeds O^T = V^T . P^T without any cross-lane movement.  V^T is the
//     A operand; the head_dim index of the M rows is permuted (row m of
//     m-block b is d = (D/16)*m + b) so that every lane loads D/16 contiguous
//     elements of a V row and only repacks registers.
//   * Online softmax in fp32 with exp2 (scale folded with log2 e).  The row
//     max needs two cross-lane exchanges per block.
// A second kernel merges the partials of the sequences that span waves and writes
// zeros for sequences with nothing to attend.
//
// Small batches (kv heads x sequences x NW waves within the resident waves, at most 32
// tiles per wave at head_dim 64, 16 at 128): one workgroup of NW = 8 waves per (kv head,
// sequence) instead.  Wave w takes every NW-th tile (w, w + NW, ..) through the same
// per-tile code, and the waves combine their (m, l, acc) through LDS with one barrier: one
// launch, no workspace traffic.  With few sequences the stream split would cut every
// sequence into many 2-tile pieces and the merge kernel would cost as much as the attention.
//
// float32 pools and activations go to paged_decode_f32.hip (the entry points below check the
// arguments every format shares, then dispatch).
#include <stdlib.h>

#include "ndl_common.hpp"

namespace ndl {

// The fewest tiles a wave of the automatic split takes: shorter pieces cost more in
// partials and merge work than their parallelism gains (Llama-3-8B decode at one GPU's
// share of 8-way tensor parallelism, 1 kv head, ~4.4 tiles per resident wave: 25.4 us per
// layer at 5 tiles per wave, 23.3 at 8; shares with longer even splits are unchanged).
constexpr int kDecodeMinChunk = 8;
// Waves per workgroup of the per-sequence split, and the most tiles per wave for which
// the automatic choice takes it (a table of up to 256 columns at head_dim 64, 128 at
// 128).  Eight waves (two per SIMD) measured faster than sixteen (four per SIMD) at
// head_dim 64, e.g. the Qwen2-0.5B decode step 6.07 against 7.46 us with cold pools,
// and faster than four at both head dims.
template <int D> constexpr int seq_split_waves() { return 8; }
template <int D> constexpr int seq_split_max_tiles() { return D == 64 ? 32 : 16; }

template <int D> struct VRow;
template <> struct VRow<128> { using T = u32x4; };  // 8 bf16 per lane per token
template <> struct VRow<64> { using T = u32x2; };   // 4 bf16 per lane per token

template <int D>
__device__ __forceinline__ typename VRow<D>::T load_vrow(const u16* p) {
  if constexpr (D == 128)
    return ldg16(p);
  else
    return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}

struct DecodeArgs {
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
  // log2(block_size / 16): a block (table column) holds 1 << tile_shift tiles of 16 tokens;
  // tile t of a sequence is rows 16 (t mod 2^shift) .. + 16 of its column t >> shift.
  int tile_shift;
  const int32_t* context_lens;
  int num_heads;
  int group;
  float scale_log2;
  int num_seqs;
  int chunk;      // C: stream slots per wave; 0: ceil(T / waves) from the stream length T
  int waves;      // waves per kv head
  int nseg;       // segment slots per kv head: waves per kv head + num_seqs
  float* ws_ml;   // [kv head][segment][group head][2] = (m, l)
  float* ws_acc;  // [kv head][segment][group head][D]
  // Fused append (null: none): the step's new k/v rows, [seq][kv head][D] with these token
  // strides, written into the cache and attended in the same pass.
  const u16* k_new;
  const u16* v_new;
  int64_t k_new_stride, v_new_stride;
  // Rotary embedding of the step (null: q and k_new are already rotated): cos/sin rows of
  // each sequence's new token, [seq][D] with row stride rope_stride.
  const u16* rope_cos;
  const u16* rope_sin;
  int64_t rope_stride;
};

__device__ __forceinline__ int64_t attended_len(const DecodeArgs& a, int seq) {
  int64_t L = (int64_t)a.context_lens[seq] + 1;  // attention.py:299
  // a table row holds at most W blocks of 16 << tile_shift tokens
  const int64_t cap = (int64_t)a.max_blocks << (4 + a.tile_shift);
  return L < cap ? L : cap;
}

__device__ __forceinline__ int seq_tiles(const DecodeArgs& a, int q) {
  const int64_t L = attended_len(a, q);
  return L <= 0 ? 0 : (int)((L + 15) >> 4);
}

// Stream slots of a sequence with n tiles: kStreamPad empty slots, then its tiles (none for
// a sequence with nothing to attend).  The empty slots stand for what a wave spends on
// starting a sequence (its q rows, its table window and its first block load before any
// tile computes), so that the waves that cross a sequence boundary take fewer tiles and
// finish with the others.
constexpr int kStreamPad = 1;
__device__ __forceinline__ int stream_slots(int n) { return n > 0 ? n + kStreamPad : 0; }

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

// Stream position of sequence `target`'s first slot, or of the first sequence whose slots
// reach past stream slot `tile` (target < 0).  Sequences are scanned 64 at a time; the scan
// stops at the chunk that holds the answer.  Returns the sequence in *seq (num_seqs if none) and
// its first slot in *first.
__device__ __forceinline__ void stream_locate(const DecodeArgs& a, int lane, int target,
                                              int64_t tile, int* seq, int64_t* first) {
  int64_t carry = 0;
  for (int base = 0; base < a.num_seqs; base += 64) {
    const int q = base + lane;
    const int n = q < a.num_seqs ? seq_tiles(a, q) : 0;
    const int v = stream_slots(n);
    const int incl = wave_incl_scan(v, lane);
    const int64_t excl = carry + incl - v;
    const uint64_t hit = target >= 0
        ? __builtin_amdgcn_ballot_w64(q == target)
        : __builtin_amdgcn_ballot_w64(q < a.num_seqs && n > 0 && excl + v > tile);
    if (hit) {
      const int l = __builtin_ctzll(hit);
      *seq = base + l;
      *first = __builtin_amdgcn_readlane((int)(excl - carry), l) + carry;
      return;
    }
    carry += __builtin_amdgcn_readlane(incl, 63);
  }
  *seq = a.num_seqs;
  *first = carry;
}

// Slots per wave: the fixed chunk, or the stream length (slots of all sequences of one
// kv head) over the waves of a kv head, at least kDecodeMinChunk.
// The chunk for a stream of `total` slots.
__device__ __forceinline__ int64_t stream_chunk_of(const DecodeArgs& a, int64_t total) {
  if (a.chunk > 0) return a.chunk;
  const int64_t c = (total + a.waves - 1) / a.waves;
  return c < kDecodeMinChunk ? kDecodeMinChunk : c;
}
__device__ __forceinline__ int64_t stream_chunk(const DecodeArgs& a, int lane) {
  if (a.chunk > 0) return a.chunk;
  int64_t total = 0;
  for (int base = 0; base < a.num_seqs; base += 64) {
    const int q = base + lane;
    const int n = q < a.num_seqs ? seq_tiles(a, q) : 0;
    total += __builtin_amdgcn_readlane(wave_incl_scan(stream_slots(n), lane), 63);
  }
  return stream_chunk_of(a, total);
}

// NW == 1: one wave per workgroup, wave s of a kv head takes stream slots s*C .. s*C + C.
// NW > 1: one workgroup per (kv head, sequence); wave w takes tiles w, w + NW, .. of the
// sequence and the waves combine through LDS.
// Two waves per SIMD for the default two-deep stream kernel (its 256-register budget), so
// that the fused append's few extra registers do not halve its occupancy.
// F16: the elements are fp16 (else bf16).
template <int D, int NBUF, int NW, bool APP, bool ROPE = false, bool F16 = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(
    NW == 1 && NBUF == 2 ? 2 : 1))) void paged_decode_kernel(DecodeArgs a) {
  static_assert(APP || !ROPE, "the rotary form is a form of the fused append");
  using T = Elt<F16>;
  using X8 = typename T::x8;
  constexpr int KS = D / 32;   // k-steps of the QK^T MFMA
  constexpr int DPL = D / 16;  // head_dim elements per lane per V row
  constexpr int E = 4 * DPL;   // accumulator elements per lane (head_dim E*j .. + E of head c)
  using VT = typename VRow<D>::T;
  // With the fused append, the new row reaches the cache from this kernel when the
  // workgroups are per sequence (NW > 1: no merge launch follows); in the stream split the
  // merge kernel stores it, and this kernel only attends it from registers.
  constexpr bool kStoreRow = APP && NW > 1;

  // kv head is the fastest grid index: the 8 head slices of one block (adjacent in
  // memory) are fetched by waves dispatched together.
  const int kvh = (int)(blockIdx.x % (unsigned)a.num_kv_heads);
  // NW == 1: stream wave of the kv head; NW > 1: the sequence
  const int sw = (int)(blockIdx.x / (unsigned)a.num_kv_heads);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, j = lane >> 4, c = lane & 15;
  const bool head_ok = c < a.group;
  const int head = kvh * a.group + c;

  const int tshift = a.tile_shift, tmask = (1 << tshift) - 1;
  const int64_t blk_stride = (int64_t)a.num_kv_heads * (16 << tshift) * D;
  const int64_t head_off = (int64_t)kvh * (16 << tshift) * D;
  // K is fetched in row layout (each load instruction reads RPI whole rows, 1 KiB
  // contiguous), staged in LDS and read back in the MFMA A-operand layout.
  constexpr int CPR = D / 8;      // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;   // rows per load instruction
  const int k_row = lane / CPR, k_chunk = lane % CPR;
  const int k_off = k_row * D + 8 * k_chunk;  // + RPI * D * s
  const int v_off = 4 * j * D + DPL * c;      // token rows 4j..4j+3, head_dim DPL*c..
  // Per wave: a 16 x D K tile.  With NW > 1 each wave's K tile sits at the start of a slot
  // of [E][64] floats (twice the tile) that later holds the wave's accumulators for the
  // combine, so that no wave writes LDS another wave may still be reading; (m, l) follow the
  // slots.
  constexpr int kSmemFloats = NW == 1 ? 8 * D : NW * 64 * E + NW * 32;
  __shared__ __attribute__((aligned(16))) float smem[kSmemFloats];
  u16* const ktile = NW == 1 ? reinterpret_cast<u16*>(smem) + wv * 16 * D
                             : reinterpret_cast<u16*>(smem + wv * 64 * E);
  // Chunk q of row r lives at r*D + 8*(q ^ swz(r)): conflict-free for both the
  // row-layout writes and the A-operand reads.
  auto swz = [](int r) { return D == 128 ? (r & 15) : ((r >> 1) & 7); };

  // One cache block (16 tokens) of K and V in registers.
  struct Tile {
    u32x4 k[KS];
    VT v[4];
    bool bad;
  };

  // Partial (fp32 m, l, unnormalised acc) of a piece into segment slot segid.
  auto store_partial = [&](const int segid, const f32x4 (&o)[DPL], const float mv,
                           const float lv) {
    const int64_t slot = ((int64_t)kvh * a.nseg + segid) * a.group + c;
    float* dst = a.ws_acc + slot * D + DPL * 4 * j;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int b = 0; b < DPL; b += 4)
        *reinterpret_cast<f32x4*>(dst + DPL * i + b) =
            f32x4{o[b][i], o[b + 1][i], o[b + 2][i], o[b + 3][i]};
    }
    if (j == 0) {
      a.ws_ml[slot * 2] = mv;
      a.ws_ml[slot * 2 + 1] = lv;
    }
  };
  // The piece that ends a sequence at the start of this wave's tiles is held in registers
  // and stored after the walk: stores count in the same in-order counter as loads, so
  // storing it at once would make the next sequence's first loads wait for the stores.
  // With NW > 1 the same registers hold this wave's share of its sequence.
  f32x4 held[DPL];
  float held_m = kNegInf, held_l = 0.f;
  int held_seg = -1;
#pragma unroll
  for (int b = 0; b < DPL; ++b) held[b] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Tiles lt0 .. lt1 of sequence seq (n_tiles in all) for the g heads of kv head kvh,
  // as segment segid of this kv head.
  // The tiles are lt0, lt0 + NW, .. below lt1 (consecutive in the stream split, every
  // NW-th in the per-sequence split); first_bt, if not null, holds this lane's block id of
  // the first window (column lt0 + NW * lane, clamped to the row), loaded by the caller.
  constexpr int stride = NW;

  // B operand of S^T = K Q^T: lane (j, c) supplies Q[head c][32 s + 8 j .. +8), rotated
  // (ROPE, attention.py:88, :277-283): the lane's element d = 32 s + 8 j + e pairs with
  // d + D/2, which is the same lane's chunk s + KS/2.
  auto load_q = [&](const int seq, X8 (&qb)[KS]) {
    // Lanes past the group read the group's first head (no branch around the loads, so the
    // compiler can count them) and zero it.
    const u16* qrow = a.q + (int64_t)seq * a.q_tok_stride +
                      (int64_t)(head_ok ? head : kvh * a.group) * D + 8 * j;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4 w = ld16(qrow + 32 * s);
      qb[s] = __builtin_bit_cast(X8, head_ok ? w : u32x4{0u, 0u, 0u, 0u});
    }
    if constexpr (ROPE) {
      const u16* crow = a.rope_cos + (int64_t)seq * a.rope_stride + 8 * j;
      const u16* srow = a.rope_sin + (int64_t)seq * a.rope_stride + 8 * j;
      u32x4 rc[KS], rs[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        rc[s] = ld16(crow + 32 * s);
        rs[s] = ld16(srow + 32 * s);
      }
#pragma unroll
      for (int s = 0; s < KS / 2; ++s) {
        u32x4 lo, hi;
        rope8<F16>(__builtin_bit_cast(u32x4, qb[s]), __builtin_bit_cast(u32x4, qb[s + KS / 2]),
              rc[s], rc[s + KS / 2], rs[s], rs[s + KS / 2], lo, hi);
        qb[s] = __builtin_bit_cast(X8, lo);
        qb[s + KS / 2] = __builtin_bit_cast(X8, hi);
      }
    }
  };

  // K (in row layout, staged through LDS) and V of the tile at block id blk.  An invalid
  // id reads block 0 (always mapped) and marks the tile bad.
  // Tile `sub` (16 rows) of block blk.  live = false: a placeholder load of the same
  // instructions whose lanes all read the tile's first bytes (one cache line per
  // instruction), never computed.
  auto load_tile_blk = [&](int64_t blk, int sub, Tile& t, const bool live = true) {
    t.bad = blk < 0 || blk >= a.num_blocks;  // wave-uniform
    if (t.bad) blk = 0;
    const int64_t tile_off = blk * blk_stride + head_off + (int64_t)sub * 16 * D;
    const u16* kb = a.kplane + tile_off + (live ? k_off : 0);
    const u16* vb = a.vplane + tile_off + (live ? v_off : 0);
#pragma unroll
    for (int s = 0; s < KS; ++s) t.k[s] = ldg16(kb + RPI * D * s);
#pragma unroll
    for (int i = 0; i < 4; ++i) t.v[i] = load_vrow<D>(vb + i * D);
  };

  auto segment = [&](const int seq, const int lt0, const int lt1, const int n_tiles,
                     const int segid, const int* first_bt) {
    const int64_t L = attended_len(a, seq);
    const int t1 = (int)(lt1 * 16 < L ? lt1 * 16 : L);   // one past the last token attended

    X8 qb[KS];
    load_q(seq, qb);
    const int32_t* bt_row = a.block_table + (int64_t)seq * a.bt_row_stride;

    // Fused append (attention.py:141-154 before :156-159): the new token of the step sits
    // at position p = context_lens[seq], row p % bs of table column min(p / bs, W - 1)
    // (:144-146), i.e. row p % 16 of tile app_tile, an attended tile (the last one unless
    // the table row clamps with blocks of more than 16 tokens).  The wave that owns that
    // tile writes the row into the cache and uses it in place of the row it loaded; no
    // other wave reads the tile.  Each lane loads the pieces of the new rows it holds in
    // the tile layouts: chunk k_chunk of K, head_dim DPL*c .. of V.  The row is stored
    // while the segment's first tile computes: stores count in the in-order memory
    // counter, and stored there, only loads issued after it (a tile later) wait for it.
    int app_tile = -1;
    if constexpr (APP) {
      const int p = a.context_lens[seq];   // >= 0: the sequence attends tiles
      const int pc = p >> (4 + tshift);
      app_tile = ((pc < a.max_blocks - 1 ? pc : a.max_blocks - 1) << tshift) | ((p >> 4) & tmask);
    }
    // wave-uniform: this wave attends the appended row's tile
    const bool app = APP && app_tile >= lt0 && app_tile < lt1 && (app_tile - lt0) % stride == 0;
    const int r_new = app ? a.context_lens[seq] & 15 : 0;
    // the row's offset in its block's (kv head) slice
    const int64_t app_row_off = (int64_t)(((app_tile & tmask) << 4) + r_new) * D;
    u32x4 k_app = {0u, 0u, 0u, 0u};
    VT v_app = {};
    int64_t app_blk = -1;   // the appended row's block (its table column), if valid
    if (app) {
      const u16* krow = a.k_new + (int64_t)seq * a.k_new_stride + (int64_t)kvh * D;
      k_app = ld16(krow + 8 * k_chunk);
      if constexpr (ROPE) {
        // RoPE of the new key row: chunk k_chunk pairs with chunk k_chunk ^ CPR/2
        constexpr int HC = CPR / 2;
        const bool first_half = k_chunk < HC;
        const int lo_c = first_half ? k_chunk : k_chunk - HC;
        const u32x4 partner = ld16(krow + 8 * (k_chunk ^ HC));
        const u16* crow = a.rope_cos + (int64_t)seq * a.rope_stride + 8 * lo_c;
        const u16* srow = a.rope_sin + (int64_t)seq * a.rope_stride + 8 * lo_c;
        u32x4 lo, hi;
        rope8<F16>(first_half ? k_app : partner, first_half ? partner : k_app, ld16(crow),
              ld16(crow + 8 * HC), ld16(srow), ld16(srow + 8 * HC), lo, hi);
        k_app = first_half ? lo : hi;
      }
      v_app = load_vrow<D>(a.v_new + (int64_t)seq * a.v_new_stride + (int64_t)kvh * D + DPL * c);
      if constexpr (kStoreRow) {
        const int64_t b = a.block_table[(int64_t)seq * a.bt_row_stride + (app_tile >> tshift)];
        app_blk = b >= 0 && b < a.num_blocks ? b : -1;
      }
    }

    f32x4 acc[DPL];
#pragma unroll
    for (int b = 0; b < DPL; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = kNegInf, lsum = 0.f;

    // Tiles go in windows of 64 (block ids of a window held one per lane).
    for (int w0 = lt0; w0 < lt1; w0 += 64 * stride) {
      const int left = (lt1 - w0 + stride - 1) / stride;          // tiles from w0 on
      const int ntiles = left < 64 ? left : 64;
      const int bt_lane = (first_bt != nullptr && w0 == lt0) ? *first_bt
                          : lane < ntiles ? bt_row[(w0 + stride * lane) >> tshift] : 0;
      // The window's ids are waited for here, once: a use inside the tile ring below would
      // otherwise wait for every load in flight (the compiler cannot tell which load the
      // register came from on the loop's first trip), emptying the ring at each tile.
      asm volatile("" ::"v"(bt_lane));

      auto load_tile = [&](int it, Tile& t, const bool live = true) {
        load_tile_blk(__builtin_amdgcn_readlane(bt_lane, it), (w0 + stride * it) & tmask, t,
                      live);
      };

      auto compute_tile = [&](int it, Tile& t) {
        const int tix = w0 + stride * it;   // the tile's index in the sequence
        if (kStoreRow && app && tix == lt0 && app_blk >= 0) {   // the segment's first tile
          u16* const kb = const_cast<u16*>(a.kplane) + app_blk * blk_stride + head_off + app_row_off;
          u16* const vb = const_cast<u16*>(a.vplane) + app_blk * blk_stride + head_off + app_row_off;
          if (k_row == r_new % RPI) st16(kb + 8 * k_chunk, k_app);
          if (j == (r_new >> 2)) {
            if constexpr (D == 128)
              st16(vb + DPL * c, v_app);
            else
              *reinterpret_cast<VT*>(vb + DPL * c) = v_app;
          }
        }
        if (app && tix == app_tile && !t.bad) {   // the appended token's tile
#pragma unroll
          for (int s = 0; s < KS; ++s)
            if (RPI * s + k_row == r_new) t.k[s] = k_app;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (4 * j + i == r_new) t.v[i] = v_app;
        }
        __builtin_amdgcn_wave_barrier();  // previous block's LDS reads are issued first
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int r = RPI * s + k_row;
          *reinterpret_cast<u32x4*>(ktile + r * D + 8 * (k_chunk ^ swz(r))) = t.k[s];
        }
        __builtin_amdgcn_wave_barrier();  // one wave: LDS executes its writes before its reads
        f32x4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const u32x4 ka =
              *reinterpret_cast<const u32x4*>(ktile + c * D + 8 * ((j + 4 * s) ^ swz(c)));
          st = T::mfma16x16x32(__builtin_bit_cast(X8, ka), qb[s], st);
        }
        // st[i] is the score of token tix*16 + 4j + i for head c.
        const int pos0 = tix * 16 + 4 * j;
        const bool partial = t.bad || (tix * 16 + 16 > t1);  // wave-uniform
        // This lane's tokens pos0 + i are attended for i < lim: all four in a full tile of
        // a valid block, none in an invalid one.  (A select per score, no branches.)
        const int lim = t.bad ? 0 : t1 - pos0;
        float sc[4];
        float mt = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sc[i] = i < lim ? st[i] * a.scale_log2 : kNegInf;
          mt = fmaxf(mt, sc[i]);
        }
        mt = max_xor32(max_xor16(mt));
        const float m_new = fmaxf(m, mt);
        const float m_use = m_new == kNegInf ? 0.f : m_new;
        const float alpha = fast_exp2(m - m_use);
        float p[4];
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          p[i] = fast_exp2(sc[i] - m_use);
          ps += p[i];
        }
        lsum = lsum * alpha + ps;
        m = m_new;
        if (__ballot(alpha != 1.f)) {  // rescale only when some head's max moved
#pragma unroll
          for (int b = 0; b < DPL; ++b) acc[b] *= alpha;
        }

        if (partial) {  // masked rows may hold stale bits (NaN * 0 = NaN): clear them
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (i >= lim) t.v[i] = VT{};
        }

        const u32x2 pb = {T::pack(p[0], p[1]), T::pack(p[2], p[3])};
#pragma unroll
        for (int b = 0; b < DPL; ++b) {
          const uint32_t w01 = pack_halves(t.v[0][b >> 1], t.v[1][b >> 1], b & 1);
          const uint32_t w23 = pack_halves(t.v[2][b >> 1], t.v[3][b >> 1], b & 1);
          acc[b] = T::mfma16x16x16(u32x2{w01, w23}, pb, acc[b]);
        }
      };

      // NBUF-deep ring: while block `it` computes, blocks it+1 .. it+NBUF-1 are in flight.
      const int last = ntiles - 1;
      Tile buf[NBUF];
      if constexpr (NW > 1) {
        // Per-sequence workgroups (few tiles per wave, latency-bound): every compute in
        // the loop follows its slot's load; once the next slot would lie past the window's
        // last tile, the tiles still loaded compute at that point and the walk leaves the
        // window.  (A load skipped on some path into a compute makes the compiler's wait
        // before each tile, which must hold on every path, "all loads", so the tile in
        // flight behind it is waited for too.)  Prologue slots past the end of a window
        // shorter than the ring are placeholder loads.
#pragma unroll
        for (int u = 0; u < NBUF - 1; ++u) load_tile(u < last ? u : last, buf[u], u <= last);
        bool drained = false;
        for (int it = 0; !drained; it += NBUF) {
#pragma unroll
          for (int u = 0; u < NBUF; ++u) {
            const int nxt = it + u + NBUF - 1;
            if (nxt > last) {   // tiles it+u .. last are loaded, in slots u, u+1, ..
#pragma unroll
              for (int d = 0; d < NBUF - 1; ++d)
                if (it + u + d <= last) compute_tile(it + u + d, buf[(u + d) % NBUF]);
              drained = true;
              break;
            }
            load_tile(nxt, buf[(u + NBUF - 1) % NBUF]);
            compute_tile(it + u, buf[u]);
          }
        }
      } else {
        // The stream split (many waves per SIMD hide the latency; a second copy of the
        // tile code for the ring's tail would exceed its register budget).
#pragma unroll
        for (int u = 0; u < NBUF - 1; ++u)
          if (u <= last) load_tile(u, buf[u]);
        for (int it = 0; it < ntiles; it += NBUF) {
#pragma unroll
          for (int u = 0; u < NBUF; ++u) {
            const int nxt = it + u + NBUF - 1;
            if (nxt <= last) load_tile(nxt, buf[(u + NBUF - 1) % NBUF]);
            if (it + u <= last) compute_tile(it + u, buf[u]);
          }
        }
      }
    }

    lsum = add_xor32(add_xor16(lsum));
    if (!head_ok) return;

    // acc[b][i] holds O[head c][d = DPL * (4 j + i) + b].
    if constexpr (NW > 1) {
#pragma unroll
      for (int b = 0; b < DPL; ++b) held[b] = acc[b];
      held_m = m;
      held_l = lsum;
    } else if (lt0 == 0 && lt1 == n_tiles) {  // the whole sequence: final output
      u16* const out_row = a.out + ((int64_t)seq * a.num_heads + head) * D + DPL * 4 * j;
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t w[DPL / 2];
#pragma unroll
        for (int b = 0; b < DPL; b += 2)
          w[b / 2] = T::pack(acc[b][i] * inv, acc[b + 1][i] * inv);
        if constexpr (DPL == 8)
          st16(out_row + DPL * i, u32x4{w[0], w[1], w[2], w[3]});
        else
          *reinterpret_cast<u32x2*>(out_row + DPL * i) = u32x2{w[0], w[1]};
      }
    } else if (lt0 > 0 && lt1 == n_tiles && held_seg < 0) {
#pragma unroll
      for (int b = 0; b < DPL; ++b) held[b] = acc[b];
      held_m = m;
      held_l = lsum;
      held_seg = segid;
    } else {
      store_partial(segid, acc, m, lsum);
    }
  };

  if constexpr (NW == 1) {
    // Walk the sequences that own tiles start .. end of this kv head's stream.  Up to 64
    // sequences, one load gives every sequence's tiles (lane i: sequence i): the chunk,
    // the first sequence and each sequence's tiles then come from registers.
    const bool one_load = a.num_seqs <= 64;
    int n_lane = 0;
    int64_t chunk, first;
    int seq;
    if (one_load) {
      n_lane = lane < a.num_seqs ? seq_tiles(a, lane) : 0;
      const int v_lane = stream_slots(n_lane);
      const int incl = wave_incl_scan(v_lane, lane);
      const int total = __builtin_amdgcn_readlane(incl, 63);
      chunk = stream_chunk_of(a, total);
      const int64_t tile = (int64_t)sw * chunk;
      const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < a.num_seqs && n_lane > 0 &&
                                                       (int64_t)incl > tile);
      seq = hit ? __builtin_ctzll(hit) : a.num_seqs;
      first = hit ? __builtin_amdgcn_readlane(incl - v_lane, seq) : total;
    } else {
      chunk = stream_chunk(a, lane);
      stream_locate(a, lane, -1, (int64_t)sw * chunk, &seq, &first);
    }
    const int64_t start = (int64_t)sw * chunk, end = start + chunk;
    while (seq < a.num_seqs && first < end) {
      const int nt = one_load ? __builtin_amdgcn_readlane(n_lane, seq) : seq_tiles(a, seq);
      if (nt > 0) {
        const int64_t t0 = first + kStreamPad;   // the sequence's first tile
        const int64_t s0 = start > t0 ? start : t0;
        const int64_t s1 = end < t0 + nt ? end : t0 + nt;
        if (s1 > s0)
          segment(seq, (int)(s0 - t0), (int)(s1 - t0), nt, sw + seq, nullptr);
      }
      first += stream_slots(nt);
      ++seq;
    }
    if (held_seg >= 0) store_partial(held_seg, held, held_m, held_l);
  } else {
    // Wave w takes tiles w, w + NW, w + 2 NW, .. of the sequence.  Their block ids (one
    // column per lane) do not depend on the context length, so they load alongside it.
    const int seq = sw;
    const int col = (wv + NW * lane) >> tshift;   // the table column of this lane's tile
    const int first_bt =
        a.block_table[(int64_t)seq * a.bt_row_stride + (col < a.max_blocks ? col : a.max_blocks - 1)];
    const int nt = seq_tiles(a, seq);
    if (wv < nt) segment(seq, wv, nt, nt, 0, &first_bt);
    // Combine: every wave writes its m, l and unscaled accumulators into its own LDS slot
    // (over its own K tile: one wave's LDS accesses complete in order), one barrier; then
    // each lane takes the maximum M over the waves for its head, and wave w sums elements
    // w*KPW .. + KPW of every lane over the NW waves in a fixed order, each term scaled by
    // 2^(m - M) (products rounded before the sum).  A sequence with nothing to attend (no
    // tiles) comes out as zeros (attention.py:307-308 on an empty context).
    static_assert(16 * D * 2 <= 64 * E * 4, "a wave's K tile fits its accumulator slot");
    constexpr int KPW = E / NW;
    static_assert(KPW * NW == E, "waves must divide the accumulator elements");
    float* const sacc = smem;                 // [wave][E][64]: accumulators
    float* const sm = smem + NW * 64 * E;     // [wave][16]: m
    float* const sl = sm + NW * 16;           // [wave][16]: l
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int b = 0; b < DPL; ++b) sacc[(wv * E + DPL * i + b) * 64 + lane] = held[b][i];
    }
    if (j == 0) {
      sm[wv * 16 + c] = held_m;
      sl[wv * 16 + c] = held_l;
    }
    __syncthreads();
    if (!head_ok) return;
    float mw[NW];
    float mx = kNegInf;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      mw[w] = sm[w * 16 + c];
      mx = fmaxf(mx, mw[w]);
    }
    float den = 0.f, o[KPW];
#pragma unroll
    for (int k = 0; k < KPW; ++k) o[k] = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float wt = mw[w] == kNegInf ? 0.f : fast_exp2(mw[w] - mx);
      den += __fmul_rn(sl[w * 16 + c], wt);
#pragma unroll
      for (int k = 0; k < KPW; ++k) o[k] += __fmul_rn(sacc[(w * E + wv * KPW + k) * 64 + lane], wt);
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
    u16* const out_row =
        a.out + ((int64_t)seq * a.num_heads + head) * D + E * j + wv * KPW;
    if constexpr (KPW == 1) {
      out_row[0] = T::one(o[0] * inv);
    } else {
      uint32_t w2[KPW / 2];
#pragma unroll
      for (int k = 0; k < KPW; k += 2) w2[k / 2] = T::pack(o[k] * inv, o[k + 1] * inv);
      if constexpr (KPW == 4)
        *reinterpret_cast<u32x2*>(out_row) = u32x2{w2[0], w2[1]};
      else
        *reinterpret_cast<uint32_t*>(out_row) = w2[0];
    }
  }
}

// Merge of the segment partials: one wave per (query head, sequence).  A sequence
// whose tiles lie in waves s0 .. s1 of its kv head's stream has its partials in
// segment slots s0 + seq .. s1 + seq; a sequence inside one wave was written by the
// attention kernel, and one with nothing to attend gets zeros here
// (attention.py:307-308 on an empty context).
// Pass 1 (lane-parallel over segments): global max, weights w_p = 2^(m_p - M)
// into LDS, denominator sum_p w_p l_p.  Pass 2: sum_p w_p acc_p; the first
// kMergePrefetch partials were loaded together with the (m, l) pairs, the rest
// with independent, unrolled loads.
constexpr int kMergeMaxParts = 2048;
constexpr int kMergePrefetch = 8;

template <int D, bool F16>
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(DecodeArgs a) {
  constexpr int PER_LANE = D / 64;
  __shared__ float wsh[kMergeMaxParts];
  const int head = blockIdx.x, seq = blockIdx.y, lane = threadIdx.x;
  const int kvh = head / a.group, hc = head - kvh * a.group;
  // The decode step's new K/V row (ndl_paged_decode_append): the attention kernel attended
  // it from registers; the first query head's wave of each (kv head, sequence) stores it,
  // with the separate append's rule (attention.py:141-154): column min(ctx / bs, W - 1),
  // row ctx % bs, nothing for a negative context or an invalid block id.
  if (a.k_new != nullptr && hc == 0) {
    constexpr int CH = D / 8;   // 16-byte chunks per row; lanes < CH: K, < 2 CH: V
    const int ctx = a.context_lens[seq];
    if (ctx >= 0 && lane < 2 * CH) {
      const int bshift = 4 + a.tile_shift;   // log2(block_size)
      const int pc = ctx >> bshift;
      const int col = pc < a.max_blocks - 1 ? pc : a.max_blocks - 1;
      const int64_t b = a.block_table[(int64_t)seq * a.bt_row_stride + col];
      if (b >= 0 && b < a.num_blocks) {
        const bool is_v = lane >= CH;
        const int ch = is_v ? lane - CH : lane;
        const u16* src_row = (is_v ? a.v_new + (int64_t)seq * a.v_new_stride
                                   : a.k_new + (int64_t)seq * a.k_new_stride) + (int64_t)kvh * D;
        u16* row = const_cast<u16*>(is_v ? a.vplane : a.kplane) +
                   ((b * a.num_kv_heads + kvh) << bshift) * D +
                   (int64_t)(ctx & ((1 << bshift) - 1)) * D + 8 * ch;
        u32x4 val = ld16(src_row + 8 * ch);
        if (!is_v && a.rope_cos != nullptr) {   // the key row rotated as the attention did
          constexpr int HC = CH / 2;
          const bool first_half = ch < HC;
          const int lo_c = first_half ? ch : ch - HC;
          const u32x4 partner = ld16(src_row + 8 * (ch ^ HC));
          const u16* crow = a.rope_cos + (int64_t)seq * a.rope_stride + 8 * lo_c;
          const u16* srow = a.rope_sin + (int64_t)seq * a.rope_stride + 8 * lo_c;
          u32x4 lo, hi;
          rope8<F16>(first_half ? val : partner, first_half ? partner : val, ld16(crow),
                ld16(crow + 8 * HC), ld16(srow), ld16(srow + 8 * HC), lo, hi);
          val = first_half ? lo : hi;
        }
        st16(row, val);
      }
    }
  }
  u16* dst = a.out + ((int64_t)seq * a.num_heads + head) * D + lane * PER_LANE;
  // One pass over context_lens (one load per 64 sequences, nothing else in flight before
  // it): this sequence's tiles, its first stream tile and the stream's total, i.e. what
  // seq_tiles, stream_locate and stream_chunk give.
  int nt = 0;
  int64_t first = 0, total = 0;
  for (int base = 0; base < a.num_seqs; base += 64) {
    const int q = base + lane;
    const int n = q < a.num_seqs ? seq_tiles(a, q) : 0;
    const int v = stream_slots(n);
    const int incl = wave_incl_scan(v, lane);
    if (seq >= base && seq < base + 64) {   // the sequence's tile count and first tile
      nt = __builtin_amdgcn_readlane(n, seq - base);
      first = total + __builtin_amdgcn_readlane(incl - v, seq - base) + kStreamPad;
    }
    total += __builtin_amdgcn_readlane(incl, 63);
  }
  if (nt == 0) {
    if constexpr (PER_LANE == 2)
      *reinterpret_cast<uint32_t*>(dst) = 0u;
    else
      dst[0] = 0;
    return;
  }
  const int64_t chunk = stream_chunk_of(a, total);
  const int64_t s0 = first / chunk, s1 = (first + nt - 1) / chunk;
  if (s0 == s1) return;
  const int nparts = (int)(s1 - s0 + 1);
  const int64_t slot0 = ((int64_t)kvh * a.nseg + s0 + seq) * a.group + hc;
  const int64_t ml_stride = 2 * (int64_t)a.group, acc_stride = (int64_t)a.group * D;
  const float* __restrict__ ml = a.ws_ml + slot0 * 2;
  const float* __restrict__ src = a.ws_acc + slot0 * D + lane * PER_LANE;

  // The first partials do not depend on the weights: load them with the (m, l) pairs.
  float pre[kMergePrefetch][PER_LANE];
#pragma unroll
  for (int u = 0; u < kMergePrefetch; ++u)
#pragma unroll
    for (int e = 0; e < PER_LANE; ++e) pre[u][e] = u < nparts ? src[u * acc_stride + e] : 0.f;

  // Part `lane`'s (m, l) pair (one 8-byte load) serves both passes below; parts from 64 on
  // (a sequence over more than 64 stream waves) are read again in the second.
  float m0 = kNegInf, l0 = 0.f;
  if (lane < nparts) {
    const float2 v = *reinterpret_cast<const float2*>(ml + lane * ml_stride);
    m0 = v.x;
    l0 = v.y;
  }
  float mx = m0;
  for (int p = lane + 64; p < nparts; p += 64) mx = fmaxf(mx, ml[p * ml_stride]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, xor_shfl(mx, o));
  float den = 0.f;
  if (lane < nparts) {
    const float w = (m0 == kNegInf || mx == kNegInf) ? 0.f : fast_exp2(m0 - mx);
    wsh[lane] = w;
    den += w * l0;
  }
  for (int p = lane + 64; p < nparts; p += 64) {
    const float mp = ml[p * ml_stride];
    const float w = (mp == kNegInf || mx == kNegInf) ? 0.f : fast_exp2(mp - mx);
    wsh[p] = w;
    den += w * ml[p * ml_stride + 1];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) den += xor_shfl(den, o);
  __syncthreads();

  float acc[PER_LANE];
#pragma unroll
  for (int e = 0; e < PER_LANE; ++e) acc[e] = 0.f;
#pragma unroll
  for (int u = 0; u < kMergePrefetch; ++u)
    if (u < nparts)
#pragma unroll
      for (int e = 0; e < PER_LANE; ++e) acc[e] += wsh[u] * pre[u][e];
  int p = kMergePrefetch;
  for (; p + 4 <= nparts; p += 4) {
    float v[4][PER_LANE];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < PER_LANE; ++e) v[u][e] = src[(p + u) * acc_stride + e];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < PER_LANE; ++e) acc[e] += wsh[p + u] * v[u][e];
  }
  for (; p < nparts; ++p)
#pragma unroll
    for (int e = 0; e < PER_LANE; ++e) acc[e] += wsh[p] * src[p * acc_stride + e];

  const float inv = den > 0.f ? 1.f / den : 0.f;
  if constexpr (PER_LANE == 2)
    *reinterpret_cast<uint32_t*>(dst) = Elt<F16>::pack(acc[0] * inv, acc[1] * inv);
  else
    dst[0] = Elt<F16>::one(acc[0] * inv);
}

// Blocks in flight per wave (2..4).  NDL_DECODE_DEPTH overrides the default for tuning.
inline int decode_pipeline_depth() {
  static const int depth = [] {
    const char* e = getenv("NDL_DECODE_DEPTH");
    const int d = e ? atoi(e) : 2;
    return (d >= 2 && d <= 4) ? d : 2;
  }();
  return depth;
}

// Resident waves of an attention kernel launched with `block` threads per workgroup on
// the current device (CUs times workgroups per CU times waves per workgroup); 0 when the
// device cannot be queried.
inline int64_t decode_resident_waves(const void* fn, int block = 64) {
  return resident_workgroups(fn, block) * (block / 64);
}

// APP: with the fused append (a separate instantiation, so that the attention-only kernel
// carries none of its registers).
// (The fp16 stream kernel is built at the default depth only.)
template <int D, bool APP = false, bool ROPE = false, bool F16 = false>
const void* decode_kernel_fn(int depth) {
  if constexpr (F16) {
    (void)depth;
    return (const void*)paged_decode_kernel<D, 2, 1, APP, ROPE, true>;
  } else {
    return depth == 2 ? (const void*)paged_decode_kernel<D, 2, 1, APP, ROPE>
                      : depth == 4 ? (const void*)paged_decode_kernel<D, 4, 1, APP, ROPE>
                                   : (const void*)paged_decode_kernel<D, 3, 1, APP, ROPE>;
  }
}
template <int D, bool APP = false, bool ROPE = false, bool F16 = false>
const void* seq_split_kernel_fn() {
  return (const void*)paged_decode_kernel<D, 2, seq_split_waves<D>(), APP, ROPE, F16>;
}

template <int D, bool F16>
inline const void* pick_decode_kernel_dt(bool app, bool rope, bool seq_split, int depth) {
  if (seq_split)
    return rope ? seq_split_kernel_fn<D, true, true, F16>()
                : app ? seq_split_kernel_fn<D, true, false, F16>()
                      : seq_split_kernel_fn<D, false, false, F16>();
  return rope ? decode_kernel_fn<D, true, true, F16>(depth)
              : app ? decode_kernel_fn<D, true, false, F16>(depth)
                    : decode_kernel_fn<D, false, false, F16>(depth);
}

// The attention kernel for one call: head_dim, element format, fused append, rotary form,
// split.
inline const void* pick_decode_kernel(int head_dim, bool f16, bool app, bool rope,
                                      bool seq_split, int depth) {
  if (head_dim == 128)
    return f16 ? pick_decode_kernel_dt<128, true>(app, rope, seq_split, depth)
               : pick_decode_kernel_dt<128, false>(app, rope, seq_split, depth);
  return f16 ? pick_decode_kernel_dt<64, true>(app, rope, seq_split, depth)
             : pick_decode_kernel_dt<64, false>(app, rope, seq_split, depth);
}

struct DecodeLayout {
  int seq_split;        // waves per (kv head, sequence) workgroup, or 0 for the stream split
  int64_t chunk;        // fixed stream slots per wave, or 0 (from the stream length on the device)
  int64_t waves;        // waves per kv head
  int64_t nseg;         // segment slots per kv head
  size_t ml_bytes;      // (m, l) region, 256-byte aligned
  size_t bytes;         // whole workspace
};

// Split of the work.  partition_tokens = -1: one workgroup of seq_split_waves() waves per
// (kv head, sequence).  partition_tokens > 0 (a multiple of 16): the stream split with
// that many tokens per wave.  0: the per-sequence workgroups when all of them are
// resident at once and a sequence of the full table width needs at most
// seq_split_max_tiles() tiles per wave; otherwise the stream split over as many waves as
// can be resident at once, shared by the kv heads, so that every wave that has tiles
// runs from the start (a device that cannot be queried counts as 2048 waves); each
// takes ceil(T / waves) tiles of its stream.
// max_tiles: 16-token tiles of a full table row (its width times block_size / 16).
inline int decode_layout(int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                         int64_t max_tiles, int partition_tokens, DecodeLayout* lay) {
  lay->seq_split = 0;
  const int nw = head_dim == 128 ? seq_split_waves<128>() : seq_split_waves<64>();
  if (partition_tokens == -1) {
    lay->seq_split = nw;
  } else if (partition_tokens < 0) {
    return NDL_ERR_INVALID_ARG;
  } else if (partition_tokens == 0) {
    int64_t resident = decode_resident_waves(
        head_dim == 128 ? seq_split_kernel_fn<128>() : seq_split_kernel_fn<64>(), 64 * nw);
    if (resident <= 0) resident = 2048;
    if ((int64_t)num_kv_heads * num_seqs * nw <= resident &&
        (max_tiles + nw - 1) / nw <=
            (head_dim == 128 ? seq_split_max_tiles<128>() : seq_split_max_tiles<64>()))
      lay->seq_split = nw;
  }
  if (lay->seq_split) {  // no partials leave the workgroup
    lay->chunk = 0;
    lay->waves = 1;
    lay->nseg = 0;
    lay->ml_bytes = 0;
    lay->bytes = 256;
    return NDL_OK;
  }
  if (partition_tokens > 0) {
    if (partition_tokens % 16 != 0) return NDL_ERR_INVALID_ARG;
    lay->chunk = partition_tokens / 16;
    // stream slots: every sequence's tiles and its kStreamPad empty slots
    lay->waves = ((int64_t)num_seqs * (max_tiles + kStreamPad) + lay->chunk - 1) / lay->chunk;
  } else {
    int64_t resident = decode_resident_waves(
        head_dim == 128 ? decode_kernel_fn<128>(decode_pipeline_depth())
                        : decode_kernel_fn<64>(decode_pipeline_depth()));
    if (resident <= 0) resident = 2048;
    int64_t w = resident / num_kv_heads;
    if (w < 1) w = 1;
    if (w > kMergeMaxParts - 2) w = kMergeMaxParts - 2;  // segments of one sequence
    lay->chunk = 0;
    lay->waves = w;
  }
  lay->nseg = lay->waves + num_seqs;
  const size_t slots = (size_t)num_kv_heads * lay->nseg * (num_heads / num_kv_heads);
  lay->ml_bytes = (slots * 2 * sizeof(float) + 255) & ~(size_t)255;
  lay->bytes = lay->ml_bytes + slots * head_dim * sizeof(float);
  return NDL_OK;
}

}  // namespace ndl

extern "C" size_t ndl_paged_decode_workspace_bytes(int num_seqs, int num_heads, int num_kv_heads,
                                                   int head_dim, int max_blocks_per_seq,
                                                   int block_size, int partition_tokens) {
  using namespace ndl;
  const int tshift = block_tile_shift(block_size);
  if (num_seqs <= 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0 ||
      head_dim <= 0 || max_blocks_per_seq <= 0 || tshift < 0)
    return 0;
  DecodeLayout lay;
  if (decode_layout(num_seqs, num_heads, num_kv_heads, head_dim,
                    (int64_t)max_blocks_per_seq << tshift, partition_tokens, &lay) != NDL_OK)
    return 0;
  return lay.bytes;
}

namespace ndl {

// Allocation-free decode (ndl_paged_decode_append_noalloc): the split-K partials go to a
// file-scope device array instead of a caller workspace.  Every GPU the library runs on
// holds its own copy of the array (at its own address) until the process ends.  The host
// name `scratch` is only a stand-in for the device symbol: kernels get the address that
// hipGetSymbolAddress returns for the current device, looked up once per device and kept.
// Nothing in the array needs to start at zero (the kernels write every partial they later
// read), so no call clears it.
constexpr size_t kStaticScratchBytes = NDL_DECODE_STATIC_SCRATCH_BYTES;
constexpr int kStaticScratchDevices = 64;

static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kStaticScratchDevices] = {};

// The device address of `scratch` on the current device (looked up on the first call per
// device, with that device current).  The lookup can load the code object, which allocates:
// refused while `stream` is being captured.
static int static_scratch_ptr(hipStream_t stream, void** ptr) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return NDL_ERR_LAUNCH;
  }
  if (dev < 0 || dev >= kStaticScratchDevices) return NDL_ERR_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus capturing = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capturing) != hipSuccess) {
      (void)hipGetLastError();
      return NDL_ERR_LAUNCH;
    }
    if (capturing != hipStreamCaptureStatusNone) return NDL_ERR_CAPTURE;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return NDL_ERR_LAUNCH;
    }
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return NDL_OK;
}

// static_scratch: ignore workspace/workspace_bytes and use the static array (after every
// argument check, so that a rejected call never touches the device).
static int launch_decode(void* out, const void* q, int64_t q_tok_stride, const void* kv_cache,
                         int64_t num_blocks, const int32_t* block_table, int64_t bt_row_stride,
                         int max_blocks_per_seq, const int32_t* context_lens, int num_seqs,
                         int num_heads, int num_kv_heads, int head_dim, int block_size, int dtype,
                         float scale, int partition_tokens, void* workspace,
                         size_t workspace_bytes, const void* k_new, int64_t k_new_stride,
                         const void* v_new, int64_t v_new_stride, ndl_stream_t stream,
                         bool static_scratch = false, const void* rope_cos = nullptr,
                         const void* rope_sin = nullptr, int64_t rope_stride = 0) {
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  const int tshift = block_tile_shift(block_size);
  if (tshift < 0 || (head_dim != 64 && head_dim != 128)) return NDL_ERR_UNSUPPORTED;
  if (num_kv_heads <= 0 || num_heads <= 0 || num_heads % num_kv_heads != 0)
    return NDL_ERR_INVALID_ARG;
  const int group = num_heads / num_kv_heads;
  const bool f16 = dtype_is_f16(dtype);
  if (group > 16) return NDL_ERR_UNSUPPORTED;
  if (num_seqs < 0 || num_blocks <= 0 || max_blocks_per_seq <= 0 ||
      bt_row_stride < max_blocks_per_seq || q_tok_stride < (int64_t)num_heads * head_dim)
    return NDL_ERR_INVALID_ARG;
  if (num_seqs == 0)  // nothing to do; the allocation-free form looks its array up
    return static_scratch ? static_scratch_ptr((hipStream_t)stream, &workspace) : NDL_OK;
  if (!out || !q || !kv_cache || !block_table || !context_lens) return NDL_ERR_INVALID_ARG;
  if (((uintptr_t)out | (uintptr_t)q | (uintptr_t)kv_cache) & 15u) return NDL_ERR_INVALID_ARG;
  if (q_tok_stride & 7) return NDL_ERR_INVALID_ARG;
  if (num_seqs > 65535) return NDL_ERR_UNSUPPORTED;
  if (dtype_is_f32(dtype)) {
    // One workgroup per (kv head, sequence) whatever the split asks for (the values are
    // checked as for the other formats); no partials, so neither workspace nor scratch.
    if (partition_tokens < -1 || (partition_tokens > 0 && partition_tokens % 16 != 0))
      return NDL_ERR_INVALID_ARG;
    return launch_decode_f32(out, q, q_tok_stride, k_new, k_new_stride, v_new, v_new_stride,
                             rope_cos, rope_sin, rope_stride, const_cast<void*>(kv_cache),
                             num_blocks, block_table, bt_row_stride, max_blocks_per_seq,
                             context_lens, num_seqs, num_heads, num_kv_heads, head_dim,
                             block_size, scale, stream);
  }
  DecodeLayout lay;
  const int64_t max_tiles = (int64_t)max_blocks_per_seq << tshift;
  if (max_tiles > 0x7fffffff) return NDL_ERR_UNSUPPORTED;
  const int rc0 = decode_layout(num_seqs, num_heads, num_kv_heads, head_dim, max_tiles,
                                partition_tokens, &lay);
  if (rc0 != NDL_OK) return rc0;
  // Segments one sequence can span: its tiles over the chunk, plus the partial ends
  // (the automatic split keeps waves <= kMergeMaxParts - 2).
  if (!lay.seq_split && lay.chunk > 0 && max_tiles / lay.chunk + 2 > kMergeMaxParts)
    return NDL_ERR_UNSUPPORTED;
  const int64_t grid_waves = lay.seq_split ? (int64_t)num_seqs * num_kv_heads
                                           : lay.waves * num_kv_heads;
  if (grid_waves > 0x7fffffff || lay.nseg > 0x7fffffff) return NDL_ERR_UNSUPPORTED;
  if (static_scratch) {
    if (lay.bytes > kStaticScratchBytes) return NDL_ERR_SCRATCH_LIMIT;
    const int rc = static_scratch_ptr((hipStream_t)stream, &workspace);
    if (rc != NDL_OK) return rc;
    workspace_bytes = kStaticScratchBytes;
  }
  if (workspace == nullptr || workspace_bytes < lay.bytes || ((uintptr_t)workspace & 15u))
    return NDL_ERR_WORKSPACE;

  DecodeArgs a;
  a.out = (u16*)out;
  a.q = (const u16*)q;
  a.q_tok_stride = q_tok_stride;
  a.kplane = (const u16*)kv_cache;
  a.vplane = a.kplane + num_blocks * num_kv_heads * (int64_t)block_size * head_dim;
  a.num_blocks = num_blocks;
  a.num_kv_heads = num_kv_heads;
  a.block_table = block_table;
  a.bt_row_stride = bt_row_stride;
  a.max_blocks = max_blocks_per_seq;
  a.tile_shift = tshift;
  a.context_lens = context_lens;
  a.num_heads = num_heads;
  a.group = group;
  a.scale_log2 = scale * kLog2e;
  a.num_seqs = num_seqs;
  a.chunk = (int)lay.chunk;
  a.waves = (int)lay.waves;
  a.nseg = (int)lay.nseg;
  a.ws_ml = (float*)workspace;
  a.ws_acc = (float*)((char*)workspace + lay.ml_bytes);
  a.k_new = (const u16*)k_new;
  a.v_new = (const u16*)v_new;
  a.k_new_stride = k_new_stride;
  a.v_new_stride = v_new_stride;
  a.rope_cos = (const u16*)rope_cos;
  a.rope_sin = (const u16*)rope_sin;
  a.rope_stride = rope_stride;

  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)grid_waves);
  const bool app = k_new != nullptr;
  const bool rope = rope_cos != nullptr;
  void* args[] = {&a};
  if (lay.seq_split) {  // one workgroup per (kv head, sequence), kv head fastest
    const void* fn = pick_decode_kernel(head_dim, f16, app, rope, true, 2);
    if (hipLaunchKernel(fn, grid, dim3(64 * lay.seq_split), args, 0, s) != hipSuccess) {
      (void)hipGetLastError();
      return NDL_ERR_LAUNCH;
    }
    return check_launch();
  }
  const void* fn = pick_decode_kernel(head_dim, f16, app, rope, false, decode_pipeline_depth());
  if (hipLaunchKernel(fn, grid, dim3(64), args, 0, s) != hipSuccess) {
    (void)hipGetLastError();
    return NDL_ERR_LAUNCH;
  }
  int rc = check_launch();
  if (rc != NDL_OK) return rc;
  const dim3 mgrid((unsigned)num_heads, (unsigned)num_seqs);
  if (head_dim == 128)
    hipLaunchKernelGGL((f16 ? paged_decode_merge_kernel<128, true>
                            : paged_decode_merge_kernel<128, false>), mgrid, dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL((f16 ? paged_decode_merge_kernel<64, true>
                            : paged_decode_merge_kernel<64, false>), mgrid, dim3(64), 0, s, a);
  return check_launch();
}

}  // namespace ndl

extern "C" int ndl_paged_decode(void* out, const void* q, int64_t q_tok_stride,
                                const void* kv_cache, int64_t num_blocks,
                                const int32_t* block_table, int64_t bt_row_stride,
                                int max_blocks_per_seq, const int32_t* context_lens, int num_seqs,
                                int num_heads, int num_kv_heads, int head_dim, int block_size,
                                int dtype, float scale, int partition_tokens, void* workspace,
                                size_t workspace_bytes, ndl_stream_t stream) {
  return ndl::launch_decode(out, q, q_tok_stride, kv_cache, num_blocks, block_table,
                            bt_row_stride, max_blocks_per_seq, context_lens, num_seqs, num_heads,
                            num_kv_heads, head_dim, block_size, dtype, scale, partition_tokens,
                            workspace, workspace_bytes, nullptr, 0, nullptr, 0, stream);
}

namespace ndl {

// The fused append's own argument checks, then the launch.
static int launch_decode_append(void* out, const void* q, int64_t q_tok_stride, const void* k,
                                int64_t k_tok_stride, const void* v, int64_t v_tok_stride,
                                void* kv_cache, int64_t num_blocks, const int32_t* block_table,
                                int64_t bt_row_stride, int max_blocks_per_seq,
                                const int32_t* context_lens, int num_seqs, int num_heads,
                                int num_kv_heads, int head_dim, int block_size, int dtype,
                                float scale, int partition_tokens, void* workspace,
                                size_t workspace_bytes, ndl_stream_t stream,
                                bool static_scratch, const void* rope_cos = nullptr,
                                const void* rope_sin = nullptr, int64_t rope_stride = 0) {
  if (num_seqs > 0) {
    if (!k || !v) return NDL_ERR_INVALID_ARG;
    if (rope_cos != nullptr || rope_sin != nullptr) {
      if (!rope_cos || !rope_sin || rope_stride < head_dim || (rope_stride & 7) ||
          (((uintptr_t)rope_cos | (uintptr_t)rope_sin) & 15u))
        return NDL_ERR_INVALID_ARG;
    }
    if (((uintptr_t)k | (uintptr_t)v) & 15u) return NDL_ERR_INVALID_ARG;
    if (k_tok_stride < (int64_t)num_kv_heads * head_dim ||
        v_tok_stride < (int64_t)num_kv_heads * head_dim || ((k_tok_stride | v_tok_stride) & 7))
      return NDL_ERR_INVALID_ARG;
  }
  return launch_decode(out, q, q_tok_stride, kv_cache, num_blocks, block_table, bt_row_stride,
                       max_blocks_per_seq, context_lens, num_seqs, num_heads, num_kv_heads,
                       head_dim, block_size, dtype, scale, partition_tokens, workspace,
                       workspace_bytes, k, k_tok_stride, v, v_tok_stride, stream,
                       static_scratch, rope_cos, rope_sin, rope_stride);
}

}  // namespace ndl

extern "C" int ndl_paged_decode_append(void* out, const void* q, int64_t q_tok_stride,
                                       const void* k, int64_t k_tok_stride, const void* v,
                                       int64_t v_tok_stride, void* kv_cache, int64_t num_blocks,
                                       const int32_t* block_table, int64_t bt_row_stride,
                                       int max_blocks_per_seq, const int32_t* context_lens,
                                       int num_seqs, int num_heads, int num_kv_heads, int head_dim,
                                       int block_size, int dtype, float scale,
                                       int partition_tokens, void* workspace,
                                       size_t workspace_bytes, ndl_stream_t stream) {
  return ndl::launch_decode_append(out, q, q_tok_stride, k, k_tok_stride, v, v_tok_stride,
                                   kv_cache, num_blocks, block_table, bt_row_stride,
                                   max_blocks_per_seq, context_lens, num_seqs, num_heads,
                                   num_kv_heads, head_dim, block_size, dtype, scale,
                                   partition_tokens, workspace, workspace_bytes, stream, false);
}

// Allocation-free form: the partials live in the static array `scratch` (see above).
extern "C" int ndl_paged_decode_append_noalloc(
    void* out, const void* q, int64_t q_tok_stride, const void* k, int64_t k_tok_stride,
    const void* v, int64_t v_tok_stride, void* kv_cache, int64_t num_blocks,
    const int32_t* block_table, int64_t bt_row_stride, int max_blocks_per_seq,
    const int32_t* context_lens, int num_seqs, int num_heads, int num_kv_heads, int head_dim,
    int block_size, int dtype, float scale, int partition_tokens, ndl_stream_t stream) {
  return ndl::launch_decode_append(out, q, q_tok_stride, k, k_tok_stride, v, v_tok_stride,
                                   kv_cache, num_blocks, block_table, bt_row_stride,
                                   max_blocks_per_seq, context_lens, num_seqs, num_heads,
                                   num_kv_heads, head_dim, block_size, dtype, scale,
                                   partition_tokens, nullptr, 0, stream, true);
}

// RoPE of q and the new key row folded into the fused decode (see above).
extern "C" int ndl_rope_paged_decode_append(
    void* out, const void* q, int64_t q_tok_stride, const void* k, int64_t k_tok_stride,
    const void* v, int64_t v_tok_stride, const void* cos, const void* sin,
    int64_t cs_tok_stride, void* kv_cache, int64_t num_blocks, const int32_t* block_table,
    int64_t bt_row_stride, int max_blocks_per_seq, const int32_t* context_lens, int num_seqs,
    int num_heads, int num_kv_heads, int head_dim, int block_size, int dtype, float scale,
    int partition_tokens, void* workspace, size_t workspace_bytes, ndl_stream_t stream) {
  if (num_seqs > 0 && (cos == nullptr || sin == nullptr)) return NDL_ERR_INVALID_ARG;
  return ndl::launch_decode_append(out, q, q_tok_stride, k, k_tok_stride, v, v_tok_stride,
                                   kv_cache, num_blocks, block_table, bt_row_stride,
                                   max_blocks_per_seq, context_lens, num_seqs, num_heads,
                                   num_kv_heads, head_dim, block_size, dtype, scale,
                                   partition_tokens, workspace, workspace_bytes, stream, false,
                                   cos, sin, cs_tok_stride);
}
