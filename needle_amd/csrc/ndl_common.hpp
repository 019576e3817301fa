// Shared device helpers for the gfx950 paged-KV kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "../../include/needle_amd.h"

namespace ndl {

// 16-bit payloads are moved as raw bits; arithmetic converts to fp32.
using u16 = uint16_t;

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) short i16x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// fp32 pair -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// fp32 -> bf16 bits (low half), round-to-nearest-even.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return pack_bf16x2(f, 0.f) & 0xffffu;
}

// Pack the low (sel_hi = false) or high halves of two words: {lo.half, hi.half}.
__device__ __forceinline__ uint32_t pack_halves(uint32_t lo, uint32_t hi, bool high_half) {
  return __builtin_amdgcn_perm(hi, lo, high_half ? 0x07060302u : 0x05040100u);
}

typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

// The 16-bit element format of the pools and activations: bfloat16 (Elt<false>) or
// float16 (Elt<true>), the model dtypes the reference runs its attention in
// (needle/args.py:80-84).  Elements are moved as raw bits; these are the only places the
// format matters: conversions (fp32 <-> 16 bits, round to nearest even) and the MFMA
// instructions.
template <bool kF16> struct Elt;
template <> struct Elt<false> {
  using x8 = bf16x8;                                   // 8-element MFMA operand
  static __device__ __forceinline__ float lo(uint32_t w) { return bf16_lo(w); }
  static __device__ __forceinline__ float hi(uint32_t w) { return bf16_hi(w); }
  static __device__ __forceinline__ uint32_t pack(float a, float b) { return pack_bf16x2(a, b); }
  static __device__ __forceinline__ u16 one(float a) { return (u16)f32_to_bf16_bits(a); }
  static __device__ __forceinline__ f32x16 mfma32x32x16(x8 a, x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16x16x32(x8 a, x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // 4-element operands given as two words each
  static __device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                     __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
  }
};
template <> struct Elt<true> {
  using x8 = f16x8;
  static __device__ __forceinline__ float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (u16)(w & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (u16)(w >> 16));
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
  }
  static __device__ __forceinline__ u16 one(float a) {
    return __builtin_bit_cast(u16, (_Float16)a);
  }
  static __device__ __forceinline__ f32x16 mfma32x32x16(x8 a, x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16x16x32(x8 a, x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a),
                                                 __builtin_bit_cast(f16x4, b), c, 0, 0, 0);
  }
};

// Rotary embedding with the reference's rounding (attention.py:277-288, op for op in the
// model dtype):
//   out[d] = r( r(x[d] * cos[d]) + r(rot(x)[d] * sin[d]) ),
//   rot(x)[d] = -x[d + D/2] (d < D/2), x[d - D/2] (d >= D/2);
// every product and the sum are formed in fp32 from 16-bit operands and rounded (r) to the
// element format, nearest even, as torch does for bf16 and fp16 tensors.
// 8 elements of x[d..d+8) and x[d+D/2..d+D/2+8) -> rotated halves.  The two elements of a
// word are rounded together (one packing conversion per pair of products, each half rounded
// to nearest even on its own, exactly as two single roundings).
// Contraction stays off: the fp32 product of two fp16 values is exact, so the compiler may
// narrow product-then-round to an fp16 multiply, and with contraction on it would then fuse
// that multiply into the sum (v_pk_fma_f16), skipping the product's rounding.
template <bool kF16 = false>
__device__ __forceinline__ void rope8(const u32x4& lo, const u32x4& hi, const u32x4& clo,
                                      const u32x4& chi, const u32x4& slo, const u32x4& shi,
                                      u32x4& out_lo, u32x4& out_hi) {
#pragma clang fp contract(off)
  using T = Elt<kF16>;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float xl0 = T::lo(lo[w]), xl1 = T::hi(lo[w]);
    const float xh0 = T::lo(hi[w]), xh1 = T::hi(hi[w]);
    // -x_hi by its sign bits (exact, as the 16-bit negation of rotate_half)
    const uint32_t nh = hi[w] ^ 0x80008000u;
    // first half: x*cos + (-x_hi)*sin ; second half: x_hi*cos + x*sin
    const uint32_t p_xc = T::pack(xl0 * T::lo(clo[w]), xl1 * T::hi(clo[w]));
    const uint32_t p_rs = T::pack(T::lo(nh) * T::lo(slo[w]), T::hi(nh) * T::hi(slo[w]));
    const uint32_t p_hc = T::pack(xh0 * T::lo(chi[w]), xh1 * T::hi(chi[w]));
    const uint32_t p_ls = T::pack(xl0 * T::lo(shi[w]), xl1 * T::hi(shi[w]));
    out_lo[w] = T::pack(T::lo(p_xc) + T::lo(p_rs), T::hi(p_xc) + T::hi(p_rs));
    out_hi[w] = T::pack(T::lo(p_hc) + T::lo(p_ls), T::hi(p_hc) + T::hi(p_ls));
  }
}

// The same rotation in float32 (the reference's --dtype float32): 4 elements of each half
// per 16 bytes, every product and the sum rounded to fp32 (contraction off: the reference's
// x * cos + rotate_half(x) * sin is two multiplies and an add).
__device__ __forceinline__ void rope4_f32(const u32x4& lo, const u32x4& hi, const u32x4& clo,
                                          const u32x4& chi, const u32x4& slo, const u32x4& shi,
                                          u32x4& out_lo, u32x4& out_hi) {
#pragma clang fp contract(off)
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float xl = __uint_as_float(lo[w]), xh = __uint_as_float(hi[w]);
    const float nxh = __uint_as_float(hi[w] ^ 0x80000000u);   // -x_hi, exact
    out_lo[w] = __float_as_uint(xl * __uint_as_float(clo[w]) + nxh * __uint_as_float(slo[w]));
    out_hi[w] = __float_as_uint(xh * __uint_as_float(chi[w]) + xl * __uint_as_float(shi[w]));
  }
}

// Element formats on the device: the ABI dtype codes (NDL_DTYPE_*).
enum Fmt { kFmtBF16 = 0, kFmtF16 = 1, kFmtF32 = 2 };

// The rotation of 16 bytes of each half in format FMT (8 16-bit or 4 fp32 elements).
template <int FMT>
__device__ __forceinline__ void rope16(const u32x4& lo, const u32x4& hi, const u32x4& clo,
                                       const u32x4& chi, const u32x4& slo, const u32x4& shi,
                                       u32x4& out_lo, u32x4& out_hi) {
  if constexpr (FMT == kFmtF32)
    rope4_f32(lo, hi, clo, chi, slo, shi, out_lo, out_hi);
  else
    rope8<FMT == kFmtF16>(lo, hi, clo, chi, slo, shi, out_lo, out_hi);
}

// Block sizes the attention kernels take: powers of two from 16 to 1024 tokens, each block
// read as 16-token tiles.  log2(block_size / 16), or -1 for any other size.
constexpr int kMaxBlockSize = 1024;
inline int block_tile_shift(int block_size) {
  if (block_size < 16 || block_size > kMaxBlockSize || (block_size & (block_size - 1)))
    return -1;
  int s = 0;
  while ((16 << s) < block_size) ++s;
  return s;
}

// The element format of an ABI dtype code (false: bf16, true: fp16); false for others.
inline bool dtype_is_f16(int dtype) { return dtype == NDL_DTYPE_F16; }
inline bool dtype_is_f32(int dtype) { return dtype == NDL_DTYPE_F32; }
// The 16-bit formats (the MFMA kernels' element formats).
inline bool dtype_supported(int dtype) {
  return dtype == NDL_DTYPE_BF16 || dtype == NDL_DTYPE_F16;
}
// Any format the library takes.
inline bool dtype_known(int dtype) { return dtype_supported(dtype) || dtype == NDL_DTYPE_F32; }
// Bytes per element.
inline int dtype_bytes(int dtype) { return dtype == NDL_DTYPE_F32 ? 4 : 2; }

// exp2 on the hardware transcendental unit (v_exp_f32).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Butterfly exchange across lanes (lane ^ mask) inside a wave64 (ds_bpermute).
__device__ __forceinline__ float xor_shfl(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// v[l] op v[l ^ 16] and v[l] op v[l ^ 32] on the VALU: v_permlane16_swap / v_permlane32_swap
// of a register with itself returns, in every lane, the pair's value of the lower row (or
// half) in one result and of the upper one in the other, so both lanes of a pair combine
// the same two values in the same order (no LDS crossbar round trip).
__device__ __forceinline__ float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ u32x4 ldg16(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x2 ld8(const void* p) {
  return *reinterpret_cast<const u32x2*>(p);
}
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

inline int check_launch() {
  return hipGetLastError() == hipSuccess ? NDL_OK : NDL_ERR_LAUNCH;
}

// Workgroups of `fn`, launched with `block` threads, that can be resident at once on the
// current device (CUs times workgroups per CU); 0 when the device cannot be queried.  The
// answer is cached per (kernel, block size, device) under a lock: the entry points may be
// called from several host threads at once.
inline int64_t resident_workgroups(const void* fn, int block) {
  struct Entry { const void* fn; int block; int dev; int64_t wgs; };
  static std::mutex mu;
  static Entry cache[64];
  static int used = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i)
      if (cache[i].fn == fn && cache[i].block == block && cache[i].dev == dev)
        return cache[i].wgs;
  }
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, block, 0) != hipSuccess ||
      cus <= 0 || per_cu <= 0)
    return 0;
  const int64_t wgs = (int64_t)cus * per_cu;
  std::lock_guard<std::mutex> lock(mu);
  if (used < 64) cache[used++] = Entry{fn, block, dev, wgs};
  return wgs;
}

// The append launcher of kv_append.hip (rope_cos != nullptr: k rotated in format fmt, a
// Fmt; head_dim and strides in elements of that format).
int launch_kv_append(void* kv_cache, int64_t num_blocks, int num_kv_heads, int block_size,
                     int head_dim, const void* k, int64_t k_tok_stride, const void* v,
                     int64_t v_tok_stride, const int32_t* block_table, int64_t bt_row_stride,
                     int max_blocks_per_seq, const int32_t* cu_seqlens,
                     const int32_t* context_lens, int num_seqs, int64_t num_tokens,
                     const void* rope_cos, const void* rope_sin, int64_t rope_stride,
                     int fmt, ndl_stream_t stream);

// The float32 attention launchers (paged_decode_f32.hip, varlen_prefill_f32.hip); the entry
// points check the arguments common to all formats first.  k_new/v_new non-null: the step's
// rows are appended first (by ndl_kv_append's kernel); cos/sin non-null: q (and k_new) are
// rotated.
int launch_decode_f32(void* out, const void* q, int64_t q_tok_stride, const void* k_new,
                      int64_t k_tok_stride, const void* v_new, int64_t v_tok_stride,
                      const void* cos, const void* sin, int64_t cs_tok_stride, void* kv_cache,
                      int64_t num_blocks, const int32_t* block_table, int64_t bt_row_stride,
                      int max_blocks_per_seq, const int32_t* context_lens, int num_seqs,
                      int num_heads, int num_kv_heads, int head_dim, int block_size, float scale,
                      ndl_stream_t stream);
int launch_prefill_f32(void* out, const void* q, int64_t q_tok_stride, const void* cos,
                       const void* sin, int64_t cs_tok_stride, const void* kv_cache,
                       int64_t num_blocks, const int32_t* block_table, int64_t bt_row_stride,
                       int max_blocks_per_seq, const int32_t* cu_seqlens,
                       const int32_t* context_lens, int num_seqs, int64_t num_tokens,
                       int max_seqlen, int max_context_len, int num_heads, int num_kv_heads,
                       int head_dim, int block_size, float scale, ndl_stream_t stream);

}  // namespace ndl
