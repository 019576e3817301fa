// The decoder layer's elementwise work around the attention, for gfx950.
//
// Reference: needle/model/qwen2.py:52-65 (Qwen2DecoderLayer.forward: residual adds around
// the attention and the MLP, an RMSNorm before each), needle/layers/norm.py:14-17 (RMSNorm),
// needle/model/llama.py:36-37 (LlamaMLP: silu(gate) * up).
//
// The reference runs these as torch ops, one kernel each: the residual add, the RMSNorm's
// fp32 statistic, reciprocal square root, products and casts, the weight product, the SiLU
// and the product with up.  Here the residual add, the RMSNorm and its weight product are one
// kernel, and SiLU(gate) * up another, each keeping the reference's roundings:
//   h   = round(x + residual)                                  (qwen2.py:58, :63)
//   var = (sum_i float(h_i)^2) * (1 / hidden)                   (norm.py:15, torch's mean)
//   y   = round(float(h) * rsqrt(var + eps))                    (norm.py:16, cast to the dtype)
//   out = round(float(weight) * float(y))                       (norm.py:17)
//   act = round(round(silu(g)) * u), silu(g) = g / (1 + exp(-g)) (llama.py:37, torch's silu)
// round() is the model dtype's round-to-nearest-even (identity for float32).  Only the order
// of the sum of squares differs from torch's reduction, which can move the statistic by an
// ulp and an element of the output by an ulp of its format now and then.
//
// Both kernels are latency-bound at decode sizes (one row per wave, tens of rows) and
// HBM-bound at prefill sizes: every element is read and written once.
#include "ndl_common.hpp"

namespace ndl {
namespace {

constexpr int kThreads = 256;           // four waves
constexpr int kMaxHidden = 8192;        // 16 chunks of 8 elements per lane

// Eight consecutive elements of a row as fp32 (16 bytes of a 16-bit format, 32 of float32).
template <int FMT>
__device__ __forceinline__ void load8(const void* p, float (&v)[8]) {
  if constexpr (FMT == kFmtF32) {
    const u32x4 a = ld16(p), b = ld16(static_cast<const char*>(p) + 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = __uint_as_float(a[i]);
      v[4 + i] = __uint_as_float(b[i]);
    }
  } else {
    using T = Elt<FMT == kFmtF16>;
    const u32x4 w = ld16(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = T::lo(w[i]);
      v[2 * i + 1] = T::hi(w[i]);
    }
  }
}

// v, already representable in the format, stored as eight elements.
template <int FMT>
__device__ __forceinline__ void store8(void* p, const float (&v)[8]) {
  if constexpr (FMT == kFmtF32) {
    st16(p, u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                  __float_as_uint(v[3])});
    st16(static_cast<char*>(p) + 16, u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]),
                                            __float_as_uint(v[6]), __float_as_uint(v[7])});
  } else {
    using T = Elt<FMT == kFmtF16>;
    st16(p, u32x4{T::pack(v[0], v[1]), T::pack(v[2], v[3]), T::pack(v[4], v[5]),
                  T::pack(v[6], v[7])});
  }
}

// x rounded to the format (round to nearest even), as fp32.
template <int FMT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (FMT == kFmtF32) {
    return x;
  } else {
    using T = Elt<FMT == kFmtF16>;
    return T::lo(T::pack(x, 0.f));
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += xor_shfl(v, m);
  return v;
}

struct NormArgs {
  void* out;                // [rows][hidden]
  void* residual_out;       // [rows][hidden]: x + residual (may be residual itself)
  const void* x;            // [rows] rows of hidden elements, row stride x_stride
  const void* residual;     // [rows][hidden], or null
  const void* weight;       // [hidden]
  int64_t rows, x_stride;   // x_stride in elements
  int hidden;
  float eps, inv_hidden;
};

// One wave per row; lane l holds chunks l, l + 64, .. (8 elements each) of the row, and the
// same chunks of the weight (loaded with the row: one memory round trip), in registers
// between the statistic and the products.
template <int FMT, int NC, bool RES>
__global__ __launch_bounds__(kThreads) void rms_norm_kernel(NormArgs a) {
  constexpr int EB = FMT == kFmtF32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int chunks = a.hidden / 8;
  const char* x = static_cast<const char*>(a.x) + row * a.x_stride * EB;
  const int64_t row_off = row * a.hidden * EB;
  float h[NC][8], w[NC][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= chunks) continue;
    load8<FMT>(x + ch * 8 * EB, h[c]);
    load8<FMT>(static_cast<const char*>(a.weight) + ch * 8 * EB, w[c]);
    if constexpr (RES) {
      float r[8];
      load8<FMT>(static_cast<const char*>(a.residual) + row_off + ch * 8 * EB, r);
#pragma unroll
      for (int e = 0; e < 8; ++e) h[c][e] = round_to<FMT>(__fadd_rn(h[c][e], r[e]));
      store8<FMT>(static_cast<char*>(a.residual_out) + row_off + ch * 8 * EB, h[c]);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __fadd_rn(ss, __fmul_rn(h[c][e], h[c][e]));
  }
  const float var = __fmul_rn(wave_sum(ss), a.inv_hidden);
  const float rstd = rsqrtf(__fadd_rn(var, a.eps));
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= chunks) continue;
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = round_to<FMT>(__fmul_rn(w[c][e], round_to<FMT>(__fmul_rn(h[c][e], rstd))));
    store8<FMT>(static_cast<char*>(a.out) + row_off + ch * 8 * EB, o);
  }
}

struct SiluArgs {
  void* out;                          // [rows][inter]
  const void* gate;                   // row stride gate_stride (elements)
  const void* up;                     // row stride up_stride
  int64_t rows, gate_stride, up_stride;
  int inter;
};

// One thread per 8 elements of a row.
template <int FMT>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(SiluArgs a) {
  constexpr int EB = FMT == kFmtF32 ? 4 : 2;
  const int cpr = a.inter / 8;
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  const int64_t row = idx / cpr;
  if (row >= a.rows) return;
  const int ch = (int)(idx - row * cpr);
  float g[8], u[8], o[8];
  load8<FMT>(static_cast<const char*>(a.gate) + (row * a.gate_stride + ch * 8) * EB, g);
  load8<FMT>(static_cast<const char*>(a.up) + (row * a.up_stride + ch * 8) * EB, u);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float s = round_to<FMT>(g[e] / __fadd_rn(1.f, expf(-g[e])));
    o[e] = round_to<FMT>(__fmul_rn(s, u[e]));
  }
  store8<FMT>(static_cast<char*>(a.out) + (row * a.inter + ch * 8) * EB, o);
}

template <int FMT, bool RES>
int launch_norm(const NormArgs& a, hipStream_t stream) {
  const int nc = (a.hidden / 8 + 63) / 64;
  const dim3 grid((unsigned)((a.rows + kThreads / 64 - 1) / (kThreads / 64)));
  if (nc <= 1)
    hipLaunchKernelGGL((rms_norm_kernel<FMT, 1, RES>), grid, dim3(kThreads), 0, stream, a);
  else if (nc <= 2)
    hipLaunchKernelGGL((rms_norm_kernel<FMT, 2, RES>), grid, dim3(kThreads), 0, stream, a);
  else if (nc <= 4)
    hipLaunchKernelGGL((rms_norm_kernel<FMT, 4, RES>), grid, dim3(kThreads), 0, stream, a);
  else if (nc <= 8)
    hipLaunchKernelGGL((rms_norm_kernel<FMT, 8, RES>), grid, dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((rms_norm_kernel<FMT, 16, RES>), grid, dim3(kThreads), 0, stream, a);
  return check_launch();
}

template <int FMT>
int launch_norm_fmt(const NormArgs& a, hipStream_t stream) {
  return a.residual != nullptr ? launch_norm<FMT, true>(a, stream)
                               : launch_norm<FMT, false>(a, stream);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace ndl

extern "C" int ndl_rms_norm(void* out, void* residual_out, const void* x, int64_t x_row_stride,
                            const void* residual, const void* weight, int64_t rows, int hidden,
                            float eps, int dtype, ndl_stream_t stream) {
  using namespace ndl;
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  if (rows < 0 || hidden <= 0) return NDL_ERR_INVALID_ARG;
  if (hidden % 8 != 0 || hidden > kMaxHidden) return NDL_ERR_UNSUPPORTED;
  if (rows == 0) return NDL_OK;
  if (!out || !x || !weight || (residual && !residual_out)) return NDL_ERR_INVALID_ARG;
  if (x_row_stride < hidden || x_row_stride % 8 != 0) return NDL_ERR_INVALID_ARG;
  if (!aligned16(out) || !aligned16(x) || !aligned16(weight) ||
      (residual && (!aligned16(residual) || !aligned16(residual_out))))
    return NDL_ERR_INVALID_ARG;
  if ((rows + 3) / 4 > 0x7fffffff) return NDL_ERR_UNSUPPORTED;
  NormArgs a;
  a.out = out;
  a.residual_out = residual ? residual_out : nullptr;
  a.x = x;
  a.residual = residual;
  a.weight = weight;
  a.rows = rows;
  a.x_stride = x_row_stride;
  a.hidden = hidden;
  a.eps = eps;
  a.inv_hidden = 1.f / (float)hidden;
  const hipStream_t s = (hipStream_t)stream;
  if (dtype_is_f32(dtype)) return launch_norm_fmt<kFmtF32>(a, s);
  if (dtype_is_f16(dtype)) return launch_norm_fmt<kFmtF16>(a, s);
  return launch_norm_fmt<kFmtBF16>(a, s);
}

extern "C" int ndl_silu_mul(void* out, const void* gate, int64_t gate_row_stride,
                            const void* up, int64_t up_row_stride, int64_t rows,
                            int intermediate, int dtype, ndl_stream_t stream) {
  using namespace ndl;
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  if (rows < 0 || intermediate <= 0) return NDL_ERR_INVALID_ARG;
  if (intermediate % 8 != 0) return NDL_ERR_UNSUPPORTED;
  if (rows == 0) return NDL_OK;
  if (!out || !gate || !up) return NDL_ERR_INVALID_ARG;
  if (gate_row_stride < intermediate || up_row_stride < intermediate ||
      gate_row_stride % 8 != 0 || up_row_stride % 8 != 0)
    return NDL_ERR_INVALID_ARG;
  if (!aligned16(out) || !aligned16(gate) || !aligned16(up)) return NDL_ERR_INVALID_ARG;
  const int64_t items = rows * (intermediate / 8);
  const int64_t blocks = (items + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return NDL_ERR_UNSUPPORTED;
  SiluArgs a;
  a.out = out;
  a.gate = gate;
  a.up = up;
  a.rows = rows;
  a.gate_stride = gate_row_stride;
  a.up_stride = up_row_stride;
  a.inter = intermediate;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks);
  if (dtype_is_f32(dtype))
    hipLaunchKernelGGL((silu_mul_kernel<kFmtF32>), grid, dim3(kThreads), 0, s, a);
  else if (dtype_is_f16(dtype))
    hipLaunchKernelGGL((silu_mul_kernel<kFmtF16>), grid, dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL((silu_mul_kernel<kFmtBF16>), grid, dim3(kThreads), 0, s, a);
  return check_launch();
}
