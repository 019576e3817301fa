// Greedy sampling of a batch of logit rows on gfx950: the index of each row's maximum.
//
// Reference: needle/model/sampler.py:27-28 (a greedy row: int(logit.argmax()), one row and
// one host sync at a time), called once per step from needle/model/runner.py:156.  Here one
// launch covers the batch.
//
// The index is torch's argmax's: a NaN counts as larger than every number (the first NaN
// wins), and of equal maxima the lowest index wins (-0 and +0 are equal).  One workgroup per
// row: each thread scans 8-element chunks t, t + T, .. in increasing index order keeping
// its best (value, index), then the waves and the workgroup reduce the pairs with the same
// order.  No memset, no atomics: the launch can be recorded in a HIP graph and writes the
// next step's input tokens directly.  Bound by reading the row once (a 151,936-entry bf16
// vocabulary row is 297 KiB per workgroup).
#include "ndl_common.hpp"

namespace ndl {
namespace {

constexpr int kArgThreads = 1024;

struct ArgmaxArgs {
  const void* logits;    // rows of `vocab` elements, row stride `stride`
  void* out;             // int32 or int64 [rows]
  int64_t rows, stride;
  int vocab;
  int out64;
};

// (va, ia) comes before (vb, ib) in torch's argmax order.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  const bool na = va != va, nb = vb != vb;
  if (na || nb) return na && (!nb || ia < ib);
  return va > vb || (va == vb && ia < ib);
}

template <int FMT>
__device__ __forceinline__ float elem(const char* row, int i) {
  if constexpr (FMT == kFmtF32) {
    return reinterpret_cast<const float*>(row)[i];
  } else {
    using T = Elt<FMT == kFmtF16>;
    return T::lo(reinterpret_cast<const u16*>(row)[i]);
  }
}

template <int FMT>
__global__ __launch_bounds__(kArgThreads) void greedy_argmax_kernel(ArgmaxArgs a) {
  constexpr int EB = FMT == kFmtF32 ? 4 : 2;
  const int64_t r = blockIdx.x;
  const char* row = static_cast<const char*>(a.logits) + r * a.stride * EB;
  float bv = kNegInf;
  int bi = 0x7fffffff;
  const int chunks = a.vocab / 8;
  // kBatch chunks per thread are loaded before any is compared, so that many loads are in
  // flight at once; a chunk past the row is not loaded and not compared.
  constexpr int kBatch = FMT == kFmtF32 ? 4 : 8;
  constexpr int CW = FMT == kFmtF32 ? 2 : 1;   // 16-byte words per chunk
  for (int ch0 = threadIdx.x; ch0 < chunks; ch0 += kBatch * kArgThreads) {
    u32x4 p[kBatch][CW];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int ch = ch0 + u * kArgThreads;
#pragma unroll
      for (int w = 0; w < CW; ++w)
        p[u][w] = ch < chunks ? ld16(row + (ch * CW + w) * 16) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int ch = ch0 + u * kArgThreads;
      if (ch >= chunks) break;
      float v[8];
      if constexpr (FMT == kFmtF32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[e] = __uint_as_float(p[u][0][e]);
          v[4 + e] = __uint_as_float(p[u][1][e]);
        }
      } else {
        using T = Elt<FMT == kFmtF16>;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = T::lo(p[u][0][e]);
          v[2 * e + 1] = T::hi(p[u][0][e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (better(v[e], 8 * ch + e, bv, bi)) {
          bv = v[e];
          bi = 8 * ch + e;
        }
    }
  }
  // the vocab % 8 last entries
  for (int i = 8 * chunks + (int)threadIdx.x; i < a.vocab; i += kArgThreads) {
    const float v = elem<FMT>(row, i);
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __shared__ float sv[kArgThreads / 64];
  __shared__ int si[kArgThreads / 64];
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wv] = bv;
    si[wv] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgThreads / 64; ++w)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    if (a.out64)
      static_cast<int64_t*>(a.out)[r] = bi;
    else
      static_cast<int32_t*>(a.out)[r] = bi;
  }
}

}  // namespace
}  // namespace ndl

extern "C" int ndl_greedy_argmax(void* out, int out_is_int64, const void* logits,
                                 int64_t row_stride, int64_t rows, int vocab, int dtype,
                                 ndl_stream_t stream) {
  using namespace ndl;
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  if (rows < 0 || vocab <= 0) return NDL_ERR_INVALID_ARG;
  if (rows == 0) return NDL_OK;
  if (!out || !logits) return NDL_ERR_INVALID_ARG;
  if (row_stride < vocab || row_stride % 8 != 0 || ((uintptr_t)logits & 15u))
    return NDL_ERR_INVALID_ARG;
  if (rows > 0x7fffffff) return NDL_ERR_UNSUPPORTED;
  ArgmaxArgs a;
  a.logits = logits;
  a.out = out;
  a.rows = rows;
  a.stride = row_stride;
  a.vocab = vocab;
  a.out64 = out_is_int64 ? 1 : 0;
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)rows);
  if (dtype_is_f32(dtype))
    hipLaunchKernelGGL((greedy_argmax_kernel<kFmtF32>), grid, dim3(kArgThreads), 0, s, a);
  else if (dtype_is_f16(dtype))
    hipLaunchKernelGGL((greedy_argmax_kernel<kFmtF16>), grid, dim3(kArgThreads), 0, s, a);
  else
    hipLaunchKernelGGL((greedy_argmax_kernel<kFmtBF16>), grid, dim3(kArgThreads), 0, s, a);
  return check_launch();
}
