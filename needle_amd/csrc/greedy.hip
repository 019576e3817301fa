// Greedy sampling of a batch of logit rows on gfx950: the index of each row's maximum.
//
// Reference: needle/model/sampler.py:27-28 (a greedy row: int(logit.argmax()), one row and
// one host sync at a time), called once per step from needle/model/runner.py:156.  Here one
// launch covers the batch.
//
// The index is torch's argmax's: a NaN counts as larger than every number (the first NaN
// wins), and of equal maxima the lowest index wins (-0 and +0 are equal).  Each row is cut
// into slices of at least 8,192 entries, enough of them for the batch to cover the GPU
// (about 512 workgroups in all): a workgroup finds its slice's best entry, each thread
// scanning 8-element chunks in increasing index order with 8 loads in flight, and a second,
// one-wave-per-row kernel takes the best of the row's slices in the same order (a single
// slice per row writes the index at once).  The partials go to a caller-provided workspace;
// no memset, no atomics, so the launches can be recorded in a HIP graph.  Bound by reading
// every logit once: a batch of 16 rows of a 151,936-entry bf16 vocabulary is 4.9 MB.
#include "ndl_common.hpp"

namespace ndl {
namespace {

constexpr int kArgThreads = 256;
constexpr int kArgMinSlice = 8192;    // elements a slice scans at least
constexpr int kArgTargetWgs = 512;    // slices over all rows, about two per CU

struct ArgmaxArgs {
  const void* logits;    // rows of `vocab` elements, row stride `stride`
  void* out;             // int32 or int64 [rows]
  float* part_v;         // [rows][slices]: each slice's best value and index
  int* part_i;
  int64_t rows, stride;
  int vocab, slices, slice_len;   // slice_len: a multiple of 8
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

__device__ __forceinline__ void wave_best(float& bv, int& bi) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
}

__device__ __forceinline__ void write_index(const ArgmaxArgs& a, int64_t r, int bi) {
  if (a.out64)
    static_cast<int64_t*>(a.out)[r] = bi;
  else
    static_cast<int32_t*>(a.out)[r] = bi;
}

// Workgroup (slice s, row r): the best entry of elements s * slice_len .. of row r, written
// to the partials (or, with one slice per row, as the row's index).  Each thread scans
// 8-element chunks t, t + T, .. of the slice in increasing index order, kBatch chunk loads
// in flight before any is compared.
template <int FMT>
__global__ __launch_bounds__(kArgThreads) void greedy_argmax_kernel(ArgmaxArgs a) {
  constexpr int EB = FMT == kFmtF32 ? 4 : 2;
  constexpr int kBatch = FMT == kFmtF32 ? 4 : 8;
  constexpr int CW = FMT == kFmtF32 ? 2 : 1;   // 16-byte words per chunk
  const int s = blockIdx.x;
  const int64_t r = blockIdx.y;
  const char* row = static_cast<const char*>(a.logits) + r * a.stride * EB;
  const int lo = s * a.slice_len;
  const int hi = lo + a.slice_len < a.vocab ? lo + a.slice_len : a.vocab;
  const int c0 = lo / 8, c1 = hi / 8;          // whole chunks of the slice
  float bv = kNegInf;
  int bi = 0x7fffffff;
  for (int ch0 = c0 + (int)threadIdx.x; ch0 < c1; ch0 += kBatch * kArgThreads) {
    u32x4 p[kBatch][CW];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int ch = ch0 + u * kArgThreads;
#pragma unroll
      for (int w = 0; w < CW; ++w)
        p[u][w] = ch < c1 ? ld16(row + (ch * CW + w) * 16) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int ch = ch0 + u * kArgThreads;
      if (ch >= c1) break;
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
  // the vocab % 8 last entries (only the last slice has them: slice_len is a multiple of 8)
  for (int i = 8 * c1 + (int)threadIdx.x; i < hi; i += kArgThreads) {
    const float v = elem<FMT>(row, i);
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  wave_best(bv, bi);
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
    if (a.slices == 1) {
      write_index(a, r, bi);
    } else {
      a.part_v[r * a.slices + s] = bv;
      a.part_i[r * a.slices + s] = bi;
    }
  }
}

// One wave per row: the best of the row's slice partials (at most 64).
__global__ __launch_bounds__(64) void greedy_argmax_combine_kernel(ArgmaxArgs a) {
  const int64_t r = blockIdx.x;
  const int lane = threadIdx.x;
  float bv = kNegInf;
  int bi = 0x7fffffff;
  if (lane < a.slices) {
    bv = a.part_v[r * a.slices + lane];
    bi = a.part_i[r * a.slices + lane];
  }
  wave_best(bv, bi);
  if (lane == 0) write_index(a, r, bi);
}

// Slices per row: enough workgroups to spread the batch over the GPU, each scanning at
// least kArgMinSlice elements; at most 64 (one combine wave).
inline int argmax_slices(int64_t rows, int vocab) {
  const int64_t by_len = (vocab + kArgMinSlice - 1) / kArgMinSlice;
  const int64_t by_wgs = rows > 0 ? (kArgTargetWgs + rows - 1) / rows : 1;
  int64_t s = by_len < by_wgs ? by_len : by_wgs;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return (int)s;
}

}  // namespace
}  // namespace ndl

extern "C" size_t ndl_greedy_argmax_workspace_bytes(int64_t rows, int vocab) {
  using namespace ndl;
  if (rows <= 0 || vocab <= 0) return 0;
  const int sl = argmax_slices(rows, vocab);
  return sl == 1 ? 0 : (size_t)rows * sl * 8;
}

extern "C" int ndl_greedy_argmax(void* out, int out_is_int64, const void* logits,
                                 int64_t row_stride, int64_t rows, int vocab, int dtype,
                                 void* workspace, size_t workspace_bytes, ndl_stream_t stream) {
  using namespace ndl;
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  if (rows < 0 || vocab <= 0) return NDL_ERR_INVALID_ARG;
  if (rows == 0) return NDL_OK;
  if (!out || !logits) return NDL_ERR_INVALID_ARG;
  if (row_stride < vocab || row_stride % 8 != 0 || ((uintptr_t)logits & 15u))
    return NDL_ERR_INVALID_ARG;
  if (rows > 65535) return NDL_ERR_UNSUPPORTED;   // grid y
  ArgmaxArgs a;
  a.logits = logits;
  a.out = out;
  a.rows = rows;
  a.stride = row_stride;
  a.vocab = vocab;
  a.slices = argmax_slices(rows, vocab);
  const int per = (vocab + a.slices - 1) / a.slices;
  a.slice_len = (per + 7) / 8 * 8;
  a.out64 = out_is_int64 ? 1 : 0;
  a.part_v = nullptr;
  a.part_i = nullptr;
  if (a.slices > 1) {
    const size_t need = (size_t)rows * a.slices * 8;
    if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 3u))
      return NDL_ERR_WORKSPACE;
    a.part_v = static_cast<float*>(workspace);
    a.part_i = reinterpret_cast<int*>(a.part_v + rows * a.slices);
  }
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)a.slices, (unsigned)rows);
  if (dtype_is_f32(dtype))
    hipLaunchKernelGGL((greedy_argmax_kernel<kFmtF32>), grid, dim3(kArgThreads), 0, s, a);
  else if (dtype_is_f16(dtype))
    hipLaunchKernelGGL((greedy_argmax_kernel<kFmtF16>), grid, dim3(kArgThreads), 0, s, a);
  else
    hipLaunchKernelGGL((greedy_argmax_kernel<kFmtBF16>), grid, dim3(kArgThreads), 0, s, a);
  if (a.slices > 1) {
    const int rc = check_launch();
    if (rc != NDL_OK) return rc;
    hipLaunchKernelGGL(greedy_argmax_combine_kernel, dim3((unsigned)rows), dim3(64), 0, s, a);
  }
  return check_launch();
}
