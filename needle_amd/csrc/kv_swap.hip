// Whole-block copies between two KV pools: the copies behind swap-out (GPU pool -> pinned
// CPU pool) and swap-in (CPU pool -> GPU pool).
//
// Reference: needle/model/runner.py:175-192 (_swap_kv_blocks) copies one (layer, block)
// slice per torch call, i.e. 2 x layers x blocks host-issued copies; the block ids come
// from BlockAllocator.swap_out / swap_in (block_allocator.py:88-106) through the
// scheduler's preemption and resume steps (scheduler.py:54-67, 90-102).
//
// Here one launch moves every block of every layer.  A pool is [2][NB][Hkv][16][D]; one
// plane of one block is a contiguous row of Hkv*16*D elements (4 KiB for Qwen2-0.5B,
// 32 KiB for Llama-3-8B).  Workgroup (x, plane, layer) copies 4 KiB pieces of the rows of
// pairs x / pieces_per_row with 16-byte loads and stores.  The pinned CPU pool is read or
// written directly through its device mapping: the copy runs at the PCIe link's rate with
// no staging buffer and no per-block host call.
#include "ndl_common.hpp"

namespace ndl {

constexpr int kSwapMaxLayers = 128;
constexpr int kSwapThreads = 256;
constexpr int64_t kSwapPiece = (int64_t)kSwapThreads * 16;  // bytes per workgroup pass

struct SwapArgs {
  const char* src[kSwapMaxLayers];
  char* dst[kSwapMaxLayers];
  const int32_t* src_ids;
  const int32_t* dst_ids;
  int64_t src_num_blocks, dst_num_blocks;
  int64_t row_bytes;         // one plane of one block
  int64_t pieces_per_row;    // ceil(row_bytes / kSwapPiece)
};

__global__ __launch_bounds__(kSwapThreads) void kv_block_copy_kernel(SwapArgs a) {
  const int64_t item = blockIdx.x;
  const int plane = blockIdx.y;
  const int layer = blockIdx.z;
  const int64_t pair = item / a.pieces_per_row;
  const int64_t piece = item - pair * a.pieces_per_row;
  const int64_t s = a.src_ids[pair];
  const int64_t d = a.dst_ids[pair];
  // ids outside a pool are never dereferenced (the pair is skipped)
  if (s < 0 || s >= a.src_num_blocks || d < 0 || d >= a.dst_num_blocks) return;
  const int64_t off = piece * kSwapPiece + (int64_t)threadIdx.x * 16;
  if (off >= a.row_bytes) return;
  const char* src = a.src[layer] + ((int64_t)plane * a.src_num_blocks + s) * a.row_bytes + off;
  char* dst = a.dst[layer] + ((int64_t)plane * a.dst_num_blocks + d) * a.row_bytes + off;
  st16(dst, ld16(src));
}

// Device address under which the kernel can reach `p`: device memory as is, pinned host
// memory through its (identity) device mapping; null for memory the device cannot address.
static const void* device_view(const void* p) {
  hipPointerAttribute_t attr;
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (attr.type == hipMemoryTypeDevice) return p;
  // Pinned host memory is mapped at the same virtual address on the device.  Any other
  // mapping is refused rather than translated.
  if (attr.type == hipMemoryTypeHost && attr.devicePointer != nullptr &&
      attr.devicePointer == attr.hostPointer)
    return p;
  return nullptr;
}

}  // namespace ndl

extern "C" int ndl_kv_block_copy(void* const* dst_pools, int64_t dst_num_blocks,
                                 const void* const* src_pools, int64_t src_num_blocks,
                                 int num_layers, int num_kv_heads, int block_size, int head_dim,
                                 int dtype, const int32_t* src_ids, const int32_t* dst_ids,
                                 int num_pairs, ndl_stream_t stream) {
  using namespace ndl;
  if (!dtype_known(dtype)) return NDL_ERR_UNSUPPORTED;
  if (num_layers < 0 || num_pairs < 0 || num_kv_heads <= 0 || block_size <= 0 ||
      head_dim <= 0 || dst_num_blocks <= 0 || src_num_blocks <= 0)
    return NDL_ERR_INVALID_ARG;
  if (num_layers > kSwapMaxLayers) return NDL_ERR_UNSUPPORTED;
  if (num_layers == 0 || num_pairs == 0) return NDL_OK;
  if (!dst_pools || !src_pools || !src_ids || !dst_ids) return NDL_ERR_INVALID_ARG;
  const int64_t row_bytes = (int64_t)num_kv_heads * block_size * head_dim * dtype_bytes(dtype);
  if (row_bytes % 16) return NDL_ERR_UNSUPPORTED;
  SwapArgs a;
  for (int l = 0; l < num_layers; ++l) {
    const void* s = src_pools[l];
    const void* d = dst_pools[l];
    if (!s || !d || (((uintptr_t)s | (uintptr_t)d) & 15u)) return NDL_ERR_INVALID_ARG;
    s = device_view(s);
    d = device_view(d);
    if (!s || !d) return NDL_ERR_INVALID_ARG;
    a.src[l] = (const char*)s;
    a.dst[l] = (char*)d;
  }
  const void* si = device_view(src_ids);
  const void* di = device_view(dst_ids);
  if (!si || !di) return NDL_ERR_INVALID_ARG;
  a.src_ids = (const int32_t*)si;
  a.dst_ids = (const int32_t*)di;
  a.src_num_blocks = src_num_blocks;
  a.dst_num_blocks = dst_num_blocks;
  a.row_bytes = row_bytes;
  a.pieces_per_row = (row_bytes + kSwapPiece - 1) / kSwapPiece;
  const int64_t items = (int64_t)num_pairs * a.pieces_per_row;
  if (items > 0x7fffffff) return NDL_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(kv_block_copy_kernel, dim3((unsigned)items, 2, (unsigned)num_layers),
                     dim3(kSwapThreads), 0, (hipStream_t)stream, a);
  return check_launch();
}
