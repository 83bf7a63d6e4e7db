// Measurement probes, built into libabridgekv_probes.so beside the product library and loaded by the benchmark
// only. They have no counterpart in the reference: each one is the plainest kernel with a product kernel's access
// pattern, so the product kernel's bandwidth can be read against what that pattern allows.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kMaxProbeLayers = 16;

struct ProbeLayers {
  const char* src[kMaxProbeLayers];
  char* dst[kMaxProbeLayers];
};

using u32x4 = __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t;

// Row copy with a compaction launch's addresses and none of its ordering: op i of layer l copies the row at
// (src_block, src_off) of src[l] to (dst_block, dst_off) of dst[l], a different tensor, so every op is independent.
// Workgroup = kRows ops of one layer, thread t = the t-th 16-byte vector of a row (K half, then V half); each thread
// issues its kRows loads back to back, then its kRows stores, streaming (non-temporal) as the mover does. Ops outside
// the cache are skipped.
template <int kRows>
__global__ __launch_bounds__(256) void probe_row_copy_kernel(ProbeLayers L, const int32_t* __restrict__ ops, int n_ops,
                                                             long page_bytes, long half_bytes, int slot_bytes,
                                                             int num_pages, int block_size) {
  const int layer = blockIdx.y;
  const int c0 = blockIdx.x * kRows;
  const int row_vec = (2 * slot_bytes) / 16;
  const char* src = L.src[layer];
  char* dst = L.dst[layer];
  for (int v = threadIdx.x; v < row_vec; v += 256) {
    const int half = v >= row_vec / 2;
    const long inner = (long)half * half_bytes + (long)(v - half * (row_vec / 2)) * 16;
    long soff[kRows], doff[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int i = c0 + r;
      soff[r] = doff[r] = -1;
      if (i < n_ops) {
        const int32_t* op = ops + 4L * i;
        const int sb = op[0], so = op[1], db = op[2], dof = op[3];
        if ((unsigned)sb < (unsigned)num_pages && (unsigned)db < (unsigned)num_pages &&
            (unsigned)so < (unsigned)block_size && (unsigned)dof < (unsigned)block_size) {
          soff[r] = (long)sb * page_bytes + (long)so * slot_bytes + inner;
          doff[r] = (long)db * page_bytes + (long)dof * slot_bytes + inner;
        }
      }
    }
    u32x4 buf[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r)
      buf[r] = soff[r] >= 0 ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + soff[r]))
                            : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < kRows; ++r)
      if (doff[r] >= 0) __builtin_nontemporal_store(buf[r], reinterpret_cast<u32x4*>(dst + doff[r]));
  }
}

}  // namespace

extern "C" {

// Copy the rows named by ops [n_ops, 4] int32 (src_block, src_off, dst_block, dst_off; device memory) from
// src_layers[l] to dst_layers[l] for every layer l < n_layers (at most 16), rows_per_block ops per workgroup
// (4, 8 or 16). Caches are [num_pages, 2, block_size, ...] with K at byte 0 and V at half_bytes of each page.
// Returns 0 or a hipError_t value.
int abkv_probe_row_copy(const void* const* src_layers, void* const* dst_layers, int n_layers, const int32_t* ops,
                        int n_ops, long page_bytes, long half_bytes, int slot_bytes, int num_pages, int block_size,
                        int rows_per_block, hipStream_t stream) {
  if (n_ops <= 0 || n_layers <= 0) return 0;
  if (n_layers > kMaxProbeLayers || ops == nullptr || src_layers == nullptr || dst_layers == nullptr ||
      slot_bytes <= 0 || slot_bytes % 16 != 0 || 2L * slot_bytes * block_size > page_bytes ||
      half_bytes < (long)slot_bytes * block_size || num_pages <= 0 || block_size <= 0)
    return (int)hipErrorInvalidValue;
  ProbeLayers L;
  for (int l = 0; l < n_layers; ++l) {
    if (src_layers[l] == nullptr || dst_layers[l] == nullptr) return (int)hipErrorInvalidValue;
    L.src[l] = static_cast<const char*>(src_layers[l]);
    L.dst[l] = static_cast<char*>(dst_layers[l]);
  }
  const dim3 grid((unsigned)((n_ops + rows_per_block - 1) / rows_per_block), (unsigned)n_layers);
  switch (rows_per_block) {
    case 4: hipLaunchKernelGGL(probe_row_copy_kernel<4>, grid, dim3(256), 0, stream, L, ops, n_ops, page_bytes,
                               half_bytes, slot_bytes, num_pages, block_size); break;
    case 8: hipLaunchKernelGGL(probe_row_copy_kernel<8>, grid, dim3(256), 0, stream, L, ops, n_ops, page_bytes,
                               half_bytes, slot_bytes, num_pages, block_size); break;
    case 16: hipLaunchKernelGGL(probe_row_copy_kernel<16>, grid, dim3(256), 0, stream, L, ops, n_ops, page_bytes,
                                half_bytes, slot_bytes, num_pages, block_size); break;
    default: return (int)hipErrorInvalidValue;
  }
  return (int)hipGetLastError();
}

}  // extern "C"
