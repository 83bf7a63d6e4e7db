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

// LDS read throughput: a workgroup of 4 waves fills 64 KiB of LDS, then every wave issues `iters` x 8 reads, either
// ds_read_b128 of conflict-free 1 KiB blocks (kMode 0) or ds_read_b64_tr_b16 with the masked-prefill kernels' swizzled
// V / Q^T operand addressing (kMode 1). The addresses are computed once; per iteration only a wave-uniform tile
// offset (runtime stride) changes, so the loop is the reads plus one add per read. cycles[wg] = shader-clock ticks of
// the read loop; sink keeps the read values alive.
template <int kMode>
__global__ __launch_bounds__(256) void probe_lds_read_kernel(uint32_t* sink, long long* cycles, int iters, int stride) {
  __shared__ __attribute__((aligned(16))) uint32_t buf[16384];     // 4 tiles of 64 rows x 256 B
  for (int i = threadIdx.x; i < 16384; i += 256) buf[i] = i * 2654435761u;
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int base[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if constexpr (kMode == 0) {
      base[u] = ((u * 4 + w) & 15) * 256 + lane * 4;                // words; max 4092 (+3)
    } else {
      const int kb = (u & 1) * 32, t = (u >> 1) * 2 + (w & 1);
      const int g = lane >> 4, i = lane & 15, e = i >> 2, c = i & 3;
      const int dim = 32 * c + 4 * (t ^ (c & 1));
      const int row0 = kb + 4 * g + e;                               // < 48
      base[u] = row0 * 64 + 4 * ((dim >> 3) ^ (row0 & 15)) + ((dim & 7) >> 1);   // max 3071 (+1)
    }
  }
  typedef short s4 __attribute__((ext_vector_type(4)));
  typedef int i2 __attribute__((ext_vector_type(2)));
  uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
  const long long t0 = __builtin_readcyclecounter();
  for (int it = 0; it < iters; ++it) {
    const int tile = ((it * stride) & 3) * 4096;                      // + 12288 at most: inside the 16384 words
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if constexpr (kMode == 0) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(&buf[base[u] + tile]);
        a0 += v[0];
        a1 += v[1];
        a2 += v[2];
        a3 += v[3];
      } else {
        const s4 v =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(&buf[base[u] + tile]));
        const i2 y = __builtin_bit_cast(i2, v);
        a0 += (uint32_t)y[0];
        a1 += (uint32_t)y[1];
      }
    }
  }
  const long long t1 = __builtin_readcyclecounter();
  sink[blockIdx.x * 256 + threadIdx.x] = a0 ^ a1 ^ a2 ^ a3;
  if (threadIdx.x == 0) cycles[blockIdx.x] = t1 - t0;
}

}  // namespace

extern "C" {

// LDS read throughput probe: n_workgroups workgroups of 256 threads (64 KiB of LDS each), mode 0 ds_read_b128, mode 1
// ds_read_b64_tr_b16; sink [n_workgroups * 256] uint32 and cycles [n_workgroups] int64 are device buffers. Every
// wave reads iters * 8 times (1 KiB per b128 read, 512 B per transposed read).
int abkv_probe_lds_read(int mode, int n_workgroups, int iters, int stride, uint32_t* sink, long long* cycles,
                        hipStream_t stream) {
  if (n_workgroups <= 0 || iters <= 0 || sink == nullptr || cycles == nullptr || (mode != 0 && mode != 1))
    return (int)hipErrorInvalidValue;
  if (mode == 0)
    hipLaunchKernelGGL(probe_lds_read_kernel<0>, dim3(n_workgroups), dim3(256), 0, stream, sink, cycles, iters, stride);
  else
    hipLaunchKernelGGL(probe_lds_read_kernel<1>, dim3(n_workgroups), dim3(256), 0, stream, sink, cycles, iters, stride);
  return (int)hipGetLastError();
}

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
