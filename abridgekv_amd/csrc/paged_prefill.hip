// Multi-query attention over the paged abridged cache: prompt-chunk prefill (causal) and the CompressLM code step.
//
// The code step is the serving twin of the training mask (third_party/vllm_overlay/vllm/v1/worker/
// gpu_model_runner.py:2042-2107; masks from compresslm_masks.py:165-239; trim form trim_code_kv.patch:15-63): the
// K_max code rows of the block being closed attend non-causally to every resident row of their KV-cache group before
// them and to the first q_g code rows of their own block (own-block slots >= q_g are hidden). In a group's physical
// layout that is exactly "keys < code_start + q_g", so each request carries a key limit instead of a dense mask:
//   query row i of request r sits at physical position kv_start[r] + i and sees keys k < kv_limit[r]
//   (and k <= its own position when request r is causal; a batch may mix causal chunks and code steps).
// Prompt chunks are the causal case with kv_limit = seq_len. Same tile machinery as the masked-prefill kernel
// (attn_tile.h): 8 waves x (16 rows x 2 heads), 64-key tiles DMA'd from the page table into double-buffered LDS.
#include "attn_tile.h"

namespace abkv {

struct PagedPrefillArgs {
  const __bf16* q;  long q_st, q_sh;           // [T, 32, 128]
  const __bf16* kv; int num_pages;             // [pages, 2, 16, 8, 128]
  const int32_t* block_table; long bt_stride; int bt_width;  // [B, W]
  const int32_t* q_start;                      // [B + 1] first query token of each request
  const int32_t* kv_start;                     // [B] physical position of each request's first query token
  const int32_t* kv_limit;                     // [B] visible keys: physical slots [0, kv_limit)
  const int32_t* tile_req;                     // [n_tiles] request of each 64-row query tile
  const int32_t* tile_q0;                      // [n_tiles] first query row (within its request) of the tile
  const int32_t* causal;                       // [B] 1 = causal, 0 = non-causal (nullptr: causal_default)
  int causal_default;
  float scale_log2;
  __bf16* out; long o_st, o_sh;                // [T, 32, 128]
  float* lse;                                  // [T, 32] natural log, or nullptr
};

__global__ __launch_bounds__(512, 1) void paged_prefill_kernel(PagedPrefillArgs a) {
  constexpr int H = 2, kWaves = 8;
  __shared__ __attribute__((aligned(16))) __bf16 Kb[2 * kTileElems];
  __shared__ __attribute__((aligned(16))) __bf16 Vb[2 * kTileElems];

  const int r = a.tile_req[blockIdx.x];
  const int q0 = a.tile_q0[blockIdx.x];
  const int kvh = blockIdx.y;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int m16 = lane & 15;
  const int j = lane >> 4;
  const int rg = w >> 1;
  const int hbase = H * (w & 1);
  const int t0 = a.q_start[r];
  const int nq = a.q_start[r + 1] - t0;
  const int kv0 = a.kv_start[r];
  const int limit = a.kv_limit[r];
  const bool causal = a.causal ? a.causal[r] != 0 : a.causal_default != 0;
  const int qi = q0 + 16 * rg + m16;                        // query row within the request (MFMA column)
  const bool qvalid = qi < nq;
  const int pos = kv0 + qi;
  const int lane_limit = causal ? min(limit, pos + 1) : limit;

  bf16x8 qop[H][4];
  {
    const __bf16* qb = a.q + (long)(t0 + min(qi, nq - 1)) * a.q_st;
#pragma unroll
    for (int u = 0; u < H; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x4 x = ld16g(qb + (long)(kvh * kGroup + hbase + u) * a.q_sh + 8 * (4 * i + j));
        if (!qvalid) x = u32x4{0, 0, 0, 0};
        qop[u][i] = __builtin_bit_cast(bf16x8, x);
      }
  }
  floatx4 o[8][H];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int u = 0; u < H; ++u) o[i][u] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run[H], l_run[H];
#pragma unroll
  for (int u = 0; u < H; ++u) {
    m_run[u] = -INFINITY;
    l_run[u] = 0.f;
  }

  // key range of the tile: the largest lane limit bounds the walk, the smallest one marks the fully visible tiles
  const int q_hi = min(q0 + kBM, nq) - 1;
  const int k_end = causal ? min(limit, kv0 + q_hi + 1) : limit;
  const int k_full = causal ? min(limit, kv0 + q0 + 1) : limit;
  const int n_k_tiles = (k_end + kBN - 1) / kBN;
  const PagedRows rows{a.kv + kvh * kHeadDim, a.block_table + (long)r * a.bt_stride, a.bt_width, a.num_pages};
  const MaskGeom geo{};
  TileMask tm;
  tm.mode = 0;

  if (n_k_tiles > 0) issue_tile<kWaves>(rows, 0, k_end, Kb, Vb, w, lane);
  for (int kt = 0; kt < n_k_tiles; ++kt) {
    const int off_cur = (kt & 1) * kTileElems, off_nxt = ((kt & 1) ^ 1) * kTileElems;
    if (kt + 1 < n_k_tiles) {
      issue_tile<kWaves>(rows, (kt + 1) * kBN, k_end, Kb + off_nxt, Vb + off_nxt, w, lane);
      __asm__ volatile("s_waitcnt vmcnt(4)" ::: "memory");
    } else {
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    tm.mode = (kt + 1) * kBN <= k_full ? 0 : 1;
    tile_compute<H, true>(Kb + off_cur, Vb + off_cur, qop, o, m_run, l_run, kt * kBN, tm, lane_limit, a.scale_log2,
                          geo, hbase, m16, j);
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
  }

  if (!qvalid) return;
#pragma unroll
  for (int u = 0; u < H; ++u) {
    const float l = sum_xor32(sum_xor16(l_run[u]));
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int head = kvh * kGroup + hbase + u;
    __bf16* oh = a.out + (long)(t0 + qi) * a.o_st + (long)head * a.o_sh + 32 * j;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      u32x4 wv;
#pragma unroll
      for (int c = 0; c < 4; ++c) wv[c] = pack_bf16x2(o[2 * c][u][rr] * inv, o[2 * c + 1][u][rr] * inv);
      *reinterpret_cast<u32x4*>(oh + 8 * rr) = wv;
    }
    if (a.lse != nullptr && j == 0)
      a.lse[(long)(t0 + qi) * kHeadsQ + head] = l > 0.f ? (m_run[u] + __log2f(l)) * 0.69314718055994531f : -INFINITY;
  }
}

}  // namespace abkv

extern "C" {

int abkv_paged_prefill_attn(const void* q, long q_stride_t, long q_stride_h, const void* kv_cache, int num_pages,
                            const int32_t* block_table, long block_table_stride, int block_table_width,
                            const int32_t* q_start,
                            const int32_t* kv_start, const int32_t* kv_limit, const int32_t* tile_req,
                            const int32_t* tile_q0, int num_tiles, const int32_t* causal, int causal_default,
                            float scale, void* out,
                            long out_stride_t, long out_stride_h, float* lse, hipStream_t stream) {
  using namespace abkv;
  if (num_tiles <= 0) return 0;
  if (q == nullptr || kv_cache == nullptr || block_table == nullptr || q_start == nullptr || kv_start == nullptr ||
      kv_limit == nullptr || tile_req == nullptr || tile_q0 == nullptr || out == nullptr || num_pages <= 0 ||
      block_table_width <= 0)
    return (int)hipErrorInvalidValue;
  PagedPrefillArgs a;
  a.q = static_cast<const __bf16*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.kv = static_cast<const __bf16*>(kv_cache);
  a.num_pages = num_pages;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.bt_width = block_table_width;
  a.q_start = q_start;
  a.kv_start = kv_start;
  a.kv_limit = kv_limit;
  a.tile_req = tile_req;
  a.tile_q0 = tile_q0;
  a.causal = causal;
  a.causal_default = causal_default;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = static_cast<__bf16*>(out);
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.lse = lse;
  hipLaunchKernelGGL(paged_prefill_kernel, dim3(num_tiles, kHeadsKV), dim3(512), 0, stream, a);
  return (int)hipGetLastError();
}

}  // extern "C"
