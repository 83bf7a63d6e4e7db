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
  const int32_t* kv_excluded;                  // [B][2] physical [start, end) hidden from the request, or nullptr
  const int32_t* tile_req;                     // [n_tiles] request of each 64-row query tile
  const int32_t* tile_q0;                      // [n_tiles] first query row (within its request) of the tile
  const int32_t* causal;                       // [B] 1 = causal, 0 = non-causal (nullptr: causal_default)
  int causal_default;
  float scale_log2;
  __bf16* out; long o_st, o_sh;                // [T, 32, 128]
  float* lse;                                  // [T, 32] natural log, or nullptr
  int num_tiles;                               // query tiles; the grid is 8 x num_tiles x splits (linear_block)
  int split_tiles;                             // > 0: key tiles per split, partials to part_*
  int num_tokens;
  _Float16* part_o;                            // [splits, T, 32, 128] split output / (l * scale), fp16
  float* part_ml;                              // [splits, T, 32, 4] (max in log2 units, weight sum l, scale, unused)
  int split_base;                              // first partial slot of this launch's splits
  const int32_t* head_quota;                   // [8] or nullptr: a non-causal request sees keys < kv_start + q_h
  // side rows (per-head packed code pages, attended by every query of the request); see PackedRows
  const __bf16* side_kv; int side_rows; int side_pool_pages;
  const int32_t* side_table; long side_stride; const int32_t* side_count; int side_max_pages;
  int side_q[kHeadsKV], side_o[kHeadsKV];
};

// Dims 8p .. 8p + 7 of an accumulator column (lane group j) times f, as one 16-byte fp16 store (the column layout of
// store_acc_bf16x8).
__device__ __forceinline__ void store_acc_f16x8(_Float16* dst, const floatx4& a, const floatx4& b, int j, float f) {
  const bool odd = j & 1;
  typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
  f16x8 h;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    h[r] = (_Float16)((odd ? b[r] : a[r]) * f);
    h[4 + r] = (_Float16)((odd ? a[r] : b[r]) * f);
  }
  *reinterpret_cast<f16x8*>(dst) = h;
}

constexpr int kMaxSideTable = 2048;             // packed pages per request the side launch stages in LDS

// Side rows of one request for KV head h: row r is row side_o[h] + r % q_h of packed page table[r / q_h]
// ([2][rows][128] pages). The request's packed page ids are staged in LDS once; r / q_h by a float reciprocal is
// exact while r < 2^21 (0.5 / q_h exceeds the rounding error r / q_h * 2^-22).
struct PackedRows {
  const __bf16* base;      // pool + side_o[h] * 128
  const int32_t* table;    // LDS copy of the request's page ids
  int q;
  float inv_q;
  long page_elems, v_off;
  struct Src {
    int k0;
  };
  template <int kPerWave>
  __device__ __forceinline__ Src src(int k0, int, int) const { return Src{k0}; }
  template <bool kV>
  __device__ __forceinline__ const __bf16* addr(const Src& t, int row, int chunk, int n_keys) const {
    const int r = min(t.k0 + row, n_keys - 1);             // past the end: row n_keys - 1 (finite, weight 0)
    const int p = (int)(((float)r + 0.5f) * inv_q);
    const int slot = r - p * q;
    return base + (long)table[p] * page_elems + slot * kHeadDim + (kV ? v_off : 0) + 8 * chunk;
  }
};

// Contiguous key tiles [kt_begin, kt_end); tiles past k_full (the smallest lane limit) are masked per lane, and tiles
// that meet the excluded key range [ex_lo, ex_hi) (empty when ex_lo >= ex_hi) mask it as well.
struct RangeWalk {
  static constexpr bool kHole = true;
  static constexpr bool kElem = false;
  static constexpr bool kBand = false;
  int kt_begin, kt_end, k_full, ex_lo, ex_hi;
  __device__ __forceinline__ bool next(int& kt, TileMask& tm, bool first) {
    kt = first ? kt_begin : kt + 1;
    tm.mode = (kt + 1) * kBN <= k_full ? 0 : 1;
    if (kt * kBN < ex_hi && (kt + 1) * kBN > ex_lo) {
      tm.mode = 4;
      tm.limit[0] = ex_lo;
      tm.limit[1] = ex_hi;
    }
    return kt < kt_end;
  }
};

// kSide = false: the paged rows of the request; true: its side rows (all visible to every query).
template <bool kSide>
__global__ __launch_bounds__(512, 1) void paged_prefill_kernel(PagedPrefillArgs a) {
  constexpr int H = 2, kWaves = 8;
  __shared__ __attribute__((aligned(16))) __bf16 K0[kTileElems], K1[kTileElems], K2[kTileElems];
  __shared__ __attribute__((aligned(16))) __bf16 V0[kTileElems], V1[kTileElems], V2[kTileElems];
  __bf16* const Kbuf[kStages] = {K0, K1, K2};
  __bf16* const Vbuf[kStages] = {V0, V1, V2};
  // linear grid, KV head fastest, then query tile, then key split: workgroups go to the 8 XCDs round-robin by
  // linear id, so the query tiles of one request that read the same K/V tiles (same head, same split) share an L2
  const int l = blockIdx.x;
  const int kvh = l % kHeadsKV;
  const int tile = (l / kHeadsKV) % a.num_tiles;
  const int split = l / (kHeadsKV * a.num_tiles);
  const int r = a.tile_req[tile];
  const int q0 = a.tile_q0[tile];
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index (uniform)
  const int lane = tid & 63;
  const int m16 = lane & 15;
  const int j = lane >> 4;
  const int rg = w >> 1;
  const int hbase = H * (w & 1);
  const int t0 = a.q_start[r];
  const int nq = a.q_start[r + 1] - t0;
  const int kv0 = a.kv_start[r];
  const bool causal = kSide ? false : (a.causal ? a.causal[r] != 0 : a.causal_default != 0);
  int limit = a.kv_limit[r];
  if (!kSide && !causal && a.head_quota != nullptr) limit = min(limit, kv0 + a.head_quota[kvh]);
  int side_q = 0, side_n = 0;
  if constexpr (kSide) {
    side_q = a.side_q[kvh];
    side_n = min(max(a.side_count[r], 0), a.side_max_pages);
    limit = side_n * side_q;                                 // side rows of this head
  }
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
  const MaskGeom geo{};
  // key tiles of this block: all of them, or split z's share when the launch is split along the keys
  RangeWalk walk;
  walk.kt_begin = a.split_tiles > 0 ? split * a.split_tiles : 0;
  walk.kt_end = a.split_tiles > 0 ? min(n_k_tiles, walk.kt_begin + a.split_tiles) : n_k_tiles;
  walk.k_full = k_full;
  walk.ex_lo = walk.ex_hi = 0;
  if (!kSide && a.kv_excluded != nullptr) {
    walk.ex_lo = a.kv_excluded[2 * r];
    walk.ex_hi = a.kv_excluded[2 * r + 1];
  }
  if constexpr (kSide) {
    __shared__ int32_t side_table[kMaxSideTable];
    const int32_t* src = a.side_table + (long)r * a.side_stride;
    for (int i = tid; i < side_n; i += 512) side_table[i] = min(max(src[i], 0), a.side_pool_pages - 1);
    __syncthreads();
    const PackedRows rows{a.side_kv + (long)a.side_o[kvh] * kHeadDim, side_table, side_q, 1.f / (float)side_q,
                          2L * a.side_rows * kHeadDim, (long)a.side_rows * kHeadDim};
    attend_tiles<H, true, kWaves>(rows, walk, k_end, Kbuf, Vbuf, qop, o, m_run, l_run, lane_limit, a.scale_log2, geo,
                                  w, lane);
  } else {
    const PagedRows rows{a.kv + kvh * kHeadDim, a.block_table + (long)r * a.bt_stride, a.bt_width, a.num_pages};
    attend_tiles<H, true, kWaves>(rows, walk, k_end, Kbuf, Vbuf, qop, o, m_run, l_run, lane_limit, a.scale_log2, geo,
                                  w, lane);
  }

  // Split partials: the split's output normalised by its weight sum l, in fp16 (half the bytes the epilogue writes
  // and the merge reads), divided by a scale that keeps every value within +-32768 (1 unless the split's V rows
  // exceed that), and the record (m, l, scale). The scale needs the row's largest |o| over its 128 dims, which lie in
  // the row's four lane groups (lanes m16 + 16j): reduced before any lane leaves.
  float amax[H];
  if (a.split_tiles > 0) {
#pragma unroll
    for (int u = 0; u < H; ++u) {
      float x = 0.f;
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) x = fmaxf(x, fabsf(o[t][u][r]));
      amax[u] = max_xor32(max_xor16(x));
    }
  }
  if (!qvalid) return;
  if (a.split_tiles > 0) {                                   // partials of this key split
#pragma unroll
    for (int u = 0; u < H; ++u) {
      const float l = l_run[u];
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const float an = amax[u] * inv;
      const float scale = an > 32768.f ? an * (1.f / 32768.f) : 1.f;
      const int head = kvh * kGroup + hbase + u;
      const long row = ((long)(a.split_base + split) * a.num_tokens + (t0 + qi)) * kHeadsQ + head;
      _Float16* po = a.part_o + row * kHeadDim + 32 * j;
#pragma unroll
      for (int p = 0; p < 4; ++p) store_acc_f16x8(po + 8 * p, o[2 * p][u], o[2 * p + 1][u], j, inv / scale);
      if (j == 0) *reinterpret_cast<floatx4*>(a.part_ml + row * 4) = floatx4{m_run[u], l, scale, 0.f};
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < H; ++u) {
    const float l = l_run[u];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int head = kvh * kGroup + hbase + u;
    __bf16* oh = a.out + (long)(t0 + qi) * a.o_st + (long)head * a.o_sh + 32 * j;
#pragma unroll
    for (int p = 0; p < 4; ++p) store_acc_bf16x8(oh + 8 * p, o[2 * p][u], o[2 * p + 1][u], j, inv);
    if (a.lse != nullptr && j == 0)
      a.lse[(long)(t0 + qi) * kHeadsQ + head] = l > 0.f ? (m_run[u] + __log2f(l)) * 0.69314718055994531f : -INFINITY;
  }
}

// Combine the key-split partials of every query token: workgroup (token, group of 8 heads); thread t handles head
// 8 * blockIdx.y + t / 32 and dims 4 * (t % 32) .. +4.
__global__ __launch_bounds__(256) void paged_merge_kernel(PagedPrefillArgs a, int n_splits) {
  typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
  const long tok = blockIdx.x;
  const int head = 8 * blockIdx.y + (threadIdx.x >> 5);
  const int d0 = (threadIdx.x & 31) * 4;
  const long stride = (long)a.num_tokens * kHeadsQ;          // rows per split
  const float* pml = a.part_ml + (tok * kHeadsQ + head) * 4;
  float M = -INFINITY;
#pragma unroll 8
  for (int s = 0; s < n_splits; ++s) M = fmaxf(M, pml[s * stride * 4]);
  float L = 0.f;
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  if (M != -INFINITY) {
#pragma unroll 8
    for (int s = 0; s < n_splits; ++s) {
      const floatx4 rec = *reinterpret_cast<const floatx4*>(pml + s * stride * 4);     // m, l, scale
      const float w = fast_exp2(rec[0] - M) * rec[1];      // the split's weight (0 for a split that saw no key)
      const float ws = w * rec[2];
      L += w;
      const f16x4 h = *reinterpret_cast<const f16x4*>(a.part_o + ((s * stride) + tok * kHeadsQ + head) * kHeadDim + d0);
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] += ws * (float)h[r];
    }
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  __bf16* oh = a.out + tok * a.o_st + (long)head * a.o_sh + d0;
  u32x2 wv;
  wv[0] = pack_bf16x2(acc[0] * inv, acc[1] * inv);
  wv[1] = pack_bf16x2(acc[2] * inv, acc[3] * inv);
  *reinterpret_cast<u32x2*>(oh) = wv;
  if (a.lse != nullptr && (threadIdx.x & 31) == 0)
    a.lse[tok * kHeadsQ + head] = L > 0.f ? (M + __log2f(L)) * 0.69314718055994531f : -INFINITY;
}

}  // namespace abkv

namespace {
// Workgroups of a paged_prefill_kernel launch (8 x num_tiles x splits, 512 threads each); 0 when the work-item count
// would not fit the 32-bit grid size.
unsigned paged_grid(int num_tiles, int splits) {
  const long n = (long)num_tiles * abkv::kHeadsKV * splits;
  return n <= 0 || n * 512 > 0xFFFFFFFFL ? 0u : (unsigned)n;
}
}  // namespace

extern "C" {

size_t abkv_paged_prefill_workspace_size(int num_tokens, int num_splits) {
  return (size_t)num_tokens * (size_t)num_splits * abkv::kHeadsQ *
         (abkv::kHeadDim * sizeof(_Float16) + 4 * sizeof(float));
}


int abkv_paged_prefill_attn(const void* q, long q_stride_t, long q_stride_h, const void* kv_cache, int num_pages,
                            const int32_t* block_table, long block_table_stride, int block_table_width,
                            const int32_t* q_start,
                            const int32_t* kv_start, const int32_t* kv_limit, const int32_t* kv_excluded,
                            const int32_t* tile_req,
                            const int32_t* tile_q0, int num_tiles, const int32_t* causal, int causal_default,
                            float scale, void* out,
                            long out_stride_t, long out_stride_h, float* lse, int num_tokens, int num_splits,
                            int split_tiles, void* workspace, size_t workspace_bytes, hipStream_t stream) {
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
  a.kv_excluded = kv_excluded;
  a.tile_req = tile_req;
  a.tile_q0 = tile_q0;
  a.causal = causal;
  a.causal_default = causal_default;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = static_cast<__bf16*>(out);
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.lse = lse;
  a.num_tokens = num_tokens;
  a.split_tiles = 0;
  a.part_o = nullptr;
  a.part_ml = nullptr;
  a.split_base = 0;
  a.head_quota = nullptr;
  a.side_count = nullptr;
  if (num_splits > 1) {
    if (split_tiles <= 0 || num_tokens <= 0 || workspace == nullptr ||
        workspace_bytes < abkv_paged_prefill_workspace_size(num_tokens, num_splits))
      return (int)hipErrorInvalidValue;
    a.split_tiles = split_tiles;
    a.part_o = static_cast<_Float16*>(workspace);
    a.part_ml = reinterpret_cast<float*>(a.part_o + (size_t)num_splits * num_tokens * kHeadsQ * kHeadDim);
  }
  const unsigned grid = paged_grid(num_tiles, num_splits > 1 ? num_splits : 1);
  if (grid == 0) return (int)hipErrorInvalidValue;
  a.num_tiles = num_tiles;
  hipLaunchKernelGGL(paged_prefill_kernel<false>, dim3(grid), dim3(512), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || num_splits <= 1) return (int)err;
  hipLaunchKernelGGL(paged_merge_kernel, dim3(num_tokens, kHeadsQ / 8), dim3(256), 0, stream, a, num_splits);
  return (int)hipGetLastError();
}

int abkv_paged_prefill_attn_packed(const void* q, long q_stride_t, long q_stride_h, const void* kv_cache,
                                   int num_pages, const int32_t* block_table, long block_table_stride,
                                   int block_table_width, const int32_t* q_start, const int32_t* kv_start,
                                   const int32_t* kv_limit, const int32_t* kv_excluded, const int32_t* tile_req,
                                   const int32_t* tile_q0,
                                   int num_tiles, const int32_t* causal, int causal_default,
                                   const int32_t* head_quota_dev, const void* packed_kv, int packed_pool_pages,
                                   int packed_rows, const int32_t* head_quota, const int32_t* packed_table,
                                   long packed_table_stride, const int32_t* packed_count, int max_packed_per_seq,
                                   float scale, void* out, long out_stride_t, long out_stride_h, float* lse,
                                   int num_tokens, int num_splits, int split_tiles, int side_splits,
                                   int side_split_tiles, void* workspace, size_t workspace_bytes,
                                   hipStream_t stream) {
  using namespace abkv;
  if (num_tiles <= 0) return 0;
  if (q == nullptr || kv_cache == nullptr || block_table == nullptr || q_start == nullptr || kv_start == nullptr ||
      kv_limit == nullptr || tile_req == nullptr || tile_q0 == nullptr || out == nullptr || num_pages <= 0 ||
      block_table_width <= 0 || head_quota_dev == nullptr || packed_kv == nullptr || head_quota == nullptr ||
      packed_table == nullptr || packed_count == nullptr || packed_pool_pages <= 0 || max_packed_per_seq < 0 ||
      max_packed_per_seq > kMaxSideTable || packed_table_stride < max_packed_per_seq || num_splits < 1 ||
      split_tiles <= 0 || side_splits < 1 || side_split_tiles <= 0 || num_tokens <= 0)
    return (int)hipErrorInvalidValue;
  PagedPrefillArgs a;
  int rows = 0, qmax = 0;
  for (int h = 0; h < kHeadsKV; ++h) {
    if (head_quota[h] <= 0 || head_quota[h] > 2048) return (int)hipErrorInvalidValue;
    a.side_q[h] = head_quota[h];
    a.side_o[h] = rows;
    rows += head_quota[h];
    qmax = head_quota[h] > qmax ? head_quota[h] : qmax;
  }
  if (rows != packed_rows || (long)max_packed_per_seq * qmax >= (1L << 21) ||
      (long)side_splits * side_split_tiles * kBN < (long)max_packed_per_seq * qmax)
    return (int)hipErrorInvalidValue;
  const int total = num_splits + side_splits;
  if (workspace == nullptr || workspace_bytes < abkv_paged_prefill_workspace_size(num_tokens, total))
    return (int)hipErrorInvalidValue;
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
  a.kv_excluded = kv_excluded;
  a.tile_req = tile_req;
  a.tile_q0 = tile_q0;
  a.causal = causal;
  a.causal_default = causal_default;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = static_cast<__bf16*>(out);
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.lse = lse;
  a.num_tokens = num_tokens;
  a.part_o = static_cast<_Float16*>(workspace);
  a.part_ml = reinterpret_cast<float*>(a.part_o + (size_t)total * num_tokens * kHeadsQ * kHeadDim);
  a.head_quota = head_quota_dev;
  a.side_kv = static_cast<const __bf16*>(packed_kv);
  a.side_rows = packed_rows;
  a.side_pool_pages = packed_pool_pages;
  a.side_table = packed_table;
  a.side_stride = packed_table_stride;
  a.side_count = packed_count;
  a.side_max_pages = max_packed_per_seq;
  a.split_tiles = split_tiles;
  a.split_base = 0;
  const unsigned grid_main = paged_grid(num_tiles, num_splits), grid_side = paged_grid(num_tiles, side_splits);
  if (grid_main == 0 || grid_side == 0) return (int)hipErrorInvalidValue;
  a.num_tiles = num_tiles;
  hipLaunchKernelGGL(paged_prefill_kernel<false>, dim3(grid_main), dim3(512), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  a.split_tiles = side_split_tiles;
  a.split_base = num_splits;
  hipLaunchKernelGGL(paged_prefill_kernel<true>, dim3(grid_side), dim3(512), 0, stream, a);
  err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  hipLaunchKernelGGL(paged_merge_kernel, dim3(num_tokens, kHeadsQ / 8), dim3(256), 0, stream, a, total);
  return (int)hipGetLastError();
}

}  // extern "C"
