// KV-cache row movement for block-boundary compaction, KV append and slot mapping (gfx950).
//
// Compaction executor: replaces GPUModelRunner._execute_kv_copy_operations / _execute_kv_copy_group
// (third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:1147-1224), which applies one ordered batch of
// (src_block, src_off, dst_block, dst_off) ops per KV-cache group with gather-then-scatter semantics to every layer
// tensor of the group. Here one launch takes up to two op lists and applies them to up to kMaxLayers layer tensors:
// ordered *segments* (one per request run whose ops depend on each other's order) and *independent* ops.
//
// Exactness without a staging buffer: a workgroup walks an ordered segment in op order, kMoveRows ops at a time,
// loading every source row of the chunk into registers, then (after a barrier) storing every destination row, then
// a barrier. This equals gather-then-scatter, for any chunk size, whenever no op of the segment reads a slot that an
// EARLIER op of the same segment writes (a later op may overwrite a slot an earlier op read: that read has happened)
// -- true for compaction ops, which are emitted in increasing source order with dst < src
// (single_type_kv_cache_manager.py:378-381) -- and no two ops write one slot. Segments must touch disjoint pages
// (different requests' pages are disjoint; one request contributes one segment per batch). Independent ops read and
// write no slot that another op of the launch writes (a request run in which no op's destination is another op's
// source: the planner's fused moves of a run whose shift is at least its length), so they run in any order and any
// split. For op lists that violate the ordering precondition the two-phase gather/scatter entry points below stage
// rows through a workspace instead.
//
// KV append: replaces the stock vLLM compiled op reshape_and_cache(_flash) that writes each new token's K and V
// rows at slot_mapping[t] (slots from block_table.py:186-197); slot < 0 is skipped (padding).
#include "common.h"

namespace abkv {

constexpr int kMaxLayers = 16;
constexpr int kMoveRows = 64;     // ordered segments: ops per chunk, 64 rows x 1 KiB (one byte part) in flight
constexpr int kMoveParts = 4;     // ordered segments: workgroups per (segment, layer), one quarter of every row each
constexpr int kFreeRows = 4;      // independent ops: ops (whole rows) per workgroup

struct LayerPtrs {
  char* p[kMaxLayers];
};

// Row moves read every moved byte once and write it once, far more bytes per step than any cache holds: streaming
// (non-temporal) loads and stores, which leave L2 and the last-level cache alone. Same-process A/B of the 64-sequence
// step (six group launches), bytes bit-identical: 490.7 -> 446.9 us (4.92 -> 5.41 TB/s). The hint changes where lines
// are kept, not the order of the accesses: every load and store is issued where it was, and the launch's ordering
// argument (no op reads a slot that an earlier op of its segment writes; independent ops touch no slot another op
// writes) does not depend on caching.
__device__ __forceinline__ u32x4 ld16_stream(const char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16_stream(char* p, const u32x4& v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

struct MoveArgs {
  LayerPtrs layers;
  const int32_t* ops;          // [n_ops, 4] (src_block, src_off, dst_block, dst_off)
  const int32_t* seg_offsets;  // [n_seg + 1]
  long page_bytes;             // bytes of one page of one layer (2 * block_size * slot_bytes)
  long half_bytes;             // offset of the V half inside a page
  int slot_bytes;              // bytes of one slot of K (or V), multiple of 16
  int num_pages;               // pages per layer cache: ops outside [0, num_pages) x [0, block_size) are skipped
  int block_size;
};

__device__ __forceinline__ bool op_ok(const int32_t* op, int num_pages, int block_size) {
  return (unsigned)op[0] < (unsigned)num_pages && (unsigned)op[2] < (unsigned)num_pages &&
         (unsigned)op[1] < (unsigned)block_size && (unsigned)op[3] < (unsigned)block_size;
}

// One "row" of an op = slot_bytes of K plus slot_bytes of V (4 KiB in the served geometry). One launch moves two
// kinds of op lists, each workgroup taking one kind (blockIdx.x below n_ordered_wgs: ordered segments, first in
// dispatch order since they are the longest; above: independent ops).
//  Ordered segment (move_ordered): kMoveParts workgroups per (segment, layer), adjacent in dispatch order, each owning
//    one byte part of the rows (byte parts of a row never interact). The workgroup walks its segment kMoveRows ops at
//    a time: lane l of every wave fetches op c0 + l once per chunk, the row offsets are broadcast with readlane
//    (wave-uniform), wave w moves rows w, w+4, ..., lane l the l-th 16-byte vector of the part; the 16 source loads
//    of a thread issue back to back and land in registers before the barrier, the 16 stores follow it.
//  Independent ops (move_free): no op reads or writes a slot another op of the list writes, so any split and order
//    is exact; a workgroup moves kFreeRows consecutive ops as whole rows (consecutive ops are mostly consecutive slots
//    of one page, so the workgroup reads and writes kFreeRows x 2 KiB contiguous runs of K and of V), thread t the
//    t-th 16-byte vector of every row, kFreeRows loads back to back, then the stores.
// Ordered segment, software-pipelined: the op fetch and source loads of chunk c + 1 are issued before the stores of
// chunk c (a later op never reads a slot an earlier op writes, so those loads may run ahead of the stores), and the
// stores of chunk c + 1 follow the barrier that closes its loads. One memory round trip per chunk on the critical
// path instead of two.
struct OrderedChunk {
  long soff[kMoveRows / 4], doff[kMoveRows / 4];
  u32x4 buf[kMoveRows / 4];
};

__device__ __forceinline__ void ordered_fetch(const MoveArgs& a, int c0, int s1, int wave, int lane, OrderedChunk& ch) {
  const int n = min(kMoveRows, s1 - c0);
  int o0 = -1, o1 = -1, o2 = -1, o3 = -1;                 // lane l: op c0 + l
  if (lane < n) {
    const int32_t* op = a.ops + 4L * (c0 + lane);
    o0 = op[0];
    o1 = op[1];
    o2 = op[2];
    o3 = op[3];
  }
  const bool ok_l = lane < n && (unsigned)o0 < (unsigned)a.num_pages && (unsigned)o2 < (unsigned)a.num_pages &&
                    (unsigned)o1 < (unsigned)a.block_size && (unsigned)o3 < (unsigned)a.block_size;
  const unsigned long long ok_mask = __ballot(ok_l);
  // wave-uniform byte offsets of this wave's rows (invalid rows read slot 0 of page 0 and store nothing)
#pragma unroll
  for (int k = 0; k < kMoveRows / 4; ++k) {
    const int r = wave + 4 * k;                            // < 64: a lane of this wave
    const bool ok = (ok_mask >> r) & 1ull;
    ch.soff[k] = ok ? (long)__builtin_amdgcn_readlane(o0, r) * a.page_bytes +
                          (long)__builtin_amdgcn_readlane(o1, r) * a.slot_bytes : 0;
    ch.doff[k] = ok ? (long)__builtin_amdgcn_readlane(o2, r) * a.page_bytes +
                          (long)__builtin_amdgcn_readlane(o3, r) * a.slot_bytes : -1;
  }
}

__device__ __forceinline__ void move_ordered(const MoveArgs& a, char* base, int seg, int part) {
  const int s0 = a.seg_offsets[seg], s1 = a.seg_offsets[seg + 1];
  const int row_vec = (2 * a.slot_bytes) / 16;          // 16-byte vectors per row
  const int vpp = (row_vec + kMoveParts - 1) / kMoveParts;   // vectors per part
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (s0 >= s1) return;
  for (int u0 = 0; u0 < vpp; u0 += 64) {                  // one round in the served geometry (vpp = 64)
    const int u = u0 + lane;
    const int v = part * vpp + u;
    const bool active = u < vpp && v < row_vec;
    const int half = v >= row_vec / 2;                     // 0: K, 1: V
    const long inner = active ? (long)half * a.half_bytes + (long)(v - half * (row_vec / 2)) * 16 : 0;
    OrderedChunk cur, nxt;
    ordered_fetch(a, s0, s1, wave, lane, cur);
#pragma unroll
    for (int k = 0; k < kMoveRows / 4; ++k) cur.buf[k] = ld16_stream(base + cur.soff[k] + inner);
    for (int c0 = s0; c0 < s1; c0 += kMoveRows) {
      const bool more = c0 + kMoveRows < s1;
      if (more) ordered_fetch(a, c0 + kMoveRows, s1, wave, lane, nxt);
      // every source row of chunk c is in registers before any wave stores it (a store may hit a slot another wave
      // of the chunk reads); this also completes the op fetch of chunk c + 1
      __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (more) {
#pragma unroll
        for (int k = 0; k < kMoveRows / 4; ++k)
          nxt.buf[k] = ld16_stream(base + nxt.soff[k] + inner);
      }
#pragma unroll
      for (int k = 0; k < kMoveRows / 4; ++k)
        if (cur.doff[k] >= 0 && active) st16_stream(base + cur.doff[k] + inner, cur.buf[k]);
      cur = nxt;
    }
  }
}

__device__ __forceinline__ void move_free(const MoveArgs& a, const int32_t* __restrict__ free_ops, char* base, int i0,
                                          int i1) {
  // the workgroup's ops, read once before any store (uniform addresses, nothing written before them: scalar loads)
  long sb[kFreeRows], db[kFreeRows];
#pragma unroll
  for (int r = 0; r < kFreeRows; ++r) {
    const int i = i0 + r;
    const int32_t* op = free_ops + 4L * i;
    const bool ok = i < i1 && op_ok(op, a.num_pages, a.block_size);
    sb[r] = ok ? (long)op[0] * a.page_bytes + (long)op[1] * a.slot_bytes : 0;
    db[r] = ok ? (long)op[2] * a.page_bytes + (long)op[3] * a.slot_bytes : -1;
  }
  const int row_vec = (2 * a.slot_bytes) / 16;
  for (int v = threadIdx.x; v < row_vec; v += 256) {
    const int half = v >= row_vec / 2;
    const long inner = (long)half * a.half_bytes + (long)(v - half * (row_vec / 2)) * 16;
    u32x4 buf[kFreeRows];
#pragma unroll
    for (int r = 0; r < kFreeRows; ++r) buf[r] = ld16_stream(base + sb[r] + inner);
#pragma unroll
    for (int r = 0; r < kFreeRows; ++r)
      if (db[r] >= 0) st16_stream(base + db[r] + inner, buf[r]);
  }
}

// free_ops is its own argument (not an offset read from seg_offsets): an independent-op workgroup lives for a few
// memory round trips, and a dependent load before its op fetch would add one.
__global__ __launch_bounds__(256) void kv_move_kernel(MoveArgs a, int n_ordered_wgs,
                                                      const int32_t* __restrict__ free_ops, int n_free) {
  char* base = a.layers.p[blockIdx.y];
  const int x = blockIdx.x;
  if (x < n_ordered_wgs) {
    move_ordered(a, base, x / kMoveParts, x % kMoveParts);
  } else {
    const int i0 = (x - n_ordered_wgs) * kFreeRows;
    move_free(a, free_ops, base, i0, min(i0 + kFreeRows, n_free));
  }
}

// Two-phase form for arbitrary op lists: gather every source row into `stage` [n_layers, n_ops, row], then scatter.
__global__ __launch_bounds__(256) void kv_gather_kernel(MoveArgs a, char* stage, int n_ops) {
  const int op_i = blockIdx.x;
  const int layer = blockIdx.y;
  const char* base = a.layers.p[layer];
  const int row_vec = (2 * a.slot_bytes) / 16;
  const int32_t* op = a.ops + 4L * op_i;
  if (!op_ok(op, a.num_pages, a.block_size)) return;
  char* out = stage + ((long)layer * n_ops + op_i) * (2L * a.slot_bytes);
  for (int v = threadIdx.x; v < row_vec; v += 256) {
    const int half = v >= row_vec / 2;
    const long inner = (long)half * a.half_bytes + (long)(v - half * (row_vec / 2)) * 16;
    *reinterpret_cast<u32x4*>(out + 16L * v) =
        *reinterpret_cast<const u32x4*>(base + (long)op[0] * a.page_bytes + (long)op[1] * a.slot_bytes + inner);
  }
}

__global__ __launch_bounds__(256) void kv_scatter_kernel(MoveArgs a, const char* stage, int n_ops) {
  const int op_i = blockIdx.x;
  const int layer = blockIdx.y;
  char* base = a.layers.p[layer];
  const int row_vec = (2 * a.slot_bytes) / 16;
  const int32_t* op = a.ops + 4L * op_i;
  if (!op_ok(op, a.num_pages, a.block_size)) return;
  const char* in = stage + ((long)layer * n_ops + op_i) * (2L * a.slot_bytes);
  for (int v = threadIdx.x; v < row_vec; v += 256) {
    const int half = v >= row_vec / 2;
    const long inner = (long)half * a.half_bytes + (long)(v - half * (row_vec / 2)) * 16;
    *reinterpret_cast<u32x4*>(base + (long)op[2] * a.page_bytes + (long)op[3] * a.slot_bytes + inner) =
        *reinterpret_cast<const u32x4*>(in + 16L * v);
  }
}

// KV append: one workgroup of 256 threads per token; thread moves 16 B of K or V.
__global__ __launch_bounds__(256) void kv_append_kernel(const char* key, long k_stride, const char* value,
                                                       long v_stride, const int64_t* slot_mapping, char* cache,
                                                       long page_bytes, long half_bytes, int slot_bytes,
                                                       int block_size, long num_pages) {
  const int t = blockIdx.x;
  const long slot = slot_mapping[t];
  if (slot < 0 || slot >= num_pages * block_size) return;
  const long page = slot / block_size, off = slot % block_size;
  const int vecs = slot_bytes / 16;
  for (int v = threadIdx.x; v < 2 * vecs; v += 256) {
    const int half = v >= vecs;
    const int w = v - half * vecs;
    const char* src = (half ? value + (long)t * v_stride : key + (long)t * k_stride) + 16L * w;
    char* dst = cache + page * page_bytes + (long)half * half_bytes + off * slot_bytes + 16L * w;
    *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
  }
}

// Fused rotary embedding + KV append for the served geometry (32 query / 8 KV heads, head size 128, NeoX halves):
// q[t] rotated in place, key[t] rotated in place and, with value[t], written to the cache at slot_mapping[t].
// Replaces the model-side rotary op plus reshape_and_cache of the overlay's attention path, and computes the RoPE
// position of an abridged-layout token on the device when block_c > 0 (logical position of period block_c +
// codes_k -> block * block_c + (offset < block_c ? offset : bitrev code offset over the code span, block_c minus a
// static retained tail), config/compresslm.py:192-216).
struct RopeArgs {
  __bf16* q; long q_st, q_sh;                  // [T, 32, 128]
  __bf16* k; long k_st;                        // [T, 8, 128] (heads contiguous)
  const __bf16* v; long v_st;                  // [T, 8, 128]
  const int64_t* positions;                    // [T]
  const float* cos_sin;                        // [max_pos, 128]: cos of the 64 frequencies, then sin
  long max_pos;
  int block_c, codes_k, log2_k;                // block_c == 0: positions are RoPE positions already
  int code_span;                               // code rows spread over in-block offsets [0, code_span)
  const int64_t* slot_mapping;                 // [T] or nullptr (rotate only); < 0 or past the cache = skip
  __bf16* cache; long num_pages;
};

__device__ __forceinline__ long rope_position(const RopeArgs& a, long pos) {
  if (pos < 0) pos = 0;
  if (a.block_c > 0) {
    const long per = a.block_c + a.codes_k;
    const long blk = pos / per;
    const int w = (int)(pos - blk * per);
    long off = w;
    if (w >= a.block_c) {
      const unsigned k = (unsigned)(w - a.block_c);
      const unsigned rev = a.log2_k > 0 ? (__brev(k) >> (32 - a.log2_k)) : 0u;
      off = ((long)rev * a.code_span) / a.codes_k;
    }
    pos = blk * a.block_c + off;
  }
  return pos < a.max_pos ? pos : a.max_pos - 1;
}

// One workgroup per token: 512 q units + 128 k units of 4 rotation pairs (dims 4g..4g+3 with 64+4g..64+4g+3).
__global__ __launch_bounds__(256) void rope_append_kernel(RopeArgs a) {
  const int t = blockIdx.x;
  const long pos = rope_position(a, a.positions[t]);
  const float* cs = a.cos_sin + pos * kHeadDim;
  long slot = a.slot_mapping ? a.slot_mapping[t] : -1;
  if (slot >= a.num_pages * kPage) slot = -1;
  __bf16* kv_slot = slot >= 0 ? a.cache + (slot / kPage) * kPageElems + (slot % kPage) * kSlotElems : nullptr;
  for (int u = threadIdx.x; u < (kHeadsQ + kHeadsKV) * 16; u += 256) {
    const bool isq = u < kHeadsQ * 16;
    const int uu = isq ? u : u - kHeadsQ * 16;
    const int h = uu >> 4, g = uu & 15;
    __bf16* row = isq ? a.q + (long)t * a.q_st + (long)h * a.q_sh : a.k + (long)t * a.k_st + h * kHeadDim;
    const u32x2 x1w = *reinterpret_cast<const u32x2*>(row + 4 * g);
    const u32x2 x2w = *reinterpret_cast<const u32x2*>(row + 64 + 4 * g);
    const floatx4 c = *reinterpret_cast<const floatx4*>(cs + 4 * g);
    const floatx4 sn = *reinterpret_cast<const floatx4*>(cs + 64 + 4 * g);
    float x1[4], x2[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      x1[2 * i] = __uint_as_float(x1w[i] << 16);
      x1[2 * i + 1] = __uint_as_float(x1w[i] & 0xffff0000u);
      x2[2 * i] = __uint_as_float(x2w[i] << 16);
      x2[2 * i + 1] = __uint_as_float(x2w[i] & 0xffff0000u);
    }
    u32x2 o1, o2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      o1[i] = pack_bf16x2(x1[2 * i] * c[2 * i] - x2[2 * i] * sn[2 * i],
                          x1[2 * i + 1] * c[2 * i + 1] - x2[2 * i + 1] * sn[2 * i + 1]);
      o2[i] = pack_bf16x2(x2[2 * i] * c[2 * i] + x1[2 * i] * sn[2 * i],
                          x2[2 * i + 1] * c[2 * i + 1] + x1[2 * i + 1] * sn[2 * i + 1]);
    }
    *reinterpret_cast<u32x2*>(row + 4 * g) = o1;
    *reinterpret_cast<u32x2*>(row + 64 + 4 * g) = o2;
    if (!isq && kv_slot != nullptr) {
      *reinterpret_cast<u32x2*>(kv_slot + h * kHeadDim + 4 * g) = o1;
      *reinterpret_cast<u32x2*>(kv_slot + h * kHeadDim + 64 + 4 * g) = o2;
    }
  }
  if (kv_slot != nullptr && threadIdx.x < kSlotElems / 8) {      // V row: 128 x 16 B
    const int i = threadIdx.x;
    *reinterpret_cast<u32x4*>(kv_slot + kHalfElems + 8 * i) =
        *reinterpret_cast<const u32x4*>(a.v + (long)t * a.v_st + 8 * i);
  }
}

// slot_mapping[t] = table[req[t]][pos[t] / block_size] * block_size + pos[t] % block_size; -1 for a negative
// position or one past the table (pos >= width * block_size) or a request index outside [0, num_reqs).
__global__ void slot_mapping_kernel(const int32_t* req_idx, const int64_t* positions, const int32_t* block_table,
                                    int num_reqs, long bt_stride, int block_size, const int32_t* compacted,
                                    int64_t* slots, int n) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const int r = req_idx[t];
  if (r < 0 || r >= num_reqs) {
    slots[t] = -1;
    return;
  }
  const long pos = positions[t] - (compacted != nullptr ? compacted[r] : 0);   // logical -> physical in the group
  if (pos < 0 || pos >= bt_stride * block_size) {
    slots[t] = -1;
    return;
  }
  const long blk = block_table[(long)req_idx[t] * bt_stride + pos / block_size];
  slots[t] = blk * block_size + pos % block_size;
}

static bool fill_layers(LayerPtrs& lp, void* const* layer_caches, int n_layers) {
  if (n_layers <= 0 || n_layers > kMaxLayers) return false;
  for (int i = 0; i < kMaxLayers; ++i) lp.p[i] = i < n_layers ? static_cast<char*>(layer_caches[i]) : nullptr;
  for (int i = 0; i < n_layers; ++i)
    if (lp.p[i] == nullptr) return false;
  return true;
}

// Per-head packed code pages (reference: PackedKVLayout.pack_layer + PackedKVSidecar.capture,
// third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:112-128, 259-284): the K_max code rows of a closed
// block, read from the paged cache, are stored as one packed page per layer, [2][rows_l][128] with head h's first
// q_lh code rows at rows off_lh .. off_lh + q_lh - 1 (off = running sum of the quotas over the heads).
struct CaptureArgs {
  const void* const* layer_kv;   // [L] paged caches [num_pages, 2, 16, 8, 128]
  void* const* layer_pool;       // [L] packed pools [pool_pages, 2, rows_l, 128]
  const int32_t* layer_rows;     // [L] rows_l = sum of the layer's head quotas
  const int32_t* layer_quota;    // [L, 8]
  const int32_t* block_table;    // [n, bt_stride] page table row of each capture's sequence
  long bt_stride;
  int bt_width;
  const int32_t* code_start;     // [n] physical position of the block's first code row
  const int32_t* dst_page;       // [n] packed page receiving the capture
  int num_pages, pool_pages;
};

// Grid (capture, layer), 256 threads; thread t moves 16-byte chunk t % 32 (K chunks 0-15, V chunks 16-31) of packed
// rows t / 32, t / 32 + 8, ...
__global__ __launch_bounds__(256) void packed_capture_kernel(CaptureArgs a) {
  const int c = blockIdx.x, l = blockIdx.y;
  const int rows = a.layer_rows[l];
  const int32_t* quota = a.layer_quota + l * kHeadsKV;
  const __bf16* kv = static_cast<const __bf16*>(a.layer_kv[l]);
  __bf16* pool = static_cast<__bf16*>(a.layer_pool[l]);
  const int start = a.code_start[c];
  const int dst = min(max(a.dst_page[c], 0), a.pool_pages - 1);
  const int32_t* bt = a.block_table + (long)c * a.bt_stride;
  const int part = threadIdx.x & 31, half = part >> 4, chunk = part & 15;
  for (int row = threadIdx.x >> 5; row < rows; row += 8) {
    int h = 0, off = 0;
#pragma unroll
    for (int k = 0; k < kHeadsKV - 1; ++k) {   // head of packed row `row`: off_h <= row < off_h + q_h
      if (row >= off + quota[h]) {
        off += quota[h];
        ++h;
      }
    }
    const int pos = start + (row - off);
    const int page = min(max(bt[min(pos >> 4, a.bt_width - 1)], 0), a.num_pages - 1);
    const __bf16* src = kv + (long)page * kPageElems + half * kHalfElems + (pos & 15) * kSlotElems + h * kHeadDim +
                        8 * chunk;
    __bf16* d = pool + ((long)dst * 2 + half) * rows * kHeadDim + (long)row * kHeadDim + 8 * chunk;
    *reinterpret_cast<u32x4*>(d) = *reinterpret_cast<const u32x4*>(src);
  }
}


// Expansion of the run descriptors of abkv_planner_take_move_runs into the move lists abkv_planner_take_moves_packed
// writes (same positions, same values). Workgroup r < n_runs takes run r: final row i of the run (relative to its
// first row) came from row f(i) = i + c[J(i)], J(i) = the thresholds tau <= i; rows [t_star, n) move. Row i's op is
// ordered when it reads a row the run writes (i in A = [t_star, a_end)) or writes a row the run reads (i in B =
// f(A)); its rank among the run's ordered ops is |A before i| + |B before i| - |A n B before i|, all three read off
// the monotone map, and independent ops take the remaining ranks in row order. Workgroups past n_runs write each
// group's first segment offset (0) and padding. Every store is checked against the run's counts and out_elems, every
// page read against the run's window and the window against the n_pages entries of `pages`; negative positions,
// rows and offsets are skipped. A record that disagrees with the map therefore writes nothing out of place and reads
// nothing outside its inputs.
constexpr int kRunRemovalsMax = 8;
constexpr int kRunFields = 14 + 2 * kRunRemovalsMax;

__global__ __launch_bounds__(256) void moves_expand_kernel(const int32_t* __restrict__ runs, int n_runs,
                                                           const int32_t* __restrict__ pages, long n_pages,
                                                           const int32_t* __restrict__ groups, int page_shift,
                                                           int32_t* __restrict__ out, long out_elems) {
  const int r = blockIdx.x;
  if (r >= n_runs) {
    const int32_t* gr = groups + 4 * (r - n_runs);
    const int offs_at = gr[0], n_seg = gr[1], pad_end = gr[2];
    if (offs_at < 0 || n_seg < 0) return;
    if (threadIdx.x == 0 && offs_at < out_elems) out[offs_at] = 0;
    for (long k = (long)offs_at + 1 + n_seg + threadIdx.x; k < pad_end && k < out_elems; k += blockDim.x) out[k] = 0;
    return;
  }
  const int32_t* rec = runs + (long)kRunFields * r;
  const int n = rec[0], lo_w = rec[1], pages_at = rec[2], ord_at = rec[3], free_at = rec[4], n_ch = rec[5];
  const int n_free = rec[6], seg_at = rec[7], seg_val = rec[8], m = rec[9], t_star = rec[10], a_end = rec[11];
  const int win_n = rec[12];
  if (pages_at < 0 || win_n < 0 || (long)pages_at + win_n > n_pages) return;   // window outside `pages`
  int tau[kRunRemovalsMax], c[kRunRemovalsMax];
#pragma unroll
  for (int j = 0; j < kRunRemovalsMax; ++j) {
    tau[j] = rec[14 + j];
    c[j] = rec[14 + kRunRemovalsMax + j];
  }
  if (threadIdx.x == 0 && seg_at >= 0 && seg_at < out_elems) out[seg_at] = seg_val;
  auto f = [&](int x) {
    int add = 0;
#pragma unroll
    for (int j = 0; j < kRunRemovalsMax; ++j) add = (j < m && x >= tau[j]) ? c[j] : add;
    return x + add;
  };
  auto inv = [&](int y) {                        // smallest x >= 0 with f(x) >= y
    int x = max(0, y);
    bool found = m == 0 || x < tau[0];
#pragma unroll
    for (int j = 1; j <= kRunRemovalsMax; ++j) {
      if (found || j > m) break;
      const int cand = max(tau[j - 1], y - c[j - 1]);
      if (j == m || (j < kRunRemovalsMax && cand < tau[j])) {
        x = cand;
        found = true;
      }
    }
    return x;
  };
  const int mask = (1 << page_shift) - 1;
  for (int i = t_star + (int)threadIdx.x; i < n; i += blockDim.x) {
    const int src = lo_w + f(i), dst = lo_w + i;
    const int gi = inv(i);
    const bool ordered = i < a_end || (gi >= t_star && gi < a_end && f(gi) == i);
    const int cnt_a = min(i - t_star, a_end - t_star);
    const int cnt_b = max(0, min(a_end, gi) - t_star);
    const int cnt_ab = max(0, min(a_end, inv(min(i, a_end))) - t_star);
    const int rank = cnt_a + cnt_b - cnt_ab;
    long pos;
    if (ordered) {
      if (rank < 0 || rank >= n_ch) continue;
      pos = (long)ord_at + 4L * rank;
    } else {
      const int fr = i - t_star - rank;
      if (fr < 0 || fr >= n_free) continue;
      pos = (long)free_at + 4L * fr;
    }
    const int sp = src >> page_shift, dp = dst >> page_shift;
    if (pos < 0 || pos + 4 > out_elems || src < 0 || dst < 0 || sp >= win_n || dp >= win_n) continue;
    int32_t* o = out + pos;
    o[0] = pages[pages_at + sp];
    o[1] = src & mask;
    o[2] = pages[pages_at + dp];
    o[3] = dst & mask;
  }
}

}  // namespace abkv

extern "C" {

int abkv_kv_move_mixed(void* const* layer_caches, int n_layers, int num_pages, int block_size, long page_bytes,
                       long half_bytes, int slot_bytes, const int32_t* ops, const int32_t* seg_offsets, int n_segments,
                       const int32_t* free_ops, int n_free, hipStream_t stream) {
  using namespace abkv;
  if (n_segments < 0 || n_free < 0) return (int)hipErrorInvalidValue;
  if (n_segments == 0 && n_free == 0) return 0;
  if ((n_segments > 0 && (ops == nullptr || seg_offsets == nullptr)) || (n_free > 0 && free_ops == nullptr) ||
      slot_bytes <= 0 || slot_bytes % 16 != 0)
    return (int)hipErrorInvalidValue;
  const long wgs = (long)n_segments * kMoveParts + (n_free + kFreeRows - 1) / kFreeRows;
  if (wgs > 0x7FFFFFFFL) return (int)hipErrorInvalidValue;
  MoveArgs a;
  if (!fill_layers(a.layers, layer_caches, n_layers)) return (int)hipErrorInvalidValue;
  a.ops = ops;
  a.seg_offsets = seg_offsets;
  a.page_bytes = page_bytes;
  a.half_bytes = half_bytes;
  a.slot_bytes = slot_bytes;
  a.num_pages = num_pages;
  a.block_size = block_size;
  hipLaunchKernelGGL(kv_move_kernel, dim3((unsigned)wgs, n_layers), dim3(256), 0, stream, a, n_segments * kMoveParts,
                     free_ops, n_free);
  return (int)hipGetLastError();
}

int abkv_kv_move_segments(void* const* layer_caches, int n_layers, int num_pages, int block_size, long page_bytes,
                          long half_bytes, int slot_bytes, const int32_t* ops, const int32_t* seg_offsets,
                          int n_segments, hipStream_t stream) {
  if (n_segments <= 0) return 0;
  return abkv_kv_move_mixed(layer_caches, n_layers, num_pages, block_size, page_bytes, half_bytes, slot_bytes, ops,
                            seg_offsets, n_segments, nullptr, 0, stream);
}

size_t abkv_kv_stage_bytes(int n_layers, int n_ops, int slot_bytes) {
  return (size_t)n_layers * (size_t)n_ops * 2u * (size_t)slot_bytes;
}

int abkv_kv_copy_staged(void* const* layer_caches, int n_layers, int num_pages, int block_size, long page_bytes,
                        long half_bytes, int slot_bytes, const int32_t* ops, int n_ops, void* stage, size_t stage_bytes, hipStream_t stream) {
  using namespace abkv;
  if (n_ops <= 0) return 0;
  if (ops == nullptr || slot_bytes <= 0 || slot_bytes % 16 != 0 ||
      stage == nullptr || stage_bytes < abkv_kv_stage_bytes(n_layers, n_ops, slot_bytes))
    return (int)hipErrorInvalidValue;
  MoveArgs a;
  if (!fill_layers(a.layers, layer_caches, n_layers)) return (int)hipErrorInvalidValue;
  a.ops = ops;
  a.seg_offsets = nullptr;
  a.page_bytes = page_bytes;
  a.half_bytes = half_bytes;
  a.slot_bytes = slot_bytes;
  a.num_pages = num_pages;
  a.block_size = block_size;
  hipLaunchKernelGGL(kv_gather_kernel, dim3(n_ops, n_layers), dim3(256), 0, stream, a, static_cast<char*>(stage),
                     n_ops);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  hipLaunchKernelGGL(kv_scatter_kernel, dim3(n_ops, n_layers), dim3(256), 0, stream, a,
                     static_cast<const char*>(stage), n_ops);
  return (int)hipGetLastError();
}

int abkv_kv_append(const void* key, long key_stride, const void* value, long value_stride,
                   const int64_t* slot_mapping, int num_tokens, void* kv_cache, int num_pages, long page_bytes,
                   long half_bytes, int slot_bytes, int block_size, hipStream_t stream) {
  using namespace abkv;
  if (num_tokens <= 0) return 0;
  if (key == nullptr || value == nullptr || slot_mapping == nullptr || kv_cache == nullptr || slot_bytes % 16 != 0 ||
      block_size <= 0)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(kv_append_kernel, dim3(num_tokens), dim3(256), 0, stream, static_cast<const char*>(key),
                     key_stride, static_cast<const char*>(value), value_stride, slot_mapping,
                     static_cast<char*>(kv_cache), page_bytes, half_bytes, slot_bytes, block_size, (long)num_pages);
  return (int)hipGetLastError();
}

int abkv_rope_kv_append(void* q, long q_stride_t, long q_stride_h, void* key, long key_stride_t, const void* value,
                        long value_stride_t, const int64_t* positions, int num_tokens, int block_c, int codes_k,
                        int code_span, const float* cos_sin, long max_pos, const int64_t* slot_mapping,
                        void* kv_cache, int num_pages, hipStream_t stream) {
  using namespace abkv;
  if (num_tokens <= 0) return 0;
  if (q == nullptr || key == nullptr || value == nullptr || positions == nullptr || cos_sin == nullptr ||
      max_pos <= 0 || block_c < 0 || (slot_mapping != nullptr && (kv_cache == nullptr || num_pages <= 0)))
    return (int)hipErrorInvalidValue;
  int log2_k = 0;
  if (code_span == 0) code_span = block_c;
  if (block_c > 0) {
    if (codes_k <= 0 || (codes_k & (codes_k - 1)) || codes_k > block_c || code_span < codes_k ||
        code_span > block_c)
      return (int)hipErrorInvalidValue;
    while ((1 << log2_k) < codes_k) ++log2_k;
  }
  RopeArgs a;
  a.q = static_cast<__bf16*>(q);
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.k = static_cast<__bf16*>(key);
  a.k_st = key_stride_t;
  a.v = static_cast<const __bf16*>(value);
  a.v_st = value_stride_t;
  a.positions = positions;
  a.cos_sin = cos_sin;
  a.max_pos = max_pos;
  a.block_c = block_c;
  a.codes_k = codes_k;
  a.log2_k = log2_k;
  a.code_span = code_span;
  a.slot_mapping = slot_mapping;
  a.cache = static_cast<__bf16*>(kv_cache);
  a.num_pages = num_pages;
  hipLaunchKernelGGL(rope_append_kernel, dim3(num_tokens), dim3(256), 0, stream, a);
  return (int)hipGetLastError();
}

int abkv_slot_mapping(const int32_t* req_idx, const int64_t* positions, int num_tokens, const int32_t* block_table,
                      int num_reqs, long block_table_stride, int block_size, const int32_t* compacted,
                      int64_t* slot_mapping, hipStream_t stream) {
  if (num_tokens <= 0) return 0;
  if (req_idx == nullptr || positions == nullptr || block_table == nullptr || slot_mapping == nullptr ||
      block_size <= 0)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(abkv::slot_mapping_kernel, dim3((num_tokens + 255) / 256), dim3(256), 0, stream, req_idx,
                     positions, block_table, num_reqs, block_table_stride, block_size, compacted, slot_mapping,
                     num_tokens);
  return (int)hipGetLastError();
}

int abkv_packed_capture(const void* const* layer_kv, void* const* layer_pool, const int32_t* layer_rows,
                        const int32_t* layer_quota, int num_layers, int num_pages, int pool_pages,
                        const int32_t* block_table, long block_table_stride, int block_table_width,
                        const int32_t* code_start, const int32_t* dst_page, int num_captures, hipStream_t stream) {
  using namespace abkv;
  if (num_captures <= 0 || num_layers <= 0) return 0;
  if (layer_kv == nullptr || layer_pool == nullptr || layer_rows == nullptr || layer_quota == nullptr ||
      block_table == nullptr || code_start == nullptr || dst_page == nullptr || num_pages <= 0 || pool_pages <= 0 ||
      block_table_width <= 0 || block_table_stride < block_table_width)
    return (int)hipErrorInvalidValue;
  CaptureArgs a;
  a.layer_kv = layer_kv;
  a.layer_pool = layer_pool;
  a.layer_rows = layer_rows;
  a.layer_quota = layer_quota;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.bt_width = block_table_width;
  a.code_start = code_start;
  a.dst_page = dst_page;
  a.num_pages = num_pages;
  a.pool_pages = pool_pages;
  hipLaunchKernelGGL(packed_capture_kernel, dim3(num_captures, num_layers), dim3(256), 0, stream, a);
  return (int)hipGetLastError();
}

// Device half of the planner's fused moves: the run descriptors of abkv_planner_take_move_runs (runs [n_runs, 30]
// int32, their page windows, groups [num_groups, 4]) expanded into `out` (out_elems = sizes[2] of that call), the
// move lists abkv_planner_take_moves_packed would write for the same step. page_shift = log2 of the page size.
int abkv_moves_expand(const int32_t* runs, int n_runs, const int32_t* pages, long n_pages, const int32_t* groups,
                      int num_groups, int page_shift, int32_t* out, long out_elems, hipStream_t stream) {
  using namespace abkv;
  if (n_runs < 0 || n_pages < 0 || num_groups < 0 || page_shift < 0 || page_shift > 16 || out_elems < 0)
    return (int)hipErrorInvalidValue;
  if (n_runs + num_groups == 0) return 0;
  if ((n_runs > 0 && (runs == nullptr || pages == nullptr)) || (num_groups > 0 && groups == nullptr) || out == nullptr)
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(moves_expand_kernel, dim3(n_runs + num_groups), dim3(256), 0, stream, runs, n_runs, pages,
                     n_pages, groups, page_shift, out, out_elems);
  return (int)hipGetLastError();
}

}  // extern "C"
