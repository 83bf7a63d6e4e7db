// Split-KV GQA decode attention over a per-group abridged paged KV cache (gfx950).
//
// Replaces the decode call the reference's vLLM overlay makes through the stock FlashInfer backend
// (BatchDecodeWithPagedKVCache; metadata built in third_party/vllm_overlay/vllm/v1/worker/gpu_model_runner.py:
// 1872-1887, 2184-2276) and the pure-torch consumer PackedKVSidecar._attend_decode_batched
// (third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:564-616). Under physical per-layer quotas a
// decode step needs no mask (gpu_model_runner.py:2042-2050): compaction already left each group's rows
// contiguous as [prompt rows | q_l code rows per closed block | open block], so the kernel attends over physical
// slots [0, seq_len) of the group's page table.
//
// Work decomposition: four workgroups of 2 waves per (sequence, split), each for two KV heads; a wave owns one KV
// head and its 4 query heads.
// A split covers `split_pages` pages; the wave walks it 32 slots (two pages) at a time:
//   S^T[32 slots x 16 cols] = K_tile . Q^T          two row tiles x 4 MFMA 16x16x32 (cols 0..3 = the 4 q heads)
//   online softmax in fp32 (exp2 domain), per-head max shared across the 4 lane groups by two xor shuffles
//   O^T[128 dims x 16 cols] += V^T . P^T            8 MFMA 16x16x32, V transposed in registers with v_perm
// Operand layouts are chosen so that every global load is a 16-byte load straight into MFMA operand registers
// (no LDS): for QK a lane loads 16 B of one slot's K row; for PV a lane loads 16 B (8 dims) of 8 slots' V rows and
// an 8x8 bf16 transpose in registers produces the 8 V^T operands. The slot order inside the PV contraction is
// picked so that the S^T accumulator registers of a lane are exactly its P^T operand (no cross-lane movement).
//
// Output: normalised bf16 out [B, 32, 128] and natural-log LSE [B, 32] directly when a sequence has one split;
// otherwise per split a normalised fp16 partial output with an fp32 record (m, l, scale), and a merge kernel (fp16
// partials move half the bytes of fp32 ones: 2.1 % of the saturated launch time).
#include "abridgekv_amd.h"
#include "common.h"

#include <mutex>

namespace abkv {

struct DecodeArgs {
  const __bf16* q;           // [B, 32, 128] (strides q_sb, q_sh in elements; dims contiguous)
  long q_sb, q_sh;
  const __bf16* kv;          // [num_pages, 2, 16, 8, 128]
  const int32_t* block_table;  // [B, bt_stride]
  long bt_stride;
  const int32_t* seq_lens;   // [B]
  int split_pages;           // pages per split (even)
  int max_splits;
  int max_pages;             // bound on pages per sequence (<= block-table width); longer sequences are clamped
  int num_pages;             // pages in the cache; page ids are clamped into [0, num_pages)
  float scale_log2;          // softmax scale * log2(e)
  __bf16* out;               // [B, 32, 128] (strides o_sb, o_sh)
  long o_sb, o_sh;
  float* lse;                // [B, 32] or nullptr
  _Float16* part_o;          // [B, part_stride, 32, 128] fp16: split output / (l * scale)
  float* part_ml;            // [B, part_stride, 32, 4] fp32: m (log2 units), l, scale, unused
  int part_stride;           // split slots per sequence in the partial buffers (max_splits, + side splits)
  int force_partials;        // write partials even for one split (the side rows are merged in afterwards)
  // Side rows (per-head packed code pages; unused when side_count is null): packed page p of a sequence holds, for
  // KV head h, rows side_o[h] .. side_o[h] + side_q[h] - 1 of a [2][side_rows][128] page in side_kv.
  const __bf16* side_kv;     // [side_pool_pages, 2, side_rows, 128]
  int side_rows;
  int side_pool_pages;
  const int32_t* side_table; // [B, side_stride] packed page ids per sequence
  long side_stride;
  const int32_t* side_count; // [B] packed pages per sequence
  int side_max_pages;        // bound on side_count
  int side_split_rows;       // side rows per split and head (multiple of 32, <= 63 * min quota)
  int side_q[kHeadsKV], side_o[kHeadsKV];
};

__device__ __forceinline__ u32x4 ld16(const __bf16* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// K/V rows: every byte is read by exactly one wave of one launch and a decode step streams far more rows than any
// cache holds, so the loads are non-temporal (no allocation in L2 / the last-level cache). Same-process A/B over the
// same pages, outputs bit-identical: saturated B=256 1723.8 -> 1687.4 us; full-model B=64 groups q64 143.5 -> 141.0,
// q128 236.4 -> 224.8, q256 426.3 -> 412.1 us.
__device__ __forceinline__ u32x4 ld16_stream(const __bf16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  const _Float16 x = (_Float16)lo, y = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, x) | ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
}

// Largest |o| over the 128 dims of this lane's column (the lane groups j hold dims 32j .. 32j + 31).
__device__ __forceinline__ float column_absmax(const floatx4 (&o)[8]) {
  float x = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) x = fmaxf(x, fabsf(o[i][r]));
  return max_xor32(max_xor16(x));
}

// Split partial of one query head: the split's output normalised by its weight sum l, stored in fp16 (11-bit
// mantissa, half the bytes of fp32), divided by a scale that keeps every value within +-32768 (1 unless the split's
// V rows exceed that), and the record (m, l, scale). o[i][r] = un-normalised out[dim 32j + 8r + i]; amax =
// column_absmax(o).
__device__ __forceinline__ void store_partial(const DecodeArgs& a, long slot, int head, int j, const floatx4 (&o)[8],
                                              float amax, float m_run, float l_tot) {
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  const float an = amax * inv;
  const float scale = an > 32768.f ? an * (1.f / 32768.f) : 1.f;
  const float f = inv / scale;
  _Float16* po = a.part_o + (slot * kHeadsQ + head) * kHeadDim + 32 * j;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    u32x4 w;
#pragma unroll
    for (int c = 0; c < 4; ++c) w[c] = pack_f16x2(o[2 * c][r] * f, o[2 * c + 1][r] * f);
    *reinterpret_cast<u32x4*>(po + 8 * r) = w;
  }
  if (j == 0)
    *reinterpret_cast<floatx4*>(a.part_ml + (slot * kHeadsQ + head) * 4) = floatx4{m_run, l_tot, scale, 0.f};
}

template <int kW>
__global__ __launch_bounds__(64 * kW) void decode_attn_kernel(DecodeArgs a) {
  // Grid (max_splits * 8 / kW, B): kW waves per workgroup, wave = KV head; the 8 / kW workgroups of a split are
  // adjacent in x. Split fastest (dispatch order: the splits of sequence 0, then of sequence 1, ...), measured faster
  // than sequence-fastest orders on the saturated workload.
  const int b = blockIdx.y;
  constexpr int kParts = kHeadsKV / kW;
  const int split = blockIdx.x / kParts;
  const int kvh = (int)(blockIdx.x % kParts) * kW + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int m16 = lane & 15;                  // MFMA row/col index of this lane
  const int j = lane >> 4;                    // lane group (k-chunk index)

  const int seq_len = max(min(a.seq_lens[b], a.max_pages * kPage), 0);
  const int n_pages = (seq_len + kPage - 1) / kPage;
  const int n_splits = max(1, (n_pages + a.split_pages - 1) / a.split_pages);
  if (split >= n_splits) return;
  const int pg_begin = split * a.split_pages;
  const int pg_end = min(n_pages, pg_begin + a.split_pages);
  const int row_end = seq_len;                                       // rows of this split: [pg_begin*16, row_end)
  const int32_t* bt = a.block_table + (long)b * a.bt_stride;

  // Q^T operand: lane supplies q[head m16][dims 8*(4i+j) .. +8] for MFMA i (zero for the 12 padding columns).
  bf16x8 qop[4];
  {
    const __bf16* qh = a.q + (long)b * a.q_sb + (long)(kvh * kGroup + min(m16, kGroup - 1)) * a.q_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 v = ld16(qh + 8 * (4 * i + j));
      if (m16 >= kGroup) v = u32x4{0, 0, 0, 0};
      qop[i] = __builtin_bit_cast(bf16x8, v);
    }
  }

  floatx4 o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;   // running max of this lane's head (log2 domain), identical across the lane group
  float l_run = 0.f;         // partial row sum over this lane's slots

  // Page ids of the split, fetched once: lane l holds page pg_begin + l (clamped into the cache); the loop reads them
  // with readlane, so no page-table load sits between one chunk's compute and the next chunk's K/V loads.
  int pid_l = 0;
  if (lane < pg_end - pg_begin) pid_l = min(max(bt[pg_begin + lane], 0), a.num_pages - 1);
  const __bf16* kv_h = a.kv + kvh * kHeadDim;
  for (int pg = pg_begin; pg < pg_end; pg += 2) {
    const int p0 = __builtin_amdgcn_readlane(pid_l, pg - pg_begin);
    const int p1 = __builtin_amdgcn_readlane(pid_l, min(pg + 1, pg_end - 1) - pg_begin);
    const __bf16* base0 = kv_h + (long)p0 * kPageElems;
    const __bf16* base1 = kv_h + (long)p1 * kPageElems;

    // K tiles: tile t row m16 = slot 16t + m16 of page p_t; lane loads dims 8*(4i+j)..+8 for MFMA i.
    u32x4 kr[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kr[0][i] = ld16_stream(base0 + m16 * kSlotElems + 8 * (4 * i + j));
      kr[1][i] = ld16_stream(base1 + m16 * kSlotElems + 8 * (4 * i + j));
    }
    // V rows: contraction index e<4 -> slot 4j+e of p0, e>=4 -> slot 4j+e-4 of p1; lane loads dims 8*m16..+8.
    u32x4 vr[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vr[e] = ld16_stream(base0 + kHalfElems + (4 * j + e) * kSlotElems + 8 * m16);
      vr[4 + e] = ld16_stream(base1 + kHalfElems + (4 * j + e) * kSlotElems + 8 * m16);
    }

    floatx4 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) s[t] = mfma16x16x32(__builtin_bit_cast(bf16x8, kr[t][i]), qop[i], s[t]);
    }
    // s[t][r] = score of slot pg*16 + 16t + 4j + r for head m16.
    const bool tail = (pg + 2) * kPage > row_end;
    float sv[8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = s[t][r] * a.scale_log2;
        if (tail) {
          const int slot = pg * kPage + 16 * t + 4 * j + r;
          x = slot < row_end ? x : -INFINITY;
        }
        sv[4 * t + r] = x;
      }
    if (tail) {
      // Rows past the split may hold stale bytes: zero their V contribution (0 * NaN would poison the MFMA).
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int slot = pg * kPage + (e < 4 ? 0 : 16) + 4 * j + (e & 3);
        if (slot >= row_end) vr[e] = u32x4{0, 0, 0, 0};
      }
    }
    float mx = sv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
    mx = max_xor16(mx);
    mx = max_xor32(mx);
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sv[e] = fast_exp2(sv[e] - m_new);
      psum += sv[e];
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= alpha;

    u32x4 pw;
    pw[0] = pack_bf16x2(sv[0], sv[1]);
    pw[1] = pack_bf16x2(sv[2], sv[3]);
    pw[2] = pack_bf16x2(sv[4], sv[5]);
    pw[3] = pack_bf16x2(sv[6], sv[7]);
    const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);

    // 8x8 transpose: vt[i] dword k = (V[slot e=2k][dim 8*m16+i], V[slot e=2k+1][dim 8*m16+i]).
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u32x4 lo, hi;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        lo[k] = __builtin_amdgcn_perm(vr[2 * k + 1][c], vr[2 * k][c], 0x05040100u);
        hi[k] = __builtin_amdgcn_perm(vr[2 * k + 1][c], vr[2 * k][c], 0x07060302u);
      }
      o[2 * c] = mfma16x16x32(__builtin_bit_cast(bf16x8, lo), pop, o[2 * c]);
      o[2 * c + 1] = mfma16x16x32(__builtin_bit_cast(bf16x8, hi), pop, o[2 * c + 1]);
    }
  }

  // o[i][r] = un-normalised out[head m16][dim 32j + 8r + i]; l_run partial over this lane's slots.
  const float l_tot = sum_xor32(sum_xor16(l_run));
  const bool partial = n_splits > 1 || a.force_partials;
  const float amax = partial ? column_absmax(o) : 0.f;    // (a uniform branch: all lanes take part in the shuffles)
  if (m16 >= kGroup) return;
  const int head = kvh * kGroup + m16;
  if (!partial) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    __bf16* oh = a.out + (long)b * a.o_sb + (long)head * a.o_sh + 32 * j;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      u32x4 w;
#pragma unroll
      for (int c = 0; c < 4; ++c) w[c] = pack_bf16x2(o[2 * c][r] * inv, o[2 * c + 1][r] * inv);
      *reinterpret_cast<u32x4*>(oh + 8 * r) = w;
    }
    if (a.lse != nullptr && j == 0)
      a.lse[(long)b * kHeadsQ + head] = l_tot > 0.f ? (m_run + __log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
  } else {
    store_partial(a, (long)b * a.part_stride + split, head, j, o, amax, m_run, l_tot);
  }
}

// Side splits of sequence b for KV head h (0 without side rows): its packed pages times the head's quota, in split
// rows.
__device__ __forceinline__ int side_splits(const DecodeArgs& a, int b, int h) {
  if (a.side_count == nullptr) return 0;
  const int count = min(max(a.side_count[b], 0), a.side_max_pages);
  return (count * a.side_q[h] + a.side_split_rows - 1) / a.side_split_rows;
}

// The two values of v held by lanes l and l ^ 16 (resp. l ^ 32), in an order fixed by the lane (the same for every
// call, so pairing several variables through these keeps them matched).
__device__ __forceinline__ void pair_xor16(float v, float& x, float& y) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair_xor32(float v, float& x, float& y) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  x = __uint_as_float(r[0]);
  y = __uint_as_float(r[1]);
}

// Online-softmax state of a merge lane: running max M (log2 units), weight sum L, weighted output dims acc.
struct MergeState {
  float M, L, acc[8];
};

// Combine the states of lane pairs {l, l ^ 16} (kXor32 = false) or {l, l ^ 32}: symmetric in the two states.
template <bool kXor32>
__device__ __forceinline__ void merge_pair(MergeState& st) {
  auto pair = [](float v, float& x, float& y) {
    if constexpr (kXor32) pair_xor32(v, x, y);
    else pair_xor16(v, x, y);
  };
  float mx, my, lx, ly;
  pair(st.M, mx, my);
  pair(st.L, lx, ly);
  const float mn = fmaxf(mx, my);
  const float ax = mx == -INFINITY ? 0.f : fast_exp2(mx - mn);
  const float ay = my == -INFINITY ? 0.f : fast_exp2(my - mn);
  st.M = mn;
  st.L = lx * ax + ly * ay;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float x, y;
    pair(st.acc[i], x, y);
    st.acc[i] = x * ax + y * ay;
  }
}

// Merge the split partials of every sequence with more than one split (main splits at slots [0, n_main), side splits
// at [max_splits, max_splits + n_side)). Workgroup (sequence, group of 4 heads), one wave per head; the wave's four
// 16-lane groups g take the splits k = g, g + 4, ... (lane c of a group: dims 8c .. 8c + 7, one 16-byte load per
// split), each keeping a running max, and the four states are combined with two cross-lane swaps.
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
  const int b = blockIdx.x;
  const int seq_len = max(min(a.seq_lens[b], a.max_pages * kPage), 0);
  const int n_pages = (seq_len + kPage - 1) / kPage;
  const int n_main = max(1, (n_pages + a.split_pages - 1) / a.split_pages);
  if (!a.force_partials && n_main <= 1) return;
  const int head = 4 * blockIdx.y + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int g = lane >> 4, c = lane & 15;
  const int n_side = side_splits(a, b, head / kGroup);
  const int n_all = n_main + n_side;
  const float* pml = a.part_ml + ((long)b * a.part_stride * kHeadsQ + head) * 4;
  const _Float16* pob = a.part_o + ((long)b * a.part_stride * kHeadsQ + head) * kHeadDim + 8 * c;
  // split k of the n_all: main split k, or side split k - n_main at slot max_splits + (k - n_main)
  auto slot = [&](int k) { return k < n_main ? k : a.max_splits + (k - n_main); };
  MergeState st;
  st.M = -INFINITY;
  st.L = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) st.acc[i] = 0.f;
#pragma unroll 4
  for (int k = g; k < n_all; k += 4) {
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    const long s = slot(k);
    const floatx4 rec = *reinterpret_cast<const floatx4*>(pml + s * kHeadsQ * 4);     // m, l, scale
    const f16x8 h = *reinterpret_cast<const f16x8*>(pob + s * kHeadsQ * kHeadDim);
    const float mn = fmaxf(st.M, rec[0]);
    const float alpha = mn == -INFINITY ? 1.f : fast_exp2(st.M - mn);
    const float w = mn == -INFINITY ? 0.f : fast_exp2(rec[0] - mn) * rec[1];    // the split's weight
    const float ws = w * rec[2];
    st.L = st.L * alpha + w;
#pragma unroll
    for (int i = 0; i < 8; ++i) st.acc[i] = st.acc[i] * alpha + (float)h[i] * ws;
    st.M = mn;
  }
  merge_pair<false>(st);
  merge_pair<true>(st);
  if (g != 0) return;
  const float inv = st.L > 0.f ? 1.f / st.L : 0.f;
  u32x4 wv;
#pragma unroll
  for (int i = 0; i < 4; ++i) wv[i] = pack_bf16x2(st.acc[2 * i] * inv, st.acc[2 * i + 1] * inv);
  *reinterpret_cast<u32x4*>(a.out + (long)b * a.o_sb + (long)head * a.o_sh + 8 * c) = wv;
  if (a.lse != nullptr && c == 0)
    a.lse[(long)b * kHeadsQ + head] = st.L > 0.f ? (st.M + __log2f(st.L)) * 0.69314718055994531f : -INFINITY;
}

// Attention of each sequence's 32 query heads over its side rows (per-head packed code pages; the reference keeps
// them as PackedKVSidecar pages, third_party/vllm_overlay/vllm/v1/worker/compresslm_packed_kv.py:242-270, and
// attends them ahead of the paged rows, :564-616). Grid (side split, KV head h, B), one wave per workgroup (heads
// hold different row counts, so waves of one workgroup would idle): head h's rows are r = 0 .. count * q_h - 1, row
// r being row side_o[h] + r % q_h of packed page r / q_h of the sequence. A split covers side_split_rows rows, 32
// rows per step with the decode kernel's operand layout; partials go to slot max_splits + split.
__global__ __launch_bounds__(64) void decode_side_kernel(DecodeArgs a) {
  const int b = blockIdx.z;
  const int split = blockIdx.x;
  const int kvh = blockIdx.y;
  if (split >= side_splits(a, b, kvh)) return;
  const int lane = threadIdx.x & 63;
  const int m16 = lane & 15;
  const int j = lane >> 4;
  const int count = min(max(a.side_count[b], 0), a.side_max_pages);
  const int qh = a.side_q[kvh], oh = a.side_o[kvh];
  const int r_begin = split * a.side_split_rows;
  const int r_end = min(count * qh, r_begin + a.side_split_rows);

  bf16x8 qop[4];
  {
    const __bf16* qp = a.q + (long)b * a.q_sb + (long)(kvh * kGroup + min(m16, kGroup - 1)) * a.q_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 v = ld16(qp + 8 * (4 * i + j));
      if (m16 >= kGroup) v = u32x4{0, 0, 0, 0};
      qop[i] = __builtin_bit_cast(bf16x8, v);
    }
  }
  floatx4 o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_run = 0.f;

  // Packed page ids of the split: lane l holds page p0 + l; the split's rows of this head lie in at most 64 pages
  // (side_split_rows <= 63 * quota). Row r -> page r / q_h by a float reciprocal: exact while r < 2^21 (the distance
  // of (r + 0.5) / q_h to an integer, 0.5 / q_h, exceeds the rounding error r / q_h * 2^-22).
  const int p0 = r_begin / qh;
  int pid_l = 0;
  if (p0 + lane < count) pid_l = min(max(a.side_table[(long)b * a.side_stride + p0 + lane], 0), a.side_pool_pages - 1);
  const float inv_q = 1.f / (float)qh;
  const long page_elems = 2L * a.side_rows * kHeadDim;
  const __bf16* base_h = a.side_kv + (long)oh * kHeadDim;
  auto row_ptr = [&](int r) -> const __bf16* {
    const int p = (int)(((float)r + 0.5f) * inv_q);
    const int slot = r - p * qh;
    const int pid = __shfl(pid_l, p - p0, 64);
    return base_h + (long)pid * page_elems + slot * kHeadDim;
  };
  const long v_off = (long)a.side_rows * kHeadDim;

  for (int c0 = r_begin; c0 < r_end; c0 += 32) {
    // With q_h >= 32 the chunk's 32 rows lie in pages pa and pa + 1: both ids by readlane (scalar) and a select per
    // row; smaller quotas look each row's page up across lanes.
    const int pa = (int)(((float)c0 + 0.5f) * inv_q);
    const int pid_a = __builtin_amdgcn_readlane(pid_l, min(pa - p0, 63));
    const int pid_b = __builtin_amdgcn_readlane(pid_l, min(pa + 1 - p0, 63));
    const int bound = (pa + 1) * qh;
    auto chunk_row_ptr = [&](int r) -> const __bf16* {
      if (qh < 32) return row_ptr(r);
      const bool second = r >= bound;
      const int slot = r - (second ? bound : pa * qh);
      return base_h + (long)(second ? pid_b : pid_a) * page_elems + slot * kHeadDim;
    };
    // rows past r_end read row r_end - 1 instead (finite data; their weight is exactly 0)
    u32x4 kr[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const __bf16* kp = chunk_row_ptr(min(c0 + 16 * t + m16, r_end - 1));
#pragma unroll
      for (int i = 0; i < 4; ++i) kr[t][i] = ld16_stream(kp + 8 * (4 * i + j));
    }
    // V rows: contraction index e < 4 -> row c0 + 4j + e, e >= 4 -> row c0 + 16 + 4j + e - 4; dims 8*m16 .. +8
    u32x4 vr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      vr[e] = ld16_stream(chunk_row_ptr(min(c0 + (e < 4 ? 0 : 16) + 4 * j + (e & 3), r_end - 1)) + v_off + 8 * m16);

    floatx4 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) s[t] = mfma16x16x32(__builtin_bit_cast(bf16x8, kr[t][i]), qop[i], s[t]);
    }
    float sv[8];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) sv[4 * t + r] = c0 + 16 * t + 4 * j + r < r_end ? s[t][r] * a.scale_log2 : -INFINITY;
    float mx = sv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
    mx = max_xor16(mx);
    mx = max_xor32(mx);
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sv[e] = fast_exp2(sv[e] - m_new);
      psum += sv[e];
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] *= alpha;
    u32x4 pw;
    pw[0] = pack_bf16x2(sv[0], sv[1]);
    pw[1] = pack_bf16x2(sv[2], sv[3]);
    pw[2] = pack_bf16x2(sv[4], sv[5]);
    pw[3] = pack_bf16x2(sv[6], sv[7]);
    const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u32x4 lo, hi;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        lo[k] = __builtin_amdgcn_perm(vr[2 * k + 1][c], vr[2 * k][c], 0x05040100u);
        hi[k] = __builtin_amdgcn_perm(vr[2 * k + 1][c], vr[2 * k][c], 0x07060302u);
      }
      o[2 * c] = mfma16x16x32(__builtin_bit_cast(bf16x8, lo), pop, o[2 * c]);
      o[2 * c + 1] = mfma16x16x32(__builtin_bit_cast(bf16x8, hi), pop, o[2 * c + 1]);
    }
  }

  const float l_tot = sum_xor32(sum_xor16(l_run));
  const float amax = column_absmax(o);
  if (m16 >= kGroup) return;
  store_partial(a, (long)b * a.part_stride + a.max_splits + split, kvh * kGroup + m16, j, o, amax, m_run, l_tot);
}

// Two waves (two KV heads) per workgroup: the four workgroups of a split are adjacent in dispatch order. Measured in
// one process over the same pages: two waves 952.9 us per launch against four 959.1 and eight 990.5 on the saturated
// B=256 workload, 241.5 against 245.1 and 254.7 on the B=64 full-model decode; one wave 4 % slower than four.
inline void launch_decode(const DecodeArgs& a, int max_splits, int num_seqs, hipStream_t stream) {
  constexpr int kW = 2;
  hipLaunchKernelGGL(decode_attn_kernel<kW>, dim3(max_splits * (kHeadsKV / kW), num_seqs), dim3(64 * kW), 0, stream,
                     a);
}

// Static split-partial scratch of abkv_decode_attn_noalloc: part of the library image, so every GPU the library runs
// on holds its own copy from module load until the process ends, and no call allocates. Host code must never pass
// the array's name to a kernel (on the host it is only a stand-in for the symbol): the device address comes from
// hipGetSymbolAddress, fetched once per device with that device current.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch` (nullptr and *err set when the lookup fails).
static void* scratch_ptr(hipError_t* err) {
  int dev = -1;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    *err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (*err != hipSuccess) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace abkv

extern "C" {

// Workspace bytes needed by abkv_decode_attn for `num_seqs` sequences and `max_splits` splits per sequence.
size_t abkv_decode_workspace_size(int num_seqs, int max_splits) {
  const size_t per = (size_t)abkv::kHeadsQ * (abkv::kHeadDim * sizeof(_Float16) + 4 * sizeof(float));
  return (size_t)num_seqs * (size_t)max_splits * per;
}

int abkv_decode_attn(const void* q, long q_stride_seq, long q_stride_head,
                     const void* kv_cache, int num_pages, const int32_t* block_table, long block_table_stride,
                     const int32_t* seq_lens, int num_seqs, int max_pages_per_seq, int split_pages,
                     float scale, void* out, long out_stride_seq, long out_stride_head, float* lse,
                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  using namespace abkv;
  if (num_seqs <= 0) return 0;
  if (split_pages <= 0 || (split_pages & 1) || split_pages > 64 || max_pages_per_seq <= 0 || num_pages <= 0 ||
      block_table_stride < max_pages_per_seq)
    return (int)hipErrorInvalidValue;
  if (q == nullptr || kv_cache == nullptr || block_table == nullptr || seq_lens == nullptr || out == nullptr)
    return (int)hipErrorInvalidValue;
  const int max_splits = (max_pages_per_seq + split_pages - 1) / split_pages;
  if (max_splits > 1 && (workspace == nullptr || workspace_bytes < abkv_decode_workspace_size(num_seqs, max_splits)))
    return (int)hipErrorInvalidValue;
  DecodeArgs a;
  a.q = static_cast<const __bf16*>(q);
  a.q_sb = q_stride_seq;
  a.q_sh = q_stride_head;
  a.kv = static_cast<const __bf16*>(kv_cache);
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.seq_lens = seq_lens;
  a.split_pages = split_pages;
  a.max_splits = max_splits;
  a.max_pages = max_pages_per_seq;
  a.num_pages = num_pages;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = static_cast<__bf16*>(out);
  a.o_sb = out_stride_seq;
  a.o_sh = out_stride_head;
  a.lse = lse;
  a.part_o = static_cast<_Float16*>(workspace);
  a.part_ml = reinterpret_cast<float*>(a.part_o + (size_t)num_seqs * max_splits * kHeadsQ * kHeadDim);
  a.part_stride = max_splits;
  a.force_partials = 0;
  a.side_count = nullptr;
  launch_decode(a, max_splits, num_seqs, stream);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  if (max_splits > 1) {
    hipLaunchKernelGGL(decode_merge_kernel, dim3(num_seqs, kHeadsQ / 4), dim3(256), 0, stream, a);
    err = hipGetLastError();
  }
  return (int)err;
}

// abkv_decode_attn with the split partials in the library's static scratch (no workspace argument, no allocation).
int abkv_decode_attn_noalloc(const void* q, long q_stride_seq, long q_stride_head, const void* kv_cache,
                             int num_pages, const int32_t* block_table, long block_table_stride,
                             const int32_t* seq_lens, int num_seqs, int max_pages_per_seq, int split_pages,
                             float scale, void* out, long out_stride_seq, long out_stride_head, float* lse,
                             hipStream_t stream) {
  using namespace abkv;
  if (num_seqs <= 0) return 0;
  if (split_pages <= 0 || (split_pages & 1) || split_pages > 64 || max_pages_per_seq <= 0)
    return (int)hipErrorInvalidValue;
  const int max_splits = (max_pages_per_seq + split_pages - 1) / split_pages;
  size_t need = 0;
  void* ws = nullptr;
  if (max_splits > 1) {
    need = abkv_decode_workspace_size(num_seqs, max_splits);
    if (need > kNoAllocScratchBytes) return ABKV_ERR_SCRATCH;
    hipError_t err = hipSuccess;
    ws = scratch_ptr(&err);
    if (ws == nullptr) return (int)err;
  }
  return abkv_decode_attn(q, q_stride_seq, q_stride_head, kv_cache, num_pages, block_table, block_table_stride,
                          seq_lens, num_seqs, max_pages_per_seq, split_pages, scale, out, out_stride_seq,
                          out_stride_head, lse, ws, need, stream);
}

// Side rows per split and head for a packed layout whose smallest head quota is q_min (multiple of 32, at most
// 63 * q_min so that a split's rows of any head lie in at most 64 packed pages, at most 512).
int abkv_decode_side_split_rows(int q_min) {
  if (q_min <= 0) return 0;
  const int r = (63 * q_min / 32) * 32;
  return r < 32 ? 32 : (r > 512 ? 512 : r);
}

// Workspace bytes for abkv_decode_attn_packed: partials of (main splits + side splits) per sequence.
size_t abkv_decode_packed_workspace_size(int num_seqs, int max_pages_per_seq, int split_pages, int max_side_pages,
                                         int side_q_max, int side_split_rows) {
  if (num_seqs <= 0 || split_pages <= 0 || side_split_rows <= 0) return 0;
  const int main_splits = (max_pages_per_seq + split_pages - 1) / split_pages;
  const int side = (max_side_pages * side_q_max + side_split_rows - 1) / side_split_rows;
  return abkv_decode_workspace_size(num_seqs, main_splits + side);
}

int abkv_decode_attn_packed(const void* q, long q_stride_seq, long q_stride_head, const void* kv_cache, int num_pages,
                            const int32_t* block_table, long block_table_stride, const int32_t* seq_lens,
                            int num_seqs, int max_pages_per_seq, int split_pages, const void* packed_kv,
                            int packed_pool_pages, int packed_rows, const int32_t* head_quota,
                            const int32_t* packed_table, long packed_table_stride, const int32_t* packed_count,
                            int max_packed_per_seq, int side_split_rows, float scale, void* out, long out_stride_seq,
                            long out_stride_head, float* lse, void* workspace, size_t workspace_bytes,
                            hipStream_t stream) {
  using namespace abkv;
  if (num_seqs <= 0) return 0;
  if (split_pages <= 0 || (split_pages & 1) || split_pages > 64 || max_pages_per_seq <= 0 || num_pages <= 0 ||
      block_table_stride < max_pages_per_seq)
    return (int)hipErrorInvalidValue;
  if (q == nullptr || kv_cache == nullptr || block_table == nullptr || seq_lens == nullptr || out == nullptr ||
      packed_kv == nullptr || packed_table == nullptr || packed_count == nullptr || head_quota == nullptr ||
      packed_pool_pages <= 0 || max_packed_per_seq < 0 || packed_table_stride < max_packed_per_seq)
    return (int)hipErrorInvalidValue;
  // head quotas (host array): each in [1, 2048], rows = their sum
  int qmin = 1 << 30, qmax = 0, rows = 0;
  DecodeArgs a;
  for (int h = 0; h < kHeadsKV; ++h) {
    const int qh = head_quota[h];
    if (qh <= 0 || qh > 2048) return (int)hipErrorInvalidValue;
    a.side_q[h] = qh;
    a.side_o[h] = rows;
    rows += qh;
    qmin = qh < qmin ? qh : qmin;
    qmax = qh > qmax ? qh : qmax;
  }
  if (rows != packed_rows || side_split_rows <= 0 || (side_split_rows & 31) || side_split_rows > 63 * qmin ||
      (long)max_packed_per_seq * qmax >= (1L << 21))
    return (int)hipErrorInvalidValue;
  const int max_splits = (max_pages_per_seq + split_pages - 1) / split_pages;
  const int side_max = (max_packed_per_seq * qmax + side_split_rows - 1) / side_split_rows;
  const int stride = max_splits + side_max;
  if (workspace == nullptr || workspace_bytes < abkv_decode_workspace_size(num_seqs, stride))
    return (int)hipErrorInvalidValue;
  a.q = static_cast<const __bf16*>(q);
  a.q_sb = q_stride_seq;
  a.q_sh = q_stride_head;
  a.kv = static_cast<const __bf16*>(kv_cache);
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.seq_lens = seq_lens;
  a.split_pages = split_pages;
  a.max_splits = max_splits;
  a.max_pages = max_pages_per_seq;
  a.num_pages = num_pages;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = static_cast<__bf16*>(out);
  a.o_sb = out_stride_seq;
  a.o_sh = out_stride_head;
  a.lse = lse;
  a.part_o = static_cast<_Float16*>(workspace);
  a.part_ml = reinterpret_cast<float*>(a.part_o + (size_t)num_seqs * stride * kHeadsQ * kHeadDim);
  a.part_stride = stride;
  a.force_partials = 1;
  a.side_kv = static_cast<const __bf16*>(packed_kv);
  a.side_rows = packed_rows;
  a.side_pool_pages = packed_pool_pages;
  a.side_table = packed_table;
  a.side_stride = packed_table_stride;
  a.side_count = packed_count;
  a.side_max_pages = max_packed_per_seq;
  a.side_split_rows = side_split_rows;
  launch_decode(a, max_splits, num_seqs, stream);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  if (side_max > 0) {
    hipLaunchKernelGGL(decode_side_kernel, dim3(side_max, kHeadsKV, num_seqs), dim3(64), 0, stream, a);
    err = hipGetLastError();
    if (err != hipSuccess) return (int)err;
  }
  hipLaunchKernelGGL(decode_merge_kernel, dim3(num_seqs, kHeadsQ / 4), dim3(256), 0, stream, a);
  return (int)hipGetLastError();
}

}  // extern "C"
