// Shared attention tile machinery for the masked-prefill and paged-prefill kernels (gfx950).
//
// A workgroup stages 64-key K/V tiles in double-buffered LDS (global_load_lds_dwordx4, XOR-swizzled 256-byte rows)
// and each wave attends 16 query rows x H heads (MFMA columns) against them with v_mfma_f32_16x16x32_bf16:
//   S^T[32 keys x 16H cols] = K . Q^T, online softmax in the exp2 domain (lazy rescale), O^T += V^T . P^T.
#pragma once
#include "common.h"

namespace abkv {

constexpr int kBM = 64;                  // query rows per workgroup
constexpr int kBN = 64;                  // keys per tile
constexpr int kTileElems = kBN * kHeadDim;

// Per-element visibility for layouts whose tiles cannot be classified (unaligned masked prefill); other kernels
// never call it (their tiles are always aligned: kAligned = true).
struct MaskGeom {
  int qrow, S0, C, per, plen;
  const int* quota;        // per head of the KV group
  __device__ __forceinline__ bool visible(int kv, int head) const {
    if (kv >= S0 || qrow >= S0) return false;
    const int qb = qrow / per, kb = kv / per;
    const int qw = qrow - qb * per, kw = kv - kb * per;
    const bool kc = kw < C;
    bool v = (kc && kb == qb) || (!kc && kb < qb) || (kc && kb * C + kw < plen);
    v = v && kv <= qrow;
    v = v || (qw >= C && !kc && kb == qb);
    return v && (kc || kw - C < quota[head]);
  }
};

__device__ __forceinline__ u32x4 ld16g(const __bf16* p) { return *reinterpret_cast<const u32x4*>(p); }

#define ABKV_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// K/V tiles live in LDS as 64 rows x 256 B without padding; 16-byte chunk c of row r is stored at chunk c ^ (r % 16),
// which makes both operand read patterns conflict-free (16 lanes hit 16 distinct chunks). Tiles are filled with
// global_load_lds_dwordx4: a wave instruction writes 1 KiB contiguously (lane L -> bytes 16L), so each lane fetches
// the global chunk that belongs at its swizzled position. Rows past the sequence end re-read the last row (finite data,
// masked to probability 0).
// Row addressing of a contiguous [S, heads, 128] K/V pair (one KV head selected by the base pointers).
struct DenseRows {
  const __bf16* k;
  const __bf16* v;
  long k_ss, v_ss;
  __device__ __forceinline__ const __bf16* krow(int key) const { return k + (long)key * k_ss; }
  __device__ __forceinline__ const __bf16* vrow(int key) const { return v + (long)key * v_ss; }
};

// Row addressing of one sequence in the paged cache [pages, 2, 16, 8, 128] (one KV head): physical slot -> page.
struct PagedRows {
  const __bf16* kv;        // cache base + kvh * 128
  const int32_t* table;    // the sequence's page-table row
  int width;               // entries in the row
  int num_pages;
  __device__ __forceinline__ const __bf16* krow(int key) const {
    const int page = min(max(table[min(key >> 4, width - 1)], 0), num_pages - 1);
    return kv + (long)page * kPageElems + (key & 15) * kSlotElems;
  }
  __device__ __forceinline__ const __bf16* vrow(int key) const { return krow(key) + kHalfElems; }
};

// Fill one K and one V tile of 64 keys (rows >= n_keys re-read row n_keys - 1: finite data, masked to zero weight).
template <int kWaves, class Rows>
__device__ __forceinline__ void issue_tile(const Rows& rows, int k0, int n_keys, __bf16* Kbuf, __bf16* Vbuf, int w,
                                           int lane) {
  constexpr int kPerWave = 16 / kWaves;        // 1 KiB blocks of the 16 KiB K (and V) tile per wave
#pragma unroll
  for (int n = 0; n < kPerWave; ++n) {
    const int blk = kPerWave * w + n;
    const int row = 4 * blk + (lane >> 4);
    const int logical = (lane & 15) ^ (row & 15);
    const int key = min(k0 + row, n_keys - 1);
    __builtin_amdgcn_global_load_lds((const void*)(rows.krow(key) + 8 * logical), ABKV_LDS(Kbuf + 512 * blk), 16,
                                     0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(rows.vrow(key) + 8 * logical), ABKV_LDS(Vbuf + 512 * blk), 16,
                                     0, 0);
  }
}

__device__ __forceinline__ u32x4 lds16(const __bf16* buf, int row, int chunk) {
  return *reinterpret_cast<const u32x4*>(buf + row * kHeadDim + 8 * (chunk ^ (row & 15)));
}

// Eight consecutive output dims (the four of accumulator lo, then the four of hi) times inv, as one 16-byte store.
__device__ __forceinline__ void store_bf16x8(__bf16* dst, const floatx4& lo, const floatx4& hi, float inv) {
  u32x4 wv;
  wv[0] = pack_bf16x2(lo[0] * inv, lo[1] * inv);
  wv[1] = pack_bf16x2(lo[2] * inv, lo[3] * inv);
  wv[2] = pack_bf16x2(hi[0] * inv, hi[1] * inv);
  wv[3] = pack_bf16x2(hi[2] * inv, hi[3] * inv);
  *reinterpret_cast<u32x4*>(dst) = wv;
}

struct TileMask {
  int mode;        // 0 none, 1 key < this lane's limit, 2 key < limit[head], 3 general (per-element arithmetic)
  int limit[4];
};

// V^T operand of one PV MFMA from the swizzled V tile with two ds_read_b64_tr_b16 (LDS transpose reads). Within a
// 16-lane group, lane i of a transpose read receives element i % 4 of the 8-byte chunk addressed by lane
// 4e + i / 4, for e = 0..3. The operand row m of dim slab t is dim 32 * (m / 4) + 4t + m % 4 and its k-index
// 8g + e (g = lane group) is key kb + 4g + e for e < 4 and kb + 16 + 4g + e - 4 for e >= 4 (the contraction order the
// P^T operand uses); so lane 4e + c of the group addresses row kb + 4g + e (then + 16), dims 32c + 4t .. +3.
__device__ __forceinline__ bf16x8 vt_operand(const __bf16* Vbuf, int kb, int t, int lane) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  const int g = lane >> 4, i = lane & 15;
  const int e = i >> 2, c = i & 3;
  const int dim = 32 * c + 4 * t;                   // 8-byte aligned, inside 16-byte chunk dim / 8
  const int row0 = kb + 4 * g + e, row1 = row0 + 16;
  const __bf16* p0 = Vbuf + row0 * kHeadDim + 8 * ((dim >> 3) ^ (row0 & 15)) + (dim & 7);
  const __bf16* p1 = Vbuf + row1 * kHeadDim + 8 * ((dim >> 3) ^ (row1 & 15)) + (dim & 7);
  const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(p0));
  const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4*)(p1));
  typedef short s8 __attribute__((ext_vector_type(8)));
  const s8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// Attention of this wave's 16H columns against one 64-key tile held in (Kbuf, Vbuf): S^T for all 64 keys first
// (the MFMA results of the second half are not needed before the softmax of the first starts), one masked online
// softmax step over the tile, then O^T += V^T . P^T per 32-key half. o[t][u][r] accumulates out dim
// 32 * (lane >> 4) + 4t + r of column (head hbase + u, query row m16).
template <int H, bool kAligned>
__device__ __forceinline__ void tile_compute(const __bf16* Kbuf, const __bf16* Vbuf, const bf16x8 (&qop)[H][4],
                                             floatx4 (&o)[8][H], float (&m_run)[H], float (&l_run)[H], int k0,
                                             const TileMask& tm, int lane_limit, float scale_log2,
                                             const MaskGeom& geo, int hbase, int m16, int j) {
  // every partial tile of an aligned layout is "key < lim[u]" with a per-column limit (per head or per lane)
  int lim[H];
#pragma unroll
  for (int u = 0; u < H; ++u) lim[u] = tm.mode == 1 ? lane_limit : tm.limit[hbase + u];
  // S^T = K . Q^T: s[kk][t][u][r] = raw score of key k0 + 32kk + 16t + 4j + r, column (head u, query row m16)
  floatx4 s[2][2][H];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int u = 0; u < H; ++u) s[kk][t][u] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 kop = __builtin_bit_cast(bf16x8, lds16(Kbuf, 32 * kk + 16 * t + m16, 4 * i + j));
#pragma unroll
        for (int u = 0; u < H; ++u) s[kk][t][u] = mfma16x16x32(kop, qop[u][i], s[kk][t][u]);
      }
  if (tm.mode != 0) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int u = 0; u < H; ++u)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int kv = k0 + 32 * kk + 16 * t + 4 * j + r;
            bool ok;
            if constexpr (kAligned) {
              ok = kv < lim[u];
            } else {
              ok = geo.visible(kv, hbase + u);
            }
            s[kk][t][u][r] = ok ? s[kk][t][u][r] : -INFINITY;
          }
  }
  float tmax[H];
#pragma unroll
  for (int u = 0; u < H; ++u) {
    float mx = -INFINITY;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        mx = fmaxf(mx, fmaxf(fmaxf(s[kk][t][u][0], s[kk][t][u][1]), fmaxf(s[kk][t][u][2], s[kk][t][u][3])));
    mx = max_xor16(mx);
    mx = max_xor32(mx);
    tmax[u] = mx * scale_log2;                          // log2-domain max (scale > 0)
  }
  // lazy rescale: the running max moves only when a column max grows by more than 8 (2^8 headroom in P)
  bool need = false;
#pragma unroll
  for (int u = 0; u < H; ++u) need |= tmax[u] > m_run[u] + 8.f;
  if (__any(need)) {
#pragma unroll
    for (int u = 0; u < H; ++u) {
      const float m_new = fmaxf(m_run[u], tmax[u]);
      const float alpha = fast_exp2(m_run[u] - (m_new == -INFINITY ? 0.f : m_new));
      m_run[u] = m_new;
      l_run[u] *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i][u] *= alpha;
    }
  }
  bf16x8 pop[2][H];
#pragma unroll
  for (int u = 0; u < H; ++u) {
    const float neg_m = m_run[u] == -INFINITY ? 0.f : -m_run[u];
    float ps = 0.f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = fast_exp2(fmaf(s[kk][t][u][r], scale_log2, neg_m));
          s[kk][t][u][r] = p;
          ps += p;
        }
      // P^T operand of half kk: k-index e < 4 -> key 32kk + 4j + e, e >= 4 -> key 32kk + 16 + 4j + e - 4
      u32x4 pw;
      pw[0] = pack_bf16x2(s[kk][0][u][0], s[kk][0][u][1]);
      pw[1] = pack_bf16x2(s[kk][0][u][2], s[kk][0][u][3]);
      pw[2] = pack_bf16x2(s[kk][1][u][0], s[kk][1][u][1]);
      pw[3] = pack_bf16x2(s[kk][1][u][2], s[kk][1][u][3]);
      pop[kk][u] = __builtin_bit_cast(bf16x8, pw);
    }
    l_run[u] += ps;
  }
  // O^T += V^T . P^T, one 32-key half at a time, V^T straight from LDS with transpose reads
  const int lane = 16 * j + m16;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const bf16x8 vop = vt_operand(Vbuf, 32 * kk, t, lane);
#pragma unroll
      for (int u = 0; u < H; ++u) o[t][u] = mfma16x16x32(vop, pop[kk][u], o[t][u]);
    }
}

}  // namespace abkv
