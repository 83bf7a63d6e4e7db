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
// Tile row sources for the DMA. tile_base<kV>(k0, blk) is the (wave-uniform) address that DMA block blk (rows
// 4blk .. 4blk+3 of the tile at key k0) starts from and lane_off(row, chunk) the per-lane element offset from it, so
// a full tile costs no per-tile vector address arithmetic. Rows at or past n_keys are never read (they may lie past
// the tensor, or hold non-finite data that a zero weight would not cancel in P.V): the last tile of a walk takes the
// per-row path, which re-reads row n_keys - 1 in their place (finite data, masked to zero weight).
// Contiguous [S, heads, 128] K/V pair (one KV head selected by the base pointers).
struct DenseRows {
  const __bf16* k;
  const __bf16* v;
  long k_ss, v_ss;
  template <bool kV>
  __device__ __forceinline__ const __bf16* tile_base(int k0, int) const {
    return kV ? v + (long)k0 * v_ss : k + (long)k0 * k_ss;
  }
  template <bool kV>
  __device__ __forceinline__ int lane_off(int row, int chunk) const {
    return row * (int)(kV ? v_ss : k_ss) + 8 * chunk;
  }
  template <bool kV>
  __device__ __forceinline__ const __bf16* row_ptr(int key) const {
    return kV ? v + (long)key * v_ss : k + (long)key * k_ss;
  }
};

// One sequence in the paged cache [pages, 2, 16, 8, 128] (one KV head): a DMA block's 4 rows lie in one page, whose
// id is a wave-uniform load; page-table positions past the row and page ids out of range are clamped.
struct PagedRows {
  const __bf16* kv;        // cache base + kvh * 128
  const int32_t* table;    // the sequence's page-table row
  int width;               // entries in the row
  int num_pages;
  template <bool kV>
  __device__ __forceinline__ const __bf16* tile_base(int k0, int blk) const {
    const int page = min(max(table[min((k0 >> 4) + (blk >> 2), width - 1)], 0), num_pages - 1);
    return kv + (long)page * kPageElems + (kV ? kHalfElems : 0);
  }
  template <bool kV>
  __device__ __forceinline__ int lane_off(int row, int chunk) const {
    return (row & 15) * kSlotElems + 8 * chunk;
  }
  template <bool kV>
  __device__ __forceinline__ const __bf16* row_ptr(int key) const {
    return tile_base<kV>(key & ~15, 0) + (key & 15) * kSlotElems;
  }
};

// Fill the K (kV = false) or V (kV = true) tile of 64 keys at k0. Each wave issues 16 / kWaves DMA instructions (one
// 1 KiB block of the 16 KiB tile each); w must be wave-uniform.
template <int kWaves, bool kV, class Rows>
__device__ __forceinline__ void issue_half(const Rows& rows, int k0, int n_keys, __bf16* buf, int w, int lane) {
  constexpr int kPerWave = 16 / kWaves;
  if (k0 + kBN <= n_keys) {
#pragma unroll
    for (int n = 0; n < kPerWave; ++n) {
      const int blk = kPerWave * w + n;
      const int row = 4 * blk + (lane >> 4);
      const int chunk = (lane & 15) ^ (row & 15);
      const char* base = reinterpret_cast<const char*>(rows.template tile_base<kV>(k0, blk));
      const unsigned off = 2u * (unsigned)rows.template lane_off<kV>(row, chunk);
      __builtin_amdgcn_global_load_lds((const void*)(base + off), ABKV_LDS(buf + 512 * blk), 16, 0, 0);
    }
  } else {
#pragma unroll
    for (int n = 0; n < kPerWave; ++n) {
      const int blk = kPerWave * w + n;
      const int row = 4 * blk + (lane >> 4);
      const int chunk = (lane & 15) ^ (row & 15);
      const __bf16* src = rows.template row_ptr<kV>(min(k0 + row, n_keys - 1)) + 8 * chunk;
      __builtin_amdgcn_global_load_lds((const void*)src, ABKV_LDS(buf + 512 * blk), 16, 0, 0);
    }
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

// Raw scores of one 64-key tile: s[kk][t][u][r] = q(column: head u, query row m16) . k(key k0 + 32kk + 16t + 4j + r),
// S^T = K . Q^T with the K operand read from the swizzled tile (16 ds_read_b128, 8H MFMAs).
template <int H>
__device__ __forceinline__ void tile_scores(const __bf16* Kbuf, const bf16x8 (&qop)[H][4], floatx4 (&s)[2][2][H],
                                            int m16, int j) {
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
}

// Hidden keys of a partial tile get score -inf (tm.mode 0: nothing hidden).
template <int H, bool kAligned>
__device__ __forceinline__ void tile_mask(floatx4 (&s)[2][2][H], int k0, const TileMask& tm, int lane_limit,
                                          const MaskGeom& geo, int hbase, int j) {
  if (tm.mode == 0) return;
  // every partial tile of an aligned layout is "key < lim[u]" with a per-column limit (per head or per lane)
  int lim[H];
#pragma unroll
  for (int u = 0; u < H; ++u) lim[u] = tm.mode == 1 ? lane_limit : tm.limit[hbase + u];
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

// Online-softmax bookkeeping of one tile: column maxima (log2 domain) and the lazy rescale, which moves the running
// max only when a column max grows by more than 8 (P stays below 2^8) and then rescales l and O.
template <int H>
__device__ __forceinline__ void tile_rescale(const floatx4 (&s)[2][2][H], floatx4 (&o)[8][H], float (&m_run)[H],
                                             floatx4 (&lsum)[H], float scale_log2) {
  float tmax[H];
#pragma unroll
  for (int u = 0; u < H; ++u) {
    float mx = fmaxf(fmaxf(s[0][0][u][0], s[0][0][u][1]), fmaxf(s[0][0][u][2], s[0][0][u][3]));
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (kk == 0 && t == 0) continue;
        mx = fmaxf(mx, fmaxf(fmaxf(s[kk][t][u][0], s[kk][t][u][1]), fmaxf(s[kk][t][u][2], s[kk][t][u][3])));
      }
    mx = max_xor16(mx);
    mx = max_xor32(mx);
    tmax[u] = mx * scale_log2;                          // log2-domain max (scale > 0)
  }
  bool need = false;
#pragma unroll
  for (int u = 0; u < H; ++u) need |= tmax[u] > m_run[u] + 8.f;
  if (__any(need)) {
#pragma unroll
    for (int u = 0; u < H; ++u) {
      const float m_new = fmaxf(m_run[u], tmax[u]);
      const float alpha = fast_exp2(m_run[u] - (m_new == -INFINITY ? 0.f : m_new));
      m_run[u] = m_new;
      lsum[u] *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i][u] *= alpha;
    }
  }
}

// Probabilities of one tile as the P^T operands of its two 32-key halves. P^T k-index e < 4 of half kk is key
// 32kk + 4j + e, e >= 4 is key 32kk + 16 + 4j + e - 4 (the order vt_operand reads V in).
template <int H>
__device__ __forceinline__ void tile_probs(const floatx4 (&s)[2][2][H], const float (&m_run)[H], float scale_log2,
                                           bf16x8 (&pop)[2][H]) {
#pragma unroll
  for (int u = 0; u < H; ++u) {
    const float neg_m = m_run[u] == -INFINITY ? 0.f : -m_run[u];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      float p[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) p[t][r] = fast_exp2(fmaf(s[kk][t][u][r], scale_log2, neg_m));
      u32x4 pw;
      pw[0] = pack_bf16x2(p[0][0], p[0][1]);
      pw[1] = pack_bf16x2(p[0][2], p[0][3]);
      pw[2] = pack_bf16x2(p[1][0], p[1][1]);
      pw[3] = pack_bf16x2(p[1][2], p[1][3]);
      pop[kk][u] = __builtin_bit_cast(bf16x8, pw);
    }
  }
}

// O^T += V^T . P^T over one tile: o[t][u][r] accumulates out dim 32 * (lane >> 4) + 4t + r of column (u, m16).
// The row sums ride on the MFMA too: lsum[u] += ones . P^T puts the column's sum of the (bf16) weights in every
// entry, the same weights the output accumulates.
template <int H>
__device__ __forceinline__ void tile_pv(const __bf16* Vbuf, const bf16x8 (&pop)[2][H], floatx4 (&o)[8][H],
                                        floatx4 (&lsum)[H], int lane) {
  typedef short s8 __attribute__((ext_vector_type(8)));
  const bf16x8 ones = __builtin_bit_cast(bf16x8, s8{0x3f80, 0x3f80, 0x3f80, 0x3f80, 0x3f80, 0x3f80, 0x3f80, 0x3f80});
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const bf16x8 vop = vt_operand(Vbuf, 32 * kk, t, lane);
#pragma unroll
      for (int u = 0; u < H; ++u) o[t][u] = mfma16x16x32(vop, pop[kk][u], o[t][u]);
    }
#pragma unroll
    for (int u = 0; u < H; ++u) lsum[u] = mfma16x16x32(ones, pop[kk][u], lsum[u]);
  }
}

// Software-pipelined walk over a query tile's key tiles. Iteration n (tile n's scores already in s_cur):
//   wait for this wave's DMA, barrier (publishes K(n+1), V(n); every wave is done reading K(n), V(n-1))
//   DMA K(n+2) -> K buffer n % 2, V(n+1) -> V buffer (n+1) % 2
//   mask + rescale of tile n; then the scores of tile n+1 (MFMA) interleaved with the probabilities of tile n (VALU),
//   then O += V(n) . P(n).
// Walk::next(kt, tm, first) yields the tiles in order. Rows addresses key rows; keys >= n_keys are never read.
// On return l_run[u] is the full weight sum of column (u, m16) in every lane of the column (o and m_run as above).
template <int H, bool kAligned, int kWaves, class Rows, class Walk>
__device__ __forceinline__ void attend_tiles(const Rows& rows, Walk& walk, int n_keys, __bf16* Kb, __bf16* Vb,
                                             const bf16x8 (&qop)[H][4], floatx4 (&o)[8][H], float (&m_run)[H],
                                             float (&l_run)[H], int lane_limit, float scale_log2,
                                             const MaskGeom& geo, int hbase, int w, int lane) {
  const int m16 = lane & 15, j = lane >> 4;
  int t_cur = 0, t_nxt = 0;
  TileMask tm_cur, tm_nxt;
  if (!walk.next(t_cur, tm_cur, true)) return;
  t_nxt = t_cur;
  bool has_nxt = walk.next(t_nxt, tm_nxt, false);
  issue_half<kWaves, false>(rows, t_cur * kBN, n_keys, Kb, w, lane);
  issue_half<kWaves, true>(rows, t_cur * kBN, n_keys, Vb, w, lane);
  if (has_nxt) issue_half<kWaves, false>(rows, t_nxt * kBN, n_keys, Kb + kTileElems, w, lane);
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  floatx4 sa[2][2][H], sb[2][2][H], lsum[H];
#pragma unroll
  for (int u = 0; u < H; ++u) lsum[u] = floatx4{0.f, 0.f, 0.f, 0.f};
  tile_scores<H>(Kb, qop, sa, m16, j);

  // one iteration; s_cur holds tile n's scores, s_nxt receives tile n+1's. p = n % 2. Returns false after the last.
  auto step = [&](floatx4 (&s_cur)[2][2][H], floatx4 (&s_nxt)[2][2][H], int p) -> bool {
    int t_nn = t_nxt;
    TileMask tm_nn;
    const bool has_nn = has_nxt && walk.next(t_nn, tm_nn, false);
    // Plain s_barrier: each wave first waits for its own DMA (vmcnt) and its LDS reads (lgkmcnt).
    __asm__ volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    if (has_nn) issue_half<kWaves, false>(rows, t_nn * kBN, n_keys, Kb + p * kTileElems, w, lane);
    if (has_nxt) issue_half<kWaves, true>(rows, t_nxt * kBN, n_keys, Vb + (p ^ 1) * kTileElems, w, lane);
    tile_mask<H, kAligned>(s_cur, t_cur * kBN, tm_cur, lane_limit, geo, hbase, j);
    tile_rescale<H>(s_cur, o, m_run, lsum, scale_log2);
    bf16x8 pop[2][H];
    // Branch-free so that both land in one scheduling region: after the last tile the scores are computed from the
    // current K buffer (valid data) and discarded.
    tile_scores<H>(Kb + (has_nxt ? p ^ 1 : p) * kTileElems, qop, s_nxt, m16, j);
    tile_probs<H>(s_cur, m_run, scale_log2, pop);
    tile_pv<H>(Vb + p * kTileElems, pop, o, lsum, lane);
    if (!has_nxt) return false;
    t_cur = t_nxt;
    tm_cur = tm_nxt;
    t_nxt = t_nn;
    tm_nxt = tm_nn;
    has_nxt = has_nn;
    return true;
  };
  for (;;) {
    if (!step(sa, sb, 0)) break;
    if (!step(sb, sa, 1)) break;
  }
#pragma unroll
  for (int u = 0; u < H; ++u) l_run[u] = lsum[u][0];
}

}  // namespace abkv
