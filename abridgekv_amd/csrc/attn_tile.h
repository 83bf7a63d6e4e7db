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

// Per-element visibility for layouts whose tiles cannot be classified (unaligned masked prefill); other kernels never
// call it (their tiles are always aligned: kAligned = true). quota[u]: code slots visible to this wave's head u;
// tail: the retained tail T under ``policy`` (a block's codes never see its own last T content rows).
struct MaskGeom {
  int qrow, S0, C, per, plen;
  int quota[2];
  int tail;
  int policy;
  int xattn;      // code rows' attention to their own pass's code rows (kXattn*)
  int K, L;       // code rows per pause pass, passes per block
  int copy;       // copy-region rows at the end of the S0 rows
  int R;          // replay rows per block
  bool rx;        // the codes do not see the block's last R content rows
  __device__ __forceinline__ bool visible(int kv, int u) const {
    return compress_visible(qrow, kv, S0, copy, C, K, L, per, plen, quota[u], tail, policy, xattn, R, rx);
  }
};

__device__ __forceinline__ u32x4 ld16g(const __bf16* p) { return *reinterpret_cast<const u32x4*>(p); }

#define ABKV_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// K/V tiles live in LDS as 64 rows x 256 B without padding; 16-byte chunk c of row r is stored at chunk c ^ (r % 16),
// which makes both operand read patterns conflict-free (16 lanes hit 16 distinct chunks). Tiles are filled with
// global_load_lds_dwordx4: a wave instruction writes 1 KiB contiguously (lane L -> bytes 16L), so each lane fetches
// the global chunk that belongs at its swizzled position. Rows past the sequence end re-read the last row (finite data,
// masked to probability 0).
// Tile row sources for the DMA. src(k0, w, n_keys) gathers, before the barrier that precedes the issue, the
// wave-uniform facts one wave's DMA of the 64-key tile at k0 needs (its rows 4 * kPerWave * w .. +4 * kPerWave - 1 lie
// in one page); addr<kV>(src, row, chunk, n_keys) is the per-lane source of LDS row `row`, chunk `chunk`. Rows at or
// past n_keys are never read (they may lie past the tensor, or hold non-finite data that a zero weight would not
// cancel in P.V): a valid row is re-read in their place (finite data, masked to zero weight). Both are branch-free
// selects, so the compiler has no speculated slow path to hoist into every tile.
// Contiguous [S, heads, 128] K/V pair (one KV head selected by the base pointers). kFull: every tile lies inside
// [0, n_keys) (no row needs replacing).
template <bool kFull>
struct DenseRows {
  const __bf16* k;
  const __bf16* v;
  long k_ss, v_ss;
  struct Src {
    int k0;
  };
  template <int kPerWave>
  __device__ __forceinline__ Src src(int k0, int, int) const { return Src{k0}; }
  template <bool kV>
  __device__ __forceinline__ const __bf16* addr(const Src& t, int row, int chunk, int n_keys) const {
    const __bf16* base = kV ? v : k;
    const long ss = kV ? v_ss : k_ss;
    const int off = row * (int)ss + 8 * chunk;
    if constexpr (kFull) return base + (long)t.k0 * ss + off;
    // past the end: the tile's first row (key k0 < n_keys)
    return base + (long)t.k0 * ss + (t.k0 + row < n_keys ? off : 8 * chunk);
  }
};

// One sequence in the paged cache [pages, 2, 16, 8, 128] (one KV head). The page ids are scalar loads through the
// constant address space (the table is not written while a kernel runs); table positions past the row and page ids
// out of range are clamped.
struct PagedRows {
  const __bf16* kv;        // cache base + kvh * 128
  const int32_t* table;    // the sequence's page-table row
  int width;               // entries in the row
  int num_pages;
  struct Src {
    int k0;
    const __bf16* blk;     // page of the wave's rows
    const __bf16* last;    // row n_keys - 1
  };
  __device__ __forceinline__ int page_of(int idx) const {
    const __attribute__((address_space(4))) int32_t* t = (const __attribute__((address_space(4))) int32_t*)table;
    return min(max(t[min(max(idx, 0), width - 1)], 0), num_pages - 1);
  }
  template <int kPerWave>
  __device__ __forceinline__ Src src(int k0, int w, int n_keys) const {
    const int last = n_keys - 1;
    return Src{k0, kv + (long)page_of((k0 >> 4) + (4 * kPerWave * w >> 4)) * kPageElems,
               kv + (long)page_of(last >> 4) * kPageElems + (last & 15) * kSlotElems};
  }
  template <bool kV>
  __device__ __forceinline__ const __bf16* addr(const Src& t, int row, int chunk, int n_keys) const {
    const bool in = t.k0 + row < n_keys;
    const __bf16* base = in ? t.blk + (row & 15) * kSlotElems : t.last;
    return base + ((kV ? kHalfElems : 0) + 8 * chunk);
  }
};

// Fill the K (kV = false) or V (kV = true) tile described by src. Each wave issues 16 / kWaves DMA instructions (one
// 1 KiB block = 4 rows of the 16 KiB tile each); w must be wave-uniform.
template <int kWaves, bool kV, class Rows>
__device__ __forceinline__ void issue_half(const Rows& rows, const typename Rows::Src& src, int n_keys, __bf16* buf,
                                           int w, int lane) {
  constexpr int kPerWave = 16 / kWaves;
#pragma unroll
  for (int n = 0; n < kPerWave; ++n) {
    const int blk = kPerWave * w + n;
    const int row = 4 * blk + (lane >> 4);
    const int chunk = (lane & 15) ^ (row & 15);
    const __bf16* p = rows.template addr<kV>(src, row, chunk, n_keys);
    __builtin_amdgcn_global_load_lds((const void*)p, ABKV_LDS(buf + 512 * blk), 16, 0, 0);
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
  int mode;        // 0 none, 1 key < this lane's limit, 2 key < limit[u] (this wave's head u), 3 per-element mask,
                   // 4 key < this lane's limit and outside the excluded range [limit[0], limit[1]),
                   // 5 key < limit[0] or key >= this lane's limit + limit[1] (a band that moves with the query row)
  int limit[2];
};

// V^T operand of one PV MFMA from the swizzled V tile with two ds_read_b64_tr_b16 (LDS transpose reads). Within a
// 16-lane group, lane i of a transpose read receives element i % 4 of the 8-byte chunk addressed by lane
// 4e + i / 4, for e = 0..3. The operand row m of dim slab t is dim 32 * (m / 4) + 4t + m % 4 and its k-index
// 8g + e (g = lane group) is key kb + 4g + e for e < 4 and kb + 16 + 4g + e - 4 for e >= 4 (the contraction order the
// P^T operand uses); so lane 4e + c of the group addresses row kb + 4g + e (then + 16), dims 32c + 4t .. +3.
// Dim slab of accumulator tile t in lane group j: tile t of a PV-style product holds dims 32j + 4 * acc_tile(t, j)
// .. + 3. Odd groups take the slabs in swapped pairs so that one transposed read's lanes use both 8-byte halves of
// their 16-byte chunks, i.e. all LDS banks (with every lane on the same half, each bank was hit twice as often).
__device__ __forceinline__ int acc_tile(int t, int j) { return t ^ (j & 1); }

// Dims 8p .. 8p + 7 of an accumulator column (lane group j) times inv, as one 16-byte bf16 store.
__device__ __forceinline__ void store_acc_bf16x8(__bf16* dst, const floatx4& a, const floatx4& b, int j, float inv) {
  const bool odd = j & 1;
  floatx4 lo, hi;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    lo[r] = odd ? b[r] : a[r];
    hi[r] = odd ? a[r] : b[r];
  }
  store_bf16x8(dst, lo, hi, inv);
}

__device__ __forceinline__ bf16x8 vt_operand(const __bf16* Vbuf, int kb, int t, int lane) {
  typedef short s4 __attribute__((ext_vector_type(4)));
  const int g = lane >> 4, i = lane & 15;
  const int e = i >> 2, c = i & 3;
  const int dim = 32 * c + 4 * acc_tile(t, c);       // 8-byte aligned, inside 16-byte chunk dim / 8
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

// Hidden keys of a partial tile get score -inf (tm.mode 0: nothing hidden). kElem: an aligned walk that may yield
// per-element tiles (mode 3, the full predicate MaskGeom::visible) beside the limit modes. kBand: a walk that may
// yield band tiles (mode 5, the rolling retained tail).
template <int H, bool kAligned, bool kHole = false, bool kElem = false, bool kBand = false>
__device__ __forceinline__ void tile_mask(floatx4 (&s)[2][2][H], int k0, const TileMask& tm, int lane_limit,
                                          const MaskGeom& geo, int j) {
  static_assert(H <= 2, "TileMask holds two per-head limits");
  if (tm.mode == 0) return;
  if constexpr (kHole) {
    if (tm.mode == 4 || (kBand && tm.mode == 5)) {       // an excluded key range (code step, retained tail) or a band
      const bool band = kBand && tm.mode == 5;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int kv = k0 + 32 * kk + 16 * t + 4 * j + r;
            const bool ok = band ? (kv < tm.limit[0] || kv >= lane_limit + tm.limit[1])
                                 : kv < lane_limit && (kv < tm.limit[0] || kv >= tm.limit[1]);
#pragma unroll
            for (int u = 0; u < H; ++u) s[kk][t][u][r] = ok ? s[kk][t][u][r] : -INFINITY;
          }
      return;
    }
  }
  // every partial tile of an aligned layout is "key < lim[u]" with a per-column limit (per head or per lane)
  int lim[H];
#pragma unroll
  for (int u = 0; u < H; ++u) lim[u] = tm.mode == 1 ? lane_limit : tm.limit[u];
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
          if constexpr (kAligned && kElem) {
            ok = tm.mode == 3 ? geo.visible(kv, u) : kv < lim[u];
          } else if constexpr (kAligned) {
            ok = kv < lim[u];
          } else {
            ok = geo.visible(kv, u);
          }
          s[kk][t][u][r] = ok ? s[kk][t][u][r] : -INFINITY;
        }
}

// Online softmax of one tile, in place: s becomes t = s * scale_log2 - m_run (log2 domain, relative to the running
// max; an arithmetic result, so the maxima below need no NaN canonicalisation), then the P^T operands exp2(t) of the
// two 32-key halves. Lazy rescale: the running max moves only when a column's max exceeds it by more than 8 (P stays
// below 2^8); then O and the weight sums are rescaled and t shifted. P^T k-index e < 4 of half kk is key
// 32kk + 4j + e, e >= 4 is key 32kk + 16 + 4j + e - 4 (the order vt_operand reads V in).
// Max of this lane's 16 scores of head u, as a chain of three-operand maxima (v_max3_f32: 8 instructions).
template <int H>
__device__ __forceinline__ float lane_max(const floatx4 (&s)[2][2][H], int u) {
  float mx = fmaxf(fmaxf(s[0][0][u][0], s[0][0][u][1]), s[0][0][u][2]);
  mx = fmaxf(fmaxf(mx, s[0][0][u][3]), s[0][1][u][0]);
  mx = fmaxf(fmaxf(mx, s[0][1][u][1]), s[0][1][u][2]);
  mx = fmaxf(fmaxf(mx, s[0][1][u][3]), s[1][0][u][0]);
  mx = fmaxf(fmaxf(mx, s[1][0][u][1]), s[1][0][u][2]);
  mx = fmaxf(fmaxf(mx, s[1][0][u][3]), s[1][1][u][0]);
  mx = fmaxf(fmaxf(mx, s[1][1][u][1]), s[1][1][u][2]);
  return fmaxf(mx, s[1][1][u][3]);
}

template <int H>
__device__ __forceinline__ void tile_softmax(floatx4 (&s)[2][2][H], floatx4 (&o)[8][H], float (&m_run)[H],
                                             floatx4 (&lsum)[H], float scale_log2, bf16x8 (&pop)[2][H]) {
  float neg_m[H];
  bool need = false;
#pragma unroll
  for (int u = 0; u < H; ++u) {
    neg_m[u] = m_run[u] == -INFINITY ? 0.f : -m_run[u];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) s[kk][t][u][r] = fmaf(s[kk][t][u][r], scale_log2, neg_m[u]);
    const float mx = lane_max(s, u);
    // this lane's part of the column beyond the headroom: t > 8 (log2 units) once a max is set, any finite t before;
    // some lane of a column is beyond it exactly when the column's max is, so the wave-wide vote needs no
    // cross-lane max on the common path
    need |= mx > (m_run[u] == -INFINITY ? -INFINITY : 8.f);
  }
  if (__any(need)) {
#pragma unroll
    for (int u = 0; u < H; ++u) {
      // the column's max (all four lane groups); the lane max recomputed here holds no register across the vote
      const float tmax = max_xor32(max_xor16(lane_max(s, u)));
      const float m_new = fmaxf(m_run[u], tmax - neg_m[u]);
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run[u] - m_new);
      const float d = m_new == -INFINITY ? 0.f : m_new + neg_m[u];    // new max minus the offset t was taken at
      m_run[u] = m_new;
      lsum[u] *= alpha;
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i][u] *= alpha;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int t = 0; t < 2; ++t) s[kk][t][u] -= d;
    }
  }
#pragma unroll
  for (int u = 0; u < H; ++u)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 pw;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        pw[2 * t] = pack_bf16x2(fast_exp2(s[kk][t][u][0]), fast_exp2(s[kk][t][u][1]));
        pw[2 * t + 1] = pack_bf16x2(fast_exp2(s[kk][t][u][2]), fast_exp2(s[kk][t][u][3]));
      }
      pop[kk][u] = __builtin_bit_cast(bf16x8, pw);
    }
}

// O^T += V^T . P^T over one tile: o[t][u][r] accumulates out dim 32j + 4 * acc_tile(t, j) + r of column (u, m16),
// j = lane >> 4.
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

constexpr int kStages = 3;                 // K and V tile buffers each (LDS: 2 x 3 x 16 KiB)

template <int N>
struct Slot {
  static constexpr int value = N;
};

// Software-pipelined walk over a query tile's key tiles; tile m lives in buffers K[m % 3], V[m % 3], six distinct LDS
// arrays, so the compiler can tell a pending DMA into one slot from reads of another (a single array with computed
// slot offsets makes it wait for every DMA in flight before each LDS read). Iteration n (tile n's scores in s_cur):
//   wait for this wave's DMAs of iteration n-2 (K(n+1), V(n)), barrier (publishes them; every wave is done reading
//   K(n) and V(n-1))
//   DMA K(n+3) -> K[n % 3], V(n+2) -> V[(n+2) % 3]: two iterations of latency cover. Both are issued every
//   iteration (past the last tile they re-load tile n into slots nobody reads again) so that each iteration has the
//   same count of loads in flight: the waits below and the compiler's own then stay exact.
//   mask + rescale of tile n; scores of tile n+1 (MFMA) with the probabilities of tile n (VALU); O += V(n) . P(n)
// Walk::next(kt, tm, first) yields the tiles in order. Rows addresses key rows; keys >= n_keys are never read.
// On return l_run[u] is the full weight sum of column (u, m16) in every lane of the column (o and m_run as above).
template <int H, bool kAligned, int kWaves, class Rows, class Walk>
__device__ __forceinline__ void attend_tiles(const Rows& rows, Walk& walk, int n_keys, __bf16* const (&K)[kStages],
                                             __bf16* const (&V)[kStages], const bf16x8 (&qop)[H][4],
                                             floatx4 (&o)[8][H], float (&m_run)[H], float (&l_run)[H],
                                             int lane_limit, float scale_log2, const MaskGeom& geo, int w, int lane) {
  constexpr int kPerWave = 16 / kWaves;
  const int m16 = lane & 15, j = lane >> 4;
  int t0 = 0, t1 = 0, t2 = 0;                      // tiles n, n+1, n+2
  TileMask m0, m1, m2;
  if (!walk.next(t0, m0, true)) return;
  t1 = t0;
  bool h1 = walk.next(t1, m1, false);
  t2 = t1;
  bool h2 = h1 && walk.next(t2, m2, false);
  {
    const auto s0 = rows.template src<kPerWave>(t0 * kBN, w, n_keys);
    issue_half<kWaves, false>(rows, s0, n_keys, K[0], w, lane);
    issue_half<kWaves, true>(rows, s0, n_keys, V[0], w, lane);
    if (h1) {
      const auto s1 = rows.template src<kPerWave>(t1 * kBN, w, n_keys);
      issue_half<kWaves, false>(rows, s1, n_keys, K[1], w, lane);
      issue_half<kWaves, true>(rows, s1, n_keys, V[1], w, lane);
    }
    if (h2) issue_half<kWaves, false>(rows, rows.template src<kPerWave>(t2 * kBN, w, n_keys), n_keys, K[2], w, lane);
  }
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  floatx4 sa[2][2][H], sb[2][2][H], lsum[H];
#pragma unroll
  for (int u = 0; u < H; ++u) lsum[u] = floatx4{0.f, 0.f, 0.f, 0.f};
  tile_scores<H>(K[0], qop, sa, m16, j);

  // one iteration, slot = n % 3; s_cur holds tile n's scores, s_nxt receives tile n+1's. False after the last tile.
  auto step = [&](floatx4 (&s_cur)[2][2][H], floatx4 (&s_nxt)[2][2][H], auto slot_c) -> bool {
    constexpr int slot = decltype(slot_c)::value;
    constexpr int slot1 = (slot + 1) % kStages, slot2 = (slot + 2) % kStages;
    int t3 = t2;
    TileMask m3;
    const bool h3 = h2 && walk.next(t3, m3, false);
    const auto src_k = rows.template src<kPerWave>((h3 ? t3 : t0) * kBN, w, n_keys);
    const auto src_v = rows.template src<kPerWave>((h2 ? t2 : t0) * kBN, w, n_keys);
    // Plain s_barrier: each wave first waits for its own DMAs of two iterations back (vmcnt: the last iteration's
    // 2 x 16 / kWaves stay in flight) and its LDS and scalar reads (lgkmcnt).
    if constexpr (kWaves == 8) __asm__ volatile("s_waitcnt vmcnt(4) lgkmcnt(0)" ::: "memory");
    else __asm__ volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    issue_half<kWaves, false>(rows, src_k, n_keys, K[slot], w, lane);
    issue_half<kWaves, true>(rows, src_v, n_keys, V[slot2], w, lane);
    tile_mask<H, kAligned, Walk::kHole, Walk::kElem, Walk::kBand>(s_cur, t0 * kBN, m0, lane_limit, geo, j);
    bf16x8 pop[2][H];
    tile_softmax<H>(s_cur, o, m_run, lsum, scale_log2, pop);
    // Unconditional so that the MFMAs can overlap the softmax work: after the last tile the scores are computed from
    // whatever K[slot1] holds (finite data: a tile or its re-load) and discarded.
    tile_scores<H>(K[slot1], qop, s_nxt, m16, j);
    tile_pv<H>(V[slot], pop, o, lsum, lane);
    if (!h1) return false;
    t0 = t1; m0 = m1;
    t1 = t2; m1 = m2; h1 = h2;
    t2 = t3; m2 = m3; h2 = h3;
    return true;
  };
  for (;;) {
    if (!step(sa, sb, Slot<0>{})) break;
    if (!step(sb, sa, Slot<1>{})) break;
    if (!step(sa, sb, Slot<2>{})) break;
    if (!step(sb, sa, Slot<0>{})) break;
    if (!step(sa, sb, Slot<1>{})) break;
    if (!step(sb, sa, Slot<2>{})) break;
  }
  // the re-loads issued by the last iterations land in LDS that this workgroup no longer reads, but they must finish
  // before the workgroup ends and its LDS is handed to another
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int u = 0; u < H; ++u) l_run[u] = lsum[u][0];
}

}  // namespace abkv
