// Block-masked teacher-forced attention (the compression mask) for gfx950.
//
// Replaces the FlexAttention call of CompressLM.forward (abridgekv/compress_forward.py:1134-1230) for the production
// configuration (L=1, full code<->code attention, no replay / raw tail, an optional static retained tail), whose
// mask is the closed form _arith_mask_mod (abridgekv/compress_forward.py:695-727) plus the per-query-head code quota
// (:725-726, _quota_key_allowed :230-236). Sequence layout: N blocks of [C content | K codes], S0 = N * (C + K):
//   visible(q, kv) = (kv <= q) & (own-block content | earlier blocks' codes | raw-prompt content
//                                 | earlier blocks' last T content rows)
//                  | (code query & code key & same block),     and a code key needs slot < quota[head];
//   a code query never sees its own block's last T content rows (static retained tail T, :714-715, :721-722).
//
// Work decomposition: one workgroup of 8 waves per (sequence, KV head, 64-row query tile). A wave owns 16 query rows
// for 2 of the 4 query heads of the KV head: 32 MFMA columns (column = head u x row), so one K operand feeds 2 heads
// and the wave fits in 2 waves per SIMD. Key tiles of 64 are DMA'd into double-buffered, XOR-swizzled LDS one visible
// tile ahead (global_load_lds_dwordx4: no VGPR staging), so loads overlap the previous tile's MFMA work. Per tile:
//   S^T[64 keys x 32 cols]   = K . Q^T            4 key sub-tiles x 2 heads x 4 dim steps, MFMA 16x16x32 bf16
//   online softmax over the 64 keys (exp2 domain, lazy rescale: the running max moves only when a column max exceeds
//   it by > 8)
//   O^T[128 dims x 32 cols] += V^T . P^T          2 key halves x 8 dim tiles x 2 heads; V^T by LDS transpose reads
// Aligned layouts (C and K multiples of 64) walk only the visible tiles, jumping over hidden segments, and tag each
// tile full (unmasked), diagonal (key <= row) or bounded (key < per-head limit). Unaligned shapes and layouts with a
// retained tail run every tile of the visible prefix with the mask evaluated per element (correct, slower).
#include "attn_tile.h"

namespace abkv {

struct PrefillArgs {
  const __bf16* q;  long q_sb, q_ss, q_sh;   // [B, S0, 32, 128]
  const __bf16* k;  long k_sb, k_ss, k_sh;   // [B, S0, 8, 128]
  const __bf16* v;  long v_sb, v_ss, v_sh;
  int B, S0, C, K, N;
  const int32_t* prompt_len;                 // [B] raw-prompt content tokens (nullptr: none)
  const int32_t* head_quota;                 // [32] code slots visible per query head (nullptr: all K)
  float scale_log2;
  __bf16* out;      long o_sb, o_ss, o_sh;   // [B, S0, 32, 128]
  float* lse;                                // [B, 32, S0] natural log, or nullptr
  int aligned;                               // C % 64 == 0 && K % 64 == 0 and no retained tail
  int num_q_tiles;
  int tail;                                  // static retained tail T (0: none)
};

// Workgroup -> (tile rank, KV head, sequence) for a linear grid of num_tiles x 8 x B workgroups: KV head fastest,
// tile rank slowest. Workgroups go to the 8 XCDs round-robin by linear id, so every workgroup of one KV head runs on
// one XCD and that XCD's L2 serves all re-reads of the head's rows; and each tile rank is issued for every (head,
// sequence) before the next, so the costly tiles (which the callers rank first) do not trail at the end of the grid.
struct GridPos {
  int rank, kvh, b;
};
__device__ __forceinline__ GridPos grid_pos(int batch) {
  const int l = blockIdx.x;
  return {l / (kHeadsKV * batch), l % kHeadsKV, (l / kHeadsKV) % batch};
}

// Walk over the key tiles one query tile attends to, with the mask mode of each.
// Aligned layouts (C and K multiples of 64): a key tile is named by (block kb, tile tw of the block's C + K rows).
// Within a segment (one block's content, one block's codes) visibility is monotone in tw, so the first invisible tile
// ends the segment and the walk jumps to the next one: no per-tile test of skipped tiles and no integer division.
// Unaligned layouts: every tile up to the last visible block, mask evaluated per element (mode 3).
template <bool kAligned>
struct TileWalk {
  static constexpr bool kHole = false;                      // never yields an excluded key range (mode 4)
  int q0, q_last, qb, C, per, tpb, ct, plen, qmin, qmax, n_tiles;
  bool q_code;
  int kb, tw;
  int wq0, wq1;                                             // code quotas of this wave's two heads

  __device__ __forceinline__ TileWalk(int q0_, int q_last_, int C_, int per_, int S0, int plen_, int qmin_, int qmax_,
                                      int wq0_, int wq1_)
      : q0(q0_), q_last(q_last_), C(C_), per(per_), plen(plen_), qmin(qmin_), qmax(qmax_), kb(0), tw(0),
        wq0(wq0_), wq1(wq1_) {
    qb = q0 / per;
    q_code = q0 - qb * per >= C;
    tpb = per / kBN;
    ct = C / kBN;
    n_tiles = (S0 + kBN - 1) / kBN;
  }

  // aligned: move (kb, tw) to the first visible tile at or after it; false when none is left
  __device__ __forceinline__ bool seek() {
    for (;;) {
      if (kb > qb) return false;
      if (tw < ct) {
        const bool vis = kb == qb ? (q_code || kb * per + kBN * tw <= q_last) : (kb * C + kBN * tw < plen);
        if (vis) return true;
        tw = ct;                                            // the rest of this block's content is hidden too
      }
      if ((kb < qb || q_code) && tw < tpb && kBN * (tw - ct) < qmax) return true;
      if (kb == qb) return false;                           // blocks after the query's own block are hidden
      ++kb;
      tw = 0;
    }
  }

  // aligned: mask mode of the visible tile (kb, tw)
  __device__ __forceinline__ void mask(TileMask& tm) const {
    const int k0 = kb * per + kBN * tw;
    tm.mode = 0;
    if (tw < ct) {
      if (kb == qb) {
        if (!q_code && k0 + kBN - 1 > q0) tm.mode = 1;      // diagonal tile of the block's content
      } else if (kb * C + kBN * tw + kBN > plen) {
        tm.mode = 2;                                        // raw-prompt boundary inside the tile
        tm.limit[0] = tm.limit[1] = kb * per + (plen - kb * C);
      }
    } else if (kBN * (tw - ct) + kBN > qmin) {
      tm.mode = 2;                                          // quota boundary inside a code tile
      tm.limit[0] = kb * per + C + wq0;
      tm.limit[1] = kb * per + C + wq1;
    }
  }

  // next tile to attend (the first call gives the first); false when the walk is done
  __device__ __forceinline__ bool next(int& kt, TileMask& tm, bool first) {
    if constexpr (kAligned) {
      if (!first) ++tw;
      if (!seek()) return false;
      kt = kb * tpb + tw;
      mask(tm);
      return true;
    } else {
      kt = first ? 0 : kt + 1;
      tm.mode = 3;
      // keys up to the query tile's last row, or in a block up to its own (codes of the own block): a prefix
      return kt < n_tiles && (kt * kBN <= q_last || (kt * kBN) / per <= q_last / per);
    }
  }
};

template <int H, bool kAligned>
__global__ __launch_bounds__(64 * 4 * (4 / H), 1) void prefill_masked_kernel(PrefillArgs a) {
  constexpr int kWaves = 4 * (4 / H);                       // 16 query rows x H heads per wave
  __shared__ __attribute__((aligned(16))) __bf16 K0[kTileElems], K1[kTileElems], K2[kTileElems];
  __shared__ __attribute__((aligned(16))) __bf16 V0[kTileElems], V1[kTileElems], V2[kTileElems];
  __bf16* const Kbuf[kStages] = {K0, K1, K2};
  __bf16* const Vbuf[kStages] = {V0, V1, V2};

  const GridPos gp = grid_pos(a.B);
  const int qt = a.num_q_tiles - 1 - gp.rank;               // heavier (later) query tiles first
  const int kvh = gp.kvh;
  const int b = gp.b;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave index (uniform)
  const int lane = tid & 63;
  const int m16 = lane & 15;
  const int j = lane >> 4;
  const int rg = w / (4 / H);                               // row group (16 rows)
  const int hbase = H * (w % (4 / H));                      // first head of this wave inside the GQA group
  const int per = a.C + a.K;
  const int q0 = qt * kBM;
  const int qrow = q0 + 16 * rg + m16;                      // this lane's query row (MFMA column)
  const int plen = a.prompt_len ? a.prompt_len[b] : 0;
  int quota_all[4];
  int qmin = 1 << 30, qmax = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    quota_all[u] = a.head_quota ? a.head_quota[kvh * kGroup + u] : a.K;
    qmin = min(qmin, quota_all[u]);
    qmax = max(qmax, quota_all[u]);
  }

  bf16x8 qop[H][4];
  {
    const bool ok = qrow < a.S0;
    const __bf16* qb = a.q + (long)b * a.q_sb + (long)min(qrow, a.S0 - 1) * a.q_ss;
#pragma unroll
    for (int u = 0; u < H; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x4 x = ld16g(qb + (long)(kvh * kGroup + hbase + u) * a.q_sh + 8 * (4 * i + j));
        if (!ok) x = u32x4{0, 0, 0, 0};
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

  const DenseRows<kAligned> rows{a.k + (long)b * a.k_sb + (long)kvh * a.k_sh, a.v + (long)b * a.v_sb + (long)kvh * a.v_sh,
                       a.k_ss, a.v_ss};
  // this wave's heads hbase, hbase + 1 (hbase is 0 or 2): quotas by selection, not by a computed index
  const int wq0 = hbase ? quota_all[2] : quota_all[0], wq1 = hbase ? quota_all[3] : quota_all[1];
  const MaskGeom geo{qrow, a.S0, a.C, per, plen, {wq0, wq1}, a.tail};
  const int q_last = min(q0 + kBM, a.S0) - 1;

  TileWalk<kAligned> walk(q0, q_last, a.C, per, a.S0, plen, qmin, qmax, wq0, wq1);
  attend_tiles<H, kAligned, kWaves>(rows, walk, a.S0, Kbuf, Vbuf, qop, o, m_run, l_run, qrow + 1, a.scale_log2, geo, w,
                                    lane);

  if (qrow >= a.S0) return;
  // o[t][u][r] = un-normalised out[row qrow][head hbase + u][dim 32j + 4 * acc_tile(t, j) + r]
#pragma unroll
  for (int u = 0; u < H; ++u) {
    const float l = l_run[u];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int head = kvh * kGroup + hbase + u;
    __bf16* oh = a.out + (long)b * a.o_sb + (long)qrow * a.o_ss + (long)head * a.o_sh + 32 * j;
#pragma unroll
    for (int p = 0; p < 4; ++p) store_acc_bf16x8(oh + 8 * p, o[2 * p][u], o[2 * p + 1][u], j, inv);
    if (a.lse != nullptr && j == 0)
      a.lse[((long)b * kHeadsQ + head) * a.S0 + qrow] =
          l > 0.f ? (m_run[u] + __log2f(l)) * 0.69314718055994531f : -INFINITY;
  }
}

// ------------------------------------------------------------------------------------------------------------------
// Backward pass (gradients of q, k, v through the same mask), the FlashAttention-2 decomposition with the forward's
// LSE: P = exp2(S * scale * log2(e) - lse * log2(e)), dS = P o (dP - rowsum(dO o O)), dQ = scale * dS K,
// dK = scale * dS^T Q, dV = P^T dO. The reference trains through FlexAttention's backward of the same mask
// (abridgekv/compress_forward.py:1134-1230 called under autograd, :1329).
//   prefill_bwd_prep_kernel  per (row, query head): lse2 = lse * log2(e) and D = sum_d dO * O, in a workspace padded
//                            to whole 64-row tiles (lse2 = +inf and D = 0 past S0, so padded rows weigh 0)
//   prefill_bwd_dq_kernel    the forward's work decomposition and tile walk (query tile x KV head; wave = 16 rows x
//                            2 heads); per key tile S^T = K Q^T and dP^T = V dO^T, dQ^T += K^T dS^T
//   prefill_bwd_dkv_kernel   roles swapped: workgroup = 64 keys of a KV head, wave = 16 keys; the (query tile, head)
//                            pairs that see the key tile are staged in LDS (Q, dO, lse2, D); S = Q K^T and
//                            dP = dO V^T as the forward's score tiles, dV^T += dO^T P and dK^T += Q^T dS as its PV step
struct PrefillBwdArgs {
  PrefillArgs f;                              // q, k, v, geometry, prompt_len, head_quota, scale_log2
  const __bf16* o;    long o_sb, o_ss, o_sh;  // forward output [B, S0, 32, 128]
  const __bf16* dout; long g_sb, g_ss, g_sh;  // its gradient
  const float* lse;                           // [B, 32, S0] natural log, from the forward
  float* lse2;                                // workspace [B, 32, S0p]
  float* dvec;                                // workspace [B, 32, S0p]
  int S0p;                                    // S0 rounded up to a multiple of 64
  float scale;                                // softmax scale
  __bf16* dq; long dq_sb, dq_ss, dq_sh;       // [B, S0, 32, 128]
  __bf16* dk; long dk_sb, dk_ss, dk_sh;       // [B, S0, 8, 128]
  __bf16* dv; long dv_sb, dv_ss, dv_sh;
};

__global__ __launch_bounds__(256) void prefill_bwd_prep_kernel(PrefillBwdArgs a) {
  // 16 lanes per (row, query head): lane c takes dims 8c .. 8c + 7 of O and dO (one 16-byte load each, so a wave reads
  // four whole 256-byte rows), and the 16 partial dot products are summed by lane shuffles inside the group
  const long idx = ((long)blockIdx.x * 256 + threadIdx.x) >> 4;
  const int c = threadIdx.x & 15;
  if (idx >= (long)a.f.B * kHeadsQ * a.S0p) return;         // uniform over the 16 lanes of a row
  const int i = (int)(idx % a.S0p);
  const long bh = idx / a.S0p;
  const int h = (int)(bh % kHeadsQ), b = (int)(bh / kHeadsQ);
  float d = 0.f;
  if (i < a.f.S0) {
    const __bf16* op = a.o + (long)b * a.o_sb + (long)i * a.o_ss + (long)h * a.o_sh;
    const __bf16* gp = a.dout + (long)b * a.g_sb + (long)i * a.g_ss + (long)h * a.g_sh;
    const u32x4 x = ld16g(op + 8 * c), y = ld16g(gp + 8 * c);
#pragma unroll
    for (int e = 0; e < 4; ++e) d += bf16_lo(x[e]) * bf16_lo(y[e]) + bf16_hi(x[e]) * bf16_hi(y[e]);
  }
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) d += __shfl_xor(d, m, 64);
  if (c != 0) return;
  a.lse2[idx] = i < a.f.S0 ? a.lse[bh * a.f.S0 + i] * 1.4426950408889634f : INFINITY;
  a.dvec[idx] = d;
}

// acc[t][u] += A^T . B^T over one 64-row tile: A^T operands by LDS transpose reads of the tile, B^T the packed bf16
// operands (the forward's PV step without its row sums). acc[t][u][r] = dim 32j + 4 * acc_tile(t, j) + r of column
// (u, m16), j = lane >> 4.
template <int H>
__device__ __forceinline__ void tile_acc(const __bf16* buf, const bf16x8 (&op)[2][H], floatx4 (&acc)[8][H], int lane) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const bf16x8 a = vt_operand(buf, 32 * kk, t, lane);
#pragma unroll
      for (int u = 0; u < H; ++u) acc[t][u] = mfma16x16x32(a, op[kk][u], acc[t][u]);
    }
}

// bf16 MFMA operand of a 64-row score tile x[kk][t][u][r] (row 32kk + 16t + 4j + r): k-index e < 4 is row
// 32kk + 4j + e, e >= 4 row 32kk + 16 + 4j + e - 4 (the order vt_operand reads the tile in).
template <int H>
__device__ __forceinline__ void pack_tile_op(const floatx4 (&x)[2][2][H], bf16x8 (&op)[2][H]) {
#pragma unroll
  for (int u = 0; u < H; ++u)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      u32x4 pw;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        pw[2 * t] = pack_bf16x2(x[kk][t][u][0], x[kk][t][u][1]);
        pw[2 * t + 1] = pack_bf16x2(x[kk][t][u][2], x[kk][t][u][3]);
      }
      op[kk][u] = __builtin_bit_cast(bf16x8, pw);
    }
}

// Visibility of key kv to query row q under the compression mask (the per-element predicate of MaskGeom::visible
// with the query as an argument), for unaligned layouts and layouts with a static retained tail.
__device__ __forceinline__ bool elem_visible(int q, int kv, int S0, int C, int per, int plen, int quota, int tail) {
  if (kv >= S0 || q >= S0) return false;
  const int qb = q / per, kb = kv / per;
  const int qw = q - qb * per, kw = kv - kb * per;
  const bool kc = kw < C;
  const bool in_tail = kc && kw >= C - tail;
  bool v = (kc && kb == qb) || (!kc && kb < qb) || (kc && kb * C + kw < plen) || (in_tail && kb < qb);
  v = v && kv <= q;
  v = v || (qw >= C && !kc && kb == qb);
  v = v && !(qw >= C && kb == qb && in_tail);
  return v && (kc || kw - C < quota);
}

template <int N>
struct Buf {
  static constexpr int value = N;
};

template <bool kAligned>
__global__ __launch_bounds__(512, 1) void prefill_bwd_dq_kernel(PrefillBwdArgs a) {
  constexpr int H = 2, kWaves = 8;
  __shared__ __attribute__((aligned(16))) __bf16 K0[kTileElems], K1[kTileElems], V0[kTileElems], V1[kTileElems];
  __bf16* const Kb[2] = {K0, K1};
  __bf16* const Vb[2] = {V0, V1};
  const PrefillArgs& f = a.f;
  const GridPos gp = grid_pos(f.B);
  const int qt = f.num_q_tiles - 1 - gp.rank;               // heavier (later) query tiles first
  const int kvh = gp.kvh;
  const int b = gp.b;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int m16 = lane & 15, j = lane >> 4;
  const int rg = w / 2, hbase = H * (w % 2);
  const int per = f.C + f.K;
  const int q0 = qt * kBM;
  const int qrow = q0 + 16 * rg + m16;
  const int plen = f.prompt_len ? f.prompt_len[b] : 0;
  int quota_all[4];
  int qmin = 1 << 30, qmax = 0;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    quota_all[u] = f.head_quota ? f.head_quota[kvh * kGroup + u] : f.K;
    qmin = min(qmin, quota_all[u]);
    qmax = max(qmax, quota_all[u]);
  }
  bf16x8 qop[H][4], gop[H][4];
  float l2[H], dd[H];
  {
    const bool ok = qrow < f.S0;
    const int r = min(qrow, f.S0 - 1);
#pragma unroll
    for (int u = 0; u < H; ++u) {
      const int head = kvh * kGroup + hbase + u;
      const __bf16* qp = f.q + (long)b * f.q_sb + (long)r * f.q_ss + (long)head * f.q_sh;
      const __bf16* gp = a.dout + (long)b * a.g_sb + (long)r * a.g_ss + (long)head * a.g_sh;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u32x4 x = ld16g(qp + 8 * (4 * i + j)), y = ld16g(gp + 8 * (4 * i + j));
        if (!ok) x = y = u32x4{0, 0, 0, 0};
        qop[u][i] = __builtin_bit_cast(bf16x8, x);
        gop[u][i] = __builtin_bit_cast(bf16x8, y);
      }
      const long wi = ((long)b * kHeadsQ + head) * a.S0p + qrow;      // qrow < S0p
      l2[u] = a.lse2[wi];
      dd[u] = a.dvec[wi];
    }
  }
  floatx4 dq[8][H];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int u = 0; u < H; ++u) dq[i][u] = floatx4{0.f, 0.f, 0.f, 0.f};

  const DenseRows<kAligned> rows{f.k + (long)b * f.k_sb + (long)kvh * f.k_sh, f.v + (long)b * f.v_sb + (long)kvh * f.v_sh,
                                 f.k_ss, f.v_ss};
  const int wq0 = hbase ? quota_all[2] : quota_all[0], wq1 = hbase ? quota_all[3] : quota_all[1];
  const MaskGeom geo{qrow, f.S0, f.C, per, plen, {wq0, wq1}, f.tail};
  const int q_last = min(q0 + kBM, f.S0) - 1;
  TileWalk<kAligned> walk(q0, q_last, f.C, per, f.S0, plen, qmin, qmax, wq0, wq1);

  int tc = 0;
  TileMask mc;
  if (walk.next(tc, mc, true)) {
    {
      const auto s0 = rows.template src<2>(tc * kBN, w, f.S0);
      issue_half<kWaves, false>(rows, s0, f.S0, Kb[0], w, lane);
      issue_half<kWaves, true>(rows, s0, f.S0, Vb[0], w, lane);
    }
    // Double buffer: iteration n waits for tile n (every wave's DMAs, then a barrier, which also ends all reads of
    // the other buffer), issues tile n+1 (or re-loads tile n past the end) into the other buffer, computes tile n.
    auto step = [&](auto buf_c) -> bool {
      constexpr int sl = decltype(buf_c)::value;
      int tn = tc;
      TileMask mn;
      const bool hn = walk.next(tn, mn, false);
      const auto src = rows.template src<2>((hn ? tn : tc) * kBN, w, f.S0);
      __asm__ volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      issue_half<kWaves, false>(rows, src, f.S0, Kb[1 - sl], w, lane);
      issue_half<kWaves, true>(rows, src, f.S0, Vb[1 - sl], w, lane);
      floatx4 s[2][2][H], dp[2][2][H];
      tile_scores<H>(Kb[sl], qop, s, m16, j);
      tile_scores<H>(Vb[sl], gop, dp, m16, j);
      tile_mask<H, kAligned>(s, tc * kBN, mc, qrow + 1, geo, j);
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int u = 0; u < H; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float pr = fast_exp2(fmaf(s[kk][t][u][r], f.scale_log2, -l2[u]));
              s[kk][t][u][r] = pr * (dp[kk][t][u][r] - dd[u]);
            }
      bf16x8 dsop[2][H];
      pack_tile_op<H>(s, dsop);
      tile_acc<H>(Kb[sl], dsop, dq, lane);
      if (!hn) return false;
      tc = tn;
      mc = mn;
      return true;
    };
    for (;;) {
      if (!step(Buf<0>{})) break;
      if (!step(Buf<1>{})) break;
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  if (qrow >= f.S0) return;
#pragma unroll
  for (int u = 0; u < H; ++u) {
    __bf16* dp = a.dq + (long)b * a.dq_sb + (long)qrow * a.dq_ss + (long)(kvh * kGroup + hbase + u) * a.dq_sh + 32 * j;
#pragma unroll
    for (int p = 0; p < 4; ++p) store_acc_bf16x8(dp + 8 * p, dq[2 * p][u], dq[2 * p + 1][u], j, a.scale);
  }
}

// Visibility of the 64-key tile kt to the 64-row query tile qt for a head of code quota qh, aligned layouts (C, K
// multiples of 64; the classification of the forward's TileWalk::seek / mask for one key tile): -1 hidden, 0 every
// pair visible, 1 key <= query, 2 key < limit.
__device__ __forceinline__ int pair_mode(int qt, int kt, int qh, int S0, int C, int per, int plen, int& limit) {
  const int q0 = qt * kBN, k0 = kt * kBN;
  const int qb = q0 / per, kb = k0 / per;
  if (kb > qb) return -1;
  const bool q_code = q0 - qb * per >= C;
  const int tw = (k0 - kb * per) / kBN, ct = C / kBN;
  if (tw < ct) {
    if (kb == qb) {
      const int q_last = min(q0 + kBN, S0) - 1;
      if (!(q_code || k0 <= q_last)) return -1;
      return (!q_code && k0 + kBN - 1 > q0) ? 1 : 0;
    }
    if (kb * C + kBN * tw >= plen) return -1;
    if (kb * C + kBN * tw + kBN > plen) {
      limit = kb * per + (plen - kb * C);
      return 2;
    }
    return 0;
  }
  if (!(kb < qb || q_code) || kBN * (tw - ct) >= qh) return -1;
  if (kBN * (tw - ct) + kBN > qh) {
    limit = kb * per + C + qh;
    return 2;
  }
  return 0;
}

// S = Q K^T and dP = dO V^T of a wave's 16 keys over one staged tile (32 ds_read_b128, 32 MFMAs). The two products
// are interleaved and the reads run eight ahead of the MFMAs: at 2 waves per SIMD the other wave alone cannot cover
// an LDS round trip per MFMA.
__device__ __forceinline__ void dkv_scores(const __bf16* Qbuf, const __bf16* Gbuf, const bf16x8 (&kop)[4],
                                           const bf16x8 (&vop)[4], floatx4 (&s)[2][2][1], floatx4 (&dp)[2][2][1],
                                           int m16, int j) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int t = 0; t < 2; ++t) s[kk][t][0] = dp[kk][t][0] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const bf16x8 qa = __builtin_bit_cast(bf16x8, lds16(Qbuf, 32 * kk + 16 * t + m16, 4 * i + j));
        const bf16x8 ga = __builtin_bit_cast(bf16x8, lds16(Gbuf, 32 * kk + 16 * t + m16, 4 * i + j));
        s[kk][t][0] = mfma16x16x32(qa, kop[i], s[kk][t][0]);
        dp[kk][t][0] = mfma16x16x32(ga, vop[i], dp[kk][t][0]);
      }
  // scheduling groups (mask 0x100 LDS reads, 0x008 MFMA): 8 reads, then one MFMA per read, then the last 8 MFMAs
  __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
  for (int n = 0; n < 24; ++n) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
}

// dV^T += dO^T P and dK^T += Q^T dS over one staged tile (the forward's PV step twice, interleaved; 64 transposed
// reads, 32 MFMAs), the reads running ahead of the MFMAs as in dkv_scores.
__device__ __forceinline__ void dkv_acc(const __bf16* Qbuf, const __bf16* Gbuf, const bf16x8 (&pop)[2][1],
                                        const bf16x8 (&dsop)[2][1], floatx4 (&dk)[8][1], floatx4 (&dv)[8][1],
                                        int lane) {
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const bf16x8 ga = vt_operand(Gbuf, 32 * kk, t, lane);
      const bf16x8 qa = vt_operand(Qbuf, 32 * kk, t, lane);
      dv[t][0] = mfma16x16x32(ga, pop[kk][0], dv[t][0]);
      dk[t][0] = mfma16x16x32(qa, dsop[kk][0], dk[t][0]);
    }
  __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);
#pragma unroll
  for (int n = 0; n < 28; ++n) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
}

template <bool kAligned>
__global__ __launch_bounds__(256, 2) void prefill_bwd_dkv_kernel(PrefillBwdArgs a) {
  constexpr int kWaves = 4;
  __shared__ __attribute__((aligned(16))) __bf16 Q0[kTileElems], Q1[kTileElems], G0[kTileElems], G1[kTileElems];
  __shared__ __attribute__((aligned(16))) float L0[kBN], L1[kBN], E0[kBN], E1[kBN];
  __bf16* const Qb[2] = {Q0, Q1};
  __bf16* const Gb[2] = {G0, G1};
  float* const Lb[2] = {L0, L1};
  float* const Eb[2] = {E0, E1};
  const PrefillArgs& f = a.f;
  const GridPos gp = grid_pos(f.B);
  const int kt = gp.rank;                                   // earlier key tiles are seen by more query tiles
  const int kvh = gp.kvh;
  const int b = gp.b;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int m16 = lane & 15, j = lane >> 4;
  const int per = f.C + f.K;
  const int k0 = kt * kBN;
  const int key = k0 + 16 * w + m16;                        // this lane's column
  const int plen = f.prompt_len ? f.prompt_len[b] : 0;
  int quota_all[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) quota_all[u] = f.head_quota ? f.head_quota[kvh * kGroup + u] : f.K;

  bf16x8 kop[4], vop[4];
  {
    const bool ok = key < f.S0;
    const int r = min(key, f.S0 - 1);
    const __bf16* kp = f.k + (long)b * f.k_sb + (long)r * f.k_ss + (long)kvh * f.k_sh;
    const __bf16* vp = f.v + (long)b * f.v_sb + (long)r * f.v_ss + (long)kvh * f.v_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      u32x4 x = ld16g(kp + 8 * (4 * i + j)), y = ld16g(vp + 8 * (4 * i + j));
      if (!ok) x = y = u32x4{0, 0, 0, 0};
      kop[i] = __builtin_bit_cast(bf16x8, x);
      vop[i] = __builtin_bit_cast(bf16x8, y);
    }
  }
  floatx4 dk[8][1], dv[8][1];
#pragma unroll
  for (int i = 0; i < 8; ++i) dk[i][0] = dv[i][0] = floatx4{0.f, 0.f, 0.f, 0.f};

  // (query tile, head) pairs that can see this key tile, head fastest; queries start at the key's block
  const int qt_lo = (k0 / per) * per / kBN;
  // aligned: a content tile outside the raw prompt is seen by its own block's rows only, so the walk ends there
  int qt_end = f.num_q_tiles;
  if (kAligned && k0 - (k0 / per) * per < f.C && (k0 / per) * f.C + (k0 - (k0 / per) * per) >= plen)
    qt_end = min(qt_end, (k0 / per + 1) * per / kBN);
  int qt = qt_lo, h = -1, mode = 0, limit = 0;
  auto next_pair = [&]() -> bool {
    for (;;) {
      if (++h == kGroup) {
        h = 0;
        ++qt;
      }
      if (qt >= qt_end) return false;
      if constexpr (kAligned) {
        const int qh = h == 0 ? quota_all[0] : h == 1 ? quota_all[1] : h == 2 ? quota_all[2] : quota_all[3];
        mode = pair_mode(qt, kt, qh, f.S0, f.C, per, plen, limit);
        if (mode >= 0) return true;
      } else {
        mode = 3;
        return true;
      }
    }
  };
  // Q / dO rows of (qt, head) as the tile rows, lse2 / D rows beside them (waves 0 and 1, 4 bytes per lane)
  auto issue = [&](int pq, int ph, int sl_dst) {
    const int head = kvh * kGroup + ph;
    const DenseRows<false> rows{f.q + (long)b * f.q_sb + (long)head * f.q_sh,
                                a.dout + (long)b * a.g_sb + (long)head * a.g_sh, f.q_ss, a.g_ss};
    const auto src = rows.template src<4>(pq * kBN, w, f.S0);
    issue_half<kWaves, false>(rows, src, f.S0, Qb[sl_dst], w, lane);
    issue_half<kWaves, true>(rows, src, f.S0, Gb[sl_dst], w, lane);
    const long wi = ((long)b * kHeadsQ + head) * a.S0p + pq * kBN + lane;
    if (w == 0) __builtin_amdgcn_global_load_lds((const void*)(a.lse2 + wi), ABKV_LDS(Lb[sl_dst]), 4, 0, 0);
    if (w == 1) __builtin_amdgcn_global_load_lds((const void*)(a.dvec + wi), ABKV_LDS(Eb[sl_dst]), 4, 0, 0);
  };
  if (next_pair()) {
    issue(qt, h, 0);
    auto step = [&](auto buf_c) -> bool {
      constexpr int sl = decltype(buf_c)::value;
      const int cq = qt, ch = h, cmode = mode;
      const bool hn = next_pair();
      __asm__ volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      if (hn) issue(qt, h, 1 - sl);
      floatx4 s[2][2][1], dp[2][2][1];
      dkv_scores(Qb[sl], Gb[sl], kop, vop, s, dp, m16, j);
      const int qh = ch == 0 ? quota_all[0] : ch == 1 ? quota_all[1] : ch == 2 ? quota_all[2] : quota_all[3];
      if (cmode == 0) {                                     // wave-uniform: every pair of the tile visible
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int r0 = 32 * kk + 16 * t + 4 * j;
            const floatx4 l4 = *reinterpret_cast<const floatx4*>(Lb[sl] + r0);
            const floatx4 e4 = *reinterpret_cast<const floatx4*>(Eb[sl] + r0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float pr = fast_exp2(fmaf(s[kk][t][0][r], f.scale_log2, -l4[r]));
              s[kk][t][0][r] = pr;
              dp[kk][t][0][r] = pr * (dp[kk][t][0][r] - e4[r]);
            }
          }
      } else {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int r0 = 32 * kk + 16 * t + 4 * j;
            const floatx4 l4 = *reinterpret_cast<const floatx4*>(Lb[sl] + r0);
            const floatx4 e4 = *reinterpret_cast<const floatx4*>(Eb[sl] + r0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int qrow = cq * kBN + r0 + r;
              // diagonal tiles: key <= row; bounded (mode 2) and unaligned tiles: the per-element predicate
              const bool vis = cmode == 1 ? key <= qrow : elem_visible(qrow, key, f.S0, f.C, per, plen, qh, f.tail);
              const float pr = vis ? fast_exp2(fmaf(s[kk][t][0][r], f.scale_log2, -l4[r])) : 0.f;
              s[kk][t][0][r] = pr;
              dp[kk][t][0][r] = pr * (dp[kk][t][0][r] - e4[r]);
            }
          }
      }
      bf16x8 pop[2][1], dsop[2][1];
      pack_tile_op<1>(s, pop);
      pack_tile_op<1>(dp, dsop);
      dkv_acc(Qb[sl], Gb[sl], pop, dsop, dk, dv, lane);
      return hn;
    };
    for (;;) {
      if (!step(Buf<0>{})) break;
      if (!step(Buf<1>{})) break;
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  if (key >= f.S0) return;
  __bf16* kp = a.dk + (long)b * a.dk_sb + (long)key * a.dk_ss + (long)kvh * a.dk_sh + 32 * j;
  __bf16* vp = a.dv + (long)b * a.dv_sb + (long)key * a.dv_ss + (long)kvh * a.dv_sh + 32 * j;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    store_acc_bf16x8(kp + 8 * p, dk[2 * p][0], dk[2 * p + 1][0], j, a.scale);
    store_acc_bf16x8(vp + 8 * p, dv[2 * p][0], dv[2 * p + 1][0], j, 1.f);
  }
}

}  // namespace abkv

namespace {
// Linear grid of the prefill kernels (grid_pos): num_q_tiles x 8 x batch workgroups; 0 when the launch's work-item
// count would not fit the 32-bit grid size.
unsigned prefill_grid(int num_q_tiles, int batch, int threads) {
  const long n = (long)num_q_tiles * abkv::kHeadsKV * batch;
  return n * threads > 0xFFFFFFFFL ? 0u : (unsigned)n;
}
}  // namespace

extern "C" {

int abkv_prefill_masked_attn(const void* q, long q_stride_b, long q_stride_s, long q_stride_h, const void* k,
                             long k_stride_b, long k_stride_s, long k_stride_h, const void* v, long v_stride_b,
                             long v_stride_s, long v_stride_h, int batch, int block_c, int codes_k, int num_blocks,
                             int seq_len, const int32_t* prompt_len, const int32_t* head_quota, int retain_tail,
                             float scale, void* out, long out_stride_b, long out_stride_s, long out_stride_h,
                             float* lse, hipStream_t stream) {
  using namespace abkv;
  if (batch <= 0 || seq_len <= 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || block_c <= 0 || codes_k <= 0 ||
      num_blocks <= 0 || seq_len != num_blocks * (block_c + codes_k) || retain_tail < 0 || retain_tail >= block_c)
    return (int)hipErrorInvalidValue;
  PrefillArgs a;
  a.q = static_cast<const __bf16*>(q);
  a.q_sb = q_stride_b; a.q_ss = q_stride_s; a.q_sh = q_stride_h;
  a.k = static_cast<const __bf16*>(k);
  a.k_sb = k_stride_b; a.k_ss = k_stride_s; a.k_sh = k_stride_h;
  a.v = static_cast<const __bf16*>(v);
  a.v_sb = v_stride_b; a.v_ss = v_stride_s; a.v_sh = v_stride_h;
  a.B = batch; a.S0 = seq_len; a.C = block_c; a.K = codes_k; a.N = num_blocks;
  a.prompt_len = prompt_len;
  a.head_quota = head_quota;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = static_cast<__bf16*>(out);
  a.o_sb = out_stride_b; a.o_ss = out_stride_s; a.o_sh = out_stride_h;
  a.lse = lse;
  a.tail = retain_tail;
  a.aligned = (block_c % kBN == 0) && (codes_k % kBN == 0) && retain_tail == 0;
  a.num_q_tiles = (seq_len + kBM - 1) / kBM;
  // 8 waves, 2 heads x 16 rows each: 216 VGPRs -> 2 waves per SIMD (the 4-head form needs 480 registers and runs
  // one wave per SIMD: 416 vs 500 TFLOP/s on the B=4, S0=10240 workload).
  const unsigned grid = prefill_grid(a.num_q_tiles, batch, 512);
  if (grid == 0) return (int)hipErrorInvalidValue;
  if (a.aligned) hipLaunchKernelGGL((prefill_masked_kernel<2, true>), grid, dim3(512), 0, stream, a);
  else hipLaunchKernelGGL((prefill_masked_kernel<2, false>), grid, dim3(512), 0, stream, a);
  return (int)hipGetLastError();
}


// Workspace bytes of abkv_prefill_masked_attn_bwd: lse * log2(e) and rowsum(dO * O) per (batch, query head, row),
// rows padded to whole 64-row tiles.
size_t abkv_prefill_masked_bwd_workspace_size(int batch, int seq_len) {
  const size_t s0p = ((size_t)(seq_len > 0 ? seq_len : 0) + 63) / 64 * 64;
  return 2 * (size_t)(batch > 0 ? batch : 0) * abkv::kHeadsQ * s0p * sizeof(float);
}

int abkv_prefill_masked_attn_bwd(const void* q, long q_stride_b, long q_stride_s, long q_stride_h, const void* k,
                                 long k_stride_b, long k_stride_s, long k_stride_h, const void* v, long v_stride_b,
                                 long v_stride_s, long v_stride_h, const void* out, long out_stride_b,
                                 long out_stride_s, long out_stride_h, const void* dout, long dout_stride_b,
                                 long dout_stride_s, long dout_stride_h, const float* lse, int batch, int block_c,
                                 int codes_k, int num_blocks, int seq_len, const int32_t* prompt_len,
                                 const int32_t* head_quota, int retain_tail, float scale, void* dq, long dq_stride_b,
                                 long dq_stride_s, long dq_stride_h, void* dk, long dk_stride_b, long dk_stride_s,
                                 long dk_stride_h, void* dv, long dv_stride_b, long dv_stride_s, long dv_stride_h,
                                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
  using namespace abkv;
  if (batch <= 0 || seq_len <= 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || dout == nullptr || lse == nullptr ||
      dq == nullptr || dk == nullptr || dv == nullptr || block_c <= 0 || codes_k <= 0 || num_blocks <= 0 ||
      seq_len != num_blocks * (block_c + codes_k) || retain_tail < 0 || retain_tail >= block_c)
    return (int)hipErrorInvalidValue;
  if (workspace == nullptr || workspace_bytes < abkv_prefill_masked_bwd_workspace_size(batch, seq_len))
    return (int)hipErrorInvalidValue;
  PrefillBwdArgs a;
  PrefillArgs& f = a.f;
  f.q = static_cast<const __bf16*>(q);
  f.q_sb = q_stride_b; f.q_ss = q_stride_s; f.q_sh = q_stride_h;
  f.k = static_cast<const __bf16*>(k);
  f.k_sb = k_stride_b; f.k_ss = k_stride_s; f.k_sh = k_stride_h;
  f.v = static_cast<const __bf16*>(v);
  f.v_sb = v_stride_b; f.v_ss = v_stride_s; f.v_sh = v_stride_h;
  f.B = batch; f.S0 = seq_len; f.C = block_c; f.K = codes_k; f.N = num_blocks;
  f.prompt_len = prompt_len;
  f.head_quota = head_quota;
  f.scale_log2 = scale * 1.4426950408889634f;
  f.out = nullptr; f.o_sb = f.o_ss = f.o_sh = 0;
  f.lse = nullptr;
  f.tail = retain_tail;
  f.aligned = (block_c % kBN == 0) && (codes_k % kBN == 0) && retain_tail == 0;
  f.num_q_tiles = (seq_len + kBM - 1) / kBM;
  a.o = static_cast<const __bf16*>(out);
  a.o_sb = out_stride_b; a.o_ss = out_stride_s; a.o_sh = out_stride_h;
  a.dout = static_cast<const __bf16*>(dout);
  a.g_sb = dout_stride_b; a.g_ss = dout_stride_s; a.g_sh = dout_stride_h;
  a.lse = lse;
  a.S0p = f.num_q_tiles * kBM;
  a.lse2 = static_cast<float*>(workspace);
  a.dvec = a.lse2 + (size_t)batch * kHeadsQ * a.S0p;
  a.scale = scale;
  a.dq = static_cast<__bf16*>(dq);
  a.dq_sb = dq_stride_b; a.dq_ss = dq_stride_s; a.dq_sh = dq_stride_h;
  a.dk = static_cast<__bf16*>(dk);
  a.dk_sb = dk_stride_b; a.dk_ss = dk_stride_s; a.dk_sh = dk_stride_h;
  a.dv = static_cast<__bf16*>(dv);
  a.dv_sb = dv_stride_b; a.dv_ss = dv_stride_s; a.dv_sh = dv_stride_h;
  if (prefill_grid(f.num_q_tiles, batch, 512) == 0) return (int)hipErrorInvalidValue;
  const long rows = (long)batch * kHeadsQ * a.S0p;
  if (rows * 16 > 0xFFFFFFFFL) return (int)hipErrorInvalidValue;  // prep: 16 work-items per row and head
  hipLaunchKernelGGL(prefill_bwd_prep_kernel, dim3((unsigned)((rows * 16 + 255) / 256)), dim3(256), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  const unsigned gq = prefill_grid(f.num_q_tiles, batch, 512);
  if (f.aligned) hipLaunchKernelGGL((prefill_bwd_dq_kernel<true>), gq, dim3(512), 0, stream, a);
  else hipLaunchKernelGGL((prefill_bwd_dq_kernel<false>), gq, dim3(512), 0, stream, a);
  err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  const unsigned gk = prefill_grid(f.num_q_tiles, batch, 256);
  if (f.aligned) hipLaunchKernelGGL((prefill_bwd_dkv_kernel<true>), gk, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((prefill_bwd_dkv_kernel<false>), gk, dim3(256), 0, stream, a);
  return (int)hipGetLastError();
}

}  // extern "C"
