// Shared pieces of the masked-prefill forward (prefill_attn.hip) and backward (prefill_bwd.hip): the kernel
// arguments, the workgroup -> (query tile, KV head, sequence) grid order and the tile walk over the visible key tiles
// of the compression mask (abridgekv/compress_forward.py:695-727).
#pragma once
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
  int aligned;                               // C % 64 == 0 && K % 64 == 0 (the walk over visible tiles)
  int num_q_tiles;
  int tail;                                  // retained tail T (0: none)
  int policy;                                // its policy: kTailStatic, kTailRolling, kTailSticky, kTailRaw
  int xattn;                                 // code <-> code attention in a block (kXattn*; the aligned walks
                                             // serve kXattnFull, the others take the per-element walk)
  int L;                                     // pause passes of K code rows per block (the aligned walks serve 1)
  int copy;                                  // copy-region rows after the N blocks (S0 counts them; aligned: 0)
  int R;                                     // replay rows after each block's codes (aligned: 0)
  int rx;                                    // code_exclude_replay_tail: the codes do not see the last R content rows
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
// kTail (aligned layouts with a retained tail of T rows): an earlier block's content is visible where it is raw
// prompt (a prefix) or tail (the last T rows, to the rows the policy names), so after the prompt prefix the walk jumps
// to the first tile holding visible tail rows; a code query tile sees its own block's content below C - T only. The
// tile where hidden rows give way to the tail (at most one per earlier block) hides the key range between the prompt's
// end and the tail (mode 4). kWindow (the rolling and sticky policies): only content query tiles of the next block see
// a block's tail; under "rolling" query row i of the block sees tail rows i.. (content rows >= C - T + i), so the tile
// where the band starts, and those it crosses, take the band mask (mode 5).
// Unaligned layouts: every tile up to the last visible block, mask evaluated per element (mode 3).
template <bool kAligned, bool kTail = false, bool kWindow = false>
struct TileWalk {
  static_assert(kTail || !kWindow, "a window tail is a retained tail");
  static constexpr bool kHole = kTail;                      // yields excluded key ranges (mode 4) with a tail
  static constexpr bool kElem = false;                      // aligned walks never yield per-element tiles
  static constexpr bool kBand = kWindow;                    // yields band tiles (mode 5) under the rolling policy
  int q0, q_last, qb, C, per, tpb, ct, plen, qmin, qmax, n_tiles, tail;
  bool q_code;
  int kb, tw;
  int wq0, wq1;                                             // code quotas of this wave's two heads
  int first_tail;                                           // first content row of the previous block's tail that
                                                            // this query tile sees (kWindow)
  bool rolling;

  __device__ __forceinline__ TileWalk(int q0_, int q_last_, int C_, int per_, int S0, int plen_, int qmin_, int qmax_,
                                      int wq0_, int wq1_, int tail_ = 0, int policy_ = kTailStatic)
      : q0(q0_), q_last(q_last_), C(C_), per(per_), plen(plen_), qmin(qmin_), qmax(qmax_), tail(kTail ? tail_ : 0),
        kb(0), tw(0), wq0(wq0_), wq1(wq1_) {
    qb = q0 / per;
    q_code = q0 - qb * per >= C;
    tpb = per / kBN;
    ct = C / kBN;
    n_tiles = (S0 + kBN - 1) / kBN;
    rolling = kWindow && policy_ == kTailRolling;
    first_tail = C - tail + (rolling ? q0 - qb * per : 0);
  }

  // whether an earlier block kb's tail rows are visible to this query tile at all
  __device__ __forceinline__ bool sees_tail() const {
    if (!kTail || tail <= 0) return false;
    if constexpr (kWindow) return !q_code && kb + 1 == qb && first_tail < C;
    return true;
  }

  // aligned: move (kb, tw) to the first visible tile at or after it; false when none is left
  __device__ __forceinline__ bool seek() {
    for (;;) {
      if (kb > qb) return false;
      if (tw < ct) {
        if (kb == qb) {
          // own block: content rows causally; codes see the content below C - T
          if (q_code ? (!kTail || kBN * tw < C - tail) : kb * per + kBN * tw <= q_last) return true;
          tw = ct;                                          // the rest of this block's content is hidden too
        } else {
          if (kb * C + kBN * tw < plen) return true;        // raw-prompt prefix
          if constexpr (kTail) {
            if (sees_tail()) {
              const int tail_tile = (kWindow ? first_tail : C - tail) / kBN;   // first tile holding visible tail rows
              if (tw <= tail_tile) {
                tw = tail_tile;
                return true;
              }
              if (tw < ct) return true;                     // later tiles of the tail
            }
          }
          tw = ct;
        }
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
        if (kTail && q_code && kBN * tw + kBN > C - tail) {
          tm.mode = 2;                                      // the codes' own tail begins inside the tile
          tm.limit[0] = tm.limit[1] = kb * per + C - tail;
        }
      } else {
        const int pl = min(max(plen - kb * C, 0), C);       // raw-prompt rows of this block's content
        const int lo = kBN * tw, hi = lo + kBN;
        const bool in_prompt = hi <= pl;
        const bool tail_seen = kTail && sees_tail();
        const bool in_tail = tail_seen && lo >= first_tail + (rolling ? kBN - 1 : 0);
        if (!in_prompt && !in_tail) {
          if (!tail_seen || hi <= C - tail) {               // raw-prompt boundary inside the tile
            tm.mode = 2;
            tm.limit[0] = tm.limit[1] = kb * per + pl;
          } else if (rolling) {                             // [prompt rows,] rows >= C - T + (query row's offset)
            tm.mode = 5;
            tm.limit[0] = kb * per + pl;
            tm.limit[1] = C - tail - per - 1;               // key >= row + 1 + limit[1] <=> kw >= C - T + qw
          } else if (pl < C - tail) {                       // [prompt rows,] hidden rows, tail rows
            tm.mode = 4;
            tm.limit[0] = kb * per + pl;
            tm.limit[1] = kb * per + C - tail;
          }                                                 // else prompt rows up to the tail: all visible
        }
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

// Linear grid of the prefill kernels (grid_pos): num_q_tiles x 8 x batch workgroups; 0 when the launch's work-item
// count would not fit the 32-bit grid size.
inline unsigned prefill_grid(int num_q_tiles, int batch, int threads) {
  const long n = (long)num_q_tiles * kHeadsKV * batch;
  return n * threads > 0xFFFFFFFFL ? 0u : (unsigned)n;
}

}  // namespace abkv
