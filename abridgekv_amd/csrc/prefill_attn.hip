// Block-masked teacher-forced attention (the compression mask) for gfx950.
//
// Replaces the FlexAttention call of CompressLM.forward (abridgekv/compress_forward.py:1134-1230) for the production
// configuration (L=1, full code<->code attention, no replay / raw / retained tails), whose mask is the closed form
// _arith_mask_mod (abridgekv/compress_forward.py:695-727) plus the per-query-head code quota (:725-726,
// _quota_key_allowed :230-236). Sequence layout: N blocks of [C content | K codes], S0 = N * (C + K):
//   visible(q, kv) = (kv <= q) & (own-block content | earlier blocks' codes | raw-prompt content)
//                  | (code query & code key & same block),     and a code key needs slot < quota[head].
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
// tile full (unmasked), diagonal (key <= row) or bounded (key < per-head limit). Unaligned shapes run every tile of
// the visible prefix with the mask evaluated per element (correct, slower).
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
  int aligned;                               // C % 64 == 0 && K % 64 == 0
  int num_q_tiles;
};

// Walk over the key tiles one query tile attends to, with the mask mode of each.
// Aligned layouts (C and K multiples of 64): a key tile is named by (block kb, tile tw of the block's C + K rows).
// Within a segment (one block's content, one block's codes) visibility is monotone in tw, so the first invisible tile
// ends the segment and the walk jumps to the next one: no per-tile test of skipped tiles and no integer division.
// Unaligned layouts: every tile up to the last visible block, mask evaluated per element (mode 3).
template <bool kAligned>
struct TileWalk {
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

  const int qt = a.num_q_tiles - 1 - blockIdx.x;            // heavier (later) query tiles first
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
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
  const MaskGeom geo{qrow, a.S0, a.C, per, plen, {wq0, wq1}};
  const int q_last = min(q0 + kBM, a.S0) - 1;

  TileWalk<kAligned> walk(q0, q_last, a.C, per, a.S0, plen, qmin, qmax, wq0, wq1);
  attend_tiles<H, kAligned, kWaves>(rows, walk, a.S0, Kbuf, Vbuf, qop, o, m_run, l_run, qrow + 1, a.scale_log2, geo, w,
                                    lane);

  if (qrow >= a.S0) return;
  // o[t][u][r] = un-normalised out[row qrow][head hbase + u][dim 32j + 4t + r]
#pragma unroll
  for (int u = 0; u < H; ++u) {
    const float l = l_run[u];
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int head = kvh * kGroup + hbase + u;
    __bf16* oh = a.out + (long)b * a.o_sb + (long)qrow * a.o_ss + (long)head * a.o_sh + 32 * j;
#pragma unroll
    for (int p = 0; p < 4; ++p) store_bf16x8(oh + 8 * p, o[2 * p][u], o[2 * p + 1][u], inv);
    if (a.lse != nullptr && j == 0)
      a.lse[((long)b * kHeadsQ + head) * a.S0 + qrow] =
          l > 0.f ? (m_run[u] + __log2f(l)) * 0.69314718055994531f : -INFINITY;
  }
}

}  // namespace abkv

extern "C" {

int abkv_prefill_masked_attn(const void* q, long q_stride_b, long q_stride_s, long q_stride_h, const void* k,
                             long k_stride_b, long k_stride_s, long k_stride_h, const void* v, long v_stride_b,
                             long v_stride_s, long v_stride_h, int batch, int block_c, int codes_k, int num_blocks,
                             int seq_len, const int32_t* prompt_len, const int32_t* head_quota, float scale,
                             void* out, long out_stride_b, long out_stride_s, long out_stride_h, float* lse,
                             hipStream_t stream) {
  using namespace abkv;
  if (batch <= 0 || seq_len <= 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || block_c <= 0 || codes_k <= 0 ||
      num_blocks <= 0 || seq_len != num_blocks * (block_c + codes_k))
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
  a.aligned = (block_c % kBN == 0) && (codes_k % kBN == 0);
  a.num_q_tiles = (seq_len + kBM - 1) / kBM;
  // 8 waves, 2 heads x 16 rows each: 216 VGPRs -> 2 waves per SIMD (the 4-head form needs 480 registers and runs
  // one wave per SIMD: 416 vs 500 TFLOP/s on the B=4, S0=10240 workload).
  const dim3 grid(a.num_q_tiles, kHeadsKV, batch);
  if (a.aligned) hipLaunchKernelGGL((prefill_masked_kernel<2, true>), grid, dim3(512), 0, stream, a);
  else hipLaunchKernelGGL((prefill_masked_kernel<2, false>), grid, dim3(512), 0, stream, a);
  return (int)hipGetLastError();
}

}  // extern "C"
