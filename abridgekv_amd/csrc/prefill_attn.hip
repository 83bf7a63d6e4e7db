// Block-masked teacher-forced attention (the compression mask) for gfx950.
//
// Replaces the FlexAttention call of CompressLM.forward (abridgekv/compress_forward.py:1134-1230) for the production
// configuration (L=1, full code<->code attention, no replay / raw tail, an optional retained tail), whose mask is the
// closed form _arith_mask_mod (abridgekv/compress_forward.py:695-727) plus the per-query-head code quota (:725-726,
// _quota_key_allowed :230-236), and for the window tail policies the retained-tail term of _mask_mod (:566-649,
// _retained_tail_visible :99-124). Sequence layout: N blocks of [C content | K codes], S0 = N * (C + K):
//   visible(q, kv) = (kv <= q) & (own-block content | earlier blocks' codes | raw-prompt content
//                                 | retained-tail rows of earlier blocks)
//                  | (code query & code key & same block),     and a code key needs slot < quota[head];
//   a code query never sees its own block's last T content rows (retained tail T, :714-715, :721-722). The tail
//   rows (the last T content rows of a block) are visible to every later row (static), to every content row of the
//   next block (sticky), or to content row i of the next block from tail row i on (rolling).
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
// tile full (unmasked), diagonal (key <= row) or bounded (key < per-head limit); with a retained tail the walk also
// visits the tail tiles the policy shows the query tile, the tile that mixes hidden and tail rows takes an excluded
// range and the rolling policy's band a per-lane bound. Unaligned shapes run every tile of the visible prefix with the
// mask evaluated per element (correct, slower).
#include "prefill_common.h"

namespace abkv {

template <int H, bool kAligned, bool kTail, bool kWindow>
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
  const int per = kAligned ? a.C + a.K : a.C + a.L * a.K + a.R;
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
  const MaskGeom geo{qrow, a.S0, a.C, per, plen, {wq0, wq1}, a.tail, a.policy, a.xattn, a.K, kAligned ? 1 : a.L,
                     kAligned ? 0 : a.copy, kAligned ? 0 : a.R, !kAligned && a.rx};
  const int q_last = min(q0 + kBM, a.S0) - 1;

  TileWalk<kAligned, kTail, kWindow> walk(q0, q_last, a.C, per, a.S0, plen, qmin, qmax, wq0, wq1, a.tail, a.policy);
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

}  // namespace abkv

extern "C" {


int abkv_prefill_masked_attn(const void* q, long q_stride_b, long q_stride_s, long q_stride_h, const void* k,
                             long k_stride_b, long k_stride_s, long k_stride_h, const void* v, long v_stride_b,
                             long v_stride_s, long v_stride_h, int batch, int block_c, int codes_k, int num_blocks,
                             int seq_len, const int32_t* prompt_len, const int32_t* head_quota, int retain_tail,
                             int tail_policy, int pause_xattn, int pause_passes, int copy_rows, int replay_rows,
                             int replay_exclude, float scale, void* out, long out_stride_b,
                             long out_stride_s, long out_stride_h, float* lse, hipStream_t stream) {
  using namespace abkv;
  if (batch <= 0 || seq_len <= 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || block_c <= 0 || codes_k < 0 ||
      num_blocks <= 0 || pause_passes <= 0 || copy_rows < 0 || (codes_k == 0 && (pause_passes != 1 || copy_rows)) ||
      replay_rows < 0 || replay_rows > block_c || (replay_rows && (retain_tail || codes_k == 0)) ||
      (replay_exclude && (replay_rows <= 0 || replay_rows >= block_c)) ||
      (long)seq_len != (long)num_blocks * (block_c + (long)pause_passes * codes_k + replay_rows) + copy_rows ||
      retain_tail < 0 ||
      retain_tail > block_c || (retain_tail == block_c && tail_policy != kTailRaw) ||
      tail_policy < kTailStatic || tail_policy > kTailRaw || pause_xattn < kXattnFull ||
      pause_xattn > kXattnNone)
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
  a.policy = tail_policy;
  a.xattn = pause_xattn;
  a.L = pause_passes;
  a.copy = copy_rows;
  a.R = replay_rows;
  a.rx = replay_exclude != 0;
  a.aligned = (block_c % kBN == 0) && (codes_k % kBN == 0) && pause_xattn == kXattnFull && pause_passes == 1 &&
              copy_rows == 0 && replay_rows == 0 && tail_policy != kTailRaw;
  a.num_q_tiles = (seq_len + kBM - 1) / kBM;
  // 8 waves, 2 heads x 16 rows each: 216 VGPRs -> 2 waves per SIMD (the 4-head form needs 480 registers and runs
  // one wave per SIMD: 416 vs 500 TFLOP/s on the B=4, S0=10240 workload).
  const unsigned grid = prefill_grid(a.num_q_tiles, batch, 512);
  if (grid == 0) return (int)hipErrorInvalidValue;
  if (a.aligned && retain_tail == 0)
    hipLaunchKernelGGL((prefill_masked_kernel<2, true, false, false>), grid, dim3(512), 0, stream, a);
  else if (a.aligned && tail_policy == kTailStatic)
    hipLaunchKernelGGL((prefill_masked_kernel<2, true, true, false>), grid, dim3(512), 0, stream, a);
  else if (a.aligned) hipLaunchKernelGGL((prefill_masked_kernel<2, true, true, true>), grid, dim3(512), 0, stream, a);
  else hipLaunchKernelGGL((prefill_masked_kernel<2, false, false, false>), grid, dim3(512), 0, stream, a);
  return (int)hipGetLastError();
}

}  // extern "C"
