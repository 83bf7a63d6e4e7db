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
#include "prefill_common.h"

namespace abkv {

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

template <int N>
struct Buf {
  static constexpr int value = N;
};

template <bool kAligned, bool kTail, bool kWindow>
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
  const int per = kAligned ? f.C + f.K : f.C + f.L * f.K + f.R;
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
  const MaskGeom geo{qrow, f.S0, f.C, per, plen, {wq0, wq1}, f.tail, f.policy, f.xattn, f.K, kAligned ? 1 : f.L,
                     kAligned ? 0 : f.copy, kAligned ? 0 : f.R, !kAligned && f.rx};
  const int q_last = min(q0 + kBM, f.S0) - 1;
  TileWalk<kAligned, kTail, kWindow> walk(q0, q_last, f.C, per, f.S0, plen, qmin, qmax, wq0, wq1, f.tail, f.policy);

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
      tile_mask<H, kAligned, kTail, false, kWindow>(s, tc * kBN, mc, qrow + 1, geo, j);
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
// pair visible, 1 key <= query, 2 key < lim0 (without a tail the per-element predicate decides these tiles),
// kTail: 4 key outside [lim0, lim1) (the tile of an earlier block where hidden rows give way to its retained tail).
// kWindow (rolling / sticky tails: only the next block's content tiles see a block's tail): rolling, 5 key < lim0 or
// key - query >= lim1 (query row i of the block sees tail rows i..).
template <bool kTail, bool kWindow>
__device__ __forceinline__ int pair_mode(int qt, int kt, int qh, int S0, int C, int per, int plen, int tail,
                                         bool rolling, int& lim0, int& lim1) {
  const int q0 = qt * kBN, k0 = kt * kBN;
  const int qb = q0 / per, kb = k0 / per;
  if (kb > qb) return -1;
  const bool q_code = q0 - qb * per >= C;
  const int tw = (k0 - kb * per) / kBN, ct = C / kBN;
  if (tw < ct) {
    if (kb == qb) {
      if (kTail && q_code) {                                // codes see their block's content below C - T
        const int lo = kBN * tw;
        if (lo >= C - tail) return -1;
        if (lo + kBN > C - tail) {
          lim0 = kb * per + C - tail;
          return 2;
        }
        return 0;
      }
      const int q_last = min(q0 + kBN, S0) - 1;
      if (!(q_code || k0 <= q_last)) return -1;
      return (!q_code && k0 + kBN - 1 > q0) ? 1 : 0;
    }
    if constexpr (kTail) {
      const int pl = min(max(plen - kb * C, 0), C);         // raw-prompt rows of this block's content
      const int lo = kBN * tw, hi = lo + kBN;
      if constexpr (kWindow) {
        if (hi <= pl) return 0;                             // all prompt
        const int first = C - tail + (rolling ? q0 - qb * per : 0);   // first tail row the query tile sees
        if (q_code || kb + 1 != qb || first >= C || hi <= C - tail) {  // no tail rows seen: a prompt prefix or nothing
          if (lo >= pl) return -1;
          lim0 = kb * per + pl;
          return 2;
        }
        if (rolling) {
          if (lo >= pl && hi <= first) return -1;           // no prompt row, no row of any query row's band
          if (lo >= first + kBN - 1) return 0;              // past every query row's band start
          lim0 = kb * per + pl;
          lim1 = C - tail - per;
          return 5;
        }
      }
      if (hi <= pl || lo >= C - tail) return 0;             // all prompt, or all tail
      if (hi <= C - tail) {                                 // no tail rows: a prompt prefix or nothing
        if (lo >= pl) return -1;
        lim0 = kb * per + pl;
        return 2;
      }
      if (pl >= C - tail) return 0;                         // prompt rows up to the tail
      lim0 = kb * per + pl;                                 // [prompt rows,] hidden rows, tail rows
      lim1 = kb * per + C - tail;
      return 4;
    }
    if (kb * C + kBN * tw >= plen) return -1;
    if (kb * C + kBN * tw + kBN > plen) {
      lim0 = kb * per + (plen - kb * C);
      return 2;
    }
    return 0;
  }
  if (!(kb < qb || q_code) || kBN * (tw - ct) >= qh) return -1;
  if (kBN * (tw - ct) + kBN > qh) {
    lim0 = kb * per + C + qh;
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

template <bool kAligned, bool kTail, bool kWindow>
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
  const int per = kAligned ? f.C + f.K : f.C + f.L * f.K + f.R;
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
  // aligned: a content tile outside the raw prompt and the retained tail is seen by its own block's rows only, so
  // the walk ends there
  const int tail = kTail ? f.tail : 0;
  int qt_end = f.num_q_tiles;
  if (kAligned && k0 - (k0 / per) * per + kBN <= f.C - tail && (k0 / per) * f.C + (k0 - (k0 / per) * per) >= plen)
    qt_end = min(qt_end, (k0 / per + 1) * per / kBN);
  if constexpr (kWindow) {                                  // a window tail: the next block's rows at most
    if (k0 - (k0 / per) * per < f.C && (k0 / per) * f.C + (k0 - (k0 / per) * per) >= plen)
      qt_end = min(qt_end, (k0 / per + 2) * per / kBN);
  }
  const bool rolling = kWindow && f.policy == kTailRolling;
  // the per-element predicate's tail: none in the aligned no-tail instance, static in the aligned static one
  const int etail = kAligned && !kTail ? 0 : f.tail;
  const int epolicy = kAligned && !kWindow ? kTailStatic : f.policy;
  const int exattn = kAligned ? kXattnFull : f.xattn;
  const int epasses = kAligned ? 1 : f.L;
  const int ecopy = kAligned ? 0 : f.copy;
  const int erep = kAligned ? 0 : f.R;
  const bool erx = !kAligned && f.rx;
  int qt = qt_lo, h = -1, mode = 0, lim0 = 0, lim1 = 0;
  auto next_pair = [&]() -> bool {
    for (;;) {
      if (++h == kGroup) {
        h = 0;
        ++qt;
      }
      if (qt >= qt_end) return false;
      if constexpr (kAligned) {
        const int qh = h == 0 ? quota_all[0] : h == 1 ? quota_all[1] : h == 2 ? quota_all[2] : quota_all[3];
        mode = pair_mode<kTail, kWindow>(qt, kt, qh, f.S0, f.C, per, plen, tail, rolling, lim0, lim1);
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
      const int clim0 = kTail ? lim0 : 0, clim1 = kTail ? lim1 : 0;
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
      } else if (kTail && (cmode == 2 || cmode == 4)) {     // visibility independent of the query row
        // mode 2 key < lim0; mode 4 key outside [lim0, lim1): one flag for this lane's key column
        const bool vis = cmode == 2 ? key < clim0 : (key < clim0 || key >= clim1);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int r0 = 32 * kk + 16 * t + 4 * j;
            const floatx4 l4 = *reinterpret_cast<const floatx4*>(Lb[sl] + r0);
            const floatx4 e4 = *reinterpret_cast<const floatx4*>(Eb[sl] + r0);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float pr = vis ? fast_exp2(fmaf(s[kk][t][0][r], f.scale_log2, -l4[r])) : 0.f;
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
              // diagonal tiles: key <= row; a rolling tail's band (mode 5); bounded (mode 2, no tail) and unaligned
              // tiles: the per-element predicate
              const bool vis = cmode == 1                   ? key <= qrow
                               : (kWindow && cmode == 5) ? (key < clim0 || key - qrow >= clim1)
                                                         : compress_visible(qrow, key, f.S0, ecopy, f.C, f.K,
                                                                            epasses, per, plen, qh, etail, epolicy,
                                                                            exattn, erep, erx);
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

extern "C" {

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
                                 const int32_t* head_quota, int retain_tail, int tail_policy, int pause_xattn,
                                 int pause_passes, int copy_rows, int replay_rows, int replay_exclude, float scale,
                                 void* dq,
                                 long dq_stride_b, long dq_stride_s, long dq_stride_h, void* dk, long dk_stride_b,
                                 long dk_stride_s, long dk_stride_h, void* dv, long dv_stride_b, long dv_stride_s,
                                 long dv_stride_h, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  using namespace abkv;
  if (batch <= 0 || seq_len <= 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr || dout == nullptr || lse == nullptr ||
      dq == nullptr || dk == nullptr || dv == nullptr || block_c <= 0 || codes_k < 0 || num_blocks <= 0 ||
      pause_passes <= 0 || copy_rows < 0 || (codes_k == 0 && (pause_passes != 1 || copy_rows)) ||
      replay_rows < 0 || replay_rows > block_c || (replay_rows && (retain_tail || codes_k == 0)) ||
      (replay_exclude && (replay_rows <= 0 || replay_rows >= block_c)) ||
      (long)seq_len != (long)num_blocks * (block_c + (long)pause_passes * codes_k + replay_rows) + copy_rows ||
      retain_tail < 0 || retain_tail > block_c || (retain_tail == block_c && tail_policy != kTailRaw) ||
      tail_policy < kTailStatic || tail_policy > kTailRaw ||
      pause_xattn < kXattnFull || pause_xattn > kXattnNone)
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
  f.policy = tail_policy;
  f.xattn = pause_xattn;
  f.L = pause_passes;
  f.copy = copy_rows;
  f.R = replay_rows;
  f.rx = replay_exclude != 0;
  f.aligned = (block_c % kBN == 0) && (codes_k % kBN == 0) && pause_xattn == kXattnFull && pause_passes == 1 &&
              copy_rows == 0 && replay_rows == 0 && tail_policy != kTailRaw;
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
  const bool window = retain_tail > 0 && tail_policy != kTailStatic;
  if (f.aligned && retain_tail == 0)
    hipLaunchKernelGGL((prefill_bwd_dq_kernel<true, false, false>), gq, dim3(512), 0, stream, a);
  else if (f.aligned && !window)
    hipLaunchKernelGGL((prefill_bwd_dq_kernel<true, true, false>), gq, dim3(512), 0, stream, a);
  else if (f.aligned) hipLaunchKernelGGL((prefill_bwd_dq_kernel<true, true, true>), gq, dim3(512), 0, stream, a);
  else hipLaunchKernelGGL((prefill_bwd_dq_kernel<false, false, false>), gq, dim3(512), 0, stream, a);
  err = hipGetLastError();
  if (err != hipSuccess) return (int)err;
  const unsigned gk = prefill_grid(f.num_q_tiles, batch, 256);
  if (f.aligned && retain_tail == 0)
    hipLaunchKernelGGL((prefill_bwd_dkv_kernel<true, false, false>), gk, dim3(256), 0, stream, a);
  else if (f.aligned && !window)
    hipLaunchKernelGGL((prefill_bwd_dkv_kernel<true, true, false>), gk, dim3(256), 0, stream, a);
  else if (f.aligned) hipLaunchKernelGGL((prefill_bwd_dkv_kernel<true, true, true>), gk, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((prefill_bwd_dkv_kernel<false, false, false>), gk, dim3(256), 0, stream, a);
  return (int)hipGetLastError();
}

}  // extern "C"
