// fp32 mode of the three attention paths (decode, paged multi-query, compression-masked prefill) for gfx950.
//
// Same semantics as the bf16 kernels (decode_attn.hip, paged_prefill.hip, prefill_attn.hip), with fp32 queries,
// keys, values and outputs, fp32 accumulation in a fixed order and accurate expf/logf: the mode the reference's
// PyTorch paths run in fp32 (abridgekv/gen_compress.py:359-360, 555; compresslm_packed_kv.py:608-613;
// compress_forward.py:695-727 under FlexAttention) for tight parity checks. It is a correctness mode: plain VALU
// arithmetic, one wave per (query token, KV head), keys in tiles of 64 (lane = key for QK^T, lane = 2 output dims for
// PV with the tile's probabilities broadcast from LDS).
#include <cstring>

#include "common.h"

namespace abkv {

struct F32Args {
  int mode;                    // 0: paged, per-request key limits; 1: dense, compression mask; 2: paged decode
  const float* q;
  long q_sb, q_st, q_sh;       // mode 1: [B, S, 32, 128]; modes 0/2: [T, 32, 128] (q_sb unused)
  // paged keys (modes 0 and 2): [num_pages, 2, 16, 8, 128]
  const float* kv;
  int num_pages;
  const int32_t* block_table;
  long bt_stride;
  int bt_width;
  // dense keys (mode 1): [B, S, 8, 128]
  const float* k;
  const float* v;
  long k_sb, k_ss, k_sh, v_sb, v_ss, v_sh;
  // mode 0
  const int32_t* tok_req;      // [T] request of every query token
  const int32_t* q_start;      // [B + 1]
  const int32_t* kv_start;     // [B]
  const int32_t* kv_limit;     // [B]
  const int32_t* kv_excluded;  // [B][2] physical [start, end) hidden from the request, or nullptr
  const int32_t* causal;       // [B] or nullptr (causal_default)
  int causal_default;
  // mode 2
  const int32_t* seq_lens;     // [B]
  int max_pages;
  // mode 1
  int block_c, codes_k, seq_len;
  const int32_t* prompt_len;   // [B] or nullptr
  const int32_t* head_quota;   // [32] or nullptr
  int retain_tail;             // retained tail T (0: none)
  int tail_policy;             // its policy (kTailStatic, kTailRolling, kTailSticky, kTailRaw)
  int pause_xattn;             // code <-> code attention in a block (kXattn*)
  int pause_passes;            // pause passes of codes_k rows per block
  int copy_rows;               // copy-region rows at the end of the seq_len rows
  int replay_rows;             // replay rows after each block's codes
  int replay_exclude;          // the codes do not see the block's last replay_rows content rows
  int num_tokens;
  float scale;
  float* out;
  long o_sb, o_st, o_sh;
  float* lse;                  // modes 0/2: [T, 32]; mode 1: [B, 32, S]; or nullptr
};

constexpr int kF32Waves = 4;

// LDS written by some lanes of a wave and read by others: order the accesses within the wave.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Compression-mask visibility of key row kr for query row qr (L = 1; _arith_mask_mod, abridgekv/compress_forward.py:
// 695-727, with the retained-tail term of _retained_tail_visible :99-124):
//   (k <= q) & (own-block content | earlier blocks' codes | raw-prompt content | earlier blocks' tail rows the policy
//   shows this row) | (code q & code k & same block), a code query never sees its own block's last T content rows,
//   and a code key of slot s is visible to a head only if s < quota.
__device__ __forceinline__ bool f32_visible(const F32Args& a, int qr, int kr, int plen, int quota) {
  return compress_visible(qr, kr, a.seq_len, a.copy_rows, a.block_c, a.codes_k, a.pause_passes,
                          a.block_c + a.pause_passes * a.codes_k + a.replay_rows, plen, quota, a.retain_tail,
                          a.tail_policy, a.pause_xattn, a.replay_rows, a.replay_exclude != 0);
}

__global__ __launch_bounds__(64 * kF32Waves) void attn_f32_kernel(F32Args a) {
  __shared__ float q_lds[kF32Waves][kGroup][kHeadDim];
  __shared__ float p_lds[kF32Waves][kGroup][64];
  const int w = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * kF32Waves + w;          // query token (mode 1: b * seq_len + row)
  const int kvh = blockIdx.y;
  if (t >= a.num_tokens) return;                      // whole wave exits together; no block barrier below

  // Which keys, and how a key row is addressed.
  int b = 0, qrow = 0, n_keys = 0, lim_lane = 0, plen = 0, ex_lo = 0, ex_hi = 0;
  const int32_t* table = nullptr;
  int quota[kGroup] = {1 << 30, 1 << 30, 1 << 30, 1 << 30};
  if (a.mode == 1) {
    b = t / a.seq_len;
    qrow = t - b * a.seq_len;
    const int per = a.block_c + a.pause_passes * a.codes_k + a.replay_rows;
    const int s0 = a.seq_len - a.copy_rows;
    // nothing after the query's own block is visible; a copy row sees up to itself
    n_keys = qrow >= s0 ? qrow + 1 : min(s0, (qrow / per + 1) * per);
    plen = a.prompt_len ? a.prompt_len[b] : 0;
    if (a.head_quota)
#pragma unroll
      for (int u = 0; u < kGroup; ++u) quota[u] = a.head_quota[kvh * kGroup + u];
  } else if (a.mode == 0) {
    b = a.tok_req[t];
    const int i = t - a.q_start[b];
    const int pos = a.kv_start[b] + i;
    const int limit = a.kv_limit[b];
    const bool causal = a.causal ? a.causal[b] != 0 : a.causal_default != 0;
    n_keys = min(causal ? min(limit, pos + 1) : limit, a.bt_width * kPage);
    table = a.block_table + (long)b * a.bt_stride;
    if (a.kv_excluded != nullptr) {
      ex_lo = a.kv_excluded[2 * b];
      ex_hi = a.kv_excluded[2 * b + 1];
    }
  } else {
    b = t;
    n_keys = max(min(a.seq_lens[b], a.max_pages * kPage), 0);
    table = a.block_table + (long)b * a.bt_stride;
  }
  lim_lane = n_keys;

  // Query heads of this KV head into LDS.
  const float* qbase = a.mode == 1 ? a.q + (long)b * a.q_sb + (long)qrow * a.q_st : a.q + (long)t * a.q_st;
  for (int i = lane; i < kGroup * kHeadDim; i += 64)
    q_lds[w][i / kHeadDim][i % kHeadDim] = qbase[(long)(kvh * kGroup + i / kHeadDim) * a.q_sh + (i % kHeadDim)];
  wave_sync();

  float m[kGroup], l[kGroup], o[kGroup][2];
#pragma unroll
  for (int u = 0; u < kGroup; ++u) {
    m[u] = -INFINITY;
    l[u] = 0.f;
    o[u][0] = o[u][1] = 0.f;
  }

  for (int j0 = 0; j0 < n_keys; j0 += 64) {
    const int j = j0 + lane;
    float s[kGroup];
    bool vis[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      vis[u] = j < lim_lane && (j < ex_lo || j >= ex_hi) && (a.mode != 1 || f32_visible(a, qrow, j, plen, quota[u]));
      s[u] = -INFINITY;
    }
    if (vis[0] || vis[1] || vis[2] || vis[3]) {
      const float* krow;
      if (a.mode == 1) {
        krow = a.k + (long)b * a.k_sb + (long)j * a.k_ss + (long)kvh * a.k_sh;
      } else {
        const int page = min(max(table[j / kPage], 0), a.num_pages - 1);
        krow = a.kv + (long)page * kPageElems + (j % kPage) * kSlotElems + kvh * kHeadDim;
      }
      float acc[kGroup] = {0.f, 0.f, 0.f, 0.f};
      for (int d = 0; d < kHeadDim; d += 4) {
        const floatx4 kx = *reinterpret_cast<const floatx4*>(krow + d);
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
          acc[u] = fmaf(q_lds[w][u][d], kx[0], acc[u]);
          acc[u] = fmaf(q_lds[w][u][d + 1], kx[1], acc[u]);
          acc[u] = fmaf(q_lds[w][u][d + 2], kx[2], acc[u]);
          acc[u] = fmaf(q_lds[w][u][d + 3], kx[3], acc[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < kGroup; ++u)
        if (vis[u]) s[u] = acc[u] * a.scale;
    }
    // online softmax per head over the tile
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      float tmax = s[u];
      for (int off = 32; off > 0; off >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, off, 64));
      const float m_new = fmaxf(m[u], tmax);
      const float alpha = m[u] == -INFINITY ? 0.f : expf(m[u] - m_new);
      const float p = vis[u] ? expf(s[u] - m_new) : 0.f;
      float psum = p;
      for (int off = 32; off > 0; off >>= 1) psum += __shfl_xor(psum, off, 64);
      l[u] = l[u] * alpha + psum;
      o[u][0] *= alpha;
      o[u][1] *= alpha;
      m[u] = m_new;
      p_lds[w][u][lane] = p;
    }
    wave_sync();
    const int n_tile = min(64, n_keys - j0);
    for (int jj = 0; jj < n_tile; ++jj) {
      const int jk = j0 + jj;
      const float* vrow;
      if (a.mode == 1) {
        vrow = a.v + (long)b * a.v_sb + (long)jk * a.v_ss + (long)kvh * a.v_sh;
      } else {
        const int page = min(max(table[jk / kPage], 0), a.num_pages - 1);
        vrow = a.kv + (long)page * kPageElems + kHalfElems + (jk % kPage) * kSlotElems + kvh * kHeadDim;
      }
      const float2 vx = *reinterpret_cast<const float2*>(vrow + 2 * lane);
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        const float p = p_lds[w][u][jj];
        o[u][0] = fmaf(p, vx.x, o[u][0]);
        o[u][1] = fmaf(p, vx.y, o[u][1]);
      }
    }
    wave_sync();
  }

#pragma unroll
  for (int u = 0; u < kGroup; ++u) {
    const int head = kvh * kGroup + u;
    const float inv = l[u] > 0.f ? 1.f / l[u] : 0.f;
    float* orow = a.mode == 1 ? a.out + (long)b * a.o_sb + (long)qrow * a.o_st + (long)head * a.o_sh
                              : a.out + (long)t * a.o_st + (long)head * a.o_sh;
    *reinterpret_cast<float2*>(orow + 2 * lane) = make_float2(o[u][0] * inv, o[u][1] * inv);
    if (a.lse != nullptr && lane == 0) {
      const float v = l[u] > 0.f ? m[u] + logf(l[u]) : -INFINITY;
      if (a.mode == 1)
        a.lse[((long)b * kHeadsQ + head) * a.seq_len + qrow] = v;
      else
        a.lse[(long)t * kHeadsQ + head] = v;
    }
  }
}

static int launch_f32(const F32Args& a, hipStream_t stream) {
  if (a.num_tokens <= 0) return 0;
  dim3 grid((a.num_tokens + kF32Waves - 1) / kF32Waves, kHeadsKV);
  hipLaunchKernelGGL(attn_f32_kernel, grid, dim3(64 * kF32Waves), 0, stream, a);
  return (int)hipGetLastError();
}

static F32Args f32_defaults() {
  F32Args a;
  memset(&a, 0, sizeof(a));
  return a;
}

}  // namespace abkv

extern "C" {

int abkv_decode_attn_f32(const float* q, long q_stride_seq, long q_stride_head, const float* kv_cache, int num_pages,
                         const int32_t* block_table, long block_table_stride, const int32_t* seq_lens, int num_seqs,
                         int max_pages_per_seq, float scale, float* out, long out_stride_seq, long out_stride_head,
                         float* lse, hipStream_t stream) {
  using namespace abkv;
  if (num_seqs <= 0) return 0;
  if (q == nullptr || kv_cache == nullptr || block_table == nullptr || seq_lens == nullptr || out == nullptr ||
      num_pages <= 0 || max_pages_per_seq <= 0 || block_table_stride < max_pages_per_seq)
    return (int)hipErrorInvalidValue;
  F32Args a = f32_defaults();
  a.mode = 2;
  a.q = q;
  a.q_st = q_stride_seq;
  a.q_sh = q_stride_head;
  a.kv = kv_cache;
  a.num_pages = num_pages;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.seq_lens = seq_lens;
  a.max_pages = max_pages_per_seq;
  a.num_tokens = num_seqs;
  a.scale = scale;
  a.out = out;
  a.o_st = out_stride_seq;
  a.o_sh = out_stride_head;
  a.lse = lse;
  return launch_f32(a, stream);
}

int abkv_paged_prefill_attn_f32(const float* q, long q_stride_t, long q_stride_h, const float* kv_cache, int num_pages,
                                const int32_t* block_table, long block_table_stride, int block_table_width,
                                const int32_t* q_start, const int32_t* kv_start, const int32_t* kv_limit,
                                const int32_t* kv_excluded, const int32_t* tok_req, int num_tokens,
                                const int32_t* causal, int causal_default, float scale, float* out, long out_stride_t,
                                long out_stride_h, float* lse, hipStream_t stream) {
  using namespace abkv;
  if (num_tokens <= 0) return 0;
  if (q == nullptr || kv_cache == nullptr || block_table == nullptr || q_start == nullptr || kv_start == nullptr ||
      kv_limit == nullptr || tok_req == nullptr || out == nullptr || num_pages <= 0 || block_table_width <= 0)
    return (int)hipErrorInvalidValue;
  F32Args a = f32_defaults();
  a.mode = 0;
  a.q = q;
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.kv = kv_cache;
  a.num_pages = num_pages;
  a.block_table = block_table;
  a.bt_stride = block_table_stride;
  a.bt_width = block_table_width;
  a.q_start = q_start;
  a.kv_start = kv_start;
  a.kv_limit = kv_limit;
  a.kv_excluded = kv_excluded;
  a.tok_req = tok_req;
  a.causal = causal;
  a.causal_default = causal_default;
  a.num_tokens = num_tokens;
  a.scale = scale;
  a.out = out;
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.lse = lse;
  return launch_f32(a, stream);
}

int abkv_prefill_masked_attn_f32(const float* q, long q_sb, long q_ss, long q_sh, const float* k, long k_sb,
                                 long k_ss, long k_sh, const float* v, long v_sb, long v_ss, long v_sh, int batch,
                                 int block_c, int codes_k, int num_blocks, int seq_len, const int32_t* prompt_len,
                                 const int32_t* head_quota, int retain_tail, int tail_policy, int pause_xattn,
                                 int pause_passes, int copy_rows, int replay_rows, int replay_exclude, float scale,
                                 float* out, long o_sb, long o_ss, long o_sh, float* lse,
                                 hipStream_t stream) {
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
  F32Args a = f32_defaults();
  a.mode = 1;
  a.q = q;
  a.q_sb = q_sb;
  a.q_st = q_ss;
  a.q_sh = q_sh;
  a.k = k;
  a.v = v;
  a.k_sb = k_sb;
  a.k_ss = k_ss;
  a.k_sh = k_sh;
  a.v_sb = v_sb;
  a.v_ss = v_ss;
  a.v_sh = v_sh;
  a.block_c = block_c;
  a.codes_k = codes_k;
  a.seq_len = seq_len;
  a.prompt_len = prompt_len;
  a.head_quota = head_quota;
  a.retain_tail = retain_tail;
  a.tail_policy = tail_policy;
  a.pause_xattn = pause_xattn;
  a.pause_passes = pause_passes;
  a.copy_rows = copy_rows;
  a.replay_rows = replay_rows;
  a.replay_exclude = replay_exclude;
  a.num_tokens = batch * seq_len;
  a.scale = scale;
  a.out = out;
  a.o_sb = o_sb;
  a.o_st = o_ss;
  a.o_sh = o_sh;
  a.lse = lse;
  return launch_f32(a, stream);
}

}  // extern "C"
