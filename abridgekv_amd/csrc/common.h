// Shared device helpers for the abridged-KV kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace abkv {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Paged cache geometry of the served model (Qwen3-4B attention: 8 KV heads x 128, pages of 16 slots):
// one page of one layer is [2 (K,V)][16 slots][8 heads][128 dims] bf16 = 64 KiB.
constexpr int kPage = 16;
constexpr int kHeadsKV = 8;
constexpr int kHeadDim = 128;
constexpr int kGroup = 4;                                  // query heads per KV head
constexpr int kHeadsQ = kHeadsKV * kGroup;
constexpr int kSlotElems = kHeadsKV * kHeadDim;            // 1024 elements = 2 KiB per slot per K or V
constexpr int kHalfElems = kPage * kSlotElems;             // 16384 elements = 32 KiB (K half of a page)
constexpr int kPageElems = 2 * kHalfElems;                 // 32768 elements = 64 KiB

// Retained-tail policies (retain_tail_policy): which later rows see an earlier block's last T content rows.
constexpr int kTailStatic = 0;   // every later row
constexpr int kTailRolling = 1;  // the next block's i-th content row sees the tail's rows i .. T-1
constexpr int kTailSticky = 2;   // every content row of the next block
constexpr int kTailRaw = 3;      // the rolling window of raw_tail (compress_forward.py:89-96): the codes see the whole
                                 // block, their own tail included (code_excluded_tail = 0, :309-311)

// pause_xattn: which code rows of its own pass and block a code row sees (compress_forward.py:313-314, 622-625).
constexpr int kXattnFull = 0;     // all of them (bidirectional)
constexpr int kXattnCausal = 1;   // those at or before its own position
constexpr int kXattnNone = 2;     // none, itself included

// Whether content row kw (in-block offset) of block kb is a retained-tail row visible to row qw of block qb under the
// policy (abridgekv/compress_forward.py:99-124; the caller adds causality, the raw prompt and the codes' exclusion of
// their own block's tail).
__device__ __forceinline__ bool tail_visible(int policy, int tail, int C, int qb, int qw, int kb, int kw) {
  if (kw >= C || kw < C - tail) return false;
  if (policy == kTailStatic) return kb < qb;
  return qw < C && kb + 1 == qb && (policy == kTailSticky || kw - (C - tail) >= qw);
}

// Visibility of key row kv to query row q (sequence rows) under the compression mask over blocks of
// [C content | L pause passes of K code rows | R replay rows] (per = C + L K + R; abridgekv/compress_forward.py:
// 566-649, _mask_mod):
//   causal & (own-block content | earlier blocks' final-pass codes | raw-prompt content (< plen) | retained tail
//             | a replay row's own block's final pass and replay rows | for content row i, the previous block's
//             replay rows r >= i (_replay_tail_visible))
//   | a code row's own block's previous pass | its own pass by xattn,
// less a code row's own block's last `tail` content rows (R of them with rx: code_exclude_replay_tail; none under
// kTailRaw), and less a
// code key whose slot (its index within its pass) is >= quota. The last `copy` of the S rows are the copy region
// (copy_lambda, :631-633): they see the last block's final pass (slot < quota) and the copy rows up to themselves,
// and no other row sees them. K = 0 (no codes) is block-local causal attention. With L = 1, R = 0 and copy = 0
// (compile-time constants at most call sites) the pass, replay and copy arithmetic folds away.
__device__ __forceinline__ bool compress_visible(int q, int kv, int S, int copy, int C, int K, int L, int per,
                                                 int plen, int quota, int tail, int policy, int xattn, int R = 0,
                                                 bool rx = false) {
  if (kv >= S || q >= S) return false;
  const int S0 = S - copy;                                  // rows of the compressed layout
  if (copy > 0 && q >= S0) {
    if (kv >= S0) return kv <= q;
    const int lo = S0 - per + C + (L - 1) * K;              // the last block's final pass
    return kv >= lo && kv - lo < min(K, quota);
  }
  if (copy > 0 && kv >= S0) return false;
  const int qb = q / per, kb = kv / per;
  const int qw = q - qb * per, kw = kv - kb * per;
  const int code_end = C + L * K;                           // in-block end of the code rows
  const bool kc = kw < C, qc = qw < C;
  const bool krep = R > 0 && kw >= code_end, qrep = R > 0 && qw >= code_end;
  const bool kcode = !kc && !krep, qcode = !qc && !qrep;
  const int kp = L == 1 ? 1 : (kw - C) / K + 1;            // pass of a code key (1..L)
  const int qp = L == 1 ? 1 : (qw - C) / K + 1;            // pass of a code query
  const int X = rx ? R : policy == kTailRaw ? 0 : tail;    // the own-block content rows hidden from the codes
  bool v = (kc && kb == qb) || (kcode && kp == L && kb < qb) || (kc && kb * C + kw < plen) ||
           tail_visible(policy, tail, C, qb, qw, kb, kw);
  if (R > 0)
    v = v || (qrep && kb == qb && (krep || (kcode && kp == L))) || (qc && krep && kb + 1 == qb && kw - code_end >= qw);
  v = v && kv <= q;
  const bool own_codes = qcode && kcode && kb == qb;
  v = v || (own_codes && kp + 1 == qp);
  v = v || (own_codes && kp == qp && (xattn == kXattnFull || (xattn == kXattnCausal && kv <= q)));
  v = v && !(qcode && kb == qb && kc && kw >= C - X);
  return v && (!kcode || kw - C - (kp - 1) * K < quota);
}

__device__ __forceinline__ floatx4 mfma16x16x32(const bf16x8 a, const bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  // v_cvt_pk_bf16_f32: round-to-nearest-even of both halves
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float xor_shfl(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Reductions over the lane pairs {l, l ^ 16} and {l, l ^ 32} with gfx950's v_permlane16_swap / v_permlane32_swap:
// with both operands = v, the two results hold v[l] and v[l ^ 16] (resp. ^ 32) in some order, so combining them
// reduces the pair in VALU (no LDS round trip).
__device__ __forceinline__ float max_xor16(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace abkv
