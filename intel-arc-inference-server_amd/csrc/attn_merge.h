// attn_merge.h - attn_reduce_v2's merge of a row's block partials (src/kernels/attn_v2.cl:383-428),
// as device pieces shared by the reduce launch (attn.hip) and the o GEMV's fused prologue
// (gemv_w4a16.hip), so the two form the same bits.
//
// For one (q head, row): M = max over the nb blocks of mx_b, f_b = exp(mx_b - M), sum =
// sum_b sm_b f_b, each dim's acc = sum_b acc_b f_b in ascending b, o = acc / sum, then
// rne(o) or, gated, rne(rne(o) * sigmoid(gate)): mathematically the reference's sequential
// rescaling merge, the roundings differing at the last place.
#pragma once
#include "mi_common.h"

namespace mi {

// the row's block count under the v2 blocking: keys [0, pos + m] (capped at kv_len when set),
// ppw(L) positions per block, at most tgt blocks
__device__ __forceinline__ uint32_t merge_blocks(uint32_t pos, uint32_t m, uint32_t kv_len, uint32_t tgt) {
  uint32_t L = pos + m + 1;
  if (kv_len && L > kv_len) L = kv_len;
  uint32_t p = (L + tgt - 1) / tgt;
  p = (p + 63u) & ~63u;
  p = p < 64u ? 64u : p;
  const uint32_t nb = (L - 1) / p + 1;
  return nb > tgt ? tgt : nb;
}

// One wave: the common max and the per-block factors of a (head, row) whose partial for block b
// sits at base + b * bstride ({mx, sm, acc[]}); lane l takes blocks l, l + 64, ... (mx_of /
// sm_of give block b's values); fac[b] = f_b; returns the weighted sum (every lane).
template <typename MxOf, typename SmOf>
__device__ __forceinline__ float merge_factors(uint32_t lane, uint32_t nb, MxOf mx_of, SmOf sm_of, float* fac) {
  float mx = -INFINITY;
  for (uint32_t b = lane; b < nb; b += 64) mx = fmaxf(mx, mx_of(b));
  mx = wave_max(mx);
  float sm = 0.f;
  for (uint32_t b = lane; b < nb; b += 64) {
    const float f = expf(mx_of(b) - mx);
    fac[b] = f;
    sm = __builtin_fmaf(sm_of(b), f, sm);
  }
  return wave_sum(sm);
}

// the merged value of one dim, rounded as attn_reduce writes it (act: mi_attn_shape.act)
__device__ __forceinline__ uint16_t merge_out(float acc, float sm, bool gated, float gate, uint32_t act = 0u) {
  const float o = acc / sm;
  return gated ? act_enc(act_round(o, act) * sigmoid_f32(gate), act) : act_enc(o, act);
}

}  // namespace mi
