// attn_core.h - the pieces the decode attention kernels share (attn_dma.h's decode block,
// attn_verify.hip): the v2 blocking rule, the kernel arguments and the int8 K widening.
#pragma once
#include "mi_common.h"
#include "gemv_core.h"

namespace mi {

__device__ __forceinline__ uint32_t v2_ppw(uint32_t len, uint32_t tgt) {
  uint32_t p = (len + tgt - 1) / tgt;
  p = (p + 63u) & ~63u;
  return p < 64u ? 64u : p;
}

// list rows one decode work-group takes: the ct tiles of 16 columns of the matrix products
// hold 16 ct / GQA rows' q heads (the fused prep: one row)
__host__ __device__ constexpr uint32_t attn_rows_per_wg(uint32_t gqa, bool fused_prep, uint32_t ct) {
  return fused_prep || gqa == 0 || gqa > 16u * ct ? 1u : 16u * ct / gqa;
}
// column tiles for an M-row list: enough for every row's heads, at most 3 (f16 rows of 128) or
// 2 (int8 rows of 128, rows of 256: a third tile's accumulators would not leave two waves per
// SIMD, or any, the registers)
__host__ __device__ constexpr uint32_t attn_ct_cap(uint32_t hd, uint32_t kv8) {
  return hd == 128u && kv8 == 0u ? 3u : 2u;
}
__host__ inline uint32_t attn_col_tiles(uint32_t M, uint32_t gqa, uint32_t hd, uint32_t kv8) {
  const uint32_t need = (M * gqa + 15u) / 16u, cap = attn_ct_cap(hd, kv8);
  return need < 1u ? 1u : (need > cap ? cap : need);
}
// work-groups over the rows of an M-row list: RPW at a time, plus one for the split where the
// block size changes
__host__ inline uint32_t attn_row_groups(uint32_t M, uint32_t gqa, uint32_t ct) {
  const uint32_t rpw = attn_rows_per_wg(gqa, false, ct);
  return (M + rpw - 1) / rpw + (M > 1 && rpw > 1 ? 1u : 0u);
}

// 16-position groups whose cache rows one work-group stages for a paged cache (a block of
// ppw positions holds ppw / 16 groups; ppw is a multiple of 64)
constexpr uint32_t kMaxBlockGroups = 512;

struct AttnDecodeArgs {
  const uint32_t* ctrl;
  const float* attn_q;
  const void* kv_k;
  const void* kv_v;
  const uint16_t* k_scale;
  const uint16_t* v_scale;
  const uint32_t* pages;
  float* attn_part;
  size_t row_stride, head_stride, sc_row_stride, sc_head_stride;
  uint32_t page, M, q_heads, kv_heads, tgt;
  uint32_t kv_len;  // positions the cache holds; keys past it are never read (0 = unchecked)
  float scale;
  // the fused prep (attn_prep's work done by the decode kernel; f16 cache): the qkv partials
  // [S][M][qkv_n] and attn_prep's parameters
  const float* partials;
  const float* q_norm;
  const float* k_norm;
  const float* rope;
  float* attn_gate;
  uint32_t* ctrl_w;
  uint32_t S, qkv_n, k_off, v_off, rot_dim, gated;
  float eps;
};

// 8 consecutive K elements of one row, raw (f16: 16 bytes; int8: 8 bytes)
template <int KV8>
struct KvChunk {
  u4_t w;
};
template <>
struct KvChunk<1> {
  u2_t w;
};
// 8 K values of one row as an f16 MFMA operand (int8 values are exact in f16; their row
// scale is applied to the score afterwards)
template <int KV8>
__device__ __forceinline__ h8_t chunk_h8(const KvChunk<KV8>& c) {
  if constexpr (KV8 == 0) {
    return __builtin_bit_cast(h8_t, c.w);
  } else {
    // byte permute: each biased byte u = q8 + 128 under an f16 exponent byte 0x64 is the f16
    // 1024 + u; subtracting 1152 leaves q8 exactly (f16 integers up to 2048 are exact)
    const uint32_t x0 = c.w.x ^ 0x80808080u, x1 = c.w.y ^ 0x80808080u, hi = 0x64646464u;
    const h2_t bias = {(half_t)1152.0f, (half_t)1152.0f};
    const h2_t p0 = as_h2(__builtin_amdgcn_perm(hi, x0, 0x04010400u)) - bias;
    const h2_t p1 = as_h2(__builtin_amdgcn_perm(hi, x0, 0x04030402u)) - bias;
    const h2_t p2 = as_h2(__builtin_amdgcn_perm(hi, x1, 0x04010400u)) - bias;
    const h2_t p3 = as_h2(__builtin_amdgcn_perm(hi, x1, 0x04030402u)) - bias;
    return h8_t{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  }
}

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));

}  // namespace mi
