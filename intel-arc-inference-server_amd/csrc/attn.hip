// attn.hip - GQA decode attention over a (paged) fp16 or int8 KV cache, on gfx950.
//
// Replaces `attn_decode_v2` / `attn_reduce_v2` (src/kernels/attn_v2.cl:172, :383) and the
// int8 reader `attn_decode_v2_kv8` (src/kernels/kv8.cl:535) with the reference's contract:
//   * row m of a step attends to keys [0, pos + m]; the keys are cut into blocks of
//     ppw(L) = max(64, roundup64(ceil(L / tgt))) positions (attn_v2.cl:138-142) and the
//     grid is (kv_heads, tgt, M): at most `tgt` blocks per row for any L;
//   * each block leaves a partial {mx, sm, acc[HD]} per (q head, row) at
//     attn_part[qh][tgt][M][HD + 2]; the reduce merges a row's nb = (pos+m)/ppw + 1 blocks
//     in ascending block order with the reference's formula and writes
//     rne(acc / sm) (or the gated rne(rne(o) * sigmoid(gate)));
//   * KV paging (attn_v2.cl:123-131): logical position p lives at cache row
//     pages[p / page] * page + p % page; element (row, kv head, d) at
//     row * row_stride + head * head_stride + d, so both the reference's [pos][kvh][hd]
//     layout and this build's head-major [kvh][rows][hd] are expressible;
//   * int8 KV (kv8.h:126): k = float(q8) * f16(scale[row][kvh]), exact in fp32.
//
// Inside a block the work is MI355X-shaped rather than the B70's waves of 16: each of the
// four waves runs its own online softmax over 16-position groups with both products (q.K and
// P.V) on the matrix cores, and the waves merge once at the end (kernel comment below).
// Scores and the softmax are fp32; no atomics, so replays are bitwise.
#include "mi_capi_internal.h"
#include "mi_common.h"
#include "attn_core.h"
#include "attn_dma.h"
#include "attn_merge.h"

namespace mi {
namespace {


template <int HD, int KV8, int GQA, bool FP, int CT>
__global__ __launch_bounds__(256) void attn_decode_wave_kernel(AttnDecodeArgs a) {
  attn_block_dma<HD, KV8, GQA, FP, CT>(a, blockIdx.x, blockIdx.y, blockIdx.z);
}

// attn_v2.cl:383-428's merge of a row's nb block partials, as one common max M = max mx_b,
// factors f_b = exp(mx_b - M), sum = sum_b sm_b f_b and acc = sum_b acc_b f_b added in
// ascending b: mathematically the reference's sequential rescaling merge, the roundings
// differing at the last place. grid (q_heads, M), HD threads, one dim each. The first PRE
// blocks' values do not depend on the factors and are loaded before them, together with
// wave 0's (mx, sm) loads, so a merge of up to PRE blocks is one memory round trip; further
// blocks follow 64 at a time. PRE = 64 when tgt <= 64, else 128.
// ROT (attn_reduce_v2_kv8, kv8.cl:814-860; head_dim 256): the merged output is in the int8
// cache's rotated basis and is un-rotated per head before the gate.
template <bool ROT, uint32_t PRE>
__global__ __launch_bounds__(256) void attn_reduce_kernel(const uint32_t* __restrict__ ctrl,
                                                          const float* __restrict__ attn_part,
                                                          const float* __restrict__ attn_gate,
                                                          uint16_t* __restrict__ attn_out, uint32_t M,
                                                          uint32_t q_heads, uint32_t HD, uint32_t tgt,
                                                          uint32_t gated, uint32_t kv_len, uint32_t act) {
  __shared__ float fac[1024];
  __shared__ float s_sm;
  const uint32_t h = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
  const size_t PART = HD + 2;
  const float* base = attn_part + ((size_t)h * tgt * M + m) * PART;  // block b at + b * M * PART
  const size_t bstride = (size_t)M * PART;
  // The first PRE blocks' values and wave 0's (mx, sm) of blocks d and d + 64 do not depend on
  // the row's block count nb, so they are loaded before the control words arrive, bounded by
  // tgt (a slot past nb is read but never added); runs of 16 behind a uniform bound keep a
  // small tgt's merge to few loads.
  float v[PRE];
#pragma unroll
  for (uint32_t c = 0; c < PRE; c += 16)
    if (c < tgt) {
#pragma unroll
      for (uint32_t u = c; u < c + 16; ++u) v[u] = base[min(u, tgt - 1) * bstride + 2 + d];
    }
  float pm[2] = {0.f, 0.f}, ps[2] = {0.f, 0.f};
  if (d < 64) {
#pragma unroll
    for (uint32_t k = 0; k < 2; ++k)
      if (d + 64u * k < tgt) {
        pm[k] = base[(d + 64u * k) * bstride];
        ps[k] = base[(d + 64u * k) * bstride + 1];
      }
  }
  const float gv = gated && attn_gate ? attn_gate[((size_t)m * q_heads + h) * HD + d] : 0.f;
  if (m >= ctrl[CTRL_NACT]) return;  // uniform
  const uint32_t nb = merge_blocks(ctrl[CTRL_POS], m, kv_len, tgt);
  constexpr uint32_t BAT = 64;
  // wave 0: the common max and the per-block factors
  if (d < 64) {
    auto mx_of = [&](uint32_t b) { return b < 128u ? pm[b >> 6] : base[b * bstride]; };
    auto sm_of = [&](uint32_t b) { return b < 128u ? ps[b >> 6] : base[b * bstride + 1]; };
    const float sm = merge_factors(d, nb, mx_of, sm_of, fac);
    if (d == 0) s_sm = sm;
  }
  __syncthreads();
  float acc = 0.f;
#pragma unroll
  for (uint32_t u = 0; u < PRE; ++u)
    if (u < nb) acc = __builtin_fmaf(v[u], fac[u], acc);
  for (uint32_t b = PRE; b < nb; b += BAT) {
#pragma unroll
    for (uint32_t c = 0; c < BAT; c += 16)
      if (b + c < nb) {
#pragma unroll
        for (uint32_t u = c; u < c + 16; ++u) v[u] = base[min(b + u, nb - 1) * bstride + 2 + d];
      }
#pragma unroll
    for (uint32_t u = 0; u < BAT; ++u)
      if (b + u < nb) acc = __builtin_fmaf(v[u], fac[b + u], acc);
  }
  uint16_t r;
  if constexpr (ROT) {
    float o = acc / s_sm;
    __shared__ float xch[256];
    float v1[1] = {kv8_flip(o, kv8_sign_neg(d))};
    fwht256<1>(v1, d, xch);  // HD = 256: every thread of the work-group is here
    o = v1[0] * 0.0625f;
    if (gated && attn_gate)
      r = f2h(h2f(f2h(o)) * sigmoid_f32(gv));
    else
      r = f2h(o);
  } else {
    r = merge_out(acc, s_sm, gated && attn_gate, gv, act);
  }
  attn_out[(size_t)m * q_heads * HD + (size_t)h * HD + d] = r;
}

template <int HD, int KV8, int GQA, bool FP>
void launch_decode_ct(const AttnDecodeArgs& a, uint32_t ct, dim3 grid, hipStream_t st) {
  // the tiles an M-row list can use: GQA at most (16 rows), and attn_ct_cap
  constexpr int CAP = (int)attn_ct_cap(HD, KV8);
  constexpr int CTMAX = FP ? 1 : (GQA < CAP ? GQA : CAP);
  if (CTMAX >= 3 && ct == 3)
    attn_decode_wave_kernel<HD, KV8, GQA, FP, (CTMAX >= 3 ? 3 : 1)><<<grid, 256, 0, st>>>(a);
  else if (CTMAX >= 2 && ct == 2)
    attn_decode_wave_kernel<HD, KV8, GQA, FP, (CTMAX >= 2 ? 2 : 1)><<<grid, 256, 0, st>>>(a);
  else
    attn_decode_wave_kernel<HD, KV8, GQA, FP, 1><<<grid, 256, 0, st>>>(a);
}

// ct: the column tiles (attn_col_tiles; the fused prep: 1), grid z already sized for them
template <int HD, int KV8, bool FP>
int launch_decode(const AttnDecodeArgs& a, uint32_t gqa, uint32_t ct, dim3 grid, hipStream_t st) {
  switch (gqa) {
    case 1: launch_decode_ct<HD, KV8, 1, FP>(a, ct, grid, st); break;
    case 2: launch_decode_ct<HD, KV8, 2, FP>(a, ct, grid, st); break;
    case 4: launch_decode_ct<HD, KV8, 4, FP>(a, ct, grid, st); break;
    case 5: launch_decode_ct<HD, KV8, 5, FP>(a, ct, grid, st); break;
    case 6: launch_decode_ct<HD, KV8, 6, FP>(a, ct, grid, st); break;
    case 8: launch_decode_ct<HD, KV8, 8, FP>(a, ct, grid, st); break;
    default: return -1;
  }
  return 0;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

uint32_t mi_attn_ppw(uint32_t len, uint32_t tgt) {
  uint32_t p = (len + tgt - 1) / tgt;
  p = (p + 63u) & ~63u;
  return p < 64u ? 64u : p;
}

int mi_attn_decode(const uint32_t* ctrl, const float* attn_q, uint32_t kv_kind, const void* kv_k,
                   const void* kv_v, const uint16_t* k_scale, const uint16_t* v_scale, size_t row_stride,
                   size_t head_stride, size_t sc_row_stride, size_t sc_head_stride, const uint32_t* pages,
                   uint32_t page, uint32_t kv_len, float* attn_part, uint32_t M, uint32_t tgt,
                   const mi_attn_shape* shape, void* stream) {
  if (!ctrl || !attn_q || !kv_k || !kv_v || !attn_part || !shape || M == 0 || M > 16 || tgt == 0)
    return mi_fail(MI_ERR_ARG, "attn_decode: bad arguments");
  if (kv_kind > 1 || (kv_kind == 1 && (!k_scale || !v_scale)))
    return mi_fail(MI_ERR_ARG, "attn_decode: kv_kind 0 (fp16) or 1 (int8 + fp16 scales)");
  const uint32_t HD = shape->head_dim;
  if (HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_decode: head_dim must be 128 or 256");
  const uint32_t gqa = shape->kv_heads ? shape->q_heads / shape->kv_heads : 0;
  if (shape->kv_heads == 0 || shape->q_heads % shape->kv_heads ||
      !(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 5 || gqa == 6 || gqa == 8))
    return mi_fail(MI_ERR_SHAPE, "attn_decode: q_heads / kv_heads must be 1, 2, 4, 5, 6 or 8");
  if (pages && (page == 0 || page % 16))
    return mi_fail(MI_ERR_SHAPE, "attn_decode: a KV page holds a multiple of 16 positions");
  if (pages && (!kv_len || mi_attn_ppw(kv_len, tgt) / 16 > kMaxBlockGroups))
    return mi_fail(MI_ERR_SHAPE, "attn_decode: a paged cache needs kv_len, and at most 8192 positions per block");
  if ((row_stride % 8) || (head_stride % 8))
    return mi_fail(MI_ERR_ARG, "attn_decode: KV strides must keep 8-element alignment");
  AttnDecodeArgs a{};
  a.ctrl = ctrl; a.attn_q = attn_q; a.kv_k = kv_k; a.kv_v = kv_v; a.k_scale = k_scale; a.v_scale = v_scale;
  a.pages = pages; a.attn_part = attn_part; a.row_stride = row_stride; a.head_stride = head_stride;
  a.sc_row_stride = sc_row_stride; a.sc_head_stride = sc_head_stride; a.page = page; a.M = M;
  a.q_heads = shape->q_heads; a.kv_heads = shape->kv_heads; a.tgt = tgt; a.kv_len = kv_len; a.scale = shape->scale;
  const uint32_t ct = attn_col_tiles(M, gqa, HD, kv_kind);
  dim3 grid(shape->kv_heads, tgt, attn_row_groups(M, gqa, ct));
  hipStream_t st = (hipStream_t)stream;
  if (HD == 128) {
    if (kv_kind == 0) launch_decode<128, 0, false>(a, gqa, ct, grid, st);
    else launch_decode<128, 1, false>(a, gqa, ct, grid, st);
  } else {
    if (kv_kind == 0) launch_decode<256, 0, false>(a, gqa, ct, grid, st);
    else launch_decode<256, 1, false>(a, gqa, ct, grid, st);
  }
  return mi_hip((int)hipGetLastError(), "attn_decode");
}

int mi_attn_prep_decode(uint32_t* ctrl, const float* partials, uint32_t S, uint32_t M, const mi_attn_shape* shape,
                        const float* q_norm, const float* k_norm, const float* rope, float* attn_gate,
                        uint16_t* kv_k, uint16_t* kv_v, size_t row_stride, size_t head_stride,
                        const uint32_t* pages, uint32_t page, uint32_t kv_len, float* attn_part, uint32_t tgt,
                        void* stream) {
  if (!ctrl || !partials || !shape || !rope || !kv_k || !kv_v || !attn_part || S == 0 || M == 0 || M > 8 ||
      tgt == 0)
    return mi_fail(MI_ERR_ARG, "attn_prep_decode: bad arguments (M <= 8)");
  if (shape->act) return mi_fail(MI_ERR_SHAPE, "attn_prep_decode: f16 activations only");
  const uint32_t HD = shape->head_dim;
  if (HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_prep_decode: head_dim must be 128 or 256");
  const uint32_t gqa = shape->kv_heads ? shape->q_heads / shape->kv_heads : 0;
  if (shape->kv_heads == 0 || shape->q_heads % shape->kv_heads ||
      !(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 5 || gqa == 6 || gqa == 8))
    return mi_fail(MI_ERR_SHAPE, "attn_prep_decode: q_heads / kv_heads must be 1, 2, 4, 5, 6 or 8");
  if (shape->rot_dim > HD || shape->rot_dim % 2)
    return mi_fail(MI_ERR_SHAPE, "attn_prep_decode: inconsistent rotary dims");
  if (pages && (page == 0 || page % 16))
    return mi_fail(MI_ERR_SHAPE, "attn_prep_decode: a KV page holds a multiple of 16 positions");
  if (pages && (!kv_len || mi_attn_ppw(kv_len, tgt) / 16 > kMaxBlockGroups))
    return mi_fail(MI_ERR_SHAPE, "attn_prep_decode: a paged cache needs kv_len, and at most 8192 positions per block");
  if ((row_stride % 8) || (head_stride % 8))
    return mi_fail(MI_ERR_ARG, "attn_prep_decode: KV strides must keep 8-element alignment");
  AttnDecodeArgs a{};
  a.ctrl = ctrl; a.kv_k = kv_k; a.kv_v = kv_v; a.pages = pages; a.attn_part = attn_part;
  a.row_stride = row_stride; a.head_stride = head_stride; a.page = page; a.M = M; a.q_heads = shape->q_heads;
  a.kv_heads = shape->kv_heads; a.tgt = tgt; a.kv_len = kv_len; a.scale = shape->scale;
  a.partials = partials; a.q_norm = q_norm; a.k_norm = k_norm; a.rope = rope; a.attn_gate = attn_gate;
  a.ctrl_w = ctrl; a.S = S; a.qkv_n = shape->qkv_n; a.k_off = shape->k_off; a.v_off = shape->v_off;
  a.rot_dim = shape->rot_dim; a.gated = shape->gated; a.eps = shape->eps;
  dim3 grid(shape->kv_heads, tgt, M);
  hipStream_t st = (hipStream_t)stream;
  if (HD == 128) launch_decode<128, 0, true>(a, gqa, 1, grid, st);
  else launch_decode<256, 0, true>(a, gqa, 1, grid, st);
  return mi_hip((int)hipGetLastError(), "attn_prep_decode");
}

int mi_attn_reduce(const uint32_t* ctrl, const float* attn_part, const float* attn_gate, uint16_t* attn_out,
                   uint32_t M, uint32_t tgt, uint32_t kv_len, const mi_attn_shape* shape, void* stream) {
  if (!ctrl || !attn_part || !attn_out || !shape || M == 0 || tgt == 0 || tgt > 1024)
    return mi_fail(MI_ERR_ARG, "attn_reduce: bad arguments (tgt <= 1024)");
  const uint32_t HD = shape->head_dim;
  if (HD != 64 && HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_reduce: head_dim 64/128/256");
  if (shape->act > 1) return mi_fail(MI_ERR_ARG, "attn_reduce: act is 0 (f16) or 1 (bf16)");
  if (tgt <= 64)
    attn_reduce_kernel<false, 64><<<dim3(shape->q_heads, M), HD, 0, (hipStream_t)stream>>>(
        ctrl, attn_part, attn_gate, attn_out, M, shape->q_heads, HD, tgt, shape->gated, kv_len, shape->act);
  else
    attn_reduce_kernel<false, 128><<<dim3(shape->q_heads, M), HD, 0, (hipStream_t)stream>>>(
        ctrl, attn_part, attn_gate, attn_out, M, shape->q_heads, HD, tgt, shape->gated, kv_len, shape->act);
  return mi_hip((int)hipGetLastError(), "attn_reduce");
}

int mi_attn_reduce_kv8(const uint32_t* ctrl, const float* attn_part, const float* attn_gate, uint16_t* attn_out,
                       uint32_t M, uint32_t tgt, uint32_t kv_len, const mi_attn_shape* shape, void* stream) {
  if (!ctrl || !attn_part || !attn_out || !shape || M == 0 || tgt == 0 || tgt > 1024)
    return mi_fail(MI_ERR_ARG, "attn_reduce_kv8: bad arguments (tgt <= 1024)");
  if (shape->head_dim != 256)
    return mi_fail(MI_ERR_SHAPE, "attn_reduce_kv8: the rotation is defined for head_dim 256 only");
  if (shape->act) return mi_fail(MI_ERR_SHAPE, "attn_reduce_kv8: f16 activations only");
  if (tgt <= 64)
    attn_reduce_kernel<true, 64><<<dim3(shape->q_heads, M), 256, 0, (hipStream_t)stream>>>(
        ctrl, attn_part, attn_gate, attn_out, M, shape->q_heads, 256, tgt, shape->gated, kv_len, 0u);
  else
    attn_reduce_kernel<true, 128><<<dim3(shape->q_heads, M), 256, 0, (hipStream_t)stream>>>(
        ctrl, attn_part, attn_gate, attn_out, M, shape->q_heads, 256, tgt, shape->gated, kv_len, 0u);
  return mi_hip((int)hipGetLastError(), "attn_reduce_kv8");
}

}  // extern "C"
