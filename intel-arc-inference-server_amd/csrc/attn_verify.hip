// attn_verify.hip - the verify step's attention for many rows at once (the role of
// attn_verify_dpas / its bind rule, src/kernels/attn_verify_dpas.cl:383 and
// src/runtime/verify_attn.h:93-100): for M = 16, 32, 64 verify rows of a 16 q / 2 kv head
// model (GQA 8), the decode partials of attn_decode_v2's blocking, reduced by the same
// attn_reduce as the plain step.
//
// The plain decode kernel (attn_core.h) runs one row per work-group: every row of a verify list
// reads the whole KV block again. Here a work-group (kv head j, block blk, rows 8 c .. 8 c + 7)
// reads the block once for eight rows: wave w owns rows 8 c + 2 w and 8 c + 2 w + 1, and the 16
// columns of its matrix-core products are (row, q head) pairs, column n = row (n / 8), head
// j * 8 + n % 8. Per 16-position group of the block, as in the decode kernel:
//   scores  S^T = K Q^T on v_mfma_f32_16x16x32_f16, q split into an f16 high part and the f16
//           rounding of the remainder (two products, hi first);
//   softmax per column over the group's positions, online across groups in fp32; a position
//           at or past the column's row bound pos + row + 1 is -inf; a group with no position
//           for a column leaves that column's state unchanged (factor 1, weights 0);
//   P V     O^T = V^T W^T on v_mfma_f32_16x16x16_f16, the weights split hi + lo like q, V
//           staged per wave in LDS.
// Each wave walks all of the block's groups itself (no merge between waves), so a column's
// values depend only on its own row's keys and the block walked: rows with the same stride
// see the same groups in the same order whatever M is or which rows share their work-group.
// The rows of one list have at most two strides (ppw(L) changes once at most over 64 rows); a
// wave whose two rows differ walks the block once per stride, each row taking only its own.
// The partials attn_part[qh][tgt][M][HD + 2] = {max, sum, acc[HD]} are those of mi_attn_decode.
#include "mi_capi_internal.h"
#include "mi_common.h"
#include "attn_core.h"

namespace mi {
namespace {

template <int HD>
__global__ __launch_bounds__(256) void attn_verify_kernel(AttnDecodeArgs a) {
  constexpr uint32_t GQA = 8, RPW = 16 / GQA;  // rows per wave
  constexpr uint32_t KK = HD / 32, NT = HD / 16;
  constexpr uint32_t ROWB = HD * 2u;      // bytes per f16 row
  constexpr uint32_t VLD = ROWB / 64u;    // 16-byte V loads per lane (4 lanes per row)
  constexpr uint32_t CW = 32u;            // bytes of one 16-dim column
  constexpr uint32_t SV = 16u * ROWB;     // one wave's staged V group
  __shared__ __align__(16) unsigned char s_buf[4u * SV];

  const uint32_t t = opaque_tid(), lane = t & 63u, wave = t >> 6;
  const uint32_t qi = lane & 15u, qq = lane >> 4;
  const uint32_t j = blockIdx.x, blk = blockIdx.y;
  const uint32_t n_act = a.ctrl[CTRL_NACT], pos = a.ctrl[CTRL_POS];
  const uint32_t row0 = blockIdx.z * (4u * RPW) + wave * RPW;  // this wave's first row

  // per row of the wave: its key bound, stride and whether it has a block blk
  uint32_t rl[RPW], rs[RPW];
  bool ron[RPW];
#pragma unroll
  for (uint32_t r = 0; r < RPW; ++r) {
    const uint32_t m = row0 + r;
    uint32_t L = pos + m + 1;
    if (a.kv_len && L > a.kv_len) L = a.kv_len;
    const uint32_t s = v2_ppw(L, a.tgt);
    uint32_t nb = (L - 1) / s + 1;
    if (nb > a.tgt) nb = a.tgt;
    rl[r] = L;
    rs[r] = s;
    ron[r] = m < n_act && m < a.M && blk < nb;
  }
  // this lane's column: row row0 + qi / GQA, q head j GQA + qi % GQA
  const uint32_t crow = qi / GQA, chead = j * GQA + qi % GQA;
  uint32_t c_L = rl[0], c_s = rs[0];
  bool c_on = ron[0];
#pragma unroll
  for (uint32_t r = 1; r < RPW; ++r)
    if (crow == r) {
      c_L = rl[r];
      c_s = rs[r];
      c_on = ron[r];
    }

  // q as the B operand, in registers (each wave has its own rows): dims 32 kk + 8 qq + e
  h8_t qh[KK], ql[KK];
#pragma unroll
  for (uint32_t kk = 0; kk < KK; ++kk) {
    float v[8];
    if (c_on) {
      const float* qp = a.attn_q + ((size_t)(row0 + crow) * a.q_heads + chead) * HD + 32 * kk + 8 * qq;
      const f4_t q0 = *as_global(reinterpret_cast<const f4_t*>(qp));
      const f4_t q1 = *as_global(reinterpret_cast<const f4_t*>(qp + 4));
      v[0] = q0.x; v[1] = q0.y; v[2] = q0.z; v[3] = q0.w;
      v[4] = q1.x; v[5] = q1.y; v[6] = q1.z; v[7] = q1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half_t h = (half_t)v[e];
      qh[kk][e] = h;
      ql[kk][e] = (half_t)(v[e] - (float)h);
    }
  }

  float m_run = -INFINITY, l_run = 0.f;
  f4_t acc[NT];
#pragma unroll
  for (uint32_t tt = 0; tt < NT; ++tt) acc[tt] = f4_t{0.f, 0.f, 0.f, 0.f};
  unsigned char* sv = s_buf + wave * SV;
  auto sv_off = [](uint32_t r, uint32_t c) -> uint32_t { return r * ROWB + ((c ^ ((r >> 2) & 3u)) * CW); };
  const size_t hoff = (size_t)j * a.head_stride;
  const uint32_t vrow = lane >> 2, vpart = lane & 3u;

  // one walk per distinct stride among the wave's rows (uniform)
#pragma unroll
  for (uint32_t w = 0; w < RPW; ++w) {
    if (!ron[w]) continue;
    bool seen = false;
#pragma unroll
    for (uint32_t r = 0; r < w; ++r) seen = seen || (ron[r] && rs[r] == rs[w]);
    if (seen) continue;
    const uint32_t s = rs[w];
    uint32_t lmax = 0;
#pragma unroll
    for (uint32_t r = 0; r < RPW; ++r)
      if (ron[r] && rs[r] == s) lmax = max(lmax, rl[r]);
    const uint32_t p_begin = blk * s, p_end = min(p_begin + s, lmax);
    const bool mine = c_on && c_s == s;  // this lane's column takes part in this walk
    for (uint32_t p0 = p_begin; p0 < p_end; p0 += 16u) {
      const uint32_t glen = min(16u, p_end - p0);
      const uint32_t rb = __builtin_amdgcn_readfirstlane(a.pages ? a.pages[p0 / a.page] * a.page + p0 % a.page : p0);
      u4_t kc[KK];
      u4_t vc[VLD];
      if (qi < glen) {
        const uint16_t* kp = static_cast<const uint16_t*>(a.kv_k) + ((size_t)rb + qi) * a.row_stride + hoff + 8 * qq;
#pragma unroll
        for (uint32_t kk = 0; kk < KK; ++kk) kc[kk] = *as_global(reinterpret_cast<const u4_t*>(kp + 32 * kk));
      } else {
#pragma unroll
        for (uint32_t kk = 0; kk < KK; ++kk) kc[kk] = u4_t{0u, 0u, 0u, 0u};
      }
      if (vrow < glen) {
        const unsigned char* vb = static_cast<const unsigned char*>(a.kv_v) +
                                  (((size_t)rb + vrow) * a.row_stride + hoff) * 2u + vpart * (ROWB / 4u);
#pragma unroll
        for (uint32_t i = 0; i < VLD; ++i) vc[i] = *as_global(reinterpret_cast<const u4_t*>(vb + 16u * i));
      } else {
#pragma unroll
        for (uint32_t i = 0; i < VLD; ++i) vc[i] = u4_t{0u, 0u, 0u, 0u};
      }
      wave_lds_sync();  // this wave's previous group is read out of its staging area
#pragma unroll
      for (uint32_t i = 0; i < VLD; ++i) {
        const uint32_t byte = vpart * (ROWB / 4u) + 16u * i;
        *reinterpret_cast<u4_t*>(sv + sv_off(vrow, byte / CW) + byte % CW) = vc[i];
      }
      wave_lds_sync();
      // scores S^T[position 4 qq + r][column qi]
      f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk) {
        const h8_t kh = __builtin_bit_cast(h8_t, kc[kk]);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[kk], d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[kk], d, 0, 0, 0);
      }
      float sc[4];
      float mx = -INFINITY;
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) {
        const uint32_t p = p0 + 4u * qq + r;
        sc[r] = (mine && 4u * qq + r < glen && p < c_L) ? d[r] * a.scale : -INFINITY;
        mx = fmaxf(mx, sc[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);
      const bool none = m_new == -INFINITY;  // no position yet for this column: unchanged
      const float alpha = none ? 1.0f : expf(m_run - m_new);
      float wv[4];
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) wv[r] = none ? 0.f : expf(sc[r] - m_new);
      l_run = __builtin_fmaf(l_run, alpha, (wv[0] + wv[1]) + (wv[2] + wv[3]));
      m_run = m_new;
      if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (uint32_t tt = 0; tt < NT; ++tt) acc[tt] *= alpha;
      }
      h4_t bh, bl;
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) {
        const half_t h = (half_t)wv[r];
        bh[r] = h;
        bl[r] = (half_t)(wv[r] - (float)h);
      }
#pragma unroll
      for (uint32_t tt = 0; tt < NT; ++tt) {
        h4_t av;
#pragma unroll
        for (uint32_t jj = 0; jj < 4; ++jj)
          av[jj] = *reinterpret_cast<const half_t*>(sv + sv_off(4u * qq + jj, tt) + 2u * qi);
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bh, acc[tt], 0, 0, 0);
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bl, acc[tt], 0, 0, 0);
      }
    }
  }
  // the column's partial: the four lanes of a column hold a quarter of its positions' sums
  float l = l_run + __shfl_xor(l_run, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  if (c_on) {
    float* out = a.attn_part + (((size_t)chead * a.tgt + blk) * a.M + row0 + crow) * (HD + 2);
#pragma unroll
    for (uint32_t tt = 0; tt < NT; ++tt)
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) out[2 + 16u * tt + 4u * qq + r] = acc[tt][r];
    if (qq == 0) {
      out[0] = m_run;
      out[1] = l;
    }
  }
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_attn_verify_binds(uint32_t M, uint32_t kv_kind, uint32_t q_heads, uint32_t kv_heads) {
  // verify_attn.h:93-96 (verify_attn_wide_heads): 16 q / 2 kv heads, an f16 cache, 16, 32 or
  // 64 rows; every other list keeps the plain decode kernel
  return q_heads == 16 && kv_heads == 2 && kv_kind == 0 && (M == 16 || M == 32 || M == 64);
}

extern "C" int mi_attn_verify(const uint32_t* ctrl, const float* attn_q, const uint16_t* kv_k, const uint16_t* kv_v,
                              size_t row_stride, size_t head_stride, const uint32_t* pages, uint32_t page,
                              uint32_t kv_len, float* attn_part, uint32_t M, uint32_t tgt, const mi_attn_shape* shape,
                              void* stream) {
  if (!ctrl || !attn_q || !kv_k || !kv_v || !attn_part || !shape || M == 0 || M > 64 || tgt == 0)
    return mi_fail(MI_ERR_ARG, "attn_verify: bad arguments (M 1..64)");
  const uint32_t HD = shape->head_dim;
  if (HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_verify: head_dim must be 128 or 256");
  if (shape->kv_heads == 0 || shape->q_heads != 8 * shape->kv_heads)
    return mi_fail(MI_ERR_SHAPE, "attn_verify: q_heads must be 8 * kv_heads");
  if (pages && (page == 0 || page % 16)) return mi_fail(MI_ERR_SHAPE, "attn_verify: a KV page holds a multiple of 16 positions");
  if ((row_stride % 8) || (head_stride % 8))
    return mi_fail(MI_ERR_ARG, "attn_verify: KV strides must keep 8-element alignment");
  AttnDecodeArgs a{};
  a.ctrl = ctrl; a.attn_q = attn_q; a.kv_k = kv_k; a.kv_v = kv_v; a.pages = pages; a.attn_part = attn_part;
  a.row_stride = row_stride; a.head_stride = head_stride; a.page = page; a.M = M; a.q_heads = shape->q_heads;
  a.kv_heads = shape->kv_heads; a.tgt = tgt; a.kv_len = kv_len; a.scale = shape->scale;
  dim3 grid(shape->kv_heads, tgt, (M + 7) / 8);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (HD == 128) attn_verify_kernel<128><<<grid, 256, 0, st>>>(a);
  else attn_verify_kernel<256><<<grid, 256, 0, st>>>(a);
  return mi_hip(static_cast<int>(hipGetLastError()), "attn_verify");
}
