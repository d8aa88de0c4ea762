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
// Inside a block the work is MI355X-shaped rather than the B70's waves of 16:
//   * one K or V row of HD dims is read by HD/8 lanes, 16 bytes (fp16) or 8 bytes (int8)
//     each - a 64-lane wave covers 4 (HD 128) or 2 (HD 256) positions with coalesced
//     256/512-byte row reads; the block's rows of one kv head are contiguous in the
//     head-major layout;
//   * all GQA q heads of the kv head share each K/V load (q held in registers, fp32);
//   * the block is walked in chunks of 64 positions, each a single HBM round trip; the
//     q.K scores run on the matrix cores, the online softmax per chunk (not per 16-position
//     wave) in LDS, and P.V on the vector ALUs (kernel comment below).
// Scores and the softmax are fp32; no atomics, so replays are bitwise.
#include "mi_capi_internal.h"
#include "mi_common.h"

namespace mi {
namespace {


__device__ __forceinline__ uint32_t v2_ppw(uint32_t len, uint32_t tgt) {
  uint32_t p = (len + tgt - 1) / tgt;
  p = (p + 63u) & ~63u;
  return p < 64u ? 64u : p;
}

// page-table entries one work-group stages (a block of ppw positions spans at most
// ppw / page + 1 pages)
constexpr uint32_t kMaxBlockPages = 256;

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
};

// 8 consecutive KV elements of one row, raw (f16: 16 bytes; int8: 8 bytes)
template <int KV8>
struct KvChunk {
  u4_t w;
};
template <>
struct KvChunk<1> {
  u2_t w;
  uint16_t s;
};

template <int KV8>
__device__ __forceinline__ KvChunk<KV8> load_chunk(const void* base, const uint16_t* sc, size_t off, size_t soff) {
  KvChunk<KV8> c;
  if constexpr (KV8 == 0) {
    c.w = *reinterpret_cast<const u4_t*>(static_cast<const uint16_t*>(base) + off);
  } else {
    c.w = *reinterpret_cast<const u2_t*>(static_cast<const int8_t*>(base) + off);
    c.s = sc[soff];
  }
  return c;
}
template <int KV8>
__device__ __forceinline__ void zero_chunk(KvChunk<KV8>& c) {
  if constexpr (KV8 == 0) c.w = u4_t{0u, 0u, 0u, 0u};
  else { c.w = u2_t{0u, 0u}; c.s = 0; }
}
// the 8 values as fp32: f16 widened exactly, or int8 * f16(scale) (exact in fp32, kv8.h:126)
template <int KV8>
__device__ __forceinline__ void widen_chunk(const KvChunk<KV8>& c, float (&v)[8]) {
  if constexpr (KV8 == 0) {
    const uint32_t ws[4] = {c.w.x, c.w.y, c.w.z, c.w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = h2f((uint16_t)(ws[i] & 0xFFFFu));
      v[2 * i + 1] = h2f((uint16_t)(ws[i] >> 16));
    }
  } else {
    const float s = h2f(c.s);
    const uint32_t ws[2] = {c.w.x, c.w.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)((ws[i / 4] >> (8 * (i % 4))) & 0xFFu) * s;
  }
}

// 8 KV values of one row as the f16 B operand of an MFMA (int8 values are exact in f16;
// their row scale is applied to the score afterwards)
template <int KV8>
__device__ __forceinline__ h8_t chunk_h8(const KvChunk<KV8>& c) {
  if constexpr (KV8 == 0) {
    return __builtin_bit_cast(h8_t, c.w);
  } else {
    h8_t r;
    const uint32_t ws[2] = {c.w.x, c.w.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = (half_t)(float)(int8_t)((ws[i / 4] >> (8 * (i % 4))) & 0xFFu);
    return r;
  }
}

// HD: head dim; KV8: int8 KV; GQA: q heads per kv head. A work-group walks its block in
// chunks of 64 positions; every thread issues all of its K and V loads for a chunk
// together, one chunk ahead of the one it computes when DB is set.
//   scores  on the matrix cores: wave w computes the 16 x 16 tile (q heads padded to 16) x
//           (positions 16w .. 16w+15) with v_mfma_f32_16x16x32_f16, A = q split into an f16
//           high part and the f16 rounding of the remainder (two MFMAs: the dot is fp32
//           accurate), B = the K rows, read 16 bytes per lane (lane l: position l % 16,
//           dims 8 (l / 16) + 32 kk) - no cross-lane reduction at all;
//   softmax per chunk per head in LDS (max, exp, sum), an online rescale between chunks;
//   P V     on the vector ALUs: HD / 8 lanes own a V row (8 dims, 16 bytes each), the
//           256 / (HD / 8) row slots accumulate sum_p w_p v_p and are merged in LDS in slot
//           order at the end.
// DB: double-buffer the chunks (blocks longer than one chunk); without it the registers of
// one chunk's K and V are all a thread holds.
template <int HD, int KV8, int GQA, bool DB>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecodeArgs a) {
  constexpr uint32_t CH = 64, KK = HD / 32;
  constexpr uint32_t LP = HD / 8, SLOTS = 256 / LP, VU = CH / SLOTS;
  __shared__ float sc[GQA][CH];
  __shared__ float st_alpha[GQA], st_m[GQA], st_l[GQA];
  __shared__ float red[SLOTS][GQA][HD];
  __shared__ uint32_t s_pages[kMaxBlockPages];  // the block's page-table entries (paged KV)

  const uint32_t j = blockIdx.x, blk = blockIdx.y, m = blockIdx.z;
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t slot = t / LP, dg = t % LP, d0 = dg * 8;
  const uint32_t qi = lane & 15u, qq = lane >> 4;
  const uint32_t n_act = a.ctrl[CTRL_NACT];
  if (m >= n_act) return;
  const uint32_t pos = a.ctrl[CTRL_POS];
  uint32_t L = pos + m + 1;
  if (a.kv_len && L > a.kv_len) L = a.kv_len;
  const uint32_t s = v2_ppw(L, a.tgt);
  uint32_t nb = (L - 1) / s + 1;
  if (nb > a.tgt) nb = a.tgt;
  if (blk >= nb) return;
  const uint32_t p_begin = blk * s, p_end = min(p_begin + s, L);

  float acc[GQA][8];
#pragma unroll
  for (uint32_t g = 0; g < GQA; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  if (t < GQA) {
    st_m[t] = -INFINITY;
    st_l[t] = 0.f;
  }

  // A paged cache's entries for this block are read once, into LDS, so a chunk's K/V loads
  // never wait on a page-table load first.
  const uint32_t pg0 = a.pages ? p_begin / a.page : 0u;
  if (a.pages) {
    const uint32_t np = (p_end - 1) / a.page - pg0 + 1;
    for (uint32_t i = t; i < np; i += 256u) s_pages[i] = a.pages[pg0 + i];
    __syncthreads();
  }
  auto row_of = [&](uint32_t p) -> size_t {
    return a.pages ? (size_t)s_pages[p / a.page - pg0] * a.page + p % a.page : (size_t)p;
  };
  const size_t hoff = (size_t)j * a.head_stride;
  const size_t shoff = (size_t)j * a.sc_head_stride;
  const uint32_t pk = 16u * wave + qi;  // this lane's score position within the chunk
  // chunk c's K and V rows into registers (zeros past the block's end)
  auto load_kv = [&](uint32_t c0, KvChunk<KV8> (&kc)[KK], KvChunk<KV8> (&vc)[VU]) {
    const uint32_t clen = c0 < p_end ? min(CH, p_end - c0) : 0u;
    if (pk < clen) {
      const size_t row = row_of(c0 + pk);
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk)
        kc[kk] = load_chunk<KV8>(a.kv_k, a.k_scale, row * a.row_stride + hoff + 32 * kk + 8 * qq,
                                 row * a.sc_row_stride + shoff);
    } else {
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk) zero_chunk<KV8>(kc[kk]);
    }
#pragma unroll
    for (uint32_t u = 0; u < VU; ++u) {
      const uint32_t pl = u * SLOTS + slot;
      if (pl < clen) {
        const size_t row = row_of(c0 + pl);
        vc[u] = load_chunk<KV8>(a.kv_v, a.v_scale, row * a.row_stride + hoff + d0, row * a.sc_row_stride + shoff);
      } else {
        zero_chunk<KV8>(vc[u]);
      }
    }
  };
  // DB: chunk c + 1's loads are issued before chunk c is used, and the barriers in the loop
  // order LDS only, so those loads stay in flight across them.
  KvChunk<KV8> kc[KK], vc[VU];
  load_kv(p_begin, kc, vc);  // the first chunk's loads go out before q is read
  // q as the MFMA A operand: row qi = head (zero past GQA), k = 32 kk + 8 qq + e
  h8_t qhi[KK], qlo[KK];
#pragma unroll
  for (uint32_t kk = 0; kk < KK; ++kk) {
    float v[8];
    if (qi < GQA) {
      const float* qp = a.attn_q + ((size_t)m * a.q_heads + j * GQA + qi) * HD + 32 * kk + 8 * qq;
      const f4_t q0 = *reinterpret_cast<const f4_t*>(qp);
      const f4_t q1 = *reinterpret_cast<const f4_t*>(qp + 4);
      v[0] = q0.x; v[1] = q0.y; v[2] = q0.z; v[3] = q0.w;
      v[4] = q1.x; v[5] = q1.y; v[6] = q1.z; v[7] = q1.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const half_t h = (half_t)v[e];
      qhi[kk][e] = h;
      qlo[kk][e] = (half_t)(v[e] - (float)h);
    }
  }
  for (uint32_t c0 = p_begin; c0 < p_end; c0 += CH) {
    const uint32_t clen = min(CH, p_end - c0);
    KvChunk<KV8> kn[KK], vn[VU];
    if constexpr (DB) load_kv(c0 + CH, kn, vn);
    // scores
    f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t kk = 0; kk < KK; ++kk) {
      const h8_t b = chunk_h8<KV8>(kc[kk]);
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qhi[kk], b, d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qlo[kk], b, d, 0, 0, 0);
    }
    float rs = a.scale;
    if constexpr (KV8 == 1) rs = a.scale * h2f(kc[0].s);
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
      const uint32_t head = 4u * qq + r;
      if (head < GQA && pk < clen) sc[head][pk] = d[r] * rs;
    }
    lds_barrier();
    // chunk max, weights and chunk sum: wave w owns heads w, w + 4
    for (uint32_t g = wave; g < GQA; g += 4) {
      const float v = lane < clen ? sc[g][lane] : -INFINITY;
      const float mx = wave_max(v);
      const float m_old = st_m[g];
      const float m_new = fmaxf(m_old, mx);
      const float w = lane < clen ? expf(v - m_new) : 0.f;
      if (lane < clen) sc[g][lane] = w;
      const float sum = wave_sum(w);
      if (lane == 0) {
        const float alpha = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
        st_alpha[g] = alpha;
        st_l[g] = __builtin_fmaf(st_l[g], alpha, sum);
        st_m[g] = m_new;
      }
    }
    lds_barrier();
    // rescale, then accumulate w * v from the registers loaded above
#pragma unroll
    for (uint32_t g = 0; g < GQA; ++g) {
      const float al = st_alpha[g];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[g][i] *= al;
    }
#pragma unroll
    for (uint32_t u = 0; u < VU; ++u) {
      const uint32_t pl = u * SLOTS + slot;
      if (pl < clen) {
        float v[8];
        widen_chunk<KV8>(vc[u], v);
#pragma unroll
        for (uint32_t g = 0; g < GQA; ++g) {
          const float w = sc[g][pl];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] = __builtin_fmaf(w, v[i], acc[g][i]);
        }
      }
    }
    lds_barrier();
    if constexpr (DB) {
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk) kc[kk] = kn[kk];
#pragma unroll
      for (uint32_t u = 0; u < VU; ++u) vc[u] = vn[u];
    } else if (c0 + CH < p_end) {
      load_kv(c0 + CH, kc, vc);
    }
  }
  // merge the row slots in slot order through LDS
#pragma unroll
  for (uint32_t g = 0; g < GQA; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) red[slot][g][d0 + i] = acc[g][i];
  __syncthreads();
  for (uint32_t idx = t; idx < GQA * HD; idx += 256) {
    const uint32_t g = idx / HD, dd = idx % HD;
    float v = red[0][g][dd];
#pragma unroll
    for (uint32_t sl = 1; sl < SLOTS; ++sl) v += red[sl][g][dd];
    float* out = a.attn_part + (((size_t)(j * GQA + g) * a.tgt + blk) * a.M + m) * (HD + 2);
    out[2 + dd] = v;
    if (dd == 0) {
      out[0] = st_m[g];
      out[1] = st_l[g];
    }
  }
}

// grid (q_heads, M), HD lanes: attn_v2.cl:383-428's merge of a row's nb block partials.
// Phase 1 reads every block's (mx, sm) in parallel and forms the common max M = max mx
// and each block's factor exp(mx_b - M); phase 2 sums acc_b * factor_b in ascending b with
// all the loads independent of each other. Mathematically the reference's sequential
// rescaling merge; the roundings differ at the last place only.
// ROT (attn_reduce_v2_kv8, kv8.cl:814-860; head_dim 256): the merged output is in the int8
// cache's rotated basis and is un-rotated per head before the gate.
template <bool ROT>
__global__ __launch_bounds__(256) void attn_reduce_kernel(const uint32_t* __restrict__ ctrl,
                                                          const float* __restrict__ attn_part,
                                                          const float* __restrict__ attn_gate,
                                                          uint16_t* __restrict__ attn_out, uint32_t M,
                                                          uint32_t q_heads, uint32_t HD, uint32_t tgt,
                                                          uint32_t gated, uint32_t kv_len) {
  __shared__ float fac[1024];
  __shared__ float s_sm;
  const uint32_t h = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
  if (m >= ctrl[CTRL_NACT]) return;
  const uint32_t pos = ctrl[CTRL_POS];
  uint32_t L = pos + m + 1;
  if (kv_len && L > kv_len) L = kv_len;
  uint32_t nb = (L - 1) / v2_ppw(L, tgt) + 1;
  if (nb > tgt) nb = tgt;
  const size_t PART = HD + 2;
  const float* base = attn_part + ((size_t)h * tgt * M + m) * PART;  // block b at + b * M * PART
  const size_t bstride = (size_t)M * PART;
  // the first 64 blocks' acc values do not depend on phase 1: their loads go out first
  // (a block past nb reloads block nb - 1 and is not added)
  float v64[64];
#pragma unroll
  for (uint32_t u = 0; u < 64; ++u) v64[u] = base[min(u, nb - 1) * bstride + 2 + d];
  // phase 1 (wave 0): the common max and the per-block factors
  if (d < 64) {
    float mx = -INFINITY;
    for (uint32_t b = d; b < nb; b += 64) mx = fmaxf(mx, base[b * bstride]);
#pragma unroll
    for (uint32_t o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    float sm = 0.f;
    for (uint32_t b = d; b < nb; b += 64) {
      const float f = expf(base[b * bstride] - mx);
      fac[b] = f;
      sm = __builtin_fmaf(base[b * bstride + 1], f, sm);
    }
#pragma unroll
    for (uint32_t o = 32; o > 0; o >>= 1) sm += __shfl_xor(sm, o, 64);
    if (d == 0) s_sm = sm;
  }
  __syncthreads();
  // added in ascending block order: the preloaded 64, then the rest 8 loads at a time
  float acc = 0.f;
#pragma unroll
  for (uint32_t u = 0; u < 64; ++u)
    if (u < nb) acc = __builtin_fmaf(v64[u], fac[u], acc);
  for (uint32_t b = 64; b < nb; b += 8) {
    float v[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) v[u] = base[min(b + u, nb - 1) * bstride + 2 + d];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u)
      if (b + u < nb) acc = __builtin_fmaf(v[u], fac[b + u], acc);
  }
  float o = acc / s_sm;
  if constexpr (ROT) {
    __shared__ float xch[256];
    float v1[1] = {kv8_flip(o, kv8_sign_neg(d))};
    fwht256<1>(v1, d, xch);
    o = v1[0] * 0.0625f;
  }
  uint16_t r;
  if (gated && attn_gate)
    r = f2h(h2f(f2h(o)) * sigmoid_f32(attn_gate[((size_t)m * q_heads + h) * HD + d]));
  else
    r = f2h(o);
  attn_out[(size_t)m * q_heads * HD + (size_t)h * HD + d] = r;
}

template <int HD, int KV8, bool DB>
int launch_decode_db(const AttnDecodeArgs& a, uint32_t gqa, dim3 grid, hipStream_t st) {
  switch (gqa) {
    case 1: attn_decode_kernel<HD, KV8, 1, DB><<<grid, 256, 0, st>>>(a); break;
    case 2: attn_decode_kernel<HD, KV8, 2, DB><<<grid, 256, 0, st>>>(a); break;
    case 4: attn_decode_kernel<HD, KV8, 4, DB><<<grid, 256, 0, st>>>(a); break;
    case 5: attn_decode_kernel<HD, KV8, 5, DB><<<grid, 256, 0, st>>>(a); break;
    case 6: attn_decode_kernel<HD, KV8, 6, DB><<<grid, 256, 0, st>>>(a); break;
    case 8: attn_decode_kernel<HD, KV8, 8, DB><<<grid, 256, 0, st>>>(a); break;
    default: return -1;
  }
  return 0;
}
// A cache of kv_len rows never gives a block more than one 64-position chunk when
// kv_len <= 64 tgt (ppw stays 64); otherwise the double-buffered kernel runs.
template <int HD, int KV8>
int launch_decode(const AttnDecodeArgs& a, uint32_t gqa, dim3 grid, hipStream_t st) {
  if (a.kv_len && a.kv_len <= 64u * a.tgt) return launch_decode_db<HD, KV8, false>(a, gqa, grid, st);
  return launch_decode_db<HD, KV8, true>(a, gqa, grid, st);
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
  if (pages && (!kv_len || mi_attn_ppw(kv_len, tgt) / page + 1 > kMaxBlockPages))
    return mi_fail(MI_ERR_SHAPE, "attn_decode: a paged cache needs kv_len, and at most 256 pages per block");
  if ((row_stride % 8) || (head_stride % 8))
    return mi_fail(MI_ERR_ARG, "attn_decode: KV strides must keep 8-element alignment");
  AttnDecodeArgs a{ctrl,  attn_q,       kv_k,           kv_v,   k_scale,         v_scale,
                   pages, attn_part,    row_stride,     head_stride, sc_row_stride, sc_head_stride,
                   page,  M,            shape->q_heads, shape->kv_heads, tgt,    kv_len,
                   shape->scale};
  dim3 grid(shape->kv_heads, tgt, M);
  hipStream_t st = (hipStream_t)stream;
  if (HD == 128) {
    if (kv_kind == 0) launch_decode<128, 0>(a, gqa, grid, st);
    else launch_decode<128, 1>(a, gqa, grid, st);
  } else {
    if (kv_kind == 0) launch_decode<256, 0>(a, gqa, grid, st);
    else launch_decode<256, 1>(a, gqa, grid, st);
  }
  return mi_hip((int)hipGetLastError(), "attn_decode");
}

int mi_attn_reduce(const uint32_t* ctrl, const float* attn_part, const float* attn_gate, uint16_t* attn_out,
                   uint32_t M, uint32_t tgt, uint32_t kv_len, const mi_attn_shape* shape, void* stream) {
  if (!ctrl || !attn_part || !attn_out || !shape || M == 0 || tgt == 0 || tgt > 1024)
    return mi_fail(MI_ERR_ARG, "attn_reduce: bad arguments (tgt <= 1024)");
  const uint32_t HD = shape->head_dim;
  if (HD != 64 && HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_reduce: head_dim 64/128/256");
  attn_reduce_kernel<false><<<dim3(shape->q_heads, M), HD, 0, (hipStream_t)stream>>>(
      ctrl, attn_part, attn_gate, attn_out, M, shape->q_heads, HD, tgt, shape->gated, kv_len);
  return mi_hip((int)hipGetLastError(), "attn_reduce");
}

int mi_attn_reduce_kv8(const uint32_t* ctrl, const float* attn_part, const float* attn_gate, uint16_t* attn_out,
                       uint32_t M, uint32_t tgt, uint32_t kv_len, const mi_attn_shape* shape, void* stream) {
  if (!ctrl || !attn_part || !attn_out || !shape || M == 0 || tgt == 0 || tgt > 1024)
    return mi_fail(MI_ERR_ARG, "attn_reduce_kv8: bad arguments (tgt <= 1024)");
  if (shape->head_dim != 256)
    return mi_fail(MI_ERR_SHAPE, "attn_reduce_kv8: the rotation is defined for head_dim 256 only");
  attn_reduce_kernel<true><<<dim3(shape->q_heads, M), 256, 0, (hipStream_t)stream>>>(
      ctrl, attn_part, attn_gate, attn_out, M, shape->q_heads, 256, tgt, shape->gated, kv_len);
  return mi_hip((int)hipGetLastError(), "attn_reduce_kv8");
}

}  // extern "C"
