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

namespace mi {
namespace {


__device__ __forceinline__ uint32_t v2_ppw(uint32_t len, uint32_t tgt) {
  uint32_t p = (len + tgt - 1) / tgt;
  p = (p + 63u) & ~63u;
  return p < 64u ? 64u : p;
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
template <int KV8>
__device__ __forceinline__ void zero_chunk(KvChunk<KV8>& c) {
  if constexpr (KV8 == 0) c.w = u4_t{0u, 0u, 0u, 0u};
  else c.w = u2_t{0u, 0u};
}

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

// HD: head dim; KV8: int8 KV; GQA: q heads per kv head. Per-wave flash decoding: the block's
// positions are cut into 16-position groups and wave w takes groups w, w + 4, ..., keeping its
// own online softmax state (running max, sum, accumulator) per q head; the four waves' states
// are merged once, at the end, into the block's partial. No work-group barrier inside the loop.
// Per group, both products run on the matrix cores:
//   scores  S^T = K Q^T with v_mfma_f32_16x16x32_f16: A = the 16 K rows (lane l: position
//           l % 16, dims 8 (l / 16) + 32 kk; int8 widened exactly to f16 by a byte permute),
//           B = q split into an f16 high part and the f16 rounding of the remainder (two
//           MFMAs: the dot is fp32 accurate), padded to 16 heads. Lane l receives the scores of
//           positions 4 (l / 16) + r, r < 4, for head l % 16;
//   softmax per head over those 4 scores and the 4 lanes l % 16 + 16 k (two lane exchanges);
//           the weights w = exp(s - max) stay in the lanes that hold the scores, which is the
//           B operand layout of the next product;
//   P V     O^T = V^T W^T with v_mfma_f32_16x16x16_f16 per 16-dim tile: A = V^T (lane l: dim
//           l % 16, positions 4 (l / 16) + j) read from the group's V rows staged in LDS with a
//           swizzle that keeps the four row groups on distinct banks; B = the weights (times the
//           row's V scale for int8), split into f16 high and low parts like q. The int8 (or f16)
//           V values are exact in f16.
// Prefetch (PF): the next group's K and V registers are loaded before the current group is used.
template <int HD, int KV8, int GQA>
__global__ __launch_bounds__(256) void attn_decode_wave_kernel(AttnDecodeArgs a) {
  constexpr uint32_t KK = HD / 32, NT = HD / 16;
  constexpr uint32_t EB = KV8 ? 1u : 2u, ROWB = HD * EB;  // bytes per row
  constexpr uint32_t VLD = ROWB / 64u;                     // 16-byte V loads per lane (4 lanes per row)
  constexpr uint32_t CW = 16u * EB;                        // bytes of one 16-dim column
  constexpr bool PF = (KK * (KV8 ? 2u : 4u) + VLD * 4u) <= 32u;
  constexpr uint32_t SV = 16u * ROWB;                      // one wave's staged V group
  constexpr uint32_t RED = 4u * GQA * HD * 4u;             // the end merge's accumulators
  __shared__ __align__(16) unsigned char s_buf[(4u * SV > RED ? 4u * SV : RED)];
  __shared__ float st_m[4][16], st_l[4][16], st_f[4][16], st_hm[16], st_hs[16];
  __shared__ uint32_t s_grow[kMaxBlockGroups];
  __shared__ h8_t s_q[2][KK][64];  // q as the B operand, per lane: f16 high and low parts

  const uint32_t j = blockIdx.x, blk = blockIdx.y, m = blockIdx.z;
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
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
  const uint32_t ng = (p_end - p_begin + 15u) / 16u;

  const size_t hoff = (size_t)j * a.head_stride;
  const size_t shoff = (size_t)j * a.sc_head_stride;
  struct Group {
    KvChunk<KV8> k[KK];
    u4_t v[VLD];
    uint16_t ks, vs;
  };
  const uint32_t vrow = lane >> 2, vpart = lane & 3u;  // the V row and quarter this lane loads
  // group gi whose first cache row is rb (uniform)
  auto load_group = [&](uint32_t gi, uint32_t rb, Group& g) {
    const uint32_t p0 = p_begin + 16u * gi;
    const uint32_t glen = min(16u, p_end - p0);
    if (qi < glen) {
      const size_t row = (size_t)rb + qi;
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk) {
        const size_t off = row * a.row_stride + hoff + 32 * kk + 8 * qq;
        if constexpr (KV8 == 0) g.k[kk].w = *reinterpret_cast<const u4_t*>(static_cast<const uint16_t*>(a.kv_k) + off);
        else g.k[kk].w = *reinterpret_cast<const u2_t*>(static_cast<const int8_t*>(a.kv_k) + off);
      }
      if constexpr (KV8 == 1) {
        g.ks = a.k_scale[row * a.sc_row_stride + shoff];
        g.vs = a.v_scale[row * a.sc_row_stride + shoff];
      }
    } else {
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk) zero_chunk<KV8>(g.k[kk]);
      g.ks = 0;
      g.vs = 0;
    }
    if (vrow < glen) {
      const unsigned char* vb = static_cast<const unsigned char*>(a.kv_v) +
                                (((size_t)rb + vrow) * a.row_stride + hoff) * EB + vpart * (ROWB / 4u);
#pragma unroll
      for (uint32_t i = 0; i < VLD; ++i) g.v[i] = *reinterpret_cast<const u4_t*>(vb + 16u * i);
    } else {
#pragma unroll
      for (uint32_t i = 0; i < VLD; ++i) g.v[i] = u4_t{0u, 0u, 0u, 0u};
    }
  };


  // this wave's first group goes out before anything else: its row straight from the page
  // table, the later groups' rows staged in LDS below
  Group cur, nxt;
  uint32_t gi = wave;
  if (gi < ng) {
    const uint32_t p0 = p_begin + 16u * gi;
    const uint32_t rb = a.pages ? a.pages[p0 / a.page] * a.page + p0 % a.page : p0;
    load_group(gi, __builtin_amdgcn_readfirstlane(rb), cur);
  }
  // A paged cache: a page holds whole 16-position groups, so a group's rows are consecutive.
  // Each group's first cache row is looked up once, into LDS (the only divisions by the page
  // size), so no later K/V load waits on a page-table load.
  if (a.pages) {
    for (uint32_t i = t; i < ng; i += 256u) {
      const uint32_t p = p_begin + 16u * i;
      s_grow[i] = a.pages[p / a.page] * a.page + p % a.page;
    }
  }
  // q as the MFMA B operand, staged once by wave 0: column qi = head (zero past GQA),
  // k = 32 kk + 8 qq + e; the waves read it from LDS per group rather than holding it
  if (wave == 0) {
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
      h8_t hi, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const half_t h = (half_t)v[e];
        hi[e] = h;
        lo[e] = (half_t)(v[e] - (float)h);
      }
      s_q[0][kk][lane] = hi;
      s_q[1][kk][lane] = lo;
    }
  }
  __syncthreads();

  // this wave's running state for head qi; acc[tt][r] = O^T[16 tt + 4 qq + r][qi]
  float m_run = -INFINITY, l_run = 0.f;
  f4_t acc[NT];
#pragma unroll
  for (uint32_t tt = 0; tt < NT; ++tt) acc[tt] = f4_t{0.f, 0.f, 0.f, 0.f};
  unsigned char* sv = s_buf + wave * SV;
  // the swizzled byte offset of (row r, 16-dim column c): the four row groups 4 k + j that one
  // A-operand read touches land on distinct banks
  auto sv_off = [](uint32_t r, uint32_t c) -> uint32_t { return r * ROWB + ((c ^ ((r >> 2) & 3u)) * CW); };

  auto group_row = [&](uint32_t g) -> uint32_t {
    return __builtin_amdgcn_readfirstlane(a.pages ? s_grow[g] : p_begin + 16u * g);
  };
  for (; gi < ng; gi += 4u) {
    if constexpr (PF) {
      if (gi + 4u < ng) load_group(gi + 4u, group_row(gi + 4u), nxt);
    }
    const uint32_t glen = min(16u, p_end - (p_begin + 16u * gi));
    // stage this group's V rows (the previous group's reads of this wave's area are done:
    // one wave's LDS operations complete in order, and the fence keeps the compiler's too)
    wave_lds_sync();
#pragma unroll
    for (uint32_t i = 0; i < VLD; ++i) {
      const uint32_t byte = vpart * (ROWB / 4u) + 16u * i;  // within the row
      *reinterpret_cast<u4_t*>(sv + sv_off(vrow, byte / CW) + byte % CW) = cur.v[i];
    }
    wave_lds_sync();
    // scores S^T[position 4 qq + r][head qi]
    f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t kk = 0; kk < KK; ++kk) {
      const h8_t kh = chunk_h8<KV8>(cur.k[kk]);
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, s_q[0][kk][lane], d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, s_q[1][kk][lane], d, 0, 0, 0);
    }
    float sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
      float rs = a.scale;
      if constexpr (KV8 == 1) rs = a.scale * h2f((uint16_t)__shfl((int)cur.ks, (int)(4u * qq + r), 64));
      sc[r] = 4u * qq + r < glen ? d[r] * rs : -INFINITY;
      mx = fmaxf(mx, sc[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = expf(m_run - m_new);  // 0 on the first group (m_run = -inf)
    float w[4];
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) w[r] = expf(sc[r] - m_new);
    l_run = __builtin_fmaf(l_run, alpha, (w[0] + w[1]) + (w[2] + w[3]));
    m_run = m_new;
    if (__ballot(alpha != 1.0f)) {  // a head's max moved (a factor of 1 leaves acc unchanged)
#pragma unroll
      for (uint32_t tt = 0; tt < NT; ++tt) acc[tt] *= alpha;
    }
    // B operand: the weights (int8: times the row's V scale), f16 high and low parts
    h4_t bh, bl;
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
      float wv = w[r];
      if constexpr (KV8 == 1) wv *= h2f((uint16_t)__shfl((int)cur.vs, (int)(4u * qq + r), 64));
      const half_t h = (half_t)wv;
      bh[r] = h;
      bl[r] = (half_t)(wv - (float)h);
    }
    // P V per 16-dim tile: A[dim qi][position 4 qq + jj] from the staged rows
#pragma unroll
    for (uint32_t tt = 0; tt < NT; ++tt) {
      h4_t av;
      if constexpr (KV8 == 1) {
        uint32_t b[4];
#pragma unroll
        for (uint32_t jj = 0; jj < 4; ++jj) b[jj] = sv[sv_off(4u * qq + jj, tt) + qi];
        const h2_t bias = {(half_t)1152.0f, (half_t)1152.0f};
        const h2_t lo = as_h2((b[0] | (b[1] << 16)) ^ 0x64806480u) - bias;
        const h2_t hi = as_h2((b[2] | (b[3] << 16)) ^ 0x64806480u) - bias;
        av = h4_t{lo[0], lo[1], hi[0], hi[1]};
      } else {
#pragma unroll
        for (uint32_t jj = 0; jj < 4; ++jj)
          av[jj] = *reinterpret_cast<const half_t*>(sv + sv_off(4u * qq + jj, tt) + 2u * qi);
      }
      acc[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bh, acc[tt], 0, 0, 0);
      acc[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bl, acc[tt], 0, 0, 0);
    }
    if constexpr (PF) {
      cur = nxt;
    } else {
      if (gi + 4u < ng) load_group(gi + 4u, group_row(gi + 4u), cur);
    }
  }
  // merge the four waves: M = max m_w, f_w = exp(m_w - M), sum and acc weighted by f_w in
  // wave order
  float l = l_run + __shfl_xor(l_run, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  if (qq == 0) {
    st_m[wave][qi] = m_run;
    st_l[wave][qi] = l;
  }
  lds_barrier();  // every wave has finished with its staging area, which the merge reuses
  float* red = reinterpret_cast<float*>(s_buf);  // [4][GQA][HD]
  if (qi < GQA) {
#pragma unroll
    for (uint32_t tt = 0; tt < NT; ++tt)
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) red[(wave * GQA + qi) * HD + 16u * tt + 4u * qq + r] = acc[tt][r];
  }
  if (t < GQA) {  // per head, once: the common max, the waves' factors, the weighted sum
    float M = st_m[0][t];
#pragma unroll
    for (uint32_t w2 = 1; w2 < 4; ++w2) M = fmaxf(M, st_m[w2][t]);
    float sm = 0.f;
#pragma unroll
    for (uint32_t w2 = 0; w2 < 4; ++w2) {
      const float f = expf(st_m[w2][t] - M);  // a wave without positions: exp(-inf) = 0
      sm = __builtin_fmaf(st_l[w2][t], f, sm);
      st_f[w2][t] = f;
    }
    st_hm[t] = M;
    st_hs[t] = sm;
  }
  lds_barrier();
  for (uint32_t idx = t; idx < GQA * HD; idx += 256u) {
    const uint32_t g = idx / HD, dd = idx % HD;
    float v = 0.f;
#pragma unroll
    for (uint32_t w2 = 0; w2 < 4; ++w2) v = __builtin_fmaf(red[(w2 * GQA + g) * HD + dd], st_f[w2][g], v);
    float* out = a.attn_part + (((size_t)(j * GQA + g) * a.tgt + blk) * a.M + m) * (HD + 2);
    out[2 + dd] = v;
    if (dd == 0) {
      out[0] = st_hm[g];
      out[1] = st_hs[g];
    }
  }
}

// attn_v2.cl:383-428's merge of a row's nb block partials, as one common max M = max mx_b,
// factors f_b = exp(mx_b - M), sum = sum_b sm_b f_b and acc = sum_b acc_b f_b added in
// ascending b: mathematically the reference's sequential rescaling merge, the roundings
// differing at the last place. grid (q_heads, M), HD threads, one dim each. The first 64
// blocks' values do not depend on the factors and are loaded before them, together with
// wave 0's (mx, sm) loads, so a merge of up to 64 blocks is one memory round trip; further
// blocks follow 64 at a time.
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
  if (m >= ctrl[CTRL_NACT]) return;  // uniform
  const uint32_t pos = ctrl[CTRL_POS];
  uint32_t L = pos + m + 1;
  if (kv_len && L > kv_len) L = kv_len;
  uint32_t nb = (L - 1) / v2_ppw(L, tgt) + 1;
  if (nb > tgt) nb = tgt;
  const size_t PART = HD + 2;
  const float* base = attn_part + ((size_t)h * tgt * M + m) * PART;  // block b at + b * M * PART
  const size_t bstride = (size_t)M * PART;
  // (a load past nb re-reads block nb - 1 and is not added)
  constexpr uint32_t PRE = 64, BAT = 64;
  // loads go out in runs of 16 behind a uniform bound, so a short merge issues few of them
  float v[PRE];
#pragma unroll
  for (uint32_t c = 0; c < PRE; c += 16)
    if (c < nb) {
#pragma unroll
      for (uint32_t u = c; u < c + 16; ++u) v[u] = base[min(u, nb - 1) * bstride + 2 + d];
    }
  // wave 0: the common max and the per-block factors
  if (d < 64) {
    float mx = -INFINITY;
    for (uint32_t b = d; b < nb; b += 64) mx = fmaxf(mx, base[b * bstride]);
    mx = wave_max(mx);
    float sm = 0.f;
    for (uint32_t b = d; b < nb; b += 64) {
      const float f = expf(base[b * bstride] - mx);
      fac[b] = f;
      sm = __builtin_fmaf(base[b * bstride + 1], f, sm);
    }
    sm = wave_sum(sm);
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
  float o = acc / s_sm;
  if constexpr (ROT) {
    __shared__ float xch[256];
    float v1[1] = {kv8_flip(o, kv8_sign_neg(d))};
    fwht256<1>(v1, d, xch);  // HD = 256: every thread of the work-group is here
    o = v1[0] * 0.0625f;
  }
  uint16_t r;
  if (gated && attn_gate)
    r = f2h(h2f(f2h(o)) * sigmoid_f32(attn_gate[((size_t)m * q_heads + h) * HD + d]));
  else
    r = f2h(o);
  attn_out[(size_t)m * q_heads * HD + (size_t)h * HD + d] = r;
}

template <int HD, int KV8>
int launch_decode(const AttnDecodeArgs& a, uint32_t gqa, dim3 grid, hipStream_t st) {
  switch (gqa) {
    case 1: attn_decode_wave_kernel<HD, KV8, 1><<<grid, 256, 0, st>>>(a); break;
    case 2: attn_decode_wave_kernel<HD, KV8, 2><<<grid, 256, 0, st>>>(a); break;
    case 4: attn_decode_wave_kernel<HD, KV8, 4><<<grid, 256, 0, st>>>(a); break;
    case 5: attn_decode_wave_kernel<HD, KV8, 5><<<grid, 256, 0, st>>>(a); break;
    case 6: attn_decode_wave_kernel<HD, KV8, 6><<<grid, 256, 0, st>>>(a); break;
    case 8: attn_decode_wave_kernel<HD, KV8, 8><<<grid, 256, 0, st>>>(a); break;
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
