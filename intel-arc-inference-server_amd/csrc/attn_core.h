// attn_core.h - the GQA decode attention block (attn_decode_v2, src/kernels/attn_v2.cl:172,
// and its int8 reader, src/kernels/kv8.cl:535) as a device function of the launch form
// (attn.hip).
#pragma once
#include "mi_common.h"
#include "gemv_core.h"

// groups in flight per wave for the int8 head_dim-128 reader
#ifndef MI_ATTN_PD8
#define MI_ATTN_PD8 3
#endif

namespace mi {

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
// Prefetch: a ring of PD groups' K and V registers per wave (PD = 3 for int8 rows of 128, 2 for
// fp16 rows of 128 or int8 rows of 256, 1 otherwise); a group's registers take the group 4 PD
// ahead as soon as it has been used.
// FP (fused prep, f16 cache): the kernel also does attn_prep's work (attn.cl:361-372) for the
// rows it needs: q of its GQA heads from the qkv partials (fold, q-norm, RoPE), and the K and V
// rows of the step's new positions that fall in its block (fold, k-norm, RoPE, f16), which it
// uses in place of the cache rows; the work-group whose row owns a new position (the last block
// of that row) writes that K/V row to the cache, block 0 writes the gate. Every value follows
// attn_prep_kernel's chain operation for operation (the same fold order, the same 256-lane
// norm tree, the same RoPE fma), so the partials, the cache rows and the gate are bitwise those
// of attn_prep followed by the plain decode.
template <int HD, int KV8, int GQA, bool FP>
__device__ __forceinline__ void attn_block(const AttnDecodeArgs& a, uint32_t j, uint32_t blk, uint32_t m) {
  constexpr uint32_t KK = HD / 32, NT = HD / 16;
  constexpr uint32_t EB = KV8 ? 1u : 2u, ROWB = HD * EB;  // bytes per row
  constexpr uint32_t VLD = ROWB / 64u;                     // 16-byte V loads per lane (4 lanes per row)
  constexpr uint32_t CW = 16u * EB;                        // bytes of one 16-dim column
  // groups in flight per wave: a ring of PD register buffers (VGPRs per group: K 2 KK (int8) or
  // 4 KK (f16), V 4 VLD, the two int8 scales)
  constexpr uint32_t GREG = KK * (KV8 ? 2u : 4u) + VLD * 4u;
  constexpr uint32_t PD = GREG <= 16u ? MI_ATTN_PD8 : (GREG <= 32u ? 2u : 1u);
  constexpr uint32_t SV = 16u * ROWB;                      // one wave's staged V group
  constexpr uint32_t RED = 4u * GQA * HD * 4u;             // the end merge's accumulators
  __shared__ __align__(16) unsigned char s_buf[(4u * SV > RED ? 4u * SV : RED)];
  __shared__ float st_m[4][16], st_l[4][16], st_f[4][16], st_hm[16], st_hs[16];
  __shared__ uint32_t s_grow[kMaxBlockGroups];
  __shared__ h8_t s_q[2][KK][64];  // q as the B operand, per lane: f16 high and low parts
  constexpr uint32_t FPQ = FP ? GQA * HD : 1u, FPN = FP ? 8u * HD : 1u, FPW = FP ? 4u * HD : 1u;
  __shared__ float s_q32[FPQ];                       // FP: the roped q of the GQA heads
  __shared__ __align__(16) uint16_t s_newk[FPN], s_newv[FPN];  // FP: new K/V rows, f16
  __shared__ float s_nrm[FPW];                       // FP: one wave's normed row (RoPE pairs)

  const uint32_t t = opaque_tid(), lane = t & 63u, wave = t >> 6;
  const uint32_t qi = lane & 15u, qq = lane >> 4;
  // q (plain form): wave 0's loads of the B operand go out before anything else, so waiting
  // for them later does not wait for the K/V loads issued after them (loads retire in order)
  constexpr bool QE = !FP;
  f4_t qv[QE ? 2u * KK : 1u];
  if constexpr (QE) {
    if (wave == 0 && qi < GQA) {
      const float* qp = a.attn_q + ((size_t)m * a.q_heads + j * GQA + qi) * HD + 8 * qq;
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk) {
        qv[2 * kk] = *as_global(reinterpret_cast<const f4_t*>(qp + 32 * kk));
        qv[2 * kk + 1] = *as_global(reinterpret_cast<const f4_t*>(qp + 32 * kk + 4));
      }
    }
  }
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
  // Every lane loads whatever the group's length: rows past it re-read the group's last row
  // (their scores are masked to -inf and their weights are 0), so no load sits under a branch
  // and the waits for one group's loads never wait for the later groups' loads.
  auto load_group = [&](uint32_t gi, uint32_t rb, Group& g) {
    const uint32_t p0 = p_begin + 16u * gi;
    const uint32_t glast = min(16u, p_end - p0) - 1u;
    const size_t row = (size_t)rb + min(qi, glast);
#pragma unroll
    for (uint32_t kk = 0; kk < KK; ++kk) {
      const size_t off = row * a.row_stride + hoff + 32 * kk + 8 * qq;
      if constexpr (KV8 == 0)
        g.k[kk].w = *as_global(reinterpret_cast<const u4_t*>(static_cast<const uint16_t*>(a.kv_k) + off));
      else
        g.k[kk].w = *as_global(reinterpret_cast<const u2_t*>(static_cast<const int8_t*>(a.kv_k) + off));
    }
    if constexpr (KV8 == 1) {
      g.ks = *as_global(a.k_scale + row * a.sc_row_stride + shoff);
      g.vs = *as_global(a.v_scale + row * a.sc_row_stride + shoff);
    }
    const unsigned char* vb = static_cast<const unsigned char*>(a.kv_v) +
                              (((size_t)rb + min(vrow, glast)) * a.row_stride + hoff) * EB + vpart * (ROWB / 4u);
#pragma unroll
    for (uint32_t i = 0; i < VLD; ++i) g.v[i] = *as_global(reinterpret_cast<const u4_t*>(vb + 16u * i));
  };


  // this wave's first group goes out before anything else: its row straight from the page
  // table, the later groups' rows staged in LDS below
  // (PF: its second group too, so both are in flight while q is staged)
  Group buf[PD];
  auto direct_row = [&](uint32_t g) -> uint32_t {
    const uint32_t p0 = p_begin + 16u * g;
    return __builtin_amdgcn_readfirstlane(a.pages ? a.pages[p0 / a.page] * a.page + p0 % a.page : p0);
  };
#pragma unroll
  for (uint32_t d = 0; d < PD; ++d)
    if (wave + 4u * d < ng) load_group(wave + 4u * d, direct_row(wave + 4u * d), buf[d]);
  // A paged cache: a page holds whole 16-position groups, so a group's rows are consecutive.
  // Each group's first cache row is looked up once, into LDS (the only divisions by the page
  // size), so no later K/V load waits on a page-table load.
  if (a.pages) {
    for (uint32_t i = t; i < ng; i += 256u) {
      const uint32_t p = p_begin + 16u * i;
      s_grow[i] = a.pages[p / a.page] * a.page + p % a.page;
    }
  }
  uint32_t pn0 = 0xFFFFFFFFu;  // FP: the block's first new position (none: past every position)
  if constexpr (FP) {
    // attn_prep's chain for one row of HD values, one wave: lane l holds elements l + 64 k
    constexpr uint32_t EPL = HD / 64u;
    const size_t pstep = (size_t)a.M * a.qkv_n;
    auto fold = [&](uint32_t r, size_t col) {  // sum_s partials in ascending s from +0
      const float* pp = a.partials + (size_t)r * a.qkv_n + col;
      float v = 0.0f;
      for (uint32_t s0 = 0; s0 < a.S; s0 += 16u) {
        float tv[16];
#pragma unroll
        for (uint32_t u = 0; u < 16; ++u) tv[u] = pp[min(s0 + u, a.S - 1u) * pstep];
#pragma unroll
        for (uint32_t u = 0; u < 16; ++u) v += s0 + u < a.S ? tv[u] : 0.f;
      }
      return v;
    };
    // the normed, roped row (fp32) of partial row r at column base, RoPE row rp
    auto prep_row = [&](uint32_t r, size_t base, const float* nw, uint32_t rp, float (&out)[EPL]) {
      const uint32_t half = a.rot_dim / 2u;
      const float* cs = a.rope + (size_t)rp * 2u * half;
      // the norm weights and the RoPE pairs go out with the partials' loads
      float wn[EPL], rc[EPL], rsn[EPL];
#pragma unroll
      for (uint32_t k = 0; k < EPL; ++k) {
        const uint32_t e = lane + 64u * k;
        wn[k] = nw ? nw[e] : 0.f;
        rc[k] = 1.f;
        rsn[k] = 0.f;
        if (e < a.rot_dim) {
          const uint32_t ii = e < half ? e : e - half;
          rc[k] = cs[ii];
          rsn[k] = cs[half + ii];
        }
      }
      float xf[EPL], nv[EPL];
#pragma unroll
      for (uint32_t k = 0; k < EPL; ++k) xf[k] = h2f(f2h(fold(r, base + lane + 64u * k)));
      if (nw) {
        // tree_hd's order: the LDS steps (v[i] + v[i + st], st >= 64) are this lane's own
        // elements, then the 64-lane shuffle tree; lane 0's total is broadcast
        float sq[EPL];
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) sq[k] = xf[k] * xf[k];
        float acc;
        if constexpr (EPL == 4) acc = (sq[0] + sq[2]) + (sq[1] + sq[3]);
        else if constexpr (EPL == 2) acc = sq[0] + sq[1];
        else acc = sq[0];
#pragma unroll
        for (int st = 32; st > 0; st >>= 1) acc += __shfl_down(acc, st, 64);
        const float tot = __shfl(acc, 0, 64);
        const float rstd = 1.0f / sqrtf(tot / (float)HD + a.eps);
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) nv[k] = h2f(f2h(xf[k] * rstd * wn[k]));
      } else {
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) nv[k] = xf[k];
      }
      float* nrm = s_nrm + wave * HD;
      wave_lds_sync();
#pragma unroll
      for (uint32_t k = 0; k < EPL; ++k) nrm[lane + 64u * k] = nv[k];
      wave_lds_sync();
#pragma unroll
      for (uint32_t k = 0; k < EPL; ++k) {
        const uint32_t e = lane + 64u * k;
        if (e < half) {
          const float tt = nrm[e + half] * rsn[k];
          out[k] = __builtin_fmaf(nv[k], rc[k], -tt);
        } else if (e < a.rot_dim) {
          const float tt = nrm[e - half] * rsn[k];
          out[k] = __builtin_fmaf(nv[k], rc[k], tt);
        } else {
          out[k] = nv[k];
        }
      }
    };
    // the step's new positions pos .. pos + m that fall in this block (row r = p - pos)
    const uint32_t first_new = max(pos, p_begin);
    const uint32_t n_new = p_end > first_new ? p_end - first_new : 0u;
    pn0 = first_new;
    const uint32_t QH = a.q_heads;
    for (uint32_t it = wave; it < GQA + n_new; it += 4u) {  // uniform per wave
      float out[EPL];
      if (it < GQA) {  // q head j GQA + it of row m
        const uint32_t h = j * GQA + it;
        const size_t base = a.gated ? (size_t)h * 2u * HD : (size_t)h * HD;
        prep_row(m, base, a.q_norm, pos + m, out);
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) s_q32[it * HD + lane + 64u * k] = out[k];
        if (a.gated && a.attn_gate && blk == 0) {
#pragma unroll
          for (uint32_t k = 0; k < EPL; ++k)
            a.attn_gate[((size_t)m * QH + h) * HD + lane + 64u * k] = h2f(f2h(fold(m, base + HD + lane + 64u * k)));
        }
      } else {  // the new K/V row of position first_new + (it - GQA), kv head j
        const uint32_t rl = it - GQA, r = first_new + rl - pos;
        prep_row(r, (size_t)a.k_off + (size_t)j * HD, a.k_norm, pos + r, out);
        uint16_t vk[EPL], vv[EPL];
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) {
          vk[k] = f2h(out[k]);
          vv[k] = f2h(fold(r, (size_t)a.v_off + (size_t)j * HD + lane + 64u * k));
          s_newk[rl * HD + lane + 64u * k] = vk[k];
          s_newv[rl * HD + lane + 64u * k] = vv[k];
        }
        if (r == m) {  // this row's own new position: the cache row is written here, once
          const uint32_t p = pos + r;
          const size_t row = a.pages ? (size_t)a.pages[p / a.page] * a.page + p % a.page : (size_t)p;
          uint16_t* kw = static_cast<uint16_t*>(const_cast<void*>(a.kv_k)) + row * a.row_stride + hoff;
          uint16_t* vw = static_cast<uint16_t*>(const_cast<void*>(a.kv_v)) + row * a.row_stride + hoff;
#pragma unroll
          for (uint32_t k = 0; k < EPL; ++k) {
            kw[lane + 64u * k] = vk[k];
            vw[lane + 64u * k] = vv[k];
          }
        }
      }
    }
    if (a.kv_len && pos + m >= a.kv_len && j == 0 && blk == 0 && t == 0)
      a.ctrl_w[CTRL_DEBUG] = 0xDEAD0002u;  // attn_prep's flag: the row's position is past the cache
    lds_barrier();
  }
  // q as the MFMA B operand, staged once by wave 0: column qi = head (zero past GQA),
  // k = 32 kk + 8 qq + e; the waves read it from LDS per group rather than holding it
  if (wave == 0) {
#pragma unroll
    for (uint32_t kk = 0; kk < KK; ++kk) {
      float v[8];
      if (qi < GQA) {
        if constexpr (FP) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = s_q32[qi * HD + 32 * kk + 8 * qq + e];
        } else {
          const f4_t q0 = qv[2 * kk], q1 = qv[2 * kk + 1];
          v[0] = q0.x; v[1] = q0.y; v[2] = q0.z; v[3] = q0.w;
          v[4] = q1.x; v[5] = q1.y; v[6] = q1.z; v[7] = q1.w;
        }
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
  lds_barrier();

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
  // the ring: group gi = gb + 4 ri sits in buf[ri]; once used, buf[ri] takes group gi + 4 PD
  for (uint32_t gb = wave; gb < ng; gb += 4u * PD) {
#pragma unroll
    for (uint32_t ri = 0; ri < PD; ++ri) {
      const uint32_t gi = gb + 4u * ri;
      if (gi >= ng) break;  // uniform
      Group& cur = buf[ri];
      const uint32_t glen = min(16u, p_end - (p_begin + 16u * gi));
      if constexpr (FP) {
        // the step's new positions take the rows computed above (the cache may not hold them yet)
        const uint32_t p0 = p_begin + 16u * gi;
        if (p0 + glen > pn0) {  // uniform
          if (qi < glen && p0 + qi >= pn0) {
            const uint16_t* nk = s_newk + (p0 + qi - pn0) * HD;
  #pragma unroll
            for (uint32_t kk = 0; kk < KK; ++kk) cur.k[kk].w = *reinterpret_cast<const u4_t*>(nk + 32 * kk + 8 * qq);
          }
          if (vrow < glen && p0 + vrow >= pn0) {
            const unsigned char* nv = reinterpret_cast<const unsigned char*>(s_newv + (p0 + vrow - pn0) * HD);
  #pragma unroll
            for (uint32_t i = 0; i < VLD; ++i) cur.v[i] = *reinterpret_cast<const u4_t*>(nv + vpart * (ROWB / 4u) + 16u * i);
          }
        }
      }
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
      if (gi + 4u * PD < ng) load_group(gi + 4u * PD, group_row(gi + 4u * PD), cur);
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
    *as_global(out + 2 + dd) = v;
    if (dd == 0) {
      out[0] = st_hm[g];
      out[1] = st_hs[g];
    }
  }
}


}  // namespace mi
