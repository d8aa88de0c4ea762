// attn_dma.h - the GQA decode attention block of the plain launch (attn_decode_v2,
// src/kernels/attn_v2.cl:172, and its int8 reader, src/kernels/kv8.cl:535) with the K/V rows
// streamed into LDS by gfx950's direct global-to-LDS loads.
//
// Per work-group (kv head j, block blk, rows r_lo .. r_hi - 1) the block's 16-position groups
// are dealt to the four waves round-robin; each wave keeps its own online softmax and the
// waves merge once at the end into each (row, head)'s partial {max, sum, acc[HD]}.
//
// Rows. The matrix products' columns are (row, q head) pairs, 16 per tile: a plain launch gives
// a work-group RPW = 16 CT / GQA consecutive rows of the list that share the block size (column
// c = 16 ct + qi = GQA rr + g is row r_lo + rr, head j GQA + g), so the block's K/V rows are
// read once for all of them; the CT tiles share every LDS read of K and V^T. Row r sees
// positions < pos + r + 1: its scores past that are -inf and a group that holds none of its
// positions leaves its state untouched (alpha 1, weights 0), so each column's values are,
// operation for operation, those of a one-row work-group for its row.
//
// Loads. A wave owns a ring of NB group slots in LDS. A group's 16 K rows and 16 V rows go
// into a slot with global_load_lds_dwordx4: one instruction moves 1 KB, lane L writing LDS
// bytes 16 L .. 16 L + 15 of it, so the wave asks HBM for whole rows (a group of a
// head-major cache is one contiguous run) and no register holds loaded data. Which 16-byte
// chunk lane L fetches is chosen so that LDS holds row r's chunk c at chunk c ^ f(r)
// (f(r) = (r ^ (r >> 3)) mod chunks-per-row): the score operand reads (16 rows, one column
// each) then fall on distinct banks. Rows past the group's end re-read its last row (their
// scores are -inf, their weights 0). The int8 reader's row scales (fp16 [row][kv head]) come
// with one global_load_lds_dword per group: lane r < 16 the aligned word that holds row r's
// K scale, lane 16 + r its V scale. A wave waits for a group with s_waitcnt vmcnt(n), n the
// loads it issued after that group; the loads are issued from inline assembly, which the
// compiler's own wait insertion does not see, so no load of its own is left outstanding
// across the loop and every wait inside the loop is this code's.
// Products, per group, on the matrix cores:
//   scores  S^T = K Q^T (v_mfma_f32_16x16x32_f16): A = 16 K rows read from LDS (lane l: row
//           l % 16, dims 8 (l / 16) + 32 kk; int8 widened exactly to f16), B = q in f16 high
//           and low parts;
//   softmax per head over the 16 positions, online across the wave's groups (fp32);
//   P V     O^T = V^T W^T (v_mfma_f32_16x16x16_f16) per 16-dim tile: A = V^T read from LDS
//           with gfx950's transposing reads - ds_read_b64_tr_b16 gives lane (i, g) dim i of
//           positions 4 g .. 4 g + 3 (f16); ds_read_b64_tr_b8 gives the same for two tiles at
//           once (int8, widened exactly to f16) - and B = the weights (int8: times the row's V
//           scale) in f16 high and low parts.
// Each wave's online softmax takes its groups in ascending order, NG groups per step, and the
// waves merge in wave order; the results are checked against attn_decode_v2's restatement and
// fp64 attention.
#pragma once
#include "attn_core.h"

namespace mi {


template <int HD, int KV8>
struct AttnDmaCfg {
  static constexpr uint32_t EB = KV8 ? 1u : 2u;
  static constexpr uint32_t ROWB = HD * EB;         // bytes per row
  static constexpr uint32_t CPR = ROWB / 16u;       // 16-byte chunks per row
  static constexpr uint32_t GB = 16u * ROWB;        // bytes of one group's K (or V) rows
  static constexpr uint32_t NI = GB / 1024u;        // 1 KB loads per group and tensor
  static constexpr uint32_t SCB = KV8 ? 256u : 0u;  // the scales' area of a slot
  static constexpr uint32_t SLOT = 2u * GB + SCB;
#ifndef MI_ATTN_NB_SMALL
#define MI_ATTN_NB_SMALL 4
#endif
  static constexpr uint32_t NB = SLOT <= 5000u ? MI_ATTN_NB_SMALL : 2u;  // slots per wave
  static constexpr uint32_t DG = 2u * NI + (KV8 ? 1u : 0u);  // loads per group
  static constexpr uint32_t RING = 4u * NB * SLOT;
};

// The direct loads set M0 (their LDS address) themselves; gfx950's LDS instructions do not read
// M0 and the compiler keeps nothing of its own there in these kernels (it would not see the
// write: M0 is a reserved register to inline assembly).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)p;
}

// 16 bytes per lane from base + voff into LDS [lds, lds + 1024), lane L at lds + 16 L (the
// caller has waited for this wave's LDS reads of that area: lds_reads_done)
__device__ __forceinline__ void dma16(uint32_t lds, const void* base, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
               :: "s"(lds), "v"(voff), "s"(base) : "memory");
}
__device__ __forceinline__ void lds_reads_done() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// 4 bytes per lane from the 64-bit address p into LDS, lane L at lds + 4 L
__device__ __forceinline__ void dma4(uint32_t lds, const void* p) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
               :: "s"(lds), "v"(p) : "memory");
}
// waits until at most N of this wave's vector memory loads are outstanding
template <uint32_t N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N < 64, "vmcnt");
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

template <uint32_t NB, uint32_t DG>
__device__ __forceinline__ void wait_group(uint32_t after) {  // after: groups issued after it
  if (after == 0) wait_vm<0>();
  else if (NB > 1 && after == 1) wait_vm<(NB > 1 ? DG : 0)>();
  else if (NB > 2 && after == 2) wait_vm<(NB > 2 ? 2 * DG : 0)>();
  else wait_vm<(NB > 3 ? 3 * DG : 0)>();
}

template <int HD, int KV8, int GQA, bool FP, int CT>
__device__ __forceinline__ void attn_block_dma(const AttnDecodeArgs& a, uint32_t j, uint32_t blk, uint32_t zg) {
  static_assert(!FP || KV8 == 0, "the fused prep writes the f16 cache");
  using C = AttnDmaCfg<HD, KV8>;
  constexpr uint32_t KK = HD / 32, NT = HD / 16;
  constexpr uint32_t ROWB = C::ROWB, CPR = C::CPR, GB = C::GB, SLOT = C::SLOT;
  static_assert(!FP || CT == 1, "the fused prep takes one row");
  constexpr uint32_t RPW = attn_rows_per_wg(GQA, FP, CT), NC = RPW * GQA;  // rows, live columns
  constexpr uint32_t RED = 4u * 16u * HD * 4u;  // the end merge's accumulators (one tile at a time)
  // groups per softmax step: two for int8 rows of 128 (two independent chains of products), else
  // one (f16 rows of 128 measured faster with one, the ring prefetching the next group); the same
  // for every CT, since the step's rounding depends on it
  constexpr uint32_t NG = HD == 128 && KV8 ? 2u : 1u;
  // slots per wave: several tiles take the fewest (a multiple of NG) that hold the merge, which
  // leaves LDS for the tiles' q
  constexpr uint32_t NBMIN = (RED + 4u * SLOT - 1u) / (4u * SLOT);
  constexpr uint32_t NB = CT == 1 ? C::NB : (NBMIN + NG - 1u) / NG * NG;
  constexpr uint32_t RING = 4u * NB * SLOT;
  static_assert(RING >= RED, "merge area");
  __shared__ __align__(16) unsigned char s_ring[RING];
  __shared__ float st_m[4][16], st_l[4][16], st_f[4][16], st_hm[16], st_hs[16];
  __shared__ uint32_t s_grow[kMaxBlockGroups];
  __shared__ h8_t s_q[CT][2][KK][64];
  // FP: the new K/V rows (f16), the roped q of the GQA heads and the waves' normed rows. At
  // rows of 256 the last two live in the ring (LDS is short), which the fused form then starts
  // to load only after its prologue; at rows of 128 they have arrays of their own and the ring's
  // first groups go out first, as in the plain form.
  constexpr uint32_t FPN = FP ? 8u * HD : 1u;
  __shared__ __align__(16) uint16_t s_newk[FPN], s_newv[FPN];
  constexpr bool kEarly = !FP || HD == 128;
  constexpr uint32_t FPQ = FP && kEarly ? GQA * HD + 4u * HD : 1u;
  __shared__ float s_fpq[FPQ];
  static_assert(kEarly || RING >= (GQA * HD + 4u * HD) * 4u, "prologue area");
  float* const s_q32 = kEarly ? s_fpq : reinterpret_cast<float*>(s_ring);
  float* const s_nrm = s_q32 + GQA * HD;

  const uint32_t t = opaque_tid(), lane = t & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const uint32_t qi = lane & 15u, qq = lane >> 4;
  const uint32_t n_act = min(a.ctrl[CTRL_NACT], a.M);
  const uint32_t pos = a.ctrl[CTRL_POS];
  auto row_len = [&](uint32_t r) {  // the keys row r sees
    const uint32_t len = pos + r + 1u;
    return a.kv_len && len > a.kv_len ? a.kv_len : len;
  };
  // this work-group's rows [r_lo, r_hi): the list's rows split where the block size changes
  // (row b on; the size is non-decreasing in the row and, rounded to 64 positions of
  // ceil(len / tgt), changes at most once over 64 consecutive rows), then RPW at a time
  uint32_t r_lo, r_hi;
  if constexpr (RPW == 1) {
    r_lo = zg;
    r_hi = zg + 1u;
    if (zg >= n_act) return;
  } else {
    const uint32_t s0 = v2_ppw(row_len(0), a.tgt);
    uint32_t b = n_act;
    for (uint32_t r = 1; r < n_act; ++r)
      if (v2_ppw(row_len(r), a.tgt) != s0) {
        b = r;
        break;
      }
    const uint32_t za = (b + RPW - 1u) / RPW;
    r_lo = zg < za ? zg * RPW : b + (zg - za) * RPW;
    r_hi = min(r_lo + RPW, zg < za ? b : n_act);
    if (r_lo >= r_hi) return;
  }
  const uint32_t m = r_lo;  // the fused prep's row (RPW = 1)
  const uint32_t L = row_len(r_hi - 1u);
  const uint32_t s = v2_ppw(L, a.tgt);
  uint32_t nb = (L - 1) / s + 1;
  if (nb > a.tgt) nb = a.tgt;
  if (blk >= nb) return;
  const uint32_t p_begin = blk * s, p_end = min(p_begin + s, L);
  // this lane's column 16 ct + qi of each tile: its row, and the row's end in the block
  // (p_begin: no column, or the row ends before the block)
  uint32_t crow[CT], pe_col[CT];
#pragma unroll
  for (uint32_t ct = 0; ct < CT; ++ct) {
    const uint32_t c = 16u * ct + qi;
    crow[ct] = r_lo + c / GQA;
    pe_col[ct] = c < NC && crow[ct] < r_hi ? max(min(p_begin + s, row_len(crow[ct])), p_begin) : p_begin;
  }
  const uint32_t ng = (p_end - p_begin + 15u) / 16u;
  const uint32_t ngw = wave < ng ? (ng - wave + 3u) / 4u : 0u;  // this wave's groups

  auto group_row = [&](uint32_t g) -> uint32_t {  // a later group's first cache row
    return __builtin_amdgcn_readfirstlane(a.pages ? s_grow[g] : p_begin + 16u * g);
  };
  const size_t hb = (size_t)j * a.head_stride * C::EB;
  const unsigned char* kbase = static_cast<const unsigned char*>(a.kv_k) + hb;
  const unsigned char* vbase = static_cast<const unsigned char*>(a.kv_v) + hb;
  const size_t rsb = a.row_stride * C::EB;  // bytes between rows
  unsigned char* ring = s_ring + wave * NB * SLOT;
  const uint32_t ring_lds = lds_addr(ring);
  auto swz = [](uint32_t r) -> uint32_t { return (r ^ (r >> 3)) & (CPR - 1u); };

  // issue this wave's group number tw (gi = wave + 4 tw, first cache row rb) into slot tw % NB
  auto issue = [&](uint32_t tw, uint32_t rb) {
    const uint32_t gi = wave + 4u * tw;
    const uint32_t glast = min(16u, p_end - (p_begin + 16u * gi)) - 1u;
    const uint32_t slot = ring_lds + (tw % NB) * SLOT;
    // the group's first row as a (uniform) 64-bit base; the lanes' offsets stay below 16 rows
    const unsigned char* kg = kbase + (size_t)rb * rsb;
    const unsigned char* vg = vbase + (size_t)rb * rsb;
    lds_reads_done();
#pragma unroll
    for (uint32_t i = 0; i < C::NI; ++i) {
      const uint32_t sidx = 64u * i + lane, r = sidx / CPR, c = (sidx % CPR) ^ swz(sidx / CPR);
      const uint32_t voff = min(r, glast) * (uint32_t)rsb + 16u * c;
      dma16(slot + 1024u * i, kg, voff);
      dma16(slot + GB + 1024u * i, vg, voff);
    }
    if constexpr (KV8 == 1) {
      const uint32_t r = min(lane & 15u, glast);
      const uint16_t* sb = (lane & 16u) ? a.v_scale : a.k_scale;
      const size_t e = (size_t)(rb + r) * a.sc_row_stride + (size_t)j * a.sc_head_stride;
      const uintptr_t ad = reinterpret_cast<uintptr_t>(sb + e) & ~(uintptr_t)3;
      dma4(slot + 2u * GB, reinterpret_cast<const void*>(ad));
    }
  };
  // The first NB groups, their rows straight from the page table (all its loads first, one wait
  // for them). The plain form sends them before anything else: the compiler's own loads below
  // (q, the page table) are issued after them, so its waits for those also wait for these -
  // all before the loop, whose waits are this code's alone. The fused form sends them after its
  // prologue, whose q and normed rows use the ring.
  auto issue_first = [&]() {
    const uint32_t npre = min(ngw, NB);
    if (npre) {
      // all page-table loads first (unconditional, a missing group re-reading the last), then
      // one wait for them
      uint32_t p0s[NB], pg[NB];
  #pragma unroll
      for (uint32_t tw = 0; tw < NB; ++tw) {
        p0s[tw] = p_begin + 16u * (wave + 4u * min(tw, npre - 1u));
        if (a.pages) pg[tw] = a.pages[p0s[tw] / a.page];
      }
  #pragma unroll
      for (uint32_t tw = 0; tw < NB; ++tw) {
        const uint32_t rb = __builtin_amdgcn_readfirstlane(a.pages ? pg[tw] * a.page + p0s[tw] % a.page : p0s[tw]);
        if (tw < npre) issue(tw, rb);
      }
    }
  };
  if constexpr (kEarly) issue_first();
  // q of the GQA heads (plain form: wave 0 loads it)
  f4_t qv[CT][FP ? 1u : 2u * KK];
  if constexpr (!FP) {
#pragma unroll
    for (uint32_t ct = 0; ct < CT; ++ct)
      if (wave == 0 && pe_col[ct] > p_begin) {
        const float* qp = a.attn_q + ((size_t)crow[ct] * a.q_heads + j * GQA + (16u * ct + qi) % GQA) * HD + 8 * qq;
#pragma unroll
        for (uint32_t kk = 0; kk < KK; ++kk) {
          qv[ct][2 * kk] = *as_global(reinterpret_cast<const f4_t*>(qp + 32 * kk));
          qv[ct][2 * kk + 1] = *as_global(reinterpret_cast<const f4_t*>(qp + 32 * kk + 4));
        }
      }
  }
  // the later groups' first cache rows (a page holds whole groups), staged in LDS
  if (a.pages) {
    for (uint32_t i = t; i < ng; i += 256u) {
      const uint32_t p = p_begin + 16u * i;
      s_grow[i] = a.pages[p / a.page] * a.page + p % a.page;
    }
  }
  uint32_t pn0 = 0xFFFFFFFFu;  // FP: the block's first new position (none: past every position)
  if constexpr (FP) {
    // attn_prep's work (attn.cl:361-372) for the rows this work-group needs: q of its GQA heads
    // from the qkv partials (fold in ascending slice order, q-norm, RoPE) and the K and V rows
    // of the step's new positions in its block (fold, k-norm, RoPE, f16), each operation as
    // attn_prep_kernel does it, so the partials, cache rows and gate are bitwise attn_prep's
    // followed by the plain decode. Lane l of a wave holds elements l + 64 k of a row.
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
    const size_t hoff = (size_t)j * a.head_stride;
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
  // q as the MFMA B operand (f16 high and low parts), staged by wave 0
  if (wave == 0) {
#pragma unroll
    for (uint32_t ct = 0; ct < CT; ++ct)
#pragma unroll
    for (uint32_t kk = 0; kk < KK; ++kk) {
      float v[8];
      if (pe_col[ct] > p_begin) {
        if constexpr (FP) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = s_q32[qi * HD + 32 * kk + 8 * qq + e];
        } else {
          const f4_t q0 = qv[ct][2 * kk], q1 = qv[ct][2 * kk + 1];
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
      s_q[ct][0][kk][lane] = hi;
      s_q[ct][1][kk][lane] = lo;
    }
  }
  wait_vm<0>();   // (the compiler's waits above have seen to this already)
  lds_barrier();  // s_grow, s_q
  if constexpr (!kEarly) issue_first();

  // the running state in log2 units: scores are scaled by log2(e) so every exponential is one
  // v_exp_f32 (exp2); the partial's max goes out in natural units
  constexpr float kLog2e = 1.4426950408889634f;
  const float qscale = a.scale * kLog2e;
  float m_run[CT], l_run[CT];
  f4_t acc[CT][NT];
#pragma unroll
  for (uint32_t ct = 0; ct < CT; ++ct) {
    m_run[ct] = -INFINITY;
    l_run[ct] = 0.f;
#pragma unroll
    for (uint32_t tt = 0; tt < NT; ++tt) acc[ct][tt] = f4_t{0.f, 0.f, 0.f, 0.f};
  }
  // the scales' halves: an element's word half is bit 1 of its address
  const uint32_t kpar0 = (uint32_t)(((uintptr_t)a.k_scale >> 1) + (size_t)j * a.sc_head_stride);
  const uint32_t vpar0 = (uint32_t)(((uintptr_t)a.v_scale >> 1) + (size_t)j * a.sc_head_stride);
  // the max over the four lanes l % 16 + 16 k that hold one head's scores: v_permlane16_swap
  // and v_permlane32_swap of x with a copy of itself leave rows (0, 0, 2, 2) / (1, 1, 3, 3) and
  // halves (lo, lo) / (hi, hi) in the two registers (VALU, no LDS round trip). Written as
  // assembly: the compiler's builtin for these swaps dropped the second result here.
  auto head_max = [](float x) {
    float a0 = x, a1 = x;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a0), "+v"(a1));
    float b0 = fmaxf(a0, a1), b1 = b0;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(b0), "+v"(b1));
    return fmaxf(b0, b1);
  };
  static_assert(NB % NG == 0, "ring");
  typedef int v2i_t __attribute__((ext_vector_type(2)));
  typedef short v4s_t __attribute__((ext_vector_type(4)));
  constexpr uint32_t NTR = KV8 ? NT / 2 : NT;  // transposing reads per group

  for (uint32_t tw = 0; tw < ngw; tw += NG) {
    const bool has1 = NG == 2 && tw + 1 < ngw;
    const uint32_t last = has1 ? tw + 1 : tw;
    wait_group<NB, C::DG>(min(ngw, tw + NB) - last - 1u);
    uint32_t glen[NG], slot[NG], p0g[NG];
#pragma unroll
    for (uint32_t u = 0; u < NG; ++u) {
      const uint32_t tg = u && has1 ? tw + 1 : tw;  // a missing second group reads the first's slot
      slot[u] = ring_lds + (tg % NB) * SLOT;
      p0g[u] = p_begin + 16u * (wave + 4u * tg);
      glen[u] = u && !has1 ? 0u : min(16u, p_end - p0g[u]);
      if constexpr (FP) {
        // the step's new positions take the rows computed above (the cache may not hold them
        // yet): they overwrite the group's loaded rows in the slot, chunk c at c ^ f(row)
        const uint32_t p0 = p_begin + 16u * (wave + 4u * tg);
        if (glen[u] && p0 + glen[u] > pn0) {  // uniform
          wave_lds_sync();
          unsigned char* sl = ring + (slot[u] - ring_lds);
          for (uint32_t p = max(p0, pn0); p < p0 + glen[u]; ++p) {
            const uint32_t r = p - p0;
            for (uint32_t c = lane; c < 2u * CPR; c += 64u) {  // K chunks, then V chunks
              const uint32_t cc = c % CPR;
              const uint16_t* src = (c < CPR ? s_newk : s_newv) + (p - pn0) * HD + 8u * cc;
              *reinterpret_cast<u4_t*>(sl + (c < CPR ? 0u : GB) + r * ROWB + 16u * (cc ^ swz(r))) =
                  *reinterpret_cast<const u4_t*>(src);
            }
          }
          wave_lds_sync();
        }
      }
    }
    // every LDS read of the iteration first: K rows, V^T tiles, scales
    h8_t kh[NG][KK];
    KvChunk<1> kc[NG][KK];
#pragma unroll
    for (uint32_t u = 0; u < NG; ++u)
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk) {
        if constexpr (KV8 == 0) {
          const uint32_t c = qq + 4u * kk;
          kh[u][kk] = *reinterpret_cast<const h8_t*>(ring + (slot[u] - ring_lds) + qi * ROWB + 16u * (c ^ swz(qi)));
        } else {
          const uint32_t b = 8u * qq + 32u * kk;
          kc[u][kk].w = *reinterpret_cast<const u2_t*>(ring + (slot[u] - ring_lds) + qi * ROWB + 16u * ((b >> 4) ^ swz(qi)) + (b & 15u));
        }
      }
    h4_t av[NG][KV8 ? 1 : NT];
    v2i_t raw[NG][KV8 ? NT / 2 : 1];
#pragma unroll
    for (uint32_t u = 0; u < NG; ++u) {
      const uint32_t vslot = slot[u] + GB;
#pragma unroll
      for (uint32_t i = 0; i < NTR; ++i) {
        if constexpr (KV8 == 0) {
          // ds_read_b64_tr_b16: lane L' = 4 jj + h of a 16-lane group supplies row 4 g + jj, dims
          // 16 tt + 4 h .. + 3; lane i receives dim 16 tt + i of rows 4 g .. 4 g + 3
          const uint32_t jj = qi >> 2, hh = qi & 3u, row = 4u * qq + jj;
          const uint32_t b = 32u * i + 8u * hh;
          const uint32_t ad = vslot + row * ROWB + 16u * ((b >> 4) ^ swz(row)) + (b & 15u);
          av[u][i] = __builtin_bit_cast(h4_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                  (v4s_t __attribute__((address_space(3)))*)(uintptr_t)ad));
        } else {
          // ds_read_b64_tr_b8: lane L' = 2 jj + h supplies row 4 g + (jj & 3), dims 16 t + 8 h .. + 7
          // (t the pair's first tile for jj < 4, else its second); lane i receives dim 16 t + i of
          // rows 4 g .. 4 g + 3 in bytes 0..3 (first tile) and 4..7 (second)
          const uint32_t jj = qi >> 1, hh = qi & 1u, row = 4u * qq + (jj & 3u);
          const uint32_t tile = 2u * i + (jj >> 2);
          const uint32_t b = 16u * tile + 8u * hh;
          const uint32_t ad = vslot + row * ROWB + 16u * ((b >> 4) ^ swz(row)) + (b & 15u);
          raw[u][i] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((v2i_t __attribute__((address_space(3)))*)(uintptr_t)ad);
        }
      }
    }
    uint32_t kw[NG][4], vw[NG][4];
    if constexpr (KV8 == 1) {
#pragma unroll
      for (uint32_t u = 0; u < NG; ++u) {
        const uint32_t* ss = reinterpret_cast<const uint32_t*>(ring + (slot[u] - ring_lds) + 2u * GB);
        const u4_t k4 = *reinterpret_cast<const u4_t*>(ss + 4u * qq);
        const u4_t v4 = *reinterpret_cast<const u4_t*>(ss + 16u + 4u * qq);
        kw[u][0] = k4.x; kw[u][1] = k4.y; kw[u][2] = k4.z; kw[u][3] = k4.w;
        vw[u][0] = v4.x; vw[u][1] = v4.y; vw[u][2] = v4.z; vw[u][3] = v4.w;
      }
    }
    // the int8 rows' score and V scales (shared by the tiles)
    float rsc[NG][4], vsv[NG][4];
#pragma unroll
    for (uint32_t u = 0; u < NG; ++u) {
      uint32_t rb = 0;
      if constexpr (KV8 == 1) rb = group_row(wave + 4u * (u && has1 ? tw + 1 : tw));
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) {
        rsc[u][r] = qscale;
        vsv[u][r] = 1.0f;
        if constexpr (KV8 == 1) {
          const uint32_t rr = glen[u] ? min(4u * qq + r, glen[u] - 1u) : 0u;
          const uint32_t er = (uint32_t)((size_t)(rb + rr) * a.sc_row_stride);
          rsc[u][r] = qscale * h2f((uint16_t)(((er + kpar0) & 1u) ? kw[u][r] >> 16 : kw[u][r] & 0xFFFFu));
          vsv[u][r] = h2f((uint16_t)(((er + vpar0) & 1u) ? vw[u][r] >> 16 : vw[u][r] & 0xFFFFu));
        }
      }
    }
#pragma unroll
    for (uint32_t ct = 0; ct < CT; ++ct) {
      // scores S^T[position 4 qq + r][column 16 ct + qi]: the f16 high and low parts of q on
      // two chains
      f4_t dh[NG], dl[NG];
#pragma unroll
      for (uint32_t u = 0; u < NG; ++u) dh[u] = dl[u] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk)
#pragma unroll
        for (uint32_t u = 0; u < NG; ++u) {
          const h8_t k8 = KV8 ? chunk_h8<1>(kc[u][kk]) : kh[u][kk];
          dh[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k8, s_q[ct][0][kk][lane], dh[u], 0, 0, 0);
          dl[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k8, s_q[ct][1][kk][lane], dl[u], 0, 0, 0);
        }
      float sc[NG][4];
      float mx = -INFINITY;
#pragma unroll
      for (uint32_t u = 0; u < NG; ++u)
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r) {
          sc[u][r] = 4u * qq + r < glen[u] && p0g[u] + 4u * qq + r < pe_col[ct] ? (dh[u][r] + dl[u][r]) * rsc[u][r]
                                                                                : -INFINITY;
          mx = fmaxf(mx, sc[u][r]);
        }
      mx = head_max(mx);
      // a column none of whose positions are in these groups keeps its state
      const bool colive = p0g[0] < pe_col[ct];
      const float m_new = colive ? fmaxf(m_run[ct], mx) : m_run[ct];
      const float alpha = colive ? __builtin_amdgcn_exp2f(m_run[ct] - m_new) : 1.0f;  // 0 on the first group
      float w[NG][4];
      float wsum = 0.f;
#pragma unroll
      for (uint32_t u = 0; u < NG; ++u) {
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r) w[u][r] = colive ? __builtin_amdgcn_exp2f(sc[u][r] - m_new) : 0.f;
        wsum += (w[u][0] + w[u][1]) + (w[u][2] + w[u][3]);
      }
      l_run[ct] = __builtin_fmaf(l_run[ct], alpha, wsum);
      m_run[ct] = m_new;
      if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (uint32_t tt = 0; tt < NT; ++tt) acc[ct][tt] *= alpha;
      }
      // B operands: the weights (int8: times the row's V scale), f16 high and low parts
      h4_t bh[NG], bl[NG];
#pragma unroll
      for (uint32_t u = 0; u < NG; ++u)
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r) {
          const float wv = w[u][r] * vsv[u][r];
          const half_t h = (half_t)wv;
          bh[u][r] = h;
          bl[u][r] = (half_t)(wv - (float)h);
        }
      // P V per 16-dim tile
#pragma unroll
      for (uint32_t i = 0; i < NTR; ++i) {
#pragma unroll
        for (uint32_t u = 0; u < NG; ++u) {
          if constexpr (KV8 == 0) {
            acc[ct][i] = __builtin_amdgcn_mfma_f32_16x16x16f16(av[u][i], bh[u], acc[ct][i], 0, 0, 0);
            acc[ct][i] = __builtin_amdgcn_mfma_f32_16x16x16f16(av[u][i], bl[u], acc[ct][i], 0, 0, 0);
          } else {
            const h2_t bias = {(half_t)1152.0f, (half_t)1152.0f};
            const uint32_t x0 = (uint32_t)raw[u][i].x ^ 0x80808080u, x1 = (uint32_t)raw[u][i].y ^ 0x80808080u;
            const uint32_t hi = 0x64646464u;
            const h2_t p0 = as_h2(__builtin_amdgcn_perm(hi, x0, 0x04010400u)) - bias;
            const h2_t p1 = as_h2(__builtin_amdgcn_perm(hi, x0, 0x04030402u)) - bias;
            const h2_t p2 = as_h2(__builtin_amdgcn_perm(hi, x1, 0x04010400u)) - bias;
            const h2_t p3 = as_h2(__builtin_amdgcn_perm(hi, x1, 0x04030402u)) - bias;
            const h4_t a0 = h4_t{p0[0], p0[1], p1[0], p1[1]}, a1 = h4_t{p2[0], p2[1], p3[0], p3[1]};
            acc[ct][2 * i] = __builtin_amdgcn_mfma_f32_16x16x16f16(a0, bh[u], acc[ct][2 * i], 0, 0, 0);
            acc[ct][2 * i] = __builtin_amdgcn_mfma_f32_16x16x16f16(a0, bl[u], acc[ct][2 * i], 0, 0, 0);
            acc[ct][2 * i + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(a1, bh[u], acc[ct][2 * i + 1], 0, 0, 0);
            acc[ct][2 * i + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(a1, bl[u], acc[ct][2 * i + 1], 0, 0, 0);
          }
        }
      }
    }
    // the slots take this wave's groups tw + NB (and tw + 1 + NB); dma16 waits for the reads
#pragma unroll
    for (uint32_t u = 0; u < NG; ++u)
      if (tw + u + NB < ngw) issue(tw + u + NB, group_row(wave + 4u * (tw + u + NB)));
  }
  wait_vm<0>();
  lds_barrier();  // every wave is done with its ring, which the merge reuses
  // merge the four waves per tile of columns: M = max m_w, f_w = exp(m_w - M), sum and acc
  // weighted by f_w in wave order (the state's max in natural units: max * ln 2)
  float* red = reinterpret_cast<float*>(s_ring);  // [4][16][HD]
  const uint32_t ncols = (r_hi - r_lo) * GQA;      // the live columns
#pragma unroll
  for (uint32_t ct = 0; ct < CT; ++ct) {
    const uint32_t nlc = ncols > 16u * ct ? min(ncols - 16u * ct, 16u) : 0u;  // this tile's
    if (nlc == 0) break;  // uniform
    if (ct) lds_barrier();  // the previous tile's merge is done with red and the st arrays
    const float mr = m_run[ct] * 0.6931471805599453f;
    float l = l_run[ct] + __shfl_xor(l_run[ct], 16, 64);
    l = l + __shfl_xor(l, 32, 64);
    if (qq == 0) {
      st_m[wave][qi] = mr;
      st_l[wave][qi] = l;
    }
    if (qi < nlc) {
#pragma unroll
      for (uint32_t tt = 0; tt < NT; ++tt)
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r) red[(wave * 16u + qi) * HD + 16u * tt + 4u * qq + r] = acc[ct][tt][r];
    }
    lds_barrier();
    if (t < nlc) {
      float M = st_m[0][t];
#pragma unroll
      for (uint32_t w2 = 1; w2 < 4; ++w2) M = fmaxf(M, st_m[w2][t]);
      float sm = 0.f;
#pragma unroll
      for (uint32_t w2 = 0; w2 < 4; ++w2) {
        const float f = expf(st_m[w2][t] - M);
        sm = __builtin_fmaf(st_l[w2][t], f, sm);
        st_f[w2][t] = f;
      }
      st_hm[t] = M;
      st_hs[t] = sm;
    }
    lds_barrier();
    for (uint32_t idx = t; idx < nlc * HD; idx += 256u) {
      const uint32_t g = idx / HD, dd = idx % HD, c = 16u * ct + g, row = r_lo + c / GQA;
      // a row whose keys end before this block has no partial here
      if (blk * s >= row_len(row)) continue;
      float v = 0.f;
#pragma unroll
      for (uint32_t w2 = 0; w2 < 4; ++w2) v = __builtin_fmaf(red[(w2 * 16u + g) * HD + dd], st_f[w2][g], v);
      float* out = a.attn_part + (((size_t)(j * GQA + c % GQA) * a.tgt + blk) * a.M + row) * (HD + 2);
      *as_global(out + 2 + dd) = v;
      if (dd == 0) {
        out[0] = st_hm[g];
        out[1] = st_hs[g];
      }
    }
  }
}

}  // namespace mi
