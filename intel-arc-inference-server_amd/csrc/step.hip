// step.hip - the batch-1 decode step as one persistent launch (the interface is step.h).
//
// The reference records a step as ~710 dependent kernel launches in one command list
// (src/runtime/capture.cc:279-319, 1332-1480) and replays it per token (Engine::replay,
// src/runtime/engine.cc:702-713). On MI355X each dependent launch costs its ramp, its tail and a
// trip through the command processor, a few microseconds that the 27B step pays ~390 times.
// Here the same work is one launch:
//
//   * Work-items. The step is a list of work-items in dependency order. Per layer:
//       qkv slices   the qkv GEMV's (tile, split-K slice) work-groups, partials published;
//       heads        one per q / k / v head: the fold of the head's qkv partials, q/k RMSNorm,
//                    RoPE, q published, K/V written to the cache row and published;
//       attention    one per (kv head, block): attn_decode_v2's block (attn_core.h);
//       merges       one per q head: attn_reduce_v2's ascending block merge;
//       o slices     the o GEMV; slice S-1 of each tile is its consumer (residual add and the
//                    tiles' sum-of-squares exchange for the next RMSNorm);
//       gate||up     the gate||up GEMV; consumers apply SwiGLU;
//       down         the down GEMV; consumers as o's, producing the next layer's input.
//     Then the head GEMV (consumers keep the logits and each tile's argmax) and the argmax.
//     Work-group w takes items w, w + P, w + 2P, ... (P = the work-groups the GPU holds at
//     once). An item only waits for items earlier in the list, and every earlier item belongs
//     to a work-group that is running or done, so the step cannot deadlock while all P
//     work-groups are resident (the engine launches exactly as many as fit).
//   * Hand-off words (gemv_core.h): every value an item hands on is stored device-coherent
//     into words that hold the empty pattern until then, and the reader polls until they are
//     not. A word with one reader is emptied again by it; words with many readers (a layer's
//     normed inputs, q, the attention output, SwiGLU's output) are emptied by the next layer's
//     merge items, which run only after every reader of them has finished (each reader fed a
//     value the merge transitively waited for). So every step leaves all words empty again.
//   * Streaming. A work-group issues the weight loads of its next item before it handles the
//     current one, so while it waits for a stage's inputs the next slice's weights are on the
//     way. At a slice stage's first item it polls the activations its items of that stage need
//     into LDS once (the whole input vector, or its items' K ranges), so the slices compute
//     from LDS and their register prefetch never waits behind a poll.
//   * Bounded waits. Each poll gives up at a deadline (Waiter): the control block's DEBUG word
//     becomes MI_STATUS_HANDOFF_TIMEOUT and every later wait of that thread takes what it finds,
//     so a broken step ends promptly with its output marked invalid.
// Every arithmetic operation is the launch path's (gemv_w4a16.hip, prep.hip, attn.hip) in the
// same order, so logits, KV rows and the control block are bitwise the graph of launches'.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <memory>
#include <cstdio>
#include <cstring>
#include <new>
#include <vector>

#include "mi_capi_internal.h"
#include "mi_common.h"
#include "gemv_core.h"
#include "attn_core.h"
#include "step.h"

namespace mi {
namespace {

enum : uint32_t { SK_EMBED = 0, SK_SLICE = 1, SK_HEAD = 2, SK_ATTN = 3, SK_REDUCE = 4, SK_FINISH = 5 };
enum : uint32_t { SE_NONE = 0, SE_RESID = 1, SE_SILU = 2, SE_LOGITS = 3 };

constexpr uint32_t kXcHalves = 8192;  // the LDS activation cache of a work-group (16 KiB)
constexpr uint32_t kMaxGps = 8;       // k-groups per slice (two per wave)
constexpr uint32_t kQuad = 4;         // producer slice items per unit
constexpr uint64_t kTimeoutTicks = 20000000ull;  // 200 ms of s_memrealtime (100 MHz)

struct Stage {
  uint32_t kind, first, count, epi;
  // units: what one work-group takes at a time. A slice stage's producer items go in groups of
  // up to kQuad adjacent tiles of one slice (their weights all in flight at once), its consumer
  // items one by one; every other stage's items one by one.
  uint32_t ufirst, units, prod_units, prod_items, ups;  // ups: producer units per slice
  // SK_SLICE: the linear and its split
  const uint32_t* qw;
  const uint16_t* sc;
  uint32_t K, N, S, gps, tiles;
  uint32_t xc_whole;   // 1: the work-group caches the whole input vector; 0: its items' K ranges
  const uint32_t* x;   // the input, f16 pairs [K / 2]
  float* part;         // hand-off partials [S][N] (a consumer slice publishes none)
  // slice consumers
  uint32_t* resid_in;   // RESID: f16 pairs [N / 2] (one reader per tile)
  uint32_t* resid_out;  // RESID
  float* sumsq;         // RESID: [tiles][tiles], consumer c's copy at row c
  const float* norm_w;  // RESID: the next RMSNorm's weights [N]
  uint32_t* x_next;     // RESID: f16 pairs [N / 2]
  uint32_t* h;          // SILU: f16 pairs [N / 4]
  float* logits;        // LOGITS: [N]
  uint32_t* am;         // LOGITS: (value bits, index) per tile
  uint32_t vocab_used;
  // SK_HEAD / SK_ATTN / SK_REDUCE: one layer's attention
  const float* part_qkv;  // HEAD: [S_qkv][qkv_n]
  uint32_t S_qkv, qkv_n;
  const float* q_norm;
  const float* k_norm;
  float* attn_q;      // [q_heads][HD]
  uint16_t* kv_k;     // the layer's cache [kv_heads][max_len][HD]
  uint16_t* kv_v;
  uint32_t* newkv;    // [kv_heads][HD]: the new row's K pairs, then its V pairs
  float* attn_part;   // [q_heads][tgt][HD + 2]
  uint32_t* attn_out; // f16 pairs [q_heads HD / 2]
  // words the stage's items empty again, split evenly between them
  uint32_t* jan;
  uint32_t jan_words;
};

struct StepArgs {
  const Stage* stages;
  uint32_t total;  // units
  uint32_t* ctrl;
  uint32_t* history;
  uint32_t history_len;
  const uint16_t* embed;
  const float* norm0;  // layer 0's input RMSNorm weights
  uint32_t* r0;        // EMBED: the residual, f16 pairs [H / 2]
  uint32_t* x0;        // EMBED: layer 0's normed input
  const float* rope;
  uint32_t hidden, vocab, q_heads, kv_heads, rot_dim, max_len, tgt;
  float eps, scale;
  uint32_t* trace;  // diagnostics (NULL normally): per unit its start and end (s_memrealtime)
};

struct SliceW {
  u4_t w[2][2];
  u2_t s[2];
};

// the weights of slice item i (tile i % tiles, slice i / tiles): wave w takes the slice's
// k-groups w and w + 4, lane l the 4 columns 4 (l % 16) .. of word rows 4 h + l / 16
__device__ __forceinline__ void slice_load(SliceW& W, const Stage& st, uint32_t i) {
  const uint32_t tiles = st.tiles, N = st.N, gps = st.gps;
  const uint32_t s = i / tiles, tile = i - s * tiles;
  const uint32_t lane = opaque_tid() & 63u, wave = opaque_tid() >> 6, c4 = lane & 15u, q = lane >> 4;
  const uint32_t ncol = tile * 64u + 4u * c4;
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    const uint32_t gl = wave + 4u * u;
    if (gl < gps) {
      const uint32_t g = s * gps + gl;
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) W.w[u][h] = load_stream16(st.qw + (size_t)(g * 8u + 4u * h + q) * N + ncol);
      W.s[u] = *as_global(reinterpret_cast<const u2_t*>(st.sc + (size_t)g * N + ncol));
    }
  }
}

struct SliceWQ {
  SliceW w[kQuad];
};
// the weights of a unit's n <= kQuad slice items i0 .. i0 + n - 1, all loads out together in
// item order
__device__ __forceinline__ void slice_loadq(SliceWQ& W, const Stage& st, uint32_t i0, uint32_t n) {
#pragma unroll
  for (uint32_t k = 0; k < kQuad; ++k)
    if (k < n) slice_load(W.w[k], st, i0 + k);
}

// Thread t polls the hand-off words of elements e = t + 256 u < n (u < PER) into dst[e] (LDS):
// element e's word sits at byte offset voff + u * ustride from base (a per-thread offset and a
// uniform one per u: buffer loads, no 64-bit address registers). All the loads go out together,
// the still-empty words are polled again together, and each word is emptied again after it is
// read when `take` (its only reader).
template <int PER>
__device__ __forceinline__ void poll_lds(Waiter& wt, const void* base, uint32_t n, uint32_t voff, uint32_t ustride,
                                         uint32_t* dst, bool take) {
  constexpr int kSc1 = 16;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFFF, 0x00020000);
  const uint32_t t = opaque_tid();
  uint32_t v[PER];
  uint32_t pending = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (t + 256u * u < n) v[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, u * ustride, kSc1);
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (t + 256u * u < n && v[u] == kEmpty) pending |= 1u << u;
  while (pending && !wt.give_up()) {
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if (pending & (1u << u)) v[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, u * ustride, kSc1);
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if ((pending & (1u << u)) && v[u] != kEmpty) pending &= ~(1u << u);
  }
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (t + 256u * u < n) {
      dst[t + 256u * u] = v[u];
      if (take) __builtin_amdgcn_raw_buffer_store_b32(kEmpty, rs, voff, u * ustride, kSc1);
    }
}

// poll_lds over any n: rounds of 2048 elements (8 per thread), element e = 2048 r + t + 256 u
// at byte offset voff + (8 r + u) * ustride
__device__ __forceinline__ void poll_lds_n(Waiter& wt, const void* base, uint32_t n, uint32_t voff, uint32_t ustride,
                                           uint32_t* dst, bool take) {
  for (uint32_t r0 = 0; r0 < n; r0 += 2048u)
    poll_lds<8>(wt, static_cast<const unsigned char*>(base) + (size_t)(r0 / 256u) * ustride, n - r0, voff, ustride,
                dst + r0, take);
}

// empties this item's share of the stage's many-reader words
__device__ __forceinline__ void janitor(const Stage& st, uint32_t i) {
  if (!st.jan_words) return;
  const uint32_t per = (st.jan_words + st.count - 1u) / st.count;
  const uint32_t b = i * per, e = min(b + per, st.jan_words);
  for (uint32_t k = b + opaque_tid(); k < e; k += 256u) st_agent(st.jan + k, kEmpty);
}

struct Lds {
  float red[4][64];
  float redq[kQuad][4][64];  // a producer unit's items
  float fold[2048];
  uint32_t words[4096];  // polled words (consumers, heads, merges, the argmax)
  uint32_t rw[32];       // a RESID consumer's residual tile (f16 pairs)
  float rowv[64];
  float misc[8];
};

// ---- slice items: the GEMV (gemv_w4a16_kernel<1, 2, EPI> at M = 1) and its consumers ----
// One slice of one tile into red[wave][col]: wave w's k-groups w and w + 4 of the slice, each an
// MFMA batch scaled per column, summed in group order (the launch kernel's per-wave partial).
__device__ __forceinline__ void slice_gemv(const Stage& st, const SliceW& W, const uint16_t* xrow,
                                           float (*red)[64]) {
  const uint32_t t = opaque_tid(), lane = t & 63u, wave = t >> 6, c4 = lane & 15u, q = lane >> 4;
  const uint32_t gps = st.gps;
  const uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u, magic = 0x64006400u;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (uint32_t u = 0; u < 2; ++u) {
    const uint32_t gl = wave + 4u * u;
    if (gl < gps) {
      f4_t d[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) d[c] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const u4_t xv = c4 == 0 ? *reinterpret_cast<const u4_t*>(xrow + gl * 64u + 32u * h + 8u * q)
                                : u4_t{0u, 0u, 0u, 0u};
        const h8_t av = perm_x(xv);
        const uint32_t ws[4] = {W.w[u][h].x, W.w[u][h].y, W.w[u][h].z, W.w[u][h].w};
        h8_t bw[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) bw[c] = dequant_word(ws[c], m_lo, m_hi, magic);
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bw[c], d[c], 0, 0, 0);
        keep_mfma_batch(av, bw, d);
      }
      const float sc[4] = {h2f((uint16_t)(W.s[u].x & 0xFFFFu)), h2f((uint16_t)(W.s[u].x >> 16)),
                           h2f((uint16_t)(W.s[u].y & 0xFFFFu)), h2f((uint16_t)(W.s[u].y >> 16))};
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = __builtin_fmaf(d[c][0], sc[c], acc[c]);
    }
  }
  if (q == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) red[wave][4u * c4 + c] = acc[c];
  }
}

// A producer unit: items i0 .. i0 + n - 1, adjacent tiles of one slice; each tile's four wave
// partials summed in wave order (wave k sums item i0 + k) and published as its slice's partial.
__device__ __forceinline__ void slice_quad(const Stage& st, uint32_t i0, uint32_t n, const SliceWQ& W,
                                           const uint16_t* xrow, Lds& L) {
  const uint32_t t = opaque_tid();
#pragma unroll
  for (uint32_t k = 0; k < kQuad; ++k)
    if (k < n) slice_gemv(st, W.w[k], xrow, L.redq[k]);
  lds_barrier();
  const uint32_t k = t >> 6, col = t & 63u;
  if (k < n) {
    const uint32_t i = i0 + k, s = i / st.tiles, n0 = (i - s * st.tiles) * 64u;
    float v = L.redq[k][0][col];
#pragma unroll
    for (int w = 1; w < 4; ++w) v += L.redq[k][w][col];
    st_agent(st.part + (size_t)s * st.N + n0 + col, publishable(v));
  }
  lds_barrier();  // L.redq is reused by the next unit
}

// A single slice item; the consumer slice (S-1) of a fused stage also folds the tile and applies
// the epilogue.
__device__ __forceinline__ void slice_item(const Stage& st, uint32_t i, const SliceW& W, const uint16_t* xrow,
                                           Lds& L, Waiter& wt) {
  const uint32_t t = opaque_tid(), lane = t & 63u, wave = t >> 6;
  const uint32_t tiles = st.tiles, N = st.N, S = st.S;
  const uint32_t s = i / tiles, tile = i - s * tiles, n0 = tile * 64u;
  slice_gemv(st, W, xrow, L.red);
  lds_barrier();
  const bool consumer = st.epi != SE_NONE && s + 1u == S;  // uniform
  float v = 0.f;
  if (t < 64u) {
    v = L.red[0][t];
#pragma unroll
    for (int w = 1; w < 4; ++w) v += L.red[w][t];
    if (!consumer) st_agent(st.part + (size_t)s * N + n0 + t, publishable(v));
  }
  if (!consumer) {
    lds_barrier();  // L.red is reused by the next item
    return;
  }
  // ---- the tile's consumer: fold the other S-1 slices in ascending s, its own last ----
  // (the RESID residual goes out with the poll)
  uint32_t* words = L.words;
  const uint32_t np = (S - 1u) * 64u;
  const float* part = st.part;
  poll_lds_n(wt, part, np, ((t >> 6) * N + n0 + (t & 63u)) * 4u, 4u * N * 4u, words, true);
  if (st.epi == SE_RESID) poll_lds<1>(wt, st.resid_in + tile * 32u, 32u, t * 4u, 0u, L.rw, true);
  lds_barrier();
  if (t < 64u) {
    float a = 0.f;
    for (uint32_t j = 0; j + 1u < S; ++j) a += __builtin_bit_cast(float, words[j * 64u + t]);
    L.rowv[t] = a + v;
  }
  lds_barrier();
  if (st.epi == SE_RESID) {
    // wave 0, a column per lane: the residual, the tile's sum of squares to every consumer's copy
    if (wave == 0) {
      const uint32_t rw = L.rw[lane / 2u];
      const uint16_t r_pre = (uint16_t)((lane & 1u) ? (rw >> 16) : (rw & 0xFFFFu));
      const uint16_t rb = f2h(h2f(r_pre) + h2f(f2h(L.rowv[lane])));
      const uint16_t rb_up = (uint16_t)__shfl((int)rb, (int)(lane + 1u), 64);
      if (!(lane & 1u)) st_agent(st.resid_out + tile * 32u + lane / 2u, publishable_pair(rb, rb_up));
      const float rv = h2f(rb);
      L.red[1][lane] = rv;
      float a2 = __builtin_fmaf(rv, rv, 0.f);
#pragma unroll
      for (int sst = 32; sst > 0; sst >>= 1) a2 += __shfl_down(a2, sst, 64);
      a2 = publishable(__shfl(a2, 0, 64));
      for (uint32_t c = lane; c < tiles; c += 64u) st_agent(st.sumsq + (size_t)c * tiles + tile, a2);
    }
    // every tile's sum (this consumer's copy), added in ascending tile order
    poll_lds<1>(wt, st.sumsq + (size_t)tile * tiles, tiles, t * 4u, 0u, words, true);
    lds_barrier();
    if (t == 0) {
      float tot = 0.f;
      for (uint32_t g = 0; g < tiles; ++g) tot += __builtin_bit_cast(float, words[g]);
      L.misc[0] = 1.0f / sqrtf(tot / (float)N + L.misc[1]);
    }
    lds_barrier();
    if (wave == 0) {
      const uint16_t xb = f2h(L.red[1][lane] * L.misc[0] * *as_global(st.norm_w + n0 + lane));
      const uint16_t xb_up = (uint16_t)__shfl((int)xb, (int)(lane + 1u), 64);
      if (!(lane & 1u)) st_agent(st.x_next + tile * 32u + lane / 2u, publishable_pair(xb, xb_up));
    }
  } else if (st.epi == SE_SILU) {
    // 64 interleave16 columns = 32 outputs tile 32 + kk (gate at gcol, up at gcol + 16)
    if (t < 16u) {
      uint16_t o[2];
#pragma unroll
      for (uint32_t k2 = 0; k2 < 2; ++k2) {
        const uint32_t kk = 2u * t + k2, gcol = (kk / 16u) * 32u + (kk % 16u);
        const uint16_t g_b = f2h(L.rowv[gcol]), u_b = f2h(L.rowv[gcol + 16u]);
        const uint16_t s_b = f2h(silu_f32(h2f(g_b)));
        o[k2] = f2h(h2f(s_b) * h2f(u_b));
      }
      st_agent(st.h + tile * 16u + t, publishable_pair(o[0], o[1]));
    }
  } else {  // SE_LOGITS
    if (wave == 0) {
      const uint32_t n = n0 + lane;
      const float lv = L.rowv[lane];
      *as_global(st.logits + n) = lv;
      float bv = n < st.vocab_used ? lv : -INFINITY;
      uint32_t bi = n;
#pragma unroll
      for (int sst = 32; sst > 0; sst >>= 1) {
        const float ov = __shfl_down(bv, sst, 64);
        const uint32_t oi = __shfl_down(bi, sst, 64);
        if (lane + sst < 64 && ((ov > bv) || (ov == bv && oi < bi))) {
          bv = ov;
          bi = oi;
        }
      }
      const bool bad = __ballot(n < st.vocab_used && !__builtin_isfinite(lv)) != 0ull;
      if (lane == 0) {
        st_agent(st.am + 2u * tile, bad ? kNanBits : __builtin_bit_cast(uint32_t, publishable(bv)));
        st_agent(st.am + 2u * tile + 1u, bi);
      }
    }
  }
  lds_barrier();
}

// ---- head items: attn_prep's chain on one head (qkv_consumer in gemv_w4a16.hip, M = 1) ----
template <int HD>
__device__ __forceinline__ void head_item(const StepArgs& a, const Stage& st, uint32_t hh, uint32_t pos, Lds& L,
                                          Waiter& wt) {
  constexpr uint32_t EPL = HD / 64u;
  const uint32_t t = opaque_tid(), lane = t & 63u, wave = t >> 6;
  const uint32_t QH = a.q_heads, KVH = a.kv_heads, N = st.qkv_n, S = st.S_qkv;
  const bool is_q = hh < QH, is_k = !is_q && hh < QH + KVH;
  const uint32_t h = is_q ? hh : (is_k ? hh - QH : hh - QH - KVH);
  const uint32_t nh0 = hh * HD;
  const float* nw = is_q ? st.q_norm : (is_k ? st.k_norm : nullptr);
  const uint32_t half = a.rot_dim / 2u;
  float wn[EPL], rc[EPL], rsn[EPL];
  if (wave == 0) {
    const float* cs = a.rope + (size_t)pos * 2u * half;
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) {
      const uint32_t e = lane + 64u * k;
      wn[k] = nw ? nw[e] : 0.f;
      rc[k] = 1.f;
      rsn[k] = 0.f;
      if ((is_q || is_k) && e < a.rot_dim) {
        const uint32_t ii = e < half ? e : e - half;
        rc[k] = cs[ii];
        rsn[k] = cs[half + ii];
      }
    }
  }
  // the fold over all S slices in ascending s from +0
  const float* part = st.part_qkv;
  poll_lds_n(wt, part, S * HD, ((t / HD) * N + nh0 + t % HD) * 4u, (256u / HD) * N * 4u, L.words, true);
  lds_barrier();
  if (t < HD) {
    float acc = 0.f;
    for (uint32_t j = 0; j < S; ++j) acc += __builtin_bit_cast(float, L.words[j * HD + t]);
    L.fold[t] = acc;
  }
  lds_barrier();
  if (wave == 0) {
    const size_t crow = (size_t)pos * HD + (size_t)h * a.max_len * HD;  // row pos of kv head h
    if (!is_q && !is_k) {
      uint16_t vb[EPL];
#pragma unroll
      for (uint32_t k = 0; k < EPL; ++k) {
        vb[k] = f2h(L.fold[lane + 64u * k]);
        *as_global(st.kv_v + crow + lane + 64u * k) = vb[k];
        const uint16_t up = (uint16_t)__shfl((int)vb[k], (int)(lane + 1u), 64);
        if (!(lane & 1u)) st_agent(st.newkv + (size_t)h * HD + HD / 2u + (lane + 64u * k) / 2u, publishable_pair(vb[k], up));
      }
    } else {
      float xf[EPL], nv[EPL];
#pragma unroll
      for (uint32_t k = 0; k < EPL; ++k) xf[k] = h2f(f2h(L.fold[lane + 64u * k]));
      if (nw) {
        float sq[EPL];
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) sq[k] = xf[k] * xf[k];
        float acc;
        if constexpr (EPL == 4) acc = (sq[0] + sq[2]) + (sq[1] + sq[3]);
        else acc = sq[0] + sq[1];
#pragma unroll
        for (int sst = 32; sst > 0; sst >>= 1) acc += __shfl_down(acc, sst, 64);
        const float tot = __shfl(acc, 0, 64);
        const float rstd = 1.0f / sqrtf(tot / (float)HD + a.eps);
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) nv[k] = h2f(f2h(xf[k] * rstd * wn[k]));
      } else {
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) nv[k] = xf[k];
      }
      float* nrm = L.fold + HD;
#pragma unroll
      for (uint32_t k = 0; k < EPL; ++k) nrm[lane + 64u * k] = nv[k];
      wave_lds_sync();
#pragma unroll
      for (uint32_t k = 0; k < EPL; ++k) {
        const uint32_t e = lane + 64u * k;
        float out;
        if (e < half) {
          const float tt = nrm[e + half] * rsn[k];
          out = __builtin_fmaf(nv[k], rc[k], -tt);
        } else if (e < a.rot_dim) {
          const float tt = nrm[e - half] * rsn[k];
          out = __builtin_fmaf(nv[k], rc[k], tt);
        } else {
          out = nv[k];
        }
        if (is_q) {
          st_agent(st.attn_q + (size_t)h * HD + e, publishable(out));
        } else {
          const uint16_t kb = f2h(out);
          *as_global(st.kv_k + crow + e) = kb;
          const uint16_t up = (uint16_t)__shfl((int)kb, (int)(lane + 1u), 64);
          if (!(lane & 1u)) st_agent(st.newkv + (size_t)h * HD + e / 2u, publishable_pair(kb, up));
        }
      }
    }
  }
  lds_barrier();
}

// ---- merge items: attn_reduce_kernel<false, 64> at M = 1, ungated ----
template <int HD>
__device__ __forceinline__ void reduce_item(const StepArgs& a, const Stage& st, uint32_t h, uint32_t pos, Lds& L,
                                            Waiter& wt) {
  const uint32_t t = opaque_tid(), d = t;
  const uint32_t L1 = pos + 1u;
  uint32_t nb = (L1 - 1u) / v2_ppw(L1, a.tgt) + 1u;
  if (nb > a.tgt) nb = a.tgt;
  const size_t PART = HD + 2u;
  float* base = st.attn_part + (size_t)h * a.tgt * PART;  // block b at + b * PART
  // every block's (max, sum)
  poll_lds<1>(wt, base, 2u * nb, ((t >> 1) * (uint32_t)PART + (t & 1u)) * 4u, 0u, L.words, true);
  lds_barrier();
  float* fac = L.fold;
  if (t < 64u) {
    float mx = -INFINITY;
    for (uint32_t b = t; b < nb; b += 64u) mx = fmaxf(mx, __builtin_bit_cast(float, L.words[2u * b]));
    mx = wave_max(mx);
    float sm = 0.f;
    for (uint32_t b = t; b < nb; b += 64u) {
      const float f = expf(__builtin_bit_cast(float, L.words[2u * b]) - mx);
      fac[b] = f;
      sm = __builtin_fmaf(__builtin_bit_cast(float, L.words[2u * b + 1u]), f, sm);
    }
    sm = wave_sum(sm);
    if (t == 0) L.misc[2] = sm;
  }
  lds_barrier();
  // the blocks' accumulators, 16 blocks per round, added in ascending block order
  float acc = 0.f;
  if (d < HD) {
    constexpr int kSc1 = 16;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7FFFFFFF, 0x00020000);
    const uint32_t voff = (2u + d) * 4u, bstride = (uint32_t)PART * 4u;
    for (uint32_t b0 = 0; b0 < nb; b0 += 16u) {
      const uint32_t nr = min(16u, nb - b0);
      uint32_t v[16];
      uint32_t pending = 0;
#pragma unroll
      for (uint32_t u = 0; u < 16; ++u)
        if (u < nr) v[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, (b0 + u) * bstride, kSc1);
#pragma unroll
      for (uint32_t u = 0; u < 16; ++u)
        if (u < nr && v[u] == kEmpty) pending |= 1u << u;
      while (pending && !wt.give_up()) {
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (uint32_t u = 0; u < 16; ++u)
          if (pending & (1u << u)) v[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, (b0 + u) * bstride, kSc1);
#pragma unroll
        for (uint32_t u = 0; u < 16; ++u)
          if ((pending & (1u << u)) && v[u] != kEmpty) pending &= ~(1u << u);
      }
#pragma unroll
      for (uint32_t u = 0; u < 16; ++u)
        if (u < nr) {
          acc = __builtin_fmaf(__builtin_bit_cast(float, v[u]), fac[b0 + u], acc);
          __builtin_amdgcn_raw_buffer_store_b32(kEmpty, rs, voff, (b0 + u) * bstride, kSc1);
        }
    }
  }
  if (d < HD) {
    const float o = acc / L.misc[2];
    const uint16_t r = f2h(o);
    const uint16_t up = (uint16_t)__shfl((int)r, (int)((d & 63u) + 1u), 64);
    if (!(d & 1u)) st_agent(st.attn_out + ((size_t)h * HD + d) / 2u, publishable_pair(r, up));
  }
  janitor(st, h);
  lds_barrier();
}

// ---- the first item: embed_gather + the first RMSNorm (embed_norm_kernel<true>, M = 1) ----
__device__ __forceinline__ void embed_item(const StepArgs& a, Lds& L) {
  const uint32_t t = opaque_tid(), lane = t & 63u, wave = t >> 6, H = a.hidden;
  const uint32_t row = a.ctrl[CTRL_CUR];
  const bool bad = row >= a.vocab;  // embed_gather's rule: flag it (the step then embeds zeros)
  if (bad && t == 0) a.ctrl[CTRL_DEBUG] = 0xDEAD0001u;
  const uint16_t* src = a.embed + (size_t)(bad ? 0u : row) * H;
  const uint32_t nch = H / 64u;
  float* chunk = L.fold;
  for (uint32_t c0 = wave; c0 < nch; c0 += 32u) {
    uint16_t v16[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) {
      const uint32_t c = c0 + 4u * u;
      v16[u] = (c < nch && !bad) ? src[c * 64u + lane] : (uint16_t)0;
    }
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) {
      const uint32_t c = c0 + 4u * u;
      if (c < nch) {
        const float v = h2f(v16[u]);
        float s2 = __builtin_fmaf(v, v, 0.f);
#pragma unroll
        for (int sst = 32; sst > 0; sst >>= 1) s2 += __shfl_down(s2, sst, 64);
        if (lane == 0) chunk[c] = s2;
      }
    }
  }
  lds_barrier();
  if (t == 0) {
    float tot = 0.f;
    for (uint32_t c = 0; c < nch; ++c) tot += chunk[c];
    L.misc[3] = 1.0f / sqrtf(tot / (float)H + a.eps);
  }
  lds_barrier();
  const float r = L.misc[3];
  for (uint32_t p = t; p < H / 2u; p += 256u) {
    const uint32_t k = 2u * p;
    const uint16_t e0 = bad ? (uint16_t)0 : src[k], e1 = bad ? (uint16_t)0 : src[k + 1u];
    st_agent(a.r0 + p, publishable_pair(e0, e1));
    const uint16_t x0 = f2h(h2f(e0) * r * a.norm0[k]), x1 = f2h(h2f(e1) * r * a.norm0[k + 1u]);
    st_agent(a.x0 + p, publishable_pair(x0, x1));
  }
  lds_barrier();
}

// ---- the last item: argmax_stage2 over the head's tile winners, the control block ----
__device__ __forceinline__ void finish_item(const StepArgs& a, const Stage& st, Lds& L, Waiter& wt) {
  const uint32_t t = opaque_tid();
  const uint32_t groups = st.count ? st.tiles : 0u;  // the head GEMV's tiles
  float bv = -INFINITY;
  uint32_t bi = 0x7FFFFFFFu;
  bool bad = false;  // a tile winner is NaN: the tile held a non-finite logit
  for (uint32_t g0 = 0; g0 < groups; g0 += 2048u) {
    const uint32_t ng = min(2048u, groups - g0);
    poll_lds_n(wt, st.am + 2u * g0, 2u * ng, t * 4u, 1024u, L.words, true);
    lds_barrier();
    for (uint32_t g = t; g < ng; g += 256u) {
      const float v = __builtin_bit_cast(float, L.words[2u * g]);
      const uint32_t ix = L.words[2u * g + 1u];
      bad |= v != v;
      if ((v > bv) || (v == bv && ix < bi)) {
        bv = v;
        bi = ix;
      }
    }
    lds_barrier();
  }
  // the comparator is exact, so any reduction order gives argmax_stage2's winner
  float* sv = L.fold;
  uint32_t* si = L.words;
  sv[t] = bv;
  si[t] = bi;
  lds_barrier();
  for (uint32_t sst = 128; sst > 0; sst >>= 1) {
    if (t < sst) {
      const float ov = sv[t + sst];
      const uint32_t oi = si[t + sst];
      if ((ov > sv[t]) || (ov == sv[t] && oi < si[t])) {
        sv[t] = ov;
        si[t] = oi;
      }
    }
    lds_barrier();
  }
  bad = __syncthreads_or(bad);
  if (t == 0 && bad && a.ctrl[CTRL_DEBUG] == 0u) a.ctrl[CTRL_DEBUG] = kStatusNonFinite;
  if (t == 0) {
    const uint32_t tok = si[0];
    a.ctrl[CTRL_OUT] = tok;
    a.ctrl[CTRL_CUR] = tok;
    const uint32_t step = a.ctrl[CTRL_STEPS];
    if (a.history && step < a.history_len) a.history[step] = tok;
    a.ctrl[CTRL_STEPS] = step + 1u;
    a.ctrl[CTRL_POS] += 1u;
  }
  janitor(st, 0);
  lds_barrier();
}

template <int HD, int GQA>
__global__ __launch_bounds__(256, 2) void step_kernel(StepArgs a, const Stage* __restrict__ stages) {
  __shared__ __align__(16) uint16_t s_xc[kXcHalves];
  __shared__ Lds L;
  const uint32_t t = opaque_tid();
  Waiter wt{__builtin_amdgcn_s_memrealtime() + kTimeoutTicks, a.ctrl + CTRL_DEBUG, false};
  const uint32_t pos = a.ctrl[CTRL_POS];
  if (pos >= a.max_len || a.ctrl[CTRL_NACT] != 1u) {  // nothing to do (the host checks both first)
    if (blockIdx.x == 0 && t == 0 && pos >= a.max_len) a.ctrl[CTRL_DEBUG] = 0xDEAD0002u;
    return;
  }
  if (t == 0) L.misc[1] = a.eps;
  uint32_t xc_stage = 0xFFFFFFFFu, xc_u0 = 0;
  uint32_t si = 0;
  const uint32_t P = gridDim.x;
  // unit ul of stage `sg` -> its first item and item count
  auto unit_items = [](const Stage& sg, uint32_t ul, uint32_t& n) -> uint32_t {
    n = 1u;
    if (sg.kind != SK_SLICE) return ul;
    if (ul < sg.prod_units) {
      const uint32_t s = ul / sg.ups, t0 = (ul - s * sg.ups) * kQuad;
      n = min(kQuad, sg.tiles - t0);
      return s * sg.tiles + t0;
    }
    return sg.prod_items + (ul - sg.prod_units);
  };
  for (uint32_t U = blockIdx.x; U < a.total; U += P) {
    while (U >= stages[si].ufirst + stages[si].units) ++si;
    const Stage& st = stages[si];
    const uint32_t ul = U - st.ufirst;
    uint32_t n = 1;
    const uint32_t i = unit_items(st, ul, n);
    const uint32_t kind = st.kind;
    const uint32_t t_begin = a.trace ? (uint32_t)__builtin_amdgcn_s_memrealtime() : 0u;
    if (kind == SK_SLICE) {
      // the unit's weights go out first, then (at this work-group's first unit of the stage) its
      // inputs are polled into LDS while they are on the way
      SliceWQ W;
      slice_loadq(W, st, i, n);
      const uint32_t span = st.gps * 64u;  // halves of K per slice
      if (xc_stage != si) {
        // the whole input vector, or the K ranges of this work-group's units of the stage (slot
        // k = unit ul + k P; a unit's items share their slice)
        lds_barrier();
        uint32_t* xw = reinterpret_cast<uint32_t*>(s_xc);
        const uint32_t* xs = st.x;
        if (st.xc_whole) {
          poll_lds_n(wt, xs, st.K / 2u, t * 4u, 1024u, xw, false);
        } else {
          const uint32_t slots = (st.units - ul + P - 1u) / P;
          const uint32_t tiles = st.tiles, half = span / 2u;
          for (uint32_t k = 0; k < slots; ++k) {
            uint32_t nk = 1;
            const uint32_t sk = unit_items(st, ul + k * P, nk) / tiles;
            poll_lds<1>(wt, xs + sk * half, half, t * 4u, 0u, xw + k * half, false);
          }
        }
        lds_barrier();
        xc_stage = si;
        xc_u0 = ul;
      }
      const uint32_t s = i / st.tiles;
      const uint16_t* xrow = st.xc_whole ? s_xc + s * span : s_xc + ((ul - xc_u0) / P) * span;
      if (ul >= st.prod_units)
        slice_item(st, i, W.w[0], xrow, L, wt);
      else
        slice_quad(st, i, n, W, xrow, L);
    } else if (kind == SK_HEAD) {
      head_item<HD>(a, st, i, pos, L, wt);
    } else if (kind == SK_ATTN) {
      AttnDecodeArgs ad{};
      ad.ctrl = a.ctrl;
      ad.attn_q = st.attn_q;
      ad.kv_k = st.kv_k;
      ad.kv_v = st.kv_v;
      ad.attn_part = st.attn_part;
      ad.row_stride = HD;
      ad.head_stride = (size_t)a.max_len * HD;
      ad.M = 1;
      ad.q_heads = a.q_heads;
      ad.kv_heads = a.kv_heads;
      ad.tgt = a.tgt;
      ad.kv_len = a.max_len;
      ad.scale = a.scale;
      ad.ps_new = st.newkv;
      attn_block<HD, 0, GQA, false, true>(ad, i / a.tgt, i % a.tgt, 0, &wt);
      lds_barrier();
    } else if (kind == SK_REDUCE) {
      reduce_item<HD>(a, st, i, pos, L, wt);
    } else if (kind == SK_EMBED) {
      embed_item(a, L);
    } else {
      finish_item(a, st, L, wt);
    }
    if (a.trace && t == 0) {
      a.trace[2u * U] = t_begin;
      a.trace[2u * U + 1u] = (uint32_t)__builtin_amdgcn_s_memrealtime();
    }
  }
}

template <int HD, int GQA>
int launch_step(const StepArgs& a, uint32_t wgs, hipStream_t st) {
  step_kernel<HD, GQA><<<wgs, 256, 0, st>>>(a, a.stages);
  return (int)hipGetLastError();
}

template <int HD, int GQA>
int occupancy_of(int* per_cu) {
  return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, step_kernel<HD, GQA>, 256, 0);
}

using LaunchFn = int (*)(const StepArgs&, uint32_t, hipStream_t);
using OccFn = int (*)(int*);

bool pick_kernel(uint32_t HD, uint32_t GQA, LaunchFn* l, OccFn* o) {
#define MI_STEP_CASE(hd, g)           \
  if (HD == hd && GQA == g) {         \
    *l = launch_step<hd, g>;          \
    *o = occupancy_of<hd, g>;         \
    return true;                      \
  }
  MI_STEP_CASE(128, 2) MI_STEP_CASE(128, 4) MI_STEP_CASE(128, 5) MI_STEP_CASE(128, 8)
  MI_STEP_CASE(256, 2) MI_STEP_CASE(256, 4) MI_STEP_CASE(256, 8)
#undef MI_STEP_CASE
  return false;
}

}  // namespace

struct StepPlan {
  StepModel m{};
  std::vector<Stage> stages;
  Stage* d_stages = nullptr;
  uint32_t* arena = nullptr;
  size_t arena_words = 0;
  uint32_t* trace = nullptr;
  StepArgs args{};
  uint32_t wgs = 0;
  LaunchFn launch = nullptr;

  ~StepPlan() {
    if (d_stages) (void)hipFree(d_stages);
    if (arena) (void)hipFree(arena);
    if (trace) (void)hipFree(trace);
  }
};

int step_plan_create(const StepModel& m, hipStream_t st, StepPlan** out) {
  *out = nullptr;
  const uint32_t H = m.hidden, HD = m.head_dim, QH = m.q_heads, KVH = m.kv_heads, I = m.inter;
  if (!KVH || QH % KVH) return mi_fail(MI_ERR_SHAPE, "step: q_heads must be a multiple of kv_heads");
  LaunchFn lf = nullptr;
  OccFn of = nullptr;
  if (!pick_kernel(HD, QH / KVH, &lf, &of))
    return mi_fail(MI_ERR_SHAPE, "step: head_dim 128 (GQA 2/4/5/8) or 256 (GQA 2/4/8) only");
  if (m.tgt == 0 || m.tgt > 64) return mi_fail(MI_ERR_SHAPE, "step: attention blocks per kv head must be <= 64");
  if (H % 512 || (QH * HD) % 512 || I % 64 || m.vocab % 64 || m.rot_dim > HD || m.rot_dim % 2)
    return mi_fail(MI_ERR_SHAPE, "step: unsupported dims");
  auto lin_ok = [&](const StepLinear& l, uint32_t K, uint32_t N) {
    if (l.K != K || l.N != N || !l.S || (K / 64) % l.S) return false;
    const uint32_t gps = K / 64 / l.S;
    return gps >= 1 && gps <= kMaxGps;
  };
  for (uint32_t li = 0; li < m.layers; ++li) {
    const StepLayerW& L = m.layer[li];
    if (!lin_ok(L.qkv, H, (QH + 2 * KVH) * HD) || !lin_ok(L.o, QH * HD, H) || !lin_ok(L.gate_up, H, 2 * I) ||
        !lin_ok(L.down, I, H))
      return mi_fail(MI_ERR_SHAPE, "step: a linear's split-K leaves more than 8 k-groups per slice");
    if (L.qkv.S * HD > 4096 || L.o.S > 65 || L.gate_up.S > 65 || L.down.S > 65)
      return mi_fail(MI_ERR_SHAPE, "step: split-K too wide for the consumers' polls");
  }
  if (!lin_ok(m.lm_head, H, m.vocab) || m.lm_head.S > 65)
    return mi_fail(MI_ERR_SHAPE, "step: the head GEMV's split");
  int per_cu = 0;
  if (of(&per_cu) != 0 || per_cu < 1) return mi_fail(MI_ERR_STATE, "step: occupancy query");
  int dev = 0;
  hipDeviceProp_t prop{};
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return mi_fail(MI_ERR_STATE, "step: device properties");
  uint32_t wgs = (uint32_t)per_cu * (uint32_t)prop.multiProcessorCount;
  if (const char* env = std::getenv("MI_STEP_WGS")) {  // fewer work-groups, for measurements
    const long v = std::strtol(env, nullptr, 10);
    if (v > 0 && (uint32_t)v < wgs) wgs = (uint32_t)v;
  }
  const uint32_t tilesH = H / 64;
  if (wgs < tilesH) return mi_fail(MI_ERR_SHAPE, "step: fewer resident work-groups than hidden / 64");

  std::unique_ptr<StepPlan> p(new (std::nothrow) StepPlan);
  if (!p) return mi_fail(MI_ERR_OOM, "step: host memory");
  p->m = m;
  p->wgs = wgs;
  p->launch = lf;

  // ---- the hand-off arena (word offsets first, then one allocation) ----
  size_t off = 0;
  auto take = [&](size_t words) {
    const size_t o = off;
    off += (words + 63) / 64 * 64;  // 256-byte aligned pieces
    return o;
  };
  const uint32_t qkv_n = (QH + 2 * KVH) * HD;
  struct LayerOff {
    size_t mr, x_in, attn_q, attn_out, x_post, h, mr_words;
    size_t part_qkv, newkv, attn_part, part_o, sumsq_o, part_gu, part_d, sumsq_d;
  };
  std::vector<LayerOff> lo(m.layers);
  std::vector<size_t> r_off(2 * m.layers + 1);
  for (uint32_t k = 0; k < 2 * m.layers; ++k) r_off[k] = take(H / 2);
  for (uint32_t li = 0; li < m.layers; ++li) {
    const StepLayerW& L = m.layer[li];
    LayerOff& o = lo[li];
    o.part_qkv = take((size_t)L.qkv.S * qkv_n);
    o.newkv = take((size_t)KVH * HD);
    o.attn_part = take((size_t)QH * m.tgt * (HD + 2));
    o.part_o = take((size_t)(L.o.S - 1) * H);
    o.sumsq_o = take((size_t)tilesH * tilesH);
    o.part_gu = take((size_t)(L.gate_up.S - 1) * 2 * I);
    o.part_d = take((size_t)(L.down.S - 1) * H);
    o.sumsq_d = take((size_t)tilesH * tilesH);
    // the layer's many-reader words, in one range the next layer's merges empty
    o.mr_words = H / 2 + (size_t)QH * HD + (size_t)QH * HD / 2 + H / 2 + I / 2;
    o.mr = take(o.mr_words);
    o.x_in = o.mr;
    o.attn_q = o.x_in + H / 2;
    o.attn_out = o.attn_q + (size_t)QH * HD;
    o.x_post = o.attn_out + (size_t)QH * HD / 2;
    o.h = o.x_post + H / 2;
  }
  // right after the last layer's many-reader words: the final residual (no reader) and the
  // final norm's output, so the last item empties one contiguous range
  r_off[2 * m.layers] = take(H / 2);
  const size_t x_final = take(H / 2);
  const size_t part_lm = take((size_t)(m.lm_head.S - 1) * m.vocab);
  const size_t am = take((size_t)(m.vocab / 64) * 2);
  p->arena_words = off;
  if (hipMalloc(&p->arena, off * 4) != hipSuccess) return mi_fail(MI_ERR_OOM, "step: hand-off arena");
  if (int e = mi_gemv_handoff_init(reinterpret_cast<float*>(p->arena), off, st)) return e;
  uint32_t* A = p->arena;
  auto W = [&](size_t o) { return A + o; };
  auto F = [&](size_t o) { return reinterpret_cast<float*>(A + o); };

  // ---- the work-item list ----
  std::vector<Stage>& S = p->stages;
  uint32_t first = 0;
  uint32_t ufirst = 0;
  auto add = [&](Stage s) {
    s.first = first;
    first += s.count;
    s.units = s.count;
    if (s.kind == SK_SLICE) {
      // producer items in units of up to kQuad adjacent tiles of one slice (items are
      // slice-major), the consumer slice's items one by one
      s.prod_items = s.epi != SE_NONE ? s.tiles * (s.S - 1) : s.count;
      s.ups = (s.tiles + kQuad - 1) / kQuad;
      s.prod_units = (s.prod_items / s.tiles) * s.ups;
      s.units = s.prod_units + (s.count - s.prod_items);
    }
    s.ufirst = ufirst;
    ufirst += s.units;
    S.push_back(s);
    return &S.back();
  };
  auto slice_stage = [&](const StepLinear& l, const uint32_t* x, float* part, uint32_t epi, uint32_t K) {
    Stage s{};
    s.kind = SK_SLICE;
    s.epi = epi;
    s.qw = l.q;
    s.sc = l.s;
    s.K = K;
    s.N = l.N;
    s.S = l.S;
    s.gps = K / 64 / l.S;
    s.tiles = l.N / 64;
    s.count = s.tiles * l.S;
    s.x = x;
    s.part = part;
    // the work-group's K ranges (one per unit) when they take less LDS than the whole vector
    const uint32_t ups = (s.tiles + kQuad - 1) / kQuad;
    const uint32_t units = epi != SE_NONE ? (l.S - 1) * ups + s.tiles : l.S * ups;
    const size_t ranges = (size_t)((units + wgs - 1) / wgs) * s.gps * 64;
    s.xc_whole = (ranges > kXcHalves || ranges >= K) ? 1u : 0u;
    return s;
  };
  {
    Stage e{};
    e.kind = SK_EMBED;
    e.count = 1;
    add(e);
  }
  for (uint32_t li = 0; li < m.layers; ++li) {
    const StepLayerW& L = m.layer[li];
    const LayerOff& o = lo[li];
    add(slice_stage(L.qkv, W(o.x_in), F(o.part_qkv), SE_NONE, H));
    Stage hd{};
    hd.kind = SK_HEAD;
    hd.count = QH + 2 * KVH;
    hd.part_qkv = F(o.part_qkv);
    hd.S_qkv = L.qkv.S;
    hd.qkv_n = qkv_n;
    hd.q_norm = L.q_norm;
    hd.k_norm = L.k_norm;
    hd.attn_q = F(o.attn_q);
    hd.kv_k = m.kv_k + (size_t)li * KVH * m.max_len * HD;
    hd.kv_v = m.kv_v + (size_t)li * KVH * m.max_len * HD;
    hd.newkv = W(o.newkv);
    add(hd);
    Stage at = hd;
    at.kind = SK_ATTN;
    at.count = KVH * m.tgt;
    at.attn_part = F(o.attn_part);
    add(at);
    Stage rd = at;
    rd.kind = SK_REDUCE;
    rd.count = QH;
    rd.attn_out = W(o.attn_out);
    if (li > 0) {  // the previous layer's many-reader words: all their readers are done here
      rd.jan = W(lo[li - 1].mr);
      rd.jan_words = (uint32_t)lo[li - 1].mr_words;
    }
    add(rd);
    Stage so = slice_stage(L.o, W(o.attn_out), F(o.part_o), SE_RESID, QH * HD);
    so.resid_in = W(r_off[2 * li]);
    so.resid_out = W(r_off[2 * li + 1]);
    so.sumsq = F(o.sumsq_o);
    so.norm_w = L.post_norm;
    so.x_next = W(o.x_post);
    add(so);
    Stage sg = slice_stage(L.gate_up, W(o.x_post), F(o.part_gu), SE_SILU, H);
    sg.h = W(o.h);
    add(sg);
    Stage sd = slice_stage(L.down, W(o.h), F(o.part_d), SE_RESID, I);
    sd.resid_in = W(r_off[2 * li + 1]);
    sd.resid_out = W(r_off[2 * li + 2]);
    sd.sumsq = F(o.sumsq_d);
    const bool last = li + 1 == m.layers;
    sd.norm_w = last ? m.final_norm : m.layer[li + 1].in_norm;
    sd.x_next = last ? W(x_final) : W(lo[li + 1].x_in);
    add(sd);
  }
  Stage lm = slice_stage(m.lm_head, W(x_final), F(part_lm), SE_LOGITS, H);
  lm.logits = m.logits;
  lm.am = W(am);
  lm.vocab_used = m.vocab_used;
  add(lm);
  {
    Stage f{};
    f.kind = SK_FINISH;
    f.count = 1;
    f.tiles = m.vocab / 64;
    f.am = W(am);
    // the last layer's many-reader words, the final residual and the final norm's output
    // (contiguous): their readers are done once the head's consumers are
    const LayerOff& o = lo[m.layers - 1];
    f.jan = W(o.mr);
    f.jan_words = (uint32_t)(x_final + H / 2 - o.mr);
    add(f);
  }
  for (const Stage& x : S)
    if (x.kind == SK_SLICE && x.xc_whole && x.K > kXcHalves)
      return mi_fail(MI_ERR_SHAPE, "step: a slice stage's inputs do not fit the activation cache");
  if (hipMalloc(&p->d_stages, S.size() * sizeof(Stage)) != hipSuccess) return mi_fail(MI_ERR_OOM, "step: stage table");
  if (hipMemcpy(p->d_stages, S.data(), S.size() * sizeof(Stage), hipMemcpyHostToDevice) != hipSuccess)
    return mi_fail(MI_ERR_STATE, "step: stage table upload");

  StepArgs& a = p->args;
  a.stages = p->d_stages;
  a.total = ufirst;
  if (std::getenv("MI_STEP_TRACE")) {  // diagnostics: item start/end times, [items][2] u32
    if (hipMalloc(&p->trace, (size_t)ufirst * 8) != hipSuccess) return mi_fail(MI_ERR_OOM, "step: trace");
    a.trace = p->trace;
    for (const Stage& x : S)  // the unit ranges the trace is read against
      std::fprintf(stderr, "step-stage kind %u epi %u ufirst %u units %u prod_units %u\n", x.kind, x.epi, x.ufirst,
                   x.units, x.prod_units);
  }
  if (const char* env = std::getenv("MI_STEP_STOP")) {  // diagnostics: only the first n stages run
    const long n = std::strtol(env, nullptr, 10);
    if (n > 0 && (size_t)n < S.size()) a.total = S[n].ufirst;
  }
  a.ctrl = m.ctrl;
  a.history = m.history;
  a.history_len = m.max_len;
  a.embed = m.embed;
  a.norm0 = m.layer[0].in_norm;
  a.r0 = W(r_off[0]);
  a.x0 = W(lo[0].x_in);
  a.rope = m.rope;
  a.hidden = H;
  a.vocab = m.vocab;
  a.q_heads = QH;
  a.kv_heads = KVH;
  a.rot_dim = m.rot_dim;
  a.max_len = m.max_len;
  a.tgt = m.tgt;
  a.eps = m.eps;
  a.scale = float(1.0 / std::sqrt(double(HD)));
  if (hipStreamSynchronize(st) != hipSuccess) return mi_fail(MI_ERR_STATE, "step: init");
  *out = p.release();
  return 0;
}

int step_plan_launch(StepPlan* p, hipStream_t st) {
  return mi_hip(p->launch(p->args, p->wgs, st), "step launch");
}

int step_plan_reset(StepPlan* p, hipStream_t st) {
  return mi_gemv_handoff_init(reinterpret_cast<float*>(p->arena), p->arena_words, st);
}

void step_plan_destroy(StepPlan* p) { delete p; }

uint32_t step_plan_wgs(const StepPlan* p) { return p ? p->wgs : 0u; }
uint32_t step_plan_items(const StepPlan* p) { return p ? p->args.total : 0u; }

void step_plan_debug(const StepPlan* p, uint32_t what, void** ptr, size_t* bytes) {
  *ptr = nullptr;
  *bytes = 0;
  if (!p) return;
  if (what == 0) {
    *ptr = p->d_stages;
    *bytes = p->stages.size() * sizeof(Stage);
  } else if (what == 1) {
    *ptr = p->arena;
    *bytes = p->arena_words * 4;
  } else {
    *ptr = p->trace;
    *bytes = p->trace ? (size_t)p->args.total * 8 : 0;
  }
}

}  // namespace mi
