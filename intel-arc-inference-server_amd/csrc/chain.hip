// chain.hip - the GEMV chain of one dense layer as one launch (the interface is chain.h).
//
// The reference records a layer's linears and the kernels between them as separate launches
// (src/runtime/capture.cc: mlp :1247, res_norm :997, fa_layer's attn_prep :1370). On MI355X each
// dependent launch pays a ramp, a tail and a trip through the command processor, and a launch of
// the 27B's o (14 MB) or q||k||v (20 MB) streams for only a few microseconds. Here the layer's
// o GEMV with the residual fold and the post-attention norm, gate||up with SwiGLU, down with the
// residual fold and the next RMSNorm, and (when a layer follows) that layer's q||k||v with
// attn_prep run as ONE launch: a work-group that has finished its o tiles already streams its
// gate||up weights while the norm is formed, and so on down the chain.
//
//   * Items. The launch is a list of items in dependency order, stage by stage: per linear the
//     (64-column tile, split-K slice) products, slice-major like the GEMV launch's grid, then
//     the tiles' consumers (RESID: the residual fold, the tiles' sum-of-squares exchange and the
//     next norm; SILU: SwiGLU), or per head the q||k||v consumer (attn_prep's chain). Work-group
//     w takes items w, w + P, w + 2P, ... with P = the work-groups resident at once; an item
//     waits only for earlier items or, for a RESID consumer, for its stage's other consumers,
//     all of which sit on other work-groups (P exceeds a stage's consumer count) whose earlier
//     items never wait on a later stage. So the launch cannot deadlock while all P are resident
//     (the engine launches exactly as many as fit).
//   * Hand-off words (gemv_core.h's empty pattern): a value one item hands to another is stored
//     device-coherent into words that hold the empty pattern until then; the reader polls until
//     they are not. A word with one reader (partials, the residual between o and down, a
//     consumer's copy of the tile sums) is emptied again by it. The many-reader words (the
//     normed x, SwiGLU's h) come in two sets used by alternate layers: each launch empties the
//     set the previous launch used, after which every reader of it has finished.
//   * Inputs from earlier launches (the attention output, the residual at the layer's start) and
//     outputs for later ones (the residual, the final norm's x, q, the K/V rows) are plain
//     memory: the launch boundary orders them.
//   * Bounded waits: a poll gives up after `poll_limit` rounds, takes what it finds and sets
//     the status word to MI_STATUS_HANDOFF_TIMEOUT, so a broken launch ends instead of hanging.
// Every arithmetic operation is the graph path's (gemv_w4a16.hip's producers and its RESID,
// SILU and QKV consumers), in the same order: the step's logits, KV rows and control block are
// bitwise those of the launch-per-linear graph.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <new>
#include <vector>

#include "mi_capi_internal.h"
#include "mi_common.h"
#include "gemv_core.h"
#include "chain.h"

namespace mi {
namespace {

enum : uint32_t { CS_SLICE = 0, CS_RESID = 1, CS_SILU = 2, CS_HEAD = 3 };
constexpr uint32_t kFoldWords = 2304;  // a consumer's polled partials: S * 64 (S <= 36), or S * HD (heads)

struct ChainStage {
  uint32_t kind, first, count;
  uint32_t items;  // SLICE: product items
  // the linear this stage produces (SLICE) or consumes (RESID / SILU / HEAD)
  const uint32_t* qw;
  const uint16_t* sc;
  uint32_t K, N, S, gps, tiles;
  const uint16_t* x_plain;  // SLICE input from an earlier launch, f16 [K]
  const uint32_t* x_words;  // or hand-off words, f16 pairs [K / 2]
  // or (n_sums set) x is the RMSNorm of a residual handed over as words (x_words: residual
  // pairs [K / 2]) with its per-tile sums of squares n_sums [K / 64] and weights n_w [K]
  const float* n_sums;
  const float* n_w;
  float* part;              // [S][N] hand-off partials
  // RESID
  const uint16_t* r_in_plain;  // the residual in (one of the two)
  uint32_t* r_in_words;
  uint32_t r_in_take;          // r_in_words has this consumer as its only reader
  float* sum_pub;              // set: publish the tile's sum of squares here [tiles] and stop
                               // (the next linear's slices form the norm); else the full norm
  uint16_t* r_out_plain;       // the residual out (either or both)
  uint32_t* r_out_words;
  float* sumsq;                // [tiles][tiles], consumer c's copy at row c
  const float* norm_w;         // the next RMSNorm's weights [N]
  uint16_t* x_out_plain;       // the next norm's x (either or both)
  uint32_t* x_out_words;
  // SILU
  uint32_t* h_words;           // [N / 4]
  // HEAD (attn_prep on the folded q||k||v, M = 1, f16-format cache [kv_heads][max_len][HD])
  const float* q_norm;
  const float* k_norm;
  float* attn_q;
  uint16_t* kv_k;
  uint16_t* kv_v;
};

struct ChainArgs {
  const ChainStage* stages;
  uint32_t nstages, total;
  uint32_t* ctrl;
  uint32_t* status;
  uint32_t poll_limit;
  uint32_t act;
  float eps, qk_eps;
  const float* rope;
  uint32_t q_heads, kv_heads, head_dim, rot_dim, max_len;
  uint32_t* jan;  // the other set's many-reader words, emptied by this launch
  uint32_t jan_words;
  uint32_t* trace;  // diagnostics (NULL normally): per item its start and end (s_memrealtime)
};

struct Lds {
  uint32_t xw[256];            // a slice's input, f16 pairs (<= 8 k-groups)
  float red[4][64];
  uint32_t words[kFoldWords];  // polled words
  uint32_t rw[32];             // a RESID consumer's residual tile (f16 pairs)
  float rowv[256];
  float nrm[256];
  float misc[4];
};

// Thread t polls the words of elements e = t + 256 u < n (u < PER) into dst[e]: element e's word
// at byte offset voff + u * ustride from base. All loads go out together, the still-empty words
// are polled again together; `take`: each word is emptied again after it is read (one reader).
template <int PER>
__device__ __forceinline__ void poll_lds(const ChainArgs& a, const void* base, uint32_t n, uint32_t voff,
                                         uint32_t ustride, uint32_t* dst, bool take) {
  constexpr int kSc1 = 16;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFFF, 0x00020000);
  const uint32_t t = threadIdx.x;
  uint32_t v[PER];
  uint32_t pending = 0;
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (t + 256u * u < n) v[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, u * ustride, kSc1);
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (t + 256u * u < n && v[u] == kEmpty) pending |= 1u << u;
  for (uint32_t r = 0; pending && r < a.poll_limit; ++r) {
    // a wait that has gone on for a while gives up at once when any wait of the step already
    // has (the status word), so a broken step ends after one time-out, not one per wait
    if ((r & 1023u) == 1023u && a.status && ld_agent(a.status) == kStatusTimeout) break;
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if (pending & (1u << u)) v[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, u * ustride, kSc1);
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if ((pending & (1u << u)) && v[u] != kEmpty) pending &= ~(1u << u);
  }
  if (pending && a.status) st_agent(a.status, kStatusTimeout);
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (t + 256u * u < n) {
      dst[t + 256u * u] = v[u];
      if (take) __builtin_amdgcn_raw_buffer_store_b32(kEmpty, rs, voff, u * ustride, kSc1);
    }
}

// poll_lds over up to kFoldWords elements in rounds of 2048 (element e = 2048 r + t + 256 u at
// byte offset voff + (8 r + u) * ustride)
__device__ __forceinline__ void poll_lds_n(const ChainArgs& a, const void* base, uint32_t n, uint32_t voff,
                                           uint32_t ustride, uint32_t* dst, bool take) {
  for (uint32_t r0 = 0; r0 < n; r0 += 2048u)
    poll_lds<8>(a, static_cast<const unsigned char*>(base) + (size_t)(r0 / 256u) * ustride, n - r0, voff, ustride,
                dst + r0, take);
}

// ---- a product item: one tile of one slice (gemv_w4a16_kernel<1, 2, EPI> at M = 1) ----
// Wave w takes the slice's k-groups w and w + 4; each an MFMA batch scaled per column, summed
// in group order; the waves' sums added in wave order: the launch kernel's slice partial.
__device__ __forceinline__ void slice_item(const ChainArgs& a, const ChainStage& st, uint32_t u, Lds& L, uint32_t si,
                                           uint32_t& inv_for) {
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6, c4 = lane & 15u, q = lane >> 4;
  const uint32_t tiles = st.tiles, N = st.N, gps = st.gps, act = a.act;
  const uint32_t s = u / tiles, tile = u - s * tiles, n0 = tile * 64u, ncol = n0 + 4u * c4;
  // the weights first (they do not depend on anything), then the input; every load goes out
  // unconditionally (a wave with no second group re-reads its first) so none waits for a branch
  u4_t wv[2][2];
  u2_t sv[2];
#pragma unroll
  for (uint32_t k = 0; k < 2; ++k) {
    const uint32_t gl = wave + 4u * k;
    const uint32_t g = s * gps + (gl < gps ? gl : wave % gps);
#pragma unroll
    for (uint32_t h = 0; h < 2; ++h) wv[k][h] = load_stream16(st.qw + (size_t)(g * 8u + 4u * h + q) * N + ncol);
    sv[k] = *as_global(reinterpret_cast<const u2_t*>(st.sc + (size_t)g * N + ncol));
  }
  const uint32_t nw = gps * 32u;  // the slice's input words
  if (st.n_sums) {
    // x = RMSNorm(residual) formed here, as the norm's consumer forms it: the tile sums added
    // in tile order from +0 (once per stage and work-group), then (v * inv) * w per element
    float w0 = 0.f, w1 = 0.f;
    if (t < nw) {
      w0 = st.n_w[2u * (s * nw + t)];
      w1 = st.n_w[2u * (s * nw + t) + 1u];
    }
    poll_lds<1>(a, st.x_words + s * nw, nw, t * 4u, 0u, L.xw, false);
    if (inv_for != si) {
      const uint32_t nt = st.K / 64u;
      poll_lds<1>(a, st.n_sums, nt, t * 4u, 0u, L.words, false);
      lds_barrier();
      if (t == 0) {
        float tot = 0.f;
        for (uint32_t g = 0; g < nt; ++g) tot += __builtin_bit_cast(float, L.words[g]);
        L.misc[1] = 1.0f / sqrtf(tot / (float)st.K + a.eps);
      }
      inv_for = si;
    }
    lds_barrier();
    if (t < nw) {
      const float inv = L.misc[1];
      const uint32_t rw = L.xw[t];
      const uint16_t x0 = act_enc(res_widen((uint16_t)(rw & 0xFFFFu), act) * inv * w0, act);
      const uint16_t x1 = act_enc(res_widen((uint16_t)(rw >> 16), act) * inv * w1, act);
      L.xw[t] = publishable_pair(x0, x1);
    }
  } else if (st.x_words) {
    poll_lds<1>(a, st.x_words + s * nw, nw, t * 4u, 0u, L.xw, false);
  } else if (t < nw) {
    L.xw[t] = *as_global(reinterpret_cast<const uint32_t*>(st.x_plain) + s * nw + t);
  }
  lds_barrier();
  const uint16_t* xrow = reinterpret_cast<const uint16_t*>(L.xw);
  const uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u, magic = 0x64006400u;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (uint32_t k = 0; k < 2; ++k) {
    const uint32_t gl = wave + 4u * k;
    if (gl < gps) {
      f4_t d[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) d[c] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const u4_t xv = c4 == 0 ? *reinterpret_cast<const u4_t*>(xrow + gl * 64u + 32u * h + 8u * q)
                                : u4_t{0u, 0u, 0u, 0u};
        const h8_t av = perm_x(xv);
        const uint32_t ws[4] = {wv[k][h].x, wv[k][h].y, wv[k][h].z, wv[k][h].w};
        h8_t bw[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) bw[c] = dequant_word(ws[c], m_lo, m_hi, magic);
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bw[c], d[c], 0, 0, 0);
        keep_mfma_batch(av, bw, d);
      }
      const float sc[4] = {h2f((uint16_t)(sv[k].x & 0xFFFFu)), h2f((uint16_t)(sv[k].x >> 16)),
                           h2f((uint16_t)(sv[k].y & 0xFFFFu)), h2f((uint16_t)(sv[k].y >> 16))};
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = __builtin_fmaf(d[c][0], sc[c], acc[c]);
    }
  }
  if (q == 0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) L.red[wave][4u * c4 + c] = acc[c];
  }
  lds_barrier();
  if (t < 64u) {
    float v = L.red[0][t];
#pragma unroll
    for (int w = 1; w < 4; ++w) v += L.red[w][t];
    st_agent(st.part + (size_t)s * N + n0 + t, publishable(v));
  }
  lds_barrier();  // L.red and L.xw are reused by the next item
}

// the tile's fold: sum over all S slices in ascending s from +0 (the launch consumer's order:
// its own slice S-1 is the last term) into L.rowv[0..64)
__device__ __forceinline__ void fold_tile(const ChainArgs& a, const ChainStage& st, uint32_t tile, Lds& L) {
  const uint32_t t = threadIdx.x, N = st.N, S = st.S;
  poll_lds_n(a, st.part, S * 64u, ((t >> 6) * N + tile * 64u + (t & 63u)) * 4u, 4u * N * 4u, L.words, true);
  lds_barrier();
  if (t < 64u) {
    float v = 0.f;
    for (uint32_t j = 0; j < S; ++j) v += __builtin_bit_cast(float, L.words[j * 64u + t]);
    L.rowv[t] = v;
  }
  lds_barrier();
}

// ---- RESID consumer: the residual fold, the tiles' sums of squares, the next norm ----
__device__ __forceinline__ void resid_item(const ChainArgs& a, const ChainStage& st, uint32_t tile, Lds& L) {
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t N = st.N, tiles = st.tiles, n0 = tile * 64u, act = a.act;
  uint16_t r_pre = 0;
  float w_pre = 0.f;
  if (wave == 0) {  // the residual (plain input) and the norm weight go out before the fold
    if (!st.r_in_words) r_pre = st.r_in_plain[n0 + lane];
    if (!st.sum_pub) w_pre = st.norm_w[n0 + lane];  // (no norm here in the publishing form)
  }
  if (st.r_in_words) poll_lds<1>(a, st.r_in_words + tile * 32u, 32u, t * 4u, 0u, L.rw, st.r_in_take != 0);
  fold_tile(a, st, tile, L);
  if (wave == 0) {
    if (st.r_in_words) {
      const uint32_t rw = L.rw[lane / 2u];
      r_pre = (uint16_t)((lane & 1u) ? (rw >> 16) : (rw & 0xFFFFu));
    }
    const uint16_t rb = res_rne(res_widen(r_pre, act) + act_round(L.rowv[lane], act), act);
    if (st.r_out_plain) st.r_out_plain[n0 + lane] = rb;
    const uint16_t rb_up = (uint16_t)__shfl((int)rb, (int)(lane + 1u), 64);
    if (st.r_out_words && !(lane & 1u)) st_agent(st.r_out_words + tile * 32u + lane / 2u, publishable_pair(rb, rb_up));
    const float v = res_widen(rb, act);
    L.nrm[lane] = v;
    float s2 = __builtin_fmaf(v, v, 0.f);
#pragma unroll
    for (int sst = 32; sst > 0; sst >>= 1) s2 += __shfl_down(s2, sst, 64);
    s2 = publishable(__shfl(s2, 0, 64));
    if (st.sum_pub) {
      if (lane == 0) st_agent(st.sum_pub + tile, s2);
    } else {
      for (uint32_t c = lane; c < tiles; c += 64u) st_agent(st.sumsq + (size_t)c * tiles + tile, s2);
    }
  }
  if (st.sum_pub) {  // the next linear's slices form the norm from the residual and the sums
    lds_barrier();
    return;
  }
  // every tile's sum (this consumer's copy), added in ascending tile order
  poll_lds<1>(a, st.sumsq + (size_t)tile * tiles, tiles, t * 4u, 0u, L.words, true);
  lds_barrier();
  if (t == 0) {
    float tot = 0.f;
    for (uint32_t g = 0; g < tiles; ++g) tot += __builtin_bit_cast(float, L.words[g]);
    L.misc[0] = 1.0f / sqrtf(tot / (float)N + a.eps);
  }
  lds_barrier();
  if (wave == 0) {
    const uint16_t xb = act_enc(L.nrm[lane] * L.misc[0] * w_pre, act);
    if (st.x_out_plain) st.x_out_plain[n0 + lane] = xb;
    const uint16_t xb_up = (uint16_t)__shfl((int)xb, (int)(lane + 1u), 64);
    if (st.x_out_words && !(lane & 1u)) st_agent(st.x_out_words + tile * 32u + lane / 2u, publishable_pair(xb, xb_up));
  }
  lds_barrier();
}

// ---- SILU consumer: 64 interleave16 columns = 32 outputs (gate at gcol, up at gcol + 16) ----
__device__ __forceinline__ void silu_item(const ChainArgs& a, const ChainStage& st, uint32_t tile, Lds& L) {
  const uint32_t t = threadIdx.x, act = a.act;
  fold_tile(a, st, tile, L);
  if (t < 16u) {
    uint16_t o[2];
#pragma unroll
    for (uint32_t k2 = 0; k2 < 2; ++k2) {
      const uint32_t kk = 2u * t + k2, gcol = (kk / 16u) * 32u + (kk % 16u);
      const float g_r = act_round(L.rowv[gcol], act), u_r = act_round(L.rowv[gcol + 16u], act);
      const float s_r = act_round(silu_f32(g_r), act);
      o[k2] = act_enc(s_r * u_r, act);
    }
    st_agent(st.h_words + tile * 16u + t, publishable_pair(o[0], o[1]));
  }
  lds_barrier();
}

// ---- HEAD consumer: attn_prep's chain on one head of the folded q||k||v row (the launch
// kernel's qkv_consumer at M = 1): q -> attn_q, K / V -> the cache row of position pos ----
template <int HD>
__device__ __forceinline__ void head_item(const ChainArgs& a, const ChainStage& st, uint32_t hh, Lds& L) {
  constexpr uint32_t EPL = HD / 64u;
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6, act = a.act;
  const uint32_t QH = a.q_heads, KVH = a.kv_heads, N = st.N, S = st.S;
  const bool is_q = hh < QH, is_k = !is_q && hh < QH + KVH;
  const uint32_t h = is_q ? hh : (is_k ? hh - QH : hh - QH - KVH);
  const uint32_t nh0 = hh * HD;
  const uint32_t pos = a.ctrl[CTRL_POS];
  const bool past = pos >= a.max_len;
  const float* nw = is_q ? st.q_norm : (is_k ? st.k_norm : nullptr);
  const uint32_t half = a.rot_dim / 2u;
  float wn[EPL], rc[EPL], rsn[EPL];
  if (wave == 0 && !past) {
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
  poll_lds_n(a, st.part, S * HD, ((t / HD) * N + nh0 + t % HD) * 4u, (256u / HD) * N * 4u, L.words, true);
  lds_barrier();
  if (t < HD) {
    float acc = 0.f;
    for (uint32_t j = 0; j < S; ++j) acc += __builtin_bit_cast(float, L.words[j * HD + t]);
    L.rowv[t] = acc;
  }
  lds_barrier();
  if (wave == 0) {
    if (past) {  // past the cache: write nothing, flag the step (attn_prep's rule)
      if (hh == 0 && lane == 0) a.ctrl[CTRL_DEBUG] = 0xDEAD0002u;
    } else {
      const size_t crow = (size_t)h * a.max_len * HD + (size_t)pos * HD;  // row pos of kv head h
      if (!is_q && !is_k) {
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) st.kv_v[crow + lane + 64u * k] = act_enc(L.rowv[lane + 64u * k], act);
      } else {
        float xf[EPL], nv[EPL];
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) xf[k] = act_round(L.rowv[lane + 64u * k], act);
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
          const float rstd = 1.0f / sqrtf(tot / (float)HD + a.qk_eps);
#pragma unroll
          for (uint32_t k = 0; k < EPL; ++k) nv[k] = act_round(xf[k] * rstd * wn[k], act);
        } else {
#pragma unroll
          for (uint32_t k = 0; k < EPL; ++k) nv[k] = xf[k];
        }
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) L.nrm[lane + 64u * k] = nv[k];
        wave_lds_sync();
#pragma unroll
        for (uint32_t k = 0; k < EPL; ++k) {
          const uint32_t e = lane + 64u * k;
          float out;
          if (e < half) {
            const float tt = L.nrm[e + half] * rsn[k];
            out = __builtin_fmaf(nv[k], rc[k], -tt);
          } else if (e < a.rot_dim) {
            const float tt = L.nrm[e - half] * rsn[k];
            out = __builtin_fmaf(nv[k], rc[k], tt);
          } else {
            out = nv[k];
          }
          if (is_q) st.attn_q[(size_t)h * HD + e] = out;
          else st.kv_k[crow + e] = act_enc(out, act);
        }
      }
    }
  }
  lds_barrier();
}

template <int HD>
__global__ __launch_bounds__(256, 4) void chain_kernel(ChainArgs a, const ChainStage* __restrict__ stages) {
  __shared__ Lds L;
  // the set of many-reader words the previous launch used: every reader of it has finished
  for (uint32_t k = blockIdx.x * 256u + threadIdx.x; k < a.jan_words; k += gridDim.x * 256u) st_agent(a.jan + k, kEmpty);
  uint32_t si = 0, inv_for = ~0u;
  for (uint32_t i = blockIdx.x; i < a.total; i += gridDim.x) {
    // the stage table as its own __restrict__ parameter: scalar loads into SGPRs (a vector load
    // of the fields would put a dependent memory round trip in front of every item)
    while (i >= stages[si].first + stages[si].count) ++si;
    const ChainStage& st = stages[si];
    const uint32_t u = i - st.first;
    const uint32_t t0 = a.trace ? (uint32_t)__builtin_amdgcn_s_memrealtime() : 0u;
    switch (st.kind) {
      case CS_SLICE: slice_item(a, st, u, L, si, inv_for); break;
      case CS_RESID: resid_item(a, st, u, L); break;
      case CS_SILU: silu_item(a, st, u, L); break;
      default: head_item<HD>(a, st, u, L); break;
    }
    if (a.trace && threadIdx.x == 0) {
      a.trace[2u * i] = t0;
      a.trace[2u * i + 1u] = (uint32_t)__builtin_amdgcn_s_memrealtime();
    }
  }
}

template <int HD>
int occupancy(int* per_cu) {
  return (int)hipOccupancyMaxActiveBlocksPerMultiprocessor(per_cu, chain_kernel<HD>, 256, 0);
}

}  // namespace

struct ChainPlan {
  ChainModel m{};
  uint32_t wgs = 0;
  std::vector<ChainArgs> args;  // one per layer
  size_t set_begin[2] = {0, 0}, set_end[2] = {0, 0};  // the two sets of many-reader words
  ChainStage* d_stages = nullptr;
  uint32_t* arena = nullptr;
  size_t arena_words = 0;
  uint32_t* trace = nullptr;
  ~ChainPlan() {
    if (trace) (void)hipFree(trace);
    if (d_stages) (void)hipFree(d_stages);
    if (arena) (void)hipFree(arena);
  }
};

int chain_plan_create(const ChainModel& m, hipStream_t st, ChainPlan** out) {
  *out = nullptr;
  const uint32_t H = m.hidden, HD = m.head_dim, QH = m.q_heads, KVH = m.kv_heads, I = m.inter;
  if (HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "chain: head_dim 128 or 256");
  if (!KVH || QH % KVH || H % 64 || I % 32 || H > 16384 || m.rot_dim > HD || m.rot_dim % 2)
    return mi_fail(MI_ERR_SHAPE, "chain: unsupported dims");
  const uint32_t qkv_n = (QH + 2 * KVH) * HD;
  auto lin_ok = [](const ChainLinear& l, uint32_t K, uint32_t N) {
    if (l.K != K || l.N != N || !l.S || (K / 64) % l.S) return false;
    const uint32_t gps = K / 64 / l.S;
    return gps >= 1 && gps <= 8 && l.S * 64u <= kFoldWords;
  };
  for (uint32_t li = 0; li < m.layers; ++li) {
    const ChainLayer& L = m.layer[li];
    if (!lin_ok(L.qkv, H, qkv_n) || !lin_ok(L.o, QH * HD, H) || !lin_ok(L.gate_up, H, 2 * I) || !lin_ok(L.down, I, H))
      return mi_fail(MI_ERR_SHAPE, "chain: a linear's split leaves more than 8 k-groups per slice");
    if (L.qkv.S * HD > kFoldWords) return mi_fail(MI_ERR_SHAPE, "chain: q||k||v split too wide for a head's fold");
  }
  int per_cu = 0;
  if ((HD == 128 ? occupancy<128>(&per_cu) : occupancy<256>(&per_cu)) != 0 || per_cu < 1)
    return mi_fail(MI_ERR_STATE, "chain: occupancy query");
  int dev = 0;
  hipDeviceProp_t prop{};
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return mi_fail(MI_ERR_STATE, "chain: device properties");
  const uint32_t wgs = (uint32_t)per_cu * (uint32_t)prop.multiProcessorCount;
  if (wgs < H / 64 + 1) return mi_fail(MI_ERR_SHAPE, "chain: fewer resident work-groups than the tiles of a norm");

  std::unique_ptr<ChainPlan> p(new (std::nothrow) ChainPlan);
  if (!p) return mi_fail(MI_ERR_OOM, "chain: host memory");
  p->m = m;
  p->wgs = wgs;

  // ---- hand-off words: per set (alternate layers) the many-reader words, first; then the
  // single-reader words (partials, tile sums, the residual between o and down), shared ----
  size_t off = 0;
  auto take = [&](size_t words) {
    const size_t o = off;
    off += (words + 63) / 64 * 64;
    return o;
  };
  const uint32_t tilesH = H / 64;
  // per set: the residual after o and its tile sums (read by gate||up's slices and down's
  // consumers), SwiGLU's h, the residual after down and its sums (the next q||k||v's slices)
  size_t r_post[2], s_post[2], hw[2], r_next[2], s_next[2], set_begin[2], set_end[2];
  for (int k = 0; k < 2; ++k) {
    set_begin[k] = off;
    r_post[k] = take(H / 2);
    s_post[k] = take(tilesH);
    hw[k] = take(I / 2);
    r_next[k] = take(H / 2);
    s_next[k] = take(tilesH);
    set_end[k] = off;
  }
  uint32_t So = 0, Sg = 0, Sd = 0, Sq = 0;
  for (uint32_t li = 0; li < m.layers; ++li) {
    So = std::max(So, m.layer[li].o.S);
    Sg = std::max(Sg, m.layer[li].gate_up.S);
    Sd = std::max(Sd, m.layer[li].down.S);
    Sq = std::max(Sq, m.layer[li].qkv.S);
  }
  const size_t part_o = take((size_t)So * H), part_g = take((size_t)Sg * 2 * I), part_d = take((size_t)Sd * H);
  const size_t part_q = take((size_t)Sq * qkv_n);
  const size_t sum_d = take((size_t)tilesH * tilesH);  // the last layer's final norm (all-to-all sums)
  p->arena_words = off;
  if (hipMalloc(&p->arena, off * 4) != hipSuccess) return mi_fail(MI_ERR_OOM, "chain: hand-off words");
  if (int e = mi_gemv_handoff_init(reinterpret_cast<float*>(p->arena), off, st)) return e;
  uint32_t* A = p->arena;
  auto W = [&](size_t o) { return A + o; };
  auto F = [&](size_t o) { return reinterpret_cast<float*>(A + o); };

  // ---- the stage lists, layer by layer ----
  std::vector<ChainStage> all;
  std::vector<size_t> layer_first(m.layers), layer_n(m.layers);
  for (uint32_t li = 0; li < m.layers; ++li) {
    const ChainLayer& L = m.layer[li];
    const int k = (int)(li & 1u);
    const bool last = li + 1 == m.layers;
    layer_first[li] = all.size();
    uint32_t first = 0;
    auto add = [&](ChainStage s) {
      s.first = first;
      first += s.count;
      all.push_back(s);
    };
    auto slice = [&](const ChainLinear& l, const uint16_t* xp, const uint32_t* xw, float* part) {
      ChainStage s{};
      s.kind = CS_SLICE;
      s.qw = l.q;
      s.sc = l.s;
      s.K = l.K;
      s.N = l.N;
      s.S = l.S;
      s.gps = l.K / 64 / l.S;
      s.tiles = l.N / 64;
      s.items = s.tiles * l.S;
      s.count = s.items;
      s.x_plain = xp;
      s.x_words = xw;
      s.part = part;
      return s;
    };
    // o, then its consumers: the residual (plain in, words out) and its tile sums
    add(slice(L.o, m.attn_out, nullptr, F(part_o)));
    ChainStage ro = all.back();
    ro.kind = CS_RESID;
    ro.count = tilesH;
    ro.r_in_plain = m.resid;
    ro.r_out_words = W(r_post[k]);
    ro.sum_pub = F(s_post[k]);
    add(ro);
    // gate||up on the post-attention norm of that residual, formed by its slices
    ChainStage gu = slice(L.gate_up, nullptr, W(r_post[k]), F(part_g));
    gu.n_sums = F(s_post[k]);
    gu.n_w = L.post_norm;
    add(gu);
    ChainStage sg = all.back();
    sg.kind = CS_SILU;
    sg.count = (2 * I) / 64;
    sg.n_sums = nullptr;
    sg.h_words = W(hw[k]);
    add(sg);
    add(slice(L.down, nullptr, W(hw[k]), F(part_d)));
    ChainStage rd = all.back();
    rd.kind = CS_RESID;
    rd.count = tilesH;
    rd.r_in_words = W(r_post[k]);
    rd.r_in_take = 0;
    rd.r_out_plain = m.resid;
    if (last) {  // the final norm, whole, for the head's launch
      rd.sumsq = F(sum_d);
      rd.norm_w = m.final_norm;
      rd.x_out_plain = m.x;
    } else {
      rd.r_out_words = W(r_next[k]);
      rd.sum_pub = F(s_next[k]);
    }
    add(rd);
    if (!last) {  // the next layer's q||k||v and attn_prep
      const ChainLayer& N1 = m.layer[li + 1];
      ChainStage qs = slice(N1.qkv, nullptr, W(r_next[k]), F(part_q));
      qs.n_sums = F(s_next[k]);
      qs.n_w = N1.in_norm;
      add(qs);
      ChainStage hq = all.back();
      hq.n_sums = nullptr;
      hq.kind = CS_HEAD;
      hq.count = QH + 2 * KVH;
      hq.q_norm = N1.q_norm;
      hq.k_norm = N1.k_norm;
      hq.attn_q = m.attn_q;
      hq.kv_k = m.kv_k + (size_t)(li + 1) * KVH * m.max_len * HD;
      hq.kv_v = m.kv_v + (size_t)(li + 1) * KVH * m.max_len * HD;
      add(hq);
    }
    layer_n[li] = all.size() - layer_first[li];
    ChainArgs a{};
    a.nstages = (uint32_t)layer_n[li];
    a.total = first;
    a.ctrl = m.ctrl;
    a.status = m.status;
    a.poll_limit = 1u << 20;
    a.act = m.act;
    a.eps = m.eps;
    a.qk_eps = m.eps;
    a.rope = m.rope;
    a.q_heads = QH;
    a.kv_heads = KVH;
    a.head_dim = HD;
    a.rot_dim = m.rot_dim;
    a.max_len = m.max_len;
    // the set the previous launch of this step used (the previous step's last set is emptied by
    // chain_finish, in its step)
    const int other = 1 - k;
    a.jan = li ? W(set_begin[other]) : nullptr;
    a.jan_words = li ? (uint32_t)(set_end[other] - set_begin[other]) : 0u;
    p->args.push_back(a);
  }
  if (hipMalloc(&p->d_stages, all.size() * sizeof(ChainStage)) != hipSuccess) return mi_fail(MI_ERR_OOM, "chain: stages");
  if (hipMemcpy(p->d_stages, all.data(), all.size() * sizeof(ChainStage), hipMemcpyHostToDevice) != hipSuccess)
    return mi_fail(MI_ERR_STATE, "chain: stage upload");
  for (uint32_t li = 0; li < m.layers; ++li) p->args[li].stages = p->d_stages + layer_first[li];
  if (std::getenv("MI_CHAIN_TRACE")) {  // diagnostics: every layer's items' start / end, [layer][item][2]
    uint32_t mx = 0;
    for (const ChainArgs& a : p->args) mx = std::max(mx, a.total);
    if (hipMalloc(&p->trace, (size_t)m.layers * mx * 8) != hipSuccess) return mi_fail(MI_ERR_OOM, "chain: trace");
    for (uint32_t li = 0; li < m.layers; ++li) p->args[li].trace = p->trace + (size_t)li * mx * 2;
    std::fprintf(stderr, "chain-trace items_per_layer %u wgs %u\n", mx, wgs);
    for (size_t i = layer_first[1 % m.layers]; i < layer_first[1 % m.layers] + layer_n[1 % m.layers]; ++i)
      std::fprintf(stderr, "chain-stage kind %u first %u count %u\n", all[i].kind, all[i].first, all[i].count);
  }
  for (int k = 0; k < 2; ++k) {
    p->set_begin[k] = set_begin[k];
    p->set_end[k] = set_end[k];
  }
  if (hipStreamSynchronize(st) != hipSuccess) return mi_fail(MI_ERR_STATE, "chain: init");
  *out = p.release();
  return 0;
}

int chain_launch(const ChainPlan* p, uint32_t layer, hipStream_t st) {
  if (!p || layer >= p->args.size()) return mi_fail(MI_ERR_ARG, "chain: layer out of range");
  if (p->m.head_dim == 128) chain_kernel<128><<<p->wgs, 256, 0, st>>>(p->args[layer], p->args[layer].stages);
  else chain_kernel<256><<<p->wgs, 256, 0, st>>>(p->args[layer], p->args[layer].stages);
  return mi_hip((int)hipGetLastError(), "chain launch");
}

int chain_finish(const ChainPlan* p, hipStream_t st) {
  const int k = (int)((p->m.layers - 1) & 1u);
  return mi_gemv_handoff_init(reinterpret_cast<float*>(p->arena + p->set_begin[k]), p->set_end[k] - p->set_begin[k],
                              st);
}

int chain_reset(const ChainPlan* p, hipStream_t st) {
  return p ? mi_gemv_handoff_init(reinterpret_cast<float*>(p->arena), p->arena_words, st) : 0;
}

void chain_destroy(ChainPlan* p) { delete p; }
void chain_debug(const ChainPlan* p, void** ptr, size_t* bytes) {
  *ptr = p ? p->trace : nullptr;
  uint32_t mx = 0;
  if (p)
    for (const ChainArgs& a : p->args) mx = std::max(mx, a.total);
  *bytes = p && p->trace ? (size_t)p->m.layers * mx * 8 : 0;
}
uint32_t chain_wgs(const ChainPlan* p) { return p ? p->wgs : 0u; }

}  // namespace mi
