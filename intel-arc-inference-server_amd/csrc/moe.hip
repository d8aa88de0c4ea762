// moe.hip - the mixture-of-experts block of a decode step: router || shared-gate GEMV,
// top-k routing, expert gate||up and down over int4 g64 layout-1 expert blocks, and the
// slot-ordered combine with the residual (src/kernels/moe.cl, src/kernels/gemv_bf16.cl;
// host twins tests/kernels/moe_ref.h:62-177).
//
// Four launches per block, as the reference's list (moe.cl:1-13): ids are produced and
// consumed on the device through the 32-word route row (moe.cl:49-56):
//   [0..7] expert id of slot k, [8..15] w_k (fp32 bits of an fp16 value), [16] shared gate
//   s (same), [17..24] p_k before renormalisation, [25] p of rank top_k.
//
// Arithmetic is the twins' order, so results are bitwise the oracle's where no exp is
// involved: a k-group's dot is (sum over its 8 words of the word's 8 ascending products)
// in word order; a K slice is `acc += gdot * scale` over its groups in ascending order; the
// slices merge by the pairwise tree (moe_ref.h:98-132). On MI355X the per-group dots run on
// separate lanes (each is independent) and one lane per (column, slice) then adds them in
// order from LDS: the same operations in the same order, spread over 256 lanes so the
// expert weights stream at HBM rate instead of one lane per column walking K.
#include "mi_common.h"
#include "mi_capi_internal.h"
#include "gemv_core.h"

namespace mi {
namespace {

constexpr uint32_t kRouteWords = 32, R_IDS = 0, R_W = 8, R_SG = 16, R_P = 17, R_P9 = 25;
constexpr uint32_t kUpKs = 4, kDnKs = 2;  // the reference's in-work-group K splits (kernels.h:591)
constexpr uint32_t kTileU32 = 136;        // layout 1: 128 words of nibbles + 16 f16 scales
constexpr uint32_t kMaxHidden = 4096, kMaxSlotsInter = 9 * 1024, kMaxGroups = kMaxHidden / 64;

__device__ __forceinline__ float rf(float v) { return h2f(f2h(v)); }


// ---- router || shared-gate GEMV (gemv_bf16.cl:103-200), fp16 weights --------------------
// grid (N/16, M), 16 * ksplit lanes: lane l of slice q sums column n_tile*16 + l over k8 in
// [q*per, (q+1)*per), 8 products per k8 in k order; slices merge by the pairwise tree.
// R rows per work-group (R > 1 for a prefill chunk's rows): the weights a lane loads serve all
// R rows, each row's sum running in the same order as with R = 1.
template <uint32_t R>
__global__ __launch_bounds__(256) void gemv_f16w_kernel(const uint16_t* __restrict__ w,
                                                        const uint16_t* __restrict__ x,
                                                        float* __restrict__ out, uint32_t M, uint32_t K,
                                                        uint32_t N, uint32_t ksplit) {
  __shared__ float red[R][16][16];
  const uint32_t lane = threadIdx.x & 15u, q = threadIdx.x >> 4;
  const uint32_t nt = blockIdx.x, m0 = blockIdx.y * R;
  const uint32_t rows = min(R, M - m0);
  const uint32_t K8 = K / 8, per = K8 / ksplit;
  const uint16_t* tile = w + (size_t)nt * K8 * 128 + (size_t)q * per * 128 + lane;
  const uint16_t* xr = x + (size_t)m0 * K + (size_t)q * per * 8;
  float acc[R];
#pragma unroll
  for (uint32_t r = 0; r < R; ++r) acc[r] = 0.f;
  uint32_t k8 = 0;
  if constexpr (R == 1) {
    // one row: a chunk of up to 16 k8 blocks' weights and activations is loaded before any of
    // it is used (one memory round trip per chunk; the sum's order is unchanged)
    constexpr uint32_t CH = 16;
    for (; k8 < per; k8 += CH) {
      uint16_t wv[CH][8];
      u4_t xv[CH];
#pragma unroll
      for (uint32_t u = 0; u < CH; ++u) {
        const uint32_t kk = min(k8 + u, per - 1u);  // (past the slice: re-read, not added)
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) wv[u][j] = tile[(size_t)kk * 128 + j * 16];
        xv[u] = *reinterpret_cast<const u4_t*>(xr + (size_t)kk * 8);
      }
#pragma unroll
      for (uint32_t u = 0; u < CH; ++u) {
        if (k8 + u < per) {
          const uint32_t xw[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
          for (uint32_t j = 0; j < 8; ++j)
            acc[0] += h2f(wv[u][j]) * h2f((uint16_t)(xw[j / 2] >> (16 * (j % 2))));
        }
      }
    }
  }
  for (; k8 + 4 <= per; k8 += 4) {
    uint16_t wv[4][8];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u)
#pragma unroll
      for (uint32_t j = 0; j < 8; ++j) wv[u][j] = tile[(size_t)(k8 + u) * 128 + j * 16];
#pragma unroll
    for (uint32_t r = 0; r < R; ++r) {
      if (r < rows) {
        u4_t xv[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) xv[u] = *reinterpret_cast<const u4_t*>(xr + (size_t)r * K + (k8 + u) * 8);
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
          const uint32_t xw[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
          for (uint32_t j = 0; j < 8; ++j)
            acc[r] += h2f(wv[u][j]) * h2f((uint16_t)(xw[j / 2] >> (16 * (j % 2))));
        }
      }
    }
  }
  for (; k8 < per; ++k8)
#pragma unroll
    for (uint32_t r = 0; r < R; ++r)
      if (r < rows)
        for (uint32_t j = 0; j < 8; ++j)
          acc[r] += h2f(tile[(size_t)k8 * 128 + j * 16]) * h2f(xr[(size_t)r * K + k8 * 8 + j]);
#pragma unroll
  for (uint32_t r = 0; r < R; ++r) red[r][q][lane] = acc[r];
  __syncthreads();
  for (uint32_t stride = ksplit / 2; stride > 0; stride >>= 1) {
    if (q < stride)
#pragma unroll
      for (uint32_t r = 0; r < R; ++r) red[r][q][lane] += red[r][q + stride][lane];
    __syncthreads();
  }
  if (q == 0)
#pragma unroll
    for (uint32_t r = 0; r < R; ++r)
      if (r < rows) out[(size_t)(m0 + r) * N + nt * 16 + lane] = red[r][0][lane];
}

// ---- routing (moe.cl:192-262; twin moe_ref.h:62-96) ----------------------------------------
// one work-group of E lanes per row: l = rne(logit); p = exp(l - max) / (pairwise sum);
// rank = #{j : p_j > p_e or (p_j == p_e and j < e)}; slots 0..top_k-1 take ranks 0..top_k-1;
// w_k = rne(p_k / sum of the top_k p in rank order); s = rne(sigmoid(rne(logit_E))).
// wave 0 finishes a tree over v[0 .. n) (n <= 64 a power of two, v[l] in lane l's `x`):
// level st combines v[l] with v[l + st], st = n/2 .. 1, the LDS tree's operations in its
// order; lane 0 ends with the root
template <typename F>
__device__ __forceinline__ float wave_tree(float x, uint32_t n, F op) {
  for (uint32_t st = n / 2; st > 0; st >>= 1) x = op(x, __shfl_down(x, st, 64));
  return x;
}

// The route row of one token from its router logits lg[0 .. E] (E + 1 values: the experts'
// and the shared gate's), into s_row (32 words of LDS; complete after the function's closing
// barrier). The whole work-group calls it; blockDim.x >= max(E, 64).
__device__ void route_compute(const float* lg, uint32_t* s_row, uint32_t E, uint32_t top_k) {
  __shared__ float s_red[256], s_top_p[9];
  __shared__ uint64_t s_key[256], s_cand[4 * 9];
  __shared__ uint32_t s_top_id[9];
  const uint32_t e = threadIdx.x, lane = e & 63u;
  const bool live = e < E;
  const float l = live ? rf(lg[e]) : -INFINITY;
  const float l_gate = e == 9u ? lg[E] : 0.f;  // the shared gate's logit (lane 9 writes s)
  const uint32_t n0 = E < 64u ? E : 64u;  // elements left when the cross-wave levels are done
  s_red[e] = l;
  if (e < 4u * 9u) s_cand[e] = 0ull;
  __syncthreads();
  // Wave 0 alone: lane l holds v[u] = element l + 64 u and applies the cross-wave levels of
  // the trees in their order (st = E/2 .. 64: s[e] = op(s[e], s[e + st])), then the levels
  // st < 64 across its lanes. The max is exact whatever the order; the sum is the pairwise
  // tree. p and the rank keys of all E elements go to LDS for the other waves.
  if (e < 64u) {
    float v[4];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) v[u] = lane + 64u * u < E ? s_red[lane + 64u * u] : -INFINITY;
    auto levels = [E](float v0, float v1, float v2, float v3, auto op) {
      return E == 256u ? op(op(v0, v2), op(v1, v3)) : (E == 128u ? op(v0, v1) : v0);
    };
    const auto fmax_op = [](float a, float b) { return fmaxf(a, b); };
    const auto add_op = [](float a, float b) { return a + b; };
    const float mloc = levels(v[0], v[1], v[2], v[3], fmax_op);
    const float mx = __shfl(wave_tree(lane < n0 ? mloc : -INFINITY, n0, fmax_op), 0, 64);
    float ex[4];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) ex[u] = lane + 64u * u < E ? expf(v[u] - mx) : 0.f;
    const float sloc = levels(ex[0], ex[1], ex[2], ex[3], add_op);
    const float sum = __shfl(wave_tree(lane < n0 ? sloc : 0.f, n0, add_op), 0, 64);
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
      const uint32_t j = lane + 64u * u;
      const uint32_t pb = __builtin_bit_cast(uint32_t, ex[u] / sum);
      s_key[j] = j < E ? ((uint64_t)pb << 32) | (uint32_t)~j : 0ull;
    }
  }
  __syncthreads();
  const uint32_t slots = top_k + 1;
  const uint64_t key = s_key[e];
  const float p = __builtin_bit_cast(float, (uint32_t)(key >> 32));
  const uint32_t nw = (blockDim.x + 63u) / 64u, wb = e & ~63u;
  uint32_t r1 = 0;
#pragma unroll 4
  for (uint32_t j0 = 0; j0 < 64u; j0 += 8u) {
    uint64_t kv[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) kv[u] = s_key[wb + j0 + u];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) r1 += kv[u] > key ? 1u : 0u;
  }
  const bool cand = live && r1 < slots;
  if (cand) s_cand[(e >> 6) * 9u + r1] = key;
  __syncthreads();
  if (cand) {
    uint32_t rank = 0;
    for (uint32_t w = 0; w < nw; ++w)
#pragma unroll
      for (uint32_t k = 0; k < 9u; ++k) rank += s_cand[w * 9u + k] > key ? 1u : 0u;
    if (rank < slots) {
      s_top_id[rank] = e;
      s_top_p[rank] = p;
    }
  }
  __syncthreads();
  // the row, one word per lane: w_k = rne(p_k / s8) with s8 the top_k p added in rank order
  float s8 = 0.f;
#pragma unroll
  for (uint32_t k = 0; k < 8; ++k)
    if (k < top_k) s8 += s_top_p[k];
  if (e < 8u) {
    const bool on = e < top_k;
    s_row[R_IDS + e] = on ? s_top_id[e] : 0u;
    s_row[R_W + e] = on ? __builtin_bit_cast(uint32_t, rf(s_top_p[e] / s8)) : 0u;
    s_row[R_P + e] = on ? __builtin_bit_cast(uint32_t, s_top_p[e]) : 0u;
  } else if (e == 8u) {
    s_row[R_P9] = __builtin_bit_cast(uint32_t, s_top_p[top_k]);
  } else if (e == 9u) {
    s_row[R_SG] = __builtin_bit_cast(uint32_t, rf(sigmoid_f32(rf(l_gate))));
  } else if (e > R_P9 && e < kRouteWords) {
    s_row[e] = 0u;
  }
  __syncthreads();
}

__global__ __launch_bounds__(256) void moe_route_kernel(const float* __restrict__ logits,
                                                        uint32_t* __restrict__ route, uint32_t E,
                                                        uint32_t top_k, uint32_t router_n) {
  __shared__ uint32_t s_row[kRouteWords];
  route_compute(logits + (size_t)blockIdx.x * router_n, s_row, E, top_k);
  if (threadIdx.x < kRouteWords) route[(size_t)blockIdx.x * kRouteWords + threadIdx.x] = s_row[threadIdx.x];
}

// expert block of slot `slot` (the shared expert is block E, slot top_k); an out-of-range id
// in a malformed route row reads the shared block rather than past the weights
__device__ __forceinline__ uint32_t slot_expert(const uint32_t* row, uint32_t slot, uint32_t E,
                                                uint32_t top_k) {
  if (slot >= top_k) return E;
  const uint32_t id = row[R_IDS + slot];
  return id < E ? id : E;
}

// The expert kernels work on half tiles: 8 of a layout-1 tile's 16 columns, so the grids
// hold twice the work-groups. A work-group reads its route row with scalar loads, sends out
// its activation loads (which do not depend on the route), then every weight load of its
// half tiles (16-byte pieces: a tile row's 8 words are 32 contiguous bytes, its 8 scales 16),
// all in flight together; the arithmetic then reads LDS. A staged half tile is 68 words:
// [8 rows][8 columns] of nibble words, then the 8 scales.
constexpr uint32_t kHalfU32 = 68, kHalfU4 = 17;

// issue the 17 16-byte loads of the half tile `ch` of the layout-1 tile at `tile`
__device__ __forceinline__ u4_t half_piece(const uint32_t* tile, uint32_t ch, uint32_t k) {
  // pieces 0..15: row k / 2, words 8 ch + 4 (k % 2); piece 16: scales 8 ch .. 8 ch + 7
  const uint32_t off = k < 16u ? (k >> 1) * 16u + ch * 8u + (k & 1u) * 4u : 128u + ch * 4u;
  return load_stream16(tile + off);
}

// LDS floats per 64-element group of a staged activation row: 4 of padding, so the groups
// that the lanes of one wave read together start in different banks
constexpr uint32_t kXs = 68;

// dst[g * kXs + k % 64] = h2f(src[k]) for k < n, g = k / 64 (n a multiple of 8, src 16-byte
// aligned), from u4_t pieces already loaded: v[u] holds piece threadIdx.x + 256 u
template <int PER>
__device__ __forceinline__ void put_f16(float* dst, const u4_t (&v)[PER], uint32_t n) {
  const uint32_t n8 = n / 8u;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const uint32_t i = threadIdx.x + 256u * u;
    if (i < n8) {
      const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      float* d = dst + (i / 8u) * kXs + (i % 8u) * 8u;
#pragma unroll
      for (uint32_t j = 0; j < 8; ++j) d[j] = h2f((uint16_t)(w[j / 2] >> (16 * (j % 2))));
    }
  }
}
// (every load unconditional, pieces past n re-reading the last: a load under a branch leaves
// its value in a register that the branch's join copies, and the copy waits for it at once)
template <int PER>
__device__ __forceinline__ void get_f16(u4_t (&v)[PER], const uint16_t* src, uint32_t n) {
  const uint32_t n8 = n / 8u;
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const uint32_t i = min(threadIdx.x + 256u * u, n8 - 1u);
    v[u] = *reinterpret_cast<const u4_t*>(src + 8u * i);
  }
}

// One k-group's dot for column c < 8 of a staged half tile (moe_ref.h:98-116's tile_dot body):
// sum over words j of (sum over nibbles i of (q - 8) * x) in ascending order, then * scale;
// xs: the group's 64 activations (16-byte aligned), read four at a time
__device__ __forceinline__ float half_term(const uint32_t* ht, uint32_t c, const float* __restrict__ xs) {
  uint32_t wd[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) wd[j] = ht[j * 8 + c];
  const uint16_t sc = reinterpret_cast<const uint16_t*>(ht + 64)[c];
  const f4_t* x4 = reinterpret_cast<const f4_t*>(xs);
  float g = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const f4_t lo = x4[2 * j], hi = x4[2 * j + 1];
    const float xv[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) a += (float)((int)((wd[j] >> (4 * i)) & 0xFu) - 8) * xv[i];
    g += a;
  }
  return g * h2f(sc);
}

// ---- gate||up + SiLU (moe.cl:335-381; twin moe_ref.h:154-168) ------------------------------
// grid (slots * inter/8, M): work-group (slot, ib, ch) makes h[m][slot][16 ib + 8 ch .. + 7]
// from half ch of the expert's gate tile 2 ib and up tile 2 ib + 1 (interleave16 columns).
// Dynamic LDS: 2 G staged half tiles.
// ROUTED: the work-group forms its row's route row itself from the router logits (every
// work-group of the row runs route_compute on the same logits, so they agree bitwise with
// each other and with moe_route_kernel) and work-group 0 of the row stores it for the down
// launch; `route` is then the output. This takes the routing launch off the block's chain.
template <bool ROUTED>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(uint32_t* __restrict__ route,
                                                          const float* __restrict__ logits,
                                                          uint32_t router_n,
                                                          const uint16_t* __restrict__ x,
                                                          const uint32_t* __restrict__ gu,
                                                          uint16_t* __restrict__ h, uint32_t E,
                                                          uint32_t top_k, uint32_t hidden,
                                                          uint32_t inter) {
  extern __shared__ uint32_t s_w[];  // [2][G][kHalfU32]
  __shared__ __align__(16) float s_x[kMaxHidden / 64 * kXs];
  __shared__ float s_t[2][8][kMaxGroups];
  __shared__ float s_r[2][8][kUpKs];
  __shared__ uint32_t s_row[ROUTED ? kRouteWords : 1];
  const uint32_t t = threadIdx.x, m = blockIdx.y;
  const uint32_t nhb = inter / 8, slot = blockIdx.x / nhb, hb = blockIdx.x % nhb, ib = hb / 2, ch = hb % 2;
  const uint32_t G = hidden / 64, slots = top_k + 1;
  constexpr int XP = kMaxHidden / 8 / 256;  // x pieces per thread
  u4_t xv[XP];
  get_f16<XP>(xv, x + (size_t)m * hidden, hidden);
  uint32_t e;
  if constexpr (ROUTED) {
    route_compute(logits + (size_t)m * router_n, s_row, E, top_k);
    e = slot_expert(s_row, slot, E, top_k);
    if (blockIdx.x == 0 && t < kRouteWords) route[(size_t)m * kRouteWords + t] = s_row[t];
  } else {
    e = slot_expert(route + (size_t)m * kRouteWords, slot, E, top_k);
  }
  {
    const size_t block = (size_t)(2 * inter / 16) * G * kTileU32;
    const uint32_t* base = gu + (size_t)e * block + (size_t)(2 * ib) * G * kTileU32;
    const uint32_t n4 = 2u * G * kHalfU4;  // pieces: (tile tl, group g, piece k)
    constexpr uint32_t kBatch = 9;         // 2 G * 17 <= 2176 pieces (hidden <= 4096)
    u4_t v[kBatch];
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t i = t + 256u * u;
      if (i < n4) {
        const uint32_t tg = i / kHalfU4, k = i - tg * kHalfU4;  // tg = tl * G + g
        v[u] = half_piece(base + (size_t)tg * kTileU32, ch, k);
      }
    }
    put_f16<XP>(s_x, xv, hidden);
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t i = t + 256u * u;
      if (i < n4) reinterpret_cast<u4_t*>(s_w)[i] = v[u];
    }
  }
  __syncthreads();
  // (tile, column, group) terms: thread t takes column t % 8 of groups (t / 8) % 16 + 16 k
  // of tile t / 128
  const uint32_t c = t & 7u, gsub = (t >> 3) & 15u, tl = t >> 7;
  const uint32_t* tiles = s_w + (size_t)tl * G * kHalfU32;
  for (uint32_t g = gsub; g < G; g += 16u) s_t[tl][c][g] = half_term(tiles + (size_t)g * kHalfU32, c, s_x + g * kXs);
  __syncthreads();
  if (t < 2u * 8u * kUpKs) {  // (tile, column, slice): the slice's groups in order
    const uint32_t tl2 = t / (8u * kUpKs), c2 = (t / kUpKs) % 8u, q = t % kUpKs;
    const uint32_t per = G / kUpKs;
    float acc = 0.f;
    for (uint32_t g = q * per; g < (q + 1) * per; ++g) acc += s_t[tl2][c2][g];
    s_r[tl2][c2][q] = acc;
  }
  __syncthreads();
  if (t < 8u) {
    float r[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      // the tree of moe_ref.h:127-131 at 4 slices: (q0 + q2) + (q1 + q3)
      const float a0 = s_r[u][t][0] + s_r[u][t][2];
      const float a1 = s_r[u][t][1] + s_r[u][t][3];
      r[u] = a0 + a1;
    }
    const uint16_t g_b = f2h(r[0]), u_b = f2h(r[1]);
    const uint16_t s_b = f2h(silu_f32(h2f(g_b)));
    h[((size_t)m * slots + slot) * inter + ib * 16 + ch * 8 + t] = f2h(h2f(s_b) * h2f(u_b));
  }
}

// ---- down + combine + residual (moe.cl:383-470; twin moe_ref.h:140-177) ---------------------
// grid (hidden/8, M): work-group (nb, ch) makes resid[m][16 nb + 8 ch .. + 7] from half ch of
// every slot's down tile nb, combined in slot order. Dynamic LDS: slots * G staged half tiles.
// The next RMSNorm in the same launch (DownNorm::x non-NULL): the grid has one more row of
// work-groups, after every producer; work-group m of it is row m's norm. Each producer also
// publishes its 8 new residual values as 4 hand-off words (f16 pairs, empty pattern between
// launches); the norm work-group polls the row's hidden/2 words, empties them again and
// runs mi_norm_rows' arithmetic on them (64-element chunk trees, chunks in ascending order).
struct DownNorm {
  uint32_t* words;      // [M][hidden / 2]
  const float* w;       // the norm's fp32 weights [hidden]
  uint16_t* x;          // [M][hidden]
  float* rstd;          // [M] or NULL
  float eps;
  uint32_t* status;     // set to kStatusTimeout when a wait gives up (NULL: none)
  uint32_t poll_limit;
  uint32_t inject;      // fault injection for tests: bit 0 = the down work-groups publish nothing
};
constexpr uint32_t kDnPollLimit = 1u << 21;

__device__ void down_norm_consumer(const DownNorm& dnm, uint32_t m, uint32_t hidden, uint32_t* s_words,
                                   float* s_chunk) {
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6, nch = hidden / 64u, nw = hidden / 2u;
  // the norm weights of this thread's elements first: chunks wave + 4 u, element lane
  constexpr uint32_t kCh = kMaxHidden / 64 / 4;  // chunks per wave
  float wv[kCh];
#pragma unroll
  for (uint32_t u = 0; u < kCh; ++u) {
    const uint32_t c = wave + 4u * u;
    wv[u] = c < nch ? dnm.w[c * 64u + lane] : 0.f;
  }
  uint32_t* words = dnm.words + (size_t)m * nw;
  constexpr uint32_t kPer = kMaxHidden / 2 / 256;
  uint32_t v[kPer];
  uint32_t pending = 0;
#pragma unroll
  for (uint32_t u = 0; u < kPer; ++u) {
    const uint32_t i = t + 256u * u;
    if (i < nw) {
      v[u] = ld_agent(words + i);
      if (v[u] == kEmpty) pending |= 1u << u;
    }
  }
  for (uint32_t n = 0; pending && n < dnm.poll_limit; ++n) {
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (uint32_t u = 0; u < kPer; ++u)
      if (pending & (1u << u)) {
        v[u] = ld_agent(words + t + 256u * u);
        if (v[u] != kEmpty) pending &= ~(1u << u);
      }
  }
  if (pending && dnm.status) st_agent(dnm.status, kStatusTimeout);
#pragma unroll
  for (uint32_t u = 0; u < kPer; ++u) {
    const uint32_t i = t + 256u * u;
    if (i < nw) {
      s_words[i] = v[u];
      st_agent(words + i, kEmpty);
    }
  }
  __syncthreads();
  const uint16_t* sres = reinterpret_cast<const uint16_t*>(s_words);
  float rv[kCh];
#pragma unroll
  for (uint32_t u = 0; u < kCh; ++u) {
    const uint32_t c = wave + 4u * u;
    rv[u] = 0.f;
    if (c < nch) {
      rv[u] = h2f(sres[c * 64u + lane]);
      float a = __builtin_fmaf(rv[u], rv[u], 0.f);
#pragma unroll
      for (int st = 32; st > 0; st >>= 1) a += __shfl_down(a, st, 64);
      if (lane == 0) s_chunk[c] = a;
    }
  }
  __syncthreads();
  __shared__ float s_rstd;
  if (t == 0) {
    float tot = 0.f;
    for (uint32_t c = 0; c < nch; ++c) tot += s_chunk[c];
    s_rstd = 1.0f / sqrtf(tot / (float)hidden + dnm.eps);
  }
  __syncthreads();
  const float r = s_rstd;
  if (t == 0 && dnm.rstd) dnm.rstd[m] = r;
#pragma unroll
  for (uint32_t u = 0; u < kCh; ++u) {
    const uint32_t c = wave + 4u * u;
    if (c < nch) dnm.x[(size_t)m * hidden + c * 64u + lane] = f2h(rv[u] * r * wv[u]);
  }
}

__global__ __launch_bounds__(256) void moe_down_kernel(const uint32_t* __restrict__ route,
                                                       const uint16_t* __restrict__ h,
                                                       const uint32_t* __restrict__ dn,
                                                       uint16_t* __restrict__ resid, uint32_t E,
                                                       uint32_t top_k, uint32_t hidden,
                                                       uint32_t inter, uint32_t M, DownNorm dnm) {
  extern __shared__ uint32_t s_w[];  // [slots][G][kHalfU32]
  __shared__ __align__(16) float s_h[kMaxSlotsInter / 64 * kXs];
  __shared__ float s_t[9][8][16];  // [slot][column][group], inter <= 1024
  __shared__ float s_d[9][8];
  if (dnm.x && blockIdx.y == M) {  // the norm row (uniform)
    if (blockIdx.x < M)
      down_norm_consumer(dnm, blockIdx.x, hidden, reinterpret_cast<uint32_t*>(s_h), &s_t[0][0][0]);
    return;
  }
  const uint32_t t = threadIdx.x, m = blockIdx.y, nb = blockIdx.x / 2, ch = blockIdx.x % 2;
  const uint32_t G = inter / 64, slots = top_k + 1;
  const uint32_t* row = route + (size_t)m * kRouteWords;
  uint32_t ids[9];
#pragma unroll
  for (uint32_t k = 0; k < 9; ++k) ids[k] = k < slots ? slot_expert(row, k, E, top_k) : E;
  // the combine's operands go out now rather than after the arithmetic: the slot weights and
  // the shared gate (uniform), and this lane's residual element (lanes 0..7)
  float wk[8];
#pragma unroll
  for (uint32_t k = 0; k < 8; ++k) wk[k] = k < top_k ? __builtin_bit_cast(float, row[R_W + k]) : 0.f;
  const float sg = __builtin_bit_cast(float, row[R_SG]);
  uint16_t* rp = resid + (size_t)m * hidden + nb * 16 + ch * 8 + (t & 7u);
  const uint16_t r_old = *rp;  // (every lane: lanes 8.. read lane t % 8's element, unused)
  constexpr int HP = kMaxSlotsInter / 8 / 256 + 1;  // h pieces per thread (<= 1152 pieces)
  u4_t hv[HP];
  get_f16<HP>(hv, h + (size_t)m * slots * inter, slots * inter);
  {
    const size_t block = (size_t)(hidden / 16) * G * kTileU32;
    const uint32_t n4 = slots * G * kHalfU4;  // pieces: (slot, group g, piece k)
    constexpr uint32_t kBatch = 10;           // 9 * 16 * 17 = 2448 pieces (inter <= 1024)
    u4_t v[kBatch];
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t i = t + 256u * u;
      if (i < n4) {
        const uint32_t sg = i / kHalfU4, k = i - sg * kHalfU4, sl = sg / G, g = sg - sl * G;
        uint32_t eid = ids[0];
#pragma unroll
        for (uint32_t q = 1; q < 9; ++q) eid = sl == q ? ids[q] : eid;
        v[u] = half_piece(dn + (size_t)eid * block + ((size_t)nb * G + g) * kTileU32, ch, k);
      }
    }
    put_f16<HP>(s_h, hv, slots * inter);
#pragma unroll
    for (uint32_t u = 0; u < kBatch; ++u) {
      const uint32_t i = t + 256u * u;
      if (i < n4) reinterpret_cast<u4_t*>(s_w)[i] = v[u];
    }
  }
  __syncthreads();
  const uint32_t tasks = slots * 8u * G;
  for (uint32_t i = t; i < tasks; i += 256u) {
    const uint32_t slot = i / (8u * G), rem = i % (8u * G), g = rem / 8u, c = rem % 8u;
    s_t[slot][c][g] = half_term(s_w + ((size_t)slot * G + g) * kHalfU32, c, s_h + (slot * G + g) * kXs);
  }
  __syncthreads();
  if (t < slots * 8u) {
    const uint32_t slot = t / 8u, c = t % 8u, per = G / kDnKs;
    float r[kDnKs];
#pragma unroll
    for (uint32_t q = 0; q < kDnKs; ++q) {
      float acc = 0.f;
      for (uint32_t g = q * per; g < (q + 1) * per; ++g) acc += s_t[slot][c][g];
      r[q] = acc;
    }
    s_d[slot][c] = r[0] + r[1];
  }
  __syncthreads();
  if (t < 8u) {
    // moe_ref.h:144-152: sum_k rne(rne(d_k) * w_k) in slot order; + rne(rne(d_shared) * s)
    float sum = 0.f;
#pragma unroll
    for (uint32_t k = 0; k < 8; ++k)
      if (k < top_k) sum += h2f(f2h(h2f(f2h(s_d[k][t])) * wk[k]));
    const uint16_t r_b = f2h(sum);
    const uint16_t sh_b = f2h(h2f(f2h(s_d[top_k][t])) * sg);
    const uint16_t o_b = f2h(h2f(r_b) + h2f(sh_b));
    const uint16_t nv = f2h(h2f(r_old) + h2f(o_b));
    *rp = nv;
    if (dnm.x && !(dnm.inject & 1u)) {  // the pair (t, t + 1) as one hand-off word for the norm work-group
      const uint16_t hi = (uint16_t)__shfl_down((int)nv, 1, 64);
      if ((t & 1u) == 0)
        st_agent(dnm.words + (size_t)m * (hidden / 2) + (nb * 16u + ch * 8u + t) / 2u, publishable_pair(nv, hi));
    }
  }
}

int check_moe(uint32_t M, uint32_t E, uint32_t top_k, uint32_t hidden, uint32_t inter) {
  if (M == 0 || M > 16) return mi_fail(MI_ERR_SHAPE, "moe: M must be 1..16");
  if (E < 16 || E > 256 || (E & (E - 1))) return mi_fail(MI_ERR_SHAPE, "moe: experts must be a power of two in [16, 256]");
  if (top_k < 1 || top_k > 8) return mi_fail(MI_ERR_SHAPE, "moe: top_k must be 1..8");
  if (hidden == 0 || hidden % 512 || hidden > kMaxHidden)
    return mi_fail(MI_ERR_SHAPE, "moe: hidden must be a multiple of 512 up to 4096");
  if (inter == 0 || inter % 128 || inter > 1024)
    return mi_fail(MI_ERR_SHAPE, "moe: inter must be a multiple of 128 up to 1024");
  return 0;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" int mi_gemv_f16w(const uint16_t* w_tiled, const uint16_t* x, float* out, uint32_t M, uint32_t K,
                            uint32_t N, uint32_t ksplit, void* stream) {
  if (!w_tiled || !x || !out) return mi_fail(MI_ERR_ARG, "gemv_f16w: null pointer");
  // one work-group per (16 columns, row), rows independent: any M up to the grid's 65535 rows
  if (M == 0 || M > 65535u || K == 0 || N == 0 || N % 16 || K % 64)
    return mi_fail(MI_ERR_SHAPE, "gemv_f16w: M 1..65535, K a multiple of 64, N a multiple of 16");
  if (ksplit == 0 || ksplit > 16 || (ksplit & (ksplit - 1)) || (K / 8) % ksplit)
    return mi_fail(MI_ERR_SHAPE, "gemv_f16w: ksplit must be a power of two <= 16 dividing K/8");
  if (reinterpret_cast<uintptr_t>(x) % 16) return mi_fail(MI_ERR_ARG, "gemv_f16w: x needs 16-byte alignment");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (M >= 64)
    gemv_f16w_kernel<8><<<dim3(N / 16, (M + 7) / 8), 16 * ksplit, 0, st>>>(w_tiled, x, out, M, K, N, ksplit);
  else
    gemv_f16w_kernel<1><<<dim3(N / 16, M), 16 * ksplit, 0, st>>>(w_tiled, x, out, M, K, N, ksplit);
  return mi_hip(static_cast<int>(hipGetLastError()), "gemv_f16w launch");
}

extern "C" int mi_moe_route(const float* logits, uint32_t* route, uint32_t M, uint32_t experts, uint32_t top_k,
                            uint32_t router_n, void* stream) {
  if (!logits || !route) return mi_fail(MI_ERR_ARG, "moe_route: null pointer");
  // one work-group per row, rows independent: any M (a prefill chunk routes all its rows at once)
  if (M == 0 || M > 65535u) return mi_fail(MI_ERR_SHAPE, "moe_route: M must be 1..65535");
  if (int e = check_moe(1, experts, top_k, 512, 128)) return e;
  if (router_n < experts + 1) return mi_fail(MI_ERR_SHAPE, "moe_route: router_n must hold experts + 1 rows");
  moe_route_kernel<<<M, experts < 64 ? 64 : experts, 0, static_cast<hipStream_t>(stream)>>>(logits, route, experts, top_k, router_n);
  return mi_hip(static_cast<int>(hipGetLastError()), "moe_route launch");
}

extern "C" int mi_moe_gate_up(const uint32_t* route, const uint16_t* x, const uint32_t* gu_blocks, uint16_t* h,
                              uint32_t M, uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                              void* stream) {
  if (!route || !x || !gu_blocks || !h) return mi_fail(MI_ERR_ARG, "moe_gate_up: null pointer");
  if (int e = check_moe(M, experts, top_k, hidden, inter)) return e;
  if (reinterpret_cast<uintptr_t>(gu_blocks) % 16 || reinterpret_cast<uintptr_t>(x) % 16)
    return mi_fail(MI_ERR_ARG, "moe_gate_up: gu_blocks and x need 16-byte alignment");
  const size_t lds = size_t(2) * (hidden / 64) * kHalfU32 * 4;
  moe_gate_up_kernel<false><<<dim3((top_k + 1) * (inter / 8), M), 256, lds, static_cast<hipStream_t>(stream)>>>(
      const_cast<uint32_t*>(route), nullptr, 0, x, gu_blocks, h, experts, top_k, hidden, inter);
  return mi_hip(static_cast<int>(hipGetLastError()), "moe_gate_up launch");
}

extern "C" int mi_moe_gate_up_routed(const float* logits, uint32_t router_n, uint32_t* route, const uint16_t* x,
                                     const uint32_t* gu_blocks, uint16_t* h, uint32_t M, uint32_t experts,
                                     uint32_t top_k, uint32_t hidden, uint32_t inter, void* stream) {
  if (!logits || !route || !x || !gu_blocks || !h) return mi_fail(MI_ERR_ARG, "moe_gate_up_routed: null pointer");
  if (int e = check_moe(M, experts, top_k, hidden, inter)) return e;
  if (router_n < experts + 1) return mi_fail(MI_ERR_SHAPE, "moe_gate_up_routed: router_n must hold experts + 1 rows");
  if (reinterpret_cast<uintptr_t>(gu_blocks) % 16 || reinterpret_cast<uintptr_t>(x) % 16)
    return mi_fail(MI_ERR_ARG, "moe_gate_up_routed: gu_blocks and x need 16-byte alignment");
  const size_t lds = size_t(2) * (hidden / 64) * kHalfU32 * 4;
  moe_gate_up_kernel<true><<<dim3((top_k + 1) * (inter / 8), M), 256, lds, static_cast<hipStream_t>(stream)>>>(
      route, logits, router_n, x, gu_blocks, h, experts, top_k, hidden, inter);
  return mi_hip(static_cast<int>(hipGetLastError()), "moe_gate_up_routed launch");
}

extern "C" int mi_moe_down(const uint32_t* route, const uint16_t* h, const uint32_t* dn_blocks, uint16_t* resid,
                           uint32_t M, uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                           void* stream) {
  if (!route || !h || !dn_blocks || !resid) return mi_fail(MI_ERR_ARG, "moe_down: null pointer");
  if (int e = check_moe(M, experts, top_k, hidden, inter)) return e;
  if (reinterpret_cast<uintptr_t>(dn_blocks) % 16 || reinterpret_cast<uintptr_t>(h) % 16)
    return mi_fail(MI_ERR_ARG, "moe_down: dn_blocks and h need 16-byte alignment");
  const size_t lds = size_t(top_k + 1) * (inter / 64) * kHalfU32 * 4;
  moe_down_kernel<<<dim3(hidden / 8, M), 256, lds, static_cast<hipStream_t>(stream)>>>(
      route, h, dn_blocks, resid, experts, top_k, hidden, inter, M, DownNorm{});
  return mi_hip(static_cast<int>(hipGetLastError()), "moe_down launch");
}

extern "C" int mi_moe_down_norm(const uint32_t* route, const uint16_t* h, const uint32_t* dn_blocks, uint16_t* resid,
                                uint32_t M, uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                                const float* norm_w, uint16_t* x_out, float* rstd, float eps, uint32_t* handoff,
                                uint32_t* status, uint32_t poll_limit, uint32_t inject, void* stream) {
  if (!route || !h || !dn_blocks || !resid || !norm_w || !x_out || !handoff)
    return mi_fail(MI_ERR_ARG, "moe_down_norm: null pointer");
  if (int e = check_moe(M, experts, top_k, hidden, inter)) return e;
  if (M > 8) return mi_fail(MI_ERR_SHAPE, "moe_down_norm: M must be <= 8");
  if (reinterpret_cast<uintptr_t>(dn_blocks) % 16 || reinterpret_cast<uintptr_t>(h) % 16)
    return mi_fail(MI_ERR_ARG, "moe_down_norm: dn_blocks and h need 16-byte alignment");
  const size_t lds = size_t(top_k + 1) * (inter / 64) * kHalfU32 * 4;
  const DownNorm dnm{handoff, norm_w, x_out, rstd, eps, status, poll_limit ? poll_limit : kDnPollLimit, inject};
  moe_down_kernel<<<dim3(hidden / 8, M + 1), 256, lds, static_cast<hipStream_t>(stream)>>>(
      route, h, dn_blocks, resid, experts, top_k, hidden, inter, M, dnm);
  return mi_hip(static_cast<int>(hipGetLastError()), "moe_down_norm launch");
}

