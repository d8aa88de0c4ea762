// prefill.hip - the chunked prefill's kernels on gfx950: the int4 linear for many rows on the
// matrix cores, the causal attention of a chunk over the KV cache, and the chunk's embedding
// gather.
//
// Replaces the reference's prefill walk (src/runtime/prefill/step.h step_chunk, Engine::prefill
// src/runtime/engine.h:97-115): per chunk of T positions, the embedding gather and first norm,
// then per layer q||k||v, attn_prep, the chunk's causal attention, o + residual + norm,
// gate||up + SiLU, down + residual + norm; the last position's head and argmax leave the control
// block as decode's ingest of the same ids would (cur_token = the argmax, pos advanced by T).
//
// gemm_w4a16_kernel: out[T][N] fp32 = x[T][K] (f16) . W[K][N] (int4 GPTQ g64, layout 0). The
// contraction is a dense GEMM here (2 T K N flops over K N / 2 weight bytes): MFMA-bound from a
// few dozen rows, so it is tiled for the matrix cores rather than streamed like the decode GEMV.
//   * 4 waves per work-group, each 16 RI rows x 64 columns = RI x 4 v_mfma_f32_16x16x32_f16
//     tiles; WM waves along the rows: tiles of 128 x 256 (RI 8, one row of waves: the B words
//     are loaded and dequantised once per work-group and serve 128 rows), 96 x 256, 64 x 256 and
//     128 x 128 (see launch_gemm for the choice);
//   * one 64-deep k-group per iteration (one scale per column). The activations go through LDS,
//     double-buffered (the next group's rows are loaded into registers while the current group
//     is multiplied, then written to the other buffer). The weights skip LDS: a B fragment of
//     v_mfma_f32_16x16x32_f16 is 8 consecutive k of one column, which is exactly one int4 word,
//     so each lane loads its own words a group ahead and dequantises them into the fragment
//     (LDS then carries the activations only, which halves its traffic per MFMA);
//   * w = f16((q - 8) * scale): q - 8 exact in f16 (the magic-number unpack of the decode GEMV),
//     one f16 rounding of the product (the reference's prefill rounds the same product to bf16,
//     pf_dequant_slab.cl); the activations are permuted to the unpack's pair order
//     (k0,k4)(k1,k5)(k2,k6)(k3,k7) inside each 8-k chunk, so the products pair up;
//   * fp32 accumulation across the whole K in MFMA order.
//
// attn_prefill_kernel: causal GQA attention of T query rows at positions pos0 .. pos0+T-1 over
// the fp16 cache rows [0, pos0 + t] (the chunk's own rows written by attn_prep before it). A
// work-group takes one kv head and 64 / GQA rows; its 4 waves each own 16 (row, q head) columns
// of the MFMA and walk the same keys, 64 per iteration staged once in LDS for all of them (K as
// rows, V transposed so that the P.V operand of 4 keys of one dimension is one 8-byte read).
// Per 16-key group the decode kernel's per-wave flash step (csrc/attn.hip): S^T = K Q^T with q
// as f16 high + low parts, the online softmax per column in fp32, O^T += V^T P^T with P as f16
// high + low parts, so the result is fp32-accurate attention; keys past a row's position are
// -inf. Every wave covers every key its rows need, so no merge across waves is needed.
#include <algorithm>
#include <string>

#include "mi_capi_internal.h"
#include "mi_common.h"

namespace mi {
namespace {

// ---------------------------------------------------------------------------------------------
// the int4 linear for many rows
// ---------------------------------------------------------------------------------------------
constexpr uint32_t GBK = 64;
constexpr uint32_t GPAD = 8;             // f16 of padding per LDS row (a 144-byte stride)
constexpr uint32_t GROW = GBK + GPAD;    // LDS row length in f16

// 8 natural-order activations (x0..x7 in four u32) into the unpack's pair order.
__device__ __forceinline__ u4_t perm_pairs(u4_t v) {
  return u4_t{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
              __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
}

// f16((q_i - 8) * s) of one word's 8 nibbles, pair order (q0,q4)(q1,q5)(q2,q6)(q3,q7)
__device__ __forceinline__ u4_t dequant_scaled(uint32_t w, h2_t s2) {
  const uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u, magic = 0x64006400u;
  const h2_t b1032 = {(half_t)1032.0f, (half_t)1032.0f};
  const h2_t s16 = {(half_t)0.0625f, (half_t)0.0625f};
  const h2_t b72 = {(half_t)-72.0f, (half_t)-72.0f};
  const uint32_t t = w >> 8;
  const h2_t p0 = as_h2(and_or(w, m_lo, magic)) - b1032;                               // q - 8, exact
  const h2_t p1 = __builtin_elementwise_fma(as_h2(and_or(w, m_hi, magic)), s16, b72);  // exact
  const h2_t p2 = as_h2(and_or(t, m_lo, magic)) - b1032;
  const h2_t p3 = __builtin_elementwise_fma(as_h2(and_or(t, m_hi, magic)), s16, b72);
  return u4_t{h2_bits(p0 * s2), h2_bits(p1 * s2), h2_bits(p2 * s2), h2_bits(p3 * s2)};
}

// SILU: the columns are gate||up in the interleave16 order (gate block, up block, ...); a wave's
// 64 columns hold two such pairs, so each lane has the gate and up value of the same output in
// its tiles j and j + 1, and writes h [T][N/2] f16 = rne(rne(silu(rne(g))) * rne(u)) (the
// arithmetic of prep_silu_mul, prep.cl:384) instead of the fp32 output.
template <bool SILU, uint32_t WM, uint32_t RI, uint32_t LB>
__global__ __launch_bounds__(256, LB) void gemm_w4a16_kernel(const uint32_t* __restrict__ qweight,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ x,
                                                         float* __restrict__ out, uint16_t* __restrict__ h_out,
                                                         uint32_t T, uint32_t K, uint32_t N) {
  // WM waves along the rows, 4 / WM along the columns, each wave 16 RI rows x 64 columns
  constexpr uint32_t BM = 16u * RI * WM, BN = 256u / WM, WN = 4u / WM, AI = BM / 32u;
  __shared__ __align__(16) uint16_t As[2][BM][GROW];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t wm = wave / WN, wn = wave % WN;
  const uint32_t n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const uint32_t G = K / GBK;
  const uint32_t fr = lane & 15u, fq = lane >> 4;  // fragment row/column, k chunk (8 k)

  // activations, staged through LDS: thread t takes rows (t >> 3) + 32 i (i < BM / 32), 8-k chunk t & 7
  const uint32_t a_row = t >> 3, a_chunk = t & 7u;
  // buffer loads: 32-bit offsets keep the addresses out of 64-bit registers; the row sits in the
  // per-thread offset, so a row at or past T lies outside the resource's T K elements and reads 0
  const __amdgpu_buffer_rsrc_t x_rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(x), 0, T * K * 2u, 0x00020000);
  const __amdgpu_buffer_rsrc_t w_rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(qweight), 0, (K / 8u) * N * 4u, 0x00020000);
  const __amdgpu_buffer_rsrc_t s_rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(scales), 0, (K / GBK) * N * 2u, 0x00020000);
  const uint32_t a_voff = ((m0 + a_row) * K + 8u * a_chunk) * 2u;
  u4_t a_st[AI];
  auto load_a = [&](uint32_t g) {
#pragma unroll
    for (uint32_t i = 0; i < AI; ++i)
      a_st[i] = __builtin_bit_cast(
          u4_t, __builtin_amdgcn_raw_buffer_load_b128(x_rs, a_voff + 32u * i * K * 2u, g * GBK * 2u, 0));
  };
  auto store_a = [&](uint32_t buf) {
#pragma unroll
    for (uint32_t i = 0; i < AI; ++i)
      *reinterpret_cast<u4_t*>(&As[buf][a_row + 32u * i][8u * a_chunk]) = perm_pairs(a_st[i]);
  };
  // weights, straight into registers: the B fragment of n-tile j and k half ks is one word per
  // lane (8 k of column 16 j + fr, word row 4 ks + fq of the group), dequantised just before use
  const uint32_t ncol = n0 + 64u * wn + fr;
  const uint32_t w_voff = (fq * N + ncol) * 4u, s_voff = ncol * 2u;
  uint32_t b_w[2][4];
  uint16_t b_s[4];
  auto load_b = [&](uint32_t g) {
#pragma unroll
    for (uint32_t ks = 0; ks < 2; ++ks)
#pragma unroll
      for (uint32_t j = 0; j < 4; ++j)
        b_w[ks][j] = __builtin_amdgcn_raw_buffer_load_b32(w_rs, w_voff, ((8u * g + 4u * ks) * N + 16u * j) * 4u, 2);
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j)
      b_s[j] = __builtin_amdgcn_raw_buffer_load_b16(s_rs, s_voff, (g * N + 16u * j) * 2u, 0);
  };

  f4_t acc[RI][4];
#pragma unroll
  for (uint32_t i = 0; i < RI; ++i)
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  load_a(0);
  load_b(0);
  store_a(0);
  lds_barrier();
  for (uint32_t g = 0; g < G; ++g) {
    const uint32_t buf = g & 1u;
    // this group's weights become fragments; the next group's loads go out
    h8_t bf[2][4];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const h2_t s2 = as_h2((uint32_t)b_s[j] | ((uint32_t)b_s[j] << 16));
#pragma unroll
      for (uint32_t ks = 0; ks < 2; ++ks) bf[ks][j] = __builtin_bit_cast(h8_t, dequant_scaled(b_w[ks][j], s2));
    }
    if (g + 1 < G) {
      load_a(g + 1);
      load_b(g + 1);
    }
#pragma unroll
    for (uint32_t ks = 0; ks < 2; ++ks) {
      h8_t af[RI];
#pragma unroll
      for (uint32_t i = 0; i < RI; ++i)
        af[i] = *reinterpret_cast<const h8_t*>(&As[buf][16u * RI * wm + 16u * i + fr][32u * ks + 8u * fq]);
#pragma unroll
      for (uint32_t i = 0; i < RI; ++i)
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[ks][j], acc[i][j], 0, 0, 0);
    }
    if (g + 1 < G) store_a(buf ^ 1u);  // the other buffer was last read before the previous barrier
    lds_barrier();
  }
  // lane holds rows 4 (lane >> 4) + r of column lane & 15 of each 16 x 16 tile
#pragma unroll
  for (uint32_t i = 0; i < RI; ++i)
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
      const uint32_t row = m0 + 16u * RI * wm + 16u * i + 4u * fq + r;
      if (row < T) {
        if constexpr (SILU) {
#pragma unroll
          for (uint32_t jp = 0; jp < 2; ++jp) {
            const uint16_t g_b = f2h(acc[i][2 * jp][r]), u_b = f2h(acc[i][2 * jp + 1][r]);
            const uint16_t s_b = f2h(silu_f32(h2f(g_b)));
            h_out[(size_t)row * (N / 2) + (n0 + 64u * wn) / 2 + 16u * jp + fr] = f2h(h2f(s_b) * h2f(u_b));
          }
        } else {
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) out[(size_t)row * N + ncol + 16u * j] = acc[i][j][r];
        }
      }
    }
}

// ---------------------------------------------------------------------------------------------
// the chunk's MoE block, grouped by expert
// ---------------------------------------------------------------------------------------------
// The decode kernels take one row at a time through every expert it routes to, which for a
// chunk reads each expert's weights once per routed row. Here the chunk's (row, slot) pairs are
// grouped by expert first (moe_group_kernel), so each expert's weights stream once per 64 of
// its pairs through the MFMA tile of gemm_w4a16_kernel (moe_gemm_kernel: layout-1 weights,
// gathered activation rows, scattered outputs), and the slot-ordered combine with the residual
// (moe.cl:383-470's epilogue, moe_ref.h:144-152) runs per row afterwards.
constexpr uint32_t kMoeRouteWords = 32, kMoeW = 8, kMoeSG = 16;  // the route row (moe.cl:49-56)
constexpr uint32_t kMoeTile = 136;                                 // layout 1: 128 words + 16 f16 scales
constexpr uint32_t kMoeRows = 64;                                  // pairs per row tile
constexpr uint32_t kMoeMaxPairs = 2048u * 9u;                      // T <= 2048, top_k <= 8

// the expert of slot s of a route row: the shared expert (index E) for s = top_k, and for an
// id outside [0, E) (moe.hip's slot_expert)
__device__ __forceinline__ uint32_t moe_slot_expert(const uint32_t* row, uint32_t s, uint32_t E, uint32_t top_k) {
  if (s >= top_k) return E;
  const uint32_t id = row[s];
  return id < E ? id : E;
}

// One work-group, a stable counting sort of the pairs p = t (top_k + 1) + s of T rows by expert:
// expert e's pairs go to list[off_e ..] in ascending p (the reference's (token, slot) order), its
// row tiles to tiles[] as {e, first list index, pair count}, the tile count to tiles_n[0]. Wave w (of
// 16) owns the pairs [w Q, (w + 1) Q): it counts them per expert, then places them 64 at a time, a
// lane's rank among the lanes of its expert coming from a match mask built from 9 ballots (one per
// bit of the expert index), so list[] is the same on every call.
__global__ __launch_bounds__(1024) void moe_group_kernel(const uint32_t* __restrict__ route, uint32_t T,
                                                        uint32_t E, uint32_t top_k, uint32_t* __restrict__ list,
                                                        u4_t* __restrict__ tiles, uint32_t* __restrict__ tiles_n) {
  __shared__ uint16_t s_ex[kMoeMaxPairs];
  constexpr uint32_t kW = 16, kT = kW * 64;
  __shared__ uint32_t s_wc[kW][257], s_off[257], s_toff[257], s_cnt[257];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6, slots = top_k + 1, P = T * slots;
  for (uint32_t e = t; e <= E; e += kT)
    for (uint32_t w = 0; w < kW; ++w) s_wc[w][e] = 0;
  for (uint32_t p = t; p < P; p += kT)
    s_ex[p] = (uint16_t)moe_slot_expert(route + (size_t)(p / slots) * kMoeRouteWords, p % slots, E, top_k);
  __syncthreads();
  const uint32_t Q = (P + kW - 1u) / kW, lo = min(P, wave * Q), hi = min(P, lo + Q);
  for (uint32_t p = lo + lane; p < hi; p += 64u) atomicAdd(&s_wc[wave][s_ex[p]], 1u);  // counts only
  __syncthreads();
  for (uint32_t e = t; e <= E; e += kT) {
    uint32_t c = 0;
    for (uint32_t w = 0; w < kW; ++w) c += s_wc[w][e];
    s_cnt[e] = c;
  }
  __syncthreads();
  if (t == 0) {
    uint32_t o = 0, to = 0;
    for (uint32_t e = 0; e <= E; ++e) {
      s_off[e] = o;
      s_toff[e] = to;
      o += s_cnt[e];
      to += (s_cnt[e] + kMoeRows - 1u) / kMoeRows;
    }
    tiles_n[0] = to;
  }
  __syncthreads();
  for (uint32_t e = t; e <= E; e += kT) {  // s_wc becomes each wave's next list index per expert
    uint32_t b = s_off[e];
    for (uint32_t w = 0; w < kW; ++w) {
      const uint32_t c = s_wc[w][e];
      s_wc[w][e] = b;
      b += c;
    }
  }
  __syncthreads();
  const uint64_t below = lane ? (~0ull >> (64u - lane)) : 0ull;
  for (uint32_t p0 = lo; p0 < hi; p0 += 64u) {
    const uint32_t p = p0 + lane;
    const bool valid = p < hi;
    const uint32_t e = valid ? s_ex[p] : 511u;  // 511: no expert index (E <= 256)
    uint64_t same = __ballot(valid);
#pragma unroll
    for (uint32_t b = 0; b < 9u; ++b) {
      const uint64_t bal = __ballot((e >> b) & 1u);
      same &= ((e >> b) & 1u) ? bal : ~bal;
    }
    const uint32_t rank = (uint32_t)__popcll(same & below);
    const uint32_t base = valid ? s_wc[wave][e] : 0u;
    if (valid) list[base + rank] = p;
    __builtin_amdgcn_wave_barrier();
    if (valid && rank == 0) s_wc[wave][e] = base + (uint32_t)__popcll(same);
    __builtin_amdgcn_wave_barrier();
  }
  for (uint32_t e = t; e <= E; e += kT) {
    const uint32_t n = s_cnt[e];
    for (uint32_t k = 0; k * kMoeRows < n; ++k)
      tiles[s_toff[e] + k] = u4_t{e, s_off[e] + k * kMoeRows, min(kMoeRows, n - k * kMoeRows), 0u};
  }
}

// out rows = pairs of one expert (a row tile) x that expert's layout-1 block (K x N, columns in
// 16-column tiles of 64-k groups: word j of the group's tile holds k 8 j .. 8 j + 7 of column c
// at j 16 + c, its f16 scale at half-word 256 + c). A row of a pair p is row p / slots of x
// (GATE_UP) or row p of h (down). GATE_UP: N = 2 inter in interleave16 order, SwiGLU in the
// epilogue into h[p][inter] (the dense GEMM's epilogue); down: d[p][N] rounded to f16 (the
// combine's first rounding of a slot's value, so nothing is lost). Tile: 64 pairs x
// 256 columns, 4 waves of 64 x 64, the dense GEMM's k loop.
template <bool GATE_UP>
__global__ __launch_bounds__(256) void moe_gemm_kernel(const u4_t* __restrict__ tiles,
                                                       const uint32_t* __restrict__ tiles_n,
                                                       const uint32_t* __restrict__ list,
                                                       const uint32_t* __restrict__ blocks, size_t block_u32,
                                                       const uint16_t* __restrict__ a, uint32_t a_rows,
                                                       uint16_t* __restrict__ h_out, uint16_t* __restrict__ d_out,
                                                       uint32_t slots, uint32_t K, uint32_t N) {
  __shared__ __align__(16) uint16_t As[2][kMoeRows][GROW];
  if (blockIdx.y >= tiles_n[0]) return;  // uniform: the grid is sized for the most tiles
  const u4_t tile = tiles[blockIdx.y];
  const uint32_t e = tile.x, first = tile.y, cnt = tile.z;
  const uint32_t t = threadIdx.x, lane = t & 63u, wn = t >> 6;
  const uint32_t n0 = blockIdx.x * 256u, G = K / GBK;
  const uint32_t fr = lane & 15u, fq = lane >> 4;

  // activations: thread t stages pairs (t >> 3) + 32 i (i < 2), 8-k chunk t & 7; a pair past
  // the tile's count gets an offset outside the resource and reads zeros
  const uint32_t a_row = t >> 3, a_chunk = t & 7u;
  const __amdgpu_buffer_rsrc_t x_rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(a), 0, a_rows * K * 2u, 0x00020000);
  uint32_t a_voff[2];
#pragma unroll
  for (uint32_t i = 0; i < 2; ++i) {
    const uint32_t r = a_row + 32u * i;
    const uint32_t p = r < cnt ? list[first + r] : 0u;
    const uint32_t src = GATE_UP ? p / slots : p;
    a_voff[i] = r < cnt ? (src * K + 8u * a_chunk) * 2u : 0x80000000u;
  }
  u4_t a_st[2];
  auto load_a = [&](uint32_t g) {
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i)
      a_st[i] = __builtin_bit_cast(u4_t, __builtin_amdgcn_raw_buffer_load_b128(x_rs, a_voff[i], g * GBK * 2u, 0));
  };
  auto store_a = [&](uint32_t buf) {
#pragma unroll
    for (uint32_t i = 0; i < 2; ++i)
      *reinterpret_cast<u4_t*>(&As[buf][a_row + 32u * i][8u * a_chunk]) = perm_pairs(a_st[i]);
  };
  // weights: column n = n0 + 64 wn + 16 j + fr sits in 16-column tile n / 16 at column fr
  const uint32_t* wb = blocks + (size_t)e * block_u32;
  const __amdgpu_buffer_rsrc_t w_rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(wb), 0, (uint32_t)(block_u32 * 4u), 0x00020000);
  const uint32_t cb0 = (n0 + 64u * wn) / 16u;
  uint32_t b_w[2][4];
  uint32_t b_s[4];
  auto load_b = [&](uint32_t g) {
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const uint32_t tb = ((cb0 + j) * G + g) * kMoeTile;  // u32 index of the tile
#pragma unroll
      for (uint32_t ks = 0; ks < 2; ++ks)
        b_w[ks][j] = __builtin_amdgcn_raw_buffer_load_b32(w_rs, ((4u * ks + fq) * 16u + fr) * 4u, tb * 4u, 2);
      b_s[j] = __builtin_amdgcn_raw_buffer_load_b16(w_rs, (256u + fr) * 2u, tb * 4u, 0);
    }
  };

  f4_t acc[4][4];
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i)
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  load_a(0);
  load_b(0);
  store_a(0);
  lds_barrier();
  for (uint32_t g = 0; g < G; ++g) {
    const uint32_t buf = g & 1u;
    h8_t bf[2][4];
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
      const h2_t s2 = as_h2(b_s[j] | (b_s[j] << 16));
#pragma unroll
      for (uint32_t ks = 0; ks < 2; ++ks) bf[ks][j] = __builtin_bit_cast(h8_t, dequant_scaled(b_w[ks][j], s2));
    }
    if (g + 1 < G) {
      load_a(g + 1);
      load_b(g + 1);
    }
#pragma unroll
    for (uint32_t ks = 0; ks < 2; ++ks) {
      h8_t af[4];
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const h8_t*>(&As[buf][16u * i + fr][32u * ks + 8u * fq]);
#pragma unroll
      for (uint32_t i = 0; i < 4; ++i)
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[ks][j], acc[i][j], 0, 0, 0);
    }
    if (g + 1 < G) store_a(buf ^ 1u);
    lds_barrier();
  }
  // lane holds pairs 4 (lane >> 4) + r of column lane & 15 of each 16 x 16 tile
#pragma unroll
  for (uint32_t i = 0; i < 4; ++i)
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
      const uint32_t q = 16u * i + 4u * fq + r;
      if (q < cnt) {
        const uint32_t p = list[first + q];
        if constexpr (GATE_UP) {
#pragma unroll
          for (uint32_t jp = 0; jp < 2; ++jp) {
            const uint16_t g_b = f2h(acc[i][2 * jp][r]), u_b = f2h(acc[i][2 * jp + 1][r]);
            const uint16_t s_b = f2h(silu_f32(h2f(g_b)));
            h_out[(size_t)p * (N / 2) + (n0 + 64u * wn) / 2 + 16u * jp + fr] = f2h(h2f(s_b) * h2f(u_b));
          }
        } else {
#pragma unroll
          for (uint32_t j = 0; j < 4; ++j) d_out[(size_t)p * N + n0 + 64u * wn + 16u * j + fr] = f2h(acc[i][j][r]);
        }
      }
    }
}

// resid[t][n] += the slot-ordered combine of row t's pair outputs (moe_down_kernel's epilogue,
// moe_ref.h:144-152): sum_k rne(rne(d_k) w_k) in slot order, + rne(rne(d_shared) s)
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint32_t* __restrict__ route,
                                                          const uint16_t* __restrict__ d, uint16_t* __restrict__ resid,
                                                          uint32_t top_k, uint32_t hidden) {
  const uint32_t t = blockIdx.y, n = blockIdx.x * 256u + threadIdx.x;
  if (n >= hidden) return;
  const uint32_t* row = route + (size_t)t * kMoeRouteWords;
  const uint32_t slots = top_k + 1;
  const uint16_t* dp = d + (size_t)t * slots * hidden + n;
  float sum = 0.f;
  for (uint32_t k = 0; k < top_k; ++k) {
    const float wk = __builtin_bit_cast(float, row[kMoeW + k]);
    sum += h2f(f2h(h2f(dp[(size_t)k * hidden]) * wk));
  }
  const uint16_t r_b = f2h(sum);
  const float sg = __builtin_bit_cast(float, row[kMoeSG]);
  const uint16_t sh_b = f2h(h2f(dp[(size_t)top_k * hidden]) * sg);
  const uint16_t o_b = f2h(h2f(r_b) + h2f(sh_b));
  uint16_t* rp = resid + (size_t)t * hidden + n;
  *rp = f2h(h2f(*rp) + h2f(o_b));
}

// ---------------------------------------------------------------------------------------------
// the chunk's causal attention
// ---------------------------------------------------------------------------------------------
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));

struct PrefillAttnArgs {
  const float* attn_q;  // [T][q_heads][HD] fp32
  const void* kv_k;     // f16, or int8 (KV8)
  const void* kv_v;
  const uint32_t* pages;
  uint16_t* attn_out;   // [T][q_heads * HD] f16
  size_t row_stride, head_stride;
  uint32_t page, T, pos0, q_heads;
  float scale;
  // KV8: fp16 row scales at row * sc_row_stride + head * sc_head_stride, and the output in
  // the cache's rotated basis, fp32 [T][q_heads][HD], for the un-rotation pass
  const uint16_t* k_scale;
  const uint16_t* v_scale;
  size_t sc_row_stride, sc_head_stride;
  float* out_rot;
};

// 8 int8 values (two u32) widened exactly to f16: each biased byte u = q8 + 128 under an f16
// exponent byte 0x64 is 1024 + u; subtracting 1152 leaves q8 (f16 integers up to 2048 are exact)
__device__ __forceinline__ u4_t widen_i8x8(uint32_t x0, uint32_t x1) {
  x0 ^= 0x80808080u;
  x1 ^= 0x80808080u;
  const uint32_t hi = 0x64646464u;
  const h2_t bias = {(half_t)1152.0f, (half_t)1152.0f};
  return u4_t{h2_bits(as_h2(__builtin_amdgcn_perm(hi, x0, 0x04010400u)) - bias),
              h2_bits(as_h2(__builtin_amdgcn_perm(hi, x0, 0x04030402u)) - bias),
              h2_bits(as_h2(__builtin_amdgcn_perm(hi, x1, 0x04010400u)) - bias),
              h2_bits(as_h2(__builtin_amdgcn_perm(hi, x1, 0x04030402u)) - bias)};
}

// KV8: the K and V rows are int8 with one fp16 scale per (position, kv head), the attn_prep_kv8
// form (kv8.cl): the rows are widened exactly to f16 in LDS, a score is scaled by its key's K
// scale and a weight by its key's V scale before P V (the decode reader's order), and the
// output stays in the rotated basis (un-rotated by unrotate_rows_kernel).
template <int HD, int GQA, int KV8>
__global__ __launch_bounds__(256) void attn_prefill_kernel(PrefillAttnArgs a) {
  constexpr uint32_t KK = HD / 32, NT = HD / 16;
  constexpr uint32_t RB = 64 / GQA;          // rows per work-group
  constexpr uint32_t KB = 64;                // keys per iteration
  constexpr uint32_t KROW = HD + 8;          // padded K row in LDS (f16)
  constexpr uint32_t ROWB = HD * 2;          // K row bytes
  constexpr uint32_t VTP = KB + 4;           // V^T row (one dimension over the 64 keys), padded
  constexpr uint32_t DPT = HD / 8;           // dimensions per staging thread of a key pair
  __shared__ __align__(16) uint16_t sK[KB * KROW];
  __shared__ __align__(16) uint16_t sVt[HD * VTP];
  __shared__ float sKs[KV8 ? KB : 1], sVs[KV8 ? KB : 1];
  // the last row blocks see the most keys: they are dispatched first, so the short blocks fill
  // the tail of the grid
  const uint32_t j = blockIdx.x, t0 = (gridDim.y - 1u - blockIdx.y) * RB;
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t qi = lane & 15u, qq = lane >> 4;
  // this lane's column: pair p = 16 wave + qi -> row t0 + p / GQA, q head j GQA + p % GQA
  const uint32_t p = 16u * wave + qi, prow = p / GQA, ph = j * GQA + p % GQA;
  const bool col_live = prow < RB && t0 + prow < a.T;
  const uint32_t rows_here = min(RB, a.T - t0);
  const uint32_t kend = a.pos0 + t0 + rows_here;  // keys [0, kend) cover every row of the block
  const uint32_t lim = col_live ? a.pos0 + t0 + prow : kend - 1u;  // last key this column sees

  // q as the B operand (f16 high and low parts): column qi, k = 32 kk + 8 qq + e
  h8_t qh[KK], ql[KK];
#pragma unroll
  for (uint32_t kk = 0; kk < KK; ++kk) {
    float v[8];
    if (col_live) {
      const float* qp = a.attn_q + ((size_t)(t0 + prow) * a.q_heads + ph) * HD + 32u * kk + 8u * qq;
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
      qh[kk][e] = h;
      ql[kk][e] = (half_t)(v[e] - (float)h);
    }
  }

  float m_run = -INFINITY, l_run = 0.f;
  f4_t acc[NT];
#pragma unroll
  for (uint32_t tt = 0; tt < NT; ++tt) acc[tt] = f4_t{0.f, 0.f, 0.f, 0.f};
  const size_t hoff = (size_t)j * a.head_stride;
  // staging: thread t loads key row t >> 2, quarter t & 3 of its K row (f16 bytes in LDS), and
  // dimensions DPT (t & 7) .. + DPT - 1 of the key pair 2 (t >> 3), 2 (t >> 3) + 1 of V, which it
  // writes transposed (V^T[dimension][key], a u32 per dimension holding both keys) so that the
  // A operand of the P.V product (4 consecutive keys of one dimension) is one 8-byte read
  constexpr uint32_t QB = ROWB / 4u;  // f16 bytes per quarter row
  const uint32_t srow = t >> 2, squart = t & 3u;
  const uint32_t vpair = t >> 3, vd0 = DPT * (t & 7u);
  auto cache_row = [&](uint32_t key) -> size_t {
    return a.pages ? (size_t)a.pages[key / a.page] * a.page + key % a.page : (size_t)key;
  };
  for (uint32_t kb = 0; kb < kend; kb += KB) {
    {
      const uint32_t key = kb + srow;
      const bool live = key < kend;
      const size_t crow = live ? cache_row(key) : 0;
      const uint32_t vk0 = kb + 2u * vpair;
      const bool vlive0 = vk0 < kend, vlive1 = vk0 + 1u < kend;
      const size_t vrow0 = vlive0 ? cache_row(vk0) : 0, vrow1 = vlive1 ? cache_row(vk0 + 1u) : 0;
      uint16_t vt0[DPT], vt1[DPT];  // dimensions vd0 .. of the pair's two keys (f16 bits)
      if constexpr (KV8 == 0) {
        const unsigned char* kp =
            static_cast<const unsigned char*>(a.kv_k) + (crow * a.row_stride + hoff) * 2u + squart * QB;
#pragma unroll
        for (uint32_t i = 0; i < QB / 16u; ++i) {
          const u4_t kv = live ? *reinterpret_cast<const u4_t*>(kp + 16u * i) : u4_t{0u, 0u, 0u, 0u};
          *reinterpret_cast<u4_t*>(reinterpret_cast<unsigned char*>(sK + srow * KROW) + squart * QB + 16u * i) = kv;
        }
        const uint16_t* v0 = static_cast<const uint16_t*>(a.kv_v) + vrow0 * a.row_stride + hoff + vd0;
        const uint16_t* v1 = static_cast<const uint16_t*>(a.kv_v) + vrow1 * a.row_stride + hoff + vd0;
#pragma unroll
        for (uint32_t i = 0; i < DPT / 8u; ++i) {
          const u4_t x0 = vlive0 ? *reinterpret_cast<const u4_t*>(v0 + 8u * i) : u4_t{0u, 0u, 0u, 0u};
          const u4_t x1 = vlive1 ? *reinterpret_cast<const u4_t*>(v1 + 8u * i) : u4_t{0u, 0u, 0u, 0u};
#pragma unroll
          for (uint32_t e = 0; e < 4; ++e) {
            vt0[8u * i + 2u * e] = (uint16_t)(x0[e] & 0xFFFFu);
            vt0[8u * i + 2u * e + 1u] = (uint16_t)(x0[e] >> 16);
            vt1[8u * i + 2u * e] = (uint16_t)(x1[e] & 0xFFFFu);
            vt1[8u * i + 2u * e + 1u] = (uint16_t)(x1[e] >> 16);
          }
        }
      } else {
        const unsigned char* kp = static_cast<const unsigned char*>(a.kv_k) + crow * a.row_stride + hoff + squart * (QB / 2u);
#pragma unroll
        for (uint32_t i = 0; i < QB / 32u; ++i) {  // 16 int8 -> 32 bytes of f16
          const u4_t kv = live ? *reinterpret_cast<const u4_t*>(kp + 16u * i) : u4_t{0u, 0u, 0u, 0u};
          unsigned char* kd = reinterpret_cast<unsigned char*>(sK + srow * KROW) + squart * QB + 32u * i;
          *reinterpret_cast<u4_t*>(kd) = widen_i8x8(kv.x, kv.y);
          *reinterpret_cast<u4_t*>(kd + 16) = widen_i8x8(kv.z, kv.w);
        }
        const unsigned char* v0 = static_cast<const unsigned char*>(a.kv_v) + vrow0 * a.row_stride + hoff + vd0;
        const unsigned char* v1 = static_cast<const unsigned char*>(a.kv_v) + vrow1 * a.row_stride + hoff + vd0;
#pragma unroll
        for (uint32_t i = 0; i < DPT / 16u; ++i) {  // 16 int8 per load
          const u4_t x0 = vlive0 ? *reinterpret_cast<const u4_t*>(v0 + 16u * i) : u4_t{0u, 0u, 0u, 0u};
          const u4_t x1 = vlive1 ? *reinterpret_cast<const u4_t*>(v1 + 16u * i) : u4_t{0u, 0u, 0u, 0u};
          const u4_t w0[2] = {widen_i8x8(x0.x, x0.y), widen_i8x8(x0.z, x0.w)};
          const u4_t w1[2] = {widen_i8x8(x1.x, x1.y), widen_i8x8(x1.z, x1.w)};
#pragma unroll
          for (uint32_t h = 0; h < 2; ++h)
#pragma unroll
            for (uint32_t e = 0; e < 4; ++e) {
              vt0[16u * i + 8u * h + 2u * e] = (uint16_t)(w0[h][e] & 0xFFFFu);
              vt0[16u * i + 8u * h + 2u * e + 1u] = (uint16_t)(w0[h][e] >> 16);
              vt1[16u * i + 8u * h + 2u * e] = (uint16_t)(w1[h][e] & 0xFFFFu);
              vt1[16u * i + 8u * h + 2u * e + 1u] = (uint16_t)(w1[h][e] >> 16);
            }
        }
        if (squart == 0) {
          const size_t so = crow * a.sc_row_stride + (size_t)j * a.sc_head_stride;
          sKs[srow] = live ? h2f(a.k_scale[so]) : 0.f;
          sVs[srow] = live ? h2f(a.v_scale[so]) : 0.f;
        }
      }
#pragma unroll
      for (uint32_t d = 0; d < DPT; ++d)
        *reinterpret_cast<uint32_t*>(sVt + (vd0 + d) * VTP + 2u * vpair) = (uint32_t)vt0[d] | ((uint32_t)vt1[d] << 16);
    }
    lds_barrier();
#pragma unroll
    for (uint32_t grp = 0; grp < KB / 16u; ++grp) {
      const uint32_t g0 = kb + 16u * grp;
      if (g0 >= kend) break;  // uniform
      // scores S^T[key g0 + 4 qq + r][column qi]
      f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (uint32_t kk = 0; kk < KK; ++kk) {
        const h8_t kh = *reinterpret_cast<const h8_t*>(sK + (16u * grp + qi) * KROW + 32u * kk + 8u * qq);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[kk], d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, ql[kk], d, 0, 0, 0);
      }
      float sc[4];
      float mx = -INFINITY;
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) {
        const uint32_t key = g0 + 4u * qq + r;
        float rs = a.scale;
        if constexpr (KV8 == 1) rs = a.scale * sKs[16u * grp + 4u * qq + r];
        sc[r] = key <= lim ? d[r] * rs : -INFINITY;
        mx = fmaxf(mx, sc[r]);
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m_run, mx);  // finite: key 0 <= lim for every column
      const float alpha = expf(m_run - m_new);
      float w[4];
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) w[r] = expf(sc[r] - m_new);
      l_run = __builtin_fmaf(l_run, alpha, (w[0] + w[1]) + (w[2] + w[3]));
      m_run = m_new;
      if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (uint32_t tt = 0; tt < NT; ++tt) acc[tt] *= alpha;
      }
      h4_t bh, bl;
#pragma unroll
      for (uint32_t r = 0; r < 4; ++r) {
        float wv = w[r];
        if constexpr (KV8 == 1) wv *= sVs[16u * grp + 4u * qq + r];
        const half_t h = (half_t)wv;
        bh[r] = h;
        bl[r] = (half_t)(wv - (float)h);
      }
#pragma unroll
      for (uint32_t tt = 0; tt < NT; ++tt) {
        const h4_t av = *reinterpret_cast<const h4_t*>(sVt + (16u * tt + qi) * VTP + 16u * grp + 4u * qq);
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bh, acc[tt], 0, 0, 0);
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x16f16(av, bl, acc[tt], 0, 0, 0);
      }
    }
    lds_barrier();  // every wave is done with this iteration's keys before they are replaced
  }
  float l = l_run + __shfl_xor(l_run, 16, 64);
  l = l + __shfl_xor(l, 32, 64);
  if (col_live) {
    if constexpr (KV8 == 1) {
      float* op = a.out_rot + ((size_t)(t0 + prow) * a.q_heads + ph) * HD;
#pragma unroll
      for (uint32_t tt = 0; tt < NT; ++tt)
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r) op[16u * tt + 4u * qq + r] = acc[tt][r] / l;
    } else {
      uint16_t* op = a.attn_out + (size_t)(t0 + prow) * a.q_heads * HD + (size_t)ph * HD;
#pragma unroll
      for (uint32_t tt = 0; tt < NT; ++tt)
#pragma unroll
        for (uint32_t r = 0; r < 4; ++r) op[16u * tt + 4u * qq + r] = f2h(acc[tt][r] / l);
    }
  }
}

// grid (q_heads, T), 256 lanes: attn_reduce_v2_kv8's un-rotation (kv8.cl:814-860) of one
// (row, head) output, head_dim 256: unrotate(y) = FWHT(s * y) / 16, then f16
__global__ __launch_bounds__(256) void unrotate_rows_kernel(const float* __restrict__ in, uint16_t* __restrict__ out,
                                                            uint32_t q_heads) {
  __shared__ float xch[256];
  const uint32_t h = blockIdx.x, row = blockIdx.y, d = threadIdx.x;
  const size_t off = ((size_t)row * q_heads + h) * 256u;
  float v1[1] = {kv8_flip(in[off + d], kv8_sign_neg(d))};
  fwht256<1>(v1, d, xch);
  out[off + d] = f2h(v1[0] * 0.0625f);
}

template <int HD, int GQA, int KV8>
void launch_prefill_gqa(const PrefillAttnArgs& a, uint32_t kv_heads, hipStream_t st) {
  constexpr uint32_t RB = 64 / GQA;
  attn_prefill_kernel<HD, GQA, KV8><<<dim3(kv_heads, (a.T + RB - 1) / RB), 256, 0, st>>>(a);
}

template <int HD, int KV8>
int launch_prefill_attn(const PrefillAttnArgs& a, uint32_t gqa, uint32_t kv_heads, hipStream_t st) {
  switch (gqa) {
    case 1: launch_prefill_gqa<HD, 1, KV8>(a, kv_heads, st); return 0;
    case 2: launch_prefill_gqa<HD, 2, KV8>(a, kv_heads, st); return 0;
    case 4: launch_prefill_gqa<HD, 4, KV8>(a, kv_heads, st); return 0;
    case 5: launch_prefill_gqa<HD, 5, KV8>(a, kv_heads, st); return 0;
    case 6: launch_prefill_gqa<HD, 6, KV8>(a, kv_heads, st); return 0;
    case 8: launch_prefill_gqa<HD, 8, KV8>(a, kv_heads, st); return 0;
    default: return -1;
  }
}

// attn_prep for the chunk's rows (prep.cl attn_prep, attn.cl:361-372) with one wave per (head,
// row): grid (q_heads + 2 kv_heads, ceil(T / 4)), 256 lanes; wave w of work-group (hh, y) takes
// row 4 y + w of head hh (q heads, then k, then v), lane l elements l + 64 k. The chain is
// attn_prep's operation for operation on a one-slice fold (qkv [T][qkv_n] fp32): q/k rounded to
// f16, the RMSNorm with the 256-lane tree's order (a lane's own elements, then the 64-lane
// shuffle tree), RoPE's rotate_half pairs, q -> attn_q fp32, k and v -> the f16 cache row of
// position pos0 + t. No work-group barrier: the waves are independent.
template <int HD>
__global__ __launch_bounds__(256) void prep_rows_kernel(const float* __restrict__ qkv, uint32_t T, uint32_t pos0,
                                                        uint32_t q_heads, uint32_t kv_heads, uint32_t rot_dim,
                                                        uint32_t qkv_n, const float* __restrict__ q_norm,
                                                        const float* __restrict__ k_norm, const float* __restrict__ rope,
                                                        float* __restrict__ attn_q, uint16_t* __restrict__ kv_k,
                                                        uint16_t* __restrict__ kv_v, size_t row_stride, size_t head_stride,
                                                        const uint32_t* __restrict__ pages, uint32_t page, float eps) {
  constexpr uint32_t EPL = HD / 64u;
  __shared__ float s_row[4][HD];
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t hh = blockIdx.x, t = blockIdx.y * 4u + wave;
  if (t >= T) return;  // uniform per wave
  const bool is_q = hh < q_heads, is_k = !is_q && hh < q_heads + kv_heads;
  const uint32_t h = is_q ? hh : (is_k ? hh - q_heads : hh - q_heads - kv_heads);
  const float* src = qkv + (size_t)t * qkv_n + (size_t)hh * HD;  // q || k || v, HD columns per head
  const uint32_t p = pos0 + t;
  const size_t crow = pages ? (size_t)pages[p / page] * page + p % page : (size_t)p;
  float raw[EPL];
#pragma unroll
  for (uint32_t k = 0; k < EPL; ++k) raw[k] = src[lane + 64u * k];
  if (!is_q && !is_k) {
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) kv_v[crow * row_stride + h * head_stride + lane + 64u * k] = f2h(raw[k]);
    return;
  }
  const float* nw = is_q ? q_norm : k_norm;
  const uint32_t half = rot_dim / 2u;
  const float* cs = rope + (size_t)p * 2u * half;
  float wn[EPL], rc[EPL], rsn[EPL], xf[EPL], nv[EPL];
#pragma unroll
  for (uint32_t k = 0; k < EPL; ++k) {
    const uint32_t e = lane + 64u * k;
    wn[k] = nw ? nw[e] : 0.f;
    rc[k] = 1.f;
    rsn[k] = 0.f;
    if (e < rot_dim) {
      const uint32_t ii = e < half ? e : e - half;
      rc[k] = cs[ii];
      rsn[k] = cs[half + ii];
    }
    xf[k] = h2f(f2h(raw[k]));
  }
  if (nw) {
    float sq[EPL];
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) sq[k] = xf[k] * xf[k];
    float acc;
    if constexpr (EPL == 4) acc = (sq[0] + sq[2]) + (sq[1] + sq[3]);
    else acc = sq[0] + sq[1];
#pragma unroll
    for (int st = 32; st > 0; st >>= 1) acc += __shfl_down(acc, st, 64);
    const float tot = __shfl(acc, 0, 64);
    const float rstd = 1.0f / sqrtf(tot / (float)HD + eps);
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) nv[k] = h2f(f2h(xf[k] * rstd * wn[k]));
  } else {
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) nv[k] = xf[k];
  }
  float* nrm = s_row[wave];
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
    } else if (e < rot_dim) {
      const float tt = nrm[e - half] * rsn[k];
      out = __builtin_fmaf(nv[k], rc[k], tt);
    } else {
      out = nv[k];
    }
    if (is_q)
      attn_q[((size_t)t * q_heads + h) * HD + e] = out;
    else
      kv_k[crow * row_stride + h * head_stride + e] = f2h(out);
  }
}

// grid (T), 256 lanes: resid[t] = embed[ids[t]]; an id outside the table leaves the row and
// sets the flag word (the caller's host check rejects such ids before launching)
__global__ __launch_bounds__(256) void embed_rows_kernel(const uint32_t* __restrict__ ids,
                                                         const uint16_t* __restrict__ embed,
                                                         uint16_t* __restrict__ resid, uint32_t hidden,
                                                         uint32_t vocab, uint32_t* flag) {
  const uint32_t row = ids[blockIdx.x];
  if (row >= vocab) {
    if (threadIdx.x == 0 && flag) *flag = 0xDEAD0001u;
    return;
  }
  const u4_t* s4 = reinterpret_cast<const u4_t*>(embed + (size_t)row * hidden);
  u4_t* d4 = reinterpret_cast<u4_t*>(resid + (size_t)blockIdx.x * hidden);
  for (uint32_t k = threadIdx.x; k < hidden / 8u; k += 256u) d4[k] = s4[k];
}

}  // namespace
}  // namespace mi

using namespace mi;

// The work-group tile of the GEMM. Every tile sums a column over the k-groups in the same MFMA
// order, so the choice changes the speed only, never a bit of the result. For N a multiple of
// 256 the tile is a row of 4 waves of R x 64 (R = 128, 96 or 64): the larger R, the less
// dequantisation and fewer loads per MFMA (measured relative rates 1 : 0.93 : 0.85), the
// coarser the grid. The choice minimises the rows the busiest CU works through over that rate,
// ceil(work-groups / CUs) R / rate: 128 rows for the qkv and gate||up linears of a long chunk,
// 96 for o and down, 64 for short chunks. Otherwise 128 x 128 (2 x 2 waves of 64 x 64).
template <bool SILU>
static int launch_gemm(const char* name, const uint32_t* qweight, const uint16_t* scales, const uint16_t* x,
                       float* out, uint16_t* h, uint32_t T, uint32_t K, uint32_t N, void* stream) {
  if (!qweight || !scales || !x || (!out && !h) || T == 0) return mi_fail(MI_ERR_ARG, (std::string(name) + ": bad arguments").c_str());
  if (K == 0 || K % GBK || N == 0 || N % 128u)
    return mi_fail(MI_ERR_SHAPE, (std::string(name) + ": K must be a multiple of 64 and N of 128").c_str());
  if (reinterpret_cast<uintptr_t>(qweight) % 16 || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(scales) % 8)
    return mi_fail(MI_ERR_ARG, (std::string(name) + ": qweight/x need 16-byte, scales 8-byte alignment").c_str());
  if ((T + 63u) / 64u > 65535u) return mi_fail(MI_ERR_SHAPE, (std::string(name) + ": too many rows").c_str());
  // the kernels' buffer loads take 32-bit byte offsets: x (with the last tile's rows past T) and
  // the packed weights stay below 2 GiB
  if (((uint64_t)T + 128u) * K * 2u >= (1ull << 31) || (uint64_t)K * N / 2u >= (1ull << 31))
    return mi_fail(MI_ERR_SHAPE, (std::string(name) + ": x or qweight beyond 2 GiB").c_str());
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return mi_hip((int)hipGetLastError(), name);
  hipStream_t st = (hipStream_t)stream;
  if (N % 256u == 0) {
    const uint64_t C = (uint64_t)(cus > 0 ? cus : 1);
    auto cost = [&](uint32_t R, uint64_t rate) {  // rows on the busiest CU x 100 / rate (percent)
      const uint64_t wg = (uint64_t)(N / 256u) * ((T + R - 1u) / R);
      return (wg + C - 1u) / C * R * 10000u / rate;
    };
    const uint64_t c128 = cost(128u, 100u), c96 = cost(96u, 93u), c64 = cost(64u, 85u);
    if (c128 <= c96 && c128 <= c64)
      gemm_w4a16_kernel<SILU, 1, 8, 2><<<dim3(N / 256u, (T + 127u) / 128u), 256, 0, st>>>(qweight, scales, x, out,
                                                                                          h, T, K, N);
    else if (c96 <= c64)
      gemm_w4a16_kernel<SILU, 1, 6, 2><<<dim3(N / 256u, (T + 95u) / 96u), 256, 0, st>>>(qweight, scales, x, out, h,
                                                                                         T, K, N);
    else
      gemm_w4a16_kernel<SILU, 1, 4, 1><<<dim3(N / 256u, (T + 63u) / 64u), 256, 0, st>>>(qweight, scales, x, out, h,
                                                                                         T, K, N);
  } else {
    gemm_w4a16_kernel<SILU, 2, 4, 1><<<dim3(N / 128u, (T + 127u) / 128u), 256, 0, st>>>(qweight, scales, x, out, h,
                                                                                         T, K, N);
  }
  return mi_hip((int)hipGetLastError(), name);
}

extern "C" {

int mi_gemm_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x, float* out, uint32_t T,
                  uint32_t K, uint32_t N, void* stream) {
  return launch_gemm<false>("gemm_w4a16", qweight, scales, x, out, nullptr, T, K, N, stream);
}

int mi_gemm_w4a16_silu(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x, uint16_t* h, uint32_t T,
                       uint32_t K, uint32_t N, void* stream) {
  if (!h) return mi_fail(MI_ERR_ARG, "gemm_w4a16_silu: bad arguments");
  return launch_gemm<true>("gemm_w4a16_silu", qweight, scales, x, nullptr, h, T, K, N, stream);
}

int mi_moe_prefill(const uint32_t* route, const uint16_t* x, const uint32_t* gu_blocks, const uint32_t* dn_blocks,
                   uint16_t* resid, uint32_t T, uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                   uint32_t* list, uint32_t* tiles, uint32_t* tiles_n, uint16_t* h, uint16_t* d, void* stream) {
  if (!route || !x || !gu_blocks || !dn_blocks || !resid || !list || !tiles || !tiles_n || !h || !d)
    return mi_fail(MI_ERR_ARG, "moe_prefill: null pointer");
  if (T == 0 || T > 2048u) return mi_fail(MI_ERR_SHAPE, "moe_prefill: T must be 1..2048");
  if (experts < 16 || experts > 256 || (experts & (experts - 1)))
    return mi_fail(MI_ERR_SHAPE, "moe_prefill: experts must be a power of two in [16, 256]");
  if (top_k < 1 || top_k > 8) return mi_fail(MI_ERR_SHAPE, "moe_prefill: top_k must be 1..8");
  if (hidden == 0 || hidden % 512 || hidden > 4096)
    return mi_fail(MI_ERR_SHAPE, "moe_prefill: hidden must be a multiple of 512 up to 4096");
  if (inter == 0 || inter % 128 || inter > 1024)
    return mi_fail(MI_ERR_SHAPE, "moe_prefill: inter must be a multiple of 128 up to 1024");
  if (reinterpret_cast<uintptr_t>(tiles) % 16 || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(h) % 16 || reinterpret_cast<uintptr_t>(gu_blocks) % 4 ||
      reinterpret_cast<uintptr_t>(dn_blocks) % 4)
    return mi_fail(MI_ERR_ARG, "moe_prefill: tiles, x and h need 16-byte, gu_blocks and dn_blocks 4-byte alignment");
  const uint32_t slots = top_k + 1, P = T * slots;
  const uint32_t max_tiles = (P + kMoeRows - 1u) / kMoeRows + experts + 1u;
  const size_t gu_block = (size_t)(2u * inter / 16u) * (hidden / GBK) * kMoeTile;
  const size_t dn_block = (size_t)(hidden / 16u) * (inter / GBK) * kMoeTile;
  hipStream_t st = (hipStream_t)stream;
  u4_t* tl = reinterpret_cast<u4_t*>(tiles);
  moe_group_kernel<<<1, 1024, 0, st>>>(route, T, experts, top_k, list, tl, tiles_n);
  moe_gemm_kernel<true><<<dim3(2u * inter / 256u, max_tiles), 256, 0, st>>>(tl, tiles_n, list, gu_blocks, gu_block,
                                                                            x, T, h, nullptr, slots, hidden,
                                                                            2u * inter);
  moe_gemm_kernel<false><<<dim3(hidden / 256u, max_tiles), 256, 0, st>>>(tl, tiles_n, list, dn_blocks, dn_block, h,
                                                                          P, nullptr, d, slots, inter, hidden);
  moe_combine_kernel<<<dim3(hidden / 256u, T), 256, 0, st>>>(route, d, resid, top_k, hidden);
  return mi_hip((int)hipGetLastError(), "moe_prefill");
}

int mi_attn_prefill(const float* attn_q, const uint16_t* kv_k, const uint16_t* kv_v, size_t row_stride,
                    size_t head_stride, const uint32_t* pages, uint32_t page, uint32_t T, uint32_t pos0,
                    const mi_attn_shape* shape, uint16_t* attn_out, void* stream) {
  if (!attn_q || !kv_k || !kv_v || !attn_out || !shape || T == 0)
    return mi_fail(MI_ERR_ARG, "attn_prefill: bad arguments");
  if (shape->act) return mi_fail(MI_ERR_SHAPE, "attn_prefill: f16 activations only");
  const uint32_t HD = shape->head_dim;
  if (HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_prefill: head_dim must be 128 or 256");
  const uint32_t gqa = shape->kv_heads ? shape->q_heads / shape->kv_heads : 0;
  if (shape->kv_heads == 0 || shape->q_heads % shape->kv_heads ||
      !(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 5 || gqa == 6 || gqa == 8))
    return mi_fail(MI_ERR_SHAPE, "attn_prefill: q_heads / kv_heads must be 1, 2, 4, 5, 6 or 8");
  if (pages && page == 0) return mi_fail(MI_ERR_ARG, "attn_prefill: page size 0");
  if ((row_stride % 8) || (head_stride % 8))
    return mi_fail(MI_ERR_ARG, "attn_prefill: KV strides must keep 8-element alignment");
  PrefillAttnArgs a{attn_q, kv_k, kv_v, pages, attn_out, row_stride, head_stride, page, T, pos0,
                    shape->q_heads, shape->scale, nullptr, nullptr, 0, 0, nullptr};
  hipStream_t st = (hipStream_t)stream;
  const int r = HD == 128 ? launch_prefill_attn<128, 0>(a, gqa, shape->kv_heads, st)
                          : launch_prefill_attn<256, 0>(a, gqa, shape->kv_heads, st);
  if (r) return mi_fail(MI_ERR_SHAPE, "attn_prefill: unsupported GQA");
  return mi_hip((int)hipGetLastError(), "attn_prefill");
}

int mi_attn_prefill_kv8(const float* attn_q, const int8_t* kv_k, const int8_t* kv_v, const uint16_t* k_scale,
                        const uint16_t* v_scale, size_t row_stride, size_t head_stride, size_t sc_row_stride,
                        size_t sc_head_stride, const uint32_t* pages, uint32_t page, uint32_t T, uint32_t pos0,
                        const mi_attn_shape* shape, float* out_rot, uint16_t* attn_out, void* stream) {
  if (!attn_q || !kv_k || !kv_v || !k_scale || !v_scale || !out_rot || !attn_out || !shape || T == 0)
    return mi_fail(MI_ERR_ARG, "attn_prefill_kv8: bad arguments");
  if (shape->act) return mi_fail(MI_ERR_SHAPE, "attn_prefill_kv8: f16 activations only");
  if (shape->head_dim != 256) return mi_fail(MI_ERR_SHAPE, "attn_prefill_kv8: the rotation is defined for head_dim 256");
  const uint32_t gqa = shape->kv_heads ? shape->q_heads / shape->kv_heads : 0;
  if (shape->kv_heads == 0 || shape->q_heads % shape->kv_heads ||
      !(gqa == 1 || gqa == 2 || gqa == 4 || gqa == 5 || gqa == 6 || gqa == 8))
    return mi_fail(MI_ERR_SHAPE, "attn_prefill_kv8: q_heads / kv_heads must be 1, 2, 4, 5, 6 or 8");
  if (pages && page == 0) return mi_fail(MI_ERR_ARG, "attn_prefill_kv8: page size 0");
  if ((row_stride % 16) || (head_stride % 16))
    return mi_fail(MI_ERR_ARG, "attn_prefill_kv8: int8 KV strides must keep 16-byte alignment");
  PrefillAttnArgs a{attn_q, kv_k, kv_v, pages, attn_out, row_stride, head_stride, page, T, pos0,
                    shape->q_heads, shape->scale, k_scale, v_scale, sc_row_stride, sc_head_stride, out_rot};
  hipStream_t st = (hipStream_t)stream;
  if (launch_prefill_attn<256, 1>(a, gqa, shape->kv_heads, st))
    return mi_fail(MI_ERR_SHAPE, "attn_prefill_kv8: unsupported GQA");
  int e = (int)hipGetLastError();
  if (e) return mi_hip(e, "attn_prefill_kv8");
  unrotate_rows_kernel<<<dim3(shape->q_heads, T), 256, 0, st>>>(out_rot, attn_out, shape->q_heads);
  return mi_hip((int)hipGetLastError(), "attn_prefill_kv8 unrotate");
}

int mi_attn_prep_rows(const float* qkv, uint32_t T, uint32_t pos0, const mi_attn_shape* shape, const float* q_norm,
                      const float* k_norm, const float* rope, float* attn_q, uint16_t* kv_k, uint16_t* kv_v,
                      size_t row_stride, size_t head_stride, const uint32_t* pages, uint32_t page, void* stream) {
  if (!qkv || !shape || !rope || !attn_q || !kv_k || !kv_v || T == 0)
    return mi_fail(MI_ERR_ARG, "attn_prep_rows: bad arguments");
  if (shape->act) return mi_fail(MI_ERR_SHAPE, "attn_prep_rows: f16 activations only");
  const uint32_t HD = shape->head_dim;
  if (HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_prep_rows: head_dim must be 128 or 256");
  if (shape->gated || shape->kv_heads == 0 || shape->k_off != shape->q_heads * HD ||
      shape->v_off != (shape->q_heads + shape->kv_heads) * HD || shape->qkv_n != shape->v_off + shape->kv_heads * HD)
    return mi_fail(MI_ERR_SHAPE, "attn_prep_rows: a plain q||k||v layout (not gated)");
  if (shape->rot_dim > HD || shape->rot_dim % 2) return mi_fail(MI_ERR_SHAPE, "attn_prep_rows: bad rot_dim");
  if (pages && page == 0) return mi_fail(MI_ERR_ARG, "attn_prep_rows: page size 0");
  const dim3 grid(shape->q_heads + 2 * shape->kv_heads, (T + 3) / 4);
  hipStream_t st = (hipStream_t)stream;
  if (HD == 128)
    prep_rows_kernel<128><<<grid, 256, 0, st>>>(qkv, T, pos0, shape->q_heads, shape->kv_heads, shape->rot_dim,
                                                shape->qkv_n, q_norm, k_norm, rope, attn_q, kv_k, kv_v, row_stride,
                                                head_stride, pages, page, shape->eps);
  else
    prep_rows_kernel<256><<<grid, 256, 0, st>>>(qkv, T, pos0, shape->q_heads, shape->kv_heads, shape->rot_dim,
                                                shape->qkv_n, q_norm, k_norm, rope, attn_q, kv_k, kv_v, row_stride,
                                                head_stride, pages, page, shape->eps);
  return mi_hip((int)hipGetLastError(), "attn_prep_rows");
}

int mi_embed_rows(const uint32_t* ids, const uint16_t* embed, uint16_t* resid, uint32_t T, uint32_t hidden,
                  uint32_t vocab, uint32_t* flag, void* stream) {
  if (!ids || !embed || !resid || T == 0 || hidden == 0 || hidden % 8)
    return mi_fail(MI_ERR_ARG, "embed_rows: bad arguments (hidden a multiple of 8)");
  embed_rows_kernel<<<T, 256, 0, (hipStream_t)stream>>>(ids, embed, resid, hidden, vocab, flag);
  return mi_hip((int)hipGetLastError(), "embed_rows");
}

}  // extern "C"
