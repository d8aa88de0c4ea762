// gemv_w4a16.hip - the W4A16 GPTQ group-64 linear for M = 1..16 rows on gfx950.
//
// Replaces the reference's `gemv` (src/kernels/gemv.cl:124-221) and, for M >= 2, its
// small-M `gemm_sm` (src/kernels/gemm_sm.cl:161): same operands and the same output
// contract - fp32 split-K partials [S][M][N] that the consumer folds in slice order
// (tests/kernels/gemm_sm_ref.h:106-136) - with an MI355X-native inner loop.
//
// Weights stay in GPTQ layout 0 (qweight u32 [K/8][N], nibble i of word (r, n) is
// k = 8r + i; scales f16 [K/64][N]; zero point 8), which already streams coalesced:
//
//   * A work-group is 4 wave64s on one 64-column tile; grid (N / 64, S). Slice s owns
//     k-groups [s G/S, (s+1) G/S); wave w takes every 4th of them.
//   * Lane l reads one 16-byte uint4 = 4 adjacent columns (n0 + 4 (l % 16) .. + 3) of word
//     row (l / 16) of a 4-row quarter group: each 16-lane quarter-wave reads 256 contiguous
//     bytes, the wave 1 KB, with non-temporal loads (weights are read once per token).
//   * The contraction runs on the matrix cores: v_mfma_f32_16x16x32_f16 with A = the M
//     activation rows (zero-padded to 16) and B = 32 k x 16 columns of dequantised
//     weights. Lane l's B operand is exactly its word: 8 consecutive k of one column, so
//     the dequant is register-local - two v_and_or_b32 of the word (and of word >> 8)
//     against the fp16 magic 0x6400 give (1024 + q) or (1024 + 16 q) in each half, and
//     one packed f16 add / fma takes them to q - 8 exactly. The halves come out paired
//     (k0,k4)(k1,k5)(k2,k6)(k3,k7); the activation octet is permuted the same way
//     (v_perm_b32), so the MFMA sums the right products.
//   * Per k-group the 16x16 fp32 tile starts from zero, then acc = fma(tile, scale, acc)
//     per column (the reference's acc += gacc * scale per group); the 4 waves' partials
//     are summed in wave order through LDS and written as one slice.
//
// Property R (gemm_sm.cl:36-41): row m's result does not depend on M or on the other
// rows - every output element is its own MFMA dot and the same fixed merges - so S and
// the wave split are functions of the shape only (mi_gemv_pick_s).
//
// Fused epilogues (mi_gemv_w4a16_ex). The work-groups of one 64-column tile count
// themselves in a self-resetting counter; the last one to finish folds the tile's S
// partials in ascending s (the consumer's fold of gemv.cl:1-10, so the result does not
// depend on which work-group is last) and applies the step's next operation:
//   RESID   resid = rne(resid + rne(sum_s part)) and the tile's sum of squares (the
//           reference's res_fold at 64-element chunks, prep_ref.h:120-156); the last tile
//           of the launch then forms rstd = 1/sqrt(sum_g sumsq / N + eps) and the next
//           RMSNorm's x = rne(r * rstd * w) (norm_finish, prep_ref.h:158-168);
//   SILU    h = rne(rne(silu(rne(g))) * rne(u)) over the interleave16 gate||up columns
//           (prep_silu_mul, prep_ref.h:170-189);
//   LOGITS  fp32 logits and the tile's (max, lowest index) for argmax_stage2
//           (argmax.cl:63-65's comparator; the vocab_used mask).
// Hand-off between the work-groups of one launch: the partials, the tiles' sums of squares
// and the folded residual are written and read with device-coherent (sc1) accesses; each
// thread waits for its own stores to complete before the work-group increments the
// counter (a relaxed device-scope integer atomic), so the last arrival reads complete data.
// No whole-L2 writeback or invalidate is needed (an agent-scope fence would emit both in
// every work-group). No float atomics: replays stay bitwise identical.
#include "mi_common.h"
#include "mi_capi_internal.h"

namespace mi {
namespace {

constexpr int kWaves = 4;
constexpr int kCols = 64;

// 8 dequantised int4 weights of one word, in the pair order (q0,q4)(q1,q5)(q2,q6)(q3,q7).
__device__ __forceinline__ h8_t dequant_word(uint32_t w, uint32_t m_lo, uint32_t m_hi,
                                             uint32_t magic) {
  const h2_t b1032 = {(half_t)1032.0f, (half_t)1032.0f};
  const h2_t s16 = {(half_t)0.0625f, (half_t)0.0625f};
  const h2_t b72 = {(half_t)-72.0f, (half_t)-72.0f};
  const uint32_t t = w >> 8;
  const h2_t p0 = as_h2(and_or(w, m_lo, magic)) - b1032;                          // 1024+q   -> q-8
  const h2_t p1 = __builtin_elementwise_fma(as_h2(and_or(w, m_hi, magic)), s16, b72);  // 1024+16q -> q-8
  const h2_t p2 = as_h2(and_or(t, m_lo, magic)) - b1032;
  const h2_t p3 = __builtin_elementwise_fma(as_h2(and_or(t, m_hi, magic)), s16, b72);
  return h8_t{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

// 8 natural-order activations (x0..x7 in four u32) into the same pair order.
__device__ __forceinline__ h8_t perm_x(u4_t v) {
  const uint32_t a0 = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);  // (x0, x4)
  const uint32_t a1 = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);  // (x1, x5)
  const uint32_t a2 = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);  // (x2, x6)
  const uint32_t a3 = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);  // (x3, x7)
  const h2_t b0 = as_h2(a0), b1 = as_h2(a1), b2 = as_h2(a2), b3 = as_h2(a3);
  return h8_t{b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
}

struct GemvEpi {
  uint32_t* counters;     // >= N/64 + 1 words, zero between launches
  uint16_t* resid;        // RESID: [M][N]
  float* sumsq;           // RESID: [N/64][M]
  float* rstd;            // RESID: [M]
  const float* next_w;    // RESID: the next RMSNorm's fp32 weights [N]
  uint16_t* x_next;       // RESID: [M][N]
  uint16_t* h;            // SILU: [M][N/2]
  float* out32;           // LOGITS: [M][N]
  u2_t* argmax_part;      // LOGITS: [M][N/64] (value bits, index), or NULL
  uint32_t vocab_used;    // LOGITS
  float eps;              // RESID
  uint16_t* out16;        // F16OUT: [M][N]
};

enum { EPI_PARTIALS = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_LOGITS = 3, EPI_F16OUT = 4 };

// argmax.cl:63-65: strictly greater wins, an exact tie keeps the lower index
__device__ __forceinline__ bool better(float av, uint32_t ai, float bv, uint32_t bi) {
  return (av > bv) || (av == bv && ai < bi);
}

// true in the work-group that arrives last at counter `c` (`total` arrivals); resets it.
// Callers write everything the last arrival reads with st_agent before calling.
__device__ __forceinline__ bool last_arrival(uint32_t* c, uint32_t total, uint32_t* s_flag) {
  wait_memory();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = prev == total - 1u;
    if (*s_flag) st_agent(c, 0u);
  }
  __syncthreads();
  return *s_flag != 0u;
}

// MR: row capacity (1, 4 or 16); U: k-groups whose loads are issued together; EPI: epilogue.
template <int MR, int U, int EPI>
__global__ __launch_bounds__(256) void gemv_w4a16_kernel(const uint32_t* __restrict__ qweight,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ x,
                                                         float* __restrict__ partials, uint32_t M,
                                                         uint32_t K, uint32_t N, uint32_t gps,
                                                         GemvEpi epi) {
  constexpr int RR = MR < 4 ? MR : 4;  // accumulator rows a lane holds (rows 4*(l/16) + r)
  __shared__ float red[kWaves][MR][kCols];
  __shared__ uint32_t s_flag;

  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t c4 = lane & 15u, q = lane >> 4;
  const uint32_t n0 = blockIdx.x * kCols;
  const uint32_t ncol = n0 + 4u * c4;
  const uint32_t s = blockIdx.y;
  const uint32_t g_begin = s * gps + wave;
  const uint32_t g_end = (s + 1) * gps;
  const bool xrow = c4 < M;  // this lane feeds activation row c4 of the A operand

  const uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u, magic = 0x64006400u;

  float acc[4][RR];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < RR; ++r) acc[c][r] = 0.f;

  for (uint32_t g0 = g_begin; g0 < g_end; g0 += kWaves * U) {
    u4_t wv[U][2];
    u2_t sv[U];
    u4_t xv[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = g0 + u * kWaves;
      if (g < g_end) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t row = g * 8u + 4u * h + q;
          wv[u][h] = load_stream16(qweight + (size_t)row * N + ncol);
          if (xrow)
            xv[u][h] = *reinterpret_cast<const u4_t*>(x + (size_t)c4 * K + g * 64u + 32u * h + 8u * q);
          else
            xv[u][h] = u4_t{0u, 0u, 0u, 0u};
        }
        sv[u] = *reinterpret_cast<const u2_t*>(scales + (size_t)g * N + ncol);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = g0 + u * kWaves;
      if (g < g_end) {
        f4_t d[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const h8_t a = perm_x(xv[u][h]);
          const uint32_t ws[4] = {wv[u][h].x, wv[u][h].y, wv[u][h].z, wv[u][h].w};
#pragma unroll
          for (int c = 0; c < 4; ++c)
            d[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, dequant_word(ws[c], m_lo, m_hi, magic), d[c], 0, 0, 0);
        }
        const float sc[4] = {h2f((uint16_t)(sv[u].x & 0xFFFFu)), h2f((uint16_t)(sv[u].x >> 16)),
                             h2f((uint16_t)(sv[u].y & 0xFFFFu)), h2f((uint16_t)(sv[u].y >> 16))};
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int r = 0; r < RR; ++r) acc[c][r] = __builtin_fmaf(d[c][r], sc[c], acc[c][r]);
      }
    }
  }

  // Lane l holds rows 4 q + r of columns ncol .. ncol+3: stage them, then sum the waves.
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    const uint32_t row = 4u * q + r;
    if (row < (uint32_t)MR) {
#pragma unroll
      for (int c = 0; c < 4; ++c) red[wave][row][4u * c4 + c] = acc[c][r];
    }
  }
  __syncthreads();
  const uint32_t total = M * kCols;
  for (uint32_t i = threadIdx.x; i < total; i += 256u) {
    const uint32_t row = i / kCols, col = i % kCols;
    float v = red[0][row][col];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += red[w][row][col];
    if constexpr (EPI == EPI_PARTIALS)
      partials[((size_t)s * M + row) * N + n0 + col] = v;
    else
      st_agent(partials + ((size_t)s * M + row) * N + n0 + col, v);
  }
  if constexpr (EPI == EPI_PARTIALS) return;

  // ---- the tile's last work-group folds the S partials and applies the epilogue ----
  const uint32_t S = gridDim.y, tile = blockIdx.x, ntiles = gridDim.x;
  if (!last_arrival(epi.counters + tile, S, &s_flag)) return;
  const uint32_t t = threadIdx.x;
  // sum_s partials[s][row][n] from 0.f in ascending s; the loads go out 8 at a time
  auto fold = [&](uint32_t row, uint32_t n) {
    const float* p = partials + (size_t)row * N + n;
    const size_t step = (size_t)M * N;
    float a = 0.f;
    uint32_t ss = 0;
    for (; ss + 8 <= S; ss += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = ld_agent(p + (ss + u) * step);
#pragma unroll
      for (int u = 0; u < 8; ++u) a += v[u];
    }
    for (; ss < S; ++ss) a += ld_agent(p + ss * step);
    return a;
  };
  if constexpr (EPI == EPI_RESID) {
    // one row per wave per pass, a column per lane; the 64-lane tree is the reference's
    // 256-lane tree over a 64-element chunk (lanes 64..255 add exact zeros)
    for (uint32_t row = wave; row < M; row += kWaves) {
      const uint32_t n = n0 + lane;
      uint16_t* rp = epi.resid + (size_t)row * N + n;
      const uint16_t rb = f2h(h2f(*rp) + h2f(f2h(fold(row, n))));
      st_agent(rp, rb);
      const float v = h2f(rb);
      float a = __builtin_fmaf(v, v, 0.f);
#pragma unroll
      for (int st = 32; st > 0; st >>= 1) a += __shfl_down(a, st, 64);
      if (lane == 0) st_agent(epi.sumsq + (size_t)tile * M + row, a);
    }
    // the launch's last tile: rstd per row and the next norm's input
    if (!last_arrival(epi.counters + ntiles, ntiles, &s_flag)) return;
    // the tiles' sums, loaded in parallel, then added in ascending tile order
    __shared__ __align__(16) float s_ss[1024];
    __shared__ float s_rstd[16];
    for (uint32_t row = 0; row < M; ++row) {
      for (uint32_t g = t; g < ntiles; g += 256u) s_ss[g] = ld_agent(epi.sumsq + (size_t)g * M + row);
      __syncthreads();
      if (t == 0) {
        float tot = 0.f;
        uint32_t g = 0;
        for (; g + 16u <= ntiles; g += 16u) {
          f4_t v[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const f4_t*>(s_ss + g + 4u * u);
#pragma unroll
          for (int u = 0; u < 4; ++u) tot = ((tot + v[u][0]) + v[u][1] + v[u][2]) + v[u][3];
        }
        for (; g < ntiles; ++g) tot += s_ss[g];
        const float r = 1.0f / sqrtf(tot / (float)N + epi.eps);
        s_rstd[row] = r;
      }
      __syncthreads();
    }
    for (uint32_t row = 0; row < M; ++row) {
      const float r = s_rstd[row];
      const uint16_t* rr = epi.resid + (size_t)row * N;
      uint16_t* xo = epi.x_next + (size_t)row * N;
      const uint32_t nq = N / 4u;
      const uint64_t* rq = reinterpret_cast<const uint64_t*>(rr);
      for (uint32_t q0 = t; q0 < nq; q0 += 8u * 256u) {
        uint64_t v[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) v[u] = ld_agent(rq + min(q0 + u * 256u, nq - 1u));
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
          const uint32_t q = q0 + u * 256u;
          if (q < nq) {
            const f4_t wv = *reinterpret_cast<const f4_t*>(epi.next_w + 4u * q);
            uint64_t o = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              o |= (uint64_t)f2h(h2f((uint16_t)(v[u] >> (16 * j))) * r * wv[j]) << (16 * j);
            reinterpret_cast<uint64_t*>(xo)[q] = o;
          }
        }
      }
    }
    // rstd goes out last: a global store before a barrier would make the barrier wait for it
    if (t < M) epi.rstd[t] = s_rstd[t];
  } else if constexpr (EPI == EPI_SILU) {
    // 64 interleave16 columns = 32 outputs k = 32 tile + i (gate at gflat, up at gflat + 16)
    for (uint32_t i = t; i < 32u * M; i += 256u) {
      const uint32_t row = i / 32u, k = tile * 32u + i % 32u;
      const uint32_t gflat = (k / 16u) * 32u + (k % 16u);
      const uint16_t g_b = f2h(fold(row, gflat)), u_b = f2h(fold(row, gflat + 16u));
      const uint16_t s_b = f2h(silu_f32(h2f(g_b)));
      epi.h[(size_t)row * (N / 2) + k] = f2h(h2f(s_b) * h2f(u_b));
    }
  } else if constexpr (EPI == EPI_F16OUT) {
    for (uint32_t row = wave; row < M; row += kWaves) {
      const uint32_t n = n0 + lane;
      epi.out16[(size_t)row * N + n] = f2h(fold(row, n));
    }
  } else if constexpr (EPI == EPI_LOGITS) {
    for (uint32_t row = wave; row < M; row += kWaves) {
      const uint32_t n = n0 + lane;
      const float v = fold(row, n);
      epi.out32[(size_t)row * N + n] = v;
      if (epi.argmax_part) {
        float bv = n < epi.vocab_used ? v : -INFINITY;
        uint32_t bi = n;
#pragma unroll
        for (int st = 32; st > 0; st >>= 1) {
          const float ov = __shfl_down(bv, st, 64);
          const uint32_t oi = __shfl_down(bi, st, 64);
          if (lane + st < 64 && better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
          }
        }
        if (lane == 0)
          epi.argmax_part[(size_t)row * ntiles + tile] = u2_t{__builtin_bit_cast(uint32_t, bv), bi};
      }
    }
  }
}

// out[m][n] (fp16 or fp32) = sum over s ascending of partials[s][m][n], from 0.f.
__global__ __launch_bounds__(256) void fold_partials_kernel(const float* __restrict__ partials,
                                                            uint16_t* __restrict__ out16,
                                                            float* __restrict__ out32,
                                                            uint32_t S, uint32_t MN) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= MN) return;
  float t = 0.f;
  for (uint32_t s = 0; s < S; ++s) t += partials[(size_t)s * MN + i];
  if (out16) out16[i] = f2h(t);
  if (out32) out32[i] = t;
}

template <int MR, int EPI>
int launch_gemv(const uint32_t* qw, const uint16_t* sc, const uint16_t* x, float* part, uint32_t M,
                uint32_t K, uint32_t N, uint32_t S, const GemvEpi& epi, hipStream_t st) {
  const uint32_t G = K / 64, gps = G / S;
  dim3 grid(N / kCols, S);
  if (gps >= 16)
    gemv_w4a16_kernel<MR, 4, EPI><<<grid, 256, 0, st>>>(qw, sc, x, part, M, K, N, gps, epi);
  else
    gemv_w4a16_kernel<MR, 2, EPI><<<grid, 256, 0, st>>>(qw, sc, x, part, M, K, N, gps, epi);
  return (int)hipGetLastError();
}

template <int EPI>
int launch_rows(const uint32_t* qw, const uint16_t* sc, const uint16_t* x, float* part, uint32_t M,
                uint32_t K, uint32_t N, uint32_t S, const GemvEpi& epi, hipStream_t st) {
  if (M == 1) return launch_gemv<1, EPI>(qw, sc, x, part, M, K, N, S, epi, st);
  if (M <= 4) return launch_gemv<4, EPI>(qw, sc, x, part, M, K, N, S, epi, st);
  return launch_gemv<16, EPI>(qw, sc, x, part, M, K, N, S, epi, st);
}

int check_gemv(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x, const float* partials,
               uint32_t M, uint32_t K, uint32_t N, uint32_t S) {
  if (!qweight || !scales || !x || !partials) return mi_fail(MI_ERR_ARG, "gemv_w4a16: null pointer");
  if (M < 1 || M > 16) return mi_fail(MI_ERR_SHAPE, "gemv_w4a16: M must be 1..16");
  if (K == 0 || K % 64 || N == 0 || N % 64)
    return mi_fail(MI_ERR_SHAPE, "gemv_w4a16: K and N must be non-zero multiples of 64");
  if (S == 0 || (K / 64) % S) return mi_fail(MI_ERR_SHAPE, "gemv_w4a16: S must divide K/64");
  if (reinterpret_cast<uintptr_t>(qweight) % 16 || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(scales) % 8)
    return mi_fail(MI_ERR_ARG, "gemv_w4a16: qweight/x need 16-byte, scales 8-byte alignment");
  return 0;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" uint32_t mi_gemv_pick_s(uint32_t K, uint32_t N) {
  // The split-K width for a plain launch (measured on MI355X over the 27B shapes at M = 1):
  // the smallest S | K/64 that gives at most 8 k-groups per split and at least 2048
  // work-groups, never going below 4 k-groups per split.
  const uint32_t G = K / 64, tiles = N / kCols;
  uint32_t best = 1;
  for (uint32_t S = 1; S <= G; ++S) {
    if (G % S) continue;
    const uint32_t gps = G / S;
    if (gps < 4 && S > 1) break;
    best = S;
    if (gps <= 8 && tiles * S >= 2048) break;
  }
  return best;
}

extern "C" uint32_t mi_gemv_pick_s_ex(uint32_t K, uint32_t N, uint32_t epilogue) {
  // A fused epilogue's last work-group per tile folds S partials with device-coherent
  // loads, so larger S lengthens the launch's serial tail; the fused launches keep S at the
  // largest divisor of K/64 no larger than 8 (and no larger than the plain choice).
  const uint32_t plain = mi_gemv_pick_s(K, N);
  if (epilogue == MI_EPI_PARTIALS) return plain;
  const uint32_t G = K / 64, cap = plain < 8u ? plain : 8u;
  uint32_t best = 1;
  for (uint32_t S = 1; S <= cap; ++S)
    if (G % S == 0) best = S;
  return best;
}

extern "C" int mi_gemv_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x,
                             float* partials, uint32_t M, uint32_t K, uint32_t N, uint32_t S,
                             void* stream) {
  if (int e = check_gemv(qweight, scales, x, partials, M, K, N, S)) return e;
  const GemvEpi none{};
  return mi_hip(launch_rows<EPI_PARTIALS>(qweight, scales, x, partials, M, K, N, S, none,
                                          static_cast<hipStream_t>(stream)),
                "gemv_w4a16 launch");
}

extern "C" int mi_gemv_w4a16_ex(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x,
                                float* partials, uint32_t M, uint32_t K, uint32_t N, uint32_t S,
                                const mi_gemv_epilogue* ep, void* stream) {
  if (int e = check_gemv(qweight, scales, x, partials, M, K, N, S)) return e;
  if (!ep) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex: null epilogue");
  hipStream_t st = static_cast<hipStream_t>(stream);
  GemvEpi e{ep->counters, ep->resid, ep->sumsq, ep->rstd, ep->next_norm_w, ep->x_next, ep->h,
            ep->logits, reinterpret_cast<u2_t*>(ep->argmax_part), ep->vocab_used, ep->eps, ep->out16};
  int r;
  switch (ep->kind) {
    case MI_EPI_PARTIALS:
      r = launch_rows<EPI_PARTIALS>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_RESID:
      if (!e.counters || !e.resid || !e.sumsq || !e.rstd || !e.next_w || !e.x_next || N / kCols > 1024)
        return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex RESID: counters, resid, sumsq, rstd, next_norm_w, x_next; N <= 65536");
      r = launch_rows<EPI_RESID>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_SILU:
      if (!e.counters || !e.h || N % 32) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex SILU: counters, h");
      r = launch_rows<EPI_SILU>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_LOGITS:
      if (!e.counters || !e.out32 || e.vocab_used > N)
        return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex LOGITS: counters, logits, vocab_used <= N");
      r = launch_rows<EPI_LOGITS>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_F16OUT:
      if (!e.counters || !e.out16) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex F16OUT: counters, out16");
      r = launch_rows<EPI_F16OUT>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    default:
      return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex: unknown epilogue");
  }
  return mi_hip(r, "gemv_w4a16_ex launch");
}

extern "C" int mi_fold_partials(const float* partials, uint16_t* out_f16, float* out_f32, uint32_t S,
                                uint32_t M, uint32_t N, void* stream) {
  if (!partials || (!out_f16 && !out_f32) || S == 0)
    return mi_fail(MI_ERR_ARG, "fold_partials: bad arguments");
  const uint32_t MN = M * N;
  fold_partials_kernel<<<(MN + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(
      partials, out_f16, out_f32, S, MN);
  return mi_hip((int)hipGetLastError(), "fold_partials launch");
}
