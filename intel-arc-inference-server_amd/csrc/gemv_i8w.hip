// gemv_i8w.hip - the int8 lm_head (W8A16): gemv_i8w (src/kernels/gemv_i8w.cl:55-106) over the
// head quantised at load (src/loader/lm_head_int8.h:1-13, lm_head_int8.cc:22-37).
//
// out[m][n] = (sum_k q[n][k] x[m][k]) * s[n]: one fp32 scale per output column applied to the
// column's fp32 dot product, no K split, no atomics (replays are bitwise).
//
// MI355X form: the weight is tiled for the matrix cores, [N/16][K/64][64 lanes][16 bytes]. In
// each 64-k chunk of a 16-column tile, lane l holds column n = l % 16 at k = 8 (l / 16) + e and
// 32 + 8 (l / 16) + e (e < 8): one 16-byte load per lane, 1 KiB per wave, contiguous across the
// tile's chunks. Those bytes are the A operands of two v_mfma_f32_16x16x32_f16 (int8 values are
// exact in f16: a byte permute under exponent 0x64 and one subtraction); x is the B operand,
// row m in lanes m, m + 16, ... (M <= 8 rows; the other columns are zero). Products are exact in
// fp32; the matrix core sums them in fp32, so the result is the reference's dot up to the order
// of the fp32 additions. Each wave owns one tile and streams its K/64 KiB with eight chunks in
// flight; the weight loads are non-temporal (the head is read once per token).
#include <cmath>

#include "mi_capi_internal.h"
#include "mi_common.h"

namespace mi {
namespace {

constexpr uint32_t kI8Ahead = 8;  // chunks in flight per wave

// 8 int8 values (two words, little-endian bytes) as 8 exact f16 values
__device__ __forceinline__ h8_t i8x8_to_h8(uint32_t w0, uint32_t w1) {
  const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u, hi = 0x64646464u;
  const h2_t bias = {(half_t)1152.0f, (half_t)1152.0f};
  const h2_t p0 = as_h2(__builtin_amdgcn_perm(hi, x0, 0x04010400u)) - bias;
  const h2_t p1 = as_h2(__builtin_amdgcn_perm(hi, x0, 0x04030402u)) - bias;
  const h2_t p2 = as_h2(__builtin_amdgcn_perm(hi, x1, 0x04010400u)) - bias;
  const h2_t p3 = as_h2(__builtin_amdgcn_perm(hi, x1, 0x04030402u)) - bias;
  return h8_t{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// grid N / 64 work-groups of 4 waves, one 16-column tile per wave
__global__ __launch_bounds__(256) void gemv_i8w_kernel(const u4_t* __restrict__ w, const float* __restrict__ scales,
                                                       const uint16_t* __restrict__ x, float* __restrict__ out,
                                                       uint32_t M, uint32_t K, uint32_t N) {
  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t tile = blockIdx.x * 4u + wave;
  const uint32_t nc = K / 64u, col = lane & 15u, q = lane >> 4;
  const uint32_t* wp = reinterpret_cast<const uint32_t*>(w + (size_t)tile * nc * 64u + lane);
  const bool xrow = col < M;
  const uint16_t* xr = x + (size_t)(xrow ? col : 0u) * K + 8u * q;
  f4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (uint32_t c0 = 0; c0 < nc; c0 += kI8Ahead) {
    u4_t wv[kI8Ahead], xa[kI8Ahead], xb[kI8Ahead];
#pragma unroll
    for (uint32_t u = 0; u < kI8Ahead; ++u)
      if (c0 + u < nc) wv[u] = load_stream16(wp + (size_t)(c0 + u) * 256u);
#pragma unroll
    for (uint32_t u = 0; u < kI8Ahead; ++u) {
      xa[u] = u4_t{0u, 0u, 0u, 0u};
      xb[u] = u4_t{0u, 0u, 0u, 0u};
      if (xrow && c0 + u < nc) {
        xa[u] = *as_global(reinterpret_cast<const u4_t*>(xr + 64u * (c0 + u)));
        xb[u] = *as_global(reinterpret_cast<const u4_t*>(xr + 64u * (c0 + u) + 32u));
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < kI8Ahead; ++u)
      if (c0 + u < nc) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(i8x8_to_h8(wv[u].x, wv[u].y), __builtin_bit_cast(h8_t, xa[u]),
                                                     acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(i8x8_to_h8(wv[u].z, wv[u].w), __builtin_bit_cast(h8_t, xb[u]),
                                                     acc, 0, 0, 0);
      }
  }
  // lane l holds the tile's columns 4 (l / 16) + r of row l % 16
  if (col < M) {
#pragma unroll
    for (uint32_t r = 0; r < 4; ++r) {
      const uint32_t n = tile * 16u + 4u * q + r;
      out[(size_t)col * N + n] = acc[r] * scales[n];
    }
  }
}

// One 16-byte unit of mi_i8w_index's layout per thread, gathered from the reference's
// int8_tiled_index layout [N/16][K/16][16 k][16 n] (src/loader/lm_head_int8.h:33).
__global__ __launch_bounds__(256) void i8w_from_ref_kernel(const int8_t* __restrict__ ref, int8_t* __restrict__ out,
                                                           uint32_t K, uint32_t N) {
  const size_t u = (size_t)blockIdx.x * 256u + threadIdx.x;  // unit (tile, chunk, lane)
  const size_t units = (size_t)K * N / 16u;
  if (u >= units) return;
  const uint32_t lane = (uint32_t)(u % 64u), nc = K / 64u;
  const uint32_t c = (uint32_t)((u / 64u) % nc), tile = (uint32_t)(u / 64u / nc);
  const uint32_t n = tile * 16u + lane % 16u, q = lane / 16u;
  uint32_t wv[4];
#pragma unroll
  for (uint32_t b = 0; b < 16u; ++b) {
    const uint32_t k = c * 64u + (b / 8u) * 32u + q * 8u + b % 8u;
    const size_t ri = ((size_t)(n / 16u) * (K / 16u) + k / 16u) * 256u + (k % 16u) * 16u + n % 16u;
    const uint32_t v = (uint8_t)ref[ri];
    if (b % 4u == 0) wv[b / 4u] = v;
    else wv[b / 4u] |= v << (8u * (b % 4u));
  }
  *reinterpret_cast<u4_t*>(out + u * 16u) = u4_t{wv[0], wv[1], wv[2], wv[3]};
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

size_t mi_i8w_index(uint32_t K, uint32_t k, uint32_t n) {
  const uint32_t c = k / 64u, kk = k % 64u, half = kk / 32u, q = (kk % 32u) / 8u, e = kk % 8u;
  const uint32_t lane = q * 16u + n % 16u;
  return (((size_t)(n / 16u) * (K / 64u) + c) * 64u + lane) * 16u + half * 8u + e;
}

// lm_head_int8.cc:22-37's quantisation, row by row: s = max|w| / 127 in fp32, q = rne(w / s)
// clamped to [-127, 127], a zero row s = 0 and q = 0; written in mi_i8w_index's layout.
int mi_lm_head_int8_quantise(const float* w, uint32_t K, uint32_t N, int8_t* q_tiled, float* scales) {
  if (!w || !q_tiled || !scales || K == 0 || N == 0 || K % 64 || N % 16)
    return mi_fail(MI_ERR_ARG, "lm_head_int8_quantise: K a multiple of 64, N of 16");
  for (uint32_t n = 0; n < N; ++n) {
    const float* row = w + (size_t)n * K;
    float amax = 0.f;
    for (uint32_t k = 0; k < K; ++k) amax = std::fmax(amax, std::fabs(row[k]));
    const float s = amax / 127.0f;
    scales[n] = s;
    for (uint32_t k = 0; k < K; ++k) {
      int8_t v = 0;
      if (s != 0.f) {
        const float r = std::nearbyint(row[k] / s);  // round to nearest even (the default mode)
        v = int8_t(r < -127.f ? -127.f : (r > 127.f ? 127.f : r));
      }
      q_tiled[mi_i8w_index(K, k, n)] = v;
    }
  }
  return 0;
}

int mi_i8w_from_ref_tiles(const int8_t* ref_tiled, uint32_t K, uint32_t N, int8_t* q_tiled, void* stream) {
  if (!ref_tiled || !q_tiled || ref_tiled == q_tiled || K == 0 || N == 0 || K % 64 || N % 16)
    return mi_fail(MI_ERR_ARG, "i8w_from_ref_tiles: two buffers, K a multiple of 64, N of 16");
  const size_t units = (size_t)K * N / 16u;
  i8w_from_ref_kernel<<<(unsigned)((units + 255u) / 256u), 256, 0, (hipStream_t)stream>>>(ref_tiled, q_tiled, K, N);
  return mi_hip((int)hipGetLastError(), "i8w_from_ref_tiles");
}

int mi_gemv_i8w(const int8_t* w, const float* scales, const uint16_t* x, float* out, uint32_t M, uint32_t K,
                uint32_t N, void* stream) {
  if (!w || !scales || !x || !out || M == 0 || M > 8 || K == 0 || K % 64 || N == 0 || N % 64)
    return mi_fail(MI_ERR_ARG, "gemv_i8w: M 1..8, K a multiple of 64, N of 64");
  gemv_i8w_kernel<<<N / 64u, 256, 0, (hipStream_t)stream>>>(reinterpret_cast<const u4_t*>(w), scales, x, out, M,
                                                            K, N);
  return mi_hip((int)hipGetLastError(), "gemv_i8w");
}

}  // extern "C"
