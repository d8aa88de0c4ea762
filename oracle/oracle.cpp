// oracle.cpp - TEST INFRASTRUCTURE: the CPU oracle (see oracle.h). A scalar C++17
// restatement of the reference engine's host twins, parameterised by shape and by
// activation type. Built with -O2 -ffp-contract=off (as the reference builds its CPU
// references, CMakeLists.txt:31-34), so `a += x * y` is a rounded multiply then a
// rounded add, and std::fma is the only fused operation.
//
// Nothing in the product library links or loads this file's output.
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

inline uint32_t fbits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}
inline float bitsf(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
inline float ninf() { return -std::numeric_limits<float>::infinity(); }

// --- activation rounding points --------------------------------------------------------
struct Act {
  int t;
  uint16_t rne(float f) const { return t == ORC_BF16 ? orc_f32_to_bf16(f) : orc_f32_to_f16(f); }
  float w(uint16_t h) const { return t == ORC_BF16 ? orc_bf16_to_f32(h) : orc_f16_to_f32(h); }
  float rf(float f) const { return w(rne(f)); }
};

// silu / sigmoid with plain exp (prep_ref.h:51, attn_ref.h:97)
inline float silu_f32(float x) { return x / (1.0f + std::exp(-x)); }
inline float sigmoid_f32(float x) { return 1.0f / (1.0f + std::exp(-x)); }

// --- weight views (tests/kernels/gemm_sm_ref.h:27-70) ----------------------------------
struct WView {
  uint32_t K, N, kind;  // kind 0: GPTQ layout 0; 1: 544-B tiles
  const uint32_t* words;
  const uint16_t* scales;
  int q(uint32_t k, uint32_t n) const {
    if (kind == 0) return int((words[size_t(k / 8) * N + n] >> (4 * (k % 8))) & 0xFu) - 8;
    const uint32_t* tile = words + (size_t(n / 16) * (K / 64) + k / 64) * 136;
    return int((tile[((k % 64) / 8) * 16 + n % 16] >> (4 * (k % 8))) & 0xFu) - 8;
  }
  float scale(uint32_t k, uint32_t n) const {
    if (kind == 0) return orc_f16_to_f32(scales[size_t(k / 64) * N + n]);
    const uint32_t* tile = words + (size_t(n / 16) * (K / 64) + k / 64) * 136;
    uint16_t h;
    std::memcpy(&h, reinterpret_cast<const uint16_t*>(tile + 128) + n % 16, 2);
    return orc_f16_to_f32(h);
  }
  uint32_t word(uint32_t r, uint32_t n) const {  // the u32 holding k = 8r .. 8r+7 of column n
    if (kind == 0) return words[size_t(r) * N + n];
    const uint32_t k = r * 8;
    const uint32_t* tile = words + (size_t(n / 16) * (K / 64) + k / 64) * 136;
    return tile[((k % 64) / 8) * 16 + n % 16];
  }
};

// gemv.cl's fp32 order for one column over groups [g0, g1) (gemm_sm_ref.h:109-136):
// per group eight dot8 chains (a = 0; a += q*x, k ascending), gacc += a, acc += gacc*scale.
inline float group_range_dot(const WView& v, uint32_t n, const float* x, uint32_t g0, uint32_t g1) {
  float acc = 0.f;
  for (uint32_t g = g0; g < g1; ++g) {
    float gacc = 0.f;
    for (uint32_t j = 0; j < 8; ++j) {
      const uint32_t wd = v.word(g * 8 + j, n);
      const float* xx = x + g * 64 + j * 8;
      float a = 0.f;
      for (uint32_t i = 0; i < 8; ++i) a += float(int((wd >> (4 * i)) & 0xFu) - 8) * xx[i];
      gacc += a;
    }
    acc += gacc * v.scale(g * 64, n);
  }
  return acc;
}

// Layout-0 fast path of the same per-column order, 64 columns at a time (the per-column
// sequence of operations is unchanged; only columns are interleaved).
void twin_slice_l0(const WView& v, const float* x, uint32_t n0, uint32_t n1, uint32_t g0,
                   uint32_t g1, float* out) {
  constexpr uint32_t B = 64;
  for (uint32_t nb = n0; nb < n1; nb += B) {
    const uint32_t nn = std::min(B, n1 - nb);
    float acc[B] = {};
    for (uint32_t g = g0; g < g1; ++g) {
      float gacc[B] = {};
      for (uint32_t j = 0; j < 8; ++j) {
        const uint32_t* wr = v.words + size_t(g * 8 + j) * v.N + nb;
        const float* xx = x + g * 64 + j * 8;
        for (uint32_t c = 0; c < nn; ++c) {
          const uint32_t wd = wr[c];
          float a = 0.f;
          for (uint32_t i = 0; i < 8; ++i) a += float(int((wd >> (4 * i)) & 0xFu) - 8) * xx[i];
          gacc[c] += a;
        }
      }
      const uint16_t* sr = v.scales + size_t(g) * v.N + nb;
      for (uint32_t c = 0; c < nn; ++c) acc[c] += gacc[c] * orc_f16_to_f32(sr[c]);
    }
    for (uint32_t c = 0; c < nn; ++c) out[nb + c] = acc[c];
  }
}

void twin_partial(const WView& v, const float* x, uint32_t S, uint32_t s, float* out /*[N]*/) {
  const uint32_t G = v.K / 64, GS = G / S;
  if (v.kind == 0) {
    const uint32_t NB = 256;
    const uint32_t nblocks = (v.N + NB - 1) / NB;
#pragma omp parallel for schedule(static)
    for (uint32_t b = 0; b < nblocks; ++b)
      twin_slice_l0(v, x, b * NB, std::min(v.N, (b + 1) * NB), s * GS, (s + 1) * GS, out);
  } else {
    for (uint32_t n = 0; n < v.N; ++n) out[n] = group_range_dot(v, n, x, s * GS, (s + 1) * GS);
  }
}

// attention helpers -----------------------------------------------------------------------
inline size_t kv_row(uint32_t p, const uint32_t* pages, uint32_t page) {
  return pages ? size_t(pages[p / page]) * page + p % page : size_t(p);
}

struct KvRead {
  uint32_t kind;
  Act act;
  const void* k;
  const void* v;
  const uint16_t* ks;
  const uint16_t* vs;
  size_t rs, hs, srs, shs;
  const uint32_t* pages;
  uint32_t page;
  float kf(uint32_t p, uint32_t h, uint32_t d) const {
    const size_t r = kv_row(p, pages, page);
    if (kind == 0) return act.w(static_cast<const uint16_t*>(k)[r * rs + h * hs + d]);
    return float(static_cast<const int8_t*>(k)[r * rs + h * hs + d]) * orc_f16_to_f32(ks[r * srs + h * shs]);
  }
  float vf(uint32_t p, uint32_t h, uint32_t d) const {
    const size_t r = kv_row(p, pages, page);
    if (kind == 0) return act.w(static_cast<const uint16_t*>(v)[r * rs + h * hs + d]);
    return float(static_cast<const int8_t*>(v)[r * rs + h * hs + d]) * orc_f16_to_f32(vs[r * srs + h * shs]);
  }
};

}  // namespace

extern "C" {

int orc_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

// Threads the OpenMP column loops use from now on (n >= 1); the result does not depend on it.
void orc_set_threads(int n) {
#ifdef _OPENMP
  if (n >= 1) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

// ---- conversions -----------------------------------------------------------------------
// src/common/bf16.h:8-16
float orc_bf16_to_f32(uint16_t h) { return bitsf(uint32_t(h) << 16); }
uint16_t orc_f32_to_bf16(float f) {
  const uint32_t u = fbits(f);
  const uint32_t rounding = ((u >> 16) & 1u) + 0x7FFFu;
  return uint16_t((u + rounding) >> 16);
}
// src/common/bf16.h:22-31: exact for every half, subnormals included
float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
  if (e == 0) {
    const float f = float(man) * 5.9604644775390625e-08f;
    return sign ? -f : f;
  }
  const uint32_t u = e == 31 ? ((sign << 31) | 0x7F800000u | (man << 13))
                             : ((sign << 31) | ((e + 112u) << 23) | (man << 13));
  return bitsf(u);
}
// src/common/bf16.h:32-43 (flushes results below 2^-14 to signed zero)
uint16_t orc_f32_to_f16_ftz(float f) {
  const uint32_t u = fbits(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const int32_t e = int32_t((u >> 23) & 0xFFu) - 127 + 15;
  const uint32_t man = u & 0x7FFFFFu;
  if (e <= 0) return uint16_t(sign);
  if (e >= 31) return uint16_t(sign | 0x7C00u);
  uint32_t half = sign | (uint32_t(e) << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half += 1u;
  return uint16_t(half);
}
// IEEE binary16 round-to-nearest-even with subnormals and overflow to inf: the rounding
// the activation stream uses (what v_cvt_f16_f32 computes). Same construction as
// src/common/kv8.h:63-75 without its saturation.
uint16_t orc_f32_to_f16(float f) {
  uint32_t u = fbits(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  u &= 0x7FFFFFFFu;
  if (u > 0x7F800000u) return uint16_t(sign | 0x7E00u);  // NaN
  if (u >= 0x477FF000u) return uint16_t(sign | 0x7C00u); // rounds to >= 65520: inf
  if (u < 0x38800000u)                                   // below 2^-14: subnormal half
    return uint16_t(sign | uint32_t(std::nearbyint(bitsf(u) * 16777216.0f)));
  const uint32_t e = (u >> 23) - 112u;
  const uint32_t m = u & 0x7FFFFFu;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return uint16_t(sign | h);
}
// src/common/kv8.h:63-75 (saturating)
uint16_t orc_f32_to_f16_sat(float f) {
  uint32_t u = fbits(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  u &= 0x7FFFFFFFu;
  if (u >= 0x477FE000u) return uint16_t(sign | 0x7BFFu);
  if (u < 0x38800000u) return uint16_t(sign | uint32_t(std::nearbyint(bitsf(u) * 16777216.0f)));
  const uint32_t e = (u >> 23) - 112u;
  const uint32_t m = u & 0x7FFFFFu;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rem = m & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return uint16_t(sign | h);
}
uint16_t orc_rne(int act, float f) { return Act{act}.rne(f); }
float orc_widen(int act, uint16_t h) { return Act{act}.w(h); }

// ---- int4 -----------------------------------------------------------------------------------
// src/common/int4.h:19-23
float orc_int4_at(const uint32_t* qweight, const uint16_t* scales, uint32_t K, uint32_t N,
                  uint32_t k, uint32_t n) {
  (void)K;
  const uint32_t word = qweight[(k / 8) * size_t(N) + n];
  const int q = int((word >> (4 * (k % 8))) & 0xFu);
  return float(q - 8) * orc_f16_to_f32(scales[(k / 64) * size_t(N) + n]);
}
void orc_int4_dequant(const uint32_t* qweight, const uint16_t* scales, uint32_t K, uint32_t N,
                      float* out) {
  for (uint32_t k = 0; k < K; ++k)
    for (uint32_t n = 0; n < N; ++n) out[size_t(k) * N + n] = orc_int4_at(qweight, scales, K, N, k, n);
}
// src/common/repack.h:17-30
void orc_repack_layout1(const uint32_t* qweight, const uint16_t* scales, uint32_t K, uint32_t N,
                        uint32_t* out) {
  const uint32_t G = K / 64, NT = N / 16;
  for (uint32_t nt = 0; nt < NT; ++nt)
    for (uint32_t g = 0; g < G; ++g) {
      uint32_t* tile = out + (size_t(nt) * G + g) * 136;
      for (uint32_t j = 0; j < 8; ++j)
        for (uint32_t l = 0; l < 16; ++l) tile[j * 16 + l] = qweight[size_t(g * 8 + j) * N + nt * 16 + l];
      for (uint32_t l = 0; l < 16; l += 2)
        tile[128 + l / 2] = uint32_t(scales[size_t(g) * N + nt * 16 + l]) |
                            (uint32_t(scales[size_t(g) * N + nt * 16 + l + 1]) << 16);
    }
}
// src/common/repack.h:64-73 + :80-95 (interleave16 column map, layout 0)
void orc_interleave16_l0(const uint32_t* aq, const uint16_t* as, const uint32_t* bq,
                         const uint16_t* bs, uint32_t K, uint32_t Np, uint32_t* oq, uint16_t* os) {
  const uint32_t NT = 2 * Np;
  for (uint32_t n = 0; n < NT; ++n) {
    const bool from_b = (n % 32) >= 16;
    const uint32_t src = (n / 32) * 16 + n % 16;
    const uint32_t* q = from_b ? bq : aq;
    const uint16_t* s = from_b ? bs : as;
    for (uint32_t r = 0; r < K / 8; ++r) oq[size_t(r) * NT + n] = q[size_t(r) * Np + src];
    for (uint32_t g = 0; g < K / 64; ++g) os[size_t(g) * NT + n] = s[size_t(g) * Np + src];
  }
}

// ---- GEMV -----------------------------------------------------------------------------------
// tests/kernels/gemm_sm_ref.h:83-104 (fp64 reference and the N2 denominator)
void orc_gemv_ref(uint32_t layout, const uint32_t* words, const uint16_t* scales, uint32_t K,
                  uint32_t N, const float* xf, uint32_t M, double* out, double* bound) {
  const WView v{K, N, layout, words, scales};
#pragma omp parallel for schedule(static)
  for (uint32_t n = 0; n < N; ++n) {
    std::vector<double> col(K);
    for (uint32_t k = 0; k < K; ++k) col[k] = double(v.q(k, n)) * double(v.scale(k, n));
    for (uint32_t m = 0; m < M; ++m) {
      const float* x = xf + size_t(m) * K;
      double a = 0, b = 0;
      for (uint32_t k = 0; k < K; ++k) {
        const double p = col[k] * double(x[k]);
        a += p;
        b += std::fabs(p);
      }
      out[size_t(m) * N + n] = a;
      if (bound) bound[size_t(m) * N + n] = b;
    }
  }
}
// tests/kernels/gemm_sm_ref.h:106-136 (slices written separately)
void orc_gemv_twin_partials(uint32_t layout, const uint32_t* words, const uint16_t* scales,
                            uint32_t K, uint32_t N, const float* xf, uint32_t M, uint32_t S,
                            float* partials) {
  const WView v{K, N, layout, words, scales};
  for (uint32_t s = 0; s < S; ++s)
    for (uint32_t m = 0; m < M; ++m)
      twin_partial(v, xf + size_t(m) * K, S, s, partials + (size_t(s) * M + m) * N);
}
// ... and summed from 0.f in s order (the host's fold in run_gemv)
void orc_gemv_twin(uint32_t layout, const uint32_t* words, const uint16_t* scales, uint32_t K,
                   uint32_t N, const float* xf, uint32_t M, uint32_t S, float* out) {
  std::vector<float> part(size_t(S) * M * N);
  orc_gemv_twin_partials(layout, words, scales, K, N, xf, M, S, part.data());
  for (size_t i = 0; i < size_t(M) * N; ++i) {
    float t = 0.f;
    for (uint32_t s = 0; s < S; ++s) t += part[size_t(s) * M * N + i];
    out[i] = t;
  }
}
// tests/kernels/gemm_sm_ref.h:180-225 (the N2 bound, per output)
size_t orc_n2_over(const float* got, const double* ref, const double* bound, size_t n,
                   double* max_ratio) {
  size_t over = 0;
  double mr = 0;
  for (size_t i = 0; i < n; ++i) {
    if (!std::isfinite(got[i])) {
      ++over;
      mr = 1e30;
      continue;
    }
    const double e = std::fabs(double(got[i]) - ref[i]);
    const double lim = std::ldexp(bound[i], -16);
    const double q = lim > 0 ? e / lim : (e == 0 ? 0.0 : 1e30);
    mr = std::max(mr, q);
    if (q > 1.0) ++over;
  }
  if (max_ratio) *max_ratio = mr;
  return over;
}

// ---- prep -----------------------------------------------------------------------------------
// tests/kernels/prep_ref.h:59-92 (single-stage residual fold + RMSNorm, 256-lane tree)
void orc_res_norm(int act, const float* partials, uint16_t* resid, const float* norm_w,
                  uint16_t* x_out, uint32_t M, uint32_t K, uint32_t S_PREV, float eps) {
  const Act A{act};
  constexpr uint32_t WG = 256;
  std::vector<float> row(K), red(WG);
  for (uint32_t m = 0; m < M; ++m) {
    uint16_t* rp = resid + size_t(m) * K;
    for (uint32_t k = 0; k < K; ++k) {
      uint16_t r_b;
      if (S_PREV == 0) {
        r_b = rp[k];
      } else {
        float acc = 0.f;
        for (uint32_t s = 0; s < S_PREV; ++s) acc += partials[(size_t(s) * M + m) * K + k];
        r_b = A.rne(A.w(rp[k]) + A.w(A.rne(acc)));
      }
      rp[k] = r_b;
      row[k] = A.w(r_b);
    }
    for (uint32_t i = 0; i < WG; ++i) {
      float s = 0.f;
      for (uint32_t k = i; k < K; k += WG) s = std::fma(row[k], row[k], s);
      red[i] = s;
    }
    for (uint32_t stride = WG / 2; stride > 0; stride >>= 1)
      for (uint32_t i = 0; i < stride; ++i) red[i] += red[i + stride];
    const float mean = red[0] / float(K);
    const float rstd = 1.0f / std::sqrt(mean + eps);
    for (uint32_t k = 0; k < K; ++k) x_out[size_t(m) * K + k] = A.rne(row[k] * rstd * norm_w[k]);
  }
}
// tests/kernels/prep_ref.h:120-156
void orc_res_fold(int act, const float* partials, uint16_t* resid, float* sumsq, uint32_t M,
                  uint32_t K, uint32_t S_PREV, uint32_t G) {
  const Act A{act};
  constexpr uint32_t WG = 256;
  const uint32_t chunk = (K + G - 1) / G;
  std::vector<float> red(WG);
  for (uint32_t m = 0; m < M; ++m) {
    uint16_t* rp = resid + size_t(m) * K;
    for (uint32_t g = 0; g < G; ++g) {
      const uint32_t k0 = g * chunk, k1 = k0 + chunk > K ? K : k0 + chunk;
      for (uint32_t i = 0; i < WG; ++i) {
        float acc2 = 0.f;
        for (uint32_t k = k0 + i; k < k1; k += WG) {
          uint16_t r_b;
          if (S_PREV == 0) {
            r_b = rp[k];
          } else {
            float acc = 0.f;
            for (uint32_t s = 0; s < S_PREV; ++s) acc += partials[(size_t(s) * M + m) * K + k];
            r_b = A.rne(A.w(rp[k]) + A.w(A.rne(acc)));
          }
          rp[k] = r_b;
          const float v = A.w(r_b);
          acc2 = std::fma(v, v, acc2);
        }
        red[i] = acc2;
      }
      for (uint32_t stride = WG / 2; stride > 0; stride >>= 1)
        for (uint32_t i = 0; i < stride; ++i) red[i] += red[i + stride];
      sumsq[size_t(g) * M + m] = red[0];
    }
  }
}
// tests/kernels/prep_ref.h:158-168
void orc_norm_finish(int act, const float* sumsq, const uint16_t* resid, const float* norm_w,
                     uint16_t* x_out, uint32_t M, uint32_t K, uint32_t G, float eps) {
  const Act A{act};
  for (uint32_t m = 0; m < M; ++m) {
    float total = 0.f;
    for (uint32_t g = 0; g < G; ++g) total += sumsq[size_t(g) * M + m];
    const float mean = total / float(K);
    const float rstd = 1.0f / std::sqrt(mean + eps);
    for (uint32_t k = 0; k < K; ++k)
      x_out[size_t(m) * K + k] = A.rne(A.w(resid[size_t(m) * K + k]) * rstd * norm_w[k]);
  }
}
// tests/kernels/prep_ref.h:170-189 (gate||up interleaved in 16-column blocks)
void orc_silu_mul(int act, const float* partials, uint16_t* x_out, uint32_t M, uint32_t N,
                  uint32_t S) {
  const Act A{act};
  const size_t FN = size_t(2) * N;
  for (uint32_t m = 0; m < M; ++m)
    for (uint32_t k = 0; k < N; ++k) {
      const size_t gflat = size_t(k / 16) * 32 + (k % 16), uflat = gflat + 16;
      float ga = 0.f, ua = 0.f;
      for (uint32_t s = 0; s < S; ++s) {
        const size_t base = (size_t(s) * M + m) * FN;
        ga += partials[base + gflat];
        ua += partials[base + uflat];
      }
      const uint16_t g_b = A.rne(ga), u_b = A.rne(ua);
      const uint16_t s_b = A.rne(silu_f32(A.w(g_b)));
      x_out[size_t(m) * N + k] = A.rne(A.w(s_b) * A.w(u_b));
    }
}

// ---- attention ----------------------------------------------------------------------------
// src/loader/loader.cc:702-716 (cos/sin in double, stored fp32), generalised to rot_dim
void orc_rope_table(double theta, uint32_t rot_dim, uint32_t max_len, float* t) {
  const uint32_t half = rot_dim / 2;
  std::vector<double> inv(half);
  for (uint32_t i = 0; i < half; ++i) inv[i] = std::pow(theta, -2.0 * double(i) / double(rot_dim));
  for (uint32_t p = 0; p < max_len; ++p)
    for (uint32_t i = 0; i < half; ++i) {
      const double a = double(p) * inv[i];
      t[(size_t(p) * 2 + 0) * half + i] = float(std::cos(a));
      t[(size_t(p) * 2 + 1) * half + i] = float(std::sin(a));
    }
}

// tests/kernels/attn_ref.h:117-199 (attn_prep), parameterised: heads, head_dim, rotary
// dims, gate on/off, q/k norm on/off (NULL weights: the linear's rounding only), KV rows
// through an optional page table.
void orc_attn_prep(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act, uint32_t M,
                   const float* partials, uint32_t S, const float* q_norm, const float* k_norm,
                   const float* rope, float* attn_q, float* attn_gate, uint16_t* kv_k,
                   uint16_t* kv_v, size_t rs, size_t hs, const uint32_t* pages, uint32_t page) {
  const Act A{act};
  const uint32_t HD = sh->head_dim, QH = sh->q_heads, KVH = sh->kv_heads;
  const uint32_t half = sh->rot_dim / 2, rot = sh->rot_dim;
  std::vector<float> red(HD), nrm(HD);
  for (uint32_t wg = 0; wg < QH + KVH; ++wg) {
    const bool is_q = wg < QH;
    const uint32_t h = is_q ? wg : wg - QH;
    const float* nw = is_q ? q_norm : k_norm;
    for (uint32_t m = 0; m < n_act; ++m) {
      const size_t base = is_q ? (sh->gated ? size_t(h) * 2 * HD : size_t(h) * HD)
                               : size_t(sh->k_off) + size_t(h) * HD;
      auto qkv_sum = [&](size_t col) {
        float v = 0.0f;
        for (uint32_t s = 0; s < S; ++s) v += partials[(size_t(s) * M + m) * sh->qkv_n + col];
        return v;
      };
      if (nw) {
        for (uint32_t i = 0; i < HD; ++i) {
          const float xf = A.w(A.rne(qkv_sum(base + i)));
          red[i] = xf * xf;
        }
        for (uint32_t stride = HD / 2; stride > 0; stride >>= 1)
          for (uint32_t i = 0; i < stride; ++i) red[i] += red[i + stride];
        const float rstd = 1.0f / std::sqrt(red[0] / float(HD) + sh->eps);
        for (uint32_t i = 0; i < HD; ++i) nrm[i] = A.w(A.rne(A.w(A.rne(qkv_sum(base + i))) * rstd * nw[i]));
      } else {
        for (uint32_t i = 0; i < HD; ++i) nrm[i] = A.w(A.rne(qkv_sum(base + i)));
      }
      const float* cs = rope + size_t(pos + m) * 2 * half;
      const size_t row = kv_row(pos + m, pages, page);
      for (uint32_t i = 0; i < HD; ++i) {
        float outv;
        if (i < half) {
          const float c = cs[i], s = cs[half + i];
          const float t = nrm[i + half] * s;
          outv = std::fma(nrm[i], c, -t);
        } else if (i < rot) {
          const uint32_t ii = i - half;
          const float c = cs[ii], s = cs[half + ii];
          const float t = nrm[ii] * s;
          outv = std::fma(nrm[i], c, t);
        } else {
          outv = nrm[i];
        }
        if (is_q)
          attn_q[(size_t(m) * QH + h) * HD + i] = outv;
        else
          kv_k[row * rs + h * hs + i] = A.rne(outv);
      }
      if (is_q) {
        if (sh->gated && attn_gate)
          for (uint32_t i = 0; i < HD; ++i)
            attn_gate[(size_t(m) * QH + h) * HD + i] = A.w(A.rne(qkv_sum(base + HD + i)));
      } else {
        for (uint32_t i = 0; i < HD; ++i)
          kv_v[row * rs + h * hs + i] = A.rne(qkv_sum(size_t(sh->v_off) + size_t(h) * HD + i));
      }
    }
  }
}

// src/kernels/attn_v2.cl:138-142
uint32_t orc_v2_ppw(uint32_t len, uint32_t tgt) {
  uint32_t p = (len + tgt - 1) / tgt;
  p = (p + 63u) & ~63u;
  return std::max(64u, p);
}

// src/kernels/attn_v2.cl:172-380 (attn_decode_v2), per row: row m walks blocks of
// ppw(pos+m+1) positions in waves of 16; the score dot is 16 lanes x (HD/16) dims per lane
// (d = l + 16t ascending, fma) merged by the pairwise tree 8,4,2,1; online softmax per
// wave; partials {mx, sm, acc[HD]} at [qh][tgt][M][HD+2]. Rows are independent: positions
// past row m's bound add exact zeros (attn_v2.cl:37-39), so the per-row walk is bitwise the
// kernel's grouped walk.
void orc_attn_decode_v2(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act,
                        uint32_t M, uint32_t tgt, const float* attn_q, uint32_t kv_kind,
                        const void* kv_k, const void* kv_v, const uint16_t* k_scale,
                        const uint16_t* v_scale, size_t rs, size_t hs, size_t srs, size_t shs,
                        const uint32_t* pages, uint32_t page, float* attn_part) {
  const KvRead kv{kv_kind, Act{act}, kv_k, kv_v, k_scale, v_scale, rs, hs, srs, shs, pages, page};
  const uint32_t HD = sh->head_dim, QH = sh->q_heads, KVH = sh->kv_heads, GQA = QH / KVH;
  const uint32_t PL = HD / 16, PART = HD + 2;
  std::vector<float> acc(HD), tsum(HD), kreg(16 * HD);
  for (uint32_t j = 0; j < KVH; ++j)
    for (uint32_t m = 0; m < n_act; ++m) {
      const uint32_t bound = pos + m, s = orc_v2_ppw(pos + m + 1, tgt);
      const uint32_t nb = std::min(tgt, bound / s + 1);
      for (uint32_t blk = 0; blk < nb; ++blk) {
        const uint32_t bstart = blk * s, bend = std::min(bstart + s, bound + 1);
        const uint32_t nwaves = (bend - bstart + 15) / 16;
        for (uint32_t qhl = 0; qhl < GQA; ++qhl) {
          const uint32_t qh = j * GQA + qhl;
          const float* q = attn_q + (size_t(m) * QH + qh) * HD;
          float mx = ninf(), sm = 0.f;
          std::fill(acc.begin(), acc.end(), 0.f);
          for (uint32_t w = 0; w < nwaves; ++w) {
            const uint32_t p0 = bstart + w * 16;
            float sc[16];
            for (uint32_t sl = 0; sl < 16; ++sl) {
              const uint32_t p = p0 + sl;
              if (p > bound) {
                sc[sl] = ninf();
                continue;
              }
              float dot[16];
              for (uint32_t l = 0; l < 16; ++l) {
                float a = 0.f;
                for (uint32_t t = 0; t < PL; ++t) {
                  const uint32_t d = l + 16 * t;
                  a = std::fma(q[d], kv.kf(p, j, d), a);
                }
                dot[l] = a;
              }
              for (uint32_t st = 8; st > 0; st >>= 1)
                for (uint32_t l = 0; l < st; ++l) dot[l] += dot[l + st];
              sc[sl] = dot[0] * sh->scale;
            }
            float nmx = mx;
            for (uint32_t sl = 0; sl < 16; ++sl) nmx = std::fmax(nmx, sc[sl]);
            float resc, wl[16];
            if (nmx > ninf()) {
              resc = std::exp(mx - nmx);
              for (uint32_t sl = 0; sl < 16; ++sl) wl[sl] = std::exp(sc[sl] - nmx);
            } else {
              resc = 1.f;
              for (uint32_t sl = 0; sl < 16; ++sl) wl[sl] = 0.f;
            }
            float ssum = 0.f;
            for (uint32_t sl = 0; sl < 16; ++sl) ssum += wl[sl];
            for (uint32_t d = 0; d < HD; ++d) {
              float t = 0.f;
              for (uint32_t sl = 0; sl < 16; ++sl) {
                const uint32_t p = p0 + sl;
                const float vf = p <= bound ? kv.vf(p, j, d) : 0.0f;
                t = std::fma(wl[sl], vf, t);
              }
              tsum[d] = t;
            }
            if (nmx > ninf()) {
              sm = std::fma(sm, resc, ssum);
              mx = nmx;
            }
            for (uint32_t d = 0; d < HD; ++d) acc[d] = std::fma(acc[d], resc, tsum[d]);
          }
          float* out = attn_part + ((size_t(qh) * tgt + blk) * M + m) * PART;
          out[0] = mx;
          out[1] = sm;
          for (uint32_t d = 0; d < HD; ++d) out[2 + d] = acc[d];
        }
      }
    }
}

// src/kernels/attn_v2.cl:383-428 (attn_reduce_v2): ascending block merge; then
// gated: rne(f32(rne(acc/sm)) * sigmoid(gate)); ungated: rne(acc/sm).
void orc_attn_reduce_v2(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act,
                        uint32_t M, uint32_t tgt, const float* attn_part, const float* attn_gate,
                        uint16_t* attn_out) {
  const Act A{act};
  const uint32_t HD = sh->head_dim, QH = sh->q_heads, PART = HD + 2, OUT_N = QH * HD;
  for (uint32_t h = 0; h < QH; ++h)
    for (uint32_t m = 0; m < n_act; ++m) {
      uint32_t nb = (pos + m) / orc_v2_ppw(pos + m + 1, tgt) + 1;
      if (nb > tgt) nb = tgt;
      for (uint32_t d = 0; d < HD; ++d) {
        float mx = ninf(), sm = 0.f, acc = 0.f;
        for (uint32_t b = 0; b < nb; ++b) {
          const float* p = attn_part + ((size_t(h) * tgt + b) * M + m) * PART;
          const float bmx = p[0], bsm = p[1], bacc = p[2 + d];
          const float nmx = std::fmax(mx, bmx);
          const float a = std::exp(mx - nmx);
          const float bs = std::exp(bmx - nmx);
          sm = std::fma(sm, a, bsm * bs);
          acc = std::fma(acc, a, bacc * bs);
          mx = nmx;
        }
        const float o = acc / sm;
        uint16_t r;
        if (sh->gated && attn_gate)
          r = A.rne(A.w(A.rne(o)) * sigmoid_f32(attn_gate[(size_t(m) * QH + h) * HD + d]));
        else
          r = A.rne(o);
        attn_out[size_t(m) * OUT_N + size_t(h) * HD + d] = r;
      }
    }
}

// fp64 softmax attention (tests/kernels/kv8_ref.h:88-110's form, without rotation)
void orc_attend64(const orc_attn_shape* sh, const float* q, uint32_t kvh, uint32_t n,
                  uint32_t kv_kind, int act, const void* kv_k, const void* kv_v,
                  const uint16_t* k_scale, const uint16_t* v_scale, size_t rs, size_t hs,
                  size_t srs, size_t shs, const uint32_t* pages, uint32_t page, double* out) {
  const KvRead kv{kv_kind, Act{act}, kv_k, kv_v, k_scale, v_scale, rs, hs, srs, shs, pages, page};
  const uint32_t HD = sh->head_dim;
  std::vector<double> sc(n);
  double mx = -INFINITY;
  for (uint32_t p = 0; p < n; ++p) {
    double a = 0;
    for (uint32_t i = 0; i < HD; ++i) a += double(q[i]) * double(kv.kf(p, kvh, i));
    sc[p] = a * double(sh->scale);
    mx = std::max(mx, sc[p]);
  }
  double sum = 0;
  std::vector<double> o(HD, 0.0);
  for (uint32_t p = 0; p < n; ++p) {
    const double w = std::exp(sc[p] - mx);
    sum += w;
    for (uint32_t i = 0; i < HD; ++i) o[i] += w * double(kv.vf(p, kvh, i));
  }
  for (uint32_t i = 0; i < HD; ++i) out[i] = o[i] / sum;
}

// ---- int8 KV (src/common/kv8.h:30-156) --------------------------------------------------
namespace {
constexpr uint32_t kSignWords[8] = {0xA197D809u, 0xA6850592u, 0xB205A73Eu, 0x20AFA769u,
                                    0x45C2CF64u, 0xBEAEAACBu, 0x75F39ADDu, 0x2385A70Cu};
inline bool sign_neg(uint32_t j) { return (kSignWords[j >> 5] >> (j & 31u)) & 1u; }
inline float flip(float v, bool neg) { return neg ? bitsf(fbits(v) ^ 0x80000000u) : v; }
void fwht(float* v, uint32_t n) {
  for (uint32_t h = 1; h < n; h <<= 1)
    for (uint32_t i = 0; i < n; ++i)
      if ((i & h) == 0) {
        const float a = v[i], c = v[i + h];
        v[i] = a + c;
        v[i + h] = a - c;
      }
}
}  // namespace
void orc_kv8_rotate256(const float* x, float* out) {
  float v[256];
  std::memcpy(v, x, sizeof v);
  fwht(v, 256);
  for (uint32_t j = 0; j < 256; ++j) out[j] = flip(v[j], sign_neg(j)) * 0.0625f;
}
void orc_kv8_unrotate256(const float* y, float* out) {
  float v[256];
  for (uint32_t j = 0; j < 256; ++j) v[j] = flip(y[j], sign_neg(j));
  fwht(v, 256);
  for (uint32_t i = 0; i < 256; ++i) out[i] = v[i] * 0.0625f;
}
uint16_t orc_kv8_quantise(const float* y, int8_t* q, uint32_t n) {
  float amax = 0.0f;
  for (uint32_t i = 0; i < n; ++i) amax = std::fmax(amax, std::fabs(y[i]));
  const uint16_t s16 = orc_f32_to_f16_sat(amax / 127.0f);
  const float sf = orc_f16_to_f32(s16);
  for (uint32_t i = 0; i < n; ++i) {
    float r = sf == 0.0f ? 0.0f : std::nearbyint(y[i] / sf);
    r = std::fmin(std::fmax(r, -127.0f), 127.0f);
    q[i] = int8_t(r);
  }
  return s16;
}
uint16_t orc_kv8_encode256(const float* x, int8_t* q) {
  float y[256];
  orc_kv8_rotate256(x, y);
  return orc_kv8_quantise(y, q, 256);
}
float orc_kv8_dequant(int8_t q, uint16_t s16) { return float(q) * orc_f16_to_f32(s16); }

// attn_prep_kv8 (src/kernels/kv8.cl:287-408): attn_prep's chain unchanged, then q rotated
// in fp32, and the K row as the 16-bit cache would store it (rne of the roped value) and
// the V row (rne of the folded v) rotated and quantised into the int8 cache. head_dim 256.
void orc_attn_prep_kv8(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act,
                       uint32_t M, const float* partials, uint32_t S, const float* q_norm,
                       const float* k_norm, const float* rope, float* attn_q, float* attn_gate,
                       int8_t* kv_k, int8_t* kv_v, uint16_t* k_scale, uint16_t* v_scale,
                       size_t rs, size_t hs, size_t srs, size_t shs, const uint32_t* pages,
                       uint32_t page) {
  const Act A{act};
  const uint32_t HD = sh->head_dim, QH = sh->q_heads, KVH = sh->kv_heads;
  if (HD != 256) return;
  // the 16-bit values the fp16 cache would hold, at rows pos .. pos + n_act - 1
  const size_t rows = size_t(pos) + n_act;
  std::vector<uint16_t> k16(rows * KVH * HD), v16(rows * KVH * HD);
  orc_attn_prep(act, sh, pos, n_act, M, partials, S, q_norm, k_norm, rope, attn_q, attn_gate, k16.data(),
                v16.data(), size_t(KVH) * HD, HD, nullptr, 0);
  float x[256], y[256];
  for (uint32_t m = 0; m < n_act; ++m) {
    for (uint32_t h = 0; h < QH; ++h) {
      float* q = attn_q + (size_t(m) * QH + h) * HD;
      orc_kv8_rotate256(q, y);
      std::memcpy(q, y, sizeof y);
    }
    const size_t row = kv_row(pos + m, pages, page);
    for (uint32_t h = 0; h < KVH; ++h) {
      const size_t src = (size_t(pos + m) * KVH + h) * HD;
      for (uint32_t i = 0; i < HD; ++i) x[i] = A.w(k16[src + i]);
      k_scale[row * srs + h * shs] = orc_kv8_encode256(x, kv_k + row * rs + h * hs);
      for (uint32_t i = 0; i < HD; ++i) x[i] = A.w(v16[src + i]);
      v_scale[row * srs + h * shs] = orc_kv8_encode256(x, kv_v + row * rs + h * hs);
    }
  }
}

// attn_reduce_v2_kv8 (src/kernels/kv8.cl:814-860): attn_reduce_v2's merge, then the head's
// output un-rotated before the gate (or the plain rounding when ungated). head_dim 256.
void orc_attn_reduce_v2_kv8(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act,
                            uint32_t M, uint32_t tgt, const float* attn_part, const float* attn_gate,
                            uint16_t* attn_out) {
  const Act A{act};
  const uint32_t HD = sh->head_dim, QH = sh->q_heads, PART = HD + 2, OUT_N = QH * HD;
  if (HD != 256) return;
  float o[256], x[256];
  for (uint32_t h = 0; h < QH; ++h)
    for (uint32_t m = 0; m < n_act; ++m) {
      uint32_t nb = (pos + m) / orc_v2_ppw(pos + m + 1, tgt) + 1;
      if (nb > tgt) nb = tgt;
      for (uint32_t d = 0; d < HD; ++d) {
        float mx = ninf(), sm = 0.f, acc = 0.f;
        for (uint32_t b = 0; b < nb; ++b) {
          const float* p = attn_part + ((size_t(h) * tgt + b) * M + m) * PART;
          const float bmx = p[0], bsm = p[1], bacc = p[2 + d];
          const float nmx = std::fmax(mx, bmx);
          const float a = std::exp(mx - nmx);
          const float bs = std::exp(bmx - nmx);
          sm = std::fma(sm, a, bsm * bs);
          acc = std::fma(acc, a, bacc * bs);
          mx = nmx;
        }
        o[d] = acc / sm;
      }
      orc_kv8_unrotate256(o, x);
      for (uint32_t d = 0; d < HD; ++d) {
        uint16_t r;
        if (sh->gated && attn_gate)
          r = A.rne(A.w(A.rne(x[d])) * sigmoid_f32(attn_gate[(size_t(m) * QH + h) * HD + d]));
        else
          r = A.rne(x[d]);
        attn_out[size_t(m) * OUT_N + size_t(h) * HD + d] = r;
      }
    }
}

// ---- token boundary -----------------------------------------------------------------------
// src/kernels/embed_gather.cl:47-69: returns 0xDEAD0001 (and writes nothing) on a bad id
int orc_embed_gather(const uint32_t* ids, uint32_t M, const uint16_t* embed, uint32_t vocab,
                     uint32_t hidden, uint16_t* resid) {
  int flag = 0;
  for (uint32_t m = 0; m < M; ++m) {
    if (ids[m] >= vocab) {
      flag = int(0xDEAD0001u);
      continue;
    }
    std::memcpy(resid + size_t(m) * hidden, embed + size_t(ids[m]) * hidden, size_t(hidden) * 2);
  }
  return flag;
}
// src/kernels/argmax.cl:63-65 comparator; masked tail (index >= vocab_used) never wins
uint32_t orc_argmax(const float* logits, uint32_t vocab, uint32_t vocab_used) {
  float bv = ninf();
  uint32_t bi = 0x7FFFFFFFu;
  for (uint32_t k = 0; k < vocab; ++k) {
    const float v = k < vocab_used ? logits[k] : ninf();
    if (v > bv || (v == bv && k < bi)) {
      bv = v;
      bi = k;
    }
  }
  return bi;
}
// src/server/spec_accept.cc:81-85
uint32_t orc_accept_greedy(const uint32_t* verify_argmax, const uint32_t* drafts, uint32_t k,
                           uint32_t* next) {
  uint32_t j = 0;
  while (j < k && drafts[j] == verify_argmax[j]) ++j;
  if (next) *next = verify_argmax[j];
  return j;
}

// ---- MoE (tests/kernels/moe_ref.h:62-177) --------------------------------------------
void orc_moe_route_fn(int act, const float* logits, uint32_t E, uint32_t top_k, orc_moe_route* r) {
  const Act A{act};
  const uint32_t slots = top_k + 1;
  std::vector<float> l(E), ex(E), red(E), p(E);
  for (uint32_t e = 0; e < E; ++e) l[e] = A.rf(logits[e]);
  float mx = l[0];
  for (uint32_t j = 1; j < E; ++j) mx = std::fmax(mx, l[j]);
  for (uint32_t e = 0; e < E; ++e) red[e] = ex[e] = std::exp(l[e] - mx);
  for (uint32_t stride = E / 2; stride > 0; stride >>= 1)
    for (uint32_t e = 0; e < stride; ++e) red[e] += red[e + stride];
  for (uint32_t e = 0; e < E; ++e) p[e] = ex[e] / red[0];
  std::vector<uint32_t> top_id(slots);
  std::vector<float> top_p(slots, 0.0f);
  for (uint32_t k = 0; k < slots; ++k) top_id[k] = k;
  for (uint32_t e = 0; e < E; ++e) {
    uint32_t rank = 0;
    for (uint32_t j = 0; j < E; ++j) rank += (p[j] > p[e] || (p[j] == p[e] && j < e)) ? 1u : 0u;
    if (rank < slots) {
      top_id[rank] = e;
      top_p[rank] = p[e];
    }
  }
  std::memset(r, 0, sizeof *r);
  float s8 = 0.0f;
  for (uint32_t k = 0; k < top_k; ++k) s8 += top_p[k];
  for (uint32_t k = 0; k < top_k; ++k) {
    r->ids[k] = top_id[k];
    r->p[k] = top_p[k];
    r->w[k] = A.rf(top_p[k] / s8);
  }
  r->p9 = top_p[top_k];
  r->sg = A.rf(sigmoid_f32(A.rf(logits[E])));
}
// moe_ref.h:98-132 (tile_dot over K slices, merged by the pairwise tree)
float orc_moe_split_dot(int act, uint32_t layout, const uint32_t* words, const uint16_t* scales,
                        uint32_t K, uint32_t N, uint32_t n, const uint16_t* x, uint32_t ks) {
  const Act A{act};
  const WView v{K, N, layout, words, scales};
  std::vector<float> xf(K);
  for (uint32_t k = 0; k < K; ++k) xf[k] = A.w(x[k]);
  const uint32_t per = K / 64 / ks;
  std::vector<float> r(ks);
  for (uint32_t q = 0; q < ks; ++q) r[q] = group_range_dot(v, n, xf.data(), q * per, (q + 1) * per);
  for (uint32_t stride = ks / 2; stride > 0; stride >>= 1)
    for (uint32_t q = 0; q < stride; ++q) r[q] += r[q + stride];
  return r[0];
}
// moe_ref.h:134-138
uint16_t orc_moe_silu_up(int act, float gate_sum, float up_sum) {
  const Act A{act};
  const uint16_t g_b = A.rne(gate_sum), u_b = A.rne(up_sum);
  const uint16_t s_b = A.rne(silu_f32(A.w(g_b)));
  return A.rne(A.w(s_b) * A.w(u_b));
}
// moe_ref.h:144-152
uint16_t orc_moe_combine(int act, const float* down, const orc_moe_route* r, uint32_t top_k,
                         uint16_t resid) {
  const Act A{act};
  float sum = 0.0f;
  for (uint32_t k = 0; k < top_k; ++k) sum += A.w(A.rne(A.w(A.rne(down[k])) * r->w[k]));
  const uint16_t r_b = A.rne(sum);
  const uint16_t sh_b = A.rne(A.w(A.rne(down[top_k])) * r->sg);
  const uint16_t o_b = A.rne(A.w(r_b) + A.w(sh_b));
  return A.rne(A.w(resid) + A.w(o_b));
}
// moe_ref.h:154-177 (gate_up then down for one token)
void orc_moe_block(int act, uint32_t layout, uint32_t experts, uint32_t top_k, uint32_t hidden,
                   uint32_t inter, const orc_moe_route* r, const uint16_t* x,
                   const uint32_t* gu_words, const uint16_t* gu_scales, size_t gu_sw, size_t gu_ss,
                   const uint32_t* dn_words, const uint16_t* dn_scales, size_t dn_sw, size_t dn_ss,
                   uint32_t up_ks, uint32_t dn_ks, uint16_t* h_out, uint16_t* resid) {
  const uint32_t slots = top_k + 1;
  std::vector<uint16_t> h(size_t(slots) * inter);
  for (uint32_t slot = 0; slot < slots; ++slot) {
    const uint32_t e = slot < top_k ? r->ids[slot] : experts;
    const uint32_t* bw = gu_words + e * gu_sw;
    const uint16_t* bs = gu_scales ? gu_scales + e * gu_ss : nullptr;
    for (uint32_t i = 0; i < inter; ++i) {
      const uint32_t gc = (i / 16) * 32 + i % 16, uc = gc + 16;
      h[size_t(slot) * inter + i] =
          orc_moe_silu_up(act, orc_moe_split_dot(act, layout, bw, bs, hidden, 2 * inter, gc, x, up_ks),
                          orc_moe_split_dot(act, layout, bw, bs, hidden, 2 * inter, uc, x, up_ks));
    }
  }
  if (h_out) std::memcpy(h_out, h.data(), h.size() * 2);
  std::vector<float> d(slots);
  for (uint32_t n = 0; n < hidden; ++n) {
    for (uint32_t slot = 0; slot < slots; ++slot) {
      const uint32_t e = slot < top_k ? r->ids[slot] : experts;
      d[slot] = orc_moe_split_dot(act, layout, dn_words + e * dn_sw,
                                  dn_scales ? dn_scales + e * dn_ss : nullptr, inter, hidden, n,
                                  h.data() + size_t(slot) * inter, dn_ks);
    }
    resid[n] = orc_moe_combine(act, d.data(), r, top_k, resid[n]);
  }
}

// ---- fp16-weight GEMV (src/kernels/gemv_bf16.cl:103-200, weights fp16 in this build) -------
// The kernel's per-lane chain: acc = 0; per 8-k step `a += w * x` eight times in k order
// (gemv_bf16.cl:149-157, BF16_STEP); slices merged by the tree of :185-192.
void orc_gemv_f16w(int act, const uint16_t* w, const uint16_t* x, uint32_t M, uint32_t K, uint32_t N,
                   uint32_t ksplit, float* out) {
  const Act A{act};
  const uint32_t K8 = K / 8, per = K8 / ksplit;
  std::vector<float> red(ksplit);
  for (uint32_t m = 0; m < M; ++m)
    for (uint32_t n = 0; n < N; ++n) {
      const uint16_t* tile = w + size_t(n / 16) * K8 * 128;
      for (uint32_t q = 0; q < ksplit; ++q) {
        float acc = 0.f;
        for (uint32_t k8 = q * per; k8 < (q + 1) * per; ++k8)
          for (uint32_t j = 0; j < 8; ++j)
            acc += orc_f16_to_f32(tile[size_t(k8) * 128 + j * 16 + n % 16]) * A.w(x[size_t(m) * K + k8 * 8 + j]);
        red[q] = acc;
      }
      for (uint32_t stride = ksplit / 2; stride > 0; stride >>= 1)
        for (uint32_t q = 0; q < stride; ++q) red[q] += red[q + stride];
      out[size_t(m) * N + n] = red[0];
    }
}
// common::Bf16Tiled::from_rowmajor's element map (the layout gemv_bf16.cl reads)
void orc_f16w_tile(const uint16_t* w_rm, uint32_t K, uint32_t N, uint16_t* wt) {
  for (uint32_t n = 0; n < N; ++n)
    for (uint32_t k = 0; k < K; ++k)
      wt[(size_t(n / 16) * (K / 8) + k / 8) * 128 + (k % 8) * 16 + n % 16] = w_rm[size_t(n) * K + k];
}

// ---- dense decode step (src/runtime/capture.cc:997, 1247-1263, 1370-1423, 1461-1480) --------
// k_scale != NULL: the int8 rotated cache (kv8.cl's writer and readers, head_dim 256), int8 rows
// [layers][kv_heads][max_len][hd] and fp16 scales [layers][kv_heads][max_len]
// ---- the int8 lm_head ------------------------------------------------------------------------
// lm_head_int8.cc:22-37: the row's largest magnitude over 127, then w / s rounded to nearest even
// (nearbyint in the default mode) and clamped
float orc_quantise_row_int8(const float* w, uint32_t K, int8_t* q) {
  float amax = 0.f;
  for (uint32_t k = 0; k < K; ++k) amax = std::fmax(amax, std::fabs(w[k]));
  const float s = amax / 127.0f;
  for (uint32_t k = 0; k < K; ++k) {
    if (s == 0.f) {
      q[k] = 0;
      continue;
    }
    const float r = std::nearbyint(w[k] / s);
    q[k] = int8_t(std::min(127.f, std::max(-127.f, r)));
  }
  return s;
}
// ---- round-to-nearest int4 g64 of a bf16 linear (src/loader/rtn.h:35-60) ------------------------
// per output column n and group of 64 k: amax = max |w| (bf16 values in fp32), s16 =
// f16_rne(2 amax / 15), q = clamp(rint(w / f32(s16)) + 8, 0, 15); a zero group: s16 = 0, q = 8.
// GPTQ packing: qweight [K/8][N] (k = 8r + j in nibble j of word (r, n)), scales [K/64][N].
void orc_rtn_int4_g64(const uint16_t* w_bf16, uint32_t K, uint32_t N, uint32_t* qweight, uint16_t* scales) {
  for (uint32_t n = 0; n < N; ++n) {
    const uint16_t* row = w_bf16 + size_t(n) * K;
    for (uint32_t g = 0; g < K / 64; ++g) {
      float amax = 0.f;
      for (uint32_t k = g * 64; k < g * 64 + 64; ++k) amax = std::fmax(amax, std::fabs(orc_bf16_to_f32(row[k])));
      const uint16_t s16 = orc_f32_to_f16(2.0f * amax / 15.0f);
      scales[size_t(g) * N + n] = s16;
      const float s = orc_f16_to_f32(s16);
      for (uint32_t r = g * 8; r < g * 8 + 8; ++r) {
        uint32_t word = 0;
        for (uint32_t j = 0; j < 8; ++j) {
          float q = s > 0.f ? std::rint(orc_bf16_to_f32(row[r * 8 + j]) / s) + 8.0f : 8.0f;
          q = std::fmin(std::fmax(q, 0.0f), 15.0f);
          word |= uint32_t(q) << (4 * j);
        }
        qweight[size_t(r) * N + n] = word;
      }
    }
  }
}

// gemv_i8w.cl:67-105: one fp32 chain per column over k ascending, then the column's scale
void orc_gemv_i8w(int act, const int8_t* q, const float* s, const uint16_t* x, uint32_t M, uint32_t K, uint32_t N,
                  float* out) {
  const Act A{act};
  for (uint32_t m = 0; m < M; ++m) {
    std::vector<float> xf(K);
    for (uint32_t k = 0; k < K; ++k) xf[k] = A.w(x[size_t(m) * K + k]);
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < int64_t(N); ++n) {
      const int8_t* r = q + size_t(n) * K;
      float a = 0.f;
      for (uint32_t k = 0; k < K; ++k) a += float(r[k]) * xf[k];
      out[size_t(m) * N + n] = a * s[n];
    }
  }
}

// the model's head: the int4 lm_head (the twin's split-K order) or the int8 one
static void head_logits(int act, const orc_dense_model* md, const uint16_t* x, float* logits) {
  const Act A{act};
  const uint32_t H = md->hidden;
  if (md->lm_i8) {
    orc_gemv_i8w(act, md->lm_i8, md->lm_i8_scales, x, 1, H, md->vocab, logits);
    return;
  }
  std::vector<float> xf(H);
  for (uint32_t i = 0; i < H; ++i) xf[i] = A.w(x[i]);
  orc_gemv_twin(0, md->lm_head.qweight, md->lm_head.scales, H, md->vocab, xf.data(), 1, md->lm_head.S, logits);
}

static uint32_t dense_step(int act, const orc_dense_model* md, uint32_t tok, uint32_t pos, void* kv_k,
                           void* kv_v, uint16_t* k_scale, uint16_t* v_scale, float* logits,
                           uint32_t n_layers_run) {
  const Act A{act};
  const uint32_t H = md->hidden, HD = md->attn.head_dim, QH = md->attn.q_heads;
  const uint32_t KVH = md->attn.kv_heads, L = md->max_len;
  std::vector<uint16_t> resid(H), x(H), attn_out(size_t(QH) * HD), hbuf(md->inter);
  std::vector<float> xf(std::max<size_t>(size_t(H), std::max<size_t>(size_t(QH) * HD, md->inter)));
  std::vector<float> part, attn_q(size_t(QH) * HD), attn_part;
  orc_embed_gather(&tok, 1, md->embed, md->vocab, H, resid.data());
  std::vector<float> sumsq(std::max<uint32_t>(md->norm_g, 1));
  auto norm = [&](const float* partials, uint32_t s_prev, const float* w) {
    if (md->norm_g == 0) {
      orc_res_norm(act, partials, resid.data(), w, x.data(), 1, H, s_prev, md->rms_eps);
    } else {
      orc_res_fold(act, partials, resid.data(), sumsq.data(), 1, H, s_prev, md->norm_g);
      orc_norm_finish(act, sumsq.data(), resid.data(), w, x.data(), 1, H, md->norm_g, md->rms_eps);
    }
  };
  auto widen = [&](const uint16_t* v, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) xf[i] = A.w(v[i]);
  };
  auto linear = [&](const orc_linear& l, const uint16_t* in) {
    widen(in, l.K);
    part.assign(size_t(l.S) * l.N, 0.f);
    orc_gemv_twin_partials(0, l.qweight, l.scales, l.K, l.N, xf.data(), 1, l.S, part.data());
  };
  const uint32_t nl = std::min(n_layers_run, md->layers);
  uint32_t s_prev = 0;
  std::vector<float> prev;  // the previous down projection's partials
  for (uint32_t li = 0; li < nl; ++li) {
    const orc_layer& ly = md->layer[li];
    norm(prev.data(), s_prev, ly.in_norm);
    linear(ly.qkv, x.data());
    const size_t lo = size_t(li) * KVH * L * HD;
    attn_part.assign(size_t(QH) * md->tgt * (HD + 2), 0.f);
    if (k_scale) {  // capture.cc fa_layer under --kv-cache int8 (kv8.cl KV8_PREP / KV8_DEC)
      int8_t* lk = static_cast<int8_t*>(kv_k) + lo;
      int8_t* lv = static_cast<int8_t*>(kv_v) + lo;
      uint16_t* lks = k_scale + size_t(li) * KVH * L;
      uint16_t* lvs = v_scale + size_t(li) * KVH * L;
      orc_attn_prep_kv8(act, &md->attn, pos, 1, 1, part.data(), ly.qkv.S, ly.q_norm, ly.k_norm, md->rope,
                        attn_q.data(), nullptr, lk, lv, lks, lvs, HD, size_t(L) * HD, 1, L, nullptr, 0);
      orc_attn_decode_v2(act, &md->attn, pos, 1, 1, md->tgt, attn_q.data(), 1, lk, lv, lks, lvs, HD,
                         size_t(L) * HD, 1, L, nullptr, 0, attn_part.data());
      orc_attn_reduce_v2_kv8(act, &md->attn, pos, 1, 1, md->tgt, attn_part.data(), nullptr, attn_out.data());
    } else {
      uint16_t* lk = static_cast<uint16_t*>(kv_k) + lo;
      uint16_t* lv = static_cast<uint16_t*>(kv_v) + lo;
      orc_attn_prep(act, &md->attn, pos, 1, 1, part.data(), ly.qkv.S, ly.q_norm, ly.k_norm, md->rope,
                    attn_q.data(), nullptr, lk, lv, HD, size_t(L) * HD, nullptr, 0);
      orc_attn_decode_v2(act, &md->attn, pos, 1, 1, md->tgt, attn_q.data(), 0, lk, lv, nullptr, nullptr,
                         HD, size_t(L) * HD, 0, 0, nullptr, 0, attn_part.data());
      orc_attn_reduce_v2(act, &md->attn, pos, 1, 1, md->tgt, attn_part.data(), nullptr, attn_out.data());
    }
    linear(ly.o, attn_out.data());
    norm(part.data(), ly.o.S, ly.post_norm);
    if (md->experts) {
      // capture.cc:1295 moe_block: router || shared gate, route, experts; moe_down folds its
      // output into the residual itself, so the next norm folds nothing (moe.cl:36-38)
      const uint32_t H2 = md->hidden;
      std::vector<float> lg(md->router_n);
      orc_gemv_f16w(act, ly.router, x.data(), 1, H2, md->router_n, md->router_ksplit, lg.data());
      orc_moe_route r;
      orc_moe_route_fn(act, lg.data(), md->experts, md->top_k, &r);
      const size_t gub = size_t(2 * md->moe_inter / 16) * (H2 / 64) * 136;
      const size_t dnb = size_t(H2 / 16) * (md->moe_inter / 64) * 136;
      orc_moe_block(act, 1, md->experts, md->top_k, H2, md->moe_inter, &r, x.data(), ly.moe_gu, nullptr, gub, 0,
                    ly.moe_dn, nullptr, dnb, 0, 4, 2, nullptr, resid.data());
      prev.clear();
      s_prev = 0;
      continue;
    }
    linear(ly.gate_up, x.data());
    orc_silu_mul(act, part.data(), hbuf.data(), 1, md->inter, ly.gate_up.S);
    linear(ly.down, hbuf.data());
    prev = part;
    s_prev = ly.down.S;
  }
  if (nl < md->layers) return 0;
  norm(prev.data(), s_prev, md->final_norm);
  head_logits(act, md, x.data(), logits);
  return orc_argmax(logits, md->vocab, md->vocab_used);
}

uint32_t orc_dense_step(int act, const orc_dense_model* md, uint32_t tok, uint32_t pos, uint16_t* kv_k,
                        uint16_t* kv_v, float* logits, uint32_t n_layers_run) {
  return dense_step(act, md, tok, pos, kv_k, kv_v, nullptr, nullptr, logits, n_layers_run);
}
uint32_t orc_dense_step_kv8(int act, const orc_dense_model* md, uint32_t tok, uint32_t pos, int8_t* kv_k,
                            int8_t* kv_v, uint16_t* k_scale, uint16_t* v_scale, float* logits,
                            uint32_t n_layers_run) {
  if (md->attn.head_dim != 256 || !k_scale || !v_scale) return 0xFFFFFFFFu;
  return dense_step(act, md, tok, pos, kv_k, kv_v, k_scale, v_scale, logits, n_layers_run);
}


// ---- the MTP head (src/runtime/capture.cc:1772-1939) ----------------------------------------
uint32_t orc_mtp_head_step(int act, const orc_dense_model* md, const orc_mtp_head* hd, uint32_t tok,
                           const uint16_t* h, uint32_t p, uint16_t* kv_k, uint16_t* kv_v, int full,
                           uint16_t* h_out, float* logits) {
  const Act A{act};
  const uint32_t H = md->hidden, HD = md->attn.head_dim, QH = md->attn.q_heads, L = md->max_len;
  const uint32_t G = H / 64;
  if (p >= L || (!hd->w16_fc && (hd->fc.K != 2 * H || hd->fc.N != H))) return 0xFFFFFFFFu;
  std::vector<uint16_t> resid(H), hrow(h, h + H), x2(size_t(2) * H), x(H), attn_out(size_t(QH) * HD);
  std::vector<uint16_t> hbuf(md->inter);
  std::vector<float> sumsq(G), part, attn_q(size_t(QH) * HD), attn_part;
  std::vector<float> xf(std::max<size_t>({size_t(2) * H, size_t(QH) * HD, size_t(md->inter)}));
  const orc_layer& ly = hd->layer;
  // one linear into `part`: the int4 twin's S slices, or (w16) the 16-bit GEMV's one slice;
  // returns the slice count the fold that follows takes
  auto linear = [&](const orc_linear& l, const uint16_t* w16, uint32_t K, uint32_t N, const uint16_t* in) {
    if (w16) {
      uint32_t ks = 16;
      while (ks > 1 && (K / 8) % ks) ks /= 2;
      part.assign(N, 0.f);
      orc_gemv_f16w(act, w16, in, 1, K, N, ks, part.data());
      return 1u;
    }
    for (uint32_t i = 0; i < l.K; ++i) xf[i] = A.w(in[i]);
    part.assign(size_t(l.S) * l.N, 0.f);
    orc_gemv_twin_partials(0, l.qweight, l.scales, l.K, l.N, xf.data(), 1, l.S, part.data());
    return l.S;
  };
  const uint32_t qkv_n = (QH + 2 * md->attn.kv_heads) * HD;
  auto norm = [&](const float* partials, uint32_t s_prev, const float* w) {  // as orc_dense_step's
    if (md->norm_g == 0) {
      orc_res_norm(act, partials, resid.data(), w, x.data(), 1, H, s_prev, md->rms_eps);
    } else {
      std::vector<float> sq(md->norm_g);
      orc_res_fold(act, partials, resid.data(), sq.data(), 1, H, s_prev, md->norm_g);
      orc_norm_finish(act, sq.data(), resid.data(), w, x.data(), 1, H, md->norm_g, md->rms_eps);
    }
  };
  // head_front: enorm(embed(tok)) into x2[0, H), hnorm(h) into x2[H, 2H) (prep_norm_finish with
  // X_STRIDE = 2 hidden), both after prep_res_fold with nothing to fold
  if (orc_embed_gather(&tok, 1, md->embed, md->vocab, H, resid.data())) return 0xFFFFFFFFu;
  orc_res_fold(act, nullptr, resid.data(), sumsq.data(), 1, H, 0, G);
  orc_norm_finish(act, sumsq.data(), resid.data(), hd->pre_e, x2.data(), 1, H, G, md->rms_eps);
  orc_res_fold(act, nullptr, hrow.data(), sumsq.data(), 1, H, 0, G);
  orc_norm_finish(act, sumsq.data(), hrow.data(), hd->pre_h, x2.data() + H, 1, H, G, md->rms_eps);
  const uint32_t s_fc = linear(hd->fc, hd->w16_fc, 2 * H, H, x2.data());
  // ZERO_RESID (prep.cl:308-309): the residual stream starts at fc's output, rne(sum_s partials)
  for (uint32_t k = 0; k < H; ++k) {
    float acc = 0.f;
    for (uint32_t s = 0; s < s_fc; ++s) acc += part[size_t(s) * H + k];
    resid[k] = A.rne(acc);
  }
  orc_res_fold(act, nullptr, resid.data(), sumsq.data(), 1, H, 0, G);
  orc_norm_finish(act, sumsq.data(), resid.data(), ly.in_norm, x.data(), 1, H, G, md->rms_eps);
  const uint32_t s_qkv = linear(ly.qkv, hd->w16_qkv, H, qkv_n, x.data());
  orc_attn_prep(act, &md->attn, p, 1, 1, part.data(), s_qkv, ly.q_norm, ly.k_norm, md->rope, attn_q.data(),
                nullptr, kv_k, kv_v, HD, size_t(L) * HD, nullptr, 0);
  if (!full) return 0;
  // draft(): the attention pair over the head's keys 0..p, o and the post-attention norm, the MLP,
  // the head's final norm, the shared lm_head
  attn_part.assign(size_t(QH) * md->tgt * (HD + 2), 0.f);
  orc_attn_decode_v2(act, &md->attn, p, 1, 1, md->tgt, attn_q.data(), 0, kv_k, kv_v, nullptr, nullptr, HD,
                     size_t(L) * HD, 0, 0, nullptr, 0, attn_part.data());
  orc_attn_reduce_v2(act, &md->attn, p, 1, 1, md->tgt, attn_part.data(), nullptr, attn_out.data());
  const uint32_t s_o = linear(ly.o, hd->w16_o, QH * HD, H, attn_out.data());
  norm(part.data(), s_o, ly.post_norm);
  if (md->experts) {  // an MoE model's head (spec 15e): one MoE layer of the model's shape
    std::vector<float> lg(md->router_n);
    orc_gemv_f16w(act, ly.router, x.data(), 1, H, md->router_n, md->router_ksplit, lg.data());
    orc_moe_route r;
    orc_moe_route_fn(act, lg.data(), md->experts, md->top_k, &r);
    const size_t gub = size_t(2 * md->moe_inter / 16) * (H / 64) * 136;
    const size_t dnb = size_t(H / 16) * (md->moe_inter / 64) * 136;
    orc_moe_block(act, 1, md->experts, md->top_k, H, md->moe_inter, &r, x.data(), ly.moe_gu, nullptr, gub, 0,
                  ly.moe_dn, nullptr, dnb, 0, 4, 2, nullptr, resid.data());
    norm(nullptr, 0, hd->final_norm);
  } else {
    const uint32_t s_gu = linear(ly.gate_up, hd->w16_gu, H, 2 * md->inter, x.data());
    orc_silu_mul(act, part.data(), hbuf.data(), 1, md->inter, s_gu);
    const uint32_t s_dn = linear(ly.down, hd->w16_dn, md->inter, H, hbuf.data());
    norm(part.data(), s_dn, hd->final_norm);
  }
  if (h_out) std::copy(x.begin(), x.end(), h_out);
  head_logits(act, md, x.data(), logits);
  return orc_argmax(logits, md->vocab, md->vocab_used);
}

// ---- the chunked prefill (src/runtime/prefill/step.h step_chunk; this build's
// Engine::prefill_chunk walk) ---------------------------------------------------------------
// The prefill's own roundings: every int4 weight dequantised ONCE to act, w = rne((q - 8) * s)
// (pf_dequant_slab.cl's slab), and each output the fp32 sum over k ascending of w * x (the
// products are exact in fp32); the residual, norms, SiLU and attention prep are the decode twins
// at one slice (S = 1) over the chunk's T rows; the causal attention of row t over keys
// [0, pos + t] in fp64, rounded once (the prefill kernel's fp32-accurate flash attention).
static void prefill_gemm(const Act& A, const orc_linear& l, const uint16_t* x, uint32_t T, float* out) {
  const uint32_t K = l.K, N = l.N;
  std::vector<float> w(size_t(K) * N);
  for (uint32_t k = 0; k < K; ++k)
    for (uint32_t n = 0; n < N; ++n) {
      const int q = int((l.qweight[size_t(k / 8) * N + n] >> (4 * (k % 8))) & 0xFu) - 8;
      w[size_t(k) * N + n] = A.rf(float(q) * orc_f16_to_f32(l.scales[size_t(k / 64) * N + n]));
    }
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < int64_t(T); ++t) {
    std::vector<float> xf(K);
    for (uint32_t k = 0; k < K; ++k) xf[k] = A.w(x[size_t(t) * K + k]);
    float* o = out + size_t(t) * N;
    for (uint32_t n = 0; n < N; ++n) o[n] = 0.f;
    for (uint32_t k = 0; k < K; ++k) {
      const float xv = xf[k];
      const float* wr = w.data() + size_t(k) * N;
      for (uint32_t n = 0; n < N; ++n) o[n] += wr[n] * xv;
    }
  }
}

uint32_t orc_prefill_chunk(int act, const orc_dense_model* md, const uint32_t* ids, uint32_t T, uint32_t pos,
                           uint16_t* kv_k, uint16_t* kv_v, float* logits) {
  if (T == 0 || size_t(pos) + T > md->max_len) return 0xFFFFFFFFu;
  const Act A{act};
  const uint32_t H = md->hidden, HD = md->attn.head_dim, QH = md->attn.q_heads, KVH = md->attn.kv_heads;
  const uint32_t L = md->max_len, G = QH / KVH, QHD = QH * HD;
  std::vector<uint16_t> resid(size_t(T) * H), x(size_t(T) * H), attn(size_t(T) * QHD), h(size_t(T) * md->inter);
  std::vector<float> out, attn_q(size_t(T) * QHD);
  if (orc_embed_gather(ids, T, md->embed, md->vocab, H, resid.data())) return 0xFFFFFFFFu;
  orc_res_norm(act, nullptr, resid.data(), md->layer[0].in_norm, x.data(), T, H, 0, md->rms_eps);
  for (uint32_t li = 0; li < md->layers; ++li) {
    const orc_layer& ly = md->layer[li];
    const size_t lo = size_t(li) * KVH * L * HD;
    uint16_t* lk = kv_k + lo;
    uint16_t* lv = kv_v + lo;
    out.assign(size_t(T) * ly.qkv.N, 0.f);
    prefill_gemm(A, ly.qkv, x.data(), T, out.data());
    orc_attn_prep(act, &md->attn, pos, T, T, out.data(), 1, ly.q_norm, ly.k_norm, md->rope, attn_q.data(), nullptr,
                  lk, lv, HD, size_t(L) * HD, nullptr, 0);
#pragma omp parallel for schedule(static)
    for (int64_t th = 0; th < int64_t(T) * QH; ++th) {
      const uint32_t t = uint32_t(th / QH), hh = uint32_t(th % QH);
      std::vector<double> o(HD);
      orc_attend64(&md->attn, attn_q.data() + (size_t(t) * QH + hh) * HD, hh / G, pos + t + 1, 0, act, lk, lv,
                   nullptr, nullptr, HD, size_t(L) * HD, 0, 0, nullptr, 0, o.data());
      for (uint32_t dd = 0; dd < HD; ++dd) attn[size_t(t) * QHD + size_t(hh) * HD + dd] = A.rne(float(o[dd]));
    }
    out.assign(size_t(T) * H, 0.f);
    prefill_gemm(A, ly.o, attn.data(), T, out.data());
    orc_res_norm(act, out.data(), resid.data(), ly.post_norm, x.data(), T, H, 1, md->rms_eps);
    const float* next_w = li + 1 < md->layers ? md->layer[li + 1].in_norm : md->final_norm;
    if (md->experts) {
      // the MoE block over the chunk: the router GEMV and the route of every row (the decode
      // twins, row by row), the experts as pf_moe_ref's values, then the next norm (moe_down
      // folds its output into the residual itself)
      std::vector<float> lg(size_t(T) * md->router_n);
      orc_gemv_f16w(act, ly.router, x.data(), T, H, md->router_n, md->router_ksplit, lg.data());
      std::vector<uint32_t> route(size_t(T) * 32, 0u);
      for (uint32_t t = 0; t < T; ++t) {
        orc_moe_route r;
        orc_moe_route_fn(act, lg.data() + size_t(t) * md->router_n, md->experts, md->top_k, &r);
        uint32_t* rw = route.data() + size_t(t) * 32;
        for (uint32_t j = 0; j < md->top_k; ++j) {
          rw[j] = r.ids[j];
          std::memcpy(rw + 8 + j, &r.w[j], 4);
          std::memcpy(rw + 17 + j, &r.p[j], 4);
        }
        std::memcpy(rw + 16, &r.sg, 4);
        std::memcpy(rw + 25, &r.p9, 4);
      }
      orc_moe_prefill(act, md->experts, md->top_k, H, md->moe_inter, route.data(), x.data(), ly.moe_gu, ly.moe_dn,
                      resid.data(), T);
      orc_res_norm(act, nullptr, resid.data(), next_w, x.data(), T, H, 0, md->rms_eps);
      continue;
    }
    out.assign(size_t(T) * ly.gate_up.N, 0.f);
    prefill_gemm(A, ly.gate_up, x.data(), T, out.data());
    orc_silu_mul(act, out.data(), h.data(), T, md->inter, 1);
    out.assign(size_t(T) * H, 0.f);
    prefill_gemm(A, ly.down, h.data(), T, out.data());
    orc_res_norm(act, out.data(), resid.data(), next_w, x.data(), T, H, 1, md->rms_eps);
  }
  // the last row's head on the decode GEMV (the engine runs the step's lm_head launch)
  head_logits(act, md, x.data() + size_t(T - 1) * H, logits);
  return orc_argmax(logits, md->vocab, md->vocab_used);
}


// ---- the chunk's MoE block (tests/kernels/pf_moe_ref.h: pf_moe_sort / dequant / grouped GEMM /
// combine) -----------------------------------------------------------------------------------
// The values pf_moe_ref's chain gives every (token, slot) pair, token by token (the sort only
// places the rows; no value depends on it): the expert's layout-1 blocks dequantised once,
// w = rne((q - 8) * scale) (dequant_block); gate||up = fp32 sums of x w in ascending k
// (gemm_rows); h = silu_up per intermediate column (silu_row); y = rne(fp32 sums of h w_down)
// (the down outputs, rounded); then combine_token: sum_j rne(y_j w_j) in slot order from +0,
// r = rne(sum), sh = rne(y_shared sg), o = rne(r + sh), resid = rne(resid + o). A slot's id
// past the last expert is clamped to it (pf_moe_sort's byte staging).
static std::vector<float> dequant_layout1(const Act& A, const uint32_t* blk, uint32_t K, uint32_t N) {
  std::vector<float> out(size_t(K) * N);
  const uint32_t G = K / 64;
  for (uint32_t n = 0; n < N; ++n)
    for (uint32_t g = 0; g < G; ++g) {
      const uint32_t* tile = blk + (size_t(n / 16) * G + g) * 136;
      uint16_t sh;
      std::memcpy(&sh, reinterpret_cast<const uint16_t*>(tile + 128) + n % 16, 2);
      const float scale = orc_f16_to_f32(sh);
      for (uint32_t j = 0; j < 8; ++j) {
        const uint32_t word = tile[j * 16 + n % 16];
        for (uint32_t i = 0; i < 8; ++i) {
          const int q = int((word >> (4 * i)) & 0xFu) - 8;
          out[size_t(g * 64 + j * 8 + i) * N + n] = A.rf(float(q) * scale);
        }
      }
    }
  return out;
}

void orc_moe_prefill(int act, uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                     const uint32_t* route, const uint16_t* x, const uint32_t* gu_blocks, const uint32_t* dn_blocks,
                     uint16_t* resid, uint32_t T) {
  const Act A{act};
  const uint32_t E = experts, slots = top_k + 1, N2 = 2 * inter;
  const size_t gub = size_t(N2 / 16) * (hidden / 64) * 136, dnb = size_t(hidden / 16) * (inter / 64) * 136;
  auto expert = [&](uint32_t t, uint32_t j) -> uint32_t {
    if (j == top_k) return E;
    return std::min(route[size_t(t) * 32 + j], E - 1);
  };
  // expert by expert (each block dequantised once, then every pair routed to it)
  std::vector<std::vector<uint32_t>> pairs(E + 1);
  for (uint32_t t = 0; t < T; ++t)
    for (uint32_t j = 0; j < slots; ++j) pairs[expert(t, j)].push_back(t * slots + j);
  std::vector<float> y(size_t(T) * slots * hidden);  // the rounded down outputs
  for (uint32_t e = 0; e <= E; ++e) {
    if (pairs[e].empty()) continue;
    const std::vector<float> gw = dequant_layout1(A, gu_blocks + e * gub, hidden, N2);
    const std::vector<float> dw = dequant_layout1(A, dn_blocks + e * dnb, inter, hidden);
    const std::vector<uint32_t>& pe = pairs[e];
#pragma omp parallel for schedule(dynamic)
    for (int64_t pi = 0; pi < int64_t(pe.size()); ++pi) {
      const uint32_t p = pe[size_t(pi)], t = p / slots;
      std::vector<float> gu(N2, 0.f), hf(inter);
      for (uint32_t k = 0; k < hidden; ++k) {
        const float av = A.w(x[size_t(t) * hidden + k]);
        const float* wr = gw.data() + size_t(k) * N2;
        for (uint32_t n = 0; n < N2; ++n) gu[n] += av * wr[n];
      }
      for (uint32_t i = 0; i < inter; ++i) {
        const uint32_t gc = (i / 16) * 32 + i % 16;
        const uint16_t g_b = A.rne(gu[gc]), u_b = A.rne(gu[gc + 16]);
        const uint16_t s_b = A.rne(silu_f32(A.w(g_b)));
        hf[i] = A.w(A.rne(A.w(s_b) * A.w(u_b)));
      }
      float* yo = y.data() + size_t(p) * hidden;
      for (uint32_t n = 0; n < hidden; ++n) yo[n] = 0.f;
      for (uint32_t k = 0; k < inter; ++k) {
        const float* wr = dw.data() + size_t(k) * hidden;
        for (uint32_t n = 0; n < hidden; ++n) yo[n] += hf[k] * wr[n];
      }
      for (uint32_t n = 0; n < hidden; ++n) yo[n] = A.rf(yo[n]);
    }
  }
  for (uint32_t t = 0; t < T; ++t) {
    const uint32_t* row = route + size_t(t) * 32;
    const float* yt = y.data() + size_t(t) * slots * hidden;
    float sg;
    std::memcpy(&sg, row + 16, 4);
    for (uint32_t n = 0; n < hidden; ++n) {
      float sum = 0.f;
      for (uint32_t j = 0; j < top_k; ++j) {
        float w;
        std::memcpy(&w, row + 8 + j, 4);
        sum += A.rf(yt[size_t(j) * hidden + n] * w);
      }
      const uint16_t r_b = A.rne(sum);
      const uint16_t sh_b = A.rne(yt[size_t(top_k) * hidden + n] * sg);
      const uint16_t o_b = A.rne(A.w(r_b) + A.w(sh_b));
      uint16_t* rp = resid + size_t(t) * hidden + n;
      *rp = A.rne(A.w(*rp) + A.w(o_b));
    }
  }
}

}  // extern "C"
