// gemv_core.h - the pieces of the W4A16 g64 linear shared by its kernels (gemv_w4a16.hip, the
// attention and MoE kernels' hand-offs): the register-local int4 dequantisation into MFMA
// operands and the hand-off words' empty pattern.
#pragma once
#include "mi_common.h"

namespace mi {

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

// Keeps a batch of four MFMAs with one A operand in distinct registers: A, every B and every
// full result stay in their own registers until the batch has been issued, so no destination
// overlaps a source or another result of the batch. Without it the register allocator may give
// the batch's last MFMA the shared A operand's registers as its destination while the earlier
// MFMAs may still be reading them; under register pressure that corrupted the middle products
// of a batch on gfx950.
__device__ __forceinline__ void keep_mfma_batch(const h8_t& a, const h8_t (&b)[4], const f4_t (&d)[4]) {
  asm volatile("" ::"v"(a), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]));
  asm volatile("" ::"v"(d[0]), "v"(d[1]), "v"(d[2]), "v"(d[3]));
}

constexpr uint32_t kEmpty = 0xFFFFFFFFu;  // a hand-off word with no value yet

__device__ __forceinline__ float empty_f() { return __builtin_bit_cast(float, kEmpty); }
__device__ __forceinline__ bool is_empty(float v) { return __builtin_bit_cast(uint32_t, v) == kEmpty; }
// a computed value never goes out with the empty pattern (it stays a NaN)
__device__ __forceinline__ float publishable(float v) {
  return is_empty(v) ? __builtin_bit_cast(float, 0x7FC00000u) : v;
}
// a pair of f16 values as one hand-off word: (lo, hi) never both 0xFFFF (an f16 NaN with every
// payload bit set becomes the canonical f16 NaN)
__device__ __forceinline__ uint32_t publishable_pair(uint16_t lo, uint16_t hi) {
  const uint32_t w = (uint32_t)lo | ((uint32_t)hi << 16);
  return w == kEmpty ? 0x7E007E00u : w;
}

constexpr uint32_t kStatusTimeout = 0xDEAD0003u;  // the status word's value after a wait gave up


}  // namespace mi
