// mi_common.h - device-side helpers shared by the decode-loop kernels (gfx950, wave64).
//
// Arithmetic contract (the reference's rounding discipline, src/kernels/prep.cl and
// tests/kernels/prep_ref.h:1-40, with fp16 activations in place of bf16):
//   * every library file is compiled with -ffp-contract=off; a fused multiply-add appears
//     only where it is spelled (__builtin_fmaf) and where the reference spells `fma`;
//   * `1.0f / sqrtf(x)` is a correctly rounded sqrt and divide (hipcc's default for fp32),
//     never an rsqrt;
//   * activations are IEEE binary16, rounded to nearest even with subnormals kept
//     (v_cvt_f16_f32);
//   * exp is the library expf (1 ulp), the one op whose result may differ from the host's.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {

typedef _Float16 half_t;
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

// The control block (src/runtime/control.h:13-24): the only per-token state the host
// and the captured step share, read by the kernels at execution time.
enum : uint32_t {
  CTRL_POS = 0,        // position of token 0 of this step
  CTRL_NACT = 1,       // active rows this step
  CTRL_CUR = 2,        // cur_token[8]: ids the step embeds
  CTRL_OUT = 10,       // out_token[8]: the step's argmax per row
  CTRL_DEBUG = 18,     // 0xDEAD0001: an id outside the embedding table
  CTRL_STEPS = 19,     // steps completed since the last reset (history index)
  CTRL_WIDE_CUR = 32,  // wide_cur[16] / wide_out[16]: a 9..16-row list's ids (control.h:35-38)
  CTRL_WIDE_OUT = 48,
  CTRL_DEEP_CUR = 64,  // deep_cur[64] / deep_out[64]: a 17..64-row list's (control.h:39-42)
  CTRL_DEEP_OUT = 128,
  CTRL_WORDS = 192
};
constexpr uint32_t kStatusNonFinite = 0xDEAD0004u;  // CTRL_DEBUG: a logit was not finite
constexpr uint32_t kNanBits = 0x7FC00000u;          // the canonical fp32 NaN

// threadIdx.x as a value the compiler cannot hoist: lane-derived addresses are then recomputed
// where they are used instead of being hoisted out of a long loop and held in registers.
__device__ __forceinline__ uint32_t opaque_tid() {
  uint32_t v = threadIdx.x;
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(half_t, h); }
// fp32 -> f16 RNE of an fp32 value that has been rounded to fp32 first. The empty asm
// pins `f` in a VGPR, so the backend cannot fold the producing multiply or add into a
// v_fma_mix*_f16 (which rounds once, straight to f16: a double-rounding difference
// from the reference's fp32 op followed by the conversion).
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (half_t)f);
}
// bf16, the reference's activation type (common/bf16.h:8-16): widening is exact, narrowing is
// round-to-nearest-even on the fp32 bits. A NaN stays a NaN (the bit formula alone can carry a
// NaN with a full payload into a zero; finite values and infinities round as the formula says).
__device__ __forceinline__ float bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
  asm("" : "+v"(f));
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  if (f != f) return (uint16_t)0x7FC0u;
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
// The activation type of a step: act 0 = f16, 1 = bf16. Under bf16 every rounding point of the
// step rounds to bf16 (rne_bf16 where the reference has it), and the activations that feed a
// linear or the attention (the normed x, SwiGLU's h, the attention output, the K/V rows) are
// stored as the f16 encoding of that bf16 value: a bf16 value of magnitude in [2^-17, 65504]
// is exact in f16 (8 significant bits), so the GEMV and attention kernels read the same
// numbers either way; a larger one is stored as inf, which the logits' finiteness check then
// reports. The residual stream, which grows past the f16 range, is stored as bf16 bits.
__device__ __forceinline__ float act_round(float f, uint32_t act) { return act ? bf2f(f2bf(f)) : h2f(f2h(f)); }
__device__ __forceinline__ uint16_t act_enc(float f, uint32_t act) { return act ? f2h(bf2f(f2bf(f))) : f2h(f); }
__device__ __forceinline__ float res_widen(uint16_t b, uint32_t act) { return act ? bf2f(b) : h2f(b); }
__device__ __forceinline__ uint16_t res_rne(float f, uint32_t act) { return act ? f2bf(f) : f2h(f); }

__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t h2_bits(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// silu / sigmoid with plain exp (prep.cl:384 / attn_v2.cl:133 spell them this way)
__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

// v_and_or_b32 with both constants in registers (a literal pair cannot be encoded).
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(mask), "v"(magic));
  return r;
}

// A pointer into global memory, typed so: the compiler then emits global_* instructions, which
// count only in the vector memory counter. Through a generic pointer it emits flat_*, which count
// in the LDS/scalar counter as well, so every later LDS wait or barrier would also wait for them
// (for a weight prefetch or a hand-off store still in flight).
template <typename T>
using gptr = __attribute__((address_space(1))) T*;
template <typename T>
__device__ __forceinline__ gptr<T> as_global(T* p) {
  return (gptr<T>)p;
}

// Streaming 16-byte load that does not allocate in the caches (weights are read once per
// token; keeping them out of L2/MALL leaves room for activations and partials).
__device__ __forceinline__ u4_t load_stream16(const uint32_t* p) {
  return __builtin_nontemporal_load(as_global(reinterpret_cast<const u4_t*>(p)));
}

// Device-coherent (agent scope) accesses for data that work-groups of one launch hand to
// each other: relaxed atomics, which the compiler emits as sc1 loads and stores that are
// coherent across the XCDs' L2s without any cache writeback or invalidate.
template <typename T>
__device__ __forceinline__ void st_agent(T* p, T v) {
  __hip_atomic_store(as_global(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_agent(const T* p) {
  return __hip_atomic_load(as_global(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Whole-wave reductions on the vector ALUs: a butterfly inside each 16-lane row through DPP
// lane swaps (quad_perm xor 1, xor 2, half-mirror, mirror), then the four row results via
// readlane. Every lane gets the result. (The cross-lane shuffle through ds_bpermute costs an
// LDS round trip per step.) The summation order is fixed, so results are deterministic.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

// Orders LDS between the lanes of one wave: lanes that hand data to each other through LDS
// need it between the writes and the reads (and before the next writes). Without it the
// compiler may keep a lane's earlier LDS value in a register (another lane's store is a data
// race to it). The hardware already executes one wave's LDS operations in order.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

// A work-group barrier that orders LDS only: it waits for this wave's LDS operations, not
// for its global loads, so loads issued before it (a prefetch) stay in flight across it.
// Use it where the barrier guards LDS data alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// Waits until this thread's memory operations have completed (vector memory counter 0),
// and keeps the compiler from moving memory operations across the wait.
__device__ __forceinline__ void wait_memory() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- the int8 KV cache's rotation and quantiser (src/common/kv8.h:1-26, :56-156) ----
// R = H_256 diag(s) / 16 with Sylvester H in natural order and s the fixed sign vector (bit j
// of word j / 32 set when s[j] = -1); rotate(x)[j] = s[j] FWHT(x)[j] / 16, unrotate(y)[i] =
// FWHT(s * y)[i] / 16. The FWHT's stages run h = 1, 2, ..., 128, the pair (i, i + h) with
// i & h == 0 becoming (a + c, a - c): each element's chain of fp32 operations is fixed, so any
// schedule that performs the same operations gives the same bits.
__device__ __forceinline__ bool kv8_sign_neg(uint32_t j) {
  constexpr uint32_t kSigns[8] = {0xA197D809u, 0xA6850592u, 0xB205A73Eu, 0x20AFA769u,
                                  0x45C2CF64u, 0xBEAEAACBu, 0x75F39ADDu, 0x2385A70Cu};
  uint32_t w = kSigns[0];
#pragma unroll
  for (uint32_t k = 1; k < 8; ++k) w = (j >> 5) == k ? kSigns[k] : w;  // no memory lookup
  return (w >> (j & 31u)) & 1u;
}
__device__ __forceinline__ float kv8_flip(float v, bool neg) {
  return __uint_as_float(__float_as_uint(v) ^ (neg ? 0x80000000u : 0u));
}
// N independent 256-point FWHTs across a 256-thread work-group, thread i holding element i of
// each. Stages 1..32 stay inside the wave (lane exchanges); stages 64 and 128 take one LDS
// round: every thread reads the four elements i & 63 + 64 k and performs the two stages'
// operations on them in the same form (a + c for the lower index, a - c for the upper).
// Every thread of the work-group must call it; `xch` is N * 256 floats of LDS, free on entry
// and on return.
template <int N>
__device__ __forceinline__ void fwht256(float (&v)[N], uint32_t i, float* xch) {
#pragma unroll
  for (uint32_t h = 1; h < 64; h <<= 1)
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const float o = __shfl_xor(v[n], (int)h, 64);
      v[n] = (i & h) ? (o - v[n]) : (v[n] + o);
    }
#pragma unroll
  for (int n = 0; n < N; ++n) xch[n * 256 + i] = v[n];
  lds_barrier();
  const uint32_t lo = i & 63u, q = i >> 6;
#pragma unroll
  for (int n = 0; n < N; ++n) {
    const float a0 = xch[n * 256 + lo], a1 = xch[n * 256 + lo + 64];
    const float a2 = xch[n * 256 + lo + 128], a3 = xch[n * 256 + lo + 192];
    // stage 64: elements lo, lo+64 from (a0, a1); lo+128, lo+192 from (a2, a3)
    const float w_lo = (q & 1u) ? (a0 - a1) : (a0 + a1);    // this thread's slot within its pair
    const float w_hi = (q & 1u) ? (a2 - a3) : (a2 + a3);
    // stage 128: the lower half adds its partner 128 up, the upper half subtracts itself
    v[n] = (q & 2u) ? (w_lo - w_hi) : (w_lo + w_hi);
  }
  lds_barrier();
}
// binary16 round-to-nearest-even of a non-negative finite scale, subnormals kept, values at or
// above 65504 saturated (kv8.h:56-72's f32_to_f16_rne)
__device__ __forceinline__ uint16_t kv8_f16_sat(float f) { return f2h(fminf(f, 65504.0f)); }
// kv8.h:103-114: the row's amax (exact in any order), s16 = f16(amax / 127) correctly
// rounded, q = s16 == 0 ? 0 : clamp(rint(y / f16f(s16)), -127, 127). `amax` is the row's max.
__device__ __forceinline__ int8_t kv8_quant(float y, float sf) {
  float r = sf == 0.0f ? 0.0f : rintf(y / sf);
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int8_t)(int)r;
}

// Launch helper: returns the launch error as an int.
#define MI_LAUNCH_CHECK() return (int)hipGetLastError()

}  // namespace mi
