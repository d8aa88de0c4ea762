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
  CTRL_WORDS = 64
};

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(half_t, h); }
// fp32 -> f16 RNE of an fp32 value that has been rounded to fp32 first. The empty asm
// pins `f` in a VGPR, so the backend cannot fold the producing multiply or add into a
// v_fma_mix*_f16 (which rounds once, straight to f16: a double-rounding difference
// from the reference's fp32 op followed by the conversion).
__device__ __forceinline__ uint16_t f2h(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (half_t)f);
}
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

// Streaming 16-byte load that does not allocate in the caches (weights are read once per
// token; keeping them out of L2/MALL leaves room for activations and partials).
__device__ __forceinline__ u4_t load_stream16(const uint32_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p));
}

// Device-coherent (agent scope) accesses for data that work-groups of one launch hand to
// each other: relaxed atomics, which the compiler emits as sc1 loads and stores that are
// coherent across the XCDs' L2s without any cache writeback or invalidate.
template <typename T>
__device__ __forceinline__ void st_agent(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ld_agent(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Launch helper: returns the launch error as an int.
#define MI_LAUNCH_CHECK() return (int)hipGetLastError()

}  // namespace mi
