/* mi355x_decode.h - the C ABI of the MI355X-native decode-loop library
 * (libmi355x_decode.so, HIP for gfx950).
 *
 * Drop-in boundary for the reference engine's kernel entry points
 * (urakozz/intel-arc-inference-server, src/kernels/ *.cl launched by
 * src/runtime/capture.cc) and its decode loop (src/runtime/engine.h). Each entry
 * cites the reference interface it replaces. Conventions:
 *   - plain device pointers and sizes; the caller owns every buffer and the library
 *     allocates nothing inside a kernel entry (the reference's ownership rule,
 *     docs/04-architecture.md:308-317);
 *   - `stream` is a hipStream_t (NULL = the default stream); entries only enqueue;
 *   - every entry returns 0 on success, a positive hipError_t from the runtime, or a
 *     negative MI_ERR_* for a rejected argument; mi_last_error() describes the last
 *     failure on the calling thread (the reference throws l0::Error / fails `require`
 *     at capture, src/l0/error.h:10-30, src/runtime/capture.cc:144);
 *   - activations, KV values and scales are IEEE binary16 bit patterns (uint16_t);
 *     partial sums and logits are fp32;
 *   - split-K partials are [S][M][N] fp32 and consumers fold them in ascending s from
 *     0.f (src/kernels/gemv.cl:1-10, tests/kernels/gemm_sm_ref.h:106-136);
 *   - the control block is CTRL words of uint32 in device memory, laid out as the
 *     reference's runtime::Control prefix (src/runtime/control.h:13-24).
 */
#ifndef MI355X_DECODE_H
#define MI355X_DECODE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MI_OK = 0,
  MI_ERR_ARG = -1,   /* null / misaligned pointer or inconsistent argument */
  MI_ERR_SHAPE = -2, /* a shape the kernels do not support */
  MI_ERR_STATE = -3, /* call out of order (engine not built, ...) */
  MI_ERR_OOM = -4
};

/* Control block word indices (src/runtime/control.h:13-24: pos, n_active, cur_token[8],
 * out_token[8], debug_flag), plus the step counter this library keeps after them. */
enum {
  MI_CTRL_POS = 0,
  MI_CTRL_NACT = 1,
  MI_CTRL_CUR = 2,
  MI_CTRL_OUT = 10,
  MI_CTRL_DEBUG = 18,
  MI_CTRL_STEPS = 19,
  MI_CTRL_WORDS = 64
};

const char* mi_last_error(void);

/* ---- runtime plumbing (the role of src/l0/memory.h / cmdlist.h, for callers that do
 * not bring their own HIP runtime) ---- */
int mi_malloc(void** p, size_t bytes);
int mi_free(void* p);
int mi_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int mi_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream); /* synchronous */
int mi_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int mi_stream_sync(void* stream);
int mi_device_sync(void);
int mi_event_create(void** ev);
int mi_event_record(void* ev, void* stream);
int mi_event_elapsed_ms(void* start, void* stop, float* ms); /* waits for `stop` */
int mi_event_destroy(void* ev);

/* ---- synthetic data on the device (the reference's tests generate on the host,
 * tests/kernels/gemv_ref.h:23-29, common/int4.h:41-50) ---- */
int mi_fill_u32(uint32_t* p, size_t n, uint64_t seed, void* stream);
/* kind 0: uniform [a, b); kind 1: normal(mean a, std b) */
int mi_fill_f16(uint16_t* p, size_t n, uint64_t seed, int kind, float a, float b, void* stream);
int mi_fill_f32(float* p, size_t n, uint64_t seed, int kind, float a, float b, int round16,
                void* stream);
int mi_fill_i8(int8_t* p, size_t n, uint64_t seed, int lo, int hi, void* stream);

/* ---- int4 GPTQ g64 unpack: replaces common::Int4Gptq::at (src/common/int4.h:19-23) as
 * a device pass; out[k][n] = (q - 8) * scale, fp32, exact ---- */
int mi_int4_dequant(const uint32_t* qweight, const uint16_t* scales, float* out, uint32_t K,
                    uint32_t N, void* stream);

/* ---- W4A16 g64 linear: replaces `gemv` (src/kernels/gemv.cl:124-131, bound at
 * src/runtime/capture.cc:1045-1080) and, at M >= 2, `gemm_sm` (src/kernels/gemm_sm.cl:161-164).
 * qweight u32 [K/8][N] (layout 0), scales f16 [K/64][N], x f16 [M][K],
 * partials fp32 [S][M][N]. 1 <= M <= 16, 64 | K, 64 | N, S | K/64. ---- */
int mi_gemv_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x,
                  float* partials, uint32_t M, uint32_t K, uint32_t N, uint32_t S, void* stream);
/* The split-K width this library uses for a shape (the role of kQwen38Tuning,
 * src/model/model_desc.cc:32, and kSmallMTuning, src/kernels/kernels.h:140-170). */
uint32_t mi_gemv_pick_s(uint32_t K, uint32_t N);
/* out = sum_s partials[s] (ascending from 0.f), as fp16 and/or fp32 (the host fold of
 * tests/kernels/gemv_harness.h:59-120, on the device) */
int mi_fold_partials(const float* partials, uint16_t* out_f16, float* out_f32, uint32_t S,
                     uint32_t M, uint32_t N, void* stream);

/* ---- measurement: a plain streaming read of `bytes` (the probe_bw rate,
 * tools/probe/probe_bw) ---- */
int mi_stream_read(const void* p, size_t bytes, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif
