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

/* The device status word's value after a fused launch's hand-off wait timed out
 * (mi_gemv_epilogue.status; the engine's control block word MI_CTRL_DEBUG). */
#define MI_STATUS_HANDOFF_TIMEOUT 0xDEAD0003u
/* The control block's MI_CTRL_DEBUG word after a step produced a logit that is not finite (an
 * activation left the fp16 range): the argmax kernels set it when the word was 0, and the
 * step's token is not to be used. */
#define MI_STATUS_NONFINITE 0xDEAD0004u

enum {
  MI_OK = 0,
  MI_ERR_ARG = -1,   /* null / misaligned pointer or inconsistent argument */
  MI_ERR_SHAPE = -2, /* a shape the kernels do not support */
  MI_ERR_STATE = -3, /* call out of order (engine not built, ...) */
  MI_ERR_OOM = -4
};

/* Control block word indices (src/runtime/control.h:13-24: pos, n_active, cur_token[8],
 * out_token[8], debug_flag), plus the step counter this library keeps after them; and the
 * many-row lists' id slots at the reference's offsets (control.h:35-42): a list of 9..16 rows
 * reads its ids at MI_CTRL_WIDE_CUR and writes its argmaxes at MI_CTRL_WIDE_OUT, a list of
 * 17..64 rows at MI_CTRL_DEEP_CUR / MI_CTRL_DEEP_OUT; lists of up to 8 rows at MI_CTRL_CUR /
 * MI_CTRL_OUT. Every list leaves its last row's argmax at MI_CTRL_CUR. */
enum {
  MI_CTRL_POS = 0,
  MI_CTRL_NACT = 1,
  MI_CTRL_CUR = 2,
  MI_CTRL_OUT = 10,
  MI_CTRL_DEBUG = 18,
  MI_CTRL_STEPS = 19,
  MI_CTRL_WIDE_CUR = 32,
  MI_CTRL_WIDE_OUT = 48,
  MI_CTRL_DEEP_CUR = 64,
  MI_CTRL_DEEP_OUT = 128,
  MI_CTRL_WORDS = 192
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
/* `tiles` int4 g64 layout-1 tiles of 136 u32 (common/repack.h:17-30): random nibble words and
 * fp16 scales uniform in [lo, hi) (synthetic expert weights) */
int mi_fill_layout1(uint32_t* p, size_t tiles, uint64_t seed, float lo, float hi, void* stream);
/* In place over n f16 values: mode 1 = to bf16 bits (round to nearest even, common/bf16.h:12-16);
 * mode 2 = to the f16 encoding of that bf16 value (the bf16 activation mode's storage of the
 * activations and the KV cache, mi_gemv_epilogue.act). */
int mi_f16_to_bf16(uint16_t* p, size_t n, uint32_t mode, void* stream);

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
/* The same linear with the step's next operation fused into one consumer work-group per
 * 64-column tile (the reference's consumers prep_res_fold + prep_norm_finish, prep_silu_mul
 * and the lm_head fold + argmax_stage1, src/kernels/prep.cl:288-384, argmax.cl:82).
 * Hand-off words: for a fused kind, partials[0 .. (S-1)*M*N) (S*M*N for QKV; and RESID's sumsq) must hold
 * the empty pattern of mi_gemv_handoff_init on entry; every launch leaves them so. Launches
 * that share hand-off words must not overlap. */
enum { MI_EPI_PARTIALS = 0, MI_EPI_RESID = 1, MI_EPI_SILU = 2, MI_EPI_LOGITS = 3, MI_EPI_F16OUT = 4,
       MI_EPI_QKV = 5 };
typedef struct mi_gemv_epilogue {
  uint32_t kind;
  /* RESID (N = hidden <= 16384): resid [M][N] += rne(sum_s partials) (rounded as
   * prep_res_fold); the 64-column tiles' sums of squares go through sumsq, hand-off words
   * [N/64][M][N/64]; then rstd [M] = 1/sqrt(sum_g sumsq_g / N + eps) and x_next [M][N] =
   * rne(resid * rstd * next_norm_w). */
  uint16_t* resid;
  float* sumsq;
  float* rstd;
  const float* next_norm_w;
  uint16_t* x_next;
  float eps;
  /* SILU (N = 2 * inter, interleave16 gate||up): h [M][N/2] = rne(rne(silu(g)) * u) */
  uint16_t* h;
  /* LOGITS: logits [M][N] fp32; argmax_part [M][N/64] of 8 bytes (value, index) for
   * mi_argmax_finish, indices >= vocab_used never win (NULL: no argmax part) */
  float* logits;
  void* argmax_part;
  uint32_t vocab_used;
  /* F16OUT: out16 [M][N] = rne_f16(sum_s partials), the fold of mi_fold_partials in the
   * GEMV launch (a plain linear with 16-bit output) */
  uint16_t* out16;
  /* QKV (N = shape->qkv_n, M <= 4, not gated, head_dim 128 or 256): mi_attn_prep on the
   * folded q||k||v row in the same launch - q/k RMSNorm, RoPE, q -> attn_q fp32
   * [M][q_heads][head_dim], K/V f16 at the cache row of position pos + m (the arguments of
   * mi_attn_prep, whose output this is bit for bit). Without `arrive` the launch takes S
   * slices plus one consumer work-group per head; partials[0 .. S*M*N) are its hand-off words. */
  uint32_t* ctrl;
  const struct mi_attn_shape* shape;
  const float* q_norm;
  const float* k_norm;
  const float* rope;
  float* attn_q;
  uint16_t* kv_k;
  uint16_t* kv_v;
  size_t row_stride, head_stride;
  const uint32_t* pages;
  uint32_t page;
  uint32_t kv_len;
  /* Every fused kind. A consumer's wait for a hand-off word is bounded: after poll_limit polls
   * of a word that stays empty (0 = the default, 2^21, about a second) it gives up, takes the
   * empty NaN as the value and sets *status = MI_STATUS_HANDOFF_TIMEOUT (status may be NULL).
   * The output of such a launch is not to be used, and the hand-off words may then hold
   * values published late: run mi_gemv_handoff_init on them before the next fused launch.
   * inject: fault injection for tests of that path, 0 in normal use; bit 0 = the producer
   * work-groups publish nothing, so every consumer's wait times out.
   * arrive: NULL, or a device array of uint32 arrival counts, zero before the first launch
   * (hipMemset, or mi_memcpy_h2d of zeros): one count per tile (QKV: per head) every 32
   * words (128 bytes), so 32 * N/64 words, which every launch leaves at zero; launches that
   * may run at the same time need separate arrays. With it the slice that completes a tile
   * (a head) is that tile's consumer, so no wait depends on the dispatch order (each
   * producer then waits for one atomic's round trip before it exits). Without it slice S-1
   * (QKV: one extra row of work-groups) is, and the waits complete because every XCD
   * dispatches its share of the grid in order and those consumers are the grid's last row.
   * RESID's consumers also need all N/64 of them resident at once, either way. */
  uint32_t* status;
  uint32_t poll_limit;
  uint32_t inject;
  uint32_t* arrive;
  /* The activation type (the reference's is bf16, common/bf16.h:8-43): 0 = f16 (every rounding
   * above is rne_f16 and resid is f16). 1 = bf16: every rounding point rounds to bf16 instead
   * (rne_bf16 where the reference has it); resid holds bf16 bits; x, x_next, h, out16 and the
   * QKV kind's K/V rows hold the f16 encoding of bf16 values (exact for magnitudes in
   * [2^-17, 65504]; a larger value is stored as inf, which the logits' finiteness check
   * reports). The linears read those activations as they are. */
  uint32_t act;
  /* The RMSNorm split across two launches (no reference counterpart: the reference forms the
   * norm in res_norm, capture.cc:997, a launch of its own): RESID with sums_out set writes
   * resid and the 64-column tiles' sums of squares, sums_out [M][N/64] (plain stores),
   * followed by M words set to 0xFFFFFFFF, and nothing else (sumsq, rstd, next_norm_w, x_next
   * unused); the launch that reads the norm then forms it: with in_sums set (the PARTIALS,
   * SILU or QKV kind; K a multiple of 256 up to 16384, at most 8 k-groups per slice) x is
   * that residual [M][K] and the input is rne(x * rstd * in_norm_w), rstd = 1/sqrt(sum_g
   * in_sums[m][g] / K + in_eps) with the sums added in ascending g from +0 - RESID's x_next
   * bit for bit. in_sums has the same layout: the M words after the sums hold 0xFFFFFFFF or
   * the rstd of these sums (the launch's work-groups share the rstd through them, so the
   * first ones form it and the later ones read it). */
  float* sums_out;
  const float* in_sums;
  const float* in_norm_w;
  float in_eps;
} mi_gemv_epilogue;
int mi_gemv_w4a16_ex(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x,
                     float* partials, uint32_t M, uint32_t K, uint32_t N, uint32_t S,
                     const mi_gemv_epilogue* epilogue, void* stream);
/* The split-K width this library uses for a shape (the role of kQwen38Tuning,
 * src/model/model_desc.cc:32, and kSmallMTuning, src/kernels/kernels.h:140-170). */
uint32_t mi_gemv_pick_s(uint32_t K, uint32_t N);
/* The split-K width for a launch with epilogue kind `epilogue` (MI_EPI_*); today the plain
 * choice for every kind (same role as above). */
uint32_t mi_gemv_pick_s_ex(uint32_t K, uint32_t N, uint32_t epilogue);
/* Writes the empty pattern into n hand-off words (a fused launch's partials, RESID's sumsq).
 * Needed once per buffer: every fused launch leaves its words empty again. */
int mi_gemv_handoff_init(float* words, size_t n, void* stream);
/* out = sum_s partials[s] (ascending from 0.f), as fp16 and/or fp32 (the host fold of
 * tests/kernels/gemv_harness.h:59-120, on the device) */
int mi_fold_partials(const float* partials, uint16_t* out_f16, float* out_f32, uint32_t S,
                     uint32_t M, uint32_t N, void* stream);


/* ---- the between-GEMV kernels (src/kernels/prep.cl). Residual stream and normed
 * activations are f16 [M][K]; norm weights fp32 [K] (the reference bakes fp32 weights,
 * src/loader/small_layout.h). ---- */
/* prep_res_fold (prep.cl:288): resid = rne(resid + rne(sum_s partials)) (S_PREV = 0: no
 * fold), sumsq[g][m] = the chunk's sum of squares, G chunks of ceil(K/G), 256-lane tree. */
int mi_res_fold(const float* partials, uint16_t* resid, float* sumsq, uint32_t M, uint32_t K,
                uint32_t S_PREV, uint32_t G, void* stream);
/* prep_norm_finish (prep.cl:350): x = rne(r * (1/sqrt(sum_g sumsq / K + eps)) * w) */
int mi_norm_finish(const float* sumsq, const uint16_t* resid, const float* norm_w, uint16_t* x_out,
                   uint32_t M, uint32_t K, uint32_t G, float eps, void* stream);
/* The int8 lm_head (spec 9: W8A16; src/loader/lm_head_int8.h, src/kernels/gemv_i8w.cl:55-58).
 * The weight is int8 in this library's matrix-core layout: element (k, n) of the [K][N] head at
 * byte mi_i8w_index(K, k, n) ([N/16][K/64][64 lanes][16 bytes]); scales fp32 [N], one per
 * output column. */
size_t mi_i8w_index(uint32_t K, uint32_t k, uint32_t n);
/* lm_head_int8.cc:22-37 on the host: each row n of w fp32 [N][K] (a 16-bit head widened)
 * quantised symmetrically, s = max|w| / 127 (fp32), q = rne(w / s) clamped to [-127, 127], a
 * zero row s = 0, q = 0; into q_tiled (K N bytes, the layout above) and scales[N]. K a
 * multiple of 64, N of 16. */
int mi_lm_head_int8_quantise(const float* w, uint32_t K, uint32_t N, int8_t* q_tiled, float* scales);
/* A head the reference quantised (loader::quantise_int8_tiled, lm_head_int8.cc) is in its own
 * layout, loader::int8_tiled_index (lm_head_int8.h:33: [N/16][K/16][16 k][16 n]). This copies
 * it, on the device, into mi_i8w_index's layout (q_tiled, K N bytes, a separate buffer); its
 * fp32 row scales are used as they are. K a multiple of 64, N of 16. */
int mi_i8w_from_ref_tiles(const int8_t* ref_tiled, uint32_t K, uint32_t N, int8_t* q_tiled, void* stream);
/* gemv_i8w: out fp32 [M][N] = (sum_k q[k][n] x[m][k]) * scales[n]; x f16 [M][K]; M <= 8, K a
 * multiple of 64, N of 64. */
int mi_gemv_i8w(const int8_t* w, const float* scales, const uint16_t* x, float* out, uint32_t M,
                uint32_t K, uint32_t N, void* stream);
/* mi_res_fold with prep.cl's ZERO_RESID (zero_resid = 1: resid = rne(sum_s partials), the
 * residual taken as zero - the MTP head's fc fold, capture.cc:1790) */
int mi_res_fold_ex(const float* partials, uint16_t* resid, float* sumsq, uint32_t M, uint32_t K,
                   uint32_t S_PREV, uint32_t G, uint32_t zero_resid, void* stream);
/* mi_norm_finish with prep.cl's X_STRIDE: row m of x at x_out + m * x_stride (the MTP head's
 * two pre-fc norms into the halves of one [M][2K] row, capture.cc:1784-1788) */
int mi_norm_finish_ex(const float* sumsq, const uint16_t* resid, const float* norm_w, uint16_t* x_out,
                      size_t x_stride, uint32_t M, uint32_t K, uint32_t G, float eps, void* stream);
/* prep_res_norm (tests/kernels/prep_ref.h:59-92): both halves in one launch per row */
int mi_res_norm(const float* partials, uint16_t* resid, const float* norm_w, uint16_t* x_out,
                uint32_t M, uint32_t K, uint32_t S_PREV, float eps, void* stream);
/* prep_silu_mul (prep.cl:384): gate||up partials [S][M][2N] interleaved in 16-column blocks
 * (src/common/repack.h:64-73) -> x = rne(rne(silu(rne(g))) * rne(u)), [M][N] */
int mi_silu_mul(const float* partials, uint16_t* x_out, uint32_t M, uint32_t N, uint32_t S,
                void* stream);

/* Attention shape. The fused qkv linear's columns: q heads (interleaved [q_h | gate_h]
 * per head when gated, src/kernels/attn.cl header) then k at k_off, v at v_off. */
typedef struct mi_attn_shape {
  uint32_t q_heads, kv_heads, head_dim, rot_dim;
  uint32_t gated;
  uint32_t qkv_n, k_off, v_off;
  float scale; /* score scale, fp32(1/sqrt(head_dim)) */
  float eps;   /* q/k RMSNorm epsilon */
  /* the activation type, as mi_gemv_epilogue.act: 1 = bf16 roundings in attn_prep (q/k before
   * and after the norm, the K/V rows as f16 encodings of bf16 values) and the reduce's output;
   * the f16 cache kernels only (mi_attn_prep, mi_attn_decode, mi_attn_reduce) */
  uint32_t act;
} mi_attn_shape;

/* attn_prep (attn.cl:361-372): fold the qkv partials [S][M][qkv_n], per-head q/k RMSNorm
 * (q_norm/k_norm fp32 [head_dim], NULL = none), RoPE (rope fp32 [max_len][2][rot_dim/2],
 * rotate_half pairs), q -> attn_q fp32 [M][q_heads][head_dim], gate -> attn_gate (gated
 * only), K/V f16 written at the row of position pos + m: element (row, head, d) at
 * row*row_stride + head*head_stride + d; row = pages[p/page]*page + p%page when pages.
 * kv_len (positions the cache holds, 0 = unchecked): a position >= kv_len writes nothing
 * and sets ctrl[MI_CTRL_DEBUG] = 0xDEAD0002. */
int mi_attn_prep(uint32_t* ctrl, const float* partials, uint32_t S, uint32_t M,
                 const mi_attn_shape* shape, const float* q_norm, const float* k_norm,
                 const float* rope, float* attn_q, float* attn_gate, uint16_t* kv_k,
                 uint16_t* kv_v, size_t row_stride, size_t head_stride, const uint32_t* pages,
                 uint32_t page, uint32_t kv_len, void* stream);
/* attn_prep_kv8 (kv8.cl:287-300, the int8 KV writer; scheme src/common/kv8.h:1-26): the
 * mi_attn_prep chain at head_dim 256, then q rotated (attn_q fp32, R = H_256 diag(s) / 16),
 * and the K row (f16 rounding of the roped k) and V row (f16 rounding of v) rotated and
 * quantised: int8 at row*row_stride + head*head_stride + d, the row's fp16 scale
 * f16(amax / 127) at row*sc_row_stride + head*sc_head_stride. */
int mi_attn_prep_kv8(uint32_t* ctrl, const float* partials, uint32_t S, uint32_t M,
                     const mi_attn_shape* shape, const float* q_norm, const float* k_norm,
                     const float* rope, float* attn_q, float* attn_gate, int8_t* kv_k,
                     int8_t* kv_v, uint16_t* k_scale, uint16_t* v_scale, size_t row_stride,
                     size_t head_stride, size_t sc_row_stride, size_t sc_head_stride,
                     const uint32_t* pages, uint32_t page, uint32_t kv_len, void* stream);
/* Positions per attention block for a row attending to `len` keys (attn_v2.cl:138-142). */
uint32_t mi_attn_ppw(uint32_t len, uint32_t tgt);
/* attn_decode_v2 (attn_v2.cl:172-188) / attn_decode_v2_kv8 (kv8.cl:535-548): grid
 * (kv_heads, tgt, M); kv_kind 0 = f16 KV, 1 = int8 KV with f16 scales at
 * row*sc_row_stride + head*sc_head_stride; attn_part fp32 [q_heads][tgt][M][head_dim+2];
 * keys at positions >= kv_len are never read (0 = unchecked). */
int mi_attn_decode(const uint32_t* ctrl, const float* attn_q, uint32_t kv_kind, const void* kv_k,
                   const void* kv_v, const uint16_t* k_scale, const uint16_t* v_scale,
                   size_t row_stride, size_t head_stride, size_t sc_row_stride,
                   size_t sc_head_stride, const uint32_t* pages, uint32_t page, uint32_t kv_len,
                   float* attn_part, uint32_t M, uint32_t tgt, const mi_attn_shape* shape,
                   void* stream);
/* The verify step's attention for many rows (attn_verify_dpas, attn_verify_dpas.cl:383; bound by
 * verify_attn.h:93-96's rule, mi_attn_verify_binds): M <= 64 rows of a model with 8 q heads per
 * kv head (16 / 2 at head_dim 256 in the reference), f16 cache. The same arguments, partials
 * and blocking as mi_attn_decode (reduce with mi_attn_reduce), each KV block read once for 8
 * rows. A row's partials depend only on its own key count, not on M or the other rows (the
 * reference's property R); they are not bitwise mi_attn_decode's (another accumulation order). */
int mi_attn_verify(const uint32_t* ctrl, const float* attn_q, const uint16_t* kv_k, const uint16_t* kv_v,
                   size_t row_stride, size_t head_stride, const uint32_t* pages, uint32_t page, uint32_t kv_len,
                   float* attn_part, uint32_t M, uint32_t tgt, const mi_attn_shape* shape, void* stream);
/* verify_attn.h:93-100 (verify_attn_wide_heads / verify_attn_kind at those heads): 1 when a verify
 * list of M rows binds mi_attn_verify (16 q / 2 kv heads, f16 cache (kv_kind 0), M = 16, 32 or
 * 64), 0 when it keeps mi_attn_decode. */
int mi_attn_verify_binds(uint32_t M, uint32_t kv_kind, uint32_t q_heads, uint32_t kv_heads);
/* attn_prep (attn.cl:361-372) and attn_decode_v2 (attn_v2.cl:172-188) in one launch, f16 cache
 * only: the decode's work-groups compute q of their heads and the new K/V rows of their block
 * from the qkv partials themselves (the same chain as mi_attn_prep, bitwise), write each new
 * K/V row once and the gate (gated shapes) once, and leave the same partials as
 * mi_attn_prep followed by mi_attn_decode. M <= 8. No q is written (attn_q is internal). */
int mi_attn_prep_decode(uint32_t* ctrl, const float* partials, uint32_t S, uint32_t M,
                        const mi_attn_shape* shape, const float* q_norm, const float* k_norm,
                        const float* rope, float* attn_gate, uint16_t* kv_k, uint16_t* kv_v,
                        size_t row_stride, size_t head_stride, const uint32_t* pages, uint32_t page,
                        uint32_t kv_len, float* attn_part, uint32_t tgt, void* stream);
/* attn_reduce_v2 (attn_v2.cl:383-386): ascending block merge -> attn_out f16
 * [M][q_heads*head_dim] (gated: rne(rne(o) * sigmoid(gate))) */
int mi_attn_reduce(const uint32_t* ctrl, const float* attn_part, const float* attn_gate,
                   uint16_t* attn_out, uint32_t M, uint32_t tgt, uint32_t kv_len,
                   const mi_attn_shape* shape, void* stream);

/* attn_reduce_v2_kv8 (kv8.cl:814-821): mi_attn_reduce's merge over partials of the rotated
 * int8 cache, the head's output un-rotated (FWHT(s * o) / 16) before the gate; head_dim 256. */
int mi_attn_reduce_kv8(const uint32_t* ctrl, const float* attn_part, const float* attn_gate,
                       uint16_t* attn_out, uint32_t M, uint32_t tgt, uint32_t kv_len,
                       const mi_attn_shape* shape, void* stream);

/* ---- the token boundary ---- */
/* embed_gather (embed_gather.cl:47-49): resid[m] = embed[cur_token[m]]; an id >= vocab
 * writes nothing and sets ctrl[MI_CTRL_DEBUG] = 0xDEAD0001 */
int mi_embed_gather(uint32_t* ctrl, const uint16_t* embed, uint16_t* resid, uint32_t M,
                    uint32_t hidden, uint32_t vocab, void* stream);
/* argmax_stage1/2 (argmax.cl:82-83, 133-134): per active row the arg-max of logits fp32
 * [M][vocab] (ties -> lower index; index >= vocab_used never wins) into out_token[m]; then
 * cur_token[0] = out_token[n-1], history[steps] = it (when history != NULL and
 * steps < history_len), steps += 1, pos += n_active. part: mi_argmax_groups(vocab) * M * 8
 * bytes of scratch. */
uint32_t mi_argmax_groups(uint32_t vocab);
/* argmax_stage2 alone (argmax.cl:133-172) over `groups` (value, index) winners per row, as
 * written by mi_gemv_w4a16_ex's LOGITS epilogue (groups = vocab / 64) or by stage 1. */
int mi_argmax_finish(uint32_t* ctrl, const void* part, uint32_t groups, uint32_t* history,
                     uint32_t history_len, void* stream);
/* embed_gather + the first RMSNorm in one launch per row: resid[m] = embed[cur_token[m]],
 * rstd[m] from 64-element chunk sums (prep_res_fold's tree at chunk 64, chunks ascending),
 * x = rne(resid * rstd * norm_w). Bad ids as embed_gather. hidden % 64 == 0. */
int mi_embed_norm(uint32_t* ctrl, const uint16_t* embed, uint16_t* resid, const float* norm_w,
                  uint16_t* x_out, float* rstd, uint32_t M, uint32_t hidden, uint32_t vocab,
                  float eps, void* stream);
/* mi_embed_norm with the activation type act (mi_gemv_epilogue.act): 1 = the embedding table
 * and resid hold bf16 bits, x the f16 encoding of the bf16-rounded norm (the reference's bf16
 * embed_gather + prep_norm_finish, prep.cl:350-353). */
int mi_embed_norm_act(uint32_t* ctrl, const uint16_t* embed, uint16_t* resid, const float* norm_w,
                      uint16_t* x_out, float* rstd, uint32_t M, uint32_t hidden, uint32_t vocab, float eps,
                      uint32_t act, void* stream);
/* The norm of the residual as it stands, rows [M][hidden]: the sum of squares in 64-element
 * chunks added in chunk order, rstd = 1/sqrt(sum / hidden + eps), x = rne(r * rstd * w)
 * (prep_res_fold with S_PREV 0 then prep_norm_finish, prep.cl:288/350) - the norm after a
 * block that folds its own output into the residual (moe_down, moe.cl:36-38). */
int mi_norm_rows(const uint16_t* resid, const float* norm_w, uint16_t* x_out, float* rstd,
                 uint32_t M, uint32_t hidden, float eps, void* stream);
int mi_argmax(uint32_t* ctrl, const float* logits, void* part, uint32_t* history,
              uint32_t history_len, uint32_t M, uint32_t vocab, uint32_t vocab_used, void* stream);
/* mi_argmax without the `part` argument, allocating nothing: the chunk winners go to a
 * file-scope device array of this library (8192 entries of 8 bytes, 64 KiB per GPU, held until
 * the process ends), so ceil(vocab / 1024) * M must be <= 8192 (MI_ERR_SHAPE otherwise). No
 * counterpart in the reference: for callers that cannot allocate device memory (code under
 * hipGraph capture, tight serving loops, harnesses that forbid hipMalloc). Every call on one
 * GPU shares that GPU's array: calls that overlap on one GPU (other streams, other threads)
 * race. The first call on a device looks the array's address up (hipGetSymbolAddress). */
int mi_argmax_static(uint32_t* ctrl, const float* logits, uint32_t* history, uint32_t history_len,
                     uint32_t M, uint32_t vocab, uint32_t vocab_used, void* stream);


/* ---- mixture of experts (src/kernels/moe.cl, src/kernels/gemv_bf16.cl) ----
 * A MoE block is four launches, as the reference's list (moe.cl:1-13): the router || shared
 * gate GEMV, routing, expert gate||up, expert down + combine + residual. Expert ids stay on
 * the device in a route row of MI_MOE_ROUTE_WORDS u32 per token (moe.cl:49-56): [0..7] ids,
 * [8..15] w_k and [16] the shared gate (fp32 bits of fp16 values), [17..24] p_k, [25] p of
 * rank top_k. The shared expert is weight block `experts` and slot top_k. */
#define MI_MOE_ROUTE_WORDS 32
/* gemv_bf16 (gemv_bf16.cl:103-200) with fp16 weights: out [M][N] fp32 = x [M][K] . w, w in
 * the tile layout [N/16][K/8][8][16] (common/repack.h:118); per column `ksplit` K slices
 * (power of two <= 16) each summed in ascending k, merged by the pairwise tree. M up to 65535
 * (one work-group per row and 16 columns). */
int mi_gemv_f16w(const uint16_t* w_tiled, const uint16_t* x, float* out, uint32_t M, uint32_t K,
                 uint32_t N, uint32_t ksplit, void* stream);
/* moe_route (moe.cl:192-262): logits [M][router_n] (experts router rows, then the shared
 * gate's row) -> route [M][MI_MOE_ROUTE_WORDS]. experts: power of two in [16, 256]; M up to
 * 65535 (rows are independent). */
int mi_moe_route(const float* logits, uint32_t* route, uint32_t M, uint32_t experts,
                 uint32_t top_k, uint32_t router_n, void* stream);
/* moe_gate_up (moe.cl:335-381): h [M][top_k + 1][inter] fp16 = rne(silu(g)) * u of each slot's
 * expert, gate||up in layout-1 int4 g64 blocks of (2 inter / 16) * (hidden / 64) * 136 u32
 * per expert (experts + 1 blocks); K split in 4 slices merged pairwise (kernels.h:591). */
int mi_moe_gate_up(const uint32_t* route, const uint16_t* x, const uint32_t* gu_blocks,
                   uint16_t* h, uint32_t M, uint32_t experts, uint32_t top_k, uint32_t hidden,
                   uint32_t inter, void* stream);
/* moe_route (moe.cl:192-262) and moe_gate_up (moe.cl:335-381) in one launch: every
 * work-group of a row forms the row's route from logits [M][router_n] (bitwise mi_moe_route's
 * row) before addressing its expert, and stores it to route [M][MI_MOE_ROUTE_WORDS] for
 * mi_moe_down; h as mi_moe_gate_up. The reference runs the two as separate kernels. */
int mi_moe_gate_up_routed(const float* logits, uint32_t router_n, uint32_t* route, const uint16_t* x,
                          const uint32_t* gu_blocks, uint16_t* h, uint32_t M, uint32_t experts,
                          uint32_t top_k, uint32_t hidden, uint32_t inter, void* stream);
/* moe_down (moe.cl:383-470): resid [M][hidden] += the slot-ordered combine of each slot's
 * down projection (layout-1 blocks of (hidden / 16) * (inter / 64) * 136 u32 per expert, K
 * split in 2 slices) weighted by w_k, plus the shared expert's times its gate. */
int mi_moe_down(const uint32_t* route, const uint16_t* h, const uint32_t* dn_blocks,
                uint16_t* resid, uint32_t M, uint32_t experts, uint32_t top_k, uint32_t hidden,
                uint32_t inter, void* stream);
/* mi_moe_down, then mi_norm_rows(resid, norm_w, x_out, rstd, M, hidden, eps) - the reference's
 * next res_norm (capture.cc:997) - in the same launch, bit for bit: one more row of
 * work-groups after the down grid takes each row's norm from the new residual values, which
 * the down work-groups also publish through `handoff` ([M][hidden/2] hand-off words that hold
 * the empty pattern between launches: mi_gemv_handoff_init once; every launch leaves them
 * empty). A wait that never completes gives up after poll_limit polls of a word (0 = 2^21,
 * about a second) and sets *status (may be NULL) to MI_STATUS_HANDOFF_TIMEOUT. inject: 0 in
 * normal use; bit 0 = the down work-groups publish nothing (tests of the timeout path). M <= 8. */
int mi_moe_down_norm(const uint32_t* route, const uint16_t* h, const uint32_t* dn_blocks,
                     uint16_t* resid, uint32_t M, uint32_t experts, uint32_t top_k, uint32_t hidden,
                     uint32_t inter, const float* norm_w, uint16_t* x_out, float* rstd, float eps,
                     uint32_t* handoff, uint32_t* status, uint32_t poll_limit, uint32_t inject, void* stream);

/* ---- the chunked prefill's kernels (src/kernels/prefill: pf_gemm_q4.cl, pf_flash_attn.cl,
 * pf_embed.cl) ---- */
/* out [T][N] fp32 = x [T][K] f16 . W (int4 GPTQ g64 layout 0) on the matrix cores, with
 * w = f16((q - 8) * scale) (the reference's prefill rounds the same product to bf16,
 * pf_dequant_slab.cl). 64 | K, 128 | N. */
int mi_gemm_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x, float* out,
                  uint32_t T, uint32_t K, uint32_t N, void* stream);
/* The same for the gate||up linear (N = 2 * inter, interleave16 columns) with prep_silu_mul
 * (prep.cl:384) in the epilogue: h [T][N/2] f16 = rne(rne(silu(rne(g))) * rne(u)), bitwise
 * mi_gemm_w4a16 followed by mi_silu_mul. */
int mi_gemm_w4a16_silu(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x, uint16_t* h,
                       uint32_t T, uint32_t K, uint32_t N, void* stream);
/* Causal attention of T rows at positions pos0 .. pos0 + T - 1 (q fp32 [T][q_heads][head_dim],
 * as mi_attn_prep writes it) over the fp16 cache rows [0, pos0 + t] (row layout and page table as
 * mi_attn_decode); attn_out [T][q_heads * head_dim] f16. head_dim 128 or 256. */
int mi_attn_prefill(const float* attn_q, const uint16_t* kv_k, const uint16_t* kv_v,
                    size_t row_stride, size_t head_stride, const uint32_t* pages, uint32_t page,
                    uint32_t T, uint32_t pos0, const mi_attn_shape* shape, uint16_t* attn_out,
                    void* stream);
/* mi_attn_prefill over the int8 rotated cache (attn_prep_kv8's rows and fp16 scales, the
 * reader of attn_decode_v2_kv8 + attn_reduce_v2_kv8, kv8.cl:535/814; head_dim 256): q as
 * mi_attn_prep_kv8 writes it (rotated), the output fp32 in the rotated basis into out_rot
 * [T][q_heads][256], then un-rotated into attn_out f16. */
int mi_attn_prefill_kv8(const float* attn_q, const int8_t* kv_k, const int8_t* kv_v,
                        const uint16_t* k_scale, const uint16_t* v_scale, size_t row_stride,
                        size_t head_stride, size_t sc_row_stride, size_t sc_head_stride,
                        const uint32_t* pages, uint32_t page, uint32_t T, uint32_t pos0,
                        const mi_attn_shape* shape, float* out_rot, uint16_t* attn_out, void* stream);
/* mi_attn_prep for a chunk's T rows (positions pos0 .. pos0 + T - 1) from a one-slice fold
 * qkv [T][qkv_n] fp32, one wave per (head, row): bitwise mi_attn_prep with S = 1 and n_act = T
 * (plain q||k||v, not gated, head_dim 128 or 256). The caller keeps pos0 + T within the cache. */
int mi_attn_prep_rows(const float* qkv, uint32_t T, uint32_t pos0, const mi_attn_shape* shape,
                      const float* q_norm, const float* k_norm, const float* rope, float* attn_q,
                      uint16_t* kv_k, uint16_t* kv_v, size_t row_stride, size_t head_stride,
                      const uint32_t* pages, uint32_t page, void* stream);
/* resid [T][hidden] = embed rows of ids [T] (pf_embed_gather); an id >= vocab leaves its row
 * and sets *flag = 0xDEAD0001 (flag may be NULL). */
int mi_embed_rows(const uint32_t* ids, const uint16_t* embed, uint16_t* resid, uint32_t T,
                  uint32_t hidden, uint32_t vocab, uint32_t* flag, void* stream);
/* The chunk's MoE expert FFN (the expert part of the reference's MoE block, moe.cl:1-13, for
 * T rows at once), grouped by expert: route [T][32] (mi_moe_route rows),
 * x [T][hidden] f16, the layer's layout-1 gate||up and down blocks (experts + 1 of each, the
 * shared expert last); resid [T][hidden] f16 += the slot-ordered combine (moe_ref.h:144-152).
 * Workspace: list [T (top_k + 1)] u32, tiles [(T (top_k + 1) + 63) / 64 + experts + 1] x 4 u32
 * (16-byte aligned), tiles_n [1], h [T (top_k + 1)][inter] f16, d [T (top_k + 1)][hidden] f16.
 * Each expert's pairs run through the int4 MFMA tile in 64-row tiles, so the per-pair values
 * round like mi_gemm_w4a16 (one f16 rounding per weight), not like the decode kernels. T <= 2048. */
int mi_moe_prefill(const uint32_t* route, const uint16_t* x, const uint32_t* gu_blocks,
                   const uint32_t* dn_blocks, uint16_t* resid, uint32_t T, uint32_t experts,
                   uint32_t top_k, uint32_t hidden, uint32_t inter, uint32_t* list, uint32_t* tiles,
                   uint32_t* tiles_n, uint16_t* h, uint16_t* d, void* stream);

/* ---- the decode loop (src/runtime/engine.h:52-331, capture.cc, control.h) ----
 * Model shape as data (model::ModelDesc, src/model/model_desc.h:67-229), restricted to the
 * GQA decoders this build runs: every layer is attention + a SwiGLU MLP (int4 g64 layout 0)
 * or a mixture-of-experts block (layout-1 experts); fp16 activations and KV. */
typedef struct mi_model_desc {
  uint32_t layers, hidden, q_heads, kv_heads, head_dim, rot_dim, inter, vocab, vocab_used;
  uint32_t max_len;  /* KV cache rows per layer (positions) */
  uint32_t qk_norm;  /* 1: per-head RMSNorm on q and k (attn.cl attn_prep) */
  uint32_t max_rows; /* largest verify step (rows) the engine captures, 1..64 (above 8: no
                      * MTP head; such lists run as row chunks of 8, see mi_engine_verify) */
  uint32_t attn_tgt; /* attention blocks per kv head (the v2 grid's TGT) */
  float rope_theta, rms_eps;
  /* experts > 0: every layer's MLP is a mixture-of-experts block (moe.cl) of `experts`
   * routed experts (power of two, 16..256), top_k of them per token plus one shared
   * expert, expert intermediate moe_inter; the router || shared gate is an fp16 linear of
   * roundup16(experts + 1) rows. `inter` is then unused. */
  uint32_t experts, top_k, moe_inter;
  /* 1: the int8 KV cache with the Hadamard rotation (kv8.cl under --kv-cache int8;
   * head_dim 256): int8 rows [layers][kv_heads][max_len][head_dim] and fp16 scales
   * [layers][kv_heads][max_len]; the step runs attn_prep_kv8 and the rotated reader pair. */
  uint32_t kv_int8;
  /* 1: the model's MTP head (loader::MtpHead; the draft lists of capture.cc:1772-1939): fc
   * [2 hidden] -> hidden behind the embedding's and the hidden's norms, one decoder layer
   * at the model's shapes (mtp_intermediate = inter; an MoE model's head: one MoE layer of the
   * model's shape, spec 15e) with its own one-layer f16 KV cache, the head's final norm, the
   * shared embedding and lm_head (the main cache f16 or int8).
   * Every step then also fills the head's K/V (capture.cc:362-370) and mi_engine_draft runs the
   * draft lists. */
  uint32_t mtp;
  /* 1: the int8 lm_head (spec 9, loader::LmHeadForm::Int8): int8 [vocab][hidden] in
   * mi_i8w_index's layout with one fp32 scale per row, read by mi_gemv_i8w, then both argmax
   * stages; a loaded checkpoint's 16-bit head is quantised at load (lm_head_int8.cc). 0: the
   * int4 g64 head. */
  uint32_t lm_head_int8;
  /* 1: bf16 activations, the reference's own type (common/bf16.h:8-43): every rounding point
   * of the step rounds to bf16, the embedding table and the residual stream hold bf16 bits, and
   * the normed activations, the attention output, SwiGLU's output and the KV cache hold the f16
   * encoding of bf16 values (mi_gemv_epilogue.act). The synthetic random-init 27B model's
   * residual leaves the f16 range on some inputs; bf16's range holds it. Dense models with the
   * f16-format cache, no MTP head; prefill refused (ingest). 0: f16 activations (BASELINE's). */
  uint32_t act_bf16;
  /* With a dense MTP head (mtp = 1, experts = 0): 1 keeps the head's five linears (fc, q||k||v,
   * o, gate||up, down) in 16 bits as the reference's loader does (loader.cc:586-597,
   * repack_bf16_tiled), run by the 16-bit GEMV (mi_gemv_f16w, gemv_bf16's order) with the
   * standalone fold, norm, SwiGLU and attn_prep kernels; a loaded checkpoint's bf16 head
   * weights are held as f16 (exact in f16's range; a weight outside it is refused). 0: the
   * head's linears quantised to int4 g64 at load (rtn.h's rule) and run as the layers'. */
  uint32_t mtp_w16;
} mi_model_desc;

typedef struct mi_engine mi_engine;

/* Weight and buffer kinds for mi_engine_tensor (per layer below MI_T_EMBED). */
enum {
  MI_T_QKV_Q = 0, MI_T_QKV_S, MI_T_O_Q, MI_T_O_S, MI_T_GU_Q, MI_T_GU_S, MI_T_DOWN_Q, MI_T_DOWN_S,
  MI_T_IN_NORM, MI_T_POST_NORM, MI_T_Q_NORM, MI_T_K_NORM,
  MI_T_ROUTER, MI_T_MOE_GU, MI_T_MOE_DN, /* MoE layers: router tiles, expert blocks */
  MI_T_EMBED = 32, MI_T_FINAL_NORM, MI_T_LM_Q, MI_T_LM_S, MI_T_ROPE, MI_T_KV_K, MI_T_KV_V,
  MI_T_LOGITS, MI_T_CTRL, MI_T_HISTORY,
  MI_T_KV_KS, MI_T_KV_VS, /* the int8 cache's fp16 row scales (kv_int8) */
  /* activations of the last step of the graph path (diagnostics): the residual [rows][hidden],
   * the normed input x, q fp32 [rows][q_heads][head_dim], the attention output, SwiGLU's output */
  MI_T_RESID, MI_T_X, MI_T_ATTN_Q, MI_T_ATTN_OUT, MI_T_HBUF,
  /* the MTP head (mtp): its layer's tensors are the per-layer kinds at layer = layers; these
   * are its fc, its three norms, its KV layer [kv_heads][max_len][head_dim] f16, the hidden rows
   * hh [max_rows + 1][hidden] (row 0: the post-final-norm hidden of position pos - 1), the
   * draft chain's hidden [hidden], its control block and the last draft's logits [vocab] */
  MI_T_MTP_FC_Q, MI_T_MTP_FC_S, MI_T_MTP_PRE_E, MI_T_MTP_PRE_H, MI_T_MTP_FINAL, MI_T_MTP_KV_K,
  MI_T_MTP_KV_V, MI_T_MTP_HH, MI_T_MTP_DH, MI_T_MTP_CTRL, MI_T_MTP_LOGITS,
  /* the int8 lm_head (lm_head_int8): its tiled int8 weight and fp32 row scales */
  MI_T_LM_I8, MI_T_LM_I8_S,
  /* MoE models: the hand-off words of mi_moe_down_norm [max_rows][hidden / 2] (0xFFFFFFFF
   * between launches; emptied again by the engine after a step whose wait timed out) */
  MI_T_MOE_HANDOFF,
  /* the 16-bit MTP head (mtp_w16): fc, q||k||v, o, gate||up (interleaved in 16-column blocks),
   * down, each f16 in mi_gemv_f16w's tile layout [N/16][K/8][8][16] */
  MI_T_MTP_W16_FC, MI_T_MTP_W16_QKV, MI_T_MTP_W16_O, MI_T_MTP_W16_GU, MI_T_MTP_W16_DN
};

/* Allocates weights (random-init on the device from `seed`, BASELINE config 2's
 * distributions: uniform nibbles, scales U(0.002, 0.02), gammas N(1, 0.02) in fp16, embed
 * and KV N(0, 1); an int8 cache holds uniform [-127, 127] with scales U(0.005, 0.05), config
 * 3's), the KV cache [layers][kv_heads][max_len][head_dim] (f16, or int8 + scales) and all
 * step buffers. stream NULL: the engine owns a stream. Returns NULL on failure (mi_last_error). */
mi_engine* mi_engine_create(const mi_model_desc* desc, uint64_t seed, void* stream);
void mi_engine_destroy(mi_engine* e);
void* mi_engine_stream(mi_engine* e);
/* Device pointer and size of a weight or buffer (for loading real weights or checks). */
int mi_engine_tensor(mi_engine* e, uint32_t kind, uint32_t layer, void** ptr, size_t* bytes);
/* Split-K width of linear `which` (0 qkv, 1 o, 2 gate||up, 3 down, 4 lm_head, 5 the MTP head's fc:
 * 0 without the head; the head's own layer takes the widths of 0..3). */
int mi_engine_linear_s(mi_engine* e, uint32_t which, uint32_t* S);
/* runtime::build / build_verify (capture.cc:2135-2144): record the M-row step as a graph. */
int mi_engine_capture(mi_engine* e, uint32_t M);
/* Engine::reset: control block cleared, pos and cur_token[0] set, n_active 1. */
int mi_engine_reset(mi_engine* e, uint32_t pos, uint32_t token);
/* Engine::replay (engine.cc:702-713): enqueue one captured M-row step (no sync). */
int mi_engine_replay(mi_engine* e, uint32_t M);
/* The same M-row step enqueued launch by launch, without the graph (no sync). */
int mi_engine_step_eager(mi_engine* e, uint32_t M);
/* Engine::generate (engine.cc:726-750): n greedy tokens; the ids land in `tokens`. */
int mi_engine_generate(mi_engine* e, uint32_t n, uint32_t* tokens);
/* Engine::ingest (engine.cc:715-724): one step per prompt id. */
int mi_engine_ingest(mi_engine* e, const uint32_t* ids, uint32_t n);
/* Engine::prefill (src/runtime/engine.h:97-115, the walk of src/runtime/prefill/step.h): the
 * ids in chunks of at most `chunk` positions (0: 2048, the cap) from the current position, on
 * the matrix cores (mi_gemm_w4a16, mi_attn_prefill). On return pos has advanced by n, the KV
 * cache holds those positions and cur_token is the argmax of the last position's logits, as
 * mi_engine_ingest of the same ids leaves them (up to the two paths' roundings). MoE layers run
 * their expert kernels over the chunk's rows in slices; the int8 cache takes attn_prep_kv8's
 * rows and mi_attn_prefill_kv8. Refused: no ids, chunk above the cap, an id outside the
 * vocabulary, past the cache. Allocates its scratch on the first call (and for a larger chunk). */
int mi_engine_prefill(mi_engine* e, const uint32_t* ids, uint32_t n, uint32_t chunk);
int mi_engine_read_ctrl(mi_engine* e, uint32_t* out /* MI_CTRL_WORDS */);
/* Measurement (no reference counterpart: the role of the reference's per-kernel timing in
 * tools/bench): `reps` rounds of one linear's step launch, exactly as the step issues it
 * (which bits 0-7 = 0 qkv with attn_prep, 1 o + residual + norm, 2 gate||up + silu*up,
 * 3 down + residual + norm: each layer's in turn; 4 the lm_head + argmax parts; bits 8-15 =
 * the rows M, 1..8, 0 meaning 1), back to back on the engine's stream; *ms_per_launch = the
 * HIP-event time per launch. The launches rewrite the step's state: reset the engine
 * (mi_engine_reset) before generating again. */
int mi_engine_bench_linear(mi_engine* e, uint32_t which, uint32_t reps, float* ms_per_launch);
/* Measurement (no reference counterpart: the role of the reference's verify-step timing,
 * docs/12-kernels.md:409-412): `reps` M-row verify steps at the current position with all M
 * rows live (ids: cur_token in each), M = bits 0-7 of rows_mode; each step = the rows' control
 * reset + the captured M-row graph (captured here if not yet; bit 8 set: the same step
 * enqueued kernel by kernel, for kernel tracers), back to back on the engine's stream;
 * *ms_per_step = the HIP-event time per step. pos and cur_token are left as they were
 * (n_active 1); the cache rows pos .. pos + M - 1 are overwritten. */
int mi_engine_bench_verify(mi_engine* e, uint32_t rows_mode, uint32_t reps, float* ms_per_step);
/* Engine::verify (engine.cc:868-926): one (k+1)-row step over [cur_token, drafts];
 * argmax_rows gets the k+1 row argmaxes; pos stays at the verify position. k + 1 <= max_rows;
 * a list of more than 8 rows (the reference's wide and deep lists, verify_attn.h:65-92) runs
 * every layer's linears, attn_prep and the head in row chunks of 8 and the attention over all
 * rows at once (mi_attn_verify where mi_attn_verify_binds, else the decode kernel per chunk):
 * each row's logits are those of the same row in a list of at most 8 rows. With the MTP head
 * the rows' post-final-norm hidden goes to hh rows 1..k+1 and the head's K/V are filled over
 * hh rows 0..k at positions pos - 1 .. pos + k - 1 (capture.cc:362-370); k > 0 needs pos >= 1. */
int mi_engine_verify(mi_engine* e, const uint32_t* drafts, uint32_t k, uint32_t* argmax_rows);
/* Engine::commit (engine.cc:927-960): pos = verify_pos + j + 1, cur_token[0] = next; with the
 * MTP head, hh row j + 1 (the accepted row's hidden) becomes row 0. */
int mi_engine_commit(mi_engine* e, uint32_t verify_pos, uint32_t j, uint32_t next);
/* Engine::draft (engine.h:259-290, capture.cc:1849-1939; mtp models): k (1..3) greedy drafts
 * from the MTP head at head positions pos - 1 .. pos + k - 2, the first from (hh row 0,
 * cur_token), each next one from the previous draft's id and the head's own output hidden.
 * drafts[i] = d_{i+1}; the main model's state is untouched (verify(k) with these ids next).
 * Needs pos >= 1 and pos + k + 1 <= max_len. */
int mi_engine_draft(mi_engine* e, uint32_t k, uint32_t* drafts);
/* ---- checkpoints (src/loader/loader.cc, quant.cc, repack.h, moe.cc; docs/13-loader.md) ----
 * A directory with config.json and *.safetensors of a GPTQ / AutoRound int4 g64 symmetric
 * checkpoint (quantization_config: bits 4, group_size 64, sym true, desc_act false or absent)
 * of a Qwen3-style GQA decoder, dense or MoE with one shared expert. */
/* The model description config.json gives (vocab padded to a multiple of 64, vocab_used the
 * real size; attn_tgt 64; qk_norm when the checkpoint has q_norm tensors). */
int mi_checkpoint_desc(const char* dir, uint32_t max_len, uint32_t max_rows, mi_model_desc* desc);
/* The quantisation checks alone (quant.cc assert_quant_invariants): the config's
 * quantization_config, then every int4 linear's shapes, qzeros, g_idx and scales; no GPU. */
int mi_checkpoint_check(const char* dir, char* report, size_t report_len);
/* Loads the checkpoint into an engine created from that description: q/k/v fused by columns,
 * gate/up interleaved in 16-column blocks, MoE experts as layout-1 tiles, the router and the
 * shared-expert gate as f16 tiles, norms fp32, embeddings f16; qzeros (all 0x77777777),
 * g_idx (the identity) and scales (finite) checked and the first two dropped; a 16-bit or
 * tied lm_head quantised to int4 g64 (GPTQ symmetric round-to-nearest). `report` (may be
 * NULL) receives a one-line summary. The KV cache and the control block are untouched. */
int mi_engine_load(mi_engine* e, const char* dir, char* report, size_t report_len);
/* server::accept_greedy (src/server/spec_accept.cc:81-85): the accepted draft count j;
 * *next = verify_argmax[j]. */
uint32_t mi_accept_greedy(const uint32_t* verify_argmax, const uint32_t* drafts, uint32_t k,
                          uint32_t* next);

/* ---- measurement: a plain streaming read of `bytes` (the probe_bw rate,
 * tools/probe/probe_bw) ---- */
int mi_stream_read(const void* p, size_t bytes, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif
