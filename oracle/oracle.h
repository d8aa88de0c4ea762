/* oracle.h - the CPU oracle's C interface.
 *
 * TEST INFRASTRUCTURE ONLY. This library is a scalar CPU restatement of the
 * reference engine's host twins (urakozz/intel-arc-inference-server,
 * tests/kernels/ *_ref.h and src/common/ *.h). Only tests/, the smoke check and
 * bench.py's CPU-baseline leg may load it, and only as the checker. The product
 * path (the HIP library) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates. Functions take an
 * activation type `act` (ORC_BF16 = 0, ORC_F16 = 1): the reference rounds its
 * activations to bf16; this build's workloads use fp16, with the same rounding
 * points (rne_bf16 -> rne_f16). Under ORC_BF16 the functions reproduce the
 * reference's own twins bit for bit (checked against oracle/_ref).
 */
#ifndef MI355X_ORACLE_H
#define MI355X_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_BF16 = 0, ORC_F16 = 1 };

/* threads the OpenMP-parallel functions use (the GEMV twins split columns; each column's
 * order is unchanged, so results do not depend on the thread count) */
int orc_threads(void);
void orc_set_threads(int n);

/* ---- scalar conversions (src/common/bf16.h:8-43, src/common/kv8.h:56-78) ---- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);          /* IEEE RNE, subnormals kept, overflow -> inf */
uint16_t orc_f32_to_f16_ftz(float f);      /* the reference's common::f32_to_f16 (flushes) */
uint16_t orc_f32_to_f16_sat(float f);      /* kv8::f32_to_f16_rne (saturates at 65504) */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_rne(int act, float f);
float orc_widen(int act, uint16_t h);

/* ---- int4 GPTQ g64 (src/common/int4.h:19-23, src/common/repack.h:17-125) ---- */
float orc_int4_at(const uint32_t* qweight, const uint16_t* scales, uint32_t K, uint32_t N,
                  uint32_t k, uint32_t n);
void orc_int4_dequant(const uint32_t* qweight, const uint16_t* scales, uint32_t K, uint32_t N,
                      float* out /* [K][N] */);
void orc_repack_layout1(const uint32_t* qweight, const uint16_t* scales, uint32_t K, uint32_t N,
                        uint32_t* out);
/* gate||up interleaved in 16-column blocks (repack.h:64-73), layout 0 */
void orc_interleave16_l0(const uint32_t* aq, const uint16_t* as, const uint32_t* bq,
                         const uint16_t* bs, uint32_t K, uint32_t Npart, uint32_t* oq,
                         uint16_t* os);

/* ---- GEMV (tests/kernels/gemm_sm_ref.h:83-136, gemv_ref.h:9-21) ----
 * layout: 0 = GPTQ [K/8][N] + scales [K/64][N]; 1 = 544-B tiles (scales unused) */
void orc_gemv_ref(uint32_t layout, const uint32_t* words, const uint16_t* scales, uint32_t K,
                  uint32_t N, const float* xf, uint32_t M, double* out, double* bound);
void orc_gemv_twin(uint32_t layout, const uint32_t* words, const uint16_t* scales, uint32_t K,
                   uint32_t N, const float* xf, uint32_t M, uint32_t S, float* out /* [M][N] */);
void orc_gemv_twin_partials(uint32_t layout, const uint32_t* words, const uint16_t* scales,
                            uint32_t K, uint32_t N, const float* xf, uint32_t M, uint32_t S,
                            float* partials /* [S][M][N] */);
/* spec-28 N2: count of outputs with |got-ref| > 2^-16 bound (NaN counts), max ratio */
size_t orc_n2_over(const float* got, const double* ref, const double* bound, size_t n,
                   double* max_ratio);

/* ---- prep (tests/kernels/prep_ref.h:59-198) ---- */
void orc_res_norm(int act, const float* partials, uint16_t* resid, const float* norm_w,
                  uint16_t* x_out, uint32_t M, uint32_t K, uint32_t S_PREV, float eps);
void orc_res_fold(int act, const float* partials, uint16_t* resid, float* sumsq, uint32_t M,
                  uint32_t K, uint32_t S_PREV, uint32_t G);
void orc_norm_finish(int act, const float* sumsq, const uint16_t* resid, const float* norm_w,
                     uint16_t* x_out, uint32_t M, uint32_t K, uint32_t G, float eps);
void orc_silu_mul(int act, const float* partials, uint16_t* x_out, uint32_t M, uint32_t N,
                  uint32_t S);

/* ---- attention (tests/kernels/attn_ref.h:84-336, src/kernels/attn_v2.cl:138-428) ---- */
typedef struct orc_attn_shape {
  uint32_t q_heads, kv_heads, head_dim, rot_dim;
  uint32_t gated;        /* 1: q columns interleave [q_h | gate_h] per head (Qwen3.8) */
  uint32_t qkv_n;        /* fused q(|gate)||k||v columns */
  uint32_t k_off, v_off; /* first column of k / v */
  float scale;           /* score scale, 1/sqrt(head_dim) rounded to fp32 */
  float eps;             /* q/k RMSNorm epsilon */
} orc_attn_shape;
/* KV element (row, kv head, d) lives at row*row_stride + h*head_stride + d. */
void orc_rope_table(double theta, uint32_t rot_dim, uint32_t max_len, float* table);
void orc_attn_prep(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act, uint32_t M,
                   const float* partials, uint32_t S, const float* q_norm, const float* k_norm,
                   const float* rope, float* attn_q, float* attn_gate, uint16_t* kv_k,
                   uint16_t* kv_v, size_t row_stride, size_t head_stride, const uint32_t* pages,
                   uint32_t page);
uint32_t orc_v2_ppw(uint32_t len, uint32_t tgt);
/* kv_kind: 0 = 16-bit act KV, 1 = int8 KV with fp16 scales [row*sc_row_stride + h*sc_head_stride] */
void orc_attn_decode_v2(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act,
                        uint32_t M, uint32_t tgt, const float* attn_q, uint32_t kv_kind,
                        const void* kv_k, const void* kv_v, const uint16_t* k_scale,
                        const uint16_t* v_scale, size_t row_stride, size_t head_stride,
                        size_t sc_row_stride, size_t sc_head_stride, const uint32_t* pages,
                        uint32_t page, float* attn_part);
void orc_attn_reduce_v2(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act,
                        uint32_t M, uint32_t tgt, const float* attn_part, const float* attn_gate,
                        uint16_t* attn_out);
/* fp64 softmax attention of one (q head, row) over keys [0, n) (kv8_ref.h:88-110 style) */
void orc_attend64(const orc_attn_shape* sh, const float* q, uint32_t kvh, uint32_t n,
                  uint32_t kv_kind, int act, const void* kv_k, const void* kv_v,
                  const uint16_t* k_scale, const uint16_t* v_scale, size_t row_stride,
                  size_t head_stride, size_t sc_row_stride, size_t sc_head_stride,
                  const uint32_t* pages, uint32_t page, double* out);

/* ---- int8 KV scheme (src/common/kv8.h:56-156), 256-point rotation ---- */
void orc_kv8_rotate256(const float* x, float* out);
void orc_kv8_unrotate256(const float* y, float* out);
uint16_t orc_kv8_quantise(const float* y, int8_t* q, uint32_t n);
uint16_t orc_kv8_encode256(const float* x, int8_t* q);
float orc_kv8_dequant(int8_t q, uint16_t s16);
/* attn_prep_kv8 (kv8.cl:287-408): orc_attn_prep's chain, q rotated (fp32), K = rne(roped k)
 * and V = rne(v) rotated and quantised: int8 at row*rs + h*hs, fp16 scale at row*srs + h*shs */
void orc_attn_prep_kv8(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act,
                       uint32_t M, const float* partials, uint32_t S, const float* q_norm,
                       const float* k_norm, const float* rope, float* attn_q, float* attn_gate,
                       int8_t* kv_k, int8_t* kv_v, uint16_t* k_scale, uint16_t* v_scale,
                       size_t rs, size_t hs, size_t srs, size_t shs, const uint32_t* pages,
                       uint32_t page);
/* attn_reduce_v2_kv8 (kv8.cl:814-860): the merge, un-rotation per head, then the gate */
void orc_attn_reduce_v2_kv8(int act, const orc_attn_shape* sh, uint32_t pos, uint32_t n_act,
                            uint32_t M, uint32_t tgt, const float* attn_part,
                            const float* attn_gate, uint16_t* attn_out);

/* ---- token boundary (src/kernels/embed_gather.cl:47-69, argmax.cl:63-172,
 *      src/server/spec_accept.cc:81-85) ---- */
int orc_embed_gather(const uint32_t* ids, uint32_t M, const uint16_t* embed, uint32_t vocab,
                     uint32_t hidden, uint16_t* resid);
uint32_t orc_argmax(const float* logits, uint32_t vocab, uint32_t vocab_used);
uint32_t orc_accept_greedy(const uint32_t* verify_argmax, const uint32_t* drafts, uint32_t k,
                           uint32_t* next);

/* ---- MoE (tests/kernels/moe_ref.h:62-177) ---- */
typedef struct orc_moe_route {
  uint32_t ids[8];
  float w[8];
  float p[8];
  float p9;
  float sg;
} orc_moe_route;
void orc_moe_route_fn(int act, const float* logits, uint32_t experts, uint32_t top_k,
                      orc_moe_route* r);
float orc_moe_split_dot(int act, uint32_t layout, const uint32_t* words, const uint16_t* scales,
                        uint32_t K, uint32_t N, uint32_t n, const uint16_t* x, uint32_t ks);
uint16_t orc_moe_silu_up(int act, float gate_sum, float up_sum);
uint16_t orc_moe_combine(int act, const float* down, const orc_moe_route* r, uint32_t top_k,
                         uint16_t resid);
/* Whole block for one token. Expert e's gate||up (interleave16, 2*inter columns, K = hidden)
 * and down (K = inter, N = hidden) live at gu_words + e*gu_stride_words (layout 0: qweight
 * then scales at gu_scales + e*gu_stride_scales). Expert `experts` is the shared one. */
void orc_moe_block(int act, uint32_t layout, uint32_t experts, uint32_t top_k, uint32_t hidden,
                   uint32_t inter, const orc_moe_route* r, const uint16_t* x,
                   const uint32_t* gu_words, const uint16_t* gu_scales, size_t gu_stride_words,
                   size_t gu_stride_scales, const uint32_t* dn_words, const uint16_t* dn_scales,
                   size_t dn_stride_words, size_t dn_stride_scales, uint32_t up_ks,
                   uint32_t dn_ks, uint16_t* h_out, uint16_t* resid);

/* ---- fp16-weight GEMV for the MoE router || shared gate (src/kernels/gemv_bf16.cl:103-200)
 * w: the canonical tile layout [N/16][K/8][8][16] (element k, n at
 * ((n/16)*(K/8) + k/8)*128 + (k%8)*16 + n%16), fp16 (the reference: bf16) weights;
 * x [M][K] activations (act). Per column, each of `ksplit` K slices sums w*x in ascending
 * k from 0.f (product and sum each rounded); the slices merge by the pairwise tree
 * stride = ksplit/2 .. 1, slice q < stride adding slice q + stride. out [M][N] fp32. */
void orc_gemv_f16w(int act, const uint16_t* w, const uint16_t* x, uint32_t M, uint32_t K,
                   uint32_t N, uint32_t ksplit, float* out);
/* row-major [N][K] fp16 -> the tile layout above */
void orc_f16w_tile(const uint16_t* w_rowmajor, uint32_t K, uint32_t N, uint16_t* w_tiled);

/* ---- the int8 lm_head (src/loader/lm_head_int8.cc:22-37, src/kernels/gemv_i8w.cl:55-106) ---- */
/* One row of K fp32 values: s = max|w| / 127 (fp32), q = rne(w / s) clamped to [-127, 127];
 * a zero row gives s = 0 and q = 0. Returns s. */
float orc_quantise_row_int8(const float* w, uint32_t K, int8_t* q);
/* Round-to-nearest int4 g64 of a bf16 row-major [N][K] linear into the GPTQ packing (qweight
 * [K/8][N], f16 scales [K/64][N], zero point 8): src/loader/rtn.h:35-60. */
void orc_rtn_int4_g64(const uint16_t* w_bf16, uint32_t K, uint32_t N, uint32_t* qweight, uint16_t* scales);
/* out[m][n] = (sum over k ascending of q[n][k] * x[m][k], fp32) * s[n]; q int8 [N][K]
 * row-major, x act [M][K] */
void orc_gemv_i8w(int act, const int8_t* q, const float* s, const uint16_t* x, uint32_t M, uint32_t K,
                  uint32_t N, float* out);

/* ---- a whole dense decode step (src/runtime/capture.cc:1247-1480 layer walk) ---- */
typedef struct orc_linear {
  const uint32_t* qweight; /* [K/8][N] */
  const uint16_t* scales;  /* [K/64][N] */
  uint32_t K, N, S;
} orc_linear;
typedef struct orc_layer {
  orc_linear qkv, o, gate_up, down; /* gate_up interleave16 */
  const float* in_norm;
  const float* post_norm;
  const float* q_norm; /* may be NULL (no q/k norm) */
  const float* k_norm;
  /* a mixture-of-experts layer (the model's experts > 0): router || shared gate fp16 in the
   * gemv_bf16 tile layout, experts + 1 layout-1 gate||up and down blocks */
  const uint16_t* router;
  const uint32_t* moe_gu;
  const uint32_t* moe_dn;
} orc_layer;
typedef struct orc_dense_model {
  uint32_t layers, hidden, inter, vocab, vocab_used, max_len;
  orc_attn_shape attn;
  float rms_eps;
  const orc_layer* layer;
  const uint16_t* embed; /* [vocab][hidden] act */
  const float* final_norm;
  orc_linear lm_head;
  const float* rope; /* [max_len][2][rot_dim/2] */
  uint32_t tgt;      /* attention blocks per kv head (the v2 grid) */
  uint32_t norm_g;   /* 0: single-launch res_norm tree; G > 0: res_fold over G chunks + norm_finish */
  /* experts > 0: every layer's MLP is the MoE block (moe.cl), router K split router_ksplit */
  uint32_t experts, top_k, moe_inter, router_n, router_ksplit;
  /* the int8 lm_head (spec 9): when lm_i8 is set the head is orc_gemv_i8w over lm_i8 int8
   * [vocab][hidden] row-major and lm_i8_scales fp32 [vocab], in place of lm_head */
  const int8_t* lm_i8;
  const float* lm_i8_scales;
} orc_dense_model;
/* One step for token `tok` at position pos. kv_k/kv_v: [layers][kv_heads][max_len][hd] act
 * (this build's layout), updated in place. Writes logits fp32 [vocab] and returns argmax. */
uint32_t orc_dense_step(int act, const orc_dense_model* m, uint32_t tok, uint32_t pos,
                        uint16_t* kv_k, uint16_t* kv_v, float* logits, uint32_t n_layers_run);
/* The same step over the int8 rotated cache (head_dim 256): kv_k/kv_v int8
 * [layers][kv_heads][max_len][hd], k_scale/v_scale fp16 [layers][kv_heads][max_len]. */
uint32_t orc_dense_step_kv8(int act, const orc_dense_model* m, uint32_t tok, uint32_t pos,
                            int8_t* kv_k, int8_t* kv_v, uint16_t* k_scale, uint16_t* v_scale,
                            float* logits, uint32_t n_layers_run);

/* The MTP head (the model's next-token predictor, src/runtime/capture.cc:1772-1939): a dense
 * decoder layer behind a projection of [enorm(embed(tok)) | hnorm(h)]. fc: [2 hidden] -> hidden;
 * layer: its q||k||v, o, gate||up, down and norms (in_norm the head's input norm, post_norm its
 * post-attention norm); final_norm the head's own output norm (mtp.norm). */
typedef struct orc_mtp_head {
  orc_linear fc;
  orc_layer layer;
  const float* pre_e; /* the embedding's norm */
  const float* pre_h; /* the hidden's norm */
  const float* final_norm;
  /* the 16-bit head (loader.cc:586-597 keeps a dense head's linears in bf16): when set, fc,
   * q||k||v, o, gate||up and down are these [N][K] 16-bit matrices in orc_f16w_tile's layout,
   * each run by orc_gemv_f16w (gemv_bf16's order; ksplit the largest power of two <= 16
   * dividing K/8) as one slice, and the orc_linear fields above are unused */
  const uint16_t* w16_fc;
  const uint16_t* w16_qkv;
  const uint16_t* w16_o;
  const uint16_t* w16_gu;
  const uint16_t* w16_dn;
} orc_mtp_head;
/* One head row at head position p for token `tok` and hidden h (act [hidden]: the main model's
 * post-final-norm hidden of position p, or the head's own output of the previous draft):
 * head_front (capture.cc:1772-1826: both pre-fc norms into one [2 hidden] row, fc, its output
 * as the residual (prep.cl ZERO_RESID), the input norm, q||k||v, attn_prep into the head's
 * one KV layer kv_k / kv_v [kv_heads][max_len][hd] at p). full = 0 stops there (the KV fill,
 * head_kv_fill :1840) and returns 0. full = 1 runs draft() (:1849-1939): attention over keys
 * 0..p, o, the post-attention norm, the MLP, the head's final norm into h_out (act [hidden]),
 * the shared lm_head into logits fp32 [vocab], and returns their argmax. The model's norm_g
 * sets the norms' order as for orc_dense_step (the head's pre-fc and input norms always take
 * prep_res_fold + prep_norm_finish over hidden / 64 chunks). */
uint32_t orc_mtp_head_step(int act, const orc_dense_model* m, const orc_mtp_head* head, uint32_t tok,
                           const uint16_t* h, uint32_t p, uint16_t* kv_k, uint16_t* kv_v, int full,
                           uint16_t* h_out, float* logits);

/* The chunk's MoE block for T rows (tests/kernels/pf_moe_ref.h's values: expert weights rounded
 * once to act, fp32 sums, the down outputs rounded, combine_token's slot-ordered combine with
 * the residual): route [T][32] (the route rows), x [T][hidden] act, experts + 1 layout-1 gate||up
 * and down blocks (the shared expert last); resid [T][hidden] act updated in place. */
void orc_moe_prefill(int act, uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                     const uint32_t* route, const uint16_t* x, const uint32_t* gu_blocks, const uint32_t* dn_blocks,
                     uint16_t* resid, uint32_t T);
/* The chunked prefill of T ids at positions pos .. pos + T - 1 (f16 cache; the walk of
 * src/runtime/prefill/step.h with the prefill's roundings: weights rounded once to act, fp32
 * sums, causal attention in fp64 rounded once; an MoE layer's experts as orc_moe_prefill). Writes the chunk's K/V rows, the logits of
 * the last row (the decode head) and returns their argmax (0xFFFFFFFF: unsupported). */
uint32_t orc_prefill_chunk(int act, const orc_dense_model* m, const uint32_t* ids, uint32_t T, uint32_t pos,
                           uint16_t* kv_k, uint16_t* kv_v, float* logits);

#ifdef __cplusplus
}
#endif
#endif
