// ref_shim.cpp - TEST INFRASTRUCTURE. Exposes the reference engine's own scalar host
// twins, compiled from their sources where they lie under /root/reference (never copied),
// through a C ABI so tests can check this repository's oracle against them bit for bit.
// Built by oracle/build_oracle.py into oracle/_ref/libref.so; only tests load it.
//
// Included reference headers: src/common/{bf16,int4,repack,kv8}.h,
// tests/kernels/{gemv_ref,gemm_sm_ref,prep_ref,attn_ref,kv8_ref,moe_ref,pf_moe_ref}.h.
#include <cstdint>
#include <cstring>
#include <vector>

#include "common/bf16.h"
#include "common/int4.h"
#include "common/kv8.h"
#include "common/repack.h"
#include "kernels/attn_ref.h"
#include "kernels/gemm_sm_ref.h"
#include "kernels/kv8_ref.h"
#include "kernels/moe_ref.h"
#include "kernels/pf_moe_ref.h"
#include "kernels/prep_ref.h"
#include "loader/lm_head_int8.h"
#include "loader/rtn.h"

extern "C" {

uint16_t ref_f32_to_bf16(float f) { return common::f32_to_bf16(f); }
float ref_bf16_to_f32(uint16_t h) { return common::bf16_to_f32(h); }
float ref_f16_to_f32(uint16_t h) { return common::f16_to_f32(h); }
uint16_t ref_f32_to_f16(float f) { return common::f32_to_f16(f); }
uint16_t ref_kv8_f32_to_f16_rne(float f) { return common::kv8::f32_to_f16_rne(f); }

static common::Int4Gptq make_w(const uint32_t* qw, const uint16_t* sc, uint32_t K, uint32_t N) {
  common::Int4Gptq w;
  w.K = K;
  w.N = N;
  w.qweight.assign(qw, qw + size_t(K / 8) * N);
  w.scales.assign(sc, sc + size_t(K / 64) * N);
  return w;
}

void ref_int4_dequant(const uint32_t* qw, const uint16_t* sc, uint32_t K, uint32_t N, float* out) {
  const common::Int4Gptq w = make_w(qw, sc, K, N);
  for (uint32_t k = 0; k < K; ++k)
    for (uint32_t n = 0; n < N; ++n) out[size_t(k) * N + n] = w.at(k, n);
}
void ref_int4_random(uint32_t K, uint32_t N, uint32_t seed, uint32_t* qw, uint16_t* sc) {
  const common::Int4Gptq w = common::Int4Gptq::random(K, N, seed);
  std::memcpy(qw, w.qweight.data(), w.qweight.size() * 4);
  std::memcpy(sc, w.scales.data(), w.scales.size() * 2);
}
void ref_repack_layout1(const uint32_t* qw, const uint16_t* sc, uint32_t K, uint32_t N, uint32_t* out) {
  common::repack_int4_layout1(qw, sc, K, N, out);
}
void ref_interleave16_l0(const uint32_t* aq, const uint16_t* as, const uint32_t* bq, const uint16_t* bs,
                         uint32_t K, uint32_t Np, uint32_t* oq, uint16_t* os) {
  const common::Part a{aq, as, Np}, b{bq, bs, Np};
  common::repack_int4_layout0_cols(K, 2 * Np, common::cols_interleave16(a, b), oq, os);
}

static gemm_sm::WeightView view(uint32_t kind, const uint32_t* words, const uint16_t* scales,
                                uint32_t K, uint32_t N) {
  gemm_sm::WeightView v;
  v.K = K;
  v.N = N;
  v.kind = kind;
  v.words = words;
  v.scales = scales;
  return v;
}
void ref_twin_gemv(uint32_t kind, const uint32_t* words, const uint16_t* scales, uint32_t K, uint32_t N,
                   const float* xf, uint32_t M, uint32_t S, float* out) {
  const std::vector<float> x(xf, xf + size_t(M) * K);
  const std::vector<float> r = gemm_sm::twin_gemv(view(kind, words, scales, K, N), x, M, S);
  std::memcpy(out, r.data(), r.size() * 4);
}
void ref_gemv_ref(uint32_t kind, const uint32_t* words, const uint16_t* scales, uint32_t K, uint32_t N,
                  const float* xf, uint32_t M, double* out, double* bound) {
  const std::vector<float> x(xf, xf + size_t(M) * K);
  std::vector<double> o, b;
  gemm_sm::ref(view(kind, words, scales, K, N), x, M, o, b);
  std::memcpy(out, o.data(), o.size() * 8);
  std::memcpy(bound, b.data(), b.size() * 8);
}

void ref_res_norm(const float* partials, uint16_t* resid, const float* norm_w, uint16_t* x_out,
                  uint32_t M, uint32_t K, uint32_t S_PREV) {
  prep_ref::res_norm(partials, resid, norm_w, x_out, M, K, S_PREV);
}
void ref_res_fold(const float* partials, uint16_t* resid, float* sumsq, uint32_t M, uint32_t K,
                  uint32_t S_PREV, uint32_t G) {
  prep_ref::res_fold(partials, resid, sumsq, M, K, S_PREV, G);
}
void ref_norm_finish(const float* sumsq, const uint16_t* resid, const float* norm_w, uint16_t* x_out,
                     uint32_t M, uint32_t K, uint32_t G) {
  prep_ref::norm_finish(sumsq, resid, norm_w, x_out, M, K, G);
}
uint32_t ref_silu_s() { return prep_ref::kSiluS; }
void ref_silu_mul(const float* partials, uint16_t* x_out, uint32_t M, uint32_t N) {
  prep_ref::silu_mul(partials, x_out, M, N);
}

// attn_ref's fixed Qwen3.8 full-attention shapes: 24 q / 4 kv heads of 256, S = 2,
// q||gate interleaved, partial RoPE over 64 dims; KV [max_len][4][256] bf16.
void ref_attn_prep(uint32_t pos, uint32_t n_act, uint32_t M, const float* partials, const float* fa_small,
                   const float* rope, float* attn_q, float* attn_gate, uint16_t* kv_k, uint16_t* kv_v) {
  attn_ref::prep(pos, n_act, M, partials, fa_small, rope, attn_q, attn_gate, kv_k, kv_v);
}
void ref_attn_decode(uint32_t pos, uint32_t n_act, uint32_t M, uint32_t max_len, const float* attn_q,
                     const uint16_t* kv_k, const uint16_t* kv_v, float* attn_part) {
  attn_ref::decode(pos, n_act, M, max_len, attn_q, kv_k, kv_v, attn_part);
}
void ref_attn_reduce(uint32_t pos, uint32_t n_act, uint32_t M, uint32_t max_len, const float* attn_part,
                     const float* attn_gate, uint16_t* attn_out) {
  attn_ref::reduce(pos, n_act, M, max_len, attn_part, attn_gate, attn_out);
}

void ref_kv8_rotate(const float* x, float* out) { common::kv8::rotate(x, out); }
void ref_kv8_unrotate(const float* y, float* out) { common::kv8::unrotate(y, out); }
uint16_t ref_kv8_encode(const float* x, int8_t* q) { return common::kv8::encode(x, q); }
float ref_kv8_dequant(int8_t q, uint16_t s) { return common::kv8::dequant(q, s); }

// kv8_ref::prep (attn_prep_kv8's twin, 24/4 heads of 256, bf16): the int8 cache
// [max_len][4][256] with scales [max_len][4] copied out of its host Cache.
void ref_kv8_prep(uint32_t pos, uint32_t n_act, uint32_t M, const float* partials, const float* fa_small,
                  const float* rope, uint32_t max_len, float* attn_q, float* attn_gate, int8_t* k, int8_t* v,
                  uint16_t* ks, uint16_t* vs) {
  kv8_ref::Cache c(max_len);
  std::memcpy(c.k.data(), k, c.k.size());
  std::memcpy(c.v.data(), v, c.v.size());
  std::memcpy(c.ks.data(), ks, c.ks.size() * 2);
  std::memcpy(c.vs.data(), vs, c.vs.size() * 2);
  kv8_ref::prep(pos, n_act, M, partials, fa_small, rope, max_len, attn_q, nullptr, attn_gate, c);
  std::memcpy(k, c.k.data(), c.k.size());
  std::memcpy(v, c.v.data(), c.v.size());
  std::memcpy(ks, c.ks.data(), c.ks.size() * 2);
  std::memcpy(vs, c.vs.data(), c.vs.size() * 2);
}
// kv8_ref::attend: the fp64 reader of one (q head, query) over keys [0, n) of kv head j,
// un-rotated (o) and rotated (o_rot) outputs.
void ref_kv8_attend(const float* q_rot, uint32_t max_len, const int8_t* k, const int8_t* v, const uint16_t* ks,
                    const uint16_t* vs, uint32_t j, uint32_t n, double* o, double* o_rot) {
  kv8_ref::Cache c(max_len);
  std::memcpy(c.k.data(), k, c.k.size());
  std::memcpy(c.v.data(), v, c.v.size());
  std::memcpy(c.ks.data(), ks, c.ks.size() * 2);
  std::memcpy(c.vs.data(), vs, c.vs.size() * 2);
  kv8_ref::attend(q_rot, c, j, n, o, o_rot);
}

struct RefRoute {
  uint32_t ids[8];
  float w[8];
  float p[8];
  float p9;
  float sg;
};
void ref_moe_route(const float* logits, uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                   uint32_t router_n, RefRoute* out) {
  const moe_ref::Shape s{experts, top_k, hidden, inter, router_n};
  const moe_ref::Route r = moe_ref::route(logits, s);
  std::memcpy(out->ids, r.ids, sizeof r.ids);
  std::memcpy(out->w, r.w, sizeof r.w);
  std::memcpy(out->p, r.p, sizeof r.p);
  out->p9 = r.p9;
  out->sg = r.sg;
}
float ref_moe_split_dot(const uint32_t* tiles, uint32_t K, uint32_t n, const uint16_t* x, uint32_t ks) {
  return moe_ref::split_dot(tiles, K, n, x, ks);
}
uint16_t ref_moe_silu_up(float g, float u) { return moe_ref::silu_up(g, u); }
uint16_t ref_moe_combine(const float* down, const RefRoute* rr, uint32_t experts, uint32_t top_k,
                         uint16_t resid) {
  const moe_ref::Shape s{experts, top_k, 0, 0, 0};
  moe_ref::Route r;
  std::memcpy(r.ids, rr->ids, sizeof r.ids);
  std::memcpy(r.w, rr->w, sizeof r.w);
  std::memcpy(r.p, rr->p, sizeof r.p);
  r.p9 = rr->p9;
  r.sg = rr->sg;
  return moe_ref::combine(down, r, s, resid);
}
// The whole block (gate_up then down) over layout-1 expert blocks.
void ref_moe_block(const float* logits, uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                   uint32_t router_n, const uint16_t* x, const uint32_t* gu, const uint32_t* dn,
                   uint32_t up_ks, uint32_t dn_ks, uint16_t* resid_inout) {
  const moe_ref::Shape s{experts, top_k, hidden, inter, router_n};
  const moe_ref::Route r = moe_ref::route(logits, s);
  const std::vector<uint16_t> h = moe_ref::gate_up(r, x, gu, s, up_ks);
  const std::vector<uint16_t> out = moe_ref::down(r, h, dn, s, resid_inout, dn_ks);
  std::memcpy(resid_inout, out.data(), out.size() * 2);
}

// common/repack.h:118 (the bf16 tile layout gemv_bf16.cl reads; element type agnostic)
void ref_repack_bf16_tiled(const uint16_t* w_rowmajor, uint32_t K, uint32_t N, uint16_t* out) {
  common::repack_bf16_tiled(w_rowmajor, K, N, out);
}

// The chunk's MoE block by pf_moe_ref's own pieces (bf16): sort, dequant_block, gemm_rows,
// silu_row over every row of every live tile (grouped), the down outputs rounded, then
// combine_token per token and column.
void ref_pf_moe_block(const uint32_t* route, uint32_t C, const uint16_t* x, const uint32_t* gu, const uint32_t* dn,
                      uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter, uint16_t* resid_inout) {
  const moe_ref::Shape s{experts, top_k, hidden, inter, 0};
  const pf_moe_ref::Sorted st = pf_moe_ref::sort(route, C, s);
  std::vector<std::vector<uint16_t>> gw(experts + 1), dw(experts + 1);
  const uint32_t rows = st.rows_used();
  std::vector<uint16_t> y(size_t(rows) * hidden, 0);
  pf_moe_ref::grouped(st, 0, experts + 1, [&](uint32_t b, uint32_t r) {
    const uint32_t tok = st.row_tok[r];
    if (tok == pf_moe_ref::kNone) return;
    if (gw[b].empty()) {
      gw[b] = pf_moe_ref::dequant_block(gu + b * s.gate_up_words(), hidden, 2 * inter);
      dw[b] = pf_moe_ref::dequant_block(dn + b * s.down_words(), inter, hidden);
    }
    const std::vector<float> g = pf_moe_ref::gemm_rows(x + size_t(tok) * hidden, gw[b].data(), hidden, 2 * inter);
    const std::vector<uint16_t> h = pf_moe_ref::silu_row(g, inter);
    const std::vector<float> d = pf_moe_ref::gemm_rows(h.data(), dw[b].data(), inter, hidden);
    for (uint32_t n = 0; n < hidden; ++n) y[size_t(r) * hidden + n] = moe_ref::rne(d[n]);
  });
  for (uint32_t t = 0; t < C; ++t)
    for (uint32_t n = 0; n < hidden; ++n)
      resid_inout[size_t(t) * hidden + n] = pf_moe_ref::combine_token(st, route + size_t(t) * moe_ref::kWords, y.data(),
                                                                     hidden, s, t, n,
                                                                     resid_inout[size_t(t) * hidden + n]);
}

// The int8 lm_head's load-time quantisation (src/loader/lm_head_int8.cc, compiled with this
// shim): bf16 [N][K] rows into gemv_i8w's tiled layout and the fp32 row scales, one thread.
void ref_quantise_int8_tiled(const uint16_t* w, uint32_t K, uint32_t N, int8_t* q_tiled, float* scales) {
  loader::quantise_int8_tiled(w, K, N, q_tiled, scales, 1);
}
size_t ref_int8_tiled_index(uint32_t K, uint32_t k, uint32_t n) { return loader::int8_tiled_index(K, k, n); }

// src/loader/rtn.h: the round-to-nearest int4 g64 quantiser of a bf16 linear (header only)
void ref_rtn_int4_g64(const uint16_t* w, uint32_t K, uint32_t N, uint32_t* qweight, uint16_t* scales) {
  loader::rtn_int4_g64(w, K, N, qweight, scales);
}

}  // extern "C"
