// engine.cpp - the decode loop: weights, buffers, one captured step replayed per token.
//
// Mirrors the reference runtime (src/runtime/engine.h:52, engine.cc:702-960, capture.cc):
//   * the model is shape-as-data (mi_model_desc ~ model::ModelDesc, model_desc.h:67-229);
//   * one step is recorded once into a hipGraph (the L0 regular command list of
//     runtime::build, capture.cc:2135-2142) and replayed per token (Engine::replay,
//     engine.cc:702-713);
//   * everything that changes per token lives in the device control block (Control,
//     control.h:13-44): embed_gather reads cur_token, argmax writes out_token /
//     cur_token / the token history and advances pos - so `generate(n)` is n graph
//     launches and one synchronisation, with no host work between tokens;
//   * verify(k drafts) replays an (k+1)-row graph, accept_greedy picks the accepted
//     prefix on the host, commit() moves pos and cur_token (engine.cc:868-960,
//     spec_accept.cc:81-85).
// The layer walk is capture.cc's dense-attention layer (fa_layer :1370 + mlp :1247, or
// moe_block :1295 for a mixture-of-experts model):
//   res_fold + norm_finish, qkv GEMV, attn_prep, attn_decode, attn_reduce, o GEMV,
//   res_fold + norm_finish, gate||up GEMV, silu_mul, down GEMV; then head() (:1461):
//   res_fold + norm_finish, lm_head GEMV, fold to logits, argmax.
// Weights are synthetic (random-init on the device) - the loader is outside this build -
// and every weight tensor is reachable through mi_engine_tensor for checks or loading.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "mi_capi_internal.h"

namespace {

#define MI_TRY(expr)              \
  do {                            \
    const int _e = (expr);        \
    if (_e != 0) return _e;       \
  } while (0)

struct Linear {
  uint32_t* q = nullptr;  // [K/8][N]
  uint16_t* s = nullptr;  // [K/64][N]
  uint32_t K = 0, N = 0, S = 1;
};

struct Layer {
  Linear qkv, o, gate_up, down;  // gate_up / down unused in a MoE layer
  uint16_t* router = nullptr;    // MoE: fp16 [router_n][hidden] in the gemv_bf16 tile layout
  uint32_t* moe_gu = nullptr;    // MoE: experts + 1 layout-1 gate||up blocks
  uint32_t* moe_dn = nullptr;    // MoE: experts + 1 layout-1 down blocks
  float* in_norm = nullptr;
  float* post_norm = nullptr;
  float* q_norm = nullptr;
  float* k_norm = nullptr;
};

__global__ void ctrl_set_kernel(uint32_t* ctrl, uint32_t word, uint32_t value) {
  if (threadIdx.x == 0) ctrl[word] = value;
}
// A list's id and argmax slots (control.h:35-42): up to 8 rows at cur_token / out_token, 9..16
// at wide_cur / wide_out, 17..64 at deep_cur / deep_out.
__host__ __device__ inline uint32_t ctrl_cur_at(uint32_t M) {
  return M <= 8 ? MI_CTRL_CUR : M <= 16 ? MI_CTRL_WIDE_CUR : MI_CTRL_DEEP_CUR;
}
__host__ __device__ inline uint32_t ctrl_out_at(uint32_t M) {
  return M <= 8 ? MI_CTRL_OUT : M <= 16 ? MI_CTRL_WIDE_OUT : MI_CTRL_DEEP_OUT;
}
constexpr uint32_t kRowChunk = 8;  // rows per launch in a list of more than 8 rows

__global__ void ctrl_set_rows_kernel(uint32_t* ctrl, uint32_t pos, uint32_t n_act, const uint32_t* ids,
                                     uint32_t n_ids) {
  const uint32_t t = threadIdx.x;
  if (t == 0) {
    ctrl[MI_CTRL_POS] = pos;
    ctrl[MI_CTRL_NACT] = n_act;
  }
  if (t < n_ids) ctrl[ctrl_cur_at(n_ids) + t] = ids[t];
}


// A many-row list's row chunks: chunk c's control block (cctl + c MI_CTRL_WORDS) holds the
// position pos + 8 c, its active rows and its ids, so every launch of the chunk reads its rows
// as an up-to-8-row list does. One thread per chunk.
__global__ void chunk_ctrl_kernel(const uint32_t* ctrl, uint32_t* cctl, uint32_t M) {
  const uint32_t c = threadIdx.x, nc = (M + kRowChunk - 1) / kRowChunk;
  if (c >= nc) return;
  uint32_t* cc = cctl + c * MI_CTRL_WORDS;
  const uint32_t pos = ctrl[MI_CTRL_POS], n = ctrl[MI_CTRL_NACT], r0 = c * kRowChunk;
  cc[MI_CTRL_POS] = pos + r0;
  cc[MI_CTRL_NACT] = n > r0 ? min(n - r0, kRowChunk) : 0u;
  cc[MI_CTRL_DEBUG] = 0u;
  cc[MI_CTRL_STEPS] = 0u;
  for (uint32_t i = 0; i < kRowChunk; ++i)
    cc[MI_CTRL_CUR + i] = r0 + i < M ? ctrl[ctrl_cur_at(M) + r0 + i] : 0u;
}
// After the chunks' heads: their argmaxes into the list's out slots, then what argmax_stage2
// does for a list (the last row's argmax as cur_token, the history entry, the step count, pos
// advanced by the active rows), and the first flag a chunk raised.
__global__ void chunk_gather_kernel(uint32_t* ctrl, const uint32_t* cctl, uint32_t M, uint32_t* history,
                                    uint32_t history_len) {
  const uint32_t t = threadIdx.x, n = ctrl[MI_CTRL_NACT], oo = ctrl_out_at(M);
  if (t < M) ctrl[oo + t] = cctl[(t / kRowChunk) * MI_CTRL_WORDS + MI_CTRL_OUT + t % kRowChunk];
  __syncthreads();
  if (t == 0) {
    for (uint32_t c = 0; c * kRowChunk < M; ++c) {
      const uint32_t f = cctl[c * MI_CTRL_WORDS + MI_CTRL_DEBUG];
      if (f && ctrl[MI_CTRL_DEBUG] == 0u) ctrl[MI_CTRL_DEBUG] = f;
    }
    if (n != 0u) {
      const uint32_t tok = ctrl[oo + min(n, M) - 1u];
      ctrl[MI_CTRL_CUR] = tok;
      const uint32_t step = ctrl[MI_CTRL_STEPS];
      if (history && step < history_len) history[step] = tok;
      ctrl[MI_CTRL_STEPS] = step + 1u;
      ctrl[MI_CTRL_POS] += n;
    }
  }
}

// The MTP head's control block for the K/V fill over a step's M rows (capture.cc:362-370):
// row r pairs hh row r (the hidden of position pos - 1 + r) with the row's id at head position
// pos - 1 + r. At pos 0 there is no h_{-1}: no row is filled (n_active 0).
__global__ void mtp_fill_ctrl_kernel(const uint32_t* ctrl, uint32_t* hctl, uint32_t M) {
  const uint32_t t = threadIdx.x, pos = ctrl[MI_CTRL_POS];
  if (t == 0) {
    hctl[MI_CTRL_POS] = pos ? pos - 1u : 0u;
    hctl[MI_CTRL_NACT] = pos ? ctrl[MI_CTRL_NACT] : 0u;
  }
  if (t < M) hctl[MI_CTRL_CUR + t] = ctrl[MI_CTRL_CUR + t];
}
// Engine::draft's start: head position pos - 1, the pending id, the chain's hidden = hh row 0.
__global__ void mtp_draft_begin_kernel(const uint32_t* ctrl, uint32_t* hctl, const uint16_t* hh0, uint16_t* dh,
                                       uint32_t H) {
  const uint32_t t = threadIdx.x;
  if (t == 0) {
    hctl[MI_CTRL_POS] = ctrl[MI_CTRL_POS] - 1u;
    hctl[MI_CTRL_NACT] = 1u;
    hctl[MI_CTRL_CUR] = ctrl[MI_CTRL_CUR];
    hctl[MI_CTRL_STEPS] = 0u;
  }
  for (uint32_t i = t; i < H; i += blockDim.x) dh[i] = hh0[i];
}

}  // namespace

constexpr uint32_t kPrefillCap = 2048;  // positions per prefill chunk at most (the reference's default cap)
constexpr uint32_t kMaxDraft = 3;       // draft lists per iteration (MtpBuffers::kMaxK, engine.h:280)

// The MTP head's weights (loader::MtpHead): fc behind the two pre-fc norms, one dense decoder
// layer, the head's final norm.
struct MtpHead {
  Linear fc;
  Layer L;
  // the 16-bit head (mtp_w16): f16 in gemv_f16w's tiles; the int4 linears above stay empty
  uint16_t *fc16 = nullptr, *qkv16 = nullptr, *o16 = nullptr, *gu16 = nullptr, *dn16 = nullptr;
  float* pre_e = nullptr;
  float* pre_h = nullptr;
  float* final_n = nullptr;
};

struct mi_engine {
  mi_model_desc d{};
  hipStream_t stream = nullptr;
  bool own_stream = false;
  std::vector<void*> allocs;
  std::vector<Layer> layer;
  uint16_t* embed = nullptr;
  float* final_norm = nullptr;
  Linear lm_head;           // the int4 head (lm_head_int8 = 0)
  int8_t* lm_i8 = nullptr;  // the int8 head (lm_head_int8): [vocab][hidden] in mi_i8w_index's layout
  float* lm_i8s = nullptr;  // its fp32 row scales [vocab]
  float* rope = nullptr;
  void* kv_k = nullptr;  // [layers][kv_heads][max_len][head_dim] f16, or int8 (kv_int8)
  void* kv_v = nullptr;
  uint16_t* kv_ks = nullptr;  // kv_int8: fp16 row scales [layers][kv_heads][max_len]
  uint16_t* kv_vs = nullptr;
  // activations / scratch
  uint32_t* ctrl = nullptr;
  uint32_t* history = nullptr;
  uint32_t* ids_dev = nullptr;
  uint16_t* resid = nullptr;
  uint16_t* x = nullptr;
  uint16_t* hbuf = nullptr;
  uint16_t* attn_out = nullptr;
  float* part = nullptr;     // the plain launches' split-K partials (qkv)
  float* part_ex = nullptr;  // the fused launches' hand-off words (empty between launches)
  float* sumsq = nullptr;    // RESID's hand-off words for the tiles' sums of squares
  size_t part_ex_n = 0, sumsq_n = 0;
  uint32_t* arrive = nullptr;  // the fused launches' arrival counts (zero between launches)
  size_t arrive_n = 0;
  // last-arriver consumers (mi_gemv_epilogue.arrive): measured slower on MI355X than the
  // fixed last-row consumers (27B step 4.79 vs 4.34 ms: every producer then waits for an
  // atomic's round trip before it exits), so the engine keeps the fixed ones
  bool use_arrive = false;
  float* attn_q = nullptr;
  float* attn_part = nullptr;
  float* logits = nullptr;
  void* argmax_part = nullptr;
  float* rstd = nullptr;
  float* nsum = nullptr;  // a residual's tile sums of squares [M][hidden / 64] and M rstd words, for the next launch's norm
  float* moe_logits = nullptr;   // [max_rows][router_n]
  uint32_t* moe_route = nullptr; // [max_rows][MI_MOE_ROUTE_WORDS]
  uint16_t* moe_h = nullptr;     // [max_rows][top_k + 1][moe_inter]
  uint32_t* dn_words = nullptr;  // [max_rows][hidden / 2] moe_down_norm's hand-off words
  uint32_t router_n = 0;
  size_t gu_block = 0, dn_block = 0;  // u32 per expert block
  mi_attn_shape ash{};
  hipGraphExec_t graphs[65] = {};
  uint32_t* cctl = nullptr;  // a many-row list's row chunks' control blocks [8][MI_CTRL_WORDS]
  // the MTP head (d.mtp): weights, its one-layer KV cache, the hidden rows, the draft chain
  MtpHead mh;
  uint16_t* hkv_k = nullptr;  // [kv_heads][max_len][head_dim] f16
  uint16_t* hkv_v = nullptr;
  uint16_t* hh = nullptr;     // [max_rows + 1][hidden]: row 0 = h_{pos-1}, rows 1.. the step's rows
  uint16_t* dh = nullptr;     // [hidden] the draft chain's hidden
  uint16_t* hx2 = nullptr;    // [max_rows][2 hidden] fc's input
  float* hsumsq = nullptr;    // [hidden / 64][max_rows] the head's norm chunk sums
  uint32_t* hctl = nullptr;   // the head's control block
  uint32_t* hhist = nullptr;  // [max_len] the drafted ids (the head's argmax history)
  float* hlogits = nullptr;   // [vocab] the last draft's logits
  hipGraphExec_t draft_graph = nullptr;

  ~mi_engine() {
    for (auto& g : graphs)
      if (g) (void)hipGraphExecDestroy(g);
    if (draft_graph) (void)hipGraphExecDestroy(draft_graph);
    for (void* p : allocs) (void)hipFree(p);
    if (own_stream && stream) (void)hipStreamDestroy(stream);
  }

  template <typename T>
  int alloc(T** p, size_t count) {
    void* v = nullptr;
    const int e = static_cast<int>(hipMalloc(&v, count * sizeof(T) + 256));
    if (e != 0) return mi_hip(e, "engine hipMalloc");
    allocs.push_back(v);
    *p = static_cast<T*>(v);
    return 0;
  }

  // frees one allocation of alloc() (the stream must have drained) and clears the pointer
  void release(void** p) {
    if (!*p) return;
    for (auto it = allocs.begin(); it != allocs.end(); ++it)
      if (*it == *p) {
        (void)hipFree(*it);
        allocs.erase(it);
        break;
      }
    *p = nullptr;
  }

  // epi: the epilogue the step runs this linear with (its split-K width depends on it)
  int alloc_linear(Linear& l, uint32_t K, uint32_t N, uint32_t epi) {
    l.K = K;
    l.N = N;
    l.S = mi_gemv_pick_s_ex(K, N, epi);
    MI_TRY(alloc(&l.q, size_t(K / 8) * N));
    MI_TRY(alloc(&l.s, size_t(K / 64) * N));
    return 0;
  }

  int init_linear(Linear& l, uint64_t& seed) {
    MI_TRY(mi_fill_u32(l.q, size_t(l.K / 8) * l.N, seed++, stream));
    MI_TRY(mi_fill_f16(l.s, size_t(l.K / 64) * l.N, seed++, 0, 0.002f, 0.02f, stream));
    return 0;
  }

  int build(uint64_t seed) {
    const mi_model_desc& m = d;
    const uint32_t H = m.hidden, HD = m.head_dim, QH = m.q_heads, KVH = m.kv_heads;
    const uint32_t R = m.max_rows;
    // rows per launch: a list of more than 8 rows runs its launches in row chunks of 8, so the
    // per-launch scratch (split-K partials, hand-off words, argmax parts) holds RL rows
    const uint32_t RL = std::min(R, kRowChunk);
    const uint32_t qkv_n = (QH + 2 * KVH) * HD;
    ash = mi_attn_shape{QH, KVH, HD, m.rot_dim, 0u, qkv_n, QH * HD, (QH + KVH) * HD,
                        1.0f / std::sqrt(float(HD)), m.rms_eps, m.act_bf16};
    ash.scale = float(1.0 / std::sqrt(double(HD)));
    layer.resize(m.layers);
    size_t part_max = 0, part_ex_max = 1;
    const bool moe = m.experts > 0;
    if (moe) {
      router_n = (m.experts + 1 + 15) / 16 * 16;
      gu_block = size_t(2 * m.moe_inter / 16) * (H / 64) * 136;
      dn_block = size_t(H / 16) * (m.moe_inter / 64) * 136;
    }
    for (Layer& L : layer) {
      MI_TRY(alloc_linear(L.qkv, H, qkv_n, MI_EPI_QKV));  // the S of the fused launch, at every M
      MI_TRY(alloc_linear(L.o, QH * HD, H, MI_EPI_RESID));
      if (moe) {
        MI_TRY(alloc(&L.router, size_t(router_n) * H));
        MI_TRY(alloc(&L.moe_gu, (m.experts + 1) * gu_block));
        MI_TRY(alloc(&L.moe_dn, (m.experts + 1) * dn_block));
      } else {
        MI_TRY(alloc_linear(L.gate_up, H, 2 * m.inter, MI_EPI_SILU));
        MI_TRY(alloc_linear(L.down, m.inter, H, MI_EPI_RESID));
      }
      MI_TRY(alloc(&L.in_norm, H));
      MI_TRY(alloc(&L.post_norm, H));
      if (m.qk_norm) {
        MI_TRY(alloc(&L.q_norm, HD));
        MI_TRY(alloc(&L.k_norm, HD));
      }
      if (L.qkv.q) part_max = std::max(part_max, size_t(L.qkv.S) * RL * L.qkv.N);
      for (const Linear* l : {&L.o, &L.gate_up, &L.down})
        if (l->q) part_ex_max = std::max(part_ex_max, size_t(l->S) * RL * l->N);
      part_ex_max = std::max(part_ex_max, size_t(L.qkv.S) * std::min(RL, 4u) * L.qkv.N);  // QKV: all S slices
    }
    if (m.mtp) {  // the head: fc (plain partials) and a dense layer at the model's shapes
      Layer& L = mh.L;
      if (m.mtp_w16) {  // the 16-bit head: its GEMVs write [rows][N] fp32 into `part`
        MI_TRY(alloc(&mh.fc16, size_t(2 * H) * H));
        MI_TRY(alloc(&mh.qkv16, size_t(H) * qkv_n));
        MI_TRY(alloc(&mh.o16, size_t(QH * HD) * H));
        MI_TRY(alloc(&mh.gu16, size_t(H) * 2 * m.inter));
        MI_TRY(alloc(&mh.dn16, size_t(m.inter) * H));
        part_max = std::max({part_max, size_t(R) * H, size_t(R) * qkv_n, size_t(R) * 2 * m.inter});
      } else {
        MI_TRY(alloc_linear(mh.fc, 2 * H, H, 0));
        MI_TRY(alloc_linear(L.qkv, H, qkv_n, MI_EPI_QKV));
        MI_TRY(alloc_linear(L.o, QH * HD, H, MI_EPI_RESID));
      }
      if (moe) {  // an MoE model's head (spec 15e): one MoE layer of the model's shape
        MI_TRY(alloc(&L.router, size_t(router_n) * H));
        MI_TRY(alloc(&L.moe_gu, (m.experts + 1) * gu_block));
        MI_TRY(alloc(&L.moe_dn, (m.experts + 1) * dn_block));
      } else if (!m.mtp_w16) {
        MI_TRY(alloc_linear(L.gate_up, H, 2 * m.inter, MI_EPI_SILU));
        MI_TRY(alloc_linear(L.down, m.inter, H, MI_EPI_RESID));
      }
      for (float** nw : {&L.in_norm, &L.post_norm, &mh.pre_e, &mh.pre_h, &mh.final_n}) MI_TRY(alloc(nw, H));
      if (m.qk_norm) {
        MI_TRY(alloc(&L.q_norm, HD));
        MI_TRY(alloc(&L.k_norm, HD));
      }
      if (!m.mtp_w16) part_max = std::max({part_max, size_t(mh.fc.S) * R * H, size_t(L.qkv.S) * R * L.qkv.N});
      MI_TRY(alloc(&hkv_k, size_t(KVH) * m.max_len * HD));
      MI_TRY(alloc(&hkv_v, size_t(KVH) * m.max_len * HD));
      MI_TRY(alloc(&hh, size_t(R + 1) * H));
      MI_TRY(alloc(&dh, H));
      MI_TRY(alloc(&hx2, size_t(R) * 2 * H));
      MI_TRY(alloc(&hsumsq, size_t(H / 64) * R));
      MI_TRY(alloc(&hctl, MI_CTRL_WORDS));
      MI_TRY(alloc(&hhist, m.max_len));
      MI_TRY(alloc(&hlogits, m.vocab));
      MI_TRY(mi_hip(static_cast<int>(hipMemsetAsync(hctl, 0, MI_CTRL_WORDS * 4, stream)), "hctl clear"));
      MI_TRY(mi_hip(static_cast<int>(hipMemsetAsync(hh, 0, size_t(R + 1) * H * 2, stream)), "hh clear"));
    }
    if (m.lm_head_int8) {
      MI_TRY(alloc(&lm_i8, size_t(m.vocab) * H));
      MI_TRY(alloc(&lm_i8s, m.vocab));
    } else {
      MI_TRY(alloc_linear(lm_head, H, m.vocab, MI_EPI_LOGITS));
      part_ex_max = std::max(part_ex_max, size_t(lm_head.S) * RL * m.vocab);
    }
    MI_TRY(alloc(&embed, size_t(m.vocab) * H));
    MI_TRY(alloc(&final_norm, H));
    MI_TRY(alloc(&rope, size_t(m.max_len) * m.rot_dim));
    const size_t kv_elems = size_t(m.layers) * KVH * m.max_len * HD;
    const size_t kv_rows = size_t(m.layers) * KVH * m.max_len;
    if (m.kv_int8) {
      MI_TRY(alloc(reinterpret_cast<int8_t**>(&kv_k), kv_elems));
      MI_TRY(alloc(reinterpret_cast<int8_t**>(&kv_v), kv_elems));
      MI_TRY(alloc(&kv_ks, kv_rows));
      MI_TRY(alloc(&kv_vs, kv_rows));
    } else {
      MI_TRY(alloc(reinterpret_cast<uint16_t**>(&kv_k), kv_elems));
      MI_TRY(alloc(reinterpret_cast<uint16_t**>(&kv_v), kv_elems));
    }
    MI_TRY(alloc(&ctrl, MI_CTRL_WORDS));
    MI_TRY(alloc(&history, m.max_len));
    MI_TRY(alloc(&ids_dev, 64));
    if (R > kRowChunk) MI_TRY(alloc(&cctl, size_t(kRowChunk) * MI_CTRL_WORDS));
    MI_TRY(alloc(&resid, size_t(R) * H));
    MI_TRY(alloc(&x, size_t(R) * std::max(H, QH * HD)));
    MI_TRY(alloc(&hbuf, size_t(R) * m.inter));
    MI_TRY(alloc(&attn_out, size_t(R) * QH * HD));
    MI_TRY(alloc(&part, part_max));
    MI_TRY(alloc(&part_ex, part_ex_max));
    part_ex_n = part_ex_max;
    MI_TRY(mi_gemv_handoff_init(part_ex, part_ex_max, stream));
    sumsq_n = size_t(H / 64) * RL * (H / 64);
    MI_TRY(alloc(&sumsq, sumsq_n));
    MI_TRY(mi_gemv_handoff_init(sumsq, sumsq_n, stream));
    arrive_n = 32 * std::max<size_t>({m.vocab / 64, 2 * m.inter / 64, qkv_n / 64, H / 64});
    MI_TRY(alloc(&arrive, arrive_n));
    MI_TRY(mi_hip(static_cast<int>(hipMemsetAsync(arrive, 0, arrive_n * 4, stream)), "arrive clear"));
    MI_TRY(alloc(&attn_q, size_t(R) * QH * HD));
    MI_TRY(alloc(&attn_part, size_t(QH) * m.attn_tgt * R * (HD + 2)));
    MI_TRY(alloc(&logits, size_t(R) * m.vocab));
    MI_TRY(alloc(reinterpret_cast<uint64_t**>(&argmax_part), size_t(RL) * (m.vocab / 64 + mi_argmax_groups(m.vocab))));
    MI_TRY(alloc(&rstd, R));
    MI_TRY(alloc(&nsum, size_t(R) * (m.hidden / 64 + 1)));
    if (moe) {
      MI_TRY(alloc(&moe_logits, size_t(R) * router_n));
      MI_TRY(alloc(&moe_route, size_t(R) * MI_MOE_ROUTE_WORDS));
      MI_TRY(alloc(&moe_h, size_t(R) * (m.top_k + 1) * m.moe_inter));
      MI_TRY(alloc(&dn_words, size_t(RL) * (H / 2)));
      MI_TRY(mi_gemv_handoff_init(reinterpret_cast<float*>(dn_words), size_t(RL) * (H / 2), stream));
    }

    // synthetic weights (BASELINE config 2's distributions)
    for (Layer& L : layer) {
      for (Linear* l : {&L.qkv, &L.o, &L.gate_up, &L.down})
        if (l->q) MI_TRY(init_linear(*l, seed));
      if (moe) {  // router N(0, 0.02), int4 g64 experts
        MI_TRY(mi_fill_f16(L.router, size_t(router_n) * H, seed++, 1, 0.0f, 0.02f, stream));
        MI_TRY(mi_fill_layout1(L.moe_gu, (m.experts + 1) * gu_block / 136, seed++, 0.002f, 0.02f, stream));
        MI_TRY(mi_fill_layout1(L.moe_dn, (m.experts + 1) * dn_block / 136, seed++, 0.002f, 0.02f, stream));
      }
      MI_TRY(mi_fill_f32(L.in_norm, H, seed++, 1, 1.0f, 0.02f, 1, stream));
      MI_TRY(mi_fill_f32(L.post_norm, H, seed++, 1, 1.0f, 0.02f, 1, stream));
      if (m.qk_norm) {
        MI_TRY(mi_fill_f32(L.q_norm, HD, seed++, 1, 1.0f, 0.02f, 1, stream));
        MI_TRY(mi_fill_f32(L.k_norm, HD, seed++, 1, 1.0f, 0.02f, 1, stream));
      }
    }
    if (m.lm_head_int8) {  // uniform int8 with row scales U(2e-4, 1.2e-3): the int4 head's spread
      MI_TRY(mi_fill_i8(lm_i8, size_t(m.vocab) * H, seed++, -127, 127, stream));
      MI_TRY(mi_fill_f32(lm_i8s, m.vocab, seed++, 0, 2e-4f, 1.2e-3f, 0, stream));
    } else {
      MI_TRY(init_linear(lm_head, seed));
    }
    MI_TRY(mi_fill_f16(embed, size_t(m.vocab) * H, seed++, 1, 0.0f, 1.0f, stream));
    if (m.act_bf16) MI_TRY(mi_f16_to_bf16(embed, size_t(m.vocab) * H, 1, stream));  // the table in bf16
    MI_TRY(mi_fill_f32(final_norm, H, seed++, 1, 1.0f, 0.02f, 1, stream));
    if (m.kv_int8) {  // BASELINE config 3's int8 cache: uniform [-127, 127], scales U(0.005, 0.05)
      MI_TRY(mi_fill_i8(static_cast<int8_t*>(kv_k), kv_elems, seed++, -127, 127, stream));
      MI_TRY(mi_fill_i8(static_cast<int8_t*>(kv_v), kv_elems, seed++, -127, 127, stream));
      MI_TRY(mi_fill_f16(kv_ks, kv_rows, seed++, 0, 0.005f, 0.05f, stream));
      MI_TRY(mi_fill_f16(kv_vs, kv_rows, seed++, 0, 0.005f, 0.05f, stream));
    } else {
      MI_TRY(mi_fill_f16(static_cast<uint16_t*>(kv_k), kv_elems, seed++, 1, 0.0f, 1.0f, stream));
      MI_TRY(mi_fill_f16(static_cast<uint16_t*>(kv_v), kv_elems, seed++, 1, 0.0f, 1.0f, stream));
      if (m.act_bf16) {  // bf16 values, in the cache's f16 encoding
        MI_TRY(mi_f16_to_bf16(static_cast<uint16_t*>(kv_k), kv_elems, 2, stream));
        MI_TRY(mi_f16_to_bf16(static_cast<uint16_t*>(kv_v), kv_elems, 2, stream));
      }
    }
    // the head last, so a model's own weights are the same with and without it
    if (m.mtp) {
      // the head's linears at a quarter of the layers' scales, U(0.0005, 0.005): its residual
      // stream starts at fc's output (K = 2 hidden over inputs with a common mode), and at the
      // layers' scales the random head's MLP output overflows fp16 at the 27B shape
      for (Linear* l : {&mh.fc, &mh.L.qkv, &mh.L.o, &mh.L.gate_up, &mh.L.down}) {
        if (!l->q) continue;  // an MoE head has no dense gate||up / down
        MI_TRY(mi_fill_u32(l->q, size_t(l->K / 8) * l->N, seed++, stream));
        MI_TRY(mi_fill_f16(l->s, size_t(l->K / 64) * l->N, seed++, 0, 0.0005f, 0.005f, stream));
      }
      // the 16-bit head: N(0, 0.01), about the int4 head's weights' spread at its scales
      for (uint16_t* w : {mh.fc16, mh.qkv16, mh.o16, mh.gu16, mh.dn16}) {
        if (!w) continue;
        const size_t n = w == mh.fc16 ? size_t(2 * H) * H : w == mh.qkv16 ? size_t(H) * qkv_n
                       : w == mh.o16 ? size_t(QH * HD) * H : w == mh.gu16 ? size_t(H) * 2 * m.inter
                                                                          : size_t(m.inter) * H;
        MI_TRY(mi_fill_f16(w, n, seed++, 1, 0.0f, 0.01f, stream));
      }
      if (m.experts) {  // the MoE head's router as the layers', its experts at the head's scales
        MI_TRY(mi_fill_f16(mh.L.router, size_t(router_n) * H, seed++, 1, 0.0f, 0.02f, stream));
        MI_TRY(mi_fill_layout1(mh.L.moe_gu, (m.experts + 1) * gu_block / 136, seed++, 0.0005f, 0.005f, stream));
        MI_TRY(mi_fill_layout1(mh.L.moe_dn, (m.experts + 1) * dn_block / 136, seed++, 0.0005f, 0.005f, stream));
      }
      for (float* nw : {mh.L.in_norm, mh.L.post_norm, mh.pre_e, mh.pre_h, mh.final_n})
        MI_TRY(mi_fill_f32(nw, H, seed++, 1, 1.0f, 0.02f, 1, stream));
      if (m.qk_norm) {
        MI_TRY(mi_fill_f32(mh.L.q_norm, HD, seed++, 1, 1.0f, 0.02f, 1, stream));
        MI_TRY(mi_fill_f32(mh.L.k_norm, HD, seed++, 1, 1.0f, 0.02f, 1, stream));
      }
      MI_TRY(mi_fill_f16(hkv_k, size_t(KVH) * m.max_len * HD, seed++, 1, 0.0f, 1.0f, stream));
      MI_TRY(mi_fill_f16(hkv_v, size_t(KVH) * m.max_len * HD, seed++, 1, 0.0f, 1.0f, stream));
    }
    // RoPE table in double, stored fp32 (src/loader/loader.cc:702-716)
    {
      const uint32_t half = m.rot_dim / 2;
      std::vector<float> t(size_t(m.max_len) * 2 * half);
      for (uint32_t p = 0; p < m.max_len; ++p)
        for (uint32_t i = 0; i < half; ++i) {
          const double a = double(p) * std::pow(double(m.rope_theta), -2.0 * double(i) / double(m.rot_dim));
          t[(size_t(p) * 2 + 0) * half + i] = float(std::cos(a));
          t[(size_t(p) * 2 + 1) * half + i] = float(std::sin(a));
        }
      MI_TRY(mi_hip(static_cast<int>(hipMemcpy(rope, t.data(), t.size() * 4, hipMemcpyHostToDevice)),
                    "rope upload"));
    }
    MI_TRY(mi_hip(static_cast<int>(hipMemsetAsync(ctrl, 0, MI_CTRL_WORDS * 4, stream)), "ctrl clear"));
    MI_TRY(mi_hip(static_cast<int>(hipStreamSynchronize(stream)), "engine init"));
    return 0;
  }

  // the router GEMV's K split: gemv_bf16's {16, 16} tiling (kernels.h gemv_bf16_tiling)
  static uint32_t router_ksplit_of(uint32_t hidden) {
    uint32_t k = 16;
    while (k > 1 && (hidden / 8) % k) k /= 2;
    return k;
  }
  uint32_t router_ksplit() const { return router_ksplit_of(d.hidden); }

  // The dense layers split each RMSNorm between two launches: o's and down's consumers write
  // the residual and its tile sums (nsum) only, and gate||up (the next qkv) forms the norm
  // itself for its slice, bitwise the x the consumers would have written; that spares the
  // consumers' all-to-all exchange of tile sums. The last layer's down (the head's input, which
  // the MTP head copies too) and MoE layers (the router and the experts read x) keep x.
  // (The launches that form the norm take at most 8 k-groups per slice and 256 tile sums: a
  // model whose split-K widths leave more keeps x throughout.) Up to 4 rows: at 5..8 rows
  // (the 16-row kernel) every work-group of gate||up forming its rows' norm costs more than the
  // exchange it spares (27B shape, per layer at 8 rows: gate||up 47.2 against 27.7 us, o and
  // down 26.1 against 32.6; at 4 rows 28.1 against 24.7 and 23.8 against 28.9).
  bool split_norm(uint32_t M) const {
    if (M > 4) return false;
    if (d.experts || d.hidden / 64 > 256 || (d.hidden / 64) % 4) return false;
    auto ok = [](const Linear& l) { return (l.K / 64) / l.S <= 8; };
    for (uint32_t li = 0; li < d.layers; ++li)
      if (!ok(layer[li].qkv) || !ok(layer[li].gate_up)) return false;
    return !d.mtp || d.mtp_w16 || ok(mh.L.gate_up);
  }
  mi_gemv_epilogue resid_epi(const float* next_w, bool sums_only) const {
    mi_gemv_epilogue e{};
    e.kind = MI_EPI_RESID;
    e.resid = resid;
    if (sums_only) {
      e.sums_out = nsum;
    } else {
      e.sumsq = sumsq;
      e.rstd = rstd;
      e.next_norm_w = next_w;
      e.x_next = x;
    }
    e.eps = d.rms_eps;
    e.status = ctrl + MI_CTRL_DEBUG;
    e.arrive = use_arrive ? arrive : nullptr;
    e.act = d.act_bf16;
    return e;
  }

  // One step over M rows, enqueued on `stream` (recorded into a graph by capture()).
  // Six launches per layer (fp16 cache, M <= 4): the qkv GEMV with attn_prep fused;
  // attn_decode; attn_reduce; the o GEMV with the residual fold + post-attention norm fused;
  // gate||up GEMV with silu*up fused; down GEMV with the residual fold + next norm fused.
  // (The int8 cache or M > 4: the qkv partials and attn_prep apart.)
  int enqueue_step(uint32_t M) {
    if (M > kRowChunk) return enqueue_wide(M);
    const uint32_t HD = d.head_dim, KVH = d.kv_heads;
    const size_t layer_kv = size_t(KVH) * d.max_len * HD;
    if (d.mtp) {  // the head's control block for this step's K/V fill, before argmax moves ctrl
      mtp_fill_ctrl_kernel<<<1, 64, 0, stream>>>(ctrl, hctl, M);
      MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "mtp_fill_ctrl"));
    }
    MI_TRY(mi_embed_norm_act(ctrl, embed, resid, layer[0].in_norm, x, rstd, M, d.hidden, d.vocab, d.rms_eps,
                             d.act_bf16, stream));
    for (uint32_t li = 0; li < d.layers; ++li) {
      const Layer& L = layer[li];
      MI_TRY(launch_qkv(li, M, li > 0 && split_norm(M)));
      if (d.kv_int8) {  // capture.cc fa_layer under --kv-cache int8: kv8.cl's writer and reader pair
        int8_t* lk = static_cast<int8_t*>(kv_k) + li * layer_kv;
        int8_t* lv = static_cast<int8_t*>(kv_v) + li * layer_kv;
        uint16_t* lks = kv_ks + size_t(li) * KVH * d.max_len;
        uint16_t* lvs = kv_vs + size_t(li) * KVH * d.max_len;
        MI_TRY(mi_attn_prep_kv8(ctrl, part, L.qkv.S, M, &ash, L.q_norm, L.k_norm, rope, attn_q, nullptr, lk, lv,
                                lks, lvs, HD, size_t(d.max_len) * HD, 1, d.max_len, nullptr, 0, d.max_len,
                                stream));
        MI_TRY(mi_attn_decode(ctrl, attn_q, 1, lk, lv, lks, lvs, HD, size_t(d.max_len) * HD, 1, d.max_len,
                              nullptr, 0, d.max_len, attn_part, M, d.attn_tgt, &ash, stream));
        MI_TRY(mi_attn_reduce_kv8(ctrl, attn_part, nullptr, attn_out, M, d.attn_tgt, d.max_len, &ash, stream));
      } else {
        // attn_prep then the decode. (mi_attn_prep_decode does both in one launch with the same
        // values, but every decode block then folds q from the qkv partials again: at context
        // 4096, 33 blocks per kv head, that costs more than the separate launch saves.)
        uint16_t* lk = static_cast<uint16_t*>(kv_k) + li * layer_kv;
        uint16_t* lv = static_cast<uint16_t*>(kv_v) + li * layer_kv;
        MI_TRY(attn_pair(L, ctrl, lk, lv, M, !qkv_is_fused(M)));
      }
      MI_TRY(launch_o(L, M));
      const float* next_w = next_norm(li);
      if (d.experts) {
        // the MoE block (moe.cl:1-13): router || shared gate, route + gate||up (one launch:
        // each work-group routes its row itself), down folding into the residual, then the
        // next norm with nothing left to fold
        MI_TRY(moe_block(L, M, next_w));
        continue;
      }
      MI_TRY(launch_gate_up(L, M));
      MI_TRY(launch_down(L, M, next_w, split_norm(M) && li + 1 < d.layers));
    }
    MI_TRY(head(ctrl, M, x, logits, history));
    if (d.mtp) {
      // capture.cc:362-370: the rows' post-final-norm hidden (what lm_head read) into hh rows
      // 1..M, then the head's K/V over hh rows 0..M-1; a single-row step commits its row at
      // once (hh row 1 becomes row 0), as generate's verify(0) + commit(0) does
      const size_t row = size_t(d.hidden) * 2;
      MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(hh + d.hidden, x, row * M, hipMemcpyDeviceToDevice, stream)),
                    "hh rows"));
      MI_TRY(head_front(hh, M));
      if (M == 1)
        MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(hh, hh + d.hidden, row, hipMemcpyDeviceToDevice, stream)),
                      "hh commit"));
    }
    return 0;
  }

  // Row chunk c of a many-row list: while the guard lives, the row buffers point at the chunk's
  // rows and ctrl at the chunk's control block, so the launches serve a chunk exactly as they
  // serve a list of up to 8 rows.
  struct RowShift {
    mi_engine& e;
    uint32_t* ctrl;
    uint16_t *x, *resid, *attn_out, *hbuf, *moe_h;
    float *rstd, *nsum, *attn_q, *logits, *moe_logits;
    uint32_t* moe_route;
    RowShift(mi_engine& en, uint32_t c)
        : e(en), ctrl(en.ctrl), x(en.x), resid(en.resid), attn_out(en.attn_out), hbuf(en.hbuf), moe_h(en.moe_h),
          rstd(en.rstd), nsum(en.nsum), attn_q(en.attn_q), logits(en.logits), moe_logits(en.moe_logits),
          moe_route(en.moe_route) {
      const mi_model_desc& d = en.d;
      const size_t r0 = size_t(c) * kRowChunk, qd = size_t(d.q_heads) * d.head_dim;
      e.ctrl = en.cctl + size_t(c) * MI_CTRL_WORDS;
      e.x += r0 * d.hidden;
      e.resid += r0 * d.hidden;
      e.rstd += r0;
      e.nsum += r0 * (d.hidden / 64 + 1);
      e.attn_q += r0 * qd;
      e.attn_out += r0 * qd;
      e.hbuf += r0 * d.inter;
      e.logits += r0 * d.vocab;
      if (e.moe_logits) {
        e.moe_logits += r0 * en.router_n;
        e.moe_route += r0 * MI_MOE_ROUTE_WORDS;
        e.moe_h += r0 * (d.top_k + 1) * d.moe_inter;
      }
    }
    ~RowShift() {
      e.ctrl = ctrl; e.x = x; e.resid = resid; e.attn_out = attn_out; e.hbuf = hbuf; e.moe_h = moe_h;
      e.rstd = rstd; e.nsum = nsum; e.attn_q = attn_q; e.logits = logits; e.moe_logits = moe_logits;
      e.moe_route = moe_route;
    }
  };

  // A list of 9..64 rows (the reference's wide and deep verify lists, control.h:35-42,
  // verify_attn.h:65-92): per layer the qkv GEMV and attn_prep chunk by chunk (8 rows each, at
  // positions pos + 8 c ..), then the attention over all rows at once - mi_attn_verify where
  // the rule binds it, else the decode kernel chunk by chunk (the K/V rows of every chunk are
  // written by then) - then o, gate||up and down chunk by chunk; the head per chunk; then the
  // chunks' argmaxes into the list's out slots and pos advanced (chunk_gather_kernel). Every
  // row is the same row of an up-to-8-row list: the GEMV rows do not depend on the launch's
  // rows (property R), nor do attn_prep's or the decode kernel's.
  int enqueue_wide(uint32_t M) {
    const uint32_t HD = d.head_dim, KVH = d.kv_heads, nc = (M + kRowChunk - 1) / kRowChunk;
    const size_t layer_kv = size_t(KVH) * d.max_len * HD;
    auto rows = [&](uint32_t c) { return std::min(kRowChunk, M - c * kRowChunk); };
    chunk_ctrl_kernel<<<1, 64, 0, stream>>>(ctrl, cctl, M);
    MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "chunk_ctrl"));
    for (uint32_t c = 0; c < nc; ++c) {
      RowShift r(*this, c);
      MI_TRY(mi_embed_norm_act(ctrl, embed, resid, layer[0].in_norm, x, rstd, rows(c), d.hidden, d.vocab, d.rms_eps,
                               d.act_bf16, stream));
    }
    const bool verify_attn = !d.kv_int8 && mi_attn_verify_binds(M, 0, d.q_heads, d.kv_heads);
    for (uint32_t li = 0; li < d.layers; ++li) {
      const Layer& L = layer[li];
      const bool ni = li > 0 && split_norm(kRowChunk);
      void* lk = d.kv_int8 ? static_cast<void*>(static_cast<int8_t*>(kv_k) + li * layer_kv)
                           : static_cast<void*>(static_cast<uint16_t*>(kv_k) + li * layer_kv);
      void* lv = d.kv_int8 ? static_cast<void*>(static_cast<int8_t*>(kv_v) + li * layer_kv)
                           : static_cast<void*>(static_cast<uint16_t*>(kv_v) + li * layer_kv);
      uint16_t* lks = d.kv_int8 ? kv_ks + size_t(li) * KVH * d.max_len : nullptr;
      uint16_t* lvs = d.kv_int8 ? kv_vs + size_t(li) * KVH * d.max_len : nullptr;
      for (uint32_t c = 0; c < nc; ++c) {
        RowShift r(*this, c);
        const uint32_t Mc = rows(c);
        if (d.kv_int8) {
          MI_TRY(qkv_plain(L, Mc, ni));
          MI_TRY(mi_attn_prep_kv8(ctrl, part, L.qkv.S, Mc, &ash, L.q_norm, L.k_norm, rope, attn_q, nullptr,
                                  static_cast<int8_t*>(lk), static_cast<int8_t*>(lv), lks, lvs, HD,
                                  size_t(d.max_len) * HD, 1, d.max_len, nullptr, 0, d.max_len, stream));
        } else {
          MI_TRY(launch_qkv_on(L, ctrl, static_cast<uint16_t*>(lk), static_cast<uint16_t*>(lv), Mc, !qkv_is_fused(Mc),
                               ni));
        }
      }
      if (verify_attn) {
        MI_TRY(mi_attn_verify(ctrl, attn_q, static_cast<uint16_t*>(lk), static_cast<uint16_t*>(lv), HD,
                              size_t(d.max_len) * HD, nullptr, 0, d.max_len, attn_part, M, d.attn_tgt, &ash, stream));
        MI_TRY(mi_attn_reduce(ctrl, attn_part, nullptr, attn_out, M, d.attn_tgt, d.max_len, &ash, stream));
      } else {
        for (uint32_t c = 0; c < nc; ++c) {
          RowShift r(*this, c);
          const uint32_t Mc = rows(c);
          if (d.kv_int8) {
            MI_TRY(mi_attn_decode(ctrl, attn_q, 1, lk, lv, lks, lvs, HD, size_t(d.max_len) * HD, 1, d.max_len, nullptr,
                                  0, d.max_len, attn_part, Mc, d.attn_tgt, &ash, stream));
            MI_TRY(mi_attn_reduce_kv8(ctrl, attn_part, nullptr, attn_out, Mc, d.attn_tgt, d.max_len, &ash, stream));
          } else {
            MI_TRY(mi_attn_decode(ctrl, attn_q, 0, lk, lv, nullptr, nullptr, HD, size_t(d.max_len) * HD, 0, 0, nullptr,
                                  0, d.max_len, attn_part, Mc, d.attn_tgt, &ash, stream));
            MI_TRY(mi_attn_reduce(ctrl, attn_part, nullptr, attn_out, Mc, d.attn_tgt, d.max_len, &ash, stream));
          }
        }
      }
      const float* next_w = next_norm(li);
      for (uint32_t c = 0; c < nc; ++c) {
        RowShift r(*this, c);
        const uint32_t Mc = rows(c);
        MI_TRY(launch_o(L, Mc));
        if (d.experts) {
          MI_TRY(moe_block(L, Mc, next_w));
        } else {
          MI_TRY(launch_gate_up(L, Mc));
          MI_TRY(launch_down(L, Mc, next_w, split_norm(kRowChunk) && li + 1 < d.layers));
        }
      }
    }
    for (uint32_t c = 0; c < nc; ++c) {
      RowShift r(*this, c);
      MI_TRY(head(ctrl, rows(c), x, logits, nullptr));
    }
    chunk_gather_kernel<<<1, 64, 0, stream>>>(ctrl, cctl, M, history, d.max_len);
    return mi_hip(static_cast<int>(hipGetLastError()), "chunk_gather");
  }

  // ---- the MTP head (capture.cc:1772-1939) ----
  // head_front over M rows on the head's control block: enorm(embed(id)) and hnorm(hid row)
  // into the two halves of fc's input row (prep_norm_finish with X_STRIDE), fc, its output as
  // the head's residual (prep_res_fold ZERO_RESID) and the input norm, then q||k||v with
  // attn_prep into the head's KV layer at the head positions hctl.pos + r.
  int head_front(uint16_t* hid, uint32_t M) {
    const uint32_t H = d.hidden, G = H / 64;
    MI_TRY(mi_embed_gather(hctl, embed, resid, M, H, d.vocab, stream));
    MI_TRY(mi_res_fold(nullptr, resid, hsumsq, M, H, 0, G, stream));
    MI_TRY(mi_norm_finish_ex(hsumsq, resid, mh.pre_e, hx2, size_t(2) * H, M, H, G, d.rms_eps, stream));
    MI_TRY(mi_res_fold(nullptr, hid, hsumsq, M, H, 0, G, stream));
    MI_TRY(mi_norm_finish_ex(hsumsq, hid, mh.pre_h, hx2 + H, size_t(2) * H, M, H, G, d.rms_eps, stream));
    if (d.mtp_w16) {  // the 16-bit head: one [M][N] output per linear (S = 1 for the folds)
      const uint32_t HD = d.head_dim, qkv_n = (d.q_heads + 2 * d.kv_heads) * HD;
      MI_TRY(mi_gemv_f16w(mh.fc16, hx2, part, M, 2 * H, H, router_ksplit_of(2 * H), stream));
      MI_TRY(mi_res_fold_ex(part, resid, hsumsq, M, H, 1, G, 1, stream));
      MI_TRY(mi_norm_finish(hsumsq, resid, mh.L.in_norm, x, M, H, G, d.rms_eps, stream));
      MI_TRY(mi_gemv_f16w(mh.qkv16, x, part, M, H, qkv_n, router_ksplit_of(H), stream));
      return mi_attn_prep(hctl, part, 1, M, &ash, mh.L.q_norm, mh.L.k_norm, rope, attn_q, nullptr, hkv_k, hkv_v, HD,
                          size_t(d.max_len) * HD, nullptr, 0, d.max_len, stream);
    }
    MI_TRY(mi_gemv_w4a16(mh.fc.q, mh.fc.s, hx2, part, M, mh.fc.K, mh.fc.N, mh.fc.S, stream));
    MI_TRY(mi_res_fold_ex(part, resid, hsumsq, M, H, mh.fc.S, G, 1, stream));
    MI_TRY(mi_norm_finish(hsumsq, resid, mh.L.in_norm, x, M, H, G, d.rms_eps, stream));
    return launch_qkv_on(mh.L, hctl, hkv_k, hkv_v, M, true);
  }
  // the 16-bit head's o with the residual and the post-attention norm, its MLP, and its final
  // norm into x (one row): the standalone kernels on the GEMV's [1][N] output (S = 1)
  int draft_tail16() {
    const uint32_t H = d.hidden, G = H / 64, QD = d.q_heads * d.head_dim, I = d.inter;
    MI_TRY(mi_gemv_f16w(mh.o16, attn_out, part, 1, QD, H, router_ksplit_of(QD), stream));
    MI_TRY(mi_res_fold(part, resid, hsumsq, 1, H, 1, G, stream));
    MI_TRY(mi_norm_finish(hsumsq, resid, mh.L.post_norm, x, 1, H, G, d.rms_eps, stream));
    MI_TRY(mi_gemv_f16w(mh.gu16, x, part, 1, H, 2 * I, router_ksplit_of(H), stream));
    MI_TRY(mi_silu_mul(part, hbuf, 1, I, 1, stream));
    MI_TRY(mi_gemv_f16w(mh.dn16, hbuf, part, 1, I, H, router_ksplit_of(I), stream));
    MI_TRY(mi_res_fold(part, resid, hsumsq, 1, H, 1, G, stream));
    return mi_norm_finish(hsumsq, resid, mh.final_n, x, 1, H, G, d.rms_eps, stream);
  }
  // an MoE layer's FFN on x (rows M): router || shared gate, route + gate||up, down + combine
  // into the residual with the next norm (weights next_w) into x
  int moe_block(const Layer& L, uint32_t M, const float* next_w) {
    MI_TRY(mi_gemv_f16w(L.router, x, moe_logits, M, d.hidden, router_n, router_ksplit(), stream));
    MI_TRY(mi_moe_gate_up_routed(moe_logits, router_n, moe_route, x, L.moe_gu, moe_h, M, d.experts, d.top_k,
                                 d.hidden, d.moe_inter, stream));
    return mi_moe_down_norm(moe_route, moe_h, L.moe_dn, resid, M, d.experts, d.top_k, d.hidden, d.moe_inter, next_w,
                            x, rstd, d.rms_eps, dn_words, ctrl + MI_CTRL_DEBUG, 0, 0, stream);
  }

  // draft() (capture.cc:1849-1939): the whole head at one row on hctl, from (hctl's id, dh);
  // its final-normed hidden back into dh, its logits into hlogits, the argmax into hctl
  int enqueue_draft() {
    MI_TRY(head_front(dh, 1));
    MI_TRY(attn_pair(mh.L, hctl, hkv_k, hkv_v, 1, false));
    if (d.mtp_w16) {
      MI_TRY(draft_tail16());
    } else {
      MI_TRY(launch_o(mh.L, 1));
      if (d.experts) {  // an MoE model's head: its MoE layer (capture.cc:1913's moe_block)
        MI_TRY(moe_block(mh.L, 1, mh.final_n));
      } else {
        MI_TRY(launch_gate_up(mh.L, 1));
        MI_TRY(launch_down(mh.L, 1, mh.final_n, false));
      }
    }
    MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(dh, x, size_t(d.hidden) * 2, hipMemcpyDeviceToDevice, stream)),
                  "dh"));
    return head(hctl, 1, x, hlogits, hhist);
  }

  // head() (capture.cc:1461-1480 / 1913-1939): the lm_head over rows xin into out and the argmax
  // into control block c (out_token, cur_token, history, pos += n_active): the int4 head's
  // LOGITS launch (logits + tile winners) and argmax_stage2, or the int8 head's gemv_i8w and
  // both argmax stages
  int head(uint32_t* c, uint32_t M, const uint16_t* xin, float* out, uint32_t* hist) {
    if (d.lm_head_int8) {
      MI_TRY(mi_gemv_i8w(lm_i8, lm_i8s, xin, out, M, d.hidden, d.vocab, stream));
      return mi_argmax(c, out, argmax_part, hist, d.max_len, M, d.vocab, d.vocab_used, stream);
    }
    MI_TRY(launch_lm_head(M, xin, out));
    return mi_argmax_finish(c, argmax_part, d.vocab / 64, hist, d.max_len, stream);
  }

  // ---- the step's int4 GEMV launches, one per linear, as enqueue_step issues them ----
  bool qkv_is_fused(uint32_t M) const {
    return !d.kv_int8 && (d.head_dim == 128 || d.head_dim == 256) && M <= 4;
  }
  const float* next_norm(uint32_t li) const { return li + 1 < d.layers ? layer[li + 1].in_norm : final_norm; }

  // the qkv GEMV of layer li; with the f16 cache and M <= 4, attn_prep inside it (one consumer
  // work-group per head), else plain partials for mi_attn_prep / mi_attn_prep_kv8
  // the qkv GEMV's input: x, or (ni) the residual with nsum, the layer's input norm formed by
  // the launch
  int qkv_plain(const Layer& L, uint32_t M, bool ni) {
    if (!ni) return mi_gemv_w4a16(L.qkv.q, L.qkv.s, x, part, M, L.qkv.K, L.qkv.N, L.qkv.S, stream);
    mi_gemv_epilogue ep{};
    ep.kind = MI_EPI_PARTIALS;
    norm_in(ep, L.in_norm);
    return mi_gemv_w4a16_ex(L.qkv.q, L.qkv.s, resid, part, M, L.qkv.K, L.qkv.N, L.qkv.S, &ep, stream);
  }
  void norm_in(mi_gemv_epilogue& e, const float* w) const {
    e.in_sums = nsum;
    e.in_norm_w = w;
    e.in_eps = d.rms_eps;
    e.act = d.act_bf16;
  }
  int launch_qkv(uint32_t li, uint32_t M, bool ni) {
    const size_t layer_kv = size_t(d.kv_heads) * d.max_len * d.head_dim;
    if (d.kv_int8) return qkv_plain(layer[li], M, ni);
    return launch_qkv_on(layer[li], ctrl, static_cast<uint16_t*>(kv_k) + li * layer_kv,
                         static_cast<uint16_t*>(kv_v) + li * layer_kv, M, false, ni);
  }
  // layer L's qkv on control block c, K/V rows into the f16 layer lk / lv; prep: run attn_prep
  // here too when it is not fused (M > 4); ni: the input norm formed by the launch
  int launch_qkv_on(const Layer& L, uint32_t* c, uint16_t* lk, uint16_t* lv, uint32_t M, bool prep, bool ni = false) {
    const uint32_t HD = d.head_dim;
    if (!qkv_is_fused(M)) {
      MI_TRY(qkv_plain(L, M, ni));
      return prep ? mi_attn_prep(c, part, L.qkv.S, M, &ash, L.q_norm, L.k_norm, rope, attn_q, nullptr, lk, lv, HD,
                                 size_t(d.max_len) * HD, nullptr, 0, d.max_len, stream)
                  : 0;
    }
    mi_gemv_epilogue eq{};
    eq.kind = MI_EPI_QKV;
    eq.ctrl = c;
    eq.shape = &ash;
    eq.q_norm = L.q_norm;
    eq.k_norm = L.k_norm;
    eq.rope = rope;
    eq.attn_q = attn_q;
    eq.kv_k = lk;
    eq.kv_v = lv;
    eq.row_stride = HD;
    eq.head_stride = size_t(d.max_len) * HD;
    eq.kv_len = d.max_len;
    eq.status = ctrl + MI_CTRL_DEBUG;
    eq.arrive = use_arrive ? arrive : nullptr;
    eq.act = d.act_bf16;
    if (ni) norm_in(eq, L.in_norm);
    return mi_gemv_w4a16_ex(L.qkv.q, L.qkv.s, ni ? resid : x, part_ex, M, L.qkv.K, L.qkv.N, L.qkv.S, &eq, stream);
  }
  // the f16 cache's attention pair on control block c over the layer lk / lv: attn_prep first
  // when `prep` (the qkv launch did not fuse it); verify_attn.h's rule picks the many-row kernel for
  // the lists it binds (16, 32, 64 rows at 16 / 2 heads), else the decode kernel (every list
  // this engine builds: M <= 8); then the merge
  int attn_pair(const Layer& L, uint32_t* c, uint16_t* lk, uint16_t* lv, uint32_t M, bool prep) {
    const uint32_t HD = d.head_dim;
    if (prep)
      MI_TRY(mi_attn_prep(c, part, L.qkv.S, M, &ash, L.q_norm, L.k_norm, rope, attn_q, nullptr, lk, lv, HD,
                          size_t(d.max_len) * HD, nullptr, 0, d.max_len, stream));
    if (mi_attn_verify_binds(M, 0, d.q_heads, d.kv_heads))
      MI_TRY(mi_attn_verify(c, attn_q, lk, lv, HD, size_t(d.max_len) * HD, nullptr, 0, d.max_len, attn_part, M,
                            d.attn_tgt, &ash, stream));
    else
      MI_TRY(mi_attn_decode(c, attn_q, 0, lk, lv, nullptr, nullptr, HD, size_t(d.max_len) * HD, 0, 0, nullptr, 0,
                            d.max_len, attn_part, M, d.attn_tgt, &ash, stream));
    return mi_attn_reduce(c, attn_part, nullptr, attn_out, M, d.attn_tgt, d.max_len, &ash, stream);
  }
  // o with the residual fold and the post-attention norm
  int launch_o(const Layer& L, uint32_t M) {
    const mi_gemv_epilogue eo = resid_epi(L.post_norm, split_norm(M));
    return mi_gemv_w4a16_ex(L.o.q, L.o.s, attn_out, part_ex, M, L.o.K, L.o.N, L.o.S, &eo, stream);
  }
  // gate||up with silu * up
  int launch_gate_up(const Layer& L, uint32_t M) {
    mi_gemv_epilogue eg{};
    eg.kind = MI_EPI_SILU;
    eg.h = hbuf;
    eg.status = ctrl + MI_CTRL_DEBUG;
    eg.arrive = use_arrive ? arrive : nullptr;
    eg.act = d.act_bf16;
    if (split_norm(M)) norm_in(eg, L.post_norm);
    return mi_gemv_w4a16_ex(L.gate_up.q, L.gate_up.s, split_norm(M) ? resid : x, part_ex, M, L.gate_up.K,
                            L.gate_up.N, L.gate_up.S, &eg, stream);
  }
  // down with the residual fold and the next norm (the next layer's, the final one, the head's);
  // sums_only: the residual and its tile sums only (the next qkv forms the norm)
  int launch_down(const Layer& L, uint32_t M, const float* next_w, bool sums_only) {
    const mi_gemv_epilogue ed = resid_epi(next_w, sums_only);
    return mi_gemv_w4a16_ex(L.down.q, L.down.s, hbuf, part_ex, M, L.down.K, L.down.N, L.down.S, &ed, stream);
  }
  // the int4 lm_head with the logits and the per-tile argmax
  int launch_lm_head(uint32_t M, const uint16_t* xin, float* out) {
    mi_gemv_epilogue el{};
    el.kind = MI_EPI_LOGITS;
    el.logits = out;
    el.argmax_part = argmax_part;
    el.vocab_used = d.vocab_used;
    el.status = ctrl + MI_CTRL_DEBUG;
    el.arrive = use_arrive ? arrive : nullptr;
    return mi_gemv_w4a16_ex(lm_head.q, lm_head.s, xin, part_ex, M, lm_head.K, lm_head.N, lm_head.S, &el, stream);
  }

  // `reps` rounds of one linear's step launch (0 qkv, 1 o, 2 gate_up, 3 down: every layer's in
  // turn; 4 the lm_head) back to back on the stream, HIP events around; *ms = the average per
  // launch. The launches rewrite the step's buffers (residual, KV row at pos, logits): the
  // caller resets the engine afterwards.
  int bench_linear(uint32_t which_rows, uint32_t reps, float* ms) {
    const uint32_t which = which_rows & 0xFFu, M = (which_rows >> 8) ? (which_rows >> 8) : 1u;
    if (which > 4 || reps == 0 || !ms || M > kRowChunk || M > d.max_rows)
      return mi_fail(MI_ERR_ARG, "engine_bench_linear: which 0..4, rows 1..8, reps > 0");
    if (d.experts && (which == 2 || which == 3))
      return mi_fail(MI_ERR_SHAPE, "engine_bench_linear: an MoE model has no dense gate_up / down");
    auto one = [&](uint32_t li) -> int {
      switch (which) {
        case 0: return launch_qkv(li, M, li > 0 && split_norm(M));
        case 1: return launch_o(layer[li], M);
        case 2: return launch_gate_up(layer[li], M);
        case 3: return launch_down(layer[li], M, next_norm(li), split_norm(M) && li + 1 < d.layers);
        default:
          return d.lm_head_int8 ? mi_gemv_i8w(lm_i8, lm_i8s, x, logits, M, d.hidden, d.vocab, stream)
                                : launch_lm_head(M, x, logits);
      }
    };
    const uint32_t per_round = which == 4 ? 1u : d.layers;
    for (uint32_t li = 0; li < per_round; ++li) MI_TRY(one(li));  // warm-up round
    hipEvent_t a, b;
    MI_TRY(mi_hip(static_cast<int>(hipEventCreate(&a)), "event"));
    MI_TRY(mi_hip(static_cast<int>(hipEventCreate(&b)), "event"));
    MI_TRY(mi_hip(static_cast<int>(hipEventRecord(a, stream)), "event record"));
    for (uint32_t r = 0; r < reps; ++r)
      for (uint32_t li = 0; li < per_round; ++li) MI_TRY(one(li));
    MI_TRY(mi_hip(static_cast<int>(hipEventRecord(b, stream)), "event record"));
    MI_TRY(mi_hip(static_cast<int>(hipEventSynchronize(b)), "event sync"));
    float t = 0.f;
    MI_TRY(mi_hip(static_cast<int>(hipEventElapsedTime(&t, a, b)), "event elapsed"));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    *ms = t / float(reps * per_round);
    return check_handoff();
  }

  // `reps` verify steps of M live rows at the current position (ids: cur_token in every row),
  // each the rows' control reset (one one-thread kernel) and the captured M-row graph (bit 8 of
  // rows_mode: the same step enqueued kernel by kernel, for kernel tracers), back to
  // back on the engine's stream; *ms = the HIP-event time per step. Leaves pos and cur as they
  // were, n_active 1; the cache rows pos .. pos + M - 1 hold the last step's K/V.
  int bench_verify(uint32_t rows_mode, uint32_t reps, float* ms) {
    const uint32_t M = rows_mode & 0xFFu;
    const bool eager = rows_mode & 0x100u;
    if (M == 0 || M > d.max_rows || reps == 0 || !ms || (rows_mode >> 9))
      return mi_fail(MI_ERR_ARG, "engine_bench_verify: bad args");
    if (!eager) MI_TRY(capture(M));
    uint32_t c[MI_CTRL_WORDS];
    MI_TRY(read_ctrl(c));
    const uint32_t pos = c[MI_CTRL_POS], cur = c[MI_CTRL_CUR];
    if (pos + M > d.max_len) return mi_fail(MI_ERR_ARG, "engine_bench_verify: past the KV cache");
    const std::vector<uint32_t> ids(M, cur);
    MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(ids_dev, ids.data(), M * 4, hipMemcpyHostToDevice, stream)),
                  "ids upload"));
    auto one = [&]() -> int {
      ctrl_set_rows_kernel<<<1, 64, 0, stream>>>(ctrl, pos, M, ids_dev, M);
      MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "ctrl_set_rows"));
      if (eager) return enqueue_step(M);
      return mi_hip(static_cast<int>(hipGraphLaunch(graphs[M], stream)), "hipGraphLaunch");
    };
    for (int w = 0; w < 3; ++w) MI_TRY(one());
    hipEvent_t a, b;
    MI_TRY(mi_hip(static_cast<int>(hipEventCreate(&a)), "event"));
    MI_TRY(mi_hip(static_cast<int>(hipEventCreate(&b)), "event"));
    MI_TRY(mi_hip(static_cast<int>(hipEventRecord(a, stream)), "event record"));
    for (uint32_t r = 0; r < reps; ++r) MI_TRY(one());
    MI_TRY(mi_hip(static_cast<int>(hipEventRecord(b, stream)), "event record"));
    MI_TRY(mi_hip(static_cast<int>(hipEventSynchronize(b)), "event sync"));
    float t = 0.f;
    MI_TRY(mi_hip(static_cast<int>(hipEventElapsedTime(&t, a, b)), "event elapsed"));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    *ms = t / float(reps);
    MI_TRY(check_handoff());
    return set_rows(pos, 1, &cur, 1);
  }

  int capture(uint32_t M) {
    if (graphs[M]) return 0;
    hipGraph_t g = nullptr;
    MI_TRY(mi_hip(static_cast<int>(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal)),
                  "hipStreamBeginCapture"));
    const int e = enqueue_step(M);
    const int e2 = static_cast<int>(hipStreamEndCapture(stream, &g));
    if (e != 0) {
      if (g) (void)hipGraphDestroy(g);
      return e;
    }
    MI_TRY(mi_hip(e2, "hipStreamEndCapture"));
    const int e3 = static_cast<int>(hipGraphInstantiate(&graphs[M], g, nullptr, nullptr, 0));
    (void)hipGraphDestroy(g);
    return mi_hip(e3, "hipGraphInstantiate");
  }

  int capture_draft() {
    if (draft_graph) return 0;
    hipGraph_t g = nullptr;
    MI_TRY(mi_hip(static_cast<int>(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal)),
                  "hipStreamBeginCapture"));
    const int e = enqueue_draft();
    const int e2 = static_cast<int>(hipStreamEndCapture(stream, &g));
    if (e != 0) {
      if (g) (void)hipGraphDestroy(g);
      return e;
    }
    MI_TRY(mi_hip(e2, "hipStreamEndCapture"));
    const int e3 = static_cast<int>(hipGraphInstantiate(&draft_graph, g, nullptr, nullptr, 0));
    (void)hipGraphDestroy(g);
    return mi_hip(e3, "hipGraphInstantiate");
  }

  // Engine::draft (engine.h:259-290): k draft lists, each one replay of the draft graph
  int draft(uint32_t k, uint32_t* out) {
    if (!d.mtp) return mi_fail(MI_ERR_STATE, "engine_draft: the model has no MTP head");
    if (k == 0 || k > kMaxDraft || !out) return mi_fail(MI_ERR_ARG, "engine_draft: k must be 1..3");
    uint32_t c[MI_CTRL_WORDS];
    MI_TRY(read_ctrl(c));
    if (c[MI_CTRL_POS] == 0 || c[MI_CTRL_POS] + k + 1 > d.max_len)
      return mi_fail(MI_ERR_ARG, "engine_draft: needs 1 <= pos and pos + k + 1 <= max_len");
    MI_TRY(capture_draft());
    mtp_draft_begin_kernel<<<1, 256, 0, stream>>>(ctrl, hctl, hh, dh, d.hidden);
    MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "mtp_draft_begin"));
    for (uint32_t i = 0; i < k; ++i)
      MI_TRY(mi_hip(static_cast<int>(hipGraphLaunch(draft_graph, stream)), "draft hipGraphLaunch"));
    MI_TRY(mi_memcpy_d2h(out, hhist, size_t(k) * 4, stream));
    MI_TRY(mi_stream_sync(stream));
    return check_handoff();
  }

  // step_mtp_kv (src/runtime/prefill/step.h:181-196) for a prefill chunk of T positions from
  // pos whose final-normed rows are in pf_x: the head's K/V at positions pos - 1 + r from
  // (h_{pos-1+r}, ids[r]) - hh row 0 for r = 0, pf_x row r - 1 after (at pos 0 from r = 1) -
  // in groups of max_rows rows through head_front, the decode step's own launches; then hh row
  // 0 = the chunk's last row.
  int prefill_head_fill(const uint32_t* ids_chunk, uint32_t pos, uint32_t T) {
    const size_t row = size_t(d.hidden) * 2;
    for (uint32_t r = pos == 0 ? 1u : 0u; r < T;) {
      const uint32_t n = std::min(d.max_rows, T - r);
      if (r == 0) {
        if (n > 1)
          MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(hh + d.hidden, pf_x, row * (n - 1), hipMemcpyDeviceToDevice,
                                                        stream)), "hh rows"));
      } else {
        MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(hh, pf_x + size_t(r - 1) * d.hidden, row * n,
                                                      hipMemcpyDeviceToDevice, stream)), "hh rows"));
      }
      ctrl_set_rows_kernel<<<1, 64, 0, stream>>>(hctl, pos + r - 1, n, ids_chunk + r, n);
      MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "head ctrl"));
      MI_TRY(head_front(hh, n));
      r += n;
    }
    return mi_hip(static_cast<int>(hipMemcpyAsync(hh, pf_x + size_t(T - 1) * d.hidden, row, hipMemcpyDeviceToDevice,
                                                  stream)), "hh row 0");
  }

  int set_rows(uint32_t pos, uint32_t n_act, const uint32_t* ids, uint32_t n_ids) {
    if (n_ids) {
      MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(ids_dev, ids, n_ids * 4, hipMemcpyHostToDevice, stream)),
                    "ids upload"));
    }
    ctrl_set_rows_kernel<<<1, 64, 0, stream>>>(ctrl, pos, n_act, ids_dev, n_ids);
    return mi_hip(static_cast<int>(hipGetLastError()), "ctrl_set_rows");
  }

  int read_ctrl(uint32_t* out) {
    return mi_memcpy_d2h(out, ctrl, MI_CTRL_WORDS * 4, stream);
  }

  // After the stream has drained: a fused launch whose hand-off wait timed out leaves
  // MI_STATUS_HANDOFF_TIMEOUT in the debug word, and its hand-off words may hold values that
  // were published late. Those are emptied again here so the next step starts clean, and the
  // caller gets an error (the tokens of that call are not to be used). The word is cleared.
  // A step whose logits were not finite (MI_STATUS_NONFINITE from the argmax) fails the call
  // the same way.
  int check_handoff() {
    uint32_t c[MI_CTRL_WORDS];
    MI_TRY(read_ctrl(c));
    if (c[MI_CTRL_DEBUG] == MI_STATUS_NONFINITE) {  // an activation left the fp16 range
      ctrl_set_kernel<<<1, 64, 0, stream>>>(ctrl, MI_CTRL_DEBUG, 0u);
      MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "ctrl_set"));
      MI_TRY(mi_stream_sync(stream));
      return mi_fail(MI_ERR_STATE, "a logit of the step was not finite (an activation left the fp16 range); "
                                   "the step's token is not to be used");
    }
    if (c[MI_CTRL_DEBUG] != MI_STATUS_HANDOFF_TIMEOUT) return 0;
    MI_TRY(mi_gemv_handoff_init(part_ex, part_ex_n, stream));
    MI_TRY(mi_gemv_handoff_init(sumsq, sumsq_n, stream));
    if (dn_words) MI_TRY(mi_gemv_handoff_init(reinterpret_cast<float*>(dn_words), size_t(std::min(d.max_rows, kRowChunk)) * (d.hidden / 2), stream));
    MI_TRY(mi_hip(static_cast<int>(hipMemsetAsync(arrive, 0, arrive_n * 4, stream)), "arrive clear"));
    ctrl_set_kernel<<<1, 64, 0, stream>>>(ctrl, MI_CTRL_DEBUG, 0u);
    MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "ctrl_set"));
    MI_TRY(mi_stream_sync(stream));
    return mi_fail(MI_ERR_STATE, "a fused GEMV's hand-off wait timed out; the step's output is invalid "
                                 "(hand-off words re-initialised)");
  }

  // ---- chunked prefill (Engine::prefill, src/runtime/engine.h:97-115; the walk of
  // src/runtime/prefill/step.h step_chunk). Scratch is allocated on the first call for the
  // largest chunk asked so far, as the reference allocates its prefill scratch on first use. ----
  uint32_t pf_cap = 0;
  uint32_t* pf_ids = nullptr;    // [max_len] the prompt's ids
  uint32_t* pf_ctrl = nullptr;   // the chunk's control block: pos = its first position, n_act = T
  float* pf_out = nullptr;       // [cap][widest linear] fp32 linear outputs
  float* pf_q = nullptr;         // [cap][q_heads][head_dim]
  uint16_t* pf_resid = nullptr;  // [cap][hidden]
  uint16_t* pf_x = nullptr;      // [cap][max(hidden, q_heads * head_dim)]
  uint16_t* pf_h = nullptr;      // [cap][inter]
  uint16_t* pf_attn = nullptr;   // [cap][q_heads * head_dim]
  // MoE chunks: route rows, the grouped pairs' list and row tiles, and the pair outputs
  float* pf_logits = nullptr;    // [cap][router_n]
  uint32_t* pf_route = nullptr;  // [cap][MI_MOE_ROUTE_WORDS]
  uint32_t* pf_list = nullptr;   // [cap (top_k + 1)]
  uint32_t* pf_tiles = nullptr;  // [(cap (top_k + 1) + 63) / 64 + experts + 1][4]
  uint32_t* pf_tiles_n = nullptr;
  uint16_t* pf_mh = nullptr;     // [cap (top_k + 1)][moe_inter]
  uint16_t* pf_md = nullptr;     // [cap (top_k + 1)][hidden] f16

  int prefill_alloc(uint32_t cap) {
    if (cap <= pf_cap) return 0;
    const size_t H = d.hidden, QHD = size_t(d.q_heads) * d.head_dim;
    const size_t qkv_n = size_t(d.q_heads + 2 * d.kv_heads) * d.head_dim;
    const size_t widest = std::max({qkv_n, 2 * size_t(d.inter), H});
    if (!pf_ids) {
      MI_TRY(alloc(&pf_ids, d.max_len));
      MI_TRY(alloc(&pf_ctrl, MI_CTRL_WORDS));
      MI_TRY(mi_hip(static_cast<int>(hipMemsetAsync(pf_ctrl, 0, MI_CTRL_WORDS * 4, stream)), "prefill ctrl clear"));
    }
    if (pf_cap) {
      // a larger chunk than before: the previous set goes (after the stream has drained)
      MI_TRY(mi_stream_sync(stream));
      for (void** p : {(void**)&pf_out, (void**)&pf_q, (void**)&pf_resid, (void**)&pf_x, (void**)&pf_h,
                       (void**)&pf_attn, (void**)&pf_logits, (void**)&pf_route, (void**)&pf_list,
                       (void**)&pf_tiles, (void**)&pf_tiles_n, (void**)&pf_mh, (void**)&pf_md})
        release(p);
    }
    MI_TRY(alloc(&pf_out, size_t(cap) * widest));
    MI_TRY(alloc(&pf_q, size_t(cap) * QHD));
    MI_TRY(alloc(&pf_resid, size_t(cap) * H));
    MI_TRY(alloc(&pf_x, size_t(cap) * std::max(H, QHD)));
    MI_TRY(alloc(&pf_h, size_t(cap) * std::max(d.inter, 1u)));
    MI_TRY(alloc(&pf_attn, size_t(cap) * QHD));
    if (d.experts) {
      const size_t pairs = size_t(cap) * (d.top_k + 1);
      MI_TRY(alloc(&pf_logits, size_t(cap) * router_n));
      MI_TRY(alloc(&pf_route, size_t(cap) * MI_MOE_ROUTE_WORDS));
      MI_TRY(alloc(&pf_list, pairs));
      MI_TRY(alloc(&pf_tiles, ((pairs + 63) / 64 + d.experts + 1) * 4));
      MI_TRY(alloc(&pf_tiles_n, 1));
      MI_TRY(alloc(&pf_mh, pairs * d.moe_inter));
      MI_TRY(alloc(&pf_md, pairs * H));
    }
    pf_cap = cap;
    return 0;
  }

  // One chunk of T positions from pos: every layer over the chunk's rows; leaves the last
  // layer's normed rows (the final norm's output) in pf_x.
  int prefill_chunk(const uint32_t* ids_dev_chunk, uint32_t pos, uint32_t T) {
    const uint32_t H = d.hidden, HD = d.head_dim, QHD = d.q_heads * d.head_dim;
    const size_t layer_kv = size_t(d.kv_heads) * d.max_len * HD;
    ctrl_set_rows_kernel<<<1, 64, 0, stream>>>(pf_ctrl, pos, T, nullptr, 0);
    MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "prefill ctrl"));
    MI_TRY(mi_embed_rows(ids_dev_chunk, embed, pf_resid, T, H, d.vocab, pf_ctrl + MI_CTRL_DEBUG, stream));
    MI_TRY(mi_res_norm(nullptr, pf_resid, layer[0].in_norm, pf_x, T, H, 0, d.rms_eps, stream));
    for (uint32_t li = 0; li < d.layers; ++li) {
      const Layer& L = layer[li];
      MI_TRY(mi_gemm_w4a16(L.qkv.q, L.qkv.s, pf_x, pf_out, T, L.qkv.K, L.qkv.N, stream));
      if (d.kv_int8) {  // attn_prep_kv8's rows, the int8 reader, the un-rotation (pf_out is free here)
        int8_t* lk = static_cast<int8_t*>(kv_k) + li * layer_kv;
        int8_t* lv = static_cast<int8_t*>(kv_v) + li * layer_kv;
        uint16_t* lks = kv_ks + size_t(li) * d.kv_heads * d.max_len;
        uint16_t* lvs = kv_vs + size_t(li) * d.kv_heads * d.max_len;
        MI_TRY(mi_attn_prep_kv8(pf_ctrl, pf_out, 1, T, &ash, L.q_norm, L.k_norm, rope, pf_q, nullptr, lk, lv, lks,
                                lvs, HD, size_t(d.max_len) * HD, 1, d.max_len, nullptr, 0, d.max_len, stream));
        MI_TRY(mi_attn_prefill_kv8(pf_q, lk, lv, lks, lvs, HD, size_t(d.max_len) * HD, 1, d.max_len, nullptr, 0, T,
                                   pos, &ash, pf_out, pf_attn, stream));
      } else {
        uint16_t* lk = static_cast<uint16_t*>(kv_k) + li * layer_kv;
        uint16_t* lv = static_cast<uint16_t*>(kv_v) + li * layer_kv;
        MI_TRY(mi_attn_prep_rows(pf_out, T, pos, &ash, L.q_norm, L.k_norm, rope, pf_q, lk, lv, HD,
                                 size_t(d.max_len) * HD, nullptr, 0, stream));
        MI_TRY(mi_attn_prefill(pf_q, lk, lv, HD, size_t(d.max_len) * HD, nullptr, 0, T, pos, &ash, pf_attn, stream));
      }
      MI_TRY(mi_gemm_w4a16(L.o.q, L.o.s, pf_attn, pf_out, T, QHD, H, stream));
      MI_TRY(mi_res_norm(pf_out, pf_resid, L.post_norm, pf_x, T, H, 1, d.rms_eps, stream));
      const float* next_w = li + 1 < d.layers ? layer[li + 1].in_norm : final_norm;
      if (d.experts) {
        // the MoE block (moe.cl:1-13): router || shared gate and the route of every row of the
        // chunk in one launch each, then the expert FFN grouped by expert
        MI_TRY(mi_gemv_f16w(L.router, pf_x, pf_logits, T, H, router_n, router_ksplit(), stream));
        MI_TRY(mi_moe_route(pf_logits, pf_route, T, d.experts, d.top_k, router_n, stream));
        MI_TRY(mi_moe_prefill(pf_route, pf_x, L.moe_gu, L.moe_dn, pf_resid, T, d.experts, d.top_k, H, d.moe_inter,
                              pf_list, pf_tiles, pf_tiles_n, pf_mh, pf_md, stream));
        MI_TRY(mi_res_norm(nullptr, pf_resid, next_w, pf_x, T, H, 0, d.rms_eps, stream));
        continue;
      }
      MI_TRY(mi_gemm_w4a16_silu(L.gate_up.q, L.gate_up.s, pf_x, pf_h, T, H, L.gate_up.N, stream));
      MI_TRY(mi_gemm_w4a16(L.down.q, L.down.s, pf_h, pf_out, T, d.inter, H, stream));
      MI_TRY(mi_res_norm(pf_out, pf_resid, next_w, pf_x, T, H, 1, d.rms_eps, stream));
    }
    return 0;
  }

  int prefill(const uint32_t* ids, uint32_t n, uint32_t chunk) {
    if (!ids || n == 0) return mi_fail(MI_ERR_ARG, "engine_prefill: no ids");
    if (d.act_bf16) return mi_fail(MI_ERR_SHAPE, "engine_prefill: f16 activations only (ingest the prompt instead)");
    if (chunk == 0) chunk = std::min(kPrefillCap, d.max_len);
    if (chunk > kPrefillCap) return mi_fail(MI_ERR_ARG, "engine_prefill: chunk above the cap (2048)");
    for (uint32_t i = 0; i < n; ++i)
      if (ids[i] >= d.vocab) return mi_fail(MI_ERR_ARG, "engine_prefill: an id outside the vocabulary");
    uint32_t c[MI_CTRL_WORDS];
    MI_TRY(read_ctrl(c));
    const uint32_t pos0 = c[MI_CTRL_POS];
    if (size_t(pos0) + n > d.max_len) return mi_fail(MI_ERR_ARG, "engine_prefill: past the KV cache");
    MI_TRY(prefill_alloc(std::min(chunk, n)));
    MI_TRY(mi_hip(static_cast<int>(hipMemsetAsync(pf_ctrl, 0, MI_CTRL_WORDS * 4, stream)), "prefill ctrl clear"));
    MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(pf_ids, ids, size_t(n) * 4, hipMemcpyHostToDevice, stream)),
                  "prefill ids upload"));
    MI_TRY(mi_stream_sync(stream));  // the host array may go once this returns
    uint32_t T = 0;
    for (uint32_t c0 = 0; c0 < n; c0 += chunk) {
      T = std::min(chunk, n - c0);
      MI_TRY(prefill_chunk(pf_ids + c0, pos0 + c0, T));
      if (d.mtp) MI_TRY(prefill_head_fill(pf_ids + c0, pos0 + c0, T));
    }
    // the last position's head and argmax, on the decode control block: the step at pos0 + n - 1
    // leaves cur_token = its argmax and pos = pos0 + n, as ingest's last replay would
    MI_TRY(set_rows(pos0 + n - 1, 1, nullptr, 0));
    MI_TRY(head(ctrl, 1, pf_x + size_t(T - 1) * d.hidden, logits, history));
    MI_TRY(mi_stream_sync(stream));
    uint32_t pc[MI_CTRL_WORDS];
    MI_TRY(mi_memcpy_d2h(pc, pf_ctrl, sizeof pc, stream));
    if (pc[MI_CTRL_DEBUG]) return mi_fail(MI_ERR_STATE, "engine_prefill: the device flagged the chunk");
    return 0;
  }
};

extern "C" {

mi_engine* mi_engine_create(const mi_model_desc* desc, uint64_t seed, void* stream) {
  if (!desc) {
    mi_fail(MI_ERR_ARG, "engine_create: null desc");
    return nullptr;
  }
  const mi_model_desc& m = *desc;
  if (m.layers == 0 || m.hidden % 256 || m.hidden > 65536 || (m.head_dim != 128 && m.head_dim != 256) || m.kv_heads == 0 ||
      m.q_heads % m.kv_heads || m.q_heads / m.kv_heads > 8 || m.inter % 64 || m.vocab % 64 ||
      m.vocab_used > m.vocab || m.max_len == 0 || m.max_rows == 0 || m.max_rows > 64 || (m.max_rows > 8 && m.mtp) ||
      m.rot_dim > m.head_dim ||
      m.attn_tgt == 0 || (m.q_heads * m.head_dim) % 64 || m.kv_int8 > 1 || (m.kv_int8 && m.head_dim != 256) ||
      m.mtp > 1 || m.mtp_w16 > 1 || (m.mtp_w16 && (!m.mtp || m.experts)) || m.lm_head_int8 > 1 || m.act_bf16 > 1 || (m.act_bf16 && (m.experts || m.kv_int8 || m.mtp)) ||
      (m.experts && (m.experts < 16 || m.experts > 256 || (m.experts & (m.experts - 1)) || m.top_k < 1 ||
                     m.top_k > 8 || m.moe_inter % 128 || m.moe_inter == 0 || m.moe_inter > 1024 ||
                     m.hidden % 512 || m.hidden > 4096))) {
    mi_fail(MI_ERR_SHAPE, "engine_create: unsupported model shape");
    return nullptr;
  }
  std::unique_ptr<mi_engine> e(new (std::nothrow) mi_engine);
  if (!e) {
    mi_fail(MI_ERR_OOM, "engine_create: out of host memory");
    return nullptr;
  }
  e->d = m;
  if (stream) {
    e->stream = static_cast<hipStream_t>(stream);
  } else {
    if (hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking) != hipSuccess) {
      mi_fail(MI_ERR_STATE, "engine_create: stream");
      return nullptr;
    }
    e->own_stream = true;
  }
  if (e->build(seed) != 0) return nullptr;
  return e.release();
}

void mi_engine_destroy(mi_engine* e) { delete e; }

void* mi_engine_stream(mi_engine* e) { return e ? e->stream : nullptr; }

bool mi_engine_has_mtp(const mi_engine* e) { return e && e->d.mtp; }
bool mi_engine_act_bf16(const mi_engine* e) { return e && e->d.act_bf16; }

int mi_engine_tensor(mi_engine* e, uint32_t kind, uint32_t layer, void** ptr, size_t* bytes) {
  if (!e || !ptr) return mi_fail(MI_ERR_ARG, "engine_tensor: null");
  const mi_model_desc& m = e->d;
  // per-layer kinds at layer == layers: the MTP head's layer
  if (kind < MI_T_EMBED && layer >= m.layers + (m.mtp ? 1u : 0u))
    return mi_fail(MI_ERR_ARG, "engine_tensor: layer out of range");
  if (kind >= MI_T_MTP_FC_Q && kind <= MI_T_MTP_LOGITS && !m.mtp)
    return mi_fail(MI_ERR_ARG, "engine_tensor: the model has no MTP head");
  const Layer* L = kind < MI_T_EMBED ? (layer == m.layers ? &e->mh.L : &e->layer[layer]) : nullptr;
  const size_t hkvb = size_t(m.kv_heads) * m.max_len * m.head_dim * 2;
  auto lin_q = [](const Linear& l, void** p, size_t* b) { *p = l.q; if (b) *b = size_t(l.K / 8) * l.N * 4; };
  auto lin_s = [](const Linear& l, void** p, size_t* b) { *p = l.s; if (b) *b = size_t(l.K / 64) * l.N * 2; };
  size_t b = 0;
  const size_t kvb = size_t(m.layers) * m.kv_heads * m.max_len * m.head_dim * (m.kv_int8 ? 1 : 2);
  const size_t kvsb = m.kv_int8 ? size_t(m.layers) * m.kv_heads * m.max_len * 2 : 0;
  switch (kind) {
    case MI_T_QKV_Q: lin_q(L->qkv, ptr, &b); break;
    case MI_T_QKV_S: lin_s(L->qkv, ptr, &b); break;
    case MI_T_O_Q: lin_q(L->o, ptr, &b); break;
    case MI_T_O_S: lin_s(L->o, ptr, &b); break;
    case MI_T_GU_Q: lin_q(L->gate_up, ptr, &b); break;
    case MI_T_GU_S: lin_s(L->gate_up, ptr, &b); break;
    case MI_T_DOWN_Q: lin_q(L->down, ptr, &b); break;
    case MI_T_DOWN_S: lin_s(L->down, ptr, &b); break;
    case MI_T_IN_NORM: *ptr = L->in_norm; b = size_t(m.hidden) * 4; break;
    case MI_T_POST_NORM: *ptr = L->post_norm; b = size_t(m.hidden) * 4; break;
    case MI_T_Q_NORM: *ptr = L->q_norm; b = L->q_norm ? size_t(m.head_dim) * 4 : 0; break;
    case MI_T_K_NORM: *ptr = L->k_norm; b = L->k_norm ? size_t(m.head_dim) * 4 : 0; break;
    case MI_T_ROUTER: *ptr = L->router; b = L->router ? size_t(e->router_n) * m.hidden * 2 : 0; break;
    case MI_T_MOE_GU: *ptr = L->moe_gu; b = L->moe_gu ? (m.experts + 1) * e->gu_block * 4 : 0; break;
    case MI_T_MOE_DN: *ptr = L->moe_dn; b = L->moe_dn ? (m.experts + 1) * e->dn_block * 4 : 0; break;
    case MI_T_EMBED: *ptr = e->embed; b = size_t(m.vocab) * m.hidden * 2; break;
    case MI_T_FINAL_NORM: *ptr = e->final_norm; b = size_t(m.hidden) * 4; break;
    case MI_T_LM_Q: lin_q(e->lm_head, ptr, &b); break;
    case MI_T_LM_S: lin_s(e->lm_head, ptr, &b); break;
    case MI_T_ROPE: *ptr = e->rope; b = size_t(m.max_len) * m.rot_dim * 4; break;
    case MI_T_KV_K: *ptr = e->kv_k; b = kvb; break;
    case MI_T_KV_V: *ptr = e->kv_v; b = kvb; break;
    case MI_T_LOGITS: *ptr = e->logits; b = size_t(m.max_rows) * m.vocab * 4; break;
    case MI_T_CTRL: *ptr = e->ctrl; b = MI_CTRL_WORDS * 4; break;
    case MI_T_HISTORY: *ptr = e->history; b = size_t(m.max_len) * 4; break;
    case MI_T_KV_KS: *ptr = e->kv_ks; b = kvsb; break;
    case MI_T_KV_VS: *ptr = e->kv_vs; b = kvsb; break;
    case MI_T_RESID: *ptr = e->resid; b = size_t(m.max_rows) * m.hidden * 2; break;
    case MI_T_X: *ptr = e->x; b = size_t(m.max_rows) * std::max(m.hidden, m.q_heads * m.head_dim) * 2; break;
    case MI_T_ATTN_Q: *ptr = e->attn_q; b = size_t(m.max_rows) * m.q_heads * m.head_dim * 4; break;
    case MI_T_ATTN_OUT: *ptr = e->attn_out; b = size_t(m.max_rows) * m.q_heads * m.head_dim * 2; break;
    case MI_T_HBUF: *ptr = e->hbuf; b = size_t(m.max_rows) * m.inter * 2; break;
    case MI_T_MTP_FC_Q: lin_q(e->mh.fc, ptr, &b); break;
    case MI_T_MTP_FC_S: lin_s(e->mh.fc, ptr, &b); break;
    case MI_T_MTP_PRE_E: *ptr = e->mh.pre_e; b = size_t(m.hidden) * 4; break;
    case MI_T_MTP_PRE_H: *ptr = e->mh.pre_h; b = size_t(m.hidden) * 4; break;
    case MI_T_MTP_FINAL: *ptr = e->mh.final_n; b = size_t(m.hidden) * 4; break;
    case MI_T_MTP_KV_K: *ptr = e->hkv_k; b = hkvb; break;
    case MI_T_MTP_KV_V: *ptr = e->hkv_v; b = hkvb; break;
    case MI_T_MTP_HH: *ptr = e->hh; b = size_t(m.max_rows + 1) * m.hidden * 2; break;
    case MI_T_MTP_DH: *ptr = e->dh; b = size_t(m.hidden) * 2; break;
    case MI_T_MTP_CTRL: *ptr = e->hctl; b = MI_CTRL_WORDS * 4; break;
    case MI_T_MTP_LOGITS: *ptr = e->hlogits; b = size_t(m.vocab) * 4; break;
    case MI_T_LM_I8: *ptr = e->lm_i8; b = e->lm_i8 ? size_t(m.vocab) * m.hidden : 0; break;
    case MI_T_LM_I8_S: *ptr = e->lm_i8s; b = e->lm_i8s ? size_t(m.vocab) * 4 : 0; break;
    case MI_T_MTP_W16_FC: *ptr = e->mh.fc16; b = e->mh.fc16 ? size_t(2 * m.hidden) * m.hidden * 2 : 0; break;
    case MI_T_MTP_W16_QKV:
      *ptr = e->mh.qkv16;
      b = e->mh.qkv16 ? size_t(m.hidden) * (m.q_heads + 2 * m.kv_heads) * m.head_dim * 2 : 0;
      break;
    case MI_T_MTP_W16_O: *ptr = e->mh.o16; b = e->mh.o16 ? size_t(m.q_heads) * m.head_dim * m.hidden * 2 : 0; break;
    case MI_T_MTP_W16_GU: *ptr = e->mh.gu16; b = e->mh.gu16 ? size_t(m.hidden) * 2 * m.inter * 2 : 0; break;
    case MI_T_MTP_W16_DN: *ptr = e->mh.dn16; b = e->mh.dn16 ? size_t(m.inter) * m.hidden * 2 : 0; break;
    case MI_T_MOE_HANDOFF: *ptr = e->dn_words; b = e->dn_words ? size_t(std::min(m.max_rows, kRowChunk)) * (m.hidden / 2) * 4 : 0; break;
    default: return mi_fail(MI_ERR_ARG, "engine_tensor: unknown kind");
  }
  if (bytes) *bytes = b;
  return 0;
}

int mi_engine_linear_s(mi_engine* e, uint32_t which, uint32_t* S) {
  if (!e || !S) return mi_fail(MI_ERR_ARG, "engine_linear_s: null");
  const Layer& L = e->layer[0];
  switch (which) {
    case 0: *S = L.qkv.S; break;
    case 1: *S = L.o.S; break;
    case 2: *S = L.gate_up.q ? L.gate_up.S : 0; break;  // 0: a MoE model has no dense MLP
    case 3: *S = L.down.q ? L.down.S : 0; break;
    case 4: *S = e->lm_head.S; break;
    case 5: *S = e->mh.fc.q ? e->mh.fc.S : 0; break;  // the MTP head's fc (0: no head)
    default: return mi_fail(MI_ERR_ARG, "engine_linear_s: which 0..5");
  }
  return 0;
}

int mi_engine_capture(mi_engine* e, uint32_t M) {
  if (!e || M == 0 || M > e->d.max_rows) return mi_fail(MI_ERR_ARG, "engine_capture: M out of range");
  return e->capture(M);
}

int mi_engine_reset(mi_engine* e, uint32_t pos, uint32_t token) {
  if (!e) return mi_fail(MI_ERR_ARG, "engine_reset: null");
  if (pos >= e->d.max_len) return mi_fail(MI_ERR_ARG, "engine_reset: pos beyond the KV cache");
  MI_TRY(mi_hip(static_cast<int>(hipMemsetAsync(e->ctrl, 0, MI_CTRL_WORDS * 4, e->stream)), "ctrl clear"));
  return e->set_rows(pos, 1, &token, 1);
}

int mi_engine_replay(mi_engine* e, uint32_t M) {
  if (!e || M == 0 || M > e->d.max_rows || !e->graphs[M]) return mi_fail(MI_ERR_STATE, "engine_replay: not captured");
  return mi_hip(static_cast<int>(hipGraphLaunch(e->graphs[M], e->stream)), "hipGraphLaunch");
}

// The same step enqueued kernel by kernel, without the graph (for tools that trace kernel
// launches, and for comparing against the graph replay).
int mi_engine_step_eager(mi_engine* e, uint32_t M) {
  if (!e || M == 0 || M > e->d.max_rows) return mi_fail(MI_ERR_ARG, "engine_step_eager: M out of range");
  return e->enqueue_step(M);
}

int mi_engine_generate(mi_engine* e, uint32_t n, uint32_t* tokens) {
  if (!e || !e->graphs[1]) return mi_fail(MI_ERR_STATE, "engine_generate: capture(1) first");
  uint32_t c[MI_CTRL_WORDS];
  MI_TRY(e->read_ctrl(c));
  if (c[MI_CTRL_POS] + n > e->d.max_len) return mi_fail(MI_ERR_ARG, "engine_generate: past the KV cache");
  if (c[MI_CTRL_NACT] != 1) return mi_fail(MI_ERR_STATE, "engine_generate: n_active must be 1");
  const uint32_t first = c[MI_CTRL_STEPS];
  for (uint32_t i = 0; i < n; ++i) MI_TRY(mi_engine_replay(e, 1));
  if (tokens) MI_TRY(mi_memcpy_d2h(tokens, e->history + first, size_t(n) * 4, e->stream));
  MI_TRY(mi_stream_sync(e->stream));
  return e->check_handoff();
}

int mi_engine_ingest(mi_engine* e, const uint32_t* ids, uint32_t n) {
  if (!e || !e->graphs[1]) return mi_fail(MI_ERR_STATE, "engine_ingest: capture(1) first");
  uint32_t c[MI_CTRL_WORDS];
  MI_TRY(e->read_ctrl(c));
  if (c[MI_CTRL_POS] + n > e->d.max_len) return mi_fail(MI_ERR_ARG, "engine_ingest: past the KV cache");
  for (uint32_t i = 0; i < n; ++i) {
    ctrl_set_kernel<<<1, 64, 0, e->stream>>>(e->ctrl, MI_CTRL_CUR, ids[i]);
    MI_TRY(mi_hip(static_cast<int>(hipGetLastError()), "ctrl_set"));
    MI_TRY(mi_engine_replay(e, 1));
  }
  MI_TRY(mi_stream_sync(e->stream));
  return e->check_handoff();
}

int mi_engine_prefill(mi_engine* e, const uint32_t* ids, uint32_t n, uint32_t chunk) {
  if (!e) return mi_fail(MI_ERR_ARG, "engine_prefill: null");
  MI_TRY(e->prefill(ids, n, chunk));
  return e->check_handoff();  // the last position's logits: a non-finite one fails the call
}

int mi_engine_bench_linear(mi_engine* e, uint32_t which, uint32_t reps, float* ms_per_launch) {
  if (!e) return mi_fail(MI_ERR_ARG, "engine_bench_linear: null");
  return e->bench_linear(which, reps, ms_per_launch);
}

int mi_engine_bench_verify(mi_engine* e, uint32_t rows_mode, uint32_t reps, float* ms_per_step) {
  if (!e) return mi_fail(MI_ERR_ARG, "engine_bench_verify: null");
  return e->bench_verify(rows_mode, reps, ms_per_step);
}

int mi_engine_read_ctrl(mi_engine* e, uint32_t* out) {
  if (!e || !out) return mi_fail(MI_ERR_ARG, "engine_read_ctrl: null");
  return e->read_ctrl(out);
}

// Engine::verify (engine.cc:868-926): rows = [cur_token, drafts...] at pos .. pos+k.
int mi_engine_verify(mi_engine* e, const uint32_t* drafts, uint32_t k, uint32_t* argmax_rows) {
  if (!e || (k && !drafts) || k + 1 > e->d.max_rows) return mi_fail(MI_ERR_ARG, "engine_verify: bad k");
  if (!e->graphs[k + 1]) MI_TRY(e->capture(k + 1));
  uint32_t c[MI_CTRL_WORDS];
  MI_TRY(e->read_ctrl(c));
  if (c[MI_CTRL_POS] + k + 1 > e->d.max_len) return mi_fail(MI_ERR_ARG, "engine_verify: past the KV cache");
  if (e->d.mtp && k && c[MI_CTRL_POS] == 0)
    return mi_fail(MI_ERR_ARG, "engine_verify: with the MTP head, drafts need pos >= 1 (engine.h:277)");
  std::vector<uint32_t> ids(k + 1);
  ids[0] = c[MI_CTRL_CUR];
  for (uint32_t i = 0; i < k; ++i) ids[i + 1] = drafts[i];
  MI_TRY(e->set_rows(c[MI_CTRL_POS], k + 1, ids.data(), k + 1));
  MI_TRY(mi_engine_replay(e, k + 1));
  uint32_t c2[MI_CTRL_WORDS];
  MI_TRY(e->read_ctrl(c2));
  MI_TRY(e->check_handoff());
  if (argmax_rows) std::memcpy(argmax_rows, c2 + ctrl_out_at(k + 1), (k + 1) * 4);
  // leave pos at the verify position until commit (Engine::commit decides the advance)
  return e->set_rows(c[MI_CTRL_POS], 1, nullptr, 0);
}

// Engine::commit (engine.cc:927-960): j accepted drafts, next token = argmax row j.
int mi_engine_commit(mi_engine* e, uint32_t verify_pos, uint32_t j, uint32_t next) {
  if (!e) return mi_fail(MI_ERR_ARG, "engine_commit: null");
  if (e->d.mtp) {  // the accepted row's hidden becomes h_{pos-1}
    if (j + 1 > e->d.max_rows) return mi_fail(MI_ERR_ARG, "engine_commit: j beyond the verify rows");
    const size_t row = size_t(e->d.hidden) * 2;
    MI_TRY(mi_hip(static_cast<int>(hipMemcpyAsync(e->hh, e->hh + size_t(j + 1) * e->d.hidden, row,
                                                  hipMemcpyDeviceToDevice, e->stream)), "hh commit"));
  }
  return e->set_rows(verify_pos + j + 1, 1, &next, 1);
}

int mi_engine_draft(mi_engine* e, uint32_t k, uint32_t* drafts) {
  if (!e) return mi_fail(MI_ERR_ARG, "engine_draft: null");
  return e->draft(k, drafts);
}

}  // extern "C"
