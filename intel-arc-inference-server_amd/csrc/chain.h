// chain.h - host side of the layer chain launch (chain.hip), used by the engine.
//
// One launch per dense layer runs the layer's o GEMV with the residual fold and the
// post-attention norm, gate||up with SwiGLU, down with the residual fold and the next norm, and
// (when a layer follows) that layer's q||k||v with attn_prep: the single-row step becomes
// embed + norm, layer 0's q||k||v, then per layer the attention pair and one chain launch, then
// the head. Every arithmetic operation is the launch-per-linear graph's, in the same order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {

struct ChainLinear {
  const uint32_t* q;
  const uint16_t* s;
  uint32_t K, N, S;
};

struct ChainLayer {
  ChainLinear qkv, o, gate_up, down;
  const float* in_norm;
  const float* post_norm;
  const float* q_norm;  // NULL: no q/k RMSNorm
  const float* k_norm;
};

struct ChainModel {
  uint32_t layers, hidden, inter, q_heads, kv_heads, head_dim, rot_dim, max_len, act;
  float eps;                  // every RMSNorm's epsilon
  const ChainLayer* layer;    // host array [layers]
  const float* final_norm;
  const float* rope;          // [max_len][2][rot_dim / 2]
  uint16_t* kv_k;             // [layers][kv_heads][max_len][head_dim] f16
  uint16_t* kv_v;
  uint32_t* ctrl;
  uint32_t* status;           // set to the timeout code when a wait gives up
  uint16_t* resid;            // the residual stream [hidden] between launches
  uint16_t* x;                // the final norm's output [hidden] (the head's input)
  const uint16_t* attn_out;   // the attention output [q_heads head_dim] (the o GEMV's input)
  float* attn_q;              // [q_heads][head_dim] (attn_prep's q, for the next attention)
};

struct ChainPlan;

// Checks the shape, allocates and empties the hand-off words, builds every layer's item list.
// MI_ERR_SHAPE for a model the chain does not serve (the caller keeps the graph of launches).
int chain_plan_create(const ChainModel& m, hipStream_t st, ChainPlan** out);
// Layer `layer`'s chain launch (row 0; ctrl's n_active must be 1), enqueued on `st`.
int chain_launch(const ChainPlan* p, uint32_t layer, hipStream_t st);
// After the last layer's launch: empties the many-reader words that launch used.
int chain_finish(const ChainPlan* p, hipStream_t st);
// Every hand-off word back to empty (after a launch whose wait timed out).
int chain_reset(const ChainPlan* p, hipStream_t st);
void chain_destroy(ChainPlan* p);
uint32_t chain_wgs(const ChainPlan* p);
// diagnostics: the per-item trace (MI_CHAIN_TRACE set when the plan is built; NULL, 0 otherwise)
void chain_debug(const ChainPlan* p, void** ptr, size_t* bytes);

}  // namespace mi
