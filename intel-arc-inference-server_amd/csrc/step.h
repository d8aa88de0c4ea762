// step.h - host side of the persistent decode step (step.hip), used by the engine.
//
// The step of one row (M = 1) of a dense decoder with an f16 KV cache runs as ONE launch: a
// fixed list of work-items in dependency order (per layer: the qkv GEMV's split-K slices, the
// heads' q/k-norm + RoPE + KV write, the attention blocks, the heads' block merge, the o / gate||up
// / down slices with their consumers; then the head GEMV and the argmax), dealt round-robin to
// as many work-groups as the GPU holds at once. Every value a work-item hands to another goes
// through hand-off words (gemv_core.h: the empty pattern), so no launch boundary separates the
// stages and a work-group streams the weights of its next slice while it waits for its inputs.
// Every arithmetic operation is the launch path's, in the same order: the step's logits, KV rows
// and control block are bitwise those of the captured graph of single launches.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {

struct StepLinear {
  const uint32_t* q;
  const uint16_t* s;
  uint32_t K, N, S;
};

struct StepLayerW {
  StepLinear qkv, o, gate_up, down;
  const float* in_norm;
  const float* post_norm;
  const float* q_norm;  // NULL: no q/k RMSNorm
  const float* k_norm;
};

struct StepModel {
  uint32_t layers, hidden, inter, q_heads, kv_heads, head_dim, rot_dim, vocab, vocab_used, max_len, tgt;
  float eps;                 // every RMSNorm's epsilon
  const StepLayerW* layer;   // host array [layers]
  const uint16_t* embed;
  const float* final_norm;
  StepLinear lm_head;
  const float* rope;         // [max_len][2][rot_dim / 2]
  uint16_t* kv_k;            // [layers][kv_heads][max_len][head_dim] f16
  uint16_t* kv_v;
  uint32_t* ctrl;
  uint32_t* history;
  float* logits;             // [vocab]
};

struct StepPlan;

// Checks the shape, allocates and empties the hand-off words and uploads the work-item list.
// Returns MI_ERR_SHAPE for a model the persistent step does not serve (the caller keeps the
// graph of launches for it).
int step_plan_create(const StepModel& m, hipStream_t st, StepPlan** out);
// One decode step of row 0 (ctrl[NACT] must be 1), enqueued on `st`.
int step_plan_launch(StepPlan* p, hipStream_t st);
// Every hand-off word back to empty (after a step whose wait timed out).
int step_plan_reset(StepPlan* p, hipStream_t st);
void step_plan_destroy(StepPlan* p);
// work-groups per launch and work-items per step
uint32_t step_plan_wgs(const StepPlan* p);
uint32_t step_plan_items(const StepPlan* p);
// diagnostics: what = 0 the device work-item table, 1 the hand-off arena (NULL, 0 without a plan)
void step_plan_debug(const StepPlan* p, uint32_t what, void** ptr, size_t* bytes);

}  // namespace mi
