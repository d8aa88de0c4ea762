// gemv_w4a16.hip - the W4A16 GPTQ group-64 linear for M = 1..16 rows on gfx950.
//
// Replaces the reference's `gemv` (src/kernels/gemv.cl:124-221) and, for M >= 2, its
// small-M `gemm_sm` (src/kernels/gemm_sm.cl:161): same operands and the same output
// contract - fp32 split-K partials [S][M][N] that the consumer folds in slice order
// (tests/kernels/gemm_sm_ref.h:106-136) - with an MI355X-native inner loop.
//
// Weights stay in GPTQ layout 0 (qweight u32 [K/8][N], nibble i of word (r, n) is
// k = 8r + i; scales f16 [K/64][N]; zero point 8), which already streams coalesced:
//
//   * A work-group is 4 wave64s on one 64-column tile; grid (N / 64, S). Slice s owns
//     k-groups [s G/S, (s+1) G/S); wave w takes every 4th of them.
//   * Lane l reads one 16-byte uint4 = 4 adjacent columns (n0 + 4 (l % 16) .. + 3) of word
//     row (l / 16) of a 4-row quarter group: each 16-lane quarter-wave reads 256 contiguous
//     bytes, the wave 1 KB, with non-temporal loads (weights are read once per token).
//   * The contraction runs on the matrix cores: v_mfma_f32_16x16x32_f16 with A = the M
//     activation rows (zero-padded to 16) and B = 32 k x 16 columns of dequantised
//     weights. Lane l's B operand is exactly its word: 8 consecutive k of one column, so
//     the dequant is register-local - two v_and_or_b32 of the word (and of word >> 8)
//     against the fp16 magic 0x6400 give (1024 + q) or (1024 + 16 q) in each half, and
//     one packed f16 add / fma takes them to q - 8 exactly. The halves come out paired
//     (k0,k4)(k1,k5)(k2,k6)(k3,k7); the activation octet is permuted the same way
//     (v_perm_b32), so the MFMA sums the right products.
//   * Per k-group the 16x16 fp32 tile starts from zero, then acc = fma(tile, scale, acc)
//     per column (the reference's acc += gacc * scale per group); the 4 waves' partials
//     are summed in wave order through LDS and written as one slice.
//
// Property R (gemm_sm.cl:36-41): row m's result does not depend on M or on the other
// rows - every output element is its own MFMA dot and the same fixed merges - so S and
// the wave split are functions of the shape only (mi_gemv_pick_s).
//
// Fused epilogues (mi_gemv_w4a16_ex). One work-group per 64-column tile is its consumer: it
// folds the tile's S partials in ascending s (the consumer's fold of gemv.cl:1-10) and applies
// the step's next operation:
//   RESID   resid = rne(resid + rne(sum_s part)) and the tile's sum of squares (the
//           reference's res_fold at 64-element chunks, prep_ref.h:120-156); every consumer
//           then sums all tiles' sums in ascending tile order, forms rstd = 1/sqrt(sum / N +
//           eps) and writes its own tile of the next RMSNorm's x = rne(r * rstd * w)
//           (norm_finish, prep_ref.h:158-168);
//   SILU    h = rne(rne(silu(rne(g))) * rne(u)) over the interleave16 gate||up columns
//           (prep_silu_mul, prep_ref.h:170-189);
//   LOGITS  fp32 logits and the tile's (max, lowest index) for argmax_stage2
//           (argmax.cl:63-65's comparator; the vocab_used mask);
//   F16OUT  the fold rounded to fp16.
// Hand-off words: the partials (and RESID's per-consumer copies of the tile sums) hold the
// empty pattern 0xFFFFFFFF between launches - a NaN that fp32 arithmetic on fp16 data never
// produces (a computed value with those bits is stored as the canonical NaN). Producers store
// with device-coherent (sc1) single-word stores; a consumer polls each word with
// device-coherent loads until it is not empty, then writes the empty pattern back, so every
// launch leaves the words as it found them. A polled word is either empty or final, so no
// ordering between words is needed.
// Who consumes. With an arrival array (epi.arrive, zero between launches) every slice
// publishes its partial and then counts itself in with one atomic add on its tile's word
// (QKV: its head's word); the work-group that arrives last is the consumer and sets the word
// back to zero. No work-group waits for another one that may not have started, whatever the
// dispatch order: the consumer's polls only cover words already stored (or about to land).
// Without it, slice S-1 of each tile is the consumer and keeps its own slice in LDS: each XCD
// dispatches its share of the grid in linear order and the consumers are the grid's last row,
// so every producer is resident or done before a consumer on its XCD waits. Either way
// RESID's consumers also wait on each other, which needs all N/64 of them resident at once
// (N <= 16384: at most 256 work-groups). A bounded poll ends a wait that never completes
// with the empty NaN in the result instead of a hang.
// No float atomics: replays stay bitwise identical.
#include <algorithm>

#include "mi_common.h"
#include "mi_capi_internal.h"
#include "gemv_core.h"

namespace mi {
namespace {

// RESID's fixed consumers as an extra grid row with no slice of their own (as QKV's):
// dispatched after every slice, they poll at once instead of first streaming a slice of their
// own (measured on MI355X at the 27B shapes: o 9.8 -> 9.5 us, down 15.8 -> 15.2 us; SILU's
// 544 consumers gain nothing that way and keep slice S-1).
#ifndef MI_GEMV_EXTRA_ROW
#define MI_GEMV_EXTRA_ROW 1
#endif
constexpr bool kExtraRow = MI_GEMV_EXTRA_ROW != 0;
constexpr int kWaves = 4;
constexpr int kCols = 64;

struct GemvEpi {
  uint16_t* resid;        // RESID: [M][N]
  float* sumsq;           // RESID: [N/64][M][N/64], empty between launches
  float* rstd;            // RESID: [M]
  const float* next_w;    // RESID: the next RMSNorm's fp32 weights [N]
  uint16_t* x_next;       // RESID: [M][N]
  uint16_t* h;            // SILU: [M][N/2]
  float* out32;           // LOGITS: [M][N]
  u2_t* argmax_part;      // LOGITS: [M][N/64] (value bits, index), or NULL
  uint32_t vocab_used;    // LOGITS
  float eps;              // RESID
  uint16_t* out16;        // F16OUT: [M][N]
  // QKV: attn_prep's chain on the folded q||k||v row (f16 cache, not gated)
  uint32_t* ctrl;
  const float* rope;
  const float* q_norm;
  const float* k_norm;
  float* attn_q;
  uint16_t* kv_k;
  uint16_t* kv_v;
  const uint32_t* pages;
  size_t row_stride, head_stride;
  uint32_t page, kv_len, q_heads, kv_heads, head_dim, rot_dim;
  float qk_eps;
  // a device word set to kStatusTimeout when a hand-off wait gives up (NULL: none)
  uint32_t* status;
  uint32_t poll_limit;  // polls of one word before giving up
  uint32_t inject;      // fault injection for tests: bit 0 = producers publish nothing
  uint32_t extra_row;   // set by the launch: the fixed consumers are an extra grid row
  uint32_t* arrive;     // per-tile (QKV: per-head) arrival counts, zero between launches; NULL:
                        // the fixed consumers (slice S-1; QKV's extra row)
  uint32_t act;         // 0: f16 activations; 1: bf16 (roundings to bf16, residual in bf16 bits)
  // the norm split across two launches: RESID with sums_out writes the residual and its tiles'
  // sums of squares [M][N/64] only; a launch with in_sums ([M][K/64]) reads x as that residual
  // and forms rne(x * rstd * in_norm_w) itself
  float* sums_out;
  const float* in_sums;
  const float* in_norm_w;
  float in_eps;
  uint32_t row_cons;  // set by the launch: RESID's extra consumers are one grid row per row m
};

// arrival words sit 128 bytes apart: no two tiles' counts share a cache line
constexpr uint32_t kArriveStride = 32;

// One atomic add on an arrival word by thread 0 after the work-group's partial stores; true
// (uniform) in the work-group that completes the count `need`, which sets the word back to 0.
__device__ __forceinline__ bool arrive_last(uint32_t* word, uint32_t need, uint32_t* s_flag) {
  lds_barrier();  // every thread's partial stores are issued (not waited for)
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(word, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old + 1u == need;
    if (last) __hip_atomic_store(word, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last;
  }
  lds_barrier();
  return *s_flag != 0u;
}

enum { EPI_PARTIALS = 0, EPI_RESID = 1, EPI_SILU = 2, EPI_LOGITS = 3, EPI_F16OUT = 4, EPI_QKV = 5 };

// argmax.cl:63-65: strictly greater wins, an exact tie keeps the lower index
__device__ __forceinline__ bool better(float av, uint32_t ai, float bv, uint32_t bi) {
  return (av > bv) || (av == bv && ai < bi);
}

// LDS words a consumer polls per round: a single-row RESID consumer takes 36 slices (the 27B
// down's S = 34 folds in one round trip; measured 15.1 -> 14.8 us), 2048 words otherwise
template <int MR, int EPI>
constexpr int fold_buf() { return MR == 1 && EPI == EPI_RESID ? 2304 : 2048; }
constexpr int kFoldBuf_QKV = 2048;
constexpr uint32_t kPollLimit = 1u << 21; // polls of one word before giving up (~seconds)

// dst[e] = the hand-off word of element e < cnt (cnt <= BUF) once it is not empty; then the
// word is emptied again. Element e = t + 256 u (t = threadIdx.x) sits at byte offset
// voff + u * ustride from base: buffer accesses with a per-thread 32-bit offset and a uniform
// one per u keep the addresses out of 64-bit registers. sc1 makes them the device-coherent
// accesses of ld_agent / st_agent. The whole work-group calls this; dst is LDS.
// A wait that reaches `limit` polls gives up: the words still empty are taken as they are
// (the empty NaN) and `status` (when not NULL) is set to kStatusTimeout, so the host learns
// that this launch's output is not to be used.
template <int BUF>
__device__ __forceinline__ void poll_into(float* dst, uint32_t cnt, float* base, uint32_t voff,
                                          uint32_t ustride, uint32_t* status, uint32_t limit) {
  constexpr int PER = BUF / 256;
  constexpr int kSc1 = 16;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(base, 0, 0x7FFFFFFF, 0x00020000);
  const uint32_t t = threadIdx.x;
  // Every load is issued unconditionally: an element past cnt (or, re-polling, one already
  // read) takes an offset past the resource's range, which the buffer unit answers with 0 and
  // no memory access. (A load under a branch leaves its value in a register that the branch's
  // join copies, and the copy waits for that load at once: one round trip per word.)
  constexpr uint32_t kOob = 0x80000000u;
  uint32_t v[PER];
  uint32_t pending = 0;  // bit u: element t + 256 u still empty
#pragma unroll
  for (int u = 0; u < PER; ++u)
    v[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, t + 256u * u < cnt ? voff + u * ustride : kOob, 0, kSc1);
  __builtin_amdgcn_sched_barrier(0);  // (all of them before the first use)
#pragma unroll
  for (int u = 0; u < PER; ++u)
    if (t + 256u * u < cnt && v[u] == kEmpty) pending |= 1u << u;
  // re-poll every still-empty word together, so a wait costs one round trip per poll, not per word
  for (uint32_t n = 0; pending && n < limit; ++n) {
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const bool p = pending & (1u << u);
      const uint32_t nv = __builtin_amdgcn_raw_buffer_load_b32(rs, p ? voff + u * ustride : kOob, 0, kSc1);
      v[u] = p ? nv : v[u];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < PER; ++u)
      if ((pending & (1u << u)) && v[u] != kEmpty) pending &= ~(1u << u);
  }
  if (pending && status) st_agent(status, kStatusTimeout);
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const uint32_t e = t + 256u * u;
    if (e < cnt) {
      dst[e] = __builtin_bit_cast(float, v[u]);
      __builtin_amdgcn_raw_buffer_store_b32(kEmpty, rs, voff, u * ustride, kSc1);
    }
  }
}

// EPI_QKV's consumer: work-group (tile, S) of grid (N/64, S + 1), no slice of its own. The last
// tile of each head folds the head's HD columns over all S slices (ascending s from +0, as
// attn_prep's fold) and runs attn_prep's chain on them (prep.cl attn_prep, attn.cl:361-372):
// q/k rounded to f16, the per-head RMSNorm with the 256-lane tree's order, RoPE's
// rotate_half pairs, then q -> attn_q (fp32) and k, v -> the f16 cache row of position pos + m.
// One wave per row (M <= 4); lane l holds elements l + 64 k.
template <int HD>
__device__ __forceinline__ void qkv_consumer(const float* partials, uint32_t M, uint32_t N, uint32_t S,
                                             uint32_t tile, const GemvEpi& epi, float* s_fold) {
  constexpr uint32_t TPH = HD / 64u, EPL = HD / 64u;
  if ((tile + 1u) % TPH) return;  // uniform
  __shared__ float s_row[4][HD];
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t hh = tile / TPH, nh0 = (tile + 1u - TPH) * kCols;
  const uint32_t QH = epi.q_heads, KVH = epi.kv_heads;
  const bool is_q = hh < QH, is_k = !is_q && hh < QH + KVH;
  const uint32_t h = is_q ? hh : (is_k ? hh - QH : hh - QH - KVH);
  const uint32_t n_act = epi.ctrl[CTRL_NACT], pos = epi.ctrl[CTRL_POS];
  const uint32_t m = wave;
  const bool live = m < M && m < n_act;
  const bool past = live && epi.kv_len && pos + m >= epi.kv_len;
  // this wave's row: norm weights, RoPE pairs and the cache row go out before the fold
  const float* nw = is_q ? epi.q_norm : (is_k ? epi.k_norm : nullptr);
  const uint32_t half = epi.rot_dim / 2u;
  float wn[EPL], rc[EPL], rsn[EPL];
  size_t crow = 0;
  if (live && !past) {
    const float* cs = epi.rope + (size_t)(pos + m) * 2u * half;
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) {
      const uint32_t e = lane + 64u * k;
      wn[k] = nw ? nw[e] : 0.f;
      rc[k] = 1.f;
      rsn[k] = 0.f;
      if (!is_q && !is_k) continue;
      if (e < epi.rot_dim) {
        const uint32_t ii = e < half ? e : e - half;
        rc[k] = cs[ii];
        rsn[k] = cs[half + ii];
      }
    }
    if (!is_q) {
      const uint32_t p = pos + m;
      crow = epi.pages ? (size_t)epi.pages[p / epi.page] * epi.page + p % epi.page : (size_t)p;
    }
  }
  // the fold: element e of the head's M x HD block, e = t + 256 u (rows-slices e / HD)
  constexpr int EL = 4 * HD / 256;
  const uint32_t total = M * HD;
  const uint32_t per_round = kFoldBuf_QKV / total;
  float a[EL];
#pragma unroll
  for (int u = 0; u < EL; ++u) a[u] = 0.f;
  for (uint32_t s0 = 0; s0 < S; s0 += per_round) {
    const uint32_t ns = min(per_round, S - s0);
    poll_into<kFoldBuf_QKV>(s_fold, ns * total, const_cast<float*>(partials) + (size_t)s0 * M * N,
                            ((t / HD) * N + nh0 + t % HD) * 4u, (256u / HD) * N * 4u, epi.status,
                            epi.poll_limit);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < EL; ++u) {
      const uint32_t i = t + 256u * u;
      if (i < total)
        for (uint32_t j = 0; j < ns; ++j) a[u] += s_fold[j * total + i];
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < EL; ++u) {
    const uint32_t i = t + 256u * u;
    if (i < total) s_fold[i] = a[u];
  }
  __syncthreads();
  if (!live) return;  // uniform per wave; no barriers below
  if (past) {  // past the cache: write nothing, flag the step (attn_prep's rule)
    if (hh == 0 && lane == 0) epi.ctrl[CTRL_DEBUG] = 0xDEAD0002u;
    return;
  }
  const float* fr = s_fold + m * HD;
  if (!is_q && !is_k) {
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k)
      epi.kv_v[crow * epi.row_stride + h * epi.head_stride + lane + 64u * k] = act_enc(fr[lane + 64u * k], epi.act);
    return;
  }
  float xf[EPL], nv[EPL];
#pragma unroll
  for (uint32_t k = 0; k < EPL; ++k) xf[k] = act_round(fr[lane + 64u * k], epi.act);
  if (nw) {
    // tree_hd's order: the LDS steps (v[i] + v[i + st], st >= 64) are this lane's own
    // elements, then the 64-lane shuffle tree; lane 0's total is broadcast
    float sq[EPL];
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) sq[k] = xf[k] * xf[k];
    float acc;
    if constexpr (EPL == 4) acc = (sq[0] + sq[2]) + (sq[1] + sq[3]);
    else acc = sq[0] + sq[1];
#pragma unroll
    for (int st = 32; st > 0; st >>= 1) acc += __shfl_down(acc, st, 64);
    const float tot = __shfl(acc, 0, 64);
    const float rstd = 1.0f / sqrtf(tot / (float)HD + epi.qk_eps);
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) nv[k] = act_round(xf[k] * rstd * wn[k], epi.act);
  } else {
#pragma unroll
    for (uint32_t k = 0; k < EPL; ++k) nv[k] = xf[k];
  }
  float* nrm = s_row[wave];
#pragma unroll
  for (uint32_t k = 0; k < EPL; ++k) nrm[lane + 64u * k] = nv[k];
  wave_lds_sync();
#pragma unroll
  for (uint32_t k = 0; k < EPL; ++k) {
    const uint32_t e = lane + 64u * k;
    float out;
    if (e < half) {
      const float tt = nrm[e + half] * rsn[k];
      out = __builtin_fmaf(nv[k], rc[k], -tt);
    } else if (e < epi.rot_dim) {
      const float tt = nrm[e - half] * rsn[k];
      out = __builtin_fmaf(nv[k], rc[k], tt);
    } else {
      out = nv[k];
    }
    if (is_q)
      epi.attn_q[((size_t)m * QH + h) * HD + e] = out;
    else
      epi.kv_k[crow * epi.row_stride + h * epi.head_stride + e] = act_enc(out, epi.act);
  }
}

// sum_{g < n} p[g] from +0 in ascending g, p in LDS: the words read 32 / 16 / 4 at a time in
// 16-byte reads (p 16-byte aligned, n % 4 == 0), so the chain of adds waits on the LDS a few
// times rather than once per pair of words
__device__ __forceinline__ float lds_seq_sum(const float* p, uint32_t n) {
  float tot = 0.f;
  uint32_t g = 0;
  const f4_t* p4 = reinterpret_cast<const f4_t*>(p);
  auto add4 = [&](const f4_t& v) {
    tot += v[0];
    tot += v[1];
    tot += v[2];
    tot += v[3];
  };
  for (; g + 32u <= n; g += 32u) {
    f4_t v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = p4[g / 4u + j];
#pragma unroll
    for (int j = 0; j < 8; ++j) add4(v[j]);
  }
  if (g + 16u <= n) {
    f4_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = p4[g / 4u + j];
#pragma unroll
    for (int j = 0; j < 4; ++j) add4(v[j]);
    g += 16u;
  }
  for (; g < n; g += 4u) add4(p4[g / 4u]);
  return tot;
}

// MR: row capacity (1, 2, 3, 4 or 16); U: k-groups whose loads are issued together; EPI: epilogue;
// NI: the input is the RMSNorm of a residual, formed by each work-group for its slice (while
// its first weight loads are in flight): every row's rstd from the residual's tile sums, added in
// tile order from +0 as the RESID consumers add them, then rne((r * rstd) * w) per element -
// the RESID kind's x_next bit for bit - into LDS, where the slice reads it.
// The 16-row kernel with one k-group per wave asks for six waves per SIMD, which it meets in
// 80 VGPRs without spilling (27B verify at 8 rows 6.47 -> 6.42 ms; at 3 rows the same request
// measured slower).
template <int MR, int U, int EPI, bool NI = false>
__global__ __launch_bounds__(256, (MR == 16 && U == 1 ? 6 : 1)) void gemv_w4a16_kernel(const uint32_t* __restrict__ qweight,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ x,
                                                         float* __restrict__ partials, uint32_t M,
                                                         uint32_t K, uint32_t N, uint32_t gps,
                                                         GemvEpi epi) {
  constexpr int RR = MR < 4 ? MR : 4;  // accumulator rows a lane holds (rows 4*(l/16) + r)
  __shared__ float red[kWaves][MR][kCols];

  const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
  const uint32_t c4 = lane & 15u, q = lane >> 4;
  const uint32_t n0 = blockIdx.x * kCols;
  const uint32_t ncol = n0 + 4u * c4;
  const uint32_t s = blockIdx.y;
  const bool dyn = EPI != EPI_PARTIALS && epi.arrive != nullptr;  // last-arriver consumers
  const uint32_t g_begin = s * gps + wave;
  // QKV's fixed consumer row (s = S) has no slice of its own
  // an extra consumer row (QKV always; the others when epi.extra_row) has no slice of its own
  // RESID over several rows (row_cons): one consumer work-group per (tile, row), in grid rows
  // S_p .. S_p + M - 1 after the S_p producer rows
  const bool rowc = MR > 1 && EPI == EPI_RESID && epi.row_cons;
  const uint32_t S_p = (K / 64u) / gps;
  const bool xrow_c = (EPI == EPI_QKV || epi.extra_row) && !dyn && (rowc ? s >= S_p : s + 1 == gridDim.y);
  const uint32_t g_end = xrow_c ? 0u : (s + 1) * gps;
  const bool xrow = c4 < M;  // this lane feeds activation row c4 of the A operand

  const uint32_t m_lo = 0x000F000Fu, m_hi = 0x00F000F0u, magic = 0x64006400u;

  float acc[4][RR];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < RR; ++r) acc[c][r] = 0.f;

  u4_t wv[U][2];
  u2_t sv[U];
  auto load_w = [&](uint32_t g0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = g0 + u * kWaves;
      if (g < g_end) {
#pragma unroll
        for (int h = 0; h < 2; ++h) wv[u][h] = load_stream16(qweight + (size_t)(g * 8u + 4u * h + q) * N + ncol);
        sv[u] = *reinterpret_cast<const u2_t*>(scales + (size_t)g * N + ncol);
      }
    }
  };
  // NI: the slice's input rows, f16 pairs [M][gps * 32] (the tile sums pass through first)
  constexpr uint32_t XIN = NI ? (uint32_t)MR * 256u : 1u;
  __shared__ __align__(16) uint32_t s_xin[XIN];
  __shared__ __align__(16) float s_nsum[NI && MR == 1 ? 256 : 1];  // one row's tile sums
  if constexpr (NI) {
    if (!xrow_c) {  // uniform: the extra consumer row has no slice
      const uint32_t t = threadIdx.x, nt = K / 64u, kw = gps * 32u, nwords = M * kw;
      const uint32_t k0 = s * gps * 64u;
      float sm[MR];
      uint32_t rw[MR];
      float w0[MR], w1[MR];
      // the rows' rstd, when a work-group of this launch has already formed it: the words
      // after the sums (empty until then)
      const uint32_t* rcache = reinterpret_cast<const uint32_t*>(epi.in_sums) + M * nt;
      const uint32_t rc = ld_agent(rcache + (MR == 1 ? 0u : min(t, M - 1u)));
      // (every load unconditional, at a clamped index: a load under a branch leaves its value
      // in a register that the join copies, and the copy waits for the load at once)
#pragma unroll
      for (int u = 0; u < MR; ++u) {
        const uint32_t e = t + 256u * u;
        sm[u] = epi.in_sums[min(e, M * nt - 1u)];
        const uint32_t ec = min(e, nwords - 1u), row = ec / kw, k = k0 + 2u * (ec - row * kw);
        rw[u] = *reinterpret_cast<const uint32_t*>(x + (size_t)row * K + k);
        const f2_t w = *reinterpret_cast<const f2_t*>(epi.in_norm_w + k);
        w0[u] = w.x;
        w1[u] = w.y;
      }
      // then the first batch's weights: the waits for the loads above (retired in order) do
      // not wait for them
      // (unconditionally, a missing group re-reading the slice's last: a load under a branch
      // makes every later wait a wait for everything)
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t g = min(g_begin + u * kWaves, g_end - 1u);
#pragma unroll
        for (int h = 0; h < 2; ++h) wv[u][h] = load_stream16(qweight + (size_t)(g * 8u + 4u * h + q) * N + ncol);
        sv[u] = *reinterpret_cast<const u2_t*>(scales + (size_t)g * N + ncol);
      }
      // (unconditional too: the words past the M * nt sums are never read)
#pragma unroll
      for (int u = 0; u < MR; ++u) {
        if constexpr (MR == 1) s_nsum[t] = sm[u];
        else s_xin[t + 256u * u] = __builtin_bit_cast(uint32_t, sm[u]);
      }
      __syncthreads();
      // the rows' rstd: at one row every thread adds the sums itself (one broadcast LDS read
      // per word for a whole wave), so no barrier waits for one thread's chain of adds, and
      // the sums keep their own words; at more rows thread m adds row m's
      float rs1 = 0.f;
      __shared__ float s_rstd_in[MR];
      // (a pure function of the sums; the grid's first work-group stores it: stores from every
      // work-group to one word would queue behind each other for tens of microseconds)
      uint32_t* rcw = const_cast<uint32_t*>(rcache);
      const bool keeper = blockIdx.x == 0 && blockIdx.y == 0;
      if constexpr (MR == 1) {
        if (rc != kEmpty) {
          rs1 = __builtin_bit_cast(float, rc);
        } else {
          rs1 = 1.0f / sqrtf(lds_seq_sum(s_nsum, nt) / (float)K + epi.in_eps);
          if (keeper && t == 0) st_agent(rcw, __builtin_bit_cast(uint32_t, rs1));
        }
      } else {
        if (t < M) {
          float r;
          if (rc != kEmpty) {
            r = __builtin_bit_cast(float, rc);
          } else {
            const float* sp = reinterpret_cast<const float*>(s_xin) + t * nt;
            r = 1.0f / sqrtf(lds_seq_sum(sp, nt) / (float)K + epi.in_eps);
            if (keeper) st_agent(rcw + t, __builtin_bit_cast(uint32_t, r));
          }
          s_rstd_in[t] = r;
        }
        __syncthreads();  // (also: the sums' words are overwritten with x below)
      }
#pragma unroll
      for (int u = 0; u < MR; ++u) {
        const uint32_t e = t + 256u * u;
        if (e < nwords) {
          const float rs = MR == 1 ? rs1 : s_rstd_in[e / kw];
          const uint16_t x0 = act_enc(res_widen((uint16_t)(rw[u] & 0xFFFFu), epi.act) * rs * w0[u], epi.act);
          const uint16_t x1 = act_enc(res_widen((uint16_t)(rw[u] >> 16), epi.act) * rs * w1[u], epi.act);
          s_xin[e] = (uint32_t)x0 | ((uint32_t)x1 << 16);
        }
      }
      __syncthreads();
    }
  }

  for (uint32_t g0 = g_begin; g0 < g_end; g0 += kWaves * U) {
    if (!NI || g0 != g_begin) load_w(g0);
    u4_t xv[U][2];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = g0 + u * kWaves;
      if (g < g_end) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (!xrow)
            xv[u][h] = u4_t{0u, 0u, 0u, 0u};
          else if constexpr (NI)
            xv[u][h] = *reinterpret_cast<const u4_t*>(s_xin + c4 * (gps * 32u) + (g - s * gps) * 32u + 16u * h + 4u * q);
          else
            xv[u][h] = *reinterpret_cast<const u4_t*>(x + (size_t)c4 * K + g * 64u + 32u * h + 8u * q);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t g = g0 + u * kWaves;
      if (g < g_end) {
        f4_t d[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const h8_t a = perm_x(xv[u][h]);
          const uint32_t ws[4] = {wv[u][h].x, wv[u][h].y, wv[u][h].z, wv[u][h].w};
          h8_t bw[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) bw[c] = dequant_word(ws[c], m_lo, m_hi, magic);
#pragma unroll
          for (int c = 0; c < 4; ++c) d[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw[c], d[c], 0, 0, 0);
          keep_mfma_batch(a, bw, d);
        }
        const float sc[4] = {h2f((uint16_t)(sv[u].x & 0xFFFFu)), h2f((uint16_t)(sv[u].x >> 16)),
                             h2f((uint16_t)(sv[u].y & 0xFFFFu)), h2f((uint16_t)(sv[u].y >> 16))};
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int r = 0; r < RR; ++r) acc[c][r] = __builtin_fmaf(d[c][r], sc[c], acc[c][r]);
      }
    }
  }

  // Lane l holds rows 4 q + r of columns ncol .. ncol+3: stage them, then sum the waves.
#pragma unroll
  for (int r = 0; r < RR; ++r) {
    const uint32_t row = 4u * q + r;
    if (row < (uint32_t)MR) {
#pragma unroll
      for (int c = 0; c < 4; ++c) red[wave][row][4u * c4 + c] = acc[c][r];
    }
  }
  __syncthreads();
  __shared__ uint32_t s_last;
  __shared__ float s_qfold[EPI == EPI_QKV ? kFoldBuf_QKV : 1];
  if constexpr (EPI == EPI_QKV) {
    if (!dyn && s + 1 == gridDim.y) {  // the fixed consumer row (uniform)
      if (epi.head_dim == 128)
        qkv_consumer<128>(partials, M, N, gridDim.y - 1, blockIdx.x, epi, s_qfold);
      else
        qkv_consumer<256>(partials, M, N, gridDim.y - 1, blockIdx.x, epi, s_qfold);
      return;
    }
  }
  const uint32_t total = M * kCols;
  const uint32_t S = rowc ? S_p + 1u : gridDim.y, tile = blockIdx.x, ntiles = gridDim.x;
  const bool consumer = EPI != EPI_PARTIALS && EPI != EPI_QKV && !dyn && (rowc ? s >= S_p : s + 1 == S);
  // the rows a consumer folds and finishes: all M, or its own row
  const uint32_t r_lo = rowc ? s - S_p : 0u, r_n = rowc ? 1u : M, rs = rowc ? M : 1u;
  for (uint32_t i = threadIdx.x; i < total; i += 256u) {
    const uint32_t row = i / kCols, col = i % kCols;
    float v = red[0][row][col];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) v += red[w][row][col];
    if constexpr (EPI == EPI_PARTIALS)
      partials[((size_t)s * M + row) * N + n0 + col] = v;
    else if (consumer)
      red[0][row][col] = v;  // the consumer's own slice stays in LDS
    else if (!(epi.inject & 1u))
      st_agent(partials + ((size_t)s * M + row) * N + n0 + col, publishable(v));
  }
  if constexpr (EPI == EPI_QKV) {
    if (dyn) {  // the head's last arriving tile-slice runs the head's consumer
      const uint32_t tph = epi.head_dim / kCols, hh = tile / tph;
      if (arrive_last(epi.arrive + hh * kArriveStride, S * tph, &s_last)) {
        if (epi.head_dim == 128)
          qkv_consumer<128>(partials, M, N, S, hh * tph + tph - 1u, epi, s_qfold);
        else
          qkv_consumer<256>(partials, M, N, S, hh * tph + tph - 1u, epi, s_qfold);
      }
    }
    return;
  }
  if (dyn) {
    if (!arrive_last(epi.arrive + tile * kArriveStride, S, &s_last)) return;
  } else if (!consumer) {
    return;
  }
  // slices to poll: all of them, except the fixed consumer's own slice S-1 (kept in LDS)
  const bool own = !dyn && !epi.extra_row;
  const uint32_t npoll = own ? S - 1u : (dyn ? S : S - 1u);

  // ---- the tile's consumer folds the S partials and applies the epilogue ----
  // RESID: the residual and the next norm's weights for rows wave, wave + 4, ... (at most 4
  // of them) go out before the fold's round trips
  uint16_t r_pre[(MR + kWaves - 1) / kWaves];
  float w_pre = 0.f;
  if constexpr (EPI == EPI_RESID) {
#pragma unroll
    for (int k = 0; k < (MR + kWaves - 1) / kWaves; ++k) {
      const uint32_t row = r_lo + wave + kWaves * k;
      if (row < r_lo + r_n) r_pre[k] = epi.resid[(size_t)row * N + n0 + lane];
    }
    if (!epi.sums_out) w_pre = epi.next_w[n0 + lane];  // (the split form has no norm weights)
  }
  constexpr int kFoldBuf = fold_buf<MR, EPI>();
  __shared__ float s_fold[kFoldBuf];
  const uint32_t t = threadIdx.x;
  {
    // sum_s partials[s][row][n] from 0.f in ascending s, polled in rounds of `per_round`
    // slices (the fixed consumer's own slice S-1 is the last term, from red[0])
    // (thread t folds elements t + 256 u of the consumer's r_n x 64)
    constexpr int EL = MR * kCols / 256 > 0 ? MR * kCols / 256 : 1;
    const uint32_t ctot = r_n * kCols;
    const uint32_t per_round = kFoldBuf / ctot;
    float a[EL];
#pragma unroll
    for (int u = 0; u < EL; ++u) a[u] = 0.f;
    for (uint32_t s0 = 0; s0 < npoll; s0 += per_round) {
      const uint32_t ns = min(per_round, npoll - s0);
      // element e: row-slice e / 64 of slices s0.. (its row at e / 64 rows of rs apart from
      // row r_lo), column e % 64 (e / 64 = t / 64 + 4 u)
      poll_into<kFoldBuf>(s_fold, ns * ctot, partials + (size_t)s0 * M * N,
                          ((t / kCols) * rs * N + r_lo * N + n0 + t % kCols) * 4u, 4u * rs * N * 4u, epi.status,
                          epi.poll_limit);
      __syncthreads();
#pragma unroll
      for (int u = 0; u < EL; ++u) {
        const uint32_t i = t + 256u * u;
        if (i < ctot)
          for (uint32_t j = 0; j < ns; ++j) a[u] += s_fold[j * ctot + i];
      }
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < EL; ++u) {
      const uint32_t i = t + 256u * u;
      if (i < ctot) red[0][r_lo + i / kCols][i % kCols] = own ? a[u] + red[0][i / kCols][i % kCols] : a[u];
    }
    __syncthreads();
  }
  auto folded = [&](uint32_t row, uint32_t col) { return red[0][row][col]; };

  if constexpr (EPI == EPI_RESID) {
    // one row per wave per pass, a column per lane; the 64-lane tree is the reference's
    // 256-lane tree over a 64-element chunk (lanes 64..255 add exact zeros)
#pragma unroll
    for (int k = 0; k < (MR + kWaves - 1) / kWaves; ++k) {
      const uint32_t row = r_lo + wave + kWaves * k;
      if (row >= r_lo + r_n) break;
      const uint16_t rb = res_rne(res_widen(r_pre[k], epi.act) + act_round(folded(row, lane), epi.act), epi.act);
      epi.resid[(size_t)row * N + n0 + lane] = rb;
      const float v = res_widen(rb, epi.act);
      red[1][row][lane] = v;
      float a = __builtin_fmaf(v, v, 0.f);
#pragma unroll
      for (int st = 32; st > 0; st >>= 1) a += __shfl_down(a, st, 64);
      a = publishable(__shfl(a, 0, 64));
      if (epi.sums_out) {  // the next launch forms the norm
        if (lane == 0) epi.sums_out[(size_t)row * ntiles + tile] = a;
        continue;
      }
      // every consumer c gets its own copy: sumsq[c][row][tile]
      for (uint32_t c = lane; c < ntiles; c += 64u) st_agent(epi.sumsq + ((size_t)c * M + row) * ntiles + tile, a);
    }
    if (epi.sums_out) {  // uniform; the rstd words after the sums are empty again
      if (tile == 0 && t < r_n) reinterpret_cast<uint32_t*>(epi.sums_out)[(size_t)M * ntiles + r_lo + t] = kEmpty;
      return;
    }
    // all tiles' sums of this launch: sumsq[tile][row][g], g ascending, polled in rounds of rows
    __shared__ float s_rstd[16];
    const uint32_t rows_per_round = kFoldBuf / ntiles;
    for (uint32_t r0 = r_lo; r0 < r_lo + r_n; r0 += rows_per_round) {
      const uint32_t nr = min(rows_per_round, r_lo + r_n - r0);
      poll_into<kFoldBuf>(s_fold, nr * ntiles, epi.sumsq + ((size_t)tile * M + r0) * ntiles, t * 4u, 1024u,
                          epi.status, epi.poll_limit);
      __syncthreads();
      if (t < nr) {
        const float* ss = s_fold + t * ntiles;
        float tot = 0.f;
        for (uint32_t g = 0; g < ntiles; ++g) tot += ss[g];
        s_rstd[r0 + t] = 1.0f / sqrtf(tot / (float)N + epi.eps);
      }
      __syncthreads();
    }
    for (uint32_t row = r_lo + wave; row < r_lo + r_n; row += kWaves) {
      const uint32_t n = n0 + lane;
      epi.x_next[(size_t)row * N + n] = act_enc(red[1][row][lane] * s_rstd[row] * w_pre, epi.act);
    }
    if (tile == 0 && t < r_n) epi.rstd[r_lo + t] = s_rstd[r_lo + t];
  } else if constexpr (EPI == EPI_SILU) {
    // 64 interleave16 columns = 32 outputs k = 32 tile + i (gate at gflat, up at gflat + 16)
    for (uint32_t i = t; i < 32u * M; i += 256u) {
      const uint32_t row = i / 32u, kk = i % 32u, k = tile * 32u + kk;
      const uint32_t gcol = (kk / 16u) * 32u + (kk % 16u);
      const float g_r = act_round(folded(row, gcol), epi.act), u_r = act_round(folded(row, gcol + 16u), epi.act);
      const float s_r = act_round(silu_f32(g_r), epi.act);
      epi.h[(size_t)row * (N / 2) + k] = act_enc(s_r * u_r, epi.act);
    }
  } else if constexpr (EPI == EPI_F16OUT) {
    for (uint32_t i = t; i < total; i += 256u)
      epi.out16[(size_t)(i / kCols) * N + n0 + i % kCols] = act_enc(folded(i / kCols, i % kCols), epi.act);
  } else if constexpr (EPI == EPI_LOGITS) {
    for (uint32_t row = wave; row < M; row += kWaves) {
      const uint32_t n = n0 + lane;
      const float v = folded(row, lane);
      epi.out32[(size_t)row * N + n] = v;
      if (epi.argmax_part) {
        float bv = n < epi.vocab_used ? v : -INFINITY;
        uint32_t bi = n;
#pragma unroll
        for (int st = 32; st > 0; st >>= 1) {
          const float ov = __shfl_down(bv, st, 64);
          const uint32_t oi = __shfl_down(bi, st, 64);
          if (lane + st < 64 && better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
          }
        }
        // a tile with a non-finite logit reports a NaN value, which argmax_stage2 flags
        const bool bad = __ballot(n < epi.vocab_used && !__builtin_isfinite(v)) != 0ull;
        if (lane == 0)
          epi.argmax_part[(size_t)row * ntiles + tile] = u2_t{bad ? kNanBits : __builtin_bit_cast(uint32_t, bv), bi};
      }
    }
  }
}

// out[m][n] (fp16 or fp32) = sum over s ascending of partials[s][m][n], from 0.f.
__global__ __launch_bounds__(256) void fold_partials_kernel(const float* __restrict__ partials,
                                                            uint16_t* __restrict__ out16,
                                                            float* __restrict__ out32,
                                                            uint32_t S, uint32_t MN) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i >= MN) return;
  float t = 0.f;
  for (uint32_t s = 0; s < S; ++s) t += partials[(size_t)s * MN + i];
  if (out16) out16[i] = f2h(t);
  if (out32) out32[i] = t;
}

__global__ __launch_bounds__(256) void handoff_init_kernel(uint32_t* __restrict__ p, size_t n) {
  for (size_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += (size_t)gridDim.x * 256u) p[i] = kEmpty;
}

template <int MR, int EPI>
int launch_gemv(const uint32_t* qw, const uint16_t* sc, const uint16_t* x, float* part, uint32_t M,
                uint32_t K, uint32_t N, uint32_t S, const GemvEpi& epi, hipStream_t st) {
  const uint32_t G = K / 64, gps = G / S;
  // QKV with fixed consumers: one more row, the heads' consumers
  // fixed consumers: a row of their own after the S slices (QKV always, the others when
  // extra_row), or slice S-1
  GemvEpi e = epi;
  e.extra_row = EPI == EPI_RESID && !epi.arrive && kExtraRow;
  e.row_cons = e.extra_row && M > 1;
  dim3 grid(N / kCols, (EPI == EPI_QKV || e.extra_row) && !epi.arrive ? S + (e.row_cons ? M : 1u) : S);
  if constexpr (EPI == EPI_PARTIALS || EPI == EPI_SILU || EPI == EPI_QKV) {
    if (epi.in_sums) {
      gemv_w4a16_kernel<MR, (MR >= 3 ? 1 : 2), EPI, true><<<grid, 256, 0, st>>>(qw, sc, x, part, M, K, N, gps, e);
      return (int)hipGetLastError();
    }
  }
  if (gps >= 16)
    gemv_w4a16_kernel<MR, 4, EPI><<<grid, 256, 0, st>>>(qw, sc, x, part, M, K, N, gps, e);
  else if (MR >= 3)  // one k-group per wave at a time: five or six waves per SIMD instead of four
    gemv_w4a16_kernel<MR, 1, EPI><<<grid, 256, 0, st>>>(qw, sc, x, part, M, K, N, gps, e);
  else
    gemv_w4a16_kernel<MR, 2, EPI><<<grid, 256, 0, st>>>(qw, sc, x, part, M, K, N, gps, e);
  return (int)hipGetLastError();
}

template <int EPI>
int launch_rows(const uint32_t* qw, const uint16_t* sc, const uint16_t* x, float* part, uint32_t M,
                uint32_t K, uint32_t N, uint32_t S, const GemvEpi& epi, hipStream_t st) {
  if (M == 1) return launch_gemv<1, EPI>(qw, sc, x, part, M, K, N, S, epi, st);
  // two and three rows: kernels of their own (94 / 96-99 VGPRs, five waves per SIMD where they
  // fit 96, against the 4-row kernel's 102 and four: 27B verify step at 2 rows 4.81 -> 4.44 ms,
  // at 3 rows 5.06 -> 4.88)
  if (M == 2) return launch_gemv<2, EPI>(qw, sc, x, part, M, K, N, S, epi, st);
  if (M == 3) return launch_gemv<3, EPI>(qw, sc, x, part, M, K, N, S, epi, st);
  if (M <= 4) return launch_gemv<4, EPI>(qw, sc, x, part, M, K, N, S, epi, st);
  return launch_gemv<16, EPI>(qw, sc, x, part, M, K, N, S, epi, st);
}

int check_gemv(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x, const float* partials,
               uint32_t M, uint32_t K, uint32_t N, uint32_t S) {
  if (!qweight || !scales || !x || !partials) return mi_fail(MI_ERR_ARG, "gemv_w4a16: null pointer");
  if (M < 1 || M > 16) return mi_fail(MI_ERR_SHAPE, "gemv_w4a16: M must be 1..16");
  if (K == 0 || K % 64 || N == 0 || N % 64)
    return mi_fail(MI_ERR_SHAPE, "gemv_w4a16: K and N must be non-zero multiples of 64");
  if (S == 0 || (K / 64) % S) return mi_fail(MI_ERR_SHAPE, "gemv_w4a16: S must divide K/64");
  if (reinterpret_cast<uintptr_t>(qweight) % 16 || reinterpret_cast<uintptr_t>(x) % 16 ||
      reinterpret_cast<uintptr_t>(scales) % 8)
    return mi_fail(MI_ERR_ARG, "gemv_w4a16: qweight/x need 16-byte, scales 8-byte alignment");
  return 0;
}

}  // namespace
}  // namespace mi

using namespace mi;

namespace {
// the smallest S | K/64 that gives at most 8 k-groups per split and at least 2048 work-groups,
// never going below min_gps k-groups per split
uint32_t pick_split(uint32_t K, uint32_t N, uint32_t min_gps) {
  const uint32_t G = K / 64, tiles = N / kCols;
  uint32_t best = 1;
  for (uint32_t S = 1; S <= G; ++S) {
    if (G % S) continue;
    const uint32_t gps = G / S;
    if (gps < min_gps && S > 1) break;
    best = S;
    if (gps <= 8 && tiles * S >= 2048) break;
  }
  return best;
}
}  // namespace

extern "C" uint32_t mi_gemv_pick_s(uint32_t K, uint32_t N) {
  // The split-K width for a plain launch (measured on MI355X over the 27B shapes at M = 1):
  // at least 4 k-groups per split.
  return pick_split(K, N, 4u);
}

extern "C" uint32_t mi_gemv_pick_s_ex(uint32_t K, uint32_t N, uint32_t epilogue) {
  // The consumer folds the tile's slices after one poll round trip whatever S is, and the
  // producers do not wait, so the fused launches keep the plain choice (measured on MI355X
  // over the 27B shapes: o 20, gate_up 10 and down 34 beat the largest S <= 8). QKV's head
  // consumers fold a whole head over every slice: there the smallest S | K/64 with at most 8
  // k-groups per slice (27B qkv: 10, measured ahead of 5, 8, 16 and 20).
  // RESID: at least 5 k-groups per split (27B o: 16 rather than 20, step 4.07 -> 4.03 ms;
  // down keeps 34).
  if (epilogue == MI_EPI_RESID) return pick_split(K, N, 5u);
  if (epilogue == MI_EPI_QKV) {
    const uint32_t G = K / 64;
    for (uint32_t S = 1; S <= G; ++S)
      if (G % S == 0 && G / S <= 8) return S;
    return G ? G : 1;
  }
  return mi_gemv_pick_s(K, N);
}

extern "C" int mi_gemv_w4a16(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x,
                             float* partials, uint32_t M, uint32_t K, uint32_t N, uint32_t S,
                             void* stream) {
  if (int e = check_gemv(qweight, scales, x, partials, M, K, N, S)) return e;
  const GemvEpi none{};
  return mi_hip(launch_rows<EPI_PARTIALS>(qweight, scales, x, partials, M, K, N, S, none,
                                          static_cast<hipStream_t>(stream)),
                "gemv_w4a16 launch");
}

extern "C" int mi_gemv_w4a16_ex(const uint32_t* qweight, const uint16_t* scales, const uint16_t* x,
                                float* partials, uint32_t M, uint32_t K, uint32_t N, uint32_t S,
                                const mi_gemv_epilogue* ep, void* stream) {
  if (int e = check_gemv(qweight, scales, x, partials, M, K, N, S)) return e;
  if (!ep) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex: null epilogue");
  hipStream_t st = static_cast<hipStream_t>(stream);
  GemvEpi e{ep->resid, ep->sumsq, ep->rstd, ep->next_norm_w, ep->x_next, ep->h,
            ep->logits, reinterpret_cast<u2_t*>(ep->argmax_part), ep->vocab_used, ep->eps, ep->out16};
  e.status = ep->status;
  e.poll_limit = ep->poll_limit ? ep->poll_limit : kPollLimit;
  e.inject = ep->inject;
  e.arrive = ep->arrive;
  if (ep->act > 1) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex: act is 0 (f16) or 1 (bf16)");
  e.act = ep->act;
  e.sums_out = ep->sums_out;
  e.in_sums = ep->in_sums;
  e.in_norm_w = ep->in_norm_w;
  e.in_eps = ep->in_eps;
  if (e.in_sums) {
    if (!e.in_norm_w) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex: in_sums needs in_norm_w");
    if (ep->kind != MI_EPI_PARTIALS && ep->kind != MI_EPI_SILU && ep->kind != MI_EPI_QKV)
      return mi_fail(MI_ERR_SHAPE, "gemv_w4a16_ex: in_sums with the PARTIALS, SILU or QKV kind only");
    if (K / 64 > 256 || (K / 64) % 4 || (K / 64) / S > 8)
      return mi_fail(MI_ERR_SHAPE, "gemv_w4a16_ex: in_sums needs K a multiple of 256 up to 16384 and at most 8 "
                                   "k-groups per slice");
  }
  int r;
  switch (ep->kind) {
    case MI_EPI_PARTIALS:
      r = launch_rows<EPI_PARTIALS>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_RESID:
      if (!e.resid || (!e.sums_out && (!e.sumsq || !e.rstd || !e.next_w || !e.x_next)))
        return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex RESID: resid, and sums_out or sumsq, rstd, next_norm_w and x_next are required");
      if (N > 16384)  // every tile's consumer must be resident at once (N/64 <= 256 work-groups)
        return mi_fail(MI_ERR_SHAPE, "gemv_w4a16_ex RESID: N must be <= 16384");
      r = launch_rows<EPI_RESID>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_SILU:
      if (!e.h) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex SILU: h is required");
      r = launch_rows<EPI_SILU>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_LOGITS:
      if (!e.out32 || e.vocab_used > N)
        return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex LOGITS: logits is required, vocab_used <= N");
      r = launch_rows<EPI_LOGITS>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_F16OUT:
      if (!e.out16) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex F16OUT: out16 is required");
      r = launch_rows<EPI_F16OUT>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    case MI_EPI_QKV: {
      const mi_attn_shape* sh = ep->shape;
      if (!ep->ctrl || !sh || !ep->rope || !ep->attn_q || !ep->kv_k || !ep->kv_v)
        return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex QKV: ctrl, shape, rope, attn_q, kv_k and kv_v are required");
      if (M > 4) return mi_fail(MI_ERR_SHAPE, "gemv_w4a16_ex QKV: M must be <= 4");
      if (sh->gated) return mi_fail(MI_ERR_SHAPE, "gemv_w4a16_ex QKV: gated attention is not fused");
      const uint32_t HD = sh->head_dim;
      if (HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "gemv_w4a16_ex QKV: head_dim must be 128 or 256");
      if (sh->kv_heads == 0 || N != (sh->q_heads + 2 * sh->kv_heads) * HD || sh->qkv_n != N ||
          sh->k_off != sh->q_heads * HD || sh->v_off != (sh->q_heads + sh->kv_heads) * HD)
        return mi_fail(MI_ERR_SHAPE, "gemv_w4a16_ex QKV: N must be the q||k||v width of the shape");
      if (sh->rot_dim > HD || sh->rot_dim % 2) return mi_fail(MI_ERR_SHAPE, "gemv_w4a16_ex QKV: bad rot_dim");
      if (ep->pages && ep->page == 0) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex QKV: page size 0");
      if (sh->act != ep->act) return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex QKV: the shape's act differs from the epilogue's");
      e.ctrl = ep->ctrl; e.rope = ep->rope; e.q_norm = ep->q_norm; e.k_norm = ep->k_norm;
      e.attn_q = ep->attn_q; e.kv_k = ep->kv_k; e.kv_v = ep->kv_v; e.pages = ep->pages;
      e.row_stride = ep->row_stride; e.head_stride = ep->head_stride; e.page = ep->page; e.kv_len = ep->kv_len;
      e.q_heads = sh->q_heads; e.kv_heads = sh->kv_heads; e.head_dim = HD; e.rot_dim = sh->rot_dim;
      e.qk_eps = sh->eps;
      r = launch_rows<EPI_QKV>(qweight, scales, x, partials, M, K, N, S, e, st);
      break;
    }
    default:
      return mi_fail(MI_ERR_ARG, "gemv_w4a16_ex: unknown epilogue");
  }
  return mi_hip(r, "gemv_w4a16_ex launch");
}

extern "C" int mi_gemv_handoff_init(float* words, size_t n, void* stream) {
  if (!words || n == 0) return mi_fail(MI_ERR_ARG, "gemv_handoff_init: bad arguments");
  const size_t blocks = std::min<size_t>((n + 255) / 256, 4096);
  handoff_init_kernel<<<(uint32_t)blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<uint32_t*>(words), n);
  return mi_hip((int)hipGetLastError(), "gemv_handoff_init launch");
}

extern "C" int mi_fold_partials(const float* partials, uint16_t* out_f16, float* out_f32, uint32_t S,
                                uint32_t M, uint32_t N, void* stream) {
  if (!partials || (!out_f16 && !out_f32) || S == 0)
    return mi_fail(MI_ERR_ARG, "fold_partials: bad arguments");
  const uint32_t MN = M * N;
  fold_partials_kernel<<<(MN + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(
      partials, out_f16, out_f32, S, MN);
  return mi_hip((int)hipGetLastError(), "fold_partials launch");
}
