// prep.hip - the between-GEMV kernels of one decode step and the token boundary.
//
//   res_fold / norm_finish   src/kernels/prep.cl:288 / :350 (twin prep_ref.h:120-168)
//   res_norm                 prep_ref.h:59-92 (the single-launch form)
//   silu_mul                 src/kernels/prep.cl:384 (twin prep_ref.h:170-189)
//   attn_prep                src/kernels/attn.cl:361 (twin attn_ref.h:117-199)
//   embed_gather             src/kernels/embed_gather.cl:47-69
//   argmax_stage1 / _stage2  src/kernels/argmax.cl:82-172
//
// Every per-element chain and every reduction tree is the reference's, so the outputs
// are bit-identical to the CPU oracle's restatement (exp aside, which is ~1 ulp): the
// variance sum is a per-lane fma over a strided slice, then the pairwise tree
// red[i] += red[i + stride] for stride = WG/2 .. 1; `1.0f / sqrtf()`; explicit fma.
// Wave64 note: strides >= 64 cross waves and go through LDS; strides < 64 are
// __shfl_down within the wave, which adds exactly the same pairs.
#include "mi_capi_internal.h"
#include <mutex>

#include "mi_common.h"

namespace mi {
namespace {

constexpr uint32_t kWG = 256;

// red[i] += red[i + stride], stride = 128 .. 1, over 256 lanes; the total lands in lane 0
// (and is returned to every lane through LDS).
__device__ __forceinline__ float tree256(float v, float* lds) {
  const uint32_t t = threadIdx.x;
  lds[t] = v;
  __syncthreads();
  if (t < 128) lds[t] = lds[t] + lds[t + 128];
  __syncthreads();
  float a = 0.f;
  if (t < 64) {
    a = lds[t] + lds[t + 64];
#pragma unroll
    for (int st = 32; st > 0; st >>= 1) a += __shfl_down(a, st, 64);
  }
  __syncthreads();
  if (t == 0) lds[0] = a;
  __syncthreads();
  const float r = lds[0];
  __syncthreads();
  return r;
}

// The same tree over HD lanes (HD = 64, 128 or 256; the work-group is HD lanes).
__device__ __forceinline__ float tree_hd(float v, float* lds, uint32_t HD) {
  const uint32_t t = threadIdx.x;
  lds[t] = v;
  __syncthreads();
  for (uint32_t st = HD / 2; st >= 64; st >>= 1) {
    if (t < st) lds[t] = lds[t] + lds[t + st];
    __syncthreads();
  }
  float a = 0.f;
  if (t < 64) {
    a = lds[t];
#pragma unroll
    for (int st = 32; st > 0; st >>= 1) a += __shfl_down(a, st, 64);
  }
  __syncthreads();
  if (t == 0) lds[0] = a;
  __syncthreads();
  const float r = lds[0];
  __syncthreads();
  return r;
}

// r_b = rne(resid + rne(sum_s partials)), or resid when S_PREV == 0; ZERO (prep.cl's
// ZERO_RESID, the MTP head's fc fold): r_b = rne(sum_s partials), the residual taken as zero
__device__ __forceinline__ uint16_t fold_resid(const float* __restrict__ partials, uint16_t rb,
                                               uint32_t S_PREV, uint32_t M, uint32_t m, uint32_t K,
                                               uint32_t k, bool zero = false) {
  if (S_PREV == 0) return rb;
  float acc = 0.f;
  for (uint32_t s = 0; s < S_PREV; ++s) acc += partials[((size_t)s * M + m) * K + k];
  return zero ? f2h(acc) : f2h(h2f(rb) + h2f(f2h(acc)));
}

// grid (G, M), 256 lanes: chunk g of K/G elements, lane i takes k = g chunk + i, + 256 ...
__global__ __launch_bounds__(256) void res_fold_kernel(const float* __restrict__ partials,
                                                       uint16_t* __restrict__ resid,
                                                       float* __restrict__ sumsq, uint32_t M,
                                                       uint32_t K, uint32_t S_PREV, uint32_t G,
                                                       uint32_t zero) {
  __shared__ float lds[kWG];
  const uint32_t g = blockIdx.x, m = blockIdx.y, i = threadIdx.x;
  const uint32_t chunk = (K + G - 1) / G;
  const uint32_t k0 = g * chunk, k1 = min(k0 + chunk, K);
  uint16_t* rp = resid + (size_t)m * K;
  float acc2 = 0.f;
  for (uint32_t k = k0 + i; k < k1; k += kWG) {
    const uint16_t rb = fold_resid(partials, rp[k], S_PREV, M, m, K, k, zero != 0);
    rp[k] = rb;
    const float v = h2f(rb);
    acc2 = __builtin_fmaf(v, v, acc2);
  }
  const float tot = tree256(acc2, lds);
  if (i == 0) sumsq[(size_t)g * M + m] = tot;
}

// grid (ceil(K / 256), M): x = rne(r * rstd * w), rstd from the G chunk sums in g order; row m
// of x at m * x_stride (prep.cl's X_STRIDE: the MTP head's two norms into one [M][2K] row).
__global__ __launch_bounds__(256) void norm_finish_kernel(const float* __restrict__ sumsq,
                                                          const uint16_t* __restrict__ resid,
                                                          const float* __restrict__ norm_w,
                                                          uint16_t* __restrict__ x_out, uint32_t M,
                                                          uint32_t K, uint32_t G, float eps, size_t x_stride) {
  const uint32_t m = blockIdx.y, k = blockIdx.x * kWG + threadIdx.x;
  float total = 0.f;
  for (uint32_t g = 0; g < G; ++g) total += sumsq[(size_t)g * M + m];
  const float mean = total / (float)K;
  const float rstd = 1.0f / sqrtf(mean + eps);
  if (k < K) x_out[(size_t)m * x_stride + k] = f2h(h2f(resid[(size_t)m * K + k]) * rstd * norm_w[k]);
}

// grid (M), 256 lanes: the single-launch residual fold + RMSNorm (prep_ref res_norm).
__global__ __launch_bounds__(256) void res_norm_kernel(const float* __restrict__ partials,
                                                       uint16_t* __restrict__ resid,
                                                       const float* __restrict__ norm_w,
                                                       uint16_t* __restrict__ x_out, uint32_t M,
                                                       uint32_t K, uint32_t S_PREV, float eps) {
  __shared__ float lds[kWG];
  const uint32_t m = blockIdx.x, i = threadIdx.x;
  uint16_t* rp = resid + (size_t)m * K;
  float acc2 = 0.f;
  for (uint32_t k = i; k < K; k += kWG) {
    const uint16_t rb = fold_resid(partials, rp[k], S_PREV, M, m, K, k);
    rp[k] = rb;
    const float v = h2f(rb);
    acc2 = __builtin_fmaf(v, v, acc2);
  }
  const float tot = tree256(acc2, lds);
  const float rstd = 1.0f / sqrtf(tot / (float)K + eps);
  for (uint32_t k = i; k < K; k += kWG) x_out[(size_t)m * K + k] = f2h(h2f(rp[k]) * rstd * norm_w[k]);
}

// grid (ceil(N / 256), M): gate||up interleaved in 16-column blocks -> silu(g) * u.
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* __restrict__ partials,
                                                       uint16_t* __restrict__ x_out, uint32_t M,
                                                       uint32_t N, uint32_t S) {
  const uint32_t m = blockIdx.y, k = blockIdx.x * kWG + threadIdx.x;
  if (k >= N) return;
  const size_t FN = (size_t)2 * N;
  const size_t gflat = (size_t)(k / 16) * 32 + (k % 16), uflat = gflat + 16;
  float ga = 0.f, ua = 0.f;
  for (uint32_t s = 0; s < S; ++s) {
    const size_t base = ((size_t)s * M + m) * FN;
    ga += partials[base + gflat];
    ua += partials[base + uflat];
  }
  const uint16_t g_b = f2h(ga), u_b = f2h(ua);
  const uint16_t s_b = f2h(silu_f32(h2f(g_b)));
  x_out[(size_t)m * N + k] = f2h(h2f(s_b) * h2f(u_b));
}

struct AttnPrepArgs {
  uint32_t* ctrl;
  const float* partials;
  const float* q_norm;
  const float* k_norm;
  const float* rope;
  float* attn_q;
  float* attn_gate;
  uint16_t* kv_k;
  uint16_t* kv_v;
  const uint32_t* pages;
  size_t row_stride, head_stride;
  uint32_t page, S, M, q_heads, kv_heads, head_dim, rot_dim, gated, qkv_n, k_off, v_off;
  uint32_t kv_len;  // positions the cache (or page table) holds; 0 = unchecked
  float eps;
  // int8 cache (attn_prep_kv8): rows of int8 at kv_k / kv_v's element offsets, fp16 scales
  // at row * sc_row_stride + head * sc_head_stride
  uint16_t* k_scale;
  uint16_t* v_scale;
  size_t sc_row_stride, sc_head_stride;
  uint32_t act;  // 0 f16, 1 bf16 roundings (the f16 cache only)
};

__device__ __forceinline__ size_t kv_row(uint32_t p, const uint32_t* pages, uint32_t page) {
  return pages ? (size_t)pages[p / page] * page + p % page : (size_t)p;
}

// grid (q_heads + kv_heads, M), HD lanes. KV8 (attn_prep_kv8, kv8.cl:287-408; head_dim 256):
// the same chain, then q rotated in fp32, and the K row as the f16 cache would hold it and
// the V row rotated and quantised into the int8 cache.
template <bool KV8>
__global__ __launch_bounds__(256) void attn_prep_kernel(AttnPrepArgs a) {
  __shared__ float red[256];
  __shared__ float nrm[256];
  const uint32_t wg = blockIdx.x, m = blockIdx.y, i = threadIdx.x, HD = a.head_dim;
  const uint32_t n_act = a.ctrl[CTRL_NACT];
  if (m >= n_act) return;  // uniform
  const uint32_t pos = a.ctrl[CTRL_POS];
  if (a.kv_len && pos + m >= a.kv_len) {  // past the cache: write nothing, flag the step
    if (i == 0 && wg == 0) a.ctrl[CTRL_DEBUG] = 0xDEAD0002u;
    return;
  }
  const bool is_q = wg < a.q_heads;
  const uint32_t h = is_q ? wg : wg - a.q_heads;
  const float* nw = is_q ? a.q_norm : a.k_norm;
  const size_t base = is_q ? (a.gated ? (size_t)h * 2 * HD : (size_t)h * HD)
                           : (size_t)a.k_off + (size_t)h * HD;
  // sum_s partials in ascending s from 0.f; the loads go out 32 at a time (past S they reload
  // the last partial and add +0.f, which leaves the sum's bits unchanged: it starts at +0.f
  // and a round-to-nearest sum of nonzero terms is never -0)
  auto qkv_sum = [&](size_t col) {
    const float* p = a.partials + (size_t)m * a.qkv_n + col;
    const size_t step = (size_t)a.M * a.qkv_n;
    float v = 0.0f;
    for (uint32_t s = 0; s < a.S; s += 32u) {
      float t8[32];
#pragma unroll
      for (uint32_t u = 0; u < 32; ++u) t8[u] = p[min(s + u, a.S - 1u) * step];
#pragma unroll
      for (uint32_t u = 0; u < 32; ++u) v += s + u < a.S ? t8[u] : 0.f;
    }
    return v;
  };
  // Everything this lane reads goes out before the norm's barriers (loads cannot move
  // across them): the head's partials, the V (or gate) partials, the RoPE pair, the norm
  // weight, the page-table entry. The arithmetic and its order are unchanged.
  const uint32_t half = a.rot_dim / 2;
  const float* cs = a.rope + (size_t)(pos + m) * 2 * half;
  float rc = 1.f, rsn = 0.f;
  if (i < a.rot_dim) {
    const uint32_t ii = i < half ? i : i - half;
    rc = cs[ii];
    rsn = cs[half + ii];
  }
  const float wn = nw ? nw[i] : 0.f;
  const size_t row = is_q ? 0 : kv_row(pos + m, a.pages, a.page);
  float vg = 0.f;
  if (!is_q) vg = qkv_sum((size_t)a.v_off + (size_t)h * HD + i);
  else if (a.gated && a.attn_gate) vg = qkv_sum(base + HD + i);
  const float xf = act_round(qkv_sum(base + i), a.act);
  float nv;
  if (nw) {
    const float tot = tree_hd(xf * xf, red, HD);
    const float rstd = 1.0f / sqrtf(tot / (float)HD + a.eps);
    nv = act_round(xf * rstd * wn, a.act);
  } else {
    nv = xf;
  }
  nrm[i] = nv;
  __syncthreads();
  float outv;
  if (i < half) {
    const float t = nrm[i + half] * rsn;
    outv = __builtin_fmaf(nv, rc, -t);
  } else if (i < a.rot_dim) {
    const float t = nrm[i - half] * rsn;
    outv = __builtin_fmaf(nv, rc, t);
  } else {
    outv = nv;
  }
  if constexpr (KV8) {
    __shared__ float xch[2 * 256];
    __shared__ float s_am[2][4];
    const bool neg = kv8_sign_neg(i);
    if (is_q) {  // uniform: every thread of the work-group reaches the barriers inside
      float v1[1] = {outv};
      fwht256<1>(v1, i, xch);
      a.attn_q[((size_t)m * a.q_heads + h) * HD + i] = kv8_flip(v1[0], neg) * 0.0625f;
      if (a.gated && a.attn_gate) a.attn_gate[((size_t)m * a.q_heads + h) * HD + i] = h2f(f2h(vg));
    } else {
      float v2[2] = {h2f(f2h(outv)), h2f(f2h(vg))};
      fwht256<2>(v2, i, xch);
      const float yk = kv8_flip(v2[0], neg) * 0.0625f, yv = kv8_flip(v2[1], neg) * 0.0625f;
      const float mk = wave_max(fabsf(yk)), mv = wave_max(fabsf(yv));
      if ((i & 63u) == 0) {
        s_am[0][i >> 6] = mk;
        s_am[1][i >> 6] = mv;
      }
      lds_barrier();
      const float ak = fmaxf(fmaxf(s_am[0][0], s_am[0][1]), fmaxf(s_am[0][2], s_am[0][3]));
      const float av = fmaxf(fmaxf(s_am[1][0], s_am[1][1]), fmaxf(s_am[1][2], s_am[1][3]));
      const uint16_t sk = kv8_f16_sat(ak / 127.0f), sv = kv8_f16_sat(av / 127.0f);
      int8_t* k8 = reinterpret_cast<int8_t*>(a.kv_k);
      int8_t* v8 = reinterpret_cast<int8_t*>(a.kv_v);
      k8[row * a.row_stride + h * a.head_stride + i] = kv8_quant(yk, h2f(sk));
      v8[row * a.row_stride + h * a.head_stride + i] = kv8_quant(yv, h2f(sv));
      if (i == 0) {
        a.k_scale[row * a.sc_row_stride + h * a.sc_head_stride] = sk;
        a.v_scale[row * a.sc_row_stride + h * a.sc_head_stride] = sv;
      }
    }
  } else {
    if (is_q) {
      a.attn_q[((size_t)m * a.q_heads + h) * HD + i] = outv;
      if (a.gated && a.attn_gate) a.attn_gate[((size_t)m * a.q_heads + h) * HD + i] = act_round(vg, a.act);
    } else {
      a.kv_k[row * a.row_stride + h * a.head_stride + i] = act_enc(outv, a.act);
      a.kv_v[row * a.row_stride + h * a.head_stride + i] = act_enc(vg, a.act);
    }
  }
}

// grid (M), 256 lanes
__global__ __launch_bounds__(256) void embed_gather_kernel(uint32_t* __restrict__ ctrl,
                                                           const uint16_t* __restrict__ embed,
                                                           uint16_t* __restrict__ resid,
                                                           uint32_t hidden, uint32_t vocab) {
  const uint32_t m = blockIdx.x, lid = threadIdx.x;
  const uint32_t row = ctrl[CTRL_CUR + m];
  if (row >= vocab) {
    if (lid == 0) ctrl[CTRL_DEBUG] = 0xDEAD0001u;
    return;
  }
  const uint16_t* src = embed + (size_t)row * hidden;
  uint16_t* dst = resid + (size_t)m * hidden;
  if ((hidden & 7u) == 0) {
    const u4_t* s4 = reinterpret_cast<const u4_t*>(src);
    u4_t* d4 = reinterpret_cast<u4_t*>(dst);
    for (uint32_t k = lid; k < hidden / 8; k += kWG) d4[k] = s4[k];
  } else {
    for (uint32_t k = lid; k < hidden; k += kWG) dst[k] = src[k];
  }
}


// grid (M), 256 lanes: embed_gather followed by the first RMSNorm, with the residual's
// sum of squares taken in 64-element chunks (the reference's res_fold tree at chunk 64:
// one element per lane, then the pairwise tree; chunks summed in ascending order).
// GATHER: resid[m] = embed[cur_token[m]] first (embed_gather), else the norm of resid[m] as it
// is (prep_res_fold with S_PREV 0, then prep_norm_finish).
template <bool GATHER>
__global__ __launch_bounds__(256) void embed_norm_kernel(uint32_t* __restrict__ ctrl,
                                                         const uint16_t* __restrict__ embed,
                                                         uint16_t* __restrict__ resid,
                                                         const float* __restrict__ norm_w,
                                                         uint16_t* __restrict__ x_out,
                                                         float* __restrict__ rstd_out, uint32_t hidden,
                                                         uint32_t vocab, float eps, uint32_t act) {
  __shared__ float chunk[1024];
  // rows up to kHeld * 64 wide stay in registers between the two passes (with their norm weights,
  // loaded alongside), so a row takes one memory round trip; wider rows are read again
  constexpr uint32_t kPass = 8, kIters = 3, kHeld = kPass * kIters * 4;
  const uint32_t m = blockIdx.x, t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint16_t* src = resid + (size_t)m * hidden;
  if constexpr (GATHER) {
    const uint32_t row = ctrl[CTRL_CUR + m];
    if (row >= vocab) {
      if (t == 0) ctrl[CTRL_DEBUG] = 0xDEAD0001u;
      return;
    }
    src = embed + (size_t)row * hidden;
  }
  uint16_t* dst = resid + (size_t)m * hidden;
  const uint32_t nch = hidden / 64;
  const bool held = nch <= kHeld;
  // wave w takes chunks w, w + 4, ...; the loads of up to kPass chunks go out together
  uint16_t hv[kIters][kPass];
  float hw[kIters][kPass];
  if (held) {
#pragma unroll
    for (uint32_t it = 0; it < kIters; ++it)
#pragma unroll
      for (uint32_t u = 0; u < kPass; ++u) {
        const uint32_t c = wave + 4u * (kPass * it + u);
        hv[it][u] = c < nch ? src[c * 64 + lane] : (uint16_t)0;
        hw[it][u] = c < nch ? norm_w[c * 64 + lane] : 0.f;
      }
  }
  for (uint32_t c0 = wave, it = 0; c0 < nch; c0 += 4u * kPass, ++it) {
    uint16_t v16[kPass];
#pragma unroll
    for (uint32_t u = 0; u < kPass; ++u) {
      const uint32_t c = c0 + 4 * u;
      if (held) {
        v16[u] = it == 0 ? hv[0][u] : (it == 1 ? hv[1][u] : hv[2][u]);
      } else {
        v16[u] = c < nch ? src[c * 64 + lane] : (uint16_t)0;
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < kPass; ++u) {
      const uint32_t c = c0 + 4 * u;
      if (c < nch) {
        if constexpr (GATHER) dst[c * 64 + lane] = v16[u];
        const float v = res_widen(v16[u], act);
        float a = __builtin_fmaf(v, v, 0.f);
#pragma unroll
        for (int st = 32; st > 0; st >>= 1) a += __shfl_down(a, st, 64);
        if (lane == 0) chunk[c] = a;
      }
    }
  }
  __syncthreads();
  __shared__ float s_rstd;
  if (t == 0) {
    float tot = 0.f;
    for (uint32_t c = 0; c < nch; ++c) tot += chunk[c];
    s_rstd = 1.0f / sqrtf(tot / (float)hidden + eps);
  }
  __syncthreads();
  const float r = s_rstd;
  if (t == 0 && rstd_out) rstd_out[m] = r;  // after the barrier, which would otherwise wait for it
  if (held) {
#pragma unroll
    for (uint32_t it = 0; it < kIters; ++it)
#pragma unroll
      for (uint32_t u = 0; u < kPass; ++u) {
        const uint32_t c = wave + 4u * (kPass * it + u);
        if (c < nch) x_out[(size_t)m * hidden + c * 64 + lane] = act_enc(res_widen(hv[it][u], act) * r * hw[it][u], act);
      }
    return;
  }
  for (uint32_t k0 = t; k0 < hidden; k0 += 8 * kWG) {
    uint16_t v16[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) v16[u] = k0 + u * kWG < hidden ? src[k0 + u * kWG] : (uint16_t)0;
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) {
      const uint32_t k = k0 + u * kWG;
      if (k < hidden) x_out[(size_t)m * hidden + k] = act_enc(res_widen(v16[u], act) * r * norm_w[k], act);
    }
  }
}

// The comparator (argmax.cl:63-65): strictly greater wins, an exact tie keeps the lower index.
__device__ __forceinline__ bool better(float av, uint32_t ai, float bv, uint32_t bi) {
  return (av > bv) || (av == bv && ai < bi);
}
constexpr uint32_t kChunk = 1024;
constexpr uint32_t kNoIdx = 0x7FFFFFFFu;

__device__ __forceinline__ void argtree(float& bv, uint32_t& bi, float* sv, uint32_t* si) {
  const uint32_t lid = threadIdx.x;
  sv[lid] = bv;
  si[lid] = bi;
  __syncthreads();
  for (uint32_t st = kWG / 2; st > 0; st >>= 1) {
    if (lid < st && better(sv[lid + st], si[lid + st], sv[lid], si[lid])) {
      sv[lid] = sv[lid + st];
      si[lid] = si[lid + st];
    }
    __syncthreads();
  }
  bv = sv[0];
  bi = si[0];
  __syncthreads();
}

// grid (ceil(vocab / 1024), M), 256 lanes: part[m][g] = {value, index as u32 bits}
__global__ __launch_bounds__(256) void argmax_stage1_kernel(const uint32_t* __restrict__ ctrl,
                                                            const float* __restrict__ logits,
                                                            u2_t* __restrict__ part, uint32_t vocab,
                                                            uint32_t vocab_used, uint32_t groups) {
  __shared__ float sv[kWG];
  __shared__ uint32_t si[kWG];
  const uint32_t g = blockIdx.x, m = blockIdx.y, lid = threadIdx.x;
  if (m >= ctrl[CTRL_NACT]) return;
  const uint32_t k0 = g * kChunk, k1 = min(k0 + kChunk, vocab);
  const float* row = logits + (size_t)m * vocab;
  float bv = -INFINITY;
  uint32_t bi = kNoIdx;
  bool bad = false;  // a used logit that is not finite
  for (uint32_t k = k0 + lid; k < k1; k += kWG) {
    const float v = k < vocab_used ? row[k] : -INFINITY;
    bad |= k < vocab_used && !__builtin_isfinite(v);
    if (better(v, k, bv, bi)) {
      bv = v;
      bi = k;
    }
  }
  argtree(bv, bi, sv, si);
  bad = __syncthreads_or(bad);
  // a chunk with a non-finite logit reports a NaN value, which stage 2 flags
  if (lid == 0) part[(size_t)m * groups + g] = u2_t{bad ? kNanBits : __builtin_bit_cast(uint32_t, bv), bi};
}

// one work-group: fold each active row's chunk winners, write out_token[m], then
// cur_token[0] = out_token[n - 1], history[steps] = that id, pos += n, steps += 1.
__global__ __launch_bounds__(256) void argmax_stage2_kernel(uint32_t* __restrict__ ctrl,
                                                            const u2_t* __restrict__ part,
                                                            uint32_t* __restrict__ history,
                                                            uint32_t history_len, uint32_t groups) {
  __shared__ float sv[kWG];
  __shared__ uint32_t si[kWG];
  const uint32_t lid = threadIdx.x;
  const uint32_t n = ctrl[CTRL_NACT];
  bool bad = false;  // a chunk winner is NaN: the chunk held a non-finite logit
  for (uint32_t m = 0; m < n; ++m) {
    float bv = -INFINITY;
    uint32_t bi = kNoIdx;
    for (uint32_t g = lid; g < groups; g += kWG) {
      const u2_t e = part[(size_t)m * groups + g];
      const float v = __builtin_bit_cast(float, e.x);
      bad |= v != v;
      if (better(v, e.y, bv, bi)) {
        bv = v;
        bi = e.y;
      }
    }
    argtree(bv, bi, sv, si);
    if (lid == 0) ctrl[CTRL_OUT + m] = bi;
  }
  bad = __syncthreads_or(bad);
  if (lid == 0 && bad && ctrl[CTRL_DEBUG] == 0u) ctrl[CTRL_DEBUG] = kStatusNonFinite;
  if (lid == 0 && n != 0u) {
    const uint32_t tok = ctrl[CTRL_OUT + n - 1u];
    ctrl[CTRL_CUR] = tok;
    const uint32_t step = ctrl[CTRL_STEPS];
    if (history && step < history_len) history[step] = tok;
    ctrl[CTRL_STEPS] = step + 1u;
    ctrl[CTRL_POS] += n;
  }
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

int mi_res_fold(const float* partials, uint16_t* resid, float* sumsq, uint32_t M, uint32_t K,
                uint32_t S_PREV, uint32_t G, void* stream) {
  if (!resid || !sumsq || (S_PREV && !partials) || G == 0 || M == 0 || K == 0)
    return mi_fail(MI_ERR_ARG, "res_fold: bad arguments");
  res_fold_kernel<<<dim3(G, M), kWG, 0, (hipStream_t)stream>>>(partials, resid, sumsq, M, K, S_PREV, G, 0u);
  return mi_hip((int)hipGetLastError(), "res_fold");
}
int mi_res_fold_ex(const float* partials, uint16_t* resid, float* sumsq, uint32_t M, uint32_t K, uint32_t S_PREV,
                   uint32_t G, uint32_t zero_resid, void* stream) {
  if (!resid || !sumsq || (S_PREV && !partials) || G == 0 || M == 0 || K == 0 || zero_resid > 1)
    return mi_fail(MI_ERR_ARG, "res_fold_ex: bad arguments");
  res_fold_kernel<<<dim3(G, M), kWG, 0, (hipStream_t)stream>>>(partials, resid, sumsq, M, K, S_PREV, G,
                                                               zero_resid);
  return mi_hip((int)hipGetLastError(), "res_fold_ex");
}
int mi_norm_finish(const float* sumsq, const uint16_t* resid, const float* norm_w, uint16_t* x_out,
                   uint32_t M, uint32_t K, uint32_t G, float eps, void* stream) {
  if (!sumsq || !resid || !norm_w || !x_out || G == 0 || M == 0 || K == 0)
    return mi_fail(MI_ERR_ARG, "norm_finish: bad arguments");
  norm_finish_kernel<<<dim3((K + kWG - 1) / kWG, M), kWG, 0, (hipStream_t)stream>>>(sumsq, resid, norm_w,
                                                                                      x_out, M, K, G, eps, K);
  return mi_hip((int)hipGetLastError(), "norm_finish");
}
int mi_norm_finish_ex(const float* sumsq, const uint16_t* resid, const float* norm_w, uint16_t* x_out,
                      size_t x_stride, uint32_t M, uint32_t K, uint32_t G, float eps, void* stream) {
  if (!sumsq || !resid || !norm_w || !x_out || G == 0 || M == 0 || K == 0 || x_stride < K)
    return mi_fail(MI_ERR_ARG, "norm_finish_ex: bad arguments (x_stride >= K)");
  norm_finish_kernel<<<dim3((K + kWG - 1) / kWG, M), kWG, 0, (hipStream_t)stream>>>(sumsq, resid, norm_w,
                                                                                      x_out, M, K, G, eps, x_stride);
  return mi_hip((int)hipGetLastError(), "norm_finish_ex");
}
int mi_res_norm(const float* partials, uint16_t* resid, const float* norm_w, uint16_t* x_out, uint32_t M,
                uint32_t K, uint32_t S_PREV, float eps, void* stream) {
  if (!resid || !norm_w || !x_out || (S_PREV && !partials) || M == 0 || K == 0)
    return mi_fail(MI_ERR_ARG, "res_norm: bad arguments");
  res_norm_kernel<<<M, kWG, 0, (hipStream_t)stream>>>(partials, resid, norm_w, x_out, M, K, S_PREV, eps);
  return mi_hip((int)hipGetLastError(), "res_norm");
}
int mi_silu_mul(const float* partials, uint16_t* x_out, uint32_t M, uint32_t N, uint32_t S, void* stream) {
  if (!partials || !x_out || S == 0 || M == 0 || N == 0 || N % 16)
    return mi_fail(MI_ERR_ARG, "silu_mul: bad arguments (N must be a multiple of 16)");
  silu_mul_kernel<<<dim3((N + kWG - 1) / kWG, M), kWG, 0, (hipStream_t)stream>>>(partials, x_out, M, N, S);
  return mi_hip((int)hipGetLastError(), "silu_mul");
}

int mi_attn_prep(uint32_t* ctrl, const float* partials, uint32_t S, uint32_t M,
                 const mi_attn_shape* shape, const float* q_norm, const float* k_norm, const float* rope,
                 float* attn_q, float* attn_gate, uint16_t* kv_k, uint16_t* kv_v, size_t row_stride,
                 size_t head_stride, const uint32_t* pages, uint32_t page, uint32_t kv_len, void* stream) {
  if (!ctrl || !partials || !shape || !rope || !attn_q || !kv_k || !kv_v || S == 0 || M == 0)
    return mi_fail(MI_ERR_ARG, "attn_prep: bad arguments");
  const uint32_t HD = shape->head_dim;
  if (HD != 64 && HD != 128 && HD != 256)
    return mi_fail(MI_ERR_SHAPE, "attn_prep: head_dim must be 64, 128 or 256");
  if (shape->rot_dim > HD || shape->rot_dim % 2 || shape->q_heads == 0 || shape->kv_heads == 0 ||
      shape->q_heads % shape->kv_heads)
    return mi_fail(MI_ERR_SHAPE, "attn_prep: inconsistent heads / rotary dims");
  if (pages && (page == 0 || page % 16))
    return mi_fail(MI_ERR_SHAPE, "attn_prep: a KV page holds a multiple of 16 positions");
  AttnPrepArgs a{ctrl, partials, q_norm, k_norm, rope, attn_q, attn_gate, kv_k, kv_v, pages, row_stride,
                 head_stride, page, S, M, shape->q_heads, shape->kv_heads, HD, shape->rot_dim,
                 shape->gated, shape->qkv_n, shape->k_off, shape->v_off, kv_len, shape->eps,
                 nullptr, nullptr, 0, 0, shape->act};
  if (shape->act > 1) return mi_fail(MI_ERR_ARG, "attn_prep: act is 0 (f16) or 1 (bf16)");
  attn_prep_kernel<false><<<dim3(shape->q_heads + shape->kv_heads, M), HD, 0, (hipStream_t)stream>>>(a);
  return mi_hip((int)hipGetLastError(), "attn_prep");
}

int mi_attn_prep_kv8(uint32_t* ctrl, const float* partials, uint32_t S, uint32_t M,
                     const mi_attn_shape* shape, const float* q_norm, const float* k_norm, const float* rope,
                     float* attn_q, float* attn_gate, int8_t* kv_k, int8_t* kv_v, uint16_t* k_scale,
                     uint16_t* v_scale, size_t row_stride, size_t head_stride, size_t sc_row_stride,
                     size_t sc_head_stride, const uint32_t* pages, uint32_t page, uint32_t kv_len,
                     void* stream) {
  if (!ctrl || !partials || !shape || !rope || !attn_q || !kv_k || !kv_v || !k_scale || !v_scale || S == 0 ||
      M == 0)
    return mi_fail(MI_ERR_ARG, "attn_prep_kv8: bad arguments");
  if (shape->head_dim != 256)
    return mi_fail(MI_ERR_SHAPE, "attn_prep_kv8: the rotation is defined for head_dim 256 only");
  if (shape->rot_dim > 256 || shape->rot_dim % 2 || shape->q_heads == 0 || shape->kv_heads == 0 ||
      shape->q_heads % shape->kv_heads)
    return mi_fail(MI_ERR_SHAPE, "attn_prep_kv8: inconsistent heads / rotary dims");
  if (pages && (page == 0 || page % 16))
    return mi_fail(MI_ERR_SHAPE, "attn_prep_kv8: a KV page holds a multiple of 16 positions");
  AttnPrepArgs a{ctrl, partials, q_norm, k_norm, rope, attn_q, attn_gate,
                 reinterpret_cast<uint16_t*>(kv_k), reinterpret_cast<uint16_t*>(kv_v), pages, row_stride,
                 head_stride, page, S, M, shape->q_heads, shape->kv_heads, 256, shape->rot_dim,
                 shape->gated, shape->qkv_n, shape->k_off, shape->v_off, kv_len, shape->eps,
                 k_scale, v_scale, sc_row_stride, sc_head_stride, 0u};
  if (shape->act) return mi_fail(MI_ERR_SHAPE, "attn_prep_kv8: f16 activations only");
  attn_prep_kernel<true><<<dim3(shape->q_heads + shape->kv_heads, M), 256, 0, (hipStream_t)stream>>>(a);
  return mi_hip((int)hipGetLastError(), "attn_prep_kv8");
}

int mi_embed_gather(uint32_t* ctrl, const uint16_t* embed, uint16_t* resid, uint32_t M, uint32_t hidden,
                    uint32_t vocab, void* stream) {
  if (!ctrl || !embed || !resid || M == 0 || M > 8)
    return mi_fail(MI_ERR_ARG, "embed_gather: bad arguments (M <= 8)");
  embed_gather_kernel<<<M, kWG, 0, (hipStream_t)stream>>>(ctrl, embed, resid, hidden, vocab);
  return mi_hip((int)hipGetLastError(), "embed_gather");
}

int mi_embed_norm(uint32_t* ctrl, const uint16_t* embed, uint16_t* resid, const float* norm_w, uint16_t* x_out,
                  float* rstd, uint32_t M, uint32_t hidden, uint32_t vocab, float eps, void* stream) {
  if (!ctrl || !embed || !resid || !norm_w || !x_out || M == 0 || M > 8 || hidden % 64 || hidden > 65536)
    return mi_fail(MI_ERR_ARG, "embed_norm: bad arguments (M <= 8, hidden a multiple of 64)");
  embed_norm_kernel<true><<<M, kWG, 0, (hipStream_t)stream>>>(ctrl, embed, resid, norm_w, x_out, rstd, hidden,
                                                               vocab, eps, 0u);
  return mi_hip((int)hipGetLastError(), "embed_norm");
}

int mi_embed_norm_act(uint32_t* ctrl, const uint16_t* embed, uint16_t* resid, const float* norm_w, uint16_t* x_out,
                      float* rstd, uint32_t M, uint32_t hidden, uint32_t vocab, float eps, uint32_t act,
                      void* stream) {
  if (!ctrl || !embed || !resid || !norm_w || !x_out || M == 0 || M > 8 || hidden % 64 || hidden > 65536 || act > 1)
    return mi_fail(MI_ERR_ARG, "embed_norm_act: bad arguments (M <= 8, hidden a multiple of 64, act 0 or 1)");
  embed_norm_kernel<true><<<M, kWG, 0, (hipStream_t)stream>>>(ctrl, embed, resid, norm_w, x_out, rstd, hidden,
                                                               vocab, eps, act);
  return mi_hip((int)hipGetLastError(), "embed_norm_act");
}

int mi_norm_rows(const uint16_t* resid, const float* norm_w, uint16_t* x_out, float* rstd, uint32_t M,
                 uint32_t hidden, float eps, void* stream) {
  if (!resid || !norm_w || !x_out || M == 0 || M > 16 || hidden % 64 || hidden > 65536)
    return mi_fail(MI_ERR_ARG, "norm_rows: bad arguments (M <= 16, hidden a multiple of 64)");
  embed_norm_kernel<false><<<M, kWG, 0, (hipStream_t)stream>>>(nullptr, nullptr, const_cast<uint16_t*>(resid),
                                                                norm_w, x_out, rstd, hidden, 0, eps, 0u);
  return mi_hip((int)hipGetLastError(), "norm_rows");
}

uint32_t mi_argmax_groups(uint32_t vocab) { return (vocab + kChunk - 1) / kChunk; }

int mi_argmax_finish(uint32_t* ctrl, const void* part, uint32_t groups, uint32_t* history, uint32_t history_len,
                     void* stream) {
  if (!ctrl || !part || groups == 0) return mi_fail(MI_ERR_ARG, "argmax_finish: bad arguments");
  argmax_stage2_kernel<<<1, kWG, 0, (hipStream_t)stream>>>(ctrl, (const u2_t*)part, history, history_len, groups);
  return mi_hip((int)hipGetLastError(), "argmax_finish");
}

int mi_argmax(uint32_t* ctrl, const float* logits, void* part, uint32_t* history, uint32_t history_len,
              uint32_t M, uint32_t vocab, uint32_t vocab_used, void* stream) {
  if (!ctrl || !logits || !part || M == 0 || M > 8 || vocab == 0 || vocab_used > vocab)
    return mi_fail(MI_ERR_ARG, "argmax: bad arguments");
  const uint32_t groups = mi_argmax_groups(vocab);
  argmax_stage1_kernel<<<dim3(groups, M), kWG, 0, (hipStream_t)stream>>>(ctrl, logits, (u2_t*)part, vocab,
                                                                         vocab_used, groups);
  int e = (int)hipGetLastError();
  if (e) return mi_hip(e, "argmax_stage1");
  argmax_stage2_kernel<<<1, kWG, 0, (hipStream_t)stream>>>(ctrl, (const u2_t*)part, history, history_len,
                                                            groups);
  return mi_hip((int)hipGetLastError(), "argmax_stage2");
}

}  // extern "C"

// ---- mi_argmax_static: mi_argmax's two stages with the chunk winners in a file-scope device
// array instead of a caller buffer, for callers that cannot allocate. ----
namespace {
constexpr uint32_t kArgmaxScratchMax = 8192;  // (value, index) pairs: groups * M at most (64 KiB)
// Each GPU holds its own copy at its own address; the host learns it with hipGetSymbolAddress.
static __device__ __align__(256) u2_t scratch[kArgmaxScratchMax];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

extern "C" int mi_argmax_static(uint32_t* ctrl, const float* logits, uint32_t* history, uint32_t history_len,
                                uint32_t M, uint32_t vocab, uint32_t vocab_used, void* stream) {
  if (!ctrl || !logits || M == 0 || M > 8 || vocab == 0 || vocab_used > vocab)
    return mi_fail(MI_ERR_ARG, "argmax_static: bad arguments");
  const uint32_t groups = mi_argmax_groups(vocab);
  if ((size_t)groups * M > kArgmaxScratchMax)
    return mi_fail(MI_ERR_SHAPE, "argmax_static: ceil(vocab / 1024) * M exceeds the 8192-entry device scratch");
  int dev = 0;
  if (int e = (int)hipGetDevice(&dev)) return mi_hip(e, "argmax_static: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return mi_fail(MI_ERR_STATE, "argmax_static: device index out of range");
  void* part = nullptr;
  {
    // once per device, with that device current: the address of this device's copy
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
      void* p = nullptr;
      if (int e = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) return mi_hip(e, "argmax_static: hipGetSymbolAddress");
      g_scratch_ptr[dev] = p;
    }
    part = g_scratch_ptr[dev];
  }
  // stage 1 writes every (row, chunk) winner that stage 2 reads, so nothing needs clearing
  argmax_stage1_kernel<<<dim3(groups, M), kWG, 0, (hipStream_t)stream>>>(ctrl, logits, (u2_t*)part, vocab,
                                                                         vocab_used, groups);
  int e = (int)hipGetLastError();
  if (e) return mi_hip(e, "argmax_static stage1");
  argmax_stage2_kernel<<<1, kWG, 0, (hipStream_t)stream>>>(ctrl, (const u2_t*)part, history, history_len,
                                                            groups);
  return mi_hip((int)hipGetLastError(), "argmax_static stage2");
}
