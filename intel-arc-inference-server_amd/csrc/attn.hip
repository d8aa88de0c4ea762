// attn.hip - GQA decode attention over a (paged) fp16 or int8 KV cache, on gfx950.
//
// Replaces `attn_decode_v2` / `attn_reduce_v2` (src/kernels/attn_v2.cl:172, :383) and the
// int8 reader `attn_decode_v2_kv8` (src/kernels/kv8.cl:535) with the reference's contract:
//   * row m of a step attends to keys [0, pos + m]; the keys are cut into blocks of
//     ppw(L) = max(64, roundup64(ceil(L / tgt))) positions (attn_v2.cl:138-142) and the
//     grid is (kv_heads, tgt, M): at most `tgt` blocks per row for any L;
//   * each block leaves a partial {mx, sm, acc[HD]} per (q head, row) at
//     attn_part[qh][tgt][M][HD + 2]; the reduce merges a row's nb = (pos+m)/ppw + 1 blocks
//     in ascending block order with the reference's formula and writes
//     rne(acc / sm) (or the gated rne(rne(o) * sigmoid(gate)));
//   * KV paging (attn_v2.cl:123-131): logical position p lives at cache row
//     pages[p / page] * page + p % page; element (row, kv head, d) at
//     row * row_stride + head * head_stride + d, so both the reference's [pos][kvh][hd]
//     layout and this build's head-major [kvh][rows][hd] are expressible;
//   * int8 KV (kv8.h:126): k = float(q8) * f16(scale[row][kvh]), exact in fp32.
//
// Inside a block the work is MI355X-shaped rather than the B70's waves of 16:
//   * one K or V row of HD dims is read by HD/8 lanes, 16 bytes (fp16) or 8 bytes (int8)
//     each - a 64-lane wave covers 4 (HD 128) or 2 (HD 256) positions with coalesced
//     256/512-byte row reads; the block's rows of one kv head are contiguous in the
//     head-major layout;
//   * all GQA q heads of the kv head share each K/V load (q held in registers, fp32);
//   * the block is walked in chunks of 256 positions: pass 1 writes the chunk's scores to
//     LDS, the chunk max updates the running max (an online softmax per chunk, not per
//     16-position wave), weights exp(s - m) go back to LDS, pass 2 accumulates
//     sum_p w_p v_p per lane; the position slots are merged at the end in a fixed order.
// Scores and the softmax are fp32; no atomics, so replays are bitwise.
#include "mi_capi_internal.h"
#include "mi_common.h"

namespace mi {
namespace {

constexpr uint32_t kChunkP = 256;  // positions per score chunk
constexpr uint32_t kGqaMax = 8;

__device__ __forceinline__ uint32_t v2_ppw(uint32_t len, uint32_t tgt) {
  uint32_t p = (len + tgt - 1) / tgt;
  p = (p + 63u) & ~63u;
  return p < 64u ? 64u : p;
}

__device__ __forceinline__ size_t kv_row(uint32_t p, const uint32_t* pages, uint32_t page) {
  return pages ? (size_t)pages[p / page] * page + p % page : (size_t)p;
}

struct AttnDecodeArgs {
  const uint32_t* ctrl;
  const float* attn_q;
  const void* kv_k;
  const void* kv_v;
  const uint16_t* k_scale;
  const uint16_t* v_scale;
  const uint32_t* pages;
  float* attn_part;
  size_t row_stride, head_stride, sc_row_stride, sc_head_stride;
  uint32_t page, M, q_heads, kv_heads, tgt;
  uint32_t kv_len;  // positions the cache holds; keys past it are never read (0 = unchecked)
  float scale;
};

// 8 consecutive KV elements of one row as fp32
template <int KV8>
__device__ __forceinline__ void load8(const void* base, const uint16_t* sc, size_t off, size_t soff,
                                      float (&v)[8]) {
  if constexpr (KV8 == 0) {
    const u4_t w = *reinterpret_cast<const u4_t*>(static_cast<const uint16_t*>(base) + off);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = h2f((uint16_t)(ws[i] & 0xFFFFu));
      v[2 * i + 1] = h2f((uint16_t)(ws[i] >> 16));
    }
  } else {
    const u2_t w = *reinterpret_cast<const u2_t*>(static_cast<const int8_t*>(base) + off);
    const float s = h2f(sc[soff]);
    const uint32_t ws[2] = {w.x, w.y};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)(int8_t)((ws[i / 4] >> (8 * (i % 4))) & 0xFFu) * s;
  }
}

// HD: head dim (128 or 256); LP = HD / 8 lanes per row; SLOTS = 256 / LP rows per pass.
template <int HD, int KV8>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnDecodeArgs a) {
  constexpr uint32_t LP = HD / 8, SLOTS = 256 / LP, WSLOTS = 64 / LP;
  __shared__ float sc[kGqaMax][kChunkP];
  __shared__ float st_alpha[kGqaMax], st_m[kGqaMax], st_l[kGqaMax];
  __shared__ float red[4][kGqaMax][HD];

  const uint32_t j = blockIdx.x, blk = blockIdx.y, m = blockIdx.z;
  const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const uint32_t slot = t / LP, dg = t % LP, d0 = dg * 8;
  const uint32_t n_act = a.ctrl[CTRL_NACT];
  if (m >= n_act) return;
  const uint32_t pos = a.ctrl[CTRL_POS];
  uint32_t L = pos + m + 1;
  if (a.kv_len && L > a.kv_len) L = a.kv_len;
  const uint32_t s = v2_ppw(L, a.tgt);
  uint32_t nb = (L - 1) / s + 1;
  if (nb > a.tgt) nb = a.tgt;
  if (blk >= nb) return;
  const uint32_t p_begin = blk * s, p_end = min(p_begin + s, L);
  const uint32_t gqa = a.q_heads / a.kv_heads;

  float q[kGqaMax][8];
#pragma unroll
  for (uint32_t g = 0; g < kGqaMax; ++g) {
    if (g < gqa) {
      const float* qp = a.attn_q + ((size_t)m * a.q_heads + j * gqa + g) * HD + d0;
      const f4_t q0 = *reinterpret_cast<const f4_t*>(qp);
      const f4_t q1 = *reinterpret_cast<const f4_t*>(qp + 4);
      q[g][0] = q0.x; q[g][1] = q0.y; q[g][2] = q0.z; q[g][3] = q0.w;
      q[g][4] = q1.x; q[g][5] = q1.y; q[g][6] = q1.z; q[g][7] = q1.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) q[g][i] = 0.f;
    }
  }
  float acc[kGqaMax][8];
#pragma unroll
  for (uint32_t g = 0; g < kGqaMax; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  if (t < kGqaMax) {
    st_m[t] = -INFINITY;
    st_l[t] = 0.f;
  }

  const size_t hoff = (size_t)j * a.head_stride + d0;
  const size_t shoff = (size_t)j * a.sc_head_stride;
  for (uint32_t c0 = p_begin; c0 < p_end; c0 += kChunkP) {
    const uint32_t clen = min(kChunkP, p_end - c0);
    // pass 1: scores of the chunk
    for (uint32_t pl = slot; pl < clen; pl += SLOTS) {
      const size_t row = kv_row(c0 + pl, a.pages, a.page);
      float k[8];
      load8<KV8>(a.kv_k, a.k_scale, row * a.row_stride + hoff, row * a.sc_row_stride + shoff, k);
#pragma unroll
      for (uint32_t g = 0; g < kGqaMax; ++g) {
        if (g < gqa) {
          float d = 0.f;
#pragma unroll
          for (int i = 0; i < 8; ++i) d = __builtin_fmaf(q[g][i], k[i], d);
#pragma unroll
          for (uint32_t o = LP / 2; o > 0; o >>= 1) d += __shfl_xor(d, o, 64);
          if (dg == 0) sc[g][pl] = d * a.scale;
        }
      }
    }
    __syncthreads();
    // chunk max, weights and chunk sum: wave w owns heads w, w + 4
    for (uint32_t g = wave; g < gqa; g += 4) {
      float mx = -INFINITY;
      for (uint32_t p = lane; p < clen; p += 64) mx = fmaxf(mx, sc[g][p]);
#pragma unroll
      for (uint32_t o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
      const float m_old = st_m[g];
      const float m_new = fmaxf(m_old, mx);
      float sum = 0.f;
      for (uint32_t p = lane; p < clen; p += 64) {
        const float w = expf(sc[g][p] - m_new);
        sc[g][p] = w;
        sum += w;
      }
#pragma unroll
      for (uint32_t o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
      if (lane == 0) {
        const float alpha = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
        st_alpha[g] = alpha;
        st_l[g] = __builtin_fmaf(st_l[g], alpha, sum);
        st_m[g] = m_new;
      }
    }
    __syncthreads();
    // pass 2: rescale, then accumulate w * v
#pragma unroll
    for (uint32_t g = 0; g < kGqaMax; ++g) {
      if (g < gqa) {
        const float al = st_alpha[g];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] *= al;
      }
    }
    for (uint32_t pl = slot; pl < clen; pl += SLOTS) {
      const size_t row = kv_row(c0 + pl, a.pages, a.page);
      float v[8];
      load8<KV8>(a.kv_v, a.v_scale, row * a.row_stride + hoff, row * a.sc_row_stride + shoff, v);
#pragma unroll
      for (uint32_t g = 0; g < kGqaMax; ++g) {
        if (g < gqa) {
          const float w = sc[g][pl];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] = __builtin_fmaf(w, v[i], acc[g][i]);
        }
      }
    }
    __syncthreads();
  }
  // merge the position slots: within the wave (xor over the slot bits), then the 4 waves
#pragma unroll
  for (uint32_t g = 0; g < kGqaMax; ++g) {
    if (g < gqa) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v = acc[g][i];
#pragma unroll
        for (uint32_t o = LP; o < 64; o <<= 1) v += __shfl_xor(v, o, 64);
        acc[g][i] = v;
      }
      if (lane < LP) {
#pragma unroll
        for (int i = 0; i < 8; ++i) red[wave][g][d0 + i] = acc[g][i];
      }
    }
  }
  (void)WSLOTS;
  __syncthreads();
  for (uint32_t idx = t; idx < gqa * HD; idx += 256) {
    const uint32_t g = idx / HD, d = idx % HD;
    const float v = ((red[0][g][d] + red[1][g][d]) + red[2][g][d]) + red[3][g][d];
    float* out = a.attn_part + (((size_t)(j * gqa + g) * a.tgt + blk) * a.M + m) * (HD + 2);
    out[2 + d] = v;
    if (d == 0) {
      out[0] = st_m[g];
      out[1] = st_l[g];
    }
  }
}

// grid (q_heads, M), HD lanes: attn_v2.cl:383-428.
__global__ __launch_bounds__(256) void attn_reduce_kernel(const uint32_t* __restrict__ ctrl,
                                                          const float* __restrict__ attn_part,
                                                          const float* __restrict__ attn_gate,
                                                          uint16_t* __restrict__ attn_out, uint32_t M,
                                                          uint32_t q_heads, uint32_t HD, uint32_t tgt,
                                                          uint32_t gated) {
  const uint32_t h = blockIdx.x, m = blockIdx.y, d = threadIdx.x;
  if (m >= ctrl[CTRL_NACT]) return;
  const uint32_t pos = ctrl[CTRL_POS];
  uint32_t nb = (pos + m) / v2_ppw(pos + m + 1, tgt) + 1;
  if (nb > tgt) nb = tgt;
  float mx = -INFINITY, sm = 0.f, acc = 0.f;
  const size_t PART = HD + 2;
  for (uint32_t b = 0; b < nb; ++b) {
    const float* p = attn_part + (((size_t)h * tgt + b) * M + m) * PART;
    const float bmx = p[0], bsm = p[1], bacc = p[2 + d];
    const float nmx = fmaxf(mx, bmx);
    const float al = expf(mx - nmx);
    const float bs = expf(bmx - nmx);
    sm = __builtin_fmaf(sm, al, bsm * bs);
    acc = __builtin_fmaf(acc, al, bacc * bs);
    mx = nmx;
  }
  const float o = acc / sm;
  uint16_t r;
  if (gated && attn_gate)
    r = f2h(h2f(f2h(o)) * sigmoid_f32(attn_gate[((size_t)m * q_heads + h) * HD + d]));
  else
    r = f2h(o);
  attn_out[(size_t)m * q_heads * HD + (size_t)h * HD + d] = r;
}

}  // namespace
}  // namespace mi

using namespace mi;

extern "C" {

uint32_t mi_attn_ppw(uint32_t len, uint32_t tgt) {
  uint32_t p = (len + tgt - 1) / tgt;
  p = (p + 63u) & ~63u;
  return p < 64u ? 64u : p;
}

int mi_attn_decode(const uint32_t* ctrl, const float* attn_q, uint32_t kv_kind, const void* kv_k,
                   const void* kv_v, const uint16_t* k_scale, const uint16_t* v_scale, size_t row_stride,
                   size_t head_stride, size_t sc_row_stride, size_t sc_head_stride, const uint32_t* pages,
                   uint32_t page, uint32_t kv_len, float* attn_part, uint32_t M, uint32_t tgt,
                   const mi_attn_shape* shape, void* stream) {
  if (!ctrl || !attn_q || !kv_k || !kv_v || !attn_part || !shape || M == 0 || M > 16 || tgt == 0)
    return mi_fail(MI_ERR_ARG, "attn_decode: bad arguments");
  if (kv_kind > 1 || (kv_kind == 1 && (!k_scale || !v_scale)))
    return mi_fail(MI_ERR_ARG, "attn_decode: kv_kind 0 (fp16) or 1 (int8 + fp16 scales)");
  const uint32_t HD = shape->head_dim;
  if (HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_decode: head_dim must be 128 or 256");
  if (shape->kv_heads == 0 || shape->q_heads % shape->kv_heads || shape->q_heads / shape->kv_heads > kGqaMax)
    return mi_fail(MI_ERR_SHAPE, "attn_decode: q_heads / kv_heads must be an integer <= 8");
  if (pages && (page == 0 || page % 16))
    return mi_fail(MI_ERR_SHAPE, "attn_decode: a KV page holds a multiple of 16 positions");
  if ((row_stride % 8) || (head_stride % 8))
    return mi_fail(MI_ERR_ARG, "attn_decode: KV strides must keep 8-element alignment");
  AttnDecodeArgs a{ctrl,  attn_q,       kv_k,           kv_v,   k_scale,         v_scale,
                   pages, attn_part,    row_stride,     head_stride, sc_row_stride, sc_head_stride,
                   page,  M,            shape->q_heads, shape->kv_heads, tgt,    kv_len,
                   shape->scale};
  dim3 grid(shape->kv_heads, tgt, M);
  hipStream_t st = (hipStream_t)stream;
  if (HD == 128) {
    if (kv_kind == 0) attn_decode_kernel<128, 0><<<grid, 256, 0, st>>>(a);
    else attn_decode_kernel<128, 1><<<grid, 256, 0, st>>>(a);
  } else {
    if (kv_kind == 0) attn_decode_kernel<256, 0><<<grid, 256, 0, st>>>(a);
    else attn_decode_kernel<256, 1><<<grid, 256, 0, st>>>(a);
  }
  return mi_hip((int)hipGetLastError(), "attn_decode");
}

int mi_attn_reduce(const uint32_t* ctrl, const float* attn_part, const float* attn_gate, uint16_t* attn_out,
                   uint32_t M, uint32_t tgt, const mi_attn_shape* shape, void* stream) {
  if (!ctrl || !attn_part || !attn_out || !shape || M == 0 || tgt == 0)
    return mi_fail(MI_ERR_ARG, "attn_reduce: bad arguments");
  const uint32_t HD = shape->head_dim;
  if (HD != 64 && HD != 128 && HD != 256) return mi_fail(MI_ERR_SHAPE, "attn_reduce: head_dim 64/128/256");
  attn_reduce_kernel<<<dim3(shape->q_heads, M), HD, 0, (hipStream_t)stream>>>(
      ctrl, attn_part, attn_gate, attn_out, M, shape->q_heads, HD, tgt, shape->gated);
  return mi_hip((int)hipGetLastError(), "attn_reduce");
}

}  // extern "C"
