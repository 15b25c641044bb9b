// prefill.hip - the prompt prefill on the device: S rows through the decoder
// with each weight matrix streamed once per block of rows (Qwen3Decoder::prefill,
// src/qwen3_decoder.cpp:162-166, which runs the fused prompt as one batch).
//
// The verify path processes at most 16 rows per weight pass; a 1,600-row prompt
// through it costs 100 full weight streams. Here every layer is a short
// sequence of kernels over all rows of a block (up to kPfRows):
//   k_pf_norm_quant  RMSNorm * gain and the q8_0 activation conversion, compact
//                    layout: codes [S][K] int8, scales [S][K/32] (f16 values)
//   k_pf_gemm        q8_0 weight tiles x activation rows on v_mfma_i32_16x16x64_i8
//                    (block-diagonal B operand: two exact per-block int32 dots per
//                    MFMA), epilogue store / residual add / SwiGLU
//   k_pf_quant       q8_0 conversion of f32 rows (the SwiGLU output)
//   k_pf_qk_rope     q/k RMSNorm + NEOX RoPE, K/V written into the cache
//   k_pf_attn        causal attention of 16 query rows x 2 q heads per
//                    workgroup over the cache, in two passes over the 64-key
//                    chunks, writing the o-projection's q8_0 activation
// Every reduction follows the canonical order of device_common.hpp, so hidden
// rows and the KV cache equal the verify path's and the oracle's bit for bit:
//   * GEMM: per output, 4 K-slices of block pairs, even / odd fma chains per
//     slice in block order, ((s0 + s1) + s2) + s3 per parity, then even + odd;
//   * attention: pass 1 takes every chunk's column maxima m_c (exact in any
//     order) and M = max m_c; pass 2 recomputes the scores, p = exp(w - m_c),
//     l_c = butterfly sum, O_c = fma chain over the chunk's keys, and merges in
//     chunk order, L = fma(l_c, f_c, L), O = fma(O_c, f_c, O), f_c = exp(m_c - M)
//     -- the same fma chains the verify path's merge runs, without storing the
//     per-chunk partials.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "device_common.hpp"

namespace mtg {
namespace {
using namespace dev;

constexpr int kH = 1024;         // hidden (the RMSNorm partials assume 1024)
constexpr int kPfQStride = 132;  // LDS row strides (floats)
constexpr int kPfPStride = 68;

// ---------------------------------------------------------- activations ----
// One wave per row of 1024: lane l holds elements 16 l .. 16 l + 15 (the
// canonical RMSNorm partials); q8_0 blocks are lanes (2 b, 2 b + 1).
__global__ void __launch_bounds__(256)
k_pf_norm_quant(const float* __restrict__ src, int S, const float* __restrict__ gain, float eps,
                int8_t* __restrict__ codes, float* __restrict__ scales, float* __restrict__ normed_out) {
  const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= S) return;
  const float* xr = src + (size_t)row * kH + 16 * lane;
  float v[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const v4f q = *(const v4f*)(xr + 4 * i);
    v[4 * i] = q[0];
    v[4 * i + 1] = q[1];
    v[4 * i + 2] = q[2];
    v[4 * i + 3] = q[3];
  }
  double s = 0.0;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += (double)__fmul_rn(v[e], v[e]);
  s = wave_sum_d(s);
  const float scale = dev_rms_scale((float)(s / (double)kH), eps);
  float y[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) y[e] = __fmul_rn(__fmul_rn(v[e], scale), gain[16 * lane + e]);
  if (normed_out) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v4f o = {y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]};
      *(v4f*)(normed_out + (size_t)row * kH + 16 * lane + 4 * i) = o;
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(y[e]));
  amax = __uint_as_float(max(__float_as_uint(amax), dpp_u<kDppQuadXor1>(__float_as_uint(amax))));
  const float d = __fdiv_rn(amax, 127.0f);
  const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
  uint32_t packed[4];
#pragma unroll
  for (int w4 = 0; w4 < 4; ++w4) {
    uint32_t u = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) u |= (uint32_t)(uint8_t)(int8_t)rintf(__fmul_rn(y[4 * w4 + b], id)) << (8 * b);
    packed[w4] = u;
  }
  *(uint4*)(codes + (size_t)row * kH + 16 * lane) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  if ((lane & 1) == 0) scales[(size_t)row * (kH / 32) + lane / 2] = __half2float(__float2half_rn(d));
}

// q8_0 conversion of f32 rows of K (a multiple of 32): one wave per row, lane =
// one 32-element block at a time.
__global__ void __launch_bounds__(256)
k_pf_quant(const float* __restrict__ src, int S, int K, int8_t* __restrict__ codes, float* __restrict__ scales) {
  const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= S) return;
  for (int b = lane; b < K / 32; b += 64) {
    const float* xr = src + (size_t)row * K + 32 * b;
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const v4f q = *(const v4f*)(xr + 4 * i);
      v[4 * i] = q[0];
      v[4 * i + 1] = q[1];
      v[4 * i + 2] = q[2];
      v[4 * i + 3] = q[3];
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) amax = fmaxf(amax, fabsf(v[e]));
    const float d = __fdiv_rn(amax, 127.0f);
    const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    uint32_t packed[8];
#pragma unroll
    for (int w4 = 0; w4 < 8; ++w4) {
      uint32_t u = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) u |= (uint32_t)(uint8_t)(int8_t)rintf(__fmul_rn(v[4 * w4 + e], id)) << (8 * e);
      packed[w4] = u;
    }
    uint4* dst = (uint4*)(codes + (size_t)row * K + 32 * b);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    scales[(size_t)row * (K / 32) + b] = __half2float(__float2half_rn(d));
  }
}

// ----------------------------------------------------------------- GEMM ----
// out[s][n] for weight tiles tile0 .. tile0 + TPW - 1 (16 rows each) and the 64
// activation rows of blockIdx.y; wave w takes rows s0 + 16 w .. + 15 as two
// column groups of 8. Per block pair the lane's B operand holds 16 code bytes of
// row (8 cg + j % 8), block 2 bp + j / 8, when (lane / 16) / 2 == j / 8 (j =
// lane % 16), else zeros, so each MFMA returns the exact int32 dot of every
// (weight row, activation row, block). EPI_SWIGLU: TPW tiles of w (gate) and the
// same TPW tiles of w2 (up).
enum { PF_STORE = 0, PF_RESID = 1, PF_SWIGLU = 2 };

template <int EPI, int TPW>
__global__ void __launch_bounds__(256)
k_pf_gemm(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, int N, int K,
          const int8_t* __restrict__ codes, const float* __restrict__ scales, int S, float* __restrict__ out) {
  constexpr int NM = EPI == PF_SWIGLU ? 2 : 1;
  constexpr int NT = NM * TPW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tile0 = blockIdx.x * TPW;
  const int s0 = blockIdx.y * 64 + 16 * wave;
  const int bps = K / kPairK;
  const int j = lane & 15, g = lane >> 4, par = j >> 3;
  const bool holds = (g >> 1) == par;
  const int srow = par * 16 + 4 * (lane >> 4);
  int rows[2];
  bool rin[2];
#pragma unroll
  for (int cg = 0; cg < 2; ++cg) {
    rows[cg] = s0 + 8 * cg + (j & 7);
    rin[cg] = rows[cg] < S;
  }
  const v4i zero = {0, 0, 0, 0};
  float part[4][NT][2][4];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl)
#pragma unroll
    for (int m = 0; m < NT; ++m)
#pragma unroll
      for (int cg = 0; cg < 2; ++cg)
#pragma unroll
        for (int q = 0; q < 4; ++q) part[sl][m][cg][q] = 0.0f;
#pragma unroll
  for (int sl = 0; sl < 4; ++sl) {
    const int bp1 = (bps * (sl + 1)) / 4;
#pragma unroll 2
    for (int bp = (bps * sl) / 4; bp < bp1; ++bp) {
      v4i b[2];
      float dx[2];
#pragma unroll
      for (int cg = 0; cg < 2; ++cg) {
        b[cg] = (holds && rin[cg])
                    ? *(const v4i*)(codes + (size_t)rows[cg] * K + 64 * bp + 32 * par + 16 * (g & 1))
                    : zero;
        dx[cg] = rin[cg] ? scales[(size_t)rows[cg] * (K / 32) + 2 * bp + par] : 0.0f;
      }
#pragma unroll
      for (int m = 0; m < NT; ++m) {
        const uint8_t* mat = m < TPW ? w : w2;
        const uint8_t* unit = mat + ((size_t)(tile0 + m % TPW) * bps + bp) * kUnitBytes;
        const v4i a = __builtin_nontemporal_load((const v4i*)(unit + lane * 16));
        const uint2 sw = *(const uint2*)(unit + 1024 + srow * 2);
        float dw[4];
        dw[0] = half_bits_to_float((uint16_t)(sw.x & 0xffff));
        dw[1] = half_bits_to_float((uint16_t)(sw.x >> 16));
        dw[2] = half_bits_to_float((uint16_t)(sw.y & 0xffff));
        dw[3] = half_bits_to_float((uint16_t)(sw.y >> 16));
#pragma unroll
        for (int cg = 0; cg < 2; ++cg) {
          const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[cg], zero, 0, 0, 0);
#pragma unroll
          for (int q = 0; q < 4; ++q) part[sl][m][cg][q] = fmaf((float)c[q], dw[q] * dx[cg], part[sl][m][cg][q]);
        }
      }
    }
  }
  float acc[NT][2][4];
#pragma unroll
  for (int m = 0; m < NT; ++m)
#pragma unroll
    for (int cg = 0; cg < 2; ++cg)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float v = __fadd_rn(__fadd_rn(__fadd_rn(part[0][m][cg][q], part[1][m][cg][q]), part[2][m][cg][q]),
                                  part[3][m][cg][q]);
        acc[m][cg][q] = __fadd_rn(v, dpp_f<kDppRor8>(v));  // even + odd parity
      }
  if (j < 8) {
#pragma unroll
    for (int cg = 0; cg < 2; ++cg) {
      if (!rin[cg]) continue;
      const size_t rowoff = (size_t)rows[cg] * N;
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int n = (tile0 + t) * 16 + 4 * (lane >> 4);
        v4f v;
        if (EPI == PF_STORE) {
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = acc[t][cg][q];
        } else if (EPI == PF_RESID) {
          const v4f x = *(const v4f*)(out + rowoff + n);
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = __fadd_rn(x[q], acc[t][cg][q]);
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = dev_swiglu(acc[t][cg][q], acc[TPW + t][cg][q]);
        }
        *(v4f*)(out + rowoff + n) = v;
      }
    }
  }
}

// ------------------------------------------------- q/k norm, rope, append ---
// grid (S rows, n_heads + 2 n_kv_heads units), one wave per unit: the same
// arithmetic as the verify path's k_qk_rope_append at position past0 + row.
__global__ void __launch_bounds__(64)
k_pf_qk_rope(const float* __restrict__ qkv, int S, int past0, int n_heads, int n_kv_heads,
             const float* __restrict__ q_norm, const float* __restrict__ k_norm, float eps,
             const float* __restrict__ rope, float* __restrict__ q_out, KvLayer kv) {
  const int t = blockIdx.x;
  if (t >= S) return;
  const int u = blockIdx.y, i = threadIdx.x;
  const int QN = n_heads * kHeadDim, KN = n_kv_heads * kHeadDim, N = QN + 2 * KN;
  const int pos = past0 + t;
  const float* row = qkv + (size_t)t * N;
  const bool is_q = u < n_heads, is_k = !is_q && u < n_heads + n_kv_heads;
  const int col = is_q ? u * kHeadDim : is_k ? QN + (u - n_heads) * kHeadDim
                                             : QN + KN + (u - n_heads - n_kv_heads) * kHeadDim;
  float x0 = row[col + i], x1 = row[col + i + 64];
  if (is_q || is_k) {
    const float* gn = is_q ? q_norm : k_norm;
    double s = (double)__fmul_rn(x0, x0) + (double)__fmul_rn(x1, x1);
    s = wave_sum_d(s);
    const float scale = dev_rms_scale((float)(s / (double)kHeadDim), eps);
    const float y0 = __fmul_rn(__fmul_rn(x0, scale), gn[i]);
    const float y1 = __fmul_rn(__fmul_rn(x1, scale), gn[i + 64]);
    const float c = rope[(size_t)pos * kHeadDim + 2 * i], sn = rope[(size_t)pos * kHeadDim + 2 * i + 1];
    x0 = __fsub_rn(__fmul_rn(y0, c), __fmul_rn(y1, sn));
    x1 = __fadd_rn(__fmul_rn(y0, sn), __fmul_rn(y1, c));
  }
  if (is_q) {
    float* q = q_out + ((size_t)t * n_heads + u) * kHeadDim;
    q[i] = x0;
    q[i + 64] = x1;
    return;
  }
  const int h = is_k ? u - n_heads : u - n_heads - n_kv_heads;
  void* base = is_k ? kv.k : kv.v;
  const size_t off = ((size_t)h * kv.max_seq + pos) * kHeadDim;
  if (kv.f16) {
    __half* p = (__half*)base + off;
    p[i] = __float2half_rn(x0);
    p[i + 64] = __float2half_rn(x1);
  } else {
    float* p = (float*)base + off;
    p[i] = x0;
    p[i + 64] = x1;
  }
}

// ------------------------------------------------------------ attention ----
// grid (n_kv_heads, ceil(S / 16)): workgroup (g, qb) takes query rows
// r0 = 16 qb .. r0 + 15 (positions past0 + r0 + t) of q heads 2 g and 2 g + 1,
// columns col = 16 hl + t. Keys 0 .. past0 + r0 + 15 come from the cache (this
// block's rows were appended by k_pf_qk_rope). The output rows leave as the
// o-projection's q8_0 activation: codes [S][n_heads * 128], scales [S][n_heads * 4].
__device__ __forceinline__ int pf_perm128(int d) { return (d & 3) * 32 + (d >> 2); }

// K (and V) rows of chunk key0 into LDS as f32: K permuted (element 4 s + kk at
// kk * 32 + s), V plain; zeros past kvlen.
template <bool WITH_V>
__device__ __forceinline__ void pf_load_chunk(const KvLayer& kv, size_t head, int key0, int kvlen, float* s_k,
                                              float* s_v) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < kChunk * kHeadDim / 4 / 256; ++i) {
    const int idx = i * 256 + tid, jk = idx / (kHeadDim / 4), d = (idx % (kHeadDim / 4)) * 4;
    const int key = key0 + jk;
    const bool in = key < kvlen;
    const v4f kf = in ? kv_load4(kv.k, kv.f16, head + (size_t)key * kHeadDim + d) : (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) s_k[jk * kPfQStride + pf_perm128(d + e)] = kf[e];
    if (WITH_V) {
      const v4f vf = in ? kv_load4(kv.v, kv.f16, head + (size_t)key * kHeadDim + d) : (v4f){0.f, 0.f, 0.f, 0.f};
      *(v4f*)(s_v + jk * kPfQStride + d) = vf;
    }
  }
}

// Scores of keys 16 wave + 4 kk + r (r < 4) for columns 16 ct + kl, scaled and
// masked: acc[ct][r]. The fma chain over head_dim is 32 chained MFMAs.
__device__ __forceinline__ void pf_scores(const float* s_q, const float* s_k, int key0, int kvlen, int past0,
                                          int r0, int nq, float scale, float (&w)[2][4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kl = lane & 15, kk = lane >> 4;
  const float* krow = s_k + (16 * wave + kl) * kPfQStride + kk * 32;
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const float* qrow = s_q + (ct * 16 + kl) * kPfQStride + kk * 32;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const v4f k4 = *(const v4f*)(krow + 4 * i);
      const v4f q4 = *(const v4f*)(qrow + 4 * i);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[jj], q4[jj], acc, 0, 0, 0);
    }
    // the MFMA's column kl is this lane's column; rows are keys 16 wave + 4 kk + r
    const int t = kl;  // column 16 ct + kl is query row kl of head 2 g + ct
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = key0 + 16 * wave + 4 * kk + r;
      w[ct][r] = (t < nq && key < kvlen && key <= past0 + r0 + t) ? __fmul_rn(acc[r], scale) : -INFINITY;
    }
  }
}

constexpr int kPfMaxChunks = 320;  // 20,480 positions
constexpr size_t kPfAttnLds =
    ((size_t)32 * kPfQStride + 2 * (size_t)kChunk * kPfQStride + 32 * kPfPStride + (size_t)kPfMaxChunks * 32 +
     4 * 32 + 3 * 32) * 4;

__global__ void __launch_bounds__(256)
k_pf_attn(const float* __restrict__ q, int n_heads, KvLayer kv, int past0, int S, int8_t* __restrict__ ocodes,
          float* __restrict__ oscales) {
  const int g = blockIdx.x, r0 = blockIdx.y * 16;
  const int nq = min(16, S - r0);
  const int kvlen = past0 + S;
  const int last = past0 + r0 + nq - 1;  // the block's last query position
  const int nch = last / kChunk + 1;
  extern __shared__ v4f pf_lds_v4[];
  float* s_q = (float*)pf_lds_v4;                  // [32][132] permuted
  float* s_k = s_q + 32 * kPfQStride;              // [64][132] permuted
  float* s_v = s_k + kChunk * kPfQStride;          // [64][132]
  float* s_p = s_v + kChunk * kPfQStride;          // [32][68] permuted keys
  float* s_m = s_p + 32 * kPfPStride;              // [chunk][32] column maxima
  float* s_wm = s_m + kPfMaxChunks * 32;           // [4 waves][32]
  float* s_l = s_wm + 4 * 32;                      // [32] chunk sums
  float* s_f = s_l + 32;                           // [32] chunk factors
  float* s_M = s_f + 32;                           // [32] column maxima over all chunks
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, kl = lane & 15, kk = lane >> 4;
  const bool f16kv = kv.f16 != 0;
  // q rows (f16-rounded for an f16 cache: mul_mat(f16 K, f32 q) converts q)
  for (int idx = tid; idx < 32 * (kHeadDim / 4); idx += 256) {
    const int col = idx / (kHeadDim / 4), d = (idx % (kHeadDim / 4)) * 4, hl = col >> 4, t = col & 15;
    v4f v = {0.f, 0.f, 0.f, 0.f};
    if (t < nq) v = *(const v4f*)(q + ((size_t)(r0 + t) * n_heads + 2 * g + hl) * kHeadDim + d);
#pragma unroll
    for (int e = 0; e < 4; ++e) s_q[col * kPfQStride + pf_perm128(d + e)] = f16kv ? f16_round(v[e]) : v[e];
  }
  const size_t head = (size_t)g * kv.max_seq * kHeadDim;
  const float scale = __fdiv_rn(1.0f, dev_sqrtf((float)kHeadDim));
  // pass 1: chunk maxima per column
  for (int c = 0; c < nch; ++c) {
    __syncthreads();
    pf_load_chunk<false>(kv, head, c * kChunk, kvlen, s_k, s_v);
    __syncthreads();
    float w[2][4];
    pf_scores(s_q, s_k, c * kChunk, kvlen, past0, r0, nq, scale, w);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      int mk = max(max(ord_key(w[ct][0]), ord_key(w[ct][1])), max(ord_key(w[ct][2]), ord_key(w[ct][3])));
      uint32_t a, b;
      pair_split<16>((uint32_t)mk, a, b);  // lanes kk and kk ^ 1 (same column)
      mk = max((int)a, (int)b);
      pair_split<32>((uint32_t)mk, a, b);  // kk ^ 2
      mk = max((int)a, (int)b);
      if (kk == 0) s_wm[wave * 32 + ct * 16 + kl] = ord_val(mk);
    }
    __syncthreads();
    if (tid < 32)
      s_m[c * 32 + tid] = fmaxf(fmaxf(s_wm[tid], s_wm[32 + tid]), fmaxf(s_wm[64 + tid], s_wm[96 + tid]));
  }
  __syncthreads();
  if (tid < 32) {  // the columns' overall maxima (exact in any order)
    float M = -INFINITY;
    for (int c = 0; c < nch; ++c) M = fmaxf(M, s_m[c * 32 + tid]);
    s_M[tid] = M;
  }
  // pass 2: probabilities, chunk sums, P.V, merged in chunk order
  float O[2][2][4], L[2][4];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      L[ct][r] = 0.0f;
      O[ct][0][r] = O[ct][1][r] = 0.0f;
    }
  const int sp_pos = (lane & 3) * 16 + (lane >> 2);
  for (int c = 0; c < nch; ++c) {
    __syncthreads();
    pf_load_chunk<true>(kv, head, c * kChunk, kvlen, s_k, s_v);
    __syncthreads();
    float w[2][4];
    pf_scores(s_q, s_k, c * kChunk, kvlen, past0, r0, nq, scale, w);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r)  // key 16 wave + 4 kk + r sits at r * 16 + 4 wave + kk
        s_p[(ct * 16 + kl) * kPfPStride + r * 16 + 4 * wave + kk] = w[ct][r];
    __syncthreads();
    // chunk softmax per column (one wave per column, lane = key)
    for (int col = wave; col < 32; col += 4) {
      const float wv = s_p[col * kPfPStride + sp_pos];
      const float m = s_m[c * 32 + col];
      float p = (m == -INFINITY || wv == -INFINITY) ? 0.0f : dev_expf(__fsub_rn(wv, m));
      if (f16kv) p = f16_round(p);
      const float l = wave_sum_f(p);
      s_p[col * kPfPStride + sp_pos] = p;
      if (lane == 0) s_l[col] = l;
    }
    if (tid < 32) {
      const float m = s_m[c * 32 + tid];
      s_f[tid] = m == -INFINITY ? 0.0f : dev_expf(__fsub_rn(m, s_M[tid]));
    }
    __syncthreads();
    // O_c[col][d]: fma chain over the chunk's keys; wave w takes head_dim tiles 2w, 2w+1
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      float pa[16];
      const float* prow = s_p + (ct * 16 + kl) * kPfPStride + kk * 16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4f p4 = *(const v4f*)(prow + 4 * i);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) pa[4 * i + jj] = p4[jj];
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int d = 16 * (2 * wave + h) + kl;
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s2], s_v[(4 * s2 + kk) * kPfQStride + d], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float f = s_f[ct * 16 + 4 * kk + r];
          O[ct][h][r] = fmaf(acc[r], f, O[ct][h][r]);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = ct * 16 + 4 * kk + r;
        L[ct][r] = fmaf(s_l[col], s_f[col], L[ct][r]);
      }
    }
  }
  // out = O / L, then the q8_0 blocks of 32 head_dim elements (wave w: block w)
  const int QN = n_heads * kHeadDim;
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 4 * kk + r;  // query row of column 16 ct + 4 kk + r
      const float o0 = __fdiv_rn(O[ct][0][r], L[ct][r]);
      const float o1 = __fdiv_rn(O[ct][1][r], L[ct][r]);
      float amax = fmaxf(fabsf(o0), fabsf(o1));
      uint32_t u = __float_as_uint(amax);  // max over the 16 lanes kl of this row
      u = max(u, dpp_u<kDppRor8>(u));
      u = max(u, dpp_u<kDppRor4>(u));
      u = max(u, dpp_u<kDppRor2>(u));
      u = max(u, dpp_u<kDppRor1>(u));
      amax = __uint_as_float(u);
      if (t < nq) {
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        const size_t rowoff = (size_t)(r0 + t) * QN + (2 * g + ct) * kHeadDim;
        ocodes[rowoff + 32 * wave + kl] = (int8_t)rintf(__fmul_rn(o0, id));
        ocodes[rowoff + 32 * wave + 16 + kl] = (int8_t)rintf(__fmul_rn(o1, id));
        if (kl == 0)
          oscales[(size_t)(r0 + t) * (QN / 32) + ((2 * g + ct) * kHeadDim) / 32 + wave] =
              __half2float(__float2half_rn(__fdiv_rn(amax, 127.0f)));
      }
    }
}

}  // namespace

// ================================================================ launches ==
int pf_max_context() { return kPfMaxChunks * kChunk; }

void launch_pf_norm_quant(hipStream_t s, const float* src, int S, const float* gain, float eps, int8_t* codes,
                          float* scales, float* normed_out) {
  hipLaunchKernelGGL(k_pf_norm_quant, dim3((S + 3) / 4), dim3(256), 0, s, src, S, gain, eps, codes, scales,
                     normed_out);
}

void launch_pf_quant(hipStream_t s, const float* src, int S, int K, int8_t* codes, float* scales) {
  hipLaunchKernelGGL(k_pf_quant, dim3((S + 3) / 4), dim3(256), 0, s, src, S, K, codes, scales);
}

void launch_pf_gemm(hipStream_t s, int epi, const uint8_t* w, const uint8_t* w2, int N, int K, const int8_t* codes,
                    const float* scales, int S, float* out) {
  const dim3 blocks((unsigned)(N / 16 / 2), (unsigned)((S + 63) / 64));
  if (epi == PF_STORE)
    hipLaunchKernelGGL((k_pf_gemm<PF_STORE, 2>), blocks, dim3(256), 0, s, w, w2, N, K, codes, scales, S, out);
  else if (epi == PF_RESID)
    hipLaunchKernelGGL((k_pf_gemm<PF_RESID, 2>), blocks, dim3(256), 0, s, w, w2, N, K, codes, scales, S, out);
  else
    hipLaunchKernelGGL((k_pf_gemm<PF_SWIGLU, 2>), blocks, dim3(256), 0, s, w, w2, N, K, codes, scales, S, out);
}

void launch_pf_qk_rope(hipStream_t s, const float* qkv, int S, int past0, int n_heads, int n_kv_heads,
                       const float* q_norm, const float* k_norm, float eps, const float* rope, float* q_out,
                       KvLayer kv) {
  hipLaunchKernelGGL(k_pf_qk_rope, dim3((unsigned)S, (unsigned)(n_heads + 2 * n_kv_heads)), dim3(64), 0, s, qkv, S,
                     past0, n_heads, n_kv_heads, q_norm, k_norm, eps, rope, q_out, kv);
}

void launch_pf_attn(hipStream_t s, const float* q, int n_heads, int n_kv_heads, KvLayer kv, int past0, int S,
                    int8_t* ocodes, float* oscales) {
  hipLaunchKernelGGL(k_pf_attn, dim3((unsigned)n_kv_heads, (unsigned)((S + 15) / 16)), dim3(256), kPfAttnLds, s, q,
                     n_heads, kv, past0, S, ocodes, oscales);
}

hipError_t prepare_kernels_pf() {
  return hipFuncSetAttribute((const void*)k_pf_attn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPfAttnLds);
}

}  // namespace mtg
