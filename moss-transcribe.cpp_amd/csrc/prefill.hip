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
//                    (block-diagonal B operand from LDS-staged codes: two exact
//                    per-block int32 dots per MFMA), epilogue store / residual
//                    add / SwiGLU
//   k_pf_quant       q8_0 conversion of f32 rows (the SwiGLU output)
//   k_pf_qk_rope     q/k RMSNorm + NEOX RoPE, K/V written into the cache
//   k_pf_attn        causal attention of 16 query rows of one q head per
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
// out[s][n] for the 64 weight rows of blockIdx.x (wave w: tile 4 blockIdx.x + w;
// for SwiGLU waves 0, 1 take gate tiles 2 blockIdx.x + {0, 1} and waves 2, 3 the
// same tiles of the up matrix, meeting in LDS for the epilogue) and the 64
// activation rows of blockIdx.y (8 column groups of 8). The block pairs run in
// order; per pair the activation codes of the 64 rows are staged in LDS (the
// next pair's already in flight in registers), and each wave's B operand of
// column group cg holds 16 code bytes of row 8 cg + j % 8, block 2 bp + j / 8,
// when (lane / 16) / 2 == j / 8 (j = lane % 16), else zeros, so each MFMA returns
// the exact int32 dot of every (weight row, activation row, block). The K-slices
// run one after the other, so one accumulator per slice and a running total
// give ((s0 + s1) + s2) + s3 per parity, then even + odd.
enum { PF_STORE = 0, PF_RESID = 1, PF_SWIGLU = 2, PF_BIAS = 3, PF_BIAS_GELU = 4, PF_BIAS_SILU = 5, PF_BIAS_RESID = 6 };
constexpr int kPfRowBytes = 80;  // LDS stride of a staged 64-byte code row (bank spread)

template <int EPI>
__global__ void __launch_bounds__(256)
k_pf_gemm(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, int N, int K,
          const int8_t* __restrict__ codes, const float* __restrict__ scales, int S, float* __restrict__ out,
          const float* __restrict__ bias) {
  constexpr bool GLU = EPI == PF_SWIGLU;
  __shared__ __align__(16) uint8_t s_codes[2][64 * kPfRowBytes];
  __shared__ float s_dx[2][64 * 2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tile = GLU ? blockIdx.x * 2 + (wave & 1) : blockIdx.x * 4 + wave;
  const uint8_t* mat = (GLU && wave >= 2) ? w2 : w;
  const int s0 = blockIdx.y * 64;
  const int bps = K / kPairK;
  const int j = lane & 15, g = lane >> 4, par = j >> 3;
  const bool holds = (g >> 1) == par;
  const int srow = par * 16 + 4 * (lane >> 4);
  const v4i zero = {0, 0, 0, 0};
  // staging: thread t loads 16 bytes of row t / 4 (part t % 4); threads < 128 a scale
  const int st_row = tid >> 2, st_part = tid & 3;
  const bool st_in = s0 + st_row < S;
  const int sc_row = tid >> 1, sc_par = tid & 1;
  const bool sc_in = tid < 128 && s0 + sc_row < S;
  auto fetch = [&](int bp, v4i& c, float& d) {
    c = st_in ? *(const v4i*)(codes + (size_t)(s0 + st_row) * K + 64 * bp + 16 * st_part) : zero;
    d = sc_in ? scales[(size_t)(s0 + sc_row) * (K / 32) + 2 * bp + sc_par] : 0.0f;
  };
  auto stage = [&](int buf, const v4i& c, float d) {
    *(v4i*)(s_codes[buf] + st_row * kPfRowBytes + 16 * st_part) = c;
    if (tid < 128) s_dx[buf][sc_row * 2 + sc_par] = d;
  };
  v4i nc;
  float nd;
  fetch(0, nc, nd);
  stage(0, nc, nd);
  float part[8][4], tot[8][4];
#pragma unroll
  for (int cg = 0; cg < 8; ++cg)
#pragma unroll
    for (int q = 0; q < 4; ++q) part[cg][q] = tot[cg][q] = 0.0f;
  // the weight unit of the next pair is in flight while a pair computes
  const uint8_t* wtile = mat + (size_t)tile * bps * kUnitBytes;
  v4i na = __builtin_nontemporal_load((const v4i*)(wtile + lane * 16));
  uint2 nsw = *(const uint2*)(wtile + 1024 + srow * 2);
  int sl = 0, sl_end = bps / 4;
  for (int bp = 0; bp < bps; ++bp) {
    const int buf = bp & 1;
    if (bp + 1 < bps) fetch(bp + 1, nc, nd);
    const v4i a = na;
    const uint2 sw = nsw;
    if (bp + 1 < bps) {
      const uint8_t* unit = wtile + (size_t)(bp + 1) * kUnitBytes;
      na = __builtin_nontemporal_load((const v4i*)(unit + lane * 16));
      nsw = *(const uint2*)(unit + 1024 + srow * 2);
    }
    float dw[4];
    dw[0] = half_bits_to_float((uint16_t)(sw.x & 0xffff));
    dw[1] = half_bits_to_float((uint16_t)(sw.x >> 16));
    dw[2] = half_bits_to_float((uint16_t)(sw.y & 0xffff));
    dw[3] = half_bits_to_float((uint16_t)(sw.y >> 16));
    __syncthreads();  // the staged pair bp is complete
#pragma unroll
    for (int cg = 0; cg < 8; ++cg) {
      const int row = 8 * cg + (j & 7);
      const v4i b = holds ? *(const v4i*)(s_codes[buf] + row * kPfRowBytes + 32 * par + 16 * (g & 1)) : zero;
      const float dx = s_dx[buf][row * 2 + par];
      const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, zero, 0, 0, 0);
#pragma unroll
      for (int q = 0; q < 4; ++q) part[cg][q] = fmaf((float)c[q], dw[q] * dx, part[cg][q]);
    }
    if (bp + 1 == sl_end) {  // a K-slice ends: fold it into the running total
#pragma unroll
      for (int cg = 0; cg < 8; ++cg)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          tot[cg][q] = sl == 0 ? part[cg][q] : __fadd_rn(tot[cg][q], part[cg][q]);
          part[cg][q] = 0.0f;
        }
      ++sl;
      sl_end = (bps * (sl + 1)) / 4;
    }
    if (bp + 1 < bps) stage(buf ^ 1, nc, nd);  // the other buffer: read two steps ago, behind the barrier
  }
#pragma unroll
  for (int cg = 0; cg < 8; ++cg)
#pragma unroll
    for (int q = 0; q < 4; ++q) tot[cg][q] = __fadd_rn(tot[cg][q], dpp_f<kDppRor8>(tot[cg][q]));  // even + odd
  if constexpr (GLU) {
    // the up waves hand their values to the gate waves of the same tile
    __syncthreads();
    __shared__ __align__(16) float s_up[2 * 8 * 64 * 4];  // [2 tiles][8 cg][64 lanes][4]
    if (wave >= 2)
#pragma unroll
      for (int cg = 0; cg < 8; ++cg)
        *(v4f*)(s_up + (((wave & 1) * 8 + cg) * 64 + lane) * 4) = (v4f){tot[cg][0], tot[cg][1], tot[cg][2], tot[cg][3]};
    __syncthreads();
    if (wave >= 2) return;
#pragma unroll
    for (int cg = 0; cg < 8; ++cg) {
      const v4f u = *(const v4f*)(s_up + (((wave & 1) * 8 + cg) * 64 + lane) * 4);
#pragma unroll
      for (int q = 0; q < 4; ++q) tot[cg][q] = dev_swiglu(tot[cg][q], u[q]);
    }
  }
  // lanes j and j + 8 hold the same sums: lane j takes row groups 0..3 of
  // rows s0 + 8 cg + j, lane j + 8 groups 4..7
  {
    const int n = tile * 16 + 4 * (lane >> 4), hi = j >> 3;
    // a mask the compiler cannot see through: a plain select between tot[c] and
    // tot[4 + c] becomes a lane-dependent index into tot, which moves tot to
    // scratch memory for the whole kernel
    uint32_t m = 0u - (uint32_t)hi;
    asm volatile("" : "+v"(m));
    float y[4][4];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t lo = __float_as_uint(tot[c][q]);
        y[c][q] = __uint_as_float(lo ^ ((lo ^ __float_as_uint(tot[4 + c][q])) & m));
      }
    if constexpr (EPI >= PF_BIAS) {
      // linear = mul_mat + bias, then the activation or the residual add
      const v4f b = *(const v4f*)(bias + n);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) y[c][q] = __fadd_rn(y[c][q], b[q]);
      if constexpr (EPI == PF_BIAS_GELU) {
#pragma unroll
        for (int c = 0; c < 4; c += 2) {
          float g[8];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            g[q] = y[c][q];
            g[4 + q] = y[c + 1][q];
          }
          dev_gelu_erf_n<8>(g);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            y[c][q] = g[q];
            y[c + 1][q] = g[4 + q];
          }
        }
      }
      if constexpr (EPI == PF_BIAS_SILU)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int q = 0; q < 4; ++q) y[c][q] = dev_silu(y[c][q]);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int row = s0 + 8 * (4 * hi + c) + (j & 7);
      if (row >= S) continue;
      float* dst = out + (size_t)row * N + n;
      v4f v;
      if constexpr (EPI == PF_RESID || EPI == PF_BIAS_RESID) {
        const v4f x = *(const v4f*)dst;
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = __fadd_rn(x[q], y[c][q]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = y[c][q];
      }
      *(v4f*)dst = v;
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
// grid (n_heads / kPfHeads, ceil(S / kPfRows)): a workgroup takes query rows
// r0 .. r0 + kPfRows - 1 (positions past0 + r0 + t) of the kPfHeads q heads of
// one kv head, columns col = kPfRows hl + t; the blocks with the most chunks are
// numbered first. Keys 0 .. past0 + r0 + kPfRows - 1 come from the cache (this block's
// rows were appended by k_pf_qk_rope). The output rows leave as the
// o-projection's q8_0 activation: codes [S][n_heads * 128], scales [S][n_heads * 4].
__device__ __forceinline__ int pf_perm128(int d) { return (d & 3) * 32 + (d >> 2); }

// K and V of the 64-key chunk at key0 in MFMA operand layout, loaded straight
// into registers (f32, or f16 widened; zeros past kvlen). Wave w: scores of keys
// 16 w + kl, k[m] = K[key0 + 16 w + kl][4 m + kk] (m < 32, the fma chain over
// head_dim in order); P.V of head_dim tiles 2 w, 2 w + 1,
// v[h][s] = V[key0 + 4 s + kk][16 (2 w + h) + kl] (s < 16, the chain over keys).
constexpr int kPfHeads = 2;     // q heads per workgroup (one kv head's group)
constexpr int kPfRowTiles = 2;  // query rows per workgroup / 16
constexpr int kPfRows = 16 * kPfRowTiles;
constexpr int kPfCols = kPfHeads * kPfRows;  // column tile ct: q head ct / kPfRowTiles, rows 16 (ct % kPfRowTiles) + kl

typedef __amdgpu_buffer_rsrc_t PfRsrc;
// A buffer descriptor over kv head rows [0, kvlen): loads past its end return 0.
// The range check covers the per-lane offset only, so every key-dependent part
// of an address goes there (the scalar offset stays 0).
__device__ __forceinline__ PfRsrc pf_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
template <int KVH>
__device__ __forceinline__ float pf_kv(PfRsrc r, uint32_t voff, uint32_t soff) {
  if constexpr (KVH)
    return half_bits_to_float((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0));
  else
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0));
}
template <int KVH>
__device__ __forceinline__ void pf_load_k(PfRsrc rk, int key0, float (&k)[32]) {
  constexpr int es = KVH ? 2 : 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kl = lane & 15, kk = lane >> 4;
  const uint32_t voff = (uint32_t)(((key0 + 16 * wave + kl) * kHeadDim + kk) * es);
#pragma unroll
  for (int m = 0; m < 32; ++m) k[m] = pf_kv<KVH>(rk, voff + 4 * m * es, 0);
}
template <int KVH>
__device__ __forceinline__ void pf_load_v(PfRsrc rv, int key0, float (&v)[2][16]) {
  constexpr int es = KVH ? 2 : 4;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kl = lane & 15, kk = lane >> 4;
  const uint32_t voff = (uint32_t)(((key0 + kk) * kHeadDim + 32 * wave + kl) * es);
#pragma unroll
  for (int s2 = 0; s2 < 16; ++s2)
#pragma unroll
    for (int h = 0; h < 2; ++h) v[h][s2] = pf_kv<KVH>(rv, voff + (4 * s2 * kHeadDim + 16 * h) * es, 0);
}

// Scores of keys 16 wave + 4 kk + r (r < 4) for columns 16 ct + kl, scaled and
// masked: the fma chain over head_dim is 32 chained MFMAs.
template <int NCT>
__device__ __forceinline__ void pf_scores(const float* s_q, const float (&k)[32], int key0, int kvlen, int past0,
                                          int r0, int nq, float scale, float (&w)[NCT][4]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kl = lane & 15, kk = lane >> 4;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const float* qrow = s_q + (ct * 16 + kl) * kPfQStride + kk * 32;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const v4f q4 = *(const v4f*)(qrow + 4 * i);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k[4 * i + jj], q4[jj], acc, 0, 0, 0);
    }
    const int t = 16 * (ct % kPfRowTiles) + kl;  // column 16 ct + kl: row t of q head ct / kPfRowTiles
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = key0 + 16 * wave + 4 * kk + r;
      w[ct][r] = (t < nq && key < kvlen && key <= past0 + r0 + t) ? __fmul_rn(acc[r], scale) : -INFINITY;
    }
  }
}

constexpr size_t kPfAttnLds =
    ((size_t)kPfCols * kPfQStride + kPfCols * kPfPStride + 4 * kPfCols + 3 * kPfCols) * 4;

// OUTF: the output rows as f32 [S][n_heads * 128] in ofl (the f16 / q4_K weight
// paths convert them to their vec_dot_type), instead of q8_0 codes.
template <int KVH, bool OUTF = false>
__global__ void __launch_bounds__(256)
k_pf_attn(const float* __restrict__ q, int n_heads, int n_kv_heads, KvLayer kv, int past0, int S,
          int8_t* __restrict__ ocodes, float* __restrict__ oscales, float* __restrict__ ofl) {
  constexpr int NCT = kPfCols / 16, NC = kPfCols;
  // the query blocks with the most chunks start first
  const int hq0 = blockIdx.x * kPfHeads, g = hq0 / (n_heads / n_kv_heads);
  const int r0 = (gridDim.y - 1 - blockIdx.y) * kPfRows;
  const int nq = min(kPfRows, S - r0);
  const int kvlen = past0 + S;
  const int last = past0 + r0 + nq - 1;  // the block's last query position
  const int nch = last / kChunk + 1;
  extern __shared__ v4f pf_lds_v4[];
  float* s_q = (float*)pf_lds_v4;                  // [NC][132] permuted
  float* s_p = s_q + NC * kPfQStride;              // [NC][68] permuted keys
  float* s_wm = s_p + NC * kPfPStride;             // [4 waves][NC]
  float* s_l = s_wm + 4 * NC;                      // [NC] chunk sums
  float* s_f = s_l + NC;                           // [NC] chunk factors
  float* s_M = s_f + NC;                           // [NC] column maxima over all chunks
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, kl = lane & 15, kk = lane >> 4;
  constexpr bool f16kv = KVH != 0;
  // q rows (f16-rounded for an f16 cache: mul_mat(f16 K, f32 q) converts q)
  for (int idx = tid; idx < NC * (kHeadDim / 4); idx += 256) {
    const int col = idx / (kHeadDim / 4), d = (idx % (kHeadDim / 4)) * 4, hl = col / kPfRows, t = col % kPfRows;
    v4f v = {0.f, 0.f, 0.f, 0.f};
    if (t < nq) v = *(const v4f*)(q + ((size_t)(r0 + t) * n_heads + hq0 + hl) * kHeadDim + d);
#pragma unroll
    for (int e = 0; e < 4; ++e) s_q[col * kPfQStride + pf_perm128(d + e)] = f16kv ? f16_round(v[e]) : v[e];
  }
  constexpr int es = KVH ? 2 : 4;
  const size_t head = (size_t)g * kv.max_seq * kHeadDim * es;
  const uint32_t kvbytes = (uint32_t)kvlen * kHeadDim * es;
  const PfRsrc rk = pf_rsrc((const uint8_t*)kv.k + head, kvbytes);
  const PfRsrc rv = pf_rsrc((const uint8_t*)kv.v + head, kvbytes);
  const float scale = __fdiv_rn(1.0f, dev_sqrtf((float)kHeadDim));
  float kr[32], vr[2][16];
  // pass 1: each column's maximum over all chunks (exact in any order)
  pf_load_k<KVH>(rk, 0, kr);
  __syncthreads();
  int colmax[NCT];  // per column tile: the lane's column kl
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) colmax[ct] = ord_key(-INFINITY);
  for (int c = 0; c < nch; ++c) {
    float w[NCT][4];
    pf_scores<NCT>(s_q, kr, c * kChunk, kvlen, past0, r0, nq, scale, w);
    if (c + 1 < nch) pf_load_k<KVH>(rk, (c + 1) * kChunk, kr);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r) colmax[ct] = max(colmax[ct], ord_key(w[ct][r]));
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    uint32_t a, b;
    pair_split<16>((uint32_t)colmax[ct], a, b);  // the lanes kk of one column
    colmax[ct] = max((int)a, (int)b);
    pair_split<32>((uint32_t)colmax[ct], a, b);
    colmax[ct] = max((int)a, (int)b);
    if (kk == 0) s_wm[wave * NC + ct * 16 + kl] = ord_val(colmax[ct]);
  }
  __syncthreads();
  if (tid < NC)
    s_M[tid] = fmaxf(fmaxf(s_wm[tid], s_wm[NC + tid]), fmaxf(s_wm[2 * NC + tid], s_wm[3 * NC + tid]));
  // pass 2: probabilities, chunk sums, P.V, merged in chunk order
  float O[NCT][2][4], L[NCT][4];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      L[ct][r] = 0.0f;
      O[ct][0][r] = O[ct][1][r] = 0.0f;
    }
  const int sp_pos = (lane & 3) * 16 + (lane >> 2);
  pf_load_k<KVH>(rk, 0, kr);
  pf_load_v<KVH>(rv, 0, vr);
  for (int c = 0; c < nch; ++c) {
    float w[NCT][4];
    pf_scores<NCT>(s_q, kr, c * kChunk, kvlen, past0, r0, nq, scale, w);
    if (c + 1 < nch) pf_load_k<KVH>(rk, (c + 1) * kChunk, kr);
    __syncthreads();  // the previous chunk's probabilities are consumed
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
      for (int r = 0; r < 4; ++r)  // key 16 wave + 4 kk + r sits at r * 16 + 4 wave + kk
        s_p[(ct * 16 + kl) * kPfPStride + r * 16 + 4 * wave + kk] = w[ct][r];
    __syncthreads();
    // chunk softmax per column (one wave per column, lane = key)
    for (int col = wave; col < NC; col += 4) {
      const float wv = s_p[col * kPfPStride + sp_pos];
      const float m = wave_max_f(wv);
      float p = (m == -INFINITY || wv == -INFINITY) ? 0.0f : dev_expf(__fsub_rn(wv, m));
      if (f16kv) p = f16_round(p);
      const float l = wave_sum_f(p);
      s_p[col * kPfPStride + sp_pos] = p;
      if (lane == 0) {
        s_l[col] = l;
        s_f[col] = m == -INFINITY ? 0.0f : dev_expf(__fsub_rn(m, s_M[col]));
      }
    }
    __syncthreads();
    // O_c[col][d]: fma chain over the chunk's keys; wave w takes head_dim tiles 2w, 2w+1
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
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
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < 16; ++s2) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s2], vr[h][s2], acc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) O[ct][h][r] = fmaf(acc[r], s_f[ct * 16 + 4 * kk + r], O[ct][h][r]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = ct * 16 + 4 * kk + r;
        L[ct][r] = fmaf(s_l[col], s_f[col], L[ct][r]);
      }
    }
    if (c + 1 < nch) pf_load_v<KVH>(rv, (c + 1) * kChunk, vr);
  }
  // out = O / L, then the q8_0 blocks of 32 head_dim elements (wave w: block w)
  const int QN = n_heads * kHeadDim;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * (ct % kPfRowTiles) + 4 * kk + r;  // query row of column 16 ct + 4 kk + r
      const float o0 = __fdiv_rn(O[ct][0][r], L[ct][r]);
      const float o1 = __fdiv_rn(O[ct][1][r], L[ct][r]);
      if constexpr (OUTF) {
        if (t < nq) {
          float* orow = ofl + (size_t)(r0 + t) * QN + (hq0 + ct / kPfRowTiles) * kHeadDim + 32 * wave + kl;
          orow[0] = o0;
          orow[16] = o1;
        }
        continue;
      }
      float amax = fmaxf(fabsf(o0), fabsf(o1));
      uint32_t u = __float_as_uint(amax);  // max over the 16 lanes kl of this row
      u = max(u, dpp_u<kDppRor8>(u));
      u = max(u, dpp_u<kDppRor4>(u));
      u = max(u, dpp_u<kDppRor2>(u));
      u = max(u, dpp_u<kDppRor1>(u));
      amax = __uint_as_float(u);
      if (t < nq) {
        const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        const size_t rowoff = (size_t)(r0 + t) * QN + (hq0 + ct / kPfRowTiles) * kHeadDim;
        ocodes[rowoff + 32 * wave + kl] = (int8_t)rintf(__fmul_rn(o0, id));
        ocodes[rowoff + 32 * wave + 16 + kl] = (int8_t)rintf(__fmul_rn(o1, id));
        if (kl == 0)
          oscales[(size_t)(r0 + t) * (QN / 32) + ((hq0 + ct / kPfRowTiles) * kHeadDim) / 32 + wave] =
              __half2float(__float2half_rn(__fdiv_rn(amax, 127.0f)));
      }
    }
}

}  // namespace

// ================================================================ launches ==
// The buffer descriptors of the attention cover a kv head's rows with a 32-bit
// byte count.
int pf_max_context() { return (int)(0x7fffffffu / (kHeadDim * 4)); }

void launch_pf_norm_quant(hipStream_t s, const float* src, int S, const float* gain, float eps, int8_t* codes,
                          float* scales, float* normed_out) {
  hipLaunchKernelGGL(k_pf_norm_quant, dim3((S + 3) / 4), dim3(256), 0, s, src, S, gain, eps, codes, scales,
                     normed_out);
}

void launch_pf_quant(hipStream_t s, const float* src, int S, int K, int8_t* codes, float* scales) {
  hipLaunchKernelGGL(k_pf_quant, dim3((S + 3) / 4), dim3(256), 0, s, src, S, K, codes, scales);
}

void launch_pf_gemm(hipStream_t s, int epi, const uint8_t* w, const uint8_t* w2, int N, int K, const int8_t* codes,
                    const float* scales, int S, float* out, const float* bias) {
  const dim3 blocks((unsigned)(epi == PF_SWIGLU ? N / 32 : N / 64), (unsigned)((S + 63) / 64));
#define MTG_PF_GEMM(E) \
  hipLaunchKernelGGL(k_pf_gemm<E>, blocks, dim3(256), 0, s, w, w2, N, K, codes, scales, S, out, bias)
  switch (epi) {
    case PF_STORE: MTG_PF_GEMM(PF_STORE); break;
    case PF_RESID: MTG_PF_GEMM(PF_RESID); break;
    case PF_SWIGLU: MTG_PF_GEMM(PF_SWIGLU); break;
    case PF_BIAS: MTG_PF_GEMM(PF_BIAS); break;
    case PF_BIAS_GELU: MTG_PF_GEMM(PF_BIAS_GELU); break;
    case PF_BIAS_SILU: MTG_PF_GEMM(PF_BIAS_SILU); break;
    default: MTG_PF_GEMM(PF_BIAS_RESID); break;
  }
#undef MTG_PF_GEMM
}

void launch_pf_qk_rope(hipStream_t s, const float* qkv, int S, int past0, int n_heads, int n_kv_heads,
                       const float* q_norm, const float* k_norm, float eps, const float* rope, float* q_out,
                       KvLayer kv) {
  hipLaunchKernelGGL(k_pf_qk_rope, dim3((unsigned)S, (unsigned)(n_heads + 2 * n_kv_heads)), dim3(64), 0, s, qkv, S,
                     past0, n_heads, n_kv_heads, q_norm, k_norm, eps, rope, q_out, kv);
}

void launch_pf_attn(hipStream_t s, const float* q, int n_heads, int n_kv_heads, KvLayer kv, int past0, int S,
                    int8_t* ocodes, float* oscales, float* ofl) {
  const dim3 grid((unsigned)(n_heads / kPfHeads), (unsigned)((S + kPfRows - 1) / kPfRows));
#define MTG_PF_ATTN(KVH, OUTF)                                                                                 \
  hipLaunchKernelGGL((k_pf_attn<KVH, OUTF>), grid, dim3(256), kPfAttnLds, s, q, n_heads, n_kv_heads, kv, past0, S, \
                     ocodes, oscales, ofl)
  if (ofl) {
    if (kv.f16) MTG_PF_ATTN(1, true);
    else MTG_PF_ATTN(0, true);
  } else {
    if (kv.f16) MTG_PF_ATTN(1, false);
    else MTG_PF_ATTN(0, false);
  }
#undef MTG_PF_ATTN
}

hipError_t prepare_kernels_pf() {
  const void* fns[] = {(const void*)k_pf_attn<0, false>, (const void*)k_pf_attn<1, false>,
                       (const void*)k_pf_attn<0, true>, (const void*)k_pf_attn<1, true>};
  for (const void* f : fns) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPfAttnLds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace mtg
