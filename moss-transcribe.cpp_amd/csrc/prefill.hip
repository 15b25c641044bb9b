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
//   k_pf_attn_mma    causal attention on f32 MFMA, 16 query rows of one q
//                    head per wave over the cache, in two passes over the
//                    64-key chunks, writing the o-projection's q8_0 activation
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
// one kv head; the blocks with the most chunks are numbered first. Keys
// 0 .. past0 + r0 + kPfRows - 1 come from the cache (this block's rows were
// appended by k_pf_qk_rope). The output rows leave as the o-projection's q8_0
// activation: codes [S][n_heads * 128], scales [S][n_heads * 4].
constexpr int kPfHeads = 2;     // q heads per workgroup (one kv head's group)
constexpr int kPfRowTiles = 2;  // query rows per workgroup / 16
constexpr int kPfRows = 16 * kPfRowTiles;

// ------------------------------------------------ attention on f32 MFMA ----
// k_pf_attn_mma: the causal attention of k_pf_attn with the chunk softmax kept in
// registers. Workgroup = the two q heads of one kv head x 32 query rows; wave w
// owns the 16 rows r0 + 16 (w & 1) + j (j = lane % 16) of q head hq0 + w / 2.
//   scores: key tile t (16 keys) is one chain of 32 MFMAs over head_dim,
//     A = K rows, B = the wave's q rows (registers). Row i of the A operand is
//     key 16 t + 4 (i % 4) + i / 4, so output register r of lane (g, j)
//     (g = lane / 16) holds key 16 t + 4 r + g: the B operand of P.V MFMA
//     m = 4 t + r (keys 4 m .. 4 m + 3 in order) with no data movement.
//   chunk max and sum: in-lane over t and r, then across lanes xor 32, 16 (the
//     sum in the butterfly's pairing: key levels 32, 16, 8, 4 in the lane, 2, 1
//     across lanes).
//   P.V: head_dim tile dt (16) is one chain of 16 MFMAs over the chunk's keys,
//     A = V^T.
// The chunks go through LDS: K rows at slot 16 t + 4 g + r for key 16 t + 4 r + g,
// element 4 s + g at g * 32 + s; V^T rows d with key 4 m + g at g * 16 + m. Pass 1
// (row maxima) double-buffers K in the two regions; pass 2 holds K in one and
// V^T in the other, the next chunk's loads in flight during the arithmetic.
// A wave skips the chunks that lie wholly after its last row (their terms are
// exact zeros of the merge).
constexpr int kPaKs = kHeadDim + 4;              // K slab row stride (floats)
constexpr int kPaVs = 64 + 4;                    // V^T slab row stride
constexpr int kPaRegion = kHeadDim * kPaVs;      // floats per region (>= 64 * kPaKs)
constexpr size_t kPaLds = (size_t)2 * kPaRegion * 4;
static_assert(64 * kPaKs <= kPaRegion, "K slab fits a region");

// this thread's share of a chunk of K (keys key0 ..): key tid / 4, elements
// 32 (tid % 4) .. + 31; of V: keys 4 (4 mq + x) + g (x < 4), elements 8 u .. 8 u + 7
// with (g, mq, u) = (tid / 64, tid / 16 % 4, tid % 16). Rows past kvlen read row
// kvlen - 1 and are zeroed at the store.
template <int KVH>
struct PaRegs {
  v4f r[8];
};
template <int KVH>
__device__ __forceinline__ void pa_load_k(const uint8_t* kh, int key0, int kvlen, PaRegs<KVH>& R) {
  constexpr int es = KVH ? 2 : 4;
  const int tid = threadIdx.x, key = min(key0 + (tid >> 2), kvlen - 1), q = tid & 3;
  const uint8_t* src = kh + ((size_t)key * kHeadDim + 32 * q) * es;
  if constexpr (KVH) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const v4i h = *(const v4i*)(src + 16 * x);  // 8 halves: elements 32 q + 8 x ..
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        R.r[2 * x + e / 2][2 * (e % 2)] = half_bits_to_float((uint16_t)((uint32_t)h[e] & 0xffff));
        R.r[2 * x + e / 2][2 * (e % 2) + 1] = half_bits_to_float((uint16_t)((uint32_t)h[e] >> 16));
      }
    }
  } else {
#pragma unroll
    for (int x = 0; x < 8; ++x) R.r[x] = *(const v4f*)(src + 16 * x);
  }
}
template <int KVH>
__device__ __forceinline__ void pa_store_k(float* s, int key0, int kvlen, const PaRegs<KVH>& R) {
  const int tid = threadIdx.x, key = tid >> 2, q = tid & 3;
  const int slot = (key & ~15) | ((key & 3) << 2) | ((key >> 2) & 3);
  const bool live = key0 + key < kvlen;
  // R.r[x][e] is element 32 q + 4 x + e = 4 s + g with s = 8 q + x, g = e
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4f o;
#pragma unroll
      for (int x = 0; x < 4; ++x) o[x] = live ? R.r[4 * h + x][e] : 0.0f;
      *(v4f*)(s + slot * kPaKs + e * 32 + 8 * q + 4 * h) = o;
    }
}
template <int KVH>
__device__ __forceinline__ void pa_load_v(const uint8_t* vh, int key0, int kvlen, PaRegs<KVH>& R) {
  constexpr int es = KVH ? 2 : 4;
  const int tid = threadIdx.x, u = tid & 15, mq = (tid >> 4) & 3, g = tid >> 6;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int key = min(key0 + 4 * (4 * mq + x) + g, kvlen - 1);
    const uint8_t* src = vh + ((size_t)key * kHeadDim + 8 * u) * es;
    if constexpr (KVH) {
      const v4i h = *(const v4i*)src;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        R.r[2 * x + e / 2][2 * (e % 2)] = half_bits_to_float((uint16_t)((uint32_t)h[e] & 0xffff));
        R.r[2 * x + e / 2][2 * (e % 2) + 1] = half_bits_to_float((uint16_t)((uint32_t)h[e] >> 16));
      }
    } else {
      R.r[2 * x] = *(const v4f*)src;
      R.r[2 * x + 1] = *(const v4f*)(src + 16);
    }
  }
}
template <int KVH>
__device__ __forceinline__ void pa_store_v(float* s, int key0, int kvlen, const PaRegs<KVH>& R) {
  const int tid = threadIdx.x, u = tid & 15, mq = (tid >> 4) & 3, g = tid >> 6;
  // R.r[2 x + e / 4][e % 4] is element 8 u + e of key 4 (4 mq + x) + g
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    v4f o;
#pragma unroll
    for (int x = 0; x < 4; ++x) o[x] = key0 + 4 * (4 * mq + x) + g < kvlen ? R.r[2 * x + e / 4][e % 4] : 0.0f;
    *(v4f*)(s + (8 * u + e) * kPaVs + g * 16 + 4 * mq) = o;
  }
}

template <int KVH, bool OUTF>
__global__ void __launch_bounds__(256, 2)
k_pf_attn_mma(const float* __restrict__ q, int n_heads, int n_kv_heads, KvLayer kv, int past0, int S,
              int8_t* __restrict__ ocodes, float* __restrict__ oscales, float* __restrict__ ofl) {
  extern __shared__ v4f pa_lds_v4[];
  float* reg0 = (float*)pa_lds_v4;
  float* reg1 = reg0 + kPaRegion;
  const int hq0 = blockIdx.x * kPfHeads, g_kv = hq0 / (n_heads / n_kv_heads);
  const int r0 = (gridDim.y - 1 - blockIdx.y) * kPfRows;  // the blocks with the most chunks start first
  const int kvlen = past0 + S;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, g = lane >> 4;
  const int hq = hq0 + (wave >> 1), rw = r0 + 16 * (wave & 1);  // this wave's head and first row
  const int row = rw + j;
  const int nch = min(past0 + r0 + kPfRows - 1, kvlen - 1) / kChunk + 1;  // the workgroup's chunks
  const int wlast = min(past0 + rw + 15, kvlen - 1);                    // this wave's last key
  constexpr int es = KVH ? 2 : 4;
  const uint8_t* kh = (const uint8_t*)kv.k + (size_t)g_kv * kv.max_seq * kHeadDim * es;
  const uint8_t* vh = (const uint8_t*)kv.v + (size_t)g_kv * kv.max_seq * kHeadDim * es;
  const float scale = __fdiv_rn(1.0f, dev_sqrtf((float)kHeadDim));
  // B operand of the scores: q[row][4 s + g] (f16-rounded for an f16 cache)
  float qb[32];
  {
    const float* qr = q + ((size_t)min(row, S - 1) * n_heads + hq) * kHeadDim + g;
#pragma unroll
    for (int s = 0; s < 32; ++s) {
      const float v = row < S ? qr[4 * s] : 0.0f;
      qb[s] = KVH ? f16_round(v) : v;
    }
  }
  const int pos = past0 + row;  // this row's last key
  auto scores = [&](const float* sk, int key0, float (&w)[4][4]) {
    v4f acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      v4f a[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) a[t] = *(const v4f*)(sk + (16 * t + j) * kPaKs + g * 32 + 4 * x);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][e], qb[4 * x + e], acc[t], 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = key0 + 16 * t + 4 * r + g;
        w[t][r] = (row < S && key <= pos) ? __fmul_rn(acc[t][r], scale) : -INFINITY;
      }
  };
  PaRegs<KVH> R;
  // pass 1: row maxima over all chunks; K double-buffered in the two regions
  pa_load_k<KVH>(kh, 0, kvlen, R);
  pa_store_k<KVH>(reg0, 0, kvlen, R);
  __syncthreads();
  float M = -INFINITY;
  for (int c = 0; c < nch; ++c) {
    const bool last = c + 1 == nch;
    pa_load_k<KVH>(kh, last ? 0 : 64 * (c + 1), kvlen, R);  // pass 2 starts again at chunk 0
    if (64 * c <= wlast) {
      float w[4][4];
      scores((c & 1) ? reg1 : reg0, 64 * c, w);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) M = fmaxf(M, w[t][r]);
    }
    pa_store_k<KVH>(((c + 1) & 1) ? reg1 : reg0, last ? 0 : 64 * (c + 1), kvlen, R);
    __syncthreads();
  }
  M = pair_max_f<32>(M);
  M = pair_max_f<16>(M);
  // pass 2: K of chunk 0 sits in region nch & 1; V^T goes to the other region
  float* sk = (nch & 1) ? reg1 : reg0;
  float* sv = (nch & 1) ? reg0 : reg1;
  pa_load_v<KVH>(vh, 0, kvlen, R);
  pa_store_v<KVH>(sv, 0, kvlen, R);
  __syncthreads();
  float L = 0.0f;
  v4f O[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) O[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < nch; ++c) {
    const bool more = c + 1 < nch, live = 64 * c <= wlast;
    if (more) pa_load_k<KVH>(kh, 64 * (c + 1), kvlen, R);
    float p[4][4];
    float mc = -INFINITY, lc = 0.0f;
    if (live) {
      float w[4][4];
      scores(sk, 64 * c, w);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) mc = fmaxf(mc, w[t][r]);
      mc = pair_max_f<32>(mc);
      mc = pair_max_f<16>(mc);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float pv = (mc == -INFINITY || w[t][r] == -INFINITY) ? 0.0f : dev_expf(__fsub_rn(w[t][r], mc));
          p[t][r] = KVH ? f16_round(pv) : pv;
        }
      float u[2][4], x4[4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) u[t][r] = __fadd_rn(p[t][r], p[t + 2][r]);
#pragma unroll
      for (int r = 0; r < 4; ++r) x4[r] = __fadd_rn(u[0][r], u[1][r]);
      lc = pair_add_f<32>(__fadd_rn(__fadd_rn(x4[0], x4[2]), __fadd_rn(x4[1], x4[3])));
      lc = pair_add_f<16>(lc);
    }
    __syncthreads();  // K of chunk c is consumed
    if (more) {
      pa_store_k<KVH>(sk, 64 * (c + 1), kvlen, R);
      pa_load_v<KVH>(vh, 64 * (c + 1), kvlen, R);
    }
    if (live) {
      v4f oc[8];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) oc[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        v4f av[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) av[dt] = *(const v4f*)(sv + (16 * dt + j) * kPaVs + g * 16 + 4 * x);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int dt = 0; dt < 8; ++dt)
            oc[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[dt][e], p[x][e], oc[dt], 0, 0, 0);
      }
      const float f = mc == -INFINITY ? 0.0f : dev_expf(__fsub_rn(mc, M));
      L = fmaf(lc, f, L);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) O[dt][r] = fmaf(oc[dt][r], f, O[dt][r]);
    }
    __syncthreads();  // V^T of chunk c is consumed, K of chunk c + 1 is staged
    if (more) pa_store_v<KVH>(sv, 64 * (c + 1), kvlen, R);
  }
  // O[dt][r]: element 16 dt + 4 g + r of row `row`
  const int QN = n_heads * kHeadDim;
  float o[8][4];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) o[dt][r] = __fdiv_rn(O[dt][r], L);
  if constexpr (OUTF) {
    if (row < S) {
      float* orow = ofl + (size_t)row * QN + hq * kHeadDim + 4 * g;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) *(v4f*)(orow + 16 * dt) = v4f{o[dt][0], o[dt][1], o[dt][2], o[dt][3]};
    }
  } else {
    // q8_0 block b = elements 32 b .. 32 b + 31 = tiles 2 b, 2 b + 1 over the four lane groups
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      uint32_t u = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) u = max(u, __float_as_uint(fabsf(o[2 * b + h][r])));
      u = pair_max_u<32>(u);
      u = pair_max_u<16>(u);
      const float amax = __uint_as_float(u);
      const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
      if (row < S) {
        const size_t rowoff = (size_t)row * QN + hq * kHeadDim;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint32_t word = 0;
#pragma unroll
          for (int r = 0; r < 4; ++r)
            word |= (uint32_t)(uint8_t)(int8_t)rintf(__fmul_rn(o[2 * b + h][r], id)) << (8 * r);
          *(uint32_t*)(ocodes + rowoff + 16 * (2 * b + h) + 4 * g) = word;
        }
        if (g == 0)
          oscales[(size_t)row * (QN / 32) + (hq * kHeadDim) / 32 + b] =
              __half2float(__float2half_rn(__fdiv_rn(amax, 127.0f)));
      }
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
#define MTG_PF_ATTN(KVH, OUTF)                                                                                \
  hipLaunchKernelGGL((k_pf_attn_mma<KVH, OUTF>), grid, dim3(256), kPaLds, s, q, n_heads, n_kv_heads, kv, past0, S, \
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
  const void* fns[] = {(const void*)k_pf_attn_mma<0, false>, (const void*)k_pf_attn_mma<1, false>,
                       (const void*)k_pf_attn_mma<0, true>, (const void*)k_pf_attn_mma<1, true>};
  for (const void* f : fns) {
    const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kPaLds);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace mtg
