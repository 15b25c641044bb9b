// kernels_wt.hip - the f16, f32 and q4_K weight paths of the verify step (gfx950).
//
// Reference ops replaced (moss-transcribe.cpp through ggml's CPU backend; ggml
// itself is absent, its published semantics are restated):
//   k_act_f16 / k_act_q8k   rms_norm * gain, then mul_mat's conversion of the
//                           activation to vec_dot_type (F16 for f16 weights,
//                           Q8_K for q4_K)                src/qwen3.cpp:27-30,80,196
//   k_gemm_f16 / k_gemm_q4m mul_mat(W, x) (+ add / silu*mul); k_gemm_q4k and
//                           k_gemm_wt for other q4_K shapes
//                                                         src/qwen3.cpp:92-97,192-193,204-216
//   k_lm_head_f16m (f16 and f32) / k_lm_head_q4m
//                           tied lm_head + cpu_greedy_choice keys
//                                                         src/qwen3_decoder.cpp:174-205,
//                                                         src/cpu_speculative.cpp:39-50
//   k_attn_combine_wt / k_attn_combine_f16q
//                           the attention's chunk merge, written as the
//                           o-projection's activation     src/qwen3.cpp:172-189
//   k_embed_wt              get_rows / embed_rows_f32     src/generate.cpp:68-111
//
// Weights stay in the GGUF row layout: f16 [N][K] halves, q4_K [N][K/256] blocks
// of 144 bytes. The f16 kernels stage the activation in LDS and give a wave a
// group of rows; the q4_K kernels compute the exact integer sums of 16-row tiles
// on int8 MFMA.
//
// Canonical orders (shared with the oracle, which restates them on the CPU):
//   f16  : x rounded to f16; lane l of a wave takes the K/64 consecutive
//          elements [l*K/64, (l+1)*K/64) in an fma chain from 0 (the products of
//          two f16 values are exact in f32), then the 64 partials meet in the xor
//          butterfly 32, 16, 8, 4, 2, 1.
//   q4_K : x quantized to q8_K (ggml quantize_row_q8_K); per 256-superblock the
//          exact int32 sums dot = sum_s sc_s * dot_s and mins = sum_s mn_s * bsum_s;
//          then in superblock order acc = acc + (d_w*d_x)*dot, acc = acc -
//          (dmin_w*d_x)*mins.
#include <algorithm>
#include <type_traits>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "device_common.hpp"
#include "kernels.hpp"
#include "lm_f16.hpp"

namespace mtg {

namespace {
using namespace dev;
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

// Copy of n 16-byte pieces src[i] (i = tid, tid + nt, ...; at most MAXJ per thread)
// to dst(i), with every load of the thread issued before the first store: one
// memory round trip (a load / store loop waits for each load in turn).
template <int MAXJ, class Dst>
__device__ __forceinline__ void stage_pieces(const v4i* __restrict__ src, int n, int tid, int nt, Dst dst) {
  v4i r[MAXJ];
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int i = tid + j * nt;
    if (i < n) r[j] = src[i];
  }
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int i = tid + j * nt;
    if (i < n) *dst(i) = r[j];
  }
}


// ------------------------------------------------------- activations ------
// Grid (16 rows, K / 256), 256 threads: one element per thread. gain == nullptr:
// no norm (the SwiGLU product goes in as it is); otherwise every workgroup of a
// row recomputes the row's RMS scale (same order, same value). F32: the rows go
// out as they are (vec_dot_type F32), otherwise as f16.
template <bool F32>
__global__ void __launch_bounds__(256)
k_act_f16(const StepDesc* __restrict__ desc, const float* __restrict__ src, int K,
          const float* __restrict__ gain, float eps, uint16_t* __restrict__ out, float* __restrict__ out32,
          float* __restrict__ normed_out) {
  const int t = blockIdx.x, k = blockIdx.y * 256 + threadIdx.x;
  if (t >= desc->T) return;
  const float* xr = src + (size_t)t * K;
  __shared__ float s_scale;
  // the element and its gain load together with wave 0's row (one round trip)
  float y = xr[k];
  const float gk = gain ? gain[k] : 0.0f;
  if (gain) {
    if (threadIdx.x < 64) {
      const float sc = row_rms_scale(xr, K, eps);
      if (threadIdx.x == 0) s_scale = sc;
    }
    __syncthreads();
    y = __fmul_rn(__fmul_rn(y, s_scale), gk);
  }
  if (normed_out) normed_out[(size_t)t * K + k] = y;
  if constexpr (F32) out32[(size_t)t * K + k] = y;
  else out[(size_t)t * K + k] = __half_as_ushort(__float2half_rn(y));  // vec_dot_type F16
}


// Grid (16 rows, K / 256), 256 threads: block blockIdx.y of row blockIdx.x.
__global__ void __launch_bounds__(256)
k_act_q8k(const StepDesc* __restrict__ desc, const float* __restrict__ src, int K,
          const float* __restrict__ gain, float eps, ActQ8K a, float* __restrict__ normed_out) {
  const int t = blockIdx.x, b = blockIdx.y, k = b * 256 + threadIdx.x;
  if (t >= desc->T) return;
  const float* xr = src + (size_t)t * K;
  __shared__ float s_scale;
  // the element and its gain load together with wave 0's row (one round trip)
  float y = xr[k];
  const float gk = gain ? gain[k] : 0.0f;
  if (gain) {
    if (threadIdx.x < 64) {
      const float sc = row_rms_scale(xr, K, eps);
      if (threadIdx.x == 0) s_scale = sc;
    }
    __syncthreads();
    y = __fmul_rn(__fmul_rn(y, s_scale), gk);
  }
  if (normed_out) normed_out[(size_t)t * K + k] = y;
  q8k_block256(y, a, t, K, b);
}

// ------------------------------------------------- attention merge + act ---
// The chunk merge of the attention output (attn_merge's arithmetic: M = max of
// the chunk maxima, then the chunk-ordered chains L = fma(l_c, f_c, L) and
// O = fma(o_c, f_c, O), f_c = exp(m_c - M), out = O / L), fused with the
// conversion of the row to the o-projection's vec_dot_type. Grid (n_heads / 2,
// 16 rows), kCombSeg x 256 threads: thread (seg, hl, d) = (tid / 256, tid / 128
// % 2, tid % 128) takes q head 2 blockIdx.x + hl, element d, and the chunks of
// segment seg. Every segment's partials are loaded at once (one round trip for
// up to kCombPass chunks); the chains then run segment after segment, each
// continuing from the previous one's (L, O) in LDS, so the order stays the
// chunk order. A fully masked chunk (m = -inf) has f = 0, l = 0 and O = 0: its
// fma terms add exact zeros.
constexpr int kCombSeg = 4, kCombPer = 80, kCombPass = kCombSeg * kCombPer;

template <int WT>
__global__ void __launch_bounds__(256 * kCombSeg)
k_attn_combine_wt(const StepDesc* __restrict__ desc, AttnWork work, int n_heads, int max_chunks, WtAct act) {
  const int g = blockIdx.x, t = blockIdx.y;
  const int seg = threadIdx.x >> 8, tid = threadIdx.x & 255, hl = tid >> 7, d = tid & 127, lane = tid & 63;
  const int T = desc->T;
  if (t >= T) return;
  const int col = hl * T + t;  // q head 2 g + hl shares kv head g
  const int nch = (desc->past + T + kChunk - 1) / kChunk;
  constexpr uint32_t so = kMaxCols * kHeadDim * 4, sml = kMaxCols * 2 * 4;  // bytes per chunk
  const size_t item0 = (size_t)g * max_chunks;
  // a chunk >= nch reads past num_records: zeros, no memory traffic
  const auto ro = __builtin_amdgcn_make_buffer_rsrc(work.part_o + item0 * kMaxCols * kHeadDim, 0,
                                                    (int)(nch * so), 0x00020000);
  const auto rml = __builtin_amdgcn_make_buffer_rsrc(work.part_ml + item0 * kMaxCols * 2, 0, (int)(nch * sml),
                                                     0x00020000);
  __shared__ float s_f[2][kCombPass], s_l[2][kCombPass];
  __shared__ float s_L[256], s_O[256];
  // waves 0 and 2 (segment 0, d < 64) compute M and the chunk factors of q head hl;
  // the (m, l) of the first pass stay in their registers (one round trip)
  const bool factors = seg == 0 && d < 64;
  constexpr int kMl = kCombPass / 64;
  float M = -INFINITY, m1[kMl], l1[kMl];
  if (factors) {
#pragma unroll
    for (int i = 0; i < kMl; ++i) {
      const uint32_t off = (uint32_t)(64 * i + lane) * sml + col * 8;
      const v2u ml = __builtin_amdgcn_raw_buffer_load_b64(rml, off, 0, 0);  // past nch: zeros
      const bool in = 64 * i + lane < nch;
      m1[i] = in ? __uint_as_float(ml.x) : -INFINITY;
      l1[i] = in ? __uint_as_float(ml.y) : 0.0f;
      M = fmaxf(M, m1[i]);
    }
    for (int c0 = kCombPass; c0 < nch; c0 += 64) {
      const float m = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rml, (c0 + lane) * sml + col * 8, 0, 0));
      M = fmaxf(M, c0 + lane < nch ? m : -INFINITY);
    }
    M = wave_max_f(M);
  }
  float L = 0.0f, O = 0.0f;
  for (int p0 = 0; p0 < nch; p0 += kCombPass) {
    const int c_lo = p0 + seg * kCombPer;
    float o[kCombPer];
#pragma unroll
    for (int i = 0; i < kCombPer; ++i)
      o[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           ro, (uint32_t)(c_lo + i) * so + (col * kHeadDim + d) * 4, 0, 0));
    if (factors) {
#pragma unroll
      for (int i = 0; i < kMl; ++i) {
        const int c = 64 * i + lane;
        float m = m1[i], l = l1[i];
        if (p0 > 0) {
          const uint32_t off = (uint32_t)(p0 + c) * sml + col * 8;
          const v2u ml = __builtin_amdgcn_raw_buffer_load_b64(rml, off, 0, 0);
          const bool in = p0 + c < nch;
          m = in ? __uint_as_float(ml.x) : -INFINITY;
          l = in ? __uint_as_float(ml.y) : 0.0f;
        }
        s_f[hl][c] = m == -INFINITY ? 0.0f : dev_expf(__fsub_rn(m, M));
        s_l[hl][c] = l;
      }
    }
    __syncthreads();
    for (int sg = 0; sg < kCombSeg; ++sg) {
      if (seg == sg) {
        if (sg > 0 || p0 > 0) {
          L = s_L[tid];
          O = s_O[tid];
        }
        // groups of 4 chunks up to the last one; the chunks past nch in the last
        // group have f = l = o = 0 (exact zero terms)
        const int n = nch - c_lo;
        if (n > 0) {
#pragma unroll
          for (int i = 0; i < kCombPer; i += 4) {
            if (i < n) {
              const v4f f4 = *(const v4f*)&s_f[hl][seg * kCombPer + i];
              const v4f l4 = *(const v4f*)&s_l[hl][seg * kCombPer + i];
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                L = fmaf(l4[j], f4[j], L);
                O = fmaf(o[i + j], f4[j], O);
              }
            }
          }
          s_L[tid] = L;
          s_O[tid] = O;
        }
      }
      __syncthreads();
    }
  }
  const float val = __fdiv_rn(s_O[tid], s_L[tid]);
  const int QN = n_heads * kHeadDim;
  if constexpr (WT == MTG_TYPE_F16) {
    if (seg == 0) act.f16h[(size_t)t * QN + g * 256 + tid] = __half_as_ushort(__float2half_rn(val));
  } else {
    q8k_block256(val, act.q8k, t, QN, g);
  }
}

// The same merge for an f16 o-projection activation, which needs no 256-element
// block per workgroup: grid (n_heads / 2, 16 rows, 4 quarters of head_dim), one
// wave per segment, lane (hl, e) = (lane / 32, lane % 32) takes q head
// 2 blockIdx.x + hl, element 32 blockIdx.z + e. Waves 0 and 1 compute the chunk
// factors of q heads 2 blockIdx.x and 2 blockIdx.x + 1. Four times the workgroups
// of k_attn_combine_wt, a quarter of the partial loads each.
constexpr int kCombDq = 32;

template <bool F32>
__global__ void __launch_bounds__(64 * kCombSeg)
k_attn_combine_f16q(const StepDesc* __restrict__ desc, AttnWork work, int n_heads, int max_chunks, WtAct act) {
  const int g = blockIdx.x, t = blockIdx.y;
  const int seg = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int hl = lane >> 5, d = kCombDq * (int)blockIdx.z + (lane & 31);
  const int T = desc->T;
  if (t >= T) return;
  const int col = hl * T + t;  // q head 2 g + hl shares kv head g
  const int nch = (desc->past + T + kChunk - 1) / kChunk;
  constexpr uint32_t so = kMaxCols * kHeadDim * 4, sml = kMaxCols * 2 * 4;  // bytes per chunk
  const size_t item0 = (size_t)g * max_chunks;
  // a chunk >= nch reads past num_records: zeros, no memory traffic
  const auto ro = __builtin_amdgcn_make_buffer_rsrc(work.part_o + item0 * kMaxCols * kHeadDim, 0,
                                                    (int)(nch * so), 0x00020000);
  const auto rml = __builtin_amdgcn_make_buffer_rsrc(work.part_ml + item0 * kMaxCols * 2, 0, (int)(nch * sml),
                                                     0x00020000);
  __shared__ float s_f[2][kCombPass], s_l[2][kCombPass];
  __shared__ float s_L[64], s_O[64];
  // waves 0 and 1 compute M and the chunk factors of q head fh = seg; the (m, l)
  // of the first pass stay in their registers (one round trip)
  const bool factors = seg < 2;
  const int fcol = seg * T + t;
  constexpr int kMl = kCombPass / 64;
  float M = -INFINITY, m1[kMl], l1[kMl];
  if (factors) {
#pragma unroll
    for (int i = 0; i < kMl; ++i) {
      const uint32_t off = (uint32_t)(64 * i + lane) * sml + fcol * 8;
      const v2u ml = __builtin_amdgcn_raw_buffer_load_b64(rml, off, 0, 0);  // past nch: zeros
      const bool in = 64 * i + lane < nch;
      m1[i] = in ? __uint_as_float(ml.x) : -INFINITY;
      l1[i] = in ? __uint_as_float(ml.y) : 0.0f;
      M = fmaxf(M, m1[i]);
    }
    for (int c0 = kCombPass; c0 < nch; c0 += 64) {
      const float m = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rml, (c0 + lane) * sml + fcol * 8, 0, 0));
      M = fmaxf(M, c0 + lane < nch ? m : -INFINITY);
    }
    M = wave_max_f(M);
  }
  float L = 0.0f, O = 0.0f;
  for (int p0 = 0; p0 < nch; p0 += kCombPass) {
    const int c_lo = p0 + seg * kCombPer;
    float o[kCombPer];
#pragma unroll
    for (int i = 0; i < kCombPer; ++i)
      o[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           ro, (uint32_t)(c_lo + i) * so + (col * kHeadDim + d) * 4, 0, 0));
    if (factors) {
#pragma unroll
      for (int i = 0; i < kMl; ++i) {
        const int c = 64 * i + lane;
        float m = m1[i], l = l1[i];
        if (p0 > 0) {
          const uint32_t off = (uint32_t)(p0 + c) * sml + fcol * 8;
          const v2u ml = __builtin_amdgcn_raw_buffer_load_b64(rml, off, 0, 0);
          const bool in = p0 + c < nch;
          m = in ? __uint_as_float(ml.x) : -INFINITY;
          l = in ? __uint_as_float(ml.y) : 0.0f;
        }
        s_f[seg][c] = m == -INFINITY ? 0.0f : dev_expf(__fsub_rn(m, M));
        s_l[seg][c] = l;
      }
    }
    __syncthreads();
    for (int sg = 0; sg < kCombSeg; ++sg) {
      if (seg == sg) {
        if (sg > 0 || p0 > 0) {
          L = s_L[lane];
          O = s_O[lane];
        }
        // groups of 4 chunks up to the last one; the chunks past nch in the last
        // group have f = l = o = 0 (exact zero terms)
        const int n = nch - c_lo;
        if (n > 0) {
#pragma unroll
          for (int i = 0; i < kCombPer; i += 4) {
            if (i < n) {
              const v4f f4 = *(const v4f*)&s_f[hl][seg * kCombPer + i];
              const v4f l4 = *(const v4f*)&s_l[hl][seg * kCombPer + i];
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                L = fmaf(l4[j], f4[j], L);
                O = fmaf(o[i + j], f4[j], O);
              }
            }
          }
          s_L[lane] = L;
          s_O[lane] = O;
        }
      }
      __syncthreads();
    }
  }
  if (seg == 0) {
    const float val = __fdiv_rn(s_O[lane], s_L[lane]);
    const size_t i = (size_t)t * n_heads * kHeadDim + g * 256 + hl * kHeadDim + d;
    if constexpr (F32) act.f32[i] = val;
    else act.f16h[i] = __half_as_ushort(__float2half_rn(val));
  }
}

// ------------------------------------------------------------ row dots ----
// q4_K: lane l takes elements 4(l%8)..+3 of sub-block l/8 of each superblock.
__device__ __forceinline__ void q4k_row_dots(const uint8_t* __restrict__ wrow, const ActQ8K& a,
                                             int K, int T, float* res) {
  const int lane = threadIdx.x & 63, s = lane >> 3, j0 = 4 * (lane & 7);
  const int nb = K / 256;
#pragma unroll
  for (int t = 0; t < kMaxRows; ++t) res[t] = 0.0f;
  for (int b = 0; b < nb; ++b) {
    const uint8_t* blk = wrow + (size_t)b * 144;
    const float dw = half_bits_to_float(*(const uint16_t*)blk);
    const float dminw = half_bits_to_float(*(const uint16_t*)(blk + 2));
    const uint8_t* sc12 = blk + 4;
    int sc, mn;  // get_scale_min_k4 of sub-block s
    if (s < 4) {
      sc = sc12[s] & 63;
      mn = sc12[s + 4] & 63;
    } else {
      sc = (sc12[s + 4] & 0xF) | ((sc12[s - 4] >> 6) << 4);
      mn = (sc12[s + 4] >> 4) | ((sc12[s] >> 6) << 4);
    }
    const uint32_t qb = *(const uint32_t*)(blk + 16 + (s >> 1) * 32 + j0);
    const int nib = (int)((s & 1) ? (qb >> 4) & 0x0F0F0F0Fu : qb & 0x0F0F0F0Fu);
#pragma unroll
    for (int t = 0; t < kMaxRows; ++t) {
      if (t >= T) break;
      const int xq = *(const int*)(a.qs + (size_t)t * K + b * 256 + s * 32 + j0);
      const int part = __builtin_amdgcn_sdot4(nib, xq, 0, false);
      const int dot = wave_sum_i(sc * part);
      const int mcontrib =
          (lane & 7) == 0
              ? mn * (a.bsums[(size_t)t * (K / 16) + b * 16 + 2 * s] + a.bsums[(size_t)t * (K / 16) + b * 16 + 2 * s + 1])
              : 0;
      const int mins = wave_sum_i(mcontrib);
      const float dx = a.d[(size_t)t * nb + b];
      const float d = __fmul_rn(dw, dx), dmin = __fmul_rn(dminw, dx);
      res[t] = __fadd_rn(res[t], __fmul_rn(d, (float)dot));
      res[t] = __fsub_rn(res[t], __fmul_rn(dmin, (float)mins));
    }
  }
}

template <int WT, int SEG>
__device__ __forceinline__ void row_dots(const uint8_t* w, int row, int K, const float* xa, const ActQ8K& a,
                                         int T, float* res) {
  static_assert(WT == MTG_TYPE_Q4_K, "f16 rows go through k_gemm_f16 / k_lm_head_f16m");
  q4k_row_dots(w + (size_t)row * (K / 256) * 144, a, K, T, res);
}

// ---------------------------------------------------------------- GEMM ----
// EPI 0: store, 1: residual add, 2: silu(W x) * (W2 x). One wave per row.
template <int WT, int SEG, int EPI>
__global__ void __launch_bounds__(256)
k_gemm_wt(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w,
          const uint8_t* __restrict__ w2, int n, int K, const float* __restrict__ xa, ActQ8K a,
          float* __restrict__ out) {
  const int T = desc->T;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= n) return;
  float r1[kMaxRows], r2[kMaxRows];
  row_dots<WT, SEG>(w, row, K, xa, a, T, r1);
  if (EPI == 2) row_dots<WT, SEG>(w2, row, K, xa, a, T, r2);
  if (lane != 0) return;
#pragma unroll
  for (int t = 0; t < kMaxRows; ++t) {
    if (t >= T) break;
    float* dst = out + (size_t)t * n + row;
    if (EPI == 0) *dst = r1[t];
    else if (EPI == 1) *dst = __fadd_rn(*dst, r1[t]);
    else *dst = dev_swiglu(r1[t], r2[t]);
  }
}

// ------------------------------------------------------------- lm_head ----
// Grid-stride over rows; per verify row the best 64-bit key (value bits, lowest
// index on ties) of each workgroup goes to part_keys, as the q8_0 lm_head does.
template <int WT, int SEG>
__global__ void __launch_bounds__(256)
k_lm_head_wt(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, int vocab, int K,
             const float* __restrict__ xa, ActQ8K a, const uint32_t* __restrict__ bitmap,
             float* __restrict__ logits, uint64_t* __restrict__ part_keys) {
  const int T = desc->T;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int nwaves = gridDim.x * 4;
  const bool pen = desc->penalty > 1.0f;
  const float penalty = desc->penalty;
  const int words = (vocab + 31) / 32;
  uint64_t best[kMaxRows];
#pragma unroll
  for (int t = 0; t < kMaxRows; ++t) best[t] = 0;
  float res[kMaxRows];
  for (int row = blockIdx.x * 4 + wave; row < vocab; row += nwaves) {
    row_dots<WT, SEG>(w, row, K, xa, a, T, res);
#pragma unroll
    for (int t = 0; t < kMaxRows; ++t) {
      if (t >= T) break;
      float v = res[t];
      if (desc->write_logits && lane == 0) logits[(size_t)t * vocab + row] = v;
      if (pen && ((bitmap[(size_t)t * words + (row >> 5)] >> (row & 31)) & 1u))
        v = v > 0.0f ? __fdiv_rn(v, penalty) : __fmul_rn(v, penalty);
      const uint64_t key = argmax_key(v, row);
      best[t] = key > best[t] ? key : best[t];
    }
  }
  __shared__ uint64_t s_best[4][kMaxRows];
  if (lane == 0)
#pragma unroll
    for (int t = 0; t < kMaxRows; ++t) s_best[wave][t] = best[t];
  __syncthreads();
  if ((int)threadIdx.x < T) {
    uint64_t b = s_best[0][threadIdx.x];
    for (int wv = 1; wv < 4; ++wv) b = s_best[wv][threadIdx.x] > b ? s_best[wv][threadIdx.x] : b;
    part_keys[(size_t)blockIdx.x * kMaxRows + threadIdx.x] = b;
  }
}

// --------------------------------------------------------------- embed -----
template <int WT>
__global__ void k_embed_wt(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, int hidden,
                           const float* __restrict__ host_rows, float* __restrict__ x) {
  const int t = blockIdx.x;
  if (t >= desc->T) return;
  float* xr = x + (size_t)t * hidden;
  if (desc->use_embeds) {
    for (int k = threadIdx.x; k < hidden; k += blockDim.x) xr[k] = host_rows[(size_t)t * hidden + k];
    return;
  }
  const int n = desc->tokens[t];
  for (int k = threadIdx.x; k < hidden; k += blockDim.x) {
    if constexpr (WT == MTG_TYPE_F16) {
      xr[k] = half_bits_to_float(((const uint16_t*)w)[(size_t)n * hidden + k]);
    } else if constexpr (WT == MTG_TYPE_F32) {
      xr[k] = ((const float*)w)[(size_t)n * hidden + k];
    } else {  // dequantize_row_q4_K
      const uint8_t* blk = w + ((size_t)n * (hidden / 256) + k / 256) * 144;
      const int e = k % 256, s = e / 32, l = e % 32;
      const uint8_t* sc12 = blk + 4;
      int sc, mn;
      if (s < 4) {
        sc = sc12[s] & 63;
        mn = sc12[s + 4] & 63;
      } else {
        sc = (sc12[s + 4] & 0xF) | ((sc12[s - 4] >> 6) << 4);
        mn = (sc12[s + 4] >> 4) | ((sc12[s] >> 6) << 4);
      }
      const uint8_t qb = blk[16 + (s / 2) * 32 + l];
      const int v = (s & 1) ? (qb >> 4) : (qb & 0xF);
      const float d1 = __fmul_rn(half_bits_to_float(*(const uint16_t*)blk), (float)sc);
      const float m1 = __fmul_rn(half_bits_to_float(*(const uint16_t*)(blk + 2)), (float)mn);
      xr[k] = __fsub_rn(__fmul_rn(d1, (float)v), m1);
    }
  }
}

// ------------------------------------------------- q4_K, task per lane ----
// The workgroup stages the q8_K activation of every verify row in LDS; each wave
// stages a batch of D weight rows (NM matrices) there, the next batch already in
// flight in registers. Lane = task (row of the batch, superblock b, verify row t):
// the exact int32 dot sum_s sc_s * dot_s over the superblock's 256 elements
// (64 sdot4) and mins = sum_s mn_s * bsum_s, with no lane exchanges (integer sums
// are exact in any order). A lane per (batch row, verify row) then runs the
// canonical float chain over superblocks in order:
//   acc = acc + (d_w*d_x)*dot,  acc = acc - (dmin_w*d_x)*mins.
constexpr int kQ4MaxK = 3072;
constexpr int kQ4Slots = (kQ4MaxK / 256 * 9 + 63) / 64;  // 16-byte weight pieces per lane and row
constexpr int kQ4GemmD = 1, kQ4LmD = 4;                   // weight rows per wave and batch

__host__ __device__ constexpr int q4_act_stride(int K) { return K + 16; }        // bytes; spreads LDS banks
__host__ __device__ constexpr int q4_bs_stride(int K) { return K / 16 + 4; }     // ints
__host__ __device__ constexpr size_t q4_lds_bytes(int K, int rows_per_wave) {
  // act [16][K+16] + bsums [16][K/16+4] + dx [16][K/256] + per wave: the batch's
  // weight rows and their (dot, mins) [rows][K/256][16][2]
  return (size_t)kMaxRows * q4_act_stride(K) + (size_t)kMaxRows * q4_bs_stride(K) * 4 +
         (size_t)kMaxRows * (K / 256) * 4 + 4 * (size_t)rows_per_wave * (K / 256) * (144 + kMaxRows * 8);
}

struct Q4Lds {
  const int8_t* act;
  const int* bs;
  const float* dx;
  uint8_t* w;  // this wave's weight rows
  int* r;      // this wave's (dot, mins) results
};

__device__ __forceinline__ Q4Lds q4_stage(const ActQ8K& a, int K, int T, int rows_per_wave, uint8_t* lds) {
  const int tid = threadIdx.x, wave = tid >> 6, nb = K / 256;
  const int as = q4_act_stride(K), bst = q4_bs_stride(K);
  int8_t* act = (int8_t*)lds;
  int* bs = (int*)(lds + (size_t)kMaxRows * as);
  float* dx = (float*)(bs + kMaxRows * bst);
  uint8_t* wbase = (uint8_t*)(dx + kMaxRows * nb);
  const int pa = K / 16, pb = K / 64, nt = 256;  // 16-byte pieces per row; 256-thread workgroups
  // the scales first (one load each), then the codes and group sums with every
  // load in flight before the first LDS write
  float dxr[(kMaxRows * kQ4MaxK / 256 + 255) / 256];
#pragma unroll
  for (int j = 0; j < (kMaxRows * kQ4MaxK / 256 + 255) / 256; ++j)
    if (tid + j * nt < T * nb) dxr[j] = a.d[tid + j * nt];
  stage_pieces<kMaxRows * kQ4MaxK / 16 / 256>((const v4i*)a.qs, T * pa, tid, nt, [&](int i) {
    return (v4i*)(act + (size_t)(i / pa) * as + (i % pa) * 16);
  });
  stage_pieces<kMaxRows * kQ4MaxK / 64 / 256>((const v4i*)a.bsums, T * pb, tid, nt, [&](int i) {
    return (v4i*)(bs + (size_t)(i / pb) * bst + (i % pb) * 4);
  });
#pragma unroll
  for (int j = 0; j < (kMaxRows * kQ4MaxK / 256 + 255) / 256; ++j)
    if (tid + j * nt < T * nb) dx[tid + j * nt] = dxr[j];
  __syncthreads();
  Q4Lds q;
  q.act = act;
  q.bs = bs;
  q.dx = dx;
  q.w = wbase + (size_t)wave * rows_per_wave * nb * 144;
  q.r = (int*)(wbase + 4 * (size_t)rows_per_wave * nb * 144) + (size_t)wave * rows_per_wave * nb * kMaxRows * 2;
  return q;
}

// get_scale_min_k4 of the 8 sub-blocks from the 12 packed bytes
__device__ __forceinline__ void q4k_scales(const uint8_t* sc12, int sc[8], int mn[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = sc12[j] & 63;
    mn[j] = sc12[j + 4] & 63;
  }
#pragma unroll
  for (int j = 4; j < 8; ++j) {
    sc[j] = (sc12[j + 4] & 0xF) | ((sc12[j - 4] >> 6) << 4);
    mn[j] = (sc12[j + 4] >> 4) | ((sc12[j] >> 6) << 4);
  }
}

// Registers of one batch: rows row0 + d*rstride (d < D) of the NM matrices.
template <int NM, int D>
struct Q4Batch {
  v4i v[NM][D][kQ4Slots];
};

template <int NM, int D>
__device__ __forceinline__ void q4k_load(const uint8_t* const (&base)[NM], int n, int nb, int row0, int rstride,
                                         Q4Batch<NM, D>& bt) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    const int row = row0 + d * rstride;
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int j = 0; j < kQ4Slots; ++j) {
        const int i = lane + 64 * j;
        if (row < n && i < nb * 9) bt.v[m][d][j] = ((const v4i*)(base[m] + (size_t)row * nb * 144))[i];
      }
  }
}

// The batch in registers to the wave's LDS rows, then every (row, superblock,
// verify row) task; lane (d, t) = (lane >> 4, lane & 15) returns res[m] of batch
// row d (d < D, in steps of 4 for D > 4) and verify row t < T.
template <int NM, int D>
__device__ __forceinline__ void q4k_batch(const Q4Batch<NM, D>& bt, int K, int T, const Q4Lds& q,
                                          float (&res)[NM][(D + 3) / 4]) {
  const int lane = threadIdx.x & 63, nb = K / 256;
  const int as = q4_act_stride(K), bst = q4_bs_stride(K);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous batch's LDS reads are done
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int j = 0; j < kQ4Slots; ++j) {
        const int i = lane + 64 * j;
        if (i < nb * 9) ((v4i*)(q.w + (size_t)(m * D + d) * nb * 144))[i] = bt.v[m][d][j];
      }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's LDS writes are done
  const int ntask = NM * D * nb * T;
  for (int task = lane; task < ntask; task += 64) {
    const int rb = task / T, t = task - rb * T;  // rb = (m*D + d)*nb + b
    const int b = rb % nb;
    const uint8_t* blk = q.w + (size_t)rb * 144;
    int sc[8], mn[8];
    q4k_scales(blk + 4, sc, mn);
    const v4i* xq = (const v4i*)(q.act + (size_t)t * as + b * 256);
    const v4i* qs = (const v4i*)(blk + 16);
    int dot = 0;
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {  // sub-blocks 2 mm (low nibbles) and 2 mm + 1 (high)
      int d0 = 0, d1 = 0;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const v4i wq = qs[mm * 2 + i];
        const v4i x0 = xq[(2 * mm) * 2 + i], x1 = xq[(2 * mm + 1) * 2 + i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          d0 = __builtin_amdgcn_sdot4(wq[e] & 0x0F0F0F0F, x0[e], d0, false);
          d1 = __builtin_amdgcn_sdot4((wq[e] >> 4) & 0x0F0F0F0F, x1[e], d1, false);
        }
      }
      dot += sc[2 * mm] * d0 + sc[2 * mm + 1] * d1;
    }
    const int* bsr = q.bs + (size_t)t * bst + b * 16;
    int mins = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) mins += mn[j] * (bsr[2 * j] + bsr[2 * j + 1]);
    int* r = q.r + ((size_t)rb * kMaxRows + t) * 2;
    r[0] = dot;
    r[1] = mins;
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const int t = lane & 15;
#pragma unroll
  for (int dd = 0; dd < (D + 3) / 4; ++dd) {
    const int d = (lane >> 4) + 4 * dd;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      float acc = 0.0f;
      if (t < T && d < D) {
        for (int b = 0; b < nb; ++b) {
          const int rb = (m * D + d) * nb + b;
          const uint8_t* blk = q.w + (size_t)rb * 144;
          const float dw = half_bits_to_float(*(const uint16_t*)blk);
          const float dminw = half_bits_to_float(*(const uint16_t*)(blk + 2));
          const float dxv = q.dx[t * nb + b];
          const int* r = q.r + ((size_t)rb * kMaxRows + t) * 2;
          const float dm = __fmul_rn(dw, dxv), dmin = __fmul_rn(dminw, dxv);
          acc = __fadd_rn(acc, __fmul_rn(dm, (float)r[0]));
          acc = __fsub_rn(acc, __fmul_rn(dmin, (float)r[1]));
        }
      }
      res[m][dd] = acc;
    }
  }
}

// EPI 0: store, 1: residual add, 2: silu(W x) * (W2 x). Wave w of the grid owns
// rows w + nwaves * (j*D + d).
template <int EPI, int D>
__global__ void __launch_bounds__(256)
k_gemm_q4k(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
           int n, int K, ActQ8K a, float* __restrict__ out) {
  extern __shared__ v4i q4_lds_v4[];
  constexpr int NM = EPI == 2 ? 2 : 1, DD = (D + 3) / 4;
  const int T = desc->T, lane = threadIdx.x & 63, nb = K / 256;
  const int nwaves = gridDim.x * 4;
  const uint8_t* base[NM];
  base[0] = w;
  if (EPI == 2) base[NM - 1] = w2;
  int row0 = blockIdx.x * 4 + (threadIdx.x >> 6);
  Q4Batch<NM, D> bt;
  q4k_load<NM, D>(base, n, nb, row0, nwaves, bt);  // before the staging: in flight meanwhile
  const Q4Lds q = q4_stage(a, K, T, NM * D, (uint8_t*)q4_lds_v4);
  for (; row0 < n; row0 += nwaves * D) {
    const Q4Batch<NM, D> cur = bt;
    if (row0 + nwaves * D < n) q4k_load<NM, D>(base, n, nb, row0 + nwaves * D, nwaves, bt);
    float res[NM][DD];
    q4k_batch<NM, D>(cur, K, T, q, res);
    const int t = lane & 15;
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) {
      const int d = (lane >> 4) + 4 * dd, row = row0 + d * nwaves;
      if (t < T && d < D && row < n) {
        float* dst = out + (size_t)t * n + row;
        if (EPI == 0) *dst = res[0][dd];
        else if (EPI == 1) *dst = __fadd_rn(*dst, res[0][dd]);
        else *dst = dev_swiglu(res[0][dd], res[NM - 1][dd]);
      }
    }
  }
}

// q4_K lm_head over the rows of the tied embedding, distributed as in k_gemm_q4k;
// per verify row the best 64-bit key (value bits, lowest index on ties) of each
// workgroup goes to part_keys.
__global__ void __launch_bounds__(256)
k_lm_head_q4k(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, int vocab, int K, ActQ8K a,
              const uint32_t* __restrict__ bitmap, float* __restrict__ logits, uint64_t* __restrict__ part_keys) {
  extern __shared__ v4i q4_lds_v4[];
  constexpr int D = kQ4LmD, DD = (D + 3) / 4;
  const int T = desc->T, wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nb = K / 256;
  const bool pen = desc->penalty > 1.0f;
  const float penalty = desc->penalty;
  const bool write_logits = desc->write_logits != 0;
  const int words = (vocab + 31) / 32;
  const int nwaves = gridDim.x * 4, t = lane & 15;
  const uint8_t* base[1] = {w};
  int row0 = blockIdx.x * 4 + wave;
  Q4Batch<1, D> bt;
  q4k_load<1, D>(base, vocab, nb, row0, nwaves, bt);
  const Q4Lds q = q4_stage(a, K, T, D, (uint8_t*)q4_lds_v4);
  uint64_t best = 0;  // lane (d, t): verify row t
  for (; row0 < vocab; row0 += nwaves * D) {
    const Q4Batch<1, D> cur = bt;
    if (row0 + nwaves * D < vocab) q4k_load<1, D>(base, vocab, nb, row0 + nwaves * D, nwaves, bt);
    float res[1][DD];
    q4k_batch<1, D>(cur, K, T, q, res);
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) {
      const int d = (lane >> 4) + 4 * dd, row = row0 + d * nwaves;
      if (t < T && d < D && row < vocab) {
        float v = res[0][dd];
        if (write_logits) logits[(size_t)t * vocab + row] = v;
        if (pen && ((bitmap[(size_t)t * words + (row >> 5)] >> (row & 31)) & 1u))
          v = v > 0.0f ? __fdiv_rn(v, penalty) : __fmul_rn(v, penalty);
        const uint64_t key = argmax_key(v, row);
        best = key > best ? key : best;
      }
    }
  }
  __shared__ uint64_t s_best[4][64];
  s_best[wave][lane] = best;
  __syncthreads();
  if ((int)threadIdx.x < T) {
    uint64_t b = 0;
    for (int i = 0; i < 16; ++i) {
      const uint64_t c = s_best[i >> 2][(i & 3) * 16 + threadIdx.x];
      b = c > b ? c : b;
    }
    part_keys[(size_t)blockIdx.x * kMaxRows + threadIdx.x] = b;
  }
}

// ------------------------------------------------ q4_K lm_head, int8 MFMA ----
// Tile = 16 rows of the tied embedding, all 16 verify rows. Per superblock the
// exact int32 sums come from v_mfma_i32_16x16x32_i8, one sub-block (32 elements)
// per instruction, accumulated over the superblock's 8 sub-blocks:
//   A = the nibbles q (0..15) of row l % 16, elements 8 (l / 16) .. + 7, times a
//       small factor (bytewise exact: every product fits a byte);
//   B = the q8_K codes x of verify row l % 16, the same elements.
// With the 6-bit scale split as sc = 8 hi + lo (hi, lo <= 7, q * hi <= 105):
//   dot  = sum_s sc_s sum_e q x = 8 * sum_s (hi_s q) . x + sum_s (lo_s q) . x
//   mins = sum_s mn_s bsum_s     =     sum_s (mn_s 1) . x
// Lane l then holds rows 4 (l / 16) + r (r < 4) of verify row l % 16 and runs the
// canonical float chain over the superblocks (d, dmin of its rows from LDS).
__host__ __device__ constexpr size_t q4m_lds_bytes(int K) {
  return q4_lds_bytes(K, 0) + 4 * (size_t)16 * 2 * 4;  // + per wave: d|dmin [16][2]
}


template <int NB>
struct Q4Tile {
  uint32_t q[NB][4][2];  // per superblock, pair mm: the lane's 8 nibble bytes
  v4i head[NB];          // the lane's row's d, dmin and 12 scale bytes
};

template <int NB>
__device__ __forceinline__ void q4m_load(const uint8_t* w, int n_tiles, int tile, Q4Tile<NB>& tl) {
  const int lane = threadIdx.x & 63, row = lane & 15, g = lane >> 4;
  if (tile >= n_tiles) return;
  const uint8_t* rb = w + ((size_t)tile * 16 + row) * NB * 144;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
      const uint2 u = *(const uint2*)(rb + b * 144 + 16 + 32 * mm + 8 * g);
      tl.q[b][mm][0] = u.x;
      tl.q[b][mm][1] = u.y;
    }
    tl.head[b] = *(const v4i*)(rb + b * 144);
  }
}

// res[r]: row 4 (lane / 16) + r of the tile, verify row lane % 16. The q8_K codes
// and scales come from the workgroup's LDS copy (xq / dxp in LDS, row stride as)
// or, for a single tile, straight from the activation buffers.
template <int NB>
__device__ __forceinline__ void q4m_tile(const Q4Tile<NB>& tl, const int8_t* xq, int as, const float* dxp,
                                         float* s_d, float (&res)[4]) {
  const int lane = threadIdx.x & 63, t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int r = 0; r < 4; ++r) res[r] = 0.0f;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const v4i h = tl.head[b];
    int sc[8], mn[8];
    q4k_scales_w((uint32_t)h[1], (uint32_t)h[2], (uint32_t)h[3], sc, mn);
    v4i ahi = {0, 0, 0, 0}, alo = {0, 0, 0, 0}, amn = {0, 0, 0, 0};
    const int8_t* xa = xq + (size_t)t * as + b * 256 + 8 * g;
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {  // sub-block 2 mm + hi: the low or high nibbles
        const int s = 2 * mm + hi;
        const uint32_t q0 = hi ? (tl.q[b][mm][0] >> 4) & 0x0F0F0F0Fu : tl.q[b][mm][0] & 0x0F0F0F0Fu;
        const uint32_t q1 = hi ? (tl.q[b][mm][1] >> 4) & 0x0F0F0F0Fu : tl.q[b][mm][1] & 0x0F0F0F0Fu;
        const uint32_t fh = (uint32_t)(sc[s] >> 3), fl = (uint32_t)(sc[s] & 7), fm = (uint32_t)mn[s] * 0x01010101u;
        const long bv = *(const long*)(xa + 32 * s);
        ahi = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)(((uint64_t)(q1 * fh) << 32) | (q0 * fh)), bv, ahi, 0, 0, 0);
        alo = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)(((uint64_t)(q1 * fl) << 32) | (q0 * fl)), bv, alo, 0, 0, 0);
        amn = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)(((uint64_t)fm << 32) | fm), bv, amn, 0, 0, 0);
      }
    }
    // d, dmin of the tile's rows through the wave's LDS slot (lanes 0..15 own them)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (g == 0) {
      s_d[t * 2] = half_bits_to_float((uint16_t)((uint32_t)h[0] & 0xffffu));
      s_d[t * 2 + 1] = half_bits_to_float((uint16_t)((uint32_t)h[0] >> 16));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const float dxv = dxp[t * NB + b];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int dot = 8 * ahi[r] + alo[r];
      const float dm = __fmul_rn(s_d[(4 * g + r) * 2], dxv), dmin = __fmul_rn(s_d[(4 * g + r) * 2 + 1], dxv);
      res[r] = __fadd_rn(res[r], __fmul_rn(dm, (float)dot));
      res[r] = __fsub_rn(res[r], __fmul_rn(dmin, (float)amn[r]));
    }
  }
}

// q4_K GEMM on the same tiles: one workgroup of 4 or 8 waves per 16-row tile (and
// per matrix pair for EPI 2). Wave w takes superblocks w, w + NW, ...: their exact
// int32 sums (dot, mins) of every (row, verify row) and the rows' d, dmin go to
// LDS, and wave 0 runs the canonical float chain over the superblocks in order.
// The activation operands come straight from the q8_K buffers (every tile reads
// them, from L2). EPI 0: store, 1: residual add, 2: silu(W x) * (W2 x).
__host__ __device__ constexpr size_t q4g_lds_bytes(int nb, int nm) {
  return (size_t)nm * nb * (2 * 4 * 64 * 4 + 16 * 2 * 4);  // [m][b] (dot, mins) [2][4][64] + d|dmin [16][2]
}

// waves per tile: 8 for the long rows (K >= 2048), whose few tiles would leave
// most of the machine idle with 4
__host__ __device__ constexpr int q4g_waves(int nb) { return nb >= 8 ? 8 : 4; }

// Every load of a workgroup goes out at its start, in one round trip: the weights,
// the activation codes of the wave's superblocks, and (wave 0) the chain's
// activation scales and the residual values of EPI 1. (Left to the compiler, the
// activation loads went out one sub-block at a time, each waited for before its
// MFMA.)
template <int EPI, int NB>
__global__ void __launch_bounds__(64 * q4g_waves(NB), 1)
k_gemm_q4m(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, int n,
           ActQ8K a, float* __restrict__ out) {
  constexpr int K = NB * 256, NM = EPI == 2 ? 2 : 1, NW = q4g_waves(NB), NBW = (NB + NW - 1) / NW;
  extern __shared__ v4i q4_lds_v4[];
  int* s_i = (int*)q4_lds_v4;                                 // [m][b][2][4][64]
  float* s_dd = (float*)(s_i + NM * NB * 2 * 4 * 64);        // [m][b][16][2]
  const int T = desc->T, wave = threadIdx.x >> 6, lane = threadIdx.x & 63, t = lane & 15, g = lane >> 4;
  const int row = lane & 15, tile = blockIdx.x;
  const uint8_t* const base[2] = {w, w2};
  uint32_t qw[NM][NBW][4][2];
  v4i head[NM][NBW];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int b = wave + NW * j;
      if (b < NB) {
        const uint8_t* rb = base[m] + ((size_t)tile * 16 + row) * NB * 144 + b * 144;
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
          const uint2 u = *(const uint2*)(rb + 16 + 32 * mm + 8 * g);
          qw[m][j][mm][0] = u.x;
          qw[m][j][mm][1] = u.y;
        }
        head[m][j] = *(const v4i*)rb;
      }
    }
  long xv[NBW][8];
#pragma unroll
  for (int j = 0; j < NBW; ++j) {
    const int b = wave + NW * j;
#pragma unroll
    for (int s = 0; s < 8; ++s) xv[j][s] = b < NB ? *(const long*)(a.qs + (size_t)t * K + b * 256 + 8 * g + 32 * s) : 0;
  }
  float dxv[NB], xres[4];
  if (wave == 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) dxv[b] = a.d[t * NB + b];
#pragma unroll
    for (int r = 0; r < 4; ++r) xres[r] = EPI == 1 && t < T ? out[(size_t)t * n + tile * 16 + 4 * g + r] : 0.0f;
  }
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int j = 0; j < NBW; ++j) {
      const int b = wave + NW * j;
      if (b >= NB) continue;
      const v4i h = head[m][j];
      int sc[8], mn[8];
      q4k_scales_w((uint32_t)h[1], (uint32_t)h[2], (uint32_t)h[3], sc, mn);
      v4i ahi = {0, 0, 0, 0}, alo = {0, 0, 0, 0}, amn = {0, 0, 0, 0};
#pragma unroll
      for (int mm = 0; mm < 4; ++mm)
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
          const int s = 2 * mm + hi;
          const uint32_t q0 = hi ? (qw[m][j][mm][0] >> 4) & 0x0F0F0F0Fu : qw[m][j][mm][0] & 0x0F0F0F0Fu;
          const uint32_t q1 = hi ? (qw[m][j][mm][1] >> 4) & 0x0F0F0F0Fu : qw[m][j][mm][1] & 0x0F0F0F0Fu;
          const uint32_t fh = (uint32_t)(sc[s] >> 3), fl = (uint32_t)(sc[s] & 7), fm = (uint32_t)mn[s] * 0x01010101u;
          const long bv = xv[j][s];
          ahi = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)(((uint64_t)(q1 * fh) << 32) | (q0 * fh)), bv, ahi, 0, 0, 0);
          alo = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)(((uint64_t)(q1 * fl) << 32) | (q0 * fl)), bv, alo, 0, 0, 0);
          amn = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)(((uint64_t)fm << 32) | fm), bv, amn, 0, 0, 0);
        }
      int* si = s_i + ((m * NB + b) * 2) * 4 * 64;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        si[r * 64 + lane] = 8 * ahi[r] + alo[r];
        si[(4 + r) * 64 + lane] = amn[r];
      }
      if (g == 0) {
        float* dd = s_dd + ((m * NB + b) * 16 + row) * 2;
        dd[0] = half_bits_to_float((uint16_t)((uint32_t)h[0] & 0xffffu));
        dd[1] = half_bits_to_float((uint16_t)((uint32_t)h[0] >> 16));
      }
    }
  __syncthreads();
  if (wave != 0) return;
  float res[NM][4];
#pragma unroll
  for (int m = 0; m < NM; ++m) {
#pragma unroll
    for (int r = 0; r < 4; ++r) res[m][r] = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int* si = s_i + ((m * NB + b) * 2) * 4 * 64;
      const float* dd = s_dd + (m * NB + b) * 16 * 2;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float dm = __fmul_rn(dd[(4 * g + r) * 2], dxv[b]), dmin = __fmul_rn(dd[(4 * g + r) * 2 + 1], dxv[b]);
        res[m][r] = __fadd_rn(res[m][r], __fmul_rn(dm, (float)si[r * 64 + lane]));
        res[m][r] = __fsub_rn(res[m][r], __fmul_rn(dmin, (float)si[(4 + r) * 64 + lane]));
      }
    }
  }
  if (t < T) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* dst = out + (size_t)t * n + tile * 16 + 4 * g + r;
      if (EPI == 0) *dst = res[0][r];
      else if (EPI == 1) *dst = __fadd_rn(xres[r], res[0][r]);
      else *dst = dev_swiglu(res[0][r], res[NM - 1][r]);
    }
  }
}

template <int NB>
__global__ void __launch_bounds__(256)
k_lm_head_q4m(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, int vocab, ActQ8K a,
              const uint32_t* __restrict__ bitmap, float* __restrict__ logits, uint64_t* __restrict__ part_keys) {
  constexpr int K = NB * 256;
  extern __shared__ v4i q4_lds_v4[];
  const int T = desc->T, wave = threadIdx.x >> 6, lane = threadIdx.x & 63, t = lane & 15, g = lane >> 4;
  const bool pen = desc->penalty > 1.0f;
  const float penalty = desc->penalty;
  const bool write_logits = desc->write_logits != 0;
  const int words = (vocab + 31) / 32, n_tiles = vocab / 16, nwaves = gridDim.x * 4;
  int tile = blockIdx.x * 4 + wave;
  Q4Tile<NB> nx;
  q4m_load<NB>(w, n_tiles, tile, nx);
  const Q4Lds q = q4_stage(a, K, T, 0, (uint8_t*)q4_lds_v4);
  float* s_d = (float*)((uint8_t*)q4_lds_v4 + q4_lds_bytes(K, 0)) + wave * 16 * 2;
  uint64_t best = 0;  // lane (g, t): verify row t
  for (; tile < n_tiles; tile += nwaves) {
    const Q4Tile<NB> cur = nx;
    if (tile + nwaves < n_tiles) q4m_load<NB>(w, n_tiles, tile + nwaves, nx);
    float res[4];
    q4m_tile<NB>(cur, q.act, q4_act_stride(K), q.dx, s_d, res);
    if (t < T) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = tile * 16 + 4 * g + r;
        float v = res[r];
        if (write_logits) logits[(size_t)t * vocab + row] = v;
        if (pen && ((bitmap[(size_t)t * words + (row >> 5)] >> (row & 31)) & 1u))
          v = v > 0.0f ? __fdiv_rn(v, penalty) : __fmul_rn(v, penalty);
        const uint64_t key = argmax_key(v, row);
        best = key > best ? key : best;
      }
    }
  }
  __shared__ uint64_t s_best[4][64];
  s_best[wave][lane] = best;
  __syncthreads();
  if ((int)threadIdx.x < T) {
    uint64_t b = 0;
    for (int i = 0; i < 16; ++i) {
      const uint64_t c = s_best[i >> 2][(i & 3) * 16 + threadIdx.x];
      b = c > b ? c : b;
    }
    part_keys[(size_t)blockIdx.x * kMaxRows + threadIdx.x] = b;
  }
}

// ------------------------------------------------------ f16, row groups ----
// The workgroup stages the f16 activation rows [T][K] in LDS once; a wave takes
// NR weight rows (of each of NM matrices) at a time, the next group's rows in
// flight in registers. Lane l runs the canonical fma chain over its K/64
// elements for every (matrix, row, verify row) output; the 64 lane partials of
// an output meet in LDS as one row of kF16PStride words (lane writes: consecutive
// words; one lane then reads the row with 16-byte loads, conflict-free) and that
// lane adds them in the pairing of the xor butterfly 32, 16, 8, 4, 2, 1 (the same
// additions as wave_sum_f: IEEE sums commute). Lane j < 16 NR ends with the
// outputs of row j / 16, verify row j % 16.
//
// Order of the memory traffic: the activation loads are issued first, then the
// weight rows (loads complete in order, so the activation's arrival, its LDS
// writes and the norm prologue's arithmetic overlap the weights' flight), then
// the residual values an EPI 1 store adds to.
template <int SEG, int NM, int NR>
struct F16Group {
  v4i w[NM][NR][SEG / 8];  // the lane's K/64 halves of each row, 8 per piece
};

constexpr int kF16PStride = 68;  // words per partial row (a multiple of 4 for 16-byte reads)

__host__ __device__ constexpr size_t f16_lds_bytes(int K, int nm_nr, int nwv = 4) {
  return (size_t)kMaxRows * K * 2 + (size_t)nwv * nm_nr * kMaxRows * kF16PStride * 4;
}

// rows past n are clamped to row n - 1 (loaded, never stored): no branches
// between the loads
template <int SEG, int NM, int NR>
__device__ __forceinline__ void f16_load(const uint16_t* const (&base)[NM], int n, int row0,
                                         F16Group<SEG, NM, NR>& g) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int row = min(row0 + r, n - 1);
#pragma unroll
      for (int c = 0; c < SEG / 8; ++c)
        g.w[m][r][c] = *(const v4i*)(base[m] + (size_t)row * (SEG * 64) + lane * SEG + 8 * c);
    }
}

__device__ __forceinline__ float h_lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
__device__ __forceinline__ float h_hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// verify rows per pass of f16_group (their fma chains interleaved; measured best
// for every row group here, one to six rows per wave)
constexpr int kF16TT = 2;

template <int SEG, int NM, int NR, int TT = kF16TT>
__device__ __forceinline__ void f16_group(const F16Group<SEG, NM, NR>& g, const uint16_t* s_x, int T, float* s_p,
                                          float (&res)[NM]) {
  constexpr int K = SEG * 64, NC = SEG / 8;
  static_assert(kMaxRows % TT == 0, "passes of TT rows cover the LDS rows");
  const int lane = threadIdx.x & 63;
  float wf[NM][NR][SEG];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t u = (uint32_t)g.w[m][r][c][q];
          wf[m][r][8 * c + 2 * q] = h_lo(u);
          wf[m][r][8 * c + 2 * q + 1] = h_hi(u);
        }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous group's partial reads are done
  // a pass takes verify rows t0 .. t0 + TT - 1; rows from T on (stale LDS rows,
  // inside the kMaxRows staged) are computed and their partials written to slots
  // the sums never read
  const uint16_t* xr = s_x + lane * SEG;
  v4i xv[TT][NC], xnext[TT][NC];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt)
#pragma unroll
    for (int c = 0; c < NC; ++c) xv[tt][c] = *(const v4i*)(xr + tt * K + 8 * c);
#pragma unroll
  for (int t0 = 0; t0 < kMaxRows; t0 += TT) {  // constant indices keep the sums in registers
    if (t0 >= T) break;
    if (t0 + TT < T) {  // the next pass's activation in flight during this one's chains
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int c = 0; c < NC; ++c) xnext[tt][c] = *(const v4i*)(xr + (t0 + TT + tt) * K + 8 * c);
    }
    float acc[TT][NM][NR];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[tt][m][r] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float xf[TT][8];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          xf[tt][2 * q] = h_lo((uint32_t)xv[tt][c][q]);
          xf[tt][2 * q + 1] = h_hi((uint32_t)xv[tt][c][q]);
        }
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[tt][m][r] = fmaf(wf[m][r][8 * c + e], xf[tt][e], acc[tt][m][r]);
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r)
          s_p[((m * NR + r) * kMaxRows + t0 + tt) * kF16PStride + lane] = acc[tt][m][r];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int c = 0; c < NC; ++c) xv[tt][c] = xnext[tt][c];
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's partial writes are done
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    float v[64];
    const v4f* col = (const v4f*)(s_p + ((m * NR) * kMaxRows + lane) * kF16PStride);
    if (lane < NR * kMaxRows && (lane & 15) < T) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const v4f q = col[i];
        v[4 * i] = q[0];
        v[4 * i + 1] = q[1];
        v[4 * i + 2] = q[2];
        v[4 * i + 3] = q[3];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 64; ++i) v[i] = 0.0f;
    }
#pragma unroll
    for (int h = 32; h >= 1; h >>= 1)
#pragma unroll
      for (int i = 0; i < h; ++i) v[i] = v[i] + v[i + h];
    res[m] = v[0];
  }
}

// The f16 activation rows of a K = 1024 GEMM computed in the workgroup from the
// residual rows x: RMSNorm(x) * gain rounded to f16, k_act_f16's arithmetic (lane l
// sums the squares of elements 16 l .. 16 l + 15 in double, the butterfly, the
// correctly rounded 1 / sqrt, y = (x * scale) * gain, then f16), written to s_x.
// Wave w of NWV takes rows w, w + NWV, .. (16 / NWV of them), their double sums
// side by side.
// load() issues the loads of all kMaxRows rows of x (rows from T on are in the
// buffer and never stored: the loads need not wait for the step descriptor's T),
// store() waits for them and writes rows 0 .. T - 1.
template <int NWV>
struct F16NormRows {
  static constexpr int RW = kMaxRows / NWV;  // rows per wave
  static_assert(kMaxRows % NWV == 0 && RW % 2 == 0, "an even number of rows per wave");
  v4f raw[RW][4], gv[4];

  __device__ __forceinline__ void load(const float* __restrict__ x, const float* __restrict__ gain) {
    constexpr int K = 1024;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      const int t = wave + NWV * j;
#pragma unroll
      for (int i = 0; i < 4; ++i) raw[j][i] = *(const v4f*)(x + (size_t)t * K + 16 * lane + 4 * i);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) gv[i] = *(const v4f*)(gain + 16 * lane + 4 * i);
  }

  __device__ __forceinline__ void store(float eps, int T, uint16_t* s_x) {
    constexpr int K = 1024;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    double sq[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) sq[j] = 0.0;
#pragma unroll
    for (int e = 0; e < 16; ++e)
#pragma unroll
      for (int j = 0; j < RW; ++j) sq[j] += (double)__fmul_rn(raw[j][e >> 2][e & 3], raw[j][e >> 2][e & 3]);
    float sc[RW];
    rms_scales<RW, K>(sq, eps, sc);
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      const int t = wave + NWV * j;
      if (t >= T) break;
      const float scale = sc[j];
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        float y0 = __fmul_rn(__fmul_rn(raw[j][e >> 2][e & 3], scale), gv[e >> 2][e & 3]);
        float y1 = __fmul_rn(__fmul_rn(raw[j][(e + 1) >> 2][(e + 1) & 3], scale), gv[(e + 1) >> 2][(e + 1) & 3]);
        // the float products first: the compiler would otherwise fold the last
        // multiply and the conversion into one fma_mix (one rounding, not two)
        asm volatile("" : "+v"(y0), "+v"(y1));
        h[e / 2] = (uint32_t)__half_as_ushort(__float2half_rn(y0)) |
                   ((uint32_t)__half_as_ushort(__float2half_rn(y1)) << 16);
      }
      uint4* dst = (uint4*)(s_x + t * K + 16 * lane);
      dst[0] = make_uint4(h[0], h[1], h[2], h[3]);
      dst[1] = make_uint4(h[4], h[5], h[6], h[7]);
    }
  }
};

// The f16 activation rows [T][K] copied to LDS: load() issues every load of the
// thread (all kMaxRows rows of the buffer, without waiting for T), store() writes
// rows 0 .. T - 1 (one memory round trip).
template <int K, int NT>
struct F16StageRows {
  static constexpr int kPieces = kMaxRows * K / 8 / NT;
  v4i r[kPieces];

  __device__ __forceinline__ void load(const uint16_t* __restrict__ xh) {
#pragma unroll
    for (int j = 0; j < kPieces; ++j) r[j] = ((const v4i*)xh)[(int)threadIdx.x + NT * j];
  }

  __device__ __forceinline__ void store(int T, uint16_t* s_x) {
    const int n = T * K / 8;
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const int i = (int)threadIdx.x + NT * j;
      if (i < n) ((v4i*)s_x)[i] = r[j];
    }
  }
};

// EPI 0: store, 1: residual add, 2: silu(W x) * (W2 x) written as f16 (the
// down projection's vec_dot_type: out then holds f16 rows [T][n], in place of
// the float rows and their conversion by k_act_f16, which gives the same bits).
// NORM (K = 1024): the activation is RMSNorm(xn) * gain of the residual rows xn,
// computed here (F16NormRows) instead of by a k_act_f16 launch before. NWV waves
// per workgroup (one workgroup per CU: its LDS admits no second).
template <int EPI, int SEG, int NR, bool NORM = false, int NWV = 4>
__global__ void __launch_bounds__(64 * NWV)
k_gemm_f16(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, int n,
           const uint16_t* __restrict__ xh, float* __restrict__ out, const float* __restrict__ xn = nullptr,
           const float* __restrict__ gain = nullptr, float eps = 0.0f) {
  constexpr int K = SEG * 64, NM = EPI == 2 ? 2 : 1;
  static_assert(!NORM || K == 1024, "the norm prologue covers the hidden rows");
  extern __shared__ v4i f16_lds_v4[];
  uint16_t* s_x = (uint16_t*)f16_lds_v4;
  const int T = desc->T, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* s_p = (float*)(s_x + kMaxRows * K) + wave * (NM * NR * kMaxRows * kF16PStride);
  const int ngroups = (n + NR - 1) / NR, nwaves = gridDim.x * NWV;
  const uint16_t* base[NM];
  base[0] = (const uint16_t*)w;
  if (NM == 2) base[NM - 1] = (const uint16_t*)w2;
  const int r = lane >> 4, t = lane & 15;
  int g = blockIdx.x * NWV + wave;
  typename std::conditional<NORM, F16NormRows<NWV>, F16StageRows<K, 64 * NWV>>::type act;
  if constexpr (NORM)
    act.load(xn, gain);
  else
    act.load(xh);
  F16Group<SEG, NM, NR> bt;
  f16_load<SEG, NM, NR>(base, n, g * NR, bt);
  float old = 0.0f;  // EPI 1: the value the first group's output adds to
  if (EPI == 1 && g < ngroups && r < NR && t < T && g * NR + r < n) old = out[(size_t)t * n + g * NR + r];
  if constexpr (NORM)
    act.store(eps, T, s_x);
  else
    act.store(T, s_x);
  __syncthreads();
  for (bool first = true; g < ngroups; g += nwaves, first = false) {
    const F16Group<SEG, NM, NR> cur = bt;
    const int row = g * NR + r;
    const bool mine = r < NR && t < T && row < n;
    if (EPI == 1 && !first && mine) old = out[(size_t)t * n + row];
    if (g + nwaves < ngroups) f16_load<SEG, NM, NR>(base, n, (g + nwaves) * NR, bt);
    float res[NM];
    f16_group<SEG, NM, NR>(cur, s_x, T, s_p, res);
    if (mine) {
      float* dst = out + (size_t)t * n + row;
      if (EPI == 0) *dst = res[0];
      else if (EPI == 1) *dst = __fadd_rn(old, res[0]);
      else {
        // the float product first: the compiler would otherwise fold the multiply
        // and the conversion into one fma_mix, rounding once instead of twice
        float v = dev_swiglu(res[0], res[NM - 1]);
        asm volatile("" : "+v"(v));
        ((uint16_t*)out)[(size_t)t * n + row] = __half_as_ushort(__float2half_rn(v));
      }
    }
  }
}

// ------------------------------------------------- f16 lm_head, f32 MFMA ----
// The canonical f16 dots of the tied lm_head as chained v_mfma_f32_16x16x4f32
// segment chains folded by the butterfly's tree (lm_f16.hpp), over a copy of the
// embedding re-tiled at load time.
//
// k_lm16_retile: thread = (tile, piece, lane) of the copy, 16 bytes: the halves
// 16 l + 4 s + kk (s < 4) of row 16 tile + m for the piece's two segments.
__global__ void __launch_bounds__(256)
k_lm16_retile(const uint16_t* __restrict__ w, int n_tiles, uint16_t* __restrict__ out) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)n_tiles * kLm16Pieces * 64) return;
  const int lane = (int)(i & 63), q = (int)((i >> 6) & (kLm16Pieces - 1)), m = lane & 15, kk = lane >> 4;
  const uint16_t* row = w + ((i >> 11) * 16 + m) * 1024;
  uint32_t h[4];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const uint16_t* e = row + 16 * lm16_bitrev6(2 * q + s2) + kk;
    h[2 * s2] = (uint32_t)e[0] | ((uint32_t)e[4] << 16);
    h[2 * s2 + 1] = (uint32_t)e[8] | ((uint32_t)e[12] << 16);
  }
  *(uint4*)(out + i * 8) = make_uint4(h[0], h[1], h[2], h[3]);
}

// The f32 copy: thread = (tile, piece, lane), 16 bytes: the floats 16 l + 4 s + kk
// (s < 4) of row 16 tile + m, segment l = bitrev6(piece).
__global__ void __launch_bounds__(256)
k_lm32_retile(const float* __restrict__ w, int n_tiles, float* __restrict__ out) {
  constexpr int NPC = LmTile<true>::kPieces;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)n_tiles * NPC * 64) return;
  const int lane = (int)(i & 63), q = (int)((i >> 6) & (NPC - 1)), m = lane & 15, kk = lane >> 4;
  const float* e = w + ((i >> 12) * 16 + m) * 1024 + 16 * lm16_bitrev6(q) + kk;
  *(v4f*)(out + i * 4) = v4f{e[0], e[4], e[8], e[12]};
}

// The per-op lm_head of f16 (and F32: f32) weights: 256 workgroups of 8 waves (two
// per SIMD), wave gw taking tiles gw, gw + 2,048, ..; the activation rows [T][1024]
// staged in LDS, then their B operands (96 / 128 KB). Per verify row the best key of
// each workgroup goes to part_keys (kLmWorkgroups slots per row: the first of the
// workgroup's four, the smallest key, 0, in the others).
constexpr int kLm16NWV = 8, kLm16Blocks = kLmWorkgroups / 4;
__host__ __device__ constexpr size_t lm_lds_bytes(bool f32) {
  return (size_t)kLm16BFloats * 4 + (size_t)kMaxRows * 1024 * (f32 ? 4 : 2);
}

template <bool F32>
__global__ void __launch_bounds__(64 * kLm16NWV)
k_lm_head_f16m(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, int vocab,
               const void* __restrict__ xa, const uint32_t* __restrict__ bitmap, float* __restrict__ logits,
               uint64_t* __restrict__ part_keys) {
  constexpr int NT = 64 * kLm16NWV, EB = F32 ? 4 : 2;
  extern __shared__ v4i lm16_lds_v4[];
  float* s_b = (float*)lm16_lds_v4;
  v4i* s_x = (v4i*)(s_b + kLm16BFloats);
  const int T = desc->T, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  stage_pieces<kMaxRows * 1024 * EB / 16 / NT>((const v4i*)xa, T * 1024 * EB / 16, threadIdx.x, NT,
                                               [&](int i) { return s_x + i; });
  __syncthreads();
  lm16_stage_b<NT, F32>(s_x, T, s_b);
  __syncthreads();
  uint64_t b = lm16_run<16, F32>(w, blockIdx.x * kLm16NWV + wave, gridDim.x * kLm16NWV, vocab / 16, s_b, T, vocab,
                                 desc->penalty, bitmap, desc->write_logits ? logits : nullptr);
  // the four lanes of a verify row: m, m + 16, m + 32, m + 48
  uint64_t o = shfl_xor_u64(b, 16);
  b = o > b ? o : b;
  o = shfl_xor_u64(b, 32);
  b = o > b ? o : b;
  __shared__ uint64_t s_best[kLm16NWV][16];
  if (lane < 16) s_best[wave][lane] = b;
  __syncthreads();
  if ((int)threadIdx.x < T) {
    uint64_t best = 0;
    for (int i = 0; i < kLm16NWV; ++i) best = s_best[i][threadIdx.x] > best ? s_best[i][threadIdx.x] : best;
    const int pk = kLmWorkgroups / gridDim.x;
    for (int k = 0; k < pk; ++k)
      part_keys[((size_t)blockIdx.x * pk + k) * kMaxRows + threadIdx.x] = k == 0 ? best : 0;
  }
}

// ------------------------------------------------------------- f32 rows ----
// f32 weights (vec_dot_type F32: the activation rows as they are). A wave takes
// NR rows of each of the NM matrices; lane l holds elements [l SEG, (l + 1) SEG)
// of each row and runs their fma chain from 0 for one verify row after the other,
// then wave_sum_f_n reduces the NM * NR partials of that verify row side by side
// (the xor butterfly 32, 16, .. 1: the f16 order's segments and tree, each step
// of a chain one rounding). The activation rows come from memory (at most
// 16 x 3,072 floats: cache-resident); the next group's weights are in flight
// during the current group's chains.
template <int SEG, int NM, int NR>
struct F32Group {
  v4f w[NM][NR][SEG / 4];
};

template <int SEG, int NM, int NR>
__device__ __forceinline__ void f32_load(const float* const (&base)[NM], int n, int row0, F32Group<SEG, NM, NR>& g) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int row = min(row0 + r, n - 1);  // rows past n: loaded, never stored
#pragma unroll
      for (int p = 0; p < SEG / 4; ++p)
        g.w[m][r][p] = *(const v4f*)(base[m] + (size_t)row * (SEG * 64) + lane * SEG + 4 * p);
    }
}

// acc[m * NR + r] <- the dot of row r of matrix m with verify row t (every lane)
template <int SEG, int NM, int NR>
__device__ __forceinline__ void f32_dots(const F32Group<SEG, NM, NR>& g, const float* __restrict__ x, int t,
                                         float (&acc)[NM * NR]) {
  const int lane = threadIdx.x & 63;
  v4f xv[SEG / 4];
#pragma unroll
  for (int p = 0; p < SEG / 4; ++p) xv[p] = *(const v4f*)(x + (size_t)t * (SEG * 64) + lane * SEG + 4 * p);
#pragma unroll
  for (int i = 0; i < NM * NR; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int p = 0; p < SEG / 4; ++p)
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[m * NR + r] = fmaf(g.w[m][r][p][e], xv[p][e], acc[m * NR + r]);
  wave_sum_f_n<NM * NR>(acc);
}

// EPI 0: store, 1: residual add, 2: silu(W x) * (W2 x) (f32 rows: the down
// projection's activation as it is). Lane r < NR stores row r of the group.
template <int EPI, int SEG, int NR>
__global__ void __launch_bounds__(256)
k_gemm_f32(const StepDesc* __restrict__ desc, const float* __restrict__ w, const float* __restrict__ w2, int n,
           const float* __restrict__ x, float* __restrict__ out) {
  constexpr int NM = EPI == 2 ? 2 : 1;
  const int T = desc->T, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ngroups = (n + NR - 1) / NR, nwaves = gridDim.x * 4;
  const float* base[NM];
  base[0] = w;
  if (NM == 2) base[NM - 1] = w2;
  int g = blockIdx.x * 4 + wave;
  F32Group<SEG, NM, NR> nxt;
  if (g < ngroups) f32_load<SEG, NM, NR>(base, n, g * NR, nxt);
  for (; g < ngroups; g += nwaves) {
    const F32Group<SEG, NM, NR> cur = nxt;
    if (g + nwaves < ngroups) f32_load<SEG, NM, NR>(base, n, (g + nwaves) * NR, nxt);
    const int row = g * NR + lane;
    for (int t = 0; t < T; ++t) {
      float acc[NM * NR];
      f32_dots<SEG, NM, NR>(cur, x, t, acc);
      float v0 = acc[0], v1 = acc[NM * NR - NR];
#pragma unroll
      for (int r = 1; r < NR; ++r)
        if (lane == r) {
          v0 = acc[r];
          v1 = acc[NM * NR - NR + r];
        }
      if (lane < NR && row < n) {
        float* dst = out + (size_t)t * n + row;
        if (EPI == 0) *dst = v0;
        else if (EPI == 1) *dst = __fadd_rn(*dst, v0);
        else *dst = dev_swiglu(v0, v1);
      }
    }
  }
}

// weight rows per wave and group of the f32 GEMM: NM * NR * K / 64 <= 64 weight
// floats per lane (twice that with the next group in flight)
constexpr int f32_nr(int nm, int seg) { return seg == 16 ? 4 / nm : seg == 32 ? (nm == 1 ? 2 : 1) : 1; }

template <int EPI>
void gemm_f32(hipStream_t s, const StepDesc* desc, const uint8_t* w, const uint8_t* w2, int n, int k, const float* x,
              float* out) {
  constexpr int NM = EPI == 2 ? 2 : 1;
  const float* wf = (const float*)w;
  const float* w2f = (const float*)w2;
#define MTG_F32_GEMM(SEG)                                                                                    \
  {                                                                                                          \
    constexpr int NR = f32_nr(NM, SEG);                                                                      \
    const int blocks = std::min(((n + NR - 1) / NR + 3) / 4, 4 * kLmWorkgroups);                             \
    hipLaunchKernelGGL((k_gemm_f32<EPI, SEG, NR>), dim3(blocks), dim3(256), 0, s, desc, wf, w2f, n, x, out); \
  }
  if (k == 1024) MTG_F32_GEMM(16)
  else if (k == 2048) MTG_F32_GEMM(32)
  else MTG_F32_GEMM(48)
#undef MTG_F32_GEMM
}

// weight rows per wave and group of the f16 GEMM (NM * NR * 16 partial rows of LDS per wave)
constexpr int f16_nr(int epi, int seg) { return seg == 16 ? (epi == 2 ? 3 : 4) : 1; }
// at most one workgroup per CU (its LDS admits no second): more groups go to the
// waves' loops, with the next group in flight, instead of a second round of
// workgroups that would stage the activation again
constexpr int kF16GemmWorkgroups = 256;

template <int WT, int EPI>
void gemm_wt(hipStream_t s, const StepDesc* desc, const uint8_t* w, const uint8_t* w2, int n, int k,
             const WtAct& act, float* out) {
  const dim3 grid((n + 3) / 4), block(256);
  if constexpr (WT == MTG_TYPE_F16) {
    constexpr int NM = EPI == 2 ? 2 : 1;
    if (k == 1024) {
      constexpr int NR = f16_nr(EPI, 16);
      const int blocks = std::min(((n + NR - 1) / NR + 3) / 4, kF16GemmWorkgroups);
      hipLaunchKernelGGL((k_gemm_f16<EPI, 16, NR>), dim3(blocks), block, f16_lds_bytes(k, NM * NR), s, desc, w, w2,
                         n, act.f16h, out);
    } else if (k == 2048) {
      constexpr int NR = f16_nr(EPI, 32);
      const int blocks = std::min(((n + NR - 1) / NR + 3) / 4, kF16GemmWorkgroups);
      hipLaunchKernelGGL((k_gemm_f16<EPI, 32, NR>), dim3(blocks), block, f16_lds_bytes(k, NM * NR), s, desc, w, w2,
                         n, act.f16h, out);
    } else {
      constexpr int NR = f16_nr(EPI, 48);
      const int blocks = std::min(((n + NR - 1) / NR + 3) / 4, kF16GemmWorkgroups);
      hipLaunchKernelGGL((k_gemm_f16<EPI, 48, NR>), dim3(blocks), block, f16_lds_bytes(k, NM * NR), s, desc, w, w2,
                         n, act.f16h, out);
    }
  } else if (n % 16 == 0 && (k == 1024 || k == 2048 || k == 3072)) {
    constexpr int NM = EPI == 2 ? 2 : 1;
    if (k == 1024)
      hipLaunchKernelGGL((k_gemm_q4m<EPI, 4>), dim3(n / 16), dim3(64 * q4g_waves(4)), q4g_lds_bytes(4, NM), s, desc,
                         w, w2, n, act.q8k, out);
    else if (k == 2048)
      hipLaunchKernelGGL((k_gemm_q4m<EPI, 8>), dim3(n / 16), dim3(64 * q4g_waves(8)), q4g_lds_bytes(8, NM), s, desc,
                         w, w2, n, act.q8k, out);
    else
      hipLaunchKernelGGL((k_gemm_q4m<EPI, 12>), dim3(n / 16), dim3(64 * q4g_waves(12)), q4g_lds_bytes(12, NM), s,
                         desc, w, w2, n, act.q8k, out);
  } else if (k <= kQ4MaxK) {
    constexpr int NM = EPI == 2 ? 2 : 1;
    const int blocks = std::min((n + 4 * kQ4GemmD - 1) / (4 * kQ4GemmD), kLmWorkgroups);
    hipLaunchKernelGGL((k_gemm_q4k<EPI, kQ4GemmD>), dim3(blocks), block, q4_lds_bytes(k, NM * kQ4GemmD), s, desc,
                       w, w2, n, k, act.q8k, out);
  } else {
    hipLaunchKernelGGL((k_gemm_wt<WT, 0, EPI>), grid, block, 0, s, desc, w, w2, n, k, nullptr, act.q8k, out);
  }
}

// The f16 GEMM of a K = 1024 matrix whose activation is RMSNorm(x) * gain (EPI 0
// or 2): the norm runs in the GEMM's workgroups. q|k|v (EPI 0) runs 8 waves of
// 2 rows per workgroup: two waves per SIMD share the fma issue (a lone wave leaves
// about half of it idle), measured 6.8 -> 6.4 us at T = 8; gate/up keeps 4 waves
// of 3 rows per matrix (its 8-wave form, 1 row per matrix, was slower).
constexpr int f16n_nwv(int epi) { return epi == 2 ? 4 : 8; }
constexpr int f16n_nr(int epi) { return epi == 2 ? f16_nr(2, 16) : 2; }

template <int EPI>
void gemm_f16_norm(hipStream_t s, const StepDesc* desc, const uint8_t* w, const uint8_t* w2, int n, const float* x,
                   const float* gain, float eps, float* out) {
  constexpr int NM = EPI == 2 ? 2 : 1, NR = f16n_nr(EPI), NWV = f16n_nwv(EPI);
  const int blocks = std::min(((n + NR - 1) / NR + NWV - 1) / NWV, kF16GemmWorkgroups);
  hipLaunchKernelGGL((k_gemm_f16<EPI, 16, NR, true, NWV>), dim3(blocks), dim3(64 * NWV),
                     f16_lds_bytes(1024, NM * NR, NWV), s, desc, w, w2, n, nullptr, out, x, gain, eps);
}

}  // namespace

// ================================================================ launches ==
hipError_t prepare_kernels_wt() {
  const void* fns[4] = {(const void*)k_gemm_q4k<0, kQ4GemmD>, (const void*)k_gemm_q4k<1, kQ4GemmD>,
                        (const void*)k_gemm_q4k<2, kQ4GemmD>, (const void*)k_lm_head_q4k};
  const int rows[4] = {kQ4GemmD, kQ4GemmD, 2 * kQ4GemmD, kQ4LmD};
  for (int i = 0; i < 4; ++i) {
    const hipError_t e = hipFuncSetAttribute(fns[i], hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)q4_lds_bytes(kQ4MaxK, rows[i]));
    if (e != hipSuccess) return e;
  }
#define MTG_F16_ATTR(EPI, SEG)                                                                              \
  {                                                                                                          \
    constexpr int NR = f16_nr(EPI, SEG), NM = EPI == 2 ? 2 : 1;                                              \
    const hipError_t e = hipFuncSetAttribute((const void*)k_gemm_f16<EPI, SEG, NR>,                          \
                                             hipFuncAttributeMaxDynamicSharedMemorySize,                     \
                                             (int)f16_lds_bytes(SEG * 64, NM * NR));                         \
    if (e != hipSuccess) return e;                                                                           \
  }
  MTG_F16_ATTR(0, 16) MTG_F16_ATTR(1, 16) MTG_F16_ATTR(2, 16)
  MTG_F16_ATTR(0, 32) MTG_F16_ATTR(1, 32) MTG_F16_ATTR(2, 32)
  MTG_F16_ATTR(0, 48) MTG_F16_ATTR(1, 48) MTG_F16_ATTR(2, 48)
#undef MTG_F16_ATTR
  for (int epi = 0; epi <= 2; epi += 2) {
    const int nm_nr = epi == 2 ? 2 * f16n_nr(2) : f16n_nr(0);
    const hipError_t e = hipFuncSetAttribute(
        epi == 2 ? (const void*)k_gemm_f16<2, 16, f16n_nr(2), true, f16n_nwv(2)>
                 : (const void*)k_gemm_f16<0, 16, f16n_nr(0), true, f16n_nwv(0)>,
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)f16_lds_bytes(1024, nm_nr, epi == 2 ? f16n_nwv(2) : f16n_nwv(0)));
    if (e != hipSuccess) return e;
  }
  for (int f32 = 0; f32 < 2; ++f32) {
    const hipError_t e = hipFuncSetAttribute(f32 ? (const void*)k_lm_head_f16m<true> : (const void*)k_lm_head_f16m<false>,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lm_lds_bytes(f32 != 0));
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

bool wt_shape_supported(int wtype, int k) {
  if (wtype == MTG_TYPE_F16 || wtype == MTG_TYPE_F32) return k == 1024 || k == 2048 || k == 3072;
  if (wtype == MTG_TYPE_Q4_K) return k % 256 == 0;
  return false;
}

void launch_act_wt(hipStream_t s, int wtype, const StepDesc* desc, const float* src, int K,
                   const float* gain, float eps, const WtAct& act, float* normed_out) {
  const dim3 grid(kMaxRows, K / 256);
  if (wtype == MTG_TYPE_F16)
    hipLaunchKernelGGL(k_act_f16<false>, grid, dim3(256), 0, s, desc, src, K, gain, eps, act.f16h, nullptr,
                       normed_out);
  else if (wtype == MTG_TYPE_F32)
    hipLaunchKernelGGL(k_act_f16<true>, grid, dim3(256), 0, s, desc, src, K, gain, eps, nullptr, act.f32,
                       normed_out);
  else
    hipLaunchKernelGGL(k_act_q8k, grid, dim3(256), 0, s, desc, src, K, gain, eps, act.q8k, normed_out);
}

void launch_attn_combine_wt(hipStream_t s, int wtype, const StepDesc* desc, AttnWork work, int n_heads,
                            int max_chunks, const WtAct& act) {
  const dim3 grid(n_heads / 2, kMaxRows), block(256 * kCombSeg);
  if (wtype == MTG_TYPE_F16)
    hipLaunchKernelGGL(k_attn_combine_f16q<false>, dim3(n_heads / 2, kMaxRows, kHeadDim / kCombDq),
                       dim3(64 * kCombSeg), 0, s, desc, work, n_heads, max_chunks, act);
  else if (wtype == MTG_TYPE_F32)
    hipLaunchKernelGGL(k_attn_combine_f16q<true>, dim3(n_heads / 2, kMaxRows, kHeadDim / kCombDq),
                       dim3(64 * kCombSeg), 0, s, desc, work, n_heads, max_chunks, act);
  else
    hipLaunchKernelGGL(k_attn_combine_wt<MTG_TYPE_Q4_K>, grid, block, 0, s, desc, work, n_heads, max_chunks, act);
}

void launch_gemm_f16_norm(hipStream_t s, int epi, const StepDesc* desc, const uint8_t* w, const uint8_t* w2, int n,
                          const float* x, const float* gain, float eps, float* out) {
  if (epi == 2) gemm_f16_norm<2>(s, desc, w, w2, n, x, gain, eps, out);
  else gemm_f16_norm<0>(s, desc, w, w2, n, x, gain, eps, out);
}

void launch_gemm_wt(hipStream_t s, int wtype, int epi, const StepDesc* desc, const uint8_t* w,
                    const uint8_t* w2, int n, int k, const WtAct& act, float* out) {
  if (wtype == MTG_TYPE_F16) {
    if (epi == 0) gemm_wt<MTG_TYPE_F16, 0>(s, desc, w, w2, n, k, act, out);
    else if (epi == 1) gemm_wt<MTG_TYPE_F16, 1>(s, desc, w, w2, n, k, act, out);
    else gemm_wt<MTG_TYPE_F16, 2>(s, desc, w, w2, n, k, act, out);
  } else if (wtype == MTG_TYPE_F32) {
    if (epi == 0) gemm_f32<0>(s, desc, w, w2, n, k, act.f32, out);
    else if (epi == 1) gemm_f32<1>(s, desc, w, w2, n, k, act.f32, out);
    else gemm_f32<2>(s, desc, w, w2, n, k, act.f32, out);
  } else {
    if (epi == 0) gemm_wt<MTG_TYPE_Q4_K, 0>(s, desc, w, w2, n, k, act, out);
    else if (epi == 1) gemm_wt<MTG_TYPE_Q4_K, 1>(s, desc, w, w2, n, k, act, out);
    else gemm_wt<MTG_TYPE_Q4_K, 2>(s, desc, w, w2, n, k, act, out);
  }
}

void launch_lm_head_wt(hipStream_t s, int wtype, const StepDesc* desc, const uint8_t* w, int vocab, int k,
                       const WtAct& act, const uint32_t* bitmap, float* logits, uint64_t* part_keys) {
  const dim3 grid(kLmWorkgroups), block(256);
  if (wtype == MTG_TYPE_F16)  // w: the lm_head copy of the embedding (launch_lm16_retile)
    hipLaunchKernelGGL(k_lm_head_f16m<false>, dim3(kLm16Blocks), dim3(64 * kLm16NWV), lm_lds_bytes(false), s, desc, w,
                       vocab, (const void*)act.f16h, bitmap, logits, part_keys);
  else if (wtype == MTG_TYPE_F32)  // w: the lm_head copy of the embedding (launch_lm16_retile)
    hipLaunchKernelGGL(k_lm_head_f16m<true>, dim3(kLm16Blocks), dim3(64 * kLm16NWV), lm_lds_bytes(true), s, desc, w,
                       vocab, (const void*)act.f32, bitmap, logits, part_keys);
  else if (k == 1024 && vocab % 16 == 0)
    hipLaunchKernelGGL(k_lm_head_q4m<4>, grid, block, q4m_lds_bytes(k), s, desc, w, vocab, act.q8k, bitmap, logits,
                       part_keys);
  else if (k <= kQ4MaxK)
    hipLaunchKernelGGL(k_lm_head_q4k, grid, block, q4_lds_bytes(k, kQ4LmD), s, desc, w, vocab, k, act.q8k, bitmap,
                       logits, part_keys);
  else
    hipLaunchKernelGGL((k_lm_head_wt<MTG_TYPE_Q4_K, 0>), grid, block, 0, s, desc, w, vocab, k, nullptr,
                       act.q8k, bitmap, logits, part_keys);
}

void launch_lm16_retile(hipStream_t s, int wtype, const uint8_t* embd, int vocab, uint8_t* out) {
  const bool f32 = wtype == MTG_TYPE_F32;
  const size_t threads = (size_t)(vocab / 16) * (f32 ? LmTile<true>::kPieces : LmTile<false>::kPieces) * 64;
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (f32)
    hipLaunchKernelGGL(k_lm32_retile, grid, dim3(256), 0, s, (const float*)embd, vocab / 16, (float*)out);
  else
    hipLaunchKernelGGL(k_lm16_retile, grid, dim3(256), 0, s, (const uint16_t*)embd, vocab / 16, (uint16_t*)out);
}

void launch_embed_wt(hipStream_t s, int wtype, const StepDesc* desc, const uint8_t* w, int hidden,
                     const float* host_rows, float* x) {
  if (wtype == MTG_TYPE_F16)
    hipLaunchKernelGGL(k_embed_wt<MTG_TYPE_F16>, dim3(kMaxRows), dim3(256), 0, s, desc, w, hidden, host_rows, x);
  else if (wtype == MTG_TYPE_F32)
    hipLaunchKernelGGL(k_embed_wt<MTG_TYPE_F32>, dim3(kMaxRows), dim3(256), 0, s, desc, w, hidden, host_rows, x);
  else
    hipLaunchKernelGGL(k_embed_wt<MTG_TYPE_Q4_K>, dim3(kMaxRows), dim3(256), 0, s, desc, w, hidden, host_rows, x);
}

}  // namespace mtg
