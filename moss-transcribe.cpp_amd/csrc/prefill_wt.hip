// prefill_wt.hip - the block prefill for f16 and q4_K weights: the prompt rows go
// through the decoder in blocks of up to 2,048 rows with each weight matrix
// streamed once per block (Qwen3Decoder::prefill, src/qwen3_decoder.cpp:162-166),
// as prefill.hip does for q8_0. Per layer:
//   k_pf_act_wt     RMSNorm * gain (or the rows as they are) and the weight type's
//                   vec_dot_type: f16 values, or q8_K blocks (quantize_row_q8_K)
//   k_pf_gemm_f16   f16 weights x f16 activations on f32 MFMA, in the canonical
//                   segment order (below)
//   k_pf_gemm_q4k   q4_K weights x q8_K activations: exact int32 sums per
//                   superblock on int8 MFMA, the float chain over superblocks
// with prefill.hip's q/k norm + RoPE + KV append and causal attention (its f32
// output variant) in between. Outputs equal the oracle's and the verify path's
// bit for bit (the same orders as the per-op kernels of kernels_wt.hip).
#include <type_traits>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "device_common.hpp"

namespace mtg {
namespace {
using namespace dev;

// ---------------------------------------------------------- activations ----
// Grid (S rows, K / 256), 256 threads, one element per thread: the arithmetic of
// k_act_f16 / k_act_q8k for any number of rows. gain == nullptr: no norm.
template <int WT>
__global__ void __launch_bounds__(256)
k_pf_act_wt(const float* __restrict__ src, int S, int K, const float* __restrict__ gain, float eps,
            uint16_t* __restrict__ f16_out, ActQ8K a, float* __restrict__ f32_out) {
  const int t = blockIdx.x, b = blockIdx.y, k = b * 256 + threadIdx.x;
  if (t >= S) return;
  const float* xr = src + (size_t)t * K;
  __shared__ float s_scale;
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
  if constexpr (WT == MTG_TYPE_F16) {
    f16_out[(size_t)t * K + k] = __half_as_ushort(__float2half_rn(y));  // vec_dot_type F16
  } else if constexpr (WT == MTG_TYPE_F32) {
    f32_out[(size_t)t * K + k] = y;  // vec_dot_type F32: the row as it is
  } else {
    q8k_block256(y, a, t, K, b);
  }
}

// The rows of the output tile that this lane holds (the MFMA result layout:
// lane (n, g) = (lane % 16, lane / 16) holds weight rows 4 g + r, r < 4, of the
// wave's 16, for activation row n of the column tile), after the epilogue
// (epi: store, residual add, or the encoder's linear = mul_mat + bias, then GELU,
// SiLU or the residual add; the SwiGLU is applied before this).
// n0: the first of the 4 weight rows in the output's row space.
__device__ __forceinline__ void pf_store4(int epi, float* out, int N, int t, int n0, const float (&v)[4],
                                          const float* bias) {
  float* dst = out + (size_t)t * N + n0;
  float y[4] = {v[0], v[1], v[2], v[3]};
  if (epi >= PF_EPI_BIAS) {
    const v4f b = *(const v4f*)(bias + n0);
#pragma unroll
    for (int q = 0; q < 4; ++q) y[q] = __fadd_rn(y[q], b[q]);
    if (epi == PF_EPI_BIAS_GELU) {
      dev_gelu_erf_n<4>(y);
    } else if (epi == PF_EPI_BIAS_SILU) {
#pragma unroll
      for (int q = 0; q < 4; ++q) y[q] = dev_silu(y[q]);
    }
  }
  v4f o;
  if (epi == PF_EPI_RESID || epi == PF_EPI_BIAS_RESID) {
    const v4f x = *(const v4f*)dst;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = __fadd_rn(x[q], y[q]);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = y[q];
  }
  *(v4f*)dst = o;
}

// ------------------------------------------------------- f16 / f32 GEMM ----
// out[s][n] for 64 weight rows x 64 activation rows per workgroup (wave w: the
// 16-row tile 4 blockIdx.x + w; for the SwiGLU epilogue waves 0, 1 take gate rows
// 32 blockIdx.x + 16 w and waves 2, 3 the same rows of up, meeting in LDS).
// The canonical f16 dot (the oracle's mul_mat_f16, the per-op k_gemm_f16): K in
// 64 consecutive segments of L = K / 64 elements, each an fma chain from 0 over
// its elements in order (a product of two f16 values is exact in f32), the 64
// partials reduced by the xor butterfly (v[i] + v[i ^ 32], then 16, .. 1, lane 0).
// v_mfma_f32_16x16x4f32 returns fma(a3, b3, fma(a2, b2, fma(a1, b1, fma(a0, b0, c))))
// per output, so L / 4 chained MFMAs from a zero accumulator are one segment's
// chain (k-step s: elements 4 s + kk held by lane group kk). The segments run in
// 6-bit bit-reversed order: the butterfly's tree is then the balanced binary tree
// over the run, folded as it goes with a stack of six partials (a binary counter).
// Every segment's weight and activation rows are staged in LDS as f32 (row stride
// L + 4 floats: the operand reads of a wave hit 64 distinct banks), the next
// segment's rows already in flight in registers.
// F32: f32 weights and activations (vec_dot_type F32), the same segments, MFMA
// chains and tree: each step of a segment's chain is one fma of two f32 values,
// as the oracle's mul_mat_f32 and the per-op k_gemm_f32 take it.
__device__ __forceinline__ int bitrev6(int k) { return (int)(__builtin_bitreverse32((uint32_t)k) >> 26); }

template <bool GLU, int L, bool F32 = false>
__global__ void __launch_bounds__(256)
k_pf_gemm_f16(const void* __restrict__ wv, const void* __restrict__ w2v, int N, const void* __restrict__ xv, int S,
              float* __restrict__ out, int epi, const float* __restrict__ bias) {
  using E = typename std::conditional<F32, float, uint16_t>::type;
  constexpr int EP = 16 / (int)sizeof(E);  // elements per 16-byte piece
  constexpr int K = 64 * L, LS = L + 4, NP = L / EP;  // pieces per row and segment
  constexpr int NPIECE = 2 * 64 * NP, PPT = (NPIECE + 255) / 256;
  const E* w = (const E*)wv;
  const E* w2 = (const E*)w2v;
  const E* x = (const E*)xv;
  __shared__ __align__(16) float s_w[2][64 * LS];
  __shared__ __align__(16) float s_x[2][64 * LS];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, m = lane & 15, kk = lane >> 4;
  const int s0 = blockIdx.y * 64;
  // weight row r (< 64) of the workgroup
  auto wrow = [&](int r) -> const E* {
    if constexpr (GLU) return (r < 32 ? w : w2) + (size_t)(32 * blockIdx.x + (r & 31)) * K;
    return w + (size_t)(64 * blockIdx.x + r) * K;
  };
  uint4 reg[PPT];
  auto fetch = [&](int seg) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + 256 * i;
      if (p < NPIECE) {
        const int half = p / (64 * NP), q = p % (64 * NP), r = q / NP, j = q % NP;
        if (half == 0)
          reg[i] = *(const uint4*)(wrow(r) + seg * L + EP * j);
        else
          reg[i] = s0 + r < S ? *(const uint4*)(x + (size_t)(s0 + r) * K + seg * L + EP * j) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + 256 * i;
      if (p < NPIECE) {
        const int half = p / (64 * NP), q = p % (64 * NP), r = q / NP, j = q % NP;
        float* dst = (half ? s_x[buf] : s_w[buf]) + r * LS + EP * j;
        const uint32_t u[4] = {reg[i].x, reg[i].y, reg[i].z, reg[i].w};
        if constexpr (F32) {
          *(v4f*)dst = v4f{__uint_as_float(u[0]), __uint_as_float(u[1]), __uint_as_float(u[2]), __uint_as_float(u[3])};
          continue;
        }
        v4f lo, hi;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          lo[2 * e] = half_bits_to_float((uint16_t)(u[e] & 0xffffu));
          lo[2 * e + 1] = half_bits_to_float((uint16_t)(u[e] >> 16));
          hi[2 * e] = half_bits_to_float((uint16_t)(u[2 + e] & 0xffffu));
          hi[2 * e + 1] = half_bits_to_float((uint16_t)(u[2 + e] >> 16));
        }
        *(v4f*)dst = lo;
        *(v4f*)(dst + 4) = hi;
      }
    }
  };
  v4f stk[6][4], res[4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    res[ct] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int lvl = 0; lvl < 6; ++lvl) stk[lvl][ct] = res[ct];
  }
  fetch(bitrev6(0));
  stage(0);
  for (int k = 0; k < 64; ++k) {
    const int buf = k & 1;
    if (k + 1 < 64) fetch(bitrev6(k + 1));
    __syncthreads();  // segment k is staged; the other buffer's readers (segment k - 1) are done
    const float* aw = s_w[buf] + (16 * wave + m) * LS + kk;
    v4f cur[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) cur[ct] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < L / 4; ++s) {
      const float av = aw[4 * s];
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        cur[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, s_x[buf][(16 * ct + m) * LS + 4 * s + kk], cur[ct], 0, 0, 0);
    }
    // fold leaf k into the stack: while bit lvl of k is set, the left sibling
    // (the earlier subtree) is added; the first clear bit keeps the partial
    bool carry = true;
#pragma unroll
    for (int lvl = 0; lvl < 6; ++lvl) {
      if (carry) {
        if ((k >> lvl) & 1) {
#pragma unroll
          for (int ct = 0; ct < 4; ++ct)
#pragma unroll
            for (int q = 0; q < 4; ++q) cur[ct][q] = __fadd_rn(stk[lvl][ct][q], cur[ct][q]);
        } else {
#pragma unroll
          for (int ct = 0; ct < 4; ++ct) stk[lvl][ct] = cur[ct];
          carry = false;
        }
      }
    }
    if (carry) {  // k == 63: the root
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) res[ct] = cur[ct];
    }
    if (k + 1 < 64) stage(buf ^ 1);
  }
  const int g = kk, n = m;
  if constexpr (GLU) {
    // the up waves hand their values to the gate waves of the same rows
    __syncthreads();
    float* s_up = &s_w[0][0];  // [2 tiles][4 ct][64 lanes][4]: 2,048 of the 2 x 64 x LS floats
    if (wave >= 2)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) *(v4f*)(s_up + (((wave & 1) * 4 + ct) * 64 + lane) * 4) = res[ct];
    __syncthreads();
    if (wave >= 2) return;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int t = s0 + 16 * ct + n;
      if (t >= S) continue;
      const v4f u = *(const v4f*)(s_up + (((wave & 1) * 4 + ct) * 64 + lane) * 4);
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = dev_swiglu(res[ct][q], u[q]);
      pf_store4(PF_EPI_STORE, out, N, t, 32 * blockIdx.x + 16 * (wave & 1) + 4 * g, v, nullptr);
    }
  } else {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int t = s0 + 16 * ct + n;
      if (t >= S) continue;
      const float v[4] = {res[ct][0], res[ct][1], res[ct][2], res[ct][3]};
      pf_store4(epi, out, N, t, 64 * blockIdx.x + 16 * wave + 4 * g, v, bias);
    }
  }
}

// ------------------------------------------------------------ q4_K GEMM ----
// 64 weight rows x 64 activation rows per workgroup (the same wave roles as
// k_pf_gemm_f16). Per superblock of 256: the activation codes and scales of the
// 64 rows are staged in LDS (row stride 288 bytes: a wave's 8-byte operand reads
// take the minimum two passes), the next superblock's in flight in registers with
// the wave's weight bytes. For each 16 x 16 output tile the exact int32 sums
// dot = sum_j sc_j * sub_j (the 6-bit scale split as 8 * (sc >> 3) + (sc & 7): two
// int8 MFMA accumulators of nibble * factor <= 105) and mins = sum_j mn_j * sum(x_j)
// come from v_mfma_i32_16x16x32_i8 (the per-op k_gemm_q4m's sums), then the
// oracle's chain over superblocks in order: acc = (acc + (d_w d_x) dot) -
// (dmin_w d_x) mins.
constexpr int kQ4RowStride = 288;

template <bool GLU>
__global__ void __launch_bounds__(256)
k_pf_gemm_q4k(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2, int N, int K, ActQ8K a, int S,
              float* __restrict__ out, int epi, const float* __restrict__ bias) {
  __shared__ __align__(16) int8_t s_q[2][64 * kQ4RowStride];
  __shared__ float s_dx[2][64];
  __shared__ float s_dw[4][16 * 2];  // per wave: d, dmin of its 16 weight rows
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, row = lane & 15, g = lane >> 4;
  const int NB = K / 256, s0 = blockIdx.y * 64;
  const uint8_t* wr = GLU ? (wave < 2 ? w : w2) + (size_t)(32 * blockIdx.x + 16 * (wave & 1) + row) * NB * 144
                          : w + (size_t)(64 * blockIdx.x + 16 * wave + row) * NB * 144;
  // staging: thread tid takes 16-byte pieces tid + 256 i (i < 4) of the 64 x 256
  // code block (row p / 16, bytes 16 (p % 16) ..); threads < 64 a row's scale
  uint4 nq[4];
  float ndx = 0.0f;
  uint2 nw[4];
  v4i nh;
  auto fetch = [&](int b) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + 256 * i, r = p >> 4, c = p & 15;
      nq[i] = s0 + r < S ? *(const uint4*)(a.qs + (size_t)(s0 + r) * K + b * 256 + 16 * c) : make_uint4(0, 0, 0, 0);
    }
    if (tid < 64) ndx = s0 + tid < S ? a.d[(size_t)(s0 + tid) * NB + b] : 0.0f;
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) nw[mm] = *(const uint2*)(wr + b * 144 + 16 + 32 * mm + 8 * g);
    nh = *(const v4i*)(wr + b * 144);
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = tid + 256 * i, r = p >> 4, c = p & 15;
      *(uint4*)(s_q[buf] + r * kQ4RowStride + 16 * c) = nq[i];
    }
    if (tid < 64) s_dx[buf][tid] = ndx;
  };
  float res[4][4];
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) res[ct][r] = 0.0f;
  fetch(0);
  stage(0);
  for (int b = 0; b < NB; ++b) {
    const int buf = b & 1;
    const uint2 qw[4] = {nw[0], nw[1], nw[2], nw[3]};
    const v4i h = nh;
    if (b + 1 < NB) fetch(b + 1);
    __syncthreads();  // superblock b is staged; the other buffer's readers are done
    int sc[8], mn[8];
    q4k_scales_w((uint32_t)h[1], (uint32_t)h[2], (uint32_t)h[3], sc, mn);
    // d, dmin of the wave's rows through its LDS slot (lanes 0..15 own them; LDS
    // accesses of a wave execute in order)
    if (g == 0) {
      s_dw[wave][row * 2] = half_bits_to_float((uint16_t)((uint32_t)h[0] & 0xffffu));
      s_dw[wave][row * 2 + 1] = half_bits_to_float((uint16_t)((uint32_t)h[0] >> 16));
    }
    float dw[4], dmw[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      dw[r] = s_dw[wave][(4 * g + r) * 2];
      dmw[r] = s_dw[wave][(4 * g + r) * 2 + 1];
    }
    // the A operands of the 8 sub-blocks: nibbles x (sc >> 3), x (sc & 7), and mn
    long ah[8], al[8], am[8];
#pragma unroll
    for (int mm = 0; mm < 4; ++mm)
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int s = 2 * mm + hi;
        const uint32_t q0 = hi ? (qw[mm].x >> 4) & 0x0F0F0F0Fu : qw[mm].x & 0x0F0F0F0Fu;
        const uint32_t q1 = hi ? (qw[mm].y >> 4) & 0x0F0F0F0Fu : qw[mm].y & 0x0F0F0F0Fu;
        const uint32_t fh = (uint32_t)(sc[s] >> 3), fl = (uint32_t)(sc[s] & 7), fm = (uint32_t)mn[s] * 0x01010101u;
        ah[s] = (long)(((uint64_t)(q1 * fh) << 32) | (q0 * fh));
        al[s] = (long)(((uint64_t)(q1 * fl) << 32) | (q0 * fl));
        am[s] = (long)(((uint64_t)fm << 32) | fm);
      }
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      v4i ahi = {0, 0, 0, 0}, alo = {0, 0, 0, 0}, amn = {0, 0, 0, 0};
      const int8_t* xb = s_q[buf] + (16 * ct + row) * kQ4RowStride + 8 * g;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const long bv = *(const long*)(xb + 32 * s);
        ahi = __builtin_amdgcn_mfma_i32_16x16x32_i8(ah[s], bv, ahi, 0, 0, 0);
        alo = __builtin_amdgcn_mfma_i32_16x16x32_i8(al[s], bv, alo, 0, 0, 0);
        amn = __builtin_amdgcn_mfma_i32_16x16x32_i8(am[s], bv, amn, 0, 0, 0);
      }
      const float dx = s_dx[buf][16 * ct + row];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int dot = 8 * ahi[r] + alo[r];
        const float dm = __fmul_rn(dw[r], dx), dmin = __fmul_rn(dmw[r], dx);
        res[ct][r] = __fadd_rn(res[ct][r], __fmul_rn(dm, (float)dot));
        res[ct][r] = __fsub_rn(res[ct][r], __fmul_rn(dmin, (float)amn[r]));
      }
    }
    if (b + 1 < NB) stage(buf ^ 1);
  }
  if constexpr (GLU) {
    __syncthreads();
    float* s_up = (float*)s_q[0];  // [2 tiles][4 ct][64 lanes][4]
    if (wave >= 2)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        *(v4f*)(s_up + (((wave & 1) * 4 + ct) * 64 + lane) * 4) = v4f{res[ct][0], res[ct][1], res[ct][2], res[ct][3]};
    __syncthreads();
    if (wave >= 2) return;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int t = s0 + 16 * ct + row;
      if (t >= S) continue;
      const v4f u = *(const v4f*)(s_up + (((wave & 1) * 4 + ct) * 64 + lane) * 4);
      float v[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = dev_swiglu(res[ct][q], u[q]);
      pf_store4(PF_EPI_STORE, out, N, t, 32 * blockIdx.x + 16 * (wave & 1) + 4 * g, v, nullptr);
    }
  } else {
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int t = s0 + 16 * ct + row;
      if (t >= S) continue;
      pf_store4(epi, out, N, t, 64 * blockIdx.x + 16 * wave + 4 * g, res[ct], bias);
    }
  }
}

}  // namespace

// ================================================================ launches ==
void launch_pf_act_wt(hipStream_t s, int wtype, const float* src, int S, int K, const float* gain, float eps,
                      const WtAct& act) {
  const dim3 grid((unsigned)S, (unsigned)(K / 256));
  if (wtype == MTG_TYPE_F16)
    hipLaunchKernelGGL(k_pf_act_wt<MTG_TYPE_F16>, grid, dim3(256), 0, s, src, S, K, gain, eps, act.f16h, act.q8k,
                       act.f32);
  else if (wtype == MTG_TYPE_F32)
    hipLaunchKernelGGL(k_pf_act_wt<MTG_TYPE_F32>, grid, dim3(256), 0, s, src, S, K, gain, eps, act.f16h, act.q8k,
                       act.f32);
  else
    hipLaunchKernelGGL(k_pf_act_wt<MTG_TYPE_Q4_K>, grid, dim3(256), 0, s, src, S, K, gain, eps, act.f16h, act.q8k,
                       act.f32);
}

void launch_pf_gemm_wt(hipStream_t s, int wtype, int epi, const uint8_t* w, const uint8_t* w2, int N, int K,
                       const WtAct& act, int S, float* out, const float* bias) {
  const bool glu = epi == PF_EPI_SWIGLU;
  const dim3 grid((unsigned)(glu ? N / 32 : N / 64), (unsigned)((S + 63) / 64));
  if (wtype == MTG_TYPE_Q4_K) {
    if (glu)
      hipLaunchKernelGGL(k_pf_gemm_q4k<true>, grid, dim3(256), 0, s, w, w2, N, K, act.q8k, S, out, epi, bias);
    else
      hipLaunchKernelGGL(k_pf_gemm_q4k<false>, grid, dim3(256), 0, s, w, w2, N, K, act.q8k, S, out, epi, bias);
    return;
  }
  const bool f32 = wtype == MTG_TYPE_F32;
  const void* xa = f32 ? (const void*)act.f32 : (const void*)act.f16h;
#define MTG_PF_F16(G, L)                                                                                       \
  if (f32)                                                                                                     \
    hipLaunchKernelGGL((k_pf_gemm_f16<G, L, true>), grid, dim3(256), 0, s, w, w2, N, xa, S, out, epi, bias); \
  else                                                                                                         \
    hipLaunchKernelGGL((k_pf_gemm_f16<G, L, false>), grid, dim3(256), 0, s, w, w2, N, xa, S, out, epi, bias)
#define MTG_PF_F16_K(G)                        \
  switch (K) {                                 \
    case 1024: MTG_PF_F16(G, 16); break;       \
    case 2048: MTG_PF_F16(G, 32); break;       \
    case 3072: MTG_PF_F16(G, 48); break;       \
    default: MTG_PF_F16(G, 64); break;         \
  }
  if (glu) { MTG_PF_F16_K(true); }
  else { MTG_PF_F16_K(false); }
#undef MTG_PF_F16_K
#undef MTG_PF_F16
}

int pf_gemm_wt_supported(int wtype, int K) {
  if (wtype == MTG_TYPE_Q4_K) return K % 256 == 0;
  return K == 1024 || K == 2048 || K == 3072 || K == 4096;
}

}  // namespace mtg
