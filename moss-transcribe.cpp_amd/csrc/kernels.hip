// kernels.hip - gfx950 kernels of the speculative verify step.
//
// Reference ops replaced (moss-transcribe.cpp, via ggml's CPU backend):
//   k_embed            get_rows / embed_rows_f32             src/generate.cpp:68-111
//   k_norm_quant       rms_norm * gain, then the q8_0 activation conversion of
//                      mul_mat (vec_dot_type Q8_0)            src/qwen3.cpp:27-30,80,196
//   k_gemm_*           mul_mat(q8_0 W, f32 x) (+ add / silu*mul)
//                                                             src/qwen3.cpp:92-97,192-193,204-216
//   k_qk_rope_append   q/k rms_norm, rope_ext NEOX, cpy into the cache views
//                                                             src/qwen3.cpp:105-139
//   k_attn_split/combine  scores (F32), soft_max_ext(mask, 1/sqrt(hd)),
//                      causal context at the valid length    src/qwen3.cpp:172-189,
//                                                             src/cpu_context.cpp:13-32
//   k_lm_head + k_accept  tied lm_head, cpu_greedy_choice, the accept loop
//                                                             src/qwen3_decoder.cpp:174-205,
//                                                             src/cpu_speculative.cpp:39-50,124-130
#include <hip/hip_fp16.h>
#include <algorithm>

#include <hip/hip_runtime.h>

#include "device_common.hpp"

namespace mtg {

namespace {
using namespace dev;

// ------------------------------------------------------------- embed -------
__global__ void k_embed(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ tiles,
                        int hidden, const float* __restrict__ host_rows, float* __restrict__ x) {
  const int t = blockIdx.x;
  if (t >= desc->T) return;
  float* xr = x + (size_t)t * hidden;
  if (desc->use_embeds) {
    for (int k = threadIdx.x; k < hidden; k += blockDim.x) xr[k] = host_rows[(size_t)t * hidden + k];
    return;
  }
  const int n = desc->tokens[t];
  const int bps = hidden / kPairK, tile = n >> 4, r = n & 15;
  for (int k = threadIdx.x; k < hidden; k += blockDim.x) {
    const int b = k >> 5, bp = b >> 1, par = b & 1, half = (k >> 4) & 1;
    const uint8_t* unit = tiles + ((size_t)tile * bps + bp) * kUnitBytes;
    const int lane = r + 16 * (2 * par + half);
    const int8_t q = (int8_t)unit[lane * 16 + (k & 15)];
    const float d = half_bits_to_float(((const uint16_t*)(unit + 1024))[par * 16 + r]);
    xr[k] = d * (float)q;  // dequantize_row_q8_0
  }
}

// --------------------------------------------------------- norm+quant -------
// One workgroup per verify row; 256 threads, 8 lanes per 32-block.
__global__ void k_norm_quant(const StepDesc* __restrict__ desc, const float* __restrict__ src,
                             int K, const float* __restrict__ gain, float eps, Panel panel,
                             float* __restrict__ normed_out) {
  const int t = blockIdx.x;
  if (t >= desc->T) return;
  const float* xr = src + (size_t)t * K;
  const int tid = threadIdx.x;
  __shared__ float s_scale;
  float scale = 1.0f;
  if (gain) {
    // canonical row sum (K == 1024): lane l sums elements 16l..16l+15, butterfly
    if (tid < 64) {
      double s = 0.0;
      for (int e = 0; e < 16; ++e) {
        const float v = xr[tid * 16 + e];
        s += (double)__fmul_rn(v, v);
      }
      s = wave_sum_d(s);
      if (tid == 0) {
        const float mean = (float)(s / (double)K);
        s_scale = dev_rms_scale(mean, eps);
      }
    }
    __syncthreads();
    scale = s_scale;
  }
  const int bps = K / kPairK;
  for (int base = 0; base < K; base += 1024) {
    const int k0 = base + tid * 4;  // K is a multiple of 1024 or of 256 below
    if (k0 >= K) break;             // whole 8-lane groups leave together (K % 32 == 0)
    float v[4];
    for (int e = 0; e < 4; ++e) {
      float y = xr[k0 + e];
      if (gain) y = __fmul_rn(__fmul_rn(y, scale), gain[k0 + e]);
      v[e] = y;
    }
    if (normed_out)
      for (int e = 0; e < 4; ++e) normed_out[(size_t)t * K + k0 + e] = v[e];
    int8_t q[4];
    const float d = quant_block8(v, q);
    panel_store4(panel, bps, t, k0, q);
    if ((tid & 7) == 0) panel_store_scale(panel, bps, t, k0 >> 5, d);
  }
}

// Split-K GEMM over one tile per workgroup: SPLIT waves each take a slice of
// the block pairs; partial sums meet in LDS in wave order (deterministic).
// EPI 0: store, 1: residual add, 2: swiglu (second matrix in w2).
template <int EPI, int SPLIT, int G>
__global__ void __launch_bounds__(SPLIT * 64)
k_gemm(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w,
       const uint8_t* __restrict__ w2, int n, int bps, Panel x, float* __restrict__ out) {
  const int T = desc->T;
  if ((T + 7) / 8 != G) return;  // launched once per supported group count
  const int tile = blockIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int bp0 = (bps * wave) / SPLIT, bp1 = (bps * (wave + 1)) / SPLIT;
  constexpr int NM = EPI == 2 ? 2 : 1;
  float acc[NM][G][4];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int cg = 0; cg < G; ++cg)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[m][cg][r] = 0.0f;
  tile_accumulate<G>(w + (size_t)tile * bps * kUnitBytes, bp0, bp1, x.codes, x.scales, bps, acc[0]);
  if (EPI == 2)
    tile_accumulate<G>(w2 + (size_t)tile * bps * kUnitBytes, bp0, bp1, x.codes, x.scales, bps,
                       acc[NM - 1]);
  __shared__ float red[SPLIT > 1 ? SPLIT : 1][NM * G * 4][64];
  if (SPLIT > 1) {
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int cg = 0; cg < G; ++cg)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][(m * G + cg) * 4 + r][lane] = acc[m][cg][r];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int cg = 0; cg < G; ++cg)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float s = red[0][(m * G + cg) * 4 + r][lane];
          for (int wv = 1; wv < SPLIT; ++wv) s = __fadd_rn(s, red[wv][(m * G + cg) * 4 + r][lane]);
          acc[m][cg][r] = s;
        }
  }
  // even + odd block halves of the same (row, t)
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int cg = 0; cg < G; ++cg)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[m][cg][r] = __fadd_rn(acc[m][cg][r], dpp_f<kDppRor8>(acc[m][cg][r]));
  if ((lane & 15) >= 8) return;
#pragma unroll
  for (int cg = 0; cg < G; ++cg) {
    const int t = cg * 8 + (lane & 7);
    if (t >= T) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = tile * 16 + 4 * (lane >> 4) + r;
      float* dst = out + (size_t)t * n + row;
      if (EPI == 0) {
        *dst = acc[0][cg][r];
      } else if (EPI == 1) {
        *dst = __fadd_rn(*dst, acc[0][cg][r]);
      } else {
        *dst = dev_swiglu(acc[0][cg][r], acc[NM - 1][cg][r]);
      }
    }
  }
}

// ------------------------------------------------- q/k norm, rope, append ---
// grid (16 rows, n_heads + 2*n_kv_heads units), one wave per unit; lane i owns
// the NEOX pair (i, i + 64) of head_dim 128.
__global__ void __launch_bounds__(64)
k_qk_rope_append(const StepDesc* __restrict__ desc, const float* __restrict__ qkv, int n_heads,
                 int n_kv_heads, const float* __restrict__ q_norm,
                 const float* __restrict__ k_norm, float eps, const float* __restrict__ rope,
                 float* __restrict__ q_out, KvLayer kv) {
  const int t = blockIdx.x;
  if (t >= desc->T) return;
  const int u = blockIdx.y, i = threadIdx.x;
  const int QN = n_heads * kHeadDim, KN = n_kv_heads * kHeadDim, N = QN + 2 * KN;
  const int pos = desc->past + t;
  const float* row = qkv + (size_t)t * N;
  float x0, x1;
  const bool is_q = u < n_heads, is_k = !is_q && u < n_heads + n_kv_heads;
  const int col = is_q ? u * kHeadDim : is_k ? QN + (u - n_heads) * kHeadDim
                                             : QN + KN + (u - n_heads - n_kv_heads) * kHeadDim;
  x0 = row[col + i];
  x1 = row[col + i + 64];
  if (is_q || is_k) {
    const float* g = is_q ? q_norm : k_norm;
    double s = (double)__fmul_rn(x0, x0) + (double)__fmul_rn(x1, x1);
    s = wave_sum_d(s);
    const float mean = (float)(s / (double)kHeadDim);
    const float scale = dev_rms_scale(mean, eps);
    const float y0 = __fmul_rn(__fmul_rn(x0, scale), g[i]);
    const float y1 = __fmul_rn(__fmul_rn(x1, scale), g[i + 64]);
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

// -------------------------------------------------------------- attention --
// One workgroup per (kv head g, chunk of 64 keys); query columns col = hl*T + t
// for q heads 2g + hl. Canonical chunk arithmetic (device_common.hpp) on
// v_mfma_f32_16x16x4f32, whose 4-term dot is a sequential fma chain: scores are a
// chain of 32 MFMAs over head_dim, P.V a chain of 16 over the chunk's keys.
// The chunk's K and V come to LDS with 16-byte loads (as f32, zeros past kvlen);
// q and K rows are kept permuted (element 4 s + kk at kk * 32 + s) and the
// probabilities too (key 4 s + kk at kk * 16 + s), so that every MFMA operand of
// a lane is one run of consecutive floats.
constexpr int kAqStride = 132, kApStride = 68;
constexpr size_t kAttnLds = (size_t)(kMaxCols * kAqStride + 2 * kChunk * kAqStride + kMaxCols * kApStride) * 4;

__device__ __forceinline__ int attn_perm128(int d) { return (d & 3) * 32 + (d >> 2); }

__global__ void __launch_bounds__(256)
k_attn_chunk(const StepDesc* __restrict__ desc, const float* __restrict__ q, int n_heads,
             KvLayer kv, AttnWork work, int max_chunks) {
  const int g = blockIdx.x, chunk = blockIdx.y;
  const int T = desc->T, past = desc->past, kvlen = past + T;
  const int key0 = chunk * kChunk;
  if (key0 >= kvlen) return;
  extern __shared__ v4f attn_lds_v4[];
  float* s_q = (float*)attn_lds_v4;                 // [32][132] permuted
  float* s_k = s_q + kMaxCols * kAqStride;          // [64][132] permuted
  float* s_v = s_k + kChunk * kAqStride;            // [64][132]
  float* s_p = s_v + kChunk * kAqStride;            // [32][68] permuted
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, kl = lane & 15, kk = lane >> 4;
  const int ncol = 2 * T;
  const bool f16kv = kv.f16 != 0;
  // 1. q rows (f16-rounded for an f16 cache: mul_mat(f16 K, f32 q) converts q),
  //    and the chunk's K / V rows, 4 consecutive elements per thread and pass
  for (int idx = tid; idx < ncol * (kHeadDim / 4); idx += 256) {
    const int col = idx / (kHeadDim / 4), d = (idx % (kHeadDim / 4)) * 4, hl = col / T, t = col % T;
    const v4f v = *(const v4f*)(q + ((size_t)t * n_heads + 2 * g + hl) * kHeadDim + d);
#pragma unroll
    for (int e = 0; e < 4; ++e) s_q[col * kAqStride + attn_perm128(d + e)] = f16kv ? f16_round(v[e]) : v[e];
  }
  const size_t head = (size_t)g * kv.max_seq * kHeadDim;
#pragma unroll
  for (int i = 0; i < kChunk * kHeadDim / 4 / 256; ++i) {
    const int idx = i * 256 + tid, j = idx / (kHeadDim / 4), d = (idx % (kHeadDim / 4)) * 4;
    const int key = key0 + j;
    const bool in = key < kvlen;
    const v4f kf = in ? kv_load4(kv.k, kv.f16, head + (size_t)key * kHeadDim + d) : (v4f){0.f, 0.f, 0.f, 0.f};
    const v4f vf = in ? kv_load4(kv.v, kv.f16, head + (size_t)key * kHeadDim + d) : (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < 4; ++e) s_k[j * kAqStride + attn_perm128(d + e)] = kf[e];
    *(v4f*)(s_v + j * kAqStride + d) = vf;
  }
  __syncthreads();
  // 2. scores of keys 16 wave + kl (A operand) for 16 columns per tile (B)
  const float scale = __fdiv_rn(1.0f, dev_sqrtf((float)kHeadDim));
  for (int ct = 0; ct * 16 < ncol; ++ct) {
    const int colb = ct * 16 + kl;
    const float* krow = s_k + (16 * wave + kl) * kAqStride + kk * 32;
    const float* qrow = s_q + min(colb, ncol - 1) * kAqStride + kk * 32;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const v4f k4 = *(const v4f*)(krow + 4 * i);
      const v4f q4 = *(const v4f*)(qrow + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[j], colb < ncol ? q4[j] : 0.0f, acc, 0, 0, 0);
    }
    if (colb < ncol) {
      const int t = colb % T;
#pragma unroll
      for (int r = 0; r < 4; ++r) {  // key 16 wave + 4 kk + r sits at r * 16 + 4 wave + kk
        const int key = key0 + 16 * wave + 4 * kk + r;
        s_p[colb * kApStride + r * 16 + 4 * wave + kk] =
            (key < kvlen && key <= past + t) ? __fmul_rn(acc[r], scale) : -INFINITY;
      }
    }
  }
  __syncthreads();
  // 3. chunk softmax per column (one wave per column, lane = key)
  const size_t item = (size_t)g * max_chunks + chunk;
  float* out_ml = work.part_ml + item * kMaxCols * 2;
  float* out_o = work.part_o + item * kMaxCols * kHeadDim;
  const int sp_pos = (lane & 3) * 16 + (lane >> 2);
  for (int col = wave; col < ncol; col += 4) {
    const float w = s_p[col * kApStride + sp_pos];
    const float m = wave_max_f(w);
    float p = (m == -INFINITY || w == -INFINITY) ? 0.0f : dev_expf(__fsub_rn(w, m));
    if (f16kv) p = f16_round(p);
    const float l = wave_sum_f(p);
    s_p[col * kApStride + sp_pos] = p;
    if (lane == 0) {
      out_ml[col * 2] = m;
      out_ml[col * 2 + 1] = l;
    }
  }
  __syncthreads();
  // 4. O[col][d] = fma chain over the chunk's keys of p * v: wave w takes head_dim
  //    tiles 2w, 2w + 1
  for (int ct = 0; ct * 16 < ncol; ++ct) {
    const int cola = ct * 16 + kl;
    float pa[16];
    const float* prow = s_p + min(cola, ncol - 1) * kApStride + kk * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v4f p4 = *(const v4f*)(prow + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) pa[4 * i + j] = cola < ncol ? p4[j] : 0.0f;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int d = 16 * (2 * wave + h) + kl;
      v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s2 = 0; s2 < 16; ++s2)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[s2], s_v[(4 * s2 + kk) * kAqStride + d], acc, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int col = ct * 16 + 4 * kk + r;
        if (col < ncol) out_o[col * kHeadDim + d] = acc[r];
      }
    }
  }
}

// ------------------------------------------------ attention, f16 cache ----
// The same chunk arithmetic for an f16 cache, laid out for three workgroups per CU
// and back-to-back MFMA chains. A workgroup keeps its q columns in registers and
// walks the chunks blockIdx.y, blockIdx.y + gridDim.y, ..., the next chunk's K / V
// rows in flight in registers while the current one computes. K / V sit in LDS
// as f16: K rows permuted as above (element 4 i + kk at kk * 32 + i), V rows 65
// words apart. In P.V lane (kl, kk) owns head_dim elements 8 kl + 2 wave + {0, 1},
// read as one 32-bit word per MFMA pair; the 4 lanes kk of a key group and the
// 16 lanes kl then hit 64 different banks.
constexpr int kAkStrideH = 136;  // halves per permuted K row
constexpr int kAvStrideW = 65;   // 32-bit words per V row
constexpr size_t kAttnF16Lds =
    (size_t)kMaxCols * kAqStride * 4 + (size_t)kChunk * kAkStrideH * 2 + (size_t)kChunk * kAvStrideW * 4;
constexpr int kAttnF16Waves = 3 * 256;  // resident workgroups targeted by the grid (3 per CU)

__device__ __forceinline__ float h_lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)w); }
__device__ __forceinline__ float h_hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// K / V rows of the chunk at key0: thread piece p = i * 256 + tid is key p / 16,
// halves 8 (p % 16) .. + 7; zeros past kvlen.
__device__ __forceinline__ void attn_f16_load(const uint16_t* kb, const uint16_t* vb, int key0, int kvlen,
                                              v4i (&pk)[4], v4i (&pv)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = i * 256 + (int)threadIdx.x, key = key0 + (p >> 4), d8 = (p & 15) * 8;
    if (key < kvlen) {
      // streamed once per step: kept out of the caches, which then still hold the
      // chunk partials when the merge (same XCD: kv head g) reads them
      pk[i] = __builtin_nontemporal_load((const v4i*)(kb + (size_t)key * kHeadDim + d8));
      pv[i] = __builtin_nontemporal_load((const v4i*)(vb + (size_t)key * kHeadDim + d8));
    } else {
      pk[i] = (v4i){0, 0, 0, 0};
      pv[i] = (v4i){0, 0, 0, 0};
    }
  }
}

template <int NCT>
__device__ __forceinline__ void attn_f16_scores(const uint16_t* s_k, const float (&qreg)[2][32], float* s_p,
                                                int key0, int kvlen, int past, int T, int ncol, float scale) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kl = lane & 15, kk = lane >> 4;
  const uint16_t* krow = s_k + (16 * wave + kl) * kAkStrideH + kk * 32;
  v4f acc[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) acc[ct] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const v4i kw = *(const v4i*)(krow + 8 * m);
#pragma unroll
    for (int h = 0; h < 8; ++h) {  // head_dim elements 4 (8 m + h) + kk, in order
      const uint32_t word = (uint32_t)kw[h >> 1];
      const float kv = (h & 1) ? h_hi(word) : h_lo(word);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv, qreg[ct][8 * m + h], acc[ct], 0, 0, 0);
    }
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int colb = ct * 16 + kl;
    if (colb < ncol) {
      const int t = colb % T;
#pragma unroll
      for (int r = 0; r < 4; ++r) {  // key 16 wave + 4 kk + r sits at r * 16 + 4 wave + kk
        const int key = key0 + 16 * wave + 4 * kk + r;
        s_p[colb * kApStride + r * 16 + 4 * wave + kk] =
            (key < kvlen && key <= past + t) ? __fmul_rn(acc[ct][r], scale) : -INFINITY;
      }
    }
  }
}

template <int NCT>
__device__ __forceinline__ void attn_f16_pv(const uint32_t* s_v, const float* s_p, int ncol, float* out_o) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, kl = lane & 15, kk = lane >> 4;
  float pa[NCT][16];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int cola = ct * 16 + kl;
    const float* prow = s_p + min(cola, ncol - 1) * kApStride + kk * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v4f p4 = *(const v4f*)(prow + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) pa[ct][4 * i + j] = cola < ncol ? p4[j] : 0.0f;
    }
  }
  v4f acc[NCT][2];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) acc[ct][0] = acc[ct][1] = (v4f){0.f, 0.f, 0.f, 0.f};
  const uint32_t* vcol = s_v + kk * kAvStrideW + 4 * kl + wave;
#pragma unroll
  for (int s2 = 0; s2 < 16; ++s2) {  // keys 4 s2 + kk, in order
    const uint32_t word = vcol[4 * s2 * kAvStrideW];
    const float v0 = h_lo(word), v1 = h_hi(word);
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      acc[ct][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[ct][s2], v0, acc[ct][0], 0, 0, 0);
      acc[ct][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[ct][s2], v1, acc[ct][1], 0, 0, 0);
    }
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int col = ct * 16 + 4 * kk + r;
      if (col < ncol) *(float2*)(out_o + col * kHeadDim + 8 * kl + 2 * wave) = make_float2(acc[ct][0][r], acc[ct][1][r]);
    }
}

// Chunk softmax of this wave's columns wave + 4 c (c < NC): lane (c, j) =
// (lane / LG, lane % LG), LG = 64 / NC lanes per column, holds keys j + LG a
// (a < NC) of column c. The maximum runs on order-preserving integer keys (exact
// in any order; the sign of a zero maximum changes no exp(w - m)). The sum keeps
// wave_sum_f's pairing over the keys: the partners at xor 32 .. LG sit in the
// same lane (a ^ (32 / LG) .. a ^ 1), those at xor LG / 2 .. 1 in lanes j ^ 8
// (LG = 16: a row rotation by 8 is that exchange), j ^ 4, j ^ 2, j ^ 1.
template <int NC>
__device__ __forceinline__ void attn_f16_softmax(float* s_p, int ncol, float* out_ml) {
  static_assert(NC == 4 || NC == 8, "4 or 8 columns per wave");
  constexpr int LG = 64 / NC;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, c = lane / LG, j = lane % LG;
  const int col = wave + 4 * c;
  const bool live = col < ncol;
  float* row = s_p + min(col, ncol - 1) * kApStride;
  float w[NC];
  int mk = ord_key(-INFINITY);
#pragma unroll
  for (int a = 0; a < NC; ++a) {
    w[a] = live ? row[sp_key_pos(j + LG * a)] : -INFINITY;
    mk = max(mk, ord_key(w[a]));
  }
  if (LG == 16) mk = max(mk, (int)dpp_u<kDppRor8>((uint32_t)mk));
  mk = max(mk, (int)lane_xor4((uint32_t)mk));
  mk = max(mk, (int)dpp_u<kDppQuadXor2>((uint32_t)mk));
  mk = max(mk, (int)dpp_u<kDppQuadXor1>((uint32_t)mk));
  const float m = ord_val(mk);
  float p[NC], v[NC];
#pragma unroll
  for (int a = 0; a < NC; ++a) {
    p[a] = f16_round((m == -INFINITY || w[a] == -INFINITY) ? 0.0f : dev_expf(__fsub_rn(w[a], m)));
    v[a] = p[a];
  }
#pragma unroll
  for (int h = NC / 2; h >= 1; h /= 2)
#pragma unroll
    for (int a = 0; a < h; ++a) v[a] = __fadd_rn(v[a], v[a + h]);
  float l = v[0];
  if (LG == 16) l = __fadd_rn(l, dpp_f<kDppRor8>(l));
  l = __fadd_rn(l, __uint_as_float(lane_xor4(__float_as_uint(l))));
  l = __fadd_rn(l, dpp_f<kDppQuadXor2>(l));
  l = __fadd_rn(l, dpp_f<kDppQuadXor1>(l));
  if (live) {
#pragma unroll
    for (int a = 0; a < NC; ++a) row[sp_key_pos(j + LG * a)] = p[a];
    if (j == 0) {
      out_ml[col * 2] = m;
      out_ml[col * 2 + 1] = l;
    }
  }
}

__global__ void __launch_bounds__(256, 3)
k_attn_f16(const StepDesc* __restrict__ desc, const float* __restrict__ q, int n_heads, KvLayer kv,
           AttnWork work, int max_chunks) {
  const int g = blockIdx.x;
  const int T = desc->T, past = desc->past, kvlen = past + T;
  const int nch = (kvlen + kChunk - 1) / kChunk;
  int chunk = blockIdx.y;
  if (chunk >= nch) return;
  extern __shared__ v4f attn_lds_v4[];
  float* s_q = (float*)attn_lds_v4;  // [32][132] permuted; then the chunk's scores / probabilities
  float* s_p = s_q;
  uint16_t* s_k = (uint16_t*)(s_q + kMaxCols * kAqStride);  // [64][136] permuted
  uint32_t* s_v = (uint32_t*)(s_k + kChunk * kAkStrideH);   // [64][65] words
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, kl = lane & 15, kk = lane >> 4;
  const int ncol = 2 * T;
  const uint16_t* kb = (const uint16_t*)kv.k + (size_t)g * kv.max_seq * kHeadDim;
  const uint16_t* vb = (const uint16_t*)kv.v + (size_t)g * kv.max_seq * kHeadDim;
  // q columns, f16-rounded (mul_mat(f16 K, f32 q) converts q), into registers:
  // lane (kl, kk) of column tile ct holds column 16 ct + kl, elements 4 i + kk.
  // The q loads go out first, all of them, then the first chunk's K / V: the
  // staging below waits for q only (loads complete in order).
  constexpr int kQPieces = kMaxCols * (kHeadDim / 4) / 256;
  v4f qv[kQPieces];
#pragma unroll
  for (int j = 0; j < kQPieces; ++j) {
    const int idx = tid + 256 * j, col = idx / (kHeadDim / 4), d = (idx % (kHeadDim / 4)) * 4;
    if (col < ncol) qv[j] = *(const v4f*)(q + ((size_t)(col % T) * n_heads + 2 * g + col / T) * kHeadDim + d);
  }
  v4i pk[4], pv[4];
  attn_f16_load(kb, vb, chunk * kChunk, kvlen, pk, pv);
#pragma unroll
  for (int j = 0; j < kQPieces; ++j) {
    const int idx = tid + 256 * j, col = idx / (kHeadDim / 4), d = (idx % (kHeadDim / 4)) * 4;
    if (col < ncol)
#pragma unroll
      for (int e = 0; e < 4; ++e) s_q[col * kAqStride + attn_perm128(d + e)] = f16_round(qv[j][e]);
  }
  __syncthreads();
  float qreg[2][32];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    const int col = ct * 16 + kl;
    const float* qrow = s_q + min(col, ncol - 1) * kAqStride + kk * 32;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const v4f q4 = *(const v4f*)(qrow + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) qreg[ct][4 * i + j] = col < ncol ? q4[j] : 0.0f;
    }
  }
  __syncthreads();  // s_q is s_p from here on
  const float scale = __fdiv_rn(1.0f, dev_sqrtf((float)kHeadDim));
  for (; chunk < nch; chunk += gridDim.y) {
    const int key0 = chunk * kChunk;
    // 1. the chunk's rows to LDS; the next chunk's loads go out
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = i * 256 + tid, j = p >> 4, d8 = (p & 15) * 8;
      const uint32_t w0 = (uint32_t)pk[i][0], w1 = (uint32_t)pk[i][1], w2 = (uint32_t)pk[i][2],
                     w3 = (uint32_t)pk[i][3];
      // halves d8 + e and d8 + e + 4 are elements 4 (d8/4) + e and 4 (d8/4 + 1) + e
      uint32_t* kr = (uint32_t*)(s_k + j * kAkStrideH + d8 / 4);
      kr[0] = (w0 & 0xffffu) | (w2 << 16);
      kr[16] = (w0 >> 16) | (w2 & 0xffff0000u);
      kr[32] = (w1 & 0xffffu) | (w3 << 16);
      kr[48] = (w1 >> 16) | (w3 & 0xffff0000u);
      uint32_t* vr = s_v + j * kAvStrideW + d8 / 2;
      vr[0] = (uint32_t)pv[i][0];
      vr[1] = (uint32_t)pv[i][1];
      vr[2] = (uint32_t)pv[i][2];
      vr[3] = (uint32_t)pv[i][3];
    }
    if (chunk + (int)gridDim.y < nch) attn_f16_load(kb, vb, (chunk + gridDim.y) * kChunk, kvlen, pk, pv);
    __syncthreads();
    // 2. scores
    if (ncol > 16)
      attn_f16_scores<2>(s_k, qreg, s_p, key0, kvlen, past, T, ncol, scale);
    else
      attn_f16_scores<1>(s_k, qreg, s_p, key0, kvlen, past, T, ncol, scale);
    __syncthreads();
    // 3. chunk softmax per column (lane = key), a wave's columns side by side
    const size_t item = (size_t)g * max_chunks + chunk;
    float* out_ml = work.part_ml + item * kMaxCols * 2;
    float* out_o = work.part_o + item * kMaxCols * kHeadDim;
    if (ncol > 16)
      attn_f16_softmax<kMaxCols / 4>(s_p, ncol, out_ml);
    else
      attn_f16_softmax<4>(s_p, ncol, out_ml);
    __syncthreads();
    // 4. O = fma chain over the chunk's keys of p * v
    if (ncol > 16)
      attn_f16_pv<2>(s_v, s_p, ncol, out_o);
    else
      attn_f16_pv<1>(s_v, s_p, ncol, out_o);
    __syncthreads();  // s_k / s_v / s_p are rewritten by the next chunk
  }
}

// grid (n_heads, 16 rows), 128 threads: merge the chunks of one (head, row),
// write o (f32) and its q8_0 panel for the o-projection.
__global__ void __launch_bounds__(128)
k_attn_combine(const StepDesc* __restrict__ desc, AttnWork work, int n_heads, int max_chunks,
               Panel o_panel, float* __restrict__ o_out) {
  const int hq = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
  const int T = desc->T;
  if (t >= T) return;
  const int g = hq / 2, col = (hq & 1) * T + t;
  const int nch = (desc->past + T + kChunk - 1) / kChunk;
  const size_t item0 = (size_t)g * max_chunks;
  const float val = attn_merge<false>(work.part_ml + item0 * kMaxCols * 2 + col * 2,
                                      work.part_o + item0 * kMaxCols * kHeadDim + col * kHeadDim, nch,
                                      (size_t)kMaxCols * 2, (size_t)kMaxCols * kHeadDim, d);
  const int QN = n_heads * kHeadDim;
  o_out[(size_t)t * QN + hq * kHeadDim + d] = val;
  __shared__ float s_v[kHeadDim];
  s_v[d] = val;
  __syncthreads();
  if (d < 32) {
    float v[4];
    for (int e = 0; e < 4; ++e) v[e] = s_v[d * 4 + e];
    int8_t qv[4];
    const float ds = quant_block8(v, qv);
    const int k = hq * kHeadDim + d * 4;
    panel_store4(o_panel, QN / kPairK, t, k, qv);
    if ((d & 7) == 0) panel_store_scale(o_panel, QN / kPairK, t, k >> 5, ds);
  }
}

// ------------------------------------------------------- penalty bitmap -----
__global__ void k_penalty_bitmap(const StepDesc* __restrict__ desc, int vocab,
                                 uint32_t* __restrict__ bitmap) {
  const int t = blockIdx.x;
  if (t >= desc->T || !(desc->penalty > 1.0f)) return;
  const int words = (vocab + 31) / 32;
  uint32_t* row = bitmap + (size_t)t * words;
  for (int i = threadIdx.x; i < words; i += blockDim.x) row[i] = 0u;
  __syncthreads();
  __threadfence_block();
  const int end = desc->pen_base + t + 1;
  const int begin = max(0, end - kPenaltyWindow);
  for (int i = begin + (int)threadIdx.x; i < end; i += blockDim.x) {
    const int id = desc->pen_ids[i];
    if (id >= 0 && id < vocab) atomicOr(row + (id >> 5), 1u << (id & 31));
  }
}

// --------------------------------------------------------------- lm_head ----
// Grid-stride over 16-row tiles of the tied embedding; the activation panel is
// staged in LDS once per workgroup. Each lane keeps the best (value, index) key
// per verify row; ties keep the lowest index (first maximum).
template <int G>
__global__ void __launch_bounds__(256)
k_lm_head(const StepDesc* __restrict__ desc, const uint8_t* __restrict__ w, int vocab, int bps,
          Panel x, const uint32_t* __restrict__ bitmap, float* __restrict__ logits,
          uint64_t* __restrict__ part_keys) {
  const int T = desc->T;
  if ((T + 7) / 8 != G) return;
  extern __shared__ v4i lds_v4[];  // 16-byte aligned for the 128-bit panel reads
  uint8_t* lds = (uint8_t*)lds_v4;
  uint8_t* lcodes = lds;
  float* lscales = (float*)(lds + (size_t)G * bps * 1024);
  for (int i = threadIdx.x; i < G * bps * 64; i += blockDim.x)
    ((v4i*)lcodes)[i] = ((const v4i*)x.codes)[i];
  for (int i = threadIdx.x; i < G * bps * 16; i += blockDim.x) lscales[i] = x.scales[i];
  __syncthreads();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int n_tiles = vocab / 16;
  const int nwaves = gridDim.x * 4;
  const bool pen = desc->penalty > 1.0f;
  const float penalty = desc->penalty;
  const int words = (vocab + 31) / 32;
  uint64_t best[G];
#pragma unroll
  for (int cg = 0; cg < G; ++cg) best[cg] = 0;
  for (int tile = blockIdx.x * 4 + wave; tile < n_tiles; tile += nwaves) {
    float acc[G][4];
    tile_accumulate_canonical<G>(w + (size_t)tile * bps * kUnitBytes, bps, lcodes, lscales, acc);
    if ((lane & 15) < 8) {
#pragma unroll
      for (int cg = 0; cg < G; ++cg) {
        const int t = cg * 8 + (lane & 7);
        if (t < T) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = tile * 16 + 4 * (lane >> 4) + r;
            float v = acc[cg][r];
            if (desc->write_logits) logits[(size_t)t * vocab + row] = v;
            if (pen && ((bitmap[(size_t)t * words + (row >> 5)] >> (row & 31)) & 1u))
              v = v > 0.0f ? __fdiv_rn(v, penalty) : __fmul_rn(v, penalty);
            const uint64_t key = argmax_key(v, row);
            best[cg] = key > best[cg] ? key : best[cg];
          }
        }
      }
    }
  }
  // lanes with the same row t: xor 16, 32 (and the odd-parity lanes hold 0)
#pragma unroll
  for (int cg = 0; cg < G; ++cg) {
    uint64_t b = best[cg];
    uint64_t o = shfl_xor_u64(b, 16);
    b = o > b ? o : b;
    o = shfl_xor_u64(b, 32);
    b = o > b ? o : b;
    o = shfl_xor_u64(b, 8);
    b = o > b ? o : b;
    best[cg] = b;
  }
  __shared__ uint64_t s_best[4][kMaxRows];
  if (lane < 8)
#pragma unroll
    for (int cg = 0; cg < G; ++cg) s_best[wave][cg * 8 + lane] = best[cg];
  __syncthreads();
  if (threadIdx.x < G * 8) {
    uint64_t b = s_best[0][threadIdx.x];
    for (int wv = 1; wv < 4; ++wv) b = s_best[wv][threadIdx.x] > b ? s_best[wv][threadIdx.x] : b;
    part_keys[(size_t)blockIdx.x * kMaxRows + threadIdx.x] = b;
  }
}

// ---------------------------------------------------------------- accept ----
__global__ void __launch_bounds__(256)
k_accept(const StepDesc* __restrict__ desc, const uint64_t* __restrict__ part_keys, int nparts,
         StepResult* __restrict__ result) {
  const int T = desc->T;
  __shared__ uint64_t s_red[4][kMaxRows];
  __shared__ int32_t s_choice[kMaxRows];
  // thread (j, t) = (tid / 16, tid % 16) takes the keys of verify row t in the
  // parts j, j + 16, ... (a wave reads 512 contiguous bytes per pass); the
  // maxima meet over lanes xor 16 and 32, then over the four waves
  const int t = threadIdx.x & 15, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint64_t b = 0;
#pragma unroll 8
  for (int i = threadIdx.x >> 4; i < nparts; i += 16) {
    const uint64_t k = part_keys[(size_t)i * kMaxRows + t];
    b = k > b ? k : b;
  }
  {
    uint32_t alo, blo, ahi, bhi;
    pair_split<32>((uint32_t)b, alo, blo);
    pair_split<32>((uint32_t)(b >> 32), ahi, bhi);
    b = max(((uint64_t)ahi << 32) | alo, ((uint64_t)bhi << 32) | blo);
    pair_split<16>((uint32_t)b, alo, blo);
    pair_split<16>((uint32_t)(b >> 32), ahi, bhi);
    b = max(((uint64_t)ahi << 32) | alo, ((uint64_t)bhi << 32) | blo);
  }
  if (lane < 16) s_red[wave][lane] = b;
  __syncthreads();
  if ((int)threadIdx.x < T) {
    uint64_t m = s_red[0][threadIdx.x];
    for (int w = 1; w < 4; ++w) m = s_red[w][threadIdx.x] > m ? s_red[w][threadIdx.x] : m;
    s_choice[threadIdx.x] = (int32_t)(0xffffffffu - (uint32_t)(m & 0xffffffffu));
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int m = 0;
    while (m + 1 < T && desc->tokens[m + 1] == s_choice[m]) ++m;
    for (int t = 0; t < kMaxRows; ++t) result->choice[t] = t < T ? s_choice[t] : -1;
    result->n_match = m;
  }
}

// ------------------------------------------------------ causal context -----
// cpu_causal_context on device pointers: one thread per (head, query, f),
// summing exactly the valid length in key order.
__global__ void k_causal_context(const float* __restrict__ v, const float* __restrict__ p,
                                 int head_dim, int kv_heads, int heads, int queries, int kv_len,
                                 float* __restrict__ out) {
  const size_t total = (size_t)heads * queries * head_dim;
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int f = (int)(i % head_dim), q = (int)((i / head_dim) % queries), h = (int)(i / ((size_t)head_dim * queries));
  const int groups = heads / kv_heads, past = kv_len - queries;
  const float* vr = v + (size_t)(h / groups) * kv_len * head_dim + f;
  const float* pr = p + ((size_t)h * queries + q) * kv_len;
  float acc = 0.0f;
  for (int k = 0; k < past + q + 1; ++k) acc = __fadd_rn(acc, __fmul_rn(vr[(size_t)k * head_dim], pr[k]));
  out[i] = acc;
}

// --------------------------------------------------------------- retile -----
// ggml q8_0 rows (34-byte blocks) -> MFMA panel tiles. One thread per
// (tile, pair, lane): 16 code bytes, and lanes < 32 also move one f16 scale.
__global__ void k_q8_retile(const uint8_t* __restrict__ blocks, int n, int k,
                            uint8_t* __restrict__ tiles) {
  const int bps = k / kPairK, nb = k / 32;
  const size_t units = (size_t)(n / 16) * bps;
  const size_t gid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (gid >= units * 64) return;
  const int lane = (int)(gid & 63);
  const size_t unit = gid >> 6;
  const int tile = (int)(unit / bps), bp = (int)(unit % bps);
  uint8_t* dst = tiles + unit * kUnitBytes;
  {
    const int row = tile * 16 + (lane & 15), g = lane >> 4;
    const int block = 2 * bp + (g >> 1);
    const uint8_t* src = blocks + ((size_t)row * nb + block) * 34 + 2 + (g & 1) * 16;
    for (int b = 0; b < 16; ++b) dst[lane * 16 + b] = src[b];
  }
  if (lane < 32) {
    const int par = lane >> 4, r = lane & 15;
    const uint8_t* src = blocks + ((size_t)(tile * 16 + r) * nb + 2 * bp + par) * 34;
    dst[1024 + (par * 16 + r) * 2] = src[0];
    dst[1024 + (par * 16 + r) * 2 + 1] = src[1];
  }
}

}  // namespace

// ================================================================ launches ==
void launch_embed(hipStream_t s, const StepDesc* desc, const uint8_t* embd_tiles, int hidden,
                  const float* host_rows, float* x) {
  hipLaunchKernelGGL(k_embed, dim3(kMaxRows), dim3(256), 0, s, desc, embd_tiles, hidden, host_rows, x);
}

void launch_norm_quant(hipStream_t s, const StepDesc* desc, const float* src, int K,
                       const float* gain, float eps, Panel panel, float* normed_out) {
  hipLaunchKernelGGL(k_norm_quant, dim3(kMaxRows), dim3(256), 0, s, desc, src, K, gain, eps, panel,
                     normed_out);
}

template <int EPI, int SPLIT>
static void gemm_launch(hipStream_t s, int G, const StepDesc* desc, const uint8_t* w,
                        const uint8_t* w2, int n, int k, Panel x, float* out) {
  const int tiles = n / 16, bps = k / kPairK;
  if (G == 1)
    hipLaunchKernelGGL((k_gemm<EPI, SPLIT, 1>), dim3(tiles), dim3(SPLIT * 64), 0, s, desc, w, w2, n,
                       bps, x, out);
  else
    hipLaunchKernelGGL((k_gemm<EPI, SPLIT, 2>), dim3(tiles), dim3(SPLIT * 64), 0, s, desc, w, w2, n,
                       bps, x, out);
}

void launch_gemm_store(hipStream_t s, int G, const StepDesc* desc, const uint8_t* w, int n, int k,
                       Panel x, float* out) {
  gemm_launch<0, 4>(s, G, desc, w, nullptr, n, k, x, out);
}
void launch_gemm_residual(hipStream_t s, int G, const StepDesc* desc, const uint8_t* w, int n,
                          int k, Panel x, float* resid) {
  gemm_launch<1, 4>(s, G, desc, w, nullptr, n, k, x, resid);
}
void launch_gemm_swiglu(hipStream_t s, int G, const StepDesc* desc, const uint8_t* wg,
                        const uint8_t* wu, int n, int k, Panel x, float* act) {
  gemm_launch<2, 4>(s, G, desc, wg, wu, n, k, x, act);
}

void launch_qk_rope_append(hipStream_t s, const StepDesc* desc, const float* qkv, int n_heads,
                           int n_kv_heads, const float* q_norm, const float* k_norm, float eps,
                           const float* rope, float* q_out, KvLayer kv) {
  hipLaunchKernelGGL(k_qk_rope_append, dim3(kMaxRows, n_heads + 2 * n_kv_heads), dim3(64), 0, s,
                     desc, qkv, n_heads, n_kv_heads, q_norm, k_norm, eps, rope, q_out, kv);
}

hipError_t prepare_kernels() {
  const hipError_t e =
      hipFuncSetAttribute((const void*)k_attn_chunk, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kAttnLds);
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute((const void*)k_attn_f16, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)kAttnF16Lds);
}

int attn_max_chunks(const KvLayer& kv) { return (kv.max_seq + kChunk - 1) / kChunk; }

void launch_attn_chunks(hipStream_t s, const StepDesc* desc, const float* q, int n_heads, int n_kv_heads,
                        KvLayer kv, AttnWork work) {
  const int max_chunks = attn_max_chunks(kv);
  if (kv.f16) {
    const int ny = std::max(1, std::min(max_chunks, kAttnF16Waves / n_kv_heads));
    hipLaunchKernelGGL(k_attn_f16, dim3(n_kv_heads, ny), dim3(256), kAttnF16Lds, s, desc, q, n_heads, kv, work,
                       max_chunks);
  } else {
    hipLaunchKernelGGL(k_attn_chunk, dim3(n_kv_heads, max_chunks), dim3(256), kAttnLds, s, desc, q, n_heads,
                       kv, work, max_chunks);
  }
}

void launch_attention(hipStream_t s, const StepDesc* desc, const float* q, int n_heads,
                      int n_kv_heads, KvLayer kv, AttnWork work, Panel o_panel, float* o_out) {
  const int max_chunks = attn_max_chunks(kv);
  launch_attn_chunks(s, desc, q, n_heads, n_kv_heads, kv, work);
  hipLaunchKernelGGL(k_attn_combine, dim3(n_heads, kMaxRows), dim3(kHeadDim), 0, s, desc, work,
                     n_heads, max_chunks, o_panel, o_out);
}

void launch_penalty_bitmap(hipStream_t s, const StepDesc* desc, int vocab, uint32_t* bitmap) {
  hipLaunchKernelGGL(k_penalty_bitmap, dim3(kMaxRows), dim3(256), 0, s, desc, vocab, bitmap);
}

void launch_lm_head(hipStream_t s, int G, const StepDesc* desc, const uint8_t* w, int vocab,
                    int k, Panel x, const uint32_t* bitmap, float* logits, uint64_t* part_keys) {
  const int bps = k / kPairK;
  const size_t lds = (size_t)G * bps * (1024 + 64);
  if (G == 1)
    hipLaunchKernelGGL(k_lm_head<1>, dim3(kLmWorkgroups), dim3(256), lds, s, desc, w, vocab, bps,
                       x, bitmap, logits, part_keys);
  else
    hipLaunchKernelGGL(k_lm_head<2>, dim3(kLmWorkgroups), dim3(256), lds, s, desc, w, vocab, bps,
                       x, bitmap, logits, part_keys);
}

void launch_accept(hipStream_t s, const StepDesc* desc, const uint64_t* part_keys,
                   StepResult* result) {
  hipLaunchKernelGGL(k_accept, dim3(1), dim3(256), 0, s, desc, part_keys, kLmWorkgroups, result);
}

void launch_causal_context(hipStream_t s, const float* v, const float* p, int head_dim,
                           int kv_heads, int heads, int queries, int kv_len, float* out) {
  const size_t total = (size_t)heads * queries * head_dim;
  hipLaunchKernelGGL(k_causal_context, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, v, p,
                     head_dim, kv_heads, heads, queries, kv_len, out);
}

void launch_q8_retile(hipStream_t s, const uint8_t* blocks, int n, int k, uint8_t* tiles) {
  const size_t threads = (size_t)(n / 16) * (k / kPairK) * 64;
  hipLaunchKernelGGL(k_q8_retile, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, blocks, n,
                     k, tiles);
}

}  // namespace mtg
