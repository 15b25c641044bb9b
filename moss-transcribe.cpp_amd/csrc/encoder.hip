// encoder.hip - the Whisper audio encoder and the audio adaptor on the device
// (reference WhisperEncoder::encode, src/whisper_encoder.cpp:103-209, and
// AudioAdaptor::apply, src/audio_adaptor.cpp:38-97).
//
//   conv stem  k_enc_conv_mma: conv1d (kernel 3, pad 1) on f32 MFMA, one fma
//              chain per output over (input channel, tap), + bias, GELU (erf);
//              conv2 (stride 2) also adds the positional embedding and writes
//              [rows][d]
//   layers     k_enc_ln: LayerNorm (mean and variance as double sums over 64
//              lane partials, butterfly) -> q8_0 codes for the next GEMM;
//              q / k / v / out / fc1 / fc2 on the block GEMM of the prefill
//              (q8_0 weights x q8_0 activations, int8 MFMA) with bias, GELU or
//              residual epilogues; k_enc_attn_mma: bidirectional attention
//              on f32 MFMA, 16 query rows of one head per wave over all rows
//              in 64-key chunks (two passes: row maxima, then exp / sums /
//              context merged in chunk order)
//   adaptor    merge consecutive rows (a view), fc1 + SiLU, fc2, LayerNorm
// Every reduction keeps the oracle's order (oracle/oracle.cpp, encoder
// section), so results equal it bit for bit.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "device_common.hpp"
#include "mtg_internal.hpp"

namespace mtg {
namespace {
using namespace dev;

constexpr int kEncHd = 64;      // head_dim
constexpr int kEncRows = 64;    // query rows per attention workgroup (16 per wave)
constexpr int kEncMaxChunks = 32;  // rows <= 2048
constexpr int kConvTile = 64;   // outputs per conv workgroup: 64 rows x 64 channels
constexpr int kConvIcb = 16;    // input channels staged per step

// ------------------------------------------------------------- conv stem ---
// out = gelu(conv(x) + b) (+ pos) on f32 MFMA: the conv as a GEMM over
// n = 3 c + k (input channel c, tap k), out[t][o] = sum_n w[o][n] X[n][t] with
// X[n][t] = x[c][t * STRIDE + k - 1] (0 outside the frames). One MFMA chain per
// 16 x 16 output tile over n in order is the canonical fma chain (tap fastest).
// Workgroup: outputs o0 .. o0 + 63 x t0 .. t0 + 63; wave w: channels
// o0 + 16 w + i (A = w rows) x four 16-row tiles of t (B = X columns). Per block
// of 16 input channels (48 values of n) the w slab (element n = 4 s + g at
// g * 12 + s) and the x rows are staged in LDS; the next block's loads are in
// flight during the current block's MFMAs.
// TRANS: out [OC][OL] (conv2's input layout), else out [OL][OC].
constexpr int kCvNb = 3 * kConvIcb;  // values of n per staged block
constexpr int kCvWs = kCvNb + 4;     // w slab row stride (floats)
template <int STRIDE, bool TRANS>
__global__ void __launch_bounds__(256)
k_enc_conv_mma(const float* __restrict__ w, const float* __restrict__ b, const float* __restrict__ x, int IC, int L,
               int OC, const float* __restrict__ pos, float* __restrict__ out) {
  constexpr int XW = kConvTile * STRIDE + 2;
  constexpr int XN = (kConvIcb * XW + 255) / 256;  // x values per thread and block
  __shared__ __align__(16) float xs[kConvIcb * XW];
  __shared__ __align__(16) float ws[kConvTile * kCvWs];
  const int OL = (L - 1) / STRIDE + 1;
  const int t0 = blockIdx.x * kConvTile, o0 = blockIdx.y * kConvTile;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, g = lane >> 4;
  const int p0 = t0 * STRIDE - 1;  // the input position of tap 0 of row t0
  // this lane's x offsets in the staged block: n = 4 s + g -> (c, k) = (n / 3, n % 3)
  int xo[12];
#pragma unroll
  for (int s = 0; s < 12; ++s) {
    const int n = 4 * s + g;
    xo[s] = (n / 3) * XW + n % 3 + j * STRIDE;
  }
  v4f wr[3];
  float xr[XN];
  auto load = [&](int ic0) {
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int i = tid + 256 * u, o = i / (kCvNb / 4), q = i % (kCvNb / 4);
      wr[u] = *(const v4f*)(w + (size_t)(o0 + o) * IC * 3 + (size_t)ic0 * 3 + 4 * q);
    }
#pragma unroll
    for (int u = 0; u < XN; ++u) {
      const int i = tid + 256 * u, c = i / XW, p = p0 + i % XW;
      xr[u] = (i < kConvIcb * XW && p >= 0 && p < L) ? x[(size_t)(ic0 + min(c, kConvIcb - 1)) * L + min(max(p, 0), L - 1)]
                                                      : 0.0f;
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int i = tid + 256 * u, o = i / (kCvNb / 4), q = i % (kCvNb / 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) ws[o * kCvWs + e * 12 + q] = wr[u][e];  // n = 4 q + e
    }
#pragma unroll
    for (int u = 0; u < XN; ++u) {
      const int i = tid + 256 * u;
      if (i < kConvIcb * XW) xs[i] = xr[u];
    }
  };
  v4f acc[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) acc[tt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  load(0);
  for (int ic0 = 0; ic0 < IC; ic0 += kConvIcb) {
    __syncthreads();  // the previous block's operands are consumed
    stage();
    __syncthreads();
    if (ic0 + kConvIcb < IC) load(ic0 + kConvIcb);
    v4f a[3];
    const float* wrow = ws + (16 * wave + j) * kCvWs + g * 12;
#pragma unroll
    for (int u = 0; u < 3; ++u) a[u] = *(const v4f*)(wrow + 4 * u);
#pragma unroll
    for (int s = 0; s < 12; ++s)
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s >> 2][s & 3], xs[xo[s] + 16 * tt * STRIDE], acc[tt], 0, 0,
                                                       0);
  }
  // acc[tt][r]: output channel o0 + 16 wave + 4 g + r, row t0 + 16 tt + j
  const int ob = o0 + 16 * wave + 4 * g;
  const v4f bias = *(const v4f*)(b + ob);
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = __fadd_rn(acc[2 * h + e / 4][e % 4], bias[e % 4]);
    dev_gelu_erf_n<8>(y);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = t0 + 16 * (2 * h + u) + j;
      if (t >= OL) continue;
      v4f v;
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = y[4 * u + r];
      if (pos) {
        const v4f pv = *(const v4f*)(pos + (size_t)t * OC + ob);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = __fadd_rn(v[r], pv[r]);
      }
      if constexpr (TRANS) {
#pragma unroll
        for (int r = 0; r < 4; ++r) out[(size_t)(ob + r) * OL + t] = v[r];
      } else {
        *(v4f*)(out + (size_t)t * OC + ob) = v;
      }
    }
  }
}

// ------------------------------------------------------------ LayerNorm ----
// One wave per row of 1024 (lane l: elements 16 l .. 16 l + 15): mean and
// variance as double sums of the lanes' sequential partials, wave_sum_d; y =
// ((x - mean) * scale) * w + b with scale = 1 / sqrt(variance + eps). codes /
// scales (nullable): y as q8_0; yout (nullable): y as f32.
__global__ void __launch_bounds__(256)
k_enc_ln(const float* __restrict__ src, int S, const float* __restrict__ w, const float* __restrict__ b, float eps,
         int8_t* __restrict__ codes, float* __restrict__ scales, float* __restrict__ yout) {
  constexpr int D = 1024;
  const int row = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= S) return;
  const float* xr = src + (size_t)row * D + 16 * lane;
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
  for (int e = 0; e < 16; ++e) s = __dadd_rn(s, (double)v[e]);
  s = wave_sum_d(s);
  const float mean = (float)__ddiv_rn(s, (double)D);
  double s2 = 0.0;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    v[e] = __fsub_rn(v[e], mean);
    s2 = __dadd_rn(s2, (double)__fmul_rn(v[e], v[e]));
  }
  s2 = wave_sum_d(s2);
  const float variance = (float)__ddiv_rn(s2, (double)D);
  const float scale = dev_rms_scale(variance, eps);  // 1 / sqrt(variance + eps), correctly rounded
  float y[16];
#pragma unroll
  for (int e = 0; e < 16; ++e)
    y[e] = __fadd_rn(__fmul_rn(__fmul_rn(v[e], scale), w[16 * lane + e]), b[16 * lane + e]);
  if (yout)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *(v4f*)(yout + (size_t)row * D + 16 * lane + 4 * i) = v4f{y[4 * i], y[4 * i + 1], y[4 * i + 2], y[4 * i + 3]};
  if (codes) {
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
      for (int q = 0; q < 4; ++q) u |= (uint32_t)(uint8_t)(int8_t)rintf(__fmul_rn(y[4 * w4 + q], id)) << (8 * q);
      packed[w4] = u;
    }
    *(uint4*)(codes + (size_t)row * D + 16 * lane) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    if ((lane & 1) == 0) scales[(size_t)row * (D / 32) + lane / 2] = __half2float(__float2half_rn(d));
  }
}

// ------------------------------------------------------------ attention ----
// Bidirectional attention on f32 MFMA (v_mfma_f32_16x16x4f32, whose 4-term dot
// is the sequential fma chain fma(a3, b3, fma(a2, b2, fma(a1, b1, fma(a0, b0, c))))).
// Workgroup = head blockIdx.x, rows r0 .. r0 + 63; wave w owns the 16 query rows
// r0 + 16 w + j (j = lane % 16) over all keys, in 64-key chunks staged in LDS by
// the whole workgroup (double-buffered, the next chunk's loads in flight during
// the current chunk's arithmetic).
//   scores: key tile t (16 keys) is one MFMA chain over head_dim, A = K rows,
//     B = this wave's q rows (registers). A row i of tile t is key
//     16 t + 4 (i % 4) + i / 4, so the output register r of lane (g, j)
//     (g = lane / 16) holds the score of key 16 t + 4 r + g: key 4 m + g with
//     m = 4 t + r, which is where the P.V MFMA m (keys 4 m .. 4 m + 3, in order)
//     wants its B operand. The probabilities never leave the registers.
//   chunk sum: the xor butterfly over the chunk's keys: levels 32 and 16 (t),
//     8 and 4 (r) inside the lane, 2 and 1 (g) across lanes xor 32 and 16.
//   P.V: head_dim tile dt is one MFMA chain over the chunk's keys, A = V^T.
// Pass 1 takes each row's maximum over all keys; pass 2 recomputes the scores,
// the chunk maxima m_c, p = exp(w - m_c), l_c and O_c, and merges the chunks in
// order with f = exp(m_c - M): L = fma(l_c, f, L), O = fma(O_c, f, O).
// LDS: K rows at slot 16 t + 4 g + r for key 16 t + 4 r + g, element 4 s + kk at
// kk * 16 + s; V^T rows d with key 4 m + g at g * 16 + m. Rows 68 floats apart.
constexpr int kEaStride = 68;
constexpr int kEaBuf = 64 * kEaStride;  // floats per staged chunk (K or V^T)
constexpr size_t kEaLds = (size_t)4 * kEaBuf * 4;  // K and V^T, two buffers each

__device__ __forceinline__ void ea_load_k(const float* __restrict__ k, int key0, int T, int W, int h, v4f (&r)[4]) {
  const int tid = threadIdx.x, key = tid >> 2, q = tid & 3;
  const float* src = k + (size_t)min(key0 + key, T - 1) * W + h * kEncHd + 16 * q;
#pragma unroll
  for (int x = 0; x < 4; ++x) r[x] = *(const v4f*)(src + 4 * x);
}
// K row key (element 16 q + 4 x + e = 4 s + kk with s = 4 q + x, kk = e) to slot
// 16 t + 4 g + r of key 16 t + 4 r + g; rows past T are zero
__device__ __forceinline__ void ea_store_k(float* s_k, int key0, int T, const v4f (&r)[4]) {
  const int tid = threadIdx.x, key = tid >> 2, q = tid & 3;
  const int slot = (key & ~15) | ((key & 3) << 2) | ((key >> 2) & 3);
  const bool live = key0 + key < T;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v4f o;
#pragma unroll
    for (int x = 0; x < 4; ++x) o[x] = live ? r[x][e] : 0.0f;
    *(v4f*)(s_k + slot * kEaStride + e * 16 + 4 * q) = o;
  }
}
// V: thread (g, mq, u) loads keys 4 (4 mq + x) + g, elements 4 u .. 4 u + 3
__device__ __forceinline__ void ea_load_v(const float* __restrict__ v, int key0, int T, int W, int h, v4f (&r)[4]) {
  const int tid = threadIdx.x, u = tid & 15, mq = (tid >> 4) & 3, g = tid >> 6;
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int key = 4 * (4 * mq + x) + g;
    r[x] = *(const v4f*)(v + (size_t)min(key0 + key, T - 1) * W + h * kEncHd + 4 * u);
  }
}
__device__ __forceinline__ void ea_store_v(float* s_v, int key0, int T, const v4f (&r)[4]) {
  const int tid = threadIdx.x, u = tid & 15, mq = (tid >> 4) & 3, g = tid >> 6;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v4f o;
#pragma unroll
    for (int x = 0; x < 4; ++x) o[x] = key0 + 4 * (4 * mq + x) + g < T ? r[x][e] : 0.0f;
    *(v4f*)(s_v + (4 * u + e) * kEaStride + g * 16 + 4 * mq) = o;
  }
}

__global__ void __launch_bounds__(256, 2)
k_enc_attn_mma(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, int T, int W,
               float* __restrict__ out) {
  extern __shared__ v4f ea_lds_v4[];
  float* s_k = (float*)ea_lds_v4;  // [2][kEaBuf]
  float* s_v = s_k + 2 * kEaBuf;   // [2][kEaBuf]
  const int h = blockIdx.x, r0 = blockIdx.y * kEncRows;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, j = lane & 15, g = lane >> 4;
  const int nch = (T + 63) / 64;
  const float scale = __fdiv_rn(1.0f, dev_sqrtf((float)kEncHd));
  // the B operand of the scores: q[row][4 s + g], s < 16 (rows past T: zeros)
  const int row = r0 + 16 * wave + j;
  float qb[16];
  {
    const float* qr = q + (size_t)min(row, T - 1) * W + h * kEncHd + g;
#pragma unroll
    for (int s = 0; s < 16; ++s) qb[s] = row < T ? qr[4 * s] : 0.0f;
  }
  // scores of the staged chunk at key0: w[t][r] = key 16 t + 4 r + g, row j
  auto scores = [&](const float* sk, int key0, float (&w)[4][4]) {
    v4f acc[4];
    v4f a[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      const float* kr = sk + (16 * t + j) * kEaStride + g * 16;
#pragma unroll
      for (int x = 0; x < 4; ++x) a[t][x] = *(const v4f*)(kr + 4 * x);
    }
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t][s >> 2][s & 3], qb[s], acc[t], 0, 0, 0);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) w[t][r] = key0 + 16 * t + 4 * r + g < T ? __fmul_rn(acc[t][r], scale) : -INFINITY;
  };
  v4f kr[4], vr[4];
  // chunk n of the whole walk: n < nch is pass 1 (K only), n >= nch pass 2 (K and V)
  ea_load_k(k, 0, T, W, h, kr);
  ea_store_k(s_k, 0, T, kr);
  __syncthreads();
  float M = -INFINITY;
  for (int n = 0; n < nch; ++n) {
    const int nx = n + 1 < nch ? n + 1 : 0;  // the next staged chunk (pass 2 starts at chunk 0)
    ea_load_k(k, 64 * nx, T, W, h, kr);
    if (n + 1 == nch) ea_load_v(v, 0, T, W, h, vr);
    float w[4][4];
    scores(s_k + (n & 1) * kEaBuf, 64 * n, w);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) M = fmaxf(M, w[t][r]);
    ea_store_k(s_k + ((n + 1) & 1) * kEaBuf, 64 * nx, T, kr);
    if (n + 1 == nch) ea_store_v(s_v + ((n + 1) & 1) * kEaBuf, 0, T, vr);
    __syncthreads();
  }
  M = pair_max_f<32>(M);
  M = pair_max_f<16>(M);
  float L = 0.0f;
  v4f O[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) O[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  for (int c = 0; c < nch; ++c) {
    const int b = (nch + c) & 1;
    const bool more = c + 1 < nch;
    if (more) {
      ea_load_k(k, 64 * (c + 1), T, W, h, kr);
      ea_load_v(v, 64 * (c + 1), T, W, h, vr);
    }
    float w[4][4];
    scores(s_k + b * kEaBuf, 64 * c, w);
    float mc = -INFINITY;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) mc = fmaxf(mc, w[t][r]);
    mc = pair_max_f<32>(mc);
    mc = pair_max_f<16>(mc);
    float p[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) p[t][r] = w[t][r] == -INFINITY ? 0.0f : dev_expf(__fsub_rn(w[t][r], mc));
    // l_c: key levels 32, 16 (t), 8, 4 (r) in the lane, 2, 1 (g) across lanes
    float lc;
    {
      float u[2][4];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) u[t][r] = __fadd_rn(p[t][r], p[t + 2][r]);
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = __fadd_rn(u[0][r], u[1][r]);
      const float y0 = __fadd_rn(x[0], x[2]), y1 = __fadd_rn(x[1], x[3]);
      lc = pair_add_f<32>(__fadd_rn(y0, y1));
      lc = pair_add_f<16>(lc);
    }
    // O_c: head_dim tiles dt, A = V^T rows 16 dt + j, B = p (key 4 m + g at p[m / 4][m % 4])
    const float* sv = s_v + b * kEaBuf;
    v4f oc[4];
    v4f av[4][4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      oc[dt] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      const float* vrow = sv + (16 * dt + j) * kEaStride + g * 16;
#pragma unroll
      for (int x = 0; x < 4; ++x) av[dt][x] = *(const v4f*)(vrow + 4 * x);
    }
#pragma unroll
    for (int m = 0; m < 16; ++m)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        oc[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[dt][m >> 2][m & 3], p[m >> 2][m & 3], oc[dt], 0, 0, 0);
    const float f = dev_expf(__fsub_rn(mc, M));
    L = fmaf(lc, f, L);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) O[dt][r] = fmaf(oc[dt][r], f, O[dt][r]);
    if (more) {
      ea_store_k(s_k + (b ^ 1) * kEaBuf, 64 * (c + 1), T, kr);
      ea_store_v(s_v + (b ^ 1) * kEaBuf, 64 * (c + 1), T, vr);
    }
    __syncthreads();
  }
  // O[dt][r] is element 16 dt + 4 g + r of row j
  if (row < T) {
    float* orow = out + (size_t)row * W + h * kEncHd + 4 * g;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      v4f o4;
#pragma unroll
      for (int r = 0; r < 4; ++r) o4[r] = __fdiv_rn(O[dt][r], L);
      *(v4f*)(orow + 16 * dt) = o4;
    }
  }
}

size_t q8_tiles_bytes(int n, int k) { return (size_t)(n / 16) * (k / kPairK) * kUnitBytes; }

}  // namespace
}  // namespace mtg

// ------------------------------------------------------------------ host ---
using namespace mtg;

struct mtg_encoder {
  mtg_encoder_hparams hp{};
  int rows = 0;  // encoder output rows per chunk
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  std::vector<void*> allocs;
  std::string error;
  double last_ms = 0.0;
  int last_rows = 0;
  struct Layer {
    float *attn_ln_w, *attn_ln_b, *q_b, *v_b, *o_b, *ffn_ln_w, *ffn_ln_b, *fc1_b, *fc2_b;
    uint8_t *q_w, *k_w, *v_w, *o_w, *fc1_w, *fc2_w;
  };
  std::vector<Layer> layers;
  float *conv1_w = nullptr, *conv1_b = nullptr, *conv2_w = nullptr, *conv2_b = nullptr, *pos = nullptr,
        *ln_post_w = nullptr, *ln_post_b = nullptr;
  uint8_t *ad_fc1_w = nullptr, *ad_fc2_w = nullptr;
  float *ad_fc1_b = nullptr, *ad_fc2_b = nullptr, *ad_ln_w = nullptr, *ad_ln_b = nullptr;
  // activations
  float *mel = nullptr, *c1 = nullptr, *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *a = nullptr,
        *f = nullptr, *out_rows = nullptr, *in_rows = nullptr, *h1 = nullptr, *h2 = nullptr, *ad_out = nullptr;
  int8_t* codes = nullptr;
  float* scales = nullptr;
  // f16 / q4_K matrices (GGUF row layout): the GEMMs' activation (f16 values or
  // q8_K blocks) and the LayerNorm rows it is made from
  int wtype = MTG_TYPE_Q8_0;
  WtAct act{};
  float* xn = nullptr;

  ~mtg_encoder() {
    for (void* p : allocs) (void)hipFree(p);
    if (ev0) (void)hipEventDestroy(ev0);
    if (ev1) (void)hipEventDestroy(ev1);
    if (stream) (void)hipStreamDestroy(stream);
  }
  int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    error = buf;
    return code;
  }
  int check(hipError_t e, const char* what) {
    return e == hipSuccess ? MTG_OK : fail(MTG_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
  }
  void* dalloc(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return nullptr;
    allocs.push_back(p);
    return p;
  }
  float* up_f(const float* src, size_t n, int& rc) {
    if (rc) return nullptr;
    if (!src) {
      rc = fail(MTG_ERR_INVALID, "a tensor pointer is NULL");
      return nullptr;
    }
    float* d = (float*)dalloc(n * 4);
    if (!d) {
      rc = fail(MTG_ERR_NOMEM, "device memory");
      return nullptr;
    }
    rc = check(hipMemcpy(d, src, n * 4, hipMemcpyHostToDevice), "upload");
    return d;
  }
  uint8_t* up_q8(const void* src, int n, int kk, uint8_t* staging, int& rc) {
    if (rc) return nullptr;
    if (!src) {
      rc = fail(MTG_ERR_INVALID, "a tensor pointer is NULL");
      return nullptr;
    }
    uint8_t* d = (uint8_t*)dalloc(q8_tiles_bytes(n, kk));
    if (!d) {
      rc = fail(MTG_ERR_NOMEM, "device memory");
      return nullptr;
    }
    const size_t raw = (size_t)n * (kk / 32) * 34;
    if ((rc = check(hipMemcpy(staging, src, raw, hipMemcpyHostToDevice), "upload"))) return nullptr;
    launch_q8_retile(stream, staging, n, kk, d);
    if ((rc = check(hipGetLastError(), "retile"))) return nullptr;
    rc = check(hipStreamSynchronize(stream), "retile");
    return d;
  }
  // an n x kk matrix: q8_0 re-tiled for the int8 MFMA GEMM, f16 / f32 / q4_K as they are
  uint8_t* up_w(const void* src, int n, int kk, uint8_t* staging, int& rc) {
    if (wtype == MTG_TYPE_Q8_0) return up_q8(src, n, kk, staging, rc);
    if (rc) return nullptr;
    if (!src) {
      rc = fail(MTG_ERR_INVALID, "a tensor pointer is NULL");
      return nullptr;
    }
    const size_t bytes = (size_t)n * (wtype == MTG_TYPE_F16   ? (size_t)kk * 2
                                      : wtype == MTG_TYPE_F32 ? (size_t)kk * 4
                                                              : (size_t)(kk / 256) * 144);
    uint8_t* d = (uint8_t*)dalloc(bytes);
    if (!d) {
      rc = fail(MTG_ERR_NOMEM, "device memory");
      return nullptr;
    }
    rc = check(hipMemcpy(d, src, bytes, hipMemcpyHostToDevice), "upload");
    return d;
  }
  // src rows as the next GEMM's activation
  void quant(const float* src, int S, int K) {
    if (wtype == MTG_TYPE_Q8_0) launch_pf_quant(stream, src, S, K, codes, scales);
    else launch_pf_act_wt(stream, wtype, src, S, K, nullptr, 0.0f, act);
  }
  void gemm(int epi, const uint8_t* w, int N, int K, int S, float* out, const float* bias) {
    if (wtype == MTG_TYPE_Q8_0) launch_pf_gemm(stream, epi, w, nullptr, N, K, codes, scales, S, out, bias);
    else launch_pf_gemm_wt(stream, wtype, epi, w, nullptr, N, K, act, S, out, bias);
  }
  // LayerNorm of S rows of d_model: as the next GEMM's activation (q8), or as f32
  // rows in yout
  void ln(const float* src, int S, const float* w, const float* b, float eps, bool q8, float* yout) {
    if (q8 && wtype != MTG_TYPE_Q8_0) {
      hipLaunchKernelGGL(k_enc_ln, dim3((S + 3) / 4), dim3(256), 0, stream, src, S, w, b, eps, nullptr, nullptr, xn);
      quant(xn, S, hp.d_model);
      return;
    }
    hipLaunchKernelGGL(k_enc_ln, dim3((S + 3) / 4), dim3(256), 0, stream, src, S, w, b, eps, q8 ? codes : nullptr,
                       q8 ? scales : nullptr, yout);
  }
};

extern "C" {

int mtg_encoder_create(const mtg_encoder_desc* d, mtg_encoder** out) {
  if (!d || !out) return MTG_ERR_INVALID;
  *out = nullptr;
  const mtg_encoder_hparams& hp = d->hp;
  const int wt = d->weight_type;
  const bool wt_ok = wt == MTG_TYPE_Q8_0 ||
                     ((wt == MTG_TYPE_F16 || wt == MTG_TYPE_F32 || wt == MTG_TYPE_Q4_K) &&
                      pf_gemm_wt_supported(wt, hp.d_model) &&
                      pf_gemm_wt_supported(wt, hp.ffn) && pf_gemm_wt_supported(wt, hp.hidden) &&
                      pf_gemm_wt_supported(wt, hp.d_model * hp.merge));
  if (!wt_ok || hp.d_model != 1024 || hp.hidden != 1024 || hp.n_heads <= 0 ||
      hp.d_model / hp.n_heads != kEncHd || hp.d_model % hp.n_heads || hp.ffn % 64 || hp.n_mels % kConvIcb ||
      hp.n_mels <= 0 || hp.merge <= 0 || hp.n_layers < 0 || hp.n_frames < 2 ||
      (hp.n_frames - 1) / 2 + 1 > 64 * kEncMaxChunks)
    return MTG_ERR_UNSUPPORTED;
  if (!d->layers && hp.n_layers > 0) return MTG_ERR_INVALID;
  mtg_encoder* e = new (std::nothrow) mtg_encoder();
  if (!e) return MTG_ERR_NOMEM;
  e->hp = hp;
  e->wtype = wt;
  const int D = hp.d_model, F = hp.ffn, M = hp.n_mels, NF = hp.n_frames, R = (NF - 1) / 2 + 1, H = hp.hidden,
            IN = D * hp.merge;
  e->rows = R;
  int rc = e->check(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking), "stream");
  if (!rc) rc = e->check(hipEventCreate(&e->ev0), "event");
  if (!rc) rc = e->check(hipEventCreate(&e->ev1), "event");
  if (!rc)
    rc = e->check(hipFuncSetAttribute((const void*)k_enc_attn_mma, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      (int)kEaLds),
                  "attention LDS");
  // staging for the raw q8_0 rows of the largest matrix
  size_t raw_max = (size_t)std::max(F, std::max(D, H)) * (std::max(F, IN) / 32) * 34;
  uint8_t* staging = rc ? nullptr : (uint8_t*)e->dalloc(raw_max);
  if (!rc && !staging) rc = e->fail(MTG_ERR_NOMEM, "device memory");
  e->conv1_w = e->up_f(d->conv1_w, (size_t)D * M * 3, rc);
  e->conv1_b = e->up_f(d->conv1_b, D, rc);
  e->conv2_w = e->up_f(d->conv2_w, (size_t)D * D * 3, rc);
  e->conv2_b = e->up_f(d->conv2_b, D, rc);
  e->pos = e->up_f(d->pos_embd, (size_t)R * D, rc);
  e->ln_post_w = e->up_f(d->ln_post_w, D, rc);
  e->ln_post_b = e->up_f(d->ln_post_b, D, rc);
  for (int l = 0; l < hp.n_layers && !rc; ++l) {
    const mtg_encoder_layer& s = d->layers[l];
    mtg_encoder::Layer L{};
    L.attn_ln_w = e->up_f(s.attn_ln_w, D, rc);
    L.attn_ln_b = e->up_f(s.attn_ln_b, D, rc);
    L.q_w = e->up_w(s.q_w, D, D, staging, rc);
    L.k_w = e->up_w(s.k_w, D, D, staging, rc);
    L.v_w = e->up_w(s.v_w, D, D, staging, rc);
    L.o_w = e->up_w(s.o_w, D, D, staging, rc);
    L.q_b = e->up_f(s.q_b, D, rc);
    L.v_b = e->up_f(s.v_b, D, rc);
    L.o_b = e->up_f(s.o_b, D, rc);
    L.ffn_ln_w = e->up_f(s.ffn_ln_w, D, rc);
    L.ffn_ln_b = e->up_f(s.ffn_ln_b, D, rc);
    L.fc1_w = e->up_w(s.fc1_w, F, D, staging, rc);
    L.fc1_b = e->up_f(s.fc1_b, F, rc);
    L.fc2_w = e->up_w(s.fc2_w, D, F, staging, rc);
    L.fc2_b = e->up_f(s.fc2_b, D, rc);
    e->layers.push_back(L);
  }
  e->ad_fc1_w = e->up_w(d->ad_fc1_w, H, IN, staging, rc);
  e->ad_fc1_b = e->up_f(d->ad_fc1_b, H, rc);
  e->ad_fc2_w = e->up_w(d->ad_fc2_w, H, H, staging, rc);
  e->ad_fc2_b = e->up_f(d->ad_fc2_b, H, rc);
  e->ad_ln_w = e->up_f(d->ad_ln_w, H, rc);
  e->ad_ln_b = e->up_f(d->ad_ln_b, H, rc);
  if (!rc) {
    const size_t RD = (size_t)R * D;
    e->mel = (float*)e->dalloc((size_t)M * NF * 4);
    e->c1 = (float*)e->dalloc((size_t)D * NF * 4);
    e->x = (float*)e->dalloc(RD * 4);
    e->q = (float*)e->dalloc(RD * 4);
    e->k = (float*)e->dalloc(RD * 4);
    e->v = (float*)e->dalloc(RD * 4);
    e->a = (float*)e->dalloc(RD * 4);
    e->f = (float*)e->dalloc((size_t)R * F * 4);
    e->out_rows = (float*)e->dalloc(RD * 4);
    e->in_rows = (float*)e->dalloc(RD * 4);
    const int N = R / hp.merge + 1;
    e->h1 = (float*)e->dalloc((size_t)N * H * 4);
    e->h2 = (float*)e->dalloc((size_t)N * H * 4);
    e->ad_out = (float*)e->dalloc((size_t)N * H * 4);
    const size_t KC = std::max((size_t)R * std::max(F, D), (size_t)N * IN);
    e->codes = (int8_t*)e->dalloc(KC);
    e->scales = (float*)e->dalloc(KC / 32 * 4);
    if (wt == MTG_TYPE_F16) {
      e->act.f16h = (uint16_t*)e->dalloc(KC * 2);
      if (!e->act.f16h) rc = e->fail(MTG_ERR_NOMEM, "device memory");
    } else if (wt == MTG_TYPE_F32) {
      e->act.f32 = (float*)e->dalloc(KC * 4);
      if (!e->act.f32) rc = e->fail(MTG_ERR_NOMEM, "device memory");
    } else if (wt == MTG_TYPE_Q4_K) {
      e->act.q8k.qs = (int8_t*)e->dalloc(KC);
      e->act.q8k.d = (float*)e->dalloc(KC / 256 * 4);
      e->act.q8k.bsums = (int32_t*)e->dalloc(KC / 16 * 4);
      if (!e->act.q8k.qs || !e->act.q8k.d || !e->act.q8k.bsums) rc = e->fail(MTG_ERR_NOMEM, "device memory");
    }
    if (wt != MTG_TYPE_Q8_0) {
      e->xn = (float*)e->dalloc(RD * 4);
      if (!e->xn) rc = e->fail(MTG_ERR_NOMEM, "device memory");
    }
    if (!e->mel || !e->c1 || !e->x || !e->q || !e->k || !e->v || !e->a || !e->f || !e->out_rows || !e->in_rows ||
        !e->h1 || !e->h2 || !e->ad_out || !e->codes || !e->scales)
      rc = e->fail(MTG_ERR_NOMEM, "device memory");
  }
  if (rc) {
    delete e;
    return rc;
  }
  *out = e;
  return MTG_OK;
}

void mtg_encoder_destroy(mtg_encoder* e) { delete e; }

const char* mtg_encoder_error(const mtg_encoder* e) { return e ? e->error.c_str() : "no encoder"; }

double mtg_encoder_last_ms(const mtg_encoder* e) { return e ? e->last_ms : 0.0; }

int mtg_encoder_encode(mtg_encoder* e, const float* mel, float* out, int32_t* rows_out) {
  if (!e || !mel) return MTG_ERR_INVALID;
  const mtg_encoder_hparams& hp = e->hp;
  const int D = hp.d_model, F = hp.ffn, M = hp.n_mels, NF = hp.n_frames, R = e->rows;
  hipStream_t s = e->stream;
  int rc = e->check(hipMemcpyAsync(e->mel, mel, (size_t)M * NF * 4, hipMemcpyHostToDevice, s), "mel");
  if (rc) return rc;
  if ((rc = e->check(hipEventRecord(e->ev0, s), "event"))) return rc;
  // conv stem
  hipLaunchKernelGGL((k_enc_conv_mma<1, true>), dim3((NF + kConvTile - 1) / kConvTile, D / kConvTile), dim3(256), 0, s,
                     e->conv1_w, e->conv1_b, e->mel, M, NF, D, (const float*)nullptr, e->c1);
  hipLaunchKernelGGL((k_enc_conv_mma<2, false>), dim3((R + kConvTile - 1) / kConvTile, D / kConvTile), dim3(256), 0, s,
                     e->conv2_w, e->conv2_b, e->c1, D, NF, D, e->pos, e->x);
  const dim3 agrid((unsigned)hp.n_heads, (unsigned)((R + kEncRows - 1) / kEncRows));
  for (const mtg_encoder::Layer& L : e->layers) {
    e->ln(e->x, R, L.attn_ln_w, L.attn_ln_b, 1e-5f, true, nullptr);
    e->gemm(PF_EPI_BIAS, L.q_w, D, D, R, e->q, L.q_b);
    e->gemm(PF_EPI_STORE, L.k_w, D, D, R, e->k, nullptr);
    e->gemm(PF_EPI_BIAS, L.v_w, D, D, R, e->v, L.v_b);
    hipLaunchKernelGGL(k_enc_attn_mma, agrid, dim3(256), kEaLds, s, e->q, e->k, e->v, R, D, e->a);
    e->quant(e->a, R, D);
    e->gemm(PF_EPI_BIAS_RESID, L.o_w, D, D, R, e->x, L.o_b);
    e->ln(e->x, R, L.ffn_ln_w, L.ffn_ln_b, 1e-5f, true, nullptr);
    e->gemm(PF_EPI_BIAS_GELU, L.fc1_w, F, D, R, e->f, L.fc1_b);
    e->quant(e->f, R, F);
    e->gemm(PF_EPI_BIAS_RESID, L.fc2_w, D, F, R, e->x, L.fc2_b);
  }
  e->ln(e->x, R, e->ln_post_w, e->ln_post_b, 1e-5f, false, e->out_rows);
  if ((rc = e->check(hipGetLastError(), "encoder launch"))) return rc;
  if ((rc = e->check(hipEventRecord(e->ev1, s), "event"))) return rc;
  if (out && (rc = e->check(hipMemcpyAsync(out, e->out_rows, (size_t)R * D * 4, hipMemcpyDeviceToHost, s), "rows")))
    return rc;
  if ((rc = e->check(hipStreamSynchronize(s), "encode"))) return rc;
  float ms = 0.0f;
  if ((rc = e->check(hipEventElapsedTime(&ms, e->ev0, e->ev1), "timing"))) return rc;
  e->last_ms = ms;
  e->last_rows = R;
  if (rows_out) *rows_out = R;
  return MTG_OK;
}

int mtg_encoder_adapt(mtg_encoder* e, const float* rows, int32_t T, float* out, int32_t* n_out) {
  if (!e || !out || T < 0) return MTG_ERR_INVALID;
  const mtg_encoder_hparams& hp = e->hp;
  const int D = hp.d_model, H = hp.hidden, IN = D * hp.merge, N = T / hp.merge;
  if (T > e->rows || (!rows && T > e->last_rows))
    return e->fail(MTG_ERR_INVALID, "adapt: %d rows, the encoder holds %d", T, rows ? e->rows : e->last_rows);
  if (n_out) *n_out = N;
  if (N <= 0) return MTG_OK;
  hipStream_t s = e->stream;
  int rc = MTG_OK;
  const float* src = e->out_rows;
  if (rows) {
    if ((rc = e->check(hipMemcpyAsync(e->in_rows, rows, (size_t)N * IN * 4, hipMemcpyHostToDevice, s), "rows")))
      return rc;
    src = e->in_rows;
  }
  if ((rc = e->check(hipEventRecord(e->ev0, s), "event"))) return rc;
  // [D * merge, N]: merge consecutive rows per adaptor row (a plain view)
  e->quant(src, N, IN);
  e->gemm(PF_EPI_BIAS_SILU, e->ad_fc1_w, H, IN, N, e->h1, e->ad_fc1_b);
  e->quant(e->h1, N, H);
  e->gemm(PF_EPI_BIAS, e->ad_fc2_w, H, H, N, e->h2, e->ad_fc2_b);
  e->ln(e->h2, N, e->ad_ln_w, e->ad_ln_b, hp.adaptor_eps, false, e->ad_out);
  if ((rc = e->check(hipGetLastError(), "adaptor launch"))) return rc;
  if ((rc = e->check(hipEventRecord(e->ev1, s), "event"))) return rc;
  if ((rc = e->check(hipMemcpyAsync(out, e->ad_out, (size_t)N * H * 4, hipMemcpyDeviceToHost, s), "adaptor rows")))
    return rc;
  if ((rc = e->check(hipStreamSynchronize(s), "adapt"))) return rc;
  float ms = 0.0f;
  if ((rc = e->check(hipEventElapsedTime(&ms, e->ev0, e->ev1), "timing"))) return rc;
  e->last_ms = ms;
  return MTG_OK;
}

}  // extern "C"
