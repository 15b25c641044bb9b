// encoder.hip - the Whisper audio encoder and the audio adaptor on the device
// (reference WhisperEncoder::encode, src/whisper_encoder.cpp:103-209, and
// AudioAdaptor::apply, src/audio_adaptor.cpp:38-97).
//
//   conv stem  k_enc_conv: conv1d (kernel 3, pad 1) as one fma chain per output
//              over (input channel, tap), + bias, GELU (erf); conv2 (stride 2)
//              also adds the positional embedding and writes [rows][d]
//   layers     k_enc_ln: LayerNorm (mean and variance as double sums over 64
//              lane partials, butterfly) -> q8_0 codes for the next GEMM;
//              q / k / v / out / fc1 / fc2 on the block GEMM of the prefill
//              (q8_0 weights x q8_0 activations, int8 MFMA) with bias, GELU or
//              residual epilogues; k_enc_attn: bidirectional attention of 16
//              query rows of one head per workgroup over all rows in 64-key
//              chunks (two passes: chunk maxima, then exp / sums / context
//              merged in chunk order)
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
constexpr int kEncRows = 64;    // query rows per attention workgroup
constexpr int kEncMaxChunks = 32;  // rows <= 2048
constexpr int kConvTile = 64;   // outputs per conv workgroup: 64 rows x 64 channels
constexpr int kConvIcb = 16;    // input channels staged per step

// ------------------------------------------------------------- conv stem ---
// out = gelu(conv(x) + b) (+ pos): x [IC][L] (frames fastest), w [OC][IC][3].
// Thread (tx, ty): rows t0 + tx + 16 i, channels o0 + ty + 16 j (i, j < 4).
// TRANS: out [OC][OL] (conv2's input layout), else out [OL][OC].
template <int STRIDE, bool TRANS>
__global__ void __launch_bounds__(256)
k_enc_conv(const float* __restrict__ w, const float* __restrict__ b, const float* __restrict__ x, int IC, int L,
           int OC, const float* __restrict__ pos, float* __restrict__ out) {
  constexpr int XW = kConvTile * STRIDE + 2;
  __shared__ float xs[kConvIcb][XW];
  __shared__ float ws[kConvTile][kConvIcb * 3 + 1];
  const int OL = (L - 1) / STRIDE + 1;
  const int t0 = blockIdx.x * kConvTile, o0 = blockIdx.y * kConvTile;
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  const int p0 = t0 * STRIDE - 1;  // the input position of tap 0 of row t0
  for (int ic0 = 0; ic0 < IC; ic0 += kConvIcb) {
    for (int i = tid; i < kConvIcb * XW; i += 256) {
      const int c = i / XW, q = i % XW, p = p0 + q;
      xs[c][q] = (p >= 0 && p < L) ? x[(size_t)(ic0 + c) * L + p] : 0.0f;
    }
    for (int i = tid; i < kConvTile * kConvIcb * 3; i += 256) {
      const int o = i / (kConvIcb * 3), e = i % (kConvIcb * 3);
      ws[o][e] = w[((size_t)(o0 + o) * IC + ic0) * 3 + e];
    }
    __syncthreads();
    for (int c = 0; c < kConvIcb; ++c)
#pragma unroll
      for (int k = 0; k < 3; ++k) {
        float xv[4], wv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = xs[c][(tx + 16 * i) * STRIDE + k];
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[j] = ws[ty + 16 * j][c * 3 + k];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(wv[j], xv[i], acc[i][j]);
      }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = t0 + tx + 16 * i;
    if (t >= OL) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int o = o0 + ty + 16 * j;
      float y = dev_gelu_erf(__fadd_rn(acc[i][j], b[o]));
      if (pos) y = __fadd_rn(y, pos[(size_t)t * OC + o]);
      if (TRANS) out[(size_t)o * OL + t] = y;
      else out[(size_t)t * OC + o] = y;
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
// Rows r0 .. r0 + 63 of head blockIdx.x over all T rows (no mask), q / k / v /
// out [T][W] (W = heads * 64). Thread (tr, tk) = (tid / 16, tid % 16) holds a
// 4 x 4 register tile: the scores of rows 4 tr + i and keys 4 tk + j of a chunk
// (fma chains over head_dim from 16-byte LDS reads), then the context of rows
// 4 tr + i and elements 4 tk + e (fma chains over the chunk's keys). Pass 1
// takes every chunk's row maxima; pass 2 recomputes the scores, p = exp(w - m_c),
// l_c (fold-in-half over the 64 keys, the butterfly's order), O_c, and merges
// the chunks in order.
constexpr int kAS = kEncHd + 4;  // LDS row stride, floats (16-byte rows)
__global__ void __launch_bounds__(256)
k_enc_attn(const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v, int T, int W,
           float* __restrict__ out) {
  __shared__ __align__(16) float qs[kEncRows][kAS];
  __shared__ __align__(16) float kv[64][kAS];  // the chunk's K, then its V
  __shared__ __align__(16) float ps[kEncRows][kAS];
  __shared__ float cm[kEncRows][kEncMaxChunks + 1];
  __shared__ float cl[kEncRows];
  const int h = blockIdx.x, r0 = blockIdx.y * kEncRows;
  const int tid = threadIdx.x, tr = tid >> 4, tk = tid & 15;
  const int nch = (T + 63) / 64;
  const float scale = __fdiv_rn(1.0f, dev_sqrtf((float)kEncHd));
  const v4f zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
  // 64 rows x 64 floats of src from row0 (zeros past T): load4 issues the four
  // 16-byte loads of this thread (rows past T read row T - 1 and are zeroed after
  // the load, so no branch splits them), store4 writes them to dst. A chunk's
  // loads go out one chunk ahead and land during the previous chunk's arithmetic.
  auto load4 = [&](const float* src, int row0, v4f (&r)[4]) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int i = tid + 256 * x, rr = i >> 4, d4 = i & 15;
      r[x] = *(const v4f*)(src + (size_t)min(row0 + rr, T - 1) * W + h * kEncHd + 4 * d4);
      if (row0 + rr >= T) r[x] = zero4;
    }
  };
  auto store4 = [&](float (*dst)[kAS], const v4f (&r)[4]) {
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int i = tid + 256 * x, rr = i >> 4, d4 = i & 15;
      *(v4f*)&dst[rr][4 * d4] = r[x];
    }
  };
  auto scores = [&](int key0, float (&w)[4][4]) {
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int d0 = 0; d0 < kEncHd; d0 += 4) {
      v4f qv[4], kx[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) qv[i] = *(const v4f*)&qs[4 * tr + i][d0];
#pragma unroll
      for (int j = 0; j < 4; ++j) kx[j] = *(const v4f*)&kv[4 * tk + j][d0];
#pragma unroll
      for (int dd = 0; dd < 4; ++dd)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(qv[i][dd], kx[j][dd], acc[i][j]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) w[i][j] = key0 + 4 * tk + j < T ? __fmul_rn(acc[i][j], scale) : -INFINITY;
  };
  v4f kr[4], vr[4];
  load4(q, r0, vr);
  load4(k, 0, kr);
  store4(qs, vr);
  // pass 1: chunk maxima per row (over the 16 threads of a row group)
  for (int c = 0; c < nch; ++c) {
    __syncthreads();
    store4(kv, kr);
    __syncthreads();
    if (c + 1 < nch) load4(k, 64 * (c + 1), kr);
    float w[4][4];
    scores(64 * c, w);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float m = fmaxf(fmaxf(w[i][0], w[i][1]), fmaxf(w[i][2], w[i][3]));
#pragma unroll
      for (int o = 8; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
      if (tk == 0) cm[4 * tr + i][c] = m;
    }
  }
  __syncthreads();
  float M[4], L[4], O[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    M[i] = -INFINITY;
    for (int c = 0; c < nch; ++c) M[i] = fmaxf(M[i], cm[4 * tr + i][c]);
    L[i] = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) O[i][e] = 0.0f;
  }
  // pass 2
  load4(k, 0, kr);
  load4(v, 0, vr);
  for (int c = 0; c < nch; ++c) {
    __syncthreads();
    store4(kv, kr);
    __syncthreads();
    if (c + 1 < nch) load4(k, 64 * (c + 1), kr);
    float w[4][4];
    scores(64 * c, w);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float mc = cm[4 * tr + i][c];
      v4f p4;
#pragma unroll
      for (int j = 0; j < 4; ++j) p4[j] = w[i][j] == -INFINITY ? 0.0f : dev_expf(__fsub_rn(w[i][j], mc));
      *(v4f*)&ps[4 * tr + i][4 * tk] = p4;
    }
    __syncthreads();  // K consumed, p complete
    store4(kv, vr);
    if (c + 1 < nch) load4(v, 64 * (c + 1), vr);
    if (tid < kEncRows) {
      float t[64];
#pragma unroll
      for (int j = 0; j < 64; j += 4) {
        const v4f p4 = *(const v4f*)&ps[tid][j];
        t[j] = p4[0];
        t[j + 1] = p4[1];
        t[j + 2] = p4[2];
        t[j + 3] = p4[3];
      }
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1)
#pragma unroll
        for (int j = 0; j < o; ++j) t[j] = __fadd_rn(t[j], t[j + o]);
      cl[tid] = t[0];
    }
    __syncthreads();  // V staged, l_c ready
    float oc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) oc[i][e] = 0.0f;
    for (int j0 = 0; j0 < 64; j0 += 4) {
      v4f pv[4], vv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) pv[i] = *(const v4f*)&ps[4 * tr + i][j0];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) vv[jj] = *(const v4f*)&kv[j0 + jj][4 * tk];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int e = 0; e < 4; ++e) oc[i][e] = fmaf(pv[i][jj], vv[jj][e], oc[i][e]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = dev_expf(__fsub_rn(cm[4 * tr + i][c], M[i]));
      L[i] = fmaf(cl[4 * tr + i], f, L[i]);
#pragma unroll
      for (int e = 0; e < 4; ++e) O[i][e] = fmaf(oc[i][e], f, O[i][e]);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = r0 + 4 * tr + i;
    if (row >= T) continue;
    v4f o4;
#pragma unroll
    for (int e = 0; e < 4; ++e) o4[e] = __fdiv_rn(O[i][e], L[i]);
    *(v4f*)(out + (size_t)row * W + h * kEncHd + 4 * tk) = o4;
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
  void quant(const float* src, int S, int K) { launch_pf_quant(stream, src, S, K, codes, scales); }
  void gemm(int epi, const uint8_t* w, int N, int K, int S, float* out, const float* bias) {
    launch_pf_gemm(stream, epi, w, nullptr, N, K, codes, scales, S, out, bias);
  }
  void ln(const float* src, int S, const float* w, const float* b, float eps, bool q8, float* yout) {
    hipLaunchKernelGGL(k_enc_ln, dim3((S + 3) / 4), dim3(256), 0, stream, src, S, w, b, eps, q8 ? codes : nullptr,
                       q8 ? scales : nullptr, yout);
  }
};

extern "C" {

int mtg_encoder_create(const mtg_encoder_desc* d, mtg_encoder** out) {
  if (!d || !out) return MTG_ERR_INVALID;
  *out = nullptr;
  const mtg_encoder_hparams& hp = d->hp;
  if (d->weight_type != MTG_TYPE_Q8_0 || hp.d_model != 1024 || hp.hidden != 1024 || hp.n_heads <= 0 ||
      hp.d_model / hp.n_heads != kEncHd || hp.d_model % hp.n_heads || hp.ffn % 64 || hp.n_mels % kConvIcb ||
      hp.n_mels <= 0 || hp.merge <= 0 || hp.n_layers < 0 || hp.n_frames < 2 ||
      (hp.n_frames - 1) / 2 + 1 > 64 * kEncMaxChunks)
    return MTG_ERR_UNSUPPORTED;
  if (!d->layers && hp.n_layers > 0) return MTG_ERR_INVALID;
  mtg_encoder* e = new (std::nothrow) mtg_encoder();
  if (!e) return MTG_ERR_NOMEM;
  e->hp = hp;
  const int D = hp.d_model, F = hp.ffn, M = hp.n_mels, NF = hp.n_frames, R = (NF - 1) / 2 + 1, H = hp.hidden,
            IN = D * hp.merge;
  e->rows = R;
  int rc = e->check(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking), "stream");
  if (!rc) rc = e->check(hipEventCreate(&e->ev0), "event");
  if (!rc) rc = e->check(hipEventCreate(&e->ev1), "event");
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
    L.q_w = e->up_q8(s.q_w, D, D, staging, rc);
    L.k_w = e->up_q8(s.k_w, D, D, staging, rc);
    L.v_w = e->up_q8(s.v_w, D, D, staging, rc);
    L.o_w = e->up_q8(s.o_w, D, D, staging, rc);
    L.q_b = e->up_f(s.q_b, D, rc);
    L.v_b = e->up_f(s.v_b, D, rc);
    L.o_b = e->up_f(s.o_b, D, rc);
    L.ffn_ln_w = e->up_f(s.ffn_ln_w, D, rc);
    L.ffn_ln_b = e->up_f(s.ffn_ln_b, D, rc);
    L.fc1_w = e->up_q8(s.fc1_w, F, D, staging, rc);
    L.fc1_b = e->up_f(s.fc1_b, F, rc);
    L.fc2_w = e->up_q8(s.fc2_w, D, F, staging, rc);
    L.fc2_b = e->up_f(s.fc2_b, D, rc);
    e->layers.push_back(L);
  }
  e->ad_fc1_w = e->up_q8(d->ad_fc1_w, H, IN, staging, rc);
  e->ad_fc1_b = e->up_f(d->ad_fc1_b, H, rc);
  e->ad_fc2_w = e->up_q8(d->ad_fc2_w, H, H, staging, rc);
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
  hipLaunchKernelGGL((k_enc_conv<1, true>), dim3((NF + kConvTile - 1) / kConvTile, D / kConvTile), dim3(256), 0, s,
                     e->conv1_w, e->conv1_b, e->mel, M, NF, D, (const float*)nullptr, e->c1);
  hipLaunchKernelGGL((k_enc_conv<2, false>), dim3((R + kConvTile - 1) / kConvTile, D / kConvTile), dim3(256), 0, s,
                     e->conv2_w, e->conv2_b, e->c1, D, NF, D, e->pos, e->x);
  const dim3 agrid((unsigned)hp.n_heads, (unsigned)((R + kEncRows - 1) / kEncRows));
  for (const mtg_encoder::Layer& L : e->layers) {
    e->ln(e->x, R, L.attn_ln_w, L.attn_ln_b, 1e-5f, true, nullptr);
    e->gemm(PF_EPI_BIAS, L.q_w, D, D, R, e->q, L.q_b);
    e->gemm(PF_EPI_STORE, L.k_w, D, D, R, e->k, nullptr);
    e->gemm(PF_EPI_BIAS, L.v_w, D, D, R, e->v, L.v_b);
    hipLaunchKernelGGL(k_enc_attn, agrid, dim3(256), 0, s, e->q, e->k, e->v, R, D, e->a);
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
