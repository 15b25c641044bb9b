// step_kernel.hip - the whole verify step as one persistent gfx950 kernel.
//
// One workgroup per CU (cooperative launch, so all are co-resident). The step is a
// fixed sequence of phases; between phases every workgroup meets at a grid
// barrier made of per-workgroup arrival words (no atomics, no cache-wide
// writeback/invalidate). Data produced and consumed inside the launch (residual
// stream, qkv, attention partials, o, act, argmax keys) moves through
// device-coherent loads and stores, so no L2 maintenance is needed; weights and
// the KV prefix are read with ordinary cached loads.
//
// Per layer (src/qwen3.cpp:62-218):
//   QKV    every WG: RMSNorm(x)*attn_norm -> q8_0 panel in LDS; one 16-row tile of
//          the fused q|k|v matrix per WG (256 tiles)
//   ATTN   WG = (kv head, split): q/k RMSNorm + NEOX RoPE of its rows in LDS, the
//          new K/V rows appended to the cache by the split holding `past`,
//          split-KV f32-MFMA attention with online softmax -> partial (m, l, O)
//   COMB   (head, row) items: merge the splits -> o
//   OPROJ  q8_0(o) panel; 64 tiles; x += W_o o
//   GATEUP RMSNorm(x)*ffn_norm panel; 192 tile pairs; act = silu(g) * u
//   DOWN   q8_0(act) panel; 64 tiles; x += W_d act
// then the final norm, the tied lm_head with fused argmax keys, and the
// on-device acceptance (src/qwen3_decoder.cpp:129,174-205,
// src/cpu_speculative.cpp:39-50,124-130).
//
// Every barrier wait is bounded: a workgroup that waits too long raises the
// error word and returns, every other workgroup sees it and returns too, and the
// host reports the failure.
#include "device_common.hpp"
#include "step_kernel.hpp"

namespace mtg {

namespace {
using namespace dev;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr unsigned kSpinLimit = 1u << 22;

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
  return v;
}

__device__ __forceinline__ void mark(const StepParams& P, int slot) {
  if (P.timing && blockIdx.x == 0 && threadIdx.x == 0) P.timing[slot] = wall_clock64();
}

// Grid barrier: each workgroup publishes the barrier number in its own arrival
// word once its coherent stores completed; workgroup 0 gathers all words and
// publishes the number in the release word, which the others poll with one
// lane. Returns false when the step was aborted (a bounded wait ran out here or
// elsewhere).
__device__ bool grid_sync(const StepParams& P, uint32_t target, int* s_flag) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");  // this wave's stores are complete
  __syncthreads();
  if (threadIdx.x == 0) st_coh_u32(P.flags + blockIdx.x, target);
  if (blockIdx.x == 0) {
    if (threadIdx.x < 64) {
      unsigned spins = 0;
      int ok = 1;
      for (;;) {
        uint32_t mn = 0xffffffffu;
        for (int i = threadIdx.x; i < (int)gridDim.x; i += 64) mn = min(mn, ld_coh_u32(P.flags + i));
        mn = wave_min_u32(mn);
        if (mn >= target) break;
        if (ld_coh_u32((const uint32_t*)P.err)) { ok = 0; break; }
        if (++spins > kSpinLimit) {
          st_coh_u32((uint32_t*)P.err, 1u);
          ok = 0;
          break;
        }
      }
      if (threadIdx.x == 0) {
        if (ok) st_coh_u32(P.release, target);
        *s_flag = ok;
      }
    }
  } else if (threadIdx.x == 0) {
    unsigned spins = 0;
    int ok = 1;
    while (ld_coh_u32(P.release) < target) {
      if (ld_coh_u32((const uint32_t*)P.err)) { ok = 0; break; }
      if (++spins > kSpinLimit) {
        st_coh_u32((uint32_t*)P.err, 1u);
        ok = 0;
        break;
      }
    }
    *s_flag = ok;
  }
  __syncthreads();
  return *s_flag != 0;
}
#define SYNC_OR_RETURN()                     \
  do {                                       \
    if (!grid_sync(P, ++b, &s_flag)) return; \
    mark(P, (int)(b - epoch));               \
  } while (0)

// ---------------------------------------------------------------- panels ----
// Build the q8_0 activation panel of T rows of src (K columns, K a multiple of
// 1024) in LDS, optionally after RMSNorm * gain (then K == 1024). A wave pass is
// 64 half-block chunks = 1024 consecutive floats of one row: they are fetched
// with coalesced coherent loads into the wave's LDS scratch, then lane l takes
// elements 16l..16l+15 (the two halves of a 32-block sit in lanes l and l^1).
// normed_out (nullable) receives the f32 normalized rows.
__device__ __forceinline__ void load_pass(const float* src, int K, int c0, float* sw, float v[16]) {
  const int lane = threadIdx.x & 63, cpr = K / 16;
  const float* base = src + (size_t)(c0 / cpr) * K + (c0 % cpr) * 16;
#pragma unroll
  for (int e = 0; e < 16; ++e) sw[64 * e + lane] = ld_coh(base + 64 * e + lane);
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const v4f x = *(const v4f*)(sw + 16 * lane + 4 * q);
    v[4 * q] = x[0];
    v[4 * q + 1] = x[1];
    v[4 * q + 2] = x[2];
    v[4 * q + 3] = x[3];
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

template <int G>
__device__ __forceinline__ void quant_store(const float v[16], int t, int kc, int bps, uint8_t* pcodes,
                                            float* pscales) {
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
  const float d = __fdiv_rn(amax, 127.0f);
  const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
  uint32_t packed[4];
#pragma unroll
  for (int w4 = 0; w4 < 4; ++w4) {
    uint32_t u = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int8_t q = (int8_t)rintf(__fmul_rn(v[w4 * 4 + b], id));
      u |= (uint32_t)(uint8_t)q << (8 * b);
    }
    packed[w4] = u;
  }
  const int blk = kc >> 1, half = kc & 1, bp = blk >> 1, par = blk & 1;
  const int cg = t >> 3, j = par * 8 + (t & 7);
  uint8_t* unit = pcodes + (size_t)(cg * bps + bp) * 1024;
  *(uint4*)(unit + (j + 16 * (2 * par + half)) * 16) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  *(uint4*)(unit + (j + 16 * (2 * (1 - par) + half)) * 16) = make_uint4(0u, 0u, 0u, 0u);
  if (half == 0) pscales[(size_t)(cg * bps + bp) * 16 + j] = __half2float(__float2half_rn(d));
}

template <int G>
__device__ void build_panel(const float* src, int K, int T, const float* gain, float eps,
                            uint8_t* pcodes, float* pscales, double* s_part, float* scratch,
                            float* normed_out) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int cpr = K / 16, chunks = T * cpr, bps = K / kPairK;
  const int passes = (chunks + kThreads - 1) / kThreads;
  float* sw = scratch + wave * 1024;
  if (gain) {
    // K == 1024: one wave pass = one row; at most 4 passes (T <= 16)
    float v[4][16];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int c0 = p * kThreads + wave * 64;
      if (p < passes && c0 < chunks) {
        const float* base = src + (size_t)(c0 / cpr) * K + (c0 % cpr) * 16;
#pragma unroll
        for (int e = 0; e < 16; ++e) v[p][e] = ld_coh(base + 64 * e + lane);
      }
    }
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      if (p >= passes) break;
      const int c0 = p * kThreads + wave * 64;
      double s = 0.0;
      if (c0 < chunks) {
        // transpose the coalesced fetch through the wave's LDS scratch
#pragma unroll
        for (int e = 0; e < 16; ++e) sw[64 * e + lane] = v[p][e];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const v4f x4 = *(const v4f*)(sw + 16 * lane + 4 * qq);
          v[p][4 * qq] = x4[0];
          v[p][4 * qq + 1] = x4[1];
          v[p][4 * qq + 2] = x4[2];
          v[p][4 * qq + 3] = x4[3];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
#pragma unroll
        for (int e = 0; e < 16; ++e) s += (double)__fmul_rn(v[p][e], v[p][e]);
      }
      s = wave_sum_d(s);
      if (lane == 0) s_part[p * kWaves + wave] = s;
    }
    __syncthreads();
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int c = p * kThreads + tid;
      if (p >= passes || c >= chunks) break;  // whole waves
      const int t = c / cpr, kc = c % cpr, k0 = kc * 16;
      const float mean = (float)(s_part[p * kWaves + wave] / (double)K);
      const float scale = dev_rms_scale(mean, eps);
      float y[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) y[e] = __fmul_rn(__fmul_rn(v[p][e], scale), gain[k0 + e]);
      if (normed_out)
#pragma unroll
        for (int e = 0; e < 16; ++e) normed_out[(size_t)t * K + k0 + e] = y[e];
      quant_store<G>(y, t, kc, bps, pcodes, pscales);
    }
  } else {
    for (int p0 = 0; p0 < passes; p0 += 4) {
      // fetch up to four passes of this wave with independent coherent loads
      float raw[4][16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c0 = (p0 + q) * kThreads + wave * 64;
        if (p0 + q < passes && c0 < chunks) {
          const float* base = src + (size_t)(c0 / cpr) * K + (c0 % cpr) * 16;
#pragma unroll
          for (int e = 0; e < 16; ++e) raw[q][e] = ld_coh(base + 64 * e + lane);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c0 = (p0 + q) * kThreads + wave * 64;
        if (p0 + q >= passes || c0 >= chunks) break;  // whole waves
#pragma unroll
        for (int e = 0; e < 16; ++e) sw[64 * e + lane] = raw[q][e];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        float v[16];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const v4f x4 = *(const v4f*)(sw + 16 * lane + 4 * qq);
          v[4 * qq] = x4[0];
          v[4 * qq + 1] = x4[1];
          v[4 * qq + 2] = x4[2];
          v[4 * qq + 3] = x4[3];
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        const int c = c0 + lane;
        quant_store<G>(v, c / cpr, c % cpr, bps, pcodes, pscales);
      }
    }
  }
  __syncthreads();
}

// ------------------------------------------------------------------ GEMM ----
enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

// Tiles tile = blockIdx.x, +gridDim.x, ...; the 4 waves split K and meet in
// LDS in wave order; the epilogue writes coherently.
template <int G, int EPI>
__device__ void gemm_phase(const uint8_t* __restrict__ w, const uint8_t* __restrict__ w2,
                           int n_tiles, int bps, const uint8_t* pcodes, const float* pscales,
                           float* red, float* out, int n, int T) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  constexpr int NM = EPI == EPI_SWIGLU ? 2 : 1;
  const int bp0 = (bps * wave) / kWaves, bp1 = (bps * (wave + 1)) / kWaves;
  for (int tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
    float acc[NM][G][4];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int cg = 0; cg < G; ++cg)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[m][cg][r] = 0.0f;
    tile_accumulate<G>(w + (size_t)tile * bps * kUnitBytes, bp0, bp1, pcodes, pscales, bps, acc[0]);
    if (EPI == EPI_SWIGLU)
      tile_accumulate<G>(w2 + (size_t)tile * bps * kUnitBytes, bp0, bp1, pcodes, pscales, bps,
                         acc[NM - 1]);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int cg = 0; cg < G; ++cg)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((wave * NM + m) * G * 4 + cg * 4 + r) * 64 + lane] = acc[m][cg][r];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int cg = 0; cg < G; ++cg)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float s = red[((0 * NM + m) * G * 4 + cg * 4 + r) * 64 + lane];
            for (int wv = 1; wv < kWaves; ++wv) s = __fadd_rn(s, red[((wv * NM + m) * G * 4 + cg * 4 + r) * 64 + lane]);
            acc[m][cg][r] = __fadd_rn(s, __shfl_xor(s, 8, 64));
          }
      if ((lane & 15) < 8) {
#pragma unroll
        for (int cg = 0; cg < G; ++cg) {
          const int t = cg * 8 + (lane & 7);
          if (t < T) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int row = tile * 16 + 4 * (lane >> 4) + r;
              float* dst = out + (size_t)t * n + row;
              if (EPI == EPI_STORE) {
                st_coh(dst, acc[0][cg][r]);
              } else if (EPI == EPI_RESID) {
                st_coh(dst, __fadd_rn(ld_coh(dst), acc[0][cg][r]));
              } else {
                st_coh(dst, dev_swiglu(acc[0][cg][r], acc[NM - 1][cg][r]));
              }
            }
          }
        }
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------- attention ----
// q/k RMSNorm (head_dim 128) + NEOX RoPE of one row, one wave, lane i owns the
// pair (i, i+64); returns the rotated pair.
__device__ __forceinline__ void norm_rope_pair(float& x0, float& x1, const float* g, float eps,
                                               const float* rope_row, int i) {
  double s = (double)__fmul_rn(x0, x0) + (double)__fmul_rn(x1, x1);
  s = wave_sum_d(s);
  const float mean = (float)(s / (double)kHeadDim);
  const float scale = dev_rms_scale(mean, eps);
  const float y0 = __fmul_rn(__fmul_rn(x0, scale), g[i]);
  const float y1 = __fmul_rn(__fmul_rn(x1, scale), g[i + 64]);
  const float c = rope_row[2 * i], sn = rope_row[2 * i + 1];
  x0 = __fsub_rn(__fmul_rn(y0, c), __fmul_rn(y1, sn));
  x1 = __fadd_rn(__fmul_rn(y0, sn), __fmul_rn(y1, c));
}

// Items (kv head g, chunk of 64 keys), grid-stride. Each workgroup stages the
// roped q of heads 2g, 2g+1 and, when its chunk reaches the new keys, the new
// K/V rows (q/k RMSNorm + NEOX RoPE from qkv); the workgroup whose chunk holds
// position `past` also appends them to the cache for later steps.
__device__ void attn_phase(const StepParams& P, const LayerDev& Ly, int T, int past, uint8_t* lds) {
  const int NKV = P.NKV, NH = P.NH;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int NQKV = (NH + 2 * NKV) * kHeadDim;
  const bool f16kv = P.kv_f16 != 0;
  const int kvlen = past + T, nch = (kvlen + kChunk - 1) / kChunk;
  float* q_lds = (float*)lds;                  // [kMaxCols][128]
  float* knew = q_lds + kMaxCols * kHeadDim;   // [16][128]
  float* vnew = knew + kMaxRows * kHeadDim;    // [16][128]
  float* vbuf = vnew + kMaxRows * kHeadDim;    // [64][128]
  float* sp = vbuf + kChunk * kHeadDim;        // [kMaxCols][64]
  const int ncol = 2 * T;
  int staged_g = -1;
  for (int item = blockIdx.x; item < NKV * nch; item += gridDim.x) {
    const int g = item / nch, chunk = item % nch, key0 = chunk * kChunk;
    const bool has_new = key0 + kChunk > past;
    const bool appender = key0 <= past && past < key0 + kChunk;
    if (g != staged_g || has_new) {
      // q rows (col = hl*T + t) and, if needed, the new k / v rows
      const int nrows = ncol + (has_new ? 2 * T : 0);
      for (int r = wave; r < nrows; r += kWaves) {
        int kind, t, col;
        if (r < ncol) {
          kind = 0;
          t = r % T;
          col = (2 * g + r / T) * kHeadDim;
        } else if (r < ncol + T) {
          kind = 1;
          t = r - ncol;
          col = (NH + g) * kHeadDim;
        } else {
          kind = 2;
          t = r - ncol - T;
          col = (NH + NKV + g) * kHeadDim;
        }
        const float* src = P.qkv + (size_t)t * NQKV + col;
        float x0 = ld_coh(src + lane), x1 = ld_coh(src + lane + 64);
        if (kind < 2)
          norm_rope_pair(x0, x1, kind == 0 ? Ly.q_norm : Ly.k_norm, P.eps,
                         P.rope + (size_t)(past + t) * kHeadDim, lane);
        if (kind == 0) {
          float* q = q_lds + r * kHeadDim;
          q[lane] = f16kv ? f16_round(x0) : x0;
          q[lane + 64] = f16kv ? f16_round(x1) : x1;
        } else {
          if (appender) {
            const size_t off = ((size_t)g * P.max_seq + past + t) * kHeadDim;
            uint8_t* cache = kind == 1 ? Ly.kc : Ly.vc;
            if (f16kv) {
              ((__half*)cache)[off + lane] = __float2half_rn(x0);
              ((__half*)cache)[off + lane + 64] = __float2half_rn(x1);
            } else {
              ((float*)cache)[off + lane] = x0;
              ((float*)cache)[off + lane + 64] = x1;
            }
          }
          float* dst = (kind == 1 ? knew : vnew) + t * kHeadDim;
          dst[lane] = f16kv ? f16_round(x0) : x0;
          dst[lane + 64] = f16kv ? f16_round(x1) : x1;
        }
      }
      __syncthreads();
      staged_g = has_new ? -1 : g;
    }
    AttnSrc a;
    a.kc = Ly.kc;
    a.vc = Ly.vc;
    a.f16 = P.kv_f16;
    a.head_base = (size_t)g * P.max_seq * kHeadDim;
    a.knew = knew;
    a.vnew = vnew;
    a.new_from = has_new ? past : kvlen;
    const size_t pi = (size_t)g * P.max_chunks + chunk;
    attn_chunk<true>(a, q_lds, ncol, T, past, kvlen, key0, __fdiv_rn(1.0f, dev_sqrtf((float)kHeadDim)), vbuf, sp,
                     P.part_ml + pi * kMaxCols * 2, P.part_o + pi * kMaxCols * kHeadDim);
  }
}

// (head, row) items: merge the chunks into o[t][head*128 + d]. Each half
// workgroup takes one item; the partials of up to 32 chunks are fetched with
// independent coherent loads before the canonical merge runs over them.
__device__ void combine_phase(const StepParams& P, int T, int past, float* s_ml) {
  const int items = P.NH * T, nch = (past + T + kChunk - 1) / kChunk;
  const int d = threadIdx.x & 127, half = threadIdx.x >> 7;
  float* ml = s_ml + half * 64;  // [32 chunks][2]
  for (int base = 2 * blockIdx.x; base < items; base += 2 * gridDim.x) {
    const int item = base + half;
    const bool active = item < items;
    const int hq = active ? item / T : 0, t = active ? item % T : 0;
    const int g = hq / 2, col = (hq & 1) * T + t;
    const float* pml = P.part_ml + (size_t)g * P.max_chunks * kMaxCols * 2 + col * 2;
    const float* po = P.part_o + (size_t)g * P.max_chunks * kMaxCols * kHeadDim + col * kHeadDim + d;
    const size_t sml = (size_t)kMaxCols * 2, so = (size_t)kMaxCols * kHeadDim;
    // pass 1: the maximum over all chunks
    float M = -INFINITY;
    for (int c0 = 0; c0 < nch; c0 += 64) {
      const int c = c0 + (d & 63);
      float m = -INFINITY;
      if (active && d < 64 && c < nch) m = ld_coh(pml + c * sml);
      M = fmaxf(M, m);
    }
    // M is reduced over the half workgroup's first wave-half... use LDS
    __shared__ float s_max[2][2];
    M = wave_max_f(M);
    if ((threadIdx.x & 63) == 0 && ((threadIdx.x >> 6) & 1) == 0) s_max[half][0] = M;
    __syncthreads();
    M = s_max[half][0];
    float L = 0.0f, O = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += 32) {
      const int nb = min(32, nch - c0);
      if (active && d < 2 * nb) ml[d] = ld_coh(pml + (c0 + (d >> 1)) * sml + (d & 1));
      float ov[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) ov[i] = (active && i < nb) ? ld_coh(po + (c0 + i) * so) : 0.0f;
      __syncthreads();
      if (active) {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          if (i >= nb) break;
          const float m = ml[2 * i];
          if (m == -INFINITY) continue;
          const float f = dev_expf(__fsub_rn(m, M));
          L = fmaf(ml[2 * i + 1], f, L);
          O = fmaf(ov[i], f, O);
        }
      }
      __syncthreads();
    }
    if (active) st_coh(P.o + (size_t)t * P.NH * kHeadDim + hq * kHeadDim + d, __fdiv_rn(O, L));
  }
}

// ------------------------------------------------------------- lm_head -----
template <int G>
__device__ void lm_head_phase(const StepParams& P, const StepDesc* desc, int T, const uint8_t* pcodes,
                              const float* pscales, uint64_t* s_best) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int V = P.V, bps = P.H / kPairK, n_tiles = V / 16;
  const bool pen = desc->penalty > 1.0f;
  const float penalty = desc->penalty;
  const int words = (V + 31) / 32;
  const bool write_logits = desc->write_logits != 0;
  uint64_t best[G];
#pragma unroll
  for (int cg = 0; cg < G; ++cg) best[cg] = 0;
  const int nwaves = gridDim.x * kWaves;
  for (int tile = blockIdx.x * kWaves + wave; tile < n_tiles; tile += nwaves) {
    float acc[G][4];
    tile_accumulate_canonical<G>(P.embd + (size_t)tile * bps * kUnitBytes, bps, pcodes, pscales, acc);
    if ((lane & 15) < 8) {
#pragma unroll
      for (int cg = 0; cg < G; ++cg) {
        const int t = cg * 8 + (lane & 7);
        if (t < T) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = tile * 16 + 4 * (lane >> 4) + r;
            float v = acc[cg][r];
            if (write_logits) P.logits[(size_t)t * V + row] = v;
            if (pen && ((ld_coh_u32(P.bitmap + (size_t)t * words + (row >> 5)) >> (row & 31)) & 1u))
              v = v > 0.0f ? __fdiv_rn(v, penalty) : __fmul_rn(v, penalty);
            const uint64_t key = argmax_key(v, row);
            best[cg] = key > best[cg] ? key : best[cg];
          }
        }
      }
    }
  }
#pragma unroll
  for (int cg = 0; cg < G; ++cg) {
    uint64_t b = best[cg], o;
    o = shfl_xor_u64(b, 16);
    b = o > b ? o : b;
    o = shfl_xor_u64(b, 32);
    b = o > b ? o : b;
    o = shfl_xor_u64(b, 8);
    b = o > b ? o : b;
    best[cg] = b;
  }
  if (lane < 8)
#pragma unroll
    for (int cg = 0; cg < G; ++cg) s_best[wave * kMaxRows + cg * 8 + lane] = best[cg];
  __syncthreads();
  if (threadIdx.x < G * 8) {
    uint64_t b = s_best[threadIdx.x];
    for (int wv = 1; wv < kWaves; ++wv) b = s_best[wv * kMaxRows + threadIdx.x] > b ? s_best[wv * kMaxRows + threadIdx.x] : b;
    st_coh_u64(P.part_keys + (size_t)blockIdx.x * kMaxRows + threadIdx.x, b);
  }
  __syncthreads();
}

__device__ void accept_phase(const StepParams& P, const StepDesc* desc, int T, uint64_t* s_red,
                             int32_t* s_choice) {
  for (int t = 0; t < T; ++t) {
    uint64_t b = 0;
    for (int i = threadIdx.x; i < (int)gridDim.x; i += kThreads) {
      const uint64_t k = ld_coh_u64(P.part_keys + (size_t)i * kMaxRows + t);
      b = k > b ? k : b;
    }
    s_red[threadIdx.x] = b;
    __syncthreads();
    for (int o = kThreads / 2; o > 0; o >>= 1) {
      if ((int)threadIdx.x < o && s_red[threadIdx.x + o] > s_red[threadIdx.x]) s_red[threadIdx.x] = s_red[threadIdx.x + o];
      __syncthreads();
    }
    if (threadIdx.x == 0) s_choice[t] = (int32_t)(0xffffffffu - (uint32_t)(s_red[0] & 0xffffffffu));
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    int m = 0;
    while (m + 1 < T && desc->tokens[m + 1] == s_choice[m]) ++m;
    for (int t = 0; t < kMaxRows; ++t) P.result->choice[t] = t < T ? s_choice[t] : -1;
    P.result->n_match = m;
  }
}

// ---------------------------------------------------------------- kernel ----
template <int G>
__global__ void __launch_bounds__(kThreads, 1)
k_step(const StepParams* __restrict__ Pp, const StepDesc* __restrict__ desc, uint32_t epoch,
       int mode) {
  const StepParams& P = *Pp;
  extern __shared__ v4i lds_v4[];
  uint8_t* lds = (uint8_t*)lds_v4;
  const int T = desc->T, past = desc->past;
  const int H = P.H, QN = P.NH * kHeadDim, KN = P.NKV * kHeadDim, F = P.F;
  const int bps_max = P.bps_max;
  uint8_t* pcodes = lds;
  float* pscales = (float*)(lds + (size_t)G * bps_max * 1024);
  float* red = (float*)(lds + (size_t)G * bps_max * (1024 + 64));
  float* scratch = red;  // panel builds and GEMM reductions never overlap in time
  __shared__ double s_part[64];
  __shared__ int s_flag;
  __shared__ uint64_t s_best[kWaves * kMaxRows];
  __shared__ uint64_t s_red[kThreads];
  __shared__ int32_t s_choice[kMaxRows];
  uint32_t b = epoch;
  mark(P, 0);

  // embeddings (and the penalty bitmap)
  if ((int)blockIdx.x < T) {
    const int t = blockIdx.x;
    float* xr = P.x + (size_t)t * H;
    if (desc->use_embeds) {
      for (int k = threadIdx.x; k < H; k += kThreads) st_coh(xr + k, P.embeds[(size_t)t * H + k]);
    } else {
      const int n = desc->tokens[t], bps = H / kPairK, tile = n >> 4, r = n & 15;
      for (int k = threadIdx.x; k < H; k += kThreads) {
        const int bk = k >> 5, bp = bk >> 1, par = bk & 1, half = (k >> 4) & 1;
        const uint8_t* unit = P.embd + ((size_t)tile * bps + bp) * kUnitBytes;
        const int8_t q = (int8_t)unit[(r + 16 * (2 * par + half)) * 16 + (k & 15)];
        const float d = half_bits_to_float(((const uint16_t*)(unit + 1024))[par * 16 + r]);
        st_coh(xr + k, d * (float)q);
      }
    }
    if (mode == kStepVerify && desc->penalty > 1.0f) {
      const int words = (P.V + 31) / 32;
      uint32_t* row = P.bitmap + (size_t)t * words;
      for (int i = threadIdx.x; i < words; i += kThreads) st_coh_u32(row + i, 0u);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __syncthreads();
      const int end = desc->pen_base + t + 1, begin = max(0, end - kPenaltyWindow);
      for (int i = begin + (int)threadIdx.x; i < end; i += kThreads) {
        const int id = desc->pen_ids[i];
        if (id >= 0 && id < P.V) atomicOr(row + (id >> 5), 1u << (id & 31));
      }
    }
  }
  SYNC_OR_RETURN();

  for (int l = 0; l < P.L; ++l) {
    const LayerDev& Ly = P.layers[l];
    // QKV
    if ((int)blockIdx.x < (QN + 2 * KN) / 16) {
      build_panel<G>(P.x, H, T, Ly.attn_norm, P.eps, pcodes, pscales, s_part, scratch, nullptr);
      gemm_phase<G, EPI_STORE>(Ly.wqkv, nullptr, (QN + 2 * KN) / 16, H / kPairK, pcodes, pscales, red,
                               P.qkv, QN + 2 * KN, T);
    }
    SYNC_OR_RETURN();
    attn_phase(P, Ly, T, past, lds);
    SYNC_OR_RETURN();
    combine_phase(P, T, past, (float*)lds);
    SYNC_OR_RETURN();
    if ((int)blockIdx.x < H / 16) {
      build_panel<G>(P.o, QN, T, nullptr, 0.0f, pcodes, pscales, s_part, scratch, nullptr);
      gemm_phase<G, EPI_RESID>(Ly.wo, nullptr, H / 16, QN / kPairK, pcodes, pscales, red, P.x, H, T);
    }
    SYNC_OR_RETURN();
    if ((int)blockIdx.x < F / 16) {
      build_panel<G>(P.x, H, T, Ly.ffn_norm, P.eps, pcodes, pscales, s_part, scratch, nullptr);
      gemm_phase<G, EPI_SWIGLU>(Ly.wg, Ly.wu, F / 16, H / kPairK, pcodes, pscales, red, P.act, F, T);
    }
    SYNC_OR_RETURN();
    if ((int)blockIdx.x < H / 16) {
      build_panel<G>(P.act, F, T, nullptr, 0.0f, pcodes, pscales, s_part, scratch, nullptr);
      gemm_phase<G, EPI_RESID>(Ly.wd, nullptr, H / 16, F / kPairK, pcodes, pscales, red, P.x, H, T);
    }
    SYNC_OR_RETURN();
  }
  // final RMSNorm * output_norm (workgroup 0 also returns the f32 rows)
  build_panel<G>(P.x, H, T, P.out_norm, P.eps, pcodes, pscales, s_part, scratch,
                 blockIdx.x == 0 ? P.hid : nullptr);
  if (mode != kStepVerify) return;
  lm_head_phase<G>(P, desc, T, pcodes, pscales, s_best);
  SYNC_OR_RETURN();
  if (blockIdx.x == 0) accept_phase(P, desc, T, s_red, s_choice);
  mark(P, (int)(b - epoch) + 1);
}

}  // namespace

int step_barriers(int n_layers, int mode) { return 1 + 6 * n_layers + (mode == kStepVerify ? 1 : 0); }

size_t step_lds_bytes(int G, int bps_max) {
  const size_t panel = (size_t)G * bps_max * (1024 + 64);
  size_t red = (size_t)kWaves * 2 * G * 4 * 64 * 4;
  if (red < (size_t)kWaves * 1024 * 4) red = (size_t)kWaves * 1024 * 4;  // panel-build scratch
  const size_t attn = ((size_t)kMaxCols * kHeadDim + 2 * kMaxRows * kHeadDim + kChunk * kHeadDim +
                       (size_t)kMaxCols * kChunk) * 4;
  return (panel > attn ? panel : attn) + red;
}

hipError_t launch_step(hipStream_t s, int G, int nwg, const StepParams* P, const StepDesc* desc,
                       uint32_t epoch, int mode, int bps_max) {
  const size_t lds = step_lds_bytes(G, bps_max);
  void* args[] = {(void*)&P, (void*)&desc, (void*)&epoch, (void*)&mode};
  if (G == 1)
    return hipLaunchCooperativeKernel((const void*)k_step<1>, dim3(nwg), dim3(kThreads), args, lds, s);
  return hipLaunchCooperativeKernel((const void*)k_step<2>, dim3(nwg), dim3(kThreads), args, lds, s);
}

hipError_t prepare_step_kernels(int bps_max) {
  hipError_t e = hipFuncSetAttribute((const void*)k_step<1>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)step_lds_bytes(1, bps_max));
  if (e != hipSuccess) return e;
  return hipFuncSetAttribute((const void*)k_step<2>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)step_lds_bytes(2, bps_max));
}

}  // namespace mtg
