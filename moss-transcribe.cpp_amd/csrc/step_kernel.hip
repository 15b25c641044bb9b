// step_kernel.hip - the Qwen3-0.6B verify step as one persistent dataflow kernel (gfx950).
//
// One 256-thread workgroup per CU (exactly 256 workgroups, all resident together).
// Every workgroup owns fixed roles per layer:
//   QKV   tile w of the fused q|k|v matrix (256 tiles of 16 rows, K = 1024)
//   ATTN  items (kv head, 64-key chunk), numbered head-major; item i runs on
//         workgroup (i + 64) mod 256, so the 192 workgroups without o/down
//         tiles take the first items
//   MERGE (q head, row) items on workgroups 160..255; the merged rows leave as
//         q8_0 codes + scales (the o-proj's activation quantization)
//   OPROJ tile w < 64 (K = 2048) and DOWN tile w < 64 (K = 3072)
//   GATEUP rows 32j..32j+31 of gate and up on workgroup 64 + j (j < 96); the
//         SwiGLU rows leave as q8_0 blocks (the down-proj's quantization)
// (src/qwen3.cpp:62-218.) Instead of grid barriers, each workgroup publishes a
// monotone progress word: after its work in a phase it announces the last phase
// before its next work as done, so a phase it takes no part in never delays
// anyone. A phase waits until every progress word has reached the phase before
// it; this orders every reuse of the exchange buffers (x, q|k|v, attention
// partials, o, act) globally.
//
// Latency hiding: after publishing, a workgroup issues the loads of the weights
// (and, for attention, of its 64-key K and V slices) of its next phase into
// registers, so the HBM stream of a phase overlaps the wait for its inputs.
// Weights are re-tiled q8_0 MFMA panels read with non-temporal 16-byte loads;
// exchange buffers move through 16-byte device-coherent (sc1) buffer accesses.
//
// Arithmetic follows the canonical order shared with the oracle: the q8_0 GEMM
// in 4 K-slices (one per wave) with exact int8 MFMA block dots; attention scores
// and P.V as fma chains over head_dim / keys, which v_mfma_f32_16x16x4f32
// computes exactly (its 4-term dot is a sequential fma chain); chunk softmax,
// butterfly sums and the chunk merge as in device_common.hpp.
#include "device_common.hpp"
#include "lm_f16.hpp"
#include "step_kernel.hpp"

namespace mtg {

namespace {
using namespace dev;

constexpr int kT = 256;                 // threads per workgroup
constexpr int kNwg = 256;               // workgroups (one per CU)
// shapes the kernel is written for (Qwen3-0.6B)
constexpr int cH = 1024, cQN = 2048, cNQKV = 4096, cF = 3072, cNH = 16, cNKV = 8, cHD = 128;
constexpr int cBH = cH / kPairK, cBQ = cQN / kPairK, cBF = cF / kPairK;  // 16, 32, 48
constexpr int cOTiles = cH / 16;         // 64 (o-proj and down tiles, on workgroups 0..63)
constexpr int cGuBlocks = cF / 32;       // 96 (gate/up 32-row blocks, on workgroups 64..159)
constexpr int kMergeWg0 = 160;           // merge items on workgroups 160..255 (then 64..159)
constexpr int kMergeSlots = kNwg - kMergeWg0 + cGuBlocks;
// LDS stride of one activation-panel unit (the 1024 code bytes of a block pair as
// the MFMA B operand): 16 bytes of padding put the 16 units a wave's lanes write at
// once (a row's 64 half blocks) on different banks; without it every 16-byte
// write of a panel build was a 32-way bank conflict.
constexpr int kPanelUnit = 1024 + 16;
// the panel's f32 block scales: one row of 16 (8 even-, 8 odd-block columns) per
// unit, 17 floats apart for the same reason
constexpr int kScaleStride = 17;
constexpr int cQStride = 132;            // LDS row strides (conflict-free MFMA operand reads)
constexpr int cPStride = 68;
constexpr int kStageFloats = cH + cH / 4;  // one padded row image per wave (panel_norm)

enum { kPhQkv = 0, kPhAttn = 1, kPhMerge = 2, kPhO = 3, kPhGu = 4, kPhD = 5, kPhases = 6 };

typedef __amdgpu_buffer_rsrc_t Rsrc;
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// A pointer the whole wave shares, moved to scalar registers (a value that came
// through a generic load or a call argument sits in vector registers, and a
// buffer descriptor built from it would make every load a loop over lanes).
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t u = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return (T*)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ Rsrc mk_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, 0x00020000);
}
// device-coherent (agent scope) 16- and 4-byte accesses
__device__ __forceinline__ v4f ldc4(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16));
}
__device__ __forceinline__ float ldc1(Rsrc r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 16));
}
__device__ __forceinline__ void stc4(Rsrc r, uint32_t off, v4f v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), r, (int)off, 0, 16);
}
__device__ __forceinline__ void stc1(Rsrc r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, (int)off, 0, 16);
}

// Global-address-space access to memory reached through the parameter block:
// without the cast such pointers are generic and their loads become flat
// loads, which also count against the LDS counter, so every LDS wait would
// drain the prefetched weights.
#define MTG_GLOBAL __attribute__((address_space(1)))
template <class T>
__device__ __forceinline__ T gld(const void* p) { return *(const MTG_GLOBAL T*)p; }
template <class T>
__device__ __forceinline__ T gld_nt(const void* p) { return __builtin_nontemporal_load((const MTG_GLOBAL T*)p); }
template <class T>
__device__ __forceinline__ void gst(void* p, T v) { *(MTG_GLOBAL T*)p = v; }

// Workgroup barrier that waits only for LDS traffic, so loads issued ahead of
// it stay in flight.
__device__ __forceinline__ void bar() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }


// Layer l's pointers (scalar loads from the parameter block; a read through a
// generic pointer would be a flat load, and every use of it would wait for all
// vector loads in flight, the prefetched weights included).
__device__ __forceinline__ const LayerDev& layer_at(const StepParams& P, int l) { return P.layer[l]; }

struct Ctl {
  const StepParams* P;
  uint32_t epoch;
  uint32_t published;
  int* s_ok;
};

// A wait's bound: P.wait_polls polls, or P.wait_ticks of the device clock from
// its 256th poll on (read only every 256 polls, so a short wait never reads it).
__device__ __forceinline__ bool wait_expired(const StepParams& P, unsigned spins, uint64_t& t0) {
  if (spins > P.wait_polls) return true;
  if ((spins & 255u) == 0u) {
    const uint64_t now = wall_clock64();
    if (spins == 256u) t0 = now;
    else if (now - t0 > (uint64_t)P.wait_ticks) return true;
  }
  return false;
}

// All of this thread's stores have completed; then workgroup w announces v.
__device__ __forceinline__ void publish(Ctl& c, uint32_t v) {
  if (v <= c.published) return;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  bar();
  if (threadIdx.x == 0)  // device-coherent buffer store: no LDS-counter wait covers it
    __builtin_amdgcn_raw_buffer_store_b32(c.epoch + v, mk_rsrc(c.P->flags, kNwg * kFlagStride * 4),
                                          blockIdx.x * kFlagStride * 4, 0, 16);
  c.published = v;
}

// Wait until every workgroup has announced at least v. Returns false when the
// step is aborted (a bounded wait ran out here or elsewhere).
__device__ __forceinline__ bool wait_all(Ctl& c, uint32_t v, int prof_slot = -1) {
  const StepParams& P = *c.P;
  if (threadIdx.x < 64) {
    if (prof_slot >= 0 && P.timing && threadIdx.x == 0) gst<uint64_t>(P.timing + prof_slot, wall_clock64());
    const int lane = threadIdx.x;
    const Rsrc rf = mk_rsrc(P.flags, kNwg * kFlagStride * 4);
    const Rsrc re = mk_rsrc(P.err, 4);
    const uint32_t target = c.epoch + v;
    unsigned spins = 0;
    uint64_t t0 = 0;
    int ok = 1;
    // lane j watches the words of workgroups j, j+64, j+128, j+192 and keeps a
    // bit per word that has reached the target. The four loads issue back to
    // back; a word already seen gets an offset past the buffer's end, which the
    // range check answers with 0 and no memory request.
    constexpr uint32_t kGone = 0x80000000u;
    unsigned hv = 0;
    bool have = false;
    for (;;) {
      uint32_t f[kNwg / 64];
#pragma unroll
      for (int k = 0; k < kNwg / 64; ++k)
        f[k] = __builtin_amdgcn_raw_buffer_load_b32(
            rf, (hv & (1u << k)) ? kGone : (uint32_t)((k * 64 + lane) * kFlagStride * 4), 0, 16);
#pragma unroll
      for (int k = 0; k < kNwg / 64; ++k)
        if (f[k] >= target) hv |= 1u << k;
      have = hv == (1u << (kNwg / 64)) - 1;
      if (__all(have)) break;
      if (__builtin_amdgcn_raw_buffer_load_b32(re, 0, 0, 16)) { ok = 0; break; }
      if (wait_expired(P, ++spins, t0)) {
        if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(1u, re, 0, 0, 16);
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) *c.s_ok = ok;
  }
  bar();
  return *c.s_ok != 0;
}

// Values read from a tagged exchange buffer: each 8-byte pair is (value bits,
// tag), written by one 8-byte part of a store, so a pair whose tag is the phase's
// progress value holds that phase's value. Re-reads the pairs whose tag is not yet
// `want` until all are (bounded, like wait_all). Per lane: N pairs at byte offsets
// off[j] (live[j] false: not needed). When the wait runs out it raises the error
// word and returns with what it has: the workgroup leaves at its next progress
// wait, and the host discards the step (only positions from `past` on were
// written). The workgroup does not leave from here: an exit from inside the
// attention costs the whole kernel its register allocation.
template <int N>
__device__ __forceinline__ void tagged_wait(const StepParams& P, Rsrc r, v2u (&a)[N], const uint32_t (&off)[N],
                                            const bool (&live)[N], uint32_t want) {
  const Rsrc re = mk_rsrc(P.err, 4);
  uint64_t t0 = 0;
  for (unsigned spins = 0;; ++spins) {
    bool stale = false;
#pragma unroll
    for (int j = 0; j < N; ++j) stale |= live[j] && a[j].y != want;
    if (!__any(stale)) return;
    if (__builtin_amdgcn_raw_buffer_load_b32(re, 0, 0, 16)) return;
    if (spins > 0 && wait_expired(P, spins, t0)) {
      if ((threadIdx.x & 63) == 0) __builtin_amdgcn_raw_buffer_store_b32(1u, re, 0, 0, 16);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (live[j] && a[j].y != want) a[j] = __builtin_amdgcn_raw_buffer_load_b64(r, off[j], 0, 16);
  }
}

__device__ __forceinline__ void mark(const StepParams& P, int slot) {
  if (P.timing && blockIdx.x == 0 && threadIdx.x == 0) gst<uint64_t>(P.timing + slot, wall_clock64());
}
// every workgroup's marks of one layer: slots 1024 + 32 w + k
__device__ __forceinline__ int wslot(int w, int k) { return 1024 + 32 * w + k; }
__device__ __forceinline__ void wmark(const StepParams& P, int l, int k) {
  if (P.timing && l == 1 && threadIdx.x == 0) gst<uint64_t>(P.timing + wslot(blockIdx.x, k), wall_clock64());
}

// ----------------------------------------------------------- weight tiles ---
// NP block pairs of one wave's K-slice of a 16-row tile, held in registers:
// a[p] = the lane's 16 code bytes, s[p] = the 4 f16 row scales it needs.
template <int NP>
__device__ __forceinline__ void wt_load(const uint8_t* __restrict__ tile, int bp0, v4i* a, uint2* s) {
  const int lane = threadIdx.x & 63;
  const int srow = ((lane & 15) >> 3) * 16 + 4 * (lane >> 4);
  // buffer loads: per-lane 32-bit offset + wave-uniform scalar offset per unit
  const Rsrc r = mk_rsrc(tile, cBF * kUnitBytes);
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int so = (bp0 + p) * kUnitBytes;
    a[p] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, so, 2));
    const v2u sv = __builtin_amdgcn_raw_buffer_load_b64(r, 1024 + srow * 2, so, 2);
    s[p] = make_uint2(sv.x, sv.y);
  }
}

// acc[cg][r] += the tile slice against the activation panel (canonical: per
// block, acc = fma(isum, dw * dx, acc) in block-pair order).
template <int G, int NP>
__device__ __forceinline__ void wt_mma(const v4i* a, const uint2* sc, int bp0, int bps,
                                       const uint8_t* __restrict__ pcodes,
                                       const float* __restrict__ pscales, float acc[G][4]) {
  const int lane = threadIdx.x & 63;
  const v4i zero = {0, 0, 0, 0};
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    float dw[4];
    dw[0] = half_bits_to_float((uint16_t)(sc[p].x & 0xffff));
    dw[1] = half_bits_to_float((uint16_t)(sc[p].x >> 16));
    dw[2] = half_bits_to_float((uint16_t)(sc[p].y & 0xffff));
    dw[3] = half_bits_to_float((uint16_t)(sc[p].y >> 16));
#pragma unroll
    for (int cg = 0; cg < G; ++cg) {
      const int bp = bp0 + p;
      const v4i b = *(const v4i*)(pcodes + ((size_t)(cg * bps + bp)) * kPanelUnit + lane * 16);
      const float dx = pscales[(size_t)(cg * bps + bp) * kScaleStride + (lane & 15)];
      const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[p], b, zero, 0, 0, 0);
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[cg][q] = fmaf((float)c[q], dw[q] * dx, acc[cg][q]);
    }
  }
}

// q8_0 code of v with the block's scale: d = amax / 127 rounded to f16,
// code = rint(v * 127 / amax) (the activation quantizer of the q8_0 GEMMs).
__device__ __forceinline__ float q8_scale(float amax) { return __half2float(__float2half_rn(__fdiv_rn(amax, 127.0f))); }
__device__ __forceinline__ uint32_t q8_code(float v, float amax) {
  const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
  return (uint32_t)(uint8_t)(int8_t)rintf(__fmul_rn(v, id));
}

enum { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2 };

// The four waves' slice sums meet in LDS and are added in wave order, then the
// even and odd block halves; wave 0 writes T x 16 outputs with 16-byte stores.
template <int G, int NM, int EPI>
__device__ __forceinline__ void gemm_finish(float acc[NM][G][4], float* red, Rsrc out, int n,
                                            int tile, int T, float* xs = nullptr, bool xs_valid = false,
                                            uint32_t tag = 0) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int cg = 0; cg < G; ++cg)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[((wave * NM + m) * G * 4 + cg * 4 + q) * 64 + lane] = acc[m][cg][q];
  bar();
  if (wave == 0) {
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
      for (int cg = 0; cg < G; ++cg)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float s = red[((0 * NM + m) * G * 4 + cg * 4 + q) * 64 + lane];
#pragma unroll
          for (int wv = 1; wv < 4; ++wv) s = __fadd_rn(s, red[((wv * NM + m) * G * 4 + cg * 4 + q) * 64 + lane]);
          acc[m][cg][q] = __fadd_rn(s, dpp_f<kDppRor8>(s));
        }
    if ((lane & 15) < 8) {
#pragma unroll
      for (int cg = 0; cg < G; ++cg) {
        const int t = cg * 8 + (lane & 7);
        if (t < T) {
          const uint32_t off = (uint32_t)((t * n + tile * 16 + 4 * (lane >> 4)) * 4);
          v4f v;
          if (EPI == EPI_STORE) {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = acc[0][cg][q];
          } else if (EPI == EPI_RESID) {
            // this workgroup is the only writer of its 16 residual columns: after
            // the first time they come from its LDS copy, not from memory
            v4f* xl = (v4f*)(xs + t * 16 + 4 * (lane >> 4));
            const v4f x = xs_valid ? *xl : ldc4(out, off);
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = __fadd_rn(x[q], acc[0][cg][q]);
            *xl = v;
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = dev_swiglu(acc[0][cg][q], acc[NM - 1][cg][q]);
          }
          if (EPI == EPI_STORE) {
            // (value, tag) pairs, two per 16-byte store: readers check the tags
            // instead of waiting for this workgroup's progress word
            const v4u p0 = {__float_as_uint(v[0]), tag, __float_as_uint(v[1]), tag};
            const v4u p1 = {__float_as_uint(v[2]), tag, __float_as_uint(v[3]), tag};
            __builtin_amdgcn_raw_buffer_store_b128(p0, out, (int)(2 * off), 0, 16);
            __builtin_amdgcn_raw_buffer_store_b128(p1, out, (int)(2 * off + 16), 0, 16);
          } else {
            stc4(out, off, v);
          }
        }
      }
    }
  }
  bar();
}

// Gate and up of rows 32j..32j+31 (two 16-row tiles; acc[0], acc[1] gate,
// acc[2], acc[3] up): the wave slice sums meet in LDS in wave order, then the
// even and odd halves, SwiGLU, and each row t's 32 values leave as one q8_0
// block. Wave w finishes the values of row slot q = w of every tile (lane l
// holds tile rows 4 (l / 16) + q for verify row t = 8 cg + l % 8), so the four
// waves share the SwiGLU and quantization; the block maxima meet in LDS (amx).
template <int G>
__device__ __forceinline__ void gu_finish(float acc[4][G][4], float* red, float* amx, const StepParams& P,
                                          int j, int T) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int cg = 0; cg < G; ++cg)
#pragma unroll
      for (int q = 0; q < 4; ++q) red[((wave * 4 + m) * G * 4 + cg * 4 + q) * 64 + lane] = acc[m][cg][q];
  bar();
  const int q = wave;
  float va[G], vb[G];
#pragma unroll
  for (int cg = 0; cg < G; ++cg) {
    float v4[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      float s = red[((0 * 4 + m) * G * 4 + cg * 4 + q) * 64 + lane];
#pragma unroll
      for (int wv = 1; wv < 4; ++wv) s = __fadd_rn(s, red[((wv * 4 + m) * G * 4 + cg * 4 + q) * 64 + lane]);
      v4[m] = __fadd_rn(s, dpp_f<kDppRor8>(s));
    }
    va[cg] = dev_swiglu(v4[0], v4[2]);
    vb[cg] = dev_swiglu(v4[1], v4[3]);
    // this wave's part of the block maximum: its two values, over the lanes of
    // the same t (xor 16, 32)
    const float am = __uint_as_float(
        pair_max_u<32>(pair_max_u<16>(__float_as_uint(fmaxf(fabsf(va[cg]), fabsf(vb[cg]))))));
    if (lane < 16) amx[(wave * G + cg) * 16 + lane] = am;
  }
  bar();
  const Rsrc rq = mk_rsrc(P.aq, kMaxRows * cF);
  const Rsrc rs = mk_rsrc(P.aqs, kMaxRows * (cF / 32) * 4);
  // The block's 32 codes of each verify row meet in LDS (the reduction space is
  // free now) and leave as two 16-byte stores: byte stores from 96 producers
  // into shared lines cost more to acknowledge and to read back.
  uint8_t* cl = (uint8_t*)red;
#pragma unroll
  for (int cg = 0; cg < G; ++cg) {
    const int t = cg * 8 + (lane & 7);
    if ((lane & 15) < 8 && t < T) {
      float amax = amx[(0 * G + cg) * 16 + (lane & 15)];
#pragma unroll
      for (int wv = 1; wv < 4; ++wv) amax = fmaxf(amax, amx[(wv * G + cg) * 16 + (lane & 15)]);
      const float id = amax != 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
      const int r = 4 * (lane >> 4) + q;
      cl[t * 32 + r] = (uint8_t)(int8_t)rintf(__fmul_rn(va[cg], id));
      cl[t * 32 + r + 16] = (uint8_t)(int8_t)rintf(__fmul_rn(vb[cg], id));
      if (wave == 0 && lane < 16) stc1(rs, (uint32_t)((t * (cF / 32) + j) * 4), q8_scale(amax));
    }
  }
  bar();
  if ((int)threadIdx.x < 2 * T) {
    const int t = threadIdx.x >> 1, h = threadIdx.x & 1;
    const v4u v = *(const v4u*)(cl + t * 32 + 16 * h);
    __builtin_amdgcn_raw_buffer_store_b128(v, rq, t * cF + 32 * j + 16 * h, 0, 16);
  }
  bar();
}

// two floats as f16 bits (round to nearest even), the first in the low half
__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  return (uint32_t)__half_as_ushort(__float2half_rn(a)) | ((uint32_t)__half_as_ushort(__float2half_rn(b)) << 16);
}

// --------------------------------------------------------------- panels -----
// 16 elements (a half q8_0 block) -> codes in the LDS panel; lanes l and l^1 hold
// the two halves of one block.
__device__ __forceinline__ void quant16(const float v[16], int t, int kc, int bps, uint8_t* pcodes,
                                        float* pscales) {
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = __uint_as_float(max(__float_as_uint(amax), dpp_u<kDppQuadXor1>(__float_as_uint(amax))));
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
  uint8_t* unit = pcodes + (size_t)(cg * bps + bp) * kPanelUnit;
  *(uint4*)(unit + (j + 16 * (2 * par + half)) * 16) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  *(uint4*)(unit + (j + 16 * (2 * (1 - par) + half)) * 16) = make_uint4(0u, 0u, 0u, 0u);
  if (half == 0) pscales[(size_t)(cg * bps + bp) * kScaleStride + j] = __half2float(__float2half_rn(d));
}

// Panel of RMSNorm(x) * gain for T rows of 1024 (one wave per row): lane l
// holds elements 16l..16l+15. normed_out (nullable): the f32 rows.
// The 16 gain values of lane l (elements 16 l .. 16 l + 15) of a 1024 norm. The
// layers' norms are loaded with the weights of the phase that uses them, before
// its wait: a load from HBM issued just before the activation loads would hold
// them up (loads complete in order).
__device__ __forceinline__ void gain16_load(const float* __restrict__ gain, float (&gv)[16]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const v4f g = gld<v4f>(gain + 16 * lane + 4 * i);
    gv[4 * i] = g[0];
    gv[4 * i + 1] = g[1];
    gv[4 * i + 2] = g[2];
    gv[4 * i + 3] = g[3];
  }
}

// COAL: the rows come with coalesced loads (lane l: 16 bytes at 16 l + 1024 i)
// and reach their lanes through this wave's LDS row image (element e at
// e + 4 (e / 16): the 16-byte reads of 16 consecutive elements per lane are free
// of bank conflicts; LDS accesses of one wave execute in order, no barrier).
// Otherwise each lane loads its own 64 bytes (every load instruction then
// touches all 32 lines of a row, ~20 % slower in a 256-workgroup broadcast, but
// no LDS image and fewer registers: the 16-row variant keeps that form).
// gain_late (nullable): the gains are loaded here, after the rows, instead of
// coming prefetched in gv (the 16-row variant: 16 fewer registers held across
// the phases, for 0.3 us more per panel).
// HOUT 1 / 2: the normed rows leave as f16 / f32 rows [t][1024] at pcodes (the f16
// and f32 GEMMs' vec_dot_type; lane l writes its elements 16 l .. 16 l + 15) instead
// of q8_0 codes.
template <bool COAL, int HOUT = 0>
__device__ __forceinline__ void panel_norm(Rsrc x, int T, const float (&gv_in)[16], float eps, uint8_t* pcodes,
                                           float* pscales, float* normed_out, float* stage,
                                           const float* gain_late = nullptr, const StepParams* prof = nullptr) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  float gv[16];
  for (int t0 = wave; t0 < T; t0 += 8) {
    // two rows per pass (t0 and t0 + 4), all loads issued before any arithmetic;
    // their arithmetic runs side by side (the double sums are dependent chains)
    const bool two = t0 + 4 < T;
    v4f raw[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = t0 + 4 * j;
      if (j == 0 || two) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          raw[j][i] = ldc4(x, (uint32_t)((t * cH + (COAL ? 4 * lane + 256 * i : 16 * lane + 4 * i)) * 4));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) raw[j][i] = v4f{0.f, 0.f, 0.f, 0.f};
      }
    }
    if (gain_late) {
      if (t0 == wave) gain16_load(gain_late, gv);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) gv[e] = gv_in[e];
    }
    if (prof && t0 == wave) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); wmark(*prof, 1, 13); }
    float v[2][16];
    if constexpr (COAL) {
      // one row image per row and wave (LDS accesses of a wave execute in order)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float* stg = stage + (2 * wave + j) * kStageFloats;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e0 = 4 * lane + 256 * i;
          *(v4f*)(stg + e0 + 4 * (e0 >> 4)) = raw[j][i];
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float* stg = stage + (2 * wave + j) * kStageFloats;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const v4f q = *(const v4f*)(stg + 20 * lane + 4 * i);
          v[j][4 * i] = q[0];
          v[j][4 * i + 1] = q[1];
          v[j][4 * i + 2] = q[2];
          v[j][4 * i + 3] = q[3];
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[j][4 * i] = raw[j][i][0];
          v[j][4 * i + 1] = raw[j][i][1];
          v[j][4 * i + 2] = raw[j][i][2];
          v[j][4 * i + 3] = raw[j][i][3];
        }
    }
    double s[2] = {0.0, 0.0};
#pragma unroll
    for (int e = 0; e < 16; ++e)
#pragma unroll
      for (int j = 0; j < 2; ++j) s[j] += (double)__fmul_rn(v[j][e], v[j][e]);
    float scale[2];
    rms_scales<2, cH>(s, eps, scale);
    float y[2][16];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) y[j][e] = __fmul_rn(__fmul_rn(v[j][e], scale[j]), gv[e]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = t0 + 4 * j;
      if (j == 1 && !two) break;
      if (normed_out)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const v4f o = {y[j][4 * i], y[j][4 * i + 1], y[j][4 * i + 2], y[j][4 * i + 3]};
          gst<v4f>(normed_out + (size_t)t * cH + 16 * lane + 4 * i, o);
        }
      if constexpr (HOUT == 2) {
        v4f* dst = (v4f*)((float*)pcodes + t * cH + 16 * lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) dst[i] = v4f{y[j][4 * i], y[j][4 * i + 1], y[j][4 * i + 2], y[j][4 * i + 3]};
      } else if constexpr (HOUT == 1) {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 16; e += 2) {
          // the float products first: the compiler would otherwise fold the last
          // multiply and the conversion into one fma_mix (one rounding, not two)
          float a = y[j][e], b = y[j][e + 1];
          asm volatile("" : "+v"(a), "+v"(b));
          h[e / 2] = pack_half2(a, b);
        }
        uint4* dst = (uint4*)((uint16_t*)pcodes + t * cH + 16 * lane);
        dst[0] = make_uint4(h[0], h[1], h[2], h[3]);
        dst[1] = make_uint4(h[4], h[5], h[6], h[7]);
      } else {
        quant16(y[j], t, lane, cBH, pcodes, pscales);
      }
    }
  }
  bar();
}

// Panel of T rows of K activations already quantized by their producer:
// codes [t][K] int8, scales [t][K/32]. Thread = 16 codes (a half block); every
// load is issued before the first LDS write (one round trip).
template <int K, int G>
__device__ __forceinline__ void panel_from_q(const int8_t* codes, const float* scales, int T, uint8_t* pcodes,
                                             float* pscales) {
  constexpr int cpr = K / 16, bps = K / kPairK;
  constexpr int NC = (8 * G * cpr + kT - 1) / kT;  // chunks per thread at the largest T
  const Rsrc rc = mk_rsrc(codes, kMaxRows * K);
  const Rsrc rs = mk_rsrc(scales, kMaxRows * (K / 32) * 4);
  const int chunks = T * cpr;
  // the thread index through an empty asm: the chunk addresses below are then
  // computed here, on every call. As loop invariants of the layer loop they were
  // hoisted out of it and, in the 16-row variant, spilled to scratch; each
  // reload then waited for all the panel's loads before it (one round trip per
  // chunk: 8 us more per down panel).
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  v4u q[NC];
  float d[NC];
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = j * kT + tid;
    // a chunk past the rows reads past the buffers' ends: zeros, no memory traffic
    const int t = c / cpr, kc = c % cpr;
    const bool in = c < chunks;
    q[j] = __builtin_amdgcn_raw_buffer_load_b128(rc, in ? (uint32_t)(t * K + kc * 16) : 0x80000000u, 0, 16);
    d[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                         rs, in ? (uint32_t)((t * (K / 32) + (kc >> 1)) * 4) : 0x80000000u, 0, 16));
  }
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = j * kT + tid;
    if (c < chunks) {
      const int t = c / cpr, kc = c % cpr;
      const int blk = kc >> 1, half = kc & 1, bp = blk >> 1, par = blk & 1;
      const int cg = t >> 3, jc = par * 8 + (t & 7);
      uint8_t* unit = pcodes + (size_t)(cg * bps + bp) * kPanelUnit;
      *(uint4*)(unit + (jc + 16 * (2 * par + half)) * 16) = make_uint4(q[j].x, q[j].y, q[j].z, q[j].w);
      *(uint4*)(unit + (jc + 16 * (2 * (1 - par) + half)) * 16) = make_uint4(0u, 0u, 0u, 0u);
      if (half == 0) pscales[(size_t)(cg * bps + bp) * kScaleStride + jc] = d[j];
    }
  }
  bar();
}

// ------------------------------------------------------------ attention -----
// K and V of one 64-key chunk, raw cache bytes in 16-byte pieces: piece p =
// j * 256 + thread (j < NP) is bytes 16 p .. 16 p + 15 of the chunk's rows, K
// pieces first, then V (NP = 8 for an f32 cache, 4 for f16). Coalesced: a wave's
// load covers 1 KB of consecutive rows. (Loading the MFMA operand layout
// directly, an element per lane and load, made every load touch 16 cache lines:
// the address unit, not the memory, then set the time.) Zero from row `past`
// on: the loads' range ends there.
struct KvRegs {
  v4u p[16];
};

template <int KVH>
__device__ __forceinline__ void kv_prefetch(const LayerDev& Ly, const StepParams& P, int g, int key0,
                                            int past, KvRegs& r) {
  constexpr int es = KVH ? 2 : 4, NP = KVH ? 4 : 8;
  const size_t head = (size_t)g * P.max_seq * cHD * es;
  const Rsrc rk = mk_rsrc(Ly.kc + head, (uint32_t)(past * cHD * es));
  const Rsrc rv = mk_rsrc(Ly.vc + head, (uint32_t)(past * cHD * es));
  // the whole offset per lane (scalar offset 0): a piece at or past `past` lies
  // beyond num_records and reads 0 without touching memory
  const uint32_t o0 = (uint32_t)(key0 * cHD * es) + 16u * threadIdx.x;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    r.p[j] = __builtin_amdgcn_raw_buffer_load_b128(rk, o0 + 16u * kT * j, 0, 0);
    r.p[NP + j] = __builtin_amdgcn_raw_buffer_load_b128(rv, o0 + 16u * kT * j, 0, 0);
  }
}

// LDS rows of the chunk's K and V as f32, padded so that the operand reads of
// attn_item are free of bank conflicts: K row key at key * kKStride, V row at
// key * kVStride.
constexpr int kKStride = cHD + 4, kVStride = cHD + 16;
constexpr int kKvLdsFloats = kChunk * (kKStride + kVStride);

template <int KVH>
__device__ __forceinline__ void kv_to_lds(const KvRegs& r, float* ks, float* vs) {
  constexpr int NP = KVH ? 4 : 8;
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int p = j * kT + threadIdx.x;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const v4u q = r.p[t * NP + j];
      float* base = t == 0 ? ks : vs;
      const int stride = t == 0 ? kKStride : kVStride;
      if constexpr (KVH != 0) {  // 8 halves: elements 8 (p % 16) .. of row p / 16
        float* d = base + (p / 16) * stride + 8 * (p % 16);
        const v4f lo = {half_bits_to_float((uint16_t)q.x), half_bits_to_float((uint16_t)(q.x >> 16)),
                        half_bits_to_float((uint16_t)q.y), half_bits_to_float((uint16_t)(q.y >> 16))};
        const v4f hi = {half_bits_to_float((uint16_t)q.z), half_bits_to_float((uint16_t)(q.z >> 16)),
                        half_bits_to_float((uint16_t)q.w), half_bits_to_float((uint16_t)(q.w >> 16))};
        *(v4f*)d = lo;
        *(v4f*)(d + 4) = hi;
      } else {  // 4 floats: elements 4 (p % 32) .. of row p / 32
        *(v4u*)(base + (p / 32) * stride + 4 * (p % 32)) = q;
      }
    }
  }
}

// One staging pass of an attention item: wave `wave` takes rows r0 + 4 j,
// j < NS (q rows, then the new k rows, then the new v rows), loads them all,
// then norms (q, k) and ropes them side by side and writes them to LDS.
// Straight-line over the NS slots; slots past the rows compute on zeros and store
// nothing.
template <int NS, int KVH>
__device__ __forceinline__ void stage_pass(const StepParams& P, const LayerDev& Ly, int T, int past, int g,
                                           int r0, int nrows, uint32_t tag, float* q_lds, float* knew,
                                           float* vnew, bool prof = false, int hsel = -1) {
  // hsel >= 0: the q rows are those of q head 2 g + hsel only (T of them)
  const int lane = threadIdx.x & 63, ncol = hsel < 0 ? 2 * T : T;
  constexpr bool f16kv = KVH != 0;
  const Rsrc rq = mk_rsrc(P.qkvt, kMaxRows * cNQKV * 8);
  float x0[NS], x1[NS], g0[NS], g1[NS], rc[NS], rs[NS];
  int kind[NS], tt[NS];
  v2u pr[2 * NS];  // (value, tag) of elements lane and lane + 64 of each slot
  uint32_t po[2 * NS];
  bool live[2 * NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int r = r0 + 4 * j;
    kind[j] = r < ncol ? 0 : (r < ncol + T ? 1 : 2);
    tt[j] = kind[j] == 0 ? r % T : (kind[j] == 1 ? r - ncol : r - ncol - T);
    g0[j] = g1[j] = rc[j] = rs[j] = 0.0f;
    live[2 * j] = live[2 * j + 1] = r < nrows;
    const int col = kind[j] == 0 ? (2 * g + (hsel < 0 ? r / T : hsel)) * cHD
                                 : (kind[j] == 1 ? (cNH + g) * cHD : (cNH + cNKV + g) * cHD);
    po[2 * j] = (uint32_t)((min(tt[j], kMaxRows - 1) * cNQKV + col + lane) * 8);
    po[2 * j + 1] = po[2 * j] + 64 * 8;
    pr[2 * j] = pr[2 * j + 1] = v2u{0u, tag};
    if (r < nrows) {
      pr[2 * j] = __builtin_amdgcn_raw_buffer_load_b64(rq, po[2 * j], 0, 16);
      pr[2 * j + 1] = __builtin_amdgcn_raw_buffer_load_b64(rq, po[2 * j + 1], 0, 16);
      if (kind[j] < 2) {
        const float* gn = kind[j] == 0 ? Ly.q_norm : Ly.k_norm;
        g0[j] = gld<float>(gn + lane);
        g1[j] = gld<float>(gn + lane + 64);
        const v2f cs = gld<v2f>(P.rope + (size_t)(past + tt[j]) * cHD + 2 * lane);
        rc[j] = cs.x;
        rs[j] = cs.y;
      }
    }
  }
  tagged_wait<2 * NS>(P, rq, pr, po, live, tag);
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    x0[j] = __uint_as_float(pr[2 * j].x);
    x1[j] = __uint_as_float(pr[2 * j + 1].x);
  }
  if (prof) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); wmark(P, 1, 15); }
  double sq[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) sq[j] = (double)__fmul_rn(x0[j], x0[j]) + (double)__fmul_rn(x1[j], x1[j]);
  float scale[NS];
  rms_scales<NS, cHD>(sq, P.eps, scale);
  float y0[NS], y1[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const float n0 = __fmul_rn(__fmul_rn(x0[j], scale[j]), g0[j]);
    const float n1 = __fmul_rn(__fmul_rn(x1[j], scale[j]), g1[j]);
    y0[j] = __fsub_rn(__fmul_rn(n0, rc[j]), __fmul_rn(n1, rs[j]));
    y1[j] = __fadd_rn(__fmul_rn(n0, rs[j]), __fmul_rn(n1, rc[j]));
  }
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int r = r0 + 4 * j, t = tt[j];
    if (r >= nrows) break;
    const float a0 = kind[j] < 2 ? y0[j] : x0[j], a1 = kind[j] < 2 ? y1[j] : x1[j];
    // q and new k rows are kept permuted (element 4 s + kk at kk * 32 + s), so that
    // a lane reads its 32 score operands of one row with 16-byte LDS reads
    const int o0 = kind[j] < 2 ? (lane & 3) * 32 + (lane >> 2) : lane;
    const int o1 = kind[j] < 2 ? o0 + 16 : lane + 64;
    float* dst = kind[j] == 0 ? q_lds + r * cQStride : (kind[j] == 1 ? knew : vnew) + t * cQStride;
    dst[o0] = f16kv ? f16_round(a0) : a0;
    dst[o1] = f16kv ? f16_round(a1) : a1;
  }
}

// The new v rows of kv head g: wave w copies rows w + 4 j (j < NV, row < T) of
// this step's v to LDS (f16-rounded for an f16 cache). stage_v_issue sends the
// loads (before the q / k staging, so that both are in flight together);
// stage_v_finish checks their tags and writes the rows.
template <int NV>
struct VStage {
  v2u pr[2 * NV];
  uint32_t po[2 * NV];
  bool live[2 * NV];
};

template <int NV>
__device__ __forceinline__ void stage_v_issue(const StepParams& P, int g, int T, VStage<NV>& v) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const Rsrc rq = mk_rsrc(P.qkvt, kMaxRows * cNQKV * 8);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int t = wave + 4 * j;
    v.po[2 * j] = (uint32_t)((min(t, T - 1) * cNQKV + (cNH + cNKV + g) * cHD + lane) * 8);
    v.po[2 * j + 1] = v.po[2 * j] + 64 * 8;
    v.live[2 * j] = v.live[2 * j + 1] = t < T;
    v.pr[2 * j] = __builtin_amdgcn_raw_buffer_load_b64(rq, v.po[2 * j], 0, 16);
    v.pr[2 * j + 1] = __builtin_amdgcn_raw_buffer_load_b64(rq, v.po[2 * j + 1], 0, 16);
  }
}

template <int NV, int KVH>
__device__ __forceinline__ void stage_v_finish(const StepParams& P, int T, uint32_t tag, VStage<NV>& v,
                                               float* vnew) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const Rsrc rq = mk_rsrc(P.qkvt, kMaxRows * cNQKV * 8);
  tagged_wait<2 * NV>(P, rq, v.pr, v.po, v.live, tag);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int t = wave + 4 * j;
    if (t >= T) break;
    const float x0 = __uint_as_float(v.pr[2 * j].x), x1 = __uint_as_float(v.pr[2 * j + 1].x);
    vnew[t * cQStride + lane] = KVH ? f16_round(x0) : x0;
    vnew[t * cQStride + lane + 64] = KVH ? f16_round(x1) : x1;
  }
}

// This step's k / v rows of kv head g, staged in LDS (knew: normed, roped and
// permuted, vnew: plain; f16-rounded for an f16 cache), written to the KV cache
// at positions past .. past + T - 1 with 16-byte stores.
template <int KVH>
__device__ __forceinline__ void kv_append(const StepParams& P, const LayerDev& Ly, int T, int past, int g,
                                          const float* knew, const float* vnew) {
  constexpr bool f16kv = KVH != 0;
  // wave-uniform cache pointers (a per-lane choice between the two fields
  // would load the pointer with a vector load before every store)
  uint8_t* const kcp = uniform_ptr(Ly.kc);
  uint8_t* const vcp = uniform_ptr(Ly.vc);
  for (int i = threadIdx.x; i < T * (cHD / 4); i += kT) {  // 4 elements of one row
    const int t = i / (cHD / 4), m = i % (cHD / 4), d = 4 * m;
    const size_t off = ((size_t)g * P.max_seq + past + t) * cHD + d;
    const float* kr = knew + t * cQStride + m;  // element 4 m + kk sits at kk * 32 + m
    const v4f kq = {kr[0], kr[32], kr[64], kr[96]};
    const v4f vq = *(const v4f*)(vnew + t * cQStride + d);
    if (f16kv) {
      const v2u kh = {pack_half2(kq[0], kq[1]), pack_half2(kq[2], kq[3])};
      const v2u vh = {pack_half2(vq[0], vq[1]), pack_half2(vq[2], vq[3])};
      gst<v2u>((uint16_t*)kcp + off, kh);
      gst<v2u>((uint16_t*)vcp + off, vh);
    } else {
      gst<v4f>((float*)kcp + off, kq);
      gst<v4f>((float*)vcp + off, vq);
    }
  }
}

// The KV append of kv head g by a workgroup without attention items: the new k
// rows normed and roped and the new v rows, staged from the tagged q|k|v buffer
// as the attention items stage them, then written to the cache. Nothing in this
// step reads them from the cache (the items take new rows from their own
// staging), so this runs beside the attention, off its critical path.
template <int G, int KVH>
__device__ __forceinline__ void append_item(const StepParams& P, const LayerDev& Ly, int T, int past, int g,
                                            uint32_t tag, uint8_t* lds) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), ncol = 2 * T;
  float* q_lds = (float*)lds;
  float* knew = q_lds + kMaxCols * cQStride;
  float* vnew = knew + kMaxRows * cQStride;
  stage_pass<4 * G, KVH>(P, Ly, T, past, g, ncol + wave, ncol + 2 * T, tag, q_lds, knew, vnew);
  bar();
  kv_append<KVH>(P, Ly, T, past, g, knew, vnew);
}

// One attention item: chunk `chunk` of kv head g over the ncol = 2T query
// columns (col = hl*T + t for q head 2g + hl). LDS: q [32][132], knew/vnew
// [16][132], sp [32][68], the chunk's K [64][132] and V [64][144]. stage: stage the q rows (the first item of a
// workgroup; later items of the same kv head find them in LDS), with the new k /
// v rows if stage_new. next_chunk >= 0: the K / V of that chunk of the same head
// are loaded into kv once this item's operands are out of it. hsel >= 0: the item
// covers q head 2g + hsel only (its T columns, the partials' columns hsel T + t;
// another workgroup takes the other head): the last chunk's item is split when
// free workgroups exist, so that each half norms and ropes 2T rows, not 3T.
template <int G, int KVH>
__device__ __forceinline__ void attn_item(const StepParams& P, const LayerDev& Ly, int T, int past, int g, int chunk,
                                          uint32_t tag, KvRegs& kv, uint8_t* lds, bool self_append, bool prof,
                                          bool stage, bool stage_new, int next_chunk, int hsel) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63, kl = lane & 15,
            kk = lane >> 4;
  constexpr bool f16kv = KVH != 0;
  // ncol local columns; column c of this item is column c + col_off of the chunk's partials
  const int kvlen = past + T, ncol = hsel < 0 ? 2 * T : T, col_off = hsel == 1 ? T : 0, key0 = chunk * kChunk;
  float* q_lds = (float*)lds;
  float* knew = q_lds + kMaxCols * cQStride;
  float* vnew = knew + kMaxRows * cQStride;
  float* sp = vnew + kMaxRows * cQStride;
  float* ks = sp + kMaxCols * cPStride;
  float* vs = ks + kChunk * kKStride;
  const bool has_new = key0 + kChunk > past;
  const bool appender = key0 <= past && past < key0 + kChunk;
  // 1. stage the roped q rows and, if this chunk reaches them, the new k / v rows
  //    (q rows: 4G per wave; with the new rows up to 8 per wave and pass). The
  //    rows come from the tagged q|k|v buffer: no wait for the q|k|v phase's
  //    progress, each value is checked by its tag.
  if (prof) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); bar(); wmark(P, 1, 21); }
  // this chunk's K / V into the LDS rows (ordered before the operand reads by
  // the barrier below)
  kv_to_lds<KVH>(kv, ks, vs);
  if (stage) {
    if (!stage_new) {
      stage_pass<4 * G, KVH>(P, Ly, T, past, g, wave, ncol, tag, q_lds, knew, vnew, prof, hsel);
    } else {
      // q and new k rows are normed and roped; the new v rows are plain copies
      VStage<2 * G> vst;
      stage_v_issue<2 * G>(P, g, T, vst);
      if (hsel >= 0)  // T q rows + T k rows: at most 4G per wave (T <= 8 G)
        stage_pass<4 * G, KVH>(P, Ly, T, past, g, wave, ncol + T, tag, q_lds, knew, vnew, prof, hsel);
      else
        stage_pass<6 * G, KVH>(P, Ly, T, past, g, wave, ncol + T, tag, q_lds, knew, vnew, prof);
      if (prof) wmark(P, 1, 14);
      stage_v_finish<2 * G, KVH>(P, T, tag, vst, vnew);
    }
  }
  bar();
  if (prof) wmark(P, 1, 16);
  // 2. operands: cache rows from the LDS rows (zero from `past` on), new rows
  //    [past, kvlen) from the staged rows. Lane (kl, kk) of wave w: K[16 w + kl]
  //    [4 s + kk] (s < 32) for the scores, V[4 s + kk][16 (2 w + h) + kl] (s < 16)
  //    for P.V.
  float ka[32], vb[2][16];
#pragma unroll
  for (int s = 0; s < 32; ++s) ka[s] = ks[(16 * wave + kl) * kKStride + 4 * s + kk];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int s = 0; s < 16; ++s) vb[h][s] = vs[(4 * s + kk) * kVStride + 16 * (2 * wave + h) + kl];
  // Without a helper workgroup (every workgroup holds attention items), the
  // appending item writes this step's k / v rows to the KV cache from the staged
  // rows (for an f16 cache they are f16 values already); their acknowledgement
  // overlaps the scores instead of delaying the publish.
  if (appender && self_append) kv_append<KVH>(P, Ly, T, past, g, knew, vnew);
  if (has_new) {
    // score operands: the lane's key, all 32 values from one permuted row
    const int key = key0 + 16 * wave + kl;
    if (key >= past && key < kvlen) {
      const float* kr = knew + (key - past) * cQStride + kk * 32;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const v4f q = *(const v4f*)(kr + 4 * i);
        ka[4 * i] = q[0];
        ka[4 * i + 1] = q[1];
        ka[4 * i + 2] = q[2];
        ka[4 * i + 3] = q[3];
      }
    }
    // P.V operands: only the key groups that reach a new key
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const int g0 = key0 + 4 * s;  // wave-uniform
      if (g0 + 3 < past || g0 >= kvlen) continue;
      const int vk = g0 + kk;
      if (vk >= past && vk < kvlen) {
        const float* vrow = vnew + (vk - past) * cQStride + 32 * wave + kl;
        vb[0][s] = vrow[0];
        vb[1][s] = vrow[16];
      }
    }
  }
  // the next chunk's K / V: in flight during this chunk's arithmetic. Issued
  // after the operand reads: a wait that the compiler puts before writes of
  // registers (conservative where earlier loads wrote them) would otherwise wait
  // for these loads too.
  if (next_chunk >= 0) kv_prefetch<KVH>(Ly, P, g, next_chunk * kChunk, past, kv);
  if (prof) { bar(); wmark(P, 1, 17); }
  // 3. scores S[key][col] = fma chain over head_dim, scaled and masked -> sp
  // (the G column tiles' chains run interleaved: 2 T <= 16 G columns)
  const float scale = __fdiv_rn(1.0f, dev_sqrtf((float)cHD));
  {
    v4f acc[G];
    const float* qrow[G];
#pragma unroll
    for (int ct = 0; ct < G; ++ct) {
      acc[ct] = v4f{0.f, 0.f, 0.f, 0.f};
      // the column's permuted q row: element 4 s + kk at kk * 32 + s
      qrow[ct] = q_lds + min(ct * 16 + kl, ncol - 1) * cQStride + kk * 32;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v4f q4[G];
#pragma unroll
      for (int ct = 0; ct < G; ++ct) q4[ct] = *(const v4f*)(qrow[ct] + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int ct = 0; ct < G; ++ct) {
          const float b = ct * 16 + kl < ncol ? q4[ct][j] : 0.0f;
          acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[4 * i + j], b, acc[ct], 0, 0, 0);
        }
    }
#pragma unroll
    for (int ct = 0; ct < G; ++ct) {
      const int colb = ct * 16 + kl;
      if (colb < ncol) {
        const int t = colb % T;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          // key 16 w + 4 kk + q of the chunk sits at sp_pos(key) = q * 16 + 4 w + kk
          const int kloc = 16 * wave + 4 * kk + q, key = key0 + kloc;
          sp[colb * cPStride + q * 16 + 4 * wave + kk] =
              (key < kvlen && key <= past + t) ? __fmul_rn(acc[ct][q], scale) : -INFINITY;
        }
      }
    }
  }
  bar();
  if (prof) wmark(P, 1, 18);
  // 4. chunk softmax per column (one wave per column, lane = key)
  const size_t pi = (size_t)g * P.max_chunks + chunk;
  const Rsrc rml = mk_rsrc(P.part_ml + pi * kMaxCols * 2, kMaxCols * 2 * 4);
  // this wave's columns wave + 4 c (c < NC = 4G): lane (c, j) = (lane / LG,
  // lane % LG), LG = 64 / NC, holds keys j + LG a (a < NC) of column c. The max
  // runs on order-preserving integer keys of the scores (exact in any order; no
  // NaN here; the sign of a zero maximum changes no exp(w - m)). The sum keeps
  // wave_sum_f's pairing over the keys: the partners at xor 32 .. LG sit in the
  // same lane, those at xor LG / 2 .. 1 in lanes j ^ 8 (LG = 16: a row rotation
  // by 8), j ^ 4, j ^ 2, j ^ 1. Probabilities of a column are kept permuted (key
  // 4 s + kk at kk * 16 + s), so that the P.V operands of a lane are 16
  // consecutive floats.
  {
    constexpr int NC = 4 * G, LG = 64 / NC;
    const int c = lane / LG, j = lane % LG, col = wave + 4 * c;
    const bool live = col < ncol;
    float* row = sp + min(col, ncol - 1) * cPStride;
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
    float pv[NC], v[NC];
#pragma unroll
    for (int a = 0; a < NC; ++a) {
      float p = (m == -INFINITY || w[a] == -INFINITY) ? 0.0f : dev_expf(__fsub_rn(w[a], m));
      if (f16kv) p = f16_round(p);
      pv[a] = p;
      v[a] = p;
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
      for (int a = 0; a < NC; ++a) row[sp_key_pos(j + LG * a)] = pv[a];
      if (j == 0) {
        stc1(rml, (uint32_t)((col + col_off) * 2 * 4), m);
        stc1(rml, (uint32_t)(((col + col_off) * 2 + 1) * 4), l);
      }
    }
  }
  bar();
  if (prof) wmark(P, 1, 19);
  // 5. O[col][d] = fma chain over the chunk's keys of p * v
  const Rsrc ro = mk_rsrc(P.part_o + pi * kMaxCols * cHD, kMaxCols * cHD * 4);
  {
    // the 2 G chains (column tile, head_dim tile) run interleaved
    float pa[G][16];
#pragma unroll
    for (int ct = 0; ct < G; ++ct) {
      const int cola = ct * 16 + kl;
      const float* prow = sp + min(cola, ncol - 1) * cPStride + kk * 16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4f p4 = *(const v4f*)(prow + 4 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) pa[ct][4 * i + j] = cola < ncol ? p4[j] : 0.0f;
      }
    }
    v4f acc[G][2];
#pragma unroll
    for (int ct = 0; ct < G; ++ct)
#pragma unroll
      for (int h = 0; h < 2; ++h) acc[ct][h] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; ++s)
#pragma unroll
      for (int ct = 0; ct < G; ++ct)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          acc[ct][h] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[ct][s], vb[h][s], acc[ct][h], 0, 0, 0);
#pragma unroll
    for (int ct = 0; ct < G; ++ct)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int d = 16 * (2 * wave + h) + kl;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = ct * 16 + 4 * kk + q;
          if (col < ncol) stc1(ro, (uint32_t)(((col + col_off) * cHD + d) * 4), acc[ct][h][q]);
        }
      }
  }
  bar();
  if (prof) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); bar(); wmark(P, 1, 20); }
}

// Merge the chunk partials of (q head hq, row t) in chunk order; 128 threads,
// thread = head_dim element d (two waves). The merged row leaves as four q8_0
// blocks (32 lanes each), or (HOUT 1) as f16 values (the f16 o-projection's
// vec_dot_type), two per 4-byte store, or (HOUT 2) as f32 values. valid == false:
// the lanes only take part in the lane exchanges.
template <int HOUT = 0>
__device__ __forceinline__ void merge_item(const StepParams& P, int T, int nch, int hq, int t, int d,
                                           bool valid, bool prof, float* fl) {
  // the item is uniform over each wave (two waves per item): made visibly so, or
  // the buffer descriptors below would sit in vector registers and every load
  // would become a loop over the distinct descriptors
  hq = __builtin_amdgcn_readfirstlane(hq);
  t = __builtin_amdgcn_readfirstlane(t);
  T = __builtin_amdgcn_readfirstlane(T);
  nch = __builtin_amdgcn_readfirstlane(nch);
  valid = __builtin_amdgcn_readfirstlane((int)valid) != 0;
  const int g = hq / 2, col = (hq & 1) * T + t;
  const Rsrc rml = mk_rsrc(P.part_ml + (size_t)g * P.max_chunks * kMaxCols * 2,
                           (uint32_t)P.max_chunks * kMaxCols * 2 * 4);
  const Rsrc ro = mk_rsrc(P.part_o + (size_t)g * P.max_chunks * kMaxCols * cHD,
                          (uint32_t)P.max_chunks * kMaxCols * cHD * 4);
  // Chunk factors once per wave: lane c holds m_c, l_c and f_c = exp(m_c - M),
  // written to this wave's LDS slots (fl[0..63] factors, fl[64..127] sums); every
  // thread then reads them back four chunks at a time (same address in all lanes)
  // while it runs the two chunk-ordered fma chains over its own O values. A fully
  // masked chunk (m = -inf) has f = 0, l = 0 and O = 0, so its fma terms add
  // exact zeros. The first 64 chunks' (m, l) and the first 32 chunks' O are
  // loaded together: one round trip at the usual context lengths.
  const int lane = threadIdx.x & 63;
  float out = 0.0f;
  auto ld_m = [&](int c) {
    return valid && c < nch ? ldc1(rml, (uint32_t)((c * kMaxCols + col) * 2 * 4)) : -INFINITY;
  };
  auto ld_l = [&](int c) {
    return valid && c < nch ? ldc1(rml, (uint32_t)(((c * kMaxCols + col) * 2 + 1) * 4)) : 0.0f;
  };
  float o[32];
  auto ld_o = [&](int b0) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int c = min(b0 + i, nch - 1);
      o[i] = valid ? ldc1(ro, (uint32_t)(((c * kMaxCols + col) * cHD + d) * 4)) : 0.0f;
    }
  };
  float m = ld_m(lane), l = ld_l(lane);
  ld_o(0);
  float M = wave_max_f(m);
  for (int c0 = 64; c0 < nch; c0 += 64) M = fmaxf(M, wave_max_f(ld_m(c0 + lane)));
  if (prof) wmark(P, 1, 23);
  float L = 0.0f, O = 0.0f;
  for (int c0 = 0; c0 < nch; c0 += 64) {
    if (c0 > 0) {
      m = ld_m(c0 + lane);
      l = ld_l(c0 + lane);
    }
    // LDS accesses of one wave execute in order: the reads below see these
    // writes, and the next block's writes follow this block's reads
    fl[lane] = m == -INFINITY ? 0.0f : dev_expf(__fsub_rn(m, M));
    fl[64 + lane] = l;
    const int nb = min(64, nch - c0);
    for (int i0 = 0; i0 < nb; i0 += 32) {
      if (c0 + i0 > 0) ld_o(c0 + i0);
#pragma unroll
      for (int i = 0; i < 32; i += 4) {
        if (i0 + i >= nb) break;
        const v4f f4 = *(const v4f*)(fl + i0 + i);
        const v4f l4 = *(const v4f*)(fl + 64 + i0 + i);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (i0 + i + j >= nb) break;
          L = fmaf(l4[j], f4[j], L);
          O = fmaf(o[i + j], f4[j], O);
        }
      }
    }
  }
  if (prof) wmark(P, 1, 31);
  if (valid) out = __fdiv_rn(O, L);
  if constexpr (HOUT == 2) {
    if (valid) stc1(mk_rsrc(P.o32, kMaxRows * cQN * 4), (uint32_t)((t * cQN + hq * cHD + d) * 4), out);
    return;
  }
  if constexpr (HOUT == 1) {
    // lane d (even) stores elements d and d + 1
    const uint32_t h = (uint32_t)__half_as_ushort(__float2half_rn(out));
    const uint32_t pair = h | (dpp_u<kDppQuadXor1>(h) << 16);
    if (valid && (d & 1) == 0)
      __builtin_amdgcn_raw_buffer_store_b32(pair, mk_rsrc(P.oh, kMaxRows * cQN * 2),
                                            (t * cQN + hq * cHD + d) * 2, 0, 16);
    return;
  }
  // q8_0 blocks of 32 consecutive d (32 lanes of one wave)
  const float amax = group32_max_nonneg(fabsf(out));
  // the codes of d .. d + 3 packed into lane d (d % 4 == 0) with quad permutes:
  // one 4-byte store per four lanes instead of byte stores into shared lines
  const uint32_t code = valid ? q8_code(out, amax) : 0u;
  const uint32_t packed = code | (dpp_u<0x39>(code) << 8) | (dpp_u<kDppQuadXor2>(code) << 16) |
                          (dpp_u<0x93>(code) << 24);
  if (valid) {
    const Rsrc rq = mk_rsrc(P.oq, kMaxRows * cQN);
    const Rsrc rs = mk_rsrc(P.oqs, kMaxRows * (cQN / 32) * 4);
    if ((d & 3) == 0) __builtin_amdgcn_raw_buffer_store_b32(packed, rq, t * cQN + hq * cHD + d, 0, 16);
    if ((d & 31) == 0) stc1(rs, (uint32_t)((t * (cQN / 32) + (hq * cHD + d) / 32) * 4), q8_scale(amax));
  }
}

// ---------------------------------------------------------------- lm_head ---
// Wave-strided tiles of the tied embedding; a tile's 16 block pairs stream
// through a register ring one tile ahead; per tile the canonical 4-slice sums,
// the penalty and 64-bit first-max keys.
template <int G>
__device__ __forceinline__ void lm_head(const StepParams& P, float penalty, bool write_logits, int T,
                                        const uint8_t* pcodes, const float* pscales, uint64_t* s_best) {
  // a called function receives P's fields and T in vector registers: make the
  // tile arithmetic wave-uniform again, or every buffer load with a scalar
  // offset becomes a loop over its distinct values
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  T = __builtin_amdgcn_readfirstlane(T);
  const int V = __builtin_amdgcn_readfirstlane(P.V), n_tiles = V / 16, gw = blockIdx.x * 4 + wave,
            nwaves = gridDim.x * 4;
  const bool pen = penalty > 1.0f;
  const int words = (V + 31) / 32;
  float* const logits = uniform_ptr(P.logits);
  const Rsrc rb = mk_rsrc(uniform_ptr(P.bitmap), (uint32_t)(kMaxRows * words * 4));
  // the penalty bits of a tile's 16 rows share one word per verify row; it is
  // loaded with the tile's first unit and used at its last
  uint32_t pword[G];
#pragma unroll
  for (int cg = 0; cg < G; ++cg) pword[cg] = 0;
  const int srow = ((lane & 15) >> 3) * 16 + 4 * (lane >> 4);
  const v4i zero = {0, 0, 0, 0};
  uint64_t best[G];
#pragma unroll
  for (int cg = 0; cg < G; ++cg) best[cg] = 0;
  const int my_tiles = gw < n_tiles ? (n_tiles - 1 - gw) / nwaves + 1 : 0;
  // The activation panel is the same for every tile: its operands stay in
  // registers (no LDS read, and no LDS latency, per unit).
  v4i pb[cBH][G];
  float pdx[cBH][G];
#pragma unroll
  for (int bp = 0; bp < cBH; ++bp)
#pragma unroll
    for (int cg = 0; cg < G; ++cg) {
      pb[bp][cg] = *(const v4i*)(pcodes + ((size_t)(cg * cBH + bp)) * kPanelUnit + lane * 16);
      pdx[bp][cg] = pscales[(size_t)(cg * cBH + bp) * kScaleStride + (lane & 15)];
    }
  // A ring of one tile of loads in flight per wave: slot bp holds block pair bp
  // of the tile being computed and is refilled with block pair bp of the next
  // tile. Past this wave's last tile a load gets a per-lane offset past the
  // buffer's end (the range check covers the per-lane offset, not the scalar
  // one): zeros, no memory traffic, never used.
  v4i ra[cBH];
  uint2 rs[cBH];
  const Rsrc re = mk_rsrc(uniform_ptr(P.embd), (uint32_t)((size_t)n_tiles * cBH * kUnitBytes));
  auto issue = [&](int ti, int bp) {
    const bool in = ti < my_tiles;
    const int so = in ? ((gw + ti * nwaves) * cBH + bp) * kUnitBytes : 0;
    const uint32_t gone = 0x80000000u;
    ra[bp] = __builtin_bit_cast(
        v4i, __builtin_amdgcn_raw_buffer_load_b128(re, in ? (uint32_t)(lane * 16) : gone, so, 2));
    const v2u sv = __builtin_amdgcn_raw_buffer_load_b64(re, in ? (uint32_t)(1024 + srow * 2) : gone, so, 2);
    rs[bp] = make_uint2(sv.x, sv.y);
  };
#pragma unroll
  for (int bp = 0; bp < cBH; ++bp) issue(0, bp);
  for (int ti = 0; ti < my_tiles; ++ti) {
    const int tile = gw + ti * nwaves;
    if (pen) {
#pragma unroll
      for (int cg = 0; cg < G; ++cg) {
        const int t = min(cg * 8 + (lane & 7), T - 1);
        pword[cg] = __builtin_amdgcn_raw_buffer_load_b32(rb, (t * words + (tile >> 1)) * 4, 0, 16);
      }
    }
    float part[4][G][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int cg = 0; cg < G; ++cg)
#pragma unroll
        for (int q = 0; q < 4; ++q) part[a][cg][q] = 0.0f;
#pragma unroll
    for (int bp = 0; bp < cBH; ++bp) {
      const int sl = bp >> 2;  // the K slice of this block pair
      float dw[4];
      dw[0] = half_bits_to_float((uint16_t)(rs[bp].x & 0xffff));
      dw[1] = half_bits_to_float((uint16_t)(rs[bp].x >> 16));
      dw[2] = half_bits_to_float((uint16_t)(rs[bp].y & 0xffff));
      dw[3] = half_bits_to_float((uint16_t)(rs[bp].y >> 16));
      const v4i a = ra[bp];
      issue(ti + 1, bp);
#pragma unroll
      for (int cg = 0; cg < G; ++cg) {
        const v4i c = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, pb[bp][cg], zero, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) part[sl][cg][q] = fmaf((float)c[q], dw[q] * pdx[bp][cg], part[sl][cg][q]);
      }
    }
#pragma unroll
    for (int cg = 0; cg < G; ++cg)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v = __fadd_rn(__fadd_rn(__fadd_rn(part[0][cg][q], part[1][cg][q]), part[2][cg][q]), part[3][cg][q]);
        v = __fadd_rn(v, dpp_f<kDppRor8>(v));
        part[0][cg][q] = v;
      }
    if ((lane & 15) < 8) {
#pragma unroll
      for (int cg = 0; cg < G; ++cg) {
        const int t = cg * 8 + (lane & 7);
        if (t < T) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int row = tile * 16 + 4 * (lane >> 4) + q;
            float v = part[0][cg][q];
            if (write_logits) gst<float>(logits + (size_t)t * V + row, v);
            if (pen && ((pword[cg] >> (row & 31)) & 1u))
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
  bar();
  if (threadIdx.x < G * 8) {
    uint64_t b = s_best[threadIdx.x];
    for (int wv = 1; wv < 4; ++wv) b = s_best[wv * kMaxRows + threadIdx.x] > b ? s_best[wv * kMaxRows + threadIdx.x] : b;
    st_coh_u64(P.part_keys + (size_t)blockIdx.x * kMaxRows + threadIdx.x, b);
  }
}

// Greedy choice per verify row from the workgroups' best keys, then the longest
// prefix of drafts that matches. Thread i holds workgroup i's keys of every row;
// those loads and the draft tokens' are in flight together. Per row a wave max,
// then the four waves.
template <int G>
__device__ void accept(const uint64_t* part_keys, int32_t tok, StepResult* result, int T, int nwg,
                       uint64_t* s_red, int32_t* s_choice, int32_t* s_tok, int32_t* s_nmatch, uint64_t* timing,
                       int slot) {
  static_assert(kNwg <= kT, "one thread per workgroup's keys");
  T = __builtin_amdgcn_readfirstlane(T);
  nwg = __builtin_amdgcn_readfirstlane(nwg);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const Rsrc rk = mk_rsrc(uniform_ptr(part_keys), (uint32_t)(nwg * kMaxRows * 8));
  constexpr int R = 8 * G;  // rows of this launch's column groups
  uint64_t key[R];
#pragma unroll
  for (int h = 0; h < R / 2; ++h) {
    const v4u q = __builtin_amdgcn_raw_buffer_load_b128(
        rk, (int)threadIdx.x < nwg ? (uint32_t)((threadIdx.x * kMaxRows + 2 * h) * 8) : 0x80000000u, 0, 16);
    key[2 * h] = ((uint64_t)q.y << 32) | q.x;
    key[2 * h + 1] = ((uint64_t)q.w << 32) | q.z;
  }
  if ((int)threadIdx.x < T) s_tok[threadIdx.x] = tok;
  if (timing) { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); if (threadIdx.x == 0) gst<uint64_t>(uniform_ptr(timing) + slot, wall_clock64()); }
#pragma unroll
  for (int t = 0; t < R; ++t) {  // every row slot, so that key[] stays in registers
    const uint64_t b = wave_max_u64(key[t]);
    if (lane == 0) s_red[wave * kMaxRows + t] = b;
  }
  __syncthreads();
  if ((int)threadIdx.x < T) {
    uint64_t b = s_red[threadIdx.x];
    for (int wv = 1; wv < kT / 64; ++wv) b = s_red[wv * kMaxRows + threadIdx.x] > b ? s_red[wv * kMaxRows + threadIdx.x] : b;
    s_choice[threadIdx.x] = (int32_t)(0xffffffffu - (uint32_t)(b & 0xffffffffu));
  }
  __syncthreads();
  if (timing && threadIdx.x == 0) gst<uint64_t>(uniform_ptr(timing) + slot + 1, wall_clock64());
  if (threadIdx.x == 0) {
    int m = 0;
    while (m + 1 < T && s_tok[m + 1] == s_choice[m]) ++m;
    StepResult* r = uniform_ptr(result);
    for (int t = 0; t < kMaxRows; ++t) r->choice[t] = t < T ? s_choice[t] : -1;
    r->n_match = m;
    *s_nmatch = m;
  }
}

// ------------------------------------------------------ f16 and f32 weights ---
// f16 weights (vec_dot_type F16) and f32 weights (vec_dot_type F32) stay in the
// GGUF row layout, [N][K] halves or floats, and the GEMM phases of these row
// variants spread over all 256 workgroups: q|k|v rows 16 w + 4 wave + r (r < 4),
// o-proj and down row 4 w + wave, gate and up rows 12 w + 3 wave + r (r < 3).
// Canonical order (mul_mat_f16 / mul_mat_f32 of the oracle): the activation
// rounded to f16 (f16 weights) or as it is (f32); lane l runs the fma chain from 0
// over elements [l K/64, (l + 1) K/64) (the product of two f16 values is exact in
// f32, and the compiler folds the conversions into v_fma_mix_f32); the 64 lane
// partials of an output meet in LDS and one lane adds them in the pairing of the
// xor butterfly 32, 16, 8, 4, 2, 1. The variants run 8-row steps (T <= 8).
constexpr int kHT = 8;                 // verify-row slots
constexpr int kHP = 68;                // words per partial row in LDS (16-byte reads)
constexpr int cGuRows = cF / kNwg;     // 12 gate and 12 up rows per workgroup
static_assert(cNQKV == 16 * kNwg && cH == 4 * kNwg && cGuRows == 12, "row split of the row variants");

template <int SEG, int NM, int NR, bool F32 = false>
struct HRows {
  v4i w[NM][NR][F32 ? SEG / 4 : SEG / 8];  // the lane's SEG elements of each row, 16 bytes per piece
};

// NR consecutive rows starting at rows[m] (wave-uniform) of each matrix, K = 64 SEG
// elements of 2 (f16) or 4 (F32) bytes: lane l's SEG elements, non-temporal 16-byte
// loads.
template <int SEG, int NM, int NR, bool F32 = false>
__device__ __forceinline__ void h_load(const uint8_t* const (&rows)[NM], HRows<SEG, NM, NR, F32>& g) {
  constexpr int K = SEG * 64, EB = F32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    const Rsrc r = mk_rsrc(rows[m], (uint32_t)(NR * K * EB));
#pragma unroll
    for (int rr = 0; rr < NR; ++rr)
#pragma unroll
      for (int c = 0; c < SEG * EB / 16; ++c)
        g.w[m][rr][c] = __builtin_bit_cast(
            v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(rr * K * EB + lane * SEG * EB + 16 * c), 0, 2));
  }
}

// The NM x NR x T outputs of a wave's rows against the f16 activation rows s_x
// [kHT][K] (LDS). TT verify rows per pass, their NM NR TT chains interleaved (the
// variant has one wave per SIMD: independent chains keep the fma issue busy); the
// activation comes in 8-element pieces, the next piece in flight during the current
// one's chains. Rows from T on in the last pass are computed from stale LDS rows
// and their partials written to slots no sum reads. s_p: this wave's NM NR kHT
// partial rows. Lane j < kHT NR ends with res[m] = output (row j / kHT, verify row
// j % kHT).
// F32: f32 weights and activation rows (each step of a chain one fma of two f32
// values, the oracle's mul_mat_f32); otherwise f16 (exact products).
template <int SEG, int NM, int NR, int TT, bool F32 = false>
__device__ __forceinline__ void h_dots(const HRows<SEG, NM, NR, F32>& g, const void* s_xv, int T, float* s_p,
                                       float (&res)[NM]) {
  constexpr int K = SEG * 64, EB = F32 ? 4 : 2, EP = 16 / EB, NC = SEG / EP;
  static_assert(kHT % TT == 0, "passes of TT rows cover the slots");
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
          if constexpr (F32) {
            wf[m][r][4 * c + q] = __uint_as_float(u);
          } else {
            wf[m][r][8 * c + 2 * q] = half_bits_to_float((uint16_t)u);
            wf[m][r][8 * c + 2 * q + 1] = half_bits_to_float((uint16_t)(u >> 16));
          }
        }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the previous call's partial reads are done
  // lane l's elements of row t: bytes (t K + l SEG) EB
  const uint8_t* xr = (const uint8_t*)s_xv + lane * SEG * EB;
#pragma unroll
  for (int t0 = 0; t0 < kHT; t0 += TT) {
    if (t0 >= T) break;
    float acc[TT][NM][NR];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r) acc[tt][m][r] = 0.0f;
    v4i xa[TT], xb[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) xa[tt] = *(const v4i*)(xr + (t0 + tt) * K * EB);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (c + 1 < NC) {
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) xb[tt] = *(const v4i*)(xr + (t0 + tt) * K * EB + 16 * (c + 1));
      }
      float xf[TT][EP];
#pragma unroll
      for (int tt = 0; tt < TT; ++tt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t u = (uint32_t)xa[tt][q];
          if constexpr (F32) {
            xf[tt][q] = __uint_as_float(u);
          } else {
            xf[tt][2 * q] = half_bits_to_float((uint16_t)u);
            xf[tt][2 * q + 1] = half_bits_to_float((uint16_t)(u >> 16));
          }
        }
#pragma unroll
      for (int e = 0; e < EP; ++e)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
#pragma unroll
          for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < NR; ++r) acc[tt][m][r] = fmaf(wf[m][r][EP * c + e], xf[tt][e], acc[tt][m][r]);
#pragma unroll
      for (int tt = 0; tt < TT; ++tt) xa[tt] = xb[tt];
    }
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < NR; ++r) s_p[((m * NR + r) * kHT + t0 + tt) * kHP + lane] = acc[tt][m][r];
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave's partial writes are done
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    float v[64];
    const v4f* col = (const v4f*)(s_p + ((m * NR) * kHT + lane) * kHP);
    if (lane < NR * kHT && (lane % kHT) < T) {
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

// verify rows per pass of each f16 phase
constexpr int kTTQkv = 4, kTTO = 8, kTTGu = 4, kTTD = 8, kTTLm = 4;

// f16 (F32: f32) rows [T][K] of an exchange buffer (written by other workgroups in
// this launch) into s_x: every device-coherent 16-byte load of the thread issued before
// the first LDS write (one round trip); pieces past the T rows read past the
// range (zeros, no memory traffic) and are not written.
template <int K, bool F32 = false>
__device__ __forceinline__ void stage_h(const void* src, int T, void* s_x) {
  constexpr int EB = F32 ? 4 : 2, NP = kHT * K * EB / 16 / kT;
  const Rsrc r = mk_rsrc(src, (uint32_t)(T * K * EB));
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));  // addresses computed here, not hoisted out of the layer loop
  v4u q[NP];
#pragma unroll
  for (int j = 0; j < NP; ++j) q[j] = __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)((j * kT + tid) * 16), 0, 16);
  const int n = T * K * EB / 16;
#pragma unroll
  for (int j = 0; j < NP; ++j)
    if (j * kT + tid < n) ((v4u*)s_x)[j * kT + tid] = q[j];
  bar();
}

// The residual add of the o-proj / down output of row 4 w + wave: lane t < T holds
// verify row t. The workgroup is the only writer of its 4 columns: after the first
// time they come from its LDS copy xs ([kHT][16], columns 0..3); each row's 4 new
// values leave as one 16-byte store.
__device__ __forceinline__ void resid_h(float v, Rsrc x, int T, float* xs, bool xs_valid) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int col = 4 * blockIdx.x + wave;
  if (lane < T) {
    const float old = xs_valid ? xs[lane * 16 + wave] : ldc1(x, (uint32_t)((lane * cH + col) * 4));
    xs[lane * 16 + wave] = __fadd_rn(old, v);
  }
  bar();
  if ((int)threadIdx.x < T)
    stc4(x, (uint32_t)((threadIdx.x * cH + 4 * blockIdx.x) * 4), *(const v4f*)(xs + threadIdx.x * 16));
  bar();
}

// The tied f16 / f32 lm_head (lm_f16.hpp): the B operands of the final normed rows
// s_x built in LDS (s_b), then wave gw takes 16-row tiles gw, gw + 1,024, .. of the
// embedding's lm_head copy on f32 MFMA; per verify row the workgroup's best key.
template <bool F32>
__device__ __forceinline__ void lm_head_h(const StepParams& P, float penalty, bool write_logits, int T,
                                          const void* s_x, float* s_b, uint64_t* s_best) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  T = __builtin_amdgcn_readfirstlane(T);
  const int V = __builtin_amdgcn_readfirstlane(P.V);
  lm16_stage_b<kT, F32>(s_x, T, s_b);
  bar();
  uint64_t b = lm16_run<32, F32>(uniform_ptr(P.lm_copy), blockIdx.x * 4 + wave, kNwg * 4, V / 16, s_b, T, V,
                                 penalty, uniform_ptr(P.bitmap), write_logits ? uniform_ptr(P.logits) : nullptr);
  // the four lanes of a verify row: m, m + 16, m + 32, m + 48
  uint64_t o = shfl_xor_u64(b, 16);
  b = o > b ? o : b;
  o = shfl_xor_u64(b, 32);
  b = o > b ? o : b;
  if (lane < kHT) s_best[wave * kMaxRows + lane] = b;
  bar();
  if ((int)threadIdx.x < kHT) {
    uint64_t best = s_best[threadIdx.x];
    for (int wv = 1; wv < 4; ++wv) best = s_best[wv * kMaxRows + threadIdx.x] > best ? s_best[wv * kMaxRows + threadIdx.x] : best;
    st_coh_u64(P.part_keys + (size_t)blockIdx.x * kMaxRows + threadIdx.x, best);
  }
}

// ---------------------------------------------------------------- kernel ----
// per column group: the wave slice sums of four tiles, then the SwiGLU block maxima
constexpr size_t kRedBytes = (size_t)4 * 4 * 4 * 64 * 4 + 4 * 16 * 4;
// LDS: the GEMM panel + reduction space, or the attention's q / new rows /
// probabilities (the phases reuse it), then the residual columns of the o-proj /
// down tile ([8G rows][16], kept across phases).
constexpr size_t kAttnLdsBytes =
    ((size_t)kMaxCols * cQStride + 2 * kMaxRows * cQStride + kMaxCols * cPStride + kKvLdsFloats) * 4;
__host__ __device__ constexpr size_t step_lds_x_offset(int G) {
  return ((size_t)G * cBF * (kPanelUnit + 4 * kScaleStride) + kRedBytes * G > kAttnLdsBytes)
             ? (size_t)G * cBF * (kPanelUnit + 4 * kScaleStride) + kRedBytes * G
             : kAttnLdsBytes;
}
// after the residual columns: two row images per wave for the norm panel (8-row
// variant only)
__host__ __device__ constexpr size_t step_lds_stage_offset(int G) {
  return step_lds_x_offset(G) + (size_t)G * 8 * 16 * 4;
}
__device__ __forceinline__ uint32_t ph(int l, int p) { return 2u + (uint32_t)(l * kPhases + p); }

// The step descriptor: the kernel argument, or (DEV) the one in device memory
// that the device-side controller wrote.
template <bool DEV>
__device__ __forceinline__ const StepDesc& step_desc(const StepDesc& arg, const StepDesc* dev);
template <>
__device__ __forceinline__ const StepDesc& step_desc<false>(const StepDesc& arg, const StepDesc*) { return arg; }
template <>
__device__ __forceinline__ const StepDesc& step_desc<true>(const StepDesc&, const StepDesc* dev) { return *dev; }

// LDS of the f16 / f32 variants' GEMM phases (inside the attention's region, before
// the residual columns): a phase's activation rows [kHT][K] (eb bytes per element)
// at 0, then each wave's partial rows (NM NR kHT rows of kHP words); the gate/up
// outputs gathered for their stores at kHgOff; the lm_head's B operands after the
// final rows [kHT][1024].
__host__ __device__ constexpr size_t h_act_bytes(int K, int eb) { return (size_t)kHT * K * eb; }
__host__ __device__ constexpr size_t h_part_bytes(int rows) { return (size_t)rows * kHT * kHP * 4; }
constexpr size_t kHgOff = kAttnLdsBytes - 512;
static_assert(h_act_bytes(cF, 4) + 4 * h_part_bytes(1) <= kHgOff, "f32 down phase inside the attention's region");
static_assert(h_act_bytes(cQN, 4) + 4 * h_part_bytes(1) <= kHgOff, "f32 o-proj phase");
static_assert(h_act_bytes(cH, 4) + 4 * h_part_bytes(6) <= kHgOff, "f32 gate/up phase");
static_assert(h_act_bytes(cH, 4) + 4 * h_part_bytes(4) <= kHgOff, "f32 q|k|v phase");
static_assert(h_act_bytes(cH, 4) + (size_t)kLm16BFloats * 4 <= kAttnLdsBytes, "f32 lm_head");
static_assert(kHT * cGuRows * 4 <= 512, "the gate/up gather");

// The step itself; the kernel below adds the device loop's controller pass. The
// return value matters in workgroup 0 only: true once its acceptance is done.
// WF: 0 q8_0 weights (MFMA panel tiles), 1 f16 and 2 f32 weights (GGUF rows; 8-row
// steps).
template <int G, int KVH, bool PROF, bool DEV, int WF>
__device__ __forceinline__ bool step_body(const StepParams* __restrict__ Pp, const StepDesc& desc_arg,
                                          uint32_t epoch, int mode, const StepDesc* __restrict__ desc_dev,
                                          uint8_t* lds, int& s_ok, uint64_t* s_best, uint64_t* s_red,
                                          int32_t* s_choice, int32_t* s_tok, int32_t* s_nmatch) {
#define MARK(...) do { if constexpr (PROF) mark(__VA_ARGS__); } while (0)
#define WMARK(...) do { if constexpr (PROF) wmark(__VA_ARGS__); } while (0)
  static_assert(WF == 0 || G == 1, "the f16 and f32 variants run 8-row steps");
  constexpr bool F32 = WF == 2;
  constexpr int EB = F32 ? 4 : 2;  // bytes per weight / activation element of the row variants
  const StepParams& P = *Pp;
  const int w = blockIdx.x, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // The step descriptor arrives by value in the kernel arguments (no copy to
  // device memory before the launch). Its fields are read in place; its address
  // is never taken (that would give every thread a private copy).
  const StepDesc& desc = step_desc<DEV>(desc_arg, desc_dev);
  const int T = desc.T, past = desc.past, L = P.L;
  const int nch = (past + T + kChunk - 1) / kChunk, n_items = cNKV * nch;
  uint8_t* pcodes = lds;
  float* pscales = (float*)(lds + (size_t)G * cBF * kPanelUnit);
  float* red = (float*)(lds + (size_t)G * cBF * (kPanelUnit + 4 * kScaleStride));
  float* xs = (float*)(lds + step_lds_x_offset(G));  // this workgroup's residual columns
  float* stg = (float*)(lds + step_lds_stage_offset(G));
  // the f16 / f32 variants' GEMM space: the activation rows, then a phase's partial
  // rows (K, rows of the wave)
  void* s_x = lds;
  auto s_p_for = [&](int K, int rows) { return (float*)(lds + h_act_bytes(K, EB) + wave * h_part_bytes(rows)); };
  uint8_t* s_h = lds + kHgOff;
  bool xs_valid = false;
  Ctl c{&P, epoch, 0, &s_ok};
#define RX mk_rsrc(P.x, kMaxRows * cH * 4)
#define RQKVT mk_rsrc(P.qkvt, kMaxRows * cNQKV * 8)

  // roles
  // Attention items are (kv head, 64-key chunk). Up to 256 items: item i =
  // (head i / nch, chunk i % nch) on workgroup (i + 64) % 256. Beyond that, each
  // kv head has 32 slots of m = ceil(nch / 32) consecutive chunks, slot s =
  // (head s / 32, chunks m (s % 32) ..) on workgroup (s + 64) % 256: the chunks of
  // a workgroup share their q rows (staged once) and each chunk's K / V loads are
  // issued during the previous chunk's arithmetic.
  const int slot = (w + kNwg - 64) % kNwg;
  int att_g, att_c0, att_c1;
  if (n_items <= kNwg) {
    att_g = slot / nch;
    att_c0 = slot % nch;
    att_c1 = att_c0 + 1;
  } else {
    const int m = (nch + 31) / 32;
    att_g = slot / 32;
    att_c0 = (slot % 32) * m;
    att_c1 = min(att_c0 + m, nch);
  }
  bool has_attn = n_items <= kNwg ? slot < n_items : att_c0 < nch;
  // KV append helpers: when 8 workgroups hold no attention item, workgroup
  // (n_items + 64 + g) mod 256 appends kv head g's new rows
  const bool helpers = n_items + cNKV <= kNwg;
  const int help_g = (w - n_items - 64 + 2 * kNwg) % kNwg;
  const bool helper = helpers && help_g < cNKV;
  // split last chunk: when 8 more workgroups are free, kv head g's last chunk (it
  // holds the new keys) runs as two items, q head 2g on its own workgroup and q head
  // 2g + 1 on workgroup (n_items + 72 + g) mod 256
  int att_hsel = -1;
  if (n_items + 2 * cNKV <= kNwg) {
    const int split_g = (w - n_items - 64 - cNKV + 3 * kNwg) % kNwg;
    if (has_attn && att_c0 == nch - 1) att_hsel = 0;
    if (split_g < cNKV) {
      has_attn = true;
      att_g = split_g;
      att_c0 = nch - 1;
      att_c1 = nch;
      att_hsel = 1;
    }
  }
  // chunks run from the last down: the first one staged holds the new rows if any does
  const int att_first = att_c1 - 1;
  const bool att_new = att_c1 * kChunk > past;
  // o-proj and down tiles, gate/up rows 32j..32j+31 (the row variants: every
  // workgroup has rows of all three)
  const bool gu_blk = w >= cOTiles && w < cOTiles + cGuBlocks;
  const bool od = WF ? true : w < cOTiles;
  const bool gu = WF ? true : gu_blk;
  const int n_merge = cNH * T;                    // (head, row) items, in pairs
  // merge pair slots: workgroups 160..255, then the gate/up workgroups (their own
  // phase comes after the o-proj), so that 16 rows need one round, not two
  const int merge_slot = w >= kMergeWg0 ? w - kMergeWg0 : (gu_blk ? kNwg - kMergeWg0 + (w - cOTiles) : -1);
  const bool has_merge = w >= kMergeWg0 || (merge_slot >= 0 && 2 * merge_slot < n_merge);
  // phase mask of this workgroup (bit p = works in phase p)
  const int mask = 1 | (has_attn ? 2 : 0) | (has_merge ? 4 : 0) | (od ? 8 | 32 : 0) | (gu ? 16 : 0);
  auto next_done = [&](int l, int p) -> uint32_t {  // progress after working in phase p of layer l
    for (int q = p + 1; q < kPhases; ++q)
      if (mask & (1 << q)) return ph(l, q) - 1;
    return ph(l, kPhases) - 1;  // next work: the next layer's QKV (or the lm_head)
  };
  MARK(P, 0);

  // registers carried across phases
  v4i qa[4];              // this layer's q|k|v tile slice
  uint2 qs[4];
  v4i ba[16];             // o-proj (8 pairs) then down (12), or gate A|B, up A|B (4 each)
  uint2 bs[16];
  KvRegs kv;              // K / V of the first attention item
  float gq[16], gf[16];   // attn_norm / ffn_norm gains of the lane's 16 elements
  // the f16 / f32 variants' rows: q|k|v, o-proj, gate|up, down
  HRows<16, 1, 4, F32> hqkv;
  HRows<32, 1, 1, F32> ho;
  HRows<16, 2, 3, F32> hgu;
  HRows<48, 1, 1, F32> hd;
  auto h_qkv_load = [&](const LayerDev& Ly) {
    const uint8_t* r[1] = {Ly.wqkv + (size_t)(16 * w + 4 * wave) * cH * EB};
    h_load<16, 1, 4, F32>(r, hqkv);
  };

  // ---- embeddings (and the penalty bitmap) ----
  if (w < T) {
    const int t = w;
    const int k = threadIdx.x * 4;
    v4f e;
    if (desc.use_embeds) {
      e = gld<v4f>(P.embeds + (size_t)t * cH + k);
    } else if constexpr (WF == 2) {
      e = gld<v4f>((const float*)P.embd + (size_t)desc.tokens[t] * cH + k);
    } else if constexpr (WF == 1) {
      const v2u h = gld<v2u>((const uint16_t*)P.embd + (size_t)desc.tokens[t] * cH + k);
      e = v4f{half_bits_to_float((uint16_t)h.x), half_bits_to_float((uint16_t)(h.x >> 16)),
              half_bits_to_float((uint16_t)h.y), half_bits_to_float((uint16_t)(h.y >> 16))};
    } else {
      const int n = desc.tokens[t], tile = n >> 4, r = n & 15;
      const int bk = k >> 5, bp = bk >> 1, par = bk & 1, half = (k >> 4) & 1;
      const uint8_t* unit = P.embd + ((size_t)tile * cBH + bp) * kUnitBytes;
      const uint32_t q4 = gld<uint32_t>(unit + (r + 16 * (2 * par + half)) * 16 + (k & 15));
      const float d = half_bits_to_float(gld<uint16_t>(unit + 1024 + (par * 16 + r) * 2));
#pragma unroll
      for (int i = 0; i < 4; ++i) e[i] = d * (float)(int8_t)(q4 >> (8 * i));
    }
    stc4(RX, (uint32_t)((t * cH + k) * 4), e);
  }
  publish(c, 1);
  // the penalty bitmap is read only by the lm_head: built after the publish (a
  // later publish of this workgroup covers its stores)
  if (w < T) {
    const int t = w;
    if (mode == kStepVerify && desc.penalty > 1.0f) {
      const int words = (P.V + 31) / 32;
      uint32_t* row = P.bitmap + (size_t)t * words;
      for (int i = threadIdx.x; i < words; i += kT) st_coh_u32(row + i, 0u);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __syncthreads();
      const int end = desc.pen_base + t + 1, begin = max(0, end - kPenaltyWindow);
      for (int i = begin + (int)threadIdx.x; i < end; i += kT) {
        const int id = desc.pen_ids[i];
        if (id >= 0 && id < P.V) atomicOr(row + (id >> 5), 1u << (id & 31));
      }
    }
  }
  // prefetch layer 0: q|k|v tile and the first attention item's K / V
  if constexpr (WF != 0) h_qkv_load(layer_at(P, 0));
  else wt_load<4>(layer_at(P, 0).wqkv + (size_t)w * cBH * kUnitBytes, 4 * wave, qa, qs);
  if constexpr (G == 1) gain16_load(layer_at(P, 0).attn_norm, gq);
  if (has_attn) kv_prefetch<KVH>(layer_at(P, 0), P, att_g, att_first * kChunk, past, kv);

  for (int l = 0; l < L; ++l) {
    const LayerDev& Ly = layer_at(P, l);
    // ---- QKV: tile w ----
    if (!wait_all(c, ph(l, kPhQkv) - 1)) return false;
    MARK(P, 3 + 12 * l + 0);
    WMARK(P, l, 0);
    if constexpr (WF != 0) {
      panel_norm<true, WF>(RX, T, gq, P.eps, (uint8_t*)s_x, nullptr, nullptr, stg, nullptr,
                           (PROF && P.timing && l == 1) ? &P : nullptr);
      WMARK(P, l, 25);
      float res[1];
      h_dots<16, 1, 4, kTTQkv, F32>(hqkv, s_x, T, s_p_for(cH, 4), res);
      WMARK(P, l, 26);
      // (value, tag) pairs of rows 16 w + 4 wave + lane / 8, verify row lane % 8
      const int lane = threadIdx.x & 63, t = lane & 7;
      if (lane < 4 * kHT && t < T) {
        const v2u pr = {__float_as_uint(res[0]), c.epoch + ph(l, kPhQkv)};
        __builtin_amdgcn_raw_buffer_store_b64(pr, RQKVT, (t * cNQKV + 16 * w + 4 * wave + (lane >> 3)) * 8, 0, 16);
      }
      bar();
    } else {
      panel_norm<G == 1>(RX, T, gq, P.eps, pcodes, pscales, nullptr, stg, G == 1 ? nullptr : Ly.attn_norm,
                         (PROF && P.timing && l == 1) ? &P : nullptr);
      WMARK(P, l, 25);
      float acc[1][G][4] = {};
      wt_mma<G, 4>(qa, qs, 4 * wave, cBH, pcodes, pscales, acc[0]);
      WMARK(P, l, 26);
      gemm_finish<G, 1, EPI_STORE>(acc, red, RQKVT, cNQKV, w, T, nullptr, false, c.epoch + ph(l, kPhQkv));
    }
    // the attention reads q|k|v by their tags: a workgroup with attention items
    // announces its q|k|v tile together with its attention partials
    if (!has_attn) publish(c, next_done(l, kPhQkv));
    MARK(P, 3 + 12 * l + 1);
    WMARK(P, l, 1);
    if (helper) append_item<G, KVH>(P, Ly, T, past, help_g, c.epoch + ph(l, kPhQkv), lds);
    // ---- ATTN: items of this workgroup ----
    if (has_attn) {
      MARK(P, 3 + 12 * l + 2);
      WMARK(P, l, 2);
      for (int ch = att_first; ch >= att_c0; --ch)
        attn_item<G, KVH>(P, Ly, T, past, att_g, ch, c.epoch + ph(l, kPhQkv), kv, lds, !helpers,
                          PROF && l == 1 && P.timing != nullptr && ch == att_first, ch == att_first, att_new,
                          ch > att_c0 ? ch - 1 : -1, att_hsel);
      publish(c, next_done(l, kPhAttn));
      MARK(P, 3 + 12 * l + 3);
      WMARK(P, l, 3);
    }
    // the o-proj tile's weights: issued after the attention, so that no register
    // holds them through it (the o-proj starts after the merge, well after they land).
    // Row variants: a merge workgroup issues its o-proj and gate/up rows after its
    // merge (loads complete in order: issued first, 64 or 128 KB of rows would hold
    // up the merge's progress polls and partials)
    auto row_loads = [&]() {
      if constexpr (WF != 0) {
        const uint8_t* ro[1] = {Ly.wo + (size_t)(4 * w + wave) * cQN * EB};
        h_load<32, 1, 1, F32>(ro, ho);
        const uint8_t* rg[2] = {Ly.wg + (size_t)(cGuRows * w + 3 * wave) * cH * EB,
                                Ly.wu + (size_t)(cGuRows * w + 3 * wave) * cH * EB};
        h_load<16, 2, 3, F32>(rg, hgu);
        gain16_load(Ly.ffn_norm, gf);
      }
    };
    if (WF != 0 && !has_merge) row_loads();
    if (WF == 0 && od) wt_load<8>(Ly.wo + (size_t)w * cBQ * kUnitBytes, 8 * wave, ba, bs);
    if (WF == 0 && gu) {  // gate / up tiles 2j, 2j + 1 of this layer
      const int j = w - cOTiles;
      wt_load<4>(Ly.wg + (size_t)(2 * j) * cBH * kUnitBytes, 4 * wave, ba, bs);
      wt_load<4>(Ly.wg + (size_t)(2 * j + 1) * cBH * kUnitBytes, 4 * wave, ba + 4, bs + 4);
      wt_load<4>(Ly.wu + (size_t)(2 * j) * cBH * kUnitBytes, 4 * wave, ba + 8, bs + 8);
      wt_load<4>(Ly.wu + (size_t)(2 * j + 1) * cBH * kUnitBytes, 4 * wave, ba + 12, bs + 12);
      if constexpr (G == 1) gain16_load(Ly.ffn_norm, gf);
    }
    // ---- MERGE: (head, row) items, two at a time ----
    if (has_merge) {
      if (!wait_all(c, ph(l, kPhMerge) - 1)) return false;
      WMARK(P, l, 4);
      const int half = threadIdx.x >> 7;
      for (int i0 = 2 * merge_slot; i0 < n_merge; i0 += 2 * kMergeSlots) {
        const int item = i0 + half;
        const bool valid = item < n_merge;
        merge_item<WF>(P, T, nch, valid ? item / T : 0, valid ? item % T : 0, threadIdx.x & 127, valid,
                            PROF && l == 1 && i0 == 2 * merge_slot, (float*)lds + wave * 128);
      }
      WMARK(P, l, 22);
      publish(c, next_done(l, kPhMerge));
      WMARK(P, l, 5);
      if (WF != 0) row_loads();
      if (!gu && l + 1 < L) {  // nothing more in this layer: prefetch the next one
        const LayerDev& Ln = layer_at(P, l + 1);
        wt_load<4>(Ln.wqkv + (size_t)w * cBH * kUnitBytes, 4 * wave, qa, qs);
        if constexpr (G == 1) gain16_load(Ln.attn_norm, gq);
        if (has_attn) kv_prefetch<KVH>(Ln, P, att_g, att_first * kChunk, past, kv);
      }
    }
    // ---- O-proj: x += W_o o ----
    if (od) {
      if (!wait_all(c, ph(l, kPhO) - 1, PROF && l == 1 ? wslot(w, 12) : -1)) return false;
      MARK(P, 3 + 12 * l + 4);
      WMARK(P, l, 6);
      if constexpr (WF != 0) {
        stage_h<cQN, F32>(F32 ? (const void*)P.o32 : (const void*)P.oh, T, s_x);
        WMARK(P, l, 27);
        float res[1];
        h_dots<32, 1, 1, kTTO, F32>(ho, s_x, T, s_p_for(cQN, 1), res);
        WMARK(P, l, 28);
        resid_h(res[0], RX, T, xs, xs_valid);
      } else {
        panel_from_q<cQN, G>(P.oq, P.oqs, T, pcodes, pscales);
        WMARK(P, l, 27);
        float acc[1][G][4] = {};
        wt_mma<G, 8>(ba, bs, 8 * wave, cBQ, pcodes, pscales, acc[0]);
        WMARK(P, l, 28);
        gemm_finish<G, 1, EPI_RESID>(acc, red, RX, cH, w, T, xs, xs_valid);
      }
      xs_valid = true;
      WMARK(P, l, 24);
      publish(c, next_done(l, kPhO));
      MARK(P, 3 + 12 * l + 5);
      WMARK(P, l, 7);
      if constexpr (WF != 0) {
        const uint8_t* rd[1] = {Ly.wd + (size_t)(4 * w + wave) * cF * EB};
        h_load<48, 1, 1, F32>(rd, hd);
      } else {
        wt_load<12>(Ly.wd + (size_t)w * cBF * kUnitBytes, 12 * wave, ba, bs);
      }
      // the next layer's q|k|v tile and attention K / V, so that they are in flight
      // before the down wait (issued after the down phase, the tile's loads would
      // hold up the residual rows of the next q|k|v panel: loads complete in order);
      // the row variants issue them after their gate/up phase
      if (WF == 0 && l + 1 < L) {
        wt_load<4>(layer_at(P, l + 1).wqkv + (size_t)w * cBH * kUnitBytes, 4 * wave, qa, qs);
        if constexpr (G == 1) gain16_load(layer_at(P, l + 1).attn_norm, gq);
        if (has_attn)
          kv_prefetch<KVH>(layer_at(P, l + 1), P, att_g, att_first * kChunk, past, kv);
      }
    }
    // ---- GATE/UP: act = silu(g) * u, as q8_0 blocks ----
    if (gu) {
      if (!wait_all(c, ph(l, kPhGu) - 1, PROF && l == 1 ? wslot(w, 12) : -1)) return false;
      WMARK(P, l, 8);
      if constexpr (WF != 0) {
        panel_norm<true, WF>(RX, T, gf, P.eps, (uint8_t*)s_x, nullptr, nullptr, stg);
        WMARK(P, l, 27);
        float res[2];
        h_dots<16, 2, 3, kTTGu, F32>(hgu, s_x, T, s_p_for(cH, 6), res);
        WMARK(P, l, 28);
        // SwiGLU rows as f16 / f32 (the down projection's vec_dot_type); the
        // workgroup's 12 values of each verify row meet in LDS and leave as three
        // 8-byte (f16) or 16-byte (f32) stores
        const int lane = threadIdx.x & 63, t = lane & 7;
        if (lane < 3 * kHT && t < T) {
          float v = dev_swiglu(res[0], res[1]);
          const int i = t * cGuRows + 3 * wave + (lane >> 3);
          if constexpr (F32) {
            ((float*)s_h)[i] = v;
          } else {
            // the float product first (no fma_mix: one rounding instead of two)
            asm volatile("" : "+v"(v));
            ((uint16_t*)s_h)[i] = __half_as_ushort(__float2half_rn(v));
          }
        }
        bar();
        if ((int)threadIdx.x < 3 * T) {
          const int tt = threadIdx.x / 3, pc = threadIdx.x % 3;
          if constexpr (F32) {
            const v4u v = *(const v4u*)((const float*)s_h + tt * cGuRows + 4 * pc);
            __builtin_amdgcn_raw_buffer_store_b128(v, mk_rsrc(P.a32, kMaxRows * cF * 4),
                                                   (tt * cF + cGuRows * w + 4 * pc) * 4, 0, 16);
          } else {
            const v2u v = *(const v2u*)((const uint16_t*)s_h + tt * cGuRows + 4 * pc);
            __builtin_amdgcn_raw_buffer_store_b64(v, mk_rsrc(P.ah, kMaxRows * cF * 2),
                                                  (tt * cF + cGuRows * w + 4 * pc) * 2, 0, 16);
          }
        }
      } else {
        panel_norm<G == 1>(RX, T, gf, P.eps, pcodes, pscales, nullptr, stg, G == 1 ? nullptr : Ly.ffn_norm);
        WMARK(P, l, 27);
        float acc[4][G][4] = {};
#pragma unroll
        for (int m = 0; m < 4; ++m) wt_mma<G, 4>(ba + 4 * m, bs + 4 * m, 4 * wave, cBH, pcodes, pscales, acc[m]);
        WMARK(P, l, 28);
        gu_finish<G>(acc, red, red + 4 * 4 * G * 4 * 64, P, w - cOTiles, T);
      }
      WMARK(P, l, 24);
      publish(c, next_done(l, kPhGu));
      WMARK(P, l, 9);
      if (l + 1 < L) {
        const LayerDev& Ln = layer_at(P, l + 1);
        if constexpr (WF != 0) h_qkv_load(Ln);
        else wt_load<4>(Ln.wqkv + (size_t)w * cBH * kUnitBytes, 4 * wave, qa, qs);
        if constexpr (G == 1) gain16_load(Ln.attn_norm, gq);
        if (has_attn) kv_prefetch<KVH>(Ln, P, att_g, att_first * kChunk, past, kv);
      }
    }
    // ---- DOWN: x += W_d act ----
    if (od) {
      if (!wait_all(c, ph(l, kPhD) - 1)) return false;
      MARK(P, 3 + 12 * l + 6);
      WMARK(P, l, 10);
      if constexpr (WF != 0) {
        stage_h<cF, F32>(F32 ? (const void*)P.a32 : (const void*)P.ah, T, s_x);
        WMARK(P, l, 29);
        float res[1];
        h_dots<48, 1, 1, kTTD, F32>(hd, s_x, T, s_p_for(cF, 1), res);
        WMARK(P, l, 30);
        resid_h(res[0], RX, T, xs, xs_valid);
      } else {
        panel_from_q<cF, G>(P.aq, P.aqs, T, pcodes, pscales);
        WMARK(P, l, 29);
        float acc[1][G][4] = {};
        wt_mma<G, 12>(ba, bs, 12 * wave, cBF, pcodes, pscales, acc[0]);
        WMARK(P, l, 30);
        gemm_finish<G, 1, EPI_RESID>(acc, red, RX, cH, w, T, xs, xs_valid);
      }
      xs_valid = true;
      publish(c, next_done(l, kPhD));
      MARK(P, 3 + 12 * l + 7);
      WMARK(P, l, 11);
    }
    // workgroups with only q|k|v and attention work
    if (!od && !gu && !has_merge && l + 1 < L) {
      const LayerDev& Ln = layer_at(P, l + 1);
      wt_load<4>(Ln.wqkv + (size_t)w * cBH * kUnitBytes, 4 * wave, qa, qs);
      if constexpr (G == 1) gain16_load(Ln.attn_norm, gq);
      if (has_attn) kv_prefetch<KVH>(Ln, P, att_g, att_first * kChunk, past, kv);
    }
  }

  // ---- final RMSNorm * output_norm, tied lm_head, acceptance ----
  const uint32_t lm = ph(L, 0);
  if (mode != kStepVerify) {
    if (w == 0) {
      if (!wait_all(c, lm - 1)) return false;
      if constexpr (G == 1) gain16_load(P.out_norm, gq);
      panel_norm<G == 1, WF>(RX, T, gq, P.eps, pcodes, pscales, P.hid, stg, G == 1 ? nullptr : P.out_norm);
      MARK(P, 2);
    }
    return false;
  }
  if (!wait_all(c, lm - 1)) return false;
  MARK(P, 3 + 12 * L);
  if constexpr (G == 1) gain16_load(P.out_norm, gq);
  panel_norm<G == 1, WF>(RX, T, gq, P.eps, pcodes, pscales, w == 0 ? P.hid : nullptr, stg,
                         G == 1 ? nullptr : P.out_norm);
  if constexpr (WF != 0)
    lm_head_h<F32>(P, desc.penalty, desc.write_logits != 0, T, s_x, (float*)(lds + h_act_bytes(cH, EB)), s_best);
  else lm_head<G>(P, desc.penalty, desc.write_logits != 0, T, pcodes, pscales, s_best);
  publish(c, lm);
  MARK(P, 4 + 12 * L);
  if (w == 0) {
    if (!wait_all(c, lm)) return false;
    MARK(P, 5 + 12 * L);
    accept<G>(P.part_keys, (int)threadIdx.x < T ? desc.tokens[threadIdx.x] : 0, P.result, T, kNwg, s_red,
              s_choice, s_tok, s_nmatch, PROF ? P.timing : nullptr, 7 + 12 * L);
    MARK(P, 6 + 12 * L);
    return true;
  }
  return false;
#undef MARK
#undef WMARK
#undef RX
#undef RQKVT
}

static_assert(step_lds_stage_offset(1) >= (size_t)kGenLdsIds * 4, "the controller pass stages ids in the step's LDS");

// PROF: the profiled variant (clock marks into P.timing); the production
// variant carries no marks at all (they would cost code size and registers).
// DEV: the descriptor comes from desc_dev (nothing to do once T == 0 there or
// gc.g->done is set); with gc.g, workgroup 0 then runs the device loop's
// controller pass on this step's outcome: the acceptance done, or (the
// workgroup left at a wait that ran out) a failed step, in which case the
// descriptor stays as it is (other workgroups may still read it) and the next
// launches return on g->done.
template <int G, int KVH, bool PROF, bool DEV = false, int WF = 0>
__global__ void __launch_bounds__(kT, 1)
k_step(const StepParams* __restrict__ Pp, const StepDesc desc_arg, uint32_t epoch,
        int mode, const StepDesc* __restrict__ desc_dev, GenCtl gc) {
  extern __shared__ v4i lds_v4[];
  uint8_t* lds = (uint8_t*)lds_v4;
  __shared__ int s_ok;
  __shared__ uint64_t s_best[4 * kMaxRows];
  __shared__ uint64_t s_red[kT];
  __shared__ int32_t s_choice[kMaxRows];
  __shared__ int32_t s_tok[kMaxRows];
  __shared__ int32_t s_nmatch;
  if constexpr (DEV) {
    if (desc_dev->T == 0 || (gc.g && gc.g->done)) return;  // the controller has stopped
  }
  const bool accepted = step_body<G, KVH, PROF, DEV, WF>(Pp, desc_arg, epoch, mode, desc_dev, lds, s_ok, s_best, s_red,
                                                     s_choice, s_tok, &s_nmatch);
  if constexpr (DEV) {
    if (gc.g && blockIdx.x == 0) {
      __syncthreads();
      const GenStepOutcome prev{!accepted, s_choice, s_nmatch};
      gen_ctrl_pass(gc, prev, accepted, (int32_t*)lds, (int*)s_red, (int*)(s_red + 8));
    }
  }
}

}  // namespace

int step_kernel_supported(int hidden, int n_heads, int n_kv_heads, int head_dim, int intermediate,
                          int n_layers, int cus) {
  return hidden == cH && n_heads == cNH && n_kv_heads == cNKV && head_dim == cHD &&
         intermediate == cF && n_layers >= 1 && n_layers <= kStepMaxLayers && cus >= kNwg;
}

int step_kernel_workgroups() { return kNwg; }

uint32_t step_progress_per_step(int n_layers) { return 2u + (uint32_t)(n_layers * kPhases); }

size_t step_lds_bytes(int G) { return step_lds_stage_offset(G) + (G == 1 ? (size_t)8 * kStageFloats * 4 : 0); }

namespace {
// [G - 1][f16 KV][profiled]; the f16- and f32-weight variants (wf 1, 2): 8-row steps only
const void* step_fn(int G, int kv_f16, bool prof, int wf) {
  static const void* fns[2][2][2] = {
      {{(const void*)k_step<1, 0, false>, (const void*)k_step<1, 0, true>},
       {(const void*)k_step<1, 1, false>, (const void*)k_step<1, 1, true>}},
      {{(const void*)k_step<2, 0, false>, (const void*)k_step<2, 0, true>},
       {(const void*)k_step<2, 1, false>, (const void*)k_step<2, 1, true>}}};
  static const void* fns_h[2][2][2] = {
      {{(const void*)k_step<1, 0, false, false, 1>, (const void*)k_step<1, 0, true, false, 1>},
       {(const void*)k_step<1, 1, false, false, 1>, (const void*)k_step<1, 1, true, false, 1>}},
      {{(const void*)k_step<1, 0, false, false, 2>, (const void*)k_step<1, 0, true, false, 2>},
       {(const void*)k_step<1, 1, false, false, 2>, (const void*)k_step<1, 1, true, false, 2>}}};
  if (wf) return G == 1 ? fns_h[wf - 1][kv_f16 ? 1 : 0][prof ? 1 : 0] : nullptr;
  return fns[G - 1][kv_f16 ? 1 : 0][prof ? 1 : 0];
}
// the 8- and 16-row variants that read the descriptor from device memory
const void* step_fn_dev(int G, int kv_f16, int wf) {
  static const void* fns[2][2] = {
      {(const void*)k_step<1, 0, false, true>, (const void*)k_step<1, 1, false, true>},
      {(const void*)k_step<2, 0, false, true>, (const void*)k_step<2, 1, false, true>}};
  static const void* fns_h[2][2] = {
      {(const void*)k_step<1, 0, false, true, 1>, (const void*)k_step<1, 1, false, true, 1>},
      {(const void*)k_step<1, 0, false, true, 2>, (const void*)k_step<1, 1, false, true, 2>}};
  if (wf) return G == 1 ? fns_h[wf - 1][kv_f16 ? 1 : 0] : nullptr;
  return fns[G - 1][kv_f16 ? 1 : 0];
}
}  // namespace

hipError_t prepare_step_kernels() {
  for (int wf = 0; wf < 3; ++wf)
    for (int G = 1; G <= (wf ? 1 : 2); ++G)
      for (int kv = 0; kv < 2; ++kv) {
        for (int prof = 0; prof < 2; ++prof) {
          const hipError_t e = hipFuncSetAttribute(step_fn(G, kv, prof != 0, wf),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)step_lds_bytes(G));
          if (e != hipSuccess) return e;
        }
        const hipError_t e = hipFuncSetAttribute(step_fn_dev(G, kv, wf), hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)step_lds_bytes(G));
        if (e != hipSuccess) return e;
      }
  return hipSuccess;
}

hipError_t launch_step(hipStream_t s, int G, int kv_f16, int wf, const StepParams* P, const StepDesc* desc,
                        uint32_t epoch, int mode, bool profiled, const StepDesc* desc_dev, const GenCtl* gc) {
  // desc: host memory; the launch copies it into the kernel arguments. desc_dev
  // (verify steps of up to 8 G rows): the kernel reads the descriptor there instead.
  if (G < 1 || G > (wf ? 1 : 2) || wf < 0 || wf > 2) return hipErrorInvalidValue;
  GenCtl ctl{};
  if (gc) ctl = *gc;
  void* args[] = {(void*)&P, (void*)desc, (void*)&epoch, (void*)&mode, (void*)&desc_dev, (void*)&ctl};
  if (desc_dev) {
    if (profiled) return hipErrorInvalidValue;
    return hipLaunchKernel(step_fn_dev(G, kv_f16, wf), dim3(kNwg), dim3(kT), args, step_lds_bytes(G), s);
  }
  const size_t lds = step_lds_bytes(G);
  // A plain launch: one workgroup per CU (the kernel's registers and LDS allow
  // no second), so on an idle device the whole grid is resident at once. The
  // cooperative launch guarantees that too, at 15 us more per step. Every wait
  // in the kernel is bounded: if another kernel holds CUs, the late workgroups
  // join when it ends, and a wait that outlasts its bound ends the step with an
  // error instead of a hang.
  return hipLaunchKernel(step_fn(G, kv_f16, profiled, wf), dim3(kNwg), dim3(kT), args, lds, s);
}

}  // namespace mtg
