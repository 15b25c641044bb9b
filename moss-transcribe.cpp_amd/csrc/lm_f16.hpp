// lm_f16.hpp - the tied lm_head of f16 and f32 weights (hidden 1024) on f32 MFMA,
// in the canonical order of the oracle's mul_mat_f16 / mul_mat_f32: the activation
// rounded to f16 (f16 weights) or as it is (f32); K in 64 segments of 16 consecutive
// elements, each an fma chain from 0 in element order; the 64 partials of an output
// added in the pairing of the xor butterfly 32, 16, 8, 4, 2, 1. v_mfma_f32_16x16x4f32 returns fma(a3, b3, fma(a2, b2,
// fma(a1, b1, fma(a0, b0, c)))) per output, so four chained MFMAs from a zero
// accumulator are one segment's chain for 16 weight rows x 16 verify rows. The
// segments run in 6-bit bit-reversed order, so the butterfly's tree is the balanced
// binary tree over the run, folded as it goes with a stack of six partials.
// Used by the per-op kernel (kernels_wt.hip) and the lm_head of the step kernel's
// f16 and f32 variants (step_kernel.hip); the weights come from a copy of the
// embedding re-tiled once at load time (k_lm16_retile, k_lm32_retile) so that every
// lane's 16-byte load is its MFMA operands.
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.hpp"

namespace mtg {
namespace dev {

typedef unsigned int lm16_u4 __attribute__((ext_vector_type(4)));

// The re-tiled copy: tile i (rows 16 i .. 16 i + 15 of [V][1024]) in pieces of 1 KB;
// lane (m, kk) = (lane % 16, lane / 16) of a piece holds 16 bytes. f16: 32 pieces,
// piece q holds run positions o = 2 q and 2 q + 1 (segment l = bitrev6(o), elements
// 16 l .. 16 l + 15), for each of its two segments the four halves 16 l + 4 s + kk,
// s < 4, of row 16 i + m (the A operand of the segment's MFMA k-steps s). f32: 64
// pieces, piece o holds run position o, the four floats 16 l + 4 s + kk.
constexpr int kLm16PieceBytes = 1024;
template <bool F32>
struct LmTile {
  static constexpr int kPieces = F32 ? 64 : 32, kSegsPerPiece = F32 ? 1 : 2;
  static constexpr int kBytes = kPieces * kLm16PieceBytes;
};
constexpr int kLm16Pieces = LmTile<false>::kPieces, kLm16TileBytes = LmTile<false>::kBytes;
// The activation's B operands in LDS: [64 run positions][64 lanes][4] floats, lane
// (t, kk) = (lane % 16, lane / 16) of position o holding x[t][16 bitrev6(o) + 4 s + kk]
// (s < 4), zeros for t >= T.
constexpr int kLm16BFloats = 64 * 64 * 4;

__host__ __device__ constexpr int lm16_bitrev6(int k) {
  return ((k & 1) << 5) | ((k & 2) << 3) | ((k & 4) << 1) | ((k & 8) >> 1) | ((k & 16) >> 3) | ((k & 32) >> 5);
}

// B operands of the activation rows x [T][1024] (LDS or global, T <= 16; f16 values,
// or F32: f32 values), by NT threads.
template <int NT, bool F32 = false>
__device__ __forceinline__ void lm16_stage_b(const void* x, int T, float* s_b) {
  for (int idx = threadIdx.x; idx < 64 * 64; idx += NT) {
    const int o = idx >> 6, ln = idx & 63, t = ln & 15, kk = ln >> 4, l = lm16_bitrev6(o);
    v4f v = {0.f, 0.f, 0.f, 0.f};
    if (t < T) {
      const int e0 = t * 1024 + 16 * l + kk;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        v[s] = F32 ? ((const float*)x)[e0 + 4 * s] : half_bits_to_float(((const uint16_t*)x)[e0 + 4 * s]);
    }
    *(v4f*)(s_b + idx * 4) = v;
  }
}

// The lm_head over tiles first, first + stride, .. (< n_tiles) of one wave: a ring of
// RING pieces in flight (16 or 32, a divisor of the tile's pieces; a lone wave per
// SIMD needs the deeper one); per tile the 64 segment chains, the tree, then per
// output (row 16 i + 4 kk + r, verify row t = lane % 16 < T) the logit (written when
// logits != nullptr), the repetition penalty (bitmap word of the tile's 16 rows,
// loaded one tile ahead; device-coherent, it may come from this launch) and the
// 64-bit first-max key. Returns the lane's best key (verify row lane % 16; 0 for the
// lanes of rows >= T).
template <int RING, bool F32 = false>
__device__ __forceinline__ uint64_t lm16_run(const uint8_t* w, int first, int stride, int n_tiles, const float* s_b,
                                             int T, int V, float penalty, const uint32_t* bitmap, float* logits) {
  const int lane = threadIdx.x & 63, m = lane & 15, kk = lane >> 4;
  const int my = first < n_tiles ? (n_tiles - 1 - first) / stride + 1 : 0;
  using LT = LmTile<F32>;
  constexpr int NPC = LT::kPieces;
  const auto rw = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(w), 0,
                                                    (int)((uint32_t)n_tiles * LT::kBytes), 0x00020000);
  const bool pen = penalty > 1.0f;
  const int words = (V + 31) / 32;
  const auto rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(bitmap), 0, (int)(kMaxRows * words * 4),
                                                    0x00020000);
  // piece gi = NPC i + q of this wave's run; past the last tile: an offset past the
  // range (zeros, no memory traffic)
  auto issue = [&](int gi) -> lm16_u4 {
    const int i = gi / NPC, q = gi % NPC;
    const uint32_t off = i < my ? (uint32_t)((first + i * stride) * NPC + q) * kLm16PieceBytes +
                                      (uint32_t)lane * 16u
                                : 0x80000000u;
    return __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 2);
  };
  auto pword = [&](int i) -> uint32_t {
    const bool in = pen && i < my && m < T;
    return __builtin_amdgcn_raw_buffer_load_b32(
        rb, in ? (uint32_t)((m * words + (((first + i * stride) * 16) >> 5)) * 4) : 0x80000000u, 0, 16);
  };
  lm16_u4 ring[RING];
#pragma unroll
  for (int p = 0; p < RING; ++p) ring[p] = issue(p);
  uint32_t pw = pword(0);
  uint64_t best = 0;
  for (int i = 0; i < my; ++i) {
    const uint32_t pw_cur = pw;
    pw = pword(i + 1);
    // the B operands are the same for every tile: an offset opaque to the compiler
    // keeps their 64 LDS reads inside the loop (hoisted, they would hold 256
    // registers across it and spill)
    int bo = lane * 4;
    asm volatile("" : "+v"(bo));
    v4f stk[6], res = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int lvl = 0; lvl < 6; ++lvl) stk[lvl] = res;
    // fold run position o into the stack: while bit lvl of o is set, the left
    // sibling (the earlier subtree) is added; the first clear bit keeps the partial
    auto fold = [&](int o, v4f cur) {
      bool carry = true;
#pragma unroll
      for (int lvl = 0; lvl < 6; ++lvl) {
        if (carry) {
          if ((o >> lvl) & 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e) cur[e] = __fadd_rn(stk[lvl][e], cur[e]);
          } else {
            stk[lvl] = cur;
            carry = false;
          }
        }
      }
      if (carry) res = cur;  // o == 63: the root
    };
    // B operands one piece ahead (an LDS read waited for at once would stall a lone
    // wave on every piece); a piece's results are folded during the next piece's
    // MFMAs (p0, p1), so that the adds do not wait for the MFMA pipe. f32: one
    // segment per piece, the pieces taken in pairs (the same two chains).
    v4f nb0 = *(const v4f*)(s_b + bo), nb1 = *(const v4f*)(s_b + 256 + bo);
    v4f p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0;
#pragma unroll
    for (int q = 0; q < 32; ++q) {
      lm16_u4 wv0, wv1;
      if constexpr (F32) {
        wv0 = ring[(2 * q) % RING];
        ring[(2 * q) % RING] = issue(NPC * i + 2 * q + RING);
        wv1 = ring[(2 * q + 1) % RING];
        ring[(2 * q + 1) % RING] = issue(NPC * i + 2 * q + 1 + RING);
      } else {
        wv0 = ring[q % RING];
        ring[q % RING] = issue(NPC * i + q + RING);
        wv1 = wv0;
      }
      const v4f b0 = nb0, b1 = nb1;
      if (q + 1 < 32) {
        nb0 = *(const v4f*)(s_b + (2 * q + 2) * 256 + bo);
        nb1 = *(const v4f*)(s_b + (2 * q + 3) * 256 + bo);
      }
      __builtin_amdgcn_sched_barrier(0);  // the reads above go out before the MFMAs
      // run positions 2q, 2q + 1: their MFMA chains interleaved (two independent
      // chains keep the MFMA pipe busy)
      v4f c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        float a0, a1;
        if constexpr (F32) {
          a0 = __uint_as_float(wv0[st]);
          a1 = __uint_as_float(wv1[st]);
        } else {
          const uint32_t u[4] = {wv0.x, wv0.y, wv0.z, wv0.w};
          a0 = half_bits_to_float((uint16_t)(u[st >> 1] >> (16 * (st & 1))));
          a1 = half_bits_to_float((uint16_t)(u[2 + (st >> 1)] >> (16 * (st & 1))));
        }
        c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0[st], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1[st], c1, 0, 0, 0);
      }
      if (q > 0) {
        fold(2 * q - 2, p0);
        fold(2 * q - 1, p1);
      }
      p0 = c0;
      p1 = c1;
      // the folds happen here: the stack passes through an empty asm after every
      // piece (without it the adds, free of any ordering, were sunk below the
      // tile's last MFMA, keeping every segment's result live and spilling)
#pragma unroll
      for (int lvl = 0; lvl < 6; ++lvl)
#pragma unroll
        for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(stk[lvl][e]));
      __builtin_amdgcn_sched_barrier(0);
    }
    fold(62, p0);
    fold(63, p1);
    if (m < T) {
      const int tile = first + i * stride;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * tile + 4 * kk + r;
        float v = res[r];
        if (logits) logits[(size_t)m * V + row] = v;
        if (pen && ((pw_cur >> (row & 31)) & 1u)) v = v > 0.0f ? __fdiv_rn(v, penalty) : __fmul_rn(v, penalty);
        const uint64_t key = argmax_key(v, row);
        best = key > best ? key : best;
      }
    }
  }
  return best;
}

}  // namespace dev
}  // namespace mtg
