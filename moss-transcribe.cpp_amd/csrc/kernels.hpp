// kernels.hpp - launch wrappers of the gfx950 kernels (defined in kernels.hip).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "gen_ctrl.hpp"
#include "mtg_internal.hpp"

namespace mtg {

// Error text of the calls without a context (mtg_last_error(NULL)).
void set_call_error(const std::string& msg);
// Device tiles and shape of a packed q8_0 matrix.
const uint8_t* q8_packed_view(const mtg_q8_packed* p, int* k, int* n);

// Activation panel of one GEMM input (B operand, see mtg_internal.hpp).
struct Panel {
  uint8_t* codes;  // [group][pair][1024]
  float* scales;   // [group][pair][16]
};

struct KvLayer {
  void* k;  // [kv_head][max_seq][head_dim]
  void* v;
  int f16;
  int max_seq;
};

// Activation of a GEMM whose weights are f16 or q4_K (kernels_wt.hip): the
// rows as f16 [16][K], or the q8_K blocks of the rows.
struct ActQ8K {
  int8_t* qs;      // [16][K]
  float* d;        // [16][K/256]
  int32_t* bsums;  // [16][K/16]
};
struct WtAct {
  uint16_t* f16h;  // [16][K] f16 bits
  ActQ8K q8k;
  float* f32;  // [16][K] the rows as they are (f32 weights)
};

struct AttnWork {
  float* part_ml;  // [kv_head][split][group][16 cols][2]
  float* part_o;   // [kv_head][split][group][16 cols][head_dim]
};

// x[t] = embeddings of desc->tokens (or the uploaded rows when desc->use_embeds).
void launch_embed(hipStream_t s, const StepDesc* desc, const uint8_t* embd_tiles, int hidden,
                  const float* host_rows, float* x);
// panel <- q8_0(RMSNorm(src) * gain) (gain == nullptr: quantize src as is);
// normed_out (nullable) receives the f32 normalized rows.
void launch_norm_quant(hipStream_t s, const StepDesc* desc, const float* src, int K,
                       const float* gain, float eps, Panel panel, float* normed_out);
// out[t][n] = W . x[t] for all rows of a packed matrix (epilogue: store).
void launch_gemm_store(hipStream_t s, int G, const StepDesc* desc, const uint8_t* w, int n, int k,
                       Panel x, float* out);
// x[t][n] += W . act[t] (o-proj and down-proj with residual).
void launch_gemm_residual(hipStream_t s, int G, const StepDesc* desc, const uint8_t* w, int n, int k,
                          Panel x, float* resid);
// act[t][n] = silu(gate . x) * (up . x).
void launch_gemm_swiglu(hipStream_t s, int G, const StepDesc* desc, const uint8_t* wg, const uint8_t* wu,
                        int n, int k, Panel x, float* act);
// q/k per-head RMSNorm + NEOX RoPE (host-built table), K/V append at past.
void launch_qk_rope_append(hipStream_t s, const StepDesc* desc, const float* qkv, int n_heads,
                           int n_kv_heads, const float* q_norm, const float* k_norm, float eps,
                           const float* rope, float* q_out, KvLayer kv);
// Launch attributes of the per-op kernels (the chunk attention's LDS); once per
// context, before any launch or graph capture.
hipError_t prepare_kernels();
hipError_t prepare_kernels_wt();  // the same for the f16 / q4_K weight kernels
void launch_attention(hipStream_t s, const StepDesc* desc, const float* q, int n_heads,
                      int n_kv_heads, KvLayer kv, AttnWork work, Panel o_panel, float* o_out);
// The chunk half of launch_attention: (m, l, o) partials of every (kv head, chunk)
// into work; attn_max_chunks is the chunk capacity of the cache (work's stride).
void launch_attn_chunks(hipStream_t s, const StepDesc* desc, const float* q, int n_heads, int n_kv_heads,
                        KvLayer kv, AttnWork work);
int attn_max_chunks(const KvLayer& kv);
void launch_penalty_bitmap(hipStream_t s, const StepDesc* desc, int vocab, uint32_t* bitmap);
void launch_lm_head(hipStream_t s, int G, const StepDesc* desc, const uint8_t* w, int vocab, int k,
                    Panel x, const uint32_t* bitmap, float* logits, uint64_t* part_keys);
void launch_accept(hipStream_t s, const StepDesc* desc, const uint64_t* part_keys,
                   StepResult* result);
// kernel-level entry points
void launch_causal_context(hipStream_t s, const float* v, const float* p, int head_dim,
                           int kv_heads, int heads, int queries, int kv_len, float* out);
void launch_q8_retile(hipStream_t s, const uint8_t* blocks, int n, int k, uint8_t* tiles);

// ---- prompt prefill over S rows (prefill.hip); activations in the compact
// q8_0 layout codes [S][K] int8 + scales [S][K/32] ----
enum { PF_EPI_STORE = 0, PF_EPI_RESID = 1, PF_EPI_SWIGLU = 2, PF_EPI_BIAS = 3, PF_EPI_BIAS_GELU = 4,
       PF_EPI_BIAS_SILU = 5, PF_EPI_BIAS_RESID = 6 };
int pf_max_context();  // positions the prefill attention supports
hipError_t prepare_kernels_pf();
// RMSNorm(src) * gain (hidden 1024) -> q8_0 codes / scales; normed_out (nullable)
void launch_pf_norm_quant(hipStream_t s, const float* src, int S, const float* gain, float eps, int8_t* codes,
                          float* scales, float* normed_out);
void launch_pf_quant(hipStream_t s, const float* src, int S, int K, int8_t* codes, float* scales);
// out[s][n] (= / += / swiglu with w2) q8_0 GEMM of packed tiles (N % 64 == 0)
// epi: PF_EPI_*; bias [N] for the PF_EPI_BIAS* epilogues (out = act(W x + b),
// or out += W x + b)
void launch_pf_gemm(hipStream_t s, int epi, const uint8_t* w, const uint8_t* w2, int N, int K, const int8_t* codes,
                    const float* scales, int S, float* out, const float* bias = nullptr);
void launch_pf_qk_rope(hipStream_t s, const float* qkv, int S, int past0, int n_heads, int n_kv_heads,
                       const float* q_norm, const float* k_norm, float eps, const float* rope, float* q_out,
                       KvLayer kv);
// ofl == nullptr: the output rows as q8_0 codes / scales; otherwise as f32 rows in ofl
void launch_pf_attn(hipStream_t s, const float* q, int n_heads, int n_kv_heads, KvLayer kv, int past0, int S,
                    int8_t* ocodes, float* oscales, float* ofl = nullptr);
// ---- the block prefill for f16 / q4_K weights (prefill_wt.hip); activations
// [S][K] f16 or q8_K blocks in act (the compact layouts of WtAct, S rows) ----
// act <- the weight type's vec_dot_type of RMSNorm(src) * gain (gain == nullptr:
// src as is), S rows of K
void launch_pf_act_wt(hipStream_t s, int wtype, const float* src, int S, int K, const float* gain, float eps,
                      const WtAct& act);
// out[s][n] (= / += / swiglu with w2, or the encoder's bias epilogues PF_EPI_BIAS*)
// for f16 or q4_K weights in the GGUF row layout
void launch_pf_gemm_wt(hipStream_t s, int wtype, int epi, const uint8_t* w, const uint8_t* w2, int N, int K,
                       const WtAct& act, int S, float* out, const float* bias = nullptr);
// the K this GEMM takes: f16 and f32 1,024 / 2,048 / 3,072 / 4,096; q4_K any multiple of 256
int pf_gemm_wt_supported(int wtype, int K);

// ---- f16 / q4_K weights (kernels_wt.hip); weights in the GGUF row layout ----
bool wt_shape_supported(int wtype, int k);
// act <- the weight type's vec_dot_type of RMSNorm(src) * gain (gain == nullptr:
// src as is); normed_out (nullable) receives the f32 normalized rows.
void launch_act_wt(hipStream_t s, int wtype, const StepDesc* desc, const float* src, int K,
                   const float* gain, float eps, const WtAct& act, float* normed_out);
// The merge half of the attention for f16 / q4_K weights: the attention output
// rows go straight to the o-projection's vec_dot_type in act.
void launch_attn_combine_wt(hipStream_t s, int wtype, const StepDesc* desc, AttnWork work, int n_heads,
                            int max_chunks, const WtAct& act);
// epi 0: out = W act, 1: out += W act, 2: out = silu(W act) * (W2 act)
// f16 weights, K = 1024, EPI 0 or 2: out = W (RMSNorm(x) * gain), the norm computed
// in the GEMM (the activation k_act_f16 would write, without its launch)
void launch_gemm_f16_norm(hipStream_t s, int epi, const StepDesc* desc, const uint8_t* w, const uint8_t* w2, int n,
                          const float* x, const float* gain, float eps, float* out);
void launch_gemm_wt(hipStream_t s, int wtype, int epi, const StepDesc* desc, const uint8_t* w,
                    const uint8_t* w2, int n, int k, const WtAct& act, float* out);
// w: the embedding as uploaded; for f16 weights, and f32 with k == 1024, its lm_head
// copy (launch_lm16_retile)
void launch_lm_head_wt(hipStream_t s, int wtype, const StepDesc* desc, const uint8_t* w, int vocab, int k,
                       const WtAct& act, const uint32_t* bitmap, float* logits, uint64_t* part_keys);
// The lm_head's copy of an f16 or f32 embedding [vocab][1024] (vocab % 16 == 0, the
// copy under 2 GiB): 16-row tiles in the MFMA operand order (lm_f16.hpp).
void launch_lm16_retile(hipStream_t s, int wtype, const uint8_t* embd, int vocab, uint8_t* out);
void launch_embed_wt(hipStream_t s, int wtype, const StepDesc* desc, const uint8_t* w, int hidden,
                     const float* host_rows, float* x);

// ---- the speculative controller on the device (generate.hip) ----
// One controller pass (gen_ctrl.hpp) as its own launch: commit a pending step's
// result from res_map (the mapped result buffer the step kernel writes; step_err:
// its error word), apply the stop rules, draft and write the next descriptor
// (T = 0 once stopped). A device loop runs it once, before its first step.
void launch_gen_ctrl(hipStream_t s, const GenCtl& c, const StepResult* res_map, const int32_t* step_err);

}  // namespace mtg
