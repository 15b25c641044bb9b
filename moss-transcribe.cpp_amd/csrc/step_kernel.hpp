// step_kernel.hpp - the persistent verify-step kernel (step_kernel.hip).
#pragma once

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#include "gen_ctrl.hpp"
#include "mtg_internal.hpp"

namespace mtg {

enum { kStepVerify = 0, kStepAppend = 1 };

// One decoder layer's device tensors.
struct LayerDev {
  const uint8_t *wqkv, *wo, *wg, *wu, *wd;  // q8_0 MFMA panel tiles, or f16 rows [N][K]
  const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
  uint8_t *kc, *vc;                          // KV cache of the layer
};

// Layers the step kernel's parameter block holds.
constexpr int kStepMaxLayers = 48;
// KV length beyond which f16-weight steps take the per-op kernels by default:
// there the persistent kernel's attention (one workgroup per CU, each walking 2+
// chunks in turn) falls behind the per-op one (three workgroups per CU). Measured
// on MI355X at 8 rows, f16 KV: 1,024 keys 1,044 vs 1,228 us, 3,072 1,216 vs 1,316,
// 5,120 1,393 vs 1,406, 6,144 1,505 vs 1,453, 8,000 1,533 vs 1,516.
constexpr int kStepF16MaxKeys = 5120;
// The same for f32 weights, where the row streams weigh more against attention:
// the persistent kernel won at every measured length (1,024 keys 1,533 vs 1,875
// us, 5,120 1,875 vs 2,047, 6,144 1,985 vs 2,094, 8,000 2,014 vs 2,149); the
// limit is the longest measured length.
constexpr int kStepF32MaxKeys = 8192;
// Default wait bounds: 2^23 polls, 50 ms.
constexpr uint32_t kWaitPolls = 1u << 23;
constexpr uint32_t kWaitTicks = 5000000u;

// Constant for a context; lives in device memory.
struct StepParams {
  int H, NH, NKV, F, V, L, max_seq, kv_f16, max_chunks;
  float eps;
  // The layer table sits inside the block: the kernel reads the block through a
  // const restrict argument, so these pointers come in with scalar loads.
  LayerDev layer[kStepMaxLayers];
  const uint8_t* embd;
  const uint8_t* lm_copy;  // f16 / f32 weights: the lm_head's copy of embd (lm_f16.hpp)
  const float* out_norm;
  const float* rope;
  const float* embeds;  // host rows uploaded for append
  float *x, *qkv, *o, *act, *hid, *logits;
  float *part_ml, *part_o;  // [kv head][chunk][col][2] and [kv head][chunk][col][head_dim]
  // q8_0 activations exchanged between phases: o (merge -> o-proj) and the
  // SwiGLU output (gate/up -> down): codes [16][K] and f16-valued scales [16][K/32]
  int8_t *oq, *aq;
  float *oqs, *aqs;
  // the same two activations as f16 rows [16][K] (f16 weights) or f32 rows (f32)
  uint16_t *oh, *ah;
  float *o32, *a32;
  uint32_t* bitmap;
  uint64_t* part_keys;      // [nwg][16]
  StepResult* result;
  uint32_t* flags;          // [nwg][kFlagStride] progress words, one per 128-byte line
  // q|k|v of the step's rows as (value bits, tag) pairs, [16][4096][2]: the tag is
  // the progress value of the phase that wrote it, so a reader needs no flag
  uint32_t* qkvt;
  int32_t* err;             // raised by a wait that ran out (inside *result)
  // bounds of every wait: polls, and device-clock ticks (100 MHz) measured from
  // the wait's 256th poll, checked every 256 polls
  uint32_t wait_polls, wait_ticks;
  uint64_t* timing;         // nullable: phase clock marks (profiling)
};

// The Qwen3-0.6B verify step as one persistent dataflow kernel (256
// workgroups with fixed, prefetching roles; step_kernel.hip). Progress words
// advance by step_progress_per_step per launch.
int step_kernel_supported(int hidden, int n_heads, int n_kv_heads, int head_dim, int intermediate,
                          int n_layers, int cus);
int step_kernel_workgroups();
// Words between two workgroups' progress words: each word owns a 128-byte line,
// so a publish does not contend with the polls of its neighbours' words.
constexpr int kFlagStride = 32;
uint32_t step_progress_per_step(int n_layers);
size_t step_lds_bytes(int G);
hipError_t prepare_step_kernels();
// wf: the weight variant, 0 q8_0, 1 f16, 2 f32 (1 and 2: G == 1 only). desc: the host copy of the
// step descriptor (passed by value as a kernel argument). profiled: the variant
// that writes clock marks into StepParams::timing.
// desc_dev: the variant that reads the descriptor from device memory (a device
// loop); with gc, its workgroup 0 then runs the controller pass on the step's
// outcome (gen_ctrl.hpp), and the launch returns at once once gc->g->done is set.
hipError_t launch_step(hipStream_t s, int G, int kv_f16, int wf, const StepParams* P, const StepDesc* desc,
                        uint32_t epoch, int mode, bool profiled, const StepDesc* desc_dev = nullptr,
                        const GenCtl* gc = nullptr);

}  // namespace mtg
