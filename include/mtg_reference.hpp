// mtg_reference.hpp - the reference's verify-path interfaces, ggml-free, on libmtg.
//
// moss-transcribe.cpp declares the speculative path in three headers whose
// signatures carry ggml types (src/cpu_speculative.hpp:7-17, src/cpu_q8.hpp:13-27,
// src/cpu_context.hpp:7-13) and a decoder class (src/qwen3_decoder.hpp:28-79).
// This header keeps their names, argument meaning and error behaviour in
// namespace mt, with ggml tensors replaced by host vectors or device pointers and
// the decoder backed by one gfx950 context of libmtg (include/mtg_verify.h):
//   * cpu_ngram_draft / cpu_greedy_choice / CpuSpeculativeHooks /
//     cpu_speculative_generate: same semantics; cpu_greedy_choice throws on empty
//     logits, cpu_speculative_generate returns {} when it cannot start and throws
//     std::runtime_error on an invalid draft token, as the reference does.
//   * GpuDecoder: the public part of Qwen3Decoder (load, prefill, decode_one,
//     logits_from_hidden, reset, past_len, hidden) plus the verify batch the
//     reference reaches only through its friend CpuSpeculativeDecoder.
//   * PackedQ8 / cpu_pack_q8 / cpu_decode_mul_mat: the packed q8_0 GEMM on device
//     pointers; unsupported shapes return null / false so the caller keeps its own
//     path, as the reference's nullptr does.
//   * cpu_causal_context / cpu_causal_context_counts: the valid-length context on
//     device pointers; false (the reference's nullptr) for unsupported layouts.
#ifndef MTG_REFERENCE_HPP
#define MTG_REFERENCE_HPP

#include <cstdint>
#include <functional>
#include <memory>
#include <vector>

#include "mtg_verify.h"

namespace mt {

// ---- src/qwen3_decoder.hpp:28-79 ----
class GpuDecoder {
 public:
  GpuDecoder() = default;
  ~GpuDecoder();
  GpuDecoder(const GpuDecoder&) = delete;
  GpuDecoder& operator=(const GpuDecoder&) = delete;

  // Upload the model and allocate a KV cache of max_seq positions (kv_type
  // MTG_TYPE_F32, the reference's cache type, or MTG_TYPE_F16).
  bool load(const mtg_model_desc& model, int max_seq, int kv_type = MTG_TYPE_F32);
  int hidden() const;
  // reset + run S rows; all_hidden receives S x hidden final-normed rows.
  bool prefill(const std::vector<float>& embeds, int S, std::vector<float>* all_hidden);
  std::vector<float> logits_from_hidden(const std::vector<float>& hidden_row);
  std::vector<float> decode_one(const std::vector<float>& embed);
  void reset();
  int past_len() const;
  int max_seq() const;
  // CpuSpeculativeDecoder::append / rewind / remaining (src/cpu_speculative.cpp:17-26)
  bool append(const std::vector<float>& x, int count, std::vector<float>* h);
  bool rewind(int position);
  int remaining() const;
  mtg_ctx* context() const { return ctx_; }
  const char* last_error() const;

 private:
  mtg_ctx* ctx_ = nullptr;
  int hidden_ = 0, vocab_ = 0;
};

// ---- src/cpu_speculative.hpp:7-17 ----
std::vector<int32_t> cpu_ngram_draft(const std::vector<int32_t>& committed, int maximum);
int cpu_greedy_choice(const std::vector<float>& raw, const std::vector<int32_t>& history,
                      float penalty);
struct CpuSpeculativeHooks {
  std::function<std::vector<int32_t>(const std::vector<int32_t>&, int)> draft;
  std::function<void(const std::vector<float>&)> prefilled;
  // inputs (seed + drafts) and their final-normed hidden rows
  std::function<void(const std::vector<int32_t>&, const std::vector<float>&)> appended;
  // decoder, committed ids, logits of the last kept row, whether a stop rule fired
  std::function<void(GpuDecoder&, const std::vector<int32_t>&, const std::vector<float>&, bool)>
      committed;
};
// The reference reads the repetition penalty from MTD_REPETITION_PENALTY
// (clamped to [1, 1.5]) and fixes the draft width at 4 (src/cpu_speculative.cpp:
// 85-86,104); both are the defaults here. The loop guard needs the tokenizer and
// is not part of this path.
std::vector<int32_t> cpu_speculative_generate(GpuDecoder& dec, const std::vector<float>& fused,
                                              int seq, int max_new, int eos,
                                              const CpuSpeculativeHooks* hooks = nullptr,
                                              int max_draft = 4);

// ---- src/cpu_q8.hpp:13-27 ----
struct PackedQ8 {
  int k = 0, n = 0;
  mtg_q8_packed* device = nullptr;  // MFMA panel tiles in HBM
  // Packing is lossless: the tiles hold exactly the q8_0 blocks it was given.
  bool round_trip_exact(const void* ordinary) const;
  ~PackedQ8();
};
bool cpu_exact_q8_supported();
// blocks: n rows of k as ggml block_q8_0 (the ggml_tensor of the reference).
std::unique_ptr<PackedQ8> cpu_pack_q8(const void* blocks, int k, int n);
// y_dev[t][n] = the packed rows . x_dev[t] for T rows (q8_0 activations);
// false for an unsupported batch (the reference: eager ggml fallback).
bool cpu_decode_mul_mat(const PackedQ8* packed, const float* x_dev, int T, float* y_dev);

// ---- src/cpu_context.hpp:7-13 ----
bool cpu_causal_context(const float* values_dev, const float* probabilities_dev, int head_dim,
                        int kv_heads, int heads, int queries, int kv_len, float* out_dev);
struct CpuContextCounts {
  uint64_t built, executed;
};
CpuContextCounts cpu_causal_context_counts();

}  // namespace mt

#endif
