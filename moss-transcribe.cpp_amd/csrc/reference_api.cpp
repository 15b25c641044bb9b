// reference_api.cpp - the reference's verify-path interfaces (include/mtg_reference.hpp)
// implemented on the C ABI of this library.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>

#include "../../include/mtg_reference.hpp"

namespace mt {

// ---------------------------------------------------------------- decoder ----
GpuDecoder::~GpuDecoder() { mtg_destroy(ctx_); }

bool GpuDecoder::load(const mtg_model_desc& model, int max_seq, int kv_type) {
  mtg_destroy(ctx_);
  ctx_ = nullptr;
  if (mtg_create(&model, max_seq, kv_type, &ctx_) != MTG_OK) return false;
  hidden_ = model.hp.hidden;
  vocab_ = model.hp.vocab;
  return true;
}

int GpuDecoder::hidden() const { return hidden_; }
int GpuDecoder::past_len() const { return mtg_past_len(ctx_); }
int GpuDecoder::remaining() const { return mtg_remaining(ctx_); }
int GpuDecoder::max_seq() const { return ctx_ ? mtg_past_len(ctx_) + mtg_remaining(ctx_) : 0; }
const char* GpuDecoder::last_error() const { return mtg_last_error(ctx_); }
void GpuDecoder::reset() {
  if (ctx_) mtg_rewind(ctx_, 0);  // views are bounded by past_len; stale rows are never read
}
bool GpuDecoder::rewind(int position) { return ctx_ && mtg_rewind(ctx_, position) == MTG_OK; }

// src/cpu_speculative.cpp:19-21: size checks, capacity, then run; batches wider
// than one verify step are appended in steps of MTG_MAX_BATCH rows.
bool GpuDecoder::append(const std::vector<float>& x, int count, std::vector<float>* h) {
  if (!ctx_ || !h || count <= 0 || x.size() != (size_t)count * hidden_ || count > remaining())
    return false;
  h->resize((size_t)count * hidden_);
  for (int r = 0; r < count; r += MTG_MAX_BATCH) {
    const int n = std::min(MTG_MAX_BATCH, count - r);
    if (mtg_append(ctx_, x.data() + (size_t)r * hidden_, n, h->data() + (size_t)r * hidden_))
      return false;
  }
  return true;
}

bool GpuDecoder::prefill(const std::vector<float>& embeds, int S, std::vector<float>* all_hidden) {
  if (!ctx_ || !all_hidden || S <= 0 || embeds.size() < (size_t)S * hidden_) return false;
  all_hidden->resize((size_t)S * hidden_);
  return mtg_prefill(ctx_, embeds.data(), S, all_hidden->data()) == MTG_OK;
}

std::vector<float> GpuDecoder::logits_from_hidden(const std::vector<float>& hidden_row) {
  std::vector<float> out;
  if (!ctx_ || (int)hidden_row.size() < hidden_) return out;
  out.resize(vocab_);
  if (mtg_logits(ctx_, hidden_row.data(), 1, out.data()) != MTG_OK) out.clear();
  return out;
}

std::vector<float> GpuDecoder::decode_one(const std::vector<float>& embed) {
  std::vector<float> hidden;
  if (!append(embed, 1, &hidden)) hidden.clear();
  return hidden;
}

// ----------------------------------------------------------------- policy ----
std::vector<int32_t> cpu_ngram_draft(const std::vector<int32_t>& committed, int maximum) {
  if (maximum <= 0) return {};
  std::vector<int32_t> out((size_t)maximum);
  const int n = mtg_ngram_draft(committed.data(), (int)committed.size(), maximum, out.data());
  out.resize((size_t)n);
  return out;
}

int cpu_greedy_choice(const std::vector<float>& raw, const std::vector<int32_t>& history,
                      float penalty) {
  if (raw.empty()) throw std::runtime_error("empty target logits");
  return mtg_greedy_choice(raw.data(), (int)raw.size(), history.data(), (int)history.size(),
                           penalty);
}

namespace {
// The verify target and hook adaptor of cpu_speculative_generate.
struct HookedTarget {
  GpuDecoder* dec;
  const CpuSpeculativeHooks* hooks;
  int32_t* past;  // the controller's past_len
  int hidden, vocab, before = 0;
  std::vector<float> raw;     // logits of the last kept row (for `committed`)
  std::vector<float> logits;  // all rows of the last verify (only with `committed`)
  bool bad_draft = false;
  // An exception thrown by a hook is held here, the loop is stopped at the next
  // callback that can return an error, and cpu_speculative_generate rethrows it.
  std::exception_ptr error;
};

int32_t hooked_verify(void* self, const int32_t* tokens, int32_t T, const int32_t* history,
                      int32_t n_history, float penalty, int32_t* choice, int32_t* n_match) {
  HookedTarget& h = *(HookedTarget*)self;
  if (h.error) return MTG_ERR_STATE;
  // the controller's logical rewind reaches the context at commit; keep in step
  if (*h.past != h.dec->past_len() && !h.dec->rewind(*h.past)) return MTG_ERR_STATE;
  h.before = *h.past;
  const bool want_hidden = h.hooks && h.hooks->appended;
  const bool want_logits = h.hooks && h.hooks->committed;
  std::vector<float> hid(want_hidden ? (size_t)T * h.hidden : 0);
  h.logits.resize(want_logits ? (size_t)T * h.vocab : 0);
  const int rc = mtg_verify(h.dec->context(), tokens, T, history, n_history, penalty, choice,
                            n_match, want_hidden ? hid.data() : nullptr,
                            want_logits ? h.logits.data() : nullptr);
  if (rc == MTG_OK && want_hidden) {
    try {
      h.hooks->appended(std::vector<int32_t>(tokens, tokens + T), hid);
    } catch (...) {
      h.error = std::current_exception();
      return MTG_ERR_STATE;
    }
  }
  return rc;
}

int32_t hooked_draft(void* user, const int32_t* ids, int32_t n_ids, int32_t budget, int32_t* out) {
  HookedTarget& h = *(HookedTarget*)user;
  std::vector<int32_t> proposal;
  try {
    proposal = h.hooks->draft(std::vector<int32_t>(ids, ids + n_ids), budget);
  } catch (...) {
    h.error = std::current_exception();
    return 0;
  }
  if (proposal.size() > (size_t)budget) proposal.resize((size_t)budget);
  for (int32_t id : proposal)
    if (id < 0 || id >= h.vocab) h.bad_draft = true;
  std::copy(proposal.begin(), proposal.end(), out);
  return (int32_t)proposal.size();
}

void hooked_commit(void* user, const int32_t* ids, int32_t n_ids, int32_t past_len, int32_t stopped) {
  HookedTarget& h = *(HookedTarget*)user;
  // the logical rewind of this step (src/cpu_speculative.cpp:131-135), before the hook
  if (past_len < h.dec->past_len()) h.dec->rewind(past_len);
  if (!h.hooks || !h.hooks->committed || h.error) return;
  const int row = past_len - h.before - 1;  // the last kept row of this step
  if (!h.logits.empty() && row >= 0 && (size_t)(row + 1) * h.vocab <= h.logits.size())
    h.raw.assign(h.logits.begin() + (size_t)row * h.vocab,
                 h.logits.begin() + (size_t)(row + 1) * h.vocab);
  try {
    h.hooks->committed(*h.dec, std::vector<int32_t>(ids, ids + n_ids), h.raw, stopped != 0);
  } catch (...) {
    h.error = std::current_exception();
  }
}
}  // namespace

// src/cpu_speculative.cpp:68-147 on the device decoder.
std::vector<int32_t> cpu_speculative_generate(GpuDecoder& dec, const std::vector<float>& fused,
                                              int seq, int max_new, int eos,
                                              const CpuSpeculativeHooks* hooks, int max_draft) {
  const int hidden = dec.hidden();
  if (!dec.context() || hidden <= 0 || seq <= 0 || max_new <= 0 ||
      fused.size() != (size_t)hidden * seq)
    return {};
  std::vector<float> all_hidden;
  if (!dec.prefill(fused, seq, &all_hidden)) return {};
  if (hooks && hooks->prefilled) hooks->prefilled(all_hidden);
  std::vector<float> last(all_hidden.end() - hidden, all_hidden.end());
  int32_t past = 0;
  HookedTarget h{&dec, hooks, &past, hidden, 0};
  h.raw = dec.logits_from_hidden(last);
  h.vocab = (int)h.raw.size();
  if (h.vocab <= 0) return {};
  const char* penalty_env = std::getenv("MTD_REPETITION_PENALTY");
  float penalty = penalty_env ? (float)std::atof(penalty_env) : 1.0f;
  penalty = std::max(1.0f, std::min(1.5f, penalty));
  const int32_t first = cpu_greedy_choice(h.raw, {}, penalty);
  past = dec.past_len();
  mtg_target target{&h, hooked_verify, &past, dec.max_seq(), h.vocab};
  std::vector<int32_t> ids((size_t)max_new);
  int32_t n = 0;
  const bool own_draft = hooks && hooks->draft;
  const int rc = mtg_speculative_run(&target, first, nullptr, 0, max_new, 0, eos, penalty,
                                     max_draft, own_draft ? hooked_draft : nullptr,
                                     hooked_commit, &h, ids.data(), &n, nullptr);
  // the controller moved `past`; mirror it into the context (a logical rewind)
  if (past <= dec.past_len()) dec.rewind(past);
  if (h.error) std::rethrow_exception(h.error);
  if (rc == MTG_ERR_INVALID && h.bad_draft) throw std::runtime_error("invalid draft token");
  ids.resize((size_t)std::max(0, n));
  return ids;
}

// ------------------------------------------------------------------- q8_0 ----
PackedQ8::~PackedQ8() { mtg_q8_free(device); }

bool PackedQ8::round_trip_exact(const void* ordinary) const {
  if (!device || !ordinary) return false;
  std::vector<uint8_t> back((size_t)n * (k / 32) * 34);
  if (mtg_q8_unpack(device, back.data()) != MTG_OK) return false;
  return std::memcmp(back.data(), ordinary, back.size()) == 0;
}

bool cpu_exact_q8_supported() {
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return false;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
}

std::unique_ptr<PackedQ8> cpu_pack_q8(const void* blocks, int k, int n) {
  mtg_q8_packed* dev = nullptr;
  if (mtg_q8_pack(blocks, k, n, &dev) != MTG_OK) return nullptr;
  auto p = std::make_unique<PackedQ8>();
  p->k = k;
  p->n = n;
  p->device = dev;
  return p;
}

bool cpu_decode_mul_mat(const PackedQ8* packed, const float* x_dev, int T, float* y_dev) {
  return packed && packed->device && mtg_q8_mul_mat_dev(packed->device, x_dev, T, y_dev) == MTG_OK;
}

// ---------------------------------------------------------------- context ----
namespace {
std::atomic<uint64_t> g_built{0}, g_executed{0};
}

bool cpu_causal_context(const float* v, const float* p, int head_dim, int kv_heads, int heads,
                        int queries, int kv_len, float* out) {
  const int rc = mtg_causal_context_dev(v, p, head_dim, kv_heads, heads, queries, kv_len, out);
  if (rc == MTG_ERR_UNSUPPORTED) return false;
  g_built.fetch_add(1, std::memory_order_relaxed);
  if (rc != MTG_OK) return false;
  g_executed.fetch_add(1, std::memory_order_relaxed);
  return true;
}

CpuContextCounts cpu_causal_context_counts() {
  return {g_built.load(std::memory_order_relaxed), g_executed.load(std::memory_order_relaxed)};
}

}  // namespace mt
