// capi.cpp - the extern "C" boundary and the speculative generation controller.
//
// Every entry point catches all exceptions and reports through an int status and
// the context's error text, as moss_transcribe_capi.cpp:80-94 does for the
// product API.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <memory>
#include <new>
#include <set>
#include <vector>

#include "kernels.hpp"
#include "runtime.hpp"

using mtg::Ctx;

namespace {

constexpr int kProfileSlots = MTG_PROFILE_SLOTS;
thread_local std::string g_create_error;

double seconds_since(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}
}  // namespace

extern "C" {

int mtg_abi_version(void) { return MTG_ABI_VERSION; }

int mtg_create(const mtg_model_desc* desc, int32_t max_seq, int32_t kv_type, mtg_ctx** out) {
  if (!out) return MTG_ERR_INVALID;
  *out = nullptr;
  if (!desc || !desc->layers || !desc->token_embd || !desc->output_norm) return MTG_ERR_INVALID;
  try {
    auto* c = new (std::nothrow) mtg_ctx();
    if (!c) return MTG_ERR_NOMEM;
    const int rc = c->impl.init(desc, max_seq, kv_type);
    if (rc) {
      g_create_error = c->impl.error;
      delete c;
      return rc;
    }
    *out = c;
    return MTG_OK;
  } catch (...) {
    return MTG_ERR_NOMEM;
  }
}

void mtg_destroy(mtg_ctx* ctx) { delete ctx; }

const char* mtg_last_error(const mtg_ctx* ctx) {
  return ctx ? ctx->impl.error.c_str() : g_create_error.c_str();
}

int mtg_set_exec_mode(mtg_ctx* ctx, int32_t mode) {
  if (!ctx || mode < MTG_EXEC_STEP_KERNEL || mode > MTG_EXEC_EAGER) return MTG_ERR_INVALID;
  if (mode == MTG_EXEC_STEP_KERNEL && !ctx->impl.step_ok)
    return ctx->impl.fail(MTG_ERR_UNSUPPORTED, "persistent step kernel unavailable for this shape");
  ctx->impl.exec = mode;
  return MTG_OK;
}

int32_t mtg_exec_mode(const mtg_ctx* ctx) { return ctx ? ctx->impl.exec : -1; }

int mtg_set_step_max_keys(mtg_ctx* ctx, int32_t max_keys) {
  if (!ctx) return MTG_ERR_INVALID;
  ctx->impl.step_max_keys = max_keys > 0 ? max_keys : 0;
  return MTG_OK;
}

int64_t mtg_step_kernel_runs(const mtg_ctx* ctx) { return ctx ? ctx->impl.step_runs : 0; }

int mtg_step_profile(mtg_ctx* ctx, int32_t enable) {
  if (!ctx) return MTG_ERR_INVALID;
  Ctx& c = ctx->impl;
  if (!c.step_ok) return c.fail(MTG_ERR_UNSUPPORTED, "no step kernel");
  if (enable && !c.timing_dev) {
    c.timing_dev = (uint64_t*)c.dalloc(sizeof(uint64_t) * kProfileSlots, true);
    if (!c.timing_dev) return c.fail(MTG_ERR_NOMEM, "timing buffer");
  }
  c.params_host.timing = enable ? c.timing_dev : nullptr;
  return hipMemcpy(c.params_dev, &c.params_host, sizeof(c.params_host), hipMemcpyHostToDevice) == hipSuccess
             ? MTG_OK
             : MTG_ERR_DEVICE;
}

int mtg_launch_timing(mtg_ctx* ctx, int32_t enable) {
  if (!ctx) return MTG_ERR_INVALID;
  Ctx& c = ctx->impl;
  if (enable && !c.ev_start) {
    if (int rc = c.check(hipEventCreate(&c.ev_start), "event")) return rc;
    if (int rc = c.check(hipEventCreate(&c.ev_stop), "event")) return rc;
  }
  c.timing = enable != 0;
  c.timing_ms = 0.0;
  c.timing_launches = c.timing_past = c.timing_rows = 0;
  return MTG_OK;
}

int mtg_launch_timing_read(const mtg_ctx* ctx, double* total_ms, int64_t* launches,
                           int64_t* past_sum, int64_t* rows_sum) {
  if (!ctx || !total_ms || !launches || !past_sum || !rows_sum) return MTG_ERR_INVALID;
  const Ctx& c = ctx->impl;
  *total_ms = c.timing_ms;
  *launches = c.timing_launches;
  *past_sum = c.timing_past;
  *rows_sum = c.timing_rows;
  return MTG_OK;
}

int32_t mtg_step_profile_read(mtg_ctx* ctx, uint64_t* marks, int32_t n) {
  if (!ctx || !marks || !ctx->impl.timing_dev) return 0;
  const int count = std::min<int>(n, kProfileSlots);
  if (hipMemcpy(marks, ctx->impl.timing_dev, sizeof(uint64_t) * count, hipMemcpyDeviceToHost) != hipSuccess)
    return 0;
  return count;
}

int mtg_debug_abort_next_step(mtg_ctx* ctx) {
  if (!ctx) return MTG_ERR_INVALID;
  if (!ctx->impl.step_ok) return ctx->impl.fail(MTG_ERR_UNSUPPORTED, "no step kernel");
  ctx->impl.abort_next = true;
  return MTG_OK;
}

int mtg_debug_wait_limit(mtg_ctx* ctx, int32_t polls) {
  if (!ctx) return MTG_ERR_INVALID;
  Ctx& c = ctx->impl;
  if (!c.step_ok) return c.fail(MTG_ERR_UNSUPPORTED, "no step kernel");
  c.params_host.wait_polls = polls > 0 ? (uint32_t)polls : mtg::kWaitPolls;
  return c.check(hipMemcpy(c.params_dev, &c.params_host, sizeof(c.params_host), hipMemcpyHostToDevice),
                 "step params");
}

int64_t mtg_step_fallbacks(const mtg_ctx* ctx) { return ctx ? ctx->impl.step_fallbacks : 0; }

int mtg_debug_copy(mtg_ctx* ctx, int32_t which, void* out, size_t bytes) {
  if (!ctx || !out) return MTG_ERR_INVALID;
  const Ctx& c = ctx->impl;
  const int R = mtg::kMaxRows, H = c.hp.hidden, QN = c.hp.n_heads * c.hp.head_dim,
            KN = c.hp.n_kv_heads * c.hp.head_dim, F = c.hp.intermediate;
  const void* src = nullptr;
  size_t size = 0;
  switch (which) {
    case MTG_DEBUG_X: src = c.x; size = (size_t)R * H * 4; break;
    case MTG_DEBUG_QKV: src = c.qkv; size = (size_t)R * (QN + 2 * KN) * 4; break;
    case MTG_DEBUG_O: src = c.obuf; size = (size_t)R * QN * 4; break;
    case MTG_DEBUG_ACT: src = c.act; size = (size_t)R * F * 4; break;
    case MTG_DEBUG_HIDDEN: src = c.hid; size = (size_t)R * H * 4; break;
    default: return MTG_ERR_INVALID;
  }
  if (bytes < size) return MTG_ERR_INVALID;
  return hipMemcpy(out, src, size, hipMemcpyDeviceToHost) == hipSuccess ? MTG_OK : MTG_ERR_DEVICE;
}

int32_t mtg_past_len(const mtg_ctx* ctx) { return ctx ? ctx->impl.past : 0; }
int32_t mtg_remaining(const mtg_ctx* ctx) { return ctx ? ctx->impl.max_seq - ctx->impl.past : 0; }

// CpuSpeculativeDecoder::rewind (src/cpu_speculative.cpp:22-24): logical only;
// positions >= past_len are never read again before being rewritten.
int mtg_rewind(mtg_ctx* ctx, int32_t position) {
  if (!ctx) return MTG_ERR_INVALID;
  if (position < 0 || position > ctx->impl.past)
    return ctx->impl.fail(MTG_ERR_STATE, "invalid rewind to %d (past_len %d)", position, ctx->impl.past);
  ctx->impl.past = position;
  return MTG_OK;
}

int mtg_embed(mtg_ctx* ctx, const int32_t* ids, int32_t n, float* out) {
  if (!ctx) return MTG_ERR_INVALID;
  try {
    return ctx->impl.embed(ids, n, out);
  } catch (...) {
    return ctx->impl.fail(MTG_ERR_DEVICE, "embed: exception");
  }
}

int mtg_append(mtg_ctx* ctx, const float* embeds, int32_t T, float* hidden_out) {
  if (!ctx) return MTG_ERR_INVALID;
  try {
    return ctx->impl.append(embeds, T, hidden_out);
  } catch (...) {
    return ctx->impl.fail(MTG_ERR_DEVICE, "append: exception");
  }
}

int mtg_prefill(mtg_ctx* ctx, const float* embeds, int32_t S, float* hidden_out) {
  if (!ctx) return MTG_ERR_INVALID;
  try {
    return ctx->impl.prefill(embeds, S, hidden_out);
  } catch (...) {
    return ctx->impl.fail(MTG_ERR_DEVICE, "prefill: exception");
  }
}

int mtg_prefill_mode(mtg_ctx* ctx, int32_t blocks) {
  if (!ctx) return MTG_ERR_INVALID;
  ctx->impl.prefill_fast_enabled = blocks != 0;
  return MTG_OK;
}

double mtg_last_prefill_ms(const mtg_ctx* ctx) { return ctx ? ctx->impl.last_prefill_ms : 0.0; }

int mtg_logits(mtg_ctx* ctx, const float* hidden, int32_t T, float* logits_out) {
  if (!ctx) return MTG_ERR_INVALID;
  try {
    return ctx->impl.logits_of(hidden, T, logits_out);
  } catch (...) {
    return ctx->impl.fail(MTG_ERR_DEVICE, "logits: exception");
  }
}

int mtg_verify(mtg_ctx* ctx, const int32_t* tokens, int32_t T, const int32_t* history,
               int32_t n_history, float penalty, int32_t* choice_out, int32_t* n_match_out,
               float* hidden_out, float* logits_out) {
  if (!ctx) return MTG_ERR_INVALID;
  try {
    return ctx->impl.verify(tokens, T, history, n_history, penalty, choice_out, n_match_out,
                            hidden_out, logits_out);
  } catch (...) {
    return ctx->impl.fail(MTG_ERR_DEVICE, "verify: exception");
  }
}

int mtg_kv_write(mtg_ctx* ctx, const void* k, const void* v, int32_t n_pos) {
  if (!ctx) return MTG_ERR_INVALID;
  return ctx->impl.kv_io(const_cast<void*>(k), const_cast<void*>(v), n_pos, true);
}

int mtg_kv_read(mtg_ctx* ctx, void* k, void* v, int32_t n_pos) {
  if (!ctx) return MTG_ERR_INVALID;
  return ctx->impl.kv_io(k, v, n_pos, false);
}

// cpu_ngram_draft (src/cpu_speculative.cpp:27-38).
int32_t mtg_ngram_draft(const int32_t* h, int32_t size, int32_t maximum, int32_t* out) {
  if (!h || !out || maximum <= 0 || size < 3) return 0;
  for (int n = std::min<int>(16, size - 1); n >= 2; --n)
    for (int start = size - n - 1; start >= 0; --start)
      if (std::equal(h + size - n, h + size, h + start)) {
        const int begin = start + n, count = std::min<int>(maximum, size - begin);
        std::copy(h + begin, h + begin + count, out);
        return count;
      }
  return 0;
}

// cpu_greedy_choice (src/cpu_speculative.cpp:39-50).
int32_t mtg_greedy_choice(const float* raw, int32_t n, const int32_t* history, int32_t nh,
                          float penalty) {
  if (!raw || n <= 0) return -1;
  auto value = [&](int i) { return raw[i]; };
  if (!(penalty > 1.0f)) {
    int best = 0;
    for (int i = 1; i < n; ++i)
      if (value(i) > value(best)) best = i;
    return best;
  }
  std::vector<float> adj(raw, raw + n);
  std::set<int32_t> recent;
  for (int i = std::max(0, nh - 100); i < nh; ++i) recent.insert(history[i]);
  for (int32_t id : recent)
    if (id >= 0 && id < n) adj[id] = adj[id] > 0 ? adj[id] / penalty : adj[id] * penalty;
  int best = 0;
  for (int i = 1; i < n; ++i)
    if (adj[i] > adj[best]) best = i;
  return best;
}

// The loop of cpu_speculative_generate (src/cpu_speculative.cpp:89-137) over any
// verify target. Differences from the reference: the draft width is a parameter
// (the reference fixes 4, :104) and a target returns the greedy choice of every
// row at once (the device computes all T logits rows in one lm_head pass)
// instead of one lazily computed row at a time (:118-130); the emitted ids, the
// kept KV rows, the rewinds and the counters are the same.
int mtg_speculative_run(const mtg_target* tg, int32_t first_seed, const int32_t* prior_ids,
                        int32_t n_prior, int32_t max_new, int32_t max_steps, int32_t eos,
                        float penalty, int32_t max_draft, mtg_draft_fn draft,
                        mtg_commit_fn commit, void* user, int32_t* ids_out, int32_t* n_ids_out,
                        mtg_gen_stats* stats) {
  if (!tg || !tg->verify || !tg->past || !ids_out || !n_ids_out || max_new <= 0 || n_prior < 0 ||
      first_seed < 0 || first_seed >= tg->vocab)
    return MTG_ERR_INVALID;
  try {
    penalty = std::max(1.0f, std::min(1.5f, penalty));  // :85-86
    max_draft = std::max(0, std::min(max_draft, MTG_MAX_BATCH - 1));
    std::vector<int32_t> ids(prior_ids, prior_ids + (prior_ids ? n_prior : 0));
    const size_t first_new = ids.size();
    ids.reserve(first_new + (size_t)max_new);
    mtg_gen_stats st{};
    int stop = 0;
    auto emit = [&](int32_t id) {  // :90-98 (the loop guard needs the tokenizer)
      ids.push_back(id);
      if (id == eos) stop = 1;
      else if ((int)(ids.size() - first_new) >= max_new) stop = 2;
    };
    int32_t proposal[MTG_MAX_BATCH], choice[MTG_MAX_BATCH], inputs[MTG_MAX_BATCH];
    int32_t raw_choice = first_seed;
    int steps = 0, rc = MTG_OK;
    while (!stop) {
      if (max_steps > 0 && steps >= max_steps) break;
      const int32_t seed = raw_choice;
      emit(seed);
      if (stop) {
        if (commit) commit(user, ids.data(), (int)ids.size(), *tg->past, 1);
        break;
      }
      const int before = *tg->past;
      if (tg->max_seq - before < 1) {
        // no room for the seed's row: the reference's append fails and its loop
        // breaks with the seed emitted (src/cpu_speculative.cpp:113-114)
        stop = 3;
        break;
      }
      const int budget = std::max(0, std::min({max_draft, max_new - (int)(ids.size() - first_new),
                                               tg->max_seq - before - 1}));
      auto t0 = std::chrono::steady_clock::now();
      int np = draft ? draft(user, ids.data(), (int)ids.size(), budget, proposal)
                     : mtg_ngram_draft(ids.data(), (int)ids.size(), budget, proposal);
      st.draft_seconds += seconds_since(t0);
      np = std::max(0, std::min(np, budget));
      for (int i = 0; i < np; ++i)
        if (proposal[i] < 0 || proposal[i] >= tg->vocab) rc = MTG_ERR_INVALID;  // :108
      if (rc) break;
      inputs[0] = seed;
      std::copy(proposal, proposal + np, inputs + 1);
      int32_t n_match = 0;
      t0 = std::chrono::steady_clock::now();
      // row i's penalty window: ids before the seed ++ inputs[0..i]
      rc = tg->verify(tg->self, inputs, np + 1, ids.data(), (int)ids.size() - 1, penalty, choice,
                      &n_match);
      st.verify_seconds += seconds_since(t0);
      if (rc) break;
      *tg->past = before + np + 1;
      ++steps;
      ++st.target_calls;
      st.drafted_calls += np > 0;
      st.proposed += np;
      st.target_input_tokens += np + 1;
      int keep = 1;
      raw_choice = choice[0];
      for (int i = 0; i < np && i < n_match; ++i) {
        ++st.accepted;
        emit(proposal[i]);
        if (stop) break;  // the terminating token is emitted, not kept (:128)
        ++keep;
        raw_choice = choice[i + 1];
      }
      const int position = before + keep;
      if (*tg->past != position) {  // :131-135
        *tg->past = position;
        ++st.rewinds;
      }
      if (commit) commit(user, ids.data(), (int)ids.size(), *tg->past, stop != 0);
    }
    st.stop_reason = stop;
    st.next_seed = raw_choice;
    const int n_new = (int)(ids.size() - first_new);
    std::copy(ids.begin() + first_new, ids.end(), ids_out);
    *n_ids_out = n_new;
    if (stats) *stats = st;
    return rc;
  } catch (...) {
    return MTG_ERR_NOMEM;
  }
}

namespace {

int32_t ctx_verify(void* self, const int32_t* tokens, int32_t T, const int32_t* history,
                   int32_t n_history, float penalty, int32_t* choice_out, int32_t* n_match_out) {
  // Ctx::verify advances past by T itself; the controller sets it again.
  return ((Ctx*)self)->verify(tokens, T, history, n_history, penalty, choice_out, n_match_out,
                              nullptr, nullptr);
}
}  // namespace

int mtg_generate_from(mtg_ctx* ctx, int32_t first_seed, const int32_t* prior_ids, int32_t n_prior,
                      int32_t max_new, int32_t max_steps, int32_t eos, float penalty,
                      int32_t max_draft, mtg_draft_fn draft, mtg_commit_fn commit, void* user,
                      int32_t* ids_out, int32_t* n_ids_out, mtg_gen_stats* stats) {
  if (!ctx) return MTG_ERR_INVALID;
  Ctx& c = ctx->impl;
  if (!ids_out || !n_ids_out || max_new <= 0 || first_seed < 0 || first_seed >= c.hp.vocab)
    return c.fail(MTG_ERR_INVALID, "generate: bad arguments");
  mtg_target tg{&c, ctx_verify, &c.past, c.max_seq, c.hp.vocab};
  c.error.clear();
  const int rc = mtg_speculative_run(&tg, first_seed, prior_ids, n_prior, max_new, max_steps, eos,
                                     penalty, max_draft, draft, commit, user, ids_out, n_ids_out,
                                     stats);
  if (rc && c.error.empty()) c.fail(rc, "generate: invalid draft token or argument");
  return rc;
}

int mtg_generate_device(mtg_ctx* ctx, int32_t first_seed, const int32_t* prior_ids, int32_t n_prior,
                        int32_t max_new, int32_t max_steps, int32_t eos, float penalty, int32_t max_draft,
                        int32_t* ids_out, int32_t* n_ids_out, mtg_gen_stats* stats) {
  return mtg_generate_device_stream(ctx, first_seed, prior_ids, n_prior, max_new, max_steps, eos, penalty, max_draft,
                                    nullptr, ids_out, n_ids_out, stats);
}

int mtg_generate_device_stream(mtg_ctx* ctx, int32_t first_seed, const int32_t* prior_ids, int32_t n_prior,
                               int32_t max_new, int32_t max_steps, int32_t eos, float penalty, int32_t max_draft,
                               const mtg_stream_drafter* drafter, int32_t* ids_out, int32_t* n_ids_out,
                               mtg_gen_stats* stats) {
  if (!ctx) return MTG_ERR_INVALID;
  Ctx& c = ctx->impl;
  if (!ids_out || !n_ids_out || max_new <= 0 || n_prior < 0 || (n_prior > 0 && !prior_ids) || first_seed < 0 ||
      first_seed >= c.hp.vocab)
    return c.fail(MTG_ERR_INVALID, "generate_device: bad arguments");
  for (int i = 0; i < n_prior; ++i)
    if (prior_ids[i] < 0 || prior_ids[i] >= c.hp.vocab) return c.fail(MTG_ERR_INVALID, "prior id %d", prior_ids[i]);
  if (drafter && (drafter->n_prompt < 0 || drafter->period < 0 || (drafter->n_prompt > 0 && !drafter->prompt) ||
                  (drafter->period > 0 && !drafter->stream)))
    return c.fail(MTG_ERR_INVALID, "generate_device: bad stream drafter");
  if (drafter) {
    for (int i = 0; i < drafter->n_prompt; ++i)
      if (drafter->prompt[i] < 0 || drafter->prompt[i] >= c.hp.vocab)
        return c.fail(MTG_ERR_INVALID, "drafter prompt id %d", drafter->prompt[i]);
    for (int i = 0; i < drafter->period; ++i)
      if (drafter->stream[i] < 0 || drafter->stream[i] >= c.hp.vocab)
        return c.fail(MTG_ERR_INVALID, "drafter stream id %d", drafter->stream[i]);
  }
  c.error.clear();
  try {
    mtg::GenState g{};
    g.first_new = n_prior;
    g.max_new = max_new;
    g.max_steps = max_steps;
    g.eos = eos;
    g.max_draft = std::max(0, std::min(max_draft, MTG_MAX_BATCH - 1));  // :85-86
    g.max_seq = c.max_seq;
    g.penalty = std::max(1.0f, std::min(1.5f, penalty));
    g.n_ids = n_prior;
    g.past = c.past;
    g.raw_choice = first_seed;
    g.n_prompt = drafter ? drafter->n_prompt : 0;
    g.period = drafter ? drafter->period : 0;
    // room for the prior ids and every id the run can emit: max_new, or fewer
    // when a step limit bounds the run (each step emits at most max_draft + 1)
    int64_t most = max_new;
    if (max_steps > 0) most = std::min<int64_t>(most, (int64_t)max_steps * (g.max_draft + 1));
    const int cap = n_prior + (int)most + 1;
    // the controller kernel packs positions of prompt ++ ids into 26 bits
    if ((int64_t)g.n_prompt + cap >= (1 << 26))
      return c.fail(MTG_ERR_INVALID, "generate_device: prompt and ids exceed 2^26 positions");
    std::unique_ptr<int32_t[]> ids(new int32_t[(size_t)cap]);  // not cleared: only written ids are read
    std::copy(prior_ids, prior_ids + n_prior, ids.get());
    const auto t0 = std::chrono::steady_clock::now();
    int rc = c.generate_device(g, ids.get(), cap, drafter ? drafter->prompt : nullptr,
                               drafter ? drafter->stream : nullptr);
    if (rc) return rc;
    mtg_gen_stats st{};
    st.target_calls = g.target_calls;
    st.drafted_calls = g.drafted_calls;
    st.proposed = g.proposed;
    st.accepted = g.accepted;
    st.target_input_tokens = g.target_input_tokens;
    st.rewinds = g.rewinds;
    st.stop_reason = g.stop;
    st.next_seed = g.raw_choice;
    int n_new = g.n_ids - n_prior;
    if (g.err) {
      // a step of the device loop was abandoned (a bounded wait ran out): the host
      // controller finishes from the same state, its steps with the per-op fallback
      int32_t more = 0;
      mtg_gen_stats rest{};
      const int left_steps = max_steps > 0 ? max_steps - g.steps : 0;  // >= 1: the abandoned step did not count
      rc = mtg_generate_from(ctx, g.raw_choice, ids.get(), g.n_ids, max_new - n_new, left_steps, eos, penalty,
                             max_draft, drafter ? mtg_stream_draft : nullptr, nullptr,
                             drafter ? const_cast<mtg_stream_drafter*>(drafter) : nullptr, ids.get() + g.n_ids,
                             &more, &rest);
      if (rc) return rc;
      n_new += more;
      st.target_calls += rest.target_calls;
      st.drafted_calls += rest.drafted_calls;
      st.proposed += rest.proposed;
      st.accepted += rest.accepted;
      st.target_input_tokens += rest.target_input_tokens;
      st.rewinds += rest.rewinds;
      st.stop_reason = rest.stop_reason;
      st.next_seed = rest.next_seed;
    }
    st.verify_seconds = seconds_since(t0);
    std::copy(ids.get() + n_prior, ids.get() + n_prior + n_new, ids_out);
    *n_ids_out = n_new;
    if (stats) *stats = st;
    return MTG_OK;
  } catch (...) {
    return c.fail(MTG_ERR_NOMEM, "generate_device: out of host memory");
  }
}

int mtg_generate(mtg_ctx* ctx, const float* fused, int32_t seq, int32_t max_new, int32_t eos,
                 float penalty, int32_t max_draft, mtg_draft_fn draft, mtg_commit_fn commit,
                 void* user, int32_t* ids_out, int32_t* n_ids_out, mtg_gen_stats* stats) {
  if (!ctx) return MTG_ERR_INVALID;
  Ctx& c = ctx->impl;
  if (!fused || seq <= 0 || max_new <= 0 || !ids_out || !n_ids_out)
    return c.fail(MTG_ERR_INVALID, "generate: bad arguments");
  try {
    const int H = c.hp.hidden;
    auto t0 = std::chrono::steady_clock::now();
    std::vector<float> hidden((size_t)seq * H);
    int rc = mtg_prefill(ctx, fused, seq, hidden.data());
    if (rc) return rc;
    std::vector<float> raw(c.hp.vocab);
    if ((rc = c.logits_of(hidden.data() + (size_t)(seq - 1) * H, 1, raw.data()))) return rc;
    const double prefill_s = seconds_since(t0);
    const int32_t first = mtg_greedy_choice(raw.data(), c.hp.vocab, nullptr, 0, 1.0f);
    rc = mtg_generate_from(ctx, first, nullptr, 0, max_new, 0, eos, penalty, max_draft, draft,
                           commit, user, ids_out, n_ids_out, stats);
    if (stats) stats->prefill_seconds = prefill_s;
    return rc;
  } catch (...) {
    return c.fail(MTG_ERR_DEVICE, "generate: exception");
  }
}

// Draft hook used by the long-context workloads: n-gram proposal over
// prompt ++ ids (the reference drafter), completed from a seeded periodic token
// stream aligned to the absolute position of the next token.
int32_t mtg_stream_draft(void* user, const int32_t* ids, int32_t n_ids, int32_t budget,
                         int32_t* out) {
  const mtg_stream_drafter* d = (const mtg_stream_drafter*)user;
  if (!d || budget <= 0) return 0;
  std::vector<int32_t> hist(d->prompt, d->prompt + d->n_prompt);
  hist.insert(hist.end(), ids, ids + n_ids);
  int n = mtg_ngram_draft(hist.data(), (int)hist.size(), budget, out);
  if (d->period > 0)
    for (; n < budget; ++n) out[n] = d->stream[(size_t)(hist.size() + n) % (size_t)d->period];
  return n;
}

// ---- kernel-level entry points ----
struct mtg_q8_packed {
  uint8_t* tiles = nullptr;
  int k = 0, n = 0;
};

}  // extern "C"

namespace mtg {
void set_call_error(const std::string& msg) { g_create_error = msg; }
const uint8_t* q8_packed_view(const mtg_q8_packed* p, int* k, int* n) {
  *k = p->k;
  *n = p->n;
  return p->tiles;
}
}  // namespace mtg

extern "C" {

int mtg_q8_pack(const void* blocks, int32_t k, int32_t n, mtg_q8_packed** out) {
  if (!blocks || !out || k <= 0 || n <= 0) return MTG_ERR_INVALID;
  if (k % 64 || n % 16) return MTG_ERR_UNSUPPORTED;
  auto* p = new (std::nothrow) mtg_q8_packed();
  if (!p) return MTG_ERR_NOMEM;
  p->k = k;
  p->n = n;
  const size_t raw = (size_t)n * (k / 32) * 34, tiles = (size_t)(n / 16) * (k / 64) * mtg::kUnitBytes;
  uint8_t* staging = nullptr;
  if (hipMalloc(&staging, raw) != hipSuccess || hipMalloc(&p->tiles, tiles) != hipSuccess ||
      hipMemcpy(staging, blocks, raw, hipMemcpyHostToDevice) != hipSuccess) {
    hipFree(staging);
    hipFree(p->tiles);
    delete p;
    return MTG_ERR_DEVICE;
  }
  mtg::launch_q8_retile(nullptr, staging, n, k, p->tiles);
  const hipError_t e = hipDeviceSynchronize();
  hipFree(staging);
  if (e != hipSuccess) {
    hipFree(p->tiles);
    delete p;
    return MTG_ERR_DEVICE;
  }
  *out = p;
  return MTG_OK;
}

// Inverse of the re-tiling: download the tiles and restore n rows of ggml
// block_q8_0 (lets a caller check that packing kept every byte).
int mtg_q8_unpack(const mtg_q8_packed* p, void* blocks) {
  if (!p || !blocks) return MTG_ERR_INVALID;
  const int bps = p->k / 64, nb = p->k / 32;
  const size_t units = (size_t)(p->n / 16) * bps;
  std::vector<uint8_t> tiles(units * mtg::kUnitBytes);
  if (hipMemcpy(tiles.data(), p->tiles, tiles.size(), hipMemcpyDeviceToHost) != hipSuccess)
    return MTG_ERR_DEVICE;
  uint8_t* out = (uint8_t*)blocks;
  for (size_t u = 0; u < units; ++u) {
    const int tile = (int)(u / bps), bp = (int)(u % bps);
    const uint8_t* unit = tiles.data() + u * mtg::kUnitBytes;
    for (int lane = 0; lane < 64; ++lane) {
      const int row = tile * 16 + (lane & 15), g = lane >> 4, block = 2 * bp + (g >> 1);
      std::memcpy(out + ((size_t)row * nb + block) * 34 + 2 + (g & 1) * 16, unit + lane * 16, 16);
    }
    for (int par = 0; par < 2; ++par)
      for (int r = 0; r < 16; ++r)
        std::memcpy(out + ((size_t)(tile * 16 + r) * nb + 2 * bp + par) * 34,
                    unit + 1024 + (par * 16 + r) * 2, 2);
  }
  return MTG_OK;
}

void mtg_q8_free(mtg_q8_packed* p) {
  if (!p) return;
  hipFree(p->tiles);
  delete p;
}

int mtg_q8_mul_mat_dev(const mtg_q8_packed* w, const float* x_dev, int32_t T, float* y_dev) {
  if (!w || !x_dev || !y_dev || T <= 0 || T > MTG_MAX_BATCH) return MTG_ERR_INVALID;
  mtg::StepDesc host{};
  host.T = T;
  host.groups = (T + 7) / 8;
  mtg::StepDesc* desc = nullptr;
  mtg::Panel panel{};
  const size_t pairs = (size_t)w->k / 64;
  if (hipMalloc(&desc, sizeof(host)) != hipSuccess) return MTG_ERR_DEVICE;
  if (hipMalloc(&panel.codes, mtg::kMaxGroups * pairs * 1024) != hipSuccess ||
      hipMalloc(&panel.scales, mtg::kMaxGroups * pairs * 64) != hipSuccess) {
    hipFree(desc);
    hipFree(panel.codes);
    return MTG_ERR_DEVICE;
  }
  hipError_t e = hipMemcpy(desc, &host, sizeof(host), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(panel.codes, 0, mtg::kMaxGroups * pairs * 1024);
  if (e == hipSuccess) {
    mtg::launch_norm_quant(nullptr, desc, x_dev, w->k, nullptr, 0.0f, panel, nullptr);
    mtg::launch_gemm_store(nullptr, host.groups, desc, w->tiles, w->n, w->k, panel, y_dev);
    e = hipDeviceSynchronize();
  }
  hipFree(desc);
  hipFree(panel.codes);
  hipFree(panel.scales);
  return e == hipSuccess ? MTG_OK : MTG_ERR_DEVICE;
}

int mtg_causal_context_dev(const float* v_dev, const float* p_dev, int32_t head_dim,
                           int32_t kv_heads, int32_t heads, int32_t queries, int32_t kv_len,
                           float* out_dev) {
  if (!v_dev || !p_dev || !out_dev || head_dim <= 0 || kv_heads <= 0 || heads <= 0 ||
      heads % kv_heads || queries < 2 || kv_len <= queries)
    return MTG_ERR_UNSUPPORTED;  // the reference's cpu_causal_context returns nullptr here
  mtg::launch_causal_context(nullptr, v_dev, p_dev, head_dim, kv_heads, heads, queries, kv_len,
                             out_dev);
  return hipDeviceSynchronize() == hipSuccess ? MTG_OK : MTG_ERR_DEVICE;
}

}  // extern "C"
