// Speculative generation on the GPU decoder against serial greedy decoding,
// through the reference-named interface (include/mtg_reference.hpp), in the manner
// of moss-transcribe.cpp's lab gate (cpu-lab/moss_speculative_gate.cpp:149-260):
// a hooked drafter replays the serial greedy continuation with one forced
// rejection per step; the generated ids must equal the serial ids, every commit
// must leave past_len == prefix + |ids| - stop, and an out-of-vocabulary draft
// must throw. Synthetic seeded q8_0 model, 2 layers, vocabulary 4096.
#include <cstdio>
#include <stdexcept>
#include <string>
#include <vector>

#include "mtg_reference.hpp"

namespace {
void check(bool ok, const std::string& what) {
  if (!ok) throw std::runtime_error(what);
}
}  // namespace

int main() {
  try {
    mtg_hparams hp{1024, 16, 8, 128, 3072, 2, 4096, 1e6f, 1e-6f};
    mtg_synth_model* synth = nullptr;
    check(mtg_synth_create(&hp, MTG_TYPE_Q8_0, 31, 0.02f, 0.05f, &synth) == MTG_OK, "synthetic model");
    const mtg_model_desc& desc = *mtg_synth_desc(synth);
    const int prefix = 37, max_new = 40;
    // fused prompt rows: embeddings of seeded ids
    mt::GpuDecoder serial, spec;
    check(serial.load(desc, 256) && spec.load(desc, 256), "load");
    std::vector<int32_t> prompt(prefix);
    for (int i = 0; i < prefix; ++i) prompt[i] = (i * 2654435761u) % hp.vocab;
    std::vector<float> fused((size_t)prefix * hp.hidden);
    check(mtg_embed(serial.context(), prompt.data(), prefix, fused.data()) == MTG_OK, "embed");

    // serial greedy decoding (one row per step): the gold sequence
    std::vector<float> all;
    check(serial.prefill(fused, prefix, &all), "serial prefill");
    std::vector<float> raw = serial.logits_from_hidden(
        std::vector<float>(all.end() - hp.hidden, all.end()));
    std::vector<int32_t> gold;
    for (int i = 0; i < max_new; ++i) {
      const int id = mt::cpu_greedy_choice(raw, gold, 1.0f);
      gold.push_back(id);
      std::vector<float> e(hp.hidden);
      check(mtg_embed(serial.context(), &gold.back(), 1, e.data()) == MTG_OK, "embed row");
      const std::vector<float> h = serial.decode_one(e);
      check(h.size() == (size_t)hp.hidden, "decode_one");
      raw = serial.logits_from_hidden(h);
    }

    // speculative: drafts = the gold continuation, with the draft at rank
    // (step % 4) + 1 replaced by a wrong id (one forced rejection per step)
    int step = 0, commits = 0;
    mt::CpuSpeculativeHooks hooks;
    hooks.draft = [&](const std::vector<int32_t>& ids, int budget) {
      std::vector<int32_t> out;
      for (int r = 0; r < budget && ids.size() + r < gold.size(); ++r) out.push_back(gold[ids.size() + r]);
      const size_t bad = (size_t)(step++ % 4) + 1;
      if (bad < out.size()) out[bad] = (out[bad] + 1) % hp.vocab;
      return out;
    };
    hooks.committed = [&](mt::GpuDecoder& d, const std::vector<int32_t>& ids,
                          const std::vector<float>& last, bool stop) {
      ++commits;
      check(d.past_len() == prefix + (int)ids.size() - (stop ? 1 : 0), "past_len after commit");
      check(last.size() == (size_t)hp.vocab, "committed logits row");
    };
    const std::vector<int32_t> ids = mt::cpu_speculative_generate(spec, fused, prefix, max_new, -1, &hooks, 7);
    check(ids == gold, "speculative ids equal serial greedy ids");
    check(commits > 0 && commits < max_new, "fewer target calls than tokens");

    // an out-of-vocabulary proposal is an error, as in the reference
    mt::CpuSpeculativeHooks bad;
    bad.draft = [&](const std::vector<int32_t>&, int budget) {
      return std::vector<int32_t>(budget > 0 ? 1 : 0, hp.vocab + 5);
    };
    bool threw = false;
    try {
      mt::cpu_speculative_generate(spec, fused, prefix, 8, -1, &bad, 4);
    } catch (const std::runtime_error&) {
      threw = true;
    }
    check(threw, "invalid draft throws");
    mtg_synth_free(synth);
    std::printf("{\"record\":\"speculativeGate\",\"tokens\":%zu,\"commits\":%d,\"passed\":true}\n",
                ids.size(), commits);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "gate failed: %s\n", e.what());
    return 1;
  }
}
