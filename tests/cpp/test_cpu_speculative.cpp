// Policy controls of the speculative path through the reference-named interface
// (include/mtg_reference.hpp): the n-gram proposal, first-max greedy choice and
// the recent-100 repetition penalty. Vectors: tests/test_cpu_speculative.cpp:9-21
// of moss-transcribe.cpp. Host code only; no GPU is touched.
#include <cstdio>
#include <stdexcept>
#include <vector>

#include "mtg_reference.hpp"

namespace {
int controls = 0;
void check(bool ok, const char* what) {
  ++controls;
  if (!ok) throw std::runtime_error(what);
}
using Ids = std::vector<int32_t>;
}  // namespace

int main() {
  try {
    check(mt::cpu_ngram_draft({1, 2, 3, 4, 1, 2}, 4) == Ids({3, 4, 1, 2}), "draft: full continuation");
    check(mt::cpu_ngram_draft({1, 2, 3, 4, 1, 2}, 2) == Ids({3, 4}), "draft: truncated to maximum");
    check(mt::cpu_ngram_draft({1, 2, 3, 1, 2, 9, 1, 2}, 4) == Ids({9, 1, 2}), "draft: latest occurrence");
    check(mt::cpu_ngram_draft({1, 2, 3, 4, 5}, 4).empty(), "draft: no repeated suffix");
    check(mt::cpu_ngram_draft({1, 2}, 4).empty(), "draft: history too short");
    check(mt::cpu_ngram_draft({1, 2, 1, 2}, 0).empty(), "draft: zero budget");
    check(mt::cpu_greedy_choice({2, 2, 1}, {}, 1.0f) == 0, "choice: first maximum wins ties");
    check(mt::cpu_greedy_choice({2, 1.9f}, {0, 0}, 1.1f) == 1, "choice: positive logit divided");
    check(mt::cpu_greedy_choice({-2, -2.1f}, {0, 0}, 1.1f) == 1, "choice: negative logit multiplied");
    check(mt::cpu_greedy_choice({2, 1.9f}, {0}, 1.0f) == 0, "choice: penalty 1 disables");
    std::vector<int32_t> history(101, 2);
    history[0] = 0;  // id 0 is 101 entries back: outside the window
    check(mt::cpu_greedy_choice({2, 1.9f}, history, 1.1f) == 0, "choice: window is the last 100");
    history[1] = 0;  // now inside the window
    check(mt::cpu_greedy_choice({2, 1.9f}, history, 1.1f) == 1, "choice: id inside the window");
    bool threw = false;
    try {
      mt::cpu_greedy_choice({}, {}, 1.0f);
    } catch (const std::runtime_error&) {
      threw = true;
    }
    check(threw, "choice: empty logits throw");
    std::printf("{\"record\":\"speculativePolicy\",\"controls\":%d,\"passed\":true}\n", controls);
    return 0;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "%s (control %d)\n", e.what(), controls);
    return 1;
  }
}
