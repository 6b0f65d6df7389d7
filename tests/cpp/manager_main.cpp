// Drives the C++ engine API the way the reference's main.cpp / manager.cpp do:
// a Manager over random-init weights generates greedily from a fixed prompt of
// token ids (stopping after max tokens or an EOS id) and prints one line: the generated ids
// and the timing.  Arguments: prompt length, new tokens, seed, EOS id (default none).
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "infengine/manager.h"

int main(int argc, char** argv) {
  const int prompt_len = argc > 1 ? std::atoi(argv[1]) : 16;
  const int new_tokens = argc > 2 ? std::atoi(argv[2]) : 8;
  const unsigned long long seed = argc > 3 ? std::strtoull(argv[3], nullptr, 10) : 7;
  const int eos = argc > 4 ? std::atoi(argv[4]) : -1;
  try {
    Manager manager(seed, 0.02f);
    std::vector<int> prompt;
    for (int i = 0; i < prompt_len; ++i) prompt.push_back((i * 7919 + 17) % InfEngineConfig::VOCAB_SIZE);
    std::vector<int> out = manager.handle_request(prompt, new_tokens, eos);
    std::printf("tokens");
    for (size_t i = prompt.size(); i < out.size(); ++i) std::printf(" %d", out[i]);
    const auto& t = manager.last_timing();
    std::printf("\nprefill_ms %.3f decode_ms_per_token %.4f\n", t.prefill_ms, t.ms_per_token());
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
  return 0;
}
