// Drives the continuous batcher (include/infengine/batcher.h) over random-init weights: four
// requests run (a) all admitted at once, (b) joining at different steps, (c) one at a time.
// A request's tokens must not depend on which requests share its steps, so all three
// schedules must produce the same tokens; every page must be back in the pool afterwards.
// Then (d) the same requests with EOS ids stop right after them, and (e) a prefill that fails
// leaves its request queued and no page lost.
// Prints the tokens of schedule (a), then "OK" or the first mismatch; exit status 0 on OK.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "infengine/batcher.h"

namespace {

struct Spec {
  int prompt_len, new_tokens;
};
const Spec kSpecs[] = {{20, 12}, {33, 10}, {7, 14}, {70, 16}};  // the last crosses a page
constexpr int kPages = 12;

std::vector<int> prompt_of(int r, int len) {
  std::vector<int> p;
  for (int i = 0; i < len; ++i) p.push_back((i * 7919 + 104729 * (r + 1)) % InfEngineConfig::VOCAB_SIZE);
  return p;
}

using Result = std::vector<std::vector<int>>;

Result run(IEHandle h, const ModelWeights& w, int schedule) {
  ContinuousBatcher cb(h, w, kPages);
  const int n = (int)(sizeof(kSpecs) / sizeof(kSpecs[0]));
  std::vector<int> ids;
  if (schedule == 0) {
    for (int r = 0; r < n; ++r) ids.push_back(cb.submit(prompt_of(r, kSpecs[r].prompt_len), kSpecs[r].new_tokens));
    cb.run();
  } else if (schedule == 1) {
    ids.push_back(cb.submit(prompt_of(0, kSpecs[0].prompt_len), kSpecs[0].new_tokens));
    cb.step();
    cb.step();
    ids.push_back(cb.submit(prompt_of(1, kSpecs[1].prompt_len), kSpecs[1].new_tokens));
    for (int i = 0; i < 3; ++i) cb.step();
    for (int r = 2; r < n; ++r) ids.push_back(cb.submit(prompt_of(r, kSpecs[r].prompt_len), kSpecs[r].new_tokens));
    cb.run();
  } else {
    for (int r = 0; r < n; ++r) {
      ids.push_back(cb.submit(prompt_of(r, kSpecs[r].prompt_len), kSpecs[r].new_tokens));
      cb.run();
    }
  }
  Result out;
  for (int r = 0; r < n; ++r) {
    if (!cb.finished(ids[r])) throw std::runtime_error("request not finished");
    const auto& t = cb.tokens(ids[r]);
    out.emplace_back(t.begin() + kSpecs[r].prompt_len, t.end());
    if ((int)out.back().size() != kSpecs[r].new_tokens) throw std::runtime_error("wrong token count");
  }
  if (cb.free_pages() != kPages) throw std::runtime_error("pages not returned to the pool");
  return out;
}

// (d) every request stops right after a token chosen from its schedule-(a) output (the first
// occurrence of that token): the tokens must be that prefix, and all pages back in the pool.
bool run_eos(IEHandle h, const ModelWeights& w, const Result& a) {
  ContinuousBatcher cb(h, w, kPages);
  const int n = (int)a.size();
  std::vector<int> ids;
  std::vector<std::vector<int>> want;
  for (int r = 0; r < n; ++r) {
    const int eos = a[r][2 + r % 3];
    const size_t first = std::find(a[r].begin(), a[r].end(), eos) - a[r].begin();
    want.emplace_back(a[r].begin(), a[r].begin() + first + 1);
    ids.push_back(cb.submit(prompt_of(r, kSpecs[r].prompt_len), kSpecs[r].new_tokens, eos));
  }
  cb.run();
  bool ok = cb.free_pages() == kPages;
  for (int r = 0; r < n; ++r) {
    const auto& t = cb.tokens(ids[r]);
    const std::vector<int> got(t.begin() + kSpecs[r].prompt_len, t.end());
    ok = ok && cb.finished(ids[r]) && got == want[r];
    std::printf("eos %d stop_after %zu\n", r, got.size());
  }
  return ok;
}

// (e) a prefill that fails (incomplete weights: rejected on the host before any GPU work)
// throws out of step(), leaves the request queued and returns every page to the pool.
bool run_failed_prefill(IEHandle h) {
  const ModelWeights empty;
  ContinuousBatcher cb(h, empty, kPages);
  const int id = cb.submit(prompt_of(0, 100), 20);
  for (int attempt = 0; attempt < 2; ++attempt) {
    bool threw = false;
    try {
      cb.step();
    } catch (const std::exception&) {
      threw = true;
    }
    if (!threw || cb.free_pages() != kPages || cb.finished(id)) return false;
  }
  std::printf("failed prefill: pages %d of %d free\n", cb.free_pages(), kPages);
  return true;
}

}  // namespace

int main() {
  try {
    ModelWeights w = ModelWeights::random_init(7, 0.02f);
    IEHandle h = ie_create_handle(0);
    const Result a = run(h, w, 0), b = run(h, w, 1), c = run(h, w, 2);
    for (size_t r = 0; r < a.size(); ++r) {
      std::printf("tokens %zu", r);
      for (int t : a[r]) std::printf(" %d", t);
      std::printf("\n");
    }
    int rc = 0;
    for (size_t r = 0; r < a.size(); ++r)
      if (a[r] != b[r] || a[r] != c[r]) {
        std::printf("MISMATCH request %zu\n", r);
        rc = 1;
      }
    if (!run_eos(h, w, a)) {
      std::printf("EOS MISMATCH\n");
      rc = 1;
    }
    if (!run_failed_prefill(h)) {
      std::printf("FAILED PREFILL LEAKED PAGES\n");
      rc = 1;
    }
    if (!rc) std::printf("OK\n");
    ie_destroy_handle(h);
    w.free();
    return rc;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 2;
  }
}
