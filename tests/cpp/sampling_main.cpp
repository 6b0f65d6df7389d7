// The reference's argmax test (tests/test_sampling.cu) in this build's spelling: device buffers
// from the runtime, the handle-free sample_token_amax(d_logits, d_output) launcher, the result
// copied back.  Arguments: a file of 128256 fp32 logits; prints the sampled id.
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <vector>

#include "infengine/engine.h"

int main(int argc, char** argv) {
  if (argc < 2) {
    std::fprintf(stderr, "usage: %s logits.f32\n", argv[0]);
    return 2;
  }
  std::vector<float> input(InfEngineConfig::VOCAB_SIZE);
  std::FILE* f = std::fopen(argv[1], "rb");
  if (!f || std::fread(input.data(), sizeof(float), input.size(), f) != input.size()) {
    std::fprintf(stderr, "cannot read %s\n", argv[1]);
    return 2;
  }
  std::fclose(f);

  float* d_input = nullptr;
  int* d_output = nullptr;
  int actual = -1;
  if (hipMalloc(&d_input, sizeof(float) * input.size()) != hipSuccess ||
      hipMalloc(&d_output, sizeof(int)) != hipSuccess ||
      hipMemcpy(d_input, input.data(), sizeof(float) * input.size(), hipMemcpyHostToDevice) !=
          hipSuccess) {
    std::fprintf(stderr, "HIP setup failed\n");
    return 1;
  }
  try {
    sample_token_amax(d_input, d_output);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
  if (hipMemcpy(&actual, d_output, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return 1;
  std::printf("%d\n", actual);
  (void)hipFree(d_input);
  (void)hipFree(d_output);
  return 0;
}
