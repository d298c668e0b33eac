// A C++ caller of the engine written the way the reference's callers are,
// through include/cuqwen_compat.hpp, so the drop-in claim is compiled and run:
//
//   bench <bin> <warmup> <window_len> <start>...
//       benchmark/cuqwen_benchmark.cu:41-123: load_weights, malloc_qwen_state,
//       mt19937(42) dummy tokens, an untimed warm-up that records the graph,
//       then timed windows of qwen_forward(dummy[pos], pos, ..., dummy, pos)
//       bracketed by events; with --stream the steps run on a stream the
//       caller created (the qwen_forward stream argument).
//   chat <bin> <max_new> <prompt id>...
//       src/main.cu:29-112 for one turn without the tokenizer: the prompt
//       through one qwen_forward per token (no history), then greedy decode
//       with the generated ids as the penalty history until <|endoftext|>,
//       <|im_end|>, max_seq_len - 2 or max_new tokens.
//
// Prints one JSON object on stdout.  Built by cuqwen_amd/build.py with
// -DQWEN_MODEL_0_5B -DQUANT_INT8; run by tests/test_gpu_compat.py.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "cuqwen_compat.hpp"

#define HIP_OK(call)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (call);                                                            \
    if (e_ != hipSuccess) {                                                            \
      std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      std::exit(1);                                                                    \
    }                                                                                  \
  } while (0)

static void print_ints(const char* key, const std::vector<int>& v, bool last = false) {
  std::printf("\"%s\": [", key);
  for (size_t i = 0; i < v.size(); ++i) std::printf(i ? ", %d" : "%d", v[i]);
  std::printf("]%s", last ? "" : ", ");
}

static int bench(int argc, char** argv) {
  if (argc < 6) return 2;
  const std::string bin = argv[2];
  const int warmup = std::atoi(argv[3]), window = std::atoi(argv[4]);
  std::vector<int> starts;
  bool own_stream = false;
  for (int i = 5; i < argc; ++i) {
    if (std::strcmp(argv[i], "--stream") == 0) own_stream = true;
    else starts.push_back(std::atoi(argv[i]));
  }
  QwenWeights weights;
  QwenConfig config = load_weights(bin, weights);
  QwenState state;
  malloc_qwen_state(config, state);
  hipStream_t stream = 0;
  if (own_stream) HIP_OK(hipStreamCreate(&stream));

  const int max_context = std::min(32000, QwenConfig::max_seq_len - 2);
  std::mt19937 rng(42);
  std::uniform_int_distribution<int> dist(0, config.vocab_size - 1);
  std::vector<int> dummy(max_context);
  for (int i = 0; i < max_context; ++i) dummy[i] = dist(rng);

  hipEvent_t ev0, ev1;
  HIP_OK(hipEventCreate(&ev0));
  HIP_OK(hipEventCreate(&ev1));
  std::vector<int> positions, returned;
  std::vector<double> tok_s;
  for (int pos = 0; pos < warmup; ++pos) {
    returned.push_back(qwen_forward(dummy[pos], pos, config, state, weights, dummy.data(), pos, stream));
    positions.push_back(pos);
  }
  HIP_OK(hipDeviceSynchronize());
  for (int start : starts) {
    const int end = start + window;
    if (end > max_context) break;
    HIP_OK(hipEventRecord(ev0, stream));
    for (int pos = start; pos < end; ++pos) {
      returned.push_back(qwen_forward(dummy[pos], pos, config, state, weights, dummy.data(), pos, stream));
      positions.push_back(pos);
    }
    HIP_OK(hipEventRecord(ev1, stream));
    HIP_OK(hipEventSynchronize(ev1));
    float ms = 0.f;
    HIP_OK(hipEventElapsedTime(&ms, ev0, ev1));
    tok_s.push_back(window / (ms / 1000.0));
  }
  const int used = positions.empty() ? 0 : *std::max_element(positions.begin(), positions.end()) + 1;
  std::printf("{");
  print_ints("dummy", std::vector<int>(dummy.begin(), dummy.begin() + used));
  print_ints("positions", positions);
  print_ints("returned", returned);
  std::printf("\"tok_per_s\": [");
  for (size_t i = 0; i < tok_s.size(); ++i) std::printf(i ? ", %.2f" : "%.2f", tok_s[i]);
  std::printf("]}\n");
  HIP_OK(hipEventDestroy(ev0));
  HIP_OK(hipEventDestroy(ev1));
  if (own_stream) HIP_OK(hipStreamDestroy(stream));
  free_qwen_state(state);
  free_weights(weights, config);
  return 0;
}

static int chat(int argc, char** argv) {
  if (argc < 5) return 2;
  const std::string bin = argv[2];
  const int max_new = std::atoi(argv[3]);
  std::vector<int> prompt;
  for (int i = 4; i < argc; ++i) prompt.push_back(std::atoi(argv[i]));
  const int eos_id = 151643, im_end_id = 151645;
  QwenWeights weights;
  QwenConfig config = load_weights(bin, weights);
  QwenState state;
  malloc_qwen_state(config, state);
  const int max_allowed_pos = QwenConfig::max_seq_len - 2;
  int current_pos = 0;
  int next_token = 0;
  for (size_t i = 0; i < prompt.size(); ++i) {
    next_token = qwen_forward(prompt[i], current_pos, config, state, weights);
    current_pos++;
  }
  const int after_prefill = next_token;
  std::vector<int> generated;
  while (next_token != eos_id && next_token != im_end_id && current_pos < max_allowed_pos &&
         (int)generated.size() < max_new) {
    generated.push_back(next_token);
    next_token = qwen_forward(next_token, current_pos, config, state, weights, generated.data(),
                              static_cast<int>(generated.size()));
    current_pos++;
  }
  std::printf("{\"after_prefill\": %d, ", after_prefill);
  print_ints("generated", generated);
  std::printf("\"last\": %d, \"pos\": %d}\n", next_token, current_pos);
  free_qwen_state(state);
  free_weights(weights, config);
  return 0;
}

int main(int argc, char** argv) {
  try {
    if (argc > 1 && std::strcmp(argv[1], "bench") == 0) return bench(argc, argv);
    if (argc > 1 && std::strcmp(argv[1], "chat") == 0) return chat(argc, argv);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "compat_caller: %s\n", e.what());
    return 1;
  }
  std::fprintf(stderr, "usage: compat_caller bench <bin> <warmup> <window> <start>... [--stream]\n"
                       "       compat_caller chat <bin> <max_new> <prompt id>...\n");
  return 2;
}
