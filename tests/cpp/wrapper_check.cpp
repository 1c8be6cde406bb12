// Exercises include/carat_hip_runner.hpp the way the reference's code calls its own runner and
// speculation helpers (tests/speculation_tests.cpp, src/ragged_batch_parity.cu, the scheduler).
//
//   wrapper_check vectors FILE   speculation helpers against the reference's golden vectors
//                                (one case per line, written by tests/test_cpp_wrapper.py)
//   wrapper_check runner         a tiny synthetic model on the GPU: prefill, clone, draft,
//                                verify, append_ragged, and the reference's error texts
#include "carat_hip_runner.hpp"
#include "carat_hip_speculation.hpp"

#include <cstdio>
#include <fstream>
#include <sstream>
#include <string>

namespace {

int failures = 0;

void check(bool ok, const std::string &what) {
  if (!ok) {
    std::printf("FAIL %s\n", what.c_str());
    ++failures;
  }
}

template <typename F> void check_throws(F &&f, const std::string &fragment) {
  try {
    f();
    check(false, "no exception, expected: " + fragment);
  } catch (const std::runtime_error &e) {
    check(std::string(e.what()).find(fragment) != std::string::npos,
          "message '" + std::string(e.what()) + "' lacks '" + fragment + "'");
  }
}

std::vector<int> read_list(std::istringstream &in) {
  int n = 0;
  in >> n;
  std::vector<int> v(static_cast<size_t>(n));
  for (int &x : v) in >> x;
  return v;
}

int vectors(const char *path) {
  std::ifstream file(path);
  std::string line;
  int cases = 0;
  while (std::getline(file, line)) {
    std::istringstream in(line);
    std::string kind;
    in >> kind;
    if (kind == "cap") {
      int depth = 0, remaining = 0, expected = 0;
      in >> depth >> remaining;
      const std::vector<int> proposals = read_list(in);
      const std::vector<int> stops = read_list(in);
      in >> expected;
      const std::unordered_set<int> stop_set(stops.begin(), stops.end());
      check(carat::acceptance_cap(depth, remaining, proposals, stop_set) == expected, "cap: " + line);
    } else if (kind == "commit") {
      int forced = 0, next = 0, want_next = 0, want_stopped = 0;
      in >> forced;
      const std::vector<int> drafts = read_list(in);
      in >> next;
      const std::vector<int> stops = read_list(in);
      const std::vector<int> resident = read_list(in);
      const std::vector<int> emitted = read_list(in);
      in >> want_next >> want_stopped;
      const std::unordered_set<int> stop_set(stops.begin(), stops.end());
      const carat::SpeculativeCommit got = carat::commit_speculation(forced, drafts, next, stop_set);
      check(got.resident_tokens == resident && got.emitted_tokens == emitted &&
                got.next_token == want_next && got.stopped == (want_stopped != 0),
            "commit: " + line);
    } else {
      continue;
    }
    ++cases;
  }
  std::printf("%d speculation cases, %d failures\n", cases, failures);
  return failures == 0 && cases > 0 ? 0 : 1;
}

int runner() {
  const carat_hip_layer_desc layers[3] = {{1, 4, 2, 128, 0}, {1, 4, 2, 128, 0}, {0, 4, 2, 128, 1}};
  carat_hip_model_desc desc{};
  desc.hidden = 256;
  desc.intermediate = 512;
  desc.vocabulary = 2048;
  desc.sliding_window = 32;
  desc.rms_norm_epsilon = 1e-6f;
  desc.layer_count = 3;
  desc.layers = layers;
  desc.assistant = 1;
  desc.assistant_hidden = 256;
  desc.assistant_intermediate = 512;
  desc.assistant_layers = 2;
  desc.assistant_query_heads = 4;
  desc.seed = 9;
  desc.weight_std = 0.05f;
  carat::Gemma4BatchModelRunner runner(desc, 4, 128);
  check(runner.batch() == 4 && runner.has_assistant(), "shape");
  std::vector<int> prompt;
  for (int i = 0; i < 40; ++i) prompt.push_back((i * 37 + 11) % 2048);
  const int first = runner.prefill_slot(0, prompt, 16);
  check(runner.slot_position(0) == 40, "prefill position");
  for (int slot = 1; slot < 4; ++slot) runner.clone_slot(0, slot);
  check(runner.slot_position(3) == 40, "clone position");
  // speculative-parity style patterns (ragged_batch_parity.cu:212-229): the draft with the
  // target's first token forced, then the same with a rejected first proposal
  const std::vector<int> slots{0, 1, 2, 3};
  const std::vector<int> last(4, prompt.back()), forced(4, first);
  auto proposals = runner.draft_four(last, slots, forced, 4);
  for (const auto &row : proposals) check(row.size() == 4 && row[0] == first, "draft row 0 is forced");
  proposals[1][0] = (first + 1) % 2048;
  const auto result = runner.verify_greedy_proposals(proposals, forced, slots, {4, 4, 4, 0});
  check(result.accepted_tokens[1] == 0 && result.next_tokens[1] == first, "reject at 0");
  check(result.accepted_tokens[3] == 0, "cap 0");
  check(result.accepted_tokens[0] >= 1 && result.accepted_tokens[2] == result.accepted_tokens[0] &&
            result.next_tokens[2] == result.next_tokens[0],
        "identical clones verify identically");
  for (int r = 0; r < 4; ++r)
    check(runner.slot_position(r) == 40 + result.accepted_tokens[static_cast<size_t>(r)], "commit");
  // the accepted == 0 fallback (native_runtime_main.cpp:637-648)
  const auto fallback = runner.append_ragged({first, first}, {1, 3});
  check(fallback.size() == 2 && fallback[0] == fallback[1], "fallback decode of identical slots");
  check(runner.slot_position(1) == 41 && runner.slot_position(3) == 41, "fallback positions");
  check_throws([&] { runner.verify_greedy_proposals({{1, 2}, {3, 4}}, {1, 3}, {0, 0}); },
               "invalid or repeated speculative slot");
  check_throws([&] { runner.prefill_slot(0, {}, 8); }, "invalid slot prefill shape");
  check_throws([&] { runner.clone_slot(2, 2); }, "invalid cache slot clone");
  std::printf("runner checks done, %d failures\n", failures);
  return failures == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char **argv) {
  try {
    if (argc == 3 && std::string(argv[1]) == "vectors") return vectors(argv[2]);
    if (argc == 2 && std::string(argv[1]) == "runner") return runner();
  } catch (const std::exception &e) {
    std::printf("FAIL exception: %s\n", e.what());
    return 1;
  }
  std::printf("usage: wrapper_check vectors FILE | runner\n");
  return 2;
}
