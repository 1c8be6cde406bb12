// C++ drop-in for the reference's speculation helpers (src/runtime/speculation.h:11-27),
// header-only over the C ABI in carat_hip.h: the same names, argument meaning and results.
// Failures are rethrown as std::runtime_error with the library's message. A build that keeps the
// reference's own speculation.cpp does not include this header.
#pragma once

#include "carat_hip.h"

#include <cstdint>
#include <span>
#include <stdexcept>
#include <unordered_set>
#include <vector>

namespace carat {

inline void hip_speculation_ok(int status) {
  if (status != 0) throw std::runtime_error(carat_hip_last_error());
}

// ------------------------------------------------------------------ speculation.h:11-27
[[nodiscard]] inline int acceptance_cap(int depth, int remaining, std::span<const int> proposals,
                                        const std::unordered_set<int> &stop_ids) {
  const std::vector<int32_t> stops(stop_ids.begin(), stop_ids.end());
  int cap = 0;
  hip_speculation_ok(carat_hip_acceptance_cap(depth, remaining, proposals.data(),
                                  static_cast<int>(proposals.size()), stops.data(),
                                  static_cast<int>(stops.size()), &cap));
  return cap;
}

struct SpeculativeCommit {
  std::vector<int> resident_tokens;
  std::vector<int> emitted_tokens;
  int next_token{0};
  bool stopped{false};
};

[[nodiscard]] inline SpeculativeCommit commit_speculation(int forced_token,
                                                          std::span<const int> accepted_drafts,
                                                          int next_token,
                                                          const std::unordered_set<int> &stop_ids) {
  const std::vector<int32_t> stops(stop_ids.begin(), stop_ids.end());
  const size_t n = accepted_drafts.size() + 1;
  SpeculativeCommit out;
  out.resident_tokens.resize(n);
  out.emitted_tokens.resize(n);
  int resident = 0, emitted = 0, stopped = 0;
  int32_t next = 0;
  hip_speculation_ok(carat_hip_commit_speculation(forced_token, accepted_drafts.data(),
                                      static_cast<int>(accepted_drafts.size()), next_token,
                                      stops.data(), static_cast<int>(stops.size()),
                                      out.resident_tokens.data(), &resident,
                                      out.emitted_tokens.data(), &emitted, &next, &stopped));
  out.resident_tokens.resize(static_cast<size_t>(resident));
  out.emitted_tokens.resize(static_cast<size_t>(emitted));
  out.next_token = next;
  out.stopped = stopped != 0;
  return out;
}

}  // namespace carat
