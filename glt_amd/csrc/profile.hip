// Per-label launch timing with HIP events (the reference's
// --profile-graft-gemms, src/gemm_impl.inc:153-199 and :408-444, keeps one
// event pair per GEMM and synchronises after each; here events are taken
// from a pool created up front, bound to the kernel dispatch by
// hipExtLaunchKernelGGL, and resolved in one pass at collect time, so
// profiled runs keep the stream busy).
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"

namespace glt {

namespace {
struct Rec {
  const char* label;
  int a, b;  // event indices
};
std::mutex g_mu;
bool g_on = false;
std::vector<hipEvent_t> g_pool;
std::vector<Rec> g_recs;
int g_next = 0;
constexpr int kPool = 16384;
}  // namespace

int prof_slot(const char* label, hipEvent_t* start, hipEvent_t* stop) {
  if (!g_on) return -1;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_next + 2 > (int)g_pool.size()) return -1;
  const int a = g_next, b = g_next + 1;
  g_next += 2;
  *start = g_pool[a];
  *stop = g_pool[b];
  g_recs.push_back(Rec{label, a, b});
  return (int)g_recs.size() - 1;
}

}  // namespace glt

using namespace glt;

extern "C" {

glt_status glt_profile_enable(int32_t on) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (on && g_pool.empty()) {
    g_pool.resize(kPool);
    // Timing only: no system-scope fence (cache writeback and invalidate)
    // when an event completes, so the bracketed kernel ends as it does in
    // an unprofiled run and its neighbours do not pay for a flush.
    for (auto& e : g_pool) GLT_TRY_HIP(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
  }
  g_on = on != 0;
  return GLT_OK;
}

int32_t glt_profile_collect(char* names, size_t names_len, double* total_ms, int64_t* counts, int32_t max_labels) {
  std::lock_guard<std::mutex> lk(g_mu);
  std::vector<std::string> labels;
  std::vector<double> tot;
  std::vector<int64_t> cnt;
  for (const Rec& r : g_recs) {
    if (hipEventSynchronize(g_pool[r.b]) != hipSuccess) continue;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, g_pool[r.a], g_pool[r.b]) != hipSuccess) continue;
    size_t i = 0;
    while (i < labels.size() && labels[i] != r.label) ++i;
    if (i == labels.size()) {
      labels.emplace_back(r.label);
      tot.push_back(0.0);
      cnt.push_back(0);
    }
    tot[i] += ms;
    cnt[i] += 1;
  }
  g_recs.clear();
  g_next = 0;
  int n = 0;
  size_t pos = 0;
  for (size_t i = 0; i < labels.size() && n < max_labels; ++i, ++n) {
    if (names && pos + labels[i].size() + 1 <= names_len) {
      memcpy(names + pos, labels[i].c_str(), labels[i].size() + 1);
      pos += labels[i].size() + 1;
    }
    if (total_ms) total_ms[n] = tot[i];
    if (counts) counts[n] = cnt[i];
  }
  return n;
}

}  // extern "C"
