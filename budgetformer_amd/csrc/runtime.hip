// Library-wide state of the C ABI: version, per-thread error messages, and the
// optional per-kernel timer (HIP event pairs around each launch, accumulated
// per kernel name when collected).
#include "bf_common.h"

#include <mutex>
#include <string>
#include <vector>

namespace bf {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

namespace {

struct Pending {
  const char* name;
  hipEvent_t start;
  hipEvent_t stop;
};

struct Stat {
  std::string name;
  double total_ms;
  int64_t launches;
};

std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_free_events;
std::vector<Stat> g_stats;

hipEvent_t take_event() {
  if (!g_free_events.empty()) {
    hipEvent_t e = g_free_events.back();
    g_free_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

}  // namespace

bool prof_enabled() { return g_prof_on; }

void prof_begin(const char* name, hipStream_t st, int* token) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  *token = -1;
  hipEvent_t a = take_event(), b = take_event();
  if (!a || !b) return;
  if (hipEventRecord(a, st) != hipSuccess) return;
  g_pending.push_back(Pending{name, a, b});
  *token = int(g_pending.size()) - 1;
}

void prof_end(int token, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (token < 0 || token >= int(g_pending.size())) return;
  (void)hipEventRecord(g_pending[token].stop, st);
}

}  // namespace bf

using namespace bf;

extern "C" int bf_version(void) { return 100; }

extern "C" const char* bf_last_error(void) { return bf::g_error; }

extern "C" int bf_prof_enable(int32_t on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_on = on != 0;
  return BF_OK;
}

extern "C" int bf_prof_reset(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  for (auto& p : g_pending) {
    (void)hipEventSynchronize(p.stop);
    g_free_events.push_back(p.start);
    g_free_events.push_back(p.stop);
  }
  g_pending.clear();
  g_stats.clear();
  return BF_OK;
}

extern "C" int bf_prof_collect(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  for (auto& p : g_pending) {
    BF_CHECK_HIP(hipEventSynchronize(p.stop));
    float ms = 0.f;
    BF_CHECK_HIP(hipEventElapsedTime(&ms, p.start, p.stop));
    bool found = false;
    for (auto& s : g_stats) {
      if (s.name == p.name) {
        s.total_ms += ms;
        s.launches += 1;
        found = true;
        break;
      }
    }
    if (!found) g_stats.push_back(Stat{p.name, double(ms), 1});
    g_free_events.push_back(p.start);
    g_free_events.push_back(p.stop);
  }
  g_pending.clear();
  return BF_OK;
}

extern "C" int32_t bf_prof_count(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  return int32_t(g_stats.size());
}

extern "C" int bf_prof_get(int32_t i, const char** name, double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  BF_CHECK_ARG(i >= 0 && i < int32_t(g_stats.size()) && name && total_ms && launches, "prof_get: bad index");
  *name = g_stats[i].name.c_str();
  *total_ms = g_stats[i].total_ms;
  *launches = g_stats[i].launches;
  return BF_OK;
}
