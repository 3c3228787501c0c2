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

// The timer's lists live in one heap object that is created on first use and
// never freed: the library then has no static destructor of its own to run
// while the process exits (when the HIP runtime and a profiler's tool library
// may already be tearing down).
struct ProfState {
  std::vector<Pending> pending;
  std::vector<hipEvent_t> free_events;
  std::vector<Stat> stats;
};

std::mutex g_prof_mu;
bool g_prof_on = false;
thread_local bool t_prof_paused = false;

ProfState& prof_state() {
  static ProfState* s = new ProfState();
  return *s;
}

hipEvent_t take_event() {
  auto& fe = prof_state().free_events;
  if (!fe.empty()) {
    hipEvent_t e = fe.back();
    fe.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

}  // namespace

bool prof_enabled() { return g_prof_on && !t_prof_paused; }

ProfPause::ProfPause() : prev(t_prof_paused) { t_prof_paused = true; }
ProfPause::~ProfPause() { t_prof_paused = prev; }

void prof_begin(const char* name, hipStream_t st, int* token) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  *token = -1;
  hipEvent_t a = take_event(), b = take_event();
  if (!a || !b) return;
  if (hipEventRecord(a, st) != hipSuccess) return;
  auto& pending = prof_state().pending;
  pending.push_back(Pending{name, a, b});
  *token = int(pending.size()) - 1;
}

void prof_end(int token, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  auto& pending = prof_state().pending;
  if (token < 0 || token >= int(pending.size())) return;
  (void)hipEventRecord(pending[token].stop, st);
}

}  // namespace bf

using namespace bf;

extern "C" int bf_version(void) { return BF_ABI_VERSION; }

extern "C" const char* bf_last_error(void) { return bf::g_error; }

extern "C" int bf_prof_enable(int32_t on) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof_on = on != 0;
  return BF_OK;
}

extern "C" int bf_prof_reset(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  ProfState& ps = prof_state();
  for (auto& p : ps.pending) {
    (void)hipEventSynchronize(p.stop);
    ps.free_events.push_back(p.start);
    ps.free_events.push_back(p.stop);
  }
  ps.pending.clear();
  ps.stats.clear();
  return BF_OK;
}

extern "C" int bf_prof_collect(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  ProfState& ps = prof_state();
  for (auto& p : ps.pending) {
    BF_CHECK_HIP(hipEventSynchronize(p.stop));
    float ms = 0.f;
    BF_CHECK_HIP(hipEventElapsedTime(&ms, p.start, p.stop));
    bool found = false;
    for (auto& s : ps.stats) {
      if (s.name == p.name) {
        s.total_ms += ms;
        s.launches += 1;
        found = true;
        break;
      }
    }
    if (!found) ps.stats.push_back(Stat{p.name, double(ms), 1});
    ps.free_events.push_back(p.start);
    ps.free_events.push_back(p.stop);
  }
  ps.pending.clear();
  return BF_OK;
}

extern "C" int32_t bf_prof_count(void) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  return int32_t(prof_state().stats.size());
}

extern "C" int bf_prof_get(int32_t i, const char** name, double* total_ms, int64_t* launches) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  const auto& stats = prof_state().stats;
  BF_CHECK_ARG(i >= 0 && i < int32_t(stats.size()) && name && total_ms && launches, "prof_get: bad index");
  *name = stats[i].name.c_str();
  *total_ms = stats[i].total_ms;
  *launches = stats[i].launches;
  return BF_OK;
}
