// Kernel timing probes (diagnostic; see tsattn_profile_enable in tsattn.h).
//
// Each probed launch records a start and a stop hipEvent on the launch's own
// stream.  Events come from a recycled pool so steady-state probing does not
// allocate.  tsattn_profile_read synchronises on the recorded stop events,
// folds the elapsed times into per-name totals and recycles the events.
#include <string.h>

#include <atomic>
#include <mutex>
#include <string>
#include <vector>

#include "tsattn_internal.h"

namespace tsattn {
namespace {

struct Pending {
  const char *name;
  hipEvent_t start, stop;
};
struct Total {
  std::string name;
  long long launches = 0;
  double ms = 0.0;
};

std::mutex g_mu;
// Read without the mutex on every launch; the pools and totals stay under it.
std::atomic<bool> g_on{false};
std::vector<hipEvent_t> g_pool;
std::vector<Pending> g_pending;
std::vector<Total> g_totals;
thread_local Pending g_open{nullptr, nullptr, nullptr};

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void fold_locked() {
  for (const Pending &p : g_pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      Total *t = nullptr;
      for (Total &x : g_totals)
        if (x.name == p.name) t = &x;
      if (!t) {
        g_totals.push_back(Total{p.name, 0, 0.0});
        t = &g_totals.back();
      }
      t->launches += 1;
      t->ms += ms;
    }
    g_pool.push_back(p.start);
    g_pool.push_back(p.stop);
  }
  g_pending.clear();
}

}  // namespace

bool probes_on() { return g_on.load(std::memory_order_relaxed); }

void probe_begin(const char *name, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_open = Pending{name, take_event(), take_event()};
  if (g_open.start) hipEventRecord(g_open.start, st);
}

void probe_end(hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_open.start || !g_open.stop) return;
  hipEventRecord(g_open.stop, st);
  g_pending.push_back(g_open);
  g_open = Pending{nullptr, nullptr, nullptr};
}

}  // namespace tsattn

extern "C" {

int tsattn_profile_enable(int on) {
  std::lock_guard<std::mutex> lk(tsattn::g_mu);
  tsattn::g_on.store(on != 0, std::memory_order_relaxed);
  return TSATTN_OK;
}

int tsattn_profile_reset(void) {
  std::lock_guard<std::mutex> lk(tsattn::g_mu);
  tsattn::fold_locked();
  tsattn::g_totals.clear();
  return TSATTN_OK;
}

int tsattn_profile_read(int index, char *name, size_t name_len, long long *launches,
                        double *total_ms) {
  std::lock_guard<std::mutex> lk(tsattn::g_mu);
  tsattn::fold_locked();
  if (index < 0 || index >= static_cast<int>(tsattn::g_totals.size())) return -1;
  const tsattn::Total &t = tsattn::g_totals[index];
  if (name && name_len) {
    strncpy(name, t.name.c_str(), name_len - 1);
    name[name_len - 1] = '\0';
  }
  if (launches) *launches = t.launches;
  if (total_ms) *total_ms = t.ms;
  return TSATTN_OK;
}

}  // extern "C"
