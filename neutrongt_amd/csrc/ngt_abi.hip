// Error reporting, version query and the optional per-kernel timing used by
// the benchmark (events recorded on the launch stream around each kernel).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "ngt_common.h"

namespace ngt {
namespace {
thread_local char g_last_error[512] = "";

struct Pending {
  const char* name;
  hipEvent_t start;
  hipEvent_t stop;
};

std::atomic<bool> g_timing{false};
std::mutex g_mu;
std::vector<Pending> g_pending;      // completed start/stop pairs
std::vector<Pending> g_open;         // started, not yet stopped (stack per call site)
std::vector<hipEvent_t> g_pool;      // reusable events

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
}  // namespace

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

bool timing_enabled() { return g_timing.load(std::memory_order_relaxed); }

void timing_record(const char* name, hipStream_t st, bool start) {
  std::lock_guard<std::mutex> lk(g_mu);
  // A record that fails leaves no half pair behind: the kernel goes untimed.
  if (start) {
    hipEvent_t e = take_event();
    if (!e) return;
    if (hipEventRecord(e, st) != hipSuccess) {
      g_pool.push_back(e);
      return;
    }
    g_open.push_back(Pending{name, e, nullptr});
    return;
  }
  for (size_t i = g_open.size(); i-- > 0;) {
    if (g_open[i].name == name) {
      Pending p = g_open[i];
      g_open.erase(g_open.begin() + static_cast<long>(i));
      hipEvent_t e = take_event();
      if (e && hipEventRecord(e, st) == hipSuccess) {
        p.stop = e;
        g_pending.push_back(p);
        return;
      }
      if (e) g_pool.push_back(e);
      g_pool.push_back(p.start);
      return;
    }
  }
}

}  // namespace ngt

extern "C" int ngt_abi_version(void) { return NGT_ABI_VERSION; }

extern "C" const char* ngt_last_error(void) { return ngt::g_last_error; }

extern "C" int ngt_timing_enable(int on) {
  std::lock_guard<std::mutex> lk(ngt::g_mu);
  ngt::g_timing.store(on != 0);
  return NGT_OK;
}

// Waits for every recorded pair, then writes "name count total_ms\n" lines
// (one per kernel name, in name order) into buf and forgets the records.
extern "C" int ngt_timing_summary(char* buf, size_t len) {
  using namespace ngt;
  std::lock_guard<std::mutex> lk(g_mu);
  std::map<std::string, std::pair<long long, double>> agg;
  int rc = NGT_OK;
  for (const Pending& p : g_pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) != hipSuccess ||
        hipEventElapsedTime(&ms, p.start, p.stop) != hipSuccess)
      rc = set_error(NGT_ERR_HIP, "ngt_timing_summary: event query failed");
    auto& a = agg[p.name];
    a.first += 1;
    a.second += ms;
    g_pool.push_back(p.start);
    g_pool.push_back(p.stop);
  }
  g_pending.clear();
  std::string out;
  char line[256];
  for (const auto& kv : agg) {
    snprintf(line, sizeof(line), "%s %lld %.6f\n", kv.first.c_str(), kv.second.first,
             kv.second.second);
    out += line;
  }
  if (buf && len > 0) {
    const size_t n = out.size() < len - 1 ? out.size() : len - 1;
    memcpy(buf, out.data(), n);
    buf[n] = 0;
    if (out.size() >= len) rc = set_error(NGT_ERR_ARG, "ngt_timing_summary: buffer too small");
  }
  return rc;
}
