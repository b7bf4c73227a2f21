// Opt-in kernel timing: while enabled, every library launch is bracketed by a
// pair of HIP events recorded on the launch stream; ns_profile_end() waits for
// them and reports per-kernel launch counts and total milliseconds.
#include <atomic>
#include <mutex>
#include <string.h>
#include <string>
#include <vector>

#include "../../include/nanospec_hip.h"
#include "ns_profile.h"

namespace ns {
namespace {

struct Record {
  const char* name;
  hipEvent_t start, stop;
  hipError_t err;   // a failed stop record: reported by ns_profile_end
};

std::mutex g_mu;
// read without the mutex on every launch (profiling()), written under it
std::atomic<bool> g_on{false};
std::vector<Record> g_records;
std::vector<hipEvent_t> g_pool;
// ns_profile_select: ",name1,name2," or empty (every launch timed)
std::string g_only;

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

bool profiling() { return g_on.load(std::memory_order_acquire); }

void* profile_start(const char* name, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_on.load(std::memory_order_relaxed)) return nullptr;
  if (!g_only.empty() && g_only.find("," + std::string(name) + ",") == std::string::npos) return nullptr;
  Record r{name, take_event(), take_event(), hipSuccess};
  if (!r.start || !r.stop || hipEventRecord(r.start, st) != hipSuccess) {
    if (r.start) g_pool.push_back(r.start);
    if (r.stop) g_pool.push_back(r.stop);
    return nullptr;   // this launch goes untimed
  }
  g_records.push_back(r);
  return reinterpret_cast<void*>(g_records.size());
}

void profile_stop(void* token, hipStream_t st) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!token) return;
  const size_t i = reinterpret_cast<size_t>(token) - 1;
  if (i < g_records.size()) g_records[i].err = hipEventRecord(g_records[i].stop, st);
}

}  // namespace ns

extern "C" {

int ns_profile_select(const char* names) {
  std::lock_guard<std::mutex> lk(ns::g_mu);
  ns::g_only = names && *names ? "," + std::string(names) + "," : std::string();
  return NS_OK;
}

int ns_profile_begin(void) {
  std::lock_guard<std::mutex> lk(ns::g_mu);
  ns::g_on.store(true, std::memory_order_release);
  return NS_OK;
}

int ns_profile_end(ns_kernel_time* out, int capacity, int* count) {
  std::lock_guard<std::mutex> lk(ns::g_mu);
  ns::g_on.store(false, std::memory_order_release);
  std::vector<std::string> names;
  std::vector<ns_kernel_time> acc;
  int status = NS_OK;
  for (auto& r : ns::g_records) {
    float ms = 0.f;
    hipError_t e = r.err;
    if (e == hipSuccess) e = hipEventSynchronize(r.stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.start, r.stop);
    if (e != hipSuccess && status == NS_OK) status = (int)e;
    size_t j = 0;
    while (j < names.size() && names[j] != r.name) ++j;
    if (j == names.size()) {
      names.push_back(r.name);
      ns_kernel_time t;
      memset(&t, 0, sizeof(t));
      strncpy(t.name, r.name, sizeof(t.name) - 1);
      acc.push_back(t);
    }
    acc[j].launches += 1;
    acc[j].total_ms += ms;
    ns::g_pool.push_back(r.start);
    ns::g_pool.push_back(r.stop);
  }
  ns::g_records.clear();
  const int n = (int)acc.size();
  if (count) *count = n;
  for (int i = 0; i < n && i < capacity && out; ++i) out[i] = acc[i];
  return status;
}

}  // extern "C"
