// Optional per-kernel timing: while enabled, every launch of the library is
// bracketed by two hipEvents recorded on its own stream; pisa_profile_end
// waits for them and returns the summed duration and launch count per kernel.
// Disabled (the default) it costs one branch per launch.

#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "pisa_device.h"
#include "pisa_internal.h"

namespace pisa {

namespace {

struct Record {
  const char* name;
  hipEvent_t start, stop;
};

std::mutex g_mutex;
bool g_enabled = false;
std::vector<Record> g_records;

}  // namespace

ProfScope::ProfScope(const char* name, hipStream_t stream) : name_(name), stream_(stream) {
  if (!g_enabled) return;
  if (hipEventCreate(&start_) != hipSuccess) return;
  if (hipEventCreate(&stop_) != hipSuccess) {
    (void)hipEventDestroy(start_);
    return;
  }
  (void)hipEventRecord(start_, stream_);
  armed_ = true;
}

ProfScope::~ProfScope() {
  if (!armed_) return;
  (void)hipEventRecord(stop_, stream_);
  std::lock_guard<std::mutex> lock(g_mutex);
  g_records.push_back({name_, start_, stop_});
}

}  // namespace pisa

using namespace pisa;

extern "C" int pisa_profile_begin(void) {
  std::lock_guard<std::mutex> lock(g_mutex);
  for (auto& r : g_records) {
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  g_records.clear();
  g_enabled = true;
  return PISA_OK;
}

extern "C" int pisa_profile_end(pisa_kernel_time* out, int32_t capacity, int32_t* count) {
  std::vector<Record> records;
  {
    std::lock_guard<std::mutex> lock(g_mutex);
    g_enabled = false;
    records.swap(g_records);
  }
  std::vector<pisa_kernel_time> agg;
  int rc = PISA_OK;
  for (auto& r : records) {
    float ms = 0.f;
    if (hipEventSynchronize(r.stop) != hipSuccess ||
        hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess)
      rc = fail(PISA_ERR_LAUNCH, "profiling event of %s failed", r.name);
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
    size_t i = 0;
    while (i < agg.size() && strncmp(agg[i].name, r.name, sizeof(agg[i].name)) != 0) ++i;
    if (i == agg.size()) {
      pisa_kernel_time t;
      memset(&t, 0, sizeof(t));
      strncpy(t.name, r.name, sizeof(t.name) - 1);
      agg.push_back(t);
    }
    agg[i].launches += 1;
    agg[i].total_ms += ms;
  }
  const int n = (int)agg.size();
  if (count) *count = n;
  for (int i = 0; i < n && i < capacity; ++i) out[i] = agg[i];
  return rc;
}
