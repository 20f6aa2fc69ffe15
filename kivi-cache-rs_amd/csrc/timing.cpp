// timing.cpp — per-kernel-family launch timing for measurement harnesses.
//
// While enabled, TimedLaunch brackets one kernel launch with a pair of HIP events recorded
// on the launch stream, so the elapsed time is that launch's duration on the device (the
// queue runs one stream's work in order). Pending pairs are resolved lazily by
// kivi_timing_read, which waits for them. Events are pooled per device.
#include "common.hpp"
#include "kivi.h"

#include <cstdio>
#include <map>
#include <mutex>
#include <vector>

namespace kivi {
namespace {

struct Pending {
  int family;
  int device;
  hipEvent_t start, end;
  double bytes;
};

struct Registry {
  std::mutex mu;
  bool enabled = false;
  std::vector<Pending> pending;
  std::map<int, std::vector<hipEvent_t>> pool;
  kivi_kernel_timing totals[KIVI_KERNEL_FAMILIES]{};

  hipEvent_t take(int device) {
    auto& v = pool[device];
    if (!v.empty()) {
      hipEvent_t e = v.back();
      v.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }

  // Resolve every pending pair into the totals (waits for the events).
  hipError_t resolve(bool keep) {
    hipError_t first = hipSuccess;
    for (const Pending& p : pending) {
      float ms = 0.f;
      hipError_t e = hipEventSynchronize(p.end);
      if (e == hipSuccess) e = hipEventElapsedTime(&ms, p.start, p.end);
      if (e == hipSuccess && keep) {
        totals[p.family].launches += 1;
        totals[p.family].total_ms += ms;
        totals[p.family].bytes += p.bytes;
      }
      if (e != hipSuccess && first == hipSuccess) first = e;
      pool[p.device].push_back(p.start);
      pool[p.device].push_back(p.end);
    }
    pending.clear();
    return first;
  }
};

Registry& registry() {
  static Registry* r = new Registry();  // never destroyed: events may outlive static teardown
  return *r;
}

}  // namespace

TimedLaunch::TimedLaunch(int family, hipStream_t stream, double bytes)
    : family_(family), stream_(stream), bytes_(bytes) {
  Registry& r = registry();
  std::lock_guard<std::mutex> lock(r.mu);
  if (!r.enabled || family < 0 || family >= KIVI_KERNEL_FAMILIES) return;
  if (hipGetDevice(&device_) != hipSuccess) return;
  start_ = r.take(device_);
  end_ = r.take(device_);
  if (start_ == nullptr || end_ == nullptr || hipEventRecord(start_, stream_) != hipSuccess) {
    if (start_ != nullptr) r.pool[device_].push_back(start_);
    if (end_ != nullptr) r.pool[device_].push_back(end_);
    start_ = end_ = nullptr;
  }
}

TimedLaunch::~TimedLaunch() {
  if (start_ == nullptr) return;
  Registry& r = registry();
  std::lock_guard<std::mutex> lock(r.mu);
  if (hipEventRecord(end_, stream_) != hipSuccess) {
    r.pool[device_].push_back(start_);
    r.pool[device_].push_back(end_);
    return;
  }
  r.pending.push_back(Pending{family_, device_, start_, end_, bytes_});
}

}  // namespace kivi

using namespace kivi;

extern "C" {

void kivi_timing_enable(int32_t enable) {
  Registry& r = registry();
  std::lock_guard<std::mutex> lock(r.mu);
  (void)r.resolve(false);
  for (auto& t : r.totals) t = kivi_kernel_timing{};
  r.enabled = enable != 0;
}

kivi_status kivi_timing_read(int32_t family, kivi_kernel_timing* out, kivi_error* err) {
  kivi_error e{};
  if (out == nullptr) {
    e.code = KIVI_ERR_NULL_ARGUMENT;
    snprintf(e.name, sizeof(e.name), "out");
    snprintf(e.message, sizeof(e.message), "out must not be null");
  } else if (family < 0 || family >= KIVI_KERNEL_FAMILIES) {
    e.code = KIVI_ERR_UNSUPPORTED;
    e.a = static_cast<uint64_t>(static_cast<uint32_t>(family));
    e.b = KIVI_KERNEL_FAMILIES - 1;
    snprintf(e.name, sizeof(e.name), "kernel family");
    snprintf(e.message, sizeof(e.message), "kernel family %llu is outside this build's limit %llu",
             static_cast<unsigned long long>(e.a), static_cast<unsigned long long>(e.b));
  } else {
    Registry& r = registry();
    std::lock_guard<std::mutex> lock(r.mu);
    const hipError_t h = r.resolve(true);
    *out = r.totals[family];
    if (h != hipSuccess) {
      e.code = KIVI_ERR_DEVICE;
      snprintf(e.message, sizeof(e.message), "HIP error in kernel timing: %s", hipGetErrorString(h));
    }
  }
  if (err != nullptr) *err = e;
  return static_cast<kivi_status>(e.code);
}

}  // extern "C"
