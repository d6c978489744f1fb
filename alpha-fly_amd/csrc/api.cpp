// Version, error reporting and launch timing of the C ABI.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "common.hpp"

namespace fly {
namespace {
thread_local std::string g_last_error;

struct Record {
  int cls;
  hipEvent_t start, stop;
};

struct Profiler {
  std::mutex mu;
  bool on = false;
  std::vector<Record> records;
  std::vector<hipEvent_t> spare;
  hipEvent_t take() {
    if (!spare.empty()) {
      hipEvent_t e = spare.back();
      spare.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    FLY_HIP(hipEventCreate(&e));
    return e;
  }
};

Profiler &profiler() {
  static Profiler p;
  return p;
}
}  // namespace

void set_error(const std::string &msg) { g_last_error = msg; }

namespace {
thread_local int g_quiet = 0;
}  // namespace

NoLaunchEvents::NoLaunchEvents() { ++g_quiet; }
NoLaunchEvents::~NoLaunchEvents() { --g_quiet; }

LaunchTimer::LaunchTimer(int kernel_class, hipStream_t st) : cls_(kernel_class), st_(st) {
  if (g_quiet) return;
  Profiler &p = profiler();
  std::lock_guard<std::mutex> lock(p.mu);
  if (!p.on) return;
  start_ = p.take();
  FLY_HIP(hipEventRecord(start_, st_));
}

LaunchTimer::~LaunchTimer() {
  if (!start_) return;
  Profiler &p = profiler();
  std::lock_guard<std::mutex> lock(p.mu);
  hipEvent_t stop = nullptr;
  if (hipEventCreate(&stop) != hipSuccess || hipEventRecord(stop, st_) != hipSuccess) {
    p.spare.push_back(start_);
    return;
  }
  p.records.push_back({cls_, start_, stop});
}
}  // namespace fly

using namespace fly;

extern "C" int fly_abi_version(void) { return FLY_ABI_VERSION; }

extern "C" const char *fly_last_error(void) { return fly::g_last_error.c_str(); }

extern "C" int fly_profile_enable(int32_t on) {
  return guard([&] {
    Profiler &p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    if (on) {
      for (const Record &r : p.records) {
        FLY_HIP(hipEventSynchronize(r.stop));
        p.spare.push_back(r.start);
        p.spare.push_back(r.stop);
      }
      p.records.clear();
    }
    p.on = on != 0;
  });
}

extern "C" int fly_profile_read(double *ms, int64_t *launches) {
  return guard([&] {
    Profiler &p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    double tot[FLY_K_CLASSES] = {0, 0, 0, 0};
    int64_t cnt[FLY_K_CLASSES] = {0, 0, 0, 0};
    for (const Record &r : p.records) {
      FLY_HIP(hipEventSynchronize(r.stop));
      float t = 0.f;
      FLY_HIP(hipEventElapsedTime(&t, r.start, r.stop));
      if (r.cls >= 0 && r.cls < FLY_K_CLASSES) {
        tot[r.cls] += t;
        cnt[r.cls] += 1;
      }
    }
    for (int c = 0; c < FLY_K_CLASSES; ++c) {
      if (ms) ms[c] = tot[c];
      if (launches) launches[c] = cnt[c];
    }
  });
}

extern "C" int64_t fly_profile_launches(int32_t *cls, double *ms, int64_t cap) {
  int64_t n = -1;
  const int rc = guard([&] {
    Profiler &p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    n = (int64_t)p.records.size();
    for (int64_t i = 0; i < std::min<int64_t>(n, cap); ++i) {
      const Record &r = p.records[(size_t)i];
      FLY_HIP(hipEventSynchronize(r.stop));
      float t = 0.f;
      FLY_HIP(hipEventElapsedTime(&t, r.start, r.stop));
      if (cls) cls[i] = r.cls;
      if (ms) ms[i] = t;
    }
  });
  return rc == FLY_OK ? n : -1;
}
