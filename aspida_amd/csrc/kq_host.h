// kq_host.h -- host-side helpers for the launchers' device queries.
//
// Device attribute, occupancy and kernel attribute queries have fallbacks
// (256 CUs, one resident workgroup per CU, no dynamic LDS), but when one
// fails it also leaves HIP's per-thread error set, which the next launch's
// own check would then report.  The helpers here clear only an error that a
// query itself left: with an error already pending from the calling thread's
// earlier work, they run nothing, so that error stays pending for that work's
// check, and they cache nothing either.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <mutex>

namespace kq {

// Runs f when no error is pending and clears whatever error f left; returns
// whether f ran.
template <class F>
inline bool query_clean(F&& f) {
  if (hipPeekAtLastError() != hipSuccess) return false;
  f();
  (void)hipGetLastError();
  return true;
}

// A query result computed once per process, when it can be run cleanly;
// until then each call returns `fallback` without caching it.
template <class T>
struct OnceQuery {
  std::atomic<bool> known{false};
  std::mutex mu;
  T value{};
  template <class F>
  T get(F&& f, const T& fallback) {
    if (known.load(std::memory_order_acquire)) return value;
    std::lock_guard<std::mutex> lk(mu);
    if (!known.load(std::memory_order_relaxed)) {
      T t{};
      if (!query_clean([&] { t = f(); })) return fallback;
      value = t;
      known.store(true, std::memory_order_release);
    }
    return value;
  }
};

}  // namespace kq
