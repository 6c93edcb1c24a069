// Launch timer of the C ABI's t2w_timer_arm / t2w_timer_read (a measurement aid shared by the DiT and HiFT layers).
#pragma once

#include <hip/hip_runtime.h>

#include <vector>

namespace t2w {

// Launch timer (t2w_timer_arm / t2w_timer_read): while armed on this thread, instrumented launches on a stream that is
// not capturing are bracketed by a pair of HIP events and recorded with their kind and algorithmic HBM bytes.
struct TimedLaunch {
  int kind;
  double bytes;
  hipEvent_t e0, e1;
};
struct LaunchTimer {
  bool armed = false;
  int cap = 0;
  std::vector<TimedLaunch> v;
};
LaunchTimer& launch_timer();  // this thread's

template <class F>
hipError_t timed_launch(int kind, double bytes, hipStream_t st, F&& launch) {
  LaunchTimer& t = launch_timer();
  if (!t.armed || (int)t.v.size() >= t.cap) return launch();
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(st, &cs);
  if (e != hipSuccess) return e;
  if (cs != hipStreamCaptureStatusNone) return launch();  // events are read back: nothing is timed inside a graph
  TimedLaunch x{kind, bytes, nullptr, nullptr};
  if ((e = hipEventCreate(&x.e0)) != hipSuccess) return e;
  if ((e = hipEventCreate(&x.e1)) != hipSuccess) {
    (void)hipEventDestroy(x.e0);
    return e;
  }
  t.v.push_back(x);
  if ((e = hipEventRecord(x.e0, st)) != hipSuccess) return e;
  if ((e = launch()) != hipSuccess) return e;
  return hipEventRecord(x.e1, st);
}

}  // namespace t2w
