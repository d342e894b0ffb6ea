// Side streams that execute concurrently with the serving stream.
//
// HIP maps streams onto a fixed set of hardware queues per process
// (GPU_MAX_HW_QUEUES, 4 by default), round-robin in creation order, and two
// streams on one queue execute in order: a Load or Store stream that lands
// on the serving stream's queue serializes with the model's compute. Which
// queue a new stream gets depends on every stream created before it
// (torch's stream pools included), so it is measured instead of assumed: a
// candidate non-blocking stream is kept only when a short spin kernel on it
// overlaps one on the serving stream and one on every stream already kept.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <vector>

#include "cbk_common.hpp"

namespace {

// Spins for `ticks` of the constant-rate wall clock; the iteration cap ends
// the loop even if the clock never advanced.
__global__ void spin_kernel(long long ticks, long long max_iters) {
  const long long t0 = wall_clock64();
  for (long long i = 0; i < max_iters; ++i) {
    if (wall_clock64() - t0 >= ticks) break;
    __builtin_amdgcn_s_sleep(4);
  }
}

struct Probe {
  long long ticks;
  long long max_iters;
  float spin_ms;
};

// *overlap = both spins together took well under two spins' time
int spins_overlap(hipStream_t a, hipStream_t b, const Probe& p, bool* overlap) {
  hipEvent_t start = nullptr, end_a = nullptr, end_b = nullptr;
  hipError_t e = hipEventCreate(&start);
  if (e == hipSuccess) e = hipEventCreate(&end_a);
  if (e == hipSuccess) e = hipEventCreate(&end_b);
  if (e == hipSuccess) e = hipEventRecord(start, a);
  if (e == hipSuccess) e = hipStreamWaitEvent(b, start, 0);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(spin_kernel, dim3(1), dim3(64), 0, a, p.ticks, p.max_iters);
    hipLaunchKernelGGL(spin_kernel, dim3(1), dim3(64), 0, b, p.ticks, p.max_iters);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipEventRecord(end_a, a);
  if (e == hipSuccess) e = hipEventRecord(end_b, b);
  if (e == hipSuccess) e = hipEventSynchronize(end_a);
  if (e == hipSuccess) e = hipEventSynchronize(end_b);
  float ta = 0.f, tb = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ta, start, end_a);
  if (e == hipSuccess) e = hipEventElapsedTime(&tb, start, end_b);
  for (hipEvent_t ev : {start, end_a, end_b})
    if (ev) (void)hipEventDestroy(ev);
  if (e != hipSuccess) return cbk::set_error(CBK_ERR_LAUNCH, "stream probe: %s", hipGetErrorString(e));
  *overlap = std::max(ta, tb) < 1.5f * p.spin_ms;
  return CBK_OK;
}

}  // namespace

extern "C" {

int cbk_side_streams(cbk_stream_t serving, int32_t n, int32_t max_candidates, float spin_ms,
                     cbk_stream_t* out_streams, int32_t* found) {
  cbk::clear_error();
  CBK_REQUIRE(out_streams != nullptr && found != nullptr, "NULL output");
  CBK_REQUIRE(n > 0 && n <= 16 && max_candidates >= n && max_candidates <= 64, "n / max_candidates out of range");
  CBK_REQUIRE(spin_ms > 0.f && spin_ms <= 5.f, "spin_ms must be in (0, 5]");
  *found = 0;
  int device = 0;
  int rate_khz = 0;
  if (hipGetDevice(&device) != hipSuccess ||
      hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, device) != hipSuccess || rate_khz <= 0)
    return cbk::set_error(CBK_ERR_LAUNCH, "wall clock rate unavailable");
  Probe p;
  p.spin_ms = spin_ms;
  p.ticks = static_cast<long long>(double(spin_ms) * rate_khz);
  p.max_iters = p.ticks * 64 + 1024;  // far above the iterations the spin needs
  hipStream_t serve = static_cast<hipStream_t>(serving);
  if (hipStreamSynchronize(serve) != hipSuccess)
    return cbk::set_error(CBK_ERR_LAUNCH, "serving stream synchronize failed");
  std::vector<hipStream_t> kept, rejected;
  int rc = CBK_OK;
  for (int32_t c = 0; c < max_candidates && int32_t(kept.size()) < n && rc == CBK_OK; ++c) {
    hipStream_t s = nullptr;
    if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
      rc = cbk::set_error(CBK_ERR_LAUNCH, "hipStreamCreateWithFlags failed");
      break;
    }
    bool ok = true;
    rc = spins_overlap(serve, s, p, &ok);
    for (size_t k = 0; rc == CBK_OK && ok && k < kept.size(); ++k) rc = spins_overlap(kept[k], s, p, &ok);
    (rc == CBK_OK && ok ? kept : rejected).push_back(s);
  }
  // rejected candidates live until the search ends, so a later candidate is
  // not handed the queue one of them had
  for (hipStream_t s : rejected) (void)hipStreamDestroy(s);
  if (rc != CBK_OK) {
    for (hipStream_t s : kept) (void)hipStreamDestroy(s);
    return rc;
  }
  for (size_t k = 0; k < kept.size(); ++k) out_streams[k] = kept[k];
  *found = int32_t(kept.size());
  return CBK_OK;
}

int cbk_stream_destroy(cbk_stream_t stream) {
  cbk::clear_error();
  CBK_REQUIRE(stream != nullptr, "NULL stream");
  if (hipStreamDestroy(static_cast<hipStream_t>(stream)) != hipSuccess)
    return cbk::set_error(CBK_ERR_LAUNCH, "hipStreamDestroy failed");
  return CBK_OK;
}

}  // extern "C"
