// Library-wide C ABI entry points (version, thread-local error text) and the library's second stream.
#include <cstring>
#include <mutex>
#include <string>

#include "pdm_common.h"

namespace pdm {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

namespace {

constexpr int kMaxDevices = 64;
constexpr int kSideEvents = 16;

struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork[kSideEvents] = {}, join[kSideEvents] = {};
  int next = 0;
  bool failed = false;
};

std::mutex g_side_mu;
SideStream g_side[kMaxDevices];

// Called with g_side_mu held.
SideStream* side_stream(int dev, hipStream_t caller) {
  SideStream& ss = g_side[dev];
  if (ss.s) return &ss;
  if (ss.failed) return nullptr;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(caller, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return nullptr;  // made outside a capture only
  }
  bool ok = hipStreamCreateWithFlags(&ss.s, hipStreamNonBlocking) == hipSuccess;
  for (int i = 0; ok && i < kSideEvents; ++i)
    ok = hipEventCreateWithFlags(&ss.fork[i], hipEventDisableTiming) == hipSuccess &&
         hipEventCreateWithFlags(&ss.join[i], hipEventDisableTiming) == hipSuccess;
  if (!ok) {
    for (int i = 0; i < kSideEvents; ++i) {
      if (ss.fork[i]) (void)hipEventDestroy(ss.fork[i]);
      if (ss.join[i]) (void)hipEventDestroy(ss.join[i]);
      ss.fork[i] = ss.join[i] = nullptr;
    }
    if (ss.s) (void)hipStreamDestroy(ss.s);
    ss.s = nullptr;
    (void)hipGetLastError();
    ss.failed = true;
    return nullptr;
  }
  return &ss;
}

}  // namespace

int side_fork(hipStream_t caller, SideFork& f) {
  f = SideFork{};
  PDM_CHECK_HIP(hipGetDevice(&f.dev));
  PDM_CHECK_ARG(f.dev >= 0 && f.dev < kMaxDevices, "device index out of range");
  std::lock_guard<std::mutex> lk(g_side_mu);
  SideStream* ss = side_stream(f.dev, caller);
  if (!ss) return PDM_OK;
  f.ev = ss->next;
  ss->next = (ss->next + 1) % kSideEvents;
  PDM_CHECK_HIP(hipEventRecord(ss->fork[f.ev], caller));
  PDM_CHECK_HIP(hipStreamWaitEvent(ss->s, ss->fork[f.ev], 0));
  f.side = ss->s;
  return PDM_OK;
}

int side_join(hipStream_t caller, const SideFork& f) {
  if (!f.side) return PDM_OK;
  SideStream& ss = g_side[f.dev];
  PDM_CHECK_HIP(hipEventRecord(ss.join[f.ev], f.side));
  PDM_CHECK_HIP(hipStreamWaitEvent(caller, ss.join[f.ev], 0));
  return PDM_OK;
}

}  // namespace pdm

extern "C" int32_t pdm_abi_version(void) { return 10000; }

extern "C" size_t pdm_last_error(char* buf, size_t n) {
  const std::string& e = pdm::g_last_error;
  if (buf && n > 0) {
    const size_t k = e.size() < n - 1 ? e.size() : n - 1;
    std::memcpy(buf, e.data(), k);
    buf[k] = '\0';
  }
  return e.size();
}
