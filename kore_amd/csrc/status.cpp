// Per-thread error reporting for the C ABI.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "../../include/kore_amd.h"
#include "kore_common.hpp"

namespace kore {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(KORE_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  g_last_error[0] = '\0';
  return KORE_OK;
}

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Scratch for the packed and split-K paths: one grow-only device buffer per (device,
// stream), kept until the process ends.  Work on one stream runs in order, so the next
// call on that stream may reuse the buffer as soon as it is enqueued; different streams
// get different buffers.  Growing synchronises the stream before freeing the old buffer.
// A capturing stream gets none (see scratch_alloc).
namespace {
struct ScratchSlot {
  hipStream_t stream;
  void* ptr;
  size_t bytes;
};
constexpr int kScratchSlots = 16;
ScratchSlot g_scratch[64][kScratchSlots] = {};
std::mutex g_scratch_mu;  // host threads may call on different streams at once
}  // namespace

void* scratch_alloc(size_t bytes, hipStream_t stream) {
  // Under graph capture: no scratch, so the caller takes a path that needs none.  A
  // captured graph may be replayed on any stream, concurrently with eager work on the
  // stream it was captured on, so it must not hold the cached buffer; graphs holding
  // stream-ordered allocation nodes instead faulted on replay on this platform.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  ScratchSlot* slot = nullptr;
  for (int i = 0; i < kScratchSlots && slot == nullptr; ++i)
    if (g_scratch[dev][i].ptr != nullptr && g_scratch[dev][i].stream == stream) slot = &g_scratch[dev][i];
  for (int i = 0; i < kScratchSlots && slot == nullptr; ++i)
    if (g_scratch[dev][i].ptr == nullptr) slot = &g_scratch[dev][i];
  if (slot == nullptr) return nullptr;  // more streams than slots: fallback path
  if (slot->ptr != nullptr && slot->bytes >= bytes) return slot->ptr;
  if (slot->ptr != nullptr) {
    if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
    (void)hipFree(slot->ptr);
    slot->ptr = nullptr;
    slot->bytes = 0;
  }
  const size_t want = (bytes + (1u << 20) - 1) / (1u << 20) * (1u << 20);  // whole MiB
  void* p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess || p == nullptr) {
    (void)hipGetLastError();
    return nullptr;
  }
  slot->stream = stream;
  slot->ptr = p;
  slot->bytes = want;
  return p;
}

void scratch_free(void*, hipStream_t) {}  // the buffer stays with its stream

}  // namespace kore

extern "C" const char* kore_last_error(void) { return kore::g_last_error; }
extern "C" int kore_abi_version(void) { return 100; }
