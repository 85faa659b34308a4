// C-ABI utilities: error reporting, version, pointer probe, slot upload.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <new>
#include <thread>

#include "pl_common.h"

namespace {
thread_local char g_last_error[512] = {0};
}

void pl_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int pl_launch_status(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    pl_set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return PL_ERR_LAUNCH;
  }
  return PL_OK;
}

extern "C" int pl_version(void) { return 100; }

extern "C" const char* pl_last_error(void) { return g_last_error; }

extern "C" int pl_is_device_pointer(const void* ptr) {
  hipPointerAttribute_t attr;
  const hipError_t err = hipPointerGetAttributes(&attr, ptr);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    pl_set_error("hipPointerGetAttributes: %s", hipGetErrorString(err));
    return -1;
  }
  return (attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged) ? 1 : 0;
}

// Page-locked host memory of exactly `nbytes` (the caching host allocators
// of frameworks round requests up, e.g. to powers of two, which matters when
// adapter images fill most of the page-lockable memory).  A failed
// allocation returns null and clears the runtime's error state, so the
// caller can fall back to pageable memory.
extern "C" void* pl_host_alloc(int64_t nbytes) {
  if (nbytes <= 0) {
    pl_set_error("pl_host_alloc: size must be positive (got %lld)", (long long)nbytes);
    return nullptr;
  }
  void* p = nullptr;
  const hipError_t err = hipHostMalloc(&p, (size_t)nbytes, hipHostMallocDefault);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    pl_set_error("pl_host_alloc: %lld bytes: %s", (long long)nbytes, hipGetErrorString(err));
    return nullptr;
  }
  return p;
}

extern "C" int pl_host_free(void* ptr) {
  if (!ptr) return PL_OK;
  const hipError_t err = hipHostFree(ptr);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    pl_set_error("pl_host_free: %s", hipGetErrorString(err));
    return PL_ERR_LAUNCH;
  }
  return PL_OK;
}

// cache.py:138-145 copies each module's A and B separately with .to(device)
// and .copy_(); here one packed adapter image (all modules, compact ranks)
// moves with one host->device copy, followed by its 32-byte-per-module table
// row.  Both copies are ordered on `stream` (a side stream the caller orders
// against compute with events), so the table row never becomes visible to a
// kernel on that stream before the weights it points at.
extern "C" int pl_slot_upload(void* arena_dst, const void* host_src, int64_t nbytes,
                              void* table_dst, const void* table_src, int64_t table_bytes,
                              void* stream) {
  if (nbytes < 0 || table_bytes < 0 || (nbytes > 0 && (!arena_dst || !host_src)) ||
      (table_bytes > 0 && (!table_dst || !table_src))) {
    pl_set_error("pl_slot_upload: bad arguments");
    return PL_ERR_ARG;
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (nbytes > 0) {
    const hipError_t err =
        hipMemcpyAsync(arena_dst, host_src, (size_t)nbytes, hipMemcpyHostToDevice, s);
    if (err != hipSuccess) {
      pl_set_error("pl_slot_upload: weights copy failed: %s", hipGetErrorString(err));
      return PL_ERR_LAUNCH;
    }
  }
  if (table_bytes > 0) {
    const hipError_t err =
        hipMemcpyAsync(table_dst, table_src, (size_t)table_bytes, hipMemcpyHostToDevice, s);
    if (err != hipSuccess) {
      pl_set_error("pl_slot_upload: table copy failed: %s", hipGetErrorString(err));
      return PL_ERR_LAUNCH;
    }
  }
  return PL_OK;
}

namespace {

// A host -> host copy run in a stream's order (hipLaunchHostFunc).  Large
// copies are split over a few threads (one thread moves ~10 GB/s).
struct pl_staged_copy {
  void* dst;
  const void* src;
  int64_t n;
};

constexpr int kStageThreads = 8;
constexpr int64_t kStageSplitMin = 8 << 20;

void pl_staged_copy_run(void* arg) {
  pl_staged_copy* c = static_cast<pl_staged_copy*>(arg);
  char* dst = static_cast<char*>(c->dst);
  const char* src = static_cast<const char*>(c->src);
  const int64_t n = c->n;
  if (n < kStageSplitMin) {
    memcpy(dst, src, (size_t)n);
  } else {
    const int64_t part = ((n + kStageThreads - 1) / kStageThreads + 4095) & ~(int64_t)4095;
    std::thread workers[kStageThreads - 1];
    for (int i = 1; i < kStageThreads; ++i) {
      const int64_t lo = i * part;
      const int64_t len = lo >= n ? 0 : (n - lo < part ? n - lo : part);
      if (len <= 0) continue;
      try {
        workers[i - 1] = std::thread([=] { memcpy(dst + lo, src + lo, (size_t)len); });
      } catch (...) {
        // no thread to be had (this runs as the runtime's callback, where an
        // exception must not escape): this piece is copied here instead
        memcpy(dst + lo, src + lo, (size_t)len);
      }
    }
    memcpy(dst, src, (size_t)(part < n ? part : n));
    for (auto& w : workers)
      if (w.joinable()) w.join();
  }
  delete c;
}

}  // namespace

// Host -> host copy of nbytes from `src` to `dst` run in `stream`'s order as
// a host function (hipLaunchHostFunc), split over a few threads: the copy of
// a pageable adapter image into a page-locked staging buffer, which a DMA
// queued behind it (on this stream, or on another after an event) then
// reads.  The calling thread never waits; both buffers must stay valid until
// the stream has passed the copy.
extern "C" int pl_host_copy_async(void* dst, const void* src, int64_t nbytes, void* stream) {
  if (nbytes <= 0 || !dst || !src) {
    pl_set_error("pl_host_copy_async: bad arguments");
    return PL_ERR_ARG;
  }
  pl_staged_copy* c = new (std::nothrow) pl_staged_copy{dst, src, nbytes};
  if (!c) {
    pl_set_error("pl_host_copy_async: out of host memory");
    return PL_ERR_LIMIT;
  }
  const hipError_t err =
      hipLaunchHostFunc(reinterpret_cast<hipStream_t>(stream), pl_staged_copy_run, c);
  if (err != hipSuccess) {
    delete c;
    pl_set_error("pl_host_copy_async: %s", hipGetErrorString(err));
    return PL_ERR_LAUNCH;
  }
  return PL_OK;
}
