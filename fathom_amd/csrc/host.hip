// Host-side plumbing of the C ABI: error text, version, pinned mapped host
// memory and async copies.
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "common.hpp"

namespace fathom {

static thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(FATHOM_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

}  // namespace fathom

extern "C" const char *fathom_version(void) { return "fathom-hip 0.1.0 gfx950"; }

extern "C" const char *fathom_last_error(void) { return fathom::g_last_error.c_str(); }

// scripts/B_e2e_offload_v2.py:33-39 (host_mapped: cudaHostAlloc(portable|mapped) +
// cudaHostGetDevicePointer).  Pinned allocation only; hipHostRegister of
// existing memory is never used.
extern "C" int fathom_host_alloc_mapped(size_t bytes, int coherent, void **host_ptr, void **dev_ptr) {
  if (!host_ptr || !dev_ptr) return fathom::fail(FATHOM_ERR_INVALID, "host_alloc_mapped: null output pointer");
  *host_ptr = nullptr;
  *dev_ptr = nullptr;
  if (bytes == 0) return fathom::fail(FATHOM_ERR_INVALID, "host_alloc_mapped: zero bytes");
  unsigned flags = hipHostMallocMapped | hipHostMallocPortable;
  flags |= coherent ? hipHostMallocCoherent : hipHostMallocNonCoherent;
  void *h = nullptr;
  hipError_t e = hipHostMalloc(&h, bytes, flags);
  if (e != hipSuccess || !h) {
    (void)hipGetLastError();
    return fathom::fail(FATHOM_ERR_ALLOC, "hipHostMalloc(%zu bytes) failed: %s", bytes, hipGetErrorString(e));
  }
  void *d = nullptr;
  e = hipHostGetDevicePointer(&d, h, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(h);
    return fathom::hip_fail(e, "hipHostGetDevicePointer");
  }
  *host_ptr = h;
  *dev_ptr = d;
  return FATHOM_OK;
}

extern "C" int fathom_host_free(void *host_ptr) {
  if (!host_ptr) return FATHOM_OK;
  hipError_t e = hipHostFree(host_ptr);
  return e == hipSuccess ? FATHOM_OK : fathom::hip_fail(e, "hipHostFree");
}

extern "C" int fathom_memcpy(void *dst, const void *src, size_t bytes, void *stream) {
  if (bytes == 0) return FATHOM_OK;
  if (!dst || !src) return fathom::fail(FATHOM_ERR_INVALID, "memcpy: null pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, (hipStream_t)stream);
  return e == hipSuccess ? FATHOM_OK : fathom::hip_fail(e, "hipMemcpyAsync");
}
