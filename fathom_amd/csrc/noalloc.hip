// The fused scan + top-k for callers that cannot allocate device memory (code
// under graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// Its workspace is `scratch`, a static device array of this library of
// FATHOM_NOALLOC_SCRATCH_BYTES: each device holds its own copy from the first
// call on that device until the process ends.  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address): the first call on a device looks its address up with
// hipGetSymbolAddress, with that device current, and keeps it per device.
//
// Every call on a device reuses that device's array, which keeps the state of
// the last call.  Nothing needs clearing first: the kernels re-initialise all
// the state they read (the selection kernel zeroes the candidate counters, the
// candidate pass writes every region count it later reads), as they do for a
// reused caller workspace.  Calls that overlap on one device (two streams, two
// threads) race on the array.
#include <atomic>
#include <mutex>

#include "scan_internal.hpp"
#include "topk_internal.hpp"

namespace fathom {
namespace {

constexpr size_t kScratchBytes = (size_t)FATHOM_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch is a whole number of 256-byte sections");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch[kMaxDevices];  // device address of `scratch` per device (null: not looked up)
std::mutex g_lookup;

// scratch's address on the current device.
int scratch_on_current_device(void **out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "scan_topk_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(FATHOM_ERR_INVALID, "scan_topk_noalloc: device %d outside [0, %d)", dev, kMaxDevices);
  void *p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_lookup);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return hip_fail(e, "scan_topk_noalloc: hipGetSymbolAddress(scratch)");
      if (!p) return fail(FATHOM_ERR_HIP, "scan_topk_noalloc: scratch has no address on device %d", dev);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return FATHOM_OK;
}

}  // namespace
}  // namespace fathom

using namespace fathom;

extern "C" int fathom_scan_topk_noalloc(const float *q, int64_t BH, int64_t G, int64_t D, const int32_t *cls,
                                        const int32_t *clsn, int bmax, int64_t units_max, const void *planes_sb,
                                        const void *scales_sb, int64_t n, int64_t nsb, int64_t sub, int64_t m,
                                        int64_t k, int64_t sink, int64_t local, int64_t *idx, void *stream) {
  // the fused path's own shape limits, checked first so that the size below cannot overflow
  if (BH < 1 || BH > 65535 || G < 1 || G > 8)
    return fail(FATHOM_ERR_INVALID, "scan_topk_noalloc: BH=%lld G=%lld rejected", (long long)BH, (long long)G);
  int rc = check_topk_args(BH * G, n, m, k, sink, local, "scan_topk_noalloc");
  if (rc) return rc;
  // k == sink + local: only the fixed positions are written, with no workspace
  if (k - sink - local == 0)
    return scan_topk_run(q, BH, G, D, cls, clsn, bmax, units_max, planes_sb, scales_sb, n, nsb, sub, m, k, sink,
                         local, idx, nullptr, 0, FATHOM_STAGE_ALL, stream);
  const size_t need = scan_topk_ws(BH * G, n, k, k - sink - local);
  if (need > kScratchBytes)
    return fail(FATHOM_ERR_WORKSPACE,
                "scan_topk_noalloc: BH=%lld G=%lld n=%lld k=%lld needs %zu bytes of scratch, the static array holds "
                "%zu (use fathom_scan_topk with a caller workspace)",
                (long long)BH, (long long)G, (long long)n, (long long)k, need, kScratchBytes);
  void *ws = nullptr;
  rc = scratch_on_current_device(&ws);
  if (rc) return rc;
  return scan_topk_run(q, BH, G, D, cls, clsn, bmax, units_max, planes_sb, scales_sb, n, nsb, sub, m, k, sink, local,
                       idx, ws, kScratchBytes, FATHOM_STAGE_ALL, stream);
}
