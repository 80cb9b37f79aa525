// dsa_noalloc.hip -- dsa_attn_fwd_noalloc: the attention call with its split
// workspace in a library-owned device array instead of caller memory.
//
// For callers that cannot allocate device memory (code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc).  The fp32
// split partials live in `scratch`, a file-scope device array of
// DSA_NOALLOC_SCRATCH_BYTES (32 MiB) that every device the library runs on
// holds until the process ends.  Its address on a device is looked up once,
// with that device current, on the entry point's first call there
// (hipGetSymbolAddress); host code uses only that address, never the array's
// name (on the host the name is a stand-in, not a device address).  The
// lookup may load the library's code object onto the device, so it runs with
// this thread's stream-capture mode set to relaxed: a first call made while
// a graph is being captured does not invalidate the capture.  The call merges
// the splits with the separate merge kernel, so nothing in the array has to
// start at zero: every call writes the partials it later reads.  With an
// automatic split count (num_splits = 0) the call takes the largest count up
// to the automatic one whose workspace fits the array (down to the fewest
// splits the row length allows: one for top-k up to 2048, which needs no
// workspace).  Calls that overlap on one device share the array and race.
#include <atomic>
#include <cstdio>
#include <mutex>

#include "../../include/dsa_abi.h"
#include "dsa_internal.h"

static __device__ __align__(256) unsigned char scratch[DSA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr size_t kScratchBytes = DSA_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

std::mutex g_scratch_mutex;
std::atomic<void *> g_scratch_ptr[kMaxDevices] = {};

// Address of this device's `scratch` (set up on first use, with the device
// current); null with the error string set when the lookup fails.
void *scratch_of_current_device(int *status) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *status = dsa::set_error(DSA_ELAUNCH, "dsa_attn_fwd_noalloc: no current HIP device");
    return nullptr;
  }
  void *cached = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (cached != nullptr) return cached;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  cached = g_scratch_ptr[dev].load(std::memory_order_relaxed);
  if (cached != nullptr) return cached;
  void *ptr = nullptr;
  // relaxed capture mode for this thread while the lookup runs (restored after)
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  const hipError_t em = hipThreadExchangeStreamCaptureMode(&mode);
  e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (em == hipSuccess) (void)hipThreadExchangeStreamCaptureMode(&mode);
  if (e != hipSuccess || ptr == nullptr) {
    char msg[256];
    snprintf(msg, sizeof(msg),
             "dsa_attn_fwd_noalloc: hipGetSymbolAddress of the scratch array failed on device "
             "%d: %s",
             dev, hipGetErrorString(e));
    *status = dsa::set_error(DSA_ELAUNCH, msg);
    return nullptr;
  }
  g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  return ptr;
}

}  // namespace

extern "C" {

int dsa_attn_fwd_noalloc(const dsa_attn_args *a, void *stream) {
  const char *fn = "dsa_attn_fwd_noalloc";
  if (!a) return dsa::set_error(DSA_EINVAL, "dsa_attn_fwd_noalloc: args is NULL");
  if (a->workspace != nullptr || a->split_counters != nullptr)
    return dsa::set_error(DSA_EINVAL, "dsa_attn_fwd_noalloc: workspace and split_counters must "
                                      "be NULL (the call uses the library's scratch array)");
  dsa_attn_args b = *a;
  if (a->num_tokens > 0 && a->num_heads > 0 && a->topk > 0 && a->num_splits >= 0 &&
      a->num_tokens <= (1 << 26) && a->num_heads <= 4096 && a->topk <= (1 << 30)) {
    size_t need =
        dsa::attn_split_workspace(a->num_tokens, a->num_heads, a->topk, a->num_splits);
    if (need > kScratchBytes && a->num_splits == 0) {
      // automatic count: the most splits below it whose workspace fits
      const int32_t auto_s = dsa_attn_num_splits(a->num_tokens, a->num_heads, a->topk, 0);
      for (int32_t s = auto_s - 1; s >= 1; --s) {
        const size_t n = dsa::attn_split_workspace(a->num_tokens, a->num_heads, a->topk, s);
        if (n <= kScratchBytes) {
          b.num_splits = s;
          need = n;
          break;
        }
      }
    }
    if (need > kScratchBytes) {
      char msg[256];
      snprintf(msg, sizeof(msg),
               "dsa_attn_fwd_noalloc: this call's split workspace is %zu bytes, above the "
               "%zu-byte scratch array; use dsa_attn_fwd with a caller workspace or fewer "
               "splits",
               need, kScratchBytes);
      return dsa::set_error(DSA_EWORKSPACE, msg);
    }
    if (need > 0) {
      int status = DSA_OK;
      void *ptr = scratch_of_current_device(&status);
      if (ptr == nullptr) return status;
      b.workspace = ptr;
      b.workspace_bytes = kScratchBytes;
    }
  }
  return dsa::attn_fwd(fn, &b, stream);
}

}  // extern "C"
