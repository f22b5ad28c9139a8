// Tree-verify attention with no caller workspace and no allocation, for callers that cannot allocate device memory
// (code under HIP graph capture that must not call hipMalloc, serving loops and harnesses that forbid it).
//
// It runs the kernels of eagle4_verify_attention unchanged; their split partials (fp32 partial rows, log2-sum-exp
// values and the per-request tile offsets) go to `scratch`, a file-scope device array of kScratchBytes that every GPU
// the library runs on holds from the module's load until the process ends. The streamed schedule numbers its partial
// slots by workgroup, so any batch it takes fits; launches whose workspace would exceed the array (the split-context
// schedule's per-request partials, past 1024 requests) are refused with EAGLE4_SCRATCH_TOO_SMALL before anything is
// launched. Nothing here calls hipMalloc or hipFree.
//
// Sharing: every call on one GPU uses that GPU's single array, which keeps the last call's contents. The kernels
// write every workspace word they read within the same call (no zeroed state is assumed), so back-to-back calls on
// one stream are safe; calls that overlap in time on one GPU (other streams, other threads) race on it.
//
// The array's name is a host-side stand-in that must never reach a kernel: hipGetSymbolAddress gives the address of
// each GPU's copy. eagle4_init looks it up for the current GPU (the binding calls it when it loads the library, so
// before any graph capture); the entry point looks up a device init did not see on its first call there.

#include <mutex>

#include "common.h"

namespace {

constexpr int64_t kScratchBytes = int64_t(64) << 20;  // 64 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_lock;
float* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each GPU, looked up once per device

// The current device's address of `scratch`, looked up on its first use there.
int current_scratch(float** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return EAGLE4_NOT_COVERED;
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (g_scratch_ptr[dev] == nullptr) {
    void* addr = nullptr;
    const hipError_t got = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (got != hipSuccess) return got;
    if (addr == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = static_cast<float*>(addr);
  }
  *out = g_scratch_ptr[dev];
  return EAGLE4_OK;
}

}  // namespace

extern "C" int eagle4_init(void) {
  float* ptr = nullptr;
  return current_scratch(&ptr);
}

extern "C" int64_t eagle4_verify_attention_static_bytes(void) { return kScratchBytes; }

extern "C" int eagle4_verify_attention_static(const eagle4_attn_args* args, void* stream) {
  if (args->num_reqs == 0) return EAGLE4_OK;
  const int64_t need = eagle4_verify_attention_workspace(args);
  if (need < 0) return EAGLE4_NOT_COVERED;
  if (need > kScratchBytes) return EAGLE4_SCRATCH_TOO_SMALL;
  eagle4_attn_args a = *args;
  a.workspace = nullptr;
  a.workspace_bytes = 0;
  if (need > 0) {
    float* ptr = nullptr;
    const int status = current_scratch(&ptr);
    if (status != EAGLE4_OK) return status;
    a.workspace = ptr;
    a.workspace_bytes = kScratchBytes;
  }
  return eagle4_verify_attention(&a, stream);
}
