// velokv_noalloc.hip -- vk_paged_decode_noalloc: paged decode whose split-K
// scratch is a fixed per-device array instead of allocated memory, for callers
// that cannot allocate device memory (code under HIP graph capture, serving
// loops or harnesses that forbid hipMalloc). No counterpart in the reference.
//
// Compiled by hipcc (host + gfx950 device code) and linked into libvelokv.so
// beside the C++ host library; the attention kernels themselves live in the
// code object that the host library loads with hipModuleLoad and take the
// scratch address as an ordinary argument.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "velokv.h"

int vk_internal_set_error(int code, const char* msg);
int vk_internal_ctx_device(const vk_ctx* ctx);

// The split-K partials (acc, (M, l), stream-K unit prefix) of one decode call.
// Each GPU holds its own copy until the process ends. In host code `scratch`
// names a host-side stand-in, not device memory: only the address that
// hipGetSymbolAddress returns for the current device is ever passed on.
static __device__ __align__(256) unsigned char scratch[VK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch_ptr[kMaxDevices];   // device address of `scratch` on each device, once resolved
char g_init_error[kMaxDevices][160];  // why resolving it failed, if it did

int set_error(int code, const char* fmt, const char* a, int b) {
  char buf[256];
  snprintf(buf, sizeof buf, fmt, a, b);
  return vk_internal_set_error(code, buf);
}

}  // namespace

// Called by vk_ctx_create with `device` current: resolves this device's copy of
// the scratch array once per device.
int vk_internal_noalloc_init(int device) {
  if (device < 0 || device >= kMaxDevices)
    return set_error(VK_ERR_UNSUPPORTED, "%sdevice %d is beyond the library's device table", "", device);
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_scratch_ptr[device]) return VK_OK;
  void* ptr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !ptr) {
    snprintf(g_init_error[device], sizeof g_init_error[device], "hipGetSymbolAddress(scratch) failed: %s",
             hipGetErrorString(e));
    return set_error(VK_ERR_HIP, "%s (device %d)", g_init_error[device], device);
  }
  g_scratch_ptr[device] = ptr;
  return VK_OK;
}

extern "C" int vk_paged_decode_noalloc(vk_ctx* ctx, vk_pool* pool, const vk_decode_args* a, void* stream) {
  if (!ctx || !pool || !a) return vk_internal_set_error(VK_ERR_BAD_ARG, "null argument");
  if (a->workspace || a->workspace_bytes)
    return vk_internal_set_error(VK_ERR_BAD_ARG,
                                 "vk_paged_decode_noalloc takes its scratch from the library's per-device array: "
                                 "workspace must be NULL and workspace_bytes 0");
  const int device = vk_internal_ctx_device(ctx);
  void* ptr = nullptr;
  char why[160] = "";
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (device >= 0 && device < kMaxDevices) {
      ptr = g_scratch_ptr[device];
      snprintf(why, sizeof why, "%s", g_init_error[device]);
    }
  }
  if (!ptr) return set_error(VK_ERR_NOT_WIRED, "no scratch resolved (%s) for device %d", why, device);
  uint64_t need = 0;
  int rc = vk_paged_decode_workspace(pool, a, &need);
  if (rc != VK_OK) return rc;
  if (need > VK_NOALLOC_SCRATCH_BYTES) {
    char buf[256];
    snprintf(buf, sizeof buf,
             "this decode needs %llu bytes of split-K scratch; vk_paged_decode_noalloc holds %llu per GPU "
             "(use vk_paged_decode with a workspace)",
             (unsigned long long)need, (unsigned long long)VK_NOALLOC_SCRATCH_BYTES);
    return vk_internal_set_error(VK_ERR_BAD_ARG, buf);
  }
  vk_decode_args b = *a;
  b.workspace = ptr;  // the kernels take the resolved device address, never `scratch` itself
  b.workspace_bytes = VK_NOALLOC_SCRATCH_BYTES;
  return vk_paged_decode(ctx, pool, &b, stream);
}
