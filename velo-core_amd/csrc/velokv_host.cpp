// velokv_host.cpp -- C ABI (include/velokv.h) over the gfx950 code object.
//
// Host side of the KV hot path: context (device + code object), pools (HBM
// layout, slot block table), argument validation, kernel launches through
// hipModuleLaunchKernel, and the host block manager. Plain C++17 over the HIP
// runtime API; no kernels are compiled into this library.
#include "velokv.h"

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "velokv_params.h"

using namespace velokv;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

#define HIP_TRY(expr)                                                              \
  do {                                                                             \
    hipError_t _e = (expr);                                                        \
    if (_e != hipSuccess)                                                          \
      return fail(VK_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e));     \
  } while (0)

constexpr int kBS = 16;   // tokens per tile, the kernels' block
constexpr int kMaxPageTiles = 16;  // pages of 16 * k tokens, k <= 16 (up to 256 tokens)
constexpr int kHD = 128;  // head_dim the kernels are built for
constexpr int kMaxPartTokens = 4096;  // 256 blocks: four block-id windows of one wave
constexpr int kMaxTreeNodes = 32;     // one 32-bit mask row per node

uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

int kv_esz(int kv) {
  switch (kv) {
    case VK_KV_F32: return 4;
    case VK_KV_F16: return 2;
    case VK_KV_I8_REF:
    case VK_KV_I8_BLK: return 1;
    default: return 0;
  }
}
int kv_stile(int kv, int bs) {
  if (kv == VK_KV_I8_BLK) return 2;
  if (kv == VK_KV_I8_REF) return 4 * bs;
  return 0;
}

// Page view of a pool's geometry (COW copy, NIXL): one block = one page of
// 16 * page_tiles tokens, its tiles back to back.
PoolGeom page_geom(const PoolGeom& t) {
  PoolGeom g = t;
  g.tile_bytes = t.tile_bytes * (uint32_t)t.page_tiles;
  g.stile_bytes = t.stile_bytes * (uint32_t)t.page_tiles;
  g.n_blocks = t.n_blocks / t.page_tiles;
  g.block_size = t.block_size * t.page_tiles;
  g.page_tiles = 1;
  return g;
}

// Tile width of a pool: heads of up to 64 dims are stored in 64-dim tiles, wider
// ones in 128-dim tiles; the dims past head_dim hold zeros.
int tile_hd(int head_dim) { return head_dim <= kHD / 2 ? kHD / 2 : kHD; }
// The append kernel of a pool (the I8_BLK rule has its own build for 64-dim tiles).
std::string append_kernel_name(int kv_type, int head_dim) {
  return "vk_append_kv" + std::to_string(kv_type) + (kv_type == VK_KV_I8_BLK && tile_hd(head_dim) != kHD ? "_d64" : "");
}

std::string default_code_object_path() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&vk_ctx_create), &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    const size_t slash = p.find_last_of('/');
    return (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/velokv_gfx950.co";
  }
  return "velokv_gfx950.co";
}

}  // namespace

// Error channel shared with the other translation units of the library
// (velokv_radix.cpp, velokv_noalloc.hip): sets the calling thread's
// vk_last_error() message.
int vk_internal_set_error(int code, const char* msg) {
  g_last_error = msg ? msg : "";
  return code;
}

// Resolves the no-alloc scratch of `device` (velokv_noalloc.hip); the device
// must be current.
int vk_internal_noalloc_init(int device);

struct vk_ctx {
  int device = 0;
  std::string arch;
  hipModule_t module = nullptr;
  std::unordered_map<std::string, hipFunction_t> fns;
  // threads per workgroup each kernel was compiled for (__launch_bounds__), read
  // once at vk_ctx_create: a launch with more faults the device, so launch()
  // refuses it
  std::unordered_map<std::string, int> max_threads;
  std::mutex ws_mu;
  void* ws = nullptr;
  uint64_t ws_bytes = 0;
  // Buffers the context's workspace outgrew: a call on another host thread may
  // still have kernels queued that use one, so they are freed only by
  // vk_ctx_destroy (growth is rare: once per new largest shape).
  std::vector<void*> ws_retired;
  uint32_t* err_word = nullptr;  // device: misuse flags (VK_MISUSE_*) or-ed by the kernels
  int decode_kind = VK_DECODE_AUTO;
  int decode_sched = VK_SCHED_AUTO;
  int n_cu = 256;
  std::mutex res_mu;                                   // guards resident
  std::unordered_map<std::string, int64_t> resident;  // kernel -> resident waves

  hipFunction_t fn(const std::string& name) const {
    auto it = fns.find(name);
    return it == fns.end() ? nullptr : it->second;
  }
};

struct vk_pool {
  vk_ctx* ctx = nullptr;
  vk_pool_desc desc{};
  PoolGeom geom{};
  uint8_t* base = nullptr;
  uint64_t bytes = 0;
  int32_t* table = nullptr;  // [max_slots][max_pages_per_slot]
  uint64_t table_bytes = 0;
  // I8_BLK: per block, (epoch << 32 | first token) of the last append run on it,
  // so that a call with two runs on one block is reported (VK_MISUSE_BLK_SPLIT_RUN)
  unsigned long long* claim = nullptr;
  std::atomic<uint32_t> epoch{0};
  uint32_t next_epoch() {
    uint32_t e = ++epoch;
    while (e == 0) e = ++epoch;  // 0 marks a never-claimed block
    return e;
  }
};

namespace {

const char* const kKernelNames[] = {
    "vk_decode_merge", "vk_decode_merge_sk", "vk_append_kv0", "vk_append_kv1", "vk_append_kv2", "vk_append_kv3",
    "vk_append_kv3_d64",
    "vk_slot_mapping", "vk_copy_blocks", "vk_fill_normal_f16", "vk_nixl_check", "vk_nixl_copy",
    "vk_tree_commit_kv0", "vk_tree_commit_kv1", "vk_tree_commit_kv2", "vk_tree_commit_kv3",
};

// GQA group sizes with kernels of their own; any other size up to kMaxGroup
// runs the "_gx" kernels, which take the size at run time.
bool fixed_group(int g) { return g == 1 || g == 2 || g == 4 || g == 8; }
constexpr int kMaxGroupTile = 16;  // one 16-row matrix-core tile
constexpr int kMaxGroup = 32;      // two tiles (split-K decode; tree verify takes any)
std::string gtag(int g) { return fixed_group(g) ? "_g" + std::to_string(g) : std::string("_gx"); }

std::string decode_name(int kv, int g, int qt) {
  return "vk_decode_kv" + std::to_string(kv) + "_g" + std::to_string(g) + "_q" + std::to_string(qt);
}
// Matrix-core decode kernels: fp16 q, or (int8 KV only, suffix _q0) fp32 q split
// into fp16 hi + lo parts.
std::string q0_suffix(int qt) { return qt == VK_DT_F32 ? "_q0" : ""; }
// d64: the head_dim-64 kernels (64-dim pieces, runtime group size up to 16)
std::string decode_mfma_name(int kv, int g, int qt = VK_DT_F16, bool d64 = false) {
  if (d64) return "vk_decode_mfma_kv" + std::to_string(kv) + "_gx_d64" + q0_suffix(qt);
  const std::string t = fixed_group(g) ? gtag(g) : (g > kMaxGroupTile ? "_gx2" : "_gx");
  return "vk_decode_mfma_kv" + std::to_string(kv) + t + q0_suffix(qt);
}
std::string decode_wg_name(int kv, int g, int qt = VK_DT_F16, bool d64 = false) {
  return "vk_decode_wg_kv" + std::to_string(kv) + (d64 ? std::string("_gx_d64") : gtag(g)) + q0_suffix(qt);
}
std::string decode_sk_name(int kv, int g, int qt = VK_DT_F16, bool d64 = false) {
  return "vk_decode_sk_kv" + std::to_string(kv) + (d64 ? std::string("_gx_d64") : gtag(g)) + q0_suffix(qt);
}
// The head_dim-64 decode kernels serve this pool and group size: pools of
// 64-dim tiles (heads of up to 64 dims), one 16-row tile of query rows per
// (sequence, KV head).
bool use_d64(const vk_pool_desc& d, int g) {
  return tile_hd(d.head_dim) == kHD / 2 && g <= kMaxGroupTile;
}
// The folding kernels' variants that also rotate the new K row and q (RoPE)
const char* const kRopeSuffix = "_rope";
std::string decode_pk_name(int kv, int g, int qt = VK_DT_F16) {
  return "vk_decode_pk_kv" + std::to_string(kv) + "_g" + std::to_string(g) + q0_suffix(qt);
}
std::string tree_pfx_name(int kv, int g, int qt, bool d64 = false) {
  return "vk_tree_pfx_kv" + std::to_string(kv) + (d64 ? std::string("_gx_d64") : gtag(g)) + "_q" + std::to_string(qt);
}
// d64: the head_dim-64 tree kernels (64-dim pieces, runtime group size)
std::string tree_name(int kv, int g, int rt, int qt, bool d64 = false) {
  return "vk_tree_kv" + std::to_string(kv) + (d64 ? std::string("_gx_d64") : gtag(g)) + "_r" + std::to_string(rt) +
         "_q" + std::to_string(qt);
}

int set_device(const vk_ctx* ctx) {
  HIP_TRY(hipSetDevice(ctx->device));
  return VK_OK;
}

// A workgroup shape the kernel was compiled for: at least one thread and at most
// its __launch_bounds__ (HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK).
int check_launch_shape(const vk_ctx* ctx, const char* name, uint64_t threads) {
  auto it = ctx->max_threads.find(name);
  if (it == ctx->max_threads.end()) return fail(VK_ERR_NOT_WIRED, "kernel %s is not in the code object", name);
  if (threads == 0 || threads > (uint64_t)it->second)
    return fail(VK_ERR_BAD_ARG, "kernel %s launched with %llu threads per workgroup; it was compiled for at most %d",
                name, (unsigned long long)threads, it->second);
  return VK_OK;
}

template <typename P>
int launch(const vk_ctx* ctx, const char* name, dim3 grid, dim3 block, const P& params, void* stream) {
  hipFunction_t f = ctx->fn(name);
  if (!f) return fail(VK_ERR_NOT_WIRED, "kernel %s is not in the code object", name);
  int rc = check_launch_shape(ctx, name, (uint64_t)block.x * block.y * block.z);
  if (rc) return rc;
  void* args[] = {const_cast<P*>(&params)};
  HIP_TRY(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z, 0,
                                reinterpret_cast<hipStream_t>(stream), args, nullptr));
  return VK_OK;
}

// Waves of a kernel that fit on the device at once, launched with workgroups of
// `block` threads (one wave each by default).
int64_t resident_waves(vk_ctx* ctx, const std::string& name, int block = 64) {
  const std::string key = name + "/" + std::to_string(block);
  std::lock_guard<std::mutex> lk(ctx->res_mu);  // planners may run on several host threads
  auto it = ctx->resident.find(key);
  if (it != ctx->resident.end()) return it->second;
  int64_t waves = 2048;
  hipFunction_t f = ctx->fn(name);
  int per_cu = 0;
  if (f && hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, block, 0) == hipSuccess && per_cu > 0)
    waves = (int64_t)per_cu * (block / 64) * ctx->n_cu;
  ctx->resident[key] = waves;
  return waves;
}


int check_pool(const vk_ctx* ctx, const vk_pool* pool) {
  if (!ctx) return fail(VK_ERR_NOT_WIRED, "context is null");
  if (!pool) return fail(VK_ERR_NOT_WIRED, "pool is null");
  if (pool->ctx != ctx) return fail(VK_ERR_BAD_ARG, "pool belongs to another context");
  return VK_OK;
}

}  // namespace

// ============================================================================
// context
// ============================================================================
extern "C" const char* vk_last_error(void) { return g_last_error.c_str(); }

extern "C" int vk_ctx_create(int device, const char* code_object_path, vk_ctx** out) {
  if (!out) return fail(VK_ERR_BAD_ARG, "out is null");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) return fail(VK_ERR_NO_DEVICE, "no HIP device visible (%s)", hipGetErrorString(e));
  if (device < 0 || device >= n) return fail(VK_ERR_NO_DEVICE, "device %d out of range (0..%d)", device, n - 1);
  HIP_TRY(hipSetDevice(device));
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device));
  std::string arch = prop.gcnArchName;
  const size_t colon = arch.find(':');
  if (colon != std::string::npos) arch = arch.substr(0, colon);
  if (arch != "gfx950")
    return fail(VK_ERR_UNSUPPORTED, "device %d is %s; the code object is built for gfx950", device, arch.c_str());

  const std::string path = code_object_path ? std::string(code_object_path) : default_code_object_path();
  FILE* fp = fopen(path.c_str(), "rb");
  if (!fp) return fail(VK_ERR_NOT_WIRED, "code object %s not found (build the extension first)", path.c_str());
  fclose(fp);

  auto* ctx = new vk_ctx();
  ctx->device = device;
  ctx->arch = arch;
  ctx->n_cu = prop.multiProcessorCount;
  e = hipModuleLoad(&ctx->module, path.c_str());
  if (e != hipSuccess) {
    delete ctx;
    return fail(VK_ERR_NOT_WIRED, "hipModuleLoad(%s) failed: %s", path.c_str(), hipGetErrorString(e));
  }
  std::vector<std::string> names(std::begin(kKernelNames), std::end(kKernelNames));
  for (int kv = 0; kv < 4; ++kv) {  // the runtime-group-size ("_gx") kernels
    for (int qt : {VK_DT_F16, VK_DT_F32}) {
      names.push_back(decode_mfma_name(kv, 3, qt));
      names.push_back(decode_mfma_name(kv, kMaxGroup, qt));
      names.push_back(decode_sk_name(kv, 3, qt));
      if (kv != VK_KV_F16) names.push_back(decode_wg_name(kv, 3, qt));
      if (kv == VK_KV_F16 || kv == VK_KV_I8_BLK) names.push_back(tree_pfx_name(kv, 3, qt));
      for (int rt : {1, 2}) names.push_back(tree_name(kv, 3, rt, qt));
      names.push_back(decode_mfma_name(kv, 3, qt, true));  // head_dim 64
      names.push_back(decode_sk_name(kv, 3, qt, true));
      names.push_back(decode_wg_name(kv, 3, qt, true));
      for (int rt : {1, 2}) names.push_back(tree_name(kv, 3, rt, qt, true));  // tree verify at head_dim 64
      if (kv == VK_KV_F16 || kv == VK_KV_I8_BLK) names.push_back(tree_pfx_name(kv, 3, qt, true));
    }
  }
  // vk_append_rope_decode's kernels: every kernel that folds the append, suffix _rope
  for (int kv : {VK_KV_F16, VK_KV_I8_BLK})
    for (int g : {1, 2, 4, 8, 3})
      for (int qt : {VK_DT_F16, VK_DT_F32})
        for (bool d64 : {false, true}) {
          if (d64 && g != 3) continue;
          names.push_back(decode_sk_name(kv, g, qt, d64) + kRopeSuffix);
          if (kv == VK_KV_I8_BLK) names.push_back(decode_wg_name(kv, g, qt, d64) + kRopeSuffix);
        }
  for (int kv = 0; kv < 4; ++kv)
    for (int g : {1, 2, 4, 8}) {
      for (int qt = 0; qt < 2; ++qt) names.push_back(decode_name(kv, g, qt));
      for (int qt : {VK_DT_F16, VK_DT_F32}) {
        names.push_back(decode_mfma_name(kv, g, qt));
        names.push_back(decode_sk_name(kv, g, qt));
        if (kv != VK_KV_F32) names.push_back(decode_pk_name(kv, g, qt));
        if (kv != VK_KV_F16) names.push_back(decode_wg_name(kv, g, qt));
      }
      for (int rt : {1, 2})
        for (int qt = 0; qt < 2; ++qt) names.push_back(tree_name(kv, g, rt, qt));
      if (kv == VK_KV_F16 || kv == VK_KV_I8_BLK)
        for (int qt = 0; qt < 2; ++qt) names.push_back(tree_pfx_name(kv, g, qt));
    }
  for (const auto& nm : names) {
    hipFunction_t f = nullptr;
    e = hipModuleGetFunction(&f, ctx->module, nm.c_str());
    if (e != hipSuccess) {
      hipModuleUnload(ctx->module);
      delete ctx;
      return fail(VK_ERR_NOT_WIRED, "kernel %s missing from %s: %s", nm.c_str(), path.c_str(), hipGetErrorString(e));
    }
    int max_threads = 0;
    e = hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f);
    if (e != hipSuccess || max_threads <= 0) {
      hipModuleUnload(ctx->module);
      delete ctx;
      return fail(VK_ERR_NOT_WIRED, "workgroup limit of kernel %s unreadable: %s", nm.c_str(), hipGetErrorString(e));
    }
    ctx->fns[nm] = f;
    ctx->max_threads[nm] = max_threads;
  }
  e = hipMalloc(reinterpret_cast<void**>(&ctx->err_word), 256);
  if (e == hipSuccess) e = hipMemset(ctx->err_word, 0, 256);
  if (e != hipSuccess) {
    if (ctx->err_word) hipFree(ctx->err_word);
    hipModuleUnload(ctx->module);
    delete ctx;
    return fail(VK_ERR_HIP, "error word allocation failed: %s", hipGetErrorString(e));
  }
  // the no-alloc entry point's scratch: a failure here fails that entry point
  // (with this message), not the context
  vk_internal_noalloc_init(device);
  g_last_error.clear();
  *out = ctx;
  return VK_OK;
}

// Device index of a context (velokv_noalloc.hip).
int vk_internal_ctx_device(const vk_ctx* ctx) { return ctx ? ctx->device : -1; }

extern "C" int vk_ctx_destroy(vk_ctx* ctx) {
  if (!ctx) return VK_OK;
  hipSetDevice(ctx->device);
  hipDeviceSynchronize();
  if (ctx->ws) hipFree(ctx->ws);
  for (void* p : ctx->ws_retired) hipFree(p);
  if (ctx->err_word) hipFree(ctx->err_word);
  if (ctx->module) hipModuleUnload(ctx->module);
  delete ctx;
  return VK_OK;
}

extern "C" int vk_ctx_set_decode_kernel(vk_ctx* ctx, int kind) {
  if (!ctx) return fail(VK_ERR_NOT_WIRED, "context is null");
  if (kind != VK_DECODE_AUTO && kind != VK_DECODE_VALU && kind != VK_DECODE_MFMA)
    return fail(VK_ERR_BAD_ARG, "unknown decode kernel kind %d", kind);
  ctx->decode_kind = kind;
  return VK_OK;
}

extern "C" int vk_ctx_set_decode_schedule(vk_ctx* ctx, int schedule) {
  if (!ctx) return fail(VK_ERR_NOT_WIRED, "context is null");
  if (schedule != VK_SCHED_AUTO && schedule != VK_SCHED_SPLIT && schedule != VK_SCHED_STREAM &&
      schedule != VK_SCHED_PACKED)
    return fail(VK_ERR_BAD_ARG, "unknown decode schedule %d", schedule);
  ctx->decode_sched = schedule;
  return VK_OK;
}

extern "C" int vk_ctx_arch(const vk_ctx* ctx, char* buf, size_t cap) {
  if (!ctx || !buf || cap == 0) return fail(VK_ERR_BAD_ARG, "bad argument");
  snprintf(buf, cap, "%s", ctx->arch.c_str());
  return VK_OK;
}

extern "C" int vk_kernel_launch_check(const vk_ctx* ctx, const char* kernel, int32_t threads, int32_t* max_threads) {
  if (!ctx || !kernel) return fail(VK_ERR_BAD_ARG, "null argument");
  auto it = ctx->max_threads.find(kernel);
  if (max_threads) *max_threads = it == ctx->max_threads.end() ? 0 : it->second;
  return check_launch_shape(ctx, kernel, threads < 0 ? 0 : (uint64_t)threads);
}

// ============================================================================
// pools
// ============================================================================
extern "C" int vk_pool_create(vk_ctx* ctx, const vk_pool_desc* d, vk_pool** out) {
  if (!ctx) return fail(VK_ERR_NOT_WIRED, "context is null");
  if (!d || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  *out = nullptr;
  if (d->block_size <= 0) return fail(VK_ERR_INVALID_BLOCK_SIZE, "block size must be greater than zero");
  if (d->n_layer <= 0 || d->n_blocks <= 0 || d->n_kv_heads <= 0 || d->head_dim <= 0 || d->max_slots < 0 ||
      d->max_pages_per_slot < 0)
    return fail(VK_ERR_BAD_ARG, "pool sizes must be positive");
  if (kv_esz(d->kv_type) == 0) return fail(VK_ERR_BAD_ARG, "unknown kv_type %d", d->kv_type);
  if (d->head_dim > kHD || d->head_dim % 8 != 0)
    return fail(VK_ERR_UNSUPPORTED, "head_dim %d: the kernels take multiples of 8 up to 128", d->head_dim);
  // pages of 16 * pt tokens: 16-token tiles, pt per page
  const int pt = d->block_size / kBS;
  if (d->block_size % kBS != 0 || pt > kMaxPageTiles)
    return fail(VK_ERR_UNSUPPORTED, "block_size %d: the kernels take pages of 16 * k tokens, k = 1..%d", d->block_size,
                kMaxPageTiles);
  if ((int64_t)d->n_blocks * pt > 0x7FFFFFFF) return fail(VK_ERR_UNSUPPORTED, "pool too large");
  auto* p = new vk_pool();
  p->ctx = ctx;
  p->desc = *d;
  if (p->desc.max_pages_per_slot == 0) p->desc.max_pages_per_slot = d->n_blocks;
  const int esz = kv_esz(d->kv_type);
  PoolGeom& g = p->geom;  // tile view: 16-token tiles, pt per page
  // a tile holds 16 tokens of one head, 64 or 128 dims wide (zeros past head_dim)
  const int tw = tile_hd(d->head_dim);
  g.tile_bytes = (uint32_t)(kBS * tw * esz);
  g.stile_bytes = (uint32_t)kv_stile(d->kv_type, kBS);
  g.n_blocks = d->n_blocks * pt;
  g.page_tiles = pt;
  g.n_kv_heads = d->n_kv_heads;
  g.block_size = kBS;
  g.head_dim = tw;
  g.io_hd = d->head_dim;
  g.kv_type = d->kv_type;
  g.n_layer = d->n_layer;
  const uint64_t codes = (uint64_t)g.n_blocks * d->n_kv_heads * g.tile_bytes;
  const uint64_t scales = (uint64_t)g.n_blocks * d->n_kv_heads * g.stile_bytes;
  g.k_off = 0;
  g.v_off = align_up(codes, 256);
  g.ks_off = g.v_off + align_up(codes, 256);
  if (d->kv_type == VK_KV_I8_BLK) {
    // one array of (K, V) scale words: V is the high half of each word
    g.s_step = kBlkScaleStep;
    g.vs_off = g.ks_off + 2;
    g.layer_stride = g.ks_off + align_up(2 * scales, 256);
  } else {
    g.s_step = scales ? 2 : 0;
    g.vs_off = g.ks_off + align_up(scales, 256);
    g.layer_stride = g.vs_off + align_up(scales, 256);
  }
  p->bytes = g.layer_stride * (uint64_t)d->n_layer;
  int rc = set_device(ctx);
  if (rc) { delete p; return rc; }
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&p->base), p->bytes);
  if (e != hipSuccess) {
    delete p;
    return fail(VK_ERR_HIP, "hipMalloc of %.3f GB for the KV pool failed: %s", p->bytes / 1e9, hipGetErrorString(e));
  }
  e = hipMemset(p->base, 0, p->bytes);
  if (e == hipSuccess && d->max_slots > 0) {
    p->table_bytes = (uint64_t)d->max_slots * p->desc.max_pages_per_slot * sizeof(int32_t);
    e = hipMalloc(reinterpret_cast<void**>(&p->table), p->table_bytes);
    if (e == hipSuccess) e = hipMemset(p->table, 0, p->table_bytes);
  }
  if (e == hipSuccess && d->kv_type == VK_KV_I8_BLK) {
    e = hipMalloc(reinterpret_cast<void**>(&p->claim), (uint64_t)g.n_blocks * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemset(p->claim, 0, (uint64_t)g.n_blocks * sizeof(unsigned long long));
  }
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    hipFree(p->base);
    if (p->table) hipFree(p->table);
    if (p->claim) hipFree(p->claim);
    delete p;
    return fail(VK_ERR_HIP, "pool initialisation failed: %s", hipGetErrorString(e));
  }
  *out = p;
  return VK_OK;
}

extern "C" int vk_pool_destroy(vk_pool* pool) {
  if (!pool) return VK_OK;
  hipSetDevice(pool->ctx->device);
  hipDeviceSynchronize();
  hipFree(pool->base);
  if (pool->table) hipFree(pool->table);
  if (pool->claim) hipFree(pool->claim);
  delete pool;
  return VK_OK;
}

extern "C" int vk_pool_get_desc(const vk_pool* pool, vk_pool_desc* out) {
  if (!pool || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  *out = pool->desc;
  return VK_OK;
}

extern "C" int vk_pool_layer_view(const vk_pool* pool, int32_t layer, vk_layer_view* out) {
  if (!pool || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  if (layer < 0 || layer >= pool->desc.n_layer) return fail(VK_ERR_BAD_ARG, "layer %d out of range", layer);
  const PoolGeom& g = pool->geom;
  uint8_t* L = pool->base + g.layer_stride * (uint64_t)layer;
  out->k_codes = L + g.k_off;
  out->v_codes = L + g.v_off;
  out->codes_bytes = (uint64_t)g.n_blocks * g.n_kv_heads * g.tile_bytes;
  out->scales_bytes = (uint64_t)g.n_blocks * g.n_kv_heads * g.stile_bytes;
  out->k_scales = g.stile_bytes ? L + g.ks_off : nullptr;
  out->v_scales = g.stile_bytes ? L + g.vs_off : nullptr;
  out->scale_step = g.s_step;
  return VK_OK;
}

extern "C" int vk_pool_block_table(const vk_pool* pool, int32_t** table_dev, int32_t* row_stride) {
  if (!pool || !table_dev || !row_stride) return fail(VK_ERR_BAD_ARG, "null argument");
  *table_dev = pool->table;
  *row_stride = pool->desc.max_pages_per_slot;
  return VK_OK;
}

extern "C" int vk_pool_bytes(const vk_pool* pool, uint64_t* out) {
  if (!pool || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  *out = pool->bytes + pool->table_bytes;
  return VK_OK;
}

extern "C" int vk_bind_slot(vk_pool* pool, uint32_t slot, const uint32_t* pages, int32_t n_pages) {
  if (!pool) return fail(VK_ERR_NOT_WIRED, "pool is null");
  if (n_pages < 0 || (n_pages > 0 && !pages)) return fail(VK_ERR_BAD_ARG, "bad page list");
  const int32_t maxp = pool->desc.max_pages_per_slot;
  if (n_pages > maxp)
    return fail(VK_ERR_TOO_MANY_PAGES, "Request pages (%d) exceed max pages per slot (%d)", n_pages, maxp);
  if ((int64_t)slot >= pool->desc.max_slots)
    return fail(VK_ERR_BAD_ARG, "slot %u out of range (max_slots %d)", slot, pool->desc.max_slots);
  std::vector<int32_t> row((size_t)maxp, 0);
  for (int32_t i = 0; i < n_pages; ++i) {
    if (pages[i] >= (uint32_t)pool->desc.n_blocks)
      return fail(VK_ERR_BAD_ARG, "page id %u out of range (n_blocks %d)", pages[i], pool->desc.n_blocks);
    row[(size_t)i] = (int32_t)pages[i];
  }
  int rc = set_device(pool->ctx);
  if (rc) return rc;
  HIP_TRY(hipMemcpy(pool->table + (uint64_t)slot * maxp, row.data(), row.size() * sizeof(int32_t),
                    hipMemcpyHostToDevice));
  return VK_OK;
}

// ============================================================================
// hot path
// ============================================================================
extern "C" int vk_slot_mapping(vk_ctx* ctx, vk_pool* pool, const int32_t* block_tables, int32_t bt_stride,
                               const int32_t* seq_rows, const int32_t* positions, int32_t n_tok,
                               int64_t* slot_mapping_out, void* stream) {
  int rc = check_pool(ctx, pool);
  if (rc) return rc;
  if (n_tok < 0) return fail(VK_ERR_BAD_ARG, "n_tok < 0");
  if (n_tok == 0) return VK_OK;
  if (!positions || !slot_mapping_out) return fail(VK_ERR_BAD_ARG, "null device pointer");
  if (!block_tables) {
    if (!pool->table) return fail(VK_ERR_BAD_ARG, "pool has no slot table (max_slots = 0)");
    block_tables = pool->table;
    bt_stride = pool->desc.max_pages_per_slot;
  }
  if (bt_stride <= 0) return fail(VK_ERR_BAD_ARG, "bt_stride must be positive");
  SlotMapParams p{block_tables, seq_rows, positions, slot_mapping_out, bt_stride, pool->desc.block_size, n_tok,
                  pool->desc.n_blocks};
  if ((rc = set_device(ctx))) return rc;
  return launch(ctx, "vk_slot_mapping", dim3((n_tok + 255) / 256), dim3(256), p, stream);
}

namespace {
// Tokens per append workgroup: enough workgroups to spread the runs over the GPU
// (about 2048 per call), at most 64 (one slot load per lane); a workgroup per
// token for small calls.
int append_tok_per_wg(int32_t n_tok, int32_t n_kv_heads) {
  const int64_t t = ((int64_t)n_tok * n_kv_heads + 2047) / 2048;
  return (int)std::max<int64_t>(1, std::min<int64_t>(64, t));
}
}  // namespace

extern "C" int vk_append(vk_ctx* ctx, vk_pool* pool, int32_t layer, const void* k, const void* v, int32_t in_dtype,
                         const int64_t* slot_mapping, int32_t n_tok, void* stream) {
  int rc = check_pool(ctx, pool);
  if (rc) return rc;
  if (layer < 0 || layer >= pool->desc.n_layer) return fail(VK_ERR_BAD_ARG, "layer %d out of range", layer);
  if (in_dtype != VK_DT_F32 && in_dtype != VK_DT_F16) return fail(VK_ERR_BAD_ARG, "in_dtype %d", in_dtype);
  if (n_tok < 0) return fail(VK_ERR_BAD_ARG, "n_tok < 0");
  if (n_tok == 0) return VK_OK;
  if (!k || !v || !slot_mapping) return fail(VK_ERR_BAD_ARG, "null device pointer");
  AppendParams p{};
  p.base = pool->base;
  p.g = pool->geom;
  p.layer = layer;
  p.in_dtype = in_dtype;
  p.k = k;
  p.v = v;
  p.slot_mapping = slot_mapping;
  p.n_tok = n_tok;
  p.tok_per_wg = append_tok_per_wg(n_tok, pool->desc.n_kv_heads);
  p.err = ctx->err_word;
  p.claim = pool->claim;
  p.epoch = pool->claim ? pool->next_epoch() : 0u;
  const std::string name = append_kernel_name(pool->desc.kv_type, pool->desc.head_dim);
  if ((rc = set_device(ctx))) return rc;
  return launch(ctx, name.c_str(), dim3((unsigned)((n_tok + p.tok_per_wg - 1) / p.tok_per_wg),
                                        (unsigned)pool->desc.n_kv_heads), dim3(128), p, stream);
}

extern "C" int vk_rope_table(float* out, int32_t n_pos, int32_t head_dim, float freq_base) {
  if (!out || n_pos < 0 || head_dim <= 0 || head_dim % 2) return fail(VK_ERR_BAD_ARG, "bad rope table arguments");
  if (!(freq_base > 0.f)) return fail(VK_ERR_BAD_ARG, "freq_base must be positive");
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i) {
    const double inv = std::pow((double)freq_base, -2.0 * (double)i / (double)head_dim);
    for (int32_t p = 0; p < n_pos; ++p) {
      const double a = (double)p * inv;
      out[((int64_t)p * half + i) * 2] = (float)std::cos(a);
      out[((int64_t)p * half + i) * 2 + 1] = (float)std::sin(a);
    }
  }
  return VK_OK;
}

extern "C" int vk_append_rope(vk_ctx* ctx, vk_pool* pool, int32_t layer, void* q, int32_t q_dtype, int32_t n_heads,
                              const void* k, const void* v, int32_t in_dtype, const int32_t* positions,
                              const int64_t* slot_mapping, int32_t n_tok, const float* cos_sin, int32_t n_pos,
                              int32_t rope_style, void* stream) {
  int rc = check_pool(ctx, pool);
  if (rc) return rc;
  if (layer < 0 || layer >= pool->desc.n_layer) return fail(VK_ERR_BAD_ARG, "layer %d out of range", layer);
  if (in_dtype != VK_DT_F32 && in_dtype != VK_DT_F16) return fail(VK_ERR_BAD_ARG, "in_dtype %d", in_dtype);
  if (rope_style != VK_ROPE_INTERLEAVED && rope_style != VK_ROPE_HALF)
    return fail(VK_ERR_BAD_ARG, "rope_style %d (VK_ROPE_INTERLEAVED or VK_ROPE_HALF)", rope_style);
  if (n_tok < 0 || n_pos <= 0) return fail(VK_ERR_BAD_ARG, "n_tok < 0 or n_pos <= 0");
  if (q && (n_heads <= 0 || (q_dtype != VK_DT_F32 && q_dtype != VK_DT_F16)))
    return fail(VK_ERR_BAD_ARG, "q needs n_heads > 0 and q_dtype VK_DT_F32 / VK_DT_F16");
  if (n_tok == 0) return VK_OK;
  if (!k || !v || !slot_mapping || !positions || !cos_sin) return fail(VK_ERR_BAD_ARG, "null device pointer");
  if (reinterpret_cast<uintptr_t>(cos_sin) % 16) return fail(VK_ERR_BAD_ARG, "cos_sin must be 16-byte aligned");
  AppendParams p{};
  p.base = pool->base;
  p.g = pool->geom;
  p.layer = layer;
  p.in_dtype = in_dtype;
  p.k = k;
  p.v = v;
  p.slot_mapping = slot_mapping;
  p.n_tok = n_tok;
  p.rope = rope_style;
  p.positions = positions;
  p.cos_sin = cos_sin;
  p.n_pos = n_pos;
  p.n_heads = q ? n_heads : 0;
  p.q = q;
  p.q_dtype = q_dtype;
  const unsigned rows = (unsigned)pool->desc.n_kv_heads + (q ? (unsigned)((n_heads + 1) / 2) : 0u);
  p.tok_per_wg = append_tok_per_wg(n_tok, (int32_t)rows);
  p.err = ctx->err_word;
  p.claim = pool->claim;
  p.epoch = pool->claim ? pool->next_epoch() : 0u;
  const std::string name = append_kernel_name(pool->desc.kv_type, pool->desc.head_dim);
  if ((rc = set_device(ctx))) return rc;
  return launch(ctx, name.c_str(), dim3((unsigned)((n_tok + p.tok_per_wg - 1) / p.tok_per_wg), rows), dim3(128), p,
                stream);
}

// Size the context's own split-K workspace grows to when it holds `cur` bytes
// and a call needs `need`: at least twice `cur`, so that the buffers it retires
// (kept until vk_ctx_destroy) always sum to less than the live one, however
// slowly the calls' needs grow.
extern "C" uint64_t vk_workspace_grow_bytes(uint64_t cur, uint64_t need) {
  if (need <= cur) return cur;
  const uint64_t twice = cur > UINT64_MAX / 2 ? UINT64_MAX : 2 * cur;
  return align_up(std::max(need, twice), 256);
}

namespace {

// Split-K workspace: the caller's buffer when given (and large enough), else the
// context's own, grown on demand.
int split_workspace(vk_ctx* ctx, void* given, uint64_t given_bytes, uint64_t need, uint8_t** out) {
  if (given) {
    if (given_bytes < need)
      return fail(VK_ERR_BAD_ARG, "workspace of %llu bytes, need %llu", (unsigned long long)given_bytes,
                  (unsigned long long)need);
    *out = reinterpret_cast<uint8_t*>(given);
    return VK_OK;
  }
  std::lock_guard<std::mutex> lk(ctx->ws_mu);
  if (ctx->ws_bytes < need) {
    // never freed here: work queued by another thread may still use the old one
    const uint64_t bytes = vk_workspace_grow_bytes(ctx->ws_bytes, need);
    void* grown = nullptr;
    HIP_TRY(hipMalloc(&grown, bytes));
    if (ctx->ws) ctx->ws_retired.push_back(ctx->ws);
    ctx->ws = grown;
    ctx->ws_bytes = bytes;
  }
  *out = reinterpret_cast<uint8_t*>(ctx->ws);
  return VK_OK;
}

constexpr int kWgMaxWaves = 8;  // waves per workgroup of vk_decode_wg_* / vk_decode_pk_* at most (velokv_kernels.hip)
constexpr int kPkMaxSeqs = 256;  // sequences a vk_decode_pk_* workgroup ranks
constexpr int kPkMaxRounds = 16; // items per vk_decode_pk_* workgroup

// Stream-K cost units charged to each segment ahead of its blocks, for what a
// worker spends starting a second piece (per-wave traces on config 3: ~5 us).
// Measured on configs 2 and 3 with 0, 4, 8, 12, 16, 24: 8 was fastest (config 3
// 110.7 -> 109.2 us per call, config 2 208 -> 206 us).
constexpr int kSkPenalty = 8;
// Blocks' worth of time the append costs the wave that folds it into a
// workgroup-split decode (vk_append_decode over I8_BLK pools): that wave's range
// is this much shorter.
constexpr int kFoldBlocks = 3;

struct DecodePlan {
  const int32_t* bt;
  int32_t bt_stride;
  int32_t bt_rows;
  int32_t part_tokens;
  int32_t max_parts;
  bool stream_k;
  bool packed;       // packed workgroup split: n_workers workgroups of kWgMaxWaves waves
  int32_t n_workers;
  int32_t wg_waves;  // > 0: workgroup-split kernel with this many waves per (sequence, KV head)
  int32_t max_wave_blocks;  // packed: bound on the blocks of one wave's range
  std::string kernel;
  uint64_t acc_bytes, ml_bytes, prefix_bytes;
};

// Schedule and kernel family for these arguments: stream-K when requested, or
// under AUTO unless the batch is known to be uniform or the VALU family was
// requested; fixed partitions run the matrix cores for int8 and fp32 KV and for
// fp32 queries, and the dot2 VALU kernel for fp16 queries over fp16 KV under
// AUTO (measured faster for each; the VALU kernels compute an fp32 q in fp32
// and at GQA 8 spill). Over fp16 / int8 KV an fp32 q is split into fp16 hi + lo
// for the matrix cores; over fp32 KV the matrix cores take q, K, p and V in fp32.
void decode_choice(const vk_ctx* ctx, const vk_pool* pool, const vk_decode_args* a, bool* stream_k, bool* mfma) {
  const vk_pool_desc& d = pool->desc;
  const int kind = ctx ? ctx->decode_kind : VK_DECODE_AUTO;
  const int sched = ctx ? ctx->decode_sched : VK_SCHED_AUTO;
  const bool uniform = a->sum_context_len > 0 &&
                       (double)a->sum_context_len >= 0.97 * (double)a->n_seqs * (double)a->max_context_len;
  const int G = a->n_heads / d.n_kv_heads;
  // the VALU kernels exist for group sizes 1, 2, 4, 8 and head_dim 128 only: the rest always
  // take the matrix cores, and beyond one 16-row tile only fixed partitions
  const bool valu_ok = fixed_group(G) && d.head_dim == kHD;
  *stream_k = a->partition_tokens == 0 && (kind != VK_DECODE_VALU || !valu_ok) && G <= kMaxGroupTile &&
              (sched == VK_SCHED_STREAM || sched == VK_SCHED_PACKED || (sched == VK_SCHED_AUTO && !uniform));
  *mfma = *stream_k || !valu_ok || kind == VK_DECODE_MFMA ||
          (kind == VK_DECODE_AUTO && (d.kv_type != VK_KV_F16 || a->q_dtype == VK_DT_F32));
}

// Smallest partition (256..4096 tokens) whose units fit in one round of resident
// waves; longer contexts get 4096-token partitions.
int auto_partition(const vk_decode_args* a, const vk_pool_desc& d, int64_t resident_waves) {
  const int64_t ctx = std::max(1, a->max_context_len);
  const int64_t pairs = std::max<int64_t>(1, (int64_t)a->n_seqs * d.n_kv_heads);
  for (int P = 256; P < kMaxPartTokens; P *= 2)
    if (pairs * ((ctx + P - 1) / P) <= resident_waves) return P;
  return kMaxPartTokens;
}

int plan_decode(vk_ctx* ctx, const vk_pool* pool, const vk_decode_args* a, DecodePlan* pl) {
  if (!a) return fail(VK_ERR_BAD_ARG, "args is null");
  const vk_pool_desc& d = pool->desc;
  if (a->layer < 0 || a->layer >= d.n_layer) return fail(VK_ERR_BAD_ARG, "layer %d out of range", a->layer);
  if (a->n_seqs < 0 || a->n_heads <= 0 || a->max_context_len < 0) return fail(VK_ERR_BAD_ARG, "bad sizes");
  if (a->n_heads % d.n_kv_heads) return fail(VK_ERR_BAD_ARG, "n_heads %d not a multiple of n_kv_heads %d", a->n_heads, d.n_kv_heads);
  const int G = a->n_heads / d.n_kv_heads;
  if (G > kMaxGroup) return fail(VK_ERR_UNSUPPORTED, "GQA group size %d (decode supports up to %d)", G, kMaxGroup);
  if (a->q_dtype != VK_DT_F32 && a->q_dtype != VK_DT_F16) return fail(VK_ERR_BAD_ARG, "q_dtype %d", a->q_dtype);
  const bool d64 = use_d64(d, G);
  pl->bt = a->block_tables;
  pl->bt_stride = a->bt_stride;
  pl->bt_rows = 0;
  if (!pl->bt) {
    if (!pool->table) return fail(VK_ERR_BAD_ARG, "no block table given and the pool has no slot table");
    pl->bt = pool->table;
    pl->bt_stride = d.max_pages_per_slot;
    pl->bt_rows = d.max_slots;
  }
  if (pl->bt_stride <= 0) return fail(VK_ERR_BAD_ARG, "bt_stride must be positive");
  if ((int64_t)a->max_context_len > (int64_t)pl->bt_stride * d.block_size)
    return fail(VK_ERR_BAD_ARG, "max_context_len %d exceeds the block-table row (%d pages)", a->max_context_len, pl->bt_stride);
  int P = a->partition_tokens;
  if (P < 0 || P % kBS || P > kMaxPartTokens)
    return fail(VK_ERR_BAD_ARG, "partition_tokens must be a multiple of 16 in [16, %d]", kMaxPartTokens);
  bool mfma = false;
  decode_choice(ctx, pool, a, &pl->stream_k, &mfma);
  pl->acc_bytes = pl->ml_bytes = pl->prefix_bytes = 0;
  pl->n_workers = 0;
  pl->wg_waves = 0;
  pl->packed = false;
  pl->max_wave_blocks = 0;
  const int sched = ctx ? ctx->decode_sched : VK_SCHED_AUTO;
  if (pl->stream_k && sched == VK_SCHED_PACKED && fixed_group(G) && d.kv_type != VK_KV_F32 && a->n_seqs > 0 &&
      a->n_seqs <= kPkMaxSeqs) {
    // Packed workgroup split: one workgroup per resident slot (n_workers bins), the
    // batch's (sequence, KV head) items dealt to them longest first in snake
    // order, so that they fill the GPU, each workgroup gets at most kPkMaxRounds
    // items and no wave's range can pass 256 blocks (four block-id windows).
    const std::string name = decode_pk_name(d.kv_type, G, a->q_dtype);
    const int64_t wgs = std::max<int64_t>(1, (ctx ? resident_waves(ctx, name, 64 * kWgMaxWaves) : 2048) / kWgMaxWaves);
    const int64_t items = (int64_t)a->n_seqs * d.n_kv_heads;
    const int64_t bins = std::min(wgs, items);
    const int64_t rounds = (items + bins - 1) / bins;
    const int64_t nb = ((int64_t)a->max_context_len + kBS - 1) / kBS;
    const int64_t wave_units = (rounds * (nb + kSkPenalty) + kWgMaxWaves - 1) / kWgMaxWaves;
    if (rounds <= kPkMaxRounds && wave_units <= kMaxPartTokens / kBS) {
      pl->stream_k = false;
      pl->packed = true;
      pl->kernel = name;
      pl->n_workers = (int32_t)bins;
      pl->part_tokens = kMaxPartTokens;
      pl->max_parts = 1;
      pl->max_wave_blocks = (int32_t)std::min<int64_t>(nb, wave_units);
      return VK_OK;
    }
  }
  if (pl->stream_k) {
    pl->kernel = decode_sk_name(d.kv_type, G, a->q_dtype, d64);
    // one wave per resident slot, and at most 256 blocks (four id windows) per
    // worker: a worker's blocks are at most its units, ceil(units / nw)
    const int64_t units_max = (int64_t)a->n_seqs * d.n_kv_heads *
                              ((a->max_context_len + kBS - 1) / kBS + kSkPenalty);
    const int64_t waves = ctx ? resident_waves(ctx, pl->kernel, 64 * kSkWaves) : 2048;
    const int64_t nw = std::max<int64_t>(1, std::max(waves, (units_max + 255) / 256));
    if (units_max > 0x7FFFFFFF) return fail(VK_ERR_UNSUPPORTED, "batch too large for the stream-K schedule");
    if (nw > 0x7FFFFFFF) return fail(VK_ERR_UNSUPPORTED, "grid too large");
    pl->n_workers = (int32_t)nw;
    pl->part_tokens = kMaxPartTokens;  // unused by the stream-K kernels
    pl->max_parts = 1;
    const uint64_t prow = (uint64_t)nw * 2 * G;
    pl->acc_bytes = align_up(prow * kHD * sizeof(float), 256);
    pl->ml_bytes = align_up(prow * 2 * sizeof(float), 256);
    pl->prefix_bytes = align_up(((uint64_t)a->n_seqs + 1) * sizeof(int32_t), 256);
    return VK_OK;
  }
  pl->wg_waves = 0;
  // (fp16 pools at 128 dims: the dot2 split-K, or the matrix-core split-K with an
  // fp32 q, measured faster than a workgroup split; at 64 dims the split wins)
  if (mfma && P == 0 && G <= kMaxGroupTile && (d.kv_type != VK_KV_F16 || d64)) {
    // Workgroup split: NW waves per (sequence, KV head), the smallest power of two
    // whose workgroups fill one round of resident waves, when each wave's share
    // fits its four block-id windows (256 blocks).
    const int64_t pairs = (int64_t)a->n_seqs * d.n_kv_heads;
    const int64_t waves = ctx ? resident_waves(ctx, decode_wg_name(d.kv_type, G, a->q_dtype, d64), 64 * kWgMaxWaves) : 2048;
    int nw = 1;
    while (nw < 8 && pairs * nw < waves) nw *= 2;
    const int64_t nb = ((int64_t)a->max_context_len + kBS - 1) / kBS;
    if (pairs > 0 && pairs * nw >= waves && (nb + nw - 1) / nw <= kMaxPartTokens / kBS &&
        pairs <= 0x7FFFFFFF) {
      pl->wg_waves = nw;
      pl->kernel = decode_wg_name(d.kv_type, G, a->q_dtype, d64);
      pl->part_tokens = kMaxPartTokens;
      pl->max_parts = 1;
      return VK_OK;
    }
  }
  pl->kernel = mfma ? decode_mfma_name(d.kv_type, G, a->q_dtype, d64) : decode_name(d.kv_type, G, a->q_dtype);
  if (P == 0) P = auto_partition(a, d, ctx ? resident_waves(ctx, pl->kernel) : 2048);
  pl->part_tokens = P;
  pl->max_parts = std::max(1, (a->max_context_len + P - 1) / P);
  pl->acc_bytes = align_up((uint64_t)a->n_seqs * a->n_heads * pl->max_parts * kHD * sizeof(float), 256);
  pl->ml_bytes = align_up((uint64_t)a->n_seqs * a->n_heads * pl->max_parts * 2 * sizeof(float), 256);
  return VK_OK;
}

}  // namespace

extern "C" int vk_paged_decode_workspace(const vk_pool* pool, const vk_decode_args* a, uint64_t* bytes) {
  if (!pool || !bytes || !a) return fail(VK_ERR_BAD_ARG, "null argument");
  DecodePlan pl;
  int rc = plan_decode(pool->ctx, pool, a, &pl);
  if (rc) return rc;
  *bytes = pl.acc_bytes + pl.ml_bytes + pl.prefix_bytes;
  return VK_OK;
}

extern "C" int vk_paged_decode_kernel(const vk_pool* pool, const vk_decode_args* a, char* buf, size_t cap) {
  if (!pool || !a || !buf || cap == 0) return fail(VK_ERR_BAD_ARG, "null argument");
  DecodePlan pl;
  int rc = plan_decode(pool->ctx, pool, a, &pl);
  if (rc) return rc;
  snprintf(buf, cap, "%s", pl.kernel.c_str());
  return VK_OK;
}

extern "C" int vk_paged_decode_plan(const vk_pool* pool, const vk_decode_args* a, vk_decode_plan* out) {
  if (!pool || !a || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  DecodePlan pl;
  int rc = plan_decode(pool->ctx, pool, a, &pl);
  if (rc) return rc;
  const vk_pool_desc& d = pool->desc;
  memset(out, 0, sizeof *out);
  snprintf(out->kernel, sizeof out->kernel, "%s", pl.kernel.c_str());
  const int64_t nb = ((int64_t)a->max_context_len + kBS - 1) / kBS;
  out->workspace_bytes = pl.acc_bytes + pl.ml_bytes + pl.prefix_bytes;
  if (pl.packed) {
    out->schedule = VK_SCHED_PACKED;
    out->wg_waves = kWgMaxWaves;
    out->n_workers = pl.n_workers;
    out->max_blocks_per_wave = pl.max_wave_blocks;
  } else if (pl.stream_k) {
    const int64_t units_max = (int64_t)a->n_seqs * d.n_kv_heads * (nb + kSkPenalty);
    out->schedule = VK_SCHED_STREAM;
    out->wg_waves = kSkWaves;
    out->n_workers = pl.n_workers;
    out->max_blocks_per_wave = (int32_t)std::min<int64_t>(nb, (units_max + pl.n_workers - 1) / pl.n_workers);
    out->merge_launch = 1;
  } else if (pl.wg_waves) {
    out->schedule = VK_SCHED_WORKGROUP;
    out->wg_waves = pl.wg_waves;
    out->max_blocks_per_wave = (int32_t)((nb + pl.wg_waves - 1) / pl.wg_waves);
  } else {
    out->schedule = VK_SCHED_SPLIT;
    out->partition_tokens = pl.part_tokens;
    out->max_partitions = pl.max_parts;
    out->max_blocks_per_wave = (int32_t)std::min<int64_t>(nb, pl.part_tokens / kBS);
    out->merge_launch = pl.max_parts > 1 ? 1 : 0;
  }
  return VK_OK;
}

namespace {

// The new token of every sequence (k_new / v_new rows [S][Hkv][D] of in_dtype)
// appended at position context_len - 1 of its table row by the append kernel,
// slots derived in the kernel (the unfused half of vk_append_decode).
// Whether the decode launch of this plan appends the new tokens itself
// (vk_append_decode): I8_BLK pools under the workgroup split or stream-K, fp16
// pools under stream-K, over tiles the folded kernels are built for.
bool plan_folds_append(const vk_pool* pool, const vk_decode_args* a, const DecodePlan& pl) {
  const int kvt = pool->desc.kv_type;
  return ((kvt == VK_KV_I8_BLK && (pl.wg_waves > 0 || pl.stream_k)) || (kvt == VK_KV_F16 && pl.stream_k)) &&
         (tile_hd(pool->desc.head_dim) == kHD || use_d64(pool->desc, a->n_heads / pool->desc.n_kv_heads));
}

// vk_append_rope_decode rotates the new K row and q inside the folding decode
// kernel (its _rope variant) when the plan folds the append and q's half-split
// partner chunk sits in lane ^ 32 (head_dim equal to the tile width); otherwise
// the RoPE append writes the rotated q rows into the workspace and the decode
// reads them there.
bool plan_folds_rope(const vk_pool* pool, const vk_decode_args* a, const DecodePlan& pl) {
  return plan_folds_append(pool, a, pl) && pool->geom.io_hd == pool->geom.head_dim;
}

// RoPE of vk_append_rope_decode (style ROPE_NONE: none).
struct RopeArgs {
  int32_t style = ROPE_NONE;
  const float* cos_sin = nullptr;
  int32_t n_pos = 0;
};

int append_new_tokens(vk_ctx* ctx, vk_pool* pool, const vk_decode_args* a, const DecodePlan& pl, const void* k_new,
                      const void* v_new, int in_dtype, void* stream, const RopeArgs& rope = RopeArgs(),
                      void* q_out = nullptr) {
  AppendParams p{};
  p.base = pool->base;
  p.g = pool->geom;
  p.layer = a->layer;
  p.in_dtype = in_dtype;
  p.k = k_new;
  p.v = v_new;
  p.slot_mapping = nullptr;
  p.block_tables = pl.bt;
  p.seq_rows = a->seq_rows;
  p.context_lens = a->context_lens;
  p.bt_stride = pl.bt_stride;
  p.bt_rows = pl.bt_rows;
  p.cap_tokens = a->max_context_len;
  p.n_tok = a->n_seqs;
  p.tok_per_wg = append_tok_per_wg(a->n_seqs, pool->desc.n_kv_heads);
  p.err = ctx->err_word;
  p.claim = pool->claim;
  p.epoch = pool->claim ? pool->next_epoch() : 0u;
  unsigned rows = (unsigned)pool->desc.n_kv_heads;
  if (rope.style != ROPE_NONE) {  // positions derived (context_len - 1); q rotated into q_out
    p.rope = rope.style;
    p.positions = nullptr;
    p.cos_sin = rope.cos_sin;
    p.n_pos = rope.n_pos;
    p.n_heads = a->n_heads;
    p.q = const_cast<void*>(a->q);
    p.q_out = q_out;
    p.q_dtype = a->q_dtype;
    rows += (unsigned)((a->n_heads + 1) / 2);
  }
  const std::string name = append_kernel_name(pool->desc.kv_type, pool->desc.head_dim);
  return launch(ctx, name.c_str(), dim3((unsigned)((a->n_seqs + p.tok_per_wg - 1) / p.tok_per_wg), rows), dim3(128),
                p, stream);
}

// vk_paged_decode, and with k_new the append of vk_append_decode as a launch
// before it.
int run_decode(vk_ctx* ctx, vk_pool* pool, const vk_decode_args* a, void* stream, const void* k_new,
               const void* v_new, int in_dtype, const RopeArgs& rope = RopeArgs()) {
  int rc = check_pool(ctx, pool);
  if (rc) return rc;
  DecodePlan pl;
  if ((rc = plan_decode(ctx, pool, a, &pl))) return rc;
  if (a->n_seqs == 0) return VK_OK;
  if (!a->q || !a->out || !a->context_lens) return fail(VK_ERR_BAD_ARG, "null device pointer");
  if ((rc = set_device(ctx))) return rc;
  // I8_BLK pools under the workgroup split or stream-K, and fp16 pools under
  // stream-K, take the append inside the decode launch (the wave that holds a
  // sequence's last block appends the token before loading it); every other
  // plan appends in a launch of its own first
  const int kvt = pool->desc.kv_type;
  const bool fold = k_new && plan_folds_append(pool, a, pl);
  const bool rope_fold = fold && rope.style != ROPE_NONE && plan_folds_rope(pool, a, pl);
  const std::string kernel = rope_fold ? pl.kernel + kRopeSuffix : pl.kernel;
  const bool rope_copy = rope.style != ROPE_NONE && !rope_fold;
  const uint64_t q_bytes = rope_copy ? align_up((uint64_t)a->n_seqs * a->n_heads * pool->geom.io_hd *
                                                (a->q_dtype == VK_DT_F32 ? 4 : 2), 256) : 0;
  uint8_t* ws = nullptr;
  if ((rc = split_workspace(ctx, a->workspace, a->workspace_bytes,
                            pl.acc_bytes + pl.ml_bytes + pl.prefix_bytes + q_bytes, &ws)))
    return rc;
  void* q_rot = rope_copy ? ws + pl.acc_bytes + pl.ml_bytes + pl.prefix_bytes : nullptr;
  if (k_new && (!fold || rope_copy) &&
      (rc = append_new_tokens(ctx, pool, a, pl, k_new, v_new, in_dtype, stream, rope, q_rot)))
    return rc;
  const vk_pool_desc& d = pool->desc;
  const PoolGeom& g = pool->geom;
  const uint8_t* L = pool->base + g.layer_stride * (uint64_t)a->layer;
  const float scale = a->scale != 0.f ? a->scale : 1.0f / std::sqrt((float)d.head_dim);

  DecodeParams p{};
  p.io_hd = pool->geom.io_hd;
  p.tile_hd = pool->geom.head_dim;
  p.kc = L + g.k_off;
  p.vc = L + g.v_off;
  p.ks = g.stile_bytes ? L + g.ks_off : nullptr;
  p.vs = g.stile_bytes ? L + g.vs_off : nullptr;
  p.q = rope_copy ? q_rot : a->q;
  p.out = a->out;
  p.part_acc = reinterpret_cast<float*>(ws);
  p.part_ml = reinterpret_cast<float*>(ws + pl.acc_bytes);
  p.sk_prefix = pl.stream_k ? reinterpret_cast<int32_t*>(ws + pl.acc_bytes + pl.ml_bytes) : nullptr;
  p.block_tables = pl.bt;
  p.seq_rows = a->seq_rows;
  p.context_lens = a->context_lens;
  p.tile_bytes = g.tile_bytes;
  p.stile_bytes = g.stile_bytes;
  p.bt_stride = pl.bt_stride;
  p.bt_rows = pl.bt_rows;
  p.n_seqs = a->n_seqs;
  p.n_heads = a->n_heads;
  p.n_kv_heads = d.n_kv_heads;
  p.n_blocks = d.n_blocks;
  p.page_tiles = g.page_tiles;
  p.max_parts = pl.max_parts;
  p.part_tokens = pl.part_tokens;
  // stream-K: contexts are clamped to max_context_len, which bounds every worker's
  // range to 256 blocks (the planner sized the grid for it)
  p.cap_tokens = (pl.stream_k || pl.packed) ? a->max_context_len
                : pl.wg_waves ? a->max_context_len  // bounds every wave's share to 256 blocks (planner)
                              : (int32_t)std::min<int64_t>((int64_t)pl.max_parts * pl.part_tokens,
                                                           (int64_t)pl.bt_stride * d.block_size);
  p.n_nodes = 1;
  p.n_rgroups = 1;
  p.n_workers = pl.n_workers;
  p.sk_penalty = (pl.stream_k || pl.packed) ? kSkPenalty : 0;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.err = ctx->err_word;
  if (fold && !rope_copy) {
    if (rope_fold) {
      p.rope = rope.style;
      p.cos_sin = rope.cos_sin;
      p.rope_n_pos = rope.n_pos;
    }
    p.fold_k = k_new;
    p.fold_v = v_new;
    p.fold_dtype = in_dtype;
    p.claim = pool->claim;
    p.fold_epoch = pool->claim ? pool->next_epoch() : 0u;
    // workgroup split: the folding wave's range is shortened by kFoldBlocks
    // while every wave's share stays within its four block-id windows (stream-K
    // ranges are not shortened)
    const int64_t nb = ((int64_t)a->max_context_len + kBS - 1) / kBS;
    p.fold_blocks = pl.wg_waves > 0 && (nb + kFoldBlocks + pl.wg_waves - 1) / pl.wg_waves <= kMaxPartTokens / kBS
                        ? kFoldBlocks : 0;
  }

  MergeParams m{};
  m.io_hd = pool->geom.io_hd;
  m.part_acc = p.part_acc;
  m.part_ml = p.part_ml;
  m.context_lens = a->context_lens;
  m.out = a->out;
  m.n_rows = a->n_seqs * a->n_heads;
  m.rows_per_seq = a->n_heads;
  m.extra_tokens = 0;
  m.max_parts = pl.max_parts;
  m.part_tokens = pl.part_tokens;
  m.cap_tokens = p.cap_tokens;
  m.sk_prefix = p.sk_prefix;
  m.n_workers = pl.n_workers;
  m.sk_penalty = p.sk_penalty;
  m.n_kv_heads = d.n_kv_heads;
  m.n_seqs = a->n_seqs;
  const dim3 merge_grid((unsigned)((m.n_rows + 3) / 4));
  if (pl.stream_k) {
    // kSkWaves workers per workgroup; the waves past n_workers return at once
    if ((rc = launch(ctx, kernel.c_str(), dim3((unsigned)((pl.n_workers + kSkWaves - 1) / kSkWaves)),
                     dim3(64 * kSkWaves), p, stream)))
      return rc;
    return launch(ctx, "vk_decode_merge_sk", merge_grid, dim3(256), m, stream);
  }
  if (pl.packed)
    return launch(ctx, kernel.c_str(), dim3((unsigned)pl.n_workers), dim3(64 * kWgMaxWaves), p, stream);
  if (pl.wg_waves)
    return launch(ctx, kernel.c_str(), dim3((unsigned)(a->n_seqs * d.n_kv_heads)), dim3(64 * (unsigned)pl.wg_waves),
                  p, stream);
  const uint64_t units = (uint64_t)a->n_seqs * pl.max_parts * d.n_kv_heads;
  if (units > 0x7FFFFFFFull) return fail(VK_ERR_UNSUPPORTED, "grid too large");
  if ((rc = launch(ctx, kernel.c_str(), dim3((unsigned)units), dim3(64), p, stream))) return rc;
  if (pl.max_parts == 1) return VK_OK;  // every sequence was finished by the decode kernel
  return launch(ctx, "vk_decode_merge", merge_grid, dim3(256), m, stream);
}

}  // namespace

extern "C" int vk_paged_decode(vk_ctx* ctx, vk_pool* pool, const vk_decode_args* a, void* stream) {
  return run_decode(ctx, pool, a, stream, nullptr, nullptr, VK_DT_F16);
}

extern "C" int vk_append_rope_decode(vk_ctx* ctx, vk_pool* pool, const void* k_new, const void* v_new,
                                     int32_t in_dtype, const float* cos_sin, int32_t n_pos, int32_t rope_style,
                                     const vk_decode_args* a, void* stream) {
  if (in_dtype != VK_DT_F32 && in_dtype != VK_DT_F16) return fail(VK_ERR_BAD_ARG, "in_dtype %d", in_dtype);
  if (rope_style != VK_ROPE_INTERLEAVED && rope_style != VK_ROPE_HALF)
    return fail(VK_ERR_BAD_ARG, "rope_style %d (VK_ROPE_INTERLEAVED or VK_ROPE_HALF)", rope_style);
  if (!a) return fail(VK_ERR_BAD_ARG, "args is null");
  if (n_pos <= 0) return fail(VK_ERR_BAD_ARG, "n_pos must be positive");
  if (a->n_seqs > 0 && (!k_new || !v_new || !cos_sin)) return fail(VK_ERR_BAD_ARG, "null device pointer");
  if (reinterpret_cast<uintptr_t>(cos_sin) % 16) return fail(VK_ERR_BAD_ARG, "cos_sin must be 16-byte aligned");
  RopeArgs r;
  r.style = rope_style;
  r.cos_sin = cos_sin;
  r.n_pos = n_pos;
  return run_decode(ctx, pool, a, stream, k_new, v_new, in_dtype, r);
}

extern "C" int vk_append_rope_decode_workspace(const vk_pool* pool, const vk_decode_args* a, uint64_t* bytes) {
  if (!pool || !a || !bytes) return fail(VK_ERR_BAD_ARG, "null argument");
  DecodePlan pl;
  int rc = plan_decode(pool->ctx, pool, a, &pl);
  if (rc) return rc;
  *bytes = pl.acc_bytes + pl.ml_bytes + pl.prefix_bytes;
  if (!plan_folds_rope(pool, a, pl))
    *bytes += align_up((uint64_t)a->n_seqs * a->n_heads * pool->geom.io_hd * (a->q_dtype == VK_DT_F32 ? 4 : 2), 256);
  return VK_OK;
}

extern "C" int vk_append_decode(vk_ctx* ctx, vk_pool* pool, const void* k_new, const void* v_new, int32_t in_dtype,
                                const vk_decode_args* a, void* stream) {
  if (in_dtype != VK_DT_F32 && in_dtype != VK_DT_F16) return fail(VK_ERR_BAD_ARG, "in_dtype %d", in_dtype);
  if (!a) return fail(VK_ERR_BAD_ARG, "args is null");
  if (a->n_seqs > 0 && (!k_new || !v_new)) return fail(VK_ERR_BAD_ARG, "null device pointer");
  return run_decode(ctx, pool, a, stream, k_new, v_new, in_dtype);
}

namespace {

constexpr int kPfxRowsPerGroup = kPfxRows;  // query rows per workgroup of the shared-prefix pass
constexpr int kPfxThreads = 64 * kPfxWaves;

struct TreePlan {
  const int32_t* bt;
  int32_t bt_stride, bt_rows, part_tokens, max_parts, rt, n_rgroups;
  // shared-prefix pass: prefix pages, chunks (partial slots 0..prefix_chunks-1),
  // row tiles of kPfxRows query rows per KV head; 0 chunks = no prefix pass
  int32_t prefix_blocks, prefix_chunks, pfx_row_tiles;
  uint64_t acc_bytes, ml_bytes;
  std::string kernel, pfx_kernel;
};

int plan_tree(vk_ctx* ctx, const vk_pool* pool, const vk_tree_args* a, TreePlan* pl) {
  if (!a) return fail(VK_ERR_BAD_ARG, "args is null");
  const vk_pool_desc& d = pool->desc;
  if (a->layer < 0 || a->layer >= d.n_layer) return fail(VK_ERR_BAD_ARG, "layer %d out of range", a->layer);
  if (a->n_seqs < 0 || a->n_heads <= 0 || a->max_context_len < 0) return fail(VK_ERR_BAD_ARG, "bad sizes");
  if (a->n_nodes < 1 || a->n_nodes > kMaxTreeNodes)
    return fail(VK_ERR_BAD_ARG, "n_nodes %d out of range [1, %d]", a->n_nodes, kMaxTreeNodes);
  if (a->n_heads % d.n_kv_heads) return fail(VK_ERR_BAD_ARG, "n_heads %d not a multiple of n_kv_heads %d", a->n_heads, d.n_kv_heads);
  const int G = a->n_heads / d.n_kv_heads;  // any group size: rows of (node, head) in 16-row tiles
  if (a->q_dtype != VK_DT_F32 && a->q_dtype != VK_DT_F16) return fail(VK_ERR_BAD_ARG, "q_dtype %d", a->q_dtype);
  pl->bt = a->block_tables;
  pl->bt_stride = a->bt_stride;
  pl->bt_rows = 0;
  if (!pl->bt) {
    if (!pool->table) return fail(VK_ERR_BAD_ARG, "no block table given and the pool has no slot table");
    pl->bt = pool->table;
    pl->bt_stride = d.max_pages_per_slot;
    pl->bt_rows = d.max_slots;
  }
  if (pl->bt_stride <= 0) return fail(VK_ERR_BAD_ARG, "bt_stride must be positive");
  if ((int64_t)a->max_context_len + a->n_nodes > (int64_t)pl->bt_stride * d.block_size)
    return fail(VK_ERR_BAD_ARG, "max_context_len %d + n_nodes %d exceeds the block-table row (%d pages)",
                a->max_context_len, a->n_nodes, pl->bt_stride);
  const int rows = a->n_nodes * G;
  pl->rt = rows > 16 ? 2 : 1;
  pl->n_rgroups = (rows + 16 * pl->rt - 1) / (16 * pl->rt);
  // pools of 64-dim tiles take the 64-dim tree kernels
  pl->kernel = tree_name(d.kv_type, G, pl->rt, a->q_dtype, tile_hd(d.head_dim) == kHD / 2);
  if (a->shared_blocks < 0 || a->shared_blocks > pl->bt_stride ||
      (int64_t)a->shared_blocks * d.block_size > a->max_context_len)
    return fail(VK_ERR_BAD_ARG, "shared_blocks %d: must be within the table row (%d pages) and max_context_len %d",
                a->shared_blocks, pl->bt_stride, a->max_context_len);
  pl->prefix_blocks = pl->prefix_chunks = pl->pfx_row_tiles = 0;
  int64_t tokens = (int64_t)a->max_context_len + a->n_nodes;
  if (a->shared_blocks > 0 && (d.kv_type == VK_KV_F16 || d.kv_type == VK_KV_I8_BLK)) {
    // One workgroup per (256 query rows, KV head, prefix chunk); the prefix is cut
    // into chunks of at least 16 pages until the workgroups cover the CUs, and of
    // at most kPfxMaxChunkBlocks pages.
    const int64_t qrows = (int64_t)a->n_seqs * rows;
    pl->pfx_row_tiles = (int32_t)((qrows + kPfxRowsPerGroup - 1) / kPfxRowsPerGroup);
    const int64_t groups = std::max<int64_t>(1, (int64_t)pl->pfx_row_tiles * d.n_kv_heads);
    const int64_t n_cu = ctx ? ctx->n_cu : 256;
    const int32_t tiles = a->shared_blocks * pool->geom.page_tiles;  // the prefix in 16-token tiles
    const int64_t max_chunks = std::max(1, tiles / 16);
    const int64_t min_chunks = (tiles + kPfxMaxChunkBlocks - 1) / kPfxMaxChunkBlocks;
    pl->prefix_chunks = (int32_t)std::max(
        min_chunks, std::min(max_chunks, std::max<int64_t>(1, (n_cu + groups - 1) / groups)));
    pl->prefix_blocks = tiles;
    pl->pfx_kernel = tree_pfx_name(d.kv_type, G, a->q_dtype, tile_hd(d.head_dim) == kHD / 2);
    // the rest of a context: past the prefix, or the last partial page of a
    // context shorter than the prefix, then the tree nodes
    tokens = std::max<int64_t>((int64_t)a->max_context_len - (int64_t)a->shared_blocks * d.block_size,
                               kBS - 1) + a->n_nodes;
  }
  int P = a->partition_tokens;
  if (P < 0 || P % kBS || P > kMaxPartTokens)
    return fail(VK_ERR_BAD_ARG, "partition_tokens must be a multiple of 16 in [16, %d]", kMaxPartTokens);
  if (P == 0 && pl->prefix_chunks > 0 && tokens <= kMaxPartTokens) {
    // after a shared prefix, the rest of each context in one partition: the
    // tree kernel then folds the prefix partials into the output itself and no
    // merge launch follows
    P = (int)((tokens + kBS - 1) / kBS * kBS);
  } else if (P == 0) {
    // Smallest partition with at most four units per resident wave: the tree
    // kernels are bound by issue, not by HBM, and short partitions even out
    // contexts of different lengths (a 4096-token prefix plus a short suffix
    // would otherwise leave one long and one short unit per sequence).
    const int64_t waves = ctx ? resident_waves(ctx, pl->kernel) : 2048;
    const int64_t pairs = std::max<int64_t>(1, (int64_t)a->n_seqs * d.n_kv_heads * pl->n_rgroups);
    P = kMaxPartTokens;
    for (int c = 256; c < kMaxPartTokens; c *= 2)
      if (pairs * ((tokens + c - 1) / c) <= 4 * waves) { P = c; break; }
  }
  pl->part_tokens = P;
  pl->max_parts = pl->prefix_chunks + (int32_t)std::max<int64_t>(1, (tokens + P - 1) / P);
  const uint64_t rows_total = (uint64_t)a->n_seqs * a->n_nodes * a->n_heads * pl->max_parts;
  pl->acc_bytes = align_up(rows_total * kHD * sizeof(float), 256);
  pl->ml_bytes = align_up(rows_total * 2 * sizeof(float), 256);
  return VK_OK;
}

}  // namespace

extern "C" int vk_tree_verify_workspace(const vk_pool* pool, const vk_tree_args* a, uint64_t* bytes) {
  if (!pool || !bytes || !a) return fail(VK_ERR_BAD_ARG, "null argument");
  TreePlan pl;
  int rc = plan_tree(pool->ctx, pool, a, &pl);
  if (rc) return rc;
  *bytes = pl.max_parts > 1 ? pl.acc_bytes + pl.ml_bytes : 0;
  return VK_OK;
}

extern "C" int vk_tree_verify_plan(const vk_pool* pool, const vk_tree_args* a, vk_tree_plan* out) {
  if (!pool || !a || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  TreePlan pl;
  int rc = plan_tree(pool->ctx, pool, a, &pl);
  if (rc) return rc;
  memset(out, 0, sizeof *out);
  snprintf(out->kernel, sizeof out->kernel, "%s", pl.kernel.c_str());
  snprintf(out->prefix_kernel, sizeof out->prefix_kernel, "%s", pl.prefix_chunks > 0 ? pl.pfx_kernel.c_str() : "");
  out->prefix_chunks = pl.prefix_chunks;
  out->prefix_row_tiles = pl.pfx_row_tiles;
  out->row_tiles = pl.n_rgroups;
  out->rows_per_tile = 16 * pl.rt;
  out->partition_tokens = pl.part_tokens;
  out->max_partitions = pl.max_parts;
  out->workspace_bytes = pl.max_parts > 1 ? pl.acc_bytes + pl.ml_bytes : 0;
  out->merge_launch = pl.max_parts == pl.prefix_chunks + 1 ? 0 : 1;
  return VK_OK;
}

extern "C" int vk_tree_verify(vk_ctx* ctx, vk_pool* pool, const vk_tree_args* a, void* stream) {
  int rc = check_pool(ctx, pool);
  if (rc) return rc;
  TreePlan pl;
  if ((rc = plan_tree(ctx, pool, a, &pl))) return rc;
  if (a->n_seqs == 0) return VK_OK;
  if (!a->q || !a->out || !a->context_lens || !a->tree_mask) return fail(VK_ERR_BAD_ARG, "null device pointer");
  if ((rc = set_device(ctx))) return rc;
  uint8_t* ws = nullptr;
  if (pl.max_parts > 1 &&
      (rc = split_workspace(ctx, a->workspace, a->workspace_bytes, pl.acc_bytes + pl.ml_bytes, &ws)))
    return rc;
  const vk_pool_desc& d = pool->desc;
  const PoolGeom& g = pool->geom;
  const uint8_t* L = pool->base + g.layer_stride * (uint64_t)a->layer;
  const float scale = a->scale != 0.f ? a->scale : 1.0f / std::sqrt((float)d.head_dim);

  DecodeParams p{};
  p.io_hd = pool->geom.io_hd;
  p.tile_hd = pool->geom.head_dim;
  p.kc = L + g.k_off;
  p.vc = L + g.v_off;
  p.ks = g.stile_bytes ? L + g.ks_off : nullptr;
  p.vs = g.stile_bytes ? L + g.vs_off : nullptr;
  p.q = a->q;
  p.out = a->out;
  p.part_acc = reinterpret_cast<float*>(ws);
  p.part_ml = ws ? reinterpret_cast<float*>(ws + pl.acc_bytes) : nullptr;
  p.block_tables = pl.bt;
  p.seq_rows = a->seq_rows;
  p.context_lens = a->context_lens;
  p.tree_mask = a->tree_mask;
  p.tile_bytes = g.tile_bytes;
  p.stile_bytes = g.stile_bytes;
  p.bt_stride = pl.bt_stride;
  p.bt_rows = pl.bt_rows;
  p.n_seqs = a->n_seqs;
  p.n_heads = a->n_heads;
  p.n_kv_heads = d.n_kv_heads;
  p.n_blocks = d.n_blocks;
  p.page_tiles = pool->geom.page_tiles;
  p.max_parts = pl.max_parts;
  p.part_tokens = pl.part_tokens;
  p.cap_tokens = (int32_t)std::min<int64_t>((int64_t)pl.prefix_blocks * kBS +
                                                (int64_t)(pl.max_parts - pl.prefix_chunks) * pl.part_tokens,
                                            (int64_t)pl.bt_stride * d.block_size);
  p.n_nodes = a->n_nodes;
  p.n_rgroups = pl.n_rgroups;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.prefix_blocks = pl.prefix_blocks;
  p.prefix_chunks = pl.prefix_chunks;
  p.err = ctx->err_word;
  const uint64_t units = (uint64_t)a->n_seqs * (pl.max_parts - pl.prefix_chunks) * d.n_kv_heads * pl.n_rgroups;
  if (units > 0x7FFFFFFFull) return fail(VK_ERR_UNSUPPORTED, "grid too large");
  if (pl.prefix_chunks > 0 &&
      (rc = launch(ctx, pl.pfx_kernel.c_str(), dim3((unsigned)pl.pfx_row_tiles, (unsigned)d.n_kv_heads,
                                                    (unsigned)pl.prefix_chunks),
                   dim3(kPfxThreads), p, stream)))
    return rc;
  if ((rc = launch(ctx, pl.kernel.c_str(), dim3((unsigned)units), dim3(64), p, stream))) return rc;
  // one partition (after any prefix chunks): the tree kernel wrote the output
  if (pl.max_parts == pl.prefix_chunks + 1) return VK_OK;

  MergeParams m{};
  m.io_hd = pool->geom.io_hd;
  m.part_acc = p.part_acc;
  m.part_ml = p.part_ml;
  m.context_lens = a->context_lens;
  m.out = a->out;
  m.n_rows = a->n_seqs * a->n_nodes * a->n_heads;
  m.rows_per_seq = a->n_nodes * a->n_heads;
  m.extra_tokens = a->n_nodes;
  m.max_parts = pl.max_parts;
  m.part_tokens = pl.part_tokens;
  m.cap_tokens = p.cap_tokens;
  m.prefix_blocks = pl.prefix_blocks;
  m.prefix_chunks = pl.prefix_chunks;
  return launch(ctx, "vk_decode_merge", dim3((unsigned)((m.n_rows + 3) / 4)), dim3(256), m, stream);
}

extern "C" int vk_tree_mask(const int32_t* parents, int32_t n_nodes, uint32_t* mask_out) {
  if (!parents || !mask_out) return fail(VK_ERR_BAD_ARG, "null argument");
  if (n_nodes < 1 || n_nodes > kMaxTreeNodes) return fail(VK_ERR_BAD_ARG, "n_nodes %d out of range [1, %d]", n_nodes, kMaxTreeNodes);
  if (parents[0] != -1) return fail(VK_ERR_BAD_ARG, "node 0 must be the root (parent -1)");
  mask_out[0] = 1u;
  for (int32_t i = 1; i < n_nodes; ++i) {
    const int32_t p = parents[i];
    if (p < 0 || p >= i) return fail(VK_ERR_BAD_ARG, "node %d has parent %d (must be in [0, %d))", i, p, i);
    mask_out[i] = mask_out[p] | (1u << i);
  }
  return VK_OK;
}

extern "C" int vk_copy_blocks(vk_ctx* ctx, vk_pool* pool, const int32_t* pairs, int32_t n_pairs, void* stream) {
  int rc = check_pool(ctx, pool);
  if (rc) return rc;
  if (n_pairs < 0 || (n_pairs > 0 && !pairs)) return fail(VK_ERR_BAD_ARG, "bad pair list");
  if (n_pairs == 0) return VK_OK;
  const int nb = pool->desc.n_blocks;
  std::vector<char> is_dst((size_t)nb, 0), is_src((size_t)nb, 0);
  for (int i = 0; i < n_pairs; ++i) {
    const int s = pairs[2 * i], t = pairs[2 * i + 1];
    if (s < 0 || s >= nb || t < 0 || t >= nb) return fail(VK_ERR_BAD_ARG, "pair %d (%d -> %d) out of range", i, s, t);
    if (is_dst[(size_t)t]) return fail(VK_ERR_BAD_ARG, "block %d is the destination of two pairs", t);
    is_dst[(size_t)t] = 1;
    is_src[(size_t)s] = 1;
  }
  for (int i = 0; i < n_pairs; ++i)
    if (is_src[(size_t)pairs[2 * i + 1]]) return fail(VK_ERR_BAD_ARG, "block %d is both a source and a destination", pairs[2 * i + 1]);
  if ((rc = set_device(ctx))) return rc;
  for (int i0 = 0; i0 < n_pairs; i0 += kMaxCopyPairs) {
    CopyParams p{};
    p.base = pool->base;
    p.g = page_geom(pool->geom);
    p.n_pairs = std::min(kMaxCopyPairs, n_pairs - i0);
    memcpy(p.pairs, pairs + 2 * i0, sizeof(int32_t) * 2 * (size_t)p.n_pairs);
    if ((rc = launch(ctx, "vk_copy_blocks", dim3((unsigned)p.n_pairs, (unsigned)pool->desc.n_layer, 2), dim3(256), p,
                     stream)))
      return rc;
  }
  return VK_OK;
}

extern "C" int vk_tree_commit(vk_ctx* ctx, vk_pool* pool, int32_t layer0, int32_t n_layers,
                              const int32_t* block_tables, int32_t bt_stride, const int32_t* context_lens,
                              const int32_t* accept, int32_t accept_stride, const int32_t* n_accept, int32_t n_seqs,
                              int32_t* status, void* stream) {
  int rc = check_pool(ctx, pool);
  if (rc) return rc;
  const vk_pool_desc& d = pool->desc;
  if (layer0 < 0 || n_layers < 0 || layer0 + n_layers > d.n_layer)
    return fail(VK_ERR_BAD_ARG, "layer range [%d, %d) outside [0, %d)", layer0, layer0 + n_layers, d.n_layer);
  if (n_seqs < 0) return fail(VK_ERR_BAD_ARG, "n_seqs < 0");
  if (bt_stride <= 0 || accept_stride <= 0) return fail(VK_ERR_BAD_ARG, "strides must be positive");
  if (n_seqs == 0 || n_layers == 0) return VK_OK;
  if (!block_tables || !context_lens || !accept || !n_accept) return fail(VK_ERR_BAD_ARG, "null device pointer");
  CommitParams p{};
  p.base = pool->base;
  p.g = pool->geom;
  p.block_tables = block_tables;
  p.context_lens = context_lens;
  p.accept = accept;
  p.n_accept = n_accept;
  p.status = status;
  p.bt_stride = bt_stride;
  p.accept_stride = accept_stride;
  p.n_seqs = n_seqs;
  p.layer0 = layer0;
  p.n_layers = n_layers;
  const std::string name = "vk_tree_commit_kv" + std::to_string(d.kv_type);
  if ((rc = set_device(ctx))) return rc;
  constexpr int kCommitLayers = 8;  // layers per workgroup (velokv_kernels.hip)
  return launch(ctx, name.c_str(),
                dim3((unsigned)n_seqs, (unsigned)d.n_kv_heads, (unsigned)((n_layers + kCommitLayers - 1) / kCommitLayers)),
                dim3(128), p, stream);
}

// ---- NIXL wire records ------------------------------------------------------
namespace {

uint64_t nixl_payload(const vk_pool* pool, int32_t n_layers, uint32_t token_len) {
  const vk_pool_desc& d = pool->desc;
  const uint64_t pages = ((uint64_t)token_len + d.block_size - 1) / d.block_size;
  const PoolGeom g = page_geom(pool->geom);
  return pages * (uint64_t)n_layers * 2 * (uint64_t)d.n_kv_heads * (g.tile_bytes + g.stile_bytes);
}

int nixl_run(vk_ctx* ctx, vk_pool* pool, int32_t layer0, int32_t n_layers, const vk_nixl_item* items,
             int32_t n_items, const int32_t* pages, int32_t n_pages, const void* wire, uint64_t wire_bytes,
             int32_t* status, void* stream, bool unpack) {
  int rc = check_pool(ctx, pool);
  if (rc) return rc;
  const vk_pool_desc& d = pool->desc;
  if (layer0 < 0 || n_layers <= 0 || layer0 + n_layers > d.n_layer)
    return fail(VK_ERR_BAD_ARG, "layer range [%d, %d) outside [0, %d)", layer0, layer0 + n_layers, d.n_layer);
  if (n_items < 0 || n_pages < 0) return fail(VK_ERR_BAD_ARG, "negative count");
  if (n_items == 0) return VK_OK;
  if (!items || !wire || !status) return fail(VK_ERR_BAD_ARG, "null argument");
  std::vector<NixlItemArg> args((size_t)n_items);
  std::vector<std::pair<uint64_t, uint64_t>> spans;  // pack: [offset, end) of each record
  for (int32_t i = 0; i < n_items; ++i) {
    const vk_nixl_item& it = items[i];
    if (it.wire_offset % 16) return fail(VK_ERR_BAD_ARG, "record %d: wire_offset %llu is not 16-aligned", i,
                                         (unsigned long long)it.wire_offset);
    const uint64_t np = ((uint64_t)it.token_len + d.block_size - 1) / d.block_size;
    if (it.first_page < 0 || (uint64_t)it.first_page + np > (uint64_t)n_pages)
      return fail(VK_ERR_BAD_ARG, "record %d: pages [%d, %llu) outside the %d page ids given", i, it.first_page,
                  (unsigned long long)(it.first_page + np), n_pages);
    if (np > 0 && !pages) return fail(VK_ERR_BAD_ARG, "pages is null");
    const uint64_t payload = nixl_payload(pool, n_layers, it.token_len);
    if (payload > 0xFFFFFFFFull)
      return fail(VK_ERR_BAD_ARG, "record %d: payload of %llu bytes exceeds the wire format's u32 byte_len", i,
                  (unsigned long long)payload);
    if (!unpack) {
      if (it.wire_offset > wire_bytes || wire_bytes - it.wire_offset < VK_NIXL_HEADER_BYTES + payload)
        return fail(VK_ERR_BAD_ARG, "record %d (%llu bytes at %llu) runs past the %llu-byte wire buffer", i,
                    (unsigned long long)(VK_NIXL_HEADER_BYTES + payload), (unsigned long long)it.wire_offset,
                    (unsigned long long)wire_bytes);
      spans.emplace_back(it.wire_offset, it.wire_offset + VK_NIXL_HEADER_BYTES + payload);
    }
    NixlItemArg& a = args[(size_t)i];
    a.block_id = it.block_id;
    a.wire_offset = it.wire_offset;
    a.token_len = it.token_len;
    a.first_page = it.first_page;
    a.n_pages = (uint32_t)np;
    a.byte_len = (uint32_t)payload;
  }
  if (!unpack) {
    std::sort(spans.begin(), spans.end());
    for (size_t i = 1; i < spans.size(); ++i)
      if (spans[i].first < spans[i - 1].second) return fail(VK_ERR_BAD_ARG, "wire records overlap");
  }
  if ((rc = set_device(ctx))) return rc;
  const PoolGeom pg = page_geom(pool->geom);
  const uint64_t page_codes = 2ull * (uint64_t)d.n_kv_heads * pg.tile_bytes;  // K + V of one page
  const int32_t n_slices = (int32_t)((page_codes / 16 + kNixlSliceVecs - 1) / kNixlSliceVecs);
  for (int32_t i0 = 0; i0 < n_items;) {
    NixlParams p{};
    p.base = pool->base;
    p.g = pg;
    p.pages = pages;
    p.wire = reinterpret_cast<uint8_t*>(const_cast<void*>(wire));
    p.wire_bytes = wire_bytes;
    p.status = status + i0;
    p.layer0 = layer0;
    p.n_layers = n_layers;
    p.unpack = unpack ? 1 : 0;
    p.n_slices = n_slices;
    uint64_t units = 0;  // slices of this launch
    int n = 0;
    while (i0 + n < n_items && n < kMaxNixlItems) {
      const uint64_t u = (uint64_t)args[(size_t)(i0 + n)].n_pages * (uint64_t)n_layers * (uint64_t)n_slices;
      if (n > 0 && units + u > 0x7FFFFFFFull) break;
      if (u > 0x7FFFFFFFull) return fail(VK_ERR_UNSUPPORTED, "record %d has too many pages x layers", i0 + n);
      p.items[n] = args[(size_t)(i0 + n)];
      p.items[n].unit_begin = (uint32_t)units;
      units += u;
      ++n;
    }
    p.n_items = n;
    if ((rc = launch(ctx, "vk_nixl_check", dim3((unsigned)n), dim3(256), p, stream))) return rc;
    if (units > 0 && (rc = launch(ctx, "vk_nixl_copy", dim3((unsigned)units), dim3(256), p, stream))) return rc;
    i0 += n;
  }
  return VK_OK;
}

}  // namespace

extern "C" int vk_nixl_payload_bytes(const vk_pool* pool, int32_t n_layers, uint32_t token_len, uint64_t* bytes) {
  if (!pool || !bytes) return fail(VK_ERR_BAD_ARG, "null argument");
  if (n_layers <= 0 || n_layers > pool->desc.n_layer) return fail(VK_ERR_BAD_ARG, "n_layers %d out of range", n_layers);
  *bytes = nixl_payload(pool, n_layers, token_len);
  return VK_OK;
}

extern "C" int vk_nixl_pack(vk_ctx* ctx, vk_pool* pool, int32_t layer0, int32_t n_layers, const vk_nixl_item* items,
                            int32_t n_items, const int32_t* pages, int32_t n_pages, void* wire, uint64_t wire_bytes,
                            int32_t* status, void* stream) {
  return nixl_run(ctx, pool, layer0, n_layers, items, n_items, pages, n_pages, wire, wire_bytes, status, stream, false);
}

extern "C" int vk_nixl_unpack(vk_ctx* ctx, vk_pool* pool, int32_t layer0, int32_t n_layers, const vk_nixl_item* items,
                              int32_t n_items, const int32_t* pages, int32_t n_pages, const void* wire,
                              uint64_t wire_bytes, int32_t* status, void* stream) {
  return nixl_run(ctx, pool, layer0, n_layers, items, n_items, pages, n_pages, wire, wire_bytes, status, stream, true);
}

// ============================================================================
// host block manager: PagedAttentionBlockManager (paged_attention.rs:92-212)
// plus per-page reference counts.
// ============================================================================
struct vk_block_manager {
  int32_t block_size = 0;
  int32_t total_pages = 0;
  std::deque<uint32_t> free_pages;                    // FIFO (paged_attention.rs:130-133)
  std::map<uint64_t, std::vector<uint32_t>> mappings; // handle -> pages
  std::vector<int32_t> refs;                          // per-page reference count
  int64_t pages_for(int64_t tokens) const { return (tokens + block_size - 1) / block_size; }
};

namespace {
int copy_pages(const std::vector<uint32_t>& v, uint32_t* out, int32_t cap, int32_t* n_out) {
  if (n_out) *n_out = (int32_t)v.size();
  if (out) {
    if ((int64_t)v.size() > cap) return fail(VK_ERR_BAD_ARG, "output capacity %d < %zu pages", cap, v.size());
    std::copy(v.begin(), v.end(), out);
  }
  return VK_OK;
}
int take_pages(vk_block_manager* bm, int64_t n, std::vector<uint32_t>* pages) {
  if (n > (int64_t)bm->free_pages.size())
    return fail(VK_ERR_OUT_OF_PAGES, "requested %lld pages but only %zu are available", (long long)n,
                bm->free_pages.size());
  for (int64_t i = 0; i < n; ++i) {
    const uint32_t pg = bm->free_pages.front();
    bm->free_pages.pop_front();
    bm->refs[pg] = 1;
    pages->push_back(pg);
  }
  return VK_OK;
}
}  // namespace

extern "C" int vk_bm_create(int32_t block_size, int32_t total_pages, vk_block_manager** out) {
  if (!out) return fail(VK_ERR_BAD_ARG, "out is null");
  *out = nullptr;
  if (block_size <= 0) return fail(VK_ERR_INVALID_BLOCK_SIZE, "block size must be greater than zero");
  if (total_pages < 0) return fail(VK_ERR_BAD_ARG, "total_pages < 0");
  auto* bm = new vk_block_manager();
  bm->block_size = block_size;
  bm->total_pages = total_pages;
  bm->refs.assign((size_t)total_pages, 0);
  for (int32_t i = 0; i < total_pages; ++i) bm->free_pages.push_back((uint32_t)i);
  *out = bm;
  return VK_OK;
}

extern "C" int vk_bm_destroy(vk_block_manager* bm) {
  delete bm;
  return VK_OK;
}

extern "C" int vk_bm_block_size(const vk_block_manager* bm, int32_t* out) {
  if (!bm || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  *out = bm->block_size;
  return VK_OK;
}

extern "C" int vk_bm_free_pages(const vk_block_manager* bm, int32_t* out) {
  if (!bm || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  *out = (int32_t)bm->free_pages.size();
  return VK_OK;
}

extern "C" int vk_bm_allocate(vk_block_manager* bm, uint64_t handle, int64_t token_len, uint32_t* pages_out,
                              int32_t cap, int32_t* n_out) {
  if (!bm) return fail(VK_ERR_BAD_ARG, "null manager");
  if (token_len < 0) return fail(VK_ERR_BAD_ARG, "token_len < 0");
  if (bm->mappings.count(handle)) return fail(VK_ERR_BAD_ARG, "handle %llu already mapped", (unsigned long long)handle);
  std::vector<uint32_t> pages;
  int rc = take_pages(bm, bm->pages_for(token_len), &pages);
  if (rc) return rc;
  bm->mappings[handle] = pages;
  return copy_pages(pages, pages_out, cap, n_out);
}

extern "C" int vk_bm_release(vk_block_manager* bm, uint64_t handle) {
  if (!bm) return fail(VK_ERR_BAD_ARG, "null manager");
  auto it = bm->mappings.find(handle);
  if (it == bm->mappings.end()) return fail(VK_ERR_UNKNOWN_HANDLE, "unknown KV handle %llu", (unsigned long long)handle);
  for (uint32_t pg : it->second)
    if (--bm->refs[pg] == 0) bm->free_pages.push_back(pg);
  bm->mappings.erase(it);
  return VK_OK;
}

extern "C" int vk_bm_pages(const vk_block_manager* bm, uint64_t handle, uint32_t* pages_out, int32_t cap,
                           int32_t* n_out) {
  if (!bm) return fail(VK_ERR_BAD_ARG, "null manager");
  auto it = bm->mappings.find(handle);
  if (it == bm->mappings.end()) return fail(VK_ERR_UNKNOWN_HANDLE, "unknown KV handle %llu", (unsigned long long)handle);
  return copy_pages(it->second, pages_out, cap, n_out);
}

extern "C" int vk_bm_fork(vk_block_manager* bm, uint64_t parent, uint64_t child, int64_t shared_tokens,
                          int64_t token_len, uint32_t* pages_out, int32_t cap, int32_t* n_out) {
  if (!bm) return fail(VK_ERR_BAD_ARG, "null manager");
  auto it = bm->mappings.find(parent);
  if (it == bm->mappings.end()) return fail(VK_ERR_UNKNOWN_HANDLE, "unknown KV handle %llu", (unsigned long long)parent);
  if (bm->mappings.count(child)) return fail(VK_ERR_BAD_ARG, "handle %llu already mapped", (unsigned long long)child);
  if (shared_tokens < 0 || token_len < shared_tokens) return fail(VK_ERR_BAD_ARG, "need 0 <= shared_tokens <= token_len");
  const int64_t n_shared = bm->pages_for(shared_tokens);
  if (n_shared > (int64_t)it->second.size()) return fail(VK_ERR_BAD_ARG, "parent holds only %zu pages", it->second.size());
  std::vector<uint32_t> pages(it->second.begin(), it->second.begin() + n_shared);
  const int64_t n_new = bm->pages_for(token_len) - n_shared;
  std::vector<uint32_t> fresh;
  int rc = take_pages(bm, n_new, &fresh);
  if (rc) return rc;
  for (uint32_t pg : pages) ++bm->refs[pg];
  pages.insert(pages.end(), fresh.begin(), fresh.end());
  bm->mappings[child] = pages;
  return copy_pages(pages, pages_out, cap, n_out);
}

extern "C" int vk_bm_extend(vk_block_manager* bm, uint64_t handle, int64_t token_len, uint32_t* pages_out,
                            int32_t cap, int32_t* n_out) {
  if (!bm) return fail(VK_ERR_BAD_ARG, "null manager");
  auto it = bm->mappings.find(handle);
  if (it == bm->mappings.end()) return fail(VK_ERR_UNKNOWN_HANDLE, "unknown KV handle %llu", (unsigned long long)handle);
  if (token_len < 0) return fail(VK_ERR_BAD_ARG, "token_len < 0");
  const int64_t need = bm->pages_for(token_len) - (int64_t)it->second.size();
  if (need > 0) {
    std::vector<uint32_t> fresh;
    int rc = take_pages(bm, need, &fresh);
    if (rc) return rc;
    it->second.insert(it->second.end(), fresh.begin(), fresh.end());
  }
  return copy_pages(it->second, pages_out, cap, n_out);
}

extern "C" int vk_bm_cow(vk_block_manager* bm, uint64_t handle, int32_t page_idx, int32_t* src, int32_t* dst,
                         int32_t* copied) {
  if (!bm || !src || !dst || !copied) return fail(VK_ERR_BAD_ARG, "null argument");
  auto it = bm->mappings.find(handle);
  if (it == bm->mappings.end()) return fail(VK_ERR_UNKNOWN_HANDLE, "unknown KV handle %llu", (unsigned long long)handle);
  if (page_idx < 0 || page_idx >= (int32_t)it->second.size()) return fail(VK_ERR_BAD_ARG, "page index %d out of range", page_idx);
  const uint32_t old = it->second[(size_t)page_idx];
  *copied = 0;
  *src = *dst = (int32_t)old;
  if (bm->refs[old] <= 1) return VK_OK;
  std::vector<uint32_t> fresh;
  int rc = take_pages(bm, 1, &fresh);
  if (rc) return rc;
  --bm->refs[old];
  it->second[(size_t)page_idx] = fresh[0];
  *dst = (int32_t)fresh[0];
  *copied = 1;
  return VK_OK;
}

extern "C" int vk_bm_refcount(const vk_block_manager* bm, uint32_t page, int32_t* out) {
  if (!bm || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  if (page >= (uint32_t)bm->total_pages) return fail(VK_ERR_BAD_ARG, "page %u out of range", page);
  *out = bm->refs[page];
  return VK_OK;
}

// ============================================================================
// device memory / stream helpers
// ============================================================================
extern "C" int vk_dev_alloc(vk_ctx* ctx, uint64_t bytes, void** out) {
  if (!ctx || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  int rc = set_device(ctx);
  if (rc) return rc;
  HIP_TRY(hipMalloc(out, std::max<uint64_t>(bytes, 1)));
  return VK_OK;
}
extern "C" int vk_dev_free(vk_ctx* ctx, void* p) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  int rc = set_device(ctx);
  if (rc) return rc;
  HIP_TRY(hipFree(p));
  return VK_OK;
}
extern "C" int vk_memcpy_h2d(vk_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  if (!bytes) return VK_OK;
  int rc = set_device(ctx);
  if (rc) return rc;
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return VK_OK;
}
extern "C" int vk_memcpy_d2h(vk_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  if (!bytes) return VK_OK;
  int rc = set_device(ctx);
  if (rc) return rc;
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return VK_OK;
}
extern "C" int vk_memset_d(vk_ctx* ctx, void* dst, int value, uint64_t bytes) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  int rc = set_device(ctx);
  if (rc) return rc;
  HIP_TRY(hipMemset(dst, value, bytes));
  return VK_OK;
}
extern "C" int vk_stream_create(vk_ctx* ctx, void** out) {
  if (!ctx || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  int rc = set_device(ctx);
  if (rc) return rc;
  hipStream_t s;
  HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = s;
  return VK_OK;
}
extern "C" int vk_stream_destroy(vk_ctx* ctx, void* stream) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  HIP_TRY(hipStreamDestroy(reinterpret_cast<hipStream_t>(stream)));
  return VK_OK;
}
namespace {
// Reads and clears the context's misuse word; VK_ERR_BAD_ARG naming the misuse
// when a kernel set a flag since the last read.
int take_misuse(vk_ctx* ctx, uint32_t* flags_out) {
  uint32_t flags = 0;
  HIP_TRY(hipMemcpy(&flags, ctx->err_word, sizeof flags, hipMemcpyDeviceToHost));
  if (flags_out) *flags_out = flags;
  if (flags == 0) return VK_OK;
  const uint32_t zero = 0;
  HIP_TRY(hipMemcpy(ctx->err_word, &zero, sizeof zero, hipMemcpyHostToDevice));
  std::string what;
  if (flags & VK_MISUSE_PAGE_OUT_OF_POOL)
    what += "a block table handed to an attention call held a page id outside the pool (clamped into the pool); ";
  if (flags & VK_MISUSE_BLK_SPLIT_RUN)
    what += "an INT8 per-block append had tokens of one block that were not adjacent in the call "
            "(its codes are not defined); ";
  return fail(VK_ERR_BAD_ARG, "misuse reported by the kernels (flags 0x%x): %s", flags, what.c_str());
}
}  // namespace

extern "C" int vk_stream_sync(vk_ctx* ctx, void* stream) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  int rc = set_device(ctx);
  if (rc) return rc;
  HIP_TRY(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)));
  return take_misuse(ctx, nullptr);
}

extern "C" int vk_ctx_check(vk_ctx* ctx, uint32_t* flags) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  int rc = set_device(ctx);
  if (rc) return rc;
  HIP_TRY(hipDeviceSynchronize());
  return take_misuse(ctx, flags);
}
extern "C" int vk_event_create(vk_ctx* ctx, void** out) {
  if (!ctx || !out) return fail(VK_ERR_BAD_ARG, "null argument");
  int rc = set_device(ctx);
  if (rc) return rc;
  hipEvent_t e;
  HIP_TRY(hipEventCreate(&e));
  *out = e;
  return VK_OK;
}
extern "C" int vk_event_destroy(vk_ctx* ctx, void* ev) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  HIP_TRY(hipEventDestroy(reinterpret_cast<hipEvent_t>(ev)));
  return VK_OK;
}
extern "C" int vk_event_record(vk_ctx* ctx, void* ev, void* stream) {
  if (!ctx) return fail(VK_ERR_BAD_ARG, "null context");
  HIP_TRY(hipEventRecord(reinterpret_cast<hipEvent_t>(ev), reinterpret_cast<hipStream_t>(stream)));
  return VK_OK;
}
extern "C" int vk_event_elapsed_ms(vk_ctx* ctx, void* start, void* end, float* ms) {
  if (!ctx || !ms) return fail(VK_ERR_BAD_ARG, "null argument");
  HIP_TRY(hipEventSynchronize(reinterpret_cast<hipEvent_t>(end)));
  HIP_TRY(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start), reinterpret_cast<hipEvent_t>(end)));
  return VK_OK;
}

extern "C" int vk_fill_normal_f16(vk_ctx* ctx, void* dev, uint64_t n, uint64_t seed, int32_t row_len,
                                  float outlier_scale, void* stream) {
  if (!ctx) return fail(VK_ERR_NOT_WIRED, "context is null");
  if (!dev && n) return fail(VK_ERR_BAD_ARG, "null device pointer");
  if (row_len <= 0) return fail(VK_ERR_BAD_ARG, "row_len must be positive");
  if (n == 0) return VK_OK;
  int rc = set_device(ctx);
  if (rc) return rc;
  FillParams p{reinterpret_cast<uint16_t*>(dev), n, seed, row_len, outlier_scale};
  const uint64_t blocks = (n + 255) / 256;
  if (blocks > 0x7FFFFFFFull) return fail(VK_ERR_BAD_ARG, "fill too large");
  return launch(ctx, "vk_fill_normal_f16", dim3((unsigned)blocks), dim3(256), p, stream);
}
