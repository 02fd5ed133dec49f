// The library's GPU kernels, loaded with the module API.
//
// The kernels (sh_unpack.hip, sh_digest.hip) are compiled for gfx950 into code objects of their
// own, which the build embeds in this library (symbols sh_co_<name> .. sh_co_<name>_end, from the
// generated sh_code_objects.S). Nothing in the library registers a fat binary with the HIP
// runtime, so the library leaves no handler to the process's exit: the compiler-emitted module
// constructor of a .hip translation unit would register its fat binary at load and queue an
// unregistration (a call into HIP that unloads the code on every device) for the exit-time
// destructors, to run in whatever order the runtime, a profiler's tool library and the other
// libraries end in. Here each device loads the code objects on first use, with that device
// current, and sh_shutdown unloads them (unload_kernels) while the runtime is whole.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <mutex>
#include <new>

#include "sh_internal.h"

extern "C" {
extern const unsigned char sh_co_unpack[];
extern const unsigned char sh_co_digest[];
}

namespace {

enum ModuleId : int { kModUnpack = 0, kModDigest, kModules };

struct KernelSpec {
  ModuleId module;
  const char* name;
};

// Indexed by sh::KernelId.
constexpr KernelSpec kKernelSpecs[sh::kKernelCount] = {
    {kModUnpack, "sh_dequant_i8_bf16_kernel"},
    {kModUnpack, "sh_dequant_i8_bf16_zp_kernel"},
    {kModUnpack, "sh_cast_f32_bf16_kernel"},
    {kModUnpack, "sh_unpack_mixed_kernel"},
    {kModUnpack, "sh_unpack_mixed_zp_kernel"},
    {kModUnpack, "sh_put_descs_kernel"},
    {kModUnpack, "sh_fill_tile_map_kernel"},
    {kModDigest, "sh_digest_kernel"},
    {kModDigest, "sh_digest_compare_kernel"},
};

struct DeviceKernels {
  hipModule_t module[kModules] = {};
  hipFunction_t fn[sh::kKernelCount] = {};
  void* scratch = nullptr;  // the unpack module's `scratch` array on this device
  size_t scratch_bytes = 0;
};

constexpr int kMaxDevices = 64;
// Published once loaded (release); read without the lock on every launch (acquire).
std::atomic<DeviceKernels*> g_kernels[kMaxDevices];
std::mutex g_load_mu;

const void* image_of(ModuleId m) { return m == kModUnpack ? (const void*)sh_co_unpack : (const void*)sh_co_digest; }

int unload(DeviceKernels* k) {
  hipError_t first = hipSuccess;
  for (hipModule_t& m : k->module) {
    if (m == nullptr) continue;
    const hipError_t e = hipModuleUnload(m);
    if (first == hipSuccess) first = e;
    m = nullptr;
  }
  return first == hipSuccess ? SH_OK
                             : sh::fail(SH_ERR_HIP, "hipModuleUnload: HIP error %d (%s)", (int)first,
                                        hipGetErrorString(first));
}

// Loads the code objects on device `dev` (current) and resolves every kernel and the scratch.
int load(int dev, DeviceKernels** out, const char* who) {
  DeviceKernels* k = new (std::nothrow) DeviceKernels();
  if (k == nullptr) return sh::fail(SH_ERR_OOM, "%s: out of host memory", who);
  auto bail = [&](hipError_t e, const char* what, const char* name) {
    (void)unload(k);
    delete k;
    return sh::fail(e == hipErrorOutOfMemory ? SH_ERR_OOM : SH_ERR_HIP, "%s: %s %s on device %d: HIP error %d (%s)",
                    who, what, name, dev, (int)e, hipGetErrorString(e));
  };
  for (int m = 0; m < kModules; ++m) {
    const hipError_t e = hipModuleLoadData(&k->module[m], image_of((ModuleId)m));
    if (e != hipSuccess) return bail(e, "loading code object", m == kModUnpack ? "unpack" : "digest");
  }
  for (int i = 0; i < sh::kKernelCount; ++i) {
    const hipError_t e = hipModuleGetFunction(&k->fn[i], k->module[kKernelSpecs[i].module], kKernelSpecs[i].name);
    if (e != hipSuccess) return bail(e, "resolving kernel", kKernelSpecs[i].name);
  }
  hipDeviceptr_t p = nullptr;
  const hipError_t e = hipModuleGetGlobal(&p, &k->scratch_bytes, k->module[kModUnpack], "scratch");
  if (e != hipSuccess || p == nullptr) return bail(e, "resolving the device array", "scratch");
  if (k->scratch_bytes < SH_UNPACK_NOALLOC_SCRATCH_BYTES) {
    const size_t got = k->scratch_bytes;
    (void)unload(k);
    delete k;
    return sh::fail(SH_ERR_HIP, "%s: the scratch array on device %d holds %zu bytes, not %u", who, dev, got,
                    (unsigned)SH_UNPACK_NOALLOC_SCRATCH_BYTES);
  }
  k->scratch = (void*)p;
  *out = k;
  return SH_OK;
}

int current(DeviceKernels** out, const char* who) {
  int dev = -1;
  SH_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return sh::fail(SH_ERR_INVALID, "%s: device %d out of range", who, dev);
  DeviceKernels* k = g_kernels[dev].load(std::memory_order_acquire);
  if (k == nullptr) {
    std::lock_guard<std::mutex> lk(g_load_mu);
    k = g_kernels[dev].load(std::memory_order_relaxed);
    if (k == nullptr) {
      if (int st = load(dev, &k, who)) return st;
      g_kernels[dev].store(k, std::memory_order_release);
    }
  }
  *out = k;
  return SH_OK;
}

}  // namespace

namespace sh {

int launch_kernel(KernelId id, uint32_t grid, uint32_t block, hipStream_t stream, void** args, const char* who) {
  DeviceKernels* k = nullptr;
  if (int st = current(&k, who)) return st;
  const hipError_t e = hipModuleLaunchKernel(k->fn[id], grid, 1, 1, block, 1, 1, 0, stream, args, nullptr);
  if (e != hipSuccess)
    return fail(SH_ERR_HIP, "%s: launching %s (%u workgroups): HIP error %d (%s)", who, kKernelSpecs[id].name, grid,
                (int)e, hipGetErrorString(e));
  return SH_OK;
}

int noalloc_scratch(void** ptr, const char* who) {
  DeviceKernels* k = nullptr;
  if (int st = current(&k, who)) return st;
  *ptr = k->scratch;
  return SH_OK;
}

int unload_kernels() {
  std::lock_guard<std::mutex> lk(g_load_mu);
  int cur = -1;
  (void)hipGetDevice(&cur);
  int status = SH_OK;
  for (int dev = 0; dev < kMaxDevices; ++dev) {
    DeviceKernels* k = g_kernels[dev].load(std::memory_order_acquire);
    if (k == nullptr) continue;
    // Work queued with these kernels must end before their code is unloaded.
    hipError_t e = hipSetDevice(dev);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
      if (status == SH_OK)
        status = fail(SH_ERR_HIP, "sh_shutdown: synchronizing device %d before unloading kernels: HIP error %d (%s)",
                      dev, (int)e, hipGetErrorString(e));
      continue;  // left loaded: something may still run them
    }
    g_kernels[dev].store(nullptr, std::memory_order_release);
    const int st = unload(k);
    if (status == SH_OK) status = st;
    delete k;
  }
  if (cur >= 0) (void)hipSetDevice(cur);
  return status;
}

int kernels_loaded() {
  int n = 0;
  for (int dev = 0; dev < kMaxDevices; ++dev) n += g_kernels[dev].load(std::memory_order_acquire) != nullptr;
  return n;
}

}  // namespace sh
