// libak: compile (hiprtc), load and launch generated gfx950 kernels behind a plain C ABI (include/ak.h).
#include "../../include/ak.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

struct ak_module {
  hipModule_t module;
};

struct ak_kernel {
  hipFunction_t function;
};

// The workspace of ak_launch_scratch: one array per device (each GPU holds its own copy once the library's
// code object is loaded there). Host code never uses its name as an address: the per-device pointer comes
// from hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) unsigned char scratch[AK_SCRATCH_BYTES];

namespace {

thread_local std::string last_error;

int fail(const std::string& what) {
  last_error = what;
  return 1;
}

int hip_fail(const char* what, hipError_t e) {
  return fail(std::string(what) + ": " + hipGetErrorName(e) + ": " + hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices] = {};

int scratch_pointer(void** out) {
  int device = 0;
  hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return hip_fail("hipGetDevice", e);
  if (device < 0 || device >= kMaxDevices) return fail("ak_launch_scratch: device index out of range");
  std::lock_guard<std::mutex> hold(scratch_mutex);
  if (!scratch_ptr[device]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail("hipGetSymbolAddress(scratch)", e);
    if (!p) return fail("hipGetSymbolAddress(scratch) gave a null address");
    scratch_ptr[device] = p;
  }
  *out = scratch_ptr[device];
  return 0;
}

std::vector<const char*> split_options(const char* opts) {
  std::vector<const char*> out;
  if (!opts) return out;
  for (const char* p = opts; *p; p += std::strlen(p) + 1) out.push_back(p);
  return out;
}

}  // namespace

extern "C" {

int ak_version(void) { return (1 << 16) | 1; }

const char* ak_last_error(void) { return last_error.c_str(); }

int ak_compile(const char* source, const char* name, const char* opts, void** code, size_t* size) {
  last_error.clear();
  if (!source || !code || !size) return fail("ak_compile: null argument");
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, name ? name : "kernel.hip", 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) return fail(std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r));
  std::vector<const char*> options = split_options(opts);
  r = hiprtcCompileProgram(prog, static_cast<int>(options.size()), options.data());
  size_t log_size = 0;
  hiprtcGetProgramLogSize(prog, &log_size);
  std::string log(log_size, '\0');
  if (log_size) hiprtcGetProgramLog(prog, &log[0]);
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    return fail(std::string("hiprtc: ") + hiprtcGetErrorString(r) + "\n" + log);
  }
  size_t n = 0;
  r = hiprtcGetCodeSize(prog, &n);
  if (r != HIPRTC_SUCCESS || n == 0) {
    hiprtcDestroyProgram(&prog);
    return fail("hiprtcGetCodeSize failed");
  }
  void* buffer = std::malloc(n);
  if (!buffer) {
    hiprtcDestroyProgram(&prog);
    return fail("out of host memory");
  }
  r = hiprtcGetCode(prog, static_cast<char*>(buffer));
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS) {
    std::free(buffer);
    return fail(std::string("hiprtcGetCode: ") + hiprtcGetErrorString(r));
  }
  *code = buffer;
  *size = n;
  return 0;
}

void ak_free(void* p) { std::free(p); }

int ak_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int ak_module_load(const void* code, size_t size, ak_module** out) {
  last_error.clear();
  if (!code || !size || !out) return fail("ak_module_load: null argument");
  hipModule_t m;
  hipError_t e = hipModuleLoadData(&m, code);
  if (e != hipSuccess) return hip_fail("hipModuleLoadData", e);
  *out = new ak_module{m};
  return 0;
}

int ak_module_free(ak_module* module) {
  if (!module) return 0;
  hipError_t e = hipModuleUnload(module->module);
  delete module;
  if (e != hipSuccess) return hip_fail("hipModuleUnload", e);
  return 0;
}

int ak_get_kernel(ak_module* module, const char* symbol, ak_kernel** out) {
  last_error.clear();
  if (!module || !symbol || !out) return fail("ak_get_kernel: null argument");
  hipFunction_t f;
  hipError_t e = hipModuleGetFunction(&f, module->module, symbol);
  if (e != hipSuccess) return hip_fail((std::string("hipModuleGetFunction ") + symbol).c_str(), e);
  *out = new ak_kernel{f};
  return 0;
}

int ak_kernel_info(ak_kernel* kernel, int* vgprs, int* lds_bytes, int* private_bytes, int* max_threads) {
  last_error.clear();
  if (!kernel) return fail("ak_kernel_info: null kernel");
  int v = 0;
  if (vgprs && hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_NUM_REGS, kernel->function) == hipSuccess) *vgprs = v;
  if (lds_bytes && hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, kernel->function) == hipSuccess)
    *lds_bytes = v;
  if (private_bytes && hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES, kernel->function) == hipSuccess)
    *private_bytes = v;
  if (max_threads &&
      hipFuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, kernel->function) == hipSuccess)
    *max_threads = v;
  return 0;
}

int ak_launch(ak_kernel* kernel, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t by, uint32_t bz,
              uint32_t lds_bytes, const void* args, size_t args_size, void* stream) {
  last_error.clear();
  if (!kernel) return fail("ak_launch: null kernel");
  if (gx == 0 || gy == 0 || gz == 0 || bx == 0 || by == 0 || bz == 0) return fail("ak_launch: empty grid or block");
  size_t size = args_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(args), HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                    HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(kernel->function, gx, gy, gz, bx, by, bz, lds_bytes,
                                       static_cast<hipStream_t>(stream), nullptr, args_size ? config : nullptr);
  if (e != hipSuccess) return hip_fail("hipModuleLaunchKernel", e);
  return 0;
}

int ak_launch_scratch(ak_kernel* kernel, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t by,
                      uint32_t bz, uint32_t lds_bytes, const void* args, size_t args_size, const size_t* fields,
                      const uint64_t* offsets, const uint64_t* sizes, size_t count, void* stream) {
  last_error.clear();
  if (!kernel) return fail("ak_launch_scratch: null kernel");
  if (gx == 0 || gy == 0 || gz == 0 || bx == 0 || by == 0 || bz == 0)
    return fail("ak_launch_scratch: empty grid or block");
  if (args_size > AK_SCRATCH_MAX_ARGS) return fail("ak_launch_scratch: argument struct larger than 4096 bytes");
  if (args_size && !args) return fail("ak_launch_scratch: null arguments");
  if (count && (!fields || !offsets || !sizes)) return fail("ak_launch_scratch: null workspace description");
  for (size_t i = 0; i < count; ++i) {
    if (fields[i] % 8 || fields[i] + 8 > args_size)
      return fail("ak_launch_scratch: workspace field " + std::to_string(i) + " is not a pointer field of the arguments");
    if (offsets[i] % 256) return fail("ak_launch_scratch: workspace offset " + std::to_string(offsets[i]) +
                                      " is not 256-byte aligned");
    if (offsets[i] > AK_SCRATCH_BYTES || sizes[i] > AK_SCRATCH_BYTES - offsets[i])
      return fail("ak_launch_scratch: workspace of " + std::to_string(sizes[i]) + " bytes at offset " +
                  std::to_string(offsets[i]) + " exceeds the scratch array of " + std::to_string(AK_SCRATCH_BYTES) +
                  " bytes");
  }
  unsigned char patched[AK_SCRATCH_MAX_ARGS];
  if (args_size) std::memcpy(patched, args, args_size);
  if (count) {
    void* base = nullptr;
    if (scratch_pointer(&base)) return 1;
    for (size_t i = 0; i < count; ++i) {
      void* p = static_cast<unsigned char*>(base) + offsets[i];
      std::memcpy(patched + fields[i], &p, sizeof p);
    }
  }
  size_t size = args_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, patched, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                    HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(kernel->function, gx, gy, gz, bx, by, bz, lds_bytes,
                                       static_cast<hipStream_t>(stream), nullptr, args_size ? config : nullptr);
  if (e != hipSuccess) return hip_fail("hipModuleLaunchKernel", e);
  return 0;
}

int ak_event_create(void** event) {
  last_error.clear();
  hipEvent_t ev;
  hipError_t e = hipEventCreate(&ev);
  if (e != hipSuccess) return hip_fail("hipEventCreate", e);
  *event = ev;
  return 0;
}

int ak_event_record(void* event, void* stream) {
  hipError_t e = hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail("hipEventRecord", e);
  return 0;
}

int ak_event_elapsed_ms(void* start, void* stop, float* ms) {
  hipError_t e = hipEventSynchronize(static_cast<hipEvent_t>(stop));
  if (e != hipSuccess) return hip_fail("hipEventSynchronize", e);
  e = hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop));
  if (e != hipSuccess) return hip_fail("hipEventElapsedTime", e);
  return 0;
}

int ak_event_destroy(void* event) {
  hipError_t e = hipEventDestroy(static_cast<hipEvent_t>(event));
  if (e != hipSuccess) return hip_fail("hipEventDestroy", e);
  return 0;
}

int ak_stream_synchronize(void* stream) {
  hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail("hipStreamSynchronize", e);
  return 0;
}

}  // extern "C"
