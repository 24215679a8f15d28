// libak: compile (hiprtc), load and launch generated gfx950 kernels behind a plain C ABI (include/ak.h).
#include "../../include/ak.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

struct ak_module {
  hipModule_t module;
};

struct ak_kernel {
  hipFunction_t function;
};

namespace {

thread_local std::string last_error;

int fail(const std::string& what) {
  last_error = what;
  return 1;
}

int hip_fail(const char* what, hipError_t e) {
  return fail(std::string(what) + ": " + hipGetErrorName(e) + ": " + hipGetErrorString(e));
}

std::vector<const char*> split_options(const char* opts) {
  std::vector<const char*> out;
  if (!opts) return out;
  for (const char* p = opts; *p; p += std::strlen(p) + 1) out.push_back(p);
  return out;
}

}  // namespace

extern "C" {

int ak_version(void) { return (1 << 16) | 0; }

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
