/* libak: the C-ABI between the kernel compiler (Python, tilejax_amd) and the GPU (HIP on gfx950).
 *
 * The reference reaches its compiled kernels only through the generated `entry(*inputs)`, whose body is
 * one `pl.pallas_call(kernel, out_shape, in_specs, out_specs, scratch_shapes, ...)(*tables, *inputs)`
 * (src/autokernel/codegen.py:456-502), jitted by `Lowered.run` (src/autokernel/api.py:69-72) and timed by
 * the profiler (src/autokernel/profiling.py:231-264). On gfx950 the generated module is HIP C++ text;
 * these entry points compile it (hiprtc), load it, and launch its kernels on the caller's stream with
 * raw device pointers. Every buffer belongs to the caller (PyTorch allocates them); the library only owns
 * modules and kernel handles.
 *
 * Conventions: functions return 0 on success, nonzero on failure; the failure's text is then
 * `ak_last_error()` (thread-local, valid until the thread's next call). Plain C types only.
 */
#ifndef TILEJAX_AK_H
#define TILEJAX_AK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ak_module ak_module; /* a loaded code object */
typedef struct ak_kernel ak_kernel; /* one __global__ function of it */

/* The library's version, (major << 16) | minor. */
int ak_version(void);

/* The last error of this thread, or "" if none. */
const char* ak_last_error(void);

/* Compile HIP source to a gfx950 code object with hiprtc (no GPU needed). `opts` is a NUL-separated,
 * double-NUL-terminated list of options, e.g. "--offload-arch=gfx950\0-O3\0\0". On success *code is a
 * buffer of *size bytes that the caller frees with ak_free. On a compile error the log is
 * ak_last_error(). Replaces the Mosaic compile behind `pl.pallas_call` (codegen.py:468-501). */
int ak_compile(const char* source, const char* name, const char* opts, void** code, size_t* size);

/* Free a buffer this library returned. */
void ak_free(void* p);

/* Number of GPUs HIP sees (0 without one; never an error). */
int ak_device_count(void);

/* Load a code object onto the current device. Replaces the exec of the generated module
 * (api.py:306-312, `_load`). */
int ak_module_load(const void* code, size_t size, ak_module** out);

/* Unload a module; its kernels become invalid. */
int ak_module_free(ak_module* module);

/* Find a __global__ function by its (extern "C") symbol. */
int ak_get_kernel(ak_module* module, const char* symbol, ak_kernel** out);

/* Registers, LDS and scratch a kernel takes: vgprs, agprs(or -1 if unknown), static LDS bytes, private
 * (spill) bytes per lane, max threads per block. */
int ak_kernel_info(ak_kernel* kernel, int* vgprs, int* lds_bytes, int* private_bytes, int* max_threads);

/* Launch `kernel` on `stream` (a hipStream_t; NULL is the default stream) with grid (gx, gy, gz),
 * blocks of (bx, by, bz) threads, `lds_bytes` of dynamic LDS, and its kernel arguments packed as one
 * struct of `args_size` bytes at `args`. Replaces one `pl.pallas_call(...)(...)` (codegen.py:468-501). */
int ak_launch(ak_kernel* kernel, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t by, uint32_t bz,
              uint32_t lds_bytes, const void* args, size_t args_size, void* stream);

/* HIP events for device time on a stream: what the profiler reads in place of libtpu trace regions
 * (profiling.py:160-174, `device_events`). */
int ak_event_create(void** event);
int ak_event_record(void* event, void* stream);
int ak_event_elapsed_ms(void* start, void* stop, float* ms);
int ak_event_destroy(void* event);
int ak_stream_synchronize(void* stream);

/* Bytes of the library's own scratch array on each device: the most ak_launch_scratch can lay out. */
#define AK_SCRATCH_BYTES (64u << 20)
/* The most argument bytes ak_launch_scratch takes (it patches a copy held on the stack). */
#define AK_SCRATCH_MAX_ARGS 4096u

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): ak_launch, with the kernel's workspace
 * buffers (partial results, step tables, staging) placed in the library's own scratch array of
 * AK_SCRATCH_BYTES on the current device instead of buffers the caller allocated. For each i < count, the
 * 8-byte pointer field at byte fields[i] of the argument struct is set to scratch + offsets[i], a buffer of
 * sizes[i] bytes (offsets 256-aligned, offsets[i] + sizes[i] <= AK_SCRATCH_BYTES, else an error and nothing
 * is launched). Inputs and outputs are still the caller's. The array is set up on a device's first call and
 * kept until the process ends; it keeps the last call's contents (nothing is cleared: the generated kernels
 * write every workspace byte they read). Every call on one device shares that device's array, so calls that
 * overlap in time on one device (two streams, two threads) race. Allocates nothing: no hipMalloc, hipFree
 * or allocating library routine. */
int ak_launch_scratch(ak_kernel* kernel, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t by,
                      uint32_t bz, uint32_t lds_bytes, const void* args, size_t args_size, const size_t* fields,
                      const uint64_t* offsets, const uint64_t* sizes, size_t count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TILEJAX_AK_H */
