/* C ABI of the HIP runtime shim used by hip_runtime (ctypes).
 *
 * The shim is the MI355X replacement for the CuPy objects the reference's CUDA
 * runtime drives from Python: cupy.RawKernel JIT + launch
 * (reference cuda_runtime/cuda_executor.py:38-51, 166-168), cupy.cuda.Device and
 * its synchronize() (cuda_runtime/cuda_backend.py:97-101, 148-150), and the
 * host<->device copies behind CUDABuffer.from_numpy/to_numpy
 * (cuda_runtime/cuda_backend.py:52-91). Device memory itself is allocated by
 * PyTorch-ROCm; the shim only receives raw device pointers and never frees them.
 *
 * Conventions: every entry point returns 0 on success or a hipError_t /
 * hiprtcResult value (hiprtc results offset by 10000) and never aborts; the text
 * of the last failure on the calling thread is available from hs_last_error().
 * Handles are opaque pointers. Nothing here is thread-safe per stream.
 */
#ifndef HIPSHIM_H
#define HIPSHIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One prebuilt kernel launch: function, grid, block, dynamic LDS and the packed
 * kernarg segment (the by-value argument struct). */
typedef struct hs_launch_rec {
  void* fn;
  uint32_t grid[3];
  uint32_t block[3];
  uint32_t lds_bytes;
  uint32_t kernarg_size;
  const void* kernarg;
} hs_launch_rec;

/* Select the device and create its primary context (replaces cp.cuda.Device(id)). */
int hs_init(int device);
int hs_device_count(int* count);
const char* hs_last_error(void);

/* Code objects (replace cupy.RawKernel's NVRTC module + function lookup). */
int hs_module_load(const void* image, size_t size, void** module);
int hs_module_unload(void* module);
int hs_module_function(void* module, const char* name, void** fn);

/* Runtime compilation of generated kernels with hiprtc (replaces NVRTC). The
 * returned image and log are malloc'd; release them with hs_free_host. */
int hs_rtc_compile(const char* source, const char* name, const char* arch, const char* include_dir,
                   void** image, size_t* image_size, char** log);
void hs_free_host(void* p);

/* Launches: one kernel, a prebuilt list replayed in one call, or a list captured
 * once into a HIP graph and relaunched (the reference's per-step Python dispatch
 * loop, cuda_executor.py:166-168, becomes one call per step). */
int hs_launch(void* fn, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t by, uint32_t bz,
              uint32_t lds_bytes, void* stream, const void* kernarg, size_t kernarg_size);
int hs_replay(const hs_launch_rec* recs, size_t n, void* stream);
int hs_graph_capture(const hs_launch_rec* recs, size_t n, void* stream, void** graph_exec);
int hs_graph_launch(void* graph_exec, void* stream);
int hs_graph_destroy(void* graph_exec);

/* Streams, events and copies. A NULL stream is the legacy default stream. */
int hs_stream_create(void** stream);
int hs_stream_destroy(void* stream);
int hs_stream_sync(void* stream);
int hs_device_sync(void);
int hs_event_create(void** event);
int hs_event_destroy(void* event);
int hs_event_record(void* event, void* stream);
int hs_event_sync(void* event);
int hs_event_elapsed_ms(void* start, void* stop, float* ms);
int hs_memcpy_htod(void* dst, const void* src, size_t n, void* stream);
int hs_memcpy_dtoh(void* dst, const void* src, size_t n, void* stream);
int hs_memcpy_dtod(void* dst, const void* src, size_t n, void* stream);

/* Device argmax of every row of a row-major [rows, cols] bf16 (dtype 2) or fp16 (dtype 1)
 * matrix, written as int64 to out[rows]: the largest value's first index (np.argmax's tie
 * rule), NaN above every number, -0.0 equal to +0.0. Replaces the host-side
 * np.argmax(logits[0, -1, :]) of the reference's generation loops (examples/run_qwen.py:125,180;
 * examples/run_qwen_graph.py:227) for callers that hold logits on the device.
 * x: 16-byte aligned; cols: a positive multiple of 8; rows <= 65535. workspace: device memory of
 * at least hs_argmax_workspace_bytes(rows, cols) bytes (8-byte aligned) for the per-segment keys;
 * its contents need no initialisation. Two launches on `stream`, nothing allocated. */
size_t hs_argmax_workspace_bytes(int64_t rows, int64_t cols);
int hs_argmax_rows(const void* x, int dtype, int64_t rows, int64_t cols, int64_t* out, void* workspace,
                   size_t workspace_bytes, void* stream);

/* hs_argmax_rows without a workspace argument and without any allocation: the per-segment keys go
 * to a 512 KiB device array inside the library, one per GPU, held until the process ends. No
 * counterpart in the reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Limit:
 * rows * ceil(cols / 8192) <= 65536 (e.g. 3449 rows of a 151936-entry vocabulary); larger calls
 * return hipErrorInvalidValue. Calls that overlap on one GPU share that array and race. */
int hs_argmax_rows_noalloc(const void* x, int dtype, int64_t rows, int64_t cols, int64_t* out, void* stream);

/* Device facts for launches that need every workgroup resident at once (the persistent decode
 * step): the current device's CU count, and how many workgroups of `fn` with `block` threads and
 * `dyn_lds` bytes of dynamic LDS fit on one CU. No counterpart in the reference, whose CUDA path
 * launches one kernel per IR op (cuda_runtime/cuda_executor.py:166-168) and never needs
 * co-residency; they stand beside cupy.cuda.Device (cuda_runtime/cuda_backend.py:97-101). */
int hs_device_cus(int* cus);
int hs_occupancy(void* fn, uint32_t block, size_t dyn_lds, int* blocks_per_cu);

/* `bytes` of zeroed, pinned, coherent host memory mapped into the device's address space: `host`
 * for the CPU, `device` for kernels. A kernel reports a failure into it (the persistent decode
 * step's timeout flag) and the host reads it without synchronising. Held until the process ends.
 * No counterpart in the reference, which raises from host-side checks only
 * (npu_runtime/dag_executor.py:319-323). */
int hs_host_alloc_mapped(size_t bytes, void** host, void** device);

/* sizeof() of the kernel argument struct with the given name (e.g. "LinearArgs"),
 * or 0 when unknown; lets the host check its ctypes mirrors. */
size_t hs_argsize(const char* struct_name);

#ifdef __cplusplus
}
#endif
#endif /* HIPSHIM_H */
