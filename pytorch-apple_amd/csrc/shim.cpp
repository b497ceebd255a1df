// HIP runtime shim: the C ABI declared in include/hipshim.h.
#include "../../include/hipshim.h"

#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "kernels/common.h"

namespace {

thread_local std::string g_err;

int fail_hip(hipError_t e, const char* what) {
  g_err = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  return (int)e;
}

#define HS_CHECK(call)                                  \
  do {                                                  \
    hipError_t e_ = (call);                             \
    if (e_ != hipSuccess) return fail_hip(e_, #call);   \
  } while (0)

// ---- device argmax over rows (hs_argmax_rows): the bodies are the code objects' k_argmax_part /
// k_argmax_finalize, compiled into this library so the entry point needs no module load
__global__ void __launch_bounds__(256) shim_argmax_part(const ArgmaxPartArgs a) {
  argmax_part_body(a, blockIdx.x, blockIdx.y);
}
__global__ void __launch_bounds__(256) shim_argmax_finalize(const ArgmaxFinalizeArgs a) {
  argmax_finalize_body(a, blockIdx.x);
}

constexpr int64_t kArgmaxSeg = 8192;    // columns per part (one workgroup)
constexpr int64_t kArgmaxMaxRows = 65535;

int64_t argmax_parts(int64_t cols) { return (cols + kArgmaxSeg - 1) / kArgmaxSeg; }

int fail_arg(const std::string& what) {
  g_err = what;
  return (int)hipErrorInvalidValue;
}

// Checks the operands of a row argmax; 0 when the call may launch.
int argmax_check(const void* x, int dtype, int64_t rows, int64_t cols, const int64_t* out) {
  if (rows < 0 || rows > kArgmaxMaxRows) return fail_arg("hs_argmax_rows: rows must be in [0, 65535]");
  if (rows == 0) return 0;
  if (!x || !out) return fail_arg("hs_argmax_rows: null x or out");
  if (dtype != HS_BF16 && dtype != HS_F16) return fail_arg("hs_argmax_rows: dtype must be bf16 (2) or fp16 (1)");
  if (cols < 8 || cols % 8 != 0 || cols > 0xFFFFFFFFll)
    return fail_arg("hs_argmax_rows: cols must be a positive multiple of 8 below 2^32");
  if (((uintptr_t)x) % 16 != 0) return fail_arg("hs_argmax_rows: x must be 16-byte aligned");
  return 0;
}

// Two launches on `s`: per-part keys into `slot` ([rows, parts] 64-bit keys), then one index per row.
int argmax_launch(const void* x, int dtype, int64_t rows, int64_t cols, int64_t* out, unsigned long long* slot,
                  hipStream_t s) {
  const int64_t parts = argmax_parts(cols);
  const int64_t seg = (cols + parts - 1) / parts + 7 & ~(int64_t)7;
  const ArgmaxPartArgs pa{x, slot, rows, cols, seg, dtype, (int)parts};
  hipLaunchKernelGGL(shim_argmax_part, dim3((unsigned)parts, (unsigned)rows), dim3(256), 0, s, pa);
  HS_CHECK(hipGetLastError());
  const ArgmaxFinalizeArgs fa{slot, out, rows, (int)parts, HS_I64};
  hipLaunchKernelGGL(shim_argmax_finalize, dim3((unsigned)rows), dim3(256), 0, s, fa);
  HS_CHECK(hipGetLastError());
  return 0;
}

// ---- hs_argmax_rows_noalloc: the per-segment keys live in a file-scope device array, one copy per
// GPU, so the entry point allocates nothing. Host code never passes `scratch` itself (in host code
// the name is only a stand-in for the symbol); each device's address comes from
// hipGetSymbolAddress with that device current, once, and is kept in g_scratch.
constexpr size_t kScratchKeys = 65536;   // 512 KiB per device: rows * ceil(cols / 8192) keys at most
static __device__ __align__(256) unsigned long long scratch[kScratchKeys];
constexpr int kMaxDevices = 64;
unsigned long long* g_scratch[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The current device's address of `scratch` (looked up on the first use on that device).
int scratch_current(unsigned long long** p) {
  int dev = 0;
  HS_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return fail_arg("no-alloc scratch: device index out of range");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    HS_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return fail_arg("hipGetSymbolAddress(scratch) returned null");
    g_scratch[dev] = (unsigned long long*)ptr;
  }
  *p = g_scratch[dev];
  return 0;
}

int launch_one(const hs_launch_rec& r, hipStream_t s) {
  size_t sz = r.kernarg_size;
  void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(r.kernarg), HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                 HIP_LAUNCH_PARAM_END};
  HS_CHECK(hipModuleLaunchKernel((hipFunction_t)r.fn, r.grid[0], r.grid[1], r.grid[2], r.block[0], r.block[1],
                                 r.block[2], r.lds_bytes, s, nullptr, cfg));
  return 0;
}

}  // namespace

extern "C" {

const char* hs_last_error(void) { return g_err.c_str(); }

int hs_device_count(int* count) {
  HS_CHECK(hipGetDeviceCount(count));
  return 0;
}

int hs_init(int device) {
  int n = 0;
  HS_CHECK(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) {
    g_err = "hs_init: device " + std::to_string(device) + " out of range (" + std::to_string(n) + " devices)";
    return (int)hipErrorInvalidDevice;
  }
  HS_CHECK(hipSetDevice(device));
  HS_CHECK(hipFree(nullptr));
  unsigned long long* p = nullptr;   // set up the device's no-alloc scratch address now
  return scratch_current(&p);
}

int hs_module_load(const void* image, size_t size, void** module) {
  (void)size;
  hipModule_t m = nullptr;
  HS_CHECK(hipModuleLoadData(&m, image));
  *module = m;
  return 0;
}

int hs_module_unload(void* module) {
  HS_CHECK(hipModuleUnload((hipModule_t)module));
  return 0;
}

int hs_module_function(void* module, const char* name, void** fn) {
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, (hipModule_t)module, name);
  if (e != hipSuccess) return fail_hip(e, (std::string("hipModuleGetFunction ") + name).c_str());
  *fn = f;
  return 0;
}

int hs_rtc_compile(const char* source, const char* name, const char* arch, const char* include_dir, void** image,
                   size_t* image_size, char** log) {
  *image = nullptr;
  *image_size = 0;
  if (log) *log = nullptr;
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, name, 0, nullptr, nullptr);
  if (r != HIPRTC_SUCCESS) {
    g_err = std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(r);
    return 10000 + (int)r;
  }
  std::string arch_opt = std::string("--offload-arch=") + (arch ? arch : "gfx950");
  std::string inc_opt = std::string("-I") + (include_dir ? include_dir : ".");
  std::vector<const char*> opts = {arch_opt.c_str(), inc_opt.c_str(), "-O3", "-std=c++17", "-mllvm",
                                   "-amdgpu-early-inline-all=true"};
  r = hiprtcCompileProgram(prog, (int)opts.size(), opts.data());
  size_t log_size = 0;
  hiprtcGetProgramLogSize(prog, &log_size);
  if (log && log_size > 1) {
    *log = (char*)malloc(log_size + 1);
    hiprtcGetProgramLog(prog, *log);
    (*log)[log_size] = 0;
  }
  if (r != HIPRTC_SUCCESS) {
    g_err = std::string("hiprtcCompileProgram: ") + hiprtcGetErrorString(r);
    hiprtcDestroyProgram(&prog);
    return 10000 + (int)r;
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  void* buf = malloc(n);
  hiprtcGetCode(prog, (char*)buf);
  hiprtcDestroyProgram(&prog);
  *image = buf;
  *image_size = n;
  return 0;
}

void hs_free_host(void* p) { free(p); }

int hs_launch(void* fn, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx, uint32_t by, uint32_t bz,
              uint32_t lds_bytes, void* stream, const void* kernarg, size_t kernarg_size) {
  hs_launch_rec r{fn, {gx, gy, gz}, {bx, by, bz}, lds_bytes, (uint32_t)kernarg_size, kernarg};
  return launch_one(r, (hipStream_t)stream);
}

int hs_replay(const hs_launch_rec* recs, size_t n, void* stream) {
  for (size_t i = 0; i < n; ++i) {
    int rc = launch_one(recs[i], (hipStream_t)stream);
    if (rc) {
      g_err = "launch " + std::to_string(i) + ": " + g_err;
      return rc;
    }
  }
  return 0;
}

int hs_graph_capture(const hs_launch_rec* recs, size_t n, void* stream, void** graph_exec) {
  hipStream_t s = (hipStream_t)stream;
  HS_CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int rc = 0;
  for (size_t i = 0; i < n && rc == 0; ++i) rc = launch_one(recs[i], s);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(s, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return fail_hip(e, "hipStreamEndCapture");
  hipGraphExec_t ex = nullptr;
  e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return fail_hip(e, "hipGraphInstantiate");
  *graph_exec = ex;
  return 0;
}

int hs_graph_launch(void* graph_exec, void* stream) {
  HS_CHECK(hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream));
  return 0;
}

int hs_graph_destroy(void* graph_exec) {
  HS_CHECK(hipGraphExecDestroy((hipGraphExec_t)graph_exec));
  return 0;
}

int hs_device_cus(int* cus) {
  int dev = 0;
  HS_CHECK(hipGetDevice(&dev));
  HS_CHECK(hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev));
  return 0;
}

int hs_occupancy(void* fn, uint32_t block, size_t dyn_lds, int* blocks_per_cu) {
  if (!fn || !blocks_per_cu) return fail_arg("hs_occupancy: null function or output");
  HS_CHECK(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, (hipFunction_t)fn, (int)block,
                                                              dyn_lds));
  return 0;
}

int hs_host_alloc_mapped(size_t bytes, void** host, void** device) {
  if (!host || !device || bytes == 0) return fail_arg("hs_host_alloc_mapped: null output or zero size");
  void* h = nullptr;
  HS_CHECK(hipHostMalloc(&h, bytes, hipHostMallocMapped | hipHostMallocCoherent));
  std::memset(h, 0, bytes);
  void* d = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&d, h, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(h);
    return fail_hip(e, "hipHostGetDevicePointer");
  }
  *host = h;
  *device = d;
  return 0;
}

int hs_stream_create(void** stream) {
  hipStream_t s;
  HS_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *stream = s;
  return 0;
}

int hs_stream_destroy(void* stream) {
  HS_CHECK(hipStreamDestroy((hipStream_t)stream));
  return 0;
}

int hs_stream_sync(void* stream) {
  HS_CHECK(hipStreamSynchronize((hipStream_t)stream));
  return 0;
}

int hs_device_sync(void) {
  HS_CHECK(hipDeviceSynchronize());
  return 0;
}

int hs_event_create(void** event) {
  hipEvent_t e;
  HS_CHECK(hipEventCreate(&e));
  *event = e;
  return 0;
}

int hs_event_destroy(void* event) {
  HS_CHECK(hipEventDestroy((hipEvent_t)event));
  return 0;
}

int hs_event_record(void* event, void* stream) {
  HS_CHECK(hipEventRecord((hipEvent_t)event, (hipStream_t)stream));
  return 0;
}

int hs_event_sync(void* event) {
  HS_CHECK(hipEventSynchronize((hipEvent_t)event));
  return 0;
}

int hs_event_elapsed_ms(void* start, void* stop, float* ms) {
  HS_CHECK(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return 0;
}

int hs_memcpy_htod(void* dst, const void* src, size_t n, void* stream) {
  HS_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, (hipStream_t)stream));
  return 0;
}

int hs_memcpy_dtoh(void* dst, const void* src, size_t n, void* stream) {
  HS_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, (hipStream_t)stream));
  HS_CHECK(hipStreamSynchronize((hipStream_t)stream));
  return 0;
}

int hs_memcpy_dtod(void* dst, const void* src, size_t n, void* stream) {
  HS_CHECK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, (hipStream_t)stream));
  return 0;
}

size_t hs_argmax_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return (size_t)rows * (size_t)argmax_parts(cols) * sizeof(unsigned long long);
}

int hs_argmax_rows(const void* x, int dtype, int64_t rows, int64_t cols, int64_t* out, void* workspace,
                   size_t workspace_bytes, void* stream) {
  if (int rc = argmax_check(x, dtype, rows, cols, out)) return rc;
  if (rows == 0) return 0;
  const size_t need = hs_argmax_workspace_bytes(rows, cols);
  if (!workspace || workspace_bytes < need)
    return fail_arg("hs_argmax_rows: workspace smaller than hs_argmax_workspace_bytes(rows, cols) = " +
                    std::to_string(need));
  if (((uintptr_t)workspace) % 8 != 0) return fail_arg("hs_argmax_rows: workspace must be 8-byte aligned");
  return argmax_launch(x, dtype, rows, cols, out, (unsigned long long*)workspace, (hipStream_t)stream);
}

int hs_argmax_rows_noalloc(const void* x, int dtype, int64_t rows, int64_t cols, int64_t* out, void* stream) {
  if (int rc = argmax_check(x, dtype, rows, cols, out)) return rc;
  if (rows == 0) return 0;
  const size_t keys = (size_t)rows * (size_t)argmax_parts(cols);
  if (keys > kScratchKeys)
    return fail_arg("hs_argmax_rows_noalloc: rows * ceil(cols / 8192) = " + std::to_string(keys) +
                    " exceeds the no-alloc scratch of " + std::to_string(kScratchKeys) + " keys");
  unsigned long long* slot = nullptr;
  if (int rc = scratch_current(&slot)) return rc;
  return argmax_launch(x, dtype, rows, cols, out, slot, (hipStream_t)stream);
}

size_t hs_argsize(const char* s) {
#define HS_SZ(T) \
  if (!strcmp(s, #T)) return sizeof(T);
  HS_SZ(CopyArgs)
  HS_SZ(FillArgs)
  HS_SZ(AdvanceArgs)
  HS_SZ(RMSNormArgs)
  HS_SZ(EmbeddingArgs)
  HS_SZ(RopeTableArgs)
  HS_SZ(IndexCopyArgs)
  HS_SZ(SoftmaxArgs)
  HS_SZ(ReduceLastArgs)
  HS_SZ(BmmArgs)
  HS_SZ(LinearArgs)
  HS_SZ(RopeCacheArgs)
  HS_SZ(PrefillAttnArgs)
  HS_SZ(MaskExtentArgs)
  HS_SZ(ReduceNormArgs)
  HS_SZ(ArgmaxPartArgs)
  HS_SZ(GemmArgs)
  HS_SZ(ConvArgs)
  HS_SZ(PoolArgs)
  HS_SZ(MeanNHWCArgs)
  HS_SZ(PermuteOHWIArgs)
  HS_SZ(PadNHWCArgs)
  HS_SZ(BatchNormArgs)
  HS_SZ(DecodeAttnArgs)
  HS_SZ(FusedArgs)
  HS_SZ(GemvArgs)
  HS_SZ(ArgmaxFinalizeArgs)
  HS_SZ(QKVArgs)
  HS_SZ(AttnOutArgs)
  HS_SZ(FlashArgs)
  HS_SZ(CombineArgs)
  HS_SZ(PersistArgs)
  HS_SZ(DecodeLayerPtrs)
#undef HS_SZ
  return 0;
}

}  // extern "C"
