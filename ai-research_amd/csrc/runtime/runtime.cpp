// runtime.cpp -- context, buffers, events, code-object loading and the
// kernel-level C ABI of include/gemma_hip.h.
//
// Replaces the reference's Vulkan plumbing (src/gpu/context.zig,
// buffer.zig, pipeline.zig, descriptors.zig, kernels.zig): one HIP device,
// one in-order stream, kernels from gfx950 code objects loaded with
// hipModuleLoad and launched with hipModuleLaunchKernel.
#include "runtime.hpp"

#include <dlfcn.h>
#include <string.h>

#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../common/quant_block.h"
#include "../common/synth.h"

namespace gh {

thread_local std::string g_last_error;

gh_status fail(gh_status st, const std::string& msg) {
  g_last_error = msg;
  return st;
}

gh_status hip_fail(hipError_t e, const char* what) {
  return fail(GH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

static std::string library_dir() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&library_dir), &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    size_t s = p.rfind('/');
    if (s != std::string::npos) return p.substr(0, s);
  }
  return ".";
}

// Code objects built by ai-research_amd/build.py next to libgemma_hip.so.
static const char* kCodeObjects[] = {"gh_gemv.hsaco", "gh_gemv_norm.hsaco", "gh_util.hsaco",
                                     "gh_attn.hsaco", "gh_norm.hsaco", "gh_prefill.hsaco"};

}  // namespace gh

using gh::fail;
using gh::hip_fail;

gh_status gh_context::load(const char* dir) {
  std::string base = dir ? std::string(dir) : gh::library_dir();
  for (const char* name : gh::kCodeObjects) {
    std::string path = base + "/" + name;
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) continue;  // a family not built yet simply contributes no kernels
    fclose(f);
    hipModule_t m;
    hipError_t e = hipModuleLoad(&m, path.c_str());
    if (e != hipSuccess)
      return fail(GH_ERR_CODE_OBJECT, "hipModuleLoad(" + path + "): " + hipGetErrorString(e));
    modules.push_back(m);
  }
  if (modules.empty()) return fail(GH_ERR_CODE_OBJECT, "no gfx950 code objects found in " + base);
  return GH_OK;
}

hipFunction_t gh_context::fn(const std::string& name) {
  std::lock_guard<std::mutex> lk(mu);
  auto it = fns.find(name);
  if (it != fns.end()) return it->second;
  for (hipModule_t m : modules) {
    hipFunction_t f;
    if (hipModuleGetFunction(&f, m, name.c_str()) == hipSuccess) {
      fns[name] = f;
      return f;
    }
  }
  return nullptr;
}

gh_status gh_context::launch(const std::string& name, dim3 grid, dim3 block, unsigned lds,
                             void** args) {
  hipFunction_t f = fn(name);
  if (!f) return fail(GH_ERR_CODE_OBJECT, "kernel not found in the code objects: " + name);
  hipError_t e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                       lds, stream, args, nullptr);
  if (e != hipSuccess) return hip_fail(e, ("launch " + name).c_str());
  return GH_OK;
}

int gh_context::occupancy(const std::string& name, int block, unsigned lds) {
  const std::string key = name + "/" + std::to_string(block) + "/" + std::to_string(lds);
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = occ.find(key);
    if (it != occ.end()) return it->second;
  }
  hipFunction_t f = fn(name);
  if (!f) return 0;
  int n = 0;
  if (hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, block, lds) != hipSuccess) n = 1;
  std::lock_guard<std::mutex> lk(mu);
  occ[key] = n;
  return n;
}

gh_status gh_context::ensure_zeroed(void** buf, size_t* have, size_t need) {
  if (*have >= need) return GH_OK;
  if (*buf) {
    hipStreamSynchronize(stream);
    hipFree(*buf);
    *buf = nullptr;
    *have = 0;
  }
  hipError_t e = hipMalloc(buf, need);
  if (e != hipSuccess) return fail(GH_ERR_ALLOC, std::string("scratch hipMalloc: ") + hipGetErrorString(e));
  uint64_t n = need / 4;
  void* args[] = {buf, nullptr, &n};
  uint32_t zero = 0;
  args[1] = &zero;
  gh_status st = launch("gh_fill_u32_k", dim3((unsigned)std::min<uint64_t>((n + 255) / 256, 4096)),
                        dim3(256), 0, args);
  if (st != GH_OK) return st;
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "scratch zero-fill");
  *have = need;
  return GH_OK;
}

gh_context::~gh_context() {
  if (stream) {
    hipStreamSynchronize(stream);
    if (attn_scratch) hipFree(attn_scratch);
    if (argmax_scratch) hipFree(argmax_scratch);
    if (gemm_scratch) hipFree(gemm_scratch);
    if (half_scratch) hipFree(half_scratch);
    hipStreamDestroy(stream);
  }
  for (hipModule_t m : modules) hipModuleUnload(m);
}

template <typename F>
static void host_parallel(size_t n, F f) {
  unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (n < 65536 || nt == 1) {
    f(0, n);
    return;
  }
  std::vector<std::thread> th;
  size_t chunk = (n + nt - 1) / nt;
  for (unsigned t = 0; t < nt; t++) {
    size_t a = (size_t)t * chunk;
    if (a >= n) break;
    th.emplace_back(f, a, std::min(n, a + chunk));
  }
  for (auto& t : th) t.join();
}


extern "C" {

const char* gh_last_error(void) { return gh::g_last_error.c_str(); }

int gh_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

gh_status gh_context_init(const char* code_object_dir, gh_context** out) {
  if (!out) return fail(GH_ERR_INVALID, "out is null");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return fail(GH_ERR_NO_DEVICE, "no HIP device visible");
  hipError_t e = hipSetDevice(0);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, 0);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(GH_ERR_NO_DEVICE, std::string("device is ") + prop.gcnArchName +
                                      ", this build targets gfx950 only");
  gh_context* ctx = new gh_context();
  ctx->device = 0;
  char dev_name[128] = {0};
  if (hipDeviceGetName(dev_name, sizeof(dev_name) - 1, 0) != hipSuccess || !dev_name[0])
    snprintf(dev_name, sizeof(dev_name), "%s", prop.name[0] ? prop.name : "AMD Instinct");
  snprintf(ctx->name, sizeof(ctx->name), "%s (%s, %d CUs)", dev_name, prop.gcnArchName,
           prop.multiProcessorCount);
  ctx->num_cus = prop.multiProcessorCount;
  ctx->max_lds = prop.sharedMemPerBlock;
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return hip_fail(e, "hipStreamCreate");
  }
  gh_status st = ctx->load(code_object_dir);
  if (st != GH_OK) {
    delete ctx;
    return st;
  }
  // the allocation-free entry point's scratch address on this device; a
  // failure is reported by that entry point, the rest of the library works
  gh::noalloc_setup(ctx->device);
  *out = ctx;
  return GH_OK;
}

void gh_context_deinit(gh_context* ctx) { delete ctx; }

const char* gh_context_device_name(const gh_context* ctx) { return ctx ? ctx->name : ""; }

gh_status gh_sync(gh_context* ctx) {
  if (!ctx) return fail(GH_ERR_INVALID, "ctx is null");
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  return GH_OK;
}

// ---- buffers ---------------------------------------------------------------
gh_status gh_buffer_alloc(gh_context* ctx, size_t bytes, void** dev) {
  if (!ctx || !dev || bytes == 0) return fail(GH_ERR_INVALID, "gh_buffer_alloc: bad argument");
  hipError_t e = hipMalloc(dev, bytes);
  if (e != hipSuccess) {
    *dev = nullptr;
    return fail(GH_ERR_ALLOC, std::string("hipMalloc: ") + hipGetErrorString(e));
  }
  return GH_OK;
}

gh_status gh_buffer_free(gh_context* ctx, void* dev) {
  if (!ctx) return fail(GH_ERR_INVALID, "ctx is null");
  if (!dev) return GH_OK;
  hipStreamSynchronize(ctx->stream);
  hipError_t e = hipFree(dev);
  if (e != hipSuccess) return hip_fail(e, "hipFree");
  return GH_OK;
}

gh_status gh_buffer_write(gh_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(GH_ERR_INVALID, "gh_buffer_write");
  if (!bytes) return GH_OK;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "gh_buffer_write");
  return GH_OK;
}

gh_status gh_buffer_read(gh_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(GH_ERR_INVALID, "gh_buffer_read");
  if (!bytes) return GH_OK;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "gh_buffer_read");
  return GH_OK;
}

gh_status gh_buffer_copy(gh_context* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return fail(GH_ERR_INVALID, "gh_buffer_copy");
  if (!bytes) return GH_OK;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "gh_buffer_copy");
  return GH_OK;
}

gh_status gh_buffer_fill_u32(gh_context* ctx, void* dev, uint32_t value, size_t count) {
  if (!ctx || (!dev && count)) return fail(GH_ERR_INVALID, "gh_buffer_fill_u32");
  if (!count) return GH_OK;
  uint64_t n = count;
  void* args[] = {&dev, &value, &n};
  unsigned grid = (unsigned)std::min<uint64_t>((n + 255) / 256, 4096);
  return ctx->launch("gh_fill_u32_k", dim3(grid), dim3(256), 0, args);
}

gh_status gh_read_probe(gh_context* ctx, const void* dev, size_t bytes, uint32_t per_lane,
                        uint32_t contiguous, uint32_t grid, float* sums) {
  if (!ctx || !dev || !sums) return fail(GH_ERR_INVALID, "gh_read_probe: null pointer");
  if (per_lane != 1 && per_lane != 2 && per_lane != 4 && per_lane != 8)
    return fail(GH_ERR_INVALID, "gh_read_probe: per_lane must be 1, 2, 4 or 8");
  if (contiguous > 1) return fail(GH_ERR_INVALID, "gh_read_probe: contiguous must be 0 or 1");
  if (grid == 0) grid = 4u * (uint32_t)ctx->num_cus;
  if (reinterpret_cast<uintptr_t>(dev) & 15)
    return fail(GH_ERR_INVALID, "gh_read_probe: buffer not 16-byte aligned");
  const uint64_t chunk = 16ull * 256 * per_lane * grid;  // bytes one round of the grid reads
  if (bytes == 0 || bytes % chunk != 0)
    return fail(GH_ERR_INVALID, "gh_read_probe: bytes must be a positive multiple of " +
                                    std::to_string(chunk) + " (16 B x 256 x per_lane x grid)");
  uint64_t n4 = bytes / 16;
  void* args[] = {&dev, &n4, &sums};
  const std::string name = "gh_read_probe_u" + std::to_string(per_lane) + "_c" +
                           std::to_string(contiguous) + "_k";
  return ctx->launch(name, dim3(grid), dim3(256), 0, args);
}

// ---- events ----------------------------------------------------------------
gh_status gh_event_create(gh_context* ctx, void** ev) {
  if (!ctx || !ev) return fail(GH_ERR_INVALID, "gh_event_create");
  hipEvent_t e;
  hipError_t r = hipEventCreate(&e);
  if (r != hipSuccess) return hip_fail(r, "hipEventCreate");
  *ev = e;
  return GH_OK;
}

gh_status gh_event_record(gh_context* ctx, void* ev) {
  if (!ctx || !ev) return fail(GH_ERR_INVALID, "gh_event_record");
  hipError_t r = hipEventRecord(static_cast<hipEvent_t>(ev), ctx->stream);
  if (r != hipSuccess) return hip_fail(r, "hipEventRecord");
  return GH_OK;
}

gh_status gh_event_elapsed_ms(void* a, void* b, float* ms) {
  if (!a || !b || !ms) return fail(GH_ERR_INVALID, "gh_event_elapsed_ms");
  hipError_t r = hipEventSynchronize(static_cast<hipEvent_t>(b));
  if (r == hipSuccess) r = hipEventElapsedTime(ms, static_cast<hipEvent_t>(a), static_cast<hipEvent_t>(b));
  if (r != hipSuccess) return hip_fail(r, "hipEventElapsedTime");
  return GH_OK;
}

gh_status gh_event_destroy(void* ev) {
  if (ev) hipEventDestroy(static_cast<hipEvent_t>(ev));
  return GH_OK;
}

// ---- graphs ------------------------------------------------------------------
struct gh_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

gh_status gh_graph_begin(gh_context* ctx) {
  if (!ctx) return fail(GH_ERR_INVALID, "gh_graph_begin: ctx is null");
  hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed);
  if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
  return GH_OK;
}

gh_status gh_graph_end(gh_context* ctx, void** out) {
  if (!ctx || !out) return fail(GH_ERR_INVALID, "gh_graph_end: null argument");
  *out = nullptr;
  gh_graph* g = new gh_graph();
  hipError_t e = hipStreamEndCapture(ctx->stream, &g->graph);
  if (e != hipSuccess) {
    delete g;
    return hip_fail(e, "hipStreamEndCapture");
  }
  e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    hipGraphDestroy(g->graph);
    delete g;
    return hip_fail(e, "hipGraphInstantiate");
  }
  *out = g;
  return GH_OK;
}

gh_status gh_graph_launch(gh_context* ctx, void* graph) {
  if (!ctx || !graph) return fail(GH_ERR_INVALID, "gh_graph_launch: null argument");
  hipError_t e = hipGraphLaunch(static_cast<gh_graph*>(graph)->exec, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
  return GH_OK;
}

gh_status gh_graph_destroy(void* graph) {
  gh_graph* g = static_cast<gh_graph*>(graph);
  if (!g) return GH_OK;
  if (g->exec) hipGraphExecDestroy(g->exec);
  if (g->graph) hipGraphDestroy(g->graph);
  delete g;
  return GH_OK;
}

// ---- quantization ------------------------------------------------------------
size_t gh_quantized_row_words(size_t cols, gh_quant_mode mode) {
  size_t nb = (cols + 31) / 32;
  if (mode == GH_QUANT_Q8) return nb * 9;
  if (mode == GH_QUANT_Q4) return nb * 5;
  return cols / 2;
}

size_t gh_quantized_size_bytes(size_t rows, size_t cols, gh_quant_mode mode) {
  return rows * gh_quantized_row_words(cols, mode) * 4;
}

gh_status gh_quantize_matrix(uint32_t* dst, const uint16_t* src, size_t rows, size_t cols,
                             gh_quant_mode mode, int nthreads) {
  if (mode != GH_QUANT_Q4 && mode != GH_QUANT_Q8)
    return fail(GH_ERR_INVALID, "gh_quantize_matrix: mode must be Q4 or Q8");
  if (rows == 0 || cols == 0) return GH_OK;  // quant.zig:93
  if (!dst || !src) return fail(GH_ERR_INVALID, "gh_quantize_matrix: null pointer");
  const size_t wpr = gh_quantized_row_words(cols, mode);
  const size_t nb = cols / 32;  // only floor(cols/32) blocks are written (quant.zig:21,56)
  auto work = [=](size_t r0, size_t r1) {
    for (size_t r = r0; r < r1; r++)
      for (size_t b = 0; b < nb; b++) {
        if (mode == GH_QUANT_Q4)
          gh_quantize_block_q4(src + r * cols + b * 32, dst + r * wpr + b * 5);
        else
          gh_quantize_block_q8(src + r * cols + b * 32, dst + r * wpr + b * 9);
      }
  };
  int nt = nthreads <= 0 ? 16 : nthreads;
  if (nt == 1 || rows < (size_t)nt * 4) {
    work(0, rows);
    return GH_OK;
  }
  std::vector<std::thread> th;
  size_t chunk = (rows + nt - 1) / nt;
  for (int t = 0; t < nt; t++) {
    size_t a = (size_t)t * chunk;
    if (a >= rows) break;
    th.emplace_back(work, a, std::min(rows, a + chunk));
  }
  for (auto& t : th) t.join();
  return GH_OK;
}

gh_status gh_quantize_matrix_dev(gh_context* ctx, void* dst, const void* src, size_t rows,
                                 size_t cols, gh_quant_mode mode) {
  if (!ctx || !dst || !src) return fail(GH_ERR_INVALID, "gh_quantize_matrix_dev: null");
  if (mode != GH_QUANT_Q4 && mode != GH_QUANT_Q8)
    return fail(GH_ERR_INVALID, "gh_quantize_matrix_dev: mode must be Q4 or Q8");
  if (cols % 32 != 0) return fail(GH_ERR_UNSUPPORTED, "gh_quantize_matrix_dev: cols % 32 != 0");
  if ((reinterpret_cast<uintptr_t>(src) & 15) || (reinterpret_cast<uintptr_t>(dst) & 3))
    return fail(GH_ERR_INVALID, "gh_quantize_matrix_dev: misaligned buffer");
  if (rows == 0 || cols == 0) return GH_OK;
  uint64_t r = rows;
  uint32_t c = (uint32_t)cols;
  void* args[] = {&dst, const_cast<void**>(&src), &r, &c};
  uint64_t blocks = rows * (cols / 32);
  unsigned grid = (unsigned)std::min<uint64_t>((blocks + 255) / 256, 65536);
  return ctx->launch(mode == GH_QUANT_Q4 ? "gh_quantize_q4_k" : "gh_quantize_q8_k", dim3(grid),
                     dim3(256), 0, args);
}

// ---- synthetic inputs --------------------------------------------------------
gh_status gh_synth_normal_f32(float* dst, size_t n, uint64_t seed, uint64_t stream, double mean,
                              double stddev, uint64_t offset) {
  if (!dst && n) return fail(GH_ERR_INVALID, "gh_synth_normal_f32: null");
  const uint64_t key = gh_stream_key(seed, stream);
  host_parallel(n, [=](size_t a, size_t b) {
    for (size_t i = a; i < b; i++) dst[i] = gh_normal_f32(key, offset + i, mean, stddev);
  });
  return GH_OK;
}

gh_status gh_synth_normal_bf16(uint16_t* dst, size_t n, uint64_t seed, uint64_t stream,
                               double mean, double stddev, uint64_t offset) {
  if (!dst && n) return fail(GH_ERR_INVALID, "gh_synth_normal_bf16: null");
  const uint64_t key = gh_stream_key(seed, stream);
  host_parallel(n, [=](size_t a, size_t b) {
    for (size_t i = a; i < b; i++) dst[i] = gh_bf16_rne(gh_normal_f32(key, offset + i, mean, stddev));
  });
  return GH_OK;
}

static gh_status synth_dev(gh_context* ctx, const char* kname, void* dst, size_t n, uint64_t seed,
                           uint64_t stream, double mean, double stddev, uint64_t offset) {
  if (!ctx || (!dst && n)) return fail(GH_ERR_INVALID, "synth: null");
  if (!n) return GH_OK;
  uint64_t key = gh_stream_key(seed, stream), nn = n;
  void* args[] = {&dst, &nn, &key, &mean, &stddev, &offset};
  unsigned grid = (unsigned)std::min<uint64_t>((n / 8 + 255) / 256 + 1, (uint64_t)ctx->num_cus * 16);
  return ctx->launch(kname, dim3(grid), dim3(256), 0, args);
}

gh_status gh_synth_normal_f32_dev(gh_context* ctx, float* dst, size_t n, uint64_t seed,
                                  uint64_t stream, double mean, double stddev, uint64_t offset) {
  return synth_dev(ctx, "gh_synth_normal_f32_k", dst, n, seed, stream, mean, stddev, offset);
}

gh_status gh_synth_normal_bf16_dev(gh_context* ctx, uint16_t* dst, size_t n, uint64_t seed,
                                   uint64_t stream, double mean, double stddev, uint64_t offset) {
  return synth_dev(ctx, "gh_synth_normal_bf16_k", dst, n, seed, stream, mean, stddev, offset);
}

gh_status gh_synth_uniform_u32(uint32_t* dst, size_t n, uint64_t seed, uint64_t stream,
                               uint32_t bound) {
  if ((!dst && n) || bound == 0) return fail(GH_ERR_INVALID, "gh_synth_uniform_u32");
  const uint64_t key = gh_stream_key(seed, stream);
  for (size_t i = 0; i < n; i++) dst[i] = gh_uniform_u32(key, i, bound);
  return GH_OK;
}

}  // extern "C"
