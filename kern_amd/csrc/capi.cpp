// Host side of the C ABI (include/kern_amd.h): module layer over the HIP runtime, and the op layer
// that validates shapes and launches the gfx950 entries of kern_mx.hsaco through it.
#include "../../include/kern_amd.h"

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "elf_meta.h"
#include "sha256.h"

#ifndef KERN_MX_SHA256
#error "KERN_MX_SHA256 must name the sha256 of kern_mx.hsaco"
#endif

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[4096];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(KERN_ERR_HIP, "hip: %s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define HIP_TRY(call, what)              \
  do {                                   \
    hipError_t e_ = (call);              \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

}  // namespace

// the same thread-local message, for the other host source files of the library
int kern_amd_fail(int code, const char* fmt, ...) {
  char buf[4096];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

struct kern_module_s {
  hipModule_t mod = nullptr;
  int device = -1;
  std::map<std::string, std::vector<uint32_t>> params;   // entry -> explicit arg sizes (code object metadata)
  std::map<std::string, std::vector<uint32_t>> offsets;  // entry -> their kernarg byte offsets
};

struct kern_function_s {
  hipFunction_t fn = nullptr;
  std::string entry;
  std::vector<uint32_t> params;
  std::vector<uint32_t> offsets;
};

struct kern_graph_s {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

extern "C" const char* kern_last_error(void) { return g_err.c_str(); }

extern "C" int kern_sha256_hex(const void* data, size_t len, char out[65]) {
  if (!data && len) return fail(KERN_ERR_API, "kern_sha256_hex: null data");
  kern::sha256_hex(static_cast<const uint8_t*>(data), len, out);
  return KERN_OK;
}

extern "C" int kern_module_load(const void* image, size_t len, const char* sha256_hex, kern_module* out) {
  if (!image || !len || !out) return fail(KERN_ERR_API, "kern_module_load: null image or output");
  if (sha256_hex) {
    char got[65];
    kern::sha256_hex(static_cast<const uint8_t*>(image), len, got);
    if (strncmp(got, sha256_hex, 64) != 0 || strlen(sha256_hex) != 64)
      return fail(KERN_ERR_KERNEL_ARTIFACT, "code object sha256 mismatch: expected %s, got %s", sha256_hex, got);
  }
  std::unique_ptr<kern_module_s> m(new kern_module_s);
  std::string perr;
  if (!kern::read_kernel_params(static_cast<const uint8_t*>(image), len, m->params, perr, &m->offsets))
    return fail(KERN_ERR_KERNEL_ARTIFACT, "code object metadata: %s", perr.c_str());
  HIP_TRY(hipGetDevice(&m->device), "hipGetDevice");
  HIP_TRY(hipModuleLoadData(&m->mod, image), "hipModuleLoadData");
  *out = m.release();
  return KERN_OK;
}

extern "C" int kern_module_unload(kern_module mod) {
  if (!mod) return KERN_OK;
  hipError_t e = hipModuleUnload(mod->mod);
  delete mod;
  if (e != hipSuccess) return hip_fail(e, "hipModuleUnload");
  return KERN_OK;
}

extern "C" int kern_module_function(kern_module mod, const char* entry, kern_function* out) {
  if (!mod || !entry || !out) return fail(KERN_ERR_API, "kern_module_function: null argument");
  auto it = mod->params.find(entry);
  if (it == mod->params.end()) return fail(KERN_ERR_KERNEL_ARTIFACT, "entry %s not in the code object", entry);
  std::unique_ptr<kern_function_s> f(new kern_function_s);
  HIP_TRY(hipModuleGetFunction(&f->fn, mod->mod, entry), "hipModuleGetFunction");
  f->entry = entry;
  f->params = it->second;
  f->offsets = mod->offsets[entry];
  *out = f.release();
  return KERN_OK;
}

extern "C" int kern_function_release(kern_function fn) {
  delete fn;  // the hipFunction_t belongs to its module
  return KERN_OK;
}

extern "C" int kern_function_param_sizes(kern_function fn, uint32_t* sizes, int cap, int* n) {
  if (!fn || !n) return fail(KERN_ERR_API, "kern_function_param_sizes: null argument");
  *n = (int)fn->params.size();
  for (int i = 0; i < cap && i < *n; ++i) sizes[i] = fn->params[i];
  return KERN_OK;
}

extern "C" int kern_function_param_offsets(kern_function fn, uint32_t* offsets, int cap, int* n) {
  if (!fn || !n) return fail(KERN_ERR_API, "kern_function_param_offsets: null argument");
  *n = (int)fn->offsets.size();
  for (int i = 0; i < cap && i < *n; ++i) offsets[i] = fn->offsets[i];
  return KERN_OK;
}

extern "C" int kern_code_object_param_sizes(const void* image, size_t len, const char* entry, uint32_t* sizes,
                                            int cap, int* n) {
  if (!image || !entry || !n) return fail(KERN_ERR_API, "kern_code_object_param_sizes: null argument");
  std::map<std::string, std::vector<uint32_t>> params;
  std::string perr;
  if (!kern::read_kernel_params(static_cast<const uint8_t*>(image), len, params, perr))
    return fail(KERN_ERR_KERNEL_ARTIFACT, "code object metadata: %s", perr.c_str());
  auto it = params.find(entry);
  if (it == params.end()) return fail(KERN_ERR_KERNEL_ARTIFACT, "entry %s not in the code object", entry);
  *n = (int)it->second.size();
  for (int i = 0; i < cap && i < *n; ++i) sizes[i] = it->second[i];
  return KERN_OK;
}

extern "C" int kern_function_check_params(kern_function fn, const uint32_t* sizes, int n) {
  if (!fn || (n && !sizes)) return fail(KERN_ERR_API, "kern_function_check_params: null argument");
  std::string want, got;
  for (int i = 0; i < n; ++i) want += (i ? "," : "") + std::to_string(sizes[i]);
  for (size_t i = 0; i < fn->params.size(); ++i) got += (i ? "," : "") + std::to_string(fn->params[i]);
  if ((int)fn->params.size() != n || want != got)
    return fail(KERN_ERR_KERNEL_ARTIFACT, "entry %s: launch declares param sizes [%s], code object has [%s]",
                fn->entry.c_str(), want.c_str(), got.c_str());
  return KERN_OK;
}

extern "C" int kern_launch(kern_function fn, const uint32_t grid[3], const uint32_t block[3], uint32_t shared_bytes,
                           void* stream, const void* kernargs, size_t kernargs_size) {
  if (!fn || !grid || !block) return fail(KERN_ERR_API, "kern_launch: null argument");
  if (grid[0] == 0 || grid[1] == 0 || grid[2] == 0) return KERN_OK;  // nothing to run
  if (block[0] * block[1] * block[2] > 1024)
    return fail(KERN_ERR_API, "kern_launch %s: block %ux%ux%u exceeds 1024 threads", fn->entry.c_str(), block[0],
                block[1], block[2]);
  size_t sz = kernargs_size;
  void* cfg[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void*>(kernargs), HIP_LAUNCH_PARAM_BUFFER_SIZE, &sz,
                 HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(fn->fn, grid[0], grid[1], grid[2], block[0], block[1], block[2], shared_bytes,
                                       static_cast<hipStream_t>(stream), nullptr, cfg);
  if (e != hipSuccess) return fail(KERN_ERR_HIP, "launch %s: %s", fn->entry.c_str(), hipGetErrorString(e));
  return KERN_OK;
}

static std::mutex g_capture_mu;  // graph capture is serialised process-wide (exec.rs:435-440)

extern "C" int kern_graph_begin(void* stream) {
  if (!stream) return fail(KERN_ERR_API, "kern_graph_begin: capture needs a non-null stream");
  g_capture_mu.lock();
  hipError_t e = hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) {
    g_capture_mu.unlock();
    return hip_fail(e, "hipStreamBeginCapture");
  }
  return KERN_OK;
}

extern "C" int kern_graph_end(void* stream, kern_graph* out) {
  if (!stream || !out) return fail(KERN_ERR_API, "kern_graph_end: null argument");
  std::unique_ptr<kern_graph_s> g(new kern_graph_s);
  hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g->graph);
  g_capture_mu.unlock();
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g->graph);
    return hip_fail(e, "hipGraphInstantiate");
  }
  *out = g.release();
  return KERN_OK;
}

extern "C" int kern_graph_launch(kern_graph g, void* stream) {
  if (!g) return fail(KERN_ERR_API, "kern_graph_launch: null graph");
  HIP_TRY(hipGraphLaunch(g->exec, static_cast<hipStream_t>(stream)), "hipGraphLaunch");
  return KERN_OK;
}

extern "C" int kern_graph_destroy(kern_graph g) {
  if (!g) return KERN_OK;
  if (g->exec) (void)hipGraphExecDestroy(g->exec);
  if (g->graph) (void)hipGraphDestroy(g->graph);
  delete g;
  return KERN_OK;
}

// ============================================================================ op layer

namespace {

std::mutex g_mu;
std::string g_path;
std::map<int, kern_module> g_mods;  // device -> module of kern_mx.hsaco
std::map<int, std::map<std::string, kern_function>> g_fns;

std::string default_path() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&kern_init), &info) && info.dli_fname) {
    std::string p = info.dli_fname;
    size_t slash = p.rfind('/');
    return (slash == std::string::npos ? std::string(".") : p.substr(0, slash)) + "/kern_mx.hsaco";
  }
  return "kern_mx.hsaco";
}

// module of the current device, loaded and pinned on first use
int module_for_device(kern_module* out) {
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_mods.find(dev);
  if (it != g_mods.end()) {
    *out = it->second;
    return KERN_OK;
  }
  if (g_path.empty()) g_path = default_path();
  std::ifstream f(g_path, std::ios::binary);
  if (!f) return fail(KERN_ERR_KERNEL_ARTIFACT, "cannot read code object %s", g_path.c_str());
  std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  kern_module m = nullptr;
  int rc = kern_module_load(bytes.data(), bytes.size(), KERN_MX_SHA256, &m);
  if (rc) return fail(rc, "%s (%s)", kern_last_error(), g_path.c_str());
  g_mods[dev] = m;
  *out = m;
  return KERN_OK;
}

int function(const char* entry, kern_function* out) {
  kern_module m = nullptr;
  if (int rc = module_for_device(&m)) return rc;
  int dev = m->device;
  std::lock_guard<std::mutex> lk(g_mu);
  auto& fns = g_fns[dev];
  auto it = fns.find(entry);
  if (it != fns.end()) {
    *out = it->second;
    return KERN_OK;
  }
  kern_function f = nullptr;
  if (int rc = kern_module_function(m, entry, &f)) return rc;
  fns[entry] = f;
  *out = f;
  return KERN_OK;
}

// AMDGPU kernarg packing: every argument at its natural alignment
struct Args {
  alignas(16) unsigned char buf[512];
  size_t n = 0;
  std::vector<uint32_t> sizes;
  template <class T>
  void put(T v) {
    n = (n + alignof(T) - 1) & ~(alignof(T) - 1);
    memcpy(buf + n, &v, sizeof(T));
    n += sizeof(T);
    sizes.push_back((uint32_t)sizeof(T));
  }
};

// threads of one GEMM workgroup (8 waves)
constexpr uint32_t kBmmThreads = 512;
// the MoE GEMMs are persistent: one workgroup per CU (MI355X: 256), looping over the live slots' tiles
constexpr uint32_t kMoeWorkgroups = 256;

int launch(const char* entry, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t block, void* stream, Args& a,
           uint32_t shared_bytes = 0) {
  kern_function f = nullptr;
  if (int rc = function(entry, &f)) return rc;
  if (int rc = kern_function_check_params(f, a.sizes.data(), (int)a.sizes.size())) return rc;
  const uint32_t grid[3] = {gx, gy, gz}, blk[3] = {block, 1, 1};
  return kern_launch(f, grid, blk, shared_bytes, stream, a.buf, (a.n + 7) & ~size_t(7));
}

// moe_routing: one workgroup below kRouteChunkedMin expanded indices, else the chunked three launches over
// min(kRouteMaxChunks, ceil(n / kRouteChunk)) workgroups (constants shared with kern_mx.hip's routing)
constexpr int64_t kRouteChunkedMin = 16384, kRouteChunk = 4096, kRouteMaxChunks = 64;

#define REQUIRE(cond, ...) \
  do {                     \
    if (!(cond)) return fail(KERN_ERR_API, __VA_ARGS__); \
  } while (0)

}  // namespace

extern "C" int kern_init(const char* code_object_path) {
  {
    std::lock_guard<std::mutex> lk(g_mu);
    g_path = code_object_path ? code_object_path : default_path();
  }
  kern_module m = nullptr;
  return module_for_device(&m);
}

extern "C" const char* kern_code_object_sha256(void) { return KERN_MX_SHA256; }

extern "C" int kern_mx_module(kern_module* out) {
  if (!out) return fail(KERN_ERR_API, "kern_mx_module: null output");
  return module_for_device(out);
}

extern "C" int kern_moe_quant(const void* x, void* q, void* sf, int32_t tokens, int32_t K, void* stream) {
  REQUIRE(tokens >= 0 && K > 0 && K % 32 == 0, "moe_quant: need K %% 32 == 0 and tokens >= 0 (K=%d tokens=%d)", K,
          tokens);
  if (tokens == 0) return KERN_OK;
  REQUIRE(x && q && sf, "moe_quant: null buffer");
  const int64_t chunks = (int64_t)tokens * (K / 8);  // 8-element chunks; a workgroup takes 512 (16 elements a lane)
  REQUIRE((chunks + 511) / 512 < (int64_t)1 << 31, "moe_quant: %lld elements exceed the grid",
          (long long)chunks * 8);
  Args a;
  a.put(x), a.put(q), a.put(sf), a.put(tokens), a.put(K);
  return launch("kern_mx_quant_bf16", (uint32_t)((chunks + 511) / 512), 1, 1, 256, stream, a);
}

extern "C" int kern_mxfp8_quant_f32(const float* x, void* q, void* sf, int32_t tokens, int32_t K, void* stream) {
  REQUIRE(tokens >= 0 && K > 0 && K % 32 == 0, "mxfp8_quant_f32: need K %% 32 == 0 and tokens >= 0 (K=%d tokens=%d)",
          K, tokens);
  if (tokens == 0) return KERN_OK;
  REQUIRE(x && q && sf, "mxfp8_quant_f32: null buffer");
  const int64_t pieces = (int64_t)tokens * (K / 8);  // 8-element pieces, one a lane
  REQUIRE((pieces + 255) / 256 < (int64_t)1 << 31, "mxfp8_quant_f32: %lld elements exceed the grid",
          (long long)pieces * 8);
  Args a;
  a.put(x), a.put(q), a.put(sf), a.put(tokens), a.put(K);
  return launch("kern_mx_quant_f32", (uint32_t)((pieces + 255) / 256), 1, 1, 256, stream, a);
}

extern "C" int kern_moe_w_shuffle(const void* raw, void* out, int32_t experts, int32_t rows, int32_t row_bytes,
                                  int32_t gated, void* stream) {
  REQUIRE(experts > 0 && rows > 0 && rows % 16 == 0 && row_bytes > 0 && row_bytes % 256 == 0,
          "k3_moe_w_shuffle: need rows %% 16 == 0 and row_bytes %% 256 == 0 (rows=%d row_bytes=%d)", rows, row_bytes);
  REQUIRE(gated == 0 || gated == 1, "k3_moe_w_shuffle: gated must be 0 or 1 (got %d)", gated);
  REQUIRE(raw && out && raw != out, "k3_moe_w_shuffle: null or aliased buffers");
  const int64_t slots = (int64_t)experts * rows * row_bytes / 16;
  Args a;
  a.put(raw), a.put(out), a.put(experts), a.put(rows), a.put(row_bytes), a.put(gated);
  return launch("kern_mx_w_shuffle", (uint32_t)((slots + 255) / 256), 1, 1, 256, stream, a);
}

extern "C" int kern_moe_sf_shuffle(const void* raw, void* out, int32_t experts, int32_t rows, int32_t sf_cols,
                                   int32_t gated, void* stream) {
  REQUIRE(experts > 0 && rows > 0 && rows % 16 == 0 && sf_cols > 0 && sf_cols % 16 == 0,
          "k3_moe_sf_shuffle: need rows %% 16 == 0 and sf_cols %% 16 == 0 (rows=%d sf_cols=%d)", rows, sf_cols);
  REQUIRE(gated == 0 || gated == 1, "k3_moe_sf_shuffle: gated must be 0 or 1 (got %d)", gated);
  REQUIRE(raw && out && raw != out, "k3_moe_sf_shuffle: null or aliased buffers");
  const int64_t dwords = (int64_t)experts * rows * sf_cols / 4;
  Args a;
  a.put(raw), a.put(out), a.put(experts), a.put(rows), a.put(sf_cols), a.put(gated);
  return launch("kern_mx_sf_shuffle", (uint32_t)((dwords + 255) / 256), 1, 1, 256, stream, a);
}

extern "C" int kern_moe_routing(const int32_t* topk_idx, int32_t* counts, int32_t* cta_batch, int32_t* cta_limit,
                                int32_t* num_non_exiting, int32_t* total_padded, int32_t* route_map,
                                int32_t* exp2perm, int32_t tokens, int32_t topk, int32_t local_start,
                                int32_t local_experts, void* stream) {
  REQUIRE(tokens >= 0 && topk > 0 && local_experts > 0 && local_experts <= 512 && local_start >= 0,
          "moe_routing: need tokens >= 0, topk > 0, 0 < local_experts <= 512 (got %d, %d, %d)", tokens, topk,
          local_experts);
  // the tables are written at every token count (zero live slots for an empty batch); the ids and exp2perm
  // are empty at zero tokens and may then be null
  REQUIRE(counts && cta_batch && cta_limit && num_non_exiting && total_padded && route_map, "moe_routing: null buffer");
  REQUIRE(tokens == 0 || (topk_idx && exp2perm), "moe_routing: null buffer");
  // expanded ids and padded rows (at most tokens * topk + 128 * local_experts) are i32 in the tables
  const int64_t n = (int64_t)tokens * topk;
  REQUIRE(n + 128LL * local_experts <= INT32_MAX,
          "moe_routing: tokens * topk = %lld leaves the padded rows past the i32 tables", (long long)n);
  Args a;
  a.put(topk_idx), a.put(counts), a.put(cta_batch), a.put(cta_limit), a.put(num_non_exiting), a.put(total_padded);
  a.put(route_map), a.put(exp2perm), a.put(tokens), a.put(topk), a.put(local_start), a.put(local_experts);
  if (n < kRouteChunkedMin) return launch("kern_mx_routing", 1, 1, 1, 1024, stream, a);
  // count, scan and rank over G chunks of the expanded indices (the kernels derive G from n the same way)
  const uint32_t G = (uint32_t)std::min<int64_t>(kRouteMaxChunks, (n + kRouteChunk - 1) / kRouteChunk);
  if (int rc = launch("kern_mx_routing_count", G, 1, 1, 1024, stream, a)) return rc;
  if (int rc = launch("kern_mx_routing_scan", 1, 1, 1, 1024, stream, a)) return rc;
  return launch("kern_mx_routing_rank", G, 1, 1, 1024, stream, a);
}

extern "C" int kern_moe_quant_routing(const void* x, void* q, void* sf, int32_t tokens, int32_t K,
                                      const int32_t* topk_idx, int32_t* counts, int32_t* cta_batch,
                                      int32_t* cta_limit, int32_t* num_non_exiting, int32_t* total_padded,
                                      int32_t* route_map, int32_t* exp2perm, int32_t topk, int32_t local_start,
                                      int32_t local_experts, void* stream) {
  REQUIRE(tokens >= 0 && K > 0 && K % 32 == 0, "moe_quant_routing: need K %% 32 == 0 and tokens >= 0 (K=%d tokens=%d)",
          K, tokens);
  REQUIRE(topk > 0 && local_experts > 0 && local_experts <= 512 && local_start >= 0,
          "moe_quant_routing: need topk > 0, 0 < local_experts <= 512 (got %d, %d)", topk, local_experts);
  REQUIRE(counts && cta_batch && cta_limit && num_non_exiting && total_padded && route_map,
          "moe_quant_routing: null buffer");
  REQUIRE(tokens == 0 || (x && q && sf && topk_idx && exp2perm), "moe_quant_routing: null buffer");
  // quantizer workgroups of 1024 lanes (16 elements a lane); the routing block's LDS holds every workgroup
  // of the launch to one per CU, so the fused launch is taken when all of them fit in one round
  const int64_t qwg = ((int64_t)tokens * (K / 16) + 1023) / 1024;
  if (qwg > 255) {
    const int rc = kern_moe_routing(topk_idx, counts, cta_batch, cta_limit, num_non_exiting, total_padded, route_map,
                                    exp2perm, tokens, topk, local_start, local_experts, stream);
    if (rc != KERN_OK) return rc;
    return kern_moe_quant(x, q, sf, tokens, K, stream);
  }
  Args a;
  a.put(x), a.put(q), a.put(sf), a.put(K), a.put(topk_idx), a.put(counts), a.put(cta_batch), a.put(cta_limit);
  a.put(num_non_exiting), a.put(total_padded), a.put(route_map), a.put(exp2perm), a.put(tokens), a.put(topk);
  a.put(local_start), a.put(local_experts);
  return launch("kern_mx_quant_routing", (uint32_t)(1 + qwg), 1, 1, 1024, stream, a);
}

extern "C" int kern_trtllm_bmm_bf16_mxe2m1_mxe4m3(const void* a_, const void* sf_a, const void* b, const void* sf_b,
                                                  void* c, const int32_t* num_non_exiting,
                                                  const int32_t* total_padded, const int32_t* cta_batch,
                                                  const int32_t* cta_limit, int32_t m, int32_t k, int32_t ctas,
                                                  int32_t sf_b_r128c4, float* dbg, void* stream) {
  REQUIRE(m > 0 && m % 256 == 0 && m <= 131072 && k > 0 && k % 512 == 0 && ctas >= 0 && ctas < 65536,
          "trtllm_bmm_bf16_mxe2m1_mxe4m3: need m %% 256 == 0, m <= 131072, k %% 512 == 0, 0 <= ctas < 65536 (m=%d k=%d ctas=%d)",
          m, k, ctas);
  REQUIRE(a_ && sf_a && b && sf_b && c && num_non_exiting && total_padded && cta_batch && cta_limit,
          "trtllm_bmm_bf16_mxe2m1_mxe4m3: null buffer");
  // the ring addresses the activations by 32-bit byte offsets from the buffer's base
  REQUIRE((int64_t)ctas * 128 * k < ((int64_t)1 << 32),
          "trtllm_bmm_bf16_mxe2m1_mxe4m3: activations of ctas * 128 rows x k bytes must stay below 4 GiB (ctas=%d k=%d)",
          ctas, k);
  if (ctas == 0) return KERN_OK;
  Args a;
  a.put(a_), a.put(sf_a), a.put(b), a.put(sf_b), a.put((void*)c), a.put(num_non_exiting), a.put(total_padded);
  a.put(cta_batch), a.put(cta_limit), a.put(m), a.put(k), a.put(ctas), a.put(sf_b_r128c4 ? 1 : 0), a.put(dbg);
  return launch("kern_mx_bmm_fc2", kMoeWorkgroups, 1, 1, kBmmThreads, stream, a);
}

extern "C" int kern_trtllm_bmm_mxe4m3_mxe2m1_mxe4m3(const void* a_, const void* sf_a, const void* b,
                                                    const void* sf_b, void* c, void* sf_c, const int32_t* route_map,
                                                    const float* alpha, const float* beta,
                                                    const int32_t* num_non_exiting, const int32_t* total_padded,
                                                    const int32_t* cta_batch, const int32_t* cta_limit, int32_t m,
                                                    int32_t k, int32_t ctas, float* dbg, void* stream) {
  REQUIRE(m > 0 && m % 256 == 0 && m <= 131072 && k > 0 && k % 512 == 0 && ctas >= 0 && ctas < 65536,
          "trtllm_bmm_mxe4m3_mxe2m1_mxe4m3: need m %% 256 == 0, m <= 131072, k %% 512 == 0, 0 <= ctas < 65536 (m=%d k=%d ctas=%d)",
          m, k, ctas);
  REQUIRE(a_ && sf_a && b && sf_b && c && sf_c && route_map && alpha && beta && num_non_exiting && total_padded &&
              cta_batch && cta_limit,
          "trtllm_bmm_mxe4m3_mxe2m1_mxe4m3: null buffer");
  if (ctas == 0) return KERN_OK;
  Args a;
  a.put(a_), a.put(sf_a), a.put(b), a.put(sf_b), a.put(c), a.put(sf_c), a.put(route_map), a.put(alpha), a.put(beta);
  a.put(num_non_exiting), a.put(total_padded), a.put(cta_batch), a.put(cta_limit), a.put(m), a.put(k), a.put(ctas);
  a.put(dbg);
  return launch("kern_mx_bmm_fc1", kMoeWorkgroups, 1, 1, kBmmThreads, stream, a);
}

extern "C" int kern_mxfp4_gemm_e4m3(const void* a_, const void* sf_a, const void* b, const void* sf_b, void* c,
                                    const float* d_scale, int32_t M, int32_t m, int32_t k, float* dbg, void* stream) {
  REQUIRE(M >= 0 && m > 0 && m % 256 == 0 && k > 0 && k % 512 == 0,
          "mxfp4_gemm_e4m3: need m %% 256 == 0, k %% 512 == 0 (M=%d m=%d k=%d)", M, m, k);
  REQUIRE(a_ && sf_a && b && sf_b && c && d_scale, "mxfp4_gemm_e4m3: null buffer");
  REQUIRE((int64_t)M * k < ((int64_t)1 << 32), "mxfp4_gemm_e4m3: activations [M, k] must stay below 4 GiB (M=%d k=%d)",
          M, k);
  if (M == 0) return KERN_OK;
  Args a;
  a.put(a_), a.put(sf_a), a.put(b), a.put(sf_b), a.put(c), a.put(d_scale), a.put(M), a.put(m), a.put(k), a.put(dbg);
  return launch("kern_mx_gemm_e4m3", (uint32_t)(m / 256), (uint32_t)((M + 127) / 128), 1, kBmmThreads, stream, a);
}

extern "C" int kern_mxfp4_gemm_bf16(const void* a_, const void* sf_a, const void* b, const void* sf_b, void* c,
                                    int32_t M, int32_t m, int32_t k, float* dbg, void* stream) {
  REQUIRE(M >= 0 && m > 0 && m % 256 == 0 && k > 0 && k % 512 == 0,
          "mxfp4_gemm_bf16: need m %% 256 == 0, k %% 512 == 0 (M=%d m=%d k=%d)", M, m, k);
  REQUIRE(a_ && sf_a && b && sf_b && c, "mxfp4_gemm_bf16: null buffer");
  REQUIRE((int64_t)M * k < ((int64_t)1 << 32), "mxfp4_gemm_bf16: activations [M, k] must stay below 4 GiB (M=%d k=%d)",
          M, k);
  if (M == 0) return KERN_OK;
  // M <= 64 tokens with K = 1024 * {1, 2, 4, 7, 8}: the persistent walk over the weights, about 256
  // workgroups of 8 waves with hb <= 9 half groups of 8 weight rows each (the tiled grid has one workgroup
  // per 256 weight rows, 36 at N = 9216). Config 5 at M = 64: 17.0 against 24.9 us (N = 9216, K = 7168),
  // 16.3 against 27.8 (N = 7168, K = 8192).
  static const char* const skinny[9] = {nullptr, "kern_mx_gemm_bf16_s1", "kern_mx_gemm_bf16_s2", nullptr,
                                        "kern_mx_gemm_bf16_s4", nullptr, nullptr, "kern_mx_gemm_bf16_s7",
                                        "kern_mx_gemm_bf16_s8"};
  if (M <= 64 && k % 1024 == 0 && k / 1024 <= 8 && skinny[k / 1024]) {
    const int32_t H = m / 8;
    const int32_t hb = std::min<int32_t>(9, (H + 255) / 256);
    Args a;
    a.put(a_), a.put(sf_a), a.put(b), a.put(sf_b), a.put(c), a.put(dbg), a.put(M), a.put(m), a.put(k), a.put(hb);
    return launch(skinny[k / 1024], (uint32_t)((H + hb - 1) / hb), 1, 1, 512, stream, a);
  }
  Args a;
  a.put(a_), a.put(sf_a), a.put(b), a.put(sf_b), a.put(c), a.put(M), a.put(m), a.put(k), a.put(dbg);
  return launch("kern_mx_gemm_bf16", (uint32_t)(m / 256), (uint32_t)((M + 127) / 128), 1, kBmmThreads, stream, a);
}

extern "C" int kern_mxfp4_gemv_bf16(const void* x, const void* w, const void* w_sf, void* y, int32_t M, int32_t N,
                                    int32_t K, void* stream) {
  REQUIRE(M >= 1 && M <= 16 && N > 0 && N % 16 == 0 && K > 0 && K % 512 == 0 && K <= 16384,
          "mxfp4_gemv_bf16: need 1 <= M <= 16, N %% 16 == 0, K %% 512 == 0, K <= 16384 (M=%d N=%d K=%d)", M, N, K);
  REQUIRE(x && w && w_sf && y, "mxfp4_gemv_bf16: null buffer");
  const int32_t kg = K / 512;
  // K = 512 * NKT with an unrolled instance for NKT: each of the four waves owns NKT consecutive k-tiles
  const char* fixed = kg == 2 ? "kern_mx_gemv_bf16_r2" : kg == 4 ? "kern_mx_gemv_bf16_r4" : kg == 8 ? "kern_mx_gemv_bf16_r8"
                      : kg == 14 ? "kern_mx_gemv_bf16_r14" : kg == 16 ? "kern_mx_gemv_bf16_r16" : nullptr;
  // Also taken at M = 3, and at any M while N <= 8192, as long as the x slices fit in 144 KiB of LDS.
  // Each workgroup reads all of x, so the persistent kernel's x reuse wins from M = 4 on at large N
  // (K = 7168, N = 9216: 9.8 against 10.1 us; N = 18432: 13.2 against 16.3). At M = 3 the two are within
  // 5% either way (N = 9216: 9.2 against 9.7 us; N = 18432: 13.6 against 13.2). At N <= 8192 the
  // persistent workgroups own four or fewer half groups, and the row-group kernel stays ahead:
  //   N = 7168, K = 8192, M = 8: 10.0 against 10.5 us;
  //   N = 4096, K = 4096, M = 16: 5.3 against 7.5 us.
  if (fixed && 2 * M * K <= 144 * 1024 && (M <= 3 || N <= 8192)) {
    // one workgroup per 16-row group; each wave's x slice (M * NKT * 256 B) in its own LDS region
    Args a;
    a.put(x), a.put(w), a.put(w_sf), a.put(y), a.put(M), a.put(N), a.put(K);
    return launch(fixed, (uint32_t)(N / 16), 1, 1, 256, stream, a, 2u * (uint32_t)M * (uint32_t)K);
  }
  if (M <= 2) {
    // other K: the same, each wave owning whole 512-wide k groups (a floor or ceiling of KG/4) in a loop,
    // and keeping their x (1 KiB per token and group) in its own LDS region
    const int32_t gmax = (kg + 3) / 4;
    Args a;
    a.put(x), a.put(w), a.put(w_sf), a.put(y), a.put(M), a.put(N), a.put(K), a.put(gmax);
    return launch("kern_mx_gemv_bf16_rg", (uint32_t)(N / 16), 1, 1, 256, stream, a, 4u * (uint32_t)(gmax * M) * 1024u);
  }
  static const char* const persistent[9] = {nullptr, "kern_mx_gemv_bf16_p1", "kern_mx_gemv_bf16_p2", nullptr,
                                            "kern_mx_gemv_bf16_p4", nullptr, nullptr, "kern_mx_gemv_bf16_p7",
                                            "kern_mx_gemv_bf16_p8"};
  if (K % 1024 == 0 && K / 1024 <= 8 && persistent[K / 1024]) {
    // about 256 workgroups of 8 waves, each owning hb <= 9 half groups of 8 rows (at most five 16-row
    // groups); wave w owns k-tiles [w*K/1024, (w+1)*K/1024) and holds their x in registers, one k-tile
    // at a time, passed through 4 KiB of LDS of its own
    const int32_t H = N / 8;
    const int32_t hb = std::min<int32_t>(9, (H + 255) / 256);
    Args a;
    a.put(x), a.put(w), a.put(w_sf), a.put(y), a.put(M), a.put(N), a.put(K), a.put(hb);
    return launch(persistent[K / 1024], (uint32_t)((H + hb - 1) / hb), 1, 1, 512, stream, a);
  }
  // any other shape: one workgroup per row group, x staged per workgroup in slices
  // sb: k-tiles per wave whose slice of x is staged in LDS at once (at most four 16-byte pieces per lane,
  // M * sb <= 16, sb divides K/512); nb: k-tiles per wave whose weights are in flight together (the
  // largest of the kernel's batch sizes dividing sb)
  const int32_t kq = K / 512;
  int32_t sb = 1;
  for (int32_t cand = std::min(kq, 16 / M); cand >= 1; --cand)
    if (kq % cand == 0) {
      sb = cand;
      break;
    }
  int32_t nb = 1;
  for (int32_t cand : {7, 4, 2})
    if (sb % cand == 0) {
      nb = cand;
      break;
    }
  // the x slice of every token, then the row group's scales (256 B per 512 of K)
  const uint32_t lds = (uint32_t)M * (uint32_t)(sb * 1024 + 16) + (uint32_t)(kq * 256);
  Args a;
  a.put(x), a.put(w), a.put(w_sf), a.put(y), a.put(M), a.put(N), a.put(K), a.put(nb), a.put(sb);
  return launch("kern_mx_gemv_bf16", (uint32_t)(N / 16), 1, 1, 256, stream, a, lds);
}

extern "C" int kern_silu_mul(void* out, const void* in, int32_t tokens, int32_t d, void* stream) {
  REQUIRE(tokens >= 0 && d > 0 && d % 8 == 0, "silu_mul: need d > 0, d %% 8 == 0, tokens >= 0 (d=%d tokens=%d)", d,
          tokens);
  if (tokens == 0) return KERN_OK;
  REQUIRE(out && in, "silu_mul: null buffer");
  REQUIRE(tokens <= 0x7fffffff && (d + 2047) / 2048 <= 65535, "silu_mul: grid too large (d=%d)", d);
  Args a;
  a.put(out), a.put(in), a.put(d);
  kern_function f = nullptr;
  if (int rc = function("kern_silu_mul_bf16", &f)) return rc;
  if (int rc = kern_function_check_params(f, a.sizes.data(), (int)a.sizes.size())) return rc;
  const uint32_t grid[3] = {(uint32_t)tokens, (uint32_t)((d + 2047) / 2048), 1}, blk[3] = {256, 1, 1};
  return kern_launch(f, grid, blk, 0, stream, a.buf, (a.n + 7) & ~size_t(7));
}

extern "C" int kern_moe_finalize_rms(const void* fc2_out, const int32_t* exp2perm, const float* topk_weight,
                                     const void* gamma, void* out, int32_t tokens, int32_t H, int32_t topk, float eps,
                                     void* stream) {
  REQUIRE(tokens >= 0 && H > 0 && H % 8 == 0 && H <= 8192 && topk > 0 && eps >= 0.f,
          "moe_finalize_rms: need 0 < H <= 8192, H %% 8 == 0, topk > 0, eps >= 0 (H=%d topk=%d)", H, topk);
  if (tokens == 0) return KERN_OK;
  REQUIRE(fc2_out && exp2perm && topk_weight && gamma && out, "moe_finalize_rms: null buffer");
  Args a;
  a.put(fc2_out), a.put(exp2perm), a.put(topk_weight), a.put(gamma), a.put(out), a.put(tokens), a.put(H);
  a.put(topk), a.put(eps);
  // one thread per 8-column chunk of the row, in whole waves (at most 1024 threads: H <= 8192)
  const uint32_t block = (uint32_t)(((H >> 3) + 63) / 64 * 64);
  return launch("kern_mx_moe_finalize_rms", (uint32_t)tokens, 1, 1, block, stream, a);
}

extern "C" int kern_moe_finalize(const void* fc2_out, const int32_t* exp2perm, const float* topk_weight, void* out,
                                 int32_t tokens, int32_t H, int32_t topk, void* stream) {
  REQUIRE(tokens >= 0 && H > 0 && H % 8 == 0 && topk > 0, "moe_finalize: need H > 0, H %% 8 == 0, topk > 0 (H=%d topk=%d)",
          H, topk);
  if (tokens == 0) return KERN_OK;
  REQUIRE(fc2_out && exp2perm && topk_weight && out, "moe_finalize: null buffer");
  Args a;
  a.put(fc2_out), a.put(exp2perm), a.put(topk_weight), a.put(out), a.put(tokens), a.put(H), a.put(topk);
  return launch("kern_mx_moe_finalize", (uint32_t)tokens, 1, 1, 256, stream, a);
}

extern "C" int kern_mxfp8_gemm_bf16(const void* a, const void* w, void* c, const void* a_sf, const void* w_sf, int32_t m,
                                    int32_t n, int32_t k, int32_t ldc, void* stream) {
  REQUIRE(m >= 0 && n >= 0 && k >= 0 && k % 32 == 0 && ldc >= n,
          "cublaslt_mxfp8_tn: need k %% 32 == 0 and ldc >= n (m=%d n=%d k=%d ldc=%d)", m, n, k, ldc);
  if (m == 0 || n == 0) return KERN_OK;
  REQUIRE((int64_t)m * k < ((int64_t)1 << 31) && (int64_t)n * k < ((int64_t)1 << 31) && (m + 127) / 128 <= 65535,
          "cublaslt_mxfp8_tn: operands beyond 2 GiB or m beyond the grid (m=%d n=%d k=%d)", m, n, k);
  REQUIRE(a && w && c && a_sf && w_sf, "cublaslt_mxfp8_tn: null buffer");
  if (k == 0) return fail(KERN_ERR_API, "cublaslt_mxfp8_tn: k == 0 leaves c undefined; zero it instead");
  Args x;
  x.put(a), x.put(w), x.put(c), x.put(a_sf), x.put(w_sf), x.put(m), x.put(n), x.put(k), x.put(ldc);
  return launch("kern_mx_gemm_mxfp8", (uint32_t)((n + 255) / 256), (uint32_t)((m + 127) / 128), 1, 512, stream, x);
}

// weight_prep family: one thread per element, 256 per workgroup (tools/kernels-src/weight_prep.cu)
static int elementwise(const char* entry, int32_t n, void* stream, Args& a) {
  if (n == 0) return KERN_OK;
  return launch(entry, (uint32_t)((n + 255) / 256), 1, 1, 256, stream, a);
}

extern "C" int kern_weight_p1_bf16_f32(const void* w, float* out, int32_t n, void* stream) {
  REQUIRE(n >= 0 && (n == 0 || (w && out)), "weight_p1_bf16_f32: need n >= 0 and buffers (n=%d)", n);
  Args a;
  a.put(w), a.put(out), a.put(n);
  return elementwise("kern_weight_p1_bf16_f32", n, stream, a);
}

extern "C" int kern_cast_bf16_f32(const void* w, float* out, int32_t n, void* stream) {
  REQUIRE(n >= 0 && (n == 0 || (w && out)), "cast_bf16_f32: need n >= 0 and buffers (n=%d)", n);
  Args a;
  a.put(w), a.put(out), a.put(n);
  return elementwise("kern_cast_bf16_f32", n, stream, a);
}

extern "C" int kern_rope_table_bf16(void* cos_t, void* sin_t, int32_t rows, int32_t half, int32_t stride, float base,
                                    void* stream) {
  REQUIRE(rows >= 0 && half > 0 && half <= 1024 && stride >= half && base > 0.f,
          "rope_table_bf16: need 0 < half <= 1024, stride >= half, base > 0 (rows=%d half=%d stride=%d)", rows, half,
          stride);
  if (rows == 0) return KERN_OK;
  REQUIRE(cos_t && sin_t, "rope_table_bf16: null buffer");
  Args a;
  a.put(cos_t), a.put(sin_t), a.put(rows), a.put(half), a.put(stride), a.put(base);
  return launch("kern_rope_table_bf16", (uint32_t)rows, 1, 1, (uint32_t)((half + 63) / 64 * 64), stream, a);
}

extern "C" int kern_fill_f32(float* p, int32_t n, float v, void* stream) {
  REQUIRE(n >= 0 && (n == 0 || p), "fill_f32: need n >= 0 and a buffer (n=%d)", n);
  Args a;
  a.put(p), a.put(n), a.put(v);
  return elementwise("kern_fill_f32", n, stream, a);
}

extern "C" int kern_fill_i32(int32_t* p, int32_t n, int32_t v, void* stream) {
  REQUIRE(n >= 0 && (n == 0 || p), "fill_i32: need n >= 0 and a buffer (n=%d)", n);
  Args a;
  a.put(p), a.put(n), a.put(v);
  return elementwise("kern_fill_i32", n, stream, a);
}

extern "C" int kern_fill_i64(int64_t* p, int32_t n, int64_t v, void* stream) {
  REQUIRE(n >= 0 && (n == 0 || p), "fill_i64: need n >= 0 and a buffer (n=%d)", n);
  Args a;
  a.put(p), a.put(n), a.put(v);
  return elementwise("kern_fill_i64", n, stream, a);
}

extern "C" int kern_fill_u8(uint8_t* p, int32_t n, int32_t v, void* stream) {
  REQUIRE(n >= 0 && (n == 0 || p), "fill_u8: need n >= 0 and a buffer (n=%d)", n);
  Args a;
  a.put(p), a.put(n), a.put(v);
  return elementwise("kern_fill_u8", n, stream, a);
}

extern "C" int kern_fill_bf16(void* p, int32_t n, float v, void* stream) {
  REQUIRE(n >= 0 && (n == 0 || p), "fill_bf16: need n >= 0 and a buffer (n=%d)", n);
  Args a;
  a.put(p), a.put(n), a.put(v);
  return elementwise("kern_fill_bf16", n, stream, a);
}

extern "C" int kern_iota_i32(int32_t* p, int32_t n, int32_t start, int32_t step, int32_t stride, void* stream) {
  REQUIRE(n >= 0 && stride >= 1 && (n == 0 || p), "iota_i32: need n >= 0, stride >= 1 and a buffer (n=%d stride=%d)",
          n, stride);
  Args a;
  a.put(p), a.put(n), a.put(start), a.put(step), a.put(stride);
  return elementwise("kern_iota_i32", n, stream, a);
}

extern "C" int kern_fill_random_u8(void* out, int64_t n, uint64_t seed, int32_t lo, int32_t span, void* stream) {
  REQUIRE(n >= 0 && span >= 1 && span <= 256, "fill_random_u8: need n >= 0 and 1 <= span <= 256");
  if (n == 0) return KERN_OK;
  REQUIRE(out, "fill_random_u8: null buffer");
  const int64_t threads = (n + 15) / 16;
  REQUIRE((threads + 255) / 256 < ((int64_t)1 << 31), "fill_random_u8: n too large");
  Args a;
  a.put(out), a.put(n), a.put(seed), a.put(lo), a.put(span);
  return launch("kern_mx_fill_random_u8", (uint32_t)((threads + 255) / 256), 1, 1, 256, stream, a);
}
