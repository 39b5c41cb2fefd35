// runtime.cpp — the tcacomp runtime over plain HIP, behind the C ABI of
// include/tca_rt.h.
//
// Reference counterparts:
//   runtime/tca/check.h:18-44      TCA_REQUIRE / TCA_CUDA_CHECK (exceptions)
//   runtime/tca/launch.h:37-58     ValidateLaunch (32-lane grammar, SMEM opt-in)
//   internal/cg/cxx/launch.go:23-156  the generated per-kernel launcher
// The launcher is data-driven here: the emitter writes a launch plan next to
// the code object and tca_program_launch interprets it, so the shape contract
// (every dim occurrence must agree), geometry validation and argument packing
// live in one audited place instead of being re-emitted per kernel.
#include "tca_rt.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "plan.h"
#include "scratch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

// The HIP error becomes this library's status and message; HIP's per-thread
// last-error slot is cleared, so another user of HIP in the process (a
// framework checking hipGetLastError after its own launches) does not
// inherit a failure that was already reported here.
int hip_fail(hipError_t e, const char* what) {
  (void)hipGetLastError();
  return fail(TCA_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
}

#define TCA_HIP_TRY(expr)                       \
  do {                                          \
    hipError_t e_ = (expr);                     \
    if (e_ != hipSuccess) return hip_fail(e_, #expr); \
  } while (0)

// Per-device launch limits, queried once per device.
struct DeviceLimits {
  bool valid = false;
  int max_threads = 1024;
  int max_lds = 65536;
};

std::mutex g_limits_mu;
DeviceLimits g_limits[64];

int query_limits(DeviceLimits* out) {
  int dev = 0;
  TCA_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(TCA_ERR_INVALID, "device id %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_limits_mu);
  if (!g_limits[dev].valid) {
    DeviceLimits l;
    TCA_HIP_TRY(hipDeviceGetAttribute(&l.max_threads, hipDeviceAttributeMaxThreadsPerBlock, dev));
    TCA_HIP_TRY(hipDeviceGetAttribute(&l.max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    l.valid = true;
    g_limits[dev] = l;
  }
  *out = g_limits[dev];
  return TCA_OK;
}

// Launch grammar shared by the GPU path and the host-only validator: the
// wave64 restatement of runtime/tca/launch.h:37-58.
int check_geometry(uint32_t grid, uint32_t block, uint32_t lds, int max_threads, int max_lds) {
  if (grid == 0) return fail(TCA_ERR_LAUNCH, "launch: grid must be >= 1 workgroup");
  if (grid > 0x7fffffffu) return fail(TCA_ERR_LAUNCH, "launch: grid %u exceeds 2^31-1 workgroups", grid);
  if (block == 0 || block % 64u != 0)
    return fail(TCA_ERR_LAUNCH, "launch: block %u is not a positive multiple of the 64-lane wavefront", block);
  if (block > static_cast<uint32_t>(max_threads))
    return fail(TCA_ERR_LAUNCH, "launch: block %u exceeds the device limit of %d threads", block, max_threads);
  if (lds > static_cast<uint32_t>(max_lds))
    return fail(TCA_ERR_LAUNCH, "launch: %u bytes of LDS exceed the device limit of %d", lds, max_lds);
  return TCA_OK;
}

}  // namespace

struct tca_module_s {
  hipModule_t mod = nullptr;
};

struct tca_event_s {
  hipEvent_t ev = nullptr;
};

struct tca_program_s {
  struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
  };
  // Everything a launch decides from the shapes alone, kept for the last
  // shape launched: a repeat launch at that shape compares the shapes,
  // checks the pointers, fills pointer and scalar slots into copies of the
  // argument blobs and launches (no Bind, no guard or grid evaluation, no
  // heap allocation).
  struct Prepared {
    uint32_t n_tensors = 0, n_free = 0;
    std::vector<uint32_t> key;        // per tensor: rank, dtype, dims...; then the free dims
    std::vector<uint8_t> nonempty;    // per tensor parameter: it has elements (data must be valid)
    std::vector<int> param_of;        // per plan tensor: its parameter index, -1 for a local
    std::vector<size_t> local_off;    // per plan tensor: offset of a local in the workspace
    size_t ws_bytes = 0;
    struct Launch {
      hipFunction_t fn = nullptr;
      uint32_t grid = 0, block = 0, lds = 0;
      std::vector<unsigned char> blob;         // dims written, pointer and scalar slots zero
      std::vector<tca::plan::ArgSlot> slots;
    };
    std::vector<Launch> launches;
  };
  tca::plan::Plan plan;
  hipModule_t mod = nullptr;
  std::vector<hipFunction_t> funcs;
  // HBM locals and partial scratch, one workspace per stream the program is
  // launched on: launches on one stream are ordered and may share it,
  // launches on different streams may overlap and must not.
  std::map<tca_stream_t, Workspace> workspaces;
  std::mutex mu;  // guards `workspaces` and `prepared`
  std::shared_ptr<const Prepared> prepared;
  std::string plan_text;  // tca_program_plan_text's buffer, filled on first request
};

extern "C" {

const char* tca_rt_last_error(void) { return g_last_error.c_str(); }

int tca_rt_init(int device) {
  int n = 0;
  TCA_HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(TCA_ERR_INVALID, "init: device %d not present (%d devices)", device, n);
  TCA_HIP_TRY(hipSetDevice(device));
  DeviceLimits l;
  int rc = query_limits(&l);
  if (rc != TCA_OK) return rc;
  // The allocation-free launch's scratch: its device address on this device.
  TCA_HIP_TRY(tca::rt::ScratchInit(device));
  return TCA_OK;
}

int tca_rt_device_info(int device, tca_device_info* out) {
  if (out == nullptr) return fail(TCA_ERR_INVALID, "device_info: null output");
  hipDeviceProp_t p;
  TCA_HIP_TRY(hipGetDeviceProperties(&p, device));
  std::memset(out, 0, sizeof(*out));
  std::snprintf(out->name, sizeof(out->name), "%s", p.name);
  std::snprintf(out->arch, sizeof(out->arch), "%.63s", p.gcnArchName);
  out->compute_units = p.multiProcessorCount;
  out->wavefront_size = p.warpSize;
  out->max_threads_per_block = p.maxThreadsPerBlock;
  out->max_lds_per_block = static_cast<int32_t>(p.sharedMemPerBlock);
  out->clock_khz = p.clockRate;
  out->total_global_mem = p.totalGlobalMem;
  return TCA_OK;
}

int tca_rt_device_sync(void) {
  TCA_HIP_TRY(hipDeviceSynchronize());
  return TCA_OK;
}

int tca_rt_malloc(void** ptr, size_t bytes) {
  if (ptr == nullptr) return fail(TCA_ERR_INVALID, "malloc: null output");
  *ptr = nullptr;
  if (bytes == 0) return TCA_OK;
  TCA_HIP_TRY(hipMalloc(ptr, bytes));
  return TCA_OK;
}

int tca_rt_free(void* ptr) {
  if (ptr == nullptr) return TCA_OK;
  TCA_HIP_TRY(hipFree(ptr));
  return TCA_OK;
}

int tca_rt_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return TCA_OK;
  if (dst == nullptr || src == nullptr) return fail(TCA_ERR_INVALID, "memcpy_h2d: null pointer for %zu bytes", bytes);
  TCA_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return TCA_OK;
}

int tca_rt_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  if (bytes == 0) return TCA_OK;
  if (dst == nullptr || src == nullptr) return fail(TCA_ERR_INVALID, "memcpy_d2h: null pointer for %zu bytes", bytes);
  TCA_HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return TCA_OK;
}

int tca_rt_memset(void* dst, int value, size_t bytes) {
  if (bytes == 0) return TCA_OK;
  if (dst == nullptr) return fail(TCA_ERR_INVALID, "memset: null pointer for %zu bytes", bytes);
  TCA_HIP_TRY(hipMemset(dst, value, bytes));
  return TCA_OK;
}

int tca_rt_stream_create(tca_stream_t* out) {
  if (out == nullptr) return fail(TCA_ERR_INVALID, "stream_create: null output");
  hipStream_t s = nullptr;
  // Default priority only: the stream carries no priority attribute.
  TCA_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  *out = s;
  return TCA_OK;
}

int tca_rt_stream_destroy(tca_stream_t s) {
  if (s == nullptr) return TCA_OK;
  TCA_HIP_TRY(hipStreamDestroy(static_cast<hipStream_t>(s)));
  return TCA_OK;
}

int tca_rt_stream_sync(tca_stream_t s) {
  TCA_HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(s)));
  return TCA_OK;
}

int tca_rt_event_create(tca_event* out) {
  if (out == nullptr) return fail(TCA_ERR_INVALID, "event_create: null output");
  auto* e = new tca_event_s;
  hipError_t err = hipEventCreate(&e->ev);
  if (err != hipSuccess) {
    delete e;
    return hip_fail(err, "hipEventCreate");
  }
  *out = e;
  return TCA_OK;
}

int tca_rt_event_destroy(tca_event ev) {
  if (ev == nullptr) return TCA_OK;
  hipError_t err = hipEventDestroy(ev->ev);
  delete ev;
  if (err != hipSuccess) return hip_fail(err, "hipEventDestroy");
  return TCA_OK;
}

int tca_rt_event_record(tca_event ev, tca_stream_t s) {
  if (ev == nullptr) return fail(TCA_ERR_INVALID, "event_record: null event");
  TCA_HIP_TRY(hipEventRecord(ev->ev, static_cast<hipStream_t>(s)));
  return TCA_OK;
}

int tca_rt_event_elapsed_ms(tca_event start, tca_event stop, float* ms) {
  if (start == nullptr || stop == nullptr || ms == nullptr) return fail(TCA_ERR_INVALID, "event_elapsed: null argument");
  TCA_HIP_TRY(hipEventSynchronize(stop->ev));
  TCA_HIP_TRY(hipEventElapsedTime(ms, start->ev, stop->ev));
  return TCA_OK;
}

int tca_rt_module_load(const char* hsaco_path, tca_module* out) {
  if (hsaco_path == nullptr || out == nullptr) return fail(TCA_ERR_INVALID, "module_load: null argument");
  std::ifstream f(hsaco_path, std::ios::binary);
  if (!f) return fail(TCA_ERR_NOT_FOUND, "module_load: cannot open %s", hsaco_path);
  auto* m = new tca_module_s;
  hipError_t err = hipModuleLoad(&m->mod, hsaco_path);
  if (err != hipSuccess) {
    delete m;
    return hip_fail(err, "hipModuleLoad");
  }
  *out = m;
  return TCA_OK;
}

int tca_rt_module_unload(tca_module m) {
  if (m == nullptr) return TCA_OK;
  hipError_t err = hipModuleUnload(m->mod);
  delete m;
  if (err != hipSuccess) return hip_fail(err, "hipModuleUnload");
  return TCA_OK;
}

int tca_rt_validate_launch(uint32_t grid, uint32_t block, uint32_t lds_bytes) {
  int max_threads = 1024, max_lds = 160 * 1024;  // gfx950 limits when no device is queried
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) == hipSuccess && ndev > 0) {
    DeviceLimits l;
    if (query_limits(&l) == TCA_OK) {
      max_threads = l.max_threads;
      max_lds = l.max_lds;
    }
  }
  return check_geometry(grid, block, lds_bytes, max_threads, max_lds);
}

int tca_rt_launch(tca_module m, const char* kernel, uint32_t grid, uint32_t block, uint32_t lds_bytes,
                  void* args, size_t args_size, tca_stream_t s) {
  if (m == nullptr || kernel == nullptr) return fail(TCA_ERR_INVALID, "launch: null module or kernel name");
  if (args == nullptr && args_size > 0) return fail(TCA_ERR_INVALID, "launch: null argument blob of %zu bytes", args_size);
  DeviceLimits l;
  int rc = query_limits(&l);
  if (rc != TCA_OK) return rc;
  rc = check_geometry(grid, block, lds_bytes, l.max_threads, l.max_lds);
  if (rc != TCA_OK) return rc;
  hipFunction_t fn = nullptr;
  hipError_t err = hipModuleGetFunction(&fn, m->mod, kernel);
  if (err != hipSuccess) return fail(TCA_ERR_NOT_FOUND, "launch: kernel %s not in module (%s)", kernel, hipGetErrorString(err));
  size_t size = args_size;
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  TCA_HIP_TRY(hipModuleLaunchKernel(fn, grid, 1, 1, block, 1, 1, lds_bytes, static_cast<hipStream_t>(s), nullptr, config));
  return TCA_OK;
}

int tca_program_parse(const char* plan_text, tca_program* out) {
  if (plan_text == nullptr || out == nullptr) return fail(TCA_ERR_INVALID, "program_parse: null argument");
  auto* p = new tca_program_s;
  std::string err;
  if (!tca::plan::Parse(plan_text, &p->plan, &err)) {
    delete p;
    return fail(TCA_ERR_INVALID, "plan: %s", err.c_str());
  }
  *out = p;
  return TCA_OK;
}

int tca_program_load(const char* hsaco_path, const char* plan_text, tca_program* out) {
  if (hsaco_path == nullptr || out == nullptr) return fail(TCA_ERR_INVALID, "program_load: null argument");
  tca_program p = nullptr;
  int rc = tca_program_parse(plan_text, &p);
  if (rc != TCA_OK) return rc;
  std::ifstream f(hsaco_path, std::ios::binary);
  if (!f) {
    delete p;
    return fail(TCA_ERR_NOT_FOUND, "program_load: cannot open %s", hsaco_path);
  }
  hipError_t err = hipModuleLoad(&p->mod, hsaco_path);
  if (err != hipSuccess) {
    delete p;
    return hip_fail(err, "hipModuleLoad");
  }
  for (const auto& k : p->plan.kernels) {
    hipFunction_t fn = nullptr;
    err = hipModuleGetFunction(&fn, p->mod, k.symbol.c_str());
    if (err != hipSuccess) {
      (void)hipModuleUnload(p->mod);
      delete p;
      return fail(TCA_ERR_NOT_FOUND, "program_load: kernel %s missing from %s", k.symbol.c_str(), hsaco_path);
    }
    p->funcs.push_back(fn);
  }
  *out = p;
  return TCA_OK;
}

int tca_program_unload(tca_program p) {
  if (p == nullptr) return TCA_OK;
  int rc = TCA_OK;
  for (auto& kv : p->workspaces) {
    if (kv.second.ptr == nullptr) continue;
    hipError_t e = hipFree(kv.second.ptr);
    if (e != hipSuccess && rc == TCA_OK) rc = hip_fail(e, "hipFree(workspace)");
  }
  if (p->mod != nullptr) {
    hipError_t e = hipModuleUnload(p->mod);
    if (e != hipSuccess && rc == TCA_OK) rc = hip_fail(e, "hipModuleUnload");
  }
  delete p;
  return rc;
}

int tca_program_signature(tca_program p, uint32_t* n_tensors, uint32_t* n_free_dims, uint32_t* n_scalars,
                          uint32_t* n_kernels) {
  if (p == nullptr) return fail(TCA_ERR_INVALID, "program_signature: null program");
  const auto& pl = p->plan;
  if (n_tensors) *n_tensors = static_cast<uint32_t>(pl.ParamTensorCount());
  if (n_free_dims) *n_free_dims = static_cast<uint32_t>(pl.FreeDims().size());
  if (n_scalars) *n_scalars = static_cast<uint32_t>(pl.scalars.size());
  if (n_kernels) *n_kernels = static_cast<uint32_t>(pl.kernels.size());
  return TCA_OK;
}

const char* tca_program_kernel_name(tca_program p, uint32_t i) {
  if (p == nullptr || i >= p->plan.kernels.size()) return nullptr;
  return p->plan.kernels[i].symbol.c_str();
}

const char* tca_program_plan_text(tca_program p) {
  if (p == nullptr) return nullptr;
  std::lock_guard<std::mutex> lk(p->mu);
  if (p->plan_text.empty()) p->plan_text = tca::plan::Serialize(p->plan);
  return p->plan_text.c_str();
}

int tca_program_check(tca_program p, const tca_tensor* tensors, uint32_t n_tensors, const uint32_t* free_dims,
                      uint32_t n_free_dims) {
  if (p == nullptr) return fail(TCA_ERR_INVALID, "program_check: null program");
  std::vector<uint32_t> dims;
  std::string err;
  int code = tca::plan::Bind(p->plan, tensors, n_tensors, free_dims, n_free_dims, &dims, &err);
  if (code != TCA_OK) return fail(code, "%s", err.c_str());
  return TCA_OK;
}

int tca_program_selected(tca_program p, const tca_tensor* tensors, uint32_t n_tensors, const uint32_t* free_dims,
                         uint32_t n_free_dims, uint8_t* selected, uint64_t* grids, uint32_t* blocks,
                         uint32_t n_selected) {
  if (p == nullptr) return fail(TCA_ERR_INVALID, "program_selected: null program");
  if (n_selected != p->plan.kernels.size())
    return fail(TCA_ERR_INVALID, "program_selected: program has %zu kernel(s), got room for %u", p->plan.kernels.size(),
                n_selected);
  if (n_selected > 0 && selected == nullptr) return fail(TCA_ERR_INVALID, "program_selected: null output");
  std::vector<uint32_t> dims;
  std::string err;
  int code = tca::plan::Bind(p->plan, tensors, n_tensors, free_dims, n_free_dims, &dims, &err);
  if (code != TCA_OK) return fail(code, "%s", err.c_str());
  for (uint32_t i = 0; i < n_selected; ++i) {
    const auto& k = p->plan.kernels[i];
    selected[i] = tca::plan::Selected(k, dims) ? 1 : 0;
    if (blocks != nullptr) {
      blocks[i] = 0;
      if (selected[i]) (void)tca::plan::PackRows(k, dims, &blocks[i]);
    }
    if (grids == nullptr) continue;
    grids[i] = 0;
    if (selected[i] && !tca::plan::GridSize(k, p->plan, dims, &grids[i], &err)) return fail(TCA_ERR_LAUNCH, "%s", err.c_str());
  }
  return TCA_OK;
}

}  // extern "C"

namespace {

// Writes this call's pointers and scalars into the slots of a prepared
// argument blob: a parameter's data pointer, or a local's address in the
// workspace `ws`.
void fill_args(unsigned char* blob, const std::vector<tca::plan::ArgSlot>& slots, const std::vector<int>& param_of,
               const std::vector<size_t>& local_off, const tca_tensor* tensors, void* ws, const double* scalars) {
  for (const auto& sl : slots) {
    if (sl.kind == tca::plan::ArgKind::Ptr) {
      const int pi = param_of[sl.index];
      // integer arithmetic: the host-only query lays locals out from address 0
      void* ptr = pi >= 0 ? tensors[pi].data
                          : reinterpret_cast<void*>(reinterpret_cast<uintptr_t>(ws) + local_off[sl.index]);
      std::memcpy(blob + sl.offset, &ptr, sizeof ptr);
    } else {
      tca::plan::SetScalar(blob, sl, scalars[sl.index]);
    }
  }
}

// The launch decisions for one shape (the slow path, run when the shapes
// differ from the cached ones): Bind (the shape contract and its errors),
// the workspace layout, then per kernel its guards, grid, block, geometry
// and argument layout.
int prepare_launch(tca_program p, const tca_tensor* tensors, uint32_t n_tensors, const uint32_t* free_dims,
                   uint32_t n_free_dims, std::shared_ptr<tca_program_s::Prepared>* out) {
  const auto& pl = p->plan;
  std::vector<uint32_t> dims;
  std::string err;
  int code = tca::plan::Bind(pl, tensors, n_tensors, free_dims, n_free_dims, &dims, &err);
  if (code != TCA_OK) return fail(code, "%s", err.c_str());
  auto pr = std::make_shared<tca_program_s::Prepared>();
  pr->n_tensors = n_tensors;
  pr->n_free = n_free_dims;
  for (uint32_t i = 0; i < n_tensors; ++i) {
    const tca_tensor& t = tensors[i];
    pr->key.push_back(t.rank);
    pr->key.push_back(static_cast<uint32_t>(t.dtype));
    uint64_t elems = 1;
    for (uint32_t a = 0; a < t.rank; ++a) {
      pr->key.push_back(t.dims[a]);
      elems *= t.dims[a];
    }
    pr->nonempty.push_back(elems > 0 ? 1 : 0);
  }
  for (uint32_t i = 0; i < n_free_dims; ++i) pr->key.push_back(free_dims[i]);

  // HBM locals: one workspace, each local at a 256-byte aligned offset; only
  // the locals some kernel selected for these dims takes (a variant's
  // scratch is sized for the dims it runs on).
  std::vector<bool> used(pl.tensors.size(), false);
  for (const auto& k : pl.kernels) {
    if (!tca::plan::Selected(k, dims)) continue;
    for (const auto& a : k.args)
      if (a.kind == tca::plan::ArgKind::Ptr) used[a.index] = true;
  }
  if (!tca::plan::WorkspaceLayout(pl, dims, used, &pr->local_off, &pr->ws_bytes, &err))
    return fail(TCA_ERR_INVALID, "%s", err.c_str());
  pr->param_of.assign(pl.tensors.size(), -1);
  int next_param = 0;
  for (size_t t = 0; t < pl.tensors.size(); ++t)
    if (pl.tensors[t].role != tca::plan::Role::Local) pr->param_of[t] = next_param++;

  DeviceLimits l;
  int rc = query_limits(&l);
  if (rc != TCA_OK) return rc;
  for (size_t ki = 0; ki < pl.kernels.size(); ++ki) {
    const auto& k = pl.kernels[ki];
    if (!tca::plan::Selected(k, dims)) continue;  // a variant for other dims
    uint64_t grid = 0;
    if (!tca::plan::GridSize(k, pl, dims, &grid, &err)) return fail(TCA_ERR_LAUNCH, "%s", err.c_str());
    if (grid == 0) continue;  // nothing to compute (an empty output)
    if (grid > 0x7fffffffull)
      return fail(TCA_ERR_LAUNCH, "kernel %s: grid %llu exceeds 2^31-1", k.symbol.c_str(),
                  static_cast<unsigned long long>(grid));
    uint32_t block = k.block;
    (void)tca::plan::PackRows(k, dims, &block);  // packed row kernels size the block at launch
    rc = check_geometry(static_cast<uint32_t>(grid), block, k.lds, l.max_threads, l.max_lds);
    if (rc != TCA_OK) return rc;
    tca_program_s::Prepared::Launch L;
    L.fn = p->funcs.empty() ? nullptr : p->funcs[ki];
    L.grid = static_cast<uint32_t>(grid);
    L.block = block;
    L.lds = k.lds;
    if (!tca::plan::LayoutArgs(k, pl, dims, &L.blob, &L.slots, &err)) return fail(TCA_ERR_INVALID, "%s", err.c_str());
    pr->launches.push_back(std::move(L));
  }
  *out = std::move(pr);
  return TCA_OK;
}

// Whether a launch with these arguments repeats the prepared shape with
// usable pointers; anything else takes the slow path, which reports the
// error a mismatch deserves.
bool repeats(const tca_program_s::Prepared& pr, const tca_tensor* tensors, uint32_t n_tensors,
             const uint32_t* free_dims, uint32_t n_free_dims) {
  if (n_tensors != pr.n_tensors || n_free_dims != pr.n_free) return false;
  if ((n_tensors > 0 && tensors == nullptr) || (n_free_dims > 0 && free_dims == nullptr)) return false;
  const uint32_t* k = pr.key.data();
  for (uint32_t i = 0; i < n_tensors; ++i) {
    const tca_tensor& t = tensors[i];
    if (t.rank != *k++ || static_cast<uint32_t>(t.dtype) != *k++) return false;
    for (uint32_t a = 0; a < t.rank; ++a)
      if (t.dims[a] != *k++) return false;
    if (pr.nonempty[i] && (t.data == nullptr || (reinterpret_cast<uintptr_t>(t.data) % 16u) != 0u)) return false;
  }
  for (uint32_t i = 0; i < n_free_dims; ++i)
    if (free_dims[i] != *k++) return false;
  return true;
}

// The body of both launch entry points. `noalloc` takes the workspace from
// the device's scratch array instead of the program's per-stream workspace.
int launch_program(tca_program p, const tca_tensor* tensors, uint32_t n_tensors, const uint32_t* free_dims,
                   uint32_t n_free_dims, const double* scalars, uint32_t n_scalars, tca_stream_t stream,
                   bool noalloc) {
  if (p == nullptr) return fail(TCA_ERR_INVALID, "program_launch: null program");
  if (p->mod == nullptr) return fail(TCA_ERR_INVALID, "program_launch: program was parsed, not loaded");
  const auto& pl = p->plan;
  std::shared_ptr<const tca_program_s::Prepared> pr;
  {
    std::lock_guard<std::mutex> lk(p->mu);
    pr = p->prepared;
  }
  if (!pr || !repeats(*pr, tensors, n_tensors, free_dims, n_free_dims)) {
    std::shared_ptr<tca_program_s::Prepared> fresh;
    int rc = prepare_launch(p, tensors, n_tensors, free_dims, n_free_dims, &fresh);
    if (rc != TCA_OK) return rc;
    pr = fresh;
    std::lock_guard<std::mutex> lk(p->mu);
    p->prepared = fresh;
  }
  if (n_scalars != pl.scalars.size())
    return fail(TCA_ERR_INVALID, "program %s takes %zu scalar(s), got %u", pl.name.c_str(), pl.scalars.size(), n_scalars);
  if (n_scalars > 0 && scalars == nullptr) return fail(TCA_ERR_INVALID, "program_launch: null scalars");

  void* ws = nullptr;
  // Held until the last kernel is enqueued: a launch of this program on the
  // same stream from another thread that grows the workspace synchronizes
  // the stream and frees the old buffer, which must not happen between
  // reading the pointer here and queueing the kernels that use it.
  std::unique_lock<std::mutex> lk(p->mu, std::defer_lock);
  if (pr->ws_bytes > 0 && noalloc) {
    int dev = 0;
    TCA_HIP_TRY(hipGetDevice(&dev));
    if (pr->ws_bytes > tca::rt::kScratchBytes)
      return fail(TCA_ERR_INVALID,
                  "program_launch_noalloc: program %s needs %zu bytes of scratch at these dims, more than the %zu "
                  "bytes the allocation-free launch has (use tca_program_launch)",
                  pl.name.c_str(), pr->ws_bytes, tca::rt::kScratchBytes);
    ws = tca::rt::ScratchPtr(dev);
    if (ws == nullptr)
      return fail(TCA_ERR_INVALID, "program_launch_noalloc: tca_rt_init(%d) has not set up this device", dev);
  } else if (pr->ws_bytes > 0) {
    lk.lock();
    tca_program_s::Workspace& w = p->workspaces[stream];
    if (w.bytes < pr->ws_bytes) {
      if (w.ptr != nullptr) {
        // Kernels queued on this stream may still use the smaller workspace.
        TCA_HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
        TCA_HIP_TRY(hipFree(w.ptr));
        w.ptr = nullptr;
        w.bytes = 0;
      }
      TCA_HIP_TRY(hipMalloc(&w.ptr, pr->ws_bytes));
      w.bytes = pr->ws_bytes;
    }
    ws = w.ptr;
  }

  for (const auto& L : pr->launches) {
    // The kernel arguments: the prepared blob with the pointers and scalars
    // of this call written into their slots (on the stack for every
    // kernarg block this emitter writes).
    unsigned char small[512];
    std::vector<unsigned char> big;
    unsigned char* blob = small;
    if (L.blob.size() > sizeof small) {
      big.resize(L.blob.size());
      blob = big.data();
    }
    std::memcpy(blob, L.blob.data(), L.blob.size());
    fill_args(blob, L.slots, pr->param_of, pr->local_off, tensors, ws, scalars);
    size_t size = L.blob.size();
    void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, blob, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                      HIP_LAUNCH_PARAM_END};
    hipError_t e = hipModuleLaunchKernel(L.fn, L.grid, 1, 1, L.block, 1, 1, L.lds, static_cast<hipStream_t>(stream),
                                         nullptr, config);
    if (e != hipSuccess) return hip_fail(e, "hipModuleLaunchKernel");
  }
  return TCA_OK;
}

}  // namespace

extern "C" {

int tca_program_launch(tca_program p, const tca_tensor* tensors, uint32_t n_tensors, const uint32_t* free_dims,
                       uint32_t n_free_dims, const double* scalars, uint32_t n_scalars, tca_stream_t stream) {
  return launch_program(p, tensors, n_tensors, free_dims, n_free_dims, scalars, n_scalars, stream, false);
}

int tca_program_launch_noalloc(tca_program p, const tca_tensor* tensors, uint32_t n_tensors,
                               const uint32_t* free_dims, uint32_t n_free_dims, const double* scalars,
                               uint32_t n_scalars, tca_stream_t stream) {
  return launch_program(p, tensors, n_tensors, free_dims, n_free_dims, scalars, n_scalars, stream, true);
}

int tca_program_kernel_args(tca_program p, const tca_tensor* tensors, uint32_t n_tensors, const uint32_t* free_dims,
                            uint32_t n_free_dims, const double* scalars, uint32_t n_scalars, uint32_t kernel,
                            void* buf, size_t cap, size_t* size) {
  if (p == nullptr) return fail(TCA_ERR_INVALID, "program_kernel_args: null program");
  const auto& pl = p->plan;
  if (kernel >= pl.kernels.size())
    return fail(TCA_ERR_INVALID, "program_kernel_args: program has %zu kernel(s), asked for %u", pl.kernels.size(), kernel);
  std::vector<uint32_t> dims;
  std::string err;
  int code = tca::plan::Bind(pl, tensors, n_tensors, free_dims, n_free_dims, &dims, &err);
  if (code != TCA_OK) return fail(code, "%s", err.c_str());
  if (n_scalars != pl.scalars.size())
    return fail(TCA_ERR_INVALID, "program %s takes %zu scalar(s), got %u", pl.name.c_str(), pl.scalars.size(), n_scalars);
  if (n_scalars > 0 && scalars == nullptr) return fail(TCA_ERR_INVALID, "program_kernel_args: null scalars");
  const auto& k = pl.kernels[kernel];
  uint64_t grid = 0;
  if (!tca::plan::Selected(k, dims) || !tca::plan::GridSize(k, pl, dims, &grid, &err) || grid == 0)
    return fail(TCA_ERR_INVALID, "program_kernel_args: kernel %s does not run at these dims", k.symbol.c_str());
  // The workspace layout of a launch at these dims (the locals of the
  // selected kernels at 256-byte aligned offsets).
  std::vector<bool> used(pl.tensors.size(), false);
  for (const auto& kk : pl.kernels) {
    if (!tca::plan::Selected(kk, dims)) continue;
    for (const auto& a : kk.args)
      if (a.kind == tca::plan::ArgKind::Ptr) used[a.index] = true;
  }
  std::vector<size_t> local_off;
  std::vector<int> param_of(pl.tensors.size(), -1);
  size_t ws_bytes = 0;
  if (!tca::plan::WorkspaceLayout(pl, dims, used, &local_off, &ws_bytes, &err))
    return fail(TCA_ERR_INVALID, "%s", err.c_str());
  int next_param = 0;
  for (size_t t = 0; t < pl.tensors.size(); ++t)
    if (pl.tensors[t].role != tca::plan::Role::Local) param_of[t] = next_param++;
  std::vector<unsigned char> blob;
  std::vector<tca::plan::ArgSlot> slots;
  if (!tca::plan::LayoutArgs(k, pl, dims, &blob, &slots, &err)) return fail(TCA_ERR_INVALID, "%s", err.c_str());
  fill_args(blob.data(), slots, param_of, local_off, tensors, nullptr, scalars);
  if (size != nullptr) *size = blob.size();
  if (buf == nullptr || cap < blob.size())
    return fail(TCA_ERR_INVALID, "program_kernel_args: %zu bytes needed, room for %zu", blob.size(), cap);
  std::memcpy(buf, blob.data(), blob.size());
  return TCA_OK;
}

}  // extern "C"
