/*
 * tca_rt.h — C ABI of the tcacomp MI355X runtime (plain HIP, gfx950).
 *
 * This is the run-time operator seam. In the reference every compiled DSL
 * kernel exports one C++ launcher
 *     void <Kernel>Launch(uint32_t e<N>..., const tca::Tensor<T,R>& in...,
 *                         tca::Tensor<T,R>& out..., <scalars>..., cudaStream_t)
 * (emitted by internal/cg/cxx/launch.go:23-156, instance
 * testing/runners/softmax.cu:10-11) that derives every dim from the tensors,
 * cross-checks each dim occurrence (launch.go:98-130), validates the launch
 * grammar (runtime/tca/launch.h:37-58) and launches. Errors are C++
 * exceptions (runtime/tca/check.h:18-44).
 *
 * Here a compiled DSL program is a `tca_program`: a code object (.hsaco,
 * produced by hipcc from the emitted HIP source) plus the launch plan the
 * emitter wrote beside it. `tca_program_launch` is the one launcher for every
 * program. Rules of this ABI:
 *   - every function returns an int status (TCA_OK == 0); no exception ever
 *     crosses it; `tca_rt_last_error()` holds the calling thread's last
 *     message;
 *   - handles are opaque; device memory is owned by the caller;
 *   - launches are asynchronous on the caller's stream (NULL = default).
 */
#ifndef TCA_RT_H_
#define TCA_RT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
enum {
  TCA_OK = 0,
  TCA_ERR_INVALID = 1,     /* bad argument / malformed plan */
  TCA_ERR_SHAPE = 2,       /* tensor shape disagrees with the program */
  TCA_ERR_LAUNCH = 3,      /* launch geometry refused by the validator */
  TCA_ERR_HIP = 4,         /* a HIP call failed (message names it) */
  TCA_ERR_NOT_FOUND = 5,   /* file / kernel symbol missing */
  TCA_ERR_UNSUPPORTED = 6, /* construct the backend does not lower */
  TCA_ERR_BUILD = 7        /* DSL program rejected by the builder/verifier */
};

/* Element types; the numbering is shared with tca_cg.h. */
enum {
  TCA_F32 = 0,
  TCA_F16 = 1,
  TCA_BF16 = 2,
  TCA_I32 = 3,
  TCA_U32 = 4,
  TCA_I8 = 5,
  TCA_I16 = 6,
  TCA_U8 = 7,
  TCA_U16 = 8,
  TCA_BOOL = 9
};

#define TCA_MAX_RANK 8

/* Non-owning, row-major tensor descriptor: the C face of the reference's
 * tca::Tensor<T,R> (runtime/tca/tensor.h:17-40). At most 2^32 - 2^16 - 1
 * elements (TCA_ERR_SHAPE beyond): the u32 index domain less the headroom
 * the kernels' index steps need. */
typedef struct tca_tensor {
  void* data;
  uint32_t rank;
  uint32_t dims[TCA_MAX_RANK];
  int32_t dtype;
} tca_tensor;

typedef void* tca_stream_t; /* a hipStream_t */
typedef struct tca_module_s* tca_module;
typedef struct tca_program_s* tca_program;
typedef struct tca_event_s* tca_event;

typedef struct tca_device_info {
  char name[256];
  char arch[64];             /* e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t wavefront_size;
  int32_t max_threads_per_block;
  int32_t max_lds_per_block; /* bytes */
  int32_t clock_khz;
  uint64_t total_global_mem; /* bytes */
} tca_device_info;

/* ---- errors / device (runtime/tca/check.h:18-44) ---- */
const char* tca_rt_last_error(void);
int tca_rt_init(int device);
int tca_rt_device_info(int device, tca_device_info* out);
int tca_rt_device_sync(void);

/* ---- memory (the runners' cudaMalloc/cudaMemcpy, testing/runners/gemm.cu:26-32) ---- */
int tca_rt_malloc(void** ptr, size_t bytes);
int tca_rt_free(void* ptr);
int tca_rt_memcpy_h2d(void* dst, const void* src, size_t bytes);
int tca_rt_memcpy_d2h(void* dst, const void* src, size_t bytes);
int tca_rt_memset(void* dst, int value, size_t bytes);

/* ---- streams and hipEvent timing (replaces the host steady_clock of
 *      testing/runners/common.cuh:71-90) ---- */
int tca_rt_stream_create(tca_stream_t* out);
int tca_rt_stream_destroy(tca_stream_t s);
int tca_rt_stream_sync(tca_stream_t s);
int tca_rt_event_create(tca_event* out);
int tca_rt_event_destroy(tca_event ev);
int tca_rt_event_record(tca_event ev, tca_stream_t s);
int tca_rt_event_elapsed_ms(tca_event start, tca_event stop, float* ms);

/* ---- code objects and raw launches (hipModuleLoad / hipModuleLaunchKernel) ---- */
int tca_rt_module_load(const char* hsaco_path, tca_module* out);
int tca_rt_module_unload(tca_module m);
/* Launch grammar for wave64 (replaces runtime/tca/launch.h:37-58): 1-D grid
 * of >= 1 workgroups, block a multiple of 64 and <= 1024, LDS <= the device's
 * per-workgroup limit (queried; 160 KiB on gfx950). Host-only check. */
int tca_rt_validate_launch(uint32_t grid, uint32_t block, uint32_t lds_bytes);
int tca_rt_launch(tca_module m, const char* kernel, uint32_t grid, uint32_t block,
                  uint32_t lds_bytes, void* args, size_t args_size, tca_stream_t s);

/* ---- compiled DSL programs: the generated <Kernel>Launch, as one entry ----
 * `plan` is the text the emitter wrote beside the code object. */
int tca_program_load(const char* hsaco_path, const char* plan, tca_program* out);
int tca_program_unload(tca_program p);
/* Parses `plan` and checks it without touching a GPU (no code object). The
 * returned handle can be queried and validated but not launched. */
int tca_program_parse(const char* plan, tca_program* out);
/* Number of tensor parameters the launcher takes (inputs and outputs, in
 * declaration order; locals excluded), free dims and scalars. */
int tca_program_signature(tca_program p, uint32_t* n_tensors, uint32_t* n_free_dims,
                          uint32_t* n_scalars, uint32_t* n_kernels);
/* Shape contract only (the launch.go:98-130 checks plus rank/dtype/const
 * extents) — no launch, no GPU. */
int tca_program_check(tca_program p, const tca_tensor* tensors, uint32_t n_tensors,
                      const uint32_t* free_dims, uint32_t n_free_dims);
/* Which kernels a launch with these tensors would run: selected[i] = 1 when
 * every launch guard of kernel i holds for the bound dims (a program may
 * carry variants of one kernel specialised on a run-time dim; their guards
 * pick one), and, when `grids` / `blocks` are not NULL, the grid and block
 * each selected kernel would launch with (0 for the others; packed row
 * kernels size their block at launch). Host-only. No counterpart in the
 * reference (its launcher has a single kernel per DSL kernel); for tests and
 * profilers. */
int tca_program_selected(tca_program p, const tca_tensor* tensors, uint32_t n_tensors,
                         const uint32_t* free_dims, uint32_t n_free_dims, uint8_t* selected,
                         uint64_t* grids, uint32_t* blocks, uint32_t n_selected);
/* Checks the contract, then launches, in order on `stream`, every kernel of
 * the program whose launch guards hold. Scalars are passed as doubles in declaration order and converted
 * to their declared types. Locals that live in HBM (and the partials of
 * split reductions) use a workspace the program allocates on first need per
 * stream and keeps until unload: launches of one program on different
 * streams may overlap safely. Thread-safe: calls that use a workspace hold
 * the program's lock from sizing it until their last kernel is queued, so
 * calls on one stream from several threads serialize (a larger launch
 * synchronizes the stream before it replaces the buffer). The first launch
 * that needs a workspace allocates (hipMalloc), so it cannot be captured
 * into a HIP graph. */
int tca_program_launch(tca_program p, const tca_tensor* tensors, uint32_t n_tensors,
                       const uint32_t* free_dims, uint32_t n_free_dims,
                       const double* scalars, uint32_t n_scalars, tca_stream_t stream);
/* Name of kernel i of the program (for profiling), or NULL. */
const char* tca_program_kernel_name(tca_program p, uint32_t i);
/* The argument block kernel `kernel` would be launched with for these
 * tensors, free dims and scalars, written to buf (the HIP kernarg layout:
 * natural alignment, pointers 8 bytes, dims and scalars 4), *size receiving
 * its length. A local in the program's workspace appears as its byte offset
 * from a workspace at address 0. Host-only (no GPU, no launch); the same
 * shape contract as tca_program_launch, TCA_ERR_INVALID when that kernel does
 * not run at these dims or `cap` is too small. No counterpart in the
 * reference; for tests and for tools that launch the code object themselves. */
int tca_program_kernel_args(tca_program p, const tca_tensor* tensors, uint32_t n_tensors,
                            const uint32_t* free_dims, uint32_t n_free_dims, const double* scalars,
                            uint32_t n_scalars, uint32_t kernel, void* buf, size_t cap, size_t* size);
/* The program's plan as this library reads it, printed back in the plan
 * format (one canonical spelling of every record: parsing it again gives the
 * same plan), or NULL for a null program. The text lives until the program
 * is unloaded. No counterpart in the reference (its launcher is emitted
 * code, not data); for tools and tests that inspect or rewrite plans. */
const char* tca_program_plan_text(tca_program p);

/* tca_program_launch without any allocation: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * same contract checks and kernels as tca_program_launch; HBM locals and the
 * partials of split and column reductions live in one 32 MiB scratch array
 * per device, part of this library's device code, whose address
 * tca_rt_init(device) takes (call it first on every device used; a launch
 * with no workspace at these dims uses no scratch and runs without it, one
 * that needs scratch on a device tca_rt_init has not set up fails with
 * TCA_ERR_INVALID). A launch whose workspace at these dims exceeds 32 MiB
 * fails with TCA_ERR_INVALID before anything is queued. Every call on one GPU shares that array and it
 * keeps the last call's contents: calls whose kernels overlap on one GPU
 * (other streams, other threads) race; calls on one stream are ordered. */
int tca_program_launch_noalloc(tca_program p, const tca_tensor* tensors, uint32_t n_tensors,
                               const uint32_t* free_dims, uint32_t n_free_dims, const double* scalars,
                               uint32_t n_scalars, tca_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TCA_RT_H_ */
