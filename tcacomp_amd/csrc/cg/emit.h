// emit.h — the HIP code-generation plugin: the compile-time seam.
//
// Reference: `func Emit(g *ir.Graph, opts cg.Options) (*cg.Result, error)`
// (internal/cg/cxx/emit.go:85; types internal/cg/cg.go:17-64). Same contract:
// a deterministic, read-only consumer of the finished graph that fails
// closed with an error and never aborts. The result carries the HIP source
// (one code object per program), the launch plan the runtime interprets,
// and the hipcc argv that builds the code object (the reference emits a
// CMakeLists.txt for nvcc, internal/cg/cxx/launch.go:162-186; the compiler
// itself never runs the toolchain).
#ifndef TCA_CG_EMIT_H_
#define TCA_CG_EMIT_H_

#include <string>
#include <vector>

#include "ir.h"

namespace tca {
namespace cg {

enum class Family {
  Elementwise,  // E: no real reduction; vectorised flat streaming
  Row,          // R/F: reductions (and maps) over the contiguous last axis of a fused nest
  Stream,       // S: the same nests with a run-time (or register-exceeding) row length, streamed
  Col,          // C: reductions over a non-contiguous axis (the reduced axis outside the contiguous one)
  Gemm,         // G: dense K-contraction on MFMA
  Generic,      // X: one thread per output element, sequential folds
  Seg           // chained reductions in one kernel: a row reduction into a local, folded over rows per block
};

const char* FamilyName(Family f);

struct Options {
  std::string kernel_name;       // symbol prefix; empty = the graph's name
  std::string target = "gfx950"; // the only supported target
  bool comments = true;
  bool allow_fused = true;       // false: every chain lowers to the generic family
  bool allow_gemm = true;
  // The contractions' small-tile kernels for output planes of M*N <= 2^20.
  bool allow_gemm_split = true;
  // Two passes of a nest that read one input fused into one read where the
  // arithmetic allows (online softmax normaliser, pairwise mean/variance).
  bool allow_pass_fusion = true;
  // Geometry knobs (power-of-two values; 0 = default). Row family: target
  // 16-byte vectors per lane and row operand (lanes per row follow from it).
  // Elementwise family: 16-byte vectors per thread and operand.
  int row_vectors_per_lane = 0;
  int elementwise_unroll = 0;
};

struct KernelInfo {
  std::string symbol;
  Family family = Family::Generic;
  std::vector<int> chains;  // statement indices lowered into this kernel
  std::string detail;       // geometry summary
};

struct Result {
  std::string source;               // <name>.hip
  std::string plan;                 // launch plan text (rt/plan.h format)
  std::vector<std::string> hipcc;   // argv after "hipcc" (the build recipe)
  std::vector<KernelInfo> kernels;
  std::string report;               // one line per kernel: family + geometry
};

// Runs the HIR-equivalent passes the HIP path needs (dead-chain elimination,
// nest fusion of chains with identical iteration order, local placement),
// classifies every nest into a kernel family and emits it.
bool Emit(const ir::Graph& g, const Options& opts, Result* out, std::string* err);

// Flags every emitted kernel is compiled with. Contraction is OFF so
// `a*x + y` is a multiply then an add on both the device and the CPU oracle;
// fused multiply-add exists only where the program calls fmaf. Denormals are
// kept (IEEE, no FTZ), division and sqrt correctly rounded.
std::vector<std::string> DeviceFlags(const std::string& target);

}  // namespace cg
}  // namespace tca

#endif  // TCA_CG_EMIT_H_
