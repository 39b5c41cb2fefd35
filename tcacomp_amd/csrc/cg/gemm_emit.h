// gemm_emit.h — recognition and emission of the MFMA contraction family.
//
// A chain is a dense K-contraction exactly when (the reference's gemm
// corpus: testing/kernels/llm/gemm.tca:7-22, mlp.tca, qk_score.tca):
//   - the root map has two tensor operands and its body is l*r, or
//     cast<f32>(l)*cast<f32>(r) for bf16 operands;
//   - exactly one reduce, over the last `as` axis k, with init +0.0f and
//     combiner acc+now (either order);
//   - the store writes out[m][n] (f32) over the two remaining axes, or
//     out[b][m][n] with a leading batch axis b (one contraction per b);
//   - one operand is indexed [m][k], the other [k][n] or [n][k], each
//     optionally led by the batch axis (an operand without it is shared by
//     every batch);
//   - an optional piped map becomes the MFMA epilogue (scalars and tensor
//     operands indexed by m and/or n).
// Anything else falls back to another family; the match never guesses.
#ifndef TCA_CG_GEMM_EMIT_H_
#define TCA_CG_GEMM_EMIT_H_

#include <sstream>
#include <string>
#include <vector>

#include "ir.h"

namespace tca {
namespace cg {

struct GemmMatch {
  int a_op = -1, b_op = -1;  // root operand indices
  int m = -1, n = -1, k = -1;
  int batch = -1;                          // leading batch axis, or -1
  bool a_batched = false, b_batched = false;  // operand led by the batch axis
  bool b_nk = false;                       // B indexed [n][k]
  ir::Elem in = ir::Elem::F32;
};

// One kernel of a contraction: its symbol is the nest's symbol + suffix.
struct GemmKernel {
  std::string suffix;
  uint32_t block = 256, lds = 0;
  std::vector<std::string> grid, when, unless;
  std::vector<std::string> extra_args;  // plan args after the signature's ("ptr <local>")
  std::string split;                    // the plan's split record, if any
  std::string detail;
};

struct GemmEmitted {
  std::vector<GemmKernel> kernels;
  std::vector<std::string> extra_dims;     // plan-only dims: "<name> <extent>"
  std::vector<std::string> extra_tensors;  // plan-only locals: "<name> <dtype> local <rank> <dims...>"
};

// Output planes of at most kGemmSmallMax elements (M*N) take the small-tile
// kernel (32x32 tiles, K split over the waves of a workgroup and, when the
// tiles are few, over workgroups); larger ones the 128/256 tile kernels.
constexpr uint64_t kGemmSmallMax = 1ull << 20;

// `nest` names the partial scratch of the small kernel's K split
// (__gemmpart<nest>); `small` false leaves the small kernel out.
bool MatchGemm(const ir::Graph& g, const ir::Chain& c, GemmMatch* m);
bool EmitGemm(const ir::Graph& g, const ir::Chain& c, const GemmMatch& m, const std::string& symbol,
              const std::string& signature, int nest, bool small, int* counter, std::ostringstream* src,
              GemmEmitted* out, std::string* err);

namespace detail {
std::string CType(ir::Elem e);
std::string ExtentExpr(const ir::Graph& g, int d);
}  // namespace detail

}  // namespace cg
}  // namespace tca

#endif  // TCA_CG_GEMM_EMIT_H_
