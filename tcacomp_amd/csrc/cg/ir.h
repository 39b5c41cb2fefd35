// ir.h — the map+reduce program IR the builder constructs and the HIP
// emitter lowers.
//
// The reference keeps a sea-of-nodes SSA graph (internal/ir/doc.go:1-129)
// scheduled into an AST CFG for its CUDA emitter. The HIP path only needs
// what the reference's HIR window produces (internal/pipeline/pipeline.go:
// 41-52): typed, de-duplicated statement chains
//     iter(dims) | map(operands, fn) as(perm) | reduce(init, fn)* |
//     [map(operands, fn) as(live)] | store(tensor, axes)
// with each lambda body a pure scalar expression DAG. This IR holds exactly
// that: a structured list of chains over an arena of hash-consed scalar
// expressions (hash-consing is the value numbering the reference's GVN pass
// performs on lambda bodies, internal/opt/gvn/gvn.go:1-60).
#ifndef TCA_CG_IR_H_
#define TCA_CG_IR_H_

#include <cstdint>
#include <string>
#include <vector>

namespace tca {
namespace ir {

// Element types; numbering shared with the C ABI (TCA_F32 ...).
enum class Elem : int { F32 = 0, F16, BF16, I32, U32, I8, I16, U8, U16, Bool };

const char* ElemName(Elem e);
bool IsFloat(Elem e);
bool IsInt(Elem e);
bool IsArith(Elem e);
size_t ElemBytes(Elem e);
// The v0 cast registry (internal/ir/types.go:60-62): arithmetic to
// arithmetic, never a redundant cast.
bool CastPairOK(Elem from, Elem to);

enum class Op { Error, Const, Param, Scalar, Bin, Un, Select, Cast, Call };

enum class BinOp { Add, Sub, Mul, Div, Mod, Eq, Ne, Lt, Le, Gt, Ge, LAnd, LOr, And, Or, Xor, Shl, Shr };
enum class UnOp { Neg, Pos, LNot, Not };

const char* BinOpName(BinOp op);
const char* UnOpName(UnOp op);

struct Expr {
  Op op = Op::Error;
  Elem type = Elem::F32;
  double value = 0.0;   // Const
  int index = -1;       // Param: owning lambda-param slot; Scalar: scalar index
  int code = 0;         // BinOp / UnOp
  std::string text;     // Call: builtin name; Param: parameter name; Error: message
  std::vector<int> args;
};

struct Dim {
  std::string name;
  uint64_t extent = 0;  // 0 = dynamic
};

struct Tensor {
  std::string name;
  Elem elem = Elem::F32;
  std::vector<int> dims;
  bool local = false;
};

struct Scalar {
  std::string name;
  Elem elem = Elem::F32;
};

// One structural access t[axes...]: subscript i binds dim i of t.
struct Operand {
  int tensor = -1;
  std::vector<int> axes;
};

struct Lambda {
  std::vector<int> params;  // expr ids of Op::Param nodes
  int body = -1;
};

struct MapStage {
  std::vector<Operand> ops;
  Lambda fn;
  std::vector<int> as;  // axis order after this stage
};

struct ReduceStage {
  int init = -1;  // expr id
  Lambda fn;      // (acc, now)
  int axis = -1;  // the axis reduced away (last live axis)
};

struct Chain {
  std::vector<int> iters;
  MapStage root;
  std::vector<ReduceStage> reduces;
  bool has_piped = false;
  MapStage piped;  // operands follow the piped value (params[0])
  int store_tensor = -1;
  std::vector<int> store_axes;
  // The reference builder's construction-time IDs (pkg/builder.go:310-318):
  // Stmt() reserves the statement's ID and an end-node ID before any of the
  // chain's nodes exist. Only the canonical print reads them.
  uint64_t stmt_id = 0;
  uint64_t ret_id = 0;

  // Live axes at the store, in order.
  std::vector<int> LiveAxes() const;
};

struct Graph {
  std::string name;
  std::vector<Dim> dims;
  std::vector<Tensor> tensors;  // parameters and locals, declaration order
  std::vector<Scalar> scalars;
  std::vector<Expr> exprs;
  std::vector<Chain> chains;
  std::vector<int> outputs;  // non-local stored tensors, first-store order
  uint64_t end_stmt_id = 0;  // the end node's statement ID: the first output chain's reserved one

  bool IsStored(int tensor) const;
  bool IsRead(int tensor) const;
};

// The reference's canonical print (internal/ir/print.go:34-57): one
// `statement #ID:` block per stored chain, stages in the doc notation
//   iter(@m, @k) -> map(x[@m][@k], lambda(v): v) as (@m, @k) |
//   reduce(init=0.0, %0, lambda(acc, now): acc + now) |
//   memstore(%out[@m], %0)
// then the end node `return %out, ...`. Statement IDs follow the reference
// builder's construction-time numbering (Chain::stmt_id).
std::string PrintReference(const Graph& g);
// This build's structural dump: every declaration with its type and extent,
// each chain's operand axes, reduced axes and lambda bodies in SSA form. Two
// programs are the same program iff their dumps are equal.
std::string Print(const Graph& g);
// Go's strconv.FormatFloat(v, 'g', -1, 32) (shortest round-trip float32
// digits; %e when the decimal exponent is < -4 or >= 6), the spelling the
// reference's printer uses for float constants before appending ".0".
std::string FormatFloat32Go(double v);
// Structural verifier (the reference's ir.Verify role, internal/ir/verify.go:58).
bool Verify(const Graph& g, std::string* err);
// Type of a binary operation's result, given its (equal) operand type.
Elem BinResult(BinOp op, Elem operand);

}  // namespace ir
}  // namespace tca

#endif  // TCA_CG_IR_H_
