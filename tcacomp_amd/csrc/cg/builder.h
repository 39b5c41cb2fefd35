// builder.h — the DSL builder core: declarations, typed scalar expressions
// and the statement-chain typestate, with deferred errors.
//
// Reference: pkg/builder.go:35-370 (Builder, Dim, Tensor, Local,
// ScalarParam, Stmt, Build), pkg/chain.go:16-552 (rung table and checks),
// pkg/expr.go:34-341 (typed operators, literals, Select, Cast, Call).
// Semantics kept from the reference:
//   - declaration violations (duplicate names, negative extents, foreign
//     handles) are recorded and surface at the next error-returning rung or
//     at Build; the library never aborts;
//   - structural indexing: subscript i of an operand binds dim i of its
//     tensor and must be a live axis;
//   - root `as` is a permutation of the iteration cluster; a reduce drops the
//     last live axis; a piped map's `as` is exactly the live axes in order;
//   - reducers are homogeneous (init, piped value, both combiner parameters
//     and the result share one type);
//   - no implicit promotions in expressions.
// One extension over the reference v0 rungs (its wall W1,
// design/RELEASE-v0.0.0.md:118-162): a chain may Store directly after the
// root map's `as` (an elementwise chain), and locals of any rank may be
// stored and read (they live in registers when the consumer is fused with
// the producer, otherwise in an HBM workspace).
#ifndef TCA_CG_BUILDER_H_
#define TCA_CG_BUILDER_H_

#include <map>
#include <string>
#include <vector>

#include "ir.h"

namespace tca {
namespace pkg {

// One registered pure scalar builtin: arity, the (shared) argument type and
// the result type.
struct BuiltinSig {
  int arity;
  ir::Elem arg, result;
};
bool LookupBuiltin(const std::string& name, BuiltinSig* sig);

class Builder {
 public:
  explicit Builder(std::string name);

  // Declarations. Return handles (indices); violations are deferred.
  int Dim(const std::string& name, int64_t extent);
  int Tensor(const std::string& name, ir::Elem elem, const std::vector<int>& dims);
  int Local(const std::string& name, ir::Elem elem, const std::vector<int>& dims);
  int ScalarParam(const std::string& name, ir::Elem elem);  // returns an expr id

  // Expressions. Return an expr id; a type error yields an Error node whose
  // message surfaces at the rung consuming it.
  int Const(ir::Elem elem, double value);
  int Bin(ir::BinOp op, int x, int y);
  int Un(ir::UnOp op, int x);
  int Select(int cond, int a, int b);
  int Cast(int x, ir::Elem to);
  int Call(const std::string& name, const std::vector<int>& args);
  bool ExprOK(int id) const;
  std::string ExprError(int id) const;
  ir::Elem ExprType(int id) const;

  // Statement chains (Stmt() -> Iter -> Map -> As -> Reduce* -> [Map -> As] -> Store).
  int Stmt();
  void Iter(int chain, const std::vector<int>& dims);
  // Starts a map stage (root or piped, by the chain's position) and returns
  // its lambda parameter expressions; MapEnd supplies the body.
  bool MapBegin(int chain, const std::vector<ir::Operand>& ops, std::vector<int>* params);
  bool MapEnd(int chain, int body);
  void As(int chain, const std::vector<int>& dims);
  bool ReduceBegin(int chain, int init, int* acc, int* now);
  bool ReduceEnd(int chain, int body);
  bool Store(int chain, int tensor, const std::vector<int>& axes);

  // Verifies and hands out the finished graph.
  bool Build(ir::Graph* out);

  const std::string& Error() const { return last_err_; }
  const ir::Graph& graph() const { return g_; }
  int ChainStage(int chain) const;

  // Chain stages (the typestate of pkg/chain.go:16-26).
  enum Stage {
    kFresh,        // StmtIter
    kRootMap,      // RootMap: after Iter
    kRootMapOpen,  // inside the root map's lambda
    kRootAs,       // RootAs: root lambda built, waiting for As
    kMid,          // MidChain: after root As (Reduce; Store is the extension)
    kReduceOpen,   // inside a reducer lambda
    kAfterReduce,  // AfterReduce
    kPipedOpen,    // inside the piped map's lambda
    kAfterMap,     // AfterMap: waiting for As
    kTail,         // Tail
    kStored,       // Stored (terminal)
    kBroken        // a rung failed; only Stmt() can continue
  };

 private:
  struct ChainState {
    Stage stage = kFresh;
    ir::Chain chain;
    std::vector<int> live;
    ir::Elem elem = ir::Elem::F32;  // pipe element type
    std::vector<ir::Operand> pending_ops;
    std::vector<int> pending_params;
    int pending_init = -1;
    std::string err;
  };

  bool Fail(const std::string& msg);
  void NoteDecl(const std::string& msg);
  void Defer(ChainState& c, const std::string& msg);
  bool Pending(ChainState& c);
  bool CheckChain(int chain, Stage want, const char* rung);
  bool CheckDim(int d, const std::string& what, std::string* msg) const;
  int Intern(const ir::Expr& e);
  int ErrorExpr(const std::string& msg);
  int NewParam(const std::string& name, ir::Elem type);
  bool CheckOperands(ChainState& c, const std::vector<ir::Operand>& ops, std::vector<ir::Elem>* elems);
  int FirstError(const std::vector<int>& ids) const;

  // The reference builder's graph-ID counter (internal/ir/node.go:176-183),
  // advanced by the number of nodes each reference call allocates, so the
  // print can number statements as the reference does: params 1 each, a
  // local 2 (extent const, MemNew), an expression node 1 plus 1 per lazy
  // scalar-param reference it materializes (pkg/expr.go:43-52), Stmt 2
  // reserved IDs, a map 1 per operand reference and 2 per lambda parameter
  // and then As + lambda + map + iteration cluster, a reduce 4 for its
  // parameters and then attribute + lambda + reduce, a store 1.
  uint64_t Take(uint64_t n) {
    const uint64_t id = ref_next_;
    ref_next_ += n;
    return id;
  }
  uint64_t ScalarRefs(const std::vector<int>& ids) const;
  uint64_t ref_next_ = 1;

  ir::Graph g_;
  std::map<std::string, int> dim_by_name_, tensor_by_name_, scalar_by_name_;
  std::map<std::string, int> intern_;
  std::vector<int> scalar_expr_;  // scalar index -> expr id
  std::vector<ChainState> chains_;
  int open_chain_ = -1;
  bool final_ = false;
  std::string decl_err_;
  std::string last_err_;
};

const char* StageName(int stage);

}  // namespace pkg
}  // namespace tca

#endif  // TCA_CG_BUILDER_H_
