// builder.cpp — see builder.h. Error texts follow the reference's wording
// (pkg/builder.go, pkg/chain.go, pkg/expr.go) so diagnostics read the same.
#include "builder.h"

#include <cstring>
#include <set>
#include <sstream>

namespace tca {
namespace pkg {

// The pure scalar-builtin registry (internal/ir/builtins.go:25-33).
bool LookupBuiltin(const std::string& name, BuiltinSig* sig) {
  static const std::map<std::string, BuiltinSig> kBuiltins = {
      {"expf", {1, ir::Elem::F32, ir::Elem::F32}},  {"logf", {1, ir::Elem::F32, ir::Elem::F32}},
      {"sqrtf", {1, ir::Elem::F32, ir::Elem::F32}}, {"rsqrtf", {1, ir::Elem::F32, ir::Elem::F32}},
      {"fabsf", {1, ir::Elem::F32, ir::Elem::F32}}, {"tanhf", {1, ir::Elem::F32, ir::Elem::F32}},
      {"sinf", {1, ir::Elem::F32, ir::Elem::F32}},  {"cosf", {1, ir::Elem::F32, ir::Elem::F32}},
      {"fminf", {2, ir::Elem::F32, ir::Elem::F32}}, {"fmaxf", {2, ir::Elem::F32, ir::Elem::F32}},
      {"fmaf", {3, ir::Elem::F32, ir::Elem::F32}},  {"umin", {2, ir::Elem::U32, ir::Elem::U32}},
      {"umax", {2, ir::Elem::U32, ir::Elem::U32}},
  };
  auto it = kBuiltins.find(name);
  if (it == kBuiltins.end()) return false;
  *sig = it->second;
  return true;
}

namespace {

// Lambda-parameter names (pkg/chain.go:83-87).
const char* kRootNames[] = {"l", "r", "s", "t", "u", "w", "x", "y", "z"};
const char* kPipedNames[] = {"v", "w", "x", "y", "z"};

enum class Class { Arith, Int, Bool, Cmp };

Class ClassOf(ir::BinOp op) {
  switch (op) {
    case ir::BinOp::Add:
    case ir::BinOp::Sub:
    case ir::BinOp::Mul:
    case ir::BinOp::Div:
      return Class::Arith;
    case ir::BinOp::Eq:
    case ir::BinOp::Ne:
    case ir::BinOp::Lt:
    case ir::BinOp::Le:
    case ir::BinOp::Gt:
    case ir::BinOp::Ge:
      return Class::Cmp;
    case ir::BinOp::LAnd:
    case ir::BinOp::LOr:
      return Class::Bool;
    default:
      return Class::Int;
  }
}

}  // namespace

const char* StageName(int stage) {
  static const char* kNames[] = {"Stmt",   "Iter",       "Map(root)",  "RootAs", "MidChain", "Reduce",
                                 "AfterReduce", "Map(piped)", "AfterMap", "Tail",   "Stored",  "broken"};
  if (stage < 0 || stage > Builder::kBroken) return "?";
  return kNames[stage];
}

Builder::Builder(std::string name) { g_.name = std::move(name); }

bool Builder::Fail(const std::string& msg) {
  last_err_ = msg;
  return false;
}

void Builder::NoteDecl(const std::string& msg) {
  if (decl_err_.empty()) decl_err_ = msg;
}

void Builder::Defer(ChainState& c, const std::string& msg) {
  if (c.err.empty()) c.err = msg;
}

// The first error recorded anywhere on the builder or chain (pkg/chain.go:50).
bool Builder::Pending(ChainState& c) {
  if (!decl_err_.empty()) return Fail(decl_err_);
  if (!c.err.empty()) return Fail(c.err);
  return true;
}

bool Builder::CheckChain(int chain, Stage want, const char* rung) {
  if (chain < 0 || chain >= static_cast<int>(chains_.size()))
    return Fail(std::string(rung) + ": unknown statement chain");
  ChainState& c = chains_[chain];
  if (chain != open_chain_) return Fail(std::string(rung) + ": statement chain is no longer open");
  if (c.stage != want)
    return Fail(std::string(rung) + ": not legal after " + StageName(c.stage) + " (chain rungs: " +
                "Stmt -> Iter -> Map -> As -> Reduce* -> [Map -> As] -> Store)");
  return true;
}

bool Builder::CheckDim(int d, const std::string& what, std::string* msg) const {
  if (d < 0 || d >= static_cast<int>(g_.dims.size())) {
    *msg = what + ": dim is not declared in this builder";
    return false;
  }
  return true;
}

int Builder::Dim(const std::string& name, int64_t extent) {
  if (final_) NoteDecl("dim " + name + ": builder already finalized by Build");
  if (extent < 0) NoteDecl("dim " + name + ": extent must be >= 0 (0 = dynamic), got " + std::to_string(extent));
  if (extent > 0xffffffffll) NoteDecl("dim " + name + ": extent exceeds the u32 index domain");
  if (dim_by_name_.count(name)) NoteDecl("dim " + name + ": already declared");
  ir::Dim d;
  d.name = name;
  d.extent = extent > 0 ? static_cast<uint64_t>(extent) : 0;
  g_.dims.push_back(d);
  const int id = static_cast<int>(g_.dims.size()) - 1;
  dim_by_name_[name] = id;
  Take(1);
  return id;
}

int Builder::Tensor(const std::string& name, ir::Elem elem, const std::vector<int>& dims) {
  if (final_) NoteDecl("tensor " + name + ": builder already finalized by Build");
  if (tensor_by_name_.count(name)) NoteDecl("tensor " + name + ": already declared");
  if (dims.size() > 8) NoteDecl("tensor " + name + ": rank exceeds 8");
  std::vector<int> ds;
  for (int d : dims) {
    std::string msg;
    if (!CheckDim(d, "tensor " + name, &msg)) {
      NoteDecl(msg);
      continue;
    }
    ds.push_back(d);
  }
  ir::Tensor t;
  t.name = name;
  t.elem = elem;
  t.dims = ds;
  g_.tensors.push_back(t);
  const int id = static_cast<int>(g_.tensors.size()) - 1;
  tensor_by_name_[name] = id;
  Take(1);
  return id;
}

int Builder::Local(const std::string& name, ir::Elem elem, const std::vector<int>& dims) {
  if (final_) NoteDecl("local " + name + ": builder already finalized by Build");
  if (dims.empty()) NoteDecl("local " + name + ": must be a tensor type");
  const int id = Tensor(name, elem, dims);  // one ID, as the MemNew node
  g_.tensors[id].local = true;
  Take(1);  // the extent const (pkg/builder.go:270)
  return id;
}

int Builder::ScalarParam(const std::string& name, ir::Elem elem) {
  if (final_) NoteDecl("scalar " + name + ": builder already finalized by Build");
  if (scalar_by_name_.count(name)) NoteDecl("scalar " + name + ": already declared");
  ir::Scalar s;
  s.name = name;
  s.elem = elem;
  g_.scalars.push_back(s);
  const int idx = static_cast<int>(g_.scalars.size()) - 1;
  scalar_by_name_[name] = idx;
  ir::Expr e;
  e.op = ir::Op::Scalar;
  e.type = elem;
  e.index = idx;
  const int id = Intern(e);
  scalar_expr_.push_back(id);
  Take(1);
  return id;
}

int Builder::Intern(const ir::Expr& e) {
  std::ostringstream k;
  uint64_t bits = 0;
  std::memcpy(&bits, &e.value, sizeof(bits));
  k << static_cast<int>(e.op) << "|" << static_cast<int>(e.type) << "|" << bits << "|" << e.index << "|" << e.code
    << "|" << e.text;
  for (int a : e.args) k << "|" << a;
  auto it = intern_.find(k.str());
  if (it != intern_.end()) return it->second;
  g_.exprs.push_back(e);
  const int id = static_cast<int>(g_.exprs.size()) - 1;
  intern_[k.str()] = id;
  return id;
}

int Builder::ErrorExpr(const std::string& msg) {
  ir::Expr e;
  e.op = ir::Op::Error;
  e.text = msg;
  g_.exprs.push_back(e);
  return static_cast<int>(g_.exprs.size()) - 1;
}

int Builder::NewParam(const std::string& name, ir::Elem type) {
  ir::Expr e;
  e.op = ir::Op::Param;
  e.type = type;
  e.text = name;
  e.index = static_cast<int>(g_.exprs.size());
  g_.exprs.push_back(e);
  return static_cast<int>(g_.exprs.size()) - 1;
}

bool Builder::ExprOK(int id) const {
  return id >= 0 && id < static_cast<int>(g_.exprs.size()) && g_.exprs[id].op != ir::Op::Error;
}

std::string Builder::ExprError(int id) const {
  if (id < 0 || id >= static_cast<int>(g_.exprs.size())) return "expression handle is not from this builder";
  if (g_.exprs[id].op == ir::Op::Error) return g_.exprs[id].text;
  return "";
}

ir::Elem Builder::ExprType(int id) const {
  if (!ExprOK(id)) return ir::Elem::F32;
  return g_.exprs[id].type;
}

uint64_t Builder::ScalarRefs(const std::vector<int>& ids) const {
  uint64_t n = 0;
  for (int id : ids)
    if (id >= 0 && id < static_cast<int>(g_.exprs.size()) && g_.exprs[id].op == ir::Op::Scalar) ++n;
  return n;
}

int Builder::FirstError(const std::vector<int>& ids) const {
  for (int id : ids) {
    if (id < 0 || id >= static_cast<int>(g_.exprs.size())) return -2;
    if (g_.exprs[id].op == ir::Op::Error) return id;
  }
  return -1;
}

int Builder::Const(ir::Elem elem, double value) {
  ir::Expr e;
  e.op = ir::Op::Const;
  e.type = elem;
  if (elem == ir::Elem::F32) value = static_cast<double>(static_cast<float>(value));
  if (elem == ir::Elem::Bool) value = value != 0.0 ? 1.0 : 0.0;
  e.value = value;
  Take(1);
  return Intern(e);
}

int Builder::Bin(ir::BinOp op, int x, int y) {
  const char* name = ir::BinOpName(op);
  int fe = FirstError({x, y});
  if (fe == -2) return ErrorExpr(std::string(name) + ": operands come from a different builder");
  if (fe >= 0) return fe;
  const ir::Elem tx = g_.exprs[x].type, ty = g_.exprs[y].type;
  if (tx != ty)
    return ErrorExpr(std::string(name) + ": operand types differ (" + ir::ElemName(tx) + " vs " + ir::ElemName(ty) +
                     "); implicit promotions are not supported");
  switch (ClassOf(op)) {
    case Class::Arith:
      if (!ir::IsArith(tx))
        return ErrorExpr(std::string(name) + ": operands must have the same arithmetic type, got " + ir::ElemName(tx));
      break;
    case Class::Int:
      if (!ir::IsInt(tx))
        return ErrorExpr(std::string(name) + ": operands must have the same integer type, got " + ir::ElemName(tx));
      break;
    case Class::Bool:
      if (tx != ir::Elem::Bool) return ErrorExpr(std::string(name) + ": operands must be bool, got " + ir::ElemName(tx));
      break;
    case Class::Cmp:
      break;
  }
  ir::Expr e;
  e.op = ir::Op::Bin;
  e.code = static_cast<int>(op);
  e.type = ir::BinResult(op, tx);
  e.args = {x, y};
  Take(1 + ScalarRefs(e.args));
  return Intern(e);
}

int Builder::Un(ir::UnOp op, int x) {
  const char* name = ir::UnOpName(op);
  int fe = FirstError({x});
  if (fe == -2) return ErrorExpr(std::string(name) + ": operand comes from a different builder");
  if (fe >= 0) return fe;
  const ir::Elem t = g_.exprs[x].type;
  bool ok = true;
  std::string want;
  switch (op) {
    case ir::UnOp::Neg:
    case ir::UnOp::Pos:
      ok = ir::IsArith(t);
      want = "an arithmetic type";
      break;
    case ir::UnOp::LNot:
      ok = t == ir::Elem::Bool;
      want = "bool";
      break;
    case ir::UnOp::Not:
      ok = ir::IsInt(t);
      want = "an integer type";
      break;
  }
  if (!ok) return ErrorExpr(std::string(name) + ": operand must have " + want + ", got " + ir::ElemName(t));
  ir::Expr e;
  e.op = ir::Op::Un;
  e.code = static_cast<int>(op);
  e.type = t;
  e.args = {x};
  Take(1 + ScalarRefs(e.args));
  return Intern(e);
}

int Builder::Select(int cond, int a, int b) {
  int fe = FirstError({cond, a, b});
  if (fe == -2) return ErrorExpr("select: operands come from different builders");
  if (fe >= 0) return fe;
  if (g_.exprs[cond].type != ir::Elem::Bool)
    return ErrorExpr(std::string("select: condition must be bool, got ") + ir::ElemName(g_.exprs[cond].type));
  if (g_.exprs[a].type != g_.exprs[b].type)
    return ErrorExpr(std::string("select: branches must have identical types, got ") +
                     ir::ElemName(g_.exprs[a].type) + " vs " + ir::ElemName(g_.exprs[b].type));
  ir::Expr e;
  e.op = ir::Op::Select;
  e.type = g_.exprs[a].type;
  e.args = {cond, a, b};
  Take(1 + ScalarRefs(e.args));
  return Intern(e);
}

int Builder::Cast(int x, ir::Elem to) {
  int fe = FirstError({x});
  if (fe == -2) return ErrorExpr("cast: operand comes from a different builder");
  if (fe >= 0) return fe;
  const ir::Elem from = g_.exprs[x].type;
  if (from == to) return ErrorExpr(std::string("cast: redundant cast to ") + ir::ElemName(to));
  if (!ir::CastPairOK(from, to))
    return ErrorExpr(std::string("cast: pair ") + ir::ElemName(from) + " -> " + ir::ElemName(to) +
                     " is not in the v0 cast registry (arithmetic-to-arithmetic only)");
  ir::Expr e;
  e.op = ir::Op::Cast;
  e.type = to;
  e.args = {x};
  Take(1 + ScalarRefs(e.args));
  return Intern(e);
}

int Builder::Call(const std::string& name, const std::vector<int>& args) {
  BuiltinSig sig;
  if (!LookupBuiltin(name, &sig)) return ErrorExpr("function " + name + " is not a registered pure scalar builtin");
  if (static_cast<int>(args.size()) != sig.arity)
    return ErrorExpr("builtin " + name + " expects " + std::to_string(sig.arity) + " argument(s), got " +
                     std::to_string(args.size()));
  int fe = FirstError(args);
  if (fe == -2) return ErrorExpr("call " + name + ": argument comes from a different builder");
  if (fe >= 0) return fe;
  for (size_t i = 0; i < args.size(); ++i) {
    if (g_.exprs[args[i]].type != sig.arg)
      return ErrorExpr("call " + name + ": argument " + std::to_string(i) + " must be " + ir::ElemName(sig.arg) +
                       ", got " + ir::ElemName(g_.exprs[args[i]].type));
  }
  ir::Expr e;
  e.op = ir::Op::Call;
  e.type = sig.result;
  e.text = name;
  e.args = args;
  Take(1 + ScalarRefs(e.args));
  return Intern(e);
}

int Builder::Stmt() {
  if (final_) NoteDecl("stmt: builder already finalized by Build");
  chains_.emplace_back();
  open_chain_ = static_cast<int>(chains_.size()) - 1;
  chains_.back().chain.stmt_id = Take(1);
  chains_.back().chain.ret_id = Take(1);
  return open_chain_;
}

int Builder::ChainStage(int chain) const {
  if (chain < 0 || chain >= static_cast<int>(chains_.size())) return -1;
  return chains_[chain].stage;
}

void Builder::Iter(int chain, const std::vector<int>& dims) {
  if (!CheckChain(chain, kFresh, "iter")) {
    if (chain >= 0 && chain < static_cast<int>(chains_.size())) Defer(chains_[chain], last_err_);
    return;
  }
  ChainState& c = chains_[chain];
  if (dims.empty()) Defer(c, "iter: an iteration cluster needs at least one dim");
  std::set<int> seen;
  for (int d : dims) {
    std::string msg;
    if (!CheckDim(d, "iter", &msg)) {
      Defer(c, msg);
      continue;
    }
    if (seen.count(d)) {
      Defer(c, "iter: dim @" + g_.dims[d].name + " is listed twice");
      continue;
    }
    seen.insert(d);
    c.chain.iters.push_back(d);
    c.live.push_back(d);
  }
  c.stage = kRootMap;
}

bool Builder::CheckOperands(ChainState& c, const std::vector<ir::Operand>& ops, std::vector<ir::Elem>* elems) {
  for (const auto& op : ops) {
    if (op.tensor < 0 || op.tensor >= static_cast<int>(g_.tensors.size()))
      return Fail("map: tensor is not declared in this builder");
    const ir::Tensor& t = g_.tensors[op.tensor];
    if (op.axes.size() != t.dims.size())
      return Fail("map: operand " + t.name + " has " + std::to_string(op.axes.size()) + " subscripts for rank " +
                  std::to_string(t.dims.size()) + " (structural indexing)");
    for (size_t i = 0; i < op.axes.size(); ++i) {
      std::string msg;
      if (!CheckDim(op.axes[i], "map operand " + t.name, &msg)) return Fail(msg);
      if (op.axes[i] != t.dims[i])
        return Fail("map: operand " + t.name + " subscript " + std::to_string(i) + " binds @" +
                    g_.dims[op.axes[i]].name + ", but dim " + std::to_string(i) + " of " + t.name + " is @" +
                    g_.dims[t.dims[i]].name + " (structural indexing binds subscripts positionally)");
      bool live = false;
      for (int l : c.live) live |= (l == op.axes[i]);
      if (!live)
        return Fail("map: operand " + t.name + " binds @" + g_.dims[op.axes[i]].name +
                    ", which is not a live axis at this point of the chain");
    }
    if (t.local) {
      bool stored = false;
      for (const auto& other : chains_)
        if (other.stage == kStored && other.chain.store_tensor == op.tensor) stored = true;
      if (!stored) return Fail("map: local " + t.name + " is read before any statement stores it");
    }
    elems->push_back(t.elem);
  }
  return true;
}

bool Builder::MapBegin(int chain, const std::vector<ir::Operand>& ops, std::vector<int>* params) {
  if (chain < 0 || chain >= static_cast<int>(chains_.size())) return Fail("map: unknown statement chain");
  ChainState& c = chains_[chain];
  const bool piped = c.stage == kAfterReduce;
  if (!CheckChain(chain, piped ? kAfterReduce : kRootMap, "map")) return false;
  if (!Pending(c)) {
    c.stage = kBroken;
    return false;
  }
  if (!piped && c.chain.iters.empty()) {
    c.stage = kBroken;
    return Fail("map: the iteration cluster is empty");
  }
  std::vector<ir::Elem> elems;
  if (piped) elems.push_back(c.elem);
  if (!CheckOperands(c, ops, &elems)) {
    c.stage = kBroken;
    return false;
  }
  const size_t n = elems.size();
  const size_t cap = piped ? 5 : 9;
  if (n > cap && n != 1) {
    c.stage = kBroken;
    return Fail("map: " + std::to_string(n) + " operands exceed the v0 lambda-name table (" + std::to_string(cap) + ")");
  }
  params->clear();
  for (size_t i = 0; i < n; ++i) {
    std::string pname = n == 1 ? "v" : (piped ? kPipedNames[i] : kRootNames[i]);
    params->push_back(NewParam(pname, elems[i]));
  }
  c.pending_ops = ops;
  c.pending_params = *params;
  c.stage = piped ? kPipedOpen : kRootMapOpen;
  Take(ops.size() + 2 * n);  // operand references; each parameter and its reference
  return true;
}

bool Builder::MapEnd(int chain, int body) {
  if (chain < 0 || chain >= static_cast<int>(chains_.size())) return Fail("map: unknown statement chain");
  ChainState& c = chains_[chain];
  const bool piped = c.stage == kPipedOpen;
  if (!CheckChain(chain, piped ? kPipedOpen : kRootMapOpen, "map")) return false;
  if (!ExprOK(body)) {
    c.stage = kBroken;
    return Fail(ExprError(body));
  }
  ir::MapStage& st = piped ? c.chain.piped : c.chain.root;
  st.ops = c.pending_ops;
  st.fn.params = c.pending_params;
  st.fn.body = body;
  c.stage = piped ? kAfterMap : kRootAs;
  Take(ScalarRefs({body}));
  return true;
}

void Builder::As(int chain, const std::vector<int>& dims) {
  if (chain < 0 || chain >= static_cast<int>(chains_.size())) return;
  ChainState& c = chains_[chain];
  const bool piped = c.stage == kAfterMap;
  if (!CheckChain(chain, piped ? kAfterMap : kRootAs, "as")) {
    Defer(c, last_err_);
    c.stage = kBroken;
    return;
  }
  const std::string what = piped ? "piped map" : "root map";
  Take((dims.empty() ? 0 : 1) + 3);  // As (when axes are listed), lambda, map, iteration cluster
  for (int d : dims) {
    std::string msg;
    if (!CheckDim(d, what + " as", &msg)) {
      Defer(c, msg);
      c.stage = kBroken;
      return;
    }
  }
  if (!piped) {
    // A permutation of the iteration cluster (pkg/chain.go:265-298).
    if (dims.size() != c.chain.iters.size()) {
      Defer(c, what + ": as lists " + std::to_string(dims.size()) + " axes, the iteration cluster has " +
                   std::to_string(c.chain.iters.size()));
    } else {
      std::set<int> seen, iters(c.chain.iters.begin(), c.chain.iters.end());
      std::string dups, missing;
      for (int d : dims) {
        if (seen.count(d)) dups += (dups.empty() ? "@" : ", @") + g_.dims[d].name;
        seen.insert(d);
      }
      for (int it : c.chain.iters)
        if (!seen.count(it)) missing += (missing.empty() ? "@" : ", @") + g_.dims[it].name;
      if (!dups.empty() || !missing.empty())
        Defer(c, what + ": as must list every live axis exactly once; duplicated: " + dups + "; missing: " + missing);
    }
    c.chain.root.as = dims;
    c.live = dims;
    c.elem = g_.exprs[c.chain.root.fn.body].type;
    c.stage = kMid;
  } else {
    // Exactly the live axes in order (pkg/chain.go:300-322).
    if (dims.size() != c.live.size()) {
      Defer(c, what + ": as lists " + std::to_string(dims.size()) + " axes, " + std::to_string(c.live.size()) +
                   " are live at this point of the chain (producer's as minus reduced axes, in order)");
    } else {
      for (size_t i = 0; i < dims.size(); ++i) {
        if (dims[i] != c.live[i]) {
          Defer(c, what + ": as position " + std::to_string(i) + " binds @" + g_.dims[dims[i]].name +
                       ", the incoming axis order requires @" + g_.dims[c.live[i]].name +
                       " (fused maps cannot reorder axes in v0)");
          break;
        }
      }
    }
    c.chain.has_piped = true;
    c.chain.piped.as = dims;
    c.elem = g_.exprs[c.chain.piped.fn.body].type;
    c.stage = kTail;
  }
}

bool Builder::ReduceBegin(int chain, int init, int* acc, int* now) {
  if (chain < 0 || chain >= static_cast<int>(chains_.size())) return Fail("reduce: unknown statement chain");
  ChainState& c = chains_[chain];
  const Stage want = c.stage == kAfterReduce ? kAfterReduce : kMid;
  if (!CheckChain(chain, want, "reduce")) return false;
  if (!Pending(c)) {
    c.stage = kBroken;
    return false;
  }
  if (!ExprOK(init)) {
    c.stage = kBroken;
    return Fail(ExprError(init));
  }
  if (c.live.empty()) {
    c.stage = kBroken;
    return Fail("reduce: no live axis left to reduce");
  }
  if (g_.exprs[init].type != c.elem) {
    c.stage = kBroken;
    return Fail(std::string("reduce: homogeneous reducer violated: init has type ") +
                ir::ElemName(g_.exprs[init].type) + ", the piped value has element type " + ir::ElemName(c.elem));
  }
  *acc = NewParam("acc", c.elem);
  *now = NewParam("now", c.elem);
  c.pending_params = {*acc, *now};
  c.pending_init = init;
  c.stage = kReduceOpen;
  Take(4);
  return true;
}

bool Builder::ReduceEnd(int chain, int body) {
  if (!CheckChain(chain, kReduceOpen, "reduce")) return false;
  ChainState& c = chains_[chain];
  if (!ExprOK(body)) {
    c.stage = kBroken;
    return Fail(ExprError(body));
  }
  if (g_.exprs[body].type != c.elem) {
    c.stage = kBroken;
    return Fail(std::string("reduce: homogeneous reducer violated: combiner returns ") +
                ir::ElemName(g_.exprs[body].type) + ", want " + ir::ElemName(c.elem));
  }
  ir::ReduceStage r;
  r.init = c.pending_init;
  r.fn.params = c.pending_params;
  r.fn.body = body;
  r.axis = c.live.back();
  c.live.pop_back();
  c.chain.reduces.push_back(r);
  c.stage = kAfterReduce;
  Take(ScalarRefs({r.init, body}) + 3);  // keyed init attribute, lambda, reduce
  return true;
}

bool Builder::Store(int chain, int tensor, const std::vector<int>& axes) {
  if (chain < 0 || chain >= static_cast<int>(chains_.size())) return Fail("store: unknown statement chain");
  ChainState& c = chains_[chain];
  if (c.stage != kAfterReduce && c.stage != kTail && c.stage != kMid) {
    CheckChain(chain, kTail, "store");
    if (last_err_.empty() || chain == open_chain_)
      Fail(std::string("store: not legal after ") + StageName(c.stage));
    return false;
  }
  if (chain != open_chain_) return Fail("store: statement chain is no longer open");
  if (!Pending(c)) {
    c.stage = kBroken;
    return false;
  }
  if (tensor < 0 || tensor >= static_cast<int>(g_.tensors.size())) {
    c.stage = kBroken;
    return Fail("store: tensor is not declared in this builder");
  }
  const ir::Tensor& t = g_.tensors[tensor];
  if (axes.size() != t.dims.size()) {
    c.stage = kBroken;
    return Fail("store: " + t.name + " has rank " + std::to_string(t.dims.size()) + ", got " +
                std::to_string(axes.size()) + " index axes");
  }
  for (size_t i = 0; i < axes.size(); ++i) {
    std::string msg;
    if (!CheckDim(axes[i], "store " + t.name, &msg)) {
      c.stage = kBroken;
      return Fail(msg);
    }
    if (axes[i] != t.dims[i]) {
      c.stage = kBroken;
      return Fail("store: index " + std::to_string(i) + " of " + t.name + " binds @" + g_.dims[axes[i]].name +
                  ", but dim " + std::to_string(i) + " of " + t.name + " is @" + g_.dims[t.dims[i]].name);
    }
    bool live = false;
    for (int l : c.live) live |= (l == axes[i]);
    if (!live) {
      c.stage = kBroken;
      return Fail("store: @" + g_.dims[axes[i]].name + " is not a live axis at this point of the chain");
    }
  }
  if (axes.size() != c.live.size()) {
    c.stage = kBroken;
    return Fail("store: " + t.name + " binds " + std::to_string(axes.size()) + " of the " +
                std::to_string(c.live.size()) + " live axes; every live axis must be stored (single-owner store)");
  }
  if (c.elem != t.elem) {
    c.stage = kBroken;
    return Fail(std::string("store: value of type ") + ir::ElemName(c.elem) + " cannot be stored into " + t.name +
                " of element type " + ir::ElemName(t.elem));
  }
  c.chain.store_tensor = tensor;
  c.chain.store_axes = axes;
  c.stage = kStored;
  open_chain_ = -1;
  Take(1);
  if (!t.local) {
    bool seen = false;
    for (int o : g_.outputs) seen |= (o == tensor);
    if (!seen) {
      // The end node takes the reserved ID of the first chain that stores
      // an output (pkg/builder.go:351-356).
      if (g_.outputs.empty()) g_.end_stmt_id = c.chain.ret_id;
      g_.outputs.push_back(tensor);
    }
  }
  return true;
}

bool Builder::Build(ir::Graph* out) {
  if (!decl_err_.empty()) return Fail(decl_err_);
  if (open_chain_ >= 0) {
    return Fail("build: statement chain (statement #" + std::to_string(open_chain_) + ") was never stored");
  }
  final_ = true;
  ir::Graph g = g_;
  g.chains.clear();
  for (const auto& c : chains_)
    if (c.stage == kStored) g.chains.push_back(c.chain);
  std::string err;
  if (!ir::Verify(g, &err)) return Fail(err);
  *out = g;
  return true;
}

}  // namespace pkg
}  // namespace tca
