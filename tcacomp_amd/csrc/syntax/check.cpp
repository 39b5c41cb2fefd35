// check.cpp — semantic checks and cell resolution for parsed .tca kernels.
//
// Rules and diagnostics follow internal/syntax/semacheck/{semacheck,chain,
// stages,expr,module}.go (design/syntax-design.md §4-§5.1):
//   1  kernel names are unique in a module;          3  @runtime(cxx_path=string);
//   4  the only kernel annotation is @name(cxx=string);
//   5  one namespace for params, dims, dimvars and lets;
//   6  every return-shape dim appears in a parameter shape;
//   7  signature tensors have a shape of rank >= 1;   8  written types agree;
//   9  a binding has one subscript per tensor axis;  10  subscripts are dimvars,
//      each bound to one shape dim;
//   11 `as` clauses: root = permutation of the bound dimvars, reduce = the
//      live axes minus one in order, piped map = the live axes exactly;
//   13 lambda arity; 14 captures are scalar params; 15 scope;
//   17-20 expression typing (no promotion, cast registry, builtins);
//   25 exactly one return, last, naming a let;      26 a chain starts with a
//      root map with >= 1 binding.
// Omitted cells (root/reduce/piped `as`, lambda return and parameter types,
// the let type) are filled in place, as the reference's forward pass does.
#include <map>
#include <set>

#include "syntax.h"

namespace tca {
namespace syntax {

bool ElemOf(const std::string& s, ir::Elem* out) {
  static const std::map<std::string, ir::Elem> k = {
      {"f32", ir::Elem::F32}, {"f16", ir::Elem::F16}, {"bf16", ir::Elem::BF16}, {"i32", ir::Elem::I32},
      {"u32", ir::Elem::U32}, {"i8", ir::Elem::I8},   {"i16", ir::Elem::I16},   {"u8", ir::Elem::U8},
      {"u16", ir::Elem::U16}, {"bool", ir::Elem::Bool},
  };
  auto it = k.find(s);
  if (it == k.end()) return false;
  *out = it->second;
  return true;
}

std::string ShapeDim::Key() const { return symbolic() ? name : "e" + std::to_string(extent); }

namespace {

std::string Join(const std::vector<std::string>& v, const char* sep) {
  std::string s;
  for (size_t i = 0; i < v.size(); ++i) s += (i ? sep : "") + v[i];
  return s;
}
// Go's %v of a []string: [a b c].
std::string ListV(const std::vector<std::string>& v) { return "[" + Join(v, " ") + "]"; }

bool SameDim(const ShapeDim& a, const ShapeDim& b) {
  if (a.symbolic() != b.symbolic()) return false;
  return a.symbolic() ? a.name == b.name : a.extent == b.extent;
}
std::string DimText(const ShapeDim& d) { return d.symbolic() ? d.name : std::to_string(d.extent); }

struct Axis {
  std::string name;
  ShapeDim src;
};
std::vector<std::string> Names(const std::vector<Axis>& axes) {
  std::vector<std::string> n;
  for (const auto& a : axes) n.push_back(a.name);
  return n;
}

bool BinOpOf(const std::string& s, ir::BinOp* op) {
  static const std::map<std::string, ir::BinOp> k = {
      {"||", ir::BinOp::LOr}, {"&&", ir::BinOp::LAnd}, {"|", ir::BinOp::Or},   {"^", ir::BinOp::Xor},
      {"&", ir::BinOp::And},  {"==", ir::BinOp::Eq},   {"!=", ir::BinOp::Ne},  {"<", ir::BinOp::Lt},
      {"<=", ir::BinOp::Le},  {">", ir::BinOp::Gt},    {">=", ir::BinOp::Ge},  {"<<", ir::BinOp::Shl},
      {">>", ir::BinOp::Shr}, {"+", ir::BinOp::Add},   {"-", ir::BinOp::Sub},  {"*", ir::BinOp::Mul},
      {"/", ir::BinOp::Div},  {"%", ir::BinOp::Mod},
  };
  auto it = k.find(s);
  if (it == k.end()) return false;
  *op = it->second;
  return true;
}

struct Scope {
  std::map<std::string, ir::Elem> params, captures;
  std::set<std::string> used_captures;
  bool has_pipe = false;
  ir::Elem pipe = ir::Elem::F32;
};

class Checker {
 public:
  Checker(Kernel* k, std::vector<Diagnostic>* diags) : k_(k), diags_(diags) {}

  void Run() {
    CollectSignature();
    CheckBody();
  }

 private:
  struct DimVarInfo {
    Pos pos;
    ShapeDim src;
    bool set = false;
  };
  struct LetInfo {
    Pos pos;
    ir::Elem elem = ir::Elem::F32;
    std::vector<ShapeDim> shape;
    bool valid = false;
  };

  void Error(const Pos& p, const std::string& msg) {
    Diagnostic d;
    d.pos = p;
    d.msg = msg;
    diags_->push_back(d);
  }
  void Warn(const Pos& p, const std::string& msg) {
    Diagnostic d;
    d.error = false;
    d.pos = p;
    d.msg = msg;
    diags_->push_back(d);
  }

  bool Taken(const std::string& n) const {
    return tensor_params_.count(n) || scalar_params_.count(n) || dims_.count(n) || dimvars_.count(n) || lets_.count(n);
  }

  // ----------------------------------------------------- signature (5-8)
  void CollectSignature() {
    for (auto& p : k_->params) RegisterParam(&p);
    for (const Type& ret : k_->rets) {
      if (ret.tensor) {
        CheckSignatureTensor(ret, "kernel return type");
        for (const auto& d : ret.shape)
          if (d.symbolic() && !dims_.count(d.name))
            Error(ret.pos, "return shape dim \"" + d.name + "\" does not appear in any parameter shape (unbindable, rule 6)");
      } else {
        ir::Elem e;
        if (!ElemOf(ret.elem, &e)) Error(ret.pos, "unknown element type \"" + ret.elem + "\"");
      }
    }
  }

  void RegisterParam(Param* p) {
    if (Taken(p->name)) {
      Error(p->pos, "duplicate name \"" + p->name + "\" (one namespace: params, dims, dimvars, lets must all be distinct, rule 5)");
      return;
    }
    if (p->type.tensor) {
      CheckSignatureTensor(p->type, "parameter " + p->name);
      tensor_params_[p->name] = p;
    } else {
      ir::Elem e;
      if (!ElemOf(p->type.elem, &e)) {
        Error(p->type.pos, "unknown element type \"" + p->type.elem + "\"");
        return;
      }
      scalar_params_[p->name] = e;
    }
  }

  void CheckSignatureTensor(const Type& t, const std::string& what) {
    ir::Elem e;
    if (!ElemOf(t.elem, &e)) Error(t.pos, what + ": unknown element type \"" + t.elem + "\"");
    if (!t.has_shape) {
      Error(t.pos, what + ": tensor shape is required in a kernel signature (rank is always static, §2.4)");
      return;
    }
    if (t.shape.empty()) {
      Error(t.pos, what + ": tensor rank must be ≥ 1 (rule 7)");
      return;
    }
    for (const auto& d : t.shape) {
      if (!d.symbolic()) continue;
      auto it = dims_.find(d.name);
      if (it != dims_.end()) {
        if (!SameDim(it->second, d)) Error(d.pos, "shape dim \"" + d.name + "\" redeclared with a different extent");
        continue;
      }
      dims_[d.name] = d;
    }
  }

  // ------------------------------------------------------- body (25, 26)
  void CheckBody() {
    int returns = 0;
    for (size_t i = 0; i < k_->body.size(); ++i) {
      Stmt& s = k_->body[i];
      switch (s.kind) {
        case StmtKind::DimVar:
          for (const auto& n : s.names) {
            if (Taken(n)) {
              Error(s.pos, "duplicate name \"" + n + "\" (one namespace, rule 5)");
              continue;
            }
            DimVarInfo info;
            info.pos = s.pos;
            dimvars_[n] = info;
          }
          break;
        case StmtKind::Let:
          CheckLet(&s);
          break;
        case StmtKind::Return:
          ++returns;
          if (i + 1 != k_->body.size()) Error(s.pos, "return must be the last statement (rule 25)");
          CheckReturn(s);
          break;
      }
    }
    if (returns == 0) Error(k_->pos, "kernel " + k_->name + " must end with exactly one return (rule 25)");
  }

  void CheckLet(Stmt* l) {
    if (Taken(l->name)) {
      Error(l->pos, "duplicate name \"" + l->name + "\" (a second let of the same name is a duplicate, not a reassignment, rules 5/23)");
      return;
    }
    if (l->chain.empty()) {
      Error(l->pos, "let " + l->name + " requires a stage chain");
      return;
    }
    ir::Elem elem;
    std::vector<Axis> axes;
    LetInfo info;
    info.pos = l->pos;
    if (!ResolveChain(&l->chain, &elem, &axes)) {
      lets_[l->name] = info;
      return;
    }
    std::vector<ShapeDim> out;
    for (const auto& a : axes) out.push_back(a.src);
    if (!l->type.present) {
      l->type.present = true;
      l->type.pos = l->pos;
      l->type.tensor = true;
      l->type.elem = ir::ElemName(elem);
      l->type.has_shape = true;
      l->type.shape = out;
    } else if (!l->type.tensor) {
      Error(l->type.pos, "let " + l->name + " annotation must be a tensor type; a chain always produces a tensor");
      return;
    } else {
      CheckShapeCompat(l->type, elem, out, "let " + l->name);
    }
    info.elem = elem;
    info.shape = out;
    info.valid = true;
    lets_[l->name] = info;
  }

  void CheckShapeCompat(const Type& t, ir::Elem inferred, const std::vector<ShapeDim>& axes, const std::string& what) {
    ir::Elem ann;
    if (!ElemOf(t.elem, &ann)) {
      Error(t.pos, what + ": unknown element type \"" + t.elem + "\"");
      return;
    }
    if (ann != inferred)
      Error(t.pos, what + ": annotated element " + ir::ElemName(ann) + " does not match inferred " + ir::ElemName(inferred) + " (rule 8)");
    if (!t.has_shape) {
      Error(t.pos, what + ": tensor shape is required on a let annotation");
      return;
    }
    if (t.shape.size() != axes.size()) {
      Error(t.pos, what + ": annotated rank " + std::to_string(t.shape.size()) + " does not match the chain's live axes " +
                       std::to_string(axes.size()) + " (rule 26)");
      return;
    }
    for (size_t i = 0; i < t.shape.size(); ++i) {
      const ShapeDim& d = t.shape[i];
      const ShapeDim& want = axes[i];
      const std::string idx = std::to_string(i);
      if (d.symbolic() && want.symbolic()) {
        if (d.name != want.name)
          Error(d.pos, what + ": dim " + idx + " is bound to shape dim \"" + want.name + "\", annotated \"" + d.name + "\" (rule 26)");
      } else if (d.symbolic() != want.symbolic()) {
        Error(d.pos, what + ": dim " + idx + " mixes a symbolic dim with a static extent (rule 26)");
      } else if (d.extent != want.extent) {
        Error(d.pos, what + ": dim " + idx + " has extent " + std::to_string(d.extent) + ", the chain's axis has " +
                         std::to_string(want.extent) + " (rule 26)");
      }
    }
  }

  void CheckReturn(const Stmt& r) {
    if (r.names.size() != k_->rets.size()) {
      Error(r.pos, "return lists " + std::to_string(r.names.size()) + " tensor(s), the kernel signature declares " +
                       std::to_string(k_->rets.size()) + " (rule 25)");
      return;
    }
    std::set<std::string> seen;
    for (size_t i = 0; i < r.names.size(); ++i) {
      const std::string& name = r.names[i];
      const Type& ret = k_->rets[i];
      if (!seen.insert(name).second) {
        Error(r.pos, "return lists \"" + name + "\" twice (rule 25)");
        continue;
      }
      auto it = lets_.find(name);
      if (it == lets_.end()) {
        if (Taken(name))
          Error(r.pos, "return names \"" + name + "\", which is not a let-bound tensor (rule 25)");
        else
          Error(r.pos, "return names unknown let \"" + name + "\" (rule 25)");
        continue;
      }
      const LetInfo& info = it->second;
      if (!info.valid) continue;  // the let's own error names the problem
      if (ret.tensor) {
        ir::Elem ann;
        if (!ElemOf(ret.elem, &ann)) continue;
        if (ann != info.elem) {
          Error(r.pos, "return type mismatch: " + name + " is tensor<" + ir::ElemName(info.elem) + ">, kernel returns tensor<" +
                           ir::ElemName(ann) + "> (rule 8/25)");
          continue;
        }
        CheckShapeCompat(ret, info.elem, info.shape, "return of " + name);
      } else {
        Error(r.pos, "return type mismatch: " + name + " is a tensor, kernel returns scalar " + ret.elem + " (rule 25)");
      }
    }
  }

  // ----------------------------------------------------------- chains
  bool ResolveChain(std::vector<Stage>* chain, ir::Elem* elem, std::vector<Axis>* live) {
    for (size_t i = 0; i < chain->size(); ++i) {
      Stage& st = (*chain)[i];
      if (st.is_map) {
        std::vector<Axis> out;
        const bool ok = i == 0 ? ResolveRootMap(&st, elem, &out) : ResolvePipedMap(&st, elem, *live, &out);
        if (!ok) return false;
        *live = out;
      } else {
        std::vector<Axis> out;
        if (!ResolveReduce(&st, *elem, *live, &out)) return false;
        *live = out;
      }
    }
    return true;
  }

  bool BindOperand(const Binding& b, ir::Elem* elem) {
    std::vector<ShapeDim> shape;
    auto tp = tensor_params_.find(b.tensor);
    auto lt = lets_.find(b.tensor);
    *elem = ir::Elem::F32;
    if (tp != tensor_params_.end()) {
      ElemOf(tp->second->type.elem, elem);
      shape = tp->second->type.shape;
    } else if (lt != lets_.end()) {
      *elem = lt->second.elem;
      shape = lt->second.shape;
    } else {
      if (Taken(b.tensor))
        Error(b.pos, "binding \"" + b.tensor + "\" is not a tensor (rule 9)");
      else
        Error(b.pos, "binding references unknown tensor \"" + b.tensor + "\" (rule 9)");
      return false;
    }
    if (b.dims.size() != shape.size()) {
      Error(b.pos, "binding " + b.tensor + ListV(b.dims) + ": subscript count " + std::to_string(b.dims.size()) +
                       " does not match tensor rank " + std::to_string(shape.size()) + " (structural indexing, rule 9)");
      return false;
    }
    for (size_t i = 0; i < b.dims.size(); ++i) {
      const std::string& dv = b.dims[i];
      auto it = dimvars_.find(dv);
      if (it == dimvars_.end()) {
        if (dims_.count(dv))
          Error(b.pos, "binding " + b.tensor + " uses shape dim \"" + dv + "\" where a dimvar is required (rule 10)");
        else
          Error(b.pos, "binding " + b.tensor + " uses undeclared dimvar \"" + dv + "\" (rule 10)");
        continue;
      }
      if (it->second.set) {
        if (!SameDim(it->second.src, shape[i]))
          Error(b.pos, "dimvar \"" + dv + "\" is bound both to shape dim \"" + DimText(it->second.src) + "\" and \"" +
                           DimText(shape[i]) + "\" (inconsistent structural binding)");
        continue;
      }
      it->second.src = shape[i];
      it->second.set = true;
    }
    return true;
  }

  bool AxisOf(const std::string& n, Axis* a) const {
    auto it = dimvars_.find(n);
    if (it == dimvars_.end() || !it->second.set) return false;
    a->name = n;
    a->src = it->second.src;
    return true;
  }

  bool ResolveRootMap(Stage* st, ir::Elem* out_elem, std::vector<Axis>* axes) {
    if (st->bindings.empty()) {
      Error(st->pos, "a let's chain must begin with a root map holding ≥ 1 tensor binding (rule 26)");
      return false;
    }
    bool ok = true;
    std::vector<ir::Elem> elems;
    for (const auto& b : st->bindings) {
      ir::Elem e;
      ok = BindOperand(b, &e) && ok;
      elems.push_back(e);
    }
    Lambda& lam = st->lambda;
    if (lam.params.size() != st->bindings.size()) {
      Error(lam.pos, "root map lambda has " + std::to_string(lam.params.size()) + " params, want " +
                         std::to_string(st->bindings.size()) + " (one per binding, rule 13)");
      ok = false;
    }
    Scope scope;
    ok = LambdaScope(&lam, elems, ir::Elem::F32, false, &scope) && ok;
    const ir::Elem t = TypeExpr(lam.body.get(), &scope);
    WarnUnusedCaptures(lam, scope);
    ok = CheckLambdaRet(&lam, t) && ok;
    ok = ResolveRootAs(st, axes) && ok;
    *out_elem = t;
    return ok;
  }

  bool ResolvePipedMap(Stage* st, ir::Elem* elem, const std::vector<Axis>& live, std::vector<Axis>* axes) {
    bool ok = true;
    std::vector<ir::Elem> elems;
    for (const auto& b : st->bindings) {
      ir::Elem e;
      ok = BindOperand(b, &e) && ok;
      elems.push_back(e);
    }
    Lambda& lam = st->lambda;
    if (lam.params.size() != 1 + st->bindings.size()) {
      Error(lam.pos, "piped map lambda has " + std::to_string(lam.params.size()) + " params, want " +
                         std::to_string(1 + st->bindings.size()) + " (the pipe value plus one per binding, rule 13)");
      ok = false;
    }
    Scope scope;
    ok = LambdaScope(&lam, elems, *elem, true, &scope) && ok;
    const ir::Elem t = TypeExpr(lam.body.get(), &scope);
    WarnUnusedCaptures(lam, scope);
    ok = CheckLambdaRet(&lam, t) && ok;
    ok = ResolveAsExact(st->pos, st, live, axes) && ok;
    *elem = t;
    return ok;
  }

  bool CheckLambdaRet(Lambda* lam, ir::Elem t) {
    if (lam->ret.empty()) {
      lam->ret = ir::ElemName(t);
      return true;
    }
    ir::Elem want;
    if (!ElemOf(lam->ret, &want) || want != t) {
      Error(lam->pos, "map lambda return annotation " + lam->ret + " does not match inferred " + ir::ElemName(t) + " (rule 8)");
      return false;
    }
    return true;
  }

  bool ResolveReduce(Stage* st, ir::Elem pipe, const std::vector<Axis>& live, std::vector<Axis>* axes) {
    bool ok = true;
    if (st->on_params.size() != 2) {
      Error(st->pos, "reduce requires exactly two on-params (accumulator, element), got " + std::to_string(st->on_params.size()) +
                         " (rule 13)");
      return false;
    }
    ParamSpec& acc = st->on_params[0];
    ParamSpec& el = st->on_params[1];
    if (acc.pipe) {
      Error(acc.pos, "reduce accumulator must be named; " + acc.name + " may only fill the element param (design §7.3)");
      ok = false;
    }
    ir::Elem ret;
    if (!ElemOf(st->ret, &ret) || ret != pipe) {
      Error(st->pos, "reduce return type " + st->ret + " does not match the pipe element type " + ir::ElemName(pipe) +
                         " (homogeneous reducer, rule 8)");
      ok = false;
    }
    CheckParamSpec(&acc, pipe);
    CheckParamSpec(&el, pipe);
    if (!st->init) {
      Error(st->pos, "reduce requires init = ... in v0 (omitted init is the deferred scan-seed feature, §8.1)");
      ok = false;
    } else {
      Scope init_scope;
      init_scope.params = scalar_params_;
      const ir::Elem it = TypeExpr(st->init.get(), &init_scope);
      if (it != pipe) {
        Error(st->init->pos, std::string("reduce init has type ") + ir::ElemName(it) + ", want " + ir::ElemName(pipe) +
                                 " (the homogeneous reducer type)");
        ok = false;
      }
    }
    if (live.size() < 2) {
      Error(st->pos, "reduce requires ≥ 1 surviving axis; reducing (" + ListV(Names(live)) +
                         ") would leave a scalar (fully-reduced results are not v0, §8.4)");
      return false;
    }
    ok = ResolveReduceAs(st, live, axes) && ok;
    Scope scope;
    scope.params[acc.name] = pipe;
    std::string ename = el.name;
    if (el.pipe) {
      ename = "%0";
      scope.has_pipe = true;
      scope.pipe = pipe;
    }
    scope.params[ename] = pipe;
    const ir::Elem bt = TypeExpr(st->body.get(), &scope);
    if (bt != pipe) {
      Error(st->body ? st->body->pos : st->pos, std::string("reduce body has type ") + ir::ElemName(bt) + ", want " +
                                                    ir::ElemName(pipe) + " (homogeneous reducer)");
      ok = false;
    }
    return ok;
  }

  bool LambdaScope(Lambda* lam, const std::vector<ir::Elem>& elems, ir::Elem pipe, bool piped, Scope* scope) {
    bool ok = true;
    for (const auto& n : lam->captures) {
      auto it = scalar_params_.find(n);
      if (it == scalar_params_.end()) {
        if (Taken(n))
          Error(lam->pos, "capture \"" + n + "\" is not a kernel scalar param (no tensor/dim/dimvar capture, rule 14)");
        else
          Error(lam->pos, "capture references unknown name \"" + n + "\" (rule 14)");
        ok = false;
        continue;
      }
      scope->captures[n] = it->second;
    }
    size_t offset = 0;
    if (piped) {
      offset = 1;
      if (!lam->params.empty()) {
        ParamSpec& p0 = lam->params[0];
        CheckParamSpec(&p0, pipe);
        if (p0.pipe) {
          scope->has_pipe = true;
          scope->pipe = pipe;
          scope->params["%0"] = pipe;
        } else {
          scope->params[p0.name] = pipe;
        }
      }
    }
    for (size_t i = offset; i < lam->params.size(); ++i) {
      const size_t bi = i - offset;
      if (bi >= elems.size()) break;  // arity error already reported
      ParamSpec& p = lam->params[i];
      CheckParamSpec(&p, elems[bi]);
      scope->params[p.name] = elems[bi];
    }
    return ok;
  }

  void WarnUnusedCaptures(const Lambda& lam, const Scope& scope) {
    for (const auto& n : lam.captures)
      if (scope.captures.count(n) && !scope.used_captures.count(n)) Warn(lam.pos, "capture \"" + n + "\" is never used");
  }

  void CheckParamSpec(ParamSpec* p, ir::Elem want) {
    if (p->type.empty()) {
      p->type = ir::ElemName(want);
      return;
    }
    ir::Elem got;
    if (!ElemOf(p->type, &got) || got != want)
      Error(p->pos, "param annotation " + p->type + " does not match inferred " + ir::ElemName(want) + " (rule 8)");
  }

  // ------------------------------------------------------------ as (11)
  bool ResolveRootAs(Stage* st, std::vector<Axis>* out) {
    std::vector<Axis> cand;
    std::set<std::string> seen;
    for (const auto& b : st->bindings)
      for (const auto& dv : b.dims) {
        if (!seen.insert(dv).second) continue;
        Axis a;
        if (AxisOf(dv, &a)) cand.push_back(a);
      }
    if (!st->has_as) {
      st->has_as = true;
      st->as = Names(cand);
      *out = cand;
      return true;
    }
    if (st->as.size() != cand.size())
      Error(st->pos, "as (" + ListV(st->as) + ") lists " + std::to_string(st->as.size()) + " axes, the stage binds " +
                         std::to_string(cand.size()) + " (rule 11)");
    std::map<std::string, Axis> by;
    for (const auto& a : cand) by[a.name] = a;
    bool ok = true;
    seen.clear();
    out->clear();
    for (const auto& n : st->as) {
      if (!seen.insert(n).second) {
        Error(st->pos, "as lists \"" + n + "\" twice (rule 11)");
        ok = false;
        continue;
      }
      auto it = by.find(n);
      if (it == by.end()) {
        Error(st->pos, "as references \"" + n + "\", which is not one of the bound dimvars (rule 11)");
        ok = false;
        continue;
      }
      out->push_back(it->second);
    }
    return ok;
  }

  bool ResolveAsExact(const Pos& pos, Stage* st, const std::vector<Axis>& live, std::vector<Axis>* out) {
    const std::vector<std::string> expected = Names(live);
    if (!st->has_as) {
      st->has_as = true;
      st->as = expected;
      *out = live;
      return true;
    }
    if (st->as.size() != expected.size()) {
      Error(pos, "as (" + ListV(st->as) + ") does not match the live axes (" + ListV(expected) + ") in order (rule 11)");
      return false;
    }
    std::map<std::string, Axis> by;
    for (const auto& a : live) by[a.name] = a;
    bool ok = true;
    out->clear();
    for (size_t i = 0; i < st->as.size(); ++i) {
      auto it = by.find(st->as[i]);
      if (it == by.end()) {
        Error(pos, "as references \"" + st->as[i] + "\", which is not a live axis (rule 11)");
        ok = false;
        continue;
      }
      if (st->as[i] != expected[i]) {
        Error(pos, "as (" + ListV(st->as) + ") must equal the live axes (" + ListV(expected) + ") exactly, in order (rule 11)");
        ok = false;
      }
      out->push_back(it->second);
    }
    return ok;
  }

  bool ResolveReduceAs(Stage* st, const std::vector<Axis>& live, std::vector<Axis>* out) {
    if (!st->has_as) {
      st->has_as = true;
      out->assign(live.begin(), live.end() - 1);
      st->as = Names(*out);
      return true;
    }
    if (st->as.size() != live.size() - 1) {
      Error(st->pos, "reduce as (" + ListV(st->as) + ") must list the live axes (" + ListV(Names(live)) +
                         ") minus exactly one (the reduced axis, rule 11)");
      return false;
    }
    std::map<std::string, Axis> by;
    for (const auto& a : live) by[a.name] = a;
    bool ok = true;
    std::set<std::string> seen;
    out->clear();
    for (const auto& n : st->as) {
      if (!seen.insert(n).second) {
        Error(st->pos, "reduce as lists \"" + n + "\" twice (rule 11)");
        ok = false;
        continue;
      }
      auto it = by.find(n);
      if (it == by.end()) {
        Error(st->pos, "reduce as references \"" + n + "\", which is not a live axis (rule 11)");
        ok = false;
        continue;
      }
      out->push_back(it->second);
    }
    size_t oi = 0;
    for (const auto& a : live)
      if (oi < out->size() && (*out)[oi].name == a.name) ++oi;
    if (oi != out->size()) {
      Error(st->pos, "reduce as (" + ListV(st->as) + ") must preserve the live axes' order (" + ListV(Names(live)) + ", rule 11)");
      ok = false;
    }
    return ok;
  }

  // -------------------------------------------------- expressions (15-20)
  ir::Elem TypeExpr(const Expr* e, Scope* s) {
    if (e == nullptr) return ir::Elem::F32;  // the parser reported it
    switch (e->kind) {
      case ExprKind::Lit:
        switch (e->lit) {
          case LitKind::Int: return ir::Elem::I32;
          case LitKind::Uint: return ir::Elem::U32;
          case LitKind::Float: return ir::Elem::F32;
          case LitKind::Bool: return ir::Elem::Bool;
        }
        return ir::Elem::F32;
      case ExprKind::Name: {
        auto p = s->params.find(e->text);
        if (p != s->params.end()) return p->second;
        auto c = s->captures.find(e->text);
        if (c != s->captures.end()) {
          s->used_captures.insert(e->text);
          return c->second;
        }
        Error(e->pos, "unknown name \"" + e->text +
                          "\" in expression (rule 15: only lambda params, captures, and kernel scalar params in init are visible)");
        return ir::Elem::F32;
      }
      case ExprKind::Pipe:
        if (!s->has_pipe) {
          Error(e->pos, "%0 has no pipe slot here (only piped maps and reduce bodies carry one)");
          return ir::Elem::F32;
        }
        return s->pipe;
      case ExprKind::Binary: return TypeBinary(e, s);
      case ExprKind::Unary: return TypeUnary(e, s);
      case ExprKind::Select: {
        const ir::Elem ct = TypeExpr(e->kids[0].get(), s);
        if (ct != ir::Elem::Bool)
          Error(e->kids[0] ? e->kids[0]->pos : e->pos,
                std::string("select condition must be bool, got ") + ir::ElemName(ct) + " (rule 18)");
        const ir::Elem tt = TypeExpr(e->kids[1].get(), s);
        const ir::Elem ft = TypeExpr(e->kids[2].get(), s);
        if (tt != ft)
          Error(e->pos, std::string("select branches must have identical types, got ") + ir::ElemName(tt) + " vs " +
                            ir::ElemName(ft) + " (rule 18)");
        return tt;
      }
      case ExprKind::Call: {
        pkg::BuiltinSig sig;
        if (!pkg::LookupBuiltin(e->text, &sig)) {
          Error(e->pos, "function " + e->text + " is not a registered pure scalar builtin (rule 20)");
          return ir::Elem::F32;
        }
        if (static_cast<int>(e->kids.size()) != sig.arity)
          Error(e->pos, "builtin " + e->text + " expects " + std::to_string(sig.arity) + " argument(s), got " +
                            std::to_string(e->kids.size()) + " (rule 20)");
        for (size_t i = 0; i < e->kids.size(); ++i) {
          const ir::Elem t = TypeExpr(e->kids[i].get(), s);
          if (static_cast<int>(e->kids.size()) == sig.arity && t != sig.arg)
            Error(e->kids[i] ? e->kids[i]->pos : e->pos, "call " + e->text + ": argument " + std::to_string(i) + " must be " +
                                                             ir::ElemName(sig.arg) + ", got " + ir::ElemName(t) + " (rule 20)");
        }
        return sig.result;
      }
      case ExprKind::Cast: {
        const ir::Elem from = TypeExpr(e->kids[0].get(), s);
        ir::Elem to;
        if (!ElemOf(e->cast_to, &to)) {
          Error(e->pos, "unknown cast target \"" + e->cast_to + "\"");
          return ir::Elem::F32;
        }
        if (from == to) {
          Error(e->pos, std::string("cast: redundant cast to ") + ir::ElemName(to) + " (rule 19)");
          return to;
        }
        if (!ir::CastPairOK(from, to))
          Error(e->pos, std::string("cast: pair ") + ir::ElemName(from) + " -> " + ir::ElemName(to) +
                            " is not in the v0 cast registry (arithmetic-to-arithmetic only, rule 19)");
        return to;
      }
    }
    return ir::Elem::F32;
  }

  ir::Elem TypeBinary(const Expr* e, Scope* s) {
    ir::BinOp op;
    if (!BinOpOf(e->text, &op)) {
      Error(e->pos, "unknown operator \"" + e->text + "\"");
      return ir::Elem::F32;
    }
    const ir::Elem lt = TypeExpr(e->kids[0].get(), s);
    const ir::Elem rt = TypeExpr(e->kids[1].get(), s);
    const std::string name = ir::BinOpName(op);
    if (lt != rt) {
      Error(e->pos, name + ": operand types differ (" + ir::ElemName(lt) + " vs " + ir::ElemName(rt) +
                        "); implicit promotions are not supported (rule 17)");
      return lt;
    }
    switch (op) {
      case ir::BinOp::LOr:
      case ir::BinOp::LAnd:
        if (lt != ir::Elem::Bool) Error(e->pos, name + ": operands must be bool, got " + ir::ElemName(lt) + " (rule 17)");
        return ir::Elem::Bool;
      case ir::BinOp::Eq: case ir::BinOp::Ne: case ir::BinOp::Lt:
      case ir::BinOp::Le: case ir::BinOp::Gt: case ir::BinOp::Ge:
        return ir::Elem::Bool;
      case ir::BinOp::Mod: case ir::BinOp::Shl: case ir::BinOp::Shr:
      case ir::BinOp::And: case ir::BinOp::Or: case ir::BinOp::Xor:
        if (!ir::IsInt(lt))
          Error(e->pos, name + ": operands must have the same integer type, got " + ir::ElemName(lt) + " (rule 17)");
        return lt;
      default:
        if (!ir::IsArith(lt))
          Error(e->pos, name + ": operands must have the same arithmetic type, got " + ir::ElemName(lt) + " (rule 17)");
        return lt;
    }
  }

  ir::Elem TypeUnary(const Expr* e, Scope* s) {
    const ir::Elem t = TypeExpr(e->kids[0].get(), s);
    const std::string& op = e->text;
    if (op == "!") {
      if (t != ir::Elem::Bool) Error(e->pos, std::string("lnot: operand must be bool, got ") + ir::ElemName(t) + " (rule 17)");
    } else if (op == "~") {
      if (!ir::IsInt(t)) Error(e->pos, std::string("not: operand must have an integer type, got ") + ir::ElemName(t) + " (rule 17)");
    } else if (op == "-" || op == "+") {
      if (!ir::IsArith(t))
        Error(e->pos, std::string(op == "-" ? "neg" : "pos") + ": operand must have an arithmetic type, got " +
                          ir::ElemName(t) + " (rule 17)");
    } else {
      Error(e->pos, "unknown unary operator \"" + op + "\"");
    }
    return t;
  }

  Kernel* k_;
  std::vector<Diagnostic>* diags_;
  std::map<std::string, Param*> tensor_params_;
  std::map<std::string, ir::Elem> scalar_params_;
  std::map<std::string, ShapeDim> dims_;
  std::map<std::string, DimVarInfo> dimvars_;
  std::map<std::string, LetInfo> lets_;
};

void ModuleError(std::vector<Diagnostic>* diags, const Pos& p, const std::string& msg) {
  Diagnostic d;
  d.pos = p;
  d.msg = msg;
  diags->push_back(d);
}

}  // namespace

void Check(Kernel* k, std::vector<Diagnostic>* diags) { Checker(k, diags).Run(); }

void CheckModule(const Module& m, std::vector<Diagnostic>* diags) {
  std::set<std::string> seen;
  for (const auto& k : m.kernels) {
    if (!seen.insert(k.name).second) ModuleError(diags, k.pos, "duplicate kernel name " + k.name + " (rule 1)");
  }
  if (m.has_runtime) {
    const KeyedConst* cxx = nullptr;
    for (const auto& a : m.runtime.args) {
      if (a.key == "cxx_path")
        cxx = &a;
      else
        ModuleError(diags, a.pos, "unknown @runtime key " + a.key + " (want cxx_path, rule 3)");
    }
    if (cxx == nullptr)
      ModuleError(diags, m.runtime.pos, "@runtime requires cxx_path=\"...\" (rule 3)");
    else if (cxx->kind != ConstKind::String)
      ModuleError(diags, cxx->pos, "@runtime cxx_path must be a string literal (rule 3)");
  }
  for (const auto& k : m.kernels) {
    for (const auto& ann : k.anns) {
      if (ann.name == "name") {
        if (ann.args.size() != 1 || ann.args[0].key != "cxx") {
          ModuleError(diags, ann.pos, "@name accepts exactly {cxx=string} (rule 4)");
          continue;
        }
        if (ann.args[0].kind != ConstKind::String)
          ModuleError(diags, ann.args[0].pos, "@name cxx must be a string literal (rule 4)");
      } else {
        ModuleError(diags, ann.pos, "unknown annotation @" + ann.name + " (rule 4: the v0 registry holds only @name{cxx})");
      }
    }
  }
}

}  // namespace syntax
}  // namespace tca
