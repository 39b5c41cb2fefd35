// lower.cpp — replays a checked kernel through the builder rungs.
//
// Follows internal/syntax/build/build.go:36-671 (the per-kernel driver):
// declaration order (dims by first appearance, tensor params, the returned
// lets as output tensors in return order, scalar params), every other let as a Local, and
// per chain: the iteration/root-as order with the surviving axes first and
// the reduced axes last in reverse reduce order, operands indexed by their
// tensor's own dims (structural indexing), lambda parameters bound by
// position, the store over the target's dims. The checker has already
// enforced the rules; failures here are rung errors, reported with the
// kernel and let names.
#include <map>

#include "syntax.h"

namespace tca {
namespace syntax {

namespace {

using Scope = std::map<std::string, int>;  // name -> builder expr id

class Driver {
 public:
  Driver(const Kernel& k, pkg::Builder* b) : k_(k), b_(*b) {}

  bool Run(std::string* err) {
    std::vector<const Stmt*> lets;
    std::vector<std::string> ret_names;
    for (const auto& s : k_.body) {
      if (s.kind == StmtKind::Let) lets.push_back(&s);
      if (s.kind == StmtKind::Return) ret_names = s.names;
    }
    std::vector<const Stmt*> out_lets;  // in return order
    for (const auto& rn : ret_names) {
      const Stmt* found = nullptr;
      for (const Stmt* l : lets)
        if (l->name == rn) found = l;
      if (found == nullptr) return Fail(err, "frontend: kernel " + k_.name + ": return names no let");
      out_lets.push_back(found);
    }
    if (out_lets.empty()) return Fail(err, "frontend: kernel " + k_.name + ": return names no let");
    auto is_output = [&](const Stmt* l) {
      for (const Stmt* o : out_lets)
        if (o == l) return true;
      return false;
    };

    // Dims in first-appearance order: parameters, then lets.
    auto declare = [&](const Type& t) {
      for (const auto& d : t.shape) {
        const std::string key = d.Key();
        if (dims_.count(key)) continue;
        dims_[key] = b_.Dim(key, d.symbolic() ? 0 : static_cast<int64_t>(d.extent));
      }
    };
    for (const auto& p : k_.params)
      if (p.type.tensor) declare(p.type);
    for (const Stmt* l : lets) {
      if (!l->type.present || !l->type.tensor)
        return Fail(err, "frontend: kernel " + k_.name + ": let " + l->name + " has no inferred tensor type (run semacheck first)");
      declare(l->type);
    }
    // Tensor parameters, then the output, then scalars (the launcher order).
    for (const auto& p : k_.params) {
      if (!p.type.tensor) continue;
      ir::Elem e;
      if (!ElemOf(p.type.elem, &e))
        return Fail(err, "frontend: kernel " + k_.name + ": param " + p.name + " has unmappable element type \"" + p.type.elem + "\"");
      DeclareTensor(p.name, e, p.type, false);
    }
    for (const Stmt* out_let : out_lets) {
      ir::Elem e;
      if (!ElemOf(out_let->type.elem, &e))
        return Fail(err, "frontend: kernel " + k_.name + ": output has unmappable element type \"" + out_let->type.elem + "\"");
      DeclareTensor(out_let->name, e, out_let->type, false);
    }
    for (const auto& p : k_.params) {
      if (p.type.tensor) continue;
      ir::Elem e;
      if (!ElemOf(p.type.elem, &e))
        return Fail(err, "frontend: kernel " + k_.name + ": scalar " + p.name + " has unmappable element type \"" + p.type.elem + "\"");
      scalars_[p.name] = b_.ScalarParam(p.name, e);
    }
    for (const Stmt* l : lets) {
      if (!is_output(l)) {
        ir::Elem e;
        if (!ElemOf(l->type.elem, &e))
          return Fail(err, "frontend: kernel " + k_.name + ": let " + l->name + " has unmappable element type \"" + l->type.elem + "\"");
        DeclareTensor(l->name, e, l->type, true);
      }
      if (!LowerChain(*l, err)) return false;
    }
    return true;
  }

 private:
  static bool Fail(std::string* err, const std::string& msg) {
    *err = msg;
    return false;
  }

  void DeclareTensor(const std::string& name, ir::Elem e, const Type& t, bool local) {
    std::vector<int> handles;
    for (const auto& d : t.shape) handles.push_back(dims_[d.Key()]);
    tensors_[name] = local ? b_.Local(name, e, handles) : b_.Tensor(name, e, handles);
    tensor_dims_[name] = handles;
  }

  std::string Where(const Stmt& l) const { return "frontend: kernel " + k_.name + ": let " + l.name + ": "; }

  // The iteration and root-as order (build.go relocate): surviving root-as
  // axes in their order, then each reduce's dropped axis, first reduce last.
  bool Relocate(const Stmt& l, std::vector<std::string>* order, std::string* err) {
    const Stage& root = l.chain[0];
    std::vector<std::string> live = root.as, reduced_order;
    std::map<std::string, bool> reduced;
    for (size_t i = 1; i < l.chain.size(); ++i) {
      const Stage& st = l.chain[i];
      if (st.is_map) continue;
      if (!st.has_as) return Fail(err, Where(l) + "a reduce's as clause was not inferred (run semacheck first)");
      std::map<std::string, bool> kept;
      for (const auto& dv : st.as) kept[dv] = true;
      std::vector<std::string> dropped;
      for (const auto& dv : live)
        if (!kept.count(dv)) dropped.push_back(dv);
      if (dropped.size() != 1)
        return Fail(err, Where(l) + "reduce drops " + std::to_string(dropped.size()) + " axes, want exactly 1 (run semacheck first)");
      reduced[dropped[0]] = true;
      reduced_order.push_back(dropped[0]);
      live = st.as;
    }
    order->clear();
    for (const auto& dv : root.as)
      if (!reduced.count(dv)) order->push_back(dv);
    for (auto it = reduced_order.rbegin(); it != reduced_order.rend(); ++it) order->push_back(*it);
    return true;
  }

  std::vector<ir::Operand> Operands(const std::vector<Binding>& bindings) {
    std::vector<ir::Operand> ops;
    for (const auto& b : bindings) {
      ir::Operand o;
      o.tensor = tensors_[b.tensor];
      o.axes = tensor_dims_[b.tensor];
      ops.push_back(o);
    }
    return ops;
  }

  bool LowerChain(const Stmt& l, std::string* err) {
    const Stage& root = l.chain[0];
    if (!root.is_map) return Fail(err, Where(l) + "the chain must open with a map stage");
    if (!root.has_as) return Fail(err, Where(l) + "the root map's as clause was not inferred (run semacheck first)");
    dimvars_.clear();
    for (const auto& b : root.bindings) {
      auto td = tensor_dims_.find(b.tensor);
      if (td == tensor_dims_.end()) return Fail(err, Where(l) + "binding names unknown tensor \"" + b.tensor + "\"");
      if (b.dims.size() != td->second.size())
        return Fail(err, Where(l) + "binding " + b.tensor + " has " + std::to_string(b.dims.size()) + " subscripts, want " +
                             std::to_string(td->second.size()) + " (run semacheck first)");
      for (size_t i = 0; i < b.dims.size(); ++i) {
        auto prev = dimvars_.find(b.dims[i]);
        if (prev != dimvars_.end() && prev->second != td->second[i])
          return Fail(err, Where(l) + "dimvar @" + b.dims[i] + " binds two distinct shape dims");
        dimvars_[b.dims[i]] = td->second[i];
      }
    }
    std::vector<std::string> order;
    if (!Relocate(l, &order, err)) return false;
    std::vector<int> iters;
    for (const auto& dv : order) {
      auto it = dimvars_.find(dv);
      if (it == dimvars_.end()) return Fail(err, Where(l) + "dimvar @" + dv + " is not bound by the root map");
      iters.push_back(it->second);
    }

    // Root map.
    const int chain = b_.Stmt();
    b_.Iter(chain, iters);
    std::vector<int> params;
    if (!b_.MapBegin(chain, Operands(root.bindings), &params)) return Fail(err, Where(l) + "map: " + b_.Error());
    int body = LowerExpr(root.lambda.body.get(), LambdaScope(root.lambda, params));
    if (!expr_err_.empty()) return Fail(err, Where(l) + expr_err_);
    if (!b_.MapEnd(chain, body)) return Fail(err, Where(l) + "map: " + b_.Error());
    b_.As(chain, iters);

    bool reduced = false, piped = false;
    for (size_t i = 1; i < l.chain.size(); ++i) {
      const Stage& st = l.chain[i];
      if (!st.is_map) {
        if (piped) return Fail(err, Where(l) + "a reduction cannot follow a piped map (pkg v0 rung shape)");
        const int init = st.init ? LowerExpr(st.init.get(), ScalarScope()) : b_.Const(ir::Elem::F32, 0.0);
        if (!expr_err_.empty()) return Fail(err, Where(l) + expr_err_);
        int acc = -1, now = -1;
        if (!b_.ReduceBegin(chain, init, &acc, &now)) return Fail(err, Where(l) + "reduce: " + b_.Error());
        Scope scope = ScalarScope();
        if (!st.on_params.empty()) scope[SpecName(st.on_params[0])] = acc;
        if (st.on_params.size() > 1) scope[SpecName(st.on_params[1])] = now;
        body = LowerExpr(st.body.get(), scope);
        if (!expr_err_.empty()) return Fail(err, Where(l) + expr_err_);
        if (!b_.ReduceEnd(chain, body)) return Fail(err, Where(l) + "reduce: " + b_.Error());
        reduced = true;
        continue;
      }
      if (piped) return Fail(err, Where(l) + "v0 pkg rungs admit at most one piped map per chain");
      if (!reduced) return Fail(err, Where(l) + "a piped map requires a preceding reduction (pkg v0 rung shape)");
      if (!st.has_as) return Fail(err, Where(l) + "the piped map's as clause was not inferred (run semacheck first)");
      params.clear();
      if (!b_.MapBegin(chain, Operands(st.bindings), &params)) return Fail(err, Where(l) + "piped map: " + b_.Error());
      body = LowerExpr(st.lambda.body.get(), LambdaScope(st.lambda, params));
      if (!expr_err_.empty()) return Fail(err, Where(l) + expr_err_);
      if (!b_.MapEnd(chain, body)) return Fail(err, Where(l) + "piped map: " + b_.Error());
      std::vector<int> as;
      for (const auto& dv : st.as) as.push_back(dimvars_[dv]);
      b_.As(chain, as);
      piped = true;
    }
    // A chain with no reduction stores straight after the root map (the
    // builder's elementwise extension).
    if (!b_.Store(chain, tensors_[l.name], tensor_dims_[l.name])) return Fail(err, Where(l) + "store: " + b_.Error());
    return true;
  }

  static std::string SpecName(const ParamSpec& p) { return p.pipe ? "%0" : p.name; }

  Scope ScalarScope() const { return Scope(scalars_.begin(), scalars_.end()); }

  Scope LambdaScope(const Lambda& lam, const std::vector<int>& args) const {
    Scope s = ScalarScope();
    for (size_t i = 0; i < lam.params.size() && i < args.size(); ++i) s[SpecName(lam.params[i])] = args[i];
    return s;
  }

  int LowerExpr(const Expr* e, const Scope& s) {
    if (!expr_err_.empty()) return -1;
    if (e == nullptr) {
      expr_err_ = "missing expression";
      return -1;
    }
    switch (e->kind) {
      case ExprKind::Lit:
        switch (e->lit) {
          case LitKind::Int: return b_.Const(ir::Elem::I32, static_cast<double>(e->ival));
          case LitKind::Uint: return b_.Const(ir::Elem::U32, static_cast<double>(e->ival));
          case LitKind::Float: return b_.Const(ir::Elem::F32, static_cast<double>(e->fval));
          case LitKind::Bool: return b_.Const(ir::Elem::Bool, e->bval ? 1.0 : 0.0);
        }
        break;
      case ExprKind::Name: {
        auto it = s.find(e->text);
        if (it != s.end()) return it->second;
        expr_err_ = "unknown name \"" + e->text + "\" in expression (run semacheck first)";
        return -1;
      }
      case ExprKind::Pipe: {
        auto it = s.find("%0");
        if (it != s.end()) return it->second;
        expr_err_ = "pipe reference outside a reduction (run semacheck first)";
        return -1;
      }
      case ExprKind::Binary: {
        const int l = LowerExpr(e->kids[0].get(), s), r = LowerExpr(e->kids[1].get(), s);
        if (!expr_err_.empty()) return -1;
        static const std::map<std::string, ir::BinOp> kOps = {
            {"||", ir::BinOp::LOr}, {"&&", ir::BinOp::LAnd}, {"|", ir::BinOp::Or},   {"^", ir::BinOp::Xor},
            {"&", ir::BinOp::And},  {"==", ir::BinOp::Eq},   {"!=", ir::BinOp::Ne},  {"<", ir::BinOp::Lt},
            {"<=", ir::BinOp::Le},  {">", ir::BinOp::Gt},    {">=", ir::BinOp::Ge},  {"<<", ir::BinOp::Shl},
            {">>", ir::BinOp::Shr}, {"+", ir::BinOp::Add},   {"-", ir::BinOp::Sub},  {"*", ir::BinOp::Mul},
            {"/", ir::BinOp::Div},  {"%", ir::BinOp::Mod},
        };
        auto it = kOps.find(e->text);
        if (it == kOps.end()) {
          expr_err_ = "unsupported binary operator \"" + e->text + "\"";
          return -1;
        }
        return b_.Bin(it->second, l, r);
      }
      case ExprKind::Unary: {
        const int x = LowerExpr(e->kids[0].get(), s);
        if (!expr_err_.empty()) return -1;
        if (e->text == "-") return b_.Un(ir::UnOp::Neg, x);
        if (e->text == "+") return b_.Un(ir::UnOp::Pos, x);
        if (e->text == "!") return b_.Un(ir::UnOp::LNot, x);
        if (e->text == "~") return b_.Un(ir::UnOp::Not, x);
        expr_err_ = "unsupported unary operator \"" + e->text + "\"";
        return -1;
      }
      case ExprKind::Select: {
        const int c = LowerExpr(e->kids[0].get(), s), t = LowerExpr(e->kids[1].get(), s), f = LowerExpr(e->kids[2].get(), s);
        if (!expr_err_.empty()) return -1;
        return b_.Select(c, t, f);
      }
      case ExprKind::Call: {
        std::vector<int> args;
        for (const auto& a : e->kids) args.push_back(LowerExpr(a.get(), s));
        if (!expr_err_.empty()) return -1;
        const int id = b_.Call(e->text, args);
        if (!b_.ExprOK(id)) {
          expr_err_ = b_.ExprError(id);
          return -1;
        }
        return id;
      }
      case ExprKind::Cast: {
        const int x = LowerExpr(e->kids[0].get(), s);
        if (!expr_err_.empty()) return -1;
        ir::Elem to;
        if (!ElemOf(e->cast_to, &to)) {
          expr_err_ = "cast target \"" + e->cast_to + "\" has no ir element type";
          return -1;
        }
        return b_.Cast(x, to);
      }
    }
    expr_err_ = "unsupported expression node";
    return -1;
  }

  const Kernel& k_;
  pkg::Builder& b_;
  std::map<std::string, int> dims_, tensors_, scalars_, dimvars_;
  std::map<std::string, std::vector<int>> tensor_dims_;
  std::string expr_err_;
};

}  // namespace

bool Lower(const Kernel& k, pkg::Builder* b, std::string* err) { return Driver(k, b).Run(err); }

std::string Kernel::CxxName() const {
  for (const auto& a : anns)
    if (a.name == "name")
      for (const auto& kc : a.args)
        if (kc.key == "cxx" && kc.kind == ConstKind::String) return kc.text;
  return "";
}

std::string Module::RuntimePath() const {
  if (!has_runtime) return "";
  for (const auto& kc : runtime.args)
    if (kc.key == "cxx_path" && kc.kind == ConstKind::String) return kc.text;
  return "";
}

}  // namespace syntax
}  // namespace tca
