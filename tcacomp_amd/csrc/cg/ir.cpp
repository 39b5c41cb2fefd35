// ir.cpp — element-type tables, the canonical printer and the verifier.
#include "ir.h"

#include <charconv>
#include <cmath>
#include <cstdio>
#include <functional>
#include <map>
#include <set>
#include <sstream>

namespace tca {
namespace ir {

namespace {
const char* kElemNames[] = {"f32", "f16", "bf16", "i32", "u32", "i8", "i16", "u8", "u16", "bool"};
const size_t kElemBytes[] = {4, 2, 2, 4, 4, 1, 2, 1, 2, 1};
const char* kBinNames[] = {"add", "sub", "mul", "div", "mod", "eq",  "ne",  "lt",  "le",
                           "gt",  "ge",  "land", "lor", "and", "or", "xor", "shl", "shr"};
const char* kUnNames[] = {"neg", "pos", "lnot", "not"};

std::string FormatConst(const Expr& e) {
  char buf[64];
  if (IsFloat(e.type)) {
    if (std::isnan(e.value)) return "nan";
    if (std::isinf(e.value)) return e.value > 0 ? "inf" : "-inf";
    std::snprintf(buf, sizeof(buf), "%.9g", e.value);
  } else if (e.type == Elem::Bool) {
    return e.value != 0.0 ? "true" : "false";
  } else {
    std::snprintf(buf, sizeof(buf), "%.0f", e.value);
  }
  return buf;
}
}  // namespace

const char* ElemName(Elem e) { return kElemNames[static_cast<int>(e)]; }
bool IsFloat(Elem e) { return e == Elem::F32 || e == Elem::F16 || e == Elem::BF16; }
bool IsInt(Elem e) {
  return e == Elem::I32 || e == Elem::U32 || e == Elem::I8 || e == Elem::I16 || e == Elem::U8 || e == Elem::U16;
}
bool IsArith(Elem e) { return IsFloat(e) || IsInt(e); }
size_t ElemBytes(Elem e) { return kElemBytes[static_cast<int>(e)]; }
bool CastPairOK(Elem from, Elem to) { return from != to && IsArith(from) && IsArith(to); }
const char* BinOpName(BinOp op) { return kBinNames[static_cast<int>(op)]; }
const char* UnOpName(UnOp op) { return kUnNames[static_cast<int>(op)]; }

Elem BinResult(BinOp op, Elem operand) {
  switch (op) {
    case BinOp::Eq:
    case BinOp::Ne:
    case BinOp::Lt:
    case BinOp::Le:
    case BinOp::Gt:
    case BinOp::Ge:
      return Elem::Bool;
    default:
      return operand;
  }
}

std::vector<int> Chain::LiveAxes() const {
  std::vector<int> live = root.as;
  live.resize(live.size() - reduces.size());
  return live;
}

bool Graph::IsStored(int tensor) const {
  for (const auto& c : chains)
    if (c.store_tensor == tensor) return true;
  return false;
}

bool Graph::IsRead(int tensor) const {
  for (const auto& c : chains) {
    for (const auto& o : c.root.ops)
      if (o.tensor == tensor) return true;
    if (c.has_piped)
      for (const auto& o : c.piped.ops)
        if (o.tensor == tensor) return true;
  }
  return false;
}

namespace {

class Printer {
 public:
  explicit Printer(const Graph& g) : g_(g) {}

  std::string Run() {
    o_ << "program " << g_.name << "\n";
    for (const auto& d : g_.dims) {
      o_ << "  dim @" << d.name << " ";
      if (d.extent == 0) o_ << "dynamic";
      else o_ << d.extent;
      o_ << "\n";
    }
    for (const auto& t : g_.tensors) {
      o_ << "  " << (t.local ? "local " : "tensor ") << t.name << ": " << ElemName(t.elem) << "[";
      for (size_t i = 0; i < t.dims.size(); ++i) o_ << (i ? ", @" : "@") << g_.dims[t.dims[i]].name;
      o_ << "]\n";
    }
    for (const auto& s : g_.scalars) o_ << "  scalar " << s.name << ": " << ElemName(s.elem) << "\n";
    for (size_t ci = 0; ci < g_.chains.size(); ++ci) {
      const Chain& c = g_.chains[ci];
      o_ << "  statement #" << ci << " iter(" << Axes(c.iters) << ")\n";
      o_ << "    map " << Ops(c.root.ops) << " " << Lambda(c.root.fn) << " as(" << Axes(c.root.as) << ")\n";
      for (const auto& r : c.reduces) {
        o_ << "    reduce init=" << Inline(r.init) << " over @" << g_.dims[r.axis].name << " " << Lambda(r.fn) << "\n";
      }
      if (c.has_piped)
        o_ << "    map pipe+" << Ops(c.piped.ops) << " " << Lambda(c.piped.fn) << " as(" << Axes(c.piped.as) << ")\n";
      o_ << "    store " << g_.tensors[c.store_tensor].name;
      for (int a : c.store_axes) o_ << "[@" << g_.dims[a].name << "]";
      o_ << "\n";
    }
    o_ << "  return";
    for (int t : g_.outputs) o_ << " " << g_.tensors[t].name;
    o_ << "\n";
    return o_.str();
  }

 private:
  std::string Axes(const std::vector<int>& axes) {
    std::string s;
    for (size_t i = 0; i < axes.size(); ++i) s += (i ? ", @" : "@") + g_.dims[axes[i]].name;
    return s;
  }
  std::string Ops(const std::vector<Operand>& ops) {
    std::string s = "on(";
    for (size_t i = 0; i < ops.size(); ++i) {
      if (i) s += ", ";
      s += g_.tensors[ops[i].tensor].name;
      for (int a : ops[i].axes) s += "[@" + g_.dims[a].name + "]";
    }
    return s + ")";
  }
  std::string Inline(int id) {
    const Expr& e = g_.exprs[id];
    if (e.op == Op::Const) return FormatConst(e) + ":" + ElemName(e.type);
    if (e.op == Op::Scalar) return "$" + g_.scalars[e.index].name;
    return "%" + std::to_string(id);
  }
  // Lambda: params, then the body's nodes in dependency order with numbers
  // local to the lambda (so the print is stable under arena growth).
  std::string Lambda(const ir::Lambda& fn) {
    std::map<int, int> local;
    std::vector<int> order;
    int next = 0;
    std::function<void(int)> visit = [&](int id) {
      if (local.count(id)) return;
      for (int a : g_.exprs[id].args) visit(a);
      const Op op = g_.exprs[id].op;
      const bool leaf = op == Op::Param || op == Op::Const || op == Op::Scalar;
      local[id] = leaf ? 0 : next++;
      order.push_back(id);
    };
    std::ostringstream s;
    s << "(";
    for (size_t i = 0; i < fn.params.size(); ++i) {
      const Expr& p = g_.exprs[fn.params[i]];
      if (i) s << ", ";
      s << p.text << ": " << ElemName(p.type);
      local[fn.params[i]] = -1 - static_cast<int>(i);
    }
    s << ") {";
    visit(fn.body);
    auto ref = [&](int id) -> std::string {
      int l = local[id];
      if (l < 0) return g_.exprs[id].text;
      const Expr& e = g_.exprs[id];
      if (e.op == Op::Const) return FormatConst(e);
      if (e.op == Op::Scalar) return "$" + g_.scalars[e.index].name;
      return "%" + std::to_string(l);
    };
    for (int id : order) {
      const Expr& e = g_.exprs[id];
      if (e.op == Op::Param || e.op == Op::Const || e.op == Op::Scalar) continue;
      s << " %" << local[id] << " = ";
      switch (e.op) {
        case Op::Bin: s << BinOpName(static_cast<BinOp>(e.code)); break;
        case Op::Un: s << UnOpName(static_cast<UnOp>(e.code)); break;
        case Op::Select: s << "select"; break;
        case Op::Cast: s << "cast." << ElemName(e.type); break;
        case Op::Call: s << e.text; break;
        default: s << "?"; break;
      }
      for (int a : e.args) s << " " << ref(a);
      s << ";";
    }
    s << " -> " << ref(fn.body) << ": " << ElemName(g_.exprs[fn.body].type) << " }";
    return s.str();
  }

  const Graph& g_;
  std::ostringstream o_;
};

}  // namespace

std::string Print(const Graph& g) { return Printer(g).Run(); }

std::string FormatFloat32Go(double v) {
  const float f = static_cast<float>(v);
  if (std::isnan(f)) return "NaN";
  if (std::isinf(f)) return f > 0 ? "+Inf" : "-Inf";
  const bool neg = std::signbit(f);
  if (f == 0.0f) return neg ? "-0" : "0";
  // Shortest digits that round-trip to f, as d.ddde[+-]XX.
  char buf[64];
  const auto r = std::to_chars(buf, buf + sizeof(buf), neg ? -f : f, std::chars_format::scientific);
  const std::string sci(buf, r.ptr);
  const size_t epos = sci.find('e');
  const int exp10 = std::stoi(sci.substr(epos + 1));
  std::string digits;
  for (size_t i = 0; i < epos; ++i)
    if (sci[i] != '.') digits += sci[i];
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  const int nd = static_cast<int>(digits.size()), dp = exp10 + 1;
  std::string out = neg ? "-" : "";
  if (exp10 < -4 || exp10 >= 6) {  // %e with nd - 1 fraction digits, >= 2 exponent digits
    out += digits[0];
    if (nd > 1) out += "." + digits.substr(1);
    const int ae = exp10 < 0 ? -exp10 : exp10;
    out += exp10 < 0 ? "e-" : "e+";
    if (ae < 10) out += "0";
    out += std::to_string(ae);
    return out;
  }
  // %f with max(nd - dp, 0) fraction digits.
  if (dp > 0) {
    for (int i = 0; i < dp; ++i) out += i < nd ? digits[i] : '0';
  } else {
    out += "0";
  }
  const int frac = nd - dp > 0 ? nd - dp : 0;
  if (frac > 0) {
    out += ".";
    for (int i = 0; i < frac; ++i) {
      const int k = dp + i;
      out += (k >= 0 && k < nd) ? digits[k] : '0';
    }
  }
  return out;
}

namespace {

// The reference printer's rendering (internal/ir/print.go): chains as stage
// lines, scalar expressions with its precedence table (binPrec/exprPrec),
// constants spelled by type (constText/FormatConst).
class RefPrinter {
 public:
  explicit RefPrinter(const Graph& g) : g_(g) {}

  std::string Run() {
    std::ostringstream o;
    bool first = true;
    for (const Chain& c : g_.chains) {
      if (!first) o << "\n";
      first = false;
      o << "statement #" << c.stmt_id << ":\n";
      std::vector<std::string> stages;
      stages.push_back("iter(" + DimList(c.iters) + ") -> " + MapText(c.root, false));
      for (const ReduceStage& r : c.reduces)
        stages.push_back("reduce(init=" + Value(r.init) + ", %0, " + LambdaText(r.fn) + ")");
      if (c.has_piped) stages.push_back("iter() -> " + MapText(c.piped, true));
      std::string st = "memstore(%" + TensorName(c.store_tensor);
      for (int a : c.store_axes) st += "[@" + g_.dims[a].name + "]";
      stages.push_back(st + ", %0)");
      for (size_t i = 0; i < stages.size(); ++i) {
        o << "  " << stages[i];
        if (i + 1 < stages.size()) o << " |\n";
      }
      o << "\n";
    }
    if (!g_.outputs.empty()) {
      if (!first) o << "\n";
      o << "statement #" << g_.end_stmt_id << ":\n  return ";
      for (size_t i = 0; i < g_.outputs.size(); ++i) o << (i ? ", %" : "%") << g_.tensors[g_.outputs[i]].name;
      o << "\n";
    }
    return o.str();
  }

 private:
  // A local is a MemNew allocation in the reference, not a named parameter:
  // its printer has no name for it.
  std::string TensorName(int t) const { return g_.tensors[t].local ? "?" : g_.tensors[t].name; }

  std::string DimList(const std::vector<int>& dims) const {
    std::string s;
    for (size_t i = 0; i < dims.size(); ++i) s += (i ? ", @" : "@") + g_.dims[dims[i]].name;
    return s;
  }

  // A tensor operand renders as its declared type's axes (paramRef case of
  // the reference's value()), a local as "?".
  std::string OperandText(const Operand& op) const {
    const Tensor& t = g_.tensors[op.tensor];
    if (t.local) return "?";
    std::string s = t.name;
    for (int d : t.dims) s += "[@" + g_.dims[d].name + "]";
    return s;
  }

  std::string MapText(const MapStage& m, bool piped) const {
    std::string s = "map(";
    std::vector<std::string> vals;
    if (piped) vals.push_back("%0");
    for (const Operand& op : m.ops) vals.push_back(OperandText(op));
    for (size_t i = 0; i < vals.size(); ++i) s += (i ? ", " : "") + vals[i];
    s += ", " + LambdaText(m.fn) + ")";
    if (!m.as.empty()) s += " as (" + DimList(m.as) + ")";
    return s;
  }

  std::string LambdaText(const Lambda& fn) const {
    std::string s = "lambda(";
    for (size_t i = 0; i < fn.params.size(); ++i) s += (i ? ", " : "") + g_.exprs[fn.params[i]].text;
    return s + "): " + Value(fn.body);
  }

  static int BinPrec(BinOp op) {
    switch (op) {
      case BinOp::LOr: return 1;
      case BinOp::LAnd: return 2;
      case BinOp::Or: return 3;
      case BinOp::Xor: return 4;
      case BinOp::And: return 5;
      case BinOp::Eq: case BinOp::Ne: return 6;
      case BinOp::Lt: case BinOp::Le: case BinOp::Gt: case BinOp::Ge: return 7;
      case BinOp::Shl: case BinOp::Shr: return 8;
      case BinOp::Add: case BinOp::Sub: return 9;
      case BinOp::Mul: case BinOp::Div: case BinOp::Mod: return 10;
    }
    return 0;
  }
  static const char* BinSym(BinOp op) {
    switch (op) {
      case BinOp::LOr: return "||";
      case BinOp::LAnd: return "&&";
      case BinOp::Or: return "|";
      case BinOp::Xor: return "^";
      case BinOp::And: return "&";
      case BinOp::Eq: return "==";
      case BinOp::Ne: return "!=";
      case BinOp::Lt: return "<";
      case BinOp::Le: return "<=";
      case BinOp::Gt: return ">";
      case BinOp::Ge: return ">=";
      case BinOp::Shl: return "<<";
      case BinOp::Shr: return ">>";
      case BinOp::Add: return "+";
      case BinOp::Sub: return "-";
      case BinOp::Mul: return "*";
      case BinOp::Div: return "/";
      case BinOp::Mod: return "%";
    }
    return "?";
  }
  static const char* UnSym(UnOp op) {
    switch (op) {
      case UnOp::Pos: return "+";
      case UnOp::Neg: return "-";
      case UnOp::LNot: return "!";
      case UnOp::Not: return "~";
    }
    return "?";
  }
  int Prec(int id) const {
    const Expr& e = g_.exprs[id];
    if (e.op == Op::Bin) return BinPrec(static_cast<BinOp>(e.code));
    if (e.op == Op::Un) return 11;
    if (e.op == Op::Select) return 0;
    return 12;
  }

  std::string ConstText(const Expr& e) const {
    switch (e.type) {
      case Elem::I8: case Elem::I16: case Elem::I32:
        return std::to_string(static_cast<int64_t>(e.value));
      case Elem::U8: case Elem::U16: case Elem::U32:
        return std::to_string(static_cast<uint64_t>(e.value));
      case Elem::Bool:
        return e.value != 0.0 ? "true" : "false";
      default: {
        std::string s = FormatFloat32Go(e.value);
        if (s.find_first_of(".eE") == std::string::npos) s += ".0";
        return s;
      }
    }
  }

  std::string Value(int id) const {
    const Expr& e = g_.exprs[id];
    switch (e.op) {
      case Op::Const: return ConstText(e);
      case Op::Param: return e.text;
      case Op::Scalar: return g_.scalars[e.index].name;
      case Op::Bin: {
        const int p = BinPrec(static_cast<BinOp>(e.code));
        std::string l = Value(e.args[0]), r = Value(e.args[1]);
        if (Prec(e.args[0]) < p) l = "(" + l + ")";
        if (Prec(e.args[1]) <= p) r = "(" + r + ")";
        return l + " " + BinSym(static_cast<BinOp>(e.code)) + " " + r;
      }
      case Op::Un: {
        std::string x = Value(e.args[0]);
        if (Prec(e.args[0]) <= 11) x = "(" + x + ")";
        return UnSym(static_cast<UnOp>(e.code)) + x;
      }
      case Op::Select:
        return Value(e.args[0]) + " ? " + Value(e.args[1]) + " : " + Value(e.args[2]);
      case Op::Cast:
        return std::string("cast<") + ElemName(e.type) + ">(" + Value(e.args[0]) + ")";
      case Op::Call: {
        std::string s = e.text + "(";
        for (size_t i = 0; i < e.args.size(); ++i) s += (i ? ", " : "") + Value(e.args[i]);
        return s + ")";
      }
      default:
        return "<nil>";
    }
  }

  const Graph& g_;
};

}  // namespace

std::string PrintReference(const Graph& g) { return RefPrinter(g).Run(); }

bool Verify(const Graph& g, std::string* err) {
  auto bad = [&](const std::string& m) {
    *err = "verify " + g.name + ": " + m;
    return false;
  };
  const int nd = static_cast<int>(g.dims.size());
  const int nt = static_cast<int>(g.tensors.size());
  const int ne = static_cast<int>(g.exprs.size());
  for (const auto& t : g.tensors) {
    if (t.dims.size() > 8) return bad("tensor " + t.name + " exceeds rank 8");
    for (int d : t.dims)
      if (d < 0 || d >= nd) return bad("tensor " + t.name + " has a dangling dim");
  }
  for (int i = 0; i < ne; ++i) {
    const Expr& e = g.exprs[i];
    if (e.op == Op::Error) continue;  // unreachable error nodes are inert
    for (int a : e.args)
      if (a < 0 || a >= i) return bad("expression %" + std::to_string(i) + " is not in dependency order");
  }
  std::function<bool(int, const std::set<int>&)> exprOK = [&](int id, const std::set<int>& params) -> bool {
    if (id < 0 || id >= ne) return false;
    const Expr& e = g.exprs[id];
    if (e.op == Op::Error) return false;
    if (e.op == Op::Param) return params.count(id) > 0;
    if (e.op == Op::Scalar) return e.index >= 0 && e.index < static_cast<int>(g.scalars.size());
    for (int a : e.args)
      if (!exprOK(a, params)) return false;
    return true;
  };
  std::set<int> stored;
  for (size_t ci = 0; ci < g.chains.size(); ++ci) {
    const Chain& c = g.chains[ci];
    const std::string where = "statement #" + std::to_string(ci);
    if (c.iters.empty()) return bad(where + ": empty iteration cluster");
    std::set<int> iterSet(c.iters.begin(), c.iters.end());
    if (iterSet.size() != c.iters.size()) return bad(where + ": repeated iteration dim");
    std::set<int> asSet(c.root.as.begin(), c.root.as.end());
    if (asSet != iterSet || c.root.as.size() != c.iters.size())
      return bad(where + ": root as is not a permutation of the iteration cluster");
    auto checkOps = [&](const std::vector<Operand>& ops, const std::set<int>& live) -> bool {
      for (const auto& o : ops) {
        if (o.tensor < 0 || o.tensor >= nt) return false;
        const Tensor& t = g.tensors[o.tensor];
        if (o.axes.size() != t.dims.size()) return false;
        for (size_t i = 0; i < o.axes.size(); ++i)
          if (o.axes[i] != t.dims[i] || !live.count(o.axes[i])) return false;
        if (t.local && !stored.count(o.tensor)) return false;
      }
      return true;
    };
    if (!checkOps(c.root.ops, iterSet)) return bad(where + ": root map operand binding is invalid (or reads a local before it is stored)");
    if (c.root.fn.params.size() != c.root.ops.size()) return bad(where + ": root map arity");
    {
      std::set<int> ps(c.root.fn.params.begin(), c.root.fn.params.end());
      if (!exprOK(c.root.fn.body, ps)) return bad(where + ": root map body is malformed");
      for (size_t i = 0; i < c.root.ops.size(); ++i)
        if (g.exprs[c.root.fn.params[i]].type != g.tensors[c.root.ops[i].tensor].elem)
          return bad(where + ": root map parameter type differs from its operand");
    }
    Elem pipe = g.exprs[c.root.fn.body].type;
    std::vector<int> live = c.root.as;
    for (const auto& r : c.reduces) {
      if (live.empty()) return bad(where + ": reduce with no live axis");
      if (r.axis != live.back()) return bad(where + ": reduce must drop the last live axis");
      live.pop_back();
      std::set<int> ps(r.fn.params.begin(), r.fn.params.end());
      if (r.fn.params.size() != 2 || !exprOK(r.fn.body, ps) || !exprOK(r.init, {}))
        return bad(where + ": reduce lambda is malformed");
      if (g.exprs[r.init].type != pipe || g.exprs[r.fn.body].type != pipe)
        return bad(where + ": homogeneous reducer violated");
    }
    std::set<int> liveSet(live.begin(), live.end());
    if (c.has_piped) {
      if (c.reduces.empty()) return bad(where + ": piped map without a preceding reduce");
      if (c.piped.as != live) return bad(where + ": piped as must be exactly the live axes in order");
      if (!checkOps(c.piped.ops, liveSet)) return bad(where + ": piped map operand binding is invalid");
      if (c.piped.fn.params.size() != c.piped.ops.size() + 1) return bad(where + ": piped map arity");
      std::set<int> ps(c.piped.fn.params.begin(), c.piped.fn.params.end());
      if (!exprOK(c.piped.fn.body, ps)) return bad(where + ": piped map body is malformed");
      if (g.exprs[c.piped.fn.params[0]].type != pipe) return bad(where + ": piped value type mismatch");
      pipe = g.exprs[c.piped.fn.body].type;
    }
    if (c.store_tensor < 0 || c.store_tensor >= nt) return bad(where + ": store target is invalid");
    const Tensor& st = g.tensors[c.store_tensor];
    if (c.store_axes.size() != st.dims.size()) return bad(where + ": store rank mismatch");
    std::set<int> storeSet;
    for (size_t i = 0; i < c.store_axes.size(); ++i) {
      if (c.store_axes[i] != st.dims[i]) return bad(where + ": store axis binds the wrong dim");
      if (!liveSet.count(c.store_axes[i])) return bad(where + ": store axis is not live");
      storeSet.insert(c.store_axes[i]);
    }
    if (storeSet != liveSet)
      return bad(where + ": store of " + st.name +
                 " does not cover every live axis (each output element needs a single owner)");
    if (pipe != st.elem) return bad(where + ": stored value type differs from " + st.name + "'s element type");
    stored.insert(c.store_tensor);
  }
  for (int t : g.outputs)
    if (t < 0 || t >= nt || g.tensors[t].local || !stored.count(t)) return bad("output list is inconsistent");
  return true;
}

}  // namespace ir
}  // namespace tca
