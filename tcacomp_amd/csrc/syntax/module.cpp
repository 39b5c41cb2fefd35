// module.cpp — module loading with @include resolution, and the canonical
// AST dump.
//
// Include policy follows internal/syntax/module.go:27-180: a path is
// relative to the including file and may not escape that file's directory;
// a cycle is an error; a file reached twice (diamond) merges once; included
// kernels append after the includer's in depth-first order; the root's
// @runtime wins, else the first one an include declares. The dump renders
// the tree the way the reference's parser golden does
// (internal/syntax/parser/dump_test.go): one node per line, two-space
// indents, prefix expressions, no positions.
#include <fstream>
#include <set>
#include <sstream>

#include <sys/stat.h>

#include "syntax.h"

namespace tca {
namespace syntax {

namespace {

bool ReadFile(const std::string& path, std::string* out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream ss;
  ss << f.rdbuf();
  *out = ss.str();
  return true;
}

bool Exists(const std::string& p) {
  struct stat st;
  return stat(p.c_str(), &st) == 0;
}

std::string Dir(const std::string& path) {
  const size_t slash = path.find_last_of('/');
  if (slash == std::string::npos) return ".";
  if (slash == 0) return "/";
  return path.substr(0, slash);
}

// Lexical path cleaning (Go's filepath.Clean): collapses "//", "." and
// "x/.." without touching the file system.
std::string Clean(const std::string& path) {
  if (path.empty()) return ".";
  const bool abs = path[0] == '/';
  std::vector<std::string> parts;
  std::stringstream ss(path);
  std::string seg;
  while (std::getline(ss, seg, '/')) {
    if (seg.empty() || seg == ".") continue;
    if (seg == "..") {
      if (!parts.empty() && parts.back() != "..") {
        parts.pop_back();
      } else if (!abs) {
        parts.push_back("..");
      }
      continue;
    }
    parts.push_back(seg);
  }
  std::string out = abs ? "/" : "";
  for (size_t i = 0; i < parts.size(); ++i) out += (i ? "/" : "") + parts[i];
  if (out.empty()) out = abs ? "/" : ".";
  return out;
}

class Loader {
 public:
  explicit Loader(std::vector<Diagnostic>* diags) : diags_(diags) {}

  bool LoadFile(const std::string& path, Module* m) {
    std::string src;
    if (!ReadFile(path, &src)) {
      Diagnostic d;
      d.pos.file = path;
      d.msg = "cannot read source file: " + path;
      diags_->push_back(d);
      return false;
    }
    *m = Parse(path, src, diags_);
    return true;
  }

  void ResolveIncludes(Module* m, const std::string& path, std::set<std::string> stack) {
    for (auto& inc : m->includes) {
      std::string resolved;
      if (!ResolvePath(inc, path, &resolved)) continue;
      inc.resolved = resolved;
      if (stack.count(resolved)) {
        Error(inc.pos, "@include cycle: " + resolved + " is already being loaded");
        continue;
      }
      if (processed_.count(resolved)) continue;  // include guard (diamond)
      Module sub;
      if (!LoadFile(resolved, &sub)) continue;
      if (sub.has_runtime && !have_first_runtime_) {
        first_runtime_ = sub.runtime;
        have_first_runtime_ = true;
      }
      processed_.insert(resolved);
      std::set<std::string> inner = stack;
      inner.insert(resolved);
      ResolveIncludes(&sub, resolved, inner);
      for (auto& k : sub.kernels) m->kernels.push_back(std::move(k));
    }
  }

  bool have_first_runtime_ = false;
  Annotation first_runtime_;

 private:
  void Error(const Pos& p, const std::string& msg) {
    Diagnostic d;
    d.pos = p;
    d.msg = msg;
    diags_->push_back(d);
  }

  bool ResolvePath(const Include& inc, const std::string& including, std::string* out) {
    if (!inc.path.empty() && inc.path[0] == '/') {
      Error(inc.pos, "@include path \"" + inc.path + "\" must be relative to the including file");
      return false;
    }
    const std::string dir = Clean(Dir(including));
    const std::string resolved = Clean(dir + "/" + inc.path);
    const bool within = resolved == dir || resolved.compare(0, dir.size() + 1, dir + "/") == 0 ||
                        (dir == "." && resolved.compare(0, 3, "../") != 0 && resolved != "..");
    if (!within) {
      Error(inc.pos, "@include path \"" + inc.path + "\" escapes the including file's directory");
      return false;
    }
    if (!Exists(resolved)) {
      Error(inc.pos, "missing include file \"" + inc.path + "\"");
      return false;
    }
    *out = resolved;
    return true;
  }

  std::vector<Diagnostic>* diags_;
  std::set<std::string> processed_;
};

// Go's %q for the plain strings annotations carry.
std::string Quote(const std::string& s) {
  std::string out = "\"";
  for (char c : s) {
    if (c == '"' || c == '\\') out += '\\';
    out += c;
  }
  return out + "\"";
}

std::string Keyed(const std::vector<KeyedConst>& args) {
  std::string s = "(";
  for (size_t i = 0; i < args.size(); ++i) {
    if (i) s += ", ";
    s += args[i].key + "=" + (args[i].kind == ConstKind::String ? Quote(args[i].text) : args[i].text);
  }
  return s + ")";
}

std::string TypeText(const Type& t) {
  if (!t.tensor) return t.elem;
  std::string s = "tensor<" + t.elem + ",[";
  for (size_t i = 0; i < t.shape.size(); ++i) s += (i ? "," : "") + (t.shape[i].symbolic() ? t.shape[i].name : std::to_string(t.shape[i].extent));
  return s + "]>";
}

std::string ExprText(const Expr* e) {
  if (e == nullptr) return "?";
  switch (e->kind) {
    case ExprKind::Lit: return e->text;
    case ExprKind::Name: return "name(" + e->text + ")";
    case ExprKind::Pipe: return "%0";
    case ExprKind::Binary: return "(" + e->text + " " + ExprText(e->kids[0].get()) + " " + ExprText(e->kids[1].get()) + ")";
    case ExprKind::Unary: return "(" + e->text + " " + ExprText(e->kids[0].get()) + ")";
    case ExprKind::Select:
      return "(select " + ExprText(e->kids[0].get()) + " " + ExprText(e->kids[1].get()) + " " + ExprText(e->kids[2].get()) + ")";
    case ExprKind::Call: {
      std::string s = "call(" + e->text + " ";
      for (size_t i = 0; i < e->kids.size(); ++i) s += (i ? ", " : "") + ExprText(e->kids[i].get());
      return s + ")";
    }
    case ExprKind::Cast: return "(cast " + e->cast_to + " " + ExprText(e->kids[0].get()) + ")";
  }
  return "?";
}

std::string Specs(const std::vector<ParamSpec>& ps) {
  std::string s;
  for (size_t i = 0; i < ps.size(); ++i) {
    if (i) s += ", ";
    s += (ps[i].pipe ? std::string("%0") : ps[i].name) + (ps[i].type.empty() ? "" : ":" + ps[i].type);
  }
  return s;
}

std::string AsText(const Stage& st) {
  if (!st.has_as) return "";
  std::string s = " as(";
  for (size_t i = 0; i < st.as.size(); ++i) s += (i ? "," : "") + st.as[i];
  return s + ")";
}

}  // namespace

Module Load(const std::string& path, std::vector<Diagnostic>* diags) {
  Loader ld(diags);
  Module root;
  if (!ld.LoadFile(path, &root)) return Module();
  const std::string clean = Clean(path);
  ld.ResolveIncludes(&root, path, {clean});
  if (!root.has_runtime && ld.have_first_runtime_) {
    root.has_runtime = true;
    root.runtime = ld.first_runtime_;
  }
  CheckModule(root, diags);
  for (auto& k : root.kernels) Check(&k, diags);
  return root;
}

std::string Dump(const Module& m) {
  std::ostringstream b;
  b << "module\n";
  for (const auto& inc : m.includes) b << "  include " << Quote(inc.path) << "\n";
  if (m.has_runtime) b << "  runtime " << Keyed(m.runtime.args) << "\n";
  for (const auto& k : m.kernels) {
    for (const auto& a : k.anns) b << "  annotation @" << a.name << " " << Keyed(a.args) << "\n";
    b << "  kernel " << k.name << "\n";
    for (const auto& p : k.params) b << "    param " << p.name << " " << TypeText(p.type) << "\n";
    for (const auto& r : k.rets) b << "    ret " << TypeText(r) << "\n";
    for (const auto& s : k.body) {
      switch (s.kind) {
        case StmtKind::DimVar: {
          b << "    dimvar";
          for (const auto& n : s.names) b << " " << n;
          b << "\n";
          break;
        }
        case StmtKind::Return: {
          b << "    return ";
          for (size_t i = 0; i < s.names.size(); ++i) b << (i ? ", " : "") << s.names[i];
          b << "\n";
          break;
        }
        case StmtKind::Let:
          b << "    let " << s.name << (s.type.present ? ": " + TypeText(s.type) : "") << "\n";
          for (const auto& st : s.chain) {
            if (st.is_map) {
              std::string ops;
              for (size_t i = 0; i < st.bindings.size(); ++i) {
                ops += (i ? ", " : "") + st.bindings[i].tensor;
                for (const auto& d : st.bindings[i].dims) ops += "[" + d + "]";
              }
              b << "      map on(" << ops << ")" << AsText(st) << "\n";
              const Lambda& l = st.lambda;
              std::string caps;
              if (!l.captures.empty()) {
                caps = "[";
                for (size_t i = 0; i < l.captures.size(); ++i) caps += (i ? "," : "") + l.captures[i];
                caps += "] ";
              }
              b << "        " << caps << "(" << Specs(l.params) << ")" << (l.ret.empty() ? "" : " -> " + l.ret) << ": "
                << ExprText(l.body.get()) << "\n";
            } else {
              b << "      reduce(" << (st.init ? "init=" + ExprText(st.init.get()) : "") << ") on(" << Specs(st.on_params) << ")"
                << AsText(st) << " -> " << st.ret << ": " << ExprText(st.body.get()) << "\n";
            }
          }
          break;
      }
    }
  }
  return b.str();
}

}  // namespace syntax
}  // namespace tca
