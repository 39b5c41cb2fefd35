// syntax.h — the .tca text frontend: lexer, parser, semantic checker and the
// lowering driver that replays a checked kernel through the builder rungs.
//
// Reference (behaviour, not code): internal/syntax/{lexer,parser,ast,
// semacheck,build}/*.go and internal/syntax/{api,module}.go, specified in
// design/syntax.md and design/syntax-design.md. Kept from the reference:
//   - the token set, literal forms (f32 needs the f/F suffix, u32 the u/U
//     suffix, %0 is the only legal placeholder) and comment forms;
//   - operator precedence: ?: < || < && < | < ^ < & < == != < relational <
//     + - < * / % < unary; a '|' followed by `map` or `reduce` at a stage
//     body's top level is the pipe, everywhere else bitwise-or;
//   - the per-kernel rules 5-26 (one namespace, implicit dims, bindings,
//     `as` inference and checks, lambda arity, captures, expression typing)
//     and the module rules 1, 3, 4, with the same diagnostic wording;
//   - the lowering: dims in first-appearance order (static extents named
//     e<extent>), tensor params, then the returned let as the output tensor,
//     then scalar params; every other let becomes a Local; each chain's
//     iteration order puts the surviving axes first and the reduced axes last
//     in reverse reduce order, so each rung Reduce drops the right axis.
// Extensions: a let whose chain is a single map is lowered as an elementwise
// chain (the builder's own extension; the reference rejects it at lowering,
// "require at least one reduction before the store"); a kernel may return
// several lets (`-> (T1, T2)` and `return a, b;`), each an output tensor in
// return order (the reference allows one); `<<` / `>>` parse at C
// precedence (the reference scans them but has no grammar level).
#ifndef TCA_SYNTAX_SYNTAX_H_
#define TCA_SYNTAX_SYNTAX_H_

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "../cg/builder.h"
#include "../cg/ir.h"

namespace tca {
namespace syntax {

struct Pos {
  std::string file;
  int line = 0, col = 0;
  bool valid() const { return line > 0; }
};

struct Diagnostic {
  bool error = true;
  Pos pos;
  std::string msg;
  std::string String() const;  // "file:line:col: error: msg"
};

// ------------------------------------------------------------------ tokens
enum class Tok {
  Illegal, Eof, Ident, IntLit, UintLit, FloatLit, StringLit, Placeholder,
  Kernel, Let, Return, DimVar, Map, On, As, Reduce, Init, True, False, InfF32,
  TBool, TF32, TF16, TBF16, TI8, TI16, TI32, TU8, TU16, TU32,
  At, LParen, RParen, LBracket, RBracket, LBrace, RBrace, Lt, Gt, Comma, Semi, Colon, Assign, Question,
  Pipe, Amp, Caret, Tilde, Bang, Plus, Minus, Star, Slash, Percent, Arrow, EqEq, Ne, Le, Ge, AndAnd, OrOr,
  Shl, Shr
};
const char* TokName(Tok k);
bool IsElemTok(Tok k);

struct Token {
  Tok kind = Tok::Illegal;
  std::string lit;
  Pos pos;
  int64_t ival = 0;   // IntLit (i32), UintLit (u32), Placeholder index
  float fval = 0.0f;  // FloatLit
};

// Scans the whole file; lexical errors are appended to diags.
std::vector<Token> Scan(const std::string& file, const std::string& src, std::vector<Diagnostic>* diags);

// --------------------------------------------------------------------- AST
struct ShapeDim {
  Pos pos;
  std::string name;     // symbolic dim (dynamic extent)
  uint64_t extent = 0;  // compile-time extent when name is empty
  bool symbolic() const { return !name.empty(); }
  std::string Key() const;  // name, or e<extent> for a static extent
};

struct Type {
  Pos pos;
  bool present = false;  // an optional annotation that was written
  bool tensor = false;
  std::string elem;      // spelling: f32, bf16, ...
  bool has_shape = false;
  std::vector<ShapeDim> shape;
};

enum class ExprKind { Lit, Name, Pipe, Binary, Unary, Select, Call, Cast };
enum class LitKind { Int, Uint, Float, Bool };

struct Expr {
  ExprKind kind = ExprKind::Lit;
  Pos pos;
  std::string text;  // literal spelling, name, operator or callee
  LitKind lit = LitKind::Int;
  int64_t ival = 0;
  float fval = 0.0f;
  bool bval = false;
  std::string cast_to;
  std::vector<std::unique_ptr<Expr>> kids;
};
using ExprP = std::unique_ptr<Expr>;

struct ParamSpec {
  Pos pos;
  bool pipe = false;  // %0
  std::string name;
  std::string type;   // empty = omitted (filled by the checker)
};

struct Binding {
  Pos pos;
  std::string tensor;
  std::vector<std::string> dims;
};

struct Lambda {
  Pos pos;
  std::vector<std::string> captures;
  std::vector<ParamSpec> params;
  std::string ret;  // empty = omitted (filled by the checker)
  ExprP body;
};

struct Stage {
  bool is_map = true;
  Pos pos;
  bool has_as = false;
  std::vector<std::string> as;
  // map
  std::vector<Binding> bindings;
  Lambda lambda;
  // reduce
  ExprP init;
  std::vector<ParamSpec> on_params;
  std::string ret;
  ExprP body;
};

enum class StmtKind { DimVar, Let, Return };

struct Stmt {
  StmtKind kind = StmtKind::DimVar;
  Pos pos;
  std::vector<std::string> names;  // dimvar names; returned lets
  std::string name;                // let; first returned let
  Type type;                       // let annotation (filled by the checker)
  std::vector<Stage> chain;
};

enum class ConstKind { Int, Uint, Float, String, Bool, None };
struct KeyedConst {
  Pos pos;
  std::string key;
  ConstKind kind = ConstKind::None;
  std::string text;
};

struct Annotation {
  Pos pos;
  std::string name;
  std::vector<KeyedConst> args;
};

struct Param {
  Pos pos;
  std::string name;
  Type type;
  bool is_tensor() const { return type.tensor; }
};

struct Kernel {
  Pos pos;
  std::vector<Annotation> anns;
  std::string name;
  std::vector<Param> params;
  std::vector<Type> rets;  // one per returned let
  std::vector<Stmt> body;
  std::string CxxName() const;  // @name(cxx=...) or empty
};

struct Include {
  Pos pos;
  std::string path, resolved;
};

struct Module {
  std::vector<Include> includes;
  bool has_runtime = false;
  Annotation runtime;
  std::vector<Kernel> kernels;
  std::string RuntimePath() const;  // @runtime cxx_path or empty
};

// ------------------------------------------------------------------- passes
// Parses one file's text (no include resolution).
Module Parse(const std::string& file, const std::string& src, std::vector<Diagnostic>* diags);
// Module rules 1, 3, 4.
void CheckModule(const Module& m, std::vector<Diagnostic>* diags);
// Per-kernel rules 5-26; fills the omitted cells (as clauses, lambda and
// parameter types, let types) in place.
void Check(Kernel* k, std::vector<Diagnostic>* diags);
// Loads path, resolves @include (relative to the including file, no escape
// from its directory, cycle and diamond safe), runs CheckModule and Check.
Module Load(const std::string& path, std::vector<Diagnostic>* diags);
// Drives a checked kernel through the builder rungs; false with *err set on
// failure. The builder is left un-built (the caller runs Build).
bool Lower(const Kernel& k, pkg::Builder* b, std::string* err);
// Canonical indented rendering of the AST (no positions).
std::string Dump(const Module& m);

bool HasErrors(const std::vector<Diagnostic>& d);
std::string JoinDiagnostics(const std::vector<Diagnostic>& d, bool errors_only);
bool ElemOf(const std::string& spelling, ir::Elem* out);

}  // namespace syntax
}  // namespace tca

#endif  // TCA_SYNTAX_SYNTAX_H_
