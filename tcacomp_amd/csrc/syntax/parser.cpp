// parser.cpp — recursive-descent parser for .tca modules. Grammar and error
// recovery follow internal/syntax/parser/{parser,stmt,expr,type}.go: one
// method per precedence level, `sync` to the next ';', '}', `kernel` or '@'
// after a statement-level error, annotations attach to the next kernel.
#include <cmath>
#include <limits>

#include "syntax.h"

namespace tca {
namespace syntax {

namespace {

class Parser {
 public:
  Parser(std::vector<Token> toks, std::vector<Diagnostic>* diags) : toks_(std::move(toks)), diags_(diags) {}

  Module ParseModule() {
    Module m;
    std::vector<Annotation> pending;
    while (!At(Tok::Eof)) {
      if (At(Tok::At)) {
        AtDecl(&m, &pending);
      } else if (At(Tok::Kernel)) {
        Kernel k;
        if (ParseKernel(std::move(pending), &k)) m.kernels.push_back(std::move(k));
        pending.clear();
      } else {
        Error(Cur().pos, std::string("expected declaration, found ") + TokName(Cur().kind));
        const size_t before = pos_;
        Sync();
        // Sync stops at a '}' it does not consume; stepping over it here is
        // what keeps a stray '}' from being reported forever (the loop
        // would otherwise never advance).
        if (pos_ == before) Advance();
      }
    }
    for (const auto& a : pending) Error(a.pos, "annotation @" + a.name + " does not precede a kernel");
    return m;
  }

 private:
  // ---------------------------------------------------------------- tokens
  const Token& Cur() const { return toks_[pos_]; }
  const Token& PeekTok(size_t n) const { return pos_ + n < toks_.size() ? toks_[pos_ + n] : toks_.back(); }
  bool At(Tok k) const { return Cur().kind == k; }
  Token Advance() {
    Token t = toks_[pos_];
    if (pos_ + 1 < toks_.size()) ++pos_;
    return t;
  }
  // Returns the token when it matches; otherwise records "expected X, found
  // Y" and returns a token with an invalid position.
  Token Expect(Tok k) {
    if (At(k)) return Advance();
    Error(Cur().pos, std::string("expected ") + TokName(k) + ", found " + TokName(Cur().kind));
    return Token{};
  }
  bool ExpectContextual(const char* lit) {
    if (At(Tok::Ident) && Cur().lit == lit) {
      Advance();
      return true;
    }
    Error(Cur().pos, std::string("expected \"") + lit + "\", found " + Describe());
    return false;
  }
  std::string Describe() const {
    if (At(Tok::Ident)) return "identifier " + Cur().lit;
    return TokName(Cur().kind);
  }
  void Error(const Pos& p, const std::string& msg) {
    Diagnostic d;
    d.pos = p;
    d.msg = msg;
    diags_->push_back(d);
  }
  void Sync() {
    while (!At(Tok::Eof) && !At(Tok::Semi) && !At(Tok::RBrace) && !At(Tok::Kernel) && !At(Tok::At)) Advance();
    if (At(Tok::Semi)) Advance();
  }

  // ------------------------------------------------------ module level
  void AtDecl(Module* m, std::vector<Annotation>* pending) {
    const Token at = Expect(Tok::At);
    const Token name = Expect(Tok::Ident);
    if (!name.pos.valid()) {
      Sync();
      return;
    }
    if (name.lit == "include") {
      const Token path = Cur();
      if (path.kind != Tok::StringLit) {
        Error(path.pos, std::string("@include expects a single string literal path, found ") + TokName(path.kind));
        Sync();
        return;
      }
      Advance();
      Expect(Tok::Semi);
      Include inc;
      inc.pos = at.pos;
      inc.path = path.lit;
      m->includes.push_back(inc);
      return;
    }
    if (name.lit == "runtime") {
      if (m->has_runtime) Error(at.pos, "at most one @runtime per module (rule 3)");
      Annotation rt;
      rt.pos = at.pos;
      rt.name = "runtime";
      rt.args = KeyedConstList();
      Expect(Tok::Semi);
      m->has_runtime = true;
      m->runtime = rt;
      return;
    }
    Annotation ann;
    ann.pos = at.pos;
    ann.name = name.lit;
    ann.args = KeyedConstList();
    pending->push_back(ann);
  }

  std::vector<KeyedConst> KeyedConstList() {
    std::vector<KeyedConst> args;
    Expect(Tok::LParen);
    while (!At(Tok::RParen) && !At(Tok::Eof)) {
      const Token key = Expect(Tok::Ident);
      if (!key.pos.valid()) {
        Sync();
        return args;
      }
      Expect(Tok::Assign);
      KeyedConst kc;
      kc.pos = key.pos;
      kc.key = key.lit;
      const Token v = Cur();
      switch (v.kind) {
        case Tok::IntLit: kc.kind = ConstKind::Int; kc.text = v.lit; Advance(); break;
        case Tok::UintLit: kc.kind = ConstKind::Uint; kc.text = v.lit; Advance(); break;
        case Tok::FloatLit: kc.kind = ConstKind::Float; kc.text = v.lit; Advance(); break;
        case Tok::StringLit: kc.kind = ConstKind::String; kc.text = v.lit; Advance(); break;
        case Tok::True:
        case Tok::False: kc.kind = ConstKind::Bool; kc.text = v.lit; Advance(); break;
        default: Error(v.pos, std::string("expected constant value, found ") + TokName(v.kind));
      }
      args.push_back(kc);
      if (At(Tok::Comma)) {
        Advance();
        continue;
      }
      break;
    }
    Expect(Tok::RParen);
    return args;
  }

  bool ParseKernel(std::vector<Annotation> anns, Kernel* k) {
    const Token kw = Expect(Tok::Kernel);
    const Token name = Expect(Tok::Ident);
    if (!name.pos.valid()) {
      Sync();
      return false;
    }
    k->pos = kw.pos;
    k->anns = std::move(anns);
    k->name = name.lit;
    Expect(Tok::LParen);
    while (!At(Tok::RParen) && !At(Tok::Eof)) {
      const Token pn = Expect(Tok::Ident);
      if (!pn.pos.valid()) {
        Sync();
        break;
      }
      Expect(Tok::Colon);
      Param p;
      p.pos = pn.pos;
      p.name = pn.lit;
      p.type = ParseType();
      k->params.push_back(std::move(p));
      if (At(Tok::Comma)) {
        Advance();
        continue;
      }
      break;
    }
    Expect(Tok::RParen);
    Expect(Tok::Arrow);
    if (At(Tok::LParen)) {  // several outputs (extension)
      Advance();
      while (!At(Tok::RParen) && !At(Tok::Eof)) {
        k->rets.push_back(ParseType());
        if (At(Tok::Comma)) {
          Advance();
          continue;
        }
        break;
      }
      Expect(Tok::RParen);
    } else {
      k->rets.push_back(ParseType());
    }
    Expect(Tok::LBrace);
    while (!At(Tok::RBrace) && !At(Tok::Eof)) {
      Stmt s;
      const size_t before = pos_;
      if (ParseStmt(&s)) k->body.push_back(std::move(s));
      // A statement that fails on a token its recovery stops at ('kernel',
      // '@') consumes nothing; the body then ends there, so the module loop
      // takes that declaration up again.
      if (pos_ == before) break;
    }
    Expect(Tok::RBrace);
    return true;
  }

  // ----------------------------------------------------------------- types
  Type ParseType() {
    Type t;
    t.pos = Cur().pos;
    t.present = true;
    if (At(Tok::Ident) && Cur().lit == "tensor") {
      Advance();
      t.tensor = true;
      Expect(Tok::Lt);
      ExpectContextual("dtype");
      Expect(Tok::Assign);
      const Token e = Cur();
      if (!IsElemTok(e.kind)) {
        Error(e.pos, std::string("tensor dtype must be an element type, found ") + TokName(e.kind));
        Sync();
        t.elem = "f32";
        return t;
      }
      Advance();
      t.elem = e.lit;
      while (At(Tok::Comma)) {
        Advance();
        if (At(Tok::Ident) && Cur().lit == "shape") {
          Advance();
          Expect(Tok::Assign);
          Expect(Tok::LBracket);
          t.has_shape = true;
          t.shape = ShapeDims();
          Expect(Tok::RBracket);
        }
      }
      Expect(Tok::Gt);
      return t;
    }
    if (IsElemTok(Cur().kind)) {
      t.elem = Advance().lit;
      return t;
    }
    Error(Cur().pos, std::string("expected type, found ") + TokName(Cur().kind));
    t.elem = "f32";
    return t;
  }

  std::vector<ShapeDim> ShapeDims() {
    std::vector<ShapeDim> dims;
    while (!At(Tok::RBracket) && !At(Tok::Eof)) {
      const Token t = Cur();
      ShapeDim d;
      d.pos = t.pos;
      if (t.kind == Tok::UintLit) {
        Advance();
        d.extent = static_cast<uint64_t>(t.ival);
      } else if (t.kind == Tok::Ident) {
        Advance();
        d.name = t.lit;
      } else {
        Error(t.pos, std::string("expected shape dimension (uint literal or identifier), found ") + TokName(t.kind));
        Advance();
        return dims;
      }
      dims.push_back(d);
      if (At(Tok::Comma)) {
        Advance();
        continue;
      }
      break;
    }
    return dims;
  }

  // ------------------------------------------------------------ statements
  bool ParseStmt(Stmt* s) {
    s->pos = Cur().pos;
    switch (Cur().kind) {
      case Tok::DimVar: {
        Advance();
        s->kind = StmtKind::DimVar;
        const bool paren = At(Tok::LParen);
        if (paren) Advance();
        s->names = IdentList();
        if (paren) Expect(Tok::RParen);
        Expect(Tok::Semi);
        return true;
      }
      case Tok::Let: {
        Advance();
        s->kind = StmtKind::Let;
        s->name = Expect(Tok::Ident).lit;
        if (At(Tok::Colon)) {
          Advance();
          s->type = ParseType();
        }
        Expect(Tok::Assign);
        StageChain(&s->chain);
        Expect(Tok::Semi);
        return true;
      }
      case Tok::Return: {
        Advance();
        s->kind = StmtKind::Return;
        s->name = Expect(Tok::Ident).lit;
        s->names.push_back(s->name);
        while (At(Tok::Comma)) {  // several outputs (extension)
          Advance();
          s->names.push_back(Expect(Tok::Ident).lit);
        }
        Expect(Tok::Semi);
        return true;
      }
      default:
        Error(Cur().pos, std::string("expected statement, found ") + TokName(Cur().kind));
        Sync();
        return false;
    }
  }

  std::vector<std::string> IdentList() {
    std::vector<std::string> names;
    while (At(Tok::Ident)) {
      names.push_back(Advance().lit);
      if (At(Tok::Comma)) {
        Advance();
        continue;
      }
      break;
    }
    return names;
  }

  void StageChain(std::vector<Stage>* out) {
    for (;;) {
      Stage st;
      if (ParseStage(&st)) out->push_back(std::move(st));
      if (!At(Tok::Pipe)) break;
      Advance();  // the pipe (the escape was decided inside the '|' level)
    }
  }

  bool ParseStage(Stage* st) {
    st->pos = Cur().pos;
    if (At(Tok::Map)) {
      Advance();
      st->is_map = true;
      Expect(Tok::On);
      Expect(Tok::LParen);
      while (At(Tok::Ident)) {
        Binding b;
        b.pos = Cur().pos;
        b.tensor = Advance().lit;
        while (At(Tok::LBracket)) {
          Advance();
          const Token d = Expect(Tok::Ident);
          if (d.pos.valid()) b.dims.push_back(d.lit);
          Expect(Tok::RBracket);
        }
        st->bindings.push_back(b);
        if (At(Tok::Comma)) {
          Advance();
          continue;
        }
        break;
      }
      Expect(Tok::RParen);
      if (At(Tok::As)) DimList(st);
      return ParseLambda(&st->lambda);
    }
    if (At(Tok::Reduce)) {
      Advance();
      st->is_map = false;
      Expect(Tok::LParen);
      if (At(Tok::Init)) {
        Advance();
        Expect(Tok::Assign);
        st->init = ExprNested();
      }
      Expect(Tok::RParen);
      Expect(Tok::On);
      Expect(Tok::LParen);
      st->on_params = ParamSpecs();
      Expect(Tok::RParen);
      if (At(Tok::As)) DimList(st);
      Expect(Tok::Arrow);
      const Token rt = Cur();
      if (IsElemTok(rt.kind)) {
        st->ret = Advance().lit;
      } else {
        Error(rt.pos, std::string("reduce requires '->' scalarType, found ") + TokName(rt.kind));
        st->ret = "f32";
      }
      Expect(Tok::Colon);
      st->body = ExprTop();
      return true;
    }
    Error(Cur().pos, std::string("expected stage (map or reduce), found ") + TokName(Cur().kind));
    Sync();
    return false;
  }

  void DimList(Stage* st) {
    Advance();  // 'as'
    Expect(Tok::LParen);
    st->has_as = true;
    st->as = IdentList();
    Expect(Tok::RParen);
  }

  bool ParseLambda(Lambda* l) {
    l->pos = Cur().pos;
    if (At(Tok::LBracket)) {
      Advance();
      l->captures = IdentList();
      Expect(Tok::RBracket);
    }
    Expect(Tok::LParen);
    l->params = ParamSpecs();
    Expect(Tok::RParen);
    if (At(Tok::Arrow)) {
      Advance();
      const Token rt = Cur();
      if (IsElemTok(rt.kind)) {
        l->ret = Advance().lit;
      } else {
        Error(rt.pos, std::string("lambda return annotation must be an element type, found ") + TokName(rt.kind));
        l->ret = "f32";
      }
    }
    Expect(Tok::Colon);
    l->body = ExprTop();
    return true;
  }

  std::vector<ParamSpec> ParamSpecs() {
    std::vector<ParamSpec> specs;
    while (!At(Tok::RParen) && !At(Tok::Eof)) {
      const Token t = Cur();
      ParamSpec ps;
      ps.pos = t.pos;
      bool ok = true;
      if (t.kind == Tok::Placeholder) {
        Advance();
        if (t.ival != 0) Error(t.pos, "placeholder " + t.lit + " is reserved in v0 (only %0 is legal, design §7.3)");
        ps.pipe = true;
        ps.name = t.lit;
        if (At(Tok::Colon)) {
          Advance();
          if (IsElemTok(Cur().kind)) {
            ps.type = Advance().lit;
          } else {
            Error(Cur().pos, std::string("placeholder annotation must be an element type, found ") + TokName(Cur().kind));
          }
        }
      } else if (t.kind == Tok::Ident) {
        Advance();
        ps.name = t.lit;
        Expect(Tok::Colon);
        if (IsElemTok(Cur().kind)) {
          ps.type = Advance().lit;
        } else {
          Error(Cur().pos, "parameter " + t.lit + " requires an element type, found " + TokName(Cur().kind));
          ps.type = "f32";
        }
      } else {
        Error(t.pos, std::string("expected stage parameter, found ") + TokName(t.kind));
        ok = false;
      }
      if (ok) specs.push_back(ps);
      if (At(Tok::Comma)) {
        Advance();
        continue;
      }
      break;
    }
    return specs;
  }

  // ----------------------------------------------------------- expressions
  ExprP ExprTop() {
    const bool saved = allow_pipe_;
    allow_pipe_ = true;
    ExprP e = Ternary();
    allow_pipe_ = saved;
    return e;
  }
  ExprP ExprNested() {
    const bool saved = allow_pipe_;
    allow_pipe_ = false;
    ExprP e = Ternary();
    allow_pipe_ = saved;
    return e;
  }

  static ExprP Binary(const Token& t, ExprP l, ExprP r) {
    ExprP e(new Expr);
    e->kind = ExprKind::Binary;
    e->pos = t.pos;
    e->text = t.lit;
    e->kids.push_back(std::move(l));
    e->kids.push_back(std::move(r));
    return e;
  }

  // ternary ::= lor [ '?' expr ':' expr ]; the branches keep the caller's
  // pipe allowance.
  ExprP Ternary() {
    ExprP x = Lor();
    if (!At(Tok::Question)) return x;
    const Token q = Advance();
    ExprP then = Ternary();
    Expect(Tok::Colon);
    ExprP els = Ternary();
    ExprP e(new Expr);
    e->kind = ExprKind::Select;
    e->pos = q.pos;
    e->kids.push_back(std::move(x));
    e->kids.push_back(std::move(then));
    e->kids.push_back(std::move(els));
    return e;
  }
  ExprP Lor() {
    ExprP x = Land();
    while (At(Tok::OrOr)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Land());
    }
    return x;
  }
  ExprP Land() {
    ExprP x = Bitor();
    while (At(Tok::AndAnd)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Bitor());
    }
    return x;
  }
  // The pipe escape: at a stage body's top level, '|' followed by `map` or
  // `reduce` ends the stage and is left for the chain.
  ExprP Bitor() {
    ExprP x = Bitxor();
    while (At(Tok::Pipe)) {
      if (allow_pipe_) {
        const Tok nk = PeekTok(1).kind;
        if (nk == Tok::Map || nk == Tok::Reduce) return x;
      }
      const Token t = Advance();
      x = Binary(t, std::move(x), Bitxor());
    }
    return x;
  }
  ExprP Bitxor() {
    ExprP x = Bitand();
    while (At(Tok::Caret)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Bitand());
    }
    return x;
  }
  ExprP Bitand() {
    ExprP x = Equality();
    while (At(Tok::Amp)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Equality());
    }
    return x;
  }
  ExprP Equality() {
    ExprP x = Relational();
    while (At(Tok::EqEq) || At(Tok::Ne)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Relational());
    }
    return x;
  }
  ExprP Relational() {
    ExprP x = Shift();
    while (At(Tok::Lt) || At(Tok::Le) || At(Tok::Gt) || At(Tok::Ge)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Shift());
    }
    return x;
  }
  ExprP Shift() {
    ExprP x = Additive();
    while (At(Tok::Shl) || At(Tok::Shr)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Additive());
    }
    return x;
  }
  ExprP Additive() {
    ExprP x = Multiplicative();
    while (At(Tok::Plus) || At(Tok::Minus)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Multiplicative());
    }
    return x;
  }
  ExprP Multiplicative() {
    ExprP x = Unary();
    while (At(Tok::Star) || At(Tok::Slash) || At(Tok::Percent)) {
      const Token t = Advance();
      x = Binary(t, std::move(x), Unary());
    }
    return x;
  }
  ExprP Unary() {
    if (At(Tok::Minus) || At(Tok::Plus) || At(Tok::Bang) || At(Tok::Tilde)) {
      const Token t = Advance();
      ExprP e(new Expr);
      e->kind = ExprKind::Unary;
      e->pos = t.pos;
      e->text = t.lit;
      e->kids.push_back(Unary());
      return e;
    }
    return Primary();
  }
  ExprP Primary() {
    const Token t = Cur();
    ExprP e(new Expr);
    e->pos = t.pos;
    switch (t.kind) {
      case Tok::IntLit:
      case Tok::UintLit:
        Advance();
        e->kind = ExprKind::Lit;
        e->lit = t.kind == Tok::IntLit ? LitKind::Int : LitKind::Uint;
        e->text = t.lit;
        e->ival = t.ival;
        return e;
      case Tok::FloatLit:
        Advance();
        e->kind = ExprKind::Lit;
        e->lit = LitKind::Float;
        e->text = t.lit;
        e->fval = t.fval;
        return e;
      case Tok::True:
      case Tok::False:
        Advance();
        e->kind = ExprKind::Lit;
        e->lit = LitKind::Bool;
        e->text = t.lit;
        e->bval = t.kind == Tok::True;
        return e;
      case Tok::InfF32:
        Advance();
        e->kind = ExprKind::Lit;
        e->lit = LitKind::Float;
        e->text = t.lit;
        e->fval = std::numeric_limits<float>::infinity();
        return e;
      case Tok::Ident:
        if (PeekTok(1).kind == Tok::LParen) {
          Advance();
          Advance();  // '('
          e->kind = ExprKind::Call;
          e->text = t.lit;
          while (!At(Tok::RParen) && !At(Tok::Eof)) {
            e->kids.push_back(ExprNested());
            if (At(Tok::Comma)) {
              Advance();
              continue;
            }
            break;
          }
          Expect(Tok::RParen);
          return e;
        }
        Advance();
        e->kind = ExprKind::Name;
        e->text = t.lit;
        return e;
      case Tok::LParen: {
        Advance();
        ExprP x = ExprNested();
        Expect(Tok::RParen);
        return x;
      }
      case Tok::Placeholder:
        Advance();
        if (t.ival != 0) Error(t.pos, "placeholder " + t.lit + " is reserved in v0 (only %0 is legal, design §7.3)");
        e->kind = ExprKind::Pipe;
        e->text = "%0";
        return e;
      default:
        if (IsElemTok(t.kind)) {  // cast: elem '(' expr ')'
          Advance();
          Expect(Tok::LParen);
          e->kind = ExprKind::Cast;
          e->cast_to = t.lit;
          e->kids.push_back(ExprNested());
          Expect(Tok::RParen);
          return e;
        }
        Error(t.pos, std::string("expected expression, found ") + TokName(t.kind));
        return nullptr;
    }
  }

  std::vector<Token> toks_;
  std::vector<Diagnostic>* diags_;
  size_t pos_ = 0;
  bool allow_pipe_ = false;
};

}  // namespace

Module Parse(const std::string& file, const std::string& src, std::vector<Diagnostic>* diags) {
  std::vector<Token> toks = Scan(file, src, diags);
  return Parser(std::move(toks), diags).ParseModule();
}

}  // namespace syntax
}  // namespace tca
