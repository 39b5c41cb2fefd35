// lexer.cpp — the .tca scanner. Behaviour follows internal/syntax/lexer/
// lexer.go:100-409 and token.go (token set, keyword table, literal rules and
// their error messages); the implementation is a single forward pass over
// the bytes with UTF-8 aware columns.
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <map>

#include "syntax.h"

namespace tca {
namespace syntax {

namespace {

const std::map<std::string, Tok>& Keywords() {
  static const std::map<std::string, Tok> k = {
      {"kernel", Tok::Kernel}, {"let", Tok::Let},       {"return", Tok::Return}, {"dimvar", Tok::DimVar},
      {"map", Tok::Map},       {"on", Tok::On},         {"as", Tok::As},         {"reduce", Tok::Reduce},
      {"init", Tok::Init},     {"true", Tok::True},     {"false", Tok::False},   {"inf_f32", Tok::InfF32},
      {"bool", Tok::TBool},    {"f32", Tok::TF32},      {"f16", Tok::TF16},      {"bf16", Tok::TBF16},
      {"i8", Tok::TI8},        {"i16", Tok::TI16},      {"i32", Tok::TI32},      {"u8", Tok::TU8},
      {"u16", Tok::TU16},      {"u32", Tok::TU32},
  };
  return k;
}

bool IsDigit(unsigned char c) { return c >= '0' && c <= '9'; }
// Identifier characters: ASCII letters, '_' and any byte of a multi-byte
// UTF-8 sequence (non-ASCII letters).
bool IsLetter(unsigned char c) { return c == '_' || (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || c >= 0x80; }

class Scanner {
 public:
  Scanner(const std::string& file, const std::string& src, std::vector<Diagnostic>* diags)
      : file_(file), src_(src), diags_(diags) {}

  std::vector<Token> Run() {
    std::vector<Token> out;
    for (;;) {
      SkipSpaceAndComments();
      Token t;
      t.pos = Here();
      if (off_ >= src_.size()) {
        t.kind = Tok::Eof;
        out.push_back(t);
        return out;
      }
      const unsigned char c = src_[off_];
      if (IsLetter(c)) {
        Identifier(&t);
      } else if (IsDigit(c)) {
        Number(&t);
      } else if (c == '"') {
        String(&t);
      } else if (c == '%' && off_ + 1 < src_.size() && IsDigit(src_[off_ + 1])) {
        Placeholder(&t);
      } else {
        Operator(&t);
      }
      out.push_back(t);
    }
  }

 private:
  Pos Here() const {
    Pos p;
    p.file = file_;
    p.line = line_;
    p.col = col_;
    return p;
  }
  void Error(const Pos& p, const std::string& msg) {
    Diagnostic d;
    d.pos = p;
    d.msg = msg;
    diags_->push_back(d);
  }
  void Advance() {
    if (off_ >= src_.size()) return;
    const unsigned char c = src_[off_++];
    if (c == '\n') {
      ++line_;
      col_ = 1;
    } else if ((c & 0xC0) != 0x80) {
      // one column per code point: continuation bytes do not advance it
      if (off_ < src_.size() && (static_cast<unsigned char>(src_[off_]) & 0xC0) == 0x80) {
        while (off_ < src_.size() && (static_cast<unsigned char>(src_[off_]) & 0xC0) == 0x80) ++off_;
      }
      ++col_;
    }
  }
  char Cur() const { return off_ < src_.size() ? src_[off_] : '\0'; }
  char Peek() const { return off_ + 1 < src_.size() ? src_[off_ + 1] : '\0'; }
  bool AtEnd() const { return off_ >= src_.size(); }

  void SkipSpaceAndComments() {
    for (;;) {
      const char c = Cur();
      if (!AtEnd() && (c == ' ' || c == '\t' || c == '\r' || c == '\n')) {
        Advance();
      } else if (c == '/' && Peek() == '/') {
        while (!AtEnd() && Cur() != '\n') Advance();
      } else if (c == '/' && Peek() == '*') {
        const Pos start = Here();
        Advance();
        Advance();
        for (;;) {
          if (AtEnd()) {
            Error(start, "block comment not terminated");
            break;
          }
          if (Cur() == '*' && Peek() == '/') {
            Advance();
            Advance();
            break;
          }
          Advance();
        }
      } else {
        return;
      }
    }
  }

  void Identifier(Token* t) {
    const size_t start = off_;
    while (!AtEnd() && (IsLetter(Cur()) || IsDigit(Cur()))) Advance();
    t->lit = src_.substr(start, off_ - start);
    auto it = Keywords().find(t->lit);
    t->kind = it == Keywords().end() ? Tok::Ident : it->second;
  }

  // Consumes the rest of an alphanumeric run and reports it as one
  // malformed literal ("123abc", "1.5fx").
  void Malformed(Token* t, size_t start) {
    while (!AtEnd() && (IsLetter(Cur()) || IsDigit(Cur()))) Advance();
    t->kind = Tok::Illegal;
    t->lit = src_.substr(start, off_ - start);
    Error(t->pos, "malformed numeric literal \"" + t->lit + "\"");
  }

  void Number(Token* t) {
    const size_t start = off_;
    bool is_float = false;
    while (IsDigit(Cur())) Advance();
    if (Cur() == '.') {
      is_float = true;
      Advance();
      if (!IsDigit(Cur())) Error(t->pos, "malformed float literal: expected digits after '.'");
      while (IsDigit(Cur())) Advance();
    }
    if (Cur() == 'e' || Cur() == 'E') {
      is_float = true;
      Advance();
      if (Cur() == '+' || Cur() == '-') Advance();
      if (!IsDigit(Cur())) Error(t->pos, "malformed float literal: exponent has no digits");
      while (IsDigit(Cur())) Advance();
    }
    std::string digits = src_.substr(start, off_ - start);
    if (is_float) {
      if (Cur() != 'f' && Cur() != 'F') {
        t->kind = Tok::Illegal;
        t->lit = digits;
        Error(t->pos, "float literal \"" + digits + "\" requires the f/F suffix (design §2.1)");
        return;
      }
      Advance();
      if (!AtEnd() && (IsLetter(Cur()) || IsDigit(Cur()))) return Malformed(t, start);
      t->lit = src_.substr(start, off_ - start);
      errno = 0;
      char* end = nullptr;
      const float v = std::strtof(digits.c_str(), &end);  // rounds once, straight to f32
      if (errno == ERANGE && (v == HUGE_VALF || v == -HUGE_VALF)) {
        t->kind = Tok::Illegal;
        Error(t->pos, "malformed float literal \"" + t->lit + "\": value out of range");
        return;
      }
      t->kind = Tok::FloatLit;
      t->fval = v;
      return;
    }
    if (Cur() == 'u' || Cur() == 'U') {
      Advance();
      if (!AtEnd() && (IsLetter(Cur()) || IsDigit(Cur()))) return Malformed(t, start);
      t->lit = src_.substr(start, off_ - start);
      const unsigned long long v = std::strtoull(digits.c_str(), nullptr, 10);
      if (digits.size() > 10 || v > 0xFFFFFFFFull) {
        t->kind = Tok::Illegal;
        Error(t->pos, "uint literal \"" + t->lit + "\" does not fit u32");
        return;
      }
      t->kind = Tok::UintLit;
      t->ival = static_cast<int64_t>(v);
      return;
    }
    if (!AtEnd() && IsLetter(Cur())) return Malformed(t, start);
    t->lit = digits;
    const unsigned long long v = std::strtoull(digits.c_str(), nullptr, 10);
    if (digits.size() > 10 || v > 0x7FFFFFFFull) {
      t->kind = Tok::Illegal;
      Error(t->pos, "int literal \"" + digits + "\" does not fit i32");
      return;
    }
    t->kind = Tok::IntLit;
    t->ival = static_cast<int64_t>(v);
  }

  void String(Token* t) {
    Advance();  // opening quote
    const size_t start = off_;
    while (Cur() != '"') {
      if (AtEnd() || Cur() == '\n') {
        t->kind = Tok::Illegal;
        t->lit = src_.substr(start, off_ - start);
        Error(t->pos, "string literal not terminated");
        return;
      }
      Advance();
    }
    t->lit = src_.substr(start, off_ - start);
    Advance();  // closing quote
    t->kind = Tok::StringLit;
  }

  void Placeholder(Token* t) {
    const size_t start = off_;
    Advance();  // '%'
    while (IsDigit(Cur())) Advance();
    t->lit = src_.substr(start, off_ - start);
    const std::string n = t->lit.substr(1);
    if (n.size() > 9) {
      t->kind = Tok::Illegal;
      Error(t->pos, "malformed placeholder \"" + t->lit + "\"");
      return;
    }
    t->kind = Tok::Placeholder;
    t->ival = std::strtoll(n.c_str(), nullptr, 10);
  }

  void Operator(Token* t) {
    const char c = Cur();
    Advance();
    auto one = [&](Tok k, const char* s) {
      t->kind = k;
      t->lit = s;
    };
    auto two = [&](Tok k, const char* s) {
      Advance();
      t->kind = k;
      t->lit = s;
    };
    switch (c) {
      case '@': return one(Tok::At, "@");
      case '(': return one(Tok::LParen, "(");
      case ')': return one(Tok::RParen, ")");
      case '[': return one(Tok::LBracket, "[");
      case ']': return one(Tok::RBracket, "]");
      case '{': return one(Tok::LBrace, "{");
      case '}': return one(Tok::RBrace, "}");
      case ',': return one(Tok::Comma, ",");
      case ';': return one(Tok::Semi, ";");
      case ':': return one(Tok::Colon, ":");
      case '?': return one(Tok::Question, "?");
      case '~': return one(Tok::Tilde, "~");
      case '+': return one(Tok::Plus, "+");
      case '*': return one(Tok::Star, "*");
      case '/': return one(Tok::Slash, "/");
      case '^': return one(Tok::Caret, "^");
      case '%': return one(Tok::Percent, "%");
      case '<':
        if (Cur() == '<') return two(Tok::Shl, "<<");
        if (Cur() == '=') return two(Tok::Le, "<=");
        return one(Tok::Lt, "<");
      case '>':
        if (Cur() == '>') return two(Tok::Shr, ">>");
        if (Cur() == '=') return two(Tok::Ge, ">=");
        return one(Tok::Gt, ">");
      case '=':
        if (Cur() == '=') return two(Tok::EqEq, "==");
        return one(Tok::Assign, "=");
      case '!':
        if (Cur() == '=') return two(Tok::Ne, "!=");
        return one(Tok::Bang, "!");
      case '-':
        if (Cur() == '>') return two(Tok::Arrow, "->");
        return one(Tok::Minus, "-");
      case '&':
        if (Cur() == '&') return two(Tok::AndAnd, "&&");
        return one(Tok::Amp, "&");
      case '|':
        if (Cur() == '|') return two(Tok::OrOr, "||");
        return one(Tok::Pipe, "|");
      default: {
        t->kind = Tok::Illegal;
        t->lit = std::string(1, c);
        std::string shown = (static_cast<unsigned char>(c) >= 0x20 && static_cast<unsigned char>(c) < 0x7f)
                                ? std::string("'") + c + "'"
                                : "byte 0x" + std::string(1, "0123456789abcdef"[(c >> 4) & 15]) +
                                      std::string(1, "0123456789abcdef"[c & 15]);
        Error(t->pos, "unexpected character " + shown);
        return;
      }
    }
  }

  std::string file_;
  const std::string& src_;
  std::vector<Diagnostic>* diags_;
  size_t off_ = 0;
  int line_ = 1, col_ = 1;
};

}  // namespace

const char* TokName(Tok k) {
  switch (k) {
    case Tok::Illegal: return "Illegal";
    case Tok::Eof: return "EOF";
    case Tok::Ident: return "identifier";
    case Tok::IntLit: return "int literal";
    case Tok::UintLit: return "uint literal";
    case Tok::FloatLit: return "float literal";
    case Tok::StringLit: return "string literal";
    case Tok::Placeholder: return "%N placeholder";
    case Tok::Kernel: return "kernel";
    case Tok::Let: return "let";
    case Tok::Return: return "return";
    case Tok::DimVar: return "dimvar";
    case Tok::Map: return "map";
    case Tok::On: return "on";
    case Tok::As: return "as";
    case Tok::Reduce: return "reduce";
    case Tok::Init: return "init";
    case Tok::True: return "true";
    case Tok::False: return "false";
    case Tok::InfF32: return "inf_f32";
    case Tok::TBool: return "bool";
    case Tok::TF32: return "f32";
    case Tok::TF16: return "f16";
    case Tok::TBF16: return "bf16";
    case Tok::TI8: return "i8";
    case Tok::TI16: return "i16";
    case Tok::TI32: return "i32";
    case Tok::TU8: return "u8";
    case Tok::TU16: return "u16";
    case Tok::TU32: return "u32";
    case Tok::At: return "@";
    case Tok::LParen: return "(";
    case Tok::RParen: return ")";
    case Tok::LBracket: return "[";
    case Tok::RBracket: return "]";
    case Tok::LBrace: return "{";
    case Tok::RBrace: return "}";
    case Tok::Lt: return "<";
    case Tok::Gt: return ">";
    case Tok::Comma: return ",";
    case Tok::Semi: return ";";
    case Tok::Colon: return ":";
    case Tok::Assign: return "=";
    case Tok::Question: return "?";
    case Tok::Pipe: return "|";
    case Tok::Amp: return "&";
    case Tok::Caret: return "^";
    case Tok::Tilde: return "~";
    case Tok::Bang: return "!";
    case Tok::Plus: return "+";
    case Tok::Minus: return "-";
    case Tok::Star: return "*";
    case Tok::Slash: return "/";
    case Tok::Percent: return "%";
    case Tok::Arrow: return "->";
    case Tok::EqEq: return "==";
    case Tok::Ne: return "!=";
    case Tok::Le: return "<=";
    case Tok::Ge: return ">=";
    case Tok::AndAnd: return "&&";
    case Tok::OrOr: return "||";
    case Tok::Shl: return "<<";
    case Tok::Shr: return ">>";
  }
  return "?";
}

bool IsElemTok(Tok k) {
  switch (k) {
    case Tok::TBool: case Tok::TF32: case Tok::TF16: case Tok::TBF16: case Tok::TI8:
    case Tok::TI16: case Tok::TI32: case Tok::TU8: case Tok::TU16: case Tok::TU32:
      return true;
    default:
      return false;
  }
}

std::vector<Token> Scan(const std::string& file, const std::string& src, std::vector<Diagnostic>* diags) {
  return Scanner(file, src, diags).Run();
}

std::string Diagnostic::String() const {
  std::string s = pos.file.empty() ? "<source>" : pos.file;
  if (pos.valid()) s += ":" + std::to_string(pos.line) + ":" + std::to_string(pos.col);
  return s + (error ? ": error: " : ": warning: ") + msg;
}

bool HasErrors(const std::vector<Diagnostic>& d) {
  for (const auto& x : d)
    if (x.error) return true;
  return false;
}

std::string JoinDiagnostics(const std::vector<Diagnostic>& d, bool errors_only) {
  std::string s;
  for (const auto& x : d) {
    if (errors_only && !x.error) continue;
    if (!s.empty()) s += "\n";
    s += x.String();
  }
  return s;
}

}  // namespace syntax
}  // namespace tca
