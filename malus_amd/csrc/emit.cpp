// HIP emitter: malus `kernel` items -> HIP C++ for hipRTC on gfx950.
//
// Replaces the MSL emitter of crates/malus-codegen-gpu/src/lib.rs.  The
// reference lowers sema's typed kernels; with no Rust front end here, this
// file carries its own lexer, parser and type checker for the kernel
// sub-language, following the reference's rules:
//   - syntax: indentation blocks, Pratt precedence and `let shared`
//     (crates/malus-syntax/src/lexer.rs, parser.rs:332-680);
//   - kernel-body typing (crates/malus-sema/src/check.rs:432-501, 948-1080,
//     2261-2290): integer literals default to i32, thread intrinsics, loop
//     variables, t.shape[k], t.strides[k] and t.ndim are i32, binary operands
//     must have one type, a comparison yields its operand type;
//   - form selection (check.rs:574-588): a body of only lets and a final
//     return is an implicit map, anything else is explicit.
// Each kernel becomes one `extern "C" __global__ malus_kernel_<id>` with the
// runtime's launch ABI (dispatch.cpp):
//   v1 (implicit form, synthesized builtins): (in..., out, unsigned n), one
//      thread per output element, tid < n guarded;
//   v2 (explicit form): (in..., out, [Uniforms_<id> u], TensorMeta per input,
//      TensorMeta out), the uniforms struct by value in parameter order, one
//      4-byte slot per scalar as the JIT packs them
//      (codegen-cpu/lib.rs:2261-2293).
// exp/log/tanh/pow/rsqrt are evaluated in double and rounded once (correctly
// rounded f32), as the library's hand-written kernels and the oracle do.

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <sstream>
#include <string>
#include <vector>

#include "api.h"
#include "common.h"

namespace malus {
bool dispatch_has_builtin(const std::string& name);  // dispatch.cpp
}

namespace {

using malus::fail;

// ---- types ----------------------------------------------------------------
enum class Sc { F32, F16, BF16, I8, I16, I32, I64, U8, U16, U32, U64 };

bool sc_from_name(const std::string& n, Sc* out) {
  static const std::map<std::string, Sc> m = {{"f32", Sc::F32}, {"f16", Sc::F16}, {"bf16", Sc::BF16},
                                              {"i8", Sc::I8},   {"i16", Sc::I16}, {"i32", Sc::I32},
                                              {"i64", Sc::I64}, {"u8", Sc::U8},   {"u16", Sc::U16},
                                              {"u32", Sc::U32}, {"u64", Sc::U64}};
  auto it = m.find(n);
  if (it == m.end()) return false;
  *out = it->second;
  return true;
}
bool sc_is_float(Sc s) { return s == Sc::F32 || s == Sc::F16 || s == Sc::BF16; }
const char* sc_name(Sc s) {
  static const char* n[] = {"f32", "f16", "bf16", "i8", "i16", "i32", "i64", "u8", "u16", "u32", "u64"};
  return n[(int)s];
}
int sc_bytes(Sc s) {
  static const int n[] = {4, 2, 2, 1, 2, 4, 8, 1, 2, 4, 8};
  return n[(int)s];
}
// dtype_to_msl (codegen-gpu/lib.rs:1060-1074), mapped to HIP C++ types.
const char* sc_hip(Sc s) {
  static const char* n[] = {"float",      "_Float16",       "__bf16",         "signed char",
                            "short",      "int",            "long long",      "unsigned char",
                            "unsigned short", "unsigned int", "unsigned long long"};
  return n[(int)s];
}

struct Ty {
  enum K { None, Scalar, Tensor, Array, Bool, Unit } k = None;
  Sc s = Sc::F32;
  long long len = 0;
  static Ty scalar(Sc s) { Ty t; t.k = Scalar; t.s = s; return t; }
  static Ty tensor(Sc s) { Ty t; t.k = Tensor; t.s = s; return t; }
  static Ty unit() { Ty t; t.k = Unit; return t; }
  static Ty boolean() { Ty t; t.k = Bool; return t; }
  bool operator==(const Ty& o) const {
    if (k != o.k) return false;
    if (k == Scalar || k == Tensor) return s == o.s;
    if (k == Array) return s == o.s && len == o.len;
    return true;
  }
  bool operator!=(const Ty& o) const { return !(*this == o); }
  bool is_int() const { return k == Scalar && !sc_is_float(s); }
  std::string str() const {
    switch (k) {
      case Scalar: return sc_name(s);
      case Tensor: return std::string("Tensor<") + sc_name(s) + ">";
      case Array: return std::string("Array<") + sc_name(s) + ", " + std::to_string(len) + ">";
      case Bool: return "bool";
      case Unit: return "()";
      default: return "<unsupported type>";
    }
  }
};

// ---- lexer (crates/malus-syntax/src/lexer.rs) -------------------------------
enum class Tk {
  Ident, Int, Float, Str, Newline, Indent, Dedent, Eof,
  LParen, RParen, LBracket, RBracket, LBrace, RBrace, Comma, Colon, Dot, Arrow,
  Plus, Minus, Star, StarStar, Slash, At, Percent, Assign, EqEq, NotEq, Lt, LtEq, Gt, GtEq, Other,
  KwKernel, KwFn, KwLet, KwMut, KwReturn, KwIf, KwElse, KwFor, KwIn, KwWhile, KwBreak, KwContinue,
  KwAnd, KwOr, KwNot, KwTrue, KwFalse, KwInout, KwItem,  // KwItem: struct/enum/trait/impl/import/from/with/match
};

struct Token {
  Tk k;
  std::string text;
  long long ival = 0;
  double fval = 0;
  int line = 0;
};

class Lexer {
 public:
  explicit Lexer(const std::string& src) : s_(src) {}

  std::vector<Token> run() {
    indents_.push_back(0);
    at_line_start_ = true;
    while (true) {
      if (at_line_start_) {
        if (!line_start()) continue;
      }
      if (pos_ >= s_.size()) break;
      char c = s_[pos_];
      if (c == '\n') {
        ++line_;
        ++pos_;
        if (depth_ == 0) push(Tk::Newline, "\\n");
        at_line_start_ = true;
        continue;
      }
      if (c == ' ' || c == '\t' || c == '\r') { ++pos_; continue; }
      if (c == '#') { while (pos_ < s_.size() && s_[pos_] != '\n') ++pos_; continue; }
      if (isalpha((unsigned char)c) || c == '_') { ident(); continue; }
      if (isdigit((unsigned char)c)) { number(); continue; }
      if (c == '"') { str(); continue; }
      punct();
    }
    if (!out_.empty() && out_.back().k != Tk::Newline) push(Tk::Newline, "\\n");
    while (indents_.size() > 1) { indents_.pop_back(); push(Tk::Dedent, ""); }
    push(Tk::Eof, "");
    return out_;
  }

 private:
  // Handles indentation at the start of a line; returns false when the line
  // was blank or a comment (consumed), true when tokens follow.
  bool line_start() {
    size_t p = pos_;
    int width = 0;
    while (p < s_.size() && (s_[p] == ' ' || s_[p] == '\t')) { ++width; ++p; }
    if (p >= s_.size() || s_[p] == '\n' || s_[p] == '#' || s_[p] == '\r') {
      while (p < s_.size() && s_[p] != '\n') ++p;
      if (p < s_.size()) { ++p; ++line_; }
      pos_ = p;
      if (p >= s_.size()) at_line_start_ = false;
      return false;
    }
    pos_ = p;
    at_line_start_ = false;
    if (depth_ > 0) return true;
    if (width > indents_.back()) {
      indents_.push_back(width);
      push(Tk::Indent, "");
    } else {
      while (width < indents_.back()) {
        indents_.pop_back();
        push(Tk::Dedent, "");
      }
      if (width != indents_.back()) fail("malus: emit: line %d: inconsistent dedent", line_);
    }
    return true;
  }
  void push(Tk k, std::string t) {
    Token tok;
    tok.k = k;
    tok.text = std::move(t);
    tok.line = line_;
    out_.push_back(std::move(tok));
  }
  void ident() {
    size_t b = pos_;
    while (pos_ < s_.size() && (isalnum((unsigned char)s_[pos_]) || s_[pos_] == '_')) ++pos_;
    std::string t = s_.substr(b, pos_ - b);
    static const std::map<std::string, Tk> kw = {
        {"kernel", Tk::KwKernel}, {"fn", Tk::KwFn},         {"let", Tk::KwLet},       {"mut", Tk::KwMut},
        {"return", Tk::KwReturn}, {"if", Tk::KwIf},         {"else", Tk::KwElse},     {"for", Tk::KwFor},
        {"in", Tk::KwIn},         {"while", Tk::KwWhile},   {"break", Tk::KwBreak},   {"continue", Tk::KwContinue},
        {"and", Tk::KwAnd},       {"or", Tk::KwOr},         {"not", Tk::KwNot},       {"true", Tk::KwTrue},
        {"false", Tk::KwFalse},   {"inout", Tk::KwInout},   {"struct", Tk::KwItem},   {"enum", Tk::KwItem},
        {"trait", Tk::KwItem},    {"impl", Tk::KwItem},     {"import", Tk::KwItem},   {"from", Tk::KwItem},
        {"with", Tk::KwItem},     {"match", Tk::KwItem}};
    auto it = kw.find(t);
    push(it == kw.end() ? Tk::Ident : it->second, t);
  }
  void number() {
    size_t b = pos_;
    bool is_float = false;
    auto digits = [&] { while (pos_ < s_.size() && (isdigit((unsigned char)s_[pos_]) || s_[pos_] == '_')) ++pos_; };
    digits();
    if (pos_ + 1 < s_.size() && s_[pos_] == '.' && isdigit((unsigned char)s_[pos_ + 1])) {
      is_float = true;
      ++pos_;
      digits();
    }
    if (pos_ < s_.size() && (s_[pos_] == 'e' || s_[pos_] == 'E')) {
      is_float = true;
      ++pos_;
      if (pos_ < s_.size() && (s_[pos_] == '+' || s_[pos_] == '-')) ++pos_;
      if (pos_ >= s_.size() || !isdigit((unsigned char)s_[pos_])) fail("malus: emit: line %d: invalid number", line_);
      digits();
    }
    std::string raw;
    for (size_t i = b; i < pos_; ++i)
      if (s_[i] != '_') raw += s_[i];
    push(is_float ? Tk::Float : Tk::Int, raw);
    if (is_float) out_.back().fval = strtod(raw.c_str(), nullptr);
    else out_.back().ival = strtoll(raw.c_str(), nullptr, 10);
  }
  void str() {
    size_t b = ++pos_;
    while (pos_ < s_.size() && s_[pos_] != '"') {
      if (s_[pos_] == '\\') ++pos_;
      if (pos_ < s_.size() && s_[pos_] == '\n') ++line_;
      ++pos_;
    }
    push(Tk::Str, s_.substr(b, pos_ - b));
    if (pos_ < s_.size()) ++pos_;
  }
  void punct() {
    char c = s_[pos_];
    char n = pos_ + 1 < s_.size() ? s_[pos_ + 1] : '\0';
    auto two = [&](Tk k, const char* t) { pos_ += 2; push(k, t); };
    auto one = [&](Tk k) { push(k, std::string(1, c)); ++pos_; };
    switch (c) {
      case '(': ++depth_; one(Tk::LParen); return;
      case ')': if (depth_ > 0) --depth_; one(Tk::RParen); return;
      case '[': ++depth_; one(Tk::LBracket); return;
      case ']': if (depth_ > 0) --depth_; one(Tk::RBracket); return;
      case '{': ++depth_; one(Tk::LBrace); return;
      case '}': if (depth_ > 0) --depth_; one(Tk::RBrace); return;
      case ',': one(Tk::Comma); return;
      case ':': one(Tk::Colon); return;
      case '.': one(Tk::Dot); return;
      case '+': one(Tk::Plus); return;
      case '-': if (n == '>') two(Tk::Arrow, "->"); else one(Tk::Minus); return;
      case '*': if (n == '*') two(Tk::StarStar, "**"); else one(Tk::Star); return;
      case '/': one(Tk::Slash); return;
      case '@': one(Tk::At); return;
      case '%': one(Tk::Percent); return;
      case '=': if (n == '=') two(Tk::EqEq, "=="); else one(Tk::Assign); return;
      case '!': if (n == '=') two(Tk::NotEq, "!="); else one(Tk::Other); return;
      case '<': if (n == '=') two(Tk::LtEq, "<="); else one(Tk::Lt); return;
      case '>': if (n == '=') two(Tk::GtEq, ">="); else one(Tk::Gt); return;
      default: one(Tk::Other); return;
    }
  }

  const std::string& s_;
  size_t pos_ = 0;
  int line_ = 1;
  int depth_ = 0;
  bool at_line_start_ = true;
  std::vector<int> indents_;
  std::vector<Token> out_;
};

// ---- AST ---------------------------------------------------------------------
enum class Op { Add, Sub, Mul, Div, Matmul, Pow, Eq, NotEq, Lt, LtEq, Gt, GtEq, And, Or };

struct Expr;
using EP = std::unique_ptr<Expr>;
struct Expr {
  enum K { Ident, Int, Float, Bool, Str, Bin, Neg, Not, Call, Index, Field, Unsupported } k;
  int line = 0;
  std::string name;    // Ident / Call callee / Field name
  long long ival = 0;
  double fval = 0;
  bool bval = false;
  Op op = Op::Add;
  EP lhs, rhs;         // Bin; Neg/Not/Field/Index base in lhs
  std::vector<EP> args;  // Call args / Index indices
  Ty ty;               // filled by the checker
};

struct Stmt {
  enum K { Let, LetMut, LetShared, Assign, ExprS, Return, If, For, While, Break, Continue, Unsupported } k;
  int line = 0;
  std::string name;
  EP a, b;             // Let: a; Assign: a = target, b = value; Return/ExprS: a; If/While: a; For: a..b
  std::vector<Stmt> body, else_body;
  bool has_else = false;
  Sc elem = Sc::F32;   // LetShared
  long long size = 0;
};

struct Param {
  std::string name;
  Ty ty;
  bool inout = false;
};

struct Kernel {
  std::string name;
  std::vector<Param> params;
  Ty ret;
  std::vector<Stmt> body;
  bool implicit = false;
  int line = 0;
};

// ---- parser (parser.rs) --------------------------------------------------------
class Parser {
 public:
  explicit Parser(std::vector<Token> t) : t_(std::move(t)) {}

  std::vector<Kernel> kernels() {
    std::vector<Kernel> ks;
    while (cur().k != Tk::Eof) {
      if (cur().k == Tk::Newline || cur().k == Tk::Indent || cur().k == Tk::Dedent) { ++p_; continue; }
      if (cur().k == Tk::KwKernel) ks.push_back(kernel());
      else skip_item();
    }
    return ks;
  }

 private:
  const Token& cur() const { return t_[p_]; }
  const Token& at(size_t k) const { return t_[std::min(p_ + k, t_.size() - 1)]; }
  [[noreturn]] void err(const char* what) {
    fail("malus: emit: line %d: %s (at '%s')", cur().line, what, cur().text.c_str());
  }
  void expect(Tk k, const char* what) {
    if (cur().k != k) err(what);
    ++p_;
  }
  std::string ident(const char* what) {
    if (cur().k != Tk::Ident) err(what);
    return t_[p_++].text;
  }
  // A non-kernel top-level item: skip to the next line at indentation 0.
  void skip_item() {
    int depth = 0;
    while (cur().k != Tk::Eof) {
      Tk k = cur().k;
      ++p_;
      if (k == Tk::Indent) ++depth;
      else if (k == Tk::Dedent) --depth;
      else if (k == Tk::Newline && depth == 0 && cur().k != Tk::Indent) return;
      if (depth == 0 && k == Tk::Dedent) return;
    }
  }

  Ty type() {
    std::string n = ident("expected a type");
    Sc s;
    if (sc_from_name(n, &s)) return Ty::scalar(s);
    if (n == "Tensor" || n == "Array") {
      expect(Tk::Lt, "expected '<'");
      std::string e = ident("expected an element type");
      if (!sc_from_name(e, &s)) err("element type must be a scalar type");
      Ty t = n == "Tensor" ? Ty::tensor(s) : Ty::scalar(s);
      if (n == "Array") {
        expect(Tk::Comma, "expected ', N' in Array<T, N>");
        if (cur().k != Tk::Int) err("expected the array length");
        t.k = Ty::Array;
        t.len = t_[p_++].ival;
      }
      expect(Tk::Gt, "expected '>'");
      return t;
    }
    if (n == "bool") return Ty::boolean();
    // other types (List<...>, structs) are not valid in kernel signatures
    if (cur().k == Tk::Lt) {
      int d = 0;
      do {
        if (cur().k == Tk::Lt) ++d;
        if (cur().k == Tk::Gt) --d;
        ++p_;
      } while (d > 0 && cur().k != Tk::Eof);
    }
    return Ty();
  }

  Kernel kernel() {
    Kernel k;
    k.line = cur().line;
    expect(Tk::KwKernel, "expected 'kernel'");
    k.name = ident("expected the kernel name");
    expect(Tk::LParen, "expected '('");
    while (cur().k != Tk::RParen && cur().k != Tk::Eof) {
      Param p;
      if (cur().k == Tk::KwInout) { p.inout = true; ++p_; }
      p.name = ident("expected a parameter name");
      expect(Tk::Colon, "expected ':' after the parameter name");
      p.ty = type();
      k.params.push_back(p);
      if (cur().k == Tk::Comma) ++p_;
      else break;
    }
    expect(Tk::RParen, "expected ')'");
    expect(Tk::Arrow, "expected '->'");
    k.ret = type();
    expect(Tk::Colon, "expected ':'");
    k.body = block();
    return k;
  }

  std::vector<Stmt> block() {
    expect(Tk::Newline, "expected a newline");
    expect(Tk::Indent, "expected an indented block");
    std::vector<Stmt> out;
    while (true) {
      while (cur().k == Tk::Newline) ++p_;
      if (cur().k == Tk::Dedent || cur().k == Tk::Eof) break;
      out.push_back(stmt());
    }
    if (cur().k == Tk::Dedent) ++p_;
    if (out.empty()) err("empty block");
    return out;
  }

  void end_of_stmt() {
    if (cur().k == Tk::Newline) { ++p_; return; }
    if (cur().k == Tk::Eof || cur().k == Tk::Dedent) return;
    err("expected a newline");
  }

  Stmt stmt() {
    Stmt s;
    s.line = cur().line;
    switch (cur().k) {
      case Tk::KwLet: {
        ++p_;
        if (cur().k == Tk::Ident && cur().text == "shared") {
          ++p_;
          s.k = Stmt::LetShared;
          s.name = ident("expected the shared array name");
          expect(Tk::Colon, "expected ':'");
          Ty t = type();
          if (t.k != Ty::Array) err("expected `Array<T, N>` after `let shared name:`");
          s.elem = t.s;
          s.size = t.len;
          end_of_stmt();
          return s;
        }
        s.k = Stmt::Let;
        if (cur().k == Tk::KwMut) { s.k = Stmt::LetMut; ++p_; }
        if (cur().k == Tk::LParen) err("tuple destructuring is not valid in a kernel body");
        s.name = ident("expected a binding name");
        expect(Tk::Assign, "expected '='");
        s.a = expr();
        end_of_stmt();
        return s;
      }
      case Tk::KwReturn:
        ++p_;
        s.k = Stmt::Return;
        if (cur().k != Tk::Newline && cur().k != Tk::Dedent && cur().k != Tk::Eof) s.a = expr();
        end_of_stmt();
        return s;
      case Tk::KwBreak: ++p_; s.k = Stmt::Break; end_of_stmt(); return s;
      case Tk::KwContinue: ++p_; s.k = Stmt::Continue; end_of_stmt(); return s;
      case Tk::KwIf:
        ++p_;
        s.k = Stmt::If;
        s.a = expr();
        expect(Tk::Colon, "expected ':'");
        s.body = block();
        if (cur().k == Tk::KwElse) {
          ++p_;
          expect(Tk::Colon, "expected ':' after else");
          s.has_else = true;
          s.else_body = block();
        }
        return s;
      case Tk::KwWhile:
        ++p_;
        s.k = Stmt::While;
        s.a = expr();
        expect(Tk::Colon, "expected ':'");
        s.body = block();
        return s;
      case Tk::KwFor: {
        ++p_;
        s.k = Stmt::For;
        s.name = ident("expected the loop variable");
        expect(Tk::KwIn, "expected 'in'");
        if (!(cur().k == Tk::Ident && cur().text == "range")) err("kernel loops iterate over range(...)");
        ++p_;
        expect(Tk::LParen, "expected '('");
        EP first = expr();
        if (cur().k == Tk::Comma) {
          ++p_;
          s.a = std::move(first);
          s.b = expr();
        } else {
          s.a.reset(new Expr{Expr::Int});
          s.a->line = s.line;
          s.b = std::move(first);
        }
        expect(Tk::RParen, "expected ')'");
        expect(Tk::Colon, "expected ':'");
        s.body = block();
        return s;
      }
      case Tk::KwItem:
        err("statement not valid in a kernel body");
      default: {
        EP e = expr();
        if (cur().k == Tk::Assign && (e->k == Expr::Ident || e->k == Expr::Index || e->k == Expr::Field)) {
          ++p_;
          s.k = Stmt::Assign;
          s.a = std::move(e);
          s.b = expr();
        } else {
          s.k = Stmt::ExprS;
          s.a = std::move(e);
        }
        end_of_stmt();
        return s;
      }
    }
  }

  // Pratt binding powers (parser.rs:609-624)
  static bool infix(Tk k, int* l, int* r, Op* op) {
    switch (k) {
      case Tk::KwOr: *l = 1; *r = 2; *op = Op::Or; return true;
      case Tk::KwAnd: *l = 3; *r = 4; *op = Op::And; return true;
      case Tk::EqEq: *l = 5; *r = 6; *op = Op::Eq; return true;
      case Tk::NotEq: *l = 5; *r = 6; *op = Op::NotEq; return true;
      case Tk::Lt: *l = 5; *r = 6; *op = Op::Lt; return true;
      case Tk::LtEq: *l = 5; *r = 6; *op = Op::LtEq; return true;
      case Tk::Gt: *l = 5; *r = 6; *op = Op::Gt; return true;
      case Tk::GtEq: *l = 5; *r = 6; *op = Op::GtEq; return true;
      case Tk::Plus: *l = 7; *r = 8; *op = Op::Add; return true;
      case Tk::Minus: *l = 7; *r = 8; *op = Op::Sub; return true;
      case Tk::Star: *l = 9; *r = 10; *op = Op::Mul; return true;
      case Tk::Slash: *l = 9; *r = 10; *op = Op::Div; return true;
      case Tk::At: *l = 9; *r = 10; *op = Op::Matmul; return true;
      case Tk::StarStar: *l = 12; *r = 11; *op = Op::Pow; return true;
      default: return false;
    }
  }

  EP expr(int min_bp = 0) {
    EP lhs = unary();
    while (true) {
      int l, r;
      Op op;
      if (!infix(cur().k, &l, &r, &op) || l < min_bp) break;
      int line = cur().line;
      ++p_;
      EP rhs = expr(r);
      EP e(new Expr{Expr::Bin});
      e->line = line;
      e->op = op;
      e->lhs = std::move(lhs);
      e->rhs = std::move(rhs);
      lhs = std::move(e);
    }
    return lhs;
  }

  EP unary() {
    if (cur().k == Tk::Minus || cur().k == Tk::KwNot) {
      EP e(new Expr{cur().k == Tk::Minus ? Expr::Neg : Expr::Not});
      e->line = cur().line;
      ++p_;
      e->lhs = unary();
      return e;
    }
    return postfix();
  }

  EP postfix() {
    EP base = primary();
    while (true) {
      if (cur().k == Tk::LParen) {
        ++p_;
        EP e(new Expr{Expr::Call});
        e->line = base->line;
        if (base->k != Expr::Ident) err("only named functions can be called in a kernel body");
        e->name = base->name;
        while (cur().k != Tk::RParen && cur().k != Tk::Eof) {
          if (cur().k == Tk::Ident && at(1).k == Tk::Assign) err("named arguments are not valid in a kernel body");
          e->args.push_back(expr());
          if (cur().k == Tk::Comma) ++p_;
          else break;
        }
        expect(Tk::RParen, "expected ')'");
        base = std::move(e);
      } else if (cur().k == Tk::LBracket) {
        if (base->k == Expr::Ident && at(1).k == Tk::Ident && at(2).k == Tk::Assign)
          err("kernel launches are not valid in a kernel body");
        ++p_;
        EP e(new Expr{Expr::Index});
        e->line = base->line;
        e->lhs = std::move(base);
        while (cur().k != Tk::RBracket && cur().k != Tk::Eof) {
          e->args.push_back(expr());
          if (cur().k == Tk::Comma) ++p_;
          else break;
        }
        expect(Tk::RBracket, "expected ']'");
        base = std::move(e);
      } else if (cur().k == Tk::Dot) {
        ++p_;
        EP e(new Expr{Expr::Field});
        e->line = base->line;
        e->name = ident("expected a field name");
        e->lhs = std::move(base);
        base = std::move(e);
      } else {
        break;
      }
    }
    return base;
  }

  EP primary() {
    const Token& t = cur();
    EP e;
    switch (t.k) {
      case Tk::Ident: e.reset(new Expr{Expr::Ident}); e->name = t.text; break;
      case Tk::Int: e.reset(new Expr{Expr::Int}); e->ival = t.ival; break;
      case Tk::Float: e.reset(new Expr{Expr::Float}); e->fval = t.fval; break;
      case Tk::KwTrue: case Tk::KwFalse: e.reset(new Expr{Expr::Bool}); e->bval = t.k == Tk::KwTrue; break;
      case Tk::Str: e.reset(new Expr{Expr::Str}); e->name = t.text; break;
      case Tk::LParen: {
        ++p_;
        EP inner = expr();
        expect(Tk::RParen, "expected ')'");
        return inner;
      }
      default: err("expected an expression");
    }
    e->line = t.line;
    ++p_;
    return e;
  }

  std::vector<Token> t_;
  size_t p_ = 0;
};

// ---- type checker (check.rs, kernel-body rules) --------------------------------
struct Binding {
  Ty ty;
  bool mut_ = false;
  bool tensor_param = false;
};

class Checker {
 public:
  explicit Checker(Kernel& k) : k_(k) {}

  void run() {
    for (auto& p : k_.params)
      if (p.ty.k == Ty::None || p.ty.k == Ty::Array || p.ty.k == Ty::Bool)
        fail("malus: emit: kernel %s: parameter %s must be a tensor or a scalar, got %s", k_.name.c_str(),
             p.name.c_str(), p.ty.str().c_str());
    if (k_.ret.k != Ty::Tensor)
      fail("malus: emit: kernel must return a tensor, got: %s (kernel %s)", k_.ret.str().c_str(), k_.name.c_str());
    k_.implicit = is_implicit(k_.body);
    scopes_.emplace_back();
    for (auto& p : k_.params) {
      Binding b;
      if (k_.implicit) {
        // element-space rebinding: tensor params are seen as their element type
        if (p.ty.k != Ty::Tensor)
          fail("malus: emit: kernel param must be a tensor, got: %s (kernel %s)", p.ty.str().c_str(), k_.name.c_str());
        b.ty = Ty::scalar(p.ty.s);
      } else {
        b.ty = p.ty;
        b.tensor_param = p.ty.k == Ty::Tensor;
        b.mut_ = p.inout;
      }
      scopes_.back()[p.name] = b;
    }
    if (!k_.implicit) {
      Binding o;
      o.ty = k_.ret;
      o.mut_ = true;
      o.tensor_param = true;
      scopes_.back()["out"] = o;
    }
    ret_ = k_.implicit ? Ty::scalar(k_.ret.s) : Ty::unit();
    body(k_.body, 0);
  }

  // check.rs:574-588
  static bool is_implicit(const std::vector<Stmt>& b) {
    if (b.empty()) return false;
    for (auto& s : b)
      if (s.k != Stmt::Let && s.k != Stmt::LetMut && s.k != Stmt::Return) return false;
    return b.back().k == Stmt::Return;
  }

 private:
  [[noreturn]] void err(int line, const char* fmt, ...) __attribute__((format(printf, 3, 4))) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    fail("malus: emit: kernel %s, line %d: %s", k_.name.c_str(), line, buf);
  }

  const Binding* lookup(const std::string& n) const {
    for (auto it = scopes_.rbegin(); it != scopes_.rend(); ++it) {
      auto f = it->find(n);
      if (f != it->end()) return &f->second;
    }
    return nullptr;
  }

  void body(std::vector<Stmt>& stmts, int loop_depth) {
    for (auto& s : stmts) stmt(s, loop_depth);
  }

  void stmt(Stmt& s, int loop_depth) {
    switch (s.k) {
      case Stmt::Let:
      case Stmt::LetMut: {
        Ty t = expr(*s.a, nullptr);
        if (t.k != Ty::Scalar) err(s.line, "expected scalar type for kernel local, got: %s", t.str().c_str());
        Binding b;
        b.ty = t;
        b.mut_ = s.k == Stmt::LetMut;
        scopes_.back()[s.name] = b;
        return;
      }
      case Stmt::LetShared: {
        Binding b;
        b.ty.k = Ty::Array;
        b.ty.s = s.elem;
        b.ty.len = s.size;
        b.mut_ = true;
        if (s.size <= 0) err(s.line, "shared array %s needs a positive length", s.name.c_str());
        scopes_.back()[s.name] = b;
        return;
      }
      case Stmt::Assign: assign(s); return;
      case Stmt::ExprS: expr(*s.a, nullptr); return;
      case Stmt::Return:
        if (k_.implicit) {
          if (!s.a) err(s.line, "return needs a value in an implicit-map kernel");
          Ty t = expr(*s.a, &ret_);
          if (t != ret_) err(s.line, "return type mismatch: expected %s, found %s", ret_.str().c_str(), t.str().c_str());
        } else if (s.a) {
          Ty t = expr(*s.a, &ret_);
          if (t != ret_) err(s.line, "return type mismatch: expected (), found %s (explicit kernels write to out)",
                             t.str().c_str());
        }
        return;
      case Stmt::If: {
        Ty b = Ty::boolean();
        expr(*s.a, &b);
        scopes_.emplace_back();
        body(s.body, loop_depth);
        scopes_.pop_back();
        if (s.has_else) {
          scopes_.emplace_back();
          body(s.else_body, loop_depth);
          scopes_.pop_back();
        }
        return;
      }
      case Stmt::For: {
        Ty i32 = Ty::scalar(Sc::I32);
        Ty a = expr(*s.a, &i32), b = expr(*s.b, &i32);
        if (!a.is_int() || !b.is_int()) err(s.line, "range bounds must be integers");
        scopes_.emplace_back();
        Binding v;
        v.ty = i32;
        scopes_.back()[s.name] = v;
        body(s.body, loop_depth + 1);
        scopes_.pop_back();
        return;
      }
      case Stmt::While: {
        Ty b = Ty::boolean();
        expr(*s.a, &b);
        scopes_.emplace_back();
        body(s.body, loop_depth + 1);
        scopes_.pop_back();
        return;
      }
      case Stmt::Break:
      case Stmt::Continue:
        if (loop_depth == 0) err(s.line, "%s outside a loop", s.k == Stmt::Break ? "break" : "continue");
        return;
      default: err(s.line, "statement not valid in a kernel body");
    }
  }

  void assign(Stmt& s) {
    Expr& tgt = *s.a;
    if (tgt.k == Expr::Ident) {
      const Binding* b = lookup(tgt.name);
      if (!b) err(s.line, "unknown identifier in kernel: %s", tgt.name.c_str());
      if (!b->mut_ || b->ty.k != Ty::Scalar) err(s.line, "cannot assign to immutable binding %s", tgt.name.c_str());
      tgt.ty = b->ty;
      Ty t = expr(*s.b, &b->ty);
      if (t != b->ty) err(s.line, "type mismatch: expected %s, found %s", b->ty.str().c_str(), t.str().c_str());
      return;
    }
    if (tgt.k == Expr::Index) {
      if (tgt.lhs->k != Expr::Ident) err(s.line, "unsupported lvalue target in kernel");
      const Binding* b = lookup(tgt.lhs->name);
      if (!b) err(s.line, "unknown identifier in kernel: %s", tgt.lhs->name.c_str());
      if (!b->mut_) err(s.line, "cannot assign to immutable binding %s", tgt.lhs->name.c_str());
      if (b->ty.k != Ty::Tensor && b->ty.k != Ty::Array) err(s.line, "%s is not indexable", tgt.lhs->name.c_str());
      if (tgt.args.size() != 1) err(s.line, "unsupported lvalue target in kernel: assignments take one flat index");
      tgt.lhs->ty = b->ty;
      Ty i64 = Ty::scalar(Sc::I64);
      Ty it = expr(*tgt.args[0], &i64);
      if (!it.is_int()) err(s.line, "index must be an integer, got %s", it.str().c_str());
      Ty elem = Ty::scalar(b->ty.s);
      tgt.ty = elem;
      Ty t = expr(*s.b, &elem);
      if (t != elem) err(s.line, "type mismatch: expected %s, found %s", elem.str().c_str(), t.str().c_str());
      return;
    }
    err(s.line, "unsupported lvalue target in kernel");
  }

  static bool is_intrinsic(const std::string& n) {
    return n == "thread_id" || n == "threadgroup_id" || n == "thread_in_threadgroup" ||
           n == "threads_per_threadgroup" || n == "threads_per_grid";
  }

  Ty expr(Expr& e, const Ty* expected) {
    e.ty = expr_ty(e, expected);
    return e.ty;
  }

  Ty expr_ty(Expr& e, const Ty* expected) {
    switch (e.k) {
      case Expr::Int:  // check.rs:948-958
        if (expected && expected->k == Ty::Scalar && sc_is_float(expected->s)) return *expected;
        return Ty::scalar(Sc::I32);
      case Expr::Float: return Ty::scalar(Sc::F32);
      case Expr::Bool: return Ty::boolean();
      case Expr::Str: err(e.line, "string literals not supported in kernel bodies");
      case Expr::Ident: {
        const Binding* b = lookup(e.name);
        if (!b) err(e.line, "unknown identifier in kernel: %s", e.name.c_str());
        return b->ty;
      }
      case Expr::Neg:
      case Expr::Not: {
        Ty t = expr(*e.lhs, expected);
        if (e.k == Expr::Not && k_.implicit) err(e.line, "logical not not supported in kernel bodies");
        if (t.k != Ty::Scalar && t.k != Ty::Bool) err(e.line, "unary operand must be a scalar, got %s", t.str().c_str());
        return t;
      }
      case Expr::Bin: return binop(e);
      case Expr::Call: return call(e);
      case Expr::Index: return index(e);
      case Expr::Field: {
        if (e.lhs->k != Expr::Ident)
          err(e.line, "shape/stride/ndim access requires a simple tensor parameter name");
        Ty bt = expr(*e.lhs, nullptr);
        if (bt.k != Ty::Tensor) err(e.line, "field '%s' on a non-tensor", e.name.c_str());
        if (e.name == "ndim") return Ty::scalar(Sc::I32);
        if (e.name == "shape" || e.name == "strides")
          err(e.line, "field '%s' on tensor must be indexed (e.g. t.shape[i])", e.name.c_str());
        err(e.line, "unsupported tensor field '%s' in a kernel body", e.name.c_str());
      }
      default: err(e.line, "unsupported expression in a kernel body");
    }
  }

  Ty binop(Expr& e) {
    if (e.op == Op::Pow) {  // check.rs:993-1011
      Ty f32 = Ty::scalar(Sc::F32);
      Ty l = expr(*e.lhs, &f32), r = expr(*e.rhs, nullptr);
      bool rok = r.k == Ty::Scalar && (r.s == Sc::F32 || r.s == Sc::I32 || r.s == Sc::I64);
      if (l != f32 || !rok) err(e.line, "** takes an f32 base and an f32/i32/i64 exponent");
      return f32;
    }
    Ty l = expr(*e.lhs, nullptr), r = expr(*e.rhs, nullptr);
    if (l.k == Ty::Tensor || r.k == Ty::Tensor)
      err(e.line, "tensor operands are not element-wise inside a kernel body (index them)");
    if (e.op == Op::Matmul) err(e.line, "matmul is not element-wise");
    if (l != r) err(e.line, "type mismatch: %s vs %s", l.str().c_str(), r.str().c_str());
    switch (e.op) {
      case Op::Eq: case Op::NotEq: case Op::Lt: case Op::LtEq: case Op::Gt: case Op::GtEq:
        return l;  // element space: the comparison is a mask of the operand dtype
      case Op::And: case Op::Or:
        return Ty::boolean();
      default:
        return l;
    }
  }

  Ty call(Expr& e) {
    const std::string& n = e.name;
    auto nargs = [&](size_t want) {
      if (e.args.size() != want) err(e.line, "%s takes %zu argument(s), got %zu", n.c_str(), want, e.args.size());
    };
    Ty f32 = Ty::scalar(Sc::F32);
    if (is_intrinsic(n)) {
      if (k_.implicit) err(e.line, "thread intrinsics are not valid in implicit-map kernels");
      nargs(0);
      return Ty::scalar(Sc::I32);
    }
    if (n == "barrier") {
      nargs(0);
      return Ty::unit();
    }
    if (k_.implicit) err(e.line, "unsupported expression kind in implicit-map kernel body (call to %s)", n.c_str());
    static const std::set<std::string> unary = {"exp", "log", "sqrt", "rsqrt", "tanh", "abs", "relu", "sigmoid"};
    static const std::set<std::string> binary = {"fmax", "fmin", "pow"};
    if (unary.count(n) || binary.count(n)) {
      nargs(unary.count(n) ? 1 : 2);
      for (auto& a : e.args) {
        Ty t = expr(*a, &f32);
        if (t != f32) err(e.line, "%s takes f32 arguments, got %s", n.c_str(), t.str().c_str());
      }
      return f32;
    }
    err(e.line, "unsupported call in explicit kernel body: %s", n.c_str());
  }

  Ty index(Expr& e) {
    Expr& base = *e.lhs;
    if (base.k == Expr::Field && (base.name == "shape" || base.name == "strides")) {
      if (e.args.size() != 1) err(e.line, "shape/strides index must be single-dimensional");
      if (base.lhs->k != Expr::Ident) err(e.line, "shape/stride/ndim access requires a simple tensor parameter name");
      Ty bt = expr(*base.lhs, nullptr);
      if (bt.k != Ty::Tensor) err(e.line, "%s.%s on a non-tensor", base.lhs->name.c_str(), base.name.c_str());
      Ty i32 = Ty::scalar(Sc::I32);
      Ty it = expr(*e.args[0], &i32);
      if (!it.is_int()) err(e.line, "index must be an integer, got %s", it.str().c_str());
      base.ty = Ty::scalar(Sc::I32);
      return Ty::scalar(Sc::I32);
    }
    Ty bt = expr(base, nullptr);
    if (bt.k != Ty::Tensor && bt.k != Ty::Array) err(e.line, "indexing a non-indexable value (%s)", bt.str().c_str());
    if (e.args.empty()) err(e.line, "empty index");
    if (e.args.size() > 1 && (bt.k != Ty::Tensor || base.k != Expr::Ident))
      err(e.line, "multi-dimensional indexing needs a tensor parameter");
    for (auto& a : e.args) {
      Ty i64 = Ty::scalar(Sc::I64);
      Ty it = expr(*a, &i64);
      if (!it.is_int()) err(e.line, "index must be an integer, got %s", it.str().c_str());
    }
    return Ty::scalar(bt.s);
  }

  Kernel& k_;
  Ty ret_;
  std::vector<std::map<std::string, Binding>> scopes_;
};

// ---- HIP lowering --------------------------------------------------------------

// Float literal: the shortest decimal that reads back as the same double (the
// digits of Rust's `{:?}`, codegen-gpu/lib.rs:1010-1019), as an f32 literal.
std::string float_lit(double v) {
  char buf[64];
  for (int prec = 1; prec <= 17; ++prec) {
    snprintf(buf, sizeof buf, "%.*g", prec, v);
    if (strtod(buf, nullptr) == v) break;
  }
  std::string s = buf;
  if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
  return s + "f";
}

const char* op_infix(Op op) {
  switch (op) {
    case Op::Add: return "+";
    case Op::Sub: return "-";
    case Op::Mul: return "*";
    case Op::Div: return "/";
    case Op::Eq: return "==";
    case Op::NotEq: return "!=";
    case Op::Lt: return "<";
    case Op::LtEq: return "<=";
    case Op::Gt: return ">";
    case Op::GtEq: return ">=";
    case Op::And: return "&&";
    case Op::Or: return "||";
    default: return nullptr;
  }
}

// Device helpers for the math builtins: evaluated in double and rounded once.
// Only the helpers a kernel's body calls are emitted (prelude_for).
const char* kHelpers[][2] = {
    {"__malus_exp(", "__device__ static inline float __malus_exp(float x) { return (float)exp((double)x); }\n"},
    {"__malus_log(", "__device__ static inline float __malus_log(float x) { return (float)log((double)x); }\n"},
    {"__malus_tanh(", "__device__ static inline float __malus_tanh(float x) { return (float)tanh((double)x); }\n"},
    {"__malus_rsqrt(",
     "__device__ static inline float __malus_rsqrt(float x) { return (float)(1.0 / sqrt((double)x)); }\n"},
    {"__malus_pow(",
     "__device__ static inline float __malus_pow(float x, float y) { return (float)pow((double)x, (double)y); }\n"},
    {"__malus_sigmoid(",
     "__device__ static inline float __malus_sigmoid(float x) { return 1.0f / (1.0f + (float)exp(-(double)x)); }\n"},
};

std::string prelude_for(const std::string& body) {
  std::string out;
  for (auto& h : kHelpers)
    if (body.find(h[0]) != std::string::npos) out += h[1];
  return out;
}

const char* kTensorMeta = "struct TensorMeta {\n    unsigned int ndim;\n    unsigned int shape[8];\n    unsigned int strides[8];\n};\n";

class Lower {
 public:
  Lower(const Kernel& k, uint64_t id) : k_(k), id_(id) {}

  std::string run(std::string* notes) {
    return k_.implicit ? implicit(notes) : explicit_(notes);
  }

 private:
  [[noreturn]] void err(int line, const char* what) {
    fail("malus: emit: kernel %s, line %d: %s", k_.name.c_str(), line, what);
  }

  // codegen-gpu/lib.rs:432-562
  std::string implicit(std::string* notes) {
    std::ostringstream o;
    o << "extern \"C\" __global__ void malus_kernel_" << id_ << "(";
    for (auto& p : k_.params) o << "const " << sc_hip(p.ty.s) << "* __restrict__ " << p.name << ", ";
    o << sc_hip(k_.ret.s) << "* __restrict__ out, unsigned int n) {\n";
    o << "    const unsigned int tid = blockIdx.x * blockDim.x + threadIdx.x;\n";
    o << "    if (tid >= n) return;\n";
    for (auto& p : k_.params) params_.insert(p.name);
    for (size_t i = 0; i < k_.body.size(); ++i) {
      const Stmt& s = k_.body[i];
      if (s.k == Stmt::Return) {
        o << "    out[tid] = " << iexpr(*s.a) << ";\n";
      } else {
        o << "    " << sc_hip(s.a->ty.s) << " " << s.name << " = " << iexpr(*s.a) << ";\n";
        locals_.insert(s.name);
      }
    }
    o << "}\n";
    *notes = "//@malus-v1-elem-bytes " + std::to_string(sc_bytes(k_.ret.s));
    for (auto& p : k_.params) *notes += " " + std::to_string(sc_bytes(p.ty.s));
    *notes += "\n";
    return "// malus kernel " + k_.name + " (implicit map, v1 ABI)\n" + prelude_for(o.str()) + o.str();
  }

  std::string iexpr(const Expr& e) {
    switch (e.k) {
      case Expr::Ident:
        if (params_.count(e.name)) return e.name + "[tid]";
        if (locals_.count(e.name)) return e.name;
        err(e.line, "unknown identifier in kernel");
      case Expr::Int: return std::to_string(e.ival);
      case Expr::Float: return float_lit(e.fval);
      case Expr::Bool: return e.bval ? "true" : "false";
      case Expr::Bin: {
        const char* op = op_infix(e.op);
        if (!op) err(e.line, e.op == Op::Pow ? "** is not supported in implicit-map kernel bodies" : "matmul is not element-wise");
        return "(" + iexpr(*e.lhs) + " " + op + " " + iexpr(*e.rhs) + ")";
      }
      case Expr::Neg: return "(-" + iexpr(*e.lhs) + ")";
      default: err(e.line, "unsupported expression kind in implicit-map kernel body");
    }
  }

  // codegen-gpu/lib.rs:564-1006
  std::string explicit_(std::string* notes) {
    std::vector<const Param*> tensors, scalars;
    for (auto& p : k_.params) (p.ty.k == Ty::Tensor ? tensors : scalars).push_back(&p);
    for (auto* p : tensors) tensor_names_.insert(p->name);
    tensor_names_.insert("out");
    for (auto* p : scalars) scalar_names_.insert(p->name);
    collect_intrinsics(k_.body);

    std::ostringstream o;
    if (!scalars.empty()) {
      // one 4-byte slot per scalar in parameter order, as kernel_dispatch_v2's
      // uniforms blob is packed (integers as their low 32 bits)
      o << "struct Uniforms_" << id_ << " {\n";
      for (auto* p : scalars) {
        if (p->ty.s == Sc::F32) o << "    float " << p->name << ";\n";
        else if (p->ty.s == Sc::F16) o << "    _Float16 " << p->name << ";\n    unsigned short _pad_" << p->name << ";\n";
        else if (p->ty.s == Sc::BF16) o << "    __bf16 " << p->name << ";\n    unsigned short _pad_" << p->name << ";\n";
        else if (p->ty.s == Sc::U32 || p->ty.s == Sc::U64) o << "    unsigned int " << p->name << ";\n";
        else o << "    int " << p->name << ";\n";
      }
      o << "};\n";
    }
    std::string decls = o.str();
    o.str("");
    o << "extern \"C\" __global__ void malus_kernel_" << id_ << "(\n";
    std::vector<std::string> ps;
    for (auto* p : tensors)
      ps.push_back(std::string(p->inout ? "" : "const ") + sc_hip(p->ty.s) + "* __restrict__ " + p->name);
    ps.push_back(std::string(sc_hip(k_.ret.s)) + "* __restrict__ out");
    if (!scalars.empty()) ps.push_back("Uniforms_" + std::to_string(id_) + " u");
    for (auto* p : tensors) ps.push_back("TensorMeta " + p->name + "_meta");
    ps.push_back("TensorMeta out_meta");
    for (size_t i = 0; i < ps.size(); ++i) o << "    " << ps[i] << (i + 1 < ps.size() ? ",\n" : ") {\n");
    // thread-hierarchy intrinsics, only those the body uses (1-D launch)
    if (used_.count("thread_id")) o << "    const int _tid = (int)(blockIdx.x * blockDim.x + threadIdx.x);\n";
    if (used_.count("threadgroup_id")) o << "    const int _tgid = (int)blockIdx.x;\n";
    if (used_.count("thread_in_threadgroup")) o << "    const int _lid = (int)threadIdx.x;\n";
    if (used_.count("threads_per_threadgroup")) o << "    const int _tgsize = (int)blockDim.x;\n";
    if (used_.count("threads_per_grid")) o << "    const int _gridsize = (int)(gridDim.x * blockDim.x);\n";
    block(k_.body, 1, o);
    o << "}\n";
    size_t ubytes = 0;
    for (auto* p : scalars) { (void)p; ubytes += 4; }
    *notes = "//@malus-v2-uniform-bytes " + std::to_string(ubytes) + "\n";
    return "// malus kernel " + k_.name + " (explicit form, v2 ABI)\n" + kTensorMeta + decls + prelude_for(o.str()) +
           o.str();
  }

  void collect_intrinsics(const std::vector<Stmt>& b) {
    for (auto& s : b) {
      if (s.a) collect_intrinsics(*s.a);
      if (s.b) collect_intrinsics(*s.b);
      collect_intrinsics(s.body);
      collect_intrinsics(s.else_body);
    }
  }
  void collect_intrinsics(const Expr& e) {
    if (e.k == Expr::Call) used_.insert(e.name);
    if (e.lhs) collect_intrinsics(*e.lhs);
    if (e.rhs) collect_intrinsics(*e.rhs);
    for (auto& a : e.args) collect_intrinsics(*a);
  }

  void block(const std::vector<Stmt>& b, int depth, std::ostringstream& o) {
    std::string ind(4 * depth, ' ');
    for (auto& s : b) {
      switch (s.k) {
        case Stmt::Let:
        case Stmt::LetMut:
          o << ind << sc_hip(s.a->ty.s) << " " << s.name << " = " << x(*s.a) << ";\n";
          break;
        case Stmt::LetShared:
          o << ind << "__shared__ " << sc_hip(s.elem) << " " << s.name << "[" << s.size << "];\n";
          break;
        case Stmt::Assign:
          if (s.a->k == Expr::Ident) o << ind << s.a->name << " = " << x(*s.b) << ";\n";
          else o << ind << s.a->lhs->name << "[" << x(*s.a->args[0]) << "] = " << x(*s.b) << ";\n";
          break;
        case Stmt::ExprS:
          if (s.a->k == Expr::Call && s.a->name == "barrier") o << ind << "__syncthreads();\n";
          else o << ind << x(*s.a) << ";\n";
          break;
        case Stmt::If:
          o << ind << "if (" << x(*s.a) << ") {\n";
          block(s.body, depth + 1, o);
          if (s.has_else) {
            o << ind << "} else {\n";
            block(s.else_body, depth + 1, o);
          }
          o << ind << "}\n";
          break;
        case Stmt::For:
          o << ind << "for (" << sc_hip(s.a->ty.s) << " " << s.name << " = " << x(*s.a) << "; " << s.name << " < "
            << x(*s.b) << "; " << s.name << "++) {\n";
          block(s.body, depth + 1, o);
          o << ind << "}\n";
          break;
        case Stmt::While:
          o << ind << "while (" << x(*s.a) << ") {\n";
          block(s.body, depth + 1, o);
          o << ind << "}\n";
          break;
        case Stmt::Return:
          o << ind << "return;\n";  // an early exit: explicit kernels write to out
          break;
        case Stmt::Break:
        case Stmt::Continue:
          // lower_kernel_body_explicit (lib.rs:851-858) rejects these
          err(s.line, "statement not valid in explicit kernel body: break/continue");
        default: err(s.line, "statement not valid in explicit kernel body");
      }
    }
  }

  std::string x(const Expr& e) {
    switch (e.k) {
      case Expr::Ident:
        if (scalar_names_.count(e.name)) return "u." + e.name;
        return e.name;
      case Expr::Int: return std::to_string(e.ival);
      case Expr::Float: return float_lit(e.fval);
      case Expr::Bool: return e.bval ? "true" : "false";
      case Expr::Bin: {
        if (e.op == Op::Pow) return "__malus_pow(" + x(*e.lhs) + ", " + x(*e.rhs) + ")";
        const char* op = op_infix(e.op);
        if (!op) err(e.line, "matmul is not element-wise");
        return "(" + x(*e.lhs) + " " + op + " " + x(*e.rhs) + ")";
      }
      case Expr::Neg: return "(-" + x(*e.lhs) + ")";
      case Expr::Not: return "(!" + x(*e.lhs) + ")";
      case Expr::Field:
        return "(int)" + e.lhs->name + "_meta.ndim";
      case Expr::Index: {
        const Expr& b = *e.lhs;
        if (b.k == Expr::Field)
          return "(int)" + b.lhs->name + "_meta." + b.name + "[" + x(*e.args[0]) + "]";
        if (e.args.size() > 1) {
          std::string flat;
          for (size_t d = 0; d < e.args.size(); ++d) {
            if (d) flat += " + ";
            flat += "(" + x(*e.args[d]) + ") * (int)" + b.name + "_meta.strides[" + std::to_string(d) + "]";
          }
          return b.name + "[" + flat + "]";
        }
        return x(b) + "[" + x(*e.args[0]) + "]";
      }
      case Expr::Call: {
        const std::string& n = e.name;
        if (n == "thread_id") return "_tid";
        if (n == "threadgroup_id") return "_tgid";
        if (n == "thread_in_threadgroup") return "_lid";
        if (n == "threads_per_threadgroup") return "_tgsize";
        if (n == "threads_per_grid") return "_gridsize";
        if (n == "barrier") return "__syncthreads()";
        std::string a0 = e.args.empty() ? "" : x(*e.args[0]);
        if (n == "relu") return "fmaxf(0.0f, " + a0 + ")";
        if (n == "sigmoid") return "__malus_sigmoid(" + a0 + ")";
        if (n == "abs") return "fabsf(" + a0 + ")";
        if (n == "sqrt") return "sqrtf(" + a0 + ")";
        if (n == "exp" || n == "log" || n == "tanh" || n == "rsqrt") return "__malus_" + n + "(" + a0 + ")";
        if (n == "fmax" || n == "fmin") return n + "f(" + a0 + ", " + x(*e.args[1]) + ")";
        if (n == "pow") return "__malus_pow(" + a0 + ", " + x(*e.args[1]) + ")";
        err(e.line, "unsupported call in explicit kernel body");
      }
      default: err(e.line, "unsupported expression kind in explicit kernel");
    }
  }

  const Kernel& k_;
  uint64_t id_;
  std::set<std::string> params_, locals_;
  std::set<std::string> tensor_names_, scalar_names_, used_;
};

// ---- synthesized builtins (codegen-gpu/lib.rs:373-418) -------------------------

std::string v1_header(const std::string& name, uint64_t id, const std::vector<std::string>& ins) {
  std::ostringstream o;
  o << "//@malus-v1-elem-bytes 4";
  for (size_t i = 0; i < ins.size(); ++i) o << " 4";
  o << "\n// malus builtin " << name << " (v1 ABI)\n";
  o << "extern \"C\" __global__ void malus_kernel_" << id << "(";
  for (auto& i : ins) o << "const float* __restrict__ " << i << ", ";
  o << "float* __restrict__ out, unsigned int n) {\n";
  o << "    const unsigned int tid = blockIdx.x * blockDim.x + threadIdx.x;\n";
  o << "    if (tid >= n) return;\n";
  return o.str();
}

std::string synth_unary(const std::string& name, uint64_t id) {
  std::string e;
  if (name == "relu") e = "fmaxf(0.0f, a[tid])";
  else if (name == "sigmoid") e = "1.0f / (1.0f + __malus_exp(-a[tid]))";
  else if (name == "tanh") e = "__malus_tanh(a[tid])";
  else if (name == "exp") e = "__malus_exp(a[tid])";
  else if (name == "log") e = "__malus_log(a[tid])";
  else if (name == "sqrt") e = "sqrtf(a[tid])";
  else if (name == "abs") e = "fabsf(a[tid])";
  else fail("malus: emit: unknown unary builtin: %s", name.c_str());
  std::string body = "    out[tid] = " + e + ";\n}\n";
  return prelude_for(body) + v1_header(name, id, {"a"}) + body;
}

std::string synth_elementwise(const std::string& name, Op op, uint64_t id) {
  return v1_header(name, id, {"a", "b"}) + "    out[tid] = (a[tid] " + op_infix(op) + " b[tid]);\n}\n";
}

// a@0, scalar_val@1 (a 1-element tensor), out@2
std::string synth_scalar(const std::string& name, Op op, bool scalar_on_right, uint64_t id) {
  std::string e = scalar_on_right ? std::string("(a[tid] ") + op_infix(op) + " scalar_val[0])"
                                  : std::string("(scalar_val[0] ") + op_infix(op) + " a[tid])";
  return "//@malus-v1-scalar-inputs 1\n" + v1_header(name, id, {"a", "scalar_val"}) + "    out[tid] = " + e + ";\n}\n";
}

// Process-global ids, never reset (codegen-gpu/lib.rs:9-11, ADR-0033).
std::atomic<uint64_t> g_next_id{0};

struct Entry {
  std::string name;
  uint64_t id;
  std::string source;
};

}  // namespace

struct malus_registry {
  std::vector<Entry> entries;
};

namespace malus {

// compile_kernels (codegen-gpu/lib.rs:95-155): user kernels in source order,
// then the tensor-tensor builtins (op order), then the scalar-broadcast
// builtins ((op, scalar_on_right) order; commutative forms share one kernel),
// then the unary builtins in name order.
malus_registry* compile_kernels(const std::string& program, const std::vector<std::string>& builtins, bool tags) {
  std::vector<Kernel> ks = Parser(Lexer(program).run()).kernels();
  for (auto& k : ks) Checker(k).run();
  auto reg = std::make_unique<malus_registry>();
  std::set<std::string> seen;
  auto add = [&](const std::string& name, uint64_t id, std::string src) {
    if (tags && dispatch_has_builtin(name)) src = "//@malus-builtin " + name + "\n" + src;
    reg->entries.push_back({name, id, std::move(src)});
    seen.insert(name);
  };
  for (auto& k : ks) {
    if (seen.count(k.name)) fail("malus: emit: kernel %s is defined twice", k.name.c_str());
    uint64_t id = g_next_id.fetch_add(1);
    std::string notes;
    std::string src = Lower(k, id).run(&notes);
    add(k.name, id, notes + src);
  }
  struct Key {
    int op;
    int right;
    std::string name;
    int kind;  // 0 tensor-tensor, 1 scalar, 2 unary
  };
  static const std::map<std::string, Key> known = {
      {"malus_add", {0, 0, "malus_add", 0}},          {"malus_sub", {1, 0, "malus_sub", 0}},
      {"malus_mul", {2, 0, "malus_mul", 0}},          {"malus_div", {3, 0, "malus_div", 0}},
      {"malus_add_scalar", {0, 1, "", 1}},            {"malus_rsub_scalar", {1, 0, "", 1}},
      {"malus_sub_scalar", {1, 1, "", 1}},            {"malus_mul_scalar", {2, 1, "", 1}},
      {"malus_rdiv_scalar", {3, 0, "", 1}},           {"malus_div_scalar", {3, 1, "", 1}},
      {"abs", {0, 0, "", 2}},  {"exp", {0, 0, "", 2}}, {"log", {0, 0, "", 2}}, {"relu", {0, 0, "", 2}},
      {"sigmoid", {0, 0, "", 2}}, {"sqrt", {0, 0, "", 2}}, {"tanh", {0, 0, "", 2}}};
  std::vector<std::pair<Key, std::string>> want;
  for (auto& b : builtins) {
    auto it = known.find(b);
    if (it == known.end()) fail("malus: emit: unknown builtin kernel name '%s'", b.c_str());
    if (seen.count(b)) fail("malus: emit: builtin %s collides with a kernel of that name", b.c_str());
    bool dup = false;
    for (auto& w : want) dup |= w.second == b;
    if (!dup) want.emplace_back(it->second, b);
  }
  std::stable_sort(want.begin(), want.end(), [](const auto& x, const auto& y) {
    if (x.first.kind != y.first.kind) return x.first.kind < y.first.kind;
    if (x.first.kind == 2) return x.second < y.second;
    if (x.first.op != y.first.op) return x.first.op < y.first.op;
    return x.first.right < y.first.right;
  });
  static const Op ops[4] = {Op::Add, Op::Sub, Op::Mul, Op::Div};
  for (auto& w : want) {
    uint64_t id = g_next_id.fetch_add(1);
    const Key& key = w.first;
    std::string src;
    if (key.kind == 0) src = synth_elementwise(w.second, ops[key.op], id);
    else if (key.kind == 1) src = synth_scalar(w.second, ops[key.op], key.right != 0, id);
    else src = synth_unary(w.second, id);
    add(w.second, id, src);
  }
  return reg.release();
}

}  // namespace malus

extern "C" {

malus_registry* malus_compile_kernels(const char* program, const char* const* builtins, size_t nbuiltins, int flags) {
  API_TRY
  std::vector<std::string> b;
  for (size_t i = 0; i < nbuiltins; ++i) b.emplace_back(builtins[i] ? builtins[i] : "");
  return malus::compile_kernels(program ? program : "", b, (flags & 1) != 0);
  API_CATCH(nullptr)
}

size_t malus_registry_len(const malus_registry* r) { return r ? r->entries.size() : 0; }
uint64_t malus_registry_id(const malus_registry* r, size_t i) { return r->entries.at(i).id; }
const char* malus_registry_name(const malus_registry* r, size_t i) { return r->entries.at(i).name.c_str(); }
const char* malus_registry_source(const malus_registry* r, size_t i) { return r->entries.at(i).source.c_str(); }
int malus_registry_lookup(const malus_registry* r, const char* name, uint64_t* id) {
  if (!r || !name) return 0;
  for (auto& e : r->entries)
    if (e.name == name) {
      if (id) *id = e.id;
      return 1;
    }
  return 0;
}
void malus_registry_free(malus_registry* r) { delete r; }

}  // extern "C"
