// Types, attributes, diagnostics, the textual parser and the printer for the
// `xt` IR subset.  The accepted syntax is the MLIR generic/custom form that the
// reference tracer emits (xtile/dsl.py:490-620) and that the reference's lit
// tests feed to xt-opt (test/xt/parse.mlir, test/xt/serialize.mlir).  Op
// assembly formats follow include/xt/XTOps.td:15-170.
#include "ir.h"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <unordered_map>

namespace xt {

// ---------------------------------------------------------------------------
// element types, types, attributes
// ---------------------------------------------------------------------------

const char* elem_name(Elem e) {
  switch (e) {
    case Elem::F32: return "f32";
    case Elem::F16: return "f16";
    case Elem::BF16: return "bf16";
    case Elem::I8: return "i8";
    case Elem::I32: return "i32";
    case Elem::I64: return "i64";
    case Elem::I1: return "i1";
    case Elem::Index: return "index";
    default: return "?";
  }
}

int elem_bytes(Elem e) {
  switch (e) {
    case Elem::F32: case Elem::I32: return 4;
    case Elem::F16: case Elem::BF16: return 2;
    case Elem::I8: case Elem::I1: return 1;
    case Elem::I64: case Elem::Index: return 8;
    default: return 0;
  }
}

bool elem_is_float(Elem e) { return e == Elem::F32 || e == Elem::F16 || e == Elem::BF16; }
bool elem_is_int(Elem e) {
  return e == Elem::I8 || e == Elem::I32 || e == Elem::I64 || e == Elem::I1;
}

static bool elem_from_name(const std::string& n, Elem& out) {
  static const std::pair<const char*, Elem> table[] = {
      {"f32", Elem::F32}, {"f16", Elem::F16}, {"bf16", Elem::BF16}, {"i8", Elem::I8},
      {"i32", Elem::I32}, {"i64", Elem::I64}, {"i1", Elem::I1},     {"index", Elem::Index}};
  for (auto& [name, e] : table)
    if (n == name) {
      out = e;
      return true;
    }
  return false;
}

int64_t Type::numel() const {
  int64_t n = 1;
  for (int64_t d : shape) n *= d;
  return n;
}

std::string Type::str() const {
  if (kind == Scalar) return elem_name(elem);
  if (kind != Tensor && kind != MemRef) return "<invalid>";
  std::string out = kind == Tensor ? "tensor<" : "memref<";
  for (int64_t d : shape) out += std::to_string(d) + "x";
  out += elem_name(elem);
  out += ">";
  return out;
}

static std::string format_float(double v) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.6e", v);
  if (std::strtod(buf, nullptr) == v) return buf;
  std::snprintf(buf, sizeof buf, "%.17g", v);
  std::string s = buf;
  if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
  return s;
}

std::string Attr::str() const {
  switch (kind) {
    case Unit: return "";
    case Int: return std::to_string(i) + " : " + type.str();
    case Float: return format_float(f) + " : " + type.str();
    case Bool: return i ? "true" : "false";
    case DenseArray: {
      std::string out = std::string("array<") + elem_name(type.elem);
      for (size_t k = 0; k < ints.size(); ++k) out += (k ? ", " : ": ") + std::to_string(ints[k]);
      return out + ">";
    }
    case List: {
      std::string out = "[";
      for (size_t k = 0; k < ints.size(); ++k) out += (k ? ", " : "") + std::to_string(ints[k]);
      return out + "]";
    }
    case DenseSplat: {
      std::string v;
      if (type.elem == Elem::I1) v = i ? "true" : "false";
      else if (splat_is_float) v = format_float(f);
      else v = std::to_string(i);
      return "dense<" + v + "> : " + type.str();
    }
    case String: return "\"" + s + "\"";
  }
  return "";
}

const Attr* find_attr(const AttrDict& d, const std::string& name) {
  for (auto& kv : d)
    if (kv.first == name) return &kv.second;
  return nullptr;
}

void set_attr(AttrDict& d, const std::string& name, Attr a) {
  for (auto& kv : d)
    if (kv.first == name) {
      kv.second = std::move(a);
      return;
    }
  d.emplace_back(name, std::move(a));
  std::sort(d.begin(), d.end(), [](auto& x, auto& y) { return x.first < y.first; });
}

void erase_attr(AttrDict& d, const std::string& name) {
  d.erase(std::remove_if(d.begin(), d.end(), [&](auto& kv) { return kv.first == name; }),
          d.end());
}

void Diag::error(const std::string& src, Loc loc, const std::string& msg) {
  lines.push_back(src + ":" + std::to_string(loc.line) + ":" + std::to_string(loc.col) +
                  ": error: " + msg);
}

std::string Diag::joined() const {
  std::string out;
  for (size_t k = 0; k < lines.size(); ++k) out += (k ? "\n" : "") + lines[k];
  return out;
}

const Func* find_func(const Module& m, const std::string& name) {
  for (auto& f : m.funcs)
    if (f.name == name) return &f;
  return nullptr;
}

bool get_grid(const Func& f, int32_t grid[3]) {
  const Attr* a = find_attr(f.attrs, "xt.grid");
  if (!a || a->kind != Attr::DenseArray || a->type.elem != Elem::I32 || a->ints.size() != 3)
    return false;
  for (int k = 0; k < 3; ++k) grid[k] = static_cast<int32_t>(a->ints[k]);
  return true;
}

bool is_pure_op(const std::string& n) {
  // Ops carrying the `Pure` trait in include/xt/XTOps.td plus arith.constant.
  static const char* pure[] = {"xt.get_tile_block_id", "xt.add", "xt.sub", "xt.mul",
                               "xt.exp", "xt.cos", "xt.sin", "xt.reciprocal", "xt.rsqrt",
                               "xt.sigmoid", "xt.tanh", "xt.silu", "xt.itof", "xt.ftoi",
                               "xt.matmul", "xt.mma", "xt.reduce_sum", "xt.reduce_max",
                               "xt.reshape", "xt.transpose", "xt.permute", "arith.constant"};
  for (const char* p : pure)
    if (n == p) return true;
  return false;
}

std::vector<std::string> split_input_chunks(const std::string& text) {
  std::vector<std::string> chunks;
  std::string cur;
  std::istringstream in(text);
  std::string line;
  while (std::getline(in, line)) {
    size_t a = line.find_first_not_of(" \t");
    if (a != std::string::npos && line.compare(a, 8, "// -----") == 0) {
      chunks.push_back(cur);
      cur.clear();
      continue;
    }
    cur += line + "\n";
  }
  chunks.push_back(cur);
  return chunks;
}

// ---------------------------------------------------------------------------
// parser
// ---------------------------------------------------------------------------

namespace {

enum class Fmt {
  BlockId,     // xt.get_tile_block_id attr-dict : t, t, t
  Constant,    // arith.constant <attr-value>
  Functional,  // ( operands ) attr-dict : ( types ) -> type | ()
  Arith,       // ( operands ) attr-dict : types -> type
  Permute,     // ( %a ) { permutation = [..] } attr-dict : t -> t
  Return,      // func.return [operands : types]
  Br,          // cf.br ^bb [( operands : types )]
  CondBr,      // cf.cond_br %c, ^a, ^b
};

struct OpInfo {
  Fmt fmt;
  int min_operands;
  int max_operands;  // -1: variadic
  int results;       // -1: any
};

const std::unordered_map<std::string, OpInfo>& op_table() {
  static const std::unordered_map<std::string, OpInfo> t = {
      {"xt.get_tile_block_id", {Fmt::BlockId, 0, 0, 3}},
      {"arith.constant", {Fmt::Constant, 0, 0, 1}},
      {"xt.load", {Fmt::Functional, 1, -1, 1}},
      {"xt.load_conv2d", {Fmt::Functional, 6, 6, 1}},
      {"xt.store", {Fmt::Functional, 2, -1, 0}},
      {"xt.add", {Fmt::Arith, 2, 2, 1}},
      {"xt.sub", {Fmt::Arith, 2, 2, 1}},
      {"xt.mul", {Fmt::Arith, 2, 2, 1}},
      {"xt.matmul", {Fmt::Arith, 2, 2, 1}},
      {"xt.mma", {Fmt::Arith, 3, 3, 1}},
      {"xt.exp", {Fmt::Arith, 1, 1, 1}},
      {"xt.cos", {Fmt::Arith, 1, 1, 1}},
      {"xt.sin", {Fmt::Arith, 1, 1, 1}},
      {"xt.reciprocal", {Fmt::Arith, 1, 1, 1}},
      {"xt.rsqrt", {Fmt::Arith, 1, 1, 1}},
      {"xt.sigmoid", {Fmt::Arith, 1, 1, 1}},
      {"xt.tanh", {Fmt::Arith, 1, 1, 1}},
      {"xt.silu", {Fmt::Arith, 1, 1, 1}},
      {"xt.itof", {Fmt::Arith, 1, 1, 1}},
      {"xt.ftoi", {Fmt::Arith, 1, 1, 1}},
      {"xt.reduce_sum", {Fmt::Arith, 1, 1, 1}},
      {"xt.reduce_max", {Fmt::Arith, 1, 1, 1}},
      {"xt.reshape", {Fmt::Arith, 1, 1, 1}},
      {"xt.transpose", {Fmt::Arith, 1, 1, 1}},
      {"xt.permute", {Fmt::Permute, 1, 1, 1}},
      {"func.return", {Fmt::Return, 0, -1, 0}},
      {"cf.br", {Fmt::Br, 0, -1, 0}},
      {"cf.cond_br", {Fmt::CondBr, 1, 1, 0}},
  };
  return t;
}

bool is_id_char(char c) {
  return std::isalnum(static_cast<unsigned char>(c)) || c == '_' || c == '$' || c == '.' ||
         c == '-';
}

class Parser {
 public:
  Parser(const std::string& text, Diag& diag, std::string src)
      : s_(text), diag_(diag), src_(std::move(src)) {}

  std::unique_ptr<Module> run() {
    auto m = std::make_unique<Module>();
    m->source_name = src_;
    ws();
    m->loc = loc();
    if (keyword("module")) {
      ws();
      if (peek() == '@') {  // optional module symbol name
        adv();
        ident_chars();
        ws();
      }
      if (keyword("attributes")) {
        if (!attr_dict(m->attrs)) return nullptr;
      }
      if (!expect('{')) return nullptr;
      while (true) {
        ws();
        if (peek() == '}') {
          adv();
          break;
        }
        if (at_end()) return fail("expected '}' to close module"), nullptr;
        if (!func(*m)) return nullptr;
      }
      ws();
      if (!at_end()) return fail("unexpected text after module"), nullptr;
    } else {
      while (true) {
        ws();
        if (at_end()) break;
        if (!func(*m)) return nullptr;
      }
    }
    return m;
  }

 private:
  const std::string& s_;
  size_t p_ = 0;
  int line_ = 1, col_ = 1;
  Diag& diag_;
  std::string src_;
  bool failed_ = false;

  // value scope of the function being parsed
  std::unordered_map<std::string, int> names_;
  Func* fn_ = nullptr;

  // -- characters --
  bool at_end() const { return p_ >= s_.size(); }
  char peek(size_t k = 0) const { return p_ + k < s_.size() ? s_[p_ + k] : '\0'; }
  void adv() {
    if (at_end()) return;
    if (s_[p_] == '\n') {
      ++line_;
      col_ = 1;
    } else {
      ++col_;
    }
    ++p_;
  }
  Loc loc() const { return Loc{line_, col_}; }
  void ws() {
    while (!at_end()) {
      char c = peek();
      if (c == ' ' || c == '\t' || c == '\n' || c == '\r') {
        adv();
      } else if (c == '/' && peek(1) == '/') {
        while (!at_end() && peek() != '\n') adv();
      } else {
        break;
      }
    }
  }
  bool fail(const std::string& msg) { return fail_at(loc(), msg); }
  bool fail_at(Loc l, const std::string& msg) {
    if (!failed_) diag_.error(src_, l, msg);
    failed_ = true;
    return false;
  }
  bool expect(char c) {
    ws();
    if (peek() != c) return fail(std::string("expected '") + c + "'");
    adv();
    return true;
  }
  bool eat(char c) {
    ws();
    if (peek() != c) return false;
    adv();
    return true;
  }
  bool eat_arrow() {
    ws();
    if (peek() == '-' && peek(1) == '>') {
      adv();
      adv();
      return true;
    }
    return false;
  }
  // keyword followed by a non-identifier character
  bool keyword(const char* kw) {
    ws();
    size_t n = std::strlen(kw);
    if (s_.compare(p_, n, kw) != 0) return false;
    char after = p_ + n < s_.size() ? s_[p_ + n] : '\0';
    if (std::isalnum(static_cast<unsigned char>(after)) || after == '_' || after == '.')
      return false;
    for (size_t k = 0; k < n; ++k) adv();
    return true;
  }
  std::string ident_chars() {
    std::string out;
    while (!at_end() && is_id_char(peek())) {
      out += peek();
      adv();
    }
    return out;
  }
  std::string bare_ident() {
    ws();
    std::string out;
    if (!(std::isalpha(static_cast<unsigned char>(peek())) || peek() == '_')) return out;
    while (!at_end()) {
      char c = peek();
      if (std::isalnum(static_cast<unsigned char>(c)) || c == '_' || c == '$' || c == '.') {
        out += c;
        adv();
      } else {
        break;
      }
    }
    return out;
  }
  bool integer(int64_t& v) {
    ws();
    bool neg = false;
    size_t save = p_;
    int sl = line_, sc = col_;
    if (peek() == '-') {
      neg = true;
      adv();
    }
    if (!std::isdigit(static_cast<unsigned char>(peek()))) {
      p_ = save;
      line_ = sl;
      col_ = sc;
      return false;
    }
    int64_t acc = 0;
    while (std::isdigit(static_cast<unsigned char>(peek()))) {
      acc = acc * 10 + (peek() - '0');
      adv();
    }
    v = neg ? -acc : acc;
    return true;
  }
  // number literal: returns is_float and value
  bool number(bool& is_float, int64_t& iv, double& fv) {
    ws();
    size_t start = p_;
    if (peek() == '-' || peek() == '+') adv();
    if (!std::isdigit(static_cast<unsigned char>(peek()))) return fail("expected number");
    if (peek() == '0' && (peek(1) == 'x' || peek(1) == 'X')) {
      adv();
      adv();
      while (std::isxdigit(static_cast<unsigned char>(peek()))) adv();
      std::string text = s_.substr(start, p_ - start);
      is_float = false;
      iv = std::strtoll(text.c_str(), nullptr, 16);
      return true;
    }
    while (std::isdigit(static_cast<unsigned char>(peek()))) adv();
    is_float = false;
    if (peek() == '.') {
      is_float = true;
      adv();
      while (std::isdigit(static_cast<unsigned char>(peek()))) adv();
    }
    if (peek() == 'e' || peek() == 'E') {
      is_float = true;
      adv();
      if (peek() == '-' || peek() == '+') adv();
      while (std::isdigit(static_cast<unsigned char>(peek()))) adv();
    }
    std::string text = s_.substr(start, p_ - start);
    if (is_float) fv = std::strtod(text.c_str(), nullptr);
    else iv = std::strtoll(text.c_str(), nullptr, 10);
    return true;
  }

  // -- types --
  bool elem_type(Elem& e) {
    ws();
    Loc l = loc();
    std::string n;
    while (std::isalnum(static_cast<unsigned char>(peek()))) {
      n += peek();
      adv();
    }
    if (!elem_from_name(n, e)) return fail_at(l, "unsupported element type '" + n + "'");
    return true;
  }
  bool type(Type& t) {
    ws();
    Loc l = loc();
    bool is_tensor = false;
    if (keyword("tensor")) is_tensor = true;
    else if (!keyword("memref")) {
      Elem e;
      if (!elem_type(e)) return false;
      t = Type::scalar(e);
      return true;
    }
    if (!expect('<')) return false;
    std::vector<int64_t> shape;
    ws();
    while (std::isdigit(static_cast<unsigned char>(peek())) || peek() == '?') {
      if (peek() == '?') return fail_at(l, "dynamic shapes are not supported");
      int64_t d = 0;
      while (std::isdigit(static_cast<unsigned char>(peek()))) {
        d = d * 10 + (peek() - '0');
        adv();
      }
      shape.push_back(d);
      if (peek() != 'x') return fail("expected 'x' in shaped type");
      adv();
    }
    Elem e;
    if (!elem_type(e)) return false;
    ws();
    if (peek() == ',') return fail_at(l, "memref layouts and memory spaces are not supported");
    if (!expect('>')) return false;
    t = is_tensor ? Type::tensor(e, shape) : Type::memref(e, shape);
    return true;
  }

  // -- attributes --
  bool attr_value(Attr& a) {
    ws();
    Loc l = loc();
    if (keyword("array")) {
      if (!expect('<')) return false;
      Elem e;
      if (!elem_type(e)) return false;
      a.kind = Attr::DenseArray;
      a.type = Type::scalar(e);
      if (eat(':')) {
        do {
          int64_t v;
          if (!integer(v)) return fail("expected integer in array attribute");
          a.ints.push_back(v);
        } while (eat(','));
      }
      return expect('>');
    }
    if (keyword("dense")) {
      if (!expect('<')) return false;
      a.kind = Attr::DenseSplat;
      ws();
      if (peek() == '[') return fail_at(l, "only splat dense attributes are supported");
      if (keyword("true")) {
        a.i = 1;
      } else if (keyword("false")) {
        a.i = 0;
      } else {
        bool is_f;
        if (!number(is_f, a.i, a.f)) return false;
        a.splat_is_float = is_f;
        if (is_f) a.i = static_cast<int64_t>(a.f);
        else a.f = static_cast<double>(a.i);
      }
      if (!expect('>')) return false;
      if (!expect(':')) return false;
      if (!type(a.type)) return false;
      if (!a.type.is_tensor()) return fail_at(l, "dense attribute requires a tensor type");
      if (elem_is_float(a.type.elem)) a.splat_is_float = true;
      return true;
    }
    if (keyword("true")) {
      a.kind = Attr::Bool;
      a.i = 1;
      a.type = Type::scalar(Elem::I1);
      return true;
    }
    if (keyword("false")) {
      a.kind = Attr::Bool;
      a.i = 0;
      a.type = Type::scalar(Elem::I1);
      return true;
    }
    if (keyword("unit")) {
      a.kind = Attr::Unit;
      return true;
    }
    if (peek() == '[') {
      adv();
      a.kind = Attr::List;
      if (!eat(']')) {
        do {
          int64_t v;
          if (!integer(v)) return fail("expected integer in list attribute");
          a.ints.push_back(v);
        } while (eat(','));
        if (!expect(']')) return false;
      }
      return true;
    }
    if (peek() == '"') {
      adv();
      a.kind = Attr::String;
      while (!at_end() && peek() != '"') {
        a.s += peek();
        adv();
      }
      return expect('"');
    }
    bool is_f;
    if (!number(is_f, a.i, a.f)) return false;
    a.kind = is_f ? Attr::Float : Attr::Int;
    a.type = Type::scalar(is_f ? Elem::F32 : Elem::I64);
    if (eat(':')) {
      if (!type(a.type)) return false;
      if (!a.type.is_scalar()) return fail_at(l, "expected a scalar attribute type");
      if (elem_is_float(a.type.elem) && !is_f) {
        a.kind = Attr::Float;
        a.f = static_cast<double>(a.i);
      }
    }
    return true;
  }
  bool attr_dict(AttrDict& d) {
    if (!expect('{')) return false;
    if (eat('}')) return true;
    do {
      ws();
      std::string name;
      if (peek() == '"') {
        adv();
        while (!at_end() && peek() != '"') {
          name += peek();
          adv();
        }
        if (!expect('"')) return false;
      } else {
        name = bare_ident();
      }
      if (name.empty()) return fail("expected attribute name");
      Attr a;
      if (eat('=')) {
        if (!attr_value(a)) return false;
      }
      set_attr(d, name, a);
    } while (eat(','));
    return expect('}');
  }

  // -- SSA values --
  bool value_ref(int& id, std::string& spelled) {
    ws();
    Loc l = loc();
    if (peek() != '%') return fail("expected SSA value");
    adv();
    std::string n = ident_chars();
    if (peek() == '#') {
      adv();
      n += '#';
      while (std::isdigit(static_cast<unsigned char>(peek()))) {
        n += peek();
        adv();
      }
    }
    spelled = "%" + n;
    auto it = names_.find(n);
    if (it == names_.end()) return fail_at(l, "use of undeclared SSA value name");
    id = it->second;
    return true;
  }
  bool define(const std::string& n, int id, Loc l) {
    if (names_.count(n)) return fail_at(l, "redefinition of SSA value '%" + n + "'");
    names_[n] = id;
    return true;
  }
  bool check_type(int id, const Type& t, const std::string& spelled, Loc l) {
    const Type& have = fn_->type_of(id);
    if (have != t)
      return fail_at(l, "use of value '" + spelled +
                            "' expects different type than prior uses: '" + t.str() + "' vs '" +
                            have.str() + "'");
    return true;
  }

  // -- functions --
  bool func(Module& m) {
    ws();
    Loc fl = loc();
    if (!keyword("func.func")) {
      std::string w = bare_ident();
      if (w.empty()) return fail("expected 'func.func'");
      return fail_at(fl, "custom op '" + w + "' is unknown");
    }
    if (keyword("private") || keyword("public") || keyword("nested")) {
    }
    ws();
    if (peek() != '@') return fail("expected function symbol name");
    adv();
    m.funcs.emplace_back();
    Func& f = m.funcs.back();
    f.loc = fl;
    f.name = ident_chars();
    fn_ = &f;
    names_.clear();
    if (!expect('(')) return false;
    if (!eat(')')) {
      do {
        ws();
        Loc al = loc();
        if (peek() != '%') return fail("expected argument name");
        adv();
        std::string n = ident_chars();
        if (!expect(':')) return false;
        Type t;
        if (!type(t)) return false;
        int id = f.add_value(t, "%" + n);
        f.values[id].def_op = -1;
        if (!define(n, id, al)) return false;
        f.args.push_back(id);
        ws();
        if (peek() == '{') {  // argument attributes: parsed and dropped
          AttrDict ignored;
          if (!attr_dict(ignored)) return false;
        }
      } while (eat(','));
      if (!expect(')')) return false;
    }
    if (eat_arrow()) {
      if (eat('(')) {
        if (!eat(')')) {
          do {
            Type t;
            if (!type(t)) return false;
            f.result_types.push_back(t);
          } while (eat(','));
          if (!expect(')')) return false;
        }
      } else {
        Type t;
        if (!type(t)) return false;
        f.result_types.push_back(t);
      }
    }
    if (keyword("attributes")) {
      if (!attr_dict(f.attrs)) return false;
    }
    ws();
    if (peek() != '{') return true;  // declaration only
    adv();
    f.blocks.emplace_back();
    while (true) {
      ws();
      if (peek() == '}') {
        adv();
        break;
      }
      if (at_end()) return fail("expected '}' to close function body");
      if (peek() == '^') {
        adv();
        Block b;
        b.label = ident_chars();
        if (eat('(')) {
          if (!eat(')')) {
            do {
              ws();
              Loc al = loc();
              if (!expect('%')) return false;
              std::string n = ident_chars();
              if (!expect(':')) return false;
              Type t;
              if (!type(t)) return false;
              int id = f.add_value(t, "%" + n);
              f.values[id].def_block = static_cast<int>(f.blocks.size());
              if (!define(n, id, al)) return false;
              b.args.push_back(id);
            } while (eat(','));
            if (!expect(')')) return false;
          }
        }
        if (!expect(':')) return false;
        if (f.blocks.size() == 1 && f.blocks[0].ops.empty() && f.blocks[0].label.empty() &&
            f.blocks[0].args.empty()) {
          f.blocks[0] = std::move(b);
        } else {
          f.blocks.push_back(std::move(b));
        }
        continue;
      }
      if (!op(f)) return false;
    }
    // every block must end in a terminator
    for (auto& b : f.blocks) {
      if (b.ops.empty() || (b.ops.back().name != "func.return" && b.ops.back().name != "cf.br" &&
                            b.ops.back().name != "cf.cond_br"))
        return fail_at(b.ops.empty() ? f.loc : b.ops.back().loc,
                       "block with no terminator, has " +
                           (b.ops.empty() ? std::string("no operations") : b.ops.back().name));
    }
    return true;
  }

  bool op(Func& f) {
    ws();
    Loc l = loc();
    // result list
    struct ResName {
      std::string name;
      int count;
      Loc loc;
    };
    std::vector<ResName> res;
    if (peek() == '%') {
      do {
        ws();
        Loc rl = loc();
        if (!expect('%')) return false;
        std::string n = ident_chars();
        int count = 1;
        if (peek() == ':') {
          adv();
          int64_t c;
          if (!integer(c) || c <= 0) return fail("expected result count");
          count = static_cast<int>(c);
        }
        res.push_back({n, count, rl});
      } while (eat(','));
      if (!expect('=')) return false;
    }
    ws();
    Loc name_loc = loc();
    std::string name;
    bool generic = false;
    if (peek() == '"') {
      generic = true;
      adv();
      while (!at_end() && peek() != '"') {
        name += peek();
        adv();
      }
      if (!expect('"')) return false;
    } else {
      name = bare_ident();
    }
    if (name == "return") name = "func.return";
    auto& table = op_table();
    auto it = table.find(name);
    if (it == table.end()) {
      if (name.empty()) return fail_at(name_loc, "expected operation name");
      return fail_at(name_loc, "custom op '" + name + "' is unknown");
    }
    const OpInfo& info = it->second;
    Op o;
    o.name = name;
    o.loc = l;
    std::vector<Type> result_types;
    std::vector<std::pair<std::string, Loc>> spelled;  // operand spellings

    auto operand_list = [&](char close) -> bool {
      if (eat(close)) return true;
      do {
        int id;
        std::string sp;
        ws();
        Loc ol = loc();
        if (!value_ref(id, sp)) return false;
        o.operands.push_back(id);
        spelled.push_back({sp, ol});
      } while (eat(','));
      return expect(close);
    };
    auto check_operand_types = [&](const std::vector<Type>& types) -> bool {
      if (types.size() != o.operands.size())
        return fail_at(l, std::to_string(o.operands.size()) + " operands present, but expected " +
                              std::to_string(types.size()));
      for (size_t k = 0; k < types.size(); ++k)
        if (!check_type(o.operands[k], types[k], spelled[k].first, spelled[k].second))
          return false;
      return true;
    };

    if (generic) {
      if (!expect('(')) return false;
      if (!operand_list(')')) return false;
      ws();
      if (peek() == '[') {
        adv();
        do {
          ws();
          if (!expect('^')) return false;
          o.successors.push_back(ident_chars());
        } while (eat(','));
        if (!expect(']')) return false;
      }
      ws();
      if (peek() == '{' && !attr_dict(o.attrs)) return false;
      if (!expect(':')) return false;
      std::vector<Type> ins;
      if (!expect('(')) return false;
      if (!eat(')')) {
        do {
          Type t;
          if (!type(t)) return false;
          ins.push_back(t);
        } while (eat(','));
        if (!expect(')')) return false;
      }
      if (!check_operand_types(ins)) return false;
      if (!eat_arrow()) return fail("expected '->'");
      if (eat('(')) {
        if (!eat(')')) {
          do {
            Type t;
            if (!type(t)) return false;
            result_types.push_back(t);
          } while (eat(','));
          if (!expect(')')) return false;
        }
      } else {
        Type t;
        if (!type(t)) return false;
        result_types.push_back(t);
      }
    } else {
      switch (info.fmt) {
        case Fmt::BlockId: {
          ws();
          if (peek() == '{' && !attr_dict(o.attrs)) return false;
          if (!expect(':')) return false;
          do {
            Type t;
            if (!type(t)) return false;
            result_types.push_back(t);
          } while (eat(','));
          break;
        }
        case Fmt::Constant: {
          ws();
          if (peek() == '{' && !attr_dict(o.attrs)) return false;
          Attr v;
          if (!attr_value(v)) return false;
          if (v.kind == Attr::Int || v.kind == Attr::Float) {
            result_types.push_back(v.type);
          } else if (v.kind == Attr::Bool) {
            result_types.push_back(Type::scalar(Elem::I1));
          } else if (v.kind == Attr::DenseSplat) {
            result_types.push_back(v.type);
          } else {
            return fail_at(l, "unsupported arith.constant value");
          }
          set_attr(o.attrs, "value", v);
          break;
        }
        case Fmt::Functional: {
          if (!expect('(')) return false;
          if (!operand_list(')')) return false;
          ws();
          if (peek() == '{' && !attr_dict(o.attrs)) return false;
          if (!expect(':')) return false;
          if (!expect('(')) return false;
          std::vector<Type> ins;
          if (!eat(')')) {
            do {
              Type t;
              if (!type(t)) return false;
              ins.push_back(t);
            } while (eat(','));
            if (!expect(')')) return false;
          }
          if (!check_operand_types(ins)) return false;
          if (!eat_arrow()) return fail("expected '->'");
          if (eat('(')) {
            if (!expect(')')) return false;
          } else {
            Type t;
            if (!type(t)) return false;
            result_types.push_back(t);
          }
          break;
        }
        case Fmt::Arith: {
          if (!expect('(')) return false;
          if (!operand_list(')')) return false;
          ws();
          if (peek() == '{' && !attr_dict(o.attrs)) return false;
          if (!expect(':')) return false;
          std::vector<Type> ins;
          do {
            Type t;
            if (!type(t)) return false;
            ins.push_back(t);
          } while (eat(','));
          if (!check_operand_types(ins)) return false;
          if (!eat_arrow()) return fail("expected '->'");
          Type t;
          if (!type(t)) return false;
          result_types.push_back(t);
          break;
        }
        case Fmt::Permute: {
          if (!expect('(')) return false;
          if (!operand_list(')')) return false;
          if (!expect('{')) return false;
          if (!keyword("permutation")) return fail("expected 'permutation'");
          if (!expect('=')) return false;
          Attr perm;
          ws();
          if (peek() != '[') return fail("expected '['");
          if (!attr_value(perm)) return false;
          if (!expect('}')) return false;
          ws();
          if (peek() == '{' && !attr_dict(o.attrs)) return false;
          set_attr(o.attrs, "permutation", perm);
          if (!expect(':')) return false;
          Type tin, tout;
          if (!type(tin)) return false;
          if (!check_operand_types({tin})) return false;
          if (!eat_arrow()) return fail("expected '->'");
          if (!type(tout)) return false;
          result_types.push_back(tout);
          break;
        }
        case Fmt::Return: {
          ws();
          if (peek() == '%') {
            do {
              int id;
              std::string sp;
              ws();
              Loc ol = loc();
              if (!value_ref(id, sp)) return false;
              o.operands.push_back(id);
              spelled.push_back({sp, ol});
            } while (eat(','));
            if (!expect(':')) return false;
            std::vector<Type> ins;
            do {
              Type t;
              if (!type(t)) return false;
              ins.push_back(t);
            } while (eat(','));
            if (!check_operand_types(ins)) return false;
          }
          break;
        }
        case Fmt::Br: {
          ws();
          if (!expect('^')) return false;
          o.successors.push_back(ident_chars());
          if (eat('(')) {
            do {
              int id;
              std::string sp;
              ws();
              Loc ol = loc();
              if (!value_ref(id, sp)) return false;
              o.operands.push_back(id);
              spelled.push_back({sp, ol});
            } while (eat(','));
            if (!expect(':')) return false;
            std::vector<Type> ins;
            do {
              Type t;
              if (!type(t)) return false;
              ins.push_back(t);
            } while (eat(','));
            if (!expect(')')) return false;
            if (!check_operand_types(ins)) return false;
          }
          break;
        }
        case Fmt::CondBr: {
          int id;
          std::string sp;
          ws();
          Loc ol = loc();
          if (!value_ref(id, sp)) return false;
          o.operands.push_back(id);
          spelled.push_back({sp, ol});
          if (!check_type(id, Type::scalar(Elem::I1), sp, ol)) return false;
          for (int k = 0; k < 2; ++k) {
            if (!expect(',')) return false;
            ws();
            if (!expect('^')) return false;
            o.successors.push_back(ident_chars());
          }
          break;
        }
      }
    }

    // arity
    int nops = static_cast<int>(o.operands.size());
    if (nops < info.min_operands || (info.max_operands >= 0 && nops > info.max_operands))
      return fail_at(l, "'" + name + "' op unexpected number of operands (" +
                            std::to_string(nops) + ")");
    if (info.results >= 0 && static_cast<int>(result_types.size()) != info.results)
      return fail_at(l, "'" + name + "' op requires " + std::to_string(info.results) +
                            " results, got " + std::to_string(result_types.size()));
    int declared = 0;
    for (auto& r : res) declared += r.count;
    if (declared != static_cast<int>(result_types.size()))
      return fail_at(l, "operation defines " + std::to_string(result_types.size()) +
                            " results but was provided " + std::to_string(declared) +
                            " to bind");

    int block_index = static_cast<int>(f.blocks.size()) - 1;
    int op_index = static_cast<int>(f.blocks.back().ops.size());
    size_t k = 0;
    for (auto& r : res) {
      for (int j = 0; j < r.count; ++j, ++k) {
        int id = f.add_value(result_types[k], "%" + r.name);
        f.values[id].def_op = op_index;
        f.values[id].def_block = block_index;
        f.values[id].result_no = static_cast<int>(k);
        o.results.push_back(id);
        std::string key = r.count == 1 ? r.name : r.name + "#" + std::to_string(j);
        if (!define(key, id, r.loc)) return false;
        if (r.count > 1 && j == 0) names_.emplace(r.name, id);
      }
    }
    f.blocks.back().ops.push_back(std::move(o));
    return true;
  }
};

}  // namespace

std::unique_ptr<Module> parse_module(const std::string& text, Diag& diag,
                                     const std::string& source_name) {
  Parser p(text, diag, source_name);
  auto m = p.run();
  if (!m || !diag.empty()) return nullptr;
  if (!verify_module(*m, diag)) return nullptr;
  return m;
}

// ---------------------------------------------------------------------------
// printer
// ---------------------------------------------------------------------------

namespace {

std::string attr_dict_text(const AttrDict& d, const std::vector<std::string>& skip = {}) {
  std::string out;
  for (auto& [name, a] : d) {
    if (std::find(skip.begin(), skip.end(), name) != skip.end()) continue;
    out += out.empty() ? "" : ", ";
    out += name;
    if (a.kind != Attr::Unit) out += " = " + a.str();
  }
  return out.empty() ? out : "{" + out + "}";
}

struct Printer {
  const Func& f;
  std::vector<std::string> names;

  explicit Printer(const Func& fn) : f(fn), names(fn.values.size()) {
    int next = 0;
    for (size_t k = 0; k < f.args.size(); ++k) names[f.args[k]] = "%arg" + std::to_string(k);
    for (auto& b : f.blocks) {
      for (int a : b.args) names[a] = "%" + std::to_string(next++);
      for (auto& o : b.ops)
        for (int r : o.results) names[r] = "%" + std::to_string(next++);
    }
  }

  std::string types_of(const std::vector<int>& vs) const {
    std::string out;
    for (size_t k = 0; k < vs.size(); ++k) out += (k ? ", " : "") + f.type_of(vs[k]).str();
    return out;
  }
  std::string refs(const std::vector<int>& vs) const {
    std::string out;
    for (size_t k = 0; k < vs.size(); ++k) out += (k ? ", " : "") + names[vs[k]];
    return out;
  }

  std::string op(const Op& o) const {
    std::string out;
    if (!o.results.empty()) out += refs(o.results) + " = ";
    auto attrs = [&](const std::vector<std::string>& skip = {}) {
      std::string a = attr_dict_text(o.attrs, skip);
      return a.empty() ? a : " " + a;
    };
    auto it = op_table().find(o.name);
    Fmt fmt = it == op_table().end() ? Fmt::Functional : it->second.fmt;
    if (o.name.rfind("nova.", 0) == 0) return out + nova(o);
    if (o.name == "func.return") {
      out += "return";
      if (!o.operands.empty()) out += " " + refs(o.operands) + " : " + types_of(o.operands);
      return out;
    }
    out += o.name;
    switch (fmt) {
      case Fmt::BlockId:
        out += attrs() + " : " + types_of(o.results);
        break;
      case Fmt::Constant: {
        const Attr* v = find_attr(o.attrs, "value");
        out += attrs({"value"});
        out += " " + (v ? v->str() : std::string("<missing>"));
        break;
      }
      case Fmt::Functional:
        out += "(" + refs(o.operands) + ")" + attrs() + " : (" + types_of(o.operands) + ") -> ";
        out += o.results.empty() ? "()" : f.type_of(o.results[0]).str();
        break;
      case Fmt::Arith:
        out += "(" + refs(o.operands) + ")" + attrs() + " : " + types_of(o.operands) + " -> " +
               f.type_of(o.results[0]).str();
        break;
      case Fmt::Permute: {
        const Attr* perm = find_attr(o.attrs, "permutation");
        out += "(" + refs(o.operands) + ") {permutation = " + (perm ? perm->str() : "[]") + "}" +
               attrs({"permutation"}) + " : " + types_of(o.operands) + " -> " +
               f.type_of(o.results[0]).str();
        break;
      }
      case Fmt::Br:
        out += " ^" + o.successors[0];
        if (!o.operands.empty())
          out += "(" + refs(o.operands) + " : " + types_of(o.operands) + ")";
        break;
      case Fmt::CondBr:
        out += " " + refs(o.operands) + ", ^" + o.successors[0] + ", ^" + o.successors[1];
        break;
      case Fmt::Return:
        break;
    }
    return out;
  }

  // Assembly forms of the reference's nova ops that xt-to-nova produces
  // (include/nova/NovaOps.td of the reference; test/xt/to_nova.mlir).
  std::string nova(const Op& o) const {
    auto i64 = [&](const char* name) {
      const Attr* a = find_attr(o.attrs, name);
      return a ? a->i : 0;
    };
    auto flt = [&](const char* name) {
      const Attr* a = find_attr(o.attrs, name);
      return format_float(a ? a->f : 0.0);
    };
    auto list = [&](const char* name) {
      const Attr* a = find_attr(o.attrs, name);
      return a ? a->str() : std::string("[]");
    };
    auto res = [&]() { return o.results.empty() ? std::string("()") : f.type_of(o.results[0]).str(); };
    const std::string& n = o.name;
    std::string out = n;
    if (n == "nova.reduce") {
      out += " " + std::to_string(i64("mode")) + " " + refs(o.operands) + " {axis = " + std::to_string(i64("axis")) +
             " : i64} : " + types_of(o.operands) + " -> " + res();
    } else if (n == "nova.broadcast" || n == "nova.elementwise") {
      out += " " + std::to_string(i64("mode")) + " " + refs(o.operands) + " lhs " + flt("lhs_a") + " " +
             flt("lhs_b") + " rhs " + flt("rhs_a") + " " + flt("rhs_b") + " : " + types_of(o.operands) + " -> " +
             res();
    } else if (n == "nova.scalar") {
      out += " " + std::to_string(i64("mode")) + " " + refs(o.operands) + ", " + flt("rhs") + " : " +
             types_of(o.operands) + " -> " + res();
    } else if (n == "nova.load") {
      out += " " + refs(o.operands) + " " + list("start") + attr_dict_text_pad(o.attrs, {"start"}) + " : " +
             types_of(o.operands) + " -> " + res();
    } else if (n == "nova.store") {
      out += " " + refs(o.operands) + " " + list("start") + attr_dict_text_pad(o.attrs, {"start"}) + " : (" +
             types_of(o.operands) + ") -> ()";
    } else if (n == "nova.conv2d") {
      out += " " + refs(o.operands) + " group " + std::to_string(i64("group")) + " pad " + list("pad") +
             " stride " + list("stride") + " dilation " + list("dilation") + " : " + types_of(o.operands) + " -> " +
             res();
    } else if (n == "nova.permute") {
      out += " " + refs(o.operands) + " " + list("permutation") + " : " + types_of(o.operands) + " -> " + res();
    } else {  // nova.matmul and the unary forms
      out += " " + refs(o.operands) + " : " + types_of(o.operands) + " -> " + res();
    }
    return out;
  }

  static std::string attr_dict_text_pad(const AttrDict& d, const std::vector<std::string>& skip) {
    std::string a = attr_dict_text(d, skip);
    return a.empty() ? a : " " + a;
  }

  std::string func(const std::string& indent) const {
    std::string out = indent + "func.func @" + f.name + "(";
    for (size_t k = 0; k < f.args.size(); ++k)
      out += (k ? ", " : "") + names[f.args[k]] + ": " + f.type_of(f.args[k]).str();
    out += ")";
    if (f.result_types.size() == 1) {
      out += " -> " + f.result_types[0].str();
    } else if (f.result_types.size() > 1) {
      out += " -> (";
      for (size_t k = 0; k < f.result_types.size(); ++k)
        out += (k ? ", " : "") + f.result_types[k].str();
      out += ")";
    }
    std::string a = attr_dict_text(f.attrs);
    if (!a.empty()) out += " attributes " + a;
    if (f.blocks.empty()) return out + "\n";
    out += " {\n";
    for (size_t b = 0; b < f.blocks.size(); ++b) {
      const Block& blk = f.blocks[b];
      if (b > 0 || !blk.label.empty()) {
        out += indent + "^" + blk.label;
        if (!blk.args.empty()) {
          out += "(";
          for (size_t k = 0; k < blk.args.size(); ++k)
            out += (k ? ", " : "") + names[blk.args[k]] + ": " + f.type_of(blk.args[k]).str();
          out += ")";
        }
        out += ":\n";
      }
      for (auto& o : blk.ops) out += indent + "  " + op(o) + "\n";
    }
    out += indent + "}\n";
    return out;
  }
};

}  // namespace

std::string print_module(const Module& m) {
  std::string out = "module";
  std::string a = attr_dict_text(m.attrs);
  if (!a.empty()) out += " attributes " + a;
  out += " {\n";
  for (auto& f : m.funcs) out += Printer(f).func("  ");
  out += "}\n";
  return out;
}

}  // namespace xt
