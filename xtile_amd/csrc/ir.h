// In-memory `xt` IR: an MLIR-free representation of the textual subset the
// xtile DSL emits (func.func + arith.constant + xt.* ops + func.return, plus
// the cf branch ops the reference's negative tests use).
//
// The op set, operand order and assembly formats follow the reference dialect
// definition (include/xt/XTOps.td:15-170); attribute semantics follow
// lib/xt/XTDialect.cpp:18-36 and lib/xt/XTOps.cpp.  Nothing here depends on
// HIP: the parser, printer, verifier and passes run on any host.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace xt {

enum class Elem : uint8_t { None, F32, F16, BF16, I8, I32, I64, I1, Index };

const char* elem_name(Elem e);
int elem_bytes(Elem e);
bool elem_is_float(Elem e);
bool elem_is_int(Elem e);

struct Type {
  enum Kind : uint8_t { Invalid, Scalar, Tensor, MemRef } kind = Invalid;
  Elem elem = Elem::None;
  std::vector<int64_t> shape;  // tensor / memref only

  static Type scalar(Elem e) { return Type{Scalar, e, {}}; }
  static Type tensor(Elem e, std::vector<int64_t> s) { return Type{Tensor, e, std::move(s)}; }
  static Type memref(Elem e, std::vector<int64_t> s) { return Type{MemRef, e, std::move(s)}; }

  bool is_tensor() const { return kind == Tensor; }
  bool is_memref() const { return kind == MemRef; }
  bool is_scalar() const { return kind == Scalar; }
  int rank() const { return static_cast<int>(shape.size()); }
  int64_t numel() const;
  bool operator==(const Type& o) const {
    return kind == o.kind && elem == o.elem && shape == o.shape;
  }
  bool operator!=(const Type& o) const { return !(*this == o); }
  std::string str() const;
};

struct Attr {
  enum Kind : uint8_t {
    Unit,       // bare name
    Int,        // 1 : i64   (type held in `type`)
    Float,      // 1.0 : f32
    Bool,       // true / false
    DenseArray, // array<i32: 1, 2>  (elem in type.elem)
    List,       // [2, 0, 1]
    DenseSplat, // dense<0.0> : tensor<..>
    String,     // "text"
  } kind = Unit;
  int64_t i = 0;
  double f = 0.0;
  bool splat_is_float = false;
  std::vector<int64_t> ints;
  Type type;
  std::string s;

  std::string str() const;
};

using AttrDict = std::vector<std::pair<std::string, Attr>>;  // kept sorted by name

const Attr* find_attr(const AttrDict& d, const std::string& name);
void set_attr(AttrDict& d, const std::string& name, Attr a);
void erase_attr(AttrDict& d, const std::string& name);

struct Loc {
  int line = 0;
  int col = 0;
};

struct Value {
  Type type;
  int def_op = -1;      // index into the owning block's op list (-1: block argument)
  int def_block = 0;
  int result_no = 0;
  std::string hint;     // name used in the source text (diagnostics only)
};

struct Op {
  std::string name;
  std::vector<int> operands;  // value ids
  std::vector<int> results;   // value ids
  AttrDict attrs;
  std::vector<std::string> successors;  // block labels (cf ops)
  Loc loc;
};

struct Block {
  std::string label;     // empty for the entry block
  std::vector<int> args; // value ids
  std::vector<Op> ops;
};

struct Func {
  std::string name;
  std::vector<int> args;           // value ids
  std::vector<Type> result_types;
  AttrDict attrs;
  std::vector<Block> blocks;
  std::vector<Value> values;       // value table owned by the function
  Loc loc;

  int add_value(Type t, std::string hint = {}) {
    Value v;
    v.type = std::move(t);
    v.hint = std::move(hint);
    values.push_back(std::move(v));
    return static_cast<int>(values.size()) - 1;
  }
  const Type& type_of(int v) const { return values[v].type; }
};

struct Module {
  AttrDict attrs;
  std::vector<Func> funcs;
  Loc loc;
  std::string source_name = "<input>";
};

// Diagnostics collected while parsing / verifying / running passes.  Each
// entry is already formatted as `<source>:<line>:<col>: error: <message>`.
struct Diag {
  std::vector<std::string> lines;
  void error(const std::string& src, Loc loc, const std::string& msg);
  bool empty() const { return lines.empty(); }
  std::string joined() const;
};

// parse + verify (like MLIR's parseSourceString, which verifies after parsing)
std::unique_ptr<Module> parse_module(const std::string& text, Diag& diag,
                                     const std::string& source_name = "<input>");
bool verify_module(const Module& m, Diag& diag);
std::string print_module(const Module& m);

// Passes.  Each mutates the module in place and returns false on failure.
bool pass_xt_serialize(Module& m, Diag& diag);
bool pass_canonicalize(Module& m, Diag& diag);
// lib/xt/XTToNova.cpp restated: xt ops -> the reference's nova ops (printing only)
bool pass_xt_to_nova(Module& m, Diag& diag);

// Helpers shared by passes and the launch planner.
const Func* find_func(const Module& m, const std::string& name);
bool is_pure_op(const std::string& name);
bool get_grid(const Func& f, int32_t grid[3]);

// Split `--split-input-file` style chunks ("// -----" separators).
std::vector<std::string> split_input_chunks(const std::string& text);

}  // namespace xt
