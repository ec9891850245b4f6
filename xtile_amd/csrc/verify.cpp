// Verifier for the `xt` IR.  Each rule and its diagnostic text restates the
// reference verifiers so that error behaviour is a drop-in:
//   xt.grid attribute                lib/xt/XTDialect.cpp:18-36
//   load / store memref-tensor rules lib/xt/XTOps.cpp:14-41,92-102
//   load_conv2d                      lib/xt/XTOps.cpp:43-90
//   broadcast binary ops             lib/xt/XTOps.cpp:104-145
//   unary / cast ops                 lib/xt/XTOps.cpp:147-216
//   matmul / mma                     lib/xt/XTOps.cpp:218-272
//   reductions                       lib/xt/XTOps.cpp:274-307
//   reshape / transpose / permute    lib/xt/XTOps.cpp:309-397
// Extension (not in the reference): matmul and load_conv2d also accept
// f16 x f16 and bf16 x bf16 inputs with an f32 result.
#include <algorithm>

#include "ir.h"

namespace xt {
namespace {

struct Verifier {
  const Module& m;
  Diag& diag;
  bool ok = true;

  bool fail(Loc l, const std::string& op, const std::string& msg) {
    diag.error(m.source_name, l, "'" + op + "' op " + msg);
    ok = false;
    return false;
  }

  bool verify_grid_attr(const AttrDict& attrs, Loc l, bool on_func, const std::string& opname) {
    const Attr* g = find_attr(attrs, "xt.grid");
    if (!g) return true;
    if (!on_func) return fail(l, opname, "xt.grid is only valid on func.func operations");
    if (g->kind != Attr::DenseArray || g->type.elem != Elem::I32)
      return fail(l, opname, "xt.grid must be a dense i32 array attribute");
    if (g->ints.size() != 3) return fail(l, opname, "xt.grid must have exactly 3 entries");
    for (int64_t d : g->ints)
      if (d <= 0) return fail(l, opname, "xt.grid entries must be positive");
    return true;
  }

  bool coord_type_ok(const Type& t) {
    return t.is_scalar() && (t.elem == Elem::I32 || t.elem == Elem::Index);
  }

  bool memref_tensor(const Op& o, const Type& mem, const Type& ten) {
    if (!mem.is_memref()) return fail(o.loc, o.name, "requires a ranked memref operand");
    if (!ten.is_tensor()) return fail(o.loc, o.name, "requires a statically shaped tensor");
    if (mem.rank() != ten.rank()) return fail(o.loc, o.name, "memref rank must match tensor rank");
    if (mem.elem != ten.elem)
      return fail(o.loc, o.name, "requires matching memref/tensor element types");
    return true;
  }

  const Attr* need_attr(const Op& o, const char* name) {
    const Attr* a = find_attr(o.attrs, name);
    if (!a) fail(o.loc, o.name, std::string("requires attribute '") + name + "'");
    return a;
  }

  bool verify_op(const Func& f, const Op& o) {
    auto T = [&](int v) -> const Type& { return f.type_of(v); };
    const std::string& n = o.name;

    if (n == "xt.get_tile_block_id") {
      for (size_t k = 0; k < o.results.size(); ++k)
        if (T(o.results[k]) != Type::scalar(Elem::I32))
          return fail(o.loc, n, "result #" + std::to_string(k) +
                                    " must be 32-bit signless integer, but got '" +
                                    T(o.results[k]).str() + "'");
      return true;
    }
    if (n == "arith.constant") {
      const Attr* v = find_attr(o.attrs, "value");
      if (!v) return fail(o.loc, n, "requires attribute 'value'");
      return true;
    }
    if (n == "xt.load") {
      const Type& res = T(o.results[0]);
      if (!res.is_tensor()) return fail(o.loc, n, "requires a ranked tensor result");
      size_t ncoords = o.operands.size() - 1;
      for (size_t k = 1; k < o.operands.size(); ++k)
        if (!coord_type_ok(T(o.operands[k])))
          return fail(o.loc, n, "operand #" + std::to_string(k) +
                                    " must be 32-bit signless integer or index");
      if (ncoords == 0) return fail(o.loc, n, "requires at least one coordinate");
      if (const Attr* sh = find_attr(o.attrs, "shared")) {
        if (sh->kind != Attr::Int || sh->i < 0 || sh->i > 2)
          return fail(o.loc, n, "shared attribute must be 0, 1, or 2");
      }
      if (static_cast<int>(ncoords) != res.rank())
        return fail(o.loc, n, "coordinate count must match tensor rank");
      return memref_tensor(o, T(o.operands[0]), res);
    }
    if (n == "xt.store") {
      const Type& val = T(o.operands[0]);
      if (!val.is_tensor()) return fail(o.loc, n, "requires a ranked tensor operand");
      size_t ncoords = o.operands.size() - 2;
      for (size_t k = 2; k < o.operands.size(); ++k)
        if (!coord_type_ok(T(o.operands[k])))
          return fail(o.loc, n, "operand #" + std::to_string(k) +
                                    " must be 32-bit signless integer or index");
      if (ncoords == 0) return fail(o.loc, n, "requires at least one coordinate");
      if (static_cast<int>(ncoords) != val.rank())
        return fail(o.loc, n, "coordinate count must match tensor rank");
      return memref_tensor(o, T(o.operands[1]), val);
    }
    if (n == "xt.load_conv2d") {
      const Type& src = T(o.operands[0]);
      const Type& filt = T(o.operands[1]);
      const Type& res = T(o.results[0]);
      for (size_t k = 2; k < 6; ++k)
        if (!coord_type_ok(T(o.operands[k])))
          return fail(o.loc, n, "operand #" + std::to_string(k) +
                                    " must be 32-bit signless integer or index");
      if (!src.is_memref()) return fail(o.loc, n, "requires a ranked memref source operand");
      if (!filt.is_tensor() || !res.is_tensor())
        return fail(o.loc, n, "requires ranked tensor filter operand and result");
      if (src.rank() != 4 || filt.rank() != 4 || res.rank() != 4)
        return fail(o.loc, n, "requires rank-4 source, filter, and result types");
      const Attr* pad = need_attr(o, "pad");
      const Attr* stride = need_attr(o, "stride");
      const Attr* dil = need_attr(o, "dilation");
      if (!pad || !stride || !dil) return false;
      if (pad->kind != Attr::DenseArray || pad->ints.size() != 4)
        return fail(o.loc, n, "pad attribute must have exactly 4 entries");
      if (stride->kind != Attr::DenseArray || stride->ints.size() != 2)
        return fail(o.loc, n, "stride attribute must have exactly 2 entries");
      if (dil->kind != Attr::DenseArray || dil->ints.size() != 2)
        return fail(o.loc, n, "dilation attribute must have exactly 2 entries");
      if (const Attr* g = find_attr(o.attrs, "group"))
        if (g->kind != Attr::Int || g->i <= 0)
          return fail(o.loc, n, "group attribute must be positive");
      for (int64_t v : pad->ints)
        if (v < 0) return fail(o.loc, n, "pad attribute entries must be non-negative");
      for (int64_t v : stride->ints)
        if (v <= 0) return fail(o.loc, n, "stride attribute entries must be positive");
      for (int64_t v : dil->ints)
        if (v <= 0) return fail(o.loc, n, "dilation attribute entries must be positive");
      bool in_ok = src.elem == filt.elem &&
                   (src.elem == Elem::I8 || src.elem == Elem::F16 || src.elem == Elem::BF16);
      if (!in_ok)
        return fail(o.loc, n,
                    "load_conv2d requires i8 source and filter element types (or matching "
                    "f16/bf16 source and filter)");
      if (res.elem != Elem::F32 && res.elem != Elem::BF16)
        return fail(o.loc, n, "load_conv2d requires f32 or bf16 result element type");
      if (src.shape[3] != filt.shape[2])
        return fail(o.loc, n,
                    "load_conv2d requires source and filter channel dimensions to match");
      if (res.shape[3] > filt.shape[3])
        return fail(o.loc, n,
                    "load_conv2d result channel dimension must not exceed filter output channels");
      return true;
    }
    if (n == "xt.add" || n == "xt.sub" || n == "xt.mul") {
      const Type& a = T(o.operands[0]);
      const Type& b = T(o.operands[1]);
      const Type& r = T(o.results[0]);
      if (!a.is_tensor() || !b.is_tensor() || !r.is_tensor())
        return fail(o.loc, n, "requires ranked tensor operands and result");
      if (a.elem != b.elem || a.elem != r.elem)
        return fail(o.loc, n, "requires operand and result element types to match");
      int rank = std::max(a.rank(), b.rank());
      std::vector<int64_t> shape(rank, 1);
      for (int i = 0; i < rank; ++i) {
        int ia = a.rank() - 1 - i, ib = b.rank() - 1 - i;
        int64_t da = ia >= 0 ? a.shape[ia] : 1, db = ib >= 0 ? b.shape[ib] : 1;
        if (da != db && da != 1 && db != 1)
          return fail(o.loc, n, "operands are not broadcast-compatible with result tensor type");
        shape[rank - 1 - i] = std::max(da, db);
      }
      if (shape != r.shape)
        return fail(o.loc, n, "operands are not broadcast-compatible with result tensor type");
      return true;
    }
    if (n == "xt.exp" || n == "xt.cos" || n == "xt.sin" || n == "xt.reciprocal" ||
        n == "xt.rsqrt" || n == "xt.sigmoid" || n == "xt.tanh" || n == "xt.silu") {
      const Type& a = T(o.operands[0]);
      const Type& r = T(o.results[0]);
      if (!a.is_tensor() || !r.is_tensor())
        return fail(o.loc, n, "requires ranked tensor operand and result");
      if (a != r) return fail(o.loc, n, "requires operand and result tensor types to match");
      return true;
    }
    if (n == "xt.itof" || n == "xt.ftoi") {
      const Type& a = T(o.operands[0]);
      const Type& r = T(o.results[0]);
      if (!a.is_tensor() || !r.is_tensor())
        return fail(o.loc, n, "requires ranked tensor operand and result");
      if (a.shape != r.shape)
        return fail(o.loc, n, "requires operand and result tensor shapes to match");
      if (n == "xt.itof") {
        if (!elem_is_int(a.elem) || !elem_is_float(r.elem))
          return fail(o.loc, n, "requires integer input and floating-point result element types");
      } else {
        if (!elem_is_float(a.elem) || !elem_is_int(r.elem))
          return fail(o.loc, n, "requires floating-point input and integer result element types");
      }
      return true;
    }
    if (n == "xt.matmul" || n == "xt.mma") {
      const Type& a = T(o.operands[0]);
      const Type& b = T(o.operands[1]);
      const Type& r = T(o.results[0]);
      if (!a.is_tensor() || !b.is_tensor() || !r.is_tensor())
        return fail(o.loc, n, "requires ranked tensor operands and result");
      if (a.rank() != 2 || b.rank() != 2 || r.rank() != 2)
        return fail(o.loc, n, "requires rank-2 tensors");
      if (a.shape[1] != b.shape[0])
        return fail(o.loc, n, "matmul requires lhs inner dimension to match rhs outer dimension");
      if (r.shape[0] != a.shape[0] || r.shape[1] != b.shape[1])
        return fail(o.loc, n, "result shape must match matmul output shape");
      if (n == "xt.matmul") {
        if (a.elem == b.elem && a.elem == r.elem) return true;
        if (a.elem == Elem::I8 && b.elem == Elem::I8 &&
            (r.elem == Elem::F32 || r.elem == Elem::BF16))
          return true;
        if (a.elem == b.elem && (a.elem == Elem::F16 || a.elem == Elem::BF16) &&
            r.elem == Elem::F32)
          return true;
        return fail(o.loc, n, "requires matching element types or i8 inputs with f32/bf16 result");
      }
      const Type& acc = T(o.operands[2]);
      if (!acc.is_tensor() || acc.rank() != 2)
        return fail(o.loc, n, "requires a rank-2 statically shaped accumulator");
      if (acc != r) return fail(o.loc, n, "accumulator and result tensor types must match");
      if (a.elem != Elem::I8 || b.elem != Elem::I8)
        return fail(o.loc, n, "mma requires i8 input tensors");
      if (acc.elem != Elem::F32 && acc.elem != Elem::BF16)
        return fail(o.loc, n, "mma requires f32 or bf16 accumulator and result tensors");
      return true;
    }
    if (n == "xt.reduce_sum" || n == "xt.reduce_max") {
      const Type& a = T(o.operands[0]);
      const Type& r = T(o.results[0]);
      const Attr* ax = need_attr(o, "axis");
      if (!ax) return false;
      if (!a.is_tensor() || !r.is_tensor())
        return fail(o.loc, n, "requires ranked tensor operand and result");
      if (a.elem != r.elem)
        return fail(o.loc, n, "requires operand and result element types to match");
      if (a.rank() != r.rank()) return fail(o.loc, n, "requires operand and result ranks to match");
      if (a.rank() != 2) return fail(o.loc, n, "reduce currently supports rank-2 tensors only");
      int64_t rank = a.rank(), axis = ax->i;
      if (axis < -rank || axis >= rank) return fail(o.loc, n, "axis must be in range [-rank, rank)");
      if (axis < 0) axis += rank;
      for (int64_t i = 0; i < rank; ++i) {
        int64_t want = i == axis ? 1 : a.shape[i];
        if (r.shape[i] != want)
          return fail(o.loc, n,
                      "reduce result shape must match input shape except for the reduced "
                      "dimension, which must be 1");
      }
      return true;
    }
    if (n == "xt.reshape") {
      const Type& a = T(o.operands[0]);
      const Type& r = T(o.results[0]);
      if (!a.is_tensor() || !r.is_tensor())
        return fail(o.loc, n, "requires ranked tensor operand and result");
      if (a.elem != r.elem)
        return fail(o.loc, n, "requires operand and result element types to match");
      if (a.numel() != r.numel())
        return fail(o.loc, n,
                    "reshape requires operand and result to have the same number of elements");
      return true;
    }
    if (n == "xt.transpose") {
      const Type& a = T(o.operands[0]);
      const Type& r = T(o.results[0]);
      if (!a.is_tensor() || !r.is_tensor())
        return fail(o.loc, n, "requires ranked tensor operand and result");
      if (a.elem != r.elem)
        return fail(o.loc, n, "requires operand and result element types to match");
      if (a.rank() != 3 || r.rank() != 3)
        return fail(o.loc, n, "transpose requires rank-3 operand and result tensors");
      if (a.shape[0] != r.shape[0] || a.shape[1] != r.shape[2] || a.shape[2] != r.shape[1])
        return fail(o.loc, n, "transpose result shape must preserve dim 0 and swap dims 1 and 2");
      return true;
    }
    if (n == "xt.permute") {
      const Type& a = T(o.operands[0]);
      const Type& r = T(o.results[0]);
      if (!a.is_tensor() || !r.is_tensor())
        return fail(o.loc, n, "requires ranked tensor operand and result");
      if (a.elem != r.elem)
        return fail(o.loc, n, "requires operand and result element types to match");
      if (a.rank() != r.rank()) return fail(o.loc, n, "requires operand and result ranks to match");
      const Attr* perm = need_attr(o, "permutation");
      if (!perm) return false;
      int64_t rank = a.rank();
      if (static_cast<int64_t>(perm->ints.size()) != rank)
        return fail(o.loc, n, "permutation attribute length must match tensor rank");
      std::vector<bool> seen(rank, false);
      for (int64_t d : perm->ints) {
        if (d < 0 || d >= rank) return fail(o.loc, n, "permutation entries must be in range [0, rank)");
        if (seen[d])
          return fail(o.loc, n, "permutation attribute must contain each dimension exactly once");
        seen[d] = true;
      }
      for (int64_t i = 0; i < rank; ++i)
        if (r.shape[i] != a.shape[perm->ints[i]])
          return fail(o.loc, n,
                      "permute result shape must match the input shape reordered by permutation");
      return true;
    }
    if (n == "func.return") {
      if (o.operands.size() != f.result_types.size())
        return fail(o.loc, n, "has " + std::to_string(o.operands.size()) +
                                  " operands, but enclosing function (@" + f.name + ") returns " +
                                  std::to_string(f.result_types.size()));
      for (size_t k = 0; k < o.operands.size(); ++k)
        if (T(o.operands[k]) != f.result_types[k])
          return fail(o.loc, n, "type of return operand " + std::to_string(k) + " ('" +
                                    T(o.operands[k]).str() +
                                    "') doesn't match function result type ('" +
                                    f.result_types[k].str() + "') in function @" + f.name);
      return true;
    }
    // nova ops exist only as the output of xt-to-nova (their dialect's
    // verifier is the reference's NPU toolchain)
    if (n.rfind("nova.", 0) == 0) return true;
    if (n == "cf.br" || n == "cf.cond_br") {
      for (auto& succ : o.successors) {
        bool found = false;
        for (auto& b : f.blocks) found |= b.label == succ;
        if (!found) return fail(o.loc, n, "reference to an undefined block '^" + succ + "'");
      }
      return true;
    }
    return fail(o.loc, n, "unknown operation");
  }
};

}  // namespace

bool verify_module(const Module& m, Diag& diag) {
  Verifier v{m, diag};
  v.verify_grid_attr(m.attrs, m.loc, false, "builtin.module");
  for (auto& f : m.funcs) {
    v.verify_grid_attr(f.attrs, f.loc, true, "func.func");
    for (auto& b : f.blocks)
      for (auto& o : b.ops) v.verify_op(f, o);
  }
  return v.ok;
}

}  // namespace xt
