// `xt-to-nova`: the reference's op-by-op lowering of xt to its NPU dialect
// (lib/xt/XTToNova.cpp), kept for lit parity of xt-opt and for the tile
// offsets and conv halo slices it prints, which this backend's launch planner
// must agree with.  The nova ops are produced and printed, never executed.
//
// Rules (lib/xt/XTToNova.cpp:145-460):
//   add / sub / mul: x * x -> nova.square; a constant splat right operand ->
//     nova.scalar (sub c becomes add -c); a single-element operand otherwise
//     stays xt; equal operand and result types -> nova.elementwise, else
//     nova.broadcast; modes add 1, mul 2, sub 3, unit lhs / rhs affines.
//   reduce_sum / reduce_max -> nova.reduce 0 / 1 with the axis.
//   exp, reciprocal, rsqrt, itof, ftoi -> nova.<name>; permute -> nova.permute.
//   matmul -> nova.matmul with constant scale 1 and bias 0 (1x1 tensors).
//   load / store whose coordinates are all constants -> nova.load / nova.store
//     at element offset coordinate * tile extent per dim.
//   load_conv2d with constant coordinates -> nova.load of the halo slice
//     (computeConv2DSpatialSlice, :110-142) and nova.conv2d with the residual
//     pads [top, left, bottom, right].
// Unused side-effect-free ops are dropped afterwards, as the greedy rewrite
// driver does.
#include <algorithm>
#include <optional>

#include "ir.h"

namespace xt {
namespace {

struct Slice {
  int64_t start, size, pad_before, pad_after;
};

// lib/xt/XTToNova.cpp:110-142
std::optional<Slice> conv_slice(int64_t src_dim, int64_t index, int64_t res_dim, int64_t k, int64_t pad_before,
                                int64_t stride, int64_t dil) {
  if (src_dim < 0 || index < 0 || res_dim < 0 || k <= 0 || pad_before < 0 || stride <= 0 || dil <= 0)
    return std::nullopt;
  const int64_t rf = (res_dim - 1) * stride + dil * (k - 1) + 1;
  const int64_t ideal = index * res_dim * stride - pad_before;
  const int64_t start = std::max<int64_t>(ideal, 0);
  const int64_t pb = start - ideal;
  const int64_t end = std::min<int64_t>(start + (rf - pb), src_dim);
  const int64_t size = end - start;
  const int64_t pa = ideal + rf - end;
  if (size <= 0 || pa < 0) return std::nullopt;
  return Slice{start, size, pb, pa};
}

struct Lowering {
  Func& f;
  std::vector<const Op*> def;  // value -> defining op (in the original list)

  explicit Lowering(Func& fn) : f(fn), def(fn.values.size(), nullptr) {
    for (auto& b : f.blocks)
      for (auto& o : b.ops)
        for (int r : o.results) def[r] = &o;
  }

  std::optional<int64_t> const_int(int v) const {
    const Op* o = v < (int)def.size() ? def[v] : nullptr;
    if (!o || o->name != "arith.constant") return std::nullopt;
    const Attr* a = find_attr(o->attrs, "value");
    if (!a || a->kind != Attr::Int) return std::nullopt;
    return a->i;
  }

  std::optional<double> const_float(int v) const {
    const Op* o = v < (int)def.size() ? def[v] : nullptr;
    if (!o || o->name != "arith.constant") return std::nullopt;
    const Attr* a = find_attr(o->attrs, "value");
    if (!a) return std::nullopt;
    if (a->kind == Attr::Float) return a->f;
    if (a->kind == Attr::DenseSplat && a->splat_is_float) return a->f;
    return std::nullopt;
  }

  // coordinate * extent per dim, when every coordinate is a constant
  std::optional<std::vector<int64_t>> starts(const std::vector<int>& coords, const Type& tile) const {
    if (tile.rank() != static_cast<int>(coords.size())) return std::nullopt;
    std::vector<int64_t> out;
    for (size_t d = 0; d < coords.size(); ++d) {
      auto c = const_int(coords[d]);
      if (!c) return std::nullopt;
      out.push_back(*c * tile.shape[d]);
    }
    return out;
  }

  static Attr int_attr(int64_t v, Elem e) {
    Attr a;
    a.kind = Attr::Int;
    a.i = v;
    a.type = Type::scalar(e);
    return a;
  }
  static Attr f32_attr(double v) {
    Attr a;
    a.kind = Attr::Float;
    a.f = static_cast<float>(v);
    a.type = Type::scalar(Elem::F32);
    return a;
  }
  static Attr list_attr(std::vector<int64_t> v) {
    Attr a;
    a.kind = Attr::List;
    a.ints = std::move(v);
    return a;
  }

  static Op make(const Op& from, const std::string& name) {
    Op o;
    o.name = name;
    o.loc = from.loc;
    return o;
  }

  // Appends the lowering of `o` to `out`; false keeps `o` as it is.
  bool lower(const Op& o, std::vector<Op>& out) {
    const std::string& n = o.name;
    if (n == "xt.add" || n == "xt.sub" || n == "xt.mul") {
      const int mode = n == "xt.add" ? 1 : n == "xt.mul" ? 2 : 3;
      const Type tl = f.type_of(o.operands[0]);
      const Type tr = f.type_of(o.operands[1]);
      const Type tres = f.type_of(o.results[0]);
      if (!tl.is_tensor() || !tr.is_tensor() || !tres.is_tensor()) return false;
      if (mode == 2 && o.operands[0] == o.operands[1]) {
        Op s = make(o, "nova.square");
        s.operands = {o.operands[0]};
        s.results = o.results;
        out.push_back(s);
        return true;
      }
      if (auto c = const_float(o.operands[1])) {
        Op s = make(o, "nova.scalar");
        s.operands = {o.operands[0]};
        s.results = o.results;
        const float rhs = static_cast<float>(*c);
        set_attr(s.attrs, "mode", int_attr(mode == 3 ? 1 : mode, Elem::I32));
        set_attr(s.attrs, "rhs", f32_attr(mode == 3 ? -rhs : rhs));
        out.push_back(s);
        return true;
      }
      if (tl.numel() == 1 || tr.numel() == 1) return false;
      Op s = make(o, tl == tres && tr == tres ? "nova.elementwise" : "nova.broadcast");
      s.operands = o.operands;
      s.results = o.results;
      set_attr(s.attrs, "mode", int_attr(mode, Elem::I32));
      set_attr(s.attrs, "lhs_a", f32_attr(1.0));
      set_attr(s.attrs, "lhs_b", f32_attr(0.0));
      set_attr(s.attrs, "rhs_a", f32_attr(1.0));
      set_attr(s.attrs, "rhs_b", f32_attr(0.0));
      out.push_back(s);
      return true;
    }
    if (n == "xt.reduce_sum" || n == "xt.reduce_max") {
      Op s = make(o, "nova.reduce");
      s.operands = o.operands;
      s.results = o.results;
      set_attr(s.attrs, "mode", int_attr(n == "xt.reduce_sum" ? 0 : 1, Elem::I32));
      if (const Attr* ax = find_attr(o.attrs, "axis")) set_attr(s.attrs, "axis", int_attr(ax->i, Elem::I64));
      out.push_back(s);
      return true;
    }
    static const char* unary[] = {"xt.exp", "xt.reciprocal", "xt.rsqrt", "xt.itof", "xt.ftoi"};
    for (const char* u : unary)
      if (n == u) {
        Op s = make(o, std::string("nova.") + (u + 3));
        s.operands = o.operands;
        s.results = o.results;
        out.push_back(s);
        return true;
      }
    if (n == "xt.permute") {
      const Attr* p = find_attr(o.attrs, "permutation");
      if (!p) return false;
      Op s = make(o, "nova.permute");
      s.operands = o.operands;
      s.results = o.results;
      set_attr(s.attrs, "permutation", list_attr(p->ints));
      out.push_back(s);
      return true;
    }
    if (n == "xt.matmul") {
      int consts[2];
      for (int k = 0; k < 2; ++k) {
        Op c = make(o, "arith.constant");
        Attr v;
        v.kind = Attr::DenseSplat;
        v.splat_is_float = true;
        v.f = k == 0 ? 1.0 : 0.0;
        v.type = Type::tensor(Elem::F32, {1, 1});
        set_attr(c.attrs, "value", v);
        consts[k] = f.add_value(v.type);
        c.results = {consts[k]};
        out.push_back(c);
      }
      Op s = make(o, "nova.matmul");
      s.operands = {o.operands[0], o.operands[1], consts[0], consts[1]};
      s.results = o.results;
      out.push_back(s);
      return true;
    }
    if (n == "xt.load") {
      std::vector<int> coords(o.operands.begin() + 1, o.operands.end());
      auto st = starts(coords, f.type_of(o.results[0]));
      if (!st) return false;
      Op s = make(o, "nova.load");
      s.operands = {o.operands[0]};
      s.results = o.results;
      set_attr(s.attrs, "start", list_attr(*st));
      if (const Attr* sh = find_attr(o.attrs, "shared")) set_attr(s.attrs, "shared", *sh);
      out.push_back(s);
      return true;
    }
    if (n == "xt.store") {
      std::vector<int> coords(o.operands.begin() + 2, o.operands.end());
      auto st = starts(coords, f.type_of(o.operands[0]));
      if (!st) return false;
      Op s = make(o, "nova.store");
      s.operands = {o.operands[0], o.operands[1]};
      set_attr(s.attrs, "start", list_attr(*st));
      out.push_back(s);
      return true;
    }
    if (n == "xt.load_conv2d") {
      // copies: add_value below may grow the value table
      const Type src = f.type_of(o.operands[0]);
      const Type flt = f.type_of(o.operands[1]);
      const Type res = f.type_of(o.results[0]);
      if (src.rank() != 4 || flt.rank() != 4 || res.rank() != 4) return false;
      int64_t idx[4];
      for (int d = 0; d < 4; ++d) {
        auto c = const_int(o.operands[2 + d]);
        if (!c) return false;
        idx[d] = *c;
      }
      const Attr* pad = find_attr(o.attrs, "pad");
      const Attr* stride = find_attr(o.attrs, "stride");
      const Attr* dil = find_attr(o.attrs, "dilation");
      if (!pad || !stride || !dil || pad->ints.size() != 4 || stride->ints.size() != 2 || dil->ints.size() != 2)
        return false;
      auto hs = conv_slice(src.shape[1], idx[1], res.shape[1], flt.shape[0], pad->ints[0], stride->ints[0],
                           dil->ints[0]);
      auto ws = conv_slice(src.shape[2], idx[2], res.shape[2], flt.shape[1], pad->ints[1], stride->ints[1],
                           dil->ints[1]);
      if (!hs || !ws) return false;
      const int64_t cin = flt.shape[2];
      if (cin <= 0 || res.shape[3] != flt.shape[3]) return false;
      Op ld = make(o, "nova.load");
      ld.operands = {o.operands[0]};
      const Type halo = Type::tensor(src.elem, {res.shape[0], hs->size, ws->size, cin});
      ld.results = {f.add_value(halo)};
      set_attr(ld.attrs, "start", list_attr({idx[0] * res.shape[0], hs->start, ws->start, idx[3] * cin}));
      out.push_back(ld);
      Op cv = make(o, "nova.conv2d");
      cv.operands = {ld.results[0], o.operands[1]};
      cv.results = o.results;
      set_attr(cv.attrs, "pad", list_attr({hs->pad_before, ws->pad_before, hs->pad_after, ws->pad_after}));
      set_attr(cv.attrs, "stride", list_attr(stride->ints));
      set_attr(cv.attrs, "dilation", list_attr(dil->ints));
      const Attr* g = find_attr(o.attrs, "group");
      set_attr(cv.attrs, "group", int_attr(g ? g->i : 1, Elem::I64));
      out.push_back(cv);
      return true;
    }
    return false;
  }
};

bool side_effect_free(const std::string& n) {
  return n == "arith.constant" || n == "xt.get_tile_block_id" || n == "nova.load" ||
         (n.rfind("nova.", 0) == 0 && n != "nova.store") || is_pure_op(n);
}

}  // namespace

bool pass_xt_to_nova(Module& m, Diag& diag) {
  (void)diag;
  for (Func& f : m.funcs) {
    Lowering low(f);
    for (Block& b : f.blocks) {
      std::vector<Op> out;
      for (const Op& o : b.ops)
        if (!low.lower(o, out)) out.push_back(o);
      b.ops = std::move(out);
    }
    // drop unused side-effect-free ops until none is left
    for (bool changed = true; changed;) {
      changed = false;
      std::vector<int> uses(f.values.size(), 0);
      for (auto& b : f.blocks)
        for (auto& o : b.ops)
          for (int v : o.operands) uses[v]++;
      for (auto& b : f.blocks) {
        std::vector<Op> keep;
        for (auto& o : b.ops) {
          bool dead = !o.results.empty() && side_effect_free(o.name);
          for (int r : o.results) dead = dead && uses[r] == 0;
          if (dead) changed = true;
          else keep.push_back(o);
        }
        b.ops = std::move(keep);
      }
    }
    for (size_t bi = 0; bi < f.blocks.size(); ++bi)
      for (size_t k = 0; k < f.blocks[bi].ops.size(); ++k) {
        const Op& o = f.blocks[bi].ops[k];
        for (size_t r = 0; r < o.results.size(); ++r) {
          Value& v = f.values[o.results[r]];
          v.def_op = static_cast<int>(k);
          v.def_block = static_cast<int>(bi);
          v.result_no = static_cast<int>(r);
        }
      }
  }
  return true;
}

}  // namespace xt
