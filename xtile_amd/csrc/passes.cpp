// IR passes: `xt-serialize` and `canonicalize`.
//
// xt-serialize restates lib/xt/XTSerialize.cpp:25-104: the single-block body is
// replicated once per grid point in z -> y -> x order, block ids become i32
// constants, and a load carrying `shared = k` (k > 0) is emitted only for the
// first block of its sharing group; later blocks of the group reuse its value.
// The group key is (load, y or 0 when k == 2, z), i.e. blocks that agree on
// every grid axis >= k share (README.md:206-230).
//
// canonicalize restates the fold patterns of lib/xt/XTOps.cpp:399-449
// (x + 0 -> x, 0 + x -> x, x - 0 -> x for splat-zero dense constants) followed
// by removal of unused side-effect-free ops, which MLIR's canonicalizer does.
#include <map>
#include <tuple>

#include "ir.h"

namespace xt {
namespace {

void reindex(Func& f) {
  for (size_t b = 0; b < f.blocks.size(); ++b)
    for (size_t k = 0; k < f.blocks[b].ops.size(); ++k) {
      const Op& o = f.blocks[b].ops[k];
      for (size_t r = 0; r < o.results.size(); ++r) {
        Value& v = f.values[o.results[r]];
        v.def_op = static_cast<int>(k);
        v.def_block = static_cast<int>(b);
        v.result_no = static_cast<int>(r);
      }
    }
}

Op make_i32_constant(Func& f, int32_t value, Loc loc) {
  Op c;
  c.name = "arith.constant";
  c.loc = loc;
  Attr a;
  a.kind = Attr::Int;
  a.i = value;
  a.type = Type::scalar(Elem::I32);
  set_attr(c.attrs, "value", a);
  c.results.push_back(f.add_value(Type::scalar(Elem::I32)));
  return c;
}

bool serialize_func(Func& f, const std::string& src, Diag& diag) {
  int32_t grid[3];
  auto fail = [&](const std::string& msg) {
    diag.error(src, f.loc, "'func.func' op " + msg);
    return false;
  };
  if (!find_attr(f.attrs, "xt.grid") || !get_grid(f, grid))
    return fail("xt-serialize requires func.func xt.grid attribute");
  if (!f.result_types.empty()) return fail("xt-serialize only supports void functions");
  if (f.blocks.size() != 1) return fail("xt-serialize only supports single-block functions");
  Block& entry = f.blocks[0];
  if (entry.ops.empty() || entry.ops.back().name != "func.return" ||
      !entry.ops.back().operands.empty())
    return fail("xt-serialize only supports void functions");

  std::vector<Op> body(entry.ops.begin(), entry.ops.end() - 1);
  Op ret = entry.ops.back();
  std::vector<Op> out;
  std::map<std::tuple<size_t, int32_t, int32_t>, int> shared_values;

  for (int32_t z = 0; z < grid[2]; ++z)
    for (int32_t y = 0; y < grid[1]; ++y)
      for (int32_t x = 0; x < grid[0]; ++x) {
        std::map<int, int> remap;
        auto mapped = [&](int v) {
          auto it = remap.find(v);
          return it == remap.end() ? v : it->second;
        };
        Op cx = make_i32_constant(f, x, f.loc);
        Op cy = make_i32_constant(f, y, f.loc);
        Op cz = make_i32_constant(f, z, f.loc);
        int ids[3] = {cx.results[0], cy.results[0], cz.results[0]};
        out.push_back(std::move(cx));
        out.push_back(std::move(cy));
        out.push_back(std::move(cz));
        for (size_t k = 0; k < body.size(); ++k) {
          const Op& o = body[k];
          if (o.name == "xt.get_tile_block_id") {
            for (int r = 0; r < 3 && r < static_cast<int>(o.results.size()); ++r)
              remap[o.results[r]] = ids[r];
            continue;
          }
          bool shared_load = false;
          std::tuple<size_t, int32_t, int32_t> key;
          if (o.name == "xt.load") {
            const Attr* sh = find_attr(o.attrs, "shared");
            if (sh && sh->i > 0) {
              shared_load = true;
              key = {k, sh->i == 2 ? 0 : y, z};
              auto it = shared_values.find(key);
              if (it != shared_values.end()) {
                remap[o.results[0]] = it->second;
                continue;
              }
            }
          }
          Op c = o;
          for (int& v : c.operands) v = mapped(v);
          for (int& r : c.results) {
            int fresh = f.add_value(f.type_of(r), f.values[r].hint);
            remap[r] = fresh;
            r = fresh;
          }
          if (shared_load) shared_values[key] = c.results[0];
          out.push_back(std::move(c));
        }
      }
  out.push_back(std::move(ret));
  entry.ops = std::move(out);
  reindex(f);
  return true;
}

bool is_zero_splat(const Func& f, const Block& b, int v) {
  const Value& val = f.values[v];
  if (val.def_op < 0) return false;
  const Op& def = f.blocks[val.def_block].ops[val.def_op];
  (void)b;
  if (def.name != "arith.constant") return false;
  const Attr* a = find_attr(def.attrs, "value");
  if (!a || a->kind != Attr::DenseSplat) return false;
  return a->splat_is_float ? a->f == 0.0 : a->i == 0;
}

void replace_uses(Func& f, int from, int to) {
  for (auto& b : f.blocks)
    for (auto& o : b.ops)
      for (int& v : o.operands)
        if (v == from) v = to;
}

void canonicalize_func(Func& f) {
  bool changed = true;
  while (changed) {
    changed = false;
    reindex(f);
    for (auto& b : f.blocks) {
      for (auto& o : b.ops) {
        if (o.results.empty()) continue;
        int r = o.results[0];
        int repl = -1;
        if (o.name == "xt.add") {
          if (is_zero_splat(f, b, o.operands[0])) repl = o.operands[1];
          else if (is_zero_splat(f, b, o.operands[1])) repl = o.operands[0];
        } else if (o.name == "xt.sub") {
          if (is_zero_splat(f, b, o.operands[1])) repl = o.operands[0];
        }
        if (repl >= 0 && f.type_of(repl) == f.type_of(r)) {
          replace_uses(f, r, repl);
          changed = true;
        }
      }
    }
    // drop unused side-effect-free ops
    std::vector<int> uses(f.values.size(), 0);
    for (auto& b : f.blocks)
      for (auto& o : b.ops)
        for (int v : o.operands) uses[v]++;
    for (auto& b : f.blocks) {
      std::vector<Op> kept;
      for (auto& o : b.ops) {
        bool dead = is_pure_op(o.name) && !o.results.empty();
        for (int r : o.results) dead = dead && uses[r] == 0;
        if (dead) {
          changed = true;
          continue;
        }
        kept.push_back(std::move(o));
      }
      b.ops = std::move(kept);
    }
  }
  reindex(f);
}

}  // namespace

bool pass_xt_serialize(Module& m, Diag& diag) {
  bool ok = true;
  for (auto& f : m.funcs) {
    if (f.blocks.empty()) continue;
    if (!serialize_func(f, m.source_name, diag)) ok = false;
  }
  return ok;
}

bool pass_canonicalize(Module& m, Diag& diag) {
  (void)diag;
  for (auto& f : m.funcs) canonicalize_func(f);
  return true;
}

}  // namespace xt
