// Tile-program matcher.  See plan.h for the addressing model.
//
// Recognised programs (each maps onto one hand-written gfx950 kernel family):
//   EwBinary   store(op(load A, load B))             op in {add, sub, mul}, f32
//              (kernels/add.py:6-13; xtile/dsl.py:321-325,351-352)
//   RowSoftmax load -> reduce_max -> sub -> exp -> reduce_sum -> reciprocal
//              -> mul -> store, reductions over axis 1
//              (kernels/softmax.py:10-19; test/python/dsl_convert.py:25-40)
//   Gemm       store([ftoi]((matmul(load A, load B) [* load S]) [+ load Bias]))
//              f16/bf16/i8 in, f32 or i8 out (kernels/matmul.py:6-19)
//   Conv2d     store(load_conv2d(S, load F))         i8/f16/bf16 in, f32/bf16 out
//              (kernels/conv2d.py:10-37; conv slice math lib/xt/XTToNova.cpp:110-142)
#include "plan.h"

#include <algorithm>
#include <map>
#include <set>
#include <cstdlib>
#include <sstream>

namespace xt {
namespace {

struct Analysis {
  const Func& f;
  const int32_t* grid;
  std::map<int, Coord> coords;          // i32 value -> block id axis / constant
  std::vector<const Op*> compute;       // everything except bid / constants / return
  std::vector<int> uses;
  std::map<int, const Op*> def;

  Analysis(const Func& fn, const int32_t* g) : f(fn), grid(g), uses(fn.values.size(), 0) {
    for (auto& o : f.blocks[0].ops) {
      for (int v : o.operands) uses[v]++;
      for (int r : o.results) def[r] = &o;
      if (o.name == "xt.get_tile_block_id") {
        for (int k = 0; k < 3; ++k) coords[o.results[k]] = Coord{k, 0};
      } else if (o.name == "arith.constant") {
        const Attr* v = find_attr(o.attrs, "value");
        if (v && v->kind == Attr::Int) coords[o.results[0]] = Coord{-1, v->i};
      } else if (o.name != "func.return") {
        compute.push_back(&o);
      }
    }
  }

  int arg_index(int value) const {
    for (size_t k = 0; k < f.args.size(); ++k)
      if (f.args[k] == value) return static_cast<int>(k);
    return -1;
  }
};

bool coord_of(const Analysis& an, int v, int shared, Coord& out, std::string& err) {
  auto it = an.coords.find(v);
  if (it == an.coords.end()) {
    err = "tile coordinates must be xt.get_tile_block_id results or integer constants";
    return false;
  }
  out = it->second;
  if (out.axis >= 0 && out.axis < shared) out = Coord{-1, 0};  // sharing-group leader
  return true;
}

// Element strides of a row-major memref.
std::vector<int64_t> strides_of(const std::vector<int64_t>& shape) {
  std::vector<int64_t> s(shape.size(), 1);
  for (int d = static_cast<int>(shape.size()) - 2; d >= 0; --d) s[d] = s[d + 1] * shape[d + 1];
  return s;
}

// Shared by loads and stores: coordinates -> affine tile origin, bounds check.
bool tile_origin(const Analysis& an, const std::vector<int>& coord_values, int shared,
                 const std::vector<int64_t>& tile, const std::vector<int64_t>& mem,
                 const std::string& what, TileAddr& addr, std::vector<Coord>* coords_out,
                 std::string& err) {
  std::vector<int64_t> st = strides_of(mem);
  addr = TileAddr{};
  for (size_t d = 0; d < tile.size(); ++d) {
    Coord c;
    if (!coord_of(an, coord_values[d], shared, c, err)) return false;
    if (coords_out) coords_out->push_back(c);
    int64_t lo = c.axis < 0 ? c.value : 0;
    int64_t hi = c.axis < 0 ? c.value : an.grid[c.axis] - 1;
    if (lo < 0 || (hi + 1) * tile[d] > mem[d]) {
      std::ostringstream os;
      os << what << ": tile coordinate range [" << lo << ", " << hi << "] x " << tile[d]
         << " exceeds extent " << mem[d] << " of dim " << d;
      err = os.str();
      return false;
    }
    int64_t step = tile[d] * st[d];
    if (c.axis < 0) addr.c0 += c.value * step;
    else if (c.axis == 0) addr.sx += step;
    else if (c.axis == 1) addr.sy += step;
    else addr.sz += step;
  }
  return true;
}

// View a tile of `tile` within memref `mem` as rows x cols with row pitch ld.
bool as_2d(const std::vector<int64_t>& tile, const std::vector<int64_t>& mem, Access2D& a,
           bool merge_rows, std::string& err) {
  int r = static_cast<int>(tile.size());
  std::vector<int64_t> st = strides_of(mem);
  if (!merge_rows) {
    // keep the tile's own rows: rank 1 is one row, rank 2 is rows x cols
    if (r > 2) {
      err = "tile must be rank 1 or 2";
      return false;
    }
    a.rows = r == 1 ? 1 : tile[0];
    a.cols = tile[r - 1];
    a.ld = mem[r - 1];
    return true;
  }
  int64_t cols = tile[r - 1];
  int d = r - 2;
  for (; d >= 0; --d) {
    if (tile[d + 1] != mem[d + 1]) break;
    cols *= tile[d];
  }
  // dims 0..d remain: at most one of them may have extent > 1
  int64_t rows = 1, ld = cols;
  int outer = -1;
  for (int k = 0; k <= d; ++k)
    if (tile[k] > 1) {
      if (outer >= 0) {
        err = "tile is not a 2-D strided block of its memref";
        return false;
      }
      outer = k;
    }
  if (outer >= 0) {
    rows = tile[outer];
    ld = st[outer];
    // the run below `outer` must be contiguous: cols == product of inner tile dims
    int64_t inner = 1;
    for (int k = outer + 1; k < r; ++k) inner *= tile[k];
    if (inner != cols) {
      err = "tile is not a 2-D strided block of its memref";
      return false;
    }
  }
  a.rows = rows;
  a.cols = cols;
  a.ld = ld;
  return true;
}

// merge_rows: elementwise programs may treat full-width rows as one long row.
bool access_of(const Analysis& an, const Op& o, Access2D& a, std::string& err,
               bool merge_rows = false) {
  bool is_load = o.name == "xt.load";
  int mem_v = is_load ? o.operands[0] : o.operands[1];
  const Type& mem = an.f.type_of(mem_v);
  const Type& ten = is_load ? an.f.type_of(o.results[0]) : an.f.type_of(o.operands[0]);
  a.arg = an.arg_index(mem_v);
  if (a.arg < 0) {
    err = o.name + " must access a function argument";
    return false;
  }
  a.elem = mem.elem;
  a.shared = 0;
  if (is_load)
    if (const Attr* sh = find_attr(o.attrs, "shared")) a.shared = static_cast<int>(sh->i);
  std::vector<int> cv(o.operands.begin() + (is_load ? 1 : 2), o.operands.end());
  std::string what = o.name + " of argument #" + std::to_string(a.arg);
  if (!tile_origin(an, cv, a.shared, ten.shape, mem.shape, what, a.addr, nullptr, err))
    return false;
  return as_2d(ten.shape, mem.shape, a, merge_rows, err);
}

const Op* only(const Analysis& an, const char* name, int& count) {
  const Op* found = nullptr;
  count = 0;
  for (const Op* o : an.compute)
    if (o->name == name) {
      found = o;
      ++count;
    }
  return found;
}

int count_ops(const Analysis& an) { return static_cast<int>(an.compute.size()); }

const Op* def_of(const Analysis& an, int v) {
  auto it = an.def.find(v);
  return it == an.def.end() ? nullptr : it->second;
}

// -- Block independence --------------------------------------------------------

// The reference's xt-serialize runs the Blocks one after another in z -> y ->
// x order (lib/xt/XTSerialize.cpp:68-104), so where two Blocks store to one
// tile the later one's values remain, and a Block that loads a tile another
// Block stores sees it before or after that store depending on the order.
// Every kernel here runs Blocks concurrently and in any order.  The two agree
// exactly when no two Blocks store different values to one tile and no Block
// loads a tile that another Block stores; programs outside that are refused
// (README.md:85-89 leaves multi-writer results undefined).
bool check_independent(const Analysis& an, std::string& err) {
  unsigned live = 0;  // grid axes with more than one Block
  for (int k = 0; k < 3; ++k)
    if (an.grid[k] > 1) live |= 1u << k;
  auto axes_of = [&](const Op* o, size_t first, size_t last, int shared, unsigned& out) {
    out = 0;
    for (size_t i = first; i < last && i < o->operands.size(); ++i) {
      Coord c;
      if (!coord_of(an, o->operands[i], shared, c, err)) return false;
      if (c.axis >= 0) out |= 1u << c.axis;
    }
    return true;
  };
  std::map<int, unsigned> dep;  // tensor value -> grid axes its elements vary along
  std::map<int, std::vector<const Op*>> loads, stores;  // by memref value
  for (const Op* o : an.compute) {
    unsigned d = 0;
    if (o->name == "xt.load") {
      int shared = 0;
      if (const Attr* sh = find_attr(o->attrs, "shared")) shared = static_cast<int>(sh->i);
      if (!axes_of(o, 1, o->operands.size(), shared, d)) return false;
      loads[o->operands[0]].push_back(o);
    } else if (o->name == "xt.load_conv2d") {
      if (!axes_of(o, 2, o->operands.size(), 0, d)) return false;
      if (o->operands.size() > 1 && dep.count(o->operands[1])) d |= dep[o->operands[1]];
      loads[o->operands[0]].push_back(o);
    } else if (o->name == "xt.store") {
      unsigned at = 0;
      if (!axes_of(o, 2, o->operands.size(), 0, at)) return false;
      const unsigned vd = (dep.count(o->operands[0]) ? dep[o->operands[0]] : 0) & live & ~at;
      if (vd) {
        const int ax = __builtin_ctz(vd);
        err = "Blocks along grid axis " + std::to_string(ax) + " store different values to the same tile of " +
              "memref argument #" + std::to_string(an.arg_index(o->operands[1])) +
              "; the reference's serial Block order keeps the last one's, which concurrent Blocks do not "
              "reproduce (give the store a coordinate on that axis)";
        return false;
      }
      stores[o->operands[1]].push_back(o);
      continue;
    } else {
      for (int v : o->operands)
        if (dep.count(v)) d |= dep[v];
    }
    for (int r : o->results) dep[r] = d;
  }
  // a memref that is stored and also loaded (or stored twice): every access
  // must be the same tile at the same coordinates, so a Block only ever reads
  // and writes its own tile
  for (const auto& kv : stores) {
    std::vector<const Op*> acc = kv.second;
    auto it = loads.find(kv.first);
    if (it != loads.end()) acc.insert(acc.end(), it->second.begin(), it->second.end());
    if (acc.size() < 2) continue;
    auto key = [&](const Op* o) {
      std::vector<int64_t> k;
      const bool st = o->name == "xt.store";
      const Type& t = st ? an.f.type_of(o->operands[0]) : an.f.type_of(o->results[0]);
      k.insert(k.end(), t.shape.begin(), t.shape.end());
      k.push_back(o->name == "xt.load_conv2d" ? 1 : 0);
      const size_t first = st ? 2 : (o->name == "xt.load_conv2d" ? 2 : 1);
      int shared = 0;
      if (const Attr* sh = find_attr(o->attrs, "shared")) shared = static_cast<int>(sh->i);
      for (size_t i = first; i < o->operands.size(); ++i) {
        Coord c;
        std::string e;
        coord_of(an, o->operands[i], shared, c, e);
        k.push_back(c.axis);
        k.push_back(c.value);
      }
      return k;
    };
    const auto k0 = key(acc[0]);
    for (size_t i = 1; i < acc.size(); ++i)
      if (key(acc[i]) != k0) {
        err = "memref argument #" + std::to_string(an.arg_index(kv.first)) +
              " is stored and also accessed at another tile; concurrent Blocks would read or overwrite "
              "tiles other Blocks store, which the reference's serial Block order defines and this "
              "backend does not reproduce";
        return false;
      }
  }
  return true;
}

// -- EwBinary ----------------------------------------------------------------

// Element (Block x, y, z; row r, column c) of an access sits at
// c0 + c + r*ld + x*sx + y*sy + z*sz: a mixed-radix number whose digits are the
// column, the row and the grid axes of extent > 1.  When those (stride,
// extent) pairs, sorted by stride, start at stride 1 and every stride is the
// product of the extents before it, the map is a bijection onto
// [c0, c0 + product of the extents): the tiles cover one contiguous run,
// each element once.  Returns the run's length, or 0.
int64_t contiguous_run(const Plan& p, const Access2D& a) {
  std::vector<std::pair<int64_t, int64_t>> d;  // (stride, extent)
  if (a.cols < 1 || a.rows < 1) return 0;
  d.push_back({1, a.cols});
  if (a.rows > 1) d.push_back({a.ld, a.rows});
  const int64_t st[3] = {a.addr.sx, a.addr.sy, a.addr.sz};
  for (int ax = 0; ax < 3; ++ax)
    if (p.grid[ax] > 1) {
      if (st[ax] <= 0) return 0;
      d.push_back({st[ax], p.grid[ax]});
    }
  std::sort(d.begin(), d.end());
  int64_t next = 1;
  for (const auto& e : d) {
    if (e.first != next) return 0;
    if (next > (int64_t(1) << 40) / e.second) return 0;
    next *= e.second;
  }
  return next;
}

bool match_ew(const Analysis& an, Plan& p, std::string& err) {
  int nstore = 0;
  const Op* st = only(an, "xt.store", nstore);
  if (nstore != 1 || !st) return false;
  const Op* bin = def_of(an, st->operands[0]);
  if (!bin || (bin->name != "xt.add" && bin->name != "xt.sub" && bin->name != "xt.mul"))
    return false;
  const Op* la = def_of(an, bin->operands[0]);
  const Op* lb = def_of(an, bin->operands[1]);
  if (!la || !lb || la->name != "xt.load" || lb->name != "xt.load") return false;
  int expected = la == lb ? 3 : 4;
  if (count_ops(an) != expected) return false;
  const Type& ta = an.f.type_of(la->results[0]);
  const Type& tb = an.f.type_of(lb->results[0]);
  if (ta != tb || ta.elem != Elem::F32) return false;  // broadcast or non-f32: the interpreter
  if (!access_of(an, *la, p.a, err, true) || !access_of(an, *lb, p.b, err, true) ||
      !access_of(an, *st, p.c, err, true))
    return false;
  auto same_view = [&]() {
    return p.a.rows == p.c.rows && p.a.cols == p.c.cols && p.b.rows == p.c.rows &&
           p.b.cols == p.c.cols;
  };
  if (!same_view()) {
    // the three memrefs disagree on which rows are full-width: keep tile rows
    if (ta.rank() > 2) {
      err = "elementwise tiles of rank > 2 must be contiguous runs in every operand";
      return false;
    }
    if (!access_of(an, *la, p.a, err) || !access_of(an, *lb, p.b, err) ||
        !access_of(an, *st, p.c, err))
      return false;
  }
  p.kind = PlanKind::EwBinary;
  p.ew_op = bin->name == "xt.add" ? EwOp::Add : bin->name == "xt.sub" ? EwOp::Sub : EwOp::Mul;
  // strides of grid axes of extent 1 never move a tile
  auto same_walk = [&](const Access2D& x) {
    return (p.grid[0] == 1 || x.addr.sx == p.c.addr.sx) && (p.grid[1] == 1 || x.addr.sy == p.c.addr.sy) &&
           (p.grid[2] == 1 || x.addr.sz == p.c.addr.sz) && x.ld == p.c.ld && x.rows == p.c.rows &&
           x.cols == p.c.cols;
  };
  p.ew_flat = same_walk(p.a) && same_walk(p.b) ? contiguous_run(p, p.c) : 0;
  double blocks = double(p.grid[0]) * p.grid[1] * p.grid[2];
  double tile_bytes = double(ta.numel()) * 4;
  p.algo_bytes = blocks * tile_bytes * (la == lb ? 2 : 3);
  return true;
}

// -- RowSoftmax ----------------------------------------------------------------

bool axis_is(const Op* o, int64_t axis) {
  const Attr* a = find_attr(o->attrs, "axis");
  return a && (a->i == axis || a->i == axis - 2);
}

bool match_softmax(const Analysis& an, Plan& p, std::string& err) {
  if (count_ops(an) != 8) return false;
  int n;
  const Op* st = only(an, "xt.store", n);
  if (n != 1) return false;
  const Op* mul = def_of(an, st->operands[0]);
  if (!mul || mul->name != "xt.mul") return false;
  const Op* e = def_of(an, mul->operands[0]);
  const Op* inv = def_of(an, mul->operands[1]);
  if (e && e->name == "xt.reciprocal") std::swap(e, inv);
  if (!e || !inv || e->name != "xt.exp" || inv->name != "xt.reciprocal") return false;
  const Op* rsum = def_of(an, inv->operands[0]);
  if (!rsum || rsum->name != "xt.reduce_sum" || rsum->operands[0] != e->results[0] ||
      !axis_is(rsum, 1))
    return false;
  const Op* sub = def_of(an, e->operands[0]);
  if (!sub || sub->name != "xt.sub") return false;
  const Op* ld = def_of(an, sub->operands[0]);
  const Op* rmax = def_of(an, sub->operands[1]);
  if (!ld || !rmax || ld->name != "xt.load" || rmax->name != "xt.reduce_max" ||
      rmax->operands[0] != ld->results[0] || !axis_is(rmax, 1))
    return false;
  const Type& t = an.f.type_of(ld->results[0]);
  // other shapes and types run on the tile interpreter
  if (t.elem != Elem::F32 || t.rank() != 2 || t.shape[1] > 8192) return false;
  if (!access_of(an, *ld, p.a, err) || !access_of(an, *st, p.c, err)) return false;
  // rows above 2048 floats are held as float4 vectors: columns, pitches and
  // tile origins must be multiples of 4 (the buffers' 16-byte alignment is
  // checked at launch)
  auto vec4 = [](const Access2D& a) {
    return a.cols % 4 == 0 && a.ld % 4 == 0 && a.addr.c0 % 4 == 0 && a.addr.sx % 4 == 0 && a.addr.sy % 4 == 0 &&
           a.addr.sz % 4 == 0;
  };
  if (t.shape[1] > 2048 && !(vec4(p.a) && vec4(p.c))) return false;
  p.kind = PlanKind::RowSoftmax;
  double blocks = double(p.grid[0]) * p.grid[1] * p.grid[2];
  p.algo_bytes = blocks * double(t.numel()) * 8;
  return true;
}

// -- Gemm ----------------------------------------------------------------------

// store([ftoi](([matmul * load S] | matmul) [+ load Bias])): the epilogue of
// kernels/matmul.py:15-17, every part optional.  Scale and bias are (1, TN)
// f32 row tiles broadcast over the rows (xtile/dsl.py:658-679,754-759).
bool epilogue_row(const Analysis& an, const Op* bin, const Type& tile, Access2D& acc, std::string& err) {
  const Op* ld = def_of(an, bin->operands[1]);
  if (!ld || ld->name != "xt.load") {
    err = "matmul epilogue operands must be loaded (1, N) f32 tiles";
    return false;
  }
  const Type& t = an.f.type_of(ld->results[0]);
  if (t.elem != Elem::F32 || t.rank() != 2 || t.shape[0] != 1 || t.shape[1] != tile.shape[1]) {
    err = "matmul epilogue operands must be (1, N) f32 tiles matching the result columns";
    return false;
  }
  return access_of(an, *ld, acc, err);
}

bool match_gemm(const Analysis& an, Plan& p, std::string& err) {
  int nmm, nst;
  const Op* mm = only(an, "xt.matmul", nmm);
  const Op* st = only(an, "xt.store", nst);
  if (nmm != 1 || nst != 1) {
    if (nmm >= 1) err = "matmul programs must hold one matmul and one store";
    return false;
  }
  const Type& tc = an.f.type_of(mm->results[0]);
  p.gemm_scale = p.gemm_bias = p.gemm_ftoi = false;
  int expected = 4;
  const Op* o = def_of(an, st->operands[0]);
  if (o && o->name == "xt.ftoi") {
    p.gemm_ftoi = true;
    ++expected;
    o = def_of(an, o->operands[0]);
  }
  if (o && o->name == "xt.add" && o != mm) {
    if (!epilogue_row(an, o, tc, p.bias, err)) return false;
    p.gemm_bias = true;
    expected += 2;
    o = def_of(an, o->operands[0]);
  }
  if (o && o->name == "xt.mul" && o != mm) {
    if (!epilogue_row(an, o, tc, p.scale, err)) return false;
    p.gemm_scale = true;
    expected += 2;
    o = def_of(an, o->operands[0]);
  }
  if (o != mm || count_ops(an) != expected) {
    err = "matmul programs must be store([ftoi]((matmul [* scale]) [+ bias])) with loaded operands";
    return false;
  }
  const Op* la = def_of(an, mm->operands[0]);
  const Op* lb = def_of(an, mm->operands[1]);
  if (!la || !lb || la->name != "xt.load" || lb->name != "xt.load") {
    err = "matmul operands must be loaded tiles";
    return false;
  }
  const Type& ta = an.f.type_of(la->results[0]);
  const Type& tb = an.f.type_of(lb->results[0]);
  if (!((ta.elem == Elem::F16 || ta.elem == Elem::BF16 || ta.elem == Elem::I8) && tb.elem == ta.elem &&
        tc.elem == Elem::F32)) {
    err = "the HIP matmul kernel takes f16 x f16, bf16 x bf16 or i8 x i8 tiles with an f32 result";
    return false;
  }
  if (!access_of(an, *la, p.a, err) || !access_of(an, *lb, p.b, err) ||
      !access_of(an, *st, p.c, err))
    return false;
  if (p.c.elem != (p.gemm_ftoi ? Elem::I8 : Elem::F32)) {
    err = "matmul result must be stored as f32, or as i8 after astype(int8)";
    return false;
  }
  const bool i8 = ta.elem == Elem::I8;
  int64_t M = ta.shape[0], K = ta.shape[1], N = tb.shape[1];
  if (M % 64 || N % 64 || K % (i8 ? 128 : 64)) {
    err = i8 ? "the HIP i8 matmul kernel needs tile M, N multiples of 64 and K a multiple of 128"
             : "the HIP matmul kernel needs tile M, N and K to be multiples of 64";
    return false;
  }
  if (p.a.ld % (i8 ? 16 : 8) || p.b.ld % (i8 ? 16 : 8) || p.c.ld % 4) {
    err = "the HIP matmul kernel needs 16-byte aligned rows";
    return false;
  }
  p.kind = PlanKind::Gemm;
  p.gemm_k = K;
  double blocks = double(p.grid[0]) * p.grid[1] * p.grid[2];
  p.algo_flops = blocks * 2.0 * double(M) * double(N) * double(K);
  // minimum HBM traffic: each argument once
  double bytes = 0;
  std::vector<int> args = {p.a.arg, p.b.arg, p.c.arg};
  if (p.gemm_scale) args.push_back(p.scale.arg);
  if (p.gemm_bias) args.push_back(p.bias.arg);
  for (int arg : args) {
    const Type& t = an.f.type_of(an.f.args[arg]);
    bytes += double(t.numel()) * elem_bytes(t.elem);
  }
  p.algo_bytes = bytes;
  return true;
}

// -- Conv2d ----------------------------------------------------------------------

bool match_conv(const Analysis& an, Plan& p, std::string& err) {
  int nc, nst;
  const Op* cv = only(an, "xt.load_conv2d", nc);
  const Op* st = only(an, "xt.store", nst);
  if (nc != 1) return false;
  if (nst != 1 || count_ops(an) != 3 || st->operands[0] != cv->results[0]) {
    err = "conv2d programs must be store(load_conv2d(src, load filter))";
    return false;
  }
  const Op* lf = def_of(an, cv->operands[1]);
  if (!lf || lf->name != "xt.load") {
    err = "the load_conv2d filter must be a loaded tile";
    return false;
  }
  ConvPlan& c = p.conv;
  const Type& src = an.f.type_of(cv->operands[0]);
  const Type& ft = an.f.type_of(lf->results[0]);
  const Type& fm = an.f.type_of(lf->operands[0]);
  const Type& res = an.f.type_of(cv->results[0]);
  const Type& outm = an.f.type_of(st->operands[1]);
  // i8 is the reference's own load_conv2d dtype (xtile/dsl.py:284-285); f16
  // and bf16 are the narrow-float extension
  // the result is f32 or bf16 (lib/xt/XTOps.cpp:80-82), stored into a memref of its type
  if (!((src.elem == Elem::F16 || src.elem == Elem::BF16 || src.elem == Elem::I8) &&
        ft.elem == src.elem && (res.elem == Elem::F32 || res.elem == Elem::BF16))) {
    err = "the HIP conv2d kernels take i8, f16 or bf16 source and filter of one type with an f32 or bf16 "
          "result";
    return false;
  }
  // the filter tile is one whole filter out of a stack along KH: its last
  // three dims are the memref's, so it is one contiguous K x Cout block
  if (ft.shape.size() != 4 || fm.shape.size() != 4 ||
      !std::equal(ft.shape.begin() + 1, ft.shape.end(), fm.shape.begin() + 1)) {
    err = "the HIP conv2d kernels need the filter tile to span the filter array's KW, Cin and Cout dims";
    return false;
  }
  if (const Attr* g = find_attr(cv->attrs, "group"))
    if (g->i != 1) {
      err = "the HIP conv2d kernel supports group = 1 only";
      return false;
    }
  c.src_arg = an.arg_index(cv->operands[0]);
  c.filt_arg = an.arg_index(lf->operands[0]);
  c.out_arg = an.arg_index(st->operands[1]);
  if (c.src_arg < 0 || c.filt_arg < 0 || c.out_arg < 0) {
    err = "conv2d operands must be function arguments";
    return false;
  }
  c.elem = src.elem;
  c.N = src.shape[0];
  c.H = src.shape[1];
  c.W = src.shape[2];
  c.C = src.shape[3];
  c.KH = ft.shape[0];
  c.KW = ft.shape[1];
  c.CO = ft.shape[3];
  c.TB = res.shape[0];
  c.TH = res.shape[1];
  c.TW = res.shape[2];
  c.TC = res.shape[3];
  c.out_elem = res.elem;
  if (c.TB * c.TH * c.TW <= 0 || c.TC <= 0) {
    err = "load_conv2d result tile must not be empty";
    return false;
  }
  const Attr* pad = find_attr(cv->attrs, "pad");
  const Attr* stride = find_attr(cv->attrs, "stride");
  const Attr* dil = find_attr(cv->attrs, "dilation");
  c.pad_top = pad->ints[0];
  c.pad_left = pad->ints[1];
  c.stride_h = stride->ints[0];
  c.stride_w = stride->ints[1];
  c.dil_h = dil->ints[0];
  c.dil_w = dil->ints[1];
  // conv tile coordinates; the channel coordinate selects input channels
  // [idx_c * Cin, ...) (lib/xt/XTToNova.cpp:396-401), which is in range only for 0.
  if (!coord_of(an, cv->operands[2], 0, c.cb, err) || !coord_of(an, cv->operands[3], 0, c.ch, err) ||
      !coord_of(an, cv->operands[4], 0, c.cw, err))
    return false;
  Coord cc;
  if (!coord_of(an, cv->operands[5], 0, cc, err)) return false;
  if (cc.axis >= 0 || cc.value != 0) {
    err = "load_conv2d channel tile coordinate must be the constant 0";
    return false;
  }
  // batch coordinate must stay inside the source
  int64_t bhi = c.cb.axis < 0 ? c.cb.value : p.grid[c.cb.axis] - 1;
  int64_t blo = c.cb.axis < 0 ? c.cb.value : 0;
  if (blo < 0 || (bhi + 1) * c.TB > c.N) {
    err = "load_conv2d batch tile coordinate exceeds the source batch";
    return false;
  }
  for (const Coord* k : {&c.ch, &c.cw})
    if (k->axis < 0 && k->value < 0) {
      err = "load_conv2d tile coordinates must be non-negative";
      return false;
    }
  // filter tile origin (shared loads take the group leader's coordinates)
  int fshared = 0;
  if (const Attr* sh = find_attr(lf->attrs, "shared")) fshared = static_cast<int>(sh->i);
  std::vector<int> fcv(lf->operands.begin() + 1, lf->operands.end());
  if (!tile_origin(an, fcv, fshared, ft.shape, fm.shape, "filter load", c.filt_addr, nullptr, err))
    return false;
  std::vector<int> scv(st->operands.begin() + 2, st->operands.end());
  if (!tile_origin(an, scv, 0, res.shape, outm.shape, "conv2d store", c.out_addr, nullptr, err))
    return false;
  c.out_H = outm.shape[1];
  c.out_W = outm.shape[2];
  c.out_C = outm.shape[3];
  p.kind = PlanKind::Conv2d;
  double blocks = double(p.grid[0]) * p.grid[1] * p.grid[2];
  double pixels = blocks * double(c.TB * c.TH * c.TW);
  p.algo_flops = 2.0 * pixels * double(c.TC) * double(c.KH * c.KW * c.C);
  p.algo_bytes = double(src.numel()) * elem_bytes(src.elem) + double(fm.numel()) * elem_bytes(fm.elem) +
                 pixels * double(c.TC) * elem_bytes(res.elem);
  return true;
}

// -- TileVM ----------------------------------------------------------------------
//
// Every other program without conv: the Block's ops, in program order, become
// tile instructions over LDS slots (one workgroup per Block).  Values are held
// as f32 whatever their element type, as the reference's loop-lowered
// execution holds them; loads and stores convert.  Slots are assigned by
// liveness, first fit; reshape and itof rename a slot (row-major data, and an
// i8 value is already held exactly); transpose swaps the last two dims and
// permute reorders dims (include/xt/XTOps.td), both as a Permute.

bool vm_unary(const std::string& n, VmUnary& k) {
  static const std::pair<const char*, VmUnary> table[] = {
      {"xt.exp", VmUnary::Exp},       {"xt.cos", VmUnary::Cos},         {"xt.sin", VmUnary::Sin},
      {"xt.reciprocal", VmUnary::Recip}, {"xt.rsqrt", VmUnary::Rsqrt}, {"xt.sigmoid", VmUnary::Sigmoid},
      {"xt.tanh", VmUnary::Tanh},     {"xt.silu", VmUnary::Silu},       {"xt.ftoi", VmUnary::Ftoi}};
  for (auto& e : table)
    if (n == e.first) {
      k = e.second;
      return true;
    }
  return false;
}

// shape padded to rank 3 with leading 1s
bool pad3(const std::vector<int64_t>& s, int dims[3], std::string& err) {
  if (s.empty() || s.size() > 3) {
    err = "tile programs on the HIP backend take tensors of rank 1 to 3";
    return false;
  }
  const int off = 3 - static_cast<int>(s.size());
  for (int d = 0; d < 3; ++d) dims[d] = d < off ? 1 : static_cast<int>(s[d - off]);
  return true;
}

bool vm_elem(Elem e) { return e == Elem::F32 || e == Elem::F16 || e == Elem::BF16 || e == Elem::I8; }

bool match_vm(const Analysis& an, Plan& p, std::string& err) {
  const int nops = static_cast<int>(an.compute.size());
  // every op must be one the interpreter runs
  for (const Op* o : an.compute) {
    VmUnary u;
    const std::string& n = o->name;
    const bool ok = n == "xt.load" || n == "xt.store" || n == "xt.add" || n == "xt.sub" || n == "xt.mul" ||
                    n == "xt.reduce_sum" || n == "xt.reduce_max" || n == "xt.reshape" ||
                    n == "xt.transpose" || n == "xt.permute" || n == "xt.matmul" || n == "xt.mma" ||
                    n == "xt.itof" || vm_unary(n, u);
    if (!ok) return false;
  }
  for (const Op* o : an.compute) {
    const std::string& n = o->name;
    for (int r : o->results)
      if (!vm_elem(an.f.type_of(r).elem)) {
        err = "tile programs on the HIP backend hold f32, f16, bf16 or i8 tensors (" + n + " yields " +
              elem_name(an.f.type_of(r).elem) + ")";
        return false;
      }
    if (n == "xt.store" && !vm_elem(an.f.type_of(o->operands[1]).elem)) {
      err = "tile programs on the HIP backend store f32, f16, bf16 or i8 tiles";
      return false;
    }
  }
  // storage roots (reshape results share their operand's slot) and last uses
  std::map<int, int> root;
  auto root_of = [&](int v) {
    auto it = root.find(v);
    return it == root.end() ? v : it->second;
  };
  std::map<int, int> last_use;
  for (int i = 0; i < nops; ++i) {
    const Op* o = an.compute[i];
    if (o->name == "xt.reshape" || o->name == "xt.itof") root[o->results[0]] = root_of(o->operands[0]);
    for (int v : o->operands) {
      if (!an.f.type_of(v).is_tensor()) continue;
      last_use[root_of(v)] = i;
    }
  }
  // first-fit allocation over [0, inf) in floats, 4-float granules
  std::vector<std::pair<int, int>> used;  // (offset, size) of live slots
  std::map<int, std::pair<int, int>> slot; // root -> (offset, size)
  int high = 0;
  auto alloc = [&](int floats) {
    floats = (floats + 3) & ~3;
    int at = 0;
    for (;;) {
      bool clash = false;
      for (auto& u : used)
        if (at < u.first + u.second && u.first < at + floats) {
          at = u.first + u.second;
          clash = true;
        }
      if (!clash) break;
    }
    used.push_back({at, floats});
    high = std::max(high, at + floats);
    return std::make_pair(at, floats);
  };
  auto release = [&](int r) {
    auto it = slot.find(r);
    if (it == slot.end()) return;
    for (size_t k = 0; k < used.size(); ++k)
      if (used[k].first == it->second.first) {
        used.erase(used.begin() + k);
        break;
      }
  };
  // values known to be integers in [-128, 127]: i8 loads and ftoi results
  // (and their renamings, transposes and permutes)
  std::set<int> small_int;
  for (const Op* o : an.compute) {
    const std::string& n = o->name;
    if ((n == "xt.load" && an.f.type_of(o->results[0]).elem == Elem::I8) || n == "xt.ftoi" ||
        ((n == "xt.transpose" || n == "xt.permute") && small_int.count(root_of(o->operands[0]))))
      small_int.insert(o->results[0]);
  }
  VmPlan vm;
  double once_bytes = 0, flops = 0;
  for (int i = 0; i < nops; ++i) {
    const Op* o = an.compute[i];
    const std::string& n = o->name;
    VmInst in;
    if (n == "xt.load" || n == "xt.store") {
      const bool is_load = n == "xt.load";
      const int mem_v = is_load ? o->operands[0] : o->operands[1];
      const Type& mem = an.f.type_of(mem_v);
      const Type& ten = is_load ? an.f.type_of(o->results[0]) : an.f.type_of(o->operands[0]);
      VmAccess acc;
      acc.arg = an.arg_index(mem_v);
      acc.elem = mem.elem;
      if (acc.arg < 0) {
        err = n + " must access a function argument";
        return false;
      }
      int shared = 0;
      if (is_load)
        if (const Attr* sh = find_attr(o->attrs, "shared")) shared = static_cast<int>(sh->i);
      std::vector<int> cv(o->operands.begin() + (is_load ? 1 : 2), o->operands.end());
      const std::string what = n + " of argument #" + std::to_string(acc.arg);
      if (!tile_origin(an, cv, shared, ten.shape, mem.shape, what, acc.addr, nullptr, err)) return false;
      if (!pad3(ten.shape, in.dims, err)) return false;
      std::vector<int64_t> st = strides_of(mem.shape);
      const int off = 3 - static_cast<int>(st.size());
      for (int d = 0; d < 3; ++d) acc.stride[d] = d < off ? 0 : st[d - off];
      in.op = is_load ? VmOp::Load : VmOp::Store;
      in.kind = static_cast<int16_t>(vm.access.size());
      vm.access.push_back(acc);
      // algorithmic traffic: each distinct tile once.  The tile origin moves
      // only along the grid axes with a nonzero step (a shared load's leader
      // rule has already zeroed the axes below k), so Blocks that differ only
      // along the other axes read the same tile: a tile at the same place in
      // every Block (weights, scalars) moves from HBM once, a shared=k tile
      // once per sharing group.
      const double tb = double(ten.numel()) * elem_bytes(mem.elem);
      const double distinct = (acc.addr.sx ? double(p.grid[0]) : 1.0) * (acc.addr.sy ? double(p.grid[1]) : 1.0) *
                              (acc.addr.sz ? double(p.grid[2]) : 1.0);
      once_bytes += tb * distinct;
      if (is_load) {
        auto sl = alloc(static_cast<int>(ten.numel()));
        slot[o->results[0]] = sl;
        in.dst = sl.first;
      } else {
        in.a = slot.at(root_of(o->operands[0])).first;
      }
    } else if (n == "xt.reshape" || n == "xt.itof") {
      continue;  // same slot, new shape or type
    } else {
      const Type& res = an.f.type_of(o->results[0]);
      const Type& ta = an.f.type_of(o->operands[0]);
      in.a = slot.at(root_of(o->operands[0])).first;
      VmUnary u;
      if (vm_unary(n, u)) {
        in.op = VmOp::Unary;
        in.kind = static_cast<int16_t>(u);
        if (!pad3(res.shape, in.dims, err)) return false;
      } else if (n == "xt.add" || n == "xt.sub" || n == "xt.mul") {
        const Type& tb = an.f.type_of(o->operands[1]);
        in.op = VmOp::Binary;
        in.kind = static_cast<int16_t>(n == "xt.add" ? VmBinary::Add : n == "xt.sub" ? VmBinary::Sub : VmBinary::Mul);
        in.b = slot.at(root_of(o->operands[1])).first;
        // numpy broadcasting, right-aligned (lib/xt/XTOps.cpp:104-145)
        if (ta.rank() > res.rank() || tb.rank() > res.rank()) {
          err = "broadcast operands must not outrank the result";
          return false;
        }
        if (!pad3(res.shape, in.dims, err) || !pad3(ta.shape, in.lhs, err) || !pad3(tb.shape, in.aux, err))
          return false;
        for (int d = 0; d < 3; ++d)
          if ((in.aux[d] != in.dims[d] && in.aux[d] != 1) || (in.lhs[d] != in.dims[d] && in.lhs[d] != 1)) {
            err = "broadcast operand dims must equal the result's or be 1";
            return false;
          }
      } else if (n == "xt.reduce_sum" || n == "xt.reduce_max") {
        if (ta.rank() != 2) {
          err = "reductions take rank-2 tiles (lib/xt/XTOps.cpp:274-307)";
          return false;
        }
        int64_t axis = find_attr(o->attrs, "axis")->i;
        if (axis < 0) axis += 2;
        in.op = VmOp::Reduce;
        in.kind = static_cast<int16_t>(n == "xt.reduce_sum" ? VmReduce::Sum : VmReduce::Max);
        if (!pad3(ta.shape, in.dims, err)) return false;
        in.aux[0] = static_cast<int>(axis);
      } else if (n == "xt.matmul" || n == "xt.mma") {
        const Type& tb = an.f.type_of(o->operands[1]);
        if (ta.rank() != 2 || tb.rank() != 2 || res.rank() != 2 || ta.shape[1] != tb.shape[0]) {
          err = "matmul takes [M, K] x [K, N] tiles (lib/xt/XTOps.cpp:218-235)";
          return false;
        }
        in.op = VmOp::Matmul;
        in.b = slot.at(root_of(o->operands[1])).first;
        if (n == "xt.mma") in.c = slot.at(root_of(o->operands[2])).first;
        const int64_t K = ta.shape[1];
        in.dims[0] = 1;
        in.dims[1] = static_cast<int>(ta.shape[0]);
        in.dims[2] = static_cast<int>(tb.shape[1]);
        in.aux[0] = static_cast<int>(K);
        // i8 x i8 sums stay exact in i32 for K < 2^17 (|a*b| <= 2^14)
        in.aux[1] = small_int.count(root_of(o->operands[0])) && small_int.count(root_of(o->operands[1])) &&
                    K < (int64_t(1) << 17);
        in.aux[2] = 0;
        flops += 2.0 * double(ta.shape[0]) * double(tb.shape[1]) * double(K);
      } else {  // transpose / permute
        in.op = VmOp::Permute;
        if (!pad3(ta.shape, in.dims, err)) return false;
        const int r = ta.rank(), off = 3 - r;
        int perm[3] = {0, 1, 2};
        if (n == "xt.transpose") {
          if (r < 2) {
            err = "transpose needs a tile of rank >= 2";
            return false;
          }
          std::swap(perm[1], perm[2]);
        } else {
          const Attr* pa = find_attr(o->attrs, "permutation");
          if (!pa || static_cast<int>(pa->ints.size()) != r) {
            err = "permute needs a permutation attribute of the tile's rank";
            return false;
          }
          for (int d = 0; d < r; ++d) perm[off + d] = static_cast<int>(pa->ints[d]) + off;
        }
        for (int d = 0; d < 3; ++d) in.aux[d] = perm[d];
      }
      auto sl = alloc(static_cast<int>(res.numel()));
      slot[o->results[0]] = sl;
      in.dst = sl.first;
    }
    vm.inst.push_back(in);
    // free the slots whose last use was this op
    for (int v : o->operands) {
      if (!an.f.type_of(v).is_tensor()) continue;
      const int r = root_of(v);
      if (last_use[r] == i) release(r);
    }
  }
  vm.lds_floats = high;
  p.kind = PlanKind::TileVM;
  p.vm = std::move(vm);
  const double blocks = double(p.grid[0]) * p.grid[1] * p.grid[2];
  p.algo_bytes = once_bytes;
  p.algo_flops = blocks * flops;
  return true;
}

// The interpreter holds every live tile in LDS and takes its instruction list
// as a kernel argument.
bool vm_fits_interpreter(const VmPlan& vm, std::string& err) {
  if (int64_t(vm.lds_floats) * 4 > 160 * 1024) {
    err = "tile program needs " + std::to_string((int64_t(vm.lds_floats) * 4 + 1023) / 1024) +
          " KB of LDS for its live tiles (at most 160 KB per workgroup)";
    return false;
  }
  if (vm.inst.size() > 40 || vm.access.size() > 8) {
    err = "tile program too long for the HIP interpreter (at most 40 instructions and 8 loads/stores)";
    return false;
  }
  return true;
}

}  // namespace

std::string Plan::describe() const {
  std::ostringstream os;
  auto tile = [&](const Access2D& a) {
    std::ostringstream t;
    t << a.rows << "x" << a.cols;
    return t.str();
  };
  switch (kind) {
    case PlanKind::EwBinary:
      os << "ew_binary op=" << (ew_op == EwOp::Add ? "add" : ew_op == EwOp::Sub ? "sub" : "mul")
         << " f32 tile=" << tile(c);
      if (ew_flat) os << " flat=" << ew_flat;
      break;
    case PlanKind::RowSoftmax:
      os << "row_softmax f32 tile=" << tile(a);
      break;
    case PlanKind::Gemm:
      os << "gemm " << elem_name(a.elem) << "->f32 tile=" << a.rows << "x" << b.cols
         << " k=" << gemm_k;
      if (gemm_scale || gemm_bias || gemm_ftoi) {
        os << " epilogue=";
        const char* sep = "";
        if (gemm_scale) os << sep << "scale", sep = ",";
        if (gemm_bias) os << sep << "bias", sep = ",";
        if (gemm_ftoi) os << sep << "ftoi->i8";
      }
      break;
    case PlanKind::TileVM: {
      int loads = 0, stores = 0;
      for (const VmInst& in : vm.inst) {
        loads += in.op == VmOp::Load;
        stores += in.op == VmOp::Store;
      }
      os << "tile_vm f32 insts=" << vm.inst.size() << " loads=" << loads << " stores=" << stores
         << " lds=" << vm.lds_floats * 4 << "B";
      if (!unfused.empty()) os << " (not fused: " << unfused << ")";
      break;
    }
    case PlanKind::Fused:
      os << fused->layout << " insts=" << vm.inst.size();
      break;
    case PlanKind::Conv2d:
      os << "conv2d_nhwc " << elem_name(conv.elem) << "->" << elem_name(conv.out_elem) << " tile=" << conv.TB
         << "x" << conv.TH << "x" << conv.TW << "x" << conv.TC << " filter=" << conv.KH << "x" << conv.KW << "x"
         << conv.C << "x" << conv.CO;
      break;
  }
  os << " grid=(" << grid[0] << "," << grid[1] << "," << grid[2] << ")";
  return os.str();
}

bool build_plan(const Module& m, const std::string& func, Plan& p, std::string& err) {
  const Func* f = nullptr;
  if (func.empty()) {
    if (m.funcs.size() != 1) {
      err = "module has " + std::to_string(m.funcs.size()) + " functions; name one";
      return false;
    }
    f = &m.funcs[0];
  } else {
    f = find_func(m, func);
    if (!f) {
      err = "no function named @" + func;
      return false;
    }
  }
  p = Plan{};
  p.func = f->name;
  if (!find_attr(f->attrs, "xt.grid") || !get_grid(*f, p.grid)) {
    err = "@" + f->name + " has no xt.grid attribute";
    return false;
  }
  if (!f->result_types.empty() || f->blocks.size() != 1) {
    err = "@" + f->name + " must be a void single-block function";
    return false;
  }
  for (int a : f->args) {
    if (!f->type_of(a).is_memref()) {
      err = "@" + f->name + " arguments must all be memrefs";
      return false;
    }
    p.arg_types.push_back(f->type_of(a));
  }
  Analysis an(*f, p.grid);
  for (const Op* o : an.compute)
    if (o->name == "xt.store" && an.def.count(o->operands[0]) == 0) {
      err = "stored values must be computed in the function";
      return false;
    }
  if (!check_independent(an, err)) {
    err = "@" + f->name + ": " + err;
    return false;
  }
  // the specialised kernels first; what they decline (with a reason) goes to
  // the tile interpreter, and the first reason is reported if that fails too
  err.clear();
  std::string first;
  for (auto match : {match_ew, match_softmax, match_gemm, match_conv}) {
    std::string why;
    if (match(an, p, why)) {
      if (p.kind == PlanKind::RowSoftmax) {
        // the interpreter lowering, for buffers the softmax kernel cannot vectorise
        Plan q = p;
        std::string e2;
        if (match_vm(an, q, e2) && vm_fits_interpreter(q.vm, e2)) {
          p.vm = std::move(q.vm);
          p.vm_fallback = true;
        } else {
          p.vm_fallback_why = e2.empty() ? "no interpreter lowering" : e2;
        }
      }
      return true;
    }
    if (first.empty()) first = why;
  }
  if (match_vm(an, p, err)) {
    // compiled for itself: the register-resident fused kernel when every
    // value fits its layout, else the LDS-staged kernel (XTILE_AMD_FUSE=0
    // keeps the interpreter; XTILE_AMD_STAGE=0 keeps it for what the fused
    // layout declines)
    const char* env = std::getenv("XTILE_AMD_FUSE");
    const char* stage_env = std::getenv("XTILE_AMD_STAGE");
    const bool fuse_off = env && std::string(env) == "0";
    FusedPlan fp;
    std::string why, why_staged;
    if (!fuse_off && (fuse_vm(p.vm, p.grid, fp, why) ||
                      (!(stage_env && std::string(stage_env) == "0") && stage_vm(p.vm, p.grid, fp, why_staged)))) {
      p.kind = PlanKind::Fused;
      p.fused = std::make_shared<FusedPlan>(std::move(fp));
      p.vm_fallback = vm_fits_interpreter(p.vm, p.vm_fallback_why);
      return true;
    }
    if (fuse_off) p.unfused = "XTILE_AMD_FUSE=0";
    else if (stage_env && std::string(stage_env) == "0") p.unfused = why + "; XTILE_AMD_STAGE=0";
    else p.unfused = why + "; not staged: " + why_staged;
    if (vm_fits_interpreter(p.vm, err)) return true;
    err += " (not fused: " + p.unfused + ")";
  }
  if (!first.empty()) {
    err = first + (err.empty() ? "" : "; the tile interpreter declines it too: " + err);
    return false;
  }
  if (!err.empty()) return false;
  std::ostringstream os;
  os << "unsupported tile program for the HIP backend: @" << f->name << " uses";
  for (const Op* o : an.compute) os << " " << o->name;
  err = os.str();
  return false;
}

}  // namespace xt
