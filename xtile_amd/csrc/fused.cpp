// Fused tile programs: the tile interpreter's lowering of a program (VmPlan)
// turned into the source of one HIP kernel that keeps every value in
// registers.  The runtime compiles the source with hiprtc (jit.cpp).
//
// Layout.  The program's main tile is [R, C] (the largest extents of its
// values); every value is that tile or a [1, C], [R, 1] or [1, 1] broadcast of
// it.  A workgroup of TR x TC threads runs one Block; thread (tr, tc) owns rows
// tr + sr TR (sr < SR = R / TR) and column vectors tc + sc TC (sc < SC = C /
// (VW TC)) of VW consecutive columns, so each row access is a VW-wide vector
// load or store and consecutive threads touch consecutive vectors.  A [1, C]
// value is held by every tr, an [R, 1] value by every tc, a [1, 1] value by
// every thread: broadcasts are register reads.  TC divides the CV = C / VW
// vectors of a row when that keeps at most 64 elements a thread; otherwise
// (rows whose vector count has no large power-of-two divisor, e.g. 3798
// floats = 1899 float2) the row is "ragged": TC is the largest power of two
// <= min(CV, 512), SC = ceil(CV / TC), and vector tc + sc TC exists only below
// CV: its loads read zeros, its stores are skipped and column reductions
// skip it.
//
// Ops (the interpreter's semantics, kernels/tilevm.hip): loads convert f16 /
// bf16 / i8 exactly and stores round (nearest even for f16 / bf16; round,
// saturate and NaN -> 0 for i8); add / sub / mul and the unary ops use the same
// f32 formulas with contraction off; reductions keep the reduced dim at 1 and
// combine within a thread, then across the TC threads of a row by lane
// shuffles (and LDS when a row spans waves), or across the TR threads of a
// column through LDS.
#include <algorithm>
#include <cmath>
#include <map>
#include <sstream>

#include "fused_common.h"
#include "plan.h"

namespace xt {
namespace {


struct Layout {
  int R = 1, C = 1, VW = 1, TR = 1, TC = 1, SR = 1, SC = 1;
  int CV = 1;           // vectors of VW columns in a row
  bool ragged = false;  // SC * TC > CV: the last vectors of a thread row are absent
  int threads() const { return TR * TC; }
  int cols() const { return SC * VW; }  // register columns of a thread
};

struct VKind {
  bool r = false, c = false;  // varies along R / along C
};

int pow2_divisor(int v, int cap) {
  int p = 1;
  while (p * 2 <= cap && v % (p * 2) == 0) p *= 2;
  return p;
}

class Gen {
 public:
  Gen(const VmPlan& vm, const int32_t grid[3], int max_vw) : vm_(vm), max_vw_(max_vw) {
    for (int d = 0; d < 3; ++d) grid_[d] = grid[d];
  }

  bool run(FusedPlan& out, std::string& why) {
    if (!shapes(why) || !layout(why)) return false;
    // Block-invariant loads (weights, scalars) are read once per workgroup when
    // workgroups outnumber what the chip holds: each workgroup then walks a
    // grid-stride list of Blocks with those values kept in registers.
    const long long blocks = (long long)grid_[0] * grid_[1] * grid_[2];
    const long long resident = 256LL * std::max(1, std::min(32, 2048 / L.threads()));
    bool invariant = false;
    long long stream_bytes = 0;  // streamed tile bytes one Block reads
    for (const VmInst& in : vm_.inst)
      if (in.op == VmOp::Load) {
        invariant |= !streamed(in.kind);
        if (streamed(in.kind)) stream_bytes += (long long)in.dims[1] * in.dims[2] * elem_bytes(vm_.access[in.kind].elem);
      }
    hoist_ = invariant && blocks > 2 * resident && blocks < (1LL << 30);
    const long long wgs = hoist_ ? walkers(blocks, resident, stream_bytes) : blocks;
    pre_.str("");
    body_.str("");
    for (size_t i = 0; i < vm_.inst.size(); ++i)
      if (!emit(static_cast<int>(i), why)) return false;
    if (red_floats_ * 4 > 64 * 1024) {
      why = "fused kernel reductions need more than 64 KB of LDS";
      return false;
    }
    std::ostringstream k;
    k << "extern \"C\" __global__ void __launch_bounds__(" << L.threads() << ") xt_fused(FusedArgs a) {\n"
      << "#pragma clang fp contract(off)\n"
      << "  const int t = threadIdx.x, tc = t % " << L.TC << ", tr = t / " << L.TC << ";\n"
      << "  (void)tr; (void)tc;\n";
    if (red_floats_ > 0) k << "  __shared__ float red[" << red_floats_ << "];\n";
    k << pre_.str();
    if (hoist_) k << "  for (int bid = blockIdx.x; bid < " << blocks << "; bid += " << wgs << ") {\n";
    else k << "  {\n    const int bid = blockIdx.x;\n";
    k << "  const int x = bid % " << grid_[0] << ", y = (bid / " << grid_[0] << ") % " << grid_[1]
      << ", z = bid / " << (long long)grid_[0] * grid_[1] << ";\n"
      << "  (void)x; (void)y; (void)z;\n";
    k << body_.str();
    // with one LDS region, the next Block's write to it waits for this Block's reads
    if (hoist_ && n_red_ == 1) k << "  __syncthreads();\n";
    k << "  }\n}\n";
    out.source = std::string(fused_preamble()) + k.str();
    out.threads = L.threads();
    out.vw = L.VW;
    out.workgroups = static_cast<int>(wgs);
    std::ostringstream lay;
    lay << "fused f32 tile=" << L.R << "x" << L.C << " threads=" << L.TR << "x" << L.TC << " vw=" << L.VW;
    if (L.ragged) lay << " ragged";
    if (hoist_) lay << " workgroups=" << wgs;
    out.layout = lay.str();
    return true;
  }

 private:
  const VmPlan& vm_;
  int max_vw_ = 4;
  int grid_[3];
  Layout L;
  std::map<int, std::pair<int, VKind>> slot_;  // LDS slot -> (value id, kind)
  std::ostringstream pre_, body_;  // hoisted Block-invariant loads; the per-Block body
  bool hoist_ = false;
  int red_floats_ = 0;
  int n_red_ = 0;                   // reductions that go through LDS

  // Workgroups of a kernel that walks the Blocks: each holds its Block's
  // streamed tiles and the next Block's prefetch, so the grid keeps about
  // 2 * wgs * stream_bytes of reads in flight.  About 16 MB is best: on an
  // 8192 x 4096 f32 layernorm (16 KB rows) 512 workgroups, two per CU with 16
  // rows each, ran 44.5 us per launch against 47.0 with 1024 (full occupancy,
  // 32 MB in flight) and 60.7 with 256.  A multiple of the 256 CUs, within
  // [256, resident], and among those near the target the one that deals the
  // Blocks most evenly (384 workgroups over 8192 rows, 21.3 rows each, ran
  // 47.7 us).
  static long long walkers(long long blocks, long long resident, long long stream_bytes) {
    constexpr long long kInFlight = 16LL << 20;
    long long target = stream_bytes > 0 ? kInFlight / (2 * stream_bytes) : resident;
    // the nearest multiple of 256 (rows a little over 16 KB are not halved)
    target = std::max(256LL, std::min(resident, (target + 128) / 256 * 256));
    long long best = target;
    double best_cost = 1e300;
    for (long long w = std::max(256LL, target / 2 / 256 * 256); w <= std::min(resident, target * 2); w += 256) {
      const double per = (double)blocks / w, imbalance = std::ceil(per) / per;
      // prefer the target; a workgroup count off it by 2x costs as much as 10% imbalance
      const double cost = imbalance * (1.0 + 0.1 * std::fabs(std::log2((double)w / target)));
      if (cost < best_cost) {
        best_cost = cost;
        best = w;
      }
    }
    return best;
  }

  static void dims2(const int d[3], int& a, int& b) {
    a = d[1];
    b = d[2];
  }

  // every value: rank <= 2 and a broadcast of one [R, C]
  bool shapes(std::string& why) {
    int R = 1, C = 1;
    std::vector<std::pair<int, int>> all;
    for (const VmInst& in : vm_.inst) {
      if (in.op != VmOp::Load && in.op != VmOp::Store && in.op != VmOp::Unary && in.op != VmOp::Binary &&
          in.op != VmOp::Reduce) {
        why = "fused kernels take loads, stores, unary, binary and reduce ops";
        return false;
      }
      if (in.dims[0] != 1 || (in.op == VmOp::Binary && (in.aux[0] != 1 || in.lhs[0] != 1))) {
        why = "fused kernels take tiles of rank <= 2";
        return false;
      }
      all.push_back({in.dims[1], in.dims[2]});
      if (in.op == VmOp::Binary) {
        all.push_back({in.aux[1], in.aux[2]});
        all.push_back({in.lhs[1], in.lhs[2]});
      }
    }
    for (auto& s : all) {
      R = std::max(R, s.first);
      C = std::max(C, s.second);
    }
    for (auto& s : all)
      if ((s.first != 1 && s.first != R) || (s.second != 1 && s.second != C)) {
        why = "fused kernels need every value to be one [R, C] tile or a broadcast of it";
        return false;
      }
    L.R = R;
    L.C = C;
    return true;
  }

  bool layout(std::string& why) {
    int vw = max_vw_ >= 4 ? 4 : max_vw_ >= 2 ? 2 : 1;
    for (; vw > 1; vw /= 2) {
      if (L.C % vw) continue;
      bool ok = true;
      for (size_t k = 0; k < vm_.inst.size() && ok; ++k) {
        const VmInst& in = vm_.inst[k];
        if ((in.op != VmOp::Load && in.op != VmOp::Store) || in.dims[2] == 1) continue;
        const VmAccess& acc = vm_.access[in.kind];
        const TileAddr& o = acc.addr;
        ok = acc.stride[2] == 1 && acc.stride[1] % vw == 0 && o.c0 % vw == 0 && o.sx % vw == 0 &&
             o.sy % vw == 0 && o.sz % vw == 0;
      }
      if (ok) break;
    }
    L.VW = vw;
    const int cv = L.C / L.VW;
    L.CV = cv;
    // up to 512 threads (8 waves) a workgroup: 4096-float rows at two float4 a thread
    L.TC = pow2_divisor(cv, 512);
    L.TR = pow2_divisor(L.R, 512 / L.TC);
    L.SR = L.R / L.TR;
    L.SC = cv / L.TC;
    L.ragged = false;
    if (L.SR * L.cols() > 64) {
      // ragged rows: the widest power-of-two thread row, the last vectors guarded
      int tc = 1;
      while (tc * 2 <= std::min(cv, 512)) tc *= 2;
      if (tc > L.TC) {
        L.TC = tc;
        L.TR = pow2_divisor(L.R, 512 / L.TC);
        L.SR = L.R / L.TR;
        L.SC = (cv + tc - 1) / tc;
        L.ragged = L.SC * tc != cv;
      }
    }
    if (L.SR * L.cols() > 64) {
      why = "fused kernels keep at most 64 elements of a tile per thread";
      return false;
    }
    return true;
  }

  int size_of(VKind k) const { return (k.r ? L.SR : 1) * (k.c ? L.cols() : 1); }
  std::string idx(VKind k, const std::string& sr, const std::string& j) const {
    std::string s;
    if (k.r) s += sr + " * " + std::to_string(k.c ? L.cols() : 1);
    if (k.c) s += (s.empty() ? "" : " + ") + j;
    return s.empty() ? "0" : s;
  }
  static VKind kind_of(int d1, int d2) { return VKind{d1 != 1, d2 != 1}; }

  std::string origin(const TileAddr& o) const {
    std::ostringstream s;
    s << "(" << o.c0 << "LL";
    if (o.sx) s << " + (long long)x * " << o.sx << "LL";
    if (o.sy) s << " + (long long)y * " << o.sy << "LL";
    if (o.sz) s << " + (long long)z * " << o.sz << "LL";
    s << ")";
    return s.str();
  }

  // vector sc of this thread's row exists (ragged rows only)
  std::string present(const std::string& sc) const {
    return "tc + (" + sc + ") * " + std::to_string(L.TC) + " < " + std::to_string(L.CV);
  }

  // element offset of register (sr, sc) of a tile of kind k (row pitch ld)
  std::string elem_off(VKind k, long long ld) const {
    std::string s = "0";
    if (k.r) s = "(long long)(tr + sr * " + std::to_string(L.TR) + ") * " + std::to_string(ld) + "LL";
    if (k.c) s += " + (long long)(tc + sc * " + std::to_string(L.TC) + ") * " + std::to_string(L.VW);
    return s;
  }

  bool emit(int i, std::string& why) {
    const VmInst& in = vm_.inst[i];
    std::ostringstream& b = in.op == VmOp::Load && hoist_ && !streamed(in.kind) ? pre_ : body_;
    const std::string v = "v" + std::to_string(i);
    switch (in.op) {
      case VmOp::Load: {
        const VmAccess& acc = vm_.access[in.kind];
        const VKind k = kind_of(in.dims[1], in.dims[2]);
        const int vw = k.c ? L.VW : 1;
        b << "  float " << v << "[" << size_of(k) << "];\n  {\n";
        b << "    const long long org = " << origin(acc.addr) << ";\n";
        b << "#pragma unroll\n    for (int sr = 0; sr < " << (k.r ? L.SR : 1) << "; ++sr)\n";
        b << "#pragma unroll\n    for (int sc = 0; sc < " << (k.c ? L.SC : 1) << "; ++sc) {\n";
        b << "      const long long off = org + " << elem_off(k, acc.stride[1]) << ";\n";
        const std::string dst = v + "[" + idx(k, "sr", "sc * " + std::to_string(vw) + " + e") + "]";
        if (k.c && L.ragged) {
          b << "      if (" << present("sc") << ") {\n";
          load_code(b, in.kind, acc.elem, vw, dst);
          b << "      } else {\n#pragma unroll\n        for (int e = 0; e < " << vw << "; ++e) " << dst
            << " = 0.0f;\n      }\n";
        } else {
          load_code(b, in.kind, acc.elem, vw, dst);
        }
        b << "    }\n  }\n";
        slot_[in.dst] = {i, k};
        return true;
      }
      case VmOp::Store: {
        const VmAccess& acc = vm_.access[in.kind];
        const VKind k = kind_of(in.dims[1], in.dims[2]);
        auto it = slot_.find(in.a);
        if (it == slot_.end()) return fail(why, "store of an unknown value");
        const VKind vk = it->second.second;
        if (vk.r != k.r || vk.c != k.c) return fail(why, "store of a value with another shape");
        const std::string src = "v" + std::to_string(it->second.first);
        const int vw = k.c ? L.VW : 1;
        // a broadcast value is held by every thread along its unit dim; one stores it
        std::string guard;
        if (!k.r && L.TR > 1) guard = "tr == 0";
        if (!k.c && L.TC > 1) guard += std::string(guard.empty() ? "" : " && ") + "tc == 0";
        b << "  if (" << (guard.empty() ? "true" : guard) << ") {\n";
        b << "    const long long org = " << origin(acc.addr) << ";\n";
        b << "#pragma unroll\n    for (int sr = 0; sr < " << (k.r ? L.SR : 1) << "; ++sr)\n";
        b << "#pragma unroll\n    for (int sc = 0; sc < " << (k.c ? L.SC : 1) << "; ++sc) {\n";
        b << "      const long long off = org + " << elem_off(k, acc.stride[1]) << ";\n";
        const std::string s = src + "[" + idx(k, "sr", "sc * " + std::to_string(vw) + " + e") + "]";
        if (k.c && L.ragged) b << "      if (" << present("sc") << ") {\n";
        store_code(b, in.kind, acc.elem, vw, s);
        if (k.c && L.ragged) b << "      }\n";
        b << "    }\n  }\n";
        return true;
      }
      case VmOp::Unary: {
        auto it = slot_.find(in.a);
        if (it == slot_.end()) return fail(why, "unary op of an unknown value");
        const VKind k = it->second.second;
        const std::string a = "v" + std::to_string(it->second.first);
        b << "  float " << v << "[" << size_of(k) << "];\n";
        b << "#pragma unroll\n  for (int q = 0; q < " << size_of(k) << "; ++q) " << v
          << "[q] = " << replace_x(unary_expr(in.kind), a + "[q]") << ";\n";
        slot_[in.dst] = {i, k};
        return true;
      }
      case VmOp::Binary: {
        auto ia = slot_.find(in.a), ib = slot_.find(in.b);
        if (ia == slot_.end() || ib == slot_.end()) return fail(why, "binary op of an unknown value");
        const VKind ka = ia->second.second, kb = ib->second.second;
        const VKind ko = VKind{ka.r || kb.r, ka.c || kb.c};
        if (ko.r != (in.dims[1] != 1) || ko.c != (in.dims[2] != 1))
          return fail(why, "binary op result shape outside the fused layout");
        const char* op = in.kind == 0 ? "+" : in.kind == 1 ? "-" : "*";
        const std::string a = "v" + std::to_string(ia->second.first), c = "v" + std::to_string(ib->second.first);
        b << "  float " << v << "[" << size_of(ko) << "];\n";
        b << "#pragma unroll\n  for (int sr = 0; sr < " << (ko.r ? L.SR : 1) << "; ++sr)\n";
        b << "#pragma unroll\n  for (int j = 0; j < " << (ko.c ? L.cols() : 1) << "; ++j) " << v << "["
          << idx(ko, "sr", "j") << "] = " << a << "[" << idx(ka, "sr", "j") << "] " << op << " " << c << "["
          << idx(kb, "sr", "j") << "];\n";
        slot_[in.dst] = {i, ko};
        return true;
      }
      case VmOp::Reduce: {
        auto it = slot_.find(in.a);
        if (it == slot_.end()) return fail(why, "reduction of an unknown value");
        const VKind ks = it->second.second;
        const std::string s = "v" + std::to_string(it->second.first);
        const bool is_max = in.kind == 1;
        const std::string init = is_max ? "-__builtin_huge_valf()" : "0.0f";
        auto comb = [&](const std::string& p, const std::string& q) {
          return is_max ? "fmaxf(" + p + ", " + q + ")" : p + " + " + q;
        };
        const int axis = in.aux[0];
        if ((axis == 1 && !ks.c) || (axis == 0 && !ks.r)) {  // over an extent of 1: a copy
          b << "  float " << v << "[" << size_of(ks) << "];\n";
          b << "#pragma unroll\n  for (int q = 0; q < " << size_of(ks) << "; ++q) " << v << "[q] = " << s
            << "[q];\n";
          slot_[in.dst] = {i, ks};
          return true;
        }
        if (axis == 1) {  // over columns: within the thread, then across the TC threads of the row
          const VKind ko{ks.r, false};
          const int nr = ks.r ? L.SR : 1;
          b << "  float " << v << "[" << nr << "];\n";
          b << "#pragma unroll\n  for (int sr = 0; sr < " << nr << "; ++sr) {\n    float m = " << init << ";\n";
          if (L.ragged)  // absent vectors take no part
            b << "#pragma unroll\n    for (int j = 0; j < " << L.cols() << "; ++j) if ("
              << present("j / " + std::to_string(L.VW)) << ") m = " << comb("m", s + "[" + idx(ks, "sr", "j") + "]")
              << ";\n";
          else
            b << "#pragma unroll\n    for (int j = 0; j < " << L.cols() << "; ++j) m = "
              << comb("m", s + "[" + idx(ks, "sr", "j") + "]") << ";\n";
          // a whole wave along the row: DPP steps to lane 63 (xwred), else a
          // butterfly over the row's TC lanes
          if (L.TC >= 64)
            b << "    m = xwred<" << (is_max ? "true" : "false") << ">(m);\n";
          else
            b << "#pragma unroll\n    for (int o = " << L.TC / 2 << "; o > 0; o >>= 1) m = "
              << comb("m", "__shfl_xor(m, o, 64)") << ";\n";
          b << "    " << v << "[sr] = m;\n  }\n";
          if (L.TC > 64) {  // the row spans TC / 64 waves: combine through LDS
            // each reduction has LDS of its own, so one barrier orders its writes before its reads
            const int W = L.TC / 64;
            const std::string base = std::to_string(red_floats_) + " + ";
            red_floats_ += nr * L.TR * W;
            ++n_red_;
            b << "  if ((tc & 63) == 0) {\n#pragma unroll\n    for (int sr = 0; sr < " << nr << "; ++sr) red[" << base
              << "(sr * " << L.TR << " + tr) * " << W << " + (tc >> 6)] = " << v << "[sr];\n  }\n";
            b << "  __syncthreads();\n";
            b << "#pragma unroll\n  for (int sr = 0; sr < " << nr << "; ++sr) {\n    float m = red[" << base
              << "(sr * " << L.TR << " + tr) * " << W << "];\n";
            b << "#pragma unroll\n    for (int q = 1; q < " << W << "; ++q) m = "
              << comb("m", "red[" + base + "(sr * " + std::to_string(L.TR) + " + tr) * " + std::to_string(W) + " + q]")
              << ";\n    " << v << "[sr] = m;\n  }\n";
          }
          slot_[in.dst] = {i, ko};
          return true;
        }
        // over rows: within the thread, then across the TR threads of the column through LDS
        const VKind ko{false, ks.c};
        const int nc = ks.c ? L.cols() : 1;
        b << "  float " << v << "[" << nc << "];\n";
        b << "#pragma unroll\n  for (int j = 0; j < " << nc << "; ++j) {\n    float m = " << init << ";\n";
        b << "#pragma unroll\n    for (int sr = 0; sr < " << L.SR << "; ++sr) m = "
          << comb("m", s + "[" + idx(ks, "sr", "j") + "]") << ";\n    " << v << "[j] = m;\n  }\n";
        if (L.TR > 1) {
          const std::string base = std::to_string(red_floats_) + " + ";
          red_floats_ += L.threads() * nc;
          ++n_red_;
          b << "#pragma unroll\n  for (int j = 0; j < " << nc << "; ++j) red[" << base << "t * " << nc
            << " + j] = " << v << "[j];\n";
          b << "  __syncthreads();\n";
          b << "#pragma unroll\n  for (int j = 0; j < " << nc << "; ++j) {\n    float m = red[" << base << "tc * "
            << nc << " + j];\n";
          b << "#pragma unroll\n    for (int q = 1; q < " << L.TR << "; ++q) m = "
            << comb("m", "red[" + base + "(q * " + std::to_string(L.TC) + " + tc) * " + std::to_string(nc) + " + j]")
            << ";\n    " << v << "[j] = m;\n  }\n";
        }
        slot_[in.dst] = {i, ko};
        return true;
      }
      default:
        return fail(why, "unsupported op in a fused kernel");
    }
  }

  static bool fail(std::string& why, const char* msg) {
    why = msg;
    return false;
  }

  // vw consecutive elements at `off` -> dst (an expression in e = 0..vw-1)
  // Tiles that move with the block id stream through once: nontemporal loads
  // and stores keep them from displacing what every Block reads (weights).
  bool streamed(int acc) const {
    const TileAddr& o = vm_.access[acc].addr;
    return o.sx != 0 || o.sy != 0 || o.sz != 0;
  }

  void load_code(std::ostringstream& b, int acc, Elem e, int vw, const std::string& dst) const {
    const std::string P = "a.p[" + std::to_string(acc) + "]";
    const bool stream = streamed(acc);
    std::string ty, conv;
    switch (e) {
      case Elem::F32: ty = vw == 4 ? "xf4" : vw == 2 ? "xf2" : "float"; conv = "q"; break;
      case Elem::F16: ty = vw == 4 ? "xh4" : vw == 2 ? "xh2" : "_Float16"; conv = "(float)q"; break;
      case Elem::BF16: ty = vw == 4 ? "xu4" : vw == 2 ? "xu2" : "unsigned short"; conv = "xbf(q)"; break;
      default: ty = vw == 4 ? "xc4" : vw == 2 ? "xc2" : "signed char"; conv = "(float)q"; break;
    }
    const char* base = e == Elem::F32 ? "float" : e == Elem::F16 ? "_Float16" : e == Elem::BF16 ? "unsigned short"
                                                                                                 : "signed char";
    b << "      const " << ty << " qv = " << (stream ? "__builtin_nontemporal_load(" : "*(") << "reinterpret_cast<const "
      << ty << "*>(static_cast<const " << base << "*>(" << P << ") + off));\n";
    if (vw == 1) {
      b << "      { const int e = 0; const auto q = qv; " << dst << " = " << conv << "; }\n";
    } else {
      b << "#pragma unroll\n      for (int e = 0; e < " << vw << "; ++e) { const auto q = qv[e]; " << dst << " = "
        << conv << "; }\n";
    }
  }

  void store_code(std::ostringstream& b, int acc, Elem e, int vw, const std::string& src) const {
    const std::string P = "a.p[" + std::to_string(acc) + "]";
    const bool stream = streamed(acc);
    std::string ty, conv;
    switch (e) {
      case Elem::F32: ty = vw == 4 ? "xf4" : vw == 2 ? "xf2" : "float"; conv = "w"; break;
      case Elem::F16: ty = vw == 4 ? "xu4" : vw == 2 ? "xu2" : "unsigned short"; conv = "xto_f16(w)"; break;
      case Elem::BF16: ty = vw == 4 ? "xu4" : vw == 2 ? "xu2" : "unsigned short"; conv = "xto_bf16(w)"; break;
      default: ty = vw == 4 ? "xc4" : vw == 2 ? "xc2" : "signed char"; conv = "(signed char)xto_i8(w)"; break;
    }
    const char* base = e == Elem::F32 ? "float" : (e == Elem::F16 || e == Elem::BF16) ? "unsigned short"
                                                                                         : "signed char";
    if (vw == 1) {
      b << "      { const int e = 0; const float w = " << src << "; *(static_cast<" << base
        << "*>(" << P << ") + off) = " << conv << "; }\n";
    } else {
      b << "      " << ty << " qv;\n#pragma unroll\n      for (int e = 0; e < " << vw << "; ++e) { const float w = "
        << src << "; qv[e] = " << conv << "; }\n";
      if (stream)
        b << "      __builtin_nontemporal_store(qv, reinterpret_cast<" << ty << "*>(static_cast<" << base << "*>(" << P
          << ") + off));\n";
      else
        b << "      *reinterpret_cast<" << ty << "*>(static_cast<" << base << "*>(" << P << ") + off) = qv;\n";
    }
  }
};

}  // namespace

bool fuse_vm(const VmPlan& vm, const int32_t grid[3], FusedPlan& out, std::string& why, int max_vw) {
  if (vm.access.size() > 8) {
    why = "fused kernels take at most 8 loads and stores";
    return false;
  }
  // values stay in registers, so no load may read what the program stored
  std::vector<int> stored;
  for (const VmInst& in : vm.inst) {
    if (in.op != VmOp::Load && in.op != VmOp::Store) continue;
    const VmAccess& acc = vm.access[in.kind];
    if (in.dims[2] != 1 && acc.stride[2] != 1) {
      why = "fused kernels read and write rows of contiguous elements";
      return false;
    }
    if (in.op == VmOp::Store) stored.push_back(acc.arg);
    else if (std::find(stored.begin(), stored.end(), acc.arg) != stored.end()) {
      why = "fused kernels do not load a memref the program has stored to";
      return false;
    }
  }
  Gen g(vm, grid, max_vw);
  return g.run(out, why);
}

}  // namespace xt
