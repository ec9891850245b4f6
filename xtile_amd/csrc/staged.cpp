// Staged tile programs: the tile interpreter's lowering of a program (VmPlan)
// that the register-resident fused kernel declines - matmul / mma, transposes
// and permutes, values of several shapes - turned into the source of one HIP
// kernel.  The runtime compiles it with hiprtc (kernels/fused_jit.cpp) and
// launches it like a fused kernel.
//
// Execution.  One 256-thread workgroup (four waves) runs one Block.  Values
// live in LDS, as f32 (as the interpreter and the oracle hold them) or, for
// f16 / bf16 tiles as loaded whose every reader is an MFMA operand, as their
// 16-bit patterns; every instruction is straight-line code with its shapes,
// strides and tile origins as compile-time constants, and a barrier (one
// that orders LDS only) separates an instruction from the next one that
// reads what it wrote or writes where it read.  The global reads of a run of
// loads are issued together; the LDS write of a load whose first reader
// comes later waits in registers until that reader (so its LDS is not held
// meanwhile).
//   * matmul / mma: 32 x 32 output tiles dealt over the four waves, K in MFMA
//     steps: v_mfma_f32_32x32x16_f16 / _bf16 when both operands are f16 / bf16
//     tiles as loaded (or transposed / permuted: the values are then exact in
//     that type), v_mfma_i32_32x32x32_i8 with exact i32 sums for the
//     interpreter's exact i8 x i8 products, v_mfma_f32_32x32x2_f32 otherwise;
//     two accumulators (even and odd steps), a ring of fragment sets read
//     ahead of the MFMAs.  The mma accumulator is added to the finished sum,
//     as the interpreter does.  A result whose only reader is a store goes
//     from the accumulators straight to global memory.
//   * a transpose / permute whose every reader is a matmul operand is a view:
//     the matmul reads its source through the permutation.  Other permutes
//     copy, one thread per output element.
//   * reductions along a row: a power-of-two group of lanes per row with a
//     shuffle butterfly; along a column: one thread per column.  A run of
//     row reductions and the elementwise ops around them over one [R, C]
//     tile (a softmax, a normalisation) is one step in registers (a row
//     segment, emit_rows).
//   * elementwise ops: every LDS read of a chunk of elements before its
//     writes, four elements at a time where the layouts allow.
//
// LDS layout.  The generator allocates its own slots (liveness, first fit,
// 16-byte granules): a value of n elements is stored as rows of `krow`
// elements `pitch` apart in the value's row-major element order, so reshapes
// keep their meaning.  krow = pitch = the innermost dim, except for
//   * matmul operands: rows that the lanes of a fragment read side by side
//     (A's rows; the source rows of a transposed view) get a pitch of 4 mod 8
//     floats or 8 mod 16 halves: the 16-byte reads of the narrow types put
//     sixteen rows in sixteen distinct bank groups, and f32's single floats
//     of 32 rows meet at most two to a bank while rows stay float4-aligned
//     for the elementwise ops that write them; B[K, N] read across columns
//     gets 4 mod 8 floats / 8 mod 16 halves for the narrow types (the two
//     half-waves' rows, 8 apart, in distinct banks);
//   * the source of a copying permute: an odd pitch (a column read is
//     conflict-free).
// The first consumer in program order decides.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <map>
#include <sstream>
#include <vector>

#include "fused_common.h"
#include "plan.h"

namespace xt {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxLdsFloats = 160 * 1024 / 4;

enum MmMode { kMmF32 = 0, kMmF16 = 1, kMmBF16 = 2, kMmI8 = 3 };
// what a value is known to hold exactly: any f32, or values of a narrow type
enum VType { kVF32 = 0, kVF16 = 1, kVBF16 = 2, kVI8 = 3 };

struct Val {
  int def = -1, last = -1;  // producing instruction, last reader
  long long numel = 0;
  int dims[3] = {1, 1, 1};  // dims at the definition
  int krow = 0, pitch = 0;  // layout (0: not chosen yet), in elements
  int off = -1;             // LDS offset in floats (-1: no storage)
  int vt = kVF32;
  bool h16 = false;         // held as 16-bit patterns (pitch and offsets in halves)
  int src = -1;             // a view: element (j0, j1, j2) is src's element with index perm[d] = j_d
  int perm[3] = {0, 1, 2};
  int alloc_at = -1;        // the instruction from which it holds LDS (a deferred load: its first reader)
  int gstore = -1;          // a matmul result its only reader, this store, takes from the accumulators
  int alias = -1;           // written in place over this value (an elementwise operand that dies there)
  std::vector<int> users;   // instructions that read it
  long long floats() const {
    const long long e = numel / krow * pitch;
    return h16 ? (e + 1) / 2 : e;
  }
};

struct Reads {
  int a = -1, b = -1, c = -1, dst = -1;  // value ids
  int mode = kMmF32;                     // matmul
};

int pad_to(int k, int mod, int rem) { return k + ((rem - k % mod) % mod + mod) % mod; }

std::string S(long long v) { return std::to_string(v); }

// phys index = base + sr * r + sc * c of a matmul operand viewed as [R, C]
struct Aff {
  bool ok = false;
  int store = -1;  // the value holding the data
  long long base = 0, sr = 0, sc = 0;
};

class StagedGen {
 public:
  StagedGen(const VmPlan& vm, const int32_t grid[3], int max_vw) : vm_(vm), max_vw_(max_vw) {
    for (int d = 0; d < 3; ++d) grid_[d] = grid[d];
  }

  bool run(FusedPlan& out, std::string& why) {
    if (!analyze(why) || !views() || !layouts(why) || !plan_loads() || !allocate(why)) return false;
    earlier_writes();
    if (std::getenv("XTILE_AMD_STAGE_DUMP"))
      for (size_t v = 0; v < vals_.size(); ++v) {
        const Val& w = vals_[v];
        std::fprintf(stderr, "v%zu def=%d last=%d alloc=%d dims=%dx%dx%d krow=%d pitch=%d off=%d h16=%d src=%d alias=%d gstore=%d\n",
                     v, w.def, w.last, w.alloc_at, w.dims[0], w.dims[1], w.dims[2], w.krow, w.pitch, w.off, (int)w.h16,
                     w.src, w.alias, w.gstore);
      }
    std::ostringstream b;
    const int n = static_cast<int>(vm_.inst.size());
    bool any_mm[4] = {false, false, false, false};
    int prev = -1;  // the last instruction that emitted code
    int i = 0;
    auto barrier_before = [&](int next) {
      if (prev < 0) return;
      if (vm_.inst[prev].op == VmOp::Store && vm_.inst[next].op == VmOp::Store) return;
      b << "  xbar();\n";
    };
    while (i < n) {
      const VmInst& in = vm_.inst[i];
      if (in.op == VmOp::Load) {
        // a run of loads: every global read, then the LDS writes that are not deferred
        int j = i, regs = 0;
        while (j < n && vm_.inst[j].op == VmOp::Load) {
          const int r = load_regs(j);
          if (j > i && regs + r > 160) break;
          regs += r;
          ++j;
        }
        barrier_before(i);
        for (int k = i; k < j; ++k) emit_load_read(b, k);
        for (int k = i; k < j; ++k)
          if (!deferred(k)) emit_load_write(b, k);
        prev = j - 1;
        i = j;
        continue;
      }
      const Reads& r = rd_[i];
      const bool silent = (in.op == VmOp::Permute && vals_[r.dst].src >= 0) ||
                          (in.op == VmOp::Store && vals_[r.a].gstore == i);
      if (silent) {
        ++i;
        continue;
      }
      barrier_before(i);
      // the step: instruction i, or the row segment or elementwise chain that starts there
      const int seg = row_segment_end(i);
      const int end = seg > i ? seg
                      : (in.op == VmOp::Unary || in.op == VmOp::Binary) ? ew_chain_end(i)
                                                                         : i;
      // deferred loads written in this step: before their first reader's
      // barrier, or (written in the reader's own step) behind one more
      bool wrote = false;
      for (int k = 0; k < i; ++k)
        if (vm_.inst[k].op == VmOp::Load && deferred(k) && vals_[rd_[k].dst].alloc_at == i) {
          emit_load_write(b, k);
          const auto& us = vals_[rd_[k].dst].users;
          wrote = wrote || *std::min_element(us.begin(), us.end()) <= end;
        }
      if (wrote) b << "  xbar();\n";
      if (seg > i) {
        emit_rows(b, i, end);
        prev = end;
        i = end + 1;
        continue;
      }
      switch (in.op) {
        case VmOp::Store: emit_store(b, i); break;
        case VmOp::Unary:
        case VmOp::Binary: {
          emit_elementwise(b, i, end);
          i = end;  // the run's later instructions are done
          break;
        }
        case VmOp::Reduce: emit_reduce(b, i); break;
        case VmOp::Permute: emit_permute(b, i); break;
        case VmOp::Matmul:
          emit_matmul(b, i);
          any_mm[r.mode] = true;
          break;
        default: why = "staged kernels take the interpreter's instructions"; return false;
      }
      prev = i;
      ++i;
    }
    std::ostringstream k;
    k << "typedef float xf16v __attribute__((ext_vector_type(16)));\n"
      << "typedef int xi16v __attribute__((ext_vector_type(16)));\n"
      << "typedef int xi4v __attribute__((ext_vector_type(4)));\n"
      << "typedef _Float16 xh8 __attribute__((ext_vector_type(8)));\n"
      << "typedef short xs8 __attribute__((ext_vector_type(8)));\n"
      << "typedef __bf16 xb8 __attribute__((ext_vector_type(8)));\n"
      // a workgroup barrier that orders LDS only: the program's global
      // accesses need no ordering between waves (no memref is loaded after
      // the program stores to it), and a load still in flight (a deferred
      // load's registers) is not waited for here
      << "__device__ __forceinline__ void xbar() {\n"
      << "  __builtin_amdgcn_fence(__ATOMIC_RELEASE, \"workgroup\", \"local\");\n"
      << "  __builtin_amdgcn_s_barrier();\n"
      << "  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, \"workgroup\", \"local\");\n}\n";
    k << "extern \"C\" __global__ void __launch_bounds__(" << kThreads << ") xt_fused(FusedArgs a) {\n"
      << "#pragma clang fp contract(off)\n"
      << "  __shared__ __attribute__((aligned(16))) float S[" << std::max(4LL, high_) << "];\n"
      << "  unsigned short* const H = reinterpret_cast<unsigned short*>(S);\n  (void)H;\n"
      << "  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);\n"
      << "  (void)lane; (void)wave;\n"
      << "  const int bid = blockIdx.x;\n"
      << "  const int x = bid % " << grid_[0] << ", y = (bid / " << grid_[0] << ") % " << grid_[1]
      << ", z = bid / " << (long long)grid_[0] * grid_[1] << ";\n"
      << "  (void)x; (void)y; (void)z;\n";
    k << b.str() << "}\n";
    out.source = std::string(fused_preamble()) + k.str();
    out.threads = kThreads;
    out.vw = gvw_max_;
    out.staged = true;
    const long long blocks = (long long)grid_[0] * grid_[1] * grid_[2];
    out.workgroups = static_cast<int>(blocks);
    std::ostringstream lay;
    lay << "staged f32 threads=" << kThreads << " lds=" << high_ * 4 << "B";
    const char* names[4] = {"f32", "f16", "bf16", "i8"};
    std::string mm;
    for (int m = 0; m < 4; ++m)
      if (any_mm[m]) mm += (mm.empty() ? "" : ",") + std::string(names[m]);
    if (!mm.empty()) lay << " mfma=" << mm;
    out.layout = lay.str();
    return true;
  }

 private:
  const VmPlan& vm_;
  int max_vw_ = 4;
  int grid_[3];
  std::vector<Val> vals_;
  std::vector<Reads> rd_;
  long long high_ = 0;
  int gvw_max_ = 1;

  static bool fail(std::string& why, const std::string& msg) {
    why = msg;
    return false;
  }

  int new_val(int def, const int d[3], int vt) {
    Val v;
    v.def = v.last = v.alloc_at = def;
    for (int k = 0; k < 3; ++k) v.dims[k] = d[k];
    v.numel = (long long)d[0] * d[1] * d[2];
    v.vt = vt;
    vals_.push_back(v);
    return static_cast<int>(vals_.size()) - 1;
  }

  static long long prod(const int d[3]) { return (long long)d[0] * d[1] * d[2]; }

  bool analyze(std::string& why) {
    std::map<int, int> cur;  // LDS slot offset of the interpreter -> value id
    rd_.assign(vm_.inst.size(), Reads{});
    for (size_t i = 0; i < vm_.inst.size(); ++i) {
      const VmInst& in = vm_.inst[i];
      Reads& r = rd_[i];
      auto rd = [&](int slot, int& out) {
        auto it = cur.find(slot);
        if (it == cur.end()) return false;
        out = it->second;
        vals_[out].last = static_cast<int>(i);
        vals_[out].users.push_back(static_cast<int>(i));
        return true;
      };
      switch (in.op) {
        case VmOp::Load: {
          const Elem e = vm_.access[in.kind].elem;
          const int vt = e == Elem::F16 ? kVF16 : e == Elem::BF16 ? kVBF16 : e == Elem::I8 ? kVI8 : kVF32;
          r.dst = new_val(static_cast<int>(i), in.dims, vt);
          break;
        }
        case VmOp::Store:
          if (!rd(in.a, r.a)) return fail(why, "store of an unknown value");
          break;
        case VmOp::Unary:
          if (!rd(in.a, r.a)) return fail(why, "unary op of an unknown value");
          r.dst = new_val(static_cast<int>(i), in.dims, in.kind == static_cast<int16_t>(VmUnary::Ftoi) ? kVI8 : kVF32);
          break;
        case VmOp::Binary:
          if (!rd(in.a, r.a) || !rd(in.b, r.b)) return fail(why, "binary op of an unknown value");
          r.dst = new_val(static_cast<int>(i), in.dims, kVF32);
          break;
        case VmOp::Reduce: {
          if (!rd(in.a, r.a)) return fail(why, "reduction of an unknown value");
          if (in.dims[0] != 1) return fail(why, "reductions take rank-2 tiles");
          const bool rows = in.aux[0] == 1;
          const int d[3] = {1, rows ? in.dims[1] : 1, rows ? 1 : in.dims[2]};
          r.dst = new_val(static_cast<int>(i), d, kVF32);
          break;
        }
        case VmOp::Permute: {
          if (!rd(in.a, r.a)) return fail(why, "permute of an unknown value");
          const int d[3] = {in.dims[in.aux[0]], in.dims[in.aux[1]], in.dims[in.aux[2]]};
          r.dst = new_val(static_cast<int>(i), d, vals_[r.a].vt);
          break;
        }
        case VmOp::Matmul: {
          if (!rd(in.a, r.a) || !rd(in.b, r.b) || (in.c >= 0 && !rd(in.c, r.c)))
            return fail(why, "matmul of an unknown value");
          const Val &A = vals_[r.a], &B = vals_[r.b];
          if (in.aux[1]) {
            if (A.vt != kVI8 || B.vt != kVI8) return fail(why, "an exact matmul of values that are not i8 tiles");
            r.mode = kMmI8;
          } else if (A.vt == kVF16 && B.vt == kVF16) {
            r.mode = kMmF16;
          } else if (A.vt == kVBF16 && B.vt == kVBF16) {
            r.mode = kMmBF16;
          } else {
            r.mode = kMmF32;
          }
          const int d[3] = {1, in.dims[1], in.dims[2]};
          r.dst = new_val(static_cast<int>(i), d, kVF32);
          break;
        }
      }
      if (r.dst >= 0) cur[in.dst] = r.dst;
    }
    return true;
  }

  bool is_operand(int inst, int v) const {
    const VmInst& in = vm_.inst[inst];
    return in.op == VmOp::Matmul && (rd_[inst].a == v || rd_[inst].b == v) && rd_[inst].c != v;
  }

  // Permutes read only by matmul operands become views of their source;
  // matmul results read only by one store go to global memory directly.
  bool views() {
    for (size_t i = 0; i < vm_.inst.size(); ++i) {
      const VmInst& in = vm_.inst[i];
      const Reads& r = rd_[i];
      if (in.op == VmOp::Permute) {
        Val& X = vals_[r.dst];
        if (X.users.empty() || vals_[r.a].src >= 0) continue;
        bool all = true;
        for (int u : X.users) all = all && is_operand(u, r.dst);
        if (!all) continue;
        X.src = r.a;
        for (int d = 0; d < 3; ++d) X.perm[d] = in.aux[d];
        Val& Y = vals_[r.a];
        Y.users.erase(std::remove(Y.users.begin(), Y.users.end(), static_cast<int>(i)), Y.users.end());
        for (int u : X.users) Y.users.push_back(u);
        Y.last = Y.users.empty() ? Y.def : *std::max_element(Y.users.begin(), Y.users.end());
      } else if (in.op == VmOp::Matmul) {
        Val& D = vals_[r.dst];
        if (D.users.size() == 1 && vm_.inst[D.users[0]].op == VmOp::Store) D.gstore = D.users[0];
      }
    }
    return true;
  }

  // the value holding v's data (v itself, or a view's source)
  int storage_of(int v) const { return vals_[v].src >= 0 ? vals_[v].src : v; }

  bool layouts(std::string& why) {
    // 16-bit storage: f16 / bf16 loads read only as operands of f16 / bf16 MFMAs
    for (size_t i = 0; i < vm_.inst.size(); ++i)
      if (vm_.inst[i].op == VmOp::Load) {
        Val& v = vals_[rd_[i].dst];
        if ((v.vt != kVF16 && v.vt != kVBF16) || v.users.empty()) continue;
        bool all = true;
        for (int u : v.users) {
          const int m = rd_[u].mode;
          all = all && vm_.inst[u].op == VmOp::Matmul && (m == kMmF16 || m == kMmBF16) &&
                (storage_of(rd_[u].a) == rd_[i].dst || storage_of(rd_[u].b) == rd_[i].dst) &&
                rd_[u].c != rd_[i].dst;
        }
        v.h16 = all;
      }
    for (size_t i = 0; i < vm_.inst.size(); ++i) {
      const VmInst& in = vm_.inst[i];
      const Reads& r = rd_[i];
      if (in.op == VmOp::Matmul) {
        const int M = in.dims[1], K = in.aux[0], N = in.dims[2];
        for (int side = 0; side < 2; ++side) {
          const int vid = side == 0 ? r.a : r.b;
          Val& st = vals_[storage_of(vid)];
          if (st.krow) continue;
          // which storage row the fragment's lanes walk: A's rows (lanes = M),
          // B's columns (lanes = N); through a view, the permuted dim
          bool lanes_on_rows;
          if (vals_[vid].src < 0) {
            lanes_on_rows = side == 0;
            st.krow = side == 0 ? K : N;
          } else {
            const Val& X = vals_[vid];
            // the view's dim that the lanes walk: dim 1 (rows) for A, dim 2 for B
            lanes_on_rows = X.perm[side == 0 ? 1 : 2] == 1;
            st.krow = st.dims[2];
          }
          (void)M;
          if (st.h16) st.pitch = pad_to(st.krow, 16, 8);
          else if (r.mode == kMmF32) st.pitch = lanes_on_rows ? pad_to(st.krow, 8, 4) : st.krow;
          else st.pitch = pad_to(st.krow, 8, 4);
        }
      } else if (in.op == VmOp::Permute && vals_[r.dst].src < 0) {
        Val& src = vals_[r.a];
        if (!src.krow) {
          src.krow = in.dims[2];
          src.pitch = in.dims[2] % 2 ? in.dims[2] : in.dims[2] + 1;
        }
      }
    }
    coalesce();
    for (Val& v : vals_) {
      if (v.alias >= 0) continue;
      if (!v.krow) v.krow = v.pitch = std::max(1, v.dims[2]);
      if (v.numel % v.krow) return fail(why, "staged layout rows do not divide a value");
    }
    for (Val& v : vals_)
      if (v.alias >= 0) {
        const Val& root = vals_[root_of(static_cast<int>(&v - &vals_[0]))];
        v.krow = root.krow;
        v.pitch = root.pitch;
      }
    return true;
  }

  int root_of(int v) const {
    while (vals_[v].alias >= 0) v = vals_[v].alias;
    return v;
  }

  // An elementwise result whose same-shaped operand is last read by that
  // instruction is written in place over it: each thread reads the elements
  // it then writes, at the same indices, and no other thread touches them.
  // The chain of such values shares one slot and one layout (the operand
  // layouts already chosen for any member, which must agree).
  void coalesce() {
    for (size_t i = 0; i < vm_.inst.size(); ++i) {
      const VmInst& in = vm_.inst[i];
      if (in.op != VmOp::Unary && in.op != VmOp::Binary) continue;
      const Reads& r = rd_[i];
      Val& D = vals_[r.dst];
      if (D.gstore >= 0 || D.src >= 0) continue;
      for (int side = 0; side < (in.op == VmOp::Binary ? 2 : 1); ++side) {
        const int xv = side == 0 ? r.a : r.b;
        const int* od = in.op == VmOp::Unary ? in.dims : side == 0 ? in.lhs : in.aux;
        if (od[0] != in.dims[0] || od[1] != in.dims[1] || od[2] != in.dims[2]) continue;  // broadcast
        Val& X = vals_[xv];
        if (X.src >= 0 || X.h16 || X.gstore >= 0 || X.last != static_cast<int>(i) || X.numel != D.numel) continue;
        if (in.op == VmOp::Binary && r.a == r.b) continue;
        // the chain's layout: X's root's, or D's, whichever is set; both set must agree
        const int root = root_of(xv);
        const Val& R = vals_[root];
        if (R.krow && D.krow && (R.krow != D.krow || R.pitch != D.pitch)) continue;
        bool member_has = false;  // another member of X's chain carries a layout
        for (size_t w = 0; w < vals_.size(); ++w)
          if (vals_[w].alias >= 0 && root_of(static_cast<int>(w)) == root && vals_[w].krow &&
              D.krow && (vals_[w].krow != D.krow || vals_[w].pitch != D.pitch))
            member_has = true;
        if (member_has) continue;
        if (!vals_[root].krow && D.krow) {
          vals_[root].krow = D.krow;
          vals_[root].pitch = D.pitch;
        }
        D.alias = xv;
        break;
      }
    }
  }

  bool deferred(int load_inst) const {
    const Val& v = vals_[rd_[load_inst].dst];
    return v.alloc_at > load_inst;
  }

  // A load whose first reader is not the first instruction to run after its
  // run of loads keeps its data in registers until that reader.
  bool plan_loads() {
    const int n = static_cast<int>(vm_.inst.size());
    for (int i = 0; i < n; ++i) {
      if (vm_.inst[i].op != VmOp::Load) continue;
      Val& v = vals_[rd_[i].dst];
      int end = i;
      while (end + 1 < n && vm_.inst[end + 1].op == VmOp::Load) ++end;
      // the first instruction after the run that emits code
      int next = end + 1;
      while (next < n && silent(next)) ++next;
      if (v.users.empty()) {
        // never read: its slot stays reserved until the run's writes are ordered
        v.last = std::min(n - 1, end + 1);
        continue;
      }
      const int first = *std::min_element(v.users.begin(), v.users.end());
      if (first > next) v.alloc_at = first;
    }
    return true;
  }

  // A deferred load written at its first reader costs a barrier of its own.
  // Written during the step before (an instruction that begins a step: not
  // silent, not a load, not the continuation of an in-place elementwise
  // chain), the barrier after that step orders it; kept when the packed LDS
  // does not grow.
  void earlier_writes() {
    const int n = static_cast<int>(vm_.inst.size());
    for (int i = 0; i < n; ++i) {
      if (vm_.inst[i].op != VmOp::Load || !deferred(i)) continue;
      Val& v = vals_[rd_[i].dst];
      const int c = v.alloc_at - 1;
      if (c <= i || silent(c) || vm_.inst[c].op == VmOp::Load) continue;
      const VmInst& ci = vm_.inst[c];
      if ((ci.op == VmOp::Unary || ci.op == VmOp::Binary) && c > 0 &&
          (vm_.inst[c - 1].op == VmOp::Unary || vm_.inst[c - 1].op == VmOp::Binary) &&
          vals_[rd_[c].dst].alias == rd_[c - 1].dst)
        continue;  // c may continue the previous step's chain
      const long long before = high_;
      const int keep_at = v.alloc_at;
      std::vector<int> offs(vals_.size());
      for (size_t w = 0; w < vals_.size(); ++w) offs[w] = vals_[w].off;
      v.alloc_at = c;
      std::string why;
      if (!allocate(why) || high_ > before) {
        v.alloc_at = keep_at;
        for (size_t w = 0; w < vals_.size(); ++w) vals_[w].off = offs[w];
        high_ = before;
      }
    }
  }

  bool silent(int i) const {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    return (in.op == VmOp::Permute && vals_[r.dst].src >= 0) || (in.op == VmOp::Store && vals_[r.a].gstore == i);
  }

  bool allocate(std::string& why) {
    const int n = static_cast<int>(vm_.inst.size());
    // a chain of in-place values holds its root's slot until its last member's last read
    for (size_t v = 0; v < vals_.size(); ++v)
      if (vals_[v].alias >= 0) {
        Val& root = vals_[root_of(static_cast<int>(v))];
        root.last = std::max(root.last, vals_[v].last);
      }
    // Every slot's life [alloc_at, last] is known, so two packings are
    // tried and the smaller kept: first fit in program order, and largest
    // first at the lowest offset clear of every placed slot whose life
    // overlaps (first fit leaves holes that a later, larger slot cannot use).
    std::vector<int> items;
    for (size_t v = 0; v < vals_.size(); ++v) {
      const Val& w = vals_[v];
      if (w.src < 0 && w.gstore < 0 && w.alias < 0 && w.alloc_at >= 0 && w.alloc_at < n) items.push_back(static_cast<int>(v));
    }
    auto size_of = [&](int v) { return (vals_[v].floats() + 3) & ~3LL; };
    auto overlap = [&](int a, int b) { return vals_[a].alloc_at <= vals_[b].last && vals_[b].alloc_at <= vals_[a].last; };
    auto pack = [&](std::vector<int> order, std::vector<long long>& off) {
      off.assign(vals_.size(), -1);
      long long high = 0;
      std::vector<int> placed;
      for (int v : order) {
        const long long fl = size_of(v);
        std::vector<long long> cand = {0};
        for (int p : placed) cand.push_back(off[p] + size_of(p));
        std::sort(cand.begin(), cand.end());
        for (long long at : cand) {
          bool clash = false;
          for (int p : placed)
            if (overlap(v, p) && at < off[p] + size_of(p) && off[p] < at + fl) clash = true;
          if (!clash) {
            off[v] = at;
            break;
          }
        }
        placed.push_back(v);
        high = std::max(high, off[v] + fl);
      }
      return high;
    };
    std::vector<int> by_time = items, by_size = items;
    std::stable_sort(by_time.begin(), by_time.end(), [&](int a, int b) { return vals_[a].alloc_at < vals_[b].alloc_at; });
    std::stable_sort(by_size.begin(), by_size.end(), [&](int a, int b) {
      return size_of(a) != size_of(b) ? size_of(a) > size_of(b) : vals_[a].alloc_at < vals_[b].alloc_at;
    });
    std::vector<long long> off_t, off_s;
    const long long high_t = pack(by_time, off_t), high_s = pack(by_size, off_s);
    const std::vector<long long>& off = high_s < high_t ? off_s : off_t;
    high_ = std::min(high_t, high_s);
    for (int v : items) vals_[v].off = static_cast<int>(off[v]);
    for (size_t v = 0; v < vals_.size(); ++v)
      if (vals_[v].alias >= 0) vals_[v].off = vals_[root_of(static_cast<int>(v))].off;
    if (high_ > kMaxLdsFloats)
      return fail(why, "staged kernel needs " + S((high_ * 4 + 1023) / 1024) + " KB of LDS (at most 160 KB)");
    return true;
  }

  // LDS index (floats, or halves for 16-bit values) of logical element `lin` of a stored value
  std::string phys(const Val& v, const std::string& lin) const {
    const long long base = v.h16 ? 2LL * v.off : v.off;
    if (v.krow == v.pitch) return "(" + S(base) + " + (" + lin + "))";
    return "(" + S(base) + " + (" + lin + ") / " + S(v.krow) + " * " + S(v.pitch) + " + (" + lin + ") % " +
           S(v.krow) + ")";
  }

  // the f32 value of element `lin` of value v (through a view, from its source)
  std::string elem(int vid, const std::string& lin) const {
    const Val& v = vals_[vid];
    if (v.src >= 0) {
      const Val& y = vals_[v.src];
      // lin -> (j0, j1, j2) in v.dims; source index iv[perm[d]] = j_d
      const std::string j[3] = {"((" + lin + ") / " + S((long long)v.dims[1] * v.dims[2]) + ")",
                                "(((" + lin + ") / " + S(v.dims[2]) + ") % " + S(v.dims[1]) + ")",
                                "((" + lin + ") % " + S(v.dims[2]) + ")"};
      std::string iv[3];
      for (int d = 0; d < 3; ++d) iv[v.perm[d]] = j[d];
      return elem(v.src, "(" + iv[0] + " * " + S(y.dims[1]) + " + " + iv[1] + ") * " + S(y.dims[2]) + " + " + iv[2]);
    }
    if (v.h16)
      return v.vt == kVBF16 ? "xbf(H[" + phys(v, lin) + "])"
                            : "(float)__builtin_bit_cast(_Float16, H[" + phys(v, lin) + "])";
    return "S[" + phys(v, lin) + "]";
  }

  // element (r, c) of operand vid viewed as [R, C], as an affine LDS index
  Aff affine(int vid, int R, int C) const {
    Aff f;
    const Val& v = vals_[vid];
    if (v.src < 0) {
      if (v.krow != C) return f;
      f.ok = true;
      f.store = vid;
      f.base = v.h16 ? 2LL * v.off : v.off;
      f.sr = v.pitch;
      f.sc = 1;
      return f;
    }
    const Val& y = vals_[v.src];
    if (v.dims[0] != 1 || v.dims[1] != R || v.dims[2] != C || y.krow != y.dims[2]) return f;
    const long long st[3] = {(long long)y.dims[1] * y.pitch, y.pitch, 1};
    f.ok = true;
    f.store = v.src;
    f.base = y.h16 ? 2LL * y.off : y.off;
    f.sr = st[v.perm[1]];
    f.sc = st[v.perm[2]];
    return f;
  }

  // four consecutive f32 elements from a multiple of 4 stay contiguous and aligned
  static bool vec4(const Val& v) { return !v.h16 && v.krow % 4 == 0 && v.pitch % 4 == 0 && v.off % 4 == 0; }

  std::string origin(const TileAddr& o) const {
    std::ostringstream s;
    s << "(" << o.c0 << "LL";
    if (o.sx) s << " + (long long)x * " << o.sx << "LL";
    if (o.sy) s << " + (long long)y * " << o.sy << "LL";
    if (o.sz) s << " + (long long)z * " << o.sz << "LL";
    s << ")";
    return s.str();
  }

  // global vector width of a load / store: elements along a contiguous row
  int gvw(const VmInst& in) const {
    const VmAccess& acc = vm_.access[in.kind];
    const TileAddr& o = acc.addr;
    for (int w = std::min(4, max_vw_); w > 1; w /= 2) {
      if (in.dims[2] % w || acc.stride[2] != 1) continue;
      if (acc.stride[1] % w || acc.stride[0] % w || o.c0 % w || o.sx % w || o.sy % w || o.sz % w) continue;
      return w;
    }
    return 1;
  }

  // the element loop prologue: `e` the first of vw elements of this
  // thread's q-th group, i0 / i1 / i2 its coordinates in `d`
  void loop_open(std::ostringstream& b, long long n, int vw, const int d[3]) const {
    const long long groups = n / vw, iters = (groups + kThreads - 1) / kThreads;
    b << "#pragma unroll " << (iters <= 8 ? iters : 4) << "\n  for (int q = 0; q < " << iters << "; ++q) {\n"
      << "    const int e = (t + q * " << kThreads << ") * " << vw << ";\n";
    if (groups % kThreads) b << "    if (e < " << n << ") {\n";
    else b << "    {\n";
    b << "    const int i2 = e % " << d[2] << ", i1 = (e / " << d[2] << ") % " << d[1] << ", i0 = e / "
      << (long long)d[1] * d[2] << ";\n    (void)i0; (void)i1; (void)i2;\n";
  }
  static void loop_close(std::ostringstream& b) { b << "    }\n  }\n"; }

  // An element loop in two phases per chunk of CH groups of vw elements:
  // every LDS read of the chunk into registers indexed by j, then every
  // computation and LDS write.  (In one pass the compiler must keep each
  // read behind the previous group's write to the same shared array, and
  // with one wave per SIMD every group then waits out the LDS latency.)
  // `regs` floats a group; `read` / `write` emit a group's code given e,
  // i0, i1, i2 and j.
  long long chunk(long long n, int vw, int regs) const {
    const long long iters = (n / vw + kThreads - 1) / kThreads;
    return std::max(1LL, std::min(iters, (long long)(64 / std::max(1, regs))));
  }
  void two_phase(std::ostringstream& b, long long n, int vw, const int d[3], int regs,
                 const std::function<void(std::ostringstream&)>& read,
                 const std::function<void(std::ostringstream&)>& write) const {
    const long long groups = n / vw, iters = (groups + kThreads - 1) / kThreads;
    const long long CH = chunk(n, vw, regs);
    const long long chunks = (iters + CH - 1) / CH;
    std::string g;
    if (iters % CH) g = "q < " + S(iters);
    if (groups % kThreads) g += std::string(g.empty() ? "" : " && ") + "e < " + S(n);
    if (g.empty()) g = "true";
    b << "#pragma unroll " << (chunks <= 4 ? chunks : 1) << "\n  for (int q0 = 0; q0 < " << iters << "; q0 += " << CH
      << ") {\n";
    for (int phase = 0; phase < 2; ++phase) {
      b << "#pragma unroll\n    for (int j = 0; j < " << CH << "; ++j) {\n      const int q = q0 + j;\n"
        << "      const int e = (t + q * " << kThreads << ") * " << vw << ";\n      if (" << g << ") {\n"
        << "      const int i2 = e % " << d[2] << ", i1 = (e / " << d[2] << ") % " << d[1] << ", i0 = e / "
        << (long long)d[1] * d[2] << ";\n      (void)i0; (void)i1; (void)i2;\n";
      (phase == 0 ? read : write)(b);
      b << "      }\n    }\n";
    }
    b << "  }\n";
  }

  int load_regs(int i) const {
    const VmInst& in = vm_.inst[i];
    const int w = gvw(in);
    return static_cast<int>((prod(in.dims) / w + kThreads - 1) / kThreads * w);
  }

  static const char* gtype(Elem e, int w) {
    switch (e) {
      case Elem::F32: return w == 4 ? "xf4" : w == 2 ? "xf2" : "float";
      case Elem::F16: return w == 4 ? "xh4" : w == 2 ? "xh2" : "_Float16";
      case Elem::BF16: return w == 4 ? "xu4" : w == 2 ? "xu2" : "unsigned short";
      default: return w == 4 ? "xc4" : w == 2 ? "xc2" : "signed char";
    }
  }
  static const char* gbase(Elem e) {
    return e == Elem::F32 ? "float" : e == Elem::F16 ? "_Float16" : e == Elem::BF16 ? "unsigned short" : "signed char";
  }
  static std::string to_f32(Elem e, const std::string& q) {
    return e == Elem::BF16 ? "xbf(" + q + ")" : e == Elem::F32 ? q : "(float)" + q;
  }
  bool streamed(int acc) const {
    const TileAddr& o = vm_.access[acc].addr;
    return o.sx != 0 || o.sy != 0 || o.sz != 0;
  }

  // global reads of load i into registers r<i>: f32 values, or the 16-bit
  // patterns of a value held as 16 bits
  void emit_load_read(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const VmAccess& acc = vm_.access[in.kind];
    const bool h16 = vals_[rd_[i].dst].h16;
    const int w = gvw(in);
    gvw_max_ = std::max(gvw_max_, w);
    const long long n = prod(in.dims);
    const long long iters = (n / w + kThreads - 1) / kThreads;
    const std::string R = "r" + S(i);
    b << "  // load " << i << ": [" << in.dims[0] << "," << in.dims[1] << "," << in.dims[2] << "] of a.p["
      << in.kind << "]" << (h16 ? ", held as 16 bits" : "") << (deferred(i) ? ", written to LDS at its first reader" : "")
      << "\n";
    b << "  " << (h16 ? "unsigned short " : "float ") << R << "[" << iters * w << "];\n  {\n    const long long org = "
      << origin(acc.addr) << ";\n";
    loop_open(b, n, w, in.dims);
    b << "    const long long off = org + (long long)i0 * " << acc.stride[0] << "LL + (long long)i1 * "
      << acc.stride[1] << "LL + (long long)i2 * " << acc.stride[2] << "LL;\n";
    const Elem le = h16 ? Elem::BF16 : acc.elem;  // 16-bit patterns load as unsigned short vectors
    const char* ty = gtype(le, w);
    b << "    const " << ty << " qv = " << (streamed(in.kind) ? "__builtin_nontemporal_load(" : "*(")
      << "reinterpret_cast<const " << ty << "*>(static_cast<const " << gbase(le) << "*>(a.p[" << in.kind
      << "]) + off));\n";
    const std::string conv = h16 ? "qv" : "";
    if (w == 1) b << "    " << R << "[q] = " << (h16 ? "qv" : to_f32(acc.elem, "qv")) << ";\n";
    else
      b << "#pragma unroll\n    for (int c = 0; c < " << w << "; ++c) " << R << "[q * " << w << " + c] = "
        << (h16 ? "qv[c]" : to_f32(acc.elem, "qv[c]")) << ";\n";
    loop_close(b);
    b << "  }\n";
  }

  void emit_load_write(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Val& v = vals_[rd_[i].dst];
    const int w = gvw(in);
    const long long n = prod(in.dims);
    const std::string R = "r" + S(i);
    b << "  {\n";
    loop_open(b, n, w, in.dims);
    if (w == 4 && vec4(v))
      b << "    *reinterpret_cast<xf4*>(&S[" << phys(v, "e") << "]) = xf4{" << R << "[q * 4], " << R
        << "[q * 4 + 1], " << R << "[q * 4 + 2], " << R << "[q * 4 + 3]};\n";
    else if (w == 4 && v.h16 && v.krow % 4 == 0 && v.pitch % 4 == 0)
      b << "    *reinterpret_cast<xu4*>(&H[" << phys(v, "e") << "]) = xu4{" << R << "[q * 4], " << R
        << "[q * 4 + 1], " << R << "[q * 4 + 2], " << R << "[q * 4 + 3]};\n";
    else
      b << "#pragma unroll\n    for (int c = 0; c < " << w << "; ++c) " << (v.h16 ? "H[" : "S[") << phys(v, "e + c")
        << "] = " << R << "[q * " << w << " + c];\n";
    loop_close(b);
    b << "  }\n";
  }

  static std::string store_conv(Elem e, const std::string& f) {
    switch (e) {
      case Elem::F32: return f;
      case Elem::F16: return "xto_f16(" + f + ")";
      case Elem::BF16: return "xto_bf16(" + f + ")";
      default: return "(signed char)xto_i8(" + f + ")";
    }
  }

  void emit_store(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const VmAccess& acc = vm_.access[in.kind];
    const int vid = rd_[i].a;
    const Val& v = vals_[vid];
    const int w = gvw(in);
    gvw_max_ = std::max(gvw_max_, w);
    const long long n = prod(in.dims);
    b << "  // store " << i << ": [" << in.dims[0] << "," << in.dims[1] << "," << in.dims[2] << "] to a.p["
      << in.kind << "]\n  {\n    const long long org = " << origin(acc.addr) << ";\n";
    loop_open(b, n, w, in.dims);
    b << "    const long long off = org + (long long)i0 * " << acc.stride[0] << "LL + (long long)i1 * "
      << acc.stride[1] << "LL + (long long)i2 * " << acc.stride[2] << "LL;\n";
    if (w == 4 && v.src < 0 && vec4(v))
      b << "    const xf4 f = *reinterpret_cast<const xf4*>(&S[" << phys(v, "e") << "]);\n";
    else {
      b << "    float f[" << w << "];\n";
      b << "#pragma unroll\n    for (int c = 0; c < " << w << "; ++c) f[c] = " << elem(vid, "e + c") << ";\n";
    }
    const std::string conv = store_conv(acc.elem, "f[c]");
    const char* base = acc.elem == Elem::F32 ? "float" : acc.elem == Elem::I8 ? "signed char" : "unsigned short";
    const char* ty = acc.elem == Elem::F32 ? gtype(Elem::F32, w) : acc.elem == Elem::I8 ? gtype(Elem::I8, w)
                                                                                          : gtype(Elem::BF16, w);
    if (w == 1) {
      b << "    { const int c = 0; *(static_cast<" << base << "*>(a.p[" << in.kind << "]) + off) = " << conv
        << "; }\n";
    } else {
      b << "    " << ty << " qv;\n#pragma unroll\n    for (int c = 0; c < " << w << "; ++c) qv[c] = " << conv
        << ";\n";
      b << "    " << (streamed(in.kind) ? "__builtin_nontemporal_store(qv, " : "*(") << "reinterpret_cast<" << ty
        << "*>(static_cast<" << base << "*>(a.p[" << in.kind << "]) + off)" << (streamed(in.kind) ? ");" : ") = qv;")
        << "\n";
    }
    loop_close(b);
    b << "  }\n";
  }

  // logical element index of an operand of dims `od` broadcast to the
  // result's (i0, i1, i2)
  static std::string bcast(const int od[3]) {
    std::string i0 = od[0] == 1 ? "0" : "i0", i1 = od[1] == 1 ? "0" : "i1", i2 = od[2] == 1 ? "0" : "i2";
    return "((" + i0 + " * " + S(od[1]) + " + " + i1 + ") * " + S(od[2]) + " + " + i2 + ")";
  }

  // The longest run of elementwise instructions from i in which each one
  // writes in place over the previous one's result (its only reader), with
  // the same shape and element grouping: one loop computes the run in
  // registers, reading the other operands (complete before the run's first
  // barrier) and writing only the last result.
  int ew_chain_end(int i) const {
    int j = i;
    const int w = ew_width(i);
    while (j + 1 < static_cast<int>(vm_.inst.size())) {
      const VmInst& nx = vm_.inst[j + 1];
      if (nx.op != VmOp::Unary && nx.op != VmOp::Binary) break;
      const Val& D = vals_[rd_[j + 1].dst];
      if (D.alias != rd_[j].dst || vals_[rd_[j].dst].users.size() != 1) break;
      if (nx.dims[0] != vm_.inst[i].dims[0] || nx.dims[1] != vm_.inst[i].dims[1] || nx.dims[2] != vm_.inst[i].dims[2])
        break;
      if (ew_width(j + 1) != w) break;
      // a load whose LDS write waits for this reader is written before it, behind a barrier
      bool waits = false;
      for (int k = 0; k <= j; ++k)
        if (vm_.inst[k].op == VmOp::Load && deferred(k) && vals_[rd_[k].dst].alloc_at == j + 1) waits = true;
      if (waits) break;
      ++j;
    }
    return j;
  }

  // elements a thread takes at once: four when every operand that varies
  // along the innermost dim is contiguous there
  int ew_width(int i) const {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    const Val& D = vals_[r.dst];
    const long long n = prod(in.dims);
    const bool bin = in.op == VmOp::Binary;
    const Val& A = vals_[r.a];
    const Val* B = bin ? &vals_[r.b] : nullptr;
    const int* ad = bin ? in.lhs : in.dims;
    const bool v4 = in.dims[2] % 4 == 0 && n % 4 == 0 && vec4(D) && (ad[2] == 1 || (A.src < 0 && vec4(A))) &&
                    (!bin || in.aux[2] == 1 || (B->src < 0 && vec4(*B)));
    return v4 ? 4 : 1;
  }

  // the f32 formula of a unary op; exp is exp2 of x log2(e) on the hardware
  // exp2 (relative error at most |x| 2^-24 plus one ulp: below 5.3e-6 for
  // normal results; results below FLT_MIN may flush to 0)
  static std::string unary_formula(int kind, const std::string& x) {
    if (kind == static_cast<int>(VmUnary::Exp)) return "__builtin_amdgcn_exp2f((" + x + ") * 1.44269504088896340736f)";
    return replace_x(unary_expr(kind), x);
  }

  void emit_elementwise(std::ostringstream& b, int i0, int i1) {
    const VmInst& first = vm_.inst[i0];
    const long long n = prod(first.dims);
    const int w = ew_width(i0);
    const char* ty = w == 4 ? "xf4" : "float";
    b << "  // elementwise " << i0;
    for (int i = i0 + 1; i <= i1; ++i) b << ", " << i;
    b << (i1 > i0 ? " in registers" : "") << "\n  {\n";
    // operands read from LDS: both of the first op's, then the other operand of each later one
    struct Opnd {
      int vid;
      int dims[3];
      std::string name;
    };
    std::vector<Opnd> ops;
    std::vector<std::string> a_of(i1 - i0 + 1), b_of(i1 - i0 + 1);
    for (int i = i0; i <= i1; ++i) {
      const VmInst& in = vm_.inst[i];
      const Reads& r = rd_[i];
      const bool bin = in.op == VmOp::Binary;
      const int* ad = bin ? in.lhs : in.dims;
      const int* bd = in.aux;
      const int k = i - i0;
      auto add = [&](int vid, const int* d) {
        Opnd o;
        o.vid = vid;
        for (int q = 0; q < 3; ++q) o.dims[q] = d[q];
        o.name = "v" + S(ops.size());
        ops.push_back(o);
        return ops.back().name + "[j]";
      };
      const std::string prevv = "t" + S(k - 1);
      if (k == 0) {
        a_of[k] = add(r.a, ad);
        if (bin) b_of[k] = add(r.b, bd);
      } else {
        const int chain = rd_[i - 1].dst;
        a_of[k] = r.a == chain ? prevv : add(r.a, ad);
        if (bin) b_of[k] = r.b == chain ? prevv : add(r.b, bd);
      }
    }
    const int regs = w * static_cast<int>(ops.size());
    const long long ch = chunk(n, w, regs);
    for (const Opnd& o : ops) b << "  " << ty << " " << o.name << "[" << ch << "];\n";
    auto operand = [&](std::ostringstream& o, const Opnd& op) {
      const std::string lin = bcast(op.dims);
      const Val& v = vals_[op.vid];
      if (w == 4 && op.dims[2] != 1)
        o << "      " << op.name << "[j] = *reinterpret_cast<const xf4*>(&S[" << phys(v, lin) << "]);\n";
      else if (w == 4)
        o << "      { const float s1 = " << elem(op.vid, lin) << "; " << op.name << "[j] = xf4{s1, s1, s1, s1}; }\n";
      else
        o << "      " << op.name << "[j] = " << elem(op.vid, lin) << ";\n";
    };
    const Val& D = vals_[rd_[i1].dst];
    two_phase(
        b, n, w, first.dims, regs,
        [&](std::ostringstream& o) {
          for (const Opnd& op : ops) operand(o, op);
        },
        [&](std::ostringstream& o) {
          const int lanes = w;
          o << "      " << ty << " ov;\n#pragma unroll\n      for (int c = 0; c < " << lanes << "; ++c) {\n";
          for (int i = i0; i <= i1; ++i) {
            const VmInst& in = vm_.inst[i];
            const int k = i - i0;
            auto lane = [&](const std::string& x) {
              if (x.rfind("t", 0) == 0) return x;                   // a chain value, already a lane scalar
              return w == 4 ? x + "[c]" : x;                        // an operand register
            };
            std::string expr;
            if (in.op == VmOp::Binary) {
              const char* op = in.kind == 0 ? " + " : in.kind == 1 ? " - " : " * ";
              expr = lane(a_of[k]) + op + lane(b_of[k]);
            } else {
              expr = unary_formula(in.kind, lane(a_of[k]));
            }
            o << "        const float t" << k << " = " << expr << ";\n";
          }
          o << "        " << (w == 4 ? "ov[c]" : "ov") << " = t" << (i1 - i0) << ";\n      }\n";
          if (w == 4) o << "      *reinterpret_cast<xf4*>(&S[" << phys(D, "e") << "]) = ov;\n";
          else o << "      S[" << phys(D, "e") << "] = ov;\n";
        });
    b << "  }\n";
  }

  // A row segment: a run of instructions over one [R, C] tile and its row
  // vectors ([R, 1]), column vectors ([1, C]) and scalars - elementwise ops
  // and reductions along rows, as in a softmax or a normalisation - computed
  // in registers with G lanes a row and CPL = C / G contiguous elements a
  // lane: the segment's inputs are read from LDS once, row reductions
  // combine a lane's elements in order and then the row's lanes by a
  // shuffle butterfly, and only values read after the segment are written
  // back.  One step instead of a barrier-separated step per instruction.
  //
  // Kind of an operand of dims d: 0 the tile, 1 a row vector, 2 a column
  // vector, 3 a scalar, -1 none of them.
  static int seg_kind(const int d[3], int R, int C) {
    if (d[0] != 1) return -1;
    if (d[1] == R && d[2] == C) return 0;
    if (d[1] == R && d[2] == 1) return 1;
    if (d[1] == 1 && d[2] == C) return 2;
    if (d[1] == 1 && d[2] == 1) return 3;
    return -1;
  }
  bool seg_ok(int i, int R, int C) const {
    const VmInst& in = vm_.inst[i];
    if (in.op == VmOp::Reduce) return in.aux[0] == 1 && seg_kind(in.dims, R, C) == 0;
    const int kd = seg_kind(in.dims, R, C);
    if (kd != 0 && kd != 1) return false;
    if (in.op == VmOp::Unary) return true;  // its operand has the result's shape
    if (in.op != VmOp::Binary) return false;
    const int ka = seg_kind(in.lhs, R, C), kb = seg_kind(in.aux, R, C);
    if (ka < 0 || kb < 0) return false;
    return kd == 0 || ((ka == 1 || ka == 3) && (kb == 1 || kb == 3));
  }
  // lanes a row: the fewest that give the 256 threads a row each, with at
  // most 32 elements a lane; 0 when the row does not split evenly
  static int seg_lanes(int R, int C) {
    int G = 1;
    while (G < 64 && ((long long)R * G < kThreads || C / G > 32)) G *= 2;
    return C % G == 0 ? G : 0;
  }
  // The last instruction of the row segment that starts at i (i itself when
  // none does: a segment holds a row reduction and another instruction).
  int row_segment_end(int i) const {
    const VmInst& in = vm_.inst[i];
    int R, C;
    if (in.op == VmOp::Reduce) {
      if (in.aux[0] != 1 || in.dims[0] != 1) return i;
      R = in.dims[1];
      C = in.dims[2];
    } else if ((in.op == VmOp::Unary || in.op == VmOp::Binary) && in.dims[0] == 1) {
      R = in.dims[1];
      C = in.dims[2];
    } else {
      return i;
    }
    if (C < 2 || !seg_ok(i, R, C) || seg_lanes(R, C) == 0) return i;
    const int n = static_cast<int>(vm_.inst.size());
    int end = i;
    while (end + 1 < n && seg_ok(end + 1, R, C)) ++end;
    // a deferred load written inside the segment must not be read there
    for (bool again = true; again && end > i;) {
      again = false;
      for (int k = 0; k < n; ++k) {
        if (vm_.inst[k].op != VmOp::Load || !deferred(k)) continue;
        const Val& v = vals_[rd_[k].dst];
        const int first = *std::min_element(v.users.begin(), v.users.end());
        if (v.alloc_at > i && v.alloc_at <= end && first <= end) {
          end = v.alloc_at - 1;
          again = true;
        }
      }
    }
    // registers: every tile value of the segment, CPL floats each
    const int cpl = C / seg_lanes(R, C);
    int tiles = 0;
    std::vector<int> seen;
    for (int j = i; j <= end; ++j) {
      for (int v : {rd_[j].a, rd_[j].b, rd_[j].dst})
        if (v >= 0 && std::find(seen.begin(), seen.end(), v) == seen.end()) {
          seen.push_back(v);
          if (vals_[v].numel == (long long)R * C && R > 1) ++tiles;
        }
      if (tiles * cpl > 160) {
        end = j - 1;
        break;
      }
    }
    bool has_reduce = false;
    for (int j = i; j <= end; ++j) has_reduce |= vm_.inst[j].op == VmOp::Reduce;
    return has_reduce && end > i ? end : i;
  }

  void emit_rows(std::ostringstream& b, int i0, int i1) {
    const VmInst& first = vm_.inst[i0];
    const int R = first.dims[1], C = first.dims[2];
    const int G = seg_lanes(R, C), cpl = C / G, rows_per = kThreads / G;
    const long long passes = (R + rows_per - 1) / rows_per;
    b << "  // rows " << i0 << "-" << i1 << ": " << G << " lanes a row of [" << R << "," << C << "], " << cpl
      << " elements a lane, in registers\n  {\n";
    b << "    const int g = t % " << G << ", r0 = t / " << G << ", c0 = g * " << cpl << ";\n";
    b << "#pragma unroll 1\n    for (int p = 0; p < " << passes << "; ++p) {\n      const int r = r0 + p * "
      << rows_per << ";\n";
    b << (R % rows_per ? "      if (r < " + S(R) + ") {\n" : "      {\n");
    // register names: tiles and column vectors arrays of cpl, row vectors and scalars one float
    std::map<int, std::string> name;
    std::map<int, int> kind;
    auto defined_here = [&](int v) { return vals_[v].def >= i0 && vals_[v].def <= i1; };
    auto in_name = [&](int v, const int* d) -> std::string {
      auto it = name.find(v);
      if (it != name.end()) return it->second;
      const int k = seg_kind(d, R, C);
      const std::string nm = "w" + S(v);
      name[v] = nm;
      kind[v] = k;
      const Val& V = vals_[v];
      if (k == 0 || k == 2) {
        const std::string lin0 = k == 0 ? "r * " + S(C) + " + c0" : "c0";
        b << "        float " << nm << "[" << cpl << "];\n";
        if (cpl % 4 == 0 && V.src < 0 && vec4(V))
          b << "#pragma unroll\n        for (int c = 0; c < " << cpl << "; c += 4) {\n          const xf4 q4 = "
            << "*reinterpret_cast<const xf4*>(&S[" << phys(V, lin0 + " + c") << "]);\n          " << nm << "[c] = q4[0]; "
            << nm << "[c + 1] = q4[1]; " << nm << "[c + 2] = q4[2]; " << nm << "[c + 3] = q4[3];\n        }\n";
        else
          b << "#pragma unroll\n        for (int c = 0; c < " << cpl << "; ++c) " << nm << "[c] = "
            << elem(v, lin0 + " + c") << ";\n";
      } else {
        b << "        const float " << nm << " = " << elem(v, k == 1 ? "r" : "0") << ";\n";
      }
      return nm;
    };
    // inputs first: every LDS read of the pass before any write
    for (int i = i0; i <= i1; ++i) {
      const VmInst& in = vm_.inst[i];
      const Reads& r = rd_[i];
      const int* ad = in.op == VmOp::Binary ? in.lhs : in.dims;
      if (!defined_here(r.a)) in_name(r.a, ad);
      if (in.op == VmOp::Binary && !defined_here(r.b)) in_name(r.b, in.aux);
    }
    auto at = [&](int v, const std::string& c) {
      const std::string& nm = name.at(v);
      return kind.at(v) == 0 || kind.at(v) == 2 ? nm + "[" + c + "]" : nm;
    };
    for (int i = i0; i <= i1; ++i) {
      const VmInst& in = vm_.inst[i];
      const Reads& r = rd_[i];
      const std::string nm = "w" + S(r.dst);
      if (in.op == VmOp::Reduce) {
        const bool mx = in.kind == 1;
        auto comb = [&](const std::string& p, const std::string& q) {
          return mx ? "fmaxf(" + p + ", " + q + ")" : p + " + " + q;
        };
        b << "        float " << nm << " = " << (mx ? "-__builtin_huge_valf()" : "0.0f") << ";\n"
          << "#pragma unroll\n        for (int c = 0; c < " << cpl << "; ++c) " << nm << " = "
          << comb(nm, at(r.a, "c")) << ";\n";
        for (int o = G / 2; o > 0; o /= 2)
          b << "        " << nm << " = " << comb(nm, "__shfl_xor(" + nm + ", " + S(o) + ", " + S(G) + ")") << ";\n";
        name[r.dst] = nm;
        kind[r.dst] = 1;
        continue;
      }
      const int kd = seg_kind(in.dims, R, C);
      std::string expr;
      auto fx = [&](const std::string& c) {
        if (in.op == VmOp::Binary) {
          const char* op = in.kind == 0 ? " + " : in.kind == 1 ? " - " : " * ";
          return at(r.a, c) + op + at(r.b, c);
        }
        return unary_formula(in.kind, at(r.a, c));
      };
      if (kd == 0)
        b << "        float " << nm << "[" << cpl << "];\n#pragma unroll\n        for (int c = 0; c < " << cpl
          << "; ++c) " << nm << "[c] = " << fx("c") << ";\n";
      else
        b << "        const float " << nm << " = " << fx("0") << ";\n";
      name[r.dst] = nm;
      kind[r.dst] = kd == 0 ? 0 : 1;
    }
    // values read after the segment go back to LDS
    for (int i = i0; i <= i1; ++i) {
      const int v = rd_[i].dst;
      const Val& D = vals_[v];
      bool later = false;
      for (int u : D.users) later |= u > i1;
      if (!later) continue;
      const std::string& nm = name.at(v);
      if (kind.at(v) == 0) {
        const std::string lin0 = "r * " + S(C) + " + c0";
        if (cpl % 4 == 0 && vec4(D))
          b << "#pragma unroll\n        for (int c = 0; c < " << cpl << "; c += 4) *reinterpret_cast<xf4*>(&S["
            << phys(D, lin0 + " + c") << "]) = xf4{" << nm << "[c], " << nm << "[c + 1], " << nm << "[c + 2], " << nm
            << "[c + 3]};\n";
        else
          b << "#pragma unroll\n        for (int c = 0; c < " << cpl << "; ++c) S[" << phys(D, lin0 + " + c") << "] = "
            << nm << "[c];\n";
      } else {
        b << "        if (g == 0) S[" << phys(D, "r") << "] = " << nm << ";\n";
      }
    }
    b << "      }\n    }\n  }\n";
    // deferred loads whose slot opens inside the segment (their readers come
    // after it): written now, behind a barrier when the slot overlaps
    // anything the segment read from LDS
    bool fenced = false;
    for (int k = 0; k < i0; ++k) {
      if (vm_.inst[k].op != VmOp::Load || !deferred(k)) continue;
      const Val& L = vals_[rd_[k].dst];
      if (L.alloc_at <= i0 || L.alloc_at > i1) continue;
      const long long lo = L.off, hi = L.off + L.floats();
      bool overlap = false;
      for (const auto& kv : name) {
        if (defined_here(kv.first)) continue;
        const Val& V = vals_[storage_of(kv.first)];
        if (V.off < hi && lo < V.off + V.floats()) overlap = true;
      }
      if (overlap && !fenced) {
        b << "  xbar();\n";
        fenced = true;
      }
      emit_load_write(b, k);
    }
  }

  void emit_reduce(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    const Val &A = vals_[r.a], &D = vals_[r.dst];
    const int R = in.dims[1], C = in.dims[2];
    const bool mx = in.kind == 1;
    const std::string init = mx ? "-__builtin_huge_valf()" : "0.0f";
    auto comb = [&](const std::string& p, const std::string& q) {
      return mx ? "fmaxf(" + p + ", " + q + ")" : p + " + " + q;
    };
    b << "  // reduce " << i << " over axis " << in.aux[0] << " of [" << R << "," << C << "]\n  {\n";
    if (in.aux[0] == 1) {
      // G lanes a row, G the smallest power of two that gives every thread
      // a row (at most 64, at most the row length): each lane combines its
      // share of the row in registers (float4 chunks g, g + G, ... when the
      // row allows), then log2(G) shuffle steps; rows beyond the 256
      // threads' first pass run in further passes, unrolled so that their
      // read and shuffle chains overlap.
      int G = 1;
      while (G < 64 && G * 2 <= C && (long long)R * G < kThreads) G *= 2;
      const int rows_per = kThreads / G;
      const long long passes = (R + rows_per - 1) / rows_per;
      const bool v4 = C % (4 * G) == 0 && A.src < 0 && vec4(A);
      const long long per = v4 ? C / (4 * G) : (C + G - 1) / G;
      b << "    const int g = t % " << G << ", r0 = t / " << G << ";\n";
      b << "#pragma unroll " << (passes <= 8 ? passes : 4) << "\n    for (int p = 0; p < " << passes << "; ++p) {\n"
        << "      const int r = r0 + p * " << rows_per << ";\n      float m = " << init << ";\n";
      if (R % rows_per) b << "      if (r < " << R << ") {\n";
      else b << "      {\n";
      b << "#pragma unroll " << (per <= 16 ? per : 8) << "\n        for (int j = 0; j < " << per << "; ++j) {\n";
      if (v4) {
        b << "          const xf4 q4 = *reinterpret_cast<const xf4*>(&S["
          << phys(A, "r * " + S(C) + " + 4 * (g + j * " + S(G) + ")") << "]);\n";
        b << "          m = " << comb(comb(comb(comb("m", "q4[0]"), "q4[1]"), "q4[2]"), "q4[3]") << ";\n";
      } else {
        b << "          const int c = g + j * " << G << ";\n";
        if (C % G) b << "          if (c < " << C << ") m = " << comb("m", elem(r.a, "r * " + S(C) + " + c")) << ";\n";
        else b << "          m = " << comb("m", elem(r.a, "r * " + S(C) + " + c")) << ";\n";
      }
      b << "        }\n      }\n";
      for (int o = G / 2; o > 0; o /= 2)
        b << "      m = " << comb("m", "__shfl_xor(m, " + S(o) + ", " + S(G) + ")") << ";\n";
      b << "      if (g == 0" << (R % rows_per ? " && r < " + S(R) : "") << ") S[" << phys(D, "r") << "] = m;\n";
      b << "    }\n";
    } else {
      const long long iters = (C + kThreads - 1) / kThreads;
      b << "#pragma unroll\n    for (int q = 0; q < " << iters << "; ++q) {\n      const int c = t + q * " << kThreads
        << ";\n";
      if (C % kThreads) b << "      if (c < " << C << ") {\n";
      else b << "      {\n";
      b << "        float m = " << init << ";\n#pragma unroll 8\n        for (int rr = 0; rr < " << R
        << "; ++rr) m = " << comb("m", elem(r.a, "rr * " + S(C) + " + c")) << ";\n        S[" << phys(D, "c")
        << "] = m;\n      }\n    }\n";
    }
    b << "  }\n";
  }

  void emit_permute(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    const Val& D = vals_[r.dst];
    const int od[3] = {in.dims[in.aux[0]], in.dims[in.aux[1]], in.dims[in.aux[2]]};
    const long long n = prod(in.dims);
    b << "  // permute " << i << "\n  {\n";
    // output (i0, i1, i2) = input index with dim perm[d] at i_d
    const std::string src = "(iv[0] * " + S(in.dims[1]) + " + iv[1]) * " + S(in.dims[2]) + " + iv[2]";
    b << "  float pv[" << chunk(n, 1, 1) << "];\n";
    two_phase(
        b, n, 1, od, 1,
        [&](std::ostringstream& o) {
          o << "      int iv[3];\n      iv[" << in.aux[0] << "] = i0;\n      iv[" << in.aux[1] << "] = i1;\n      iv["
            << in.aux[2] << "] = i2;\n      pv[j] = " << elem(r.a, src) << ";\n";
        },
        [&](std::ostringstream& o) { o << "      S[" << phys(D, "e") << "] = pv[j];\n"; });
    b << "  }\n";
  }

  void emit_matmul(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    const Val& D = vals_[r.dst];
    const int M = in.dims[1], N = in.dims[2], K = in.aux[0];
    const int mode = r.mode;
    // K elements per step and per lane.  An f32 step is four MFMAs of K = 2:
    // lane half h takes k = 8 s + 4 h + j into MFMA j (the order of the sum
    // over k is free, and A and B use the same order), so a lane reads its A
    // row's four floats with one 16-byte read (conflict-free at A's pitch of
    // 4 mod 8 floats) instead of four single floats.
    const int KB = mode == kMmF32 ? 8 : mode == kMmI8 ? 32 : 16, KL = KB / 2;
    const int MT = (M + 31) / 32, NT = (N + 31) / 32, steps = (K + KB - 1) / KB;
    const bool mg = M % 32 != 0, ng = N % 32 != 0, kg = K % KB != 0;
    const bool narrow = mode == kMmF16 || mode == kMmBF16;
    b << "  // matmul " << i << ": [" << M << "," << K << "] x [" << K << "," << N << "]" << (r.c >= 0 ? " + acc" : "")
      << ", " << (mode == kMmF32 ? "f32" : mode == kMmF16 ? "f16" : mode == kMmBF16 ? "bf16" : "i8") << " MFMA"
      << (D.gstore >= 0 ? ", result stored to global memory" : "") << "\n  {\n";
    b << "    const int l32 = lane & 31, h = lane >> 5;\n";
    b << "    for (int u = wave; u < " << MT * NT << "; u += 4) {\n"
      << "      const int row = (u / " << NT << ") * 32 + l32, col = (u % " << NT << ") * 32 + l32;\n";
    // two accumulators, even and odd K steps: consecutive MFMAs are then
    // independent and issue back to back; their sum is the tile's (exact for i8)
    b << "      " << (mode == kMmI8 ? "xi16v" : "xf16v") << " acc0 = {}, acc1 = {};\n";
    // Operand fragments of K step `st` into set p: a lane takes KL elements
    // along K at its row of A (lane = row) / its column of B (lane = column).
    // Narrow modes keep the 16-bit patterns (fa<p> / fb<p> as xs8), the
    // others f32 values.
    const Aff fa = affine(r.a, M, K), fb = affine(r.b, K, N);
    auto frag = [&](int vid, const Aff& af, bool is_a, const std::string& name) -> std::string {
      std::ostringstream o;
      const std::string lanev = is_a ? "row" : "col";  // the lane's row of A / column of B
      const int lim = is_a ? M : N;
      const bool lg = is_a ? mg : ng;
      std::string cond;
      if (lg) cond = lanev + " < " + S(lim);
      const Val& st = vals_[af.ok ? af.store : storage_of(vid)];
      // contiguous along K: one vector read of KL elements
      const long long sk = af.ok ? (is_a ? af.sc : af.sr) : 0, sl = af.ok ? (is_a ? af.sr : af.sc) : 0;
      const int esz = st.h16 ? 2 : 4;
      const bool vec = af.ok && sk == 1 && !kg && (af.base * esz) % 16 == 0 && (sl * esz) % 16 == 0 &&
                       (KL * esz) % 16 == 0 && (narrow ? st.h16 || KL % 4 == 0 : KL % 4 == 0) &&
                       (mode != kMmI8 && mode != kMmF32 ? true : !st.h16);
      const std::string idx0 = S(af.base) + " + " + S(sl) + " * " + lanev + " + " + S(sk) + " * k0";
      if (vec && st.h16) {
        o << "            " << name << " = " << (cond.empty() ? "" : "(" + cond + ") ? ")
          << "*reinterpret_cast<const xs8*>(&H[" << idx0 << "])" << (cond.empty() ? "" : " : xs8{}") << ";\n";
        return o.str();
      }
      if (vec) {  // f32 storage, KL a multiple of 4
        o << "            {\n";
        for (int q = 0; q < KL / 4; ++q)
          o << "              const xf4 q" << q << " = " << (cond.empty() ? "" : "(" + cond + ") ? ")
            << "*reinterpret_cast<const xf4*>(&S[" << idx0 << " + " << 4 * q << "])"
            << (cond.empty() ? "" : " : xf4{}") << ";\n";
        for (int j = 0; j < KL; ++j) {
          const std::string f = "q" + S(j / 4) + "[" + S(j % 4) + "]";
          if (mode == kMmF16)
            o << "              " << name << "[" << j << "] = __builtin_bit_cast(short, (_Float16)" << f << ");\n";
          else if (mode == kMmBF16)
            o << "              " << name << "[" << j << "] = (short)(__float_as_uint(" << f << ") >> 16);\n";
          else
            o << "              " << name << "[" << j << "] = " << f << ";\n";
        }
        o << "            }\n";
        return o.str();
      }
      // element by element (a view or layout that is not affine, a partial K step)
      std::string c2 = cond;
      if (kg) c2 += (c2.empty() ? "" : " && ") + std::string("k < ") + S(K);
      o << "#pragma unroll\n            for (int j = 0; j < " << KL << "; ++j) {\n              const int k = k0 + j;\n";
      const std::string lin = is_a ? "row * " + S(K) + " + k" : "k * " + S(N) + " + col";
      std::string val;
      const bool raw16 = af.ok && st.h16;  // val is a 16-bit pattern, not an f32 value
      if (raw16) val = "H[" + S(af.base) + " + " + S(sl) + " * " + lanev + " + " + S(sk) + " * k]";
      else if (af.ok) val = "S[" + S(af.base) + " + " + S(sl) + " * " + lanev + " + " + S(sk) + " * k]";
      else val = elem(vid, lin);
      if (narrow) {
        std::string bits;
        if (raw16) bits = "(short)" + val;
        else if (mode == kMmF16) bits = "__builtin_bit_cast(short, (_Float16)" + val + ")";
        else bits = "(short)(__float_as_uint(" + val + ") >> 16)";
        o << "              " << name << "[j] = " << (c2.empty() ? bits : "(" + c2 + ") ? " + bits + " : (short)0")
          << ";\n";
      } else {
        o << "              " << name << "[j] = " << (c2.empty() ? val : "(" + c2 + ") ? " + val + " : 0.0f") << ";\n";
      }
      o << "            }\n";
      return o.str();
    };
    auto read = [&](const std::string& st, int p) -> std::string {
      std::ostringstream o;
      o << "        {\n          const int k0 = (" << st << ") * " << KB << " + h * " << KL << ";\n"
        << frag(r.a, fa, true, "fa" + S(p)) << frag(r.b, fb, false, "fb" + S(p)) << "        }\n";
      return o.str();
    };
    auto mfma = [&](int p) -> std::string {
      std::ostringstream o;
      const std::string FA = "fa" + S(p), FB = "fb" + S(p);
      const std::string acc = "acc" + S(p % 2);
      switch (mode) {
        case kMmF32:
          for (int j = 0; j < KL; ++j)
            o << "        acc" << j % 2 << " = __builtin_amdgcn_mfma_f32_32x32x2f32(" << FA << "[" << j << "], " << FB
              << "[" << j << "], acc" << j % 2 << ", 0, 0, 0);\n";
          break;
        case kMmF16:
          o << "        " << acc << " = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(xh8, " << FA
            << "), __builtin_bit_cast(xh8, " << FB << "), " << acc << ", 0, 0, 0);\n";
          break;
        case kMmBF16:
          o << "        " << acc << " = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(xb8, " << FA
            << "), __builtin_bit_cast(xb8, " << FB << "), " << acc << ", 0, 0, 0);\n";
          break;
        default:
          o << "        {\n          xi4v ia, ib;\n#pragma unroll\n          for (int j = 0; j < 4; ++j) {\n";
          for (const char* F : {"ia", "ib"}) {
            const std::string X = std::string(F) == "ia" ? FA : FB;
            o << "            " << F << "[j] = (int)((unsigned)((int)" << X << "[4 * j] & 255) | ((unsigned)((int)"
              << X << "[4 * j + 1] & 255) << 8) | ((unsigned)((int)" << X << "[4 * j + 2] & 255) << 16) | "
              << "((unsigned)((int)" << X << "[4 * j + 3] & 255) << 24));\n";
          }
          o << "          }\n          " << acc << " = __builtin_amdgcn_mfma_i32_32x32x32_i8(ia, ib, " << acc
            << ", 0, 0, 0);\n        }\n";
          break;
      }
      return o.str();
    };
    // A ring of NS fragment sets: the reads of steps s + 1 .. s + NS - 1 are
    // in flight while step s's MFMAs run.  The loop runs the
    // groups of NS steps whose look-ahead reads stay within K, with no branch
    // in its body (the compiler waits for every LDS read at a block
    // boundary); the last steps follow unrolled, reading ahead only while
    // steps remain.  Scheduling fences keep each step's look-ahead reads
    // ahead of its MFMA (left alone, the compiler sinks them next to their
    // use).  NS is even, so set j always holds steps of parity j % 2.
    int NS = std::max(1, std::min(steps, 4));
    if (NS > 1 && NS % 2) --NS;
    for (int q = 0; q < NS; ++q) {
      if (narrow) b << "      xs8 fa" << q << ", fb" << q << ";\n";
      else b << "      float fa" << q << "[" << KL << "], fb" << q << "[" << KL << "];\n";
    }
    const std::string fence = "        __builtin_amdgcn_sched_barrier(0);\n";
    if (NS == 1) {
      b << "#pragma unroll 1\n      for (int s = 0; s < " << steps << "; ++s) {\n" << read("s", 0) << fence << mfma(0)
        << fence << "      }\n";
    } else {
      for (int q = 0; q + 1 < NS; ++q) b << read(S(q), q);
      // groups starting at s read up to step s + 2 NS - 2
      const int groups = steps >= 2 * NS - 1 ? (steps - (2 * NS - 1)) / NS + 1 : 0;
      if (groups > 0) {
        b << "#pragma unroll 1\n      for (int s = 0; s < " << groups * NS << "; s += " << NS << ") {\n";
        for (int j = 0; j < NS; ++j)
          b << read("s + " + S(j + NS - 1), (j + NS - 1) % NS) << fence << mfma(j) << fence;
        b << "      }\n";
      }
      for (int t = groups * NS; t < steps; ++t) {
        if (t + NS - 1 < steps) b << read(S(t + NS - 1), (t + NS - 1) % NS);
        b << fence << mfma(t % NS) << fence;
      }
    }
    b << "      const auto acc = acc0 + acc1;\n";
    // D: lane l holds column col; register v holds row 8 (v / 4) + 4 h + v % 4 of the tile
    b << "#pragma unroll\n      for (int v = 0; v < 16; ++v) {\n"
      << "        const int rr = (u / " << NT << ") * 32 + 8 * (v >> 2) + 4 * h + (v & 3);\n";
    std::string cond;
    if (mg) cond = "rr < " + S(M);
    if (ng) cond += (cond.empty() ? "" : " && ") + std::string("col < ") + S(N);
    b << "        " << (cond.empty() ? "{" : "if (" + cond + ") {") << "\n";
    b << "          float o = " << (mode == kMmI8 ? "(float)acc[v]" : "acc[v]") << ";\n";
    if (r.c >= 0) b << "          o = o + " << elem(r.c, "rr * " + S(N) + " + col") << ";\n";
    if (D.gstore >= 0) {
      // element (rr, col) is the store's element rr * N + col of its own dims
      const VmInst& st = vm_.inst[D.gstore];
      const VmAccess& acc = vm_.access[st.kind];
      const char* base = acc.elem == Elem::F32 ? "float" : acc.elem == Elem::I8 ? "signed char" : "unsigned short";
      b << "          const int e = rr * " << N << " + col;\n"
        << "          const int i2 = e % " << st.dims[2] << ", i1 = (e / " << st.dims[2] << ") % " << st.dims[1]
        << ", i0 = e / " << (long long)st.dims[1] * st.dims[2] << ";\n"
        << "          const long long off = " << origin(acc.addr) << " + (long long)i0 * " << acc.stride[0]
        << "LL + (long long)i1 * " << acc.stride[1] << "LL + (long long)i2 * " << acc.stride[2] << "LL;\n";
      const std::string dst = "static_cast<" + std::string(base) + "*>(a.p[" + S(st.kind) + "]) + off";
      if (streamed(st.kind)) b << "          __builtin_nontemporal_store(" << store_conv(acc.elem, "o") << ", " << dst << ");\n";
      else b << "          *(" << dst << ") = " << store_conv(acc.elem, "o") << ";\n";
    } else {
      b << "          S[" << phys(D, "rr * " + S(N) + " + col") << "] = o;\n";
    }
    b << "        }\n      }\n    }\n  }\n";
  }
};

}  // namespace

bool stage_vm(const VmPlan& vm, const int32_t grid[3], FusedPlan& out, std::string& why, int max_vw) {
  if (vm.access.size() > 8) {
    why = "staged kernels take at most 8 loads and stores";
    return false;
  }
  // a load must not read what the program stored (global writes are not
  // ordered before later reads of the workgroup)
  std::vector<int> stored;
  for (const VmInst& in : vm.inst) {
    if (in.op != VmOp::Load && in.op != VmOp::Store) continue;
    const int arg = vm.access[in.kind].arg;
    if (in.op == VmOp::Store) stored.push_back(arg);
    else if (std::find(stored.begin(), stored.end(), arg) != stored.end()) {
      why = "staged kernels do not load a memref the program has stored to";
      return false;
    }
  }
  const long long blocks = (long long)grid[0] * grid[1] * grid[2];
  if (blocks < 1 || blocks > 0x7fffffffLL) {
    why = "staged kernel grid out of range";
    return false;
  }
  StagedGen g(vm, grid, max_vw);
  return g.run(out, why);
}

}  // namespace xt
