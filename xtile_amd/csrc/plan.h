// Launch planner: recognises the tile program of an `xt` function and turns
// it into a kernel descriptor for the HIP runtime.  Host-only (no HIP types),
// so the matcher and its error paths are testable without a GPU.
//
// Tile addressing follows the reference lowering: a tile at tile coordinate c
// of shape S starts at element offset c * S (lib/xt/XTToNova.cpp:82-101).  A
// load with `shared = k` takes the value of the first block of its sharing
// group, which equals evaluating its coordinates with block-id axes < k set
// to 0 (lib/xt/XTSerialize.cpp:86-101).  Because every coordinate is either a
// block id or a constant, the element offset of a tile origin is affine in the
// block id: off(x, y, z) = c0 + x*sx + y*sy + z*sz.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "ir.h"

namespace xt {

// Element offset of a tile origin as a function of the block id.
struct TileAddr {
  int64_t c0 = 0, sx = 0, sy = 0, sz = 0;
};

// One tile access (load or store) against a memref argument, viewed as a
// 2-D strided block: `rows` rows of `cols` contiguous elements, row pitch `ld`.
struct Access2D {
  int arg = -1;
  Elem elem = Elem::None;
  TileAddr addr;
  int64_t rows = 0, cols = 0, ld = 0;
  int shared = 0;
};

// Tile coordinate source: a block-id axis (0..2) or a constant.
struct Coord {
  int axis = -1;  // -1: constant
  int64_t value = 0;
};

enum class PlanKind { EwBinary, RowSoftmax, Gemm, Conv2d, TileVM, Fused };
enum class EwOp { Add = 0, Sub = 1, Mul = 2 };

struct ConvPlan {
  int src_arg = -1, filt_arg = -1, out_arg = -1;
  Elem elem = Elem::None;                 // source / filter element type
  int64_t N = 0, H = 0, W = 0, C = 0;     // source memref
  int64_t KH = 0, KW = 0, CO = 0;         // filter
  int64_t TB = 0, TH = 0, TW = 0, TC = 0; // output tile per block (TC <= CO: the first TC channels)
  Elem out_elem = Elem::F32;              // result / output element type (f32 or bf16)
  int64_t pad_top = 0, pad_left = 0, stride_h = 1, stride_w = 1, dil_h = 1, dil_w = 1;
  Coord cb, ch, cw;                       // conv tile coordinates (batch, row, col)
  TileAddr filt_addr;                     // filter tile origin
  TileAddr out_addr;                      // stored tile origin in the output
  int64_t out_H = 0, out_W = 0, out_C = 0;  // output memref dims 1..3
};

// General tile programs (anything without conv that the specialised kernels
// do not take): the Block's ops become a straight-line list of tile
// instructions over LDS slots, run by one workgroup per Block
// (kernels/tilevm.hip).  Values are held as f32 whatever their element type.
// Shapes are padded to rank 3 with leading 1s.
enum class VmOp : int16_t { Load, Store, Unary, Binary, Reduce, Permute, Matmul };
enum class VmUnary : int16_t { Exp, Cos, Sin, Recip, Rsqrt, Sigmoid, Tanh, Silu, Ftoi };
enum class VmBinary : int16_t { Add, Sub, Mul };
enum class VmReduce : int16_t { Sum, Max };

struct VmAccess {                 // a load or store tile against a memref argument
  int arg = -1;
  Elem elem = Elem::F32;          // memref element type (converted at the access)
  TileAddr addr;                  // tile origin (element offset), affine in the block id
  int64_t stride[3] = {0, 0, 0};  // memref element strides of the tile's dims
};

struct VmInst {
  VmOp op = VmOp::Load;
  int16_t kind = 0;               // VmUnary / VmBinary / VmReduce, or the access index
  int dst = 0, a = 0, b = 0;      // LDS float offsets of the operands' slots
  int c = -1;                     // Matmul: slot of the mma accumulator, -1 for none
  int dims[3] = {1, 1, 1};        // result dims (Reduce, Permute: source dims)
  int aux[3] = {1, 1, 1};         // Binary: rhs dims; Reduce: axis in aux[0]; Permute: perm;
                                  // Matmul: K, exact i32 sums (0/1), unused
  int lhs[3] = {1, 1, 1};         // Binary: lhs dims
};

struct VmPlan {
  std::vector<VmAccess> access;
  std::vector<VmInst> inst;
  int lds_floats = 0;             // LDS slots, in floats
};

// A tile program compiled for itself (fused.cpp): the tile interpreter's
// lowering (VmPlan) turned into the source of one HIP kernel with every value
// in registers, compiled at run time by hiprtc.  The kernel `xt_fused` takes
// one argument: the memref pointers of the VmPlan's accesses, in order.
struct FusedPlan {
  std::string source;
  int threads = 0;
  int vw = 1;                // vector width of the row accesses (elements)
  int workgroups = 0;        // launch size: one per Block, or fewer walking the Blocks
  std::string layout;        // for describe()
  std::string code;          // the gfx950 code object (filled by the runtime's compile)
  uint64_t id = 0;           // hash of `source` (filled with `code`), keys the loaded kernels
  // the same program with scalar row accesses (vw = 1), built and compiled by
  // the first launch whose buffers are not aligned to the vw-element vectors
  std::shared_ptr<FusedPlan> scalar;
  bool staged = false;       // written by stage_vm (values in LDS), not fuse_vm
};

struct Plan {
  PlanKind kind = PlanKind::EwBinary;
  std::string func;
  int32_t grid[3] = {1, 1, 1};
  std::vector<Type> arg_types;   // memref argument types, in order
  // EwBinary: a op b -> c.   RowSoftmax: a -> c.   Gemm: a @ b -> c.
  Access2D a, b, c;
  EwOp ew_op = EwOp::Add;
  // EwBinary: when every operand's tiles over the whole grid cover one
  // contiguous run of elements, each once, and the same (Block, row, column)
  // sits at the same position of every operand's run, the run's length (the
  // Blocks then execute as one flat stream); 0 otherwise.
  int64_t ew_flat = 0;
  int64_t gemm_k = 0;
  // Gemm epilogue (kernels/matmul.py:15-17): t * scale + bias with (1, TN)
  // row tiles, then an optional ftoi (the store's element type is then i8).
  bool gemm_scale = false, gemm_bias = false, gemm_ftoi = false;
  Access2D scale, bias;
  ConvPlan conv;
  VmPlan vm;
  std::shared_ptr<FusedPlan> fused;  // Fused: the generated kernel (vm keeps the accesses)
  std::string unfused;               // TileVM: why the program is not fused
  // RowSoftmax and Fused plans fall back to the tile interpreter at launch
  // when a buffer is not aligned to their vectors; vm_fallback says whether
  // `vm` holds an interpreter lowering that fits, vm_fallback_why why not.
  bool vm_fallback = false;
  std::string vm_fallback_why;
  double algo_bytes = 0;  // algorithmic HBM bytes per launch
  double algo_flops = 0;  // algorithmic FLOPs per launch
  std::string describe() const;
};

// The fused kernel for a tile-interpreter plan, when every value is the
// program's main [R, C] tile or a [1, C] / [R, 1] / [1, 1] broadcast of it and
// the ops are loads, stores, unary, binary and reductions (fused.cpp).
// Returns false, with `why` set, when the program does not fit.
// max_vw caps the row vector width (4, 2 or 1 elements)
bool fuse_vm(const VmPlan& vm, const int32_t grid[3], FusedPlan& out, std::string& why, int max_vw = 4);

// The staged kernel for a tile-interpreter plan the fused layout declines
// (staged.cpp): every instruction compiled, values in LDS, matmul / mma on
// MFMA.  Returns false, with `why` set, when the program does not fit
// (LDS beyond 160 KB, more than 8 accesses, an exact matmul of values that
// are not i8 tiles, a load of a memref the program stored to).
bool stage_vm(const VmPlan& vm, const int32_t grid[3], FusedPlan& out, std::string& why, int max_vw = 4);

// Builds the plan of function `func` (empty name: the only function).
// Returns false and sets `error` when the program is not one the HIP
// backend runs.
bool build_plan(const Module& m, const std::string& func, Plan& plan, std::string& error);

}  // namespace xt
