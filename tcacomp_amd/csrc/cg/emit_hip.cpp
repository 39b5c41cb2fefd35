// emit_hip.cpp — lowers a finished map+reduce graph to one HIP source file
// (gfx950) plus its launch plan.
//
// Pass structure (the reference's HIR window, internal/pipeline/pipeline.go:
// 41-52, restated for what the HIP path needs; the sm_86 LOWER window —
// tiling search, tile-lower, schedule, final-lower — has no counterpart: each
// family below fixes its own wave64 geometry):
//   1. dead-chain elimination: a chain survives if it stores an output, or a
//      local that a surviving later chain reads (internal/opt/dce/dce.go);
//   2. nest fusion: consecutive chains with the identical iteration order
//      fuse into one kernel when the fused family accepts them — the
//      reference's GVN loop-nest fusion (design/optana/loop_fusion.md:7-22);
//   3. local placement (memopt): a local whose producer and every reader sit
//      in one fused kernel lives in registers; any other local lives in an
//      HBM workspace the runtime provides (lifting the reference's
//      "GMEM temporaries are refused" gate, internal/cg/cxx/emit.go:274-276);
//   4. family classification + emission, one __global__ per nest.
#include "emit.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <functional>
#include <map>
#include <set>
#include <sstream>
#include <tuple>

#include "gemm_emit.h"

namespace tca {
namespace cg {

using ir::BinOp;
using ir::Elem;
using ir::Graph;
using ir::Op;

const char* FamilyName(Family f) {
  switch (f) {
    case Family::Elementwise: return "elementwise";
    case Family::Row: return "row";
    case Family::Stream: return "stream";
    case Family::Col: return "col";
    case Family::Gemm: return "gemm";
    case Family::Generic: return "generic";
    case Family::Seg: return "seg";
  }
  return "?";
}

std::vector<std::string> DeviceFlags(const std::string& target) {
  return {"--genco",
          "--offload-arch=" + target,
          "-O3",
          "-std=c++17",
          "-ffp-contract=off",
          "-fno-gpu-flush-denormals-to-zero",
          "-fhip-fp32-correctly-rounded-divide-sqrt",
          "-Xclang",
          "-target-feature",
          "-Xclang",
          "-packed-fp32-ops",
          "-Wno-unused-variable",
          "-Wno-unused-but-set-variable"};
}

namespace detail {

std::string CType(Elem e) {
  switch (e) {
    case Elem::F32: return "float";
    case Elem::F16: return "_Float16";
    case Elem::BF16: return "__bf16";
    case Elem::I32: return "int32_t";
    case Elem::U32: return "uint32_t";
    case Elem::I8: return "int8_t";
    case Elem::I16: return "int16_t";
    case Elem::U8: return "uint8_t";
    case Elem::U16: return "uint16_t";
    case Elem::Bool: return "bool";
  }
  return "float";
}

// Scalar kernel-parameter type: 4-byte slots (rt/plan.cpp PackArgs).
std::string ScalarArgType(Elem e) {
  if (ir::IsFloat(e)) return "float";
  if (e == Elem::U32 || e == Elem::U16 || e == Elem::U8) return "uint32_t";
  return "int32_t";
}

std::string Literal(const ir::Expr& e) {
  char buf[80];
  switch (e.type) {
    case Elem::F32:
    case Elem::F16:
    case Elem::BF16: {
      std::string f;
      if (std::isnan(e.value)) f = "__builtin_nanf(\"\")";
      else if (std::isinf(e.value)) f = e.value > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
      else {
        std::snprintf(buf, sizeof(buf), "%af", static_cast<float>(e.value));
        f = buf;
      }
      if (e.type == Elem::F32) return f;
      return "static_cast<" + CType(e.type) + ">(" + f + ")";
    }
    case Elem::Bool:
      return e.value != 0.0 ? "true" : "false";
    case Elem::U32:
      std::snprintf(buf, sizeof(buf), "%.0fu", e.value);
      return buf;
    default:
      std::snprintf(buf, sizeof(buf), "static_cast<%s>(%.0f)", CType(e.type).c_str(), e.value);
      return buf;
  }
}

std::string ExtentExpr(const Graph& g, int d) {
  if (g.dims[d].extent > 0) return std::to_string(g.dims[d].extent) + "u";
  return "d" + std::to_string(d);
}

// Emits pure scalar expression DAGs as SSA temporaries. One instance per
// lexical scope: its memo is the common-subexpression table of that scope.
class ExprGen {
 public:
  ExprGen(const Graph& g, std::ostringstream& out, std::string indent, int* counter)
      : g_(g), out_(out), indent_(std::move(indent)), counter_(counter) {}

  void Bind(int param, const std::string& value) { memo_[param] = value; }

  std::string Gen(int id) {
    auto it = memo_.find(id);
    if (it != memo_.end()) return it->second;
    const ir::Expr& e = g_.exprs[id];
    std::string val;
    switch (e.op) {
      case Op::Const:
        val = Literal(e);
        memo_[id] = val;
        return val;
      case Op::Scalar: {
        const Elem t = g_.scalars[e.index].elem;
        val = "s" + std::to_string(e.index);
        if (ScalarArgType(t) != CType(t)) val = "static_cast<" + CType(t) + ">(" + val + ")";
        memo_[id] = val;
        return val;
      }
      case Op::Param:
        // Unbound lambda parameter: a classifier bug, never user error.
        val = "/*unbound " + e.text + "*/0";
        memo_[id] = val;
        return val;
      default:
        break;
    }
    std::vector<std::string> a;
    for (int x : e.args) a.push_back(Gen(x));
    const std::string T = CType(e.type);
    std::string rhs;
    switch (e.op) {
      case Op::Bin: {
        const BinOp op = static_cast<BinOp>(e.code);
        static const char* sym[] = {"+", "-", "*", "/", "%", "==", "!=", "<", "<=", ">", ">=", "&&", "||",
                                    "&", "|", "^", "<<", ">>"};
        std::string core = "(" + a[0] + " " + sym[static_cast<int>(op)] + " " + a[1] + ")";
        const Elem in = g_.exprs[e.args[0]].type;
        if (e.type == Elem::Bool || in == Elem::F32 || in == Elem::I32 || in == Elem::U32) rhs = core;
        else rhs = "static_cast<" + T + ">" + core;
        break;
      }
      case Op::Un: {
        // The operand is parenthesized: a negative literal operand would
        // otherwise spell the decrement operator (--0x1p+1f).
        static const char* sym[] = {"-", "+", "!", "~"};
        rhs = "static_cast<" + T + ">(" + std::string(sym[e.code]) + "(" + a[0] + "))";
        break;
      }
      case Op::Select:
        rhs = "(" + a[0] + " ? " + a[1] + " : " + a[2] + ")";
        break;
      case Op::Cast:
        rhs = "static_cast<" + T + ">(" + a[0] + ")";
        break;
      case Op::Call: {
        if (e.text == "fmaf") rhs = "__builtin_fmaf(" + a[0] + ", " + a[1] + ", " + a[2] + ")";
        else if (e.text == "umin") rhs = "min(" + a[0] + ", " + a[1] + ")";
        else if (e.text == "umax") rhs = "max(" + a[0] + ", " + a[1] + ")";
        else {
          rhs = e.text + "(";
          for (size_t i = 0; i < a.size(); ++i) rhs += (i ? ", " : "") + a[i];
          rhs += ")";
        }
        break;
      }
      default:
        rhs = "0";
        break;
    }
    val = "v" + std::to_string((*counter_)++);
    out_ << indent_ << "const " << T << " " << val << " = " << rhs << ";\n";
    memo_[id] = val;
    return val;
  }

 private:
  const Graph& g_;
  std::ostringstream& out_;
  std::string indent_;
  int* counter_;
  std::map<int, std::string> memo_;
};

void CollectScalars(const Graph& g, int id, std::set<int>* out) {
  const ir::Expr& e = g.exprs[id];
  if (e.op == Op::Scalar) out->insert(e.index);
  for (int a : e.args) CollectScalars(g, a, out);
}

std::set<int> ChainScalars(const Graph& g, const ir::Chain& c) {
  std::set<int> s;
  CollectScalars(g, c.root.fn.body, &s);
  for (const auto& r : c.reduces) {
    CollectScalars(g, r.init, &s);
    CollectScalars(g, r.fn.body, &s);
  }
  if (c.has_piped) CollectScalars(g, c.piped.fn.body, &s);
  return s;
}

// Combiners a tree reduction may reassociate: acc OP now (either order)
// with OP one of + * min max (float +,* reassociate within tolerance, as the
// reference's WarpReducer does), integer bitwise ops, logical and/or.
bool IsMonoidCombiner(const Graph& g, const ir::ReduceStage& r) {
  const ir::Expr& b = g.exprs[r.fn.body];
  const int acc = r.fn.params[0], now = r.fn.params[1];
  if (b.args.size() != 2) return false;
  const bool params = (b.args[0] == acc && b.args[1] == now) || (b.args[0] == now && b.args[1] == acc);
  if (!params) return false;
  if (b.op == Op::Bin) {
    switch (static_cast<BinOp>(b.code)) {
      case BinOp::Add:
      case BinOp::Mul:
      case BinOp::And:
      case BinOp::Or:
      case BinOp::Xor:
      case BinOp::LAnd:
      case BinOp::LOr:
        return true;
      default:
        return false;
    }
  }
  if (b.op == Op::Call)
    return b.text == "fmaxf" || b.text == "fminf" || b.text == "umin" || b.text == "umax";
  return false;
}

std::string Sym(const Graph& g, const std::string& prefix, int k) {
  (void)g;
  return prefix + "_k" + std::to_string(k);
}

}  // namespace detail

using namespace detail;

bool EmitGemm(const Graph& g, const ir::Chain& c, const GemmMatch& m, const std::string& symbol,
              const std::string& signature, int nest, bool small, int* counter, std::ostringstream* src,
              GemmEmitted* out, std::string* err) {
  (void)err;
  std::ostringstream& o = *src;
  const int ta = c.root.ops[m.a_op].tensor, tb = c.root.ops[m.b_op].tensor, tc = c.store_tensor;
  // 16-bit inputs (bf16 or f16) share the bf16 kernels; f16 selects their
  // _f16 MFMAs and hands them its tensors as 16-bit words.
  const bool f16 = m.in == Elem::F16;
  const bool bf16 = m.in == Elem::BF16 || f16;
  // The fused epilogue (the piped map at (cm, cn)), the same in every kernel.
  std::ostringstream epi;
  epi << "  const uint32_t M = " << ExtentExpr(g, m.m) << ", N = " << ExtentExpr(g, m.n) << ", K = "
      << ExtentExpr(g, m.k) << ";\n";
  epi << "  const auto epi = [&](float acc, uint32_t cm, uint32_t cn) -> float {\n";
  std::string val = "acc";
  if (c.has_piped) {
    ExprGen pg(g, epi, "    ", counter);
    pg.Bind(c.piped.fn.params[0], "acc");
    for (size_t k = 0; k < c.piped.ops.size(); ++k) {
      const auto& op = c.piped.ops[k];
      const ir::Tensor& tt = g.tensors[op.tensor];
      std::string off = "0u";
      for (size_t i = 0; i < op.axes.size(); ++i) {
        const std::string cc = op.axes[i] == m.m ? "cm" : "cn";
        off = i == 0 ? cc : "(" + off + ") * " + ExtentExpr(g, tt.dims[i]) + " + " + cc;
      }
      pg.Bind(c.piped.fn.params[k + 1], "t" + std::to_string(op.tensor) + "[" + off + "]");
    }
    val = pg.Gen(c.piped.fn.body);
  }
  epi << "    return " << val << ";\n  };\n";
  // A batched contraction runs one grid of tiles per batch: the workgroup id
  // splits into (batch, tile), the operands led by the batch axis and C are
  // offset to that batch, and the kernel maps the tile index as it maps the
  // workgroup id of a single contraction. `args(T)` is the call for square
  // tiles of T.
  const bool batched = m.batch >= 0;
  auto args = [&](uint32_t T) {
    std::string a = "t" + std::to_string(ta), b = "t" + std::to_string(tb), cc = "t" + std::to_string(tc);
    std::string pre, tile;
    if (batched) {
      const std::string Ts = std::to_string(T) + "u";
      pre = "  const uint32_t tiles = ((M + " + Ts + " - 1u) / " + Ts + ") * ((N + " + Ts + " - 1u) / " + Ts +
            "), bb = blockIdx.x / tiles;\n";
      if (m.a_batched) a = "(" + a + " + (size_t)bb * M * K)";
      if (m.b_batched) b = "(" + b + " + (size_t)bb * K * N)";
      cc = "(" + cc + " + (size_t)bb * M * N)";
      tile = ", blockIdx.x - bb * tiles";
    }
    if (f16) {
      a = "reinterpret_cast<const __bf16*>(" + a + ")";
      b = "reinterpret_cast<const __bf16*>(" + b + ")";
    }
    return std::make_pair(pre, "(" + a + ", " + b + ", " + cc + ", M, N, K, epi" + tile + ");\n}\n\n");
  };
  const std::string nk = m.b_nk ? "true" : "false";
  // Grid terms: [batch x] tiles of the (m, n) plane.
  auto tiles = [&](uint32_t T) {
    std::vector<std::string> t;
    if (batched) t.push_back(g.dims[m.batch].name + "/1");
    t.push_back(g.dims[m.m].name + "/" + std::to_string(T));
    t.push_back(g.dims[m.n].name + "/" + std::to_string(T));
    return t;
  };
  const std::vector<std::string> grid = tiles(256);
  std::string orient = m.b_nk ? " B=[n][k]" : " B=[k][n]";
  if (batched)
    orient += std::string(" batch=@") + g.dims[m.batch].name + " A " + (m.a_batched ? "per batch" : "shared") + ", B " +
              (m.b_batched ? "per batch" : "shared");
  o << "// " << (batched ? "batched (over @" + g.dims[m.batch].name + ") " : "") << "contraction over @"
    << g.dims[m.k].name << " on MFMA ("
    << (f16 ? "f16 16x16x32 whole tiles, 32x32x16 edges" : bf16 ? "bf16 16x16x32 whole tiles, 32x32x16 edges" : "f32 32x32x2")
    << "), B indexed " << (m.b_nk ? "[n][k]" : "[k][n]") << "\n";
  // Output planes of at most kGemmSmallMax elements: 32x32 tiles with K
  // split over the 16 waves of a workgroup and, when the tiles are fewer
  // than the split target, over P chunks (the split record; P > 1 adds the
  // merge kernel). The tile kernels below carry the complementary guard.
  std::string bigWhen;
  if (small) {
    const std::string Ms = g.dims[m.m].name, Ns = g.dims[m.n].name, Ks = g.dims[m.k].name;
    const uint32_t kKcMin = bf16 ? 1024u : 512u;  // 4 steps per wave and chunk
    const uint32_t kBlocks = 512u;                // two 16-wave workgroups per CU
    const std::string part = "__gemmpart" + std::to_string(nest), pdim = "__gemmdim" + std::to_string(nest);
    out->extra_dims.push_back(pdim + " " + std::to_string(uint64_t{kBlocks} * 1024u));
    out->extra_tensors.push_back(part + " f32 local 1 " + pdim);
    const std::string psig = ",\n    float* __restrict__ pw /* " + part + " */";
    auto body = [&](bool merge) {
      std::ostringstream b;
      b << epi.str() << "  const uint32_t tiles = ((M + 31u) / 32u) * ((N + 31u) / 32u);\n"
        << "  const uint32_t T = " << (batched ? ExtentExpr(g, m.batch) + " * tiles" : std::string("tiles")) << ";\n"
        << "  const uint32_t P = tca::hip::gemm_split_chunks(K, T, " << kKcMin << "u, " << kBlocks << "u);\n"
        << (merge ? "  const uint32_t gt = blockIdx.x;\n" : "  const uint32_t gt = blockIdx.x % T, p = blockIdx.x / T;\n");
      std::string a = "t" + std::to_string(ta), bo = "t" + std::to_string(tb), cc = "t" + std::to_string(tc);
      if (batched) {
        b << "  const uint32_t bb = gt / tiles, tile = gt - bb * tiles;\n";
        if (m.a_batched) a = "(" + a + " + (size_t)bb * M * K)";
        if (m.b_batched) bo = "(" + bo + " + (size_t)bb * K * N)";
        cc = "(" + cc + " + (size_t)bb * M * N)";
      } else {
        b << "  const uint32_t tile = gt;\n";
      }
      if (merge)
        b << "  tca::hip::gemm_small_merge(" << cc << ", pw, M, N, epi, tile, gt, T, P);\n}\n\n";
      else
        b << "  tca::hip::gemm_small<" << (bf16 ? "true" : "false") << ", " << (m.b_nk ? "true" : "false")
          << ", decltype(epi)" << (f16 ? ", true" : "") << ">(" << a << ", " << bo << ", " << cc
          << ", pw, M, N, K, epi, tile, gt, T, p, P);\n}\n\n";
      return b.str();
    };
    o << "extern \"C\" __global__ void __launch_bounds__(1024) " << symbol << "_s(\n    " << signature << psig
      << ") {\n" << body(false);
    o << "extern \"C\" __global__ void __launch_bounds__(1024) " << symbol << "_sm(\n    " << signature << psig
      << ") {\n" << body(true);
    std::vector<std::string> t32;
    if (batched) t32.push_back(g.dims[m.batch].name + "/1");
    t32.push_back(Ms + "/32");
    t32.push_back(Ns + "/32");
    std::string splitTerms = std::to_string(t32.size());
    for (const auto& t : t32) splitTerms += " " + t;
    const std::string splitRec = Ks + " " + std::to_string(kKcMin) + " " + std::to_string(kBlocks);
    const std::string smallWhen = Ms + "*" + Ns + " 0 " + std::to_string(kGemmSmallMax) + " 1 0";
    bigWhen = Ms + "*" + Ns + " " + std::to_string(kGemmSmallMax + 1) + " 18446744073709551615 1 0";
    const std::string ty = f16 ? "f16 mfma 32x32x16" : bf16 ? "bf16 mfma 32x32x16" : "f32 mfma 32x32x2";
    GemmKernel s;
    s.suffix = "_s";
    s.block = 1024;
    s.grid = t32;
    s.when = {smallWhen};
    s.extra_args = {"ptr " + part};
    s.split = splitRec + " 0 " + splitTerms;
    s.detail = ty + " tile=32x32, K split over 16 waves (and P chunks of >= " + std::to_string(kKcMin) +
               " when the tiles are fewer than " + std::to_string(kBlocks) + "; M*N <= " +
               std::to_string(kGemmSmallMax) + ")" + orient;
    GemmKernel sm = s;
    sm.suffix = "_sm";
    sm.split = splitRec + " 1 " + splitTerms;
    sm.detail = ty + " small-tile merge: the P chunk partials of each 32x32 tile added in chunk order (P > 1 only)";
    out->kernels.push_back(s);
    out->kernels.push_back(sm);
  }
  if (!bf16) {
    // From M, N >= 4096 on (at least 256 tiles of 256x256): whole tiles with
    // K % 32 == 0 and K >= 128 on 4 waves of 128x128 fed by a direct-to-LDS
    // ring (_w); otherwise 256x256 tiles with 16 waves of 64x64 (_v). Below,
    // 128x128 tiles with 4 waves (more tiles over the 256 CUs). _v and the
    // 128x128 kernel are two instances of one loop with edge guards; both run
    // 4 waves per SIMD: at most 128 registers per lane.
    const std::string M = g.dims[m.m].name, N = g.dims[m.n].name, K = g.dims[m.k].name;
    const auto a256 = args(256), a128 = args(128);
    o << "extern \"C\" __global__ void __launch_bounds__(256) " << symbol << "_w(\n    " << signature << ") {\n"
      << epi.str() << a256.first << "  tca::hip::gemm_f32_4w<" << nk << ">" << a256.second;
    o << "extern \"C\" __global__ void __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(4))) " << symbol
      << "_v(\n    " << signature << ") {\n"
      << epi.str() << a256.first << "  tca::hip::gemm_f32_tile<" << nk << ", 256, 256>" << a256.second;
    o << "extern \"C\" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) " << symbol
      << "(\n    " << signature << ") {\n"
      << epi.str() << a128.first << "  tca::hip::gemm_f32_tile<" << nk << ", 128, 128>" << a128.second;
    GemmKernel w;
    w.suffix = "_w";
    w.block = 256;
    w.grid = tiles(256);
    w.when = {M + " 4096 4294967295 256 0", N + " 4096 4294967295 256 0", K + " 128 4294967295 32 0"};
    w.detail = "f32 mfma 32x32 tile=256x256 bk=16 4 waves of 128x128, direct-to-LDS ring (whole tiles, M, N >= 4096, K % 32 == 0, K >= 128)" + orient;
    GemmKernel v;
    v.suffix = "_v";
    v.block = 1024;
    v.grid = tiles(256);
    v.when = {M + " 4096 4294967295 1 0", N + " 4096 4294967295 1 0"};
    v.unless = w.when;
    v.detail = "f32 mfma 32x32 tile=256x256 bk=16 16 waves, two LDS buffers (M, N >= 4096)" + orient;
    GemmKernel k;
    k.grid = tiles(128);
    k.unless = v.when;
    if (!bigWhen.empty()) k.when.push_back(bigWhen);
    k.detail = "f32 mfma 32x32 tile=128x128 bk=16 4 waves, two LDS buffers" + orient;
    out->kernels.push_back(w);
    out->kernels.push_back(v);
    out->kernels.push_back(k);
    return true;
  }
  // bf16: the direct-to-LDS tiles (whole 256x256 blocks, K a positive
  // multiple of 32, N % 8 == 0), launched when there can be one: on 4 waves
  // of 128x128 with A in 64-deep slices when K % 64 == 0 and K >= 256 (_w),
  // else on 8 waves of 128x64 with 32-deep slices (_v); every other tile on
  // the 256-thread register-staged kernel, skipped when every tile is a
  // direct-to-LDS one (M, N multiples of 256, K a positive multiple of 32).
  // Each kernel returns at once on the other kernels' tiles.
  const std::string M = g.dims[m.m].name, N = g.dims[m.n].name, K = g.dims[m.k].name;
  const auto a256 = args(256);
  o << "extern \"C\" __global__ void __launch_bounds__(256) " << symbol << "_w(\n    " << signature << ") {\n"
    << epi.str() << a256.first << "  tca::hip::gemm_bf16_4w<" << nk << (f16 ? ", decltype(epi), true" : "") << ">"
    << a256.second;
  o << "extern \"C\" __global__ void __launch_bounds__(512) " << symbol << "_v(\n    " << signature << ") {\n"
    << epi.str() << a256.first << "  tca::hip::gemm_bf16_256_w8<" << nk << (f16 ? ", decltype(epi), 4, true" : "")
    << ">" << a256.second;
  o << "extern \"C\" __global__ void __launch_bounds__(256) " << symbol << "(\n    " << signature << ") {\n"
    << epi.str() << a256.first << "  tca::hip::gemm_bf16_256<" << nk << ", decltype(epi), 1, true, true, true"
    << (f16 ? ", true" : "") << ">" << a256.second;
  GemmKernel w;
  w.suffix = "_w";
  w.block = 256;
  w.grid = grid;
  w.when = {M + " 256 4294967295 1 0", N + " 256 4294967295 8 0", K + " 256 4294967295 64 0"};
  const std::string ty = f16 ? "f16" : "bf16";
  w.detail = ty + " mfma 16x16x32 tile=256x256 4 waves of 128x128, A in 64-deep slices (direct-to-LDS rings; whole tiles, K % 64 == 0, K >= 256)" + orient;
  GemmKernel v;
  v.suffix = "_v";
  v.block = 512;
  v.grid = grid;
  v.when = {M + " 256 4294967295 1 0", N + " 256 4294967295 8 0", K + " 32 4294967295 32 0"};
  v.unless = {K + " 256 4294967295 64 0"};
  v.detail = ty + " mfma 16x16x32 tile=256x256 bk=32 8 waves (direct-to-LDS ring; whole tiles, K % 64 != 0 or K < 256)" + orient;
  GemmKernel e;
  e.grid = grid;
  e.unless = {M + " 0 4294967295 256 0", N + " 0 4294967295 256 0", K + " 32 4294967295 32 0"};
  e.detail = ty + " mfma 32x32 tile=256x256 bk=64 4 waves (edge tiles, K % 32 != 0, N % 8 != 0)" + orient;
  if (!bigWhen.empty())
    for (GemmKernel* k : {&w, &v, &e}) k->when.push_back(bigWhen);
  out->kernels.push_back(w);
  out->kernels.push_back(v);
  out->kernels.push_back(e);
  return true;
}

namespace {

struct Nest {
  std::vector<int> chains;
  Family family = Family::Generic;
  // Chained reductions folded in one kernel (the segment kernel): 1 on the
  // inner nest (a row reduction into a local), 2 on the next nest (its
  // fold over rows). seg_guard names the segment dim whose run-time value
  // picks between the segment kernel and the two nests' own kernels; empty:
  // the segment kernel alone.
  int seg = 0;
  std::string seg_guard;
};

struct Analysis {
  std::vector<bool> live;
  std::vector<Nest> nests;
  std::vector<bool> hbm_local;  // per tensor
  std::vector<int> reg_nest;    // per tensor: nest holding it in registers, or -1
};

// Tensors a chain reads (operands of both maps).
std::set<int> ReadSet(const ir::Chain& c) {
  std::set<int> s;
  for (const auto& o : c.root.ops) s.insert(o.tensor);
  if (c.has_piped)
    for (const auto& o : c.piped.ops) s.insert(o.tensor);
  return s;
}

// ---- row family geometry --------------------------------------------------

struct RowGeom {
  bool ok = false;
  std::string why;
  std::vector<int> as;  // common iteration order
  std::vector<int> outer;
  int col = -1;
  uint32_t C = 0, V = 1, vecs = 0, tpr = 1, nv = 1, block = 256, rpb = 1;
  bool tail = false;
};

enum class OpKind { RowTile, ColVec, RowScalar, Bad };

OpKind Classify(const ir::Operand& o, const RowGeom& geo) {
  if (o.axes == geo.as) return OpKind::RowTile;
  if (o.axes.size() == 1 && o.axes[0] == geo.col) return OpKind::ColVec;
  for (int a : o.axes)
    if (a == geo.col) return OpKind::Bad;
  std::set<int> outer(geo.outer.begin(), geo.outer.end());
  for (int a : o.axes)
    if (!outer.count(a)) return OpKind::Bad;
  return OpKind::RowScalar;
}

// True for a chain of a row nest that iterates only the outer axes (one level
// shallower than the nest): a per-row scalar computation.
bool IsRowScalarChain(const ir::Chain& c, const RowGeom& geo) { return c.root.as.size() + 1 == geo.as.size(); }

// Structural equality of two root-map bodies (expression a in chain ca, b in
// chain cb): the same operators, types, constants and builtins, and a
// parameter of one equal to a parameter of the other when both read the same
// operand (tensor and subscripts).
bool SameRowExpr(const ir::Graph& g, int a, const ir::Chain& ca, int b, const ir::Chain& cb) {
  const ir::Expr& x = g.exprs[a];
  const ir::Expr& y = g.exprs[b];
  if (x.op == ir::Op::Param || y.op == ir::Op::Param) {
    if (x.op != y.op) return false;
    auto operandOf = [](const ir::Chain& c, int pid) -> const ir::Operand* {
      for (size_t k = 0; k < c.root.fn.params.size(); ++k)
        if (c.root.fn.params[k] == pid) return &c.root.ops[k];
      return nullptr;
    };
    const ir::Operand* oa = operandOf(ca, a);
    const ir::Operand* ob = operandOf(cb, b);
    return oa != nullptr && ob != nullptr && oa->tensor == ob->tensor && oa->axes == ob->axes;
  }
  if (a == b) return true;  // one hash-consed node with no parameter below it
  if (x.op != y.op || x.type != y.type || x.code != y.code || x.index != y.index || x.text != y.text ||
      x.args.size() != y.args.size())
    return false;
  if (x.op == ir::Op::Const && !(x.value == y.value && std::signbit(x.value) == std::signbit(y.value))) return false;
  for (size_t i = 0; i < x.args.size(); ++i)
    if (!SameRowExpr(g, x.args[i], ca, y.args[i], cb)) return false;
  return true;
}

// A softmax's two reductions, fusable into one read of the row with the
// online normaliser (tca::hip::online_expsum_add): chain A folds t over the
// row with fmaxf from -inf (f32, no piped map) into a row scalar, and chain
// B folds expf(t - a) with + (f32), where a is A's result read at the row
// and t is A's root body. Then
//   sum over the row of expf(t - a) = sum over chunks of s_c * expf(m_c - a),
// m_c a chunk's maximum and s_c its sum of expf(t - m_c). B's init and piped
// map are applied at its merge as usual.
bool OnlineMaxExpSum(const ir::Graph& g, const ir::Chain& A, const ir::Chain& B, const RowGeom& geo) {
  if (A.reduces.size() != 1 || B.reduces.size() != 1 || A.has_piped) return false;
  if (g.exprs[A.root.fn.body].type != ir::Elem::F32 || g.exprs[B.root.fn.body].type != ir::Elem::F32) return false;
  if (g.tensors[A.store_tensor].elem != ir::Elem::F32) return false;
  const ir::ReduceStage& ra = A.reduces[0];
  // -inf: a literal, or a negated +inf literal (how the .tca source spells it)
  auto negInf = [&](int id) {
    const ir::Expr& e = g.exprs[id];
    if (e.op == ir::Op::Const) return std::isinf(e.value) && e.value < 0;
    if (e.op != ir::Op::Un || static_cast<ir::UnOp>(e.code) != ir::UnOp::Neg) return false;
    const ir::Expr& v = g.exprs[e.args[0]];
    return v.op == ir::Op::Const && std::isinf(v.value) && v.value > 0;
  };
  if (g.exprs[ra.init].type != ir::Elem::F32 || !negInf(ra.init)) return false;
  auto accNow = [&](const ir::ReduceStage& r, const ir::Expr& e) {
    const int acc = r.fn.params[0], now = r.fn.params[1];
    return e.args.size() == 2 && ((e.args[0] == acc && e.args[1] == now) || (e.args[0] == now && e.args[1] == acc));
  };
  const ir::Expr& ca = g.exprs[ra.fn.body];
  if (ca.op != ir::Op::Call || ca.text != "fmaxf" || !accNow(ra, ca)) return false;
  const ir::ReduceStage& rb = B.reduces[0];
  const ir::Expr& cb = g.exprs[rb.fn.body];
  if (cb.op != ir::Op::Bin || static_cast<ir::BinOp>(cb.code) != ir::BinOp::Add || !accNow(rb, cb)) return false;
  const ir::Expr& bb = g.exprs[B.root.fn.body];
  if (bb.op != ir::Op::Call || bb.text != "expf" || bb.args.size() != 1) return false;
  const ir::Expr& sub = g.exprs[bb.args[0]];
  if (sub.op != ir::Op::Bin || static_cast<ir::BinOp>(sub.code) != ir::BinOp::Sub) return false;
  const ir::Expr& pa = g.exprs[sub.args[1]];
  if (pa.op != ir::Op::Param) return false;
  for (size_t k = 0; k < B.root.fn.params.size(); ++k) {
    if (B.root.fn.params[k] != sub.args[1]) continue;
    const ir::Operand& op = B.root.ops[k];
    if (op.tensor != A.store_tensor || op.axes != A.store_axes || Classify(op, geo) != OpKind::RowScalar) return false;
    return SameRowExpr(g, A.root.fn.body, A, sub.args[0], B);
  }
  return false;
}

// The structural conditions shared by the register-resident row family and
// the streaming row family: every chain iterates (outer..., col) in one
// order, or only (outer...) — the prefix fusion of a shallower nest
// (internal/opt/gvn/gvn_test.go:458-518): a map over row scalars storing a
// row scalar, evaluated once per row. At most one reduction per chain (over
// col) with an associative-commutative combiner; operands are row tiles,
// column vectors or row scalars. `stream` additionally refuses elementwise
// chains into locals (a streamed row is never held, so a row-tile local
// could not be re-read).
bool RowShape(const Graph& g, const std::vector<int>& chains, bool stream, RowGeom* out) {
  RowGeom& geo = *out;
  auto no = [&](const std::string& w) {
    geo.ok = false;
    geo.why = w;
    return false;
  };
  // The nest's iteration order is its deepest chain's.
  geo.as = g.chains[chains[0]].root.as;
  for (int ci : chains)
    if (g.chains[ci].root.as.size() > geo.as.size()) geo.as = g.chains[ci].root.as;
  if (geo.as.empty()) return no("no iteration axis");
  geo.col = geo.as.back();
  geo.outer.assign(geo.as.begin(), geo.as.end() - 1);
  bool deep = false;
  std::set<int> produced_tile, produced_scalar;
  for (int ci : chains) {
    const ir::Chain& c = g.chains[ci];
    if (IsRowScalarChain(c, geo) && c.root.as == geo.outer && !geo.outer.empty()) {
      if (!c.reduces.empty()) return no("a per-row chain with a reduction");
      for (const auto& o : c.root.ops)
        if (Classify(o, geo) != OpKind::RowScalar) return no("per-row chain operand is not a row scalar");
      if (c.store_axes != geo.outer) return no("per-row store is not in iteration order");
      if (g.tensors[c.store_tensor].local) produced_scalar.insert(c.store_tensor);
      continue;
    }
    if (c.root.as != geo.as) return no("iteration orders differ");
    deep = true;
    if (c.reduces.size() > 1) return no("more than one reduction in a chain");
    if (c.reduces.size() == 1 && !IsMonoidCombiner(g, c.reduces[0]))
      return no("combiner is not an associative-commutative op over (acc, now)");
    for (const auto& o : c.root.ops) {
      OpKind k = Classify(o, geo);
      if (k == OpKind::Bad) return no("operand " + g.tensors[o.tensor].name + " is not row-shaped");
      if (g.tensors[o.tensor].local) {
        bool inside_tile = produced_tile.count(o.tensor) > 0, inside_scalar = produced_scalar.count(o.tensor) > 0;
        if (inside_tile && k != OpKind::RowTile) return no("local read with a different shape");
        if (inside_scalar && k != OpKind::RowScalar) return no("local read with a different shape");
      }
    }
    if (c.has_piped)
      for (const auto& o : c.piped.ops)
        if (Classify(o, geo) != OpKind::RowScalar) return no("piped operand is not a row scalar");
    const ir::Tensor& st = g.tensors[c.store_tensor];
    if (c.reduces.empty()) {
      if (c.store_axes != geo.as) return no("elementwise store is not in iteration order");
      if (st.local && stream) return no("a streamed row cannot hold a row-tile local");
      if (st.local) produced_tile.insert(c.store_tensor);
    } else {
      if (st.local) produced_scalar.insert(c.store_tensor);
    }
  }
  if (!deep) return no("no chain iterates the row");
  geo.ok = true;
  return true;
}

// Streaming row family: row length known only at run time (or too long for
// registers); every chain of the nest streams the row.
RowGeom StreamCheck(const Graph& g, const std::vector<int>& chains) {
  RowGeom geo;
  RowShape(g, chains, true, &geo);
  return geo;
}

// Integer partials of 32 bits get a fold fence after each vector (the
// compiler would otherwise reassociate the adds of all vectors in flight).
bool FoldFenced(ir::Elem e) { return ir::IsInt(e) && ir::ElemBytes(e) == 4; }

// Elements per vector of a row nest: 16 bytes of its widest row-shaped
// tensor (row tiles and column vectors it reads, row tiles it writes,
// register locals included), so the widest moves in 16-byte vectors and the
// narrower ones in shorter vectors of the same element count (a bf16 row
// summed into f32: 8 elements, 16 bytes per load; a bf16 row mapped into an
// f32 tile: 4 elements, 8 + 16 bytes).
uint32_t RowVecMax(const Graph& g, const std::vector<int>& chains, const RowGeom& geo) {
  size_t widest = 1;
  for (int ci : chains) {
    const ir::Chain& c = g.chains[ci];
    if (IsRowScalarChain(c, geo)) continue;
    for (const auto& o : c.root.ops) {
      const OpKind k = Classify(o, geo);
      if (k == OpKind::RowTile || k == OpKind::ColVec) widest = std::max(widest, ir::ElemBytes(g.tensors[o.tensor].elem));
    }
    if (c.reduces.empty()) widest = std::max(widest, ir::ElemBytes(g.tensors[c.store_tensor].elem));
  }
  return static_cast<uint32_t>(std::max<size_t>(1, 16 / widest));
}

RowGeom RowCheck(const Graph& g, const std::vector<int>& chains, uint32_t nv_target) {
  RowGeom geo;
  auto no = [&](const std::string& w) {
    geo.ok = false;
    geo.why = w;
    return geo;
  };
  if (!RowShape(g, chains, false, &geo)) return geo;
  if (g.dims[geo.col].extent == 0) return no("row axis @" + g.dims[geo.col].name + " has a dynamic extent");
  geo.C = static_cast<uint32_t>(g.dims[geo.col].extent);
  geo.V = RowVecMax(g, chains, geo);  // then the widest power of two dividing the row
  while (geo.C % geo.V != 0) geo.V /= 2;
  geo.vecs = geo.C / geo.V;
  uint32_t tpr = 1;
  while (tpr * 2 <= geo.vecs / nv_target && tpr * 2 <= 1024) tpr *= 2;
  geo.tpr = tpr;
  geo.nv = (geo.vecs + tpr - 1) / tpr;
  if (geo.nv > 16) return no("row of " + std::to_string(geo.C) + " elements exceeds the register-resident limit");
  geo.tail = (geo.vecs % tpr) != 0;
  geo.block = std::max<uint32_t>(256, tpr);
  geo.rpb = geo.block / tpr;
  geo.ok = true;
  return geo;
}

// ---- column family geometry -----------------------------------------------

// Column family: a reduction over an axis that is not the contiguous one —
// the reference's middle-axis reductions (testing/kernels/runtime/
// row_sum.tca, softmax.tca): every chain iterates (outer..., c, r), the
// reduced axis r last, over tiles laid out (outer..., r, c) with c
// contiguous. One reduce per chain with an associative-commutative
// combiner, stored at (outer..., c); operands are tiles, column vectors
// ((outer...,) c: one value per output), row vectors ((outer...,) r) and
// outer scalars; piped maps read column vectors and outer scalars. A chain
// may read the result of an earlier chain of the nest, as a column vector
// only (the value at its own output): it then runs in a later pass, one
// pass after the latest chain it reads. Chains read no result of their own
// or of a later chain, and no two store one tensor.
struct ColGeom {
  bool ok = false;
  std::string why;
  std::vector<int> as, outer;
  int c = -1, r = -1;
  std::vector<int> pass;  // per chain of the nest, in nest order: 0, 1, ...
  int passes = 1;
};

enum class ColKind { Tile, ColVec, RowVec, Outer, Bad };

ColKind ClassifyCol(const ir::Operand& o, const ColGeom& geo) {
  std::vector<int> tile(geo.outer), cv(geo.outer), rv(geo.outer);
  tile.push_back(geo.r);
  tile.push_back(geo.c);
  cv.push_back(geo.c);
  rv.push_back(geo.r);
  if (o.axes == tile) return ColKind::Tile;
  if (o.axes == cv || (o.axes.size() == 1 && o.axes[0] == geo.c)) return ColKind::ColVec;
  if (o.axes == rv || (o.axes.size() == 1 && o.axes[0] == geo.r)) return ColKind::RowVec;
  const std::set<int> outer(geo.outer.begin(), geo.outer.end());
  for (int a : o.axes)
    if (!outer.count(a)) return ColKind::Bad;
  return ColKind::Outer;
}

ColGeom ColCheck(const Graph& g, const std::vector<int>& chains) {
  ColGeom geo;
  auto no = [&](const std::string& w) {
    geo.ok = false;
    geo.why = w;
    return geo;
  };
  geo.as = g.chains[chains[0]].root.as;
  if (geo.as.size() < 2) return no("fewer than two iteration axes");
  geo.r = geo.as.back();
  geo.c = geo.as[geo.as.size() - 2];
  geo.outer.assign(geo.as.begin(), geo.as.end() - 2);
  std::map<int, size_t> stored;  // result tensor -> position of its chain in the nest
  for (size_t i = 0; i < chains.size(); ++i)
    if (!stored.emplace(g.chains[chains[i]].store_tensor, i).second) return no("two chains store one tensor");
  std::vector<int> out_axes(geo.outer);
  out_axes.push_back(geo.c);
  geo.pass.assign(chains.size(), 0);
  for (size_t i = 0; i < chains.size(); ++i) {
    const ir::Chain& c = g.chains[chains[i]];
    if (c.root.as != geo.as) return no("iteration orders differ");
    if (c.reduces.size() != 1) return no("not exactly one reduction");
    if (!IsMonoidCombiner(g, c.reduces[0])) return no("combiner is not an associative-commutative op over (acc, now)");
    if (c.store_axes != out_axes) return no("store is not at (outer..., column)");
    // A read of a result of the nest: the producer's pass + 1, or a refusal.
    auto result = [&](const ir::Operand& o, ColKind k) -> bool {
      const auto it = stored.find(o.tensor);
      if (it == stored.end()) return true;
      if (it->second >= i) {
        geo.why = "a chain reads a result of itself or of a later chain of the nest";
        return false;
      }
      if (k != ColKind::ColVec) {
        geo.why = "a chain reads a result of the nest other than at its own column";
        return false;
      }
      geo.pass[i] = std::max(geo.pass[i], geo.pass[it->second] + 1);
      return true;
    };
    for (const auto& o : c.root.ops) {
      const ColKind k = ClassifyCol(o, geo);
      if (k == ColKind::Bad) return no("operand " + g.tensors[o.tensor].name + " is not column-shaped");
      if (!result(o, k)) return no(geo.why);
    }
    if (c.has_piped)
      for (const auto& o : c.piped.ops) {
        const ColKind k = ClassifyCol(o, geo);
        if (k != ColKind::ColVec && k != ColKind::Outer) return no("piped operand is not per output");
        if (!result(o, k)) return no(geo.why);
      }
    geo.passes = std::max(geo.passes, geo.pass[i] + 1);
  }
  geo.ok = true;
  return geo;
}

// A mean and a centred sum of squares over the reduced axis, fusable into
// one read of the input (Chan, Golub & LeVeque, "Updating formulae and a
// pairwise algorithm for computing sample variances", 1979): chain A folds t
// with + from 0 (f32) into m (its result after init and piped map, f32), and
// chain B folds (t - m) * (t - m) with + from 0 (f32), where m is read at
// B's own output index (`atOwnIndex` says whether an operand of B is that
// read) and t is A's root body. For rows split into groups g of n_g rows with
// sums S_g and M2_g = sum over g of (t - S_g / n_g)^2,
//   sum over the rows of (t - m)^2 = M2 + n (S / n - m)^2,
//   M2 of a union a + b = M2_a + M2_b + (S_b / n_b - S_a / n_a)^2 n_a n_b / (n_a + n_b),
// exactly in real arithmetic and every term non-negative, so no
// cancellation. B's piped map is applied to that sum as usual.
bool MeanSquaresPair(const ir::Graph& g, const ir::Chain& A, const ir::Chain& B,
                     const std::function<bool(const ir::Operand&)>& atOwnIndex) {
  if (A.reduces.size() != 1 || B.reduces.size() != 1) return false;
  if (g.exprs[A.root.fn.body].type != ir::Elem::F32 || g.exprs[B.root.fn.body].type != ir::Elem::F32) return false;
  if (g.tensors[A.store_tensor].elem != ir::Elem::F32) return false;
  auto zeroAdd = [&](const ir::ReduceStage& r) {
    const ir::Expr& init = g.exprs[r.init];
    if (init.op != ir::Op::Const || init.type != ir::Elem::F32 || init.value != 0.0) return false;
    const ir::Expr& e = g.exprs[r.fn.body];
    const int acc = r.fn.params[0], now = r.fn.params[1];
    return e.op == ir::Op::Bin && static_cast<ir::BinOp>(e.code) == ir::BinOp::Add && e.args.size() == 2 &&
           ((e.args[0] == acc && e.args[1] == now) || (e.args[0] == now && e.args[1] == acc));
  };
  if (!zeroAdd(A.reduces[0]) || !zeroAdd(B.reduces[0])) return false;
  const ir::Expr& sq = g.exprs[B.root.fn.body];
  if (sq.op != ir::Op::Bin || static_cast<ir::BinOp>(sq.code) != ir::BinOp::Mul || sq.args.size() != 2) return false;
  if (!SameRowExpr(g, sq.args[0], B, sq.args[1], B)) return false;
  const ir::Expr& d = g.exprs[sq.args[0]];
  if (d.op != ir::Op::Bin || static_cast<ir::BinOp>(d.code) != ir::BinOp::Sub || d.args.size() != 2) return false;
  if (g.exprs[d.args[1]].op != ir::Op::Param) return false;
  for (size_t k = 0; k < B.root.fn.params.size(); ++k) {
    if (B.root.fn.params[k] != d.args[1]) continue;
    const ir::Operand& op = B.root.ops[k];
    if (op.tensor != A.store_tensor || op.axes != A.store_axes || !atOwnIndex(op)) return false;
    return SameRowExpr(g, A.root.fn.body, A, d.args[0], B);
  }
  return false;
}

// The column family's form: m read as a column vector at B's own column, and
// B's piped map reading no result of the nest (the one-read kernels never
// load the mean from memory).
bool ChanMeanVar(const ir::Graph& g, const ir::Chain& A, const ir::Chain& B, const ColGeom& geo) {
  if (B.has_piped)
    for (const auto& po : B.piped.ops)
      if (po.tensor == A.store_tensor) return false;
  return MeanSquaresPair(g, A, B, [&](const ir::Operand& op) { return ClassifyCol(op, geo) == ColKind::ColVec; });
}

// The streaming row family's form: m read as a row scalar at B's own row.
bool ChanRowMeanVar(const ir::Graph& g, const ir::Chain& A, const ir::Chain& B, const RowGeom& geo) {
  return MeanSquaresPair(g, A, B, [&](const ir::Operand& op) { return Classify(op, geo) == OpKind::RowScalar; });
}

// ---- elementwise family check --------------------------------------------

bool DegenerateReduces(const Graph& g, const ir::Chain& c) {
  for (const auto& r : c.reduces)
    if (g.dims[r.axis].extent != 1) return false;
  return true;
}

std::vector<int> DropUnit(const Graph& g, const std::vector<int>& axes) {
  std::vector<int> out;
  for (int a : axes)
    if (g.dims[a].extent != 1) out.push_back(a);
  return out;
}

class Emitter {
 public:
  Emitter(const Graph& g, const Options& o) : g_(g), opts_(o) {
    prefix_ = opts_.kernel_name.empty() ? g.name : opts_.kernel_name;
    std::string clean;
    for (char ch : prefix_) clean += (isalnum(static_cast<unsigned char>(ch)) || ch == '_') ? ch : '_';
    prefix_ = "tca_" + clean;
  }

  bool Run(Result* out, std::string* err) {
    if (opts_.target != "gfx950") {
      *err = "emit: unsupported target " + opts_.target + " (this backend emits CDNA4 code for gfx950 only)";
      return false;
    }
    Analyze();
    src_ << "// Generated by the tcacomp HIP emitter for " << opts_.target << ". Do not edit.\n";
    src_ << "// program: " << g_.name << "\n";
    src_ << "#include \"tca/hip/device.h\"\n";
    if (uses_gemm_) src_ << "#include \"tca/hip/gemm.h\"\n";
    src_ << "\n";
    for (size_t ni = 0; ni < an_.nests.size(); ++ni) {
      if (!EmitNest(static_cast<int>(ni), err)) return false;
    }
    if (an_.nests.empty()) {
      *err = "emit: program " + g_.name + " stores no output";
      return false;
    }
    out->source = src_.str();
    out->plan = PlanText();
    out->hipcc = DeviceFlags(opts_.target);
    out->kernels = kernels_;
    std::ostringstream rep;
    for (const auto& k : kernels_) {
      rep << k.symbol << " " << FamilyName(k.family) << " chains=";
      for (size_t i = 0; i < k.chains.size(); ++i) rep << (i ? "," : "") << k.chains[i];
      rep << " " << k.detail << "\n";
    }
    out->report = rep.str();
    return true;
  }

 private:
  struct PlanKernel {
    std::string symbol;
    uint32_t block = 256, lds = 0;
    std::vector<std::string> grid;
    std::vector<std::string> args;
    std::vector<std::string> when;  // launch guards: "<dim> <lo> <hi> <mod> <rem>"
    std::vector<std::string> unless;  // skip guards: the kernel is skipped when all of them hold
    std::string pack;               // packed row kernel: "<dim> <epl> <min block>"
    std::string split;              // row-split reduction: "<dim> <rows-min> <blocks> <merge> <n> <terms>"
  };

  // -------------------------------------------------------------- analysis
  void Analyze() {
    const int nc = static_cast<int>(g_.chains.size());
    an_.live.assign(nc, false);
    std::set<int> needed;
    for (int i = nc - 1; i >= 0; --i) {
      const ir::Chain& c = g_.chains[i];
      const ir::Tensor& t = g_.tensors[c.store_tensor];
      bool live = !t.local || needed.count(c.store_tensor);
      if (!live) continue;
      an_.live[i] = true;
      if (t.local) needed.erase(c.store_tensor);
      for (int r : ReadSet(c))
        if (g_.tensors[r].local) needed.insert(r);
    }
    // Nest fusion.
    std::vector<int> cur;
    auto close = [&]() {
      if (cur.empty()) return;
      Nest n;
      n.chains = cur;
      n.family = ClassifyNest(cur);
      an_.nests.push_back(n);
      cur.clear();
    };
    for (int i = 0; i < nc; ++i) {
      if (!an_.live[i]) continue;
      if (!cur.empty() && opts_.allow_fused) {
        std::vector<int> cand = cur;
        cand.push_back(i);
        if ((RowCheck(g_, cand, RowNV()).ok || StreamCheck(g_, cand).ok || ColCheck(g_, cand).ok) && !IsGemm(cur)) {
          cur = cand;
          continue;
        }
      }
      close();
      cur.push_back(i);
    }
    close();
    // Local placement.
    an_.hbm_local.assign(g_.tensors.size(), false);
    an_.reg_nest.assign(g_.tensors.size(), -1);
    for (size_t t = 0; t < g_.tensors.size(); ++t) {
      if (!g_.tensors[t].local) continue;
      int producer = -1;
      std::set<int> readers;
      for (size_t ni = 0; ni < an_.nests.size(); ++ni) {
        for (int ci : an_.nests[ni].chains) {
          if (g_.chains[ci].store_tensor == static_cast<int>(t)) producer = static_cast<int>(ni);
          if (ReadSet(g_.chains[ci]).count(static_cast<int>(t))) readers.insert(static_cast<int>(ni));
        }
      }
      if (producer < 0) continue;  // dead local
      const Family pf = an_.nests[producer].family;
      bool fused = (pf == Family::Row || pf == Family::Stream) && readers.size() == 1 && readers.count(producer);
      if (fused) an_.reg_nest[t] = producer;
      else an_.hbm_local[t] = true;
    }
    for (const auto& n : an_.nests) uses_gemm_ |= (n.family == Family::Gemm);
    // Chained reductions folded in one kernel.
    for (size_t ni = 0; ni + 1 < an_.nests.size(); ++ni) {
      std::string guard;
      if (an_.nests[ni].seg || !MatchSeg(static_cast<int>(ni), &guard)) continue;
      an_.nests[ni].seg = 1;
      an_.nests[ni + 1].seg = 2;
      an_.nests[ni].seg_guard = an_.nests[ni + 1].seg_guard = guard;
      if (guard.empty()) {  // the local never exists
        const int L = g_.chains[an_.nests[ni].chains[0]].store_tensor;
        an_.hbm_local[L] = false;
        an_.reg_nest[L] = -1;
      }
    }
  }

  // Segments per block of the segment kernel below which the two nests'
  // own kernels run instead (they spread a segment over many blocks).
  static constexpr uint64_t kSegMin = 1024;

  // A row reduction into a local L (S..., r), then the next nest's single
  // chain reducing L over r into (S...): the pattern a chained reduction
  // splits into (row sums, then their max over the rows of each batch),
  // and any program written that way. The segment kernel folds both with
  // one block per segment (an output of the outer reduction), L never
  // leaving registers. Requires: the inner nest is one chain of the row or
  // streaming family with one reduction, no piped map, storing the local
  // at its rows; the outer chain iterates exactly those rows, reads L there
  // and otherwise only per-segment operands, has one associative-
  // commutative reduction over r and stores at (S...); no other chain
  // reads L. *guard receives the segment dim when its extent is a run-time
  // value (then S must be that one dim), empty when the extents are known
  // (then at least kSegMin segments).
  bool MatchSeg(int ni, std::string* guard) {
    if (!opts_.allow_fused) return false;
    const Nest& in = an_.nests[ni];
    const Nest& out = an_.nests[ni + 1];
    if (in.chains.size() != 1 || out.chains.size() != 1) return false;
    if (in.family != Family::Row && in.family != Family::Stream) return false;
    const int ci = in.chains[0], cj = out.chains[0];
    const ir::Chain& a = g_.chains[ci];
    const ir::Chain& b = g_.chains[cj];
    if (a.reduces.size() != 1 || a.has_piped) return false;
    const int L = a.store_tensor;
    if (!g_.tensors[L].local) return false;
    RowGeom geo;
    if (!RowShape(g_, {ci}, true, &geo) || geo.outer.empty() || a.root.as != geo.as) return false;
    if (a.store_axes != geo.outer) return false;
    const std::vector<int> S(geo.outer.begin(), geo.outer.end() - 1);
    if (S.empty()) return false;
    if (b.root.as != geo.outer || b.reduces.size() != 1 || !IsMonoidCombiner(g_, b.reduces[0])) return false;
    if (b.store_axes != S) return false;
    auto segShaped = [&](const ir::Operand& o) {
      for (int x : o.axes)
        if (std::find(S.begin(), S.end(), x) == S.end()) return false;
      return true;
    };
    bool readsL = false;
    for (const auto& o : b.root.ops) {
      if (o.tensor == L) {
        if (o.axes != geo.outer) return false;
        readsL = true;
      } else if (!segShaped(o)) {
        return false;
      }
    }
    if (!readsL) return false;
    if (b.has_piped)
      for (const auto& o : b.piped.ops)
        if (o.tensor == L || !segShaped(o)) return false;
    if (ReadSet(a).count(b.store_tensor)) return false;
    for (size_t k = 0; k < g_.chains.size(); ++k)
      if (an_.live[k] && static_cast<int>(k) != cj && ReadSet(g_.chains[k]).count(L)) return false;
    bool dynamic = false;
    uint64_t nseg = 1;
    for (int d : S) {
      if (g_.dims[d].extent == 0) dynamic = true;
      else nseg *= g_.dims[d].extent;
    }
    if (!dynamic) {
      guard->clear();
      return nseg >= kSegMin;
    }
    if (S.size() != 1) return false;
    *guard = g_.dims[S[0]].name;
    return true;
  }

  bool IsGemm(const std::vector<int>& chains) {
    if (!opts_.allow_gemm || chains.size() != 1) return false;
    GemmMatch m;
    return MatchGemm(g_, g_.chains[chains[0]], &m);
  }

  Family ClassifyNest(const std::vector<int>& chains) {
    if (chains.size() == 1) {
      const ir::Chain& c = g_.chains[chains[0]];
      if (IsGemm(chains)) return Family::Gemm;
      if (opts_.allow_fused && DegenerateReduces(g_, c) && !ReadsRegLocalCandidate(c)) return Family::Elementwise;
      if (opts_.allow_fused && RowCheck(g_, chains, RowNV()).ok) return Family::Row;
      if (opts_.allow_fused && StreamCheck(g_, chains).ok) return Family::Stream;
      if (opts_.allow_fused && ColCheck(g_, chains).ok) return Family::Col;
      return Family::Generic;
    }
    if (RowCheck(g_, chains, RowNV()).ok) return Family::Row;
    return StreamCheck(g_, chains).ok ? Family::Stream : Family::Col;
  }

  bool ReadsRegLocalCandidate(const ir::Chain&) { return false; }

  // Geometry defaults, swept on MI355X: 4 16-byte vectors per lane for fused
  // rows (softmax 4096: 6.31 TB/s vs 6.00 at 8; layernorm 1024: 5.94 vs 5.77)
  // and 4 per operand and thread for elementwise streams.
  uint32_t RowNV() const { return opts_.row_vectors_per_lane > 0 ? static_cast<uint32_t>(opts_.row_vectors_per_lane) : 4u; }
  uint32_t EwUnroll() const { return opts_.elementwise_unroll > 0 ? static_cast<uint32_t>(opts_.elementwise_unroll) : 4u; }

  // ------------------------------------------------------------- plumbing
  std::set<int> NestTensors(const Nest& n) {
    std::set<int> ts;
    for (int ci : n.chains) {
      const ir::Chain& c = g_.chains[ci];
      for (int t : ReadSet(c)) ts.insert(t);
      ts.insert(c.store_tensor);
    }
    std::set<int> out;
    for (int t : ts)
      if (!g_.tensors[t].local || an_.hbm_local[t]) out.insert(t);
    return out;
  }

  std::set<int> NestScalars(const Nest& n) {
    std::set<int> s;
    for (int ci : n.chains) {
      auto cs = ChainScalars(g_, g_.chains[ci]);
      s.insert(cs.begin(), cs.end());
    }
    return s;
  }

  bool IsStoredInNest(const Nest& n, int t) {
    for (int ci : n.chains)
      if (g_.chains[ci].store_tensor == t) return true;
    return false;
  }

  // Kernel signature: tensors (declaration order), all dims, used scalars.
  std::string Signature(const Nest& n, PlanKernel* pk) {
    std::ostringstream s;
    bool first = true;
    auto sep = [&]() {
      if (!first) s << ",\n    ";
      first = false;
    };
    for (int t : NestTensors(n)) {
      sep();
      const bool written = IsStoredInNest(n, t);
      s << (written ? "" : "const ") << CType(g_.tensors[t].elem) << "* __restrict__ t" << t << " /* "
        << g_.tensors[t].name << " */";
      pk->args.push_back("ptr " + g_.tensors[t].name);
    }
    for (size_t d = 0; d < g_.dims.size(); ++d) {
      sep();
      s << "uint32_t d" << d << " /* @" << g_.dims[d].name << " */";
      pk->args.push_back("dim " + g_.dims[d].name);
    }
    for (int sc : NestScalars(n)) {
      sep();
      s << ScalarArgType(g_.scalars[sc].elem) << " s" << sc << " /* " << g_.scalars[sc].name << " */";
      pk->args.push_back("scalar " + g_.scalars[sc].name);
    }
    return s.str();
  }

  std::string DimProduct(const std::vector<int>& axes) {
    if (axes.empty()) return "1";
    std::string s;
    for (size_t i = 0; i < axes.size(); ++i) s += (i ? "*" : "") + g_.dims[axes[i]].name;
    return s;
  }

  // Flat row-major offset of operand/store `axes` over tensor t, with the
  // coordinate of axis a spelled coord(a).
  std::string Offset(int t, const std::vector<int>& axes, const std::function<std::string(int)>& coord) {
    const ir::Tensor& tt = g_.tensors[t];
    if (axes.empty()) return "0u";
    std::string off = coord(axes[0]);
    for (size_t i = 1; i < axes.size(); ++i)
      off = "(" + off + ") * " + ExtentExpr(g_, tt.dims[i]) + " + " + coord(axes[i]);
    return off;
  }

  std::string Indent(int n) { return std::string(static_cast<size_t>(n) * 2, ' '); }

  // ------------------------------------------------------------- families
  bool EmitNest(int ni, std::string* err) {
    const Nest& n = an_.nests[ni];
    if (n.seg == 1 && !EmitSeg(ni, err)) return false;
    if (n.seg && n.seg_guard.empty()) return true;  // the segment kernel alone
    const size_t k0 = plan_kernels_.size();
    if (!EmitFamily(ni, err)) return false;
    if (n.seg)  // the two nests' own kernels: fewer segments than kSegMin
      for (size_t k = k0; k < plan_kernels_.size(); ++k)
        plan_kernels_[k].when.push_back(n.seg_guard + " 0 " + std::to_string(kSegMin - 1) + " 1 0");
    return true;
  }

  bool EmitFamily(int ni, std::string* err) {
    const Nest& n = an_.nests[ni];
    switch (n.family) {
      case Family::Elementwise: return EmitElementwise(ni, err);
      case Family::Row: return EmitRow(ni, err);
      case Family::Stream: return EmitStream(ni, err);
      case Family::Col: return EmitCol(ni, err);
      case Family::Gemm: return EmitGemmNest(ni, err);
      case Family::Generic: return EmitGeneric(ni, err);
      case Family::Seg: break;  // emitted with its inner nest (EmitSeg)
    }
    return false;
  }

  // E: flat streaming over the stored tensor; operands whose non-unit axes
  // match the store's are read with 16-byte vector loads, others by index.
  // ---- elementwise maps with transposed operands: 64x64 tiles through LDS
  // An operand contiguous along the second-innermost store axis P (its last
  // index) while the store is contiguous along the innermost axis L is read
  // across rows by a flat strip: every lane a different cache line. Here a
  // 256-thread block owns a 64 (P) x 64 (L) output tile. Each such operand's
  // [64 L][64 P] tile is read with 16-byte loads along P, staged in LDS rows
  // of 65 floats (the odd stride puts the 64 lanes of both the row-wise
  // writes and the column-wise reads on 64 distinct banks), and read back
  // transposed; the output, and operands aligned with it along L, move as
  // 16-byte vectors along L. 4-byte element types only, at most 4 such
  // operands (66 KiB of LDS). With at most 2 such operands the tile is
  // 128 x 128 for a 1024-thread block (LDS rows of 129 floats, 66 KiB per
  // operand): measured on y = x * g[c] + b[r] + z^T at 8192^2, 125.8 us
  // against 164 us for 64 x 64 tiles (128 x 64: 141, 64 x 128: 134,
  // 128 x 128 with 512 or 256 threads: 130 / 133, 128 x 256: 132); the
  // longer row segments each block reads and writes (512 bytes) are what
  // pays.
  static constexpr int kTrTile = 64, kTrMax = 4, kTrLarge = 128, kTrMaxLarge = 2;

  enum class TileCls { Aligned, RowVec, Bcast, Tr, Other };

  // The class of operand `op` in a tile over (P, L).
  TileCls TileClass(const ir::Operand& op, const std::vector<int>& outAxes, int P, int L) const {
    if (DropUnit(g_, op.axes) == outAxes) return TileCls::Aligned;
    int atL = -1, atP = -1, usesL = 0, usesP = 0;
    for (size_t i = 0; i < op.axes.size(); ++i) {
      if (op.axes[i] == L) atL = static_cast<int>(i), ++usesL;
      if (op.axes[i] == P) atP = static_cast<int>(i), ++usesP;
    }
    auto lastNonUnit = [&]() {
      for (int i = static_cast<int>(op.axes.size()) - 1; i >= 0; --i)
        if (g_.dims[op.axes[i]].extent != 1) return i;
      return -1;
    };
    const int last = lastNonUnit();
    if (usesL == 0) return TileCls::Bcast;
    if (usesL == 1 && last == atL) return TileCls::RowVec;
    if (usesL == 1 && usesP == 1 && last == atP) return TileCls::Tr;
    return TileCls::Other;
  }

  // Whether chain c takes the tiled kernel: two or more non-unit store axes,
  // 4-byte elements throughout, and 1..kTrMax transposed operands.
  bool TiledElementwise(const ir::Chain& c) const {
    const std::vector<int> outAxes = DropUnit(g_, c.store_axes);
    if (outAxes.size() < 2) return false;
    const int L = outAxes.back(), P = outAxes[outAxes.size() - 2];
    if (ir::ElemBytes(g_.tensors[c.store_tensor].elem) != 4) return false;
    int tr = 0;
    auto scan = [&](const std::vector<ir::Operand>& ops) {
      for (const auto& op : ops) {
        if (ir::ElemBytes(g_.tensors[op.tensor].elem) != 4) return false;
        if (TileClass(op, outAxes, P, L) == TileCls::Tr) ++tr;
      }
      return true;
    };
    if (!scan(c.root.ops)) return false;
    if (c.has_piped && !scan(c.piped.ops)) return false;
    return tr >= 1 && tr <= kTrMax;
  }

  bool EmitElementwiseTiled(int ni) {
    const Nest& n = an_.nests[ni];
    const ir::Chain& c = g_.chains[n.chains[0]];
    const std::vector<int> outAxes = DropUnit(g_, c.store_axes);
    const int L = outAxes.back(), P = outAxes[outAxes.size() - 2];
    const std::vector<int> outer(outAxes.begin(), outAxes.end() - 2);
    // Tile edge T: 128 while the LDS tiles (T (T + 1) floats each) fit two
    // workgroups per CU, else 64. Q = T / 4 lanes per row of 4-element
    // vectors, and Q rows per step of the T * T / 16 threads.
    int nTr = 0;
    for (const auto& op : c.root.ops) nTr += TileClass(op, outAxes, P, L) == TileCls::Tr;
    if (c.has_piped)
      for (const auto& op : c.piped.ops) nTr += TileClass(op, outAxes, P, L) == TileCls::Tr;
    const int T = nTr <= kTrMaxLarge ? kTrLarge : kTrTile, Q = T / 4, S = T + 1, NT = T * T / 16;
    const std::string Ts = std::to_string(T) + "u", Qs = std::to_string(Q) + "u", Ss = std::to_string(S) + "u";
    PlanKernel pk;
    pk.symbol = Sym(g_, prefix_, ni);
    pk.block = NT;
    pk.grid.push_back(DimProduct(outer) + "/1");
    pk.grid.push_back(g_.dims[P].name + "/" + std::to_string(T));
    pk.grid.push_back(g_.dims[L].name + "/" + std::to_string(T));
    const std::string sig = Signature(n, &pk);
    std::ostringstream& o = src_;
    const ir::Tensor& st = g_.tensors[c.store_tensor];
    const std::string sT = CType(st.elem), EL = ExtentExpr(g_, L), EP = ExtentExpr(g_, P);
    struct OpRef {
      bool piped;
      int k;
      const ir::Operand* op;
      TileCls cls;
      int tile;  // LDS tile index of a Tr operand
    };
    std::vector<OpRef> ops;
    int nTiles = 0;
    for (size_t k = 0; k < c.root.ops.size(); ++k) {
      const TileCls cls = TileClass(c.root.ops[k], outAxes, P, L);
      ops.push_back({false, static_cast<int>(k), &c.root.ops[k], cls, cls == TileCls::Tr ? nTiles++ : -1});
    }
    if (c.has_piped)
      for (size_t k = 0; k < c.piped.ops.size(); ++k) {
        const TileCls cls = TileClass(c.piped.ops[k], outAxes, P, L);
        ops.push_back({true, static_cast<int>(k), &c.piped.ops[k], cls, cls == TileCls::Tr ? nTiles++ : -1});
      }
    auto find = [&](bool piped, int k) -> const OpRef& {
      for (const auto& r : ops)
        if (r.piped == piped && r.k == k) return r;
      return ops.front();
    };
    o << "// statement #" << n.chains[0] << ": elementwise family, " << T << "x" << T << " tiles, " << nTiles
      << " transposed operand(s) staged in LDS\n";
    o << "extern \"C\" __global__ void __launch_bounds__(" << NT << ") " << pk.symbol << "(\n    " << sig << ") {\n";
    o << "  __shared__ uint32_t tr_lds[" << nTiles << "][" << T * S << "];\n";
    o << "  const uint32_t nl = tca::hip::ceil_div(" << EL << ", " << Ts << "), np = tca::hip::ceil_div(" << EP << ", "
      << Ts << ");\n";
    o << "  uint32_t bid = blockIdx.x;\n";
    o << "  const uint32_t l0 = (bid % nl) * " << Ts << "; bid /= nl;\n";
    o << "  const uint32_t p0 = (bid % np) * " << Ts << "; bid /= np;\n";
    for (int i = static_cast<int>(outer.size()) - 1; i >= 0; --i)
      o << "  const uint32_t c" << outer[i] << " = bid % " << ExtentExpr(g_, outer[i]) << "; bid /= "
        << ExtentExpr(g_, outer[i]) << ";\n";
    o << "  const uint32_t tr = threadIdx.x / " << Qs << ", tc = threadIdx.x % " << Qs << ";\n";
    // Coordinates: L and P spelled by the caller, outer axes c<a>, unit 0.
    auto coordFn = [&](const std::string& l, const std::string& p) {
      return [this, l, p, L, P](int a) -> std::string {
        if (g_.dims[a].extent == 1) return "0u";
        if (a == L) return l;
        if (a == P) return p;
        return "c" + std::to_string(a);
      };
    };
    // 1. Output rows p0 + tr + Q i, 4 L values each. The operands read
    // straight from memory are loaded first, so their latency overlaps the
    // tile's (whose LDS writes wait for its own loads).
    o << "  const bool l_vec = " << EL << " % 4u == 0u;\n";
    o << "  const uint32_t lb = l0 + 4u * tc;\n";
    o << "  bool full[4];\n";
    for (const auto& r : ops) {
      const std::string T = CType(g_.tensors[r.op->tensor].elem);
      const std::string nm = std::string(r.piped ? "tp" : "ta") + std::to_string(r.k);
      if (r.cls == TileCls::Aligned || r.cls == TileCls::RowVec)
        o << "  tca::hip::vec<" << T << ", 4> " << nm << "[4];\n";
      else if (r.cls == TileCls::Bcast)
        o << "  " << T << " " << nm << "[4];\n";
    }
    o << "#pragma unroll\n  for (uint32_t i = 0; i < 4u; ++i) {\n";
    o << "    const uint32_t p = p0 + tr + " << Qs << " * i;\n";
    o << "    full[i] = p < " << EP << " && l_vec && lb + 3u < " << EL << ";\n";
    o << "    if (full[i]) {\n";
    for (const auto& r : ops) {
      const std::string T = CType(g_.tensors[r.op->tensor].elem), t = "t" + std::to_string(r.op->tensor);
      const std::string nm = std::string(r.piped ? "tp" : "ta") + std::to_string(r.k);
      // Aligned operands are read once (streamed); row-contiguous ones are
      // re-read by every row of the grid.
      if (r.cls == TileCls::Aligned || r.cls == TileCls::RowVec)
        o << "      " << nm << "[i] = tca::hip::load_vec" << (r.cls == TileCls::Aligned ? "_nt" : "") << "<" << T
          << ", 4>(" << t << " + " << Offset(r.op->tensor, r.op->axes, coordFn("lb", "p")) << ");\n";
      else if (r.cls == TileCls::Bcast)
        o << "      " << nm << "[i] = " << t << "[" << Offset(r.op->tensor, r.op->axes, coordFn("lb", "p")) << "];\n";
    }
    o << "    }\n  }\n";
    // 2. Transposed operands: rows l0 + tr + Q i of the [L][P] tile, 4 P values each.
    o << "  const bool p_vec = " << EP << " % 4u == 0u;\n";
    for (const auto& r : ops) {
      if (r.cls != TileCls::Tr) continue;
      const std::string T = CType(g_.tensors[r.op->tensor].elem), t = "t" + std::to_string(r.op->tensor);
      const std::string zv = "zv" + std::to_string(r.tile), zf = "zf" + std::to_string(r.tile);
      // All four row loads first, then the LDS writes (which wait for them).
      o << "  tca::hip::vec<" << T << ", 4> " << zv << "[4];\n  bool " << zf << "[4];\n";
      o << "#pragma unroll\n  for (uint32_t i = 0; i < 4u; ++i) {\n";
      o << "    const uint32_t l = l0 + tr + " << Qs << " * i, p = p0 + 4u * tc;\n";
      o << "    " << zf << "[i] = l < " << EL << " && p_vec && p + 3u < " << EP << ";\n";
      o << "    if (" << zf << "[i]) " << zv << "[i] = tca::hip::load_vec_nt<" << T << ", 4>(" << t << " + "
        << Offset(r.op->tensor, r.op->axes, coordFn("l", "p")) << ");\n";
      o << "  }\n";
      o << "#pragma unroll\n  for (uint32_t i = 0; i < 4u; ++i) {\n";
      o << "    const uint32_t lr = tr + " << Qs << " * i, l = l0 + lr, p = p0 + 4u * tc;\n";
      o << "    uint32_t* row = &tr_lds[" << r.tile << "][lr * " << Ss << " + 4u * tc];\n";
      o << "    if (" << zf << "[i]) {\n";
      o << "#pragma unroll\n      for (uint32_t j = 0; j < 4u; ++j) row[j] = __builtin_bit_cast(uint32_t, " << zv
        << "[i][j]);\n";
      o << "    } else {\n";
      o << "      for (uint32_t j = 0; j < 4u; ++j)\n";
      o << "        if (l < " << EL << " && p + j < " << EP << ") row[j] = __builtin_bit_cast(uint32_t, " << t << "["
        << Offset(r.op->tensor, r.op->axes, coordFn("l", "(p + j)")) << "]);\n";
      o << "    }\n  }\n";
    }
    o << "  __syncthreads();\n";
    // 3. Compute and store.
    o << "#pragma unroll\n  for (uint32_t i = 0; i < 4u; ++i) {\n";
    o << "    const uint32_t pr = tr + " << Qs << " * i, p = p0 + pr;\n";
    o << "    if (p >= " << EP << ") continue;\n";
    auto trVal = [&](const OpRef& r, const std::string& lr) {
      return "__builtin_bit_cast(" + CType(g_.tensors[r.op->tensor].elem) + ", tr_lds[" + std::to_string(r.tile) +
             "][(" + lr + ") * " + Ss + " + pr])";
    };
    // Whole vector along L.
    o << "    if (full[i]) {\n";
    {
      o << "      tca::hip::vec<" << sT << ", 4> out{};\n";
      o << "#pragma unroll\n      for (uint32_t q = 0; q < 4u; ++q) {\n";
      std::ostringstream bodyS;
      std::string val = TiledBody(c, bodyS, Indent(4), [&](bool piped, int k) -> std::string {
        const OpRef& r = find(piped, k);
        const std::string nm = std::string(piped ? "tp" : "ta") + std::to_string(k);
        switch (r.cls) {
          case TileCls::Aligned:
          case TileCls::RowVec: return nm + "[i][q]";
          case TileCls::Bcast: return nm + "[i]";
          case TileCls::Tr: return trVal(r, "4u * tc + q");
          case TileCls::Other: break;
        }
        return "t" + std::to_string(r.op->tensor) + "[" + Offset(r.op->tensor, r.op->axes, coordFn("(lb + q)", "p")) + "]";
      });
      o << bodyS.str();
      o << "        out.set(q, " << val << ");\n";
      o << "      }\n";
      o << "      tca::hip::store_vec_nt<" << sT << ", 4>(t" << c.store_tensor << " + "
        << Offset(c.store_tensor, c.store_axes, coordFn("lb", "p")) << ", out);\n";
    }
    // Ragged edge or L not a multiple of 4: element by element.
    o << "    } else {\n";
    o << "      for (uint32_t q = 0; q < 4u; ++q) {\n";
    o << "        if (lb + q >= " << EL << ") break;\n";
    {
      std::ostringstream bodyS;
      std::string val = TiledBody(c, bodyS, Indent(4), [&](bool piped, int k) -> std::string {
        const OpRef& r = find(piped, k);
        if (r.cls == TileCls::Tr) return trVal(r, "4u * tc + q");
        return "t" + std::to_string(r.op->tensor) + "[" + Offset(r.op->tensor, r.op->axes, coordFn("(lb + q)", "p")) + "]";
      });
      o << bodyS.str();
      o << "        t" << c.store_tensor << "[" << Offset(c.store_tensor, c.store_axes, coordFn("(lb + q)", "p"))
        << "] = " << val << ";\n";
    }
    o << "      }\n    }\n  }\n}\n\n";
    AddKernel(pk, Family::Elementwise, n.chains,
              "tile=" + std::to_string(T) + "x" + std::to_string(T) + " lds_tiles=" + std::to_string(nTiles) +
                  " block=" + std::to_string(NT));
    return true;
  }

  // The element body of chain c (root map, degenerate reduces, piped map)
  // with operand values from `val(piped, k)`.
  std::string TiledBody(const ir::Chain& c, std::ostringstream& os, const std::string& ind,
                        const std::function<std::string(bool, int)>& val) {
    ExprGen eg(g_, os, ind, &counter_);
    for (size_t k = 0; k < c.root.ops.size(); ++k) eg.Bind(c.root.fn.params[k], val(false, static_cast<int>(k)));
    std::string v = eg.Gen(c.root.fn.body);
    for (const auto& r : c.reduces) {
      ExprGen rg(g_, os, ind, &counter_);
      rg.Bind(r.fn.params[0], rg.Gen(r.init));
      rg.Bind(r.fn.params[1], v);
      v = rg.Gen(r.fn.body);
    }
    if (c.has_piped) {
      ExprGen pg(g_, os, ind, &counter_);
      pg.Bind(c.piped.fn.params[0], v);
      for (size_t k = 0; k < c.piped.ops.size(); ++k) pg.Bind(c.piped.fn.params[k + 1], val(true, static_cast<int>(k)));
      v = pg.Gen(c.piped.fn.body);
    }
    return v;
  }

  bool EmitElementwise(int ni, std::string* err) {
    (void)err;
    const Nest& n = an_.nests[ni];
    const ir::Chain& c = g_.chains[n.chains[0]];
    if (TiledElementwise(c)) return EmitElementwiseTiled(ni);
    PlanKernel pk;
    pk.symbol = Sym(g_, prefix_, ni);
    // Elements per vector: 16 bytes of the widest tensor moved in vectors
    // (the store and the operands aligned with it).
    size_t widest = ir::ElemBytes(g_.tensors[c.store_tensor].elem);
    {
      const std::vector<int> storeAxes = DropUnit(g_, c.store_axes);
      for (const auto& op : c.root.ops)
        if (DropUnit(g_, op.axes) == storeAxes) widest = std::max(widest, ir::ElemBytes(g_.tensors[op.tensor].elem));
      if (c.has_piped)
        for (const auto& op : c.piped.ops)
          if (DropUnit(g_, op.axes) == storeAxes) widest = std::max(widest, ir::ElemBytes(g_.tensors[op.tensor].elem));
    }
    const uint32_t kVec = static_cast<uint32_t>(std::max<size_t>(1, 16 / widest)), kUnroll = EwUnroll(), kBlock = 256,
                   kPerBlock = kVec * kUnroll * kBlock;
    pk.block = kBlock;
    pk.grid.push_back(DimProduct(c.store_axes) + "/" + std::to_string(kPerBlock));
    const std::string sig = Signature(n, &pk);
    const std::vector<int> outAxes = DropUnit(g_, c.store_axes);
    std::ostringstream& o = src_;
    o << "// statement #" << n.chains[0] << ": elementwise family, " << kVec << "-wide vectors x " << kUnroll
      << " per thread\n";
    o << "extern \"C\" __global__ void __launch_bounds__(" << kBlock << ") " << pk.symbol << "(\n    " << sig
      << ") {\n";
    o << "  const uint32_t n = " << ProductExpr(c.store_axes) << ";\n";
    o << "  const uint64_t base = static_cast<uint64_t>(blockIdx.x) * " << kPerBlock << "u + threadIdx.x * " << kVec
      << "u;\n";
    // Operand classes.
    struct Acc {
      bool aligned;
    };
    std::vector<bool> rootAligned, pipedAligned;
    for (const auto& op : c.root.ops) rootAligned.push_back(DropUnit(g_, op.axes) == outAxes);
    if (c.has_piped)
      for (const auto& op : c.piped.ops) pipedAligned.push_back(DropUnit(g_, op.axes) == outAxes);
    const ir::Tensor& st = g_.tensors[c.store_tensor];
    // Coordinates of element index `i` (only needed by unaligned operands).
    auto coordDecl = [&](std::ostringstream& os, const std::string& ind, const std::string& idx) {
      std::string rem = "rem_" + idx;
      os << ind << "uint32_t " << rem << " = static_cast<uint32_t>(" << idx << ");\n";
      for (int k = static_cast<int>(c.store_axes.size()) - 1; k >= 0; --k) {
        int a = c.store_axes[k];
        os << ind << "const uint32_t c" << a << "_" << idx << " = " << rem << " % " << ExtentExpr(g_, a) << "; "
           << rem << " /= " << ExtentExpr(g_, a) << ";\n";
      }
    };
    bool anyUnaligned = false;
    for (bool b : rootAligned) anyUnaligned |= !b;
    for (bool b : pipedAligned) anyUnaligned |= !b;
    // Element body: value of element with flat index expression `idx`, where
    // aligned operand k's value is `al(k)`.
    auto body = [&](std::ostringstream& os, const std::string& ind, const std::string& idx,
                    const std::function<std::string(bool piped, int k)>& alignedVal) -> std::string {
      if (anyUnaligned) coordDecl(os, ind, idx);
      auto coord = [&](int a) -> std::string {
        if (g_.dims[a].extent == 1) return "0u";
        return "c" + std::to_string(a) + "_" + idx;
      };
      ExprGen eg(g_, os, ind, &counter_);
      for (size_t k = 0; k < c.root.ops.size(); ++k) {
        const auto& op = c.root.ops[k];
        std::string v = rootAligned[k] ? alignedVal(false, static_cast<int>(k))
                                       : "t" + std::to_string(op.tensor) + "[" + Offset(op.tensor, op.axes, coord) + "]";
        eg.Bind(c.root.fn.params[k], v);
      }
      std::string val = eg.Gen(c.root.fn.body);
      for (const auto& r : c.reduces) {
        ExprGen rg(g_, os, ind, &counter_);
        rg.Bind(r.fn.params[0], rg.Gen(r.init));
        rg.Bind(r.fn.params[1], val);
        val = rg.Gen(r.fn.body);
      }
      if (c.has_piped) {
        ExprGen pg(g_, os, ind, &counter_);
        pg.Bind(c.piped.fn.params[0], val);
        for (size_t k = 0; k < c.piped.ops.size(); ++k) {
          const auto& op = c.piped.ops[k];
          std::string v = pipedAligned[k] ? alignedVal(true, static_cast<int>(k))
                                          : "t" + std::to_string(op.tensor) + "[" + Offset(op.tensor, op.axes, coord) + "]";
          pg.Bind(c.piped.fn.params[k + 1], v);
        }
        val = pg.Gen(c.piped.fn.body);
      }
      return val;
    };
    // The element body with every operand's value given by `val(piped, k)`.
    auto bodyWith = [&](std::ostringstream& os, const std::string& ind,
                        const std::function<std::string(bool piped, int k)>& val) -> std::string {
      ExprGen eg(g_, os, ind, &counter_);
      for (size_t k = 0; k < c.root.ops.size(); ++k) eg.Bind(c.root.fn.params[k], val(false, static_cast<int>(k)));
      std::string v = eg.Gen(c.root.fn.body);
      for (const auto& r : c.reduces) {
        ExprGen rg(g_, os, ind, &counter_);
        rg.Bind(r.fn.params[0], rg.Gen(r.init));
        rg.Bind(r.fn.params[1], v);
        v = rg.Gen(r.fn.body);
      }
      if (c.has_piped) {
        ExprGen pg(g_, os, ind, &counter_);
        pg.Bind(c.piped.fn.params[0], v);
        for (size_t k = 0; k < c.piped.ops.size(); ++k) pg.Bind(c.piped.fn.params[k + 1], val(true, static_cast<int>(k)));
        v = pg.Gen(c.piped.fn.body);
      }
      return v;
    };
    // Fast path: the whole strip is in range.
    o << "  if (base + " << (kUnroll - 1) * kVec * kBlock + kVec - 1 << "u < n) {\n";
    for (size_t k = 0; k < c.root.ops.size(); ++k) {
      if (!rootAligned[k]) continue;
      const auto& op = c.root.ops[k];
      o << "    tca::hip::vec<" << CType(g_.tensors[op.tensor].elem) << ", " << kVec << "> a" << k << "[" << kUnroll
        << "];\n";
    }
    for (size_t k = 0; k < pipedAligned.size(); ++k) {
      if (!pipedAligned[k]) continue;
      const auto& op = c.piped.ops[k];
      o << "    tca::hip::vec<" << CType(g_.tensors[op.tensor].elem) << ", " << kVec << "> p" << k << "[" << kUnroll
        << "];\n";
    }
    o << "#pragma unroll\n    for (uint32_t u = 0; u < " << kUnroll << "u; ++u) {\n";
    for (size_t k = 0; k < c.root.ops.size(); ++k) {
      if (!rootAligned[k]) continue;
      const auto& op = c.root.ops[k];
      o << "      a" << k << "[u] = tca::hip::load_vec_nt<" << CType(g_.tensors[op.tensor].elem) << ", " << kVec << ">(t"
        << op.tensor << " + base + u * " << kVec * kBlock << "u);\n";
    }
    for (size_t k = 0; k < pipedAligned.size(); ++k) {
      if (!pipedAligned[k]) continue;
      const auto& op = c.piped.ops[k];
      o << "      p" << k << "[u] = tca::hip::load_vec_nt<" << CType(g_.tensors[op.tensor].elem) << ", " << kVec << ">(t"
        << op.tensor << " + base + u * " << kVec * kBlock << "u);\n";
    }
    o << "    }\n";
    // Operands not aligned with the store (broadcast or permuted), when the
    // innermost store extent is a multiple of the vector width (a uniform
    // test at run time): a vector never crosses a row, so its coordinates are
    // decomposed once, an operand whose last index is the innermost axis
    // (contiguous there) is one vector load, and an operand that does not
    // depend on that axis is one scalar load per vector.
    const int lastAxis = outAxes.empty() ? -1 : outAxes.back();
    const bool rowVecPath = anyUnaligned && lastAxis >= 0 && kVec > 1;
    enum class OpCls { Aligned, RowVec, Bcast, Other };
    auto classify = [&](const ir::Operand& op, bool aligned) {
      if (aligned) return OpCls::Aligned;
      int at = -1, uses = 0;
      for (size_t i = 0; i < op.axes.size(); ++i)
        if (op.axes[i] == lastAxis) {
          at = static_cast<int>(i);
          ++uses;
        }
      if (uses == 0) return OpCls::Bcast;
      if (uses > 1) return OpCls::Other;
      for (size_t i = static_cast<size_t>(at) + 1; i < op.axes.size(); ++i)
        if (g_.dims[op.axes[i]].extent != 1) return OpCls::Other;
      // One load of at most 16 bytes (the tensor alignment the launcher checks).
      if (kVec * ir::ElemBytes(g_.tensors[op.tensor].elem) > 16) return OpCls::Other;
      return OpCls::RowVec;
    };
    auto emitComputeLoop = [&](const std::string& ind, bool rowvec) {
      o << "#pragma unroll\n" << ind << "for (uint32_t u = 0; u < " << kUnroll << "u; ++u) {\n";
      std::ostringstream pre;
      std::function<std::string(bool, int, const std::function<std::string(int)>&)> opVal;
      if (rowvec) {
        const std::string in2 = ind + "  ";
        pre << in2 << "const uint64_t v = base + u * " << kVec * kBlock << "u;\n";
        coordDecl(pre, in2, "v");
        auto coordV = [&](int a) -> std::string {
          if (g_.dims[a].extent == 1) return "0u";
          return "c" + std::to_string(a) + "_v";
        };
        auto preload = [&](bool piped, size_t k, const ir::Operand& op, OpCls cls) {
          const std::string T = CType(g_.tensors[op.tensor].elem);
          const std::string nm = std::string(piped ? "rp" : "ra") + std::to_string(k);
          if (cls == OpCls::RowVec)
            pre << in2 << "const auto " << nm << " = tca::hip::load_vec<" << T << ", " << kVec << ">(t" << op.tensor
                << " + " << Offset(op.tensor, op.axes, coordV) << ");\n";
          else if (cls == OpCls::Bcast)
            pre << in2 << "const " << T << " " << nm << " = t" << op.tensor << "[" << Offset(op.tensor, op.axes, coordV)
                << "];\n";
        };
        for (size_t k = 0; k < c.root.ops.size(); ++k) preload(false, k, c.root.ops[k], classify(c.root.ops[k], rootAligned[k]));
        for (size_t k = 0; k < pipedAligned.size(); ++k)
          preload(true, k, c.piped.ops[k], classify(c.piped.ops[k], pipedAligned[k]));
        opVal = [&](bool piped, int k, const std::function<std::string(int)>& coordQ) -> std::string {
          const auto& op = piped ? c.piped.ops[k] : c.root.ops[k];
          const OpCls cls = classify(op, piped ? pipedAligned[k] : rootAligned[k]);
          const std::string nm = std::string(piped ? "rp" : "ra") + std::to_string(k);
          switch (cls) {
            case OpCls::Aligned: return std::string(piped ? "p" : "a") + std::to_string(k) + "[u][q]";
            case OpCls::RowVec: return nm + "[q]";
            case OpCls::Bcast: return nm;
            case OpCls::Other: break;
          }
          return "t" + std::to_string(op.tensor) + "[" + Offset(op.tensor, op.axes, coordQ) + "]";
        };
      }
      o << pre.str();
      o << ind << "  tca::hip::vec<" << CType(st.elem) << ", " << kVec << "> out{};\n";
      o << "#pragma unroll\n" << ind << "  for (uint32_t q = 0; q < " << kVec << "u; ++q) {\n";
      std::ostringstream bodyS;
      std::string val;
      if (rowvec) {
        auto coordQ = [&](int a) -> std::string {
          if (g_.dims[a].extent == 1) return "0u";
          if (a == lastAxis) return "(c" + std::to_string(a) + "_v + q)";
          return "c" + std::to_string(a) + "_v";
        };
        val = bodyWith(bodyS, ind + "    ", [&](bool piped, int k) { return opVal(piped, k, coordQ); });
      } else {
        o << ind << "    const uint64_t e = base + u * " << kVec * kBlock << "u + q;\n";
        val = body(bodyS, ind + "    ", "e", [&](bool piped, int k) {
          return std::string(piped ? "p" : "a") + std::to_string(k) + "[u][q]";
        });
      }
      o << bodyS.str();
      o << ind << "    out.set(q, " << val << ");\n";
      o << ind << "  }\n";
      o << ind << "  tca::hip::store_vec_nt<" << CType(st.elem) << ", " << kVec << ">(t" << c.store_tensor
        << " + base + u * " << kVec * kBlock << "u, out);\n";
      o << ind << "}\n";
    };
    if (rowVecPath) {
      o << "    if (" << ExtentExpr(g_, lastAxis) << " % " << kVec << "u == 0u) {\n";
      emitComputeLoop("      ", true);
      o << "    } else {\n";
      emitComputeLoop("      ", false);
      o << "    }\n";
    } else {
      emitComputeLoop("    ", false);
    }
    o << "  } else {\n";
    o << "    for (uint32_t u = 0; u < " << kUnroll << "u; ++u) {\n";
    o << "      for (uint32_t q = 0; q < " << kVec << "u; ++q) {\n";
    o << "        const uint64_t e = base + u * " << kVec * kBlock << "u + q;\n";
    o << "        if (e >= n) continue;\n";
    {
      std::ostringstream bodyS;
      std::string val = body(bodyS, Indent(4), "e", [&](bool piped, int k) {
        const auto& op = piped ? c.piped.ops[k] : c.root.ops[k];
        return "t" + std::to_string(op.tensor) + "[e]";
      });
      o << bodyS.str();
      o << "        t" << c.store_tensor << "[e] = " << val << ";\n";
    }
    o << "      }\n    }\n  }\n}\n\n";
    AddKernel(pk, Family::Elementwise, n.chains,
              "vec=" + std::to_string(kVec) + " unroll=" + std::to_string(kUnroll) + " block=256");
    return true;
  }

  std::string ProductExpr(const std::vector<int>& axes) {
    if (axes.empty()) return "1u";
    std::string s;
    for (size_t i = 0; i < axes.size(); ++i) s += (i ? " * " : "") + ExtentExpr(g_, axes[i]);
    return s;
  }

  // X: one thread per output element; reductions fold sequentially in
  // ascending index order from init — the reference's SeqReducer order
  // (runtime/tca/reducer.h:36-57), hence bit-identical to the CPU oracle
  // for every combiner.
  bool EmitGeneric(int ni, std::string* err) {
    (void)err;
    const Nest& n = an_.nests[ni];
    for (size_t k = 0; k < n.chains.size(); ++k) {
      Nest single;
      single.chains = {n.chains[k]};
      single.family = Family::Generic;
      const ir::Chain& c = g_.chains[n.chains[k]];
      PlanKernel pk;
      pk.symbol = Sym(g_, prefix_, ni) + (n.chains.size() > 1 ? "_" + std::to_string(k) : "");
      pk.block = 256;
      pk.grid.push_back(DimProduct(c.store_axes) + "/256");
      const std::string sig = Signature(single, &pk);
      std::ostringstream& o = src_;
      o << "// statement #" << n.chains[k] << ": generic family, one thread per output element\n";
      o << "extern \"C\" __global__ void __launch_bounds__(256) " << pk.symbol << "(\n    " << sig << ") {\n";
      o << "  const uint32_t total = " << ProductExpr(c.store_axes) << ";\n";
      o << "  const uint32_t o = blockIdx.x * 256u + threadIdx.x;\n";
      o << "  if (o >= total) return;\n";
      o << "  uint32_t rem = o;\n";
      for (int k2 = static_cast<int>(c.store_axes.size()) - 1; k2 >= 0; --k2) {
        int a = c.store_axes[k2];
        o << "  const uint32_t c" << a << " = rem % " << ExtentExpr(g_, a) << "; rem /= " << ExtentExpr(g_, a)
          << ";\n";
      }
      auto coord = [&](int a) { return "c" + std::to_string(a); };
      const int R = static_cast<int>(c.reduces.size());
      const std::string T = CType(g_.exprs[c.root.fn.body].type);
      std::string val;
      if (R == 0) {
        ExprGen eg(g_, o, "  ", &counter_);
        for (size_t q = 0; q < c.root.ops.size(); ++q) {
          const auto& op = c.root.ops[q];
          eg.Bind(c.root.fn.params[q], "t" + std::to_string(op.tensor) + "[" + Offset(op.tensor, op.axes, coord) + "]");
        }
        val = eg.Gen(c.root.fn.body);
      } else {
        // acc_r for reduce r; loops from the outermost reduce (R-1) inwards.
        std::string ind = "  ";
        {
          ExprGen ig(g_, o, ind, &counter_);
          const std::string iv = ig.Gen(c.reduces[R - 1].init);
          o << ind << T << " acc" << R - 1 << " = " << iv << ";\n";
        }
        for (int r = R - 1; r >= 0; --r) {
          const int a = c.reduces[r].axis;
          o << ind << "for (uint32_t c" << a << " = 0; c" << a << " < " << ExtentExpr(g_, a) << "; ++c" << a
            << ") {\n";
          ind += "  ";
          if (r > 0) {
            ExprGen ig(g_, o, ind, &counter_);
            const std::string iv = ig.Gen(c.reduces[r - 1].init);
            o << ind << T << " acc" << r - 1 << " = " << iv << ";\n";
          }
        }
        {
          ExprGen eg(g_, o, ind, &counter_);
          for (size_t q = 0; q < c.root.ops.size(); ++q) {
            const auto& op = c.root.ops[q];
            eg.Bind(c.root.fn.params[q],
                    "t" + std::to_string(op.tensor) + "[" + Offset(op.tensor, op.axes, coord) + "]");
          }
          std::string v = eg.Gen(c.root.fn.body);
          ExprGen rg(g_, o, ind, &counter_);
          rg.Bind(c.reduces[0].fn.params[0], "acc0");
          rg.Bind(c.reduces[0].fn.params[1], v);
          const std::string nv = rg.Gen(c.reduces[0].fn.body);
          o << ind << "acc0 = " << nv << ";\n";
        }
        for (int r = 0; r < R; ++r) {
          ind.resize(ind.size() - 2);
          o << ind << "}\n";
          if (r + 1 < R) {
            ExprGen rg(g_, o, ind, &counter_);
            rg.Bind(c.reduces[r + 1].fn.params[0], "acc" + std::to_string(r + 1));
            rg.Bind(c.reduces[r + 1].fn.params[1], "acc" + std::to_string(r));
            const std::string nv = rg.Gen(c.reduces[r + 1].fn.body);
            o << ind << "acc" << r + 1 << " = " << nv << ";\n";
          }
        }
        val = "acc" + std::to_string(R - 1);
      }
      if (c.has_piped) {
        ExprGen pg(g_, o, "  ", &counter_);
        pg.Bind(c.piped.fn.params[0], val);
        for (size_t q = 0; q < c.piped.ops.size(); ++q) {
          const auto& op = c.piped.ops[q];
          pg.Bind(c.piped.fn.params[q + 1],
                  "t" + std::to_string(op.tensor) + "[" + Offset(op.tensor, op.axes, coord) + "]");
        }
        val = pg.Gen(c.piped.fn.body);
      }
      o << "  t" << c.store_tensor << "[o] = " << val << ";\n}\n\n";
      AddKernel(pk, Family::Generic, {n.chains[k]}, "block=256 thread-per-output");
    }
    return true;
  }

  // R/F: one fused kernel per nest; each row is held in registers, every
  // reduction folds per thread then meets across lanes once.
  bool EmitRow(int ni, std::string* err) {
    const Nest& n = an_.nests[ni];
    RowGeom geo = RowCheck(g_, n.chains, RowNV());
    if (!geo.ok) {
      *err = "emit: row family rejected a nest it classified: " + geo.why;
      return false;
    }
    PlanKernel pk;
    pk.symbol = Sym(g_, prefix_, ni);
    pk.block = geo.block;
    pk.grid.push_back(DimProduct(geo.outer) + "/" + std::to_string(geo.rpb));
    const std::string sig = Signature(n, &pk);
    std::ostringstream& o = src_;
    const uint32_t seg = std::min<uint32_t>(geo.tpr, 64);
    const uint32_t wpb = geo.block / 64;
    o << "// statements";
    for (int ci : n.chains) o << " #" << ci;
    o << ": fused row family; row @" << g_.dims[geo.col].name << " = " << geo.C << " held in registers\n";
    o << "// lanes/row " << geo.tpr << ", vectors/lane " << geo.nv << " x " << geo.V << ", rows/block " << geo.rpb
      << "\n";
    o << "extern \"C\" __global__ void __launch_bounds__(" << geo.block << ") " << pk.symbol << "(\n    " << sig
      << ") {\n";
    o << "  constexpr uint32_t TPR = " << geo.tpr << "u, NV = " << geo.nv << "u, V = " << geo.V
      << "u, C = " << geo.C << "u, VECS = " << geo.vecs << "u, RPB = " << geo.rpb << "u;\n";
    o << "  const uint32_t nrows = " << ProductExpr(geo.outer) << ";\n";
    o << "  const uint32_t row = blockIdx.x * RPB + threadIdx.x / TPR;\n";
    o << "  const uint32_t lane = threadIdx.x % TPR;\n";
    o << "  const bool active = row < nrows;\n";
    if (geo.tail) o << "  const bool tail_ok = (NV - 1u) * TPR + lane < VECS;\n";
    else o << "  constexpr bool tail_ok = true;\n";
    o << "  const uint64_t row_base = static_cast<uint64_t>(active ? row : 0u) * C;\n";
    // Row coordinates.
    o << "  uint32_t rrem = active ? row : 0u;\n";
    for (int k = static_cast<int>(geo.outer.size()) - 1; k >= 0; --k) {
      int a = geo.outer[k];
      if (k == 0)  // the outermost coordinate is what remains (row < nrows)
        o << "  const uint32_t c" << a << " = rrem;\n";
      else
        o << "  const uint32_t c" << a << " = rrem % " << ExtentExpr(g_, a) << "; rrem /= " << ExtentExpr(g_, a)
          << ";\n";
    }
    auto coord = [&](int a) { return "c" + std::to_string(a); };
    // Which tensors are register locals of this nest. Anything a chain of the
    // nest stores is consumed by later chains of the nest from registers,
    // never re-read from memory inside the same kernel (a store by one lane
    // is not visible to the others without a barrier).
    auto isReg = [&](int t) { return g_.tensors[t].local && an_.reg_nest[t] == ni; };
    std::set<int> produced;
    for (int ci : n.chains) produced.insert(g_.chains[ci].store_tensor);
    // Preload row tiles and column vectors read from memory.
    std::set<int> tiles, cols, rscal;
    for (int ci : n.chains) {
      const ir::Chain& c = g_.chains[ci];
      for (const auto& op : c.root.ops) {
        OpKind k = Classify(op, geo);
        if (isReg(op.tensor) || produced.count(op.tensor)) continue;
        if (k == OpKind::RowTile) tiles.insert(op.tensor);
        else if (k == OpKind::ColVec) cols.insert(op.tensor);
      }
    }
    for (int t : tiles) {
      const std::string T = CType(g_.tensors[t].elem);
      o << "  tca::hip::vec<" << T << ", V> x" << t << "[NV];\n";
      o << "#pragma unroll\n  for (uint32_t j = 0; j < NV; ++j) {\n";
      o << "    if (active && (j + 1u < NV || tail_ok)) x" << t << "[j] = tca::hip::load_vec_nt<" << T << ", V>(t" << t
        << " + row_base + (j * TPR + lane) * V);\n";
      o << "    else x" << t << "[j] = tca::hip::vec<" << T << ", V>{};\n  }\n";
    }
    for (int t : cols) {
      const std::string T = CType(g_.tensors[t].elem);
      o << "  tca::hip::vec<" << T << ", V> x" << t << "[NV];\n";
      o << "#pragma unroll\n  for (uint32_t j = 0; j < NV; ++j) {\n";
      o << "    if (j + 1u < NV || tail_ok) x" << t << "[j] = tca::hip::load_vec<" << T << ", V>(t" << t
        << " + (j * TPR + lane) * V);\n";
      o << "    else x" << t << "[j] = tca::hip::vec<" << T << ", V>{};\n  }\n";
    }
    // Row-scalar value of operand `op` (memory or register local).
    std::map<int, std::string> regScalar;  // tensor produced in this nest -> register variable
    auto rowScalar = [&](const ir::Operand& op) -> std::string {
      if (regScalar.count(op.tensor)) return regScalar[op.tensor];
      return "(active ? t" + std::to_string(op.tensor) + "[" + Offset(op.tensor, op.axes, coord) + "] : " +
             CType(g_.tensors[op.tensor].elem) + "(0))";
    };
    // Element value of the root map of chain c at (j, q).
    auto elemValue = [&](std::ostringstream& os, const std::string& ind, const ir::Chain& c) -> std::string {
      ExprGen eg(g_, os, ind, &counter_);
      for (size_t k = 0; k < c.root.ops.size(); ++k) {
        const auto& op = c.root.ops[k];
        OpKind kind = Classify(op, geo);
        std::string v;
        if (kind == OpKind::RowTile || kind == OpKind::ColVec) v = "x" + std::to_string(op.tensor) + "[j][q]";
        else v = rowScalar(op);
        eg.Bind(c.root.fn.params[k], v);
      }
      return eg.Gen(c.root.fn.body);
    };
    std::vector<int> group;  // reduce chains with partials, not yet finalized
    std::set<int> groupOut;
    int groupNo = 0;
    uint32_t lds = 0;
    auto finalize = [&]() {
      if (group.empty()) return;
      // Lane reduction inside each segment/wave.
      for (int ci : group) {
        const ir::Chain& c = g_.chains[ci];
        const std::string T = CType(g_.exprs[c.root.fn.body].type);
        o << "  const auto comb" << ci << " = [](" << T << " acc, " << T << " now) -> " << T << " {\n";
        ExprGen cg(g_, o, "    ", &counter_);
        cg.Bind(c.reduces[0].fn.params[0], "acc");
        cg.Bind(c.reduces[0].fn.params[1], "now");
        std::string r = cg.Gen(c.reduces[0].fn.body);
        o << "    return " << r << ";\n  };\n";
        o << "  part" << ci << " = tca::hip::seg_allreduce<" << seg << ">(part" << ci << ", comb" << ci << ");\n";
      }
      if (geo.tpr > 64) {
        const uint32_t wpr = geo.tpr / 64;
        for (int ci : group) {
          const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
          o << "  __shared__ " << T << " red" << ci << "[" << wpb << "];\n";
          o << "  if (tca::hip::lane_id() == 0u) red" << ci << "[tca::hip::wave_id()] = part" << ci << ";\n";
          lds += static_cast<uint32_t>(ir::ElemBytes(g_.exprs[g_.chains[ci].root.fn.body].type)) * wpb;
        }
        o << "  __syncthreads();\n";
        o << "  {\n    const uint32_t w0 = (threadIdx.x / TPR) * " << wpr << "u;\n";
        for (int ci : group) {
          o << "    part" << ci << " = red" << ci << "[w0];\n";
          o << "    for (uint32_t w = 1; w < " << wpr << "u; ++w) part" << ci << " = comb" << ci << "(part" << ci
            << ", red" << ci << "[w0 + w]);\n";
        }
        o << "  }\n";
      }
      // init applied once per output, then the piped map, then the store.
      for (int ci : group) {
        const ir::Chain& c = g_.chains[ci];
        const ir::ReduceStage& r = c.reduces[0];
        ExprGen fg(g_, o, "  ", &counter_);
        fg.Bind(r.fn.params[0], fg.Gen(r.init));
        fg.Bind(r.fn.params[1], "part" + std::to_string(ci));
        std::string val = fg.Gen(r.fn.body);
        if (c.has_piped) {
          ExprGen pg(g_, o, "  ", &counter_);
          pg.Bind(c.piped.fn.params[0], val);
          for (size_t k = 0; k < c.piped.ops.size(); ++k) pg.Bind(c.piped.fn.params[k + 1], rowScalar(c.piped.ops[k]));
          val = pg.Gen(c.piped.fn.body);
        }
        const int st = c.store_tensor;
        const std::string T = CType(g_.tensors[st].elem);
        const std::string var = "r" + std::to_string(ci);
        o << "  const " << T << " " << var << " = " << val << ";\n";
        regScalar[st] = var;
        if (!isReg(st) || an_.hbm_local[st]) {
          o << "  if (active && lane == 0u) t" << st << "[" << Offset(st, c.store_axes, coord) << "] = " << var
            << ";\n";
        }
      }
      group.clear();
      groupOut.clear();
      ++groupNo;
    };
    std::set<int> regTiles;  // register row-tile locals produced so far
    for (int ci : n.chains) {
      const ir::Chain& c = g_.chains[ci];
      const std::set<int> reads = ReadSet(c);
      bool dep = false;
      for (int t : reads) dep |= groupOut.count(t) > 0;
      if (c.reduces.empty() || dep) finalize();
      if (IsRowScalarChain(c, geo)) {
        // Per-row map: evaluated once per row (by every lane of it).
        const int st = c.store_tensor;
        const std::string T = CType(g_.tensors[st].elem);
        o << "  // statement #" << ci << ": per-row map into " << g_.tensors[st].name << "\n";
        ExprGen eg(g_, o, "  ", &counter_);
        for (size_t k = 0; k < c.root.ops.size(); ++k) eg.Bind(c.root.fn.params[k], rowScalar(c.root.ops[k]));
        const std::string val = eg.Gen(c.root.fn.body);
        const std::string var = "r" + std::to_string(ci);
        o << "  const " << T << " " << var << " = " << val << ";\n";
        regScalar[st] = var;
        if (!isReg(st) || an_.hbm_local[st])
          o << "  if (active && lane == 0u) t" << st << "[" << Offset(st, c.store_axes, coord) << "] = " << var << ";\n";
        continue;
      }
      if (!c.reduces.empty()) {
        const std::string T = CType(g_.exprs[c.root.fn.body].type);
        o << "  // statement #" << ci << ": reduce over @" << g_.dims[geo.col].name << " into "
          << g_.tensors[c.store_tensor].name << "\n";
        o << "  " << T << " part" << ci << " = " << T << "(0);\n";
        o << "#pragma unroll\n  for (uint32_t j = 0; j < NV; ++j) {\n";
        if (geo.tail) o << "    if (j + 1u == NV && !tail_ok) break;\n";
        o << "#pragma unroll\n    for (uint32_t q = 0; q < V; ++q) {\n";
        std::ostringstream bs;
        std::string v = elemValue(bs, "      ", c);
        o << bs.str();
        std::ostringstream cs;
        ExprGen rg2(g_, cs, "        ", &counter_);
        rg2.Bind(c.reduces[0].fn.params[0], "part" + std::to_string(ci));
        rg2.Bind(c.reduces[0].fn.params[1], v);
        std::string folded = rg2.Gen(c.reduces[0].fn.body);
        o << "      if (j == 0u && q == 0u) part" << ci << " = " << v << ";\n";
        o << "      else {\n" << cs.str() << "        part" << ci << " = " << folded << ";\n      }\n";
        o << "    }\n";
        if (FoldFenced(g_.exprs[c.root.fn.body].type)) o << "    tca::hip::fold_fence(part" << ci << ");\n";
        o << "  }\n";
        group.push_back(ci);
        groupOut.insert(c.store_tensor);
      } else {
        // Elementwise chain over the row: write a tile (memory or registers).
        const int st = c.store_tensor;
        const std::string T = CType(g_.tensors[st].elem);
        o << "  // statement #" << ci << ": elementwise over the row into " << g_.tensors[st].name << "\n";
        const bool reg = true;  // later chains of the nest read the register copy
        if (reg) o << "  tca::hip::vec<" << T << ", V> x" << st << "[NV];\n";
        o << "#pragma unroll\n  for (uint32_t j = 0; j < NV; ++j) {\n";
        o << "    tca::hip::vec<" << T << ", V> outv{};\n";
        o << "#pragma unroll\n    for (uint32_t q = 0; q < V; ++q) {\n";
        std::ostringstream bs;
        std::string v = elemValue(bs, "      ", c);
        o << bs.str();
        o << "      outv.set(q, " << v << ");\n    }\n";
        if (reg) o << "    x" << st << "[j] = outv;\n";
        if (!isReg(st) || an_.hbm_local[st]) {  // outputs and locals other nests read
          o << "    if (active && (j + 1u < NV || tail_ok)) tca::hip::store_vec_nt<" << T << ", V>(t" << st
            << " + row_base + (j * TPR + lane) * V, outv);\n";
        }
        o << "  }\n";
        if (reg) regTiles.insert(st);
      }
    }
    finalize();
    o << "}\n\n";
    pk.lds = 0;  // static LDS only; the code object records it
    (void)lds;
    std::ostringstream det;
    det << "row=" << geo.C << " lanes/row=" << geo.tpr << " vec/lane=" << geo.nv << "x" << geo.V
        << " rows/block=" << geo.rpb << " block=" << geo.block;
    AddKernel(pk, Family::Row, n.chains, det.str());
    return true;
  }

  // The argument names of Signature(n), in its order.
  std::string CallArgs(const Nest& n) {
    std::string s;
    auto add = [&](const std::string& a) { s += (s.empty() ? "" : ", ") + a; };
    for (int t : NestTensors(n)) add("t" + std::to_string(t));
    for (size_t d = 0; d < g_.dims.size(); ++d) add("d" + std::to_string(d));
    for (int sc : NestScalars(n)) add("s" + std::to_string(sc));
    return s;
  }

  // S: the row nests of family R with a row length known only at run time
  // (or too long for registers). The row is read in 16-byte vectors (of
  // its widest row-shaped tensor: 4 f32, 8 bf16, 16 u8 elements, when the
  // length allows it; halved down to 1 otherwise) by S lanes, S
  // chosen at run time as the smallest power of two <= the block that
  // leaves no lane more than 4 vectors, so short rows pack many rows per
  // block and long ones spread over up to sixteen waves. Rows of <= 1024 x 4
  // vectors are read from HBM once into a per-lane register cache of 4
  // vectors (every later pass over the row reads registers; the small cache
  // keeps occupancy at 8 waves per SIMD); longer rows are streamed, one pass
  // per group of statements, 4 vectors in flight per lane, re-reads through
  // the caches. The block is sized at launch (the plan's pack record):
  // max(256, S) lanes, so a row of many waves has a block of its own and a
  // cross-wave meeting stalls only that row's waves. Consecutive reductions that read none of each other's results
  // share a pass. Lane l of a row holds vectors l, l + S, ...: NFULL of them,
  // one more for l < REM. The loops run over the longest share (a count
  // uniform over the block) with the vector index clamped into the row, so
  // no load is under a lane mask; a lane folds or stores only its own
  // vectors. Every lane of a non-empty row holds >= 1 vector (S <= vectors),
  // so a lane's fold starts from its first element and the segment meets by
  // shuffles and, past 64 lanes, through LDS; an empty row yields init. Row
  // scalars produced in the nest stay in registers. Lanes past the last row
  // read row 0 (in bounds) and store nothing. One block per row group: the
  // pack record repeats the lane choice at launch (the loop over groups is
  // grid-stride, so any grid is correct). One kernel per (vector width,
  // cached | streamed), chosen at launch by guards on the row length.
  bool EmitStream(int ni, std::string* err) {
    constexpr uint32_t kBlock = 1024, kMinBlock = 256, kCache = 4, kUnroll = 4;
    const Nest& n = an_.nests[ni];
    RowGeom geo = StreamCheck(g_, n.chains);
    if (!geo.ok) {
      *err = "emit: stream family rejected a nest it classified: " + geo.why;
      return false;
    }
    PlanKernel pk;
    pk.symbol = Sym(g_, prefix_, ni);
    const std::string sig = Signature(n, &pk);
    std::ostringstream& o = src_;
    const std::string body_fn = pk.symbol + "_rows";
    auto coord = [&](int a) { return "c" + std::to_string(a); };
    auto isReg = [&](int t) { return g_.tensors[t].local && an_.reg_nest[t] == ni; };
    std::set<int> produced;
    for (int ci : n.chains) produced.insert(g_.chains[ci].store_tensor);
    // Passes over the row.
    std::vector<std::vector<int>> passes;
    {
      std::set<int> outs;
      for (int ci : n.chains) {
        const ir::Chain& c = g_.chains[ci];
        bool dep = false;
        for (int t : ReadSet(c)) dep |= outs.count(t) > 0;
        const bool red = !c.reduces.empty();
        if (passes.empty() || !red || dep || g_.chains[passes.back()[0]].reduces.empty()) {
          passes.push_back({ci});
          outs.clear();
        } else {
          passes.back().push_back(ci);
        }
        outs.insert(c.store_tensor);
      }
    }
    // Row tiles and column vectors per pass; the last pass reading each tile.
    std::vector<std::vector<int>> passTiles(passes.size()), passCols(passes.size());
    std::map<int, int> lastPass;
    std::set<int> tiles;
    for (size_t p = 0; p < passes.size(); ++p) {
      std::set<int> seenT, seenC;
      for (int ci : passes[p])
        for (const auto& op : g_.chains[ci].root.ops) {
          const OpKind k = Classify(op, geo);
          if (k == OpKind::RowTile && seenT.insert(op.tensor).second) {
            passTiles[p].push_back(op.tensor);
            lastPass[op.tensor] = static_cast<int>(p);
            tiles.insert(op.tensor);
          } else if (k == OpKind::ColVec && seenC.insert(op.tensor).second) {
            passCols[p].push_back(op.tensor);
          }
        }
    }

    o << "// statements";
    for (int ci : n.chains) o << " #" << ci;
    o << ": streaming row family; row @" << g_.dims[geo.col].name
      << " of run-time length, lanes/row chosen at run time; NV > 0: the row is cached in registers\n";
    // EX: every lane holds exactly NV vectors (the row is NV * S vectors):
    // no loop exit, ownership test or index clamp.
    o << "template <uint32_t V, uint32_t NV, bool EX>\n__device__ __forceinline__ void " << body_fn << "(\n    "
      << sig << ") {\n";
    // Block and lane counts are powers of two: shifts, not divisions.
    // The launch block is max(kMinBlock, S) (the plan's pack record): derived
    // here from the row length rather than read from the dispatch packet.
    const uint32_t lgBlock = 31 - __builtin_clz(kBlock), lgMin = 31 - __builtin_clz(kMinBlock);
    o << "  const uint32_t C = " << ExtentExpr(g_, geo.col) << ";\n";
    o << "  const uint32_t VECS = C / V;\n";
    o << "  const uint32_t LS = tca::hip::pack_lanes_log2(VECS, NV > 0u ? NV : " << kCache << "u, " << lgBlock
      << "u);  // S = 2^LS lanes per row\n";
    o << "  const uint32_t LB = LS > " << lgMin << "u ? LS : " << lgMin << "u;  // the block: 2^LB = max(" << kMinBlock
      << ", S) lanes\n";
    o << "  const uint32_t S = 1u << LS, LR = LB - LS;  // 2^LR rows per block\n";
    o << "  const uint32_t SEG = S < 64u ? S : 64u, WPR = S > 64u ? S >> 6 : 1u;\n";
    o << "  const uint32_t NFULL = VECS >> LS, REM = VECS & (S - 1u);  // lane < REM holds NFULL + 1 vectors\n";
    o << "  const uint32_t NLANE = NFULL + (REM > 0u ? 1u : 0u);\n";
    o << "  const uint32_t nrows = " << ProductExpr(geo.outer) << ";\n";
    o << "  const uint32_t ngroups = static_cast<uint32_t>((static_cast<uint64_t>(nrows) + (1u << LR) - 1u) >> LR);\n";
    for (int ci : n.chains) {
      const ir::Chain& c = g_.chains[ci];
      if (c.reduces.empty()) continue;
      const std::string T = CType(g_.exprs[c.root.fn.body].type);
      o << "  __shared__ " << T << " red" << ci << "[" << kBlock / 64 << "];\n";
      o << "  const auto comb" << ci << " = [](" << T << " acc, " << T << " now) -> " << T << " {\n";
      ExprGen cg(g_, o, "    ", &counter_);
      cg.Bind(c.reduces[0].fn.params[0], "acc");
      cg.Bind(c.reduces[0].fn.params[1], "now");
      const std::string r = cg.Gen(c.reduces[0].fn.body);
      o << "    return " << r << ";\n  };\n";
    }
    o << "  for (uint32_t grp = blockIdx.x; grp < ngroups; grp += gridDim.x) {\n";
    o << "    const uint32_t row = (grp << LR) + (threadIdx.x >> LS);\n";
    o << "    const uint32_t lane = threadIdx.x & (S - 1u);\n";
    o << "    const bool active = row < nrows;\n";
    o << "    const uint64_t row_base = static_cast<uint64_t>(active ? row : 0u) * C;\n";
    o << "    uint32_t rrem = active ? row : 0u;\n";
    for (int k = static_cast<int>(geo.outer.size()) - 1; k >= 0; --k) {
      const int a = geo.outer[k];
      if (k == 0)  // the outermost coordinate is what remains (row < nrows)
        o << "    const uint32_t c" << a << " = rrem;\n";
      else
        o << "    const uint32_t c" << a << " = rrem % " << ExtentExpr(g_, a) << "; rrem /= " << ExtentExpr(g_, a)
          << ";\n";
    }
    // Row scalars read from memory: once per row.
    std::map<int, std::string> regScalar;
    std::set<int> loadedScalar;
    for (int ci : n.chains) {
      const ir::Chain& c = g_.chains[ci];
      std::vector<const ir::Operand*> ops;
      for (const auto& op : c.root.ops) ops.push_back(&op);
      if (c.has_piped)
        for (const auto& op : c.piped.ops) ops.push_back(&op);
      for (const ir::Operand* op : ops) {
        if (Classify(*op, geo) != OpKind::RowScalar || produced.count(op->tensor) || isReg(op->tensor)) continue;
        if (!loadedScalar.insert(op->tensor).second) continue;
        const std::string T = CType(g_.tensors[op->tensor].elem);
        const std::string var = "rs" + std::to_string(op->tensor);
        o << "    const " << T << " " << var << " = t" << op->tensor << "[" << Offset(op->tensor, op->axes, coord)
          << "];\n";
        regScalar[op->tensor] = var;
      }
    }
    auto rowScalar = [&](const ir::Operand& op) -> std::string {
      auto it = regScalar.find(op.tensor);
      return it != regScalar.end() ? it->second : std::string("/*missing row scalar*/0");
    };
    // Register cache of the row tiles (NV > 0 only); tiles from memory are
    // loaded up front, tiles produced in the nest as they are produced.
    for (int t : tiles)
      o << "    tca::hip::vec<" << CType(g_.tensors[t].elem) << ", V> xc" << t << "[NV > 0u ? NV : 1u];\n";
    std::vector<int> fromMemory;
    for (int t : tiles)
      if (!produced.count(t)) fromMemory.push_back(t);
    if (!fromMemory.empty()) {
      o << "    if constexpr (NV > 0u) {\n#pragma unroll\n      for (uint32_t j = 0; j < NV; ++j) {\n";
      o << "        if (!EX && j >= NLANE) break;\n";
      o << "        const uint32_t v = EX ? lane + j * S : min(lane + j * S, VECS - 1u);\n";
      for (int t : fromMemory)
        o << "        xc" << t << "[j] = tca::hip::load_vec_nt<" << CType(g_.tensors[t].elem) << ", V>(t" << t
          << " + row_base + static_cast<uint64_t>(v) * V);\n";
      o << "      }\n    }\n";
    }
    // The exp-sum of a softmax pair (a max, then a sum of expf(E - max)) in
    // the general register-cached body: its terms take the hardware
    // exponential (tca::hip::exp_term, relative error <= 2.7e-6 for
    // arguments down to -44, as the split rows' online normaliser sums), not
    // ocml's expf. They only form the denominator; the row map's own expf is
    // kept. Rows of 12000-32000 floats held in registers were bound by the
    // two expf per element: 16384 x 32000 1012 -> 922 us, x 12000 324 -> 290
    // us. The exact-fit bodies (EX) and the streamed one (NV = 0) keep expf:
    // there the same change measured 1-7% slower. With pass fusion off every
    // expf stays ocml's.
    std::set<const ir::Chain*> expTermSum;
    if (opts_.allow_pass_fusion)
      for (size_t p = 0; p + 1 < passes.size(); ++p)
        if (passes[p].size() == 1 && passes[p + 1].size() == 1 &&
            OnlineMaxExpSum(g_, g_.chains[passes[p][0]], g_.chains[passes[p + 1][0]], geo))
          expTermSum.insert(&g_.chains[passes[p + 1][0]]);
    // Element value of chain c at element q of the vector whose operands are
    // bound to x<t> (tiles and column vectors) at suffix `sfx`.
    auto elemValue = [&](std::ostringstream& os, const std::string& ind, const ir::Chain& c,
                         const std::string& sfx) -> std::string {
      ExprGen eg(g_, os, ind, &counter_);
      for (size_t k = 0; k < c.root.ops.size(); ++k) {
        const auto& op = c.root.ops[k];
        const OpKind kind = Classify(op, geo);
        eg.Bind(c.root.fn.params[k], (kind == OpKind::RowTile || kind == OpKind::ColVec)
                                         ? "x" + std::to_string(op.tensor) + sfx + "[q]"
                                         : rowScalar(op));
      }
      if (expTermSum.count(&c)) {  // the body is expf(E - a) (OnlineMaxExpSum)
        const std::string arg = eg.Gen(g_.exprs[c.root.fn.body].args[0]);
        const std::string v = "v" + std::to_string(counter_++);
        os << ind << "const float " << v << " = (EX || NV == 0u) ? expf(" << arg << ") : tca::hip::exp_term(" << arg
           << ");\n";
        return v;
      }
      return eg.Gen(c.root.fn.body);
    };
    // Operand vectors of pass p at the (clamped) vector index variable `vc`,
    // named x<t><sfx>: cached tiles alias the cache, others are loaded.
    auto operands = [&](std::ostringstream& b, size_t p, const std::string& ind, bool cached, const std::string& vc,
                        const std::string& sfx) {
      for (int t : passTiles[p]) {
        const std::string T = CType(g_.tensors[t].elem);
        if (cached) {
          b << ind << "const auto& x" << t << sfx << " = xc" << t << "[j];\n";
        } else {
          // Re-read by a later pass: let the caches keep it.
          const bool again = lastPass[t] != static_cast<int>(p) || produced.count(t);
          b << ind << "const auto x" << t << sfx << " = tca::hip::" << (again ? "load_vec" : "load_vec_nt") << "<"
            << T << ", V>(t" << t << " + row_base + static_cast<uint64_t>(" << vc << ") * V);\n";
        }
      }
      for (int t : passCols[p])
        b << ind << "const auto x" << t << sfx << " = tca::hip::load_vec<" << CType(g_.tensors[t].elem) << ", V>(t"
          << t << " + static_cast<uint64_t>(" << vc << ") * V);\n";
    };
    // Work of pass p on one vector (operands x<t><sfx>, index `vc`). `ok`: the
    // vector is the lane's own (else the clamped index points elsewhere and
    // nothing is folded or stored); "true" when known. `first`: the lane's
    // first vector (the fold starts from its element 0).
    auto work = [&](std::ostringstream& b, size_t p, const std::string& ind, bool cached, const std::string& vc,
                    const std::string& ok, const std::string& sfx, bool first) {
      const ir::Chain& c0 = g_.chains[passes[p][0]];
      if (!c0.reduces.empty()) {
        b << "#pragma unroll\n" << ind << "for (uint32_t q = 0; q < V; ++q) {\n";
        for (int ci : passes[p]) {
          const ir::Chain& c = g_.chains[ci];
          const std::string P = "part" + std::to_string(ci);
          std::ostringstream es;
          const std::string ev = elemValue(es, ind + "  ", c, sfx);
          b << es.str();
          const std::string folded = "comb" + std::to_string(ci) + "(" + P + ", " + ev + ")";
          if (first)
            b << ind << "  " << P << " = q == 0u ? " << ev << " : " << folded << ";\n";
          else if (ok == "true")
            b << ind << "  " << P << " = " << folded << ";\n";
          else
            b << ind << "  " << P << " = " << ok << " ? " << folded << " : " << P << ";\n";
        }
        b << ind << "}\n";
        for (int ci : passes[p])
          if (FoldFenced(g_.exprs[g_.chains[ci].root.fn.body].type))
            b << ind << "tca::hip::fold_fence(part" << ci << ");\n";
        return;
      }
      const int st = c0.store_tensor;
      const std::string T = CType(g_.tensors[st].elem);
      b << ind << "tca::hip::vec<" << T << ", V> outv" << sfx << "{};\n";
      b << "#pragma unroll\n" << ind << "for (uint32_t q = 0; q < V; ++q) {\n";
      std::ostringstream es;
      const std::string ev = elemValue(es, ind + "  ", c0, sfx);
      b << es.str() << ind << "  outv" << sfx << ".set(q, " << ev << ");\n" << ind << "}\n";
      if (!isReg(st) || an_.hbm_local[st]) {
        const bool again = tiles.count(st) > 0 && !cached;
        b << ind << "if (active" << (ok == "true" ? std::string() : " && " + ok) << ") tca::hip::"
          << (again ? "store_vec" : "store_vec_nt") << "<" << T << ", V>(t" << st
          << " + row_base + static_cast<uint64_t>(" << vc << ") * V, outv" << sfx << ");\n";
      }
      if (cached && tiles.count(st)) b << ind << "xc" << st << "[j] = outv" << sfx << ";\n";
    };
    // Vector k of the lane: index, ownership, clamped index.
    auto index = [&](std::ostringstream& b, const std::string& ind, const std::string& k, const std::string& sfx) {
      b << ind << "const uint32_t v" << sfx << " = lane + (" << k << ") * S;\n";
      b << ind << "const bool ok" << sfx << " = EX || v" << sfx << " < VECS;\n";
      b << ind << "const uint32_t vc" << sfx << " = ok" << sfx << " ? v" << sfx << " : VECS - 1u;\n";
    };
    // One pass of the row body. assign: the pass's results (r<chain>) were
    // declared by the caller and are assigned here.
    auto emitPass = [&](size_t p, bool assign) {
      const ir::Chain& c0 = g_.chains[passes[p][0]];
      const bool red = !c0.reduces.empty();
      if (IsRowScalarChain(c0, geo)) {
        // Per-row map: evaluated once per row (by every lane of it).
        const int st = c0.store_tensor;
        const std::string T = CType(g_.tensors[st].elem);
        o << "    // statement #" << passes[p][0] << ": per-row map into " << g_.tensors[st].name << "\n";
        ExprGen eg(g_, o, "    ", &counter_);
        for (size_t k = 0; k < c0.root.ops.size(); ++k) eg.Bind(c0.root.fn.params[k], rowScalar(c0.root.ops[k]));
        const std::string val = eg.Gen(c0.root.fn.body);
        const std::string var = "r" + std::to_string(passes[p][0]);
        o << "    const " << T << " " << var << " = " << val << ";\n";
        regScalar[st] = var;
        if (!isReg(st) || an_.hbm_local[st])
          o << "    if (active && lane == 0u) t" << st << "[" << Offset(st, c0.store_axes, coord) << "] = " << var
            << ";\n";
        return;
      }
      o << "    // statement";
      for (int ci : passes[p]) o << " #" << ci;
      if (red) {
        o << ": reduce over @" << g_.dims[geo.col].name << " into";
        for (int ci : passes[p]) o << " " << g_.tensors[g_.chains[ci].store_tensor].name;
      } else {
        o << ": elementwise over the row into " << g_.tensors[c0.store_tensor].name;
      }
      o << "\n";
      if (red)
        for (int ci : passes[p]) {
          const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
          o << "    " << T << " part" << ci << " = " << T << "(0);\n";
        }
      std::ostringstream b;
      // Cached: vector j of the cache; j == 0 is always the lane's own.
      b << "    if constexpr (NV > 0u) {\n#pragma unroll\n      for (uint32_t j = 0; j < NV; ++j) {\n";
      b << "        if (!EX && j >= NLANE) break;\n";
      index(b, "        ", "j", "");
      operands(b, p, "        ", true, "vc", "");
      b << "        if (j == 0u) {\n";
      work(b, p, "          ", true, "vc", "true", "", red);
      b << "        } else {\n";
      work(b, p, "          ", true, "vc", "ok", "", false);
      b << "        }\n      }\n";
      // Streamed: the lane's first vector, then kUnroll in flight, then the rest.
      b << "    } else if (NLANE > 0u) {\n      {\n";
      b << "        const uint32_t vc = lane;\n";
      operands(b, p, "        ", false, "vc", "");
      work(b, p, "        ", false, "vc", "true", "", red);
      b << "      }\n      uint32_t k = 1u;\n";
      b << "      for (; k + " << kUnroll - 1 << "u < NLANE; k += " << kUnroll << "u) {\n";
      for (uint32_t u = 0; u < kUnroll; ++u)
        index(b, "        ", "k + " + std::to_string(u) + "u", "_" + std::to_string(u));
      for (uint32_t u = 0; u < kUnroll; ++u)
        operands(b, p, "        ", false, "vc_" + std::to_string(u), "_" + std::to_string(u));
      for (uint32_t u = 0; u < kUnroll; ++u)
        work(b, p, "        ", false, "vc_" + std::to_string(u), "ok_" + std::to_string(u), "_" + std::to_string(u),
             false);
      b << "      }\n      for (; k < NLANE; ++k) {\n";
      index(b, "        ", "k", "");
      operands(b, p, "        ", false, "vc", "");
      work(b, p, "        ", false, "vc", "ok", "", false);
      b << "      }\n    }\n";
      o << b.str();
      if (!red) return;
      for (int ci : passes[p])
        o << "    part" << ci << " = tca::hip::seg_allreduce_rt(part" << ci << ", SEG, comb" << ci << ");\n";
      o << "    if (WPR > 1u) {\n      if ((threadIdx.x & 63u) == 0u) {\n";
      for (int ci : passes[p]) o << "        red" << ci << "[threadIdx.x >> 6] = part" << ci << ";\n";
      o << "      }\n      __syncthreads();\n      const uint32_t w0 = (threadIdx.x >> 6) & ~(WPR - 1u);  // the row's first wave\n";
      for (int ci : passes[p]) {
        o << "      part" << ci << " = red" << ci << "[w0];\n";
        o << "      for (uint32_t w = 1; w < WPR; ++w) part" << ci << " = comb" << ci << "(part" << ci << ", red" << ci
          << "[w0 + w]);\n";
      }
      o << "    }\n";
      // init once per output (an empty row yields init), then the piped map.
      for (int ci : passes[p]) {
        const ir::Chain& c = g_.chains[ci];
        const int st = c.store_tensor;
        const std::string T = CType(g_.exprs[c.root.fn.body].type);
        const ir::ReduceStage& r = c.reduces[0];
        std::string init;
        {
          ExprGen ig(g_, o, "    ", &counter_);
          init = ig.Gen(r.init);
        }
        std::string val;
        {
          std::ostringstream fs;
          ExprGen fg(g_, fs, "      ", &counter_);
          fg.Bind(r.fn.params[0], init);
          fg.Bind(r.fn.params[1], "part" + std::to_string(ci));
          val = fg.Gen(r.fn.body);
          o << "    " << T << " fin" << ci << " = " << init << ";\n";
          o << "    if (VECS > 0u) {\n" << fs.str() << "      fin" << ci << " = " << val << ";\n    }\n";
          val = "fin" + std::to_string(ci);
        }
        if (c.has_piped) {
          ExprGen pg(g_, o, "    ", &counter_);
          pg.Bind(c.piped.fn.params[0], val);
          for (size_t k = 0; k < c.piped.ops.size(); ++k) pg.Bind(c.piped.fn.params[k + 1], rowScalar(c.piped.ops[k]));
          val = pg.Gen(c.piped.fn.body);
        }
        const std::string ST = CType(g_.tensors[st].elem);
        const std::string var = "r" + std::to_string(ci);
        o << "    " << (assign ? std::string() : "const " + ST + " ") << var << " = " << val << ";\n";
        regScalar[st] = var;
        if (!isReg(st) || an_.hbm_local[st])
          o << "    if (active && lane == 0u) t" << st << "[" << Offset(st, c.store_axes, coord) << "] = " << var
            << ";\n";
      }
    };
    // A softmax pair (a max, then the sum of expf(E - max)) or a mean with its
    // centred sum of squares, in the streamed body (NV = 0): one read of the
    // row instead of two. Each lane folds its vectors into the online pair
    // (tca::hip::online_expsum_add) or the pairwise triple (sum, centred sum
    // of squares, count: tca::hip::chan_add); the row's lanes meet by
    // shuffles (both merges are symmetric, so every lane ends with the same
    // value) and its waves through LDS in wave order. The register-cached
    // bodies keep the two passes (the row is read from registers either way).
    std::vector<int> streamPair(passes.size(), 0);  // 1 softmax (online), 2 mean and centred squares
    if (opts_.allow_pass_fusion)
      for (size_t p = 0; p + 1 < passes.size(); ++p) {
        if (passes[p].size() != 1 || passes[p + 1].size() != 1 || (p > 0 && streamPair[p - 1])) continue;
        const ir::Chain& A = g_.chains[passes[p][0]];
        const ir::Chain& B = g_.chains[passes[p + 1][0]];
        if (IsRowScalarChain(A, geo) || IsRowScalarChain(B, geo)) continue;
        if (OnlineMaxExpSum(g_, A, B, geo))
          streamPair[p] = 1;
        else if (ChanRowMeanVar(g_, A, B, geo))
          streamPair[p] = 2;
      }
    auto emitStreamPair = [&](size_t p) {
      const bool online = streamPair[p] == 1;
      const int ca = passes[p][0], cb = passes[p + 1][0];
      const ir::Chain& A = g_.chains[ca];
      const ir::Chain& B = g_.chains[cb];
      const int ta = A.store_tensor, tb = B.store_tensor;
      const std::string sa = std::to_string(ca), sb = std::to_string(cb);
      const std::string ra = "r" + sa, rb = "r" + sb;
      const std::string STA = CType(g_.tensors[ta].elem), STB = CType(g_.tensors[tb].elem);
      o << "    // statements #" << ca << " #" << cb << ": "
        << (online ? "max and exp-sum" : "sum and centred sum of squares")
        << " in one read of a streamed row; the register-cached bodies run the two passes\n";
      o << "    " << STA << " " << ra << ";\n    " << STB << " " << rb << ";\n";
      o << "    if constexpr (NV > 0u) {\n";
      emitPass(p, true);
      emitPass(p + 1, true);
      o << "    } else {\n";
      const std::string I = "      ";
      if (online)
        o << I << "float om = -__builtin_inff(), os = 0.0f;\n";
      else
        o << I << "float cs = 0.0f, cm = 0.0f, cn = 0.0f;\n";
      // The values of A's element expression for vector `sfx` into
      // ev[at * V + q]; `ok`: the vector is the lane's (else -inf for the
      // online pair, whose max and sum it then leaves unchanged).
      auto values = [&](std::ostringstream& b, const std::string& ind, const std::string& sfx, uint32_t at,
                        const std::string& ok) {
        b << "#pragma unroll\n" << ind << "for (uint32_t q = 0; q < V; ++q) {\n";
        std::ostringstream es;
        const std::string ev = elemValue(es, ind + "  ", A, sfx);
        b << es.str() << ind << "  ev[" << at << "u * V + q] = "
          << (online && !ok.empty() ? ok + " ? " + ev + " : -__builtin_inff()" : ev) << ";\n" << ind << "}\n";
      };
      const std::string upd = online ? "tca::hip::online_expsum_add(om, os, ev);\n" : "tca::hip::chan_add(cs, cm, cn, ev);\n";
      std::ostringstream b;
      const std::string J = I + "  ", K = J + "  ";
      b << I << "if (NLANE > 0u) {  // every lane of a streamed row holds >= 1 vector\n" << J << "{\n";
      b << K << "const uint32_t vc = lane;\n";
      operands(b, p, K, false, "vc", "");
      b << K << "float ev[V];\n";
      values(b, K, "", 0, "");
      b << K << upd << J << "}\n" << J << "uint32_t k = 1u;\n";
      b << J << "for (; k + " << kUnroll - 1 << "u < NLANE; k += " << kUnroll << "u) {\n";
      for (uint32_t u = 0; u < kUnroll; ++u) index(b, K, "k + " + std::to_string(u) + "u", "_" + std::to_string(u));
      for (uint32_t u = 0; u < kUnroll; ++u) operands(b, p, K, false, "vc_" + std::to_string(u), "_" + std::to_string(u));
      b << K << "float ev[" << kUnroll << " * V];\n";
      for (uint32_t u = 0; u < kUnroll; ++u)
        values(b, K, "_" + std::to_string(u), u, "ok_" + std::to_string(u));
      if (online) {
        b << K << upd;
      } else {  // a lane's last vector may be past the row: fold vector by vector then
        b << K << "if (ok_" << kUnroll - 1 << ") {\n" << K << "  " << upd << K << "} else {\n";
        for (uint32_t u = 0; u < kUnroll; ++u)
          b << K << "  if (ok_" << u << ") tca::hip::chan_add_n<V>(cs, cm, cn, ev + " << u << "u * V);\n";
        b << K << "}\n";
      }
      b << J << "}\n" << J << "for (; k < NLANE; ++k) {\n";
      index(b, K, "k", "");
      operands(b, p, K, false, "vc", "");
      b << K << "float ev[V];\n";
      values(b, K, "", 0, "ok");
      if (online)
        b << K << upd;
      else
        b << K << "if (ok) " << upd;
      b << J << "}\n" << I << "}\n";
      o << b.str();
      // The row's lanes (SEG per segment), then its waves in order.
      if (online) {
        o << I << "for (uint32_t off = SEG >> 1; off > 0u; off >>= 1)\n"
          << I << "  tca::hip::online_expsum_merge(om, os, __shfl_xor(om, off, 64), __shfl_xor(os, off, 64));\n";
        o << I << "if (WPR > 1u) {\n" << J << "if ((threadIdx.x & 63u) == 0u) {\n" << K << "red" << sa
          << "[threadIdx.x >> 6] = om;\n" << K << "red" << sb << "[threadIdx.x >> 6] = os;\n" << J << "}\n";
        o << J << "__syncthreads();\n" << J << "const uint32_t w0 = (threadIdx.x >> 6) & ~(WPR - 1u);\n";
        o << J << "om = red" << sa << "[w0];\n" << J << "os = red" << sb << "[w0];\n";
        o << J << "for (uint32_t w = 1; w < WPR; ++w) tca::hip::online_expsum_merge(om, os, red" << sa << "[w0 + w], red"
          << sb << "[w0 + w]);\n" << I << "}\n";
      } else {
        o << I << "__shared__ float rn" << sa << "[" << kBlock / 64 << "];\n";
        o << I << "for (uint32_t off = SEG >> 1; off > 0u; off >>= 1)\n"
          << I << "  tca::hip::chan_merge_present(cs, cm, cn, __shfl_xor(cs, off, 64), __shfl_xor(cm, off, 64), "
             "__shfl_xor(cn, off, 64));\n";
        o << I << "if (WPR > 1u) {\n" << J << "if ((threadIdx.x & 63u) == 0u) {\n" << K << "red" << sa
          << "[threadIdx.x >> 6] = cs;\n" << K << "red" << sb << "[threadIdx.x >> 6] = cm;\n" << K << "rn" << sa
          << "[threadIdx.x >> 6] = cn;\n" << J << "}\n";
        o << J << "__syncthreads();\n" << J << "const uint32_t w0 = (threadIdx.x >> 6) & ~(WPR - 1u);\n";
        o << J << "cs = red" << sa << "[w0];\n" << J << "cm = red" << sb << "[w0];\n" << J << "cn = rn" << sa << "[w0];\n";
        o << J << "for (uint32_t w = 1; w < WPR; ++w)\n" << J << "  tca::hip::chan_merge_present(cs, cm, cn, red" << sa
          << "[w0 + w], red" << sb << "[w0 + w], rn" << sa << "[w0 + w]);\n" << I << "}\n";
      }
      // A's result: init once (an empty row yields init), the fold, then
      // its piped map.
      {
        const ir::ReduceStage& r = A.reduces[0];
        ExprGen ig(g_, o, I, &counter_);
        const std::string init = ig.Gen(r.init);
        std::ostringstream fs;
        ExprGen fg(g_, fs, J, &counter_);
        fg.Bind(r.fn.params[0], init);
        fg.Bind(r.fn.params[1], online ? "om" : "cs");
        const std::string v = fg.Gen(r.fn.body);
        const std::string T = CType(g_.exprs[A.root.fn.body].type);
        o << I << T << " fin" << sa << " = " << init << ";\n";
        o << I << "if (VECS > 0u) {\n" << fs.str() << J << "fin" << sa << " = " << v << ";\n" << I << "}\n";
        std::string val = "fin" + sa;
        if (A.has_piped) {
          ExprGen pg(g_, o, I, &counter_);
          pg.Bind(A.piped.fn.params[0], val);
          for (size_t k = 0; k < A.piped.ops.size(); ++k) pg.Bind(A.piped.fn.params[k + 1], rowScalar(A.piped.ops[k]));
          val = pg.Gen(A.piped.fn.body);
        }
        o << I << ra << " = " << val << ";\n";
      }
      regScalar[ta] = ra;
      // B's reduced total against A's result: the sum of expf(t - a) as
      // s * expf(m - a) (NaN when a is -inf: every term expf(-inf - -inf)),
      // or the sum of squares about a as M2 + n (S / n - a)^2.
      {
        const ir::ReduceStage& r = B.reduces[0];
        ExprGen ig(g_, o, I, &counter_);
        const std::string init = ig.Gen(r.init);
        std::ostringstream fs;
        if (online)
          fs << J << "const float ptotal = " << ra << " == -__builtin_inff() ? __builtin_nanf(\"\") : os * expf(om - " << ra
             << ");\n";
        else
          fs << J << "const float pd = cs / cn - " << ra << ";\n" << J << "const float ptotal = cm + cn * pd * pd;\n";
        ExprGen fg(g_, fs, J, &counter_);
        fg.Bind(r.fn.params[0], init);
        fg.Bind(r.fn.params[1], "ptotal");
        const std::string v = fg.Gen(r.fn.body);
        const std::string T = CType(g_.exprs[B.root.fn.body].type);
        o << I << T << " fin" << sb << " = " << init << ";\n";
        o << I << "if (VECS > 0u) {\n" << fs.str() << J << "fin" << sb << " = " << v << ";\n" << I << "}\n";
        std::string val = "fin" + sb;
        if (B.has_piped) {
          ExprGen pg(g_, o, I, &counter_);
          pg.Bind(B.piped.fn.params[0], val);
          for (size_t k = 0; k < B.piped.ops.size(); ++k) pg.Bind(B.piped.fn.params[k + 1], rowScalar(B.piped.ops[k]));
          val = pg.Gen(B.piped.fn.body);
        }
        o << I << rb << " = " << val << ";\n";
      }
      for (const auto& [t, ch] : {std::pair<int, const ir::Chain*>{ta, &A}, std::pair<int, const ir::Chain*>{tb, &B}})
        if (!isReg(t) || an_.hbm_local[t])
          o << I << "if (active && lane == 0u) t" << t << "[" << Offset(t, ch->store_axes, coord) << "] = r"
            << (t == ta ? sa : sb) << ";\n";
      o << "    }\n";
      regScalar[ta] = ra;
      regScalar[tb] = rb;
    };
    for (size_t p = 0; p < passes.size(); ++p) {
      if (!streamPair[p]) {
        emitPass(p, false);
        continue;
      }
      emitStreamPair(p);
      ++p;  // pass p + 1 is part of the pair
    }
    // Each reduction has its own LDS slots, written once per group: only a
    // next group (a grid-stride step, block-uniform) must wait until every
    // wave has read them.
    o << "    if (grp + gridDim.x < ngroups) __syncthreads();\n";
    o << "  }\n}\n";
    // Few long rows: each row split over many blocks. Applies when the nest
    // is one pass of reductions (no row maps, no per-row chains) and the
    // rows are indexed by at most one axis. A partial kernel folds a chunk
    // of >= 2048 vectors per block (P chunks per row, P = min(512,
    // ceil(vectors / 4096)): 512 blocks of 1024 lanes are what the CUs hold
    // at once, 1024 chunks measured 10% slower on a full reduction; with
    // chunks of ceil(vectors / P) every chunk, the last included, holds >=
    // 2048 vectors for rows > 4096 vectors, so every thread holds >= 1) and
    // writes one partial per block and reduction into an HBM scratch
    // [rows][512]; a
    // merge kernel folds a row's P partials with one wave, applies init once
    // and the piped map, and stores. Guards: the streamed row lengths with
    // rows <= kSplitRows (one block per row would leave most CUs idle);
    // with no row axis (a full reduction) the split replaces the streamed
    // kernel outright.
    constexpr uint32_t kSplitRows = 255, kChunkVecs = 4096, kMaxParts = 512, kPartBlock = 1024;
    // Nests of several passes also split rows of >= kSplitLongVecs vectors
    // when there are up to kSplitRowsLong of them: the streamed kernel reads
    // such a row once per pass (softmax three times), the split passes twice
    // (the first two passes fused). Softmax [512, 131072]: 161.7 -> 125.2 us,
    // [1024, 65536]: 152.8 -> 125.0 us, [256, 1 Mi]: 718 -> 529-540 us;
    // layernorm [512, 131072] 154.8 -> 125.4 us. Shorter rows stay streamed
    // (layernorm [4096, 40000]: 316 us streamed, 398 split: many short map
    // chunks, each computing the pair's values), and so do more rows (the
    // partials are [rows][512]: 8 MiB each at 4095 rows).
    constexpr uint32_t kSplitRowsLong = 4095, kSplitLongVecs = 16384;
    const bool split = passes.size() == 1 && !g_.chains[passes[0][0]].reduces.empty() && geo.outer.size() <= 1;
    std::string part_fn, merge_fn;
    std::vector<std::string> part_names;
    if (split) {
      part_fn = pk.symbol + "_part";
      merge_fn = pk.symbol + "_merge";
      const std::string splitDim = "__split";
      // One plan dim serves every split kernel of the program (same extent).
      const std::string splitDecl = splitDim + " " + std::to_string(kMaxParts);
      if (std::find(extra_dims_.begin(), extra_dims_.end(), splitDecl) == extra_dims_.end())
        extra_dims_.push_back(splitDecl);
      std::string partSig;
      for (int ci : passes[0]) {
        const ir::Chain& c = g_.chains[ci];
        const ir::Elem pe = g_.exprs[c.root.fn.body].type;
        const std::string nm = "__part" + std::to_string(ci);
        part_names.push_back(nm);
        std::string t = nm + " " + ir::ElemName(pe) + " local " + std::to_string(geo.outer.size() + 1);
        for (int a : geo.outer) t += " " + g_.dims[a].name;
        extra_tensors_.push_back(t + " " + splitDim);
        partSig += ",\n    " + CType(pe) + "* __restrict__ p" + std::to_string(ci) + " /* " + nm + " */";
      }
      const std::string rowExpr = ProductExpr(geo.outer);
      auto combs = [&](const std::string& ind) {
        for (int ci : passes[0]) {
          const ir::Chain& c = g_.chains[ci];
          const std::string T = CType(g_.exprs[c.root.fn.body].type);
          o << ind << "const auto comb" << ci << " = [](" << T << " acc, " << T << " now) -> " << T << " {\n";
          ExprGen cg(g_, o, ind + "  ", &counter_);
          cg.Bind(c.reduces[0].fn.params[0], "acc");
          cg.Bind(c.reduces[0].fn.params[1], "now");
          const std::string r = cg.Gen(c.reduces[0].fn.body);
          o << ind << "  return " << r << ";\n" << ind << "};\n";
        }
      };
      auto rowCoords = [&](const std::string& ind) {
        for (int a : geo.outer) o << ind << "const uint32_t c" << a << " = r;\n";
      };
      // Row scalars the fold or the piped maps read from memory.
      auto rowScalars = [&](const std::string& ind) {
        std::set<int> done;
        for (int ci : passes[0]) {
          const ir::Chain& c = g_.chains[ci];
          std::vector<const ir::Operand*> ops;
          for (const auto& op : c.root.ops) ops.push_back(&op);
          if (c.has_piped)
            for (const auto& op : c.piped.ops) ops.push_back(&op);
          for (const ir::Operand* op : ops) {
            if (Classify(*op, geo) != OpKind::RowScalar || !done.insert(op->tensor).second) continue;
            const std::string T = CType(g_.tensors[op->tensor].elem);
            o << ind << "const " << T << " rs" << op->tensor << " = t" << op->tensor << "["
              << Offset(op->tensor, op->axes, coord) << "];\n";
          }
        }
      };
      o << "// statements";
      for (int ci : passes[0]) o << " #" << ci;
      o << ": split rows, partial folds (" << kPartBlock << " lanes per chunk of a row)\n";
      o << "template <uint32_t V>\n__device__ __forceinline__ void " << part_fn << "(\n    " << sig << partSig
        << ") {\n";
      o << "  constexpr uint32_t CV = " << kChunkVecs << "u, PMAX = " << kMaxParts << "u;\n";
      o << "  const uint32_t C = " << ExtentExpr(g_, geo.col) << ";\n";
      o << "  const uint32_t VECS = C / V;\n";
      o << "  const uint32_t P = min(PMAX, tca::hip::ceil_div(VECS, CV));  // VECS >= 1 (launch guard)\n";
      o << "  const uint32_t r = blockIdx.x / P, p = blockIdx.x - r * P;\n";
      o << "  if (r >= " << rowExpr << ") return;  // the grid is rows x P: never taken\n";
      o << "  const uint32_t L = tca::hip::ceil_div(VECS, P);\n";
      o << "  const uint32_t lo = p * L, hi = lo + min(L, VECS - lo);  // lo < VECS; hi - lo > " << kPartBlock << "\n";
      o << "  const uint64_t row_base = static_cast<uint64_t>(r) * C;\n";
      o << "  const bool active = true;\n";
      rowCoords("  ");
      rowScalars("  ");
      combs("  ");
      for (int ci : passes[0]) {
        const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
        o << "  " << T << " part" << ci << " = " << T << "(0);\n";
      }
      std::ostringstream b;
      b << "  {\n    const uint32_t vc = lo + threadIdx.x;\n";
      operands(b, 0, "    ", false, "vc", "");
      work(b, 0, "    ", false, "vc", "true", "", true);
      b << "  }\n  uint32_t v0 = lo + threadIdx.x + " << kPartBlock << "u;\n";
      b << "  for (; v0 + " << 3 * kPartBlock << "u < hi; v0 += " << 4 * kPartBlock << "u) {\n";
      for (uint32_t u = 0; u < 4; ++u)
        b << "    const uint32_t vc_" << u << " = v0 + " << u * kPartBlock << "u;\n";
      for (uint32_t u = 0; u < 4; ++u) operands(b, 0, "    ", false, "vc_" + std::to_string(u), "_" + std::to_string(u));
      for (uint32_t u = 0; u < 4; ++u)
        work(b, 0, "    ", false, "vc_" + std::to_string(u), "true", "_" + std::to_string(u), false);
      b << "  }\n  for (; v0 < hi; v0 += " << kPartBlock << "u) {\n    const uint32_t vc = v0;\n";
      operands(b, 0, "    ", false, "vc", "");
      work(b, 0, "    ", false, "vc", "true", "", false);
      b << "  }\n";
      o << b.str();
      for (int ci : passes[0]) {
        const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
        o << "  part" << ci << " = tca::hip::seg_allreduce<64>(part" << ci << ", comb" << ci << ");\n";
        o << "  __shared__ " << T << " red" << ci << "[" << kPartBlock / 64 << "];\n";
        o << "  if ((threadIdx.x & 63u) == 0u) red" << ci << "[threadIdx.x >> 6] = part" << ci << ";\n";
      }
      o << "  __syncthreads();\n  if (threadIdx.x == 0u) {\n";
      for (int ci : passes[0]) {
        const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
        o << "    " << T << " acc" << ci << " = red" << ci << "[0];\n";
        o << "    for (uint32_t w = 1; w < " << kPartBlock / 64 << "u; ++w) acc" << ci << " = comb" << ci << "(acc" << ci
          << ", red" << ci << "[w]);\n";
        o << "    p" << ci << "[static_cast<uint64_t>(r) * PMAX + p] = acc" << ci << ";\n";
      }
      o << "  }\n}\n";
      // Merge: one wave per row.
      o << "template <uint32_t V>\n__device__ __forceinline__ void " << merge_fn << "(\n    " << sig << partSig
        << ") {\n";
      o << "  constexpr uint32_t CV = " << kChunkVecs << "u, PMAX = " << kMaxParts << "u;\n";
      o << "  const uint32_t C = " << ExtentExpr(g_, geo.col) << ";\n";
      o << "  const uint32_t P = min(PMAX, tca::hip::ceil_div(C / V, CV));\n";
      o << "  const uint32_t r = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;\n";
      o << "  if (r >= " << rowExpr << ") return;  // whole waves\n";
      rowCoords("  ");
      rowScalars("  ");
      combs("  ");
      for (int ci : passes[0]) {
        const ir::Chain& c = g_.chains[ci];
        const int st = c.store_tensor;
        const std::string T = CType(g_.exprs[c.root.fn.body].type);
        const std::string A = "m" + std::to_string(ci), H = "h" + std::to_string(ci);
        // P <= PMAX = 8 x 64: each lane's (at most 8) partials are loaded at
        // once, indices clamped into the row's partials, then folded in order.
        o << "  " << T << " " << A << " = " << T << "(0);\n  bool " << H << " = false;\n";
        o << "  {\n    " << T << " pv[PMAX / 64u];\n";
        o << "#pragma unroll\n    for (uint32_t k = 0; k < PMAX / 64u; ++k)\n";
        o << "      pv[k] = p" << ci << "[static_cast<uint64_t>(r) * PMAX + min(lane + 64u * k, P - 1u)];\n";
        o << "#pragma unroll\n    for (uint32_t k = 0; k < PMAX / 64u; ++k) {\n";
        o << "      if (lane + 64u * k < P) {\n";
        o << "        " << A << " = " << H << " ? comb" << ci << "(" << A << ", pv[k]) : pv[k];\n        " << H
          << " = true;\n      }\n    }\n  }\n";
        o << "  " << A << " = tca::hip::wave_allreduce_present(" << A << ", " << H << ", comb" << ci << ");\n";
        o << "  if (lane == 0u) {\n";
        const ir::ReduceStage& rs = c.reduces[0];
        ExprGen fg(g_, o, "    ", &counter_);
        fg.Bind(rs.fn.params[0], fg.Gen(rs.init));
        fg.Bind(rs.fn.params[1], A);
        std::string val = fg.Gen(rs.fn.body);  // P >= 1: init applied once to the row's total
        if (c.has_piped) {
          ExprGen pg(g_, o, "    ", &counter_);
          pg.Bind(c.piped.fn.params[0], val);
          for (size_t k = 0; k < c.piped.ops.size(); ++k)
            pg.Bind(c.piped.fn.params[k + 1], "rs" + std::to_string(c.piped.ops[k].tensor));
          val = pg.Gen(c.piped.fn.body);
        }
        if (!isReg(st) || an_.hbm_local[st])
          o << "    t" << st << "[" << Offset(st, c.store_axes, coord) << "] = " << val << ";\n";
        o << "  }\n";
      }
      o << "}\n";
    }
    // Few long rows of a nest of several passes (softmax, layernorm): each
    // pass over its own grid of row chunks. A reduction pass is a partial
    // kernel (a chunk of >= 2048 vectors per 1024-lane block, one partial per
    // chunk into the [rows][512] scratch) and a merge (one wave per row: init,
    // piped map, store); a row-map pass is one kernel writing its chunk of the
    // row tile. Results a later pass reads come from memory: outputs where
    // they are, register locals in plan-only locals of their own shape.
    // Applies to nests of reduction and row-map passes only (no per-row
    // chains, no pass reading a tile the nest produces), rows indexed by at
    // most one axis, in the streamed range with rows <= kSplitRows.
    bool splitMulti = passes.size() > 1 && geo.outer.size() <= 1;
    for (const auto& ps : passes)
      if (IsRowScalarChain(g_.chains[ps[0]], geo)) splitMulti = false;
    for (int t : tiles)
      if (produced.count(t)) splitMulti = false;
    // Softmax's max and exp-sum passes, fused into one pass over the row's
    // chunks with the online normaliser, and a mean with its centred sum of
    // squares (layernorm's), fused with the pairwise update (chanPair):
    // onlinePair[p] for the first pass of such a pair (pass p + 1 then has
    // no kernels of its own); the chunk maxima the softmax sums were taken
    // against go to a partial of their own.
    std::vector<bool> onlinePair(passes.size(), false);
    std::vector<bool> chanPair(passes.size(), false);  // of those, a mean and its centred sum of squares
    std::set<int> onlineSum;  // chain B of each fused softmax pair
    if (splitMulti && opts_.allow_pass_fusion)
      for (size_t p = 0; p + 1 < passes.size(); ++p) {
        if (passes[p].size() != 1 || passes[p + 1].size() != 1 || (p > 0 && onlinePair[p - 1])) continue;
        const ir::Chain& A = g_.chains[passes[p][0]];
        const ir::Chain& B = g_.chains[passes[p + 1][0]];
        if (OnlineMaxExpSum(g_, A, B, geo)) {
          onlinePair[p] = true;
          onlineSum.insert(passes[p + 1][0]);
        } else if (ChanRowMeanVar(g_, A, B, geo)) {
          onlinePair[p] = chanPair[p] = true;
        }
      }
    // A fused pair followed by the nest's last pass, a row map (softmax's
    // normalisation): each row-map workgroup computes the pair's two values
    // for its row from the partials (at most 512 pairs, read from the L2)
    // instead of a merge kernel storing them first; one workgroup per row
    // still stores them. The merge launch and its dependency were 4.6 us of
    // the 131 us of softmax over [64, 1 Mi].
    std::set<size_t> foldedMerge;
    for (size_t p = 0; p + 3 == passes.size(); ++p)
      if (onlinePair[p] && g_.chains[passes[p + 2][0]].reduces.empty()) foldedMerge.insert(p);
    std::string smSig, smArgs;
    std::vector<std::string> smPlanArgs;
    std::vector<std::pair<std::string, size_t>> smFns;  // (device function, pass)
    // Vectors per chunk of a split kernel whose chunks are not kChunkVecs.
    std::map<std::string, uint32_t> smChunk;
    // Row maps with a mean/variance pair's merge folded in take their chunk
    // length as a template argument: kChunkVecs below kLongMapVecs vectors a
    // row, 4x from there (every wave computes the pair's values before it
    // streams, and longer chunks spread that over more vectors). Layernorm
    // over [8, 4 Mi]: 93 -> 79 us, [64, 1 Mi]: 137 -> 131 us; rows of 16 Ki
    // vectors keep 4 chunks (17 us, not 19, at 32 rows). Softmax's map
    // measured no better with longer chunks at [64, 1 Mi] and keeps
    // kChunkVecs.
    std::set<std::string> longMaps;
    constexpr uint32_t kLongMapVecs = 16 * kChunkVecs;
    // The fused softmax passes take chunks 4x as long (16 vectors per lane):
    // with 4 a lane, the many short workgroups spent a quarter of their time
    // in the block's tail (the pair merges, the partials' stores); 8x (32 a
    // lane, one round of workgroups at [64, 1 Mi]) measured 3% slower.
    constexpr uint32_t kOnlineChunkVecs = 4 * kChunkVecs;
    if (splitMulti) {
      const std::string splitDim = "__split";
      const std::string splitDecl = splitDim + " " + std::to_string(kMaxParts);
      if (std::find(extra_dims_.begin(), extra_dims_.end(), splitDecl) == extra_dims_.end())
        extra_dims_.push_back(splitDecl);
      for (const auto& ps : passes) {
        if (g_.chains[ps[0]].reduces.empty()) continue;
        for (int ci : ps) {
          const ir::Elem pe = g_.exprs[g_.chains[ci].root.fn.body].type;
          const std::string nm = "__part" + std::to_string(ci);
          std::string t = nm + " " + ir::ElemName(pe) + " local " + std::to_string(geo.outer.size() + 1);
          for (int a : geo.outer) t += " " + g_.dims[a].name;
          t += " " + splitDim;
          if (std::find(extra_tensors_.begin(), extra_tensors_.end(), t) == extra_tensors_.end())
            extra_tensors_.push_back(t);
          smSig += ",\n    " + CType(pe) + "* __restrict__ p" + std::to_string(ci) + " /* " + nm + " */";
          smArgs += ", p" + std::to_string(ci);
          smPlanArgs.push_back("ptr " + nm);
          if (onlineSum.count(ci)) {
            const std::string sn = "__shift" + std::to_string(ci);
            std::string st = sn + " f32 local " + std::to_string(geo.outer.size() + 1);
            for (int a : geo.outer) st += " " + g_.dims[a].name;
            st += " " + splitDim;
            if (std::find(extra_tensors_.begin(), extra_tensors_.end(), st) == extra_tensors_.end())
              extra_tensors_.push_back(st);
            smSig += ",\n    float* __restrict__ q" + std::to_string(ci) + " /* " + sn + " */";
            smArgs += ", q" + std::to_string(ci);
            smPlanArgs.push_back("ptr " + sn);
          }
          // A register local gets memory of its own shape for the later passes.
          const int st = g_.chains[ci].store_tensor;
          if (isReg(st) && !an_.hbm_local[st]) {
            const ir::Tensor& tt = g_.tensors[st];
            std::string lt = tt.name + " " + ir::ElemName(tt.elem) + " local " + std::to_string(tt.dims.size());
            for (int d : tt.dims) lt += " " + g_.dims[d].name;
            if (std::find(extra_tensors_.begin(), extra_tensors_.end(), lt) == extra_tensors_.end())
              extra_tensors_.push_back(lt);
            smSig += ",\n    " + CType(tt.elem) + "* __restrict__ t" + std::to_string(st) + " /* " + tt.name +
                     " (row results of the split passes) */";
            smArgs += ", t" + std::to_string(st);
            smPlanArgs.push_back("ptr " + tt.name);
          }
        }
      }
      const std::string rowExpr = ProductExpr(geo.outer);
      // Row scalars of pass p's chains, loaded from memory; bound for elemValue.
      // Those in `computed` are values the kernel computes itself (a folded
      // merge's aval and bval): bound, not loaded.
      std::map<int, std::string> computed;
      auto loadRowScalars = [&](size_t p, const std::string& ind) {
        std::set<int> done;
        for (const auto& kv : computed) {
          regScalar[kv.first] = kv.second;
          done.insert(kv.first);
        }
        for (int ci : passes[p]) {
          const ir::Chain& c = g_.chains[ci];
          std::vector<const ir::Operand*> ops;
          for (const auto& op : c.root.ops) ops.push_back(&op);
          if (c.has_piped)
            for (const auto& op : c.piped.ops) ops.push_back(&op);
          for (const ir::Operand* op : ops) {
            if (Classify(*op, geo) != OpKind::RowScalar || !done.insert(op->tensor).second) continue;
            const std::string T = CType(g_.tensors[op->tensor].elem);
            o << ind << "const " << T << " rs" << op->tensor << " = t" << op->tensor << "["
              << Offset(op->tensor, op->axes, coord) << "];\n";
            regScalar[op->tensor] = "rs" + std::to_string(op->tensor);
          }
        }
      };
      auto combsOf = [&](size_t p, const std::string& ind) {
        for (int ci : passes[p]) {
          const ir::Chain& c = g_.chains[ci];
          const std::string T = CType(g_.exprs[c.root.fn.body].type);
          o << ind << "const auto comb" << ci << " = [](" << T << " acc, " << T << " now) -> " << T << " {\n";
          ExprGen cg(g_, o, ind + "  ", &counter_);
          cg.Bind(c.reduces[0].fn.params[0], "acc");
          cg.Bind(c.reduces[0].fn.params[1], "now");
          const std::string r = cg.Gen(c.reduces[0].fn.body);
          o << ind << "  return " << r << ";\n" << ind << "};\n";
        }
      };
      auto chunkHead = [&](const std::string& cv) {
        o << "  constexpr uint32_t CV = " << cv << ", PMAX = " << kMaxParts << "u;\n";
        o << "  const uint32_t C = " << ExtentExpr(g_, geo.col) << ";\n";
        o << "  const uint32_t VECS = C / V;\n";
        o << "  const uint32_t P = min(PMAX, tca::hip::ceil_div(VECS, CV));  // VECS >= 1 (launch guard)\n";
        o << "  const uint32_t r = blockIdx.x / P, p = blockIdx.x - r * P;\n";
        o << "  if (r >= " << rowExpr << ") return;  // the grid is rows x P: never taken\n";
        o << "  const uint32_t L = tca::hip::ceil_div(VECS, P);\n";
        o << "  const uint32_t lo = p * L, hi = lo + min(L, VECS - lo);  // lo < VECS; hi - lo > " << kPartBlock << "\n";
        o << "  const uint64_t row_base = static_cast<uint64_t>(r) * C;\n";
        o << "  const bool active = true;\n";
        for (int a : geo.outer) o << "  const uint32_t c" << a << " = r;\n";
      };
      // B's result from its reduced total `total` (its init and piped map,
      // A's result bound to aval), declared as bval.
      auto pairFinishB = [&](size_t p, const std::string& ind, const std::string& total) {
        const ir::Chain& A = g_.chains[passes[p][0]];
        const ir::Chain& B = g_.chains[passes[p + 1][0]];
        const int ta = A.store_tensor;
        // Row scalars B's piped map reads besides A's result.
        std::map<int, std::string> piped;
        if (B.has_piped)
          for (const auto& op : B.piped.ops) {
            if (op.tensor == ta || piped.count(op.tensor)) continue;
            piped[op.tensor] = "prs" + std::to_string(op.tensor);
            o << ind << "const " << CType(g_.tensors[op.tensor].elem) << " prs" << op.tensor << " = t" << op.tensor
              << "[" << Offset(op.tensor, op.axes, coord) << "];\n";
          }
        const ir::ReduceStage& rs = B.reduces[0];
        ExprGen fg(g_, o, ind, &counter_);
        fg.Bind(rs.fn.params[0], fg.Gen(rs.init));
        fg.Bind(rs.fn.params[1], total);
        std::string val = fg.Gen(rs.fn.body);
        if (B.has_piped) {
          ExprGen pg(g_, o, ind, &counter_);
          pg.Bind(B.piped.fn.params[0], val);
          for (size_t k = 0; k < B.piped.ops.size(); ++k) {
            const int t = B.piped.ops[k].tensor;
            pg.Bind(B.piped.fn.params[k + 1], t == ta ? std::string("aval") : piped[t]);
          }
          val = pg.Gen(B.piped.fn.body);
        }
        o << ind << "const " << CType(g_.tensors[B.store_tensor].elem) << " bval = " << val << ";\n";
      };
      // pairValues for a mean and its centred sum of squares, from the chunks'
      // sums S_c and sums of squares about their own means M2_c (n_c values
      // each, from the chunk bounds): aval = A's init, sum of S_c and piped
      // map; B's total = sum over c of M2_c + n_c (S_c / n_c - aval)^2, the
      // sum of squares about aval (each chunk's, exactly, by the parallel
      // axis theorem). Two butterflies of plain sums: every lane holds the
      // same values.
      auto chanPairValues = [&](size_t p, const std::string& ind) {
        const int ca = passes[p][0], cb = passes[p + 1][0];
        const ir::Chain& A = g_.chains[ca];
        const std::string sa = std::to_string(ca), sb = std::to_string(cb);
        const uint32_t K = kMaxParts / 64;
        o << ind << "const uint32_t PF = min(" << kMaxParts << "u, tca::hip::ceil_div(C / V, " << kOnlineChunkVecs
          << "u));  // the fused partial's chunks\n";
        o << ind << "const uint32_t PVECS = C / V, PL = tca::hip::ceil_div(PVECS, PF);\n";
        o << ind << "float sv[" << K << "], mv[" << K << "];\n#pragma unroll\n" << ind << "for (uint32_t k = 0; k < " << K
          << "u; ++k) {\n" << ind << "  const uint64_t at = static_cast<uint64_t>(r) * " << kMaxParts
          << "u + min((threadIdx.x & 63u) + 64u * k, PF - 1u);\n" << ind << "  sv[k] = p" << sa << "[at];\n" << ind
          << "  mv[k] = p" << sb << "[at];\n" << ind << "}\n";
        // Lanes past the row's chunks add 0 (their loads were clamped to the
        // last chunk).
        o << ind << "float ps = 0.0f;\n#pragma unroll\n" << ind << "for (uint32_t k = 0; k < " << K << "u; ++k)\n"
          << ind << "  ps += (threadIdx.x & 63u) + 64u * k < PF ? sv[k] : 0.0f;\n";
        o << ind << "for (int off = 32; off > 0; off >>= 1) ps += __shfl_xor(ps, off, 64);\n";
        {
          const ir::ReduceStage& rs = A.reduces[0];
          ExprGen fg(g_, o, ind, &counter_);
          fg.Bind(rs.fn.params[0], fg.Gen(rs.init));
          fg.Bind(rs.fn.params[1], "ps");
          std::string val = fg.Gen(rs.fn.body);
          if (A.has_piped) {
            std::map<int, std::string> piped;
            for (const auto& op : A.piped.ops) {
              if (piped.count(op.tensor)) continue;
              piped[op.tensor] = "ars" + std::to_string(op.tensor);
              o << ind << "const " << CType(g_.tensors[op.tensor].elem) << " ars" << op.tensor << " = t" << op.tensor
                << "[" << Offset(op.tensor, op.axes, coord) << "];\n";
            }
            ExprGen pg(g_, o, ind, &counter_);
            pg.Bind(A.piped.fn.params[0], val);
            for (size_t k = 0; k < A.piped.ops.size(); ++k)
              pg.Bind(A.piped.fn.params[k + 1], piped[A.piped.ops[k].tensor]);
            val = pg.Gen(A.piped.fn.body);
          }
          // Every lane holds the same value (the butterfly's sums are
          // symmetric): a scalar register, as a row scalar loaded from
          // memory would be.
          o << ind << "const float aval = tca::hip::wave_uniform(" << val << ");  // the value A stores and B reads\n";
        }
        o << ind << "float ptotal = 0.0f;\n#pragma unroll\n" << ind << "for (uint32_t k = 0; k < " << K << "u; ++k) {\n"
          << ind << "  const uint32_t c = (threadIdx.x & 63u) + 64u * k, cc = min(c, PF - 1u);  // sv[k], mv[k]: chunk cc\n"
          << ind << "  const float nc = static_cast<float>(min(PL, PVECS - cc * PL) * V);  // cc PL < PVECS\n" << ind
          << "  const float dc = sv[k] / nc - aval;\n" << ind << "  ptotal += c < PF ? mv[k] + nc * dc * dc : 0.0f;\n"
          << ind << "}\n";
        o << ind << "for (int off = 32; off > 0; off >>= 1) ptotal += __shfl_xor(ptotal, off, 64);  // about aval\n";
        o << ind << "ptotal = tca::hip::wave_uniform(ptotal);\n";
        // The compiler turns the chunk terms' selects into branches (a
        // division is costly); a load used only inside such a branch counts
        // as pending on the path that skipped it, and the compiler then
        // waited for all memory operations (vmcnt(0), stores included) at
        // the head of the row map's loop, every iteration. Settled here, once.
        o << ind << "tca::hip::wait_vector_memory();\n";
        pairFinishB(p, ind, "ptotal");
      };
      // pairValues for softmax's pair (max, then the sum of expf(t - max)):
      // aval, A's result (its partial maxima folded, init applied), and B's
      // total, the chunk pairs summed as s_c * expf(m_c - aval) (NaN when
      // aval is -inf).
      auto onlinePairValues = [&](size_t p, const std::string& ind) {
        const int ca = passes[p][0], cb = passes[p + 1][0];
        const ir::Chain& A = g_.chains[ca];
        const std::string sa = std::to_string(ca), sb = std::to_string(cb);
        o << ind << "const uint32_t PF = min(" << kMaxParts << "u, tca::hip::ceil_div(C / V, " << kOnlineChunkVecs
          << "u));  // the fused partial's chunks\n";
        o << ind << "const auto pcomb = [](float acc, float now) -> float {\n";
        {
          ExprGen cg(g_, o, ind + "  ", &counter_);
          cg.Bind(A.reduces[0].fn.params[0], "acc");
          cg.Bind(A.reduces[0].fn.params[1], "now");
          const std::string rr = cg.Gen(A.reduces[0].fn.body);
          o << ind << "  return " << rr << ";\n" << ind << "};\n";
        }
        o << ind << "float pm = 0.0f;\n" << ind << "bool ph = false;\n";
        o << ind << "{\n" << ind << "  float pv[" << kMaxParts / 64 << "];\n#pragma unroll\n" << ind
          << "  for (uint32_t k = 0; k < " << kMaxParts / 64 << "u; ++k)\n" << ind << "    pv[k] = p" << sa
          << "[static_cast<uint64_t>(r) * " << kMaxParts << "u + min((threadIdx.x & 63u) + 64u * k, PF - 1u)];\n"
          << "#pragma unroll\n" << ind << "  for (uint32_t k = 0; k < " << kMaxParts / 64 << "u; ++k) {\n" << ind
          << "    if ((threadIdx.x & 63u) + 64u * k < PF) {\n" << ind << "      pm = ph ? pcomb(pm, pv[k]) : pv[k];\n"
          << ind << "      ph = true;\n" << ind << "    }\n" << ind << "  }\n" << ind << "}\n";
        o << ind << "pm = tca::hip::wave_allreduce_present(pm, ph, pcomb);\n";
        {
          const ir::ReduceStage& rs = A.reduces[0];
          ExprGen fg(g_, o, ind, &counter_);
          fg.Bind(rs.fn.params[0], fg.Gen(rs.init));
          fg.Bind(rs.fn.params[1], "pm");
          const std::string val = fg.Gen(rs.fn.body);  // PF >= 1: init applied once to the row's total
          o << ind << "const float aval = " << val << ";  // the value A stores and B reads\n";
        }
        o << ind << "float psum = 0.0f;\n#pragma unroll\n" << ind << "for (uint32_t k = 0; k < " << kMaxParts / 64
          << "u; ++k) {\n" << ind << "  const uint32_t c = (threadIdx.x & 63u) + 64u * k;\n" << ind
          << "  if (c < PF)\n" << ind << "    psum += p" << sb << "[static_cast<uint64_t>(r) * " << kMaxParts
          << "u + c] * expf(q" << sb << "[static_cast<uint64_t>(r) * " << kMaxParts << "u + c] - aval);\n" << ind
          << "}\n" << ind << "for (int off = 32; off > 0; off >>= 1) psum += __shfl_xor(psum, off, 64);\n";
        o << ind << "const float ptotal = aval == -__builtin_inff() ? __builtin_nanf(\"\") : psum;\n";
        pairFinishB(p, ind, "ptotal");
      };
      // The values the fused pair (passes p, p + 1) stores for row r, in every
      // lane of each wave that runs this: aval, A's result, and bval, B's
      // (its init and piped map applied). Needs r and C in scope; names are
      // prefixed so the code can sit in the row map that reads the two
      // values.
      auto pairValues = [&](size_t p, const std::string& ind) {
        if (chanPair[p])
          chanPairValues(p, ind);
        else
          onlinePairValues(p, ind);
      };
      // Passes p (A: max of t) and p + 1 (B: sum of expf(t - a)) of a
      // softmax in one read of each chunk: the partial folds A's maximum as
      // pass p's partial does and, from the same element values, the online
      // pair (m_c, s_c) (tca::hip::online_expsum_add), merged over the lanes
      // and waves in a fixed order; the merge (one wave per row) finishes A
      // (init, store) and then B from the pairs: sum over chunks of
      // s_c * expf(m_c - a), a the value A stored (NaN when a is -inf: every
      // element -inf or NaN, where the direct sum is NaN), then B's init and
      // piped map.
      auto emitOnlinePair = [&](size_t p) {
        const int ca = passes[p][0], cb = passes[p + 1][0];
        const ir::Chain& A = g_.chains[ca];
        const ir::Chain& B = g_.chains[cb];
        const int ta = A.store_tensor, tb = B.store_tensor;
        const std::string tag = std::to_string(p + 1), sa = std::to_string(ca), sb = std::to_string(cb);
        const std::string fn = pk.symbol + "_spart" + tag;
        smFns.push_back({fn, p});
        smChunk[fn] = kOnlineChunkVecs;
        const bool chanKind = chanPair[p];
        o << "// statements #" << ca << " #" << cb << ": split rows, passes " << p + 1 << " and " << p + 2
          << (chanKind ? " in one read (a sum and the centred sum of squares about it, pairwise), partial folds\n"
                       : " in one read (max, then the online exp-sum against the chunk maxima), partial folds\n");
        o << "template <uint32_t V>\n__device__ __forceinline__ void " << fn << "(\n    " << sig << smSig << ") {\n";
        chunkHead(std::to_string(kOnlineChunkVecs) + "u");
        loadRowScalars(p, "  ");
        // Per lane: softmax's running maximum om (chain A's partial too: a
        // fold of the same values with fmaxf from -inf, which A's init is)
        // and sum os; or the values' sum cs (A's partial), centred sum of
        // squares cm (B's) and count cn.
        if (chanKind)
          o << "  float cs = 0.0f, cm = 0.0f, cn = 0.0f;\n";
        else
          o << "  float om = -__builtin_inff(), os = 0.0f;\n";
        const std::string upd = chanKind ? "tca::hip::chan_add(cs, cm, cn, ev);\n"
                                         : "tca::hip::online_expsum_add(om, os, ev);\n";
        // The values of vector `sfx` into ev[at * V + q].
        auto values = [&](std::ostringstream& b, const std::string& ind, const std::string& sfx, uint32_t at) {
          b << "#pragma unroll\n" << ind << "for (uint32_t q = 0; q < V; ++q) {\n";
          std::ostringstream es;
          const std::string ev = elemValue(es, ind + "  ", A, sfx);
          b << es.str() << ind << "  ev[" << at << "u * V + q] = " << ev << ";\n" << ind << "}\n";
        };
        // One update per kU vectors (kU V values: for softmax one rescale
        // test and at most one rescale per group). 8 vectors in flight per
        // lane measured 5% slower.
        constexpr uint32_t kU = 4;
        std::ostringstream b;
        b << "  {\n    const uint32_t vc = lo + threadIdx.x;\n";
        operands(b, p, "    ", false, "vc", "");
        b << "    float ev[V];\n";
        values(b, "    ", "", 0);
        b << "    " << upd;
        b << "  }\n  uint32_t v0 = lo + threadIdx.x + " << kPartBlock << "u;\n";
        b << "  for (; v0 + " << (kU - 1) * kPartBlock << "u < hi; v0 += " << kU * kPartBlock << "u) {\n";
        for (uint32_t u = 0; u < kU; ++u) b << "    const uint32_t vc_" << u << " = v0 + " << u * kPartBlock << "u;\n";
        for (uint32_t u = 0; u < kU; ++u) operands(b, p, "    ", false, "vc_" + std::to_string(u), "_" + std::to_string(u));
        b << "    float ev[" << kU << " * V];\n";
        for (uint32_t u = 0; u < kU; ++u) values(b, "    ", "_" + std::to_string(u), u);
        b << "    " << upd;
        b << "  }\n  for (; v0 < hi; v0 += " << kPartBlock << "u) {\n    const uint32_t vc = v0;\n";
        operands(b, p, "    ", false, "vc", "");
        b << "    float ev[V];\n";
        values(b, "    ", "", 0);
        b << "    " << upd;
        b << "  }\n";
        o << b.str();
        // The waves' results meet in lanes 0..15 of wave 0 (a 4-step
        // butterfly: a serial fold by one thread was the tail of every one
        // of the many short workgroups).
        static_assert(kPartBlock / 64 == 16, "16 waves per chunk");
        if (chanKind) {
          o << "  for (int off = 32; off > 0; off >>= 1)\n"
            << "    tca::hip::chan_merge_present(cs, cm, cn, __shfl_xor(cs, off, 64), __shfl_xor(cm, off, 64), "
               "__shfl_xor(cn, off, 64));\n";
          o << "  __shared__ float reds[" << kPartBlock / 64 << "], redm[" << kPartBlock / 64 << "], redn["
            << kPartBlock / 64 << "];\n";
          o << "  if ((threadIdx.x & 63u) == 0u) {\n    reds[threadIdx.x >> 6] = cs;\n    redm[threadIdx.x >> 6] = cm;\n"
               "    redn[threadIdx.x >> 6] = cn;\n  }\n";
          o << "  __syncthreads();\n  if (threadIdx.x < 64u) {\n";
          o << "    const uint32_t w = threadIdx.x & 15u;\n";
          o << "    const bool in = threadIdx.x < 16u;\n";
          o << "    float s = in ? reds[w] : 0.0f, m = in ? redm[w] : 0.0f, n = in ? redn[w] : 0.0f;\n";
          o << "    for (int off = 8; off > 0; off >>= 1)\n"
            << "      tca::hip::chan_merge_present(s, m, n, __shfl_xor(s, off, 64), __shfl_xor(m, off, 64), "
               "__shfl_xor(n, off, 64));\n";
          o << "    if (threadIdx.x == 0u) {  // the chunk's count is its vectors times V\n";
          o << "      p" << sa << "[static_cast<uint64_t>(r) * PMAX + p] = s;\n";
          o << "      p" << sb << "[static_cast<uint64_t>(r) * PMAX + p] = m;\n    }\n  }\n}\n";
        } else {
          o << "  for (int off = 32; off > 0; off >>= 1)\n"
            << "    tca::hip::online_expsum_merge(om, os, __shfl_xor(om, off, 64), __shfl_xor(os, off, 64));\n";
          o << "  __shared__ float redm[" << kPartBlock / 64 << "], reds[" << kPartBlock / 64 << "];\n";
          o << "  if ((threadIdx.x & 63u) == 0u) {\n    redm[threadIdx.x >> 6] = om;\n    reds[threadIdx.x >> 6] = os;\n  }\n";
          o << "  __syncthreads();\n  if (threadIdx.x < 64u) {\n";
          o << "    const uint32_t w = threadIdx.x & 15u;\n";
          o << "    float m = threadIdx.x < 16u ? redm[w] : -__builtin_inff(), s = threadIdx.x < 16u ? reds[w] : 0.0f;\n";
          o << "    for (int off = 8; off > 0; off >>= 1)\n"
            << "      tca::hip::online_expsum_merge(m, s, __shfl_xor(m, off, 64), __shfl_xor(s, off, 64));\n";
          o << "    if (threadIdx.x == 0u) {\n";
          o << "      p" << sa << "[static_cast<uint64_t>(r) * PMAX + p] = m;  // chain A's partial: the chunk's maximum\n";
          o << "      p" << sb << "[static_cast<uint64_t>(r) * PMAX + p] = s;\n";
          o << "      q" << sb << "[static_cast<uint64_t>(r) * PMAX + p] = m;\n    }\n  }\n}\n";
        }
        if (foldedMerge.count(p)) return;  // the row map computes (a, S) itself
        // The merge: one wave per row.
        const std::string mfn = pk.symbol + "_smerge" + tag;
        smFns.push_back({mfn, p});
        smChunk[mfn] = kOnlineChunkVecs;
        o << "template <uint32_t V>\n__device__ __forceinline__ void " << mfn << "(\n    " << sig << smSig << ") {\n";
        o << "  constexpr uint32_t PMAX = " << kMaxParts << "u;\n";
        o << "  const uint32_t C = " << ExtentExpr(g_, geo.col) << ";\n";
        o << "  const uint32_t r = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;\n";
        o << "  if (r >= " << ProductExpr(geo.outer) << ") return;  // whole waves\n";
        for (int a : geo.outer) o << "  const uint32_t c" << a << " = r;\n";
        pairValues(p, "  ");
        o << "  if (lane == 0u) {\n    t" << ta << "[" << Offset(ta, A.store_axes, coord) << "] = aval;\n    t" << tb
          << "[" << Offset(tb, B.store_axes, coord) << "] = bval;\n  }\n}\n";
      };
      for (size_t p = 0; p < passes.size(); ++p) {
        const ir::Chain& c0 = g_.chains[passes[p][0]];
        const bool red = !c0.reduces.empty();
        const std::string tag = std::to_string(p + 1);
        if (onlinePair[p]) {
          emitOnlinePair(p);
          ++p;  // pass p + 1 is folded into pass p's kernels
          continue;
        }
        if (red) {
          // Partial folds of pass p.
          const std::string fn = pk.symbol + "_spart" + tag;
          smFns.push_back({fn, p});
          o << "// statements";
          for (int ci : passes[p]) o << " #" << ci;
          o << ": split rows, pass " << tag << ", partial folds\n";
          o << "template <uint32_t V>\n__device__ __forceinline__ void " << fn << "(\n    " << sig << smSig << ") {\n";
          chunkHead(std::to_string(kChunkVecs) + "u");
          loadRowScalars(p, "  ");
          combsOf(p, "  ");
          for (int ci : passes[p]) {
            const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
            o << "  " << T << " part" << ci << " = " << T << "(0);\n";
          }
          std::ostringstream b;
          b << "  {\n    const uint32_t vc = lo + threadIdx.x;\n";
          operands(b, p, "    ", false, "vc", "");
          work(b, p, "    ", false, "vc", "true", "", true);
          b << "  }\n  uint32_t v0 = lo + threadIdx.x + " << kPartBlock << "u;\n";
          b << "  for (; v0 + " << 3 * kPartBlock << "u < hi; v0 += " << 4 * kPartBlock << "u) {\n";
          for (uint32_t u = 0; u < 4; ++u) b << "    const uint32_t vc_" << u << " = v0 + " << u * kPartBlock << "u;\n";
          for (uint32_t u = 0; u < 4; ++u) operands(b, p, "    ", false, "vc_" + std::to_string(u), "_" + std::to_string(u));
          for (uint32_t u = 0; u < 4; ++u)
            work(b, p, "    ", false, "vc_" + std::to_string(u), "true", "_" + std::to_string(u), false);
          b << "  }\n  for (; v0 < hi; v0 += " << kPartBlock << "u) {\n    const uint32_t vc = v0;\n";
          operands(b, p, "    ", false, "vc", "");
          work(b, p, "    ", false, "vc", "true", "", false);
          b << "  }\n";
          o << b.str();
          for (int ci : passes[p]) {
            const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
            o << "  part" << ci << " = tca::hip::seg_allreduce<64>(part" << ci << ", comb" << ci << ");\n";
            o << "  __shared__ " << T << " red" << ci << "[" << kPartBlock / 64 << "];\n";
            o << "  if ((threadIdx.x & 63u) == 0u) red" << ci << "[threadIdx.x >> 6] = part" << ci << ";\n";
          }
          o << "  __syncthreads();\n  if (threadIdx.x == 0u) {\n";
          for (int ci : passes[p]) {
            const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
            o << "    " << T << " acc" << ci << " = red" << ci << "[0];\n";
            o << "    for (uint32_t w = 1; w < " << kPartBlock / 64 << "u; ++w) acc" << ci << " = comb" << ci << "(acc"
              << ci << ", red" << ci << "[w]);\n";
            o << "    p" << ci << "[static_cast<uint64_t>(r) * PMAX + p] = acc" << ci << ";\n";
          }
          o << "  }\n}\n";
          // Merge of pass p: one wave per row.
          const std::string mfn = pk.symbol + "_smerge" + tag;
          smFns.push_back({mfn, p});
          o << "template <uint32_t V>\n__device__ __forceinline__ void " << mfn << "(\n    " << sig << smSig << ") {\n";
          o << "  constexpr uint32_t CV = " << kChunkVecs << "u, PMAX = " << kMaxParts << "u;\n";
          o << "  const uint32_t C = " << ExtentExpr(g_, geo.col) << ";\n";
          o << "  const uint32_t P = min(PMAX, tca::hip::ceil_div(C / V, CV));\n";
          o << "  const uint32_t r = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;\n";
          o << "  if (r >= " << rowExpr << ") return;  // whole waves\n";
          for (int a : geo.outer) o << "  const uint32_t c" << a << " = r;\n";
          loadRowScalars(p, "  ");
          combsOf(p, "  ");
          for (int ci : passes[p]) {
            const ir::Chain& c = g_.chains[ci];
            const int st = c.store_tensor;
            const std::string T = CType(g_.exprs[c.root.fn.body].type);
            const std::string A = "m" + std::to_string(ci), H = "h" + std::to_string(ci);
            o << "  " << T << " " << A << " = " << T << "(0);\n  bool " << H << " = false;\n";
            o << "  {\n    " << T << " pv[PMAX / 64u];\n";
            o << "#pragma unroll\n    for (uint32_t k = 0; k < PMAX / 64u; ++k)\n";
            o << "      pv[k] = p" << ci << "[static_cast<uint64_t>(r) * PMAX + min(lane + 64u * k, P - 1u)];\n";
            o << "#pragma unroll\n    for (uint32_t k = 0; k < PMAX / 64u; ++k) {\n";
            o << "      if (lane + 64u * k < P) {\n";
            o << "        " << A << " = " << H << " ? comb" << ci << "(" << A << ", pv[k]) : pv[k];\n        " << H
              << " = true;\n      }\n    }\n  }\n";
            o << "  " << A << " = tca::hip::wave_allreduce_present(" << A << ", " << H << ", comb" << ci << ");\n";
            o << "  if (lane == 0u) {\n";
            const ir::ReduceStage& rs = c.reduces[0];
            ExprGen fg(g_, o, "    ", &counter_);
            fg.Bind(rs.fn.params[0], fg.Gen(rs.init));
            fg.Bind(rs.fn.params[1], A);
            std::string val = fg.Gen(rs.fn.body);  // P >= 1: init applied once to the row's total
            if (c.has_piped) {
              ExprGen pg(g_, o, "    ", &counter_);
              pg.Bind(c.piped.fn.params[0], val);
              for (size_t k = 0; k < c.piped.ops.size(); ++k)
                pg.Bind(c.piped.fn.params[k + 1], "rs" + std::to_string(c.piped.ops[k].tensor));
              val = pg.Gen(c.piped.fn.body);
            }
            o << "    t" << st << "[" << Offset(st, c.store_axes, coord) << "] = " << val << ";\n";
            o << "  }\n";
          }
          o << "}\n";
        } else {
          // Row map of pass p over the chunk.
          const std::string fn = pk.symbol + "_smap" + tag;
          smFns.push_back({fn, p});
          const bool folded = p >= 2 && foldedMerge.count(p - 2);
          // A map that folds a mean/variance pair's merge takes its chunk
          // length CVM as a template argument (longMaps).
          const bool longMap = folded && chanPair[p - 2];
          if (longMap) longMaps.insert(fn);
          o << "// statement #" << passes[p][0] << ": split rows, pass " << tag << ", row map over a chunk\n";
          o << "template <uint32_t V" << (longMap ? ", uint32_t CVM" : "") << ">\n__device__ __forceinline__ void " << fn
            << "(\n    " << sig << smSig << ") {\n";
          chunkHead(longMap ? std::string("CVM") : std::to_string(kChunkVecs) + "u");
          if (folded) {
            // The fused pair's values for this row, computed here (every wave).
            const ir::Chain& A = g_.chains[passes[p - 2][0]];
            const ir::Chain& B = g_.chains[passes[p - 1][0]];
            pairValues(p - 2, "  ");
            o << "  if (p == 0u && threadIdx.x == 0u) {\n    t" << A.store_tensor << "["
              << Offset(A.store_tensor, A.store_axes, coord) << "] = aval;\n    t" << B.store_tensor << "["
              << Offset(B.store_tensor, B.store_axes, coord) << "] = bval;\n  }\n";
            computed[A.store_tensor] = "aval";
            computed[B.store_tensor] = "bval";
          }
          loadRowScalars(p, "  ");
          computed.clear();
          std::ostringstream b;
          b << "  uint32_t v0 = lo + threadIdx.x;\n";
          b << "  for (; v0 + " << 3 * kPartBlock << "u < hi; v0 += " << 4 * kPartBlock << "u) {\n";
          for (uint32_t u = 0; u < 4; ++u) b << "    const uint32_t vc_" << u << " = v0 + " << u * kPartBlock << "u;\n";
          for (uint32_t u = 0; u < 4; ++u) operands(b, p, "    ", false, "vc_" + std::to_string(u), "_" + std::to_string(u));
          for (uint32_t u = 0; u < 4; ++u)
            work(b, p, "    ", false, "vc_" + std::to_string(u), "true", "_" + std::to_string(u), false);
          b << "  }\n  for (; v0 < hi; v0 += " << kPartBlock << "u) {\n    const uint32_t vc = v0;\n";
          operands(b, p, "    ", false, "vc", "");
          work(b, p, "    ", false, "vc", "true", "", false);
          b << "  }\n";
          o << b.str() << "}\n";
        }
      }
    }
    // One kernel per (vector width, cached | streamed); launch guards on the
    // row length pick exactly one: the widest width W (16 bytes of the
    // widest row-shaped tensor) for C % W == 0, then each smaller power of
    // two v for C % 2v == v (f32: C % 4 == 0: V 4; C % 4 == 2: V 2; odd:
    // V 1), then the row length in vectors.
    const std::string args = CallArgs(n);
    const std::string cdim = g_.dims[geo.col].name;
    struct Width {
      uint32_t v, mod, rem;
    };
    std::vector<Width> widths;
    {
      const uint32_t vmax = RowVecMax(g_, n.chains, geo);
      widths.push_back({vmax, vmax, 0});
      for (uint32_t v = vmax / 2; v >= 1; v /= 2) widths.push_back({v, 2 * v, v});
    }
    // A nest of several passes re-reads a streamed row once per pass; longer
    // rows stay in registers for it: 8 vectors per lane of a 1024-lane block
    // (rows of up to 8192 vectors), a variant of its own (its register count
    // is set by its cache depth; 16 vectors spilled to scratch for 16- and
    // 8-byte vectors). A single pass reads the row once either way and keeps
    // the 4-vector cache only.
    // A column vector read by several passes stays live across them (the
    // compiler keeps its loads for the later passes): 8 more vectors beside
    // the 8-deep cached row spill to scratch, so such nests keep the 4-deep
    // cache and stream longer rows.
    size_t colVecPasses = 0;
    for (const auto& ps : passes) {
      bool reads = false;
      for (int ci : ps)
        for (const auto& op : g_.chains[ci].root.ops) reads = reads || Classify(op, geo) == OpKind::ColVec;
      colVecPasses += reads ? 1 : 0;
    }
    std::vector<uint32_t> caches = {kCache};
    if (passes.size() > 1 && colVecPasses < 2) caches.push_back(2 * kCache);
    const uint64_t cachedVecs = uint64_t{kBlock} * caches.back();
    const std::string symbol = pk.symbol;
    const std::string rowGuard =
        geo.outer.size() == 1 ? g_.dims[geo.outer[0]].name : std::string();  // the split's row-count dim
    for (const auto& w : widths) {
      for (size_t ci = 0; ci <= caches.size(); ++ci) {
        const bool cached = ci < caches.size();
        const uint32_t kc = cached ? caches[ci] : 0u;
        const uint64_t lo = !cached ? (cachedVecs + 1) * w.v : ci == 0 ? 0 : (uint64_t{kBlock} * caches[ci - 1] + 1) * w.v;
        const uint64_t hi = cached ? uint64_t{kBlock} * kc * w.v : 0xffffffffull;
        if (!cached && (split || splitMulti) && rowGuard.empty()) continue;  // one row: always split
        // A cached row of exactly kc * 2^k vectors (every lane holds kc: no
        // ownership test or clamp) runs a kernel of its own, so the general
        // path's registers do not set its occupancy (layernorm, 1024-lane
        // rows of 8192 floats: 99 -> 75 VGPRs, 25% faster). Only the widest
        // width can fit exactly: the narrower ones take rows of an odd vector
        // count. Not at the 8-vector depth: one 1024-lane block per CU either
        // way, and there one kernel branching to both bodies at run time was
        // the fastest softmax (111.8 us at [2048, 32768], against 118 exact-fit
        // only and 131 general only). exact: 0 general, 1 exact-fit.
        const bool canExact = cached && w.rem == 0 && kc == kCache;
        for (int exact = 0; exact <= (canExact ? 1 : 0); ++exact) {
          PlanKernel vk = pk;
          vk.symbol = symbol + (cached ? "_c" : "_s") + std::to_string(w.v) +
                      (kc > kCache ? "x" + std::to_string(kc) : "") + (exact ? "e" : "");
          vk.block = kBlock;
          vk.pack = cdim + " " + std::to_string((cached ? kc : kCache) * w.v) + " " + std::to_string(kMinBlock);
          vk.grid.push_back(DimProduct(geo.outer) + "/pack");
          vk.when.push_back(cdim + " " + std::to_string(lo) + " " + std::to_string(hi) + " " + std::to_string(w.mod) +
                            " " + std::to_string(w.rem));
          const std::string fit = cdim + " 0 4294967295 " + std::to_string(uint64_t{kc} * w.v) + " 0 pow2";
          if (exact) vk.when.push_back(fit);
          else if (canExact) vk.unless.push_back(fit);
          if (!cached && (split || splitMulti)) {
            vk.when.push_back(rowGuard + " " + std::to_string(kSplitRows + 1) + " 4294967295 1 0");
            if (splitMulti) {  // not long rows of at most kSplitRowsLong rows: those split
              vk.unless.push_back(rowGuard + " 0 " + std::to_string(kSplitRowsLong) + " 1 0");
              vk.unless.push_back(cdim + " " + std::to_string(uint64_t{kSplitLongVecs} * w.v) + " 4294967295 1 0");
            }
          }
          o << "extern \"C\" __global__ void __launch_bounds__(" << kBlock << ") " << vk.symbol << "(\n    " << sig
            << ") {\n";
          if (cached && canExact) {
            o << "  " << body_fn << "<" << w.v << "u, " << kc << "u, " << (exact ? "true" : "false") << ">(" << args
              << ");\n}\n";
          } else if (cached) {
            o << "  const uint32_t vecs = (" << ExtentExpr(g_, geo.col) << ") / " << w.v << "u;\n";
            o << "  const uint32_t ls = tca::hip::pack_lanes_log2(vecs, " << kc << "u, " << lgBlock << "u);\n";
            o << "  if (vecs == (" << kc << "u << ls)) " << body_fn << "<" << w.v << "u, " << kc << "u, true>(" << args
              << ");\n";
            o << "  else " << body_fn << "<" << w.v << "u, " << kc << "u, false>(" << args << ");\n}\n";
          } else
            o << "  " << body_fn << "<" << w.v << "u, 0u, false>(" << args << ");\n}\n";
          std::ostringstream det;
          det << "row=runtime (" << cdim << " % " << w.mod << " == " << w.rem << ", " << lo << ".." << hi << ": "
              << (cached ? "cached " + std::to_string(kc) + " vectors/lane" + (exact ? ", exact fit" : "")
                         : std::string("streamed"))
              << ") vec=" << w.v << " lanes/row=runtime(<=" << kBlock << ") passes=" << passes.size() << " block=max("
              << kMinBlock << ",lanes/row)";
          AddKernel(vk, Family::Stream, n.chains, det.str());
        }
      }
      if (splitMulti) {
        const uint64_t lo = (cachedVecs + 1) * w.v;
        // (device function, pass, chunk of a long map's kernel or 0)
        std::vector<std::tuple<std::string, size_t, uint32_t>> kernels;
        for (const auto& fp : smFns) {
          if (!longMaps.count(fp.first)) {
            kernels.emplace_back(fp.first, fp.second, 0u);
            continue;
          }
          kernels.emplace_back(fp.first, fp.second, kChunkVecs);
          kernels.emplace_back(fp.first, fp.second, 4 * kChunkVecs);
        }
        for (const auto& kf : kernels) {
          const std::string& fn = std::get<0>(kf);
          const uint32_t mapChunk = std::get<2>(kf);
          const bool merge = fn.find("_smerge") != std::string::npos, map = fn.find("_smap") != std::string::npos;
          const bool longChunk = mapChunk > kChunkVecs;
          const std::string tag = std::to_string(std::get<1>(kf) + 1);
          PlanKernel sk = pk;
          sk.symbol = symbol + (merge ? "_m" : map ? (longChunk ? "_wl" : "_w") : "_p") + std::to_string(w.v) + "_" + tag;
          sk.block = merge ? 256 : kPartBlock;
          for (const auto& a : smPlanArgs) sk.args.push_back(a);
          if (merge) {
            sk.grid.push_back(rowGuard.empty() ? std::string("1/1") : DimProduct(geo.outer) + "/4");
          } else {
            if (!rowGuard.empty()) sk.grid.push_back(DimProduct(geo.outer) + "/1");
            const auto cv = smChunk.find(fn);
            const uint64_t chunk = mapChunk ? mapChunk : cv == smChunk.end() ? kChunkVecs : cv->second;
            sk.grid.push_back(cdim + "/" + std::to_string(chunk * w.v) + ":" + std::to_string(kMaxParts));
          }
          // A long map's two kernels split the row lengths at kLongMapVecs vectors.
          const uint64_t longFrom = uint64_t{kLongMapVecs} * w.v;
          const uint64_t klo = longChunk ? longFrom : lo;
          const std::string khi = mapChunk == kChunkVecs ? std::to_string(longFrom - 1) : std::string("4294967295");
          sk.when.push_back(cdim + " " + std::to_string(klo) + " " + khi + " " + std::to_string(w.mod) + " " +
                            std::to_string(w.rem));
          if (!rowGuard.empty()) {  // rows <= kSplitRows, or long rows of at most kSplitRowsLong rows
            sk.when.push_back(rowGuard + " 0 " + std::to_string(kSplitRowsLong) + " 1 0");
            sk.unless.push_back(rowGuard + " " + std::to_string(kSplitRows + 1) + " 4294967295 1 0");
            sk.unless.push_back(cdim + " 0 " + std::to_string(uint64_t{kSplitLongVecs} * w.v - 1) + " 1 0");
          }
          o << "extern \"C\" __global__ void __launch_bounds__(" << sk.block << ") " << sk.symbol << "(\n    " << sig
            << smSig << ") {\n  " << fn << "<" << w.v << "u" << (mapChunk ? ", " + std::to_string(mapChunk) + "u" : "")
            << ">(" << args << smArgs << ");\n}\n";
          std::ostringstream det;
          det << "row=runtime (" << cdim << " % " << w.mod << " == " << w.rem << ", " << klo << ".." << khi
              << (rowGuard.empty() ? std::string()
                                   : ", rows <= " + std::to_string(kSplitRows) + ", or <= " +
                                         std::to_string(kSplitRowsLong) + " of >= " +
                                         std::to_string(uint64_t{kSplitLongVecs} * w.v))
              << ": split, pass "
              << tag << ") vec=" << w.v
              << (merge ? " merge: one wave per row over <= " + std::to_string(kMaxParts) + " partials"
                        : (map ? " row map: " : " partial: ") + std::to_string(kPartBlock) + " lanes per chunk of >= " +
                              std::to_string((longChunk ? mapChunk : kChunkVecs) / 2) + " vectors");
          AddKernel(sk, Family::Stream, n.chains, det.str());
        }
      }
      if (!split) continue;
      // The split pair for this width: partial folds, then the merge.
      const uint64_t lo = (cachedVecs + 1) * w.v;
      std::string partArgs = args;
      for (int ci : passes[0]) partArgs += ", p" + std::to_string(ci);
      std::string partSig2;
      for (int ci : passes[0]) {
        const ir::Elem pe = g_.exprs[g_.chains[ci].root.fn.body].type;
        partSig2 += ",\n    " + CType(pe) + "* __restrict__ p" + std::to_string(ci);
      }
      for (int merge = 0; merge <= 1; ++merge) {
        PlanKernel sk = pk;
        sk.symbol = symbol + (merge ? "_m" : "_p") + std::to_string(w.v);
        sk.block = merge ? 256 : kPartBlock;
        for (const auto& nm : part_names) sk.args.push_back("ptr " + nm);
        if (merge) {
          sk.grid.push_back(rowGuard.empty() ? std::string("1/1") : DimProduct(geo.outer) + "/4");
        } else {
          if (!rowGuard.empty()) sk.grid.push_back(DimProduct(geo.outer) + "/1");
          sk.grid.push_back(cdim + "/" + std::to_string(uint64_t{kChunkVecs} * w.v) + ":" + std::to_string(kMaxParts));
        }
        sk.when.push_back(cdim + " " + std::to_string(lo) + " 4294967295 " + std::to_string(w.mod) + " " +
                          std::to_string(w.rem));
        if (!rowGuard.empty()) sk.when.push_back(rowGuard + " 0 " + std::to_string(kSplitRows) + " 1 0");
        o << "extern \"C\" __global__ void __launch_bounds__(" << sk.block << ") " << sk.symbol << "(\n    " << sig
          << partSig2 << ") {\n  " << (merge ? merge_fn : part_fn) << "<" << w.v << "u>(" << partArgs << ");\n}\n";
        std::ostringstream det;
        det << "row=runtime (" << cdim << " % " << w.mod << " == " << w.rem << ", >= " << lo
            << (rowGuard.empty() ? std::string() : ", rows <= " + std::to_string(kSplitRows)) << ": split) vec=" << w.v
            << (merge ? " merge: one wave per row over <= " + std::to_string(kMaxParts) + " partials"
                      : " partial: " + std::to_string(kPartBlock) + " lanes per chunk of >= " +
                            std::to_string(kChunkVecs / 2) + " vectors");
        AddKernel(sk, Family::Stream, n.chains, det.str());
      }
    }
    o << "\n";
    return true;
  }

  // C: reductions over a non-contiguous axis. Threads span the contiguous
  // axis in vectors of V elements (16 bytes of the widest tile or column
  // vector): SL = min(32, smallest power of two >= C / V) threads per row
  // and 256 / SL rows per block step, 256 threads per block. A block owns 32
  // column vectors of one outer index and a chunk of the reduced axis: P
  // chunks, P = col_split(R, column blocks, 64, 1024) — enough blocks to
  // fill the GPU, >= 64 rows each, and a partial scratch of at most
  // 1024 x 32 vectors. Chunk p covers rows [p R / P, (p + 1) R / P), never empty when
  // P > 1 (P <= R). Each thread folds its columns over its rows in registers
  // with 4 rows in flight; the row slots of a block meet in LDS. With P = 1
  // the block applies init and the piped map and stores; otherwise it writes
  // its partials and a merge kernel (launched only when P > 1; 64 outputs
  // per block, its 16 waves folding every 16th chunk) combines them. Loads
  // are unmasked: lanes past the last column read the row's last vector and
  // store nothing.
  //
  // A nest of several passes (a chain that reads the result of an earlier
  // one, e.g. a variance reading its mean) has two lowerings, picked at
  // launch by the same P: with P = 1 one whole-column kernel runs every pass
  // in turn over all rows, the results a later pass reads handed from the
  // finishing threads to the block through LDS (no HBM round trip; results
  // that are locals read only inside the nest are not stored at all); with
  // P > 1 each pass is its own partial + merge pair, and a later pass loads
  // an earlier one's result from HBM like any column vector.
  bool EmitCol(int ni, std::string* err) {
    // Swept on MI355X (column sum+max, [8192, 8192] .. [16, 4 Mi]): spans of
    // 64 vectors beat 256 (4.7-5.7 against 4.3-4.8 TB/s); a 1024-block
    // split target beats 512, 2048 and 4096; 8 and 16 waves per block lose
    // 3-20% except on [8192, 8192]; two 16-byte vectors per thread and row
    // (8 f32 columns) lose 11-25%. Groups of 16 rows in flight per thread
    // gain 9-11% on [8192, 8192] over groups of 4; as the first and the
    // last group they cost 18-40% on [16, 4 Mi] (4 rows per wave: clamped
    // rows re-read, guarded loads wait one by one), so only the main loop
    // takes 16 rows and the ends keep clamped groups of 4: +7% on
    // [8192, 8192], +2% on [16, 4 Mi], within 2% on the other shapes.
    // Column blocks of 32 vectors (512 bytes of a row): swept on [8192, 8192]
    // with 256 threads, 32 vectors read at 6.5 TB/s against 5.4 for 64 and 6.0
    // for 16, whatever the thread count (256-1024) or rows in flight (8-32).
    constexpr uint32_t kWaves = 4, kRowsMin = 64, kBlocks = 1024, kUnroll = 16, kEdge = 4, kMergeWaves = 16, kSpan = 32,
                       kLogSpan = 5;
    const Nest& n = an_.nests[ni];
    const ColGeom geo = ColCheck(g_, n.chains);
    if (!geo.ok) {
      *err = "emit: column family rejected a nest it classified: " + geo.why;
      return false;
    }
    PlanKernel pk;
    pk.symbol = Sym(g_, prefix_, ni);
    const std::string sig = Signature(n, &pk);
    const std::string sym = pk.symbol;
    std::ostringstream& o = src_;
    // The chains of each pass.
    std::vector<std::vector<int>> passChains(geo.passes);
    for (size_t i = 0; i < n.chains.size(); ++i) passChains[geo.pass[i]].push_back(n.chains[i]);
    // A mean and its centred sum of squares: one read (ChanMeanVar).
    const bool chan = opts_.allow_pass_fusion && geo.passes == 2 && passChains[0].size() == 1 &&
                      passChains[1].size() == 1 &&
                      ChanMeanVar(g_, g_.chains[passChains[0][0]], g_.chains[passChains[1][0]], geo);
    // Vectors are 16 bytes of the widest tile or column vector a kernel
    // loads (the one-read kernels never load the nest's own results).
    size_t widest = 1;
    for (int ci : n.chains)
      for (const auto& op : g_.chains[ci].root.ops) {
        const ColKind k = ClassifyCol(op, geo);
        if (chan && k == ColKind::ColVec && op.tensor == g_.chains[passChains[0][0]].store_tensor) continue;
        if (k == ColKind::Tile || k == ColKind::ColVec)
          widest = std::max(widest, ir::ElemBytes(g_.tensors[op.tensor].elem));
      }
    const uint32_t vmax = static_cast<uint32_t>(std::max<size_t>(1, 16 / widest));
    // Partial scratch: one plan-only local per reduction.
    const std::string partDim = "__coldim" + std::to_string(ni);
    extra_dims_.push_back(partDim + " " + std::to_string(uint64_t{kBlocks} * kSpan * vmax));
    std::string partSig, partArgs;
    std::vector<std::string> partNames;
    for (int ci : n.chains) {
      const ir::Elem pe = g_.exprs[g_.chains[ci].root.fn.body].type;
      const std::string nm = "__colpart" + std::to_string(ci);
      partNames.push_back(nm);
      extra_tensors_.push_back(nm + " " + ir::ElemName(pe) + " local 1 " + partDim);
      partSig += ",\n    " + CType(pe) + "* __restrict__ p" + std::to_string(ci) + " /* " + nm + " */";
      partArgs += ", p" + std::to_string(ci);
    }
    // The results of the nest a later pass reads.
    std::set<int> results, readLater;
    for (int ci : n.chains) results.insert(g_.chains[ci].store_tensor);
    // Operands by kind (root and piped maps) over a set of chains, each
    // loaded once per kind.
    struct Ops {
      std::vector<int> tiles, colvecs, rowvecs, outers;
    };
    std::map<int, const ir::Operand*> opOf;
    auto opsOf = [&](const std::vector<int>& cs) {
      Ops k;
      auto note = [](std::vector<int>& v, int t) {
        if (std::find(v.begin(), v.end(), t) == v.end()) v.push_back(t);
      };
      for (int ci : cs) {
        const ir::Chain& c = g_.chains[ci];
        std::vector<const ir::Operand*> ops;
        for (const auto& op : c.root.ops) ops.push_back(&op);
        if (c.has_piped)
          for (const auto& op : c.piped.ops) ops.push_back(&op);
        for (const ir::Operand* op : ops) {
          opOf[op->tensor] = op;
          switch (ClassifyCol(*op, geo)) {
            case ColKind::Tile: note(k.tiles, op->tensor); break;
            case ColKind::ColVec: note(k.colvecs, op->tensor); break;
            case ColKind::RowVec: note(k.rowvecs, op->tensor); break;
            default: note(k.outers, op->tensor); break;
          }
        }
      }
      return k;
    };
    const Ops all = opsOf(n.chains);
    for (int t : all.colvecs)
      if (results.count(t)) readLater.insert(t);
    auto kindOf = [&](int t) { return ClassifyCol(*opOf[t], geo); };
    // A result the whole-column kernel need not store: a local no chain
    // outside this nest reads.
    auto internalLocal = [&](int t) {
      if (!g_.tensors[t].local) return false;
      for (size_t nj = 0; nj < an_.nests.size(); ++nj)
        if (static_cast<int>(nj) != ni)
          for (int cj : an_.nests[nj].chains)
            if (ReadSet(g_.chains[cj]).count(t)) return false;
      return true;
    };
    // Coordinates: outer axes c<a>, the column `colv`, the row `rowv`.
    auto coordFn = [&](const std::string& colv, const std::string& rowv) {
      return [&, colv, rowv](int a) -> std::string {
        if (a == geo.c) return colv;
        if (a == geo.r) return rowv;
        return "c" + std::to_string(a);
      };
    };
    auto outerCoords = [&](const std::string& ind, const std::string& flat) {
      o << ind << "uint32_t orem = " << flat << ";\n";
      for (int k = static_cast<int>(geo.outer.size()) - 1; k >= 0; --k) {
        const int a = geo.outer[k];
        if (k == 0)
          o << ind << "const uint32_t c" << a << " = orem;\n";
        else
          o << ind << "const uint32_t c" << a << " = orem % " << ExtentExpr(g_, a) << "; orem /= " << ExtentExpr(g_, a)
            << ";\n";
      }
      o << ind << "(void)orem;\n";
    };
    auto combs = [&](const std::string& ind, const std::vector<int>& cs) {
      for (int ci : cs) {
        const ir::Chain& c = g_.chains[ci];
        const std::string T = CType(g_.exprs[c.root.fn.body].type);
        o << ind << "const auto comb" << ci << " = [](" << T << " acc, " << T << " now) -> " << T << " {\n";
        ExprGen cg(g_, o, ind + "  ", &counter_);
        cg.Bind(c.reduces[0].fn.params[0], "acc");
        cg.Bind(c.reduces[0].fn.params[1], "now");
        const std::string r = cg.Gen(c.reduces[0].fn.body);
        o << ind << "  return " << r << ";\n" << ind << "};\n";
      }
    };
    // init, the piped map and the store of chain ci's reduced value `acc`
    // (`present`: the value folded anything) at column `col`, with column
    // vectors read by `colval`; `store` false skips the store, and a
    // non-empty `bcast` also receives the stored value.
    auto finish = [&](std::ostringstream& b, const std::string& ind, int ci, const std::string& acc,
                      const std::string& present, const std::string& col,
                      const std::function<std::string(int)>& colval, bool store = true,
                      const std::string& bcast = std::string()) {
      const ir::Chain& c = g_.chains[ci];
      const ir::ReduceStage& r = c.reduces[0];
      const std::string T = CType(g_.exprs[c.root.fn.body].type);
      ExprGen ig(g_, b, ind, &counter_);
      const std::string init = ig.Gen(r.init);
      const std::string fin = "fin" + std::to_string(ci);
      b << ind << T << " " << fin << " = " << init << ";\n";
      b << ind << "if (" << present << ") {\n";
      {
        ExprGen fg(g_, b, ind + "  ", &counter_);
        fg.Bind(r.fn.params[0], init);
        fg.Bind(r.fn.params[1], acc);
        const std::string v = fg.Gen(r.fn.body);
        b << ind << "  " << fin << " = " << v << ";\n";
      }
      b << ind << "}\n";
      std::string val = fin;
      if (c.has_piped) {
        ExprGen pg(g_, b, ind, &counter_);
        pg.Bind(c.piped.fn.params[0], val);
        for (size_t k = 0; k < c.piped.ops.size(); ++k) {
          const int t = c.piped.ops[k].tensor;
          pg.Bind(c.piped.fn.params[k + 1], kindOf(t) == ColKind::ColVec ? colval(t) : "os" + std::to_string(t));
        }
        val = pg.Gen(c.piped.fn.body);
      }
      const int st = c.store_tensor;
      if (store) b << ind << "t" << st << "[" << Offset(st, c.store_axes, coordFn(col, "0u")) << "] = " << val << ";\n";
      if (!bcast.empty()) b << ind << bcast << " = " << val << ";\n";
    };
    // Loads of row `rv` into x<t><sfx> / rv<t><sfx>, then the fold of the
    // chains `cs` into part<ci>.
    auto loads = [&](std::ostringstream& b, const Ops& k, const std::string& ind, const std::string& rv,
                     const std::string& sfx) {
      const auto at = coordFn("col0", rv);
      for (int t : k.tiles)
        b << ind << "const auto x" << t << sfx << " = tca::hip::load_vec_nt<" << CType(g_.tensors[t].elem) << ", V>(t"
          << t << " + " << Offset(t, opOf[t]->axes, at) << ");\n";
      for (int t : k.rowvecs)
        b << ind << "const " << CType(g_.tensors[t].elem) << " rv" << t << sfx << " = t" << t << "["
          << Offset(t, opOf[t]->axes, at) << "];\n";
    };
    auto fold = [&](std::ostringstream& b, const std::vector<int>& cs, const std::string& ind, const std::string& sfx,
                    bool first, const std::string& ok) {
      b << "#pragma unroll\n" << ind << "for (uint32_t q = 0; q < V; ++q) {\n";
      for (int ci : cs) {
        const ir::Chain& c = g_.chains[ci];
        ExprGen eg(g_, b, ind + "  ", &counter_);
        for (size_t k = 0; k < c.root.ops.size(); ++k) {
          const int t = c.root.ops[k].tensor;
          std::string v;
          switch (kindOf(t)) {
            case ColKind::Tile: v = "x" + std::to_string(t) + sfx + "[q]"; break;
            case ColKind::ColVec: v = "cv" + std::to_string(t) + "[q]"; break;
            case ColKind::RowVec: v = "rv" + std::to_string(t) + sfx; break;
            default: v = "os" + std::to_string(t); break;
          }
          eg.Bind(c.root.fn.params[k], v);
        }
        const std::string ev = eg.Gen(c.root.fn.body);
        const std::string P = "part" + std::to_string(ci) + "[q]";
        if (first) b << ind << "  " << P << " = " << ev << ";\n";
        else if (ok.empty()) b << ind << "  " << P << " = comb" << ci << "(" << P << ", " << ev << ");\n";
        else b << ind << "  " << P << " = " << ok << " ? comb" << ci << "(" << P << ", " << ev << ") : " << P << ";\n";
      }
      b << ind << "}\n";
      for (int ci : cs)
        if (FoldFenced(g_.exprs[g_.chains[ci].root.fn.body].type))
          b << "#pragma unroll\n" << ind << "for (uint32_t q = 0; q < V; ++q) tca::hip::fold_fence(part" << ci
            << "[q]);\n";
    };
    // The row loop of a block over [r_lo, r_hi) for the chains `cs`: a
    // first group of kUnroll rows when every slot owns that many, else of
    // kEdge rows, groups of kUnroll rows while whole ones fit, then groups
    // of kEdge to the chunk's end. The edge groups clamp
    // rows past the chunk to its last row (unconditional loads stay in
    // flight together) and fold only the rows they own; row 0 of each is
    // always owned. Declares `has` (the thread's slot holds a row).
    // The loads of one group of `rows` rows from row r into x<t>_u / rv<t>_u;
    // `clamped` groups also declare ok_u (row u is the chunk's) and read a
    // row past the chunk as its last row.
    auto groupLoads = [&](std::ostringstream& b, const Ops& k, const std::string& ind, uint32_t rows, bool clamped) {
      for (uint32_t u = 0; u < rows; ++u) {
        const std::string us = std::to_string(u);
        if (clamped && u > 0) {
          b << ind << "const bool ok_" << us << " = r + " << us << "u * STEP < r_hi;\n";
          b << ind << "const uint32_t rr_" << us << " = ok_" << us << " ? r + " << us << "u * STEP : r_hi - 1u;\n";
          loads(b, k, ind, "rr_" + us, "_" + us);
        } else {
          loads(b, k, ind, "r + " + us + "u * STEP", "_" + us);
        }
      }
    };
    // The skeleton of a block's row loop, `group(ind, rows, clamped, first)`
    // emitting each group: declares `has` (the thread's slot holds a row)
    // and walks r over the slot's rows.
    auto rowSkeleton = [&](std::ostringstream& b, const std::string& hasName,
                           const std::function<void(const std::string&, uint32_t, bool, bool)>& group) {
      b << "  uint32_t r = r_lo + slot;\n  const bool " << hasName << " = r < r_hi;\n  if (" << hasName << ") {\n";
      // A first group of 16 when every slot of the block owns >= 16 rows
      // (block-uniform), else of 4 (clamped).
      b << "    if (r_hi - r_lo >= " << kUnroll << "u * STEP) {\n";
      group("      ", kUnroll, false, true);
      b << "      r += " << kUnroll << "u * STEP;\n    } else {\n";
      group("      ", kEdge, true, true);
      b << "      r += " << kEdge << "u * STEP;\n    }\n";
      b << "    for (; r + " << kUnroll - 1 << "u * STEP < r_hi; r += " << kUnroll << "u * STEP) {\n";
      group("      ", kUnroll, false, false);
      b << "    }\n    for (; r < r_hi; r += " << kEdge << "u * STEP) {\n";
      group("      ", kEdge, true, false);
      b << "    }\n  }\n";
    };
    auto rowLoop = [&](const std::vector<int>& cs, const Ops& k, const std::string& hasName) {
      std::ostringstream b;
      rowSkeleton(b, hasName, [&](const std::string& ind, uint32_t rows, bool clamped, bool first) {
        groupLoads(b, k, ind, rows, clamped);
        for (uint32_t u = 0; u < rows; ++u)
          fold(b, cs, ind, "_" + std::to_string(u), first && u == 0, clamped && u > 0 ? "ok_" + std::to_string(u) : "");
      });
      return b.str();
    };
    auto partDecls = [&](const std::vector<int>& cs) {
      for (int ci : cs) {
        const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
        o << "  " << T << " part" << ci << "[V];\n";
        o << "#pragma unroll\n  for (uint32_t q = 0; q < V; ++q) part" << ci << "[q] = " << T << "(0);\n";
      }
    };
    // Block geometry shared by the partial and whole-column kernels.
    auto blockGeom = [&]() {
      o << "  uint32_t LSL = 0u;  // SL = 2^LSL lanes per row, the smallest power of two >= VEC, at most SPAN\n";
      o << "  while (LSL < LSPAN && (1u << LSL) < VEC) ++LSL;\n";
      o << "  const uint32_t SL = 1u << LSL, STEP = (W * 64u) >> LSL;  // STEP rows per block step\n";
      o << "  const uint32_t cg = threadIdx.x & (SL - 1u), slot = threadIdx.x >> LSL;\n";
      o << "  const uint32_t cvec = cb * SPAN + cg;\n";
      o << "  const uint32_t col0 = (cvec < VEC ? cvec : VEC - 1u) * V;  // clamped: loads stay in the row\n";
    };
    const auto at0 = coordFn("col0", "0u");
    auto colvecLoads = [&](const Ops& k, bool skipResults) {
      for (int t : k.colvecs) {
        if (skipResults && results.count(t)) continue;
        o << "  const auto cv" << t << " = tca::hip::load_vec<" << CType(g_.tensors[t].elem) << ", V>(t" << t << " + "
          << Offset(t, opOf[t]->axes, at0) << ");\n";
      }
      for (int t : k.outers)
        o << "  const " << CType(g_.tensors[t].elem) << " os" << t << " = t" << t << "["
          << Offset(t, opOf[t]->axes, at0) << "];\n";
    };

    // ---- partial folds of the chains `cs` (a whole nest of one pass, or
    // one pass of several)
    auto emitPart = [&](const std::string& name, const std::vector<int>& cs) {
      const Ops k = opsOf(cs);
      o << "template <uint32_t V>\n__device__ __forceinline__ void " << name << "(\n    " << sig << partSig << ") {\n";
      o << "  constexpr uint32_t W = " << kWaves << "u, RMIN = " << kRowsMin << "u, BLOCKS = " << kBlocks
        << "u, SPAN = " << kSpan << "u, LSPAN = " << kLogSpan << "u;  // SPAN column vectors per block\n";
      o << "  const uint32_t C = " << ExtentExpr(g_, geo.c) << ", R = " << ExtentExpr(g_, geo.r) << ";\n";
      o << "  const uint32_t NOUT = " << ProductExpr(geo.outer) << ";\n";
      o << "  const uint32_t VEC = C / V, CB = tca::hip::ceil_div(VEC, SPAN), NCB = NOUT * CB;\n";
      o << "  const uint32_t P = tca::hip::col_split(R, NCB, RMIN, BLOCKS);\n";
      o << "  const uint32_t p = blockIdx.x / NCB, cbk = blockIdx.x - p * NCB;\n";
      o << "  const uint32_t ob = cbk / CB, cb = cbk - ob * CB;\n";
      blockGeom();
      o << "  const uint32_t r_lo = static_cast<uint32_t>(static_cast<uint64_t>(p) * R / P);\n";
      o << "  const uint32_t r_hi = static_cast<uint32_t>(static_cast<uint64_t>(p + 1u) * R / P);\n";
      outerCoords("  ", "ob");
      combs("  ", cs);
      colvecLoads(k, false);
      partDecls(cs);
      o << rowLoop(cs, k, "has");
      // Row slots meet in LDS: slot s holds rows r_lo + s + k STEP.
      for (int ci : cs) {
        const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
        o << "  __shared__ " << T << " red" << ci << "[W * 64u * V];\n";
        o << "  if (has) {\n#pragma unroll\n    for (uint32_t q = 0; q < V; ++q) red" << ci
          << "[slot * (SL * V) + cg * V + q] = part" << ci << "[q];\n  }\n";
      }
      o << "  __syncthreads();\n";
      o << "  const uint32_t nrow = r_hi - r_lo, nslot = nrow < STEP ? nrow : STEP;  // slots holding rows\n";
      o << "  if (slot == 0u && cvec < VEC) {  // the threads of slot 0 (threadIdx.x < SL) finish\n";
      o << "#pragma unroll\n    for (uint32_t q = 0; q < V; ++q) {\n";
      o << "      const uint32_t cq = cvec * V + q;  // this thread's output column (col0 + q)\n";
      o << "      (void)cq;\n";
      for (int ci : cs) {
        const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
        o << "      " << T << " acc" << ci << " = red" << ci << "[cg * V + q];\n";
        o << "      for (uint32_t s2 = 1u; s2 < nslot; ++s2) acc" << ci << " = comb" << ci << "(acc" << ci << ", red"
          << ci << "[s2 * (SL * V) + cg * V + q]);\n";
      }
      o << "      if (P == 1u) {\n";
      {
        std::ostringstream b;
        for (int ci : cs)
          finish(b, "        ", ci, "acc" + std::to_string(ci), "nslot > 0u", "cq",
                 [&](int t) { return "cv" + std::to_string(t) + "[q]"; });
        o << b.str();
      }
      o << "      } else {\n";
      for (int ci : cs)
        o << "        p" << ci << "[(static_cast<uint64_t>(p) * NCB + cbk) * (SPAN * V) + cg * V + q] = acc" << ci
          << ";\n";
      o << "      }\n    }\n  }\n}\n";
    };
    // ---- merge of the P chunks of the chains `cs`: a block takes 64
    // consecutive outputs, its 16 waves fold chunks w, w + 16, ... (4 loads
    // in flight, 64 outputs per load: one 256-byte segment), and the waves
    // meet in LDS.
    auto emitMerge = [&](const std::string& name, const std::vector<int>& cs) {
      const Ops k = opsOf(cs);
      o << "template <uint32_t V>\n__device__ __forceinline__ void " << name << "(\n    " << sig << partSig << ") {\n";
      o << "  constexpr uint32_t RMIN = " << kRowsMin << "u, BLOCKS = " << kBlocks << "u, MW = " << kMergeWaves
        << "u, SPAN = " << kSpan << "u;\n";
      o << "  const uint32_t C = " << ExtentExpr(g_, geo.c) << ", R = " << ExtentExpr(g_, geo.r) << ";\n";
      o << "  const uint32_t NOUT = " << ProductExpr(geo.outer) << ";\n";
      o << "  const uint32_t VEC = C / V, CB = tca::hip::ceil_div(VEC, SPAN), NCB = NOUT * CB;\n";
      o << "  const uint32_t P = tca::hip::col_split(R, NCB, RMIN, BLOCKS);  // > 1: launched only then\n";
      o << "  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;\n";
      o << "  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 64u + lane;\n";
      o << "  const bool active = i < static_cast<uint64_t>(NOUT) * C;\n";
      o << "  const uint64_t ic = active ? i : 0u;  // lanes past the end read output 0 and store nothing\n";
      o << "  const uint32_t ob = static_cast<uint32_t>(ic / C), cq = static_cast<uint32_t>(ic - static_cast<uint64_t>(ob) * C);\n";
      o << "  const uint32_t cb = cq / (SPAN * V), within = cq - cb * (SPAN * V), cbk = ob * CB + cb;\n";
      o << "  const uint64_t stride = static_cast<uint64_t>(NCB) * (SPAN * V);\n";
      o << "  const uint64_t base = static_cast<uint64_t>(cbk) * (SPAN * V) + within;\n";
      outerCoords("  ", "ob");
      combs("  ", cs);
      const auto atq = coordFn("cq", "0u");
      for (int t : k.outers)
        o << "  const " << CType(g_.tensors[t].elem) << " os" << t << " = t" << t << "["
          << Offset(t, opOf[t]->axes, atq) << "];\n";
      for (int ci : cs) {
        const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
        const std::string A = "acc" + std::to_string(ci), pp = "p" + std::to_string(ci);
        o << "  " << T << " " << A << " = " << T << "(0);\n";
        o << "  if (w < P) {\n";
        o << "    " << A << " = " << pp << "[static_cast<uint64_t>(w) * stride + base];\n";
        o << "    uint32_t k = w + MW;\n";
        o << "    for (; k + 3u * MW < P; k += 4u * MW) {\n";
        for (int u = 0; u < 4; ++u)
          o << "      const " << T << " m" << u << " = " << pp << "[static_cast<uint64_t>(k + " << u
            << "u * MW) * stride + base];\n";
        for (int u = 0; u < 4; ++u) o << "      " << A << " = comb" << ci << "(" << A << ", m" << u << ");\n";
        o << "    }\n";
        o << "    for (; k < P; k += MW) " << A << " = comb" << ci << "(" << A << ", " << pp
          << "[static_cast<uint64_t>(k) * stride + base]);\n";
        o << "  }\n";
        o << "  __shared__ " << T << " mred" << ci << "[MW * 64u];\n";
        o << "  if (w < P) mred" << ci << "[w * 64u + lane] = " << A << ";\n";
      }
      o << "  __syncthreads();\n";
      o << "  if (w != 0u || !active) return;\n";
      o << "  const uint32_t nw = P < MW ? P : MW;  // waves holding chunks (every one of them holds >= 1)\n";
      std::ostringstream b;
      for (int ci : cs) {
        const std::string A = "acc" + std::to_string(ci);
        b << "  for (uint32_t s2 = 1u; s2 < nw; ++s2) " << A << " = comb" << ci << "(" << A << ", mred" << ci
          << "[s2 * 64u + lane]);\n";
        finish(b, "  ", ci, A, "true", "cq", [&](int t) {
          return "t" + std::to_string(t) + "[" + Offset(t, opOf[t]->axes, atq) + "]";
        });
      }
      o << b.str();
      o << "}\n";
    };
    // ---- every pass of a nest in one block over all rows (P = 1)
    auto emitWhole = [&](const std::string& name) {
      o << "template <uint32_t V>\n__device__ __forceinline__ void " << name << "(\n    " << sig << partSig << ") {\n";
      o << "  constexpr uint32_t W = " << kWaves << "u, SPAN = " << kSpan << "u, LSPAN = " << kLogSpan
        << "u;  // SPAN column vectors per block\n";
      o << "  const uint32_t C = " << ExtentExpr(g_, geo.c) << ", R = " << ExtentExpr(g_, geo.r) << ";\n";
      o << "  const uint32_t VEC = C / V, CB = tca::hip::ceil_div(VEC, SPAN);\n";
      o << "  const uint32_t cbk = blockIdx.x;  // SPAN column vectors of one outer index, every row\n";
      o << "  const uint32_t ob = cbk / CB, cb = cbk - ob * CB;\n";
      blockGeom();
      o << "  const uint32_t r_lo = 0u, r_hi = R;\n";
      o << "  const uint32_t nslot = R < STEP ? R : STEP;  // slots holding rows\n";
      outerCoords("  ", "ob");
      combs("  ", n.chains);
      colvecLoads(all, true);
      // Results a later pass reads: the finishing threads hand each to the
      // block through LDS, converted to the result's element type as a
      // store and load would.
      for (int t : readLater) {
        const std::string E = CType(g_.tensors[t].elem);
        o << "  __shared__ " << E << " bc" << t << "[64u * V];\n";
        o << "  " << E << " cv" << t << "[V];\n";
      }
      // The row slots of each pass meet in one LDS area, reused by the next
      // pass after a barrier.
      size_t area = 0;
      std::vector<std::map<int, size_t>> at(geo.passes);
      for (int ps = 0; ps < geo.passes; ++ps) {
        size_t off = 0;
        for (int ci : passChains[ps]) {
          at[ps][ci] = off;
          off += (ir::ElemBytes(g_.exprs[g_.chains[ci].root.fn.body].type) * kWaves * 64 * vmax + 15) / 16 * 16;
        }
        area = std::max(area, off);
      }
      o << "  __shared__ __attribute__((aligned(16))) unsigned char lds[" << area << "];\n";
      o << "  (void)lds;\n";
      for (int ps = 0; ps < geo.passes; ++ps) {
        const std::vector<int>& cs = passChains[ps];
        const Ops k = opsOf(cs);
        o << "  {  // pass " << ps + 1 << " of " << geo.passes << ": statements";
        for (int ci : cs) o << " #" << ci;
        o << "\n";
        partDecls(cs);
        o << rowLoop(cs, k, "has");
        for (int ci : cs) {
          const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
          o << "  " << T << "* red" << ci << " = reinterpret_cast<" << T << "*>(lds + " << at[ps][ci] << "u);\n";
          o << "  if (has) {\n#pragma unroll\n    for (uint32_t q = 0; q < V; ++q) red" << ci
            << "[slot * (SL * V) + cg * V + q] = part" << ci << "[q];\n  }\n";
        }
        o << "  __syncthreads();\n";
        o << "  if (slot == 0u && cvec < VEC) {  // the threads of slot 0 (threadIdx.x < SL) finish\n";
        o << "#pragma unroll\n    for (uint32_t q = 0; q < V; ++q) {\n";
        o << "      const uint32_t cq = cvec * V + q;  // this thread's output column (col0 + q)\n";
        o << "      (void)cq;\n";
        std::ostringstream b;
        for (int ci : cs) {
          const std::string T = CType(g_.exprs[g_.chains[ci].root.fn.body].type);
          b << "      " << T << " acc" << ci << " = red" << ci << "[cg * V + q];\n";
          b << "      for (uint32_t s2 = 1u; s2 < nslot; ++s2) acc" << ci << " = comb" << ci << "(acc" << ci << ", red"
            << ci << "[s2 * (SL * V) + cg * V + q]);\n";
          const int st = g_.chains[ci].store_tensor;
          finish(b, "      ", ci, "acc" + std::to_string(ci), "nslot > 0u", "cq",
                 [&](int t) { return "cv" + std::to_string(t) + "[q]"; }, !internalLocal(st),
                 readLater.count(st) ? "bc" + std::to_string(st) + "[cg * V + q]" : std::string());
        }
        o << b.str();
        o << "    }\n  }\n";
        if (ps + 1 < geo.passes)
          o << "  __syncthreads();  // the partials are read and the handed results written\n";
        for (int ci : cs) {
          const int st = g_.chains[ci].store_tensor;
          if (readLater.count(st))
            o << "#pragma unroll\n  for (uint32_t q = 0; q < V; ++q) cv" << st << "[q] = bc" << st << "[cg * V + q];\n";
        }
        o << "  }\n";
      }
      o << "}\n";
    };

    // ---- a mean and its centred sum of squares in one read (chan): the
    // partial keeps per thread the sum S of chain A's values (folded row by
    // row, as the unfused pass folds it) and M2, the sum of squares about the
    // mean of the rows folded so far, updated per group of rows held in
    // registers (tca::hip::chan_merge's formula); row slots and chunks merge
    // the same way, in slot and chunk order, and the finish takes
    // m = A's result and B's sum as M2 + n (S / n - m)^2.
    const int chA = chan ? passChains[0][0] : -1, chB = chan ? passChains[1][0] : -1;
    auto chanLoop = [&](const Ops& k) {
      std::ostringstream b;
      const ir::Chain& A = g_.chains[chA];
      const std::string SA = "part" + std::to_string(chA);
      auto group = [&](const std::string& ind, uint32_t rows, bool clamped, bool first) {
        groupLoads(b, k, ind, rows, clamped);
        if (clamped) {
          b << ind << "const float nu = 1.0f";
          for (uint32_t u = 1; u < rows; ++u) b << " + (ok_" << u << " ? 1.0f : 0.0f)";
          b << ";  // rows of this group\n" << ind << "const float rnu = 1.0f / nu;\n";
        } else {
          b << ind << "constexpr float nu = " << rows << ".0f, rnu = 1.0f / nu;\n";
        }
        if (!first) b << ind << "const float rcn = 1.0f / cn, wgt = cn * nu / (cn + nu);\n";
        b << "#pragma unroll\n" << ind << "for (uint32_t q = 0; q < V; ++q) {\n";
        for (uint32_t u = 0; u < rows; ++u) {
          ExprGen eg(g_, b, ind + "  ", &counter_);
          for (size_t j = 0; j < A.root.ops.size(); ++j) {
            const int t = A.root.ops[j].tensor;
            std::string v;
            switch (kindOf(t)) {
              case ColKind::Tile: v = "x" + std::to_string(t) + "_" + std::to_string(u) + "[q]"; break;
              case ColKind::ColVec: v = "cv" + std::to_string(t) + "[q]"; break;
              case ColKind::RowVec: v = "rv" + std::to_string(t) + "_" + std::to_string(u); break;
              default: v = "os" + std::to_string(t); break;
            }
            eg.Bind(A.root.fn.params[j], v);
          }
          const std::string ev = eg.Gen(A.root.fn.body);
          b << ind << "  const float e" << u << " = " << ev << ";\n";
        }
        b << ind << "  float gs = e0;  // the group's sum, mean and centred sum of squares\n";
        for (uint32_t u = 1; u < rows; ++u)
          b << ind << "  gs = " << (clamped ? "ok_" + std::to_string(u) + " ? gs + e" + std::to_string(u) + " : gs"
                                            : "gs + e" + std::to_string(u))
            << ";\n";
        b << ind << "  const float gm = gs * rnu;\n";
        b << ind << "  float g2 = (e0 - gm) * (e0 - gm);\n";
        for (uint32_t u = 1; u < rows; ++u) {
          b << ind << "  { const float d = e" << u << " - gm; g2 = ";
          if (clamped) b << "ok_" << u << " ? fmaf(d, d, g2) : g2; }\n";
          else b << "fmaf(d, d, g2); }\n";
        }
        if (first) {
          b << ind << "  m2[q] = g2;\n";
        } else {
          b << ind << "  const float dl = gm - " << SA << "[q] * rcn;  // the group's mean less the running mean\n";
          b << ind << "  m2[q] += g2 + dl * dl * wgt;\n";
        }
        for (uint32_t u = 0; u < rows; ++u) {
          const std::string e = "e" + std::to_string(u);
          if (first && u == 0) b << ind << "  " << SA << "[q] = e0;\n";
          else if (clamped && u > 0)
            b << ind << "  " << SA << "[q] = ok_" << u << " ? comb" << chA << "(" << SA << "[q], " << e << ") : " << SA
              << "[q];\n";
          else b << ind << "  " << SA << "[q] = comb" << chA << "(" << SA << "[q], " << e << ");\n";
        }
        b << ind << "}\n" << ind << "cn += nu;\n";
      };
      b << "  float cn = 0.0f;  // rows this thread folded\n";
      rowSkeleton(b, "has", group);
      b << "  (void)cn;\n";
      return b.str();
    };
    // The finish of a fused pair from (S, M2, n) in acc<A>, m2a, na.
    auto chanFinish = [&](std::ostringstream& b, const std::string& ind, const std::string& present,
                          const std::function<std::string(int)>& colval) {
      const int sa = g_.chains[chA].store_tensor;
      b << ind << "float mv = 0.0f;  // chain A's result, as chain B reads it\n";
      finish(b, ind, chA, "acc" + std::to_string(chA), present, "cq", colval, !internalLocal(sa), "mv");
      b << ind << "const float dm = acc" << chA << " * (1.0f / na) - mv;\n";
      b << ind << "const float tot = m2a + na * dm * dm;  // the sum over the rows of (t - m)^2\n";
      finish(b, ind, chB, "tot", present, "cq", colval);
    };
    auto emitChanPart = [&](const std::string& name) {
      const Ops k = opsOf(n.chains);
      const std::string SA = "part" + std::to_string(chA);
      o << "template <uint32_t V>\n__device__ __forceinline__ void " << name << "(\n    " << sig << partSig << ") {\n";
      o << "  constexpr uint32_t W = " << kWaves << "u, RMIN = " << kRowsMin << "u, BLOCKS = " << kBlocks
        << "u, SPAN = " << kSpan << "u, LSPAN = " << kLogSpan << "u;  // SPAN column vectors per block\n";
      o << "  const uint32_t C = " << ExtentExpr(g_, geo.c) << ", R = " << ExtentExpr(g_, geo.r) << ";\n";
      o << "  const uint32_t NOUT = " << ProductExpr(geo.outer) << ";\n";
      o << "  const uint32_t VEC = C / V, CB = tca::hip::ceil_div(VEC, SPAN), NCB = NOUT * CB;\n";
      o << "  const uint32_t P = tca::hip::col_split(R, NCB, RMIN, BLOCKS);\n";
      o << "  const uint32_t p = blockIdx.x / NCB, cbk = blockIdx.x - p * NCB;\n";
      o << "  const uint32_t ob = cbk / CB, cb = cbk - ob * CB;\n";
      blockGeom();
      o << "  const uint32_t r_lo = static_cast<uint32_t>(static_cast<uint64_t>(p) * R / P);\n";
      o << "  const uint32_t r_hi = static_cast<uint32_t>(static_cast<uint64_t>(p + 1u) * R / P);\n";
      outerCoords("  ", "ob");
      combs("  ", {chA});
      colvecLoads(k, true);
      partDecls({chA});
      o << "  float m2[V];\n#pragma unroll\n  for (uint32_t q = 0; q < V; ++q) m2[q] = 0.0f;\n";
      o << chanLoop(k);
      o << "  __shared__ float red" << chA << "[W * 64u * V], red" << chB << "[W * 64u * V];\n";
      o << "  if (has) {\n#pragma unroll\n    for (uint32_t q = 0; q < V; ++q) {\n";
      o << "      red" << chA << "[slot * (SL * V) + cg * V + q] = " << SA << "[q];\n";
      o << "      red" << chB << "[slot * (SL * V) + cg * V + q] = m2[q];\n    }\n  }\n";
      o << "  __syncthreads();\n";
      o << "  const uint32_t nrow = r_hi - r_lo, nslot = nrow < STEP ? nrow : STEP;  // slots holding rows\n";
      o << "  if (slot == 0u && cvec < VEC) {  // the threads of slot 0 (threadIdx.x < SL) finish\n";
      o << "#pragma unroll\n    for (uint32_t q = 0; q < V; ++q) {\n";
      o << "      const uint32_t cq = cvec * V + q;  // this thread's output column (col0 + q)\n";
      o << "      (void)cq;\n";
      o << "      float acc" << chA << " = red" << chA << "[cg * V + q], m2a = red" << chB << "[cg * V + q];\n";
      o << "      float na = nslot > 0u ? static_cast<float>((nrow - 1u) / STEP + 1u) : 0.0f;  // slot 0's rows\n";
      o << "      for (uint32_t s2 = 1u; s2 < nslot; ++s2)\n";
      o << "        tca::hip::chan_merge(acc" << chA << ", m2a, na, red" << chA << "[s2 * (SL * V) + cg * V + q], red" << chB
        << "[s2 * (SL * V) + cg * V + q], static_cast<float>((nrow - s2 - 1u) / STEP + 1u));\n";
      o << "      if (P == 1u) {\n";
      {
        std::ostringstream b;
        chanFinish(b, "        ", "nslot > 0u", [&](int t) { return "cv" + std::to_string(t) + "[q]"; });
        o << b.str();
      }
      o << "      } else {\n";
      o << "        const uint64_t at = (static_cast<uint64_t>(p) * NCB + cbk) * (SPAN * V) + cg * V + q;\n";
      o << "        p" << chA << "[at] = acc" << chA << ";\n        p" << chB << "[at] = m2a;\n";
      o << "      }\n    }\n  }\n}\n";
    };
    // Merge: as emitMerge, folding (S, M2, n) of the chunks with chan_merge.
    auto emitChanMerge = [&](const std::string& name) {
      const Ops k = opsOf(n.chains);
      const std::string A = "acc" + std::to_string(chA), pa = "p" + std::to_string(chA), pb = "p" + std::to_string(chB);
      o << "template <uint32_t V>\n__device__ __forceinline__ void " << name << "(\n    " << sig << partSig << ") {\n";
      o << "  constexpr uint32_t RMIN = " << kRowsMin << "u, BLOCKS = " << kBlocks << "u, MW = " << kMergeWaves
        << "u, SPAN = " << kSpan << "u;\n";
      o << "  const uint32_t C = " << ExtentExpr(g_, geo.c) << ", R = " << ExtentExpr(g_, geo.r) << ";\n";
      o << "  const uint32_t NOUT = " << ProductExpr(geo.outer) << ";\n";
      o << "  const uint32_t VEC = C / V, CB = tca::hip::ceil_div(VEC, SPAN), NCB = NOUT * CB;\n";
      o << "  const uint32_t P = tca::hip::col_split(R, NCB, RMIN, BLOCKS);  // > 1: launched only then\n";
      o << "  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;\n";
      o << "  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * 64u + lane;\n";
      o << "  const bool active = i < static_cast<uint64_t>(NOUT) * C;\n";
      o << "  const uint64_t ic = active ? i : 0u;  // lanes past the end read output 0 and store nothing\n";
      o << "  const uint32_t ob = static_cast<uint32_t>(ic / C), cq = static_cast<uint32_t>(ic - static_cast<uint64_t>(ob) * C);\n";
      o << "  const uint32_t cb = cq / (SPAN * V), within = cq - cb * (SPAN * V), cbk = ob * CB + cb;\n";
      o << "  const uint64_t stride = static_cast<uint64_t>(NCB) * (SPAN * V);\n";
      o << "  const uint64_t base = static_cast<uint64_t>(cbk) * (SPAN * V) + within;\n";
      o << "  // rows of chunk c: [c R / P, (c + 1) R / P)\n";
      o << "  const auto rows = [&](uint32_t c) {\n";
      o << "    return static_cast<float>(static_cast<uint32_t>(static_cast<uint64_t>(c + 1u) * R / P - "
           "static_cast<uint64_t>(c) * R / P));\n  };\n";
      outerCoords("  ", "ob");
      const auto atq = coordFn("cq", "0u");
      for (int t : k.outers)
        o << "  const " << CType(g_.tensors[t].elem) << " os" << t << " = t" << t << "["
          << Offset(t, opOf[t]->axes, atq) << "];\n";
      o << "  float " << A << " = 0.0f, m2a = 0.0f, na = 0.0f;\n";
      o << "  if (w < P) {\n";
      o << "    " << A << " = " << pa << "[static_cast<uint64_t>(w) * stride + base];\n";
      o << "    m2a = " << pb << "[static_cast<uint64_t>(w) * stride + base];\n";
      o << "    na = rows(w);\n";
      o << "    uint32_t k = w + MW;\n";
      o << "    for (; k + 3u * MW < P; k += 4u * MW) {\n";
      for (int u = 0; u < 4; ++u)
        o << "      const float cs" << u << " = " << pa << "[static_cast<uint64_t>(k + " << u << "u * MW) * stride + base], cm"
          << u << " = " << pb << "[static_cast<uint64_t>(k + " << u << "u * MW) * stride + base];\n";
      for (int u = 0; u < 4; ++u)
        o << "      tca::hip::chan_merge(" << A << ", m2a, na, cs" << u << ", cm" << u << ", rows(k + " << u << "u * MW));\n";
      o << "    }\n";
      o << "    for (; k < P; k += MW)\n      tca::hip::chan_merge(" << A << ", m2a, na, " << pa
        << "[static_cast<uint64_t>(k) * stride + base], " << pb << "[static_cast<uint64_t>(k) * stride + base], rows(k));\n";
      o << "  }\n";
      o << "  __shared__ float mredS[MW * 64u], mredM[MW * 64u], mredN[MW];\n";
      o << "  if (w < P) {\n    mredS[w * 64u + lane] = " << A << ";\n    mredM[w * 64u + lane] = m2a;\n";
      o << "    if (lane == 0u) mredN[w] = na;\n  }\n";
      o << "  __syncthreads();\n";
      o << "  if (w != 0u || !active) return;\n";
      o << "  const uint32_t nw = P < MW ? P : MW;  // waves holding chunks (every one of them holds >= 1)\n";
      o << "  for (uint32_t s2 = 1u; s2 < nw; ++s2)\n";
      o << "    tca::hip::chan_merge(" << A << ", m2a, na, mredS[s2 * 64u + lane], mredM[s2 * 64u + lane], mredN[s2]);\n";
      std::ostringstream b;
      chanFinish(b, "  ", "true", [&](int t) {
        return "t" + std::to_string(t) + "[" + Offset(t, opOf[t]->axes, atq) + "]";
      });
      o << b.str();
      o << "}\n";
    };

    o << "// statements";
    for (int ci : n.chains) o << " #" << ci;
    o << ": column family; reduce over @" << g_.dims[geo.r].name << " (not contiguous) per column of @"
      << g_.dims[geo.c].name;
    if (geo.passes > 1) o << " in " << geo.passes << " passes";
    if (chan) o << ", fused into one read (a mean and its centred sum of squares)";
    o << "\n";
    if (geo.passes == 1) {
      emitPart(sym + "_part", n.chains);
      emitMerge(sym + "_merge", n.chains);
    } else if (chan) {
      emitChanPart(sym + "_chanpart");
      emitChanMerge(sym + "_chanmerge");
    } else {
      emitWhole(sym + "_whole");
      for (int ps = 0; ps < geo.passes; ++ps) {
        emitPart(sym + "_part" + std::to_string(ps + 1), passChains[ps]);
        emitMerge(sym + "_merge" + std::to_string(ps + 1), passChains[ps]);
      }
    }
    // ---- the kernels of each vector width
    const std::string args = CallArgs(n);
    const std::string cdim = g_.dims[geo.c].name, rdim = g_.dims[geo.r].name;
    struct Width {
      uint32_t v, mod, rem;
    };
    std::vector<Width> widths;
    {
      widths.push_back({vmax, vmax, 0});
      for (uint32_t v = vmax / 2; v >= 1; v /= 2) widths.push_back({v, 2 * v, v});
      const uint64_t ext = g_.dims[geo.c].extent;
      if (ext > 0) {  // a compile-time row length: only its width
        std::vector<Width> one;
        for (const auto& w : widths)
          if (ext % w.mod == w.rem) one.push_back(w);
        widths = one;
      }
    }
    const std::string outerTerm = DimProduct(geo.outer) + "/1";
    const std::string outTerm = DimProduct([&] {
      std::vector<int> a(geo.outer);
      a.push_back(geo.c);
      return a;
    }()) + "/64";
    for (const auto& wd : widths) {
      const std::string cbTerm = cdim + "/" + std::to_string(kSpan * wd.v);
      const std::string splitRec = rdim + " " + std::to_string(kRowsMin) + " " + std::to_string(kBlocks);
      // (symbol suffix, device function, split mode, merge-shaped, chains, what it does)
      struct K {
        std::string suffix, fn;
        int mode;
        bool merge;
        std::vector<int> chains;
        std::string what;
      };
      std::vector<K> ks;
      const std::string v = std::to_string(wd.v);
      if (geo.passes == 1) {
        ks.push_back({"_p" + v, "_part", 0, false, n.chains,
                      " partial: " + std::to_string(kSpan) + " column vectors x a chunk of rows per block, P = col_split"});
        ks.push_back({"_m" + v, "_merge", 1, true, n.chains,
                      " merge: 64 outputs per block, 16 waves over the P chunks (P > 1 only)"});
      } else if (chan) {
        ks.push_back({"_p" + v, "_chanpart", 0, false, n.chains,
                      " mean and centred sum of squares in one read: " + std::to_string(kSpan) +
                          " column vectors x a chunk of rows per block, P = col_split"});
        ks.push_back({"_m" + v, "_chanmerge", 1, true, n.chains,
                      " merge of (sum, centred sum of squares, rows): 64 outputs per block, 16 waves over the P chunks "
                      "(P > 1 only)"});
      } else {
        ks.push_back({"_w" + v, "_whole", 2, false, n.chains,
                      " whole: every pass over all rows of " + std::to_string(kSpan) + " column vectors per block, results handed on in LDS "
                      "(P == 1 only)"});
        for (int ps = 0; ps < geo.passes; ++ps) {
          const std::string pn = std::to_string(ps + 1);
          ks.push_back({"_p" + v + "_" + pn, "_part" + pn, 3, false, passChains[ps],
                        " pass " + pn + " partial: " + std::to_string(kSpan) + " column vectors x a chunk of rows per block (P > 1 only)"});
          ks.push_back({"_m" + v + "_" + pn, "_merge" + pn, 1, true, passChains[ps],
                        " pass " + pn + " merge: 64 outputs per block, 16 waves over the P chunks (P > 1 only)"});
        }
      }
      for (const auto& kd : ks) {
        PlanKernel k = pk;
        k.symbol = sym + kd.suffix;
        k.block = kd.merge ? 64 * kMergeWaves : 256;
        for (const auto& nm : partNames) k.args.push_back("ptr " + nm);
        if (kd.merge) {
          k.grid.push_back(outTerm);
        } else {
          k.grid.push_back(outerTerm);
          k.grid.push_back(cbTerm);
        }
        k.split = splitRec + " " + std::to_string(kd.mode) + " 2 " + outerTerm + " " + cbTerm;
        if (g_.dims[geo.c].extent == 0)
          k.when.push_back(cdim + " 0 4294967295 " + std::to_string(wd.mod) + " " + std::to_string(wd.rem));
        o << "extern \"C\" __global__ void __launch_bounds__(" << k.block << ") " << k.symbol << "(\n    " << sig
          << partSig << ") {\n  " << sym << kd.fn << "<" << wd.v << "u>(" << args << partArgs << ");\n}\n";
        std::ostringstream det;
        det << "reduce @" << rdim << " per column of @" << cdim << " vec=" << wd.v
            << (g_.dims[geo.c].extent == 0 ? " (" + cdim + " % " + std::to_string(wd.mod) + " == " +
                                                  std::to_string(wd.rem) + ")"
                                            : std::string())
            << kd.what;
        AddKernel(k, Family::Col, kd.chains, det.str());
      }
    }
    o << "\n";
    return true;
  }

  // Seg: a chained reduction folded in one kernel. One 256-thread block per
  // segment s (an output of the outer reduction) runs the rows r of the
  // segment in steps of 2 RS rows (each slot two rows, RS apart), RS = 256 /
  // SL, SL = the smallest power of two with 4 SL >= the row's vectors (at
  // most 64: longer rows loop), each lane's vectors in groups of 4: 8 loads
  // in flight per lane before a fold. A row's lanes fold their vectors with the inner
  // combiner (every lane holds >= 1 vector of a non-empty row), meet by
  // shuffles, and apply the inner init once: the value the local L would
  // hold. Lane 0 of the row maps it (the outer chain's root map) and folds
  // it into its slot's outer partial; the slots meet in LDS, and thread 0
  // applies the outer init and piped map and stores. L is never stored. The
  // row loop is uniform over the block (rows past the segment's end read
  // its last row and fold nothing), so every shuffle runs with the whole
  // wave. One kernel per vector width, chosen at launch by guards on the
  // row length.
  bool EmitSeg(int ni, std::string* err) {
    (void)err;
    const Nest& in = an_.nests[ni];
    const Nest& outn = an_.nests[ni + 1];
    const int ci = in.chains[0], cj = outn.chains[0];
    const ir::Chain& a = g_.chains[ci];
    const ir::Chain& b = g_.chains[cj];
    const int L = a.store_tensor;
    RowGeom geo;
    RowShape(g_, {ci}, true, &geo);
    const std::vector<int> S(geo.outer.begin(), geo.outer.end() - 1);
    const int raxis = geo.outer.back(), caxis = geo.col;
    Nest both;
    both.chains = {ci, cj};
    PlanKernel pk;
    pk.symbol = Sym(g_, prefix_, ni);
    const std::string sig = Signature(both, &pk);
    const std::string args = CallArgs(both);
    const std::string sym = pk.symbol;
    const uint32_t vmax = RowVecMax(g_, {ci}, geo);
    std::ostringstream& o = src_;
    const std::string Tin = CType(g_.exprs[a.root.fn.body].type);
    const std::string Tout = CType(g_.exprs[b.root.fn.body].type);
    auto coord = [&](const std::string& col) {
      return [&, col](int x) -> std::string {
        if (x == caxis) return col;
        return "c" + std::to_string(x);
      };
    };
    // Operands of the inner map: row tiles and column vectors per vector,
    // row scalars per row (r among their axes) or per segment.
    std::vector<int> tiles, cols, rowsc, segsc;
    auto note = [](std::vector<int>& v, int t) {
      if (std::find(v.begin(), v.end(), t) == v.end()) v.push_back(t);
    };
    std::map<int, const ir::Operand*> opOf;
    for (const auto& op : a.root.ops) {
      opOf[op.tensor] = &op;
      switch (Classify(op, geo)) {
        case OpKind::RowTile: note(tiles, op.tensor); break;
        case OpKind::ColVec: note(cols, op.tensor); break;
        default:
          if (std::find(op.axes.begin(), op.axes.end(), raxis) != op.axes.end()) note(rowsc, op.tensor);
          else note(segsc, op.tensor);
          break;
      }
    }
    std::vector<const ir::Operand*> outerOps;
    for (const auto& op : b.root.ops)
      if (op.tensor != L) outerOps.push_back(&op);
    if (b.has_piped)
      for (const auto& op : b.piped.ops) outerOps.push_back(&op);
    for (const ir::Operand* op : outerOps)
      if (!opOf.count(op->tensor)) {
        opOf[op->tensor] = op;
        note(segsc, op->tensor);
      }

    o << "// statements #" << ci << " and #" << cj << ": segment family; reduce @" << g_.dims[caxis].name
      << " per row, then @" << g_.dims[raxis].name << " per segment, in one kernel\n";
    o << "template <uint32_t V>\n__device__ __forceinline__ void " << sym << "_seg(\n    " << sig << ") {\n";
    o << "  const uint32_t C = " << ExtentExpr(g_, caxis) << ", R = " << ExtentExpr(g_, raxis) << ";\n";
    o << "  const uint32_t VEC = C / V;\n";
    o << "  uint32_t LSL = 0u;  // SL = 2^LSL lanes per row: the smallest power of two with 4 SL >= VEC, <= 64\n";
    o << "  while (LSL < 6u && (4u << LSL) < VEC) ++LSL;\n";
    o << "  const uint32_t SL = 1u << LSL, RS = 256u >> LSL;  // RS rows per block step\n";
    o << "  const uint32_t cg = threadIdx.x & (SL - 1u), slot = threadIdx.x >> LSL;\n";
    o << "  const uint32_t NV = tca::hip::ceil_div(VEC, SL);  // vectors of the longest lane share\n";
    o << "  uint32_t srem = blockIdx.x;  // this block's segment\n";
    for (int k = static_cast<int>(S.size()) - 1; k >= 0; --k) {
      const int x = S[k];
      if (k == 0)
        o << "  const uint32_t c" << x << " = srem;\n";
      else
        o << "  const uint32_t c" << x << " = srem % " << ExtentExpr(g_, x) << "; srem /= " << ExtentExpr(g_, x)
          << ";\n";
    }
    o << "  (void)srem;\n";
    for (int cc : {ci, cj}) {
      const ir::Chain& c = g_.chains[cc];
      const std::string T = CType(g_.exprs[c.root.fn.body].type);
      o << "  const auto comb" << cc << " = [](" << T << " acc, " << T << " now) -> " << T << " {\n";
      ExprGen cg(g_, o, "    ", &counter_);
      cg.Bind(c.reduces[0].fn.params[0], "acc");
      cg.Bind(c.reduces[0].fn.params[1], "now");
      const std::string r = cg.Gen(c.reduces[0].fn.body);
      o << "    return " << r << ";\n  };\n";
    }
    const auto segAt = coord("0u");
    for (int t : segsc)
      o << "  const " << CType(g_.tensors[t].elem) << " os" << t << " = t" << t << "["
        << Offset(t, opOf[t]->axes, segAt) << "];\n";
    o << "  " << Tout << " oacc = " << Tout << "(0);\n  bool ohas = false;\n";
    // Two rows per slot and step (RS apart), each lane's vectors in groups
    // of 4 (the first group's vector 0 always owned, the rest clamped into
    // the row and predicated): 8 loads in flight per lane before any fold.
    constexpr int kRowsPerStep = 2;
    o << "  for (uint32_t rb = 0u; rb < R; rb += " << kRowsPerStep << "u * RS) {  // uniform over the block\n";
    for (int j = 0; j < kRowsPerStep; ++j) {
      const std::string js = std::to_string(j);
      o << "    const uint32_t r" << js << " = rb + " << js << "u * RS + slot;\n";
      o << "    const bool rok" << js << " = r" << js << " < R;\n";
      o << "    const uint32_t rr" << js << " = rok" << js << " ? r" << js
        << " : R - 1u;  // rows past the end read the last one\n";
    }
    auto rowCoord = [&](int j, const std::string& col) {
      return [&, j, col](int x) -> std::string {
        if (x == caxis) return col;
        if (x == raxis) return "rr" + std::to_string(j);
        return "c" + std::to_string(x);
      };
    };
    for (int j = 0; j < kRowsPerStep; ++j)
      for (int t : rowsc)
        o << "    const " << CType(g_.tensors[t].elem) << " rs" << t << "_" << j << " = t" << t << "["
          << Offset(t, opOf[t]->axes, rowCoord(j, "0u")) << "];\n";
    for (int j = 0; j < kRowsPerStep; ++j) o << "    " << Tin << " acc" << j << " = " << Tin << "(0);\n";
    // Loads of vector vc<u> of row j into x<t>_<j>_<u> / cv<t>_<u>; then the fold.
    auto loads = [&](std::ostringstream& bo, const std::string& ind, int j, const std::string& vv,
                     const std::string& sfx) {
      const auto at = rowCoord(j, vv + " * V");
      for (int t : tiles)
        bo << ind << "const auto x" << t << sfx << " = tca::hip::load_vec_nt<" << CType(g_.tensors[t].elem) << ", V>(t"
           << t << " + " << Offset(t, opOf[t]->axes, at) << ");\n";
    };
    auto colLoads = [&](std::ostringstream& bo, const std::string& ind, const std::string& vv, const std::string& sfx) {
      const auto at = rowCoord(0, vv + " * V");
      for (int t : cols)
        bo << ind << "const auto cv" << t << sfx << " = tca::hip::load_vec<" << CType(g_.tensors[t].elem) << ", V>(t"
           << t << " + " << Offset(t, opOf[t]->axes, at) << ");\n";
    };
    auto fold = [&](std::ostringstream& bo, const std::string& ind, int j, const std::string& u, bool first,
                    const std::string& ok) {
      const std::string acc = "acc" + std::to_string(j);
      bo << "#pragma unroll\n" << ind << "for (uint32_t q = 0; q < V; ++q) {\n";
      ExprGen eg(g_, bo, ind + "  ", &counter_);
      for (size_t k = 0; k < a.root.ops.size(); ++k) {
        const int t = a.root.ops[k].tensor;
        std::string v;
        if (std::find(tiles.begin(), tiles.end(), t) != tiles.end())
          v = "x" + std::to_string(t) + "_" + std::to_string(j) + "_" + u + "[q]";
        else if (std::find(cols.begin(), cols.end(), t) != cols.end()) v = "cv" + std::to_string(t) + "_" + u + "[q]";
        else if (std::find(rowsc.begin(), rowsc.end(), t) != rowsc.end())
          v = "rs" + std::to_string(t) + "_" + std::to_string(j);
        else v = "os" + std::to_string(t);
        eg.Bind(a.root.fn.params[k], v);
      }
      const std::string ev = eg.Gen(a.root.fn.body);
      const std::string fold1 = "comb" + std::to_string(ci) + "(" + acc + ", " + ev + ")";
      if (first) bo << ind << "  " << acc << " = q == 0u ? " << ev << " : " << fold1 << ";\n";
      else bo << ind << "  " << acc << " = " << ok << " ? " << fold1 << " : " << acc << ";\n";
      bo << ind << "}\n";
      if (FoldFenced(g_.exprs[a.root.fn.body].type)) bo << ind << "tca::hip::fold_fence(" << acc << ");\n";
    };
    {
      std::ostringstream bo;
      auto group = [&](const std::string& ind, bool first) {
        for (int u = 0; u < 4; ++u) {
          const std::string us = std::to_string(u);
          bo << ind << "const uint32_t vi" << us << " = cg + (k + " << us << "u) * SL;\n";
          bo << ind << "const bool ok" << us << " = vi" << us << " < VEC;\n";
          bo << ind << "const uint32_t vc" << us << " = ok" << us << " ? vi" << us << " : VEC - 1u;\n";
          colLoads(bo, ind, "vc" + us, "_" + us);
          for (int j = 0; j < kRowsPerStep; ++j) loads(bo, ind, j, "vc" + us, "_" + std::to_string(j) + "_" + us);
        }
        for (int j = 0; j < kRowsPerStep; ++j)
          for (int u = 0; u < 4; ++u) fold(bo, ind, j, std::to_string(u), first && u == 0, "ok" + std::to_string(u));
      };
      bo << "    if (VEC > 0u) {  // uniform; a lane's first vector cg < VEC (SL <= VEC)\n";
      bo << "      {\n        const uint32_t k = 0u;\n";
      group("        ", true);
      bo << "      }\n";
      bo << "      for (uint32_t k = 4u; k < NV; k += 4u) {\n";
      group("        ", false);
      bo << "      }\n    }\n";
      o << bo.str();
    }
    for (int j = 0; j < kRowsPerStep; ++j) {
      const std::string js = std::to_string(j);
      o << "    acc" << js << " = tca::hip::seg_allreduce_rt(acc" << js << ", SL, comb" << ci << ");\n";
    }
    for (int j = 0; j < kRowsPerStep; ++j) {
      const std::string js = std::to_string(j);
      std::ostringstream bo;
      ExprGen ig(g_, bo, "    ", &counter_);
      const std::string init = ig.Gen(a.reduces[0].init);
      bo << "    " << Tin << " rowv" << js << " = " << init << ";  // the value L holds for row r" << js << "\n";
      bo << "    if (VEC > 0u) {\n";
      ExprGen fg(g_, bo, "      ", &counter_);
      fg.Bind(a.reduces[0].fn.params[0], init);
      fg.Bind(a.reduces[0].fn.params[1], "acc" + js);
      const std::string rv = fg.Gen(a.reduces[0].fn.body);
      bo << "      rowv" << js << " = " << rv << ";\n    }\n";
      ExprGen mg(g_, bo, "    ", &counter_);
      for (size_t k = 0; k < b.root.ops.size(); ++k) {
        const int t = b.root.ops[k].tensor;
        mg.Bind(b.root.fn.params[k], t == L ? "rowv" + js : "os" + std::to_string(t));
      }
      const std::string m = mg.Gen(b.root.fn.body);
      bo << "    if (cg == 0u && rok" << js << ") {\n      oacc = ohas ? comb" << cj << "(oacc, " << m << ") : " << m
         << ";\n      ohas = true;\n    }\n";
      o << bo.str();
    }
    o << "  }\n";
    o << "  __shared__ " << Tout << " oslot[256];\n  __shared__ int hslot[256];\n";
    o << "  if (cg == 0u) {\n    oslot[slot] = oacc;\n    hslot[slot] = ohas ? 1 : 0;\n  }\n";
    o << "  __syncthreads();\n";
    o << "  if (threadIdx.x != 0u) return;\n";
    o << "  " << Tout << " a = " << Tout << "(0);\n  bool any = false;\n";
    o << "  for (uint32_t s2 = 0u; s2 < RS; ++s2)\n    if (hslot[s2]) {\n      a = any ? comb" << cj
      << "(a, oslot[s2]) : oslot[s2];\n      any = true;\n    }\n";
    {
      std::ostringstream bo;
      ExprGen ig(g_, bo, "  ", &counter_);
      const std::string init = ig.Gen(b.reduces[0].init);
      bo << "  " << Tout << " fin = " << init << ";\n  if (any) {\n";
      ExprGen fg(g_, bo, "    ", &counter_);
      fg.Bind(b.reduces[0].fn.params[0], init);
      fg.Bind(b.reduces[0].fn.params[1], "a");
      const std::string fv = fg.Gen(b.reduces[0].fn.body);
      bo << "    fin = " << fv << ";\n  }\n";
      std::string val = "fin";
      if (b.has_piped) {
        ExprGen pg(g_, bo, "  ", &counter_);
        pg.Bind(b.piped.fn.params[0], val);
        for (size_t k = 0; k < b.piped.ops.size(); ++k)
          pg.Bind(b.piped.fn.params[k + 1], "os" + std::to_string(b.piped.ops[k].tensor));
        val = pg.Gen(b.piped.fn.body);
      }
      const int st = b.store_tensor;
      bo << "  t" << st << "[" << Offset(st, b.store_axes, segAt) << "] = " << val << ";\n";
      o << bo.str();
    }
    o << "}\n";
    // One kernel per vector width.
    const std::string cdim = g_.dims[caxis].name;
    struct Width {
      uint32_t v, mod, rem;
    };
    std::vector<Width> widths;
    widths.push_back({vmax, vmax, 0});
    for (uint32_t v = vmax / 2; v >= 1; v /= 2) widths.push_back({v, 2 * v, v});
    const uint64_t ext = g_.dims[caxis].extent;
    if (ext > 0) {
      std::vector<Width> one;
      for (const auto& w : widths)
        if (ext % w.mod == w.rem) {
          one.push_back(w);
          break;
        }
      widths = one;
    }
    for (const auto& wd : widths) {
      PlanKernel k = pk;
      k.symbol = sym + "_g" + std::to_string(wd.v);
      k.block = 256;
      k.grid.push_back(DimProduct(S) + "/1");
      if (ext == 0) k.when.push_back(cdim + " 0 4294967295 " + std::to_string(wd.mod) + " " + std::to_string(wd.rem));
      if (!in.seg_guard.empty()) k.when.push_back(in.seg_guard + " " + std::to_string(kSegMin) + " 4294967295 1 0");
      o << "extern \"C\" __global__ void __launch_bounds__(256) " << k.symbol << "(\n    " << sig << ") {\n  " << sym
        << "_seg<" << wd.v << "u>(" << args << ");\n}\n";
      std::ostringstream det;
      det << "reduce @" << cdim << " per row then @" << g_.dims[raxis].name << " per segment, one block per segment vec="
          << wd.v
          << (ext == 0 ? " (" + cdim + " % " + std::to_string(wd.mod) + " == " + std::to_string(wd.rem) + ")"
                       : std::string())
          << (in.seg_guard.empty() ? std::string()
                                   : " (" + in.seg_guard + " >= " + std::to_string(kSegMin) + " segments)");
      AddKernel(k, Family::Seg, {ci, cj}, det.str());
    }
    o << "\n";
    return true;
  }

  bool EmitGemmNest(int ni, std::string* err) {
    const Nest& n = an_.nests[ni];
    const ir::Chain& c = g_.chains[n.chains[0]];
    GemmMatch m;
    if (!MatchGemm(g_, c, &m)) {
      *err = "emit: gemm family rejected a nest it classified";
      return false;
    }
    PlanKernel pk;
    pk.symbol = Sym(g_, prefix_, ni);
    Nest single = n;
    const std::string sig = Signature(single, &pk);
    GemmEmitted ge;
    if (!EmitGemm(g_, c, m, pk.symbol, sig, ni, opts_.allow_gemm_split, &counter_, &src_, &ge, err)) return false;
    for (const auto& d : ge.extra_dims) extra_dims_.push_back(d);
    for (const auto& t : ge.extra_tensors) extra_tensors_.push_back(t);
    for (const auto& gk : ge.kernels) {
      PlanKernel k = pk;
      k.symbol = pk.symbol + gk.suffix;
      k.block = gk.block;
      k.lds = gk.lds;
      k.grid = gk.grid;
      k.when = gk.when;
      k.unless = gk.unless;
      for (const auto& a : gk.extra_args) k.args.push_back(a);
      k.split = gk.split;
      AddKernel(k, Family::Gemm, n.chains, gk.detail);
    }
    return true;
  }

  void AddKernel(const PlanKernel& pk, Family f, const std::vector<int>& chains, const std::string& detail) {
    plan_kernels_.push_back(pk);
    KernelInfo ki;
    ki.symbol = pk.symbol;
    ki.family = f;
    ki.chains = chains;
    ki.detail = detail;
    kernels_.push_back(ki);
  }

  std::string PlanText() {
    std::ostringstream p;
    p << "tca-plan 1\nprogram " << g_.name << "\n";
    for (const auto& d : g_.dims) p << "dim " << d.name << " " << d.extent << "\n";
    for (const auto& d : extra_dims_) p << "dim " << d << "\n";
    for (size_t t = 0; t < g_.tensors.size(); ++t) {
      const ir::Tensor& tt = g_.tensors[t];
      std::string role;
      if (!tt.local) role = g_.IsStored(static_cast<int>(t)) ? "out" : "in";
      else if (an_.hbm_local[t]) role = "local";
      else continue;  // register-resident or dead local: not part of the plan
      p << "tensor " << tt.name << " " << ir::ElemName(tt.elem) << " " << role << " " << tt.dims.size();
      for (int d : tt.dims) p << " " << g_.dims[d].name;
      p << "\n";
    }
    for (const auto& t : extra_tensors_) p << "tensor " << t << "\n";
    for (const auto& s : g_.scalars) p << "scalar " << s.name << " " << ir::ElemName(s.elem) << "\n";
    for (const auto& k : plan_kernels_) {
      p << "kernel " << k.symbol << " " << k.block << " " << k.lds << " " << k.grid.size();
      for (const auto& t : k.grid) p << " " << t;
      p << "\n";
      for (const auto& a : k.args) p << "arg " << a << "\n";
      if (!k.pack.empty()) p << "pack " << k.pack << "\n";
      if (!k.split.empty()) p << "split " << k.split << "\n";
      for (const auto& w : k.when) p << "when " << w << "\n";
      for (const auto& w : k.unless) p << "unless " << w << "\n";
    }
    p << "end\n";
    return p.str();
  }

  const Graph& g_;
  Options opts_;
  std::string prefix_;
  Analysis an_;
  std::vector<std::string> extra_dims_;     // plan-only dims: "<name> <extent>"
  std::vector<std::string> extra_tensors_;  // plan-only HBM locals: "<name> <dtype> local <rank> <dims...>"
  std::ostringstream src_;
  std::vector<PlanKernel> plan_kernels_;
  std::vector<KernelInfo> kernels_;
  int counter_ = 0;
  bool uses_gemm_ = false;
};

}  // namespace

namespace {

// Chained reductions (MidChain.Reduce then AfterReduce.Reduce,
// pkg/chain.go:262 applied twice): a chain root -> reduce 1 -> reduce 2 ...
// -> piped -> store becomes root -> reduce 1 -> store L, then L -> identity
// -> reduce 2 ... -> store, L a local over the axes left after reduce 1.
// The fold is the same (reduce 1's init once per element of L, reduce 2's
// once per output); each half is a single-reduction chain the row,
// streaming, column and split-row families take, where the chained form
// could only fold one output per thread. Repeated until every chain has at
// most one reduction.
void SplitChainedReductions(ir::Graph* g) {
  for (size_t ci = 0; ci < g->chains.size(); ++ci) {
    if (g->chains[ci].reduces.size() < 2) continue;
    ir::Chain inner = g->chains[ci];
    ir::Chain outer = g->chains[ci];
    std::vector<int> axes = inner.root.as;  // live axes after reduce 1
    axes.pop_back();
    const ir::Elem elem = g->exprs[inner.reduces[0].fn.body].type;
    ir::Tensor t;
    t.name = "__chain" + std::to_string(ci);
    t.elem = elem;
    t.dims = axes;
    t.local = true;
    g->tensors.push_back(t);
    const int tl = static_cast<int>(g->tensors.size()) - 1;
    inner.reduces.resize(1);
    inner.has_piped = false;
    inner.piped = ir::MapStage();
    inner.store_tensor = tl;
    inner.store_axes = axes;
    ir::Expr param;
    param.op = ir::Op::Param;
    param.type = elem;
    param.index = 0;
    param.text = "v";
    g->exprs.push_back(param);
    const int pid = static_cast<int>(g->exprs.size()) - 1;
    outer.iters = axes;
    outer.root = ir::MapStage();
    outer.root.ops.push_back(ir::Operand{tl, axes});
    outer.root.fn.params = {pid};
    outer.root.fn.body = pid;
    outer.root.as = axes;
    outer.reduces.erase(outer.reduces.begin());
    g->chains[ci] = inner;
    g->chains.insert(g->chains.begin() + static_cast<long>(ci) + 1, outer);
  }
}

}  // namespace

bool Emit(const ir::Graph& g, const Options& opts, Result* out, std::string* err) {
  std::string verr;
  if (!ir::Verify(g, &verr)) {
    *err = verr;
    return false;
  }
  ir::Graph split = g;
  if (opts.allow_fused) SplitChainedReductions(&split);
  Emitter e(split, opts);
  return e.Run(out, err);
}

}  // namespace cg
}  // namespace tca
