// gemm_emit.cpp — see gemm_emit.h.
#include "gemm_emit.h"

#include <cmath>
#include <map>

namespace tca {
namespace cg {

using ir::BinOp;
using ir::Elem;
using ir::Op;

namespace {

// Body operand i is param p, or cast<f32>(param p) when the param is bf16 or f16.
bool IsParamOrCast(const ir::Graph& g, int id, int param, Elem* in) {
  const ir::Expr& e = g.exprs[id];
  if (id == param) {
    *in = e.type;
    return e.type == Elem::F32;
  }
  if (e.op == Op::Cast && e.type == Elem::F32 && e.args[0] == param) {
    *in = g.exprs[param].type;
    return *in == Elem::BF16 || *in == Elem::F16;
  }
  return false;
}

}  // namespace

bool MatchGemm(const ir::Graph& g, const ir::Chain& c, GemmMatch* m) {
  if (c.root.ops.size() != 2 || c.reduces.size() != 1) return false;
  if (c.root.as.size() != 3 && c.root.as.size() != 4) return false;
  const ir::ReduceStage& r = c.reduces[0];
  // init +0.0f
  const ir::Expr& init = g.exprs[r.init];
  if (init.op != Op::Const || init.type != Elem::F32 || init.value != 0.0 || std::signbit(init.value)) return false;
  // acc + now
  const ir::Expr& comb = g.exprs[r.fn.body];
  if (comb.op != Op::Bin || static_cast<BinOp>(comb.code) != BinOp::Add) return false;
  const int acc = r.fn.params[0], now = r.fn.params[1];
  if (!((comb.args[0] == acc && comb.args[1] == now) || (comb.args[0] == now && comb.args[1] == acc))) return false;
  // body: P0 * P1
  const ir::Expr& body = g.exprs[c.root.fn.body];
  if (body.op != Op::Bin || static_cast<BinOp>(body.code) != BinOp::Mul || body.type != Elem::F32) return false;
  const int p0 = c.root.fn.params[0], p1 = c.root.fn.params[1];
  Elem e0, e1;
  bool direct = IsParamOrCast(g, body.args[0], p0, &e0) && IsParamOrCast(g, body.args[1], p1, &e1);
  bool swapped = IsParamOrCast(g, body.args[0], p1, &e1) && IsParamOrCast(g, body.args[1], p0, &e0);
  if (!direct && !swapped) return false;
  if (e0 != e1) return false;
  // Axes: [m][n], or [b][m][n] with a leading batch axis.
  const int k = r.axis;
  std::vector<int> live = c.LiveAxes();
  const size_t nst = c.root.as.size() - 1;
  if (live.size() != nst || c.store_axes.size() != nst) return false;
  if (g.tensors[c.store_tensor].elem != Elem::F32) return false;
  const int bAx = nst == 3 ? c.store_axes[0] : -1;
  const int mAx = c.store_axes[nst - 2], nAx = c.store_axes[nst - 1];
  // An operand's axes are (x, y), or (b, x, y) when batched.
  auto is2 = [&](const std::vector<int>& ax, int x, int y, bool* batched) {
    if (ax.size() == 2 && ax[0] == x && ax[1] == y) {
      *batched = false;
      return true;
    }
    if (bAx >= 0 && ax.size() == 3 && ax[0] == bAx && ax[1] == x && ax[2] == y) {
      *batched = true;
      return true;
    }
    return false;
  };
  const auto& o0 = c.root.ops[0].axes;
  const auto& o1 = c.root.ops[1].axes;
  GemmMatch out;
  bool ab = false, bb = false;
  auto tryAB = [&](const std::vector<int>& a, const std::vector<int>& b) {
    if (!is2(a, mAx, k, &ab)) return false;
    if (is2(b, k, nAx, &bb)) {
      out.b_nk = false;
      return true;
    }
    if (is2(b, nAx, k, &bb)) {
      out.b_nk = true;
      return true;
    }
    return false;
  };
  if (tryAB(o0, o1)) {
    out.a_op = 0;
    out.b_op = 1;
  } else if (tryAB(o1, o0)) {
    out.a_op = 1;
    out.b_op = 0;
  } else {
    return false;
  }
  out.batch = bAx;
  out.a_batched = ab;
  out.b_batched = bb;
  // Piped epilogue operands must be indexed by m and/or n only.
  if (c.has_piped)
    for (const auto& op : c.piped.ops)
      for (int a : op.axes)
        if (a != mAx && a != nAx) return false;
  out.m = mAx;
  out.n = nAx;
  out.k = k;
  out.in = e0;
  *m = out;
  return true;
}

}  // namespace cg
}  // namespace tca
