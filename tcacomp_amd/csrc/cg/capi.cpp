// capi.cpp — extern "C" face of the builder and emitter (include/tca_cg.h).
// Every entry catches everything: no C++ exception crosses the ABI.
#include <new>
#include <string>

#include "builder.h"
#include "capi_types.h"
#include "emit.h"
#include "tca_cg.h"

namespace {

bool ValidDtype(int32_t d) { return d >= TCA_F32 && d <= TCA_BOOL; }

int Status(tca_builder b, bool ok) {
  if (ok) return TCA_OK;
  b->err = b->b.Error();
  return TCA_ERR_BUILD;
}

template <typename F>
int Guard(tca_builder b, F f) {
  if (b == nullptr) return TCA_ERR_INVALID;
  try {
    return f();
  } catch (const std::exception& e) {
    b->err = std::string("internal error: ") + e.what();
    return TCA_ERR_BUILD;
  } catch (...) {
    b->err = "internal error";
    return TCA_ERR_BUILD;
  }
}

std::vector<int> Ints(uint32_t n, const int32_t* p) {
  std::vector<int> v;
  for (uint32_t i = 0; i < n; ++i) v.push_back(p[i]);
  return v;
}

}  // namespace

extern "C" {

tca_builder tca_builder_new(const char* name) {
  try {
    return new tca_builder_s(name);
  } catch (...) {
    return nullptr;
  }
}

void tca_builder_free(tca_builder b) { delete b; }

const char* tca_builder_error(tca_builder b) { return b ? b->err.c_str() : "null builder"; }

int32_t tca_builder_dim(tca_builder b, const char* name, int64_t extent) {
  return Guard(b, [&]() -> int { return b->b.Dim(name ? name : "", extent); });
}

int32_t tca_builder_tensor(tca_builder b, const char* name, int32_t dtype, uint32_t rank, const int32_t* dims) {
  return Guard(b, [&]() -> int {
    if (!ValidDtype(dtype)) dtype = TCA_F32;
    return b->b.Tensor(name ? name : "", static_cast<tca::ir::Elem>(dtype), Ints(rank, dims));
  });
}

int32_t tca_builder_local(tca_builder b, const char* name, int32_t dtype, uint32_t rank, const int32_t* dims) {
  return Guard(b, [&]() -> int {
    if (!ValidDtype(dtype)) dtype = TCA_F32;
    return b->b.Local(name ? name : "", static_cast<tca::ir::Elem>(dtype), Ints(rank, dims));
  });
}

int32_t tca_builder_scalar(tca_builder b, const char* name, int32_t dtype) {
  return Guard(b, [&]() -> int {
    if (!ValidDtype(dtype)) dtype = TCA_F32;
    return b->b.ScalarParam(name ? name : "", static_cast<tca::ir::Elem>(dtype));
  });
}

int32_t tca_expr_const(tca_builder b, int32_t dtype, double value) {
  return Guard(b, [&]() -> int {
    if (!ValidDtype(dtype)) dtype = TCA_F32;
    return b->b.Const(static_cast<tca::ir::Elem>(dtype), value);
  });
}

int32_t tca_expr_binop(tca_builder b, int32_t op, int32_t x, int32_t y) {
  return Guard(b, [&]() -> int {
    if (op < TCA_ADD || op > TCA_SHR) op = TCA_ADD;
    return b->b.Bin(static_cast<tca::ir::BinOp>(op), x, y);
  });
}

int32_t tca_expr_unop(tca_builder b, int32_t op, int32_t x) {
  return Guard(b, [&]() -> int {
    if (op < TCA_NEG || op > TCA_NOT) op = TCA_NEG;
    return b->b.Un(static_cast<tca::ir::UnOp>(op), x);
  });
}

int32_t tca_expr_select(tca_builder b, int32_t cond, int32_t x, int32_t y) {
  return Guard(b, [&]() -> int { return b->b.Select(cond, x, y); });
}

int32_t tca_expr_cast(tca_builder b, int32_t x, int32_t dtype) {
  return Guard(b, [&]() -> int {
    if (!ValidDtype(dtype)) dtype = TCA_F32;
    return b->b.Cast(x, static_cast<tca::ir::Elem>(dtype));
  });
}

int32_t tca_expr_call(tca_builder b, const char* name, uint32_t n, const int32_t* args) {
  return Guard(b, [&]() -> int { return b->b.Call(name ? name : "", Ints(n, args)); });
}

const char* tca_expr_error(tca_builder b, int32_t expr) {
  if (b == nullptr) return "null builder";
  b->expr_err = b->b.ExprError(expr);
  return b->expr_err.empty() ? nullptr : b->expr_err.c_str();
}

int32_t tca_expr_dtype(tca_builder b, int32_t expr) {
  if (b == nullptr || !b->b.ExprOK(expr)) return -1;
  return static_cast<int32_t>(b->b.ExprType(expr));
}

int32_t tca_stmt(tca_builder b) {
  return Guard(b, [&]() -> int { return b->b.Stmt(); });
}

int tca_chain_iter(tca_builder b, int32_t chain, uint32_t n, const int32_t* dims) {
  return Guard(b, [&]() -> int {
    b->b.Iter(chain, Ints(n, dims));
    return TCA_OK;
  });
}

int tca_chain_map_begin(tca_builder b, int32_t chain, uint32_t n_ops, const tca_operand* ops, int32_t* params_out,
                        uint32_t* n_params) {
  return Guard(b, [&]() -> int {
    std::vector<tca::ir::Operand> v;
    for (uint32_t i = 0; i < n_ops; ++i) {
      tca::ir::Operand o;
      o.tensor = ops[i].tensor;
      for (uint32_t a = 0; a < ops[i].rank && a < TCA_MAX_RANK; ++a) o.axes.push_back(ops[i].axes[a]);
      v.push_back(o);
    }
    std::vector<int> params;
    if (!b->b.MapBegin(chain, v, &params)) return Status(b, false);
    for (size_t i = 0; i < params.size(); ++i) params_out[i] = params[i];
    if (n_params) *n_params = static_cast<uint32_t>(params.size());
    return TCA_OK;
  });
}

int tca_chain_map_end(tca_builder b, int32_t chain, int32_t body) {
  return Guard(b, [&]() -> int { return Status(b, b->b.MapEnd(chain, body)); });
}

int tca_chain_as(tca_builder b, int32_t chain, uint32_t n, const int32_t* dims) {
  return Guard(b, [&]() -> int {
    b->b.As(chain, Ints(n, dims));
    return TCA_OK;
  });
}

int tca_chain_reduce_begin(tca_builder b, int32_t chain, int32_t init, int32_t* acc, int32_t* now) {
  return Guard(b, [&]() -> int {
    int a = -1, n = -1;
    if (!b->b.ReduceBegin(chain, init, &a, &n)) return Status(b, false);
    *acc = a;
    *now = n;
    return TCA_OK;
  });
}

int tca_chain_reduce_end(tca_builder b, int32_t chain, int32_t body) {
  return Guard(b, [&]() -> int { return Status(b, b->b.ReduceEnd(chain, body)); });
}

int tca_chain_store(tca_builder b, int32_t chain, int32_t tensor, uint32_t n, const int32_t* axes) {
  return Guard(b, [&]() -> int { return Status(b, b->b.Store(chain, tensor, Ints(n, axes))); });
}

int tca_builder_build(tca_builder b) {
  return Guard(b, [&]() -> int {
    if (b->is_built) return TCA_OK;
    if (!b->b.Build(&b->built)) return Status(b, false);
    b->is_built = true;
    b->ir_text = tca::ir::PrintReference(b->built);
    b->ir_full = tca::ir::Print(b->built);
    return TCA_OK;
  });
}

const char* tca_builder_ir(tca_builder b) {
  if (b == nullptr || !b->is_built) return nullptr;
  return b->ir_text.c_str();
}

const char* tca_builder_ir_full(tca_builder b) {
  if (b == nullptr || !b->is_built) return nullptr;
  return b->ir_full.c_str();
}

int tca_emit(tca_builder b, const char* kernel_name, const char* target, int32_t flags, tca_emit_result* out) {
  return Guard(b, [&]() -> int {
    if (out == nullptr) return TCA_ERR_INVALID;
    *out = nullptr;
    if (!b->is_built) {
      b->err = "emit: the program has not been built";
      return TCA_ERR_BUILD;
    }
    tca::cg::Options o;
    if (kernel_name) o.kernel_name = kernel_name;
    if (target) o.target = target;
    o.allow_fused = (flags & TCA_EMIT_NO_FUSION) == 0;
    o.allow_gemm = (flags & TCA_EMIT_NO_GEMM) == 0;
    o.allow_gemm_split = (flags & TCA_EMIT_NO_GEMM_SPLIT) == 0;
    o.allow_pass_fusion = (flags & TCA_EMIT_NO_PASS_FUSION) == 0;
    o.row_vectors_per_lane = (flags >> 8) & 0xf;
    o.elementwise_unroll = (flags >> 12) & 0xf;
    auto* r = new tca_emit_result_s;
    std::string err;
    if (!tca::cg::Emit(b->built, o, &r->r, &err)) {
      delete r;
      b->err = err;
      return TCA_ERR_UNSUPPORTED;
    }
    *out = r;
    return TCA_OK;
  });
}

const char* tca_emit_source(tca_emit_result r) { return r ? r->r.source.c_str() : nullptr; }
const char* tca_emit_plan(tca_emit_result r) { return r ? r->r.plan.c_str() : nullptr; }
const char* tca_emit_report(tca_emit_result r) { return r ? r->r.report.c_str() : nullptr; }
uint32_t tca_emit_hipcc_argc(tca_emit_result r) { return r ? static_cast<uint32_t>(r->r.hipcc.size()) : 0u; }
const char* tca_emit_hipcc_arg(tca_emit_result r, uint32_t i) {
  if (r == nullptr || i >= r->r.hipcc.size()) return nullptr;
  return r->r.hipcc[i].c_str();
}
void tca_emit_free(tca_emit_result r) { delete r; }

}  // extern "C"
