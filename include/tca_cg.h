/*
 * tca_cg.h — C ABI of the tcacomp DSL builder and HIP emitter (the
 * compile-time seam).
 *
 * Reference interfaces this replaces, one for one:
 *   pkg.NewBuilder / Builder.Dim / Tensor / Local / ScalarParam
 *        pkg/builder.go:122-295
 *   Expr operators, literals, Select, Cast, Call
 *        pkg/expr.go:140-341 (builtin registry internal/ir/builtins.go:25-33)
 *   Stmt().Iter().Map().As().Reduce()...Store() chain rungs
 *        pkg/chain.go:360-552
 *   Builder.Build                      pkg/builder.go:340-370
 *   ir.Print                           internal/ir/print.go:34-57 (tca_builder_ir)
 *   cxx.Emit(g, cg.Options) -> cg.Result   internal/cg/cxx/emit.go:85,
 *                                          internal/cg/cg.go:17-64
 * A Go lambda `func(l, r pkg.Expr) pkg.Expr` becomes a begin/end pair here:
 * *_begin hands out the lambda's parameter expressions, the caller builds
 * the body with tca_expr_*, and *_end takes the body.
 *
 * Handles are int32 indices (>= 0) into the builder; an expression whose
 * construction failed is still a valid handle whose error surfaces at the
 * rung that consumes it (the reference's deferred Expr.err). Rungs return
 * TCA_OK or TCA_ERR_BUILD with the message in tca_builder_error(). Nothing
 * here needs a GPU.
 */
#ifndef TCA_CG_H_
#define TCA_CG_H_

#include <stdint.h>

#include "tca_rt.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tca_builder_s* tca_builder;
typedef struct tca_emit_result_s* tca_emit_result;

/* One structural access t[axes...] (pkg.At, pkg/builder.go:112-118). */
typedef struct tca_operand {
  int32_t tensor;
  uint32_t rank;
  int32_t axes[TCA_MAX_RANK];
} tca_operand;

/* Binary operators (pkg/expr.go:179-231). */
enum {
  TCA_ADD = 0, TCA_SUB, TCA_MUL, TCA_DIV, TCA_MOD,
  TCA_EQ, TCA_NE, TCA_LT, TCA_LE, TCA_GT, TCA_GE,
  TCA_LAND, TCA_LOR, TCA_AND, TCA_OR, TCA_XOR, TCA_SHL, TCA_SHR
};
/* Unary operators (pkg/expr.go:233-240). */
enum { TCA_NEG = 0, TCA_POS, TCA_LNOT, TCA_NOT };

/* Emit flags. Bits 8-11 / 12-15 carry the row family's vectors per lane and
 * the elementwise family's vectors per thread (powers of two; 0 = default).
 * TCA_EMIT_NO_GEMM_SPLIT leaves out the contractions' small-tile K-split
 * kernels (every output plane then takes the 128/256 tile kernels).
 * TCA_EMIT_NO_PASS_FUSION keeps every pass of a multi-pass nest its own read
 * of the input (no online softmax normaliser and no pairwise mean/variance
 * in split or streamed rows, no pairwise mean/variance in the column
 * family). */
enum { TCA_EMIT_NO_FUSION = 1, TCA_EMIT_NO_GEMM = 2, TCA_EMIT_NO_GEMM_SPLIT = 4, TCA_EMIT_NO_PASS_FUSION = 8 };
#define TCA_EMIT_ROW_VECTORS(n) ((n) << 8)
#define TCA_EMIT_EW_UNROLL(n) ((n) << 12)

tca_builder tca_builder_new(const char* name);
void tca_builder_free(tca_builder b);
const char* tca_builder_error(tca_builder b);

int32_t tca_builder_dim(tca_builder b, const char* name, int64_t extent);
int32_t tca_builder_tensor(tca_builder b, const char* name, int32_t dtype, uint32_t rank, const int32_t* dims);
int32_t tca_builder_local(tca_builder b, const char* name, int32_t dtype, uint32_t rank, const int32_t* dims);
int32_t tca_builder_scalar(tca_builder b, const char* name, int32_t dtype);

int32_t tca_expr_const(tca_builder b, int32_t dtype, double value);
int32_t tca_expr_binop(tca_builder b, int32_t op, int32_t x, int32_t y);
int32_t tca_expr_unop(tca_builder b, int32_t op, int32_t x);
int32_t tca_expr_select(tca_builder b, int32_t cond, int32_t x, int32_t y);
int32_t tca_expr_cast(tca_builder b, int32_t x, int32_t dtype);
int32_t tca_expr_call(tca_builder b, const char* name, uint32_t n, const int32_t* args);
/* NULL when the expression is valid. */
const char* tca_expr_error(tca_builder b, int32_t expr);
int32_t tca_expr_dtype(tca_builder b, int32_t expr);

int32_t tca_stmt(tca_builder b);
int tca_chain_iter(tca_builder b, int32_t chain, uint32_t n, const int32_t* dims);
/* params_out must hold n_ops + 1 entries (a piped map's first parameter is
 * the piped value); *n_params receives the count. */
int tca_chain_map_begin(tca_builder b, int32_t chain, uint32_t n_ops, const tca_operand* ops, int32_t* params_out,
                        uint32_t* n_params);
int tca_chain_map_end(tca_builder b, int32_t chain, int32_t body);
int tca_chain_as(tca_builder b, int32_t chain, uint32_t n, const int32_t* dims);
int tca_chain_reduce_begin(tca_builder b, int32_t chain, int32_t init, int32_t* acc, int32_t* now);
int tca_chain_reduce_end(tca_builder b, int32_t chain, int32_t body);
int tca_chain_store(tca_builder b, int32_t chain, int32_t tensor, uint32_t n, const int32_t* axes);

/* Verifies and freezes the program. */
int tca_builder_build(tca_builder b);
/* The reference's canonical IR print of the built program (owned by the
 * builder): `statement #ID:` blocks in the doc notation, statement IDs
 * numbered as the reference builder allocates them (the Stmt() reservation
 * of pkg/builder.go:310-318). Byte-identical to the reference's golden
 * pkg/testdata/matmul_scale.ir for that program. */
const char* tca_builder_ir(tca_builder b);
/* This build's structural dump of the built program (owned by the builder):
 * declarations with types and extents, each chain's operand axes, reduced
 * axes and lambda bodies. Equal dumps mean the same program. No counterpart
 * in the reference (its print omits types and access axes); for tests and
 * tools that compare programs. */
const char* tca_builder_ir_full(tca_builder b);

/* Runs the HIP emitter on the built program. kernel_name NULL = the program
 * name; target NULL = "gfx950". */
int tca_emit(tca_builder b, const char* kernel_name, const char* target, int32_t flags, tca_emit_result* out);
const char* tca_emit_source(tca_emit_result r);
const char* tca_emit_plan(tca_emit_result r);
const char* tca_emit_report(tca_emit_result r);
uint32_t tca_emit_hipcc_argc(tca_emit_result r);
const char* tca_emit_hipcc_arg(tca_emit_result r, uint32_t i);
void tca_emit_free(tca_emit_result r);

#ifdef __cplusplus
}
#endif

#endif /* TCA_CG_H_ */
