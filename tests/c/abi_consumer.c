/*
 * A plain-C consumer of the three public headers, compiled with
 *   gcc -std=c99 -pedantic -Wall -Wextra -Werror -I include
 * and linked against libtcacomp.so: the path a cgo binding takes (cgo sees
 * exactly these declarations). Test program, not part of the library.
 *
 *   abi_consumer host <kcache.hip> <configs.tca>
 *       builds C2 (row sum + row max of x[R, 8192], two chains, pkg/chain.go
 *       rungs Iter -> Map -> As -> Reduce -> Store) through tca_cg.h, emits
 *       it, checks that the emitted source equals <kcache.hip> byte for
 *       byte (the code object prebuilt from it is then the one to launch),
 *       parses the plan, and exercises the shape contract and the kernel
 *       selection; then parses and builds every kernel of <configs.tca>
 *       through tca_syntax.h. No GPU.
 *   abi_consumer gpu <kcache.hip> <kcache.hsaco> <rows>
 *       the same program, loaded and launched through tca_rt.h on device 0
 *       with the reference's input formula (testing/runners/common.cuh:19-21),
 *       compared with the C oracle (oracle/oracle.c, linked by the test):
 *       max bit-identical, sum within 1e-5 * sqrt(C) * ||row||_2.
 *
 *       It then times the host side of a launch: tca_program_launch against
 *       tca_rt_launch of the same kernel with a prepacked argument blob (the
 *       hipModuleLaunchKernel call alone), both on a one-workgroup problem.
 *
 * Prints one "ok ..." line and exits 0, or prints the failure and exits 1.
 */
#define _POSIX_C_SOURCE 199309L
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "tca_cg.h"
#include "tca_rt.h"
#include "tca_syntax.h"

/* The C oracle's entry points (oracle/oracle.c; test infrastructure). */
void oracle_fill_elem(float* out, uint64_t n);
void oracle_row_sum_max(const float* x, uint32_t R, uint32_t C, float* sum, float* max, int threads);

#define COLS 8192u

static int fail(const char* what, const char* detail) {
  fprintf(stderr, "FAIL %s: %s\n", what, detail ? detail : "");
  return 1;
}

#define REQUIRE(cond, what, detail)       \
  do {                                     \
    if (!(cond)) return fail(what, detail); \
  } while (0)

/* One chain: Iter(R, C).Map(x[R][C] -> v).As(R, C).Reduce(init, fold).Store(out[R]).
 * fold_max selects fmaxf(acc, v) over acc + v. */
static int reduce_chain(tca_builder b, int32_t R, int32_t C, int32_t x, int32_t out, int32_t init, int fold_max) {
  int32_t chain = tca_stmt(b);
  int32_t dims[2];
  tca_operand op;
  int32_t params[2];
  uint32_t n_params = 0;
  int32_t acc = -1, now = -1, body;
  dims[0] = R;
  dims[1] = C;
  memset(&op, 0, sizeof op);
  op.tensor = x;
  op.rank = 2;
  op.axes[0] = R;
  op.axes[1] = C;
  if (tca_chain_iter(b, chain, 2, dims) != TCA_OK) return -1;
  if (tca_chain_map_begin(b, chain, 1, &op, params, &n_params) != TCA_OK || n_params != 1) return -1;
  if (tca_chain_map_end(b, chain, params[0]) != TCA_OK) return -1;
  if (tca_chain_as(b, chain, 2, dims) != TCA_OK) return -1;
  if (tca_chain_reduce_begin(b, chain, init, &acc, &now) != TCA_OK) return -1;
  if (fold_max) {
    int32_t args[2];
    args[0] = acc;
    args[1] = now;
    body = tca_expr_call(b, "fmaxf", 2, args);
  } else {
    body = tca_expr_binop(b, TCA_ADD, acc, now);
  }
  if (tca_chain_reduce_end(b, chain, body) != TCA_OK) return -1;
  return tca_chain_store(b, chain, out, 1, dims);
}

/* C2 as programs.row_sum_max(8192) builds it: same names, same order, so
 * the emitted source is byte-identical. */
static tca_builder build_c2(void) {
  tca_builder b = tca_builder_new("row_sum_max_8192");
  int32_t R = tca_builder_dim(b, "R", 0);
  int32_t C = tca_builder_dim(b, "e8192", COLS);
  int32_t xd[2], od[1];
  int32_t x, s, m, neg_inf;
  xd[0] = R;
  xd[1] = C;
  od[0] = R;
  x = tca_builder_tensor(b, "x", TCA_F32, 2, xd);
  s = tca_builder_tensor(b, "sum", TCA_F32, 1, od);
  m = tca_builder_tensor(b, "max", TCA_F32, 1, od);
  if (reduce_chain(b, R, C, x, s, tca_expr_const(b, TCA_F32, 0.0), 0) != TCA_OK) return b;
  neg_inf = tca_expr_unop(b, TCA_NEG, tca_expr_const(b, TCA_F32, (double)INFINITY));
  if (reduce_chain(b, R, C, x, m, neg_inf, 1) != TCA_OK) return b;
  tca_builder_build(b);
  return b;
}

static char* read_file(const char* path) {
  FILE* f = fopen(path, "rb");
  long n;
  char* buf;
  if (!f) return NULL;
  fseek(f, 0, SEEK_END);
  n = ftell(f);
  fseek(f, 0, SEEK_SET);
  buf = (char*)malloc((size_t)n + 1);
  if (buf && fread(buf, 1, (size_t)n, f) != (size_t)n) {
    free(buf);
    buf = NULL;
  }
  if (buf) buf[n] = '\0';
  fclose(f);
  return buf;
}

static void set_tensor(tca_tensor* t, void* data, uint32_t rank, uint32_t d0, uint32_t d1) {
  memset(t, 0, sizeof *t);
  t->data = data;
  t->rank = rank;
  t->dims[0] = d0;
  t->dims[1] = d1;
  t->dtype = TCA_F32;
}

/* Builds, emits, compares with the prebuilt source and parses the plan.
 * On success *plan_out is a copy of the emitted plan. */
static int emit_c2(const char* kcache_hip, char** plan_out) {
  tca_builder b = build_c2();
  tca_emit_result r = NULL;
  const char* err = tca_builder_error(b);
  const char* ir;
  char* want;
  REQUIRE(err == NULL || err[0] == '\0', "build", err);
  /* The reference's print: 5 params take IDs 1-5, the 0.0 init (built
   * before the first Stmt) 6; the first Stmt reserves 7 (statement) and 8
   * (end node, claimed by the first output store). */
  ir = tca_builder_ir(b);
  REQUIRE(ir != NULL && strncmp(ir, "statement #7:\n  iter(@R, @e8192) -> map(x[@R][@e8192], lambda(v): v)", 64) == 0,
          "ir", ir);
  REQUIRE(strstr(ir, "statement #8:\n  return %sum, %max\n") != NULL, "ir end node", ir);
  REQUIRE(tca_builder_ir_full(b) != NULL && strstr(tca_builder_ir_full(b), "program row_sum_max_8192") != NULL,
          "ir full", tca_builder_ir_full(b));
  REQUIRE(tca_emit(b, NULL, "gfx950", 0, &r) == TCA_OK, "emit", tca_builder_error(b));
  REQUIRE(tca_emit_hipcc_argc(r) > 0 && strstr(tca_emit_report(r), "row") != NULL, "emit report",
          tca_emit_report(r));
  want = read_file(kcache_hip);
  REQUIRE(want != NULL, "read prebuilt source", kcache_hip);
  REQUIRE(strcmp(want, tca_emit_source(r)) == 0, "emitted source differs from the prebuilt one", kcache_hip);
  free(want);
  *plan_out = (char*)malloc(strlen(tca_emit_plan(r)) + 1);
  strcpy(*plan_out, tca_emit_plan(r));
  tca_emit_free(r);
  tca_builder_free(b);
  return 0;
}

static int host_checks(const char* plan, const char* tca_path) {
  tca_program p = NULL;
  uint32_t nt = 0, nf = 0, ns = 0, nk = 0;
  tca_tensor ts[3];
  uint8_t sel[4];
  uint64_t grids[4];
  uint32_t blocks[4];
  void* fake = (void*)(uintptr_t)0x10000; /* never dereferenced: host-only checks */
  tca_syntax_module mod = NULL;
  uint32_t i, kernels;

  REQUIRE(tca_program_parse(plan, &p) == TCA_OK, "plan parse", tca_rt_last_error());
  REQUIRE(tca_program_signature(p, &nt, &nf, &ns, &nk) == TCA_OK, "signature", tca_rt_last_error());
  REQUIRE(nt == 3 && nf == 0 && ns == 0 && nk == 1, "signature", "expected 3 tensors, 0 dims, 0 scalars, 1 kernel");
  REQUIRE(tca_program_kernel_name(p, 0) != NULL && strcmp(tca_program_kernel_name(p, 0), "tca_row_sum_max_8192_k0") == 0,
          "kernel name", tca_program_kernel_name(p, 0));

  set_tensor(&ts[0], fake, 2, 1000, COLS);
  set_tensor(&ts[1], fake, 1, 1000, 0);
  set_tensor(&ts[2], fake, 1, 1000, 0);
  REQUIRE(tca_program_check(p, ts, 3, NULL, 0) == TCA_OK, "check", tca_rt_last_error());
  REQUIRE(tca_program_selected(p, ts, 3, NULL, 0, sel, grids, blocks, 1) == TCA_OK, "selected", tca_rt_last_error());
  REQUIRE(sel[0] == 1 && grids[0] >= 1 && blocks[0] % 64 == 0 && blocks[0] <= 1024, "selected geometry", "");

  ts[2].dims[0] = 999; /* max[R] disagrees with x[R, C] */
  REQUIRE(tca_program_check(p, ts, 3, NULL, 0) == TCA_ERR_SHAPE, "dim disagreement not refused", "");
  REQUIRE(strlen(tca_rt_last_error()) > 0, "dim disagreement message", "");
  ts[2].dims[0] = 1000;
  ts[0].dims[1] = COLS - 1; /* a compile-time extent */
  REQUIRE(tca_program_check(p, ts, 3, NULL, 0) == TCA_ERR_SHAPE, "static extent not enforced", "");
  ts[0].dims[1] = COLS;
  ts[1].dtype = TCA_BF16;
  REQUIRE(tca_program_check(p, ts, 3, NULL, 0) != TCA_OK, "dtype mismatch not refused", "");
  ts[1].dtype = TCA_F32;
  REQUIRE(tca_program_check(p, ts, 2, NULL, 0) != TCA_OK, "tensor count not checked", "");
  REQUIRE(tca_program_unload(p) == TCA_OK, "unload parsed program", tca_rt_last_error());

  /* The .tca frontend's module handle is its own type. */
  REQUIRE(tca_syntax_parse_module(tca_path, &mod) == TCA_OK, "parse .tca module", tca_syntax_last_error());
  kernels = tca_syntax_module_kernel_count(mod);
  REQUIRE(kernels >= 5, "kernel count", tca_syntax_module_diagnostics(mod));
  for (i = 0; i < kernels; ++i) {
    tca_builder kb = NULL;
    REQUIRE(tca_syntax_module_build_kernel(mod, i, &kb) == TCA_OK, "build .tca kernel", tca_syntax_last_error());
    REQUIRE(tca_builder_ir(kb) != NULL, ".tca kernel ir", tca_syntax_module_kernel_name(mod, i));
    tca_builder_free(kb);
  }
  tca_syntax_module_free(mod);
  REQUIRE(tca_syntax_parse_source("bad.tca", "kernel k( {", 1, &mod) == TCA_ERR_BUILD && mod == NULL,
          "malformed .tca accepted", "");
  REQUIRE(strstr(tca_syntax_last_error(), "bad.tca:") != NULL, "diagnostic position", tca_syntax_last_error());
  return 0;
}

static double now_us(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec * 1e6 + (double)ts.tv_nsec * 1e-3;
}

/* Median over 15 batches of the host time per call of 200 calls of `launch`
 * (the device drained between batches, so the queue never fills). */
#define LAUNCH_BATCH 200
#define LAUNCH_BATCHES 15
static int cmp_double(const void* a, const void* b) {
  double x = *(const double*)a, y = *(const double*)b;
  return x < y ? -1 : x > y;
}

static int time_launch_cost(const char* plan, const char* hsaco, void* dx, void* ds, void* dm, double* prog_us,
                            double* raw_us) {
  tca_program p = NULL;
  tca_module m = NULL;
  tca_tensor ts[3];
  unsigned char blob[32];
  uint32_t one = 1, cols = COLS;
  double tp[LAUNCH_BATCHES], tr[LAUNCH_BATCHES];
  int b, i;
  REQUIRE(tca_program_load(hsaco, plan, &p) == TCA_OK, "program load", tca_rt_last_error());
  REQUIRE(tca_rt_module_load(hsaco, &m) == TCA_OK, "module load", tca_rt_last_error());
  set_tensor(&ts[0], dx, 2, 1, COLS);
  set_tensor(&ts[1], ds, 1, 1, 0);
  set_tensor(&ts[2], dm, 1, 1, 0);
  /* The kernel's arguments (its plan: ptr x, ptr sum, ptr max, dim R, dim e8192). */
  memcpy(blob, &dx, 8);
  memcpy(blob + 8, &ds, 8);
  memcpy(blob + 16, &dm, 8);
  memcpy(blob + 24, &one, 4);
  memcpy(blob + 28, &cols, 4);
  for (b = 0; b < LAUNCH_BATCHES; ++b) {
    double t0;
    REQUIRE(tca_rt_device_sync() == TCA_OK, "sync", tca_rt_last_error());
    t0 = now_us();
    for (i = 0; i < LAUNCH_BATCH; ++i)
      REQUIRE(tca_program_launch(p, ts, 3, NULL, 0, NULL, 0, NULL) == TCA_OK, "launch", tca_rt_last_error());
    tp[b] = (now_us() - t0) / LAUNCH_BATCH;
    REQUIRE(tca_rt_device_sync() == TCA_OK, "sync", tca_rt_last_error());
    t0 = now_us();
    for (i = 0; i < LAUNCH_BATCH; ++i)
      REQUIRE(tca_rt_launch(m, "tca_row_sum_max_8192_k0", 1, 512, 0, blob, sizeof blob, NULL) == TCA_OK, "raw launch",
              tca_rt_last_error());
    tr[b] = (now_us() - t0) / LAUNCH_BATCH;
  }
  REQUIRE(tca_rt_device_sync() == TCA_OK, "sync", tca_rt_last_error());
  qsort(tp, LAUNCH_BATCHES, sizeof(double), cmp_double);
  qsort(tr, LAUNCH_BATCHES, sizeof(double), cmp_double);
  *prog_us = tp[LAUNCH_BATCHES / 2];
  *raw_us = tr[LAUNCH_BATCHES / 2];
  REQUIRE(tca_rt_module_unload(m) == TCA_OK, "module unload", tca_rt_last_error());
  REQUIRE(tca_program_unload(p) == TCA_OK, "unload", tca_rt_last_error());
  return 0;
}

static int gpu_run(const char* plan, const char* hsaco, uint32_t rows) {
  tca_program p = NULL;
  tca_event e0 = NULL, e1 = NULL;
  size_t n = (size_t)rows * COLS;
  float* x = (float*)malloc(n * sizeof(float));
  float* got_s = (float*)malloc(rows * sizeof(float));
  float* got_m = (float*)malloc(rows * sizeof(float));
  float* want_s = (float*)malloc(rows * sizeof(float));
  float* want_m = (float*)malloc(rows * sizeof(float));
  void *dx = NULL, *ds = NULL, *dm = NULL;
  tca_tensor ts[3];
  float ms = 0.0f;
  double worst = 0.0, prog_us = 0.0, raw_us = 0.0;
  uint32_t r, c;

  REQUIRE(x && got_s && got_m && want_s && want_m, "host alloc", "");
  oracle_fill_elem(x, n);
  oracle_row_sum_max(x, rows, COLS, want_s, want_m, 1);

  REQUIRE(tca_rt_init(0) == TCA_OK, "init", tca_rt_last_error());
  REQUIRE(tca_program_load(hsaco, plan, &p) == TCA_OK, "program load", tca_rt_last_error());
  REQUIRE(tca_rt_malloc(&dx, n * sizeof(float)) == TCA_OK, "malloc x", tca_rt_last_error());
  REQUIRE(tca_rt_malloc(&ds, rows * sizeof(float)) == TCA_OK, "malloc sum", tca_rt_last_error());
  REQUIRE(tca_rt_malloc(&dm, rows * sizeof(float)) == TCA_OK, "malloc max", tca_rt_last_error());
  REQUIRE(tca_rt_memcpy_h2d(dx, x, n * sizeof(float)) == TCA_OK, "h2d", tca_rt_last_error());
  /* 0xC6 bytes: a canary value (-25443.1f) no row of elem() can produce. */
  REQUIRE(tca_rt_memset(ds, 0xC6, rows * sizeof(float)) == TCA_OK, "memset", tca_rt_last_error());
  REQUIRE(tca_rt_memset(dm, 0xC6, rows * sizeof(float)) == TCA_OK, "memset", tca_rt_last_error());
  set_tensor(&ts[0], dx, 2, rows, COLS);
  set_tensor(&ts[1], ds, 1, rows, 0);
  set_tensor(&ts[2], dm, 1, rows, 0);
  REQUIRE(tca_rt_event_create(&e0) == TCA_OK && tca_rt_event_create(&e1) == TCA_OK, "events", tca_rt_last_error());
  REQUIRE(tca_rt_event_record(e0, NULL) == TCA_OK, "record", tca_rt_last_error());
  REQUIRE(tca_program_launch(p, ts, 3, NULL, 0, NULL, 0, NULL) == TCA_OK, "launch", tca_rt_last_error());
  REQUIRE(tca_rt_event_record(e1, NULL) == TCA_OK, "record", tca_rt_last_error());
  REQUIRE(tca_rt_device_sync() == TCA_OK, "sync", tca_rt_last_error());
  REQUIRE(tca_rt_event_elapsed_ms(e0, e1, &ms) == TCA_OK && ms >= 0.0f, "elapsed", tca_rt_last_error());
  REQUIRE(tca_rt_memcpy_d2h(got_s, ds, rows * sizeof(float)) == TCA_OK, "d2h", tca_rt_last_error());
  REQUIRE(tca_rt_memcpy_d2h(got_m, dm, rows * sizeof(float)) == TCA_OK, "d2h", tca_rt_last_error());

  for (r = 0; r < rows; ++r) {
    double l2 = 0.0, err;
    for (c = 0; c < COLS; ++c) l2 += (double)x[(size_t)r * COLS + c] * x[(size_t)r * COLS + c];
    err = fabs((double)got_s[r] - (double)want_s[r]);
    if (memcmp(&got_m[r], &want_m[r], sizeof(float)) != 0) {
      fprintf(stderr, "row %u: max %.9g, oracle %.9g\n", r, got_m[r], want_m[r]);
      return fail("max not bit-identical", "");
    }
    if (err > 1e-5 * sqrt((double)COLS) * sqrt(l2)) {
      fprintf(stderr, "row %u: sum %.9g, oracle %.9g\n", r, got_s[r], want_s[r]);
      return fail("sum outside 1e-5*sqrt(C)*||row||", "");
    }
    if (err > worst) worst = err;
  }
  tca_rt_event_destroy(e0);
  tca_rt_event_destroy(e1);
  REQUIRE(tca_program_unload(p) == TCA_OK, "unload", tca_rt_last_error());
  if (time_launch_cost(plan, hsaco, dx, ds, dm, &prog_us, &raw_us) != 0) return 1;
  tca_rt_free(dx);
  tca_rt_free(ds);
  tca_rt_free(dm);
  printf("ok gpu rows=%u max_abs_sum_err=%.3g launch_ms=%.4f host_us_per_launch=%.2f host_us_per_raw_launch=%.2f\n",
         rows, worst, (double)ms, prog_us, raw_us);
  free(x);
  free(got_s);
  free(got_m);
  free(want_s);
  free(want_m);
  return 0;
}

int main(int argc, char** argv) {
  char* plan = NULL;
  int rc;
  if (argc == 4 && strcmp(argv[1], "host") == 0) {
    if (emit_c2(argv[2], &plan) != 0) return 1;
    rc = host_checks(plan, argv[3]);
    free(plan);
    if (rc == 0) printf("ok host\n");
    return rc;
  }
  if (argc == 5 && strcmp(argv[1], "gpu") == 0) {
    if (emit_c2(argv[2], &plan) != 0) return 1;
    rc = gpu_run(plan, argv[3], (uint32_t)strtoul(argv[4], NULL, 10));
    free(plan);
    return rc;
  }
  fprintf(stderr, "usage: %s host <kcache.hip> <configs.tca> | gpu <kcache.hip> <kcache.hsaco> <rows>\n", argv[0]);
  return 2;
}
