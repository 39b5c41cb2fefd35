/*
 * oracle.c — TEST INFRASTRUCTURE ONLY. CPU restatement of the reference's
 * oracle loops for the map+reduce path. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this; no product path does.
 *
 * Semantics restated (every function cites its reference loop):
 *   - each output folds its reduced axis in ascending index order from
 *     init, acc = fn(acc, v) (runtime/tca/reducer.h:36-57, the SeqReducer;
 *     testing/runners/gemm.cu:46-48 and every runner's `float acc = 0.0f`
 *     loop);
 *   - fp32 IEEE arithmetic, no contraction: built with -ffp-contract=off;
 *   - rsqrtf(x) is defined as 1.0f / sqrtf(x) (correctly rounded sqrt, then
 *     a correctly rounded division);
 *   - expf / tanhf are glibc's (the reference's GPU side calls NVIDIA's
 *     closed math library, pinned only to tolerance by its own tests).
 * Multi-threaded entry points split independent output rows over pthreads;
 * the per-output fold order is unchanged, so results are bit-identical to
 * the 1-thread run.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- inputs ---------------------------------------------------------- */

/* testing/runners/common.cuh:19-21 (Go twin internal/e2e/e2e_test.go:194-200). */
float oracle_elem(uint32_t i) { return (float)((i * 2654435761u) % 1000u) / 1000.0f; }

void oracle_fill_elem(float* out, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) out[i] = oracle_elem((uint32_t)i);
}

/* bf16 round-to-nearest-even of an fp32 value (NaN kept quiet). */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ---- row-parallel driver -------------------------------------------- */

typedef void (*row_fn)(void* ctx, uint64_t r0, uint64_t r1);

typedef struct {
  row_fn fn;
  void* ctx;
  uint64_t r0, r1;
} job_t;

static void* run_job(void* p) {
  job_t* j = (job_t*)p;
  j->fn(j->ctx, j->r0, j->r1);
  return NULL;
}

static void parallel_rows(row_fn fn, void* ctx, uint64_t rows, int threads) {
  if (threads <= 1 || rows < 2) {
    fn(ctx, 0, rows);
    return;
  }
  if ((uint64_t)threads > rows) threads = (int)rows;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  job_t* jobs = (job_t*)malloc(sizeof(job_t) * (size_t)threads);
  for (int t = 0; t < threads; ++t) {
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].r0 = rows * (uint64_t)t / (uint64_t)threads;
    jobs[t].r1 = rows * (uint64_t)(t + 1) / (uint64_t)threads;
    pthread_create(&th[t], NULL, run_job, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  free(th);
  free(jobs);
}

/* ---- C1: z = max(a*x + y, 0) ----------------------------------------
 * The degenerate-reduce encoding folds one element from init 0:
 * z = 0.0f + fmaxf(a*x + y, 0.0f) (testing/runners/scale_copy.cu:52-55
 * pattern with K = 1). */
typedef struct {
  const float *x, *y;
  float a;
  float* z;
} c1_ctx;

static void c1_rows(void* p, uint64_t r0, uint64_t r1) {
  c1_ctx* c = (c1_ctx*)p;
  for (uint64_t i = r0; i < r1; ++i) {
    float acc = 0.0f;
    acc = acc + fmaxf(c->a * c->x[i] + c->y[i], 0.0f);
    c->z[i] = acc;
  }
}

void oracle_scale_relu(const float* x, const float* y, float a, float* z, uint64_t n, int threads) {
  c1_ctx c = {x, y, a, z};
  parallel_rows(c1_rows, &c, n, threads);
}

/* ---- C2: row sum and row max ----------------------------------------
 * reduceReference (internal/e2e/e2e_test.go:227-240) for the sum; the max
 * chain folds fmaxf from -inf the same way. */
typedef struct {
  const float* x;
  uint64_t C;
  float *sum, *max;
} c2_ctx;

static void c2_rows(void* p, uint64_t r0, uint64_t r1) {
  c2_ctx* c = (c2_ctx*)p;
  for (uint64_t r = r0; r < r1; ++r) {
    const float* row = c->x + r * c->C;
    float s = 0.0f, m = -INFINITY;
    for (uint64_t j = 0; j < c->C; ++j) {
      s = s + row[j];
      m = fmaxf(m, row[j]);
    }
    c->sum[r] = s;
    c->max[r] = m;
  }
}

void oracle_row_sum_max(const float* x, uint32_t R, uint32_t C, float* sum, float* max, int threads) {
  c2_ctx c = {x, C, sum, max};
  parallel_rows(c2_rows, &c, R, threads);
}

/* ---- C3: row softmax as three chains ---------------------------------
 * mx = fold fmaxf from -inf; den = fold + of expf(x - mx) from 0;
 * y = expf(x - mx) / den (the program in tcacomp_amd/programs.py:softmax;
 * the reference's own softmax core is testing/runners/softmax.cu:49-56). */
typedef struct {
  const float* x;
  uint64_t C;
  float* y;
} c3_ctx;

static void c3_rows(void* p, uint64_t r0, uint64_t r1) {
  c3_ctx* c = (c3_ctx*)p;
  for (uint64_t r = r0; r < r1; ++r) {
    const float* row = c->x + r * c->C;
    float* out = c->y + r * c->C;
    float m = -INFINITY;
    for (uint64_t j = 0; j < c->C; ++j) m = fmaxf(m, row[j]);
    float d = 0.0f;
    for (uint64_t j = 0; j < c->C; ++j) d = d + expf(row[j] - m);
    for (uint64_t j = 0; j < c->C; ++j) out[j] = expf(row[j] - m) / d;
  }
}

void oracle_softmax(const float* x, uint32_t R, uint32_t C, float* y, int threads) {
  c3_ctx c = {x, C, y};
  parallel_rows(c3_rows, &c, R, threads);
}

/* ---- C4: layernorm ---------------------------------------------------
 * mean = (fold +) * inv_n; var = (fold + of (x-mean)*(x-mean)) * inv_n;
 * y = (x - mean) * rsqrtf(var + eps) * gamma + beta, evaluated left to
 * right as written (tcacomp_amd/programs.py:layernorm; the reference's RMS
 * core is testing/runners/layernorm.cu:47-54). */
typedef struct {
  const float *x, *g, *b;
  uint64_t C;
  float inv_n, eps;
  float* y;
} c4_ctx;

static void c4_rows(void* p, uint64_t r0, uint64_t r1) {
  c4_ctx* c = (c4_ctx*)p;
  for (uint64_t r = r0; r < r1; ++r) {
    const float* row = c->x + r * c->C;
    float* out = c->y + r * c->C;
    float s = 0.0f;
    for (uint64_t j = 0; j < c->C; ++j) s = s + row[j];
    const float mean = s * c->inv_n;
    float q = 0.0f;
    for (uint64_t j = 0; j < c->C; ++j) {
      const float d = row[j] - mean;
      q = q + d * d;
    }
    const float var = q * c->inv_n;
    const float rs = 1.0f / sqrtf(var + c->eps);
    for (uint64_t j = 0; j < c->C; ++j) out[j] = (row[j] - mean) * rs * c->g[j] + c->b[j];
  }
}

void oracle_layernorm(const float* x, const float* gamma, const float* beta, uint32_t R, uint32_t C, float inv_n,
                      float eps, float* y, int threads) {
  c4_ctx c = {x, gamma, beta, C, inv_n, eps, y};
  parallel_rows(c4_rows, &c, R, threads);
}

/* ---- C5: dense contraction -------------------------------------------
 * testing/runners/gemm.cu:44-49: acc = 0; acc += A[m,k] * B[k,n] for k
 * ascending. Loop order m -> k -> n keeps each element's k order and is
 * cache-friendly (bit-identical to the runner's k-innermost loop). The
 * epilogue kinds restate testing/runners/mlp.cu:50-52 (GELU) and
 * testing/runners/qk_score.cu:51 (scale). */
enum { EPI_NONE = 0, EPI_GELU = 1, EPI_SCALE = 2 };

typedef struct {
  const float *A, *B;
  const uint16_t *A16, *B16;
  uint64_t M, N, K;
  int b_nk, epi;
  float scale;
  float* C;
} gemm_ctx;

static inline float ld_a(const gemm_ctx* c, uint64_t m, uint64_t k) {
  return c->A16 ? oracle_bf16_to_f32(c->A16[m * c->K + k]) : c->A[m * c->K + k];
}
static inline float ld_b(const gemm_ctx* c, uint64_t k, uint64_t n) {
  const uint64_t off = c->b_nk ? n * c->K + k : k * c->N + n;
  return c->B16 ? oracle_bf16_to_f32(c->B16[off]) : c->B[off];
}

static void gemm_rows(void* p, uint64_t r0, uint64_t r1) {
  gemm_ctx* c = (gemm_ctx*)p;
  float* acc = (float*)malloc(sizeof(float) * (c->N ? c->N : 1));
  for (uint64_t m = r0; m < r1; ++m) {
    for (uint64_t n = 0; n < c->N; ++n) acc[n] = 0.0f;
    for (uint64_t k = 0; k < c->K; ++k) {
      const float a = ld_a(c, m, k);
      if (!c->b_nk && !c->B16) {
        const float* brow = c->B + k * c->N;
        for (uint64_t n = 0; n < c->N; ++n) acc[n] = acc[n] + a * brow[n];
      } else {
        for (uint64_t n = 0; n < c->N; ++n) acc[n] = acc[n] + a * ld_b(c, k, n);
      }
    }
    for (uint64_t n = 0; n < c->N; ++n) {
      float u = acc[n];
      if (c->epi == EPI_GELU) u = 0.5f * u * (1.0f + tanhf(0.79788456f * (u + 0.044715f * u * u * u)));
      else if (c->epi == EPI_SCALE) u = u * c->scale;
      c->C[m * c->N + n] = u;
    }
  }
  free(acc);
}

void oracle_gemm(const float* A, const float* B, const uint16_t* A16, const uint16_t* B16, uint32_t M, uint32_t N,
                 uint32_t K, int b_nk, int epi, float scale, float* C, int threads) {
  gemm_ctx c = {A, B, A16, B16, M, N, K, b_nk, epi, scale, C};
  parallel_rows(gemm_rows, &c, M, threads);
}

/* ---- reference suite, rank-3 reductions ------------------------------
 * out[i][j] = sum_k f(x, z) for the suite kernels; `middle` selects the
 * [R][K][C] layout of row_sum.cu:48-53 and softmax.cu:49-54, otherwise
 * [R][C][K] (dup_expr.cu:51-57, dup_const.cu:49-59, axpy3.cu:49-55,
 * scale_copy.cu:51-55, transpose.cu:45-50, layernorm.cu:46-54). */
enum {
  K_DUP_EXPR = 0,
  K_DUP_CONST = 1,
  K_AXPY3 = 2,
  K_SCALE_COPY = 3,
  K_ROW_SUM = 4,
  K_SOFTMAX_CORE = 5,
  K_TRANSPOSE = 6,
  K_LAYERNORM_RMS = 7
};

void oracle_suite_rank3(int kind, const float* x, const float* z, uint32_t R, uint32_t C, uint32_t K, int middle,
                        const float* s, float* out) {
  for (uint32_t i = 0; i < R; ++i) {
    for (uint32_t j = 0; j < C; ++j) {
      float acc = 0.0f;
      for (uint32_t k = 0; k < K; ++k) {
        const uint64_t off = middle ? ((uint64_t)i * K + k) * C + j : ((uint64_t)i * C + j) * K + k;
        const float v = x[off], w = z[off];
        float t;
        switch (kind) {
          case K_DUP_EXPR:
            t = ((v * v + v * v) * s[0] + (v * v + v * v) * s[1]) * w;
            break;
          case K_DUP_CONST:
            t = (0.5f * (v + 0.5f * v * v) * (1.0f + 0.044715f * v) +
                 tanhf(0.79788456f * (v + 0.044715f * v) + 0.79788456f * 0.5f * v) * (1.0f - 0.5f)) *
                w;
            break;
          case K_AXPY3:
            t = s[0] * v + s[1] * w;
            break;
          case K_SCALE_COPY:
            t = (s[0] * v + s[1]) * w;
            break;
          case K_SOFTMAX_CORE:
            t = expf(v) * w;
            break;
          case K_LAYERNORM_RMS:
            t = (v * v) * w;
            break;
          default: /* K_ROW_SUM, K_TRANSPOSE */
            t = v * w;
            break;
        }
        acc += t;
      }
      if (kind == K_AXPY3) acc = acc + s[2] * tanhf(acc);
      if (kind == K_LAYERNORM_RMS) acc = acc * (1.0f / sqrtf(acc * s[0] + s[1]));
      out[(uint64_t)i * C + j] = acc;
    }
  }
}
