/*
 * tcacomp — the compiler driver, over the C ABI only (include/tca_syntax.h,
 * include/tca_cg.h), so it is also what a cgo host would do step for step.
 *
 * Reference interface it replaces: cmd/tcacomp/main.go:28-113
 *   tcacomp compile [-o DIR] <input.tca>
 * parses and checks the module (syntax.ParseModule, main.go:71), compiles
 * every kernel (compiler.CompileKernel, main.go:101; here
 * tca_syntax_module_build_kernel + tca_emit), writes each kernel's files into
 * DIR and prints "tcacomp: compiled <kernel> -> <DIR>" (main.go:111). Like
 * the reference it emits code and a build recipe and does not drive the
 * device compiler itself.
 *
 * Files per kernel: <kernel>.hip (the generated code object source),
 * <kernel>.plan (the launch plan tca_program_load reads beside the code
 * object). One Makefile per run (the counterpart of the reference's
 * CMakeLists.txt, emit.go:186-189) builds <kernel>.hsaco for every kernel
 * with the emitter's own hipcc arguments; its TCA_INCLUDE defaults to the
 * device headers installed beside libtcacomp.so (csrc/include).
 *
 * Flags: -o DIR (default tcacomp-out, main.go:63), -target ARCH (default
 * gfx950, the only target the emitter accepts; -target=ARCH and --target
 * are accepted as Go's flag package does). Exit status: 0 ok, 1 a compile
 * or I/O error, 2 a usage error (main.go:30-46, 64-70).
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <errno.h>
#include <libgen.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include "tca_cg.h"
#include "tca_syntax.h"

static void usage(void) {
  fprintf(stderr,
          "usage:\n"
          "  tcacomp compile [flags] <input.tca>   compile a TCA source file to HIP code objects\n"
          "\n"
          "flags:\n"
          "  -o string\n"
          "    \toutput directory for the emitted `<name>.hip` + `<name>.plan` + `Makefile` (default \"tcacomp-out\")\n"
          "  -target string\n"
          "    \tdevice architecture (default \"gfx950\")\n");
}

/* Directory of the device headers the emitted sources include: csrc/include
 * beside the loaded libtcacomp.so. */
static int device_include_dir(char* out, size_t n) {
  Dl_info info;
  char path[4096];
  if (dladdr((void*)&tca_emit, &info) == 0 || info.dli_fname == NULL) return -1;
  if (strlen(info.dli_fname) >= sizeof path) return -1;
  strcpy(path, info.dli_fname);
  char* real = realpath(dirname(path), NULL);
  if (real == NULL) return -1;
  int w = snprintf(out, n, "%s/csrc/include", real);
  free(real);
  return (w > 0 && (size_t)w < n) ? 0 : -1;
}

/* 1 when path already holds exactly text. */
static int same_content(const char* path, const char* text, size_t len) {
  FILE* f = fopen(path, "rb");
  if (f == NULL) return 0;
  int same = 1;
  size_t at = 0;
  char buf[65536];
  size_t got;
  while (same && (got = fread(buf, 1, sizeof buf, f)) > 0) {
    same = at + got <= len && memcmp(buf, text + at, got) == 0;
    at += got;
  }
  fclose(f);
  return same && at == len;
}

/* Writes text to dir/name; a file that already holds it is left untouched
 * (its time stamp too), so a rerun leaves the Makefile nothing to rebuild. */
static int write_file(const char* dir, const char* name, const char* text) {
  char path[4096];
  if (snprintf(path, sizeof path, "%s/%s", dir, name) >= (int)sizeof path) {
    fprintf(stderr, "tcacomp: path too long: %s/%s\n", dir, name);
    return -1;
  }
  if (same_content(path, text, strlen(text))) return 0;
  FILE* f = fopen(path, "w");
  if (f == NULL) {
    fprintf(stderr, "tcacomp: write %s: %s\n", path, strerror(errno));
    return -1;
  }
  size_t len = strlen(text);
  int bad = fwrite(text, 1, len, f) != len;
  bad |= fclose(f) != 0;
  if (bad) {
    fprintf(stderr, "tcacomp: write %s: %s\n", path, strerror(errno));
    return -1;
  }
  return 0;
}

static int mkdir_p(const char* dir) {
  char buf[4096];
  size_t len = strlen(dir);
  if (len == 0 || len >= sizeof buf) return -1;
  memcpy(buf, dir, len + 1);
  for (size_t i = 1; i <= len; ++i) {
    if (buf[i] == '/' || buf[i] == '\0') {
      char c = buf[i];
      buf[i] = '\0';
      if (mkdir(buf, 0755) != 0 && errno != EEXIST) return -1;
      buf[i] = c;
    }
  }
  struct stat st;
  return (stat(dir, &st) == 0 && S_ISDIR(st.st_mode)) ? 0 : -1;
}

/* A hipcc argument as make passes it to the shell: plain words as they are,
 * anything else single-quoted. */
static void put_arg(FILE* f, const char* a) {
  int plain = *a != '\0';
  for (const char* p = a; *p; ++p)
    if (!(('a' <= *p && *p <= 'z') || ('A' <= *p && *p <= 'Z') || ('0' <= *p && *p <= '9') || strchr("-_=+./,:", *p)))
      plain = 0;
  if (plain) {
    fprintf(f, " %s", a);
    return;
  }
  fputs(" '", f);
  for (const char* p = a; *p; ++p) {
    if (*p == '\'') fputs("'\\''", f);
    else if (*p == '$') fputs("$$", f);
    else fputc(*p, f);
  }
  fputc('\'', f);
}

typedef struct {
  char* name;
  char** args;
  unsigned n_args;
} built_kernel;

static int write_makefile(const char* dir, const char* include_dir, const built_kernel* ks, unsigned n) {
  char path[4096];
  if (snprintf(path, sizeof path, "%s/Makefile", dir) >= (int)sizeof path) return -1;
  FILE* f = fopen(path, "w");
  if (f == NULL) {
    fprintf(stderr, "tcacomp: write %s: %s\n", path, strerror(errno));
    return -1;
  }
  fprintf(f, "# generated by tcacomp -- do not edit\n");
  fprintf(f, "# make -C <this directory>  ->  one <kernel>.hsaco per <kernel>.hip; load it with\n");
  fprintf(f, "# tca_program_load(<kernel>.hsaco, <contents of kernel>.plan>) (include/tca_rt.h).\n");
  fprintf(f, "HIPCC ?= /opt/rocm/bin/hipcc\n");
  fprintf(f, "TCA_INCLUDE ?= %s\n\n", include_dir);
  fprintf(f, "all:");
  for (unsigned i = 0; i < n; ++i) fprintf(f, " %s.hsaco", ks[i].name);
  fprintf(f, "\n\n");
  for (unsigned i = 0; i < n; ++i) {
    fprintf(f, "%s.hsaco: %s.hip\n\t$(HIPCC)", ks[i].name, ks[i].name);
    for (unsigned j = 0; j < ks[i].n_args; ++j) put_arg(f, ks[i].args[j]);
    fprintf(f, " -I $(TCA_INCLUDE) -o $@.tmp $< && mv $@.tmp $@\n\n");
  }
  fprintf(f, "clean:\n\trm -f");
  for (unsigned i = 0; i < n; ++i) fprintf(f, " %s.hsaco", ks[i].name);
  fprintf(f, "\n\n.PHONY: all clean\n");
  if (fclose(f) != 0) {
    fprintf(stderr, "tcacomp: write %s: %s\n", path, strerror(errno));
    return -1;
  }
  return 0;
}

/* Compiles kernel i of m into dir; fills *k with what the Makefile needs. */
static int compile_kernel(tca_syntax_module m, uint32_t i, const char* target, const char* dir, built_kernel* k) {
  const char* name = tca_syntax_module_kernel_name(m, i);
  tca_builder b = NULL;
  tca_emit_result r = NULL;
  char file[1024];
  int rc = 1;
  if (tca_syntax_module_build_kernel(m, i, &b) != TCA_OK) {
    fprintf(stderr, "tcacomp: kernel %s: %s\n", name, tca_syntax_last_error());
    return 1;
  }
  if (tca_emit(b, NULL, target, 0, &r) != TCA_OK) {
    fprintf(stderr, "tcacomp: kernel %s: %s\n", name, tca_builder_error(b));
    goto out;
  }
  snprintf(file, sizeof file, "%s.hip", name);
  if (write_file(dir, file, tca_emit_source(r)) != 0) goto out;
  snprintf(file, sizeof file, "%s.plan", name);
  if (write_file(dir, file, tca_emit_plan(r)) != 0) goto out;
  k->name = strdup(name);
  k->n_args = tca_emit_hipcc_argc(r);
  k->args = calloc(k->n_args ? k->n_args : 1, sizeof(char*));
  if (k->name == NULL || k->args == NULL) goto out;
  for (unsigned j = 0; j < k->n_args; ++j)
    if ((k->args[j] = strdup(tca_emit_hipcc_arg(r, j))) == NULL) goto out;
  printf("tcacomp: compiled %s -> %s\n", name, dir);
  rc = 0;
out:
  if (r) tca_emit_free(r);
  if (b) tca_builder_free(b);
  return rc;
}

static int compile(int argc, char** argv) {
  const char* out_dir = "tcacomp-out";
  const char* target = "gfx950";
  const char* input = NULL;
  int n_inputs = 0;
  for (int i = 0; i < argc; ++i) {
    const char* a = argv[i];
    if (n_inputs > 0 || strcmp(a, "-") == 0) { /* flags end at the first argument that is not one */
      input = a;
      ++n_inputs;
      continue;
    }
    if (strcmp(a, "--") == 0) {
      for (++i; i < argc; ++i) {
        input = argv[i];
        ++n_inputs;
      }
      break;
    }
    const char* flag = a;
    if (a[0] == '-' && a[1] == '-' && a[2] != '\0') flag = a + 1; /* --x reads as -x */
    const char** slot = NULL;
    const char* val = NULL;
    if (strcmp(flag, "-o") == 0 || strncmp(flag, "-o=", 3) == 0) slot = &out_dir;
    else if (strcmp(flag, "-target") == 0 || strncmp(flag, "-target=", 8) == 0) slot = &target;
    if (slot != NULL) {
      const char* eq = strchr(flag, '=');
      if (eq) val = eq + 1;
      else if (i + 1 < argc) val = argv[++i];
      else {
        fprintf(stderr, "flag needs an argument: %s\n", a);
        usage();
        return 2;
      }
      *slot = val;
    } else if (a[0] == '-') {
      fprintf(stderr, "flag provided but not defined: %s\n", a);
      usage();
      return 2;
    } else {
      input = a;
      ++n_inputs;
    }
  }
  if (n_inputs != 1) {
    fprintf(stderr, "tcacomp compile: exactly one input file required\n");
    return 2;
  }

  tca_syntax_module m = NULL;
  if (tca_syntax_parse_module(input, &m) != TCA_OK) {
    fprintf(stderr, "tcacomp: %s\n", tca_syntax_last_error());
    return 1;
  }
  const char* warnings = tca_syntax_module_diagnostics(m);
  if (warnings && *warnings) fputs(warnings, stderr);
  uint32_t n = tca_syntax_module_kernel_count(m);
  if (n == 0) {
    fprintf(stderr, "tcacomp: %s: no kernels\n", input);
    tca_syntax_module_free(m);
    return 1;
  }
  if (mkdir_p(out_dir) != 0) {
    fprintf(stderr, "tcacomp: create output dir: %s: %s\n", out_dir, strerror(errno));
    tca_syntax_module_free(m);
    return 1;
  }
  char include_dir[4096];
  if (device_include_dir(include_dir, sizeof include_dir) != 0) {
    fprintf(stderr, "tcacomp: cannot locate the device headers beside libtcacomp.so\n");
    tca_syntax_module_free(m);
    return 1;
  }
  built_kernel* ks = calloc(n, sizeof *ks);
  int rc = ks == NULL;
  unsigned done = 0;
  for (uint32_t i = 0; i < n && rc == 0; ++i) {
    rc = compile_kernel(m, i, target, out_dir, &ks[i]);
    if (rc == 0) ++done;
  }
  if (rc == 0) rc = write_makefile(out_dir, include_dir, ks, done) != 0;
  for (unsigned i = 0; ks && i < n; ++i) {
    for (unsigned j = 0; ks[i].args && j < ks[i].n_args; ++j) free(ks[i].args[j]);
    free(ks[i].args);
    free(ks[i].name);
  }
  free(ks);
  tca_syntax_module_free(m);
  return rc;
}

int main(int argc, char** argv) {
  if (argc < 2) {
    usage();
    return 2;
  }
  if (strcmp(argv[1], "compile") == 0) return compile(argc - 2, argv + 2);
  if (strcmp(argv[1], "help") == 0 || strcmp(argv[1], "-h") == 0 || strcmp(argv[1], "--help") == 0) {
    usage();
    return 0;
  }
  fprintf(stderr, "tcacomp: unknown command \"%s\"\n", argv[1]);
  usage();
  return 2;
}
