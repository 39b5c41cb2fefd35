/*
 * tca_syntax.h — C ABI of the .tca text frontend.
 *
 * Reference interfaces this replaces:
 *   syntax.ParseModule(fset, path) -> *Module      internal/syntax/api.go:57-69
 *   Module{Kernels, Runtime, Source}                internal/syntax/api.go:21-28
 *   Kernel.Name() / Kernel.Build() -> *ir.Graph     internal/syntax/api.go:34-49
 *   parser.Parse (one file, no includes)            internal/syntax/parser/parser.go
 * A module is loaded, include-resolved and semantically checked in one call
 * that fails on the first batch of errors (warnings ride along); a kernel
 * then builds into an ordinary builder handle (tca_cg.h), already Build()-ed,
 * ready for tca_builder_ir and tca_emit. Nothing here needs a GPU.
 */
#ifndef TCA_SYNTAX_H_
#define TCA_SYNTAX_H_

#include <stdint.h>

#include "tca_cg.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tca_syntax_module_s* tca_syntax_module;

/* Loads the module rooted at path. On errors returns TCA_ERR_BUILD, *out is
 * NULL and tca_syntax_last_error() holds the diagnostics, one per line
 * ("file:line:col: error: message"). */
int tca_syntax_parse_module(const char* path, tca_syntax_module* out);
/* Parses source text held in memory (name labels diagnostics). check = 0
 * stops after parsing (the tree as written, for tca_syntax_module_dump); check = 1
 * also runs the module and kernel checks. @include is not resolved here. */
int tca_syntax_parse_source(const char* name, const char* src, int32_t check, tca_syntax_module* out);
/* Diagnostics of the last failed parse or build on this thread. */
const char* tca_syntax_last_error(void);

/* Warnings (and, for check = 0 parses, nothing else) of a loaded module. */
const char* tca_syntax_module_diagnostics(tca_syntax_module m);
uint32_t tca_syntax_module_kernel_count(tca_syntax_module m);
const char* tca_syntax_module_kernel_name(tca_syntax_module m, uint32_t i);
/* @name(cxx="...") of kernel i, or NULL. */
const char* tca_syntax_module_kernel_cxx_name(tca_syntax_module m, uint32_t i);
/* @runtime(cxx_path="...") of the module, or NULL. */
const char* tca_syntax_module_runtime_path(tca_syntax_module m);
/* Canonical indented rendering of the module's tree (owned by the module). */
const char* tca_syntax_module_dump(tca_syntax_module m);
/* Lowers kernel i through the builder rungs and builds it. On success *out
 * is a new builder (free with tca_builder_free). */
int tca_syntax_module_build_kernel(tca_syntax_module m, uint32_t i, tca_builder* out);
void tca_syntax_module_free(tca_syntax_module m);

#ifdef __cplusplus
}
#endif

#endif /* TCA_SYNTAX_H_ */
