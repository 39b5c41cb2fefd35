// capi_types.h — the objects behind the opaque handles of include/tca_cg.h,
// shared by the builder/emitter C ABI and the .tca frontend's C ABI (which
// hands out built builders).
#ifndef TCA_CG_CAPI_TYPES_H_
#define TCA_CG_CAPI_TYPES_H_

#include <string>

#include "builder.h"
#include "emit.h"
#include "ir.h"

struct tca_builder_s {
  explicit tca_builder_s(const char* name) : b(name ? name : "kernel") {}
  tca::pkg::Builder b;
  tca::ir::Graph built;
  bool is_built = false;
  std::string ir_text;  // the reference's canonical print
  std::string ir_full;  // this build's structural dump
  std::string expr_err;
  std::string err;
};

struct tca_emit_result_s {
  tca::cg::Result r;
};

#endif  // TCA_CG_CAPI_TYPES_H_
