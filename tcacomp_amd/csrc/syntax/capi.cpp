// capi.cpp — extern "C" face of the .tca frontend (include/tca_syntax.h).
// No C++ exception crosses the ABI.
#include <string>

#include "../cg/capi_types.h"
#include "syntax.h"
#include "tca_syntax.h"

struct tca_syntax_module_s {
  tca::syntax::Module m;
  bool checked = false;
  std::string diagnostics;
  std::string dump;
};

namespace {

thread_local std::string g_last_error;

int Finish(tca::syntax::Module&& m, bool checked, const std::vector<tca::syntax::Diagnostic>& d, tca_syntax_module* out) {
  if (tca::syntax::HasErrors(d)) {
    g_last_error = "frontend:\n" + tca::syntax::JoinDiagnostics(d, true);
    return TCA_ERR_BUILD;
  }
  auto* h = new tca_syntax_module_s;
  h->m = std::move(m);
  h->checked = checked;
  h->diagnostics = tca::syntax::JoinDiagnostics(d, false);
  *out = h;
  return TCA_OK;
}

}  // namespace

extern "C" {

int tca_syntax_parse_module(const char* path, tca_syntax_module* out) {
  if (out == nullptr || path == nullptr) return TCA_ERR_INVALID;
  *out = nullptr;
  try {
    std::vector<tca::syntax::Diagnostic> d;
    tca::syntax::Module m = tca::syntax::Load(path, &d);
    return Finish(std::move(m), true, d, out);
  } catch (const std::exception& e) {
    g_last_error = std::string("internal error: ") + e.what();
    return TCA_ERR_BUILD;
  }
}

int tca_syntax_parse_source(const char* name, const char* src, int32_t check, tca_syntax_module* out) {
  if (out == nullptr || src == nullptr) return TCA_ERR_INVALID;
  *out = nullptr;
  try {
    std::vector<tca::syntax::Diagnostic> d;
    const std::string file = name ? name : "<source>";
    tca::syntax::Module m = tca::syntax::Parse(file, src, &d);
    if (check && !tca::syntax::HasErrors(d)) {
      for (const auto& inc : m.includes) {
        tca::syntax::Diagnostic x;
        x.pos = inc.pos;
        x.msg = "@include \"" + inc.path + "\" needs a file-backed module (tca_syntax_parse_module)";
        d.push_back(x);
      }
      tca::syntax::CheckModule(m, &d);
      for (auto& k : m.kernels) tca::syntax::Check(&k, &d);
    }
    return Finish(std::move(m), check != 0, d, out);
  } catch (const std::exception& e) {
    g_last_error = std::string("internal error: ") + e.what();
    return TCA_ERR_BUILD;
  }
}

const char* tca_syntax_last_error(void) { return g_last_error.c_str(); }

const char* tca_syntax_module_diagnostics(tca_syntax_module m) { return m ? m->diagnostics.c_str() : ""; }

uint32_t tca_syntax_module_kernel_count(tca_syntax_module m) { return m ? static_cast<uint32_t>(m->m.kernels.size()) : 0u; }

const char* tca_syntax_module_kernel_name(tca_syntax_module m, uint32_t i) {
  if (m == nullptr || i >= m->m.kernels.size()) return nullptr;
  return m->m.kernels[i].name.c_str();
}

const char* tca_syntax_module_kernel_cxx_name(tca_syntax_module m, uint32_t i) {
  if (m == nullptr || i >= m->m.kernels.size()) return nullptr;
  for (const auto& a : m->m.kernels[i].anns)
    if (a.name == "name")
      for (const auto& kc : a.args)
        if (kc.key == "cxx" && kc.kind == tca::syntax::ConstKind::String) return kc.text.c_str();
  return nullptr;
}

const char* tca_syntax_module_runtime_path(tca_syntax_module m) {
  if (m == nullptr || !m->m.has_runtime) return nullptr;
  for (const auto& kc : m->m.runtime.args)
    if (kc.key == "cxx_path" && kc.kind == tca::syntax::ConstKind::String) return kc.text.c_str();
  return nullptr;
}

const char* tca_syntax_module_dump(tca_syntax_module m) {
  if (m == nullptr) return nullptr;
  try {
    m->dump = tca::syntax::Dump(m->m);
  } catch (...) {
    return nullptr;
  }
  return m->dump.c_str();
}

int tca_syntax_module_build_kernel(tca_syntax_module m, uint32_t i, tca_builder* out) {
  if (m == nullptr || out == nullptr || i >= m->m.kernels.size()) return TCA_ERR_INVALID;
  *out = nullptr;
  if (!m->checked) {
    g_last_error = "frontend: the module was parsed without checks; build needs a checked module";
    return TCA_ERR_BUILD;
  }
  tca_builder_s* b = nullptr;
  try {
    const tca::syntax::Kernel& k = m->m.kernels[i];
    b = new tca_builder_s(k.name.c_str());
    std::string err;
    if (!tca::syntax::Lower(k, &b->b, &err)) {
      g_last_error = err;
      delete b;
      return TCA_ERR_BUILD;
    }
    if (!b->b.Build(&b->built)) {
      g_last_error = "frontend: kernel " + k.name + ": " + b->b.Error();
      delete b;
      return TCA_ERR_BUILD;
    }
    b->is_built = true;
    b->ir_text = tca::ir::PrintReference(b->built);
    b->ir_full = tca::ir::Print(b->built);
    *out = b;
    return TCA_OK;
  } catch (const std::exception& e) {
    delete b;
    g_last_error = std::string("internal error: ") + e.what();
    return TCA_ERR_BUILD;
  }
}

void tca_syntax_module_free(tca_syntax_module m) { delete m; }

}  // extern "C"
