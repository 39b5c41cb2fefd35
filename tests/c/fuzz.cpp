// fuzz.cpp — a bounded, seeded mutation fuzzer of the library's two text
// inputs, run on the CPU against the AddressSanitizer + UBSan build of
// libtcacomp.so (tests/sanitize.py builds both and runs it). Test program,
// not part of the library.
//
//   fuzz plan <iterations> <seconds> <seed> <out-dir> <corpus file>...
//       mutates launch plans (the emitter's .plan files) and feeds each to
//       tca_program_parse; a plan that parses is printed back
//       (tca_program_plan_text) and parsed again, then bound and queried
//       (tca_program_check, tca_program_selected, tca_program_kernel_args)
//       with tensors shaped after
//       its own tensor records, dims drawn from 0, 1, small, ragged and u32
//       extremes.
//   fuzz tca <iterations> <seconds> <seed> <out-dir> <corpus file>...
//       mutates .tca sources and feeds each to tca_syntax_parse_source; every
//       kernel of a module that parses is built through the builder rungs
//       and, when it builds, emitted (tca_emit).
//
// Before each input is used it is written to <out-dir>/current.<mode>, so
// the input of a run that a sanitizer ends is on disk. The fuzzer stops at
// the first finding: a sanitizer report aborts the process (halt_on_error,
// no UBSan recovery), and any other crash ends it too. A run that ends
// normally prints "ok <mode> <iterations> inputs, <parsed> parsed".
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <sstream>
#include <string>
#include <vector>

#include "tca_cg.h"
#include "tca_rt.h"
#include "tca_syntax.h"

namespace {

struct Rng {  // splitmix64
  uint64_t s;
  uint64_t next() {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  uint32_t below(uint32_t n) { return n ? static_cast<uint32_t>(next() % n) : 0u; }
};

std::string read_file(const char* path) {
  std::ifstream f(path, std::ios::binary);
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

void write_file(const std::string& path, const std::string& text) {
  std::ofstream f(path, std::ios::binary | std::ios::trunc);
  f << text;
}

std::vector<std::string> lines_of(const std::string& t) {
  std::vector<std::string> out;
  std::string cur;
  for (char c : t) {
    if (c == '\n') {
      out.push_back(cur);
      cur.clear();
    } else {
      cur += c;
    }
  }
  if (!cur.empty()) out.push_back(cur);
  return out;
}

std::string join(const std::vector<std::string>& ls) {
  std::string out;
  for (const auto& l : ls) out += l + "\n";
  return out;
}

// One to four edits: byte flips, dictionary tokens inserted or replacing a
// word, deletions, line duplication, swap, removal and truncation, numbers
// replaced by boundary values.
std::string mutate(const std::string& in, const std::vector<std::string>& dict, Rng& r) {
  std::string t = in;
  const uint32_t edits = 1 + r.below(4);
  for (uint32_t e = 0; e < edits; ++e) {
    switch (r.below(9)) {
      case 0:
        if (!t.empty()) t[r.below(static_cast<uint32_t>(t.size()))] ^= static_cast<char>(1u << r.below(8));
        break;
      case 1:
        t.insert(r.below(static_cast<uint32_t>(t.size() + 1)), dict[r.below(static_cast<uint32_t>(dict.size()))]);
        break;
      case 2: {
        if (t.empty()) break;
        const uint32_t a = r.below(static_cast<uint32_t>(t.size()));
        t.erase(a, 1 + r.below(16));
        break;
      }
      case 3: {
        auto ls = lines_of(t);
        if (ls.empty()) break;
        const uint32_t i = r.below(static_cast<uint32_t>(ls.size()));
        ls.insert(ls.begin() + i, ls[i]);
        t = join(ls);
        break;
      }
      case 4: {
        auto ls = lines_of(t);
        if (ls.size() < 2) break;
        std::swap(ls[r.below(static_cast<uint32_t>(ls.size()))], ls[r.below(static_cast<uint32_t>(ls.size()))]);
        t = join(ls);
        break;
      }
      case 5: {
        auto ls = lines_of(t);
        if (ls.empty()) break;
        ls.erase(ls.begin() + r.below(static_cast<uint32_t>(ls.size())));
        t = join(ls);
        break;
      }
      case 6:
        t.resize(r.below(static_cast<uint32_t>(t.size() + 1)));
        break;
      case 7: {  // a number replaced by a boundary value
        static const char* nums[] = {"0", "1", "2", "7", "64", "255", "256", "4095", "4096", "65535", "2147483647",
                                     "2147483648", "4294967295", "4294967296", "18446744073709551615",
                                     "18446744073709551616", "-1", "99999999999999999999999"};
        std::vector<size_t> starts;
        for (size_t i = 0; i < t.size(); ++i)
          if (t[i] >= '0' && t[i] <= '9' && (i == 0 || t[i - 1] < '0' || t[i - 1] > '9')) starts.push_back(i);
        if (starts.empty()) break;
        const size_t a = starts[r.below(static_cast<uint32_t>(starts.size()))];
        size_t b = a;
        while (b < t.size() && t[b] >= '0' && t[b] <= '9') ++b;
        t.replace(a, b - a, nums[r.below(sizeof nums / sizeof nums[0])]);
        break;
      }
      default: {  // a word replaced by a dictionary token
        std::vector<size_t> starts;
        for (size_t i = 0; i < t.size(); ++i)
          if (t[i] != ' ' && t[i] != '\n' && (i == 0 || t[i - 1] == ' ' || t[i - 1] == '\n')) starts.push_back(i);
        if (starts.empty()) break;
        const size_t a = starts[r.below(static_cast<uint32_t>(starts.size()))];
        size_t b = a;
        while (b < t.size() && t[b] != ' ' && t[b] != '\n') ++b;
        t.replace(a, b - a, dict[r.below(static_cast<uint32_t>(dict.size()))]);
        break;
      }
    }
  }
  return t;
}

uint32_t draw_dim(Rng& r) {
  static const uint32_t vals[] = {0u, 1u, 2u, 3u, 7u, 31u, 32u, 33u, 64u, 255u, 256u, 1000u, 4096u, 65536u,
                                  1u << 20, 4294967295u, 4294967294u, 65537u};
  return vals[r.below(sizeof vals / sizeof vals[0])];
}

// Tensors shaped after the plan's own tensor records (each dim name one
// value), so the shape contract often holds and the guards, grids and
// split formulas see boundary dims.
int query_plan(tca_program p, const std::string& text, Rng& r) {
  uint32_t nt = 0, nf = 0, ns = 0, nk = 0;
  if (tca_program_signature(p, &nt, &nf, &ns, &nk) != TCA_OK) return 0;
  std::map<std::string, uint32_t> dimval;
  std::vector<tca_tensor> ts;
  static char backing[64] __attribute__((aligned(16)));  // never dereferenced: host-only queries
  for (const auto& l : lines_of(text)) {
    std::istringstream ls(l);
    std::string kw, name, dtype, role;
    uint64_t rank = 0;
    if (!(ls >> kw) || kw != "tensor") continue;
    if (!(ls >> name >> dtype >> role >> rank) || role == "local" || rank > TCA_MAX_RANK) continue;
    tca_tensor t;
    std::memset(&t, 0, sizeof t);
    t.data = backing;
    t.rank = static_cast<uint32_t>(rank);
    static const char* names[] = {"f32", "f16", "bf16", "i32", "u32", "i8", "i16", "u8", "u16", "bool"};
    t.dtype = TCA_F32;
    for (int i = 0; i < 10; ++i)
      if (dtype == names[i]) t.dtype = i;
    for (uint64_t a = 0; a < rank; ++a) {
      std::string dn;
      if (!(ls >> dn)) break;
      if (!dimval.count(dn)) dimval[dn] = draw_dim(r);
      t.dims[a] = dimval[dn];
    }
    ts.push_back(t);
  }
  if (ts.size() != nt) ts.resize(nt);  // the contract then fails cleanly
  std::vector<uint32_t> fd(nf + 1);
  for (auto& d : fd) d = draw_dim(r);
  (void)tca_program_check(p, ts.data(), nt, fd.data(), nf);
  std::vector<uint8_t> sel(nk + 1);
  std::vector<uint64_t> grids(nk + 1);
  std::vector<uint32_t> blocks(nk + 1);
  (void)tca_program_selected(p, ts.data(), nt, fd.data(), nf, sel.data(), grids.data(), blocks.data(), nk);
  std::vector<double> sc(ns + 1, 0.5);
  unsigned char blob[512];
  for (uint32_t i = 0; i < nk; ++i) {
    (void)tca_program_kernel_name(p, i);
    size_t size = 0;
    (void)tca_program_kernel_args(p, ts.data(), nt, fd.data(), nf, sc.data(), ns, i, blob, r.below(2) ? sizeof blob : 8,
                                  &size);
  }
  return 1;
}

int fuzz_plan(const std::string& text, Rng& r) {
  tca_program p = nullptr;
  if (tca_program_parse(text.c_str(), &p) != TCA_OK) return 0;
  const std::string printed = tca_program_plan_text(p);
  tca_program q = nullptr;
  if (tca_program_parse(printed.c_str(), &q) != TCA_OK) {
    std::fprintf(stderr, "FINDING: a printed plan does not parse again: %s\n--- printed ---\n%s", tca_rt_last_error(),
                 printed.c_str());
    std::abort();
  }
  if (printed != tca_program_plan_text(q)) {
    std::fprintf(stderr, "FINDING: a printed plan prints differently\n");
    std::abort();
  }
  Rng r2 = r;
  query_plan(p, text, r);
  query_plan(q, printed, r2);
  tca_program_unload(q);
  tca_program_unload(p);
  return 1;
}

int fuzz_tca(const std::string& text) {
  tca_syntax_module m = nullptr;
  if (tca_syntax_parse_source("fuzz.tca", text.c_str(), 1, &m) != TCA_OK) return 0;  // with the semantic checks
  (void)tca_syntax_module_diagnostics(m);
  (void)tca_syntax_module_dump(m);
  const uint32_t n = tca_syntax_module_kernel_count(m);
  for (uint32_t i = 0; i < n; ++i) {
    (void)tca_syntax_module_kernel_name(m, i);
    tca_builder b = nullptr;
    if (tca_syntax_module_build_kernel(m, i, &b) != TCA_OK) continue;
    (void)tca_builder_ir(b);
    tca_emit_result e = nullptr;
    if (tca_emit(b, nullptr, "gfx950", 0, &e) == TCA_OK) {
      (void)tca_emit_source(e);
      (void)tca_emit_plan(e);
      tca_emit_free(e);
    }
    tca_builder_free(b);
  }
  tca_syntax_module_free(m);
  return 1;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 7 || (std::strcmp(argv[1], "plan") != 0 && std::strcmp(argv[1], "tca") != 0)) {
    std::fprintf(stderr, "usage: %s plan|tca <iterations> <seconds> <seed> <out-dir> <corpus file>...\n", argv[0]);
    return 2;
  }
  const std::string mode = argv[1];
  const uint64_t iters = std::strtoull(argv[2], nullptr, 10);
  const double seconds = std::atof(argv[3]);
  Rng r{std::strtoull(argv[4], nullptr, 10)};
  const std::string cur = std::string(argv[5]) + "/current." + mode;
  std::vector<std::string> corpus;
  for (int i = 6; i < argc; ++i) corpus.push_back(read_file(argv[i]));
  const std::vector<std::string> plan_dict = {
      "kernel ", "arg ptr ", "arg dim ", "arg scalar ", "dim ", "tensor ", "scalar ", "split ", "when ", "unless ",
      "pack ", "program ", "end", "tca-plan 1", " pow2", "*", "/", ":", "/pack", " local ", " in ", " out ", " bf16 ",
      " u8 ", "M*N", "#", "\n", " 0 ", " 4294967295 "};
  const std::vector<std::string> tca_dict = {
      "kernel ", "let ", "return ", "map", "reduce", "iter", "as", "|", "(", ")", "[", "]", "{", "}", "<", ">", "->",
      ";", ",", ":", "f32", "bf16", "u8", "u32", "i32", "expf", "fmaxf", "rsqrtf", "select", "0", "1.5", "-0.0",
      "@include \"x.tca\"", "\n", "\"", "/*", "*/", "//", "<<", ">>"};
  const auto& dict = mode == "plan" ? plan_dict : tca_dict;
  const auto t0 = std::chrono::steady_clock::now();
  uint64_t done = 0, ok = 0;
  for (; done < iters; ++done) {
    if (std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() > seconds) break;
    const std::string in = mutate(corpus[r.below(static_cast<uint32_t>(corpus.size()))], dict, r);
    write_file(cur, in);
    ok += mode == "plan" ? fuzz_plan(in, r) : fuzz_tca(in);
  }
  std::printf("ok %s %llu inputs, %llu parsed\n", mode.c_str(), static_cast<unsigned long long>(done),
              static_cast<unsigned long long>(ok));
  return 0;
}
