// plan.cpp — parse, bind and pack a launch plan (format in plan.h).
#include "plan.h"

#include <limits>

#include <algorithm>

#include <cstring>
#include <sstream>

namespace tca {
namespace plan {

namespace {

const char* kDtypeNames[] = {"f32", "f16", "bf16", "i32", "u32", "i8", "i16", "u8", "u16", "bool"};
const size_t kDtypeBytes[] = {4, 2, 2, 4, 4, 1, 2, 1, 2, 1};

int FindDim(const Plan& p, const std::string& n) {
  for (size_t i = 0; i < p.dims.size(); ++i)
    if (p.dims[i].name == n) return static_cast<int>(i);
  return -1;
}
int FindTensor(const Plan& p, const std::string& n) {
  for (size_t i = 0; i < p.tensors.size(); ++i)
    if (p.tensors[i].name == n) return static_cast<int>(i);
  return -1;
}
int FindScalar(const Plan& p, const std::string& n) {
  for (size_t i = 0; i < p.scalars.size(); ++i)
    if (p.scalars[i].name == n) return static_cast<int>(i);
  return -1;
}

bool ParseU64(const std::string& s, uint64_t* v) {
  if (s.empty()) return false;
  uint64_t x = 0;
  for (char c : s) {
    if (c < '0' || c > '9') return false;
    uint64_t nx = x * 10 + static_cast<uint64_t>(c - '0');
    if (nx / 10 != x) return false;
    x = nx;
  }
  *v = x;
  return true;
}

bool ParseTerm(const Plan& p, const std::string& s, Term* t, std::string* err) {
  size_t slash = s.find('/');
  if (slash == std::string::npos) {
    *err = "grid term '" + s + "' lacks a '/divisor'";
    return false;
  }
  const size_t colon = s.find(':', slash);
  if (colon != std::string::npos && (!ParseU64(s.substr(colon + 1), &t->cap) || t->cap == 0)) {
    *err = "grid term '" + s + "' has a bad cap";
    return false;
  }
  const std::string div = s.substr(slash + 1, colon == std::string::npos ? std::string::npos : colon - slash - 1);
  if (div == "pack") {
    t->packed = true;  // rows per block of the kernel's pack record
  } else if (!ParseU64(div, &t->divisor) || t->divisor == 0) {
    *err = "grid term '" + s + "' has a bad divisor";
    return false;
  }
  std::string prod = s.substr(0, slash);
  size_t start = 0;
  while (start <= prod.size()) {
    size_t star = prod.find('*', start);
    std::string f = prod.substr(start, star == std::string::npos ? std::string::npos : star - start);
    uint64_t c = 0;
    if (ParseU64(f, &c)) {
      t->const_factor *= c;
    } else {
      int d = FindDim(p, f);
      if (d < 0) {
        *err = "grid term '" + s + "' names unknown dim '" + f + "'";
        return false;
      }
      t->dim_factors.push_back(d);
    }
    if (star == std::string::npos) break;
    start = star + 1;
  }
  return true;
}

}  // namespace

size_t DtypeBytes(int dtype) {
  if (dtype < 0 || dtype > TCA_BOOL) return 0;
  return kDtypeBytes[dtype];
}

const char* DtypeName(int dtype) {
  if (dtype < 0 || dtype > TCA_BOOL) return "?";
  return kDtypeNames[dtype];
}

int DtypeFromName(const std::string& s) {
  for (int i = 0; i <= TCA_BOOL; ++i)
    if (s == kDtypeNames[i]) return i;
  return -1;
}

size_t Plan::ParamTensorCount() const {
  size_t n = 0;
  for (const auto& t : tensors)
    if (t.role != Role::Local) ++n;
  return n;
}

std::vector<int> Plan::FreeDims() const {
  std::vector<bool> carried(dims.size(), false);
  for (const auto& t : tensors) {
    if (t.role == Role::Local) continue;
    for (int d : t.dims) carried[d] = true;
  }
  std::vector<int> out;
  for (size_t i = 0; i < dims.size(); ++i)
    if (dims[i].extent == 0 && !carried[i]) out.push_back(static_cast<int>(i));
  return out;
}

bool Parse(const std::string& text, Plan* out, std::string* err) {
  Plan p;
  std::istringstream in(text);
  std::string line;
  bool header = false, ended = false;
  int lineno = 0;
  auto bad = [&](const std::string& m) {
    *err = "line " + std::to_string(lineno) + ": " + m;
    return false;
  };
  while (std::getline(in, line)) {
    ++lineno;
    size_t hash = line.find('#');
    if (hash != std::string::npos) line = line.substr(0, hash);
    std::istringstream ls(line);
    std::vector<std::string> tok;
    std::string w;
    while (ls >> w) tok.push_back(w);
    if (tok.empty()) continue;
    if (ended) return bad("text after 'end'");
    const std::string& kw = tok[0];
    if (!header) {
      if (kw != "tca-plan" || tok.size() != 2 || tok[1] != "1") return bad("expected 'tca-plan 1'");
      header = true;
      continue;
    }
    if (kw == "program") {
      if (tok.size() != 2) return bad("program <name>");
      if (!p.name.empty()) return bad("duplicate program record");
      p.name = tok[1];
    } else if (kw == "dim") {
      uint64_t e = 0;
      if (tok.size() != 3 || !ParseU64(tok[2], &e)) return bad("dim <name> <extent>");
      if (e > 0xffffffffull) return bad("dim extent exceeds u32");
      if (FindDim(p, tok[1]) >= 0) return bad("duplicate dim " + tok[1]);
      p.dims.push_back({tok[1], e});
    } else if (kw == "tensor") {
      uint64_t rank = 0;
      if (tok.size() < 5 || !ParseU64(tok[4], &rank) || tok.size() != 5 + rank)
        return bad("tensor <name> <dtype> <role> <rank> <dims...>");
      if (rank > TCA_MAX_RANK) return bad("tensor rank exceeds TCA_MAX_RANK");
      Tensor t;
      t.name = tok[1];
      t.dtype = DtypeFromName(tok[2]);
      if (t.dtype < 0) return bad("unknown dtype " + tok[2]);
      if (tok[3] == "in") t.role = Role::In;
      else if (tok[3] == "out") t.role = Role::Out;
      else if (tok[3] == "local") t.role = Role::Local;
      else return bad("unknown tensor role " + tok[3]);
      for (uint64_t i = 0; i < rank; ++i) {
        int d = FindDim(p, tok[5 + i]);
        if (d < 0) return bad("tensor " + t.name + " names unknown dim " + tok[5 + i]);
        t.dims.push_back(d);
      }
      if (FindTensor(p, t.name) >= 0) return bad("duplicate tensor " + t.name);
      p.tensors.push_back(t);
    } else if (kw == "scalar") {
      if (tok.size() != 3) return bad("scalar <name> <dtype>");
      Scalar s{tok[1], DtypeFromName(tok[2])};
      if (s.dtype < 0) return bad("unknown dtype " + tok[2]);
      p.scalars.push_back(s);
    } else if (kw == "kernel") {
      uint64_t block = 0, lds = 0, nterms = 0;
      if (tok.size() < 5 || !ParseU64(tok[2], &block) || !ParseU64(tok[3], &lds) || !ParseU64(tok[4], &nterms) ||
          tok.size() != 5 + nterms)
        return bad("kernel <symbol> <block> <lds> <n-terms> <terms...>");
      Kernel k;
      k.symbol = tok[1];
      k.block = static_cast<uint32_t>(block);
      k.lds = static_cast<uint32_t>(lds);
      for (uint64_t i = 0; i < nterms; ++i) {
        Term t;
        std::string e;
        if (!ParseTerm(p, tok[5 + i], &t, &e)) return bad(e);
        k.grid.push_back(t);
      }
      p.kernels.push_back(k);
    } else if (kw == "arg") {
      if (p.kernels.empty()) return bad("arg before any kernel");
      if (tok.size() != 3) return bad("arg <ptr|dim|scalar> <name>");
      Arg a;
      if (tok[1] == "ptr") {
        a.kind = ArgKind::Ptr;
        a.index = FindTensor(p, tok[2]);
      } else if (tok[1] == "dim") {
        a.kind = ArgKind::Dim;
        a.index = FindDim(p, tok[2]);
      } else if (tok[1] == "scalar") {
        a.kind = ArgKind::Scalar;
        a.index = FindScalar(p, tok[2]);
      } else {
        return bad("unknown arg kind " + tok[1]);
      }
      if (a.index < 0) return bad("arg names unknown " + tok[1] + " " + tok[2]);
      p.kernels.back().args.push_back(a);
    } else if (kw == "pack") {
      if (p.kernels.empty()) return bad("pack before any kernel");
      Kernel& k = p.kernels.back();
      if (tok.size() != 4 || !ParseU64(tok[2], &k.pack_epl) || !ParseU64(tok[3], &k.pack_min_block))
        return bad("pack <dim> <elements per lane> <min block>");
      k.pack_dim = FindDim(p, tok[1]);
      if (k.pack_dim < 0) return bad("pack names unknown dim " + tok[1]);
      if (k.pack_epl == 0 || k.pack_min_block == 0 || k.pack_min_block > k.block || (k.block & (k.block - 1)) != 0 ||
          k.pack_min_block % 64 != 0)
        return bad("bad pack on " + tok[1] + " (power-of-two block, 64 <= min block <= block)");
    } else if (kw == "split") {
      if (p.kernels.empty()) return bad("split before any kernel");
      Kernel& k = p.kernels.back();
      uint64_t merge = 0, nt = 0;
      if (tok.size() < 6 || !ParseU64(tok[2], &k.split_rows_min) || !ParseU64(tok[3], &k.split_blocks) ||
          !ParseU64(tok[4], &merge) || !ParseU64(tok[5], &nt) || tok.size() != 6 + nt)
        return bad("split <dim> <rows-min> <blocks> <mode> <n-terms> <term>...");
      k.split_dim = FindDim(p, tok[1]);
      if (k.split_dim < 0) return bad("split names unknown dim " + tok[1]);
      if (k.split_rows_min == 0 || k.split_blocks == 0 || merge > kSplitPartialMany)
        return bad("bad split on " + tok[1]);
      k.split_mode = static_cast<int>(merge);
      for (uint64_t i = 0; i < nt; ++i) {
        Term t;
        std::string e;
        if (!ParseTerm(p, tok[6 + i], &t, &e)) return bad(e);
        if (t.packed) return bad("a split term cannot divide by 'pack'");
        k.split_terms.push_back(t);
      }
    } else if (kw == "when" || kw == "unless") {
      if (p.kernels.empty()) return bad(kw + " before any kernel");
      Guard g;
      g.pow2 = tok.size() == 7 && tok[6] == "pow2";
      if ((tok.size() != 6 && !g.pow2) || !ParseU64(tok[2], &g.lo) || !ParseU64(tok[3], &g.hi) ||
          !ParseU64(tok[4], &g.mod) || !ParseU64(tok[5], &g.rem))
        return bad(kw + " <dim> <lo> <hi> <mod> <rem> [pow2]");
      for (size_t start = 0;;) {  // d1*d2*...: the product of the named dims
        const size_t star = tok[1].find('*', start);
        const std::string dn = tok[1].substr(start, star == std::string::npos ? std::string::npos : star - start);
        const int d = FindDim(p, dn);
        if (d < 0) return bad(kw + " names unknown dim " + dn);
        g.dims.push_back(d);
        if (star == std::string::npos) break;
        start = star + 1;
      }
      if (g.mod == 0 || g.rem >= g.mod || g.lo > g.hi || (g.pow2 && g.rem != 0)) return bad("bad guard on " + tok[1]);
      (kw == "when" ? p.kernels.back().when : p.kernels.back().unless).push_back(g);
    } else if (kw == "end") {
      ended = true;
    } else {
      return bad("unknown record '" + kw + "'");
    }
  }
  if (!header) return bad("empty plan");
  if (!ended) return bad("missing 'end'");
  if (p.name.empty()) return bad("plan has no program record");
  if (p.kernels.empty()) return bad("plan has no kernel");
  for (const auto& k : p.kernels)
    for (const auto& t : k.grid)
      if (t.packed && k.pack_dim < 0) {
        *err = "kernel " + k.symbol + ": grid divisor 'pack' needs a pack record";
        return false;
      }
  *out = p;
  return true;
}

namespace {

std::string TermText(const Plan& p, const Term& t) {
  std::ostringstream o;
  bool first = true;
  if (t.const_factor != 1 || t.dim_factors.empty()) {
    o << t.const_factor;
    first = false;
  }
  for (int d : t.dim_factors) {
    if (!first) o << "*";
    o << p.dims[d].name;
    first = false;
  }
  if (t.packed) o << "/pack";
  else o << "/" << t.divisor;
  if (t.cap != 0) o << ":" << t.cap;
  return o.str();
}

// ceil(product of the term's factors / divisor), limited to the cap; the
// divisor of a packed term is the kernel's rows per block.
uint64_t TermValue(const Kernel& k, const Term& t, const std::vector<uint32_t>& dims, bool* overflow) {
  uint64_t prod = t.const_factor;
  for (int d : t.dim_factors) {
    prod *= dims[d];
    if (prod > (1ull << 62)) {
      *overflow = true;
      return 0;
    }
  }
  uint64_t div = t.divisor;
  if (t.packed) {
    uint32_t block = 0;
    div = PackRows(k, dims, &block);
  }
  uint64_t q = (prod + div - 1) / div;
  if (t.cap != 0 && q > t.cap) q = t.cap;
  return q;
}

std::string GuardText(const Plan& p, const Guard& g) {
  std::ostringstream o;
  for (size_t i = 0; i < g.dims.size(); ++i) o << (i ? "*" : "") << p.dims[g.dims[i]].name;
  o << " " << g.lo << " " << g.hi << " " << g.mod << " " << g.rem;
  if (g.pow2) o << " pow2";
  return o.str();
}

}  // namespace

std::string Serialize(const Plan& p) {
  std::ostringstream o;
  o << "tca-plan 1\nprogram " << p.name << "\n";
  for (const auto& d : p.dims) o << "dim " << d.name << " " << d.extent << "\n";
  for (const auto& t : p.tensors) {
    o << "tensor " << t.name << " " << DtypeName(t.dtype) << " "
      << (t.role == Role::In ? "in" : t.role == Role::Out ? "out" : "local") << " " << t.dims.size();
    for (int d : t.dims) o << " " << p.dims[d].name;
    o << "\n";
  }
  for (const auto& s : p.scalars) o << "scalar " << s.name << " " << DtypeName(s.dtype) << "\n";
  for (const auto& k : p.kernels) {
    o << "kernel " << k.symbol << " " << k.block << " " << k.lds << " " << k.grid.size();
    for (const auto& t : k.grid) o << " " << TermText(p, t);
    o << "\n";
    for (const auto& a : k.args) {
      if (a.kind == ArgKind::Ptr) o << "arg ptr " << p.tensors[a.index].name << "\n";
      else if (a.kind == ArgKind::Dim) o << "arg dim " << p.dims[a.index].name << "\n";
      else o << "arg scalar " << p.scalars[a.index].name << "\n";
    }
    if (k.pack_dim >= 0)
      o << "pack " << p.dims[k.pack_dim].name << " " << k.pack_epl << " " << k.pack_min_block << "\n";
    if (k.split_dim >= 0) {
      o << "split " << p.dims[k.split_dim].name << " " << k.split_rows_min << " " << k.split_blocks << " "
        << k.split_mode << " " << k.split_terms.size();
      for (const auto& t : k.split_terms) o << " " << TermText(p, t);
      o << "\n";
    }
    for (const auto& g : k.when) o << "when " << GuardText(p, g) << "\n";
    for (const auto& g : k.unless) o << "unless " << GuardText(p, g) << "\n";
  }
  o << "end\n";
  return o.str();
}

int Bind(const Plan& p, const tca_tensor* tensors, uint32_t n_tensors, const uint32_t* free_dims,
         uint32_t n_free_dims, std::vector<uint32_t>* dims, std::string* err) {
  const size_t want = p.ParamTensorCount();
  if (n_tensors != want) {
    *err = "program " + p.name + " takes " + std::to_string(want) + " tensor(s), got " + std::to_string(n_tensors);
    return TCA_ERR_INVALID;
  }
  if (want > 0 && tensors == nullptr) {
    *err = "null tensor array";
    return TCA_ERR_INVALID;
  }
  std::vector<int> free = p.FreeDims();
  if (n_free_dims != free.size()) {
    *err = "program " + p.name + " takes " + std::to_string(free.size()) + " free dim(s), got " +
           std::to_string(n_free_dims);
    return TCA_ERR_INVALID;
  }
  if (!free.empty() && free_dims == nullptr) {
    *err = "null free-dim array";
    return TCA_ERR_INVALID;
  }
  dims->assign(p.dims.size(), 0);
  std::vector<bool> known(p.dims.size(), false);
  std::vector<std::string> supplier(p.dims.size());
  for (size_t i = 0; i < p.dims.size(); ++i) {
    if (p.dims[i].extent > 0) {
      (*dims)[i] = static_cast<uint32_t>(p.dims[i].extent);
      known[i] = true;
      supplier[i] = "its const extent";
    }
  }
  for (size_t i = 0; i < free.size(); ++i) {
    (*dims)[free[i]] = free_dims[i];
    known[free[i]] = true;
    supplier[free[i]] = "the free-dim argument";
  }
  uint32_t ti = 0;
  for (const auto& t : p.tensors) {
    if (t.role == Role::Local) continue;
    const tca_tensor& a = tensors[ti++];
    if (a.rank != t.dims.size()) {
      *err = "tensor " + t.name + " has rank " + std::to_string(a.rank) + ", the program declares " +
             std::to_string(t.dims.size());
      return TCA_ERR_SHAPE;
    }
    if (a.dtype != t.dtype) {
      *err = std::string("tensor ") + t.name + " has dtype " + DtypeName(a.dtype) + ", the program declares " +
             DtypeName(t.dtype);
      return TCA_ERR_SHAPE;
    }
    // Elements, saturated at kMaxElems + 1 (three u32 extents can overflow
    // 64 bits); an extent of 0 makes the tensor empty whatever the others.
    uint64_t elems = 1;
    bool empty = false;
    for (size_t ax = 0; ax < t.dims.size(); ++ax) {
      const int d = t.dims[ax];
      if (a.dims[ax] == 0)
        empty = true;
      else
        elems = elems > kMaxElems / a.dims[ax] ? kMaxElems + 1 : elems * a.dims[ax];
      if (!known[d]) {
        (*dims)[d] = a.dims[ax];
        known[d] = true;
        supplier[d] = t.name + ".Dim(" + std::to_string(ax) + ")";
      } else if ((*dims)[d] != a.dims[ax]) {
        *err = t.name + ".Dim(" + std::to_string(ax) + ") = " + std::to_string(a.dims[ax]) + " must equal " +
               p.dims[d].name + " = " + std::to_string((*dims)[d]) + " (from " + supplier[d] + ")";
        return TCA_ERR_SHAPE;
      }
    }
    if (empty) elems = 0;
    if (elems > 0 && a.data == nullptr) {
      *err = "tensor " + t.name + " has a null data pointer";
      return TCA_ERR_INVALID;
    }
    if (elems > 0 && (reinterpret_cast<uintptr_t>(a.data) % 16u) != 0u) {
      *err = "tensor " + t.name + " data is not 16-byte aligned (vector loads need it)";
      return TCA_ERR_INVALID;
    }
    if (elems > kMaxElems) {
      *err = "tensor " + t.name + " has more than 2^32-2^16-1 elements (u32 index domain, less 2^16 of headroom "
             "for the kernels' index arithmetic)";
      return TCA_ERR_SHAPE;
    }
  }
  for (size_t i = 0; i < free.size(); ++i)
    if (free_dims[i] > kMaxElems) {
      *err = "free dim " + p.dims[free[i]].name + " = " + std::to_string(free_dims[i]) + " exceeds 2^32-2^16-1";
      return TCA_ERR_SHAPE;
    }
  for (size_t i = 0; i < p.dims.size(); ++i) {
    if (!known[i]) {
      *err = "dim " + p.dims[i].name + " is not bound by any tensor or free-dim argument";
      return TCA_ERR_SHAPE;
    }
  }
  return TCA_OK;
}

bool WorkspaceLayout(const Plan& p, const std::vector<uint32_t>& dims, const std::vector<bool>& used,
                     std::vector<size_t>* off, size_t* total, std::string* err) {
  constexpr size_t kMax = std::numeric_limits<size_t>::max();
  off->assign(p.tensors.size(), 0);
  *total = 0;
  for (size_t t = 0; t < p.tensors.size(); ++t) {
    if (p.tensors[t].role != Role::Local || !used[t]) continue;
    size_t n = DtypeBytes(p.tensors[t].dtype);
    for (int d : p.tensors[t].dims) {
      if (dims[d] != 0 && n > kMax / dims[d]) {
        *err = "program " + p.name + ": local " + p.tensors[t].name + " exceeds the address space at these dims";
        return false;
      }
      n *= dims[d];
    }
    if (n > kMax - 255u || *total > kMax - ((n + 255u) & ~static_cast<size_t>(255u))) {
      *err = "program " + p.name + ": workspace exceeds the address space at these dims";
      return false;
    }
    (*off)[t] = *total;
    *total += (n + 255u) & ~static_cast<size_t>(255u);
  }
  return true;
}

bool GridSize(const Kernel& k, const Plan& p, const std::vector<uint32_t>& dims, uint64_t* grid, std::string* err) {
  (void)p;
  uint64_t g = 1;
  bool overflow = false;
  for (const auto& t : k.grid) {
    const uint64_t q = TermValue(k, t, dims, &overflow);
    if (overflow) {
      *err = "kernel " + k.symbol + ": grid term overflows";
      return false;
    }
    g *= q;
    if (g > (1ull << 62)) {
      *err = "kernel " + k.symbol + ": grid overflows";
      return false;
    }
  }
  if (k.split_dim >= 0) {
    const uint64_t chunks = SplitChunks(k, dims);
    switch (k.split_mode) {
      case kSplitMerge: g = chunks > 1 ? g : 0; break;
      case kSplitSingle: g = chunks == 1 ? g : 0; break;
      case kSplitPartialMany: g = chunks > 1 ? g * chunks : 0; break;
      default: g *= chunks; break;
    }
    if (g > (1ull << 62)) {
      *err = "kernel " + k.symbol + ": grid overflows";
      return false;
    }
  }
  *grid = g;
  return true;
}

uint64_t SplitChunks(const Kernel& k, const std::vector<uint32_t>& dims) {
  if (k.split_dim < 0) return 1;
  uint64_t blocks = 1;
  bool overflow = false;
  for (const auto& t : k.split_terms) {
    blocks *= TermValue(k, t, dims, &overflow);
    if (overflow || blocks > (1ull << 62)) return 1;  // far more column blocks than the target: no split
  }
  const uint64_t rows = dims[k.split_dim];
  if (rows == 0 || blocks == 0) return 1;
  uint64_t chunks = (rows + k.split_rows_min - 1) / k.split_rows_min;
  const uint64_t cap = k.split_blocks / blocks;
  if (chunks > cap) chunks = cap;
  return chunks ? chunks : 1;
}

uint32_t PackRows(const Kernel& k, const std::vector<uint32_t>& dims, uint32_t* block) {
  if (k.pack_dim < 0) {
    *block = k.block;
    return 1;
  }
  // The kernel's own choice: S lanes per row, the smallest power of two <=
  // the largest block with S * epl >= the row length.
  uint64_t lanes = 1;
  while (lanes < k.block && lanes * k.pack_epl < dims[k.pack_dim]) lanes <<= 1;
  *block = static_cast<uint32_t>(std::max<uint64_t>(k.pack_min_block, lanes));
  return static_cast<uint32_t>(*block / lanes);
}

bool Selected(const Kernel& k, const std::vector<uint32_t>& dims) {
  auto holds = [&](const Guard& g) {
    uint64_t v = 1;  // a product of at most a few u32 dims; saturates rather than wraps
    for (int d : g.dims) {
      const uint64_t x = dims[d];
      v = (x != 0 && v > ~uint64_t{0} / x) ? ~uint64_t{0} : v * x;
    }
    if (!(v >= g.lo && v <= g.hi && v % g.mod == g.rem)) return false;
    if (!g.pow2) return true;
    const uint64_t q = v / g.mod;
    return q != 0 && (q & (q - 1)) == 0;
  };
  for (const auto& g : k.when)
    if (!holds(g)) return false;
  if (k.unless.empty()) return true;
  for (const auto& g : k.unless)
    if (!holds(g)) return true;
  return false;  // every unless guard holds
}

bool LayoutArgs(const Kernel& k, const Plan& p, const std::vector<uint32_t>& dims, std::vector<unsigned char>* blob,
                std::vector<ArgSlot>* slots, std::string* err) {
  blob->clear();
  slots->clear();
  auto place = [&](size_t n) {  // natural alignment
    const size_t off = (blob->size() + n - 1) / n * n;
    blob->resize(off + n, 0);
    return static_cast<uint32_t>(off);
  };
  for (const auto& a : k.args) {
    switch (a.kind) {
      case ArgKind::Ptr: {
        ArgSlot s;
        s.offset = place(sizeof(void*));
        s.kind = ArgKind::Ptr;
        s.index = a.index;
        slots->push_back(s);
        break;
      }
      case ArgKind::Dim: {
        // The offset first: place() may reallocate the blob.
        const uint32_t v = dims[a.index];
        const uint32_t off = place(sizeof(v));
        std::memcpy(blob->data() + off, &v, sizeof(v));
        break;
      }
      case ArgKind::Scalar: {
        ArgSlot s;
        s.offset = place(4);
        s.kind = ArgKind::Scalar;
        s.index = a.index;
        s.dtype = p.scalars[a.index].dtype;
        slots->push_back(s);
        break;
      }
    }
  }
  if (blob->empty()) {
    *err = "kernel " + k.symbol + " has no arguments";
    return false;
  }
  return true;
}

void SetScalar(unsigned char* blob, const ArgSlot& s, double v) {
  switch (s.dtype) {
    case TCA_F32:
    case TCA_F16:
    case TCA_BF16: {
      const float f = static_cast<float>(v);
      std::memcpy(blob + s.offset, &f, 4);
      break;
    }
    case TCA_U32:
    case TCA_U16:
    case TCA_U8: {
      const uint32_t u = static_cast<uint32_t>(v);
      std::memcpy(blob + s.offset, &u, 4);
      break;
    }
    case TCA_BOOL: {
      const int32_t b = v != 0.0 ? 1 : 0;
      std::memcpy(blob + s.offset, &b, 4);
      break;
    }
    default: {
      const int32_t i = static_cast<int32_t>(v);
      std::memcpy(blob + s.offset, &i, 4);
      break;
    }
  }
}

bool PackArgs(const Kernel& k, const Plan& p, const std::vector<void*>& ptrs, const std::vector<uint32_t>& dims,
              const double* scalars, std::vector<unsigned char>* blob, std::string* err) {
  std::vector<ArgSlot> slots;
  if (!LayoutArgs(k, p, dims, blob, &slots, err)) return false;
  for (const auto& s : slots) {
    if (s.kind == ArgKind::Ptr) std::memcpy(blob->data() + s.offset, &ptrs[s.index], sizeof(void*));
    else SetScalar(blob->data(), s, scalars[s.index]);
  }
  return true;
}

}  // namespace plan
}  // namespace tca
