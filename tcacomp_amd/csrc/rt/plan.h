// plan.h — the launch plan: what the HIP emitter writes beside a code object
// and what the runtime's one launcher interprets.
//
// Text format (one record per line, '#' starts a comment):
//   tca-plan 1
//   program <name>
//   dim <name> <extent>                        extent 0 = dynamic (u32 at run time)
//   tensor <name> <dtype> <in|out|local> <rank> <dim-name>...
//   scalar <name> <dtype>
//   kernel <symbol> <block> <lds-bytes> <n-terms> <term>...
//       term = <factor>[*<factor>...]/<divisor>[:<cap>], factor = dim name or
//       integer; grid = product over terms of ceil(product(factors) / divisor),
//       each term limited to <cap> when one is given (grid-stride kernels).
//       divisor = integer | pack: the rows per block of the kernel's pack record
//   arg ptr <tensor> | arg dim <name> | arg scalar <name>    (for the last kernel)
//   pack <dim> <epl> <min-block>    (for the last kernel) the kernel packs rows of
//       `dim` elements: S lanes share a row, S the smallest power of two <= the
//       kernel's block with S * epl >= dim; it launches with max(min-block, S)
//       lanes per block, max(min-block, S) / S rows each
//   split <rdim> <rows-min> <blocks> <mode> <n-terms> <term>...    (for the last
//       kernel) a reduction over `rdim` split into P row chunks: with B the
//       product of the terms (the column blocks), P = 1 when rdim or B is 0,
//       else min(ceil(rdim / rows-min), max(1, blocks / B)). mode 0: the
//       grid is multiplied by P; mode 1: the kernel (the merge of the P
//       partials) launches only when P > 1; mode 2: the kernel launches only
//       when P == 1 (a whole-column kernel); mode 3: as mode 0, but only when
//       P > 1 (the partials of a nest whose P == 1 case is a mode-2 kernel).
//   when <dim> <lo> <hi> <mod> <rem>    (for the last kernel) the kernel runs only
//       when lo <= dim <= hi and dim % mod == rem; every guard of a kernel must
//       hold. <dim> may be a product of dims, d1*d2*... (its value taken in
//       64 bits): the contractions pick their small-tile kernel by the size of
//       the output plane, M*N. Variants of one nest specialised on a run-time dim carry guards
//       that partition its values, so exactly one of them launches.
//   unless <dim> <lo> <hi> <mod> <rem>  (for the last kernel) the same test; the
//       kernel is skipped when every one of its unless guards holds (the
//       complement of a conjunction of when guards another kernel carries).
//       Either record may end in `pow2` (with rem 0): the guard then also
//       requires dim / mod to be a power of two (a row of exactly mod * 2^k
//       elements: the streaming family's exact-fit kernels).
//   end
//
// The shape contract Bind() enforces is the reference launcher's
// (internal/cg/cxx/launch.go:98-130): each dynamic dim takes its value from
// its first tensor occurrence in declaration order and every later
// occurrence must agree; a dynamic dim no tensor carries is a "free dim"
// passed explicitly; const extents are checked against the tensors too.
#ifndef TCA_RT_PLAN_H_
#define TCA_RT_PLAN_H_

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "tca_rt.h"

namespace tca {
namespace plan {

enum class Role { In, Out, Local };
enum class ArgKind { Ptr, Dim, Scalar };

struct Dim {
  std::string name;
  uint64_t extent = 0;  // 0 = dynamic
};

struct Tensor {
  std::string name;
  int dtype = TCA_F32;
  Role role = Role::In;
  std::vector<int> dims;  // indices into Plan::dims
};

struct Scalar {
  std::string name;
  int dtype = TCA_F32;
};

struct Term {
  std::vector<int> dim_factors;  // indices into Plan::dims
  uint64_t const_factor = 1;
  uint64_t divisor = 1;
  uint64_t cap = 0;  // 0 = none
  bool packed = false;  // the divisor is the kernel's rows per block
};

struct Arg {
  ArgKind kind = ArgKind::Ptr;
  int index = 0;  // tensor, dim or scalar index
};

struct Guard {
  std::vector<int> dims;  // indices into Plan::dims; the guarded value is their product
  uint64_t lo = 0, hi = 0xffffffffull, mod = 1, rem = 0;
  bool pow2 = false;  // additionally dim / mod is a power of two (rem == 0)
};

struct Kernel {
  std::string symbol;
  uint32_t block = 256;
  uint32_t lds = 0;
  std::vector<Term> grid;
  std::vector<Arg> args;
  std::vector<Guard> when;
  std::vector<Guard> unless;  // skipped when all of these hold
  int pack_dim = -1;  // >= 0: a packed row kernel (block chosen at launch)
  uint64_t pack_epl = 0, pack_min_block = 0;
  int split_dim = -1;  // >= 0: a row-split reduction (see the split record)
  uint64_t split_rows_min = 0, split_blocks = 0;
  // What the chunk count P does to this kernel's grid: kSplitPartial = grid
  // x P, kSplitMerge = launched only when P > 1, kSplitSingle = launched
  // only when P == 1, kSplitPartialMany = grid x P, launched only when P > 1.
  int split_mode = 0;
  std::vector<Term> split_terms;
};

enum SplitMode { kSplitPartial = 0, kSplitMerge = 1, kSplitSingle = 2, kSplitPartialMany = 3 };

struct Plan {
  std::string name;
  std::vector<Dim> dims;
  std::vector<Tensor> tensors;
  std::vector<Scalar> scalars;
  std::vector<Kernel> kernels;

  size_t ParamTensorCount() const;
  // Dynamic dims carried by no in/out tensor, in declaration order.
  std::vector<int> FreeDims() const;
};

size_t DtypeBytes(int dtype);
const char* DtypeName(int dtype);
int DtypeFromName(const std::string& s);

bool Parse(const std::string& text, Plan* out, std::string* err);
std::string Serialize(const Plan& p);

// The most elements a tensor may hold (and the largest free dim): the u32
// index domain less 2^16. The kernels step u32 indices (vectors of a row,
// rows of a column, lanes of a row) past an extent by less than 2^16 before
// comparing them with it; the headroom keeps that step from wrapping.
constexpr uint64_t kMaxElems = (uint64_t{1} << 32) - (uint64_t{1} << 16) - 1;

// Resolves every dim value from the caller's tensors and free dims. Returns
// a TCA_* status; *dims receives one value per Plan::dims entry.
int Bind(const Plan& p, const tca_tensor* tensors, uint32_t n_tensors, const uint32_t* free_dims,
         uint32_t n_free_dims, std::vector<uint32_t>* dims, std::string* err);

// The workspace at bound dims: every local that `used` marks at a 256-byte
// aligned offset, in declaration order (`off` per plan tensor, `total` the
// bytes). False, with `err` set, when a size does not fit in size_t.
bool WorkspaceLayout(const Plan& p, const std::vector<uint32_t>& dims, const std::vector<bool>& used,
                     std::vector<size_t>* off, size_t* total, std::string* err);
bool GridSize(const Kernel& k, const Plan& p, const std::vector<uint32_t>& dims, uint64_t* grid, std::string* err);
// Rows per block of a packed kernel (1 otherwise); *block receives the
// launch block size.
uint32_t PackRows(const Kernel& k, const std::vector<uint32_t>& dims, uint32_t* block);
// Row chunks P of a split kernel (1 for a kernel without a split record).
uint64_t SplitChunks(const Kernel& k, const std::vector<uint32_t>& dims);
// Whether every guard of k holds for the bound dims.
bool Selected(const Kernel& k, const std::vector<uint32_t>& dims);
// Packs the kernel arguments per the HIP kernarg ABI (natural alignment):
// pointers 8 bytes, dims u32, scalars 4 bytes (f32 for float types, i32/u32
// for integers, i32 for bool).
bool PackArgs(const Kernel& k, const Plan& p, const std::vector<void*>& ptrs, const std::vector<uint32_t>& dims,
              const double* scalars, std::vector<unsigned char>* blob, std::string* err);

// The same layout split in two, for launches that repeat one shape: a blob
// with every dim argument written (pointers and scalars zero) and the slots
// left to fill per call. SetPtr / SetScalar fill one slot.
struct ArgSlot {
  uint32_t offset = 0;
  ArgKind kind = ArgKind::Ptr;  // Ptr or Scalar
  int index = 0;                // tensor or scalar index
  int dtype = TCA_F32;          // a scalar's declared type
};
bool LayoutArgs(const Kernel& k, const Plan& p, const std::vector<uint32_t>& dims, std::vector<unsigned char>* blob,
                std::vector<ArgSlot>* slots, std::string* err);
void SetScalar(unsigned char* blob, const ArgSlot& s, double v);

}  // namespace plan
}  // namespace tca

#endif  // TCA_RT_PLAN_H_
