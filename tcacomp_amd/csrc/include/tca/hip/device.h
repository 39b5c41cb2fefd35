// device.h — device primitives the HIP emitter's kernels are built from
// (gfx950 / CDNA4, wave64). Included by every emitted .hip file.
//
// Reference counterparts and what changes:
//   runtime/tca/reducer.h:60-167 (WarpReducer): a 32-lane __shfl_down_sync
//     tree on EVERY Reduce(v) plus an SMEM slot fold per element. Here a
//     thread folds its strip in registers and the lanes meet ONCE per
//     output, through DPP (quad_perm, row_half_mirror, row_mirror) inside a
//     16-lane row and ds_bpermute (__shfl_xor) across rows.
//   runtime/tca/loader.h:60-232 (copy_row vec16, LoadTile*): per-element
//     bounds predicates; here 16-byte vector loads with the tail handled
//     once per strip.
#ifndef TCA_HIP_DEVICE_H_
#define TCA_HIP_DEVICE_H_

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tca {
namespace hip {

// ---- 32-bit lane moves -------------------------------------------------

// The bits of a lane value of 1, 2 or 4 bytes, widened to one 32-bit lane
// register (and back). Half-precision values move as their bit patterns.
template <typename T>
__device__ __forceinline__ int to_bits(T v) {
  static_assert(sizeof(T) == 1 || sizeof(T) == 2 || sizeof(T) == 4, "lane values are at most 32 bits");
  if constexpr (sizeof(T) == 4) return __builtin_bit_cast(int, v);
  else if constexpr (sizeof(T) == 2) return static_cast<int>(__builtin_bit_cast(uint16_t, v));
  else return static_cast<int>(__builtin_bit_cast(uint8_t, v));
}

template <typename T>
__device__ __forceinline__ T from_bits(int b) {
  if constexpr (sizeof(T) == 4) return __builtin_bit_cast(T, b);
  else if constexpr (sizeof(T) == 2) return __builtin_bit_cast(T, static_cast<uint16_t>(b));
  else return __builtin_bit_cast(T, static_cast<uint8_t>(b));
}

// A register vector of N elements of T (N * sizeof(T) <= 16 bytes per load),
// read by v[i] and written by v.set(i, x). Elements narrower than 32 bits
// that fill whole 32-bit words stay packed in those words and are extracted
// where they are used, so a vector costs its byte size in registers (16 u8
// elements: 4 registers; element-wise storage let the compiler widen every
// byte into a register of its own at the load, 4x the registers of the row
// cache and half the occupancy).
template <typename T, int N, bool Packed = (sizeof(T) < 4 && (sizeof(T) * N) % 4 == 0)>
struct alignas(sizeof(T) * N) vec {
  T v[N];
  __device__ __forceinline__ T operator[](int i) const { return v[i]; }
  __device__ __forceinline__ void set(int i, T x) { v[i] = x; }
};

template <typename T, int N>
struct alignas(sizeof(T) * N) vec<T, N, true> {
  static constexpr int kPer = 4 / static_cast<int>(sizeof(T));  // elements per word
  static constexpr uint32_t kMask = sizeof(T) == 1 ? 0xffu : 0xffffu;
  uint32_t w[N / kPer];
  __device__ __forceinline__ T operator[](int i) const {
    return from_bits<T>(static_cast<int>(w[i / kPer] >> ((i % kPer) * 8 * static_cast<int>(sizeof(T)))));
  }
  __device__ __forceinline__ void set(int i, T x) {
    const int sh = (i % kPer) * 8 * static_cast<int>(sizeof(T));
    w[i / kPer] = (w[i / kPer] & ~(kMask << sh)) | ((static_cast<uint32_t>(to_bits(x)) & kMask) << sh);
  }
};

template <typename T, int N>
__device__ __forceinline__ vec<T, N> load_vec(const T* __restrict__ p) {
  return *reinterpret_cast<const vec<T, N>*>(p);
}

// Streaming load: data read exactly once by this kernel.
template <typename T, int N>
__device__ __forceinline__ vec<T, N> load_vec_nt(const T* __restrict__ p) {
  if constexpr (sizeof(T) * N == 16) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    u4 r = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
    return __builtin_bit_cast(vec<T, N>, r);
  } else if constexpr (sizeof(T) * N == 8) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    u2 r = __builtin_nontemporal_load(reinterpret_cast<const u2*>(p));
    return __builtin_bit_cast(vec<T, N>, r);
  } else {
    return *reinterpret_cast<const vec<T, N>*>(p);
  }
}

template <typename T, int N>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const vec<T, N>& x) {
  *reinterpret_cast<vec<T, N>*>(p) = x;
}

// Streaming store: the output is not re-read by this kernel, so keep it out
// of the caches' way.
template <typename T, int N>
__device__ __forceinline__ void store_vec_nt(T* __restrict__ p, const vec<T, N>& x) {
  if constexpr (sizeof(T) * N == 16) {
    typedef unsigned int u4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(*reinterpret_cast<const u4*>(&x), reinterpret_cast<u4*>(p));
  } else if constexpr (sizeof(T) * N == 8) {
    typedef unsigned int u2 __attribute__((ext_vector_type(2)));
    __builtin_nontemporal_store(*reinterpret_cast<const u2*>(&x), reinterpret_cast<u2*>(p));
  } else {
    *reinterpret_cast<vec<T, N>*>(p) = x;
  }
}

template <typename T>
__device__ __forceinline__ void store_nt(T* __restrict__ p, T x) {
  if constexpr (sizeof(T) == 4 || sizeof(T) == 8) {
    __builtin_nontemporal_store(x, p);
  } else {
    *p = x;
  }
}

// Closes one vector's worth of a 32-bit integer fold: an empty asm with the
// partial as its in/out operand, so no instruction is emitted. Without it the
// compiler reassociates the integer adds of the vectors in flight, widening
// every narrow element into a register of its own before any is added (4
// vectors of 16 u8 elements: 64 live registers, occupancy 5 instead of 8;
// 4.6 -> 6.1 TB/s on a streamed u8 row sum). Floating-point folds are never
// reassociated and need no fence.
template <typename T>
__device__ __forceinline__ void fold_fence(T& v) {
  static_assert(sizeof(T) == 4, "a 32-bit partial");
  __asm__ volatile("" : "+v"(v));
}

// DPP move within a 16-lane row. Controls used (CDNA3/4 ISA, DPP_CTRL):
//   0xB1 quad_perm[1,0,3,2]  (lane ^ 1)
//   0x4E quad_perm[2,3,0,1]  (lane ^ 2)
//   0x141 row_half_mirror    (lane i <-> 7-i within each 8 lanes)
//   0x140 row_mirror         (lane i <-> 15-i within each 16 lanes)
template <int CTRL, typename T>
__device__ __forceinline__ T dpp(T v) {
  return from_bits<T>(__builtin_amdgcn_update_dpp(0, to_bits(v), CTRL, 0xF, 0xF, false));
}

template <typename T>
__device__ __forceinline__ T xor_lanes(T v, int mask) {
  return from_bits<T>(__shfl_xor(to_bits(v), mask, 64));
}

// One butterfly step of a segmented all-reduce. Before the step every group
// of OFF consecutive lanes holds one value per group; after it every group
// of 2*OFF lanes does. OFF 4 and 8 use mirrors: the partner sits in the other
// half of the 2*OFF group, which is all a reduction needs.
template <int OFF, typename T>
__device__ __forceinline__ T partner(T v) {
  if constexpr (OFF == 1) return dpp<0xB1>(v);
  else if constexpr (OFF == 2) return dpp<0x4E>(v);
  else if constexpr (OFF == 4) return dpp<0x141>(v);
  else if constexpr (OFF == 8) return dpp<0x140>(v);
  else return xor_lanes(v, OFF);
}

// All-reduce over aligned segments of SEG lanes (SEG a power of two <= 64);
// every lane of a segment ends with the segment's total. `op` must be
// associative and commutative (the classifier only admits such combiners).
template <int SEG, typename T, typename Op>
__device__ __forceinline__ T seg_allreduce(T v, Op op) {
  if constexpr (SEG >= 2) v = op(v, partner<1>(v));
  if constexpr (SEG >= 4) v = op(v, partner<2>(v));
  if constexpr (SEG >= 8) v = op(v, partner<4>(v));
  if constexpr (SEG >= 16) v = op(v, partner<8>(v));
  if constexpr (SEG >= 32) v = op(v, partner<16>(v));
  if constexpr (SEG >= 64) v = op(v, partner<32>(v));
  return v;
}

// All-reduce over aligned segments of `seg` lanes, `seg` a power of two
// <= 64 known only at run time (uniform over the wave). Every lane of the
// wave must call it; `op` must be associative and commutative.
template <typename T, typename Op>
__device__ __forceinline__ T seg_allreduce_rt(T v, uint32_t seg, Op op) {
  switch (seg) {
    case 64: return seg_allreduce<64>(v, op);
    case 32: return seg_allreduce<32>(v, op);
    case 16: return seg_allreduce<16>(v, op);
    case 8: return seg_allreduce<8>(v, op);
    case 4: return seg_allreduce<4>(v, op);
    case 2: return seg_allreduce<2>(v, op);
    default: return v;
  }
}

// All-reduce over the wave of values that may be absent (`has` false: the
// lane holds nothing). Every lane ends with the total of the present values
// and the OR of the flags. Every lane of the wave must call it; `op` must be
// associative and commutative.
template <typename T, typename Op>
__device__ __forceinline__ T wave_allreduce_present(T v, bool& has, Op op) {
  for (int off = 1; off < 64; off <<= 1) {
    const T o = xor_lanes(v, off);
    const bool oh = __shfl_xor(static_cast<int>(has), off, 64) != 0;
    if (has && oh) v = op(v, o);
    else if (oh) v = o;
    has = has || oh;
  }
  return v;
}

// Lanes per row of the packed row kernels, as log2: the smallest power of
// two 2^ls <= 2^log2_block with per_lane << ls >= vecs (no lane holds more
// than per_lane vectors unless the row needs more than the whole block).
__device__ __forceinline__ uint32_t pack_lanes_log2(uint32_t vecs, uint32_t per_lane, uint32_t log2_block) {
  uint32_t ls = 0u;
  while (ls < log2_block && (per_lane << ls) < vecs) ++ls;
  return ls;
}

// Row chunks P of a split column reduction (the plan's split record
// computes the same number at launch): at least rows_min rows per chunk,
// and no more chunks than keep col_blocks * P <= blocks; 1 when there are
// no rows or the column blocks alone reach `blocks`.
// Rounds up without forming rows + rows_min - 1, so rows up to 2^32 - 1 give
// the host's 64-bit answer. Host-callable for the tests that hold it to the
// plan's numbers.
__host__ __device__ __forceinline__ uint32_t col_split(uint32_t rows, uint32_t col_blocks, uint32_t rows_min,
                                                       uint32_t blocks) {
  if (rows == 0u || col_blocks == 0u) return 1u;
  uint32_t p = (rows - 1u) / rows_min + 1u;
  const uint32_t cap = blocks / col_blocks;
  if (p > cap) p = cap;
  return p ? p : 1u;
}

__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }
__device__ __forceinline__ uint32_t wave_id() { return threadIdx.x >> 6; }

// ceil(a / b) for b > 0, exact for every uint32 a (no a + b - 1 that wraps).
__host__ __device__ __forceinline__ uint32_t ceil_div(uint32_t a, uint32_t b) { return a == 0u ? 0u : (a - 1u) / b + 1u; }

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32, 1 ulp), for the
// terms of the online normaliser's sums: rounding the product adds at most
// |x| 2^-24 ln 2 of relative error, 2.7e-6 for |x| <= 44 (x <= 0 here; below
// -44 a term is under 2^-63 of the largest, 1, and does not register in an
// f32 sum). -inf gives 0, NaN NaN.
__device__ __forceinline__ float exp_term(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// The online normaliser of a softmax (Milakov & Gimelshein 2018, "Online
// normalizer calculation for softmax"): a running maximum m of the values
// seen (NaN never enters it; -inf until a larger value arrives) and
// s = sum of expf(v - m) over them, rescaled whenever m grows. Then
// sum(expf(v - a)) = s * expf(m - a) for any a. The special values behave as
// in that sum evaluated directly with a >= m: a NaN value or an exp(inf - inf)
// makes s NaN, and a -inf value adds nothing. The caller handles a = -inf
// (every value -inf or NaN, where the direct sum is NaN).
// N values at a time: their maximum first (fmaxf: NaN left out), one
// rescale when it exceeds m, then one exponential per value, on the
// hardware exp2 (exp_term). With a rescale per value and ocml's expf (about
// 16 instructions: range reduction with a split log2(e), ldexp, overflow
// clamps) the fused softmax partial was VALU-bound at 2.1x the time of its
// read. The rescale sits behind a wave-uniform branch (taken while some
// lane's maximum grows: rarely, after a chunk's first vectors), and a -inf
// value needs no test of its own: the shift is m, or 0 while m is -inf
// (then every value so far is -inf or NaN), and exp2(-inf) = 0, so each
// value costs a subtract, a multiply, an exp2 and an add, with s exactly
// as the per-value form gives it.
template <int N>
__device__ __forceinline__ void online_expsum_add(float& m, float& s, const float (&v)[N]) {
  float g = v[0];
#pragma unroll
  for (int i = 1; i < N; ++i) g = fmaxf(g, v[i]);
  if (__builtin_amdgcn_ballot_w64(g > m) != 0u) {
    if (g > m) {
      s *= exp_term(m - g);
      m = g;
    }
  }
  const float sh = m == -__builtin_inff() ? 0.0f : m;
#pragma unroll
  for (int i = 0; i < N; ++i) s += exp_term(v[i] - sh);
}

// Merges another lane's (m2, s2) into (m, s): commutative, so a butterfly
// over the wave leaves every lane with the same pair. The factors are
// exp_term(m - M), m <= M (the same bound as the terms).
__device__ __forceinline__ void online_expsum_merge(float& m, float& s, float m2, float s2) {
  const float M = fmaxf(m, m2);
  s = (m == M ? s : s * exp_term(m - M)) + (m2 == M ? s2 : s2 * exp_term(m2 - M));
  m = M;
}

// Pairwise union of two sets of values, each held as its sum s, its count
// n (> 0) and m2, the sum of squares about its own mean (Chan, Golub &
// LeVeque 1979): m2 of the union = m2 + m2b + (sb/nb - s/n)^2 n nb / (n + nb),
// every term non-negative. The sums add in the order written (s, then sb).
__device__ __forceinline__ void chan_merge(float& s, float& m2, float& n, float sb, float m2b, float nb) {
  const float d = sb / nb - s / n;
  m2 += m2b + d * d * (n * nb / (n + nb));
  s += sb;
  n += nb;
}

// Waits for every vector memory operation of the wave (s_waitcnt vmcnt(0),
// expcnt and lgkmcnt left at their maxima: the gfx9 encoding). Placed once
// before a loop, it settles loads that the compiler's wait pass otherwise
// counts as pending on a branch that skipped their use, and then waits for
// at the head of every iteration.
__device__ __forceinline__ void wait_vector_memory() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// A value that every lane of the wave holds bit for bit, as a wave-uniform
// (scalar register) value.
__device__ __forceinline__ float wave_uniform(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// The union as chan_merge forms it, where either side may be empty (n or
// nb = 0: nothing folded), as lanes and partials that hold no values are.
// Commutative bit for bit: the two m2 add first, and the sums, the squared
// difference of means and the weight are symmetric; so a butterfly over a
// wave leaves every lane with the same triple. The means and the weight use
// the hardware reciprocal (v_rcp_f32, 1 ulp; counts are >= 1) instead of
// divisions: a fifth of the split partial's instructions, 48.0 -> 47.0 us at
// [64, 1 Mi] rows.
__device__ __forceinline__ void chan_merge_present(float& s, float& m2, float& n, float sb, float m2b, float nb) {
  if (nb == 0.0f) return;
  if (n == 0.0f) {
    s = sb;
    m2 = m2b;
    n = nb;
    return;
  }
  const float d = sb * __builtin_amdgcn_rcpf(nb) - s * __builtin_amdgcn_rcpf(n);
  m2 = (m2 + m2b) + d * d * (n * nb * __builtin_amdgcn_rcpf(n + nb));
  s += sb;
  n += nb;
}

// Folds the N values at v into (s, m2, n): their sum, their mean (N a
// power of two: an exact scaling), their centred sum of squares, then
// chan_merge_present.
template <int N>
__device__ __forceinline__ void chan_add_n(float& s, float& m2, float& n, const float* v) {
  float gs = v[0];
#pragma unroll
  for (int i = 1; i < N; ++i) gs += v[i];
  const float gm = gs * (1.0f / N);
  float g2 = 0.0f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float d = v[i] - gm;
    g2 = fmaf(d, d, g2);
  }
  chan_merge_present(s, m2, n, gs, g2, static_cast<float>(N));
}

// chan_add_n over an array of N values.
template <int N>
__device__ __forceinline__ void chan_add(float& s, float& m2, float& n, const float (&v)[N]) {
  chan_add_n<N>(s, m2, n, v);
}

}  // namespace hip
}  // namespace tca

#endif  // TCA_HIP_DEVICE_H_
