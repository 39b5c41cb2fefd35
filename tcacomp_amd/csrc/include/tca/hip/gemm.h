// gemm.h — dense K-contraction on CDNA4 matrix cores (family G).
//
// The reference lowers C[m,n] = sum_k A[m,k] B[k,n] as a CTA-wide
// WarpReducer collective per output element (a shuffle tree per Reduce and
// two barriers per Combine; .planning/quick/261030-uai-.../after-cu/gemm.cu:
// 59-90). Here the contraction runs on MFMA:
//   bf16 inputs : v_mfma_f32_16x16x32_bf16 (gfx950) on whole 256x256 tiles
//                 (f16 inputs: the same kernels with the _f16 MFMAs)
//                 (gemm_bf16_4w when K % 64 == 0 and K >= 256, else
//                 gemm_bf16_256_w8), v_mfma_f32_32x32x16_bf16 on the edge
//                 tiles (gemm_bf16_256); fp32 accumulate
//   fp32 inputs : v_mfma_f32_32x32x2f32 (gemm_f32_4w on whole tiles from
//                 M, N >= 4096 on, else gemm_f32_tile), fp32 accumulate
// Geometry of the register-staged kernels: a 256-thread workgroup (4 waves,
// 2x2) owns a BMxBN tile of C, each wave a (BM/2)x(BN/2) sub-tile of 32x32
// MFMA blocks. K advances in
// BK slices staged through LDS; the next slice's global loads are issued
// before the current slice's MFMAs so HBM latency hides under the math.
// LDS tiles hold every MFMA operand K-contiguous for its row/column (A as
// [m][k], B as [n][k]); a [K][N] B is transposed in registers on its way
// into LDS. Rows are padded so a wave's operand reads spread over the banks.
//
// MFMA 32x32 operand/result lane layout (CDNA3/CDNA4 ISA):
//   A operand: lane l supplies row (l % 32), k = (l / 32) * KPL + [0, KPL)
//   B operand: lane l supplies col (l % 32), same k
//   result   : lane l, element i -> row 8*(i/4) + 4*(l/32) + (i%4), col l%32
// with KPL = 8 for 32x32x16 bf16 and KPL = 1 for 32x32x2 f32.
#ifndef TCA_HIP_GEMM_H_
#define TCA_HIP_GEMM_H_

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

namespace tca {
namespace hip {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// The 16-bit contractions below move raw 16-bit values (as bf16x8 registers)
// through memory, LDS and registers; F16 selects the MFMA that reads them as
// IEEE half (v_mfma_f32_*_f16) instead of bfloat16. The fp32 accumulation,
// the operand layout and every data movement are the same for both.
template <bool F16, typename Acc>
__device__ __forceinline__ Acc mfma_32x32x16_16b(const bf16x8& a, const bf16x8& b, const Acc& c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
template <bool F16, typename Acc>
__device__ __forceinline__ Acc mfma_16x16x32_16b(const bf16x8& a, const bf16x8& b, const Acc& c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Maps the linear workgroup id to a (tile_m, tile_n) pair. Workgroups are
// dealt round-robin over the 8 XCDs; regrouping so that each XCD receives a
// contiguous run of tiles (and walking those runs in GROUP_M-row bands) keeps
// the A row panels and B column panels a run touches inside one XCD's L2.
// `tile` is the linear tile index: the workgroup id, or for a batched
// contraction the workgroup id within its batch (the emitted kernel passes it).
__device__ __forceinline__ void gemm_tile_coords(uint32_t tiles_m, uint32_t tiles_n, uint32_t* tm, uint32_t* tn,
                                                 uint32_t tile) {
  const uint32_t total = tiles_m * tiles_n;
  uint32_t b = tile;
  if (total % 8u == 0u) b = (b % 8u) * (total / 8u) + b / 8u;
  const uint32_t kGroup = 8u;
  const uint32_t band = kGroup * tiles_n;
  const uint32_t g = b / band;
  const uint32_t first_m = g * kGroup;
  const uint32_t rows = (tiles_m - first_m) < kGroup ? (tiles_m - first_m) : kGroup;
  const uint32_t in = b % band;
  *tm = first_m + in % rows;
  *tn = in / rows;
}

// ------------------------------------------------------- bf16 path, 256 tiles
// Tile: BM = BN = 256, BK = 64; 4 waves as 2x2, each 128x128 = 4x4 MFMA
// blocks (256 fp32 accumulators per lane). Per 16-deep K step a wave reads
// 4 A + 4 B fragments (8 x 1 KiB of LDS) for 16 MFMAs.
//
// LDS layout: each [256][64] bf16 tile is unpadded (128-byte rows) over 64
// four-byte banks (256 bytes, two rows' worth; a 16-byte slot is (row
// parity, column group)). Logical row r is stored at physical row
// p = r ^ ((r / 8) % 2) and its column group c at c ^ ((p / 2) % 8):
//     element (r, k) -> p*64 + ((k/8) ^ ((p/2) % 8))*8 + k%8.
// A fragment read (32 consecutive rows, one column group per half-wave)
// then hits 16 distinct slots in each 16-lane cycle of a 128-bit read (the
// cycles measured on gfx950 are described at gemm_bf16_256_w8). Two such
// tile pairs (A, B) double-buffer the K loop with one barrier per step:
// 128 KiB of LDS.
// SWZ = 0 keeps the plain row-XOR swizzle (c ^ (r % 8)), optimal for a
// 32-bank / 8-lane-phase LDS; SWZ = 1 is the layout above.
template <int SWZ>
__device__ __forceinline__ uint32_t swz64(uint32_t row, uint32_t cg) {
  if constexpr (SWZ == 0) {
    return row * 64u + ((cg ^ (row & 7u)) << 3);
  } else {
    const uint32_t p = row ^ ((row >> 3) & 1u);
    return p * 64u + ((cg ^ ((p >> 1) & 7u)) << 3);
  }
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

// s_waitcnt immediate for gfx9: vmcnt[3:0] | expcnt[6:4] (7 = no wait) |
// lgkmcnt[11:8] | vmcnt[5:4] at [15:14].
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | (7 << 4) | ((lgkm & 15) << 8) | ((vm >> 4) << 14); }

// The tiles the direct-to-LDS path takes: the whole 256x256 block in range,
// K a positive multiple of 32 and [K][N] / [N][K] rows 16-byte aligned.
__device__ __forceinline__ bool gemm_bf16_dma_tile(uint32_t m0, uint32_t n0, uint32_t M, uint32_t N, uint32_t K) {
  return m0 + 256u <= M && n0 + 256u <= N && K % 32u == 0u && N % 8u == 0u && K > 0u;
}

// SKIP_DMA: the direct-to-LDS tiles belong to another kernel
// (gemm_bf16_256_w8); this one returns at once on them.
template <bool B_NK, typename Epi, int SWZ = 1, bool SPREAD = true, bool PREFETCH = true, bool SKIP_DMA = false,
          bool F16 = false>
__device__ __forceinline__ void gemm_bf16_256(const __bf16* __restrict__ A, const __bf16* __restrict__ B,
                                              float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, Epi epi,
                                              uint32_t tile = ~0u) {
  constexpr uint32_t BM = 256, BN = 256, BK = 64, TILE = BM * BK;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][TILE];  // [buffer][A, B]
  const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  uint32_t tm, tn;
  gemm_tile_coords(tiles_m, tiles_n, &tm, &tn, tile == ~0u ? blockIdx.x : tile);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  if (SKIP_DMA && gemm_bf16_dma_tile(m0, n0, M, N, K)) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wm = (wave >> 1) * 128u, wn = (wave & 1u) * 128u;
  const bool vec_a = (K % 8u) == 0u;
  const bool vec_b = B_NK ? (K % 8u) == 0u : (N % 8u) == 0u;
  const uint16_t* __restrict__ A16 = reinterpret_cast<const uint16_t*>(A);
  const uint16_t* __restrict__ B16 = reinterpret_cast<const uint16_t*>(B);

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  u32x4 ra[8], rb[8];
  // Interior tiles (the whole BMxBN block in range, rows 16-byte aligned)
  // take unguarded vector loads addressed as a workgroup-uniform base plus a
  // 32-bit per-lane byte offset; the test is uniform, so it is a scalar
  // branch, not a per-lane mask.
  const bool interior_mn = vec_a && vec_b && m0 + BM <= M && n0 + BN <= N;
  const uint32_t off_rows = ((tid >> 3) * K + (tid & 7u) * 8u) * 2u;  // row-panel vector of this lane
  const uint32_t off_kn = ((tid & 7u) * 8u * N + (tid >> 3) * 8u) * 2u;  // [K][N] block of this lane
  auto at = [](const uint16_t* base, uint32_t byte_off) {
    return *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + byte_off);
  };
  // Rows of a K-contiguous panel (A, or B as [n][k]): 2048 16-byte vectors.
  auto load_rows = [&](const uint16_t* __restrict__ P, uint32_t rows, uint32_t r0, uint32_t k0, bool vec, u32x4* r) {
    if (interior_mn && k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = at(P + static_cast<uint64_t>(r0 + i * 32u) * K + k0, off_rows);
      return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v = i * 256u + tid, rr = v >> 3, gk = k0 + (v & 7u) * 8u, gr = r0 + rr;
      if (vec && gr < rows && gk + 8u <= K) {
        r[i] = *reinterpret_cast<const u32x4*>(P + static_cast<uint64_t>(gr) * K + gk);
      } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (gr < rows && gk + e < K) ? P[static_cast<uint64_t>(gr) * K + gk + e] : 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[i][e] = h[2 * e] | (h[2 * e + 1] << 16);
      }
    }
  };
  // [K][N] panel: thread owns an 8(k) x 8(n) block; kb = tid % 8, nb = tid / 8.
  auto load_b_kn = [&](uint32_t k0) {
    const uint32_t kb = tid & 7u, nb = tid >> 3;
    if (interior_mn && k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < 8; ++i) rb[i] = at(B16 + static_cast<uint64_t>(k0 + i) * N + n0, off_kn);
      return;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t gk = k0 + kb * 8u + i, gn = n0 + nb * 8u;
      if (vec_b && gk < K && gn + 8u <= N) {
        rb[i] = *reinterpret_cast<const u32x4*>(B16 + static_cast<uint64_t>(gk) * N + gn);
      } else {
        uint32_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = (gk < K && gn + e < N) ? B16[static_cast<uint64_t>(gk) * N + gn + e] : 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) rb[i][e] = h[2 * e] | (h[2 * e + 1] << 16);
      }
    }
  };
  // Stores of the staged slice into an LDS buffer, in halves so they can be
  // spread between the MFMA steps of the current slice.
  auto store_a = [&](uint32_t buf, int half) {
    uint16_t* As = lds[buf][0];
#pragma unroll
    for (int i = half * 4; i < half * 4 + 4; ++i) {
      const uint32_t v = i * 256u + tid;
      *reinterpret_cast<u32x4*>(&As[swz64<SWZ>(v >> 3, v & 7u)]) = ra[i];
    }
  };
  auto store_b = [&](uint32_t buf, int half) {
    uint16_t* Bs = lds[buf][1];
    if constexpr (B_NK) {
#pragma unroll
      for (int i = half * 4; i < half * 4 + 4; ++i) {
        const uint32_t v = i * 256u + tid;
        *reinterpret_cast<u32x4*>(&Bs[swz64<SWZ>(v >> 3, v & 7u)]) = rb[i];
      }
    } else {
      // 8x8 transpose in registers: column n of the block gets its 8 k values.
      const uint32_t kb = tid & 7u, nb = tid >> 3;
#pragma unroll
      for (int n = half * 4; n < half * 4 + 4; ++n) {
        const int d = n >> 1;
        u32x4 w;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = rb[2 * q][d], hi = rb[2 * q + 1][d];
          w[q] = (n & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
        *reinterpret_cast<u32x4*>(&Bs[swz64<SWZ>(nb * 8u + n, kb)]) = w;
      }
    }
  };
  auto load_a = [&](uint32_t k0) { load_rows(A16, M, m0, k0, vec_a, ra); };
  auto load_b = [&](uint32_t k0) {
    if constexpr (B_NK) load_rows(B16, N, n0, k0, vec_b, rb);
    else load_b_kn(k0);
  };
  auto frag = [&](const uint16_t* T, uint32_t row0, uint32_t cg) {
    return *reinterpret_cast<const bf16x8*>(&T[swz64<SWZ>(row0 + (lane & 31u), cg)]);
  };

  // SPREAD: while slice kt is multiplied out of LDS buffer kt%2, slice kt+1
  // (already in registers) is written into the other buffer a quarter per
  // MFMA step, and the registers refill with slice kt+2 as soon as they are
  // written out. Otherwise slice kt+1 is loaded at the top of the step and
  // written after the MFMAs. One barrier per slice either way.
  //
  // The MFMA takes the B fragment as its first operand: it then computes the
  // C^T block, so each lane ends up holding four consecutive columns of one
  // row of C (a 16-byte store) instead of four rows of one column.
  const uint32_t nk = (K + BK - 1) / BK;
  if (nk > 0) {
    load_a(0);
    load_b(0);
    store_a(0, 0);
    store_a(0, 1);
    store_b(0, 0);
    store_b(0, 1);
  }
  if (SPREAD && nk > 1) {
    load_a(BK);
    load_b(BK);
  }
  __syncthreads();
  for (uint32_t kt = 0; kt < nk; ++kt) {
    const uint32_t buf = kt & 1u, nbuf = buf ^ 1u;
    const bool has1 = kt + 1 < nk, has2 = kt + 2 < nk;
    const uint16_t* As = lds[buf][0];
    const uint16_t* Bs = lds[buf][1];
    if (!SPREAD && has1) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }
    bf16x8 fa[4], fb[4];
    if constexpr (PREFETCH) {
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i] = frag(As, wm + i * 32u, lane >> 5);
#pragma unroll
      for (int j = 0; j < 4; ++j) fb[j] = frag(Bs, wn + j * 32u, lane >> 5);
    }
#pragma unroll
    for (uint32_t ks = 0; ks < BK / 16; ++ks) {
      const uint32_t cg = ks * 2u + (lane >> 5);
      bf16x8 ga[4], gb[4];
      if constexpr (PREFETCH) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ga[i] = fa[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) gb[j] = fb[j];
        if (ks + 1 < BK / 16) {
#pragma unroll
          for (int i = 0; i < 4; ++i) fa[i] = frag(As, wm + i * 32u, cg + 2u);
#pragma unroll
          for (int j = 0; j < 4; ++j) fb[j] = frag(Bs, wn + j * 32u, cg + 2u);
        }
        // Keep the next step's LDS reads issued ahead of this step's MFMAs:
        // without the fence the scheduler sinks them and re-waits on LDS
        // latency between MFMA groups.
        __builtin_amdgcn_sched_barrier(0);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) ga[i] = frag(As, wm + i * 32u, cg);
#pragma unroll
        for (int j = 0; j < 4; ++j) gb[j] = frag(Bs, wn + j * 32u, cg);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_32x32x16_16b<F16>(gb[j], ga[i], acc[i][j]);
      if (SPREAD && has1) {
        if (ks == 0) store_a(nbuf, 0);
        if (ks == 1) store_a(nbuf, 1);
        if (ks == 2) store_b(nbuf, 0);
        if (ks == 3) store_b(nbuf, 1);
      }
      if (SPREAD && has2) {
        if (ks == 1) load_a((kt + 2) * BK);
        if (ks == 3) load_b((kt + 2) * BK);
      }
    }
    if (!SPREAD && has1) {
      store_a(nbuf, 0);
      store_a(nbuf, 1);
      store_b(nbuf, 0);
      store_b(nbuf, 1);
    }
    __syncthreads();
  }
  // acc[i][j][4g + q] = C[m][n + q] with m = m0 + wm + 32i + lane%32 and
  // n = n0 + wn + 32j + 8g + 4*(lane/32).
  const uint32_t mr = m0 + wm + (lane & 31u), nc = n0 + wn + 4u * (lane >> 5);
  if (m0 + BM <= M && n0 + BN <= N && (N % 4u) == 0u) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t m = mr + 32u * i, n = nc + 32u * j + 8u * g;
          float4 v;
          v.x = epi(acc[i][j][4 * g + 0], m, n + 0);
          v.y = epi(acc[i][j][4 * g + 1], m, n + 1);
          v.z = epi(acc[i][j][4 * g + 2], m, n + 2);
          v.w = epi(acc[i][j][4 * g + 3], m, n + 3);
          *reinterpret_cast<float4*>(C + static_cast<uint64_t>(m) * N + n) = v;
        }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t m = mr + 32u * i, n = nc + 32u * j + 8u * (e >> 2) + (e & 3);
        if (m < M && n < N) C[static_cast<uint64_t>(m) * N + n] = epi(acc[i][j][e], m, n);
      }
}

// -------------------------------------------- bf16 path, 8 waves per tile
// The direct-to-LDS tiles (gemm_bf16_dma_tile): 512 threads, 2 waves per
// SIMD, each wave 128x64 of C as 8x4 blocks of v_mfma_f32_16x16x32_bf16
// (32 accumulators of 4, 225 VGPRs, no scratch).
//
// Why 16x16x32: the part is power-limited under dense MFMA load. On random
// bf16 operands an MFMA-only loop sustains 1.78 PFLOP/s with 32x32x16 (the
// clock drops to 1.81 GHz) and 2.04 PFLOP/s with 16x16x32 (2.05 GHz): half
// the accumulator traffic per flop. The operand bytes per flop, and so the
// LDS traffic, are the same for both shapes.
//
// K advances in 32-deep slices through a 4-slice ring of A [256][32] and
// [K][N] B [32][256] (or [N][K] B [256][32]) tiles, 32 KiB per slice,
// filled by global_load_lds_dwordx4 (lane i of a load writes bytes
// [16i, 16i + 16) of a 1 KiB LDS chunk, from any global address, so each
// lane's global address is the inverse of the LDS swizzle). Each slice is
// two halves of 16 MFMAs per wave:
//   half 0: A rows 0-63 of the wave x B; reads A rows 64-127 of the slice;
//   barrier (slice s+1 has landed, every wave is done with slice s-1);
//   half 1: A rows 64-127 x B; reads A rows 0-63 and B of slice s+1 into the
//           other B register set, and issues slice s+3 into slice s-1's
//           buffer, one load per quarter of the half (issued in a burst,
//           the 8 waves' loads stall their MFMA issue).
// Two slices per loop iteration, so the two B register sets alternate
// without copies; the last three slices, which load nothing, are a tail.
//
// LDS banks (measured with SQ_LDS_BANK_CONFLICT on gfx950): a 128-bit read
// is served per half-wave, in two 16-lane cycles split by the parity of
// lane bits 2^3^4; a 64-bit transposing read serves a half-wave per cycle.
// The swizzles below keep every cycle on 16 distinct 16-byte bank slots:
//   [rows][32] (64-byte rows): column group cg of row r at cg ^ 2*((r/8)%2);
//     a fragment read takes 16 rows x 4 groups (lane l: row l%16, group l/16);
//   [K][N] B (512-byte rows): 16-byte slot n/8 of row k at
//     (n/8) ^ 2*((k%4) + 4*((k/8)%2)); a transposing fragment read takes rows
//     8g..8g+3 (+4) of one 16-column block for lane group g.
__device__ __forceinline__ uint32_t swz_rows32(uint32_t row, uint32_t cg) {
  return row * 32u + ((cg ^ (((row >> 3) & 1u) << 1)) << 3);
}
__device__ __forceinline__ uint32_t kn_xor(uint32_t k) { return ((k & 3u) | (((k >> 3) & 1u) << 2)) << 1; }
__device__ __forceinline__ uint32_t swz_kn16(uint32_t k, uint32_t n) {
  return k * 256u + (((n >> 3) ^ kn_xor(k)) << 3) + (n & 7u);
}

// B operand of v_mfma_f32_16x16x32_bf16 (lane l: column n_col0 + l%16,
// k = 8(l/16) .. +8) from a [K][N] slice with the gfx950 transposing read
// ds_read_b64_tr_b16: within each 16-lane group, lane j points at four
// consecutive values R_j of one k row and lane i receives
// [R_{i/4}[i%4], R_{4+i/4}[i%4], R_{8+i/4}[i%4], R_{12+i/4}[i%4]]. With lane j
// addressing row kb + j/4, columns n_col0 + 4(j%4), lane i gets
// B[kb + e][n_col0 + i] for e = 0..3; a second read at kb + 4 completes its 8.
__device__ __forceinline__ bf16x8 frag_b16_tr(const uint16_t* Bs, uint32_t n_col0, uint32_t lane) {
  const uint32_t g = lane >> 4, j = lane & 15u;
  const uint32_t k = 8u * g + (j >> 2), n = n_col0 + 4u * (j & 3u);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(Bs + swz_kn16(k, n)));
  const i16x4 hi =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(Bs + swz_kn16(k + 4u, n)));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// Every other tile returns at once: gemm_bf16_256<..., SKIP_DMA> takes them.
// With K % 64 == 0 and K >= 256 the launch takes gemm_bf16_4w instead (4
// waves of 128x128, A in 64-deep slices, below).
template <bool B_NK, typename Epi, uint32_t STAGES = 4, bool F16 = false>
__device__ __forceinline__ void gemm_bf16_256_w8(const __bf16* __restrict__ A, const __bf16* __restrict__ B,
                                                 float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, Epi epi,
                                                 uint32_t tile = ~0u) {
  static_assert(STAGES == 4 || STAGES == 5, "a ring of 4 or 5 slices (160 KiB of LDS at most)");
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr uint32_t BM = 256, BN = 256, BK = 32, SLICE = 256u * BK;
  __shared__ __attribute__((aligned(16))) uint16_t lds[STAGES * 2 * SLICE];
  const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  uint32_t tm, tn;
  gemm_tile_coords(tiles_m, tiles_n, &tm, &tn, tile == ~0u ? blockIdx.x : tile);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  if (!gemm_bf16_dma_tile(m0, n0, M, N, K)) return;  // gemm_bf16_256<..., SKIP_DMA> takes it
  // The wave index is uniform over the wave: computed in a scalar register,
  // the LDS destination of every direct-to-LDS load (the m0 operand) is a
  // scalar value, with no readfirstlane per load.
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = (wave >> 2) * 128u, wn = (wave & 3u) * 64u;
  const uint16_t* __restrict__ A16 = reinterpret_cast<const uint16_t*>(A);
  const uint16_t* __restrict__ B16 = reinterpret_cast<const uint16_t*>(B);
  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;
  // Per-lane element offsets of the 2 chunks (of 16) this wave fills per
  // slice and operand: chunk ch = 2*wave + q covers LDS slots 64ch .. +63.
  uint32_t offa[2], offb[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const uint32_t slot = (wave * 2u + q) * 64u + lane;
    const uint32_t r = slot >> 2, c = (slot & 3u) ^ (((r >> 3) & 1u) << 1);  // inverse of swz_rows32
    offa[q] = r * K + c * 8u;
    if constexpr (B_NK) {
      offb[q] = r * K + c * 8u;
    } else {
      const uint32_t k = slot >> 5, sp = slot & 31u;  // [32][256]: 32 slots per row
      offb[q] = k * N + ((sp ^ kn_xor(k)) << 3);
    }
  }
  uint16_t* ldsp = lds;
  auto a_slice = [&](uint32_t s) { return ldsp + s * 2u * SLICE; };
  auto b_slice = [&](uint32_t s) { return ldsp + s * 2u * SLICE + SLICE; };
  auto load = [&](int q, uint32_t s, uint32_t k0) {  // q even: A chunk q/2, q odd: B chunk q/2
    const uint32_t ch = wave * 2u + (q >> 1);
    if (q & 1) {
      const uint16_t* b0 = B_NK ? B16 + static_cast<uint64_t>(n0) * K + k0 : B16 + static_cast<uint64_t>(k0) * N + n0;
      __builtin_amdgcn_global_load_lds(b0 + offb[q >> 1], (lds_void*)(b_slice(s) + ch * 512u), 16, 0, 0);
    } else {
      const uint16_t* a0 = A16 + static_cast<uint64_t>(m0) * K + k0;
      __builtin_amdgcn_global_load_lds(a0 + offa[q >> 1], (lds_void*)(a_slice(s) + ch * 512u), 16, 0, 0);
    }
  };
  auto rd_a = [&](const uint16_t* As, uint32_t i) {  // A rows wm + 16i .. +16, all 32 k
    return *reinterpret_cast<const bf16x8*>(&As[swz_rows32(wm + i * 16u + (lane & 15u), lane >> 4)]);
  };
  auto rd_b = [&](const uint16_t* Bs, uint32_t j) {  // B columns wn + 16j .. +16, all 32 k
    if constexpr (B_NK)
      return *reinterpret_cast<const bf16x8*>(&Bs[swz_rows32(wn + j * 16u + (lane & 15u), lane >> 4)]);
    else
      return frag_b16_tr(Bs, wn + j * 16u, lane);
  };
  bf16x8 fa[4], fh[4], fb0[4], fb1[4];  // A rows 0-63, A rows 64-127, the two B sets
  auto fence = []() { __builtin_amdgcn_sched_barrier(0); };
  // The MFMA takes the B fragment as its first operand: it computes the C^T
  // block, so each lane ends up holding four consecutive columns of one row
  // of C (a 16-byte store). Each group below is fenced with sched_barrier:
  // left to itself the scheduler sinks the fragment reads behind the MFMAs.
  // MFMA number c of a half (0..15) takes block (i, j) in snake order,
  // j = c/4 and i = c%4 or 3 - c%4 for odd j, so consecutive MFMAs share an
  // operand register (measured: about 3% faster at 4096^3 than j-major,
  // the part being power-limited).
  auto blk_i = [](int c) { return ((c >> 2) & 1) ? 3 - (c & 3) : (c & 3); };
  auto half0 = [&](auto set, uint32_t s) {
    bf16x8* gb = decltype(set)::value == 0 ? fb0 : fb1;
    const uint16_t* As = a_slice(s);
    auto mf = [&](int c) {
      const int i = blk_i(c), j = c >> 2;
      acc[i][j] = mfma_16x16x32_16b<F16>(gb[j], fa[i], acc[i][j]);
      fence();
    };
    fence();
    mf(0);
    fh[0] = rd_a(As, 4); fh[1] = rd_a(As, 5); fence();
    mf(1);
    fh[2] = rd_a(As, 6); fh[3] = rd_a(As, 7); fence();
#pragma unroll
    for (int c = 2; c < 16; ++c) mf(c);
  };
  auto half1 = [&](auto set, uint32_t ns, bool dma, uint32_t ds, uint32_t dk) {
    bf16x8* gb = decltype(set)::value == 0 ? fb0 : fb1;
    bf16x8* nb = decltype(set)::value == 0 ? fb1 : fb0;
    const uint16_t* As = a_slice(ns);
    const uint16_t* Bs = b_slice(ns);
    auto mf = [&](int c) {
      const int i = blk_i(c), j = c >> 2;
      acc[4 + i][j] = mfma_16x16x32_16b<F16>(gb[j], fh[i], acc[4 + i][j]);
      fence();
    };
    auto dm = [&](int q) {
      if (dma) load(q, ds, dk);
      fence();
    };
    fence();
    mf(0);
    fa[0] = rd_a(As, 0); fa[1] = rd_a(As, 1); fence();
    mf(1);
    fa[2] = rd_a(As, 2); fa[3] = rd_a(As, 3); fence();
    mf(2);
    nb[0] = rd_b(Bs, 0); fence();
    mf(3);
    nb[1] = rd_b(Bs, 1); fence();
    mf(4);
    nb[2] = rd_b(Bs, 2); fence();
    mf(5);
    nb[3] = rd_b(Bs, 3); fence();
    mf(6); dm(0);
    mf(7);
    mf(8); dm(1);
    mf(9);
    mf(10); dm(2);
    mf(11);
    mf(12); dm(3);
    mf(13); mf(14); mf(15);
  };
  // The barrier waits only for the slice about to be read (vmcnt counts in
  // issue order, 4 loads per slice and lane); its lgkmcnt leaves half 0's 4
  // fragment reads in flight but guarantees that every earlier read, the
  // last ones of the buffer the next loads overwrite, has completed: LDS
  // reads complete in order.
  constexpr int kReads = 4;
  auto wait_slices = [](uint32_t d, bool keep_reads) {  // at most d slices of loads still in flight
    if (keep_reads) {
      if (d >= 3u) __builtin_amdgcn_s_waitcnt(waitcnt_imm(12, kReads));
      else if (d == 2u) __builtin_amdgcn_s_waitcnt(waitcnt_imm(8, kReads));
      else if (d == 1u) __builtin_amdgcn_s_waitcnt(waitcnt_imm(4, kReads));
      else __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, kReads));
    } else {
      if (d >= 3u) __builtin_amdgcn_s_waitcnt(waitcnt_imm(12, 0));
      else if (d == 2u) __builtin_amdgcn_s_waitcnt(waitcnt_imm(8, 0));
      else if (d == 1u) __builtin_amdgcn_s_waitcnt(waitcnt_imm(4, 0));
      else __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    }
  };
  auto barrier = [&]() {
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;
  const uint32_t nk = K / BK;
  const uint32_t pre = nk < STAGES - 1 ? nk : STAGES - 1;
  for (uint32_t s = 0; s < pre; ++s)
    for (int q = 0; q < 4; ++q) load(q, s, s * BK);
  asm volatile("" ::: "memory");
  wait_slices(pre - 1u, false);  // slice 0 landed
  barrier();
  // Main slices kt < nk - (STAGES - 1) load slice kt + STAGES - 1: at the
  // barrier of slice kt, slices up to kt + STAGES - 2 were issued and kt+1
  // must have landed (STAGES - 3 newer slices may remain in flight).
  const uint32_t main_end = nk > STAGES - 1 ? nk - (STAGES - 1) : 0u;
  auto main_slice = [&](auto set, uint32_t kt) {
    half0(set, kt % STAGES);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(4 * static_cast<int>(STAGES - 3), kReads));
    barrier();
    half1(set, (kt + 1) % STAGES, true, (kt + STAGES - 1) % STAGES, (kt + STAGES - 1) * BK);
  };
  auto tail_slice = [&](auto set, uint32_t kt) {
    half0(set, kt % STAGES);
    if (kt + 1 < nk) {
      asm volatile("" ::: "memory");
      wait_slices(nk - 2u - kt, true);
      barrier();
    }
    half1(set, (kt + 1) % STAGES, false, 0, 0);  // the last one reads a stale buffer whose values are unused
  };
  // Slice 0's B fragments go into the set that makes the paired loop start on set 0.
  const bool odd = (main_end & 1u) != 0u;
  {
    const uint16_t* As = a_slice(0);
    const uint16_t* Bs = b_slice(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) fa[i] = rd_a(As, i);
    if (odd) {
#pragma unroll
      for (int j = 0; j < 4; ++j) fb1[j] = rd_b(Bs, j);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) fb0[j] = rd_b(Bs, j);
    }
  }
  uint32_t kt = 0;
  if (odd) {
    main_slice(Set1{}, 0);
    kt = 1;
  }
  for (; kt < main_end; kt += 2) {
    main_slice(Set0{}, kt);
    main_slice(Set1{}, kt + 1);
  }
  if (main_end < nk) tail_slice(Set0{}, main_end);
  if (main_end + 1 < nk) tail_slice(Set1{}, main_end + 1);
  if (main_end + 2 < nk) tail_slice(Set0{}, main_end + 2);
  if (STAGES > 4 && main_end + 3 < nk) tail_slice(Set1{}, main_end + 3);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));  // nothing in flight past the loop
  // acc[i][j][e] = C[m][n], m = m0 + wm + 16i + lane%16, n = n0 + wn + 16j + 4(lane/16) + e.
  const uint32_t mr = m0 + wm + (lane & 15u), nc = n0 + wn + 4u * (lane >> 4);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t m = mr + 16u * i, n = nc + 16u * j;
      float4 v;
      v.x = epi(acc[i][j][0], m, n + 0);
      v.y = epi(acc[i][j][1], m, n + 1);
      v.z = epi(acc[i][j][2], m, n + 2);
      v.w = epi(acc[i][j][3], m, n + 3);
      *reinterpret_cast<float4*>(C + static_cast<uint64_t>(m) * N + n) = v;
    }
}

// ------------------------------------- bf16 path, 4 waves, 128x128 per wave
// Whole 256x256 tiles with K % 64 == 0 and K >= 256 (the launch guards pick
// this kernel): 256 threads, one wave per SIMD, each wave a 128x128 sub-tile
// of C as 8x8 blocks of v_mfma_f32_16x16x32_bf16, accumulators in AGPRs
// (256 per lane), 160 VGPRs. Against 8 waves of 128x64 this reads a third
// less LDS per flop (each A and B fragment feeds 8 blocks instead of 4 or 8
// and 4), which leaves more of the power budget to the MFMAs: measured
// interleaved with the 8-wave kernel on one box, 4096^3 with rotated inputs
// 105.0-105.6 against 107.9-112.4 us, 8192^3 1356-1371 against 1335-1344
// TFLOP/s, K = 16384 +2%, results bitwise equal.
// LDS: A in 64-deep slices ([256][64], 128-byte rows, whole cache lines per
// direct-to-LDS load) in a 3-buffer ring, B in 32-deep slices in a 4-buffer
// ring, 160 KiB in all; slot s (32 deep) is k half s%2 of A slice s/2 and B
// slice s.
// Step kt: wait until slot kt+1 has landed and every read of slot kt has
// completed, one barrier, then 64 MFMAs on the fragments of slot kt (read
// during step kt-1) while this step reads all fragments of slot kt+1 into
// the other register set and loads part kt%2 of A slice kt/2+2 (into the
// buffer of A slice kt/2-1, last read during step kt-2) and B slice kt+4
// (into slot kt's buffer).
// The MFMAs are inline asm with the accumulator tied to one AGPR quad: the
// compiler's own MFMA, given 256 accumulators, splits them between AGPRs and
// VGPRs and moves them inside the loop (or spills). The hazards its
// recogniser does not see for inline asm are covered here:
//   the zero-initialised AGPRs are fixed (an empty asm per accumulator, so
//   no zero is re-materialised later) and 16 wait states separate the last
//   write from the first MFMA (VALU write -> MFMA SrcC read);
//   24 wait states separate the last MFMA from the epilogue's AGPR reads
//   (an 8-pass XDL write -> VALU/VMEM read);
//   the MFMA A/B operands are ds_read results only (a host test checks the
//   assembly: no VALU writes an MFMA source register), whose completion
//   s_waitcnt covers; an MFMA's accumulator is written again only by the
//   64th MFMA after it.
typedef float f32x4_t __attribute__((ext_vector_type(4)));
template <bool F16 = false>
__device__ __forceinline__ void mfma16_bf16_acc(f32x4_t& c, const bf16x8& b, const bf16x8& a) {
  if constexpr (F16)
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(b), "v"(a));
  else
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(b), "v"(a));
}

__device__ __forceinline__ uint32_t swz_rows64(uint32_t row, uint32_t g) { return row * 64u + ((g ^ (row & 6u)) << 3); }

template <bool B_NK, typename Epi, bool F16 = false>
__device__ __forceinline__ void gemm_bf16_4w(const __bf16* __restrict__ A, const __bf16* __restrict__ B,
                                             float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, Epi epi,
                                             uint32_t tile = ~0u) {
  constexpr uint32_t BM = 256, BN = 256, ASL = 256u * 64u, BSL = 256u * 32u;
  __shared__ __attribute__((aligned(16))) uint16_t lds[3 * ASL + 4 * BSL];
  const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  uint32_t tm, tn;
  gemm_tile_coords(tiles_m, tiles_n, &tm, &tn, tile == ~0u ? blockIdx.x : tile);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  if (!gemm_bf16_dma_tile(m0, n0, M, N, K) || K % 64u != 0u || K < 256u) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = (wave >> 1) * 128u, wn = (wave & 1u) * 128u;
  const uint16_t* __restrict__ A16 = reinterpret_cast<const uint16_t*>(A);
  const uint16_t* __restrict__ B16 = reinterpret_cast<const uint16_t*>(B);
  f32x4_t acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" : "+a"(acc[i][j]));
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // Per-lane element offsets of the 4 chunks this wave fills per A part
  // (16 chunks of 8 rows x 128 bytes; wave w: chunks 4w .. 4w+3) and per B
  // slice (16 chunks of 64 16-byte slots).
  uint32_t offa[4], offb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t row = 32u * wave + 8u * q + (lane >> 3);
    offa[q] = row * K + (((lane & 7u) ^ (row & 6u)) << 3);  // inverse of swz_rows64
    const uint32_t slot = (wave * 4u + q) * 64u + lane;
    if constexpr (B_NK) {
      const uint32_t r = slot >> 2, c = (slot & 3u) ^ (((r >> 3) & 1u) << 1);  // inverse of swz_rows32
      offb[q] = r * K + c * 8u;
    } else {
      const uint32_t k = slot >> 5, sp = slot & 31u;  // [32][256]: 32 slots per row
      offb[q] = k * N + ((sp ^ kn_xor(k)) << 3);
    }
  }
  uint16_t* ldsp = lds;
  auto a_buf = [&](uint32_t j) { return ldsp + (j % 3u) * ASL; };
  auto b_buf = [&](uint32_t s) { return ldsp + 3u * ASL + (s & 3u) * BSL; };
  auto load_b = [&](int q, uint32_t s) {
    const uint32_t k0 = s * 32u;
    const uint16_t* b0 = B_NK ? B16 + static_cast<uint64_t>(n0) * K + k0 : B16 + static_cast<uint64_t>(k0) * N + n0;
    __builtin_amdgcn_global_load_lds(b0 + offb[q], (lds_void*)(b_buf(s) + (wave * 4u + q) * 512u), 16, 0, 0);
  };
  auto load_a = [&](int q, uint32_t j, uint32_t p) {  // part p (rows 128p .. +127) of A slice j
    const uint16_t* a0 = A16 + static_cast<uint64_t>(m0 + 128u * p) * K + j * 64u;
    __builtin_amdgcn_global_load_lds(a0 + offa[q], (lds_void*)(a_buf(j) + (16u * p + wave * 4u + q) * 512u), 16, 0, 0);
  };
  auto rd_a = [&](uint32_t s, uint32_t i) {  // slot s: A rows wm + 16i .. +16
    const uint16_t* As = a_buf(s >> 1);
    return *reinterpret_cast<const bf16x8*>(&As[swz_rows64(wm + i * 16u + (lane & 15u), 4u * (s & 1u) + (lane >> 4))]);
  };
  auto rd_b = [&](uint32_t s, uint32_t j) {  // slot s: B columns wn + 16j .. +16
    const uint16_t* Bs = b_buf(s);
    if constexpr (B_NK)
      return *reinterpret_cast<const bf16x8*>(&Bs[swz_rows32(wn + j * 16u + (lane & 15u), lane >> 4)]);
    else
      return frag_b16_tr(Bs, wn + j * 16u, lane);
  };
  bf16x8 a0s[8], b0s[8], a1s[8], b1s[8];  // two fragment sets: this step's and the next one's
  auto fence = []() { __builtin_amdgcn_sched_barrier(0); };
  auto barrier = [&]() {
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // MFMA c (0..63) takes block (i, j) with j = c/8 and i snaking over 0..7,
  // so consecutive MFMAs share an operand register. The operand-swapped
  // MFMA computes the C^T block: each lane ends up holding four consecutive
  // columns of one row of C (a 16-byte store).
  // wait_vm: the loads that may remain in flight at the start of the step
  // (-1: no wait and no barrier, the last step).
  auto step = [&](auto set, uint32_t kt, int wait_vm, bool rd, bool ld) {
    bf16x8* ca = decltype(set)::value == 0 ? a0s : a1s;
    bf16x8* cb = decltype(set)::value == 0 ? b0s : b1s;
    bf16x8* na = decltype(set)::value == 0 ? a1s : a0s;
    bf16x8* nb = decltype(set)::value == 0 ? b1s : b0s;
    if (wait_vm >= 0) {
      asm volatile("" ::: "memory");
      if (wait_vm == 16) __builtin_amdgcn_s_waitcnt(waitcnt_imm(16, 0));
      else if (wait_vm == 8) __builtin_amdgcn_s_waitcnt(waitcnt_imm(8, 0));
      else __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
      barrier();
    }
    const uint32_t ns = kt + 1u;
    auto mf = [&](int c) {
      const int j = c >> 3, i = (j & 1) ? 7 - (c & 7) : (c & 7);
      mfma16_bf16_acc<F16>(acc[i][j], cb[j], ca[i]);
      fence();
    };
    auto da = [&](int q) { if (ld) load_a(q, (kt >> 1) + 2u, kt & 1u); fence(); };
    auto db = [&](int q) { if (ld) load_b(q, kt + 4u); fence(); };
    fence();
    if (rd) {
#pragma unroll
      for (int c = 0; c < 8; ++c) { mf(c); na[c] = rd_a(ns, c); fence(); }
#pragma unroll
      for (int c = 0; c < 8; ++c) { mf(8 + c); nb[c] = rd_b(ns, c); fence(); }
    } else {
#pragma unroll
      for (int c = 0; c < 16; ++c) mf(c);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      mf(16 + 8 * q); mf(17 + 8 * q); mf(18 + 8 * q); mf(19 + 8 * q); da(q);
      mf(20 + 8 * q); mf(21 + 8 * q); mf(22 + 8 * q); mf(23 + 8 * q); db(q);
    }
#pragma unroll
    for (int c = 48; c < 64; ++c) mf(c);
  };
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;
  const uint32_t nk = K / 32u;
  // Prologue: A0 (8 loads), B0 (4), B1 (4), A1 (8), B2 (4), B3 (4); A0 and B0 landed: 20 newer may remain.
  for (int q = 0; q < 4; ++q) load_a(q, 0, 0);
  for (int q = 0; q < 4; ++q) load_a(q, 0, 1);
  for (int q = 0; q < 4; ++q) load_b(q, 0);
  for (int q = 0; q < 4; ++q) load_b(q, 1);
  for (int q = 0; q < 4; ++q) load_a(q, 1, 0);
  for (int q = 0; q < 4; ++q) load_a(q, 1, 1);
  for (int q = 0; q < 4; ++q) load_b(q, 2);
  for (int q = 0; q < 4; ++q) load_b(q, 3);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(20, 0));
  barrier();
#pragma unroll
  for (int i = 0; i < 8; ++i) a0s[i] = rd_a(0, i);
#pragma unroll
  for (int j = 0; j < 8; ++j) b0s[j] = rd_b(0, j);
  // Loads run while kt < nk - 4 (8 per step). At the start of step kt slot
  // kt+1 must have landed: for even kt the loads of step kt-3 (16 newer may
  // remain), for odd kt the A part of step kt-2 (8 newer); in the prologue's
  // place the same counts are conservative. vmcnt counts in issue order.
  const uint32_t main_end = nk - 4u;  // even: K % 64 == 0
  for (uint32_t kt = 0; kt < main_end; kt += 2) {
    step(Set0{}, kt, 16, true, true);
    step(Set1{}, kt + 1, 8, true, true);
  }
  step(Set0{}, nk - 4u, 16, true, false);
  step(Set1{}, nk - 3u, 0, true, false);  // no loads after those of step nk-5
  step(Set0{}, nk - 2u, 0, true, false);
  step(Set1{}, nk - 1u, -1, false, false);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // acc[i][j][e] = C[m][n], m = m0 + wm + 16i + lane%16, n = n0 + wn + 16j + 4(lane/16) + e.
  const uint32_t mr = m0 + wm + (lane & 15u), nc = n0 + wn + 4u * (lane >> 4);
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t m = mr + 16u * i, n = nc + 16u * j;
      float4 v;
      v.x = epi(acc[i][j][0], m, n + 0);
      v.y = epi(acc[i][j][1], m, n + 1);
      v.z = epi(acc[i][j][2], m, n + 2);
      v.w = epi(acc[i][j][3], m, n + 3);
      *reinterpret_cast<float4*>(C + static_cast<uint64_t>(m) * N + n) = v;
    }
}

// ---------------------------------------------------------------- fp32 path
// Tile: BM x BN with BM, BN in {128, 256}, BK-deep slices; (BM/64)x(BN/64)
// waves, each 64x64 = 2x2 blocks of v_mfma_f32_32x32x2f32, 4 waves per SIMD
// (256x256: one 72 KiB block of 16 waves per CU; 128x128: four 38 KiB
// blocks of 4 waves), at most 128 registers per lane. fp32 MFMA is not
// power-limited on this part (an MFMA-only loop on random operands holds
// 2.4 GHz), so the loop is built for issue:
//   two LDS buffers, one barrier per slice: slice kt+1 is loaded into
//   registers when slice kt starts and written into the other buffer half
//   way through slice kt's MFMAs (every wave passed the barrier after that
//   buffer's last reads);
//   each 2-deep k step's fragments are read one step ahead;
//   strides chosen so a fragment read (32 rows or columns at k, the other
//   32 lanes at k+1) covers 64 distinct banks: LDA = BK + 2 (LDA/2 odd),
//   [K][N] B rows of BN + 32 floats (the k+1 row lands 32 banks over).
// Measured at 4096^3 (interleaved, one box, bitwise-equal results), TFLOP/s:
// this loop on 128x128 tiles with 4 waves 133, 256x128 with 8 waves 135,
// 256x256 with 16 waves 137 (the larger tiles read the L2 less per flop,
// but leave CUs idle below 256 tiles: the emitter takes 256x256 tiles from
// M, N >= 4096 on and 128x128 tiles below); the earlier single-buffer
// 128x128 loop with stride BK + 1, 117; 16x16x4f32 blocks on the 128x128
// loop, 127.
template <bool B_NK, int BM, int BN, int BK = 16, typename Epi>
__device__ __forceinline__ void gemm_f32_tile(const float* __restrict__ A, const float* __restrict__ B,
                                              float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, Epi epi,
                                              uint32_t tile = ~0u) {
  static_assert((BM == 128 || BM == 256) && BM == BN, "square 128 or 256 tiles");
  static_assert(BK == 16 || BK == 32, "slices of 16 or 32");
  constexpr int WN = BN / 64, THREADS = 64 * (BM / 64) * WN;
  constexpr int LPT = BM * BK / 4 / THREADS;    // float4 per thread per operand slice
  constexpr uint32_t VPN = BN / 4;              // float4 per [K][N] panel row
  constexpr int LDA = BK + 2;                   // As[m][k]
  constexpr int LDB = B_NK ? BK + 2 : BN + 32;  // Bs[n][k] (NK) or Bs[k][n] (KN)
  constexpr int SA = BM * LDA, SB = B_NK ? BN * LDB : BK * LDB;
  __shared__ __attribute__((aligned(16))) float lds[2 * (SA + SB)];
  const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  uint32_t tm, tn;
  gemm_tile_coords(tiles_m, tiles_n, &tm, &tn, tile == ~0u ? blockIdx.x : tile);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wm = (wave / WN) * 64u, wn = (wave % WN) * 64u;
  const bool vec_a = (K % 4u) == 0u;
  const bool vec_b = B_NK ? (K % 4u) == 0u : (N % 4u) == 0u;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  float4 ra[LPT], rb[LPT];
  // Row-major [rows][K] panel, BK columns: BM BK / 4 float4 -> LPT per thread.
  constexpr uint32_t VPR = BK / 4;  // float4 per panel row
  auto load_rows = [&](const float* __restrict__ P, uint32_t rows, uint32_t r0, uint32_t k0, bool vec, float4* r) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const uint32_t v = i * THREADS + tid, rr = v / VPR, kv = (v % VPR) * 4u;
      const uint32_t gr = r0 + rr, gk = k0 + kv;
      if (vec && gr < rows && gk + 4u <= K) {
        r[i] = *reinterpret_cast<const float4*>(P + static_cast<uint64_t>(gr) * K + gk);
      } else {
        float h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (gr < rows && gk + e < K) ? P[static_cast<uint64_t>(gr) * K + gk + e] : 0.0f;
        r[i] = make_float4(h[0], h[1], h[2], h[3]);
      }
    }
  };
  auto load_b_kn = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const uint32_t v = i * THREADS + tid, kr = v / VPN, nv = (v % VPN) * 4u;
      const uint32_t gk = k0 + kr, gn = n0 + nv;
      if (vec_b && gk < K && gn + 4u <= N) {
        rb[i] = *reinterpret_cast<const float4*>(B + static_cast<uint64_t>(gk) * N + gn);
      } else {
        float h[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (gk < K && gn + e < N) ? B[static_cast<uint64_t>(gk) * N + gn + e] : 0.0f;
        rb[i] = make_float4(h[0], h[1], h[2], h[3]);
      }
    }
  };
  // Interior tiles (the whole BMxBN block in range, rows 16-byte aligned,
  // K a multiple of BK) take unguarded float4 loads. The test is uniform
  // over the workgroup and made once, outside the K loop (two instances of
  // the loop): with per-lane guards alone the compiler merges the vector and
  // scalar paths into single-float loads under divergent branches, and with
  // the branch inside the loop the two paths join in register copies that
  // wait for the loads just issued (125 against 137 TFLOP/s).
  const bool interior = vec_a && vec_b && m0 + BM <= M && n0 + BN <= N && K % BK == 0u;
  auto load_interior = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const uint32_t v = i * THREADS + tid, rr = v / VPR, kv = (v % VPR) * 4u;
      ra[i] = *reinterpret_cast<const float4*>(A + static_cast<uint64_t>(m0 + rr) * K + k0 + kv);
      if constexpr (B_NK) {
        rb[i] = *reinterpret_cast<const float4*>(B + static_cast<uint64_t>(n0 + rr) * K + k0 + kv);
      } else {
        const uint32_t kr = v / VPN, nv = (v % VPN) * 4u;
        rb[i] = *reinterpret_cast<const float4*>(B + static_cast<uint64_t>(k0 + kr) * N + n0 + nv);
      }
    }
  };
  auto load_guarded = [&](uint32_t k0) {
    load_rows(A, M, m0, k0, vec_a, ra);
    if constexpr (B_NK) load_rows(B, N, n0, k0, vec_b, rb);
    else load_b_kn(k0);
  };
  // Rows of LDA (or LDB) floats are 8-byte aligned: a float4 of a [rows][k]
  // panel is written as two float2.
  auto store = [&](int buf) {
    float* As = lds + buf * (SA + SB);
    float* Bs = As + SA;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const uint32_t v = i * THREADS + tid, rr = v / VPR, kv = (v % VPR) * 4u;
      float2* p = reinterpret_cast<float2*>(&As[rr * LDA + kv]);
      p[0] = make_float2(ra[i].x, ra[i].y);
      p[1] = make_float2(ra[i].z, ra[i].w);
    }
    if constexpr (B_NK) {
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const uint32_t v = i * THREADS + tid, rr = v / VPR, kv = (v % VPR) * 4u;
        float2* p = reinterpret_cast<float2*>(&Bs[rr * LDB + kv]);
        p[0] = make_float2(rb[i].x, rb[i].y);
        p[1] = make_float2(rb[i].z, rb[i].w);
      }
    } else {
#pragma unroll
      for (int i = 0; i < LPT; ++i) {
        const uint32_t v = i * THREADS + tid, kr = v / VPN, nv = (v % VPN) * 4u;
        *reinterpret_cast<float4*>(&Bs[kr * LDB + nv]) = rb[i];
      }
    }
  };

  const uint32_t nk = (K + BK - 1) / BK;
  auto run = [&](auto load) {  // the K loop, on one of the two load paths
    if (nk > 0) {
      load(0);
      store(0);
    }
    __syncthreads();
    for (uint32_t kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      const float* As = lds + buf * (SA + SB);
      const float* Bs = As + SA;
      const bool more = kt + 1 < nk;
      if (more) load((kt + 1) * BK);
      float a0[2], b0[2], a1[2], b1[2];
      auto rd = [&](int ks, float (&fa)[2], float (&fb)[2]) {  // 2-deep step ks: lane l holds k = 2ks + l/32
        const uint32_t k = ks * 2u + (lane >> 5);
#pragma unroll
        for (int i = 0; i < 2; ++i) fa[i] = As[(wm + i * 32u + (lane & 31u)) * LDA + k];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint32_t n = wn + j * 32u + (lane & 31u);
          fb[j] = B_NK ? Bs[n * LDB + k] : Bs[k * LDB + n];
        }
      };
      auto mm = [&](const float (&fa)[2], const float (&fb)[2]) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
      };
      rd(0, a0, b0);
#pragma unroll
      for (int ks = 0; ks < BK / 2; ks += 2) {
        rd(ks + 1, a1, b1);
        mm(a0, b0);
        if (ks + 2 < BK / 2) rd(ks + 2, a0, b0);
        mm(a1, b1);
        if (ks == BK / 4 && more) store(buf ^ 1);
      }
      __syncthreads();
    }
  };
  if (interior) run(load_interior);
  else run(load_guarded);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t r = m0 + wm + i * 32u + 8u * (e >> 2) + 4u * (lane >> 5) + (e & 3);
        const uint32_t c = n0 + wn + j * 32u + (lane & 31u);
        if (r < M && c < N) C[static_cast<uint64_t>(r) * N + c] = epi(acc[i][j][e], r, c);
      }
}

// ------------------------------------- fp32 path, 4 waves, 128x128 per wave
// Whole 256x256 tiles with K % 32 == 0 and K >= 128 (the launch guards pick
// this kernel from M, N >= 4096 on): 256 threads, one wave per SIMD, each
// wave a 128x128 sub-tile of C as 4x4 blocks of v_mfma_f32_32x32x2f32,
// accumulators in AGPRs (256 per lane) through inline-asm MFMAs (the same
// scheme and hazard coverage as gemm_bf16_4w), about 150 VGPRs.
// LDS: a ring of 4 slots of 16-deep slices loaded straight from global
// memory (global_load_lds_dwordx4): A (and an [n][k] B) as [256][16] with
// the 16-byte chunk c of row r at c ^ ((r / 4) % 4), a [k][n] B as [16][264]
// (rows padded to 1056 bytes: the fragment read of rows k and k + 4 covers
// the 64 banks once). 133 KiB in all.
// Slice s: wait until slot s+1 has landed and every read of slot s has
// completed, one barrier, then 128 MFMAs on the fragments of slot s (read
// during slice s-1) while this slice reads all fragments of slot s+1 and
// loads slice s+4 into slot s's buffer.
// The 2-deep MFMA step (h, e) of a slice (h 0..1, e 0..3) takes k = 8h + e on
// lanes 0-31 and k = 8h + 4 + e on lanes 32-63, so a lane reads the four k
// of its row it needs for four steps with one 16-byte read (an [n][k] B
// too; a [k][n] B as four 4-byte reads). Every k of the slice is summed once;
// the order of the sums differs from gemm_f32_tile's.
// Measured interleaved with gemm_f32_tile<.., 256, 256> at 4096^3 (rotated
// inputs, one box): 945-947 against 1030-1033 us, 145.3 against 133.3
// TFLOP/s; the error against a float64 sum of the same products 6.95e-5
// against 8.37e-5 on 64 sampled elements.
typedef float f32x16_t __attribute__((ext_vector_type(16)));
__device__ __forceinline__ void mfma32_f32_acc(f32x16_t& c, float a, float b) {
  asm volatile("v_mfma_f32_32x32x2_f32 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>): a step's
// MFMAs with compile-time block indices (a loop over them is not unrolled
// by the compiler at this size, and run-time indices put the accumulators
// in scratch).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <bool B_NK, typename Epi>
__device__ __forceinline__ void gemm_f32_4w(const float* __restrict__ A, const float* __restrict__ B,
                                            float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, Epi epi,
                                            uint32_t tile = ~0u) {
  constexpr uint32_t BM = 256, BN = 256, ASL = 256u * 16u, LDBK = 264u, BSL = B_NK ? 256u * 16u : 16u * LDBK;
  constexpr uint32_t SLOT = ASL + BSL;
  __shared__ __attribute__((aligned(16))) float lds[4 * SLOT];
  const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  uint32_t tm, tn;
  gemm_tile_coords(tiles_m, tiles_n, &tm, &tn, tile == ~0u ? blockIdx.x : tile);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  if (m0 + BM > M || n0 + BN > N || K % 32u != 0u || K < 128u) return;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t wm = (wave >> 1) * 128u, wn = (wave & 1u) * 128u;
  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) asm volatile("" : "+a"(acc[i][j]));
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // A wave-load (1 KiB) fills 16 rows of a [256][16] slice, or one k row of
  // a [16][264] slice; wave w fills rows 16(4w) .. 16(4w+3)+15, or k rows
  // 4w .. 4w+3. Per-lane element offsets (the inverse of the chunk swizzle).
  uint32_t offa[4], offb[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t row = 16u * (4u * wave + q) + (lane >> 2);
    offa[q] = row * K + 4u * ((lane & 3u) ^ ((row >> 2) & 3u));
    if constexpr (B_NK) offb[q] = offa[q];
    else offb[q] = (4u * wave + q) * N + 4u * lane;
  }
  float* ldsp = lds;
  auto a_slot = [&](uint32_t s) { return ldsp + (s & 3u) * SLOT; };
  auto b_slot = [&](uint32_t s) { return ldsp + (s & 3u) * SLOT + ASL; };
  auto load = [&](int q, uint32_t s) {  // q 0..3: A rows, q 4..7: B rows
    const uint32_t k0 = s * 16u;
    if (q < 4) {
      const float* a0 = A + static_cast<uint64_t>(m0) * K + k0;
      __builtin_amdgcn_global_load_lds(a0 + offa[q], (lds_void*)(a_slot(s) + (4u * wave + q) * 256u), 16, 0, 0);
    } else if constexpr (B_NK) {
      const float* b0 = B + static_cast<uint64_t>(n0) * K + k0;
      __builtin_amdgcn_global_load_lds(b0 + offb[q - 4], (lds_void*)(b_slot(s) + (4u * wave + q - 4) * 256u), 16, 0, 0);
    } else {
      const float* b0 = B + static_cast<uint64_t>(k0) * N + n0;
      __builtin_amdgcn_global_load_lds(b0 + offb[q - 4], (lds_void*)(b_slot(s) + (4u * wave + q - 4) * LDBK), 16, 0, 0);
    }
  };
  auto rd_a = [&](uint32_t s, uint32_t i, uint32_t h) {  // rows wm + 32i + lane%32, k 8h + 4(lane/32) .. +3
    const float* As = a_slot(s);
    const uint32_t row = wm + 32u * i + (lane & 31u), c = 2u * h + (lane >> 5);
    return *reinterpret_cast<const f32x4_t*>(&As[row * 16u + 4u * (c ^ ((row >> 2) & 3u))]);
  };
  auto rd_b = [&](uint32_t s, uint32_t j, uint32_t h) {  // columns wn + 32j + lane%32, the same k
    const float* Bs = b_slot(s);
    const uint32_t col = wn + 32u * j + (lane & 31u);
    if constexpr (B_NK) {
      const uint32_t c = 2u * h + (lane >> 5);
      return *reinterpret_cast<const f32x4_t*>(&Bs[col * 16u + 4u * (c ^ ((col >> 2) & 3u))]);
    } else {
      const uint32_t k = 8u * h + 4u * (lane >> 5);
      f32x4_t v;
      v[0] = Bs[(k + 0u) * LDBK + col];
      v[1] = Bs[(k + 1u) * LDBK + col];
      v[2] = Bs[(k + 2u) * LDBK + col];
      v[3] = Bs[(k + 3u) * LDBK + col];
      return v;
    }
  };
  f32x4_t fa0[4][2], fb0[4][2], fa1[4][2], fb1[4][2];  // two fragment sets: this slice's and the next one's
  auto fence = []() { __builtin_amdgcn_sched_barrier(0); };
  auto barrier = [&]() {
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  auto step = [&](auto set, uint32_t s, int wait_vm, bool rd, bool ld) {
    auto& ca = decltype(set)::value == 0 ? fa0 : fa1;
    auto& cb = decltype(set)::value == 0 ? fb0 : fb1;
    auto& na = decltype(set)::value == 0 ? fa1 : fa0;
    auto& nb = decltype(set)::value == 0 ? fb1 : fb0;
    if (wait_vm >= 0) {
      asm volatile("" ::: "memory");
      if (wait_vm == 16) __builtin_amdgcn_s_waitcnt(waitcnt_imm(16, 0));
      else if (wait_vm == 8) __builtin_amdgcn_s_waitcnt(waitcnt_imm(8, 0));
      else __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
      barrier();
    }
    const uint32_t ns = s + 1u;
    fence();
    // MFMA c (0..127): 2-deep step t = c/16 (h = t/4, e = t%4), block (i, j)
    // snaking over 4x4. The next slot's 8 A and 8 B fragment reads follow
    // MFMAs 0..15, the 8 loads of slice s+4 MFMAs 55, 63, ..., 111.
    static_for<128>([&](auto ic) {
      constexpr int c = decltype(ic)::value;
      constexpr int t = c >> 4, h = t >> 2, e = t & 3, b = c & 15, i = b >> 2, j = (i & 1) ? 3 - (b & 3) : (b & 3);
      mfma32_f32_acc(acc[i][j], ca[i][h][e], cb[j][h][e]);
      fence();
      if constexpr (c < 16) {
        if (rd) {
          if constexpr (c < 8) na[c >> 1][c & 1] = rd_a(ns, c >> 1, c & 1);
          else nb[(c - 8) >> 1][(c - 8) & 1] = rd_b(ns, (c - 8) >> 1, (c - 8) & 1);
        }
        fence();
      }
      if constexpr (c >= 55 && (c - 55) % 8 == 0 && (c - 55) / 8 < 8) {
        if (ld) load((c - 55) / 8, s + 4u);
        fence();
      }
    });
  };
  using Set0 = std::integral_constant<int, 0>;
  using Set1 = std::integral_constant<int, 1>;
  const uint32_t nk = K / 16u;
  for (uint32_t s = 0; s < 4; ++s)
    for (int q = 0; q < 8; ++q) load(q, s);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(24, 0));  // slice 0 landed
  barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      fa0[i][h] = rd_a(0, i, h);
      fb0[i][h] = rd_b(0, i, h);
    }
  // At the start of slice s slot s+1 must have landed: the loads of slices
  // s+2 and s+3 may remain (16; vmcnt counts in issue order). The loop runs
  // at least once (K >= 128): a path around it kept the zeroed accumulators
  // live across an edge and spilled them.
  const uint32_t main_end = nk - 4u;  // even (K % 32 == 0), at least 4
  uint32_t s = 0;
  do {
    step(Set0{}, s, 16, true, true);
    step(Set1{}, s + 1, 16, true, true);
    s += 2;
  } while (s < main_end);
  step(Set0{}, nk - 4u, 16, true, false);
  step(Set1{}, nk - 3u, 8, true, false);
  step(Set0{}, nk - 2u, 0, true, false);
  step(Set1{}, nk - 1u, -1, false, false);
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
  __builtin_amdgcn_sched_barrier(0);
  // 32 wait states: a 16-pass XDL write before the epilogue reads the AGPRs.
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  // acc[i][j][e] = C[r][c], r = m0 + wm + 32i + 8(e/4) + 4(lane/32) + e%4, c = n0 + wn + 32j + lane%32.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t r = m0 + wm + i * 32u + 8u * (e >> 2) + 4u * (lane >> 5) + (e & 3);
        const uint32_t c = n0 + wn + j * 32u + (lane & 31u);
        C[static_cast<uint64_t>(r) * N + c] = epi(acc[i][j][e], r, c);
      }
}

// ------------------------------------------------ small contractions, K split
// The tile kernels above give one workgroup a 128x128 or 256x256 tile and
// the whole of K, so a contraction with few tiles (the reference suite's
// gemm, mlp, mm_* and qk_score have M, N <= 192: one or two workgroups) runs
// on one or two CUs, walking K alone (testing/kernels/tiling/mm_splitk.tca:1-2
// names the split-k schedule class for them). Here a workgroup of 16 waves
// owns a 32x32 tile of C and a chunk of K:
//   - the chunk's k steps (8 deep for f32, 16 deep for 16-bit inputs) are
//     dealt round-robin to the 16 waves; each wave accumulates the whole
//     32x32 tile in one MFMA block (4 x v_mfma_f32_32x32x2f32 per step, or
//     one v_mfma_f32_32x32x16_{bf16,f16});
//   - the waves' tiles meet in LDS and are summed in wave order;
//   - with P > 1 chunks (P = gemm_split_chunks(K, tiles, KCMIN, BLOCKS),
//     the formula of the launch plan's split record) the workgroup of chunk
//     p writes its sum to a partial scratch [P][tiles][1024] and a second
//     kernel (gemm_small_merge) adds the P partials in chunk order.
// Every order is fixed, so the result does not depend on the schedule.
// Operands go from memory straight into the MFMA operand registers (no LDS
// staging: the waves of a workgroup read disjoint k, so nothing is shared
// inside it; neighbouring tiles share panels through the L2):
//   f32 step at k0, lane l (r = l % 32, h = l / 32): A[m0+r][k0+4h+e] and
//   B[k0+4h+e][n0+r] for e = 0..3, one float4 where the operand is
//   K-contiguous; MFMA e sums k0+e (lanes 0-31) and k0+4+e (lanes 32-63), so
//   a step sums each of its 8 k once;
//   16-bit step at k0: lane l holds A[m0+r][k0+8h .. +7] and
//   B[k0+8h .. +7][n0+r] (the 32x32x16 operand layout), one MFMA.
// Result element i of lane l is C[m0 + 8(i/4) + 4(l/32) + i%4][n0 + l%32];
// a wave's tile goes to LDS element-major (word i*64 + l: conflict-free) and
// thread t = i*64 + l of the workgroup sums word t over the waves.
constexpr uint32_t kSmallWaves = 16;

// P chunks of K for `tiles` output tiles: enough workgroups to reach
// `blocks`, each chunk at least kc_min deep (1 when K or tiles is 0). The
// launch plan's split record computes the same number (SplitChunks).
__host__ __device__ __forceinline__ uint32_t gemm_split_chunks(uint32_t k, uint32_t tiles, uint32_t kc_min,
                                                               uint32_t blocks) {
  if (k == 0u || tiles == 0u) return 1u;
  uint32_t p = (k - 1u) / kc_min + 1u;
  const uint32_t cap = blocks / tiles;
  if (p > cap) p = cap;
  return p ? p : 1u;
}

// Coordinates (row, column) inside a 32x32 tile of the value thread t holds
// after the wave merge.
__device__ __forceinline__ uint32_t small_row(uint32_t t) {
  const uint32_t i = t >> 6, l = t & 63u;
  return 8u * (i >> 2) + 4u * (l >> 5) + (i & 3u);
}
__device__ __forceinline__ uint32_t small_col(uint32_t t) { return t & 31u; }

// A wave's steps of its chunk: s = s_begin + wave + j * kSmallWaves below
// s_end. Steps whose operands are all in range (an interior tile and a whole
// step of K) are loaded without guards, up to four before their MFMAs (the
// later ones under wave-uniform tests); the decision is made once, outside
// the loops: a load that could take either path inside the loop joins the
// two in register copies that wait for the loads just issued, which
// serialises the steps. The rest (at most one short step of K on interior
// tiles; every step of an edge tile) take the guarded loads one at a time.
// `load(fast, s, &a, &b)` loads step s into registers of type Reg,
// `mma(a, b)` accumulates it.
template <uint32_t KS, typename Reg, typename Load, typename Mma>
__device__ __forceinline__ void small_steps(uint32_t s_begin, uint32_t s_end, uint32_t wave, bool interior,
                                            uint32_t K, Load&& load, Mma&& mma) {
  using Fast = std::true_type;
  using Slow = std::false_type;
  constexpr uint32_t W = kSmallWaves;
  uint32_t s = s_begin + wave;
  if (interior) {
    const uint32_t whole = K / KS;  // steps lying wholly inside K
    const uint32_t fe = s_end < whole ? s_end : whole;
    // After a group, s moves past the steps it took: the next of this wave's
    // steps, so the guarded loop below starts at the first one at or past fe.
    for (; s < fe; s += W * (1u + (s + W < fe) + (s + 2u * W < fe) + (s + 3u * W < fe))) {
      const bool h1 = s + W < fe, h2 = s + 2u * W < fe, h3 = s + 3u * W < fe;
      Reg a0, b0, a1, b1, a2, b2, a3, b3;
      load(Fast{}, s, &a0, &b0);
      if (h1) load(Fast{}, s + W, &a1, &b1);
      if (h2) load(Fast{}, s + 2u * W, &a2, &b2);
      if (h3) load(Fast{}, s + 3u * W, &a3, &b3);
      mma(a0, b0);
      if (h1) mma(a1, b1);
      if (h2) mma(a2, b2);
      if (h3) mma(a3, b3);
    }
  }
  for (; s < s_end; s += W) {
    Reg a0, b0;
    load(Slow{}, s, &a0, &b0);
    mma(a0, b0);
  }
}

// `tile` is the tile within its contraction (row-major over ceil(N/32)
// columns of tiles), `gtile` the tile's index over all T tiles of the
// launch (batches included): the partial scratch is indexed by it.
template <bool H16, bool B_NK, typename Epi, bool F16 = false>
__device__ __forceinline__ void gemm_small(const void* __restrict__ Av, const void* __restrict__ Bv,
                                           float* __restrict__ C, float* __restrict__ part, uint32_t M, uint32_t N,
                                           uint32_t K, Epi epi, uint32_t tile, uint32_t gtile, uint32_t T, uint32_t p,
                                           uint32_t P) {
  constexpr uint32_t KS = H16 ? 16u : 8u;   // k per step
  constexpr uint32_t KPL = H16 ? 8u : 4u;   // k per lane and step
  __shared__ __attribute__((aligned(16))) float red[kSmallWaves * 1024u];
  const uint32_t tiles_n = (N + 31u) / 32u;
  const uint32_t m0 = (tile / tiles_n) * 32u, n0 = (tile % tiles_n) * 32u;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t r = lane & 31u, h = lane >> 5;
  const uint32_t am = m0 + r, bn = n0 + r;
  // Chunk p: whole steps [s_begin, s_end) (the last step of K may be short).
  const uint32_t steps = K / KS + (K % KS != 0u ? 1u : 0u);
  const uint32_t per = steps / P + (steps % P != 0u ? 1u : 0u);
  const uint32_t s_begin = p * per < steps ? p * per : steps;
  const uint32_t s_end = s_begin + per < steps ? s_begin + per : steps;
  // Unguarded vector loads: the whole tile in range and every lane's k run
  // 16-byte aligned (K a multiple of the run; the tensors are 16-byte
  // aligned and so is every batch's slice then).
  const bool interior = m0 + 32u <= M && n0 + 32u <= N && K % KPL == 0u;
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
  if constexpr (!H16) {
    const float* __restrict__ A = static_cast<const float*>(Av);
    const float* __restrict__ B = static_cast<const float*>(Bv);
    auto load = [&](auto fast, uint32_t s, float4* a, float4* b) {
      const uint32_t k0 = s * KS + KPL * h;
      if constexpr (decltype(fast)::value) {
        *a = *reinterpret_cast<const float4*>(A + static_cast<uint64_t>(am) * K + k0);
        if constexpr (B_NK) {
          *b = *reinterpret_cast<const float4*>(B + static_cast<uint64_t>(bn) * K + k0);
        } else {
          const float* q = B + static_cast<uint64_t>(k0) * N + bn;
          *b = make_float4(q[0], q[N], q[2u * N], q[3u * N]);
        }
        return;
      } else {
      float va[4], vb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t k = k0 + e;
        va[e] = (am < M && k < K) ? A[static_cast<uint64_t>(am) * K + k] : 0.0f;
        if constexpr (B_NK) vb[e] = (bn < N && k < K) ? B[static_cast<uint64_t>(bn) * K + k] : 0.0f;
        else vb[e] = (bn < N && k < K) ? B[static_cast<uint64_t>(k) * N + bn] : 0.0f;
      }
      *a = make_float4(va[0], va[1], va[2], va[3]);
      *b = make_float4(vb[0], vb[1], vb[2], vb[3]);
      }
    };
    auto mma = [&](const float4& a, const float4& b) {
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.x, b.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.y, b.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.z, b.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.w, b.w, acc, 0, 0, 0);
    };
    small_steps<KS, float4>(s_begin, s_end, wave, interior, K, load, mma);
  } else {
    const uint16_t* __restrict__ A = static_cast<const uint16_t*>(Av);
    const uint16_t* __restrict__ B = static_cast<const uint16_t*>(Bv);
    auto load = [&](auto fast, uint32_t s, u32x4* a, u32x4* b) {
      const uint32_t k0 = s * KS + KPL * h;
      if constexpr (decltype(fast)::value) {
        *a = *reinterpret_cast<const u32x4*>(A + static_cast<uint64_t>(am) * K + k0);
        if constexpr (B_NK) {
          *b = *reinterpret_cast<const u32x4*>(B + static_cast<uint64_t>(bn) * K + k0);
        } else {
          const uint16_t* q = B + static_cast<uint64_t>(k0) * N + bn;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            (*b)[e] = static_cast<uint32_t>(q[(2u * e) * N]) | (static_cast<uint32_t>(q[(2u * e + 1u) * N]) << 16);
        }
        return;
      } else {
      uint32_t va[8], vb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t k = k0 + e;
        va[e] = (am < M && k < K) ? A[static_cast<uint64_t>(am) * K + k] : 0u;
        if constexpr (B_NK) vb[e] = (bn < N && k < K) ? B[static_cast<uint64_t>(bn) * K + k] : 0u;
        else vb[e] = (bn < N && k < K) ? B[static_cast<uint64_t>(k) * N + bn] : 0u;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        (*a)[e] = va[2 * e] | (va[2 * e + 1] << 16);
        (*b)[e] = vb[2 * e] | (vb[2 * e + 1] << 16);
      }
      }
    };
    auto mma = [&](const u32x4& a, const u32x4& b) {
      acc = mfma_32x32x16_16b<F16>(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc);
    };
    small_steps<KS, u32x4>(s_begin, s_end, wave, interior, K, load, mma);
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) red[wave * 1024u + static_cast<uint32_t>(i) * 64u + lane] = acc[i];
  __syncthreads();
  float sum = red[tid];
#pragma unroll
  for (uint32_t w = 1; w < kSmallWaves; ++w) sum += red[w * 1024u + tid];
  if (P > 1u) {
    part[(static_cast<uint64_t>(p) * T + gtile) * 1024u + tid] = sum;
    return;
  }
  const uint32_t m = m0 + small_row(tid), n = n0 + small_col(tid);
  if (m < M && n < N) C[static_cast<uint64_t>(m) * N + n] = epi(sum, m, n);
}

// The P > 1 merge: one 1024-thread workgroup per tile, thread t adds word t
// of the tile's P partials in chunk order, applies the epilogue and stores.
template <typename Epi>
__device__ __forceinline__ void gemm_small_merge(float* __restrict__ C, const float* __restrict__ part, uint32_t M,
                                                 uint32_t N, Epi epi, uint32_t tile, uint32_t gtile, uint32_t T,
                                                 uint32_t P) {
  const uint32_t tid = threadIdx.x, tiles_n = (N + 31u) / 32u;
  const uint32_t m = (tile / tiles_n) * 32u + small_row(tid), n = (tile % tiles_n) * 32u + small_col(tid);
  const float* q = part + static_cast<uint64_t>(gtile) * 1024u + tid;
  const uint64_t stride = static_cast<uint64_t>(T) * 1024u;
  float sum = q[0];
  uint32_t c = 1;
  for (; c + 4u <= P; c += 4u) {
    const float v0 = q[c * stride], v1 = q[(c + 1u) * stride], v2 = q[(c + 2u) * stride], v3 = q[(c + 3u) * stride];
    sum += v0;
    sum += v1;
    sum += v2;
    sum += v3;
  }
  for (; c < P; ++c) sum += q[c * stride];
  if (m < M && n < N) C[static_cast<uint64_t>(m) * N + n] = epi(sum, m, n);
}

}  // namespace hip
}  // namespace tca

#endif  // TCA_HIP_GEMM_H_
