// gemm.h — dense K-contraction on CDNA4 matrix cores (family G).
//
// The reference lowers C[m,n] = sum_k A[m,k] B[k,n] as a CTA-wide
// WarpReducer collective per output element (a shuffle tree per Reduce and
// two barriers per Combine; .planning/quick/261030-uai-.../after-cu/gemm.cu:
// 59-90). Here the contraction runs on MFMA:
//   bf16 inputs : v_mfma_f32_32x32x16_bf16 (gfx950), fp32 accumulate
//   fp32 inputs : v_mfma_f32_32x32x2f32, fp32 accumulate
// Geometry: a 256-thread workgroup (4 waves, 2x2) owns a BMxBN tile of C,
// each wave a (BM/2)x(BN/2) sub-tile of 32x32 MFMA blocks. K advances in
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

namespace tca {
namespace hip {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Maps the linear workgroup id to a (tile_m, tile_n) pair. Workgroups are
// dealt round-robin over the 8 XCDs; regrouping so that each XCD receives a
// contiguous run of tiles (and walking those runs in GROUP_M-row bands) keeps
// the A row panels and B column panels a run touches inside one XCD's L2.
__device__ __forceinline__ void gemm_tile_coords(uint32_t tiles_m, uint32_t tiles_n, uint32_t* tm, uint32_t* tn) {
  const uint32_t total = tiles_m * tiles_n;
  uint32_t b = blockIdx.x;
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

// ---------------------------------------------------------------- bf16 path
// Tile: BM = BN = 128, BK = 64; 4 waves as 2x2, each 64x64 = 2x2 MFMA blocks.
template <bool B_NK, typename Epi>
__device__ __forceinline__ void gemm_bf16_128(const __bf16* __restrict__ A, const __bf16* __restrict__ B,
                                              float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, Epi epi) {
  constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;  // 8 bf16 = 16 B of padding per row
  __shared__ __attribute__((aligned(16))) __bf16 As[BM * LDK];
  __shared__ __attribute__((aligned(16))) __bf16 Bs[BN * LDK];
  const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  uint32_t tm, tn;
  gemm_tile_coords(tiles_m, tiles_n, &tm, &tn);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wm = (wave >> 1) * 64u, wn = (wave & 1u) * 64u;
  const bool vec_a = (K % 8u) == 0u;
  const bool vec_b = B_NK ? (K % 8u) == 0u : (N % 8u) == 0u;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Register staging of one K slice: A 4 x 16 B per thread; B 4 x 16 B.
  u32x4 ra[4], rb[4];
  auto load_a = [&](uint32_t k0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = i * 256u + tid, r = v >> 3, kv = (v & 7u) * 8u;
      const uint32_t gm = m0 + r, gk = k0 + kv;
      if (vec_a && gm < M && gk + 8u <= K) {
        ra[i] = *reinterpret_cast<const u32x4*>(A + static_cast<uint64_t>(gm) * K + gk);
      } else {
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          h[e] = (gm < M && gk + e < K) ? __builtin_bit_cast(uint16_t, A[static_cast<uint64_t>(gm) * K + gk + e]) : 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) ra[i][e] = h[2 * e] | (static_cast<uint32_t>(h[2 * e + 1]) << 16);
      }
    }
  };
  auto load_b = [&](uint32_t k0) {
    if constexpr (B_NK) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = i * 256u + tid, r = v >> 3, kv = (v & 7u) * 8u;
        const uint32_t gn = n0 + r, gk = k0 + kv;
        if (vec_b && gn < N && gk + 8u <= K) {
          rb[i] = *reinterpret_cast<const u32x4*>(B + static_cast<uint64_t>(gn) * K + gk);
        } else {
          uint16_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            h[e] = (gn < N && gk + e < K) ? __builtin_bit_cast(uint16_t, B[static_cast<uint64_t>(gn) * K + gk + e]) : 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) rb[i][e] = h[2 * e] | (static_cast<uint32_t>(h[2 * e + 1]) << 16);
        }
      }
    } else {
      // [K][N]: thread owns a 4(k) x 8(n) block: rows k0 + kb*4 + i, cols n0 + nb*8.
      const uint32_t nb = tid & 15u, kb = tid >> 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t gk = k0 + kb * 4u + i, gn = n0 + nb * 8u;
        if (vec_b && gk < K && gn + 8u <= N) {
          rb[i] = *reinterpret_cast<const u32x4*>(B + static_cast<uint64_t>(gk) * N + gn);
        } else {
          uint16_t h[8];
#pragma unroll
          for (int e = 0; e < 8; ++e)
            h[e] = (gk < K && gn + e < N) ? __builtin_bit_cast(uint16_t, B[static_cast<uint64_t>(gk) * N + gn + e]) : 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) rb[i][e] = h[2 * e] | (static_cast<uint32_t>(h[2 * e + 1]) << 16);
        }
      }
    }
  };
  auto store_lds = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = i * 256u + tid, r = v >> 3, kv = (v & 7u) * 8u;
      *reinterpret_cast<u32x4*>(&As[r * LDK + kv]) = ra[i];
    }
    if constexpr (B_NK) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = i * 256u + tid, r = v >> 3, kv = (v & 7u) * 8u;
        *reinterpret_cast<u32x4*>(&Bs[r * LDK + kv]) = rb[i];
      }
    } else {
      // Transpose the 4x8 block: column n gets its 4 k values (8 bytes).
      const uint32_t nb = tid & 15u, kb = tid >> 4;
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const int d = n >> 1, sh = (n & 1) * 16;
        const uint32_t k0v = (rb[0][d] >> sh) & 0xffffu, k1v = (rb[1][d] >> sh) & 0xffffu;
        const uint32_t k2v = (rb[2][d] >> sh) & 0xffffu, k3v = (rb[3][d] >> sh) & 0xffffu;
        u32x2 w;
        w[0] = k0v | (k1v << 16);
        w[1] = k2v | (k3v << 16);
        *reinterpret_cast<u32x2*>(&Bs[(nb * 8u + n) * LDK + kb * 4u]) = w;
      }
    }
  };

  const uint32_t nk = (K + BK - 1) / BK;
  load_a(0);
  load_b(0);
  for (uint32_t kt = 0; kt < nk; ++kt) {
    __syncthreads();
    store_lds();
    __syncthreads();
    if (kt + 1 < nk) {
      load_a((kt + 1) * BK);
      load_b((kt + 1) * BK);
    }
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const uint32_t kk = ks * 16u + (lane >> 5) * 8u;
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        fa[i] = *reinterpret_cast<const bf16x8*>(&As[(wm + i * 32u + (lane & 31u)) * LDK + kk]);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        fb[j] = *reinterpret_cast<const bf16x8*>(&Bs[(wn + j * 32u + (lane & 31u)) * LDK + kk]);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  }
  // Epilogue: lanes of one row write 32 consecutive floats.
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

// ---------------------------------------------------------------- fp32 path
// Tile: BM = BN = 128, BK = 32; 4 waves as 2x2, each 64x64 = 2x2 MFMA blocks.
template <bool B_NK, typename Epi>
__device__ __forceinline__ void gemm_f32_128(const float* __restrict__ A, const float* __restrict__ B,
                                             float* __restrict__ C, uint32_t M, uint32_t N, uint32_t K, Epi epi) {
  constexpr int BM = 128, BN = 128, BK = 32;
  constexpr int LDA = BK + 1;                  // As[m][k], odd stride: conflict-free column reads
  constexpr int LDB = B_NK ? BK + 1 : BN + 4;  // Bs[n][k] (NK) or Bs[k][n] (KN)
  __shared__ float As[BM * LDA];
  __shared__ __attribute__((aligned(16))) float Bs[B_NK ? BN * LDB : BK * LDB];
  const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  uint32_t tm, tn;
  gemm_tile_coords(tiles_m, tiles_n, &tm, &tn);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t wm = (wave >> 1) * 64u, wn = (wave & 1u) * 64u;
  const bool vec_a = (K % 4u) == 0u;
  const bool vec_b = B_NK ? (K % 4u) == 0u : (N % 4u) == 0u;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  float4 ra[4], rb[4];
  // Row-major [rows][K] panel, BK columns: 1024 float4 -> 4 per thread.
  auto load_rows = [&](const float* __restrict__ P, uint32_t rows, uint32_t r0, uint32_t k0, bool vec, float4* r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = i * 256u + tid, rr = v >> 3, kv = (v & 7u) * 4u;
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
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = i * 256u + tid, kr = v >> 5, nv = (v & 31u) * 4u;
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
  auto load = [&](uint32_t k0) {
    load_rows(A, M, m0, k0, vec_a, ra);
    if constexpr (B_NK) load_rows(B, N, n0, k0, vec_b, rb);
    else load_b_kn(k0);
  };
  auto store_lds = [&]() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = i * 256u + tid, rr = v >> 3, kv = (v & 7u) * 4u;
      float* p = &As[rr * LDA + kv];
      p[0] = ra[i].x;
      p[1] = ra[i].y;
      p[2] = ra[i].z;
      p[3] = ra[i].w;
    }
    if constexpr (B_NK) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = i * 256u + tid, rr = v >> 3, kv = (v & 7u) * 4u;
        float* p = &Bs[rr * LDB + kv];
        p[0] = rb[i].x;
        p[1] = rb[i].y;
        p[2] = rb[i].z;
        p[3] = rb[i].w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t v = i * 256u + tid, kr = v >> 5, nv = (v & 31u) * 4u;
        *reinterpret_cast<float4*>(&Bs[kr * LDB + nv]) = rb[i];
      }
    }
  };

  const uint32_t nk = (K + BK - 1) / BK;
  load(0);
  for (uint32_t kt = 0; kt < nk; ++kt) {
    __syncthreads();
    store_lds();
    __syncthreads();
    if (kt + 1 < nk) load((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 2; ++ks) {
      const uint32_t k = ks * 2u + (lane >> 5);
      float fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = As[(wm + i * 32u + (lane & 31u)) * LDA + k];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t n = wn + j * 32u + (lane & 31u);
        fb[j] = B_NK ? Bs[n * LDB + k] : Bs[k * LDB + n];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
  }
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

}  // namespace hip
}  // namespace tca

#endif  // TCA_HIP_GEMM_H_
