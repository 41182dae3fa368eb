// fp32 MFMA tile machinery for gfx950 (v_mfma_f32_16x16x4_f32, wave64).
//
// Workgroup tile BM x BN = 128 x 128, K staged through LDS BK = 32 at a time,
// double-buffered.  Four waves in a 2 x 2 arrangement each own a 64 x 64 block
// of C held as 4 x 4 MFMA tiles of 16 x 16 (64 accumulator VGPRs per lane).
//
// MFMA 16x16x4 operand layout (one block): lane l supplies A[l % 16][l / 16]
// and B[l / 16][l % 16]; the result lane l holds D[4 * (l / 16) + r][l % 16],
// r = 0..3.  Within a 16-wide K slice, lane group q = l / 16 feeds k = 4q + j
// to MFMA step j (j = 0..3), so a k-contiguous LDS row is read with one
// ds_read_b128 per 16 x 16 sub-tile and four MFMA steps.  A and B use the same
// k permutation, so the contraction is unchanged.
//
// LDS layouts (row strides padded by 4 floats so the 16-lane groups of a wave
// hit disjoint banks):
//   A "k-contiguous"  [BM][BK+4]  (A stored M x K)      -> ds_read_b128
//   A "m-contiguous"  [BK][BM+4]  (A stored K x M)      -> 4 x ds_read_b32
//   B "k-contiguous"  [BN][BK+4]  (B stored N x K)      -> ds_read_b128
//   B "n-contiguous"  [BK][BN+4]  (B stored K x N)      -> 4 x ds_read_b32
#pragma once
#include "common.hpp"

namespace gemm {

constexpr int BK = 32, NT = 256, PAD = 4;
constexpr int LDK = BK + PAD;   // row stride of k-contiguous tiles
// Default workgroup tile (and the one the convolution kernels use).
constexpr int BM = 128, BN = 128;
constexpr int LDMN = BM + PAD;  // row stride of m/n-contiguous 128-wide tiles

// A_MC: A tile is m-contiguous; B_KC: B tile is k-contiguous.  TM / TN: tile
// extent along M / N (128 or 64); KD: K depth of a stage (32 or 16).
template <bool A_MC, int TM = BM, int KD = BK>
constexpr int a_tile_floats() {
  return A_MC ? KD * (TM + PAD) : TM * (KD + PAD);
}
template <bool B_KC, int TN = BN, int KD = BK>
constexpr int b_tile_floats() {
  return B_KC ? TN * (KD + PAD) : KD * (TN + PAD);
}

// One BK-deep slice of MFMAs for this wave's (16*WM) x (16*WN) block; the
// workgroup's four waves sit 2 x 2, so the tile is (32*WM) x (32*WN).  All
// fragment reads of the slice are issued first and a scheduling barrier keeps
// the compiler from sinking them between the MFMAs: otherwise m/n-contiguous
// tiles (four ds_read_b32 per fragment) end up with an LDS wait before every
// few MFMAs.  The hardware waits only for the reads of the current 16-deep step.
template <bool A_MC, bool B_KC, int WM = 4, int WN = 4, int KD = BK>
__device__ __forceinline__ void mma_stage(const float* __restrict__ As, const float* __restrict__ Bs,
                                          f32x4 (&acc)[WM][WN], int wm, int wn, int lr, int q) {
  constexpr int KB = KD / 16;
  constexpr int LDA = 32 * WM + PAD, LDB = 32 * WN + PAD, LDKK = KD + PAD;
  f32x4 a[KB][WM], b[KB][WN];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int row = wm * 16 * WM + i * 16 + lr;
      if (!A_MC) {
        a[kb][i] = *reinterpret_cast<const f32x4*>(As + row * LDKK + kb * 16 + 4 * q);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) a[kb][i][j] = As[(kb * 16 + 4 * q + j) * LDA + row];
      }
    }
#pragma unroll
    for (int i = 0; i < WN; ++i) {
      const int col = wn * 16 * WN + i * 16 + lr;
      if (B_KC) {
        b[kb][i] = *reinterpret_cast<const f32x4*>(Bs + col * LDKK + kb * 16 + 4 * q);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) b[kb][i][j] = Bs[(kb * 16 + 4 * q + j) * LDB + col];
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int n = 0; n < WN; ++n)
          acc[i][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[kb][i][j], b[kb][n][j], acc[i][n], 0, 0, 0);
}

// Row/column of accumulator element (i, n, r) of this lane inside the tile.
template <int WM = 4>
__device__ __forceinline__ int acc_row(int wm, int i, int q, int r) {
  return wm * 16 * WM + i * 16 + 4 * q + r;
}
template <int WN = 4>
__device__ __forceinline__ int acc_col(int wn, int n, int lr) {
  return wn * 16 * WN + n * 16 + lr;
}

}  // namespace gemm
