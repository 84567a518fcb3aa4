// Block-tiled fp16 MFMA GEMM main loop (fp32 accumulation) for gfx950.
//
// C[m][n] = sum_k A(m, k) * B(k, n) over one 128 x 128 output tile per
// 256-thread workgroup (4 waves, each 64 x 64 = 2 x 2 blocks of 32x32x16
// MFMAs), k stepped by 64 through double-buffered LDS with the global loads of
// the next two k-steps in flight during the current one.
//
// Operands are described by OperandDesc. "k-contiguous" operands are staged in
// LDS row = m (or n), and read with one 16-byte load per fragment; "k-major"
// operands (k is the row index in memory, e.g. X read as X^T) are staged as
// they lie in memory and read with ds_read_b64_tr_b16, so no transposing
// stores are needed.
#pragma once

#include "common.h"

namespace morpho {

struct OperandDesc {
  const f16* p;   // segment 0
  int64_t ld;     // leading dimension of segment 0 (elements)
  const f16* p2;  // segment 1 (k >= kseg), k-contiguous operands only
  int64_t ld2;
  int kseg;       // first k of segment 1 (multiple of 8); INT_MAX if none
};

constexpr int kGemmBM = 128, kGemmBN = 128, kGemmBK = 64, kGemmThreads = 256;

template <bool KCONTIG, int ROWS>
struct GemmOperandTile {
  // LDS row stride (halves): 36 dwords for b128 fragment reads (8 rows -> 8
  // distinct bank groups), 16 (mod 64) halves for transposed reads.
  static constexpr int kStride = KCONTIG ? (kGemmBK + 8) : (ROWS + 16);
  static constexpr int kElems = KCONTIG ? ROWS * kStride : kGemmBK * kStride;  // one buffer
  static constexpr int kVecs = ROWS * kGemmBK / 8;                           // 16-byte vectors per tile
  static constexpr int kRegs = kVecs / kGemmThreads;
  static constexpr int kRowVecs = KCONTIG ? kGemmBK / 8 : ROWS / 8;           // vectors per LDS row

  f16x8 reg[kRegs];

  // Global -> registers for the tile at (row0, k0); rows >= nrows or k >= kend
  // read as zero. nrows and kend are multiples of 8 for the contiguous axis.
  __device__ __forceinline__ void load(const OperandDesc& d, int row0, int nrows, int k0, int kend, int tid) {
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      const int v = tid + kGemmThreads * i;
      const int lr = v / kRowVecs, lc = (v % kRowVecs) * 8;  // LDS row, column
      f16x8 x = {};
      if (KCONTIG) {
        const int gr = row0 + lr, gk = k0 + lc;
        if (gr < nrows && gk < kend) {
          const f16* src = gk < d.kseg ? d.p + (int64_t)gr * d.ld + gk : d.p2 + (int64_t)gr * d.ld2 + (gk - d.kseg);
          x = *reinterpret_cast<const f16x8*>(src);
        }
      } else {
        const int gk = k0 + lr, gr = row0 + lc;
        if (gk < kend && gr < nrows) x = *reinterpret_cast<const f16x8*>(d.p + (int64_t)gk * d.ld + gr);
      }
      reg[i] = x;
    }
  }

  __device__ __forceinline__ void store(f16* s, int tid) const {
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      const int v = tid + kGemmThreads * i;
      const int lr = v / kRowVecs, lc = (v % kRowVecs) * 8;
      *reinterpret_cast<f16x8*>(s + lr * kStride + lc) = reg[i];
    }
  }

  // Fragment for the 32-row block starting at `row0` (tile-local), k chunk c.
  __device__ __forceinline__ static f16x8 frag(const f16* s, int row0, int c, int lane) {
    if (KCONTIG) return frag_kcontig(s, kStride, row0 + (lane & 31), 16 * c, lane);
    return frag_kmajor(s, kStride, 16 * c, row0, lane);
  }
};

template <bool AKC, bool BKC>
struct GemmMainloop {
  using TA = GemmOperandTile<AKC, kGemmBM>;
  using TB = GemmOperandTile<BKC, kGemmBN>;
  static constexpr int kLdsHalves = 2 * (TA::kElems + TB::kElems);

  // acc[i][j] holds C rows m0 + 64*wm + 32*i + acc_row(r), cols n0 + 64*wn + 32*j + lane%32
  __device__ __forceinline__ static void compute(const f16* sa, const f16* sb, int wm, int wn, int lane,
                                                 f32x16 acc[2][2]) {
#pragma unroll
    for (int c = 0; c < kGemmBK / 16; ++c) {
      f16x8 a0 = TA::frag(sa, 64 * wm, c, lane);
      f16x8 a1 = TA::frag(sa, 64 * wm + 32, c, lane);
      f16x8 b0 = TB::frag(sb, 64 * wn, c, lane);
      f16x8 b1 = TB::frag(sb, 64 * wn + 32, c, lane);
      acc[0][0] = mfma16(a0, b0, acc[0][0]);
      acc[0][1] = mfma16(a0, b1, acc[0][1]);
      acc[1][0] = mfma16(a1, b0, acc[1][0]);
      acc[1][1] = mfma16(a1, b1, acc[1][1]);
    }
  }

  // Two register stages: while k-step kt is computed from LDS, the loads of
  // k-steps kt+1 and kt+2 are in flight. The loop is unrolled by two so the
  // stages never change registers while their loads are outstanding.
  __device__ __forceinline__ static void run(const OperandDesc& A, const OperandDesc& B, int M, int N, int m0, int n0,
                                             int kbeg, int kend, f16* lds, f32x16 acc[2][2]) {
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w >> 1, wn = w & 1;
    f16* sA[2] = {lds, lds + TA::kElems};
    f16* sB[2] = {lds + 2 * TA::kElems, lds + 2 * TA::kElems + TB::kElems};
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};
    const int nk = (kend - kbeg + kGemmBK - 1) / kGemmBK;
    if (nk <= 0) return;
    TA ta0, ta1;
    TB tb0, tb1;
    auto kof = [&](int kt) { return kbeg + kt * kGemmBK; };
    ta0.load(A, m0, M, kof(0), kend, tid);
    tb0.load(B, n0, N, kof(0), kend, tid);
    ta0.store(sA[0], tid);
    tb0.store(sB[0], tid);
    if (nk > 1) {
      ta1.load(A, m0, M, kof(1), kend, tid);
      tb1.load(B, n0, N, kof(1), kend, tid);
    }
    if (nk > 2) {
      ta0.load(A, m0, M, kof(2), kend, tid);
      tb0.load(B, n0, N, kof(2), kend, tid);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; kt += 2) {
      // even step: LDS buffer 0 holds kt; stage 1 holds kt+1; stage 0 holds kt+2
      compute(sA[0], sB[0], wm, wn, lane, acc);
      if (kt + 1 < nk) {
        ta1.store(sA[1], tid);
        tb1.store(sB[1], tid);
      }
      __syncthreads();
      if (kt + 3 < nk) {
        ta1.load(A, m0, M, kof(kt + 3), kend, tid);
        tb1.load(B, n0, N, kof(kt + 3), kend, tid);
      }
      if (kt + 1 >= nk) break;
      // odd step: LDS buffer 1 holds kt+1; stage 0 holds kt+2; stage 1 holds kt+3
      compute(sA[1], sB[1], wm, wn, lane, acc);
      if (kt + 2 < nk) {
        ta0.store(sA[0], tid);
        tb0.store(sB[0], tid);
      }
      __syncthreads();
      if (kt + 4 < nk) {
        ta0.load(A, m0, M, kof(kt + 4), kend, tid);
        tb0.load(B, n0, N, kof(kt + 4), kend, tid);
      }
    }
  }
};

// Tile order for L2 reuse: workgroups are dispatched round-robin over the 8
// XCDs (id % 8). Give all `ncols` column tiles of one row panel ids that are
// congruent mod 8, so the panel is fetched into one XCD's L2. Returns false for
// padding ids; the grid must have 8 * ceil(nrows / 8) * ncols workgroups.
__device__ __forceinline__ bool gemm_tile_map(int nrows, int ncols, int& tr, int& tc) {
  const int i = blockIdx.x, xcd = i & 7, slot = i >> 3;
  tr = 8 * (slot / ncols) + xcd;
  tc = slot % ncols;
  return tr < nrows;
}
__host__ inline unsigned gemm_tile_grid(int nrows, int ncols) {
  return 8u * (unsigned)((nrows + 7) / 8) * (unsigned)ncols;
}

}  // namespace morpho
