// Block-tiled fp16 MFMA GEMM main loop (fp32 accumulation) for gfx950.
//
// C[m][n] = sum_k A(m, k) * B(k, n) over one 128 x 128 output tile per
// 256-thread workgroup (4 waves, each 64 x 64 = 2 x 2 blocks of 32x32x16
// MFMAs), k stepped by 32 through double-buffered LDS.
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

constexpr int kGemmBM = 128, kGemmBN = 128, kGemmBK = 32, kGemmThreads = 256;

template <bool KCONTIG, int ROWS>
struct GemmOperandTile {
  // LDS footprint (halves) of one buffer of this operand
  // LDS row stride (halves): 20 dwords for b128 fragment reads (8 rows -> 8
  // distinct bank groups), 16 (mod 64) halves for transposed reads.
  static constexpr int kStride = KCONTIG ? (kGemmBK + 8) : (ROWS + 16);
  static constexpr int kElems = KCONTIG ? ROWS * kStride : kGemmBK * kStride;

  f16x8 reg[2];

  // Global -> registers for the tile at (row0, k0); rows >= nrows or k >= kend
  // read as zero. nrows and kend are multiples of 8 for the contiguous axis.
  __device__ __forceinline__ void load(const OperandDesc& d, int row0, int nrows, int k0, int kend, int tid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int v = tid + kGemmThreads * i;
      f16x8 x = {};
      if (KCONTIG) {
        const int row = v >> 2, kv = (v & 3) * 8;
        const int gr = row0 + row, gk = k0 + kv;
        if (gr < nrows && gk < kend) {
          const f16* src = gk < d.kseg ? d.p + (int64_t)gr * d.ld + gk : d.p2 + (int64_t)gr * d.ld2 + (gk - d.kseg);
          x = *reinterpret_cast<const f16x8*>(src);
        }
      } else {
        const int krow = v / (ROWS / 8), cv = (v % (ROWS / 8)) * 8;
        const int gk = k0 + krow, gr = row0 + cv;
        if (krow < kGemmBK && gk < kend && gr < nrows) x = *reinterpret_cast<const f16x8*>(d.p + (int64_t)gk * d.ld + gr);
      }
      reg[i] = x;
    }
  }

  __device__ __forceinline__ void store(f16* s, int tid) const {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int v = tid + kGemmThreads * i;
      if (KCONTIG) {
        const int row = v >> 2, kv = (v & 3) * 8;
        *reinterpret_cast<f16x8*>(s + row * kStride + kv) = reg[i];
      } else {
        const int krow = v / (ROWS / 8), cv = (v % (ROWS / 8)) * 8;
        if (krow < kGemmBK) *reinterpret_cast<f16x8*>(s + krow * kStride + cv) = reg[i];
      }
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
    TA ta;
    TB tb;
    ta.load(A, m0, M, kbeg, kend, tid);
    tb.load(B, n0, N, kbeg, kend, tid);
    ta.store(sA[0], tid);
    tb.store(sB[0], tid);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      const bool more = kt + 1 < nk;
      if (more) {
        ta.load(A, m0, M, kbeg + (kt + 1) * kGemmBK, kend, tid);
        tb.load(B, n0, N, kbeg + (kt + 1) * kGemmBK, kend, tid);
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        f16x8 a0 = TA::frag(sA[buf], 64 * wm, c, lane);
        f16x8 a1 = TA::frag(sA[buf], 64 * wm + 32, c, lane);
        f16x8 b0 = TB::frag(sB[buf], 64 * wn, c, lane);
        f16x8 b1 = TB::frag(sB[buf], 64 * wn + 32, c, lane);
        acc[0][0] = mfma16(a0, b0, acc[0][0]);
        acc[0][1] = mfma16(a0, b1, acc[0][1]);
        acc[1][0] = mfma16(a1, b0, acc[1][0]);
        acc[1][1] = mfma16(a1, b1, acc[1][1]);
      }
      if (more) {
        ta.store(sA[buf ^ 1], tid);
        tb.store(sB[buf ^ 1], tid);
      }
      __syncthreads();
    }
  }
};

}  // namespace morpho
