// Block-tiled fp16 MFMA GEMM main loop (fp32 accumulation) for gfx950.
//
// C[m][n] = sum_k A(m, k) B(k, n) over one BM x BN output tile per workgroup
// of 8 waves (512 threads, two per SIMD) in a WM x WN arrangement, each wave
// owning a (BM / WM) x (BN / WN) block of 16x16 accumulators
// (v_mfma_f32_16x16x32_f16). k advances by 64 through two LDS stages that the
// waves fill by DMA (global_load_lds_dwordx4, 1 KiB per wave instruction):
// the stage of k-step t + 1 is issued right after the barrier that opens
// k-step t and lands while t is computed, so no VGPRs hold prefetched data.
//
// Why 16x16x32: sustained over the whole chip, v_mfma_f32_16x16x32_f16 runs
// at 2.24 PFLOP/s and v_mfma_f32_32x32x16_f16 at 1.82 PFLOP/s (independent
// chains from registers, 45 ms runs); the same main loop with the former is
// 5-7 % faster (B4 N4096 D1024 projection and dX shapes, 8192^3).
//
// Why these shapes: a 256 x 256 (or 256 x 320) tile moves 64 (72) KiB from L2
// per 8.4 (10.5) MFLOP. With 256 x 128 tiles the L2 -> CU traffic at the
// MFMA rate (~25 TB/s for the whole chip) was the bound; here it is ~15 TB/s.
//
// Operand kinds:
//  * k-contiguous ("KC", element (row, k) at p[row * ld + k]): LDS rows of
//    64 halves (128 bytes), the 16-byte chunk c of row r stored at chunk
//    position c ^ ((r >> 1) & 7). A fragment is one ds_read_b128 per lane and
//    the 16 lanes of a read phase hit 16 distinct 4-bank groups.
//  * k-major ("KM", element (k, row) at p[k * ld + row], e.g. X read as X^T):
//    LDS rows k of ROWS halves (ROWS a power of two >= 128), chunk c of row k
//    stored at c ^ ((k & 3) << 2) ^ (((k >> 3) & 1) << 1). Fragments come from
//    ds_read_b64_tr_b16 (the transposing read); the 32 lanes of a phase cover
//    rows {k..k+3, k+8..k+11} x 32 bytes on 64 distinct banks.
// Rows past the operand's extent load clamped (finite) data that only feeds
// discarded outputs; k past kend is zeroed in LDS on the last k-step.
#pragma once

#include "common.h"

namespace morpho {

constexpr int kGemmWaves = 8;
constexpr int kGemmThreads = 64 * kGemmWaves;

template <bool KC, int ROWS, int BK>
struct OpTile {
  static_assert(BK == 32 || BK == 64, "k-step of 32 or 64");
  static constexpr int kBytes = ROWS * BK * 2;
  static constexpr int kDma = kBytes / 1024;            // 1 KiB DMA pieces per tile
  static constexpr int kRowChunks = KC ? BK / 8 : ROWS / 8;  // 16-byte chunks per LDS row
  // KC chunk swizzle: with 8 chunks per row (BK = 64) rows r and r + 1 share a
  // swizzle and 16 rows span 8 values; with 4 (BK = 32) rows r .. r + 3 share.
  __device__ __forceinline__ static int kc_swz(int r) { return BK == 64 ? (r >> 1) & 7 : (r >> 2) & 3; }
  __device__ __forceinline__ static int km_swz(int k) { return ((k & 3) << 2) ^ (((k >> 3) & 1) << 1); }
  static_assert(KC || (ROWS >= 128 && (ROWS & (ROWS - 1)) == 0), "KM swizzle needs 2^n >= 16 chunks per row");

  // Tile row and k of LDS chunk q = 64 piece + lane.
  __device__ __forceinline__ static void chunk(int q, int& r, int& k8) {
    if (KC) {
      r = q / kRowChunks;
      k8 = 8 * ((q % kRowChunks) ^ kc_swz(r));  // first k of the chunk
    } else {
      k8 = q / kRowChunks;                        // the chunk's k
      r = 8 * ((q % kRowChunks) ^ km_swz(k8));    // first row of the chunk
    }
  }

  // Byte offset of the chunk from the tile's base (operand at row0, k0), with
  // rows clamped into [0, rmax): rows past the extent re-read a valid row and
  // only feed discarded outputs. Fits 32 bits for ld <= 65536.
  __device__ __forceinline__ static unsigned lane_off(int64_t ld, int rmax, int piece, int lane) {
    int r, k8;
    chunk(64 * piece + lane, r, k8);
    if (KC) return (unsigned)(((int64_t)min(r, rmax - 1) * ld + k8) * 2);
    return (unsigned)(((int64_t)k8 * ld + min(r, rmax - 8)) * 2);
  }
  __device__ __forceinline__ static const char* tile_base(const f16* p, int64_t ld, int row0, int k0) {
    return reinterpret_cast<const char*>(KC ? p + (int64_t)row0 * ld + k0 : p + (int64_t)k0 * ld + row0);
  }
  // Full address with k clamped into [k0, kend) as well (the ragged last
  // k-step). KC needs kend % 8 == 0; KM needs nrows % 8 == 0.
  __device__ __forceinline__ static const f16* tail_src(const f16* p, int64_t ld, int row0, int nrows, int k0,
                                                        int kend, int piece, int lane) {
    int r, k8;
    chunk(64 * piece + lane, r, k8);
    if (KC) return p + (int64_t)min(row0 + r, nrows - 1) * ld + min(k0 + k8, kend - 8);
    return p + (int64_t)min(k0 + k8, kend - 1) * ld + min(row0 + r, nrows - 8);
  }

  // Zero the k >= kvalid part of a stage tile (kvalid < BK; last k-step only).
  __device__ __forceinline__ static void zero_tail(char* s, int kvalid, int tid) {
    for (int q = tid; q < kBytes / 16; q += kGemmThreads) {
      int r, k8;
      chunk(q, r, k8);
      if (k8 >= kvalid) *reinterpret_cast<f16x8*>(s + 16 * q) = f16x8{};
    }
  }

  // MFMA 16x16x32 operand for the 16-row block at tile row (or column) mn0,
  // k chunk kq (k = 32 kq .. 32 kq + 31): lane l supplies row mn0 + l % 16,
  // k = 32 kq + 8 (l / 16) + j.
  __device__ __forceinline__ static f16x8 frag(const char* s, int mn0, int kq, int lane) {
    if (KC) {
      const int row = mn0 + (lane & 15);  // mn0 % 16 == 0, so kc_swz(row) == kc_swz(lane & 15)
      const int c = (4 * kq + (lane >> 4)) ^ kc_swz(lane & 15);
      return *reinterpret_cast<const f16x8*>(s + row * (BK * 2) + 16 * c);
    } else {
      const int k = 32 * kq + 8 * (lane >> 4) + ((lane & 15) >> 2);
      const int col = mn0 + 4 * (lane & 3);
      auto at = [&](int kk) { return s + kk * (ROWS * 2) + 16 * ((col >> 3) ^ km_swz(kk)) + 2 * (col & 7); };
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
      const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(at(k)));
      const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(at(k + 4)));
      return __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
  }
};

template <int BM, int BN, int WM, bool AKC, bool BKC, int BK = 32, int STAGES = 4>
struct Gemm {
  static constexpr int kBK = BK;
  static constexpr int WN = kGemmWaves / WM;
  using TA = OpTile<AKC, BM, BK>;
  using TB = OpTile<BKC, BN, BK>;
  static constexpr int kStages = STAGES;
  static constexpr int kStageBytes = TA::kBytes + TB::kBytes;
  static constexpr int kLdsBytes = kStages * kStageBytes;
  static constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  static constexpr int FI = WTM / 16, FJ = WTN / 16;  // 16x16 accumulator blocks
  // DMA pieces of a stage, A's first; wave w issues pieces w, w + 8, ...
  // A's piece count is a multiple of 8, so whether a wave's i-th piece is A or
  // B is known at compile time; the first kP % 8 waves issue one piece more.
  static constexpr int kP = TA::kDma + TB::kDma;
  static constexpr int kPA = TA::kDma / kGemmWaves;      // A pieces per wave
  static constexpr int kPBmax = (TB::kDma + kGemmWaves - 1) / kGemmWaves;
  static constexpr int kNhi = (kP + kGemmWaves - 1) / kGemmWaves, kNlo = kP / kGemmWaves;
  static_assert(TA::kDma % kGemmWaves == 0, "A pieces must split evenly over the waves");
  static_assert(WTM % 16 == 0 && WTN % 16 == 0 && BK % 32 == 0, "wave tile of whole 16x16 blocks, k-step of whole 32s");
  static_assert((STAGES - 2) * kNhi < 64, "vmcnt range");

  // wait until this wave's pieces of the stage issued `ahead` stages before
  // the latest one have landed (the later `ahead` stages may be in flight)
  template <int AHEAD>
  __device__ __forceinline__ static void wait_stage(int w) {
    if (w < kP % kGemmWaves)
      wait_vmcnt_lgkm0<AHEAD * kNhi>();
    else
      wait_vmcnt_lgkm0<AHEAD * kNlo>();
  }

  // Wave w owns rows WTM * (w / WN) .. and columns WTN * (w % WN) .. of the
  // tile; acc[i][j][r] holds C row m0 + WTM * (w / WN) + 16 i + 4 (lane / 16) + r,
  // column n0 + WTN * (w % WN) + 16 j + lane % 16.
  // Operands: A (M rows) and B (N rows = columns of C), each one matrix
  // (p, ld); k runs over [kbeg, kend). lds: kLdsBytes, 16-byte aligned.
  __device__ __forceinline__ static void run(const f16* Ap, int64_t lda, const f16* Bp, int64_t ldb, int M, int N,
                                             int m0, int n0, int kbeg, int kend, char* lds, f32x4 (&acc)[FI][FJ]) {
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w / WN, wn = w % WN;
#pragma unroll
    for (int i = 0; i < FI; ++i)
#pragma unroll
      for (int j = 0; j < FJ; ++j) acc[i][j] = f32x4{};
    const int nk = (kend - kbeg + kBK - 1) / kBK;
    if (nk <= 0) return;
    const unsigned sbase = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)lds;

    // this wave's pieces: A pieces w + 8 i, B pieces w + 8 i (< TB::kDma)
    unsigned offA[kPA], offB[kPBmax];
#pragma unroll
    for (int i = 0; i < kPA; ++i) offA[i] = TA::lane_off(lda, M - m0, w + kGemmWaves * i, lane);
#pragma unroll
    for (int i = 0; i < kPBmax; ++i)
      offB[i] = TB::lane_off(ldb, N - n0, min(w + kGemmWaves * i, TB::kDma - 1), lane);
    const int64_t stepA = AKC ? 2 * kBK : 2 * kBK * lda, stepB = BKC ? 2 * kBK : 2 * kBK * ldb;  // bytes per k-step
    const char* baseA = TA::tile_base(Ap, lda, m0, kbeg);
    const char* baseB = TB::tile_base(Bp, ldb, n0, kbeg);

    auto issue = [&](int t) {
      const unsigned st = sbase + (unsigned)((t % kStages) * kStageBytes);
      const int k0 = kbeg + t * kBK;
      if (k0 + kBK <= kend) {  // uniform
#pragma unroll
        for (int i = 0; i < kPA; ++i)
          lds_dma16_so(baseA + t * stepA, offA[i], st + 1024u * (unsigned)(w + kGemmWaves * i));
#pragma unroll
        for (int i = 0; i < kPBmax; ++i)
          if (w + kGemmWaves * i < TB::kDma)  // uniform
            lds_dma16_so(baseB + t * stepB, offB[i],
                         st + (unsigned)TA::kBytes + 1024u * (unsigned)(w + kGemmWaves * i));
      } else {
#pragma unroll
        for (int i = 0; i < kPA; ++i)
          lds_dma16(TA::tail_src(Ap, lda, m0, M, k0, kend, w + kGemmWaves * i, lane),
                    st + 1024u * (unsigned)(w + kGemmWaves * i));
#pragma unroll
        for (int i = 0; i < kPBmax; ++i)
          if (w + kGemmWaves * i < TB::kDma)
            lds_dma16(TB::tail_src(Bp, ldb, n0, N, k0, kend, w + kGemmWaves * i, lane),
                      st + (unsigned)TA::kBytes + 1024u * (unsigned)(w + kGemmWaves * i));
      }
    };

    // stages t .. t + STAGES - 2 are in flight when k-step t opens
#pragma unroll
    for (int t = 0; t < STAGES - 1; ++t)
      if (t < nk) issue(t);
    for (int t = 0; t < nk; ++t) {
      // this wave's pieces of stage t have landed (later stages may not have)
      if (t + STAGES - 2 < nk)
        wait_stage<STAGES - 2>(w);
      else
        wait_vmcnt_lgkm0<0>();
      asm volatile("s_barrier" ::: "memory");  // ... and every wave's; stage t - 1 is free
      char* sa = lds + (t % kStages) * kStageBytes;
      char* sb = sa + TA::kBytes;
      const int kvalid = kend - (kbeg + t * kBK);
      if (kvalid < kBK) {  // uniform: last k-step of a ragged K
        TA::zero_tail(sa, kvalid, tid);
        TB::zero_tail(sb, kvalid, tid);
        wait_vmcnt_lgkm0<0>();
        asm volatile("s_barrier" ::: "memory");
      }
      if (t + STAGES - 1 < nk) issue(t + STAGES - 1);
#pragma unroll
      for (int kq = 0; kq < kBK / 32; ++kq) {
        f16x8 a[FI], b[FJ];
#pragma unroll
        for (int i = 0; i < FI; ++i) a[i] = TA::frag(sa, WTM * wm + 16 * i, kq, lane);
#pragma unroll
        for (int j = 0; j < FJ; ++j) b[j] = TB::frag(sb, WTN * wn + 16 * j, kq, lane);
#pragma unroll
        for (int i = 0; i < FI; ++i)
#pragma unroll
          for (int j = 0; j < FJ; ++j) acc[i][j] = mfma16x16(a[i], b[j], acc[i][j]);
      }
    }
    // every wave is done with the stages before the caller reuses the LDS
    wait_vmcnt_lgkm0<0>();
    asm volatile("s_barrier" ::: "memory");
  }
};

// Tile order for L2 reuse: workgroups are dispatched round-robin over the 8
// XCDs (id % 8). Give all `ncols` column tiles of one row panel ids that are
// congruent mod 8, so the panel is fetched into one XCD's L2. Returns false for
// padding ids; the grid must have 8 * ceil(nrows / 8) * ncols workgroups.
__device__ __forceinline__ bool gemm_tile_map(int id, int nrows, int ncols, int& tr, int& tc) {
  const int xcd = id & 7, slot = id >> 3;
  tr = 8 * (slot / ncols) + xcd;
  tc = slot % ncols;
  return tr < nrows;
}
__host__ inline unsigned gemm_tile_grid(int nrows, int ncols) {
  return 8u * (unsigned)((nrows + 7) / 8) * (unsigned)ncols;
}

}  // namespace morpho
