// Projection kernels: the dense contractions around the attention core.
//
//   forward : [Z | V] = X [W_phi | W_V]  with the soft-hypercube epilogue
//             (reference: packages/morphottention/csrc/cuda/sm120/project.cuh:16-47,
//              attention.cu:105-111; here computed once per token instead of once
//              per (query tile, key tile) pair)
//   backward: dZ = dphi * phi (1 - phi) with
//               dphi = gate_q dq + gate_k dk + gate_q gate_k dcb
//             (reference K side: project.cuh:49-101; the Q side, which the
//              reference drops, by symmetry),
//             dX = [dZ | dV] [W_phi | W_V]^T,  [dW_phi | dW_V] = X^T [dZ | dV],
//             gate gradients as deterministic fp32 column sums.
#include <climits>

#include "common.h"
#include "gemm.h"
#include "internal.h"

namespace morpho {

// ---------------------------------------------------------------- weights^T
// wt = [W_phi | W_V]^T (rows in the projection's column order) for the
// forward projection and wcat = [W_phi | W_V]
// (one row-major matrix) for dX. 64 x 64 tiles with 16-byte loads and
// stores: each thread reads two 8-column pieces of W rows (and writes them to
// wcat), and writes two 8-row pieces of wt rows gathered from the LDS tile.
// HM and D are multiples of 8, so no piece straddles W_phi / W_V or a matrix
// edge.
__global__ __launch_bounds__(256) void transpose_weights_kernel(const f16* __restrict__ W_phi,
                                                                const f16* __restrict__ W_V, f16* __restrict__ wt,
                                                                f16* __restrict__ wcat, Dims dm) {
  __shared__ __align__(16) f16 tile[64][72];  // [d][n]
  const int D = dm.D, HM = dm.HM;
  const int n0 = blockIdx.x * 64, d0 = blockIdx.y * 64, NC = HM + D;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int v = threadIdx.x + 256 * i;
    const int dd = v >> 3, nn = (v & 7) * 8;
    const int dg = d0 + dd, ng = n0 + nn;
    f16x8 x = {};
    if (dg < D && ng < NC) {
      x = ng < HM ? *reinterpret_cast<const f16x8*>(W_phi + (int64_t)dg * HM + ng)
                  : *reinterpret_cast<const f16x8*>(W_V + (int64_t)dg * D + (ng - HM));
      *reinterpret_cast<f16x8*>(wcat + (int64_t)dg * NC + ng) = x;
    }
    *reinterpret_cast<f16x8*>(&tile[dd][nn]) = x;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int v = threadIdx.x + 256 * i;
    const int nn = v >> 3, dd = (v & 7) * 8;
    const int dg = d0 + dd, ng = n0 + nn;
    if (dg < D && ng < NC) {
      f16x8 y;
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = tile[dd + e][nn];
      *reinterpret_cast<f16x8*>(wt + (int64_t)proj_row(dm, ng) * D + dg) = y;
    }
  }
}

hipError_t launch_transpose_weights(const Dims& d, const f16* W_phi, const f16* W_V, f16* wt, f16* wcat,
                                    hipStream_t s) {
  dim3 grid((d.HM + d.D + 63) / 64, (d.D + 63) / 64);
  MORPHO_KLAUNCH(transpose_weights_kernel, grid, dim3(256), 0, s, W_phi, W_V, wt, wcat, d);
  return hipGetLastError();
}

// ---------------------------------------------------------------- projection forward
// [Z | V] = X [W_phi | W_V] on BM x BN tiles: 256 x 320 when 320 divides the
// H*M + D columns (e.g. 1280 at B4 N4096 D1024 H16 m16, which makes the grid
// exactly one round of 256 tiles), 256 x 256 otherwise, and 128 x 128 when
// the large tiles would leave most CUs idle (few tokens: B8 N1024 D512 H8 m16
// has 64 large tiles, 320 small ones). The epilogue takes the tile through
// LDS in 64-row slabs (a slab holds the accumulators of the wave rows whose
// rows it covers), fp32 with row stride BN + 5 = 5 (mod 64) banks: the value
// pass below reads 8 rows x 8 columns per wave instruction on 64 distinct
// banks, and the accumulator stores (16 columns x 4 row groups) are at most
// 2-way.
template <int BM, int BN>
using ProjGemm = Gemm<BM, BN, 4, true, true, 64, 2>;

// e4m3 byte(s) of V_lo * 2^kVloExp, clamped to the format's range (e4m3 has
// no infinity: an overflowing conversion gives NaN) and rounded toward zero:
// the stored remainder is never larger than V - V_hi, so V_hi + remainder
// rounds back to V_hi in fp16 (a single key's output is then exactly V_hi,
// the value the backward's dP = dO V_hi^T sees).
// The conversion with stochastic rounding adds the given random bits below
// the last kept mantissa bit and truncates; with zero random bits it is the
// truncation of the magnitude, i.e. rounding toward zero, in one instruction
// (bit-identical, over every 7th float bit pattern of both signs, to the
// nearest conversion stepped one code toward zero where that overshot).
__device__ __forceinline__ float vlo_scaled(float r) { return fminf(fmaxf(r * (float)(1 << kVloExp), -448.f), 448.f); }
__device__ __forceinline__ unsigned vlo_code(float r) {
  return (unsigned)__builtin_amdgcn_cvt_sr_fp8_f32(vlo_scaled(r), 0, 0, 0) & 0xffu;
}
__device__ __forceinline__ uint2 vlo_pack8(const float (&r)[8]) {
  int w[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {  // byte k of the dword = r[4 i + k]
    w[i] = __builtin_amdgcn_cvt_sr_fp8_f32(vlo_scaled(r[4 * i]), 0, 0, 0);
    w[i] = __builtin_amdgcn_cvt_sr_fp8_f32(vlo_scaled(r[4 * i + 1]), 0, w[i], 1);
    w[i] = __builtin_amdgcn_cvt_sr_fp8_f32(vlo_scaled(r[4 * i + 2]), 0, w[i], 2);
    w[i] = __builtin_amdgcn_cvt_sr_fp8_f32(vlo_scaled(r[4 * i + 3]), 0, w[i], 3);
  }
  return make_uint2((unsigned)w[0], (unsigned)w[1]);
}

// GEN: a cube projection other than the sigmoid, or the masked diagonal (the
// variants take the projection from d.proj and the exact row maximum)
template <int M, int DV, int BM, int BN, bool GEN>
__global__ __launch_bounds__(kGemmThreads) void proj_fwd_kernel(const f16* __restrict__ X,
                                                               const f16* __restrict__ gate_q,
                                                               const f16* __restrict__ gate_k, Dims d, ProjBuffers p) {
  using G = ProjGemm<BM, BN>;
  constexpr int SS = BN + 5;  // stage row stride (floats)
  // epilogue LDS: the 64-row slab, then the tile's gate products G = gq gk
  static_assert(64 * SS * 4 + BN * 4 <= G::kLdsBytes, "epilogue slab and gate table must fit the main loop's LDS");
  __shared__ __align__(16) char smem[G::kLdsBytes];
  constexpr int CW = 2 * M + 8;

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / G::WN, wn = w % G::WN;
  const int NC = d.HM + d.D;
  const int T = (int)d.T;
  int tm, tn;
  if (!gemm_tile_map(blockIdx.x, (T + BM - 1) / BM, (NC + BN - 1) / BN, tm, tn)) return;
  const int n0 = tn * BN, m0 = tm * BM;
  f32x4 acc[G::FI][G::FJ];
  G::run(X, d.D, p.wt, d.D, T, NC, m0, n0, 0, d.D, smem, acc);

  float* stage = reinterpret_cast<float*>(smem);
  float* gtab = stage + 64 * SS;
  const float c1 = 2.0f * d.scale * kLog2e;
  static_assert(G::WTM == 64 || G::WTM == 32, "wave rows of 64 or 32 rows");
  // Code columns of this tile: local columns [0, ncode), whole heads (PCPT per
  // tile in the interleaved order; in the natural order those below HM).
  const int ncode = d.PCPT > 0 ? d.PCPT : max(0, min(BN, d.HM - n0));
  // Gate products of the code columns, read from global memory once per tile
  // rather than in every slab (the first slab's barrier publishes them).
  for (int lc = tid; lc < ncode; lc += kGemmThreads) {
    const int col = proj_col(d, tn, lc);  // = h M + c, the gates' index
    gtab[lc] = (float)gate_q[col] * (float)gate_k[col];
  }
  for (int slab = 0; slab < BM / 64; ++slab) {
    if (slab > 0) __syncthreads();  // the previous slab has been consumed
    if (G::WTM * wm / 64 == slab) {  // uniform: this wave row's rows are in the slab
      const int r0 = G::WTM * wm % 64;
#pragma unroll
      for (int i = 0; i < G::FI; ++i)
#pragma unroll
        for (int j = 0; j < G::FJ; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            stage[(r0 + 16 * i + 4 * (lane >> 4) + r) * SS + G::WTN * wn + 16 * j + (lane & 15)] = acc[i][j][r];
    }
    __syncthreads();
    const int row0 = m0 + 64 * slab;
    // soft-hypercube codes: one (token, head, 8-code chunk) per thread; the
    // M / 8 chunks of a (token, head) sit on consecutive lanes, which meet in
    // xor shuffles for the row sums (a head's M columns are contiguous in
    // both column orders). One thread per (token, head) had left 3/4 of the
    // workgroup idle at m = 64.
    constexpr int kChunks = M / 8;
    static_assert(kGemmThreads % kChunks == 0, "a (token, head) never straddles two passes");
    for (int idx = tid; idx < 8 * ncode; idx += kGemmThreads) {  // 64 rows x (ncode / M heads) x (M / 8 chunks)
      const int j = idx % kChunks, item = idx / kChunks;
      const int hh = item / 64, r = item % 64;
      const int col0 = proj_col(d, tn, hh * M);
      const int t = row0 + r;
      const bool active = t < T;  // the same for every chunk of the item
      const int h = col0 / M;
      const int b = t / d.N, n = t - b * d.N;
      const int64_t bhn = (int64_t)(b * d.H + h) * d.N + n;
      const int c8 = 8 * j;
      float sumb = 0.f, tii = 0.f, U = 0.f;
      if (active) {
        const float* z = stage + r * SS + hh * M + c8;
        const float4 ga = *reinterpret_cast<const float4*>(gtab + hh * M + c8);
        const float4 gb = *reinterpret_cast<const float4*>(gtab + hh * M + c8 + 4);
        const float g8[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
        f16x8 phh, phl, kch, kcl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float phi = GEN ? cube_project(z[e], d.proj) : sigmoidf_(z[e]);
          const float G = g8[e];
          const float wgt = d.scale * G;
          const float cg = c1 * G;
          f16 a, bb;
          if (GEN) {  // HardTanh01's clamped fma could convert to fp16 in one rounding
            split_exact(phi, a, bb);
            phh[e] = a;
            phl[e] = bb;
          } else {  // a quotient: nothing to fuse the conversion with
            phh[e] = (f16)phi;
            phl[e] = (f16)(phi - (float)phh[e]);
          }
          // kc = cg phi: lo is the exact product minus hi, so hi + lo carries
          // kc to ~2^-22 however hi was rounded, provided lo and the stored
          // hi are one value. The conversion (f16)(cg phi) may otherwise be
          // selected twice, as one rounding of the exact product
          // (v_fma_mixlo_f16) for the fma and as a rounding of the fp32
          // product (v_cvt_pk_f16_f32) for the store, and at an fp16 rounding
          // tie the two differ by an ulp (about 1 code in 16k); the opaque
          // copy makes hi a single value.
          f16 hi = (f16)(cg * phi);
          asm("" : "+v"(hi));
          kch[e] = hi;
          kcl[e] = (f16)__builtin_fmaf(cg, phi, -(float)hi);
          sumb += wgt * phi;
          tii += wgt * phi * (2.f * phi - 1.f);
          U += fmaxf(0.f, wgt * (2.f * phi - 1.f));
        }
        // rows: [phi_hi | aug | phi_lo] and [kc_hi | aug | kc_lo]
        f16* qrow = p.qa + bhn * CW;
        f16* krow = p.ka + bhn * CW;
        *reinterpret_cast<f16x8*>(qrow + c8) = phh;
        *reinterpret_cast<f16x8*>(qrow + M + 8 + c8) = phl;
        *reinterpret_cast<f16x8*>(krow + c8) = kch;
        *reinterpret_cast<f16x8*>(krow + M + 8 + c8) = kcl;
      }
#pragma unroll
      for (int sh = 1; sh < kChunks; sh <<= 1) {  // the item's lanes are all active or all idle
        sumb += __shfl_xor(sumb, sh);
        tii += __shfl_xor(tii, sh);
        U += __shfl_xor(U, sh);
      }
      if (!active || j != 0) continue;
      // base-2 quantities: token bias b = -log2e * sum_c w_c phi_c; self score
      // t_ii and the upper bound U of any score in this query's row (without
      // the row constant, which cancels in the softmax). U bounds the row only
      // for phi in [0, 1], and R >= U - 15 keeps the row's largest weight
      // representable only while the diagonal term is in the row: the
      // identity projection and the masked diagonal take the exact two-pass
      // maximum (an infinite gap).
      const float bias = -kLog2e * sumb;
      const float t_ii = kLog2e * tii;
      const float Ub = kLog2e * U;
      const float R = fmaxf(t_ii, Ub - 15.f);
      const float gap = (GEN && (d.proj == kProjIdentity || d.mask_diag)) ? kFltMax : Ub - t_ii;
      f16 rh, rl, bh_, bl_;
      split_hi_lo(-R, rh, rl);
      split_hi_lo(bias, bh_, bl_);
      const f16 one = (f16)1.f, zero = (f16)0.f;
      *reinterpret_cast<f16x8*>(p.qa + bhn * CW + M) = f16x8{one, one, rh, rl, zero, zero, zero, zero};
      *reinterpret_cast<f16x8*>(p.ka + bhn * CW + M) = f16x8{bh_, bl_, one, one, zero, zero, zero, zero};
      p.tstat[bhn] = make_float4(bias, R, gap, t_ii);
    }
    // values, transposed: vt[bh][dd][n] = V_hi, and the remainder V - V_hi as
    // e4m3 in vlo's tile-major, key-permuted rows. One item = one column x 8
    // consecutive tokens; 8 neighbouring threads cover the slab's 64
    // consecutive tokens of a column (128 contiguous bytes of vt, one 64-byte
    // row of vlo), a wave 8 columns.
    // A thread keeps its group of 8 tokens (tid % 8) and steps over the
    // tile's value columns [ncode, BN).
    const int rg = tid & 7, tb = row0 + 8 * rg;
    if (ncode < BN && tb < T) {
      const bool vec = d.N % 8 == 0;
      const int ntile = d.NP / 64;
      const int tbb = tb / d.N, tbn = tb - tbb * d.N;  // batch row and position of token tb
      for (int cc = ncode + (tid >> 3); cc < BN; cc += kGemmThreads / 8) {
        if (n0 + cc >= NC) break;  // columns past NC only at the end of the tile
        const int col = proj_col(d, tn, cc);
        const int vcol = col - d.HM, h = vcol / DV, dd = vcol % DV;
        const float* src = stage + 8 * rg * SS + cc;
        if (vec) {
          // N % 8 == 0 and tb % 8 == 0: the 8 tokens share one batch row and
          // land on 8 consecutive bytes of a vlo row
          const int b = tbb, n = tbn;
          const int64_t bh = (int64_t)(b * d.H + h);
          f16x8 vh;
          float vl[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = src[e * SS];  // a value read from LDS: one evaluation for V_hi and the remainder
            vh[e] = (f16)x;
            vl[e] = x - (float)vh[e];
          }
          f16* dst = p.vt + (bh * DV + dd) * d.NP + n;
          uint8_t* lrow = p.vlo + ((bh * ntile + n / 64) * DV + dd) * 64;
          *reinterpret_cast<f16x8*>(dst) = vh;
          *reinterpret_cast<uint2*>(lrow + vlo_pos(n % 64)) = vlo_pack8(vl);
          if (n + 8 == d.N)
            for (int z = 8; n + z < d.NP; z += 8) {
              *reinterpret_cast<f16x8*>(dst + z) = f16x8{};
              *reinterpret_cast<uint2*>(lrow + vlo_pos((n + z) % 64)) = make_uint2(0u, 0u);
            }
        } else {
          for (int e = 0; e < 8 && tb + e < T; ++e) {
            const int t = tb + e, b = t / d.N, n = t - b * d.N;
            const int64_t bh = (int64_t)(b * d.H + h);
            const float x = src[e * SS];
            const f16 vh = (f16)x;
            f16* dst = p.vt + (bh * DV + dd) * d.NP + n;
            uint8_t* lrow = p.vlo + ((bh * ntile + n / 64) * DV + dd) * 64;
            dst[0] = vh;
            lrow[vlo_pos(n % 64)] = (uint8_t)vlo_code(x - (float)vh);
            if (n == d.N - 1)
              for (int z = 1; n + z < d.NP; ++z) {
                dst[z] = (f16)0.f;
                lrow[vlo_pos((n + z) % 64)] = 0;
              }
          }
        }
      }
    }
  }
}

template <int M, int DV>
static hipError_t launch_proj_fwd_t(const Dims& d, const f16* X, const f16* gq, const f16* gk, const ProjBuffers& p,
                                    hipStream_t s) {
  const int NC = d.HM + d.D;
  const bool gen = d.proj != kProjSigmoid || d.mask_diag;
#define MORPHO_PROJ_LAUNCH(BM_, BN_)                                                                       \
  do {                                                                                                     \
    const dim3 g(gemm_tile_grid((int)((d.T + BM_ - 1) / BM_), (NC + BN_ - 1) / BN_));                      \
    if (gen)                                                                                               \
      MORPHO_KLAUNCH((proj_fwd_kernel<M, DV, BM_, BN_, true>), g, dim3(kGemmThreads), 0, s, X, gq, gk, d, p);  \
    else                                                                                                   \
      MORPHO_KLAUNCH((proj_fwd_kernel<M, DV, BM_, BN_, false>), g, dim3(kGemmThreads), 0, s, X, gq, gk, d, p); \
  } while (0)
  if (d.PBN == 320)
    MORPHO_PROJ_LAUNCH(256, 320);
  else if (d.PBN == 160)
    MORPHO_PROJ_LAUNCH(128, 160);
  else if (d.PBN == 128)
    MORPHO_PROJ_LAUNCH(128, 128);
  else
    MORPHO_PROJ_LAUNCH(256, 256);
#undef MORPHO_PROJ_LAUNCH
  return hipGetLastError();
}

hipError_t launch_proj_fwd(const Dims& d, const f16* X, const f16* gq, const f16* gk, const ProjBuffers& p,
                           hipStream_t s) {
#define MORPHO_PROJ_CASE(MM, VV) \
  if (d.M == MM && d.DV == VV) return launch_proj_fwd_t<MM, VV>(d, X, gq, gk, p, s);
  MORPHO_PROJ_CASE(16, 32) MORPHO_PROJ_CASE(16, 64) MORPHO_PROJ_CASE(16, 128)
  MORPHO_PROJ_CASE(32, 32) MORPHO_PROJ_CASE(32, 64) MORPHO_PROJ_CASE(32, 128)
  MORPHO_PROJ_CASE(64, 32) MORPHO_PROJ_CASE(64, 64) MORPHO_PROJ_CASE(64, 128)
#undef MORPHO_PROJ_CASE
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------- backward elementwise
// The output depends on the gates only through G = gate_q * gate_k, and with
// dq = sum_j dS_ij phi_j, dk = sum_i dS_ij phi_i, dcb = sum_i dS_ij, r =
// sum_j dS_ij (natural-log score gradients, ungated codes):
//   dL/dphi_tc = scale G_c (2 (dq_tc + dk_tc) - dcb_t - r_t)
//   dL/dG_c    = scale sum_t phi_tc (2 dk_tc - dcb_t)
// (the gate sum uses sum_j dS_ij = 0). dL/dG is taken from the key-side sums
// only, whose terms share the same rounded dS, so its cancellation stays
// exact; then d gate_q = dL/dG gate_k and d gate_k = dL/dG gate_q.
//
// Diagonal correction (softmax attention, diagonal key present). The row sum
// r_t of the rounded dS is 0 in exact arithmetic; what the kernels measure is
// the error of the row's delta: an offset nu in delta makes dS_tj wrong by
// -nu P_tj, so r_t = -nu sum_j P_tj. Where the row is concentrated on its
// diagonal (saturated codes: the other weights are tiny and so is the true
// gradient) that offset, however small (fp32 rounding of dO . O suffices),
// dominates the code gradients. Replacing dS_tt by dS_tt - r_t P_tt cancels
// it: dq, dk and dcb of token t lose c = r_t P_tt times the diagonal's
// operands (phi_hi of t, the codes both products used, and 1), and the row
// sum becomes r_t - c. P_tt = 2^(s_tt - lse_t) (s_tt = t_tt + b_t from the
// projection's statistics) comes from bwd_prep, next to r_t.
// A block of kElemThreads threads covers kGateTokensPerBlock tokens and 256
// projection columns. Each thread owns 8 consecutive columns (one head) and
// every kElemSubs-th token of the block, so all loads and stores are 16-byte
// vectors: a wave covers 32 column groups of 2 tokens, i.e. whole 512-byte dZ
// rows and, per head, 2 consecutive rows of dq / dk. The per-thread gate sums
// meet in LDS in a fixed order. (1024 threads: with a few thousand blocks in
// all, 256-thread blocks left one wave per SIMD to cover the memory latency.)
constexpr int kElemThreads = 1024, kElemSubs = kElemThreads / 32;
static_assert(kGateTokensPerBlock % kElemSubs == 0, "whole tokens per thread");
__global__ __launch_bounds__(kElemThreads) void proj_bwd_elem_kernel(const f16* __restrict__ gate_q,
                                                                     const f16* __restrict__ gate_k, Dims d,
                                                                     ProjBuffers p, BwdBuffers g, int row_corr) {
  __shared__ float red[kElemSubs][257];
  const int c8 = threadIdx.x & 31, sub = threadIdx.x >> 5;
  const int col = blockIdx.y * 256 + 8 * c8;  // first of this thread's 8 columns
  const bool active = col < d.HM;
  const int h = col / d.M, c = col - h * d.M;
  const int NC = d.HM + d.D;
  float sg[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (active) {
    float sG[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sG[e] = d.scale * (float)gate_q[col + e] * (float)gate_k[col + e];
    const int64_t t0 = (int64_t)blockIdx.x * kGateTokensPerBlock;
#pragma unroll
    for (int k = 0; k < kGateTokensPerBlock / kElemSubs; ++k) {
      const int64_t t = t0 + sub + kElemSubs * k;
      if (t >= d.T) break;
      const int b = (int)(t / d.N), n = (int)(t - (int64_t)b * d.N);
      const int64_t bhn = (int64_t)(b * d.H + h) * d.N + n;
      const f16* qrow = p.qa + bhn * d.CW;
      const f16x8 ph = *reinterpret_cast<const f16x8*>(qrow + c);
      const f16x8 pl = *reinterpret_cast<const f16x8*>(qrow + d.M + 8 + c);
      const float4* dqp = reinterpret_cast<const float4*>(g.dq + bhn * d.M + c);
      const float4* dkp = reinterpret_cast<const float4*>(g.dk + bhn * d.M + c);
      const float4 q0 = dqp[0], q1 = dqp[1], k0 = dkp[0], k1 = dkp[1];
      const float dq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
      const float dk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      float dcb = g.dcb[bhn], rs = 0.f, cr = 0.f;
      if (row_corr) {  // uniform
        const float2 rp = reinterpret_cast<const float2*>(g.dr)[bhn];  // {r, P_tt}
        cr = rp.x * rp.y;
        rs = rp.x - cr;
        dcb -= cr;
      }
      f16x8 dz;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float phi = (float)ph[e] + (float)pl[e];
        const float cp = cr * (float)ph[e];
        const float dqe = dq[e] - cp, dke = dk[e] - cp;
        const float dphi = sG[e] * (2.f * (dqe + dke) - dcb - rs);
        dz[e] = (f16)(dphi * cube_project_grad(phi, d.proj));
        sg[e] += phi * (2.f * dke - dcb);
      }
      *reinterpret_cast<f16x8*>(g.dzv + t * NC + col) = dz;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) red[sub][8 * c8 + e] = sg[e];
  __syncthreads();
  const int cc = blockIdx.y * 256 + threadIdx.x;
  if (threadIdx.x < 256 && cc < d.HM) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kElemSubs; ++i) s += red[i][threadIdx.x];
    g.gpart[(int64_t)blockIdx.x * d.HM + cc] = s;
  }
}

hipError_t launch_proj_bwd_elem(const Dims& d, const f16* gq, const f16* gk, const ProjBuffers& p,
                                const BwdBuffers& g, bool row_corr, hipStream_t s) {
  dim3 grid((unsigned)((d.T + kGateTokensPerBlock - 1) / kGateTokensPerBlock), (d.HM + 255) / 256);
  MORPHO_KLAUNCH(proj_bwd_elem_kernel, grid, dim3(kElemThreads), 0, s, gq, gk, d, p, g, row_corr ? 1 : 0);
  return hipGetLastError();
}

// ---------------------------------------------------------------- backward GEMMs
// One launch computes
//   dX = [dZ | dV] [W_phi | W_V]^T                    (dX tiles)
//   [dW_phi | dW_V] = X^T [dZ | dV]                   (dW tiles, split over tokens)
// in one round of workgroups (BwdGemmPlan): ids [0, n_a) compute g whole dX
// tiles each, ids n_a + p t + j piece j of dW tile t (a near-equal 1/p of the
// tokens) and store its fp32 partial, which dw_reduce adds in piece order.
// g and p give both kinds about the same number of k-steps. (Before, every
// dW split of T / 8 tokens and every dX tile was a workgroup of its own; at
// B4 N4096 D1024 H16 m16 a CU then ran a 32-k-step dW split or 20-k-step dX
// tiles, and the launch took about 52 k-steps per CU for 40 of work: dX alone
// 40.6 us, dW alone 53.4 us, both in one launch 90.1 us.)
// Square BT x BT tiles for both products: 256, or 128 when the plan with
// 128 tiles finishes sooner (few tokens). Either way the waves own 64-row wave
// tiles, which the dX epilogue's slabs rely on.
template <int BT>
struct BwdTiles {
  static constexpr int WM = BT == 256 ? 4 : 2;
  using Dx = Gemm<BT, BT, WM, true, true, 64, 2>;    // A = dZ|dV [T][NC], B = wcat = [W_phi | W_V] [D][NC]
  using Dw = Gemm<BT, BT, WM, false, false, 64, 2>;  // A = X (k-major) [T][D], B = dZ|dV (k-major) [T][NC]
  static constexpr int kLds = Dx::kLdsBytes > Dw::kLdsBytes ? Dx::kLdsBytes : Dw::kLdsBytes;
  static constexpr int kStageStride = BT + 8;  // halves: one 64-row slab of fp16 dX for 16-byte stores
  static_assert(64 * kStageStride * 2 <= kLds, "dX slab must fit the main loop's LDS");
  static_assert(Dx::WN == Dw::WN && Dx::WTM == 64 && Dw::WTM == 64, "shared wave grid, 64-row wave tiles");
  static_assert(Dx::kBK == 64 && Dw::kBK == 64, "the plan counts k-steps of 64");
};

// Plan for tile edge bt and `slots` workgroups (the dW pieces take
// 8 ceil(tiles_w p / 8) of them): for each g (dX tiles per type-A
// workgroup), the most pieces p per dW tile that still fit the round,
// scored by the longer of the two kinds: g kx against ceil(kw / p) k-steps
// (plus one step of epilogue per dX tile or piece). When the dW tiles alone
// fill the round, every workgroup takes one tile over several rounds. A type-A workgroup's dX
// tiles come from the row panels tr = 8 i + xcd, as before, so a panel of
// dZ|dV is read into one L2.
static BwdGemmPlan plan_for(const Dims& d, int bt, int slots, int64_t& cost) {
  BwdGemmPlan P;
  const int NC = d.HM + d.D, T = (int)d.T;
  P.bt = bt;
  const int ntm_x = (T + bt - 1) / bt;
  P.ntn_x = (d.D + bt - 1) / bt;
  P.n_dx = ntm_x * P.ntn_x;
  P.kx = (NC + 63) / 64;
  P.ntn_w = (NC + bt - 1) / bt;
  P.tiles_w = ((d.D + bt - 1) / bt) * P.ntn_w;
  P.kw = (T + 63) / 64;
  const int per_xcd = ((ntm_x + 7) / 8) * P.ntn_x;  // dX tiles of one XCD
  cost = INT64_MAX;
  P.g = per_xcd;
  P.n_a = 8;
  P.p = 1;
  for (int g = 1; g <= per_xcd; ++g) {
    const int n_a = 8 * ((per_xcd + g - 1) / g);
    int p = (slots - n_a) / P.tiles_w;
    while (p > 0 && n_a + 8 * ((P.tiles_w * p + 7) / 8) > slots) --p;  // whole runs of 8
    if (p < 1) continue;
    p = p < P.kw ? p : P.kw;
    const int64_t ca = (int64_t)g * (P.kx + 1), cb = (P.kw + p - 1) / p + 1;
    const int64_t cst = ca > cb ? ca : cb;
    if (cst < cost) {
      cost = cst;
      P.g = g;
      P.n_a = n_a;
      P.p = p;
    }
    if (ca > cost) break;  // g kx only grows from here
  }
  if (cost == INT64_MAX) {
    // dW tiles alone fill the round: one dX tile or one whole dW tile per
    // workgroup over several rounds (the dispatcher balances them)
    P.g = 1;
    P.n_a = 8 * per_xcd;
    P.p = 1;
    cost = ((int64_t)P.n_dx * (P.kx + 1) + (int64_t)P.tiles_w * (P.kw + 1) + slots - 1) / slots;
  }
  return P;
}

BwdGemmPlan bwd_gemm_plan(const Dims& d) {
  int64_t c256, c128;
  const BwdGemmPlan p256 = plan_for(d, 256, kGemmSlots, c256);
  if (d.D % 128 != 0 || (d.HM + d.D) % 128 != 0) return p256;
  // 128 x 128 tiles: two workgroups per CU (64 KiB of LDS each), so twice the
  // slots; a k-step does a quarter of the work of a 256 x 256 one at about 2/3
  // of its rate (more LDS and L2 traffic per MFMA), and shares its CU
  const BwdGemmPlan p128 = plan_for(d, 128, 2 * kGemmSlots, c128);
  return 3 * c128 < 4 * c256 ? p128 : p256;
}

struct BwdGemmArgs {
  const f16* X;
  const f16* wcat;
  f16* dX;
  BwdGemmPlan plan;
};

template <int BT>
__global__ __launch_bounds__(kGemmThreads) void bwd_gemm_kernel(Dims d, BwdBuffers g, BwdGemmArgs a) {
  using DxGemm = typename BwdTiles<BT>::Dx;
  using DwGemm = typename BwdTiles<BT>::Dw;
  constexpr int kDxStageStride = BwdTiles<BT>::kStageStride;
  __shared__ __align__(16) char smem[BwdTiles<BT>::kLds];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / DxGemm::WN, wn = w % DxGemm::WN;  // same wave grid for dX and dW
  const BwdGemmPlan& P = a.plan;
  const int NC = d.HM + d.D;
  const int T = (int)d.T;
  const int id = blockIdx.x;

  if (id < P.n_a) {
    // ---- g dX tiles: local tiles s g .. s g + g - 1 of XCD xcd, i.e. row
    // panel tr = 8 (L / ntn_x) + xcd, column tile L % ntn_x
    const int xcd = id & 7, slot = id >> 3;
    const int ntm = (T + BT - 1) / BT;
    for (int q = 0; q < P.g; ++q) {
      const int L = slot * P.g + q;
      const int tm = 8 * (L / P.ntn_x) + xcd, tn = L % P.ntn_x;
      if (tm >= ntm) break;  // uniform
      if (q > 0) __syncthreads();  // the previous tile's slab reads are done before the stages refill
      const int m0 = tm * BT, n0 = tn * BT;
      f32x4 acc[DxGemm::FI][DxGemm::FJ];
      DxGemm::run(g.dzv, NC, a.wcat, NC, T, d.D, m0, n0, 0, NC, smem, acc);
      // fp16 through LDS in 64-row slabs (slab = wave row), then 16-byte row stores
      f16* st = reinterpret_cast<f16*>(smem);
      for (int slab = 0; slab < BT / 64; ++slab) {
        if (slab > 0) __syncthreads();
        if (wm == slab) {
#pragma unroll
          for (int i = 0; i < DxGemm::FI; ++i)
#pragma unroll
            for (int j = 0; j < DxGemm::FJ; ++j)
#pragma unroll
              for (int r = 0; r < 4; ++r)
                st[(16 * i + 4 * (lane >> 4) + r) * kDxStageStride + DxGemm::WTN * wn + 16 * j + (lane & 15)] =
                    (f16)acc[i][j][r];
        }
        __syncthreads();
        for (int qq = tid; qq < 64 * (BT / 8); qq += kGemmThreads) {
          const int r = qq / (BT / 8), c = 8 * (qq % (BT / 8));
          const int row = m0 + 64 * slab + r, col = n0 + c;
          if (row < T && col < d.D)
            *reinterpret_cast<f16x8*>(a.dX + (int64_t)row * d.D + col) =
                *reinterpret_cast<const f16x8*>(st + r * kDxStageStride + c);
        }
      }
    }
    return;
  }

  // ---- dW: piece j of tile tl. The pieces, taken piece by piece (q = j
  // tiles_w + tl), are dealt to the XCDs in contiguous runs (XCD x = id % 8
  // takes q = x per_x + slot), so an XCD's workgroups share one or two token
  // ranges of X and dZ|dV in its L2.
  const int b = id - P.n_a, per_x = (P.tiles_w * P.p + 7) / 8;
  const int q = (b & 7) * per_x + (b >> 3);
  if ((b >> 3) >= per_x || q >= P.tiles_w * P.p) return;
  const int j = q / P.tiles_w, tl = q - j * P.tiles_w;
  const int ks = dw_piece_k0(P.kw, P.p, j), ke = dw_piece_k0(P.kw, P.p, j + 1);
  const int m0 = (tl / P.ntn_w) * BT, n0 = (tl % P.ntn_w) * BT;
  f32x4 acc[DwGemm::FI][DwGemm::FJ];
  DwGemm::run(a.X, d.D, g.dzv, NC, d.D, NC, m0, n0, 64 * ks, min(64 * ke, T), smem, acc);
  // the piece's partial, tile-local row-major [BT][BT], at tl p + j
  float* part = g.wpart + (int64_t)(tl * P.p + j) * BT * BT;
#pragma unroll
  for (int i = 0; i < DwGemm::FI; ++i)
#pragma unroll
    for (int jj = 0; jj < DwGemm::FJ; ++jj) {
      const int col = DwGemm::WTN * wn + 16 * jj + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) part[(DwGemm::WTM * wm + 16 * i + 4 * (lane >> 4) + r) * BT + col] = acc[i][jj][r];
    }
}

hipError_t launch_bwd_gemm(const Dims& d, const ProjBuffers& p, const BwdBuffers& g, const f16* X, f16* dX,
                           hipStream_t s) {
  BwdGemmArgs a;
  a.X = X; a.wcat = p.wcat; a.dX = dX;
  a.plan = bwd_gemm_plan(d);
  const dim3 grid((unsigned)(a.plan.n_a + 8 * ((a.plan.tiles_w * a.plan.p + 7) / 8)));
  if (a.plan.bt == 128)
    MORPHO_KLAUNCH(bwd_gemm_kernel<128>, grid, dim3(kGemmThreads), 0, s, d, g, a);
  else
    MORPHO_KLAUNCH(bwd_gemm_kernel<256>, grid, dim3(kGemmThreads), 0, s, d, g, a);
  return hipGetLastError();
}

// Finalisation of the weight and gate gradients, one launch. Blocks
// [0, nw) sum the dW pieces' partials of [dW_phi | dW_V] (4 consecutive
// outputs per thread; the pieces of the output's tile in order); blocks
// [nw, nw + ceil(HM / 16)) sum the per-block gate partials: 16 columns x 16
// row groups per block, group g summing rows g, g + 16, ... with two
// accumulators, the groups then combined in a fixed order. Both orders are
// fixed, so results are deterministic.
__global__ __launch_bounds__(256) void dw_reduce_kernel(const float* __restrict__ wpart, int bt, int ntn_w, int pieces,
                                                        int D, int HM, f16* __restrict__ dW_phi,
                                                        f16* __restrict__ dW_V, int nw,
                                                        const float* __restrict__ gpart, int nblk, float scale,
                                                        const f16* __restrict__ gate_q, const f16* __restrict__ gate_k,
                                                        f16* __restrict__ d_gate_q, f16* __restrict__ d_gate_k) {
  __shared__ float part[16][17];
  if ((int)blockIdx.x >= nw) {
    const int cl = threadIdx.x & 15, grp = threadIdx.x >> 4;
    const int col = ((int)blockIdx.x - nw) * 16 + cl;
    float s0 = 0.f, s1 = 0.f;
    if (col < HM) {
      int i = grp;
#pragma unroll 4
      for (; i + 16 < nblk; i += 32) {  // unrolled: several loads in flight, same order
        s0 += gpart[(int64_t)i * HM + col];
        s1 += gpart[(int64_t)(i + 16) * HM + col];
      }
      if (i < nblk) s0 += gpart[(int64_t)i * HM + col];
    }
    part[grp][cl] = s0 + s1;
    __syncthreads();
    if (grp == 0 && col < HM) {
      float t = 0.f;
#pragma unroll
      for (int g2 = 0; g2 < 16; ++g2) t += part[g2][cl];
      const float dG = scale * t;
      d_gate_q[col] = (f16)(dG * (float)gate_k[col]);
      d_gate_k[col] = (f16)(dG * (float)gate_q[col]);
    }
    return;
  }
  const int NC = HM + D;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (idx >= (int64_t)D * NC) return;
  const int row = (int)(idx / NC), col = (int)(idx - (int64_t)row * NC);
  const int tl = (row / bt) * ntn_w + col / bt;
  // 4 columns never straddle a tile; piece z of the tile at partial tl pieces + z
  const int64_t tsz = (int64_t)bt * bt;
  const float* src = wpart + (int64_t)tl * pieces * tsz + (int64_t)(row % bt) * bt + col % bt;
  // pieces summed in order; the loads of 8 are issued before their adds
  float4 s = *reinterpret_cast<const float4*>(src);
  int z = 1;
  for (; z + 8 <= pieces; z += 8) {
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const float4*>(src + (z + i) * tsz);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s.x += v[i].x; s.y += v[i].y; s.z += v[i].z; s.w += v[i].w;
    }
  }
  for (; z < pieces; ++z) {
    const float4 v = *reinterpret_cast<const float4*>(src + z * tsz);
    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
  }
  // 4 consecutive columns never straddle HM (HM and NC are multiples of 16)
  f16* dst = col < HM ? dW_phi + (int64_t)row * HM + col : dW_V + (int64_t)row * D + (col - HM);
  *reinterpret_cast<f16x4*>(dst) = f16x4{(f16)s.x, (f16)s.y, (f16)s.z, (f16)s.w};
}

hipError_t launch_dw_reduce(const Dims& d, const BwdBuffers& g, const f16* gq, const f16* gk, f16* dW_phi, f16* dW_V,
                            f16* dgq, f16* dgk, hipStream_t s) {
  const int64_t total = (int64_t)d.D * (d.HM + d.D);
  const int nw = (int)((total / 4 + 255) / 256);
  const int ngate = (d.HM + 15) / 16;
  const int nblk = (int)((d.T + kGateTokensPerBlock - 1) / kGateTokensPerBlock);
  const BwdGemmPlan P = bwd_gemm_plan(d);
  MORPHO_KLAUNCH(dw_reduce_kernel, dim3((unsigned)(nw + ngate)), dim3(256), 0, s, g.wpart, P.bt, P.ntn_w, P.p, d.D,
                 d.HM, dW_phi, dW_V, nw, g.gpart, nblk, d.scale, gq, gk, dgq, dgk);
  return hipGetLastError();
}

}  // namespace morpho
