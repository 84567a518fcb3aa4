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
__global__ __launch_bounds__(256) void transpose_weights_kernel(const f16* __restrict__ W_phi,
                                                                const f16* __restrict__ W_V, f16* __restrict__ wt,
                                                                int D, int HM) {
  __shared__ f16 tile[64][66];
  const int n0 = blockIdx.x * 64, d0 = blockIdx.y * 64, NC = HM + D;
  for (int idx = threadIdx.x; idx < 64 * 64; idx += 256) {
    const int dd = idx >> 6, nn = idx & 63;
    const int dg = d0 + dd, ng = n0 + nn;
    f16 x = (f16)0.f;
    if (dg < D && ng < NC) x = ng < HM ? W_phi[(int64_t)dg * HM + ng] : W_V[(int64_t)dg * D + (ng - HM)];
    tile[dd][nn] = x;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 64 * 64; idx += 256) {
    const int nn = idx >> 6, dd = idx & 63;
    const int dg = d0 + dd, ng = n0 + nn;
    if (dg < D && ng < NC) wt[(int64_t)ng * D + dg] = tile[dd][nn];
  }
}

hipError_t launch_transpose_weights(const Dims& d, const f16* W_phi, const f16* W_V, f16* wt, hipStream_t s) {
  dim3 grid((d.HM + d.D + 63) / 64, (d.D + 63) / 64);
  hipLaunchKernelGGL(transpose_weights_kernel, grid, dim3(256), 0, s, W_phi, W_V, wt, d.D, d.HM);
  return hipGetLastError();
}

// ---------------------------------------------------------------- projection forward
constexpr int kStageStride = 132;  // fp32 epilogue stage row stride

template <int M, int DV>
__global__ __launch_bounds__(256) void proj_fwd_kernel(const f16* __restrict__ X, const f16* __restrict__ gate_q,
                                                       const f16* __restrict__ gate_k, Dims d, ProjBuffers p) {
  using ML = GemmMainloop<true, true>;
  constexpr int kMainBytes = ML::kLdsHalves * 2;
  constexpr int kStageBytes = 64 * kStageStride * 4;
  __shared__ __align__(16) unsigned char smem[kMainBytes > kStageBytes ? kMainBytes : kStageBytes];
  constexpr int CW = 3 * M + 8;

  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;
  const int NC = d.HM + d.D;
  const int T = (int)d.T;
  int tm, tn;
  if (!gemm_tile_map((T + kGemmBM - 1) / kGemmBM, (NC + kGemmBN - 1) / kGemmBN, tm, tn)) return;
  const int n0 = tn * kGemmBN, m0 = tm * kGemmBM;
  OperandDesc A{X, d.D, nullptr, 0, INT_MAX};
  OperandDesc B{p.wt, d.D, nullptr, 0, INT_MAX};
  f32x16 acc[2][2];
  ML::run(A, B, T, NC, m0, n0, 0, d.D, reinterpret_cast<f16*>(smem), acc);

  float* stage = reinterpret_cast<float*>(smem);
  const float c1 = 2.0f * d.scale * kLog2e;
  for (int pass = 0; pass < 2; ++pass) {
    __syncthreads();
    if (wm == pass) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            stage[(32 * i + acc_row(r, lane)) * kStageStride + 64 * wn + 32 * j + (lane & 31)] = acc[i][j][r];
    }
    __syncthreads();
    const int row0 = m0 + 64 * pass;
    // soft-hypercube codes: one (token, head) per item
    constexpr int kHeadsPerTile = kGemmBN / M;
    for (int idx = tid; idx < 64 * kHeadsPerTile; idx += 256) {
      const int hh = idx / 64, r = idx % 64;
      const int col0 = n0 + hh * M;
      const int t = row0 + r;
      if (col0 >= d.HM || t >= T) continue;
      const int h = col0 / M;
      const int b = t / d.N, n = t - b * d.N;
      const int64_t bhn = (int64_t)(b * d.H + h) * d.N + n;
      const float* z = stage + r * kStageStride + hh * M;
      f16* qrow = p.qa + bhn * CW;
      f16* krow = p.ka + bhn * CW;
      float sumb = 0.f, tii = 0.f, U = 0.f;
#pragma unroll
      for (int c8 = 0; c8 < M; c8 += 8) {
        f16x8 phh, phl, kch, kcl;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int c = c8 + e;
          const float phi = sigmoidf_(z[c]);
          const float G = (float)gate_q[h * M + c] * (float)gate_k[h * M + c];
          const float wgt = d.scale * G;
          const float kc = c1 * G * phi;
          phh[e] = (f16)phi;
          phl[e] = (f16)(phi - (float)phh[e]);
          kch[e] = (f16)kc;
          kcl[e] = (f16)(kc - (float)kch[e]);
          sumb += wgt * phi;
          tii += wgt * phi * (2.f * phi - 1.f);
          U += fmaxf(0.f, wgt * (2.f * phi - 1.f));
        }
        // rows: [phi_hi | aug | phi_lo | phi_hi] and [kc_hi | aug | kc_hi | kc_lo]
        *reinterpret_cast<f16x8*>(qrow + c8) = phh;
        *reinterpret_cast<f16x8*>(qrow + M + 8 + c8) = phl;
        *reinterpret_cast<f16x8*>(qrow + 2 * M + 8 + c8) = phh;
        *reinterpret_cast<f16x8*>(krow + c8) = kch;
        *reinterpret_cast<f16x8*>(krow + M + 8 + c8) = kch;
        *reinterpret_cast<f16x8*>(krow + 2 * M + 8 + c8) = kcl;
      }
      // base-2 quantities: token bias b = -log2e * sum_c w_c phi_c; self score
      // t_ii and the upper bound U of any score in this query's row (without
      // the row constant, which cancels in the softmax).
      const float bias = -kLog2e * sumb;
      const float t_ii = kLog2e * tii;
      const float Ub = kLog2e * U;
      const float R = fmaxf(t_ii, Ub - 15.f);
      f16 rh, rl, bh_, bl_;
      split_hi_lo(-R, rh, rl);
      split_hi_lo(bias, bh_, bl_);
      const f16 one = (f16)1.f, zero = (f16)0.f;
      *reinterpret_cast<f16x8*>(qrow + M) = f16x8{one, one, rh, rl, zero, zero, zero, zero};
      *reinterpret_cast<f16x8*>(krow + M) = f16x8{bh_, bl_, one, one, zero, zero, zero, zero};
      p.tstat[bhn] = make_float4(bias, R, Ub - t_ii, 0.f);
    }
    // values, transposed: vt[bh][dd][n] = V_hi, vt[bh][DV + dd][n] = V_lo.
    // One item = one column x 8 consecutive tokens; 8 neighbouring threads
    // cover 64 consecutive tokens of a column (128 contiguous bytes).
    if (n0 + kGemmBN > d.HM) {  // the tile has value columns (uniform)
      const bool vec = d.N % 8 == 0;
      for (int idx = tid; idx < 8 * kGemmBN; idx += 256) {
        const int rg = idx & 7, cc = idx >> 3;
        const int col = n0 + cc, tb = row0 + 8 * rg;
        if (col < d.HM || col >= NC || tb >= T) continue;
        const int vcol = col - d.HM, h = vcol / DV, dd = vcol % DV;
        const float* src = stage + 8 * rg * kStageStride + cc;
        if (vec) {
          // N % 8 == 0 and tb % 8 == 0: the 8 tokens share one batch row
          const int b = tb / d.N, n = tb - b * d.N;
          f16x8 vh, vl;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = src[e * kStageStride];
            vh[e] = (f16)x;
            vl[e] = (f16)(x - (float)vh[e]);
          }
          f16* dst = p.vt + ((int64_t)(b * d.H + h) * 2 * DV + dd) * d.NP + n;
          const int64_t lo = (int64_t)DV * d.NP;
          *reinterpret_cast<f16x8*>(dst) = vh;
          *reinterpret_cast<f16x8*>(dst + lo) = vl;
          if (n + 8 == d.N)
            for (int z = 8; n + z < d.NP; z += 8) {
              *reinterpret_cast<f16x8*>(dst + z) = f16x8{};
              *reinterpret_cast<f16x8*>(dst + lo + z) = f16x8{};
            }
        } else {
          for (int e = 0; e < 8 && tb + e < T; ++e) {
            const int t = tb + e, b = t / d.N, n = t - b * d.N;
            const float x = src[e * kStageStride];
            const f16 vh = (f16)x, vl = (f16)(x - (float)vh);
            f16* dst = p.vt + ((int64_t)(b * d.H + h) * 2 * DV + dd) * d.NP + n;
            const int64_t lo = (int64_t)DV * d.NP;
            dst[0] = vh;
            dst[lo] = vl;
            if (n == d.N - 1)
              for (int z = 1; n + z < d.NP; ++z) {
                dst[z] = (f16)0.f;
                dst[lo + z] = (f16)0.f;
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
  const dim3 grid(gemm_tile_grid((int)((d.T + kGemmBM - 1) / kGemmBM), (d.HM + d.D + kGemmBN - 1) / kGemmBN));
  hipLaunchKernelGGL((proj_fwd_kernel<M, DV>), grid, dim3(256), 0, s, X, gq, gk, d, p);
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
// dq = sum_j dS_ij phi_j, dk = sum_i dS_ij phi_i, dcb = sum_i dS_ij (natural-log
// score gradients, ungated codes):
//   dL/dphi_tc = scale G_c (2 (dq_tc + dk_tc) - dcb_t)
//   dL/dG_c    = scale sum_t phi_tc (2 dk_tc - dcb_t)
// (both use sum_j dS_ij = 0). dL/dG is taken from the key-side sums only, whose
// terms share the same rounded dS, so its cancellation stays exact; then
// d gate_q = dL/dG gate_k and d gate_k = dL/dG gate_q.
// One thread per projection column, kGateTokensPerBlock tokens per block.
__global__ __launch_bounds__(256) void proj_bwd_elem_kernel(const f16* __restrict__ gate_q,
                                                            const f16* __restrict__ gate_k, Dims d, ProjBuffers p,
                                                            BwdBuffers g) {
  const int col = blockIdx.y * 256 + threadIdx.x;
  if (col >= d.HM) return;
  const int h = col / d.M, c = col - h * d.M;
  const float sG = d.scale * (float)gate_q[col] * (float)gate_k[col];
  const int NC = d.HM + d.D;
  const int64_t t0 = (int64_t)blockIdx.x * kGateTokensPerBlock;
  const int64_t t1 = t0 + kGateTokensPerBlock < d.T ? t0 + kGateTokensPerBlock : d.T;
  float sg = 0.f;
  for (int64_t t = t0; t < t1; ++t) {
    const int b = (int)(t / d.N), n = (int)(t - (int64_t)b * d.N);
    const int64_t bhn = (int64_t)(b * d.H + h) * d.N + n;
    const f16* qrow = p.qa + bhn * d.CW;
    const float phi = (float)qrow[c] + (float)qrow[d.M + 8 + c];
    const float dq = g.dq[bhn * d.M + c];
    const float dk = g.dk[bhn * d.M + c];
    const float dcb = g.dcb[bhn];
    const float dphi = sG * (2.f * (dq + dk) - dcb);
    g.dzv[t * NC + col] = (f16)(dphi * phi * (1.f - phi));
    sg += phi * (2.f * dk - dcb);
  }
  g.gpart[(int64_t)blockIdx.x * d.HM + col] = sg;
}

hipError_t launch_proj_bwd_elem(const Dims& d, const f16* gq, const f16* gk, const ProjBuffers& p,
                                const BwdBuffers& g, hipStream_t s) {
  dim3 grid((unsigned)((d.T + kGateTokensPerBlock - 1) / kGateTokensPerBlock), (d.HM + 255) / 256);
  hipLaunchKernelGGL(proj_bwd_elem_kernel, grid, dim3(256), 0, s, gq, gk, d, p, g);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void gate_reduce_kernel(const float* __restrict__ gpart, int nblk, int HM,
                                                          float scale, const f16* __restrict__ gate_q,
                                                          const f16* __restrict__ gate_k, f16* __restrict__ d_gate_q,
                                                          f16* __restrict__ d_gate_k) {
  // 64 columns x 4 row groups per block; fixed summation order (deterministic)
  __shared__ float part[4][64];
  const int cl = threadIdx.x & 63, grp = threadIdx.x >> 6;
  const int col = blockIdx.x * 64 + cl;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (col < HM) {
    int i = grp;
    for (; i + 12 < nblk; i += 16) {
      s0 += gpart[(int64_t)i * HM + col];
      s1 += gpart[(int64_t)(i + 4) * HM + col];
      s2 += gpart[(int64_t)(i + 8) * HM + col];
      s3 += gpart[(int64_t)(i + 12) * HM + col];
    }
    for (; i < nblk; i += 4) s0 += gpart[(int64_t)i * HM + col];
  }
  part[grp][cl] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (grp == 0 && col < HM) {
    const float dG = scale * ((part[0][cl] + part[1][cl]) + (part[2][cl] + part[3][cl]));
    d_gate_q[col] = (f16)(dG * (float)gate_k[col]);
    d_gate_k[col] = (f16)(dG * (float)gate_q[col]);
  }
}

hipError_t launch_gate_reduce(const Dims& d, const BwdBuffers& g, const f16* gq, const f16* gk, f16* dgq, f16* dgk,
                              hipStream_t s) {
  const int nblk = (int)((d.T + kGateTokensPerBlock - 1) / kGateTokensPerBlock);
  hipLaunchKernelGGL(gate_reduce_kernel, dim3((d.HM + 63) / 64), dim3(256), 0, s, g.gpart, nblk, d.HM, d.scale, gq,
                     gk, dgq, dgk);
  return hipGetLastError();
}

// ---------------------------------------------------------------- dX = [dZ | dV] [W_phi | W_V]^T
__global__ __launch_bounds__(256) void dx_gemm_kernel(const f16* __restrict__ W_phi, const f16* __restrict__ W_V,
                                                      const f16* __restrict__ dzv, f16* __restrict__ dX, Dims d) {
  using ML = GemmMainloop<true, true>;
  __shared__ __align__(16) f16 smem[ML::kLdsHalves];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;
  const int T = (int)d.T, NC = d.HM + d.D;
  int tm, tn;
  if (!gemm_tile_map((T + kGemmBM - 1) / kGemmBM, (d.D + kGemmBN - 1) / kGemmBN, tm, tn)) return;
  const int n0 = tn * kGemmBN, m0 = tm * kGemmBM;
  OperandDesc A{dzv, NC, nullptr, 0, INT_MAX};
  OperandDesc B{W_phi, d.HM, W_V, d.D, d.HM};
  f32x16 acc[2][2];
  ML::run(A, B, T, d.D, m0, n0, 0, NC, smem, acc);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + 64 * wn + 32 * j + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + 64 * wm + 32 * i + acc_row(r, lane);
        if (row < T && col < d.D) dX[(int64_t)row * d.D + col] = (f16)acc[i][j][r];
      }
    }
}

hipError_t launch_dx_gemm(const Dims& d, const f16* W_phi, const f16* W_V, const BwdBuffers& g, f16* dX,
                          hipStream_t s) {
  const dim3 grid(gemm_tile_grid((int)((d.T + kGemmBM - 1) / kGemmBM), (d.D + kGemmBN - 1) / kGemmBN));
  hipLaunchKernelGGL(dx_gemm_kernel, grid, dim3(256), 0, s, W_phi, W_V, g.dzv, dX, d);
  return hipGetLastError();
}

// ---------------------------------------------------------------- [dW_phi | dW_V] = X^T [dZ | dV]
// Split-K over tokens: one K slice per XCD (workgroup id % 8), so the tiles
// that share a slice's A and B panels run on one L2 and stream them together.
int dw_splits(const Dims& d) {
  const int kmax = (int)((d.T + 255) / 256);  // keep >= 256 tokens per split
  return kmax < 8 ? kmax : 8;
}

__global__ __launch_bounds__(256) void dw_gemm_kernel(const f16* __restrict__ X, const f16* __restrict__ dzv,
                                                      float* __restrict__ wpart, Dims d, int kchunk, int nsplit) {
  using ML = GemmMainloop<false, false>;
  __shared__ __align__(16) f16 smem[ML::kLdsHalves];
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w >> 1, wn = w & 1;
  const int NC = d.HM + d.D;
  // id = 8 * slot + xcd; split = xcd (+ 8 per extra round), tile = slot within the split
  const int ntn = (NC + kGemmBN - 1) / kGemmBN, ntm = (d.D + kGemmBM - 1) / kGemmBM;
  const int id = blockIdx.x, xcd = id & 7, slot = id >> 3;
  const int tile = slot % (ntn * ntm), z = xcd + 8 * (slot / (ntn * ntm));
  if (z >= nsplit) return;
  const int n0 = (tile % ntn) * kGemmBN, m0 = (tile / ntn) * kGemmBM;
  const int T = (int)d.T;
  const int kbeg = z * kchunk;
  const int kend = kbeg + kchunk < T ? kbeg + kchunk : T;
  OperandDesc A{X, d.D, nullptr, 0, INT_MAX};
  OperandDesc B{dzv, NC, nullptr, 0, INT_MAX};
  f32x16 acc[2][2];
  ML::run(A, B, d.D, NC, m0, n0, kbeg, kend, smem, acc);
  float* out = wpart + (int64_t)z * d.D * NC;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int col = n0 + 64 * wn + 32 * j + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + 64 * wm + 32 * i + acc_row(r, lane);
        if (row < d.D && col < NC) out[(int64_t)row * NC + col] = acc[i][j][r];
      }
    }
}

hipError_t launch_dw_gemm(const Dims& d, const f16* X, const BwdBuffers& g, hipStream_t s) {
  const int S = g.splits;
  const int T = (int)d.T;
  int kchunk = (T + S - 1) / S;
  kchunk = (kchunk + kGemmBK - 1) / kGemmBK * kGemmBK;
  const int tiles = ((d.HM + d.D + kGemmBN - 1) / kGemmBN) * ((d.D + kGemmBM - 1) / kGemmBM);
  const int rounds = (S + 7) / 8;
  dim3 grid(8u * (unsigned)tiles * (unsigned)rounds);
  hipLaunchKernelGGL(dw_gemm_kernel, grid, dim3(256), 0, s, X, g.dzv, g.wpart, d, kchunk, S);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void dw_reduce_kernel(const float* __restrict__ wpart, int splits, int D, int HM,
                                                        f16* __restrict__ dW_phi, f16* __restrict__ dW_V) {
  const int NC = HM + D;
  const int64_t total = (int64_t)D * NC;
  const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (idx >= total) return;
  float4 s = *reinterpret_cast<const float4*>(wpart + idx);
  for (int z = 1; z < splits; ++z) {
    const float4 v = *reinterpret_cast<const float4*>(wpart + (int64_t)z * total + idx);
    s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
  }
  const int row = (int)(idx / NC), col = (int)(idx - (int64_t)row * NC);
  // 4 consecutive columns never straddle HM (HM and NC are multiples of 16)
  f16* dst = col < HM ? dW_phi + (int64_t)row * HM + col : dW_V + (int64_t)row * D + (col - HM);
  dst[0] = (f16)s.x; dst[1] = (f16)s.y; dst[2] = (f16)s.z; dst[3] = (f16)s.w;
}

hipError_t launch_dw_reduce(const Dims& d, const BwdBuffers& g, f16* dW_phi, f16* dW_V, hipStream_t s) {
  const int64_t total = (int64_t)d.D * (d.HM + d.D);
  const unsigned blocks = (unsigned)((total / 4 + 255) / 256);
  hipLaunchKernelGGL(dw_reduce_kernel, dim3(blocks), dim3(256), 0, s, g.wpart, g.splits, d.D, d.HM, dW_phi, dW_V);
  return hipGetLastError();
}

}  // namespace morpho
