// Attention core: scores, softmax and value aggregation (forward) and the
// recompute-from-statistics backward.
//
// Reference: packages/morphottention/csrc/cuda/attention/attention.cu
//   forward  :7-189   (score s = (2 q.k - qb_i - cb_j) * scale * log2e,
//                      causal drop k > q, online softmax in base 2,
//                      out = O / l, lse = m + log2 l)
//   backward :191-483 (P = exp2(s - lse), dV = P^T dO, dP = dO V^T,
//                      dS = P (dP - delta), dk = dS^T q, dcb = -scale sum_i dS;
//                      the query-side dq that the reference accumulates and
//                      drops is completed here)
//
// MI355X design:
//  * The exponent is produced by one MFMA contraction over a code row of
//    width 3m + 8 (see ProjBuffers): fp16 hi/lo code pairs make the score exact
//    to ~2^-22, and the 8-wide augmentation adds the key bias and subtracts
//    the row reference, so exp2 reads the accumulator directly.
//  * Forward softmax uses a per-row reference R >= (row max - 15) computed by
//    the projection from a closed-form bound on the soft Hamming score, so no
//    running max or rescaling is needed; rows whose bound is loose (gap > 25,
//    only possible with large or negative gates) take an exact two-pass path.
//  * V is carried as an fp16 hi/lo pair and both halves are multiplied by the
//    fp16 P; the row normaliser sums exactly those rounded P values.
//  * Transposed operands (V^T, dO^T, phi^T, dS^T) are read from row-major LDS
//    tiles with ds_read_b64_tr_b16.
#include "common.h"
#include "internal.h"

namespace morpho {

constexpr float kGapExact = 25.0f;  // base-2; above this a row takes the exact-max path

__device__ __forceinline__ float sum8(const f16x8& v) {
  const f16x2 one2 = {(f16)1.f, (f16)1.f};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) s = __builtin_amdgcn_fdot2(f16x2{v[2 * i], v[2 * i + 1]}, one2, s, false);
  return s;
}

// ============================================================ forward
template <int M, int DV>
struct FwdCfg {
  static constexpr int CW = 3 * M + 8;  // code row width
  static constexpr int NCH = 3 * M / 16;  // 16-wide code chunks
  static constexpr int KT = 64;         // keys per LDS tile
  static constexpr int KS = CW + 8;     // key row stride (halves)
  static constexpr int VS = 2 * DV + 8;  // value row stride (halves): V_hi | V_lo | pad
  static constexpr int QW = 128;        // queries per workgroup (4 waves x 32)
};

template <int M, int DV, bool MAXPASS>
__device__ __forceinline__ void fwd_tile_loop(const f16* __restrict__ ka, const f16* __restrict__ vv, int64_t rowbase,
                                              int N, int causal, int kend, int qw0, int q, f16* sK, f16* sV,
                                              const f16x8 (&qf)[FwdCfg<M, DV>::NCH], const f16x4& qaug,
                                              f32x16 (&o)[DV / 32], float& lsum, float& rmax) {
  using C = FwdCfg<M, DV>;
  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int nkt = (kend + C::KT - 1) / C::KT;
  const int wave_kend = causal ? min(N, qw0 + 32) : N;
  for (int kt = 0; kt < nkt; ++kt) {
    const int k0 = kt * C::KT;
    __syncthreads();  // previous tile fully consumed
    for (int v = tid; v < C::KT * (C::CW / 8); v += 256) {
      const int r = v / (C::CW / 8), cv = (v % (C::CW / 8)) * 8;
      f16x8 x = {};
      if (k0 + r < N) x = *reinterpret_cast<const f16x8*>(ka + (rowbase + k0 + r) * C::CW + cv);
      *reinterpret_cast<f16x8*>(sK + r * C::KS + cv) = x;
    }
    if (!MAXPASS) {
      for (int v = tid; v < C::KT * (DV / 4); v += 256) {
        const int r = v / (DV / 4), cv = (v % (DV / 4)) * 8;
        f16x8 x = {};
        if (k0 + r < N) x = *reinterpret_cast<const f16x8*>(vv + (rowbase + k0 + r) * (2 * DV) + cv);
        *reinterpret_cast<f16x8*>(sV + r * C::VS + cv) = x;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kbase = k0 + 32 * kb;
      if (kbase >= wave_kend) continue;  // wave-uniform
      const f16* krow = sK + (32 * kb + swap23(l32)) * C::KS;
      f32x16 s = {};
#pragma unroll
      for (int c = 0; c < C::NCH; ++c) s = mfma16(*reinterpret_cast<const f16x8*>(krow + 16 * c + 8 * h32), qf[c], s);
      s = mfma8(*reinterpret_cast<const f16x4*>(krow + 3 * M + 4 * h32), qaug, s);
      const bool need_mask = (kbase + 31 >= N) || (causal && kbase + 31 > qw0);
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kbase + swap23(acc_row(r, lane));
          if (key >= N || (causal && key > q)) s[r] = kNegInf;
        }
      }
      if (MAXPASS) {
#pragma unroll
        for (int r = 0; r < 16; ++r) rmax = fmaxf(rmax, s[r]);
        continue;
      }
      f16x8 p0, p1;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        p0[r] = (f16)fast_exp2(s[r]);
        p1[r] = (f16)fast_exp2(s[r + 8]);
      }
      lsum += sum8(p0) + sum8(p1);
#pragma unroll
      for (int dvb = 0; dvb < DV / 32; ++dvb) {
        f32x16 acc = o[dvb];
        acc = mfma16(frag_kmajor(sV, C::VS, 32 * kb, 32 * dvb, lane), p0, acc);
        acc = mfma16(frag_kmajor(sV, C::VS, 32 * kb + 16, 32 * dvb, lane), p1, acc);
        acc = mfma16(frag_kmajor(sV, C::VS, 32 * kb, DV + 32 * dvb, lane), p0, acc);
        acc = mfma16(frag_kmajor(sV, C::VS, 32 * kb + 16, DV + 32 * dvb, lane), p1, acc);
        o[dvb] = acc;
      }
    }
  }
}

template <int M, int DV>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const f16* __restrict__ qa, const f16* __restrict__ ka,
                                                       const f16* __restrict__ vv, const float4* __restrict__ tstat,
                                                       f16* __restrict__ out, float* __restrict__ lse, int N, int H,
                                                       int D, int causal) {
  using C = FwdCfg<M, DV>;
  __shared__ __align__(16) f16 sK[C::KT * C::KS];
  __shared__ __align__(16) f16 sV[C::KT * C::VS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h32 = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.y;
  const int qblk = causal ? (int)(gridDim.x - 1 - blockIdx.x) : (int)blockIdx.x;  // longest rows first
  const int q0 = qblk * C::QW, qw0 = q0 + 32 * w, q = qw0 + l32;
  const bool qvalid = q < N;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N;

  f16x8 qf[C::NCH];
  f16x4 qaug = {};
#pragma unroll
  for (int c = 0; c < C::NCH; ++c) qf[c] = f16x8{};
  float4 ts = make_float4(0.f, 0.f, 0.f, 0.f);
  if (qvalid) {
    const f16* qrow = qa + (rowbase + q) * C::CW;
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) qf[c] = *reinterpret_cast<const f16x8*>(qrow + 16 * c + 8 * h32);
    qaug = *reinterpret_cast<const f16x4*>(qrow + 3 * M + 4 * h32);
    ts = tstat[rowbase + q];
  }
  float R = ts.y;
  const int kend = causal ? min(N, q0 + C::QW) : N;
  f32x16 o[DV / 32];
#pragma unroll
  for (int i = 0; i < DV / 32; ++i) o[i] = f32x16{};
  float lsum = 0.f, rmax = kNegInf;

  const bool exact = __syncthreads_or(qvalid && ts.z > kGapExact);
  if (exact) {
    // pass 1: exact row max of the base-2 exponent without the reference
    f16x4 qa0 = qaug;
    if (h32 == 0) { qa0[2] = (f16)0.f; qa0[3] = (f16)0.f; }
    fwd_tile_loop<M, DV, true>(ka, vv, rowbase, N, causal, kend, qw0, q, sK, sV, qf, qa0, o, lsum, rmax);
    rmax = fmaxf(rmax, __shfl_xor(rmax, 32));
    R = qvalid ? rmax : 0.f;
    f16 rh, rl;
    split_hi_lo(-R, rh, rl);
    if (h32 == 0) { qaug[2] = rh; qaug[3] = rl; }
  }
  fwd_tile_loop<M, DV, false>(ka, vv, rowbase, N, causal, kend, qw0, q, sK, sV, qf, qaug, o, lsum, rmax);

  const float ltot = lsum + __shfl_xor(lsum, 32);
  if (qvalid) {
    const float inv = ltot > 0.f ? 1.0f / ltot : 0.f;
    f16* orow = out + ((int64_t)b * N + q) * D + h * DV;
#pragma unroll
    for (int dvb = 0; dvb < DV / 32; ++dvb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (f16)(o[dvb][4 * g + e] * inv);
        *reinterpret_cast<f16x4*>(orow + 32 * dvb + 8 * g + 4 * h32) = v;
      }
    if (h32 == 0) lse[rowbase + q] = ltot > 0.f ? R + fast_log2(ltot) + ts.x : -kFltMax;
  }
}

template <int M, int DV>
static hipError_t launch_attn_fwd_t(const Dims& d, const ProjBuffers& p, f16* out, float* lse, hipStream_t s) {
  using C = FwdCfg<M, DV>;
  dim3 grid((d.N + C::QW - 1) / C::QW, d.B * d.H);
  hipLaunchKernelGGL((attn_fwd_kernel<M, DV>), grid, dim3(256), 0, s, p.qa, p.ka, p.v, p.tstat, out, lse, d.N, d.H,
                     d.D, d.causal);
  return hipGetLastError();
}

#define MORPHO_MDV_DISPATCH(FN, ...)                                                         \
  do {                                                                                       \
    if (d.M == 16 && d.DV == 32) return FN<16, 32>(__VA_ARGS__);                             \
    if (d.M == 16 && d.DV == 64) return FN<16, 64>(__VA_ARGS__);                             \
    if (d.M == 16 && d.DV == 128) return FN<16, 128>(__VA_ARGS__);                           \
    if (d.M == 32 && d.DV == 32) return FN<32, 32>(__VA_ARGS__);                             \
    if (d.M == 32 && d.DV == 64) return FN<32, 64>(__VA_ARGS__);                             \
    if (d.M == 32 && d.DV == 128) return FN<32, 128>(__VA_ARGS__);                           \
    if (d.M == 64 && d.DV == 32) return FN<64, 32>(__VA_ARGS__);                             \
    if (d.M == 64 && d.DV == 64) return FN<64, 64>(__VA_ARGS__);                             \
    if (d.M == 64 && d.DV == 128) return FN<64, 128>(__VA_ARGS__);                           \
    return hipErrorInvalidValue;                                                             \
  } while (0)

hipError_t launch_attn_fwd(const Dims& d, const ProjBuffers& p, f16* out, float* lse, hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_attn_fwd_t, d, p, out, lse, s);
}

// ============================================================ backward prep
// qstat = {-(lse - b), -delta} with delta_i = dO_i . O_i (fp32); zeroes dq.
template <int M, int DV>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const f16* __restrict__ grad_out, const f16* __restrict__ out,
                                                       const float* __restrict__ lse,
                                                       const float4* __restrict__ tstat, float2* __restrict__ qstat,
                                                       float* __restrict__ dq, int N, int H, int D) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  const int bh = blockIdx.y;
  if (n >= N) return;
  const int b = bh / H, h = bh - b * H;
  const int64_t bhn = (int64_t)bh * N + n;
  const f16* go = grad_out + ((int64_t)b * N + n) * D + h * DV;
  const f16* oo = out + ((int64_t)b * N + n) * D + h * DV;
  float delta = 0.f;
#pragma unroll
  for (int c = 0; c < DV; c += 8) {
    const f16x8 a = *reinterpret_cast<const f16x8*>(go + c);
    const f16x8 o = *reinterpret_cast<const f16x8*>(oo + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) delta += (float)a[e] * (float)o[e];
  }
  qstat[bhn] = make_float2(-(lse[bhn] - tstat[bhn].x), -delta);
  float4* z = reinterpret_cast<float4*>(dq + bhn * M);
#pragma unroll
  for (int c = 0; c < M / 4; ++c) z[c] = make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int M, int DV>
static hipError_t launch_bwd_prep_t(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* out,
                                    const float* lse, const BwdBuffers& g, hipStream_t s) {
  dim3 grid((d.N + 255) / 256, d.B * d.H);
  hipLaunchKernelGGL((bwd_prep_kernel<M, DV>), grid, dim3(256), 0, s, grad_out, out, lse, p.tstat, g.qstat, g.dq, d.N,
                     d.H, d.D);
  return hipGetLastError();
}

hipError_t launch_bwd_prep(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* out, const float* lse,
                           const BwdBuffers& g, hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_bwd_prep_t, d, p, grad_out, out, lse, g, s);
}

// ============================================================ backward
template <int M, int DV>
struct BwdCfg {
  static constexpr int CW = 3 * M + 8;
  static constexpr int NCH = 3 * M / 16;
  static constexpr int MB = (M + 1 + 31) / 32;  // 32-row blocks of dk^T (codes + the ones row)
  static constexpr int MQ = (M + 31) / 32;      // 32-column blocks of dq
  static constexpr int QT = 32;                 // queries per step
  static constexpr int QS = CW + 8;             // score-operand query tile stride
  static constexpr int PS = 32 * MB + 8;        // phi^T tile stride: phi_hi | 1 | zeros
  static constexpr int OS = DV + 16;            // dO tile stride: DV values + 8 aug + pad
  static constexpr int SS = 32 + 8;             // dS tile stride
  static constexpr int KW = 128;                // keys per workgroup (4 waves x 32)
};

template <int M, int DV>
__global__ __launch_bounds__(256) void attn_bwd_kernel(const f16* __restrict__ qa, const f16* __restrict__ ka,
                                                       const f16* __restrict__ vv, const float2* __restrict__ qstat,
                                                       const f16* __restrict__ grad_out, float* __restrict__ dq,
                                                       float* __restrict__ dk, float* __restrict__ dcb,
                                                       f16* __restrict__ dzv, int N, int H, int D, int HM,
                                                       int causal) {
  using C = BwdCfg<M, DV>;
  __shared__ __align__(16) f16 sQ[2][C::QT * C::QS];
  __shared__ __align__(16) f16 sP[2][C::QT * C::PS];
  __shared__ __align__(16) f16 sO[2][C::QT * C::OS];
  __shared__ __align__(16) f16 sdS[4][32 * C::SS];
  __shared__ __align__(16) float sdq[4][C::QT * M];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h32 = lane >> 5, l32 = lane & 31;
  const int bh = blockIdx.y;
  const int k0 = blockIdx.x * C::KW;  // causal: low key blocks see the most queries; they start first
  const int kw0 = k0 + 32 * w;
  const int key = kw0 + l32;
  const bool kvalid = key < N;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N;
  const f16 one = (f16)1.f, zero = (f16)0.f;

  // ---- per-wave key-side operands, loaded once
  f16x8 kf[C::NCH];
  f16x4 kaug = {};
  f16x8 vf[DV / 16];
  f16x8 kq[C::MQ][2];
#pragma unroll
  for (int c = 0; c < C::NCH; ++c) kf[c] = f16x8{};
#pragma unroll
  for (int c = 0; c < DV / 16; ++c) vf[c] = f16x8{};
  if (kvalid) {
    const f16* krow = ka + (rowbase + key) * C::CW;
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) kf[c] = *reinterpret_cast<const f16x8*>(krow + 16 * c + 8 * h32);
    kaug = *reinterpret_cast<const f16x4*>(krow + 3 * M + 4 * h32);
    const f16* vrow = vv + (rowbase + key) * (2 * DV);
#pragma unroll
    for (int c = 0; c < DV / 16; ++c) vf[c] = *reinterpret_cast<const f16x8*>(vrow + 16 * c + 8 * h32);
  }
  const f16x4 vaug = h32 == 0 ? f16x4{one, one, zero, zero} : f16x4{zero, zero, zero, zero};
  // B operand of dq = dS phi_keys: lane supplies phi_hi[kw0 + 16 c + 8 h32 + j][32 cb + l32]
#pragma unroll
  for (int cb = 0; cb < C::MQ; ++cb)
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      f16x8 x = {};
      const int code = 32 * cb + l32;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kk = kw0 + 16 * c + 8 * h32 + j;
        if (code < M && kk < N) x[j] = qa[(rowbase + kk) * C::CW + code];
      }
      kq[cb][c] = x;
    }

  f32x16 dva[DV / 32], dka[C::MB];
#pragma unroll
  for (int i = 0; i < DV / 32; ++i) dva[i] = f32x16{};
#pragma unroll
  for (int i = 0; i < C::MB; ++i) dka[i] = f32x16{};

  const int qstart = causal ? k0 : 0;
  const int nsteps = qstart < N ? (N - qstart + C::QT - 1) / C::QT : 0;

  auto stage = [&](int step, int buf) {
    const int qs = qstart + step * C::QT;
    // score operand rows: codes (3M) | 1, 1, -L_hi, -L_lo, 0 x4
    for (int v = tid; v < C::QT * (C::CW / 8); v += 256) {
      const int r = v / (C::CW / 8), cv = (v % (C::CW / 8)) * 8;
      const int qq = qs + r;
      f16x8 x = {};
      if (qq < N) {
        if (cv < 3 * M) {
          x = *reinterpret_cast<const f16x8*>(qa + (rowbase + qq) * C::CW + cv);
        } else {
          f16 lh, ll;
          split_hi_lo(qstat[rowbase + qq].x, lh, ll);
          x = f16x8{one, one, lh, ll, zero, zero, zero, zero};
        }
      }
      *reinterpret_cast<f16x8*>(&sQ[buf][r * C::QS + cv]) = x;
    }
    // key-gradient operand rows: phi_hi (M) | 1 | zeros to 32 MB
    for (int v = tid; v < C::QT * (32 * C::MB / 8); v += 256) {
      const int r = v / (32 * C::MB / 8), cv = (v % (32 * C::MB / 8)) * 8;
      const int qq = qs + r;
      f16x8 x = {};
      if (qq < N) {
        if (cv < M) x = *reinterpret_cast<const f16x8*>(qa + (rowbase + qq) * C::CW + cv);
        else if (cv == M) x[0] = one;
      }
      *reinterpret_cast<f16x8*>(&sP[buf][r * C::PS + cv]) = x;
    }
    // dO rows: dO_h | -delta_hi, -delta_lo, 0.. | zero pad to OS
    for (int v = tid; v < C::QT * (C::OS / 8); v += 256) {
      const int r = v / (C::OS / 8), cv = (v % (C::OS / 8)) * 8;
      const int qq = qs + r;
      f16x8 x = {};
      if (qq < N) {
        if (cv < DV) {
          x = *reinterpret_cast<const f16x8*>(grad_out + ((int64_t)b * N + qq) * D + h * DV + cv);
        } else if (cv == DV) {
          f16 dh, dl;
          split_hi_lo(qstat[rowbase + qq].y, dh, dl);
          x = f16x8{dh, dl, zero, zero, zero, zero, zero, zero};
        }
      }
      *reinterpret_cast<f16x8*>(&sO[buf][r * C::OS + cv]) = x;
    }
  };

  // Sum the per-wave dq partials of one step and add them to global memory.
  auto flush_dq = [&](int step) {
    const int qs = qstart + step * C::QT;
    int nact = 0;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww)
      if (!(causal && k0 + 32 * ww > qs + C::QT - 1) && k0 + 32 * ww < N) nact = ww + 1;
    for (int idx = tid; idx < C::QT * M; idx += 256) {
      const int r = idx / M, c = idx - r * M;
      const int qq = qs + r;
      if (qq >= N) continue;
      float s = 0.f;
      for (int ww = 0; ww < nact; ++ww) s += sdq[ww][idx];
      unsafeAtomicAdd(dq + (rowbase + qq) * M + c, s);
    }
  };

  if (nsteps > 0) stage(0, 0);
  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const int qs = qstart + step * C::QT;
    __syncthreads();  // staging of `step` visible; sdq of step-1 complete
    if (step > 0) flush_dq(step - 1);
    const bool active = !(causal && kw0 > qs + C::QT - 1) && kw0 < N;  // wave-uniform
    if (active) {
      // S = Q~ K~^T (rows: queries in swap23 order; lane: key)
      const f16* qrow = &sQ[buf][swap23(l32) * C::QS];
      f32x16 s = {};
#pragma unroll
      for (int c = 0; c < C::NCH; ++c) s = mfma16(*reinterpret_cast<const f16x8*>(qrow + 16 * c + 8 * h32), kf[c], s);
      s = mfma8(*reinterpret_cast<const f16x4*>(qrow + 3 * M + 4 * h32), kaug, s);
      // dP - delta = dO~ V~^T
      const f16* orow = &sO[buf][swap23(l32) * C::OS];
      f32x16 dp = {};
#pragma unroll
      for (int c = 0; c < DV / 16; ++c) dp = mfma16(*reinterpret_cast<const f16x8*>(orow + 16 * c + 8 * h32), vf[c], dp);
      dp = mfma8(*reinterpret_cast<const f16x4*>(orow + DV + 4 * h32), vaug, dp);
      const bool need_mask = (qs + C::QT > N) || (kw0 + 31 >= N) || (causal && kw0 + 31 > qs);
      f16x8 p16[2], ds16[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float pr = fast_exp2(s[r]);
        if (need_mask) {
          const int qq = qs + swap23(acc_row(r, lane));
          if (qq >= N || !kvalid || (causal && key > qq)) pr = 0.f;
        }
        p16[r >> 3][r & 7] = (f16)pr;
        ds16[r >> 3][r & 7] = (f16)(pr * dp[r]);
      }
      // dV^T += dO^T P ; dk^T += phi^T dS  (rows: dv / code; lane: key)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int dvb = 0; dvb < DV / 32; ++dvb)
          dva[dvb] = mfma16(frag_kmajor(sO[buf], C::OS, 16 * c, 32 * dvb, lane), p16[c], dva[dvb]);
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
          dka[mb] = mfma16(frag_kmajor(sP[buf], C::PS, 16 * c, 32 * mb, lane), ds16[c], dka[mb]);
      }
      // dS^T to LDS: row = key, 32 query columns
#pragma unroll
      for (int c = 0; c < 2; ++c) *reinterpret_cast<f16x8*>(&sdS[w][l32 * C::SS + 16 * c + 8 * h32]) = ds16[c];
    }
    if (step + 1 < nsteps) stage(step + 1, buf ^ 1);
    __syncthreads();  // dS tiles visible
    if (active) {
      // dq[q][code] = sum_key dS[q][key] phi[key][code] (rows: q natural; lane: code)
#pragma unroll
      for (int cb = 0; cb < C::MQ; ++cb) {
        f32x16 acc = {};
#pragma unroll
        for (int c = 0; c < 2; ++c) acc = mfma16(frag_kmajor(sdS[w], C::SS, 16 * c, 0, lane), kq[cb][c], acc);
        const int code = 32 * cb + l32;
        if (code < M) {
#pragma unroll
          for (int r = 0; r < 16; ++r) sdq[w][acc_row(r, lane) * M + code] = acc[r];
        }
      }
    }
  }
  if (nsteps > 0) {
    __syncthreads();
    flush_dq(nsteps - 1);
  }

  // ---- epilogue: dk, dcb (fp32, per key) and dV (fp16 into the dZ|dV buffer)
  if (kvalid) {
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int code = 32 * mb + acc_row(r, lane);
        if (code < M) dk[(rowbase + key) * M + code] = dka[mb][r];
        if (code == M) dcb[rowbase + key] = dka[mb][r];
      }
    const int NC = HM + D;
    f16* drow = dzv + ((int64_t)b * N + key) * NC + HM + h * DV;
#pragma unroll
    for (int dvb = 0; dvb < DV / 32; ++dvb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (f16)dva[dvb][4 * g + e];
        *reinterpret_cast<f16x4*>(drow + 32 * dvb + 8 * g + 4 * h32) = v;
      }
  }
}

template <int M, int DV>
static hipError_t launch_attn_bwd_t(const Dims& d, const ProjBuffers& p, const f16* grad_out, const BwdBuffers& g,
                                    hipStream_t s) {
  using C = BwdCfg<M, DV>;
  dim3 grid((d.N + C::KW - 1) / C::KW, d.B * d.H);
  hipLaunchKernelGGL((attn_bwd_kernel<M, DV>), grid, dim3(256), 0, s, p.qa, p.ka, p.v, g.qstat, grad_out, g.dq, g.dk,
                     g.dcb, g.dzv, d.N, d.H, d.D, d.HM, d.causal);
  return hipGetLastError();
}

hipError_t launch_attn_bwd(const Dims& d, const ProjBuffers& p, const f16* grad_out, const BwdBuffers& g,
                           hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_attn_bwd_t, d, p, grad_out, g, s);
}

}  // namespace morpho
