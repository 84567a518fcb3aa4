// Soft tropical aggregation of the values with the morpho scores:
//     out_ic = sgn tau ln sum_j exp(sgn (s_ij + V_jc) / tau)
// (sgn = +1 soft max-plus / dilation, sgn = -1 soft min-plus / erosion).
//
// Reference: packages/morphottention/csrc/cuda/morfology/soft_morph.cuh
//   lse_init / lse_update :21-32   running (max, sum) of exp
//   morph_accumulate      :35-38   fold sgn (s + v) / tau
//   lse_merge / warp red. :41-63   combine two accumulators
//   lse_finalize          :66-69   sgn tau (m + log l)
//   morph_weight          :71-75   P_ijc = exp(sgn ((s + v) - out_ic) / tau)
//   morph_dtau_term       :77-80   dtau_ic = (out_ic - sum_j P (s + v)) / tau
// The reference defines these and never calls them; the kernels below are
// the aggregation built from them on top of this library's projection.
//
// MI355X design:
//  * Scores come from the same code-row MFMA as the softmax path, with the
//    query affine block set to the token bias so that the accumulator is
//    exactly log2e s_ij. Everything runs in base 2: y = u + w with
//    u = sgn log2e s / tau and w = sgn log2e v / tau.
//  * Product form (the default): sum_j 2^(u_ij + w_jc) = 2^(A_i + B_c) (E F)_ic
//    with E = 2^(u - A_i), F = 2^(w - B_c) (A_i the running row maximum of u,
//    B_c the maximum of w over the head's keys), so the aggregation and both
//    of its gradient products run on the bf16 MFMA (hi/lo pairs): one exp2
//    per (query, key) instead of per (query, key, column). Each output checks
//    that its sum is at least 2^-80, below which the form could lose
//    precision; if any fails, a device flag makes the element-wise kernels
//    recompute the call.
//  * Element-wise kernels (the fallback, or on request): forward lane = query
//    with an online (max, sum) per (query, column) (lse_update, lse_merge,
//    lse_finalize); backward lane = key with P_ijc = 2^(y - zb_ic). One exp2
//    and four VALU operations per (query, key, column).
//  * Both backward paths fold the query-side row sum of ds, sum_c dO_ic (which
//    the softmax gradient does not have), into dcb, so the projection
//    backward is shared unchanged, and form dtau = (sum dO out - sum ds s -
//    sum dV V) / tau from per-workgroup partials reduced in a fixed order.
#include "common.h"
#include "internal.h"

namespace morpho {

constexpr float kLn2 = 0.6931471805599453f;

template <int M, int DV>
struct SoftCfg {
  static constexpr int CW = 2 * M + 8;
  static constexpr int NCH = M / 8;
  static constexpr int CG = DV / 32;     // 32-column groups, one per wave
  static constexpr int QBW = 4 / CG;     // forward: 32-query blocks per workgroup
  static constexpr int QW = 32 * QBW;
  static constexpr int KB = 4 / CG;      // backward: 32-key blocks per workgroup
  static constexpr int KW = 32 * KB;
  static constexpr int WS = DV + 4;      // fp32 LDS row stride of value-column rows
  static constexpr int QT = 32;          // backward: queries per step
  static constexpr int PS = M + 4;       // fp32 LDS row stride of phi rows
  static constexpr int DS = KW + 1;      // fp32 LDS row stride of ds rows (odd: conflict-free columns)
};

// V_hi + V_lo of key `key`, value column c of head bh (fp32; the remainder is
// e4m3 times 2^kVloExp in the tile-major, key-permuted layout).
__device__ __forceinline__ float load_value(const f16* __restrict__ vt, const uint8_t* __restrict__ vlo, int bh,
                                            int DV, int NP, int c, int key) {
  const float hi = (float)vt[((int64_t)bh * DV + c) * NP + key];
  const uint8_t b = vlo[(((int64_t)bh * (NP / 64) + key / 64) * DV + c) * 64 + vlo_pos(key & 63)];
  return hi + __builtin_amdgcn_cvt_f32_fp8((int)b, 0) * (1.0f / (float)(1 << kVloExp));
}

// V of keys k0 .. k0 + 7 of column c (k0 % 8 == 0, k0 + 8 <= NP), as
// load_value computes it: one 16-byte V_hi load and one 8-byte remainder
// load (vlo_pos maps 8 aligned keys to 8 consecutive bytes of their block).
__device__ __forceinline__ void load_values8(const f16* __restrict__ vt, const uint8_t* __restrict__ vlo, int bh,
                                             int DV, int NP, int c, int k0, float (&v)[8]) {
  const f16x8 hi = *reinterpret_cast<const f16x8*>(vt + ((int64_t)bh * DV + c) * NP + k0);
  const uint2 lo =
      *reinterpret_cast<const uint2*>(vlo + (((int64_t)bh * (NP / 64) + k0 / 64) * DV + c) * 64 + vlo_pos(k0 & 63));
  constexpr float s = 1.0f / (float)(1 << kVloExp);
  v[0] = (float)hi[0] + __builtin_amdgcn_cvt_f32_fp8((int)lo.x, 0) * s;
  v[1] = (float)hi[1] + __builtin_amdgcn_cvt_f32_fp8((int)lo.x, 1) * s;
  v[2] = (float)hi[2] + __builtin_amdgcn_cvt_f32_fp8((int)lo.x, 2) * s;
  v[3] = (float)hi[3] + __builtin_amdgcn_cvt_f32_fp8((int)lo.x, 3) * s;
  v[4] = (float)hi[4] + __builtin_amdgcn_cvt_f32_fp8((int)lo.y, 0) * s;
  v[5] = (float)hi[5] + __builtin_amdgcn_cvt_f32_fp8((int)lo.y, 1) * s;
  v[6] = (float)hi[6] + __builtin_amdgcn_cvt_f32_fp8((int)lo.y, 2) * s;
  v[7] = (float)hi[7] + __builtin_amdgcn_cvt_f32_fp8((int)lo.y, 3) * s;
}

// The query operand of a code row with its affine block set to {1, 1, b_hi,
// b_lo}: the score accumulator is then log2e s_ij (the projection's row
// reference R is replaced by the token bias b).
template <int M>
__device__ __forceinline__ void load_query_operand(const f16* __restrict__ qrow, float b, int h32, f16x8 (&qf)[M / 8],
                                                   f16x4& qaug) {
#pragma unroll
  for (int c = 0; c < M / 8; ++c) qf[c] = *reinterpret_cast<const f16x8*>(qrow + chunk_off<M>(c) + 8 * h32);
  qaug = *reinterpret_cast<const f16x4*>(qrow + M + 4 * h32);
  if (h32 == 0) {
    f16 bh_, bl_;
    split_hi_lo(b, bh_, bl_);
    qaug[2] = bh_;
    qaug[3] = bl_;
  }
}

template <int M>
__device__ __forceinline__ void load_key_operand(const f16* __restrict__ krow, int h32, f16x8 (&kf)[M / 8],
                                                 f16x4& kaug) {
#pragma unroll
  for (int c = 0; c < M / 8; ++c) kf[c] = *reinterpret_cast<const f16x8*>(krow + chunk_off<M>(c) + 8 * h32);
  kaug = *reinterpret_cast<const f16x4*>(krow + M + 4 * h32);
}

// ============================================================ forward
// Workgroup: QBW blocks of 32 queries x CG groups of 32 value columns, one
// wave each. Keys stream in 32-key blocks; the fp32 value tile of a block
// (scaled by sgn log2e / tau) is written by all threads into one of two LDS
// buffers while the other is read.
template <int M, int DV, bool MD>
__global__ __launch_bounds__(256) void soft_fwd_kernel(const f16* __restrict__ qa, const f16* __restrict__ ka,
                                                       const f16* __restrict__ vt, const uint8_t* __restrict__ vlo,
                                                       const float4* __restrict__ tstat, const float* __restrict__ tau_p,
                                                       f16* __restrict__ out, float* __restrict__ zb, int N, int NP,
                                                       int H, int D, int BH, int causal, float sgn,
                                                       const int* __restrict__ run_flag) {
  using C = SoftCfg<M, DV>;
  __shared__ __align__(16) float sw[2][32 * C::WS];
  if (run_flag && *run_flag == 0) return;  // the product form was exact for every output
  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nqb = (N + C::QW - 1) / C::QW;
  int bh, blk;
  if (!(causal ? xcd_map_lpt(nqb, BH, bh, blk) : xcd_map(nqb, BH, bh, blk))) return;
  const int qblk = causal ? nqb - 1 - blk : blk;  // longest rows first
  const int q0 = qblk * C::QW, qw0 = q0 + 32 * (w % C::QBW), c0 = 32 * (w / C::QBW);
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N;
  const float tau = *tau_p;
  const float ks = sgn / tau, kw = sgn * kLog2e / tau;  // score and value scales of the base-2 exponent

  const int q = qw0 + l32;
  f16x8 qf[C::NCH];
  f16x4 qaug = {};
#pragma unroll
  for (int c = 0; c < C::NCH; ++c) qf[c] = f16x8{};
  if (q < N) load_query_operand<M>(qa + (rowbase + q) * C::CW, tstat[rowbase + q].x, h32, qf, qaug);

  float mx[32], sm[32];  // running max and sum of 2^y per value column of this wave
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    mx[c] = kNegInf;
    sm[c] = 0.f;
  }
  const int kend = causal ? min(N, q0 + C::QW) : N;
  const int nkb = (kend + 31) / 32;

  auto stage = [&](int kb, float* dst) {
#pragma unroll 4
    for (int e = tid; e < 32 * DV; e += 256) {
      const int k = e & 31, c = e >> 5, key = 32 * kb + k;
      dst[k * C::WS + c] = key < N ? kw * load_value(vt, vlo, bh, DV, NP, c, key) : 0.f;
    }
  };
  if (nkb > 0) stage(0, sw[0]);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const float* tile = sw[kb & 1];
    if (kb + 1 < nkb) stage(kb + 1, sw[(kb + 1) & 1]);
    // S^T block: rows = keys 32 kb + acc_row(r), column = this lane's query
    const int key0 = 32 * kb;
    f16x8 kf[C::NCH];
    f16x4 kaug = {};
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) kf[c] = f16x8{};
    if (key0 + l32 < N) load_key_operand<M>(ka + (rowbase + key0 + l32) * C::CW, h32, kf, kaug);
    f32x16 acc = code_dot<M, true>(kf, qf, f32x16{});
    acc = mfma8(kaug, qaug, acc);
    float u[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = key0 + acc_row(r, lane);
      const bool drop = (key >= N) | (causal != 0 && key > q) | (MD && key == q);
      u[r] = drop ? kNegInf : ks * acc[r];
    }
    // online (max, sum) per value column over this lane's 16 keys
#pragma unroll
    for (int c4 = 0; c4 < 8; ++c4) {
      float y[16][4];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float4 w4 = *reinterpret_cast<const float4*>(tile + acc_row(r, lane) * C::WS + c0 + 4 * c4);
        y[r][0] = u[r] + w4.x;
        y[r][1] = u[r] + w4.y;
        y[r][2] = u[r] + w4.z;
        y[r][3] = u[r] + w4.w;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = 4 * c4 + j;
        float bm = y[0][j];
#pragma unroll
        for (int r = 1; r < 16; ++r) bm = fmaxf(bm, y[r][j]);
        const float mn = fmaxf(mx[c], bm);
        const float ref = mn == kNegInf ? 0.f : mn;  // nothing unmasked yet: every term is 0
        float add = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) add += fast_exp2(y[r][j] - ref);
        sm[c] = sm[c] * fast_exp2(mx[c] - ref) + add;
        mx[c] = mn;
      }
    }
    __syncthreads();  // the next block's tile is staged; this block's tile is free again
  }

  // lse_merge of the two half-waves (same query, complementary keys), then
  // lse_finalize; each half writes 16 of the wave's 32 columns
  float zv[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) {
    const float m2 = __shfl_xor(mx[c], 32), s2 = __shfl_xor(sm[c], 32);
    const float mn = fmaxf(mx[c], m2);
    const float ref = mn == kNegInf ? 0.f : mn;
    const float l = sm[c] * fast_exp2(mx[c] - ref) + s2 * fast_exp2(m2 - ref);
    zv[c] = l > 0.f ? mn + fast_log2(l) : -kFltMax;
  }
  if (q < N) {
    f16* orow = out + ((int64_t)b * N + q) * D + h * DV + c0 + 16 * h32;
    float* zrow = zb + (rowbase + q) * DV + c0 + 16 * h32;
    const float ko = sgn * tau * kLn2;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float z = h32 ? zv[16 + 8 * g + e] : zv[8 * g + e];
        o[e] = (f16)(z > -kFltMax ? ko * z : 0.f);
      }
      *reinterpret_cast<f16x8*>(orow + 8 * g) = o;
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float4 z4;
      z4.x = h32 ? zv[16 + 4 * g] : zv[4 * g];
      z4.y = h32 ? zv[17 + 4 * g] : zv[4 * g + 1];
      z4.z = h32 ? zv[18 + 4 * g] : zv[4 * g + 2];
      z4.w = h32 ? zv[19 + 4 * g] : zv[4 * g + 3];
      *reinterpret_cast<float4*>(zrow + 4 * g) = z4;
    }
  }
}

template <int M, int DV>
static hipError_t launch_soft_fwd_t(const Dims& d, const ProjBuffers& p, const float* tau, int sgn, f16* out,
                                    float* zb, const int* run_flag, hipStream_t s) {
  using C = SoftCfg<M, DV>;
  const dim3 grid(xcd_grid((d.N + C::QW - 1) / C::QW, d.B * d.H));
  if (d.mask_diag)
    MORPHO_KLAUNCH((soft_fwd_kernel<M, DV, true>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.vlo, p.tstat, tau,
                       out, zb, d.N, d.NP, d.H, d.D, d.B * d.H, d.causal, (float)sgn, run_flag);
  else
    MORPHO_KLAUNCH((soft_fwd_kernel<M, DV, false>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.vlo, p.tstat, tau,
                       out, zb, d.N, d.NP, d.H, d.D, d.B * d.H, d.causal, (float)sgn, run_flag);
  return hipGetLastError();
}

hipError_t launch_soft_fwd(const Dims& d, const ProjBuffers& p, const float* tau, int sgn, f16* out, float* zb,
                           const int* run_flag, hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_soft_fwd_t, d, p, tau, sgn, out, zb, run_flag, s);
}

// ============================================================ product form
// sum_j 2^(u_ij + w_jc) = 2^(A_i + B_c) sum_j E_ij F_jc with E = 2^(u - A_i) and
// F = 2^(w - B_c), A_i the running row maximum of u and B_c the maximum of w
// over the head's keys. The sum is then a matrix product, which runs on the
// bf16 MFMA with hi/lo pairs (bf16 keeps fp32's exponent range, the pairs
// carry 2^-16 relative precision). It equals the exact sum to that precision
// while the largest term is not far below 2^(A_i + B_c): every output with
// S_ic >= 2^-80 is exact (terms lost below fp32's normal range are then below
// 2^-30 S_ic). A launch where some output fails the check raises a flag, and
// the element-wise kernels recompute the whole aggregation.
typedef __bf16 bf16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
// x = hi + lo to ~2^-16 relative; x is made opaque so that both halves are
// formed from the same fp32 value
__device__ __forceinline__ void split_bf16(float x, bf16& hi, bf16& lo) {
  asm("" : "+v"(x));
  hi = (bf16)x;
  lo = (bf16)(x - (float)hi);
}
constexpr float kProductFloor = 0x1p-80f;

// Per (head, value column): max and min of V over the head's keys (the
// column reference B_c is kw max V for kw > 0, kw min V for kw < 0). One wave
// per column. Block 0 also clears the fallback flag of this call.
__global__ __launch_bounds__(256) void soft_colext_kernel(const f16* __restrict__ vt, const uint8_t* __restrict__ vlo,
                                                          float* __restrict__ vmax, float* __restrict__ vmin,
                                                          int* __restrict__ flag, int N, int NP, int DV, int ncol) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *flag = 0;
  const int col = blockIdx.x * 4 + (int)(threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (col >= ncol) return;
  const int bh = col / DV, c = col - bh * DV;
  float hi = kNegInf, lo = -kNegInf;
  for (int k0 = 8 * lane; k0 < N; k0 += 512) {  // 8 keys per lane and pass
    float v[8];
    load_values8(vt, vlo, bh, DV, NP, c, k0, v);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (k0 + j < N) {
        hi = fmaxf(hi, v[j]);
        lo = fminf(lo, v[j]);
      }
  }
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) {
    hi = fmaxf(hi, __shfl_xor(hi, sh));
    lo = fminf(lo, __shfl_xor(lo, sh));
  }
  if (lane == 0) {
    vmax[col] = hi;
    vmin[col] = lo;
  }
}

hipError_t launch_soft_colext(const Dims& d, const ProjBuffers& p, const SoftState& st, hipStream_t s) {
  const int ncol = d.B * d.H * d.DV;
  MORPHO_KLAUNCH(soft_colext_kernel, dim3((unsigned)((ncol + 3) / 4)), dim3(256), 0, s, p.vt, p.vlo, st.vmax,
                     st.vmin, st.flag, d.N, d.NP, d.DV, ncol);
  return hipGetLastError();
}

// F^T = 2^(w - B_c) of every (head, column, key) as bf16 hi / lo pairs,
// [B*H, DV, NP] with keys contiguous: the tiles every query block of the
// product-form forward reads. One thread per 8 keys of a column.
__global__ __launch_bounds__(256) void soft_fvals_kernel(const f16* __restrict__ vt, const uint8_t* __restrict__ vlo,
                                                         const float* __restrict__ tau_p, SoftState st, int N, int NP,
                                                         int DV, int64_t nchunks, float sgn) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nchunks) return;
  const int64_t col = i / (NP / 8);  // bh * DV + c
  const int k0 = 8 * (int)(i - col * (NP / 8));
  const int bh = (int)(col / DV), c = (int)(col - (int64_t)bh * DV);
  const float kw = sgn * kLog2e / *tau_p;
  const float bc = kw * (kw > 0.f ? st.vmax[col] : st.vmin[col]);
  bf16x8 hi, lo;
  float v[8];
  load_values8(vt, vlo, bh, DV, NP, c, k0, v);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float ev = fast_exp2(kw * v[j] - bc);
    const float f = k0 + j < N ? ev : 0.f;
    bf16 h, l;
    split_bf16(f, h, l);
    hi[j] = h;
    lo[j] = l;
  }
  *reinterpret_cast<bf16x8*>(st.fth + col * NP + k0) = hi;
  *reinterpret_cast<bf16x8*>(st.ftl + col * NP + k0) = lo;
}

hipError_t launch_soft_fvals(const Dims& d, const ProjBuffers& p, const float* tau, int sgn, const SoftState& st,
                             hipStream_t s) {
  const int64_t n = (int64_t)d.B * d.H * d.DV * (d.NP / 8);
  MORPHO_KLAUNCH(soft_fvals_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p.vt, p.vlo, tau, st, d.N,
                     d.NP, d.DV, n, (float)sgn);
  return hipGetLastError();
}

template <int M, int DV>
struct FastCfg {
  static constexpr int CW = 2 * M + 8;
  static constexpr int NCH = M / 8;
  static constexpr int QW = 128;   // 4 waves x 32 queries
  static constexpr int FS = 40;    // bf16 row stride of the F^T tiles (32 keys + 8: conflict-free b128 reads)
  static constexpr int CB = DV / 32;
};

// Forward, product form. Wave = 32 queries x all DV columns (O^T accumulators:
// rows = value column, lane = query). Per 32-key block: the S^T block from the
// code rows, loaded in swap23 key order so that the accumulator holds each
// lane's keys 8 h32 + 0..7 and 16 + 8 h32 + 0..7 in order (the B-operand
// layout of the next product); E = 2^(u - A_i) with A_i the running maximum
// (the accumulators are rescaled when it grows); O^T += F^T E in three bf16
// MFMAs per 16 keys (hi.hi, hi.lo, lo.hi). F^T of the block is staged by the
// whole workgroup into double-buffered LDS tiles.
template <int M, int DV, bool MD>
__global__ __launch_bounds__(256) void soft_fwd_fast_kernel(const f16* __restrict__ qa, const f16* __restrict__ ka,
                                                            const f16* __restrict__ vt,
                                                            const uint8_t* __restrict__ vlo,
                                                            const float4* __restrict__ tstat,
                                                            const float* __restrict__ tau_p, SoftState st,
                                                            f16* __restrict__ out, float* __restrict__ zb, int N,
                                                            int NP, int H, int D, int BH, int causal, float sgn) {
  using C = FastCfg<M, DV>;
  __shared__ __align__(16) bf16 sfh[2][DV * C::FS];
  __shared__ __align__(16) bf16 sfl[2][DV * C::FS];
  __shared__ float sbc[DV];
  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nqb = (N + C::QW - 1) / C::QW;
  int bh, blk;
  if (!(causal ? xcd_map_lpt(nqb, BH, bh, blk) : xcd_map(nqb, BH, bh, blk))) return;
  const int qblk = causal ? nqb - 1 - blk : blk;
  const int q0 = qblk * C::QW, qw0 = q0 + 32 * w;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N;
  const float tau = *tau_p;
  const float ks = sgn / tau, kw = sgn * kLog2e / tau;
  for (int c = tid; c < DV; c += 256) sbc[c] = kw * (kw > 0.f ? st.vmax[bh * DV + c] : st.vmin[bh * DV + c]);

  const int q = qw0 + l32;
  f16x8 qf[C::NCH];
  f16x4 qaug = {};
#pragma unroll
  for (int c = 0; c < C::NCH; ++c) qf[c] = f16x8{};
  if (q < N) load_query_operand<M>(qa + (rowbase + q) * C::CW, tstat[rowbase + q].x, h32, qf, qaug);
  f32x16 o[C::CB];
#pragma unroll
  for (int i = 0; i < C::CB; ++i) o[i] = f32x16{};
  float mrow = kNegInf;  // running maximum of u over this query's keys so far

  const int kend = causal ? min(N, q0 + C::QW) : N;
  const int nkb = (kend + 31) / 32;
  // F^T tile of keys 32 kb .. + 31: 16-byte pieces of the precomputed rows
  const bf16* fth = reinterpret_cast<const bf16*>(st.fth) + (int64_t)bh * DV * NP;
  const bf16* ftl = reinterpret_cast<const bf16*>(st.ftl) + (int64_t)bh * DV * NP;
  auto stage = [&](int kb, bf16* fh, bf16* fl) {
    for (int e = tid; e < 4 * DV; e += 256) {
      const int c = e >> 2, q4 = e & 3;
      const int64_t src = (int64_t)c * NP + 32 * kb + 8 * q4;
      *reinterpret_cast<bf16x8*>(fh + c * C::FS + 8 * q4) = *reinterpret_cast<const bf16x8*>(fth + src);
      *reinterpret_cast<bf16x8*>(fl + c * C::FS + 8 * q4) = *reinterpret_cast<const bf16x8*>(ftl + src);
    }
  };
  __syncthreads();  // sbc
  if (nkb > 0) stage(0, sfh[0], sfl[0]);
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const bf16* fh = sfh[kb & 1];
    const bf16* fl = sfl[kb & 1];
    if (kb + 1 < nkb) stage(kb + 1, sfh[(kb + 1) & 1], sfl[(kb + 1) & 1]);
    const int key0 = 32 * kb, krow = key0 + swap23(l32);
    f16x8 kf[C::NCH];
    f16x4 kaug = {};
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) kf[c] = f16x8{};
    if (krow < N) load_key_operand<M>(ka + (rowbase + krow) * C::CW, h32, kf, kaug);
    f32x16 acc = code_dot<M, true>(kf, qf, f32x16{});
    acc = mfma8(kaug, qaug, acc);
    float u[16], tm = kNegInf;
    // wave-uniform: only blocks with ragged keys, keys after some query or the
    // diagonal need the per-score mask
    const bool need_mask = (key0 + 32 > N) || (causal != 0 && key0 + 31 > qw0) ||
                           (MD && key0 <= qw0 + 31 && key0 + 31 >= qw0);
    if (need_mask) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = key0 + (r < 8 ? 8 * h32 + r : 8 + 8 * h32 + r);
        const bool drop = (key >= N) | (causal != 0 && key > q) | (MD && key == q);
        u[r] = drop ? kNegInf : ks * acc[r];
        tm = fmaxf(tm, u[r]);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        u[r] = ks * acc[r];
        tm = fmaxf(tm, u[r]);
      }
    }
    tm = fmaxf(tm, __shfl_xor(tm, 32));
    const float mn = fmaxf(mrow, tm);
    const float ref = mn == kNegInf ? 0.f : mn;
    if (__builtin_amdgcn_ballot_w64(mn > mrow) != 0) {  // some query's maximum grew: rescale its sums
      const float sc = fast_exp2(mrow - ref);
#pragma unroll
      for (int i = 0; i < C::CB; ++i) o[i] *= sc;
    }
    mrow = mn;
    bf16x8 eh[2], el[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      bf16 hi, lo;
      split_bf16(fast_exp2(u[r] - ref), hi, lo);
      eh[r >> 3][r & 7] = hi;
      el[r >> 3][r & 7] = lo;
    }
#pragma unroll
    for (int cb = 0; cb < C::CB; ++cb) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const int off = (32 * cb + l32) * C::FS + 16 * kc + 8 * h32;
        const bf16x8 ah = *reinterpret_cast<const bf16x8*>(fh + off);
        const bf16x8 al = *reinterpret_cast<const bf16x8*>(fl + off);
        o[cb] = mfma_bf16(ah, eh[kc], o[cb]);
        o[cb] = mfma_bf16(ah, el[kc], o[cb]);
        o[cb] = mfma_bf16(al, eh[kc], o[cb]);
      }
    }
    __syncthreads();
  }

  // zb = A_i + B_c + log2 S_ic; out = sgn tau ln2 zb
  bool low = false;
  if (q < N) {
    const float ko = sgn * tau * kLn2;
    f16* orow = out + ((int64_t)b * N + q) * D + h * DV;
    float* zrow = zb + (rowbase + q) * DV;
#pragma unroll
    for (int cb = 0; cb < C::CB; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float4 z4;
        f16x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 32 * cb + 8 * g + 4 * h32 + e;
          const float sv = o[cb][4 * g + e];
          float z = -kFltMax;
          if (mrow > kNegInf) {
            low = low || !(sv >= kProductFloor);
            z = mrow + sbc[c] + fast_log2(sv);
          }
          (&z4.x)[e] = z;
          o4[e] = (f16)(mrow > kNegInf ? ko * z : 0.f);
        }
        *reinterpret_cast<float4*>(zrow + 32 * cb + 8 * g + 4 * h32) = z4;
        *reinterpret_cast<f16x4*>(orow + 32 * cb + 8 * g + 4 * h32) = o4;
      }
    if (h32 == 0) st.arow[rowbase + q] = mrow;
  }
  if (__builtin_amdgcn_ballot_w64(low) != 0 && lane == 0) atomicOr(st.flag, 1);
}

template <int M, int DV>
static hipError_t launch_soft_fwd_fast_t(const Dims& d, const ProjBuffers& p, const float* tau, int sgn,
                                         const SoftState& st, f16* out, float* zb, hipStream_t s) {
  using C = FastCfg<M, DV>;
  const dim3 grid(xcd_grid((d.N + C::QW - 1) / C::QW, d.B * d.H));
  if (d.mask_diag)
    MORPHO_KLAUNCH((soft_fwd_fast_kernel<M, DV, true>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.vlo, p.tstat,
                       tau, st, out, zb, d.N, d.NP, d.H, d.D, d.B * d.H, d.causal, (float)sgn);
  else
    MORPHO_KLAUNCH((soft_fwd_fast_kernel<M, DV, false>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.vlo, p.tstat,
                       tau, st, out, zb, d.N, d.NP, d.H, d.D, d.B * d.H, d.causal, (float)sgn);
  return hipGetLastError();
}

hipError_t launch_soft_fwd_fast(const Dims& d, const ProjBuffers& p, const float* tau, int sgn, const SoftState& st,
                                f16* out, float* zb, hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_soft_fwd_fast_t, d, p, tau, sgn, st, out, zb, s);
}

// ============================================================ backward prep
// Per (head, token) row: dcb = sum_c dO_ic (the row sum of ds, for a row with
// keys), the partial sum of dO . zb for dtau, and the zeroed dq accumulator.
// DV / 8 consecutive lanes share a row, 8 columns each.
template <int DV>
__global__ __launch_bounds__(256) void soft_bwd_prep_kernel(const f16* __restrict__ grad_out,
                                                            const float* __restrict__ zb, float* __restrict__ dcb,
                                                            float* __restrict__ dq, float* __restrict__ part,
                                                            int64_t T, int N, int H, int D, int M,
                                                            const float* __restrict__ tau_p, float sgn,
                                                            const float* __restrict__ vmax,
                                                            const float* __restrict__ vmin,
                                                            const float* __restrict__ arow, bf16* __restrict__ gh,
                                                            bf16* __restrict__ gl) {
  constexpr int G = DV / 8;
  __shared__ float red[4];
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t bhn = idx / G;
  float rs = 0.f, dz = 0.f;
  bool live = false;
  if (idx < T * (D / 8)) {
    const int64_t bh = bhn / N;
    const int n = (int)(bhn - bh * N), b = (int)(bh / H), h = (int)(bh - (int64_t)b * H);
    const int c = 8 * (int)(idx & (G - 1));
    const f16x8 g = *reinterpret_cast<const f16x8*>(grad_out + ((int64_t)b * N + n) * D + h * DV + c);
    const float4 z0 = *reinterpret_cast<const float4*>(zb + bhn * DV + c);
    const float4 z1 = *reinterpret_cast<const float4*>(zb + bhn * DV + c + 4);
    const float z[8] = {z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
    live = z[0] > -kFltMax;  // every column of a row with keys is finite
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      rs += (float)g[e];
      dz += (float)g[e] * z[e];
    }
    if (!live) rs = dz = 0.f;
    if (gh) {  // G = dO 2^(A_i + B_c - zb) for the product-form backward (0 for a row without keys)
      const float kw = sgn * kLog2e / *tau_p;
      const float a = arow[bhn];
      // the 8 columns' extremes (max for dilation, min for erosion) in two 16-byte loads
      const float* ext = (kw > 0.f ? vmax : vmin) + bh * DV + c;
      const float4 x0 = *reinterpret_cast<const float4*>(ext), x1 = *reinterpret_cast<const float4*>(ext + 4);
      const float xc[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float bc = kw * xc[e];
        const float gv = (live && a > kNegInf) ? (float)g[e] * fast_exp2(a + bc - z[e]) : 0.f;
        bf16 h, l;
        split_bf16(gv, h, l);
        hi[e] = h;
        lo[e] = l;
      }
      *reinterpret_cast<bf16x8*>(gh + bhn * DV + c) = hi;
      *reinterpret_cast<bf16x8*>(gl + bhn * DV + c) = lo;
    }
  }
#pragma unroll
  for (int sh = 1; sh < G; sh <<= 1) rs += __shfl_xor(rs, sh);
  if (idx < T * (D / 8) && (threadIdx.x & (G - 1)) == 0) dcb[bhn] = rs;
  // block partial of dO . zb in a fixed order
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) dz += __shfl_xor(dz, sh);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = dz;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
  float4* zq = reinterpret_cast<float4*>(dq);
  const int64_t nz = T * H * (M / 4);
  for (int64_t i = idx; i < nz; i += (int64_t)gridDim.x * 256) zq[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

int soft_prep_blocks(const Dims& d) { return (int)((d.T * (d.D / 8) + 255) / 256); }

template <int M, int DV>
static hipError_t launch_soft_bwd_prep_t(const Dims& d, const f16* grad_out, const float* zb, const BwdBuffers& g,
                                         float* part, const float* tau, int sgn, const SoftState* st, uint16_t* gh,
                                         uint16_t* gl, hipStream_t s) {
  MORPHO_KLAUNCH((soft_bwd_prep_kernel<DV>), dim3((unsigned)soft_prep_blocks(d)), dim3(256), 0, s, grad_out, zb,
                     g.dcb, g.dq, part, d.T, d.N, d.H, d.D, d.M, tau, (float)sgn, st ? st->vmax : nullptr,
                     st ? st->vmin : nullptr, st ? st->arow : nullptr, st ? reinterpret_cast<bf16*>(gh) : nullptr,
                     st ? reinterpret_cast<bf16*>(gl) : nullptr);
  return hipGetLastError();
}

hipError_t launch_soft_bwd_prep(const Dims& d, const f16* grad_out, const float* zb, const BwdBuffers& g, float* part,
                                const float* tau, int sgn, const SoftState* st, uint16_t* gh, uint16_t* gl,
                                hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_soft_bwd_prep_t, d, grad_out, zb, g, part, tau, sgn, st, gh, gl, s);
}

// ============================================================ backward
// Workgroup: KB blocks of 32 keys x CG groups of 32 value columns, one wave
// each; lane = key. Per 32-query step the workgroup stages -zb and dO of the
// step's queries (fp32 [QT][DV]) and their phi (fp32 [QT][M]); each wave
// recomputes its S block, accumulates dV and its partial ds over its value
// columns, and stores the partial ds in LDS; then all threads form
// dk, dcb += ds^T phi_q (key side, registers) and dq = ds phi_k (query side,
// fp32 atomics) from the summed partials.
template <int M, int DV, bool MD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void soft_bwd_kernel(const f16* __restrict__ qa, const f16* __restrict__ ka,
                                                       const f16* __restrict__ vt, const uint8_t* __restrict__ vlo,
                                                       const float4* __restrict__ tstat, const float* __restrict__ tau_p,
                                                       const f16* __restrict__ grad_out, const float* __restrict__ zb,
                                                       float* __restrict__ dq, float* __restrict__ dk,
                                                       float* __restrict__ dcb, f16* __restrict__ dzv,
                                                       float* __restrict__ part, int N, int NP, int H, int D, int HM,
                                                       int BH, int causal, float sgn, const int* __restrict__ run_flag) {
  using C = SoftCfg<M, DV>;
  constexpr int NG = 256 / C::KW;   // dk phase: thread groups per key
  constexpr int CPT = M / NG;       // dk phase: codes per thread
  constexpr int CPQ = M / 8;        // dq phase: codes per thread (8 groups per query)
  __shared__ __align__(16) float snz[C::QT * C::WS];     // -zb of the step's queries
  __shared__ __align__(16) float sdo[C::QT * C::WS];     // dO of the step's queries
  __shared__ __align__(16) float sphq[C::QT * C::PS];    // phi of the step's queries
  __shared__ __align__(16) float sphk[C::KW * C::PS];    // phi of the workgroup's keys
  __shared__ __align__(16) float sds[C::CG][C::QT * C::DS];  // partial ds per column group: [query][key]
  __shared__ __align__(16) float swv[C::KW * C::WS];         // scaled values of the workgroup's keys
  __shared__ float red[2][4];

  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkb = (N + C::KW - 1) / C::KW;
  int bh, kblk;
  if ((run_flag && *run_flag == 0) || !(causal ? xcd_map_lpt(nkb, BH, bh, kblk) : xcd_map(nkb, BH, bh, kblk))) {
    if (tid == 0) {
      part[2 * blockIdx.x] = 0.f;
      part[2 * blockIdx.x + 1] = 0.f;
    }
    return;
  }
  const int k0 = kblk * C::KW, kb = w % C::KB, cg = w / C::KB;
  const int kw0 = k0 + 32 * kb, c0 = 32 * cg;
  const int key = kw0 + l32;
  const bool kvalid = key < N;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N, tokbase = (int64_t)b * N;
  const float tau = *tau_p;
  const float ks = sgn / tau, kw = sgn * kLog2e / tau;

  // key operand and this lane's scaled values (fixed for the whole kernel)
  f16x8 kf[C::NCH];
  f16x4 kaug = {};
#pragma unroll
  for (int c = 0; c < C::NCH; ++c) kf[c] = f16x8{};
  float dv[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) dv[c] = 0.f;
  if (kvalid) load_key_operand<M>(ka + (rowbase + key) * C::CW, h32, kf, kaug);
  // scaled values of the workgroup's keys, [key][column] (zero past N); each
  // lane reads its own key's row, four columns at a time
  for (int e = tid; e < C::KW * DV; e += 256) {
    const int r = e / DV, c = e % DV, kk = k0 + r;
    swv[r * C::WS + c] = kk < N ? kw * load_value(vt, vlo, bh, DV, NP, c, kk) : 0.f;
  }
  const float* wrow = swv + (32 * kb + l32) * C::WS + c0;
  // phi of the workgroup's keys (zero past N)
  for (int e = tid; e < C::KW * M; e += 256) {
    const int r = e / M, c = e % M, kk = k0 + r;
    float v = 0.f;
    if (kk < N) {
      const f16* row = qa + (rowbase + kk) * C::CW;
      v = (float)row[c] + (float)row[M + 8 + c];
    }
    sphk[r * C::PS + c] = v;
  }

  float dka[CPT], dcba = 0.f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) dka[i] = 0.f;
  float st = 0.f;  // sum ds * acc (acc = log2e s)

  const int qstart = causal ? k0 : 0;
  for (int qs = qstart; qs < N; qs += C::QT) {
    // ---- stage -zb, dO and phi of queries qs .. qs + QT - 1 (zero past N)
    for (int e = tid; e < C::QT * DV; e += 256) {
      const int r = e / DV, c = e % DV, qq = qs + r;
      float nz = 0.f, g = 0.f;
      if (qq < N) {
        nz = -zb[(rowbase + qq) * DV + c];
        g = (float)grad_out[(tokbase + qq) * D + h * DV + c];
      }
      snz[r * C::WS + c] = nz;
      sdo[r * C::WS + c] = g;
    }
    for (int e = tid; e < C::QT * M; e += 256) {
      const int r = e / M, c = e % M, qq = qs + r;
      float v = 0.f;
      if (qq < N) {
        const f16* row = qa + (rowbase + qq) * C::CW;
        v = (float)row[c] + (float)row[M + 8 + c];
      }
      sphq[r * C::PS + c] = v;
    }
    // ---- S block: rows = queries qs + acc_row(r), column = this lane's key
    f16x8 qf[C::NCH];
    f16x4 qaug = {};
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) qf[c] = f16x8{};
    if (qs + l32 < N) load_query_operand<M>(qa + (rowbase + qs + l32) * C::CW, tstat[rowbase + qs + l32].x, h32, qf,
                                            qaug);
    f32x16 acc = code_dot<M, false>(kf, qf, f32x16{});
    acc = mfma8(qaug, kaug, acc);
    float u[16], ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qq = qs + acc_row(r, lane);
      const bool drop = (qq >= N) | !kvalid | (causal != 0 && key > qq) | (MD && key == qq);
      u[r] = drop ? kNegInf : ks * acc[r];
      ds[r] = 0.f;
    }
    __syncthreads();  // staging complete
    // ---- P = 2^(y - zb); ds_ij += dO P over this wave's columns; dV_jc += dO P
#pragma unroll
    for (int c4 = 0; c4 < 8; ++c4) {
      const float4 w4 = *reinterpret_cast<const float4*>(wrow + 4 * c4);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int qr = acc_row(r, lane);
        const float4 n4 = *reinterpret_cast<const float4*>(snz + qr * C::WS + c0 + 4 * c4);
        const float4 g4 = *reinterpret_cast<const float4*>(sdo + qr * C::WS + c0 + 4 * c4);
        const float p0 = fast_exp2(u[r] + w4.x + n4.x);
        const float p1 = fast_exp2(u[r] + w4.y + n4.y);
        const float p2 = fast_exp2(u[r] + w4.z + n4.z);
        const float p3 = fast_exp2(u[r] + w4.w + n4.w);
        ds[r] = fmaf(p0, g4.x, ds[r]);
        ds[r] = fmaf(p1, g4.y, ds[r]);
        ds[r] = fmaf(p2, g4.z, ds[r]);
        ds[r] = fmaf(p3, g4.w, ds[r]);
        dv[4 * c4 + 0] = fmaf(p0, g4.x, dv[4 * c4 + 0]);
        dv[4 * c4 + 1] = fmaf(p1, g4.y, dv[4 * c4 + 1]);
        dv[4 * c4 + 2] = fmaf(p2, g4.z, dv[4 * c4 + 2]);
        dv[4 * c4 + 3] = fmaf(p3, g4.w, dv[4 * c4 + 3]);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      st = fmaf(ds[r], acc[r], st);  // ds is 0 wherever the score is masked
      sds[cg][acc_row(r, lane) * C::DS + 32 * kb + l32] = ds[r];
    }
    __syncthreads();  // every partial ds of the step is in LDS
    // ---- key side: dk_j += sum_i ds_ij phi_i, dcb_j += sum_i ds_ij
    {
      const int kk = tid % C::KW, grp = tid / C::KW;
#pragma unroll 4
      for (int i = 0; i < C::QT; ++i) {
        float dsv = 0.f;
#pragma unroll
        for (int g = 0; g < C::CG; ++g) dsv += sds[g][i * C::DS + kk];
        const float* ph = sphq + i * C::PS + grp * CPT;
#pragma unroll
        for (int c = 0; c < CPT; ++c) dka[c] = fmaf(dsv, ph[c], dka[c]);
        dcba += dsv;
      }
    }
    // ---- query side: dq_i += sum_j ds_ij phi_j (fp32 atomics)
    {
      const int i = tid % C::QT, grp = tid / C::QT;
      float dqa[CPQ];
#pragma unroll
      for (int c = 0; c < CPQ; ++c) dqa[c] = 0.f;
#pragma unroll 4
      for (int kk = 0; kk < C::KW; ++kk) {
        float dsv = 0.f;
#pragma unroll
        for (int g = 0; g < C::CG; ++g) dsv += sds[g][i * C::DS + kk];
        const float* ph = sphk + kk * C::PS + grp * CPQ;
#pragma unroll
        for (int c = 0; c < CPQ; ++c) dqa[c] = fmaf(dsv, ph[c], dqa[c]);
      }
      if (qs + i < N) {
#pragma unroll
        for (int c = 0; c < CPQ; ++c) unsafeAtomicAdd(dq + (rowbase + qs + i) * M + grp * CPQ + c, dqa[c]);
      }
    }
    __syncthreads();  // LDS tiles are free for the next step
  }

  // ---- epilogue
  // dV: the two half-waves hold the same key (different queries)
  float sv = 0.f;  // sum dV * w over the columns this lane writes
#pragma unroll
  for (int c = 0; c < 32; ++c) dv[c] += __shfl_xor(dv[c], 32);
  if (kvalid) {
    f16* drow = dzv + (tokbase + key) * (int64_t)(HM + D) + HM + h * DV + c0 + 16 * h32;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = h32 ? dv[16 + 8 * g + e] : dv[8 * g + e];
        const float wc = wrow[16 * h32 + 8 * g + e];
        o[e] = (f16)v;
        sv = fmaf(v, wc, sv);
      }
      *reinterpret_cast<f16x8*>(drow + 8 * g) = o;
    }
  }
  {
    const int kk = tid % C::KW, grp = tid / C::KW;
    if (k0 + kk < N) {
#pragma unroll
      for (int c = 0; c < CPT; ++c) dk[(rowbase + k0 + kk) * M + grp * CPT + c] = dka[c];
      if (grp == 0) dcb[rowbase + k0 + kk] += dcba;  // the prep wrote the row sum
    }
  }
  // dtau partials of the workgroup in a fixed order
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) {
    st += __shfl_xor(st, sh);
    sv += __shfl_xor(sv, sh);
  }
  if (lane == 0) {
    red[0][w] = st;
    red[1][w] = sv;
  }
  __syncthreads();
  if (tid == 0) {
    part[2 * blockIdx.x] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    part[2 * blockIdx.x + 1] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  }
}

template <int M, int DV>
static int soft_bwd_slots_t(const Dims& d) {
  return (int)xcd_grid((d.N + SoftCfg<M, DV>::KW - 1) / SoftCfg<M, DV>::KW, d.B * d.H);
}
// slots of the element-wise backward, then of the product-form backward
// (128 keys per workgroup)
int soft_bwd_slots(const Dims& d) {
  return (int)xcd_grid((d.N + 32 * (128 / d.DV) - 1) / (32 * (128 / d.DV)), d.B * d.H) +
         (int)xcd_grid((d.N + 127) / 128, d.B * d.H);
}

template <int M, int DV>
static hipError_t launch_soft_bwd_t(const Dims& d, const ProjBuffers& p, const f16* grad_out, const float* zb,
                                    const float* tau, int sgn, const BwdBuffers& g, float* part, const int* run_flag,
                                    hipStream_t s) {
  const dim3 grid((unsigned)soft_bwd_slots_t<M, DV>(d));
  if (d.mask_diag)
    MORPHO_KLAUNCH((soft_bwd_kernel<M, DV, true>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.vlo, p.tstat, tau,
                       grad_out, zb, g.dq, g.dk, g.dcb, g.dzv, part, d.N, d.NP, d.H, d.D, d.HM, d.B * d.H, d.causal,
                       (float)sgn, run_flag);
  else
    MORPHO_KLAUNCH((soft_bwd_kernel<M, DV, false>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.vlo, p.tstat, tau,
                       grad_out, zb, g.dq, g.dk, g.dcb, g.dzv, part, d.N, d.NP, d.H, d.D, d.HM, d.B * d.H, d.causal,
                       (float)sgn, run_flag);
  return hipGetLastError();
}

hipError_t launch_soft_bwd(const Dims& d, const ProjBuffers& p, const f16* grad_out, const float* zb,
                           const float* tau, int sgn, const BwdBuffers& g, float* part, const int* run_flag,
                           hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_soft_bwd_t, d, p, grad_out, zb, tau, sgn, g, part, run_flag, s);
}

// two waves per SIMD where the registers allow it without spilling
template <int M, int DV>
constexpr int soft_fast_bwd_waves() { return (M == 16 && DV <= 64) ? 2 : 1; }

// Backward, product form. With G_ic = dO_ic 2^(A_i + B_c - zb_ic) = dO_ic / S_ic:
//     ds_ij = E_ij sum_c G_ic F_jc          (X = G F^T, then times E)
//     dV_jc = F_jc sum_i E_ij G_ic          (dV^T = G^T E, then times F)
// Workgroup: 4 waves x 32 keys, lane = key; each 32-query step's tiles (the
// queries' code rows, G in bf16 hi / lo [query][column], the row references
// A_i and token biases) arrive by LDS DMA one step ahead, into the other of
// two stages; the code rows' affine block begins with a 1 after the codes, so
// they also serve as [phi_hi | 1] (the ones column at code M).
// The S block is read in swap23 query order so that E and ds are already
// B operands of the products that contract over the queries: dV^T += G^T E,
// and [dk | dcb]^T += [phi_hi | 1]^T ds (one fp16 MFMA per 16 queries; the
// ones column gives dcb). dq_i = sum_j ds_ij phi_hi_j contracts over the keys:
// every lane stores its key's fp16 ds row (the step's 32 queries) into a
// dS^T tile, and the step's 16 x 16 (query, code) dq tiles, split over the
// waves, each contract over all 128 keys of the workgroup: the A operand is
// read from the tile with transposing reads, phi_hi of the workgroup's keys
// is the B operand (registers), and each result element is one fp32 atomic
// per (query, code). The code-gradient products take
// ds rounded once to fp16 and the fp16 hi codes, as the softmax backward does
// (|ds_ij| <= sum_c |dO_ic|, well inside fp16's range): relative error ~2^-11
// per term, against the 1e-2 bar. (Three MFMAs of hi/lo pairs each had been
// used here; the products of G, E and F keep their bf16 hi/lo pairs, whose
// range they need.)
template <int M, int DV, bool MD>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(soft_fast_bwd_waves<M, DV>(), soft_fast_bwd_waves<M, DV>()))) void soft_bwd_fast_kernel(
    const f16* __restrict__ qa, const f16* __restrict__ ka, const f16* __restrict__ vt,
    const uint8_t* __restrict__ vlo, const float4* __restrict__ tstat, const float* __restrict__ tau_p, SoftState st,
    const bf16* __restrict__ gh, const bf16* __restrict__ gl, float* __restrict__ dq, float* __restrict__ dk,
    float* __restrict__ dcb, f16* __restrict__ dzv, float* __restrict__ part, int N, int NP, int H, int D, int HM,
    int BH, int causal, float sgn) {
  constexpr int CW = 2 * M + 8, NCH = M / 8, CB = DV / 32, KW = 128, QT = 32;
  constexpr int GS = DV + 8;            // bf16 row stride of the G tiles
  constexpr int MB = (M + 32) / 32;     // 32-code blocks of [phi | 1]
  constexpr int SRB = 2 * QT;           // dS^T row bytes (one key's ds over the step's queries)
  constexpr int DQTILES = (QT / 16) * (M / 16);  // 16 x 16 dq tiles of a step
  constexpr int DQT = DQTILES >= 4 ? DQTILES / 4 : 1;  // per wave (m = 16: waves 0, 1 only)
  static_assert(DQTILES < 4 || DQTILES % 4 == 0, "dq tiles must split evenly over the waves");
  // Per-step tiles, two stages filled by LDS DMA (16 bytes per lane, 1 KiB
  // pieces): the step's query code rows [QT][CW] (fp16: the score operand,
  // and with the affine block's leading 1 after the codes also [phi_hi | 1]
  // for dk and dcb), G hi and lo [QT][GS] (bf16; the last 16-byte chunk of a
  // row is padding), then A_i and the token bias b_i of the QT rows (fp32,
  // 4 bytes per lane). Rows past N load row N - 1: finite values whose every
  // score is masked.
  constexpr int QCH = CW / 8, GCH = GS / 8;        // 16-byte chunks per code row, per G row
  constexpr int NQP = (QT * QCH + 63) / 64;         // pieces of the code tile
  constexpr int NGP = (QT * GCH + 63) / 64;         // pieces of each G tile
  constexpr int NPC = NQP + 2 * NGP;
  constexpr int OGH = NQP * 1024, OGL = OGH + NGP * 1024, OAB = OGL + NGP * 1024;
  constexpr int STG = OAB + 256;                    // stage bytes
  __shared__ __align__(16) char stg[2 * STG];
  __shared__ __align__(16) char sdt[KW * SRB];  // dS^T of the step: row = key, chunks swizzled by sswz
  __shared__ float sbc[DV];
  __shared__ float red[2][4];

  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkb = (N + KW - 1) / KW;
  int bh, kblk;
  if (*st.flag != 0 || !(causal ? xcd_map_lpt(nkb, BH, bh, kblk) : xcd_map(nkb, BH, bh, kblk))) {
    if (tid == 0) {
      part[2 * blockIdx.x] = 0.f;
      part[2 * blockIdx.x + 1] = 0.f;
    }
    return;
  }
  const int k0 = kblk * KW, kw0 = k0 + 32 * w, key = kw0 + l32;
  const bool kvalid = key < N;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N, tokbase = (int64_t)b * N;
  const float tau = *tau_p;
  const float ks = sgn / tau, kw = sgn * kLog2e / tau;
  for (int c = tid; c < DV; c += 256) sbc[c] = kw * (kw > 0.f ? st.vmax[bh * DV + c] : st.vmin[bh * DV + c]);
  __syncthreads();  // sbc

  // key operand; F of this lane's key as the B operand of G F^T (chunk cc:
  // columns 16 cc + 8 h32 + 0..7); phi of the wave's keys as the B operand of
  // ds phi (chunk kc: keys 16 kc + 8 h32 + 0..7, code 32 nb + l32)
  f16x8 kf[NCH];
  f16x4 kaug = {};
#pragma unroll
  for (int c = 0; c < NCH; ++c) kf[c] = f16x8{};
  bf16x8 fh[DV / 16], fl[DV / 16];
#pragma unroll
  for (int cc = 0; cc < DV / 16; ++cc)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int c = 16 * cc + 8 * h32 + j;
      const float f = kvalid ? fast_exp2(kw * load_value(vt, vlo, bh, DV, NP, c, key) - sbc[c]) : 0.f;
      bf16 hi, lo;
      split_bf16(f, hi, lo);
      fh[cc][j] = hi;
      fl[cc][j] = lo;
    }
  // dq tiles of this wave: tile w + 4 t = (query block qt, code block ct).
  // phi_hi of the workgroup's keys as their B operand (chunk kc: keys
  // k0 + 32 kc + 8 (lane / 16) + 0..7, code 16 ct + lane % 16; zero past N),
  // and the lane offsets of the transposing A-operand reads of the dS^T tile
  // (16 x 16 x 32 layout: query 16 qt + lane % 16, keys 8 (lane / 16) + j).
  const bool dq_wave = w < DQTILES;  // uniform
  f16x8 phib[DQT][KW / 32];
  int d_s[DQT][2];
#pragma unroll
  for (int t = 0; t < DQT; ++t) {
    const int tile = w + 4 * t, qt = tile % (QT / 16), ct = tile / (QT / 16);
#pragma unroll
    for (int kc = 0; kc < KW / 32; ++kc)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kk = k0 + 32 * kc + 8 * (lane >> 4) + j;
        phib[t][kc][j] = (dq_wave && kk < N) ? qa[(rowbase + kk) * CW + 16 * ct + (lane & 15)] : (f16)0.f;
      }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 8 * (lane >> 4) + ((lane & 15) >> 2) + 4 * hh, col = 16 * qt + 4 * (lane & 3);
      d_s[t][hh] = row * SRB + 16 * ((col >> 3) ^ sswz<SRB>(row)) + 2 * (col & 7);
    }
  }
  const int kr = 32 * w + l32, sz = sswz<SRB>(kr);  // this lane's dS^T row (its key)
  if (kvalid) load_key_operand<M>(ka + (rowbase + key) * CW, h32, kf, kaug);
  f32x16 dva[CB], dka[MB];
#pragma unroll
  for (int i = 0; i < CB; ++i) dva[i] = f32x16{};
#pragma unroll
  for (int i = 0; i < MB; ++i) dka[i] = f32x16{};
  float sacc = 0.f;

  // DMA of the tiles of the step at query qs into stage par: wave w issues
  // pieces w, w + 4, ... of the stage, and wave 3 the A / b piece.
  const unsigned sbase = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)stg;
  auto issue = [&](int qs, int par) {
    const unsigned dst = sbase + (unsigned)(par * STG);
    for (int i = w; i < NPC; i += 4) {  // wave-uniform
      if (i < NQP) {
        const int q = 64 * i + lane, r = min(q / QCH, QT - 1), c = q % QCH;
        lds_dma16(qa + (rowbase + min(qs + r, N - 1)) * CW + 8 * c, dst + 1024u * (unsigned)i);
      } else {
        const int j = i < NQP + NGP ? i - NQP : i - NQP - NGP;
        const int q = 64 * j + lane, r = min(q / GCH, QT - 1), c = min(q % GCH, DV / 8 - 1);
        const bf16* g = i < NQP + NGP ? gh : gl;
        lds_dma16(reinterpret_cast<const f16*>(g + (rowbase + min(qs + r, N - 1)) * DV + 8 * c),
                  dst + 1024u * (unsigned)i);
      }
    }
    if (w == 3) {
      const int r = min(qs + (lane & 31), N - 1);
      lds_dma4(lane < 32 ? st.arow + rowbase + r : reinterpret_cast<const float*>(tstat + rowbase + r),
               dst + (unsigned)OAB);
    }
  };
  // The key-side loads above are conditional; without a wait on every path
  // the compiler treats them as possibly pending inside the step loop and
  // waits for vmcnt there, which would also drain the next stage's DMA.
  wait_vmcnt<0>();

  const int qstart = causal ? k0 : 0;
  if (qstart < N) issue(qstart, 0);
  int par = 0;
  for (int qs = qstart; qs < N; qs += QT, par ^= 1) {
    // this step's stage has landed (the previous step's dq atomics, issued
    // after it, may still be in flight), for every wave after the barrier,
    // which also frees the other stage and the dS^T tile
    if (qs == qstart)
      wait_vmcnt_lgkm0<0>();
    else if (dq_wave)  // uniform
      wait_vmcnt_lgkm0<4 * DQT>();
    else
      wait_vmcnt_lgkm0<0>();
    __syncthreads();
    if (qs + QT < N) issue(qs + QT, par ^ 1);
    const char* sq = stg + par * STG;
    const bf16* sgh = reinterpret_cast<const bf16*>(sq + OGH);
    const bf16* sgl = reinterpret_cast<const bf16*>(sq + OGL);
    const float* sa_ = reinterpret_cast<const float*>(sq + OAB);
    const float* sb_ = sa_ + QT;
    // ---- S block, query rows in swap23 order: register r holds query p(r)
    f16x8 qf[NCH];
    f16x4 qaug;
    {
      const f16* qrow = reinterpret_cast<const f16*>(sq) + swap23(l32) * CW;
#pragma unroll
      for (int c = 0; c < NCH; ++c) qf[c] = *reinterpret_cast<const f16x8*>(qrow + chunk_off<M>(c) + 8 * h32);
      qaug = *reinterpret_cast<const f16x4*>(qrow + M + 4 * h32);
      if (h32 == 0) {  // the affine block {1, 1, b_hi, b_lo}: the accumulator is log2e s_ij
        f16 bh_, bl_;
        split_hi_lo(sb_[swap23(l32)], bh_, bl_);
        qaug[2] = bh_;
        qaug[3] = bl_;
      }
    }
    f32x16 acc = code_dot<M, false>(kf, qf, f32x16{});
    acc = mfma8(qaug, kaug, acc);
    // ---- E = 2^(u - A_i) (bf16 hi/lo, the B operand of G^T E); the per-score
    // mask only for blocks with ragged queries or keys, keys after some query
    // or the diagonal (wave-uniform)
    bf16x8 eh[2], el[2];
    float e32[16];
    const bool need_mask = (qs + 32 > N) || (kw0 + 32 > N) || (causal != 0 && kw0 + 31 > qs) ||
                           (MD && kw0 <= qs + 31 && kw0 + 31 >= qs);
    if (need_mask) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int p = r < 8 ? 8 * h32 + r : 8 + 8 * h32 + r;
        const int qq = qs + p;
        const bool drop = (qq >= N) | !kvalid | (causal != 0 && key > qq) | (MD && key == qq);
        // sa_[p] (p < 32) is read for every score and the result selected:
        // a read under the condition compiles to one divergent block, with
        // its own LDS wait, per score. A row without keys has A = -inf, and
        // every one of its scores is dropped here.
        const float ev = fast_exp2(ks * acc[r] - sa_[p]);
        e32[r] = drop ? 0.f : ev;
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) e32[r] = fast_exp2(ks * acc[r] - sa_[r < 8 ? 8 * h32 + r : 8 + 8 * h32 + r]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      bf16 hi, lo;
      split_bf16(e32[r], hi, lo);
      eh[r >> 3][r & 7] = hi;
      el[r >> 3][r & 7] = lo;
    }
    // ---- X = G F^T (rows = queries in the S block's order, lane = key)
    f32x16 x = {};
    const int grow = swap23(l32) * GS;
#pragma unroll
    for (int cc = 0; cc < DV / 16; ++cc) {
      const bf16x8 ah = *reinterpret_cast<const bf16x8*>(sgh + grow + 16 * cc + 8 * h32);
      const bf16x8 al = *reinterpret_cast<const bf16x8*>(sgl + grow + 16 * cc + 8 * h32);
      x = mfma_bf16(ah, fh[cc], x);
      x = mfma_bf16(ah, fl[cc], x);
      x = mfma_bf16(al, fh[cc], x);
    }
    // ---- dV^T += G^T E (rows = value columns, lane = key)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const bf16x8 ah = __builtin_bit_cast(bf16x8, frag_kmajor(reinterpret_cast<const f16*>(sgh), GS, 16 * kc, 32 * cb, lane));
        const bf16x8 al = __builtin_bit_cast(bf16x8, frag_kmajor(reinterpret_cast<const f16*>(sgl), GS, 16 * kc, 32 * cb, lane));
        dva[cb] = mfma_bf16(ah, eh[kc], dva[cb]);
        dva[cb] = mfma_bf16(ah, el[kc], dva[cb]);
        dva[cb] = mfma_bf16(al, eh[kc], dva[cb]);
      }
    // ---- ds = E X (fp16, the B operand of [phi_hi | 1]^T ds, and the dS^T row for dq)
    f16x8 dsh[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float dsv = e32[r] * x[r];
      sacc = fmaf(dsv, acc[r], sacc);
      dsh[r >> 3][r & 7] = (f16)dsv;
    }
    // one value per rounded ds for both of its readers (dk below, dq through
    // the dS^T copy): a conversion of the product selected twice could differ
    // at fp16 ties
    asm("" : "+v"(dsh[0]), "+v"(dsh[1]));
    // dS^T row of this key: queries 8 h32 + 0..7 and 16 + 8 h32 + 0..7 are
    // logical chunks h32 and 2 + h32
#pragma unroll
    for (int c = 0; c < 2; ++c) *reinterpret_cast<f16x8*>(sdt + kr * SRB + 16 * ((2 * c + h32) ^ sz)) = dsh[c];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) dka[mb] = mfma16(frag_kmajor(reinterpret_cast<const f16*>(sq), CW, 16 * kc, 32 * mb, lane), dsh[kc], dka[mb]);
    __syncthreads();  // the dS^T tile is complete
    // ---- dq of the step's queries over the workgroup's keys
    if (dq_wave) {
      typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
#pragma unroll
      for (int t = 0; t < DQT; ++t) {
        const int tile = w + 4 * t, qt = tile % (QT / 16), ct = tile / (QT / 16);
        f32x4 a = {};
#pragma unroll
        for (int kc = 0; kc < KW / 32; ++kc) {
          const char* base = sdt + 32 * kc * SRB;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + d_s[t][0]));
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + d_s[t][1]));
          a = mfma16x16(__builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7)),
                        phib[t][kc], a);
        }
        // rows: queries 16 qt + 4 (lane / 16) + r; column: code 16 ct + lane % 16.
        // Always issued (a fixed count per step: the stage waits count on
        // it); rows past N add 0 to row N - 1.
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int qq = qs + 16 * qt + 4 * (lane >> 4) + r;
          unsafeAtomicAdd(dq + (rowbase + min(qq, N - 1)) * M + 16 * ct + (lane & 15), qq < N ? a[r] : 0.f);
        }
      }
    }
  }

  // ---- epilogue: dV_jc = F_jc (G^T E)_cj; dk, dcb; sum dV * w for dtau
  float sv = 0.f;
  if (kvalid) {
    f16* drow = dzv + (tokbase + key) * (int64_t)(HM + D) + HM + h * DV;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = 32 * cb + 8 * g + 4 * h32 + e;
          const float wv = kw * load_value(vt, vlo, bh, DV, NP, c, key);
          const float v = fast_exp2(wv - sbc[c]) * dva[cb][4 * g + e];
          o[e] = (f16)v;
          sv = fmaf(v, wv, sv);
        }
        *reinterpret_cast<f16x4*>(drow + 32 * cb + 8 * g + 4 * h32) = o;
      }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int code = 32 * mb + acc_row(r, lane);
        if (code < M) dk[(rowbase + key) * M + code] = dka[mb][r];
        if (code == M) dcb[rowbase + key] += dka[mb][r];  // the prep wrote the row sum
      }
  }
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) {
    sacc += __shfl_xor(sacc, sh);
    sv += __shfl_xor(sv, sh);
  }
  if (lane == 0) {
    red[0][w] = sacc;
    red[1][w] = sv;
  }
  __syncthreads();
  if (tid == 0) {
    part[2 * blockIdx.x] = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    part[2 * blockIdx.x + 1] = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
  }
}

template <int M, int DV>
static hipError_t launch_soft_bwd_fast_t(const Dims& d, const ProjBuffers& p, const f16* grad_out, const float* zb,
                                         const float* tau, int sgn, const SoftState& st, const uint16_t* gh,
                                         const uint16_t* gl, const BwdBuffers& g, float* part, hipStream_t s) {
  (void)grad_out;
  (void)zb;
  const dim3 grid(xcd_grid((d.N + 127) / 128, d.B * d.H));
  const auto* h = reinterpret_cast<const bf16*>(gh);
  const auto* l = reinterpret_cast<const bf16*>(gl);
  if (d.mask_diag)
    MORPHO_KLAUNCH((soft_bwd_fast_kernel<M, DV, true>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.vlo, p.tstat,
                       tau, st, h, l, g.dq, g.dk, g.dcb, g.dzv, part, d.N, d.NP, d.H, d.D, d.HM, d.B * d.H,
                       d.causal, (float)sgn);
  else
    MORPHO_KLAUNCH((soft_bwd_fast_kernel<M, DV, false>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.vlo, p.tstat,
                       tau, st, h, l, g.dq, g.dk, g.dcb, g.dzv, part, d.N, d.NP, d.H, d.D, d.HM, d.B * d.H,
                       d.causal, (float)sgn);
  return hipGetLastError();
}

hipError_t launch_soft_bwd_fast(const Dims& d, const ProjBuffers& p, const f16* grad_out, const float* zb,
                                const float* tau, int sgn, const SoftState& st, const uint16_t* gh,
                                const uint16_t* gl, const BwdBuffers& g, float* part, hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_soft_bwd_fast_t, d, p, grad_out, zb, tau, sgn, st, gh, gl, g, part, s);
}
int soft_bwd_exact_slots(const Dims& d) {
  return (int)xcd_grid((d.N + 32 * (128 / d.DV) - 1) / (32 * (128 / d.DV)), d.B * d.H);
}

// Small fills (vector stores from a kernel, so that the sequence stays free of
// memset nodes when a caller captures it in a graph).
__global__ void fill_kernel(float* __restrict__ p, int n, float v) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}
hipError_t launch_fill_zero(float* p, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  MORPHO_KLAUNCH(fill_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n, 0.f);
  return hipGetLastError();
}
__global__ void flag_kernel(int* __restrict__ p, int v) { *p = v; }
hipError_t launch_set_flag(int* p, int v, hipStream_t s) {
  MORPHO_KLAUNCH(flag_kernel, dim3(1), dim3(1), 0, s, p, v);
  return hipGetLastError();
}

// ============================================================ dtau
// dtau = (sum dO out - sum ds s - sum dV V) / tau with out = sgn tau ln2 zb,
// s = ln2 acc and V = sgn tau ln2 w:
//     dtau = ln2 (sgn sum dO zb - (sum ds acc) / tau - sgn sum dV w).
// One workgroup; each thread sums a strided slice, then a fixed tree.
__global__ __launch_bounds__(256) void soft_tau_reduce_kernel(const float* __restrict__ prep, int nprep,
                                                              const float* __restrict__ bwd, int nbwd,
                                                              const float* __restrict__ tau_p, float sgn,
                                                              float* __restrict__ dtau) {
  __shared__ float red[3][256];
  float a = 0.f, s = 0.f, v = 0.f;
  // unrolled so that 8 loads are in flight; each thread still adds its
  // partials in index order, so the result does not depend on the unrolling
#pragma unroll 8
  for (int i = threadIdx.x; i < nprep; i += 256) a += prep[i];
#pragma unroll 8
  for (int i = threadIdx.x; i < nbwd; i += 256) {
    s += bwd[2 * i];
    v += bwd[2 * i + 1];
  }
  red[0][threadIdx.x] = a;
  red[1][threadIdx.x] = s;
  red[2][threadIdx.x] = v;
  __syncthreads();
  for (int w = 128; w >= 1; w >>= 1) {
    if ((int)threadIdx.x < w) {
      red[0][threadIdx.x] += red[0][threadIdx.x + w];
      red[1][threadIdx.x] += red[1][threadIdx.x + w];
      red[2][threadIdx.x] += red[2][threadIdx.x + w];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float tau = *tau_p;
    dtau[0] = kLn2 * (sgn * red[0][0] - red[1][0] / tau - sgn * red[2][0]);
  }
}

hipError_t launch_soft_tau_reduce(const float* prep, int nprep, const float* bwd, int nbwd, const float* tau, int sgn,
                                  float* dtau, hipStream_t s) {
  MORPHO_KLAUNCH(soft_tau_reduce_kernel, dim3(1), dim3(256), 0, s, prep, nprep, bwd, nbwd, tau, (float)sgn, dtau);
  return hipGetLastError();
}

}  // namespace morpho
