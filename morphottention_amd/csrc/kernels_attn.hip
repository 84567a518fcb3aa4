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
//    to ~2^-22, and the 8-wide affine block adds the key bias and subtracts the
//    row reference, so exp2 reads the accumulator directly.
//  * Forward softmax uses a per-row reference R >= (row max - 15) computed by
//    the projection from a closed-form bound on the soft Hamming score, so no
//    running max or rescaling is needed; rows whose bound is loose (gap > 25,
//    only possible with large or negative gates) take an exact two-pass path.
//  * V is carried as an fp16 hi/lo pair and both halves are multiplied by the
//    fp16 P; the row normaliser sums exactly those rounded P values.
//  * Transposed operands (V^T, dO^T, phi^T, dS^T) are read from row-major LDS
//    tiles with ds_read_b64_tr_b16.
//  * Both loops are software-pipelined: the next tile's global loads are in
//    flight while the current LDS tile is consumed, one barrier per tile.
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

// Column offset of the c-th 16-wide code chunk of a code row (the 8-wide
// affine block sits at [M, M + 8)).
template <int M>
__device__ __forceinline__ constexpr int chunk_off(int c) {
  return c < M / 16 ? 16 * c : 16 * c + 8;
}

// Workgroups are dispatched round-robin over the 8 XCDs (id % 8), each with
// its own L2. Map a 1-D grid of 8 * ceil(BH / 8) * nblk workgroups so that all
// blocks of one (batch, head) run on the same XCD and share its L2: XCD x
// serves heads x, x + 8, ... in turn. Returns false for the padding slots.
__device__ __forceinline__ bool xcd_map(int nblk, int BH, int& bh, int& blk) {
  const int i = blockIdx.x, xcd = i & 7, slot = i >> 3;
  bh = 8 * (slot / nblk) + xcd;
  blk = slot % nblk;
  return bh < BH;
}
__host__ inline unsigned xcd_grid(int nblk, int BH) { return 8u * (unsigned)((BH + 7) / 8) * (unsigned)nblk; }

// ============================================================ forward
template <int M, int DV>
struct FwdCfg {
  static constexpr int CW = 3 * M + 8;    // code row width
  static constexpr int NCH = 3 * M / 16;  // 16-wide code chunks
  static constexpr int KT = 64;           // keys per LDS tile
  // LDS strides: rows read with ds_read_b128 want a stride = 8 (mod 16) halves
  // (8 consecutive rows then hit 8 distinct 16-byte bank groups); rows read
  // with ds_read_b64_tr_b16 want 16 (mod 64) halves (4 rows x 4 chunks of a
  // 16-lane group hit distinct banks). CW = 3M + 8 is already 8 (mod 16).
  static constexpr int KS = CW;           // key row stride (halves)
  static constexpr int VS = KT + 8;       // V^T tile row stride (halves): row = value column, 64 keys + pad
  static constexpr int QW = 128;          // queries per workgroup (4 waves x 32)
  static constexpr int KVEC = KT * CW / 8;
  static constexpr int VVEC = 2 * DV * KT / 8;
  static constexpr int NKR = (KVEC + 255) / 256;
  static constexpr int NVR = (VVEC + 255) / 256;
};

template <int M, int DV>
struct FwdPrefetch {
  using C = FwdCfg<M, DV>;
  f16x8 kr[C::NKR];
  f16x8 vr[C::NVR];

  __device__ __forceinline__ void load_k(const f16* __restrict__ ka, int64_t rowbase, int N, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < C::NKR; ++i) {
      const int v = tid + 256 * i;
      const int r = v / (C::CW / 8), cv = (v % (C::CW / 8)) * 8;
      // rows past N read the (finite) last row instead; every score they feed
      // is masked. No select here: it would wait for the load to land.
      const int row = min(k0 + r, N - 1);
      kr[i] = *reinterpret_cast<const f16x8*>(ka + (rowbase + row) * C::CW + (v < C::KVEC ? cv : 0));
    }
  }
  // V^T rows are NP >= N + pad long and zero past N, so a 64-key tile never
  // needs a guard.
  __device__ __forceinline__ void load_v(const f16* __restrict__ vt, int64_t vbase, int NP, int k0, int tid) {
#pragma unroll
    for (int i = 0; i < C::NVR; ++i) {
      const int v = tid + 256 * i;
      const int r = v / (C::KT / 8), g = v % (C::KT / 8);
      vr[i] = *reinterpret_cast<const f16x8*>(vt + vbase + (int64_t)r * NP + k0 + 8 * g);
    }
  }
  __device__ __forceinline__ void load(const f16* __restrict__ ka, const f16* __restrict__ vt, int64_t vbase,
                                       int64_t rowbase, int NP, int N, int k0, bool with_v, int tid) {
    load_k(ka, rowbase, N, k0, tid);
    if (with_v) load_v(vt, vbase, NP, k0, tid);
  }

  // Key rows are stored in swap23 order within each 32-row block, so the lanes
  // that read them in score order touch consecutive LDS rows (conflict-free
  // 16-byte reads).
  __device__ __forceinline__ void store_k(f16* sK, int tid) const {
#pragma unroll
    for (int i = 0; i < C::NKR; ++i) {
      const int v = tid + 256 * i;
      const int r = v / (C::CW / 8), cv = (v % (C::CW / 8)) * 8;
      const int lr = (r & ~31) | swap23(r & 31);
      if (v < C::KVEC) *reinterpret_cast<f16x8*>(sK + lr * C::KS + cv) = kr[i];
    }
  }
  __device__ __forceinline__ void store_v(f16* sV, int tid) const {
#pragma unroll
    for (int i = 0; i < C::NVR; ++i) {
      const int v = tid + 256 * i;
      const int r = v / (C::KT / 8), g = v % (C::KT / 8);
      *reinterpret_cast<f16x8*>(sV + r * C::VS + 8 * g) = vr[i];
    }
  }
  __device__ __forceinline__ void store(f16* sK, f16* sV, bool with_v, int tid) const {
    store_k(sK, tid);
    if (with_v) store_v(sV, tid);
  }
};

template <int M, int DV, bool MAXPASS>
__device__ __forceinline__ void fwd_tile_loop(const f16* __restrict__ ka, const f16* __restrict__ vt, int64_t vbase,
                                              int64_t rowbase, int NP, int N, int causal, int t0, int kend, int qw0,
                                              int q,
                                              f16 (*sK)[FwdCfg<M, DV>::KT * FwdCfg<M, DV>::KS],
                                              f16 (*sV)[2 * DV * FwdCfg<M, DV>::VS],
                                              const f16x8 (&qf)[FwdCfg<M, DV>::NCH], const f16x4& qaug,
                                              f32x16 (&o)[DV / 32], float& lsum, float& rmax) {
  using C = FwdCfg<M, DV>;
  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int nkt = (kend + C::KT - 1) / C::KT - t0;
  if (nkt <= 0) return;
  const int wave_kend = causal ? min(N, qw0 + 32) : N;

  auto compute = [&](const f16* tK, const f16* tV, int k0) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kbase = k0 + 32 * kb;
      if (kbase >= wave_kend) continue;  // wave-uniform
      const f16* krow = tK + (32 * kb + l32) * C::KS;
      f32x16 s = {};
#pragma unroll
      for (int c = 0; c < C::NCH; ++c)
        s = mfma16(*reinterpret_cast<const f16x8*>(krow + chunk_off<M>(c) + 8 * h32), qf[c], s);
      s = mfma8(*reinterpret_cast<const f16x4*>(krow + M + 4 * h32), qaug, s);
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
      // O^T += V^T P: A rows are value columns (hi, then lo), k = key
#pragma unroll
      for (int dvb = 0; dvb < DV / 32; ++dvb) {
        const f16* vh = tV + (32 * dvb + l32) * C::VS + 32 * kb + 8 * h32;
        const f16* vl = vh + DV * C::VS;
        f32x16 acc = o[dvb];
        acc = mfma16(*reinterpret_cast<const f16x8*>(vh), p0, acc);
        acc = mfma16(*reinterpret_cast<const f16x8*>(vh + 16), p1, acc);
        acc = mfma16(*reinterpret_cast<const f16x8*>(vl), p0, acc);
        acc = mfma16(*reinterpret_cast<const f16x8*>(vl + 16), p1, acc);
        o[dvb] = acc;
      }
    }
  };

  // Two register stages: while tile kt is consumed from LDS, the loads of
  // tiles kt+1 and kt+2 are in flight; unrolled by two so a stage never
  // changes registers while its loads are outstanding.
  FwdPrefetch<M, DV> pf0, pf1;
  const int kb0 = t0 * C::KT;
  pf0.load(ka, vt, vbase, rowbase, NP, N, kb0, !MAXPASS, tid);
  pf0.store(sK[0], sV[0], !MAXPASS, tid);
  if (nkt > 1) pf1.load(ka, vt, vbase, rowbase, NP, N, kb0 + C::KT, !MAXPASS, tid);
  if (nkt > 2) pf0.load(ka, vt, vbase, rowbase, NP, N, kb0 + 2 * C::KT, !MAXPASS, tid);
  __syncthreads();
  for (int kt = 0; kt < nkt; kt += 2) {
    compute(sK[0], sV[0], kb0 + kt * C::KT);
    if (kt + 1 < nkt) pf1.store(sK[1], sV[1], !MAXPASS, tid);
    __syncthreads();
    if (kt + 3 < nkt) pf1.load(ka, vt, vbase, rowbase, NP, N, kb0 + (kt + 3) * C::KT, !MAXPASS, tid);
    if (kt + 1 >= nkt) break;
    compute(sK[1], sV[1], kb0 + (kt + 1) * C::KT);
    if (kt + 2 < nkt) pf0.store(sK[0], sV[0], !MAXPASS, tid);
    __syncthreads();
    if (kt + 4 < nkt) pf0.load(ka, vt, vbase, rowbase, NP, N, kb0 + (kt + 4) * C::KT, !MAXPASS, tid);
  }
}

template <int M, int DV>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const f16* __restrict__ qa, const f16* __restrict__ ka,
                                                       const f16* __restrict__ vt, const float4* __restrict__ tstat,
                                                       f16* __restrict__ out, float* __restrict__ lse, int N, int NP,
                                                       int H, int D, int BH, int causal) {
  using C = FwdCfg<M, DV>;
  __shared__ __align__(16) f16 sK[2][C::KT * C::KS];
  __shared__ __align__(16) f16 sV[2][2 * DV * C::VS];
  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, scalar
  const int nqb = (N + C::QW - 1) / C::QW;
  int bh, blk;
  if (!xcd_map(nqb, BH, bh, blk)) return;
  const int qblk = causal ? nqb - 1 - blk : blk;  // longest rows first
  const int q0 = qblk * C::QW, qw0 = q0 + 32 * w, q = qw0 + l32;
  const bool qvalid = q < N;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N;
  const int64_t vbase = (int64_t)bh * 2 * DV * NP;

  f16x8 qf[C::NCH];
  f16x4 qaug = {};
#pragma unroll
  for (int c = 0; c < C::NCH; ++c) qf[c] = f16x8{};
  float4 ts = make_float4(0.f, 0.f, 0.f, 0.f);
  if (qvalid) {
    const f16* qrow = qa + (rowbase + q) * C::CW;
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) qf[c] = *reinterpret_cast<const f16x8*>(qrow + chunk_off<M>(c) + 8 * h32);
    qaug = *reinterpret_cast<const f16x4*>(qrow + M + 4 * h32);
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
    fwd_tile_loop<M, DV, true>(ka, vt, vbase, rowbase, NP, N, causal, 0, kend, qw0, q, sK, sV, qf, qa0, o, lsum, rmax);
    rmax = fmaxf(rmax, __shfl_xor(rmax, 32));
    R = qvalid ? rmax : 0.f;
    f16 rh, rl;
    split_hi_lo(-R, rh, rl);
    if (h32 == 0) { qaug[2] = rh; qaug[3] = rl; }
  }
  fwd_tile_loop<M, DV, false>(ka, vt, vbase, rowbase, NP, N, causal, 0, kend, qw0, q, sK, sV, qf, qaug, o, lsum, rmax);

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
  const dim3 grid(xcd_grid((d.N + C::QW - 1) / C::QW, d.B * d.H));
  hipLaunchKernelGGL((attn_fwd_kernel<M, DV>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, p.tstat, out, lse, d.N, d.NP,
                     d.H, d.D, d.B * d.H, d.causal);
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
// qstat = {-(lse - b), -delta} with delta_i = dO_i . O_i (fp32), one thread per
// (token, head), heads fastest so a wave reads whole contiguous rows; the same
// grid zeroes the dq accumulator with contiguous stores.
template <int M, int DV>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const f16* __restrict__ grad_out, const f16* __restrict__ out,
                                                       const float* __restrict__ lse,
                                                       const float4* __restrict__ tstat, float2* __restrict__ qstat,
                                                       float* __restrict__ dq, int64_t T, int N, int H, int D) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx < T * H) {
    const int h = (int)(idx % H);
    const int64_t t = idx / H;
    const int b = (int)(t / N), n = (int)(t - (int64_t)b * N);
    const int64_t bhn = (int64_t)(b * H + h) * N + n;
    const f16* go = grad_out + t * D + h * DV;
    const f16* oo = out + t * D + h * DV;
    float delta = 0.f;
#pragma unroll
    for (int c = 0; c < DV; c += 8) {
      const f16x8 a = *reinterpret_cast<const f16x8*>(go + c);
      const f16x8 o = *reinterpret_cast<const f16x8*>(oo + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) delta += (float)a[e] * (float)o[e];
    }
    qstat[bhn] = make_float2(-(lse[bhn] - tstat[bhn].x), -delta);
  }
  // zero dq: T * H * M floats, M / 4 float4 per (token, head)
  float4* z = reinterpret_cast<float4*>(dq);
  const int64_t nz = T * H * (M / 4);
  for (int64_t i = idx; i < nz; i += (int64_t)gridDim.x * 256) z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int M, int DV>
static hipError_t launch_bwd_prep_t(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* out,
                                    const float* lse, const BwdBuffers& g, hipStream_t s) {
  const int64_t n = d.T * d.H;
  hipLaunchKernelGGL((bwd_prep_kernel<M, DV>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, grad_out, out, lse,
                     p.tstat, g.qstat, g.dq, d.T, d.N, d.H, d.D);
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
  static constexpr int MB = M / 32 + 1;         // 32-row blocks of dk^T (codes + the ones row at row M)
  static constexpr int MQ = (M + 31) / 32;      // 32-column blocks of dq
  static constexpr int QT = M <= 32 ? 64 : 32;  // queries per step
  static constexpr int NSB = QT / 32;           // 32-query sub-blocks per step
  // strides (halves): see FwdCfg; the query and dO tiles serve both b128 and
  // transposed reads and are laid out for the b128 ones
  static constexpr int QS = CW;                 // query tile stride
  static constexpr int OS = DV + 8;             // dO tile stride: DV values + 8 aug
  static constexpr int SS = QT + 16;            // dS^T tile stride (transposed reads only)
  static constexpr int PKS = M + 16;            // key phi tile stride (transposed reads only)
  static constexpr int KW = 128;                // keys per workgroup (4 waves x 32)
  static constexpr int DQT = (QT / 16) * (M / 16) / 4;  // 16x16 dq tiles per wave per step
  // prefetch: data vectors of 8 halves per step (the affine blocks are built from qstat)
  static constexpr int QDV = 3 * M / 8;         // code vectors per query row
  static constexpr int ODV = DV / 8;            // dO vectors per query row
  static constexpr int NDV = QT * (QDV + ODV);
  static constexpr int NPR = (NDV + 255) / 256;
};

template <int M, int DV>
struct BwdPrefetch {
  using C = BwdCfg<M, DV>;
  f16x8 r[C::NPR];
  float2 st;  // qstat of query row tid (tid < QT)

  __device__ __forceinline__ void load(const f16* __restrict__ qa, const f16* __restrict__ grad_out,
                                       const float2* __restrict__ qstat, int64_t rowbase, int64_t tokbase, int hoff,
                                       int N, int D, int qs, int tid) {
#pragma unroll
    for (int i = 0; i < C::NPR; ++i) {
      const int v = tid + 256 * i;
      f16x8 x = {};
      if (v < C::QT * C::QDV) {
        const int rr = v / C::QDV, j = v % C::QDV;
        const int col = j < M / 8 ? 8 * j : 8 * j + 8;
        if (qs + rr < N) x = *reinterpret_cast<const f16x8*>(qa + (rowbase + qs + rr) * C::CW + col);
      } else if (v < C::NDV) {
        const int u = v - C::QT * C::QDV;
        const int rr = u / C::ODV, col = 8 * (u % C::ODV);
        if (qs + rr < N) x = *reinterpret_cast<const f16x8*>(grad_out + (tokbase + qs + rr) * D + hoff + col);
      }
      r[i] = x;
    }
    st = make_float2(0.f, 0.f);
    if (tid < C::QT && qs + tid < N) st = qstat[rowbase + qs + tid];
  }

  __device__ __forceinline__ void store(f16* sQ, f16* sO, int tid) const {
#pragma unroll
    for (int i = 0; i < C::NPR; ++i) {
      const int v = tid + 256 * i;
      if (v < C::QT * C::QDV) {
        const int rr = v / C::QDV, j = v % C::QDV;
        const int col = j < M / 8 ? 8 * j : 8 * j + 8;
        *reinterpret_cast<f16x8*>(sQ + rr * C::QS + col) = r[i];
      } else if (v < C::NDV) {
        const int u = v - C::QT * C::QDV;
        const int rr = u / C::ODV, col = 8 * (u % C::ODV);
        *reinterpret_cast<f16x8*>(sO + rr * C::OS + col) = r[i];
      }
    }
    if (tid < C::QT) {
      // affine blocks (rows past N get st = 0; every score they touch is masked)
      const f16 one = (f16)1.f;
      f16 lh, ll, dh, dl;
      split_hi_lo(st.x, lh, ll);
      split_hi_lo(st.y, dh, dl);
      const f16 zero = (f16)0.f;
      *reinterpret_cast<f16x8*>(sQ + tid * C::QS + M) = f16x8{one, one, lh, ll, zero, zero, zero, zero};
      *reinterpret_cast<f16x8*>(sO + tid * C::OS + DV) = f16x8{dh, dl, zero, zero, zero, zero, zero, zero};
    }
  }
};

template <int M, int DV>
__global__ __launch_bounds__(256) void attn_bwd_kernel(const f16* __restrict__ qa, const f16* __restrict__ ka,
                                                       const f16* __restrict__ vt, const float2* __restrict__ qstat,
                                                       const f16* __restrict__ grad_out, float* __restrict__ dq,
                                                       float* __restrict__ dk, float* __restrict__ dcb,
                                                       f16* __restrict__ dzv, int N, int NP, int H, int D, int HM, int BH,
                                                       int causal) {
  using C = BwdCfg<M, DV>;
  __shared__ __align__(16) f16 sQ[2][C::QT * C::QS];
  __shared__ __align__(16) f16 sO[2][C::QT * C::OS];
  __shared__ __align__(16) f16 sdS[2][C::KW * C::SS];  // dS^T of the whole workgroup: row = key
  __shared__ __align__(16) f16 sPk[C::KW * C::PKS];     // phi_hi of the workgroup's keys: row = key

  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, scalar
  int bh, kblk;
  if (!xcd_map((N + C::KW - 1) / C::KW, BH, bh, kblk)) return;
  const int k0 = kblk * C::KW;  // causal: low key blocks see the most queries; they start first
  const int kw0 = k0 + 32 * w;
  const int key = kw0 + l32;
  const bool kvalid = key < N;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N;
  const int64_t tokbase = (int64_t)b * N;
  const f16 one = (f16)1.f, zero = (f16)0.f;

  // ---- per-wave key-side operands, loaded once
  f16x8 kf[C::NCH];
  f16x4 kaug = {};
  f16x8 vf[DV / 16];
#pragma unroll
  for (int c = 0; c < C::NCH; ++c) kf[c] = f16x8{};
#pragma unroll
  for (int c = 0; c < DV / 16; ++c) vf[c] = f16x8{};
  if (kvalid) {
    const f16* krow = ka + (rowbase + key) * C::CW;
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) kf[c] = *reinterpret_cast<const f16x8*>(krow + chunk_off<M>(c) + 8 * h32);
    kaug = *reinterpret_cast<const f16x4*>(krow + M + 4 * h32);
    // V_hi[key][16c + 8 h32 + j] from the transposed layout (a wave reads 32
    // consecutive keys of each value column)
    const f16* vcol = vt + (int64_t)bh * 2 * DV * NP + key;
#pragma unroll
    for (int c = 0; c < DV / 16; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) vf[c][j] = vcol[(int64_t)(16 * c + 8 * h32 + j) * NP];
  }
  const f16x4 vaug = h32 == 0 ? f16x4{one, one, zero, zero} : f16x4{zero, zero, zero, zero};
  // phi_hi of the workgroup's keys for the dq product (zero past N)
  for (int v = tid; v < C::KW * (M / 8); v += 256) {
    const int r = v / (M / 8), cv = (v % (M / 8)) * 8;
    f16x8 x = {};
    if (k0 + r < N) x = *reinterpret_cast<const f16x8*>(qa + (rowbase + k0 + r) * C::CW + cv);
    *reinterpret_cast<f16x8*>(sPk + r * C::PKS + cv) = x;
  }

  f32x16 dva[DV / 32], dka[C::MB];
#pragma unroll
  for (int i = 0; i < DV / 32; ++i) dva[i] = f32x16{};
#pragma unroll
  for (int i = 0; i < C::MB; ++i) dka[i] = f32x16{};

  const int qstart = causal ? k0 : 0;
  const int nsteps = qstart < N ? (N - qstart + C::QT - 1) / C::QT : 0;
  // keys of this workgroup that exist: dq contracts over [0, kw_valid) only
  const int nkey = min(C::KW, N - k0);

  // Two register stages (see the forward): step s computes from LDS buffer
  // s & 1 while the loads of steps s+1 and s+2 are in flight.
  BwdPrefetch<M, DV> pf0, pf1;
  auto pf_load = [&](BwdPrefetch<M, DV>& pf, int step) {
    pf.load(qa, grad_out, qstat, rowbase, tokbase, h * DV, N, D, qstart + step * C::QT, tid);
  };
  if (nsteps > 0) {
    pf_load(pf0, 0);
    pf0.store(sQ[0], sO[0], tid);
  }
  if (nsteps > 1) pf_load(pf1, 1);
  if (nsteps > 2) pf_load(pf0, 2);
  __syncthreads();

  for (int step = 0; step < nsteps; ++step) {
    const int buf = step & 1;
    const int qs = qstart + step * C::QT;
    const bool more = step + 1 < nsteps;
    const f16* tQ = sQ[buf];
    const f16* tO = sO[buf];
    f16* tS = sdS[buf] + (32 * w + l32) * C::SS;  // this lane's key row
#pragma unroll
    for (int sb = 0; sb < C::NSB; ++sb) {
      const int q0 = qs + 32 * sb;
      f16x8 ds16[2] = {f16x8{}, f16x8{}};
      if (!((causal && kw0 > q0 + 31) || kw0 >= N || q0 >= N)) {  // wave-uniform: something unmasked
        // S = Q~ K~^T (rows: queries in swap23 order; lane: key)
        const f16* qrow = tQ + (32 * sb + swap23(l32)) * C::QS;
        f32x16 s = {};
#pragma unroll
        for (int c = 0; c < C::NCH; ++c)
          s = mfma16(*reinterpret_cast<const f16x8*>(qrow + chunk_off<M>(c) + 8 * h32), kf[c], s);
        s = mfma8(*reinterpret_cast<const f16x4*>(qrow + M + 4 * h32), kaug, s);
        // dP - delta = dO~ V~^T
        const f16* orow = tO + (32 * sb + swap23(l32)) * C::OS;
        f32x16 dp = {};
#pragma unroll
        for (int c = 0; c < DV / 16; ++c)
          dp = mfma16(*reinterpret_cast<const f16x8*>(orow + 16 * c + 8 * h32), vf[c], dp);
        dp = mfma8(*reinterpret_cast<const f16x4*>(orow + DV + 4 * h32), vaug, dp);
        const bool need_mask = (q0 + 32 > N) || (kw0 + 31 >= N) || (causal && kw0 + 31 > q0);
        f16x8 p16[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float pr = fast_exp2(s[r]);
          if (need_mask) {
            const int qq = q0 + swap23(acc_row(r, lane));
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
            dva[dvb] = mfma16(frag_kmajor(tO, C::OS, 32 * sb + 16 * c, 32 * dvb, lane), p16[c], dva[dvb]);
#pragma unroll
          for (int mb = 0; mb < C::MB; ++mb)
            dka[mb] = mfma16(frag_kmajor(tQ, C::QS, 32 * sb + 16 * c, 32 * mb, lane), ds16[c], dka[mb]);
        }
      }
      // dS^T row of this key (zeros where nothing was computed)
#pragma unroll
      for (int c = 0; c < 2; ++c) *reinterpret_cast<f16x8*>(tS + 32 * sb + 16 * c + 8 * h32) = ds16[c];
    }
    if (more) {
      if (buf == 0) pf1.store(sQ[1], sO[1], tid);
      else pf0.store(sQ[0], sO[0], tid);
    }
    __syncthreads();  // dS^T of all four waves complete; next tiles visible
    if (step + 3 < nsteps) {
      if (buf == 0) pf_load(pf1, step + 3);
      else pf_load(pf0, step + 3);
    }
    // dq[q][code] += sum_key dS[q][key] phi[key][code]: 16 x 16 output tiles
    // split over the waves, contraction over the workgroup's keys.
#pragma unroll
    for (int t = 0; t < C::DQT; ++t) {
      const int tile = w + 4 * t;
      const int qt = tile % (C::QT / 16), ct = tile / (C::QT / 16);
      const int qrow0 = qs + 16 * qt;
      if (qrow0 >= N) continue;  // uniform
      f32x4 acc = {};
      for (int kc = 0; kc < nkey; kc += 32)
        acc = mfma16x16(frag16_kmajor(sdS[buf], C::SS, kc, 16 * qt, lane),
                        frag16_kmajor(sPk, C::PKS, kc, 16 * ct, lane), acc);
      const int code = 16 * ct + (lane & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int qq = qrow0 + 4 * (lane >> 4) + r;
        if (qq < N && acc[r] != 0.f) unsafeAtomicAdd(dq + (rowbase + qq) * M + code, acc[r]);
      }
    }
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
    f16* drow = dzv + (tokbase + key) * NC + HM + h * DV;
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
  const dim3 grid(xcd_grid((d.N + C::KW - 1) / C::KW, d.B * d.H));
  hipLaunchKernelGGL((attn_bwd_kernel<M, DV>), grid, dim3(256), 0, s, p.qa, p.ka, p.vt, g.qstat, grad_out, g.dq, g.dk,
                     g.dcb, g.dzv, d.N, d.NP, d.H, d.D, d.HM, d.B * d.H, d.causal);
  return hipGetLastError();
}

hipError_t launch_attn_bwd(const Dims& d, const ProjBuffers& p, const f16* grad_out, const BwdBuffers& g,
                           hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_attn_bwd_t, d, p, grad_out, g, s);
}

}  // namespace morpho
