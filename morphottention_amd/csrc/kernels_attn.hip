// Attention backward: the recompute-from-statistics gradients of the scores,
// the softmax and the value aggregation, and the prep kernel before it (the
// forward is in kernels_attn_fwd.hip).
//
// Reference: packages/morphottention/csrc/cuda/attention/attention.cu:191-483
//   (P = exp2(s - lse), dV = P^T dO, dP = dO V^T, dS = P (dP - delta),
//   dk = dS^T q, dcb = -scale sum_i dS; the query-side dq that the reference
//   accumulates and drops is completed here)
//
// MI355X design:
//  * The exponent is recomputed by one MFMA accumulator over the code rows
//    [hi | affine(8) | lo], whose query affine block the forward rewrote to
//    {1, 1, -(lse - b)}, so exp2 reads the accumulator directly; dP - delta
//    comes out of one MFMA in the same way.
//  * Transposed operands (dO^T, phi^T, dS^T) are read from row-major LDS
//    tiles with ds_read_b64_tr_b16.
//  * The query steps stream through two LDS stages filled by DMA, one
//    barrier per step.
#include <type_traits>

#include "common.h"
#include "internal.h"

namespace morpho {

// The backward forms a query step's dS row sums (for the diagonal correction)
// only when one of its rows has a diagonal weight above this.
constexpr float kRowSumWeight = 0.5f;

// ============================================================ backward prep
// The dO rows' affine block {-delta} with delta_i = dO_i . O_i (fp32), and,
// when the backward computed the projection itself (the forward's query rows
// still hold its own reference), the query rows' block {1, 1, -(lse - b)}.
// DV / 8 consecutive lanes share one (head, token), each reading 16 bytes of
// dO and of O; consecutive lane groups take consecutive tokens of one head, so
// the per-row lse / tstat reads and aug writes are contiguous too, and a wave
// reads whole 128-byte row pieces of dO and O. The partial dot products meet
// in xor shuffles. The same grid zeroes the dq and row-sum accumulators.
template <int M, int DV>
__global__ __launch_bounds__(256) void bwd_prep_kernel(const f16* __restrict__ grad_out, const f16* __restrict__ out,
                                                       const float* __restrict__ lse,
                                                       const float4* __restrict__ tstat, f16* __restrict__ aug,
                                                       f16* __restrict__ qa, int write_q, float* __restrict__ dq,
                                                       float2* __restrict__ dr, int diag, int64_t T, int N, int H,
                                                       int D) {
  constexpr int G = DV / 8;  // lanes per (head, token): 4, 8 or 16, aligned within the wave
  constexpr int CW = 2 * M + 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nvec = T * (D / 8);
  const int64_t bhn = idx / G;  // (b * H + h) * N + n
  float delta = 0.f;
  if (idx < nvec) {
    const int64_t bh = bhn / N;
    const int n = (int)(bhn - bh * N), b = (int)(bh / H), h = (int)(bh - (int64_t)b * H);
    const int64_t off = ((int64_t)b * N + n) * D + h * DV + 8 * (int)(idx & (G - 1));
    const f16x8 a = *reinterpret_cast<const f16x8*>(grad_out + off);
    const f16x8 o = *reinterpret_cast<const f16x8*>(out + off);
#pragma unroll
    for (int e = 0; e < 8; ++e) delta += (float)a[e] * (float)o[e];
  }
#pragma unroll
  for (int sh = 1; sh < G; sh <<= 1) delta += __shfl_xor(delta, sh);
  if (idx < nvec && (threadIdx.x & (G - 1)) == 0) {
    f16 dh, dl;
    split_hi_lo(-delta, dh, dl);
    const f16 zero = (f16)0.f;
    const float l = lse[bhn];
    const float4 ts = tstat[bhn];
    // the diagonal weight P_ii = 2^(s_ii - lse) with s_ii = t + b (0 when the
    // diagonal is masked or the row has no keys), and whether the row needs
    // its dS row sum: with the diagonal in the softmax only a row with most of
    // its weight there does (elsewhere the offset the sum measures is below
    // 2^-10 of the row's gradient); without it every row keeps its sum. The
    // flag sits in the unused third slot of the affine block.
    const float pii = diag && l > -kFltMax ? fast_exp2(ts.w + ts.x - l) : 0.f;
    const f16 need = (!diag || pii > kRowSumWeight) ? (f16)1.f : zero;
    *reinterpret_cast<f16x8*>(aug + bhn * 8) = f16x8{dh, dl, need, zero, zero, zero, zero, zero};
    if (write_q) {
      f16 lh, ll;
      split_hi_lo(l > -kFltMax ? -(l - ts.x) : 0.f, lh, ll);  // a row without keys: masked anyway
      *reinterpret_cast<f16x2*>(qa + bhn * CW + M + 2) = f16x2{lh, ll};
    }
    // the row-sum accumulator (zero) and the diagonal weight
    dr[bhn] = make_float2(0.f, pii);
  }
  // zero dq: T * H * M floats, M / 4 float4 per (token, head)
  float4* z = reinterpret_cast<float4*>(dq);
  const int64_t nz = T * H * (M / 4);
  for (int64_t i = idx; i < nz; i += (int64_t)gridDim.x * 256) z[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int M, int DV>
static hipError_t launch_bwd_prep_t(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* out,
                                    const float* lse, const BwdBuffers& g, int write_q, hipStream_t s) {
  const int64_t n = d.T * (d.D / 8);
  MORPHO_KLAUNCH((bwd_prep_kernel<M, DV>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, grad_out, out, lse,
                     p.tstat, g.aug, p.qa, write_q, g.dq, reinterpret_cast<float2*>(g.dr), d.mask_diag ? 0 : 1,
                     d.T, d.N, d.H, d.D);
  return hipGetLastError();
}

hipError_t launch_bwd_prep(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* out, const float* lse,
                           const BwdBuffers& g, int write_q, hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_bwd_prep_t, d, p, grad_out, out, lse, g, write_q, s);
}

// ============================================================ backward
// Chunk swizzle of the 16-byte chunks of an LDS row of RB bytes (RB = 64, 128
// or a multiple of 256): physical chunk = logical chunk ^ rswz<RB>(row). With
// 64 banks of 4 bytes it makes both access patterns of the backward
// conflict-free:
//  (a) 16 lanes reading (b128) one logical chunk of 16 consecutive rows;
//  (b) transposing b64 reads of 32 lanes covering 4 consecutive rows x 4
//      aligned chunks (32x32x16 operands), or rows {r..r+3, r+8..r+11} x 2
//      aligned chunks (16x16x32 operands).
template <int RB>
__device__ __forceinline__ int rswz(int r) {
  static_assert(RB == 64 || RB == 128 || RB % 256 == 0, "row bytes");
  if constexpr (RB == 64) return (r >> 2) & 3;
  else if constexpr (RB == 128) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else return ((r & 3) << 2) | ((r >> 2) & 3);
}
__host__ __device__ constexpr int pow2_bytes(int x) { return x <= 64 ? 64 : 2 * pow2_bytes((x + 1) / 2); }
// stored row of logical row r in a tile whose rows are in swap23 order within each 32
__device__ __forceinline__ int srow23(int r) { return (r & ~31) | swap23(r & 31); }

// MFMA 32x32x16 operand from a row-major LDS tile (rows in swap23 order,
// chunk-swizzled rows of RB bytes) whose rows are the contraction index:
// value(mn, k) = logical row k0 + k, column mn0 + mn. Each lane's two reads
// (rows +0 and +4) stay inside one 16-byte chunk.
template <int RB>
__device__ __forceinline__ f16x8 tfrag32(const char* tile, int k0, int mn0, int lane) {
  const int g = lane >> 4;
  const int row = k0 + 8 * (g >> 1) + ((lane & 15) >> 2);
  const int col = mn0 + 16 * (g & 1) + 4 * (lane & 3);
  auto at = [&](int lr) {
    const int sr = srow23(lr);
    return tile + sr * RB + 16 * ((col >> 3) ^ rswz<RB>(sr)) + 2 * (col & 7);
  };
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(at(row)));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(at(row + 4)));
  return __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}
// MFMA 16x16x32 operand from a row-major LDS tile (rows in natural order,
// chunk-swizzled rows of RB bytes): value(mn, k) = row k0 + k, column mn0 +
// mn, mn = lane % 16, k = 8 (lane / 16) + j.
template <int RB>
__device__ __forceinline__ f16x8 tfrag16(const char* tile, int k0, int mn0, int lane) {
  const int row = k0 + 8 * (lane >> 4) + ((lane & 15) >> 2);
  const int col = mn0 + 4 * (lane & 3);
  auto at = [&](int r) { return tile + r * RB + 16 * ((col >> 3) ^ rswz<RB>(r)) + 2 * (col & 7); };
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(at(row)));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(at(row + 4)));
  return __builtin_bit_cast(f16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

template <int M, int DV>
struct BwdCfg {
  static constexpr int CW = 2 * M + 8;
  static constexpr int NCH = M / 8;             // 16-wide code chunks (hi, then lo)
  // dcb (the column sums of dS) comes from the ones row M of the query rows'
  // affine block on the MFMA when that row shares a 32-row block with codes
  // (M = 16); for M = 32 and 64 it would need a block of its own, so the VALU
  // sums the same fp16 dS values instead (v_dot2 against ones).
  static constexpr bool DCB_VALU = M % 32 == 0;
  static constexpr int MB = DCB_VALU ? M / 32 : M / 32 + 1;  // 32-row blocks of dk^T
  // Queries per step: 64 at m = 16; 32 at m = 32 and 64, which keeps two
  // workgroups per CU (LDS and registers); 64 at m = 32 needed 92 KiB and ran
  // one wave per SIMD (B1 N16384 H16 m32 causal: 1.86 -> 1.74 ms with 32).
  static constexpr int QT = M <= 16 ? 64 : 32;
  static constexpr int NSB = QT / 32;           // 32-query sub-blocks per step
  // LDS rows (bytes): query rows padded to a power of two, dO rows, the
  // per-query dO affine block (16 bytes), dS^T rows (one per key, QT
  // queries), key phi rows (at least 32 halves). Query and dO rows are stored
  // in swap23 order within each 32.
  static constexpr int QRB = pow2_bytes(2 * CW);
  static constexpr int ORB = 2 * DV;
  static constexpr int SRB = 2 * QT;
  static constexpr int PRB = 2 * (M < 32 ? 32 : M);
  // Waves per workgroup, 32 keys each. Every workgroup adds one fp32 atomic
  // per (query, code) of each step to dq, so the atomic count scales with the
  // number of key blocks: at m = 32 and 64 8 waves (256 keys) halve it, at
  // one workgroup (two waves per SIMD) per CU.
  static constexpr int NW = M >= 32 && DV <= 64 ? 8 : 4;
  static constexpr int NT = 64 * NW;                      // threads
  static constexpr int KW = 32 * NW;                      // keys per workgroup
  // 16x16 dq tiles of a step, and per wave: when there are fewer tiles than
  // waves (m = 32: 4 tiles, 8 waves) the waves w >= DQTILES have no dq work.
  static constexpr int DQTILES = (QT / 16) * (M / 16);
  static constexpr int DQT = DQTILES >= NW ? DQTILES / NW : 1;
  static_assert(DQTILES < NW || DQTILES % NW == 0, "dq tiles must split evenly over the waves");
  // a stage = query tile, dO tile, affine tile; 1 KiB DMA pieces
  static constexpr int QP = QT * QRB / 1024, OP = QT * ORB / 1024;
  static constexpr int QPW = QP / NW, OPW = (OP + NW - 1) / NW;  // pieces per wave (dO: the first OP % NW waves)
  static_assert(QP % NW == 0, "query pieces must split evenly over the waves");
  static constexpr int MIN_WG = NW == 4 ? 2 : 1;  // workgroups per CU (launch bound)
  static constexpr int OOFF = QT * QRB, AOFF = OOFF + QT * ORB;  // bytes
  static constexpr int STAGE = AOFF + 1024;
};

// Key-side (KV-outer) backward. A workgroup owns KW = 32 NW keys (32 per
// wave, kept in registers: codes, V_hi, dk / dV accumulators) and streams the
// query steps of QT queries through two LDS stages filled by DMA. Step s:
//   wait for its tiles, barrier (also publishes dS^T of step s - 1), DMA the
//   tiles of step s + 1, read the dq fragments of step s - 1, compute step s
//   (S, dP, P, dS, dV += dO^T P, dk^T += phi^T dS, dS^T -> LDS), then finish
//   dq of step s - 1 (MFMA over the workgroup's keys, fp32 atomics).
// Every wave with dq tiles issues exactly 4 DQT dq atomics per step (masked
// lanes add 0.0 to a valid address), and every wave one that adds the row
// sums of dS of step s - 1 (over the workgroup's keys) to dr when that step
// has a flagged row, so the tile wait can leave the latest step's atomics in
// flight: vector-memory operations complete in issue order.
// The query rows come from the projection's code rows, whose affine block
// holds {1, 1, -(lse - b)} by now (written by the forward, or by bwd_prep when
// the backward computed the projection itself); the dO rows come from
// grad_out and their affine block {-delta} from bwd_prep's aug rows.
// HILO: the recomputed scores use the codes' hi and lo chunks (exact to
// ~2^-22, as in the forward); without it only the hi chunks (one MFMA instead
// of three per 16 codes). The backward's P is then exp2 of a score off by
// ~2^-11 of its code terms, which moves the gradients by ~1e-3 relative for
// codes in [0, 1] at m = 16 with moderate code weights (the kernel below
// uses it only there).
// DET: instead of adding to dq and dr with atomics, every workgroup stores its
// sums over its own keys into per-key-block partials ([nkb][B*H][NQ][M] and
// [nkb][B*H][NQ] fp32, NQ = N rounded up to QT, so rows past N land in
// padding); dq_det_reduce adds them in key-block order, which makes dq and
// the row sums identical from run to run. A store replaces each atomic one
// for one, so the tile waits count the same operations (waves without a
// row-sum tile issue no row-sum store and wait as if they had sent none).
// The body of attn_bwd_kernel for key block kblk of (batch, head) bh. The
// LDS tiles are the kernel's: stg (2 stages), sdS (dS^T of the whole
// workgroup, two buffers of KW rows = keys) and sPk (phi_hi of the
// workgroup's keys, row = key).
template <int M, int DV, bool MD, bool HILO, bool DET>
__device__ __forceinline__ void attn_bwd_body(char* stg, char* sdS0, char* sPk, int bh, int kblk,
                                              const f16* __restrict__ qa, const f16* __restrict__ ka,
                                              const f16* __restrict__ vt, const f16* __restrict__ aug,
                                              const f16* __restrict__ grad_out, float* __restrict__ dq,
                                              float* __restrict__ dk, float* __restrict__ dcb, float* __restrict__ dr,
                                              f16* __restrict__ dzv, int N, int NP, int H, int D, int HM, int BH,
                                              int causal) {
  using C = BwdCfg<M, DV>;
  auto sdS = [&](int par) { return sdS0 + par * (C::KW * C::SRB); };

  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, scalar
  const int nkb = (N + C::KW - 1) / C::KW;
  const int k0 = kblk * C::KW;  // causal: low key blocks see the most queries; they start first
  const int kw0 = k0 + 32 * w;
  const int key = kw0 + l32;
  const bool kvalid = key < N;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N;
  const int64_t tokbase = (int64_t)b * N;
  const f16 one = (f16)1.f, zero = (f16)0.f;
  // DET: this workgroup's slices of the partials
  const int NQ = (N + C::QT - 1) / C::QT * C::QT;
  float* const dqk = dq + ((int64_t)kblk * BH + bh) * NQ * M;
  float* const drk = dr + ((int64_t)kblk * BH + bh) * NQ;

  // ---- per-wave key-side operands, loaded once
  constexpr int KCH = HILO ? C::NCH : C::NCH / 2;  // code chunks the scores read
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
    for (int c = 0; c < KCH; ++c) kf[c] = *reinterpret_cast<const f16x8*>(krow + chunk_off<M>(c) + 8 * h32);
    kaug = *reinterpret_cast<const f16x4*>(krow + M + 4 * h32);
    // V_hi[key][16c + 8 h32 + j] from the transposed layout (a wave reads 32
    // consecutive keys of each value column)
    const f16* vcol = vt + (int64_t)bh * DV * NP + key;
#pragma unroll
    for (int c = 0; c < DV / 16; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) vf[c][j] = vcol[(int64_t)(16 * c + 8 * h32 + j) * NP];
  }
  const f16x4 vaug = h32 == 0 ? f16x4{one, one, zero, zero} : f16x4{zero, zero, zero, zero};
  // phi_hi of the workgroup's keys for the dq product (zero past N)
  for (int v = tid; v < C::KW * (M / 8); v += C::NT) {
    const int r = v / (M / 8), c = v % (M / 8);
    f16x8 x = {};
    if (k0 + r < N) x = *reinterpret_cast<const f16x8*>(qa + (rowbase + k0 + r) * C::CW + 8 * c);
    *reinterpret_cast<f16x8*>(sPk + r * C::PRB + 16 * (c ^ rswz<C::PRB>(r))) = x;
  }

  f32x16 dva[DV / 32], dka[C::MB];
#pragma unroll
  for (int i = 0; i < DV / 32; ++i) dva[i] = f32x16{};
#pragma unroll
  for (int i = 0; i < C::MB; ++i) dka[i] = f32x16{};
  float dcb_acc = 0.f;  // DCB_VALU: this lane's share of dcb[key]

  const int qstart = causal ? k0 : 0;
  const int nsteps = qstart < N ? (N - qstart + C::QT - 1) / C::QT : 0;
  // Query tile of step st. Without the causal mask every key block visits all
  // query tiles; block kblk starts kblk / nkb of the way round, so the blocks
  // of a head add their dq and row-sum atomics to different rows at any one
  // time (in lockstep they contended for the same rows' memory-side atomics:
  // C5 attn_bwd 4.06 -> 3.71 ms, C2 0.052 -> 0.048 ms). Causal blocks already
  // start at their own keys.
  const int qrot = causal ? 0 : (int)(((int64_t)kblk * nsteps) / nkb);
  auto qstep = [&](int st) {
    const int r = st + qrot;
    return qstart + (r < nsteps ? r : r - nsteps) * C::QT;
  };

  // ---- DMA of a step's tiles. Per-lane byte offsets from the step's bases
  // (query rows qa + (rowbase + qs) CW, dO rows grad_out + (tokbase + qs) D +
  // h DV, affine rows aug + (rowbase + qs) 8), computed once; padding chunks
  // of the query rows load column 0 of the same row.
  unsigned qoff[C::QPW], ooff[C::OPW], aoff;
#pragma unroll
  for (int i = 0; i < C::QPW; ++i) {
    const int q = 64 * (w + C::NW * i) + lane, r = q / (C::QRB / 16);
    const int c = (q % (C::QRB / 16)) ^ rswz<C::QRB>(r);
    qoff[i] = (unsigned)((srow23(r) * C::CW + (8 * c < C::CW ? 8 * c : 0)) * 2);
  }
#pragma unroll
  for (int j = 0; j < C::OPW; ++j) {
    const int q = 64 * min(w + C::NW * j, C::OP - 1) + lane, r = q / (C::ORB / 16);
    const int c = (q % (C::ORB / 16)) ^ rswz<C::ORB>(r);
    ooff[j] = (unsigned)(((int64_t)srow23(r) * D + 8 * c) * 2);
  }
  aoff = (unsigned)(srow23(lane % C::QT) * 16);
  const unsigned sbase = (unsigned)(uintptr_t)(__attribute__((address_space(3))) char*)stg;
  auto issue = [&](int st) {
    const unsigned dst = sbase + (unsigned)((st & 1) * C::STAGE);
    const int qs = qstep(st);
    if (qs + C::QT <= N) {  // uniform
      const f16* qbase = qa + (rowbase + qs) * C::CW;
#pragma unroll
      for (int i = 0; i < C::QPW; ++i) lds_dma16_so(qbase, qoff[i], dst + 1024u * (unsigned)(w + C::NW * i));
      const f16* obase = grad_out + (tokbase + qs) * D + h * DV;
#pragma unroll
      for (int j = 0; j < C::OPW; ++j)
        if (w + C::NW * j < C::OP) lds_dma16_so(obase, ooff[j], dst + C::OOFF + 1024u * (unsigned)(w + C::NW * j));
      if (w == 0) lds_dma16_so(aug + (rowbase + qs) * 8, aoff, dst + C::AOFF);
    } else {  // ragged last step: rows past N read row N - 1 (every score they feed is masked)
#pragma unroll
      for (int i = 0; i < C::QPW; ++i) {
        const int q = 64 * (w + C::NW * i) + lane, r = q / (C::QRB / 16);
        const int c = (q % (C::QRB / 16)) ^ rswz<C::QRB>(r);
        const int qrow = min(qs + srow23(r), N - 1);
        lds_dma16(qa + (rowbase + qrow) * C::CW + (8 * c < C::CW ? 8 * c : 0), dst + 1024u * (unsigned)(w + C::NW * i));
      }
#pragma unroll
      for (int j = 0; j < C::OPW; ++j)
        if (w + C::NW * j < C::OP) {
          const int q = 64 * (w + C::NW * j) + lane, r = q / (C::ORB / 16);
          const int c = (q % (C::ORB / 16)) ^ rswz<C::ORB>(r);
          const int qrow = min(qs + srow23(r), N - 1);
          lds_dma16(grad_out + (tokbase + qrow) * D + h * DV + 8 * c, dst + C::OOFF + 1024u * (unsigned)(w + C::NW * j));
        }
      if (w == 0)
        lds_dma16(aug + (rowbase + min(qs + srow23(lane % C::QT), N - 1)) * 8, dst + C::AOFF);
    }
  };

  // ---- per-lane LDS offsets, computed once. Every read below is one of
  // these plus a compile-time constant (the stage, the 32-row sub-block, the
  // 16-row k half), which the compiler folds into the instruction's offset.
  // Transposing reads (32x32x16 operands, tfrag32): half hh (rows +4 hh) of
  // the column block mn0 at k0 = 0; a k0 of 16 c adds 16 c RB.
  auto toff = [&](auto RBc, int mn0, int hh) {
    constexpr int RB = decltype(RBc)::value;
    const int g = lane >> 4;
    const int sr = srow23(8 * (g >> 1) + ((lane & 15) >> 2) + 4 * hh);
    const int col = mn0 + 16 * (g & 1) + 4 * (lane & 3);
    return sr * RB + 16 * ((col >> 3) ^ rswz<RB>(sr)) + 2 * (col & 7);
  };
  using QRBc = std::integral_constant<int, C::QRB>;
  using ORBc = std::integral_constant<int, C::ORB>;
  int t_o[DV / 32][2], t_q[C::MB][2];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
    for (int dvb = 0; dvb < DV / 32; ++dvb) t_o[dvb][hh] = toff(ORBc{}, 32 * dvb, hh);
#pragma unroll
    for (int mb = 0; mb < C::MB; ++mb) t_q[mb][hh] = toff(QRBc{}, 32 * mb, hh);
  }
  auto tread = [&](const char* tile, int off, int k0rb) {
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + k0rb + off)));
  };
  auto tfrag = [&](const char* tile, const int (&offs)[2], int k0rb) {
    const f16x4 lo = tread(tile, offs[0], k0rb), hi = tread(tile, offs[1], k0rb);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };
  // Row reads of this lane's query / dO row (row 32 sb + l32): code chunks,
  // the query affine block, dO chunks.
  const int qz = rswz<C::QRB>(l32), oz = rswz<C::ORB>(l32);
  int r_q[C::NCH], r_o[DV / 16];
#pragma unroll
  for (int c = 0; c < C::NCH; ++c) r_q[c] = l32 * C::QRB + 16 * ((chunk_off<M>(c) / 8 + h32) ^ qz);
  const int r_qa = l32 * C::QRB + 16 * ((M / 8) ^ qz) + 8 * h32;
#pragma unroll
  for (int c = 0; c < DV / 16; ++c) r_o[c] = l32 * C::ORB + 16 * ((2 * c + h32) ^ oz);
  const int r_oa = l32 * 16 + 8 * h32;
  const int kr = 32 * w + l32;  // this lane's dS^T row (its key)
  const int sz = sswz<C::SRB>(kr);

  // ---- dq[q][code] += sum_key dS[q][key] phi[key][code]: 16 x 16 output
  // tiles split over the waves, contraction over all KW keys of the workgroup
  // (rows past N are zero in both operands).
  f16x8 dqa[C::DQT][C::KW / 32];
  int d_s[C::DQT][2];
#pragma unroll
  for (int t = 0; t < C::DQT; ++t) {
    const int qt = (w + C::NW * t) % (C::QT / 16);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int row = 8 * (lane >> 4) + ((lane & 15) >> 2) + 4 * hh;
      const int col = 16 * qt + 4 * (lane & 3);
      d_s[t][hh] = row * C::SRB + 16 * ((col >> 3) ^ sswz<C::SRB>(row)) + 2 * (col & 7);
    }
  }
  // The key-side operands above are loaded under a condition; without a wait
  // on every path the compiler treats them as possibly pending inside the step
  // loop and waits for vmcnt there, which then also drains the next step's DMA
  // and the dq atomics on every sub-block.
  wait_vmcnt<0>();
  __syncthreads();  // sPk is complete

  // waves with dq tiles (wave-uniform); the others issue no dq atomics
  const bool dq_wave = w < C::DQTILES;
  // The dq product's phi operand never changes. At m = 16 it stays in
  // registers (4 fragments, 16 VGPRs; C3 attn_bwd -3 %); with eight waves
  // (m = 32, 64: 256 keys, twice the fragments) it is re-read from the phi
  // tile each step (registers are the scarcer there).
  constexpr bool PHIREG = M == 16;
  f16x8 phib[PHIREG ? C::DQT : 1][PHIREG ? C::KW / 32 : 1];
  if constexpr (PHIREG) {
#pragma unroll
    for (int t = 0; t < C::DQT; ++t)
#pragma unroll
      for (int kc = 0; kc < C::KW / 32; ++kc)
        phib[t][kc] = tfrag16<C::PRB>(sPk, 32 * kc, 16 * ((w + C::NW * t) / (C::QT / 16)), lane);
  }
  auto dq_load = [&](const char* sd) {
    if (!dq_wave) return;
#pragma unroll
    for (int t = 0; t < C::DQT; ++t)
#pragma unroll
      for (int kc = 0; kc < C::KW / 32; ++kc) dqa[t][kc] = tfrag(sd, d_s[t], 32 * kc * C::SRB);
  };
  // dq atomics: rows qs + 16 qt + 4 (lane / 16) + r, column 16 ct + lane % 16,
  // one uniform base per step plus a lane offset
  int a_off[C::DQT];
#pragma unroll
  for (int t = 0; t < C::DQT; ++t) {
    const int tile = w + C::NW * t;
    const int qt = tile % (C::QT / 16), ct = tile / (C::QT / 16);
    a_off[t] = (16 * qt + 4 * (lane >> 4)) * M + 16 * ct + (lane & 15);
  }
  // Row sums sum_j dS[q][j] over the workgroup's keys: the A fragments of the
  // tile (qt, ct = 0) times a ones operand on the MFMA (tile w of the waves
  // w < QT / 16 that own such a tile). Every
  // column of the 16 x 16 result holds the row sums; lanes with (lane & 15) < 4
  // add rows 4 (lane / 16) + (lane & 3) to dr, one atomic per row. The other
  // waves add 0 there, so every wave issues one such atomic.
  // Only a step with a flagged query row (bwd_prep's flag in the third slot
  // of the dO affine block; every workgroup sees the same flags, so such a
  // row gets the sums of all key blocks) forms its sums; the others issue
  // neither the MFMAs nor the atomic, and the tile wait of the step after
  // next allows one atomic fewer in flight.
  const bool rs_wave = w < C::QT / 16;  // uniform: tile w is the (qt, ct = 0) tile
  const int rs_row = 16 * (w % (C::QT / 16)) + 4 * (lane >> 4) + (lane & 3);
  bool rs_need = false;  // the flag of the step whose sums rowsum() forms next
  bool rs_sent = false;  // whether the previous step issued a row-sum atomic
  // issued right after the fragments of step st are read, so that it overlaps
  // the next step's body
  auto rowsum = [&](int st) {
    if constexpr (DET) {  // every step stores its sums (0 without a flagged row) from the row-sum waves
      rs_sent = rs_wave;
      if (!rs_wave) return;  // uniform
      const int qs = qstep(st);
      f32x4 racc = {};
      if (rs_need) {  // uniform
        const f16 one16 = (f16)1.f;
        const f16x8 ones = {one16, one16, one16, one16, one16, one16, one16, one16};
#pragma unroll
        for (int kc = 0; kc < C::KW / 32; ++kc) racc = mfma16x16(dqa[0][kc], ones, racc);
      }
      const int j = lane & 3;
      const float rsum = j == 0 ? racc[0] : j == 1 ? racc[1] : j == 2 ? racc[2] : racc[3];
      if ((lane & 15) < 4) drk[qs + rs_row] = rsum;
      return;
    }
    rs_sent = rs_need;
    if (!rs_need) return;  // uniform
    const int qs = qstep(st);
    f32x4 racc = {};
    if (rs_wave) {
      const f16 one16 = (f16)1.f;
      const f16x8 ones = {one16, one16, one16, one16, one16, one16, one16, one16};
#pragma unroll
      for (int kc = 0; kc < C::KW / 32; ++kc) racc = mfma16x16(dqa[0][kc], ones, racc);
    }
    const int j = lane & 3;
    const float rsum = j == 0 ? racc[0] : j == 1 ? racc[1] : j == 2 ? racc[2] : racc[3];
    const int qq = qs + rs_row;
    if ((lane & 15) < 4)
      unsafeAtomicAdd(&dr[2 * (rowbase + (qq < N ? qq : N - 1))], rs_wave && qq < N ? rsum : 0.f);
  };
  auto dq_finish = [&](int st) {
    if (!dq_wave) return;
    const int qs = qstep(st);
    float* base = dq + (rowbase + qs) * M;
    const bool full = qs + C::QT <= N;  // uniform
#pragma unroll
    for (int t = 0; t < C::DQT; ++t) {
      const int tile = w + C::NW * t;
      const int qt = tile % (C::QT / 16);
      f32x4 acc = {};
#pragma unroll
      for (int kc = 0; kc < C::KW / 32; ++kc) {
        f16x8 phi_op;
        if constexpr (PHIREG)
          phi_op = phib[t][kc];
        else
          phi_op = tfrag16<C::PRB>(sPk, 32 * kc, 16 * (tile / (C::QT / 16)), lane);
        acc = mfma16x16(dqa[t][kc], phi_op, acc);
      }
      if constexpr (DET) {
#pragma unroll
        for (int r = 0; r < 4; ++r) dqk[(int64_t)qs * M + (unsigned)a_off[t] + r * M] = acc[r];
        continue;
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (full) {
          unsafeAtomicAdd(base + (unsigned)a_off[t] + r * M, acc[r]);
        } else {
          const int qq = qs + 16 * qt + 4 * (lane >> 4) + r;
          const bool ok = qq < N;
          // always issued (a fixed count per step); rows past N add 0 to row N - 1
          unsafeAtomicAdd(dq + (rowbase + (ok ? qq : N - 1)) * M + 16 * ((w + C::NW * t) / (C::QT / 16)) + (lane & 15),
                          ok ? acc[r] : 0.f);
        }
      }
    }
  };

  // ---- one query step; PAR = step & 1 (the stage and dS^T buffer), a
  // compile-time constant so every LDS address is a lane offset plus an
  // immediate.
  auto do_step = [&](auto PARc, int step) {
    constexpr int PAR = decltype(PARc)::value;
    // this step's tiles have landed (the atomics of step - 2, issued after
    // them, may still be in flight) and this wave's dS^T writes are done
    if (step >= 2) {
      if (dq_wave) {  // uniform
        if (rs_sent)
          wait_vmcnt_lgkm0<4 * C::DQT + 1>();
        else
          wait_vmcnt_lgkm0<4 * C::DQT>();
      } else {
        if (rs_sent)
          wait_vmcnt_lgkm0<1>();
        else
          wait_vmcnt_lgkm0<0>();
      }
    } else {
      wait_vmcnt_lgkm0<0>();
    }
    __builtin_amdgcn_s_barrier();
    if (step + 1 < nsteps) issue(step + 1);  // its stage last served step - 1
    if (step >= 1) {
      dq_load(sdS(PAR ^ 1));
      rowsum(step - 1);
    }

    const int qs = qstep(step);
    const char* tQ = stg + PAR * C::STAGE;
    const char* tO = tQ + C::OOFF;
    const char* tA = tQ + C::AOFF;
    char* tS = sdS(PAR);
    // this step's row-sum flag (one affine row per lane; rows repeat when
    // QT = 32), for the next step's rowsum()
    // (a whole 16-byte affine row per lane: a 2-byte read at a 16-byte stride
    // was a 4-way bank conflict)
    const bool rs_flag_here = __ballot((float)reinterpret_cast<const f16x8*>(tA)[lane][2] != 0.f) != 0;
    // S = Q~ K~^T and dP - delta = dO~ V~^T of sub-block sb (rows: queries in
    // swap23 order; lane: key)
    auto scores = [&](int sb, f32x16& s, f32x16& dp) {
      const char* qsb = tQ + 32 * sb * C::QRB;
      f16x8 qfr[C::NCH] = {};
#pragma unroll
      for (int c = 0; c < KCH; ++c) qfr[c] = *reinterpret_cast<const f16x8*>(qsb + r_q[c]);
      s = HILO ? code_dot<M, false>(kf, qfr, f32x16{}) : code_dot_hi<M, false>(kf, qfr, f32x16{});
      s = mfma8(*reinterpret_cast<const f16x4*>(qsb + r_qa), kaug, s);
      const char* osb = tO + 32 * sb * C::ORB;
      dp = f32x16{};
#pragma unroll
      for (int c = 0; c < DV / 16; ++c) dp = mfma16(*reinterpret_cast<const f16x8*>(osb + r_o[c]), vf[c], dp);
      dp = mfma8(*reinterpret_cast<const f16x4*>(tA + 32 * sb * 16 + r_oa), vaug, dp);
    };
    // P, dS = P (dP - delta), dV^T += dO^T P, dk^T += phi^T dS (rows: dv /
    // code; lane: key)
    auto soft = [&](const f32x16& s, const f32x16& dp, f16x8 (&p16)[2], f16x8 (&ds16)[2]) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = fast_exp2(s[r]);
        p16[r >> 3][r & 7] = (f16)pr;
        ds16[r >> 3][r & 7] = (f16)(pr * dp[r]);
      }
      // one value per rounded dS: the dk / dcb products read these registers
      // and dq / the row sums read their LDS copy, and the diagonal
      // correction relies on both being the same halves (a conversion
      // selected twice, once from the exact product, could differ at ties)
      asm("" : "+v"(ds16[0]), "+v"(ds16[1]));
      if (C::DCB_VALU) {
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        const h2 ones2 = {(f16)1.f, (f16)1.f};
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            dcb_acc = __builtin_amdgcn_fdot2(h2{ds16[c][2 * e], ds16[c][2 * e + 1]}, ones2, dcb_acc, false);
      }
    };
    auto prods = [&](int sb, const f16x8 (&p16)[2], const f16x8 (&ds16)[2]) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
#pragma unroll
        for (int dvb = 0; dvb < DV / 32; ++dvb)
          dva[dvb] = mfma16(tfrag(tO, t_o[dvb], (32 * sb + 16 * c) * C::ORB), p16[c], dva[dvb]);
#pragma unroll
        for (int mb = 0; mb < C::MB; ++mb)
          dka[mb] = mfma16(tfrag(tQ, t_q[mb], (32 * sb + 16 * c) * C::QRB), ds16[c], dka[mb]);
      }
    };
    auto grads = [&](int sb, const f32x16& s, const f32x16& dp, f16x8 (&ds16)[2]) {
      f16x8 p16[2];
      soft(s, dp, p16, ds16);
      prods(sb, p16, ds16);
    };
    // dS^T row of this key (zeros where nothing was computed): logical chunk
    // 4 sb + 2 c + h32 at physical chunk (4 sb + 2 c + h32) ^ sz
    auto put_ds = [&](int sb, const f16x8 (&ds16)[2]) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
        *reinterpret_cast<f16x8*>(tS + kr * C::SRB + 16 * ((4 * sb + 2 * c + h32) ^ sz)) = ds16[c];
    };
    // A step whose two sub-blocks are whole and unmasked for this wave (the
    // bulk of the work) runs as one straight block: the scores of sub-block 1
    // are on the MFMA while sub-block 0's exponentials run on the VALU. Both
    // sub-blocks' exponentials come before their dV / dk products, so the fp32
    // scores are dead by then (m = 16: 256 -> 240 VGPRs, room for the dq
    // product's phi operand).
    const bool plain = C::NSB == 2 && qs + C::QT <= N && kw0 + 31 < N && (!causal || kw0 + 31 <= qs) &&
                       (!MD || kw0 > qs + C::QT - 1 || kw0 + 31 < qs);  // wave-uniform
    if (plain) {
      f32x16 s0, dp0, s1, dp1;
      f16x8 d0[2], d1[2];
      f16x8 p0[2], p1[2];
      scores(0, s0, dp0);
      scores(1, s1, dp1);
      soft(s0, dp0, p0, d0);
      soft(s1, dp1, p1, d1);
      prods(0, p0, d0);
      prods(1, p1, d1);
      put_ds(0, d0);
      put_ds(1, d1);
    } else {
#pragma unroll
      for (int sb = 0; sb < C::NSB; ++sb) {
        const int q0 = qs + 32 * sb;
        f16x8 ds16[2] = {f16x8{}, f16x8{}};
        if (!((causal && kw0 > q0 + 31) || kw0 >= N || q0 >= N)) {  // wave-uniform: something unmasked
          f32x16 s, dp;
          scores(sb, s, dp);
          const bool need_mask = (q0 + 32 > N) || (kw0 + 31 >= N) || (causal && kw0 + 31 > q0) ||
                                 (MD && kw0 <= q0 + 31 && kw0 + 31 >= q0);
          if (need_mask) {  // wave-uniform; masked scores become -inf (P = 0)
            // one select per score from a mask built with bitwise operators:
            // written as a conditional store after a short-circuit ||, the
            // MD instances compiled to divergent blocks whose stores were
            // dropped for in-range lanes (causal and diagonal masks lost)
            const int kx = kvalid ? key : (1 << 30);  // a key past N exceeds every limit
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int qq = q0 + swap23(acc_row(r, lane));
              const int klim = causal ? qq : N - 1;  // the largest key this query sees
              const bool drop = (qq >= N) | (kx > klim) | (MD && kx == qq);
              s[r] = drop ? kNegInf : s[r];
            }
          }
          grads(sb, s, dp, ds16);
        }
        put_ds(sb, ds16);
      }
    }
    if (step >= 1) dq_finish(step - 1);
    rs_need = rs_flag_here;
  };

  if (nsteps > 0) issue(0);
  int step = 0;
  for (; step + 1 < nsteps; step += 2) {
    do_step(std::integral_constant<int, 0>{}, step);
    do_step(std::integral_constant<int, 1>{}, step + 1);
  }
  if (step < nsteps) do_step(std::integral_constant<int, 0>{}, step);
  if (nsteps > 0) {
    wait_vmcnt_lgkm0<4 * C::DQT + 1>();
    __builtin_amdgcn_s_barrier();  // dS^T of the last step from every wave
    dq_load(sdS((nsteps - 1) & 1));
    rowsum(nsteps - 1);
    dq_finish(nsteps - 1);
  }

  // ---- epilogue: dk, dcb (fp32, per key) and dV (fp16 into the dZ|dV buffer)
  const float dcb_sum = dcb_acc + __shfl_xor(dcb_acc, 32);  // lanes l, l + 32: the same key
  if (kvalid) {
    if (C::DCB_VALU && h32 == 0) dcb[rowbase + key] = dcb_sum;
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

// Bound on a head's code weights sum_c |scale gate_q_c gate_k_c| up to which
// the scores may come from the fp16 hi codes alone: the scores' error is
// then ~2^-12 of that sum, and an fp64 emulation of the backward put the
// worst gradient error at 4.4e-3 for m = 16 at scale 2 with unit gates (sum
// 32; 9.5e-3 at scale 4), against the 1e-2 bar.
constexpr float kHiOnlyWeight = 32.f;

// Key-side (KV-outer) backward kernel: maps the workgroup to its key block
// (causal: longest first) and runs the body. HIOK (m = 16, sigmoid
// projection, codes in [0, 1]): the scores come from the hi codes alone
// where the head's code weights are within kHiOnlyWeight, from hi and lo
// elsewhere (the decision is the workgroup's; both bodies share the LDS
// tiles). Without HIOK always from hi and lo.
template <int M, int DV, bool MD, bool HIOK, bool DET>
__global__ __launch_bounds__((BwdCfg<M, DV>::NT), (BwdCfg<M, DV>::MIN_WG)) void attn_bwd_kernel(
    const f16* __restrict__ qa, const f16* __restrict__ ka, const f16* __restrict__ vt, const f16* __restrict__ aug,
    const f16* __restrict__ grad_out, float* __restrict__ dq, float* __restrict__ dk, float* __restrict__ dcb,
    float* __restrict__ dr, f16* __restrict__ dzv, const f16* __restrict__ gate_q, const f16* __restrict__ gate_k,
    float scale, int N, int NP, int H, int D, int HM, int BH, int causal) {
  using C = BwdCfg<M, DV>;
  __shared__ __align__(16) char stg[2 * C::STAGE];
  __shared__ __align__(16) char sdS[2 * C::KW * C::SRB];
  __shared__ __align__(16) char sPk[C::KW * C::PRB];
  int bh, kblk;
  const int nkb = (N + C::KW - 1) / C::KW;
  if (!(causal ? xcd_map_lpt(nkb, BH, bh, kblk) : xcd_map(nkb, BH, bh, kblk))) return;
  bool hilo = true;
  if constexpr (HIOK) {
    const int h = bh % H;
    float wsum = 0.f;
#pragma unroll
    for (int c = 0; c < M; ++c) wsum += fabsf((float)gate_q[h * M + c] * (float)gate_k[h * M + c]);
    hilo = __builtin_amdgcn_readfirstlane(fabsf(scale) * wsum > kHiOnlyWeight ? 1 : 0) != 0;
  }
  if (hilo)
    attn_bwd_body<M, DV, MD, true, DET>(stg, sdS, sPk, bh, kblk, qa, ka, vt, aug, grad_out, dq, dk, dcb, dr, dzv, N,
                                        NP, H, D, HM, BH, causal);
  else if constexpr (HIOK)
    attn_bwd_body<M, DV, MD, false, DET>(stg, sdS, sPk, bh, kblk, qa, ka, vt, aug, grad_out, dq, dk, dcb, dr, dzv, N,
                                         NP, H, D, HM, BH, causal);
}

template <int M, int DV, bool HIOK, bool DET>
static hipError_t launch_attn_bwd_c(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* gate_q,
                                    const f16* gate_k, const BwdBuffers& g, hipStream_t s) {
  using C = BwdCfg<M, DV>;
  const dim3 grid(xcd_grid((d.N + C::KW - 1) / C::KW, d.B * d.H));
  float* const dq = DET ? g.dqpart : g.dq;
  float* const dr = DET ? g.drpart : g.dr;
  if (d.mask_diag)
    MORPHO_KLAUNCH((attn_bwd_kernel<M, DV, true, HIOK, DET>), grid, dim3(C::NT), 0, s, p.qa, p.ka, p.vt, g.aug,
                   grad_out, dq, g.dk, g.dcb, dr, g.dzv, gate_q, gate_k, d.scale, d.N, d.NP, d.H, d.D, d.HM,
                   d.B * d.H, d.causal);
  else
    MORPHO_KLAUNCH((attn_bwd_kernel<M, DV, false, HIOK, DET>), grid, dim3(C::NT), 0, s, p.qa, p.ka, p.vt, g.aug,
                   grad_out, dq, g.dk, g.dcb, dr, g.dzv, gate_q, gate_k, d.scale, d.N, d.NP, d.H, d.D, d.HM,
                   d.B * d.H, d.causal);
  return hipGetLastError();
}

template <int M, int DV, bool HIOK>
static hipError_t launch_attn_bwd_h(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* gate_q,
                                    const f16* gate_k, const BwdBuffers& g, hipStream_t s) {
  if (d.det) {
    if (!g.dqpart || !g.drpart) return hipErrorInvalidValue;
    return launch_attn_bwd_c<M, DV, HIOK, true>(d, p, grad_out, gate_q, gate_k, g, s);
  }
  return launch_attn_bwd_c<M, DV, HIOK, false>(d, p, grad_out, gate_q, gate_k, g, s);
}

// The hi-only scores are possible at m = 16 with the sigmoid projection
// (codes in [0, 1]; the forward's scores stay exact); hi and lo elsewhere.
template <int M, int DV>
static hipError_t launch_attn_bwd_t(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* gate_q,
                                    const f16* gate_k, const BwdBuffers& g, hipStream_t s) {
  if constexpr (M == 16)
    if (d.proj == kProjSigmoid) return launch_attn_bwd_h<M, DV, true>(d, p, grad_out, gate_q, gate_k, g, s);
  return launch_attn_bwd_h<M, DV, false>(d, p, grad_out, gate_q, gate_k, g, s);
}

hipError_t launch_attn_bwd(const Dims& d, const ProjBuffers& p, const f16* grad_out, const f16* gate_q,
                           const f16* gate_k, const BwdBuffers& g, hipStream_t s) {
  MORPHO_MDV_DISPATCH(launch_attn_bwd_t, d, p, grad_out, gate_q, gate_k, g, s);
}

// ---------------------------------------------------------------- deterministic dq
template <int M, int DV>
static hipError_t det_layout_t(const Dims& d, DetLayout* l) {
  using C = BwdCfg<M, DV>;
  l->kw = C::KW;
  l->nkb = (d.N + C::KW - 1) / C::KW;
  l->nq = (d.N + C::QT - 1) / C::QT * C::QT;
  return hipSuccess;
}

DetLayout attn_bwd_det_layout(const Dims& d) {
  DetLayout l{0, 0, 0};
  auto f = [&]() -> hipError_t { MORPHO_MDV_DISPATCH(det_layout_t, d, &l); };
  (void)f();
  return l;
}

// dq[bh][q] = sum over the key blocks kb that saw query q (all of them, or kb
// <= q / KW under the causal mask), in increasing kb, of the partials; the
// row sum dr[bh][q].x the same way (its .y, the diagonal weight, stays).
// One lane per 4 codes of a row: a wave reads 64 consecutive float4 of one
// key block's partials per load.
template <int M>
__global__ __launch_bounds__(256) void dq_det_reduce_kernel(const float* __restrict__ dqpart,
                                                            const float* __restrict__ drpart, float* __restrict__ dq,
                                                            float* __restrict__ dr, int N, int NQ, int BH, int nkb,
                                                            int KW, int causal) {
  constexpr int V = M / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)BH * N * V) return;
  const int64_t row = idx / V;  // bh N + q
  const int c4 = (int)(idx - row * V);
  const int bh = (int)(row / N), q = (int)(row - (int64_t)bh * N);
  const int nk = causal ? min(q / KW + 1, nkb) : nkb;
  const int64_t prow = (int64_t)bh * NQ + q, kstride = (int64_t)BH * NQ;
  const float4* src = reinterpret_cast<const float4*>(dqpart + prow * M) + c4;
  const int64_t kv = kstride * V;  // float4 between consecutive key blocks
  // key blocks added in order; the loads of 8 are issued before their adds
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  int kb = 0;
  for (; kb + 8 <= nk; kb += 8) {
    float4 v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = src[(kb + i) * kv];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      acc.x += v[i].x;
      acc.y += v[i].y;
      acc.z += v[i].z;
      acc.w += v[i].w;
    }
  }
  for (; kb < nk; ++kb) {
    const float4 v = src[kb * kv];
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  }
  reinterpret_cast<float4*>(dq + row * M)[c4] = acc;
  if (c4 == 0) {
    float r = 0.f, u[8];
    int k2 = 0;
    for (; k2 + 8 <= nk; k2 += 8) {
#pragma unroll
      for (int i = 0; i < 8; ++i) u[i] = drpart[(k2 + i) * kstride + prow];
#pragma unroll
      for (int i = 0; i < 8; ++i) r += u[i];
    }
    for (; k2 < nk; ++k2) r += drpart[k2 * kstride + prow];
    dr[2 * row] = r;
  }
}

hipError_t launch_dq_det_reduce(const Dims& d, const BwdBuffers& g, hipStream_t s) {
  if (!g.dqpart || !g.drpart) return hipErrorInvalidValue;
  const DetLayout l = attn_bwd_det_layout(d);
  const int BH = d.B * d.H;
  const int64_t n = (int64_t)BH * d.N * (d.M / 4);
  const dim3 grid((unsigned)((n + 255) / 256));
  switch (d.M) {
    case 16:
      MORPHO_KLAUNCH(dq_det_reduce_kernel<16>, grid, dim3(256), 0, s, g.dqpart, g.drpart, g.dq, g.dr, d.N, l.nq, BH,
                     l.nkb, l.kw, d.causal);
      break;
    case 32:
      MORPHO_KLAUNCH(dq_det_reduce_kernel<32>, grid, dim3(256), 0, s, g.dqpart, g.drpart, g.dq, g.dr, d.N, l.nq, BH,
                     l.nkb, l.kw, d.causal);
      break;
    case 64:
      MORPHO_KLAUNCH(dq_det_reduce_kernel<64>, grid, dim3(256), 0, s, g.dqpart, g.drpart, g.dq, g.dr, d.N, l.nq, BH,
                     l.nkb, l.kw, d.causal);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace morpho
