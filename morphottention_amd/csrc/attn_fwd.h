// Templates of the attention forward (kernels, launch helpers), shared by
// kernels_attn_fwd.hip (cube_m 16 and 32, compiled with the max-ilp
// machine-scheduler strategy) and kernels_attn_fwd_m64.hip (cube_m 64, the
// default strategy): each instance is compiled in exactly one of them.
#pragma once

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
// XOR swizzle of the 16-byte chunk index within a 128-byte V^T tile row: the
// 16 rows one b128 read phase touches land on distinct bank groups.
__device__ __forceinline__ int vswz(int r) { return (r ^ (r >> 3)) & 7; }

template <int M, int DV, bool SM = false>
struct FwdCfg {
  static constexpr int CW = 2 * M + 8;    // code row width
  static constexpr int NCH = M / 8;       // 16-wide code chunks (hi, then lo)
  static constexpr int KT = 64;           // keys per tile
  // Each wave owns QB blocks of 32 queries: every K / V fragment read from LDS
  // then feeds QB MFMAs. Two blocks where the registers allow it (m dv <=
  // 1024; at m = 32, dv = 64 two blocks spill).
  // SM (small problems, fewer than two of the regular workgroups per CU): one
  // query block per wave, four waves, three workgroups per CU, so the launch
  // has twice the workgroups and still covers the CUs.
  // W4 (m >= 32, dv <= 64, one block per wave): four-wave workgroups, two or
  // three per CU (LDS permitting), rather than one of eight waves; the waves
  // of a CU then wait at independent barriers (B1 N16384 H16 m32 causal:
  // forward -6 %; B16 N2048 H32 m64: -7 %).
  static constexpr int QB2 = (M <= 32 && DV <= 64 && M * DV <= 1024) ? 2 : 1;
  static constexpr bool SMALL = SM && QB2 == 2;
  static constexpr int QB = SMALL ? 1 : QB2;
  static constexpr bool W4 = QB2 == 1 && M >= 32 && DV <= 64;
  static constexpr int WAVES = (SMALL || W4) ? 4 : 8 / QB;
  static constexpr int QW = 32 * QB * WAVES;  // 128 or 256 queries per workgroup
  // A stage holds one key tile [KT][CW] (rows in swap23 order within each 32,
  // unpadded: CW = 8 (mod 16) halves keeps b128 reads conflict-free), one
  // V_hi^T tile [DV][KT] fp16 (chunk-swizzled) and one V_lo block [DV][64]
  // e4m3 (chunk-swizzled), all filled by 1 KiB DMA chunks: each wave issues
  // NKW key chunks and NVW value chunks (both kinds' slots are padded to a
  // multiple of the wave count; padding slots repeat the last chunk), so every
  // wave's i-th chunk is fixed.
  static constexpr int KCH = CW / 8;      // key tile chunks
  static constexpr int VHC = DV / 8;      // V_hi^T chunks (8 rows of 64 keys)
  static constexpr int VLC = DV / 16;     // V_lo chunks (16 rows of 64 bytes)
  static constexpr int VCH = VHC + VLC;
  static constexpr int NKW = (KCH + WAVES - 1) / WAVES;  // key chunks per wave
  static constexpr int NVW = (VCH + WAVES - 1) / WAVES;  // value chunks per wave
  static constexpr int NPW = NKW + NVW;   // chunks per wave per tile
  static constexpr int NPW_K = NKW;       // key-only tiles (exact-max pass)
  static constexpr int VOFF = NKW * WAVES * 512;  // V_hi^T offset in a stage (halves)
  static constexpr int LOFF = VOFF + VHC * 512;   // V_lo offset in a stage (halves)
  static constexpr int STAGE = WAVES * NPW * 512; // halves, incl. padding slots
  // Two workgroups per CU (four waves each, 256 VGPRs) when two stages of each
  // fit in half the 160 KiB LDS (less 1 KiB for the rest); the eight-wave
  // shapes (one query block per wave) would have to fit 128 VGPRs and spill.
  // W4: three workgroups when two stages fit a third of the LDS (m = 32,
  // 142 VGPRs), else two.
  static constexpr bool TWO = 2 * STAGE * 2 <= 79 * 1024 && QB == 2;
  static constexpr int W4WG = 2 * STAGE * 2 <= 52 * 1024 ? 3 : 2;
  static constexpr int WG_PER_CU = W4 ? W4WG : SMALL ? 3 : TWO ? 2 : 1;
  static constexpr int WAVES_PER_EU = WG_PER_CU * WAVES / 4;
  static constexpr int LDS_BUDGET = (WG_PER_CU == 3 ? 52 : WG_PER_CU == 2 ? 79 : 158) * 1024;
  static constexpr int NSTAGE = 3 * STAGE * 2 <= LDS_BUDGET ? 3 : 2;
  // both 32-key blocks of a tile in flight at once (fits the registers except
  // with the widest codes and values)
  static constexpr bool PIPE = !(M >= 64 && DV >= 128);
};

// One pass over the key tiles [0, kend) of a workgroup. Tiles stream through
// NSTAGE LDS stages by DMA: tile t + NSTAGE - 1 is issued right after the
// barrier that opens tile t (its stage last served tile t - 1, which every wave
// finished before that barrier), so each tile has NSTAGE - 1 tiles of compute
// to arrive; one barrier per tile.
// MAXPASS: key tiles only, track the row max of the exponent (exact path).
// MD: the diagonal (key == query) is masked.
template <int M, int DV, bool MAXPASS, bool MD, bool SM>
__device__ __forceinline__ void fwd_pass(const f16* __restrict__ ka, const f16* __restrict__ vt,
                                         const uint8_t* __restrict__ vlo, int64_t rowbase, int64_t vbase,
                                         int N, int NP, int causal, int kend, int q0, int qw0,
                                         f16* smem, const f16x8 (&qf)[FwdCfg<M, DV, SM>::QB][FwdCfg<M, DV, SM>::NCH],
                                         const f16x4 (&qaug)[FwdCfg<M, DV, SM>::QB],
                                         f32x16 (&o)[FwdCfg<M, DV, SM>::QB][DV / 32], float (&lsum)[FwdCfg<M, DV, SM>::QB],
                                         float (&rmax)[FwdCfg<M, DV, SM>::QB]) {
  using C = FwdCfg<M, DV, SM>;
  constexpr int QB = C::QB;
  constexpr int NPWX = MAXPASS ? C::NPW_K : C::NPW;
  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkt = (kend + C::KT - 1) / C::KT;

  // LDS byte address of the stage area (the DMA takes raw LDS addresses)
  const unsigned sbase = (unsigned)(uintptr_t)(__attribute__((address_space(3))) f16*)smem;
  // Per-lane byte offsets of this wave's chunks from the tile's key base
  // ka + (rowbase + k0) CW, V_hi^T base vt + vbase + k0 and V_lo block base
  // vlo + (vbase + 64 t) (all wave-uniform), computed once: key chunk
  // w + WAVES i (slots past KCH repeat the last chunk), value chunk
  // v = w + WAVES j: V_hi^T rows 8v.. for v < VHC, else V_lo rows 16(v - VHC)..
  unsigned koff[C::NKW], voff[C::NVW];
#pragma unroll
  for (int i = 0; i < C::NKW; ++i) {
    const int p = 64 * min(w + C::WAVES * i, C::KCH - 1) + lane;
    const int row = p / (C::CW / 8), col = 8 * (p % (C::CW / 8));
    koff[i] = (unsigned)((((row & ~31) | swap23(row & 31)) * C::CW + col) * 2);
  }
#pragma unroll
  for (int j = 0; j < C::NVW; ++j) {
    const int v = min(w + C::WAVES * j, C::VCH - 1);
    if (v < C::VHC) {
      const int pv = 64 * v + lane;
      const int r = pv >> 3, lc = (pv & 7) ^ vswz(r);
      voff[j] = (unsigned)(((int64_t)r * NP + 8 * lc) * 2);
    } else {
      const int r = 16 * (v - C::VHC) + (lane >> 2), c = (lane & 3) ^ ((r >> 2) & 3);
      voff[j] = (unsigned)(64 * r + 16 * c);
    }
  }
  auto issue = [&](int t) {
    const unsigned st = sbase + 2u * (unsigned)((t % C::NSTAGE) * C::STAGE);
    const int k0 = t * C::KT;
    if (k0 + C::KT <= N) {  // uniform: no key row past N
      const f16* kbase = ka + (rowbase + k0) * C::CW;
#pragma unroll
      for (int i = 0; i < C::NKW; ++i) lds_dma16_so(kbase, koff[i], st + 1024u * (unsigned)(w + C::WAVES * i));
    } else {
#pragma unroll
      for (int i = 0; i < C::NKW; ++i) {
        const int p = 64 * min(w + C::WAVES * i, C::KCH - 1) + lane;
        const int row = p / (C::CW / 8), col = 8 * (p % (C::CW / 8));
        // rows past N read the (finite) last row; every score they feed is masked
        const int key = min(k0 + ((row & ~31) | swap23(row & 31)), N - 1);
        lds_dma16(ka + (rowbase + key) * C::CW + col, st + 1024u * (unsigned)(w + C::WAVES * i));
      }
    }
    if (!MAXPASS) {
      // values are zero from N to NP >= k0 + KT
      const f16* vb = vt + vbase + k0;
      const uint8_t* lb = vlo + vbase + (int64_t)DV * k0;
#pragma unroll
      for (int j = 0; j < C::NVW; ++j) {
        const unsigned dst = st + 2u * C::VOFF + 1024u * (unsigned)(w + C::WAVES * j);
        if (min(w + C::WAVES * j, C::VCH - 1) < C::VHC)  // wave-uniform
          lds_dma16_so(vb, voff[j], dst);
        else
          lds_dma16_so(lb, voff[j], dst);
      }
    }
  };

  // This lane's V^T fragment offsets within a stage. Row 32 j + l32 has
  // swizzle vswz(l32) ^ 4 (j & 1), so the chunk of key half p of block kb is
  //   4 (kb ^ z2 ^ (j & 1)) + 2 (p ^ z1) + (h32 ^ z0)   (z = vswz(l32) bits),
  // i.e. four per-lane offsets cover every (kb, p, j) up to a constant.
  int vofs[2][2];
  {
    const int z = vswz(l32);
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        vofs[x][p] = C::VOFF + l32 * C::KT + 8 * (4 * (x ^ (z >> 2)) + 2 * (p ^ ((z >> 1) & 1)) + (h32 ^ (z & 1)));
  }
  // V_hi^T fragments of block kb: [part][dvb], part = k 0-15, k 16-31; A rows
  // are value columns, k = key.
  auto vfrags = [&](const f16* tile, int kb, f16x8 (&vf)[2][DV / 32]) {
#pragma unroll
    for (int part = 0; part < 2; ++part)
#pragma unroll
      for (int dvb = 0; dvb < DV / 32; ++dvb)
        vf[part][dvb] = *reinterpret_cast<const f16x8*>(tile + vofs[kb ^ (dvb & 1)][part] + 32 * C::KT * dvb);
  };
  // O^T += V_hi^T P; the DV / 32 accumulators are independent and interleaved
  auto pv = [&](const f16x8 (&vf)[2][DV / 32], int qb, const f16x8& p0, const f16x8& p1) {
#pragma unroll
    for (int part = 0; part < 2; ++part)
#pragma unroll
      for (int dvb = 0; dvb < DV / 32; ++dvb)
        o[qb][dvb] = mfma16(vf[part][dvb], part ? p1 : p0, o[qb][dvb]);
  };
  // V_lo fragments of the whole 64-key tile: lane (l32, h32) of value block dvb
  // holds row 32 dvb + l32, bytes 32 h32 .. 32 h32 + 31 (logical 16-byte chunks
  // 2 h32, 2 h32 + 1, stored at chunk ^ ((row >> 2) & 3)), i.e. keys
  // 16 q + 8 h32 + r at byte 8 q + r: the order in which the P bytes below
  // are packed.
  const unsigned lofs0 = 2 * C::LOFF + 64 * l32 + 16 * ((2 * h32) ^ ((l32 >> 2) & 3));
  const unsigned lofs1 = 2 * C::LOFF + 64 * l32 + 16 * ((2 * h32 + 1) ^ ((l32 >> 2) & 3));
  auto lfrags = [&](const f16* tile, i32x8 (&lf)[DV / 32]) {
    const char* tb = reinterpret_cast<const char*>(tile);
#pragma unroll
    for (int dvb = 0; dvb < DV / 32; ++dvb) {
      const i32x4 a = *reinterpret_cast<const i32x4*>(tb + lofs0 + 2048 * dvb);
      const i32x4 b = *reinterpret_cast<const i32x4*>(tb + lofs1 + 2048 * dvb);
      lf[dvb] = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };
  // O^T += 2^-kVloExp (V_lo 2^kVloExp)^T P over the 64 keys of a tile (fp8)
  auto pvlo = [&](const i32x8 (&lf)[DV / 32], int qb, const i32x8& p8) {
#pragma unroll
    for (int dvb = 0; dvb < DV / 32; ++dvb) o[qb][dvb] = mfma_f8bf8<127 - kVloExp>(lf[dvb], p8, o[qb][dvb]);
  };
  auto kfrags = [&](const f16* tile, int kb, f16x8 (&kf)[C::NCH], f16x4& kx) {
    const f16* krow = tile + (32 * kb + l32) * C::CW;
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) kf[c] = *reinterpret_cast<const f16x8*>(krow + chunk_off<M>(c) + 8 * h32);
    kx = *reinterpret_cast<const f16x4*>(krow + M + 4 * h32);
  };
  auto score = [&](const f16x8 (&kf)[C::NCH], const f16x4& kx, int qb) {
    return mfma8(kx, qaug[qb], code_dot<M, true>(kf, qf[qb], f32x16{}));
  };
  // P of one 32-key block: fp16 p0 (keys 8 h32 + r), p1 (keys 16 + 8 h32 + r),
  // and their e5m2 bytes (the high byte of each fp16 value, i.e. rounded
  // toward zero to 2 mantissa bits: relative error < 2^-2 on the 2^-11-relative
  // V_lo term) into dwords 4 kb .. 4 kb + 3 of the tile's fp8 B operand.
  auto expo = [&](const f32x16& sc, int qb, f16x8& p0, f16x8& p1, i32x8& p8, int kb) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      p0[r] = (f16)fast_exp2(sc[r]);
      p1[r] = (f16)fast_exp2(sc[r + 8]);
    }
    lsum[qb] += sum8(p0) + sum8(p1);
    const i32x4 u0 = __builtin_bit_cast(i32x4, p0), u1 = __builtin_bit_cast(i32x4, p1);
    p8[4 * kb + 0] = (int)__builtin_amdgcn_perm((unsigned)u0[1], (unsigned)u0[0], 0x07050301u);
    p8[4 * kb + 1] = (int)__builtin_amdgcn_perm((unsigned)u0[3], (unsigned)u0[2], 0x07050301u);
    p8[4 * kb + 2] = (int)__builtin_amdgcn_perm((unsigned)u1[1], (unsigned)u1[0], 0x07050301u);
    p8[4 * kb + 3] = (int)__builtin_amdgcn_perm((unsigned)u1[3], (unsigned)u1[2], 0x07050301u);
  };
  auto stage = [&](int t) { return smem + (t % C::NSTAGE) * C::STAGE; };

  // Any tile: per 32-key block and query block, with masks where needed; the
  // P.V_lo product follows once per query block over the whole tile (the P
  // bytes of skipped blocks stay zero).
  auto compute = [&](const f16* tile, int k0) {
    i32x8 p8[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) p8[qb] = i32x8{};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kbase = k0 + 32 * kb;
      if (kbase >= N || (causal && kbase > qw0 + 32 * QB - 1)) continue;  // wave-uniform
      f16x8 kf[C::NCH];
      f16x4 kx;
      kfrags(tile, kb, kf, kx);
      f16x8 vf[2][DV / 32];
      if (!MAXPASS) vfrags(tile, kb, vf);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int qb0 = qw0 + 32 * qb;
        if (causal && kbase > qb0 + 31) continue;  // wave-uniform
        f32x16 sc = score(kf, kx, qb);
        if ((kbase + 31 >= N) || (causal && kbase + 31 > qb0) ||
            (MD && kbase <= qb0 + 31 && kbase + 31 >= qb0)) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kbase + swap23(acc_row(r, lane));
            if (key >= N || (causal && key > qb0 + l32) || (MD && key == qb0 + l32)) sc[r] = kNegInf;
          }
        }
        if (MAXPASS) {
#pragma unroll
          for (int r = 0; r < 16; ++r) rmax[qb] = fmaxf(rmax[qb], sc[r]);
          continue;
        }
        f16x8 p0, p1;
        expo(sc, qb, p0, p1, p8[qb], kb);
        pv(vf, qb, p0, p1);
      }
    }
    if (!MAXPASS && k0 < N) {
      i32x8 lf[DV / 32];
      lfrags(tile, lf);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        if (!(causal && k0 > qw0 + 32 * qb + 31)) pvlo(lf, qb, p8[qb]);  // wave-uniform
    }
  };

  int next_issue = 0;  // tiles [0, next_issue) have been issued
  auto issue_upto = [&](int t) {
    for (; next_issue <= t && next_issue < nkt; ++next_issue) issue(next_issue);
  };
  // wait until tile t has landed in every wave's share, then publish it
  auto publish = [&](int t) {
    if (next_issue > t + 1)
      wait_vmcnt<NPWX>();  // tile t + 1 may stay in flight (never more than one tile beyond t)
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
  };

  int t = 0;
  issue_upto(1);
  if (!MAXPASS) {
    // ---- tiles whose 64 keys are unmasked for every query of the workgroup
    // (with the diagonal masked, the tiles from the workgroup's first query on
    // take the masked path)
    const int nfull = min(nkt, ((causal || MD) ? q0 : N) / C::KT);
    for (; t < nfull; ++t) {
      publish(t);
      issue_upto(t + C::NSTAGE - 1);
      const f16* tile = stage(t);
      if (!C::PIPE) {  // registers too tight for two blocks in flight: one block at a time
        i32x8 p8[QB];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          f16x8 kf[C::NCH];
          f16x4 kx;
          kfrags(tile, kb, kf, kx);
          f32x16 sc[QB];
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) sc[qb] = score(kf, kx, qb);
          f16x8 vf[2][DV / 32];
          vfrags(tile, kb, vf);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            f16x8 p0, p1;
            expo(sc[qb], qb, p0, p1, p8[qb], kb);
            pv(vf, qb, p0, p1);
          }
        }
        i32x8 lf[DV / 32];
        lfrags(tile, lf);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) pvlo(lf, qb, p8[qb]);
        continue;
      }
      // Both 32-key blocks of the tile in flight: block 1's score MFMAs are
      // independent of block 0's exponentials, and block 0's P.V MFMAs of
      // block 1's, so the scheduler can overlap them (explicit
      // sched_group_barrier patterns measured 5% slower than its own order).
      f16x8 kf0[C::NCH], kf1[C::NCH];
      f16x4 kx0, kx1;
      kfrags(tile, 0, kf0, kx0);
      kfrags(tile, 1, kf1, kx1);
      f32x16 sc0[QB], sc1[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sc0[qb] = score(kf0, kx0, qb);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) sc1[qb] = score(kf1, kx1, qb);
      f16x8 pa[QB][2], pb[QB][2];
      i32x8 p8[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) expo(sc0[qb], qb, pa[qb][0], pa[qb][1], p8[qb], 0);
      f16x8 vf0[2][DV / 32], vf1[2][DV / 32];
      vfrags(tile, 0, vf0);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) pv(vf0, qb, pa[qb][0], pa[qb][1]);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) expo(sc1[qb], qb, pb[qb][0], pb[qb][1], p8[qb], 1);
      vfrags(tile, 1, vf1);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) pv(vf1, qb, pb[qb][0], pb[qb][1]);
      i32x8 lf[DV / 32];
      lfrags(tile, lf);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) pvlo(lf, qb, p8[qb]);
    }
  }
  // ---- remaining tiles (masked ones; all of them in the exact-max pass)
  for (; t < nkt; ++t) {
    publish(t);
    issue_upto(t + C::NSTAGE - 1);
    compute(stage(t), t * C::KT);
  }
}

template <int M, int DV, bool MD, bool SM>
__global__ __launch_bounds__((64 * FwdCfg<M, DV, SM>::WAVES))
__attribute__((amdgpu_waves_per_eu(FwdCfg<M, DV, SM>::WAVES_PER_EU, FwdCfg<M, DV, SM>::WAVES_PER_EU)))
void attn_fwd_kernel(f16* __restrict__ qa, const f16* __restrict__ ka, const f16* __restrict__ vt,
                     const uint8_t* __restrict__ vlo,
                     const float4* __restrict__ tstat, f16* __restrict__ out, float* __restrict__ lse, int N, int NP,
                     int H, int D, int BH, int causal) {
  using C = FwdCfg<M, DV, SM>;
  constexpr int QB = C::QB;
  __shared__ __align__(16) f16 smem[C::NSTAGE * C::STAGE];
  const int tid = threadIdx.x, lane = tid & 63, h32 = lane >> 5, l32 = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, scalar
  const int nqb = (N + C::QW - 1) / C::QW;
  int bh, blk;
  if (!(causal ? xcd_map_lpt(nqb, BH, bh, blk) : xcd_map(nqb, BH, bh, blk))) return;
  const int qblk = causal ? nqb - 1 - blk : blk;  // longest rows first
  const int q0 = qblk * C::QW, qw0 = q0 + 32 * QB * w;
  const int b = bh / H, h = bh - b * H;
  const int64_t rowbase = (int64_t)bh * N;
  const int64_t vbase = (int64_t)bh * DV * NP;  // V_hi^T rows (halves) and V_lo blocks (bytes) of the head

  f16x8 qf[QB][C::NCH];
  f16x4 qaug[QB];
  float R[QB], lsum[QB], rmax[QB];
  float4 ts[QB];
  f32x16 o[QB][DV / 32];
  bool any_gap = false;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int q = qw0 + 32 * qb + l32;
    qaug[qb] = f16x4{};
#pragma unroll
    for (int c = 0; c < C::NCH; ++c) qf[qb][c] = f16x8{};
    ts[qb] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q < N) {
      const f16* qrow = qa + (rowbase + q) * C::CW;
#pragma unroll
      for (int c = 0; c < C::NCH; ++c) qf[qb][c] = *reinterpret_cast<const f16x8*>(qrow + chunk_off<M>(c) + 8 * h32);
      qaug[qb] = *reinterpret_cast<const f16x4*>(qrow + M + 4 * h32);
      ts[qb] = tstat[rowbase + q];
      any_gap = any_gap || ts[qb].z > kGapExact;
    }
    R[qb] = ts[qb].y;
    lsum[qb] = 0.f;
    rmax[qb] = kNegInf;
#pragma unroll
    for (int i = 0; i < DV / 32; ++i) o[qb][i] = f32x16{};
  }
  const int kend = causal ? min(N, q0 + C::QW) : N;
  // the query operands are loaded under a condition: wait on every path, or the
  // compiler waits for them inside the tile loop, draining the in-flight DMA
  wait_vmcnt<0>();

  if (__syncthreads_or(any_gap)) {
    // pass 1: exact row max of the base-2 exponent without the reference
    f16x4 qa0[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      qa0[qb] = qaug[qb];
      if (h32 == 0) { qa0[qb][2] = (f16)0.f; qa0[qb][3] = (f16)0.f; }
    }
    fwd_pass<M, DV, true, MD, SM>(ka, vt, vlo, rowbase, vbase, N, NP, causal, kend, q0, qw0, smem, qf, qa0, o, lsum, rmax);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const float m = fmaxf(rmax[qb], __shfl_xor(rmax[qb], 32));
      R[qb] = (qw0 + 32 * qb + l32 < N && m > kNegInf) ? m : 0.f;  // a row without keys keeps 0
      f16 rh, rl;
      split_hi_lo(-R[qb], rh, rl);
      if (h32 == 0) { qaug[qb][2] = rh; qaug[qb][3] = rl; }
    }
    __syncthreads();  // every wave is done with the stages before they are refilled
  }
  fwd_pass<M, DV, false, MD, SM>(ka, vt, vlo, rowbase, vbase, N, NP, causal, kend, q0, qw0, smem, qf, qaug, o, lsum, rmax);

#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int q = qw0 + 32 * qb + l32;
    const float ltot = lsum[qb] + __shfl_xor(lsum[qb], 32);
    if (q < N) {
      const float inv = ltot > 0.f ? 1.0f / ltot : 0.f;
      f16* orow = out + ((int64_t)b * N + q) * D + h * DV;
#pragma unroll
      for (int dvb = 0; dvb < DV / 32; ++dvb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          f16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (f16)(o[qb][dvb][4 * g + e] * inv);
          *reinterpret_cast<f16x4*>(orow + 32 * dvb + 8 * g + 4 * h32) = v;
        }
      if (h32 == 0) {
        const float l2 = ltot > 0.f ? R[qb] + fast_log2(ltot) : -kFltMax;  // lse - b
        lse[rowbase + q] = ltot > 0.f ? l2 + ts[qb].x : -kFltMax;
        // the query row's affine block becomes the backward's {1, 1, -(lse - b)}:
        // this wave was its only reader (0 for a row without keys, whose
        // scores the backward masks)
        f16 bh_, bl_;
        split_hi_lo(ltot > 0.f ? -l2 : 0.f, bh_, bl_);
        *reinterpret_cast<f16x2*>(qa + (rowbase + q) * C::CW + M + 2) = f16x2{bh_, bl_};
      }
    }
  }
}

template <int M, int DV, bool SM>
static hipError_t launch_attn_fwd_c(const Dims& d, const ProjBuffers& p, f16* out, float* lse, hipStream_t s) {
  using C = FwdCfg<M, DV, SM>;
  const dim3 grid(xcd_grid((d.N + C::QW - 1) / C::QW, d.B * d.H));
  if (d.mask_diag)
    MORPHO_KLAUNCH((attn_fwd_kernel<M, DV, true, SM>), grid, dim3(64 * C::WAVES), 0, s, p.qa, p.ka, p.vt, p.vlo,
                       p.tstat, out, lse, d.N, d.NP, d.H, d.D, d.B * d.H, d.causal);
  else
    MORPHO_KLAUNCH((attn_fwd_kernel<M, DV, false, SM>), grid, dim3(64 * C::WAVES), 0, s, p.qa, p.ka, p.vt,
                       p.vlo, p.tstat, out, lse, d.N, d.NP, d.H, d.D, d.B * d.H, d.causal);
  return hipGetLastError();
}

template <int M, int DV>
static hipError_t launch_attn_fwd_t(const Dims& d, const ProjBuffers& p, f16* out, float* lse, hipStream_t s) {
  using C = FwdCfg<M, DV, false>;
  if constexpr (FwdCfg<M, DV, true>::SMALL) {
    const int64_t wgs = (int64_t)((d.N + C::QW - 1) / C::QW) * d.B * d.H;
    if (wgs < 2 * 256) return launch_attn_fwd_c<M, DV, true>(d, p, out, lse, s);
  }
  return launch_attn_fwd_c<M, DV, false>(d, p, out, lse, s);
}

}  // namespace morpho
