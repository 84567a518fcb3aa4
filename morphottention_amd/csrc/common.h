// Device-side building blocks for gfx950 (CDNA4, wave64).
//
// MFMA lane layouts used throughout (checked on MI355X):
//   v_mfma_f32_32x32x16_f16  A: lane l holds A[l%32][8*(l/32) + j], j = 0..7
//                            B: lane l holds B[8*(l/32) + j][l%32]
//                            C: lane l, reg r holds C[8*(r/4) + 4*(l/32) + r%4][l%32]
//   v_mfma_f32_32x32x8_f16   as above with 4 values per lane, k = 4*(l/32) + j.
//   v_mfma_scale_f32_32x32x64_f8f6f4 (fp8 operands, 32 bytes per lane)
//                            A: lane l holds A[l%32][32*(l/32) + j], j = 0..31
//                            B: lane l holds B[32*(l/32) + j][l%32]; C as above.
//                            Each operand's E8M0 scale s multiplies by 2^(s-127).
//   fp8 formats are OCP: e4m3 (bias 7, 0x7f is NaN, so conversions of values
//   beyond 448 must be clamped first) and e5m2 (bias 15, the high byte of fp16).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace morpho {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_inff();
constexpr float kFltMax = 3.402823466e38f;

__device__ __forceinline__ f32x16 mfma16(const f16x8& a, const f16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma8(const f16x4& a, const f16x4& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, c, 0, 0, 0);
}
// C += 2^(SA - 127) A B for an e4m3 A [32 x 64] and an e5m2 B [64 x 32].
template <int SA>
__device__ __forceinline__ f32x16 mfma_f8bf8(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0 /*A e4m3*/, 1 /*B e5m2*/, 0, SA, 0, 127);
}
// v_mfma_f32_16x16x32_f16: A lane l holds A[l%16][8*(l/16) + j], B lane l holds
// B[8*(l/16) + j][l%16], C lane l reg r holds C[4*(l/16) + r][l%16].
__device__ __forceinline__ f32x4 mfma16x16(const f16x8& a, const f16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Row (within a 32-row MFMA block) held in accumulator register r by lane l.
__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Swap bits 2 and 3 of a row index in 0..31. Loading the A-operand rows of a
// 32x32 product in this order makes the accumulator registers 0..7 / 8..15 of
// lane l hold rows 8*(l/32)+0..7 / 16+8*(l/32)+0..7 in natural order, which is
// exactly the B-operand layout of the next product that contracts over them.
__device__ __forceinline__ int swap23(int x) { return (x & ~12) | ((x & 4) << 1) | ((x & 8) >> 1); }

__device__ __forceinline__ f16x4 lds_read_tr4(const f16* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  return __builtin_bit_cast(f16x4, v);
}

// MFMA 32x32x16 operand from an LDS tile whose contraction index runs along
// its rows: value(mn, k) = tile[(k0 + k) * stride + mn0 + mn], mn = lane%32.
// Two ds_read_b64_tr_b16 per lane; stride must be a multiple of 4 halves.
__device__ __forceinline__ f16x8 frag_kmajor(const f16* tile, int stride, int k0, int mn0, int lane) {
  const int g = lane >> 4;
  const int row = k0 + 8 * (g >> 1) + ((lane & 15) >> 2);
  const int col = mn0 + 16 * (g & 1) + 4 * (lane & 3);
  const f16* p = tile + row * stride + col;
  f16x4 lo = lds_read_tr4(p);
  f16x4 hi = lds_read_tr4(p + 4 * stride);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// MFMA 16x16x32 operand from an LDS tile whose contraction index runs along
// its rows: value(mn, k) = tile[(k0 + k) * stride + mn0 + mn], mn = lane%16,
// k = 8*(lane/16) + j.
__device__ __forceinline__ f16x8 frag16_kmajor(const f16* tile, int stride, int k0, int mn0, int lane) {
  const int g = lane >> 4;
  const int row = k0 + 8 * g + ((lane & 15) >> 2);
  const int col = mn0 + 4 * (lane & 3);
  const f16* p = tile + row * stride + col;
  f16x4 lo = lds_read_tr4(p);
  f16x4 hi = lds_read_tr4(p + 4 * stride);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// MFMA 32x32x16 operand from an LDS tile whose contraction index is
// contiguous: value(mn, k) = tile[row * stride + k0 + k] with `row` the tile
// row this lane supplies. One 16-byte read.
__device__ __forceinline__ f16x8 frag_kcontig(const f16* tile, int stride, int row, int k0, int lane) {
  return *reinterpret_cast<const f16x8*>(tile + row * stride + k0 + 8 * (lane >> 5));
}
__device__ __forceinline__ f16x4 frag4_kcontig(const f16* tile, int stride, int row, int k0, int lane) {
  return *reinterpret_cast<const f16x4*>(tile + row * stride + k0 + 4 * (lane >> 5));
}

// hi = fp16(x), lo = fp16(x - hi): hi + lo carries x to ~2^-22. The pair is
// only consistent if hi and lo are formed from one and the same fp32 x, so x
// is made opaque to the compiler: it may otherwise evaluate x twice (e.g. a
// product once fused into the subtraction, once rounded, or a branch
// duplicated), and at an exact fp16 rounding tie the two evaluations land on
// different sides (hi + lo then misses x by one fp16 ulp). The fp16
// conversions themselves (v_cvt_f16_f32, v_cvt_pk_f16_f32) round ties alike.
__device__ __forceinline__ void split_exact(float x, f16& hi, f16& lo) {
  asm("" : "+v"(x));  // not volatile: an opaque copy, free to be scheduled
  hi = (f16)x;
  lo = (f16)(x - (float)hi);
}
// as split_exact, with x clamped to the fp16 range first
__device__ __forceinline__ void split_hi_lo(float x, f16& hi, f16& lo) {
  split_exact(fminf(fmaxf(x, -60000.f), 60000.f), hi, lo);
}

__device__ __forceinline__ f16x8 pack8(const f32x16& v, int base) {
  f16x8 r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = (f16)v[base + j];
  return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// s_waitcnt on the vector-memory counter only (gfx9 encoding: vmcnt[3:0],
// expcnt[6:4] = 7 and lgkmcnt[11:8] = 15 mean "no wait", vmcnt[5:4] at [15:14]).
template <int CNT>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(CNT >= 0 && CNT < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((CNT & 15) | (7 << 4) | (15 << 8) | ((CNT >> 4) << 14));
}

// 16 bytes per lane from global memory straight into LDS: lane l of the wave
// writes LDS byte address lds_addr + 16 l (lds_addr wave-uniform). Issued as
// inline asm so that the compiler does not order every later LDS read after
// it: the callers wait for these loads explicitly (wait_vmcnt) before the
// barrier that publishes a stage.
__device__ __forceinline__ void lds_dma16(const f16* g, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}

// DMA of one 16-byte piece per lane from sbase + voff (32-bit unsigned lane
// offset, 64-bit wave-uniform base) to LDS byte address lds_addr + 16 lane.
__device__ __forceinline__ void lds_dma16_so(const void* sbase, unsigned voff, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}

// 4 bytes per lane from global memory straight into LDS: lane l writes LDS
// byte address lds_addr + 4 l (lds_addr wave-uniform).
__device__ __forceinline__ void lds_dma4(const float* g, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}

// s_waitcnt: vector-memory count CNT and LDS count 0 (gfx9 encoding).
template <int CNT>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  static_assert(CNT >= 0 && CNT < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((CNT & 15) | (7 << 4) | (0 << 8) | ((CNT >> 4) << 14));
}

// 1 / (1 + e^-z) with the hardware reciprocal (1 ulp; the argument is >= 1
// or +inf, whose reciprocal is 0) instead of the ten-instruction IEEE division
__device__ __forceinline__ float sigmoidf_(float z) { return __builtin_amdgcn_rcpf(1.0f + __expf(-z)); }

// Cube projection phi(z) and its derivative written in terms of phi: sigmoid,
// phi (1 - phi); clamp((z + 1) / 2, 0, 1), 1/2 where the clamp is inactive
// (0 < phi < 1, i.e. -1 < z < 1); identity, 1. `proj` is uniform.
__device__ __forceinline__ float cube_project(float z, int proj) {
  if (proj == 0) return sigmoidf_(z);
  if (proj == 1) return fminf(1.0f, fmaxf(0.0f, 0.5f * (z + 1.0f)));
  return z;
}
__device__ __forceinline__ float cube_project_grad(float phi, int proj) {
  if (proj == 0) return phi * (1.0f - phi);
  if (proj == 1) return (phi > 0.0f && phi < 1.0f) ? 0.5f : 0.0f;
  return 1.0f;
}


// Column offset of the c-th 16-wide code chunk of a code row: chunks 0 ..
// M/16 - 1 hold the hi parts, M/16 .. M/8 - 1 the lo parts (the 8-wide affine
// block sits at [M, M + 8)).
template <int M>
__device__ __forceinline__ constexpr int chunk_off(int c) {
  return c < M / 16 ? 16 * c : 16 * c + 8;
}
// The exponent's code part, sum_c kc_c phi_c to ~2^-22, from the hi / lo
// chunks of a key (kf) and a query (qf) operand: hi.hi + hi.lo + lo.hi.
// KEY_A: the key chunks are the A operand (forward: rows = keys), else the
// query chunks are (backward: rows = queries).
template <int M, bool KEY_A>
__device__ __forceinline__ f32x16 code_dot(const f16x8 (&kf)[M / 8], const f16x8 (&qf)[M / 8], f32x16 acc) {
  constexpr int HC = M / 16;
  auto mm = [&](const f16x8& k, const f16x8& q) { acc = KEY_A ? mfma16(k, q, acc) : mfma16(q, k, acc); };
#pragma unroll
  for (int i = 0; i < HC; ++i) mm(kf[i], qf[i]);
#pragma unroll
  for (int i = 0; i < HC; ++i) mm(kf[i], qf[HC + i]);
#pragma unroll
  for (int i = 0; i < HC; ++i) mm(kf[HC + i], qf[i]);
  return acc;
}

// The exponent's code part from the hi chunks alone (hi.hi): fp16 codes, so
// ~2^-11 relative per term instead of ~2^-22.
template <int M, bool KEY_A>
__device__ __forceinline__ f32x16 code_dot_hi(const f16x8 (&kf)[M / 8], const f16x8 (&qf)[M / 8], f32x16 acc) {
#pragma unroll
  for (int i = 0; i < M / 16; ++i) acc = KEY_A ? mfma16(kf[i], qf[i], acc) : mfma16(qf[i], kf[i], acc);
  return acc;
}

// Chunk swizzle of a dS^T tile (rows of RB = 128 or 64 bytes: one key's dS
// over a 64- or 32-query step). It is written with ds_write_b128, which
// serves 8 consecutive lanes per cycle within a 128-byte bank window (a
// probe under rocprofv3: an XOR pattern conflict-free for b128 reads cost 16
// LDS cycles per write, 8 of them conflicts), and read with the transposing
// 16x16x32 pattern (ds_read_b64_tr_b16 of rows {r..r+3, r+8..r+11} x 2
// chunks). Each aligned group of 8 rows takes 8 (RB = 128) or, per row
// parity, 4 (RB = 64) distinct chunks, and rows r and r + 8 differ in the
// chunk pair the transposing read touches.
template <int RB>
__device__ __forceinline__ int sswz(int r) {
  static_assert(RB == 64 || RB == 128, "dS^T row bytes");
  if constexpr (RB == 128) return (r & 7) ^ (((r >> 3) & 1) << 2);
  else return ((r >> 1) & 3) ^ (((r >> 3) & 1) << 1);
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
// Same XCD per head, but block-major within an XCD: for causal problems block
// 0 is the longest, so all heads' long blocks start first (longest processing
// time first), and the short ones fill in at the end.
__device__ __forceinline__ bool xcd_map_lpt(int nblk, int BH, int& bh, int& blk) {
  const int i = blockIdx.x, xcd = i & 7, slot = i >> 3, hx = (BH + 7) / 8;
  bh = 8 * (slot % hx) + xcd;
  blk = slot / hx;
  return bh < BH;
}
__host__ inline unsigned xcd_grid(int nblk, int BH) { return 8u * (unsigned)((BH + 7) / 8) * (unsigned)nblk; }

}  // namespace morpho
