// Internal launcher interface shared by the kernel translation units and the
// C ABI layer. Nothing here is exported from the shared library.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace morpho {

// Cube projections phi(z) (cube.cuh:9-17 of the reference): sigmoid (the
// default), clamp((z + 1) / 2, 0, 1), and z itself.
constexpr int kProjSigmoid = 0, kProjHardTanh01 = 1, kProjIdentity = 2;

struct Dims {
  int B, N, D, H, M, DV;  // batch, tokens, model dim, heads, cube_m, head_dim_v
  int NP;                 // N rounded up to a multiple of 64: row length of the V^T layout
  int64_t T;              // B * N tokens
  int HM;                 // H * M projection columns
  int CW;                 // 2 * M + 8: code row width (hi/lo split codes + affine augmentation)
  float scale;
  int causal;
  int mask_diag;          // drop key j == query i
  int proj;               // cube projection: kProjSigmoid, kProjHardTanh01 or kProjIdentity
  int det;                // deterministic backward: dq and row sums from per-key-block partials
  // Column order of the forward projection's B operand (wt rows): tiles of
  // PBN columns; when PCPT > 0 tile j holds code columns [j PCPT, (j+1) PCPT)
  // then value columns [j PVPT, (j+1) PVPT), so every tile does the same
  // epilogue work; PCPT == 0 keeps the natural order [W_phi | W_V].
  int PBN, PCPT, PVPT;
};

// Original [W_phi | W_V] column of local column lc of projection tile tn.
__host__ __device__ inline int proj_col(const Dims& d, int tn, int lc) {
  if (d.PCPT == 0) return tn * d.PBN + lc;
  return lc < d.PCPT ? tn * d.PCPT + lc : d.HM + tn * d.PVPT + (lc - d.PCPT);
}
// wt row (position in the projection's column order) of original column c.
__host__ __device__ inline int proj_row(const Dims& d, int c) {
  if (d.PCPT == 0) return c;
  if (c < d.HM) return (c / d.PCPT) * d.PBN + c % d.PCPT;
  const int v = c - d.HM;
  return (v / d.PVPT) * d.PBN + d.PCPT + v % d.PVPT;
}

// Products of the forward projection; the forward workspace holds exactly these.
//
// Code rows carry each code as an fp16 hi/lo pair (CW = 2M + 8 columns):
//   query row  [phi_hi | 1, 1, -R_hi, -R_lo, 0 x4 | phi_lo]
//              (after the forward: [.. | 1, 1, -(lse - b) hi, lo, 0 x4 | ..],
//               the backward's row reference)
//   key row    [kc_hi  | b_hi, b_lo, 1, 1, 0 x4   | kc_lo ]
// The attention kernels contract the chunk pairs (kc_hi, phi_hi), (kc_hi,
// phi_lo), (kc_lo, phi_hi) and the affine blocks in one MFMA accumulator,
// which yields (to ~2^-22) the exact base-2 exponent. The 8-wide affine block
// sits right after the first M codes so that a 32-row transposed read of the
// query row starting at column 32*floor(M/32) sees the constant-1 column at
// row M, which the backward uses to form column sums of dS in the same MFMA
// as the key-side code gradient. Here kc = c1 * G * phi, c1 = 2 scale log2e, G = gate_q * gate_k, b the token
// bias -scale log2e sum_c G_c phi_c and R the per-query softmax reference.
struct ProjBuffers {
  _Float16* qa;    // [B*H, N, CW] query rows (columns 0..M-1 are phi_hi, M+8..2M+7 phi_lo)
  _Float16* ka;    // [B*H, N, CW] key rows
  _Float16* vt;    // [B*H, DV, NP] values X W_V per head, transposed, rounded to fp16 (V_hi);
                   // zero for tokens N..NP-1
  uint8_t* vlo;    // [B*H, NP/64, DV, 64] the rounding remainders V - V_hi, times 2^kVloExp, as
                   // e4m3 bytes rounded toward zero; one [DV][64] block per 64-key tile, whose row holds key
                   // 16 q + 8 h + r at byte 32 h + 8 q + r (h < 2, q < 4, r < 8); zero past N
  float4* tstat;   // [B*H, N] {b, R, gap, t}: token bias, softmax reference, bound gap and the
                   // self score t = s_ii - b (all base 2; 2^(t + b - lse) is the diagonal weight
                   // the backward's correction needs)
  _Float16* wt;    // [H*M + D, D] transposed [W_phi | W_V]
  _Float16* wcat;  // [D, H*M + D] [W_phi | W_V] as one row-major matrix
};

// V_lo is stored as e4m3 of V_lo * 2^kVloExp (|V_lo| <= 2^-11 |V|, so the
// stored magnitude is about 2|V|, clamped to the e4m3 range at 448), and the
// P.V_lo product undoes the factor through the MFMA's operand scale.
constexpr int kVloExp = 12;
// Byte position of key k (0..63) within a 64-byte V_lo row.
__host__ __device__ inline int vlo_pos(int k) { return 32 * ((k >> 3) & 1) + 8 * (k >> 4) + (k & 7); }

struct BwdBuffers {
  _Float16* aug;   // [B*H, N, 8] per query: the dO rows' affine block {-delta hi, lo, 0 x6}
  float* dq;       // [B*H, N, M] sum_j dS_ij phi_j (query side), fp32 atomics
  float* dk;       // [B*H, N, M] sum_i dS_ij phi_i (key side)
  float* dcb;      // [B*H, N]    sum_i dS_ij
  float* dr;       // [B*H, N, 2] {r, P_ii}: r = sum_j dS_ij, the row sums of the rounded dS (0 in
                   //             exact arithmetic, fp32 atomics), and the diagonal weight
                   //             P_ii (0 when the diagonal is masked), written by bwd_prep
  _Float16* dzv;   // [T, H*M + D] dZ | dV
  float* gpart;    // [n_gate_blocks, H*M] partial sums of phi (2 dk - dcb), the gate factor dG
  float* wpart;    // [tiles, pieces, bt, bt] fp32 partials of [dW_phi | dW_V] tiles (BwdGemmPlan)
  float* dqpart;   // deterministic mode only (else null): [nkb, B*H, NQ, M] per-key-block dq sums
  float* drpart;   //                                      [nkb, B*H, NQ] per-key-block row sums
};

// Layout of the deterministic backward's partials: KW keys per key block,
// nkb key blocks, rows padded to nq (N rounded up to the query step).
struct DetLayout {
  int kw, nkb, nq;
};

constexpr int kGateTokensPerBlock = 64;

// kernels_proj.hip
hipError_t launch_transpose_weights(const Dims& d, const _Float16* W_phi, const _Float16* W_V, _Float16* wt,
                                    _Float16* wcat, hipStream_t s);
hipError_t launch_proj_fwd(const Dims& d, const _Float16* X, const _Float16* gate_q, const _Float16* gate_k,
                           const ProjBuffers& p, hipStream_t s);
// With row_corr (softmax attention) the row sums and diagonal weights in g.dr
// cancel the noise of the rows' delta at the diagonal; without (soft
// aggregation) dq, dk and dcb are used as they are.
hipError_t launch_proj_bwd_elem(const Dims& d, const _Float16* gate_q, const _Float16* gate_k, const ProjBuffers& p,
                                const BwdBuffers& g, bool row_corr, hipStream_t s);
hipError_t launch_bwd_gemm(const Dims& d, const ProjBuffers& p, const BwdBuffers& g, const _Float16* X, _Float16* dX,
                           hipStream_t s);
hipError_t launch_dw_reduce(const Dims& d, const BwdBuffers& g, const _Float16* gate_q, const _Float16* gate_k,
                            _Float16* dW_phi, _Float16* dW_V, _Float16* d_gate_q, _Float16* d_gate_k, hipStream_t s);
// Work decomposition of the backward GEMM launch: one round of kGemmSlots
// workgroups (the CUs of an MI355X; twice as many with 128 x 128 tiles, two
// per CU). Workgroups [0, n_a), n_a / 8 per XCD (workgroup id % 8), compute g
// whole dX tiles each; the next 8 ceil(tiles_w p / 8) each compute one piece
// j < p of a dW tile t (the tile's kw token k-steps split into p near-equal
// ranges; an XCD's workgroups take a contiguous run of the pieces in (j, t)
// order, so they share token ranges). g and p are chosen so that both kinds take about the
// same number of k-steps. Piece j stores an fp32 tile partial that dw_reduce
// adds in piece order, so the result does not depend on timing.
constexpr int kGemmSlots = 256;
struct BwdGemmPlan {
  int bt;                   // tile edge: 256, or 128 when that finishes sooner (few tiles)
  int n_dx, ntn_x, kx;      // dX tiles, dX column tiles, k-steps per dX tile
  int tiles_w, ntn_w, kw;   // dW tiles, dW column tiles, k-steps per dW tile (all tokens)
  int g, n_a;               // dX tiles per type-A workgroup, type-A workgroups
  int p;                    // pieces per dW tile (tiles_w p type-B workgroups and partials)
};
BwdGemmPlan bwd_gemm_plan(const Dims& d);
// token k-step where piece j of a dW tile's kw k-steps starts (j = p: the end)
__host__ __device__ inline int dw_piece_k0(int kw, int p, int j) { return (int)((int64_t)kw * j / p); }

// kernels_attn_fwd.hip (cube_m 16, 32) and kernels_attn_fwd_m64.hip
hipError_t launch_attn_fwd(const Dims& d, const ProjBuffers& p, _Float16* out, float* lse, hipStream_t s);
hipError_t launch_attn_fwd_m64(const Dims& d, const ProjBuffers& p, _Float16* out, float* lse, hipStream_t s);

// kernels_attn.hip
hipError_t launch_bwd_prep(const Dims& d, const ProjBuffers& p, const _Float16* grad_out, const _Float16* out,
                           const float* lse, const BwdBuffers& g, int write_q, hipStream_t s);
DetLayout attn_bwd_det_layout(const Dims& d);
hipError_t launch_dq_det_reduce(const Dims& d, const BwdBuffers& g, hipStream_t s);
hipError_t launch_attn_bwd(const Dims& d, const ProjBuffers& p, const _Float16* grad_out, const _Float16* gate_q,
                           const _Float16* gate_k, const BwdBuffers& g, hipStream_t s);

// kernels_soft.hip: soft tropical aggregation (out = sgn tau ln sum_j
// exp(sgn (s + v) / tau)). `tau` is a device pointer to one float; sgn is +1
// (dilation) or -1 (erosion); zb is the fp32 base-2 normaliser [B*H, N, DV].
// State of the product-form fast path, kept in the soft forward workspace
// after the projection buffers.
struct SoftState {
  float* vmax;  // [B*H, DV] max over keys of V
  float* vmin;  // [B*H, DV] min over keys of V
  float* arow;  // [B*H, N] row reference A_i (maximum of sgn log2e s_ij / tau over the row's keys)
  int* flag;    // nonzero: some output failed the product form's check; the element-wise path ran
  uint16_t* fth;  // [B*H, DV, NP] bf16 hi of F = 2^(w - B_c), keys contiguous (zero past N)
  uint16_t* ftl;  // [B*H, DV, NP] bf16 lo of F
};
// Element-wise kernels; with run_flag they do nothing unless *run_flag != 0.
hipError_t launch_soft_fwd(const Dims& d, const ProjBuffers& p, const float* tau, int sgn, _Float16* out, float* zb,
                           const int* run_flag, hipStream_t s);
hipError_t launch_soft_colext(const Dims& d, const ProjBuffers& p, const SoftState& st, hipStream_t s);
hipError_t launch_soft_fvals(const Dims& d, const ProjBuffers& p, const float* tau, int sgn, const SoftState& st,
                             hipStream_t s);
hipError_t launch_soft_fwd_fast(const Dims& d, const ProjBuffers& p, const float* tau, int sgn, const SoftState& st,
                                _Float16* out, float* zb, hipStream_t s);
// With st non-null (the product form will run) the prep also writes G =
// dO 2^(A_i + B_c - zb) as bf16 hi / lo pairs, [B*H, N, DV] each, to gh / gl.
hipError_t launch_soft_bwd_prep(const Dims& d, const _Float16* grad_out, const float* zb, const BwdBuffers& g,
                                float* part, const float* tau, int sgn, const SoftState* st, uint16_t* gh,
                                uint16_t* gl, hipStream_t s);
hipError_t launch_soft_bwd(const Dims& d, const ProjBuffers& p, const _Float16* grad_out, const float* zb,
                           const float* tau, int sgn, const BwdBuffers& g, float* part, const int* run_flag,
                           hipStream_t s);
hipError_t launch_soft_bwd_fast(const Dims& d, const ProjBuffers& p, const _Float16* grad_out, const float* zb,
                                const float* tau, int sgn, const SoftState& st, const uint16_t* gh,
                                const uint16_t* gl, const BwdBuffers& g, float* part, hipStream_t s);
int soft_bwd_exact_slots(const Dims& d);  // the element-wise backward's share of soft_bwd_slots
hipError_t launch_fill_zero(float* p, int n, hipStream_t s);
hipError_t launch_set_flag(int* p, int v, hipStream_t s);
hipError_t launch_soft_tau_reduce(const float* prep, int nprep, const float* bwd, int nbwd, const float* tau, int sgn,
                                  float* dtau, hipStream_t s);
int soft_prep_blocks(const Dims& d);  // partial sums written by the prep (one float each)
int soft_bwd_slots(const Dims& d);    // workgroup slots of both backward kernels (two floats each)

// Timing hooks (capi.hip). When timing is enabled, timing_begin opens a
// record (a name and two events) for the launcher call that follows, and the
// kernel launches inside it take the record's events through
// hipExtLaunchKernel: the first launch takes the start event, every launch the
// stop event, so the record spans the launcher's kernels. The events are bound
// to the dispatches themselves; no marker packets run between kernels (marker
// events had left about 10 us between consecutive kernels).
void timing_begin(const char* name, hipStream_t s);
void timing_end(hipStream_t s);
hipEvent_t timing_take_start();  // the open record's start event, for its first launch only (else null)
hipEvent_t timing_stop_event();  // the open record's stop event (null without an open record)

// Every kernel launch of the library: hipLaunchKernelGGL semantics (errors are
// read with hipGetLastError), with the timing record's events when one is open.
#define MORPHO_KLAUNCH(KERNEL, GRID, BLOCK, SHMEM, STREAM, ...)                                       \
  hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, SHMEM, STREAM, ::morpho::timing_take_start(),            \
                        ::morpho::timing_stop_event(), 0u, __VA_ARGS__)

// Instantiations of a launcher template FN<M, DV> for every supported shape.
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

}  // namespace morpho
