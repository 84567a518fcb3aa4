// C ABI of the MI355X morpho-attention library (declared in include/morphottention.h).
//
// Argument checks follow the reference's TORCH_CHECKs
// (packages/morphottention/csrc/cuda/attention/attention.cpp:9-38,
//  attention.cu:491-495,532-538) with the same messages, but return a status
// code with the message available from morpho_last_error().
#include <atomic>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/morphottention.h"
#include "internal.h"

#define MORPHO_EXPORT extern "C" __attribute__((visibility("default")))

namespace morpho {
namespace {

thread_local std::string g_last_error;

struct TimingRec {
  const char* name;
  hipEvent_t start, stop;
  bool bound;  // a launch took the start event (the record then has a measurement)
};
// Timing state is process-wide: autograd runs the backward on its own thread.
std::atomic<bool> g_timing{false};
std::mutex g_timing_mu;
std::string g_timing_only;         // guarded by g_timing_mu; empty: every launcher
std::vector<TimingRec> g_recs;     // guarded by g_timing_mu
std::vector<hipEvent_t> g_pool;    // guarded by g_timing_mu
thread_local int g_open_rec = -1;  // index of this thread's open record

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

size_t align_up(size_t x) { return (x + 255) & ~size_t(255); }

// Validates sizes and fills Dims; returns MORPHO_OK or an error (message set).
int make_dims(int64_t B, int64_t N, int64_t D, int64_t H, int64_t M, float scale, int causal, Dims& d) {
  if (B <= 0 || N <= 0 || D <= 0 || H <= 0) return fail(MORPHO_ERR_INVALID_ARGUMENT, "Invalid dimensions");
  if (D % H != 0) return fail(MORPHO_ERR_INVALID_ARGUMENT, "D must be divisible by H");
  const int64_t DV = D / H;
  if (M != 16 && M != 32 && M != 64)
    return fail(MORPHO_ERR_UNSUPPORTED, "cube_m must be 16, 32 or 64 (got %lld)", (long long)M);
  if (DV != 32 && DV != 64 && DV != 128)
    return fail(MORPHO_ERR_UNSUPPORTED, "head_dim_v = D / H must be 32, 64 or 128 (got %lld)", (long long)DV);
  // Every launch's grid must stay below 2^32 work-items (the dispatch
  // packet's 32-bit grid size): the element-wise kernels run one thread per
  // 8 (token, feature) elements (T D / 8), the backward's gate kernel 16 per
  // token, the deterministic dq reduction one per 4 (token, head, code)
  // values; the bounds below keep each under 2^31. They sit near what fits in
  // memory anyway (T D = 2^34 is a 32 GiB fp16 input).
  if (B > ((int64_t)1 << 28) || N > ((int64_t)1 << 28))
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "problem too large: B * N must be at most 2^28 tokens");
  const int64_t T = B * N;
  if (T > ((int64_t)1 << 28) || D > 65536 || H * M > 65536 || T * D > ((int64_t)1 << 34) ||
      T * H * M > ((int64_t)1 << 33))
    return fail(MORPHO_ERR_INVALID_ARGUMENT,
                "problem too large: needs B*N <= 2^28, B*N*D <= 2^34, B*N*H*cube_m <= 2^33, D and H*cube_m <= 65536");
  if (!__builtin_isfinite(scale)) return fail(MORPHO_ERR_INVALID_ARGUMENT, "scale must be a finite number");
  if ((causal & ~(15 | MORPHO_MODE_DETERMINISTIC)) != 0 || (causal & 12) == 12)
    return fail(MORPHO_ERR_INVALID_ARGUMENT,
                "invalid mode bits 0x%x (causal | mask_diag | one projection | deterministic)", causal);
  d.B = (int)B;
  d.N = (int)N;
  d.NP = (int)((N + 63) / 64 * 64);
  d.D = (int)D;
  d.H = (int)H;
  d.M = (int)M;
  d.DV = (int)DV;
  d.T = T;
  d.HM = (int)(H * M);
  d.CW = 2 * (int)M + 8;
  d.scale = scale;
  d.causal = causal & MORPHO_MODE_CAUSAL ? 1 : 0;
  d.mask_diag = causal & MORPHO_MODE_MASK_DIAG ? 1 : 0;
  d.proj = causal & MORPHO_MODE_PROJ_HARDTANH01 ? kProjHardTanh01
           : causal & MORPHO_MODE_PROJ_IDENTITY ? kProjIdentity
                                                : kProjSigmoid;
  d.det = causal & MORPHO_MODE_DETERMINISTIC ? 1 : 0;
  // projection tiles: 256 x 320 when 320 divides H*M + D, else 256 x 256.
  // When those would fill less than one round of the 256 CUs, 128-row tiles
  // of 160 or 128 columns (whichever divides H*M + D and needs fewer rounds
  // times tile area; 160 on a tie): e.g. H*M + D = 640, T = 8192 gives 256
  // workgroups of 128 x 160 (one round) instead of 320 of 128 x 128. The
  // interleaved column order needs whole heads and 8-column pieces per tile.
  const int NC = d.HM + d.D;
  d.PBN = NC % 320 == 0 ? 320 : 256;
  if (((T + 255) / 256) * ((NC + d.PBN - 1) / d.PBN) < 256) {
    const int64_t rows = (T + 127) / 128;
    int64_t best = -1;
    for (const int bn : {160, 128}) {
      if (NC % bn) continue;
      const int64_t cost = (rows * (NC / bn) + 255) / 256 * bn;
      if (best < 0 || cost < best) {
        best = cost;
        d.PBN = bn;
      }
    }
  }
  d.PCPT = d.PVPT = 0;
  if (NC % d.PBN == 0) {
    const int ntn = NC / d.PBN;
    if (d.HM % ntn == 0 && d.D % ntn == 0 && (d.HM / ntn) % d.M == 0 && (d.HM / ntn) % 8 == 0 &&
        (d.D / ntn) % 8 == 0) {
      d.PCPT = d.HM / ntn;
      d.PVPT = d.D / ntn;
    }
  }
  return MORPHO_OK;
}

size_t proj_bytes(const Dims& d) {
  const size_t bhn = (size_t)d.B * d.H * d.N;
  size_t s = 0;
  s += align_up(bhn * d.CW * 2);         // qa
  s += align_up(bhn * d.CW * 2);         // ka
  s += align_up((size_t)d.B * d.H * d.NP * d.DV * 2);  // vt (V_hi^T, fp16)
  s += align_up((size_t)d.B * d.H * d.NP * d.DV);      // vlo (e4m3)
  s += align_up(bhn * 16);               // tstat
  s += align_up((size_t)(d.HM + d.D) * d.D * 2);  // wt
  s += align_up((size_t)(d.HM + d.D) * d.D * 2);  // wcat
  return s;
}

ProjBuffers carve_proj(void* base, const Dims& d) {
  const size_t bhn = (size_t)d.B * d.H * d.N;
  char* p = static_cast<char*>(base);
  ProjBuffers b;
  b.qa = reinterpret_cast<_Float16*>(p); p += align_up(bhn * d.CW * 2);
  b.ka = reinterpret_cast<_Float16*>(p); p += align_up(bhn * d.CW * 2);
  b.vt = reinterpret_cast<_Float16*>(p); p += align_up((size_t)d.B * d.H * d.NP * d.DV * 2);
  b.vlo = reinterpret_cast<uint8_t*>(p); p += align_up((size_t)d.B * d.H * d.NP * d.DV);
  b.tstat = reinterpret_cast<float4*>(p); p += align_up(bhn * 16);
  b.wt = reinterpret_cast<_Float16*>(p); p += align_up((size_t)(d.HM + d.D) * d.D * 2);
  b.wcat = reinterpret_cast<_Float16*>(p);
  return b;
}

size_t bwd_bytes(const Dims& d) {
  const size_t bhn = (size_t)d.B * d.H * d.N;
  const size_t nblk = (size_t)((d.T + kGateTokensPerBlock - 1) / kGateTokensPerBlock);
  size_t s = 0;
  s += align_up(bhn * 16);                             // aug
  s += align_up(bhn * d.M * 4);                        // dq
  s += align_up(bhn * d.M * 4);                        // dk
  s += align_up(bhn * 4);                              // dcb
  s += align_up(bhn * 8);                              // dr
  s += align_up((size_t)d.T * (d.HM + d.D) * 2);       // dzv
  s += align_up(nblk * d.HM * 4);                      // gpart
  {
    const BwdGemmPlan P = bwd_gemm_plan(d);
    s += align_up((size_t)P.tiles_w * P.p * P.bt * P.bt * 4);  // wpart
  }
  if (d.det) {
    const DetLayout l = attn_bwd_det_layout(d);
    const size_t prow = (size_t)l.nkb * d.B * d.H * l.nq;
    s += align_up(prow * d.M * 4);  // dqpart
    s += align_up(prow * 4);        // drpart
  }
  return s;
}

BwdBuffers carve_bwd(void* base, const Dims& d) {
  const size_t bhn = (size_t)d.B * d.H * d.N;
  const size_t nblk = (size_t)((d.T + kGateTokensPerBlock - 1) / kGateTokensPerBlock);
  char* p = static_cast<char*>(base);
  BwdBuffers g;
  g.aug = reinterpret_cast<_Float16*>(p); p += align_up(bhn * 16);
  g.dq = reinterpret_cast<float*>(p); p += align_up(bhn * d.M * 4);
  g.dk = reinterpret_cast<float*>(p); p += align_up(bhn * d.M * 4);
  g.dcb = reinterpret_cast<float*>(p); p += align_up(bhn * 4);
  g.dr = reinterpret_cast<float*>(p); p += align_up(bhn * 8);
  g.dzv = reinterpret_cast<_Float16*>(p); p += align_up((size_t)d.T * (d.HM + d.D) * 2);
  g.gpart = reinterpret_cast<float*>(p); p += align_up(nblk * d.HM * 4);
  {
    const BwdGemmPlan P = bwd_gemm_plan(d);
    g.wpart = reinterpret_cast<float*>(p); p += align_up((size_t)P.tiles_w * P.p * P.bt * P.bt * 4);
  }
  g.dqpart = g.drpart = nullptr;
  if (d.det) {
    const DetLayout l = attn_bwd_det_layout(d);
    const size_t prow = (size_t)l.nkb * d.B * d.H * l.nq;
    g.dqpart = reinterpret_cast<float*>(p); p += align_up(prow * d.M * 4);
    g.drpart = reinterpret_cast<float*>(p);
  }
  return g;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

#define MORPHO_LAUNCH(NAME, CALL)                                                       \
  do {                                                                                  \
    timing_begin(NAME, s);                                                              \
    hipError_t e_ = (CALL);                                                             \
    timing_end(s);                                                                      \
    if (e_ != hipSuccess) return fail(MORPHO_ERR_HIP, "%s: %s", NAME, hipGetErrorString(e_)); \
  } while (0)

int run_projection(const Dims& d, const void* X, const void* W_phi, const void* gate_q, const void* gate_k,
                   const void* W_V, const ProjBuffers& p, hipStream_t s) {
  MORPHO_LAUNCH("transpose_weights", launch_transpose_weights(d, static_cast<const _Float16*>(W_phi),
                                                              static_cast<const _Float16*>(W_V), p.wt, p.wcat, s));
  MORPHO_LAUNCH("proj_fwd", launch_proj_fwd(d, static_cast<const _Float16*>(X), static_cast<const _Float16*>(gate_q),
                                            static_cast<const _Float16*>(gate_k), p, s));
  return MORPHO_OK;
}

}  // namespace

void timing_begin(const char* name, hipStream_t) {
  g_open_rec = -1;
  if (!g_timing.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (!g_timing_only.empty() && g_timing_only != name) return;
  TimingRec r{name, take_event(), take_event(), false};
  if (!r.start || !r.stop) {  // no events: nothing to bind
    if (r.start) g_pool.push_back(r.start);
    if (r.stop) g_pool.push_back(r.stop);
    return;
  }
  g_recs.push_back(r);
  g_open_rec = (int)g_recs.size() - 1;
}

void timing_end(hipStream_t) { g_open_rec = -1; }

hipEvent_t timing_take_start() {
  if (g_open_rec < 0) return nullptr;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  if (g_open_rec >= (int)g_recs.size() || g_recs[g_open_rec].bound) return nullptr;
  g_recs[g_open_rec].bound = true;
  return g_recs[g_open_rec].start;
}

hipEvent_t timing_stop_event() {
  if (g_open_rec < 0) return nullptr;
  std::lock_guard<std::mutex> lock(g_timing_mu);
  return g_open_rec < (int)g_recs.size() ? g_recs[g_open_rec].stop : nullptr;
}

}  // namespace morpho

using namespace morpho;

MORPHO_EXPORT int morpho_version(void) { return 100; }

MORPHO_EXPORT const char* morpho_status_string(int status) {
  switch (status) {
    case MORPHO_OK: return "ok";
    case MORPHO_ERR_INVALID_ARGUMENT: return "invalid argument";
    case MORPHO_ERR_UNSUPPORTED: return "unsupported";
    case MORPHO_ERR_WORKSPACE: return "workspace missing or too small";
    case MORPHO_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

MORPHO_EXPORT const char* morpho_last_error(void) { return g_last_error.c_str(); }

MORPHO_EXPORT size_t morpho_forward_workspace_size(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m) {
  Dims d;
  std::string keep = g_last_error;
  const int st = make_dims(B, N, D, H, cube_m, 1.0f, 0, d);
  g_last_error = keep;
  return st == MORPHO_OK ? proj_bytes(d) : 0;
}

MORPHO_EXPORT size_t morpho_backward_workspace_size(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m,
                                                    int have_forward_workspace) {
  Dims d;
  std::string keep = g_last_error;
  const int st = make_dims(B, N, D, H, cube_m, 1.0f, 0, d);
  g_last_error = keep;
  if (st != MORPHO_OK) return 0;
  return bwd_bytes(d) + (have_forward_workspace ? 0 : proj_bytes(d));
}

MORPHO_EXPORT size_t morpho_backward_workspace_size_for_mode(int64_t B, int64_t N, int64_t D, int64_t H,
                                                             int64_t cube_m, int have_forward_workspace, int causal) {
  Dims d;
  std::string keep = g_last_error;
  const int st = make_dims(B, N, D, H, cube_m, 1.0f, causal, d);
  g_last_error = keep;
  if (st != MORPHO_OK) return 0;
  return bwd_bytes(d) + (have_forward_workspace ? 0 : proj_bytes(d));
}

MORPHO_EXPORT int morpho_forward(const void* X, const void* W_phi, const void* gate_q, const void* gate_k,
                                 const void* W_V, void* out, float* lse, int64_t B, int64_t N, int64_t D, int64_t H,
                                 int64_t cube_m, float scale, int causal, void* workspace, size_t workspace_bytes,
                                 morpho_stream_t stream) {
  g_last_error.clear();
  Dims d;
  int st = make_dims(B, N, D, H, cube_m, scale, causal, d);
  if (st != MORPHO_OK) return st;
  if (!X || !W_phi || !gate_q || !gate_k || !W_V || !out || !lse) return fail(MORPHO_ERR_INVALID_ARGUMENT, "Null pointer");
  if (misaligned(X) || misaligned(W_phi) || misaligned(W_V) || misaligned(out) || misaligned(lse))
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "tensor pointers must be 16-byte aligned");
  const size_t need = proj_bytes(d);
  if (!workspace || workspace_bytes < need)
    return fail(MORPHO_ERR_WORKSPACE, "forward workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(MORPHO_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const ProjBuffers p = carve_proj(workspace, d);
  st = run_projection(d, X, W_phi, gate_q, gate_k, W_V, p, s);
  if (st != MORPHO_OK) return st;
  MORPHO_LAUNCH("attn_fwd", launch_attn_fwd(d, p, static_cast<_Float16*>(out), lse, s));
  return MORPHO_OK;
}

// ---------------------------------------------------------------- allocation-free forward
namespace {
// The workspace of morpho_forward_noalloc: one array per GPU the library is
// loaded on, held until the process ends. Its host-side name is not a device
// address; host code uses only the per-device address that
// hipGetSymbolAddress returns (scratch_for_current_device).
__attribute__((used)) static __device__ __align__(256) unsigned char scratch[MORPHO_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};  // guarded by g_scratch_mu

// This device's address of `scratch`, looked up on the first call with the
// device current and kept per device.
int scratch_for_current_device(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MORPHO_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(MORPHO_ERR_UNSUPPORTED, "device index %d beyond the %d this build keeps scratch for", dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    // The first call on a device may come from code under stream capture
    // (which is what the entry point is for): the lookup is no stream work,
    // so this thread's capture mode is relaxed around it and then restored.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || p == nullptr)
      return fail(MORPHO_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return MORPHO_OK;
}
}  // namespace

MORPHO_EXPORT int morpho_forward_noalloc(const void* X, const void* W_phi, const void* gate_q, const void* gate_k,
                                         const void* W_V, void* out, float* lse, int64_t B, int64_t N, int64_t D,
                                         int64_t H, int64_t cube_m, float scale, int causal, morpho_stream_t stream) {
  g_last_error.clear();
  Dims d;
  int st = make_dims(B, N, D, H, cube_m, scale, causal, d);
  if (st != MORPHO_OK) return st;
  const size_t need = proj_bytes(d);
  if (need > MORPHO_NOALLOC_SCRATCH_BYTES)
    return fail(MORPHO_ERR_WORKSPACE,
                "morpho_forward_noalloc: this problem needs %zu bytes of scratch, more than the library's %zu; "
                "use morpho_forward with a workspace",
                need, (size_t)MORPHO_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((st = scratch_for_current_device(&ws)) != MORPHO_OK) return st;
  // the same kernels as morpho_forward; every byte of the workspace they read
  // is written earlier in the same call, so nothing needs clearing
  return morpho_forward(X, W_phi, gate_q, gate_k, W_V, out, lse, B, N, D, H, cube_m, scale, causal, ws,
                        MORPHO_NOALLOC_SCRATCH_BYTES, stream);
}

MORPHO_EXPORT int morpho_backward(const void* grad_out, const void* X, const void* W_phi, const void* gate_q,
                                  const void* gate_k, const void* W_V, const void* out, const float* lse, void* dX,
                                  void* dW_phi, void* d_gate_q, void* d_gate_k, void* dW_V, int64_t B, int64_t N,
                                  int64_t D, int64_t H, int64_t cube_m, float scale, int causal,
                                  const void* forward_workspace, void* workspace, size_t workspace_bytes,
                                  morpho_stream_t stream) {
  g_last_error.clear();
  Dims d;
  int st = make_dims(B, N, D, H, cube_m, scale, causal, d);
  if (st != MORPHO_OK) return st;
  if (!grad_out || !X || !W_phi || !gate_q || !gate_k || !W_V || !out || !lse)
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "Null input pointer");
  if (!dX || !dW_phi || !d_gate_q || !d_gate_k || !dW_V) return fail(MORPHO_ERR_INVALID_ARGUMENT, "Null grad pointer");
  if (misaligned(grad_out) || misaligned(X) || misaligned(W_phi) || misaligned(W_V) || misaligned(out) ||
      misaligned(lse) || misaligned(dX) || misaligned(dW_phi) || misaligned(dW_V))
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "tensor pointers must be 16-byte aligned");
  const bool have_fwd = forward_workspace != nullptr;
  const size_t need = bwd_bytes(d) + (have_fwd ? 0 : proj_bytes(d));
  if (!workspace || workspace_bytes < need)
    return fail(MORPHO_ERR_WORKSPACE, "backward workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0 ||
      (have_fwd && (reinterpret_cast<uintptr_t>(forward_workspace) & 255) != 0))
    return fail(MORPHO_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  ProjBuffers p;
  if (have_fwd) {
    p = carve_proj(const_cast<void*>(forward_workspace), d);
  } else {
    p = carve_proj(ws, d);
    st = run_projection(d, X, W_phi, gate_q, gate_k, W_V, p, s);
    if (st != MORPHO_OK) return st;
    ws += proj_bytes(d);
  }
  const BwdBuffers g = carve_bwd(ws, d);
  const auto* go = static_cast<const _Float16*>(grad_out);
  // the forward leaves the backward's query affine block in its code rows; a
  // projection computed here still holds its own
  MORPHO_LAUNCH("bwd_prep", launch_bwd_prep(d, p, go, static_cast<const _Float16*>(out), lse, g, have_fwd ? 0 : 1, s));
  MORPHO_LAUNCH("attn_bwd", launch_attn_bwd(d, p, go, static_cast<const _Float16*>(gate_q),
                                            static_cast<const _Float16*>(gate_k), g, s));
  if (d.det) MORPHO_LAUNCH("dq_reduce", launch_dq_det_reduce(d, g, s));
  MORPHO_LAUNCH("proj_bwd_elem", launch_proj_bwd_elem(d, static_cast<const _Float16*>(gate_q),
                                                      static_cast<const _Float16*>(gate_k), p, g, true, s));
  MORPHO_LAUNCH("bwd_gemm", launch_bwd_gemm(d, p, g, static_cast<const _Float16*>(X), static_cast<_Float16*>(dX), s));
  MORPHO_LAUNCH("dw_reduce", launch_dw_reduce(d, g, static_cast<const _Float16*>(gate_q),
                                              static_cast<const _Float16*>(gate_k), static_cast<_Float16*>(dW_phi),
                                              static_cast<_Float16*>(dW_V), static_cast<_Float16*>(d_gate_q),
                                              static_cast<_Float16*>(d_gate_k), s));
  return MORPHO_OK;
}

// ---------------------------------------------------------------- soft tropical aggregation
namespace {
size_t soft_part_bytes(const Dims& d) {
  return align_up((size_t)(soft_prep_blocks(d) + 2 * soft_bwd_slots(d)) * sizeof(float));
}
size_t soft_state_bytes(const Dims& d) {
  const size_t bh = (size_t)d.B * d.H;
  return 2 * align_up(bh * d.DV * 4) + align_up(bh * d.N * 4) + align_up(4) + 2 * align_up(bh * d.DV * d.NP * 2);
}
// G hi / lo of the product-form backward, [B*H, N, DV] bf16 each
size_t soft_g_bytes(const Dims& d) { return 2 * align_up((size_t)d.B * d.H * d.N * d.DV * 2); }
SoftState carve_soft_state(void* base, const Dims& d) {
  const size_t bh = (size_t)d.B * d.H;
  char* p = static_cast<char*>(base);
  SoftState st;
  st.vmax = reinterpret_cast<float*>(p); p += align_up(bh * d.DV * 4);
  st.vmin = reinterpret_cast<float*>(p); p += align_up(bh * d.DV * 4);
  st.arow = reinterpret_cast<float*>(p); p += align_up(bh * d.N * 4);
  st.flag = reinterpret_cast<int*>(p); p += align_up(4);
  st.fth = reinterpret_cast<uint16_t*>(p); p += align_up(bh * d.DV * d.NP * 2);
  st.ftl = reinterpret_cast<uint16_t*>(p);
  return st;
}
// The soft entry points accept MORPHO_MODE_SOFT_EXACT beside the common bits.
int soft_mode(int mode, bool& exact) {
  exact = (mode & MORPHO_MODE_SOFT_EXACT) != 0;
  return mode & ~MORPHO_MODE_SOFT_EXACT;
}
int check_soft_args(const float* tau, int sgn) {
  if (!tau) return fail(MORPHO_ERR_INVALID_ARGUMENT, "Null tau pointer");
  if ((reinterpret_cast<uintptr_t>(tau) & 3) != 0)
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "tau must be 4-byte aligned");
  if (sgn != 1 && sgn != -1) return fail(MORPHO_ERR_INVALID_ARGUMENT, "sgn must be +1 (dilation) or -1 (erosion)");
  return MORPHO_OK;
}
}  // namespace

MORPHO_EXPORT size_t morpho_soft_forward_workspace_size(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m) {
  Dims d;
  std::string keep = g_last_error;
  const int st = make_dims(B, N, D, H, cube_m, 1.0f, 0, d);
  g_last_error = keep;
  return st == MORPHO_OK ? proj_bytes(d) + soft_state_bytes(d) : 0;
}

MORPHO_EXPORT size_t morpho_soft_backward_workspace_size(int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m,
                                                         int have_forward_workspace) {
  Dims d;
  std::string keep = g_last_error;
  const int st = make_dims(B, N, D, H, cube_m, 1.0f, 0, d);
  g_last_error = keep;
  if (st != MORPHO_OK) return 0;
  return bwd_bytes(d) + soft_part_bytes(d) + soft_g_bytes(d) + (have_forward_workspace ? 0 : proj_bytes(d));
}

MORPHO_EXPORT int morpho_soft_forward(const void* X, const void* W_phi, const void* gate_q, const void* gate_k,
                                      const void* W_V, const float* tau, void* out, float* zb, int64_t B, int64_t N,
                                      int64_t D, int64_t H, int64_t cube_m, float scale, int mode, int sgn,
                                      void* workspace, size_t workspace_bytes, morpho_stream_t stream) {
  g_last_error.clear();
  Dims d;
  bool exact = false;
  int st = make_dims(B, N, D, H, cube_m, scale, soft_mode(mode, exact), d);
  if (st != MORPHO_OK) return st;
  if (d.det) return fail(MORPHO_ERR_UNSUPPORTED, "MORPHO_MODE_DETERMINISTIC applies to the softmax backward only");
  if (!X || !W_phi || !gate_q || !gate_k || !W_V || !out || !zb) return fail(MORPHO_ERR_INVALID_ARGUMENT, "Null pointer");
  if ((st = check_soft_args(tau, sgn)) != MORPHO_OK) return st;
  if (misaligned(X) || misaligned(W_phi) || misaligned(W_V) || misaligned(out) || misaligned(zb))
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "tensor pointers must be 16-byte aligned");
  const size_t need = proj_bytes(d) + soft_state_bytes(d);
  if (!workspace || workspace_bytes < need)
    return fail(MORPHO_ERR_WORKSPACE, "soft forward workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
    return fail(MORPHO_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const ProjBuffers p = carve_proj(workspace, d);
  const SoftState ss = carve_soft_state(static_cast<char*>(workspace) + proj_bytes(d), d);
  st = run_projection(d, X, W_phi, gate_q, gate_k, W_V, p, s);
  if (st != MORPHO_OK) return st;
  auto* o = static_cast<_Float16*>(out);
  if (exact) {
    MORPHO_LAUNCH("soft_fwd", launch_soft_fwd(d, p, tau, sgn, o, zb, nullptr, s));
    MORPHO_LAUNCH("soft_flag", launch_set_flag(ss.flag, 1, s));  // a backward handed this workspace stays exact
    return MORPHO_OK;
  }
  // product form on MFMA; the element-wise kernel runs only if some output
  // failed its check (the flag, cleared by soft_colext)
  MORPHO_LAUNCH("soft_colext", launch_soft_colext(d, p, ss, s));
  MORPHO_LAUNCH("soft_fvals", launch_soft_fvals(d, p, tau, sgn, ss, s));
  MORPHO_LAUNCH("soft_fwd_fast", launch_soft_fwd_fast(d, p, tau, sgn, ss, o, zb, s));
  MORPHO_LAUNCH("soft_fwd", launch_soft_fwd(d, p, tau, sgn, o, zb, ss.flag, s));
  return MORPHO_OK;
}

MORPHO_EXPORT int morpho_soft_backward(const void* grad_out, const void* X, const void* W_phi, const void* gate_q,
                                       const void* gate_k, const void* W_V, const float* tau, const float* zb,
                                       void* dX, void* dW_phi, void* d_gate_q, void* d_gate_k, void* dW_V, float* dtau,
                                       int64_t B, int64_t N, int64_t D, int64_t H, int64_t cube_m, float scale,
                                       int mode, int sgn, const void* forward_workspace, void* workspace,
                                       size_t workspace_bytes, morpho_stream_t stream) {
  g_last_error.clear();
  Dims d;
  bool exact = false;
  int st = make_dims(B, N, D, H, cube_m, scale, soft_mode(mode, exact), d);
  if (st != MORPHO_OK) return st;
  if (d.det) return fail(MORPHO_ERR_UNSUPPORTED, "MORPHO_MODE_DETERMINISTIC applies to the softmax backward only");
  if (!grad_out || !X || !W_phi || !gate_q || !gate_k || !W_V || !zb)
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "Null input pointer");
  if (!dX || !dW_phi || !d_gate_q || !d_gate_k || !dW_V || !dtau)
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "Null grad pointer");
  if ((st = check_soft_args(tau, sgn)) != MORPHO_OK) return st;
  if (misaligned(grad_out) || misaligned(X) || misaligned(W_phi) || misaligned(W_V) || misaligned(zb) ||
      misaligned(dX) || misaligned(dW_phi) || misaligned(dW_V))
    return fail(MORPHO_ERR_INVALID_ARGUMENT, "tensor pointers must be 16-byte aligned");
  const bool have_fwd = forward_workspace != nullptr;
  const size_t need = bwd_bytes(d) + soft_part_bytes(d) + soft_g_bytes(d) + (have_fwd ? 0 : proj_bytes(d));
  if (!workspace || workspace_bytes < need)
    return fail(MORPHO_ERR_WORKSPACE, "backward workspace needs %zu bytes (got %zu)", need, workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) != 0 ||
      (have_fwd && (reinterpret_cast<uintptr_t>(forward_workspace) & 255) != 0))
    return fail(MORPHO_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  ProjBuffers p;
  if (have_fwd) {
    p = carve_proj(const_cast<void*>(forward_workspace), d);
  } else {
    p = carve_proj(ws, d);
    st = run_projection(d, X, W_phi, gate_q, gate_k, W_V, p, s);
    if (st != MORPHO_OK) return st;
    ws += proj_bytes(d);
  }
  const BwdBuffers g = carve_bwd(ws, d);
  float* prep_part = reinterpret_cast<float*>(ws + bwd_bytes(d));
  float* bwd_part = prep_part + soft_prep_blocks(d);
  float* fast_part = bwd_part + 2 * soft_bwd_exact_slots(d);
  auto* gh = reinterpret_cast<uint16_t*>(ws + bwd_bytes(d) + soft_part_bytes(d));
  auto* gl = gh + align_up((size_t)d.B * d.H * d.N * d.DV * 2) / 2;
  const auto* go = static_cast<const _Float16*>(grad_out);
  if (have_fwd && !exact) {
    // the forward's state: the product form when its flag stayed 0, else the
    // element-wise kernel (each writes zero partials when it does not run)
    const SoftState ss = carve_soft_state(static_cast<char*>(const_cast<void*>(forward_workspace)) + proj_bytes(d), d);
    MORPHO_LAUNCH("soft_bwd_prep", launch_soft_bwd_prep(d, go, zb, g, prep_part, tau, sgn, &ss, gh, gl, s));
    MORPHO_LAUNCH("soft_bwd_fast", launch_soft_bwd_fast(d, p, go, zb, tau, sgn, ss, gh, gl, g, fast_part, s));
    MORPHO_LAUNCH("soft_bwd", launch_soft_bwd(d, p, go, zb, tau, sgn, g, bwd_part, ss.flag, s));
  } else {
    MORPHO_LAUNCH("soft_bwd_prep", launch_soft_bwd_prep(d, go, zb, g, prep_part, tau, sgn, nullptr, nullptr, nullptr, s));
    MORPHO_LAUNCH("soft_bwd", launch_soft_bwd(d, p, go, zb, tau, sgn, g, bwd_part, nullptr, s));
    MORPHO_LAUNCH("soft_part_clear", launch_fill_zero(fast_part, 2 * (soft_bwd_slots(d) - soft_bwd_exact_slots(d)), s));
  }
  MORPHO_LAUNCH("proj_bwd_elem", launch_proj_bwd_elem(d, static_cast<const _Float16*>(gate_q),
                                                      static_cast<const _Float16*>(gate_k), p, g, false, s));
  MORPHO_LAUNCH("bwd_gemm", launch_bwd_gemm(d, p, g, static_cast<const _Float16*>(X), static_cast<_Float16*>(dX), s));
  MORPHO_LAUNCH("dw_reduce", launch_dw_reduce(d, g, static_cast<const _Float16*>(gate_q),
                                              static_cast<const _Float16*>(gate_k), static_cast<_Float16*>(dW_phi),
                                              static_cast<_Float16*>(dW_V), static_cast<_Float16*>(d_gate_q),
                                              static_cast<_Float16*>(d_gate_k), s));
  MORPHO_LAUNCH("soft_tau_reduce", launch_soft_tau_reduce(prep_part, soft_prep_blocks(d), bwd_part,
                                                          soft_bwd_slots(d), tau, sgn, dtau, s));
  return MORPHO_OK;
}

MORPHO_EXPORT int morpho_timing_enable(int enable) {
  g_timing.store(enable != 0);
  return MORPHO_OK;
}

MORPHO_EXPORT int morpho_timing_only(const char* name) {
  std::lock_guard<std::mutex> lock(g_timing_mu);
  g_timing_only = name ? name : "";
  return MORPHO_OK;
}

MORPHO_EXPORT int morpho_timing_read(const char** names, float* ms, int max_entries) {
  std::lock_guard<std::mutex> lock(g_timing_mu);
  int n = 0;
  for (const TimingRec& r : g_recs) {
    if (n < max_entries && r.bound) {
      float t = 0.f;
      if (hipEventSynchronize(r.stop) == hipSuccess && hipEventElapsedTime(&t, r.start, r.stop) == hipSuccess) {
        if (names) names[n] = r.name;
        if (ms) ms[n] = t;
        ++n;
      }
    }
    if (r.start) g_pool.push_back(r.start);
    if (r.stop) g_pool.push_back(r.stop);
  }
  g_recs.clear();
  return n;
}
