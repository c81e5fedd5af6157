// C ABI of the S6 selective-scan library: argument validation, workspace planning and
// kernel dispatch.  Validation and planning are host-only and never touch a device, so
// they can be exercised (and are, by the CPU tests) on a machine without a GPU.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "s6_internal.h"
#include "selective_state_update.h"
#include "ssd.h"

// Scratch of the no-allocation forward (s6_fwd_noalloc): one array per device, holding the
// forward's workspace (chunk summaries, B/C relayout).  Every region of it that a forward
// reads is written earlier in the same call, so nothing needs clearing between calls.  In
// host code `scratch` names a host-side stand-in, not a device address: kernels and copies
// get the address that hipGetSymbolAddress returns for each device (g_scratch_ptr below).
static __device__ __align__(256) unsigned char scratch[S6_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;

int validate_fwd(const S6FwdArgs* a, bool check_workspace);
int run_fwd(const S6FwdArgs& a, hipStream_t st);

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int fail(int code, const char* fmt, ...);

// Device address of this device's scratch array, looked up once per device with that
// device current (the stream's device; the null stream means the current one).
int scratch_for_stream(hipStream_t st, void** out) {
  int dev = -1, cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e == hipSuccess) e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_fwd_noalloc: cannot query the device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(S6_E_UNSUPPORTED, "s6_fwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
      return fail(S6_E_HIP, "s6_fwd_noalloc: hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur) {
      hipError_t e2 = hipSetDevice(cur);
      if (e == hipSuccess) e = e2;
    }
    if (e != hipSuccess || ptr == nullptr)
      return fail(S6_E_HIP, "s6_fwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return S6_OK;
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

int ok() {
  g_last_error.clear();
  return S6_OK;
}

// Chunking targets (waves per launch; shortest chunk).  The forward scan holds ~90 VGPRs
// (5 waves per SIMD) and is VALU-bound at 4 waves per SIMD; the backward scan holds ~240
// VGPRs (2 waves per SIMD) and needs more waves in flight to cover its memory latency.
constexpr int64_t kTargetWavesFwd = 4096;  // 4 per SIMD on a 256-CU MI355X
constexpr int64_t kTargetWavesBwd = 8192;
constexpr int64_t kMinChunkFwd = 128;
constexpr int64_t kMinChunkBwd = 128;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
size_t align256(size_t x) { return (x + 255) & ~size_t(255); }
int esize(int dt) { return dt == S6_F32 ? 4 : 2; }

struct Plan {
  bool lanes;  // forward: single-pass kernel, one lane per (channel, state)
  int64_t Dg, nJ, nDblk;
  int64_t K, Lc, nck;
  bool relayout_B, relayout_C;
  int64_t NP;  // padded dstate of relaid-out B / C
  size_t off_h, off_s, off_r, off_B, off_C, total_fwd;
  size_t off_pB, off_pC, off_dA, off_dD, off_db, total_bwd;
  int64_t nsg, NPr;  // backward: state groups of 16, partial row width
};

// States held per lane by the kernels: the forward pads dstate to 8/16/32 and above 32
// splits it into groups of 16, one wave per group; the backward pads to 8/16 and above 16
// splits it into groups of 16 (B / C rows padded to a multiple of 16 states).  B and C
// rows are read as NS contiguous values, so a row is used in place only when dstate == NS,
// the state axis is contiguous and 16-bit rows are 4-byte aligned.
int64_t ns_fwd(int64_t N) { return N <= 8 ? 8 : N <= 16 ? 16 : N <= 32 ? 32 : ceil_div(N, 16) * 16; }
// Forward state groups: above 32 states a workgroup holds one wave per group of 16.
int64_t nsg_fwd(int64_t N) { return N <= 32 ? 1 : ceil_div(N, 16); }
int64_t ns_bwd(int64_t N) { return N <= 8 ? 8 : ceil_div(N, s6::kBwdGroup) * s6::kBwdGroup; }

bool bc_scalar_ok(const void* ptr, const int64_t s[4], int dt, int64_t N, int64_t NS) {
  if (N != NS || s[2] != 1) return false;
  if (dt == S6_F32) return true;
  if (((uintptr_t)ptr & 3u) != 0) return false;
  if ((N & 1) != 0) return false;
  return (s[0] % 2 == 0) && (s[1] % 2 == 0) && (s[3] % 2 == 0);
}

// Forward kernel choice.  The single-pass kernel (one lane per (channel, state), 16 / 32 / 64
// lanes per channel) needs no chunk summaries, carries or B/C relayout, and does each
// element's exp once, but it has only B * D * ceil16(N) / 64 waves and each one is a serial
// chain.  Measured on the MI355X (same box, forward step time, chunked -> single-pass):
//   B32 L4096 D256 N16 bf16 (2048 waves):               0.256 -> 0.232 ms
//   B16 L16384 D256 N64 fp32 (4096 waves):              2.30  -> 1.76 ms
//   B8 L8192 D768 N16 bf16, checkpoints (1536 waves):   forward slower (0.51 vs 0.28 +
//                                                       summary pass)
//   B32 L4096 D256 N16 bf16, softplus + z gate:         0.325 -> 0.367 ms
// so it is used for dense batches with dstate 9-64, no z gate, and at least kLanesMinWaves
// waves (two per SIMD).  S6_FWD_PATH=lanes or =chunked in the environment forces either one
// (for measurement and tests); a forced single-pass choice still needs a dense batch and
// dstate 9-64.
constexpr int64_t kLanesMinWaves = 2048;

int64_t lanes_ns(int64_t N) { return N <= 16 ? 16 : N <= 32 ? 32 : 64; }
int64_t lanes_cpg(int64_t N) { return 4 * (64 / lanes_ns(N)); }  // channels per workgroup

bool lanes_eligible(const S6Problem& p) {
  if (p.nseq > 0 || p.dstate < 9 || p.dstate > 64) return false;
  const char* env = getenv("S6_FWD_PATH");
  return env == nullptr || strcmp(env, "chunked") != 0;
}

bool choose_lanes(const S6Problem& p) {
  if (!lanes_eligible(p)) return false;
  const char* env = getenv("S6_FWD_PATH");
  if (env != nullptr && strcmp(env, "lanes") == 0) return true;
  if (p.has_z) return false;
  const int64_t Dg = p.dim / p.ngroups;
  const int64_t waves = p.batch * p.ngroups * ceil_div(Dg, lanes_cpg(p.dstate)) * 4;
  return waves >= kLanesMinWaves;
}

// u / delta / out (z / out_z) with a contiguous time axis, the [B, D, L] layout zoology's
// Mamba passes.  There the chunked kernels, one lane per channel, touch one cache line per
// lane at every access and re-fetch each line for every block of it they use (5-8x the
// algorithmic bytes measured), while the single-pass kernel's 16 lanes of a channel read 16
// consecutive steps together.  Measured on such inputs (same box, forward time):
//   B32 L4096 D256 N16 bf16, softplus + bias + z gate: chunked 0.555 -> single-pass 0.263 ms
//   B8 L8192 D768 N16 bf16 with checkpoints (1536 waves): 0.669 -> 0.406 ms
// so every single-pass-eligible problem takes it on this layout, whatever the wave count and
// the z gate.  This only ever adds single-pass choices, which need no workspace: sizing from
// the problem alone stays an upper bound.
bool lcontig_rows(const S6FwdArgs& a) {
  bool ok = a.u_stride[2] == 1 && a.delta_stride[2] == 1 && a.out_stride[2] == 1;
  if (a.p.has_z) ok = ok && a.z_stride[2] == 1 && a.out_z_stride[2] == 1;
  return ok;
}

// Chunking and workspace layout; ptrs may be null (sizing only, then relayout is assumed
// to be needed).  lcontig: the forward's per-channel tensors are L-contiguous (lcontig_rows).
Plan make_plan(const S6Problem& p, bool bwd, const void* Bp, const int64_t* sB, const void* Cp,
               const int64_t* sC, bool lcontig = false) {
  Plan pl{};
  if (!bwd && (choose_lanes(p) || (lcontig && lanes_eligible(p)))) {
    pl.lanes = true;
    pl.Dg = p.dim / p.ngroups;
    pl.nJ = ceil_div(pl.Dg, lanes_cpg(p.dstate));
    pl.nDblk = p.ngroups * pl.nJ;
    pl.Lc = p.seqlen;
    pl.K = 1;
    pl.nck = ceil_div(p.seqlen, s6::kCk);
    pl.NP = lanes_ns(p.dstate);
    pl.total_fwd = 0;  // no summaries, no relayout: B / C are read at any strides
    return pl;
  }
  pl.Dg = p.dim / p.ngroups;
  pl.nJ = ceil_div(pl.Dg, 64);
  pl.nDblk = p.ngroups * pl.nJ;
  const int64_t chw = p.batch * pl.nDblk;
  const int64_t waves_per_chunk = chw * (bwd ? 1 : nsg_fwd(p.dstate));
  const int64_t ktarget =
      ceil_div(bwd ? kTargetWavesBwd : kTargetWavesFwd, waves_per_chunk > 0 ? waves_per_chunk : 1);
  int64_t Lc = ceil_div(p.seqlen, ktarget > 0 ? ktarget : 1);
  const int64_t min_chunk = bwd ? kMinChunkBwd : kMinChunkFwd;
  if (Lc < min_chunk) Lc = min_chunk;
  Lc = ceil_div(Lc, s6::kCk) * s6::kCk;
  pl.Lc = Lc;
  pl.K = ceil_div(p.seqlen, Lc);
  pl.nck = ceil_div(p.seqlen, s6::kCk);
  const int64_t NS = bwd ? ns_bwd(p.dstate) : ns_fwd(p.dstate);
  pl.relayout_B = sB ? !bc_scalar_ok(Bp, sB, p.bc_dtype, p.dstate, NS) : true;
  pl.relayout_C = sC ? !bc_scalar_ok(Cp, sC, p.bc_dtype, p.dstate, NS) : true;
  pl.NP = NS;
  const size_t nchan = (size_t)(p.batch * p.dim);
  size_t off = 0;
  pl.off_h = off;
  off += pl.K > 1 ? align256(nchan * pl.K * p.dstate * 4) : 0;
  pl.off_s = off;
  off += pl.K > 1 ? align256(nchan * pl.K * 4) : 0;
  pl.off_r = off;
  off += (pl.K > 1 && p.nseq > 0) ? align256(nchan * pl.K * 4) : 0;
  const size_t bc_bytes = align256((size_t)(p.batch * p.ngroups * p.seqlen * pl.NP) * esize(p.bc_dtype));
  pl.off_B = off;
  off += pl.relayout_B ? bc_bytes : 0;
  pl.off_C = off;
  off += pl.relayout_C ? bc_bytes : 0;
  pl.total_fwd = off;
  pl.nsg = p.dstate <= s6::kBwdGroup ? 1 : ceil_div(p.dstate, s6::kBwdGroup);
  pl.NPr = pl.nsg * s6::kBwdGroup;
  const size_t part = align256((size_t)(p.batch * p.ngroups * pl.nJ * p.seqlen * pl.NPr) * 4);
  pl.off_pB = off;
  off += part;
  pl.off_pC = off;
  off += part;
  const size_t rows = (size_t)(p.batch * pl.K);
  pl.off_dA = off;
  off += align256(rows * p.dim * p.dstate * 4);
  pl.off_dD = off;
  off += p.has_D ? align256(rows * p.dim * 4) : 0;
  pl.off_db = off;
  off += p.has_delta_bias ? align256(rows * p.dim * 4) : 0;
  pl.total_bwd = off;
  return pl;
}

// The kernels address [batch, dim, seqlen] tensors through 32-bit buffer offsets relative
// to a wave's first element: 63 channel strides plus one chunk of time strides must stay
// below 2^31 bytes.
int check_span(const int64_t* s, int es, int64_t Lc, const char* name) {
  const int64_t span = (63 * s[1] + Lc * s[2]) * (int64_t)es;
  if (span >= ((int64_t)1 << 31) - (1 << 20))
    return fail(S6_E_UNSUPPORTED,
                "%s: strides too large for 32-bit buffer offsets (63*%lld + %lld*%lld elements)",
                name, (long long)s[1], (long long)Lc, (long long)s[2]);
  return S6_OK;
}

// x_ckpt strides: all zero (contiguous), or non-negative with the states of a channel
// contiguous (the kernels load and store a channel's states as one run).
int check_ckpt(const int64_t* s) {
  if (s[0] == 0 && s[1] == 0 && s[2] == 0 && s[3] == 0) return S6_OK;
  for (int i = 0; i < 4; ++i)
    if (s[i] < 0) return fail(S6_E_INVALID, "x_ckpt has a negative stride");
  if (s[3] != 1)
    return fail(S6_E_UNSUPPORTED, "x_ckpt: the dstate stride must be 1, got %lld",
                (long long)s[3]);
  return S6_OK;
}

int check_ptr(const void* p, const char* name) {
  if (p == nullptr) return fail(S6_E_INVALID, "%s must not be NULL", name);
  return S6_OK;
}

int check_strides(const int64_t* s, int n, const char* name) {
  for (int i = 0; i < n; ++i)
    if (s[i] < 0) return fail(S6_E_INVALID, "%s has a negative stride", name);
  return S6_OK;
}

int check_common(const S6Problem& p, const void* u, const int64_t* su, const void* delta,
                 const int64_t* sdl, const float* A, const int64_t* sA, const void* B,
                 const int64_t* sB, const void* C, const int64_t* sC, const float* D,
                 const void* z, const int64_t* sz, const float* bias, const int32_t* cu) {
  int r;
  if ((r = s6_validate_problem(&p)) != S6_OK) return r;
  if ((r = check_ptr(u, "u")) || (r = check_ptr(delta, "delta")) || (r = check_ptr(A, "A")) ||
      (r = check_ptr(B, "B")) || (r = check_ptr(C, "C")))
    return r;
  if ((r = check_strides(su, 3, "u")) || (r = check_strides(sdl, 3, "delta")) ||
      (r = check_strides(sA, 2, "A")) || (r = check_strides(sB, 4, "B")) ||
      (r = check_strides(sC, 4, "C")))
    return r;
  if (p.has_D && (r = check_ptr(D, "D"))) return r;
  if (p.has_z) {
    if ((r = check_ptr(z, "z"))) return r;
    if ((r = check_strides(sz, 3, "z"))) return r;
  }
  if (p.has_delta_bias && (r = check_ptr(bias, "delta_bias"))) return r;
  if (p.nseq > 0 && (r = check_ptr(cu, "cu_seqlens"))) return r;
  return S6_OK;
}

// Batch, checkpoint and dim element strides of x_ckpt ([batch, checkpoint, dim, dstate], the
// dstate stride being 1); all zero = contiguous.
void ckpt_strides(const int64_t* given, const S6Problem& p, int64_t nck, int64_t* out) {
  if (given[0] == 0 && given[1] == 0 && given[2] == 0 && given[3] == 0) {
    out[0] = nck * p.dim * p.dstate; out[1] = p.dim * p.dstate; out[2] = p.dstate;
  } else {
    for (int i = 0; i < 3; ++i) out[i] = given[i];
  }
}

// Whole 8-step row blocks in the chunked forward (Row8 in s6_common.h): the tensor's time
// axis is contiguous and every block of 8 steps of every row starts 16-byte aligned (the
// chunk length is a multiple of 8, so whole blocks when the sequence length is too).
bool rows_vec_ok(const void* ptr, const int64_t s[3], int es, const S6Problem& p) {
  if (s[2] != 1 || ((uintptr_t)ptr & 15u) != 0) return false;
  return (p.batch == 1 || (s[0] * es) % 16 == 0) && (p.dim == 1 || (s[1] * es) % 16 == 0);
}

// S6_FWD_ROWVEC=0 in the environment keeps the per-step loads and stores (for measurement).
bool choose_rowvec(const S6FwdArgs& a, const Plan& pl) {
  const S6Problem& p = a.p;
  if (pl.lanes || p.dstate > 32 || p.seqlen % s6::kCk != 0) return false;
  const char* env = getenv("S6_FWD_ROWVEC");
  if (env != nullptr && strcmp(env, "0") == 0) return false;
  const int es = esize(p.io_dtype);
  bool ok = rows_vec_ok(a.u, a.u_stride, es, p) && rows_vec_ok(a.delta, a.delta_stride, es, p) &&
            rows_vec_ok(a.out, a.out_stride, es, p);
  if (p.has_z) ok = ok && rows_vec_ok(a.z, a.z_stride, es, p) && rows_vec_ok(a.out_z, a.out_z_stride, es, p);
  return ok;
}

// The forward's plan for these arguments (their layout can select the single-pass kernel).
Plan fwd_plan(const S6FwdArgs& a) {
  return make_plan(a.p, false, a.B, a.B_stride, a.C, a.C_stride, lcontig_rows(a));
}

// The backward's row blocks (one wave per 64-channel block, dstate <= 16): every per-channel
// tensor it reads or writes passes rows_vec_ok.  S6_BWD_ROWVEC=0 keeps per-step accesses.
bool choose_rowvec_bwd(const S6BwdArgs& a) {
  const S6Problem& p = a.p;
  if (p.dstate > s6::kBwdGroup || p.seqlen % s6::kCk != 0) return false;
  const char* env = getenv("S6_BWD_ROWVEC");
  if (env != nullptr && strcmp(env, "0") == 0) return false;
  const int es = esize(p.io_dtype);
  bool ok = rows_vec_ok(a.u, a.u_stride, es, p) && rows_vec_ok(a.delta, a.delta_stride, es, p) &&
            rows_vec_ok(a.dout, a.dout_stride, es, p) && rows_vec_ok(a.du, a.du_stride, es, p) &&
            rows_vec_ok(a.ddelta, a.ddelta_stride, es, p);
  if (p.has_z) {
    ok = ok && rows_vec_ok(a.z, a.z_stride, es, p) && rows_vec_ok(a.out, a.out_stride, es, p) &&
         rows_vec_ok(a.dz, a.dz_stride, es, p);
    if (a.out_z != nullptr) ok = ok && rows_vec_ok(a.out_z, a.out_z_stride, es, p);
  }
  return ok;
}

s6::FwdK fill_fwd(const S6FwdArgs& a, const Plan& pl) {
  s6::FwdK k{};
  const S6Problem& p = a.p;
  k.Bsz = p.batch; k.D = p.dim; k.L = p.seqlen; k.N = p.dstate; k.G = p.ngroups;
  for (int i = 0; i < 3; ++i) {
    k.su[i] = a.u_stride[i]; k.sdl[i] = a.delta_stride[i];
    k.sz[i] = p.has_z ? a.z_stride[i] : 0;
    k.so[i] = a.out_stride[i];
    k.soz[i] = p.has_z ? a.out_z_stride[i] : 0;
  }
  k.sA[0] = a.A_stride[0]; k.sA[1] = a.A_stride[1];
  k.sD = a.D_stride; k.sbias = a.delta_bias_stride;
  k.u = a.u; k.delta = a.delta; k.z = a.z; k.A = a.A; k.Dp = a.D; k.bias = a.delta_bias;
  char* ws = (char*)a.workspace;
  const int64_t NP = pl.NP;
  if (pl.relayout_B) {
    k.Bm = ws + pl.off_B;
    k.sB[0] = p.ngroups * p.seqlen * NP; k.sB[1] = p.seqlen * NP; k.sB[2] = 1; k.sB[3] = NP;
  } else {
    k.Bm = a.B;
    for (int i = 0; i < 4; ++i) k.sB[i] = a.B_stride[i];
  }
  if (pl.relayout_C) {
    k.Cm = ws + pl.off_C;
    k.sC[0] = p.ngroups * p.seqlen * NP; k.sC[1] = p.seqlen * NP; k.sC[2] = 1; k.sC[3] = NP;
  } else {
    k.Cm = a.C;
    for (int i = 0; i < 4; ++i) k.sC[i] = a.C_stride[i];
  }
  k.cu = a.cu_seqlens; k.nseq = p.nseq;
  k.out = a.out; k.out_z = a.out_z;
  k.x_ckpt = a.x_ckpt; k.nck = pl.nck; k.last_state = a.last_state;
  ckpt_strides(a.x_ckpt_stride, p, pl.nck, k.sck);
  k.ws_h = pl.K > 1 ? (float*)(ws + pl.off_h) : nullptr;
  k.ws_s = pl.K > 1 ? (float*)(ws + pl.off_s) : nullptr;
  k.ws_r = (pl.K > 1 && p.nseq > 0) ? (int32_t*)(ws + pl.off_r) : nullptr;
  k.K = pl.K; k.Lc = pl.Lc;
  k.has_D = p.has_D; k.has_z = p.has_z; k.has_bias = p.has_delta_bias; k.softplus = p.delta_softplus;
  k.nDblk = pl.nDblk;
  k.nsg = (int32_t)nsg_fwd(p.dstate);
  k.lanes = pl.lanes ? 1 : 0;
  k.rowvec = choose_rowvec(a, pl) ? 1 : 0;
  return k;
}

// ---- causal conv1d ---------------------------------------------------------------------

constexpr int64_t kConvT = 64;            // steps per wave tile
constexpr int64_t kConvTargetBlocks = 2048;

struct ConvPlan {
  int64_t T, ntile4, nsplit, tps;
  int64_t nslice, rps;   // first-level row slices of the partial rows
  size_t off_ws2, ws_bytes;
};

ConvPlan conv_plan(const S6ConvProblem& p) {
  ConvPlan c;
  c.T = kConvT;
  c.ntile4 = ceil_div(p.seqlen, 4 * kConvT);
  // Backward blocks along the sequence: enough (batch, 256-channel, split) blocks to fill
  // the chip; every block writes one partial row, so no more than that.
  const int64_t per = p.batch * ceil_div(p.dim, 256);
  int64_t ns = std::min(c.ntile4, std::max<int64_t>(1, ceil_div(kConvTargetBlocks, per)));
  c.tps = ceil_div(c.ntile4, ns);
  c.nsplit = ceil_div(c.ntile4, c.tps);
  const int64_t rows = p.batch * c.nsplit;
  c.rps = std::max<int64_t>(32, ceil_div(rows, 64));
  c.nslice = ceil_div(rows, c.rps);
  const size_t row_bytes = (size_t)(p.dim * (p.width + 1)) * 4;
  c.off_ws2 = align256(rows * row_bytes);
  c.ws_bytes = c.off_ws2 + c.nslice * row_bytes;
  return c;
}

// Channels per lane: 16 bytes of channel-contiguous storage when every tensor allows it.
bool conv_vec_ok(const void* ptr, const int64_t s[3], int64_t vec, int es) {
  return s[1] == 1 && s[0] % vec == 0 && s[2] % vec == 0 &&
         ((uintptr_t)ptr % (uintptr_t)(vec * es)) == 0;
}

// Channels per lane: the widest vector (at most 16 bytes; 8 bytes in the backward, whose
// per-lane state is W + 1 partial sums, a W-deep input window and a W-deep dx window per
// channel) that every tensor's layout allows and that leaves at most 1/8 of the lanes of
// the last channel block idle; else the allowed width that idles the fewest lanes.
int64_t conv_pick_vec(int64_t dim, int es, bool bwd, const void* const* ptrs,
                      const int64_t* const* strides, int n) {
  const int64_t maxv = (bwd ? 8 : 16) / es;
  int64_t best = 1;
  double best_waste = 2.0;
  for (int64_t v = maxv; v >= 1; v /= 2) {
    bool ok = v == 1 || dim % v == 0;
    for (int i = 0; ok && v > 1 && i < n; ++i) ok = conv_vec_ok(ptrs[i], strides[i], v, es);
    if (!ok) continue;
    const int64_t per = 64 * v;
    const double waste = 1.0 - (double)dim / (double)(ceil_div(dim, per) * per);
    if (waste <= 0.125) return v;
    if (waste < best_waste) { best = v; best_waste = waste; }
  }
  return best;
}

int conv_check_problem(const S6ConvProblem& p) {
  if (p.batch < 1 || p.dim < 1 || p.seqlen < 1)
    return fail(S6_E_INVALID, "causal_conv1d: batch, dim, seqlen must be >= 1");
  if (p.width < 2 || p.width > S6_CONV_MAX_WIDTH)
    return fail(S6_E_UNSUPPORTED, "causal_conv1d: width must be in [2, %d], got %lld",
                S6_CONV_MAX_WIDTH, (long long)p.width);
  if (p.io_dtype != S6_F32 && p.io_dtype != S6_BF16 && p.io_dtype != S6_F16)
    return fail(S6_E_INVALID, "causal_conv1d: bad io_dtype %d", p.io_dtype);
  if (p.silu != 0 && p.silu != 1) return fail(S6_E_INVALID, "causal_conv1d: silu must be 0 or 1");
  if (ceil_div(p.seqlen, 4 * kConvT) > 65535)
    return fail(S6_E_UNSUPPORTED, "causal_conv1d: seqlen %lld too long", (long long)p.seqlen);
  if (p.batch * p.dim > ((int64_t)1 << 31) - 1)
    return fail(S6_E_UNSUPPORTED, "causal_conv1d: batch * dim too large");
  return S6_OK;
}

int conv_check_common(const S6ConvProblem& p, const void* x, const int64_t* sx, const float* w,
                      const int64_t* sw) {
  int r;
  if ((r = conv_check_problem(p))) return r;
  if ((r = check_ptr(x, "x")) || (r = check_strides(sx, 3, "x")) || (r = check_ptr(w, "weight")) ||
      (r = check_strides(sw, 2, "weight")))
    return r;
  return S6_OK;
}

s6::ConvK conv_fill(const S6ConvProblem& p, const ConvPlan& c, int64_t vec) {
  s6::ConvK k{};
  k.Bsz = p.batch; k.D = p.dim; k.L = p.seqlen;
  k.T = c.T; k.ntile4 = c.ntile4; k.nsplit = c.nsplit; k.tps = c.tps;
  k.nslice = c.nslice; k.rps = c.rps;
  k.nCb = ceil_div(p.dim, 64 * vec);
  return k;
}

int ssu_check(const S6StateUpdateArgs& a) {
  int r;
  if (a.batch < 1 || a.nheads < 1 || a.dim < 1 || a.dstate < 1 || a.ngroups < 1)
    return fail(S6_E_INVALID, "selective_state_update: batch, nheads, dim, dstate, ngroups must be >= 1");
  if (a.nheads % a.ngroups != 0)
    return fail(S6_E_INVALID, "selective_state_update: nheads must be divisible by ngroups");
  if (a.dstate > S6_SSU_MAX_DSTATE)
    return fail(S6_E_UNSUPPORTED, "selective_state_update: dstate must be <= %d, got %lld",
                S6_SSU_MAX_DSTATE, (long long)a.dstate);
  if (a.batch > 65535 || a.nheads > 65535 || ceil_div(a.dim, 64) > ((int64_t)1 << 31) - 1)
    return fail(S6_E_UNSUPPORTED, "selective_state_update: batch / nheads / dim too large");
  for (int dt : {a.state_dtype, a.io_dtype, a.bc_dtype})
    if (dt != S6_F32 && dt != S6_BF16 && dt != S6_F16)
      return fail(S6_E_INVALID, "selective_state_update: bad dtype %d", dt);
  if ((r = check_ptr(a.state, "state")) || (r = check_strides(a.state_stride, 4, "state")) ||
      (r = check_ptr(a.x, "x")) || (r = check_strides(a.x_stride, 3, "x")) ||
      (r = check_ptr(a.dt, "dt")) || (r = check_strides(a.dt_stride, 3, "dt")) ||
      (r = check_ptr(a.A, "A")) || (r = check_strides(a.A_stride, 3, "A")) ||
      (r = check_ptr(a.B, "B")) || (r = check_strides(a.B_stride, 3, "B")) ||
      (r = check_ptr(a.C, "C")) || (r = check_strides(a.C_stride, 3, "C")) ||
      (r = check_ptr(a.out, "out")) || (r = check_strides(a.out_stride, 3, "out")))
    return r;
  if (a.has_D && ((r = check_ptr(a.D, "D")) || (r = check_strides(a.D_stride, 2, "D")))) return r;
  if (a.has_z && ((r = check_ptr(a.z, "z")) || (r = check_strides(a.z_stride, 3, "z")))) return r;
  if (a.has_dt_bias &&
      ((r = check_ptr(a.dt_bias, "dt_bias")) || (r = check_strides(a.dt_bias_stride, 2, "dt_bias"))))
    return r;
  return S6_OK;
}

// ---- Mamba-2 SSD ------------------------------------------------------------------------

struct SsdPlan {
  int64_t K;
  // Tile sizes of the kernels: headdim padded to 32 / 64 / 128, dstate to 32 / 64 / 128 / 256.
  // When they differ from the caller's, x, z, out (, out_x) or B, C are staged through
  // zero-padded workspace copies; zero columns add nothing to any product.
  int64_t Pp, Np;
  bool padP, padN;
  size_t off_dtq, off_dacs, off_st, off_hs, off_cb;
  size_t off_Bp, off_Cp, off_xp, off_zp, off_outp, off_outxp, total;
  size_t off_doutp, off_dxp, off_dzp;
  // backward
  int64_t nE;
  size_t off_dyw, off_dst, off_ddal, off_ddtd, off_dDp, off_qv, off_uv, off_rs, off_csp;
  size_t off_dBp, off_dCp, off_dcb, off_dAp, off_dbp, total_bwd;
};

int64_t ssd_pad_headdim(int64_t P) { return P <= 32 ? 32 : P <= 64 ? 64 : 128; }
int64_t ssd_pad_dstate(int64_t N) { return N <= 32 ? 32 : N <= 64 ? 64 : N <= 128 ? 128 : 256; }

SsdPlan ssd_plan(const S6SsdProblem& p) {
  SsdPlan s{};
  s.K = ceil_div(p.seqlen, p.chunk_size);
  s.Pp = ssd_pad_headdim(p.headdim);
  s.Np = ssd_pad_dstate(p.dstate);
  s.padP = s.Pp != p.headdim;
  s.padN = s.Np != p.dstate;
  const size_t es = (size_t)esize(p.io_dtype);
  const size_t bhkq = (size_t)(p.batch * p.nheads * s.K * p.chunk_size) * 4;
  const size_t pn = (size_t)(p.batch * s.K * p.nheads * s.Pp * s.Np);
  const size_t lhp = align256((size_t)(p.batch * p.seqlen * p.nheads * s.Pp) * es);
  const size_t lgn = align256((size_t)(p.batch * p.seqlen * p.ngroups * s.Np) * es);
  size_t off = 0;
  s.off_dtq = off; off += align256(bhkq);
  s.off_dacs = off; off += align256(bhkq);
  s.off_st = off; off += align256(pn * 4);
  s.off_hs = off; off += align256(pn * es);
  s.off_cb = off; off += align256((size_t)(p.batch * s.K * p.ngroups) * p.chunk_size * p.chunk_size * 4);
  s.off_Bp = off; off += s.padN ? lgn : 0;
  s.off_Cp = off; off += s.padN ? lgn : 0;
  s.off_xp = off; off += s.padP ? lhp : 0;
  s.off_zp = off; off += (s.padP && p.has_z) ? lhp : 0;
  s.off_outp = off; off += s.padP ? lhp : 0;
  s.off_outxp = off; off += (s.padP && p.has_z) ? lhp : 0;
  s.total = off;
  s.off_doutp = off; off += s.padP ? lhp : 0;
  s.off_dxp = off; off += s.padP ? lhp : 0;
  s.off_dzp = off; off += (s.padP && p.has_z) ? lhp : 0;
  const int64_t qt = p.chunk_size / 64;
  s.nE = s.Pp * s.Np / 1024;
  s.off_dyw = off; off += p.has_z ? lhp : 0;
  s.off_dst = off; off += align256(pn * (size_t)esize(p.io_dtype));
  s.off_ddal = off; off += align256((size_t)(p.batch * p.nheads * s.K * s.nE) * 4);
  s.off_ddtd = off; off += align256(bhkq);
  s.off_dDp = off; off += align256((size_t)(p.batch * s.K * qt * p.nheads * s.Pp) * 4);
  const size_t nsl = (size_t)(s.Np / (s.Np < 64 ? s.Np : 64));  // dstate slices of the row kernels
  s.off_qv = off; off += align256(bhkq * nsl);
  s.off_uv = off; off += align256(bhkq * nsl);
  s.off_rs = off; off += align256(bhkq * (size_t)qt);  // one partial per column tile
  s.off_csp = off; off += align256(bhkq * (size_t)qt);
  const size_t lgn4 = (size_t)(p.batch * p.seqlen * p.ngroups * s.Np) * 4;
  s.off_dBp = off; off += align256(lgn4);
  s.off_dCp = off; off += align256(lgn4);
  s.off_dcb = off; off += align256((size_t)(p.batch * s.K * p.ngroups) * p.chunk_size * p.chunk_size * 4);
  s.off_dAp = off; off += align256((size_t)(p.batch * s.K * p.nheads) * 4);
  s.off_dbp = off; off += align256((size_t)(p.batch * s.K * p.nheads) * 4);
  s.total_bwd = off;
  return s;
}

int ssd_check_problem(const S6SsdProblem& p) {
  if (p.batch < 1 || p.seqlen < 1 || p.nheads < 1 || p.ngroups < 1)
    return fail(S6_E_INVALID, "ssd: batch, seqlen, nheads, ngroups must be >= 1");
  if (p.nheads % p.ngroups != 0)
    return fail(S6_E_INVALID, "ssd: nheads must be divisible by ngroups");
  if (p.headdim < 1 || p.headdim > 128)
    return fail(S6_E_UNSUPPORTED, "ssd: headdim must be 1..128, got %lld", (long long)p.headdim);
  if (p.dstate < 1 || p.dstate > 256)
    return fail(S6_E_UNSUPPORTED, "ssd: dstate must be 1..256, got %lld", (long long)p.dstate);
  if (p.chunk_size < 64 || p.chunk_size > 256 || p.chunk_size % 64 != 0)
    return fail(S6_E_UNSUPPORTED, "ssd: chunk_size must be 64, 128, 192 or 256, got %lld",
                (long long)p.chunk_size);
  if (p.io_dtype != S6_BF16 && p.io_dtype != S6_F16 && p.io_dtype != S6_F32)
    return fail(S6_E_UNSUPPORTED, "ssd: io dtype must be bf16, fp16 or fp32");
  if (ceil_div(p.seqlen, p.chunk_size) > 65535 || p.batch * p.nheads > 65535 || p.batch > 65535)
    return fail(S6_E_UNSUPPORTED, "ssd: too many chunks or batch * nheads above 65535");
  if ((p.chunk_size / 64) * ceil_div(p.seqlen, p.chunk_size) * p.batch * p.nheads >= ((int64_t)1 << 31))
    return fail(S6_E_UNSUPPORTED, "ssd: batch * nheads * seqlen / 64 must be below 2^31");
  if (!(p.dt_min <= p.dt_max)) return fail(S6_E_INVALID, "ssd: dt_limit must satisfy min <= max");
  return S6_OK;
}

// Rows read with 16-byte vector loads: unit stride along the last axis and 16-byte aligned
// row starts.
int ssd_check_rows(const void* ptr, const int64_t* s, int es, const char* name) {
  if (s[3] != 1) return fail(S6_E_INVALID, "ssd: %s must have unit stride along its last axis", name);
  if ((uintptr_t)ptr % 16 != 0 || (s[0] * es) % 16 != 0 || (s[1] * es) % 16 != 0 ||
      (s[2] * es) % 16 != 0)
    return fail(S6_E_INVALID, "ssd: %s rows must start on 16-byte boundaries", name);
  return S6_OK;
}

int ssd_check_inputs(const S6SsdProblem& p, const void* x, const int64_t* sx, const void* dt,
                     const int64_t* sdt, const float* A, int64_t sA, const void* B,
                     const int64_t* sB, const void* C, const int64_t* sC, const float* D,
                     const int64_t* sD, const void* z, const int64_t* sz, const float* bias,
                     const float* init, const int64_t* sinit, const int32_t* seq,
                     const int64_t* sseq) {
  int r;
  if ((r = ssd_check_problem(p))) return r;
  const int es = esize(p.io_dtype);
  // tensors staged through padded copies are read element by element: any strides
  const bool padP = ssd_pad_headdim(p.headdim) != p.headdim;
  const bool padN = ssd_pad_dstate(p.dstate) != p.dstate;
  if ((r = check_ptr(x, "x")) || (r = check_strides(sx, 4, "x")) ||
      (!padP && (r = ssd_check_rows(x, sx, es, "x"))) || (r = check_ptr(dt, "dt")) ||
      (r = check_strides(sdt, 3, "dt")) || (r = check_ptr(A, "A")) || (r = check_ptr(B, "B")) ||
      (r = check_strides(sB, 4, "B")) || (!padN && (r = ssd_check_rows(B, sB, es, "B"))) ||
      (r = check_ptr(C, "C")) || (r = check_strides(sC, 4, "C")) ||
      (!padN && (r = ssd_check_rows(C, sC, es, "C"))))
    return r;
  if (sA < 0) return fail(S6_E_INVALID, "A has a negative stride");
  if (p.has_D && ((r = check_ptr(D, "D")) || (r = check_strides(sD, 2, "D")))) return r;
  if (p.has_z && ((r = check_ptr(z, "z")) || (r = check_strides(sz, 4, "z")) ||
                   (!padP && (r = ssd_check_rows(z, sz, es, "z")))))
    return r;
  if (p.has_dt_bias && (r = check_ptr(bias, "dt_bias"))) return r;
  if (p.has_initial_states &&
      ((r = check_ptr(init, "initial_states")) || (r = check_strides(sinit, 4, "initial_states"))))
    return r;
  if (p.has_seq_idx && ((r = check_ptr(seq, "seq_idx")) || (r = check_strides(sseq, 2, "seq_idx"))))
    return r;
  return S6_OK;
}

s6::SsdK ssd_fill(const S6SsdFwdArgs& a, const SsdPlan& pl);

// Strides of a dense [d0, d1, d2, d3] tensor.
void dense4(const int64_t d[4], int64_t s[4]) {
  s[3] = 1;
  s[2] = d[3];
  s[1] = d[2] * d[3];
  s[0] = d[1] * d[2] * d[3];
}

// Caller tensor (dims `small`, strides `ss`) into the dense padded buffer of dims `big`.
hipError_t ssd_pad(const void* src, const int64_t ss[4], const int64_t small[4], void* dst,
                   const int64_t big[4], int es, hipStream_t st) {
  int64_t ds[4];
  dense4(big, ds);
  return s6::launch_copy4d(src, ss, small, dst, ds, big, es, st);
}

// The leading `small` part of a dense padded buffer (dims `big`) into a caller tensor.
hipError_t ssd_unpad(const void* src, const int64_t big[4], void* dst, const int64_t ds[4],
                     const int64_t small[4], int es, hipStream_t st) {
  int64_t ss[4];
  dense4(big, ss);
  return s6::launch_copy4d(src, ss, big, dst, ds, small, es, st);
}

// Zero-padded copies of the inputs that the plan stages (B, C when dstate is padded; x, z
// when headdim is), into the buffers ssd_fill pointed the kernels at.
hipError_t ssd_stage_inputs(const S6SsdFwdArgs& a, const SsdPlan& pl, const s6::SsdK& k,
                            hipStream_t st) {
  const S6SsdProblem& p = a.p;
  const int es = esize(p.io_dtype);
  hipError_t e = hipSuccess;
  if (pl.padN) {
    const int64_t sm[4] = {p.batch, p.seqlen, p.ngroups, p.dstate};
    const int64_t bg[4] = {p.batch, p.seqlen, p.ngroups, pl.Np};
    if ((e = ssd_pad(a.B, a.B_stride, sm, const_cast<void*>(k.Bm), bg, es, st)) != hipSuccess ||
        (e = ssd_pad(a.C, a.C_stride, sm, const_cast<void*>(k.Cm), bg, es, st)) != hipSuccess)
      return e;
  }
  if (pl.padP) {
    const int64_t sm[4] = {p.batch, p.seqlen, p.nheads, p.headdim};
    const int64_t bg[4] = {p.batch, p.seqlen, p.nheads, pl.Pp};
    if ((e = ssd_pad(a.x, a.x_stride, sm, const_cast<void*>(k.x), bg, es, st)) != hipSuccess) return e;
    if (p.has_z && (e = ssd_pad(a.z, a.z_stride, sm, const_cast<void*>(k.z), bg, es, st)) != hipSuccess)
      return e;
  }
  return e;
}

}  // namespace

extern "C" {

int s6_ssd_validate_fwd(const S6SsdFwdArgs* a) {
  if (a == nullptr) return fail(S6_E_INVALID, "args must not be NULL");
  const S6SsdProblem& p = a->p;
  int r = ssd_check_inputs(p, a->x, a->x_stride, a->dt, a->dt_stride, a->A, a->A_stride, a->B,
                           a->B_stride, a->C, a->C_stride, a->D, a->D_stride, a->z, a->z_stride,
                           a->dt_bias, a->initial_states, a->initial_states_stride, a->seq_idx,
                           a->seq_idx_stride);
  if (r) return r;
  const int es = esize(p.io_dtype);
  const bool padP = ssd_pad_headdim(p.headdim) != p.headdim;
  if ((r = check_ptr(a->out, "out")) || (r = check_strides(a->out_stride, 4, "out")) ||
      (!padP && (r = ssd_check_rows(a->out, a->out_stride, es, "out"))))
    return r;
  if (p.has_z && a->out_x &&
      ((r = check_strides(a->out_x_stride, 4, "out_x")) ||
       (!padP && (r = ssd_check_rows(a->out_x, a->out_x_stride, es, "out_x")))))
    return r;
  if (a->varlen_states != nullptr) {
    if (p.batch != 1)
      return fail(S6_E_INVALID, "ssd: varlen states need batch 1, got %lld", (long long)p.batch);
    if (a->cu_seqlens == nullptr || a->nseq < 1)
      return fail(S6_E_INVALID, "ssd: varlen states need cu_seqlens with at least one sequence");
    if (a->nseq > 65535) return fail(S6_E_UNSUPPORTED, "ssd: at most 65535 varlen sequences");
    if ((uintptr_t)a->varlen_states % 16 != 0)
      return fail(S6_E_INVALID, "ssd: varlen_states must be 16-byte aligned");
  }
  const SsdPlan pl = ssd_plan(p);
  if (a->workspace == nullptr || a->workspace_bytes < pl.total)
    return fail(S6_E_WORKSPACE, "ssd forward workspace needs %zu bytes, got %zu", pl.total,
                a->workspace ? a->workspace_bytes : (size_t)0);
  return ok();
}

size_t s6_ssd_fwd_workspace_bytes(const S6SsdProblem* p) {
  if (p == nullptr || ssd_check_problem(*p) != S6_OK) return 0;
  return ssd_plan(*p).total;
}

int s6_ssd_fwd(const S6SsdFwdArgs* a, void* stream) {
  int r = s6_ssd_validate_fwd(a);
  if (r != S6_OK) return r;
  const S6SsdProblem& p = a->p;
  const SsdPlan pl = ssd_plan(p);
  s6::SsdK k = ssd_fill(*a, pl);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = ssd_stage_inputs(*a, pl, k, st);
  if (e == hipSuccess) e = s6::launch_ssd_fwd(k, st, a->kernel_events);
  if (e == hipSuccess && pl.padP) {
    const int es = esize(p.io_dtype);
    const int64_t sm[4] = {p.batch, p.seqlen, p.nheads, p.headdim};
    const int64_t bg[4] = {p.batch, p.seqlen, p.nheads, pl.Pp};
    e = ssd_unpad(k.out, bg, a->out, a->out_stride, sm, es, st);
    if (e == hipSuccess && k.out_x != nullptr)
      e = ssd_unpad(k.out_x, bg, a->out_x, a->out_x_stride, sm, es, st);
  }
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_ssd_fwd: %s", hipGetErrorString(e));
  return ok();
}

int s6_ssd_validate_bwd(const S6SsdBwdArgs* a) {
  if (a == nullptr) return fail(S6_E_INVALID, "args must not be NULL");
  const S6SsdProblem& p = a->p;
  int r = ssd_check_inputs(p, a->x, a->x_stride, a->dt, a->dt_stride, a->A, a->A_stride, a->B,
                           a->B_stride, a->C, a->C_stride, a->D, a->D_stride, a->z, a->z_stride,
                           a->dt_bias, a->initial_states, a->initial_states_stride, a->seq_idx,
                           a->seq_idx_stride);
  if (r) return r;
  const int es = esize(p.io_dtype);
  const bool padP = ssd_pad_headdim(p.headdim) != p.headdim;
  if ((r = check_ptr(a->dout, "dout")) || (r = check_strides(a->dout_stride, 4, "dout")) ||
      (!padP && (r = ssd_check_rows(a->dout, a->dout_stride, es, "dout"))) ||
      (r = check_ptr(a->dx, "dx")) || (r = check_strides(a->dx_stride, 4, "dx")) ||
      (!padP && (r = ssd_check_rows(a->dx, a->dx_stride, es, "dx"))) ||
      (r = check_ptr(a->ddt, "ddt")) || (r = check_strides(a->ddt_stride, 3, "ddt")) ||
      (r = check_ptr(a->dA, "dA")) || (r = check_ptr(a->dB, "dB")) ||
      (r = check_strides(a->dB_stride, 4, "dB")) || (r = check_ptr(a->dC, "dC")) ||
      (r = check_strides(a->dC_stride, 4, "dC")))
    return r;
  if (p.has_D && (r = check_ptr(a->dD, "dD"))) return r;
  if (p.has_z && ((r = check_ptr(a->out_x, "out_x")) || (r = check_strides(a->out_x_stride, 4, "out_x")) ||
                  (r = check_ptr(a->dz, "dz")) || (r = check_strides(a->dz_stride, 4, "dz"))))
    return r;
  if (p.has_dt_bias && (r = check_ptr(a->ddt_bias, "ddt_bias"))) return r;
  if (a->dfinal_states && (r = check_strides(a->dfinal_states_stride, 4, "dfinal_states"))) return r;
  const SsdPlan pl = ssd_plan(p);
  if (a->workspace == nullptr || a->workspace_bytes < pl.total_bwd)
    return fail(S6_E_WORKSPACE, "ssd backward workspace needs %zu bytes, got %zu", pl.total_bwd,
                a->workspace ? a->workspace_bytes : (size_t)0);
  return ok();
}

size_t s6_ssd_bwd_workspace_bytes(const S6SsdProblem* p) {
  if (p == nullptr || ssd_check_problem(*p) != S6_OK) return 0;
  return ssd_plan(*p).total_bwd;
}

int s6_ssd_bwd(const S6SsdBwdArgs* a, void* stream) {
  int r = s6_ssd_validate_bwd(a);
  if (r != S6_OK) return r;
  const S6SsdProblem& p = a->p;
  const SsdPlan pl = ssd_plan(p);
  S6SsdFwdArgs f{};
  f.p = p;
  f.x = a->x; f.dt = a->dt; f.A = a->A; f.A_stride = a->A_stride; f.B = a->B; f.C = a->C;
  f.D = a->D; f.z = a->z; f.dt_bias = a->dt_bias; f.dt_bias_stride = a->dt_bias_stride;
  f.initial_states = a->initial_states; f.seq_idx = a->seq_idx;
  for (int i = 0; i < 4; ++i) {
    f.x_stride[i] = a->x_stride[i]; f.B_stride[i] = a->B_stride[i]; f.C_stride[i] = a->C_stride[i];
    f.z_stride[i] = a->z_stride[i]; f.initial_states_stride[i] = a->initial_states_stride[i];
    f.out_x_stride[i] = a->out_x_stride[i];
  }
  for (int i = 0; i < 3; ++i) f.dt_stride[i] = a->dt_stride[i];
  for (int i = 0; i < 2; ++i) { f.D_stride[i] = a->D_stride[i]; f.seq_idx_stride[i] = a->seq_idx_stride[i]; }
  f.out_x = const_cast<void*>(a->out_x);
  f.workspace = a->workspace; f.workspace_bytes = a->workspace_bytes;
  s6::SsdK k = ssd_fill(f, pl);
  char* ws = (char*)a->workspace;
  k.final_states = nullptr;
  k.dout = a->dout;
  for (int i = 0; i < 4; ++i) {
    k.sdout[i] = a->dout_stride[i]; k.sdx[i] = a->dx_stride[i];
    k.sdBo[i] = a->dB_stride[i]; k.sdCo[i] = a->dC_stride[i];
    k.sdz[i] = p.has_z ? a->dz_stride[i] : 0;
    k.sdfinal[i] = a->dfinal_states ? a->dfinal_states_stride[i] : 0;
  }
  for (int i = 0; i < 3; ++i) k.sddt[i] = a->ddt_stride[i];
  if (p.has_z) {
    k.dyw = ws + pl.off_dyw;
    k.dy = k.dyw;
    const int64_t P = pl.Pp, H = p.nheads, L = p.seqlen;
    k.sdy[0] = L * H * P; k.sdy[1] = H * P; k.sdy[2] = P; k.sdy[3] = 1;
  } else {
    k.dy = a->dout;
    for (int i = 0; i < 4; ++i) k.sdy[i] = a->dout_stride[i];
  }
  k.dz = p.has_z ? a->dz : nullptr; k.dx = a->dx; k.ddt = a->ddt; k.dBo = a->dB; k.dCo = a->dC;
  hipStream_t st = (hipStream_t)stream;
  const int es = esize(p.io_dtype);
  const int64_t smP[4] = {p.batch, p.seqlen, p.nheads, p.headdim};
  const int64_t bgP[4] = {p.batch, p.seqlen, p.nheads, pl.Pp};
  hipError_t e = ssd_stage_inputs(f, pl, k, st);
  if (e == hipSuccess && pl.padP) {  // dout, the forward's out_x, dx and dz through padded copies
    int64_t dsP[4];
    dense4(bgP, dsP);
    k.dout = ws + pl.off_doutp;
    for (int i = 0; i < 4; ++i) k.sdout[i] = dsP[i];
    e = ssd_pad(a->dout, a->dout_stride, smP, ws + pl.off_doutp, bgP, es, st);
    if (!p.has_z) {
      k.dy = k.dout;
      for (int i = 0; i < 4; ++i) k.sdy[i] = dsP[i];
    }
    if (e == hipSuccess && p.has_z)  // ssd_fill pointed k.out_x at the padded buffer
      e = ssd_pad(a->out_x, a->out_x_stride, smP, k.out_x, bgP, es, st);
    k.dx = ws + pl.off_dxp;
    if (p.has_z) k.dz = ws + pl.off_dzp;
    for (int i = 0; i < 4; ++i) {
      k.sdx[i] = dsP[i];
      if (p.has_z) k.sdz[i] = dsP[i];
    }
  }
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_ssd_bwd: %s", hipGetErrorString(e));
  k.dA = a->dA; k.dD = p.has_D ? a->dD : nullptr; k.ddt_bias = p.has_dt_bias ? a->ddt_bias : nullptr;
  k.dinit = a->dinitial_states; k.dfinal = a->dfinal_states;
  k.dhl = k.st;  // the chunk states are consumed by the recomputed state passing first
  k.dst = ws + pl.off_dst; k.ddal = (float*)(ws + pl.off_ddal); k.nE = pl.nE;
  k.ddtd = (float*)(ws + pl.off_ddtd); k.dDp = (float*)(ws + pl.off_dDp);
  k.qv = (float*)(ws + pl.off_qv); k.uv = (float*)(ws + pl.off_uv); k.rs = (float*)(ws + pl.off_rs);
  k.csp = (float*)(ws + pl.off_csp); k.dBp = (float*)(ws + pl.off_dBp); k.dCp = (float*)(ws + pl.off_dCp);
  k.dcb = (float*)(ws + pl.off_dcb); k.dAp = (float*)(ws + pl.off_dAp); k.dbp = (float*)(ws + pl.off_dbp);
  e = s6::launch_ssd_bwd(k, st);
  if (e == hipSuccess && pl.padP) {
    e = ssd_unpad(k.dx, bgP, a->dx, a->dx_stride, smP, es, st);
    if (e == hipSuccess && p.has_z) e = ssd_unpad(k.dz, bgP, a->dz, a->dz_stride, smP, es, st);
  }
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_ssd_bwd: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"

namespace {

s6::SsdK ssd_fill(const S6SsdFwdArgs& a0, const SsdPlan& pl) {
  const S6SsdFwdArgs* a = &a0;
  const S6SsdProblem& p = a->p;
  s6::SsdK k{};
  k.Bsz = p.batch; k.L = p.seqlen; k.H = p.nheads; k.P = p.headdim; k.G = p.ngroups;
  k.N = p.dstate; k.Q = p.chunk_size; k.K = pl.K; k.hpg = p.nheads / p.ngroups;
  k.io = p.io_dtype;
  k.softplus = p.dt_softplus; k.has_bias = p.has_dt_bias; k.has_D = p.has_D;
  k.D_hdim = p.D_has_hdim; k.has_z = p.has_z; k.has_init = p.has_initial_states;
  k.has_seq = p.has_seq_idx; k.dt_min = p.dt_min; k.dt_max = p.dt_max;
  k.x = a->x; k.dt = a->dt; k.A = a->A; k.sA = a->A_stride; k.Bm = a->B; k.Cm = a->C;
  k.Dp = p.has_D ? a->D : nullptr; k.z = p.has_z ? a->z : nullptr;
  k.bias = p.has_dt_bias ? a->dt_bias : nullptr; k.sbias = a->dt_bias_stride;
  k.init = p.has_initial_states ? a->initial_states : nullptr;
  k.seq = p.has_seq_idx ? a->seq_idx : nullptr;
  k.out = a->out; k.out_x = p.has_z ? a->out_x : nullptr; k.final_states = a->final_states;
  k.cu = a->cu_seqlens; k.nseq = a->varlen_states ? a->nseq : 0; k.vst = a->varlen_states;
  for (int i = 0; i < 4; ++i) {
    k.sx[i] = a->x_stride[i]; k.sB[i] = a->B_stride[i]; k.sC[i] = a->C_stride[i];
    k.sz[i] = p.has_z ? a->z_stride[i] : 0; k.sout[i] = a->out_stride[i];
    k.soutx[i] = (p.has_z && a->out_x) ? a->out_x_stride[i] : 0;
    k.sinit[i] = p.has_initial_states ? a->initial_states_stride[i] : 0;
  }
  for (int i = 0; i < 3; ++i) k.sdt[i] = a->dt_stride[i];
  for (int i = 0; i < 2; ++i) {
    k.sD[i] = p.has_D ? a->D_stride[i] : 0;
    k.sseq[i] = p.has_seq_idx ? a->seq_idx_stride[i] : 0;
  }
  char* ws = (char*)a->workspace;
  k.dtq = (float*)(ws + pl.off_dtq); k.dacs = (float*)(ws + pl.off_dacs);
  k.st = (float*)(ws + pl.off_st); k.hs = ws + pl.off_hs; k.cb = (float*)(ws + pl.off_cb);
  k.P = pl.Pp; k.N = pl.Np; k.Pa = p.headdim; k.Na = p.dstate;
  if (pl.padN) {
    const int64_t d[4] = {p.batch, p.seqlen, p.ngroups, pl.Np};
    k.Bm = ws + pl.off_Bp; k.Cm = ws + pl.off_Cp;
    dense4(d, k.sB);
    dense4(d, k.sC);
  }
  if (pl.padP) {
    const int64_t d[4] = {p.batch, p.seqlen, p.nheads, pl.Pp};
    k.x = ws + pl.off_xp;
    dense4(d, k.sx);
    if (p.has_z) { k.z = ws + pl.off_zp; dense4(d, k.sz); }
    k.out = ws + pl.off_outp;
    dense4(d, k.sout);
    if (k.out_x != nullptr) { k.out_x = ws + pl.off_outxp; dense4(d, k.soutx); }
  }
  return k;
}

}  // namespace

extern "C" {

int s6_validate_state_update(const S6StateUpdateArgs* a) {
  if (a == nullptr) return fail(S6_E_INVALID, "args must not be NULL");
  int r = ssu_check(*a);
  return r != S6_OK ? r : ok();
}

int s6_selective_state_update(const S6StateUpdateArgs* a, void* stream) {
  int r = s6_validate_state_update(a);
  if (r != S6_OK) return r;
  s6::SsuK k{};
  k.batch = a->batch; k.nheads = a->nheads; k.dim = a->dim; k.dstate = a->dstate;
  k.hpg = a->nheads / a->ngroups;
  k.io = a->io_dtype; k.bc = a->bc_dtype;
  k.state = a->state; k.x = a->x; k.dt = a->dt; k.A = a->A; k.B = a->B; k.C = a->C;
  k.out = a->out;
  k.bias = a->has_dt_bias ? a->dt_bias : nullptr;
  k.Dp = a->has_D ? a->D : nullptr;
  k.z = a->has_z ? a->z : nullptr;
  for (int i = 0; i < 4; ++i) k.ss[i] = a->state_stride[i];
  for (int i = 0; i < 3; ++i) {
    k.sx[i] = a->x_stride[i]; k.sdt[i] = a->dt_stride[i]; k.sA[i] = a->A_stride[i];
    k.sB[i] = a->B_stride[i]; k.sC[i] = a->C_stride[i]; k.so[i] = a->out_stride[i];
    k.sz[i] = a->has_z ? a->z_stride[i] : 0;
  }
  for (int i = 0; i < 2; ++i) {
    k.sbias[i] = a->has_dt_bias ? a->dt_bias_stride[i] : 0;
    k.sD[i] = a->has_D ? a->D_stride[i] : 0;
  }
  // Row mapping: 4 contiguous states per lane in one 16-byte (fp32) or 8-byte load; A and
  // B / C rows vector-loaded when their layout allows it.
  auto rows4 = [](const void* p, const int64_t* st, int n, int es) {
    if (st[n - 1] != 1 || (uintptr_t)p % (uintptr_t)(4 * es) != 0) return false;
    for (int i = 0; i < n - 1; ++i)
      if (st[i] % 4 != 0) return false;
    return true;
  };
  const bool rows = a->dstate % 4 == 0 && rows4(a->state, a->state_stride, 4, esize(a->state_dtype));
  k.a_vec = rows4(a->A, a->A_stride, 3, 4);
  k.bc_vec = rows4(a->B, a->B_stride, 3, esize(a->bc_dtype)) &&
             rows4(a->C, a->C_stride, 3, esize(a->bc_dtype));
  hipError_t e = s6::launch_state_update(k, a->state_dtype, a->dt_softplus != 0, rows,
                                         (hipStream_t)stream);
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_selective_state_update: %s", hipGetErrorString(e));
  return ok();
}

int s6_causal_conv1d_validate_fwd(const S6ConvFwdArgs* a) {
  if (a == nullptr) return fail(S6_E_INVALID, "args must not be NULL");
  int r;
  if ((r = conv_check_common(a->p, a->x, a->x_stride, a->weight, a->weight_stride)) ||
      (r = check_ptr(a->out, "out")) || (r = check_strides(a->out_stride, 3, "out")))
    return r;
  return ok();
}

int s6_causal_conv1d_validate_bwd(const S6ConvBwdArgs* a) {
  if (a == nullptr) return fail(S6_E_INVALID, "args must not be NULL");
  int r;
  if ((r = conv_check_common(a->p, a->x, a->x_stride, a->weight, a->weight_stride)) ||
      (r = check_ptr(a->dout, "dout")) || (r = check_strides(a->dout_stride, 3, "dout")) ||
      (r = check_ptr(a->dx, "dx")) || (r = check_strides(a->dx_stride, 3, "dx")) ||
      (r = check_ptr(a->dweight, "dweight")) || (r = check_strides(a->dweight_stride, 2, "dweight")))
    return r;
  const ConvPlan c = conv_plan(a->p);
  if (a->workspace == nullptr || a->workspace_bytes < c.ws_bytes)
    return fail(S6_E_WORKSPACE, "causal_conv1d backward workspace needs %zu bytes, got %zu",
                c.ws_bytes, a->workspace ? a->workspace_bytes : (size_t)0);
  return ok();
}

size_t s6_causal_conv1d_bwd_workspace_bytes(const S6ConvProblem* p) {
  if (p == nullptr || conv_check_problem(*p) != S6_OK) return 0;
  return conv_plan(*p).ws_bytes;
}

int s6_causal_conv1d_fwd(const S6ConvFwdArgs* a, void* stream) {
  int r = s6_causal_conv1d_validate_fwd(a);
  if (r != S6_OK) return r;
  const S6ConvProblem& p = a->p;
  const int es = esize(p.io_dtype);
  const void* ptrs[2] = {a->x, a->out};
  const int64_t* strides[2] = {a->x_stride, a->out_stride};
  const int64_t vec = conv_pick_vec(p.dim, es, false, ptrs, strides, 2);
  s6::ConvK k = conv_fill(p, conv_plan(p), vec);
  for (int i = 0; i < 3; ++i) { k.sx[i] = a->x_stride[i]; k.so[i] = a->out_stride[i]; }
  k.sw[0] = a->weight_stride[0]; k.sw[1] = a->weight_stride[1]; k.sb = a->bias_stride;
  k.x = a->x; k.w = a->weight; k.bias = a->bias; k.out = a->out;
  hipError_t e = s6::launch_conv_fwd(k, p.io_dtype, (int)p.width, (int)vec, p.silu != 0,
                                     (hipStream_t)stream);
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_causal_conv1d_fwd: %s", hipGetErrorString(e));
  return ok();
}

int s6_causal_conv1d_bwd(const S6ConvBwdArgs* a, void* stream) {
  int r = s6_causal_conv1d_validate_bwd(a);
  if (r != S6_OK) return r;
  const S6ConvProblem& p = a->p;
  const int es = esize(p.io_dtype);
  const void* ptrs[3] = {a->x, a->dout, a->dx};
  const int64_t* strides[3] = {a->x_stride, a->dout_stride, a->dx_stride};
  const int64_t vec = conv_pick_vec(p.dim, es, true, ptrs, strides, 3);
  s6::ConvK k = conv_fill(p, conv_plan(p), vec);
  for (int i = 0; i < 3; ++i) {
    k.sx[i] = a->x_stride[i]; k.sdo[i] = a->dout_stride[i]; k.sdx[i] = a->dx_stride[i];
  }
  k.sw[0] = a->weight_stride[0]; k.sw[1] = a->weight_stride[1]; k.sb = a->bias_stride;
  k.sdw[0] = a->dweight_stride[0]; k.sdw[1] = a->dweight_stride[1]; k.sdb = a->dbias_stride;
  k.x = a->x; k.w = a->weight; k.bias = a->bias; k.dout = a->dout; k.dx = a->dx;
  const ConvPlan c = conv_plan(p);
  k.dw = a->dweight; k.dbias = a->dbias; k.ws = (float*)a->workspace;
  k.ws2 = (float*)((char*)a->workspace + c.off_ws2);
  hipError_t e = s6::launch_conv_bwd(k, p.io_dtype, (int)p.width, (int)vec, p.silu != 0,
                                     (hipStream_t)stream);
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_causal_conv1d_bwd: %s", hipGetErrorString(e));
  return ok();
}

int s6_abi_version(void) { return S6_ABI_VERSION; }

const char* s6_last_error(void) { return g_last_error.c_str(); }

int s6_validate_problem(const S6Problem* p) {
  if (p == nullptr) return fail(S6_E_INVALID, "problem must not be NULL");
  if (p->batch < 1 || p->dim < 1 || p->seqlen < 1 || p->dstate < 1 || p->ngroups < 1)
    return fail(S6_E_INVALID,
                "batch, dim, seqlen, dstate and ngroups must be >= 1 (got %lld, %lld, %lld, %lld, %lld)",
                (long long)p->batch, (long long)p->dim, (long long)p->seqlen,
                (long long)p->dstate, (long long)p->ngroups);
  if (p->dim % p->ngroups != 0)
    return fail(S6_E_INVALID, "dim (%lld) must be divisible by the number of B/C groups (%lld)",
                (long long)p->dim, (long long)p->ngroups);
  for (int dt : {p->io_dtype, p->bc_dtype})
    if (dt != S6_F32 && dt != S6_BF16 && dt != S6_F16)
      return fail(S6_E_INVALID, "unknown dtype code %d", dt);
  if (p->dstate > S6_MAX_DSTATE_FWD)
    return fail(S6_E_UNSUPPORTED, "dstate %lld exceeds the supported maximum %d",
                (long long)p->dstate, S6_MAX_DSTATE_FWD);
  if (p->nseq < 0) return fail(S6_E_INVALID, "nseq must be >= 0");
  if (p->nseq > 0 && p->batch != 1)
    return fail(S6_E_INVALID, "packed varlen input (cu_seqlens) requires batch == 1, got %lld",
                (long long)p->batch);
  if (p->seqlen > (int64_t)INT32_MAX)
    return fail(S6_E_UNSUPPORTED, "seqlen must fit in int32 for cu_seqlens offsets");
  return ok();
}

int s6_fwd_single_pass(const S6Problem* p) {
  int r = s6_validate_problem(p);
  if (r != S6_OK) return r;
  return make_plan(*p, false, nullptr, nullptr, nullptr, nullptr).lanes ? 1 : 0;
}

int s6_validate_cu_seqlens(const int32_t* cu, int64_t nseq, int64_t seqlen) {
  if (cu == nullptr) return fail(S6_E_INVALID, "cu_seqlens must not be NULL");
  if (nseq < 1 || nseq > (int64_t)INT32_MAX - 1)
    return fail(S6_E_INVALID, "cu_seqlens must hold nseq + 1 offsets with 1 <= nseq < 2^31-1, got nseq %lld",
                (long long)nseq);
  if (cu[0] != 0) return fail(S6_E_INVALID, "cu_seqlens[0] must be 0, got %d", cu[0]);
  for (int64_t i = 1; i <= nseq; ++i)
    if (cu[i] < cu[i - 1])
      return fail(S6_E_INVALID, "cu_seqlens must be non-decreasing: cu_seqlens[%lld] = %d < cu_seqlens[%lld] = %d",
                  (long long)i, cu[i], (long long)(i - 1), cu[i - 1]);
  if ((int64_t)cu[nseq] != seqlen)
    return fail(S6_E_INVALID, "cu_seqlens[%lld] must equal seqlen %lld, got %d", (long long)nseq,
                (long long)seqlen, cu[nseq]);
  return ok();
}

int64_t s6_num_checkpoints(const S6Problem* p) {
  if (p == nullptr || p->seqlen < 1) return 0;
  return ceil_div(p->seqlen, s6::kCk);
}

size_t s6_fwd_workspace_bytes(const S6Problem* p) {
  if (s6_validate_problem(p) != S6_OK) return 0;
  return make_plan(*p, false, nullptr, nullptr, nullptr, nullptr).total_fwd;
}

size_t s6_bwd_workspace_bytes(const S6Problem* p) {
  if (s6_validate_problem(p) != S6_OK) return 0;
  return make_plan(*p, true, nullptr, nullptr, nullptr, nullptr).total_bwd;
}

int s6_validate_fwd(const S6FwdArgs* a) { return validate_fwd(a, true); }

int s6_bwd_row_blocks(const S6BwdArgs* a) {
  if (a == nullptr) return fail(S6_E_INVALID, "args must not be NULL");
  int r = s6_validate_problem(&a->p);
  if (r != S6_OK) return r;
  return choose_rowvec_bwd(*a) ? 1 : 0;
}

int s6_fwd_kernel(const S6FwdArgs* a) {
  int r = validate_fwd(a, false);
  if (r != S6_OK) return r;
  const Plan pl = fwd_plan(*a);
  if (pl.lanes) return S6_FWD_SINGLE_PASS;
  return choose_rowvec(*a, pl) ? S6_FWD_CHUNKED_ROWS : S6_FWD_CHUNKED;
}

}  // extern "C"

namespace {

// Forward argument checks; the workspace size is checked unless the caller supplies the
// workspace itself (the no-allocation entry point).
int validate_fwd(const S6FwdArgs* a, bool check_workspace) {
  if (a == nullptr) return fail(S6_E_INVALID, "args must not be NULL");
  const S6Problem& p = a->p;
  int r = check_common(p, a->u, a->u_stride, a->delta, a->delta_stride, a->A, a->A_stride,
                       a->B, a->B_stride, a->C, a->C_stride, a->D, a->z, a->z_stride,
                       a->delta_bias, a->cu_seqlens);
  if (r != S6_OK) return r;
  if ((r = check_ptr(a->out, "out")) || (r = check_strides(a->out_stride, 3, "out"))) return r;
  if (p.has_z && ((r = check_ptr(a->out_z, "out_z")) || (r = check_strides(a->out_z_stride, 3, "out_z"))))
    return r;
  if (a->x_ckpt != nullptr && (r = check_ckpt(a->x_ckpt_stride))) return r;
  const Plan pl = fwd_plan(*a);
  const int es = esize(p.io_dtype);
  // (the single-pass kernel addresses its tensors with 64-bit indices)
  if (!pl.lanes &&
      ((r = check_span(a->u_stride, es, pl.Lc, "u")) || (r = check_span(a->delta_stride, es, pl.Lc, "delta")) ||
       (r = check_span(a->out_stride, es, pl.Lc, "out")) ||
       (p.has_z && ((r = check_span(a->z_stride, es, pl.Lc, "z")) || (r = check_span(a->out_z_stride, es, pl.Lc, "out_z"))))))
    return r;
  if (check_workspace && pl.total_fwd > 0 &&
      (a->workspace == nullptr || a->workspace_bytes < pl.total_fwd))
    return fail(S6_E_WORKSPACE, "forward workspace needs %zu bytes, got %zu", pl.total_fwd,
                a->workspace ? a->workspace_bytes : (size_t)0);
  return ok();
}

}  // namespace

extern "C" {

int s6_validate_bwd(const S6BwdArgs* a) {
  if (a == nullptr) return fail(S6_E_INVALID, "args must not be NULL");
  const S6Problem& p = a->p;
  int r = check_common(p, a->u, a->u_stride, a->delta, a->delta_stride, a->A, a->A_stride,
                       a->B, a->B_stride, a->C, a->C_stride, a->D, a->z, a->z_stride,
                       a->delta_bias, a->cu_seqlens);
  if (r != S6_OK) return r;
  if (p.dstate > S6_MAX_DSTATE_BWD)
    return fail(S6_E_UNSUPPORTED, "backward supports dstate <= %d, got %lld", S6_MAX_DSTATE_BWD,
                (long long)p.dstate);
  if ((r = check_ptr(a->dout, "dout")) || (r = check_strides(a->dout_stride, 3, "dout")) ||
      (r = check_ptr(a->x_ckpt, "x_ckpt")) || (r = check_ckpt(a->x_ckpt_stride)) ||
      (r = check_ptr(a->du, "du")) ||
      (r = check_strides(a->du_stride, 3, "du")) || (r = check_ptr(a->ddelta, "ddelta")) ||
      (r = check_strides(a->ddelta_stride, 3, "ddelta")) || (r = check_ptr(a->dA, "dA")) ||
      (r = check_strides(a->dA_stride, 2, "dA")) || (r = check_ptr(a->dB, "dB")) ||
      (r = check_strides(a->dB_stride, 4, "dB")) || (r = check_ptr(a->dC, "dC")) ||
      (r = check_strides(a->dC_stride, 4, "dC")))
    return r;
  if (p.has_D && (r = check_ptr(a->dD, "dD"))) return r;
  if (p.has_z && ((r = check_ptr(a->dz, "dz")) || (r = check_strides(a->dz_stride, 3, "dz")) ||
                  (r = check_ptr(a->out, "out")) || (r = check_strides(a->out_stride, 3, "out"))))
    return r;
  if (p.has_delta_bias && (r = check_ptr(a->ddelta_bias, "ddelta_bias"))) return r;
  const bool want_oz = p.has_z && a->out_z != nullptr;
  if (want_oz && (r = check_strides(a->out_z_stride, 3, "out_z"))) return r;
  const Plan pl = make_plan(p, true, a->B, a->B_stride, a->C, a->C_stride);
  const int es = esize(p.io_dtype);
  if ((r = check_span(a->u_stride, es, pl.Lc, "u")) || (r = check_span(a->delta_stride, es, pl.Lc, "delta")) ||
      (r = check_span(a->dout_stride, es, pl.Lc, "dout")) || (r = check_span(a->du_stride, es, pl.Lc, "du")) ||
      (r = check_span(a->ddelta_stride, es, pl.Lc, "ddelta")) ||
      (p.has_z && ((r = check_span(a->z_stride, es, pl.Lc, "z")) || (r = check_span(a->out_stride, es, pl.Lc, "out")) ||
                   (r = check_span(a->dz_stride, es, pl.Lc, "dz")))) ||
      (want_oz && (r = check_span(a->out_z_stride, es, pl.Lc, "out_z"))))
    return r;
  if (pl.total_bwd > 0 && (a->workspace == nullptr || a->workspace_bytes < pl.total_bwd))
    return fail(S6_E_WORKSPACE, "backward workspace needs %zu bytes, got %zu", pl.total_bwd,
                a->workspace ? a->workspace_bytes : (size_t)0);
  return ok();
}

int s6_fwd(const S6FwdArgs* a, void* stream) {
  int r = s6_validate_fwd(a);
  if (r != S6_OK) return r;
  return run_fwd(*a, (hipStream_t)stream);
}

// The forward with its workspace in the library's per-device scratch array.
int s6_fwd_noalloc(const S6FwdArgs* a, void* stream) {
  int r = validate_fwd(a, false);
  if (r != S6_OK) return r;
  const Plan pl = fwd_plan(*a);
  if (pl.total_fwd > (size_t)S6_NOALLOC_SCRATCH_BYTES)
    return fail(S6_E_WORKSPACE,
                "s6_fwd_noalloc: this problem needs %zu bytes of scratch, above the library's "
                "fixed %d; call s6_fwd with a workspace instead",
                pl.total_fwd, S6_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((r = scratch_for_stream((hipStream_t)stream, &ws)) != S6_OK) return r;
  S6FwdArgs b = *a;
  b.workspace = ws;
  b.workspace_bytes = S6_NOALLOC_SCRATCH_BYTES;
  return run_fwd(b, (hipStream_t)stream);
}

}  // extern "C"

namespace {

// Launches of a validated forward.
int run_fwd(const S6FwdArgs& args, hipStream_t st) {
  const S6FwdArgs* a = &args;
  const S6Problem& p = a->p;
  const Plan pl = fwd_plan(*a);
  char* ws = (char*)a->workspace;
  hipError_t e = hipSuccess;
  if (pl.relayout_B)
    e = s6::launch_relayout(a->B, a->B_stride, esize(p.bc_dtype), ws + pl.off_B, p.batch,
                            p.ngroups, p.dstate, pl.NP, p.seqlen, st);
  if (e == hipSuccess && pl.relayout_C)
    e = s6::launch_relayout(a->C, a->C_stride, esize(p.bc_dtype), ws + pl.off_C, p.batch,
                            p.ngroups, p.dstate, pl.NP, p.seqlen, st);
  if (e == hipSuccess && a->last_state != nullptr && p.nseq > 0)
    e = s6::launch_fill(a->last_state, (int64_t)p.nseq * p.dim * p.dstate, 0.f, st);
  if (e == hipSuccess) {
    s6::FwdK k = fill_fwd(*a, pl);
    e = s6::launch_fwd(k, p.io_dtype, p.bc_dtype, st, a->kernel_events);
  }
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_fwd: %s", hipGetErrorString(e));
  return ok();
}

}  // namespace

extern "C" {

int s6_bwd(const S6BwdArgs* a, void* stream) {
  int r = s6_validate_bwd(a);
  if (r != S6_OK) return r;
  const S6Problem& p = a->p;
  hipStream_t st = (hipStream_t)stream;
  const Plan pl = make_plan(p, true, a->B, a->B_stride, a->C, a->C_stride);
  char* ws = (char*)a->workspace;
  hipError_t e = hipSuccess;
  if (pl.relayout_B)
    e = s6::launch_relayout(a->B, a->B_stride, esize(p.bc_dtype), ws + pl.off_B, p.batch,
                            p.ngroups, p.dstate, pl.NP, p.seqlen, st);
  if (e == hipSuccess && pl.relayout_C)
    e = s6::launch_relayout(a->C, a->C_stride, esize(p.bc_dtype), ws + pl.off_C, p.batch,
                            p.ngroups, p.dstate, pl.NP, p.seqlen, st);
  if (e == hipSuccess) {
    s6::BwdK k{};
    k.Bsz = p.batch; k.D = p.dim; k.L = p.seqlen; k.N = p.dstate; k.G = p.ngroups;
    for (int i = 0; i < 3; ++i) {
      k.su[i] = a->u_stride[i]; k.sdl[i] = a->delta_stride[i];
      k.sz[i] = p.has_z ? a->z_stride[i] : 0;
      k.sdo[i] = a->dout_stride[i];
      k.sout[i] = p.has_z ? a->out_stride[i] : 0;
      k.sdu[i] = a->du_stride[i]; k.sddl[i] = a->ddelta_stride[i];
      k.sdz[i] = p.has_z ? a->dz_stride[i] : 0;
      k.soz[i] = (p.has_z && a->out_z) ? a->out_z_stride[i] : 0;
    }
    k.sA[0] = a->A_stride[0]; k.sA[1] = a->A_stride[1];
    k.sD = a->D_stride; k.sbias = a->delta_bias_stride;
    const int64_t NP = pl.NP;
    if (pl.relayout_B) {
      k.Bm = ws + pl.off_B;
      k.sB[0] = p.ngroups * p.seqlen * NP; k.sB[1] = p.seqlen * NP; k.sB[2] = 1; k.sB[3] = NP;
    } else {
      k.Bm = a->B;
      for (int i = 0; i < 4; ++i) k.sB[i] = a->B_stride[i];
    }
    if (pl.relayout_C) {
      k.Cm = ws + pl.off_C;
      k.sC[0] = p.ngroups * p.seqlen * NP; k.sC[1] = p.seqlen * NP; k.sC[2] = 1; k.sC[3] = NP;
    } else {
      k.Cm = a->C;
      for (int i = 0; i < 4; ++i) k.sC[i] = a->C_stride[i];
    }
    k.sdA[0] = a->dA_stride[0]; k.sdA[1] = a->dA_stride[1];
    k.sdD = a->dD_stride; k.sdbias = a->ddelta_bias_stride;
    for (int i = 0; i < 4; ++i) { k.sdB[i] = a->dB_stride[i]; k.sdC[i] = a->dC_stride[i]; }
    k.u = a->u; k.delta = a->delta; k.z = a->z; k.dout = a->dout; k.out = a->out;
    k.A = a->A; k.Dp = a->D; k.bias = a->delta_bias;
    k.cu = a->cu_seqlens; k.nseq = p.nseq;
    k.x_ckpt = a->x_ckpt; k.nck = pl.nck;
    ckpt_strides(a->x_ckpt_stride, p, pl.nck, k.sck);
    k.du = a->du; k.ddelta = a->ddelta; k.dz = a->dz;
    k.out_z = p.has_z ? a->out_z : nullptr;
    k.dA = a->dA; k.dD = a->dD; k.dbias = a->ddelta_bias; k.dB = a->dB; k.dC = a->dC;
    k.ws_g = pl.K > 1 ? (float*)(ws + pl.off_h) : nullptr;
    k.ws_s = pl.K > 1 ? (float*)(ws + pl.off_s) : nullptr;
    k.ws_r = (pl.K > 1 && p.nseq > 0) ? (int32_t*)(ws + pl.off_r) : nullptr;
    k.ws_pB = (float*)(ws + pl.off_pB);
    k.ws_pC = (float*)(ws + pl.off_pC);
    k.ws_dA = (float*)(ws + pl.off_dA);
    k.ws_dD = p.has_D ? (float*)(ws + pl.off_dD) : nullptr;
    k.ws_db = p.has_delta_bias ? (float*)(ws + pl.off_db) : nullptr;
    k.K = pl.K; k.Lc = pl.Lc;
    k.nDblk = pl.nDblk; k.nJ = pl.nJ; k.nsg = pl.nsg; k.NPr = pl.NPr;
    k.has_D = p.has_D; k.has_z = p.has_z; k.has_bias = p.has_delta_bias; k.softplus = p.delta_softplus;
    k.rowvec = choose_rowvec_bwd(*a) ? 1 : 0;
    e = s6::launch_bwd(k, p.io_dtype, p.bc_dtype, st, a->kernel_events);
  }
  if (e != hipSuccess) return fail(S6_E_HIP, "s6_bwd: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"
