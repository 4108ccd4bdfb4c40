// extern "C" entry points of libssmscan.so (declared in include/ssm_scan.h).
//
// Host-only work lives here: argument validation (callable without a device, so the error
// paths are testable on a CPU host), workspace sizing, the integer planning functions of the
// reference, and dispatch to the kernel launchers.  No device memory is allocated and no
// stream is synchronized.  One file-scope device array (`scratch`, below) serves the
// allocation-free forward ssm_fwd_noalloc.
#include <algorithm>
#include <math.h>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "../../include/ssm_scan.h"
#include "ssm_internal.hpp"

using namespace ssm;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = 0;
  return SSM_OK;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(SSM_EHIP, "%s: %s", what, hipGetErrorString(e));
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }
int state_size(int dtype) { return dtype == SSM_F64 ? 8 : 4; }

KView kv(const ssm_tensor &t) { return KView{t.data, t.stride[0], t.stride[1], t.stride[2]}; }
bool has(const ssm_tensor &t) { return t.data != nullptr; }

const char *method_name(int m) { return m == 0 ? "zoh" : m == 1 ? "euler" : m == 2 ? "bilinear" : "?"; }

int check_common(int64_t B, int64_t L, int64_t D, int64_t N, int method, int dtype) {
  if (method < 0 || method > 2)
    return fail(SSM_EINVAL, "unknown discretization %d (expected zoh=0, euler=1, bilinear=2)", method);
  if (dtype < 0 || dtype > 3) return fail(SSM_EINVAL, "unsupported dtype code %d", dtype);
  if (B < 1 || L < 1 || D < 1 || N < 1)
    return fail(SSM_EINVAL, "empty problem: batch=%lld seqlen=%lld dim=%lld dstate=%lld", (long long)B,
                (long long)L, (long long)D, (long long)N);
  if (N > 64) return fail(SSM_EINVAL, "dstate=%lld > 64 is not supported", (long long)N);
  if (B > 65535) return fail(SSM_EINVAL, "batch=%lld > 65535 is not supported", (long long)B);
  if (L > (1LL << 30) || D > (1LL << 30))
    return fail(SSM_EINVAL, "seqlen/dim must be < 2^30");
  return SSM_OK;
}

#define REQUIRE(t, name)                                                        \
  do {                                                                          \
    if (!has(t)) return fail(SSM_EINVAL, "required tensor '%s' is missing", name); \
  } while (0)

// True when every present (B,L,D) view has x's strides, Cm has Bm's, strides are non-negative
// and one batch row, with a chunk and a channel tile of over-reach, spans less than 2^31 bytes:
// the kernels then address tiles with 32-bit byte offsets (raw buffer reads).
bool same3(const ssm_tensor &a, const ssm_tensor &b) {
  return !has(a) || (a.stride[0] == b.stride[0] && a.stride[1] == b.stride[1] && a.stride[2] == b.stride[2]);
}
bool row_fits(const ssm_tensor &t, int64_t L, int64_t C, int esize) {
  const int64_t lim = (int64_t)1 << 31;
  const int64_t s1 = t.stride[1], s2 = t.stride[2];
  if (s1 < 0 || s2 < 0 || s1 >= lim || s2 >= lim) return false;
  return ((L - 1 + 2 * kCK) * s1 + (C - 1 + 64) * s2 + 1) * esize < lim;
}
// The gate z is read through its own lane offsets, so it only needs to fit (the in_proj split
// of models/mamba.py:100 has twice x's row stride).
bool uniform_layout(const ssm_tensor *bld[], int nbld, const ssm_tensor &Bm, const ssm_tensor &Cm, int64_t L,
                    int64_t D, int64_t N, int dtype, const ssm_tensor &z) {
  const int esize = dtype == SSM_F64 ? 8 : dtype == SSM_F32 ? 4 : 2;
  for (int i = 0; i < nbld; ++i)
    if (!same3(*bld[i], *bld[0])) return false;
  return same3(Cm, Bm) && row_fits(*bld[0], L, D, esize) && row_fits(Bm, L, N, esize) &&
         (!has(z) || row_fits(z, L, D, esize));
}

struct FwdLayout {
  int np, ck, nchunks;
  int64_t ckpt_bytes, ypre_bytes;
};

FwdLayout fwd_layout(int64_t B, int64_t L, int64_t D, int64_t N, int dtype, bool gate) {
  FwdLayout f;
  f.np = fused_np(N, dtype);
  f.ck = chunk_steps(dtype);
  f.nchunks = (int)cdiv(L, f.ck);
  f.ckpt_bytes = align256(B * f.nchunks * D * f.np * state_size(dtype));
  f.ypre_bytes = gate ? align256(B * L * D * state_size(dtype)) : 0;
  return f;
}

// The uniform-layout kernels also address the saved chunk states and pre-gate output through
// buffers over one batch row, with 32-bit byte offsets.
bool saved_rows_fit(const FwdLayout &f, int64_t L, int64_t D, int dtype) {
  const int64_t lim = (int64_t)1 << 31;
  return (int64_t)f.nchunks * D * f.np * state_size(dtype) < lim && L * D * state_size(dtype) < lim;
}

// Time segments.  A pass launches W = B x ceil(D / channels-per-wavefront) wavefronts per
// segment; each segment after the first also costs a summary pass over its chunks, so segments
// pay only while they supply wavefronts the GPU would otherwise lack.  The automatic count
// minimises a cost model of MI355X's 1,024 SIMDs: the busiest SIMD holds ceil(W x nseg / 1,024)
// wavefronts, `cap` at a time, and runs them in rounds, each round as long as one wavefront's walk
// over its segment at that round's occupancy.  The constants are fitted to kernel times of the
// float32 N = 16 kernels at D 512 over forced counts (B 1-16 at L 512, B1 at L 4,096-131,072,
// B2-8 at L 1,024-65,536; at each shape the model's pick is within 2 % of the fastest count
// measured): the backward's wavefronts walk nearly as fast two to a SIMD as alone
// (latency-bound), so a partly filled extra round costs a whole walk (B1 L65536: 16, 32 and 48
// segments 1.16-1.18 ms, 24 segments 1.52 ms); the forward keeps its SIMDs busy from 2
// wavefronts on, so it segments less at short lengths (B8 L512: one segment 39 us, 2 segments
// 45 us, 6 segments 53 us).  With fewer than 512 wavefronts per segment (one to three rows at
// D 512), walks over kSegLongChunks chunks end unevenly, which the rounds do not capture: there the
// plan takes the best count with segments of at most kSegLongChunks chunks when the model prices
// it within kSegLongSlack of the best (B1 D512 L131072 forward: 64 segments 0.857 ms, 24 segments
// 0.874 ms; L65536 with (B, L, D) inputs: 48-64 segments 0.60-0.62 ms, 24 segments 0.66 ms;
// backward 32 segments 1.168 ms, 16 segments 1.183 ms).  Segments are at least kSegMinChunks
// chunks long; a positive `requested` overrides the choice (clamped to the valid range).
constexpr int64_t kSimds = 1024, kSegMinChunks = 4, kSegLongChunks = 128, kSyncSegChunks = 64;
constexpr double kSegLongSlack = 1.1;

struct PassModel {
  int cap;             // wavefronts per SIMD that the kernel's registers and LDS allow
  double lat[3];       // a wavefront's time per chunk with 1..cap wavefronts on its SIMD
  double summary;      // the summary pass's time per chunk relative to the main pass's
  double per_wave;     // a wavefront's start and end, in chunks
  double fixed;        // a segmented pass's extra launches and carry, in chunks
  double per_segment;  // folding one more segment's summary, in chunks
};

constexpr PassModel kFwdModel{3, {1.0, 1.2, 1.63}, 0.5, 1.0, 8.0, 1.0};
constexpr PassModel kBwdModel{2, {1.0, 1.04, 0.0}, 0.37, 0.0, 4.0, 0.0};

double walk_cost(const PassModel &m, int64_t waves, int64_t chunks) {
  const int64_t w = cdiv(waves, kSimds), full = w / m.cap, rest = w % m.cap;
  return ((double)full * m.lat[m.cap - 1] + (rest ? m.lat[rest - 1] : 0.0)) * ((double)chunks + m.per_wave);
}

double plan_cost(const PassModel &m, int64_t waves, int64_t nchunks, int64_t n) {
  const int64_t sc = cdiv(nchunks, n), ns = cdiv(nchunks, sc);
  double c = walk_cost(m, waves * ns, sc);
  if (ns > 1) c += m.summary * walk_cost(m, waves * (ns - 1), sc) + m.fixed + m.per_segment * (double)ns;
  return c;
}

struct SegPlan {
  int nseg, seg_chunks;
};

SegPlan seg_plan(int64_t B, int64_t D, const FwdLayout &f, int requested, bool backward) {
  SegPlan s;
  const int64_t waves = B * cdiv(D, 64 / f.np);
  int64_t n = 1;
  if (requested > 0) {
    n = requested;
  } else {
    // the last automatic choice per thread, keyed by its inputs (every call plans twice or more)
    thread_local int64_t key[4] = {-1, -1, -1, -1}, memo = 1;
    const int64_t k[4] = {waves, f.nchunks, B, backward};
    if (std::equal(k, k + 4, key)) {
      n = memo;
    } else {
      const PassModel &m = backward ? kBwdModel : kFwdModel;
      // past 16 full rounds more segments only add summary work
      const int64_t nmax = std::min({(int64_t)f.nchunks / kSegMinChunks, 65535 / B, cdiv(16 * m.cap * kSimds, waves)});
      double best = plan_cost(m, waves, f.nchunks, 1), best_short = -1.0;
      int64_t n_short = 0;
      for (int64_t c = 1; c <= nmax; ++c) {
        const double v = c == 1 ? best : plan_cost(m, waves, f.nchunks, c);
        if (v < best) best = v, n = c;
        if (cdiv(f.nchunks, c) <= kSegLongChunks && (n_short == 0 || v < best_short)) best_short = v, n_short = c;
      }
      if (2 * waves < kSimds && n_short && best_short <= kSegLongSlack * best) n = n_short;
      std::copy(k, k + 4, key);
      memo = n;
    }
  }
  n = std::max((int64_t)1, std::min(n, std::min((int64_t)f.nchunks, 65535 / B)));
  s.seg_chunks = (int)cdiv(f.nchunks, n);
  s.nseg = (int)cdiv(f.nchunks, s.seg_chunks);
  return s;
}

struct BwdLayout {
  FwdLayout f;
  SegPlan sp;
  int ntiles;
  int64_t saved, dB, dC, dA, dD, db, mu, E, P, total;  // byte offsets
};

BwdLayout bwd_layout(const ssm_bwd_args *a) {
  BwdLayout w;
  w.f = fwd_layout(a->batch, a->seqlen, a->dim, a->dstate, a->dtype, has(a->z));
  // float64 runs the register-staged kernel, which has no time segments
  w.sp = a->dtype == SSM_F64 ? SegPlan{1, w.f.nchunks} : seg_plan(a->batch, a->dim, w.f, a->segments, true);
  const int ss = state_size(a->dtype);
  const int64_t rows = a->batch * w.sp.nseg;
  w.ntiles = (int)cdiv(a->dim, bwd_channels_per_block(a->dtype, w.f.np));
  int64_t off = 0;
  w.saved = off;
  if (!a->saved) off += w.f.ckpt_bytes + w.f.ypre_bytes;
  const int64_t part = align256(a->batch * w.ntiles * a->seqlen * w.f.np * ss);
  w.dB = off; off += part;
  w.dC = off; off += part;
  w.dA = off; off += align256(rows * a->dim * w.f.np * 8);  // float64 partials
  w.dD = off; off += align256(rows * a->dim * ss);
  w.db = off; off += align256(rows * a->dim * ss);
  const int64_t segs = w.sp.nseg > 1 ? rows * a->dim * w.f.np : 0;
  w.mu = off; off += align256(segs * 8);
  w.E = off; off += align256(segs * 8);
  w.P = off; off += align256(segs * 4);
  w.total = off;
  return w;
}

}  // namespace

extern "C" {

int ssm_abi_version(void) { return SSM_ABI_VERSION; }
const char *ssm_last_error(void) { return g_err; }

// ------------------------------------------------------------------ fused forward
// Low-rank delta: rank 1..kLR with a (D, R) weight, and the (B, L, R) input's row offsets in
// 32 bits (the kernels read it through raw buffers over one batch row).
static int check_lowrank(int64_t rank, const ssm_tensor &proj, const ssm_tensor &delta, int64_t L, int64_t N,
                         int dtype) {
  if (rank == 0) return ok();
  if (rank < 0 || rank > kLR)
    return fail(SSM_EINVAL, "delta_rank=%lld must be in 0..%d", (long long)rank, kLR);
  if (N > 16 || dtype == SSM_F64)
    return fail(SSM_EINVAL, "a low-rank delta needs dstate <= 16 and 16- or 32-bit inputs");
  REQUIRE(proj, "delta_proj");
  const int esize = dtype == SSM_F64 ? 8 : dtype == SSM_F32 ? 4 : 2;
  if (delta.stride[1] < 0 || delta.stride[2] < 0 || proj.stride[0] < 0 || proj.stride[1] < 0)
    return fail(SSM_EINVAL, "low-rank delta and delta_proj need non-negative strides");
  if (((L - 1 + kCK) * delta.stride[1] + (rank - 1) * delta.stride[2] + 1) * esize >= ((int64_t)1 << 31))
    return fail(SSM_EINVAL, "a batch row of the low-rank delta spans more than 2 GiB");
  return ok();
}

int ssm_fwd_check(const ssm_fwd_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  int rc = check_common(a->batch, a->seqlen, a->dim, a->dstate, a->method, a->dtype);
  if (rc) return rc;
  REQUIRE(a->x, "x");
  REQUIRE(a->delta, "delta");
  REQUIRE(a->A, "A");
  REQUIRE(a->Bm, "Bm");
  REQUIRE(a->Cm, "Cm");
  REQUIRE(a->out, "out");
  if (a->segments < 0) return fail(SSM_EINVAL, "segments=%d must be >= 0", a->segments);
  return check_lowrank(a->delta_rank, a->delta_proj, a->delta, a->seqlen, a->dstate, a->dtype);
}

int64_t ssm_fwd_saved_bytes(const ssm_fwd_args *a) {
  if (ssm_fwd_check(a)) return -1;
  FwdLayout f = fwd_layout(a->batch, a->seqlen, a->dim, a->dstate, a->dtype, has(a->z));
  return f.ckpt_bytes + f.ypre_bytes;
}

// One (B, nseg, D, NP) state-type buffer of the forward's segment summaries (0 without segments).
static int64_t seg_buf_bytes(const ssm_fwd_args *a, const FwdLayout &f, const SegPlan &sp) {
  return sp.nseg > 1 ? align256(a->batch * sp.nseg * a->dim * f.np * state_size(a->dtype)) : 0;
}

int64_t ssm_fwd_workspace_bytes(const ssm_fwd_args *a) {
  if (ssm_fwd_check(a)) return -1;
  FwdLayout f = fwd_layout(a->batch, a->seqlen, a->dim, a->dstate, a->dtype, has(a->z));
  return 3 * seg_buf_bytes(a, f, seg_plan(a->batch, a->dim, f, a->segments, false));
}

static void fill_fwd(FwdParams &p, const ssm_fwd_args *a, const FwdLayout &f) {
  memset(&p, 0, sizeof(p));
  p.B = a->batch; p.L = a->seqlen; p.D = a->dim; p.N = a->dstate;
  p.nchunks = f.nchunks;
  p.nseg = 1;
  p.seg_chunks = f.nchunks;
  p.softplus = a->delta_softplus != 0;
  p.has_D = has(a->Dskip); p.has_z = has(a->z); p.has_bias = has(a->delta_bias);
  p.has_h0 = has(a->h0); p.has_last = has(a->last); p.write_out = 1;
  p.x = kv(a->x); p.dt = kv(a->delta); p.A = kv(a->A); p.Bm = kv(a->Bm); p.Cm = kv(a->Cm);
  p.Dsk = kv(a->Dskip); p.z = kv(a->z); p.bias = kv(a->delta_bias); p.h0 = kv(a->h0);
  p.out = kv(a->out); p.last = kv(a->last);
  p.a_log = a->A_is_log != 0;
  if (a->delta_rank > 0) {  // the (B, L, D) delta view aliases x: its tiles are never used
    p.lowrank = (int)a->delta_rank;
    p.dtl = kv(a->delta); p.dtw = kv(a->delta_proj); p.dt = kv(a->x);
  }
  const ssm_tensor *bld[] = {&a->x, p.lowrank ? &a->x : &a->delta, &a->out};
  p.uniform = uniform_layout(bld, 3, a->Bm, a->Cm, a->seqlen, a->dim, a->dstate, a->dtype, a->z) &&
              saved_rows_fit(f, a->seqlen, a->dim, a->dtype);
}

int ssm_fwd(const ssm_fwd_args *a, void *stream) {
  int rc = ssm_fwd_check(a);
  if (rc) return rc;
  FwdLayout f = fwd_layout(a->batch, a->seqlen, a->dim, a->dstate, a->dtype, has(a->z));
  FwdParams p;
  fill_fwd(p, a, f);
  if (a->saved) {
    p.ckpt = a->saved;
    p.ypre = has(a->z) ? (char *)a->saved + f.ckpt_bytes : nullptr;
  }
  const SegPlan sp = seg_plan(a->batch, a->dim, f, a->segments, false);
  const int64_t bb = seg_buf_bytes(a, f, sp);
  if (sp.nseg > 1) {
    if (!a->workspace || a->workspace_bytes < 3 * bb)
      return fail(SSM_ESPACE, "workspace of %lld bytes is smaller than the %lld required",
                  (long long)a->workspace_bytes, (long long)(3 * bb));
    p.nseg = sp.nseg;
    p.seg_chunks = sp.seg_chunks;
    // (B, L, D) outputs over long segments: a workgroup barrier every 4 chunk pairs (B1 D512
    // L65536, 48 segments of 86 chunks: forward 618 -> 575 us; no gain at 43 chunks, and 1-2 %
    // slower with (B, D, L) outputs, whose 64-byte pieces each come from one wavefront)
    if (sp.seg_chunks >= kSyncSegChunks && a->out.stride[2] == 1) p.sync_pairs = 4;
    p.seg_P = a->workspace;
    p.seg_E = (char *)a->workspace + bb;
    p.seg_hin = (char *)a->workspace + 2 * bb;
  }
  hipError_t e = launch_fwd(p, a->dtype, a->method, f.np, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssm_fwd launch");
  return ok();
}

// ------------------------------------------------------------------ fused backward
int ssm_bwd_check(const ssm_bwd_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  int rc = check_common(a->batch, a->seqlen, a->dim, a->dstate, a->method, a->dtype);
  if (rc) return rc;
  REQUIRE(a->x, "x");
  REQUIRE(a->delta, "delta");
  REQUIRE(a->A, "A");
  REQUIRE(a->Bm, "Bm");
  REQUIRE(a->Cm, "Cm");
  REQUIRE(a->dout, "dout");
  REQUIRE(a->dx, "dx");
  REQUIRE(a->ddelta, "ddelta");
  REQUIRE(a->dA, "dA");
  REQUIRE(a->dBm, "dBm");
  REQUIRE(a->dCm, "dCm");
  if (has(a->Dskip)) REQUIRE(a->dD, "dD");
  if (has(a->z)) REQUIRE(a->dz, "dz");
  if (has(a->delta_bias)) REQUIRE(a->ddelta_bias, "ddelta_bias");
  if (has(a->dh0) && !has(a->h0)) return fail(SSM_EINVAL, "dh0 given without h0");
  if (a->segments < 0) return fail(SSM_EINVAL, "segments=%d must be >= 0", a->segments);
  return check_lowrank(a->delta_rank, a->delta_proj, a->delta, a->seqlen, a->dstate, a->dtype);
}

int64_t ssm_bwd_workspace_bytes(const ssm_bwd_args *a) {
  if (ssm_bwd_check(a)) return -1;
  return bwd_layout(a).total;
}

int ssm_bwd(const ssm_bwd_args *a, void *stream) {
  int rc = ssm_bwd_check(a);
  if (rc) return rc;
  BwdLayout w = bwd_layout(a);
  if (!a->workspace || a->workspace_bytes < w.total)
    return fail(SSM_ESPACE, "workspace of %lld bytes is smaller than the %lld required",
                (long long)a->workspace_bytes, (long long)w.total);
  hipStream_t s = (hipStream_t)stream;
  char *ws = (char *)a->workspace;
  const void *ckpt = a->saved;
  const void *ypre = a->saved && has(a->z) ? (const char *)a->saved + w.f.ckpt_bytes : nullptr;
  if (!a->saved) {  // recompute the chunk-boundary states (and the pre-gate output)
    ssm_fwd_args fa;
    memset(&fa, 0, sizeof(fa));
    fa.batch = a->batch; fa.seqlen = a->seqlen; fa.dim = a->dim; fa.dstate = a->dstate;
    fa.method = a->method; fa.dtype = a->dtype;
    fa.x = a->x; fa.delta = a->delta; fa.A = a->A; fa.Bm = a->Bm; fa.Cm = a->Cm;
    fa.Dskip = a->Dskip; fa.z = a->z; fa.delta_bias = a->delta_bias;
    fa.delta_softplus = a->delta_softplus; fa.h0 = a->h0;
    fa.delta_proj = a->delta_proj; fa.delta_rank = a->delta_rank;
    fa.A_is_log = a->A_is_log;
    fa.out = a->x;  // placeholder with x's layout, never written (write_out = 0)
    FwdParams fp;
    fill_fwd(fp, &fa, w.f);
    fp.write_out = 0;
    fp.has_last = 0;
    fp.ckpt = ws + w.saved;
    fp.ypre = has(a->z) ? ws + w.saved + w.f.ckpt_bytes : nullptr;
    hipError_t e = launch_fwd(fp, a->dtype, a->method, w.f.np, s);
    if (e != hipSuccess) return hip_fail(e, "ssm_bwd state recompute launch");
    ckpt = fp.ckpt;
    ypre = fp.ypre;
  }
  BwdParams p;
  memset(&p, 0, sizeof(p));
  p.B = a->batch; p.L = a->seqlen; p.D = a->dim; p.N = a->dstate;
  p.nchunks = w.f.nchunks; p.ntiles = w.ntiles;
  p.softplus = a->delta_softplus != 0;
  p.has_D = has(a->Dskip); p.has_z = has(a->z); p.has_bias = has(a->delta_bias);
  p.has_h0 = has(a->h0); p.has_dlast = has(a->dlast); p.has_dh0 = has(a->dh0);
  p.x = kv(a->x); p.dt = kv(a->delta); p.A = kv(a->A); p.Bm = kv(a->Bm); p.Cm = kv(a->Cm);
  p.Dsk = kv(a->Dskip); p.z = kv(a->z); p.bias = kv(a->delta_bias); p.h0 = kv(a->h0);
  p.dout = kv(a->dout); p.dlast = kv(a->dlast); p.dx = kv(a->dx); p.ddt = kv(a->ddelta);
  p.dz = kv(a->dz); p.dh0 = kv(a->dh0);
  p.ckpt = ckpt; p.ypre = ypre;
  p.a_log = a->A_is_log != 0;
  if (a->delta_rank > 0) {  // as in the forward: the (B, L, D) delta view aliases x
    p.lowrank = (int)a->delta_rank;
    p.dtl = kv(a->delta); p.dtw = kv(a->delta_proj); p.dt = kv(a->x);
  }
  // dz keeps its own strides (like z): it only needs 32-bit row offsets
  const ssm_tensor *bld[] = {&a->x, p.lowrank ? &a->x : &a->delta, &a->dout, &a->dx, &a->ddelta};
  p.uniform = uniform_layout(bld, 5, a->Bm, a->Cm, a->seqlen, a->dim, a->dstate, a->dtype, a->z) &&
              saved_rows_fit(w.f, a->seqlen, a->dim, a->dtype) &&
              a->seqlen * w.f.np * state_size(a->dtype) < ((int64_t)1 << 31) &&  // dB / dC partial rows
              (!has(a->dz) || row_fits(a->dz, a->seqlen, a->dim, a->dtype == SSM_F64 ? 8 : a->dtype == SSM_F32 ? 4 : 2));
  p.ws_dB = ws + w.dB; p.ws_dC = ws + w.dC; p.ws_dA = ws + w.dA; p.ws_dD = ws + w.dD; p.ws_db = ws + w.db;
  p.nseg = w.sp.nseg; p.seg_chunks = w.sp.seg_chunks;
  if (w.sp.nseg > 1) { p.seg_mu = ws + w.mu; p.seg_E = ws + w.E; p.seg_P = ws + w.P; }
  hipError_t e = launch_bwd(p, a->dtype, a->method, w.f.np, s);
  if (e != hipSuccess) return hip_fail(e, "ssm_bwd launch");
  FinParams fin;
  memset(&fin, 0, sizeof(fin));
  fin.B = a->batch; fin.L = a->seqlen; fin.D = a->dim; fin.N = a->dstate;
  fin.ntiles = w.ntiles; fin.np = w.f.np; fin.rows = a->batch * w.sp.nseg;
  fin.has_D = has(a->Dskip); fin.has_bias = has(a->delta_bias);
  fin.a_log = a->A_is_log != 0; fin.A = kv(a->A);
  fin.ws_dB = p.ws_dB; fin.ws_dC = p.ws_dC; fin.ws_dA = p.ws_dA; fin.ws_dD = p.ws_dD; fin.ws_db = p.ws_db;
  fin.dB = kv(a->dBm); fin.dC = kv(a->dCm); fin.dA = kv(a->dA); fin.dD = kv(a->dD); fin.dbias = kv(a->ddelta_bias);
  e = launch_bwd_finalize(fin, a->dtype, s);
  if (e != hipSuccess) return hip_fail(e, "ssm_bwd finalize launch");
  return ok();
}

// ------------------------------------------------------------------ decode step
int ssm_step_check(const ssm_step_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  int rc = check_common(a->batch, 1, a->dim, a->dstate, a->method, a->dtype);
  if (rc) return rc;
  REQUIRE(a->x, "x");
  REQUIRE(a->delta, "delta");
  REQUIRE(a->A, "A");
  REQUIRE(a->Bm, "Bm");
  REQUIRE(a->Cm, "Cm");
  REQUIRE(a->h, "h");
  REQUIRE(a->out, "out");
  return ok();
}

int ssm_step(const ssm_step_args *a, void *stream) {
  int rc = ssm_step_check(a);
  if (rc) return rc;
  StepParams p;
  memset(&p, 0, sizeof(p));
  p.B = a->batch; p.D = a->dim; p.N = a->dstate;
  p.softplus = a->delta_softplus != 0;
  p.has_D = has(a->Dskip); p.has_z = has(a->z); p.has_bias = has(a->delta_bias);
  p.x = kv(a->x); p.dt = kv(a->delta); p.A = kv(a->A); p.Bm = kv(a->Bm); p.Cm = kv(a->Cm);
  p.Dsk = kv(a->Dskip); p.z = kv(a->z); p.bias = kv(a->delta_bias); p.h = kv(a->h); p.out = kv(a->out);
  hipError_t e = launch_step(p, a->dtype, a->method, padded_n(a->dstate), (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssm_step launch");
  return ok();
}

// ------------------------------------------------------------------ plans
int64_t ssm_default_chunk(int64_t L) {
  // max(4, 2^ceil(log2(sqrt(L)))) == max(4, smallest 2^k with 4^k >= L), in exact integers
  if (L < 0) return -1;
  int k = 0;
  while (k < 31 && (int64_t)1 << (2 * k) < L) ++k;
  int64_t c = (int64_t)1 << k;
  return c < 4 ? 4 : c;
}

int64_t ssm_scan_blocks(int64_t B, int64_t L, int64_t D, int64_t N, int64_t d_block, int64_t *bounds,
                        int64_t capacity) {
  if (B < 1 || L < 1 || D < 1 || N < 1) return -1;
  if (d_block <= 0) {
    d_block = ((int64_t)1 << 24) / (B * L * N);
    if (d_block < 1) d_block = 1;
  }
  if (d_block > D) d_block = D;
  int64_t count = cdiv(D, d_block);
  if (bounds) {
    for (int64_t i = 0, j = 0; i < D && j < capacity; i += d_block, ++j) {
      bounds[2 * j] = i;
      bounds[2 * j + 1] = i + d_block < D ? i + d_block : D;
    }
  }
  return count;
}

int64_t ssm_block_d(int64_t B, int64_t D) {
  int64_t bd = 16;
  while (bd > 4 && B * cdiv(D, bd) < 128) bd /= 2;
  return bd;
}

int64_t ssm_bwd_tile(int64_t B, int64_t L, int64_t N, int64_t bd) {
  if (B < 1 || L < 1 || N < 1 || bd < 1) return -1;
  int64_t t = (((int64_t)1 << 27) / (B * L * N)) / bd * bd;
  return t > bd ? t : bd;
}

int32_t ssm_resolve_scan(int32_t scan_id, int32_t on_gpu, int32_t method, int64_t N, int32_t engine) {
  if (scan_id == SSM_SCAN_AUTO) {
    bool ok_ = engine && on_gpu && method >= 0 && method <= 2 && (N & (N - 1)) == 0;
    return ok_ ? SSM_SCAN_FUSED : SSM_SCAN_CHUNKED;
  }
  if (scan_id < 0 || scan_id > SSM_SCAN_FUSED) return -1;
  return scan_id;
}

// ------------------------------------------------------------------ linear scans
static int lscan_common(int64_t B, int64_t L, int64_t M, int algo, int dtype, int64_t chunk) {
  if (algo < SSM_SCAN_SEQUENTIAL || algo > SSM_SCAN_CHUNKED)
    return fail(SSM_EINVAL, "unknown scan algorithm %d (sequential=1 .. chunked=4)", algo);
  if (dtype != SSM_F32 && dtype != SSM_F64) return fail(SSM_EINVAL, "linear scans take float32 or float64");
  if (B < 1 || L < 1 || M < 1)
    return fail(SSM_EINVAL, "empty scan: batch=%lld seqlen=%lld width=%lld", (long long)B, (long long)L,
                (long long)M);
  if (B > 65535) return fail(SSM_EINVAL, "batch=%lld > 65535 is not supported", (long long)B);
  if (L >= (1LL << 30) || M >= (1LL << 31) || B * L * M >= (1LL << 39))
    return fail(SSM_EINVAL, "scan too large");
  if (chunk < 0 || chunk >= (1LL << 30)) return fail(SSM_EINVAL, "chunk=%lld out of range", (long long)chunk);
  // one lane per recurrence (per chunk of one for the chunked algorithm): a 1-D grid below 2^31 lanes
  const int64_t lanes = B * M * (algo == SSM_SCAN_CHUNKED ? cdiv(L, chunk ? chunk : ssm_default_chunk(L)) : 1);
  if (lanes >= (1LL << 31)) return fail(SSM_EINVAL, "scan too large: %lld recurrences", (long long)lanes);
  return SSM_OK;
}

static int64_t lscan_chunk(int64_t L, int64_t chunk) { return chunk ? chunk : ssm_default_chunk(L); }

static int64_t lscan_ws(int64_t B, int64_t L, int64_t M, int algo, int dtype, int64_t chunk) {
  if (algo != SSM_SCAN_CHUNKED) return 0;
  return align256(3 * B * cdiv(L, lscan_chunk(L, chunk)) * M * state_size(dtype));
}

static LscanParams lscan_params(int64_t B, int64_t L, int64_t M, int64_t chunk, int reverse, int shift) {
  LscanParams p;
  memset(&p, 0, sizeof(p));
  p.B = B;
  p.L = L;
  p.M = M;
  p.chunk = (int)lscan_chunk(L, chunk);
  p.nc = cdiv(L, p.chunk);
  p.reverse = reverse != 0;
  p.shift = shift;
  return p;
}

int ssm_lscan_check(const ssm_lscan_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  int rc = lscan_common(a->batch, a->seqlen, a->width, a->algo, a->dtype, a->chunk);
  if (rc) return rc;
  REQUIRE(a->a, "a");
  REQUIRE(a->b, "b");
  REQUIRE(a->h, "h");
  return ok();
}

int64_t ssm_lscan_workspace_bytes(const ssm_lscan_args *a) {
  if (ssm_lscan_check(a)) return -1;
  return lscan_ws(a->batch, a->seqlen, a->width, a->algo, a->dtype, a->chunk);
}

int ssm_lscan(const ssm_lscan_args *a, void *stream) {
  int rc = ssm_lscan_check(a);
  if (rc) return rc;
  const int64_t need = lscan_ws(a->batch, a->seqlen, a->width, a->algo, a->dtype, a->chunk);
  if (need && (!a->workspace || a->workspace_bytes < need))
    return fail(SSM_ESPACE, "workspace of %lld bytes required", (long long)need);
  LscanParams p = lscan_params(a->batch, a->seqlen, a->width, a->chunk, a->reverse, 0);
  p.a = kv(a->a);
  p.b = kv(a->b);
  p.h0 = kv(a->h0);
  p.h = kv(a->h);
  p.ws = a->workspace;
  hipError_t e = launch_lscan(p, a->algo, a->dtype, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_lscan");
}

int ssm_lscan_bwd_check(const ssm_lscan_bwd_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  int rc = lscan_common(a->batch, a->seqlen, a->width, a->algo, a->dtype, a->chunk);
  if (rc) return rc;
  REQUIRE(a->a, "a");
  REQUIRE(a->h, "h");
  REQUIRE(a->dh, "dh");
  REQUIRE(a->da, "da");
  REQUIRE(a->db, "db");
  if (has(a->dh0) && !has(a->h0)) return fail(SSM_EINVAL, "dh0 requested without h0");
  return ok();
}

int64_t ssm_lscan_bwd_workspace_bytes(const ssm_lscan_bwd_args *a) {
  if (ssm_lscan_bwd_check(a)) return -1;
  return lscan_ws(a->batch, a->seqlen, a->width, a->algo, a->dtype, a->chunk);
}

int ssm_lscan_bwd(const ssm_lscan_bwd_args *a, void *stream) {
  int rc = ssm_lscan_bwd_check(a);
  if (rc) return rc;
  const int64_t need = lscan_ws(a->batch, a->seqlen, a->width, a->algo, a->dtype, a->chunk);
  if (need && (!a->workspace || a->workspace_bytes < need))
    return fail(SSM_ESPACE, "workspace of %lld bytes required", (long long)need);
  // lambda = reverse-direction scan of dh with the shifted multipliers, written into db
  LscanParams p = lscan_params(a->batch, a->seqlen, a->width, a->chunk, !a->reverse, 1);
  p.a = kv(a->a);
  p.b = kv(a->dh);
  p.h = kv(a->db);
  p.ws = a->workspace;
  hipError_t e = launch_lscan(p, a->algo, a->dtype, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "ssm_lscan_bwd");
  LscanGradParams g;
  memset(&g, 0, sizeof(g));
  g.B = a->batch;
  g.L = a->seqlen;
  g.M = a->width;
  g.reverse = a->reverse != 0;
  g.a = kv(a->a);
  g.h0 = kv(a->h0);
  g.h = kv(a->h);
  g.db = kv(a->db);
  g.da = kv(a->da);
  g.dh0 = kv(a->dh0);
  e = launch_lscan_grad(g, a->dtype, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_lscan_bwd");
}

// ------------------------------------------------------------------ materialized discretization
static DiscParams disc_params(const ssm_disc_args *a) {
  DiscParams p;
  memset(&p, 0, sizeof(p));
  p.B = a->batch;
  p.L = a->seqlen;
  p.D = a->dim;
  p.N = a->dstate;
  const int64_t R = p.B * p.L;
  p.dtiles = cdiv(p.D, disc_channels(padded_n(p.N)));
  int64_t groups = cdiv(4096, p.dtiles);
  if (groups > R) groups = R;
  p.rows_per_group = cdiv(R, groups);
  p.ngroups = cdiv(R, p.rows_per_group);
  return p;
}

// The discretization kernels address a lane's channel (or state) within a row by a 31-bit
// element offset.
static int disc_lane_offsets(const ssm_tensor *t, int64_t extent) {
  if (t->stride[2] < 0 || t->stride[2] * (extent - 1) >= (1LL << 31))
    return fail(SSM_EINVAL, "inner stride %lld too large for extent %lld", (long long)t->stride[2],
                (long long)extent);
  return 0;
}

int ssm_disc_check(const ssm_disc_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  int rc = check_common(a->batch, a->seqlen, a->dim, a->dstate, a->method, a->dtype);
  if (rc) return rc;
  if (a->dtype != SSM_F32 && a->dtype != SSM_F64)
    return fail(SSM_EINVAL, "materialized discretization takes float32 or float64");
  if (a->batch * a->seqlen * a->dim * a->dstate >= (1LL << 39) || a->dim * a->dstate >= (1LL << 31))
    return fail(SSM_EINVAL, "problem too large");
  REQUIRE(a->delta, "delta");
  REQUIRE(a->x, "x");
  REQUIRE(a->A, "A");
  REQUIRE(a->Bm, "Bm");
  if ((rc = disc_lane_offsets(&a->delta, a->dim)) || (rc = disc_lane_offsets(&a->x, a->dim)) ||
      (rc = disc_lane_offsets(&a->Bm, a->dstate)))
    return rc;
  return ok();
}

int64_t ssm_disc_workspace_bytes(const ssm_disc_args *a) {
  if (ssm_disc_check(a)) return -1;
  DiscParams p = disc_params(a);
  const int ss = state_size(a->dtype);
  return align256(p.B * p.L * p.dtiles * p.N * ss) + align256(p.ngroups * p.D * p.N * ss);
}

int ssm_disc_fwd(const ssm_disc_args *a, void *stream) {
  int rc = ssm_disc_check(a);
  if (rc) return rc;
  if (!a->a || !a->b) return fail(SSM_EINVAL, "required outputs 'a' and 'b' are missing");
  DiscParams p = disc_params(a);
  p.delta = kv(a->delta);
  p.x = kv(a->x);
  p.A = kv(a->A);
  p.Bm = kv(a->Bm);
  p.a = a->a;
  p.b = a->b;
  hipError_t e = launch_disc_fwd(p, a->dtype, a->method, padded_n(a->dstate), (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_disc_fwd");
}

int ssm_disc_bwd(const ssm_disc_args *a, void *stream) {
  int rc = ssm_disc_check(a);
  if (rc) return rc;
  if (!a->da || !a->db) return fail(SSM_EINVAL, "required inputs 'da' and 'db' are missing");
  REQUIRE(a->ddelta, "ddelta");
  REQUIRE(a->dx, "dx");
  REQUIRE(a->dA, "dA");
  REQUIRE(a->dBm, "dBm");
  rc = disc_lane_offsets(&a->ddelta, a->dim);
  if (!rc) rc = disc_lane_offsets(&a->dx, a->dim);
  if (rc) return rc;
  DiscParams p = disc_params(a);
  const int ss = state_size(a->dtype);
  const int64_t wsB = align256(p.B * p.L * p.dtiles * p.N * ss);
  const int64_t need = wsB + align256(p.ngroups * p.D * p.N * ss);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(SSM_ESPACE, "workspace of %lld bytes required", (long long)need);
  p.delta = kv(a->delta);
  p.x = kv(a->x);
  p.A = kv(a->A);
  p.Bm = kv(a->Bm);
  p.da = a->da;
  p.db = a->db;
  p.ddelta = kv(a->ddelta);
  p.dx = kv(a->dx);
  p.dA = kv(a->dA);
  p.dBm = kv(a->dBm);
  p.ws_dB = a->workspace;
  p.ws_dA = (char *)a->workspace + wsB;
  hipError_t e = launch_disc_bwd(p, a->dtype, a->method, padded_n(a->dstate), (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_disc_bwd");
}

// ------------------------------------------------------------------ fused decode layer
int ssm_decode_check(const ssm_decode_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  if (a->method < 0 || a->method > 2)
    return fail(SSM_EINVAL, "unknown discretization %d (expected zoh=0, euler=1, bilinear=2)", a->method);
  if (a->batch < 1 || a->dim < 1 || a->dstate < 1 || a->d_model < 1 || a->dt_rank < 1)
    return fail(SSM_EINVAL, "empty decode layer");
  if (a->batch > 65535 * 32767LL) return fail(SSM_EINVAL, "batch too large");
  if (a->width < 1 || a->width > 8) return fail(SSM_EINVAL, "conv width %lld not in 1..8", (long long)a->width);
  if (a->dstate > 64 || a->dt_rank > 256 || a->dim > 8192)
    return fail(SSM_EINVAL, "decode layer dims out of range (dim <= 8192, dstate <= 64, dt_rank <= 256)");
  if (!a->u || !a->xz || !a->conv_w || !a->conv_b || (!a->conv_state && a->width > 1) || !a->x_proj_wt || !a->dt_proj_w ||
      !a->dt_bias || !a->A_log || !a->Dskip || !a->ssm_state || !a->y)
    return fail(SSM_EINVAL, "a required decode tensor is missing");
  if (a->conv_state_dtype != SSM_F32 && a->conv_state_dtype != SSM_BF16)
    return fail(SSM_EINVAL, "conv_state_dtype %d: the conv state is float32 or bf16", a->conv_state_dtype);
  return ok();
}

int ssm_decode_step(const ssm_decode_args *a, void *stream) {
  int rc = ssm_decode_check(a);
  if (rc) return rc;
  DecodeParams p;
  memset(&p, 0, sizeof(p));
  p.B = a->batch; p.dim = a->dim; p.N = a->dstate; p.W = a->width; p.R = a->dt_rank; p.dm = a->d_model;
  p.P = a->dt_rank + 2 * a->dstate;
  p.eps = a->eps;
  p.u = a->u; p.xz = a->xz; p.conv_w = a->conv_w; p.conv_b = a->conv_b; p.x_proj_wt = a->x_proj_wt;
  p.dt_proj_w = a->dt_proj_w; p.dt_bias = a->dt_bias; p.A_log = a->A_log; p.Dskip = a->Dskip;
  p.conv_state = a->conv_state; p.conv_bf16 = a->conv_state_dtype == SSM_BF16;
  p.ssm_state = a->ssm_state; p.y = a->y;
  if (decode_shared_bytes(p) > 64 * 1024) return fail(SSM_EINVAL, "decode layer too wide for one workgroup");
  hipError_t e = launch_decode(p, a->method, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_decode_step");
}

// ------------------------------------------------------------------ decode step of a block stack
namespace {
struct StackLayout {
  int64_t nct, ndu, P;
  int64_t off_ua, off_ub, off_du, off_xc, off_gate, off_part, off_status, total;
};
StackLayout stack_layout(const ssm_decode_stack_args *a) {
  StackLayout l;
  const int64_t B = a->batch, dm = a->d_model, Dm = a->dim;
  l.nct = cdiv(Dm, kInCh);
  l.ndu = cdiv(Dm, kScCh);
  l.P = a->dt_rank + 2 * a->dstate;
  int64_t o = 0;
  l.off_ua = o; o += align256(B * dm * 4);
  l.off_ub = o; o += align256(B * dm * 4);
  l.off_du = o; o += align256(B * l.ndu * dm * 4);
  l.off_xc = o; o += align256(B * Dm * 4);
  l.off_gate = o; o += align256(B * Dm * 4);
  l.off_part = o; o += align256(B * l.nct * l.P * 4);
  l.off_status = o; o += 256;
  l.total = o;
  return l;
}
}  // namespace

int ssm_decode_stack_check(const ssm_decode_stack_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  if (a->method < 0 || a->method > 2)
    return fail(SSM_EINVAL, "unknown discretization %d (expected zoh=0, euler=1, bilinear=2)", a->method);
  if (a->batch < 1 || a->dim < 1 || a->dstate < 1 || a->d_model < 1 || a->dt_rank < 1 || a->width < 1)
    return fail(SSM_EINVAL, "empty decode stack dimensions");
  if (a->n_blocks < 1 || !a->blocks) return fail(SSM_EINVAL, "no blocks");
  if (!a->u) return fail(SSM_EINVAL, "u (the residual stream) is missing");
  if (a->conv_state_dtype != SSM_F32 && a->conv_state_dtype != SSM_BF16)
    return fail(SSM_EINVAL, "conv_state_dtype %d: the conv state is float32 or bf16", a->conv_state_dtype);
  if (a->d_model > kStMaxDm) return fail(SSM_EINVAL, "d_model %lld > %d", (long long)a->d_model, kStMaxDm);
  if (a->dim > kStMaxDim) return fail(SSM_EINVAL, "dim %lld > %d", (long long)a->dim, kStMaxDim);
  if (a->dstate != 8 && a->dstate != 16) return fail(SSM_EINVAL, "dstate %lld not 8 or 16", (long long)a->dstate);
  if (a->dt_rank != 8 && a->dt_rank != 16 && a->dt_rank != 32)
    return fail(SSM_EINVAL, "dt_rank %lld not 8, 16 or 32", (long long)a->dt_rank);
  if (a->width > 4) return fail(SSM_EINVAL, "conv width %lld > 4", (long long)a->width);
  if (a->d_model % 4 || a->dim % 4)
    return fail(SSM_EINVAL, "d_model %lld and dim %lld must be multiples of 4", (long long)a->d_model, (long long)a->dim);
  // every buffer element is addressed by a 32-bit byte offset (with a few rows of slack)
  const StackLayout l = stack_layout(a);
  const int64_t rows = a->batch + kInRows;
  const int64_t widest = std::max({a->dim * a->dstate, l.ndu * a->d_model, l.nct * l.P, a->dim * a->width, a->d_model});
  if (rows * widest * 4 >= (1LL << 31) || a->d_model * 2 * a->dim * 4 >= (1LL << 31))
    return fail(SSM_EINVAL, "decode stack too large for 32-bit offsets (batch %lld)", (long long)a->batch);
  for (int i = 0; i < a->n_blocks; ++i) {
    const ssm_decode_block &k = a->blocks[i];
    if (!k.w_in4 || !k.conv_w || !k.conv_b || !k.x_proj_wt || !k.dt_proj_w || !k.dt_bias || !k.A_log ||
        !k.Dskip || !k.w_out4 || (!k.conv_state && a->width > 1) || !k.ssm_state)
      return fail(SSM_EINVAL, "block %d: a required tensor is missing", i);
    if (((uintptr_t)k.ssm_state | (uintptr_t)k.A_log | (uintptr_t)k.dt_proj_w | (uintptr_t)k.w_in4 |
         (uintptr_t)k.w_out4) % 16)
      return fail(SSM_EINVAL, "block %d: ssm_state, A_log, dt_proj_w, w_in4 and w_out4 must be 16-byte aligned", i);
  }
  if (((uintptr_t)a->u | (uintptr_t)a->embed | (uintptr_t)a->head_w4) % 16)
    return fail(SSM_EINVAL, "u, embed and head_w4 must be 16-byte aligned");
  if (a->tokens || a->head_w4) {
    if (a->vocab < 1) return fail(SSM_EINVAL, "vocab %lld: the embedding or head needs a vocabulary", (long long)a->vocab);
    if ((a->batch + kInRows) * a->vocab * 4 >= (1LL << 31) || a->vocab * a->d_model * 4 >= (1LL << 31))
      return fail(SSM_EINVAL, "vocabulary too large for 32-bit offsets (vocab %lld)", (long long)a->vocab);
  }
  if (a->tokens && !a->embed) return fail(SSM_EINVAL, "tokens given without the embedding table");
  if (a->head_w4 && !a->logits) return fail(SSM_EINVAL, "head weight given without a logits buffer");
  if (!a->workspace || a->workspace_bytes < l.total)
    return fail(SSM_ESPACE, "decode stack workspace %lld bytes < %lld", (long long)a->workspace_bytes,
                (long long)l.total);
  return ok();
}

int64_t ssm_decode_stack_workspace_bytes(const ssm_decode_stack_args *a) {
  if (!a || a->batch < 1 || a->dim < 1 || a->d_model < 1) return -1;
  return stack_layout(a).total;
}

int64_t ssm_decode_stack_status_offset(const ssm_decode_stack_args *a) {
  if (!a || a->batch < 1 || a->dim < 1 || a->d_model < 1) return -1;
  return stack_layout(a).off_status;
}

int ssm_decode_stack(const ssm_decode_stack_args *a, void *stream) {
  int rc = ssm_decode_stack_check(a);
  if (rc) return rc;
  const StackLayout l = stack_layout(a);
  const hipStream_t s = (hipStream_t)stream;
  char *ws = (char *)a->workspace;
  float *ua = (float *)(ws + l.off_ua), *ub = (float *)(ws + l.off_ub), *du = (float *)(ws + l.off_du);
  float *xc = (float *)(ws + l.off_xc), *gate = (float *)(ws + l.off_gate), *part = (float *)(ws + l.off_part);
  const int B = (int)a->batch, dm = (int)a->d_model, Dm = (int)a->dim;
  // k_dec_in of block i rebuilds the residual stream entering it (block 0: u or the embedding
  // rows; block i > 0: dst(i - 1) + block i - 1's partial sums) and stores it in dst(i), a
  // workspace buffer: no launch reads rows that another of its workgroups writes
  auto dst = [&](int i) { return i % 2 ? ub : ua; };
  for (int i = 0; i < a->n_blocks; ++i) {
    const ssm_decode_block &k = a->blocks[i];
    DecInParams pi;
    memset(&pi, 0, sizeof(pi));
    pi.B = B; pi.dm = dm; pi.Dm = Dm; pi.P = (int)l.P;
    pi.nrt = (int)cdiv(B, kInRows); pi.nct = (int)l.nct;
    pi.ndu = i == 0 ? 0 : (int)l.ndu;
    pi.write_u = 1;
    pi.conv_bf16 = a->conv_state_dtype == SSM_BF16;
    pi.eps = k.eps;
    pi.V = (int)a->vocab;
    pi.tokens = i == 0 ? a->tokens : nullptr;
    pi.embed = a->embed;
    pi.u_src = i == 0 ? a->u : dst(i - 1);
    pi.du = i == 0 ? nullptr : du;
    pi.u_dst = dst(i);
    pi.w_in4 = k.w_in4; pi.conv_w = k.conv_w; pi.conv_b = k.conv_b; pi.x_proj_wt = k.x_proj_wt;
    pi.conv_state = k.conv_state;
    pi.xc = xc; pi.gate = gate; pi.part = part;
    pi.bad_token = (int *)(ws + l.off_status);
    hipError_t e = launch_dec_in(pi, (int)a->width, s);
    if (e != hipSuccess) return hip_fail(e, "ssm_decode_stack in-stage launch");
    DecScanParams ps;
    memset(&ps, 0, sizeof(ps));
    ps.B = B; ps.dm = dm; ps.Dm = Dm; ps.N = (int)a->dstate; ps.R = (int)a->dt_rank; ps.P = (int)l.P;
    ps.nrt = (int)cdiv(B, kScRows); ps.nct = (int)l.nct; ps.ndu = (int)l.ndu;
    ps.xc = xc; ps.gate = gate; ps.part = part;
    ps.dt_proj_w = k.dt_proj_w; ps.dt_bias = k.dt_bias; ps.A_log = k.A_log; ps.Dskip = k.Dskip;
    ps.w_out4 = k.w_out4; ps.ssm_state = k.ssm_state; ps.du = du;
    e = launch_dec_scan(ps, a->method, s);
    if (e != hipSuccess) return hip_fail(e, "ssm_decode_stack scan-stage launch");
  }
  hipError_t e;
  if (a->head_w4) {  // the last block's sums, the final norm and the head in one launch
    DecInParams ph;
    memset(&ph, 0, sizeof(ph));
    ph.B = B; ph.dm = dm; ph.Dm = 1; ph.P = 1; ph.V = (int)a->vocab;
    ph.nrt = (int)cdiv(B, kInRows); ph.nct = (int)cdiv(a->vocab, 64); ph.ndu = (int)l.ndu;
    ph.write_u = 1; ph.eps = a->head_eps;
    ph.u_src = dst(a->n_blocks - 1); ph.du = du; ph.u_dst = a->u;
    ph.head_w4 = a->head_w4; ph.logits = a->logits;
    e = launch_dec_head(ph, s);
  } else {
    DecOutParams po;
    po.B = B; po.dm = dm; po.ndu = (int)l.ndu;
    po.u_src = dst(a->n_blocks - 1); po.du = du; po.u_out = a->u;
    e = launch_dec_out(po, s);
  }
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_decode_stack output launch");
}

// ------------------------------------------------------------------ causal depthwise conv
static constexpr int kConvTB = kConvTT * kConvTG;  // time steps per workgroup

static ConvParams conv_params(const ssm_conv_args *a) {
  ConvParams p;
  memset(&p, 0, sizeof(p));
  p.B = a->batch; p.L = a->seqlen; p.D = a->dim; p.W = a->width;
  p.TB = kConvTT;
  p.nblk = (int)cdiv(a->seqlen, kConvTB);
  p.silu = a->silu != 0;
  p.has_bias = has(a->bias); p.has_sin = has(a->state_in); p.has_sout = has(a->state_out);
  p.has_dbias = has(a->dbias);
  p.x = kv(a->x); p.w = kv(a->weight); p.bias = kv(a->bias); p.sin = kv(a->state_in);
  p.out = kv(a->out); p.sout = kv(a->state_out); p.dout = kv(a->dout); p.dx = kv(a->dx);
  p.dw = kv(a->dweight); p.dbias = kv(a->dbias);
  return p;
}

int ssm_conv_check(const ssm_conv_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  if (a->dtype < 0 || a->dtype > 3) return fail(SSM_EINVAL, "unsupported dtype code %d", a->dtype);
  if (a->batch < 1 || a->seqlen < 1 || a->dim < 1)
    return fail(SSM_EINVAL, "empty conv: batch=%lld seqlen=%lld dim=%lld", (long long)a->batch,
                (long long)a->seqlen, (long long)a->dim);
  if (a->width < 1 || a->width > 8) return fail(SSM_EINVAL, "conv width %lld not in 1..8", (long long)a->width);
  if (cdiv(a->seqlen, kConvTB) > 65535 || a->batch > 65535 || cdiv(a->dim, kConvDG) > (1LL << 31) - 1)
    return fail(SSM_EINVAL, "conv too large (seqlen <= %d, batch <= 65535)", 65535 * kConvTB);
  REQUIRE(a->x, "x");
  REQUIRE(a->weight, "weight");
  return ok();
}

int64_t ssm_conv_workspace_bytes(const ssm_conv_args *a) {
  if (ssm_conv_check(a)) return -1;
  return align256(a->batch * cdiv(a->seqlen, kConvTB) * a->dim * (a->width + 1) * state_size(a->dtype));
}

int ssm_conv_fwd(const ssm_conv_args *a, void *stream) {
  int rc = ssm_conv_check(a);
  if (rc) return rc;
  REQUIRE(a->out, "out");
  hipError_t e = launch_conv(conv_params(a), a->dtype, false, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_conv_fwd");
}

int ssm_conv_bwd(const ssm_conv_args *a, void *stream) {
  int rc = ssm_conv_check(a);
  if (rc) return rc;
  REQUIRE(a->dout, "dout");
  REQUIRE(a->dx, "dx");
  REQUIRE(a->dweight, "dweight");
  if (has(a->bias)) REQUIRE(a->dbias, "dbias");
  const int64_t need = ssm_conv_workspace_bytes(a);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(SSM_ESPACE, "workspace of %lld bytes required", (long long)need);
  ConvParams p = conv_params(a);
  p.ws = a->workspace;
  hipError_t e = launch_conv(p, a->dtype, true, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_conv_bwd");
}

// ------------------------------------------------------------------ RMSNorm
static NormParams norm_params(const ssm_norm_args *a) {
  NormParams p;
  memset(&p, 0, sizeof(p));
  p.R = a->rows;
  p.C = a->dim;
  p.eps = a->eps;
  p.x = a->x.data; p.sx = a->x.stride[0];
  p.w = a->weight.data;
  p.y = a->out.data; p.sy = a->out.stride[0];
  p.rstd = a->rstd;
  p.dy = a->dout.data; p.sdy = a->dout.stride[0];
  p.dx = a->dx.data; p.sdx = a->dx.stride[0];
  p.dw = a->dweight;
  p.rpw = norm_rows_per_wave(norm_kc_of(a->dim));
  p.nblk = cdiv(a->rows, (int64_t)kNormWaves * p.rpw);
  return p;
}

static int norm_row_view(const ssm_tensor &t, const char *name) {
  if (!has(t)) return fail(SSM_EINVAL, "required tensor '%s' is missing", name);
  if (t.stride[1] != 1) return fail(SSM_EINVAL, "%s must have unit column stride", name);
  return SSM_OK;
}

int ssm_norm_check(const ssm_norm_args *a) {
  if (!a) return fail(SSM_EINVAL, "null args");
  if (a->dtype != SSM_F32 && a->dtype != SSM_F64) return fail(SSM_EINVAL, "RMSNorm takes float32 or float64");
  if (a->rows < 1 || a->dim < 1) return fail(SSM_EINVAL, "empty RMSNorm: rows=%lld dim=%lld",
                                             (long long)a->rows, (long long)a->dim);
  if (a->dim > kNormMaxC) return fail(SSM_EINVAL, "RMSNorm dim=%lld > %d", (long long)a->dim, kNormMaxC);
  if (a->rows >= (1LL << 31)) return fail(SSM_EINVAL, "RMSNorm rows=%lld too large", (long long)a->rows);
  if (!(a->eps >= 0.0)) return fail(SSM_EINVAL, "RMSNorm eps must be >= 0");
  int rc = norm_row_view(a->x, "x");
  if (rc) return rc;
  if (!has(a->weight) || (a->dim > 1 && a->weight.stride[0] != 1))
    return fail(SSM_EINVAL, "weight must be a contiguous (dim,) tensor");
  if (!a->rstd) return fail(SSM_EINVAL, "required buffer 'rstd' is missing");
  return ok();
}

int64_t ssm_norm_workspace_bytes(const ssm_norm_args *a) {
  if (ssm_norm_check(a)) return -1;
  const NormParams p = norm_params(a);
  return align256(p.nblk * a->dim * state_size(a->dtype));
}

int ssm_norm_fwd(const ssm_norm_args *a, void *stream) {
  int rc = ssm_norm_check(a);
  if (!rc) rc = norm_row_view(a->out, "out");
  if (rc) return rc;
  hipError_t e = launch_norm(norm_params(a), a->dtype, false, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_norm_fwd");
}

int ssm_norm_bwd(const ssm_norm_args *a, void *stream) {
  int rc = ssm_norm_check(a);
  if (!rc) rc = norm_row_view(a->dout, "dout");
  if (!rc) rc = norm_row_view(a->dx, "dx");
  if (rc) return rc;
  if (!a->dweight) return fail(SSM_EINVAL, "required buffer 'dweight' is missing");
  const int64_t need = ssm_norm_workspace_bytes(a);
  if (!a->workspace || a->workspace_bytes < need)
    return fail(SSM_ESPACE, "workspace of %lld bytes required", (long long)need);
  NormParams p = norm_params(a);
  p.ws = a->workspace;
  hipError_t e = launch_norm(p, a->dtype, true, (hipStream_t)stream);
  return e == hipSuccess ? ok() : hip_fail(e, "ssm_norm_bwd");
}

// ------------------------------------------------------------------ forward without allocation
// ssm_fwd with the long-sequence workspace taken from a fixed device array instead of the
// caller's buffer, for callers that cannot allocate.  Every GPU the library runs on holds its
// own copy of the array until the process ends; host code reaches it only through the address
// hipGetSymbolAddress returns for the current device (the array's name is a host-side stand-in).
// Calls on one GPU share it, so calls that overlap on one GPU race.

}  // extern "C"

static __device__ __align__(256) unsigned char scratch[SSM_FWD_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the device that runs `stream` (which must be the
// current device), looked up once per device.
int scratch_address(void *stream, void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "ssm_fwd_noalloc: hipGetDevice");
  if (stream) {
    hipDevice_t sdev = 0;
    e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess) return hip_fail(e, "ssm_fwd_noalloc: hipStreamGetDevice");
    if ((int)sdev != dev)
      return fail(SSM_EINVAL, "ssm_fwd_noalloc: the stream belongs to device %d but device %d is current",
                  (int)sdev, dev);
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(SSM_EINVAL, "ssm_fwd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "ssm_fwd_noalloc: hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(SSM_EHIP, "ssm_fwd_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SSM_OK;
}

}  // namespace

extern "C" {

int ssm_fwd_noalloc(const ssm_fwd_args *a, void *stream) {
  int rc = ssm_fwd_check(a);
  if (rc) return rc;
  ssm_fwd_args b = *a;
  int64_t need = ssm_fwd_workspace_bytes(a);
  if (need > (int64_t)SSM_FWD_NOALLOC_SCRATCH_BYTES && a->segments <= 0) {
    // the automatic count lowered to the most segments whose three summary buffers fit the
    // array (each buffer is B x nseg x D x NP states, rounded up to 256 bytes)
    const FwdLayout f = fwd_layout(a->batch, a->seqlen, a->dim, a->dstate, a->dtype, has(a->z));
    const int64_t per = a->batch * a->dim * f.np * state_size(a->dtype);
    b.segments = (int32_t)std::max((int64_t)1, ((int64_t)SSM_FWD_NOALLOC_SCRATCH_BYTES / 3 - 255) / per);
    need = ssm_fwd_workspace_bytes(&b);
  }
  if (need > (int64_t)SSM_FWD_NOALLOC_SCRATCH_BYTES)
    return fail(SSM_ESPACE,
                "ssm_fwd_noalloc: this forward needs %lld bytes of workspace, more than the fixed scratch of "
                "%lld bytes; request fewer segments or call ssm_fwd with a workspace",
                (long long)need, (long long)SSM_FWD_NOALLOC_SCRATCH_BYTES);
  void *ptr = nullptr;
  rc = scratch_address(stream, &ptr);
  if (rc) return rc;
  b.workspace = ptr;
  b.workspace_bytes = SSM_FWD_NOALLOC_SCRATCH_BYTES;
  return ssm_fwd(&b, stream);
}

}  // extern "C"
