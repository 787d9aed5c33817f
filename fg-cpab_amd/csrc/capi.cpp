// extern "C" boundary of libcpab_hip.so (declared in include/cpab_hip.h).
//
// Responsibilities: validate every argument before touching HIP (the
// reference's TORCH_CHECK / AT_ASSERTM set, transformer_cuda.cpp:25-52 and
// transformer_cuda.cu:38-48,183-197, plus the size limits of this
// implementation), pick the launch shape for the device, enqueue, and turn any
// HIP failure into an error code + thread-local message instead of exit().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/cpab_hip.h"
#include "cpab_device.hpp"
#include "cpab_launch.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return CPAB_OK;
  return fail(CPAB_ERR_DEVICE, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

struct DeviceInfo {
  int cus = 0;
  int lds = 0;
};

DeviceInfo device_info() {
  static std::mutex mu;
  static DeviceInfo cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  std::lock_guard<std::mutex> lock(mu);
  DeviceInfo& d = cache[dev];
  if (d.cus == 0) {
    int v = 0;
    d.cus = (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) ? v : 256;
    // LDS a single workgroup may allocate (dynamic shared memory budget).
    v = 0;
    d.lds = (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0)
                ? v
                : 64 * 1024;
  }
  return d;
}

int64_t div_up(int64_t a, int64_t b) { return (a + b - 1) / b; }

int check_geometry(int ndim, int ncx, int ncy, int ncz, cpab::Geometry* g) {
  if (ndim < 1 || ndim > 3) return fail(CPAB_ERR_INVALID, "ndim must be 1, 2 or 3, got %d", ndim);
  if (ncx < 1 || (ndim >= 2 && ncy < 1) || (ndim == 3 && ncz < 1))
    return fail(CPAB_ERR_INVALID, "invalid tessellation %d x %d x %d", ncx, ncy, ncz);
  g->ndim = ndim;
  g->nx = ncx;
  g->ny = ndim >= 2 ? ncy : 1;
  g->nz = ndim == 3 ? ncz : 1;
  const int64_t nC = ndim == 1 ? (int64_t)ncx
                     : ndim == 2 ? 4LL * ncx * ncy
                                 : 5LL * ncx * ncy * ncz;
  // Cell ids are formed with 24-bit arithmetic, and a row's per-cell tables
  // (the affine maps, ppc floats per cell, and the reverse-sweep table,
  // 2 * ppc) are addressed with 32-bit byte offsets.
  if (nC >= (1LL << 24) || 2 * nC * g->ppc() >= (1LL << 30))
    return fail(CPAB_ERR_INVALID, "tessellation too large (nC=%lld, at most 2^24 - 1 cells)", (long long)nC);
  g->nC = (int)nC;
  return CPAB_OK;
}

int check_steps(int T) {
  if (T <= 0) return fail(CPAB_ERR_INVALID, "Invalid nstepsolver=%d. Expected nstepsolver > 0.", T);
  if (T > cpab::kMaxSteps)
    return fail(CPAB_ERR_INVALID,
                "Invalid nstepsolver=%d. The backward supports at most CPAB_MAX_STEPS=%d; "
                "reduce params.nstepsolver.",
                T, cpab::kMaxSteps);
  return CPAB_OK;
}

// Points (and image output positions) per row.  The kernels index a row's
// points with 32-bit ints and walk them as p0 + k * stride with k <= 2 and a
// grid stride of at most CUs * 4096 lanes, so nP + 2 * stride must stay below
// 2^31; below 2^31 / 3 it does with more than 2^30 to spare.
constexpr int64_t kMaxPoints = (1LL << 31) / 3;

int check_points(int64_t nP, int64_t n_theta, int ndim) {
  if (nP < 0 || n_theta < 0) return fail(CPAB_ERR_INVALID, "negative size (nP=%lld, n_theta=%lld)", (long long)nP, (long long)n_theta);
  if (nP >= kMaxPoints) return fail(CPAB_ERR_INVALID, "nP=%lld exceeds the 32-bit point index", (long long)nP);
  if (n_theta >= 65536) return fail(CPAB_ERR_INVALID, "n_theta=%lld exceeds the grid limit 65535", (long long)n_theta);
  (void)ndim;
  return CPAB_OK;
}

#define CPAB_REQUIRE(ptr) \
  do { if (!(ptr)) return fail(CPAB_ERR_INVALID, "%s must not be NULL", #ptr); } while (0)

// Per-cell tables are read as 8- and 16-byte vectors; every float array must
// be at least float-aligned.
#define CPAB_ALIGNED(ptr, bytes)                                                      \
  do {                                                                                \
    if ((ptr) && (reinterpret_cast<uintptr_t>(ptr) % (bytes)) != 0)                  \
      return fail(CPAB_ERR_INVALID, "%s must be %d-byte aligned", #ptr, (int)(bytes)); \
  } while (0)

// ---- launch-shape policy ---------------------------------------------------
// Fixed per problem shape and device (CU count, LDS per workgroup); each
// choice below was measured on MI355X (sweeps over block size, workgroups per
// CU and LDS staging).

cpab::LaunchCfg forward_cfg(const cpab::Geometry& g, int64_t nP, int64_t n_theta) {
  const DeviceInfo dev = device_info();
  (void)g;
  cpab::LaunchCfg c{};
  // The kernels keep the current cell's map in registers and re-read the table
  // only when a lane changes cell, through L1/L2.
  c.block = 512;
  // Two rounds of resident workgroups (2048 lanes per CU) per CU.
  const int64_t want = (int64_t)dev.cus * (2048 / c.block) * 2;
  int64_t chunks = std::max<int64_t>(1, div_up(want, std::max<int64_t>(n_theta, 1)));
  chunks = std::min(chunks, std::max<int64_t>(1, div_up(nP, c.block)));
  c.chunks = (int)chunks;
  return c;
}

// Floats per cell of the reverse-sweep table (cpab_device.hpp RevStride).
int adj_stride(int ndim) { return ndim == 1 ? 4 : (ndim == 2 ? 12 : 24); }

// Backward: full LDS bins when a theta's nC x ppc table fits in LDS, else the
// hashed LDS cell cache (at most 104 KiB, 3D).  Register variant for T = 50
// (cells, and with adaptive substeps positions, in VGPRs; one 1024-lane
// workgroup per CU, 768 with adaptive substeps); otherwise the segmented
// variant, with the affine table in LDS beside the bins when both fit.
// Returns false (message set) if the device's LDS holds neither.
bool backward_cfg(const cpab::Geometry& g, int64_t nP, int64_t n_theta, int T, int adaptive,
                  cpab::LaunchCfg* out) {
  const DeviceInfo dev = device_info();
  const int64_t table = (int64_t)g.nC * g.ppc() * 4;
  const int64_t cache = (int64_t)cpab::kCacheSlots * (g.ppc() + 1) * 4;
  cpab::LaunchCfg c{};
  c.lds_bins = table <= dev.lds ? 1 : 0;
  c.lds_cache = (!c.lds_bins && cache <= dev.lds) ? 1 : 0;
  if (!c.lds_bins && !c.lds_cache) {
    fail(CPAB_ERR_DEVICE, "the backward needs %lld bytes of LDS per workgroup, the device has %d",
         (long long)cache, dev.lds);
    return false;
  }
  const bool reg = T == cpab::kRegSteps && g.nC <= 65535 &&
                   (g.ndim <= 2 ? c.lds_bins != 0 : !adaptive);
  c.reg_steps = reg ? cpab::kRegSteps : 0;
  // Register variant with full bins in 1D/2D: the reverse-sweep table joins the
  // bins in LDS when both fit, so the entry phase 2 reloads at every cell
  // change comes from LDS (C2 backward 176 -> 170 us, C1 19.5 -> 18.6 us).
  const int64_t rev = (int64_t)g.nC * adj_stride(g.ndim) * 4 + 16;
  c.lds_rev = (reg && g.ndim <= 2 && c.lds_bins && table + rev <= dev.lds) ? 1 : 0;
  const int64_t used = c.lds_bins ? table : cache;
  c.lds_table = (!reg && used + table <= dev.lds) ? 1 : 0;
  const int64_t lds = used + (c.lds_table ? table : 0);
  int wg_per_cu;
  if (reg) {
    c.block = adaptive ? 768 : 1024;  // the kernel's launch bound
    wg_per_cu = 1;
  } else {
    // 32 waves per CU as 512-lane workgroups, as many as LDS allows; the cache
    // variant runs one workgroup per CU (104 KiB of LDS in 3D): 12 waves.
    c.block = c.lds_cache ? 768 : 512;
    wg_per_cu = (int)std::max<int64_t>(1, std::min<int64_t>(2048 / c.block, dev.lds / lds));
  }
  const int64_t want = (int64_t)dev.cus * wg_per_cu;
  int64_t chunks = std::max<int64_t>(1, div_up(want, std::max<int64_t>(n_theta, 1)));
  chunks = std::min(chunks, std::max<int64_t>(1, div_up(nP, c.block)));
  c.chunks = (int)chunks;
  *out = c;
  return true;
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- optional kernel timing (HIP events recorded on the launch stream) -----
// Events are created once per device and recycled through a pool: a timed
// launch then costs two hipEventRecord calls, which matters for small,
// host-bound problems where the timing runs inside the measured region.
struct Timed {
  const char* name;
  int device;
  hipEvent_t start, stop;
};
std::mutex g_prof_mu;
std::atomic<bool> g_prof_on{false};
std::vector<Timed> g_prof_pending;
std::vector<std::pair<int, hipEvent_t>> g_prof_pool;  // (device, free event)

// Caller holds g_prof_mu.
bool pool_take(int device, hipEvent_t* e) {
  for (size_t i = g_prof_pool.size(); i-- > 0;) {
    if (g_prof_pool[i].first == device) {
      *e = g_prof_pool[i].second;
      g_prof_pool[i] = g_prof_pool.back();
      g_prof_pool.pop_back();
      return true;
    }
  }
  return hipEventCreate(e) == hipSuccess;
}

bool prof_begin(hipStream_t s, hipEvent_t* a) {
  if (!g_prof_on.load(std::memory_order_relaxed)) return false;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return false;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  if (!pool_take(device, a)) return false;
  if (hipEventRecord(*a, s) != hipSuccess) {
    g_prof_pool.push_back({device, *a});
    return false;
  }
  return true;
}
void prof_end(bool on, hipEvent_t a, const char* name, hipStream_t s) {
  if (!on) return;
  int device = 0;
  (void)hipGetDevice(&device);
  std::lock_guard<std::mutex> lock(g_prof_mu);
  hipEvent_t b;
  if (!pool_take(device, &b)) {
    g_prof_pool.push_back({device, a});
    return;
  }
  (void)hipEventRecord(b, s);
  g_prof_pending.push_back({name, device, a, b});
}

// Forward of a chain of K stages (K = 1: one transform).  ndim 1 uses the
// closed form (Trels unused).
int forward_impl(const char* who, int ndim, int64_t nP, int64_t n_batch, int batched, int K,
                 int nstepsolver, int ncx, int ncy, int ncz, int adaptive, const float* points,
                 const float* Trels, const float* As, float* out, float* stage_points,
                 void* stream) {
  cpab::Geometry g{};
  int rc = check_geometry(ndim, ncx, ncy, ncz, &g);
  if (rc) return rc;
  if (ndim > 1 && (rc = check_steps(nstepsolver))) return rc;
  if ((rc = check_points(nP, n_batch, ndim))) return rc;
  if (K < 1 || K > 4096) return fail(CPAB_ERR_INVALID, "n_stages must be in [1, 4096], got %d", K);
  if ((int64_t)K * n_batch >= (1LL << 31)) return fail(CPAB_ERR_INVALID, "n_stages * n_batch too large");
  if (adaptive != 0 && adaptive != 1) return fail(CPAB_ERR_INVALID, "adaptive_substeps must be 0 or 1");
  if (nP == 0 || n_batch == 0) return CPAB_OK;
  CPAB_REQUIRE(points); CPAB_REQUIRE(As); CPAB_REQUIRE(out);
  if (ndim > 1) CPAB_REQUIRE(Trels);
  CPAB_ALIGNED(As, 16); CPAB_ALIGNED(Trels, 16); CPAB_ALIGNED(points, 4);
  hipStream_t s = as_stream(stream);
  hipEvent_t ev = nullptr;
  const bool timed = prof_begin(s, &ev);
  if (ndim == 1) {
    rc = check_hip(cpab::launch_forward_1d(g, nP, n_batch, batched ? 1 : 0, K, points, As, out,
                                           stage_points, s),
                   who);
  } else {
    const cpab::LaunchCfg cfg = forward_cfg(g, nP, n_batch);
    rc = check_hip(cpab::launch_forward(g, nP, n_batch, batched ? 1 : 0, nstepsolver, K, adaptive,
                                        points, Trels, As, out, stage_points, cfg, s),
                   who);
  }
  prof_end(timed, ev, "forward", s);
  return rc;
}


constexpr int64_t kAlign = 256;

int64_t align_up(int64_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Workspace of a K-stage backward (rows = K * n_batch): with full LDS bins the
// dense-part masks [rows, ceil(chunks/64)] and the partial tables
// [rows, chunks, nC, ppc]; then the inter-stage adjoint [n_batch, ndim, nP]
// (K > 1), the reverse-sweep table [rows, nC, 4|12|24] (G and the inverse
// one-step map per cell, cpab_device.hpp RevStride), the per-block norms of
// the inverse maps [rows, adjoint_table_blocks(nC)] and (2D) the per-block
// parts of the rows' domain-edge bounds [rows, adjoint_table_blocks(nC)].
struct BackwardWorkspace {
  int64_t dense_words, partials_offset, lam_offset, g_offset, amp_offset, edge_offset;
  int64_t det_stat_offset, det_sums_offset, det_flags_offset, total;
};

// Deterministic reduction (cpab_set_deterministic), per calling thread.
thread_local int t_deterministic = 0;


BackwardWorkspace backward_workspace(const cpab::Geometry& g, int64_t nP, int64_t n_batch, int K,
                                     const cpab::LaunchCfg& cfg, bool det = false) {
  BackwardWorkspace w{};
  const bool dense = cfg.lds_bins && !det;
  const int64_t parts = dense ? (int64_t)K * n_batch * cfg.chunks : 0;
  w.dense_words = dense ? (int64_t)K * n_batch * ((cfg.chunks + 63) / 64) : 0;
  w.partials_offset = align_up(w.dense_words * 8);
  w.lam_offset = align_up(w.partials_offset + parts * g.nC * g.ppc() * 4);
  w.g_offset = K > 1 ? align_up(w.lam_offset + n_batch * g.ndim * nP * 4) : w.lam_offset;
  w.amp_offset = align_up(w.g_offset + (int64_t)K * n_batch * g.nC * adj_stride(g.ndim) * 4);
  const int64_t blocks = (int64_t)K * n_batch * cpab::adjoint_table_blocks(g.nC);
  w.edge_offset = align_up(w.amp_offset + blocks * 4);
  w.total = w.edge_offset + (g.ndim == 2 ? blocks * cpab::kEdgeAccBytes : 0);
  // deterministic reduction: row stats [rows], 64-bit sums [rows, nC, ppc] and
  // non-finite flags [rows, nC, ppc]
  const int64_t comps = (int64_t)K * n_batch * g.nC * g.ppc();
  w.det_stat_offset = align_up(w.total);
  w.det_sums_offset = align_up(w.det_stat_offset + (int64_t)K * n_batch * 4);
  w.det_flags_offset = w.det_sums_offset + comps * 8;
  if (det) w.total = w.det_flags_offset + comps * 4;
  return w;
}

// Optional projection of the backward's moments onto the basis, enqueued by
// the backward entry point after the moments: grad_theta [rows, d] from B's
// CSC tables.
struct Projection {
  int d = 0;
  const int32_t* col_ptr = nullptr;
  const int32_t* row_idx = nullptr;
  const float* vals = nullptr;
  float* grad_theta = nullptr;  // null: moments only
};

int check_projection(const Projection& pr) {
  if (!pr.grad_theta) return CPAB_OK;
  if (pr.d < 0) return fail(CPAB_ERR_INVALID, "negative d");
  if (pr.d > 0) { CPAB_REQUIRE(pr.col_ptr); CPAB_REQUIRE(pr.row_idx); CPAB_REQUIRE(pr.vals); }
  return CPAB_OK;
}


// Launch shape of the deterministic passes (kDetBlock, kDetPerCU): pass 1
// keeps the row's full table of 64-bit sums in LDS when it fits in
// kDetFullBytes (lds_bins), else a hashed cache; at most one pass over a row's
// points.  The shape depends only on the device and the problem, so every run
// groups the trajectories' sums the same way.
bool det_cfg(const cpab::Geometry& g, int64_t nP, int64_t n_theta, cpab::LaunchCfg* out) {
  const DeviceInfo dev = device_info();
  cpab::LaunchCfg c{};
  c.block = cpab::kDetBlock[g.ndim];
  c.lds_bins = cpab::det_full_bytes_for(g.ndim, g.nC) <= cpab::kDetFullBytes[g.ndim] ? 1 : 0;
  const int64_t lds = c.lds_bins ? cpab::det_full_bytes_for(g.ndim, g.nC)
                                 : cpab::det_cache_bytes_for(g.ndim);
  if (lds + 16 > dev.lds) {
    fail(CPAB_ERR_DEVICE, "the deterministic backward needs %lld bytes of LDS per workgroup, the "
         "device has %d", (long long)(lds + 16), dev.lds);
    return false;
  }
  const int64_t per_cu = cpab::kDetPerCU[g.ndim];
  int64_t chunks = std::max<int64_t>(1, div_up(dev.cus * per_cu, std::max<int64_t>(n_theta, 1)));
  chunks = std::min(chunks, std::max<int64_t>(1, div_up(nP, c.block)));
  c.chunks = (int)chunks;
  *out = c;
  return true;
}

int64_t workspace_size_impl(int ndim, int64_t nP, int64_t n_batch, int K, int nC) {
  if (ndim < 1 || ndim > 3 || nP <= 0 || n_batch <= 0 || nC <= 0 || K < 1) return 0;
  cpab::Geometry g{};
  g.ndim = ndim;
  g.nC = nC;
  if (t_deterministic) {
    cpab::LaunchCfg det;
    if (!det_cfg(g, nP, n_batch, &det)) return 0;
    return backward_workspace(g, nP, n_batch, K, det, true).total;
  }
  // Whichever variant runs (register or segmented) fits.
  cpab::LaunchCfg reg, seg;
  if (!backward_cfg(g, nP, n_batch, cpab::kRegSteps, 0, &reg) || !backward_cfg(g, nP, n_batch, 0, 1, &seg))
    return 0;
  return std::max(backward_workspace(g, nP, n_batch, K, reg).total,
                  backward_workspace(g, nP, n_batch, K, seg).total);
}

// Moments from the backward's per-cell sums, then (optionally) their projection.
int finish_and_project(const char* who, int ndim, int64_t rows, int nC, const cpab::LaunchCfg& cfg,
                       int T, const float* partials, const uint64_t* dense, const float* As,
                       float* moments, const Projection& pr, hipStream_t s) {
  int rc = check_hip(cpab::launch_finish_moments(ndim, rows, nC, cfg.lds_bins ? cfg.chunks : 0, T,
                                                 partials, dense, As, moments, s),
                     who);
  if (rc || !pr.grad_theta || pr.d == 0) return rc;
  return check_hip(cpab::launch_project(rows, nC * ndim * (ndim + 1), pr.d, moments, pr.col_ptr,
                                        pr.row_idx, pr.vals, pr.grad_theta, s),
                   who);
}

// `timing`: record the backward kernel with the optional HIP-event timing
// (off for the allocation-free entry point: the event pool may create events).
int backward_impl(const char* who, int ndim, int64_t nP, int64_t n_batch, int batched, int K,
                  int nstepsolver, int ncx, int ncy, int ncz, int adaptive, const float* points,
                  const float* stage_points, const float* As, const float* grad_out,
                  float* moments, float* grad_points, void* workspace, int64_t workspace_bytes,
                  void* stream, const Projection& pr = Projection(), bool timing = true) {
  cpab::Geometry g{};
  int rc = check_geometry(ndim, ncx, ncy, ncz, &g);
  if (rc) return rc;
  if ((rc = check_steps(nstepsolver))) return rc;
  if ((rc = check_points(nP, n_batch, ndim))) return rc;
  if (K < 1 || K > 4096) return fail(CPAB_ERR_INVALID, "n_stages must be in [1, 4096], got %d", K);
  if ((int64_t)K * n_batch >= (1LL << 31)) return fail(CPAB_ERR_INVALID, "n_stages * n_batch too large");
  if (adaptive != 0 && adaptive != 1) return fail(CPAB_ERR_INVALID, "adaptive_substeps must be 0 or 1");
  if ((rc = check_projection(pr))) return rc;
  if (n_batch == 0) return CPAB_OK;
  CPAB_REQUIRE(moments);
  hipStream_t s = as_stream(stream);
  const int R = g.nC * g.ppc();
  const int64_t rows = (int64_t)K * n_batch;
  if (nP == 0) {
    rc = check_hip(cpab::launch_fill(moments, rows * R, 0.0f, s), who);
    if (rc == CPAB_OK && pr.grad_theta)
      rc = check_hip(cpab::launch_fill(pr.grad_theta, rows * pr.d, 0.0f, s), who);
    return rc;
  }
  CPAB_REQUIRE(points); CPAB_REQUIRE(As); CPAB_REQUIRE(grad_out);
  CPAB_ALIGNED(As, 16); CPAB_ALIGNED(points, 4); CPAB_ALIGNED(grad_out, 4);
  CPAB_ALIGNED(workspace, 16);
  if (K > 1) CPAB_REQUIRE(stage_points);
  const bool det = t_deterministic != 0;
  cpab::LaunchCfg cfg;
  if (det ? !det_cfg(g, nP, n_batch, &cfg) : !backward_cfg(g, nP, n_batch, nstepsolver, adaptive, &cfg))
    return CPAB_ERR_DEVICE;
  // A chain restages each stage's table: measured slower than L2 reads (C5
  // backward 185 -> 190 us), so chains keep the reverse-sweep table in HBM.
  if (K > 1) cfg.lds_rev = 0;
  const BackwardWorkspace w = backward_workspace(g, nP, n_batch, K, cfg, det);
  if (workspace == nullptr || workspace_bytes < w.total)
    return fail(CPAB_ERR_INVALID, "workspace too small: need %lld bytes, got %lld",
                (long long)w.total, (long long)workspace_bytes);
  char* ws = static_cast<char*>(workspace);
  uint64_t* dense = reinterpret_cast<uint64_t*>(ws);
  float* partials = reinterpret_cast<float*>(ws + w.partials_offset);
  float* lam = K > 1 ? reinterpret_cast<float*>(ws + w.lam_offset) : nullptr;
  float* G = reinterpret_cast<float*>(ws + w.g_offset);
  float* amp = reinterpret_cast<float*>(ws + w.amp_offset);
  // The domain-edge bound lets the replay of waves that stay inside the domain
  // skip the lookup's edge test.  Not for chains: each stage would pay the
  // bound's reduction, and a chain's slowest waves (those on the domain's
  // edge, which never qualify) set its time (C5 backward 174 -> 185 us).
  cpab::EdgeAcc* edge = ndim == 2 && K == 1 && !det
                           ? reinterpret_cast<cpab::EdgeAcc*>(ws + w.edge_offset)
                           : nullptr;
  // G table, inverse-map norms and domain-edge bound parts; the HBM sums and
  // dense-part masks cleared.
  rc = check_hip(cpab::launch_adjoint_table(ndim, rows, g.nx, g.ny, g.nC, nstepsolver, As, G,
                                            moments, amp, edge, dense, w.dense_words, s),
                 who);
  if (rc) return rc;
  if (det) {
    unsigned* stat = reinterpret_cast<unsigned*>(ws + w.det_stat_offset);
    auto* sums = reinterpret_cast<unsigned long long*>(ws + w.det_sums_offset);
    unsigned* flags = reinterpret_cast<unsigned*>(ws + w.det_flags_offset);
    rc = check_hip(cpab::launch_fill(reinterpret_cast<float*>(stat),
                                     (w.total - w.det_stat_offset) / 4, 0.0f, s),
                   who);
    hipEvent_t dev_ev = nullptr;
    const bool dtimed = rc == CPAB_OK && timing && prof_begin(s, &dev_ev);
    for (int pass = 1; rc == CPAB_OK && pass <= 2; ++pass)
      rc = check_hip(cpab::launch_backward(g, nP, n_batch, batched ? 1 : 0, nstepsolver, K,
                                           adaptive, points, stage_points, As, G, amp, nullptr,
                                           grad_out, moments, nullptr, nullptr, lam, grad_points,
                                           cfg, s, pass, stat, sums, flags),
                     who);
    prof_end(dtimed, dev_ev, "backward", s);
    if (rc) return rc;
    rc = check_hip(cpab::launch_finish_moments_det(ndim, rows, g.nC, nP, nstepsolver, stat, sums,
                                                   flags, As, moments, s),
                   who);
    if (rc || !pr.grad_theta || pr.d == 0) return rc;
    return check_hip(cpab::launch_project(rows, g.nC * g.ppc(), pr.d, moments, pr.col_ptr,
                                          pr.row_idx, pr.vals, pr.grad_theta, s),
                     who);
  }
  hipEvent_t ev = nullptr;
  const bool timed = timing && prof_begin(s, &ev);
  rc = check_hip(cpab::launch_backward(g, nP, n_batch, batched ? 1 : 0, nstepsolver, K, adaptive,
                                       points, stage_points, As, G, amp, edge, grad_out, moments,
                                       partials, dense, lam, grad_points, cfg, s),
                 who);
  prof_end(timed, ev, "backward", s);
  if (rc) return rc;
  return finish_and_project(who, ndim, rows, g.nC, cfg, nstepsolver, partials, dense, As, moments,
                            pr, s);
}

// ---- allocation-free backward --------------------------------------------
// The workspace of cpab_backward_noalloc: one array per GPU, in the library's
// code object.  Host code never passes `scratch` itself (in host code the name
// is only a stand-in, not a device address): each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current.
constexpr int64_t kScratchBytes = CPAB_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// Device address of this device's `scratch` (nullptr after an error, with the
// message set).
void* scratch_on_current_device() {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    check_hip(e, "cpab_backward_noalloc: hipGetDevice");
    return nullptr;
  }
  if (dev < 0 || dev >= 64) {
    fail(CPAB_ERR_DEVICE, "cpab_backward_noalloc: device %d beyond the supported 64", dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      check_hip(e != hipSuccess ? e : hipErrorInvalidSymbol, "cpab_backward_noalloc: hipGetSymbolAddress");
      return nullptr;
    }
    addr[dev] = p;
  }
  return addr[dev];
}

// Image geometry of the fused transform_data calls (validated like the
// resampling entry points, plus the integrator's limits).
int image_shape(int ndim, int64_t n_batch, int64_t C, const int64_t* in_size,
                const int64_t* out_size, cpab::ImageShape* img) {
  if (ndim < 1 || ndim > 3) return fail(CPAB_ERR_INVALID, "ndim must be 1, 2 or 3, got %d", ndim);
  CPAB_REQUIRE(in_size); CPAB_REQUIRE(out_size);
  if (n_batch < 0 || C < 1) return fail(CPAB_ERR_INVALID, "need n_batch >= 0 and n_channels >= 1");
  if (n_batch >= 65536) return fail(CPAB_ERR_INVALID, "n_batch=%lld exceeds the grid limit 65535", (long long)n_batch);
  int64_t nP = 1, plane = 1;
  for (int k = 0; k < ndim; ++k) {
    if (in_size[k] < 1 || out_size[k] < 1) return fail(CPAB_ERR_INVALID, "sizes must be >= 1 (axis %d)", k);
    nP *= out_size[k];
    plane *= in_size[k];
    if (nP >= kMaxPoints)
      return fail(CPAB_ERR_INVALID, "output of %lld positions exceeds the 32-bit point index", (long long)nP);
    // the gathers address one channel with 32-bit byte offsets
    if (plane > (1LL << 30)) return fail(CPAB_ERR_INVALID, "one data channel must hold at most 2^30 values");
  }
  if (n_batch * C * std::max(nP, plane) >= (1LL << 40)) return fail(CPAB_ERR_INVALID, "problem too large");
  *img = cpab::ImageShape{};
  for (int k = 0; k < 3; ++k) {
    img->o[k] = k < ndim ? (int)out_size[k] : 1;
    img->in[k] = k < ndim ? (int)in_size[k] : 1;
    img->inv_o[k] = 1.0 / (double)img->o[k];
  }
  img->walk_tiles = ndim >= 2 && img->o[ndim - 1] % cpab::kWalkW == 0 && img->o[ndim - 2] % cpab::kWalkH == 0;
  img->C = (int)C;
  img->nP = (int)nP;
  img->plane_in = plane;
  return CPAB_OK;
}

}  // namespace

extern "C" {

const char* cpab_last_error_string(void) { return g_last_error.c_str(); }

// 300: the backward entry points can also project the moments onto the basis
// (cpab_backward_project; projection arguments of the chain and
// transform_data backwards).  200: the fused transform_data entry points take
// the uniform grid's per-axis coordinates instead of the meshgrid.
int cpab_abi_version(void) { return 401; }

int cpab_affine(int ndim, int64_t n_theta, int nC, int d, const float* theta,
                const int32_t* row_ptr, const int32_t* col_idx, const float* vals, float* As,
                void* stream) {
  if (ndim < 1 || ndim > 3) return fail(CPAB_ERR_INVALID, "ndim must be 1, 2 or 3, got %d", ndim);
  if (n_theta < 0 || nC < 0 || d < 0) return fail(CPAB_ERR_INVALID, "negative size");
  if (n_theta == 0 || nC == 0) return CPAB_OK;
  CPAB_REQUIRE(row_ptr); CPAB_REQUIRE(As);
  if (d > 0) { CPAB_REQUIRE(theta); CPAB_REQUIRE(col_idx); CPAB_REQUIRE(vals); }
  const int rows = nC * ndim * (ndim + 1);
  return check_hip(cpab::launch_affine(n_theta, rows, d, theta, row_ptr, col_idx, vals, As,
                                       as_stream(stream)),
                   "cpab_affine");
}

int cpab_expm(int ndim, int64_t n_matrices, float dT, const float* As, float* Trels,
              void* stream) {
  if (ndim < 1 || ndim > 3) return fail(CPAB_ERR_INVALID, "As_in must have ndim=1,2,3, got %d", ndim);
  if (n_matrices < 0) return fail(CPAB_ERR_INVALID, "negative n_matrices");
  if (n_matrices == 0) return CPAB_OK;
  CPAB_REQUIRE(As); CPAB_REQUIRE(Trels);
  CPAB_ALIGNED(As, 16); CPAB_ALIGNED(Trels, 16);
  return check_hip(cpab::launch_expm(ndim, n_matrices, dT, As, Trels, as_stream(stream)),
                   "cpab_expm");
}

int cpab_affine_expm(int ndim, int64_t n_theta, int nC, int d, const float* theta,
                     const int32_t* row_ptr, const int32_t* col_idx, const float* vals, float dT,
                     float* As, float* Trels, void* stream) {
  if (ndim < 1 || ndim > 3) return fail(CPAB_ERR_INVALID, "ndim must be 1, 2 or 3, got %d", ndim);
  if (n_theta < 0 || nC < 0 || d < 0) return fail(CPAB_ERR_INVALID, "negative size");
  if (n_theta == 0 || nC == 0) return CPAB_OK;
  CPAB_REQUIRE(row_ptr); CPAB_REQUIRE(As); CPAB_REQUIRE(Trels);
  if (d > 0) { CPAB_REQUIRE(theta); CPAB_REQUIRE(col_idx); CPAB_REQUIRE(vals); }
  CPAB_ALIGNED(As, 16); CPAB_ALIGNED(Trels, 16);
  return check_hip(cpab::launch_affine_expm(ndim, n_theta, nC, d, theta, row_ptr, col_idx, vals,
                                            dT, As, Trels, as_stream(stream)),
                   "cpab_affine_expm");
}

int cpab_forward_1d_closed_form(int64_t nP, int64_t n_theta, int batched, int ncx,
                                const float* points, const float* As, float* out, void* stream) {
  return forward_impl("cpab_forward_1d_closed_form", 1, nP, n_theta, batched, 1, 1, ncx, 1, 1, 0,
                      points, nullptr, As, out, nullptr, stream);
}

int cpab_forward(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver, int ncx,
                 int ncy, int ncz, int adaptive, const float* points, const float* Trels,
                 const float* As, float* out, void* stream) {
  return forward_impl("cpab_forward", ndim, nP, n_theta, batched, 1, nstepsolver, ncx, ncy, ncz,
                      adaptive, points, Trels, As, out, nullptr, stream);
}

int cpab_chain_forward(int ndim, int64_t nP, int64_t n_batch, int batched, int n_stages,
                       int nstepsolver, int ncx, int ncy, int ncz, int adaptive,
                       const float* points, const float* Trels, const float* As, float* out,
                       float* stage_points, void* stream) {
  return forward_impl("cpab_chain_forward", ndim, nP, n_batch, batched, n_stages, nstepsolver, ncx,
                      ncy, ncz, adaptive, points, Trels, As, out, stage_points, stream);
}

int cpab_trace_cells(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver,
                     int ncx, int ncy, int ncz, int adaptive, const float* points,
                     const float* Trels, const float* As, int32_t* cells, void* stream) {
  if (ndim != 2 && ndim != 3) return fail(CPAB_ERR_INVALID, "cell tracing covers the 2D/3D fixed-step forward, got ndim=%d", ndim);
  cpab::Geometry g{};
  int rc = check_geometry(ndim, ncx, ncy, ncz, &g);
  if (rc) return rc;
  if ((rc = check_steps(nstepsolver))) return rc;
  if ((rc = check_points(nP, n_theta, ndim))) return rc;
  if (adaptive != 0 && adaptive != 1) return fail(CPAB_ERR_INVALID, "adaptive_substeps must be 0 or 1");
  if (nP == 0 || n_theta == 0) return CPAB_OK;
  CPAB_REQUIRE(points); CPAB_REQUIRE(Trels); CPAB_REQUIRE(As); CPAB_REQUIRE(cells);
  CPAB_ALIGNED(As, 16); CPAB_ALIGNED(Trels, 16);
  return check_hip(cpab::launch_trace_cells(g, nP, n_theta, batched ? 1 : 0, nstepsolver, adaptive,
                                            points, Trels, As, cells, as_stream(stream)),
                   "cpab_trace_cells");
}

int64_t cpab_backward_workspace_size(int ndim, int64_t nP, int64_t n_theta, int nC) {
  return workspace_size_impl(ndim, nP, n_theta, 1, nC);
}

int64_t cpab_chain_backward_workspace_size(int ndim, int64_t nP, int64_t n_batch, int n_stages,
                                           int nC) {
  return workspace_size_impl(ndim, nP, n_batch, n_stages, nC);
}

int cpab_backward(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver, int ncx,
                  int ncy, int ncz, int adaptive, const float* points, const float* As,
                  const float* grad_out, float* moments, float* grad_points, void* workspace,
                  int64_t workspace_bytes, void* stream) {
  return backward_impl("cpab_backward", ndim, nP, n_theta, batched, 1, nstepsolver, ncx, ncy, ncz,
                       adaptive, points, nullptr, As, grad_out, moments, grad_points, workspace,
                       workspace_bytes, stream);
}

int cpab_backward_project(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver,
                          int ncx, int ncy, int ncz, int adaptive, const float* points,
                          const float* As, const float* grad_out, int d, const int32_t* col_ptr,
                          const int32_t* row_idx, const float* vals, float* moments,
                          float* grad_theta, float* grad_points, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  Projection pr;
  pr.d = d;
  pr.col_ptr = col_ptr;
  pr.row_idx = row_idx;
  pr.vals = vals;
  pr.grad_theta = grad_theta;
  CPAB_REQUIRE(grad_theta);
  return backward_impl("cpab_backward_project", ndim, nP, n_theta, batched, 1, nstepsolver, ncx,
                       ncy, ncz, adaptive, points, nullptr, As, grad_out, moments, grad_points,
                       workspace, workspace_bytes, stream, pr);
}

int cpab_backward_noalloc(int ndim, int64_t nP, int64_t n_theta, int batched, int nstepsolver,
                          int ncx, int ncy, int ncz, int adaptive, const float* points,
                          const float* As, const float* grad_out, float* moments,
                          float* grad_points, void* stream) {
  // The size check needs only the geometry; backward_impl repeats the full
  // validation before anything is enqueued.
  cpab::Geometry g{};
  int rc = check_geometry(ndim, ncx, ncy, ncz, &g);
  if (rc) return rc;
  if ((rc = check_steps(nstepsolver))) return rc;
  if ((rc = check_points(nP, n_theta, ndim))) return rc;
  if (adaptive != 0 && adaptive != 1) return fail(CPAB_ERR_INVALID, "adaptive_substeps must be 0 or 1");
  if (n_theta > 0 && nP > 0) {
    cpab::LaunchCfg cfg;
    const bool det = t_deterministic != 0;
    if (det ? !det_cfg(g, nP, n_theta, &cfg)
            : !backward_cfg(g, nP, n_theta, nstepsolver, adaptive, &cfg))
      return CPAB_ERR_DEVICE;
    const int64_t need = backward_workspace(g, nP, n_theta, 1, cfg, det).total;
    if (need > kScratchBytes)
      return fail(CPAB_ERR_INVALID,
                  "cpab_backward_noalloc: this problem needs %lld bytes of workspace, beyond the "
                  "%lld-byte no-allocation limit; use cpab_backward with a workspace",
                  (long long)need, (long long)kScratchBytes);
  }
  void* ws = scratch_on_current_device();
  if (ws == nullptr) return CPAB_ERR_DEVICE;
  return backward_impl("cpab_backward_noalloc", ndim, nP, n_theta, batched, 1, nstepsolver, ncx,
                       ncy, ncz, adaptive, points, nullptr, As, grad_out, moments, grad_points, ws,
                       kScratchBytes, stream, Projection(), /*timing=*/false);
}

int cpab_chain_backward(int ndim, int64_t nP, int64_t n_batch, int batched, int n_stages,
                        int nstepsolver, int ncx, int ncy, int ncz, int adaptive,
                        const float* points, const float* stage_points, const float* As,
                        const float* grad_out, int d, const int32_t* col_ptr,
                        const int32_t* row_idx, const float* vals, float* moments,
                        float* grad_theta, float* grad_points, void* workspace,
                        int64_t workspace_bytes, void* stream) {
  Projection pr;
  pr.d = d;
  pr.col_ptr = col_ptr;
  pr.row_idx = row_idx;
  pr.vals = vals;
  pr.grad_theta = grad_theta;
  return backward_impl("cpab_chain_backward", ndim, nP, n_batch, batched, n_stages, nstepsolver,
                       ncx, ncy, ncz, adaptive, points, stage_points, As, grad_out, moments,
                       grad_points, workspace, workspace_bytes, stream, pr);
}

int cpab_transform_data_forward(int ndim, int64_t n_batch, int64_t n_channels,
                                const int64_t* in_size, const int64_t* out_size, int nstepsolver,
                                int ncx, int ncy, int ncz, int adaptive, const float* axes,
                                const float* Trels, const float* As, const float* data,
                                float* out, float* final_points, float* seed_grad, void* stream) {
  cpab::Geometry g{};
  int rc = check_geometry(ndim, ncx, ncy, ncz, &g);
  if (rc) return rc;
  if (ndim > 1 && (rc = check_steps(nstepsolver))) return rc;
  if (adaptive != 0 && adaptive != 1) return fail(CPAB_ERR_INVALID, "adaptive_substeps must be 0 or 1");
  cpab::ImageShape img;
  if ((rc = image_shape(ndim, n_batch, n_channels, in_size, out_size, &img))) return rc;
  if (n_batch == 0) return CPAB_OK;
  CPAB_REQUIRE(axes); CPAB_REQUIRE(As); CPAB_REQUIRE(data); CPAB_REQUIRE(out);
  if (ndim > 1) CPAB_REQUIRE(Trels);
  CPAB_ALIGNED(As, 16); CPAB_ALIGNED(Trels, 16);
  if (seed_grad && n_channels != 1)
    return fail(CPAB_ERR_INVALID, "seed_grad needs n_channels == 1, got %lld", (long long)n_channels);
  hipStream_t s = as_stream(stream);
  const cpab::LaunchCfg cfg = forward_cfg(g, img.nP, n_batch);
  hipEvent_t ev = nullptr;
  const bool timed = prof_begin(s, &ev);
  rc = check_hip(cpab::launch_image_forward(g, img, n_batch, nstepsolver, adaptive, axes, Trels,
                                            As, data, out, final_points, seed_grad, cfg, s),
                 "cpab_transform_data_forward");
  prof_end(timed, ev, "image_forward", s);
  return rc;
}

int64_t cpab_transform_data_backward_workspace_size(int ndim, int64_t n_batch,
                                                    const int64_t* out_size, int nC) {
  if (ndim < 1 || ndim > 3 || out_size == nullptr) return 0;
  int64_t nP = 1;
  for (int k = 0; k < ndim; ++k) nP *= std::max<int64_t>(out_size[k], 0);
  return workspace_size_impl(ndim, nP, n_batch, 1, nC);
}

// The deterministic grad_data's part of the transform_data backward's
// workspace, after backward_workspace(...).total: batch rows' scales [n_batch]
// and 64-bit sums [n_batch, n_channels, plane_in].
struct DataWorkspace {
  int64_t gstat_offset, gsums_offset, total;
};

DataWorkspace data_workspace(int64_t base, int64_t n_batch, int64_t n_channels, int64_t plane_in) {
  DataWorkspace d{};
  d.gstat_offset = align_up(base);
  d.gsums_offset = align_up(d.gstat_offset + n_batch * 4);
  d.total = d.gsums_offset + n_batch * n_channels * plane_in * 8;
  return d;
}

int64_t cpab_transform_data_backward_data_workspace_size(int ndim, int64_t n_batch,
                                                         int64_t n_channels,
                                                         const int64_t* in_size) {
  if (!t_deterministic || ndim < 1 || ndim > 3 || n_batch <= 0 || n_channels <= 0 || !in_size)
    return 0;
  int64_t plane = 1;
  for (int k = 0; k < ndim; ++k) {
    if (in_size[k] <= 0) return 0;
    plane *= in_size[k];
  }
  // the slack covers the two alignments after any base size
  return data_workspace(0, n_batch, n_channels, plane).total + 2 * kAlign;
}

int cpab_transform_data_backward(int ndim, int64_t n_batch, int64_t n_channels,
                                 const int64_t* in_size, const int64_t* out_size, int nstepsolver,
                                 int ncx, int ncy, int ncz, int adaptive, const float* axes,
                                 const float* final_points, const float* seed_grad,
                                 const float* As, const float* data,
                                 const float* grad_out, int d, const int32_t* col_ptr,
                                 const int32_t* row_idx, const float* vals, float* moments,
                                 float* grad_theta, float* grad_data, void* workspace,
                                 int64_t workspace_bytes, void* stream) {
  cpab::Geometry g{};
  int rc = check_geometry(ndim, ncx, ncy, ncz, &g);
  if (rc) return rc;
  if ((rc = check_steps(nstepsolver))) return rc;
  if (adaptive != 0 && adaptive != 1) return fail(CPAB_ERR_INVALID, "adaptive_substeps must be 0 or 1");
  cpab::ImageShape img;
  if ((rc = image_shape(ndim, n_batch, n_channels, in_size, out_size, &img))) return rc;
  Projection pr;
  pr.d = d;
  pr.col_ptr = col_ptr;
  pr.row_idx = row_idx;
  pr.vals = vals;
  pr.grad_theta = grad_theta;
  if ((rc = check_projection(pr))) return rc;
  if (n_batch == 0) return CPAB_OK;
  CPAB_REQUIRE(axes); CPAB_REQUIRE(As); CPAB_REQUIRE(data);
  // The seed comes from seed_grad (one channel) when given; grad_data's
  // scatter and the general seed need the final points.
  if (seed_grad && n_channels != 1)
    return fail(CPAB_ERR_INVALID, "seed_grad needs n_channels == 1, got %lld", (long long)n_channels);
  if (!seed_grad || grad_data) CPAB_REQUIRE(final_points);
  if (grad_data) seed_grad = nullptr;
  CPAB_ALIGNED(As, 16); CPAB_ALIGNED(workspace, 16);
  CPAB_REQUIRE(grad_out); CPAB_REQUIRE(moments);
  hipStream_t s = as_stream(stream);
  const bool det = t_deterministic != 0;
  cpab::LaunchCfg cfg;
  if (det ? !det_cfg(g, img.nP, n_batch, &cfg)
          : !backward_cfg(g, img.nP, n_batch, nstepsolver, adaptive, &cfg))
    return CPAB_ERR_DEVICE;
  const BackwardWorkspace w = backward_workspace(g, img.nP, n_batch, 1, cfg, det);
  // the deterministic grad_data's sums follow
  const bool det_data = det && grad_data != nullptr;
  const DataWorkspace dw = data_workspace(w.total, n_batch, n_channels, img.plane_in);
  const int64_t need = det_data ? dw.total : w.total;
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CPAB_ERR_INVALID,
                "workspace too small: need %lld bytes, got %lld%s", (long long)need,
                (long long)workspace_bytes,
                det_data ? " (cpab_transform_data_backward_workspace_size plus "
                           "cpab_transform_data_backward_data_workspace_size)"
                         : "");
  char* ws = static_cast<char*>(workspace);
  uint64_t* dense = reinterpret_cast<uint64_t*>(ws);
  float* partials = reinterpret_cast<float*>(ws + w.partials_offset);
  float* G = reinterpret_cast<float*>(ws + w.g_offset);
  float* amp = reinterpret_cast<float*>(ws + w.amp_offset);
  cpab::EdgeAcc* edge =
      ndim == 2 && !det ? reinterpret_cast<cpab::EdgeAcc*>(ws + w.edge_offset) : nullptr;
  const char* who = "cpab_transform_data_backward";
  rc = check_hip(cpab::launch_adjoint_table(ndim, n_batch, g.nx, g.ny, g.nC, nstepsolver, As, G,
                                            moments, amp, edge, dense, w.dense_words, s),
                 who);
  if (rc) return rc;
  if (grad_data) {
    rc = check_hip(cpab::launch_fill(grad_data, n_batch * n_channels * img.plane_in, 0.0f, s), who);
    if (rc) return rc;
  }
  hipEvent_t ev = nullptr;
  const bool timed = prof_begin(s, &ev);
  if (det) {
    unsigned* stat = reinterpret_cast<unsigned*>(ws + w.det_stat_offset);
    auto* sums = reinterpret_cast<unsigned long long*>(ws + w.det_sums_offset);
    unsigned* flags = reinterpret_cast<unsigned*>(ws + w.det_flags_offset);
    unsigned* gstat = det_data ? reinterpret_cast<unsigned*>(ws + dw.gstat_offset) : nullptr;
    auto* gsums =
        det_data ? reinterpret_cast<unsigned long long*>(ws + dw.gsums_offset) : nullptr;
    rc = check_hip(cpab::launch_fill(reinterpret_cast<float*>(stat),
                                     (need - w.det_stat_offset) / 4, 0.0f, s),
                   who);
    if (rc == CPAB_OK && det_data)
      rc = check_hip(cpab::launch_det_data_stat(ndim, img, n_batch, final_points, grad_out, gstat,
                                                s),
                     who);
    for (int pass = 1; rc == CPAB_OK && pass <= 2; ++pass)
      rc = check_hip(cpab::launch_image_backward(g, img, n_batch, nstepsolver, adaptive, axes,
                                                 final_points, seed_grad, As, G, amp, nullptr,
                                                 data, grad_out, moments, nullptr, nullptr,
                                                 grad_data, cfg, s, pass, stat, sums, flags,
                                                 gstat, gsums),
                     who);
    prof_end(timed, ev, "image_backward", s);
    if (rc == CPAB_OK && det_data)
      rc = check_hip(cpab::launch_det_data_finish(ndim, img, n_batch, gstat, gsums, grad_data, s),
                     who);
    if (rc) return rc;
    rc = check_hip(cpab::launch_finish_moments_det(ndim, n_batch, g.nC, img.nP, nstepsolver, stat,
                                                   sums, flags, As, moments, s),
                   who);
    if (rc || !pr.grad_theta || pr.d == 0) return rc;
    return check_hip(cpab::launch_project(n_batch, g.nC * g.ppc(), pr.d, moments, pr.col_ptr,
                                          pr.row_idx, pr.vals, pr.grad_theta, s),
                     who);
  }
  rc = check_hip(cpab::launch_image_backward(g, img, n_batch, nstepsolver, adaptive, axes,
                                             final_points, seed_grad, As, G, amp, edge, data,
                                             grad_out, moments, partials, dense, grad_data, cfg, s),
                 who);
  prof_end(timed, ev, "image_backward", s);
  if (rc) return rc;
  return finish_and_project(who, ndim, n_batch, g.nC, cfg, nstepsolver, partials, dense, As,
                            moments, pr, s);
}

void cpab_set_deterministic(int on) { t_deterministic = on ? 1 : 0; }

int cpab_deterministic(void) { return t_deterministic; }

int cpab_project(int64_t n_theta, int D, int d, const float* moments, const int32_t* col_ptr,
                 const int32_t* row_idx, const float* vals, float* grad_theta, void* stream) {
  if (n_theta < 0 || D < 0 || d < 0) return fail(CPAB_ERR_INVALID, "negative size");
  if (n_theta == 0 || d == 0) return CPAB_OK;
  CPAB_REQUIRE(moments); CPAB_REQUIRE(col_ptr); CPAB_REQUIRE(row_idx); CPAB_REQUIRE(vals);
  CPAB_REQUIRE(grad_theta);
  return check_hip(cpab::launch_project(n_theta, D, d, moments, col_ptr, row_idx, vals,
                                        grad_theta, as_stream(stream)),
                   "cpab_project");
}

int cpab_sum_batch(int64_t n_theta, int64_t n, const float* src, float* dst, void* stream) {
  if (n_theta < 0 || n < 0) return fail(CPAB_ERR_INVALID, "negative size");
  if (n == 0) return CPAB_OK;
  CPAB_REQUIRE(dst);
  if (n_theta > 0) CPAB_REQUIRE(src);
  return check_hip(cpab::launch_sum_batch(n_theta, n, src, dst, as_stream(stream)),
                   "cpab_sum_batch");
}

void cpab_profile_enable(int on) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  g_prof_on.store(on != 0, std::memory_order_relaxed);
}

int cpab_profile_read(const char* kernel, double* total_ms, int64_t* launches) {
  CPAB_REQUIRE(kernel); CPAB_REQUIRE(total_ms); CPAB_REQUIRE(launches);
  std::lock_guard<std::mutex> lock(g_prof_mu);
  double tot = 0.0;
  int64_t n = 0;
  hipError_t first = hipSuccess;
  std::vector<Timed> keep;
  for (const Timed& t : g_prof_pending) {
    if (std::strcmp(t.name, kernel) != 0) { keep.push_back(t); continue; }
    // Every matching record is consumed (and its events returned to the
    // pool) even if one of them fails.
    float ms = 0.0f;
    hipError_t e = hipEventSynchronize(t.stop);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, t.start, t.stop);
    g_prof_pool.push_back({t.device, t.start});
    g_prof_pool.push_back({t.device, t.stop});
    if (e != hipSuccess) {
      if (first == hipSuccess) first = e;
      continue;
    }
    tot += ms;
    ++n;
  }
  g_prof_pending.swap(keep);
  *total_ms = tot;
  *launches = n;
  return check_hip(first, "cpab_profile_read");
}

static int check_interp(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                        const int64_t* out_size) {
  if (ndim < 1 || ndim > 3) return fail(CPAB_ERR_INVALID, "interpolation supports ndim 1, 2, 3, got %d", ndim);
  CPAB_REQUIRE(in_size); CPAB_REQUIRE(out_size);
  if (B < 0 || C < 0) return fail(CPAB_ERR_INVALID, "negative batch or channel count");
  int64_t n = 1, plane = 1;
  for (int k = 0; k < ndim; ++k) {
    if (in_size[k] < 1) return fail(CPAB_ERR_INVALID, "input size %d must be >= 1", k);
    if (out_size[k] < 0) return fail(CPAB_ERR_INVALID, "output size %d must be >= 0", k);
    if (out_size[k] >= (1LL << 31) || in_size[k] >= (1LL << 31)) return fail(CPAB_ERR_INVALID, "size too large");
    // checked per axis, so that the products cannot overflow
    if (out_size[k] > 0 && n > ((1LL << 40) - 1) / out_size[k]) return fail(CPAB_ERR_INVALID, "problem too large");
    n *= out_size[k];
    plane *= in_size[k];
    // the gathers address one channel with 32-bit byte offsets
    if (plane > (1LL << 30)) return fail(CPAB_ERR_INVALID, "one data channel must hold at most 2^30 values");
  }
  const int64_t lim = (1LL << 40) - 1, c1 = C > 0 ? C : 1;
  if (n > 0 && (B > lim / n || B * n > lim / c1)) return fail(CPAB_ERR_INVALID, "problem too large");
  if (ndim >= 2) {
    // one workgroup per tile, 1D grid (fewer than 2^31 threads)
    const int64_t tiles = div_up(out_size[0], cpab::kInterpTile0) *
                          div_up(out_size[ndim - 1], cpab::kInterpTileLast) * B *
                          (ndim == 3 ? out_size[1] : 1);
    if (tiles * cpab::kInterpThreads >= (1LL << 31))
      return fail(CPAB_ERR_INVALID, "output too large for one launch");
  }
  return CPAB_OK;
}

int cpab_interp_forward(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                        const int64_t* out_size, const float* data, const float* grid, float* out,
                        void* stream) {
  int rc = check_interp(ndim, B, C, in_size, out_size);
  if (rc) return rc;
  CPAB_REQUIRE(data); CPAB_REQUIRE(grid); CPAB_REQUIRE(out);
  hipEvent_t ev = nullptr;
  const bool timed = prof_begin(as_stream(stream), &ev);
  rc = check_hip(cpab::launch_interp_forward(ndim, B, C, in_size, out_size, data, grid, out,
                                             as_stream(stream)),
                 "cpab_interp_forward");
  prof_end(timed, ev, "interp_forward", as_stream(stream));
  return rc;
}

int cpab_interp_backward(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                         const int64_t* out_size, const float* data, const float* grid,
                         const float* grad_out, float* grad_grid, float* grad_data,
                         void* stream) {
  int rc = check_interp(ndim, B, C, in_size, out_size);
  if (rc) return rc;
  CPAB_REQUIRE(data); CPAB_REQUIRE(grid); CPAB_REQUIRE(grad_out);
  hipEvent_t ev = nullptr;
  const bool timed = prof_begin(as_stream(stream), &ev);
  rc = check_hip(cpab::launch_interp_backward(ndim, B, C, in_size, out_size, data, grid,
                                              grad_out, grad_grid, grad_data, as_stream(stream)),
                 "cpab_interp_backward");
  prof_end(timed, ev, "interp_backward", as_stream(stream));
  return rc;
}

int64_t cpab_interp_backward_workspace_size(int ndim, int64_t B, int64_t C,
                                            const int64_t* in_size) {
  if (!t_deterministic || ndim < 1 || ndim > 3 || B <= 0 || C <= 0 || !in_size) return 0;
  int64_t plane = 1;
  for (int k = 0; k < ndim; ++k) {
    if (in_size[k] <= 0) return 0;
    plane *= in_size[k];
  }
  return data_workspace(0, B, C, plane).total;
}

int cpab_interp_backward_ws(int ndim, int64_t B, int64_t C, const int64_t* in_size,
                            const int64_t* out_size, const float* data, const float* grid,
                            const float* grad_out, float* grad_grid, float* grad_data,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  if (!t_deterministic || grad_data == nullptr)
    return cpab_interp_backward(ndim, B, C, in_size, out_size, data, grid, grad_out, grad_grid,
                                grad_data, stream);
  int rc = check_interp(ndim, B, C, in_size, out_size);
  if (rc) return rc;
  CPAB_REQUIRE(data); CPAB_REQUIRE(grid); CPAB_REQUIRE(grad_out);
  CPAB_ALIGNED(workspace, 16);
  if (B == 0 || C == 0) return CPAB_OK;
  int64_t plane = 1, nP = 1;
  for (int k = 0; k < ndim; ++k) {
    plane *= in_size[k];
    nP *= out_size[k];
  }
  // the deterministic scatter indexes a batch row's points with 32-bit ints
  // and takes one grid row per batch row
  if (nP >= (1LL << 31) || B >= 65536)
    return fail(CPAB_ERR_INVALID, "the deterministic grad_data takes fewer than 2^31 output "
                "points per batch row and fewer than 65536 batch rows, got %lld and %lld",
                (long long)nP, (long long)B);
  const DataWorkspace dw = data_workspace(0, B, C, plane);
  if (workspace == nullptr || workspace_bytes < dw.total)
    return fail(CPAB_ERR_INVALID,
                "workspace too small: need %lld bytes (cpab_interp_backward_workspace_size), got "
                "%lld", (long long)dw.total, (long long)workspace_bytes);
  hipStream_t s = as_stream(stream);
  const char* who = "cpab_interp_backward_ws";
  char* ws = static_cast<char*>(workspace);
  auto* gstat = reinterpret_cast<unsigned*>(ws + dw.gstat_offset);
  auto* gsums = reinterpret_cast<unsigned long long*>(ws + dw.gsums_offset);
  hipEvent_t ev = nullptr;
  const bool timed = prof_begin(s, &ev);
  // grad_grid from the gather kernel without its scatter; grad_data from the
  // deterministic scatter
  if (grad_grid)
    rc = check_hip(cpab::launch_interp_backward(ndim, B, C, in_size, out_size, data, grid,
                                                grad_out, grad_grid, nullptr, s),
                   who);
  if (rc == CPAB_OK)
    rc = check_hip(cpab::launch_fill(grad_data, B * C * plane, 0.0f, s), who);
  if (rc == CPAB_OK)
    rc = check_hip(cpab::launch_fill(reinterpret_cast<float*>(ws), dw.total / 4, 0.0f, s), who);
  if (rc == CPAB_OK)
    rc = check_hip(cpab::launch_det_interp_data(ndim, B, C, in_size, out_size, grid, grad_out,
                                                gstat, gsums, grad_data, s),
                   who);
  prof_end(timed, ev, "interp_backward", s);
  return rc;
}

}  // extern "C"
