// C ABI of the engine (include/bcjr_hip.h): validation, launch geometry,
// workspace sizing and launches on the caller's stream.  No allocation, no host
// synchronisation, no exceptions across the boundary.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>

#include "../../include/bcjr_hip.h"
#include "bcjr_device.h"
#include "bcjr_kernels.h"

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(BCJR_EHIP, "%s: %s", what, hipGetErrorString(e));
}

struct DeviceInfo {
  bool valid = false;
  int num_cu = 0;
  size_t max_lds = 0;
};

std::mutex g_dev_mu;
DeviceInfo g_dev[64];

int device_info(DeviceInfo* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= 64) return fail(BCJR_EHIP, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_dev_mu);
  if (!g_dev[dev].valid) {
    int cu = 0, lds = 0;
    e = hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(MultiprocessorCount)");
    e = hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(MaxSharedMemoryPerBlock)");
    g_dev[dev].num_cu = cu;
    g_dev[dev].max_lds = (size_t)lds;
    g_dev[dev].valid = true;
  }
  *out = g_dev[dev];
  return BCJR_OK;
}

// Launch geometry of one operation for one problem.
struct Plan {
  int KV = 0, R = 0, NSUB = 0;
  int NT = 0, NB = 0, NU = 0;
  int nthr = 0, upt = 0;
  bool cache = false;
  const void* fn = nullptr;
  size_t lds = 0;
  size_t slot_bytes = 0;
  int max_blocks = 0;  // resident blocks on the device
  bcjr::Swizzle swz = {{31, 31, 31, 31}, {0, 0, 0, 0}};
};

int validate(const bcjr_problem* p) {
  if (!p) return fail(BCJR_EINVAL, "problem is NULL");
  if (p->V != 1 && p->V != 2) return fail(BCJR_EINVAL, "V=%d must be 1 or 2", p->V);
  if (p->k < 1) return fail(BCJR_EINVAL, "k=%d must be >= 1", p->k);
  const int KV = p->k * p->V;
  if (KV != 1 && KV != 2 && KV != 4)
    return fail(BCJR_EUNSUPPORTED, "k*V=%d: only 1, 2 or 4 bits per step are built", KV);
  if (p->L < 2 * KV || p->L > 16)
    return fail(BCJR_EUNSUPPORTED, "L=%d outside [%d, 16] for k*V=%d", p->L, 2 * KV, KV);
  if (KV == 1 && p->L > 11) return fail(BCJR_EUNSUPPORTED, "k*V=1 supports L <= 11 (got %d)", p->L);
  if (KV == 1 && p->code != BCJR_CODE_TABLE)
    return fail(BCJR_EUNSUPPORTED, "k*V=1 is built for the table code only (got code %d)", p->code);
  if (p->B < 0) return fail(BCJR_EINVAL, "B=%lld must be >= 0", (long long)p->B);
  if (p->N < 1 || p->N > 4096) return fail(BCJR_EINVAL, "N=%lld outside [1, 4096]", (long long)p->N);
  switch (p->code) {
    case BCJR_CODE_TABLE: break;
    case BCJR_CODE_1MAD:
    case BCJR_CODE_3INST:
      if (p->V != 1) return fail(BCJR_EINVAL, "1MAD/3INST codes are scalar (V=1), got V=%d", p->V);
      break;
    case BCJR_CODE_HYB:
      if (p->V != 2) return fail(BCJR_EINVAL, "HYB code is 2-D (V=2), got V=%d", p->V);
      if (p->Q < 1 || p->Q > 12) return fail(BCJR_EINVAL, "HYB Q=%d outside [1, 12]", p->Q);
      break;
    default: return fail(BCJR_EINVAL, "unknown code %d", p->code);
  }
  return BCJR_OK;
}

enum { OP_FWD = BCJR_OP_FORWARD, OP_BWD = BCJR_OP_BACKWARD, OP_VIT = BCJR_OP_VITERBI, OP_FWD_INTERNALS = 3 };

// Bytes of one sequence slot of an operation's workspace (a validated problem):
// forward N * 2^(L-kV) floats (the raw alpha inputs of every step), backward
// twice that ((m~, mu) pairs), Viterbi one byte of backpointers per reduced
// state and step.  It depends on the problem only, so an undersized workspace
// is reported before any device query.
size_t slot_bytes_of(const bcjr_problem* p, int op) {
  const size_t NT = (size_t)1 << (p->L - p->k * p->V);
  size_t b = op == OP_BWD ? (size_t)p->N * 2 * NT * sizeof(float)
           : op == OP_VIT ? (size_t)p->N * NT
                          : (size_t)p->N * NT * sizeof(float);
  return (b + 255) & ~(size_t)255;
}

// Early argument checks shared by the launching entry points: the problem, then
// a workspace that holds at least one slot (BCJR_EWORKSPACE).
int check_ws(const bcjr_problem* p, int op, const void* ws, size_t ws_bytes) {
  int rc = validate(p);
  if (rc) return rc;
  if (p->B == 0) return BCJR_OK;
  if (!ws) return fail(BCJR_EINVAL, "ws must be non-NULL");
  const size_t slot = slot_bytes_of(p, op);
  if (ws_bytes < slot)
    return fail(BCJR_EWORKSPACE, "workspace of %zu bytes is smaller than one sequence slot (%zu bytes)",
                ws_bytes, slot);
  return BCJR_OK;
}

// Plans depend on (device, op, L, k, V, N, code, Q) only; they are cached so that
// steady-state calls (and calls made while a stream is being captured into a
// graph) do no attribute or occupancy queries.
struct PlanKey {
  int dev, op, L, k, V, code, Q;
  long long N;
  bool operator==(const PlanKey& o) const {
    return dev == o.dev && op == o.op && L == o.L && k == o.k && V == o.V && code == o.code &&
           Q == o.Q && N == o.N;
  }
};
constexpr int kPlanCache = 64;
std::mutex g_plan_mu;
PlanKey g_plan_keys[kPlanCache];
Plan g_plans[kPlanCache];
int g_plan_count = 0, g_plan_next = 0;

int make_plan_uncached(const bcjr_problem* p, int op, const DeviceInfo& di, Plan* pl);

int make_plan(const bcjr_problem* p, int op, Plan* pl) {
  int rc = validate(p);
  if (rc) return rc;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  const PlanKey key = {dev, op, p->L, p->k, p->V, p->code, p->code == BCJR_CODE_HYB ? p->Q : 0,
                       (long long)p->N};
  {
    std::lock_guard<std::mutex> lk(g_plan_mu);
    for (int i = 0; i < g_plan_count; ++i)
      if (g_plan_keys[i] == key) {
        *pl = g_plans[i];
        return BCJR_OK;
      }
  }
  DeviceInfo di;
  rc = device_info(&di);
  if (rc) return rc;
  rc = make_plan_uncached(p, op, di, pl);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_plan_mu);
  const int slot = g_plan_count < kPlanCache ? g_plan_count++ : (g_plan_next++ % kPlanCache);
  g_plan_keys[slot] = key;
  g_plans[slot] = *pl;
  return BCJR_OK;
}

// LDS bank conflicts of the backward kernel's in-place layout: element
// S(rotr(k*NB + u, rho)) holds slot k of butterfly u, one 8-byte (m~, mu) pair,
// read and written by the same lane.  Measured on gfx950: a 64-bit LDS read
// serves each 32-lane half of a wave from 32 eight-byte banks (conflict-free
// when the half's elements differ mod 32); a 64-bit write serves 16 lanes at a
// time from 32 four-byte banks (conflict-free when each quarter's elements
// differ mod 16).  One wave of butterflies (u = 0..63) suffices: higher bits of
// u XOR the same constant into every element of the wave.  Returns the extra
// passes summed over the rotations a sweep reaches (multiples of gcd(kV, nb))
// and the slots.
int swizzle_cost(int L, int KV, const bcjr::Swizzle& s) {
  const int nb = L - KV, NB = 1 << (nb - KV), R = 1 << KV;
  const int lanes = std::min(NB, 64);
  const uint32_t mask = (1u << nb) - 1u;
  int g = KV, h = nb;
  while (h) {
    const int r = g % h;
    g = h;
    h = r;
  }
  int cost = 0;
  uint32_t el[64];
  for (int rho = 0; rho < nb; rho += g)
    for (int k = 0; k < R; ++k) {
      for (int l = 0; l < lanes; ++l) {
        const uint32_t j = (uint32_t)(k * NB + l);
        const uint32_t x = ((j | (j << nb)) >> rho) & mask;
        uint32_t e = x;
        for (int f = 0; f < 4; ++f) e ^= (x >> s.a[f]) & s.m[f];
        el[l] = e;
      }
      for (int group = 16; group <= 32; group *= 2)  // writes: 16 mod 16; reads: 32 mod 32
        for (int l0 = 0; l0 < lanes; l0 += group) {
          int cnt[32] = {0}, worst = 0;
          for (int l = l0; l < std::min(lanes, l0 + group); ++l) worst = std::max(worst, ++cnt[el[l] % group]);
          cost += worst - 1;
        }
    }
  return cost;
}

// Cheapest swizzle: up to four fields of 4 or 5 bits at shifts >= their width,
// taken in order of increasing count and kept only when strictly better; the
// search stops at the first conflict-free layout.
bcjr::Swizzle pick_swizzle(int L, int KV) {
  const int nb = L - KV;
  bcjr::Swizzle best = {{31, 31, 31, 31}, {0, 0, 0, 0}};
  int best_cost = swizzle_cost(L, KV, best);
  for (int nf = 1; nf <= 4 && best_cost > 0; ++nf) {
    int sh[4];
    // shifts sh[0] < ... < sh[nf-1] in [4, nb), widths from the bits of wbits
    std::function<void(int, int)> rec = [&](int f, int lo) {
      if (best_cost == 0) return;
      if (f == nf) {
        for (int wbits = 0; wbits < (1 << nf) && best_cost > 0; ++wbits) {
          bcjr::Swizzle s = {{31, 31, 31, 31}, {0, 0, 0, 0}};
          bool ok = true;
          for (int i = 0; i < nf; ++i) {
            const int w = 4 + ((wbits >> i) & 1);
            if (sh[i] < w) ok = false;
            s.a[i] = sh[i];
            s.m[i] = (1u << w) - 1u;
          }
          if (!ok) continue;
          const int cost = swizzle_cost(L, KV, s);
          if (cost < best_cost) {
            best_cost = cost;
            best = s;
          }
        }
        return;
      }
      for (int a = lo; a < nb; ++a) {
        sh[f] = a;
        rec(f + 1, a + 1);
      }
    };
    rec(0, 4);
  }
  return best;
}

// State layout of the column-walk backward instance (L = 16, kV = 4), whose
// thread tid holds butterfly col_walk_unit(tid) rather than tid: with this
// swizzle every half-wave's 64-bit reads and every quarter-wave's 64-bit writes
// of S(rotr(k*NB + u, rho)) fall in distinct banks over all 256 lanes, the 16
// slots and the rotations 0, 4, 8 (the search above assumes u = tid).
constexpr bcjr::Swizzle kColWalkSwizzle = {{4, 6, 8, 31}, {3u, 31u, 15u, 0u}};

int make_plan_uncached(const bcjr_problem* p, int op, const DeviceInfo& di, Plan* pl) {
  const int KV = p->k * p->V, R = 1 << KV, RO = R < 4 ? R : 4;
  pl->KV = KV;
  pl->R = R;
  pl->NSUB = R / RO;
  pl->NT = 1 << (p->L - KV);
  pl->NB = pl->NT >> KV;
  if (op != OP_VIT) pl->NSUB = 1;  // the soft kernels take whole butterflies per unit
  pl->NU = pl->NB * pl->NSUB;
  const int max_thr = 512;
  int nthr = ((pl->NU + 63) / 64) * 64;
  nthr = std::min(nthr, max_thr);
  const int upt = (pl->NU + nthr - 1) / nthr;
  if (upt != 1 && upt != 2 && upt != 4 && upt != 8)
    return fail(BCJR_EUNSUPPORTED, "no launch shape for L=%d k*V=%d (units/thread %d)", p->L, KV, upt);
  pl->nthr = nthr;
  pl->upt = upt;
  const int nwaves = nthr / 64;
  const int N = (int)p->N;
  const int kcode = bcjr::soft_kernel_code(p->code, p->L, KV, p->Q);
  if (op == OP_FWD || op == OP_FWD_INTERNALS || op == OP_VIT) {
    const bool fwd = (op != OP_VIT);
    // The Viterbi kernel caches all of a thread's codewords in VGPRs up to 128
    // of them; the soft forward's cache is fixed per instance
    // (fwd_cached_units).
    pl->cache = !fwd && (pl->NSUB == 1) && (upt * R * R * p->V <= 128);
    int vcode = p->code;  // the Viterbi instance's code
    pl->fn = fwd ? bcjr::fwd_kernel_ptr(KV, p->V, kcode, upt, op == OP_FWD_INTERNALS)
                 : bcjr::vit_kernel_ptr(KV, p->V, p->code, upt, pl->cache, false);
    if (!fwd && pl->NU >= 1024) {
      // 1024 threads (four waves per SIMD instead of two) when an instance
      // exists: codewords cached within 64 VGPRs, or none cached (kV = 4).
      const int upt_w = pl->NU / 1024;
      const bool cache_w = (pl->NSUB == 1) && (upt_w * R * R * p->V <= 64);
      const int wcode = cache_w ? p->code : kcode;
      const void* fn_w = bcjr::vit_kernel_ptr(KV, p->V, wcode, upt_w, cache_w, true);
      // ... and its LDS fits (the HYB LUT copies of the uncached instances do
      // not beside a 2^14-state cost vector: k = 1, V = 2 at L = 16).
      if (fn_w && bcjr::vit_lds_bytes(p->L, KV, p->V, N, 16, wcode, p->Q, !cache_w) > di.max_lds) fn_w = nullptr;
      if (fn_w) {
        vcode = wcode;
        pl->fn = fn_w;
        pl->cache = cache_w;
        pl->nthr = nthr = 1024;
        pl->upt = upt_w;
      }
    }
    pl->lds = fwd ? bcjr::fwd_lds_bytes(p->L, KV, p->V, N, nwaves, kcode, p->Q)
                  : bcjr::vit_lds_bytes(p->L, KV, p->V, N, nwaves, vcode, p->Q,
                                        !pl->cache && pl->nthr == 1024);
    if (op == OP_FWD && KV == 2 && p->V == 1 && p->L >= 14 && p->code <= BCJR_CODE_3INST) {
      // Four waves per SIMD: 1024 threads, every codeword in VGPRs (bcjr_fwd4.hip).
      // Kept only where its larger LDS (N doubles and floats beside the state)
      // still fits; otherwise the 512-thread plan stands (at L = 16 it holds
      // N = 2704, the 1024-thread kernel N = 2702).
      const int upt4 = 1 << (p->L - 14);
      const void* fn4 = bcjr::fwd4_kernel_ptr(p->code, upt4);
      if (fn4 && bcjr::fwd4_lds_bytes(p->L, N) <= di.max_lds) {
        pl->fn = fn4;
        pl->nthr = nthr = 1024;
        pl->upt = upt4;
        pl->lds = bcjr::fwd4_lds_bytes(p->L, N);
      }
    }
    pl->slot_bytes = slot_bytes_of(p, fwd ? OP_FWD : OP_VIT);
  } else {
    pl->cache = false;
    pl->swz = kcode == bcjr::CODE_HYB_COL ? kColWalkSwizzle : pick_swizzle(p->L, KV);
    pl->fn = bcjr::bwd_kernel_ptr(KV, p->V, kcode, upt);
    pl->lds = bcjr::bwd_lds_bytes(p->L, KV, p->V, N, nwaves, kcode, p->Q);
    pl->slot_bytes = slot_bytes_of(p, OP_BWD);
  }
  if (!pl->fn)
    return fail(BCJR_EUNSUPPORTED, "no kernel built for L=%d k=%d V=%d code=%d (units/thread %d)",
                p->L, p->k, p->V, p->code, upt);
  if (pl->lds > di.max_lds)
    return fail(BCJR_EUNSUPPORTED, "needs %zu bytes of LDS per workgroup (device limit %zu); reduce N=%lld",
                pl->lds, di.max_lds, (long long)p->N);
  hipError_t e = hipFuncSetAttribute(pl->fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl->lds);
  if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, pl->fn, nthr, pl->lds);
  if (e != hipSuccess) return hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor");
  if (per_cu < 1) return fail(BCJR_EUNSUPPORTED, "kernel cannot be resident (%d threads, %zu B LDS)", nthr, pl->lds);
  pl->max_blocks = per_cu * di.num_cu;
  return BCJR_OK;
}

int launch(const Plan& pl, long long B, size_t ws_bytes, void* params, hipStream_t stream) {
  if (B == 0) return BCJR_OK;
  long long slots = (long long)(ws_bytes / pl.slot_bytes);
  if (slots < 1)
    return fail(BCJR_EWORKSPACE, "workspace of %zu bytes is smaller than one sequence slot (%zu bytes)",
                ws_bytes, pl.slot_bytes);
  const long long grid = std::min<long long>(std::min<long long>(B, pl.max_blocks), slots);
  void* args[] = {params};
  hipError_t e = hipLaunchKernel(pl.fn, dim3((unsigned)grid), dim3((unsigned)pl.nthr), args, pl.lds, stream);
  if (e != hipSuccess) return hip_fail(e, "hipLaunchKernel");
  e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "kernel launch");
  return BCJR_OK;
}

}  // namespace

// Sequence slots of bcjr_forward_noalloc: a static device array, one copy per
// GPU.  Host code never names it after set-up: its host-side symbol is only a
// stand-in, so the device address comes from hipGetSymbolAddress, once per
// device with that device current, and is kept per device.
static __device__ __align__(256) unsigned char scratch[BCJR_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[64];

int scratch_ptr(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= 64) return fail(BCJR_EHIP, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(BCJR_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return BCJR_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int rht_impl(const float* W, float* out, int64_t batch, int64_t m, int64_t n, const float* sign_l,
             const float* sign_r, int inverse, hipStream_t stream) {
  if (batch < 0 || batch > INT32_MAX) return fail(BCJR_EINVAL, "batch=%lld outside [0, 2^31)", (long long)batch);
  if (m < 1 || m > 16384 || (m & (m - 1)))
    return fail(BCJR_EINVAL, "m=%lld must be a power of two in [1, 16384]", (long long)m);
  if (n < 1 || n > 16384 || (n & (n - 1)))
    return fail(BCJR_EINVAL, "n=%lld must be a power of two in [1, 16384]", (long long)n);
  if (batch == 0) return BCJR_OK;
  if (!W || !out || !sign_l || !sign_r) return fail(BCJR_EINVAL, "W, out, sign_l and sign_r must be non-NULL");
  const size_t bytes = (size_t)batch * m * n * sizeof(float);
  const char *w0 = reinterpret_cast<const char*>(W), *o0 = reinterpret_cast<const char*>(out);
  if (w0 < o0 + bytes && o0 < w0 + bytes) return fail(BCJR_EINVAL, "out must not alias W");
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc) return rc;
  const float s = (float)(1.0 / sqrt((double)m * (double)n));
  const int blocks = di.num_cu * 8;
  const long long rows = batch * m;
  // forward: rows of W diag(sr) H_n, then row signs, then H_m and the scale;
  // inverse: rows of W H_n then diag(sr), then H_m, row signs and the scale.
  if (n >= 64 && aligned16(W) && aligned16(sign_r)) {  // tiled kernels: 2 passes over HBM for most shapes
    hipError_t e = inverse
        ? bcjr::launch_fwht_tiled(W, out, (int)batch, (int)m, (int)n, true, nullptr, sign_r, nullptr, sign_l, s,
                                  di.num_cu * 4, stream)
        : bcjr::launch_fwht_tiled(W, out, (int)batch, (int)m, (int)n, true, sign_r, nullptr, sign_l, nullptr, s,
                                  di.num_cu * 4, stream);
    return e == hipSuccess ? BCJR_OK : hip_fail(e, "bcjr_rht tiled passes");
  }
  hipError_t e =
      inverse ? bcjr::launch_fwht_rows(W, out, rows, (int)n, nullptr, sign_r, m, nullptr, 1.0f, blocks, stream)
              : bcjr::launch_fwht_rows(W, out, rows, (int)n, sign_r, nullptr, m, sign_l, 1.0f, blocks, stream);
  if (e != hipSuccess) return hip_fail(e, "bcjr_rht row pass");
  e = bcjr::launch_fwht_cols(out, (int)batch, (int)m, (int)n, inverse ? sign_l : nullptr, s, blocks, stream);
  return e == hipSuccess ? BCJR_OK : hip_fail(e, "bcjr_rht column pass");
}

}  // namespace

extern "C" {

int bcjr_workspace_bytes(const bcjr_problem* prob, int op, size_t* bytes) {
  if (!bytes) return fail(BCJR_EINVAL, "bytes is NULL");
  if (op != OP_FWD && op != OP_BWD && op != OP_VIT) return fail(BCJR_EINVAL, "unknown op %d", op);
  Plan pl;
  int rc = make_plan(prob, op, &pl);
  if (rc) return rc;
  const long long slots = std::max<long long>(1, std::min<long long>(prob->B, pl.max_blocks));
  *bytes = (size_t)slots * pl.slot_bytes;
  return BCJR_OK;
}

int bcjr_forward(const bcjr_problem* prob, const float* seq, const float* T, const float* codebook_or_lut,
                 float* soft, float* logZ, void* ws, size_t ws_bytes, hipStream_t stream) {
  int rc0 = check_ws(prob, OP_FWD, ws, ws_bytes);
  if (rc0 || prob->B == 0) return rc0;
  if (!seq || !T || !soft || !ws) return fail(BCJR_EINVAL, "seq, T, soft and ws must be non-NULL");
  if (prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  Plan pl;
  int rc = make_plan(prob, OP_FWD, &pl);
  if (rc) return rc;
  bcjr::FwdParams P = {};
  P.seq = seq;
  P.T = T;
  P.table = codebook_or_lut;
  P.soft = soft;
  P.logZ = logZ;
  P.ws = static_cast<float*>(ws);
  P.B = prob->B;
  P.N = (int)prob->N;
  P.L = prob->L;
  P.Q = prob->Q;
  P.t_per_seq = prob->t_per_seq ? 1 : 0;
  return launch(pl, prob->B, ws_bytes, &P, stream);
}

int bcjr_forward_noalloc(const bcjr_problem* prob, const float* seq, const float* T, const float* codebook_or_lut,
                         float* soft, float* logZ, hipStream_t stream) {
  int rc = validate(prob);
  if (rc || prob->B == 0) return rc;
  const size_t slot = slot_bytes_of(prob, OP_FWD);
  if (slot > BCJR_NOALLOC_SCRATCH_BYTES)
    return fail(BCJR_EWORKSPACE,
                "one sequence slot needs %zu bytes (N=%lld, L=%d, k*V=%d); the static scratch holds %zu",
                slot, (long long)prob->N, prob->L, prob->k * prob->V, (size_t)BCJR_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = scratch_ptr(&ws);
  if (rc) return rc;
  return bcjr_forward(prob, seq, T, codebook_or_lut, soft, logZ, ws, BCJR_NOALLOC_SCRATCH_BYTES, stream);
}

int bcjr_forward_internals(const bcjr_problem* prob, const float* seq, const float* T,
                           const float* codebook_or_lut, float* soft, float* logZ, float* marginals,
                           float* log_alpha, float* log_beta, void* ws, size_t ws_bytes, hipStream_t stream) {
  int rc0 = check_ws(prob, OP_FWD, ws, ws_bytes);
  if (rc0 || prob->B == 0) return rc0;
  if (!seq || !T || !soft || !ws || !marginals || !log_alpha || !log_beta)
    return fail(BCJR_EINVAL, "seq, T, soft, ws, marginals, log_alpha and log_beta must be non-NULL");
  if (prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  Plan pl;
  int rc = make_plan(prob, OP_FWD_INTERNALS, &pl);
  if (rc) return rc;
  bcjr::FwdParams P = {};
  P.seq = seq;
  P.T = T;
  P.table = codebook_or_lut;
  P.soft = soft;
  P.logZ = logZ;
  P.ws = static_cast<float*>(ws);
  P.P_out = marginals;
  P.la_out = log_alpha;
  P.lb_out = log_beta;
  P.B = prob->B;
  P.N = (int)prob->N;
  P.L = prob->L;
  P.Q = prob->Q;
  P.t_per_seq = prob->t_per_seq ? 1 : 0;
  return launch(pl, prob->B, ws_bytes, &P, stream);
}

int bcjr_forward_entropy(const bcjr_problem* prob, const float* seq, const float* T,
                         const float* codebook_or_lut, float* soft, float* logZ, float* entropy, void* ws,
                         size_t ws_bytes, hipStream_t stream) {
  int rc0 = check_ws(prob, OP_FWD, ws, ws_bytes);
  if (rc0 || prob->B == 0) return rc0;
  if (!seq || !T || !soft || !ws || !entropy)
    return fail(BCJR_EINVAL, "seq, T, soft, ws and entropy must be non-NULL");
  if (prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  Plan pl;
  int rc = make_plan(prob, OP_FWD_INTERNALS, &pl);
  if (rc) return rc;
  bcjr::FwdParams P = {};
  P.seq = seq;
  P.T = T;
  P.table = codebook_or_lut;
  P.soft = soft;
  P.logZ = logZ;
  P.ws = static_cast<float*>(ws);
  P.H_out = entropy;
  P.B = prob->B;
  P.N = (int)prob->N;
  P.L = prob->L;
  P.Q = prob->Q;
  P.t_per_seq = prob->t_per_seq ? 1 : 0;
  return launch(pl, prob->B, ws_bytes, &P, stream);
}

int bcjr_backward(const bcjr_problem* prob, const float* seq, const float* T, const float* codebook_or_lut,
                  const float* logZ, const float* g_soft, const float* g_logZ, float* g_seq, void* ws,
                  size_t ws_bytes, hipStream_t stream) {
  (void)logZ;
  int rc0 = check_ws(prob, OP_BWD, ws, ws_bytes);
  if (rc0 || prob->B == 0) return rc0;
  if (!seq || !T || !g_soft || !g_seq || !ws)
    return fail(BCJR_EINVAL, "seq, T, g_soft, g_seq and ws must be non-NULL");
  if (prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  Plan pl;
  int rc = make_plan(prob, OP_BWD, &pl);
  if (rc) return rc;
  bcjr::BwdParams P = {};
  P.seq = seq;
  P.T = T;
  P.table = codebook_or_lut;
  P.g_soft = g_soft;
  P.g_logZ = g_logZ;
  P.g_seq = g_seq;
  P.ws = static_cast<float*>(ws);
  P.B = prob->B;
  P.N = (int)prob->N;
  P.L = prob->L;
  P.Q = prob->Q;
  P.t_per_seq = prob->t_per_seq ? 1 : 0;
  P.swz = pl.swz;
  return launch(pl, prob->B, ws_bytes, &P, stream);
}

int bcjr_viterbi(const bcjr_problem* prob, const float* seq, const float* codebook_or_lut, int32_t* walk,
                 int32_t* bitstream, int32_t* start_state, float* recon, float* mse, uint8_t* packed, void* ws,
                 size_t ws_bytes, hipStream_t stream) {
  int rc0 = check_ws(prob, OP_VIT, ws, ws_bytes);
  if (rc0 || prob->B == 0) return rc0;
  if (!seq || !ws) return fail(BCJR_EINVAL, "seq and ws must be non-NULL");
  if (prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  if (packed && 8 % (prob->k * prob->V) != 0) return fail(BCJR_EINVAL, "packing needs k*V to divide 8");
  Plan pl;
  int rc = make_plan(prob, OP_VIT, &pl);
  if (rc) return rc;
  bcjr::VitParams P = {};
  P.seq = seq;
  P.table = codebook_or_lut;
  P.walk = walk;
  P.bits = bitstream;
  P.start = start_state;
  P.recon = recon;
  P.mse = mse;
  P.packed = packed;
  P.ws = static_cast<uint8_t*>(ws);
  P.B = prob->B;
  P.N = (int)prob->N;
  P.L = prob->L;
  P.Q = prob->Q;
  return launch(pl, prob->B, ws_bytes, &P, stream);
}

int bcjr_viterbi_constrained(const bcjr_problem* prob, const float* seq, const float* codebook_or_lut,
                             int overlap_bits, const int32_t* overlap, int32_t* walk, int32_t* bitstream,
                             int32_t* start_state, float* recon, float* mse, uint8_t* packed, void* ws,
                             size_t ws_bytes, hipStream_t stream) {
  int rc0 = check_ws(prob, OP_VIT, ws, ws_bytes);
  if (rc0 || prob->B == 0) return rc0;
  if (overlap_bits < 0 || overlap_bits > prob->L - prob->k * prob->V)
    return fail(BCJR_EINVAL, "overlap_bits=%d must lie in [0, L - k*V] = [0, %d]", overlap_bits,
                prob->L - prob->k * prob->V);
  if (!seq || !ws || !overlap) return fail(BCJR_EINVAL, "seq, overlap and ws must be non-NULL");
  if (prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  if (packed && 8 % (prob->k * prob->V) != 0) return fail(BCJR_EINVAL, "packing needs k*V to divide 8");
  Plan pl;
  int rc = make_plan(prob, OP_VIT, &pl);
  if (rc) return rc;
  bcjr::VitParams P = {};
  P.seq = seq;
  P.table = codebook_or_lut;
  P.walk = walk;
  P.bits = bitstream;
  P.start = start_state;
  P.recon = recon;
  P.mse = mse;
  P.packed = packed;
  P.ws = static_cast<uint8_t*>(ws);
  P.overlap = overlap;
  P.overlap_bits = overlap_bits;
  P.B = prob->B;
  P.N = (int)prob->N;
  P.L = prob->L;
  P.Q = prob->Q;
  return launch(pl, prob->B, ws_bytes, &P, stream);
}

int bcjr_decode(const bcjr_problem* prob, const int32_t* bitstream, const uint8_t* packed,
                const int32_t* start_state, const float* codebook_or_lut, int32_t* walk, float* recon,
                hipStream_t stream) {
  int rc = validate(prob);
  if (rc) return rc;
  if (prob->B == 0) return BCJR_OK;
  if ((!bitstream && !packed) || !start_state)
    return fail(BCJR_EINVAL, "need start_state and one of bitstream / packed");
  if (recon && prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  const int KV = prob->k * prob->V;
  const void* fn = bcjr::decode_kernel_ptr(KV, prob->V, prob->code);
  if (!fn) return fail(BCJR_EUNSUPPORTED, "no decode kernel for k*V=%d V=%d code=%d", KV, prob->V, prob->code);
  bcjr::DecParams P = {bitstream, packed, start_state, codebook_or_lut, walk, recon,
                       prob->B, (int)prob->N, prob->L, prob->Q};
  void* args[] = {&P};
  const unsigned grid = (unsigned)((prob->B + 255) / 256);
  hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(256), args, 0, stream);
  if (e != hipSuccess) return hip_fail(e, "hipLaunchKernel(decode)");
  return BCJR_OK;
}

int bcjr_viterbi_trace(const bcjr_problem* prob, const float* seq, const float* codebook_or_lut, float* trace,
                       int32_t* backptr, hipStream_t stream) {
  int rc = validate(prob);
  if (rc) return rc;
  if (prob->B == 0) return BCJR_OK;
  if (!seq || !trace || !backptr) return fail(BCJR_EINVAL, "seq, trace and backptr must be non-NULL");
  if (prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  const int KV = prob->k * prob->V;
  const void* fn = bcjr::trace_kernel_ptr(KV, prob->V, prob->code);
  if (!fn) return fail(BCJR_EUNSUPPORTED, "no trace kernel for k*V=%d V=%d code=%d", KV, prob->V, prob->code);
  DeviceInfo di;
  rc = device_info(&di);
  if (rc) return rc;
  // The reduced vector and its argmin: NT floats + NT bytes (NT <= 2^14 for a
  // validated problem, so at most 16 reduced indices per thread of 1024).
  const int NT = 1 << (prob->L - KV);
  const int nthr = NT < 64 ? 64 : (NT > 1024 ? 1024 : NT);
  const size_t lds = (size_t)NT * (sizeof(float) + 1);
  if (lds > di.max_lds)
    return fail(BCJR_EUNSUPPORTED, "viterbi trace needs %zu bytes of LDS per workgroup (device limit %zu)", lds,
                di.max_lds);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(MaxDynamicSharedMemorySize)");
  const long long cap = (long long)di.num_cu * 2;
  const unsigned grid = (unsigned)(prob->B < cap ? prob->B : cap);
  bcjr::TraceParams P = {seq, codebook_or_lut, trace, backptr, prob->B, (int)prob->N, prob->L, prob->Q};
  void* args[] = {&P};
  e = hipLaunchKernel(fn, dim3(grid), dim3(nthr), args, lds, stream);
  if (e != hipSuccess) return hip_fail(e, "hipLaunchKernel(viterbi_trace)");
  return BCJR_OK;
}

static_assert(bcjr::BITS_FMT_U8 == BCJR_BITS_U8 && bcjr::BITS_FMT_I32 == BCJR_BITS_I32 &&
                  bcjr::BITS_FMT_PACKED == BCJR_BITS_PACKED,
              "bitstream layout ids");

int bcjr_dequant(const bcjr_problem* prob, const void* bitstream, int bits_format,
                 const int32_t* start_state, const float* codebook_or_lut, int64_t m, int64_t n, int Tx,
                 int Ty, double scale, float* out, hipStream_t stream) {
  int rc = validate(prob);
  if (rc) return rc;
  if (Tx < 1 || Ty < 1) return fail(BCJR_EINVAL, "tile %dx%d must be positive", Tx, Ty);
  if (m < 0 || n < 0 || m % Tx || n % Ty)
    return fail(BCJR_EINVAL, "matrix %lldx%lld is not a whole number of %dx%d tiles", (long long)m,
                (long long)n, Tx, Ty);
  if ((long long)Tx * Ty != prob->N * prob->V)
    return fail(BCJR_EINVAL, "tile %dx%d holds %lld weights, sequences N*V=%lld", Tx, Ty,
                (long long)Tx * Ty, (long long)(prob->N * prob->V));
  if (prob->B != (m / Tx) * (n / Ty))
    return fail(BCJR_EINVAL, "B=%lld but the matrix has %lld tiles", (long long)prob->B,
                (long long)((m / Tx) * (n / Ty)));
  if (bits_format != BCJR_BITS_U8 && bits_format != BCJR_BITS_I32 && bits_format != BCJR_BITS_PACKED)
    return fail(BCJR_EINVAL, "unknown bitstream format %d", bits_format);
  if (prob->B == 0) return BCJR_OK;
  if (!bitstream || !start_state || !out) return fail(BCJR_EINVAL, "bitstream, start_state and out are required");
  if (prob->code != BCJR_CODE_1MAD && prob->code != BCJR_CODE_3INST && !codebook_or_lut)
    return fail(BCJR_EINVAL, "code %d needs a codebook/LUT pointer", prob->code);
  const int KV = prob->k * prob->V;
  const bool out16 = (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  // 16x16 tiles at k = 2: one thread per tile row, aligned vector loads of its bits.
  const size_t bits_align = bits_format == BCJR_BITS_PACKED ? 4 : 16;
  const bool t16 = Tx == 16 && Ty == 16 && prob->k == 2 && (m * n) / 4 < (1ll << 31) && out16 &&
                   (reinterpret_cast<uintptr_t>(bitstream) % bits_align) == 0;
  // Vector path: 4 columns of one tile row per thread, 16-byte stores, 32-bit indices.
  const bool vec4 = !t16 && Ty % 4 == 0 && (m * n) / 4 < (1ll << 31) && out16;
  const void* fn = t16 ? bcjr::dequant_t16_kernel_ptr(KV, prob->V, prob->code, bits_format)
                       : bcjr::dequant_kernel_ptr(KV, prob->V, prob->code, vec4);
  if (!fn) return fail(BCJR_EUNSUPPORTED, "no dequant kernel for k*V=%d V=%d code=%d", KV, prob->V, prob->code);
  auto log2_or_neg = [](int x) { return (x < 1 || (x & (x - 1))) ? -1 : __builtin_ctz((unsigned)x); };
  bcjr::DqParams P = {bits_format == BCJR_BITS_I32 ? static_cast<const int32_t*>(bitstream) : nullptr,
                      bits_format == BCJR_BITS_U8 ? static_cast<const uint8_t*>(bitstream) : nullptr,
                      bits_format == BCJR_BITS_PACKED ? static_cast<const uint8_t*>(bitstream) : nullptr,
                      start_state, codebook_or_lut, out, m, n, (int)prob->N, prob->L, prob->Q, Tx, Ty,
                      log2_or_neg(Tx), log2_or_neg(Ty), (double)(float)scale == scale ? 1 : 0, scale};
  void* args[] = {&P};
  // t16: one workgroup per 16-row x 64-column unit; others: one thread per 4 or 1 elements
  const long long blocks = t16 ? (m / 16) * ((n / 4 + 15) / 16) : (vec4 ? m * n / 4 + 255 : m * n + 255) / 256;
  long long cap = 16384;
  size_t lds = 0;
  if (t16 && prob->code == BCJR_CODE_HYB) {  // LUT staged in LDS: persistent grid
    DeviceInfo di;
    int rc2 = device_info(&di);
    if (rc2) return rc2;
    cap = (long long)di.num_cu * 8;
    lds = (size_t)(2 << prob->Q) * sizeof(float);
  }
  const unsigned grid = (unsigned)(blocks < cap ? blocks : cap);
  hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(256), args, lds, stream);
  if (e != hipSuccess) return hip_fail(e, "hipLaunchKernel(dequant)");
  return BCJR_OK;
}

int bcjr_codebook(const bcjr_problem* prob, const float* lut, float* codebook_out, hipStream_t stream) {
  if (!prob) return fail(BCJR_EINVAL, "problem is NULL");
  if (prob->L < 1 || prob->L > 24) return fail(BCJR_EINVAL, "L=%d outside [1, 24]", prob->L);
  if (!codebook_out) return fail(BCJR_EINVAL, "codebook_out is NULL");
  const void* fn = bcjr::codebook_kernel_ptr(prob->code);
  if (!fn) return fail(BCJR_EINVAL, "code %d has no generator", prob->code);
  if (prob->code == BCJR_CODE_HYB && (!lut || prob->Q < 1 || prob->Q > 12))
    return fail(BCJR_EINVAL, "HYB needs a LUT and Q in [1, 12]");
  bcjr::CbParams P = {lut, codebook_out, 1ll << prob->L, prob->Q};
  void* args[] = {&P};
  const unsigned grid = (unsigned)((P.S + 255) / 256);
  hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(256), args, 0, stream);
  if (e != hipSuccess) return hip_fail(e, "hipLaunchKernel(codebook)");
  return BCJR_OK;
}

int bcjr_hadamard(const float* x, float* out, int64_t rows, int64_t n, float scale, hipStream_t stream) {
  if (rows < 0) return fail(BCJR_EINVAL, "rows=%lld must be >= 0", (long long)rows);
  if (n < 1 || n > 16384 || (n & (n - 1)))
    return fail(BCJR_EINVAL, "n=%lld must be a power of two in [1, 16384]", (long long)n);
  if (rows == 0) return BCJR_OK;
  if (!x || !out) return fail(BCJR_EINVAL, "x and out must be non-NULL");
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc) return rc;
  hipError_t e;
  if (n >= 64 && rows <= INT32_MAX && aligned16(x))
    e = bcjr::launch_fwht_tiled(x, out, 1, (int)rows, (int)n, false, nullptr, nullptr, nullptr, nullptr, scale,
                                di.num_cu * 4, stream);
  else
    e = bcjr::launch_fwht_rows(x, out, rows, (int)n, nullptr, nullptr, rows, nullptr, scale, di.num_cu * 8, stream);
  return e == hipSuccess ? BCJR_OK : hip_fail(e, "bcjr_hadamard launch");
}


int bcjr_rht(const float* W, float* out, int64_t m, int64_t n, const float* sign_l, const float* sign_r,
             int inverse, hipStream_t stream) {
  return rht_impl(W, out, 1, m, n, sign_l, sign_r, inverse, stream);
}

int bcjr_rht_batched(const float* W, float* out, int64_t batch, int64_t m, int64_t n, const float* sign_l,
                     const float* sign_r, int inverse, hipStream_t stream) {
  return rht_impl(W, out, batch, m, n, sign_l, sign_r, inverse, stream);
}

const char* bcjr_strerror(int status) {
  switch (status) {
    case BCJR_OK: return "ok";
    case BCJR_EINVAL: return "invalid argument";
    case BCJR_EUNSUPPORTED: return "unsupported configuration";
    case BCJR_EWORKSPACE: return "workspace too small";
    case BCJR_EHIP: return "HIP runtime error";
    default: return "unknown status";
  }
}

const char* bcjr_last_error(void) { return g_last_error.c_str(); }

const char* bcjr_version(void) { return "bcjr_hip 0.1.0 (gfx950)"; }

}  // extern "C"
