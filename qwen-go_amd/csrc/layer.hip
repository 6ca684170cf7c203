// layer.hip -- the C ABI (include/qmoe.h): handle, weight upload and the
// forward orchestration of the MoE block on one gfx950 device.
//
// Forward (model/moe.go:41-99 for T tokens at once):
//   1. router: certified partials S/B per (token, expert) for T <= 32 (which
//      also zero out), else the exact sequential logits + softmax/selection
//      (router.hip)
//   2. experts: one fused kernel -- routing, gate_up + SwiGLU, transposed down
//      rows, f32 atomics into out (fused.hip); a shared expert stored in
//      another format gets a second launch of the same kernel
// All kernels run on one stream; the host-pointer entry copies x in and out
// around them and synchronises, as the cgo seam needs.
//
// Device layouts: router and gate_up as in the reference (rows along H); the
// down matrices (routed and shared) are stored transposed, (I, H) per expert,
// so that a block's 32 intermediate rows are one contiguous region.  Codes and
// scales are moved, never recomputed, so dequantisation stays bit-exact.
#include "../../include/qmoe.h"
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

using namespace qmoe;

namespace {

thread_local std::string g_create_error = "no error";

struct DevBuf {
  void *p = nullptr;
  size_t n = 0;
};

// Device scratch of one forward: router logits / partials, routing, and the
// batched path's tables and intermediate rows.  Either the handle's own
// workspace (grown with hipMalloc) or the static scratch array of
// qmoe_forward_device_noalloc.
struct Workspace {
  float *logits = nullptr, *wts = nullptr;
  double *sb = nullptr;
  int *fbl = nullptr;      // {count, tokens} for the exact routing path
  float *qlt = nullptr;    // (kExactQueueMax, E) exact logits of queued tokens (batched certified routing)
  uint32_t *qcnt = nullptr;  // (kExactQueueMax) workgroups done per queued token
  int32_t *ids = nullptr;
  // batched (MFMA) path buffers
  uint16_t *xb = nullptr, *act = nullptr;
  float *sg = nullptr;
  uint16_t *y = nullptr;
  PrefillPlan plan{};
  float *xn = nullptr;  // (T, H) normed x of the residual entries
};

}  // namespace

struct qmoe_layer {
  qmoe_desc d{};
  int scope = 0;
  int n_cu = 256;  // compute units of the device
  std::mutex mu;
  std::string err = "no error";
  bool destroyed = false;
  hipStream_t stream = nullptr;
  std::vector<DevBuf> owned;
  int64_t weight_bytes = 0;

  DevMat router, gu, dn, sgate, sup, sdown;
  // down matrices in the reference layout (E, H, I) and (H, Is) as well, for
  // the batched path (present when it supports the formats)
  DevMat dnr, sdownr;
  bool has_ref_down = false;
  // the shared expert's gate and up rows for the batched path when they are
  // kept in another format there (an f32 shared expert: bf16 copies)
  DevMat sgate_b, sup_b;
  bool shared_b = false;
  float *shared_gate = nullptr;
  bool has_router = false, has_experts = false, has_shared = false;

  // workspace, sized for ws_T tokens (the batched path's buffers present when ws_mfma)
  int ws_T = 0;
  DevBuf ws;
  Workspace w;
  float *xbuf = nullptr, *obuf = nullptr;
  bool ws_mfma = false;
  // this device's copy of the static scratch array (qmoe_forward_device_noalloc)
  unsigned char *scratch = nullptr;
  // [0] tokens routed by the exact fallback, [1] certification rescues,
  // [2] tokens whose norm recomputed its sum of squares in index order
  unsigned int *fallbacks = nullptr;
  // post-attention GemmaRMSNorm of the residual entries (qmoe_set_post_norm)
  float *norm_w = nullptr;
  float norm_eps = 0.0f;
  bool has_norm = false, norm_force_seq = false;
  // decode (T = 1): the expert kernel computes the router partials itself and
  // exchanges them between its workgroups as tagged words (one per expert)
  uint64_t *rtag = nullptr;
  uint32_t rtag_epoch = 0;            // tag of the last call, 1..255
  int *xchg_err_host = nullptr;       // host-visible flag: an exchange timed out
  int *xchg_err_dev = nullptr;
  uint64_t xchg_ticks = kExchangeTicks;  // wait budget of the exchange (qmoe_debug_exchange_budget)
  int xchg_resident = -1;             // the expert kernel's launch fits the device at once (-1: not yet known)

  // optional per-stage event timing (qmoe_profile_*)
  uint32_t prof_mask = 0;
  std::vector<hipEvent_t> ev_pool;
  size_t ev_used = 0;
  struct Rec {
    int stage;
    hipEvent_t a, b;
  };
  std::vector<Rec> recs;
  double prof_ms[QMOE_STAGE_COUNT] = {};
  int64_t prof_calls[QMOE_STAGE_COUNT] = {};
};

namespace qmoe {
thread_local ProfEvents g_prof;
}

// Scratch of the no-allocation entry (qmoe_forward_device_noalloc):
// decode-sized forwards (T <= 32 tokens) only -- router partials (T, E, 2)
// f64, logits (T, E) f32, ids and weights (T, k), the exact-path queue --
// for E <= 1024 and k <= 64.  Each device holds its own copy of the array
// until the process ends; every call on one device shares it.  Host code
// never uses the array's name as an address: its device address comes from
// hipGetSymbolAddress, once per device (scratch_address).
constexpr size_t kScratchBytes = (size_t)1 << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

qmoe_status fail(qmoe_layer *l, qmoe_status s, const std::string &msg) {
  if (l) l->err = msg;
  else g_create_error = msg;
  return s;
}

qmoe_status hip_fail(qmoe_layer *l, hipError_t e, const char *what) {
  return fail(l, QMOE_ERR_HIP, std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

#define HIP_TRY(l, expr, what)                    \
  do {                                            \
    hipError_t _e = (expr);                       \
    if (_e != hipSuccess) return hip_fail(l, _e, what); \
  } while (0)

bool valid_fmt(int f) { return f >= QMOE_F32 && f <= QMOE_INT4G32_F32S; }
// The group-32 formats with the reference's f32 scales are stored as their
// exact f32 dequantisation (float32(code) * scale, model/moe.go:134-157).
bool fmt_f32s(int f) { return f == QMOE_INT8G32_F32S || f == QMOE_INT4G32_F32S; }
int storage_fmt(int f) { return fmt_f32s(f) ? kF32 : f; }

// Allocates a (n_mat x rows x cols) stack in fmt plus its scales.
qmoe_status alloc_mat(qmoe_layer *l, DevMat &m, int fmt, int64_t n_mat, int rows, int cols,
                      bool transposed = false) {
  m.fmt = fmt;
  m.rows = rows;
  m.cols = cols;
  m.transposed = transposed;
  m.mat_bytes = fmt_matrix_bytes(fmt, rows, cols);
  m.mat_scales = fmt_quant(fmt) ? (int64_t)rows * (cols / kGroup) : 0;
  DevBuf b;
  b.n = (size_t)(m.mat_bytes * n_mat);
  if (hipMalloc(&b.p, b.n) != hipSuccess) {
    (void)hipGetLastError();
    return fail(l, QMOE_ERR_NOMEM, "hipMalloc of " + std::to_string(b.n) + " weight bytes failed");
  }
  l->owned.push_back(b);
  l->weight_bytes += (int64_t)b.n;
  m.w = (const uint8_t *)b.p;
  m.s = nullptr;
  if (m.mat_scales) {
    DevBuf sb;
    sb.n = (size_t)(m.mat_scales * n_mat) * sizeof(uint16_t);
    if (hipMalloc(&sb.p, sb.n) != hipSuccess) {
      (void)hipGetLastError();
      return fail(l, QMOE_ERR_NOMEM, "hipMalloc of " + std::to_string(sb.n) + " scale bytes failed");
    }
    l->owned.push_back(sb);
    l->weight_bytes += (int64_t)sb.n;
    m.s = (const uint16_t *)sb.p;
  }
  return QMOE_OK;
}

void free_all(qmoe_layer *l) {
  for (auto e : l->ev_pool) (void)hipEventDestroy(e);
  l->ev_pool.clear();
  l->recs.clear();
  l->ev_used = 0;
  for (auto &b : l->owned)
    if (b.p) (void)hipFree(b.p);
  l->owned.clear();
  if (l->ws.p) (void)hipFree(l->ws.p);
  l->ws = DevBuf{};
  l->ws_T = 0;
  if (l->stream) (void)hipStreamDestroy(l->stream);
  l->stream = nullptr;
  if (l->xchg_err_host) (void)hipHostFree(l->xchg_err_host);
  l->xchg_err_host = l->xchg_err_dev = nullptr;
}

// Moves n stored matrices in the reference layout from device staging into
// m (at matrix index first), transposing when m is stored transposed; a copy
// in the reference layout also goes into twin, when given -- in m's format,
// or, for an f32 m, rounded to bf16 (the batched path's copy of an f32 shared
// expert).
qmoe_status place(qmoe_layer *l, const DevMat &m, int64_t first, int64_t n, const uint8_t *src, const uint16_t *ss,
                  const DevMat *twin = nullptr) {
  uint8_t *dst = (uint8_t *)m.w + first * m.mat_bytes;
  uint16_t *ds = m.s ? (uint16_t *)m.s + first * m.mat_scales : nullptr;
  if (twin && twin->fmt == m.fmt) {
    HIP_TRY(l, hipMemcpyAsync((uint8_t *)twin->w + first * twin->mat_bytes, src, (size_t)(twin->mat_bytes * n),
                              hipMemcpyDeviceToDevice, l->stream), "copy");
    if (twin->s)
      HIP_TRY(l, hipMemcpyAsync((uint16_t *)twin->s + first * twin->mat_scales, ss, (size_t)(twin->mat_scales * n) * 2,
                                hipMemcpyDeviceToDevice, l->stream), "copy");
  } else if (twin) {
    if (m.fmt != kF32 || twin->fmt != kBF16) return fail(l, QMOE_ERR_UNSUPPORTED, "no conversion for this copy");
    HIP_TRY(l, launch_f32_to_bf16(reinterpret_cast<const float *>(src),
                                  (uint16_t *)(twin->w + first * twin->mat_bytes), n * m.rows * m.cols, l->stream),
            "bf16 copy launch");
  }
  if (m.transposed) {
    HIP_TRY(l, launch_relayout_transpose(m.fmt, src, ss, n, m.rows, m.cols, dst, ds, l->stream), "relayout launch");
  } else {
    HIP_TRY(l, hipMemcpyAsync(dst, src, (size_t)(m.mat_bytes * n), hipMemcpyDeviceToDevice, l->stream), "copy");
    if (ds)
      HIP_TRY(l, hipMemcpyAsync(ds, ss, (size_t)(m.mat_scales * n) * 2, hipMemcpyDeviceToDevice, l->stream), "copy");
  }
  HIP_TRY(l, hipStreamSynchronize(l->stream), "hipStreamSynchronize");
  return QMOE_OK;
}

// Uploads n_mat (rows, cols) matrices given in the ABI format in_fmt into m
// (and twin, see place): the storage format itself, or a group-32 format with
// f32 scales, which the device dequantises exactly into m's f32 storage.
qmoe_status upload(qmoe_layer *l, const DevMat &m, int in_fmt, int64_t n_mat, const void *w, const void *s,
                   const DevMat *twin = nullptr) {
  if (!w) return fail(l, QMOE_ERR_INVALID, "null weight pointer");
  const bool f32s = fmt_f32s(in_fmt);
  if ((fmt_quant(m.fmt) || f32s) && !s) return fail(l, QMOE_ERR_INVALID, "null scale pointer for a quantised format");
  if (!m.transposed && !twin && !f32s) {
    HIP_TRY(l, hipMemcpy((void *)m.w, w, (size_t)(m.mat_bytes * n_mat), hipMemcpyHostToDevice), "weight upload");
    if (fmt_quant(m.fmt))
      HIP_TRY(l, hipMemcpy((void *)m.s, s, (size_t)(m.mat_scales * n_mat) * sizeof(uint16_t), hipMemcpyHostToDevice),
              "scale upload");
    return QMOE_OK;
  }
  // staged through the device, at most ~256 MiB of input at a time
  const int bits = in_fmt == QMOE_INT8G32_F32S ? 8 : 4;
  const int64_t in_bytes = f32s ? fmt_matrix_bytes(bits == 8 ? kINT8 : kINT4, m.rows, m.cols) : m.mat_bytes;
  const int64_t in_sc = f32s ? (int64_t)m.rows * (m.cols / kGroup) * 4 : m.mat_scales * 2;
  const int64_t per = in_bytes + in_sc + (f32s ? m.mat_bytes : 0);
  const int64_t chunk = std::min<int64_t>(n_mat, std::max<int64_t>(1, (256ll << 20) / per));
  uint8_t *tmp = nullptr;
  HIP_TRY(l, hipMalloc(&tmp, (size_t)(chunk * per)), "hipMalloc upload staging");
  uint8_t *tsc = tmp + chunk * in_bytes;
  uint8_t *texp = tsc + chunk * in_sc;  // f32 dequantisation (f32s)
  qmoe_status st = QMOE_OK;
  for (int64_t e0 = 0; e0 < n_mat && st == QMOE_OK; e0 += chunk) {
    const int64_t n = std::min(chunk, n_mat - e0);
    hipError_t e = hipMemcpy(tmp, (const uint8_t *)w + e0 * in_bytes, (size_t)(n * in_bytes), hipMemcpyHostToDevice);
    if (e == hipSuccess && in_sc)
      e = hipMemcpy(tsc, (const uint8_t *)s + e0 * in_sc, (size_t)(n * in_sc), hipMemcpyHostToDevice);
    if (e == hipSuccess && f32s)
      e = launch_dequant_f32s(bits, tmp, reinterpret_cast<const float *>(tsc), n * m.rows, m.cols,
                              reinterpret_cast<float *>(texp), l->stream);
    if (e != hipSuccess) {
      st = hip_fail(l, e, "weight upload");
      break;
    }
    st = f32s ? place(l, m, e0, n, texp, nullptr, twin) : place(l, m, e0, n, tmp, (const uint16_t *)tsc, twin);
  }
  (void)hipFree(tmp);
  return st;
}

qmoe_status enter(qmoe_layer *l) {
  if (!l) return QMOE_ERR_INVALID;
  if (l->destroyed) return fail(l, QMOE_ERR_STATE, "handle used after qmoe_destroy");
  HIP_TRY(l, hipSetDevice(l->d.device), "hipSetDevice");
  return QMOE_OK;
}

hipError_t next_event(qmoe_layer *l, hipEvent_t *ev) {
  if (l->ev_used == l->ev_pool.size()) {
    hipEvent_t e;
    hipError_t r = hipEventCreate(&e);
    if (r != hipSuccess) return r;
    l->ev_pool.push_back(e);
  }
  *ev = l->ev_pool[l->ev_used++];
  return hipSuccess;
}

// Records an event pair around one kernel launch on its own stream when the
// stage is selected by qmoe_profile_enable.
#define STAGE(l, sid, st, expr, what)                                         \
  do {                                                                        \
    hipEvent_t _a = nullptr, _b = nullptr;                                    \
    const bool _on = ((l)->prof_mask >> (sid)) & 1u;                          \
    if (_on) {                                                                \
      HIP_TRY(l, next_event(l, &_a), "hipEventCreate");                       \
      HIP_TRY(l, next_event(l, &_b), "hipEventCreate");                       \
      g_prof = ProfEvents{_a, _b};                                            \
    }                                                                         \
    const hipError_t _se = (expr);                                            \
    g_prof = ProfEvents{};                                                    \
    if (_se != hipSuccess) return hip_fail(l, _se, what);                     \
    if (_on) (l)->recs.push_back({(sid), _a, _b});                            \
  } while (0)

size_t align_up(size_t v) { return (v + 255) & ~(size_t)255; }

// This device's address of the scratch array (the device must be current).
// Looked up once per device and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char *g_scratch_dev[kMaxDevices] = {};

hipError_t scratch_address(int dev, unsigned char **out) {
  *out = nullptr;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_dev[dev] = static_cast<unsigned char *>(p);
  }
  *out = g_scratch_dev[dev];
  return hipSuccess;
}

// The decode-path workspace of T tokens laid out in the scratch array at
// base; *bytes receives its size.
Workspace scratch_workspace(unsigned char *base, int T, int E, int k, size_t *bytes) {
  size_t off = 0;
  auto take = [&](size_t n) { size_t o = off; off += align_up(n); return base + o; };
  Workspace w;
  w.sb = reinterpret_cast<double *>(take((size_t)T * E * 16));
  w.logits = reinterpret_cast<float *>(take((size_t)T * E * 4));
  w.ids = reinterpret_cast<int32_t *>(take((size_t)T * k * 4));
  w.wts = reinterpret_cast<float *>(take((size_t)T * k * 4));
  w.fbl = reinterpret_cast<int *>(take((size_t)(T + 1) * 4));
  *bytes = off;
  return w;
}

// An exchange timeout of the decode kernel leaves the call's output
// untrustworthy.  The synchronous entry reports it for the call that hit it;
// an asynchronous call's timeout is reported by the next call on the handle.
// Either way the flag is cleared once reported.
qmoe_status take_exchange_error(qmoe_layer *l, const char *which) {
  if (!*l->xchg_err_host) return QMOE_OK;
  *l->xchg_err_host = 0;
  return fail(l, QMOE_ERR_HIP, std::string(which) +
                                   ": the decode kernel's workgroups timed out exchanging router partials (not all "
                                   "of them ran at once); that call's output and routing are not valid");
}

// Token counts above this run the batched MFMA path when its formats allow.
constexpr int kMaxGemvTokens = 32;
// Tokens x experts from which the batched routing uses the matrix-core
// partials (the exact router's cost grows with T * E * H on the VALU).
constexpr int64_t kCertManyMin = (int64_t)1 << 20;

bool use_mfma(const qmoe_layer *l, int T) {
  const qmoe_desc &d = l->d;
  return T > kMaxGemvTokens && l->has_ref_down && prefill_supported(l->gu.fmt, d.hidden, d.moe_inter, d.shared_inter);
}

qmoe_status ensure_workspace(qmoe_layer *l, int T, hipStream_t user_stream) {
  const bool mfma = use_mfma(l, T);
  if (T <= l->ws_T && (!mfma || l->ws_mfma)) return QMOE_OK;
  const qmoe_desc &d = l->d;
  int nT = std::max(std::max(T, l->ws_T), 64);
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t o = off; off += align_up(bytes); return o; };
  size_t o_logits = take((size_t)nT * d.n_experts * 4);
  size_t o_ids = take((size_t)nT * d.top_k * 4);
  size_t o_wts = take((size_t)nT * d.top_k * 4);
  size_t o_x = take((size_t)nT * d.hidden * 4);
  size_t o_o = take((size_t)nT * d.hidden * 4);
  size_t o_sb = take((size_t)nT * d.n_experts * 16);
  size_t o_fbl = take((size_t)(nT + 1) * 4);      // tokens queued for the exact routing path
  size_t o_qlt = take((size_t)kExactQueueMax * d.n_experts * 4);
  size_t o_qcnt = take((size_t)kExactQueueMax * 4);
  size_t o_xn = take((size_t)nT * d.hidden * 4);  // normed x (residual entries)
  const bool want_mfma = mfma || l->ws_mfma;
  const size_t pairs = (size_t)nT * d.top_k, slots = pairs + (size_t)nT;
  const int bm = prefill_tile_slots(l->gu.fmt);
  const int bms = d.shared_inter > 0 ? prefill_tile_slots(l->sdownr.fmt) : bm;
  const size_t tiles = (size_t)prefill_max_tiles(nT, d.top_k, d.n_experts, bm) + (nT + bms - 1) / bms;
  const int imax = std::max(d.moe_inter, d.shared_inter);
  size_t o_xb = 0, o_sg = 0, o_tok = 0, o_wsl = 0, o_slot = 0, o_goff = 0, o_gcnt = 0, o_cur = 0, o_tg = 0, o_tm = 0,
         o_nt = 0, o_act = 0, o_y = 0;
  if (want_mfma) {
    o_xb = take((size_t)nT * d.hidden * 2);
    o_sg = take((size_t)nT * 4);
    o_tok = take(slots * 4);
    o_wsl = take(slots * 4);
    o_slot = take(pairs * 4);
    o_goff = take((size_t)(d.n_experts + 1) * 4);
    o_gcnt = take((size_t)(d.n_experts + 1) * 4);
    o_cur = take((size_t)(d.n_experts + 1) * 4);
    o_tg = take(tiles * 4);
    o_tm = take(tiles * 4);
    o_nt = take(2 * 4);
    o_act = take(slots * imax * 2);
    o_y = take(slots * d.hidden * 2);
  }
  // Pending work of earlier calls may still read the old workspace.
  if (user_stream) HIP_TRY(l, hipStreamSynchronize(user_stream), "hipStreamSynchronize");
  HIP_TRY(l, hipStreamSynchronize(l->stream), "hipStreamSynchronize");
  if (l->ws.p) (void)hipFree(l->ws.p);
  l->ws = DevBuf{};
  l->ws_T = 0;
  if (hipMalloc(&l->ws.p, off) != hipSuccess) {
    (void)hipGetLastError();
    l->ws.p = nullptr;
    return fail(l, QMOE_ERR_NOMEM, "hipMalloc of " + std::to_string(off) + " workspace bytes failed");
  }
  l->ws.n = off;
  char *b = (char *)l->ws.p;
  Workspace &w = l->w;
  w = Workspace{};
  w.logits = (float *)(b + o_logits);
  w.ids = (int32_t *)(b + o_ids);
  w.wts = (float *)(b + o_wts);
  l->xbuf = (float *)(b + o_x);
  l->obuf = (float *)(b + o_o);
  w.sb = (double *)(b + o_sb);
  w.fbl = (int *)(b + o_fbl);
  w.qlt = (float *)(b + o_qlt);
  w.qcnt = (uint32_t *)(b + o_qcnt);
  w.xn = (float *)(b + o_xn);
  l->ws_mfma = want_mfma;
  if (want_mfma) {
    w.xb = (uint16_t *)(b + o_xb);
    w.sg = (float *)(b + o_sg);
    w.plan.tok = (int32_t *)(b + o_tok);
    w.plan.wslot = (float *)(b + o_wsl);
    w.plan.slot_of = (int32_t *)(b + o_slot);
    w.plan.grp_off = (int32_t *)(b + o_goff);
    w.plan.grp_cnt = (int32_t *)(b + o_gcnt);
    w.plan.cursor = (int32_t *)(b + o_cur);
    w.plan.tile_grp = (int32_t *)(b + o_tg);
    w.plan.tile_m0 = (int32_t *)(b + o_tm);
    w.plan.n_tiles = (int32_t *)(b + o_nt);
    w.act = (uint16_t *)(b + o_act);
    w.y = (uint16_t *)(b + o_y);
  }
  l->ws_T = nT;
  return QMOE_OK;
}

// T = 1 with a bf16 router of at most 4 chunks per lane: the expert kernel
// computes the router partials itself (no router launch) and initialises out.
// Its workgroups exchange those partials, so every one of them must be
// resident at once (checked once per handle with the occupancy calculator).
bool fused_router_ok(qmoe_layer *l, int T) {
  const qmoe_desc &d = l->d;
  const int H = d.hidden, E = d.n_experts, I = d.moe_inter, Is = d.shared_inter, k = d.top_k;
  if (use_mfma(l, T)) return false;
  const int rcpl = (H / 8 + 63) / 64;
  const bool fused_router = T == 1 && l->router.fmt == kBF16 && H % 8 == 0 && (rcpl == 1 || rcpl == 2 || rcpl == 4) &&
                            E <= 7 * l->n_cu && fused_supported(l->gu.fmt, H, E);
  if (fused_router && l->xchg_resident < 0) {
    FusedArgs q{};
    q.T = 1;
    q.H = H;
    q.E = E;
    q.I = I;
    q.Is = Is;
    q.fmt = l->gu.fmt;
    q.k_routed = k;
    q.with_shared = Is > 0 && l->sgate.fmt == l->gu.fmt;
    q.n_cu = l->n_cu;
    int resident = 0;
    const int blocks = fused_exchange_blocks(q, &resident);
    (void)hipGetLastError();
    l->xchg_resident = blocks <= resident && blocks <= kMaxExchangeBlocks && E <= 7 * blocks ? 1 : 0;
  }
  return fused_router && l->xchg_resident == 1;
}

// The kernels of one forward of T tokens on stream st, with scratch from ws.
// profile = false records no events (the no-allocation entry).  resid: the
// residual stream (T, H) out starts from instead of zero (may be out itself).
// norm: d_x is that residual stream and the block's input is its post-attention
// norm -- computed in the decode kernel's prologue on the T = 1 exchange path,
// else by the norm kernel into ws.xn first; the kernels then read only the
// normed x, so out may alias resid.
qmoe_status run_forward(qmoe_layer *l, const Workspace &ws, const float *d_x, int T, float *d_out, int32_t *d_ids,
                        float *d_w, hipStream_t st, bool profile = true, const float *resid = nullptr,
                        bool norm = false) {
  const qmoe_desc &d = l->d;
  if (!l->has_router || !l->has_experts || (d.shared_inter > 0 && !l->has_shared))
    return fail(l, QMOE_ERR_STATE, "weights not uploaded (router, experts and shared expert are required)");
  int32_t *ids = d_ids ? d_ids : ws.ids;
  float *wts = d_w ? d_w : ws.wts;
  const uint32_t prof_mask_saved = l->prof_mask;
  if (!profile) l->prof_mask = 0;
  struct Restore {
    qmoe_layer *l;
    uint32_t m;
    ~Restore() { l->prof_mask = m; }
  } restore{l, prof_mask_saved};
  const int H = d.hidden, E = d.n_experts, k = d.top_k, I = d.moe_inter, Is = d.shared_inter;
  // Where the norm runs: in the decode kernel's prologue (T = 1 exchange
  // path), in the certified router kernel (T <= 32; it stores the normed
  // tokens for the expert kernel), else in a launch of its own.
  const bool mfma = use_mfma(l, T);
  const bool fused_router = !mfma && fused_router_ok(l, T);
  const bool cert = !mfma && !fused_router && T <= kMaxGemvTokens && router_certified_supported(l->router);
  RouterNorm rnorm{};
  const float *xin = d_x;  // the expert kernels' x
  if (norm && !fused_router) {
    if (cert && H % 4 == 0) {
      rnorm.w = l->norm_w;
      rnorm.eps = l->norm_eps;
      rnorm.force_seq = l->norm_force_seq ? 1 : 0;
      rnorm.redo = l->fallbacks + 2;
      rnorm.xn = ws.xn;
      xin = ws.xn;
    } else {
      STAGE(l, QMOE_STAGE_ROUTER, st,
            launch_gemma_norm(d_x, T, H, l->norm_w, l->norm_eps, ws.xn, l->fallbacks + 2, l->norm_force_seq, st),
            "norm launch");
      d_x = xin = ws.xn;
    }
    norm = false;
  }

  // routing for T > 32.  Many tokens x experts with a bf16 router: bounded
  // partials on the matrix cores, then exact logits of the candidates those
  // leave; otherwise the exact sequential logits of every expert (VALU-bound)
  // and the exact softmax and selection.
  bool x_ready = false;  // the exact router stored x in bf16 for the GEMMs
  auto route_many = [&]() -> qmoe_status {
    if ((int64_t)T * E >= kCertManyMin && router_cert_mfma_supported(l->router)) {
      STAGE(l, QMOE_STAGE_ROUTER, st, launch_router_cert_mfma(d_x, T, l->router, ws.sb, ws.fbl, ws.qcnt, st),
            "router partials launch");
      STAGE(l, QMOE_STAGE_SELECT, st,
            launch_select_candidates(d_x, T, l->router, k, l->scope, ws.sb, ids, wts, ws.fbl, ws.qlt, ws.qcnt,
                                     l->fallbacks, st),
            "candidate selection launch");
      return QMOE_OK;
    }
    x_ready = mfma;
    STAGE(l, QMOE_STAGE_ROUTER, st, launch_router_logits(d_x, T, l->router, ws.logits, mfma ? ws.xb : nullptr, st),
          "router logits launch");
    STAGE(l, QMOE_STAGE_SELECT, st, launch_softmax_select(ws.logits, T, E, k, l->scope, ids, wts, st),
          "softmax/select launch");
    return QMOE_OK;
  };

  if (mfma) {
    // batched path: exact routing, then dispatch, grouped GEMMs, combine
    if (qmoe_status rs = route_many()) return rs;
    PrefillArgs pa{};
    pa.T = T;
    pa.H = H;
    pa.E = E;
    pa.k = k;
    pa.I = I;
    pa.Is = Is;
    pa.Imax = std::max(I, Is);
    pa.fmt = l->gu.fmt;
    pa.bm = prefill_tile_slots(l->gu.fmt);
    pa.sfmt = Is > 0 ? l->sdownr.fmt : pa.fmt;
    pa.bms = prefill_tile_slots(pa.sfmt);
    pa.n_cu = l->n_cu;
    pa.xb = ws.xb;
    pa.p = ws.plan;
    pa.gu = l->gu.w;
    pa.dn = l->dnr.w;
    pa.gu_s = l->gu.s;
    pa.dn_s = l->dnr.s;
    pa.gu_bytes = l->gu.mat_bytes;
    pa.gu_scales = l->gu.mat_scales;
    pa.dn_bytes = l->dnr.mat_bytes;
    pa.dn_scales = l->dnr.mat_scales;
    if (Is > 0) {
      const DevMat &bg = l->shared_b ? l->sgate_b : l->sgate, &bu = l->shared_b ? l->sup_b : l->sup;
      pa.sgate = bg.w;
      pa.sup = bu.w;
      pa.sdown = l->sdownr.w;
      pa.sgate_s = bg.s;
      pa.sup_s = bu.s;
      pa.sdown_s = l->sdownr.s;
    }
    pa.act = ws.act;
    pa.y = ws.y;
    pa.resid = resid;
    STAGE(l, QMOE_STAGE_DISPATCH, st, launch_prefill_dispatch(pa, ids, wts, d_x, l->shared_gate, ws.sg, x_ready, st),
          "dispatch launch");
    STAGE(l, QMOE_STAGE_GATE_UP, st, launch_prefill_gate_up(pa, false, st), "gate_up launch");
    if (Is > 0)
      STAGE(l, QMOE_STAGE_SHARED_GATE_UP, st, launch_prefill_gate_up(pa, true, st), "shared gate_up launch");
    STAGE(l, QMOE_STAGE_DOWN, st, launch_prefill_down(pa, false, st), "down launch");
    if (Is > 0) STAGE(l, QMOE_STAGE_DOWN, st, launch_prefill_down(pa, true, st), "shared down launch");
    STAGE(l, QMOE_STAGE_COMBINE, st, launch_prefill_combine(pa, d_out, st), "combine launch");
    return QMOE_OK;
  }

  const int rcpl = (H / 8 + 63) / 64;  // router chunks per lane of the in-kernel partials
  if (fused_router) {
    // nothing to launch before the expert kernel
  } else if (cert) {
    STAGE(l, QMOE_STAGE_ROUTER, st, launch_router_sb(d_x, T, l->router, ws.sb, d_out, resid, rnorm, st),
          "router launch");
  } else {
    if (qmoe_status rs = route_many()) return rs;
    if (resid) HIP_TRY(l, launch_copy(resid, d_out, (int64_t)T * H, st), "residual copy launch");
    else HIP_TRY(l, launch_zero(d_out, (int64_t)T * H, st), "zero launch");
  }
  FusedArgs f{};
  f.x = xin;
  f.T = T;
  f.H = H;
  f.E = E;
  f.k = k;
  f.scope = l->scope;
  f.I = I;
  f.Is = Is;
  f.rw = l->router.w;
  f.rs = l->router.s;
  f.rfmt = l->router.fmt;
  f.sb = cert ? ws.sb : nullptr;
  f.fmt = l->gu.fmt;
  f.gu = l->gu.w;
  f.gu_s = l->gu.s;
  f.gu_bytes = l->gu.mat_bytes;
  f.gu_scales = l->gu.mat_scales;
  f.dn = l->dn.w;
  f.dn_s = l->dn.s;
  f.dn_bytes = l->dn.mat_bytes;
  f.dn_scales = l->dn.mat_scales;
  if (Is > 0) {
    f.sgate = l->sgate.w;
    f.sup = l->sup.w;
    f.sdown = l->sdown.w;
    f.sgate_s = l->sgate.s;
    f.sup_s = l->sup.s;
    f.sdown_s = l->sdown.s;
    f.shared_gate = l->shared_gate;
  }
  f.ids = ids;
  f.weights = wts;
  f.fallbacks = l->fallbacks;
  if (fused_router) {
    l->rtag_epoch = l->rtag_epoch % 255 + 1;
    f.fused_router = rcpl;
    f.rtag = l->rtag;
    f.ztag = reinterpret_cast<uint32_t *>(l->rtag + (size_t)E);
    f.epoch = l->rtag_epoch;
    f.xchg_err = l->xchg_err_dev;
    f.xchg_ticks = l->xchg_ticks;
  }
  f.out = d_out;
  f.resid = resid;
  if (norm) {  // T = 1 on the exchange path: the prologue normalises x
    f.norm_w = l->norm_w;
    f.norm_eps = l->norm_eps;
    f.norm_force_seq = l->norm_force_seq ? 1 : 0;
    f.norm_redo = l->fallbacks + 2;
  }
  f.k_routed = k;
  f.with_shared = Is > 0 && l->sgate.fmt == l->gu.fmt;
  f.n_cu = l->n_cu;
  STAGE(l, QMOE_STAGE_FUSED, st, launch_expert_fused(f, st), "fused expert launch");
  if (Is > 0 && l->sgate.fmt != l->gu.fmt) {
    // shared expert in its own format: a second launch of the same kernel
    f.fmt = l->sgate.fmt;
    f.k_routed = 0;
    f.with_shared = 1;
    f.fused_router = 0;
    f.norm_redo = nullptr;  // counted once, by the first launch
    STAGE(l, QMOE_STAGE_FUSED, st, launch_expert_fused(f, st), "fused shared-expert launch");
  }
  return QMOE_OK;
}

}  // namespace

extern "C" {

const char *qmoe_status_string(qmoe_status s) {
  switch (s) {
  case QMOE_OK: return "ok";
  case QMOE_ERR_INVALID: return "invalid argument";
  case QMOE_ERR_STATE: return "invalid state";
  case QMOE_ERR_NOMEM: return "out of device memory";
  case QMOE_ERR_HIP: return "HIP runtime error";
  case QMOE_ERR_UNSUPPORTED: return "unsupported configuration";
  }
  return "unknown status";
}

const char *qmoe_last_error(const qmoe_layer *layer) {
  if (!layer) return g_create_error.c_str();
  return layer->err.c_str();
}

qmoe_status qmoe_create(const qmoe_desc *desc, qmoe_layer **out) {
  if (!desc || !out) return fail(nullptr, QMOE_ERR_INVALID, "null desc or out pointer");
  *out = nullptr;
  const qmoe_desc d = *desc;
  if (d.hidden <= 0 || d.n_experts <= 0 || d.top_k <= 0 || d.moe_inter <= 0 || d.shared_inter < 0)
    return fail(nullptr, QMOE_ERR_INVALID, "dimensions must be positive (shared_inter >= 0)");
  if (d.top_k > d.n_experts) return fail(nullptr, QMOE_ERR_INVALID, "top_k > n_experts");
  if (d.select_scope != 0 && (d.select_scope < d.top_k || d.select_scope > d.n_experts))
    return fail(nullptr, QMOE_ERR_INVALID, "select_scope must be 0 or in [top_k, n_experts]");
  if (!valid_fmt(d.router_fmt) || !valid_fmt(d.expert_fmt) || !valid_fmt(d.shared_fmt))
    return fail(nullptr, QMOE_ERR_INVALID, "unknown weight format");
  if (d.hidden % 32 || d.moe_inter % 32 || d.shared_inter % 32)
    return fail(nullptr, QMOE_ERR_UNSUPPORTED, "hidden, moe_inter and shared_inter must be multiples of 32");
  if (d.n_experts > 1024 || d.top_k > 64)
    return fail(nullptr, QMOE_ERR_UNSUPPORTED, "n_experts > 1024 or top_k > 64");
  if (d.hidden > 16384)
    return fail(nullptr, QMOE_ERR_UNSUPPORTED, "hidden > 16384");
  if (!fused_supported(storage_fmt(d.expert_fmt), d.hidden, d.n_experts) ||
      (d.shared_inter > 0 && !fused_supported(storage_fmt(d.shared_fmt), d.hidden, d.n_experts)))
    return fail(nullptr, QMOE_ERR_UNSUPPORTED, "hidden too large for the expert kernel's LDS plan");
  int ndev = 0;
  hipError_t e = hipGetDeviceCount(&ndev);
  if (e != hipSuccess) return hip_fail(nullptr, e, "hipGetDeviceCount");
  if (d.device < 0 || d.device >= ndev) return fail(nullptr, QMOE_ERR_INVALID, "device ordinal out of range");
  e = hipSetDevice(d.device);
  if (e != hipSuccess) return hip_fail(nullptr, e, "hipSetDevice");

  unsigned char *scr = nullptr;
  e = scratch_address(d.device, &scr);
  if (e != hipSuccess) return hip_fail(nullptr, e, "hipGetSymbolAddress of the scratch array");
  qmoe_layer *l = new qmoe_layer();
  l->d = d;
  l->scratch = scr;
  {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, d.device) == hipSuccess && prop.multiProcessorCount > 0)
      l->n_cu = prop.multiProcessorCount;
  }
  l->scope = d.select_scope == 0 ? d.top_k : d.select_scope;
  e = hipStreamCreate(&l->stream);
  if (e != hipSuccess) {
    delete l;
    return hip_fail(nullptr, e, "hipStreamCreate");
  }
  qmoe_status s;
  const int H = d.hidden, E = d.n_experts, I = d.moe_inter, Is = d.shared_inter;
  const int rf = storage_fmt(d.router_fmt), ef = storage_fmt(d.expert_fmt), sf = storage_fmt(d.shared_fmt);
  if ((s = alloc_mat(l, l->router, rf, 1, E, H)) != QMOE_OK ||
      (s = alloc_mat(l, l->gu, ef, E, 2 * I, H)) != QMOE_OK ||
      (s = alloc_mat(l, l->dn, ef, E, H, I, true)) != QMOE_OK ||
      (Is > 0 && ((s = alloc_mat(l, l->sgate, sf, 1, Is, H)) != QMOE_OK ||
                  (s = alloc_mat(l, l->sup, sf, 1, Is, H)) != QMOE_OK ||
                  (s = alloc_mat(l, l->sdown, sf, 1, H, Is, true)) != QMOE_OK))) {
    g_create_error = l->err;
    free_all(l);
    delete l;
    return s;
  }
  // the batched path: experts' down in the reference layout; the shared
  // expert in the format its GEMMs take (bf16 copies of an f32 one)
  l->has_ref_down = prefill_supported(ef, H, I, Is);
  const int sbf = prefill_shared_fmt(sf);
  l->shared_b = l->has_ref_down && Is > 0 && sbf != sf;
  if (l->has_ref_down && ((s = alloc_mat(l, l->dnr, ef, E, H, I)) != QMOE_OK ||
                          (Is > 0 && (s = alloc_mat(l, l->sdownr, sbf, 1, H, Is)) != QMOE_OK) ||
                          (l->shared_b && ((s = alloc_mat(l, l->sgate_b, sbf, 1, Is, H)) != QMOE_OK ||
                                           (s = alloc_mat(l, l->sup_b, sbf, 1, Is, H)) != QMOE_OK)))) {
    g_create_error = l->err;
    free_all(l);
    delete l;
    return s;
  }
  {
    DevBuf b;
    b.n = 256;
    if (hipMalloc(&b.p, b.n) != hipSuccess || hipMemset(b.p, 0, b.n) != hipSuccess) {
      (void)hipGetLastError();
      free_all(l);
      delete l;
      return fail(nullptr, QMOE_ERR_NOMEM, "hipMalloc of the fallback counter failed");
    }
    l->owned.push_back(b);
    l->fallbacks = (unsigned int *)b.p;
  }
  {
    DevBuf b;
    b.n = (size_t)E * 8 + (size_t)kMaxExchangeBlocks * 4;  // router words (one per expert), then zero flags
    if (hipMalloc(&b.p, b.n) != hipSuccess || hipMemset(b.p, 0, b.n) != hipSuccess) {
      (void)hipGetLastError();
      free_all(l);
      delete l;
      return fail(nullptr, QMOE_ERR_NOMEM, "hipMalloc of the router exchange words failed");
    }
    l->owned.push_back(b);
    l->rtag = (uint64_t *)b.p;
    void *hp = nullptr, *dp = nullptr;
    if (hipHostMalloc(&hp, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer(&dp, hp, 0) != hipSuccess) {
      (void)hipGetLastError();
      if (hp) (void)hipHostFree(hp);
      free_all(l);
      delete l;
      return fail(nullptr, QMOE_ERR_NOMEM, "hipHostMalloc of the exchange flag failed");
    }
    l->xchg_err_host = (int *)hp;
    l->xchg_err_dev = (int *)dp;
    *l->xchg_err_host = 0;
  }
  if (Is > 0) {
    DevBuf b;
    b.n = (size_t)H * 4;
    if (hipMalloc(&b.p, b.n) != hipSuccess) {
      (void)hipGetLastError();
      free_all(l);
      delete l;
      return fail(nullptr, QMOE_ERR_NOMEM, "hipMalloc of shared gate failed");
    }
    l->owned.push_back(b);
    l->weight_bytes += (int64_t)b.n;
    l->shared_gate = (float *)b.p;
  }
  *out = l;
  return QMOE_OK;
}

void qmoe_destroy(qmoe_layer *layer) {
  if (!layer) return;
  {
    std::lock_guard<std::mutex> g(layer->mu);
    if (layer->destroyed) return;
    (void)hipSetDevice(layer->d.device);
    if (layer->stream) (void)hipStreamSynchronize(layer->stream);
    free_all(layer);
    layer->destroyed = true;
  }
  delete layer;
}

qmoe_status qmoe_set_router(qmoe_layer *l, const void *w, const void *scales) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if ((s = upload(l, l->router, l->d.router_fmt, 1, w, scales)) != QMOE_OK) return s;
  l->has_router = true;
  return QMOE_OK;
}

qmoe_status qmoe_set_experts(qmoe_layer *l, const void *gate_up, const void *gate_up_scales, const void *down,
                             const void *down_scales) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  const int E = l->d.n_experts;
  const int f = l->d.expert_fmt;
  if ((s = upload(l, l->gu, f, E, gate_up, gate_up_scales)) != QMOE_OK) return s;
  if ((s = upload(l, l->dn, f, E, down, down_scales, l->has_ref_down ? &l->dnr : nullptr)) != QMOE_OK) return s;
  l->has_experts = true;
  return QMOE_OK;
}

qmoe_status qmoe_set_shared(qmoe_layer *l, const void *gate, const void *gate_scales, const void *up,
                            const void *up_scales, const void *down, const void *down_scales,
                            const float *shared_gate) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (l->d.shared_inter <= 0) return fail(l, QMOE_ERR_STATE, "layer has no shared expert (shared_inter == 0)");
  if (!shared_gate) return fail(l, QMOE_ERR_INVALID, "null shared_gate");
  const int f = l->d.shared_fmt;
  if ((s = upload(l, l->sgate, f, 1, gate, gate_scales, l->shared_b ? &l->sgate_b : nullptr)) != QMOE_OK) return s;
  if ((s = upload(l, l->sup, f, 1, up, up_scales, l->shared_b ? &l->sup_b : nullptr)) != QMOE_OK) return s;
  if ((s = upload(l, l->sdown, f, 1, down, down_scales, l->has_ref_down ? &l->sdownr : nullptr)) != QMOE_OK) return s;
  HIP_TRY(l, hipMemcpy(l->shared_gate, shared_gate, (size_t)l->d.hidden * 4, hipMemcpyHostToDevice),
          "shared gate upload");
  l->has_shared = true;
  return QMOE_OK;
}

qmoe_status qmoe_quantize_device(int32_t bits, const float *d_w, int64_t n_mat, int32_t rows, int32_t cols,
                                 void *d_codes, uint16_t *d_scales, void *stream) {
  if ((bits != 8 && bits != 4) || !d_w || !d_codes || !d_scales || n_mat < 0 || rows < 0 || cols <= 0 ||
      cols % 32)
    return fail(nullptr, QMOE_ERR_INVALID, "qmoe_quantize_device: bad arguments");
  hipError_t e = launch_quantize(bits, d_w, n_mat * rows, cols, (uint8_t *)d_codes, d_scales,
                                 (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(nullptr, e, "quantize launch");
  return QMOE_OK;
}

qmoe_status qmoe_quantize_experts(qmoe_layer *l, const float *gate_up, const float *down) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (!gate_up || !down) return fail(l, QMOE_ERR_INVALID, "null weight pointer");
  const int bits = l->d.expert_fmt == QMOE_INT8G32 ? 8 : l->d.expert_fmt == QMOE_INT4G32 ? 4 : 0;
  if (!bits) return fail(l, QMOE_ERR_STATE, "expert format is not INT8G32 or INT4G32");
  const int E = l->d.n_experts;
  // Stage at most ~256 MiB of f32 at a time.
  for (int which = 0; which < 2; which++) {
    const DevMat &m = which == 0 ? l->gu : l->dn;
    const float *src = which == 0 ? gate_up : down;
    const int64_t per = (int64_t)m.rows * m.cols;
    int64_t chunk = std::max<int64_t>(1, (256ll << 20) / (per * 4));
    chunk = std::min<int64_t>(chunk, E);
    float *tmp = nullptr;
    HIP_TRY(l, hipMalloc(&tmp, (size_t)(chunk * (per * 4 + m.mat_bytes + m.mat_scales * 2))),
            "hipMalloc quantiser staging");
    uint8_t *qc = (uint8_t *)(tmp + chunk * per);
    uint16_t *qs = (uint16_t *)(qc + chunk * m.mat_bytes);
    for (int64_t e0 = 0; e0 < E; e0 += chunk) {
      int64_t n = std::min<int64_t>(chunk, E - e0);
      hipError_t err = hipMemcpy(tmp, src + e0 * per, (size_t)(n * per * 4), hipMemcpyHostToDevice);
      if (err == hipSuccess) err = launch_quantize(bits, tmp, n * m.rows, m.cols, qc, qs, l->stream);
      if (err != hipSuccess) {
        (void)hipFree(tmp);
        return hip_fail(l, err, "expert quantisation");
      }
      qmoe_status st = place(l, m, e0, n, qc, qs, which == 1 && l->has_ref_down ? &l->dnr : nullptr);
      if (st != QMOE_OK) {
        (void)hipFree(tmp);
        return st;
      }
    }
    (void)hipFree(tmp);
  }
  l->has_experts = true;
  return QMOE_OK;
}

// Tokens per launch sequence: the batched path's slot tables hold at most
// 65535 (token, rank) pairs, so longer batches run in chunks (each output row
// depends only on its own token, so chunking changes no result).
int chunk_tokens(const qmoe_layer *l) {
  const int c = 65535 / l->d.top_k;
  return c >= 256 ? c / 64 * 64 : c;
}

qmoe_status qmoe_forward_device(qmoe_layer *l, const float *d_x, int32_t T, float *d_out, int32_t *d_ids,
                                float *d_weights, void *stream) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (T < 0) return fail(l, QMOE_ERR_INVALID, "T < 0");
  if (T == 0) return QMOE_OK;
  if (!d_x || !d_out) return fail(l, QMOE_ERR_INVALID, "null x or out pointer");
  if ((s = take_exchange_error(l, "an earlier asynchronous forward")) != QMOE_OK) return s;
  hipStream_t st = (hipStream_t)stream;
  const int tc = chunk_tokens(l);
  const int H = l->d.hidden, k = l->d.top_k;
  if ((s = ensure_workspace(l, std::min(T, tc), st)) != QMOE_OK) return s;
  for (int t0 = 0; t0 < T; t0 += tc) {
    const int n = std::min(tc, T - t0);
    if ((s = run_forward(l, l->w, d_x + (size_t)t0 * H, n, d_out + (size_t)t0 * H,
                         d_ids ? d_ids + (size_t)t0 * k : nullptr,
                         d_weights ? d_weights + (size_t)t0 * k : nullptr, st)) != QMOE_OK)
      return s;
  }
  return QMOE_OK;
}

qmoe_status qmoe_set_post_norm(qmoe_layer *l, const float *w, float eps) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (!w) return fail(l, QMOE_ERR_INVALID, "null norm weight pointer");
  const size_t n = (size_t)l->d.hidden * 4;
  if (!l->norm_w) {
    DevBuf b;
    b.n = n;
    if (hipMalloc(&b.p, b.n) != hipSuccess) {
      (void)hipGetLastError();
      return fail(l, QMOE_ERR_NOMEM, "hipMalloc of the norm weight failed");
    }
    l->owned.push_back(b);
    l->weight_bytes += (int64_t)n;
    l->norm_w = (float *)b.p;
  }
  HIP_TRY(l, hipMemcpy(l->norm_w, w, n, hipMemcpyHostToDevice), "norm weight upload");
  l->norm_eps = eps;
  l->has_norm = true;
  return QMOE_OK;
}

qmoe_status qmoe_forward_residual_device(qmoe_layer *l, const float *d_x, int32_t T, float *d_out, int32_t *d_ids,
                                         float *d_weights, void *stream) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (T < 0) return fail(l, QMOE_ERR_INVALID, "T < 0");
  if (!l->has_norm) return fail(l, QMOE_ERR_STATE, "post-attention norm not uploaded (qmoe_set_post_norm)");
  if (T == 0) return QMOE_OK;
  if (!d_x || !d_out) return fail(l, QMOE_ERR_INVALID, "null x or out pointer");
  if ((s = take_exchange_error(l, "an earlier asynchronous forward")) != QMOE_OK) return s;
  hipStream_t st = (hipStream_t)stream;
  const int tc = chunk_tokens(l);
  const int H = l->d.hidden, k = l->d.top_k;
  if ((s = ensure_workspace(l, std::min(T, tc), st)) != QMOE_OK) return s;
  for (int t0 = 0; t0 < T; t0 += tc) {
    const int n = std::min(tc, T - t0);
    const float *xr = d_x + (size_t)t0 * H;
    if ((s = run_forward(l, l->w, xr, n, d_out + (size_t)t0 * H, d_ids ? d_ids + (size_t)t0 * k : nullptr,
                         d_weights ? d_weights + (size_t)t0 * k : nullptr, st, true, xr, true)) != QMOE_OK)
      return s;
  }
  return QMOE_OK;
}

qmoe_status qmoe_forward_residual(qmoe_layer *l, float *x, int32_t T, int32_t *ids, float *weights) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (T < 0) return fail(l, QMOE_ERR_INVALID, "T < 0");
  if (!l->has_norm) return fail(l, QMOE_ERR_STATE, "post-attention norm not uploaded (qmoe_set_post_norm)");
  if (T == 0) return QMOE_OK;
  if (!x) return fail(l, QMOE_ERR_INVALID, "null x pointer");
  if ((s = take_exchange_error(l, "an earlier asynchronous forward")) != QMOE_OK) return s;
  const int tc = chunk_tokens(l);
  const int H = l->d.hidden, k = l->d.top_k;
  if ((s = ensure_workspace(l, std::min(T, tc), nullptr)) != QMOE_OK) return s;
  for (int t0 = 0; t0 < T; t0 += tc) {
    const int n = std::min(tc, T - t0);
    const size_t xb = (size_t)n * H * 4, kb = (size_t)n * k * 4;
    HIP_TRY(l, hipMemcpyAsync(l->xbuf, x + (size_t)t0 * H, xb, hipMemcpyHostToDevice, l->stream), "x upload");
    // x += block(norm(x)), in place in the staging buffer
    if ((s = run_forward(l, l->w, l->xbuf, n, l->xbuf, l->w.ids, l->w.wts, l->stream, true, l->xbuf, true)) !=
        QMOE_OK)
      return s;
    HIP_TRY(l, hipMemcpyAsync(x + (size_t)t0 * H, l->xbuf, xb, hipMemcpyDeviceToHost, l->stream), "x download");
    if (ids)
      HIP_TRY(l, hipMemcpyAsync(ids + (size_t)t0 * k, l->w.ids, kb, hipMemcpyDeviceToHost, l->stream), "ids download");
    if (weights)
      HIP_TRY(l, hipMemcpyAsync(weights + (size_t)t0 * k, l->w.wts, kb, hipMemcpyDeviceToHost, l->stream),
              "weights download");
    HIP_TRY(l, hipStreamSynchronize(l->stream), "hipStreamSynchronize");
  }
  return take_exchange_error(l, "this forward");
}

qmoe_status qmoe_norm_recomputes(qmoe_layer *l, int64_t *count) {
  if (!l || !count) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  HIP_TRY(l, hipDeviceSynchronize(), "hipDeviceSynchronize");
  unsigned int v = 0;
  HIP_TRY(l, hipMemcpy(&v, l->fallbacks + 2, sizeof(v), hipMemcpyDeviceToHost), "norm counter read");
  *count = v;
  return QMOE_OK;
}

qmoe_status qmoe_norm_debug(qmoe_layer *l, const float *x, int32_t T, float *xn) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (!l->has_norm) return fail(l, QMOE_ERR_STATE, "post-attention norm not uploaded (qmoe_set_post_norm)");
  if (T < 0 || (T > 0 && (!x || !xn))) return fail(l, QMOE_ERR_INVALID, "bad x, xn or T");
  const int H = l->d.hidden;
  for (int t0 = 0; t0 < T;) {
    const int n = std::min(T - t0, chunk_tokens(l));
    if ((s = ensure_workspace(l, n, nullptr)) != QMOE_OK) return s;
    const size_t b = (size_t)n * H * 4;
    HIP_TRY(l, hipMemcpyAsync(l->xbuf, x + (size_t)t0 * H, b, hipMemcpyHostToDevice, l->stream), "x upload");
    HIP_TRY(l, launch_gemma_norm(l->xbuf, n, H, l->norm_w, l->norm_eps, l->w.xn, l->fallbacks + 2,
                                 l->norm_force_seq, l->stream),
            "norm launch");
    HIP_TRY(l, hipMemcpyAsync(xn + (size_t)t0 * H, l->w.xn, b, hipMemcpyDeviceToHost, l->stream), "xn download");
    HIP_TRY(l, hipStreamSynchronize(l->stream), "hipStreamSynchronize");
    t0 += n;
  }
  return QMOE_OK;
}

qmoe_status qmoe_debug_norm_sequential(qmoe_layer *l, int32_t on) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  l->norm_force_seq = on != 0;
  return QMOE_OK;
}

qmoe_status qmoe_forward_device_noalloc(qmoe_layer *l, const float *d_x, int32_t T, float *d_out, int32_t *d_ids,
                                        float *d_weights, void *stream) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (T < 0) return fail(l, QMOE_ERR_INVALID, "T < 0");
  if (T == 0) return QMOE_OK;
  if (!d_x || !d_out) return fail(l, QMOE_ERR_INVALID, "null x or out pointer");
  if (T > kMaxGemvTokens)
    return fail(l, QMOE_ERR_UNSUPPORTED,
                "qmoe_forward_device_noalloc takes at most " + std::to_string(kMaxGemvTokens) + " tokens (T = " +
                    std::to_string(T) + "); use qmoe_forward_device");
  if (!l->scratch) return fail(l, QMOE_ERR_STATE, "no scratch array address for this device");
  size_t bytes = 0;
  const Workspace w = scratch_workspace(l->scratch, T, l->d.n_experts, l->d.top_k, &bytes);
  if (bytes > kScratchBytes)
    return fail(l, QMOE_ERR_UNSUPPORTED, "qmoe_forward_device_noalloc: " + std::to_string(bytes) +
                                             " scratch bytes needed, " + std::to_string(kScratchBytes) + " available");
  if ((s = take_exchange_error(l, "an earlier asynchronous forward")) != QMOE_OK) return s;
  return run_forward(l, w, d_x, T, d_out, d_ids, d_weights, (hipStream_t)stream, false);
}

qmoe_status qmoe_forward(qmoe_layer *l, const float *x, int32_t T, float *out, int32_t *ids, float *weights) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (T < 0) return fail(l, QMOE_ERR_INVALID, "T < 0");
  if (T == 0) return QMOE_OK;
  if (!x || !out) return fail(l, QMOE_ERR_INVALID, "null x or out pointer");
  if ((s = take_exchange_error(l, "an earlier asynchronous forward")) != QMOE_OK) return s;
  const int tc = chunk_tokens(l);
  const int H = l->d.hidden, k = l->d.top_k;
  if ((s = ensure_workspace(l, std::min(T, tc), nullptr)) != QMOE_OK) return s;
  for (int t0 = 0; t0 < T; t0 += tc) {
    const int n = std::min(tc, T - t0);
    const size_t xb = (size_t)n * H * 4, kb = (size_t)n * k * 4;
    HIP_TRY(l, hipMemcpyAsync(l->xbuf, x + (size_t)t0 * H, xb, hipMemcpyHostToDevice, l->stream), "x upload");
    if ((s = run_forward(l, l->w, l->xbuf, n, l->obuf, l->w.ids, l->w.wts, l->stream)) != QMOE_OK) return s;
    HIP_TRY(l, hipMemcpyAsync(out + (size_t)t0 * H, l->obuf, xb, hipMemcpyDeviceToHost, l->stream), "out download");
    if (ids)
      HIP_TRY(l, hipMemcpyAsync(ids + (size_t)t0 * k, l->w.ids, kb, hipMemcpyDeviceToHost, l->stream), "ids download");
    if (weights)
      HIP_TRY(l, hipMemcpyAsync(weights + (size_t)t0 * k, l->w.wts, kb, hipMemcpyDeviceToHost, l->stream),
              "weights download");
    // the next chunk reuses the staging buffers
    HIP_TRY(l, hipStreamSynchronize(l->stream), "hipStreamSynchronize");
  }
  return take_exchange_error(l, "this forward");
}

qmoe_status qmoe_dequant_debug(qmoe_layer *l, int32_t which, int32_t expert, float *out) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (!out) return fail(l, QMOE_ERR_INVALID, "null out pointer");
  const DevMat *m = nullptr;
  int64_t index = 0;
  switch (which) {
  case 0: m = &l->gu; index = expert; break;
  case 1: m = &l->dn; index = expert; break;
  case 2: m = &l->router; break;
  case 3: m = &l->sgate; break;
  case 4: m = &l->sup; break;
  case 5: m = &l->sdown; break;
  default: return fail(l, QMOE_ERR_INVALID, "which must be in [0, 5]");
  }
  if (which >= 3 && l->d.shared_inter <= 0) return fail(l, QMOE_ERR_STATE, "layer has no shared expert");
  if (which <= 1 && (expert < 0 || expert >= l->d.n_experts))
    return fail(l, QMOE_ERR_INVALID, "expert out of range");
  const size_t n = (size_t)m->rows * m->cols;
  float *tmp = nullptr;
  HIP_TRY(l, hipMalloc(&tmp, n * 4), "hipMalloc dequant staging");
  hipError_t e = launch_dequantize(*m, index, tmp, l->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(out, tmp, n * 4, hipMemcpyDeviceToHost, l->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(l->stream);
  (void)hipFree(tmp);
  if (e != hipSuccess) return hip_fail(l, e, "dequant_debug");
  return QMOE_OK;
}

qmoe_status qmoe_router_bounds_debug(qmoe_layer *l, const float *x, int32_t T, double *sb_out) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (!x || !sb_out || T <= 0) return fail(l, QMOE_ERR_INVALID, "null pointer or T <= 0");
  if (!l->has_router) return fail(l, QMOE_ERR_STATE, "router not uploaded");
  const bool small = T <= kMaxGemvTokens;
  if (small ? !router_certified_supported(l->router) : !router_cert_mfma_supported(l->router))
    return fail(l, QMOE_ERR_UNSUPPORTED, "no certified router for this T and router format");
  if ((s = ensure_workspace(l, T, l->stream)) != QMOE_OK) return s;
  const size_t nx = (size_t)T * l->d.hidden, nsb = (size_t)T * l->d.n_experts * 2;
  hipError_t e = hipMemcpyAsync(l->xbuf, x, nx * 4, hipMemcpyHostToDevice, l->stream);
  if (e == hipSuccess)
    e = small ? launch_router_sb(l->xbuf, T, l->router, l->w.sb, nullptr, nullptr, RouterNorm{}, l->stream)
              : launch_router_cert_mfma(l->xbuf, T, l->router, l->w.sb, nullptr, nullptr, l->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(sb_out, l->w.sb, nsb * 8, hipMemcpyDeviceToHost, l->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(l->stream);
  if (e != hipSuccess) return hip_fail(l, e, "router_bounds_debug");
  return QMOE_OK;
}

qmoe_status qmoe_profile_enable(qmoe_layer *l, uint32_t stage_mask) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  l->prof_mask = stage_mask & ((1u << QMOE_STAGE_COUNT) - 1u);
  return QMOE_OK;
}

qmoe_status qmoe_profile_read(qmoe_layer *l, double *stage_ms, int64_t *stage_launches, int32_t reset) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (!l->recs.empty()) HIP_TRY(l, hipEventSynchronize(l->recs.back().b), "hipEventSynchronize");
  for (const auto &r : l->recs) {
    float ms = 0.0f;
    HIP_TRY(l, hipEventElapsedTime(&ms, r.a, r.b), "hipEventElapsedTime");
    l->prof_ms[r.stage] += ms;
    l->prof_calls[r.stage] += 1;
  }
  l->recs.clear();
  l->ev_used = 0;
  for (int i = 0; i < QMOE_STAGE_COUNT; i++) {
    if (stage_ms) stage_ms[i] = l->prof_ms[i];
    if (stage_launches) stage_launches[i] = l->prof_calls[i];
    if (reset) {
      l->prof_ms[i] = 0.0;
      l->prof_calls[i] = 0;
    }
  }
  return QMOE_OK;
}

qmoe_status qmoe_router_fallbacks(qmoe_layer *l, int64_t *count) {
  if (!l || !count) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  HIP_TRY(l, hipDeviceSynchronize(), "hipDeviceSynchronize");
  unsigned int v = 0;
  HIP_TRY(l, hipMemcpy(&v, l->fallbacks, sizeof(v), hipMemcpyDeviceToHost), "fallback counter read");
  *count = v;
  return QMOE_OK;
}

qmoe_status qmoe_router_rescues(qmoe_layer *l, int64_t *count) {
  if (!l || !count) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  HIP_TRY(l, hipDeviceSynchronize(), "hipDeviceSynchronize");
  unsigned int v = 0;
  HIP_TRY(l, hipMemcpy(&v, l->fallbacks + 1, sizeof(v), hipMemcpyDeviceToHost), "rescue counter read");
  *count = v;
  return QMOE_OK;
}

int32_t qmoe_forward_path(const qmoe_layer *l, int32_t T) {
  if (!l) return -1;
  return use_mfma(l, T) ? QMOE_PATH_MFMA : QMOE_PATH_GEMV;
}

qmoe_status qmoe_debug_exchange_budget(qmoe_layer *l, int64_t ticks) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  l->xchg_ticks = ticks < 0 ? kExchangeTicks : (uint64_t)ticks;
  return QMOE_OK;
}

qmoe_status qmoe_reserve(qmoe_layer *l, int32_t max_T) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = enter(l);
  if (s) return s;
  if (max_T < 0) return fail(l, QMOE_ERR_INVALID, "max_T < 0");
  if (max_T == 0) return QMOE_OK;
  // the batched path's buffers are sized when that path is taken; a T that
  // takes it sizes them now (weights must be uploaded for the path choice)
  return ensure_workspace(l, std::min<int>(max_T, chunk_tokens(l)), nullptr);
}

int64_t qmoe_device_bytes(const qmoe_layer *l) {
  if (!l) return 0;
  return l->weight_bytes + (int64_t)l->ws.n;
}

}  // extern "C"
