// dense.hip -- the C ABI of the dense projection (qmoe_linear_* in
// include/qmoe.h): one weight matrix resident on the device, the exact GEMV of
// linear.hip over it, and the greedy token of the LM head.
//
// Replaces linear.matvec / mat2D / proj (model/model.go:131-205),
// quantLinear.forward (model/moe.go:159-162) and, for the LM head, the
// matvec + argmax of model.go:519-525, 582, 652-660.
#include "../../include/qmoe.h"
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <mutex>
#include <string>

using namespace qmoe;

namespace {

thread_local std::string g_lin_create_error = "no error";

}  // namespace

struct qmoe_linear {
  int out_dim = 0, in_dim = 0, fmt = 0, device = 0;
  int n_cu = 256;
  std::mutex mu;
  std::string err = "no error";
  bool has_w = false;
  hipStream_t stream = nullptr;
  LinMat m;  // the lane stream (linear.hip)
  void *wbuf = nullptr;
  // workspace: x and logits of the host-pointer calls, argmax pairs
  void *ws = nullptr;
  size_t ws_n = 0;
  int64_t weight_bytes = 0;
};

namespace {

qmoe_status lfail(qmoe_linear *l, qmoe_status s, const std::string &msg) {
  if (l) l->err = msg;
  else g_lin_create_error = msg;
  return s;
}

qmoe_status lhip(qmoe_linear *l, hipError_t e, const char *what) {
  return lfail(l, QMOE_ERR_HIP, std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

#define LHIP_TRY(l, expr, what)                       \
  do {                                                \
    hipError_t _e = (expr);                           \
    if (_e != hipSuccess) return lhip(l, _e, what);   \
  } while (0)

bool lin_f32s(int f) { return f == QMOE_INT8G32_F32S || f == QMOE_INT4G32_F32S; }

qmoe_status lenter(qmoe_linear *l) {
  if (!l) return QMOE_ERR_INVALID;
  LHIP_TRY(l, hipSetDevice(l->device), "hipSetDevice");
  if (!l->has_w) return lfail(l, QMOE_ERR_STATE, "weights not uploaded (qmoe_linear_set)");
  return QMOE_OK;
}

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace for T tokens: x (T, in), logits (T, out), argmax pairs and the
// T token ids.
struct LinWs {
  float *x, *y, *pv;
  int *pi;
  int32_t *tok;
};

qmoe_status lin_workspace(qmoe_linear *l, int T, bool need_xy, int n_argmax, LinWs *w) {
  const size_t xb = need_xy ? al256((size_t)T * l->in_dim * 4) : 0;
  const size_t yb = need_xy ? al256((size_t)T * l->out_dim * 4) : 0;
  const size_t pairs = n_argmax ? (size_t)T * argmax_partials(n_argmax) : 0;
  const size_t pb = al256(pairs * 4);
  const size_t tb = n_argmax ? al256((size_t)T * 4) : 0;
  const size_t need = xb + yb + 2 * pb + tb;
  if (need > l->ws_n) {
    // the old workspace may still be in use on a caller's stream
    LHIP_TRY(l, hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (l->ws) (void)hipFree(l->ws);
    l->ws = nullptr;
    l->ws_n = 0;
    if (hipMalloc(&l->ws, need) != hipSuccess) {
      (void)hipGetLastError();
      return lfail(l, QMOE_ERR_NOMEM, "hipMalloc of " + std::to_string(need) + " workspace bytes failed");
    }
    l->ws_n = need;
  }
  unsigned char *p = (unsigned char *)l->ws;
  w->x = (float *)p;
  w->y = (float *)(p + xb);
  w->pv = (float *)(p + xb + yb);
  w->pi = (int *)(p + xb + yb + pb);
  w->tok = (int32_t *)(p + xb + yb + 2 * pb);
  return QMOE_OK;
}

qmoe_status check_T(qmoe_linear *l, int T) {
  if (T < 0) return lfail(l, QMOE_ERR_INVALID, "T < 0");
  if ((int64_t)T * l->out_dim > INT32_MAX || (int64_t)T * l->in_dim > INT32_MAX)
    return lfail(l, QMOE_ERR_UNSUPPORTED, "T * dim exceeds 2^31 elements");
  const int tt = linear_tokens_per_pass(T, l->in_dim);
  if (T > 0 && (T + tt - 1) / tt > 65535)
    return lfail(l, QMOE_ERR_UNSUPPORTED, "T above " + std::to_string(65535 * tt) + " for this in_dim");
  return QMOE_OK;
}

}  // namespace

extern "C" {

qmoe_status qmoe_linear_create(int32_t out_dim, int32_t in_dim, int32_t fmt, int32_t device, qmoe_linear **out) {
  if (!out) return lfail(nullptr, QMOE_ERR_INVALID, "null output handle pointer");
  *out = nullptr;
  if (out_dim <= 0 || in_dim <= 0) return lfail(nullptr, QMOE_ERR_INVALID, "dimensions must be positive");
  if (fmt < QMOE_F32 || fmt > QMOE_INT4G32_F32S) return lfail(nullptr, QMOE_ERR_INVALID, "unknown format");
  const int sf = fmt;  // every format is kept as given (group-32: codes + their scales)
  if ((fmt_quant(fmt) || lin_f32s(fmt)) && in_dim % kGroup)
    return lfail(nullptr, QMOE_ERR_INVALID, "quantised formats need in_dim % 32 == 0");
  if (!linear_supported(sf, in_dim))
    return lfail(nullptr, QMOE_ERR_UNSUPPORTED, "in_dim must be a multiple of " + std::to_string(linear_step(sf)) +
                                                    " for this format and at most 40960");
  if ((int64_t)out_dim * in_dim > ((int64_t)1 << 40)) return lfail(nullptr, QMOE_ERR_UNSUPPORTED, "matrix too large");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
    (void)hipGetLastError();
    return lfail(nullptr, QMOE_ERR_INVALID, "no such HIP device: " + std::to_string(device));
  }
  qmoe_linear *l = new qmoe_linear;
  l->out_dim = out_dim;
  l->in_dim = in_dim;
  l->fmt = fmt;
  l->device = device;
  auto bail = [&](qmoe_status s) {
    g_lin_create_error = l->err;
    qmoe_linear_destroy(l);
    return s;
  };
  if (hipSetDevice(device) != hipSuccess) return bail(lhip(l, hipGetLastError(), "hipSetDevice"));
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) l->n_cu = prop.multiProcessorCount;
  hipError_t e = hipStreamCreateWithFlags(&l->stream, hipStreamNonBlocking);
  if (e != hipSuccess) return bail(lhip(l, e, "hipStreamCreate"));
  LinMat &m = l->m;
  m.n_cu = l->n_cu;
  m.fmt = sf;
  m.rows = out_dim;
  m.cols = in_dim;
  const int64_t nb = linear_stream_bytes(sf, out_dim, in_dim);
  if (hipMalloc(&l->wbuf, (size_t)nb) != hipSuccess) {
    (void)hipGetLastError();
    return bail(lfail(l, QMOE_ERR_NOMEM, "hipMalloc of " + std::to_string(nb) + " weight bytes failed"));
  }
  l->weight_bytes = nb;
  m.w = (const uint8_t *)l->wbuf;
  *out = l;
  return QMOE_OK;
}

void qmoe_linear_destroy(qmoe_linear *l) {
  if (!l) return;
  (void)hipSetDevice(l->device);
  if (l->stream) (void)hipStreamSynchronize(l->stream);
  if (l->wbuf) (void)hipFree(l->wbuf);
  if (l->ws) (void)hipFree(l->ws);
  if (l->stream) (void)hipStreamDestroy(l->stream);
  delete l;
}

const char *qmoe_linear_last_error(const qmoe_linear *l) {
  return l ? l->err.c_str() : g_lin_create_error.c_str();
}

qmoe_status qmoe_linear_set(qmoe_linear *l, const void *w, const void *scales) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  LHIP_TRY(l, hipSetDevice(l->device), "hipSetDevice");
  if (!w) return lfail(l, QMOE_ERR_INVALID, "null weight pointer");
  const bool f32s = lin_f32s(l->fmt);
  if ((fmt_quant(l->fmt) || f32s) && !scales) return lfail(l, QMOE_ERR_INVALID, "null scale pointer");
  const LinMat &m = l->m;
  // row blocks staged through the device in the reference layout (codes or
  // elements, then the scales: fp16 bits, or f32 for the f32-scale formats),
  // then rewritten into the lane stream
  const int base = f32s ? (l->fmt == QMOE_INT8G32_F32S ? (int)kINT8 : (int)kINT4) : m.fmt;
  const int64_t in_row = fmt_matrix_bytes(base, 1, m.cols);
  const int64_t sc_row = (fmt_quant(base) ? (int64_t)(m.cols / kGroup) : 0) * (f32s ? 4 : 2);
  const int64_t per = in_row + sc_row;
  int64_t chunk = std::min<int64_t>(m.rows, std::max<int64_t>(64, ((int64_t)256 << 20) / per));
  chunk = (chunk + 63) / 64 * 64;  // whole 64-row blocks of the stream
  uint8_t *tmp = nullptr;
  LHIP_TRY(l, hipMalloc(&tmp, (size_t)(chunk * per)), "hipMalloc upload staging");
  const int64_t stream_row = linear_stream_bytes(m.fmt, 64, m.cols) / 64;  // stream bytes per row
  qmoe_status st = QMOE_OK;
  for (int64_t r0 = 0; r0 < m.rows; r0 += chunk) {
    const int64_t n = std::min(chunk, (int64_t)m.rows - r0);
    uint8_t *tsc = tmp + n * in_row;
    hipError_t e = hipMemcpy(tmp, (const uint8_t *)w + r0 * in_row, (size_t)(n * in_row), hipMemcpyHostToDevice);
    if (e == hipSuccess && sc_row)
      e = hipMemcpy(tsc, (const uint8_t *)scales + r0 * sc_row, (size_t)(n * sc_row), hipMemcpyHostToDevice);
    if (e == hipSuccess)
      e = launch_linear_relayout(m.fmt, tmp, sc_row ? tsc : nullptr, (int)n, m.cols,
                                 (uint8_t *)l->wbuf + r0 * stream_row, l->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(l->stream);
    if (e != hipSuccess) {
      st = lhip(l, e, "weight upload");
      break;
    }
  }
  (void)hipFree(tmp);
  if (st == QMOE_OK) l->has_w = true;
  return st;
}

qmoe_status qmoe_linear_forward_device(qmoe_linear *l, const float *d_x, int32_t T, float *d_y, void *stream) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = lenter(l);
  if (s != QMOE_OK) return s;
  if ((s = check_T(l, T)) != QMOE_OK) return s;
  if (T == 0) return QMOE_OK;
  if (!d_x || !d_y) return lfail(l, QMOE_ERR_INVALID, "null x or y");
  LHIP_TRY(l, launch_linear(d_x, T, l->m, d_y, (hipStream_t)stream), "linear launch");
  return QMOE_OK;
}

qmoe_status qmoe_linear_forward(qmoe_linear *l, const float *x, int32_t T, float *y) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = lenter(l);
  if (s != QMOE_OK) return s;
  if ((s = check_T(l, T)) != QMOE_OK) return s;
  if (T == 0) return QMOE_OK;
  if (!x || !y) return lfail(l, QMOE_ERR_INVALID, "null x or y");
  LinWs w;
  if ((s = lin_workspace(l, T, true, 0, &w)) != QMOE_OK) return s;
  LHIP_TRY(l, hipMemcpyAsync(w.x, x, (size_t)T * l->in_dim * 4, hipMemcpyHostToDevice, l->stream), "copy x");
  LHIP_TRY(l, launch_linear(w.x, T, l->m, w.y, l->stream), "linear launch");
  LHIP_TRY(l, hipMemcpyAsync(y, w.y, (size_t)T * l->out_dim * 4, hipMemcpyDeviceToHost, l->stream), "copy y");
  LHIP_TRY(l, hipStreamSynchronize(l->stream), "hipStreamSynchronize");
  return QMOE_OK;
}

qmoe_status qmoe_linear_greedy(qmoe_linear *l, const float *x, int32_t T, int32_t *token, float *logits) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  qmoe_status s = lenter(l);
  if (s != QMOE_OK) return s;
  if ((s = check_T(l, T)) != QMOE_OK) return s;
  if (T == 0) return QMOE_OK;
  if (!x || !token) return lfail(l, QMOE_ERR_INVALID, "null x or token");
  if (T > 65535) return lfail(l, QMOE_ERR_UNSUPPORTED, "T > 65535");
  LinWs w;
  if ((s = lin_workspace(l, T, true, l->out_dim, &w)) != QMOE_OK) return s;
  LHIP_TRY(l, hipMemcpyAsync(w.x, x, (size_t)T * l->in_dim * 4, hipMemcpyHostToDevice, l->stream), "copy x");
  LHIP_TRY(l, launch_linear(w.x, T, l->m, w.y, l->stream), "linear launch");
  LHIP_TRY(l, launch_argmax(w.y, T, l->out_dim, w.pv, w.pi, w.tok, l->stream), "argmax launch");
  LHIP_TRY(l, hipMemcpyAsync(token, w.tok, (size_t)T * 4, hipMemcpyDeviceToHost, l->stream), "copy tokens");
  if (logits)
    LHIP_TRY(l, hipMemcpyAsync(logits, w.y, (size_t)T * l->out_dim * 4, hipMemcpyDeviceToHost, l->stream),
             "copy logits");
  LHIP_TRY(l, hipStreamSynchronize(l->stream), "hipStreamSynchronize");
  return QMOE_OK;
}

qmoe_status qmoe_linear_argmax_device(qmoe_linear *l, const float *d_v, int32_t T, int32_t n, int32_t *d_token,
                                      void *stream) {
  if (!l) return QMOE_ERR_INVALID;
  std::lock_guard<std::mutex> g(l->mu);
  LHIP_TRY(l, hipSetDevice(l->device), "hipSetDevice");
  if (T < 0 || n <= 0) return lfail(l, QMOE_ERR_INVALID, "T < 0 or n <= 0");
  if (T > 65535) return lfail(l, QMOE_ERR_UNSUPPORTED, "T > 65535");
  if (T == 0) return QMOE_OK;
  if (!d_v || !d_token) return lfail(l, QMOE_ERR_INVALID, "null v or token");
  LinWs w;
  qmoe_status s = lin_workspace(l, T, false, n, &w);
  if (s != QMOE_OK) return s;
  LHIP_TRY(l, launch_argmax(d_v, T, n, w.pv, w.pi, d_token, (hipStream_t)stream), "argmax launch");
  return QMOE_OK;
}

int64_t qmoe_linear_device_bytes(const qmoe_linear *l) {
  return l ? l->weight_bytes + (int64_t)l->ws_n : 0;
}

}  // extern "C"
