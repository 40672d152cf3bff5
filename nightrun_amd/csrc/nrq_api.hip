// C ABI of libnrq (declared in include/nrq.h).
//
// Host-slice entry points mirror nr-tensor's functions one for one: the same
// shape assertions (as NRQ_ERR_SHAPE with the assertion text), the same
// argument meaning, synchronous return. The row-parallel worker pool of the
// reference (parallel.rs:86-105) becomes one HIP stream: a call is one kernel
// launch whose grid covers the rows, then a stream sync.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/nrq.h"
#include "nrq_device.h"
#include "nrq_launch.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(NRQ_ERR_DEVICE, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr)                          \
  do {                                         \
    hipError_t e_ = (expr);                    \
    if (e_ != hipSuccess) return hip_fail(e_, #expr); \
  } while (0)

struct Region {
  const uint8_t* host;
  size_t bytes;
  uint8_t* dev;
};

// Grow-only device scratch: steady-state calls allocate nothing.
struct Scratch {
  void* p = nullptr;
  size_t cap = 0;
  int ensure(size_t n) {
    if (n <= cap) return 0;
    if (p) hipFree(p);
    p = nullptr;
    cap = 0;
    size_t want = (n + 4095) & ~(size_t)4095;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(scratch)");
    cap = want;
    return 0;
  }
  void release() {
    if (p) hipFree(p);
    p = nullptr;
    cap = 0;
  }
};

struct State {
  std::mutex mu;
  bool init = false;
  int device = -1;
  hipStream_t stream = nullptr;
  int order = nrq::kOrderScalar;
  std::vector<Region> regions;
  Scratch w, x, y, src;
};

State& S() {
  static State s;
  return s;
}

int qk_of(int dtype) { return dtype == NRQ_Q8_0 ? 32 : 256; }
size_t wbytes_of(int dtype) {
  return dtype == NRQ_Q8_0 ? nrq::kQ8_0Bytes : (dtype == NRQ_Q4_K ? nrq::kQ4KBytes : nrq::kQ6KBytes);
}
size_t xbytes_of(int dtype) { return dtype == NRQ_Q8_0 ? nrq::kQ8_0Bytes : nrq::kQ8KBytes; }
bool dtype_ok(int dtype) { return dtype == NRQ_Q8_0 || dtype == NRQ_Q4_K || dtype == NRQ_Q6_K; }

int launch_rc(int rc, const char* what) {
  if (rc == nrq::NRQ_LAUNCH_OK) return NRQ_OK;
  if (rc == nrq::NRQ_LAUNCH_TOO_WIDE) return fail(NRQ_ERR_UNSUPPORTED, "%s: row too wide for the LDS tile", what);
  if (rc == nrq::NRQ_LAUNCH_BAD_ARG) return fail(NRQ_ERR_ARG, "%s: bad argument", what);
  hipError_t e = hipGetLastError();
  return fail(NRQ_ERR_DEVICE, "%s: launch failed: %s", what, hipGetErrorString(e));
}

const uint8_t* lookup(State& s, const void* host, size_t bytes) {
  const uint8_t* p = (const uint8_t*)host;
  for (const Region& r : s.regions)
    if (p >= r.host && p + bytes <= r.host + r.bytes) return r.dev + (p - r.host);
  return nullptr;
}

hipStream_t stream_or_default(void* stream) {
  return stream ? (hipStream_t)stream : S().stream;
}

// Shared body of the six host-slice matvec/matmul entry points.
int host_matmul(int dtype, const char* name, float* y, size_t y_len, const void* w, size_t w_len, const void* xs,
                size_t xs_len, size_t rows, size_t cols, size_t batch, bool is_matvec) {
  State& s = S();
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.init) return fail(NRQ_ERR_NOT_INIT, "%s: nrq_init was not called", name);
  const size_t bpr = cols / qk_of(dtype);
  // kernels.rs:38-40,100-102; kquant.rs:541-543,579-581
  if (is_matvec) {
    if (y_len != rows)
      return fail(NRQ_ERR_SHAPE, "%s: assertion `left == right` failed: y.len() == rows (left: %zu, right: %zu)",
                  name, y_len, rows);
    if (xs_len != bpr)
      return fail(NRQ_ERR_SHAPE, "%s: assertion `left == right` failed: x.len() == bpr (left: %zu, right: %zu)",
                  name, xs_len, bpr);
  } else {
    if (y_len != batch * rows)
      return fail(NRQ_ERR_SHAPE,
                  "%s: assertion `left == right` failed: y.len() == batch * rows (left: %zu, right: %zu)", name,
                  y_len, batch * rows);
    if (xs_len != batch * bpr)
      return fail(NRQ_ERR_SHAPE,
                  "%s: assertion `left == right` failed: xs.len() == batch * bpr (left: %zu, right: %zu)", name,
                  xs_len, batch * bpr);
  }
  if (w_len < rows * bpr)
    return fail(NRQ_ERR_SHAPE, "%s: assertion failed: w.len() >= rows * bpr (%zu < %zu)", name, w_len, rows * bpr);
  if (y_len == 0) return NRQ_OK;
  if (!y || (bpr && (!w || !xs))) return fail(NRQ_ERR_ARG, "%s: null pointer", name);
  if (rows > 0x7fffffff || bpr > 0x7fffffff || batch > 0x7fffffff)
    return fail(NRQ_ERR_UNSUPPORTED, "%s: dimension exceeds 2^31", name);
  if (bpr == 0) {  // an empty dot is +0.0 in both orders
    for (size_t i = 0; i < y_len; i++) y[i] = 0.0f;
    return NRQ_OK;
  }
  const size_t wbytes = rows * bpr * wbytes_of(dtype);
  const size_t xbytes = batch * bpr * xbytes_of(dtype);
  const uint8_t* dw = lookup(s, w, wbytes);
  int rc;
  if (!dw) {
    if ((rc = s.w.ensure(wbytes + 64))) return rc;
    HIP_TRY(hipMemcpyAsync(s.w.p, w, wbytes, hipMemcpyHostToDevice, s.stream));
    dw = (const uint8_t*)s.w.p;
  }
  if (((uintptr_t)dw & 15) != 0)
    return fail(NRQ_ERR_ARG, "%s: weight slice is not 16-byte aligned within its registered region", name);
  if ((rc = s.x.ensure(xbytes))) return rc;
  if ((rc = s.y.ensure(y_len * sizeof(float)))) return rc;
  HIP_TRY(hipMemcpyAsync(s.x.p, xs, xbytes, hipMemcpyHostToDevice, s.stream));
  if (is_matvec) {
    nrq::MatvecLaunch L{dw, s.x.p, (float*)s.y.p, (int)rows, (int)bpr, 0, s.stream};
    if ((rc = launch_rc(nrq::launch_matvec(dtype, s.order, L), name))) return rc;
  } else {
    nrq::MatmulLaunch L{dw, s.x.p, (float*)s.y.p, (int)rows, (int)bpr, (int)batch, s.stream};
    if ((rc = launch_rc(nrq::launch_matmul(dtype, s.order, L), name))) return rc;
  }
  HIP_TRY(hipMemcpyAsync(y, s.y.p, y_len * sizeof(float), hipMemcpyDeviceToHost, s.stream));
  HIP_TRY(hipStreamSynchronize(s.stream));
  return NRQ_OK;
}

int host_quantize(bool q8k, const char* name, const float* src, size_t src_len, void* out, size_t out_len) {
  State& s = S();
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.init) return fail(NRQ_ERR_NOT_INIT, "%s: nrq_init was not called", name);
  const size_t qk = q8k ? 256 : 32;
  // q8.rs:28, kquant.rs:158
  if (src_len != out_len * qk)
    return fail(NRQ_ERR_SHAPE, "%s: assertion `left == right` failed: src.len() == out.len() * %zu (left: %zu, right: %zu)",
                name, qk, src_len, out_len * qk);
  if (out_len == 0) return NRQ_OK;
  if (!src || !out) return fail(NRQ_ERR_ARG, "%s: null pointer", name);
  const size_t ob = out_len * (q8k ? nrq::kQ8KBytes : nrq::kQ8_0Bytes);
  int rc;
  if ((rc = s.src.ensure(src_len * sizeof(float)))) return rc;
  if ((rc = s.x.ensure(ob))) return rc;
  HIP_TRY(hipMemcpyAsync(s.src.p, src, src_len * sizeof(float), hipMemcpyHostToDevice, s.stream));
  nrq::QuantLaunch L{(const float*)s.src.p, s.x.p, (long long)src_len, s.stream};
  rc = q8k ? nrq::launch_quantize_q8k(L) : nrq::launch_quantize_q8_0(L);
  if ((rc = launch_rc(rc, name))) return rc;
  HIP_TRY(hipMemcpyAsync(out, s.x.p, ob, hipMemcpyDeviceToHost, s.stream));
  HIP_TRY(hipStreamSynchronize(s.stream));
  return NRQ_OK;
}

int dev_check(const char* name, int dtype, int order) {
  if (!S().init) return fail(NRQ_ERR_NOT_INIT, "%s: nrq_init was not called", name);
  if (!dtype_ok(dtype)) return fail(NRQ_ERR_ARG, "%s: unknown dtype %d", name, dtype);
  if (order != NRQ_ORDER_SCALAR && order != NRQ_ORDER_AVX2) return fail(NRQ_ERR_ARG, "%s: unknown order %d", name, order);
  return NRQ_OK;
}

}  // namespace

namespace nrq {
void set_last_error(const char* msg) { g_err = msg; }
}  // namespace nrq

extern "C" {

int nrq_init(int device) {
  State& s = S();
  std::lock_guard<std::mutex> lk(s.mu);
  if (s.init) {
    if (device == s.device) return NRQ_OK;
    return fail(NRQ_ERR_ARG, "nrq_init: already initialised on device %d", s.device);
  }
  int n = 0;
  HIP_TRY(hipGetDeviceCount(&n));
  if (device < 0 || device >= n) return fail(NRQ_ERR_DEVICE, "nrq_init: device %d not present (%d devices)", device, n);
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(NRQ_ERR_DEVICE, "nrq_init: device %d is %s, libnrq is built for gfx950 only", device, prop.gcnArchName);
  HIP_TRY(hipSetDevice(device));
  HIP_TRY(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking));
  if (nrq::sample_scratch_setup() != NRQ_OK) {
    hipStreamDestroy(s.stream);
    s.stream = nullptr;
    return NRQ_ERR_DEVICE;
  }
  s.device = device;
  s.init = true;
  g_err.clear();
  return NRQ_OK;
}

int nrq_shutdown(void) {
  State& s = S();
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.init) return NRQ_OK;
  hipStreamSynchronize(s.stream);
  for (Region& r : s.regions) hipFree(r.dev);
  s.regions.clear();
  s.w.release();
  s.x.release();
  s.y.release();
  s.src.release();
  hipStreamDestroy(s.stream);
  s.stream = nullptr;
  s.init = false;
  s.device = -1;
  return NRQ_OK;
}

const char* nrq_last_error(void) { return g_err.c_str(); }

int nrq_device_info(char* buf, size_t len) {
  State& s = S();
  if (!s.init) return fail(NRQ_ERR_NOT_INIT, "nrq_device_info: nrq_init was not called");
  if (!buf || !len) return fail(NRQ_ERR_ARG, "nrq_device_info: null buffer");
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, s.device));
  snprintf(buf, len, "%s %s, %d CUs, %zu bytes HBM, %zu bytes LDS/block", prop.gcnArchName, prop.name,
           prop.multiProcessorCount, (size_t)prop.totalGlobalMem, (size_t)prop.sharedMemPerBlock);
  return NRQ_OK;
}

int nrq_set_order(int order) {
  if (order != NRQ_ORDER_SCALAR && order != NRQ_ORDER_AVX2)
    return fail(NRQ_ERR_ARG, "nrq_set_order: unknown order %d", order);
  State& s = S();
  std::lock_guard<std::mutex> lk(s.mu);
  s.order = order;
  return NRQ_OK;
}

int nrq_get_order(void) { return S().order; }

int nrq_register_weights(const void* host, size_t bytes) {
  State& s = S();
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.init) return fail(NRQ_ERR_NOT_INIT, "nrq_register_weights: nrq_init was not called");
  if (!host || !bytes) return fail(NRQ_ERR_ARG, "nrq_register_weights: empty region");
  for (const Region& r : s.regions)
    if ((const uint8_t*)host < r.host + r.bytes && r.host < (const uint8_t*)host + bytes)
      return fail(NRQ_ERR_ARG, "nrq_register_weights: region overlaps a registered one");
  void* dev = nullptr;
  HIP_TRY(hipMalloc(&dev, bytes + 64));
  hipError_t e = hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    hipFree(dev);
    return hip_fail(e, "nrq_register_weights: hipMemcpy");
  }
  s.regions.push_back(Region{(const uint8_t*)host, bytes, (uint8_t*)dev});
  return NRQ_OK;
}

int nrq_unregister_weights(const void* host) {
  State& s = S();
  std::lock_guard<std::mutex> lk(s.mu);
  for (size_t i = 0; i < s.regions.size(); i++) {
    if (s.regions[i].host == (const uint8_t*)host) {
      hipStreamSynchronize(s.stream);
      hipFree(s.regions[i].dev);
      s.regions.erase(s.regions.begin() + i);
      return NRQ_OK;
    }
  }
  return fail(NRQ_ERR_ARG, "nrq_unregister_weights: region not registered");
}

int nrq_matvec_q8(float* y, size_t y_len, const void* w, size_t w_len, const void* x, size_t x_len, size_t rows,
                  size_t cols) {
  return host_matmul(NRQ_Q8_0, "matvec_q8", y, y_len, w, w_len, x, x_len, rows, cols, 1, true);
}
int nrq_matmul_q8(float* y, size_t y_len, const void* w, size_t w_len, const void* xs, size_t xs_len, size_t rows,
                  size_t cols, size_t batch) {
  return host_matmul(NRQ_Q8_0, "matmul_q8", y, y_len, w, w_len, xs, xs_len, rows, cols, batch, false);
}
int nrq_matvec_q4k(float* y, size_t y_len, const void* w, size_t w_len, const void* x, size_t x_len, size_t rows,
                   size_t cols) {
  return host_matmul(NRQ_Q4_K, "matvec_q4k", y, y_len, w, w_len, x, x_len, rows, cols, 1, true);
}
int nrq_matvec_q6k(float* y, size_t y_len, const void* w, size_t w_len, const void* x, size_t x_len, size_t rows,
                   size_t cols) {
  return host_matmul(NRQ_Q6_K, "matvec_q6k", y, y_len, w, w_len, x, x_len, rows, cols, 1, true);
}
int nrq_matmul_q4k(float* y, size_t y_len, const void* w, size_t w_len, const void* xs, size_t xs_len, size_t rows,
                   size_t cols, size_t batch) {
  return host_matmul(NRQ_Q4_K, "matmul_q4k", y, y_len, w, w_len, xs, xs_len, rows, cols, batch, false);
}
int nrq_matmul_q6k(float* y, size_t y_len, const void* w, size_t w_len, const void* xs, size_t xs_len, size_t rows,
                   size_t cols, size_t batch) {
  return host_matmul(NRQ_Q6_K, "matmul_q6k", y, y_len, w, w_len, xs, xs_len, rows, cols, batch, false);
}

int nrq_quantize(const float* src, size_t src_len, void* out, size_t out_len) {
  return host_quantize(false, "quantize", src, src_len, out, out_len);
}
int nrq_quantize_q8k(const float* src, size_t src_len, void* out, size_t out_len) {
  return host_quantize(true, "quantize_q8k", src, src_len, out, out_len);
}

int nrq_dev_matvec(int dtype, int order, float* y, const void* w, const void* x, size_t rows, size_t cols,
                   void* stream) {
  int rc = dev_check("nrq_dev_matvec", dtype, order);
  if (rc) return rc;
  const size_t bpr = cols / qk_of(dtype);
  if (rows == 0) return NRQ_OK;
  if (!y || (bpr && (!w || !x))) return fail(NRQ_ERR_ARG, "nrq_dev_matvec: null pointer");
  if (((uintptr_t)w & 15) != 0) return fail(NRQ_ERR_ARG, "nrq_dev_matvec: weights not 16-byte aligned");
  if (((uintptr_t)x & (dtype == NRQ_Q8_0 ? 1 : 3)) != 0)
    return fail(NRQ_ERR_ARG, "nrq_dev_matvec: activation blocks not aligned like their Rust type");
  if (rows > 0x7fffffff || bpr > 0x7fffffff) return fail(NRQ_ERR_UNSUPPORTED, "nrq_dev_matvec: dimension exceeds 2^31");
  hipStream_t st = stream_or_default(stream);
  if (bpr == 0) {
    return launch_rc(nrq::launch_fill_zero(y, (long long)rows, st), "nrq_dev_matvec");
  }
  nrq::MatvecLaunch L{w, x, y, (int)rows, (int)bpr, 0, st};
  return launch_rc(nrq::launch_matvec(dtype, order, L), "nrq_dev_matvec");
}

int nrq_dev_matmul(int dtype, int order, float* y, const void* w, const void* xs, size_t rows, size_t cols,
                   size_t batch, void* stream) {
  int rc = dev_check("nrq_dev_matmul", dtype, order);
  if (rc) return rc;
  const size_t bpr = cols / qk_of(dtype);
  if (rows == 0 || batch == 0) return NRQ_OK;
  if (!y || (bpr && (!w || !xs))) return fail(NRQ_ERR_ARG, "nrq_dev_matmul: null pointer");
  if (((uintptr_t)w & 15) != 0) return fail(NRQ_ERR_ARG, "nrq_dev_matmul: weights not 16-byte aligned");
  if (((uintptr_t)xs & (dtype == NRQ_Q8_0 ? 1 : 3)) != 0)
    return fail(NRQ_ERR_ARG, "nrq_dev_matmul: activation blocks not aligned like their Rust type");
  if (rows > 0x7fffffff || bpr > 0x7fffffff || batch > 0x7fffffff)
    return fail(NRQ_ERR_UNSUPPORTED, "nrq_dev_matmul: dimension exceeds 2^31");
  hipStream_t st = stream_or_default(stream);
  if (bpr == 0) {
    return launch_rc(nrq::launch_fill_zero(y, (long long)(rows * batch), st), "nrq_dev_matmul");
  }
  nrq::MatmulLaunch L{w, xs, y, (int)rows, (int)bpr, (int)batch, st};
  return launch_rc(nrq::launch_matmul(dtype, order, L), "nrq_dev_matmul");
}

int nrq_dev_matmul_group(int dtype, int n, float* const* ys, const void* const* ws, const size_t* rows,
                         const void* xs, size_t cols, size_t batch, void* stream) {
  int rc = dev_check("nrq_dev_matmul_group", dtype, nrq::kOrderScalar);
  if (rc) return rc;
  if (n < 1 || n > 3 || !ys || !ws || !rows) return fail(NRQ_ERR_ARG, "nrq_dev_matmul_group: 1 to 3 matrices");
  const size_t bpr = cols / qk_of(dtype);
  if (batch == 0) return NRQ_OK;
  bool whole = bpr > 0 && (size_t)cols % qk_of(dtype) == 0;
  for (int i = 0; i < n; i++) {
    if (!ys[i] || (bpr && !ws[i])) return fail(NRQ_ERR_ARG, "nrq_dev_matmul_group: null pointer");
    if (((uintptr_t)ws[i] & 15) != 0) return fail(NRQ_ERR_ARG, "nrq_dev_matmul_group: weights not 16-byte aligned");
    if (rows[i] == 0 || rows[i] > 0x7fffffff) whole = false;
  }
  if (bpr && !xs) return fail(NRQ_ERR_ARG, "nrq_dev_matmul_group: null pointer");
  if (((uintptr_t)xs & (dtype == NRQ_Q8_0 ? 1 : 3)) != 0)
    return fail(NRQ_ERR_ARG, "nrq_dev_matmul_group: activation blocks not aligned like their Rust type");
  if (bpr > 0x7fffffff || batch > 0x7fffffff) return fail(NRQ_ERR_UNSUPPORTED, "nrq_dev_matmul_group: dimension exceeds 2^31");
  if (whole && n > 1) {
    nrq::MatmulGroupLaunch G{};
    for (int i = 0; i < n; i++) {
      G.w[i] = ws[i];
      G.y[i] = ys[i];
      G.rows[i] = (int)rows[i];
    }
    G.nmat = n;
    G.xs = xs;
    G.bpr = (int)bpr;
    G.batch = (int)batch;
    G.stream = stream_or_default(stream);
    const int lr = nrq::launch_mmt_group(dtype, G);
    if (lr != nrq::NRQ_LAUNCH_BAD_ARG) return launch_rc(lr, "nrq_dev_matmul_group");
  }
  for (int i = 0; i < n; i++)  // the group as separate launches
    if ((rc = nrq_dev_matmul(dtype, nrq::kOrderScalar, ys[i], ws[i], xs, rows[i], cols, batch, stream))) return rc;
  return NRQ_OK;
}

int nrq_dev_quantize_q8_0(const float* src, size_t n, void* out, void* stream) {
  if (!S().init) return fail(NRQ_ERR_NOT_INIT, "nrq_dev_quantize_q8_0: nrq_init was not called");
  if (n % 32) return fail(NRQ_ERR_SHAPE, "nrq_dev_quantize_q8_0: n = %zu is not a multiple of 32", n);
  if (n == 0) return NRQ_OK;
  if (!src || !out) return fail(NRQ_ERR_ARG, "nrq_dev_quantize_q8_0: null pointer");
  nrq::QuantLaunch L{src, out, (long long)n, stream_or_default(stream)};
  return launch_rc(nrq::launch_quantize_q8_0(L), "nrq_dev_quantize_q8_0");
}

int nrq_dev_quantize_q8k(const float* src, size_t n, void* out, void* stream) {
  if (!S().init) return fail(NRQ_ERR_NOT_INIT, "nrq_dev_quantize_q8k: nrq_init was not called");
  if (n % 256) return fail(NRQ_ERR_SHAPE, "nrq_dev_quantize_q8k: n = %zu is not a multiple of 256", n);
  if (n == 0) return NRQ_OK;
  if (!src || !out) return fail(NRQ_ERR_ARG, "nrq_dev_quantize_q8k: null pointer");
  if (((uintptr_t)out & 3) != 0) return fail(NRQ_ERR_ARG, "nrq_dev_quantize_q8k: output not 4-byte aligned");
  nrq::QuantLaunch L{src, out, (long long)n, stream_or_default(stream)};
  return launch_rc(nrq::launch_quantize_q8k(L), "nrq_dev_quantize_q8k");
}

int nrq_dev_block_sums(int dtype, const void* w, const void* x, int32_t* out, size_t rows, size_t cols,
                       void* stream) {
  int rc = dev_check("nrq_dev_block_sums", dtype, NRQ_ORDER_SCALAR);
  if (rc) return rc;
  const size_t bpr = cols / qk_of(dtype);
  if (rows == 0 || bpr == 0) return NRQ_OK;
  if (!w || !x || !out) return fail(NRQ_ERR_ARG, "nrq_dev_block_sums: null pointer");
  if (((uintptr_t)w & 15) != 0) return fail(NRQ_ERR_ARG, "nrq_dev_block_sums: weights not 16-byte aligned");
  if (((uintptr_t)x & (dtype == NRQ_Q8_0 ? 1 : 3)) != 0)
    return fail(NRQ_ERR_ARG, "nrq_dev_block_sums: activation blocks not aligned like their Rust type");
  return launch_rc(nrq::launch_block_sums(dtype, w, x, out, (int)rows, (int)bpr, stream_or_default(stream)),
                   "nrq_dev_block_sums");
}

int nrq_sync(void* stream) {
  if (!S().init) return fail(NRQ_ERR_NOT_INIT, "nrq_sync: nrq_init was not called");
  HIP_TRY(hipStreamSynchronize(stream_or_default(stream)));
  return NRQ_OK;
}

int nrq_dev_stream_read(const void* data, size_t bytes, uint32_t* out, void* stream) {
  if (!S().init) return fail(NRQ_ERR_NOT_INIT, "nrq_dev_stream_read: nrq_init was not called");
  if (!out || (bytes && !data)) return fail(NRQ_ERR_ARG, "nrq_dev_stream_read: null pointer");
  if (((uintptr_t)data & 15) || (bytes & 15)) return fail(NRQ_ERR_ARG, "nrq_dev_stream_read: needs 16-byte units");
  return launch_rc(nrq::launch_stream_read(data, (long long)bytes, out, stream_or_default(stream)),
                   "nrq_dev_stream_read");
}

}  // extern "C"
