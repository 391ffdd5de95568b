// extern "C" entry points declared in include/mhc_amd.h: argument checks,
// kernel selection, error reporting.  No device allocation anywhere.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "mhc_amd.h"
#include "mhc_internal.hpp"

// Scratch of mhc_pre_bwd_weights_noalloc (its token-range partial sums), for
// callers that cannot allocate.  Each device holds its own copy for the life
// of the process; calls on one device share it, so calls that overlap on one
// device (two streams, two threads) race on it.  Every byte a call reads was
// written earlier in the same call, so nothing needs clearing.
constexpr int64_t kScratchBytes = int64_t(32) << 20;
static __device__ __align__(256) float scratch[kScratchBytes / 4];

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  return fail((int)e, "%s: %s", what, hipGetErrorString(e));
}

bool dtype_ok(int dt) { return dt == mhc::kF32 || dt == mhc::kBF16 || dt == mhc::kF16; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

constexpr int kMaxN = 16;
constexpr int64_t kMaxBlocks = 0x7fffffff;

// Shared checks for the three pre-phase style entry points.
int check_pre(const mhc::PreArgs& a, const char* fn) {
  if (a.M < 0) return fail(hipErrorInvalidValue, "%s: M must be >= 0 (got %lld)", fn, (long long)a.M);
  if (a.n < 1 || a.n > kMaxN) return fail(hipErrorInvalidValue, "%s: n must be in [1, %d] (got %d)", fn, kMaxN, a.n);
  if (a.C < 1) return fail(hipErrorInvalidValue, "%s: C must be >= 1 (got %d)", fn, a.C);
  if (!dtype_ok(a.x_dtype)) return fail(hipErrorInvalidValue, "%s: bad x dtype %d", fn, a.x_dtype);
  if (a.M > kMaxBlocks) return fail(hipErrorInvalidValue, "%s: M too large", fn);
  if (a.M == 0) return 0;  // empty batch: nothing to read or write (pointers may be null)
  if (!a.x || !a.sub_in) return fail(hipErrorInvalidValue, "%s: x and the main output are required", fn);
  if (a.mode != mhc::kRms) {
    if (!a.phi) return fail(hipErrorInvalidValue, "%s: phi is required", fn);
    if (!dtype_ok(a.phi_dtype)) return fail(hipErrorInvalidValue, "%s: bad phi dtype %d", fn, a.phi_dtype);
    if (!dtype_ok(a.param_dtype)) return fail(hipErrorInvalidValue, "%s: bad param dtype %d", fn, a.param_dtype);
    if (!a.alpha[0] || !a.bias[0]) return fail(hipErrorInvalidValue, "%s: alpha/bias are required", fn);
  }
  if ((a.mode == mhc::kFull || a.mode == mhc::kNoHres) && (!a.h_post || !a.alpha[1] || !a.bias[1]))
    return fail(hipErrorInvalidValue, "%s: h_post, alpha_post and bias_post are required", fn);
  if (a.mode == mhc::kFull && (!a.alpha[2] || !a.bias[2]))
    return fail(hipErrorInvalidValue, "%s: alpha_res and bias_res are required", fn);
  if (a.norm_w && !dtype_ok(a.norm_dtype)) return fail(hipErrorInvalidValue, "%s: bad norm dtype %d", fn, a.norm_dtype);
  if (a.norm_w && !(a.norm_eps >= 0.f)) return fail(hipErrorInvalidValue, "%s: norm_eps must be >= 0", fn);
  if (a.x_ssq && !mhc::ssq_supported(a.x_dtype, a.C))
    return fail(hipErrorInvalidValue, "%s: x_ssq needs a bf16 stream with C %% %d == 0", fn, mhc::kSsqCols);
  return 0;
}

int run_pre(mhc::PreArgs& a, hipStream_t stream, const char* fn) {
  if (int rc = check_pre(a, fn)) return rc;
  if (a.M == 0) return 0;
  const bool packed_ok = a.phi_packed && a.mode != mhc::kRms && aligned16(a.x) && aligned16(a.sub_in) &&
                         aligned16(a.phi_packed);
  const bool mfma = packed_ok && mhc::mfma_supported(a.x_dtype, a.phi_dtype, a.n, a.C, a.mode);
  const bool split = packed_ok && !a.norm_w && mhc::split_supported(a.x_dtype, a.phi_dtype, a.n, a.C, a.mode);
  const bool ks32 = packed_ok && mhc::ks32_supported(a.x_dtype, a.phi_dtype, a.n, a.C, a.mode);
  if (!mfma && !split && !ks32) a.phi_packed = nullptr;
  if (!mfma || !mhc::ssq_used(a.n, a.C)) a.x_ssq = nullptr;
  if (split) return hip_status(mhc::launch_pre_split(a, mhc::device_cus(), stream), fn);
  if (ks32) return hip_status(mhc::launch_pre_kstream_f32(a, stream), fn);
  return hip_status(mfma ? mhc::launch_pre_mfma(a, stream) : mhc::launch_pre_generic(a, stream), fn);
}

// mhc_pre_bwd_weights / mhc_pre_bwd_weights_noalloc: checks and launch with the
// given workspace; max_ranges > 0 caps the token ranges to what it holds.
int weights_entry(const void* x, int x_dtype, const float* inv_rms, const float* mixes_raw,
                  const float* g_raw, const void* alpha_pre, const void* alpha_post,
                  const void* alpha_res, int param_dtype, void* g_phi, int phi_dtype,
                  void* g_alpha_pre, void* g_bias_pre, void* g_alpha_post, void* g_bias_post,
                  void* g_alpha_res, void* g_bias_res, void* workspace, int64_t workspace_bytes,
                  int64_t M, int n, int C, int mode, int max_ranges, hipStream_t stream,
                  const char* fn) {
  if (M < 0 || n < 1 || n > kMaxN || C < 1) return fail(hipErrorInvalidValue, "%s: bad shape", fn);
  if (mode != mhc::kFull && mode != mhc::kNoHres && mode != mhc::kHead) return fail(hipErrorInvalidValue, "%s: bad mode %d", fn, mode);
  if (!dtype_ok(x_dtype) || !dtype_ok(phi_dtype) || !dtype_ok(param_dtype)) return fail(hipErrorInvalidValue, "%s: bad dtype", fn);
  if (M > kMaxBlocks) return fail(hipErrorInvalidValue, "%s: M too large", fn);
  if (!g_phi) return fail(hipErrorInvalidValue, "%s: g_phi is required", fn);
  if (M == 0) return fail(hipErrorInvalidValue, "%s: M == 0 leaves the gradients undefined; zero them instead", fn);
  if (!x || !inv_rms || !mixes_raw || !g_raw || !alpha_pre) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
  if (mode != mhc::kHead && !alpha_post) return fail(hipErrorInvalidValue, "%s: alpha_post is required", fn);
  if (mode == mhc::kFull && !alpha_res) return fail(hipErrorInvalidValue, "%s: alpha_res is required", fn);
  int64_t need = mhc::weights_workspace_bytes(M, n, C, mode);
  const int64_t capped = (int64_t)max_ranges * mhc::weights_range_bytes(n, C, mode);
  if (max_ranges > 0 && capped < need) need = capped;
  if (!workspace || workspace_bytes < need)
    return fail(hipErrorInvalidValue, "%s: workspace of %lld bytes needed (got %lld)", fn, (long long)need, (long long)workspace_bytes);
  if ((reinterpret_cast<uintptr_t>(workspace) & 3) != 0) return fail(hipErrorInvalidValue, "%s: workspace must be 4-byte aligned", fn);
  mhc::WeightsArgs a{};
  a.x = x; a.inv_rms = inv_rms; a.mixes = mixes_raw; a.g_raw = g_raw;
  a.alpha[0] = alpha_pre; a.alpha[1] = alpha_post; a.alpha[2] = alpha_res;
  a.g_phi = g_phi;
  a.g_alpha[0] = g_alpha_pre; a.g_alpha[1] = mode == mhc::kHead ? nullptr : g_alpha_post;
  a.g_alpha[2] = mode == mhc::kFull ? g_alpha_res : nullptr;
  a.g_bias[0] = g_bias_pre; a.g_bias[1] = mode == mhc::kHead ? nullptr : g_bias_post;
  a.g_bias[2] = mode == mhc::kFull ? g_bias_res : nullptr;
  a.work = static_cast<float*>(workspace);
  a.M = M; a.n = n; a.C = C; a.mode = mode;
  a.x_dtype = x_dtype; a.phi_dtype = phi_dtype; a.param_dtype = param_dtype;
  a.max_ranges = max_ranges;
  return hip_status(mhc::launch_pre_bwd_weights(a, stream), fn);
}


constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Looks up device `dev`'s copy of scratch with that device current (the caller
// holds g_scratch_mu).  The host-side name `scratch` is not a device address
// and is never passed to a kernel.
int resolve_scratch(int dev, int cur, const char* fn) {
  if (g_scratch_dev[dev]) return 0;
  if (dev != cur)
    if (hipError_t e = hipSetDevice(dev); e != hipSuccess) return hip_status(e, fn);
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (dev != cur) (void)hipSetDevice(cur);
  if (e != hipSuccess || !p)
    return fail(e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol,
                "%s: hipGetSymbolAddress(scratch) on device %d failed: %s", fn, dev, hipGetErrorString(e));
  g_scratch_dev[dev] = p;
  return 0;
}

// Device address of this device's copy of scratch (the device `stream` runs
// on).  mhc_init looks it up for every device at set-up; a device it has not
// seen is looked up here on its first call, which is refused while `stream`
// is being captured (the lookup may load the code object on that device,
// which is not a capturable operation).
int scratch_ptr(hipStream_t stream, void** out, const char* fn) {
  int cur = 0;
  if (hipError_t e = hipGetDevice(&cur); e != hipSuccess) return hip_status(e, fn);
  int dev = cur;
  if (stream != nullptr)
    if (hipError_t e = hipStreamGetDevice(stream, &dev); e != hipSuccess) return hip_status(e, fn);
  if (dev < 0 || dev >= kMaxDevices) return fail(hipErrorInvalidValue, "%s: device %d out of range", fn, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipError_t e = hipStreamIsCapturing(stream, &cs); e != hipSuccess) return hip_status(e, fn);
    if (cs != hipStreamCaptureStatusNone)
      return fail(hipErrorStreamCaptureUnsupported,
                  "%s: the scratch of device %d is not set up; call mhc_init() (or this entry "
                  "point once) before capturing", fn, dev);
    if (int rc = resolve_scratch(dev, cur, fn)) return rc;
  }
  *out = g_scratch_dev[dev];
  return 0;
}

}  // namespace

extern "C" {

int mhc_abi_version(void) { return 8; }

int mhc_init(void) {
  const char* fn = "mhc_init";
  int count = 0;
  if (hipError_t e = hipGetDeviceCount(&count); e != hipSuccess) return hip_status(e, fn);
  int cur = 0;
  if (hipError_t e = hipGetDevice(&cur); e != hipSuccess) return hip_status(e, fn);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  for (int dev = 0; dev < count && dev < kMaxDevices; ++dev)
    if (int rc = resolve_scratch(dev, cur, fn)) return rc;
  return 0;
}

const char* mhc_last_error(void) { return g_err; }

int64_t mhc_phi_packed_bytes(int n, int C, int mode) { return mhc::mfma_packed_bytes(n, C, mode); }

int mhc_phi_pack(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                 hipStream_t stream) {
  const int64_t bytes = mhc::mfma_packed_bytes(n, C, mode);
  if (bytes <= 0) return fail(hipErrorInvalidValue, "mhc_phi_pack: no MFMA layout for n=%d C=%d mode=%d", n, C, mode);
  if (phi_dtype != mhc::kBF16) return fail(hipErrorInvalidValue, "mhc_phi_pack: phi must be bf16");
  if (!phi || !packed) return fail(hipErrorInvalidValue, "mhc_phi_pack: null pointer");
  return hip_status(mhc::launch_phi_pack(phi, phi_dtype, packed, n, C, mode, stream), "mhc_phi_pack");
}

int64_t mhc_phi_split_bytes(int n, int C, int mode) {
  const int64_t b = mhc::split_packed_bytes(n, C, mode);
  return b > 0 ? b : mhc::ks32_packed_bytes(n, C, mode);
}

int mhc_phi_pack_split(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                       hipStream_t stream) {
  const bool split = mhc::split_packed_bytes(n, C, mode) > 0;
  if (!split && mhc::ks32_packed_bytes(n, C, mode) <= 0)
    return fail(hipErrorInvalidValue, "mhc_phi_pack_split: no split layout for n=%d C=%d mode=%d", n, C, mode);
  if (!dtype_ok(phi_dtype)) return fail(hipErrorInvalidValue, "mhc_phi_pack_split: bad phi dtype %d", phi_dtype);
  if (!phi || !packed) return fail(hipErrorInvalidValue, "mhc_phi_pack_split: null pointer");
  return hip_status(split ? mhc::launch_phi_pack_split(phi, phi_dtype, packed, n, C, mode, stream)
                          : mhc::launch_phi_pack_ks32(phi, phi_dtype, packed, n, C, mode, stream),
                    "mhc_phi_pack_split");
}

static int pre_full(const void* x, int x_dtype, const void* phi, int phi_dtype,
                    const void* phi_packed, const void* alpha_pre, const void* bias_pre,
                    const void* alpha_post, const void* bias_post, const void* alpha_res,
                    const void* bias_res, int param_dtype, void* sublayer_in, void* h_pre,
                    void* h_post, void* h_res_raw, void* h_res, float* inv_rms, float* mixes_raw,
                    int64_t M, int n, int C, float post_mult, float pre_eps, float rms_eps,
                    int sinkhorn_iters, float sinkhorn_eps, const void* norm_w, int norm_dtype,
                    float norm_eps, const float* x_ssq, hipStream_t stream, const char* fn) {
  mhc::PreArgs a{};
  a.x_ssq = x_ssq;
  a.norm_w = norm_w;
  a.norm_dtype = norm_dtype;
  a.norm_eps = norm_eps;
  a.x = x;
  a.phi = phi;
  a.phi_packed = phi_packed;
  a.alpha[0] = alpha_pre;
  a.alpha[1] = alpha_post;
  a.alpha[2] = alpha_res;
  a.bias[0] = bias_pre;
  a.bias[1] = bias_post;
  a.bias[2] = bias_res;
  a.sub_in = sublayer_in;
  a.h_pre = h_pre;
  a.h_post = h_post;
  a.h_res_raw = h_res_raw;
  a.h_res = h_res;
  a.inv_rms = inv_rms;
  a.mixes_raw = mixes_raw;
  a.M = M;
  a.n = n;
  a.C = C;
  a.mode = mhc::kFull;
  a.x_dtype = x_dtype;
  a.phi_dtype = phi_dtype;
  a.param_dtype = param_dtype;
  a.post_mult = post_mult;
  a.pre_eps = pre_eps;
  a.rms_eps = rms_eps;
  a.sk_iters = sinkhorn_iters;
  a.sk_eps = sinkhorn_eps;
  return run_pre(a, stream, fn);
}

int mhc_pre_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype, const void* phi_packed,
                const void* alpha_pre, const void* bias_pre, const void* alpha_post,
                const void* bias_post, const void* alpha_res, const void* bias_res,
                int param_dtype, void* sublayer_in, void* h_pre, void* h_post, void* h_res_raw,
                void* h_res, float* inv_rms, float* mixes_raw, int64_t M, int n, int C,
                float post_mult, float pre_eps, float rms_eps, int sinkhorn_iters,
                float sinkhorn_eps, const float* x_ssq, hipStream_t stream) {
  return pre_full(x, x_dtype, phi, phi_dtype, phi_packed, alpha_pre, bias_pre, alpha_post,
                  bias_post, alpha_res, bias_res, param_dtype, sublayer_in, h_pre, h_post,
                  h_res_raw, h_res, inv_rms, mixes_raw, M, n, C, post_mult, pre_eps, rms_eps,
                  sinkhorn_iters, sinkhorn_eps, nullptr, 0, 0.f, x_ssq, stream, "mhc_pre_fwd");
}

int mhc_pre_norm_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                     const void* phi_packed, const void* alpha_pre, const void* bias_pre,
                     const void* alpha_post, const void* bias_post, const void* alpha_res,
                     const void* bias_res, int param_dtype, void* sublayer_in_normed, void* h_pre,
                     void* h_post, void* h_res_raw, void* h_res, float* inv_rms,
                     float* mixes_raw, int64_t M, int n, int C, float post_mult, float pre_eps,
                     float rms_eps, int sinkhorn_iters, float sinkhorn_eps,
                     const void* norm_weight, int norm_dtype, float norm_eps,
                     const float* x_ssq, hipStream_t stream) {
  if (!norm_weight && M != 0) return fail(hipErrorInvalidValue, "mhc_pre_norm_fwd: norm_weight is required");
  return pre_full(x, x_dtype, phi, phi_dtype, phi_packed, alpha_pre, bias_pre, alpha_post,
                  bias_post, alpha_res, bias_res, param_dtype, sublayer_in_normed, h_pre, h_post,
                  h_res_raw, h_res, inv_rms, mixes_raw, M, n, C, post_mult, pre_eps, rms_eps,
                  sinkhorn_iters, sinkhorn_eps, norm_weight, norm_dtype, norm_eps, x_ssq, stream,
                  "mhc_pre_norm_fwd");
}

static int pre_nohres(const void* x, int x_dtype, const void* phi, int phi_dtype,
                      const void* phi_packed, const void* alpha_pre, const void* bias_pre,
                      const void* alpha_post, const void* bias_post, int param_dtype,
                      void* sublayer_in, void* h_pre, void* h_post, float* inv_rms,
                      float* mixes_raw, int64_t M, int n, int C, float post_mult, float pre_eps,
                      float rms_eps, const void* norm_w, int norm_dtype, float norm_eps,
                      const float* x_ssq, hipStream_t stream, const char* fn) {
  mhc::PreArgs a{};
  a.x_ssq = x_ssq;
  a.norm_w = norm_w;
  a.norm_dtype = norm_dtype;
  a.norm_eps = norm_eps;
  a.x = x;
  a.phi = phi;
  a.phi_packed = phi_packed;
  a.alpha[0] = alpha_pre;
  a.alpha[1] = alpha_post;
  a.bias[0] = bias_pre;
  a.bias[1] = bias_post;
  a.sub_in = sublayer_in;
  a.h_pre = h_pre;
  a.h_post = h_post;
  a.inv_rms = inv_rms;
  a.mixes_raw = mixes_raw;
  a.M = M;
  a.n = n;
  a.C = C;
  a.mode = mhc::kNoHres;
  a.x_dtype = x_dtype;
  a.phi_dtype = phi_dtype;
  a.param_dtype = param_dtype;
  a.post_mult = post_mult;
  a.pre_eps = pre_eps;
  a.rms_eps = rms_eps;
  return run_pre(a, stream, fn);
}

int mhc_pre_nohres_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                       const void* phi_packed, const void* alpha_pre, const void* bias_pre,
                       const void* alpha_post, const void* bias_post, int param_dtype,
                       void* sublayer_in, void* h_pre, void* h_post, float* inv_rms,
                       float* mixes_raw, int64_t M, int n, int C, float post_mult, float pre_eps,
                       float rms_eps, const float* x_ssq, hipStream_t stream) {
  return pre_nohres(x, x_dtype, phi, phi_dtype, phi_packed, alpha_pre, bias_pre, alpha_post,
                    bias_post, param_dtype, sublayer_in, h_pre, h_post, inv_rms, mixes_raw, M, n,
                    C, post_mult, pre_eps, rms_eps, nullptr, 0, 0.f, x_ssq, stream,
                    "mhc_pre_nohres_fwd");
}

int mhc_pre_nohres_norm_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                            const void* phi_packed, const void* alpha_pre, const void* bias_pre,
                            const void* alpha_post, const void* bias_post, int param_dtype,
                            void* sublayer_in_normed, void* h_pre, void* h_post, float* inv_rms,
                            float* mixes_raw, int64_t M, int n, int C, float post_mult,
                            float pre_eps, float rms_eps, const void* norm_weight, int norm_dtype,
                            float norm_eps, const float* x_ssq, hipStream_t stream) {
  if (!norm_weight && M != 0) return fail(hipErrorInvalidValue, "mhc_pre_nohres_norm_fwd: norm_weight is required");
  return pre_nohres(x, x_dtype, phi, phi_dtype, phi_packed, alpha_pre, bias_pre, alpha_post,
                    bias_post, param_dtype, sublayer_in_normed, h_pre, h_post, inv_rms, mixes_raw,
                    M, n, C, post_mult, pre_eps, rms_eps, norm_weight, norm_dtype, norm_eps,
                    x_ssq, stream, "mhc_pre_nohres_norm_fwd");
}

static int head(const void* x, int x_dtype, const void* phi, int phi_dtype,
                const void* phi_packed, const void* alpha, const void* bias, int param_dtype,
                void* out, float* inv_rms, float* mix_raw, int64_t M, int n, int C, float pre_eps,
                float rms_eps, const void* norm_w, int norm_dtype, float norm_eps,
                const float* x_ssq, hipStream_t stream, const char* fn) {
  mhc::PreArgs a{};
  a.x_ssq = x_ssq;
  a.norm_w = norm_w;
  a.norm_dtype = norm_dtype;
  a.norm_eps = norm_eps;
  a.x = x;
  a.phi = phi;
  a.phi_packed = phi_packed;
  a.alpha[0] = alpha;
  a.bias[0] = bias;
  a.sub_in = out;
  a.inv_rms = inv_rms;
  a.mixes_raw = n == 1 ? nullptr : mix_raw;
  a.M = M;
  a.n = n;
  a.C = C;
  a.mode = n == 1 ? mhc::kRms : mhc::kHead;
  a.x_dtype = x_dtype;
  a.phi_dtype = phi_dtype;
  a.param_dtype = param_dtype;
  a.pre_eps = pre_eps;
  a.rms_eps = rms_eps;
  return run_pre(a, stream, fn);
}

int mhc_head_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                 const void* phi_packed, const void* alpha, const void* bias, int param_dtype,
                 void* out, float* inv_rms, float* mix_raw, int64_t M, int n, int C, float pre_eps,
                 float rms_eps, const float* x_ssq, hipStream_t stream) {
  return head(x, x_dtype, phi, phi_dtype, phi_packed, alpha, bias, param_dtype, out, inv_rms,
              mix_raw, M, n, C, pre_eps, rms_eps, nullptr, 0, 0.f, x_ssq, stream, "mhc_head_fwd");
}

int mhc_head_norm_fwd(const void* x, int x_dtype, const void* phi, int phi_dtype,
                      const void* phi_packed, const void* alpha, const void* bias, int param_dtype,
                      void* out_normed, float* inv_rms, float* mix_raw, int64_t M, int n, int C,
                      float pre_eps, float rms_eps, const void* norm_weight, int norm_dtype,
                      float norm_eps, const float* x_ssq, hipStream_t stream) {
  if (!norm_weight && M != 0) return fail(hipErrorInvalidValue, "mhc_head_norm_fwd: norm_weight is required");
  return head(x, x_dtype, phi, phi_dtype, phi_packed, alpha, bias, param_dtype, out_normed,
              inv_rms, mix_raw, M, n, C, pre_eps, rms_eps, norm_weight, norm_dtype, norm_eps,
              x_ssq, stream, "mhc_head_norm_fwd");
}

static int run_post(mhc::PostArgs& a, hipStream_t stream, const char* fn) {
  if (a.M < 0) return fail(hipErrorInvalidValue, "%s: M must be >= 0", fn);
  if (a.n < 1 || a.n > kMaxN) return fail(hipErrorInvalidValue, "%s: n must be in [1, %d] (got %d)", fn, kMaxN, a.n);
  if (a.C < 1) return fail(hipErrorInvalidValue, "%s: C must be >= 1", fn);
  if (!dtype_ok(a.x_dtype) || !dtype_ok(a.h_dtype) || !dtype_ok(a.f_dtype))
    return fail(hipErrorInvalidValue, "%s: bad dtype", fn);
  if (a.M * a.n * (int64_t)a.C / 256 + 1 > kMaxBlocks) return fail(hipErrorInvalidValue, "%s: problem too large", fn);
  if (a.M == 0) return 0;
  if (!a.x || !a.h_post || !a.f_out || !a.out) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
  if (a.out == a.x) return fail(hipErrorInvalidValue, "%s: out must not alias x", fn);
  if (a.out_ssq && !mhc::ssq_supported(a.x_dtype, a.C))
    return fail(hipErrorInvalidValue, "%s: out_ssq needs a bf16 stream with C %% %d == 0", fn, mhc::kSsqCols);
  const hipError_t e = mhc::launch_post(a, stream);
  if (e == hipErrorInvalidValue && a.out_ssq)
    return fail(e, "%s: out_ssq needs bf16 gates and F and 16-byte aligned tensors", fn);
  return hip_status(e, fn);
}

int mhc_post_fwd(const void* x, int x_dtype, const void* h_res, const void* h_post, int h_dtype,
                 const void* f_out, int f_dtype, void* out, int64_t M, int n, int C,
                 float* out_ssq, hipStream_t stream) {
  if (!h_res && M != 0) return fail(hipErrorInvalidValue, "mhc_post_fwd: h_res is required");
  mhc::PostArgs a{x, h_res, h_post, f_out, out, out_ssq, M, n, C, x_dtype, h_dtype, f_dtype};
  return run_post(a, stream, "mhc_post_fwd");
}

int mhc_post_nohres_fwd(const void* x, int x_dtype, const void* h_post, int h_dtype,
                        const void* f_out, int f_dtype, void* out, int64_t M, int n, int C,
                        float* out_ssq, hipStream_t stream) {
  mhc::PostArgs a{x, nullptr, h_post, f_out, out, out_ssq, M, n, C, x_dtype, h_dtype, f_dtype};
  return run_post(a, stream, "mhc_post_nohres_fwd");
}

int mhc_sinkhorn_fwd(const void* m_in, void* m_out, int dtype, int64_t batch, int n, int iters,
                     float eps, hipStream_t stream) {
  if (batch < 0) return fail(hipErrorInvalidValue, "mhc_sinkhorn_fwd: batch must be >= 0");
  if (n < 1 || n > 32) return fail(hipErrorInvalidValue, "mhc_sinkhorn_fwd: n must be in [1, 32] (got %d)", n);
  if (!dtype_ok(dtype)) return fail(hipErrorInvalidValue, "mhc_sinkhorn_fwd: bad dtype %d", dtype);
  if (batch > kMaxBlocks) return fail(hipErrorInvalidValue, "mhc_sinkhorn_fwd: batch too large");
  if (batch == 0) return 0;
  if (!m_in || !m_out) return fail(hipErrorInvalidValue, "mhc_sinkhorn_fwd: null pointer");
  return hip_status(mhc::launch_sinkhorn(m_in, m_out, dtype, batch, n, iters, eps, stream),
                    "mhc_sinkhorn_fwd");
}

int mhc_stream_expand_fwd(const void* x, void* out, int elem_bytes, int64_t M, int n, int C,
                          hipStream_t stream) {
  if (elem_bytes != 2 && elem_bytes != 4)
    return fail(hipErrorInvalidValue, "mhc_stream_expand_fwd: elem_bytes must be 2 or 4");
  if (M < 0 || n < 1 || C < 1) return fail(hipErrorInvalidValue, "mhc_stream_expand_fwd: bad shape");
  if (M * n * (int64_t)C / 256 + 1 > kMaxBlocks)
    return fail(hipErrorInvalidValue, "mhc_stream_expand_fwd: problem too large");
  if (M == 0) return 0;
  if (!x || !out) return fail(hipErrorInvalidValue, "mhc_stream_expand_fwd: null pointer");
  return hip_status(mhc::launch_stream_expand(x, out, elem_bytes, M, n, C, stream),
                    "mhc_stream_expand_fwd");
}

int mhc_expand_norm_fwd(const void* x, int x_dtype, const void* norm_weight, int norm_dtype,
                        void* out, int64_t M, int n, int C, float eps, float* out_ssq,
                        hipStream_t stream) {
  const char* fn = "mhc_expand_norm_fwd";
  if (M < 0 || n < 1 || n > kMaxN || C < 1) return fail(hipErrorInvalidValue, "%s: bad shape (M=%lld n=%d C=%d)", fn, (long long)M, n, C);
  if (!dtype_ok(x_dtype) || !dtype_ok(norm_dtype)) return fail(hipErrorInvalidValue, "%s: bad dtype", fn);
  if (!(eps >= 0.f)) return fail(hipErrorInvalidValue, "%s: eps must be >= 0", fn);
  if (M > kMaxBlocks) return fail(hipErrorInvalidValue, "%s: M too large", fn);
  if (M == 0) return 0;
  if (!x || !norm_weight || !out) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
  if (out_ssq && !mhc::ssq_supported(x_dtype, C))
    return fail(hipErrorInvalidValue, "%s: out_ssq needs a bf16 stream with C %% %d == 0", fn, mhc::kSsqCols);
  const hipError_t e = mhc::launch_expand_norm(x, x_dtype, norm_weight, norm_dtype, out, M, n, C,
                                               eps, stream, out_ssq);
  if (e == hipErrorInvalidValue && out_ssq) return fail(e, "%s: out_ssq needs 16-byte aligned rows", fn);
  return hip_status(e, fn);
}

int64_t mhc_pre_token_threshold(int64_t max_tokens) {
  const int64_t prev = mhc::pre_token_max_m();
  if (max_tokens >= 0) mhc::set_pre_token_max_m(max_tokens);
  return prev;
}

int mhc_pre_row_staging(int on) {
  const int prev = mhc::pre_row_staging() ? 1 : 0;
  if (on >= 0) mhc::set_pre_row_staging(on != 0);
  return prev;
}

int64_t mhc_pre_group_split_tokens(int64_t max_tokens) {
  const int64_t prev = mhc::pre_group_split_tokens();
  if (max_tokens >= 0) mhc::set_pre_group_split_tokens(max_tokens);
  return prev;
}

// ------------------------------------------------------------------ backward

int mhc_post_bwd(const void* x, int x_dtype, const void* h_res, const void* h_post, int h_dtype,
                 const void* f_out, int f_dtype, const void* g_out, void* g_x, void* g_h_res,
                 void* g_h_post, void* g_f, int64_t M, int n, int C, hipStream_t stream) {
  const char* fn = "mhc_post_bwd";
  if (M < 0 || n < 1 || n > kMaxN || C < 1) return fail(hipErrorInvalidValue, "%s: bad shape (M=%lld n=%d C=%d)", fn, (long long)M, n, C);
  if (!dtype_ok(x_dtype) || !dtype_ok(h_dtype) || !dtype_ok(f_dtype)) return fail(hipErrorInvalidValue, "%s: bad dtype", fn);
  if (M > kMaxBlocks) return fail(hipErrorInvalidValue, "%s: M too large", fn);
  if (M == 0) return 0;
  if (!x || !h_res || !h_post || !f_out || !g_out || !g_x || !g_h_res || !g_h_post || !g_f)
    return fail(hipErrorInvalidValue, "%s: null pointer", fn);
  mhc::PostBwdArgs a{x, h_res, h_post, f_out, g_out, g_x, g_h_res, g_h_post, g_f, M, n, C, x_dtype, h_dtype, f_dtype};
  return hip_status(mhc::launch_post_bwd(a, stream), fn);
}

int mhc_post_nohres_bwd(const void* h_post, int h_dtype, const void* f_out, int f_dtype,
                        const void* g_out, int x_dtype, void* g_x, void* g_h_post, void* g_f,
                        int64_t M, int n, int C, hipStream_t stream) {
  const char* fn = "mhc_post_nohres_bwd";
  if (M < 0 || n < 1 || n > kMaxN || C < 1) return fail(hipErrorInvalidValue, "%s: bad shape", fn);
  if (!dtype_ok(x_dtype) || !dtype_ok(h_dtype) || !dtype_ok(f_dtype)) return fail(hipErrorInvalidValue, "%s: bad dtype", fn);
  if (M > kMaxBlocks) return fail(hipErrorInvalidValue, "%s: M too large", fn);
  if (M == 0) return 0;
  if (!h_post || !f_out || !g_out || !g_h_post || !g_f) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
  if (g_x == g_out) g_x = nullptr;  // identity: nothing to copy
  mhc::PostBwdArgs a{nullptr, nullptr, h_post, f_out, g_out, g_x, nullptr, g_h_post, g_f, M, n, C, x_dtype, h_dtype, f_dtype};
  return hip_status(mhc::launch_post_bwd(a, stream), fn);
}

int mhc_pre_bwd(const void* x, int x_dtype, const void* phi, int phi_dtype, const void* alpha_pre,
                const void* bias_pre, const void* alpha_post, const void* bias_post,
                const void* alpha_res, int param_dtype, const float* inv_rms,
                const float* mixes_raw, const void* g_sub, const void* g_h_pre,
                const void* g_h_post, const void* g_h_res_raw, int grad_dtype, void* g_x,
                float* g_raw, int64_t M, int n, int C, int mode, float post_mult, float pre_eps,
                hipStream_t stream) {
  const char* fn = "mhc_pre_bwd";
  if (M < 0 || n < 1 || n > kMaxN || C < 1) return fail(hipErrorInvalidValue, "%s: bad shape (M=%lld n=%d C=%d)", fn, (long long)M, n, C);
  if (mode != mhc::kFull && mode != mhc::kNoHres && mode != mhc::kHead && mode != mhc::kRms)
    return fail(hipErrorInvalidValue, "%s: bad mode %d", fn, mode);
  if (!dtype_ok(x_dtype) || !dtype_ok(grad_dtype)) return fail(hipErrorInvalidValue, "%s: bad dtype", fn);
  if (M > kMaxBlocks) return fail(hipErrorInvalidValue, "%s: M too large", fn);
  if (M == 0) return 0;
  if (!x || !inv_rms || !g_x) return fail(hipErrorInvalidValue, "%s: x, inv_rms and g_x are required", fn);
  if (mode == mhc::kRms) {
    if (!g_sub) return fail(hipErrorInvalidValue, "%s: g_sub (d out) is required for the RMSNorm head", fn);
  } else {
    if (!phi || !mixes_raw || !alpha_pre || !bias_pre) return fail(hipErrorInvalidValue, "%s: phi, mixes_raw, alpha_pre and bias_pre are required", fn);
    if (!dtype_ok(phi_dtype) || !dtype_ok(param_dtype)) return fail(hipErrorInvalidValue, "%s: bad phi / param dtype", fn);
    if (mode != mhc::kHead && (!alpha_post || !bias_post)) return fail(hipErrorInvalidValue, "%s: alpha_post and bias_post are required", fn);
    if (mode == mhc::kFull && !alpha_res) return fail(hipErrorInvalidValue, "%s: alpha_res is required", fn);
    if (mode == mhc::kHead && n == 1) return fail(hipErrorInvalidValue, "%s: MHCHead with n == 1 is mode MHC_MODE_RMS", fn);
  }
  mhc::PreBwdArgs a{};
  a.x = x; a.phi = phi;
  a.alpha[0] = alpha_pre; a.alpha[1] = alpha_post; a.alpha[2] = alpha_res;
  a.bias[0] = bias_pre; a.bias[1] = bias_post; a.bias[2] = nullptr;
  a.inv_rms = inv_rms; a.mixes = mixes_raw;
  a.g_sub = g_sub; a.g_hpre = g_h_pre; a.g_hpost = g_h_post; a.g_hres = mode == mhc::kFull ? g_h_res_raw : nullptr;
  a.g_x = g_x; a.g_raw = mode == mhc::kRms ? nullptr : g_raw;
  a.M = M; a.n = n; a.C = C; a.mode = mode;
  a.x_dtype = x_dtype; a.phi_dtype = phi_dtype; a.param_dtype = param_dtype; a.grad_dtype = grad_dtype;
  a.post_mult = post_mult; a.pre_eps = pre_eps;
  return hip_status(mhc::launch_pre_bwd(a, stream), fn);
}

int64_t mhc_pre_bwd_weights_workspace_bytes(int64_t M, int n, int C, int mode) {
  if (M < 1 || n < 1 || n > kMaxN || C < 1) return 0;
  if (mode != mhc::kFull && mode != mhc::kNoHres && mode != mhc::kHead) return 0;
  return mhc::weights_workspace_bytes(M, n, C, mode);
}

int mhc_pre_bwd_weights(const void* x, int x_dtype, const float* inv_rms, const float* mixes_raw,
                        const float* g_raw, const void* alpha_pre, const void* alpha_post,
                        const void* alpha_res, int param_dtype, void* g_phi, int phi_dtype,
                        void* g_alpha_pre, void* g_bias_pre, void* g_alpha_post,
                        void* g_bias_post, void* g_alpha_res, void* g_bias_res, void* workspace,
                        int64_t workspace_bytes, int64_t M, int n, int C, int mode,
                        hipStream_t stream) {
  return weights_entry(x, x_dtype, inv_rms, mixes_raw, g_raw, alpha_pre, alpha_post, alpha_res,
                       param_dtype, g_phi, phi_dtype, g_alpha_pre, g_bias_pre, g_alpha_post,
                       g_bias_post, g_alpha_res, g_bias_res, workspace, workspace_bytes, M, n, C,
                       mode, 0, stream, "mhc_pre_bwd_weights");
}

int mhc_pre_bwd_weights_noalloc(const void* x, int x_dtype, const float* inv_rms,
                                const float* mixes_raw, const float* g_raw, const void* alpha_pre,
                                const void* alpha_post, const void* alpha_res, int param_dtype,
                                void* g_phi, int phi_dtype, void* g_alpha_pre, void* g_bias_pre,
                                void* g_alpha_post, void* g_bias_post, void* g_alpha_res,
                                void* g_bias_res, int64_t M, int n, int C, int mode,
                                hipStream_t stream) {
  const char* fn = "mhc_pre_bwd_weights_noalloc";
  if (n < 1 || n > kMaxN || C < 1) return fail(hipErrorInvalidValue, "%s: bad shape", fn);
  if (mode != mhc::kFull && mode != mhc::kNoHres && mode != mhc::kHead) return fail(hipErrorInvalidValue, "%s: bad mode %d", fn, mode);
  const int64_t per_range = mhc::weights_range_bytes(n, C, mode);
  if (per_range > kScratchBytes)
    return fail(hipErrorInvalidValue,
                "%s: n*C*FD = %lld phi partials need %lld bytes of scratch, more than its %lld bytes; "
                "use mhc_pre_bwd_weights with a workspace", fn,
                (long long)((int64_t)n * C * mhc::mode_fd(mode, n)), (long long)per_range,
                (long long)kScratchBytes);
  void* ws = nullptr;
  if (int rc = scratch_ptr(stream, &ws, fn)) return rc;
  const int64_t ranges = kScratchBytes / per_range;
  return weights_entry(x, x_dtype, inv_rms, mixes_raw, g_raw, alpha_pre, alpha_post, alpha_res,
                       param_dtype, g_phi, phi_dtype, g_alpha_pre, g_bias_pre, g_alpha_post,
                       g_bias_post, g_alpha_res, g_bias_res, ws, kScratchBytes, M, n, C, mode,
                       ranges > 64 ? 64 : (int)ranges, stream, fn);
}

int mhc_sinkhorn_bwd_max_iters(int n) {
  if (n < 1 || n > 16) return 0;
  return mhc::kSinkhornBwdMaxIters;  // checkpointed recompute: LDS grows as sqrt(iters)
}

int mhc_sinkhorn_bwd(const void* m_in, int in_dtype, const void* g_out, int g_dtype, void* g_in,
                     int gi_dtype, int64_t batch, int n, int iters, float eps, hipStream_t stream) {
  const char* fn = "mhc_sinkhorn_bwd";
  if (batch < 0) return fail(hipErrorInvalidValue, "%s: batch must be >= 0", fn);
  if (n < 1 || n > 16) return fail(hipErrorInvalidValue, "%s: n must be in [1, 16] (got %d)", fn, n);
  const int cap = mhc_sinkhorn_bwd_max_iters(n);
  if (iters > cap)
    return fail(hipErrorInvalidValue, "%s: iters must be <= %d for n = %d (got %d)", fn, cap, n, iters);
  if (!dtype_ok(in_dtype) || !dtype_ok(g_dtype) || !dtype_ok(gi_dtype)) return fail(hipErrorInvalidValue, "%s: bad dtype", fn);
  if (batch > kMaxBlocks) return fail(hipErrorInvalidValue, "%s: batch too large", fn);
  if (batch == 0) return 0;
  if (!m_in || !g_out || !g_in) return fail(hipErrorInvalidValue, "%s: null pointer", fn);
  return hip_status(mhc::launch_sinkhorn_bwd(m_in, in_dtype, g_out, g_dtype, g_in, gi_dtype, batch, n,
                                             iters, eps, stream), fn);
}

}  // extern "C"
