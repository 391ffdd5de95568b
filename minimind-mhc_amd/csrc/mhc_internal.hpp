// Host-side declarations shared between the kernel translation units and the
// C-ABI layer.  Nothing here is exported; the public surface is include/mhc_amd.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mhc_device.hpp"

namespace mhc {

// Which slice of the reference's fused projection a pre-phase launch computes.
//   kFull   : [pre n | post n | res n*n]   (MHCConnection_Fused)
//   kNoHres : [pre n | post n]             (MHCConnection_FusedNoHres)
//   kHead   : [mix n]                      (MHCHead)
//   kRms    : no projection, out = x * inv_rms (MHCHead with n == 1)
enum Mode : int { kFull = 0, kNoHres = 1, kHead = 2, kRms = 3 };

__host__ __device__ inline int mode_fd(int mode, int n) {
  switch (mode) {
    case kFull: return 2 * n + n * n;
    case kNoHres: return 2 * n;
    case kHead: return n;
    default: return 0;
  }
}

// Everything one pre-phase launch reads and writes.  Optional outputs are null
// when the caller does not want them.
struct PreArgs {
  const void* x;          // [M, n*C]   x_dtype
  const void* phi;        // [n*C, FD]  phi_dtype, reference row-major layout
  const void* phi_packed; // MFMA B-operand image of phi (bf16), or null
  const void* alpha[3];   // pre, post, res scalars (param_dtype)
  const void* bias[3];    // pre [n], post [n], res [n*n] (param_dtype)
  void* sub_in;           // [M, C]     x_dtype  (MHCHead: the head output)
  void* h_pre;            // [M, n]     x_dtype  optional
  void* h_post;           // [M, n]     x_dtype
  void* h_res_raw;        // [M, n, n]  x_dtype  optional
  void* h_res;            // [M, n, n]  x_dtype  (Sinkhorn output; null = skip)
  float* inv_rms;         // [M]        optional
  float* mixes_raw;       // [M, FD]    optional
  int64_t M;
  int n, C, mode;
  int x_dtype, phi_dtype, param_dtype;
  float post_mult, pre_eps, rms_eps;
  int sk_iters;
  float sk_eps;
  // Partial sums of squares of each x row from the kernel that wrote x
  // (mhc_post_fwd / mhc_expand_norm_fwd): [M, C / kSsqCols] fp32, row t's
  // sum of squares = sum_j x_ssq[t][j] in j order.  Optional; the kernels that
  // would otherwise need a pass over x of their own to form it (the
  // K-streamed kernel and the n = 8 group kernel) use it, the others ignore it.
  const float* x_ssq;
  // RMSNorm over C applied to the main output before it is stored (the
  // sublayer's input norm, or the model's final norm after MHCHead):
  //   out = bf16(s * (1 / sqrt(mean_c(s^2) + norm_eps)) * norm_w),  s the
  // pre-aggregate (head output) rounded to x_dtype.  Null norm_w: no norm.
  const void* norm_w;     // [C] norm_dtype
  int norm_dtype;
  float norm_eps;
};

struct PostArgs {
  const void* x;       // [M, n*C]
  const void* h_res;   // [M, n, n] or null (identity, use_mhc = 2)
  const void* h_post;  // [M, n]
  const void* f_out;   // [M, C]
  void* out;           // [M, n*C]
  float* out_ssq;      // [M, C / kSsqCols] partial sums of squares of out, or null
  int64_t M;
  int n, C;
  int x_dtype, h_dtype, f_dtype;
};

// Post-phase backward (model/mhc_fused.py:462-526, :747-772).  g_out, g_x
// share x_dtype; g_h_res, g_h_post the h dtype; g_f the f dtype.
struct PostBwdArgs {
  const void* x;       // [M, n*C]   (read only with h_res)
  const void* h_res;   // [M, n, n] or null (identity)
  const void* h_post;  // [M, n]
  const void* f_out;   // [M, C]
  const void* g_out;   // [M, n*C]
  void* g_x;           // [M, n*C]   (may be null without h_res: then g_x == g_out)
  void* g_h_res;       // [M, n, n]  (with h_res)
  void* g_h_post;      // [M, n]
  void* g_f;           // [M, C]
  int64_t M;
  int n, C;
  int x_dtype, h_dtype, f_dtype;
};

// Pre-phase backward, per token (model/mhc_fused.py:271-413, :644-717;
// model/mhc_fused_no_hres.py:150-281; model/mhc_common.py:200-295).  The
// incoming gradients share grad_dtype; any of them may be null (zero).
struct PreBwdArgs {
  const void* x;          // [M, n*C]
  const void* phi;        // [n*C, FD]
  const void* alpha[3];   // pre, post, res (0-dim)
  const void* bias[3];    // pre [n], post [n] (the sigmoids are recomputed); res unused
  const float* inv_rms;   // [M]
  const float* mixes;     // [M, FD] fp32 projection (before alpha / bias)
  const void* g_sub;      // [M, C]   d sublayer_in (or d out for MHCHead / RMSNorm)
  const void* g_hpre;     // [M, n]
  const void* g_hpost;    // [M, n]
  const void* g_hres;     // [M, n*n] d h_res_raw
  void* g_x;              // [M, n*C]  x_dtype
  float* g_raw;           // [M, FD]   fp32: d(alpha*m + bias) per segment (null for kRms)
  int64_t M;
  int n, C, mode;
  int x_dtype, phi_dtype, param_dtype, grad_dtype;
  float post_mult, pre_eps;
};

// Weight gradients of the pre phase from the per-token g_raw:
//   grad_phi[k, f] = alpha_seg(f) * sum_t x[t, k] * inv_rms[t] * g_raw[t, f]
//   grad_bias[f]   = sum_t g_raw[t, f]
//   grad_alpha[s]  = sum_t sum_{f in s} g_raw[t, f] * mixes[t, f]
// (model/mhc_fused.py:696-711).  Token-range partials go to the workspace.
struct WeightsArgs {
  const void* x;          // [M, n*C]
  const float* inv_rms;   // [M]
  const float* mixes;     // [M, FD]
  const float* g_raw;     // [M, FD]
  const void* alpha[3];
  void* g_phi;            // [n*C, FD] phi_dtype
  void* g_alpha[3];       // 0-dim, param_dtype (null: skipped)
  void* g_bias[3];        // param_dtype (null: skipped)
  float* work;            // workspace
  int64_t M;
  int n, C, mode;
  int x_dtype, phi_dtype, param_dtype;
  // Most token ranges the workspace holds (0: as many as the launcher picks,
  // i.e. weights_workspace_bytes was allocated).
  int max_ranges;
};

// Compute units of the current device (cached).
int device_cus();
// Launchers: return hipSuccess or the launch error.
hipError_t launch_pre_mfma(const PreArgs& a, hipStream_t s);   // requires mfma_supported()
// fp32 x and fp32 phi on split bf16 MFMA operands (n in {1, 2, 4}, C <= 1024,
// C % 8 == 0, no fused norm); phi_packed is the mhc_phi_pack_split image.
bool split_supported(int x_dtype, int phi_dtype, int n, int C, int mode);
int64_t split_packed_bytes(int n, int C, int mode);
hipError_t launch_phi_pack_split(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                                 hipStream_t s);
hipError_t launch_pre_split(const PreArgs& a, int num_cus, hipStream_t s);
hipError_t launch_pre_generic(const PreArgs& a, hipStream_t s);
// Tokens at or below which launch_pre_mfma picks the small-batch group kernel
// (one workgroup per group of up to 16 tokens; process-wide setting).
int64_t pre_token_max_m();
void set_pre_token_max_m(int64_t m);
// Whether the persistent pre kernel stages x tiles through LDS from row-
// contiguous loads where the shape allows it (process-wide setting, on by
// default).
bool pre_row_staging();
void set_pre_row_staging(bool on);
// Tokens at or below which the n = 8 small-batch pre phase runs in its split
// form (two launches, bit-identical; process-wide setting, default 128).
int64_t pre_group_split_tokens();
void set_pre_group_split_tokens(int64_t m);
// RMSNorm of each C row followed by n copies (StreamExpand): out[t, i*C + c].
hipError_t launch_expand_norm(const void* x, int x_dtype, const void* w, int w_dtype, void* out,
                              int64_t M, int n, int C, float eps, hipStream_t s,
                              float* out_ssq = nullptr);
hipError_t launch_post(const PostArgs& a, hipStream_t s);
hipError_t launch_post_bwd(const PostBwdArgs& a, hipStream_t s);
hipError_t launch_pre_bwd(const PreBwdArgs& a, hipStream_t s);
int64_t weights_workspace_bytes(int64_t M, int n, int C, int mode);
// Workspace bytes of one token range (its phi partials and alpha / bias sums).
int64_t weights_range_bytes(int n, int C, int mode);
hipError_t launch_pre_bwd_weights(const WeightsArgs& a, hipStream_t s);
// Sinkhorn backward schedules: n in {2, 4, 8} keep the trajectory per lane up
// to kSinkhornBwdLanesMaxIters iterations; longer schedules and other n run
// the checkpointed workgroup kernel, up to kSinkhornBwdMaxIters (its LDS,
// (J + K + 3) KiB with K ~ J ~ sqrt(2 * iters), stays under 64 KiB).
constexpr int kSinkhornBwdLanesMaxIters = 64;
constexpr int kSinkhornBwdMaxIters = 256;
int sinkhorn_bwd_segment(int iters);
size_t sinkhorn_bwd_lds_bytes(int iters);
hipError_t launch_sinkhorn_bwd(const void* m_in, int in_dtype, const void* g_out, int g_dtype,
                               void* g_in, int gi_dtype, int64_t batch, int n, int iters,
                               float eps, hipStream_t s);
hipError_t launch_sinkhorn(const void* in, void* out, int dtype, int64_t batch, int n,
                           int iters, float eps, hipStream_t s);
hipError_t launch_stream_expand(const void* x, void* out, int elem_bytes, int64_t M, int n,
                                int C, hipStream_t s);
hipError_t launch_phi_pack(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                           hipStream_t s, int lo = 0);
// fp32 stream and phi on the K-streamed kernel (n = 8; n in {2, 4} past
// C = 1024): image = packed bf16(phi), then packed phi - bf16(phi).
int64_t ks32_packed_bytes(int n, int C, int mode);
bool ks32_supported(int x_dtype, int phi_dtype, int n, int C, int mode);
hipError_t launch_phi_pack_ks32(const void* phi, int phi_dtype, void* packed, int n, int C, int mode,
                                hipStream_t s);
hipError_t launch_pre_kstream_f32(const PreArgs& a, hipStream_t s);

// Per-row sums of squares handed from the kernel that writes a stream to the
// pre kernel that reads it: one fp32 partial per kSsqCols columns of C (for
// every stream together), bf16 streams with C % kSsqCols == 0 only.
constexpr int kSsqCols = 128;
__host__ __device__ inline bool ssq_supported(int x_dtype, int C) {
  return x_dtype == kBF16 && C > 0 && C % kSsqCols == 0;
}
// Whether a pre launch of this shape uses x_ssq (the kernels that would read x
// once more to form the sums themselves): n = 8 and n = 16 at any C, n <= 4
// past C = 1024.
__host__ __device__ inline bool ssq_used(int n, int C) {
  return n == 8 || n == 16 || (n >= 2 && C > 1024);
}

// MFMA pre-phase geometry: 16-token tiles, c-blocks of 32 columns.
constexpr int kTokTile = 16;
constexpr int kCBlock = 32;
// Widest row the MFMA kernels take: 32 column blocks (C <= 1024), i.e. at most
// four blocks per wave of the 8-wave persistent kernel.
constexpr int kMfmaMaxColBlocks = 32;

// Packed size in bytes of phi for the MFMA path, or 0 when (n, C, mode) has no
// MFMA instance (the generic kernel then serves the call).
int64_t mfma_packed_bytes(int n, int C, int mode);
bool mfma_supported(int x_dtype, int phi_dtype, int n, int C, int mode);

}  // namespace mhc
