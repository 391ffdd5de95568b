// Backward of the pre phase, its weight gradients, and Sinkhorn-Knopp.
//
// Pre phase, per token (model/mhc_fused.py:271-413; no-H_res
// model/mhc_fused_no_hres.py:150-281; MHCHead model/mhc_common.py:200-295),
// recomputed in fp32 from the saved inv_rms and mixes_raw:
//   gh[i]      = g_h_pre[i] + sum_c g_sub[c] * x[i, c]
//   g_raw      = [gh * s_pre (1 - s_pre),  g_h_post * s_post (1 - s_post) * post_mult,  g_h_res_raw]
//                s_* = sigmoid(alpha_* * mixes + bias_*)
//   gxn[k]     = sum_f alpha_seg(f) g_raw[f] * phi[k, f]
//   g_x[k]     = inv * (gxn[k] - xn[k] * mean_k(xn * gxn)) + (s_pre[i(k)] + pre_eps) * g_sub[c(k)]
// The per-token g_raw (fp32) feeds the weight gradients (model/mhc_fused.py:696-711):
//   grad_phi = alpha_seg * (x * inv)^T @ g_raw,  grad_bias = sum_t g_raw,
//   grad_alpha = sum_t sum_seg g_raw * mixes.
// Sinkhorn backward: the reference recomputes the forward under autograd
// (model/mhc_fused.py:131-137); here the forward iterates are recomputed into
// LDS and the chain rule runs back through them.
#include "mhc_internal.hpp"

namespace mhc {

namespace {

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();  // red is reused by consecutive calls
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

constexpr int kMaxFD = 2 * 16 + 16 * 16;

}  // namespace

// ------------------------------------------------ pre phase, any dtype / shape
// One 256-thread workgroup per token.
__global__ __launch_bounds__(256) void pre_bwd_generic_kernel(PreBwdArgs a) {
  __shared__ float red[4];
  __shared__ float s_gm[kMaxFD];
  __shared__ float s_h[16];
  __shared__ float s_gh[16];
  const int64_t tok = blockIdx.x;
  const int tid = threadIdx.x;
  const int n = a.n;
  const int C = a.C;
  const int64_t NC = (int64_t)n * C;
  const int64_t xb = tok * NC;
  const int xdt = a.x_dtype;
  const int gdt = a.grad_dtype;
  const float inv = a.inv_rms[tok];

  if (a.mode == kRms) {  // y = x * inv_rms: g_x = inv * (g - xn * mean(xn * g))
    float part = 0.f;
    for (int64_t k = tid; k < NC; k += 256)
      part = fmaf(ld_any(a.x, xb + k, xdt) * inv, ld_any(a.g_sub, xb + k, gdt), part);
    const float mean = block_sum(part, red) / (float)NC;
    for (int64_t k = tid; k < NC; k += 256) {
      const float xn = ld_any(a.x, xb + k, xdt) * inv;
      st_any(a.g_x, xb + k, xdt, inv * (ld_any(a.g_sub, xb + k, gdt) - xn * mean));
    }
    return;
  }

  const int FD = mode_fd(a.mode, n);
  for (int i = 0; i < n; ++i) {  // uniform
    float part = 0.f;
    if (a.g_sub)
      for (int c = tid; c < C; c += 256)
        part = fmaf(ld_any(a.g_sub, tok * C + c, gdt), ld_any(a.x, xb + (int64_t)i * C + c, xdt), part);
    const float t = block_sum(part, red);
    if (tid == 0) s_gh[i] = t + (a.g_hpre ? ld_any(a.g_hpre, tok * n + i, gdt) : 0.f);
  }
  __syncthreads();
  if (tid < FD) {
    const int f = tid;
    const float m = a.mixes[tok * FD + f];
    const int pdt = a.param_dtype;
    float graw, alpha;
    if (f < n) {
      alpha = ld_any(a.alpha[0], 0, pdt);
      const float sg = sigmoid_f(fmaf(alpha, m, ld_any(a.bias[0], f, pdt)));
      graw = s_gh[f] * sg * (1.0f - sg);
      s_h[f] = sg + a.pre_eps;
    } else if (f < 2 * n) {
      alpha = ld_any(a.alpha[1], 0, pdt);
      const float sg = sigmoid_f(fmaf(alpha, m, ld_any(a.bias[1], f - n, pdt)));
      const float gp = a.g_hpost ? ld_any(a.g_hpost, tok * n + (f - n), gdt) : 0.f;
      graw = gp * sg * (1.0f - sg) * a.post_mult;
    } else {
      alpha = ld_any(a.alpha[2], 0, pdt);
      graw = a.g_hres ? ld_any(a.g_hres, tok * n * n + (f - 2 * n), gdt) : 0.f;
    }
    if (a.g_raw) a.g_raw[tok * FD + f] = graw;
    s_gm[f] = graw * alpha;
  }
  __syncthreads();
  const int pdt = a.phi_dtype;
  float part = 0.f;
  for (int64_t k = tid; k < NC; k += 256) {
    float gxn = 0.f;
    for (int f = 0; f < FD; ++f) gxn = fmaf(s_gm[f], ld_any(a.phi, k * FD + f, pdt), gxn);
    part = fmaf(ld_any(a.x, xb + k, xdt) * inv, gxn, part);
  }
  const float mean = block_sum(part, red) / (float)NC;
  for (int64_t k = tid; k < NC; k += 256) {
    float gxn = 0.f;
    for (int f = 0; f < FD; ++f) gxn = fmaf(s_gm[f], ld_any(a.phi, k * FD + f, pdt), gxn);
    const int i = (int)(k / C);
    const int c = (int)(k - (int64_t)i * C);
    const float xn = ld_any(a.x, xb + k, xdt) * inv;
    const float gs = a.g_sub ? ld_any(a.g_sub, tok * C + c, gdt) : 0.f;
    st_any(a.g_x, xb + k, xdt, inv * (gxn - xn * mean) + s_h[i] * gs);
  }
}

hipError_t launch_pre_bwd(const PreBwdArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(pre_bwd_generic_kernel, dim3((unsigned)a.M), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ----------------------------------------------------------- weight gradients
// Token ranges: R partial sums of every (k, f) in the workspace, then one
// reduction.  Workspace layout (fp32): W[R][n*C][FD], then AB[R][2][FD]
// (sum g_raw, sum g_raw * mixes).
static int weight_ranges(int64_t M) {
  const int64_t r = (M + 255) / 256;
  return (int)(r < 1 ? 1 : (r > 64 ? 64 : r));
}

int64_t weights_workspace_bytes(int64_t M, int n, int C, int mode) {
  const int FD = mode_fd(mode, n);
  const int R = weight_ranges(M);
  return ((int64_t)R * n * C * FD + (int64_t)R * 2 * FD) * 4;
}

__global__ __launch_bounds__(256) void weights_partial_generic_kernel(WeightsArgs a, int R, int64_t per) {
  const int FD = mode_fd(a.mode, a.n);
  const int64_t NC = (int64_t)a.n * a.C;
  const int r = blockIdx.x;
  const int64_t q = (int64_t)blockIdx.y * 256 + threadIdx.x;
  const int64_t t0 = (int64_t)r * per;
  const int64_t t1 = t0 + per < a.M ? t0 + per : a.M;
  if (q < NC * FD) {
    const int64_t k = q / FD;
    const int f = (int)(q - k * FD);
    float acc = 0.f;
    for (int64_t t = t0; t < t1; ++t)
      acc = fmaf(ld_any(a.x, t * NC + k, a.x_dtype) * a.inv_rms[t], a.g_raw[t * FD + f], acc);
    a.work[(r * NC + k) * FD + f] = acc;
  }
  if (blockIdx.y == 0 && threadIdx.x < FD) {  // alpha / bias partials of this range
    const int f = threadIdx.x;
    float sb = 0.f, sa = 0.f;
    for (int64_t t = t0; t < t1; ++t) {
      const float gr = a.g_raw[t * FD + f];
      sb += gr;
      sa = fmaf(gr, a.mixes[t * FD + f], sa);
    }
    float* ab = a.work + (int64_t)R * NC * FD + (int64_t)r * 2 * FD;
    ab[f] = sb;
    ab[FD + f] = sa;
  }
}

__device__ __forceinline__ int seg_of(int f, int n) { return f < n ? 0 : (f < 2 * n ? 1 : 2); }

__global__ __launch_bounds__(256) void weights_reduce_kernel(WeightsArgs a, int R) {
  const int n = a.n;
  const int FD = mode_fd(a.mode, n);
  const int64_t NC = (int64_t)n * a.C;
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q < NC * FD) {
    const int f = (int)(q % FD);
    float acc = 0.f;
    for (int r = 0; r < R; ++r) acc += a.work[(int64_t)r * NC * FD + q];
    st_any(a.g_phi, q, a.phi_dtype, acc * ld_any(a.alpha[seg_of(f, n)], 0, a.param_dtype));
  }
  if (blockIdx.x == 0) {
    __shared__ float s_a[kMaxFD];
    const float* ab = a.work + (int64_t)R * NC * FD;
    for (int f = threadIdx.x; f < FD; f += 256) {
      float sb = 0.f, sa = 0.f;
      for (int r = 0; r < R; ++r) {
        sb += ab[(int64_t)r * 2 * FD + f];
        sa += ab[(int64_t)r * 2 * FD + FD + f];
      }
      const int sg = seg_of(f, n);
      const int base = sg == 0 ? 0 : (sg == 1 ? n : 2 * n);
      if (a.g_bias[sg]) st_any(a.g_bias[sg], f - base, a.param_dtype, sb);
      s_a[f] = sa;
    }
    __syncthreads();
    if (threadIdx.x < 3) {
      const int sg = threadIdx.x;
      const int lo = sg == 0 ? 0 : (sg == 1 ? n : 2 * n);
      const int hi = sg == 0 ? n : (sg == 1 ? 2 * n : 2 * n + n * n);
      if (hi <= FD && a.g_alpha[sg]) {
        float sa = 0.f;
        for (int f = lo; f < hi; ++f) sa += s_a[f];
        st_any(a.g_alpha[sg], 0, a.param_dtype, sa);
      }
    }
  }
}

hipError_t launch_pre_bwd_weights(const WeightsArgs& a, hipStream_t s) {
  const int FD = mode_fd(a.mode, a.n);
  const int64_t NC = (int64_t)a.n * a.C;
  const int R = weight_ranges(a.M);
  const int64_t per = (a.M + R - 1) / R;
  const int64_t qb = (NC * FD + 255) / 256;
  hipLaunchKernelGGL(weights_partial_generic_kernel, dim3((unsigned)R, (unsigned)qb), dim3(256), 0, s,
                     a, R, per);
  if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  hipLaunchKernelGGL(weights_reduce_kernel, dim3((unsigned)qb), dim3(256), 0, s, a, R);
  return hipGetLastError();
}

// ------------------------------------------------------- Sinkhorn backward
// One 256-thread workgroup holds 256 / n^2 matrices, one element per thread.
// LDS: the softmax P, the 2*iters forward iterates T[s] and a scratch row.
// Forward T[0] = P + eps, T[1] = T[0] / (colsum + eps), then row / column
// steps; backward through y = x / (sum(x) + eps):  g_x = (g_y - sum(g_y * y)) / (sum(x) + eps),
// and through the softmax: g_m = P * (g - rowsum(g * P)).
__global__ __launch_bounds__(256) void sinkhorn_bwd_kernel(const void* __restrict__ m_in, int in_dt,
                                                           const void* __restrict__ g_out, int g_dt,
                                                           void* __restrict__ g_in, int gi_dt,
                                                           int64_t batch, int n, int iters, float eps) {
  extern __shared__ float lds[];
  const int G = n * n;
  const int per = 256 / G;                  // matrices per workgroup
  const int tid = threadIdx.x;
  const int m_loc = tid / G;
  const int e = tid - m_loc * G;
  const int r = e / n;
  const int c = e - r * n;
  const int64_t mat = (int64_t)blockIdx.x * per + m_loc;
  const bool live = m_loc < per && mat < batch;
  const int64_t idx = mat * G + e;
  const int steps = 2 * (iters > 1 ? iters : 1);
  float* P = lds;                           // [256]
  float* T = lds + 256;                     // [steps][256]
  float* S = T + (int64_t)steps * 256;      // [256] scratch
  // First element of this row / column (stride n).  Threads past the last
  // whole matrix (256 % n^2 of them) read matrix 0 and store nothing.
  const int rb = m_loc < per ? tid - e + r * n : 0;
  const int cb = m_loc < per ? tid - e + c : 0;
  auto row_sum = [&](const float* A) {
    float s = 0.f;
    for (int j = 0; j < n; ++j) s += A[rb + j];
    return s;
  };
  auto col_sum = [&](const float* A) {
    float s = 0.f;
    for (int i = 0; i < n; ++i) s += A[cb + i * n];
    return s;
  };

  // forward recompute
  const float v = live ? ld_any(m_in, idx, in_dt) : 0.f;
  S[tid] = v;
  __syncthreads();
  float mx = -INFINITY;
  for (int j = 0; j < n; ++j) mx = fmaxf(mx, S[rb + j]);
  const float ex = expf(v - mx);
  __syncthreads();
  S[tid] = ex;
  __syncthreads();
  const float p = ex / row_sum(S);
  P[tid] = p;
  T[tid] = p + eps;
  __syncthreads();
  for (int s = 1; s < steps; ++s) {  // odd s: column step, even s: row step
    const float* X = T + (int64_t)(s - 1) * 256;
    const float den = ((s & 1) ? col_sum(X) : row_sum(X)) + eps;
    T[(int64_t)s * 256 + tid] = X[tid] / den;
    __syncthreads();
  }
  // backward
  float g = live ? ld_any(g_out, idx, g_dt) : 0.f;
  for (int s = steps - 1; s >= 1; --s) {
    const float* X = T + (int64_t)(s - 1) * 256;
    const float* Y = T + (int64_t)s * 256;
    __syncthreads();
    S[tid] = g * Y[tid];
    __syncthreads();
    const bool col = s & 1;
    const float dot = col ? col_sum(S) : row_sum(S);
    const float den = (col ? col_sum(X) : row_sum(X)) + eps;
    g = (g - dot) / den;
  }
  __syncthreads();
  S[tid] = g * p;
  __syncthreads();
  const float gm = p * (g - row_sum(S));
  if (live) st_any(g_in, idx, gi_dt, gm);
}

hipError_t launch_sinkhorn_bwd(const void* m_in, int in_dtype, const void* g_out, int g_dtype,
                               void* g_in, int gi_dtype, int64_t batch, int n, int iters,
                               float eps, hipStream_t s) {
  const int G = n * n;
  const int per = 256 / G;
  const int64_t blocks = (batch + per - 1) / per;
  const int steps = 2 * (iters > 1 ? iters : 1);
  const size_t lds = (size_t)(steps + 2) * 256 * sizeof(float);
  hipLaunchKernelGGL(sinkhorn_bwd_kernel, dim3((unsigned)blocks), dim3(256), lds, s, m_in, in_dtype,
                     g_out, g_dtype, g_in, gi_dtype, batch, n, iters, eps);
  return hipGetLastError();
}

}  // namespace mhc
